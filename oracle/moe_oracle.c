/*
 * CPU restatement of the reference's INT4 MoE layer -- TEST INFRASTRUCTURE ONLY.
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg (as the checker / the timed CPU baseline). The product library never
 * links it.
 *
 * Pinning (how each function is checked against something other than itself):
 *   orc_bf16_to_f32 / orc_f32_to_bf16  exhaustive vs numpy bit arithmetic + golden vectors
 *   orc_dequantize / orc_qmatrix_at    bit-exact vs oracle/_ref (reference quant.cpp) + golden
 *   orc_quantize_*                     bit-exact vs oracle/_ref (reference quant.cpp) + golden
 *   orc_matmul_t(_bf16)                bit-exact vs oracle/_ref (reference cpu_ops.cpp) + golden
 *   orc_softmax / orc_silu_mul / orc_rmsnorm  bit-exact vs oracle/_ref + golden
 *   orc_matmul_int4                    vs float64 brute force over _ref's dequantize (bound),
 *                                      vs exact integer arithmetic on power-of-two scales
 *   orc_moe_gate                       known answers of tests/test_moe_gate.cpp:9-63,
 *                                      composition of _ref matmul_t_bf16 + _ref softmax,
 *                                      stable-argsort brute force for the greedy top-k
 *   orc_stable_group                   equals a stable sort of (expert, token) pairs
 *   orc_dense_matmul / orc_mlp_dense   bit-exact vs the composition of oracle/_ref's
 *                                      matmul_t(_bf16) + silu_mul, and a float64 bound
 *   orc_moe_layer                      float64 brute force from dequantized weights
 * The reference's weights.cpp (INT4 matvec) and moe_decoder.cpp (moe_gate) cannot be
 * linked here: weights.cpp needs nlohmann/json, which this image lacks.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* include/uocr/common.h:49-54 */
float orc_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* include/uocr/common.h:56-64 (round to nearest even on the upper 16 bits) */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t lsb = (bits >> 16) & 1u;
    bits = (bits + 0x7fffu + lsb) >> 16;
    return (uint16_t)bits;
}

static inline int nib(const uint8_t* prow, int c) {
    uint8_t b = prow[c >> 1];
    return (c & 1) ? (b >> 4) : (b & 0x0f);
}

static inline int n_groups(const orc_qmatrix* q) { return (q->cols + q->group_size - 1) / q->group_size; }

/* src/runtime/quant.cpp:12-20 */
float orc_qmatrix_at(const orc_qmatrix* q, int r, int c) {
    const int g = c / q->group_size;
    const int pr = (q->cols + 1) / 2;
    const size_t gi = (size_t)r * n_groups(q) + g;
    return ((float)nib(q->packed + (size_t)r * pr, c) - q->zeros[gi]) * q->scales[gi];
}

/* src/runtime/quant.cpp:22-37 */
void orc_dequantize(const orc_qmatrix* q, float* out) {
    const int pr = (q->cols + 1) / 2, ng = n_groups(q);
    for (int r = 0; r < q->rows; ++r) {
        const uint8_t* prow = q->packed + (size_t)r * pr;
        const float* s = q->scales + (size_t)r * ng;
        const float* z = q->zeros + (size_t)r * ng;
        for (int c = 0; c < q->cols; ++c) {
            const int g = c / q->group_size;
            out[(size_t)r * q->cols + c] = ((float)nib(prow, c) - z[g]) * s[g];
        }
    }
}

static inline void put_nib(uint8_t* prow, int c, int v) {
    if (c & 1)
        prow[c / 2] = (uint8_t)((prow[c / 2] & 0x0f) | (v << 4));
    else
        prow[c / 2] = (uint8_t)((prow[c / 2] & 0xf0) | v);
}

static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* src/runtime/quant.cpp:39-80 (asymmetric RTN, zero point rounded and clamped to [0,15]) */
void orc_quantize_int4_awq(const float* w, int rows, int cols, int group, uint8_t* packed,
                           float* scales, float* zeros) {
    const int ng = (cols + group - 1) / group, pr = (cols + 1) / 2;
    memset(packed, 0, (size_t)rows * pr);
    for (int r = 0; r < rows; ++r) {
        const float* wr = w + (size_t)r * cols;
        uint8_t* prow = packed + (size_t)r * pr;
        for (int g = 0; g < ng; ++g) {
            const int c0 = g * group, c1 = (c0 + group < cols) ? c0 + group : cols;
            float mn = wr[c0], mx = wr[c0];
            for (int c = c0 + 1; c < c1; ++c) {
                mn = (wr[c] < mn) ? wr[c] : mn;  /* std::min(mn, w) */
                mx = (mx < wr[c]) ? wr[c] : mx;  /* std::max(mx, w) */
            }
            float scale = (mx - mn) / 15.0f;
            if (scale < 1e-8f) scale = 1e-8f;
            float zero = clampf(roundf(-mn / scale), 0.0f, 15.0f);
            scales[(size_t)r * ng + g] = scale;
            zeros[(size_t)r * ng + g] = zero;
            for (int c = c0; c < c1; ++c) put_nib(prow, c, clampi((int)lroundf(wr[c] / scale + zero), 0, 15));
        }
    }
}

/* src/runtime/quant.cpp:82-116 (symmetric, zero point fixed at 8) */
void orc_quantize_int4_symmetric(const float* w, int rows, int cols, int group,
                                 uint8_t* packed, float* scales, float* zeros) {
    const int ng = (cols + group - 1) / group, pr = (cols + 1) / 2;
    memset(packed, 0, (size_t)rows * pr);
    for (int r = 0; r < rows; ++r) {
        const float* wr = w + (size_t)r * cols;
        uint8_t* prow = packed + (size_t)r * pr;
        for (int g = 0; g < ng; ++g) {
            const int c0 = g * group, c1 = (c0 + group < cols) ? c0 + group : cols;
            float amax = 0.0f;
            for (int c = c0; c < c1; ++c) {
                const float a = fabsf(wr[c]);
                amax = (amax < a) ? a : amax;
            }
            float scale = amax / 7.0f;
            if (scale < 1e-8f) scale = 1e-8f;
            scales[(size_t)r * ng + g] = scale;
            zeros[(size_t)r * ng + g] = 8.0f;
            for (int c = c0; c < c1; ++c) put_nib(prow, c, clampi((int)lroundf(wr[c] / scale) + 8, 0, 15));
        }
    }
}

/* src/runtime/weights.cpp:51-72: serial INT4 branch of WeightMatrix::matmul.
 * Loop order (i, r, c ascending); `acc += x * (q - z) * s` contracts to
 * fma(x * (q - z), s, acc) under the reference's -march=native build. */
void orc_matmul_int4(const orc_qmatrix* q, const float* x, float* y, int m) {
    const int ng = n_groups(q), pr = (q->cols + 1) / 2, gs = q->group_size;
    for (int i = 0; i < m; ++i) {
        const float* xi = x + (size_t)i * q->cols;
        float* yi = y + (size_t)i * q->rows;
        for (int r = 0; r < q->rows; ++r) {
            const uint8_t* prow = q->packed + (size_t)r * pr;
            const float* s = q->scales + (size_t)r * ng;
            const float* z = q->zeros + (size_t)r * ng;
            float acc = 0.0f;
            for (int c = 0; c < q->cols; ++c) {
                const int g = c / gs;
                acc = fmaf(xi[c] * ((float)nib(prow, c) - z[g]), s[g], acc);
            }
            yi[r] = acc;
        }
    }
}

/* src/kernels/cpu_ops.cpp:11-24 (row-parallel above 2^18 MACs; per-output sequential chain).
 * Unlike matmul_t_bf16, the reference build does NOT contract this loop: GCC 11
 * -O3 -march=native vectorises the products (vmulps, 8 then 4 lanes) and adds them in order
 * (vaddss), so each step is round(acc + round(x * w)); only the scalar tail
 * of k % 4 terms is fused (vfmadd231ss). Pinned bit-exact against
 * oracle/_ref and tests/golden/ref_vectors.npz (mmt_*). */
void orc_matmul_t(const float* x, const float* w, const float* bias, float* y, int m, int n,
                  int k) {
#pragma omp parallel for schedule(static) if ((long long)m * n * k > (1 << 18))
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            const float* wr = w + (size_t)j * k;
            const float* xr = x + (size_t)i * k;
            float acc = bias ? bias[j] : 0.0f;
            const int k4 = k & ~3;
            for (int t = 0; t < k4; ++t) acc = acc + xr[t] * wr[t];
            for (int t = k4; t < k; ++t) acc = fmaf(xr[t], wr[t], acc);
            y[(size_t)i * n + j] = acc;
        }
    }
}

/* src/kernels/cpu_ops.cpp:26-39 */
void orc_matmul_t_bf16(const float* x, const uint16_t* w, const float* bias, float* y, int m,
                       int n, int k) {
#pragma omp parallel for schedule(static) if ((long long)m * n * k > (1 << 18))
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            const uint16_t* wr = w + (size_t)j * k;
            const float* xr = x + (size_t)i * k;
            float acc = bias ? bias[j] : 0.0f;
            for (int t = 0; t < k; ++t) acc = fmaf(xr[t], orc_bf16_to_f32(wr[t]), acc);
            y[(size_t)i * n + j] = acc;
        }
    }
}

/* src/kernels/cpu_ops.cpp:93-106: max, exp(x - max) summed in order, multiply by 1/sum */
void orc_softmax(float* x, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        float* row = x + (size_t)r * cols;
        float mx = row[0];
        for (int c = 1; c < cols; ++c) mx = (mx < row[c]) ? row[c] : mx;
        float sum = 0.0f;
        for (int c = 0; c < cols; ++c) {
            row[c] = expf(row[c] - mx);
            sum += row[c];
        }
        const float inv = 1.0f / sum;
        for (int c = 0; c < cols; ++c) row[c] *= inv;
    }
}

/* src/kernels/cpu_ops.cpp:108-113 */
void orc_silu_mul(const float* gate, const float* up, float* out, long long n) {
    for (long long i = 0; i < n; ++i) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* src/kernels/cpu_ops.cpp:58-67 (`ss += x * x` contracts to fma) */
void orc_rmsnorm(const float* x, const float* w, float* out, int rows, int cols, float eps) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * cols;
        float ss = 0.0f;
        /* the reference build vectorises x*x (vmulps) and sums in order
         * (vaddss); the scalar tail of cols % 4 terms is fused (vfmadd231ss).
         * Pinned against oracle/_ref and tests/golden (rms_*). */
        const int c4 = cols & ~3;
        for (int c = 0; c < c4; ++c) ss = ss + xr[c] * xr[c];
        for (int c = c4; c < cols; ++c) ss = fmaf(xr[c], xr[c], ss);
        const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
        float* o = out + (size_t)r * cols;
        for (int c = 0; c < cols; ++c) o[c] = xr[c] * inv * w[c];
    }
}

/* src/engine/moe_decoder.cpp:258-288: scoring, greedy top-k (strict '>', first
 * maximum wins, chosen entry set to -1e30), optional renormalisation, scaling. */
static void gate_select(float* logits, int rows, int n_experts, int top_k, int norm,
                        float scaling, int sigmoid, int* ids, float* weights) {
    for (int r = 0; r < rows; ++r) {
        float* row = logits + (size_t)r * n_experts;
        if (sigmoid) {
            for (int e = 0; e < n_experts; ++e) row[e] = 1.0f / (1.0f + expf(-row[e]));
        } else {
            orc_softmax(row, 1, n_experts);
        }
        for (int j = 0; j < top_k; ++j) {
            int best = -1;
            float bestv = -1e30f;
            for (int e = 0; e < n_experts; ++e)
                if (row[e] > bestv) {
                    bestv = row[e];
                    best = e;
                }
            ids[(size_t)r * top_k + j] = best;
            weights[(size_t)r * top_k + j] = bestv;
            if (best >= 0) row[best] = -1e30f;
        }
        float* w = weights + (size_t)r * top_k;
        if (top_k > 1 && norm) {
            float sum = 0.0f;
            for (int j = 0; j < top_k; ++j) sum += w[j];
            const float denom = sum + 1e-20f;
            for (int j = 0; j < top_k; ++j) w[j] = w[j] / denom * scaling;
        } else {
            for (int j = 0; j < top_k; ++j) w[j] *= scaling;
        }
    }
}

/* src/engine/moe_decoder.cpp:245-289 with a BF16 router (weights.cpp:48-50 -> cpu_ops.cpp:26-39) */
void orc_moe_gate(const float* x, const uint16_t* router_bf16, int rows, int hidden,
                  int n_experts, int top_k, int norm_topk_prob, float scaling, int sigmoid,
                  int* ids, float* weights) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)rows * n_experts);
    orc_matmul_t_bf16(x, router_bf16, NULL, logits, rows, n_experts, hidden);
    gate_select(logits, rows, n_experts, top_k, norm_topk_prob, scaling, sigmoid, ids, weights);
    free(logits);
}

/* Same with an F32 router (weights.cpp:42-44 -> cpu_ops.cpp:11-24); used by the
 * known-answer tests of tests/test_moe_gate.cpp, whose router is F32_OWNED. */
void orc_moe_gate_f32router(const float* x, const float* router_f32, int rows, int hidden,
                            int n_experts, int top_k, int norm_topk_prob, float scaling,
                            int sigmoid, int* ids, float* weights) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)rows * n_experts);
    orc_matmul_t(x, router_f32, NULL, logits, rows, n_experts, hidden);
    gate_select(logits, rows, n_experts, top_k, norm_topk_prob, scaling, sigmoid, ids, weights);
    free(logits);
}

/* src/runtime/weights.cpp:185-197 (scale_columns): the matrix as f32, column c
 * times s[c], one rounding per element. */
void orc_scale_columns(const float* w, int rows, int cols, const float* s, float* out) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) out[(size_t)r * cols + c] = w[(size_t)r * cols + c] * s[c];
}

/* src/runtime/weights.cpp:199-207 (apply_expert_input_scale), for the norm and
 * the router: norm[j] /= s[j]; router = scale_columns(bf16 -> f32 router, s).
 * The shared gate/up take orc_scale_columns on their f32 values. */
void orc_fold_expert_input_scale(const float* s, int hidden, float* rms_weight,
                                 const uint16_t* router_bf16, int n_experts, float* router_f32) {
    for (int j = 0; j < hidden; ++j) rms_weight[j] /= s[j];
    for (int e = 0; e < n_experts; ++e)
        for (int c = 0; c < hidden; ++c)
            router_f32[(size_t)e * hidden + c] = orc_bf16_to_f32(router_bf16[(size_t)e * hidden + c]) * s[c];
}

/* src/scheduler/kv_cache.cpp:84-130, as the reference build computes it: the
 * score loop like matmul_t (products rounded, added in order; only the scalar
 * tail of head_dim % 4 terms fused), the accumulator update as
 * fma(acc, alpha, round(beta * v)), l * alpha + beta as fma(l, alpha, beta);
 * exp is glibc's expf (std::exp on floats). Pinned bit-exact against
 * oracle/_ref (tests/test_oracle_rswa.py). */
void orc_rswa_attention(const float* q, const float* kcache, const float* vcache, int kv_len, int seq,
                        int q_start, int heads, int kv_heads, int head_dim, int causal, float* out) {
    const int hd = head_dim, group = heads / kv_heads;
    const float scale = 1.0f / sqrtf((float)hd);
    float* acc = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int s = 0; s < seq; ++s) {
        const int qpos = q_start + s;
        for (int h = 0; h < heads; ++h) {
            const float* qh = q + ((size_t)s * heads + h) * hd;
            const int kvh = h / group;
            const int limit = causal ? (kv_len < qpos + 1 ? kv_len : qpos + 1) : kv_len;
            float m = -INFINITY, l = 0.0f;
            for (int d = 0; d < hd; ++d) acc[d] = 0.0f;
            for (int t = 0; t < limit; ++t) {
                const float* kt = kcache + ((size_t)t * kv_heads + kvh) * hd;
                const float* vt = vcache + ((size_t)t * kv_heads + kvh) * hd;
                float dot = 0.0f;
                const int hd4 = hd & ~3;
                for (int d = 0; d < hd4; ++d) dot = dot + qh[d] * kt[d];
                for (int d = hd4; d < hd; ++d) dot = fmaf(qh[d], kt[d], dot);
                dot = dot * scale;
                const float m_new = m > dot ? m : dot;
                const float alpha = expf(m - m_new);
                const float beta = expf(dot - m_new);
                l = fmaf(l, alpha, beta);
                for (int d = 0; d < hd; ++d) acc[d] = fmaf(acc[d], alpha, beta * vt[d]);
                m = m_new;
            }
            float* oh = out + ((size_t)s * heads + h) * hd;
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            for (int d = 0; d < hd; ++d) oh[d] = acc[d] * inv;
        }
    }
    free(acc);
}

/* src/scheduler/kv_cache.cpp:54-82 */
void orc_rswa_append(float* kcache, float* vcache, int* len, int* ring_pos, int* ring_started,
                     int prefill_len, int window, int stride, const float* k, const float* v) {
    int row;
    if (*len < prefill_len + window) {
        row = *len;
        *len = *len + 1;
        if (*len >= prefill_len + window) {
            *ring_started = 1;
            *ring_pos = 0;
        }
    } else {
        if (!*ring_started) {
            *ring_started = 1;
            *ring_pos = 0;
        }
        row = prefill_len + *ring_pos;
        *ring_pos = (*ring_pos + 1) % window;
    }
    memcpy(kcache + (size_t)row * stride, k, sizeof(float) * (size_t)stride);
    memcpy(vcache + (size_t)row * stride, v, sizeof(float) * (size_t)stride);
}

/* src/engine/gpu_decoder.cu:602-609: for t, for j: e_tokens[ids[t,j]].push_back(t)
 * -- a stable counting sort of the (t, j) entries by expert. */
void orc_stable_group(const int* ids, int seq, int top_k, int n_experts, int* counts,
                      int* offsets, int* perm_token, int* perm_j) {
    memset(counts, 0, sizeof(int) * n_experts);
    for (int i = 0; i < seq * top_k; ++i) counts[ids[i]]++;
    offsets[0] = 0;
    for (int e = 0; e < n_experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int* fill = (int*)calloc((size_t)n_experts, sizeof(int));
    for (int t = 0; t < seq; ++t)
        for (int j = 0; j < top_k; ++j) {
            const int e = ids[t * top_k + j];
            const int s = offsets[e] + fill[e]++;
            perm_token[s] = t;
            if (perm_j) perm_j[s] = j;
        }
    free(fill);
}

/* src/engine/moe_decoder.cpp:45-60 (mlp_forward: gate, up, silu_mul, down) */
void orc_mlp(const orc_qmatrix* gate, const orc_qmatrix* up, const orc_qmatrix* down,
             const float* x, float* out, int m) {
    const int inter = gate->rows;
    float* g = (float*)malloc(sizeof(float) * (size_t)m * inter);
    float* u = (float*)malloc(sizeof(float) * (size_t)m * inter);
    float* a = (float*)malloc(sizeof(float) * (size_t)m * inter);
    orc_matmul_int4(gate, x, g, m);
    orc_matmul_int4(up, x, u, m);
    orc_silu_mul(g, u, a, (long long)m * inter);
    orc_matmul_int4(down, a, out, m);
    free(g);
    free(u);
    free(a);
}

/* src/runtime/weights.cpp:51-60 (WeightMatrix::matmul, F32 and BF16_EXT branches) */
void orc_dense_matmul(const orc_dense* w, const float* x, float* y, int m) {
    if (w->dtype == 1)
        orc_matmul_t_bf16(x, (const uint16_t*)w->data, NULL, y, m, w->rows, w->cols);
    else
        orc_matmul_t(x, (const float*)w->data, NULL, y, m, w->rows, w->cols);
}

/* src/engine/moe_decoder.cpp:45-60 (mlp_forward) and :62-74 (routed_expert)
 * with unquantised matrices */
void orc_mlp_dense(const orc_dense* gate, const orc_dense* up, const orc_dense* down, const float* x,
                   float* out, int m) {
    const int inter = gate->rows;
    float* g = (float*)malloc(sizeof(float) * (size_t)m * inter);
    float* u = (float*)malloc(sizeof(float) * (size_t)m * inter);
    float* a = (float*)malloc(sizeof(float) * (size_t)m * inter);
    orc_dense_matmul(gate, x, g, m);
    orc_dense_matmul(up, x, u, m);
    orc_silu_mul(g, u, a, (long long)m * inter);
    orc_dense_matmul(down, a, out, m);
    free(g);
    free(u);
    free(a);
}

/* src/engine/moe_decoder.cpp:62-74 */
void orc_routed_expert(const orc_layer* L, const float* x, float* out, int e) {
    if (L->gate_w)
        orc_mlp_dense(&L->gate_w[e], &L->up_w[e], &L->down_w[e], x, out, 1);
    else
        orc_mlp(&L->gate[e], &L->up[e], &L->down[e], x, out, 1);
}

/* The routed sum of one token, src/engine/moe_decoder.cpp:86-97:
 * moe[d] += w[j] * routed(x, ids[j])[d], j ascending. */
static void routed_token(const orc_layer* L, const float* x, const int* ids, const float* w, float* moe) {
    const int H = L->hidden;
    float* acc = (float*)malloc(sizeof(float) * H);
    for (int d = 0; d < H; ++d) moe[d] = 0.0f;
    for (int j = 0; j < L->top_k; ++j) {
        orc_routed_expert(L, x, acc, ids[j]);
        for (int d = 0; d < H; ++d) moe[d] = fmaf(w[j], acc[d], moe[d]);
    }
    free(acc);
}

void orc_moe_layer(const orc_layer* L, const float* h, int seq, const int* sel, int n_sel,
                   int threads, int* ids, float* weights, float* out) {
    const int H = L->hidden;
    const float* x = h;
    float* xn = NULL;
    if (L->rms_weight) {
        xn = (float*)malloc(sizeof(float) * (size_t)seq * H);
        orc_rmsnorm(h, L->rms_weight, xn, seq, H, L->rms_eps);
        x = xn;
    }
    if (L->router_f32)
        orc_moe_gate_f32router(x, L->router_f32, seq, H, L->n_experts, L->top_k, L->norm_topk_prob,
                               L->routed_scaling_factor, L->scoring_sigmoid, ids, weights);
    else
        orc_moe_gate(x, L->router_bf16, seq, H, L->n_experts, L->top_k, L->norm_topk_prob,
                     L->routed_scaling_factor, L->scoring_sigmoid, ids, weights);
    const int n = sel ? n_sel : seq;
    if (n <= 0) {
        free(xn);
        return;
    }
    float* moe = (float*)malloc(sizeof(float) * (size_t)n * H);
    /* routed experts, token by token (the reference's loop runs on one thread;
       threads > 1 splits the tokens, each token's arithmetic unchanged) */
    (void)threads;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) if (threads > 1)
    for (int i = 0; i < n; ++i) {
        const int t = sel ? sel[i] : i;
        routed_token(L, x + (size_t)t * H, ids + (size_t)t * L->top_k, weights + (size_t)t * L->top_k,
                     moe + (size_t)i * H);
    }
    /* shared experts: one mlp_forward over the batch rows, then add_rows
       (moe_decoder.cpp:109-112); its matmuls follow the reference's OpenMP rule */
    if (L->shared_inter > 0) {
        float* xs = (float*)malloc(sizeof(float) * (size_t)n * H);
        float* sh = (float*)malloc(sizeof(float) * (size_t)n * H);
        for (int i = 0; i < n; ++i)
            memcpy(xs + (size_t)i * H, x + (size_t)(sel ? sel[i] : i) * H, sizeof(float) * H);
        if (L->shared_gate_w.data)
            orc_mlp_dense(&L->shared_gate_w, &L->shared_up_w, &L->shared_down_w, xs, sh, n);
        else
            orc_mlp(&L->shared_gate, &L->shared_up, &L->shared_down, xs, sh, n);
        for (size_t i = 0; i < (size_t)n * H; ++i) moe[i] += sh[i];
        free(xs);
        free(sh);
    }
    for (int i = 0; i < n; ++i) {
        const int t = sel ? sel[i] : i;
        float* o = out + (size_t)t * H;
        const float* m = moe + (size_t)i * H;
        if (L->rms_weight) {
            const float* hr = h + (size_t)t * H;
            for (int d = 0; d < H; ++d) o[d] = hr[d] + m[d];
        } else {
            memcpy(o, m, sizeof(float) * H);
        }
    }
    free(moe);
    free(xn);
}
