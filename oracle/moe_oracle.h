/*
 * CPU restatement of the reference's INT4 MoE layer (test infrastructure).
 *
 * This is the parity ORACLE. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker or as the
 * timed CPU baseline. Product code never links or calls it.
 *
 * Every function names the reference file:line it follows (paths relative to
 * the reference repository root). Floating-point contraction: the reference
 * is built with -march=native (CMakeLists.txt:46-48), so GCC contracts
 * `acc += a * b` into a fused multiply-add. The restatement writes those
 * FMAs explicitly with fmaf() and is itself compiled with -ffp-contract=off,
 * so its results do not depend on compiler flags.
 */
#ifndef UOCR_MOE_ORACLE_H
#define UOCR_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Host-layout INT4 matrix: mirrors uocr::QuantizedMatrix (include/uocr/quant.h:16-32).
 * packed [rows, ceil(cols/2)] (low nibble = even column), scales/zeros [rows, ceil(cols/g)]. */
typedef struct {
    const uint8_t* packed;
    const float* scales;
    const float* zeros;
    int rows;
    int cols;
    int group_size;
} orc_qmatrix;

/* Unquantised matrix [rows, cols] row-major: WeightMatrix's F32 forms
 * (dtype 0) and BF16_EXT (dtype 1, uint16 bf16 bits), include/uocr/weights.h:18-46. */
typedef struct {
    const void* data;
    int dtype;
    int rows;
    int cols;
} orc_dense;

/* One MoE layer's weights, as the reference's LayerWeights holds them
 * (include/uocr/weights.h; moe_decoder.cpp:76-113). */
typedef struct {
    int hidden;
    int inter;          /* per routed expert (moe_intermediate_size) */
    int shared_inter;   /* n_shared_experts * inter (weights.cpp:352) */
    int n_experts;
    int top_k;
    int norm_topk_prob;
    float routed_scaling_factor;
    int scoring_sigmoid;
    const uint16_t* router_bf16;     /* [n_experts, hidden] */
    const orc_qmatrix* gate;         /* [n_experts] */
    const orc_qmatrix* up;           /* [n_experts] */
    const orc_qmatrix* down;         /* [n_experts] */
    orc_qmatrix shared_gate, shared_up, shared_down;
    const float* rms_weight;         /* optional post-attention RMSNorm weight [hidden] */
    float rms_eps;
    const float* router_f32;         /* optional f32 router [n_experts, hidden] (an AWQ-folded
                                        router, weights.cpp:185-207); replaces router_bf16 */
    /* unquantised shared MLP (weights.cpp:289-292, the reference's own form); used when
       shared_gate_w.data is non-NULL, in place of the INT4 shared_* */
    orc_dense shared_gate_w, shared_up_w, shared_down_w;
    /* unquantised routed experts [n_experts] (config.h:111); used when non-NULL */
    const orc_dense* gate_w;
    const orc_dense* up_w;
    const orc_dense* down_w;
} orc_layer;

float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

float orc_qmatrix_at(const orc_qmatrix* q, int r, int c);
void orc_dequantize(const orc_qmatrix* q, float* out);
void orc_quantize_int4_awq(const float* w, int rows, int cols, int group, uint8_t* packed,
                           float* scales, float* zeros);
void orc_quantize_int4_symmetric(const float* w, int rows, int cols, int group,
                                 uint8_t* packed, float* scales, float* zeros);

void orc_matmul_int4(const orc_qmatrix* q, const float* x, float* y, int m);
void orc_matmul_t(const float* x, const float* w, const float* bias, float* y, int m, int n,
                  int k);
void orc_matmul_t_bf16(const float* x, const uint16_t* w, const float* bias, float* y, int m,
                       int n, int k);
void orc_softmax(float* x, int rows, int cols);
void orc_silu_mul(const float* gate, const float* up, float* out, long long n);
void orc_rmsnorm(const float* x, const float* w, float* out, int rows, int cols, float eps);

void orc_moe_gate(const float* x, const uint16_t* router_bf16, int rows, int hidden,
                  int n_experts, int top_k, int norm_topk_prob, float scaling, int sigmoid,
                  int* ids, float* weights);
void orc_moe_gate_f32router(const float* x, const float* router_f32, int rows, int hidden,
                            int n_experts, int top_k, int norm_topk_prob, float scaling,
                            int sigmoid, int* ids, float* weights);

/* AWQ expert input scale, src/runtime/weights.cpp:185-207: the post-attention
 * norm weight divided by s (in place), the bf16 router materialised as f32
 * with column c multiplied by s[c] (router_f32 [n_experts, hidden]). */
void orc_fold_expert_input_scale(const float* s, int hidden, float* rms_weight,
                                 const uint16_t* router_bf16, int n_experts, float* router_f32);
/* weights.cpp:185-197: out[r, c] = w[r, c] * s[c] (w already materialised as f32). */
void orc_scale_columns(const float* w, int rows, int cols, const float* s, float* out);

/* R-SWA KV cache of one layer, src/scheduler/kv_cache.cpp. Cache layout
 * [capacity, kv_heads, head_dim] f32 (capacity = prefill_len + window).
 * attention (kv_cache.cpp:84-130): q/out [seq, heads, head_dim]; query s attends
 * rows [0, causal ? min(kv_len, q_start + s + 1) : kv_len) of kv head
 * h / (heads / kv_heads), online softmax in row order. */
void orc_rswa_attention(const float* q, const float* kcache, const float* vcache, int kv_len, int seq,
                        int q_start, int heads, int kv_heads, int head_dim, int causal, float* out);
/* append_decode (kv_cache.cpp:54-82) with the cache's state (len, ring_pos,
 * ring_started) passed in and updated: grow to prefill_len + window, then
 * overwrite row prefill_len + ring_pos circularly. stride = kv_heads * head_dim. */
void orc_rswa_append(float* kcache, float* vcache, int* len, int* ring_pos, int* ring_started,
                     int prefill_len, int window, int stride, const float* k, const float* v);

void orc_stable_group(const int* ids, int seq, int top_k, int n_experts, int* counts,
                      int* offsets, int* perm_token, int* perm_j);

/* WeightMatrix::matmul, src/runtime/weights.cpp:51-60: F32 -> matmul_t,
 * BF16_EXT -> matmul_t_bf16 (y [m, rows] = x [m, cols] . W^T). */
void orc_dense_matmul(const orc_dense* w, const float* x, float* y, int m);
/* mlp_forward (moe_decoder.cpp:45-60) on unquantised gate/up/down. */
void orc_mlp_dense(const orc_dense* gate, const orc_dense* up, const orc_dense* down, const float* x,
                   float* out, int m);
void orc_routed_expert(const orc_layer* L, const float* x, float* out, int e);
void orc_mlp(const orc_qmatrix* gate, const orc_qmatrix* up, const orc_qmatrix* down,
             const float* x, float* out, int m);

/* Full layer. `h` [seq, hidden] f32. If L->rms_weight is set the layer computes
 * x = rmsnorm(h) and out = h + moe(x) (moe_decoder.cpp:166-179), otherwise
 * x = h and out = moe(x). Routing (ids/weights [seq, top_k]) is computed for all
 * rows; expert outputs only for the `n_sel` rows listed in `sel` (all rows when
 * sel == NULL); out rows not selected are left untouched. `threads` > 1 runs the
 * selected tokens in parallel (each token's arithmetic is unchanged). */
void orc_moe_layer(const orc_layer* L, const float* h, int seq, const int* sel, int n_sel,
                   int threads, int* ids, float* weights, float* out);

#ifdef __cplusplus
}
#endif
#endif
