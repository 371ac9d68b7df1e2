// extern "C" entry points onto the reference's own CPU code, compiled from the
// reference sources where they lie (src/runtime/quant.cpp, src/kernels/cpu_ops.cpp,
// src/scheduler/kv_cache.cpp).
// TEST INFRASTRUCTURE ONLY: loaded by tests/ to pin the oracle restatement and
// to write golden vectors; never part of the product.
#include <cstring>
#include <vector>

#include "uocr/kv_cache.h"
#include "uocr/ops.h"
#include "uocr/quant.h"

using uocr::QuantizedMatrix;

static QuantizedMatrix make_q(const unsigned char* packed, const float* scales,
                              const float* zeros, int rows, int cols, int group) {
    QuantizedMatrix q;
    q.rows = rows;
    q.cols = cols;
    q.group_size = group;
    const std::size_t pb = static_cast<std::size_t>(rows) * ((cols + 1) / 2);
    const std::size_t ns = static_cast<std::size_t>(rows) * q.n_groups();
    q.packed.assign(packed, packed + pb);
    q.scales.assign(scales, scales + ns);
    q.zeros.assign(zeros, zeros + ns);
    return q;
}

static void export_q(const QuantizedMatrix& q, unsigned char* packed, float* scales,
                     float* zeros) {
    std::memcpy(packed, q.packed.data(), q.packed.size());
    std::memcpy(scales, q.scales.data(), q.scales.size() * sizeof(float));
    std::memcpy(zeros, q.zeros.data(), q.zeros.size() * sizeof(float));
}

extern "C" {

void ref_dequantize(const unsigned char* packed, const float* scales, const float* zeros,
                    int rows, int cols, int group, float* out) {
    std::vector<float> o;
    make_q(packed, scales, zeros, rows, cols, group).dequantize(o);
    std::memcpy(out, o.data(), o.size() * sizeof(float));
}

float ref_qat(const unsigned char* packed, const float* scales, const float* zeros, int rows,
              int cols, int group, int r, int c) {
    return make_q(packed, scales, zeros, rows, cols, group).at(r, c);
}

void ref_quantize_awq(const float* w, int rows, int cols, int group, unsigned char* packed,
                      float* scales, float* zeros) {
    export_q(uocr::quantize_int4_awq(w, rows, cols, group), packed, scales, zeros);
}

void ref_quantize_symmetric(const float* w, int rows, int cols, int group,
                            unsigned char* packed, float* scales, float* zeros) {
    export_q(uocr::quantize_int4_symmetric(w, rows, cols, group), packed, scales, zeros);
}

void ref_matmul_t(const float* x, const float* w, const float* bias, float* y, int m, int n,
                  int k) {
    uocr::ops::matmul_t(x, w, bias, y, m, n, k);
}

void ref_matmul_t_bf16(const float* x, const unsigned short* w, const float* bias, float* y,
                       int m, int n, int k) {
    uocr::ops::matmul_t_bf16(x, w, bias, y, m, n, k);
}

void ref_softmax(float* x, int rows, int cols) { uocr::ops::softmax(x, rows, cols); }

void ref_silu_mul(const float* g, const float* u, float* out, long long n) {
    uocr::ops::silu_mul(g, u, out, n);
}

void ref_rmsnorm(const float* x, const float* w, float* out, int rows, int cols, float eps) {
    uocr::ops::rmsnorm(x, w, out, rows, cols, eps);
}

unsigned short ref_f32_to_bf16(float f) { return uocr::f32_to_bf16(f); }
float ref_bf16_to_f32(unsigned short h) { return uocr::bf16_to_f32(h); }

// R-SWA cache of one layer (src/scheduler/kv_cache.cpp)
void* ref_rswa_new(int kv_heads, int head_dim, int window) { return new uocr::RSWACache(1, kv_heads, head_dim, window); }
void ref_rswa_free(void* c) { delete static_cast<uocr::RSWACache*>(c); }
void ref_rswa_reset(void* c, int prefill_len) { static_cast<uocr::RSWACache*>(c)->reset(prefill_len); }
void ref_rswa_write_prefill(void* c, const float* k, const float* v, int seq) {
    static_cast<uocr::RSWACache*>(c)->write_prefill(0, k, v, seq);
}
void ref_rswa_append(void* c, const float* k, const float* v) { static_cast<uocr::RSWACache*>(c)->append_decode(0, k, v); }
int ref_rswa_len(void* c) { return static_cast<uocr::RSWACache*>(c)->length(0); }
int ref_rswa_ring_pos(void* c) { return static_cast<uocr::RSWACache*>(c)->ring_pos(0); }
int ref_rswa_capacity(void* c) { return static_cast<uocr::RSWACache*>(c)->capacity(); }
void ref_rswa_copy_kv(void* c, float* k, float* v) {
    auto* r = static_cast<uocr::RSWACache*>(c);
    const std::size_t n = static_cast<std::size_t>(r->capacity()) * r->kv_heads() * r->head_dim();
    std::memcpy(k, r->keys(0), n * sizeof(float));
    std::memcpy(v, r->values(0), n * sizeof(float));
}
void ref_rswa_attention(void* c, const float* q, int seq, int q_start, float* out, int heads, int causal) {
    static_cast<uocr::RSWACache*>(c)->attention(0, q, seq, q_start, out, heads, causal != 0);
}
}
