// C ABI of the reference operator mirrors (include/uocr/cuda_ops.h:134-239 in
// the reference): the same parameter lists, device pointers in the reference
// layout, `void* stream` for cudaStream_t and an int status for void.
#include <string>

#include "launch.hpp"
#include "uocr_hip/moe_capi.h"

using namespace uocr_hip;

namespace {

int bad(const char* what) { return set_error(UOCR_HIP_EINVAL, what); }

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return UOCR_HIP_OK;
    return set_error(UOCR_HIP_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// reference INT4 table checks: packed rows of ceil(cols/2) bytes, ng groups per row
int check_int4(const uint8_t* p, const float* s, const float* z, int pstride, int sstride, int ng, int rows,
               int cols, int group, int n_experts, const char* what) {
    if (!p || !s || !z) return bad(what);
    const int ng_need = (cols + group - 1) / group;
    if (ng < ng_need || (n_experts > 1 && ((long long)pstride < (long long)rows * ((cols + 1) / 2) ||
                                           (long long)sstride < (long long)rows * ng)))
        return set_error(UOCR_HIP_EINVAL, std::string(what) + ": pstride / sstride / ng smaller than the table");
    return UOCR_HIP_OK;
}

int check_common(int n_experts, int cap, int hidden, int inter, int group, bool int4) {
    if (n_experts <= 0 || cap <= 0) return bad("n_experts and cap must be positive");
    if (!mirror_shapes_ok(hidden, inter, group, int4) || !mirror_shapes_ok(inter, hidden, group, int4))
        return set_error(UOCR_HIP_EUNSUPPORTED,
                         "this build needs hidden and inter multiples of 64 (and of 32 along K) and group % 32 == 0");
    return UOCR_HIP_OK;
}

}  // namespace

extern "C" {

int uocr_hip_moe_grouped_gate_up_int4(const float* x, const uint8_t* gate_packed, const float* gate_scales,
                                      const float* gate_zeros, int gate_pstride, int gate_sstride, int gate_ng,
                                      const uint8_t* up_packed, const float* up_scales, const float* up_zeros,
                                      int up_pstride, int up_sstride, int up_ng, const int* assign_token,
                                      const int* count, int n_experts, int cap, int hidden, int inter, int group,
                                      float* act, int bn, int bm, void* stream) {
    (void)bn;
    (void)bm;  // tile hints of the reference's CUDA kernel; the tiling here is fixed
    if (n_experts <= 0 || inter <= 0) return UOCR_HIP_OK;  // reference: early return (moe_gemm_int4.cu:743)
    int rc;
    if ((rc = check_common(n_experts, cap, hidden, inter, group, true))) return rc;
    if (!x || !assign_token || !count || !act) return bad("null argument");
    if (!aligned16(x)) return bad("x must be 16-byte aligned");
    if ((rc = check_int4(gate_packed, gate_scales, gate_zeros, gate_pstride, gate_sstride, gate_ng, inter, hidden,
                         group, n_experts, "gate table")) ||
        (rc = check_int4(up_packed, up_scales, up_zeros, up_pstride, up_sstride, up_ng, inter, hidden, group,
                         n_experts, "up table")))
        return rc;
    return hip_status(mirror_gate_up_int4(x, gate_packed, gate_scales, gate_zeros, gate_pstride, gate_sstride,
                                          gate_ng, up_packed, up_scales, up_zeros, up_pstride, up_sstride, up_ng,
                                          assign_token, count, n_experts, cap, hidden, inter, group, act,
                                          (hipStream_t)stream),
                      "grouped gate/up launch");
}

int uocr_hip_moe_grouped_down_int4(const float* act, const uint8_t* packed, const float* scales,
                                   const float* zeros, int pstride, int sstride, int ng, const int* assign_token,
                                   const float* assign_w, const int* count, int n_experts, int cap, int hidden,
                                   int inter, int group, float* out, int bn, int bm, void* stream) {
    (void)bn;
    (void)bm;
    if (n_experts <= 0 || hidden <= 0) return UOCR_HIP_OK;  // reference: early return (moe_gemm_int4.cu:769)
    int rc;
    if ((rc = check_common(n_experts, cap, hidden, inter, group, true))) return rc;
    if (!act || !assign_token || !assign_w || !count || !out) return bad("null argument");
    if (!aligned16(act)) return bad("act must be 16-byte aligned");
    if ((rc = check_int4(packed, scales, zeros, pstride, sstride, ng, hidden, inter, group, n_experts, "down table")))
        return rc;
    return hip_status(mirror_down_int4(act, packed, scales, zeros, pstride, sstride, ng, assign_token, assign_w,
                                       count, n_experts, cap, hidden, inter, group, out, (hipStream_t)stream),
                      "grouped down launch");
}

int uocr_hip_moe_experts_masked_int4(const float* x, int seq, const uint8_t* gate_packed, const float* gate_scales,
                                     const float* gate_zeros, int gate_pstride, int gate_sstride, int gate_ng,
                                     const uint8_t* up_packed, const float* up_scales, const float* up_zeros,
                                     int up_pstride, int up_sstride, int up_ng, const uint8_t* down_packed,
                                     const float* down_scales, const float* down_zeros, int down_pstride,
                                     int down_sstride, int down_ng, const int* assign_token, const float* assign_w,
                                     const int* count, int n_experts, int cap, int hidden, int inter, int group,
                                     float* act, float* out, void* stream) {
    (void)seq;  // the reference ignores it too (moe_device.cu:344)
    if (n_experts == 0) return UOCR_HIP_OK;
    int rc = uocr_hip_moe_grouped_gate_up_int4(x, gate_packed, gate_scales, gate_zeros, gate_pstride, gate_sstride,
                                               gate_ng, up_packed, up_scales, up_zeros, up_pstride, up_sstride,
                                               up_ng, assign_token, count, n_experts, cap, hidden, inter, group, act,
                                               0, 0, stream);
    if (rc) return rc;
    return uocr_hip_moe_grouped_down_int4(act, down_packed, down_scales, down_zeros, down_pstride, down_sstride,
                                          down_ng, assign_token, assign_w, count, n_experts, cap, hidden, inter,
                                          group, out, 0, 0, stream);
}

int uocr_hip_moe_grouped_gate_up_bf16(const float* x, const uint16_t* const* gate_w, const uint16_t* const* up_w,
                                      const int* assign_token, const int* count, int n_experts, int cap,
                                      int hidden, int inter, float* act, int bn, int bm, void* stream) {
    (void)bn;
    (void)bm;
    if (n_experts <= 0 || inter <= 0) return UOCR_HIP_OK;
    int rc;
    if ((rc = check_common(n_experts, cap, hidden, inter, 32, false))) return rc;
    if (!x || !gate_w || !up_w || !assign_token || !count || !act) return bad("null argument");
    if (!aligned16(x)) return bad("x must be 16-byte aligned");
    return hip_status(mirror_gate_up_bf16(x, gate_w, up_w, assign_token, count, n_experts, cap, hidden, inter, act,
                                          (hipStream_t)stream),
                      "grouped bf16 gate/up launch");
}

int uocr_hip_moe_grouped_down_bf16(const float* act, const uint16_t* const* down_w, const int* assign_token,
                                   const float* assign_w, const int* count, int n_experts, int cap, int hidden,
                                   int inter, float* out, int bn, int bm, void* stream) {
    (void)bn;
    (void)bm;
    if (n_experts <= 0 || hidden <= 0) return UOCR_HIP_OK;
    int rc;
    if ((rc = check_common(n_experts, cap, hidden, inter, 32, false))) return rc;
    if (!act || !down_w || !assign_token || !assign_w || !count || !out) return bad("null argument");
    if (!aligned16(act)) return bad("act must be 16-byte aligned");
    return hip_status(mirror_down_bf16(act, down_w, assign_token, assign_w, count, n_experts, cap, hidden, inter, out,
                                       (hipStream_t)stream),
                      "grouped bf16 down launch");
}

int uocr_hip_moe_experts_masked(const float* x, int seq, const uint16_t* const* gate_w, const uint16_t* const* up_w,
                                const uint16_t* const* down_w, const int* assign_token, const float* assign_w,
                                const int* count, int n_experts, int cap, int hidden, int inter, float* act,
                                float* out, void* stream) {
    (void)seq;
    if (n_experts == 0) return UOCR_HIP_OK;
    int rc = uocr_hip_moe_grouped_gate_up_bf16(x, gate_w, up_w, assign_token, count, n_experts, cap, hidden, inter,
                                               act, 0, 0, stream);
    if (rc) return rc;
    return uocr_hip_moe_grouped_down_bf16(act, down_w, assign_token, assign_w, count, n_experts, cap, hidden, inter,
                                          out, 0, 0, stream);
}

int uocr_hip_moe_gemm_int4(const float* x, const uint8_t* packed, const float* scales, const float* zeros, int m,
                           int n, int k, int group_size, float* y, void* stream) {
    if (m <= 0 || n <= 0) return UOCR_HIP_OK;
    if (!x || !packed || !scales || !zeros || !y) return bad("null argument");
    if (!mirror_shapes_ok(k, n, group_size, true))
        return set_error(UOCR_HIP_EUNSUPPORTED, "this build needs n % 64 == 0, k % 32 == 0 and group_size % 32 == 0");
    if (!aligned16(x)) return bad("x must be 16-byte aligned");
    return hip_status(mirror_gemm_int4(x, packed, scales, zeros, m, n, k, group_size, y, (hipStream_t)stream),
                      "int4 gemm launch");
}

// The reference's tuning variants compute the same product (cuda_ops.h:211-239);
// their tile parameters are hints this build does not need.
int uocr_hip_moe_gemm_int4_tc(const float* x, const uint8_t* packed, const float* scales, const float* zeros, int m,
                              int n, int k, int group_size, float* y, void* stream) {
    return uocr_hip_moe_gemm_int4(x, packed, scales, zeros, m, n, k, group_size, y, stream);
}

int uocr_hip_moe_gemm_int4_tc_n(const float* x, const uint8_t* packed, const float* scales, const float* zeros,
                                int m, int n, int k, int group_size, float* y, int bn, void* stream) {
    (void)bn;
    return uocr_hip_moe_gemm_int4(x, packed, scales, zeros, m, n, k, group_size, y, stream);
}

int uocr_hip_moe_gemm_int4_tc_nk(const float* x, const uint8_t* packed, const float* scales, const float* zeros,
                                 int m, int n, int k, int group_size, float* y, int bn, int bk, void* stream) {
    (void)bn;
    (void)bk;
    return uocr_hip_moe_gemm_int4(x, packed, scales, zeros, m, n, k, group_size, y, stream);
}

int uocr_hip_moe_gemm_int4_tc_pipe(const float* x, const uint8_t* packed, const float* scales, const float* zeros,
                                   int m, int n, int k, int group_size, float* y, int bn, void* stream) {
    (void)bn;
    return uocr_hip_moe_gemm_int4(x, packed, scales, zeros, m, n, k, group_size, y, stream);
}

}  // extern "C"

// ---- dense and elementwise operator mirrors (include/uocr/cuda_ops.h:31-41,
// 242-253; src/kernels/cuda/backend.cu:542-627, gpu_ops.cu:12-45,85-111) ----
extern "C" {

int uocr_hip_matmul_t_bf16(const float* x, const uint16_t* w, const float* bias, float* y, int m, int n, int k,
                           void* stream) {
    if (m <= 0 || n <= 0 || k <= 0) return UOCR_HIP_OK;  // reference: early return (backend.cu:611)
    if (!x || !w || !y) return bad("null argument");
    if (!mirror_shapes_ok(k, n, 32, false))
        return set_error(UOCR_HIP_EUNSUPPORTED, "this build needs n % 64 == 0 and k % 32 == 0");
    if (!aligned16(x) || !aligned16(w)) return bad("x and w must be 16-byte aligned");
    return hip_status(mirror_gemm_bf16(x, w, bias, m, n, k, y, (hipStream_t)stream), "bf16 gemm launch");
}

int uocr_hip_matvec_bf16(const float* x, const uint16_t* w, const float* bias, float* y, int n, int k,
                         void* stream) {
    return uocr_hip_matmul_t_bf16(x, w, bias, y, 1, n, k, stream);
}

int uocr_hip_silu_mul(const float* gate, const float* up, float* out, int n, void* stream) {
    if (n <= 0) return UOCR_HIP_OK;
    if (!gate || !up || !out) return bad("null argument");
    return hip_status(mirror_silu_mul(gate, up, out, n, (hipStream_t)stream), "silu_mul launch");
}

int uocr_hip_add_scaled(float* dst, const float* src, float scale, int n, void* stream) {
    if (n <= 0) return UOCR_HIP_OK;
    if (!dst || !src) return bad("null argument");
    return hip_status(mirror_add_scaled(dst, src, scale, n, (hipStream_t)stream), "add_scaled launch");
}

int uocr_hip_scatter_add_scaled(float* out, const float* vals, const int* row_idx, const float* weights, int rows,
                                int cols, void* stream) {
    if (rows <= 0 || cols <= 0) return UOCR_HIP_OK;
    if (!out || !vals || !row_idx || !weights) return bad("null argument");
    return hip_status(mirror_scatter_add_scaled(out, vals, row_idx, weights, rows, cols, (hipStream_t)stream),
                      "scatter_add_scaled launch");
}

int uocr_hip_gather_rows(float* dst, const float* src, const int* row_idx, int rows, int cols, void* stream) {
    if (rows <= 0 || cols <= 0) return UOCR_HIP_OK;
    if (!dst || !src || !row_idx) return bad("null argument");
    return hip_status(mirror_gather_rows(dst, src, row_idx, rows, cols, (hipStream_t)stream), "gather_rows launch");
}

}  // extern "C"
