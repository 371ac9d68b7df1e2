/*
 * libuocr_hip -- MI355X (gfx950) INT4 MoE expert path, C ABI.
 *
 * Drop-in boundary for the reference's MoE operator API
 * (include/uocr/cuda_ops.h:125-202 in vaachang/unlimited-ocr.cpp) and its
 * caller GpuDecoder::mlp_block (src/engine/gpu_decoder.cu:518-658).
 *
 * Conventions (all entry points):
 *   - plain pointers and sizes; device pointers unless a parameter says "host";
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream);
 *   - work is enqueued asynchronously on `stream`; no entry point synchronizes
 *     or allocates on the per-call path (creation/upload calls do allocate);
 *   - every call returns an int status: UOCR_HIP_OK (0) or a negative code;
 *     uocr_hip_last_error() returns the calling thread's last error text.
 *     (The reference throws uocr::Error from host checks and silently drops
 *     overflows, include/uocr/common.h:33-43, moe_device.cu:92; this ABI
 *     never throws and reports instead.)
 */
#ifndef UOCR_HIP_MOE_CAPI_H
#define UOCR_HIP_MOE_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UOCR_HIP_OK 0
#define UOCR_HIP_EINVAL (-1)      /* bad argument (null, shape, alignment) */
#define UOCR_HIP_EUNSUPPORTED (-2) /* valid in the reference, not supported by this build */
#define UOCR_HIP_ENOMEM (-3)      /* device allocation failed (creation calls only) */
#define UOCR_HIP_EWORKSPACE (-4)  /* caller workspace smaller than the size query */
#define UOCR_HIP_EHIP (-5)        /* a HIP runtime call failed; see uocr_hip_last_error() */
#define UOCR_HIP_ENOTFOUND (-6)   /* a named tensor is absent (weight ingest) */

#define UOCR_HIP_DTYPE_F32 0
#define UOCR_HIP_DTYPE_BF16 1

/* Error text of the calling thread's most recent failing call ("" if none). */
const char* uocr_hip_last_error(void);

/* Library version string. */
const char* uocr_hip_version(void);

/* Host-side INT4 matrix in the reference layout; mirrors uocr::QuantizedMatrix
 * (include/uocr/quant.h:16-32): packed [rows, ceil(cols/2)] bytes, low nibble =
 * even column; scales and zeros [rows, ceil(cols/group_size)] f32;
 * value = (q - zero) * scale (src/runtime/quant.cpp:12-20). */
typedef struct {
    const uint8_t* packed;
    const float* scales;
    const float* zeros;
    int rows;
    int cols;
    int group_size;
} uocr_hip_qmatrix;

/* Unquantised host matrix [rows, cols], row-major: the reference's
 * WeightMatrix in its BF16_EXT form (a bf16 checkpoint view) or its F32
 * forms (F32_EXT / F32_OWNED, e.g. the AWQ-folded shared gate/up that
 * scale_columns materialises), include/uocr/weights.h:18-46,
 * src/runtime/weights.cpp:101-112,185-197. dtype is UOCR_HIP_DTYPE_BF16
 * (uint16 bf16 bits) or UOCR_HIP_DTYPE_F32. */
typedef struct {
    const void* data;
    int dtype;
    int rows;
    int cols;
} uocr_hip_dense_matrix;

/* One MoE layer (host pointers). Field names follow uocr::ModelConfig
 * (include/uocr/config.h:18-33) and uocr::LayerWeights (include/uocr/weights.h).
 * The shared MLP has width n_shared * inter (src/runtime/weights.cpp:352). */
typedef struct {
    int hidden;                 /* hidden_size */
    int inter;                  /* moe_intermediate_size */
    int n_experts;              /* n_routed_experts (<= 64 for the fused router) */
    int top_k;                  /* num_experts_per_tok (<= 8) */
    int n_shared;               /* n_shared_experts (0 = no shared MLP) */
    int norm_topk_prob;
    float routed_scaling_factor;
    int scoring_sigmoid;        /* 0 = softmax, 1 = sigmoid */
    const uint16_t* router_bf16;               /* [n_experts, hidden] bf16 bits */
    const uocr_hip_qmatrix* gate;              /* [n_experts], each [inter, hidden] */
    const uocr_hip_qmatrix* up;                /* [n_experts], each [inter, hidden] */
    const uocr_hip_qmatrix* down;              /* [n_experts], each [hidden, inter] */
    const uocr_hip_qmatrix* shared_gate;       /* [n_shared*inter, hidden] or NULL */
    const uocr_hip_qmatrix* shared_up;         /* [n_shared*inter, hidden] or NULL */
    const uocr_hip_qmatrix* shared_down;       /* [hidden, n_shared*inter] or NULL */
    const float* rms_weight;    /* optional post-attention RMSNorm weight [hidden] */
    float rms_eps;              /* rms_norm_eps */
    const float* router_f32;    /* optional f32 router [n_experts, hidden]; replaces
                                   router_bf16 (the router of an AWQ-folded layer,
                                   weights.cpp:199-207, is f32). Such a layer routes
                                   with the f32-weight router kernel on every path
                                   and never takes the single-kernel decode paths. */
    /* The shared MLP unquantised, as the reference loads it (load_linear with
     * quantize = false, src/runtime/weights.cpp:289-292: BF16_EXT views of the
     * checkpoint, F32 gate/up after the AWQ fold, weights.cpp:199-207) and runs
     * it (three bf16 linear_forward calls, src/engine/gpu_decoder.cu:647-652).
     * Non-NULL: [n_shared*inter, hidden] / [n_shared*inter, hidden] /
     * [hidden, n_shared*inter], each bf16 or f32 on its own, and the INT4
     * shared_gate/up/down must be NULL. */
    const uocr_hip_dense_matrix* shared_gate_w;
    const uocr_hip_dense_matrix* shared_up_w;
    const uocr_hip_dense_matrix* shared_down_w;
    /* Unquantised routed experts (the reference's default expert format,
     * include/uocr/config.h:111; grouped by moe_grouped_gate_up_bf16 /
     * _down_bf16, src/kernels/cuda/moe_gemm_bf16.cu:122-353). Non-NULL: arrays
     * [n_experts] of [inter, hidden] / [inter, hidden] / [hidden, inter]
     * matrices, the INT4 gate/up/down must be NULL, and the shared MLP must be
     * unquantised too (or absent). */
    const uocr_hip_dense_matrix* gate_w;
    const uocr_hip_dense_matrix* up_w;
    const uocr_hip_dense_matrix* down_w;
} uocr_hip_layer_desc;

typedef struct uocr_hip_moe_layer uocr_hip_moe_layer;

/* Upload + repack one layer to the current device. Replaces
 * GpuDecoder::upload_expert_table (src/engine/gpu_decoder.cu:316-358) for the
 * gate/up/down tables plus the router and shared-expert uploads
 * (gpu_decoder.cu:185-187). Requirements: hidden and inter multiples of 128,
 * group_size in {32, 64, 128} dividing inter; zeros integer-valued in [0, 15]
 * (quantize_int4_awq's asymmetric layout, src/runtime/quant.cpp:39-80, or the
 * symmetric zero 8 of quantize_int4_symmetric, quant.cpp:82-116; a layer whose
 * zeros are all 8 takes the zero-free fast path); |15 * scale| (all-8 zeros:
 * |8 * scale|) within the f16 range. Scales are stored as f16 (round to
 * nearest: relative error <= 2^-11 per scale in f16's normal range; exact for
 * bf16-valued scales there), zeros exactly. Scales below f16's normal range
 * (2^-14) are held as f16 subnormals (absolute error <= 2^-25) and scales below
 * 2^-25 become 0 (the reference quantizer's 1e-8 floor, quant.cpp:62, is such
 * a scale). Unquantised matrices (uocr_hip_dense_matrix) are stored as f16:
 * exact for bf16 values in f16's normal range, relative error <= 2^-11 for f32
 * values there; every |value| must be <= 65504 (f16's range). Anything else is
 * UOCR_HIP_EUNSUPPORTED with the reason in uocr_hip_last_error(). Allocates
 * device memory; not for the per-call path. */
int uocr_hip_moe_layer_create(const uocr_hip_layer_desc* desc, uocr_hip_moe_layer** out);
int uocr_hip_moe_layer_destroy(uocr_hip_moe_layer* layer);

/* Device bytes of the repacked layer (weights + router + scales). */
size_t uocr_hip_moe_layer_device_bytes(const uocr_hip_moe_layer* layer);

/* Workspace bytes uocr_hip_moe_layer_forward needs for `seq` tokens (the
 * reference sizes the same scratch in GpuDecoder::ensure_router_scratch,
 * src/engine/gpu_decoder.cu:438-474). */
size_t uocr_hip_moe_layer_workspace_size(const uocr_hip_moe_layer* layer, int seq);

/* One MoE layer for `seq` tokens -- the fused counterpart of the MoE part of
 * GpuDecoder::mlp_block (src/engine/gpu_decoder.cu:537-657): router logits,
 * top-k, grouping, routed experts, shared expert and combine.
 *   x         [seq, hidden], dtype UOCR_HIP_DTYPE_BF16 or _F32
 *   out       [seq, hidden] f32: moe(x) (routed + shared); for a layer created
 *             with rms_weight: out = x + moe(rmsnorm(x)) (moe_decoder.cpp:166-179),
 *             which requires f32 x
 *   ids_out, weights_out  optional [seq, top_k] routing result (NULL = internal)
 * Routing ids/weights equal the reference CPU path's bit for bit; `out`
 * follows it within rel_l2 <= 5e-3 (FP32 accumulation of exact f16 products).
 * Asynchronous on `stream`, no allocation, graph-capturable for a fixed seq. */
int uocr_hip_moe_layer_forward(const uocr_hip_moe_layer* layer, const void* x, int x_dtype,
                               int seq, float* out, int* ids_out, float* weights_out,
                               void* workspace, size_t workspace_bytes, void* stream);

/* uocr_hip_moe_layer_forward without a workspace argument and without any
 * allocation. No counterpart in the reference: for callers that cannot call
 * hipMalloc (code under HIP graph capture without a pre-allocated workspace,
 * serving loops or harnesses that forbid allocation). The workspace is a
 * library-owned device array of 64 MiB per device (held until the process
 * ends); calls whose uocr_hip_moe_layer_workspace_size exceeds it return
 * UOCR_HIP_EINVAL (about 1100 tokens at the Unlimited-OCR shapes).
 * Every call on one device shares that array: calls that overlap in time on
 * one device (different streams without ordering) race and must not be
 * issued. The layer's device must be current. */
int uocr_hip_moe_layer_forward_noalloc(const uocr_hip_moe_layer* layer, const void* x, int x_dtype,
                                       int seq, float* out, int* ids_out, float* weights_out,
                                       void* stream);

/* Per-stage timing of uocr_hip_moe_layer_forward (benchmark support): when
 * enabled, forward records HIP events between its stages on its stream.
 * read_timing synchronizes on the last event and returns the accumulated
 * milliseconds per stage (router, group, gate_up, down, combine, fused: the
 * single-kernel decode paths, fused or streamed, up to 64 tokens) and the
 * number of forwards accumulated; it then resets the totals. */
int uocr_hip_moe_layer_set_timing(uocr_hip_moe_layer* layer, int enable);
int uocr_hip_moe_layer_read_timing(uocr_hip_moe_layer* layer, float* stage_ms, int n_stages,
                                   int* n_calls);

/* Which expert kernels forward uses for `seq` tokens: 0 = decode (GEMV-like),
 * 1 = prefill (LDS-tiled MFMA GEMM). */
int uocr_hip_moe_layer_path(const uocr_hip_moe_layer* layer, int seq);

/* Decode-path kernel choice (no counterpart in the reference: a tuning and
 * testing knob of this build). AUTO picks by batch size and input; the others
 * force one implementation wherever it applies (else forward falls back to the
 * four-launch path): STREAM = one launch, every expert group streamed once with
 * gate/up and down together (split-K partials); FUSED = one launch with the
 * gate/up -> down hand-over between workgroups; FOUR_LAUNCH = router, gate/up,
 * down and combine kernels. uocr_hip_moe_layer_decode_kernel reports the
 * choice forward makes for (seq, x_dtype), -1 on the prefill path. */
enum {
    UOCR_HIP_DECODE_AUTO = 0,
    UOCR_HIP_DECODE_STREAM = 1,
    UOCR_HIP_DECODE_FUSED = 2,
    UOCR_HIP_DECODE_FOUR_LAUNCH = 3
};
int uocr_hip_moe_layer_set_decode_kernel(uocr_hip_moe_layer* layer, int kind);
int uocr_hip_moe_layer_decode_kernel(const uocr_hip_moe_layer* layer, int seq, int x_dtype);

/* Sticky fault flags of the layer (no counterpart in the reference; for
 * callers and tests that verify a run): bit 0 = a bounded wait between
 * workgroups of the single-kernel decode path timed out, bit 1 = an exact
 * top-k pick was outside the candidate experts that path's down pass was
 * computed for (either fault also makes the affected call's `out` rows NaN,
 * so a result is never silently wrong); bit 2 = an expert activation
 * (silu(g) * u) or a prefill / unquantised-expert down output staged as f16
 * left f16's range (|v| >= 65520 or NaN) and was stored as inf / NaN, which
 * reaches `out` as non-finite values.
 * Waits for the device, stores the flags in *flags and, if clear is non-zero,
 * resets them. */
int uocr_hip_moe_layer_status(uocr_hip_moe_layer* layer, int clear, int* flags);

/* The same flags copied, stream-ordered and without a host wait, into the
 * caller's device int `d_flags` (no counterpart in the reference). */
int uocr_hip_moe_layer_status_async(const uocr_hip_moe_layer* layer, int* d_flags, void* stream);

/* ---- reference operator mirrors (include/uocr/cuda_ops.h) ---------------- */

/* Mirror of uocr::cuda::moe_router_topk (include/uocr/cuda_ops.h:125-131,
 * src/kernels/cuda/moe_device.cu:24-98): scoring + greedy top-k from logits
 * [seq, n_experts], then per-expert assignment tables [n_experts, cap].
 * Differences, all toward the CPU reference (moe_decoder.cpp:245-289,
 * gpu_decoder.cu:602-609): probabilities are bit-identical to the CPU
 * softmax (the CUDA kernel uses __expf and divides); slots are filled in
 * ascending (token, j) order instead of atomicAdd order; d_count receives
 * min(count, cap) and need not be zeroed by the caller. Above 1024 routed
 * entries (seq * top_k) the grouping runs on a library-owned per-device
 * scratch (up to 131072 entries; single-workgroup rounds beyond): such calls
 * on different streams of one device must not overlap. */
int uocr_hip_moe_router_topk(const float* router_logits, int seq, int n_experts, int top_k,
                             int norm_topk_prob, float routed_scaling_factor,
                             int scoring_sigmoid, int* d_ids, float* d_weights,
                             int* d_assign_token, float* d_assign_w, int* d_count, int cap,
                             void* stream);

/* ---- expert operator mirrors on the reference's device layout ------------
 * Tables as GpuDecoder::upload_expert_table builds them (src/engine/
 * gpu_decoder.cu:316-358): INT4 packed rows [n_experts][rows][ceil(cols/2)]
 * bytes (low nibble = even column; expert stride *_pstride bytes), f32 scales
 * and zeros [n_experts][rows][ng] (expert stride *_sstride floats, row stride
 * ng); value = (q - zero) * scale. Assignment tables [n_experts, cap] and
 * count[n_experts] as moe_router_topk writes them (entries past
 * min(count, cap) are ignored). Activations f32. INT4 weights are
 * dequantised in f32 ((q - zero) * scale) and rounded once to f16, bf16
 * weights are converted to f16, and both multiply f16-rounded activations
 * with f32 accumulation (the reference stages bf16 operands for its tensor
 * cores, moe_gemm_int4.cu:456-473; f16 carries 3 more significand bits, and
 * values beyond f16's range, |v| > 65504, become infinite rather than
 * silently wrong). `bn` / `bm` are accepted and ignored.
 * This build requires hidden and inter multiples of 64 and group % 32 == 0
 * (else UOCR_HIP_EUNSUPPORTED). The down projections ADD w * y into `out`
 * with f32 atomics (the caller zeroes `out`, as in the reference); the order
 * of those additions is not fixed. */

/* Mirror of uocr::cuda::moe_grouped_gate_up_int4 (include/uocr/cuda_ops.h:
 * 170-175, src/kernels/cuda/moe_gemm_int4.cu:736-760): act[e, s, :] =
 * silu(gate_e x_t) * up_e x_t for t = assign_token[e, s], s < count[e]. */
int uocr_hip_moe_grouped_gate_up_int4(const float* x, const uint8_t* gate_packed, const float* gate_scales,
                                      const float* gate_zeros, int gate_pstride, int gate_sstride, int gate_ng,
                                      const uint8_t* up_packed, const float* up_scales, const float* up_zeros,
                                      int up_pstride, int up_sstride, int up_ng, const int* assign_token,
                                      const int* count, int n_experts, int cap, int hidden, int inter, int group,
                                      float* act, int bn, int bm, void* stream);

/* Mirror of uocr::cuda::moe_grouped_down_int4 (cuda_ops.h:177-181,
 * moe_gemm_int4.cu:762-786): out[t] += assign_w[e, s] * down_e act[e, s]. */
int uocr_hip_moe_grouped_down_int4(const float* act, const uint8_t* packed, const float* scales,
                                   const float* zeros, int pstride, int sstride, int ng, const int* assign_token,
                                   const float* assign_w, const int* count, int n_experts, int cap, int hidden,
                                   int inter, int group, float* out, int bn, int bm, void* stream);

/* Mirror of uocr::cuda::moe_experts_masked_int4 (cuda_ops.h:145-155,
 * moe_device.cu:322-347): the grouped gate/up, then the grouped down. `seq`
 * is unused, as in the reference. */
int uocr_hip_moe_experts_masked_int4(const float* x, int seq, const uint8_t* gate_packed,
                                     const float* gate_scales, const float* gate_zeros, int gate_pstride,
                                     int gate_sstride, int gate_ng, const uint8_t* up_packed,
                                     const float* up_scales, const float* up_zeros, int up_pstride,
                                     int up_sstride, int up_ng, const uint8_t* down_packed,
                                     const float* down_scales, const float* down_zeros, int down_pstride,
                                     int down_sstride, int down_ng, const int* assign_token,
                                     const float* assign_w, const int* count, int n_experts, int cap,
                                     int hidden, int inter, int group, float* act, float* out, void* stream);

/* BF16 experts: device arrays of n_experts row-major bf16 matrix pointers,
 * gate_w / up_w [inter, hidden], down_w [hidden, inter].
 * Mirror of uocr::cuda::moe_grouped_gate_up_bf16 (cuda_ops.h:192-195,
 * src/kernels/cuda/moe_gemm_bf16.cu:122-353). */
int uocr_hip_moe_grouped_gate_up_bf16(const float* x, const uint16_t* const* gate_w,
                                      const uint16_t* const* up_w, const int* assign_token, const int* count,
                                      int n_experts, int cap, int hidden, int inter, float* act, int bn, int bm,
                                      void* stream);

/* Mirror of uocr::cuda::moe_grouped_down_bf16 (cuda_ops.h:197-200). */
int uocr_hip_moe_grouped_down_bf16(const float* act, const uint16_t* const* down_w, const int* assign_token,
                                   const float* assign_w, const int* count, int n_experts, int cap, int hidden,
                                   int inter, float* out, int bn, int bm, void* stream);

/* Mirror of uocr::cuda::moe_experts_masked (cuda_ops.h:139-143,
 * moe_device.cu:300-320): bf16 gate/up, then bf16 down. */
int uocr_hip_moe_experts_masked(const float* x, int seq, const uint16_t* const* gate_w,
                                const uint16_t* const* up_w, const uint16_t* const* down_w,
                                const int* assign_token, const float* assign_w, const int* count,
                                int n_experts, int cap, int hidden, int inter, float* act, float* out,
                                void* stream);

/* Mirror of uocr::cuda::moe_gemm_int4 (cuda_ops.h:204-207,
 * moe_gemm_int4.cu:793-800): y[m, n] = x[m, :] . dequant(W)[n, :] for one
 * INT4 matrix (packed [n, ceil(k/2)], scales / zeros [n, ceil(k/group_size)]),
 * the per-expert GEMM of the host-grouping path. The _tc* variants are the
 * reference's tuning entry points (cuda_ops.h:211-239): same product, the tile
 * parameters are ignored. Requires n % 64 == 0, k % 32 == 0, group_size % 32 == 0. */
int uocr_hip_moe_gemm_int4(const float* x, const uint8_t* packed, const float* scales, const float* zeros,
                           int m, int n, int k, int group_size, float* y, void* stream);
int uocr_hip_moe_gemm_int4_tc(const float* x, const uint8_t* packed, const float* scales, const float* zeros,
                              int m, int n, int k, int group_size, float* y, void* stream);
int uocr_hip_moe_gemm_int4_tc_n(const float* x, const uint8_t* packed, const float* scales, const float* zeros,
                                int m, int n, int k, int group_size, float* y, int bn, void* stream);
int uocr_hip_moe_gemm_int4_tc_nk(const float* x, const uint8_t* packed, const float* scales, const float* zeros,
                                 int m, int n, int k, int group_size, float* y, int bn, int bk, void* stream);
int uocr_hip_moe_gemm_int4_tc_pipe(const float* x, const uint8_t* packed, const float* scales,
                                   const float* zeros, int m, int n, int k, int group_size, float* y, int bn,
                                   void* stream);

/* ---- dense and elementwise operator mirrors: the calls GpuDecoder::mlp_block's
 * host-grouping branch and shared expert make around the expert GEMMs
 * (src/engine/gpu_decoder.cu:590-657). f32 activations, device pointers. */

/* Mirror of uocr::cuda::matmul_t_bf16 (include/uocr/cuda_ops.h:31-32,
 * src/kernels/cuda/backend.cu:607-627): y[m, n] = x[m, k] . W[n, k]^T + bias[n]
 * (bias may be NULL), W bf16 row-major. x and W are rounded to f16 (exact for
 * bf16 W in f16's normal range) and multiplied on MFMA with f32 accumulation
 * (the reference rounds x to bf16 for its tensor cores). Requires n % 64 == 0
 * and k % 32 == 0 (else UOCR_HIP_EUNSUPPORTED) and 16-byte aligned x and W. */
int uocr_hip_matmul_t_bf16(const float* x, const uint16_t* w, const float* bias, float* y, int m, int n, int k,
                           void* stream);
/* Mirror of uocr::cuda::matvec_bf16 (cuda_ops.h:41-42, backend.cu:560-577):
 * y[n] = W[n, k] . x[k] + bias; matmul_t_bf16 with m = 1. */
int uocr_hip_matvec_bf16(const float* x, const uint16_t* w, const float* bias, float* y, int n, int k,
                         void* stream);
/* Mirror of uocr::cuda::silu_mul (cuda_ops.h:242-243, gpu_ops.cu:12-19):
 * out[i] = gate[i] / (1 + exp(-gate[i])) * up[i]. */
int uocr_hip_silu_mul(const float* gate, const float* up, float* out, int n, void* stream);
/* Mirror of uocr::cuda::add_scaled (cuda_ops.h:245-246, gpu_ops.cu:21-26):
 * dst[i] += scale * src[i] (one fused multiply-add per element). */
int uocr_hip_add_scaled(float* dst, const float* src, float scale, int n, void* stream);
/* Mirror of uocr::cuda::scatter_add_scaled (cuda_ops.h:248-250,
 * gpu_ops.cu:28-37): out[row_idx[r], c] += weights[r] * vals[r, c]. Rows
 * naming the same output row are added atomically (in the reference that
 * case races); distinct rows give the reference's result exactly. */
int uocr_hip_scatter_add_scaled(float* out, const float* vals, const int* row_idx, const float* weights, int rows,
                                int cols, void* stream);
/* Mirror of uocr::cuda::gather_rows (cuda_ops.h:252-253, gpu_ops.cu:39-45):
 * dst[r, :] = src[row_idx[r], :]. */
int uocr_hip_gather_rows(float* dst, const float* src, const int* row_idx, int rows, int cols, void* stream);

/* Overflow report of uocr_hip_moe_router_topk (the reference drops entries
 * past `cap` silently, moe_device.cu:90-95): *flag = 1 if any call since the
 * last clear routed more than `cap` entries to one expert (only possible when
 * cap < seq). Synchronises the device; clear != 0 resets the flag. */
int uocr_hip_moe_router_overflow(int clear, int* flag);

/* Host-only check of the fused decode kernel's static schedule (no device
 * work; no counterpart in the reference, whose decode runs one kernel per
 * stage): replays the wait/publish program of every workgroup for a grid of
 * `grid` workgroups, `seq` router workgroups, `n_groups` expert groups of
 * `rbg` gate/up and `rbd` down items each, and the live groups `live`
 * (n_live entries, in the kernel's order). UOCR_HIP_OK if every workgroup
 * finishes and every item is published where the schedule says; else
 * UOCR_HIP_EINVAL with the first violation in uocr_hip_last_error(). */
int uocr_hip_fused_schedule_check(int seq, int grid, int n_groups, int rbg, int rbd, const int* live, int n_live);

/* ---- Weight ingest (host only, no device work) ----
 * A safetensors file read whole into host memory: the counterpart of
 * uocr::SafetensorsFile (src/runtime/safetensors.cpp:30-137). Names, dtypes
 * (F32/BF16/F16/I32/I8/U8/I4/U4), shapes and the string-valued "__metadata__"
 * entries as the reference reads them. */
typedef struct uocr_hip_st_file uocr_hip_st_file;
int uocr_hip_st_open(const char* path, uocr_hip_st_file** out);
int uocr_hip_st_close(uocr_hip_st_file* file);
int uocr_hip_st_contains(const uocr_hip_st_file* file, const char* name); /* 1 or 0 */
int uocr_hip_st_numel(const uocr_hip_st_file* file, const char* name, size_t* n);
/* SafetensorsFile::read_f32 (safetensors.cpp:88-127): F32/BF16/F16/I32/I8/U8
 * converted to f32 into dst (n must equal the tensor's element count). */
int uocr_hip_st_read_f32(const uocr_hip_st_file* file, const char* name, float* dst, size_t n);
/* SafetensorsFile::read_u8 (safetensors.cpp:129-137): U8/I8 bytes. */
int uocr_hip_st_read_u8(const uocr_hip_st_file* file, const char* name, uint8_t* dst, size_t n);
/* *value = the metadata string for key, or NULL (valid until close). */
int uocr_hip_st_metadata(const uocr_hip_st_file* file, const char* key, const char** value);

/* Group size of a pre-quantized (GPTQ) file: the "group" of its "uocr_int4"
 * JSON metadata as nlohmann's get<int>() reads it (an integer; a float
 * truncated toward zero; a boolean as 0 / 1), else fallback_group -- no
 * entry, unparsable JSON or another kind (weights.cpp:140-151). */
int uocr_hip_gptq_group(const uocr_hip_st_file* file, int fallback_group);
/* make_quantized's pre-quantized branch (weights.cpp:138-165): the INT4 matrix
 * <weight_name>.packed (U8 [rows, ceil(cols/2)]), .scales and .zeros (F32
 * [rows, ceil(cols/group)]) with the file's group, as a uocr_hip_qmatrix whose
 * arrays the file owns until uocr_hip_st_close. rows/cols are the dense
 * weight's shape (the checkpoint tensor's, weights.cpp:132-135). Returns
 * UOCR_HIP_ENOTFOUND if <weight_name>.packed is absent (the reference then
 * quantizes the dense weight itself), UOCR_HIP_EINVAL on the reference's
 * element-count mismatches. */
int uocr_hip_gptq_qmatrix(const uocr_hip_st_file* file, const char* weight_name, int rows, int cols,
                          int fallback_group, uocr_hip_qmatrix* out);
/* AWQ expert input scale (apply_expert_input_scale, weights.cpp:199-207) for
 * the tensors this layer takes: rms_weight[j] /= s[j] in place, and the bf16
 * router materialised as f32 with column c times s[c] into router_f32
 * [n_experts, hidden] (pass it as uocr_hip_layer_desc.router_f32). The shared
 * gate/up columns take uocr_hip_scale_columns_f32 on their f32 values. */
int uocr_hip_fold_expert_input_scale(const float* s, int hidden, float* rms_weight, const uint16_t* router_bf16,
                                     int n_experts, float* router_f32);
/* scale_columns (weights.cpp:185-197): out[r, c] = w[r, c] * s[c]. */
int uocr_hip_scale_columns_f32(const float* w, int rows, int cols, const float* s, float* out);

/* ---- R-SWA attention and KV cache (src/kernels/cuda/rswa_attention.cu;
 * host semantics src/scheduler/kv_cache.cpp) ----
 * Mirrors of uocr::cuda::rswa_* (include/uocr/cuda_ops.h:59-124) with the same
 * parameter lists (`bool causal` becomes int, `cudaStream_t` void*, `void`
 * int). Caches are f32 [capacity, kv_heads, head_dim] per request (batched:
 * request slot s at base + s * batch_cap * kv_heads * head_dim); q/out f32.
 * Requirements: heads a multiple of kv_heads, head_dim a multiple of 4 up to
 * 256 (the reference takes any head_dim <= 256), 16-byte aligned q, caches
 * and out. Attention uses scale 1/sqrt(head_dim) and an online softmax over
 * the rows in any order (the reference kernel walks them in order with
 * __expf); results match the CPU RSWACache::attention within 1e-4 abs.
 * When the (row, head) count cannot fill the GPU (decode), the keys are split
 * over up to 8 workgroups whose partial results go through a 4 MiB
 * library-owned device buffer and a second kernel merges them: such calls on
 * different streams of one device must not overlap.
 * Decode over the first kv_len rows: q/out [heads, head_dim]
 * (cuda_ops.h:59-63). */
int uocr_hip_rswa_attention_decode(const float* q, const float* kcache, const float* vcache, int kv_len, int heads,
                                   int kv_heads, int head_dim, float* out, void* stream);
/* Query block (cuda_ops.h:65-72): q/out [seq, heads, head_dim]; causal: query s
 * attends rows [0, min(kv_len, q_start + s + 1)), else [0, kv_len). */
int uocr_hip_rswa_attention(const float* q, const float* kcache, const float* vcache, int kv_len, int seq,
                            int q_start, int heads, int kv_heads, int head_dim, int causal, float* out,
                            void* stream);
/* The same with kv_len read from device memory at run time (cuda_ops.h:74-80),
 * so a captured graph stays valid as the cache grows. The reference kernel
 * handles seq == 1 only (it indexes heads by block for seq > 1); this one
 * applies the documented [seq, heads, head_dim] layout and causal mask. */
int uocr_hip_rswa_attention_devlen(const float* q, const float* kcache, const float* vcache, const int* d_len,
                                   int seq, int q_start, int heads, int kv_heads, int head_dim, int causal,
                                   float* out, void* stream);
/* Append one decoded token's K/V [kv_heads, head_dim] (cuda_ops.h:82-86):
 * rows grow to prefill_len + window, then row prefill_len + *d_ring_pos is
 * overwritten circularly; *d_len / *d_ring_pos advance on the device. */
int uocr_hip_rswa_append_decode(const float* k, const float* v, float* kcache, float* vcache, int* d_len,
                                int* d_ring_pos, int prefill_len, int window, int kv_heads, int head_dim,
                                void* stream);
/* Batched append (cuda_ops.h:88-99): row b of k/v [batch, kv_heads, head_dim]
 * into request d_slots[b], its state d_len / d_ring_pos / d_prefill_len
 * indexed by the slot. */
int uocr_hip_rswa_append_decode_batch(const float* k, const float* v, float* kcache_base, float* vcache_base,
                                      int* d_len, int* d_ring_pos, const int* d_prefill_len, const int* d_slots,
                                      int batch, int batch_cap, int window, int kv_heads, int head_dim,
                                      void* stream);
/* Batched decode attention (cuda_ops.h:101-107): row b of q/out
 * [batch, heads, head_dim] over request d_slots[b]'s first d_len[slot] rows. */
int uocr_hip_rswa_attention_batch(const float* q, const float* kcache_base, const float* vcache_base,
                                  const int* d_len, const int* d_slots, int batch, int batch_cap, int heads,
                                  int kv_heads, int head_dim, float* out, void* stream);
/* Ragged multi-request prefill (cuda_ops.h:109-124): row t's K/V into request
 * d_slots[t] at row d_pos[t]; attention of row t over its request's rows
 * [0, d_pos[t]]. */
int uocr_hip_rswa_write_prefill_ragged(const float* k, const float* v, float* kcache_base, float* vcache_base,
                                       const int* d_slots, const int* d_pos, int total, int batch_cap, int kv_heads,
                                       int head_dim, void* stream);
int uocr_hip_rswa_attention_ragged(const float* q, const float* kcache_base, const float* vcache_base,
                                   const int* d_slots, const int* d_pos, int total, int batch_cap, int heads,
                                   int kv_heads, int head_dim, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* UOCR_HIP_MOE_CAPI_H */
