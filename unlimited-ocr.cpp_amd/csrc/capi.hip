// C ABI of libuocr_hip: layer upload/repack, workspace planning and the fused
// forward (the counterpart of GpuDecoder::mlp_block's MoE branch,
// src/engine/gpu_decoder.cu:537-657, in the reference).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "fused_schedule.hpp"
#include "launch.hpp"
#include "uocr_hip/moe_capi.h"


using namespace uocr_hip;

uocr_hip::StageEvents& uocr_hip::stage_events() {
    thread_local StageEvents e;
    return e;
}

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

}  // namespace

int uocr_hip::set_error(int code, const std::string& msg) { return fail(code, msg); }

namespace {

int hip_fail(hipError_t e, const char* what) {
    return fail(UOCR_HIP_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                         \
    do {                                            \
        hipError_t _e = (expr);                     \
        if (_e != hipSuccess) return hip_fail(_e, what); \
    } while (0)

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

uint16_t f16_bits(float f) {
    const _Float16 h = (_Float16)f;  // round to nearest even
    uint16_t out;
    std::memcpy(&out, &h, 2);
    return out;
}

// Zero points of a reference INT4 matrix: true if every zero equals 8 (the
// symmetric layout, stored implicitly); otherwise every zero must be an
// integer in [0, 15] (what quantize_int4_awq and the GPTQ files hold,
// src/runtime/quant.cpp:60-64, tools/reference/quantize_gptq.py:161).
int zero_kind(const uocr_hip_qmatrix& q, int row0, int R, bool* symmetric, std::string* err) {
    const int ng = (q.cols + q.group_size - 1) / q.group_size;
    bool sym = true;
    for (int r = row0; r < row0 + R; ++r)
        for (int g = 0; g < ng; ++g) {
            const float z = q.zeros[(size_t)r * ng + g];
            if (z == 8.0f) continue;
            sym = false;
            if (!(z >= 0.0f && z <= 15.0f) || z != std::floor(z)) {
                *err = "zero point " + std::to_string(z) + " at row " + std::to_string(r) + " group " +
                       std::to_string(g) + ": zeros must be integers in [0, 15]";
                return UOCR_HIP_EUNSUPPORTED;
            }
        }
    *symmetric = sym;
    return UOCR_HIP_OK;
}

// Repack rows [row0, row0 + R) x columns [col0, col0 + K) of a reference-layout
// INT4 matrix into the tile-16x128 device layout (common.hpp): nibbles,
// f16 scales and, if dstz is non-null, f16 zero offsets -(1024 + zero).
int repack(const uocr_hip_qmatrix& q, int row0, int R, int col0, int K, uint8_t* dst, uint16_t* dsts,
           uint16_t* dstz, std::string* err) {
    const int G = q.group_size, gpt = kTileK / G, KT = K / kTileK, RB = R / kTileRows;
    const int pr = (q.cols + 1) / 2, ng = (q.cols + G - 1) / G;
    // the largest |q - zero| the kernels form in f16 before scaling
    const float qmax = dstz ? 15.0f : 8.0f;
    for (int rb = 0; rb < RB; ++rb)
        for (int kt = 0; kt < KT; ++kt) {
            uint8_t* tile = dst + ((size_t)rb * KT + kt) * kTileBytes;
            for (int lane = 0; lane < 64; ++lane) {
                const int r = row0 + rb * kTileRows + (lane & 15);
                const uint8_t* prow = q.packed + (size_t)r * pr;
                for (int s = 0; s < 4; ++s) {
                    uint32_t w = 0;
                    for (int i = 0; i < 8; ++i) {
                        const int c = col0 + kt * kTileK + s * 32 + 8 * (lane >> 4) + i;
                        const uint8_t byte = prow[c >> 1];
                        const uint32_t nib = (c & 1) ? (byte >> 4) : (byte & 0x0f);
                        w |= nib << ((i & 1) * 16 + (i >> 1) * 4);
                    }
                    std::memcpy(tile + lane * 16 + s * 4, &w, 4);
                }
            }
            for (int rr = 0; rr < kTileRows; ++rr) {
                const int r = row0 + rb * kTileRows + rr;
                for (int gi = 0; gi < gpt; ++gi) {
                    const int g = (col0 + kt * kTileK) / G + gi;
                    const int gl = kt * gpt + gi;  // group index within the slice
                    const size_t idx = (size_t)r * ng + g;
                    const float s = q.scales[idx];
                    if (!std::isfinite(s) || std::fabs(s) * qmax > 65504.0f) {
                        *err = "scale outside the f16 range at row " + std::to_string(r);
                        return UOCR_HIP_EUNSUPPORTED;
                    }
                    const size_t o = ((size_t)rb * kTileRows + rr) * scale_row_stride(K, G) + gl;
                    dsts[o] = f16_bits(s);
                    if (dstz) dstz[o] = f16_bits(-(1024.0f + q.zeros[idx]));
                }
            }
        }
    return UOCR_HIP_OK;
}

}  // namespace

// Device scratch of uocr_hip_moe_layer_forward_noalloc: the workspace of one
// forward call for callers that cannot allocate (graph capture without a
// pre-allocated workspace, serving loops that forbid hipMalloc). One copy per
// device, held until the process ends; the host-side name `scratch` is only a
// stand-in -- its device address comes from hipGetSymbolAddress, looked up once
// per device at layer creation (scratch_ptr) and used for every access.
constexpr size_t kScratchBytes = 64u << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on `device` (the current device); looked up
// on first use per device.
int scratch_ptr(int device, void** out) {
    if (device < 0 || device >= kMaxDevices) return fail(UOCR_HIP_EINVAL, "device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return UOCR_HIP_OK;
}
}  // namespace

constexpr int kStages = 7;  // router, group, gate_up, down, combine, fused, shared

struct uocr_hip_moe_layer {
    int hidden = 0, inter = 0, n_experts = 0, top_k = 0, n_virtual = 0, group = 0;
    int norm_topk_prob = 0, scoring_sigmoid = 0;
    float scaling = 1.0f, rms_eps = 1e-6f;
    int device = 0;
    uint16_t* router_t = nullptr;
    float* router_f32 = nullptr;  // [hidden/4][64][4] (decode router)
    float* rms_weight = nullptr;
    uint8_t* gate = nullptr;   // [Ev][inter x hidden] tile layout
    uint8_t* up = nullptr;
    uint8_t* down = nullptr;   // [Ev][hidden x inter]
    uint16_t* gate_s = nullptr;
    uint16_t* up_s = nullptr;
    uint16_t* down_s = nullptr;
    uint16_t* gate_z = nullptr;  // zero offsets (null: symmetric layer, zero 8 implicit)
    uint16_t* up_z = nullptr;
    uint16_t* down_z = nullptr;
    // down scales / zero offsets of the streamed decode kernel, [Ev][inter/128][hidden][128/group]
    uint16_t* down_skt = nullptr;
    uint16_t* down_zkt = nullptr;
    // the streamed decode kernel's copy of the packed weights, in the order
    // its waves use them: unit u (1 KiB: a gate, up or down tile) of every
    // (item, wave) side by side, [kUnits][Ev * inter/128][8 waves][1 KiB]
    uint8_t* sw = nullptr;
    int decode_kernel = UOCR_HIP_DECODE_AUTO;  // uocr_hip_moe_layer_set_decode_kernel
    long long gu_wstride = 0, gu_sstride = 0, dn_wstride = 0, dn_sstride = 0;
    // unquantised matrices as f16 row-major (dense.hip): the shared MLP
    // [s_inter][hidden] / [hidden][s_inter] and the routed experts
    // [E][inter][hidden] / [E][hidden][inter]
    bool shared_dense = false, experts_dense = false;
    int s_inter = 0;
    f16* sgate = nullptr;
    f16* sup = nullptr;
    f16* sdown = nullptr;
    f16* egate = nullptr;
    f16* eup = nullptr;
    f16* edown = nullptr;
    size_t device_bytes = 0;
    bool timing = false;
    hipEvent_t ev[2 * kStages] = {};  // start/stop per stage
    unsigned stage_mask = 0;          // stages the pending call recorded
    float stage_ms[kStages] = {};
    FusedSync* sync = nullptr;        // progress words and tagged routing of the fused decode kernel
    int timed_calls = 0;
    bool pending = false;
};

namespace {

void free_layer(uocr_hip_moe_layer* L) {
    if (!L) return;
    void* ptrs[] = {L->router_t, L->router_f32, L->rms_weight, L->gate,   L->up,   L->down, L->gate_s,
                    L->up_s,     L->down_s,     L->gate_z,     L->up_z,   L->down_z, L->sync, L->down_skt, L->down_zkt, L->sw,
                    L->sgate,    L->sup,        L->sdown,      L->egate,  L->eup,    L->edown};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    for (auto& e : L->ev)
        if (e) (void)hipEventDestroy(e);
    delete L;
}

int check_qm(const uocr_hip_qmatrix* q, int rows, int cols, int group, const char* what) {
    if (!q || !q->packed || !q->scales || !q->zeros)
        return fail(UOCR_HIP_EINVAL, std::string(what) + ": null matrix pointer");
    if (q->rows != rows || q->cols != cols)
        return fail(UOCR_HIP_EINVAL, std::string(what) + ": shape " + std::to_string(q->rows) + "x" +
                                         std::to_string(q->cols) + ", expected " + std::to_string(rows) +
                                         "x" + std::to_string(cols));
    if (q->group_size != group)
        return fail(UOCR_HIP_EINVAL, std::string(what) + ": mixed group sizes in one layer");
    return UOCR_HIP_OK;
}

int check_dense(const uocr_hip_dense_matrix* m, int rows, int cols, const char* what) {
    if (!m || !m->data) return fail(UOCR_HIP_EINVAL, std::string(what) + ": null matrix pointer");
    if (m->dtype != UOCR_HIP_DTYPE_BF16 && m->dtype != UOCR_HIP_DTYPE_F32)
        return fail(UOCR_HIP_EINVAL, std::string(what) + ": dtype must be UOCR_HIP_DTYPE_BF16 or _F32");
    if (m->rows != rows || m->cols != cols)
        return fail(UOCR_HIP_EINVAL, std::string(what) + ": shape " + std::to_string(m->rows) + "x" +
                                         std::to_string(m->cols) + ", expected " + std::to_string(rows) +
                                         "x" + std::to_string(cols));
    return UOCR_HIP_OK;
}

// f16 copy of an unquantised host matrix (round to nearest; exact for bf16
// values in f16's normal range); values beyond f16's range are refused
int dense_to_f16(const uocr_hip_dense_matrix& m, uint16_t* dst, std::string* err) {
    const size_t n = (size_t)m.rows * m.cols;
    for (size_t i = 0; i < n; ++i) {
        float v;
        if (m.dtype == UOCR_HIP_DTYPE_BF16) {
            const uint32_t bits = (uint32_t) static_cast<const uint16_t*>(m.data)[i] << 16;
            std::memcpy(&v, &bits, 4);
        } else {
            v = static_cast<const float*>(m.data)[i];
        }
        if (!std::isfinite(v) || std::fabs(v) > 65504.0f) {
            *err = "value " + std::to_string(v) + " at row " + std::to_string(i / m.cols) +
                   " outside the f16 range";
            return UOCR_HIP_EUNSUPPORTED;
        }
        dst[i] = f16_bits(v);
    }
    return UOCR_HIP_OK;
}

struct WsPlan {
    size_t x16, ids, wts, counts, offsets, ntiles, slot_tok, slot_w, pos, tile_e, tile_m0, tile_info, act, y, total;
    size_t lrank, chunk_count, chunk_base;
    size_t sact, sy;  // unquantised shared MLP: act [seq, s_inter] f16, y [seq, hidden] f32
    int slots, max_tiles, bm;
};

// Prefill (LDS-tiled MFMA GEMM, 128-slot m-tiles) once experts see enough
// tokens to fill its tiles; the decode kernels (16-slot tiles, weights streamed
// once per tile) below that.
constexpr int kPrefillMinSeq = 256;
// one workgroup per token in the router up to this batch (the router matrix is
// then read once per token from L2); larger batches share it through LDS
constexpr int kRouterDecodeMaxSeq = 64;

// Decode path (per-token router, grouping-free expert passes) below
// kPrefillMinSeq tokens for the layer shapes it is instantiated for; the
// prefill path (grouped LDS-tiled MFMA GEMM) otherwise.
bool use_prefill(const uocr_hip_moe_layer* L, int seq) {
    return seq >= kPrefillMinSeq || !decode_shapes_ok(L->hidden, L->inter);
}

// Fused decode kernel (router + experts + combine in one launch) for 1 ..
// kFusedMaxSeq tokens, bf16 input without the fused RMSNorm. From
// kFusedDenseMinSeq tokens its gate/up pass covers every group for all tokens
// (no wait for routing: most experts are live anyway, 1 - (1 - 6/64)^12 = 69 %
// at top-6 of 64); below that it covers the candidate groups only, after the
// routers' candidate summary. Measured faster than the four-launch path at
// every batch size from 1 to 11.
constexpr int kFusedMinSeq = 1;

bool use_fused(const uocr_hip_moe_layer* L, int seq, int x_dtype) {
    if (L->decode_kernel == UOCR_HIP_DECODE_FOUR_LAUNCH || L->decode_kernel == UOCR_HIP_DECODE_STREAM) return false;
    // (an unquantised shared MLP runs before the launch, on bf16 input only)
    return L->sync && !L->experts_dense && L->router_t && seq >= kFusedMinSeq && seq <= kFusedMaxSeq &&
           (x_dtype == UOCR_HIP_DTYPE_BF16 || !L->shared_dense) && !L->rms_weight &&
           decode_fused_ok(L->hidden, L->inter, L->group) && L->n_experts + L->n_virtual <= kMaxExperts;
}

// Streamed decode kernel (decode_stream.hip): every expert group streams once
// for all tokens, gate/up and the matching down columns together (split-K
// partials), with no wait between expert passes. bf16 input without RMSNorm
// from kStreamMinSeq to kStreamMaxSeq tokens (below that the fused kernel is
// faster); in its wide mode (after the exact routing, per-group token blocks)
// any input, with the RMSNorm prologue, up to kStreamWideMaxSeq tokens.
constexpr int kStreamMinSeq = 6;
bool stream_layer_ok(const uocr_hip_moe_layer* L) {
    return L->sync && !L->experts_dense && (L->router_t || L->router_f32) && L->down_skt && L->sw &&
           decode_stream_ok(L->hidden, L->inter, L->group) && L->n_experts + L->n_virtual <= kMaxExperts;
}
bool stream_wide(const uocr_hip_moe_layer* L, int seq, int x_dtype) {
    (void)x_dtype;
    return seq > kStreamMaxSeq || L->rms_weight;
}
bool use_stream(const uocr_hip_moe_layer* L, int seq, int x_dtype) {
    if (L->decode_kernel == UOCR_HIP_DECODE_FOUR_LAUNCH || L->decode_kernel == UOCR_HIP_DECODE_FUSED) return false;
    if (!stream_layer_ok(L) || seq < 1) return false;
    // (an unquantised shared MLP runs before the launch, on f16 rows of the
    // normalised input when the input is f32 or takes the RMSNorm)
    if (stream_wide(L, seq, x_dtype)) return seq <= kStreamWideMaxSeq;
    // (below kStreamMinSeq the fused kernel is faster, for bf16 input; it
    // needs the bf16 router)
    const int lo = L->decode_kernel == UOCR_HIP_DECODE_STREAM || !L->router_t ? 1 : kStreamMinSeq;
    return seq >= lo && seq <= kStreamMaxSeq;
}


// Tile rows of the unquantised expert kernels: decode-sized tiles below the
// prefill threshold, 128-slot MFMA tiles from there (when the shapes allow)
int dense_experts_bm(const uocr_hip_moe_layer* L, int seq) {
    if (seq < kPrefillMinSeq) return kDenseSkinnyBM;
    // the large-tile kernel with f16 weight fragments DMA'd to LDS (K in {896, 1280})
    if (prefill_big_ok(L->hidden, L->inter)) return kPrefillBigTileRows;
    return (dense_shapes_ok(L->hidden, L->inter, true, kDenseTiledBM) &&
            dense_shapes_ok(L->inter, L->hidden, false, kDenseTiledBM))
               ? kDenseTiledBM
               : kDenseSkinnyBM;
}
// ... and of the unquantised shared MLP (every token: a plain GEMM)
int dense_shared_bm(const uocr_hip_moe_layer* L, int seq) {
    return (seq >= 128 && dense_shapes_ok(L->hidden, L->s_inter, true, kDenseTiledBM) &&
            dense_shapes_ok(L->s_inter, L->hidden, false, kDenseTiledBM))
               ? kDenseTiledBM
               : kDenseSkinnyBM;
}
// the layer runs the grouping kernels (prefill path, or unquantised experts)
bool uses_grouping(const uocr_hip_moe_layer* L, int seq) { return L->experts_dense || use_prefill(L, seq); }

WsPlan plan(const uocr_hip_moe_layer* L, int seq) {
    WsPlan p{};
    const int Ev = L->n_experts + L->n_virtual;
    p.slots = seq * (L->top_k + L->n_virtual);
    p.bm = L->experts_dense ? dense_experts_bm(L, seq)
           : !use_prefill(L, seq)
               ? kDecodeTileRows
               : (prefill_big_ok(L->hidden, L->inter) ? kPrefillBigTileRows : kPrefillTileRows);
    p.max_tiles = (seq * L->top_k) / p.bm + L->n_experts + L->n_virtual * ((seq + p.bm - 1) / p.bm) + 1;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align_up(o + bytes, 256);
        return at;
    };
    p.x16 = take((size_t)seq * L->hidden * 2);
    p.ids = take((size_t)seq * L->top_k * 4);
    p.wts = take((size_t)seq * L->top_k * 4);
    p.counts = take((size_t)Ev * 4);
    p.offsets = take((size_t)(Ev + 1) * 4);
    p.ntiles = take(4);
    p.slot_tok = take((size_t)p.slots * 4);
    p.slot_w = take((size_t)p.slots * 4);
    p.pos = take((size_t)seq * L->top_k * 4);
    p.tile_e = take((size_t)p.max_tiles * 4);
    p.tile_m0 = take((size_t)p.max_tiles * 4);
    p.tile_info = take((size_t)p.max_tiles * 16);
    // act / y: one row per slot (y: per entry), or per (group, token) when the
    // fused decode kernel may run (seq <= kFusedMaxSeq, any input dtype)
    const bool fused_rows =
        seq <= kFusedMaxSeq && L->sync && !L->experts_dense && decode_fused_ok(L->hidden, L->inter, L->group);
    const size_t rows = fused_rows ? (size_t)std::max(p.slots, Ev * seq) : (size_t)p.slots;
    // the streamed decode kernel's y: split-K partial rows [group][inter/128][token],
    // wide mode [pick or shared row][inter/128]
    const size_t ns = (size_t)(L->inter / kTileK);
    size_t yrows = rows;
    if (stream_layer_ok(L)) {
        if (seq <= kStreamMaxSeq) yrows = std::max(yrows, (size_t)Ev * ns * seq);
        if (seq <= kStreamWideMaxSeq) yrows = std::max(yrows, (size_t)(kStreamCandRows + L->n_virtual) * seq * ns);
    }
    p.act = take(rows * L->inter * 2);
    p.y = take(yrows * L->hidden * 4);
    const int chunks = group_chunks(seq, L->top_k);
    p.lrank = take((size_t)seq * L->top_k * 4);
    p.chunk_count = take((size_t)chunks * L->n_experts * 4);
    p.chunk_base = take((size_t)chunks * L->n_experts * 4);
    if (L->shared_dense) {
        p.sact = take((size_t)seq * L->s_inter * 2);
        p.sy = take((size_t)seq * L->hidden * 4);
    }
    p.total = o;
    return p;
}

}  // namespace

extern "C" {

const char* uocr_hip_last_error(void) { return g_err.c_str(); }

const char* uocr_hip_version(void) { return "uocr_hip 0.1 (gfx950)"; }

int uocr_hip_moe_layer_create(const uocr_hip_layer_desc* d, uocr_hip_moe_layer** out) {
    if (!d || !out) return fail(UOCR_HIP_EINVAL, "null argument");
    *out = nullptr;
    const int H = d->hidden, I = d->inter, E = d->n_experts;
    if (H <= 0 || I <= 0 || H % kTileK || I % kTileK)
        return fail(UOCR_HIP_EINVAL, "hidden and inter must be positive multiples of 128");
    if (router_smem_bytes(H) > 150 * 1024 || H > 1792 || I > 1792)
        return fail(UOCR_HIP_EUNSUPPORTED, "hidden/inter above 1792 are not supported by this build");
    if (E <= 0 || E > 64) return fail(UOCR_HIP_EINVAL, "n_experts must be in [1, 64]");
    if (d->top_k <= 0 || d->top_k > kMaxTopK || d->top_k > E)
        return fail(UOCR_HIP_EINVAL, "top_k must be in [1, min(8, n_experts)]");
    if (d->n_shared < 0 || E + d->n_shared > kMaxExperts) return fail(UOCR_HIP_EINVAL, "bad n_shared");
    if (!d->router_bf16 && !d->router_f32) return fail(UOCR_HIP_EINVAL, "null router pointer");
    const bool edense = d->gate_w || d->up_w || d->down_w;
    const int S = d->n_shared;
    const bool sdense = S > 0 && (d->shared_gate_w || d->shared_up_w || d->shared_down_w);
    if (edense) {
        if (d->gate || d->up || d->down)
            return fail(UOCR_HIP_EINVAL, "routed experts given both as INT4 and unquantised matrices");
        if (!d->gate_w || !d->up_w || !d->down_w) return fail(UOCR_HIP_EINVAL, "null expert weight pointer");
        if (S > 0 && !sdense)
            return fail(UOCR_HIP_EUNSUPPORTED, "unquantised routed experts need an unquantised shared MLP");
    } else if (!d->gate || !d->up || !d->down) {
        return fail(UOCR_HIP_EINVAL, "null weight pointer");
    }
    if (sdense && (d->shared_gate || d->shared_up || d->shared_down))
        return fail(UOCR_HIP_EINVAL, "shared MLP given both as INT4 and unquantised matrices");
    // group size of the INT4 matrices (unused when none is INT4)
    const int G = !edense ? d->gate[0].group_size : (S > 0 && !sdense ? d->shared_gate->group_size : 32);
    if (G != 32 && G != 64 && G != 128) return fail(UOCR_HIP_EUNSUPPORTED, "group_size must be 32, 64 or 128");
    int rc;
    for (int e = 0; e < E; ++e) {
        if (edense) {
            if ((rc = check_dense(&d->gate_w[e], I, H, "gate"))) return rc;
            if ((rc = check_dense(&d->up_w[e], I, H, "up"))) return rc;
            if ((rc = check_dense(&d->down_w[e], H, I, "down"))) return rc;
        } else {
            if ((rc = check_qm(&d->gate[e], I, H, G, "gate"))) return rc;
            if ((rc = check_qm(&d->up[e], I, H, G, "up"))) return rc;
            if ((rc = check_qm(&d->down[e], H, I, G, "down"))) return rc;
        }
    }
    if (S > 0) {
        if (sdense) {
            if ((rc = check_dense(d->shared_gate_w, S * I, H, "shared_gate"))) return rc;
            if ((rc = check_dense(d->shared_up_w, S * I, H, "shared_up"))) return rc;
            if ((rc = check_dense(d->shared_down_w, H, S * I, "shared_down"))) return rc;
        } else {
            if ((rc = check_qm(d->shared_gate, S * I, H, G, "shared_gate"))) return rc;
            if ((rc = check_qm(d->shared_up, S * I, H, G, "shared_up"))) return rc;
            if ((rc = check_qm(d->shared_down, H, S * I, G, "shared_down"))) return rc;
        }
    }
    // the unquantised kernels' decode tiles (every layer shape that passed the
    // checks above satisfies them; the prefill tiles fall back to these)
    if ((edense && !(dense_shapes_ok(H, I, true, kDenseSkinnyBM) && dense_shapes_ok(I, H, false, kDenseSkinnyBM))) ||
        (sdense && !(dense_shapes_ok(H, S * I, true, kDenseSkinnyBM) && dense_shapes_ok(S * I, H, false, kDenseSkinnyBM))))
        return fail(UOCR_HIP_EUNSUPPORTED, "unquantised matrix shapes not supported by this build");

    auto* L = new uocr_hip_moe_layer();
    L->hidden = H;
    L->inter = I;
    L->n_experts = E;
    L->top_k = d->top_k;
    // the shared MLP runs as virtual expert groups when it has the routed
    // experts' format (INT4 beside INT4, unquantised beside unquantised), as
    // its own stage (dense.hip) beside INT4 routed experts
    L->n_virtual = (sdense && !edense) ? 0 : S;
    L->shared_dense = sdense && !edense;
    L->experts_dense = edense;
    L->s_inter = S * I;
    L->group = G;
    L->norm_topk_prob = d->norm_topk_prob;
    L->scoring_sigmoid = d->scoring_sigmoid;
    L->scaling = d->routed_scaling_factor;
    L->rms_eps = d->rms_eps;
    (void)hipGetDevice(&L->device);

    const int Ev = edense ? 0 : E + L->n_virtual;  // INT4 groups to repack
    L->gu_wstride = (long long)I * H / 2;
    L->gu_sstride = (long long)I * scale_row_stride(H, G);
    L->dn_wstride = (long long)H * I / 2;
    L->dn_sstride = (long long)H * scale_row_stride(I, G);

    // zero points: one layout for the whole layer (implicit 8 unless any matrix
    // holds another zero)
    bool sym = true;
    {
        std::string err;
        auto scan = [&](const uocr_hip_qmatrix& q, const char* what) -> int {
            bool s1 = true;
            const int c = zero_kind(q, 0, q.rows, &s1, &err);
            if (c) return fail(c, std::string(what) + ": " + err);
            sym = sym && s1;
            return UOCR_HIP_OK;
        };
        for (int e = 0; e < (edense ? 0 : E); ++e)
            if ((rc = scan(d->gate[e], "gate")) || (rc = scan(d->up[e], "up")) || (rc = scan(d->down[e], "down"))) {
                delete L;
                return rc;
            }
        if (S > 0 && !sdense && ((rc = scan(*d->shared_gate, "shared_gate")) || (rc = scan(*d->shared_up, "shared_up")) ||
                      (rc = scan(*d->shared_down, "shared_down")))) {
            delete L;
            return rc;
        }
    }
    std::vector<uint8_t> hg((size_t)Ev * L->gu_wstride), hu(hg.size()), hd((size_t)Ev * L->dn_wstride);
    std::vector<uint16_t> hgs((size_t)Ev * L->gu_sstride), hus(hgs.size()), hds((size_t)Ev * L->dn_sstride);
    std::vector<uint16_t> hgz(sym ? 0 : hgs.size()), huz(hgz.size()), hdz(sym ? 0 : hds.size());
    auto zp = [&](std::vector<uint16_t>& v, long long off) -> uint16_t* { return v.empty() ? nullptr : &v[off]; };

    // repack experts in parallel (virtual experts E..E+S-1 are slices of the shared MLP)
    std::vector<int> codes(Ev, UOCR_HIP_OK);
    std::vector<std::string> errs(Ev);
    auto work = [&](int e) {
        std::string* err = &errs[e];
        const long long gw = e * L->gu_wstride, gs = e * L->gu_sstride, dw = e * L->dn_wstride, ds = e * L->dn_sstride;
        int c;
        if (e < E) {
            if ((c = repack(d->gate[e], 0, I, 0, H, &hg[gw], &hgs[gs], zp(hgz, gs), err))) goto done;
            if ((c = repack(d->up[e], 0, I, 0, H, &hu[gw], &hus[gs], zp(huz, gs), err))) goto done;
            c = repack(d->down[e], 0, H, 0, I, &hd[dw], &hds[ds], zp(hdz, ds), err);
        } else {
            const int v = e - E;
            if ((c = repack(*d->shared_gate, v * I, I, 0, H, &hg[gw], &hgs[gs], zp(hgz, gs), err))) goto done;
            if ((c = repack(*d->shared_up, v * I, I, 0, H, &hu[gw], &hus[gs], zp(huz, gs), err))) goto done;
            c = repack(*d->shared_down, 0, H, v * I, I, &hd[dw], &hds[ds], zp(hdz, ds), err);
        }
    done:
        codes[e] = c;
    };
    {
        const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        std::vector<std::thread> pool;
        for (unsigned w = 0; w < nt; ++w)
            pool.emplace_back([&, w] {
                for (int e = (int)w; e < Ev; e += (int)nt) work(e);
            });
        for (auto& th : pool) th.join();
    }
    for (int e = 0; e < Ev; ++e)
        if (codes[e]) {
            const std::string m = (e < E ? "expert " + std::to_string(e) : "shared expert") + ": " + errs[e];
            free_layer(L);
            return fail(codes[e], m);
        }

    // unquantised matrices -> f16 row-major
    std::vector<uint16_t> dsg, dsu, dsd, deg, deu, ded;
    {
        std::string err;
        auto conv = [&](const uocr_hip_dense_matrix& m, std::vector<uint16_t>& v, size_t off, const std::string& what) {
            const int c = dense_to_f16(m, v.data() + off, &err);
            if (c) fail(c, what + ": " + err);
            return c;
        };
        if (sdense) {
            dsg.resize((size_t)S * I * H);
            dsu.resize(dsg.size());
            dsd.resize(dsg.size());
            if ((rc = conv(*d->shared_gate_w, dsg, 0, "shared_gate")) || (rc = conv(*d->shared_up_w, dsu, 0, "shared_up")) ||
                (rc = conv(*d->shared_down_w, dsd, 0, "shared_down"))) {
                free_layer(L);
                return rc;
            }
        }
        if (edense) {
            // routed experts, then the shared MLP as S virtual groups of width
            // inter (gate / up rows v*I.., down columns v*I..), so the grouped
            // kernels run it as groups that see every token
            const size_t n = (size_t)I * H;
            deg.resize((size_t)(E + S) * n);
            deu.resize(deg.size());
            ded.resize(deg.size());
            for (int e = 0; e < E; ++e)
                if ((rc = conv(d->gate_w[e], deg, e * n, "expert " + std::to_string(e) + " gate")) ||
                    (rc = conv(d->up_w[e], deu, e * n, "expert " + std::to_string(e) + " up")) ||
                    (rc = conv(d->down_w[e], ded, e * n, "expert " + std::to_string(e) + " down"))) {
                    free_layer(L);
                    return rc;
                }
            if (S > 0) {
                std::copy(dsg.begin(), dsg.end(), deg.begin() + (size_t)E * n);
                std::copy(dsu.begin(), dsu.end(), deu.begin() + (size_t)E * n);
                for (int v = 0; v < S; ++v)
                    for (int h = 0; h < H; ++h)
                        std::copy(dsd.begin() + (size_t)h * S * I + (size_t)v * I,
                                  dsd.begin() + (size_t)h * S * I + (size_t)(v + 1) * I,
                                  ded.begin() + (size_t)(E + v) * n + (size_t)h * I);
                dsg.clear();
                dsu.clear();
                dsd.clear();
            }
        }
    }

    // router W (bf16) as [H/8][E][8] so lane e's 16-byte loads are coalesced
    // across the wave; an f32 router has no bf16 form (its layer takes the
    // f32-weight router on every path)
    std::vector<uint16_t> rt;
    if (!d->router_f32) {
        rt.resize((size_t)H * E);
        for (int c8 = 0; c8 < H / 8; ++c8)
            for (int e = 0; e < E; ++e)
                for (int i = 0; i < 8; ++i) rt[((size_t)c8 * E + e) * 8 + i] = d->router_bf16[(size_t)e * H + c8 * 8 + i];
    }

    // and as f32 [H/4][64][4] for the decode router (experts padded to 64 with
    // zeros, so a 64-column chunk is one contiguous 16 KiB block)
    std::vector<float> rf((size_t)H * 64, 0.0f);
    for (int c4 = 0; c4 < H / 4; ++c4)
        for (int e = 0; e < E; ++e)
            for (int i = 0; i < 4; ++i) {
                const size_t src = (size_t)e * H + c4 * 4 + i;
                float v;
                if (d->router_f32) {
                    v = d->router_f32[src];
                } else {
                    const uint32_t bits = (uint32_t)d->router_bf16[src] << 16;
                    std::memcpy(&v, &bits, 4);
                }
                rf[((size_t)c4 * 64 + e) * 4 + i] = v;
            }

    // down scales (and zero offsets) once more as [Ev][inter/128][hidden][128/group]
    // for the streamed decode kernel: an item (group, 128 inter columns) reads
    // its k-tile's scales of every hidden row as one contiguous block
    std::vector<uint16_t> hdsk, hdzk;
    if (Ev > 0 && decode_stream_ok(H, I, G)) {
        const int KTD = I / kTileK, GPT = kTileK / G, NGD = scale_row_stride(I, G);
        hdsk.resize((size_t)Ev * KTD * H * GPT);
        if (!sym) hdzk.resize(hdsk.size());
        for (int e = 0; e < Ev; ++e)
            for (int s = 0; s < KTD; ++s)
                for (int row = 0; row < H; ++row)
                    for (int gi = 0; gi < GPT; ++gi) {
                        const size_t dst = (((size_t)e * KTD + s) * H + row) * GPT + gi;
                        const size_t src = (size_t)e * L->dn_sstride + (size_t)row * NGD + s * GPT + gi;
                        hdsk[dst] = hds[src];
                        if (!sym) hdzk[dst] = hdz[src];
                    }
    }
    // streamed copy of the weights (see uocr_hip_moe_layer::sw): item
    // i = g * (inter/128) + s covers inter rows s*128.. of group g; its wave w
    // uses gate / up k-tiles kt of row block s*8 + w (units 2kt, 2kt + 1) and
    // the down tiles of row blocks w*NTD + j at k-tile s (units 2*KTG + j)
    std::vector<uint8_t> hsw;
    if (Ev > 0 && decode_stream_ok(H, I, G)) {
        constexpr int NW = 8;
        const int KTG = H / kTileK, KTD = I / kTileK, NS = KTD, NTD = H / kTileRows / NW;
        const int U = 2 * KTG + NTD;
        const size_t NI = (size_t)Ev * NS;
        hsw.resize((size_t)U * NI * NW * kTileBytes);
        for (size_t i = 0; i < NI; ++i) {
            const int g = (int)(i / NS), s = (int)(i % NS);
            for (int w = 0; w < NW; ++w)
                for (int u = 0; u < U; ++u) {
                    const uint8_t* src;
                    if (u < 2 * KTG) {
                        const int kt = u / 2, rb = s * NW + w;
                        const std::vector<uint8_t>& m = (u & 1) ? hu : hg;
                        src = &m[(size_t)g * L->gu_wstride + ((size_t)rb * KTG + kt) * kTileBytes];
                    } else {
                        const int j = u - 2 * KTG, rb = w * NTD + j;
                        src = &hd[(size_t)g * L->dn_wstride + ((size_t)rb * KTD + s) * kTileBytes];
                    }
                    std::memcpy(&hsw[(((size_t)u * NI + i) * NW + w) * kTileBytes], src, kTileBytes);
                }
        }
    }
    auto up_copy = [&](void** dst, const void* src, size_t bytes, const char* what) -> int {
        hipError_t e = hipMalloc(dst, bytes);
        if (e != hipSuccess) return fail(UOCR_HIP_ENOMEM, std::string("hipMalloc(") + what + "): " + hipGetErrorString(e));
        e = hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(e, what);
        L->device_bytes += bytes;
        return UOCR_HIP_OK;
    };
    const bool int4 = Ev > 0;
    if ((!rt.empty() && (rc = up_copy((void**)&L->router_t, rt.data(), rt.size() * 2, "router"))) ||
        (rc = up_copy((void**)&L->router_f32, rf.data(), rf.size() * 4, "router f32")) ||
        (int4 && (rc = up_copy((void**)&L->gate, hg.data(), hg.size(), "gate"))) ||
        (int4 && (rc = up_copy((void**)&L->up, hu.data(), hu.size(), "up"))) ||
        (int4 && (rc = up_copy((void**)&L->down, hd.data(), hd.size(), "down"))) ||
        (int4 && (rc = up_copy((void**)&L->gate_s, hgs.data(), hgs.size() * 2, "gate scales"))) ||
        (int4 && (rc = up_copy((void**)&L->up_s, hus.data(), hus.size() * 2, "up scales"))) ||
        (int4 && (rc = up_copy((void**)&L->down_s, hds.data(), hds.size() * 2, "down scales"))) ||
        (!hdsk.empty() && (rc = up_copy((void**)&L->down_skt, hdsk.data(), hdsk.size() * 2, "down scales (k-tile order)"))) ||
        (!hsw.empty() && (rc = up_copy((void**)&L->sw, hsw.data(), hsw.size(), "streamed weights"))) ||
        (!hdzk.empty() && (rc = up_copy((void**)&L->down_zkt, hdzk.data(), hdzk.size() * 2, "down zeros (k-tile order)"))) ||
        (L->shared_dense && (rc = up_copy((void**)&L->sgate, dsg.data(), dsg.size() * 2, "shared gate"))) ||
        (L->shared_dense && (rc = up_copy((void**)&L->sup, dsu.data(), dsu.size() * 2, "shared up"))) ||
        (L->shared_dense && (rc = up_copy((void**)&L->sdown, dsd.data(), dsd.size() * 2, "shared down"))) ||
        (edense && (rc = up_copy((void**)&L->egate, deg.data(), deg.size() * 2, "expert gate"))) ||
        (edense && (rc = up_copy((void**)&L->eup, deu.data(), deu.size() * 2, "expert up"))) ||
        (edense && (rc = up_copy((void**)&L->edown, ded.data(), ded.size() * 2, "expert down"))) ||
        (int4 && !sym && (rc = up_copy((void**)&L->gate_z, hgz.data(), hgz.size() * 2, "gate zeros"))) ||
        (int4 && !sym && (rc = up_copy((void**)&L->up_z, huz.data(), huz.size() * 2, "up zeros"))) ||
        (int4 && !sym && (rc = up_copy((void**)&L->down_z, hdz.data(), hdz.size() * 2, "down zeros"))) ||
        (d->rms_weight && (rc = up_copy((void**)&L->rms_weight, d->rms_weight, (size_t)H * 4, "rms weight")))) {
        free_layer(L);
        return rc;
    }
    {
        void* sp = nullptr;  // device address of the no-alloc scratch on this device
        if ((rc = scratch_ptr(L->device, &sp))) {
            free_layer(L);
            return rc;
        }
    }
    {
        // [0]: the fused decode kernel (its error word is the layer's status
        // word), [1]: the streamed decode kernel, [2]: its wide mode (own
        // progress words and candidate tags each, so that calls may switch
        // between kernels and modes, whose grids differ)
        hipError_t e = hipMalloc((void**)&L->sync, 3 * sizeof(FusedSync));
        if (e == hipSuccess) e = hipMemset(L->sync, 0, 3 * sizeof(FusedSync));
        if (e != hipSuccess) {
            free_layer(L);
            return hip_fail(e, "fused work queue");
        }
        L->device_bytes += 3 * sizeof(FusedSync);
    }
    *out = L;
    return UOCR_HIP_OK;
}

int uocr_hip_moe_layer_destroy(uocr_hip_moe_layer* layer) {
    free_layer(layer);
    return UOCR_HIP_OK;
}

size_t uocr_hip_moe_layer_device_bytes(const uocr_hip_moe_layer* layer) {
    return layer ? layer->device_bytes : 0;
}

size_t uocr_hip_moe_layer_workspace_size(const uocr_hip_moe_layer* layer, int seq) {
    if (!layer || seq <= 0) return 0;
    if (uses_grouping(layer, seq) && !group_fits(seq, layer->top_k, layer->n_experts)) return 0;
    return plan(layer, seq).total;
}

int uocr_hip_moe_layer_path(const uocr_hip_moe_layer* layer, int seq) {
    return (layer && use_prefill(layer, seq)) ? 1 : 0;
}

int uocr_hip_moe_layer_status(uocr_hip_moe_layer* L, int clear, int* flags) {
    if (!L || !flags) return fail(UOCR_HIP_EINVAL, "null argument");
    *flags = 0;
    if (!L->sync) return UOCR_HIP_OK;
    HIP_TRY(hipDeviceSynchronize(), "status sync");
    HIP_TRY(hipMemcpy(flags, &L->sync->error, sizeof(int), hipMemcpyDeviceToHost), "status read");
    if (clear) HIP_TRY(hipMemset(&L->sync->error, 0, sizeof(int)), "status clear");
    return UOCR_HIP_OK;
}

int uocr_hip_moe_layer_status_async(const uocr_hip_moe_layer* L, int* d_flags, void* stream) {
    if (!L || !d_flags) return fail(UOCR_HIP_EINVAL, "null argument");
    hipStream_t st = (hipStream_t)stream;
    if (!L->sync) {
        HIP_TRY(hipMemsetAsync(d_flags, 0, sizeof(int), st), "status copy");
        return UOCR_HIP_OK;
    }
    HIP_TRY(hipMemcpyAsync(d_flags, &L->sync->error, sizeof(int), hipMemcpyDeviceToDevice, st), "status copy");
    return UOCR_HIP_OK;
}

int uocr_hip_moe_layer_forward(const uocr_hip_moe_layer* L, const void* x, int x_dtype, int seq,
                               float* out, int* ids_out, float* weights_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
    if (!L || !x || !out) return fail(UOCR_HIP_EINVAL, "null argument");
    if (seq <= 0) return fail(UOCR_HIP_EINVAL, "seq must be positive");
    if (x_dtype != UOCR_HIP_DTYPE_BF16 && x_dtype != UOCR_HIP_DTYPE_F32) return fail(UOCR_HIP_EINVAL, "bad x_dtype");
    if (L->rms_weight && x_dtype != UOCR_HIP_DTYPE_F32)
        return fail(UOCR_HIP_EINVAL, "a layer with rms_weight adds the residual and needs f32 x");
    if ((uintptr_t)x % 16 || (uintptr_t)out % 16) return fail(UOCR_HIP_EINVAL, "x and out must be 16-byte aligned");
    if (uses_grouping(L, seq) && !group_fits(seq, L->top_k, L->n_experts))
        return fail(UOCR_HIP_EUNSUPPORTED, "seq * top_k too large for the grouping scan (" + std::to_string(seq) +
                                               " tokens)");
    const WsPlan p = plan(L, seq);
    if (!workspace || workspace_bytes < p.total)
        return fail(UOCR_HIP_EWORKSPACE, "workspace too small: need " + std::to_string(p.total) + " bytes");
    if ((uintptr_t)workspace % 256) return fail(UOCR_HIP_EINVAL, "workspace must be 256-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    int* ids = ids_out ? ids_out : (int*)(ws + p.ids);
    float* wts = weights_out ? weights_out : (float*)(ws + p.wts);
    f16* x16 = (f16*)(ws + p.x16);
    auto* Lm = const_cast<uocr_hip_moe_layer*>(L);
    const bool timing = L->timing;
    // stages: 0 router, 1 grouping, 2 gate/up, 3 down, 4 combine, 5 fused
    // decode kernel; stage(-1) ends timing
    if (timing) Lm->stage_mask = 0;
    // a stage counts once a launch has consumed its start event
    int cur_stage = -1;
    auto stage = [&](int i) {
        if (!timing) return;
        if (cur_stage >= 0 && !stage_events().start) Lm->stage_mask |= 1u << cur_stage;
        stage_events() = i < 0 ? StageEvents{} : StageEvents{Lm->ev[2 * i], Lm->ev[2 * i + 1]};
        cur_stage = i;
    };

    struct Disarm {  // an early error return must not leave later launches armed
        ~Disarm() { stage_events() = StageEvents{}; }
    } disarm_on_exit;
    // the unquantised shared MLP (dense.hip): act then y_shared [seq, hidden]
    // f32, added by the combine after the routed sum (moe_decoder.cpp:110-112)
    const float* shared_y = nullptr;
    auto run_shared = [&](const void* src, int kind) -> int {
        if (!L->shared_dense) return UOCR_HIP_OK;
        const int bm = dense_shared_bm(L, seq);
        stage(6);
        DenseArgs sa{};
        sa.a = src;
        sa.a_kind = kind;
        sa.w0 = L->sgate;
        sa.w1 = L->sup;
        sa.n_out = L->s_inter;
        sa.k = L->hidden;
        sa.seq = seq;
        sa.out16 = (f16*)(ws + p.sact);
        sa.status = &L->sync->error;
        // the 128-slot tiles take f16 input only
        HIP_TRY(launch_dense(sa, true, kind == 0 ? bm : kDenseSkinnyBM, 0, st), "shared gate/up launch");
        DenseArgs sd{};
        sd.a = sa.out16;
        sd.a_kind = 0;
        sd.w0 = L->sdown;
        sd.n_out = L->hidden;
        sd.k = L->s_inter;
        sd.seq = seq;
        sd.out32 = (float*)(ws + p.sy);
        HIP_TRY(launch_dense(sd, false, bm, 0, st), "shared down launch");
        shared_y = sd.out32;
        return UOCR_HIP_OK;
    };
    int rc;
    stage(0);
    if (!uses_grouping(L, seq)) {
        DecodeArgs da{};
        da.x = x;
        da.x_bf16 = x_dtype == UOCR_HIP_DTYPE_BF16;
        da.seq = seq;
        da.hidden = L->hidden;
        da.inter = L->inter;
        da.n_experts = L->n_experts;
        da.top_k = L->top_k;
        da.n_virtual = L->n_virtual;
        da.group = L->group;
        da.rms_weight = L->rms_weight;
        da.rms_eps = L->rms_eps;
        da.router_f32 = L->router_f32;
        da.router_unfused = L->router_t == nullptr;
        da.router_t = L->router_t;
        da.norm_topk_prob = L->norm_topk_prob;
        da.scoring_sigmoid = L->scoring_sigmoid;
        da.scaling = L->scaling;
        da.x16 = x16;
        da.ids = ids;
        da.wts = wts;
        da.gate = L->gate;
        da.up = L->up;
        da.down = L->down;
        da.gate_s = L->gate_s;
        da.up_s = L->up_s;
        da.down_s = L->down_s;
        da.gate_z = L->gate_z;
        da.up_z = L->up_z;
        da.down_z = L->down_z;
        da.gu_wstride = L->gu_wstride;
        da.gu_sstride = L->gu_sstride;
        da.dn_wstride = L->dn_wstride;
        da.dn_sstride = L->dn_sstride;
        da.act = (f16*)(ws + p.act);
        da.y = (float*)(ws + p.y);
        da.out = out;
        da.status = &L->sync->error;
        if (use_stream(L, seq, x_dtype)) {
            da.sync = L->sync + (stream_wide(L, seq, x_dtype) ? 2 : 1);
            da.down_skt = L->down_skt;
            da.sw = L->sw;
            da.down_zkt = L->down_zkt;
            if (L->shared_dense && (x_dtype != UOCR_HIP_DTYPE_BF16 || L->rms_weight)) {
                stage(6);
                HIP_TRY(launch_x16_prep(x, x_dtype == UOCR_HIP_DTYPE_BF16, L->rms_weight, L->rms_eps, seq, L->hidden,
                                        x16, st),
                        "shared-MLP input launch");
                if ((rc = run_shared(x16, 0))) return rc;
            } else if ((rc = run_shared(x, 1))) {
                return rc;
            }
            da.shared_y = shared_y;
            stage(5);
            HIP_TRY(launch_decode_stream(da, st), "streamed decode launch");
            stage(-1);
            if (timing) Lm->pending = true;
            return UOCR_HIP_OK;
        }
        if (use_fused(L, seq, x_dtype)) {
            da.sync = L->sync;
            if ((rc = run_shared(x, 1))) return rc;
            da.shared_y = shared_y;
            stage(5);
            HIP_TRY(launch_decode_fused(da, st), "fused decode launch");
            stage(-1);
            if (timing) Lm->pending = true;
            return UOCR_HIP_OK;
        }
        if (seq <= kRouterDecodeMaxSeq || !L->router_t) {
            HIP_TRY(launch_router_decode(da, st), "router launch");
        } else {
            RouterArgs ra{};
            ra.x = x;
            ra.seq = seq;
            ra.hidden = L->hidden;
            ra.n_experts = L->n_experts;
            ra.top_k = L->top_k;
            ra.rms_weight = L->rms_weight;
            ra.rms_eps = L->rms_eps;
            ra.router_t = L->router_t;
    ra.router_f32 = L->router_f32;
            ra.norm_topk_prob = L->norm_topk_prob;
            ra.scoring_sigmoid = L->scoring_sigmoid;
            ra.scaling = L->scaling;
            ra.x16 = x16;
            ra.ids = ids;
            ra.weights = wts;
            HIP_TRY(launch_router(ra, x_dtype == UOCR_HIP_DTYPE_BF16, st), "router launch");
        }
        if ((rc = run_shared(x16, 0))) return rc;
        da.shared_y = shared_y;
        stage(2);
        HIP_TRY(launch_experts_decode2(da, true, st), "gate/up launch");
        stage(3);
        HIP_TRY(launch_experts_decode2(da, false, st), "down launch");
        stage(4);
        HIP_TRY(launch_combine_decode(da, st), "combine launch");
        stage(-1);
        if (timing) Lm->pending = true;
        return UOCR_HIP_OK;
    }
    RouterArgs ra{};
    ra.x = x;
    ra.seq = seq;
    ra.hidden = L->hidden;
    ra.n_experts = L->n_experts;
    ra.top_k = L->top_k;
    ra.rms_weight = L->rms_weight;
    ra.rms_eps = L->rms_eps;
    ra.router_t = L->router_t;
    ra.router_f32 = L->router_f32;
    ra.norm_topk_prob = L->norm_topk_prob;
    ra.scoring_sigmoid = L->scoring_sigmoid;
    ra.scaling = L->scaling;
    ra.x16 = x16;
    ra.ids = ids;
    ra.weights = wts;

    GroupArgs g{};
    g.ids = ids;
    g.weights = wts;
    g.seq = seq;
    g.top_k = L->top_k;
    g.n_experts = L->n_experts;
    g.n_virtual = L->n_virtual;
    g.bm = p.bm;
    g.counts = (int*)(ws + p.counts);
    g.offsets = (int*)(ws + p.offsets);
    g.slot_tok = (int*)(ws + p.slot_tok);
    g.slot_w = (float*)(ws + p.slot_w);
    g.pos = (int*)(ws + p.pos);
    g.tile_e = (int*)(ws + p.tile_e);
    g.tile_m0 = (int*)(ws + p.tile_m0);
    g.tile_info = (int*)(ws + p.tile_info);
    g.n_tiles = (int*)(ws + p.ntiles);
    g.lrank = (int*)(ws + p.lrank);
    g.chunk_count = (int*)(ws + p.chunk_count);
    g.chunk_base = (int*)(ws + p.chunk_base);
    if (L->router_t && seq > kRouterDecodeMaxSeq) {
        HIP_TRY(launch_router(ra, x_dtype == UOCR_HIP_DTYPE_BF16, st), "router launch");
    } else {
        // f32 router, or few tokens: the per-token router (same outputs)
        DecodeArgs da{};
        da.x = x;
        da.x_bf16 = x_dtype == UOCR_HIP_DTYPE_BF16;
        da.seq = seq;
        da.hidden = L->hidden;
        da.inter = L->inter;
        da.n_experts = L->n_experts;
        da.top_k = L->top_k;
        da.n_virtual = L->n_virtual;
        da.group = L->group;
        da.rms_weight = L->rms_weight;
        da.rms_eps = L->rms_eps;
        da.router_f32 = L->router_f32;
        da.router_unfused = L->router_t == nullptr;
        da.norm_topk_prob = L->norm_topk_prob;
        da.scoring_sigmoid = L->scoring_sigmoid;
        da.scaling = L->scaling;
        da.x16 = x16;
        da.ids = ids;
        da.wts = wts;
        HIP_TRY(launch_router_decode(da, st), "router launch");
    }
    stage(1);
    HIP_TRY(launch_group(g, st), "group launch");
    stage(2);
    const f16* y16 = (const f16*)(ws + p.y);
    if (L->experts_dense && p.bm == kPrefillBigTileRows) {
        ExpertArgs gu{};
        gu.a = x16;
        gu.gather = 1;
        gu.w0 = reinterpret_cast<const uint8_t*>(L->egate);
        gu.w1 = reinterpret_cast<const uint8_t*>(L->eup);
        gu.w_stride = (long long)L->inter * L->hidden * 2;
        gu.n_rows = L->inter;
        gu.k = L->hidden;
        gu.bm = p.bm;
        gu.slot_tok = g.slot_tok;
        gu.counts = g.counts;
        gu.offsets = g.offsets;
        gu.tile_e = g.tile_e;
        gu.tile_m0 = g.tile_m0;
        gu.tile_info = g.tile_info;
        gu.n_tiles = g.n_tiles;
        gu.act_out = (f16*)(ws + p.act);
        gu.status = &L->sync->error;
        HIP_TRY(launch_experts_prefill_dense(gu, true, p.max_tiles, st), "gate/up launch");
        stage(3);
        ExpertArgs dn = gu;
        dn.a = gu.act_out;
        dn.gather = 0;
        dn.w0 = reinterpret_cast<const uint8_t*>(L->edown);
        dn.w1 = nullptr;
        dn.n_rows = L->hidden;
        dn.k = L->inter;
        dn.act_out = nullptr;
        dn.y_out = (f16*)(ws + p.y);
        HIP_TRY(launch_experts_prefill_dense(dn, false, p.max_tiles, st), "down launch");
    } else if (L->experts_dense) {
        DenseArgs gu{};
        gu.a = x16;
        gu.a_kind = 0;
        gu.slot_tok = g.slot_tok;
        gu.w0 = L->egate;
        gu.w1 = L->eup;
        gu.w_stride = (long long)L->inter * L->hidden;
        gu.n_out = L->inter;
        gu.k = L->hidden;
        gu.tile_info = g.tile_info;
        gu.n_tiles = g.n_tiles;
        gu.seq = seq;
        gu.out16 = (f16*)(ws + p.act);
        gu.status = &L->sync->error;
        HIP_TRY(launch_dense(gu, true, p.bm, p.max_tiles, st), "gate/up launch");
        stage(3);
        DenseArgs dn = gu;
        dn.a = gu.out16;
        dn.slot_tok = nullptr;
        dn.w0 = L->edown;
        dn.w1 = nullptr;
        dn.n_out = L->hidden;
        dn.k = L->inter;
        dn.out16 = (f16*)(ws + p.y);
        HIP_TRY(launch_dense(dn, false, p.bm, p.max_tiles, st), "down launch");
    } else {
    ExpertArgs gu{};
    gu.a = x16;
    gu.gather = 1;
    gu.w0 = L->gate;
    gu.s0 = L->gate_s;
    gu.w1 = L->up;
    gu.s1 = L->up_s;
    gu.z0 = L->gate_z;
    gu.z1 = L->up_z;
    gu.w_stride = L->gu_wstride;
    gu.s_stride = L->gu_sstride;
    gu.n_rows = L->inter;
    gu.k = L->hidden;
    gu.group = L->group;
    gu.bm = p.bm;
    gu.slot_tok = g.slot_tok;
    gu.counts = g.counts;
    gu.offsets = g.offsets;
    gu.tile_e = g.tile_e;
    gu.tile_m0 = g.tile_m0;
    gu.tile_info = g.tile_info;
    gu.n_tiles = g.n_tiles;
    gu.act_out = (f16*)(ws + p.act);
    gu.status = &L->sync->error;
    HIP_TRY(launch_experts_prefill(gu, true, p.max_tiles, st),
            "gate/up launch");
    stage(3);

    ExpertArgs dn = gu;
    dn.a = gu.act_out;
    dn.gather = 0;
    dn.w0 = L->down;
    dn.s0 = L->down_s;
    dn.w1 = nullptr;
    dn.s1 = nullptr;
    dn.z0 = L->down_z;
    dn.z1 = nullptr;
    dn.w_stride = L->dn_wstride;
    dn.s_stride = L->dn_sstride;
    dn.n_rows = L->hidden;
    dn.k = L->inter;
    dn.act_out = nullptr;
    dn.y_out = (f16*)(ws + p.y);
    HIP_TRY(launch_experts_prefill(dn, false, p.max_tiles, st),
            "down launch");
    }
    if ((rc = run_shared(x16, 0))) return rc;
    stage(4);

    CombineArgs c{};
    c.y = y16;
    c.shared_y = shared_y;
    c.pos = g.pos;
    c.weights = wts;
    c.offsets = g.offsets;
    c.residual = L->rms_weight ? (const float*)x : nullptr;
    c.out = out;
    c.seq = seq;
    c.hidden = L->hidden;
    c.top_k = L->top_k;
    c.n_experts = L->n_experts;
    c.n_virtual = L->n_virtual;
    HIP_TRY(launch_combine(c, st), "combine launch");
    stage(-1);
    if (timing) Lm->pending = true;
    return UOCR_HIP_OK;
}

int uocr_hip_moe_layer_forward_noalloc(const uocr_hip_moe_layer* L, const void* x, int x_dtype, int seq, float* out,
                                       int* ids_out, float* weights_out, void* stream) {
    if (!L) return fail(UOCR_HIP_EINVAL, "null argument");
    if (seq <= 0) return fail(UOCR_HIP_EINVAL, "seq must be positive");
    const size_t need = uocr_hip_moe_layer_workspace_size(L, seq);
    if (need == 0 || need > kScratchBytes)
        return fail(UOCR_HIP_EINVAL, "seq " + std::to_string(seq) + " needs " + std::to_string(need) +
                                         " bytes of workspace; the no-alloc scratch holds " +
                                         std::to_string(kScratchBytes) + " (use uocr_hip_moe_layer_forward)");
    void* ws = nullptr;
    int rc = scratch_ptr(L->device, &ws);
    if (rc) return rc;
    return uocr_hip_moe_layer_forward(L, x, x_dtype, seq, out, ids_out, weights_out, ws, kScratchBytes, stream);
}

int uocr_hip_moe_layer_set_decode_kernel(uocr_hip_moe_layer* L, int kind) {
    if (!L) return fail(UOCR_HIP_EINVAL, "null layer");
    if (kind < UOCR_HIP_DECODE_AUTO || kind > UOCR_HIP_DECODE_FOUR_LAUNCH)
        return fail(UOCR_HIP_EINVAL, "unknown decode kernel choice");
    L->decode_kernel = kind;
    return UOCR_HIP_OK;
}

int uocr_hip_moe_layer_decode_kernel(const uocr_hip_moe_layer* L, int seq, int x_dtype) {
    if (!L || seq <= 0) return -1;
    if (uses_grouping(L, seq)) return -1;
    if (use_stream(L, seq, x_dtype)) return UOCR_HIP_DECODE_STREAM;
    if (use_fused(L, seq, x_dtype)) return UOCR_HIP_DECODE_FUSED;
    return UOCR_HIP_DECODE_FOUR_LAUNCH;
}

int uocr_hip_moe_layer_set_timing(uocr_hip_moe_layer* L, int enable) {
    if (!L) return fail(UOCR_HIP_EINVAL, "null layer");
    if (enable && !L->ev[0])
        // no system-scope fence: a fenced event adds microseconds of cache
        // maintenance to the interval it closes
        for (auto& e : L->ev) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreate");
    L->timing = enable != 0;
    return UOCR_HIP_OK;
}

int uocr_hip_moe_layer_read_timing(uocr_hip_moe_layer* L, float* stage_ms, int n_stages, int* n_calls) {
    if (!L || !stage_ms) return fail(UOCR_HIP_EINVAL, "null argument");
    if (L->pending) {
        for (int i = 0; i < kStages; ++i) {
            if (!(L->stage_mask >> i & 1)) continue;
            float ms = 0.0f;
            HIP_TRY(hipEventSynchronize(L->ev[2 * i + 1]), "hipEventSynchronize");
            HIP_TRY(hipEventElapsedTime(&ms, L->ev[2 * i], L->ev[2 * i + 1]), "hipEventElapsedTime");
            L->stage_ms[i] += ms;
        }
        L->timed_calls++;
        L->pending = false;
    }
    for (int i = 0; i < n_stages && i < kStages; ++i) stage_ms[i] = L->stage_ms[i];
    if (n_calls) *n_calls = L->timed_calls;
    std::memset(L->stage_ms, 0, sizeof(L->stage_ms));
    L->timed_calls = 0;
    return UOCR_HIP_OK;
}

int uocr_hip_moe_router_overflow(int clear, int* flag) {
    if (!flag) return fail(UOCR_HIP_EINVAL, "null argument");
    HIP_TRY(router_overflow_read(clear, flag), "router overflow flag");
    return UOCR_HIP_OK;
}

int uocr_hip_moe_router_topk(const float* logits, int seq, int n_experts, int top_k, int norm_topk_prob,
                             float scaling, int scoring_sigmoid, int* d_ids, float* d_weights,
                             int* d_assign_token, float* d_assign_w, int* d_count, int cap, void* stream) {
    if (seq == 0 || n_experts == 0) return UOCR_HIP_OK;  // reference: early return (moe_device.cu:275)
    if (!logits || !d_ids || !d_weights || !d_assign_token || !d_assign_w || !d_count)
        return fail(UOCR_HIP_EINVAL, "null argument");
    if (seq < 0 || n_experts < 0 || n_experts > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > n_experts ||
        cap <= 0)
        return fail(UOCR_HIP_EINVAL, "bad shape (n_experts <= 128, 1 <= top_k <= min(8, n_experts), cap > 0)");
    hipStream_t st = (hipStream_t)stream;
    RouterArgs ra{};
    ra.seq = seq;
    ra.n_experts = n_experts;
    ra.top_k = top_k;
    ra.norm_topk_prob = norm_topk_prob;
    ra.scoring_sigmoid = scoring_sigmoid;
    ra.scaling = scaling;
    ra.ids = d_ids;
    ra.weights = d_weights;
    HIP_TRY(launch_router_from_logits(ra, logits, st), "router launch");
    GroupArgs g{};
    g.ids = d_ids;
    g.weights = d_weights;
    g.seq = seq;
    g.top_k = top_k;
    g.n_experts = n_experts;
    g.bm = 1;
    g.assign_token = d_assign_token;
    g.assign_w = d_assign_w;
    g.assign_count = d_count;
    g.cap = cap;
    HIP_TRY(launch_group_mirror(g, st), "group launch");
    return UOCR_HIP_OK;
}

// Host replay of the fused decode kernel's schedule (FusedSchedule, the same
// code the kernel runs): every workgroup's program as a sequence of waits and
// progress publishes -- routers publish once; workers publish one step per
// gate/up item, then wait for and publish each down item, then wait for their
// combine blocks -- executed until no workgroup can move. Fails if a workgroup
// is left waiting (a cycle or an unreachable step), if an item is published by
// another workgroup or at another step than gu_step / dn_step name, or if the
// slot mapping is not a bijection.
int uocr_hip_fused_schedule_check(int seq, int grid, int n_groups, int rbg, int rbd, const int* live, int n_live) {
    using uocr_hip::FusedSchedule;
    if (seq < 1 || grid <= seq + 1 || n_groups < 1 || rbg < 1 || rbd < 1 || n_live < 0 || n_live > n_groups ||
        (n_live > 0 && !live))
        return fail(UOCR_HIP_EINVAL, "bad schedule shape");
    const FusedSchedule sch(seq, grid, n_groups, rbg, rbd, n_live);
    const int T = seq, P = grid;
    for (int b = 0; b < P; ++b)
        if (sch.slot_of(b) < 0 || sch.slot_of(b) >= P || sch.slot_wg(sch.slot_of(b)) != b)
            return fail(UOCR_HIP_EINVAL, "slot mapping is not a bijection at workgroup " + std::to_string(b));
    struct Act {
        std::vector<std::pair<int, int>> waits;  // (owner, step)
        int kind, item;                          // kind 0 router, 1 gate/up, 2 down, 3 combine (no publish)
    };
    std::vector<std::vector<Act>> prog(P);
    for (int b = 0; b < P; ++b) {
        auto& pr = prog[b];
        if (b < T) pr.push_back({{}, 0, b});
        for (int i = b - T; b >= T && i < sch.ngu_total; i += sch.PW) pr.push_back({{}, 1, i});
        for (int j = sch.slot_of(b); j < sch.ndn_total; j += P) {
            Act a{{}, 2, j};
            for (int q = 0; q < rbg; ++q) {
                int o = 0, st = 0;
                sch.gu_step(live[j / rbd] * rbg + q, o, st);
                a.waits.push_back({o, st});
            }
            pr.push_back(a);
        }
        for (int rb = 0; rb < rbd; ++rb) {
            if (sch.combine_slot(rb) != sch.slot_of(b)) continue;
            Act a{{}, 3, rb};
            for (int q = 0; q < T; ++q) a.waits.push_back({q, 1});
            for (int q = 0; q < n_live; ++q) {
                int o = 0, st = 0;
                sch.dn_step(q * rbd + rb, o, st);
                a.waits.push_back({o, st});
            }
            pr.push_back(a);
        }
        int n_gu = 0;
        for (const Act& a : pr) n_gu += a.kind == 1;
        if (n_gu != sch.n_gu_of(b))
            return fail(UOCR_HIP_EINVAL, "n_gu_of disagrees with the items of workgroup " + std::to_string(b));
    }
    std::vector<int> done(P, 0), pc(P, 0);
    for (bool moved = true; moved;) {
        moved = false;
        for (int b = 0; b < P; ++b) {
            while (pc[b] < (int)prog[b].size()) {
                const Act& a = prog[b][pc[b]];
                bool ok = true;
                for (const auto& w : a.waits) ok = ok && w.first >= 0 && w.first < P && done[w.first] >= w.second;
                if (!ok) break;
                if (a.kind != 3) {
                    ++done[b];
                    int o = b, st = done[b];
                    if (a.kind == 1) sch.gu_step(a.item, o, st);
                    if (a.kind == 2) sch.dn_step(a.item, o, st);
                    if (a.kind == 0 && st != 1) o = -1;
                    if (o != b || st != done[b])
                        return fail(UOCR_HIP_EINVAL, "item " + std::to_string(a.item) + " (kind " +
                                                         std::to_string(a.kind) + ") published by workgroup " +
                                                         std::to_string(b) + " at step " + std::to_string(done[b]) +
                                                         ", the schedule names " + std::to_string(o) + " / " +
                                                         std::to_string(st));
                }
                ++pc[b];
                moved = true;
            }
        }
    }
    for (int b = 0; b < P; ++b)
        if (pc[b] < (int)prog[b].size())
            return fail(UOCR_HIP_EINVAL, "workgroup " + std::to_string(b) + " is left waiting (item kind " +
                                             std::to_string(prog[b][pc[b]].kind) + ")");
    return UOCR_HIP_OK;
}

}  // extern "C"
