// Kernel argument blocks and host-side launchers (internal to libuocr_hip).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include <string>

#include "common.hpp"

namespace uocr_hip {

// Per-stage kernel timing. While a stage is armed, every launch goes through
// hipExtLaunchKernelGGL, which stamps the kernel's own dispatch: the start
// event on the stage's first launch, the stop event on each launch (the last
// one wins). These are the timestamps a kernel trace reports, without the
// gaps that separate hipEventRecord markers add. Unarmed launches are plain.
struct StageEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
StageEvents& stage_events();  // thread-local

template <typename F, typename... Args>
inline void launch_k(F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t st, Args... args) {
    StageEvents& ev = stage_events();
    if (ev.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, lds, st, ev.start, ev.stop, 0, args...);
        ev.start = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    }
}

constexpr int kMaxExperts = 128;  // routed + virtual (shared-expert) groups
constexpr int kMaxTopK = 8;

struct RouterArgs {
    const void* x;            // [seq, hidden] bf16 bits or f32
    int seq, hidden, n_experts, top_k;
    const float* rms_weight;  // optional [hidden]
    float rms_eps;
    const uint16_t* router_t; // router W as [hidden/8][n_experts][8] bf16
    const float* router_f32;  // the same W as f32 [hidden/4][64][4] (experts padded to 64), or null
    int norm_topk_prob, scoring_sigmoid;
    float scaling;
    f16* x16;                 // out [seq, hidden] f16 expert input
    int* ids;                 // out [seq, top_k]
    float* weights;           // out [seq, top_k]
};

struct GroupArgs {
    const int* ids;
    const float* weights;
    int seq, top_k, n_experts, n_virtual, bm;
    // grouped-slot outputs (fused layer path); any may be null
    int* counts;     // [n_experts + n_virtual]
    int* offsets;    // [n_experts + n_virtual + 1]
    int* slot_tok;   // [slots]
    float* slot_w;   // [slots]
    int* pos;        // [seq * top_k] slot of entry (t, j)
    int* tile_e;     // [max tiles]
    int* tile_m0;    // [max tiles]
    int* tile_info;  // [max tiles][4]: e, m0, rows, first slot (16-byte aligned)
    int* n_tiles;    // [1]
    // reference [n_experts, cap] assignment tables (moe_router_topk mirror)
    int* assign_token;
    float* assign_w;
    int* assign_count;
    int cap;
    // multi-workgroup grouping scratch (seq * top_k > 1024); null = single workgroup
    int* lrank;        // [seq * top_k]
    int* chunk_count;  // [chunks * n_experts]
    int* chunk_base;   // [chunks * n_experts]
};

// Grouped INT4 expert GEMM over the tile-16x128 device layout.
struct ExpertArgs {
    const f16* a;            // activations: x16 [seq, K] (gathered via slot_tok) or act [slots, K]
    int gather;              // 1: row = slot_tok[slot], 0: row = slot
    const uint8_t* w0;       // packed weights, per expert stride w_stride bytes (gate or down)
    const uint16_t* s0;      // f16 scales, per expert stride s_stride elements
    const uint8_t* w1;       // second matrix (up) for the fused gate/up pass, else null
    const uint16_t* s1;
    const uint16_t* z0;      // zero offsets in the scale layout (null: symmetric layer)
    const uint16_t* z1;
    long long w_stride, s_stride;
    int n_rows;              // output features (N)
    int k;                   // input features (K)
    int group;
    int bm;                  // slots per m-tile of the tile list
    const int* slot_tok;
    const int* counts;
    const int* offsets;
    const int* tile_e;
    const int* tile_m0;
    const int* tile_info;    // [max tiles][4]: e, m0, rows, first slot
    const int* n_tiles;
    f16* act_out;            // gate/up: [slots, n_rows] f16
    f16* y_out;              // down: [slots, n_rows] f16 (summed in f32 by the combine)
    int* status;             // layer status word: bit 2 when a value left f16's range
};

struct CombineArgs {
    const f16* y;          // [slots, hidden] f16 down outputs
    const int* pos;        // [seq, top_k]
    const float* weights;  // [seq, top_k]
    const int* offsets;    // virtual groups start at offsets[n_experts + v]
    const float* residual; // optional [seq, hidden]
    const float* shared_y; // optional [seq, hidden] f32: the unquantised shared MLP's output
    float* out;            // [seq, hidden]
    int seq, hidden, top_k, n_experts, n_virtual;
};

// Progress words of the fused decode kernel (layer-owned device memory, zero
// at creation): workgroup b publishes the number of steps it has finished this
// call as base + steps, and leaves every call at base + kFusedSteps.
constexpr int kFusedMaxSeq = 16;
constexpr int kFusedDenseMinSeq = 12;  // fewer tokens: gate/up over the candidate groups only
constexpr int kFusedEstMaxSeq = 4;     // up to this many: candidates from per-expert estimate workgroups
constexpr int kFusedMaxGrid = 4096;
constexpr int kStreamMaxSeq = 16;      // streamed decode kernel (decode_stream.hip), bf16 input
constexpr int kStreamWideMaxSeq = 64;  // its wide mode (any input, RMSNorm prologue): token masks are 64-bit
// wide mode: partial rows per token for the routed candidates (more candidates:
// the kernel takes the exact picks instead; >= kMaxTopK)
constexpr int kStreamCandRows = 10;
constexpr int kStreamMaxItems = 4096;  // wide mode items per call (at most 896 + 296 * 7 at 64 tokens)
struct FusedSync {
    int progress[kFusedMaxGrid];
    int error;  // sticky: bit 0 a bounded wait timed out, bit 1 an exact pick outside the candidates
    unsigned call_fault;  // routing tag of the last call with a timed-out wait
    // candidate experts of token t (a superset of its top_k, known before the
    // exact routing) as (tag << 32) | mask half, experts 0..31 at 2t and 32..63
    // at 2t + 1; tag = (base >> 12) + 1 (24 bits): a reader validates each word
    // by its tag, with no separate wait for the router
    unsigned long long cand[2 * kStreamWideMaxSeq];
    // up to kFusedEstMaxSeq tokens: logit estimates of (token t, expert e),
    // one workgroup per expert, as (tag << 32) | float bits: [t][e][2] =
    // estimate, sum of |x w|
    unsigned long long est[kFusedEstMaxSeq * 64 * 2];
    // streamed kernel, wide mode: the item tickets of calls of even / odd
    // base (a call clears the other one; low half: drawn from the front of
    // the list, high half: from its end), and per item the tag of the last
    // call whose partial rows of it are stored
    unsigned long long queue[2];
    unsigned item_done[kStreamMaxItems];
};

// Decode-sized layer (seq < 256): router_decode / expert passes / combine with
// slots derived from the routing ids inside each workgroup.
struct DecodeArgs {
    const void* x;             // [seq, hidden] bf16 bits or f32 (f32 when rms_weight)
    int x_bf16;
    int seq, hidden, inter, n_experts, top_k, n_virtual, group;
    const float* rms_weight;   // optional [hidden]; also selects out = x + moe
    float rms_eps;
    const float* router_f32;   // [hidden/4][64][4], experts padded to 64
    int router_unfused;        // 1: chain steps acc + round(x * w) (an f32 router, matmul_t);
                               // 0: fma(x, w, acc) (a bf16 router, matmul_t_bf16)
    const uint16_t* router_t;  // [hidden/8][n_experts][8] bf16 (fused decode kernel)
    int norm_topk_prob, scoring_sigmoid;
    float scaling;
    f16* x16;                  // [seq, hidden]
    int* ids;                  // [seq, top_k]
    float* wts;                // [seq, top_k]
    const uint8_t* gate;       // [E + n_virtual] tile layout
    const uint8_t* up;
    const uint8_t* down;
    const uint16_t* gate_s;
    const uint16_t* up_s;
    const uint16_t* down_s;
    const uint16_t* gate_z;    // zero offsets in the scale layout (null: symmetric layer)
    const uint16_t* up_z;
    const uint16_t* down_z;
    long long gu_wstride, gu_sstride, dn_wstride, dn_sstride;
    const uint16_t* down_skt;  // down scales as [E + n_virtual][inter / 128][hidden][128 / group] (streamed kernel)
    const uint16_t* down_zkt;  // down zero offsets in that layout (null: symmetric layer)
    const uint8_t* sw;         // the streamed kernel's copy of the weights (units in order of use)
    FusedSync* sync;           // fused kernels only
    int* status;               // layer status word: bit 2 when an act value left f16's range
    const float* shared_y;     // optional [seq, hidden] f32: the unquantised shared MLP's output
    f16* act;                  // [slots, inter]; fused: [(E + n_virtual) * seq, inter]
    float* y;                  // [slots, hidden]
    float* out;                // [seq, hidden]
};
bool decode_shapes_ok(int hidden, int inter);
hipError_t launch_router_decode(const DecodeArgs& a, hipStream_t st);
hipError_t launch_experts_decode2(const DecodeArgs& a, bool gate_up, hipStream_t st);
hipError_t launch_combine_decode(const DecodeArgs& a, hipStream_t st);
bool decode_fused_ok(int hidden, int inter, int group);
hipError_t launch_decode_fused(const DecodeArgs& a, hipStream_t st);
bool decode_stream_ok(int hidden, int inter, int group);
hipError_t launch_decode_stream(const DecodeArgs& a, hipStream_t st);

hipError_t launch_router(const RouterArgs& a, bool x_is_bf16, hipStream_t st);
size_t router_smem_bytes(int hidden);
constexpr int kDecodeTileRows = 16;
constexpr int kPrefillTileRows = 128;     // generic prefill kernel
constexpr int kPrefillBigTileRows = 256;  // large-tile prefill kernel (K in {896, 1280})
// the large-tile kernel is instantiated for 7 and 10 k-tiles and tiles its
// output in 128 act columns (gate/up) and 256 hidden columns (down)
inline bool prefill_big_ok(int hidden, int inter) {
    return (hidden == 896 || hidden == 1280) && (inter == 896 || inter == 1280) && inter % 128 == 0 &&
           hidden % 256 == 0;
}
hipError_t launch_router_from_logits(const RouterArgs& a, const float* logits, hipStream_t st);
hipError_t launch_group(const GroupArgs& g, hipStream_t st);
// launch_group for the moe_router_topk mirror: the multi-workgroup grouping on
// a library-owned per-device scratch when the entries fit it
hipError_t launch_group_mirror(GroupArgs g, hipStream_t st);
int group_chunks(int seq, int top_k);  // 1024-entry chunks of the multi-workgroup grouping
constexpr size_t kGroupScanLds = 96 * 1024;  // per-(chunk, expert) counts of the grouping scan
bool group_fits(int seq, int top_k, int n_experts);  // the grouping scan's LDS holds seq * top_k entries
hipError_t router_overflow_read(int clear, int* flag);  // sticky count > cap flag of the router mirror
hipError_t launch_experts_prefill(const ExpertArgs& a, bool gate_up, int max_tiles, hipStream_t st);
hipError_t launch_experts_prefill_dense(const ExpertArgs& a, bool gate_up, int max_tiles, hipStream_t st);
hipError_t launch_combine(const CombineArgs& c, hipStream_t st);

// Unquantised (bf16 / f32 checkpoint) matrices held as f16 row-major
// [experts][rows][cols] on the device (dense.hip).
constexpr int kDenseSkinnyBM = 16;   // decode-sized tiles
constexpr int kDenseTiledBM = 128;   // prefill-sized tiles
struct DenseArgs {
    const void* a;          // A rows: f16 (x16 / act) or bf16 (the layer input x)
    int a_kind;             // 0 f16, 1 bf16
    const int* slot_tok;    // non-null: A row of slot s is slot_tok[s]; null: row s
    const f16* w0;          // gate (gate/up pass) or down, [experts][n_w][k]
    const f16* w1;          // up (gate/up pass), else null
    long long w_stride;     // elements between experts
    int n_out;              // gate/up: act columns (= gate rows); down: output columns
    int k;                  // input features
    const int* tile_info;   // grouped tiles [max][4] (e, m0, rows, slot0); null: slot tiles over seq
    const int* n_tiles;
    int seq;
    f16* out16;             // gate/up: act [slot][n_out]; down: y [slot][n_out] f16 (if out32 is null)
    float* out32;           // down: y [slot][n_out] f32
    int* status;            // layer status word: bit 2 when a value left f16's range
};
bool dense_shapes_ok(int k, int n_out, bool gate_up, int bm);
hipError_t launch_dense(const DenseArgs& a, bool gate_up, int bm, int max_tiles, hipStream_t st);
// f16 rows of x (bf16 or f32), RMS-normalised when rms_w is set, for a dense shared MLP
hipError_t launch_x16_prep(const void* x, bool x_bf16, const float* rms_w, float eps, int seq, int H, f16* x16,
                           hipStream_t st);

// reference-layout operator mirrors (mirrors.hip)
int set_error(int code, const std::string& msg);  // capi.hip: thread's last error text
bool mirror_shapes_ok(int k, int n, int group, bool int4);
hipError_t mirror_gate_up_int4(const float* x, const uint8_t* gp, const float* gs, const float* gz, long long gps,
                               long long gss, int gng, const uint8_t* up, const float* us, const float* uz,
                               long long ups, long long uss, int ung, const int* assign_token, const int* count,
                               int n_experts, int cap, int hidden, int inter, int group, float* act, hipStream_t st);
hipError_t mirror_down_int4(const float* act, const uint8_t* p, const float* s, const float* z, long long ps,
                            long long ss, int ng, const int* assign_token, const float* assign_w, const int* count,
                            int n_experts, int cap, int hidden, int inter, int group, float* out, hipStream_t st);
hipError_t mirror_gemm_int4(const float* x, const uint8_t* p, const float* s, const float* z, int m, int n, int k,
                            int group, float* y, hipStream_t st);
hipError_t mirror_gemm_bf16(const float* x, const uint16_t* w, const float* bias, int m, int n, int k, float* y,
                            hipStream_t st);
hipError_t mirror_silu_mul(const float* g, const float* u, float* out, long long n, hipStream_t st);
hipError_t mirror_add_scaled(float* dst, const float* src, float scale, long long n, hipStream_t st);
hipError_t mirror_scatter_add_scaled(float* out, const float* vals, const int* row_idx, const float* w, int rows,
                                     int cols, hipStream_t st);
hipError_t mirror_gather_rows(float* dst, const float* src, const int* row_idx, int rows, int cols, hipStream_t st);
hipError_t mirror_gate_up_bf16(const float* x, const uint16_t* const* gw, const uint16_t* const* uw,
                               const int* assign_token, const int* count, int n_experts, int cap, int hidden,
                               int inter, float* act, hipStream_t st);
hipError_t mirror_down_bf16(const float* act, const uint16_t* const* dw, const int* assign_token,
                            const float* assign_w, const int* count, int n_experts, int cap, int hidden, int inter,
                            float* out, hipStream_t st);

}  // namespace uocr_hip
