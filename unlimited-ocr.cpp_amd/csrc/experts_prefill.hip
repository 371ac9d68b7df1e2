// Prefill expert GEMM: the host-side dispatch. The kernels and their
// template launchers live in experts_prefill.hpp; the INT4 instantiations are
// split over four translation units (gate/up or down, with or without zero
// offsets: experts_prefill_{gu,dn}_z{0,1}.hip) so that they compile in
// parallel, and this file holds the unquantised (f16-weight) instantiations.
#include "experts_prefill.hpp"

namespace uocr_hip {

hipError_t launch_prefill_gu_z0(const ExpertArgs& a, int max_tiles, hipStream_t st);
hipError_t launch_prefill_gu_z1(const ExpertArgs& a, int max_tiles, hipStream_t st);
hipError_t launch_prefill_dn_z0(const ExpertArgs& a, int max_tiles, hipStream_t st);
hipError_t launch_prefill_dn_z1(const ExpertArgs& a, int max_tiles, hipStream_t st);

// unquantised experts (f16 weights) on the large-tile kernel, 256-slot tiles
hipError_t launch_experts_prefill_dense(const ExpertArgs& a, bool gate_up, int max_tiles, hipStream_t st) {
    if (max_tiles <= 0) return hipSuccess;
    if (a.bm != kBigBM || !a.w0 || (gate_up && !a.w1)) return hipErrorInvalidValue;
    const int n_ntiles = gate_up ? (a.n_rows / (kBigBN / 2)) : (a.n_rows / kBigBN);
    if (n_ntiles * (gate_up ? kBigBN / 2 : kBigBN) != a.n_rows) return hipErrorInvalidValue;
    const dim3 grid(((max_tiles + 7) / 8) * 8 * n_ntiles);
    switch (a.k / kTileK) {
        case 7:
            if (gate_up) launch_k((experts_prefill_big_kernel<4, true, 7, false, true>), grid, dim3(256), 0, st, a);
            else launch_k((experts_prefill_big_kernel<4, false, 7, false, true>), grid, dim3(256), 0, st, a);
            break;
        case 10:
            if (gate_up) launch_k((experts_prefill_big_kernel<4, true, 10, false, true>), grid, dim3(256), 0, st, a);
            else launch_k((experts_prefill_big_kernel<4, false, 10, false, true>), grid, dim3(256), 0, st, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_experts_prefill(const ExpertArgs& a, bool gate_up, int max_tiles, hipStream_t st) {
    if (max_tiles <= 0) return hipSuccess;
    if ((gate_up && a.n_rows % (kPreBN / 2)) || (!gate_up && a.n_rows % kPreBN)) return hipErrorInvalidValue;
    if (a.z0) return gate_up ? launch_prefill_gu_z1(a, max_tiles, st) : launch_prefill_dn_z1(a, max_tiles, st);
    return gate_up ? launch_prefill_gu_z0(a, max_tiles, st) : launch_prefill_dn_z0(a, max_tiles, st);
}

}  // namespace uocr_hip
