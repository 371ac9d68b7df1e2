// INT4 prefill expert GEMM, down pass, without zero offsets (one of the four
// translation units of experts_prefill.hpp's kernels, compiled in parallel).
#include "experts_prefill.hpp"

namespace uocr_hip {

hipError_t launch_prefill_dn_z0(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    return launch_prefill_g<false, false>(a, max_tiles, st);
}

}  // namespace uocr_hip
