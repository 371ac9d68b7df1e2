// INT4 prefill expert GEMM, gate/up pass, without zero offsets (one of the four
// translation units of experts_prefill.hpp's kernels, compiled in parallel).
#include "experts_prefill.hpp"

namespace uocr_hip {

hipError_t launch_prefill_gu_z0(const ExpertArgs& a, int max_tiles, hipStream_t st) {
    return launch_prefill_g<true, false>(a, max_tiles, st);
}

}  // namespace uocr_hip
