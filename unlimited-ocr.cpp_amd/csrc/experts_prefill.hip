#include "launch.hpp"
namespace uocr_hip {
hipError_t launch_experts_prefill(const ExpertArgs&, bool, int, hipStream_t) { return hipErrorNotSupported; }
}
