// Finish and class-budget kernels with the fused verifier: head_dim 64,
// float16 K / V.
#include "summon_wide.cuh"

namespace sva {
namespace wide {

int launch_finish_v64_f16(const WideArgs& a, int64_t items, hipStream_t stream) {
  return launch_finish<64, F16>(a, items, stream);
}

int launch_class_budget_v64_f16(const ClassArgs& a, int64_t items, hipStream_t stream) {
  return launch_class_budget<64, F16>(a, items, stream);
}

}  // namespace wide
}  // namespace sva
