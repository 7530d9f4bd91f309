// Finish kernel of the long-context summon without the fused verifier.
#include "summon_wide.cuh"

namespace sva {
namespace wide {

int launch_finish_nov(const WideArgs& a, int64_t items, hipStream_t stream) {
  return launch_finish<0, F32>(a, items, stream);
}

}  // namespace wide
}  // namespace sva
