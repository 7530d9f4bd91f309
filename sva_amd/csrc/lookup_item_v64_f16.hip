// The fused one-token lookup of the per-item register path with its
// verifier: head_dim 64, float16 K / V.
#include "lookup_item.cuh"

namespace sva {
namespace item_lookup {

int launch_v64_f16(const LutParams& lp, const SummonParams& p, const FusedVerify& fv, const WriteParams& wp,
                   int32_t* overshoot, hipStream_t st) {
  return launch<64, F16>(lp, p, fv, wp, overshoot, st);
}

}  // namespace item_lookup
}  // namespace sva
