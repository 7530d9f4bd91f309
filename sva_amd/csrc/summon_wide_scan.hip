// Scan kernels of the long-context summon (one variant per code width S,
// table width C <= 64 and masking).
#include "summon_wide.cuh"

namespace sva {
namespace wide {
namespace {

template <int S, bool SMALLC, bool MASKED>
int launch_wide(const WideArgs& a, int64_t items, hipStream_t stream) {
  hipLaunchKernelGGL((wide_scan_kernel<S, SMALLC, MASKED>), dim3((unsigned)(items * a.W)), dim3(WB), 0, stream, a);
  SVA_CHECK_LAUNCH("wide_scan_kernel");
  return SVA_OK;
}

template <int S>
int launch_wide_s(const WideArgs& a, int64_t items, bool masked, hipStream_t stream) {
  const bool small_c = a.p.C <= 64;
  if (small_c) return masked ? launch_wide<S, true, true>(a, items, stream) : launch_wide<S, true, false>(a, items, stream);
  return masked ? launch_wide<S, false, true>(a, items, stream) : launch_wide<S, false, false>(a, items, stream);
}

}  // namespace

int launch_scan(const WideArgs& a, int64_t items, bool masked, hipStream_t stream) {
  switch (a.p.S) {
    case 1: return launch_wide_s<1>(a, items, masked, stream);
    case 2: return launch_wide_s<2>(a, items, masked, stream);
    case 4: return launch_wide_s<4>(a, items, masked, stream);
    default: return launch_wide_s<8>(a, items, masked, stream);
  }
}

}  // namespace wide
}  // namespace sva
