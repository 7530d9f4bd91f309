// Long-context q=1 summon: many workgroups per query item (see summon.h).
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

namespace sva {

bool summon_wide_eligible(const SummonParams&, int64_t) { return false; }

int summon_wide_path(const SummonParams&, void*, size_t, hipStream_t) {
  set_error("sva_summon: wide path not built");
  return SVA_ERR_UNSUPPORTED;
}

size_t summon_wide_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t) { return 256; }

}  // namespace sva
