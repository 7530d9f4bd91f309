// Budget select: the exact top-B of each shortlist by (rank score desc, key
// index asc), written as ascending key indices (sva/llama.py:293-302).
//
// One workgroup per query item.  The shortlist is loaded into LDS as unique
// 64-bit composites, a radix select finds the B-th largest composite X, the
// entries >= X are compacted and sorted by key index (bitonic, LDS) so that
// the output does not depend on the shortlist's order.
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int SEL_BLOCK = 512;

__global__ void __launch_bounds__(SEL_BLOCK)
    budget_select_kernel(const int32_t* __restrict__ sl_idx, const float* __restrict__ sl_rank,
                         const int32_t* __restrict__ sl_count, int L, int B, int P, int32_t* __restrict__ fin_idx,
                         int32_t* __restrict__ fin_count) {
  extern __shared__ __align__(16) unsigned char lds[];
  uint64_t* comp = (uint64_t*)lds;       // [L]
  uint64_t* sel = comp + L;              // [P] (P = next pow2 of B)
  uint32_t* hist = (uint32_t*)(sel + P);  // [256]
  uint32_t* scratch = hist + 256;         // [SEL_BLOCK/64 + 1]
  uint32_t* shared = scratch + SEL_BLOCK / WAVE + 1;  // [4]
  const int item = blockIdx.x;
  const int n = min(sl_count[item], L);
  const int beff = min(B, n);
  if (beff <= 0) {
    if (threadIdx.x == 0) fin_count[item] = 0;
    return;
  }
  const int32_t* idx = sl_idx + (int64_t)item * L;
  const float* rank = sl_rank + (int64_t)item * L;
  for (int i = threadIdx.x; i < n; i += SEL_BLOCK) comp[i] = composite(f2key(rank[i]), (uint32_t)idx[i]);
  if (threadIdx.x == 0) shared[2] = 0;
  __syncthreads();
  uint64_t X = 0;
  if (beff < n) X = radix_select_u64<SEL_BLOCK>([&](int i) { return comp[i]; }, n, beff, hist, scratch, shared);
  for (int i = threadIdx.x; i < n; i += SEL_BLOCK) {
    const uint64_t c = comp[i];
    if (c >= X) {
      const uint32_t j = atomicAdd(&shared[2], 1u);
      if (j < (uint32_t)P) sel[j] = ((uint64_t)composite_index(c) << 32) | (uint64_t)composite_key(c);
    }
  }
  __syncthreads();
  for (int i = beff + threadIdx.x; i < P; i += SEL_BLOCK) sel[i] = ~0ull;
  __syncthreads();
  bitonic_sort_u64<SEL_BLOCK>(sel, P, false);
  int32_t* out = fin_idx + (int64_t)item * B;
  for (int i = threadIdx.x; i < beff; i += SEL_BLOCK) out[i] = (int32_t)(sel[i] >> 32);
  if (threadIdx.x == 0) fin_count[item] = beff;
}

}  // namespace

extern "C" int sva_budget_select(const int32_t* sl_idx, const float* sl_rank, const int32_t* sl_count,
                                 int64_t n_items, int64_t L, int64_t B, int32_t* fin_idx, int32_t* fin_count,
                                 void* stream) {
  sva::clear_error();
  SVA_REQUIRE(sl_idx && sl_rank && sl_count && fin_idx && fin_count, "sva_budget_select: null pointer");
  SVA_REQUIRE(n_items > 0 && n_items < (1ll << 31), "sva_budget_select: bad item count");
  SVA_REQUIRE(L > 0 && L <= 16384 && B > 0 && B <= 8192, "sva_budget_select: shortlist %lld / budget %lld out of range",
              (long long)L, (long long)B);
  const int P = sva::next_pow2_host((int)B);
  const size_t lds = sizeof(uint64_t) * ((size_t)L + (size_t)P) + sizeof(uint32_t) * (256 + SEL_BLOCK / 64 + 1 + 4);
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_budget_select: shortlist %lld + budget %lld exceed LDS",
                  (long long)L, (long long)B);
  static bool attr_set = false;
  if (!attr_set) {
    SVA_CHECK_HIP(hipFuncSetAttribute((const void*)budget_select_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      sva::kMaxLds),
                  "hipFuncSetAttribute(budget_select_kernel)");
    attr_set = true;
  }
  hipLaunchKernelGGL(budget_select_kernel, dim3((unsigned)n_items), dim3(SEL_BLOCK), lds, (hipStream_t)stream, sl_idx,
                     sl_rank, sl_count, (int)L, (int)B, P, fin_idx, fin_count);
  SVA_CHECK_LAUNCH("budget_select_kernel");
  return SVA_OK;
}
