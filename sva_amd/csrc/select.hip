// Budget select: the exact top-B of each shortlist by (rank score desc, key
// index asc), written as ascending key indices (sva/llama.py:293-302).
//
// One workgroup per query item.  All L shortlist slots are loaded at once
// (slots past the count are ignored) as unique 64-bit composites (rank key,
// key index) into LDS; a radix select with per-wave histograms finds the
// B-th largest composite X; the entries >= X are compacted in shortlist order
// and each is stored at its rank among the selected key indices, so the
// output is ascending whatever the shortlist's order.  Shortlist key indices
// are unique (every summon path guarantees it).
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int SEL_BLOCK = 1024;
constexpr int SEL_NW = SEL_BLOCK / WAVE;

__global__ void __launch_bounds__(SEL_BLOCK)
    budget_select_kernel(const int32_t* __restrict__ sl_idx, const float* __restrict__ sl_rank,
                         const int32_t* __restrict__ sl_count, int L, int B, int32_t* __restrict__ fin_idx,
                         int32_t* __restrict__ fin_count) {
  extern __shared__ __align__(16) unsigned char lds[];
  uint64_t* comp = (uint64_t*)lds;                             // [L]
  uint32_t* sel = (uint32_t*)(comp + ((L + 1) & ~1));          // [B] selected key indices, 16-byte aligned
  uint32_t(*whist)[256] = (uint32_t(*)[256])(sel + ((B + 3) & ~3));  // [SEL_NW][256]
  uint64_t* shared64 = (uint64_t*)(whist + SEL_NW);            // [2]
  uint32_t* scratch = (uint32_t*)(shared64 + 2);               // [SEL_NW + 1]
  uint32_t* shared = scratch + SEL_NW + 1;                     // [4]
  const int item = blockIdx.x;
  const int32_t* idx = sl_idx + (int64_t)item * L;
  const float* rank = sl_rank + (int64_t)item * L;
  const int n = max(0, min(sl_count[item], L));
  for (int i = threadIdx.x; i < L; i += SEL_BLOCK) {
    const float r = rank[i];
    const int32_t x = idx[i];
    comp[i] = composite(f2key(r), (uint32_t)x);
  }
  const int beff = min(B, n);
  if (threadIdx.x == 0) fin_count[item] = beff;
  if (beff <= 0) return;
  __syncthreads();
  auto visit = [&](auto&& f) {
    for (int i = threadIdx.x; i < n; i += SEL_BLOCK) f(comp[i]);
  };
  const uint64_t X = beff == n ? 0ull : select_largest<SEL_BLOCK>(visit, beff, whist, scratch, shared64, shared);
  // compact the selected in shortlist order: contiguous ranges per thread
  const int per = (n + SEL_BLOCK - 1) / SEL_BLOCK;
  const int i0 = min(n, (int)threadIdx.x * per), i1 = min(n, i0 + per);
  uint32_t cnt = 0;
  for (int i = i0; i < i1; ++i) cnt += comp[i] >= X;
  uint32_t tot;
  uint32_t o = block_excl_scan<SEL_BLOCK>(cnt, scratch, &tot);
  for (int i = i0; i < i1; ++i) {
    const uint64_t c = comp[i];
    if (c >= X && o < (uint32_t)beff) sel[o++] = composite_index(c);
  }
  __syncthreads();
  // ascending order: each selected index goes to its rank among the selected,
  // counted by two lanes per element over halves of the list (16-byte
  // broadcast reads, eight in flight)
  int32_t* out = fin_idx + (int64_t)item * B;
  const int hb = (((beff + 1) >> 1) + 3) & ~3;  // first half, a multiple of 4
  for (int i = threadIdx.x; i < 2 * beff; i += SEL_BLOCK) {
    const int e = i >> 1;
    const uint32_t v = sel[e];
    const int j0 = (i & 1) ? hb : 0;
    const int j1 = (i & 1) ? beff : min(hb, beff);
    int r = 0;
    int j = j0;
#pragma unroll 8
    for (; j + 4 <= j1; j += 4) {
      const uint4 u = *reinterpret_cast<const uint4*>(sel + j);
      r += (int)(u.x < v) + (int)(u.y < v) + (int)(u.z < v) + (int)(u.w < v);
    }
    for (; j < j1; ++j) r += (int)(sel[j] < v);
    r += __shfl_xor(r, 1);
    if ((i & 1) == 0) out[r] = (int32_t)v;
  }
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
  const size_t lds = sizeof(uint64_t) * ((size_t)((L + 1) & ~1) + 2) + sizeof(uint32_t) * ((size_t)((B + 3) & ~3) + SEL_NW * 256 +
                                                                              SEL_NW + 1 + 4);
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
                     sl_rank, sl_count, (int)L, (int)B, fin_idx, fin_count);
  SVA_CHECK_LAUNCH("budget_select_kernel");
  return SVA_OK;
}
