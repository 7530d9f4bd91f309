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
  uint32_t* sel = (uint32_t*)(comp + ((L + 1) & ~1));          // [B rounded up to 64] selected keys, 16-byte aligned
  uint32_t(*whist)[256] = (uint32_t(*)[256])(sel + ((B + 63) & ~63));  // [SEL_NW][256]
  uint64_t* shared64 = (uint64_t*)(whist + SEL_NW);            // [2]
  uint32_t* scratch = (uint32_t*)(shared64 + 2);               // [SEL_NW + 1]
  uint32_t* shared = scratch + SEL_NW + 1;                     // [4]
  const int item = blockIdx.x;
  const int32_t* idx = sl_idx + (int64_t)item * L;
  const float* rank = sl_rank + (int64_t)item * L;
  const int n = max(0, min(sl_count[item], L));
  uint64_t vor = 0ull, vand = ~0ull;  // over this thread's entries below n
  for (int i = threadIdx.x; i < L; i += SEL_BLOCK) {
    const float r = rank[i];
    const int32_t x = idx[i];
    const uint64_t c = composite(f2key(r), (uint32_t)x);
    comp[i] = c;
    if (i < n) {
      vor |= c;
      vand &= c;
    }
  }
  const int beff = min(B, n);
  if (threadIdx.x == 0) fin_count[item] = beff;
  if (beff <= 0) return;
  __syncthreads();
  auto visit = [&](auto&& f) {
    for (int i = threadIdx.x; i < n; i += SEL_BLOCK) f(comp[i]);
  };
  const uint64_t X =
      beff == n ? 0ull : select_largest_with_bounds<SEL_BLOCK>(visit, beff, vor, vand, whist, scratch, shared64, shared);
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
  // ascending order.  Up to SEL_BLOCK entries: each wave sorts a run of 64
  // in registers (bitonic), then every entry's rank is its place in its run
  // plus, for every other run, the number of smaller entries (binary search).
  int32_t* out = fin_idx + (int64_t)item * B;
  if (beff <= SEL_BLOCK) {
    const int runs = (beff + WAVE - 1) / WAVE;
    const int t = threadIdx.x;
    uint32_t v = t < beff ? sel[t] : 0xFFFFFFFFu;
    if (t < runs * WAVE) {
      const int lane = lane_id();
      for (int k = 2; k <= WAVE; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
          const uint32_t o = (uint32_t)__shfl_xor((int)v, j, WAVE);
          const bool up = (lane & k) == 0;
          const bool low = (lane & j) == 0;
          v = (low == up) ? min(v, o) : max(v, o);
        }
      }
    }
    __syncthreads();
    if (t < runs * WAVE) sel[t] = v;  // sorted runs, padded with 0xFFFFFFFF
    __syncthreads();
    if (t < runs * WAVE && v != 0xFFFFFFFFu) {
      const int run = t / WAVE;
      int r = t - run * WAVE;
      for (int q = 0; q < runs; ++q) {
        if (q == run) continue;
        const uint32_t* a = sel + q * WAVE;
        int lo = 0, hi = WAVE;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (a[mid] < v) lo = mid + 1;
          else hi = mid;
        }
        r += lo;
      }
      out[r] = (int32_t)v;
    }
  } else {
    // large budgets: two lanes per entry count the smaller ones
    const int hb = (((beff + 1) >> 1) + 3) & ~3;
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
  const size_t lds = sizeof(uint64_t) * ((size_t)((L + 1) & ~1) + 2) + sizeof(uint32_t) * ((size_t)((B + 63) & ~63) + SEL_NW * 256 +
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
