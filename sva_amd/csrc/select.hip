// Budget select: the exact top-B of each shortlist by (rank score desc, key
// index asc), written as ascending key indices (sva/llama.py:293-302).
//
// One workgroup per query item.  Each thread loads its NPT shortlist slots
// (coalesced, slots past the count left empty) straight into registers as
// unique 64-bit composites (rank key, key index); a register radix select
// finds the B-th largest composite X; the entries >= X are gathered in LDS
// and written in ascending key-index order, whatever the shortlist's order.
// Where the caller's shortlists are in ascending key order (the per-item
// summon writes them so), an ordered compaction of the chosen slots writes
// them instead: slot i * BLOCK + t of thread t in slot-major (slot, wave,
// lane) order is slot order, so per-(slot, wave) counts and one scan place
// every entry, where the sort of the unordered form costs O(B^2 / BLOCK)
// comparisons a thread.  Shortlist key indices are unique (every summon path
// guarantees it).
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int SEL_BLOCK = 1024;
constexpr int SEL_NW = SEL_BLOCK / WAVE;
constexpr int SEL_MAX_B = 8192;

template <int NPT>
__global__ void __launch_bounds__(SEL_BLOCK)
    budget_select_kernel(const int32_t* __restrict__ sl_idx, const float* __restrict__ sl_rank,
                         const int32_t* __restrict__ sl_count, int L, int B, int32_t* __restrict__ fin_idx,
                         int32_t* __restrict__ fin_count, int ordered) {
  __shared__ __align__(16) uint32_t hist[TOP_BINS];
  __shared__ __align__(16) uint32_t sel[SEL_MAX_B];
  __shared__ uint64_t small[TOP_SMALL];
  __shared__ uint64_t shared64[2];
  __shared__ uint32_t scratch[SEL_NW + 1];
  __shared__ uint32_t shared[4];
  const int item = blockIdx.x;
  const int32_t* idx = sl_idx + (int64_t)item * L;
  const float* rank = sl_rank + (int64_t)item * L;
  const int n = max(0, min(sl_count[item], L));
  uint64_t e[NPT];
  uint64_t vor = 0ull, vand = ~0ull;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int r = (int)threadIdx.x + i * SEL_BLOCK;
    e[i] = 0ull;
    if (r < n) {
      e[i] = composite(f2key(rank[r]), (uint32_t)idx[r]);
      vor |= e[i];
      vand &= e[i];
    }
  }
  const int beff = min(B, n);
  if (threadIdx.x == 0) {
    fin_count[item] = beff;
    shared[3] = 0u;
  }
  if (beff == 0) return;
  const TopLds tl{hist, small, scratch, shared, shared64};
  const uint64_t X = beff == n ? 1ull : select_top_regs<SEL_BLOCK, NPT>(e, beff, vor, vand, tl, (n + SEL_BLOCK - 1) / SEL_BLOCK);
  if (threadIdx.x == 0) shared[3] = 0u;
  __syncthreads();
  if (ordered) {  // block-uniform
    const int lane = lane_id(), wid = (int)threadIdx.x / WAVE;
    uint32_t* wcnt = hist;  // [NPT][SEL_NW] chosen slots per (slot, wave), then their offsets
    uint64_t m[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      m[i] = __builtin_amdgcn_ballot_w64(e[i] != 0ull && e[i] >= X);
      if (lane == 0) wcnt[i * SEL_NW + wid] = (uint32_t)__popcll(m[i]);
    }
    __syncthreads();
    const uint32_t wc = (int)threadIdx.x < NPT * SEL_NW ? wcnt[threadIdx.x] : 0u;
    const uint32_t wpre = block_excl_scan<SEL_BLOCK>(wc, scratch, nullptr);
    if ((int)threadIdx.x < NPT * SEL_NW) wcnt[threadIdx.x] = wpre;
    __syncthreads();
    int32_t* out = fin_idx + (int64_t)item * B;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      if ((m[i] >> lane) & 1ull) {
        const uint32_t o = wcnt[i * SEL_NW + wid] +
                           __builtin_amdgcn_mbcnt_hi((uint32_t)(m[i] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m[i], 0u));
        if (o < (uint32_t)beff) out[o] = (int32_t)composite_index(e[i]);
      }
    }
    return;
  }
  append_selected<NPT>(e, X, sel, beff, &shared[3]);
  __syncthreads();
  write_ascending<SEL_BLOCK>(sel, beff, fin_idx + (int64_t)item * B);
}

template <int NPT>
int launch_budget(const int32_t* sl_idx, const float* sl_rank, const int32_t* sl_count, int64_t n_items, int L, int B,
                  int32_t* fin_idx, int32_t* fin_count, bool ordered, hipStream_t stream) {
  hipLaunchKernelGGL(budget_select_kernel<NPT>, dim3((unsigned)n_items), dim3(SEL_BLOCK), 0, stream, sl_idx, sl_rank,
                     sl_count, L, B, fin_idx, fin_count, ordered ? 1 : 0);
  SVA_CHECK_LAUNCH("budget_select_kernel");
  return SVA_OK;
}

}  // namespace

namespace sva {

int budget_select_launch(const int32_t* sl_idx, const float* sl_rank, const int32_t* sl_count, int64_t n_items,
                         int64_t L, int64_t B, int32_t* fin_idx, int32_t* fin_count, bool ordered,
                         hipStream_t stream) {
  SVA_REQUIRE(L > 0 && L <= 16384 && B > 0 && B <= SEL_MAX_B,
              "sva_budget_select: shortlist %lld / budget %lld out of range", (long long)L, (long long)B);
  const int l = (int)L, b = (int)B;
  if (L <= 2 * SEL_BLOCK) return launch_budget<2>(sl_idx, sl_rank, sl_count, n_items, l, b, fin_idx, fin_count, ordered, stream);
  if (L <= 4 * SEL_BLOCK) return launch_budget<4>(sl_idx, sl_rank, sl_count, n_items, l, b, fin_idx, fin_count, ordered, stream);
  if (L <= 8 * SEL_BLOCK) return launch_budget<8>(sl_idx, sl_rank, sl_count, n_items, l, b, fin_idx, fin_count, ordered, stream);
  return launch_budget<16>(sl_idx, sl_rank, sl_count, n_items, l, b, fin_idx, fin_count, ordered, stream);
}

}  // namespace sva

extern "C" int sva_budget_select(const int32_t* sl_idx, const float* sl_rank, const int32_t* sl_count,
                                 int64_t n_items, int64_t L, int64_t B, int32_t* fin_idx, int32_t* fin_count,
                                 void* stream) {
  sva::clear_error();
  SVA_REQUIRE(sl_idx && sl_rank && sl_count && fin_idx && fin_count, "sva_budget_select: null pointer");
  SVA_REQUIRE(n_items > 0 && n_items < (1ll << 31), "sva_budget_select: bad item count");
  // the caller's shortlists in any order
  return sva::budget_select_launch(sl_idx, sl_rank, sl_count, n_items, L, B, fin_idx, fin_count, false,
                                   (hipStream_t)stream);
}
