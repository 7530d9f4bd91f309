// Long-context summon for few query items (decode, q = 1): many workgroups
// per item, one pass over the packed uint8 codes.
//
// Cooperative launch (every workgroup resident); per query item the keys are
// split into contiguous chunks, one per workgroup.
//   Phase A  each thread loads its chunk's codes with 16-byte loads, scores its
//            keys through the LUT (LDS) in the reference's order and keeps the
//            order-preserving keys in registers.  A workgroup histogram over
//            NB linear bins of [lo, hi] (monotone in the score) is built in
//            LDS; only the bins from the workgroup's own L-th-largest bin up
//            are published (atomics) to the item's global histogram -- the
//            item's threshold bin can never lie below that bin.
//   barrier
//   Phase B  every workgroup finds the item's threshold bin t (largest bin
//            whose suffix count reaches L); keys in bins above t are in the
//            shortlist, keys in bin t go to a tie buffer as unique 64-bit
//            composites.  Shortlisted keys are rescored against q_low.
//   barrier
//   Phase C  one workgroup per item takes the `need` largest composites of the
//            tie buffer (radix select), rescores them, and returns the item's
//            histogram and counters to zero for the next call.
// Selection is exact: the result equals a full sort by (score desc, key asc).
// The tie buffer holds one entry per key, so it cannot overflow; a heavily
// tied threshold bin only makes phase C slower.
#include <hip/hip_cooperative_groups.h>

#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

namespace cg = cooperative_groups;
using namespace sva;

namespace {

constexpr int WB = 256;      // threads per workgroup
constexpr int NB = 2048;     // histogram bins
constexpr int NW = WB / WAVE;
constexpr int EMIT_CAP = 512;   // sure keys a workgroup rescores itself
constexpr int64_t kWideMinKeys = 32768;
constexpr int64_t kMaxWideItems = 64;

struct WideParams {
  SummonParams p;
  int W;            // workgroups per item
  int64_t chunk;    // keys per workgroup (multiple of WB * keys-per-load)
  uint32_t* ghist;  // [items, NB]
  uint32_t* gctr;   // [items, 4]: allowed, sure, tie, spare
  uint64_t* ties;   // [items, tie_cap]
  int64_t tie_cap;  // = keys per item: the threshold bin can never overflow it
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Byte j of a 16-byte vector.
SVA_DEV uint32_t byte_of(const u32x4& v, int j) { return (v[j >> 2] >> (8 * (j & 3))) & 0xFFu; }

SVA_DEV int score_bin(float s, float lo, float inv_w) {
  const float f = (s - lo) * inv_w;  // monotone non-decreasing in s
  int b = (int)f;
  b = b < 0 ? 0 : (b >= NB ? NB - 1 : b);
  return f != f ? 0 : b;
}

// Rank score of one 64-float k_low row in torch's sum order (the same bits
// as torch_order_dot64), streamed one 8-float group pair at a time so that
// only ~24 values are live.
SVA_DEV float rank_dot64_stream(const float* __restrict__ row, const float* __restrict__ q) {
#pragma clang fp contract(off)
  const float4* r4 = reinterpret_cast<const float4*>(row);
  float part[8];
#pragma unroll 1
  for (int x = 0; x < 4; ++x) {
    const float4 a = r4[2 * x], b = r4[2 * x + 1], c = r4[2 * x + 8], d = r4[2 * x + 9];
    const float* qa = q + 8 * x;
    const float* qc = q + 32 + 8 * x;
    float ax[8];
    ax[0] = (0.0f + a.x * qa[0]) + c.x * qc[0];
    ax[1] = (0.0f + a.y * qa[1]) + c.y * qc[1];
    ax[2] = (0.0f + a.z * qa[2]) + c.z * qc[2];
    ax[3] = (0.0f + a.w * qa[3]) + c.w * qc[3];
    ax[4] = (0.0f + b.x * qa[4]) + d.x * qc[4];
    ax[5] = (0.0f + b.y * qa[5]) + d.y * qc[5];
    ax[6] = (0.0f + b.z * qa[6]) + d.z * qc[6];
    ax[7] = (0.0f + b.w * qa[7]) + d.w * qc[7];
#pragma unroll
    for (int l = 0; l < 8; ++l) part[l] = x == 0 ? ax[l] : part[l] + ax[l];
  }
  float total = 0.0f;
#pragma unroll
  for (int l = 0; l < 8; ++l) total = total + part[l];
  return total;
}

// Wave-aggregated slot reservation: returns this lane's slot (flag set) from
// one atomic per wave.
SVA_DEV uint32_t wave_reserve(uint32_t* counter, bool flag) {
  const uint64_t ballot = __ballot(flag);
  if (ballot == 0) return 0;
  const int lane = lane_id();
  const uint32_t below = (uint32_t)__popcll(ballot & ((1ull << lane) - 1ull));
  const int leader = __ffsll((long long)ballot) - 1;
  uint32_t base = 0;
  if (lane == leader) base = atomicAdd(counter, (uint32_t)__popcll(ballot));
  base = __shfl(base, leader, WAVE);
  return base + below;
}

// Exact score of key n through the LUT (codes re-read; used for the few
// threshold-bin members).
template <int S>
SVA_DEV float score_at(const uint8_t* __restrict__ codes, int n, const float* tab, int C, float sqrt_r) {
#pragma clang fp contract(off)
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    uint32_t c = codes[(int64_t)n * S + s];
    c = c < (uint32_t)C ? c : (uint32_t)(C - 1);
    acc = acc + tab[s * C + c];
  }
  return acc / sqrt_r;
}

template <int S, int RND>
__global__ void __launch_bounds__(WB, 4) summon_wide_kernel(WideParams wp) {
#pragma clang fp contract(off)
  constexpr int KPT = 16 / S;  // keys per 16-byte load
  constexpr int KEYS = RND * KPT;
  constexpr uint32_t NOBIN = 0xFFFFu;
  static_assert(KEYS <= 64 && KEYS % 2 == 0, "two 16-bit bins per register, 64-bit key masks");
  __shared__ float tab[S * 256];
  __shared__ float ql[512];
  __shared__ uint32_t hist[NB];
  __shared__ uint32_t scratch[NW + 1];
  __shared__ uint32_t shared[8];
  __shared__ int32_t emit_n[EMIT_CAP];
  __shared__ uint32_t emit_slot[EMIT_CAP];

  const SummonParams& p = wp.p;
  const int item = blockIdx.x / wp.W;
  const int w = blockIdx.x % wp.W;
  const int h = item % p.H;  // q = 1, one sequence
  const int C = p.C;
  const int N = (int)p.N;
  const int cs = (int)((int64_t)w * wp.chunk);
  const int ce = (int)min((int64_t)cs + wp.chunk, (int64_t)N);
  const float lo = p.range[2 * item];
  const float hi = p.range[2 * item + 1];
  const float span = hi - lo;
  const float inv_w = (span > 0.0f && span < INFINITY) ? (float)NB / span : 0.0f;
  const float sqrt_r = p.sqrt_r;

  for (int e = threadIdx.x; e < S * C; e += WB) tab[e] = p.lut[(int64_t)item * S * C + e];
  for (int r = threadIdx.x; r < p.R; r += WB) ql[r] = p.q_low[(int64_t)item * p.R + r];
  for (int b = threadIdx.x; b < NB; b += WB) hist[b] = 0;
  __syncthreads();

  // ---- phase A: stream codes, score, histogram ------------------------------
  const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)h * p.code_hs;
  const bool masked = p.mask_type != MASK_NONE;
  u32x4 raw[RND];
#pragma unroll
  for (int r = 0; r < RND; ++r) {
    const int base = cs + (r * WB + (int)threadIdx.x) * KPT;
    if (base + KPT <= ce) {
      raw[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + (int64_t)base * S));
    } else {
      uint32_t wv[4] = {0u, 0u, 0u, 0u};
      for (int j = 0; j < KPT * S; ++j)
        if (base + j / S < ce) wv[j >> 2] |= (uint32_t)codes[(int64_t)base * S + j] << (8 * (j & 3));
      raw[r] = u32x4{wv[0], wv[1], wv[2], wv[3]};
    }
  }
  uint32_t bins[KEYS / 2];  // two 16-bit bins per register, NOBIN = not allowed
  uint32_t n_allowed = 0;
#pragma unroll
  for (int r = 0; r < RND; ++r) {
    const int base = cs + (r * WB + (int)threadIdx.x) * KPT;
#pragma unroll
    for (int k = 0; k < KPT; ++k) {
      const int n = base + k;
      bool ok = n < ce;
      if (ok && masked) ok = mask_allows(p.mask, n, p.mask_type);
      float acc = 0.0f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        uint32_t c = byte_of(raw[r], k * S + s);
        c = c < (uint32_t)C ? c : (uint32_t)(C - 1);
        acc = acc + tab[s * C + c];
      }
      const int bin = score_bin(acc / sqrt_r, lo, inv_w);
      const uint32_t bv = ok ? (uint32_t)bin : NOBIN;
      const int i = r * KPT + k;
      if (i & 1) bins[i >> 1] |= bv << 16;
      else bins[i >> 1] = bv;
      if (ok) {
        atomicAdd(&hist[bin], 1u);
        ++n_allowed;
      }
    }
  }
  __syncthreads();
  {
    constexpr int PER = NB / WB;
    uint32_t c[PER];
    uint32_t sum = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      c[i] = hist[NB - 1 - ((int)threadIdx.x * PER + i)];
      sum += c[i];
    }
    uint32_t tot;
    const uint32_t before = block_excl_scan<WB>(sum, scratch, &tot);
    if (threadIdx.x == 0) shared[0] = 0;  // lowest bin to publish
    __syncthreads();
    uint32_t run = before;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t prev = run;
      run += c[i];
      if (prev < (uint32_t)p.L && run >= (uint32_t)p.L) shared[0] = NB - 1 - ((int)threadIdx.x * PER + i);
    }
    __syncthreads();
    const int pub_lo = (int)shared[0];
    uint32_t* gh = wp.ghist + (int64_t)item * NB;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = NB - 1 - ((int)threadIdx.x * PER + i);
      if (b >= pub_lo && c[i] != 0u) atomicAdd(&gh[b], c[i]);
    }
    const uint32_t wave_allowed = wave_sum_u32(n_allowed);
    if (lane_id() == 0 && wave_allowed) atomicAdd(&wp.gctr[(int64_t)item * 4 + 0], wave_allowed);
  }
  __threadfence();
  cg::this_grid().sync();

  // ---- phase B: threshold bin, emit sure keys and ties ----------------------
  const uint32_t* gh = wp.ghist + (int64_t)item * NB;
  const uint32_t allowed_total =
      __hip_atomic_load(&wp.gctr[(int64_t)item * 4 + 0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int leff = (int)min((int64_t)p.L, (int64_t)allowed_total);
  {
    constexpr int PER = NB / WB;
    uint32_t c[PER];
    uint32_t sum = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      c[i] = __hip_atomic_load(&gh[NB - 1 - ((int)threadIdx.x * PER + i)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sum += c[i];
    }
    uint32_t tot;
    const uint32_t before = block_excl_scan<WB>(sum, scratch, &tot);
    if (threadIdx.x == 0) {
      shared[1] = 0;  // threshold bin
      shared[2] = 0;  // count above it
    }
    __syncthreads();
    uint32_t run = before;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const uint32_t prev = run;
      run += c[i];
      if (leff > 0 && prev < (uint32_t)leff && run >= (uint32_t)leff) {
        shared[1] = NB - 1 - ((int)threadIdx.x * PER + i);
        shared[2] = prev;
      }
    }
    __syncthreads();
  }
  const uint32_t tbin = shared[1];
  const float* klow = p.k_low + (int64_t)h * p.klow_hs;
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  float* out_rank = p.sl_rank + (int64_t)item * p.L;
  uint32_t* ctr = wp.gctr + (int64_t)item * 4;
  uint64_t* ties = wp.ties + (int64_t)item * wp.tie_cap;
  uint64_t sure_mask = 0, tie_mask = 0;
  if (leff > 0) {
#pragma unroll
    for (int i = 0; i < KEYS; ++i) {
      const uint32_t bv = (bins[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      sure_mask |= (uint64_t)(bv != NOBIN && bv > tbin) << i;
      tie_mask |= (uint64_t)(bv == tbin) << i;
    }
  }
  const uint32_t n_sure = (uint32_t)__popcll(sure_mask), n_tie = (uint32_t)__popcll(tie_mask);
  uint32_t sure_tot, tie_tot;
  uint32_t s_off = block_excl_scan<WB>(n_sure, scratch, &sure_tot);
  uint32_t t_off = block_excl_scan<WB>(n_tie, scratch, &tie_tot);
  if (threadIdx.x == 0) {
    shared[3] = sure_tot;
    shared[4] = sure_tot ? atomicAdd(&ctr[1], sure_tot) : 0u;
    shared[5] = tie_tot ? atomicAdd(&ctr[2], tie_tot) : 0u;
  }
  __syncthreads();
  const uint32_t sure_base = shared[4], tie_base = shared[5];
  while (sure_mask | tie_mask) {
    const int i = __builtin_ctzll(sure_mask | tie_mask);
    const uint64_t bit = 1ull << i;
    const int n = cs + ((i / KPT) * WB + (int)threadIdx.x) * KPT + (i % KPT);
    if (sure_mask & bit) {
      const uint32_t slot = sure_base + s_off;
      if (slot < (uint32_t)p.L) {
        out_idx[slot] = n;
        if (s_off < (uint32_t)EMIT_CAP) {
          emit_n[s_off] = n;
          emit_slot[s_off] = slot;
        } else {
          out_rank[slot] = __uint_as_float(0x7FC0DEADu);  // rescored in phase C
        }
      }
      ++s_off;
    } else {
      const int64_t ts = (int64_t)tie_base + t_off;
      if (ts < wp.tie_cap) ties[ts] = composite(f2key(score_at<S>(codes, n, tab, C, sqrt_r)), (uint32_t)n);
      ++t_off;
    }
    sure_mask &= ~bit;
    tie_mask &= ~bit;
  }
  __syncthreads();
  {
    const int n_emit = (int)min(shared[3], (uint32_t)EMIT_CAP);
#pragma unroll 1
    for (int e = threadIdx.x; e < n_emit; e += WB) {
      const float* row = klow + (int64_t)emit_n[e] * p.R;
      out_rank[emit_slot[e]] = rank_dot64_stream(row, ql) / sqrt_r;
    }
  }
  __threadfence();
  cg::this_grid().sync();

  // ---- phase C: resolve the threshold bin (one workgroup per item) ---------
  if (w == 0) {
    const uint32_t above = shared[2];
    const int need = leff - (int)above;
    const uint32_t n_ties = __hip_atomic_load(&ctr[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int nt = (int)min((int64_t)n_ties, wp.tie_cap);
    if (leff > 0 && need > 0) {
      uint64_t X = 0;  // take every tie when exactly `need` of them exist
      if (nt != need) X = radix_select_u64<WB>([&](int i) { return ties[i]; }, nt, need, hist, scratch, shared + 4);
      if (threadIdx.x == 0) shared[3] = 0;
      __syncthreads();
#pragma unroll 1
      for (int i = threadIdx.x; i < nt; i += WB) {
        const uint64_t cmp = ties[i];
        if (cmp >= X) {
          const uint32_t j = atomicAdd(&shared[3], 1u);
          const uint32_t n = composite_index(cmp);
          if (above + j < (uint32_t)p.L && n < (uint32_t)N) {
            out_idx[above + j] = (int32_t)n;
            out_rank[above + j] = rank_dot64_stream(klow + (int64_t)n * p.R, ql) / sqrt_r;
          }
        }
      }
    }
    {
      // sure entries whose workgroup list overflowed carry a sentinel rank
      const int n_above = (int)min(above, (uint32_t)p.L);
#pragma unroll 1
      for (int j = threadIdx.x; j < n_above; j += WB) {
        const int32_t n = out_idx[j];
        if (__float_as_uint(out_rank[j]) == 0x7FC0DEADu && n >= 0 && n < N)
          out_rank[j] = rank_dot64_stream(klow + (int64_t)n * p.R, ql) / sqrt_r;
      }
    }
    if (threadIdx.x == 0) {
      p.sl_count[item] = leff;
      ctr[0] = 0u;
      ctr[1] = 0u;
      ctr[2] = 0u;
      ctr[3] = 0u;
    }
    uint32_t* ghw = wp.ghist + (int64_t)item * NB;
    for (int b = threadIdx.x; b < NB; b += WB) ghw[b] = 0u;
  }
}

template <int S, int RND>
const void* wide_fn() {
  return (const void*)summon_wide_kernel<S, RND>;
}

const void* wide_kernel_for(int S, int rnd) {
#define SVA_WIDE_CASE(SS, RR) \
  if (S == SS && rnd == RR) return wide_fn<SS, RR>();
  SVA_WIDE_CASE(1, 1) SVA_WIDE_CASE(1, 2) SVA_WIDE_CASE(1, 3) SVA_WIDE_CASE(1, 4)
  SVA_WIDE_CASE(2, 2) SVA_WIDE_CASE(2, 4) SVA_WIDE_CASE(2, 6) SVA_WIDE_CASE(2, 8)
  SVA_WIDE_CASE(4, 2) SVA_WIDE_CASE(4, 4) SVA_WIDE_CASE(4, 8) SVA_WIDE_CASE(4, 12) SVA_WIDE_CASE(4, 16)
  SVA_WIDE_CASE(8, 4) SVA_WIDE_CASE(8, 8) SVA_WIDE_CASE(8, 16) SVA_WIDE_CASE(8, 24) SVA_WIDE_CASE(8, 32)
#undef SVA_WIDE_CASE
  return nullptr;
}

const int* rnd_options(int S, int* count) {
  static const int r1[] = {1, 2, 3, 4};
  static const int r2[] = {2, 4, 6, 8};
  static const int r4[] = {2, 4, 8, 12, 16};
  static const int r8[] = {4, 8, 16, 24, 32};
  switch (S) {
    case 1: *count = 4; return r1;
    case 2: *count = 4; return r2;
    case 4: *count = 5; return r4;
    case 8: *count = 5; return r8;
    default: *count = 0; return nullptr;
  }
}

struct WidePlan {
  const void* fn;
  int W;
  int64_t chunk;
};

bool plan_wide(const SummonParams& p, int64_t items, WidePlan* plan) {
  int nopt = 0;
  const int* opts = rnd_options(p.S, &nopt);
  if (!opts) return false;
  const int kpt = 16 / p.S;
  const int cus = device_cu_count();
  for (int i = 0; i < nopt; ++i) {
    const void* fn = wide_kernel_for(p.S, opts[i]);
    if (!fn) continue;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, WB, 0) != hipSuccess || per_cu <= 0) continue;
    const int64_t resident = (int64_t)per_cu * cus;
    const int64_t w_max = resident / items;
    if (w_max < 2) continue;
    const int64_t per_wg = (int64_t)WB * kpt * opts[i];
    const int64_t w_need = (p.N + per_wg - 1) / per_wg;
    if (w_need > w_max) continue;
    // spread over as many workgroups as residency allows, keeping whole loads
    const int64_t W = std::max<int64_t>(w_need, std::min<int64_t>(w_max, (p.N + (int64_t)WB * kpt - 1) / ((int64_t)WB * kpt)));
    const int64_t step = (int64_t)WB * kpt;
    int64_t chunk = (p.N + W - 1) / W;
    chunk = (chunk + step - 1) / step * step;
    if (chunk > per_wg) continue;
    plan->fn = fn;
    plan->W = (int)((p.N + chunk - 1) / chunk);
    plan->chunk = chunk;
    return true;
  }
  return false;
}

}  // namespace

namespace sva {

bool summon_wide_eligible(const SummonParams& p, int64_t items) {
  if (p.Q != 1 || p.offs != nullptr || p.ctype != CODE_U8 || p.C > 256) return false;
  if (p.S != 1 && p.S != 2 && p.S != 4 && p.S != 8) return false;
  if (p.R != 64 || p.N < kWideMinKeys || p.N >= (1ll << 30) || items > kMaxWideItems) return false;
  if (((uintptr_t)p.codes & 15u) != 0 || p.code_hs % 16 != 0) return false;
  if (p.mask_type == MASK_F32 || p.mask_type == MASK_BF16 || p.mask_type == MASK_F16) {
    if (p.mask == nullptr) return false;
  }
  WidePlan plan;
  return plan_wide(p, items, &plan);
}

// Workspace layout: a fixed header of per-item histograms and counters for
// up to kMaxWideItems items (kept all-zero between calls: each call returns
// the entries it used to zero), then the tie buffers (one entry per key per
// item; no state carried across calls).  The header's offsets never depend
// on the cache length, so calls of different shapes can share one buffer.
constexpr size_t kWideHeader = (size_t)kMaxWideItems * (NB * sizeof(uint32_t) + 4 * sizeof(uint32_t));

size_t summon_wide_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t) {
  const int64_t items = n_seq * H * Q;
  if (n_seq != 1 || Q != 1 || n_keys < kWideMinKeys || items > kMaxWideItems) return 256;
  return kWideHeader + (size_t)items * (size_t)n_keys * sizeof(uint64_t) + 256;
}

int summon_wide_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int64_t items = (int64_t)p.H;  // one sequence, q = 1
  WidePlan plan;
  SVA_UNSUPPORTED(plan_wide(p, items, &plan), "sva_summon: no resident wide plan");
  const size_t need = summon_wide_workspace_bytes(1, p.H, 1, p.N, p.L);
  SVA_REQUIRE(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace & 255u) == 0,
              "sva_summon: workspace of %zu bytes (256-byte aligned, zero-filled) required, got %zu", need,
              workspace_bytes);
  WideParams wp;
  wp.p = p;
  wp.W = plan.W;
  wp.chunk = plan.chunk;
  char* ws = (char*)workspace;
  wp.ghist = (uint32_t*)ws;                         // [kMaxWideItems, NB]
  wp.gctr = wp.ghist + kMaxWideItems * NB;          // [kMaxWideItems, 4]
  wp.ties = (uint64_t*)(ws + kWideHeader);          // [items, N]
  wp.tie_cap = p.N;
  void* args[] = {&wp};
  const dim3 grid((unsigned)(items * plan.W));
  SVA_CHECK_HIP(hipLaunchCooperativeKernel(plan.fn, grid, dim3(WB), args, 0, stream), "summon_wide_kernel launch");
  SVA_CHECK_LAUNCH("summon_wide_kernel");
  return SVA_OK;
}

}  // namespace sva
