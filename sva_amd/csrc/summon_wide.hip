// Long-context summon for few query items (decode, q = 1): many workgroups
// per item, three kernels, no grid-wide synchronisation and no atomics on
// shared global words.
//
//   wide_scan     one workgroup per chunk of WB * 32 keys.  Streams the
//                 chunk's packed uint8 codes (16-byte loads, all in flight
//                 before use), scores every key through the LUT in the
//                 reference's order, and appends each allowed key whose sum
//                 reaches the item's sampled floor t_lo to its wave's own
//                 candidate list as a unique 64-bit composite (score key,
//                 key index); counts go to the wave's own counter words.
//   wide_select   one workgroup per item.  Gathers the candidates (~4x the
//                 shortlist for the sampled floor) into LDS and radix-selects
//                 the L largest composites exactly, writing their key
//                 indices.  When the floor overshot (fewer than L candidates)
//                 it selects over every key of the item instead: slower, same
//                 result.
//   wide_rescore  many workgroups per item: rank score of every shortlisted
//                 key (k_low . q_low in torch's sum order, 16 lanes per row).
// Selection equals a full sort by (score desc, key index asc): with R = 64
// the score is the sum / 8 exactly, so every key below the floor ranks
// strictly below every candidate.
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int WB = 256;          // threads per scan workgroup
constexpr int NW = WB / WAVE;    // waves per scan workgroup
constexpr int KEYS_PT = 32;      // keys per scan thread
constexpr int CHUNK = WB * KEYS_PT;
constexpr int WAVE_KEYS = WAVE * KEYS_PT;  // keys (and candidate capacity) per wave
constexpr int SB = 1024;         // threads of the select kernel
constexpr int SNW = SB / WAVE;
constexpr int LDS_CAND = 16384;  // candidates the select kernel stages in LDS
constexpr int RROWS = 64;        // rows per rescore workgroup
constexpr int RB = 256;          // threads per rescore workgroup
constexpr int64_t kWideMinKeys = 32768;
constexpr int64_t kMaxWideItems = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct WideArgs {
  SummonParams p;
  uint32_t* ncand;   // [items, W * NW] candidates of each scan wave
  uint32_t* nallow;  // [items, W * NW] allowed keys of each scan wave
  uint64_t* cand;    // [items, W * NW, WAVE_KEYS] candidate composites of each scan wave
  int W;             // scan workgroups per item
};

SVA_DEV uint32_t byte_of(const u32x4& v, int j) { return (v[j >> 2] >> (8 * (j & 3))) & 0xFFu; }

// Loads a chunk's codes: every full 16-byte group with one unconditional
// vector load (all issued before any is used); a partial last chunk falls
// back to guarded byte loads.
template <int S>
SVA_DEV void load_chunk(const uint8_t* __restrict__ codes, int cs, int ce, u32x4 (&raw)[KEYS_PT * S / 16]) {
  constexpr int KPT = 16 / S;
  constexpr int RND = KEYS_PT / KPT;
  if (ce - cs == CHUNK) {
#pragma unroll
    for (int r = 0; r < RND; ++r) {
      const int base = cs + (r * WB + (int)threadIdx.x) * KPT;
      raw[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + (int64_t)base * S));
    }
  } else {
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
  }
}

// Per-query tables for the scan.  BP: entry c of subspace s lives in lane c
// of reg[s] and is fetched with ds_bpermute (conflict-free; needs C <= 64 and
// all 64 lanes active).  Otherwise an LDS table of 256 entries per subspace
// (entries past C repeat entry C-1, so any uint8 code stays in bounds).
template <int S, bool BP>
struct ScanTables {
  float reg[BP ? S : 1];
  const float* tab;
  SVA_DEV void init(const SummonParams& p, int item, float* lds_tab) {
    const float* src = p.lut + (int64_t)item * S * p.C;
    if (BP) {
      const int c = min(lane_id(), p.C - 1);
#pragma unroll
      for (int s = 0; s < (BP ? S : 1); ++s) reg[s] = src[s * p.C + c];
    } else {
      for (int e = threadIdx.x; e < S * 256; e += blockDim.x) lds_tab[e] = src[(e >> 8) * p.C + min(e & 255, p.C - 1)];
      tab = lds_tab;
    }
  }
  SVA_DEV float get(int s, uint32_t c) const {
    if (BP) return __int_as_float(__builtin_amdgcn_ds_bpermute((int)(c << 2), __float_as_int(reg[BP ? s : 0])));
    return tab[s * 256 + c];
  }
};

// Scores the keys of one 16-byte round of the thread, branch-free so that
// the round's table lookups are in flight together: acc[k] = ((T0 + T1) +
// T2) + ... (the scan sum before the 1/8 scale; the reference's leading
// 0 + T0 only changes the sign of a zero).  bpermute lookups need all 64
// lanes, which this guarantees.  ds_bpermute reads only bits [7:2] of its
// address, so byte j of a word becomes a lane address with one shift (codes
// are below C <= 64 on that path).
template <int S, bool BP>
SVA_DEV void score_round(const u32x4& raw, const ScanTables<S, BP>& T, float (&acc)[16 / S]) {
#pragma clang fp contract(off)
  constexpr int KPT = 16 / S;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    float a = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int j = k * S + s;  // byte of the round
      float v;
      if (BP) {
        const uint32_t word = raw[j >> 2];
        const int sh = 8 * (j & 3);
        const uint32_t addr = sh == 0 ? word << 2 : word >> (sh - 2);
        v = __int_as_float(__builtin_amdgcn_ds_bpermute((int)addr, __float_as_int(T.reg[BP ? s : 0])));
      } else {
        v = T.get(s, byte_of(raw, j));
      }
      a = s == 0 ? v : a + v;
    }
    acc[k] = a;
  }
}

// Key index of slot i of this thread in the chunk starting at cs.
template <int S>
SVA_DEV int slot_key(int cs, int i) {
  constexpr int KPT = 16 / S;
  return cs + ((i / KPT) * WB + (int)threadIdx.x) * KPT + (i % KPT);
}

template <bool FULL, bool MASKED>
SVA_DEV bool key_ok(const SummonParams& p, int n, int ce) {
  bool ok = FULL || n < ce;
  if (MASKED && ok) ok = mask_allows(p.mask, n, p.mask_type);
  return ok;
}

// Rank score of a 64-float k_low row in torch's sum order, computed by the
// 16-lane group of the calling lane (lane j holds float4 j of the row; the
// pairing, lane chains and final order follow torch_order_dot64).  Every lane
// of the group receives the result.  All 16 lanes must call it.
SVA_DEV float rank_dot64_group16(const float* __restrict__ row, const float* __restrict__ q) {
#pragma clang fp contract(off)
  const int j = lane_id() & 15;
  const float4 r = reinterpret_cast<const float4*>(row)[j];
  const float4 qq = reinterpret_cast<const float4*>(q)[j];
  const float p0 = r.x * qq.x, p1 = r.y * qq.y, p2 = r.z * qq.z, p3 = r.w * qq.w;
  // element e (< 32) pairs with e + 32, held by lane j + 8
  const float a0 = (0.0f + p0) + __shfl_down(p0, 8, 16);
  const float a1 = (0.0f + p1) + __shfl_down(p1, 8, 16);
  const float a2 = (0.0f + p2) + __shfl_down(p2, 8, 16);
  const float a3 = (0.0f + p3) + __shfl_down(p3, 8, 16);
  // lanes g, g+2, g+4, g+6 hold accumulators 0..3 of lane-group g
  const float v0 = ((a0 + __shfl_down(a0, 2, 16)) + __shfl_down(a0, 4, 16)) + __shfl_down(a0, 6, 16);
  const float v1 = ((a1 + __shfl_down(a1, 2, 16)) + __shfl_down(a1, 4, 16)) + __shfl_down(a1, 6, 16);
  const float v2 = ((a2 + __shfl_down(a2, 2, 16)) + __shfl_down(a2, 4, 16)) + __shfl_down(a2, 6, 16);
  const float v3 = ((a3 + __shfl_down(a3, 2, 16)) + __shfl_down(a3, 4, 16)) + __shfl_down(a3, 6, 16);
  const float w0 = __shfl_down(v0, 1, 16), w1 = __shfl_down(v1, 1, 16);
  const float w2 = __shfl_down(v2, 1, 16), w3 = __shfl_down(v3, 1, 16);
  const float t = (((((((0.0f + v0) + v1) + v2) + v3) + w0) + w1) + w2) + w3;
  return __shfl(t, 0, 16);
}

// Exact score of key n from the global table (the reference's order, with the
// leading 0 + T0 and the division).  Used by the all-keys fallback only.
SVA_DEV float score_at(const SummonParams& p, const uint8_t* __restrict__ codes, int item, int n) {
#pragma clang fp contract(off)
  const float* lut = p.lut + (int64_t)item * p.S * p.C;
  float acc = 0.0f;
  for (int s = 0; s < p.S; ++s) {
    uint32_t c = codes[(int64_t)n * p.S + s];
    c = c < (uint32_t)p.C ? c : (uint32_t)(p.C - 1);
    acc = acc + lut[s * p.C + c];
  }
  return acc / p.sqrt_r;
}


// Candidate floor of an item: the sampled estimate, or the table minimum
// (every allowed key is a candidate) when there is none.
SVA_DEV float item_floor(const SummonParams& p, int item) {
  const float lo = p.range[4 * item + 0];
  const float est = p.range[4 * item + 2];
  return est > lo ? est : lo;
}

// Appends the keys of slot i whose flag c is set to the wave's candidate
// list (in lane order), as composites of the exact score acc / sqrt(R).
SVA_DEV void append_candidate(const SummonParams& p, bool c, float acc, int n, uint64_t* out, uint32_t& wc) {
#pragma clang fp contract(off)
  const uint64_t m = __builtin_amdgcn_ballot_w64(c);
  if (c) {
    const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    out[wc + below] = composite(f2key(acc / p.sqrt_r), (uint32_t)n);
  }
  wc += (uint32_t)__popcll(m);
}

// The scan of one thread's slots.  CHECK: the chunk is partial or masked, so
// every key is tested for being allowed; otherwise every key is, and a round
// (one 16-byte word of codes) is examined key by key only when its largest
// sum reaches the floor.
template <int S, bool BP, bool CHECK, bool MASKED>
SVA_DEV void scan_rounds(const SummonParams& p, const u32x4 (&raw)[KEYS_PT * S / 16], const ScanTables<S, BP>& T,
                         float t_lo, int cs, int ce, uint64_t* out, uint32_t& wc, uint32_t& n_allowed) {
  constexpr int KPT = 16 / S;
#pragma unroll
  for (int r = 0; r < KEYS_PT / KPT; ++r) {
    float acc[KPT];
    score_round<S, BP>(raw[r], T, acc);
    if (CHECK) {
      bool c[KPT];
      bool any = false;
#pragma unroll
      for (int k = 0; k < KPT; ++k) {
        const bool ok = key_ok<false, MASKED>(p, slot_key<S>(cs, r * KPT + k), ce);
        n_allowed += ok;
        c[k] = ok && acc[k] >= t_lo;
        any = any || c[k];
      }
      if (__builtin_amdgcn_ballot_w64(any) != 0ull) {
#pragma unroll
        for (int k = 0; k < KPT; ++k) append_candidate(p, c[k], acc[k], slot_key<S>(cs, r * KPT + k), out, wc);
      }
    } else {
      float mx = acc[0];
#pragma unroll
      for (int k = 1; k < KPT; ++k) mx = fmaxf(mx, acc[k]);
      if (__builtin_amdgcn_ballot_w64(mx >= t_lo) != 0ull) {  // rare: the shortlist and the keys near it
#pragma unroll
        for (int k = 0; k < KPT; ++k)
          append_candidate(p, acc[k] >= t_lo, acc[k], slot_key<S>(cs, r * KPT + k), out, wc);
      }
    }
  }
  if (!CHECK) n_allowed = KEYS_PT;
}

template <int S, bool BP, bool MASKED>
__global__ void __launch_bounds__(WB) wide_scan_kernel(WideArgs a) {
#pragma clang fp contract(off)
  __shared__ float tab_lds[BP ? 1 : S * 256];
  const SummonParams& p = a.p;
  const int item = blockIdx.x / a.W;
  const int w = blockIdx.x % a.W;
  const int h = item % p.H;
  const int cs = w * CHUNK;
  const int ce = (int)min((int64_t)cs + CHUNK, p.N);
  const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)h * p.code_hs;
  u32x4 raw[KEYS_PT * S / 16];
  load_chunk<S>(codes, cs, ce, raw);
  ScanTables<S, BP> T;
  T.init(p, item, tab_lds);
  const float t_lo = item_floor(p, item);
  if (!BP) __syncthreads();
  const int wid = threadIdx.x / WAVE;
  const int64_t sub = ((int64_t)item * a.W + w) * NW + wid;
  uint64_t* out = a.cand + sub * WAVE_KEYS;
  uint32_t n_allowed = 0;
  uint32_t wc = 0;  // candidates of this wave so far (wave-uniform)
  if (!MASKED && ce - cs == CHUNK) {
    scan_rounds<S, BP, false, false>(p, raw, T, t_lo, cs, ce, out, wc, n_allowed);
  } else {
    scan_rounds<S, BP, true, MASKED>(p, raw, T, t_lo, cs, ce, out, wc, n_allowed);
  }
  const uint32_t wa = wave_sum_u32(n_allowed);
  if (lane_id() == 0) {
    a.ncand[sub] = wc;
    a.nallow[sub] = wa;
  }
}

__global__ void __launch_bounds__(SB) wide_select_kernel(WideArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  uint64_t* cl = (uint64_t*)lds;                                   // [LDS_CAND]
  uint32_t(*whist)[256] = (uint32_t(*)[256])(cl + LDS_CAND);       // [SNW][256]
  uint64_t* shared64 = (uint64_t*)(whist + SNW);                   // [2]
  uint32_t* scratch = (uint32_t*)(shared64 + 2);                   // [SNW + 1]
  uint32_t* shared = scratch + SNW + 1;                            // [4]
  const SummonParams& p = a.p;
  const int item = blockIdx.x;
  const int nsub = a.W * NW;
  const uint32_t* ncand = a.ncand + (int64_t)item * nsub;
  const uint32_t* nallow = a.nallow + (int64_t)item * nsub;
  const uint64_t* cand = a.cand + (int64_t)item * nsub * WAVE_KEYS;
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  // totals: candidates M and allowed keys A.  With at most SB lists (every
  // cache up to 2M keys) one pass also yields each list's staging offset.
  const bool one_pass = nsub <= SB;
  uint32_t m = 0, al = 0;
  for (int s = threadIdx.x; s < nsub; s += SB) {
    m += ncand[s];
    al += nallow[s];
  }
  uint32_t M;
  const uint32_t my_base = block_excl_scan<SB>(m, scratch, &M);
  uint32_t A;
  block_excl_scan<SB>(al, scratch, &A);
  const int leff = (int)min((uint32_t)p.L, A);
  if (threadIdx.x == 0) {
    p.sl_count[item] = leff;
    shared[3] = 0u;  // output carry of the list-by-list path
  }
  if (leff == 0) return;
  if (M >= (uint32_t)leff && M <= (uint32_t)LDS_CAND) {
    // common case: stage the candidates contiguously in LDS, taking the
    // OR / AND bounds of the radix select on the way
    uint64_t vor = 0ull, vand = ~0ull;
    if (one_pass) {
      const int s = threadIdx.x;
      if (s < nsub) {
        const uint64_t* src = cand + (int64_t)s * WAVE_KEYS;
#pragma unroll 8
        for (uint32_t j = 0; j < m; ++j) {
          const uint64_t x = src[j];
          cl[my_base + j] = x;
          vor |= x;
          vand &= x;
        }
      }
    } else {
      uint32_t carry = 0;
      for (int g = 0; g < nsub; g += SB) {
        const int s = g + (int)threadIdx.x;
        const uint32_t c = s < nsub ? ncand[s] : 0u;
        uint32_t tot;
        const uint32_t base = carry + block_excl_scan<SB>(c, scratch, &tot);
        const uint64_t* src = cand + (int64_t)s * WAVE_KEYS;
#pragma unroll 8
        for (uint32_t j = 0; j < c; ++j) {
          const uint64_t x = src[j];
          cl[base + j] = x;
          vor |= x;
          vand &= x;
        }
        carry += tot;
      }
    }
    __syncthreads();
    const int Mi = (int)M;
    auto visit = [&](auto&& f) {
      for (int j = threadIdx.x; j < Mi; j += SB) f(cl[j]);
    };
    const uint64_t X = (uint32_t)leff == M
                           ? 1ull
                           : select_largest_with_bounds<SB>(visit, leff, vor, vand, whist, scratch, shared64, shared);
    // write the selected in staging order: contiguous ranges per thread
    const int per = (Mi + SB - 1) / SB;
    const int j0 = min(Mi, (int)threadIdx.x * per), j1 = min(Mi, j0 + per);
    uint32_t cnt = 0;
    for (int j = j0; j < j1; ++j) cnt += cl[j] >= X;
    uint32_t tot;
    uint32_t o = block_excl_scan<SB>(cnt, scratch, &tot);
    for (int j = j0; j < j1; ++j) {
      const uint64_t x = cl[j];
      if (x >= X && o < (uint32_t)leff) out_idx[o++] = (int32_t)composite_index(x);
    }
  } else if (M >= (uint32_t)leff) {
    // many candidates: select straight from the per-wave lists
    auto visit = [&](auto&& f) {
      for (int s = threadIdx.x; s < nsub; s += SB) {
        const uint32_t c = ncand[s];
        const uint64_t* src = cand + (int64_t)s * WAVE_KEYS;
        for (uint32_t j = 0; j < c; ++j) f(src[j]);
      }
    };
    const uint64_t X = (uint32_t)leff == M ? 1ull : select_largest<SB>(visit, leff, whist, scratch, shared64, shared);
    for (int g = 0; g < nsub; g += SB) {
      const int s = g + (int)threadIdx.x;
      const uint32_t c = s < nsub ? ncand[s] : 0u;
      const uint64_t* src = cand + (int64_t)s * WAVE_KEYS;
      uint32_t cnt = 0;
      for (uint32_t j = 0; j < c; ++j) cnt += src[j] >= X;
      uint32_t tot;
      uint32_t o = shared[3] + block_excl_scan<SB>(cnt, scratch, &tot);
      for (uint32_t j = 0; j < c; ++j)
        if (src[j] >= X && o < (uint32_t)leff) out_idx[o++] = (int32_t)composite_index(src[j]);
      __syncthreads();
      if (threadIdx.x == 0) shared[3] += tot;
      __syncthreads();
    }
  } else {
    // the sampled floor overshot: exact selection over every key of the item
    const int h = item % p.H;
    const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)h * p.code_hs;
    const int N = (int)p.N;
    auto key_at = [&](int n) -> uint64_t {
      if (!mask_allows(p.mask, n, p.mask_type)) return 0ull;
      return composite(f2key(score_at(p, codes, item, n)), (uint32_t)n);
    };
    auto visit = [&](auto&& f) {
      for (int n = threadIdx.x; n < N; n += SB) {
        const uint64_t x = key_at(n);
        if (x != 0ull) f(x);
      }
    };
    const uint64_t X = (uint32_t)leff == A ? 1ull : select_largest<SB>(visit, leff, whist, scratch, shared64, shared);
    const int per = (N + SB - 1) / SB;
    const int n0 = min(N, (int)threadIdx.x * per), n1 = min(N, n0 + per);
    uint32_t cnt = 0;
    for (int n = n0; n < n1; ++n) cnt += key_at(n) >= X;
    uint32_t tot;
    uint32_t o = block_excl_scan<SB>(cnt, scratch, &tot);
    for (int n = n0; n < n1; ++n)
      if (key_at(n) >= X && o < (uint32_t)leff) out_idx[o++] = n;
  }
}

constexpr size_t kSelectLds = sizeof(uint64_t) * (LDS_CAND + 2) + sizeof(uint32_t) * (SNW * 256 + SNW + 1 + 4);

// Rank scores of the shortlist: RROWS rows per workgroup, 16 lanes per row.
__global__ void __launch_bounds__(RB) wide_rescore_kernel(WideArgs a) {
  const SummonParams& p = a.p;
  const int item = blockIdx.y;
  const int h = item % p.H;
  const int count = p.sl_count[item];
  const int row0 = blockIdx.x * RROWS;
  if (row0 >= count) return;
  const float* ql = p.q_low + (int64_t)item * p.R;
  const float* klow = p.k_low + (int64_t)h * p.klow_hs;
  const int32_t* idx = p.sl_idx + (int64_t)item * p.L;
  float* rank = p.sl_rank + (int64_t)item * p.L;
  const int g = threadIdx.x >> 4;  // 16-lane group
  for (int r = row0 + g; r < row0 + RROWS; r += RB / 16) {
    if (r - g >= count) break;  // uniform per wave: every group of the wave passes the same r - g
    const bool valid = r < count;
    int32_t key = idx[valid ? r : row0];
    key = key < 0 ? 0 : (key >= (int32_t)p.N ? (int32_t)p.N - 1 : key);
    const float dot = rank_dot64_group16(klow + (int64_t)key * p.R, ql);
    if (valid && (lane_id() & 15) == 0) rank[r] = dot / p.sqrt_r;
  }
}

template <int S, bool BP, bool MASKED>
int launch_wide(const WideArgs& a, int64_t items, hipStream_t stream) {
  hipLaunchKernelGGL((wide_scan_kernel<S, BP, MASKED>), dim3((unsigned)(items * a.W)), dim3(WB), 0, stream, a);
  SVA_CHECK_LAUNCH("wide_scan_kernel");
  static bool attr_set = false;
  if (!attr_set) {
    SVA_CHECK_HIP(hipFuncSetAttribute((const void*)wide_select_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)kSelectLds),
                  "hipFuncSetAttribute(wide_select_kernel)");
    attr_set = true;
  }
  hipLaunchKernelGGL(wide_select_kernel, dim3((unsigned)items), dim3(SB), kSelectLds, stream, a);
  SVA_CHECK_LAUNCH("wide_select_kernel");
  const dim3 rgrid((unsigned)((a.p.L + RROWS - 1) / RROWS), (unsigned)items);
  hipLaunchKernelGGL(wide_rescore_kernel, rgrid, dim3(RB), 0, stream, a);
  SVA_CHECK_LAUNCH("wide_rescore_kernel");
  return SVA_OK;
}

template <int S>
int launch_wide_s(const WideArgs& a, int64_t items, bool masked, hipStream_t stream) {
  const bool bp = a.p.C <= 64;
  if (bp) return masked ? launch_wide<S, true, true>(a, items, stream) : launch_wide<S, true, false>(a, items, stream);
  return masked ? launch_wide<S, false, true>(a, items, stream) : launch_wide<S, false, false>(a, items, stream);
}

// Workspace: per-wave counters, then per-wave candidate lists.  Every word a
// call reads was written earlier in the same call, so no state is carried
// between calls and calls of any shape can share one buffer.
size_t counters_bytes(int64_t items, int64_t W) {
  return ((size_t)(2 * items * W * NW) * sizeof(uint32_t) + 255) & ~(size_t)255;
}

}  // namespace

namespace sva {

bool summon_wide_eligible(const SummonParams& p, int64_t items) {
  if (p.Q != 1 || p.offs != nullptr || p.ctype != CODE_U8 || p.C > 256) return false;
  if (p.S != 1 && p.S != 2 && p.S != 4 && p.S != 8) return false;
  if (p.R != 64 || p.N < kWideMinKeys || p.N >= (1ll << 30) || items > kMaxWideItems) return false;
  if (((uintptr_t)p.codes & 15u) != 0 || p.code_hs % 16 != 0) return false;
  if (((uintptr_t)p.k_low & 15u) != 0 || p.klow_hs % 4 != 0 || ((uintptr_t)p.q_low & 15u) != 0) return false;
  if (p.mask_type != MASK_NONE && p.mask_type != MASK_BOOL && p.mask == nullptr) return false;
  return true;
}

size_t summon_wide_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t) {
  const int64_t items = n_seq * H * Q;
  if (n_seq != 1 || Q != 1 || n_keys < kWideMinKeys || items > kMaxWideItems) return 256;
  const int64_t W = (n_keys + CHUNK - 1) / CHUNK;
  return counters_bytes(items, W) + (size_t)items * (size_t)W * CHUNK * sizeof(uint64_t);
}

int summon_wide_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int64_t items = (int64_t)p.H;  // one sequence, q = 1
  const size_t need = summon_wide_workspace_bytes(1, p.H, 1, p.N, p.L);
  SVA_REQUIRE(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace & 255u) == 0,
              "sva_summon: workspace of %zu bytes (256-byte aligned) required, got %zu", need, workspace_bytes);
  WideArgs a;
  a.p = p;
  a.W = (int)((p.N + CHUNK - 1) / CHUNK);
  char* ws = (char*)workspace;
  a.ncand = (uint32_t*)ws;
  a.nallow = a.ncand + items * a.W * NW;
  a.cand = (uint64_t*)(ws + counters_bytes(items, a.W));
  // a bool mask allows every key (the reference's `mask > -1e4` rule)
  const bool masked = p.mask_type == MASK_F32 || p.mask_type == MASK_BF16 || p.mask_type == MASK_F16;
  switch (p.S) {
    case 1: return launch_wide_s<1>(a, items, masked, stream);
    case 2: return launch_wide_s<2>(a, items, masked, stream);
    case 4: return launch_wide_s<4>(a, items, masked, stream);
    default: return launch_wide_s<8>(a, items, masked, stream);
  }
}

}  // namespace sva
