#pragma once
// Long-context summon for few query items (decode, q = 1): many workgroups
// per item for the scan, one per item for the finish (plus idle slice
// workgroups for the rare all-keys select); two kernels, no workgroup ever
// waits for another.
//
//   wide_scan     one workgroup per chunk of WB * 32 keys.  Loads the item's
//                 table and floor (sva_query_lut's outputs) first, then
//                 streams the chunk's packed uint8 codes (16-byte loads, all
//                 in flight before use), scores every key through the table
//                 in the reference's order, and appends each allowed key whose
//                 sum reaches the item's sampled floor t_lo to its wave's own
//                 candidate list as a unique 64-bit composite (score key, key
//                 index), with the candidate's rank score (k_low . q_low in
//                 torch's sum order) beside it; counts go to the wave's own
//                 counter words.
//   wide_finish   workgroup g < items finishes item g.  Gathers the
//                 candidates (about twice the shortlist for the sampled
//                 floor) and their ranks, compacts them through LDS into a
//                 dense register layout in ascending key order, selects the
//                 L largest composites exactly (shortlist) and, when a budget
//                 is asked for, the B best rank composites among them, and
//                 writes both in ascending key order; then (fused) runs the
//                 verifier over the budget list.  When the floor overshot
//                 (fewer than L candidates) the shortlist is selected over
//                 every key of the item instead, cut into K slices taken by
//                 workgroups g = item + j * items (which otherwise return at
//                 once); the workgroup completing the last slice, counted on
//                 a per-item arrival word, merges the slices and finishes.
// Selection equals a full sort by (score desc, key index asc): with R = 64
// the score is the sum / 8 exactly, so every key below the floor ranks
// strictly below every candidate.
//
// The kernels' variants are instantiated in summon_wide_*.hip, one
// translation unit per kernel family or verifier variant.
#include <algorithm>
#include <mutex>

#include "capi_internal.h"
#include "common.cuh"
#include "query.h"
#include "summon.h"

namespace sva {
namespace wide {


constexpr int WB = 256;          // threads per scan workgroup
constexpr int NW = WB / WAVE;    // waves per scan workgroup
constexpr int KEYS_PT = 32;      // keys per scan thread
constexpr int CHUNK = WB * KEYS_PT;
constexpr int WAVE_KEYS = WAVE * KEYS_PT;  // keys (and candidate capacity) per wave
constexpr int SB = 1024;         // threads of the select kernel
constexpr int SNW = SB / WAVE;
constexpr int LDS_CAND = 16384;  // candidates the finish kernel stages in LDS
constexpr int STAGE_LISTS = 4096;  // lists whose staging offsets the finish kernel keeps in LDS
// The wide path has R = 64: dividing by sqrt(R) = 8 equals multiplying by
// 0.125 exactly (both are the correctly rounded value of x / 8).
constexpr float kInvSqrtR = 0.125f;
constexpr int KL_CAP = 256;      // candidates per scan wave kept in LDS (composite and rank)
constexpr int WG_CAP = 128;      // candidates of a scan workgroup in its compact list
constexpr int64_t kWideMinKeys = 32768;
constexpr int64_t kMaxWideItems = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The fields a finish workgroup needs for its first loads lead the argument
// block, so that they share the scalar-cache lines its first loads fetch.
struct WideArgs {
  int W;               // scan workgroups per item
  int items;           // items of the call
  uint32_t* wg_count;  // [items, W, 2] candidates and allowed keys of each scan workgroup
  uint64_t* wg_cand;   // [items, W, WG_CAP] a workgroup's candidates in key order (when they fit)
  float* wg_rank;      // [items, W, WG_CAP] their rank scores
  SummonParams p;
  uint32_t* ncand;   // [items, W * NW] candidates of each scan wave
  uint32_t* nallow;  // [items, W * NW] allowed keys of each scan wave
  uint64_t* cand;    // [items, W * NW, WAVE_KEYS] candidate composites of each scan wave
  float* cand_rank;  // [items, W * NW, WAVE_KEYS] rank score of each listed candidate
  FusedVerify fv;    // fv.out != nullptr: the finish kernel also runs the verifier
  int32_t* overshoot;  // [items] or nullptr: 1 where the sampled floor overshot (all-keys select), else 0
  int K;               // slices of the all-keys select per item (finish grid: items * K workgroups)
  uint32_t* arrive;    // [items] slices of the all-keys select completed (zeroed by the scan kernel)
  uint32_t* slice_n;   // [items, K] entries of each slice list
  uint64_t* slice_list;  // [items, K, L] each slice's top composites in key order
};

SVA_DEV uint32_t byte_of(const u32x4& v, int j) { return (v[j >> 2] >> (8 * (j & 3))) & 0xFFu; }

// First key of round r of the calling lane: wave w of the workgroup owns keys
// [cs + w * WAVE_KEYS, cs + (w + 1) * WAVE_KEYS), and in round r its lanes
// take consecutive groups of 16 / S keys (one 16-byte word of codes each).
template <int S>
SVA_DEV int round_key(int cs, int r) {
  constexpr int KPT = 16 / S;
  return cs + (int)(threadIdx.x / WAVE) * WAVE_KEYS + (r * WAVE + lane_id()) * KPT;
}

// Loads a chunk's codes: a full chunk (FULL) with one unconditional vector
// load per 16-byte group, straight-line so that each round waits only for
// its own load; a partial last chunk falls back to guarded byte loads.
template <int S, bool FULL>
SVA_DEV void load_chunk(const uint8_t* __restrict__ codes, int cs, int ce, u32x4 (&raw)[KEYS_PT * S / 16]) {
  constexpr int KPT = 16 / S;
  constexpr int RND = KEYS_PT / KPT;
  if (FULL) {
#pragma unroll
    for (int r = 0; r < RND; ++r) {
      const int base = round_key<S>(cs, r);
      raw[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + (int64_t)base * S));
    }
  } else {
#pragma unroll
    for (int r = 0; r < RND; ++r) {
      const int base = round_key<S>(cs, r);
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

// Per-query tables for the scan, in LDS.  SMALLC (C <= 64): a pair table of
// subspaces 0 and 1, entry c0 + 64 c1 = T0[c0] + T1[c1], then the 64-entry
// tables of every subspace (the scan reads those of subspaces 2..); the pair
// sum equals the reference's (0 + T0) + T1 up to the sign of a zero, which
// f2key folds.  Otherwise 256-entry tables.
// Entries past C repeat entry C - 1, so every code stays in bounds.
template <int S, bool SMALLC>
struct ScanTables {
  static constexpr int PAIR = (SMALLC && S >= 2) ? 4096 : 0;
  static constexpr int SINGLE = SMALLC ? S * 64 : S * 256;  // entries of the single tables
  static constexpr int LDS_FLOATS = PAIR + SINGLE;
  static constexpr int NP = PAIR / WB;                 // pair entries per thread
  static constexpr int NS = (SINGLE + WB - 1) / WB;    // single entries per thread
  float ts[NS];
  const float* tab;
  // The single tables into registers, one coalesced read of the item's table
  // per workgroup (every workgroup of an item reads the same lines, so a
  // read per pair entry would queue thousands of requests on them): every
  // load issued, none waited for, so the caller can issue its code loads
  // behind them.
  SVA_DEV void load(const SummonParams& p, int item) {
    const float* src = p.lut + (int64_t)item * S * p.C;
    const int t = threadIdx.x;
    const int cm = p.C - 1;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int e = t + k * WB;
      ts[k] = 0.0f;
      if (e < SINGLE) {
        if (SMALLC) ts[k] = src[(e >> 6) * p.C + min(e & 63, cm)];
        else ts[k] = src[(e >> 8) * p.C + min(e & 255, cm)];
      }
    }
  }
  // Writes the tables to LDS (the caller synchronizes before use): the
  // single tables, then the pair table built from them (entry c0 + 64 c1 =
  // T0[c0] + T1[c1], thread t's c0 = t & 63 and c1 = t / 64 + 4 k).
  SVA_DEV void store(float* lds_tab) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NS; ++k)
      if (t + k * WB < SINGLE) lds_tab[PAIR + t + k * WB] = ts[k];
    tab = lds_tab;
    if (NP) {
      __syncthreads();  // the single tables
      const float a0 = lds_tab[PAIR + (t & 63)];
#pragma unroll
      for (int k = 0; k < NP; ++k) lds_tab[t + k * WB] = a0 + lds_tab[PAIR + 64 + ((t + k * WB) >> 6)];
    }
  }
  SVA_DEV float at_byte(uint32_t byte_offset) const {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + byte_offset);
  }
};

// Scores the keys of one 16-byte round of the thread, branch-free so that
// the round's table lookups are in flight together: acc[k] = ((T0 + T1) +
// T2) + ... (the scan sum before the 1/8 scale; the reference's leading
// 0 + T0 only changes the sign of a zero).  On the SMALLC path a code byte
// becomes a table byte offset with a shift and a mask (codes below 64; a
// larger byte reads the entry of its low six bits, inside the table).
template <int S, bool SMALLC>
SVA_DEV void score_round(const u32x4& raw, const ScanTables<S, SMALLC>& T, float (&acc)[16 / S]) {
#pragma clang fp contract(off)
  constexpr int KPT = 16 / S;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    float a = 0.0f;
    if (SMALLC && S == 4) {
      // codes below 64: y holds 4 c in each byte, and the pair offset
      // 4 c0 + 256 c1 is y's byte 0 beside x's byte 1 (one byte permute)
      const uint32_t x = raw[k] & 0x3F3F3F3Fu;
      const uint32_t y = x << 2;
      a = T.at_byte(__builtin_amdgcn_perm(y, x, 0x0C0C0104u));
      a = a + T.at_byte(__builtin_amdgcn_ubfe(y, 16, 8) + (uint32_t)(4 * (ScanTables<S, SMALLC>::PAIR + 2 * 64)));
      a = a + T.at_byte((y >> 24) + (uint32_t)(4 * (ScanTables<S, SMALLC>::PAIR + 3 * 64)));
    } else if (SMALLC) {
      const int j0 = k * S;
      if (S >= 2) {
        const uint32_t x = raw[j0 >> 2] >> (8 * (j0 & 3));
        a = T.at_byte(((x << 2) & 0xFCu) | (x & 0x3F00u));  // 4 (c0 + 64 c1)
      }
#pragma unroll
      for (int s = (S >= 2 ? 2 : 0); s < S; ++s) {
        const int j = j0 + s;
        const uint32_t word = raw[j >> 2];
        const int sh = 8 * (j & 3);
        const uint32_t off = ((sh == 0 ? word << 2 : word >> (sh - 2)) & 0xFCu) +
                             (uint32_t)(4 * (ScanTables<S, SMALLC>::PAIR + s * 64));
        const float v = T.at_byte(off);
        a = (S >= 2 || s > 0) ? a + v : v;
      }
    } else {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const float v = T.tab[s * 256 + byte_of(raw, k * S + s)];  // PAIR = 0 here
        a = s == 0 ? v : a + v;
      }
    }
    acc[k] = a;
  }
}

// Key index of slot i of this thread in the chunk starting at cs.
template <int S>
SVA_DEV int slot_key(int cs, int i) {
  constexpr int KPT = 16 / S;
  return round_key<S>(cs, i / KPT) + (i % KPT);
}

template <bool FULL, bool MASKED>
SVA_DEV bool key_ok(const SummonParams& p, int n, int ce) {
  bool ok = FULL || n < ce;
  if (MASKED && ok) ok = mask_allows(p.mask, n, p.mask_type);
  return ok;
}

// Candidate floor of an item: the sampled estimate, or the table minimum
// (every allowed key is a candidate) when there is none.
SVA_DEV float item_floor(const SummonParams& p, int item) {
  const float lo = p.range[4 * item + 0];
  const float est = p.range[4 * item + 2];
  return est > lo ? est : lo;
}

// LDS views of a scan wave's candidate lists.  A store that goes either to
// LDS or to global memory would otherwise be merged into one flat store, and
// a flat store makes the next round wait for every code load still in flight
// (a flat store may complete through either counter).
typedef __attribute__((address_space(3))) uint64_t lds_u64;
typedef __attribute__((address_space(3))) float lds_f32;

// Appends the flagged keys of one round (key n0 + k for flag c[k]) to the
// wave's candidate list in ascending key order (lanes in order, each lane's
// keys in order), as composites of the exact score acc / sqrt(R): the first
// KL_CAP to the wave's LDS list `kc`, later ones to its global list `out`
// (the LDS part follows there only if the workgroup has no compact list).
template <int KPT>
SVA_DEV void append_round(const SummonParams& p, const bool (&c)[KPT], const float (&acc)[KPT], int n0, uint64_t* out,
                          uint64_t* kc, uint32_t& wc) {
#pragma clang fp contract(off)
  uint32_t below = 0, tot = 0;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(c[k]);
    below += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    tot += (uint32_t)__popcll(m);
  }
  uint32_t o = wc + below;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    if (c[k]) {
      const uint64_t x = composite(f2key(acc[k] * kInvSqrtR), (uint32_t)(n0 + k));
      if (o < (uint32_t)KL_CAP) {
        ((lds_u64*)kc)[o] = x;
      } else {
        out[o] = x;
      }
      ++o;
    }
  }
  wc += tot;
}

// The scan of one thread's slots.  CHECK: the chunk is partial or masked, so
// every key is tested for being allowed; otherwise every key is, and a round
// (one 16-byte word of codes) is examined key by key only when its largest
// sum reaches the floor.  Full chunks of up to four subspaces score every
// round before any append, so the rounds' table reads are in flight
// together rather than each behind the branch of the round before (eight
// subspaces keep the per-round order: holding every round's sums would cost
// them a wave per SIMD).
template <int S, bool SMALLC, bool CHECK, bool MASKED>
SVA_DEV void scan_rounds(const SummonParams& p, const u32x4 (&raw)[KEYS_PT * S / 16], const ScanTables<S, SMALLC>& T,
                         float t_lo, int cs, int ce, uint64_t* out, uint64_t* kc, uint32_t& wc,
                         uint32_t& n_allowed) {
  constexpr int KPT = 16 / S;
  constexpr int RND = KEYS_PT / KPT;
  constexpr bool ALL_FIRST = !CHECK && S <= 4;
  if (ALL_FIRST) {
    float acc[RND][KPT];
#pragma unroll
    for (int r = 0; r < RND; ++r) score_round<S, SMALLC>(raw[r], T, acc[r]);
    uint64_t hit[RND];
#pragma unroll
    for (int r = 0; r < RND; ++r) {
      float mx = acc[r][0];
#pragma unroll
      for (int k = 1; k < KPT; ++k) mx = fmaxf(mx, acc[r][k]);
      hit[r] = __builtin_amdgcn_ballot_w64(mx >= t_lo);
    }
#pragma unroll
    for (int r = 0; r < RND; ++r) {
      if (hit[r] != 0ull) {  // rare: the shortlist and the keys near it
        bool c[KPT];
#pragma unroll
        for (int k = 0; k < KPT; ++k) c[k] = acc[r][k] >= t_lo;
        append_round<KPT>(p, c, acc[r], round_key<S>(cs, r), out, kc, wc);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < RND; ++r) {
      float acc[KPT];
      score_round<S, SMALLC>(raw[r], T, acc);
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
        if (__builtin_amdgcn_ballot_w64(any) != 0ull) append_round<KPT>(p, c, acc, round_key<S>(cs, r), out, kc, wc);
      } else {
        float mx = acc[0];
#pragma unroll
        for (int k = 1; k < KPT; ++k) mx = fmaxf(mx, acc[k]);
        if (__builtin_amdgcn_ballot_w64(mx >= t_lo) != 0ull) {  // rare: the shortlist and the keys near it
          bool c[KPT];
#pragma unroll
          for (int k = 0; k < KPT; ++k) c[k] = acc[k] >= t_lo;
          append_round<KPT>(p, c, acc, round_key<S>(cs, r), out, kc, wc);
        }
      }
    }
  }
  if (!CHECK) n_allowed = KEYS_PT;
}

// Rank scores of a scan wave's nc candidates (composites in the LDS list
// while they fit, else from the wave's candidate list): one 16-lane DPP row
// per candidate, 16 candidates in flight per wave; the first KL_CAP to the
// wave's LDS ranks `kr`, later ones beside the global list.
// qq: floats 4j .. 4j + 3 of the item's q_low for lane j of each DPP row.
// LDS_ONLY: every candidate is in the LDS list (nc <= KL_CAP, the usual
// case): no key is read from global memory, so the row loads of a group wait
// only for their keys' LDS reads (a possible global key read would make each
// row load wait for every load before it).
template <bool LDS_ONLY>
SVA_DEV void rank_list(const SummonParams& p, int item, const float4 qq, const uint64_t* kc, float* kr,
                       const uint64_t* out, float* rank, uint32_t nc) {
#pragma clang fp contract(off)
  const int j = lane_id() & 15;
  const int row = lane_id() >> 4;
  const float* klow = p.k_low + (int64_t)(item % p.H) * p.klow_hs;
  constexpr int RU = 4;
  for (uint32_t c0 = 0; c0 < nc; c0 += 4 * RU) {
    float4 rv[RU];
    uint32_t key[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const uint32_t c = c0 + 4 * u + row;
      const uint32_t cc = min(c, nc - 1);  // past the list: the last candidate again, its result unused
      key[u] = composite_index(LDS_ONLY || cc < (uint32_t)KL_CAP ? ((const lds_u64*)kc)[cc] : out[cc]);
      rv[u] = reinterpret_cast<const float4*>(klow + (int64_t)key[u] * p.R)[j];
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const float dot = rank_dot64_row16(rv[u], qq);
      const uint32_t c = c0 + 4 * u + row;
      if (c < nc && j == 0) {
        if (LDS_ONLY || c < (uint32_t)KL_CAP) {
          ((lds_f32*)kr)[c] = dot * kInvSqrtR;
        } else {
          rank[c] = dot * kInvSqrtR;
        }
      }
    }
  }
}

SVA_DEV void rank_candidates(const SummonParams& p, int item, const float4 qq, const uint64_t* kc, float* kr,
                             const uint64_t* out, float* rank, uint32_t nc) {
  if (nc <= (uint32_t)KL_CAP) {
    rank_list<true>(p, item, qq, kc, kr, out, rank, nc);
  } else {
    __threadfence();  // keys past the LDS list are read back from `out`
    rank_list<false>(p, item, qq, kc, kr, out, rank, nc);
  }
}

// One scan workgroup's chunk.  CHECK: a partial or masked chunk (every key
// tested for being allowed, guarded loads).  The item's table, floor and
// q_low are requested before the chunk's codes: every wave's loads return in
// order, so the tables are in LDS while the codes still stream and each
// round of codes is scored as soon as its own load lands.
// LDS of a scan workgroup beside its tables: each wave's first KL_CAP
// candidates (composites, ranks) and the waves' counts.
struct ScanLds {
  uint64_t kc[NW][KL_CAP];
  float kr[NW][KL_CAP];
  uint32_t wcnt[NW], walw[NW];
};

template <int S, bool SMALLC, bool CHECK, bool MASKED>
SVA_DEV void scan_chunk(const WideArgs& a, int item, int w, float* tab_lds, ScanLds& L) {
#pragma clang fp contract(off)
  const SummonParams& p = a.p;
  const int h = item % p.H;
  const int cs = w * CHUNK;
  const int ce = (int)min((int64_t)cs + CHUNK, p.N);
  const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)h * p.code_hs;
  ScanTables<S, SMALLC> T;
  T.load(p, item);
  const float t_lo = item_floor(p, item);
  const float4 qq = reinterpret_cast<const float4*>(p.q_low + (int64_t)item * p.R)[lane_id() & 15];
  u32x4 raw[KEYS_PT * S / 16];
  load_chunk<S, !CHECK>(codes, cs, ce, raw);
  T.store(tab_lds);
  __syncthreads();  // tables in LDS
  const int wid = threadIdx.x / WAVE;
  const int lane = lane_id();
  const int64_t sub = ((int64_t)item * a.W + w) * NW + wid;
  uint64_t* out = a.cand + sub * WAVE_KEYS;
  float* out_rank = a.cand_rank + sub * WAVE_KEYS;
  uint32_t n_allowed = 0;
  uint32_t wc = 0;  // candidates of this wave so far (wave-uniform)
  scan_rounds<S, SMALLC, CHECK, MASKED>(p, raw, T, t_lo, cs, ce, out, L.kc[wid], wc, n_allowed);
  rank_candidates(p, item, qq, L.kc[wid], L.kr[wid], out, out_rank, wc);
  const uint32_t wa = CHECK ? wave_sum_dpp(n_allowed) : (uint32_t)(WAVE * KEYS_PT);  // every key allowed
  if (lane == 0) {
    a.ncand[sub] = wc;
    a.nallow[sub] = wa;
    L.wcnt[wid] = wc;
    L.walw[wid] = wa;
  }
  // the workgroup's compact list: its waves' candidates in wave order (key
  // order), when there are at most WG_CAP of them (else each wave's LDS part
  // completes its global list); its counts either way
  __syncthreads();
  uint32_t off = 0, tot = 0, alw = 0;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    off += v < wid ? L.wcnt[v] : 0u;
    tot += L.wcnt[v];
    alw += L.walw[v];
  }
  const int64_t g = (int64_t)item * a.W + w;
  if (tot <= (uint32_t)WG_CAP) {
    for (uint32_t j = (uint32_t)lane; j < wc; j += WAVE) {
      a.wg_cand[g * WG_CAP + off + j] = L.kc[wid][j];
      a.wg_rank[g * WG_CAP + off + j] = L.kr[wid][j];
    }
  } else {
    const uint32_t nl = min(wc, (uint32_t)KL_CAP);
    for (uint32_t j = (uint32_t)lane; j < nl; j += WAVE) {
      out[j] = L.kc[wid][j];
      out_rank[j] = L.kr[wid][j];
    }
  }
  if (threadIdx.x == 0) {
    a.wg_count[2 * g] = tot;
    a.wg_count[2 * g + 1] = alw;
  }
}

// Five workgroups per CU (at most 102 VGPRs) keep every workgroup of a
// million-key, nine-head scan resident at once (up to four subspaces).
template <int S, bool SMALLC, bool MASKED>
__global__ void __launch_bounds__(WB, S <= 4 ? 5 : 1) wide_scan_kernel(WideArgs a) {
  __shared__ __align__(16) float tab_lds[ScanTables<S, SMALLC>::LDS_FLOATS];
  __shared__ ScanLds lds;
  const int item = blockIdx.x / a.W;
  const int w = blockIdx.x % a.W;
  if (blockIdx.x == 0)  // arrival counters of the finish kernel's all-keys select
    for (int i = threadIdx.x; i < a.items; i += WB) a.arrive[i] = 0u;
  if (!MASKED && (int64_t)(w + 1) * CHUNK <= a.p.N) {
    scan_chunk<S, SMALLC, false, false>(a, item, w, tab_lds, lds);
  } else {
    scan_chunk<S, SMALLC, true, MASKED>(a, item, w, tab_lds, lds);
  }
}

// LDS of the finish kernel.  The staging area holds gathered candidates (one
// of the paths); once the candidates sit in registers it is reused for the
// selection histogram, the shortlist, its rank composites and the last bucket
// of a selection.
constexpr int FIN_MAX_L = 8192;
constexpr size_t kFinStage = sizeof(uint64_t) * LDS_CAND;                       // 128 KB
constexpr size_t kFinHist = 0;                                                  // uint32[TOP_BINS]
constexpr size_t kFinSl = kFinHist + sizeof(uint32_t) * TOP_BINS;               // uint32[FIN_MAX_L]
constexpr size_t kFinRk = kFinSl + sizeof(uint32_t) * FIN_MAX_L;                // uint64[FIN_MAX_L]
constexpr size_t kFinSmall = kFinRk + sizeof(uint64_t) * FIN_MAX_L;             // uint64[TOP_SMALL]
constexpr size_t kFinLut = kFinSmall + sizeof(uint64_t) * TOP_SMALL;          // float[S * C], all-keys path
static_assert(kFinLut + sizeof(float) * 8 * 256 <= kFinStage, "finish LDS overlay");
// small arrays after the staging area (offsets keep every pointer in LDS)
constexpr size_t kFinWcnt = kFinStage;                                          // uint32[SNW * SNW]
constexpr size_t kFinScratch = kFinWcnt + sizeof(uint32_t) * SNW * SNW;         // uint32[SNW + 1]
constexpr size_t kFinShared = kFinScratch + sizeof(uint32_t) * (SNW + 2);       // uint32[4], 8-byte aligned
constexpr size_t kFinShared64 = kFinShared + sizeof(uint32_t) * 4;              // uint64[2]
constexpr size_t kFinRkb = kFinShared64 + sizeof(uint64_t) * 2;                 // uint32[2] rank key bounds
constexpr size_t kFinLcnt = kFinRkb + sizeof(uint32_t) * 2;                     // uint32[SB]
constexpr size_t kFinLoff = kFinLcnt + sizeof(uint32_t) * SB;                   // uint32[STAGE_LISTS]
constexpr size_t kFinLds = kFinLoff + sizeof(uint32_t) * STAGE_LISTS;
static_assert(kFinShared64 % 8 == 0, "8-byte LDS words");
static_assert(kFinLds <= (size_t)kMaxLds, "finish LDS");

// Dense path of the finish: every list holds at most DH * 16 candidates
// (DH = 2 or 3), there are at most DL_LISTS lists and at most NPD * SB
// candidates in all (the sampled floor aims at about 4K).  The lists are gathered straight into registers (16
// lanes per list, entries l + 16 h of lists k * DQ + q), then compacted
// through LDS into the dense order: candidate j of the concatenated lists at
// thread j % SB, slot j / SB, which is ascending key order.
constexpr int DQ = SB / 16;          // list groups of 16 lanes
constexpr int DK = 8;                // lists per group
constexpr int DL_LISTS = DQ * DK;    // 512 lists: caches up to 1M keys
constexpr int NPD = 7;              // dense slots per thread

// Rank score of a 64-float k_low row in torch's sum order, computed here
// for the all-keys path: rows r of sl, one 16-lane DPP row each.
SVA_DEV void rank_rows(const SummonParams& p, int item, const uint32_t* sl, int n, float* out) {
#pragma clang fp contract(off)
  const int j = lane_id() & 15;
  const float4 qq = reinterpret_cast<const float4*>(p.q_low + (int64_t)item * p.R)[j];
  const float* klow = p.k_low + (int64_t)(item % p.H) * p.klow_hs;
  for (int r = threadIdx.x >> 4; r < n; r += SB / 16) {
    const float dot = rank_dot64_row16(reinterpret_cast<const float4*>(klow + (int64_t)sl[r] * p.R)[j], qq);
    if (j == 0) out[r] = dot * kInvSqrtR;
  }
}

// Order-preserving compaction of register-held elements: element i of
// thread t stands at position t + i * BLOCK of the source order; the
// elements >= X (nonzero) get their rank o in that order, at most cap of
// them, passed as emit(o, element, i).  Slots from `slots` on are empty.
// wcnt: NPT * BLOCK / 64 uint32 in LDS.  Every thread must call it.
template <int BLOCK, int NPT, typename Emit>
SVA_DEV void compact_ordered(const uint64_t (&e)[NPT], uint64_t X, int cap, uint32_t* wcnt, uint32_t* scratch,
                             int slots, Emit emit) {
  constexpr int NWV = BLOCK / WAVE;
  const int wid = threadIdx.x / WAVE;
  const int lane = lane_id();
  uint64_t bal[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    bal[i] = 0ull;
    if (i < slots) bal[i] = __builtin_amdgcn_ballot_w64(e[i] != 0ull && e[i] >= X);
    if (lane == 0) wcnt[i * NWV + wid] = (uint32_t)__popcll(bal[i]);
  }
  __syncthreads();
  {
    const uint32_t c = threadIdx.x < NPT * NWV ? wcnt[threadIdx.x] : 0u;
    uint32_t tot;
    const uint32_t off = block_excl_scan<BLOCK>(c, scratch, &tot);
    if (threadIdx.x < NPT * NWV) wcnt[threadIdx.x] = off;
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    if (i < slots && e[i] != 0ull && e[i] >= X) {
      const uint32_t o = wcnt[i * NWV + wid] +
                         __builtin_amdgcn_mbcnt_hi((uint32_t)(bal[i] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal[i], 0u));
      if (o < (uint32_t)cap) emit(o, e[i], i);
    }
  }
}

// Budget of an item: the beff largest rank composites among the nonzero
// e2 (leff of them, dense), compacted in slot order (ascending key order) to fin.
template <int NPT>
SVA_DEV void finish_budget(const SummonParams& p, int item, int leff, int beff, const uint64_t (&e2)[NPT], uint64_t vor,
                           uint64_t vand, bool bounds_given, const TopLds& tl, uint32_t* wcnt, uint32_t* scratch) {
  const int slots = (leff + SB - 1) / SB;
  const uint64_t X2 = beff == leff ? 1ull : select_top_regs<SB, NPT>(e2, beff, vor, vand, tl, slots, bounds_given);
  int32_t* fin = p.fin_idx + (int64_t)item * p.B;
  compact_ordered<SB, NPT>(e2, X2, beff, wcnt, scratch, slots,
                           [&](uint32_t o, uint64_t x, int) { fin[o] = (int32_t)composite_index(x); });
}

// Sparse gather of the dense path: lane (q, l) loads entries l + 16 h of
// lists k * DQ + q of `src` (entries past a list's count are read but
// unused; every read stays inside the list's capacity).
template <int DH, typename T>
SVA_DEV void gather_lists(const T* src, int nsub, T (&v)[DH * DK]) {
  const int q = threadIdx.x >> 4, l = threadIdx.x & 15;
  const int kq = (nsub + DQ - 1) / DQ;
#pragma unroll
  for (int k = 0; k < DK; ++k) {
#pragma unroll
    for (int h = 0; h < DH; ++h) v[DH * k + h] = T(0);
    if (k < kq) {  // uniform
      const int64_t off = (int64_t)min(k * DQ + q, nsub - 1) * WAVE_KEYS + l;
#pragma unroll
      for (int h = 0; h < DH; ++h) v[DH * k + h] = src[off + 16 * h];
    }
  }
}

// Moves sparse register entries (list sidx, entry j) to dense slots:
// position loff[sidx] + j of the concatenated lists goes to thread
// position % SB, slot position / SB.  stage: LDS of at least M elements.
template <int DH, typename T>
SVA_DEV void densify(const T (&v)[DH * DK], T (&d)[NPD], T* stage, const uint32_t* lcnt, const uint32_t* loff,
                     int nsub, int dslots, uint32_t M) {
  const int t = threadIdx.x, q = t >> 4, l = t & 15;
  const int kq = (nsub + DQ - 1) / DQ;
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    const int sidx = k * DQ + q;
    if (k < kq && sidx < nsub) {
      const uint32_t c = lcnt[sidx], base = loff[sidx];
#pragma unroll
      for (int h = 0; h < DH; ++h)
        if ((uint32_t)(l + 16 * h) < c) stage[base + l + 16 * h] = v[DH * k + h];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    const uint32_t j = (uint32_t)(t + i * SB);
    d[i] = (i < dslots && j < M) ? stage[j] : T(0);
  }
  __syncthreads();  // the staging area is free again
}

// Dense path (see wide_finish_kernel): the item's leff shortlist keys and
// beff budget keys, both in ascending key order, from its M candidates held
// sparse in e_sp.  The ranks are gathered here, behind the composites'
// compaction and shortlist select.
template <int DH>
SVA_DEV void finish_dense(const WideArgs& a, int item, int nsub, int leff, int beff, uint32_t M, uint64_t c_lo,
                          uint64_t c_hi, const uint64_t (&e_sp)[DH * DK], unsigned char* stage, const uint32_t* lcnt,
                          const uint32_t* loff, uint32_t* rkb, uint32_t* wcnt, uint32_t* scratch, const TopLds& tl) {
#pragma clang fp contract(off)
  const SummonParams& p = a.p;
  const int dslots = ((int)M + SB - 1) / SB;
  float r_sp[DH * DK];
  gather_lists<DH>(a.cand_rank + (int64_t)item * nsub * WAVE_KEYS, nsub, r_sp);
  uint64_t e[NPD];
  densify<DH>(e_sp, e, (uint64_t*)stage, lcnt, loff, nsub, dslots, M);
  // shortlist: the leff largest score composites
  const uint64_t X = (uint32_t)leff == M ? 1ull : select_top_regs<SB, NPD>(e, leff, c_hi, c_lo, tl, dslots, true);
  float r[NPD];
  densify<DH>(r_sp, r, (float*)stage, lcnt, loff, nsub, dslots, M);
  // budget: the beff largest (rank key, key index) composites of the shortlist
  uint64_t rc[NPD];
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    rc[i] = 0ull;
    if (i < dslots && e[i] != 0ull && e[i] >= X) {
      const uint32_t rkey = f2key(r[i]);
      rc[i] = composite(rkey, composite_index(e[i]));
      kmin = min(kmin, rkey);
      kmax = max(kmax, rkey);
    }
  }
  uint64_t XB = 1ull;
  if (p.B > 0 && beff < leff) {
    wave_min_max_u32(kmin, kmax);
    if (lane_id() == 0 && kmin <= kmax) {
      atomicMin(&rkb[0], kmin);
      atomicMax(&rkb[1], kmax);
    }
    __syncthreads();
    const uint64_t b_lo = (uint64_t)rkb[0] << 32, b_hi = ((uint64_t)rkb[1] << 32) | 0xFFFFFFFFull;
    XB = select_top_regs<SB, NPD>(rc, beff, b_hi, b_lo, tl, dslots, true);
  }
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  float* out_rank = p.sl_rank + (int64_t)item * p.L;
  compact_ordered<SB, NPD>(e, X, leff, wcnt, scratch, dslots, [&](uint32_t o, uint64_t x, int i) {
    out_idx[o] = (int32_t)composite_index(x);
    out_rank[o] = r[i];
  });
  if (p.B > 0) {
    int32_t* fin = p.fin_idx + (int64_t)item * p.B;
    compact_ordered<SB, NPD>(rc, XB, beff, wcnt, scratch, dslots,
                             [&](uint32_t o, uint64_t x, int) { fin[o] = (int32_t)composite_index(x); });
  }
}

// ---------------------------------------------------------------------------
// Fast finish (every scan workgroup's candidates fit its compact list, at
// most FAST_LISTS workgroups per item, at most FAST_M candidates).
//   fill     every wave loads its share of the compact lists and places them
//            in LDS in list order (ascending key order) at offsets from a
//            wave-level scan of the list counts;
//   select   each thread takes its dense slots into registers; the shortlist
//            threshold comes from one histogram pass over the 32-bit score
//            keys in value bins over [floor, highest candidate], then an exact
//            rank of the boundary bin's members; the budget threshold the
//            same way over the shortlist's rank keys;
//   output   one ordered compaction writes the shortlist and the budget.
// Selection equals the (score desc, key index asc) top-k: bins are monotone
// in the score and the boundary bin is resolved on the full composites.
constexpr int FAST_LISTS = 256;  // scan workgroups per item (caches up to 2M keys)
constexpr int FAST_M = NPD * SB;  // candidates staged in LDS
constexpr int FAST_BATCH = 8;     // lists a wave loads per round
constexpr int SMALL_CAP = 256;    // boundary-bin members ranked directly
constexpr size_t kFastComp = 0;                                              // uint64[FAST_M]
constexpr size_t kFastRank = kFastComp + sizeof(uint64_t) * FAST_M;          // float[FAST_M]
constexpr size_t kFastHist = kFastRank + sizeof(float) * FAST_M;             // uint32[4096]
constexpr size_t kFastSmall = kFastHist + sizeof(uint32_t) * 4096;           // uint64[SMALL_CAP]
constexpr size_t kFastMisc = kFastSmall + sizeof(uint64_t) * SMALL_CAP;      // uint32[96]
constexpr size_t kFastEnd = kFastMisc + sizeof(uint32_t) * 96;
// over the staged candidates once they sit in registers (fused budget histogram)
constexpr size_t kFastRHist = kFastComp;                                      // uint32[4096]
constexpr size_t kFastSmallR = kFastRHist + sizeof(uint32_t) * 4096;          // float[SMALL_CAP]
static_assert(kFastSmallR + sizeof(float) * SMALL_CAP <= kFastRank, "budget histogram over the staged composites");
static_assert(WG_CAP == 2 * WAVE, "two compact-list entries per lane");
static_assert(kFastEnd <= kFinStage, "the fast finish stays inside the finish kernel's staging area");

// Exclusive scan within a wave (all 64 lanes active).
SVA_DEV uint32_t wave_excl_scan(uint32_t v) { return wave_incl_scan(v) - v; }
SVA_DEV uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Exclusive prefix sums, in place, of the n <= 2 * WAVE per-(slot, wave)
// count words wcnt[] (two packed 16-bit counts each), by the first wave
// alone; the caller synchronizes before and after.
SVA_DEV void slot_wave_offsets(uint32_t* wcnt, int n) {
  if (threadIdx.x >= WAVE) return;
  const int lane = lane_id();
  const uint32_t v0 = 2 * lane < n ? wcnt[2 * lane] : 0u;
  const uint32_t v1 = 2 * lane + 1 < n ? wcnt[2 * lane + 1] : 0u;
  const uint32_t b = wave_excl_scan(v0 + v1);
  if (2 * lane < n) wcnt[2 * lane] = b;
  if (2 * lane + 1 < n) wcnt[2 * lane + 1] = b + v0;
}
static_assert(NPD * SNW <= 2 * WAVE, "two (slot, wave) counts per lane of one wave");

// LDS scalars of the fast finish (misc): per-wave values at [16 * slot + wave], slots 0..4.
struct FastMisc {
  uint32_t* m;
  SVA_DEV uint32_t& wave(int slot, int w) const { return m[16 * slot + w]; }
  SVA_DEV uint32_t& res(int k) const { return m[80 + k]; }
  SVA_DEV uint64_t& res64() const { return *reinterpret_cast<uint64_t*>(m + 88); }
};

// Optional work of a shortlist select for the budget select that follows:
// the rank of every shortlisted key binned into rhist (4096 bins linear in
// the candidates' rank range [rlo, rlo + 4096 / rinv)), so the budget select
// starts from a built histogram.  smallr holds the boundary members' ranks.
struct RankFuse {
  uint32_t* rhist;
  float* smallr;
  float rlo, rinv;
};

// Threshold of the k largest nonzero composites held in e[] (dense slots),
// binned by their scores v[] (the float each composite's key encodes) into
// 4096 bins linear in [lo, lo + 4096 / inv_w): bin = (v - lo) * inv_w
// (clamped), a non-decreasing function of v, so the bins order the
// composites and only the boundary bin's members need ranking.  Values >=
// the result are exactly the k largest.  Every thread of the block calls
// it; hist must be zero on entry.  Uses misc slots 0 and res.  *exact is
// false (result 0) when the boundary bin holds more than SMALL_CAP members.
SVA_DEV int lin_bin(float v, float lo, float inv_w) {
  const float b = (v - lo) * inv_w;
  return b < 1.0f ? 0 : (b >= 4095.0f ? 4095 : (int)b);
}

// FUSE: rf's rank histogram is built on the way (rv: the elements' ranks);
// built: hist already holds the elements' bins (phase 1 skipped).
template <bool FUSE = false>
SVA_DEV uint64_t fast_select(const uint64_t (&e)[NPD], const float (&v)[NPD], int dslots, int k, float lo, float inv_w,
                             uint32_t* hist, uint64_t* small, const FastMisc& f, bool* exact, bool built = false,
                             const float (*rv)[NPD] = nullptr, const RankFuse* rf = nullptr) {
#pragma clang fp contract(off)
  const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
  if (!built) {
#pragma unroll
    for (int i = 0; i < NPD; ++i)
      if (i < dslots && e[i] != 0ull) atomicAdd(&hist[lin_bin(v[i], lo, inv_w)], 1u);
  }
  __syncthreads();
  if (FUSE) reinterpret_cast<uint4*>(rf->rhist)[t] = uint4{0u, 0u, 0u, 0u};  // the staging it overlays is read
  // thread t owns bins 4095 - 4 t - j (j = 0..3), from the top
  const uint4 h = reinterpret_cast<const uint4*>(hist)[1023 - t];
  const uint32_t c[4] = {h.w, h.z, h.y, h.x};
  const uint32_t mine = c[0] + c[1] + c[2] + c[3];
  const uint32_t incl = wave_incl_scan(mine);
  if (lane == WAVE - 1) f.wave(0, wid) = incl;
  __syncthreads();
  uint32_t above = incl - mine;
  for (int w = 0; w < wid; ++w) above += f.wave(0, w);
  {
    uint32_t a = above;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (a < (uint32_t)k && a + c[j] >= (uint32_t)k) {
        f.res(0) = 4095u - 4u * (uint32_t)t - (uint32_t)j;
        f.res(1) = a;
        f.res(2) = c[j];
      }
      a += c[j];
    }
  }
  if (t == 0) f.res(3) = 0u;
  __syncthreads();
  const int b = (int)f.res(0);
  const uint32_t need = (uint32_t)k - f.res(1), cnt = f.res(2);
  *exact = true;
  if (cnt > (uint32_t)SMALL_CAP) {
    // a massive tie class: the general register select
    *exact = false;
    return 0ull;
  }
  // the boundary bin's members, then each one's rank among them (FUSE: the
  // keys of higher bins, all shortlisted, bin their ranks)
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    if (i < dslots) {  // uniform
      const int bin = lin_bin(v[i], lo, inv_w);
      const bool in = e[i] != 0ull && bin == b;
      if (FUSE && e[i] != 0ull && bin > b) atomicAdd(&rf->rhist[lin_bin((*rv)[i], rf->rlo, rf->rinv)], 1u);
      const uint64_t m = __builtin_amdgcn_ballot_w64(in);
      if (m != 0ull) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&f.res(3), (uint32_t)__popcll(m));
        base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);  // every lane is active here
        if (in) {
          small[base + lanes_below(m)] = e[i];
          if (FUSE) rf->smallr[base + lanes_below(m)] = (*rv)[i];
        }
      }
    }
  }
  __syncthreads();
  {
    // four lanes per member: lane q of member g compares it with members q, q + 4, ...
    const int g = t >> 2, q = t & 3;
    const uint64_t x = g < (int)cnt ? small[g] : 0ull;
    uint32_t greater = 0;
    for (int o = q; o < (int)cnt; o += 4) greater += small[o] > x ? 1u : 0u;
    greater = quad_sum(greater);
    if (q == 0 && g < (int)cnt && greater == need - 1u) f.res64() = x;
    if (FUSE && q == 0 && g < (int)cnt && greater < need)  // a selected boundary member
      atomicAdd(&rf->rhist[lin_bin(rf->smallr[g], rf->rlo, rf->rinv)], 1u);
  }
  __syncthreads();
  return f.res64();
}

// 4096 / (hi - lo), or 0 (one bin) when the range is empty.
SVA_DEV float lin_scale(float lo, float hi) { return hi > lo ? 4096.0f / (hi - lo) : 0.0f; }

// The fast finish of an item; false (uniformly, before any output or LDS
// write) when its conditions do not hold.
SVA_DEV bool finish_fast(const WideArgs& a, int item, unsigned char* lds, uint32_t* rkb, uint32_t* wcnt,
                         uint32_t* scratch, const TopLds& tl, int32_t* kidl, int& beff_out) {
#pragma clang fp contract(off)
  const SummonParams& p = a.p;
  const int W = a.W;
  if (W > FAST_LISTS) return false;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wid = t / WAVE;
  const int64_t g0 = (int64_t)item * W;
  // Every load below is issued unconditionally (indices clamped to the last
  // list, values past it ignored): a load under a condition leaves the
  // compiler unsure how many loads follow an earlier one, and it then waits
  // for all of them where it needs the first.
  // list counts: lane j holds lists 4j .. 4j + 3
  uint32_t cnt_raw[4], alw_raw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int l = min(4 * lane + i, W - 1);
    cnt_raw[i] = a.wg_count[2 * (g0 + l)];
    alw_raw[i] = a.wg_count[2 * (g0 + l) + 1];
  }
  // the first round of this wave's lists (16 k + wid, k < FAST_BATCH), issued
  // with the counts: the first WAVE slots of each list (a list's later slots,
  // rarely filled, are requested after every list's first slots are placed)
  uint64_t comp[FAST_BATCH];
  float rank[FAST_BATCH];
  auto load_round = [&](int r) {
#pragma unroll
    for (int k = 0; k < FAST_BATCH; ++k) {
      const int l = min(SNW * (r * FAST_BATCH + k) + wid, W - 1);
      comp[k] = a.wg_cand[(g0 + l) * WG_CAP + lane];
      rank[k] = a.wg_rank[(g0 + l) * WG_CAP + lane];
    }
  };
  load_round(0);
  // the shortlist select's score histogram, filled as the candidates are
  // placed: 4096 bins linear in [floor, bound of any sum] (zeroed while the
  // loads are in flight; the bounds are read before the barrier, which no
  // load may cross)
  const float vlo = item_floor(p, item) * kInvSqrtR;
  const float vinv = lin_scale(vlo, p.range[4 * item + 1] * kInvSqrtR);
  uint32_t* hist = (uint32_t*)(lds + kFastHist);
  reinterpret_cast<uint4*>(hist)[t] = uint4{0u, 0u, 0u, 0u};
  __syncthreads();
  uint32_t tot[4], loc[4], lsum = 0, asum = 0;
  bool over = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool in = 4 * lane + i < W;
    tot[i] = in ? cnt_raw[i] : 0u;
    asum += in ? alw_raw[i] : 0u;
    loc[i] = lsum;
    lsum += tot[i];
    over = over || tot[i] > (uint32_t)WG_CAP;
  }
  const uint32_t M = wave_sum_dpp(lsum), A = wave_sum_dpp(asum);
  const bool overflow = __builtin_amdgcn_ballot_w64(over) != 0ull;
  const int leff = (int)min((uint32_t)p.L, A);
  const int beff = min(p.B, leff);
  if (overflow || M > (uint32_t)FAST_M || M < (uint32_t)leff) return false;
  beff_out = p.B > 0 ? beff : 0;
  if (t == 0) {
    p.sl_count[item] = leff;
    if (p.B > 0) p.fin_count[item] = beff;
  }
  if (leff == 0) return true;
  uint64_t* lcomp = (uint64_t*)(lds + kFastComp);
  float* lrank = (float*)(lds + kFastRank);
  uint64_t* small = (uint64_t*)(lds + kFastSmall);
  const FastMisc f{(uint32_t*)(lds + kFastMisc)};
  const uint32_t base = wave_excl_scan(lsum);
  // list 16 k + wid lives in lane (16 k + wid) / 4 at element wid % 4
  const int el = wid & 3;
  const uint32_t my_off = base + (el == 0 ? loc[0] : el == 1 ? loc[1] : el == 2 ? loc[2] : loc[3]);
  const uint32_t my_tot = el == 0 ? tot[0] : el == 1 ? tot[1] : el == 2 ? tot[2] : tot[3];
  uint32_t rkmin = 0xFFFFFFFFu, rkmax = 0u;  // rank keys placed by this lane
  auto place = [&](uint32_t at, uint64_t x, float rx) {
    lcomp[at] = x;
    lrank[at] = rx;
    atomicAdd(&hist[lin_bin(key2f((uint32_t)(x >> 32)), vlo, vinv)], 1u);
    rkmin = min(rkmin, f2key(rx));
    rkmax = max(rkmax, f2key(rx));
  };
  bool tails = false;  // some list of this wave holds more than WAVE candidates
  for (int r = 0; r * FAST_BATCH * SNW < W; ++r) {
    if (r > 0) load_round(r);
#pragma unroll
    for (int k = 0; k < FAST_BATCH; ++k) {
      const int l = SNW * (r * FAST_BATCH + k) + wid;
      if (l < W) {  // uniform
        const int src = l >> 2;
        const uint32_t o = (uint32_t)__shfl((int)my_off, src, WAVE);
        const uint32_t c = (uint32_t)__shfl((int)my_tot, src, WAVE);
        if ((uint32_t)lane < c) place(o + lane, comp[k], rank[k]);
        tails = tails || c > (uint32_t)WAVE;
      }
    }
  }
  if (tails) {  // uniform: the slots past WAVE of this wave's long lists
    for (int l = wid; l < W; l += SNW) {
      const int src = l >> 2;
      const uint32_t o = (uint32_t)__shfl((int)my_off, src, WAVE);
      const uint32_t c = (uint32_t)__shfl((int)my_tot, src, WAVE);
      for (uint32_t j = WAVE + lane; j < c; j += WAVE)
        place(o + j, a.wg_cand[(g0 + l) * WG_CAP + j], a.wg_rank[(g0 + l) * WG_CAP + j]);
    }
  }
  wave_min_max_u32(rkmin, rkmax);
  if (lane == 0) {
    f.wave(3, wid) = rkmin;
    f.wave(4, wid) = rkmax;
  }
  __syncthreads();
  // dense slots in registers: candidate t + i SB at thread t, slot i (list order)
  const int dslots = ((int)M + SB - 1) / SB;
  uint64_t e[NPD];
  float rv[NPD];
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    const int j = t + i * SB;
    const bool in = i < dslots && j < (int)M;
    e[i] = in ? lcomp[j] : 0ull;
    rv[i] = in ? lrank[j] : 0.0f;
  }
  uint32_t rklo = 0xFFFFFFFFu, rkhi = 0u;
  for (int v = 0; v < SNW; ++v) {
    rklo = min(rklo, f.wave(3, v));
    rkhi = max(rkhi, f.wave(4, v));
  }
  bool exact = true;
  uint64_t X = 1ull;
  // the budget select's histogram is built by the shortlist select, over the
  // rank range of every candidate
  const bool fuse = (uint32_t)leff < M && p.B > 0 && beff < leff;
  const RankFuse rf{(uint32_t*)(lds + kFastRHist), (float*)(lds + kFastSmallR), key2f(rklo),
                    lin_scale(key2f(rklo), key2f(rkhi))};
  if ((uint32_t)leff < M) {
    float sv[NPD];
#pragma unroll
    for (int i = 0; i < NPD; ++i) sv[i] = key2f((uint32_t)(e[i] >> 32));
    X = fuse ? fast_select<true>(e, sv, dslots, leff, vlo, vinv, hist, small, f, &exact, true, &rv, &rf)
             : fast_select(e, sv, dslots, leff, vlo, vinv, hist, small, f, &exact, true);
    if (!exact) {
      __syncthreads();
      return false;  // a tie class too large to rank directly: the general paths
    }
  }
  // budget composites of the shortlist: (rank key, key index)
  uint64_t rc[NPD];
  uint32_t rmin = 0xFFFFFFFFu, rmax = 0u;
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    rc[i] = 0ull;
    if (i < dslots && e[i] != 0ull && e[i] >= X) {
      const uint32_t rk = f2key(rv[i]);
      rc[i] = composite(rk, composite_index(e[i]));
      rmin = min(rmin, rk);
      rmax = max(rmax, rk);
    }
  }
  uint64_t XB = 1ull;
  if (fuse) {
    bool ex2 = true;
    XB = fast_select(rc, rv, dslots, beff, rf.rlo, rf.rinv, rf.rhist, small, f, &ex2, true);
    if (!ex2) {
      __syncthreads();
      return false;
    }
  } else if (p.B > 0 && beff < leff) {
    wave_min_max_u32(rmin, rmax);
    if (lane == 0) {
      f.wave(1, wid) = rmin;
      f.wave(2, wid) = rmax;
    }
    reinterpret_cast<uint4*>(hist)[t] = uint4{0u, 0u, 0u, 0u};
    __syncthreads();
    uint32_t lo = 0xFFFFFFFFu, hi = 0u;
    for (int v = 0; v < SNW; ++v) {
      lo = min(lo, f.wave(1, v));
      hi = max(hi, f.wave(2, v));
    }
    bool ex2 = true;
    const float rlo = key2f(lo);
    XB = fast_select(rc, rv, dslots, beff, rlo, lin_scale(rlo, key2f(hi)), hist, small, f, &ex2);
    if (!ex2) {
      __syncthreads();
      return false;
    }
  }
  // outputs in list order (ascending key order): per (slot, wave) counts of
  // both selections packed in one word, one scan, then the writes
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    if (i < dslots) {  // uniform
      const bool sl = e[i] != 0ull && e[i] >= X;
      const uint64_t ml = __builtin_amdgcn_ballot_w64(sl);
      const uint64_t mb = __builtin_amdgcn_ballot_w64(sl && rc[i] >= XB);
      if (lane == 0) wcnt[i * SNW + wid] = (uint32_t)__popcll(ml) | ((uint32_t)__popcll(mb) << 16);
    }
  }
  __syncthreads();
  slot_wave_offsets(wcnt, dslots * SNW);
  __syncthreads();
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  float* out_rank = p.sl_rank + (int64_t)item * p.L;
  int32_t* fin = p.B > 0 ? p.fin_idx + (int64_t)item * p.B : nullptr;
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    if (i < dslots) {  // uniform
      const uint32_t w = wcnt[i * SNW + wid];
      const uint32_t key = composite_index(e[i]);
      const bool sl = e[i] != 0ull && e[i] >= X;
      const bool sb = sl && rc[i] >= XB;
      const uint64_t ml = __builtin_amdgcn_ballot_w64(sl);
      const uint64_t mb = __builtin_amdgcn_ballot_w64(sb);
      if (sl) {
        const uint32_t o = (w & 0xFFFFu) + lanes_below(ml);
        if (o < (uint32_t)leff) {
          out_idx[o] = (int32_t)key;
          out_rank[o] = rv[i];
        }
      }
      if (fin != nullptr && sb) {
        const uint32_t o = (w >> 16) + lanes_below(mb);
        if (o < (uint32_t)beff) {
          fin[o] = (int32_t)key;
          if (kidl != nullptr) kidl[o] = (int32_t)key;
        }
      }
    }
  }
  return true;
}

// Finish of an item: shortlist select, its outputs with the ranks the scan
// computed, and (B > 0) the budget select, one workgroup per item.  The
// candidate lists are in ascending key order, and so is every output.
//   dense   (every list <= 48 entries, <= 512 lists, M <= 8192): lists
//           and ranks gathered into registers, 16 lanes per list, moved
//           through LDS to dense slots in ascending key order, both selects
//           and both ordered compactions there;
//   staged  (M <= LDS_CAND, <= STAGE_LISTS lists): lists staged in LDS in
//           list order, then into registers; the selected find their list
//           (binary search over the staging offsets) for their ranks;
//           slot-ordered compaction;
//   lists   (more candidates): selection straight from the global lists;
//   all keys (the sampled floor let fewer than L keys through): selection
//           over every key of the item, ranks computed here.
// The last two are slower and give the same result.  The shortlist's rank
// composites go to LDS in shortlist order for the budget.
// ---------------------------------------------------------------------------
// The all-keys select, for an item whose sampled floor overshot (fewer than
// leff candidates at or above it): the item's keys are cut into a.K slices of
// consecutive keys, one finish workgroup each (slice 0 is the item's own
// workgroup, slices 1 .. K-1 extra workgroups of the grid that return at once
// when the floor held).  Each slice writes its min(leff, allowed) largest
// composites in key order to the workspace; the workgroup that completes the
// item's last slice (a device-wide arrival counter, zeroed by the scan
// kernel) selects the item's leff largest among the slices' lists (a superset
// of them: no key outside a slice's top leff can be among the item's top
// leff) and finishes the item.  No workgroup waits for another.
//
// A slice is selected in two passes over its codes, read as 16-byte words,
// sixteen per thread in flight with every load instruction of a wave covering
// 1 KB in a row, and scored from the table in LDS exactly as the scan scores
// them:
//   pass 1: histogram of the scores over 4096 bins linear in [lo, hi] (the
//           bounds of any sum); b = the bin holding the k-th largest;
//   pass 2: composites of higher bins (fewer than k) into a list, bin b's
//           members (at most kOverBound) into LDS, sorted descending: the
//           first `need` of them complete the list, which is then sorted into
//           key order.
// A boundary bin beyond kOverBound members (a tie class) falls back to the
// radix select over the slice.
constexpr int kOverBound = 4096;     // boundary-bin members sorted in LDS
constexpr int kOverWords = 16;       // code words per thread in flight
constexpr int kOverSlicesMax = 16;   // slices per item
constexpr int kOverGrid = 256;       // items * slices at most (one workgroup per CU)
constexpr size_t kOverList = kFinSl;                                    // uint64[FIN_MAX_L] slice list
constexpr size_t kOverBnd = kOverList + sizeof(uint64_t) * FIN_MAX_L;   // uint64[kOverBound]
static_assert(kOverBnd + sizeof(uint64_t) * kOverBound <= kFinSmall, "slice select LDS below the table");

// Slices of the all-keys select for `items` items.
inline int over_slices(int64_t items) { return (int)std::max<int64_t>(1, std::min<int64_t>(kOverSlicesMax, kOverGrid / items)); }

// Keys per slice: a multiple of 16, so every slice starts on a 16-byte code word.
SVA_DEV int slice_keys(int N, int K) { return ((((N + K - 1) / K) + 15) / 16) * 16; }

// Composite <-> (key index, score key) in key-major order, for sorting by key.
SVA_DEV uint64_t by_key(uint64_t x) { return ((uint64_t)composite_index(x) << 32) | (x >> 32); }
SVA_DEV uint64_t from_key(uint64_t y) { return composite((uint32_t)y, (uint32_t)(y >> 32)); }

// Calls f(key, composite) for every key of [n0, n1) (n0 a multiple of 16):
// the exact scan score's composite, 0 for a key the mask excludes.
template <int S, typename F>
SVA_DEV void overshoot_visit(const SummonParams& p, const uint8_t* __restrict__ codes, const float* lut_l, int n0,
                             int n1, F&& f) {
#pragma clang fp contract(off)
  constexpr int KPW = 16 / S;  // keys per 16-byte code word
  const int C = p.C;
  const uint32_t cm = (uint32_t)(C - 1);
  const bool masked = p.mask_type == MASK_F32 || p.mask_type == MASK_BF16 || p.mask_type == MASK_F16;
  const int wbeg = n0 / KPW, wend = (n1 + KPW - 1) / KPW;
  // word w0 + u * SB + t for u < kOverWords: every load instruction of a wave reads 1 KB in a row
  for (int w0 = wbeg; w0 < wend; w0 += kOverWords * SB) {
    u32x4 w[kOverWords];
#pragma unroll
    for (int u = 0; u < kOverWords; ++u) {
      const int base = (w0 + u * SB + (int)threadIdx.x) * KPW;
      if (base + KPW <= n1) {
        w[u] = *reinterpret_cast<const u32x4*>(codes + (int64_t)base * S);
      } else {
        uint32_t wv[4] = {0u, 0u, 0u, 0u};
        for (int j = 0; j < KPW * S; ++j)
          if (base + j / S < n1) wv[j >> 2] |= (uint32_t)codes[(int64_t)base * S + j] << (8 * (j & 3));
        w[u] = u32x4{wv[0], wv[1], wv[2], wv[3]};
      }
    }
#pragma unroll
    for (int u = 0; u < kOverWords; ++u) {
      const int base = (w0 + u * SB + (int)threadIdx.x) * KPW;
#pragma unroll
      for (int j = 0; j < KPW; ++j) {
        const int key = base + j;
        if (key < n1) {
          float acc = 0.0f;
#pragma unroll
          for (int s2 = 0; s2 < S; ++s2) acc = acc + lut_l[s2 * C + min(byte_of(w[u], j * S + s2), cm)];
          const bool ok = !masked || mask_allows(p.mask, key, p.mask_type);
          f(key, ok ? composite(f2key(acc * kInvSqrtR), (uint32_t)key) : 0ull);
        }
      }
    }
  }
}

// Bitonic sort of P (a power of two) LDS elements in place, descending or ascending.
template <typename T, bool DESC>
SVA_DEV void lds_bitonic(T* a, int P) {
  const int t = threadIdx.x;
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = t; i < P / 2; i += SB) {
        const int lo_i = 2 * i - (i & (j - 1));  // index with bit j clear
        const int hi_i = lo_i + j;
        const bool desc = ((lo_i & k) == 0) == DESC;
        const T x = a[lo_i], y = a[hi_i];
        if ((x < y) == desc) {
          a[lo_i] = y;
          a[hi_i] = x;
        }
      }
      __syncthreads();
    }
  }
}

// The bin of the k-th largest of a 4096-bin histogram (block-wide).
struct Boundary {
  uint32_t k;      // min(k, total counted)
  uint32_t b;      // the bin of the k-th largest (when k > 0)
  uint32_t above;  // elements in higher bins (< k)
  uint32_t cnt;    // elements in bin b
};

SVA_DEV Boundary hist_boundary(const uint32_t* hist, uint32_t k, uint32_t* scratch, uint32_t* shared) {
  const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
  // thread t owns bins 4095 - 4 t - j, from the top
  const uint4 hv = reinterpret_cast<const uint4*>(hist)[SB - 1 - t];
  const uint32_t c[4] = {hv.w, hv.z, hv.y, hv.x};
  const uint32_t mine = c[0] + c[1] + c[2] + c[3];
  const uint32_t incl = wave_incl_scan(mine);
  if (lane == WAVE - 1) scratch[wid] = incl;
  __syncthreads();
  uint32_t a = incl - mine, total = 0u;
  for (int v = 0; v < SNW; ++v) {
    total += scratch[v];
    if (v < wid) a += scratch[v];
  }
  const uint32_t kk = min(k, total);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (a < kk && a + c[j] >= kk) {
      shared[1] = 4095u - 4u * (uint32_t)t - (uint32_t)j;
      shared[2] = a;
      shared[3] = c[j];
    }
    a += c[j];
  }
  __syncthreads();
  const Boundary r{kk, shared[1], shared[2], shared[3]};
  __syncthreads();
  return r;
}

// Exact composite of key n (0 when masked out), scalar: the tie-class fallback's visitor.
SVA_DEV uint64_t key_composite(const SummonParams& p, const uint8_t* codes, const float* lut_l, int n) {
#pragma clang fp contract(off)
  if (!mask_allows(p.mask, n, p.mask_type)) return 0ull;
  // the reference's exact score ((0 + T0[c0]) + T1[c1]) + ... then / sqrt(R)
  float acc = 0.0f;
  for (int s2 = 0; s2 < p.S; ++s2) {
    uint32_t c = codes[(int64_t)n * p.S + s2];
    c = c < (uint32_t)p.C ? c : (uint32_t)(p.C - 1);
    acc = acc + lut_l[s2 * p.C + c];
  }
  return composite(f2key(acc * kInvSqrtR), (uint32_t)n);
}

// The top min(k, allowed) composites of keys [n0, n1) of an item, in key
// order, to out (global); returns their number (block-uniform).
template <int S>
SVA_DEV uint32_t slice_select(const SummonParams& p, int item, uint32_t k, int n0, int n1, const float* lut_l,
                              unsigned char* lds, uint32_t* scratch, uint32_t* shared, uint64_t* shared64,
                              uint64_t* __restrict__ out) {
  const int t = threadIdx.x;
  uint32_t* hist = (uint32_t*)(lds + kFinHist);
  uint64_t* lst = (uint64_t*)(lds + kOverList);
  uint64_t* bnd = (uint64_t*)(lds + kOverBnd);
  const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)(item % p.H) * p.code_hs;
  const float lo = p.range[4 * item] * kInvSqrtR, hi = p.range[4 * item + 1] * kInvSqrtR;
  const float inv_w = lin_scale(lo, hi);
  reinterpret_cast<uint4*>(hist)[t] = uint4{0u, 0u, 0u, 0u};
  __syncthreads();
  overshoot_visit<S>(p, codes, lut_l, n0, n1, [&](int, uint64_t x) {
    if (x != 0ull) atomicAdd(&hist[lin_bin(key2f((uint32_t)(x >> 32)), lo, inv_w)], 1u);
  });
  __syncthreads();
  const Boundary bd = hist_boundary(hist, k, scratch, shared);
  if (bd.k == 0u) return 0u;
  if (bd.cnt > (uint32_t)kOverBound) {
    // a tie class beyond the LDS sort: radix passes over the slice, then its keys >= X in key order
    uint32_t(*whist)[256] = (uint32_t(*)[256])hist;
    auto visit = [&](auto&& f) {
      for (int n = n0 + t; n < n1; n += SB) {
        const uint64_t x = key_composite(p, codes, lut_l, n);
        if (x != 0ull) f(x);
      }
    };
    const uint64_t X = select_largest<SB>(visit, (int)bd.k, whist, scratch, shared64, shared);
    const int per = (n1 - n0 + SB - 1) / SB;
    const int m0 = min(n1, n0 + t * per), m1 = min(n1, m0 + per);
    uint32_t cnt = 0;
    for (int n = m0; n < m1; ++n) cnt += key_composite(p, codes, lut_l, n) >= X;
    uint32_t o = block_excl_scan<SB>(cnt, scratch, nullptr);
    for (int n = m0; n < m1; ++n) {
      const uint64_t x = key_composite(p, codes, lut_l, n);
      if (x >= X && o < bd.k) out[o++] = x;
    }
    return bd.k;
  }
  if (t == 0) {
    shared[0] = 0u;       // boundary-bin members
    scratch[SNW] = 0u;    // higher-bin composites
  }
  __syncthreads();
  overshoot_visit<S>(p, codes, lut_l, n0, n1, [&](int, uint64_t x) {
    if (x == 0ull) return;
    const uint32_t bin = (uint32_t)lin_bin(key2f((uint32_t)(x >> 32)), lo, inv_w);
    if (bin > bd.b) lst[atomicAdd(&scratch[SNW], 1u)] = by_key(x);
    else if (bin == bd.b) bnd[atomicAdd(&shared[0], 1u)] = x;
  });
  __syncthreads();
  int P = 1;
  while (P < (int)bd.cnt) P <<= 1;
  for (int i = (int)bd.cnt + t; i < P; i += SB) bnd[i] = 0ull;
  __syncthreads();
  lds_bitonic<uint64_t, true>(bnd, P);
  // the higher bins' composites, then the best `need` of the boundary bin, sorted by key
  const uint32_t need = bd.k - bd.above;
  for (int i = t; i < (int)need; i += SB) lst[bd.above + i] = by_key(bnd[i]);
  int PL = 1;
  while (PL < (int)bd.k) PL <<= 1;
  for (int i = (int)bd.k + t; i < PL; i += SB) lst[i] = ~0ull;
  __syncthreads();
  lds_bitonic<uint64_t, false>(lst, PL);
  for (int i = t; i < (int)bd.k; i += SB) out[i] = from_key(lst[i]);
  return bd.k;
}

// The item's leff largest composites among its K slice lists (key order
// within a list, lists in key-range order), as key indices in key order into
// sl (LDS).  offs: LDS uint32[K + 1].
SVA_DEV void merge_slices(const WideArgs& a, int item, uint32_t leff, unsigned char* lds, uint32_t* sl, uint32_t* offs,
                          uint32_t* scratch, uint32_t* shared, uint64_t* shared64) {
  const SummonParams& p = a.p;
  const int t = threadIdx.x, K = a.K;
  uint32_t* hist = (uint32_t*)(lds + kFinHist);
  uint64_t* bnd = (uint64_t*)(lds + kOverBnd);
  const uint64_t* lists = a.slice_list + (int64_t)item * K * p.L;
  if (t == 0) {
    uint32_t o = 0u;
    for (int j = 0; j < K; ++j) {
      offs[j] = o;
      o += a.slice_n[(int64_t)item * K + j];
    }
    offs[K] = o;
  }
  __syncthreads();
  const uint32_t U = offs[K];
  auto visit = [&](auto&& f) {
    for (int j = 0; j < K; ++j) {
      const uint32_t n = offs[j + 1] - offs[j];
      for (uint32_t e = t; e < n; e += SB) f(lists[(int64_t)j * p.L + e]);
    }
  };
  uint64_t X = 1ull;  // every listed composite (U == leff)
  if (U > leff) {
    const float lo = p.range[4 * item] * kInvSqrtR, hi = p.range[4 * item + 1] * kInvSqrtR;
    const float inv_w = lin_scale(lo, hi);
    reinterpret_cast<uint4*>(hist)[t] = uint4{0u, 0u, 0u, 0u};
    __syncthreads();
    visit([&](uint64_t x) { atomicAdd(&hist[lin_bin(key2f((uint32_t)(x >> 32)), lo, inv_w)], 1u); });
    __syncthreads();
    const Boundary bd = hist_boundary(hist, leff, scratch, shared);
    if (bd.cnt > (uint32_t)kOverBound) {
      X = select_largest<SB>(visit, (int)leff, (uint32_t(*)[256])hist, scratch, shared64, shared);
    } else {
      if (t == 0) shared[0] = 0u;
      __syncthreads();
      visit([&](uint64_t x) {
        if ((uint32_t)lin_bin(key2f((uint32_t)(x >> 32)), lo, inv_w) == bd.b) bnd[atomicAdd(&shared[0], 1u)] = x;
      });
      __syncthreads();
      int P = 1;
      while (P < (int)bd.cnt) P <<= 1;
      for (int i = (int)bd.cnt + t; i < P; i += SB) bnd[i] = 0ull;
      __syncthreads();
      lds_bitonic<uint64_t, true>(bnd, P);
      X = bnd[leff - bd.above - 1];
      __syncthreads();
    }
  }
  // composites >= X in key order: thread t takes entries [t c, (t + 1) c) of the lists laid end to end
  const uint32_t c = (U + SB - 1) / SB;
  const uint32_t e0 = min(U, (uint32_t)t * c), e1 = min(U, e0 + c);
  auto at = [&](uint32_t e, int& j) {
    while (offs[j + 1] <= e) ++j;
    return lists[(int64_t)j * p.L + (e - offs[j])];
  };
  uint32_t cnt = 0;
  int j = 0;
  for (uint32_t e = e0; e < e1; ++e) cnt += at(e, j) >= X;
  uint32_t o = block_excl_scan<SB>(cnt, scratch, nullptr);
  j = 0;
  for (uint32_t e = e0; e < e1; ++e) {
    const uint64_t x = at(e, j);
    if (x >= X && o < leff) sl[o++] = composite_index(x);
  }
  __syncthreads();
}

// Finish of an item by slice `slice` of its finish workgroups: returns 1
// (budget list in LDS) or 0 (in the budget output) when this workgroup
// finished the item, -1 when it has nothing more to do (a slice workgroup
// whose item's floor held, or that did not complete the item's last slice).
SVA_DEV int finish_item(const WideArgs& a, int item, int slice, unsigned char* lds, int32_t* kidl, int& beff_out) {
#pragma clang fp contract(off)
  uint64_t* cl = (uint64_t*)lds;                                   // staged candidates [LDS_CAND]
  uint32_t* hist = (uint32_t*)(lds + kFinHist);                    // overlays, once staging is done
  uint32_t* sl = (uint32_t*)(lds + kFinSl);
  uint64_t* rk = (uint64_t*)(lds + kFinRk);
  uint64_t* small = (uint64_t*)(lds + kFinSmall);
  uint32_t* wcnt = (uint32_t*)(lds + kFinWcnt);
  uint32_t* scratch = (uint32_t*)(lds + kFinScratch);
  uint32_t* shared = (uint32_t*)(lds + kFinShared);
  uint64_t* shared64 = (uint64_t*)(lds + kFinShared64);
  uint32_t* rkb = (uint32_t*)(lds + kFinRkb);
  uint32_t* lcnt = (uint32_t*)(lds + kFinLcnt);
  uint32_t* loff = (uint32_t*)(lds + kFinLoff);
  const TopLds tl{hist, small, scratch, shared, shared64};
  const SummonParams& p = a.p;
  if (slice == 0 && finish_fast(a, item, lds, rkb, wcnt, scratch, tl, kidl, beff_out)) return kidl != nullptr ? 1 : 0;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int nsub = a.W * NW;
  const uint32_t* ncand = a.ncand + (int64_t)item * nsub;
  const uint32_t* nallow = a.nallow + (int64_t)item * nsub;
  const uint64_t* cand = a.cand + (int64_t)item * nsub * WAVE_KEYS;
  const float* crank = a.cand_rank + (int64_t)item * nsub * WAVE_KEYS;
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  float* out_rank = p.sl_rank + (int64_t)item * p.L;
  // 1. list counts, their offsets in list order (nsub <= SB), totals:
  // candidates M, allowed keys A, longest list
  if (t == 0) {
    shared[1] = 0u;  // longest list (nsub <= SB)
    shared[3] = 0u;  // A
    rkb[0] = 0xFFFFFFFFu;  // smallest and largest rank key of the shortlist
    rkb[1] = 0u;
  }
  uint32_t m = 0, al = 0;
  for (int sidx = t; sidx < nsub; sidx += SB) {
    m += ncand[sidx];
    al += nallow[sidx];
  }
  if (nsub <= SB) lcnt[t] = m;
  uint32_t M;
  const uint32_t list_off = block_excl_scan<SB>(m, scratch, &M);
  if (nsub <= SB) loff[t] = list_off;
  {
    const uint32_t wa = wave_sum_dpp(al);
    uint32_t mn = m, mx = m;
    wave_min_max_u32(mn, mx);
    if (lane == 0) {
      atomicAdd(&shared[3], wa);
      atomicMax(&shared[1], mx);
    }
  }
  __syncthreads();
  const uint32_t A = shared[3];
  const uint32_t longest = shared[1];
  const int leff = (int)min((uint32_t)p.L, A);
  const int beff = min(p.B, leff);
  if (slice > 0 && (leff == 0 || M >= (uint32_t)leff)) return -1;  // the floor held: slice 0 finishes
  beff_out = p.B > 0 ? beff : 0;
  if (t == 0) {
    p.sl_count[item] = leff;
    if (p.B > 0) p.fin_count[item] = beff;
  }
  if (leff == 0) return 0;
  if (M >= (uint32_t)leff) {
    // the per-wave lists of scan workgroups that wrote a compact list hold
    // only candidates past their wave's first KL_CAP (none: a compact list
    // has at most WG_CAP < KL_CAP entries): copy the compact list back, one
    // finish wave per scan workgroup
    static_assert(WG_CAP < KL_CAP && NW == 4, "a compact list covers whole waves of four");
    const int wid = t / WAVE;
    for (int g = wid; g < a.W; g += SNW) {
      const int64_t gg = (int64_t)item * a.W + g;
      const uint32_t tot = a.wg_count[2 * gg];
      if (tot > (uint32_t)WG_CAP) continue;  // uniform: its per-wave lists are whole
      const uint32_t p1 = ncand[g * NW], p2 = p1 + ncand[g * NW + 1], p3 = p2 + ncand[g * NW + 2];
      for (uint32_t sidx = (uint32_t)lane; sidx < tot; sidx += WAVE) {
        const int v = (sidx >= p1) + (sidx >= p2) + (sidx >= p3);
        const uint32_t o = v == 0 ? 0u : v == 1 ? p1 : v == 2 ? p2 : p3;
        const int64_t dst = (gg * NW + v) * WAVE_KEYS + (sidx - o);
        a.cand[dst] = a.wg_cand[gg * WG_CAP + sidx];
        a.cand_rank[dst] = a.wg_rank[gg * WG_CAP + sidx];
      }
    }
    __threadfence();
    __syncthreads();
  }
  // bounds of every candidate composite: sums in [floor, upper bound of any sum]
  const uint64_t c_lo = (uint64_t)f2key(item_floor(p, item) * kInvSqrtR) << 32;
  const uint64_t c_hi = ((uint64_t)f2key(p.range[4 * item + 1] * kInvSqrtR) << 32) | 0xFFFFFFFFull;
  if (M >= (uint32_t)leff && M <= (uint32_t)(NPD * SB) && nsub <= DL_LISTS && longest <= 48u) {
    if (longest <= 32u) {
      uint64_t e_sp[2 * DK];
      gather_lists<2>(cand, nsub, e_sp);
      finish_dense<2>(a, item, nsub, leff, beff, M, c_lo, c_hi, e_sp, lds, lcnt, loff, rkb, wcnt, scratch, tl);
    } else {
      uint64_t e3[3 * DK];
      gather_lists<3>(cand, nsub, e3);
      finish_dense<3>(a, item, nsub, leff, beff, M, c_lo, c_hi, e3, lds, lcnt, loff, rkb, wcnt, scratch, tl);
    }
    return 0;
  }
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;  // rank keys this thread emitted
  auto emit = [&](uint32_t o, uint64_t x, float rank) {
    const uint32_t key = composite_index(x);
    const uint32_t rkey = f2key(rank);
    out_idx[o] = (int32_t)key;
    out_rank[o] = rank;
    rk[o] = composite(rkey, key);
    kmin = min(kmin, rkey);
    kmax = max(kmax, rkey);
  };
  bool dense = true;  // rank composites in rk (else sl + ranks in LDS)
  if (M >= (uint32_t)leff && M <= (uint32_t)LDS_CAND && nsub <= STAGE_LISTS) {
    // staged: lists into LDS in list order
    if (nsub <= SB) {
      loff[t] = block_excl_scan<SB>(m, scratch, nullptr);
      __syncthreads();  // lcnt / loff
      constexpr int KQ = SB / DQ;
      const int kq = (nsub + DQ - 1) / DQ;
      const int q = t >> 4, l = t & 15;
      for (int k = 0; k < KQ; ++k) {
        if (k >= kq) break;  // uniform
        const int sidx = k * DQ + q;
        const uint32_t c = sidx < nsub ? lcnt[sidx] : 0u;
        const uint32_t base = sidx < nsub ? loff[sidx] : 0u;
        const int64_t off = (int64_t)sidx * WAVE_KEYS;
        for (uint32_t j = l; j < c; j += 16) cl[base + j] = cand[off + j];
      }
    } else {
      uint32_t carry = 0;
      for (int g = 0; g < nsub; g += SB) {
        const int sidx = g + t;
        const uint32_t c = sidx < nsub ? ncand[sidx] : 0u;
        uint32_t tot;
        const uint32_t base = carry + block_excl_scan<SB>(c, scratch, &tot);
        if (sidx < nsub) loff[sidx] = base;
        const int64_t off = (int64_t)sidx * WAVE_KEYS;
        for (uint32_t j = 0; j < c; ++j) cl[base + j] = cand[off + j];
        carry += tot;
      }
    }
    __syncthreads();
    constexpr int NPT = LDS_CAND / SB;
    const int slots = ((int)M + SB - 1) / SB;
    uint64_t e[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int j = t + i * SB;
      e[i] = j < (int)M ? cl[j] : 0ull;
    }
    __syncthreads();  // staging area free
    const uint64_t X = (uint32_t)leff == M ? 1ull : select_top_regs<SB, NPT>(e, leff, c_hi, c_lo, tl, slots, true);
    // ranks of the selected: staging position -> list (last offset <= it)
    float rnk[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      rnk[i] = 0.0f;
      if (i < slots && e[i] != 0ull && e[i] >= X) {
        const uint32_t j = (uint32_t)(t + i * SB);
        int lo = 0, hi = nsub;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (loff[mid] <= j) lo = mid + 1;
          else hi = mid;
        }
        const int sidx = lo - 1;
        rnk[i] = crank[(int64_t)sidx * WAVE_KEYS + (j - loff[sidx])];
      }
    }
    compact_ordered<SB, NPT>(e, X, leff, wcnt, scratch, slots,
                             [&](uint32_t o, uint64_t x, int i) { emit(o, x, rnk[i]); });
  } else if (M >= (uint32_t)leff) {
    // lists: select straight from the per-wave lists in global memory
    dense = false;
    float* rkf = (float*)rk;
    uint32_t(*whist)[256] = (uint32_t(*)[256])hist;
    auto visit = [&](auto&& f) {
      for (int sidx = t; sidx < nsub; sidx += SB) {
        const uint32_t c = ncand[sidx];
        const uint64_t* src = cand + (int64_t)sidx * WAVE_KEYS;
        for (uint32_t j = 0; j < c; ++j) f(src[j]);
      }
    };
    const uint64_t X = (uint32_t)leff == M ? 1ull : select_largest<SB>(visit, leff, whist, scratch, shared64, shared);
    if (t == 0) shared[3] = 0u;
    __syncthreads();
    for (int g = 0; g < nsub; g += SB) {
      const int sidx = g + t;
      const uint32_t c = sidx < nsub ? ncand[sidx] : 0u;
      const int64_t off = (int64_t)sidx * WAVE_KEYS;
      uint32_t cnt = 0;
      for (uint32_t j = 0; j < c; ++j) cnt += cand[off + j] >= X;
      uint32_t tot;
      uint32_t o = shared[3] + block_excl_scan<SB>(cnt, scratch, &tot);
      for (uint32_t j = 0; j < c; ++j) {
        const uint64_t x = cand[off + j];
        if (x >= X && o < (uint32_t)leff) {
          sl[o] = composite_index(x);
          rkf[o] = crank[off + j];
          ++o;
        }
      }
      __syncthreads();
      if (t == 0) shared[3] += tot;
      __syncthreads();
    }
  } else {
    // all keys: the sampled floor overshot; this workgroup selects slice `slice`
    dense = false;
    if (t == 0 && slice == 0 && a.overshoot != nullptr) a.overshoot[item] = 1;
    const int N = (int)p.N, K = a.K;
    // the item's table in LDS: the slice select scores every key of the slice from it
    float* lut_l = (float*)(lds + kFinLut);
    const float* lut_g = p.lut + (int64_t)item * p.S * p.C;
    for (int e = t; e < p.S * p.C; e += SB) lut_l[e] = lut_g[e];
    __syncthreads();
    const int per = slice_keys(N, K);
    const int n0 = min(N, slice * per), n1 = min(N, n0 + per);
    uint64_t* out = a.slice_list + ((int64_t)item * K + slice) * p.L;
    uint32_t nj;
    switch (p.S) {
      case 1: nj = slice_select<1>(p, item, (uint32_t)leff, n0, n1, lut_l, lds, scratch, shared, shared64, out); break;
      case 2: nj = slice_select<2>(p, item, (uint32_t)leff, n0, n1, lut_l, lds, scratch, shared, shared64, out); break;
      case 4: nj = slice_select<4>(p, item, (uint32_t)leff, n0, n1, lut_l, lds, scratch, shared, shared64, out); break;
      default: nj = slice_select<8>(p, item, (uint32_t)leff, n0, n1, lut_l, lds, scratch, shared, shared64, out); break;
    }
    // publish the slice (release), then count it in; the item's last slice finishes the item
    if (t == 0) a.slice_n[(int64_t)item * K + slice] = nj;
    __threadfence();
    __syncthreads();
    if (t == 0) {
      const uint32_t done = atomicAdd(&a.arrive[item], 1u);
      __threadfence();
      shared[0] = done == (uint32_t)(K - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (shared[0] == 0u) return -1;
    __threadfence();  // acquire: the other slices' lists
    merge_slices(a, item, (uint32_t)leff, lds, sl, lcnt, scratch, shared, shared64);
    rank_rows(p, item, sl, leff, (float*)rk);
  }
  // bounds of the emitted rank keys (direct and staged paths) for the budget select
  wave_min_max_u32(kmin, kmax);
  if (lane == 0 && kmin <= kmax) {
    atomicMin(&rkb[0], kmin);
    atomicMax(&rkb[1], kmax);
  }
  __syncthreads();
  // shortlist outputs of the list and all-keys paths; budget input
  constexpr int NPB = FIN_MAX_L / SB;
  uint64_t e2[NPB];
  uint64_t vor = 0ull, vand = ~0ull;
#pragma unroll
  for (int i = 0; i < NPB; ++i) {
    const int r = t + i * SB;
    e2[i] = 0ull;
    if (r < leff) {
      if (dense) {
        e2[i] = rk[r];
      } else {
        const uint32_t key = sl[r];
        const float rank = ((const float*)rk)[r];
        out_idx[r] = (int32_t)key;
        out_rank[r] = rank;
        e2[i] = composite(f2key(rank), key);
      }
      vor |= e2[i];
      vand &= e2[i];
    }
  }
  if (p.B <= 0) return 0;
  const bool rb = dense && rkb[0] <= rkb[1];
  const uint64_t b_lo = (uint64_t)rkb[0] << 32, b_hi = ((uint64_t)rkb[1] << 32) | 0xFFFFFFFFull;
  finish_budget<NPB>(p, item, leff, beff, e2, rb ? b_hi : vor, rb ? b_lo : vand, rb, tl, wcnt, scratch);
  return 0;
}

// The verifier of a decode item (query head h = item), run by its finish
// workgroup over the budget list it has just selected.  Every wave takes 32
// (head_dim 128: 16) consecutive list entries per round and requests all their K and V rows at
// once (a K row by 8 lanes, 16-byte pieces; a V row by the wave, one
// dimension per lane), so a row costs two cache-line requests; scores are
// fp32 dot(K[n], q) * scaling (fused multiply-adds over each lane's piece,
// then the 8 lanes pairwise), and the wave keeps a running maximum m, exp-sum
// z and exp-weighted V sum (rescaled when m grows).  The waves' partials are
// merged at the end: out = sum_w e^(m_w - M) acc_w / sum_w e^(m_w - M) z_w,
// 0 for an empty list.  The list is read from LDS when the finish left it
// there, else from the budget output (visible after the caller's barrier).
constexpr int VLPR = 8;    // lanes per K row
constexpr int VEPW = 32;   // list entries per wave per round (D = 64; half that for D = 128)
constexpr size_t kVerifyKid = kFastEnd;  // LDS of the list: int32[B]
constexpr int kVerifyKidCap = (int)((kFinStage - kFastEnd) / sizeof(int32_t));

// n consecutive K / V elements of a compile-time dtype as floats (n a multiple of 4).
template <int KV, int NE>
SVA_DEV void kv_load(const void* base, int64_t e, bool vec, float (&v)[NE]) {
  if (vec && KV == F32) {
#pragma unroll
    for (int c = 0; c < NE / 4; ++c) {
      const float4 x = reinterpret_cast<const float4*>((const float*)base + e)[c];
      v[4 * c] = x.x, v[4 * c + 1] = x.y, v[4 * c + 2] = x.z, v[4 * c + 3] = x.w;
    }
  } else if (vec) {
#pragma unroll
    for (int c = 0; c < NE / 4; ++c) {
      const uint2 x = reinterpret_cast<const uint2*>((const uint16_t*)base + e)[c];
      const uint32_t w[4] = {x.x & 0xFFFFu, x.x >> 16, x.y & 0xFFFFu, x.y >> 16};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[4 * c + k] = KV == BF16 ? __uint_as_float(w[k] << 16) : __half2float(__ushort_as_half((unsigned short)w[k]));
    }
  } else {
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      if (KV == F32) {
        v[k] = ((const float*)base)[e + k];
      } else {
        const uint16_t x = ((const uint16_t*)base)[e + k];
        v[k] = KV == BF16 ? __uint_as_float((uint32_t)x << 16) : __half2float(__ushort_as_half(x));
      }
    }
  }
}

template <int KV>
SVA_DEV float kv_one(const void* base, int64_t e) {
  if (KV == F32) return ((const float*)base)[e];
  const uint16_t x = ((const uint16_t*)base)[e];
  return KV == BF16 ? __uint_as_float((uint32_t)x << 16) : __half2float(__ushort_as_half(x));
}

template <int D, int KV>
SVA_DEV void verify_item(const SummonParams& p, const FusedVerify& v, int item, unsigned char* lds, bool kid_in_lds,
                         const float* qsh, int budget) {
#pragma clang fp contract(off)
  const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
  constexpr int EPL = D / VLPR;      // K elements per lane of a row
  constexpr int RPI = WAVE / VLPR;   // K rows per load group
  constexpr int EPR = VEPW * 64 / D;  // list entries per wave per round
  constexpr int KI = EPR / RPI;      // K load groups per round
  constexpr int DL = D / WAVE;       // V dimensions per lane
  // 16-bit V rows at head_dim 64: a load serves two rows, lanes 0-31 the first and 32-63 the second,
  // two dimensions per lane (one 4-byte load on aligned rows); vv[2j] / vv[2j + 1] then hold the lane's
  // two dimensions of its row of the pair
  constexpr bool PAIRV = KV != F32 && D == 64;
  int32_t* kid = (int32_t*)(lds + kVerifyKid);
  float* part = (float*)(lds + kVerifyKid) + (kid_in_lds ? p.B : 0);  // [SNW][D + 2]: m, z, acc
  if (!kid_in_lds) {
    part = (float*)lds;
    kid = (int32_t*)(part + SNW * (D + 2));
  }
  const int cnt = min(max(budget, 0), p.B);  // the budget list's length, as the caller wrote it
  const int g = item / (p.H / v.G);
  const int64_t kvb = (int64_t)g * v.kv_hs;
  const int sub = lane & (VLPR - 1);
  float qv[EPL];
#pragma unroll
  for (int k = 0; k < EPL; ++k) qv[k] = qsh[sub * EPL + k];
  if (!kid_in_lds) {
    for (int j = t; j < cnt; j += SB) kid[j] = p.fin_idx[(int64_t)item * p.B + j];
    __syncthreads();
  }
  float m = -INFINITY, z = 0.0f, acc[DL], acc2[2] = {0.0f, 0.0f};
#pragma unroll
  for (int d = 0; d < DL; ++d) acc[d] = 0.0f;
  for (int r0 = wid * EPR; r0 < cnt; r0 += SNW * EPR) {  // uniform per wave
    // every K and V row of the round requested before any is used
    float kk[KI][EPL], vv[EPR][DL];
#pragma unroll
    for (int k = 0; k < KI; ++k) {
      const int e = r0 + k * RPI + lane / VLPR;
      const int64_t row = kvb + (int64_t)kid[min(e, cnt - 1)] * v.kv_rs + sub * EPL;
      kv_load<KV, EPL>(v.keys, row, v.kv_vec, kk[k]);
    }
    if constexpr (PAIRV) {
      // row r0 + 2 j + (lane >= 32), dimensions 2 (lane & 31) and 2 (lane & 31) + 1
#pragma unroll
      for (int j = 0; j < EPR / 2; ++j) {
        const int64_t row = kvb + (int64_t)kid[min(r0 + 2 * j + (lane >> 5), cnt - 1)] * v.kv_rs + 2 * (lane & 31);
        const uint16_t* src = (const uint16_t*)v.values + row;
        const uint32_t x = v.kv_vec ? *reinterpret_cast<const uint32_t*>(src)
                                    : (uint32_t)src[0] | ((uint32_t)src[1] << 16);
        vv[2 * j][0] = KV == BF16 ? __uint_as_float(x << 16) : __half2float(__ushort_as_half((unsigned short)(x & 0xFFFFu)));
        vv[2 * j + 1][0] = KV == BF16 ? __uint_as_float(x & 0xFFFF0000u) : __half2float(__ushort_as_half((unsigned short)(x >> 16)));
      }
    } else {
#pragma unroll
      for (int j = 0; j < EPR; ++j) {
        const int64_t row = kvb + (int64_t)kid[min(r0 + j, cnt - 1)] * v.kv_rs + lane;
#pragma unroll
        for (int d = 0; d < DL; ++d) vv[j][d] = kv_one<KV>(v.values, row + WAVE * d);
      }
    }
    float sc[KI], mr = -INFINITY;
#pragma unroll
    for (int k = 0; k < KI; ++k) {
      float dot = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; ++i) dot = __builtin_fmaf(kk[k][i], qv[i], dot);
      static_assert(VLPR == 8, "a K row over the 8 lanes of a half-row");
      dot = octet_sum(dot);
      const int e = r0 + k * RPI + lane / VLPR;
      sc[k] = e < cnt ? dot * v.scaling : -INFINITY;
      mr = fmaxf(mr, sc[k]);
    }
    mr = wave_max(mr);
    const float mn = fmaxf(m, mr);
    const float f = m == -INFINITY ? 0.0f : expf(m - mn);
    float pr[KI], zr = 0.0f;
#pragma unroll
    for (int k = 0; k < KI; ++k) {
      pr[k] = sc[k] == -INFINITY ? 0.0f : expf(sc[k] - mn);
      zr = zr + (sub == 0 ? pr[k] : 0.0f);
    }
    zr = wave_sum(zr);
    z = z * f + zr;
#pragma unroll
    for (int d = 0; d < DL; ++d) acc[d] = acc[d] * f;
    acc2[0] = acc2[0] * f;
    acc2[1] = acc2[1] * f;
    if constexpr (PAIRV) {
      // weight of entry r0 + 2 j + (lane >= 32): a readlane per row, the half's own
#pragma unroll
      for (int j = 0; j < EPR / 2; ++j) {
        const int e0 = 2 * j, e1 = 2 * j + 1;
        const float x0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr[e0 / RPI]), (e0 % RPI) * VLPR));
        const float x1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr[e1 / RPI]), (e1 % RPI) * VLPR));
        const float x = lane < 32 ? x0 : x1;
        acc2[0] = acc2[0] + x * vv[2 * j][0];
        acc2[1] = acc2[1] + x * vv[2 * j + 1][0];
      }
    } else {
#pragma unroll
      for (int j = 0; j < EPR; ++j) {
        // weight of entry r0 + j (0 past the list), from the lane that holds it
        const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr[j / RPI]), (j % RPI) * VLPR));
#pragma unroll
        for (int d = 0; d < DL; ++d) acc[d] = acc[d] + x * vv[j][d];
      }
    }
    m = mn;
  }
  float* mine = part + wid * (D + 2);
  if (lane == 0) {
    mine[0] = m;
    mine[1] = z;
  }
  if constexpr (PAIRV) {
    // the two halves hold the same dimensions for different rows: add them
    const float s0 = acc2[0] + __shfl_xor(acc2[0], 32, WAVE);
    const float s1 = acc2[1] + __shfl_xor(acc2[1], 32, WAVE);
    if (lane < 32) {
      mine[2 + 2 * lane] = s0;
      mine[2 + 2 * lane + 1] = s1;
    }
  } else {
#pragma unroll
    for (int d = 0; d < DL; ++d) mine[2 + lane + WAVE * d] = acc[d];
  }
  __syncthreads();
  // the merge, by the waves that hold output dimensions (whole waves): each
  // computes the wave factors e^(m_w - M) and the total exp-sum itself and
  // takes factor w from lane w, so no second barrier publishes them
  static_assert(D % WAVE == 0, "output dimensions fill whole waves");
  if (t < D) {
    const float mw = lane < SNW ? part[lane * (D + 2)] : -INFINITY;
    const float M = wave_max(mw);
    const float f = mw == -INFINITY ? 0.0f : expf(mw - M);
    const float Z = wave_sum(lane < SNW ? f * part[lane * (D + 2) + 1] : 0.0f);
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < SNW; ++w)
      o = o + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), w)) * part[w * (D + 2) + 2 + t];
    store_elem(v.out, (int64_t)item * v.o_hs + t, v.out_dtype, (cnt > 0 && Z > 0.0f) ? o / Z : 0.0f);
  }
}

// LDS the fused verifier needs when the list comes from the budget output.
inline size_t verify_item_lds(int B, int D) { return sizeof(float) * ((size_t)B + SNW * (size_t)(D + 2)); }

// The (item, slice) workgroup b of the finish grid takes.  Workgroups go to
// the 8 XCDs in turn (b to XCD b % 8), and each XCD has its own L2: with the
// fused verifier (item = query head) the finishes of one KV group's heads
// take workgroups on one XCD (group x: b = x + 8 r, member r), so K / V rows
// that their budgets share come from HBM once and from that L2 for the
// group's other heads.  The other workgroups take the slices > 0 in turn;
// without a verifier, or when the groups do not fit, b takes item b % items
// as slice b / items.
SVA_DEV void finish_slot(const WideArgs& a, int b, int& item, int& slice) {
  const int items = a.items;
  const int G = a.fv.out != nullptr ? a.fv.G : 0;
  const int per = G > 0 ? items / G : 0;  // heads per KV group
  if (G > 0 && G <= 8 && G * per == items && G - 1 + 8 * (per - 1) < items * a.K) {
    const int x = b % 8, r = b / 8;
    if (x < G && r < per) {
      item = x * per + r;
      slice = 0;
      return;
    }
    int before = 0;  // group workgroups with a smaller index
    for (int rr = 0; rr < per; ++rr) before += min(max(b - 8 * rr, 0), G);
    const int o = b - before;
    item = o % items;
    slice = 1 + o / items;
    return;
  }
  item = b % items;
  slice = b / items;
}

// Finish of an item, then (VD > 0: head_dim VD, K / V dtype VKV) its
// verifier.  Workgroup b takes the item and slice finish_slot gives it;
// slice 0 is the item's finish, slices > 0 serve the all-keys select.
template <int VD, int VKV>
__global__ void __launch_bounds__(SB) wide_finish_kernel(WideArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float qsh[VD > 0 ? VD : 1];  // the verifier's query row
  int item, slice;
  finish_slot(a, (int)blockIdx.x, item, slice);
  // the query row is requested before the finish starts and parked in LDS
  // after it (a store now would wait for the load ahead of the finish's own)
  uint32_t qbits = 0u;
  if (VD > 0 && (int)threadIdx.x < VD) qbits = load_elem_bits(a.fv.q, (int64_t)item * a.fv.q_hs + threadIdx.x, a.fv.q_dtype);
  if (slice == 0 && threadIdx.x == 0 && a.overshoot != nullptr) a.overshoot[item] = 0;  // the all-keys select sets 1
  const bool keep = VD > 0 && a.p.B <= kVerifyKidCap - SNW * (VD + 2) - SNW - 1;
  int beff = 0;
  const int done = finish_item(a, item, slice, lds, keep ? (int32_t*)(lds + kVerifyKid) : nullptr, beff);
  if (done < 0) return;  // block-uniform
  if (VD > 0) {
    if ((int)threadIdx.x < VD) qsh[threadIdx.x] = elem_from_bits(qbits, a.fv.q_dtype);
    __syncthreads();  // the query row, the budget list (LDS or global) and the LDS the finish used
    verify_item<(VD > 0 ? VD : 64), VKV>(a.p, a.fv, item, lds, done == 1, qsh, beff);
  }
}

// ---------------------------------------------------------------------------
// Code classes: one subspace of at most 256 codewords (1x256 codes).  A key's
// scan score is T[code] / sqrt(R), so the keys fall into at most 256 score
// classes and the top L keys (score descending, then lower key index) are
// whole classes plus the lowest-index keys of one boundary class.  Four
// launches replace the scan and the finish:
//   class_count   per (item, chunk of CLASS_CHUNK keys): the histogram of
//                 the chunk's allowed keys' codes;
//   class_select  per item: class totals, the boundary class (score key kb,
//                 `need` of its keys kept, shortlist length leff), and per
//                 chunk its shortlist offset and the boundary keys in earlier
//                 chunks;
//   class_extract per (item, chunk): the chunk's kept keys in key order into
//                 the shortlist, with their rank scores (computed as the scan
//                 computes them);
//   class_budget  per item: the budget select over the shortlist's rank
//                 composites, the budget list in key order and (fused) the
//                 verifier.
// The results equal the scan path's: the same scores, ranks and tie rule.
constexpr int CK_PT = 64;                 // keys per thread of a class chunk
constexpr int CLASS_CHUNK = WB * CK_PT;   // 16384
constexpr int CLASS_MAX_W = 4096;         // chunks per item: caches of up to 64M keys
static_assert(FAST_M == CLASS_MAX_L, "the class path's shortlist fits the fast finish's dense slots");

struct ClassArgs {
  SummonParams p;
  FusedVerify fv;
  int W;             // chunks per item
  uint32_t* counts;  // [items, W, 256] code histogram of each chunk's allowed keys
  uint32_t* bound;   // [items, 4]: boundary score key, its keys kept, shortlist length, 0
  uint32_t* woff;    // [items, W, 2]: shortlist offset of each chunk's keys, boundary keys in earlier chunks
  int32_t* overshoot;  // [items] or nullptr: always 0 here (no sampled floor)
};

// Codes of thread t's keys cs + 64 t .. + 63 (a partial chunk reads bytes under a guard).
SVA_DEV void class_load(const uint8_t* __restrict__ codes, int k0, int ce, u32x4 (&raw)[4]) {
  if (k0 + CK_PT <= ce) {
#pragma unroll
    for (int r = 0; r < 4; ++r) raw[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + k0 + 16 * r));
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t wv[4] = {0u, 0u, 0u, 0u};
      for (int j = 0; j < 16; ++j)
        if (k0 + 16 * r + j < ce) wv[j >> 2] |= (uint32_t)codes[k0 + 16 * r + j] << (8 * (j & 3));
      raw[r] = u32x4{wv[0], wv[1], wv[2], wv[3]};
    }
  }
}

// Score key of code c of an item: f2key(T[min(c, C - 1)] / sqrt(R)) (R = 64: exactly * 1/8), the key the
// scan gives a key with this code.
SVA_DEV uint32_t class_key(const SummonParams& p, int item, int c) {
  return f2key(p.lut[(int64_t)item * p.C + min(c, p.C - 1)] * kInvSqrtR);
}

template <bool MASKED>
SVA_DEV void class_count_chunk(const ClassArgs& a, int block) {
  __shared__ uint32_t hist[NW][256];
  const SummonParams& p = a.p;
  const int item = block / a.W, w = block % a.W;
  const int t = threadIdx.x, wid = t / WAVE;
  const int cs = w * CLASS_CHUNK, ce = (int)min((int64_t)cs + CLASS_CHUNK, p.N);
  const int k0 = cs + t * CK_PT;
  const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)(item % p.H) * p.code_hs;
  u32x4 raw[4];
  class_load(codes, k0, ce, raw);
#pragma unroll
  for (int i = 0; i < NW; ++i) hist[i][t] = 0u;
  __syncthreads();
  if (!MASKED && k0 + CK_PT <= ce) {  // every key of the thread counts: no test per key
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int j = 0; j < 16; ++j) atomicAdd(&hist[wid][byte_of(raw[r], j)], 1u);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int n = k0 + 16 * r + j;
        bool ok = n < ce;
        if (MASKED && ok) ok = mask_allows(p.mask, n, p.mask_type);
        if (ok) atomicAdd(&hist[wid][byte_of(raw[r], j)], 1u);
      }
    }
  }
  __syncthreads();
  a.counts[((int64_t)item * a.W + w) * 256 + t] = hist[0][t] + hist[1][t] + hist[2][t] + hist[3][t];
}

template <bool MASKED>
__global__ void __launch_bounds__(WB) class_count_kernel(ClassArgs a) {
  class_count_chunk<MASKED>(a, (int)blockIdx.x);
}

constexpr int CSEL_PER = CLASS_MAX_W / SB;  // chunks per thread of class_select (prefix sums)
constexpr int CSEL_G = SB / 256;              // thread groups over the chunks (code totals)

template <bool MASKED>
__global__ void __launch_bounds__(WB) class_extract_kernel(ClassArgs a) {
#pragma clang fp contract(off)
  __shared__ uint32_t flag[256], scratch[NW + 1];
  __shared__ int32_t kept_keys[CLASS_MAX_L];
  const SummonParams& p = a.p;
  const int item = blockIdx.x / a.W, w = blockIdx.x % a.W;
  const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
  const int cs = w * CLASS_CHUNK, ce = (int)min((int64_t)cs + CLASS_CHUNK, p.N);
  const int k0 = cs + t * CK_PT;
  const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)(item % p.H) * p.code_hs;
  u32x4 raw[4];
  class_load(codes, k0, ce, raw);
  const uint32_t kc = class_key(p, item, t);
  const uint32_t kb = a.bound[4 * item], need = a.bound[4 * item + 1], leff = a.bound[4 * item + 2];
  // code t's class against the boundary class: bit 0 above it, bit 16 in it
  flag[t] = (kc > kb ? 1u : 0u) | (kc == kb ? 0x10000u : 0u);
  const uint32_t* wo = a.woff + ((int64_t)item * a.W + w) * 2;
  const uint32_t off = wo[0], bpre = wo[1];
  const float4 qq = reinterpret_cast<const float4*>(p.q_low + (int64_t)item * p.R)[lane & 15];
  __syncthreads();
  // this thread's keys above the boundary class and in it (bit i: key k0 + i):
  // each 16-byte word of codes gathers its keys' flags shifted into one word
  // (above in the low half, in it in the high half), one shift-or per key
  uint64_t am = 0ull, bm = 0ull;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    uint32_t fw = 0u;
#pragma unroll
    for (int j = 0; j < 16; ++j) fw |= flag[byte_of(raw[r], j)] << j;
    am |= (uint64_t)(fw & 0xFFFFu) << (16 * r);
    bm |= (uint64_t)(fw >> 16) << (16 * r);
  }
  // keys past the cache's end or masked out are in neither set
  uint64_t okm = k0 + CK_PT <= ce ? ~0ull : (k0 >= ce ? 0ull : (1ull << (ce - k0)) - 1ull);
  if (MASKED) {
#pragma unroll
    for (int i = 0; i < CK_PT; ++i)
      if (k0 + i < ce && !mask_allows(p.mask, k0 + i, p.mask_type)) okm &= ~(1ull << i);
  }
  am &= okm;
  bm &= okm;
  // boundary keys are kept in key order up to `need` over the whole item
  const uint32_t nb = (uint32_t)__popcll(bm);
  const uint32_t before = bpre + block_excl_scan<WB>(nb, scratch, nullptr);
  uint32_t take = need > before ? min(need - before, nb) : 0u;
  uint64_t keep = am;
  for (uint64_t m = bm; take > 0u; --take) {
    const uint64_t low = m & (~m + 1ull);
    keep |= low;
    m ^= low;
  }
  uint32_t total;
  uint32_t o = block_excl_scan<WB>((uint32_t)__popcll(keep), scratch, &total);
  int32_t* sl = p.sl_idx + (int64_t)item * p.L;
  while (keep != 0ull) {
    const int i = __ffsll((long long)keep) - 1;
    keep &= keep - 1ull;
    if (off + o < leff) sl[off + o] = k0 + i;
    if (o < (uint32_t)CLASS_MAX_L) kept_keys[o] = k0 + i;
    ++o;
  }
  __syncthreads();
  // rank scores as the scan computes them: one 16-lane DPP row per key, 16 keys per wave in flight
  total = min(total, (uint32_t)CLASS_MAX_L);
  const int j = lane & 15, row = lane >> 4;
  const float* klow = p.k_low + (int64_t)(item % p.H) * p.klow_hs;
  float* rank_out = p.sl_rank + (int64_t)item * p.L + off;
  constexpr int RU = 4;
  for (uint32_t c0 = (uint32_t)wid * 4 * RU; c0 < total; c0 += NW * 4 * RU) {
    float4 rv[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const uint32_t c = c0 + 4 * u + row;
      const int n = c < total ? kept_keys[c] : 0;
      rv[u] = c < total ? reinterpret_cast<const float4*>(klow + (int64_t)n * p.R)[j] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const float dot = rank_dot64_row16(rv[u], qq);
      const uint32_t c = c0 + 4 * u + row;
      if (c < total && off + c < leff && j == 0) rank_out[c] = dot * kInvSqrtR;
    }
  }
}

// Budget of a class-path item over its shortlist (key order, leff entries),
// then (VD > 0) the verifier, in the finish kernel's LDS layout.
template <int VD, int VKV>
__global__ void __launch_bounds__(SB) class_budget_kernel(ClassArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float qsh[VD > 0 ? VD : 1];
  const SummonParams& p = a.p;
  const int item = blockIdx.x, t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
  // the verifier's query row: requested now, parked in LDS before the verifier
  const uint32_t qbits = VD > 0 && t < VD ? load_elem_bits(a.fv.q, (int64_t)item * a.fv.q_hs + t, a.fv.q_dtype) : 0u;
  const int leff = (int)a.bound[4 * item + 2];
  const int beff = min(p.B, leff);
  if (t == 0) p.fin_count[item] = beff;
  uint32_t* hist = (uint32_t*)(lds + kFastHist);
  uint64_t* small = (uint64_t*)(lds + kFastSmall);
  const FastMisc f{(uint32_t*)(lds + kFastMisc)};
  uint32_t* wcnt = (uint32_t*)(lds + kFinWcnt);
  uint32_t* scratch = (uint32_t*)(lds + kFinScratch);
  const bool keep_kid = p.B <= kVerifyKidCap - SNW * (VD + 2) - SNW - 1;
  int32_t* kidl = (int32_t*)(lds + kVerifyKid);
  reinterpret_cast<uint4*>(hist)[t] = uint4{0u, 0u, 0u, 0u};
  const int dslots = (leff + SB - 1) / SB;
  const int32_t* sl = p.sl_idx + (int64_t)item * p.L;
  const float* sr = p.sl_rank + (int64_t)item * p.L;
  uint64_t rc[NPD];
  float rv[NPD];
  uint32_t rmin = 0xFFFFFFFFu, rmax = 0u;
  // every slot is requested before any is used, unconditionally (indices
  // clamped to the buffer's L slots, which needs no load): the list's length
  // arrives with them instead of ahead of them, and no load waits on another
  // slot's use (a conditional load would end in a register merge that waits)
  int32_t kraw[NPD];
  float rraw[NPD];
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    const int jj = min(t + i * SB, p.L - 1);
    kraw[i] = sl[jj];
    rraw[i] = sr[jj];
  }
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    const int jj = t + i * SB;
    const bool in = i < dslots && jj < leff;
    rv[i] = in ? rraw[i] : 0.0f;
    const uint32_t k = f2key(rv[i]);
    rc[i] = in ? composite(k, (uint32_t)kraw[i]) : 0ull;
    if (in) {
      rmin = min(rmin, k);
      rmax = max(rmax, k);
    }
  }
  wave_min_max_u32(rmin, rmax);
  if (lane == 0) {
    f.wave(1, wid) = rmin;
    f.wave(2, wid) = rmax;
  }
  __syncthreads();
  uint32_t lo = 0xFFFFFFFFu, hi = 0u;
  for (int v = 0; v < SNW; ++v) {
    lo = min(lo, f.wave(1, v));
    hi = max(hi, f.wave(2, v));
  }
  uint64_t XB = 1ull;
  if (beff < leff) {
    bool ex = true;
    const float rlo = key2f(lo);
    XB = fast_select(rc, rv, dslots, beff, rlo, lin_scale(rlo, key2f(hi)), hist, small, f, &ex);
    if (!ex) {
      // a tie class too large to rank directly: the general register select
      __syncthreads();
      const TopLds tl{(uint32_t*)(lds + kFinHist), (uint64_t*)(lds + kFinSmall), scratch, (uint32_t*)(lds + kFinShared),
                      (uint64_t*)(lds + kFinShared64)};
      XB = select_top_regs<SB, NPD>(rc, beff, ((uint64_t)hi << 32) | 0xFFFFFFFFull, (uint64_t)lo << 32, tl, dslots,
                                    true);
    }
  }
  // the budget list in shortlist (key) order
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    if (i < dslots) {  // uniform
      const uint64_t mb = __builtin_amdgcn_ballot_w64(rc[i] != 0ull && rc[i] >= XB);
      if (lane == 0) wcnt[i * SNW + wid] = (uint32_t)__popcll(mb);
    }
  }
  __syncthreads();
  slot_wave_offsets(wcnt, dslots * SNW);
  __syncthreads();
  int32_t* fin = p.fin_idx + (int64_t)item * p.B;
#pragma unroll
  for (int i = 0; i < NPD; ++i) {
    if (i < dslots) {  // uniform
      const bool sb = rc[i] != 0ull && rc[i] >= XB;
      const uint64_t mb = __builtin_amdgcn_ballot_w64(sb);
      if (sb) {
        const uint32_t o = wcnt[i * SNW + wid] + lanes_below(mb);
        if (o < (uint32_t)beff) {
          fin[o] = (int32_t)composite_index(rc[i]);
          if (keep_kid) kidl[o] = (int32_t)composite_index(rc[i]);
        }
      }
    }
  }
  if (VD > 0) {
    if (t < VD) qsh[t] = elem_from_bits(qbits, a.fv.q_dtype);
    __syncthreads();
    verify_item<(VD > 0 ? VD : 64), VKV>(p, a.fv, item, lds, keep_kid, qsh, beff);
  }
}

// Workspace: per-wave counters, per-workgroup counters, the workgroups'
// compact lists, then the per-wave candidate lists.  Every word a call reads
// was written earlier in the same call, so no state is carried between calls
// and calls of any shape can share one buffer.
inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
// the all-keys select's arrival counters, slice counts and slice lists
inline size_t over_bytes(int64_t items, int64_t L) {
  const int64_t K = over_slices(items);
  return align256((size_t)items * sizeof(uint32_t)) + align256((size_t)(items * K) * sizeof(uint32_t)) +
         align256((size_t)(items * K * L) * sizeof(uint64_t));
}
inline size_t counters_bytes(int64_t items, int64_t W) {
  return align256((size_t)(2 * items * W * NW) * sizeof(uint32_t)) + align256((size_t)(2 * items * W) * sizeof(uint32_t)) +
         align256((size_t)(items * W * WG_CAP) * (sizeof(uint64_t) + sizeof(float)));
}


template <int VD, int VKV>
int launch_finish(const WideArgs& a, int64_t items, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((wide_finish_kernel<VD, VKV>), kFinLds, "hipFuncSetAttribute(wide_finish_kernel)");
  hipLaunchKernelGGL((wide_finish_kernel<VD, VKV>), dim3((unsigned)(items * a.K)), dim3(SB), kFinLds, stream, a);
  SVA_CHECK_LAUNCH("wide_finish_kernel");
  return SVA_OK;
}

template <int VD, int VKV>
int launch_class_budget(const ClassArgs& a, int64_t items, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((class_budget_kernel<VD, VKV>), kFinLds, "hipFuncSetAttribute(class_budget_kernel)");
  hipLaunchKernelGGL((class_budget_kernel<VD, VKV>), dim3((unsigned)items), dim3(SB), kFinLds, stream, a);
  SVA_CHECK_LAUNCH("class_budget_kernel");
  return SVA_OK;
}

// Launchers, defined one translation unit per kernel family or verifier
// variant (head_dim, K / V dtype) so that the variants compile in parallel.
int launch_scan(const WideArgs& a, int64_t items, bool masked, hipStream_t stream);
int launch_class(const ClassArgs& a, int64_t items, bool masked, const QueryLaunch* query, hipStream_t stream);
int launch_finish_nov(const WideArgs& a, int64_t items, hipStream_t stream);
int launch_class_budget_nov(const ClassArgs& a, int64_t items, hipStream_t stream);
int launch_finish_v64_bf16(const WideArgs& a, int64_t items, hipStream_t stream);
int launch_class_budget_v64_bf16(const ClassArgs& a, int64_t items, hipStream_t stream);
int launch_finish_v64_f16(const WideArgs& a, int64_t items, hipStream_t stream);
int launch_class_budget_v64_f16(const ClassArgs& a, int64_t items, hipStream_t stream);
int launch_finish_v64_f32(const WideArgs& a, int64_t items, hipStream_t stream);
int launch_class_budget_v64_f32(const ClassArgs& a, int64_t items, hipStream_t stream);
int launch_finish_v128_bf16(const WideArgs& a, int64_t items, hipStream_t stream);
int launch_class_budget_v128_bf16(const ClassArgs& a, int64_t items, hipStream_t stream);
int launch_finish_v128_f16(const WideArgs& a, int64_t items, hipStream_t stream);
int launch_class_budget_v128_f16(const ClassArgs& a, int64_t items, hipStream_t stream);
int launch_finish_v128_f32(const WideArgs& a, int64_t items, hipStream_t stream);
int launch_class_budget_v128_f32(const ClassArgs& a, int64_t items, hipStream_t stream);

}  // namespace wide
}  // namespace sva
