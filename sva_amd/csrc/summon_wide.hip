// Long-context summon for few query items (decode, q = 1): many workgroups
// per item for the scan, one per item for the rest; two kernels, no
// grid-wide synchronisation and no atomics on shared global words.
//
//   wide_scan     one workgroup per chunk of WB * 32 keys.  Streams the
//                 chunk's packed uint8 codes (16-byte loads, all in flight
//                 before use), scores every key through the LUT in the
//                 reference's order, and appends each allowed key whose sum
//                 reaches the item's sampled floor t_lo to its wave's own
//                 candidate list as a unique 64-bit composite (score key,
//                 key index); counts go to the wave's own counter words.
//                 In the fused lookup (sva_lookup_select, 4x64 codes) each
//                 scan workgroup first computes its item's q_low, table,
//                 bounds and sampled floor itself (FusedPrologue).
//   wide_finish   one workgroup per item.  Gathers the candidates (~4x the
//                 shortlist for the sampled floor) into LDS, selects the L
//                 largest composites exactly (shortlist), scores them with
//                 k_low . q_low in torch's sum order (rank), and, when a
//                 budget is asked for, selects the B best ranks and writes
//                 them in ascending key order.  When the floor overshot
//                 (fewer than L candidates) the shortlist is selected over
//                 every key of the item instead: slower, same result.
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
constexpr int LDS_CAND = 16384;  // candidates the finish kernel stages in LDS
constexpr int STAGE_LISTS = 4096;  // lists whose staging offsets the finish kernel keeps in LDS
// The wide path has R = 64: dividing by sqrt(R) = 8 equals multiplying by
// 0.125 exactly (both are the correctly rounded value of x / 8).
constexpr float kInvSqrtR = 0.125f;
constexpr int KL_CAP = 256;      // candidate keys per scan wave kept in LDS for the rank scores
constexpr int64_t kWideMinKeys = 32768;
constexpr int64_t kMaxWideItems = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct WideArgs {
  SummonParams p;
  uint32_t* ncand;   // [items, W * NW] candidates of each scan wave
  uint32_t* nallow;  // [items, W * NW] allowed keys of each scan wave
  uint64_t* cand;    // [items, W * NW, WAVE_KEYS] candidate composites of each scan wave
  float* cand_rank;  // [items, W * NW, WAVE_KEYS] rank score of each listed candidate
  int W;             // scan workgroups per item
  FusedQuery f;      // fused lookup: the query side (p.q_low, p.lut, p.range are its outputs)
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
  float t0, t1[NP ? NP : 1], ts[NS];
  const float* tab;
  // Table values into registers: every load issued, none waited for, so
  // the caller can issue its code loads behind them.
  SVA_DEV void load(const SummonParams& p, int item) {
    const float* src = p.lut + (int64_t)item * S * p.C;
    const int t = threadIdx.x;
    const int cm = p.C - 1;
    if (NP) {
      t0 = src[min(t & 63, cm)];  // (t + k * WB) & 63 == t & 63
#pragma unroll
      for (int k = 0; k < NP; ++k) t1[k] = src[p.C + min((t + k * WB) >> 6, cm)];
    }
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
  // Writes the tables to LDS (the caller synchronizes before use).
  SVA_DEV void store(float* lds_tab) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NP; ++k) lds_tab[t + k * WB] = t0 + t1[k];
#pragma unroll
    for (int k = 0; k < NS; ++k)
      if (t + k * WB < SINGLE) lds_tab[PAIR + t + k * WB] = ts[k];
    tab = lds_tab;
  }
  SVA_DEV float at_byte(uint32_t byte_offset) const {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(tab) + byte_offset);
  }
};

// Scores the keys of one 16-byte round of the thread, branch-free so that
// the round's table lookups are in flight together: acc[k] = ((T0 + T1) +
// T2) + ... (the scan sum before the 1/8 scale; the reference's leading
// 0 + T0 only changes the sign of a zero).  On the SMALLC path a code byte
// becomes a table byte offset with a shift and a mask (codes below 64).
template <int S, bool SMALLC>
SVA_DEV void score_round(const u32x4& raw, const ScanTables<S, SMALLC>& T, float (&acc)[16 / S]) {
#pragma clang fp contract(off)
  constexpr int KPT = 16 / S;
#pragma unroll
  for (int k = 0; k < KPT; ++k) {
    float a = 0.0f;
    if (SMALLC) {
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

// Appends the flagged keys of one round (key n0 + k for flag c[k]) to the
// wave's candidate list in ascending key order (lanes in order, each lane's
// keys in order), as composites of the exact score acc / sqrt(R); the first
// KL_CAP key indices also go to the wave's LDS list `keys`.
template <int KPT>
SVA_DEV void append_round(const SummonParams& p, const bool (&c)[KPT], const float (&acc)[KPT], int n0, uint64_t* out,
                          uint32_t* keys, uint32_t& wc) {
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
      out[o] = composite(f2key(acc[k] * kInvSqrtR), (uint32_t)(n0 + k));
      if (o < (uint32_t)KL_CAP) keys[o] = (uint32_t)(n0 + k);
      ++o;
    }
  }
  wc += tot;
}

// The scan of one thread's slots.  CHECK: the chunk is partial or masked, so
// every key is tested for being allowed; otherwise every key is, and a round
// (one 16-byte word of codes) is examined key by key only when its largest
// sum reaches the floor.
template <int S, bool SMALLC, bool CHECK, bool MASKED>
SVA_DEV void scan_rounds(const SummonParams& p, const u32x4 (&raw)[KEYS_PT * S / 16], const ScanTables<S, SMALLC>& T,
                         float t_lo, int cs, int ce, uint64_t* out, uint32_t* keys, uint32_t& wc,
                         uint32_t& n_allowed) {
  constexpr int KPT = 16 / S;
#pragma unroll
  for (int r = 0; r < KEYS_PT / KPT; ++r) {
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
      if (__builtin_amdgcn_ballot_w64(any) != 0ull) append_round<KPT>(p, c, acc, round_key<S>(cs, r), out, keys, wc);
    } else {
      float mx = acc[0];
#pragma unroll
      for (int k = 1; k < KPT; ++k) mx = fmaxf(mx, acc[k]);
      if (__builtin_amdgcn_ballot_w64(mx >= t_lo) != 0ull) {  // rare: the shortlist and the keys near it
        bool c[KPT];
#pragma unroll
        for (int k = 0; k < KPT; ++k) c[k] = acc[k] >= t_lo;
        append_round<KPT>(p, c, acc, round_key<S>(cs, r), out, keys, wc);
      }
    }
  }
  if (!CHECK) n_allowed = KEYS_PT;
}

// Rank scores of a scan wave's nc candidates (keys in the LDS list while
// they fit, else from the wave's candidate list): one 16-lane DPP row per
// candidate, 16 candidates in flight per wave; written beside the list.
// qq: floats 4j .. 4j + 3 of the item's q_low for lane j of each DPP row.
SVA_DEV void rank_candidates(const SummonParams& p, int item, const float4 qq, const uint32_t* keys,
                             const uint64_t* out, float* rank, uint32_t nc) {
#pragma clang fp contract(off)
  const int j = lane_id() & 15;
  const int row = lane_id() >> 4;
  const float* klow = p.k_low + (int64_t)(item % p.H) * p.klow_hs;
  if (nc > (uint32_t)KL_CAP) __threadfence();  // keys past the LDS list are read back from `out`
  constexpr int RU = 4;
  for (uint32_t c0 = 0; c0 < nc; c0 += 4 * RU) {
    float4 rv[RU];
    uint32_t key[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const uint32_t c = c0 + 4 * u + row;
      key[u] = 0u;
      if (c < nc) key[u] = c < (uint32_t)KL_CAP ? keys[c] : composite_index(out[c]);
      rv[u] = c < nc ? reinterpret_cast<const float4*>(klow + (int64_t)key[u] * p.R)[j] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const float dot = rank_dot64_row16(rv[u], qq);
      if (c0 + 4 * u + row < nc && j == 0) rank[c0 + 4 * u + row] = dot * kInvSqrtR;
    }
  }
}

// LDS of the fused prologue beside the scan tables.
struct FusedLds {
  float qf[64];
  __align__(16) float ql[64];
  uint32_t kmin[8], kmax[8];
  uint32_t misc[4];
  uint32_t scratch[NW + 2];
};

// Query side of the fused lookup for one item, computed by every scan
// workgroup of the item (D = R = 64, 4x64 codes) with the arithmetic
// of sva_query_lut: q_low by a sequential fma chain over d times the scale,
// each table entry by a sequential fma chain over its subspace, the bounds of
// any sum folded over s, and the sampled floor from the same samples and
// histogram; tables and floors are therefore bit-identical to the two-call
// path.  issue() starts the loads (before the chunk's codes); build() leaves
// the scan tables in LDS and returns the floor.  The item's first workgroup
// writes q_low, the table and the bounds to global memory.
template <int S>
struct FusedPrologue {
  static constexpr int SUB = 64 / S;         // floats per codebook row
  static constexpr int ROWS = S * 64 / WB;   // table entries (codebook rows) per thread
  static constexpr int SPT = N_SAMPLE / WB;  // sampled keys per thread
  static constexpr int SW = S / 4;           // 32-bit words of codes per key
  static_assert(ROWS * SUB == 16 && S * 64 <= 2 * WB && SAMPLE_BINS == 4 * WB, "fused prologue layout");
  float4 w[4];   // floats 16 t .. 16 t + 15 of the head's map q_proj[h] ([D][R])
  float4 cb[4];  // codebook rows t + k * WB
  uint32_t smp[SPT][SW];
  float qv, sc;
  SVA_DEV void issue(const WideArgs& a, int item) {
    const FusedQuery& f = a.f;
    const int t = threadIdx.x;
    const int h = item % a.p.H;
    const float4* w4 = reinterpret_cast<const float4*>(f.q_proj + (int64_t)h * 64 * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = w4[4 * t + i];
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const float4* c4 = reinterpret_cast<const float4*>(f.codebooks + ((int64_t)h * S * 64 + t + k * WB) * SUB);
#pragma unroll
      for (int i = 0; i < SUB / 4; ++i) cb[k * (SUB / 4) + i] = c4[i];
    }
    qv = t < 64 ? load_elem(f.q, (int64_t)h * f.q_hs + t, f.q_dtype) : 0.0f;
    sc = f.scale[h];
    if (f.sample_k > 0) {
      const uint8_t* head = (const uint8_t*)a.p.codes + (int64_t)h * a.p.code_hs;
      const int64_t N = a.p.N;
#pragma unroll
      for (int u = 0; u < SPT; ++u) {
        const int i = t + u * WB;
        const int blk = i / SAMPLE_KEYS;
        const int64_t n0 = ((int64_t)blk * (N - SAMPLE_KEYS) / (SAMPLE_BLOCKS - 1)) & ~(int64_t)15;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(head + (n0 + i % SAMPLE_KEYS) * S);
#pragma unroll
        for (int j = 0; j < SW; ++j) smp[u][j] = src[j];
      }
    }
  }
  SVA_DEV float build(const WideArgs& a, int item, bool first, float* tab, FusedLds& L) {
#pragma clang fp contract(off)
    const FusedQuery& f = a.f;
    const int t = threadIdx.x;
    constexpr int PAIR = 4096;
    // 1. map and query into LDS (the map in the pair table's place)
#pragma unroll
    for (int i = 0; i < 4; ++i) reinterpret_cast<float4*>(tab)[4 * t + i] = w[i];
    if (t < 64) L.qf[t] = qv;
    if (t == 0) L.misc[0] = 0u;  // floor bin 0 unless the samples place it
    __syncthreads();
    // 2. q_low, one lane per output
    if (t < 64) {
      float acc = 0.0f;
#pragma unroll 16
      for (int d = 0; d < 64; ++d) acc = __builtin_fmaf(L.qf[d], tab[d * 64 + t], acc);
      const float v = acc * sc;
      L.ql[t] = v;
      if (first) const_cast<float*>(a.p.q_low)[(int64_t)item * 64 + t] = v;
    }
    __syncthreads();
    // 3. table entries (every wave's 64 entries share a subspace), per-subspace
    // bounds, histogram cleared (the map is no longer read)
    float* raw = tab + PAIR;
    uint32_t* hist = reinterpret_cast<uint32_t*>(tab);
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
      const int e = t + k * WB;
      const int s = e >> 6;
      const float* row = reinterpret_cast<const float*>(&cb[k * (SUB / 4)]);
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < SUB; ++j) acc = __builtin_fmaf(L.ql[s * SUB + j], row[j], acc);
      raw[e] = acc;
      if (first) const_cast<float*>(a.p.lut)[(int64_t)item * S * 64 + e] = acc;
      uint32_t kn = f2key(acc), kx = kn;
      for (int off = 32; off > 0; off >>= 1) {
        kn = min(kn, (uint32_t)__shfl_xor((int)kn, off, WAVE));
        kx = max(kx, (uint32_t)__shfl_xor((int)kx, off, WAVE));
      }
      if (lane_id() == 0) {
        L.kmin[s] = kn;
        L.kmax[s] = kx;
      }
    }
    reinterpret_cast<uint4*>(hist)[t] = uint4{0u, 0u, 0u, 0u};
    __syncthreads();
    // 4. bounds of any sum, in the scan's order
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      lo = lo + key2f(L.kmin[s]);
      hi = hi + key2f(L.kmax[s]);
    }
    // 5. sampled floor: the histogram bin of the k-th largest sampled sum
    float t_lo = -INFINITY;
    const int k = f.sample_k;
    if (k > 0 && hi > lo) {
      const float inv_w = (float)SAMPLE_BINS / (hi - lo);
#pragma unroll
      for (int u = 0; u < SPT; ++u) {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int c = min((int)((smp[u][s >> 2] >> (8 * (s & 3))) & 0xFFu), 63);
          acc = acc + raw[s * 64 + c];
        }
        int bin = (int)((acc - lo) * inv_w);
        bin = bin < 0 ? 0 : (bin >= SAMPLE_BINS ? SAMPLE_BINS - 1 : bin);
        atomicAdd(&hist[bin], 1u);
      }
      __syncthreads();
      // thread t holds bins SAMPLE_BINS - 1 - 4 t - j (j = 0..3), from the top
      uint32_t c[4], mine = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = hist[SAMPLE_BINS - 1 - 4 * t - j];
        mine += c[j];
      }
      uint32_t total;
      uint32_t above = block_excl_scan<WB>(mine, L.scratch, &total);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (above < (uint32_t)k && above + c[j] >= (uint32_t)k) L.misc[0] = (uint32_t)(SAMPLE_BINS - 1 - 4 * t - j);
        above += c[j];
      }
      __syncthreads();
      t_lo = lo + (float)L.misc[0] / inv_w;
    }
    if (first && t == 0) {
      float* rg = const_cast<float*>(a.p.range) + (int64_t)item * 4;
      rg[0] = lo;
      rg[1] = hi;
      rg[2] = t_lo;
      rg[3] = 0.0f;
    }
    __syncthreads();  // histogram read before the pair table replaces it
    // 6. pair table: entry t + k WB = T0[t & 63] + T1[(t >> 6) + 4 k]
    const float t0 = raw[t & 63];
#pragma unroll
    for (int kk = 0; kk < PAIR / WB; ++kk) tab[t + kk * WB] = t0 + raw[64 + (t >> 6) + kk * (WB / 64)];
    __syncthreads();
    return t_lo > lo ? t_lo : lo;
  }
};

// One scan workgroup's chunk.  CHECK: a partial or masked chunk (every key
// tested for being allowed, guarded loads).  FUSED: the query side is
// computed here (FusedPrologue) instead of read.
template <int S, bool SMALLC, bool CHECK, bool MASKED, bool FUSED>
SVA_DEV void scan_chunk(const WideArgs& a, int item, int w, float* tab_lds, uint32_t (*klist)[KL_CAP], FusedLds& fl) {
#pragma clang fp contract(off)
  const SummonParams& p = a.p;
  const int h = item % p.H;
  const int cs = w * CHUNK;
  const int ce = (int)min((int64_t)cs + CHUNK, p.N);
  const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)h * p.code_hs;
  // table loads first, then the codes: loads complete in order, so the
  // tables are stored while the codes stream and each round of codes is
  // scored as soon as its own load lands
  // The tables come first and the chunk's codes are requested only once they
  // are in LDS: all workgroups start together, and query-side loads issued
  // after the first workgroups' code loads wait behind the whole code stream
  // in the memory pipeline (measured: the fused lookup 2.6 us faster this way).
  ScanTables<S, SMALLC> T;
  u32x4 raw[KEYS_PT * S / 16];
  float t_lo;
  if constexpr (FUSED) {
    FusedPrologue<S> F;
    F.issue(a, item);
    t_lo = F.build(a, item, w == 0, tab_lds, fl);  // tables in LDS
    T.tab = tab_lds;
  } else {
    T.load(p, item);
    T.store(tab_lds);
    t_lo = item_floor(p, item);
    __syncthreads();  // tables in LDS
  }
  load_chunk<S, !CHECK>(codes, cs, ce, raw);
  const int wid = threadIdx.x / WAVE;
  const int64_t sub = ((int64_t)item * a.W + w) * NW + wid;
  uint64_t* out = a.cand + sub * WAVE_KEYS;
  uint32_t n_allowed = 0;
  uint32_t wc = 0;  // candidates of this wave so far (wave-uniform)
  scan_rounds<S, SMALLC, CHECK, MASKED>(p, raw, T, t_lo, cs, ce, out, klist[wid], wc, n_allowed);
  float4 qq;
  if constexpr (FUSED) qq = reinterpret_cast<const float4*>(fl.ql)[lane_id() & 15];
  else qq = reinterpret_cast<const float4*>(p.q_low + (int64_t)item * p.R)[lane_id() & 15];
  rank_candidates(p, item, qq, klist[wid], out, a.cand_rank + sub * WAVE_KEYS, wc);
  const uint32_t wa = wave_sum_u32(n_allowed);
  if (lane_id() == 0) {
    a.ncand[sub] = wc;
    a.nallow[sub] = wa;
  }
}

// Five workgroups per CU (at most 102 VGPRs) keep every workgroup of a
// million-key, nine-head scan resident at once (up to four subspaces).
template <int S, bool SMALLC, bool MASKED, bool FUSED>
__global__ void __launch_bounds__(WB, S <= 4 ? 5 : 1) wide_scan_kernel(WideArgs a) {
  __shared__ __align__(16) float tab_lds[ScanTables<S, SMALLC>::LDS_FLOATS];
  __shared__ uint32_t klist[NW][KL_CAP];
  __shared__ FusedLds fl;
  const int item = blockIdx.x / a.W;
  const int w = blockIdx.x % a.W;
  if (!MASKED && (int64_t)(w + 1) * CHUNK <= a.p.N) {
    scan_chunk<S, SMALLC, false, false, FUSED>(a, item, w, tab_lds, klist, fl);
  } else {
    scan_chunk<S, SMALLC, true, MASKED, FUSED>(a, item, w, tab_lds, klist, fl);
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

// Direct path of the finish: lists gathered straight into registers when
// every list holds at most DCAP candidates and there are at most DL_LISTS
// lists (16 lanes per list, entries l + 16 h of lists k * 64 + q).
constexpr int DQ = SB / 16;          // list groups of 16 lanes
constexpr int DK = 8;                // lists per group
constexpr int DCAP = 48;             // entries per list (up to 3 per lane)
constexpr int DL_LISTS = DQ * DK;    // 512 lists: caches up to 1M keys

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

// Direct path of the finish (see wide_finish_kernel): DH entries per lane
// and list, slot DH * k + h = list k * DQ + q, entry l + 16 h.
template <int DH, typename Emit>
SVA_DEV void finish_direct(const WideArgs& a, int item, int nsub, int leff, uint32_t M, uint64_t c_lo, uint64_t c_hi,
                           const uint32_t* lcnt, uint32_t* loff, const TopLds& tl, uint32_t* scratch, Emit emit) {
  const uint64_t* cand = a.cand + (int64_t)item * nsub * WAVE_KEYS;
  const float* crank = a.cand_rank + (int64_t)item * nsub * WAVE_KEYS;
  const int t = threadIdx.x;
  const int q = t >> 4, l = t & 15;
  const int kq = (nsub + DQ - 1) / DQ;
  constexpr int NS = DH * DK;
  uint64_t e[NS];
#pragma unroll
  for (int k = 0; k < DK; ++k) {
#pragma unroll
    for (int h = 0; h < DH; ++h) e[DH * k + h] = 0ull;
    if (k < kq) {  // uniform; entries < DCAP are inside every list's capacity
      const int64_t off = (int64_t)min(k * DQ + q, nsub - 1) * WAVE_KEYS;
#pragma unroll
      for (int h = 0; h < DH; ++h) e[DH * k + h] = cand[off + l + 16 * h];
    }
  }
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    const int sidx = k * DQ + q;
    const uint32_t c = (k < kq && sidx < nsub) ? lcnt[sidx] : 0u;
#pragma unroll
    for (int h = 0; h < DH; ++h)
      if ((uint32_t)(l + 16 * h) >= c) e[DH * k + h] = 0ull;
  }
  const uint64_t X = (uint32_t)leff == M ? 1ull : select_top_regs<SB, NS>(e, leff, c_hi, c_lo, tl, DH * kq, true);
  // the selected load their ranks (written beside the lists by the scan)
  float rnk[NS];
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    const int64_t off = (int64_t)min(k * DQ + q, nsub - 1) * WAVE_KEYS;
#pragma unroll
    for (int h = 0; h < DH; ++h) {
      const uint64_t x = e[DH * k + h];
      rnk[DH * k + h] = (k < kq && x != 0ull && x >= X) ? crank[off + l + 16 * h] : 0.0f;
    }
  }
  // list-ordered compaction: per-list counts of the selected (ballot
  // bits of the list's 16 lanes), their scan over the lists, then each
  // entry at its list's base plus the selected before it in the list
  uint32_t mk[NS];
  const int qs = 16 * (q & 3);
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    uint32_t cnt = 0;
#pragma unroll
    for (int h = 0; h < DH; ++h) {
      mk[DH * k + h] = 0u;
      if (k < kq) {
        const uint64_t x = e[DH * k + h];
        const uint64_t b = __builtin_amdgcn_ballot_w64(x != 0ull && x >= X);
        mk[DH * k + h] = (uint32_t)(b >> qs) & 0xFFFFu;
        cnt += (uint32_t)__popc(mk[DH * k + h]);
      }
    }
    const int sidx = k * DQ + q;
    if (k < kq && l == 0 && sidx < nsub) loff[sidx] = cnt;
  }
  __syncthreads();
  {
    const uint32_t c = t < nsub ? loff[t] : 0u;
    uint32_t tot;
    const uint32_t o = block_excl_scan<SB>(c, scratch, &tot);
    if (t < nsub) loff[t] = o;
    __syncthreads();
  }
  const uint32_t below = (1u << l) - 1u;
#pragma unroll
  for (int k = 0; k < DK; ++k) {
    if (k < kq) {
      const int sidx = k * DQ + q;
      uint32_t o = sidx < nsub ? loff[sidx] : 0u;
#pragma unroll
      for (int h = 0; h < DH; ++h) {
        const uint32_t mm = mk[DH * k + h];
        if ((mm >> l) & 1u) emit(o + (uint32_t)__popc(mm & below), e[DH * k + h], rnk[DH * k + h]);
        o += (uint32_t)__popc(mm);
      }
    }
  }
}

// Finish of an item: shortlist select, its outputs with the ranks the scan
// computed, and (B > 0) the budget select, one workgroup per item.  The
// candidate lists are in ascending key order, and so is every output.
//   direct  (every list <= DCAP entries, <= 512 lists): lists gathered into
//           registers, 16 lanes per list; the selected load their ranks;
//           list-ordered compaction by per-list ballots and a scan over the
//           lists;
//   staged  (M <= LDS_CAND, <= STAGE_LISTS lists): lists staged in LDS in
//           list order, then into registers; the selected find their list
//           (binary search over the staging offsets) for their ranks;
//           slot-ordered compaction;
//   lists   (more candidates): selection straight from the global lists;
//   all keys (the sampled floor let fewer than L keys through): selection
//           over every key of the item, ranks computed here.
// The last two are slower and give the same result.  The shortlist's rank
// composites go to LDS in shortlist order for the budget.
__global__ void __launch_bounds__(SB) wide_finish_kernel(WideArgs a) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
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
  const int item = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int nsub = a.W * NW;
  const uint32_t* ncand = a.ncand + (int64_t)item * nsub;
  const uint32_t* nallow = a.nallow + (int64_t)item * nsub;
  const uint64_t* cand = a.cand + (int64_t)item * nsub * WAVE_KEYS;
  const float* crank = a.cand_rank + (int64_t)item * nsub * WAVE_KEYS;
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  float* out_rank = p.sl_rank + (int64_t)item * p.L;
  // 1. totals: candidates M, allowed keys A, longest list; list counts
  if (t == 0) {
    shared[0] = 0u;  // M
    shared[1] = 0u;  // longest list (when nsub <= SB), if over 32
    shared[2] = 0u;  // some list longer than DCAP
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
  const uint32_t wm = wave_sum_dpp(m), wa = wave_sum_dpp(al);
  __syncthreads();
  if (lane == 0) {
    atomicAdd(&shared[0], wm);
    atomicAdd(&shared[3], wa);
  }
  if (m > (uint32_t)DCAP) atomicOr(&shared[2], 1u);
  if (m > 32u) atomicMax(&shared[1], m);
  __syncthreads();
  const uint32_t M = shared[0], A = shared[3];
  const int leff = (int)min((uint32_t)p.L, A);
  const int beff = min(p.B, leff);
  if (t == 0) {
    p.sl_count[item] = leff;
    if (p.B > 0) p.fin_count[item] = beff;
  }
  if (leff == 0) return;
  const bool long_lists = shared[2] != 0u;
  const uint32_t longest = shared[1];
  // bounds of every candidate composite: sums in [floor, upper bound of any sum]
  const uint64_t c_lo = (uint64_t)f2key(item_floor(p, item) * kInvSqrtR) << 32;
  const uint64_t c_hi = ((uint64_t)f2key(p.range[4 * item + 1] * kInvSqrtR) << 32) | 0xFFFFFFFFull;
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
  if (M >= (uint32_t)leff && nsub <= DL_LISTS && !long_lists) {
    if (longest > 32u) finish_direct<3>(a, item, nsub, leff, M, c_lo, c_hi, lcnt, loff, tl, scratch, emit);
    else finish_direct<2>(a, item, nsub, leff, M, c_lo, c_hi, lcnt, loff, tl, scratch, emit);
  } else if (M >= (uint32_t)leff && M <= (uint32_t)LDS_CAND && nsub <= STAGE_LISTS) {
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
    // all keys: the sampled floor overshot
    dense = false;
    uint32_t(*whist)[256] = (uint32_t(*)[256])hist;
    const int h = item % p.H;
    const uint8_t* codes = (const uint8_t*)p.codes + (int64_t)h * p.code_hs;
    const int N = (int)p.N;
    // the item's table in LDS: every pass below rescores every key from it
    float* lut_l = (float*)(lds + kFinLut);
    const float* lut_g = p.lut + (int64_t)item * p.S * p.C;
    for (int e = t; e < p.S * p.C; e += SB) lut_l[e] = lut_g[e];
    __syncthreads();
    const int S = p.S, C = p.C;
    auto key_at = [&](int n) -> uint64_t {
      if (!mask_allows(p.mask, n, p.mask_type)) return 0ull;
      // the reference's exact score ((0 + T0[c0]) + T1[c1]) + ... then / sqrt(R)
      float acc = 0.0f;
      for (int s2 = 0; s2 < S; ++s2) {
        uint32_t c = codes[(int64_t)n * S + s2];
        c = c < (uint32_t)C ? c : (uint32_t)(C - 1);
        acc = acc + lut_l[s2 * C + c];
      }
      return composite(f2key(acc / p.sqrt_r), (uint32_t)n);
    };
    auto visit = [&](auto&& f) {
      for (int n = t; n < N; n += SB) {
        const uint64_t x = key_at(n);
        if (x != 0ull) f(x);
      }
    };
    const uint64_t X = (uint32_t)leff == A ? 1ull : select_largest<SB>(visit, leff, whist, scratch, shared64, shared);
    const int per = (N + SB - 1) / SB;
    const int n0 = min(N, t * per), n1 = min(N, n0 + per);
    uint32_t cnt = 0;
    for (int n = n0; n < n1; ++n) cnt += key_at(n) >= X;
    uint32_t tot;
    uint32_t o = block_excl_scan<SB>(cnt, scratch, &tot);
    for (int n = n0; n < n1; ++n)
      if (key_at(n) >= X && o < (uint32_t)leff) sl[o++] = (uint32_t)n;
    __syncthreads();
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
  if (p.B <= 0) return;
  const bool rb = dense && rkb[0] <= rkb[1];
  const uint64_t b_lo = (uint64_t)rkb[0] << 32, b_hi = ((uint64_t)rkb[1] << 32) | 0xFFFFFFFFull;
  finish_budget<NPB>(p, item, leff, beff, e2, rb ? b_hi : vor, rb ? b_lo : vand, rb, tl, wcnt, scratch);
}

template <int S, bool SMALLC, bool MASKED, bool FUSED = false>
int launch_wide(const WideArgs& a, int64_t items, hipStream_t stream) {
  hipLaunchKernelGGL((wide_scan_kernel<S, SMALLC, MASKED, FUSED>), dim3((unsigned)(items * a.W)), dim3(WB), 0, stream,
                     a);
  SVA_CHECK_LAUNCH("wide_scan_kernel");
  static bool attr_set = false;
  if (!attr_set) {
    SVA_CHECK_HIP(hipFuncSetAttribute((const void*)wide_finish_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)kFinLds),
                  "hipFuncSetAttribute(wide_finish_kernel)");
    attr_set = true;
  }
  hipLaunchKernelGGL(wide_finish_kernel, dim3((unsigned)items), dim3(SB), kFinLds, stream, a);
  SVA_CHECK_LAUNCH("wide_finish_kernel");
  return SVA_OK;
}

template <int S>
int launch_wide_s(const WideArgs& a, int64_t items, bool masked, hipStream_t stream) {
  const bool small_c = a.p.C <= 64;
  if (small_c) return masked ? launch_wide<S, true, true>(a, items, stream) : launch_wide<S, true, false>(a, items, stream);
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
  if (p.L > FIN_MAX_L) return false;
  if (((uintptr_t)p.codes & 15u) != 0 || p.code_hs % 16 != 0) return false;
  if (((uintptr_t)p.k_low & 15u) != 0 || p.klow_hs % 4 != 0 || ((uintptr_t)p.q_low & 15u) != 0) return false;
  if (p.mask_type != MASK_NONE && p.mask_type != MASK_BOOL && p.mask == nullptr) return false;
  return true;
}

size_t summon_wide_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t) {
  const int64_t items = n_seq * H * Q;
  if (n_seq != 1 || Q != 1 || n_keys < kWideMinKeys || items > kMaxWideItems) return 256;
  const int64_t W = (n_keys + CHUNK - 1) / CHUNK;
  return counters_bytes(items, W) + (size_t)items * (size_t)W * CHUNK * (sizeof(uint64_t) + sizeof(float));
}

bool summon_wide_fused_eligible(const SummonParams& p, const FusedQuery& f) {
  if (!summon_wide_eligible(p, p.H) || p.offs != nullptr || p.Q != 1) return false;
  if (f.D != 64 || p.R != 64 || p.C != 64 || p.S != 4) return false;
  if (p.mask_type != MASK_NONE && p.mask_type != MASK_BOOL) return false;  // every key allowed
  if (f.q_dtype < 0 || f.q_dtype > 2 || f.q == nullptr || f.scale == nullptr) return false;
  if (((uintptr_t)f.q_proj & 15u) != 0 || ((uintptr_t)f.codebooks & 15u) != 0) return false;
  return true;
}

int summon_wide_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream,
                     const FusedQuery* f) {
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
  a.cand_rank = (float*)(ws + counters_bytes(items, a.W) + (size_t)items * (size_t)a.W * CHUNK * sizeof(uint64_t));
  if (f != nullptr) {
    a.f = *f;
    return launch_wide<4, true, false, true>(a, items, stream);
  }
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
