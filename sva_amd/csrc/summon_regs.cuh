#pragma once
// The per-item register path of the summon (shortlist, rescore and budget of
// one query item in one 1024-thread workgroup, caches of up to 16K keys),
// shared by summon_regs_kernel and the fused one-token lookup.
#include <type_traits>

#include "common.cuh"
#include "summon.h"

namespace sva {

constexpr int ITEM_BLOCK = 1024;

__host__ __device__ inline int align16(int x) { return (x + 15) & ~15; }

// ---------------------------------------------------------------------------
// Fused item path for caches of up to 16K keys with a budget (R = 64,
// L <= 2048): shortlist, rescore and budget in one workgroup per item, the
// prefill shape (thousands of items of a few thousand keys each).  Thread t
// holds keys i * BLOCK + t (i < NPT) in registers as unique composites (scan
// key, key index); a register radix select finds the L-th largest; the
// shortlist is compacted in ascending key order (per-slot wave ballots and
// one scan of the wave counts); each lane octet rescores shortlisted rows in
// torch's sum order, REG_OCT rows in flight; the budget is a second
// register select over the shortlist's (rank key, key index) composites,
// compacted in shortlist order, which is ascending key order, as the budget
// select writes it.
constexpr int REG_MAX_L = 2048;

// The k-th largest 32-bit key among the nonzero composites of the slots (the
// key is a composite's high word): T and need such that the k largest by
// (key desc, index asc) are the elements with key > T and the first need
// elements with key == T in ascending index order.  kor / kand: this
// thread's OR / AND of its elements' keys.  Radix passes of up to 12 bits
// from the highest bit where the keys differ; a tie class costs no pass (the
// caller's compaction takes its first need members), and a boundary bucket
// of at most TOP_SMALL keys is ranked directly.  Every thread of the block
// must call it.
template <int BLOCK, int NPT>
SVA_DEV void select_key_regs(const uint64_t (&e)[NPT], int slots, int k, uint32_t kor, uint32_t kand,
                             const TopLds& s, uint32_t* T_out, int* need_out) {
  static_assert(BLOCK == 4 * 256 && TOP_BINS == 4 * BLOCK, "one uint4 of bins per thread");
  static_assert(TOP_SMALL * 16 == BLOCK, "16 lanes per key of the last bucket");
  const int t = (int)threadIdx.x, lane = lane_id();
#pragma unroll
  for (int o = 1; o <= 8; o <<= 1) {
    const uint32_t ko = o == 1 ? row_shr_keep<1>(kor) : o == 2 ? row_shr_keep<2>(kor)
                      : o == 4 ? row_shr_keep<4>(kor) : row_shr_keep<8>(kor);
    const uint32_t ka = o == 1 ? row_shr_keep<1>(kand) : o == 2 ? row_shr_keep<2>(kand)
                      : o == 4 ? row_shr_keep<4>(kand) : row_shr_keep<8>(kand);
    kor |= ko;
    kand &= ka;
  }
  const auto rl = [](uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); };
  kor = rl(kor, 15) | rl(kor, 31) | rl(kor, 47) | rl(kor, 63);
  kand = rl(kand, 15) & rl(kand, 31) & rl(kand, 47) & rl(kand, 63);
  if (t == 0) {
    s.shared[0] = 0u;
    s.shared[1] = 0xFFFFFFFFu;
  }
  __syncthreads();
  if (lane == 0) {
    atomicOr(&s.shared[0], kor);
    atomicAnd(&s.shared[1], kand);
  }
  __syncthreads();
  const uint32_t all_or = s.shared[0], all_and = s.shared[1];
  __syncthreads();
  const uint32_t diff = all_or ^ all_and;
  if (diff == 0u) {  // one key: the first k in index order
    *T_out = all_or;
    *need_out = k;
    return;
  }
  int top = 31 - __clz((int)diff);
  uint32_t pmask = top == 31 ? 0u : ~0u << (top + 1);
  uint32_t prefix = all_and & pmask;
  int rem = k;
  while (true) {
    const int shift = max(top - (TOP_BITS - 1), 0);
    const uint32_t dmask = (1u << (top - shift + 1)) - 1u;
    reinterpret_cast<uint4*>(s.hist)[t] = uint4{0u, 0u, 0u, 0u};
    if (t == 0) s.shared[3] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const uint32_t key = (uint32_t)(e[i] >> 32);
      if (i < slots && e[i] != 0ull && (key & pmask) == prefix) atomicAdd(&s.hist[(key >> shift) & dmask], 1u);
    }
    __syncthreads();
    // thread t owns bins 4t .. 4t+3 counted from the top
    const uint4 h = reinterpret_cast<const uint4*>(s.hist)[BLOCK - 1 - t];
    const uint32_t c[4] = {h.w, h.z, h.y, h.x};
    uint32_t total;
    uint32_t a = block_excl_scan<BLOCK>(c[0] + c[1] + c[2] + c[3], s.scratch, &total);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (a < (uint32_t)rem && a + c[j] >= (uint32_t)rem) {
        s.shared[0] = (uint32_t)(TOP_BINS - 1 - 4 * t - j);
        s.shared[1] = a;
        s.shared[2] = c[j];
      }
      a += c[j];
    }
    __syncthreads();
    const uint32_t b = s.shared[0], cb = s.shared[2];
    rem -= (int)s.shared[1];
    prefix |= b << shift;
    pmask |= dmask << shift;
    if (shift == 0) {  // every key of the bucket is prefix
      __syncthreads();
      *T_out = prefix;
      *need_out = rem;
      return;
    }
    if (cb <= (uint32_t)TOP_SMALL) {
      // the bucket's keys, then the rem-th largest among them (with repeats)
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        if (i < slots) {  // uniform
          const uint32_t key = (uint32_t)(e[i] >> 32);
          const bool match = e[i] != 0ull && (key & pmask) == prefix;
          const uint64_t m = __builtin_amdgcn_ballot_w64(match);
          if (m != 0ull) {
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&s.shared[3], (uint32_t)__popcll(m));
            base = __shfl(base, 0, WAVE);
            if (match)
              s.small[base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u))] = key;
          }
        }
      }
      __syncthreads();
      {
        // 16 lanes per key: lane g counts the bucket's keys 4g .. 4g+3 above
        // it (low half) and at or above it (high half)
        const int i = t >> 4, g = t & 15;
        const uint32_t v = i < (int)cb ? (uint32_t)s.small[i] : 0u;
        uint32_t cnt = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int o = 4 * g + j;
          if (o < (int)cb) {
            const uint32_t y = (uint32_t)s.small[o];
            cnt += (y > v ? 1u : 0u) + (y >= v ? 0x10000u : 0u);
          }
        }
        cnt += row_shr0<1>(cnt);
        cnt += row_shr0<2>(cnt);
        cnt += row_shr0<4>(cnt);
        cnt += row_shr0<8>(cnt);
        // keys equal to the rem-th largest write the same words
        if (g == 15 && i < (int)cb && (cnt & 0xFFFFu) < (uint32_t)rem && (cnt >> 16) >= (uint32_t)rem) {
          s.shared[0] = v;
          s.shared[1] = (uint32_t)rem - (cnt & 0xFFFFu);
        }
      }
      __syncthreads();
      *T_out = s.shared[0];
      *need_out = (int)s.shared[1];
      __syncthreads();
      return;
    }
    top = shift - 1;
  }
}

// Ordered compaction of a selection (key > T, or key == T among the first
// need of them): per (slot, wave) counts of both kinds packed in one word and
// one scan; pos_out(slot, lane) receives each selected element's position in
// ascending slot-major (slot, wave, lane) order.  Every thread must call it.
template <int BLOCK, int NPT, typename Out>
SVA_DEV void compact_selected(const uint64_t (&e)[NPT], int slots, uint32_t T, int need, uint32_t* wbase,
                              uint32_t* scratch, Out out) {
  constexpr int NW = BLOCK / WAVE;
  const int lane = lane_id(), wid = (int)threadIdx.x / WAVE;
  uint64_t mg[NPT], me[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const uint32_t key = (uint32_t)(e[i] >> 32);
    const bool nz = i < slots && e[i] != 0ull;
    mg[i] = __builtin_amdgcn_ballot_w64(nz && key > T);
    me[i] = __builtin_amdgcn_ballot_w64(nz && key == T);
    if (lane == 0 && i < slots) wbase[i * NW + wid] = (uint32_t)__popcll(mg[i]) | ((uint32_t)__popcll(me[i]) << 16);
  }
  __syncthreads();
  const uint32_t wc = (int)threadIdx.x < slots * NW ? wbase[threadIdx.x] : 0u;
  const uint32_t wpre = block_excl_scan<BLOCK>(wc, scratch, nullptr);
  if ((int)threadIdx.x < slots * NW) wbase[threadIdx.x] = wpre;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    if (i < slots && (((mg[i] | me[i]) >> lane) & 1ull)) {
      const uint32_t w = wbase[i * NW + wid];
      const uint32_t gb = (w & 0xFFFFu) + __builtin_amdgcn_mbcnt_hi((uint32_t)(mg[i] >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mg[i], 0u));
      const uint32_t eb = (w >> 16) + __builtin_amdgcn_mbcnt_hi((uint32_t)(me[i] >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)me[i], 0u));
      if ((mg[i] >> lane) & 1ull) out(i, gb + min(eb, (uint32_t)need));
      else if (eb < (uint32_t)need) out(i, gb + eb);
    }
  }
}
constexpr int REG_NW = ITEM_BLOCK / WAVE;
constexpr int REG_OCT = 4;  // shortlist rows per lane octet in flight

struct RegLds {
  int tab, hist, small, shared64, scratch, shared, wbase, slidx, rank, total;
};

__host__ __device__ inline RegLds reg_lds_layout(int S, int C, int L, int npt) {
  RegLds l;
  int o = 0;
  l.tab = o;
  o = align16(o + 4 * S * C);
  l.hist = o;
  o = align16(o + 4 * TOP_BINS);
  l.small = o;
  o = align16(o + 8 * TOP_SMALL);
  l.shared64 = o;
  o = align16(o + 8 * 2);
  l.scratch = o;
  o = align16(o + 4 * (REG_NW + 1));
  l.shared = o;
  o = align16(o + 4 * 4);
  l.wbase = o;
  o = align16(o + 4 * npt * REG_NW);
  l.slidx = o;
  o = align16(o + 4 * L);
  l.rank = o;
  o = align16(o + 4 * L);
  l.total = o;
  return l;
}

// Item `item` (0 <= item < n_seq * H * Q) of p on this workgroup, its dynamic LDS at
// `lds` (reg_lds_layout bytes); returns the budget length it wrote (every
// thread gets the same value).  Every thread of the workgroup must call it.
template <int NPT, int SB>
SVA_DEV int regs_item(const SummonParams& p, int item, unsigned char* lds) {
#pragma clang fp contract(off)
  const RegLds Ly = reg_lds_layout(p.S, p.C, p.L, NPT);
  float* tab = (float*)(lds + Ly.tab);
  uint32_t* shared = (uint32_t*)(lds + Ly.shared);
  uint32_t* wbase = (uint32_t*)(lds + Ly.wbase);
  int32_t* slidx = (int32_t*)(lds + Ly.slidx);
  float* rank = (float*)(lds + Ly.rank);
  const TopLds tl{(uint32_t*)(lds + Ly.hist), (uint64_t*)(lds + Ly.small), (uint32_t*)(lds + Ly.scratch), shared,
                  (uint64_t*)(lds + Ly.shared64)};
  const int t = item % p.Q;
  const int h = (item / p.Q) % p.H;
  const int b = item / (p.Q * p.H);
  // the host admits N <= NPT * BLOCK and every length is at most N
  const int64_t len = min(p.lens ? p.lens[b] : p.N, (int64_t)NPT * ITEM_BLOCK);
  const int64_t off = p.offs ? p.offs[b] : 0;
  const int SC = p.S * p.C;
  const float* lsrc = p.lut + (int64_t)item * SC;

  const int64_t code_base = (int64_t)h * p.code_hs + off * p.S;
  const int64_t causal_last = len - p.Q + t;
  const int S = p.S, C = p.C;
  // R = 64 here: dividing by sqrt(R) = 8 is multiplying by 0.125, exactly
  constexpr float inv_sqrt_r = 0.125f;
  // SB > 0: uint8 codes of SB subspaces, read as one SB-byte load per key,
  // every load of the thread issued before any is used (e[] holds the raw
  // code bytes until the composites replace them), and before the table's
  // barrier, so the code and table loads overlap; SB = 0: any code type
  uint64_t e[NPT];
  uint32_t okm = 0;  // bit i: key i * BLOCK + t is allowed
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int64_t n = (int64_t)i * ITEM_BLOCK + threadIdx.x;
    const bool ok = n < len && (p.mask_type == MASK_NONE ? n <= causal_last
                                                         : mask_allows(p.mask, (int64_t)t * p.mask_ts + n, p.mask_type));
    okm |= (ok ? 1u : 0u) << i;
    e[i] = 0ull;
  }
  if constexpr (SB > 0) {
    using Word = typename std::conditional<SB == 1, uint8_t,
                 typename std::conditional<SB == 2, uint16_t, uint32_t>::type>::type;
    const Word* cw = (const Word*)((const uint8_t*)p.codes + code_base);
#pragma unroll
    for (int i = 0; i < NPT; ++i)
      if ((okm >> i) & 1u) e[i] = cw[(int64_t)i * ITEM_BLOCK + threadIdx.x];
  }
  for (int e2 = threadIdx.x; e2 < SC; e2 += ITEM_BLOCK) tab[e2] = lsrc[e2];
  __syncthreads();
  uint32_t kor = 0u, kand = 0xFFFFFFFFu;
  uint32_t cnt = 0;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int64_t n = (int64_t)i * ITEM_BLOCK + threadIdx.x;
    if ((okm >> i) & 1u) {
      float acc = 0.0f;
      if constexpr (SB > 0) {
#pragma unroll
        for (int s = 0; s < SB; ++s) {
          const int c = (int)((e[i] >> (8 * s)) & 0xFFu);
          acc = acc + tab[s * C + (c >= C ? C - 1 : c)];
        }
      } else {
        const int64_t row = code_base + n * S;
        for (int s = 0; s < S; ++s) {
          int64_t c = load_code(p.codes, row + s, p.ctype);
          c = c < 0 ? 0 : (c >= C ? C - 1 : c);
          acc = acc + tab[s * C + c];
        }
      }
      const uint32_t key = f2key(acc * inv_sqrt_r);
      e[i] = composite(key, (uint32_t)n);
      kor |= key;
      kand &= key;
      ++cnt;
    }
  }
  uint32_t allowed_total;
  block_excl_scan<ITEM_BLOCK>(cnt, tl.scratch, &allowed_total);
  const int leff = (int)min((uint32_t)p.L, allowed_total);
  const int beff = min(p.B, leff);
  if (threadIdx.x == 0) {
    p.sl_count[item] = leff;
    p.fin_count[item] = beff;
    if (p.stats != nullptr) {  // a decode step's statistics, without a launch of their own
      atomicAdd(&p.stats[0], (unsigned long long)leff);
      atomicAdd(&p.stats[1], (unsigned long long)beff);
      atomicAdd(&p.stats[3], 1ull);
    }
  }
  if (leff == 0) return 0;
  // the shortlist: keys above T, then the first need keys at T in key order
  // (every allowed key when the shortlist takes them all)
  uint32_t T = 0u;
  int need = 0x7FFFFFFF;
  if (leff < (int)allowed_total) select_key_regs<ITEM_BLOCK, NPT>(e, NPT, leff, kor, kand, tl, &T, &need);

  // shortlist in ascending key order: slot-major (i, wave, lane) is key order
  compact_selected<ITEM_BLOCK, NPT>(e, NPT, T, need, wbase, tl.scratch, [&](int i, uint32_t pos) {
    if (pos < (uint32_t)leff) slidx[pos] = i * ITEM_BLOCK + (int)threadIdx.x;
  });
  __syncthreads();

  // rescore: lane octet o takes shortlist entries o, o + 128, ...
  {
    const int oct = (int)threadIdx.x >> 3, c = (int)threadIdx.x & 7;
    const float4* q4 = reinterpret_cast<const float4*>(p.q_low + (int64_t)item * 64);
    const float4 q0 = q4[c], q1 = q4[8 + c];
    // a row is 256 bytes (R = 64 floats) and N <= 16 * ITEM_BLOCK keys, so a
    // row's byte offset fits 32 bits: one shift-add per row, the base uniform
    const char* klb = reinterpret_cast<const char*>(p.k_low + (int64_t)h * p.klow_hs + off * 64);
    const uint32_t lane_b = 16u * (uint32_t)c;
    for (int j0 = 0; j0 < leff; j0 += REG_OCT * (ITEM_BLOCK / 8)) {
      float4 r0[REG_OCT], r1[REG_OCT];
#pragma unroll
      for (int u = 0; u < REG_OCT; ++u) {
        const int j = j0 + u * (ITEM_BLOCK / 8) + oct;
        const uint32_t o = ((uint32_t)slidx[j < leff ? j : 0] << 8) + lane_b;
        r0[u] = *reinterpret_cast<const float4*>(klb + o);
        r1[u] = *reinterpret_cast<const float4*>(klb + o + 128);
      }
#pragma unroll
      for (int u = 0; u < REG_OCT; ++u) {
        const int j = j0 + u * (ITEM_BLOCK / 8) + oct;
        const float d = rank_dot64_oct8(r0[u], r1[u], q0, q1);
        if (c == 0 && j < leff) rank[j] = d * inv_sqrt_r;
      }
    }
  }
  __syncthreads();
  if (p.sl_idx != nullptr) {  // the shortlist outputs are optional here
    int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
    float* out_rank = p.sl_rank + (int64_t)item * p.L;
    for (int j = threadIdx.x; j < leff; j += ITEM_BLOCK) {
      out_idx[j] = slidx[j];
      out_rank[j] = rank[j];
    }
  }

  // budget: top beff by (rank desc, key index asc), ascending key order
  constexpr int NB = REG_MAX_L / ITEM_BLOCK;
  uint64_t e2[NB];
  uint32_t kor2 = 0u, kand2 = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int j = (int)threadIdx.x + i * ITEM_BLOCK;
    e2[i] = 0ull;
    if (j < leff) {
      const uint32_t key = f2key(rank[j]);
      e2[i] = composite(key, (uint32_t)slidx[j]);
      kor2 |= key;
      kand2 &= key;
    }
  }
  const int slots2 = (leff + ITEM_BLOCK - 1) / ITEM_BLOCK;
  uint32_t T2 = 0u;
  int need2 = 0x7FFFFFFF;
  if (beff < leff) select_key_regs<ITEM_BLOCK, NB>(e2, slots2, beff, kor2, kand2, tl, &T2, &need2);
  // shortlist slot j = i * BLOCK + t is in ascending key order, so an ordered
  // compaction of the chosen slots writes the budget in ascending key order
  int32_t* out_fin = p.fin_idx + (int64_t)item * p.B;
  compact_selected<ITEM_BLOCK, NB>(e2, slots2, T2, need2, wbase, tl.scratch, [&](int i, uint32_t pos) {
    if (pos < (uint32_t)beff) out_fin[pos] = composite_index(e2[i]);
  });
  return beff;
}

}  // namespace sva
