// Summon: PQ scan over the cached codes, exact shortlist selection and the
// low-rank rescore of the shortlist (sva/llama.py:270-292, sva/ops.py:50-71).
//
// Item path (this file, summon_item_kernel): one workgroup per query item
// (sequence, head, token).  The LUT sits in LDS; every allowed key's score is
// turned into an order-preserving key; an LDS radix select finds the L-th
// largest key T and how many keys equal to T to take (lowest key indices
// first); a compaction in key-index order writes the shortlist; each
// shortlisted key is rescored against q_low in torch's summation order.
// Keys live in LDS when they fit, otherwise they are recomputed per pass.
//
// Fused item path (summon_regs_kernel): caches of up to 16K keys with a
// budget run shortlist, rescore and budget in one workgroup per item from
// registers (the prefill shape).
//
// The long-context q=1 path (many workgroups per item) is in summon_wide.hip.
#include <type_traits>

#include "capi_internal.h"
#include "common.cuh"
#include "query.h"
#include "summon.h"

using namespace sva;

namespace {

constexpr int ITEM_BLOCK = 1024;

struct ItemLds {
  // offsets (bytes) of the dynamic LDS regions
  int tab, ql, hist, scratch, shared, slidx, keys, total;
};

__host__ __device__ inline int align16(int x) { return (x + 15) & ~15; }

__host__ __device__ inline ItemLds item_lds_layout(int S, int C, int R, int L, int64_t N, bool keys_in_lds) {
  ItemLds l;
  int o = 0;
  l.tab = o;
  o = align16(o + 4 * S * C);
  l.ql = o;
  o = align16(o + 4 * R);
  l.hist = o;
  o = align16(o + 4 * 256);
  l.scratch = o;
  o = align16(o + 4 * (ITEM_BLOCK / WAVE + 1));
  l.shared = o;
  o = align16(o + 4 * 4);
  l.slidx = o;
  o = align16(o + 4 * L);
  l.keys = o;
  if (keys_in_lds) o = align16(o + (int)(4 * N));
  l.total = o;
  return l;
}

__global__ void __launch_bounds__(ITEM_BLOCK) summon_item_kernel(SummonParams p, int keys_in_lds) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int item = blockIdx.x;
  const int t = item % p.Q;
  const int h = (item / p.Q) % p.H;
  const int b = item / (p.Q * p.H);
  const int64_t len = p.lens ? p.lens[b] : p.N;
  const int64_t off = p.offs ? p.offs[b] : 0;
  const ItemLds L = item_lds_layout(p.S, p.C, p.R, p.L, len, keys_in_lds != 0);
  float* tab = (float*)(lds + L.tab);
  float* ql = (float*)(lds + L.ql);
  uint32_t* hist = (uint32_t*)(lds + L.hist);
  uint32_t* scratch = (uint32_t*)(lds + L.scratch);
  uint32_t* shared = (uint32_t*)(lds + L.shared);
  int32_t* slidx = (int32_t*)(lds + L.slidx);
  uint32_t* keys = (uint32_t*)(lds + L.keys);

  const int SC = p.S * p.C;
  const float* lsrc = p.lut + (int64_t)item * SC;
  for (int e = threadIdx.x; e < SC; e += ITEM_BLOCK) tab[e] = lsrc[e];
  const float* qsrc = p.q_low + (int64_t)item * p.R;
  for (int r = threadIdx.x; r < p.R; r += ITEM_BLOCK) ql[r] = qsrc[r];
  __syncthreads();

  const int64_t code_base = (int64_t)h * p.code_hs + off * p.S;
  const int64_t causal_last = len - p.Q + t;  // last allowed key without a mask
  const char* mrow = p.mask ? (const char*)p.mask : nullptr;
  const int S = p.S, C = p.C;
  const float sqrt_r = p.sqrt_r;

  auto compute_key = [&](int64_t n) -> uint32_t {
    const bool allowed =
        p.mask_type == MASK_NONE ? n <= causal_last : mask_allows(mrow, (int64_t)t * p.mask_ts + n, p.mask_type);
    if (!allowed) return 0u;
    float acc = 0.0f;
    const int64_t row = code_base + n * S;
    for (int s = 0; s < S; ++s) {
      int64_t c = load_code(p.codes, row + s, p.ctype);
      c = c < 0 ? 0 : (c >= C ? C - 1 : c);
      acc = acc + tab[s * C + c];
    }
    return f2key(acc / sqrt_r);
  };

  uint32_t cnt = 0;
  for (int64_t n = threadIdx.x; n < len; n += ITEM_BLOCK) {
    const uint32_t k = compute_key(n);
    cnt += k != 0u;
    if (keys_in_lds) keys[n] = k;
  }
  uint32_t allowed_total;
  block_excl_scan<ITEM_BLOCK>(cnt, scratch, &allowed_total);
  const int leff = (int)min((int64_t)p.L, (int64_t)allowed_total);
  if (leff == 0) {
    if (threadIdx.x == 0) p.sl_count[item] = 0;
    return;
  }

  auto get_key = [&](int64_t n) -> uint32_t { return keys_in_lds ? keys[n] : compute_key(n); };

  uint32_t T;
  int keq;
  radix_select_u32<ITEM_BLOCK>([&](int i) { return get_key(i); }, (int)len, leff, hist, scratch, shared, &T, &keq);

  // compaction in key-index order over thread-contiguous segments
  const int64_t seg = (len + ITEM_BLOCK - 1) / ITEM_BLOCK;
  const int64_t lo = min((int64_t)threadIdx.x * seg, len);
  const int64_t hi = min(lo + seg, len);
  uint32_t gt = 0, eq = 0;
  for (int64_t n = lo; n < hi; ++n) {
    const uint32_t k = get_key(n);
    gt += k > T;
    eq += k == T;
  }
  const uint32_t eq_before = block_excl_scan<ITEM_BLOCK>(eq, scratch, nullptr);
  const int take_eq = max(0, min((int)eq, keq - (int)eq_before));
  uint32_t pos = block_excl_scan<ITEM_BLOCK>(gt + (uint32_t)take_eq, scratch, nullptr);
  int taken = 0;
  for (int64_t n = lo; n < hi; ++n) {
    const uint32_t k = get_key(n);
    if (k > T) {
      slidx[pos++] = (int32_t)n;
    } else if (k == T && taken < take_eq) {
      slidx[pos++] = (int32_t)n;
      ++taken;
    }
  }
  __syncthreads();

  // exact low-rank rescore of the shortlist (torch's sum order)
  const float* kl = p.k_low + (int64_t)h * p.klow_hs + off * p.R;
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  float* out_rank = p.sl_rank + (int64_t)item * p.L;
  for (int j = threadIdx.x; j < leff; j += ITEM_BLOCK) {
    const int64_t n = slidx[j];
    const float* row = kl + n * p.R;
    const float dot = p.R == 64 ? torch_order_dot64(row, ql) : torch_order_dot(row, ql, p.R);
    out_idx[j] = (int32_t)n;
    out_rank[j] = dot / sqrt_r;
  }
  if (threadIdx.x == 0) p.sl_count[item] = leff;
}


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

// items: n_seq * H * Q; workgroups take head-major item ranges per XCD
// (xcd_range_item), so one XCD's L2 holds the k_low rows of one or two heads.
template <int NPT, int SB>
__global__ void __launch_bounds__(ITEM_BLOCK, NPT <= 8 ? 8 : 4) summon_regs_kernel(SummonParams p, int64_t items) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const RegLds Ly = reg_lds_layout(p.S, p.C, p.L, NPT);
  float* tab = (float*)(lds + Ly.tab);
  uint32_t* shared = (uint32_t*)(lds + Ly.shared);
  uint32_t* wbase = (uint32_t*)(lds + Ly.wbase);
  int32_t* slidx = (int32_t*)(lds + Ly.slidx);
  float* rank = (float*)(lds + Ly.rank);
  const TopLds tl{(uint32_t*)(lds + Ly.hist), (uint64_t*)(lds + Ly.small), (uint32_t*)(lds + Ly.scratch), shared,
                  (uint64_t*)(lds + Ly.shared64)};
  const int64_t item_x = xcd_range_item((int64_t)blockIdx.x, items);
  if (item_x < 0) return;  // block-uniform: past the last item
  const int item = (int)item_x;
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
  if (leff == 0) return;
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
}

template <int NPT, int SB>
int launch_regs(const SummonParams& p, int64_t items, size_t lds, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((summon_regs_kernel<NPT, SB>), kMaxLds, "hipFuncSetAttribute(summon_regs_kernel)");
  hipLaunchKernelGGL((summon_regs_kernel<NPT, SB>), dim3((unsigned)xcd_range_grid(items)), dim3(ITEM_BLOCK), lds,
                     stream, p, items);
  SVA_CHECK_LAUNCH("summon_regs_kernel");
  return SVA_OK;
}

template <int NPT>
int launch_regs_codes(const SummonParams& p, int64_t items, size_t lds, hipStream_t stream) {
  // one load per key for uint8 codes of 1, 2 or 4 subspaces at aligned rows
  const int64_t S = p.S;
  const bool u8 = p.ctype == CODE_U8 && (S == 1 || S == 2 || S == 4) && p.code_hs % S == 0 &&
                  ((uintptr_t)p.codes % (uintptr_t)S) == 0;
  if (u8 && S == 1) return launch_regs<NPT, 1>(p, items, lds, stream);
  if (u8 && S == 2) return launch_regs<NPT, 2>(p, items, lds, stream);
  if (u8 && S == 4) return launch_regs<NPT, 4>(p, items, lds, stream);
  return launch_regs<NPT, 0>(p, items, lds, stream);
}
}  // namespace

namespace sva {

bool summon_regs_eligible(const SummonParams& p) {
  if (p.B <= 0 || p.R != 64 || p.L > REG_MAX_L || p.N > 16 * ITEM_BLOCK) return false;
  if (((uintptr_t)p.k_low & 15u) != 0 || p.klow_hs % 4 != 0 || ((uintptr_t)p.q_low & 15u) != 0) return false;
  return reg_lds_layout(p.S, p.C, p.L, 16).total <= kMaxLds;
}

int summon_regs_path(const SummonParams& p, int64_t items, hipStream_t stream) {
  const int npt = p.N <= 4 * ITEM_BLOCK ? 4 : (p.N <= 8 * ITEM_BLOCK ? 8 : 16);
  const size_t lds = (size_t)reg_lds_layout(p.S, p.C, p.L, npt).total;
  if (npt == 4) return launch_regs_codes<4>(p, items, lds, stream);
  if (npt == 8) return launch_regs_codes<8>(p, items, lds, stream);
  return launch_regs_codes<16>(p, items, lds, stream);
}

int summon_item_path(const SummonParams& p, int64_t items, hipStream_t stream) {
  const bool keys_fit = item_lds_layout(p.S, p.C, p.R, p.L, p.N, true).total <= kMaxLds;
  const ItemLds layout = item_lds_layout(p.S, p.C, p.R, p.L, p.N, keys_fit);
  SVA_UNSUPPORTED(layout.total <= kMaxLds, "sva_summon: shortlist %d with %dx%d codes exceeds LDS", p.L, p.S, p.C);
  SVA_SET_MAX_LDS_ONCE(summon_item_kernel, kMaxLds, "hipFuncSetAttribute(summon_item_kernel)");
  hipLaunchKernelGGL(summon_item_kernel, dim3((unsigned)items), dim3(ITEM_BLOCK), (size_t)layout.total, stream, p,
                     keys_fit ? 1 : 0);
  SVA_CHECK_LAUNCH("summon_item_kernel");
  return SVA_OK;
}

}  // namespace sva

extern "C" int sva_summon_strategy(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t R, int64_t S,
                                   int64_t C, int64_t L, int code_type, int mask_type) {
  sva::SummonParams p{};
  alignas(16) static const float dummy[4] = {0, 0, 0, 0};
  p.codes = dummy;
  p.ctype = code_type;
  p.code_hs = 0;
  p.offs = n_seq == 1 ? nullptr : (const int64_t*)dummy;
  p.H = (int)H;
  p.Q = (int)Q;
  p.N = n_keys;
  p.R = (int)R;
  p.S = (int)S;
  p.C = (int)C;
  p.L = (int)L;
  p.mask = dummy;
  p.mask_type = mask_type;
  if (sva::summon_class_eligible(p, n_seq * H * Q)) return 2;
  if (sva::summon_wide_eligible(p, n_seq * H * Q)) return 1;
  p.B = 1;
  return sva::summon_regs_eligible(p) ? 3 : 0;
}

extern "C" size_t sva_summon_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t L) {
  return sva::summon_wide_workspace_bytes(n_seq, H, Q, n_keys, L);
}

namespace {

int summon_impl(const char* fn, const float* lut, const float* score_range, const float* q_low, const void* codes,
                int code_type, int64_t code_head_stride, const float* k_low, int64_t k_low_head_stride,
                const int64_t* seq_offsets, const int64_t* seq_lens, int64_t n_seq, int64_t H, int64_t Q,
                int64_t n_keys, int64_t R, int64_t S, int64_t C, int64_t L, const void* mask, int mask_type,
                int64_t mask_tok_stride, int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B,
                int32_t* fin_idx, int32_t* fin_count, void* workspace, size_t workspace_bytes, void* stream,
                const sva::FusedVerify* fv = nullptr, bool* fused = nullptr, int32_t* overshoot = nullptr,
                const sva::QueryLaunch* query = nullptr, unsigned long long* stats = nullptr) {
  if (fused != nullptr) *fused = false;
  SVA_REQUIRE(lut && score_range && q_low && codes && k_low && sl_count, "%s: null pointer", fn);
  SVA_REQUIRE((sl_idx == nullptr) == (sl_rank == nullptr), "%s: shortlist indices and ranks go together", fn);
  SVA_REQUIRE((seq_offsets == nullptr) == (seq_lens == nullptr), "%s: offsets and lengths go together", fn);
  SVA_REQUIRE(n_seq > 0 && H > 0 && Q > 0 && n_keys >= 0, "%s: bad sizes", fn);
  SVA_REQUIRE(n_keys < (1ll << 31), "%s: at most 2^31-1 keys per sequence", fn);
  SVA_REQUIRE(R > 0 && R <= 511 && S > 0 && R % S == 0 && C > 0 && S * C <= 16384,
              "%s: bad rank/PQ layout R=%lld S=%lld C=%lld", fn, (long long)R, (long long)S, (long long)C);
  SVA_REQUIRE(L > 0 && L <= 16384, "%s: shortlist %lld out of range (1..16384)", fn, (long long)L);
  SVA_REQUIRE(code_type >= 0 && code_type <= 3, "%s: bad code type", fn);
  SVA_REQUIRE(mask_type >= 0 && mask_type <= 4, "%s: bad mask type", fn);
  SVA_REQUIRE(mask_type == SVA_MASK_NONE || mask_type == SVA_MASK_BOOL || mask != nullptr,
              "%s: mask type given without a mask", fn);
  SVA_REQUIRE(R != 64 || (((uintptr_t)k_low & 15u) == 0 && k_low_head_stride % 4 == 0),
              "%s: k_low must be 16-byte aligned", fn);
  const int64_t items = n_seq * H * Q;
  SVA_REQUIRE(items < (1ll << 31), "%s: too many query items", fn);
  sva::SummonParams p;
  p.lut = lut;
  p.range = score_range;
  p.q_low = q_low;
  p.codes = codes;
  p.ctype = code_type;
  p.code_hs = code_head_stride;
  p.k_low = k_low;
  p.klow_hs = k_low_head_stride;
  p.offs = seq_offsets;
  p.lens = seq_lens;
  p.H = (int)H;
  p.Q = (int)Q;
  p.N = n_keys;
  p.R = (int)R;
  p.S = (int)S;
  p.C = (int)C;
  p.L = (int)L;
  p.mask = mask;
  p.mask_type = mask_type;
  p.mask_ts = mask_tok_stride;
  p.sqrt_r = (float)sqrt((double)R);
  p.sl_idx = sl_idx;
  p.sl_rank = sl_rank;
  p.sl_count = sl_count;
  p.B = (int)B;
  p.fin_idx = fin_idx;
  p.fin_count = fin_count;
  p.stats = stats;
  // a prepared query launch (the tables this call reads): the code-class
  // path runs its decode form in one grid with the code counts; every other
  // path launches it first
  const bool class_path = n_keys > 0 && sva::summon_class_eligible(p, items);
  SVA_REQUIRE(stats == nullptr || (n_keys > 0 && !class_path && !sva::summon_wide_eligible(p, items) &&
                                   sva::summon_regs_eligible(p)),
              "%s: a statistics row is added on the per-item register path only", fn);
  // without shortlist outputs only the fused per-item path (strategy 3) runs
  SVA_UNSUPPORTED(sl_idx != nullptr || n_keys == 0 ||
                      (B > 0 && !class_path && !sva::summon_wide_eligible(p, items) && sva::summon_regs_eligible(p)),
                  "%s: these shapes keep the shortlist in memory; pass shortlist outputs", fn);
  if (query != nullptr && !(class_path && query->form == sva::QUERY_DECODE_1_256)) {
    const int rc = sva::query_lut_launch(*query, (hipStream_t)stream);
    if (rc != SVA_OK) return rc;
    query = nullptr;
  }
  if (n_keys == 0) {
    int rc = sva::fill_i32(sl_count, items, 0, (hipStream_t)stream);
    if (rc == SVA_OK && B > 0) rc = sva::fill_i32(fin_count, items, 0, (hipStream_t)stream);
    return rc;
  }
  if (class_path) {
    const bool with_fv = fv != nullptr && sva::fused_verify_eligible(p, items, *fv);
    const int rc = sva::summon_class_path(p, workspace, workspace_bytes, (hipStream_t)stream, with_fv ? fv : nullptr,
                                          overshoot, query);
    if (rc == SVA_OK && fused != nullptr) *fused = with_fv;
    return rc;
  }
  if (sva::summon_wide_eligible(p, items)) {
    const bool with_fv = fv != nullptr && sva::fused_verify_eligible(p, items, *fv);
    const int rc = sva::summon_wide_path(p, workspace, workspace_bytes, (hipStream_t)stream, with_fv ? fv : nullptr,
                                         overshoot);
    if (rc == SVA_OK && fused != nullptr) *fused = with_fv;
    return rc;
  }
  if (overshoot != nullptr) {  // the per-item paths use no sampled floor
    const int rc = sva::fill_i32(overshoot, items, 0, (hipStream_t)stream);
    if (rc != SVA_OK) return rc;
  }
  if (sva::summon_regs_eligible(p)) return sva::summon_regs_path(p, items, (hipStream_t)stream);
  int rc = sva::summon_item_path(p, items, (hipStream_t)stream);
  if (rc == SVA_OK && B > 0)
    rc = sva::budget_select_launch(sl_idx, sl_rank, sl_count, items, L, B, fin_idx, fin_count, (hipStream_t)stream);
  return rc;
}

}  // namespace

extern "C" int sva_summon(const float* lut, const float* score_range, const float* q_low, const void* codes,
                          int code_type, int64_t code_head_stride, const float* k_low, int64_t k_low_head_stride,
                          const int64_t* seq_offsets, const int64_t* seq_lens, int64_t n_seq, int64_t H, int64_t Q,
                          int64_t n_keys, int64_t R, int64_t S, int64_t C, int64_t L, const void* mask, int mask_type,
                          int64_t mask_tok_stride, int32_t* sl_idx, float* sl_rank, int32_t* sl_count,
                          void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  return summon_impl("sva_summon", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                     k_low_head_stride, seq_offsets, seq_lens, n_seq, H, Q, n_keys, R, S, C, L, mask, mask_type,
                     mask_tok_stride, sl_idx, sl_rank, sl_count, 0, nullptr, nullptr, workspace, workspace_bytes,
                     stream);
}

extern "C" int sva_summon_select(const float* lut, const float* score_range, const float* q_low, const void* codes,
                                 int code_type, int64_t code_head_stride, const float* k_low,
                                 int64_t k_low_head_stride, const int64_t* seq_offsets, const int64_t* seq_lens,
                                 int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t R, int64_t S, int64_t C,
                                 int64_t L, const void* mask, int mask_type, int64_t mask_tok_stride, int32_t* sl_idx,
                                 float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx, int32_t* fin_count,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(fin_idx && fin_count, "sva_summon_select: null pointer");
  SVA_REQUIRE(B > 0 && B <= 8192, "sva_summon_select: budget %lld out of range (1..8192)", (long long)B);
  return summon_impl("sva_summon_select", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                     k_low_head_stride, seq_offsets, seq_lens, n_seq, H, Q, n_keys, R, S, C, L, mask, mask_type,
                     mask_tok_stride, sl_idx, sl_rank, sl_count, B, fin_idx, fin_count, workspace, workspace_bytes,
                     stream);
}

extern "C" int sva_lookup_select(const void* q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R,
                                 int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                                 const void* codes, int code_type, int64_t code_head_stride, const float* k_low,
                                 int64_t k_low_head_stride, int64_t n_keys, int64_t L, const void* mask, int mask_type,
                                 int64_t mask_tok_stride, float* q_low, float* lut, float* score_range,
                                 int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx,
                                 int32_t* fin_count, void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(q && q_proj && scale && codebooks && codes && q_low && lut && score_range,
              "sva_lookup_select: null pointer");
  SVA_REQUIRE(fin_idx && fin_count, "sva_lookup_select: null pointer");
  SVA_REQUIRE(B > 0 && B <= 8192, "sva_lookup_select: budget %lld out of range (1..8192)", (long long)B);
  SVA_REQUIRE(H > 0 && n_keys >= 0 && L > 0, "sva_lookup_select: bad sizes");
  sva::QueryLaunch ql;
  const int rc = sva::query_lut_setup(q, q_dtype, 0, q_head_stride, 0, 1, H, 1, D, R, S, C, q_proj, scale, codebooks,
                                      codes, code_type, code_head_stride, n_keys, L, q_low, lut, score_range, &ql);
  if (rc != SVA_OK) return rc;
  return summon_impl("sva_lookup_select", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                     k_low_head_stride, nullptr, nullptr, 1, H, 1, n_keys, R, S, C, L, mask, mask_type,
                     mask_tok_stride, sl_idx, sl_rank, sl_count, B, fin_idx, fin_count, workspace, workspace_bytes,
                     stream, nullptr, nullptr, nullptr, &ql);
}

namespace sva {

// sva_lookup_verify with an optional statistics row (see SummonParams::stats;
// the per-item register path only).  The caller clears the error state.
int lookup_verify_impl(const void* q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R,
                       int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                       const void* codes, int code_type, int64_t code_head_stride, const float* k_low,
                       int64_t k_low_head_stride, int64_t n_keys, int64_t L, const void* mask, int mask_type,
                       int64_t mask_tok_stride, float* q_low, float* lut, float* score_range,
                       int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx,
                       int32_t* fin_count, void* workspace, size_t workspace_bytes, const void* keys,
                       const void* values, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                       int64_t G, float scaling, void* out, int out_dtype, int64_t out_head_stride,
                       void* verify_workspace, size_t verify_workspace_bytes, int32_t* floor_overshoot,
                       void* stream, unsigned long long* stats) {
  SVA_REQUIRE(q && q_proj && scale && codebooks && codes && q_low && lut && score_range,
              "sva_lookup_verify: null pointer");
  SVA_REQUIRE(fin_idx && fin_count && keys && values && out, "sva_lookup_verify: null pointer");
  SVA_REQUIRE(B > 0 && B <= 8192, "sva_lookup_verify: budget %lld out of range (1..8192)", (long long)B);
  SVA_REQUIRE(H > 0 && G > 0 && H % G == 0 && n_keys > 0 && L > 0, "sva_lookup_verify: bad sizes");
  SVA_REQUIRE(q_dtype >= 0 && q_dtype <= 2 && kv_dtype >= 0 && kv_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
              "sva_lookup_verify: bad dtype");
  sva::QueryLaunch ql;
  int rc = sva::query_lut_setup(q, q_dtype, 0, q_head_stride, 0, 1, H, 1, D, R, S, C, q_proj, scale, codebooks, codes,
                                code_type, code_head_stride, n_keys, L, q_low, lut, score_range, &ql);
  if (rc != SVA_OK) return rc;
  sva::FusedVerify fv{};
  fv.q = q;
  fv.q_dtype = q_dtype;
  fv.q_hs = q_head_stride;
  fv.keys = keys;
  fv.values = values;
  fv.kv_dtype = kv_dtype;
  fv.kv_hs = kv_head_stride;
  fv.kv_rs = kv_row_stride;
  const uintptr_t kv_align = kv_dtype == 0 ? 15u : 7u;
  fv.kv_vec = (((uintptr_t)keys | (uintptr_t)values) & kv_align) == 0 && kv_head_stride % 4 == 0 &&
              kv_row_stride % 4 == 0;
  fv.G = (int)G;
  fv.D = (int)D;
  fv.scaling = scaling;
  fv.out = out;
  fv.out_dtype = out_dtype;
  fv.o_hs = out_head_stride;
  bool fused = false;
  rc = summon_impl("sva_lookup_verify", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                   k_low_head_stride, nullptr, nullptr, 1, H, 1, n_keys, R, S, C, L, mask, mask_type, mask_tok_stride,
                   sl_idx, sl_rank, sl_count, B, fin_idx, fin_count, workspace, workspace_bytes, stream, &fv, &fused,
                   floor_overshoot, &ql, stats);
  if (rc != SVA_OK || fused) return rc;
  return sva_verify(q, q_dtype, 0, q_head_stride, 0, keys, values, kv_dtype, kv_head_stride, kv_row_stride, nullptr,
                    nullptr, n_keys, fin_idx, fin_count, 1, H, G, 1, D, B, scaling, out, out_dtype, 0, out_head_stride,
                    0, verify_workspace, verify_workspace_bytes, stream);
}

}  // namespace sva

extern "C" int sva_lookup_verify(const void* q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R,
                                 int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                                 const void* codes, int code_type, int64_t code_head_stride, const float* k_low,
                                 int64_t k_low_head_stride, int64_t n_keys, int64_t L, const void* mask, int mask_type,
                                 int64_t mask_tok_stride, float* q_low, float* lut, float* score_range,
                                 int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx,
                                 int32_t* fin_count, void* workspace, size_t workspace_bytes, const void* keys,
                                 const void* values, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                                 int64_t G, float scaling, void* out, int out_dtype, int64_t out_head_stride,
                                 void* verify_workspace, size_t verify_workspace_bytes, int32_t* floor_overshoot,
                                 void* stream) {
  sva::clear_error();
  return sva::lookup_verify_impl(q, q_dtype, q_head_stride, H, D, R, S, C, q_proj, scale, codebooks, codes, code_type,
                                 code_head_stride, k_low, k_low_head_stride, n_keys, L, mask, mask_type,
                                 mask_tok_stride, q_low, lut, score_range, sl_idx, sl_rank, sl_count, B, fin_idx,
                                 fin_count, workspace, workspace_bytes, keys, values, kv_dtype, kv_head_stride,
                                 kv_row_stride, G, scaling, out, out_dtype, out_head_stride, verify_workspace,
                                 verify_workspace_bytes, floor_overshoot, stream, nullptr);
}
