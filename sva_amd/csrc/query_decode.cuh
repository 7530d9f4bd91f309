#pragma once
// Decode form of the query kernel (one token, one sequence, D = R = 64),
// shared by the query launch and the code-class path's fused launch.
#include "common.cuh"
#include "query.h"
#include "summon.h"

namespace sva {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Decode form (one token of one sequence, D = R = 64, uint8 codes, 16-byte
// aligned code rows, 1x256, 2x256 or 4x64 codes): one 256-thread workgroup per
// head with the layout's sizes at compile time.  The same arithmetic as query_lut_kernel (q_low and
// table entries by sequential fma chains, bounds folded per subspace, the
// floor from the same sample blocks and histogram), with the sampled code
// words loaded 16 bytes at a time into registers.  The sampled sums read the
// single tables (pair tables for four subspaces took longer to build than
// they saved), and one wave finds the floor's bin: only thread 0 writes it.
constexpr int QD = 256;
constexpr int QD_WORDS = 8;  // sampled 16-byte code words per thread (at most 32 KB per head)
// Sampled code words a thread holds for S subspaces: at most SAMPLE_MAX_BLOCKS
// blocks of SAMPLE_KEYS keys, S bytes each, over QD threads.
template <int S, int NT = QD>
constexpr int qd_words() {
  return SAMPLE_MAX_BLOCKS * SAMPLE_KEYS * S / 16 / NT < 1           ? 1
         : SAMPLE_MAX_BLOCKS * SAMPLE_KEYS * S / 16 / NT < QD_WORDS ? SAMPLE_MAX_BLOCKS * SAMPLE_KEYS * S / 16 / NT
                                                                     : QD_WORDS;
}

// NT threads per workgroup (256, or 1024 so that more waves hide the
// latency of the table, sampled-sum and histogram phases).
template <int S, int CMAX, int NT = QD>
SVA_DEV void query_decode_item(const LutParams& p, int h) {
#pragma clang fp contract(off)
  static_assert(NT % 256 == 0 && NT <= 1024, "256 or more threads, whole 64-entry table rows per wave");
  constexpr int SUB = 64 / S;
  // With at least two threads per table entry, two consecutive lanes share a
  // codebook row, PART floats each, instead of every lane loading a whole
  // row (the surplus lanes the last row again); the row's fma chain runs
  // through the pair in order (a DPP hand-off), and the second lane ends
  // with it.  (Four lanes per row measured slower at 4x64: the longer
  // hand-off chain costs more than the loads it saves.)
  constexpr int TPR = NT >= 2 * S * CMAX ? 2 : 1;
  constexpr int PART = SUB / TPR;
  static_assert(TPR == 1 || TPR == 2 || TPR == 4, "a row over 1, 2 or 4 lanes of a DPP row");
  static_assert(PART % 4 == 0, "whole float4s per lane");
  constexpr int EPT = (S * CMAX * TPR + NT - 1) / NT;  // row parts per thread
  constexpr int NW4 = 1024 / NT;                  // float4s of the map per thread
  constexpr int KPW = 16 / S;                     // keys per 16-byte code word
  __shared__ __align__(16) float W[64 * 64];
  __shared__ float qf[64], ql[64];
  __shared__ float tab[S * CMAX];
  __shared__ uint32_t kmin[S], kmax[S];
  __shared__ __align__(16) uint32_t hist[SAMPLE_BINS];
  const int t = threadIdx.x;
  const int lane = lane_id(), wid = t / WAVE;
  const int C = p.C;
  // 1. every load at once: map, query, codebook rows, sampled code words
  float4 wv[NW4];
  const float4* w4 = reinterpret_cast<const float4*>(p.q_proj + (int64_t)h * 4096);
#pragma unroll
  for (int i = 0; i < NW4; ++i) wv[i] = w4[t + i * NT];
  const uint32_t qbits = t < 64 ? load_elem_bits(p.q, (int64_t)h * p.q_hs + t, p.q_dtype) : 0u;
  float4 row[EPT][PART / 4];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = min((t + k * NT) / TPR, S * C - 1);
    const float4* c4 =
        reinterpret_cast<const float4*>(p.codebooks + ((int64_t)h * S * C + e) * SUB + (t % TPR) * PART);
#pragma unroll
    for (int j = 0; j < PART / 4; ++j) row[k][j] = c4[j];
  }
  const int k_rank = p.codes != nullptr ? p.sample_k : 0;
  const int nb = p.sample_blocks;
  const int n_words = nb * 2 * S;  // 32 keys x S bytes per block = 2 S words
  const int64_t N = p.n_keys;
  constexpr int QW = qd_words<S, NT>();
  // every lane loads a word (past the sample, the last one again): a load
  // under a per-lane condition ends in a register merge that waits for it,
  // and for every load issued before it; the sums of words past the sample
  // are discarded
  // (with no sample, the first 16 bytes of the map stand in: the loads stay
  // unconditional, and their words are not used)
  u32x4_t words[QW];
  {
    const bool smp = k_rank > 0;
    const uint8_t* head = smp ? (const uint8_t*)p.codes + (int64_t)h * p.code_hs : (const uint8_t*)p.q_proj;
#pragma unroll
    for (int i = 0; i < QW; ++i) {
      const int gw = smp ? min(t + i * NT, n_words - 1) : 0;
      const int b = gw / (2 * S), wi = gw % (2 * S);
      const int64_t n0 = smp ? ((int64_t)b * (N - SAMPLE_KEYS) / (nb - 1)) & ~(int64_t)15 : 0;
      words[i] = *reinterpret_cast<const u32x4_t*>(head + n0 * S + wi * 16);
    }
  }
  const float sc = p.scale[h];
#pragma unroll
  for (int i = 0; i < NW4; ++i) reinterpret_cast<float4*>(W)[t + i * NT] = wv[i];
  if (t < 64) qf[t] = elem_from_bits(qbits, p.q_dtype);
  if (t < S) {
    kmin[t] = 0xFFFFFFFFu;
    kmax[t] = 0u;
  }
  if (t < SAMPLE_BINS / 4) reinterpret_cast<uint4*>(hist)[t] = uint4{0u, 0u, 0u, 0u};
  __syncthreads();
  // 2. q_low: one lane per output, a sequential fma chain over d
  if (t < 64) {
    float acc = 0.0f;
#pragma unroll 16
    for (int d = 0; d < 64; ++d) acc = __builtin_fmaf(qf[d], W[d * 64 + t], acc);
    const float v = acc * sc;
    ql[t] = v;
    p.q_low[(int64_t)h * 64 + t] = v;
  }
  __syncthreads();
  // 3. table entries (sequential fma chain over the subspace) and bounds;
  // with C a multiple of 64 every wave's entries share a subspace, so the
  // bounds fold over the wave first (one atomic per wave, not per entry)
  float* lut_out = p.lut + (int64_t)h * S * C;
  const bool wave_sub = C % WAVE == 0;
  const int g = t % TPR;  // this lane's part of its row
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int e = (t + k * NT) / TPR;
    const int s = min(e, S * C - 1) / C;
    uint32_t kl = 0xFFFFFFFFu, kh = 0u;
    const float* rr = reinterpret_cast<const float*>(row[k]);
    float acc = 0.0f;
#pragma unroll
    for (int step = 0; step < TPR; ++step) {
      // lane g's chain is the row's through part g after step g: it takes
      // lane g - 1's (parts 0 .. g - 1) and continues with its own part
      if (step > 0) acc = __int_as_float((int)row_shr0<1>((uint32_t)__float_as_int(acc)));
#pragma unroll
      for (int j = 0; j < PART; ++j) acc = __builtin_fmaf(ql[s * SUB + g * PART + j], rr[j], acc);
    }
    if (e < S * C && g == TPR - 1) {
      tab[e] = acc;
      lut_out[e] = acc;
      kl = kh = f2key(acc);
      if (!wave_sub) {
        atomicMin(&kmin[s], kl);
        atomicMax(&kmax[s], kh);
      }
    }
    if (wave_sub && (k * NT + WAVE * wid) / TPR < S * C) {  // uniform: the wave's entries exist
      wave_min_max_u32(kl, kh);
      if (lane == 0) {
        atomicMin(&kmin[s], kl);
        atomicMax(&kmax[s], kh);
      }
    }
  }
  __syncthreads();
  float lo = 0.0f, hi = 0.0f;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    lo = lo + key2f(kmin[s]);
    hi = hi + key2f(kmax[s]);
  }
  float t_lo = -INFINITY;
  if (k_rank > 0 && hi > lo) {
    const uint32_t cm = (uint32_t)(C - 1);
    // 4. sampled sums, kept in registers
    float sums[QW * KPW];
#pragma unroll
    for (int i = 0; i < QW; ++i) {
      const bool valid = t + i * NT < n_words;  // every code is clamped to the table: reads stay in bounds
#pragma unroll
      for (int q = 0; q < KPW; ++q) {
        float acc = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < S; ++s2) {
          const int j = q * S + s2;
          const uint32_t c = min((words[i][j >> 2] >> (8 * (j & 3))) & 0xFFu, cm);
          acc = acc + tab[s2 * C + c];
        }
        sums[i * KPW + q] = valid ? acc : -INFINITY;
      }
    }
    // every sum first, then every bin: an LDS atomic between two table reads
    // would keep the reads from being issued together
    const float base = lo;
    const float inv_w = (float)SAMPLE_BINS / (hi - lo);
#pragma unroll
    for (int i = 0; i < QW * KPW; ++i) {
      if (sums[i] != -INFINITY) {
        int bin = (int)((sums[i] - lo) * inv_w);
        bin = bin < 0 ? 0 : (bin >= SAMPLE_BINS ? SAMPLE_BINS - 1 : bin);
        atomicAdd(&hist[bin], 1u);
      }
    }
    __syncthreads();
    // 5. the bin of the k-th largest sampled sum, found by wave 0 alone:
    // lane l owns bins SAMPLE_BINS - 1 - BPL l - j (j = 0 .. BPL - 1, in
    // descending order); the lane whose bins cross k holds it (bin 0 when
    // fewer than k sums were sampled)
    if (wid == 0) {
      constexpr int BPL = SAMPLE_BINS / WAVE;
      static_assert(BPL % 4 == 0, "whole uint4s of bins per lane");
      uint32_t c[BPL];
#pragma unroll
      for (int u = 0; u < BPL / 4; ++u) {
        const uint4 hv = reinterpret_cast<const uint4*>(hist)[SAMPLE_BINS / 4 - 1 - (lane * (BPL / 4) + u)];
        c[4 * u + 0] = hv.w;
        c[4 * u + 1] = hv.z;
        c[4 * u + 2] = hv.y;
        c[4 * u + 3] = hv.x;
      }
      uint32_t mine = 0;
#pragma unroll
      for (int j = 0; j < BPL; ++j) mine += c[j];
      uint32_t a = wave_incl_scan(mine) - mine;
      int found = -1;
#pragma unroll
      for (int j = 0; j < BPL; ++j) {
        if (a < (uint32_t)k_rank && a + c[j] >= (uint32_t)k_rank) found = SAMPLE_BINS - 1 - BPL * lane - j;
        a += c[j];
      }
      const uint64_t m = __builtin_amdgcn_ballot_w64(found >= 0);
      const int bin = m != 0ull ? __builtin_amdgcn_readlane(found, __builtin_ctzll(m)) : 0;
      t_lo = base + (float)bin / inv_w;
    }
  }
  if (t == 0) {
    float* rg = p.range + (int64_t)h * 4;
    rg[0] = lo;
    rg[1] = hi;
    rg[2] = t_lo;
    rg[3] = 0.0f;
  }
}

}  // namespace sva
