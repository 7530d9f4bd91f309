// Query side of the decode path: learned query map, per-query PQ lookup
// table, score bounds and a sampled shortlist-threshold estimate, and the
// all-keys PQ score kernel.
//
// q_low[r]  = (sum_d q[d] * q_proj[h][d][r], sequential fma over d) * scale[h]
//             (sva/llama.py:211)
// lut[s][c] = sum_j q_low[s*sub + j] * cb[h][s][c][j], sequential fma over j
//             (sva/ops.py:68)
// score     = (((0 + lut[0][c0]) + lut[1][c1]) + ...) / sqrt(R)   (sva/ops.py:64-71)
#include "capi_internal.h"
#include "common.cuh"
#include "query_decode.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int PREP_BLOCK = 1024;
static_assert(SAMPLE_BINS == PREP_BLOCK, "one histogram bin per thread");


// One workgroup per query item.  The sampled codes and the head's weights
// are staged in LDS in one round of loads; then q_low (one thread per
// output, a sequential fma chain over d), the
// table (one thread per entry, codebook rows padded for conflict-free reads),
// per-subspace key bounds folded per wave, and the sampled threshold: a
// histogram of the sampled sums and a scan from the top bin.
__global__ void __launch_bounds__(PREP_BLOCK) query_lut_kernel(LutParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int item = blockIdx.x;
  const int t = threadIdx.x;
  const int tq = item % p.Q;
  const int h = (item / p.Q) % p.H;
  const int b = item / (p.Q * p.H);
  const int D = p.D, R = p.R, S = p.S, C = p.C;
  const int sub = R / S;
  const int cbs = sub + 1;                       // padded codebook row: conflict-free column reads
  float* W = (float*)lds;                        // [D * R] learned map of head h
  float* cb = W + D * R;                         // [S * C][cbs] its codebooks
  float* qf = cb + S * C * cbs;                  // [D]
  float* ql = qf + D;                            // [R]
  float* tab = ql + R;                           // [S * C]
  uint32_t* kmin = (uint32_t*)(tab + S * C);     // [S]
  uint32_t* kmax = kmin + S;                     // [S]
  uint32_t* shist = kmax + S;                    // [SAMPLE_BINS]
  uint32_t* misc = shist + SAMPLE_BINS;          // [4]
  uint32_t* scratch = misc + 4;                  // [PREP_BLOCK / 64 + 1]
  uint8_t* scodes = (uint8_t*)(scratch + PREP_BLOCK / 64 + 1);  // [sample_blocks * SAMPLE_KEYS * S] sampled codes

  // 0. sampled codes: blocks of SAMPLE_KEYS keys spread over the cache (block
  // starts at multiples of 16 keys), staged in LDS with the weights: the loads
  // complete by the first barrier
  const int64_t N = p.n_keys;
  const int k = p.codes != nullptr ? p.sample_k : 0;
  const bool sample = k > 0;
  const int n_blocks = p.sample_blocks;
  const int n_samples = n_blocks * SAMPLE_KEYS;
  if (sample) {
    const uint8_t* head = (const uint8_t*)p.codes + (int64_t)h * p.code_hs;
    const int wpb = SAMPLE_KEYS * S / 4;  // 32-bit words per sample block (block starts are 16-byte multiples)
    if (((uintptr_t)head & 3u) == 0) {
      for (int w = t; w < n_blocks * wpb; w += PREP_BLOCK) {
        const int blk = w / wpb;
        const int64_t n0 = ((int64_t)blk * (N - SAMPLE_KEYS) / (n_blocks - 1)) & ~(int64_t)15;
        reinterpret_cast<uint32_t*>(scodes)[w] = reinterpret_cast<const uint32_t*>(head + n0 * S)[w - blk * wpb];
      }
    } else {
      for (int e = t; e < n_samples * S; e += PREP_BLOCK) {
        const int blk = e / (SAMPLE_KEYS * S);
        const int64_t n0 = ((int64_t)blk * (N - SAMPLE_KEYS) / (n_blocks - 1)) & ~(int64_t)15;
        scodes[e] = head[n0 * S + e % (SAMPLE_KEYS * S)];
      }
    }
  }
  // the head's weights into LDS with wide coalesced loads (one round)
  {
    const float4* w4 = reinterpret_cast<const float4*>(p.q_proj + (int64_t)h * D * R);
    for (int i = t; i < D * R / 4; i += PREP_BLOCK) reinterpret_cast<float4*>(W)[i] = w4[i];
    const float4* c4 = reinterpret_cast<const float4*>(p.codebooks + (int64_t)h * S * C * sub);
    for (int i = t; i < S * C * sub / 4; i += PREP_BLOCK) {
      const float4 v = c4[i];
      float* row = cb + (4 * i / sub) * cbs + (4 * i) % sub;  // sub % 4 == 0: a float4 stays in its row
      row[0] = v.x;
      row[1] = v.y;
      row[2] = v.z;
      row[3] = v.w;
    }
  }
  const int64_t qbase = (int64_t)b * p.q_bs + (int64_t)h * p.q_hs + (int64_t)tq * p.q_ts;
  for (int d = t; d < D; d += PREP_BLOCK) qf[d] = load_elem(p.q, qbase + d, p.q_dtype);
  shist[t] = 0u;
  if (t < S) {
    kmin[t] = 0xFFFFFFFFu;
    kmax[t] = 0u;
  }
  if (t == 0) misc[2] = 0u;  // threshold bin 0 when fewer than k samples exist
  __syncthreads();
  // 1. q_low
  const float sc = p.scale[h];
  for (int r = t; r < R; r += PREP_BLOCK) {
    // sequential over d; unrolled so that each group's LDS reads are in
    // flight together instead of one dependent round trip per step
    float acc = 0.0f;
#pragma unroll 16
    for (int d = 0; d < D; ++d) acc = __builtin_fmaf(qf[d], W[d * R + r], acc);
    const float v = acc * sc;
    ql[r] = v;
    p.q_low[(int64_t)item * R + r] = v;
  }
  __syncthreads();
  // 2. table and per-subspace key bounds
  float* lut_out = p.lut + (int64_t)item * S * C;
  const bool wave_subspace = C % WAVE == 0;  // every wave's entries share a subspace
  for (int e = t; e < S * C; e += PREP_BLOCK) {
    const int s = e / C;
    const float* w = cb + e * cbs;
    const float* qs = ql + s * sub;
    float acc = 0.0f;
#pragma unroll 16
    for (int j = 0; j < sub; ++j) acc = __builtin_fmaf(qs[j], w[j], acc);
    lut_out[e] = acc;
    tab[e] = acc;
    uint32_t kn = f2key(acc), kx = kn;
    if (wave_subspace) {
      for (int off = 32; off > 0; off >>= 1) {
        kn = min(kn, (uint32_t)__shfl_xor((int)kn, off, WAVE));
        kx = max(kx, (uint32_t)__shfl_xor((int)kx, off, WAVE));
      }
      if (lane_id() == 0) {
        atomicMin(&kmin[s], kn);
        atomicMax(&kmax[s], kx);
      }
    } else {
      atomicMin(&kmin[s], kn);
      atomicMax(&kmax[s], kx);
    }
  }
  __syncthreads();
  // 3. bounds of any sum of one table entry per subspace (before the 1/sqrt(R)
  // scale), in the scan's summation order; every thread folds them itself
  float lo = 0.0f, hi = 0.0f;
  for (int s = 0; s < S; ++s) {
    lo = lo + key2f(kmin[s]);
    hi = hi + key2f(kmax[s]);
  }
  float t_lo = -INFINITY;
  // 4. sampled estimate of a sum below which the shortlist threshold almost
  // surely lies.  Only a performance hint: the wide summon stays exact
  // whatever it returns.
  if (sample && hi > lo) {
    const float inv_w = (float)SAMPLE_BINS / (hi - lo);
    auto count = [&](float acc) {
      int bin = (int)((acc - lo) * inv_w);
      bin = bin < 0 ? 0 : (bin >= SAMPLE_BINS ? SAMPLE_BINS - 1 : bin);
      atomicAdd(&shist[bin], 1u);
    };
    if (S == 4 && C <= 64 && D * R >= 4096 && S * C * cbs >= 4096) {
      // two pair tables (in the place of the map and the codebooks, both
      // read for the last time above): a sampled sum is P01 + P23, two reads
      float* p01 = W;
      float* p23 = cb;
      for (int e = t; e < 4096; e += PREP_BLOCK) {
        const int c0 = min(e & 63, C - 1), c1 = min(e >> 6, C - 1);
        p01[e] = tab[c0] + tab[C + c1];
        p23[e] = tab[2 * C + c0] + tab[3 * C + c1];
      }
      __syncthreads();
      const uint32_t* sc4 = reinterpret_cast<const uint32_t*>(scodes);
      const uint32_t cm = (uint32_t)(C - 1);
      for (int i0 = t; i0 < n_samples; i0 += 4 * PREP_BLOCK) {
        float acc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = i0 + u * PREP_BLOCK;
          const uint32_t w = i < n_samples ? sc4[i] : 0u;
          const uint32_t a0 = min(w & 0xFFu, cm), a1 = min((w >> 8) & 0xFFu, cm);
          const uint32_t a2 = min((w >> 16) & 0xFFu, cm), a3 = min(w >> 24, cm);
          acc[u] = p01[a0 | (a1 << 6)] + p23[a2 | (a3 << 6)];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (i0 + u * PREP_BLOCK < n_samples) count(acc[u]);
      }
    } else {
      // four samples in flight per thread, one table read per subspace
      for (int i0 = t; i0 < n_samples; i0 += 4 * PREP_BLOCK) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s = 0; s < S; ++s) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int i = min(i0 + u * PREP_BLOCK, n_samples - 1);
            const int c = min((int)scodes[i * S + s], C - 1);
            acc[u] = acc[u] + tab[s * C + c];
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (i0 + u * PREP_BLOCK < n_samples) count(acc[u]);
      }
    }
    __syncthreads();
    // thread j owns bin SAMPLE_BINS - 1 - j: a scan from the top finds the
    // bin holding the k-th largest
    const uint32_t mine = shist[SAMPLE_BINS - 1 - t];
    uint32_t total;
    const uint32_t above = block_excl_scan<PREP_BLOCK>(mine, scratch, &total);
    if (above < (uint32_t)k && above + mine >= (uint32_t)k) misc[2] = (uint32_t)(SAMPLE_BINS - 1 - t);
    __syncthreads();
    t_lo = lo + (float)misc[2] / inv_w;
  }
  if (t == 0) {
    float* rg = p.range + (int64_t)item * 4;
    rg[0] = lo;
    rg[1] = hi;
    rg[2] = t_lo;
    rg[3] = 0.0f;
  }
}

// Decode form: the body lives in query_decode.cuh (the code-class path runs
// it in one grid with its code counts).  Two and four subspaces run 1024
// threads per head: their table, sampled-sum and histogram phases are
// LDS-latency bound, and 16 waves hide what 4 cannot.
constexpr int QD_WIDE = 1024;

template <int S, int CMAX, int NT>
__global__ void __launch_bounds__(NT) query_decode_kernel(LutParams p) {
  query_decode_item<S, CMAX, NT>(p, (int)blockIdx.x);
}

// Many query tokens per head (prefill): one workgroup per MT consecutive
// tokens of one (sequence, head).  The head's map is staged in LDS once for
// all of them; thread e keeps codebook row e (SUB floats) in registers and
// forms table entry e for every token; q_low, the table and the bounds are
// the same fma chains and folds as in query_lut_kernel (no sampled floor:
// the per-item summon does not use one).
constexpr int MT = 32;          // tokens per workgroup
constexpr int MT_BLOCK = 512;

template <int SUB>
__global__ void __launch_bounds__(MT_BLOCK) query_lut_multi_kernel(LutParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int D = p.D, R = p.R, S = p.S, C = p.C;
  const int tiles = (p.Q + MT - 1) / MT;
  const int bh = blockIdx.x / tiles;
  const int t0 = (blockIdx.x - bh * tiles) * MT;
  const int h = bh % p.H;
  const int b = bh / p.H;
  const int nt = min(MT, p.Q - t0);
  float* W = (float*)lds;                    // [D * R]
  float* qf = W + D * R;                     // [MT][D]
  float* ql = qf + MT * D;                   // [MT][R]
  uint32_t* kmin = (uint32_t*)(ql + MT * R);  // [MT][S]
  uint32_t* kmax = kmin + MT * S;            // [MT][S]
  const int t = threadIdx.x;
  {
    const float4* w4 = reinterpret_cast<const float4*>(p.q_proj + (int64_t)h * D * R);
    for (int i = t; i < D * R / 4; i += MT_BLOCK) reinterpret_cast<float4*>(W)[i] = w4[i];
  }
  const int64_t qb = (int64_t)b * p.q_bs + (int64_t)h * p.q_hs;
  for (int e = t; e < nt * D; e += MT_BLOCK) {
    const int tt = e / D, d = e - tt * D;
    qf[e] = load_elem(p.q, qb + (int64_t)(t0 + tt) * p.q_ts + d, p.q_dtype);
  }
  for (int e = t; e < MT * S; e += MT_BLOCK) {
    kmin[e] = 0xFFFFFFFFu;
    kmax[e] = 0u;
  }
  __syncthreads();
  const int64_t item0 = ((int64_t)b * p.H + h) * p.Q + t0;
  const float sc = p.scale[h];
  for (int e = t; e < nt * R; e += MT_BLOCK) {
    const int tt = e / R, r = e - tt * R;
    const float* qq = qf + tt * D;
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc = __builtin_fmaf(qq[d], W[d * R + r], acc);
    const float v = acc * sc;
    ql[e] = v;
    p.q_low[(item0 + tt) * R + r] = v;
  }
  __syncthreads();
  const bool wave_subspace = C % WAVE == 0;
  for (int e = t; e < S * C; e += MT_BLOCK) {  // uniform trip count when S * C is a multiple of the block
    const int s = e / C;
    float w[SUB];
    const float4* row = reinterpret_cast<const float4*>(p.codebooks + ((int64_t)h * S * C + e) * SUB);
#pragma unroll
    for (int j = 0; j < SUB / 4; ++j) {
      const float4 v = row[j];
      w[4 * j] = v.x, w[4 * j + 1] = v.y, w[4 * j + 2] = v.z, w[4 * j + 3] = v.w;
    }
    for (int tt = 0; tt < nt; ++tt) {
      const float* qs = ql + tt * R + s * SUB;
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < SUB; ++j) acc = __builtin_fmaf(qs[j], w[j], acc);
      p.lut[(item0 + tt) * S * C + e] = acc;
      uint32_t kn = f2key(acc), kx = kn;
      if (wave_subspace) {
        for (int off = 32; off > 0; off >>= 1) {
          kn = min(kn, (uint32_t)__shfl_xor((int)kn, off, WAVE));
          kx = max(kx, (uint32_t)__shfl_xor((int)kx, off, WAVE));
        }
        if (lane_id() == 0) {
          atomicMin(&kmin[tt * S + s], kn);
          atomicMax(&kmax[tt * S + s], kx);
        }
      } else {
        atomicMin(&kmin[tt * S + s], kn);
        atomicMax(&kmax[tt * S + s], kx);
      }
    }
  }
  __syncthreads();
  if (t < nt) {
    float lo = 0.0f, hi = 0.0f;
    for (int s = 0; s < S; ++s) {
      lo = lo + key2f(kmin[t * S + s]);
      hi = hi + key2f(kmax[t * S + s]);
    }
    float* rg = p.range + (item0 + t) * 4;
    rg[0] = lo;
    rg[1] = hi;
    rg[2] = -INFINITY;
    rg[3] = 0.0f;
  }
}

template <int SUB>
int launch_lut_multi(const LutParams& p, int64_t blocks, size_t lds, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((query_lut_multi_kernel<SUB>), sva::kMaxLds, "hipFuncSetAttribute(query_lut_multi_kernel)");
  hipLaunchKernelGGL(query_lut_multi_kernel<SUB>, dim3((unsigned)blocks), dim3(MT_BLOCK), lds, stream, p);
  SVA_CHECK_LAUNCH("query_lut_multi_kernel");
  return SVA_OK;
}

// The multi form on fp32 MFMA.  v_mfma_f32_16x16x4f32 adds its four k
// products to the running sum in k order with the rounding of the fma chain,
// so q_low = (q . W) * scale and the table row q_low[s] . codeword are the
// same values as query_lut_multi_kernel's (sequential fma chains from 0).
// Operand layout of the 16x16x4 form: lane l supplies A[l % 16][k0 + l / 16]
// and B[k0 + l / 16][l % 16] and receives D[4 * (l / 16) + i][l % 16] in
// element i.  A tile is 16 tokens x 16 ranks (q_low) or 16 tokens x 16
// codewords of one subspace (the table); a wave takes every eighth tile,
// keeps a codeword tile's B operand in registers for both token tiles, and
// folds its bounds over the tile's 16 codewords in DPP rows before one LDS
// atomic per token.  Rows of the token-major staging are padded by a float
// so the 16 rows an A operand reads fall in 16 banks.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int MF_BLOCK = 512;

__host__ __device__ inline size_t lut_mfma_lds_bytes(int64_t D, int64_t R, int64_t S) {
  return sizeof(float) * (size_t)(D * R + MT * (D + 1) + MT * (R + 1)) + sizeof(uint32_t) * (size_t)(2 * MT * S);
}

template <int SUB>
__global__ void __launch_bounds__(MF_BLOCK) query_lut_mfma_kernel(LutParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int D = p.D, R = p.R, S = p.S, C = p.C;
  const int DP = D + 1, RP = R + 1;
  const int tiles = (p.Q + MT - 1) / MT;
  const int bh = blockIdx.x / tiles;
  const int t0 = (blockIdx.x - bh * tiles) * MT;
  const int h = bh % p.H;
  const int b = bh / p.H;
  const int nt = min(MT, p.Q - t0);
  float* W = (float*)lds;                    // [D][R]
  float* qf = W + D * R;                     // [MT][D + 1]
  float* ql = qf + MT * DP;                  // [MT][R + 1]
  uint32_t* kmin = (uint32_t*)(ql + MT * RP);  // [MT][S]
  uint32_t* kmax = kmin + MT * S;            // [MT][S]
  const int t = threadIdx.x;
  const int lane = lane_id(), wid = t / WAVE, li = lane & 15, lk = lane >> 4;
  {
    const float4* w4 = reinterpret_cast<const float4*>(p.q_proj + (int64_t)h * D * R);
    for (int i = t; i < D * R / 4; i += MF_BLOCK) reinterpret_cast<float4*>(W)[i] = w4[i];
  }
  const int64_t qb = (int64_t)b * p.q_bs + (int64_t)h * p.q_hs;
  for (int e = t; e < MT * D; e += MF_BLOCK) {
    const int tt = e / D, d = e - tt * D;
    qf[tt * DP + d] = tt < nt ? load_elem(p.q, qb + (int64_t)(t0 + tt) * p.q_ts + d, p.q_dtype) : 0.0f;
  }
  for (int e = t; e < MT * S; e += MF_BLOCK) {
    kmin[e] = 0xFFFFFFFFu;
    kmax[e] = 0u;
  }
  __syncthreads();
  const int64_t item0 = ((int64_t)b * p.H + h) * p.Q + t0;
  const float sc = p.scale[h];
  // q_low tiles: (token tile, rank tile), D / 4 steps each
  for (int tile = wid; tile < (MT / 16) * (R / 16); tile += MF_BLOCK / WAVE) {
    const int tt = tile / (R / 16), r0 = (tile - tt * (R / 16)) * 16;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < D; k0 += 4)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[(tt * 16 + li) * DP + k0 + lk], W[(k0 + lk) * R + r0 + li], acc,
                                                 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = tt * 16 + 4 * lk + i;
      const float v = acc[i] * sc;
      ql[row * RP + r0 + li] = v;
      if (row < nt) p.q_low[(item0 + row) * R + r0 + li] = v;
    }
  }
  __syncthreads();
  // table tiles: (subspace, codeword tile) x both token tiles, SUB / 4 steps
  const float* cbh = p.codebooks + (int64_t)h * S * C * SUB;
  for (int tile = wid; tile < S * (C / 16); tile += MF_BLOCK / WAVE) {
    const int s = tile / (C / 16), c0 = (tile - s * (C / 16)) * 16;
    float bv[SUB / 4];
#pragma unroll
    for (int k = 0; k < SUB / 4; ++k) bv[k] = cbh[((int64_t)s * C + c0 + li) * SUB + 4 * k + lk];
#pragma unroll
    for (int tt = 0; tt < MT / 16; ++tt) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k = 0; k < SUB / 4; ++k)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ql[(tt * 16 + li) * RP + s * SUB + 4 * k + lk], bv[k], acc, 0, 0,
                                                   0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = tt * 16 + 4 * lk + i;
        if (row < nt) p.lut[(item0 + row) * S * C + s * C + c0 + li] = acc[i];
        // bounds over the tile's 16 codewords (one DPP row), then one atomic per token
        uint32_t kn = f2key(acc[i]), kx = kn;
        kn = min(kn, row_shr_keep<1>(kn));
        kx = max(kx, row_shr_keep<1>(kx));
        kn = min(kn, row_shr_keep<2>(kn));
        kx = max(kx, row_shr_keep<2>(kx));
        kn = min(kn, row_shr_keep<4>(kn));
        kx = max(kx, row_shr_keep<4>(kx));
        kn = min(kn, row_shr_keep<8>(kn));
        kx = max(kx, row_shr_keep<8>(kx));
        if (li == 15 && row < nt) {
          atomicMin(&kmin[row * S + s], kn);
          atomicMax(&kmax[row * S + s], kx);
        }
      }
    }
  }
  __syncthreads();
  if (t < nt) {
    float lo = 0.0f, hi = 0.0f;
    for (int s = 0; s < S; ++s) {
      lo = lo + key2f(kmin[t * S + s]);
      hi = hi + key2f(kmax[t * S + s]);
    }
    float* rg = p.range + (item0 + t) * 4;
    rg[0] = lo;
    rg[1] = hi;
    rg[2] = -INFINITY;
    rg[3] = 0.0f;
  }
}

template <int SUB>
int launch_lut_mfma(const LutParams& p, int64_t blocks, size_t lds, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((query_lut_mfma_kernel<SUB>), sva::kMaxLds, "hipFuncSetAttribute(query_lut_mfma_kernel)");
  hipLaunchKernelGGL(query_lut_mfma_kernel<SUB>, dim3((unsigned)blocks), dim3(MF_BLOCK), lds, stream, p);
  SVA_CHECK_LAUNCH("query_lut_mfma_kernel");
  return SVA_OK;
}

constexpr int SCORE_BLOCK = 256;

__global__ void __launch_bounds__(SCORE_BLOCK)
    pq_scores_kernel(const float* __restrict__ lut, const void* __restrict__ codes, int ctype, int64_t code_hs,
                     const int64_t* __restrict__ offs, const int64_t* __restrict__ lens, int H, int Q, int64_t N,
                     int S, int C, float sqrt_r, float* __restrict__ scores) {
#pragma clang fp contract(off)
  extern __shared__ float tab[];
  const int item = blockIdx.y;
  const int h = (item / Q) % H;
  const int b = item / (Q * H);
  const int64_t len = lens ? lens[b] : N;
  const int64_t off = offs ? offs[b] : 0;
  const float* src = lut + (int64_t)item * S * C;
  for (int e = threadIdx.x; e < S * C; e += SCORE_BLOCK) tab[e] = src[e];
  __syncthreads();
  const int64_t n = (int64_t)blockIdx.x * SCORE_BLOCK + threadIdx.x;
  if (n >= len) return;
  const int64_t row = (int64_t)h * code_hs + (off + n) * S;
  float acc = 0.0f;
  for (int s = 0; s < S; ++s) {
    int64_t c = load_code(codes, row + s, ctype);
    c = c < 0 ? 0 : (c >= C ? C - 1 : c);
    acc = acc + tab[s * C + c];
  }
  scores[(int64_t)item * N + n] = acc / sqrt_r;
}

size_t lut_lds_bytes(int64_t D, int64_t R, int64_t S, int64_t C, int sample_blocks) {
  return sizeof(float) * (size_t)(D * R + S * C * (R / S + 1) + D + R + S * C) +
         sizeof(uint32_t) * (size_t)(2 * S + SAMPLE_BINS + 4 + PREP_BLOCK / 64 + 1) +
         (size_t)sample_blocks * SAMPLE_KEYS * (size_t)S;
}

}  // namespace

namespace sva {

int query_lut_setup(const void* q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride, int64_t q_tok_stride,
                    int64_t n_seq, int64_t H, int64_t Q, int64_t D, int64_t R, int64_t S, int64_t C,
                    const float* q_proj, const float* scale, const float* codebooks, const void* codes, int code_type,
                    int64_t code_head_stride, int64_t n_keys, int64_t shortlist, float* q_low, float* lut,
                    float* score_range, QueryLaunch* out) {
  SVA_REQUIRE(q && q_proj && scale && codebooks && q_low && lut && score_range, "sva_query_lut: null pointer");
  SVA_REQUIRE(n_seq > 0 && H > 0 && Q > 0, "sva_query_lut: empty query batch");
  SVA_REQUIRE(D > 0 && D <= 512 && R > 0 && R <= 512, "sva_query_lut: head_dim %lld / rank %lld out of range",
              (long long)D, (long long)R);
  SVA_REQUIRE(S > 0 && S <= 64 && R % S == 0, "sva_query_lut: rank %lld not divisible by subspaces %lld",
              (long long)R, (long long)S);
  SVA_REQUIRE(C > 0, "sva_query_lut: codewords %lld out of range", (long long)C);
  SVA_REQUIRE((D * R) % 4 == 0 && (S * C * (R / S)) % 4 == 0 && ((uintptr_t)q_proj & 15u) == 0 &&
                  ((uintptr_t)codebooks & 15u) == 0,
              "sva_query_lut: q_proj / codebooks must be 16-byte aligned fp32");
  SVA_REQUIRE(q_dtype >= 0 && q_dtype <= 2, "sva_query_lut: bad q dtype");
  SVA_REQUIRE(codes == nullptr || (code_type >= 0 && code_type <= 3 && n_keys >= 0 && shortlist > 0),
              "sva_query_lut: bad sampling arguments");
  // the threshold estimate serves the single-query uint8 scan; otherwise skipped
  // (one subspace of at most 256 codewords selects by code class instead)
  bool sample = codes != nullptr && n_seq == 1 && Q == 1 && code_type == 0 && S <= SAMPLE_MAX_S &&
                !sva::class_shape(S, C, shortlist);
  int blocks = sample ? sva::sample_blocks(n_keys, S) : 0;
  // fewer sampled blocks when the head's weights leave less LDS
  while (blocks > SAMPLE_MIN_BLOCKS && lut_lds_bytes(D, R, S, C, blocks) > (size_t)sva::kMaxLds) blocks /= 2;
  const int sample_k = sample ? sva::sample_floor_rank(shortlist, n_keys, blocks * SAMPLE_KEYS) : 0;
  sample = sample && sample_k > 0;
  if (!sample) blocks = 0;
  const size_t lds = lut_lds_bytes(D, R, S, C, blocks);
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_query_lut: head weights of %zu bytes exceed LDS", lds);
  const int64_t items = n_seq * H * Q;
  SVA_REQUIRE(items < (1ll << 31), "sva_query_lut: too many query items");
  LutParams& p = out->p;
  p.q = q;
  p.q_dtype = q_dtype;
  p.q_bs = q_seq_stride;
  p.q_hs = q_head_stride;
  p.q_ts = q_tok_stride;
  p.H = (int)H;
  p.Q = (int)Q;
  p.D = (int)D;
  p.R = (int)R;
  p.S = (int)S;
  p.C = (int)C;
  p.q_proj = q_proj;
  p.scale = scale;
  p.codebooks = codebooks;
  p.q_low = q_low;
  p.lut = lut;
  p.range = score_range;
  p.codes = sample ? codes : nullptr;
  p.code_hs = code_head_stride;
  p.n_keys = n_keys;
  p.sample_blocks = blocks;
  p.sample_k = sample_k;
  out->form = QUERY_GENERAL;
  out->blocks = items;
  out->lds = lds;
  // many tokens per head: the head's weights are staged once per MT tokens
  const int64_t sub = R / S;
  const size_t mlds = sizeof(float) * (size_t)(D * R + MT * D + MT * R) + sizeof(uint32_t) * (size_t)(2 * MT * S);
  if (Q >= 8 && !sample && (sub == 16 || sub == 32 || sub == 64) && mlds <= (size_t)sva::kMaxLds) {
    out->form = sub == 16 ? QUERY_MULTI16 : (sub == 32 ? QUERY_MULTI32 : QUERY_MULTI64);
    out->blocks = n_seq * H * ((Q + MT - 1) / MT);
    out->lds = mlds;
    const size_t flds = lut_mfma_lds_bytes(D, R, S);
    if (D % 4 == 0 && R % 16 == 0 && C % 16 == 0 && flds <= (size_t)sva::kMaxLds) {
      out->form = sub == 16 ? QUERY_MFMA16 : (sub == 32 ? QUERY_MFMA32 : QUERY_MFMA64);
      out->lds = flds;
    }
    return SVA_OK;
  }
  // one token of one sequence at D = R = 64: the decode form
  const bool aligned = ((uintptr_t)q_proj & 15u) == 0 && ((uintptr_t)codebooks & 15u) == 0 &&
                       (!sample || (((uintptr_t)codes & 15u) == 0 && code_head_stride % 16 == 0));
  const int64_t word_room = S == 4   ? (int64_t)QD_WIDE * qd_words<4, QD_WIDE>()
                            : S == 2 ? (int64_t)QD_WIDE * qd_words<2, QD_WIDE>()
                                     : (int64_t)QD * qd_words<1>();  // sampled 16-byte words the form holds
  if (n_seq == 1 && Q == 1 && D == 64 && R == 64 && aligned && (!sample || blocks * SAMPLE_KEYS * S <= 16 * word_room)) {
    const int form = S == 4 && C <= 64 ? QUERY_DECODE_4_64
                     : S == 2 && C <= 256 ? QUERY_DECODE_2_256
                     : S == 1 && C <= 256 ? QUERY_DECODE_1_256
                                          : QUERY_GENERAL;
    if (form != QUERY_GENERAL) {
      out->form = form;
      out->blocks = H;
      out->lds = 0;
    }
  }
  return SVA_OK;
}

int query_lut_launch(const QueryLaunch& ql, hipStream_t st) {
  const LutParams& p = ql.p;
  switch (ql.form) {
    case QUERY_MULTI16: return launch_lut_multi<16>(p, ql.blocks, ql.lds, st);
    case QUERY_MULTI32: return launch_lut_multi<32>(p, ql.blocks, ql.lds, st);
    case QUERY_MULTI64: return launch_lut_multi<64>(p, ql.blocks, ql.lds, st);
    case QUERY_MFMA16: return launch_lut_mfma<16>(p, ql.blocks, ql.lds, st);
    case QUERY_MFMA32: return launch_lut_mfma<32>(p, ql.blocks, ql.lds, st);
    case QUERY_MFMA64: return launch_lut_mfma<64>(p, ql.blocks, ql.lds, st);
    case QUERY_DECODE_4_64:
      hipLaunchKernelGGL((query_decode_kernel<4, 64, QD_WIDE>), dim3((unsigned)ql.blocks), dim3(QD_WIDE), 0, st, p);
      SVA_CHECK_LAUNCH("query_decode_kernel");
      return SVA_OK;
    case QUERY_DECODE_2_256:
      hipLaunchKernelGGL((query_decode_kernel<2, 256, QD_WIDE>), dim3((unsigned)ql.blocks), dim3(QD_WIDE), 0, st, p);
      SVA_CHECK_LAUNCH("query_decode_kernel");
      return SVA_OK;
    case QUERY_DECODE_1_256:
      hipLaunchKernelGGL((query_decode_kernel<1, 256, QD>), dim3((unsigned)ql.blocks), dim3(QD), 0, st, p);
      SVA_CHECK_LAUNCH("query_decode_kernel");
      return SVA_OK;
    default:
      SVA_SET_MAX_LDS_ONCE(query_lut_kernel, sva::kMaxLds, "hipFuncSetAttribute(query_lut_kernel)");
      hipLaunchKernelGGL(query_lut_kernel, dim3((unsigned)ql.blocks), dim3(PREP_BLOCK), ql.lds, st, p);
      SVA_CHECK_LAUNCH("query_lut_kernel");
      return SVA_OK;
  }
}

}  // namespace sva

extern "C" int sva_query_lut(const void* q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride,
                             int64_t q_tok_stride, int64_t n_seq, int64_t H, int64_t Q, int64_t D, int64_t R,
                             int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                             const void* codes, int code_type, int64_t code_head_stride, int64_t n_keys,
                             int64_t shortlist, float* q_low, float* lut, float* score_range, void* stream) {
  sva::clear_error();
  sva::QueryLaunch ql;
  const int rc = sva::query_lut_setup(q, q_dtype, q_seq_stride, q_head_stride, q_tok_stride, n_seq, H, Q, D, R, S, C,
                                      q_proj, scale, codebooks, codes, code_type, code_head_stride, n_keys, shortlist,
                                      q_low, lut, score_range, &ql);
  if (rc != SVA_OK) return rc;
  return sva::query_lut_launch(ql, (hipStream_t)stream);
}

extern "C" int sva_pq_scores(const float* lut, const void* codes, int code_type, int64_t code_head_stride,
                             const int64_t* seq_offsets, const int64_t* seq_lens, int64_t n_seq, int64_t H, int64_t Q,
                             int64_t n_keys, int64_t R, int64_t S, int64_t C, float* scores, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(lut && codes && scores, "sva_pq_scores: null pointer");
  SVA_REQUIRE((seq_offsets == nullptr) == (seq_lens == nullptr), "sva_pq_scores: offsets and lengths go together");
  SVA_REQUIRE(n_seq > 0 && H > 0 && Q > 0 && n_keys >= 0, "sva_pq_scores: bad sizes");
  SVA_REQUIRE(S > 0 && R % S == 0 && C > 0 && S * C <= 16384, "sva_pq_scores: bad PQ layout %lldx%lld",
              (long long)S, (long long)C);
  SVA_REQUIRE(code_type >= 0 && code_type <= 3, "sva_pq_scores: bad code type");
  if (n_keys == 0) return SVA_OK;
  const int64_t items = n_seq * H * Q;
  SVA_REQUIRE(items <= 65535, "sva_pq_scores: at most 65535 query items per call");
  const int64_t blocks = (n_keys + SCORE_BLOCK - 1) / SCORE_BLOCK;
  SVA_REQUIRE(blocks < (1ll << 31), "sva_pq_scores: too many keys");
  const float sqrt_r = (float)sqrt((double)R);
  const size_t lds = sizeof(float) * (size_t)(S * C);
  hipLaunchKernelGGL(pq_scores_kernel, dim3((unsigned)blocks, (unsigned)items), dim3(SCORE_BLOCK), lds,
                     (hipStream_t)stream, lut, codes, code_type, code_head_stride, seq_offsets, seq_lens, (int)H, (int)Q,
                     n_keys, (int)S, (int)C, sqrt_r, scores);
  SVA_CHECK_LAUNCH("pq_scores_kernel");
  return SVA_OK;
}
