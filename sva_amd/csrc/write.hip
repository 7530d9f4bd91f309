// Write path: low-rank keys and product-quantized codes of cache rows
// (sva/llama.py:578-624, the catalog; sva/ops.py:10-47, assignment).
//
//   k_low[h][n][r] = sum_d K[g(h)][n][d] * k_proj[h][d][r]      (sva/llama.py:615)
//       a sequential fma chain over d, as torch's many-row einsum rounds it;
//       g(h) = h / (H / G) (the reference's repeat_kv expansion).
//   codes[h][n][s] = argmin_c (|x|^2 - 2 x.c + |c|^2), first index on ties,
//       x = k_low[h][n][s*sub:(s+1)*sub]                         (sva/ops.py:19-20)
//       |x|^2 and |c|^2 in torch's sum order, x.c a sequential fma chain.
//
// One workgroup per (64 rows, head).  The head's map and the rows are staged
// in LDS; each thread accumulates a 4 x 4 block of k_low.  For each subspace
// the codebook is staged (rows padded against bank conflicts) and the 4 lanes
// of a row split the centroids, then merge (distance, index) pairs keeping
// the lower index on equal distances.  NaN distances never win (the CPU
// oracle's rule).
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"
#include "write_few.cuh"

using namespace sva;

namespace {

constexpr int WT = 256;  // threads per workgroup
constexpr int KT = 64;   // rows per workgroup
constexpr int CB_PAD = 4;


// SUB: compile-time subspace width (0: runtime, x read from LDS).
template <int SUB>
__global__ void __launch_bounds__(WT) write_encode_kernel(WriteParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int D = p.D, R = p.R, S = p.S, C = p.C;
  const int sub = SUB > 0 ? SUB : R / S;
  const int h = blockIdx.y;
  const int g = h / (p.H / p.G);
  const int64_t n0 = p.row0 + (int64_t)blockIdx.x * KT;
  const int nk = (int)min((int64_t)KT, p.row0 + p.n_rows - n0);
  float* W = (float*)lds;                  // [D][R]
  float* Kt = W + D * R;                   // [KT][D + 1]
  float* Xl = Kt + KT * (D + 1);           // [KT][R + 1] k_low of the tile
  float* cb = Xl + KT * (R + 1);           // [C][sub + CB_PAD], 16-byte aligned rows
  float* cn = cb + C * (sub + CB_PAD);     // [C]
  float* xx = cn + C;                      // [KT]

  {
    const float4* w4 = reinterpret_cast<const float4*>(p.k_proj + (int64_t)h * D * R);
    for (int i = threadIdx.x; i < D * R / 4; i += WT) reinterpret_cast<float4*>(W)[i] = w4[i];
    const int64_t kb = (int64_t)g * p.kv_hs;
    for (int i = threadIdx.x; i < KT * D; i += WT) {
      const int k = i / D, d = i - k * D;
      Kt[k * (D + 1) + d] = k < nk ? load_elem(p.keys, kb + (n0 + k) * p.kv_rs + d, p.kv_dtype) : 0.0f;
    }
  }
  __syncthreads();
  // projection: 4 rows x 4 ranks per thread, fma chain over d
  float* klow = p.k_low + (int64_t)h * p.klow_hs;
  for (int blk = threadIdx.x; blk < (KT / 4) * (R / 4); blk += WT) {
    const int kb = blk / (R / 4), rb = blk - kb * (R / 4);
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int d = 0; d < D; ++d) {
      const float4 w = *reinterpret_cast<const float4*>(W + d * R + rb * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float kv = Kt[(kb * 4 + i) * (D + 1) + d];
        acc[i][0] = __builtin_fmaf(kv, w.x, acc[i][0]);
        acc[i][1] = __builtin_fmaf(kv, w.y, acc[i][1]);
        acc[i][2] = __builtin_fmaf(kv, w.z, acc[i][2]);
        acc[i][3] = __builtin_fmaf(kv, w.w, acc[i][3]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = kb * 4 + i;
#pragma unroll
      for (int j = 0; j < 4; ++j) Xl[k * (R + 1) + rb * 4 + j] = acc[i][j];
      if (k < nk)
        *reinterpret_cast<float4*>(klow + (n0 + k) * R + rb * 4) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    }
  }
  if (p.codes == nullptr) return;  // projection only
  // assignment, one subspace at a time
  const int k = threadIdx.x >> 2;  // row of this lane group
  const int qt = threadIdx.x & 3;
  for (int s = 0; s < S; ++s) {
    __syncthreads();  // Xl complete / previous subspace done with cb
    const float* src = p.codebooks + ((int64_t)h * S + s) * C * sub;
    for (int i = threadIdx.x; i < C * sub / 4; i += WT) {
      const int c = (4 * i) / sub, j = 4 * i - c * sub;
      *reinterpret_cast<float4*>(cb + c * (sub + CB_PAD) + j) = reinterpret_cast<const float4*>(src)[i];
    }
    __syncthreads();
    for (int c = threadIdx.x; c < C; c += WT) cn[c] = torch_order_dot(cb + c * (sub + CB_PAD), cb + c * (sub + CB_PAD), sub);
    for (int r = threadIdx.x; r < KT; r += WT) xx[r] = torch_order_dot(Xl + r * (R + 1) + s * sub, Xl + r * (R + 1) + s * sub, sub);
    __syncthreads();
    const float* xr = Xl + k * (R + 1) + s * sub;
    float xv[SUB > 0 ? SUB : 1];
    if (SUB > 0) {
#pragma unroll
      for (int j = 0; j < (SUB > 0 ? SUB : 1); ++j) xv[j] = xr[j];
    }
    const float xxk = xx[k];
    float best = INFINITY;
    int arg = 0;
    for (int c = qt; c < C; c += 4) {
      const float* cr = cb + c * (sub + CB_PAD);
      float xc = 0.0f;
      if (SUB > 0) {
#pragma unroll
        for (int j = 0; j < (SUB > 0 ? SUB : 1); j += 4) {
          const float4 v = *reinterpret_cast<const float4*>(cr + j);
          xc = __builtin_fmaf(xv[j], v.x, xc);
          xc = __builtin_fmaf(xv[j + 1], v.y, xc);
          xc = __builtin_fmaf(xv[j + 2], v.z, xc);
          xc = __builtin_fmaf(xv[j + 3], v.w, xc);
        }
      } else {
        for (int j = 0; j < sub; ++j) xc = __builtin_fmaf(xr[j], cr[j], xc);
      }
      const float dist = (xxk - 2.0f * xc) + cn[c];
      if (dist < best) {
        best = dist;
        arg = c;
      }
    }
#pragma unroll
    for (int o = 1; o < 4; o <<= 1) {
      const float ob = __shfl_xor(best, o, 4);
      const int oa = __shfl_xor(arg, o, 4);
      if (ob < best || (ob == best && oa < arg)) {
        best = ob;
        arg = oa;
      }
    }
    if (qt == 0 && k < nk) store_code(p.codes, (int64_t)h * p.code_hs + (n0 + k) * S + s, p.ctype, arg);
  }
}

// MFMA variant (R, C multiples of 16; D, sub multiples of 4): the projection
// and the x.c distance products on v_mfma_f32_16x16x4f32, which accumulates
// its four k products per step into the running sum in k order, the same
// rounding as the fma chain above.  Operand layout of the 16x16x4 form: lane
// l supplies A[l % 16][k0 + l / 16] and B[k0 + l / 16][l % 16] and receives
// D[4 * (l / 16) + i][l % 16] in element i.  Wave w owns rows 16w..16w+15 of
// the tile.
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(WT) write_encode_mfma_kernel(WriteParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int D = p.D, R = p.R, S = p.S, C = p.C;
  const int sub = R / S;
  const int h = blockIdx.y;
  const int g = h / (p.H / p.G);
  const int64_t n0 = p.row0 + (int64_t)blockIdx.x * KT;
  const int nk = (int)min((int64_t)KT, p.row0 + p.n_rows - n0);
  float* W = (float*)lds;                  // [D][R]
  float* Kt = W + D * R;                   // [KT][D + 1]
  float* Xl = Kt + KT * (D + 1);           // [KT][R + 1]
  float* cb = Xl + KT * (R + 1);           // [C][sub + CB_PAD]
  float* cn = cb + C * (sub + CB_PAD);     // [C]
  float* xx = cn + C;                      // [KT]
  {
    const float4* w4 = reinterpret_cast<const float4*>(p.k_proj + (int64_t)h * D * R);
    for (int i = threadIdx.x; i < D * R / 4; i += WT) reinterpret_cast<float4*>(W)[i] = w4[i];
    const int64_t kb = (int64_t)g * p.kv_hs;
    for (int i = threadIdx.x; i < KT * D; i += WT) {
      const int k = i / D, d = i - k * D;
      Kt[k * (D + 1) + d] = k < nk ? load_elem(p.keys, kb + (n0 + k) * p.kv_rs + d, p.kv_dtype) : 0.0f;
    }
  }
  __syncthreads();
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lr = l & 15, lk = l >> 4;
  const int row0 = 16 * wid;
  float* klow = p.k_low + (int64_t)h * p.klow_hs;
  // projection: R / 16 output blocks per wave
  for (int cb0 = 0; cb0 < R; cb0 += 64) {
    f32x4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int nblk = min(4, (R - cb0) / 16);
    for (int k0 = 0; k0 < D; k0 += 4) {
      const float a = Kt[(row0 + lr) * (D + 1) + k0 + lk];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (c < nblk) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, W[(k0 + lk) * R + cb0 + 16 * c + lr], acc[c], 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c < nblk) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + 4 * lk + i, col = cb0 + 16 * c + lr;
          Xl[row * (R + 1) + col] = acc[c][i];
          if (row < nk) klow[(n0 + row) * R + col] = acc[c][i];
        }
      }
    }
  }
  if (p.codes == nullptr) return;
  for (int s = 0; s < S; ++s) {
    __syncthreads();
    const float* src = p.codebooks + ((int64_t)h * S + s) * C * sub;
    for (int i = threadIdx.x; i < C * sub / 4; i += WT) {
      const int c = (4 * i) / sub, j = 4 * i - c * sub;
      *reinterpret_cast<float4*>(cb + c * (sub + CB_PAD) + j) = reinterpret_cast<const float4*>(src)[i];
    }
    __syncthreads();
    for (int c = threadIdx.x; c < C; c += WT) cn[c] = torch_order_dot(cb + c * (sub + CB_PAD), cb + c * (sub + CB_PAD), sub);
    for (int r = threadIdx.x; r < KT; r += WT) xx[r] = torch_order_dot(Xl + r * (R + 1) + s * sub, Xl + r * (R + 1) + s * sub, sub);
    __syncthreads();
    // this lane's 4 rows: running best over its centroids (l % 16 of each block)
    float best[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
    int arg[4] = {0, 0, 0, 0};
    float xxr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xxr[i] = xx[row0 + 4 * lk + i];
    for (int c0 = 0; c0 < C; c0 += 16) {
      f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int k0 = 0; k0 < sub; k0 += 4) {
        const float a = Xl[(row0 + lr) * (R + 1) + s * sub + k0 + lk];
        const float b = cb[(c0 + lr) * (sub + CB_PAD) + k0 + lk];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
      }
      const int c = c0 + lr;
      const float cnc = cn[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float dist = (xxr[i] - 2.0f * acc[i]) + cnc;
        if (dist < best[i]) {
          best[i] = dist;
          arg[i] = c;
        }
      }
    }
    // merge the 16 lanes of each row group: smaller distance, then lower index
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float ob = __shfl_xor(best[i], o, 16);
        const int oa = __shfl_xor(arg[i], o, 16);
        if (ob < best[i] || (ob == best[i] && oa < arg[i])) {
          best[i] = ob;
          arg[i] = oa;
        }
      }
      const int row = row0 + 4 * lk + i;
      if (lr == 0 && row < nk) store_code(p.codes, (int64_t)h * p.code_hs + (n0 + row) * S + s, p.ctype, arg[i]);
    }
  }
}

// Persistent MFMA variant for the common shapes (D in {64, 128}, R = 64 with
// 2 x 256 or 4 x 64 codes, keys rows 16-byte aligned).  Each workgroup serves
// one head and walks that head's 64-row tiles with stride gridDim.x, so the
// head's map, codebooks and centroid norms are loaded once, into registers.
// The map / codebook is the MFMA A operand and the rows the B operand, so a
// lane's four accumulator elements are four columns (centroids) of one row:
//   projection: wave w owns columns 16(w + 4m) .. +15 of k_low;
//   distances:  wave w owns centroids 16(w + 4m) .. +15 of every subspace.
// Products are commutative, so the k-order rounding equals the kernel above.
// The next tile's key rows are loaded into registers while this tile computes.
template <int D, int S, int SUB, int C>
__global__ void __launch_bounds__(WT, 2) write_encode_persistent_kernel(WriteParams p) {
#pragma clang fp contract(off)
  constexpr int R = S * SUB;
  constexpr int NCOLW = R / 64;  // projection column blocks per wave
  constexpr int NCBW = C / 64;   // centroid blocks per wave and subspace
  constexpr int KS = D + 4;      // Kt row stride (floats; 16-byte rows, no bank conflicts)
  constexpr int XS = R + 4;      // Xl row stride
  constexpr int KJ = D / 4, XJ = SUB / 4;
  constexpr int MAXCH = D / 16;  // 16-byte key chunks per thread and tile (fp32 keys)
  static_assert(R % 64 == 0 && C % 64 == 0 && SUB % 4 == 0 && D % 16 == 0 && (D & (D - 1)) == 0, "shape");
  static_assert(KT * S <= WT && S * C <= KT * XS, "tile");
  __shared__ __align__(16) float Kt[KT * KS];
  __shared__ __align__(16) float Xl[KT * XS];
  __shared__ float xxl[S * KT];
  __shared__ __align__(8) float2 mb[S * KT * 4];
  const int h = blockIdx.y;
  const int g = h / (p.H / p.G);
  const int wid = threadIdx.x / WAVE;
  const int l = lane_id();
  const int lr = l & 15, lk = l >> 4;
  const int64_t row_end = p.row0 + p.n_rows;
  const int64_t n_tiles = (p.n_rows + KT - 1) / KT;
  const bool want_codes = p.codes != nullptr;

  float wreg[NCOLW][KJ];
  {
    const float* W = p.k_proj + (int64_t)h * D * R;
#pragma unroll
    for (int m = 0; m < NCOLW; ++m)
#pragma unroll
      for (int j = 0; j < KJ; ++j) wreg[m][j] = W[(4 * j + lk) * R + 16 * (wid + 4 * m) + lr];
  }
  float cbreg[S][NCBW][XJ];
  float cnreg[S][NCBW][4];
  const float* CB = p.codebooks + (int64_t)h * S * C * SUB;
  if (want_codes) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int m = 0; m < NCBW; ++m)
#pragma unroll
        for (int j = 0; j < XJ; ++j) cbreg[s][m][j] = CB[((int64_t)s * C + 16 * (wid + 4 * m) + lr) * SUB + 4 * j + lk];
    for (int i = threadIdx.x; i < S * C; i += WT) Xl[i] = torch_order_dot(CB + (int64_t)i * SUB, CB + (int64_t)i * SUB, SUB);
    __syncthreads();
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int m = 0; m < NCBW; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) cnreg[s][m][i] = Xl[s * C + 16 * (wid + 4 * m) + 4 * lk + i];
    __syncthreads();
  }

  // key rows: 16-byte chunks, chunk q of a tile = row q >> cpr_shift
  const bool f32 = p.kv_dtype == F32;
  const int es = f32 ? 4 : 2;
  const int cpr_shift = __builtin_ctz(D) - (f32 ? 2 : 3);
  const int nch = (KT << cpr_shift) / WT;
  const unsigned char* kbytes = (const unsigned char*)p.keys;
  uint4 pre[MAXCH];
  auto load_tile = [&](int64_t t) {
    const int64_t n0 = p.row0 + t * KT;
#pragma unroll
    for (int c = 0; c < MAXCH; ++c) {
      if (c < nch) {
        const int q = (int)threadIdx.x + c * WT;
        const int row = q >> cpr_shift, ch = q & ((1 << cpr_shift) - 1);
        pre[c] = make_uint4(0u, 0u, 0u, 0u);
        if (n0 + row < row_end)
          pre[c] = *reinterpret_cast<const uint4*>(kbytes + ((int64_t)g * p.kv_hs + (n0 + row) * p.kv_rs) * es + 16 * ch);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int c = 0; c < MAXCH; ++c) {
      if (c < nch) {
        const int q = (int)threadIdx.x + c * WT;
        const int row = q >> cpr_shift, ch = q & ((1 << cpr_shift) - 1);
        const uint4 v = pre[c];
        if (f32) {
          *reinterpret_cast<uint4*>(Kt + row * KS + 4 * ch) = v;
        } else {
          float4 lo, hi;
          if (p.kv_dtype == BF16) {
            lo = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                             __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
            hi = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xFFFF0000u),
                             __uint_as_float(v.w << 16), __uint_as_float(v.w & 0xFFFF0000u));
          } else {
            const __half* hv = reinterpret_cast<const __half*>(&v);
            lo = make_float4(__half2float(hv[0]), __half2float(hv[1]), __half2float(hv[2]), __half2float(hv[3]));
            hi = make_float4(__half2float(hv[4]), __half2float(hv[5]), __half2float(hv[6]), __half2float(hv[7]));
          }
          *reinterpret_cast<float4*>(Kt + row * KS + 8 * ch) = lo;
          *reinterpret_cast<float4*>(Kt + row * KS + 8 * ch + 4) = hi;
        }
      }
    }
  };

  int64_t t = blockIdx.x;
  if (t < n_tiles) load_tile(t);
  for (; t < n_tiles; t += gridDim.x) {
    const int64_t n0 = p.row0 + t * KT;
    const int nk = (int)min((int64_t)KT, row_end - n0);
    store_tile();
    if (t + gridDim.x < n_tiles) load_tile(t + gridDim.x);
    __syncthreads();
    // projection: Xl[row][col] = sum_d K[row][d] * W[d][col]
    {
      f32x4 acc[NCOLW][4];
#pragma unroll
      for (int m = 0; m < NCOLW; ++m)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) acc[m][rb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        float b[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) b[rb] = Kt[(16 * rb + lr) * KS + 4 * j + lk];
#pragma unroll
        for (int m = 0; m < NCOLW; ++m)
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
            acc[m][rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wreg[m][j], b[rb], acc[m][rb], 0, 0, 0);
      }
#pragma unroll
      for (int m = 0; m < NCOLW; ++m)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
          *reinterpret_cast<f32x4*>(Xl + (16 * rb + lr) * XS + 16 * (wid + 4 * m) + 4 * lk) = acc[m][rb];
    }
    __syncthreads();
    {
      float* klow = p.k_low + (int64_t)h * p.klow_hs + n0 * R;
      for (int q = threadIdx.x; q < KT * R / 4; q += WT) {
        const int row = q / (R / 4), c4 = q - row * (R / 4);
        if (row < nk)
          *reinterpret_cast<float4*>(klow + (int64_t)row * R + 4 * c4) = *reinterpret_cast<const float4*>(Xl + row * XS + 4 * c4);
      }
      if (want_codes && threadIdx.x < KT * S) {
        const int row = threadIdx.x / S, s = threadIdx.x - row * S;
        const float* x = Xl + row * XS + s * SUB;
        xxl[s * KT + row] = torch_order_dot(x, x, SUB);
      }
    }
    if (!want_codes) continue;
    __syncthreads();
    // distances of this wave's centroids to the 16 rows of each row block
#pragma unroll 1
    for (int rb = 0; rb < 4; ++rb) {
      float xb[S][XJ];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int j = 0; j < XJ; ++j) xb[s][j] = Xl[(16 * rb + lr) * XS + s * SUB + 4 * j + lk];
      f32x4 acc[S][NCBW];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int m = 0; m < NCBW; ++m) acc[s][m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < XJ; ++j)
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int m = 0; m < NCBW; ++m)
            acc[s][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(cbreg[s][m][j], xb[s][j], acc[s][m], 0, 0, 0);
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const float xx = xxl[s * KT + 16 * rb + lr];
        float best = INFINITY;
        int kb = 0;
        // (xx - 2 x.c) + |c|^2; 2 x.c is exact, so the fma rounds like the subtraction
#pragma unroll
        for (int m = 0; m < NCBW; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float dist = __builtin_fmaf(-2.0f, acc[s][m][i], xx) + cnreg[s][m][i];
            if (dist < best) {
              best = dist;
              kb = 4 * m + i;
            }
          }
        int arg = 16 * wid + 64 * (kb >> 2) + 4 * lk + (kb & 3);
#pragma unroll
        for (int o = 16; o < WAVE; o <<= 1) {
          const float ob = __shfl_xor(best, o);
          const int oa = __shfl_xor(arg, o);
          if (ob < best || (ob == best && oa < arg)) {
            best = ob;
            arg = oa;
          }
        }
        if (lk == 0) mb[(s * KT + 16 * rb + lr) * 4 + wid] = make_float2(best, __int_as_float(arg));
      }
    }
    __syncthreads();
    if (threadIdx.x < KT * S) {
      const int row = threadIdx.x / S, s = threadIdx.x - row * S;
      float best = INFINITY;
      int arg = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float2 v = mb[(s * KT + row) * 4 + w];
        const int oa = __float_as_int(v.y);
        if (v.x < best || (v.x == best && oa < arg)) {
          best = v.x;
          arg = oa;
        }
      }
      if (row < nk) store_code(p.codes, (int64_t)h * p.code_hs + (n0 + row) * S + s, p.ctype, arg);
    }
  }
}

template <int D, int S, int SUB, int C>
int launch_persistent(const WriteParams& p, int64_t tiles, hipStream_t stream) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    SVA_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, write_encode_persistent_kernel<D, S, SUB, C>, WT, 0),
                  "hipOccupancyMaxActiveBlocksPerMultiprocessor(write_encode_persistent_kernel)");
    per_cu = n > 0 ? n : 1;
  }
  const int64_t slots = (int64_t)per_cu * device_cu_count();
  const int64_t per_head = std::max<int64_t>(1, std::min<int64_t>(tiles, slots / p.H));
  hipLaunchKernelGGL((write_encode_persistent_kernel<D, S, SUB, C>), dim3((unsigned)per_head, (unsigned)p.H), dim3(WT),
                     0, stream, p);
  SVA_CHECK_LAUNCH("write_encode_persistent_kernel");
  return SVA_OK;
}

// Any shape: one thread per row, the same arithmetic as the tiled kernel.
__global__ void __launch_bounds__(64) write_encode_rowwise_kernel(WriteParams p) {
#pragma clang fp contract(off)
  const int D = p.D, R = p.R, S = p.S, C = p.C;
  const int sub = R / S;
  const int h = blockIdx.y;
  const int g = h / (p.H / p.G);
  const int64_t n = p.row0 + (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (n >= p.row0 + p.n_rows) return;
  const int64_t kb = (int64_t)g * p.kv_hs + n * p.kv_rs;
  const float* W = p.k_proj + (int64_t)h * D * R;
  float* x = p.k_low + (int64_t)h * p.klow_hs + n * R;
  for (int r = 0; r < R; ++r) {
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc = __builtin_fmaf(load_elem(p.keys, kb + d, p.kv_dtype), W[d * R + r], acc);
    x[r] = acc;
  }
  if (p.codes == nullptr) return;
  for (int s = 0; s < S; ++s) {
    const float* xs = x + s * sub;
    const float xx = torch_order_dot(xs, xs, sub);
    const float* cbs = p.codebooks + ((int64_t)h * S + s) * C * sub;
    float best = INFINITY;
    int arg = 0;
    for (int c = 0; c < C; ++c) {
      const float* cr = cbs + (int64_t)c * sub;
      float xc = 0.0f;
      for (int j = 0; j < sub; ++j) xc = __builtin_fmaf(xs[j], cr[j], xc);
      const float dist = (xx - 2.0f * xc) + torch_order_dot(cr, cr, sub);
      if (dist < best) {
        best = dist;
        arg = c;
      }
    }
    store_code(p.codes, (int64_t)h * p.code_hs + n * S + s, p.ctype, arg);
  }
}

// A decode step's append (at most FEW_ROWS rows): few_append (write_few.cuh)
// with one 256-thread workgroup per head.
template <int SUB>
__global__ void __launch_bounds__(WT) write_encode_few_kernel(WriteParams p) {
  few_append<SUB, WT>(p, (int)blockIdx.x, (int)blockIdx.y);
}

template <int SUB>
int launch_few(const WriteParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((write_encode_few_kernel<SUB>), dim3((unsigned)p.H, (unsigned)p.n_seq), dim3(WT), 0, stream, p);
  SVA_CHECK_LAUNCH("write_encode_few_kernel");
  return SVA_OK;
}

size_t write_lds_bytes(int64_t D, int64_t R, int64_t S, int64_t C) {
  const int64_t sub = R / S;
  return sizeof(float) * (size_t)(D * R + KT * (D + 1) + KT * (R + 1) + C * (sub + CB_PAD) + C + KT) + 16;
}

template <int SUB>
int launch_write(const WriteParams& p, dim3 grid, size_t lds, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((write_encode_kernel<SUB>), sva::kMaxLds, "hipFuncSetAttribute(write_encode_kernel)");
  hipLaunchKernelGGL(write_encode_kernel<SUB>, grid, dim3(WT), lds, stream, p);
  SVA_CHECK_LAUNCH("write_encode_kernel");
  return SVA_OK;
}

}  // namespace

namespace sva {

int write_encode_setup(const void* keys, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                       int64_t row_begin, int64_t n_rows, int64_t H, int64_t G, int64_t D, int64_t R, int64_t S,
                       int64_t C, const float* k_proj, const float* codebooks, float* k_low,
                       int64_t k_low_head_stride, void* codes, int code_type, int64_t code_head_stride,
                       WriteParams* out) {
  SVA_REQUIRE(keys && k_proj && codebooks && k_low, "sva_write_encode: null pointer");
  SVA_REQUIRE(row_begin >= 0 && n_rows >= 0, "sva_write_encode: bad row range");
  SVA_REQUIRE(H > 0 && G > 0 && H % G == 0, "sva_write_encode: %lld query heads over %lld KV heads", (long long)H,
              (long long)G);
  SVA_REQUIRE(D > 0 && D <= 256 && R > 0 && R <= 256, "sva_write_encode: head_dim %lld / rank %lld unsupported",
              (long long)D, (long long)R);
  SVA_REQUIRE(S > 0 && R % S == 0, "sva_write_encode: rank_dim=%lld must be divisible by subspaces=%lld",
              (long long)R, (long long)S);
  SVA_REQUIRE(C > 0, "sva_write_encode: codewords %lld", (long long)C);
  SVA_REQUIRE(kv_dtype >= 0 && kv_dtype <= 2 && code_type >= 0 && code_type <= 3, "sva_write_encode: bad dtype");
  const int64_t code_max = code_type == 0 ? 256 : code_type == 1 ? 32768 : (1ll << 31);
  SVA_REQUIRE(C <= code_max, "sva_write_encode: %lld codewords do not fit the code type", (long long)C);
  SVA_REQUIRE((n_rows + KT - 1) / KT < (1ll << 31) && H <= 65535, "sva_write_encode: too many rows or heads");
  WriteParams& p = *out;
  p.keys = keys;
  p.kv_dtype = kv_dtype;
  p.kv_hs = kv_head_stride;
  p.kv_rs = kv_row_stride;
  p.row0 = row_begin;
  p.n_rows = n_rows;
  p.H = (int)H;
  p.G = (int)G;
  p.D = (int)D;
  p.R = (int)R;
  p.S = (int)S;
  p.C = (int)C;
  p.k_proj = k_proj;
  p.codebooks = codebooks;
  p.k_low = k_low;
  p.klow_hs = k_low_head_stride;
  p.codes = codes;
  p.ctype = code_type;
  p.code_hs = code_head_stride;
  p.n_seq = 1;
  p.seq_kv = 0;
  p.seq_rows = 0;
  return SVA_OK;
}

int write_few_form(const WriteParams& p) {
  if (p.n_rows <= 0 || p.n_rows > FEW_ROWS) return -1;
  if (((uintptr_t)p.codebooks & 15u) != 0) return 0;  // codeword rows as float4 where aligned
  const int sub = p.R / p.S;
  return sub == 16 || sub == 32 || sub == 64 ? sub : 0;
}

int write_encode_launch(const WriteParams& p, hipStream_t stream) {
  if (p.n_rows == 0 || p.n_seq <= 0) return SVA_OK;
  switch (write_few_form(p)) {  // a decode step's append, every sequence in one launch
    case 0: return launch_few<0>(p, stream);
    case 16: return launch_few<16>(p, stream);
    case 32: return launch_few<32>(p, stream);
    case 64: return launch_few<64>(p, stream);
    default: break;
  }
  if (p.n_seq > 1) {  // the tiled forms take one sequence a launch
    const int64_t kv_es = p.kv_dtype == 0 ? 4 : 2;
    const int64_t code_es = p.ctype == 0 ? 1 : p.ctype == 1 ? 2 : p.ctype == 2 ? 4 : 8;
    for (int64_t b = 0; b < p.n_seq; ++b) {
      WriteParams q = p;
      q.n_seq = 1;
      q.seq_kv = q.seq_rows = 0;
      q.keys = (const char*)p.keys + b * p.seq_kv * kv_es;
      q.k_low = p.k_low + b * p.seq_rows * p.R;
      q.codes = p.codes != nullptr ? (void*)((char*)p.codes + b * p.seq_rows * p.S * code_es) : nullptr;
      const int rc = write_encode_launch(q, stream);
      if (rc != SVA_OK) return rc;
    }
    return SVA_OK;
  }
  const int64_t D = p.D, R = p.R, S = p.S, C = p.C;
  const size_t lds = write_lds_bytes(D, R, S, C);
  const bool tiled = R % 4 == 0 && (R / S) % 4 == 0 && p.klow_hs % 4 == 0 &&
                     (((uintptr_t)p.k_proj | (uintptr_t)p.codebooks | (uintptr_t)p.k_low) & 15u) == 0 &&
                     lds <= (size_t)sva::kMaxLds;
  const int64_t tiles = (p.n_rows + KT - 1) / KT;
  const dim3 grid((unsigned)tiles, (unsigned)p.H);
  if (!tiled) {
    hipLaunchKernelGGL(write_encode_rowwise_kernel, grid, dim3(64), 0, stream, p);
    SVA_CHECK_LAUNCH("write_encode_rowwise_kernel");
    return SVA_OK;
  }
  const int64_t es = p.kv_dtype == 0 ? 4 : 2;
  const bool rows_aligned = ((uintptr_t)p.keys & 15u) == 0 && (p.kv_hs * es) % 16 == 0 && (p.kv_rs * es) % 16 == 0;
  if (rows_aligned && R == 64 && (D == 64 || D == 128)) {
    if (S == 2 && C == 256)
      return D == 64 ? launch_persistent<64, 2, 32, 256>(p, tiles, stream)
                     : launch_persistent<128, 2, 32, 256>(p, tiles, stream);
    if (S == 4 && C == 64)
      return D == 64 ? launch_persistent<64, 4, 16, 64>(p, tiles, stream)
                     : launch_persistent<128, 4, 16, 64>(p, tiles, stream);
  }
  if (R % 16 == 0 && C % 16 == 0 && D % 4 == 0) {
    SVA_SET_MAX_LDS_ONCE(write_encode_mfma_kernel, sva::kMaxLds, "hipFuncSetAttribute(write_encode_mfma_kernel)");
    hipLaunchKernelGGL(write_encode_mfma_kernel, grid, dim3(WT), lds, stream, p);
    SVA_CHECK_LAUNCH("write_encode_mfma_kernel");
    return SVA_OK;
  }
  switch (R / S) {
    case 8: return launch_write<8>(p, grid, lds, stream);
    case 16: return launch_write<16>(p, grid, lds, stream);
    case 32: return launch_write<32>(p, grid, lds, stream);
    case 64: return launch_write<64>(p, grid, lds, stream);
    default: return launch_write<0>(p, grid, lds, stream);
  }
}

}  // namespace sva

extern "C" int sva_write_encode_batch(const void* keys, int kv_dtype, int64_t kv_seq_stride, int64_t kv_head_stride,
                                      int64_t kv_row_stride, int64_t n_seq, int64_t row_begin, int64_t n_rows,
                                      int64_t H, int64_t G, int64_t D, int64_t R, int64_t S, int64_t C,
                                      const float* k_proj, const float* codebooks, float* k_low,
                                      int64_t k_low_head_stride, int64_t catalog_seq_rows, void* codes, int code_type,
                                      int64_t code_head_stride, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(n_seq > 0 && n_seq <= 65535, "sva_write_encode_batch: %lld sequences", (long long)n_seq);
  SVA_REQUIRE(kv_seq_stride >= 0 && catalog_seq_rows >= row_begin + n_rows,
              "sva_write_encode_batch: sequences overlap (catalog rows per sequence %lld, rows up to %lld)",
              (long long)catalog_seq_rows, (long long)(row_begin + n_rows));
  sva::WriteParams p;
  const int rc = sva::write_encode_setup(keys, kv_dtype, kv_head_stride, kv_row_stride, row_begin, n_rows, H, G, D,
                                         R, S, C, k_proj, codebooks, k_low, k_low_head_stride, codes, code_type,
                                         code_head_stride, &p);
  if (rc != SVA_OK) return rc;
  p.n_seq = (int)n_seq;
  p.seq_kv = kv_seq_stride;
  p.seq_rows = catalog_seq_rows;
  return sva::write_encode_launch(p, (hipStream_t)stream);
}

extern "C" int sva_write_encode(const void* keys, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                                int64_t row_begin, int64_t n_rows, int64_t H, int64_t G, int64_t D, int64_t R,
                                int64_t S, int64_t C, const float* k_proj, const float* codebooks, float* k_low,
                                int64_t k_low_head_stride, void* codes, int code_type, int64_t code_head_stride,
                                void* stream) {
  sva::clear_error();
  sva::WriteParams p;
  const int rc = sva::write_encode_setup(keys, kv_dtype, kv_head_stride, kv_row_stride, row_begin, n_rows, H, G, D,
                                         R, S, C, k_proj, codebooks, k_low, k_low_head_stride, codes, code_type,
                                         code_head_stride, &p);
  if (rc != SVA_OK) return rc;
  return sva::write_encode_launch(p, (hipStream_t)stream);
}
