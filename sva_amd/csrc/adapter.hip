// Residual output adapter of the late-layer socket
// (experiments/sva_late4_logit_distill.py:37-51): for every token,
//   x    = [hidden_states, attn_output]                  (2 * hidden, fp32)
//   corr = up(gelu(down(x))) * scale                     (fp32; exact erf GELU)
//   out  = attn_output + corr.to(attn dtype)             (in the attn dtype)
// down [rank, 2 * hidden] and up [hidden, rank] are fp32 (nn.Linear weights).
//
// One workgroup per TOK tokens: the tokens' inputs are staged in LDS as
// fp32, each thread forms down-projection outputs (token, o) as a
// sequential fma chain over the 2 * hidden inputs, the GELU values go to
// LDS, then each output (token, j) is a sequential chain over the rank.
// Consecutive threads take consecutive tokens of one output, so a wave's
// weight loads read a few rows (the same address across a row's tokens)
// rather than one row per lane; the staged rows are padded by a float so
// that the tokens' reads of one column fall in different LDS banks.
#include <cmath>

#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int AB = 256;          // threads per workgroup
constexpr int MAX_RANK = 64;
constexpr int MAX_TOK = 16;

struct AdapterParams {
  const void* hidden;
  int h_dtype;
  int64_t h_rs;
  const void* attn;
  int a_dtype;
  int64_t a_rs;
  const float* down;  // [rank, 2 * H]
  const float* up;    // [H, rank]
  float scale;
  int64_t T;
  int H, rank, tok;
  void* out;
  int o_dtype;
  int64_t o_rs;
};

// The value a float takes after a cast to dtype (round to nearest even).
SVA_DEV float round_to(float v, int dtype) {
  if (dtype == F32) return v;
  if (dtype == BF16) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7F800000u) == 0x7F800000u) return v;  // inf and nan pass through
    u += 0x7FFFu + ((u >> 16) & 1u);                 // as store_elem rounds
    return __uint_as_float(u & 0xFFFF0000u);
  }
  return __half2float(__float2half_rn(v));
}

__global__ void __launch_bounds__(AB) residual_adapter_kernel(AdapterParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float xs[];  // [tok][2 * H + 1], then z [tok][rank + 1]
  const int H2 = 2 * p.H;
  const int XS = H2 + 1, ZS = p.rank + 1;  // padded row strides
  float* z = xs + p.tok * XS;
  const int64_t t0 = (int64_t)blockIdx.x * p.tok;
  const int nt = (int)min((int64_t)p.tok, p.T - t0);
  // Both weight matrices requested by every thread at entry, one float per
  // 128-byte line: they miss the L2 at every call (the layer runs once a
  // step), and the chains below would otherwise wait on one miss after
  // another.  The values are folded into a word that is stored only in a case
  // that cannot occur (a negative token count), so the loads are kept.
  float touch = 0.0f;
  {
    const int64_t nd = (int64_t)p.rank * H2, nall = nd + (int64_t)p.H * p.rank;  // floats
    auto at = [&](int64_t f) { return f < nd ? p.down[f] : p.up[f - nd]; };
    constexpr int TU = 16;  // the first TU lines a thread, requested together (indices clamped)
    float v[TU];
#pragma unroll
    for (int u = 0; u < TU; ++u) v[u] = at(min(((int64_t)threadIdx.x + (int64_t)u * AB) * 32, nall - 1));
#pragma unroll
    for (int u = 0; u < TU; ++u) touch += v[u];
    for (int64_t f = ((int64_t)threadIdx.x + (int64_t)TU * AB) * 32; f < nall; f += (int64_t)AB * 32) touch += at(f);
  }
  {
    // the inputs, SU elements a thread per batch: raw bits requested first
    // (indices clamped, every load unconditional), converted at the store
    constexpr int SU = 8;
    const int total = nt * H2;
    for (int e0 = threadIdx.x; e0 < total; e0 += SU * AB) {
      uint32_t bits[SU];
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int e = min(e0 + u * AB, total - 1);
        const int t = e / H2, k = e - t * H2;
        const bool hid = k < p.H;
        bits[u] = load_elem_bits(hid ? p.hidden : p.attn, hid ? (t0 + t) * p.h_rs + k : (t0 + t) * p.a_rs + (k - p.H),
                                 hid ? p.h_dtype : p.a_dtype);
      }
#pragma unroll
      for (int u = 0; u < SU; ++u) {
        const int e = e0 + u * AB;
        if (e < total) {
          const int t = e / H2, k = e - t * H2;
          xs[t * XS + k] = elem_from_bits(bits[u], k < p.H ? p.h_dtype : p.a_dtype);
        }
      }
    }
  }
  __syncthreads();
  // the weight rows as float4 where aligned: a chain of 2H steps is bound by
  // its loads unless the next 32 weights are in flight while the current 32
  // are used (the same fma chain, in k order)
  constexpr int V = 8;  // float4s per batch
  const bool vec = ((uintptr_t)p.down & 15u) == 0 && ((uintptr_t)p.up & 15u) == 0 && H2 % (4 * V) == 0 &&
                   p.rank % 4 == 0;
  for (int e = threadIdx.x; e < nt * p.rank; e += AB) {
    const int o = e / nt, t = e - o * nt;
    const float* x = xs + t * XS;
    const float* w = p.down + (int64_t)o * H2;
    float acc = 0.0f;
    if (vec) {
      const float4* w4 = reinterpret_cast<const float4*>(w);
      const int nb = H2 / (4 * V);
      float4 cur[V], nxt[V];
#pragma unroll
      for (int u = 0; u < V; ++u) cur[u] = w4[u];
      for (int b = 0; b < nb; ++b) {
        const int bn = min(b + 1, nb - 1);  // the last batch loads itself again: every load unconditional
#pragma unroll
        for (int u = 0; u < V; ++u) nxt[u] = w4[bn * V + u];
#pragma unroll
        for (int u = 0; u < V; ++u) {
          const float* xk = x + (b * V + u) * 4;
          acc = __builtin_fmaf(xk[0], cur[u].x, acc);
          acc = __builtin_fmaf(xk[1], cur[u].y, acc);
          acc = __builtin_fmaf(xk[2], cur[u].z, acc);
          acc = __builtin_fmaf(xk[3], cur[u].w, acc);
        }
#pragma unroll
        for (int u = 0; u < V; ++u) cur[u] = nxt[u];
      }
    } else {
      for (int k = 0; k < H2; ++k) acc = __builtin_fmaf(x[k], w[k], acc);
    }
    z[t * ZS + o] = 0.5f * acc * (1.0f + erff(acc * 0.70710678118654752f));  // F.gelu (erf form)
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nt * p.H; e += AB) {
    const int j = e / nt, t = e - j * nt;
    const float* zz = z + t * ZS;
    const float* w = p.up + (int64_t)j * p.rank;
    float acc = 0.0f;
    if (vec && p.rank == MAX_RANK) {  // the row's 64 weights requested at once
      const float4* w4 = reinterpret_cast<const float4*>(w);
      float4 wv[MAX_RANK / 4];
#pragma unroll
      for (int u = 0; u < MAX_RANK / 4; ++u) wv[u] = w4[u];
#pragma unroll
      for (int u = 0; u < MAX_RANK / 4; ++u) {
        acc = __builtin_fmaf(zz[4 * u], wv[u].x, acc);
        acc = __builtin_fmaf(zz[4 * u + 1], wv[u].y, acc);
        acc = __builtin_fmaf(zz[4 * u + 2], wv[u].z, acc);
        acc = __builtin_fmaf(zz[4 * u + 3], wv[u].w, acc);
      }
    } else {
      for (int o = 0; o < p.rank; ++o) acc = __builtin_fmaf(zz[o], w[o], acc);
    }
    const float corr = round_to(acc * p.scale, p.a_dtype);
    const float a = xs[t * XS + p.H + j];
    store_elem(p.out, (t0 + t) * p.o_rs + j, p.o_dtype, a + corr);
  }
  if (p.T < 0) store_elem(p.out, threadIdx.x, p.o_dtype, touch);  // never: keeps the requests above
}

}  // namespace

extern "C" int sva_residual_adapter(const void* hidden, int hidden_dtype, int64_t hidden_row_stride, const void* attn,
                                    int attn_dtype, int64_t attn_row_stride, const float* down_w, const float* up_w,
                                    float scale, int64_t n_tokens, int64_t hidden_size, int64_t rank, void* out,
                                    int out_dtype, int64_t out_row_stride, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(hidden && attn && down_w && up_w && out, "sva_residual_adapter: null pointer");
  SVA_REQUIRE(n_tokens >= 0 && hidden_size > 0 && hidden_size <= 8192, "sva_residual_adapter: bad sizes");
  SVA_UNSUPPORTED(rank > 0 && rank <= MAX_RANK, "sva_residual_adapter: rank %lld (at most %d)", (long long)rank,
                  MAX_RANK);
  SVA_REQUIRE(hidden_dtype >= 0 && hidden_dtype <= 2 && attn_dtype >= 0 && attn_dtype <= 2 && out_dtype >= 0 &&
                  out_dtype <= 2,
              "sva_residual_adapter: bad dtype");
  if (n_tokens == 0) return SVA_OK;
  // tokens per workgroup: as many as fit 64 KB of staged fp32 inputs (rows padded by a float), at most MAX_TOK
  const int64_t per_tok = sizeof(float) * (2 * hidden_size + 1 + rank + 1);
  const int tok = (int)std::max<int64_t>(1, std::min<int64_t>(MAX_TOK, (64 * 1024) / per_tok));
  const size_t lds = (size_t)tok * (size_t)per_tok;
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_residual_adapter: hidden size %lld needs %zu bytes of LDS",
                  (long long)hidden_size, lds);
  const int64_t blocks = (n_tokens + tok - 1) / tok;
  SVA_REQUIRE(blocks < (1ll << 31), "sva_residual_adapter: too many tokens");
  SVA_SET_MAX_LDS_ONCE(residual_adapter_kernel, sva::kMaxLds, "hipFuncSetAttribute(residual_adapter_kernel)");
  AdapterParams p;
  p.hidden = hidden;
  p.h_dtype = hidden_dtype;
  p.h_rs = hidden_row_stride;
  p.attn = attn;
  p.a_dtype = attn_dtype;
  p.a_rs = attn_row_stride;
  p.down = down_w;
  p.up = up_w;
  p.scale = scale;
  p.T = n_tokens;
  p.H = (int)hidden_size;
  p.rank = (int)rank;
  p.tok = tok;
  p.out = out;
  p.o_dtype = out_dtype;
  p.o_rs = out_row_stride;
  hipLaunchKernelGGL(residual_adapter_kernel, dim3((unsigned)blocks), dim3(AB), lds, (hipStream_t)stream, p);
  SVA_CHECK_LAUNCH("residual_adapter_kernel");
  return SVA_OK;
}

