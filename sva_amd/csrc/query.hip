// Query side of the decode path: learned query map, per-query PQ lookup
// table, score bounds, and the all-keys PQ score kernel.
//
// q_low[r]  = (sum_d q[d] * q_proj[h][d][r], sequential fma over d) * scale[h]
//             (sva/llama.py:211)
// lut[s][c] = sum_j q_low[s*sub + j] * cb[h][s][c][j], sequential fma over j
//             (sva/ops.py:68)
// score     = (((0 + lut[0][c0]) + lut[1][c1]) + ...) / sqrt(R)   (sva/ops.py:64-71)
#include "capi_internal.h"
#include "common.cuh"

using namespace sva;

namespace {

constexpr int PREP_BLOCK = 256;

__global__ void __launch_bounds__(PREP_BLOCK)
    query_lut_kernel(const void* __restrict__ q, int q_dtype, int64_t q_bs, int64_t q_hs, int64_t q_ts, int H, int Q,
                     int D, int R, int S, int C, const float* __restrict__ q_proj, const float* __restrict__ scale,
                     const float* __restrict__ codebooks, float sqrt_r, float* __restrict__ q_low,
                     float* __restrict__ lut, float* __restrict__ range) {
#pragma clang fp contract(off)
  __shared__ float qf[512];
  __shared__ float ql[512];
  __shared__ uint32_t kmin[64];
  __shared__ uint32_t kmax[64];
  const int item = blockIdx.x;
  const int t = item % Q;
  const int h = (item / Q) % H;
  const int b = item / (Q * H);
  const int64_t qbase = (int64_t)b * q_bs + (int64_t)h * q_hs + (int64_t)t * q_ts;
  for (int d = threadIdx.x; d < D; d += PREP_BLOCK) qf[d] = load_elem(q, qbase + d, q_dtype);
  for (int s = threadIdx.x; s < S; s += PREP_BLOCK) {
    kmin[s] = 0xFFFFFFFFu;
    kmax[s] = 0u;
  }
  __syncthreads();
  const float* W = q_proj + (int64_t)h * D * R;
  const float sc = scale[h];
  for (int r = threadIdx.x; r < R; r += PREP_BLOCK) {
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc = __builtin_fmaf(qf[d], W[(int64_t)d * R + r], acc);
    const float v = acc * sc;
    ql[r] = v;
    q_low[(int64_t)item * R + r] = v;
  }
  __syncthreads();
  const int sub = R / S;
  const float* cb = codebooks + (int64_t)h * S * C * sub;
  for (int e = threadIdx.x; e < S * C; e += PREP_BLOCK) {
    const int s = e / C;
    const float* w = cb + (int64_t)e * sub;
    const float* qs = ql + s * sub;
    float acc = 0.0f;
    for (int j = 0; j < sub; ++j) acc = __builtin_fmaf(qs[j], w[j], acc);
    lut[(int64_t)item * S * C + e] = acc;
    const uint32_t k = f2key(acc);
    atomicMin(&kmin[s], k);
    atomicMax(&kmax[s], k);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float lo = 0.0f, hi = 0.0f;
    for (int s = 0; s < S; ++s) {
      lo = lo + key2f(kmin[s]);
      hi = hi + key2f(kmax[s]);
    }
    range[(int64_t)item * 2 + 0] = lo / sqrt_r;
    range[(int64_t)item * 2 + 1] = hi / sqrt_r;
  }
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

}  // namespace

extern "C" int sva_query_lut(const void* q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride,
                             int64_t q_tok_stride, int64_t n_seq, int64_t H, int64_t Q, int64_t D, int64_t R,
                             int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                             float* q_low, float* lut, float* score_range, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(q && q_proj && scale && codebooks && q_low && lut && score_range, "sva_query_lut: null pointer");
  SVA_REQUIRE(n_seq > 0 && H > 0 && Q > 0, "sva_query_lut: empty query batch");
  SVA_REQUIRE(D > 0 && D <= 512 && R > 0 && R <= 512, "sva_query_lut: head_dim %lld / rank %lld out of range",
              (long long)D, (long long)R);
  SVA_REQUIRE(S > 0 && S <= 64 && R % S == 0, "sva_query_lut: rank %lld not divisible by subspaces %lld",
              (long long)R, (long long)S);
  SVA_REQUIRE(C > 0 && S * C <= 65536, "sva_query_lut: codewords %lld out of range", (long long)C);
  SVA_REQUIRE(q_dtype >= 0 && q_dtype <= 2, "sva_query_lut: bad q dtype");
  const int64_t items = n_seq * H * Q;
  SVA_REQUIRE(items < (1ll << 31), "sva_query_lut: too many query items");
  const float sqrt_r = (float)sqrt((double)R);
  hipLaunchKernelGGL(query_lut_kernel, dim3((unsigned)items), dim3(PREP_BLOCK), 0, (hipStream_t)stream, q, q_dtype,
                     q_seq_stride, q_head_stride, q_tok_stride, (int)H, (int)Q, (int)D, (int)R, (int)S, (int)C, q_proj,
                     scale, codebooks, sqrt_r, q_low, lut, score_range);
  SVA_CHECK_LAUNCH("query_lut_kernel");
  return SVA_OK;
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
