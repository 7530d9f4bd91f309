// Codebook fit support: the k-means centroid update of the reference's
// product-codebook fits and the attention-weighted key weights of the
// codebook refresh.  Assignment is sva_write_encode (an identity map gives
// the nearest-centroid labels of the rows themselves) and the cells are
// sva_postings_build's CSR.
#include "capi_internal.h"
#include "common.cuh"

using namespace sva;

// k-means centroid update of the codebook fit (experiments/sva_pq_lookup_test.py:92-100,
// experiments/sva_supervised_coarse_pq_test.py:117-126): for every (head h,
// subspace s, cell c) with members ids[offsets[c] .. offsets[c + 1]) (the
// CSR of the current labels, ascending key order),
//   sums  = sum over members of x[n] (or w[n] * x[n], each product rounded)
//   count = member count (or the sum of their weights)
//   centroid = sums / count, or the previous centroid for an empty cell
// with every sum taken in ascending key order (what index_add_ does on the CPU).
namespace {

__global__ void __launch_bounds__(64) centroid_update_kernel(const float* __restrict__ x, int64_t x_hs, int R, int S,
                                                             int C, int64_t n_rows, const float* __restrict__ w,
                                                             const int32_t* __restrict__ offsets,
                                                             const int32_t* __restrict__ ids,
                                                             const float* __restrict__ prev, float* __restrict__ next) {
#pragma clang fp contract(off)
  const int sub = R / S;
  const int64_t cell = blockIdx.x;  // (h * S + s) * C + c
  const int64_t hs = cell / C;
  const int h = (int)(hs / S), s = (int)(hs % S);
  const int d = threadIdx.x;
  const int32_t* off = offsets + hs * (C + 1) + (cell - hs * C);
  const int o0 = off[0], o1 = off[1];
  const int32_t* mem = ids + hs * n_rows;
  const float* xh = x + (int64_t)h * x_hs + s * sub;
  const float* wh = w ? w + (int64_t)h * n_rows : nullptr;
  float acc = 0.0f, cnt = 0.0f;
  if (d < sub) {
    for (int i = o0; i < o1; ++i) {
      const int64_t n = mem[i];
      const float v = xh[n * R + d];
      if (wh) {
        const float wn = wh[n];
        acc = acc + wn * v;
        cnt = cnt + wn;
      } else {
        acc = acc + v;
      }
    }
    if (!wh) cnt = (float)(o1 - o0);
    next[cell * sub + d] = cnt > 0.0f ? acc / cnt : prev[cell * sub + d];
  }
}

}  // namespace

extern "C" int sva_centroid_update(const float* x, int64_t x_head_stride, int64_t n_rows, int64_t H, int64_t R,
                                   int64_t S, int64_t C, const float* weights, const int32_t* offsets,
                                   const int32_t* ids, const float* centroids, float* next_centroids, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(x && offsets && ids && centroids && next_centroids, "sva_centroid_update: null pointer");
  SVA_REQUIRE(n_rows > 0 && n_rows < (1ll << 31) && H > 0 && S > 0 && C > 0 && R % S == 0 && R / S <= 64 &&
                  H * S * C < (1ll << 31),
              "sva_centroid_update: bad sizes");
  hipLaunchKernelGGL(centroid_update_kernel, dim3((unsigned)(H * S * C)), dim3(64), 0, (hipStream_t)stream, x,
                     x_head_stride, (int)R, (int)S, (int)C, n_rows, weights, offsets, ids, centroids, next_centroids);
  SVA_CHECK_LAUNCH("centroid_update_kernel");
  return SVA_OK;
}

// Attention-weighted key weights of the codebook refresh
// (experiments/sva_codebook_refresh_benchmark.py:136-153): weights[h, n] is
// 1 plus `boost` once for every valid top-k hit of key n in head h, each
// addition rounded to fp32 in turn.  Every hit adds the same value, so the
// partial sums 1, 1 + boost, (1 + boost) + boost, ... do not depend on which
// hit lands first: counting the hits with integer atomics and then adding
// boost count times gives index_add_'s result bit for bit.  The weights
// buffer holds the counts (as uint32) between the two passes.
namespace {

constexpr int KW_BLOCK = 256;

__global__ void __launch_bounds__(KW_BLOCK) key_hits_clear_kernel(uint32_t* __restrict__ hits, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * KW_BLOCK + threadIdx.x;
  if (i < total) hits[i] = 0u;
}

__global__ void __launch_bounds__(KW_BLOCK) key_hits_kernel(const int64_t* __restrict__ top_idx,
                                                            const uint8_t* __restrict__ top_valid, int64_t per_head,
                                                            int64_t entries, int64_t n_keys,
                                                            uint32_t* __restrict__ hits) {
  const int64_t i = (int64_t)blockIdx.x * KW_BLOCK + threadIdx.x;
  if (i >= entries || !top_valid[i]) return;
  const int64_t h = i / per_head;
  int64_t n = top_idx[i];
  n = n < 0 ? 0 : (n >= n_keys ? n_keys - 1 : n);  // the reference clamps into [0, seq_len)
  atomicAdd(hits + h * n_keys + n, 1u);
}

__global__ void __launch_bounds__(KW_BLOCK) key_weights_kernel(float* __restrict__ weights, float boost,
                                                               int64_t total) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * KW_BLOCK + threadIdx.x;
  if (i >= total) return;
  uint32_t c = reinterpret_cast<const uint32_t*>(weights)[i];
  float w = 1.0f;
  for (; c != 0u; --c) w += boost;
  weights[i] = w;
}

}  // namespace

extern "C" int sva_key_weights(const int64_t* top_idx, const uint8_t* top_valid, int64_t H, int64_t per_head,
                               int64_t n_keys, float boost, float* weights, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(weights && (per_head == 0 || (top_idx && top_valid)), "sva_key_weights: null pointer");
  SVA_REQUIRE(H > 0 && n_keys > 0 && per_head >= 0 && H * n_keys < (1ll << 40) && H * per_head < (1ll << 40),
              "sva_key_weights: bad sizes");
  hipStream_t st = (hipStream_t)stream;
  const int64_t total = H * n_keys, entries = H * per_head;
  uint32_t* hits = reinterpret_cast<uint32_t*>(weights);
  hipLaunchKernelGGL(key_hits_clear_kernel, dim3((unsigned)((total + KW_BLOCK - 1) / KW_BLOCK)), dim3(KW_BLOCK), 0,
                     st, hits, total);
  SVA_CHECK_LAUNCH("key_hits_clear_kernel");
  if (entries > 0) {
    hipLaunchKernelGGL(key_hits_kernel, dim3((unsigned)((entries + KW_BLOCK - 1) / KW_BLOCK)), dim3(KW_BLOCK), 0, st,
                       top_idx, top_valid, per_head, entries, n_keys, hits);
    SVA_CHECK_LAUNCH("key_hits_kernel");
  }
  hipLaunchKernelGGL(key_weights_kernel, dim3((unsigned)((total + KW_BLOCK - 1) / KW_BLOCK)), dim3(KW_BLOCK), 0, st,
                     weights, boost, total);
  SVA_CHECK_LAUNCH("key_weights_kernel");
  return SVA_OK;
}
