// Codebook fit support: the k-means centroid update of the reference's
// product-codebook fits.  Assignment is sva_write_encode (an identity map
// gives the nearest-centroid labels of the rows themselves) and the cells
// are sva_postings_build's CSR.
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
