// One patched layer's decode step behind a handle: the catalog append of the
// cache's new rows, the lookup with its verifier and the step's statistics,
// issued by one C-ABI call.  The handle keeps the layer's fixed arguments
// (sizes, weights) and its bound buffers (catalog, lookup outputs,
// workspaces, statistics), so a decode step passes only what changes per
// token: the query row, the KV cache, the key count and the output.
#include <new>

#include "capi_internal.h"
#include "summon.h"
#include "write_few.cuh"

struct sva_decode_layer {
  int64_t H, G, D, R, S, C, L, B;
  const float* q_proj;
  const float* scale;
  const float* codebooks;
  const float* k_proj;
  float scaling;
  // bound buffers (sva_decode_layer_bind)
  bool bound;
  float* k_low;
  int64_t klow_hs;
  void* codes;
  int code_type;
  int64_t code_hs;
  int64_t capacity;
  float* q_low;
  float* lut;
  float* range;
  int32_t* sl_idx;
  float* sl_rank;
  int32_t* counts;  // [3, H]: shortlist sizes, budget sizes, floor overshoots
  int32_t* fin_idx;
  void* ws;
  size_t ws_bytes;
  void* vws;
  size_t vws_bytes;
  int64_t* stats;  // [4] or nullptr: summoned, verified, overshoots, queries
};

namespace {

// stats[0..3] += (sum of shortlist sizes, sum of budget sizes, overshoots, H):
// one wave over the step's count rows.
// with_floor: the step's path has a sampled floor and wrote the overshoot row.
__global__ void decode_stats_kernel(const int32_t* __restrict__ counts, int H, bool with_floor,
                                    int64_t* __restrict__ stats) {
  const int h = threadIdx.x;
  uint32_t a = 0, b = 0, c = 0;
  if (h < H) {
    a = (uint32_t)counts[h];
    b = (uint32_t)counts[H + h];
    c = with_floor ? (uint32_t)counts[2 * H + h] : 0u;
  }
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_xor(a, o, 64);
    b += __shfl_xor(b, o, 64);
    c += __shfl_xor(c, o, 64);
  }
  if (h == 0) {
    stats[0] += a;
    stats[1] += b;
    stats[2] += c;
    stats[3] += H;
  }
}

}  // namespace

extern "C" int sva_decode_layer_create(int64_t H, int64_t G, int64_t D, int64_t R, int64_t S, int64_t C, int64_t L,
                                       int64_t B, const float* q_proj, const float* scale, const float* codebooks,
                                       const float* k_proj, float scaling, sva_decode_layer** out) {
  sva::clear_error();
  SVA_REQUIRE(out != nullptr && q_proj && scale && codebooks && k_proj, "sva_decode_layer_create: null pointer");
  SVA_REQUIRE(H > 0 && H <= 64 && G > 0 && H % G == 0, "sva_decode_layer_create: %lld query heads over %lld KV heads",
              (long long)H, (long long)G);
  SVA_REQUIRE(D > 0 && R > 0 && S > 0 && R % S == 0 && C > 0, "sva_decode_layer_create: bad sizes");
  SVA_REQUIRE(L > 0 && B > 0 && B <= L && B <= 8192, "sva_decode_layer_create: shortlist %lld / budget %lld",
              (long long)L, (long long)B);
  sva_decode_layer* h = new (std::nothrow) sva_decode_layer{};
  SVA_REQUIRE(h != nullptr, "sva_decode_layer_create: out of host memory");
  h->H = H, h->G = G, h->D = D, h->R = R, h->S = S, h->C = C, h->L = L, h->B = B;
  h->q_proj = q_proj, h->scale = scale, h->codebooks = codebooks, h->k_proj = k_proj;
  h->scaling = scaling;
  h->bound = false;
  *out = h;
  return SVA_OK;
}

extern "C" int sva_decode_layer_bind(sva_decode_layer* h, float* k_low, int64_t k_low_head_stride, void* codes,
                                     int code_type, int64_t code_head_stride, int64_t capacity, float* q_low,
                                     float* lut, float* score_range, int32_t* sl_idx, float* sl_rank, int32_t* counts,
                                     int32_t* fin_idx, void* workspace, size_t workspace_bytes,
                                     void* verify_workspace, size_t verify_workspace_bytes, int64_t* stats) {
  sva::clear_error();
  SVA_REQUIRE(h != nullptr, "sva_decode_layer_bind: null handle");
  SVA_REQUIRE(k_low && codes && q_low && lut && score_range && sl_idx && sl_rank && counts && fin_idx,
              "sva_decode_layer_bind: null pointer");
  SVA_REQUIRE(code_type >= 0 && code_type <= 3 && capacity >= 0, "sva_decode_layer_bind: bad catalog");
  h->k_low = k_low, h->klow_hs = k_low_head_stride;
  h->codes = codes, h->code_type = code_type, h->code_hs = code_head_stride, h->capacity = capacity;
  h->q_low = q_low, h->lut = lut, h->range = score_range;
  h->sl_idx = sl_idx, h->sl_rank = sl_rank, h->counts = counts, h->fin_idx = fin_idx;
  h->ws = workspace, h->ws_bytes = workspace_bytes;
  h->vws = verify_workspace, h->vws_bytes = verify_workspace_bytes;
  h->stats = stats;
  h->bound = true;
  return SVA_OK;
}

extern "C" int sva_decode_layer_step(sva_decode_layer* h, const void* q, int q_dtype, int64_t q_head_stride,
                                     const void* keys, const void* values, int kv_dtype, int64_t kv_head_stride,
                                     int64_t kv_row_stride, int64_t row_begin, int64_t n_keys, void* out,
                                     int out_dtype, int64_t out_head_stride, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(h != nullptr && h->bound, "sva_decode_layer_step: handle not bound to its buffers");
  SVA_REQUIRE(q && keys && values && out, "sva_decode_layer_step: null pointer");
  SVA_REQUIRE(n_keys > 0 && n_keys <= h->capacity, "sva_decode_layer_step: %lld keys for a catalog of %lld rows",
              (long long)n_keys, (long long)h->capacity);
  SVA_REQUIRE(row_begin >= 0 && row_begin <= n_keys, "sva_decode_layer_step: rows from %lld of %lld",
              (long long)row_begin, (long long)n_keys);
  // the catalog rows the cache gained since the last step (sva/llama.py:597-616):
  // a few rows go with the lookup (inside its kernel on the one-launch path),
  // more are encoded first
  int rc = SVA_OK;
  sva::WriteParams wp;
  const sva::WriteParams* append = nullptr;
  if (n_keys > row_begin) {
    rc = sva::write_encode_setup(keys, kv_dtype, kv_head_stride, kv_row_stride, row_begin, n_keys - row_begin, h->H,
                                 h->G, h->D, h->R, h->S, h->C, h->k_proj, h->codebooks, h->k_low, h->klow_hs,
                                 h->codes, h->code_type, h->code_hs, &wp);
    if (rc != SVA_OK) return rc;
    if (sva::write_few_form(wp) >= 0) {
      append = &wp;
    } else {
      rc = sva::write_encode_launch(wp, (hipStream_t)stream);
      if (rc != SVA_OK) return rc;
    }
  }
  // the lookup and the verifier (sva/llama.py:211-317); only the paths with a
  // sampled floor (strategy 1 and 2) report overshoots, so the per-item path
  // is spared the fill of that row
  const int64_t H = h->H;
  const int strategy = sva_summon_strategy(1, H, 1, n_keys, h->R, h->S, h->C, h->L, h->code_type, 0);
  const bool with_floor = strategy == 1 || strategy == 2;
  // the per-item register path adds the statistics itself (one launch fewer)
  unsigned long long* fused_stats = strategy == 3 ? (unsigned long long*)h->stats : nullptr;
  rc = sva::lookup_verify_impl(q, q_dtype, q_head_stride, H, h->D, h->R, h->S, h->C, h->q_proj, h->scale,
                               h->codebooks, h->codes, h->code_type, h->code_hs, h->k_low, h->klow_hs, n_keys, h->L,
                               nullptr, 0, 0, h->q_low, h->lut, h->range, h->sl_idx, h->sl_rank, h->counts, h->B,
                               h->fin_idx, h->counts + H, h->ws, h->ws_bytes, keys, values, kv_dtype, kv_head_stride,
                               kv_row_stride, h->G, h->scaling, out, out_dtype, out_head_stride, h->vws, h->vws_bytes,
                               with_floor ? h->counts + 2 * H : nullptr, stream, fused_stats, append);
  if (rc != SVA_OK) return rc;
  // the step's statistics (sva/llama.py:319-326), summed on the device
  if (h->stats != nullptr && fused_stats == nullptr) {
    hipLaunchKernelGGL(decode_stats_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, h->counts, (int)H, with_floor,
                       h->stats);
    SVA_CHECK_LAUNCH("decode_stats_kernel");
  }
  return SVA_OK;
}

extern "C" void sva_decode_layer_destroy(sva_decode_layer* h) { delete h; }
