// Exact verifier, GQA-aware (sva/llama.py:304-317 and :532-553).
//
// One workgroup per (sequence, KV head g, token).  The budget lists of the
// H/G query heads sharing g are loaded (ascending key indices); the union of
// the lists is formed in a deterministic order (an entry is kept by the first
// list that contains it); each union row of K and of V is read from HBM once
// and used by every query head whose list holds it.  Scores are fp32
// dot(K[n], q_h) * scaling; softmax and the weighted V sum run in fp32 and the
// result is stored in the output dtype.
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int VER_BLOCK = 256;
constexpr int VER_WAVES = VER_BLOCK / WAVE;
constexpr int MAX_GRP = 8;
constexpr int MAX_DCH = 4;  // head_dim up to 256 (4 chunks of 64 lanes)
constexpr int ROW_UNROLL = 4;

SVA_DEV int bsearch_i32(const int32_t* a, int n, int32_t x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  return (lo < n && a[lo] == x) ? lo : -1;
}

struct VerifyParams {
  const void* q;
  int q_dtype;
  int64_t q_bs, q_hs, q_ts;
  const void* keys;
  const void* values;
  int kv_dtype;
  int64_t kv_hs, kv_rs;
  const int64_t* offs;
  const int64_t* lens;
  int64_t N;
  const int32_t* fin_idx;
  const int32_t* fin_count;
  int H, G, Q, D, B;
  float scaling;
  void* out;
  int out_dtype;
  int64_t o_bs, o_hs, o_ts;
};

__global__ void __launch_bounds__(VER_BLOCK) verify_kernel(VerifyParams p) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int grp = p.H / p.G;
  const int t = blockIdx.x % p.Q;
  const int g = (blockIdx.x / p.Q) % p.G;
  const int b = blockIdx.x / (p.Q * p.G);
  const int B = p.B, D = p.D;
  int32_t* lists = (int32_t*)lds;                   // [grp][B]
  int32_t* uni = lists + grp * B;                    // [grp*B]
  float* sc = (float*)(uni + grp * B);               // [grp][B]
  float* qv = sc + grp * B;                          // [grp][D]
  float* red = qv + grp * D;                         // [VER_WAVES][grp][D]
  uint32_t* scratch = (uint32_t*)(red + VER_WAVES * grp * D);  // [VER_WAVES + 1]
  float* fred = (float*)(scratch + VER_WAVES + 1);             // [VER_BLOCK]
  int* cnt = (int*)(fred + VER_BLOCK);                         // [MAX_GRP]
  float* stat = (float*)(cnt + MAX_GRP);                       // [2*MAX_GRP]: max, sum

  const int64_t len = p.lens ? p.lens[b] : p.N;
  const int64_t off = p.offs ? p.offs[b] : 0;
  for (int j = 0; j < grp; ++j) {
    const int h = g * grp + j;
    const int64_t item = ((int64_t)b * p.H + h) * p.Q + t;
    const int c = min(p.fin_count[item], B);
    if (threadIdx.x == 0) cnt[j] = c;
    const int32_t* src = p.fin_idx + item * B;
    for (int i = threadIdx.x; i < c; i += VER_BLOCK) {
      int32_t x = src[i];
      x = x < 0 ? 0 : (x >= len ? (int32_t)(len - 1) : x);
      lists[j * B + i] = x;
    }
    const int64_t qb = (int64_t)b * p.q_bs + (int64_t)h * p.q_hs + (int64_t)t * p.q_ts;
    for (int d = threadIdx.x; d < D; d += VER_BLOCK) qv[j * D + d] = load_elem(p.q, qb + d, p.q_dtype);
  }
  __syncthreads();

  // union of the lists in (list, position) order: an entry is kept by the
  // first list that holds its key index
  uint32_t n_uni = 0;
  for (int base = 0; base < grp * B; base += VER_BLOCK) {
    const int e = base + threadIdx.x;
    uint32_t own = 0;
    int32_t x = 0;
    if (e < grp * B) {
      const int j = e / B, i = e % B;
      if (i < cnt[j]) {
        x = lists[j * B + i];
        own = 1;
        for (int jj = 0; jj < j && own; ++jj)
          if (bsearch_i32(lists + jj * B, cnt[jj], x) >= 0) own = 0;
      }
    }
    uint32_t tot;
    const uint32_t pos = block_excl_scan<VER_BLOCK>(own, scratch, &tot);
    if (own) uni[n_uni + pos] = x;
    n_uni += tot;
  }
  __syncthreads();

  const int wid = threadIdx.x / WAVE;
  const int lane = lane_id();
  const int dch = (D + WAVE - 1) / WAVE;
  const char* kbase = (const char*)p.keys;
  const char* vbase = (const char*)p.values;
  const int64_t kv_head = (int64_t)g * p.kv_hs;

  // scores: each union row of K is read once, scored for every head holding it
  for (int u0 = wid * ROW_UNROLL; u0 < (int)n_uni; u0 += VER_WAVES * ROW_UNROLL) {
    float kr[ROW_UNROLL][MAX_DCH];
#pragma unroll
    for (int r = 0; r < ROW_UNROLL; ++r) {
      const int u = u0 + r;
      const int64_t row = u < (int)n_uni ? (off + uni[u]) : off;
#pragma unroll
      for (int k = 0; k < MAX_DCH; ++k) {
        const int d = lane + k * WAVE;
        kr[r][k] = (k < dch && d < D && u < (int)n_uni) ? load_elem(kbase, kv_head + row * p.kv_rs + d, p.kv_dtype) : 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < ROW_UNROLL; ++r) {
      const int u = u0 + r;
      if (u >= (int)n_uni) break;
      const int32_t x = uni[u];
      for (int j = 0; j < grp; ++j) {
        const int pos = bsearch_i32(lists + j * B, cnt[j], x);
        if (pos < 0) continue;
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < MAX_DCH; ++k) {
          const int d = lane + k * WAVE;
          if (k < dch && d < D) part += kr[r][k] * qv[j * D + d];
        }
        const float s = wave_sum(part);
        if (lane == 0) sc[j * B + pos] = s * p.scaling;
      }
    }
  }
  __syncthreads();

  // softmax statistics per head (deterministic block reductions)
  for (int j = 0; j < grp; ++j) {
    float m = -INFINITY;
    for (int i = threadIdx.x; i < cnt[j]; i += VER_BLOCK) m = fmaxf(m, sc[j * B + i]);
    fred[threadIdx.x] = m;
    __syncthreads();
    for (int s = VER_BLOCK / 2; s > 0; s >>= 1) {
      if ((int)threadIdx.x < s) fred[threadIdx.x] = fmaxf(fred[threadIdx.x], fred[threadIdx.x + s]);
      __syncthreads();
    }
    const float mx = fred[0];
    __syncthreads();
    float z = 0.0f;
    for (int i = threadIdx.x; i < cnt[j]; i += VER_BLOCK) {
      const float w = expf(sc[j * B + i] - mx);
      sc[j * B + i] = w;
      z += w;
    }
    fred[threadIdx.x] = z;
    __syncthreads();
    for (int s = VER_BLOCK / 2; s > 0; s >>= 1) {
      if ((int)threadIdx.x < s) fred[threadIdx.x] += fred[threadIdx.x + s];
      __syncthreads();
    }
    if (threadIdx.x == 0) stat[j] = fred[0];
    __syncthreads();
  }

  // weighted V sum: each union row of V is read once
  float acc[MAX_GRP][MAX_DCH];
#pragma unroll
  for (int j = 0; j < MAX_GRP; ++j)
#pragma unroll
    for (int k = 0; k < MAX_DCH; ++k) acc[j][k] = 0.0f;
  for (int u0 = wid * ROW_UNROLL; u0 < (int)n_uni; u0 += VER_WAVES * ROW_UNROLL) {
    float vr[ROW_UNROLL][MAX_DCH];
#pragma unroll
    for (int r = 0; r < ROW_UNROLL; ++r) {
      const int u = u0 + r;
      const int64_t row = u < (int)n_uni ? (off + uni[u]) : off;
#pragma unroll
      for (int k = 0; k < MAX_DCH; ++k) {
        const int d = lane + k * WAVE;
        vr[r][k] = (k < dch && d < D && u < (int)n_uni) ? load_elem(vbase, kv_head + row * p.kv_rs + d, p.kv_dtype) : 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < ROW_UNROLL; ++r) {
      const int u = u0 + r;
      if (u >= (int)n_uni) break;
      const int32_t x = uni[u];
#pragma unroll
      for (int j = 0; j < MAX_GRP; ++j) {
        if (j >= grp) break;
        const int pos = bsearch_i32(lists + j * B, cnt[j], x);
        if (pos < 0) continue;
        const float w = sc[j * B + pos];
#pragma unroll
        for (int k = 0; k < MAX_DCH; ++k) acc[j][k] += w * vr[r][k];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < MAX_GRP; ++j) {
    if (j >= grp) break;
#pragma unroll
    for (int k = 0; k < MAX_DCH; ++k) {
      const int d = lane + k * WAVE;
      if (k < dch && d < D) red[(wid * grp + j) * D + d] = acc[j][k];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < grp * D; e += VER_BLOCK) {
    const int j = e / D, d = e % D;
    float s = 0.0f;
    for (int w = 0; w < VER_WAVES; ++w) s += red[(w * grp + j) * D + d];
    const int h = g * grp + j;
    const float z = stat[j];
    const float v = cnt[j] > 0 ? s / z : 0.0f;
    const int64_t o = (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)t * p.o_ts + d;
    store_elem(p.out, o, p.out_dtype, v);
  }
}

}  // namespace

extern "C" int sva_verify(const void* q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride,
                          int64_t q_tok_stride, const void* keys, const void* values, int kv_dtype,
                          int64_t kv_head_stride, int64_t kv_row_stride, const int64_t* seq_offsets,
                          const int64_t* seq_lens, int64_t n_keys, const int32_t* fin_idx, const int32_t* fin_count,
                          int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D, int64_t B, float scaling,
                          void* out, int out_dtype, int64_t out_seq_stride, int64_t out_head_stride,
                          int64_t out_tok_stride, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(q && keys && values && fin_idx && fin_count && out, "sva_verify: null pointer");
  SVA_REQUIRE((seq_offsets == nullptr) == (seq_lens == nullptr), "sva_verify: offsets and lengths go together");
  SVA_REQUIRE(n_seq > 0 && H > 0 && G > 0 && Q > 0 && B > 0 && n_keys > 0, "sva_verify: bad sizes");
  SVA_REQUIRE(H % G == 0 && H / G <= MAX_GRP, "sva_verify: %lld query heads over %lld KV heads unsupported",
              (long long)H, (long long)G);
  SVA_REQUIRE(D > 0 && D <= WAVE * MAX_DCH, "sva_verify: head_dim %lld out of range", (long long)D);
  SVA_REQUIRE(q_dtype >= 0 && q_dtype <= 2 && kv_dtype >= 0 && kv_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
              "sva_verify: bad dtype");
  const int64_t grp = H / G;
  const size_t lds = sizeof(int32_t) * 2 * grp * B + sizeof(float) * grp * B + sizeof(float) * grp * D +
                     sizeof(float) * VER_WAVES * grp * D + sizeof(uint32_t) * (VER_WAVES + 1) +
                     sizeof(float) * VER_BLOCK + sizeof(int) * MAX_GRP + sizeof(float) * 2 * MAX_GRP;
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_verify: budget %lld with %lld heads per KV head exceeds LDS",
                  (long long)B, (long long)grp);
  const int64_t blocks = n_seq * G * Q;
  SVA_REQUIRE(blocks < (1ll << 31), "sva_verify: too many items");
  static bool attr_set = false;
  if (!attr_set) {
    SVA_CHECK_HIP(hipFuncSetAttribute((const void*)verify_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      sva::kMaxLds),
                  "hipFuncSetAttribute(verify_kernel)");
    attr_set = true;
  }
  VerifyParams p;
  p.q = q;
  p.q_dtype = q_dtype;
  p.q_bs = q_seq_stride;
  p.q_hs = q_head_stride;
  p.q_ts = q_tok_stride;
  p.keys = keys;
  p.values = values;
  p.kv_dtype = kv_dtype;
  p.kv_hs = kv_head_stride;
  p.kv_rs = kv_row_stride;
  p.offs = seq_offsets;
  p.lens = seq_lens;
  p.N = n_keys;
  p.fin_idx = fin_idx;
  p.fin_count = fin_count;
  p.H = (int)H;
  p.G = (int)G;
  p.Q = (int)Q;
  p.D = (int)D;
  p.B = (int)B;
  p.scaling = scaling;
  p.out = out;
  p.out_dtype = out_dtype;
  p.o_bs = out_seq_stride;
  p.o_hs = out_head_stride;
  p.o_ts = out_tok_stride;
  hipLaunchKernelGGL(verify_kernel, dim3((unsigned)blocks), dim3(VER_BLOCK), lds, (hipStream_t)stream, p);
  SVA_CHECK_LAUNCH("verify_kernel");
  return SVA_OK;
}
