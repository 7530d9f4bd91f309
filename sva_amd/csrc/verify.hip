// Exact verifier, GQA-aware (sva/llama.py:304-317 and :532-553).
//
// verify_partial: one workgroup per (sequence, KV head g, token, split).  The
// budget lists of the H/G query heads sharing g (ascending key indices) are
// read into LDS and concatenated in (head, position) order; split s takes an
// equal slice of that concatenation.  An entry is processed only by the slice
// holding its first occurrence (the lowest head whose list contains the key),
// so every selected K row and V row is read from HBM once per group and is
// scored against every query head whose list holds it.  Scores are fp32
// dot(K[n], q_h) * scaling; each split keeps, per head, the running maximum
// m, the sum z of exp(score - m) and the exp-weighted V sum.
// verify_combine: one workgroup per query item merges the splits
// (max-rescaled sums) and stores acc / z in the output dtype.
#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int VB = 256;            // threads per partial workgroup
constexpr int ROWS_PER_WG = 32;    // union entries per split (2 passes of 16 rows)
constexpr int MAX_GRP = 8;
constexpr int MAX_D = 256;

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
  int H, G, Q, D, B, split;
  float scaling;
  float* part;  // [items, split, D + 2]: m, z, acc[D]
  void* out;
  int out_dtype;
  int64_t o_bs, o_hs, o_ts;
};

__global__ void __launch_bounds__(VB) verify_partial_kernel(VerifyParams p) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int grp = p.H / p.G;
  const int s = blockIdx.x % p.split;
  const int gi = blockIdx.x / p.split;
  const int t = gi % p.Q;
  const int g = (gi / p.Q) % p.G;
  const int b = gi / (p.Q * p.G);
  const int B = p.B, D = p.D;
  int32_t* lists = (int32_t*)lds;                    // [grp][B]
  float* qv = (float*)(lists + grp * B);             // [grp][D]
  float* vrow = qv + grp * D;                        // [ROWS_PER_WG][D]
  float* sc = vrow + ROWS_PER_WG * D;                // [ROWS_PER_WG][grp]
  int32_t* rkey = (int32_t*)(sc + ROWS_PER_WG * grp);  // [ROWS_PER_WG]
  int32_t* rpos = rkey + ROWS_PER_WG;                // [ROWS_PER_WG][grp]
  int* cnt = rpos + ROWS_PER_WG * grp;               // [MAX_GRP + 1] (prefix)
  float* stat = (float*)(cnt + MAX_GRP + 1);         // [grp][2]
  int* nrows = (int*)(stat + 2 * MAX_GRP);

  const int64_t len = p.lens ? p.lens[b] : p.N;
  const int64_t off = p.offs ? p.offs[b] : 0;
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int j = 0; j < grp; ++j) {
      const int64_t item = ((int64_t)b * p.H + g * grp + j) * p.Q + t;
      cnt[j] = acc;
      acc += max(0, min(p.fin_count[item], B));
    }
    cnt[grp] = acc;
  }
  __syncthreads();
  for (int j = 0; j < grp; ++j) {
    const int h = g * grp + j;
    const int64_t item = ((int64_t)b * p.H + h) * p.Q + t;
    const int c = cnt[j + 1] - cnt[j];
    const int32_t* src = p.fin_idx + item * B;
    for (int i = threadIdx.x; i < c; i += VB) {
      int32_t x = src[i];
      x = x < 0 ? 0 : (x >= len ? (int32_t)(len - 1) : x);
      lists[j * B + i] = x;
    }
    const int64_t qb = (int64_t)b * p.q_bs + (int64_t)h * p.q_hs + (int64_t)t * p.q_ts;
    for (int d = threadIdx.x; d < D; d += VB) qv[j * D + d] = load_elem(p.q, qb + d, p.q_dtype);
  }
  __syncthreads();

  // this split's slice of the concatenated lists; keep first occurrences
  const int M = cnt[grp];
  const int e0 = (int)((int64_t)s * M / p.split);
  const int e1 = (int)((int64_t)(s + 1) * M / p.split);
  if (threadIdx.x < WAVE) {
    const int e = e0 + (int)threadIdx.x;
    bool own = false;
    int j = 0, i = 0;
    int32_t x = 0;
    if (e < e1) {
      while (j + 1 < grp && e >= cnt[j + 1]) ++j;
      i = e - cnt[j];
      x = lists[j * B + i];
      own = true;
      for (int jj = 0; jj < j && own; ++jj)
        if (bsearch_i32(lists + jj * B, cnt[jj + 1] - cnt[jj], x) >= 0) own = false;
    }
    const uint64_t bal = __ballot(own);
    const int r = (int)__popcll(bal & ((1ull << lane_id()) - 1ull));
    if (own && r < ROWS_PER_WG) {
      rkey[r] = x;
      for (int jj = 0; jj < grp; ++jj)
        rpos[r * grp + jj] = jj < j ? -1 : (jj == j ? i : bsearch_i32(lists + jj * B, cnt[jj + 1] - cnt[jj], x));
    }
    if (threadIdx.x == 0) *nrows = min((int)__popcll(bal), ROWS_PER_WG);
  }
  __syncthreads();
  const int n = *nrows;

  // scores: 16 lanes per row, each lane a D/16 slice; V slice kept in LDS
  const int grp16 = threadIdx.x >> 4;  // 16 row slots per pass
  const int l16 = threadIdx.x & 15;
  const int per = D / 16;
  const char* kb = (const char*)p.keys;
  const char* vb = (const char*)p.values;
  const int64_t kv_head = (int64_t)g * p.kv_hs;
  for (int r0 = 0; r0 < n; r0 += VB / 16) {
    const int r = r0 + grp16;
    const bool valid = r < n;
    const int64_t row = off + (valid ? rkey[r] : rkey[0]);
    float kr[MAX_D / 16], vr[MAX_D / 16];
#pragma unroll
    for (int k = 0; k < MAX_D / 16; ++k) {
      if (k < per) {
        const int64_t e = kv_head + row * p.kv_rs + l16 * per + k;
        kr[k] = load_elem(kb, e, p.kv_dtype);
        vr[k] = load_elem(vb, e, p.kv_dtype);
      }
    }
    for (int j = 0; j < grp; ++j) {
      float part = 0.0f;
#pragma unroll
      for (int k = 0; k < MAX_D / 16; ++k)
        if (k < per) part += kr[k] * qv[j * D + l16 * per + k];
      for (int o = 8; o > 0; o >>= 1) part += __shfl_xor(part, o, 16);
      if (valid && l16 == 0) sc[r * grp + j] = part * p.scaling;
    }
    if (valid) {
#pragma unroll
      for (int k = 0; k < MAX_D / 16; ++k)
        if (k < per) vrow[r * D + l16 * per + k] = vr[k];
    }
  }
  __syncthreads();

  // per-head max and exp-sum over this split's rows (fixed order)
  if ((int)threadIdx.x < grp) {
    const int j = threadIdx.x;
    float m = -INFINITY;
    for (int r = 0; r < n; ++r)
      if (rpos[r * grp + j] >= 0) m = fmaxf(m, sc[r * grp + j]);
    float z = 0.0f;
    for (int r = 0; r < n; ++r) {
      if (rpos[r * grp + j] >= 0) {
        const float w = expf(sc[r * grp + j] - m);
        sc[r * grp + j] = w;
        z += w;
      } else {
        sc[r * grp + j] = 0.0f;
      }
    }
    stat[2 * j] = m;
    stat[2 * j + 1] = z;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < grp * D; e += VB) {
    const int j = e / D, d = e % D;
    float acc = 0.0f;
    for (int r = 0; r < n; ++r) acc += sc[r * grp + j] * vrow[r * D + d];
    const int64_t item = ((int64_t)b * p.H + g * grp + j) * p.Q + t;
    float* dst = p.part + (item * p.split + s) * (D + 2);
    dst[2 + d] = acc;
    if (d == 0) {
      dst[0] = stat[2 * j];
      dst[1] = stat[2 * j + 1];
    }
  }
}

__global__ void __launch_bounds__(MAX_D) verify_combine_kernel(VerifyParams p) {
  const int item = blockIdx.x;
  const int t = item % p.Q;
  const int h = (item / p.Q) % p.H;
  const int b = item / (p.Q * p.H);
  const int D = p.D;
  const float* src = p.part + (int64_t)item * p.split * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < p.split; ++s) M = fmaxf(M, src[s * (D + 2)]);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float z = 0.0f, acc = 0.0f;
    if (M > -INFINITY) {
      for (int s = 0; s < p.split; ++s) {
        const float m = src[s * (D + 2)];
        if (m == -INFINITY) continue;
        const float f = expf(m - M);
        z += src[s * (D + 2) + 1] * f;
        acc += src[s * (D + 2) + 2 + d] * f;
      }
    }
    const float v = z > 0.0f ? acc / z : 0.0f;
    const int64_t o = (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)t * p.o_ts + d;
    store_elem(p.out, o, p.out_dtype, v);
  }
}

int verify_split(int64_t grp, int64_t B) {
  const int64_t m = grp * B;
  return (int)std::max<int64_t>(1, (m + ROWS_PER_WG - 1) / ROWS_PER_WG);
}

size_t verify_lds_bytes(int64_t grp, int64_t B, int64_t D) {
  return sizeof(int32_t) * grp * B + sizeof(float) * grp * D + sizeof(float) * ROWS_PER_WG * D +
         sizeof(float) * ROWS_PER_WG * grp + sizeof(int32_t) * ROWS_PER_WG + sizeof(int32_t) * ROWS_PER_WG * grp +
         sizeof(int) * (MAX_GRP + 1) + sizeof(float) * 2 * MAX_GRP + sizeof(int) + 16;
}

}  // namespace

extern "C" size_t sva_verify_workspace_bytes(int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D, int64_t B) {
  if (n_seq <= 0 || H <= 0 || G <= 0 || Q <= 0 || D <= 0 || B <= 0 || H % G != 0) return 0;
  return sizeof(float) * (size_t)(n_seq * H * Q) * (size_t)verify_split(H / G, B) * (size_t)(D + 2) + 256;
}

extern "C" int sva_verify(const void* q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride,
                          int64_t q_tok_stride, const void* keys, const void* values, int kv_dtype,
                          int64_t kv_head_stride, int64_t kv_row_stride, const int64_t* seq_offsets,
                          const int64_t* seq_lens, int64_t n_keys, const int32_t* fin_idx, const int32_t* fin_count,
                          int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D, int64_t B, float scaling,
                          void* out, int out_dtype, int64_t out_seq_stride, int64_t out_head_stride,
                          int64_t out_tok_stride, void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(q && keys && values && fin_idx && fin_count && out, "sva_verify: null pointer");
  SVA_REQUIRE((seq_offsets == nullptr) == (seq_lens == nullptr), "sva_verify: offsets and lengths go together");
  SVA_REQUIRE(n_seq > 0 && H > 0 && G > 0 && Q > 0 && B > 0 && n_keys > 0, "sva_verify: bad sizes");
  SVA_REQUIRE(H % G == 0 && H / G <= MAX_GRP, "sva_verify: %lld query heads over %lld KV heads unsupported",
              (long long)H, (long long)G);
  SVA_REQUIRE(D > 0 && D <= MAX_D && D % 16 == 0, "sva_verify: head_dim %lld must be a multiple of 16 up to %d",
              (long long)D, MAX_D);
  SVA_REQUIRE(q_dtype >= 0 && q_dtype <= 2 && kv_dtype >= 0 && kv_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
              "sva_verify: bad dtype");
  const int64_t grp = H / G;
  const size_t lds = verify_lds_bytes(grp, B, D);
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_verify: budget %lld with %lld heads per KV head exceeds LDS",
                  (long long)B, (long long)grp);
  const size_t need = sva_verify_workspace_bytes(n_seq, H, G, Q, D, B);
  SVA_REQUIRE(workspace != nullptr && workspace_bytes >= need, "sva_verify: workspace of %zu bytes required", need);
  const int split = verify_split(grp, B);
  const int64_t blocks = n_seq * G * Q * split;
  SVA_REQUIRE(blocks < (1ll << 31), "sva_verify: too many items");
  static bool attr_set = false;
  if (!attr_set) {
    SVA_CHECK_HIP(hipFuncSetAttribute((const void*)verify_partial_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, sva::kMaxLds),
                  "hipFuncSetAttribute(verify_partial_kernel)");
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
  p.split = split;
  p.scaling = scaling;
  p.part = (float*)workspace;
  p.out = out;
  p.out_dtype = out_dtype;
  p.o_bs = out_seq_stride;
  p.o_hs = out_head_stride;
  p.o_ts = out_tok_stride;
  hipLaunchKernelGGL(verify_partial_kernel, dim3((unsigned)blocks), dim3(VB), lds, (hipStream_t)stream, p);
  SVA_CHECK_LAUNCH("verify_partial_kernel");
  hipLaunchKernelGGL(verify_combine_kernel, dim3((unsigned)(n_seq * H * Q)), dim3(MAX_D), 0, (hipStream_t)stream, p);
  SVA_CHECK_LAUNCH("verify_combine_kernel");
  return SVA_OK;
}
