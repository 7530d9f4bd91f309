// Parameters shared by the two summon strategies (per-item and wide).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sva {

constexpr int kMaxLds = 160 * 1024;  // LDS per workgroup on gfx950

// Sampled shortlist-floor estimate of a single-query uint8 scan, computed by
// the query table kernel: `blocks` contiguous blocks of SAMPLE_KEYS keys
// spread over the cache (one block per 256 keys, at least SAMPLE_MIN_BLOCKS,
// at most SAMPLE_MAX_BLOCKS and SAMPLE_MAX_BYTES of codes), a histogram of their sums over
// SAMPLE_BINS bins, and the bin of the k-th largest sum, k chosen so that
// about max(SAMPLE_TARGET * L, SAMPLE_MIN_CAND) keys reach the floor.  The
// floor is only a hint: an overshoot (fewer than L keys above it) costs the
// slower all-keys select, never a result.  With n_s samples, the number of
// samples above the L-th largest key is ~Poisson(n_s L / N); k is about
// twice that mean and at least SAMPLE_MIN_RANK, so an overshoot is rare
// (about 1e-4 at 1M keys, L = 2048, 8K samples).
constexpr int SAMPLE_KEYS = 32;
constexpr int SAMPLE_BINS = 1024;
constexpr int SAMPLE_MIN_BLOCKS = 64;
constexpr int SAMPLE_MAX_BYTES = 32768;
constexpr int SAMPLE_MAX_BLOCKS = 256;  // at most 8K sampled keys
constexpr double SAMPLE_TARGET = 2.0;
constexpr double SAMPLE_MIN_CAND = 4096.0;
constexpr int SAMPLE_MIN_RANK = 16;
constexpr int SAMPLE_MAX_S = 8;  // subspaces of the sampled scan

// Sample blocks for a cache of n_keys keys with S subspaces.
__host__ __device__ inline int sample_blocks(int64_t n_keys, int64_t S) {
  int64_t cap = SAMPLE_MAX_BYTES / (SAMPLE_KEYS * S);
  cap = cap < SAMPLE_MAX_BLOCKS ? cap : SAMPLE_MAX_BLOCKS;
  int64_t b = n_keys / 256;
  b = b < SAMPLE_MIN_BLOCKS ? SAMPLE_MIN_BLOCKS : b;
  return (int)(b < cap ? b : cap);
}

// Rank of the sampled floor among n_samples sampled sums for a shortlist of
// L over n_keys keys; 0: no sampled floor (every key is a candidate).
__host__ __device__ inline int sample_floor_rank(int64_t L, int64_t n_keys, int n_samples) {
  if (n_samples <= 0 || n_keys < 4 * (int64_t)n_samples) return 0;
  double target = SAMPLE_TARGET * (double)L;
  if (target < SAMPLE_MIN_CAND) target = SAMPLE_MIN_CAND;
  int k = (int)(target * (double)n_samples / (double)n_keys) + 1;
  k = k < SAMPLE_MIN_RANK ? SAMPLE_MIN_RANK : k;
  return k < n_samples / 2 ? k : 0;
}

struct QueryLaunch;  // query.h: a prepared query launch the class path may fuse
struct WriteParams;  // write_few.cuh: a prepared catalog append of a few rows

struct SummonParams {
  const float* lut;    // [items, S*C]
  const float* range;  // [items, 4]: bounds of any scan sum, sampled floor, 0
  const float* q_low;  // [items, R]
  const void* codes;
  int ctype;
  int64_t code_hs;
  const float* k_low;
  int64_t klow_hs;
  const int64_t* offs;
  const int64_t* lens;
  int H, Q;
  int64_t N;  // keys of the single sequence, or the longest sequence
  int R, S, C, L;
  const void* mask;
  int mask_type;
  int64_t mask_ts;
  float sqrt_r;
  int32_t* sl_idx;
  float* sl_rank;
  int32_t* sl_count;
  // optional budget select fused into the summon (B = 0: none)
  int B;
  int32_t* fin_idx;
  int32_t* fin_count;
  // optional int64 [4] statistics row the per-item path adds each item's
  // counts to (summoned, verified, -, queries); nullptr: none
  unsigned long long* stats;
};

// The exact verifier run by the wide path's finish kernel right after each
// item's budget list (one sequence, one query token: item = query head h):
// q of head h at q + h * q_hs; K / V rows of KV head g = h / (H / G) at
// g * kv_hs + n * kv_rs; out of head h at out + h * o_hs.  D is 64 or 128.
struct FusedVerify {
  const void* q;
  int q_dtype;
  int64_t q_hs;
  const void* keys;
  const void* values;
  int kv_dtype;
  int64_t kv_hs, kv_rs;
  bool kv_vec;  // rows start 8-byte (half types) / 16-byte (fp32) aligned
  int G, D;
  float scaling;
  void* out;  // nullptr: no fused verifier
  int out_dtype;
  int64_t o_hs;
};

int summon_item_path(const SummonParams& p, int64_t items, hipStream_t stream);
bool summon_regs_eligible(const SummonParams& p);
int summon_regs_path(const SummonParams& p, int64_t items, hipStream_t stream);
// One token of one sequence on the per-item register path with the verifier
// (lookup_item.hip): the prepared catalog append of a few rows (optional),
// the prepared decode query, the summon and the verifier in one launch when
// item_fused_eligible holds for them.  overshoot (optional, [H]) is cleared:
// the per-item path has no sampled floor.
bool item_fused_eligible(const SummonParams& p, const QueryLaunch& ql, const FusedVerify& fv,
                         const WriteParams* append);
int item_lookup_verify_path(const QueryLaunch& ql, const SummonParams& p, const FusedVerify& fv,
                            const WriteParams* append, int32_t* overshoot, hipStream_t stream);
// sva_lookup_verify, adding each query head's counts to `stats` (an int64 [4]
// row: summoned, verified, -, queries) when it is not null: only where the
// per-item register path serves the shape (sva_summon_strategy 3).  append
// (optional): a prepared few-row catalog append (write_encode_setup) that
// must land before the lookup reads the catalog; it runs inside the lookup's
// kernel where the one-launch path serves the shape, else first on its own.
// The caller clears the error state.
int lookup_verify_impl(const void* q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R,
                       int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                       const void* codes, int code_type, int64_t code_head_stride, const float* k_low,
                       int64_t k_low_head_stride, int64_t n_keys, int64_t L, const void* mask, int mask_type,
                       int64_t mask_tok_stride, float* q_low, float* lut, float* score_range,
                       int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx,
                       int32_t* fin_count, void* workspace, size_t workspace_bytes, const void* keys,
                       const void* values, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                       int64_t G, float scaling, void* out, int out_dtype, int64_t out_head_stride,
                       void* verify_workspace, size_t verify_workspace_bytes, int32_t* floor_overshoot,
                       void* stream, unsigned long long* stats, const WriteParams* append = nullptr);
// ordered: every shortlist is in ascending key order (the per-item summon's),
// so the budget is compacted in slot order rather than sorted.
int budget_select_launch(const int32_t* sl_idx, const float* sl_rank, const int32_t* sl_count, int64_t n_items,
                         int64_t L, int64_t B, int32_t* fin_idx, int32_t* fin_count, bool ordered,
                         hipStream_t stream);
bool summon_wide_eligible(const SummonParams& p, int64_t items);
// overshoot (optional, [items]): 1 where the sampled floor overshot and the
// finish selected over every key, else 0.
int summon_wide_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream,
                     const FusedVerify* fv = nullptr, int32_t* overshoot = nullptr);
// One subspace of at most 256 codewords with a shortlist of at most
// CLASS_MAX_L: the wide path selects by code class (no sampled floor needed).
constexpr int CLASS_MAX_L = 7168;
inline bool class_shape(int64_t S, int64_t C, int64_t L) { return S == 1 && C <= 256 && L <= CLASS_MAX_L; }
bool summon_class_eligible(const SummonParams& p, int64_t items);
int summon_class_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream,
                      const FusedVerify* fv = nullptr, int32_t* overshoot = nullptr,
                      const QueryLaunch* query = nullptr);
// Whether summon_wide_path can run `fv` in its finish kernel for these sizes.
bool fused_verify_eligible(const SummonParams& p, int64_t items, const FusedVerify& fv);
size_t summon_wide_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t L);

inline int next_pow2_host(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// Fills n int32 with a value on the stream (graph-capture safe, no memset node).
int fill_i32(int32_t* ptr, int64_t n, int32_t value, hipStream_t stream);
int fill_u32(uint32_t* ptr, int64_t n, uint32_t value, hipStream_t stream);

}  // namespace sva
