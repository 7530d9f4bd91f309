// Parameters shared by the two summon strategies (per-item and wide).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sva {

constexpr int kMaxLds = 160 * 1024;  // LDS per workgroup on gfx950

// Sampled shortlist-floor estimate of a single-query uint8 scan (the query
// table kernel and the fused lookup compute it alike): SAMPLE_BLOCKS
// contiguous blocks of SAMPLE_KEYS keys spread over the cache, a histogram of
// their sums over SAMPLE_BINS bins, and the bin of the k-th largest, k ~
// max(SAMPLE_TARGET * L, SAMPLE_MIN_CAND) * samples / N.  The floor is only a
// hint (an overshoot, fewer than L keys above it, costs the slow all-keys
// select, never a result): the minimum keeps k >= ~12 for small shortlists,
// where the k-th largest of few samples would overshoot often.
constexpr int SAMPLE_BLOCKS = 64;
constexpr int SAMPLE_KEYS = 32;
constexpr int SAMPLE_BINS = 1024;
constexpr double SAMPLE_TARGET = 3.5;
constexpr double SAMPLE_MIN_CAND = 6144.0;
constexpr int SAMPLE_MAX_S = 8;  // subspaces of the sampled scan
constexpr int N_SAMPLE = SAMPLE_BLOCKS * SAMPLE_KEYS;

// Rank of the sampled floor among the N_SAMPLE sampled sums for a shortlist
// of L over n_keys keys; 0: no sampled floor (every key is a candidate).
__host__ __device__ inline int sample_floor_rank(int64_t L, int64_t n_keys) {
  if (n_keys < 4 * (int64_t)N_SAMPLE) return 0;
  double target = SAMPLE_TARGET * (double)L;
  if (target < SAMPLE_MIN_CAND) target = SAMPLE_MIN_CAND;
  const int k = (int)(target * (double)N_SAMPLE / (double)n_keys) + 1;
  return k < N_SAMPLE / 2 ? k : 0;
}

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
};

// Query side of the fused lookup (sva_lookup_select): the scan computes the
// item's q_low, table, bounds and sampled floor itself and writes them to
// q_low / lut / range.
struct FusedQuery {
  const void* q;
  int q_dtype;
  int64_t q_hs;  // head stride of q (one sequence, one token)
  int64_t D;
  const float* q_proj;
  const float* scale;
  const float* codebooks;
  int sample_k;  // rank of the sampled floor among the samples; 0: no sampled floor
};

int summon_item_path(const SummonParams& p, int64_t items, hipStream_t stream);
bool summon_regs_eligible(const SummonParams& p);
int summon_regs_path(const SummonParams& p, int64_t items, hipStream_t stream);
int budget_select_launch(const int32_t* sl_idx, const float* sl_rank, const int32_t* sl_count, int64_t n_items,
                         int64_t L, int64_t B, int32_t* fin_idx, int32_t* fin_count, hipStream_t stream);
bool summon_wide_eligible(const SummonParams& p, int64_t items);
bool summon_wide_fused_eligible(const SummonParams& p, const FusedQuery& f);
int summon_wide_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream,
                     const FusedQuery* f = nullptr);
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
