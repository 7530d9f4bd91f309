#pragma once
// Parameters of the query kernels (q_low, the PQ table, score bounds and the
// sampled floor) and the split of sva_query_lut into a host-side setup and a
// launch, so that a caller can run the decode form inside another grid.
#include <cstddef>
#include <cstdint>

#include <hip/hip_runtime.h>

namespace sva {

struct LutParams {
  const void* q;
  int q_dtype;
  int64_t q_bs, q_hs, q_ts;
  int H, Q, D, R, S, C;
  const float* q_proj;
  const float* scale;
  const float* codebooks;
  float* q_low;
  float* lut;
  float* range;  // [items, 4]
  const void* codes;  // optional uint8 codes: sample for the threshold estimate
  int64_t code_hs;
  int64_t n_keys;
  int sample_blocks;  // blocks of SAMPLE_KEYS sampled keys (codes != nullptr)
  int sample_k;       // rank of the floor among the sampled sums; 0: no floor
};

// The kernel an sva_query_lut call launches.
enum QueryForm : int {
  QUERY_GENERAL = 0,     // query_lut_kernel, one 1024-thread workgroup per item
  QUERY_MULTI16 = 1,     // query_lut_multi_kernel, MT tokens per workgroup (sub = 16, 32, 64)
  QUERY_MULTI32 = 2,
  QUERY_MULTI64 = 3,
  QUERY_DECODE_4_64 = 4,  // query_decode_kernel: one token, D = R = 64, 4x64 / 2x256 / 1x256 codes
  QUERY_DECODE_2_256 = 5,
  QUERY_DECODE_1_256 = 6,
  QUERY_MFMA16 = 7,      // query_lut_mfma_kernel: the multi form on fp32 MFMA (D % 4, R % 16, C % 16 == 0)
  QUERY_MFMA32 = 8,
  QUERY_MFMA64 = 9,
};

struct QueryLaunch {
  LutParams p;
  int form;
  int64_t blocks;  // workgroups (general: items; multi: per MT tokens; decode: heads)
  size_t lds;      // dynamic LDS bytes (general and multi forms)
};

// The validation and parameters of sva_query_lut (same arguments); SVA_OK or
// an error code with the message set.
int query_lut_setup(const void* q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride, int64_t q_tok_stride,
                    int64_t n_seq, int64_t H, int64_t Q, int64_t D, int64_t R, int64_t S, int64_t C,
                    const float* q_proj, const float* scale, const float* codebooks, const void* codes, int code_type,
                    int64_t code_head_stride, int64_t n_keys, int64_t shortlist, float* q_low, float* lut,
                    float* score_range, QueryLaunch* out);

// Launches the kernel of a prepared call.
int query_lut_launch(const QueryLaunch& ql, hipStream_t stream);

}  // namespace sva
