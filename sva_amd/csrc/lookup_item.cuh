#pragma once
// One token of one sequence on the per-item register path (caches of up to
// 16K keys, sva_summon_strategy 3), the whole lookup in one launch: one
// 1024-thread workgroup per query head runs, optionally, the catalog append
// of the cache's new rows for its head (sva/llama.py:597-616), then the
// decode query (q_low, the table, the score bounds and the sampled floor,
// :66-74, :211), the summon (shortlist, rescore and budget, :270-302) and the
// verifier over the budget it chose (:304-317).  Four launches become one: a
// decode step of a model with a few thousand cached keys is bound by the
// host's launch cost, not by these kernels.  The arithmetic is that of the separate
// kernels (the same device functions), so the selections and the tables are
// bit-identical to theirs.
#include "query_decode.cuh"
#include "summon_regs.cuh"
#include "summon_wide.cuh"
#include "write_few.cuh"

namespace sva {
namespace item_lookup {

// Dynamic LDS of the fused kernel, beside the decode query's static arrays
// (about 23 KB): the summon's layout, then the verifier's, in the same bytes.
constexpr size_t kDynLds = 64 * 1024;

// Whether a variant runs the catalog append of a decode step (the fp32 K / V
// verifier leaves no registers for it).
template <int VKV>
constexpr bool kAppends = VKV != F32;

template <int NPT, int S, int VD, int VKV>
__global__ void __launch_bounds__(ITEM_BLOCK) item_lookup_verify_kernel(LutParams lp, SummonParams p, FusedVerify fv,
                                                                   WriteParams wp, int32_t* overshoot) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ float qsh[VD];
  const int64_t hx = xcd_range_item((int64_t)blockIdx.x, (int64_t)p.H);
  if (hx < 0) return;  // block-uniform: past the last head
  const int h = (int)hx;
  if (overshoot != nullptr && threadIdx.x == 0) overshoot[h] = 0;  // the per-item path has no sampled floor
  // the verifier's query row, requested first and parked in LDS after the summon
  uint32_t qbits = 0u;
  if ((int)threadIdx.x < VD) qbits = load_elem_bits(fv.q, (int64_t)h * fv.q_hs + threadIdx.x, fv.q_dtype);
  // the head's new catalog rows, read back by the query's sample and the
  // summon (one subspace: codeword rows read in place, 64 floats a thread
  // would spill here; fp32 K / V: no append, its verifier needs the registers)
  if constexpr (kAppends<VKV>) {
    if (wp.n_rows > 0) {  // uniform
      few_append<S == 1 ? 0 : 64 / S, ITEM_BLOCK>(wp, h, 0);
      __syncthreads();
    }
  }
  query_decode_item<S, S == 4 ? 64 : 256, ITEM_BLOCK>(lp, h);
  // the table and q_low this workgroup wrote to global memory, read back by the summon
  __syncthreads();
  const int beff = regs_item<NPT, S>(p, h, lds);
  if ((int)threadIdx.x < VD) qsh[threadIdx.x] = elem_from_bits(qbits, fv.q_dtype);
  // the query row, the budget list the summon wrote, the LDS it used
  __syncthreads();
  wide::verify_item<VD, VKV>(p, fv, h, lds, false, qsh, beff);
}

template <int NPT, int S, int VD, int VKV>
int launch_npt_s(const LutParams& lp, const SummonParams& p, const FusedVerify& fv, const WriteParams& wp,
                 int32_t* overshoot, size_t lds, hipStream_t st) {
  SVA_SET_MAX_LDS_ONCE((item_lookup_verify_kernel<NPT, S, VD, VKV>), kDynLds,
                       "hipFuncSetAttribute(item_lookup_verify_kernel)");
  hipLaunchKernelGGL((item_lookup_verify_kernel<NPT, S, VD, VKV>), dim3((unsigned)xcd_range_grid(p.H)),
                     dim3(ITEM_BLOCK), lds, st, lp, p, fv, wp, overshoot);
  SVA_CHECK_LAUNCH("item_lookup_verify_kernel");
  return SVA_OK;
}

// Keys per thread of the register path for a cache of n keys.
inline int item_npt(int64_t n) { return n <= 4 * ITEM_BLOCK ? 4 : (n <= 8 * ITEM_BLOCK ? 8 : 16); }

// Dynamic LDS bytes of a launch: the summon's layout or the verifier's, whichever is larger.
inline size_t item_lds(const SummonParams& p, int D) {
  return std::max((size_t)reg_lds_layout(p.S, p.C, p.L, item_npt(p.N)).total, wide::verify_item_lds(p.B, D));
}

template <int VD, int VKV>
int launch(const LutParams& lp, const SummonParams& p, const FusedVerify& fv, const WriteParams& wp, int32_t* overshoot,
           hipStream_t st) {
  const int npt = item_npt(p.N);
  const size_t lds = item_lds(p, VD);
  switch (npt * 8 + p.S) {
    case 4 * 8 + 1: return launch_npt_s<4, 1, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 4 * 8 + 2: return launch_npt_s<4, 2, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 4 * 8 + 4: return launch_npt_s<4, 4, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 8 * 8 + 1: return launch_npt_s<8, 1, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 8 * 8 + 2: return launch_npt_s<8, 2, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 8 * 8 + 4: return launch_npt_s<8, 4, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 16 * 8 + 1: return launch_npt_s<16, 1, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 16 * 8 + 2: return launch_npt_s<16, 2, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    case 16 * 8 + 4: return launch_npt_s<16, 4, VD, VKV>(lp, p, fv, wp, overshoot, lds, st);
    default: break;
  }
  SVA_UNSUPPORTED(false, "item_lookup_verify: %d subspaces", p.S);
  return SVA_ERR_UNSUPPORTED;
}

// One translation unit per K / V dtype (lookup_item_v64_<dtype>.hip); head_dim
// is 64, the decode query's.
int launch_v64_bf16(const LutParams& lp, const SummonParams& p, const FusedVerify& fv, const WriteParams& wp,
                    int32_t* overshoot, hipStream_t st);
int launch_v64_f16(const LutParams& lp, const SummonParams& p, const FusedVerify& fv, const WriteParams& wp,
                   int32_t* overshoot, hipStream_t st);
int launch_v64_f32(const LutParams& lp, const SummonParams& p, const FusedVerify& fv, const WriteParams& wp,
                   int32_t* overshoot, hipStream_t st);

}  // namespace item_lookup
}  // namespace sva
