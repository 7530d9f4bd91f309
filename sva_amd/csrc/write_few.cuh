#pragma once
// The catalog append of a decode step (at most FEW_ROWS new cache rows),
// shared by write_encode_few_kernel and the one-launch decode step: k_low by
// the map's fma chain over d and each row's nearest codeword per subspace
// (sva/ops.py:24-47, the order of sva_write_encode's other kernels).
#include "common.cuh"

namespace sva {

struct WriteParams {
  const void* keys;
  int kv_dtype;
  int64_t kv_hs, kv_rs;
  int64_t row0, n_rows;
  int H, G, D, R, S, C;
  const float* k_proj;     // [H, D, R]
  const float* codebooks;  // [H, S, C, sub]
  float* k_low;            // [H, rows, R] (head stride klow_hs)
  int64_t klow_hs;
  void* codes;             // [H, rows, S] (head stride code_hs)
  int ctype;
  int64_t code_hs;
  // a batch of equal-layout caches (sva_write_encode_batch): sequence b's K
  // rows start seq_kv elements after sequence b - 1's, its catalog rows
  // seq_rows rows after; one sequence: n_seq 1, both 0
  int n_seq;
  int64_t seq_kv, seq_rows;
};

// A decode step's append (at most FEW_ROWS rows): one workgroup per head,
// the arithmetic of sva_write_encode's tiled kernels with the work spread
// over the threads instead of over a tile of rows: thread (row, r) forms
// k_low[row][r] by the fma chain over d, then, per subspace and row, thread
// c the distance to codeword c, and the workgroup the first index of the
// least distance (the result does not depend on the thread count).  The
// tiled kernels would stage a 64-row tile's map and codebooks for one row.
constexpr int FEW_ROWS = 4;
constexpr int FEW_MAP = 64 * 64;  // map floats staged in LDS

// Head h's rows [row0, row0 + n_rows) of sequence b of p (n_rows <=
// FEW_ROWS) on this workgroup of NT threads (NT a multiple of WAVE); every
// thread must call it.
template <int SUB, int NT>
SVA_DEV void few_append(const WriteParams& p, int h, int b) {
#pragma clang fp contract(off)
  __shared__ float kr[FEW_ROWS][256];  // the new K rows (D <= 256)
  __shared__ float xl[FEW_ROWS][256];  // their k_low rows (R <= 256)
  __shared__ __align__(16) float ws[FEW_MAP];  // the head's map when D * R <= FEW_MAP
  __shared__ float rbest[NT / WAVE];
  __shared__ int rarg[NT / WAVE];
  const int D = p.D, R = p.R, S = p.S, C = p.C;
  const int sub = SUB > 0 ? SUB : R / S;
  const int g = h / (p.H / p.G);
  const int nr = (int)p.n_rows;  // <= FEW_ROWS
  const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
  const float* W = p.k_proj + (int64_t)h * D * R;
  const bool map_in_lds = D * R <= FEW_MAP && (D * R) % 4 == 0 && ((uintptr_t)W & 15u) == 0;  // uniform
  // thread c < C holds codeword c's row of the current subspace (SUB > 0, C <= NT), requested for
  // subspace 0 before the projection so that both loads overlap
  const bool rows_in_regs = SUB > 0 && C <= NT;
  float crow[SUB > 0 ? SUB : 1];
  auto load_row = [&](int s) {
    if constexpr (SUB > 0) {
      const float4* src = reinterpret_cast<const float4*>(p.codebooks + (((int64_t)h * S + s) * C + min(t, C - 1)) * SUB);
#pragma unroll
      for (int k = 0; k < SUB / 4; ++k) {
        const float4 v = src[k];
        crow[4 * k] = v.x, crow[4 * k + 1] = v.y, crow[4 * k + 2] = v.z, crow[4 * k + 3] = v.w;
      }
    }
  };
  if (rows_in_regs && p.codes != nullptr) load_row(0);
  if (map_in_lds)
    for (int i = t; i < D * R / 4; i += NT) reinterpret_cast<float4*>(ws)[i] = reinterpret_cast<const float4*>(W)[i];
  for (int e = t; e < nr * D; e += NT) {
    const int j = e / D, d = e - j * D;
    kr[j][d] = load_elem(p.keys, (int64_t)b * p.seq_kv + (int64_t)g * p.kv_hs + (p.row0 + j) * p.kv_rs + d, p.kv_dtype);
  }
  __syncthreads();
  const float* Wm = map_in_lds ? ws : W;
  for (int e = t; e < nr * R; e += NT) {
    const int j = e / R, r = e - j * R;
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc = __builtin_fmaf(kr[j][d], Wm[d * R + r], acc);
    xl[j][r] = acc;
    p.k_low[(int64_t)h * p.klow_hs + ((int64_t)b * p.seq_rows + p.row0 + j) * R + r] = acc;
  }
  if (p.codes == nullptr) return;  // uniform
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    const float* cbs = p.codebooks + ((int64_t)h * S + s) * C * sub;
    if (rows_in_regs && s > 0) load_row(s);
    float cn = 0.0f;  // the codeword's squared norm in torch's sum order (rows held in registers)
    if constexpr (SUB > 0) {
      if (rows_in_regs) cn = torch_order_dot(crow, crow, SUB);
    }
    for (int j = 0; j < nr; ++j) {
      const float* xs = &xl[j][s * sub];
      const float xx = torch_order_dot(xs, xs, sub);
      // this thread's codewords in ascending order: the least distance, its
      // first index; NaN never wins, and none at all is index INT_MAX
      float best = INFINITY;
      int arg = 0x7FFFFFFF;
      if (rows_in_regs) {
        if (t < C) {
          float xc = 0.0f;
#pragma unroll
          for (int k = 0; k < (SUB > 0 ? SUB : 1); ++k) xc = __builtin_fmaf(xs[k], crow[k], xc);
          const float dist = (xx - 2.0f * xc) + cn;
          if (dist < best) {
            best = dist;
            arg = t;
          }
        }
      } else {
        for (int c = t; c < C; c += NT) {
          const float* cr = cbs + (int64_t)c * sub;
          float xc = 0.0f;
          for (int k = 0; k < sub; ++k) xc = __builtin_fmaf(xs[k], cr[k], xc);
          const float dist = (xx - 2.0f * xc) + torch_order_dot(cr, cr, sub);
          if (dist < best) {
            best = dist;
            arg = c;
          }
        }
      }
      // (best, arg) ordered by distance, then index: across the wave, then the waves
      for (int o = 1; o < WAVE; o <<= 1) {
        const float b2 = __shfl_xor(best, o, WAVE);
        const int a2 = __shfl_xor(arg, o, WAVE);
        if (b2 < best || (b2 == best && a2 < arg)) {
          best = b2;
          arg = a2;
        }
      }
      if (lane == 0) {
        rbest[wid] = best;
        rarg[wid] = arg;
      }
      __syncthreads();
      if (t == 0) {
        for (int w = 1; w < NT / WAVE; ++w)
          if (rbest[w] < best || (rbest[w] == best && rarg[w] < arg)) {
            best = rbest[w];
            arg = rarg[w];
          }
        store_code(p.codes, (int64_t)h * p.code_hs + ((int64_t)b * p.seq_rows + p.row0 + j) * S + s, p.ctype,
                   arg == 0x7FFFFFFF ? 0 : arg);
      }
      __syncthreads();
    }
  }
}

// sva_write_encode split into the validation (filling the parameters, one
// sequence) and the launch, so that a decode step can run its few-row append
// inside another kernel (write.hip).  The launch takes p.n_seq sequences.
int write_encode_setup(const void* keys, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                       int64_t row_begin, int64_t n_rows, int64_t H, int64_t G, int64_t D, int64_t R, int64_t S,
                       int64_t C, const float* k_proj, const float* codebooks, float* k_low,
                       int64_t k_low_head_stride, void* codes, int code_type, int64_t code_head_stride,
                       WriteParams* out);
// The few-row form's compile-time subspace width for p (0: read at run
// time), or -1 when p is not a few-row append (no rows, or more than FEW_ROWS).
int write_few_form(const WriteParams& p);
int write_encode_launch(const WriteParams& p, hipStream_t stream);

}  // namespace sva
