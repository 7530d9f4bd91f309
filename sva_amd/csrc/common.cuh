// Device-side building blocks shared by the SVA decode-path kernels (gfx950).
//
// Conventions
//  * Wavefront = 64 lanes.  Block sizes are multiples of 64.
//  * Scores are ranked through an order-preserving uint32 key (f2key); key 0 is
//    reserved for "not allowed" (no finite float maps to it).
//  * A ranked element is (key, key index); ties on key break toward the LOWER
//    key index.  The 64-bit composite (key << 32) | (0xFFFFFFFF - index) is
//    unique per key index and orders exactly like that rule.
//  * Every fp32 reduction whose bits matter is written with an explicit order
//    and with FP contraction disabled in its scope.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define SVA_DEV __device__ __forceinline__

namespace sva {

enum DType : int { F32 = 0, BF16 = 1, F16 = 2 };
enum CodeType : int { CODE_U8 = 0, CODE_I16 = 1, CODE_I32 = 2, CODE_I64 = 3 };

constexpr int WAVE = 64;

SVA_DEV uint32_t f2key(float x) {
  x = x + 0.0f;  // folds -0 onto +0 (not contracted or folded without nsz)
  uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

SVA_DEV float key2f(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(u);
}

SVA_DEV uint64_t composite(uint32_t key, uint32_t index) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - index);
}
SVA_DEV uint32_t composite_index(uint64_t c) { return 0xFFFFFFFFu - (uint32_t)(c & 0xFFFFFFFFu); }
SVA_DEV uint32_t composite_key(uint64_t c) { return (uint32_t)(c >> 32); }

SVA_DEV float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == F32) return ((const float*)p)[i];
  if (dtype == BF16) {
    uint16_t b = ((const uint16_t*)p)[i];
    return __uint_as_float((uint32_t)b << 16);
  }
  return __half2float(((const __half*)p)[i]);
}

// Element i's raw bits (all 32 for F32, the low 16 for BF16 / F16) and their
// value: a load whose result is not used at once, so that loads issued after
// it do not wait for it (a conversion on the load's own branch would).
SVA_DEV uint32_t load_elem_bits(const void* p, int64_t i, int dtype) {
  return dtype == F32 ? ((const uint32_t*)p)[i] : (uint32_t)((const uint16_t*)p)[i];
}
SVA_DEV float elem_from_bits(uint32_t b, int dtype) {
  return dtype == F32    ? __uint_as_float(b)
         : dtype == BF16 ? __uint_as_float(b << 16)
                         : __half2float(__ushort_as_half((unsigned short)(b & 0xFFFFu)));
}

// Four consecutive elements of a K/V row as floats.
SVA_DEV void load4(const void* base, int64_t e, int dtype, bool vec, float (&v)[4]) {
  if (vec) {
    if (dtype == F32) {
      const float4 x = *reinterpret_cast<const float4*>((const float*)base + e);
      v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
      return;
    }
    const uint2 x = *reinterpret_cast<const uint2*>((const uint16_t*)base + e);
    if (dtype == BF16) {
      v[0] = __uint_as_float(x.x << 16), v[1] = __uint_as_float(x.x & 0xFFFF0000u);
      v[2] = __uint_as_float(x.y << 16), v[3] = __uint_as_float(x.y & 0xFFFF0000u);
    } else {
      v[0] = __half2float(__ushort_as_half((unsigned short)(x.x & 0xFFFFu)));
      v[1] = __half2float(__ushort_as_half((unsigned short)(x.x >> 16)));
      v[2] = __half2float(__ushort_as_half((unsigned short)(x.y & 0xFFFFu)));
      v[3] = __half2float(__ushort_as_half((unsigned short)(x.y >> 16)));
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = load_elem(base, e + k, dtype);
}

SVA_DEV void store_elem(void* p, int64_t i, int dtype, float v) {
  if (dtype == F32) {
    ((float*)p)[i] = v;
  } else if (dtype == BF16) {
    // round to nearest even (what torch's .to(bfloat16) does for finite values)
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7F800000u) == 0x7F800000u) {
      ((uint16_t*)p)[i] = (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
    } else {
      u += 0x7FFFu + ((u >> 16) & 1u);
      ((uint16_t*)p)[i] = (uint16_t)(u >> 16);
    }
  } else {
    ((__half*)p)[i] = __float2half_rn(v);
  }
}

SVA_DEV int64_t load_code(const void* p, int64_t i, int ctype) {
  switch (ctype) {
    case CODE_U8: return ((const uint8_t*)p)[i];
    case CODE_I16: return ((const int16_t*)p)[i];
    case CODE_I32: return ((const int32_t*)p)[i];
    default: return ((const int64_t*)p)[i];
  }
}

SVA_DEV void store_code(void* p, int64_t i, int ctype, int64_t v) {
  switch (ctype) {
    case CODE_U8: ((uint8_t*)p)[i] = (uint8_t)v; break;
    case CODE_I16: ((int16_t*)p)[i] = (int16_t)v; break;
    case CODE_I32: ((int32_t*)p)[i] = (int32_t)v; break;
    default: ((int64_t*)p)[i] = v; break;
  }
}

// Additive / boolean attention-mask rule of the reference: allowed = mask > -1e4
// evaluated in the mask's dtype (a bool mask is therefore always allowed).
enum MaskType : int { MASK_NONE = 0, MASK_F32 = 1, MASK_BF16 = 2, MASK_F16 = 3, MASK_BOOL = 4 };

SVA_DEV bool mask_allows(const void* mask, int64_t i, int mtype) {
  switch (mtype) {
    case MASK_F32: return ((const float*)mask)[i] > -1e4f;
    case MASK_BF16: return __uint_as_float((uint32_t)((const uint16_t*)mask)[i] << 16) > -1e4f;
    case MASK_F16: return __half2float(((const __half*)mask)[i]) > -1e4f;
    default: return true;
  }
}

// ---------------------------------------------------------------------------
// wave / block collectives

SVA_DEV int lane_id() { return (int)__lane_id(); }

// Workgroups go to the 8 XCDs in turn (workgroup b to XCD b % 8), and each
// XCD has its own L2.  A grid of xcd_range_grid(total) workgroups where
// workgroup b takes item xcd_range_item(b, total) hands XCD x the contiguous
// items [x * per, (x + 1) * per): items in the order of their data (e.g.
// head-major) then share one XCD's L2 instead of every XCD caching every
// head's rows.  -1: a workgroup past the end (it returns).
constexpr int kXcds = 8;
__host__ __device__ inline int64_t xcd_range_grid(int64_t total) { return (total + kXcds - 1) / kXcds * kXcds; }
SVA_DEV int64_t xcd_range_item(int64_t b, int64_t total) {
  const int64_t per = (total + kXcds - 1) / kXcds;
  const int64_t item = (b % kXcds) * per + b / kXcds;
  return item < total ? item : -1;
}


// DPP row shifts (a DPP row is 16 lanes): lane j receives lane j - N of its
// row.  Lanes with no source lane receive 0 (row_shr0) or keep their own
// value (row_shr_keep: the identity for OR / AND folds).
template <int N>
SVA_DEV uint32_t row_shr0(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x110 + N, 0xF, 0xF, true);
}
template <int N>
SVA_DEV uint32_t row_shr_keep(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x110 + N, 0xF, 0xF, false);
}

// Inclusive scan within a wave: Hillis-Steele inside each DPP row, then the
// row totals (read from lanes 15, 31, 47) added to the later rows.  All 64
// lanes must be active.
SVA_DEV uint32_t wave_incl_scan(uint32_t v) {
  v += row_shr0<1>(v);
  v += row_shr0<2>(v);
  v += row_shr0<4>(v);
  v += row_shr0<8>(v);
  const uint32_t t0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t t1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t t2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const int row = lane_id() >> 4;
  return v + (row == 0 ? 0u : (row == 1 ? t0 : (row == 2 ? t0 + t1 : t0 + t1 + t2)));
}

// Sum over the wave (all 64 lanes active), wave-uniform.
SVA_DEV uint32_t wave_sum_dpp(uint32_t v) {
  v += row_shr0<1>(v);
  v += row_shr0<2>(v);
  v += row_shr0<4>(v);
  v += row_shr0<8>(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 15) + (uint32_t)__builtin_amdgcn_readlane((int)v, 31) +
         (uint32_t)__builtin_amdgcn_readlane((int)v, 47) + (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Sums over the 4 lanes of each quad and over the 8 lanes of each half-row,
// in every lane of the group (DPP quad permutes [1,0,3,2] and [2,3,0,1],
// then the half-row mirror, which pairs the two quads once each holds its
// own sum): the same pairings, and so the same results, as xor shuffles
// with masks 1, 2 and 4, without a cross-lane permute's round trip.
SVA_DEV uint32_t quad_sum(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
  return v;
}
SVA_DEV float octet_sum(float v) {
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  return v;
}

// Sum and maximum of a float over the wave (all 64 lanes active),
// wave-uniform: DPP row folds, then the four row results in a fixed order
// (short dependent steps instead of a chain of cross-lane permutes).
SVA_DEV float wave_sum(float v) {
  v = v + __int_as_float((int)row_shr0<1>((uint32_t)__float_as_int(v)));
  v = v + __int_as_float((int)row_shr0<2>((uint32_t)__float_as_int(v)));
  v = v + __int_as_float((int)row_shr0<4>((uint32_t)__float_as_int(v)));
  v = v + __int_as_float((int)row_shr0<8>((uint32_t)__float_as_int(v)));
  const auto rl = [](float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
  return ((rl(v, 15) + rl(v, 31)) + rl(v, 47)) + rl(v, 63);
}
SVA_DEV float wave_max(float v) {
  v = fmaxf(v, __int_as_float((int)row_shr_keep<1>((uint32_t)__float_as_int(v))));
  v = fmaxf(v, __int_as_float((int)row_shr_keep<2>((uint32_t)__float_as_int(v))));
  v = fmaxf(v, __int_as_float((int)row_shr_keep<4>((uint32_t)__float_as_int(v))));
  v = fmaxf(v, __int_as_float((int)row_shr_keep<8>((uint32_t)__float_as_int(v))));
  const auto rl = [](float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
  return fmaxf(fmaxf(rl(v, 15), rl(v, 31)), fmaxf(rl(v, 47), rl(v, 63)));
}

// Row shift within each 16-lane DPP row: lane j receives lane j + N of its
// row (lanes past the row end receive 0).
template <int N>
SVA_DEV float row_down(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xF, 0xF, true));
}

// Rank score of a 64-float k_low row in torch's sum order, computed by the
// 16 lanes of one DPP row (lane j holds float4 j of the row in r and of the
// query in qq): element e < 32 pairs with e + 32, the lane chains g, g+2,
// g+4, g+6 form accumulator lane 4g + c, then the eight in order, as in
// torch_order_dot64.  The result is valid in the row's first lane.
SVA_DEV float rank_dot64_row16(const float4 r, const float4 qq) {
#pragma clang fp contract(off)
  const float p0 = r.x * qq.x, p1 = r.y * qq.y, p2 = r.z * qq.z, p3 = r.w * qq.w;
  const float a0 = (0.0f + p0) + row_down<8>(p0);
  const float a1 = (0.0f + p1) + row_down<8>(p1);
  const float a2 = (0.0f + p2) + row_down<8>(p2);
  const float a3 = (0.0f + p3) + row_down<8>(p3);
  const float v0 = ((a0 + row_down<2>(a0)) + row_down<4>(a0)) + row_down<6>(a0);
  const float v1 = ((a1 + row_down<2>(a1)) + row_down<4>(a1)) + row_down<6>(a1);
  const float v2 = ((a2 + row_down<2>(a2)) + row_down<4>(a2)) + row_down<6>(a2);
  const float v3 = ((a3 + row_down<2>(a3)) + row_down<4>(a3)) + row_down<6>(a3);
  const float w0 = row_down<1>(v0), w1 = row_down<1>(v1), w2 = row_down<1>(v2), w3 = row_down<1>(v3);
  return (((((((0.0f + v0) + v1) + v2) + v3) + w0) + w1) + w2) + w3;
}

// The same rank score computed by the 8 lanes of a lane octet, two rows of
// each 16-lane DPP row: lane c holds floats 4c..4c+3 (r0) and 32+4c..32+4c+3
// (r1) of the row and of the query (q0, q1), so each lane forms the four
// pair sums a_j[l] = (0 + p[8j+l]) + p[32+8j+l] with j = c / 2,
// l = 4 (c % 2) + i locally; lanes 0 and 1 chain a_0..a_3 of their four l
// (lanes c, c+2, c+4, c+6), and lane 0 sums the eight in order.  Half the
// lanes' loads cover each 128-byte line of a row, as with 16 lanes per row,
// at about half the VALU instructions per row.  The result is valid in the
// octet's first lane.
SVA_DEV float rank_dot64_oct8(const float4 r0, const float4 r1, const float4 q0, const float4 q1) {
#pragma clang fp contract(off)
  // fma(x, y, 0) rounds x * y once and adds +0: the value of 0 + x * y
  const float a0 = __builtin_fmaf(r0.x, q0.x, 0.0f) + r1.x * q1.x;
  const float a1 = __builtin_fmaf(r0.y, q0.y, 0.0f) + r1.y * q1.y;
  const float a2 = __builtin_fmaf(r0.z, q0.z, 0.0f) + r1.z * q1.z;
  const float a3 = __builtin_fmaf(r0.w, q0.w, 0.0f) + r1.w * q1.w;
  const float v0 = ((a0 + row_down<2>(a0)) + row_down<4>(a0)) + row_down<6>(a0);
  const float v1 = ((a1 + row_down<2>(a1)) + row_down<4>(a1)) + row_down<6>(a1);
  const float v2 = ((a2 + row_down<2>(a2)) + row_down<4>(a2)) + row_down<6>(a2);
  const float v3 = ((a3 + row_down<2>(a3)) + row_down<4>(a3)) + row_down<6>(a3);
  const float w0 = row_down<1>(v0), w1 = row_down<1>(v1), w2 = row_down<1>(v2), w3 = row_down<1>(v3);
  return (((((((0.0f + v0) + v1) + v2) + v3) + w0) + w1) + w2) + w3;
}

// Maximum of a uint64 over the wave (all 64 lanes active), wave-uniform:
// DPP row shifts of both halves from the same source lane, then the four
// row maxima.
SVA_DEV uint64_t wave_max_u64(uint64_t x) {
  auto step = [](uint64_t v, uint32_t lo, uint32_t hi) {
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > v ? o : v;
  };
  x = step(x, row_shr_keep<1>((uint32_t)x), row_shr_keep<1>((uint32_t)(x >> 32)));
  x = step(x, row_shr_keep<2>((uint32_t)x), row_shr_keep<2>((uint32_t)(x >> 32)));
  x = step(x, row_shr_keep<4>((uint32_t)x), row_shr_keep<4>((uint32_t)(x >> 32)));
  x = step(x, row_shr_keep<8>((uint32_t)x), row_shr_keep<8>((uint32_t)(x >> 32)));
  uint64_t m = 0ull;
#pragma unroll
  for (int r = 15; r < WAVE; r += 16) {
    const uint64_t v = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), r) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, r);
    m = v > m ? v : m;
  }
  return m;
}

// Minimum and maximum of a uint32 over the wave (all 64 lanes active), wave-uniform.
SVA_DEV void wave_min_max_u32(uint32_t& mn, uint32_t& mx) {
  mn = min(mn, row_shr_keep<1>(mn));
  mx = max(mx, row_shr_keep<1>(mx));
  mn = min(mn, row_shr_keep<2>(mn));
  mx = max(mx, row_shr_keep<2>(mx));
  mn = min(mn, row_shr_keep<4>(mn));
  mx = max(mx, row_shr_keep<4>(mx));
  mn = min(mn, row_shr_keep<8>(mn));
  mx = max(mx, row_shr_keep<8>(mx));
  const auto rl = [](uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); };
  mn = min(min(rl(mn, 15), rl(mn, 31)), min(rl(mn, 47), rl(mn, 63)));
  mx = max(max(rl(mx, 15), rl(mx, 31)), max(rl(mx, 47), rl(mx, 63)));
}

// OR and AND of a 64-bit value over the wave (all 64 lanes active), wave-uniform.
SVA_DEV void wave_or_and_u64(uint64_t& vor, uint64_t& vand) {
  uint32_t o[2] = {(uint32_t)vor, (uint32_t)(vor >> 32)};
  uint32_t n[2] = {(uint32_t)vand, (uint32_t)(vand >> 32)};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    o[h] |= row_shr_keep<1>(o[h]);
    n[h] &= row_shr_keep<1>(n[h]);
    o[h] |= row_shr_keep<2>(o[h]);
    n[h] &= row_shr_keep<2>(n[h]);
    o[h] |= row_shr_keep<4>(o[h]);
    n[h] &= row_shr_keep<4>(n[h]);
    o[h] |= row_shr_keep<8>(o[h]);
    n[h] &= row_shr_keep<8>(n[h]);
    o[h] = (uint32_t)__builtin_amdgcn_readlane((int)o[h], 15) | (uint32_t)__builtin_amdgcn_readlane((int)o[h], 31) |
           (uint32_t)__builtin_amdgcn_readlane((int)o[h], 47) | (uint32_t)__builtin_amdgcn_readlane((int)o[h], 63);
    n[h] = (uint32_t)__builtin_amdgcn_readlane((int)n[h], 15) & (uint32_t)__builtin_amdgcn_readlane((int)n[h], 31) &
           (uint32_t)__builtin_amdgcn_readlane((int)n[h], 47) & (uint32_t)__builtin_amdgcn_readlane((int)n[h], 63);
  }
  vor = ((uint64_t)o[1] << 32) | o[0];
  vand = ((uint64_t)n[1] << 32) | n[0];
}

// Exclusive block scan of one value per thread.  `scratch` holds >= BLOCK/64 + 1
// uint32 in LDS.  Returns the exclusive prefix; *total gets the block sum.
// Every wave reads all wave totals itself (no second-level scan).
template <int BLOCK>
SVA_DEV uint32_t block_excl_scan(uint32_t v, uint32_t* scratch, uint32_t* total) {
  constexpr int NW = BLOCK / WAVE;
  const int lane = lane_id();
  const int wid = threadIdx.x / WAVE;
  const uint32_t incl = wave_incl_scan(v);
  if (lane == WAVE - 1) scratch[wid] = incl;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    const uint32_t t = scratch[q];
    before += q < wid ? t : 0u;
    all += t;
  }
  if (total) *total = all;
  __syncthreads();
  return before + incl - v;
}

// ---------------------------------------------------------------------------
// Exact selection of the k largest nonzero composites among the elements a
// visitor yields (each element exactly once per call, unique values): radix
// passes of up to 8 bits from the highest bit where elements differ, with
// one LDS histogram per wave.  vor / vand are this thread's OR and AND of the
// elements it visits (0 and ~0 when it visits none).  Returns X such that the
// selected elements are exactly those >= X.  Every thread of the block must
// call it.  whist: BLOCK/64 rows of 256 uint32; scratch: block_excl_scan
// scratch; shared64: 2 uint64; shared: 3 uint32 (all LDS).  BLOCK >= 256.
template <int BLOCK, typename Visit>
SVA_DEV uint64_t select_largest_with_bounds(Visit visit, int k, uint64_t vor, uint64_t vand, uint32_t (*whist)[256],
                                            uint32_t* scratch, uint64_t* shared64, uint32_t* shared) {
  const int wid = threadIdx.x / WAVE;
  // bits above the highest differing bit are common to every element
  for (int off = 1; off < WAVE; off <<= 1) {
    vor |= __shfl_xor(vor, off, WAVE);
    vand &= __shfl_xor(vand, off, WAVE);
  }
  if (threadIdx.x == 0) {
    shared64[0] = 0ull;
    shared64[1] = ~0ull;
  }
  __syncthreads();
  if (lane_id() == 0) {
    atomicOr((unsigned long long*)&shared64[0], (unsigned long long)vor);
    atomicAnd((unsigned long long*)&shared64[1], (unsigned long long)vand);
  }
  __syncthreads();
  const uint64_t diff = shared64[0] ^ shared64[1];
  if (diff == 0ull) return shared64[0];  // a single element
  int top = 63 - __clzll((long long)diff);
  uint64_t pmask = top == 63 ? 0ull : ~0ull << (top + 1);
  uint64_t prefix = shared64[1] & pmask;
  int need = k;
  while (true) {
    const int shift = max(top - 7, 0);
    const uint32_t dmask = (1u << (top - shift + 1)) - 1u;
    for (int i = threadIdx.x; i < (BLOCK / WAVE) * 256; i += BLOCK) whist[i >> 8][i & 255] = 0u;
    __syncthreads();
    visit([&](uint64_t x) {
      if ((x & pmask) == prefix) atomicAdd(&whist[wid][(uint32_t)(x >> shift) & dmask], 1u);
    });
    __syncthreads();
    uint32_t tot = 0;
    if (threadIdx.x < 256) {
      const int b = 255 - (int)threadIdx.x;  // bins from the top
      for (int v = 0; v < BLOCK / WAVE; ++v) tot += whist[v][b];
    }
    uint32_t total;
    const uint32_t above = block_excl_scan<BLOCK>(tot, scratch, &total);
    if (threadIdx.x < 256 && above < (uint32_t)need && above + tot >= (uint32_t)need) {
      shared[0] = 255u - threadIdx.x;
      shared[1] = above;
      shared[2] = tot;
    }
    __syncthreads();
    const uint32_t b = shared[0];
    need -= (int)shared[1];
    prefix |= (uint64_t)b << shift;
    pmask |= (uint64_t)dmask << shift;
    const bool done = shared[2] == (uint32_t)need || shift == 0;
    __syncthreads();
    if (done) return prefix;
    top = shift - 1;
  }
}

// select_largest_with_bounds with 12-bit digits over one shared 4096-bin
// LDS histogram (hist, 4096 uint32, 4-byte aligned; BLOCK = 1024): two
// passes where the 8-bit form needs three or four on wide value ranges.
template <int BLOCK, typename Visit>
SVA_DEV uint64_t select_largest12(Visit visit, int k, uint64_t vor, uint64_t vand, uint32_t* hist, uint32_t* scratch,
                                  uint64_t* shared64, uint32_t* shared) {
  static_assert(BLOCK == 1024, "4 bins per thread");
  for (int off = 1; off < WAVE; off <<= 1) {
    vor |= __shfl_xor(vor, off, WAVE);
    vand &= __shfl_xor(vand, off, WAVE);
  }
  if (threadIdx.x == 0) {
    shared64[0] = 0ull;
    shared64[1] = ~0ull;
  }
  __syncthreads();
  if (lane_id() == 0) {
    atomicOr((unsigned long long*)&shared64[0], (unsigned long long)vor);
    atomicAnd((unsigned long long*)&shared64[1], (unsigned long long)vand);
  }
  __syncthreads();
  const uint64_t diff = shared64[0] ^ shared64[1];
  if (diff == 0ull) return shared64[0];  // a single element
  int top = 63 - __clzll((long long)diff);
  uint64_t pmask = top == 63 ? 0ull : ~0ull << (top + 1);
  uint64_t prefix = shared64[1] & pmask;
  int need = k;
  while (true) {
    const int shift = max(top - 11, 0);
    const uint32_t dmask = (1u << (top - shift + 1)) - 1u;
#pragma unroll
    for (int j = 0; j < 4; ++j) hist[4 * threadIdx.x + j] = 0u;  // 4-byte aligned words (hist need not be 16)
    __syncthreads();
    visit([&](uint64_t x) {
      if ((x & pmask) == prefix) atomicAdd(&hist[(uint32_t)(x >> shift) & dmask], 1u);
    });
    __syncthreads();
    // thread t owns bins 4095 - 4t .. 4092 - 4t, from the top
    const uint32_t* hq = hist + 4 * (BLOCK - 1 - threadIdx.x);
    const uint4 hb = uint4{hq[0], hq[1], hq[2], hq[3]};
    uint32_t total;
    const uint32_t above = block_excl_scan<BLOCK>(hb.x + hb.y + hb.z + hb.w, scratch, &total);
    {
      const uint32_t c[4] = {hb.w, hb.z, hb.y, hb.x};
      uint32_t a = above;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (a < (uint32_t)need && a + c[j] >= (uint32_t)need) {
          shared[0] = 4095u - 4u * threadIdx.x - (uint32_t)j;
          shared[1] = a;
          shared[2] = c[j];
        }
        a += c[j];
      }
    }
    __syncthreads();
    const uint32_t b = shared[0];
    need -= (int)shared[1];
    prefix |= (uint64_t)b << shift;
    pmask |= (uint64_t)dmask << shift;
    const bool done = shared[2] == (uint32_t)need || shift == 0;
    __syncthreads();
    if (done) return prefix;
    top = shift - 1;
  }
}

// select_largest with the OR / AND of the elements taken in an extra pass.
template <int BLOCK, typename Visit>
SVA_DEV uint64_t select_largest(Visit visit, int k, uint32_t (*whist)[256], uint32_t* scratch, uint64_t* shared64,
                                uint32_t* shared) {
  uint64_t vor = 0ull, vand = ~0ull;
  visit([&](uint64_t x) {
    vor |= x;
    vand &= x;
  });
  return select_largest_with_bounds<BLOCK>(visit, k, vor, vand, whist, scratch, shared64, shared);
}

// ---------------------------------------------------------------------------
// Selection over elements held in registers: each thread of the block holds
// NPT nonzero composites (0 = empty slot); slots from `slots` on are empty in
// every thread and skipped.  vor / vand: this thread's OR and AND of its
// elements, or (bounds_given) block-uniform bounds hi >= every element >= lo,
// whose common high bits every element shares.  Radix passes of up to TOP_BITS
// bits from the highest bit where the elements differ, counted in one shared
// LDS histogram; as soon as the bucket holding the k-th largest has at most
// TOP_SMALL elements they are gathered and ranked directly.  Returns X such
// that the selected elements are exactly those >= X (with repeated values,
// more than k elements may reach X and the caller caps its output at k).
constexpr int TOP_BITS = 12;
constexpr int TOP_BINS = 1 << TOP_BITS;
constexpr int TOP_SMALL = 64;  // last bucket ranked directly, 16 lanes per element

struct TopLds {
  uint32_t* hist;      // [TOP_BINS]
  uint64_t* small;     // [TOP_SMALL]
  uint32_t* scratch;   // [BLOCK / 64 + 1]
  uint32_t* shared;    // [4]
  uint64_t* shared64;  // [2]
};

template <int BLOCK, int NPT>
SVA_DEV uint64_t select_top_regs(const uint64_t (&e)[NPT], int k, uint64_t vor, uint64_t vand, const TopLds& s,
                                 int slots = NPT, bool bounds_given = false) {
  static_assert(BLOCK == 4 * 256 && TOP_BINS == 4 * BLOCK, "one uint4 of bins per thread");
  static_assert(TOP_SMALL * 16 == BLOCK, "16 lanes per element of the last bucket");
  const int lane = lane_id();
  uint64_t all_or = vor, all_and = vand;  // bounds_given: block-uniform hi and lo with lo <= every element <= hi
  if (!bounds_given) {
    wave_or_and_u64(vor, vand);
    if (threadIdx.x == 0) {
      s.shared64[0] = 0ull;
      s.shared64[1] = ~0ull;
    }
    __syncthreads();
    if (lane == 0) {
      atomicOr((unsigned long long*)&s.shared64[0], (unsigned long long)vor);
      atomicAnd((unsigned long long*)&s.shared64[1], (unsigned long long)vand);
    }
    __syncthreads();
    all_or = s.shared64[0];
    all_and = s.shared64[1];
    __syncthreads();
  }
  const uint64_t diff = all_or ^ all_and;
  if (diff == 0ull) return all_or;  // one distinct value
  int top = 63 - __clzll((long long)diff);
  uint64_t pmask = top == 63 ? 0ull : ~0ull << (top + 1);
  uint64_t prefix = all_and & pmask;
  int need = k;
  while (true) {
    const int shift = max(top - (TOP_BITS - 1), 0);
    const uint32_t dmask = (1u << (top - shift + 1)) - 1u;
    reinterpret_cast<uint4*>(s.hist)[threadIdx.x] = uint4{0u, 0u, 0u, 0u};
    if (threadIdx.x == 0) s.shared[3] = 0u;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const uint64_t x = e[i];
      if (i < slots && x != 0ull && (x & pmask) == prefix) atomicAdd(&s.hist[(uint32_t)(x >> shift) & dmask], 1u);
    }
    __syncthreads();
    // thread t owns bins 4t .. 4t+3 counted from the top
    const uint4 h = reinterpret_cast<const uint4*>(s.hist)[BLOCK - 1 - threadIdx.x];
    uint32_t total;
    const uint32_t above = block_excl_scan<BLOCK>(h.x + h.y + h.z + h.w, s.scratch, &total);
    {
      const uint32_t c[4] = {h.w, h.z, h.y, h.x};
      uint32_t a = above;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (a < (uint32_t)need && a + c[j] >= (uint32_t)need) {
          s.shared[0] = (uint32_t)(TOP_BINS - 1 - 4 * (int)threadIdx.x - j);
          s.shared[1] = a;
          s.shared[2] = c[j];
        }
        a += c[j];
      }
    }
    __syncthreads();
    const uint32_t b = s.shared[0];
    const uint32_t cb = s.shared[2];
    need -= (int)s.shared[1];
    prefix |= (uint64_t)b << shift;
    pmask |= (uint64_t)dmask << shift;
    if (cb == (uint32_t)need || shift == 0) {
      __syncthreads();
      return prefix;
    }
    if (cb <= (uint32_t)TOP_SMALL) {
      // gather the bucket and rank its elements directly
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        if (i < slots) {  // uniform
          const uint64_t x = e[i];
          const bool match = x != 0ull && (x & pmask) == prefix;
          const uint64_t m = __builtin_amdgcn_ballot_w64(match);
          if (m != 0ull) {
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&s.shared[3], (uint32_t)__popcll(m));
            base = __shfl(base, 0, WAVE);
            if (match) {
              const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
              s.small[base + below] = x;
            }
          }
        }
      }
      __syncthreads();
      {
        // rank of each bucket element within the bucket: one DPP row of 16
        // lanes per element, 4 comparisons per lane counting the elements
        // above it (low half) and at or above it (high half); the need-th
        // largest has fewer than need above and at least need at or above
        // (equal elements write the same value)
        const int i = (int)threadIdx.x >> 4, g = (int)threadIdx.x & 15;
        const uint64_t v = i < (int)cb ? s.small[i] : 0ull;
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int o = 4 * g + j;
          if (o < (int)cb) {
            const uint64_t y = s.small[o];
            c += (y > v ? 1u : 0u) + (y >= v ? 0x10000u : 0u);
          }
        }
        c += row_shr0<1>(c);
        c += row_shr0<2>(c);
        c += row_shr0<4>(c);
        c += row_shr0<8>(c);
        if (g == 15 && i < (int)cb && (c & 0xFFFFu) < (uint32_t)need && (c >> 16) >= (uint32_t)need)
          s.shared64[0] = v;
      }
      __syncthreads();
      const uint64_t X = s.shared64[0];
      __syncthreads();
      return X;
    }
    top = shift - 1;
  }
}

// Writes the beff indices of sel (LDS, capacity rounded up to 64) to out in
// ascending order.  Up to BLOCK entries: each wave sorts a run of 64 in
// registers (bitonic), then an entry's place is its place in its run plus,
// for every other run, the number of smaller entries (binary search).
// Larger counts: two lanes per entry count the smaller entries.  Entries are
// distinct.  sel is overwritten.  Every thread of the block must call it.
template <int BLOCK>
SVA_DEV void write_ascending(uint32_t* sel, int beff, int32_t* out) {
  if (beff <= BLOCK) {
    const int runs = (beff + WAVE - 1) / WAVE;
    const int t = threadIdx.x;
    uint32_t v = t < beff ? sel[t] : 0xFFFFFFFFu;
    if (t < runs * WAVE) {
      const int lane = lane_id();
      for (int k = 2; k <= WAVE; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
          const uint32_t o = (uint32_t)__shfl_xor((int)v, j, WAVE);
          const bool up = (lane & k) == 0;
          const bool low = (lane & j) == 0;
          v = (low == up) ? min(v, o) : max(v, o);
        }
      }
    }
    __syncthreads();
    if (t < runs * WAVE) sel[t] = v;  // sorted runs, padded with 0xFFFFFFFF
    __syncthreads();
    if (t < runs * WAVE && v != 0xFFFFFFFFu) {
      const int run = t / WAVE;
      int r = t - run * WAVE;
      for (int q = 0; q < runs; ++q) {
        if (q == run) continue;
        const uint32_t* a = sel + q * WAVE;
        int lo = 0, hi = WAVE;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (a[mid] < v) lo = mid + 1;
          else hi = mid;
        }
        r += lo;
      }
      out[r] = (int32_t)v;
    }
  } else {
    const int hb = (((beff + 1) >> 1) + 3) & ~3;
    for (int i = threadIdx.x; i < 2 * beff; i += BLOCK) {
      const int e = i >> 1;
      const uint32_t v = sel[e];
      const int j0 = (i & 1) ? hb : 0;
      const int j1 = (i & 1) ? beff : min(hb, beff);
      int r = 0;
      int j = j0;
#pragma unroll 8
      for (; j + 4 <= j1; j += 4) {
        const uint4 u = *reinterpret_cast<const uint4*>(sel + j);
        r += (int)(u.x < v) + (int)(u.y < v) + (int)(u.z < v) + (int)(u.w < v);
      }
      for (; j < j1; ++j) r += (int)(sel[j] < v);
      r += __shfl_xor(r, 1);
      if ((i & 1) == 0) out[r] = (int32_t)v;
    }
  }
}

// Appends this thread's elements e[i] >= X (nonzero) to dst in any order,
// at most cap of them; `counter` (LDS, zeroed and synchronised by the caller)
// receives the count.  Every lane of a wave must call it.
template <int NPT>
SVA_DEV void append_selected(const uint64_t (&e)[NPT], uint64_t X, uint32_t* dst, int cap, uint32_t* counter) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const uint64_t x = e[i];
    const bool sel = x != 0ull && x >= X;
    const uint64_t m = __builtin_amdgcn_ballot_w64(sel);
    if (m != 0ull) {
      uint32_t base = 0;
      if (lane == 0) base = atomicAdd(counter, (uint32_t)__popcll(m));
      base = __shfl(base, 0, WAVE);
      const uint32_t o = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (sel && o < (uint32_t)cap) dst[o] = composite_index(x);
    }
  }
}

// ---------------------------------------------------------------------------
// Radix select over uint32 keys.  Finds the threshold key T and k_eq such that
// the k largest elements are: every element with key > T plus the k_eq
// lowest-index elements with key == T.  Elements with key 0 never count.
// get(i) returns the key of element i in [0, n).  hist: 256 uint32 in LDS,
// scratch: block_excl_scan scratch, shared: 4 uint32 in LDS.
template <int BLOCK, typename Get>
SVA_DEV void radix_select_u32(Get get, int n, int k, uint32_t* hist, uint32_t* scratch, uint32_t* shared,
                              uint32_t* T_out, int* keq_out) {
  uint32_t prefix = 0, pmask = 0;
  int k_rem = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += BLOCK) hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += BLOCK) {
      const uint32_t key = get(i);
      if (key != 0u && (key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    // cumulative count from the top digit down
    uint32_t c = 0;
    if (threadIdx.x < 256) c = hist[255 - threadIdx.x];
    uint32_t tot;
    uint32_t before = block_excl_scan<BLOCK>(threadIdx.x < 256 ? c : 0u, scratch, &tot);
    if (threadIdx.x < 256 && before < (uint32_t)k_rem && before + c >= (uint32_t)k_rem) {
      shared[0] = 255u - threadIdx.x;
      shared[1] = before;
    }
    __syncthreads();
    const uint32_t d = shared[0];
    k_rem -= (int)shared[1];
    prefix |= d << shift;
    pmask |= 255u << shift;
    __syncthreads();
  }
  *T_out = prefix;
  *keq_out = k_rem;
}

// Radix select over uint64 composites (unique per index); returns the
// k-th largest composite X: the selection is exactly {c >= X}.
template <int BLOCK, typename Get>
SVA_DEV uint64_t radix_select_u64(Get get, int n, int k, uint32_t* hist, uint32_t* scratch, uint32_t* shared) {
  uint64_t prefix = 0, pmask = 0;
  int k_rem = k;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += BLOCK) hist[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += BLOCK) {
      const uint64_t c = get(i);
      if (c != 0ull && (c & pmask) == prefix) atomicAdd(&hist[(uint32_t)(c >> shift) & 255u], 1u);
    }
    __syncthreads();
    uint32_t cnt = 0;
    if (threadIdx.x < 256) cnt = hist[255 - threadIdx.x];
    uint32_t tot;
    uint32_t before = block_excl_scan<BLOCK>(threadIdx.x < 256 ? cnt : 0u, scratch, &tot);
    if (threadIdx.x < 256 && before < (uint32_t)k_rem && before + cnt >= (uint32_t)k_rem) {
      shared[0] = 255u - threadIdx.x;
      shared[1] = before;
    }
    __syncthreads();
    const uint64_t d = shared[0];
    k_rem -= (int)shared[1];
    prefix |= d << shift;
    pmask |= 255ull << shift;
    __syncthreads();
  }
  return prefix;
}

// In-place bitonic sort of n (power of two) uint64 in LDS, descending if desc.
template <int BLOCK>
SVA_DEV void bitonic_sort_u64(uint64_t* a, int n, bool desc) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < n / 2; t += BLOCK) {
        const int lo = 2 * t - (t & (stride - 1));
        const int hi = lo + stride;
        const bool up = ((lo & size) == 0) != desc;  // ascending block?
        const uint64_t x = a[lo], y = a[hi];
        if ((x > y) == up) {
          a[lo] = y;
          a[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

SVA_DEV int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// ---------------------------------------------------------------------------
// torch.sum(dim=-1) order for a row of k <= 511 products (see the oracle):
// 8-lane vectors, 4 interleaved accumulators, leftovers into accumulator 0,
// accumulators folded in order, scalar tail first, then lanes in order.
// Products are rounded separately (no FMA).
SVA_DEV float torch_order_dot(const float* __restrict__ a, const float* __restrict__ b, int k) {
#pragma clang fp contract(off)
  const int nvec = k >> 3;
  const int rows = nvec >> 2;
  float acc[4][8];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[x][l] = 0.0f;
  for (int i = 0; i < rows; ++i) {
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const int e = (i * 4 + x) * 8 + l;
        const float p = a[e] * b[e];
        acc[x][l] = acc[x][l] + p;
      }
  }
  for (int v = rows * 4; v < nvec; ++v) {
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const float p = a[v * 8 + l] * b[v * 8 + l];
      acc[0][l] = acc[0][l] + p;
    }
  }
#pragma unroll
  for (int x = 1; x < 4; ++x)
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[0][l] = acc[0][l] + acc[x][l];
  float total = 0.0f;
  for (int t = nvec * 8; t < k; ++t) {
    const float p = a[t] * b[t];
    total = total + p;
  }
#pragma unroll
  for (int l = 0; l < 8; ++l) total = total + acc[0][l];
  return total;
}

// Same order, specialised for k == 64 with the row read as 16 float4 from
// global memory (16-byte aligned) and the other operand from LDS.
SVA_DEV float torch_order_dot64(const float* __restrict__ row, const float* __restrict__ q) {
#pragma clang fp contract(off)
  float r[64];
  const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float4 v = r4[i];
    r[4 * i + 0] = v.x;
    r[4 * i + 1] = v.y;
    r[4 * i + 2] = v.z;
    r[4 * i + 3] = v.w;
  }
  float part[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) {
    float a0 = 0.0f + r[l] * q[l];
    a0 = a0 + r[32 + l] * q[32 + l];
    float a1 = 0.0f + r[8 + l] * q[8 + l];
    a1 = a1 + r[40 + l] * q[40 + l];
    float a2 = 0.0f + r[16 + l] * q[16 + l];
    a2 = a2 + r[48 + l] * q[48 + l];
    float a3 = 0.0f + r[24 + l] * q[24 + l];
    a3 = a3 + r[56 + l] * q[56 + l];
    part[l] = ((a0 + a1) + a2) + a3;
  }
  float total = 0.0f;
#pragma unroll
  for (int l = 0; l < 8; ++l) total = total + part[l];
  return total;
}

}  // namespace sva
