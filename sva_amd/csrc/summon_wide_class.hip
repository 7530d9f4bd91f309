// Code-class path of the long-context summon (one subspace of at most 256
// codewords): the count, select and extract launches; the budget launch's
// variants live with the finish kernels of their K / V dtype.
#include "query_decode.cuh"
#include "summon_wide.cuh"

namespace sva {
namespace wide {
namespace {

// Every phase keeps its loads in flight together: the counts were written
// by workgroups on other XCDs, so each dependent round trip is long.
__global__ void __launch_bounds__(SB) class_select_kernel(ClassArgs a) {
  __shared__ __align__(16) uint32_t key[256], tot[256], flags[256], part[CSEL_G][256], gep[CSEL_G][256];
  __shared__ uint32_t scratch[SNW + 1], res[4];
  __shared__ uint64_t bmin;
  __shared__ uint32_t sa[CLASS_MAX_W], sb[CLASS_MAX_W];
  const SummonParams& p = a.p;
  const int item = blockIdx.x, t = threadIdx.x, W = a.W;
  const int c = t & 255, g = t >> 8;
  const uint32_t* cnt = a.counts + (int64_t)item * W * 256;
  // code c's total: group g sums chunks g, g + CSEL_G, ..., 16 loads in flight at a time
  {
    uint32_t acc = 0;
    for (int w0 = g; w0 < W; w0 += 16 * CSEL_G) {
      uint32_t v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int w = w0 + u * CSEL_G;
        v[u] = w < W ? cnt[(int64_t)w * 256 + c] : 0u;
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) acc += v[u];
    }
    part[g][c] = acc;
  }
  if (t < 256) key[t] = class_key(p, item, t);
  if (t == 0) {
    res[0] = 0xFFFFFFFFu;  // no boundary class (empty shortlist): no key matches
    res[1] = 0u;
    res[2] = 0u;  // keys strictly above the boundary class
    bmin = ~0ull;
  }
  __syncthreads();
  if (t < 256) {
    uint32_t n = 0;
#pragma unroll
    for (int q = 0; q < CSEL_G; ++q) n += part[q][t];
    tot[t] = n;
  }
  __syncthreads();
  uint32_t A = 0;
  for (int q = 0; q < 256; q += 64) A += tot[q + lane_id()];  // every wave sums all 256 totals
  A = wave_sum_dpp(A);
  const int leff = (int)min((uint32_t)p.L, A);
  // keys in or above code c's class, ge(c): group g over codes [64 g, 64 g + 64)
  {
    const uint32_t k = key[c];
    const uint4* k4 = reinterpret_cast<const uint4*>(key + 64 * g);
    const uint4* t4 = reinterpret_cast<const uint4*>(tot + 64 * g);
    uint32_t ge = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // both operands read before the select: no per-element branch
      const uint4 kq = k4[i], tq = t4[i];
      ge += (kq.x >= k ? tq.x : 0u) + (kq.y >= k ? tq.y : 0u) + (kq.z >= k ? tq.z : 0u) + (kq.w >= k ? tq.w : 0u);
    }
    gep[g][c] = ge;
  }
  __syncthreads();
  // ge falls as the key rises.  The boundary class is the one of lowest ge
  // among the classes holding keys with ge >= leff; the keys strictly above
  // it number the largest ge below leff (0 if none).
  if (t < 256 && leff > 0) {  // waves 0-3: every lane active
    uint32_t ge = 0;
#pragma unroll
    for (int q = 0; q < CSEL_G; ++q) ge += gep[q][t];
    const uint64_t cand = tot[t] > 0 && ge >= (uint32_t)leff ? ((uint64_t)ge << 32) | key[t] : ~0ull;
    const uint64_t lowest = ~wave_max_u64(~cand);
    uint32_t mn = 0u, below = ge < (uint32_t)leff ? ge : 0u;
    wave_min_max_u32(mn, below);
    if (lane_id() == 0) {
      atomicMin(&bmin, lowest);
      atomicMax(&res[2], below);
    }
  }
  __syncthreads();
  const uint32_t kb = leff > 0 ? (uint32_t)bmin : res[0];
  const uint32_t need = leff > 0 ? (uint32_t)leff - res[2] : res[1];
  if (t < 256) flags[t] = (key[t] > kb ? 1u : 0u) | (key[t] == kb ? 2u : 0u);
  __syncthreads();
  // per chunk: kept keys above the boundary class, keys of the boundary class; 16 lanes per chunk, each
  // over 16 codes (four 16-byte loads issued together), summed over the lanes
  {
    const int q = t & 15;
    uint32_t fl[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) fl[e] = flags[16 * q + e];
    for (int w0 = 0; w0 < W; w0 += SB / 16) {
      const int w = w0 + t / 16;
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = w < W ? reinterpret_cast<const uint4*>(cnt + (int64_t)w * 256 + 16 * q)[u] : uint4{0u, 0u, 0u, 0u};
      uint32_t x = 0, y = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x += (fl[4 * u + e] & 1u) ? vv[e] : 0u;
          y += (fl[4 * u + e] & 2u) ? vv[e] : 0u;
        }
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        x += __shfl_xor(x, o, 16);
        y += __shfl_xor(y, o, 16);
      }
      if (q == 0 && w < W) {
        sa[w] = x;
        sb[w] = y;
      }
    }
  }
  __syncthreads();
  // thread t: chunks [t * CSEL_PER, (t + 1) * CSEL_PER); boundary keys before each, then its kept keys
  const int w0 = t * CSEL_PER;
  uint32_t bsum = 0;
#pragma unroll
  for (int i = 0; i < CSEL_PER; ++i) bsum += w0 + i < W ? sb[w0 + i] : 0u;
  uint32_t bpre = block_excl_scan<SB>(bsum, scratch, nullptr);  // boundary keys in chunks before w0
  uint32_t kept[CSEL_PER], ksum = 0;
#pragma unroll
  for (int i = 0; i < CSEL_PER; ++i) {
    const int w = w0 + i;
    kept[i] = 0u;
    if (w < W) {
      const uint32_t b = sb[w];
      kept[i] = sa[w] + (need > bpre ? min(need - bpre, b) : 0u);
      sb[w] = bpre;  // this thread's own chunks only
      bpre += b;
      ksum += kept[i];
    }
  }
  uint32_t koff = block_excl_scan<SB>(ksum, scratch, nullptr);
  uint32_t* wo = a.woff + (int64_t)item * W * 2;
#pragma unroll
  for (int i = 0; i < CSEL_PER; ++i) {
    const int w = w0 + i;
    if (w < W) {
      wo[2 * w] = koff;
      wo[2 * w + 1] = sb[w];
      koff += kept[i];
    }
  }
  if (t == 0) {
    a.bound[4 * item] = kb;
    a.bound[4 * item + 1] = need;
    a.bound[4 * item + 2] = (uint32_t)leff;
    a.bound[4 * item + 3] = 0u;
    p.sl_count[item] = leff;
    if (a.overshoot != nullptr) a.overshoot[item] = 0;
  }
}

// The decode query of every head (workgroups g < H) and the code counts of
// every chunk (the rest) in one grid: the counts need nothing the query
// computes, so they run while its dependent chain does.
template <bool MASKED>
__global__ void __launch_bounds__(WB) class_query_count_kernel(LutParams q, ClassArgs a) {
  static_assert(QD == WB, "one block size for both roles");
  if ((int)blockIdx.x < q.H) query_decode_item<1, 256>(q, (int)blockIdx.x);
  else class_count_chunk<MASKED>(a, (int)blockIdx.x - q.H);
}

template <bool MASKED>
int launch_class_m(const ClassArgs& a, int64_t items, const QueryLaunch* query, hipStream_t stream) {
  if (query != nullptr && query->form == QUERY_DECODE_1_256) {
    hipLaunchKernelGGL((class_query_count_kernel<MASKED>), dim3((unsigned)(query->blocks + items * a.W)), dim3(WB), 0,
                       stream, query->p, a);
    SVA_CHECK_LAUNCH("class_query_count_kernel");
  } else {
    if (query != nullptr) {
      const int rc = query_lut_launch(*query, stream);
      if (rc != SVA_OK) return rc;
    }
    hipLaunchKernelGGL((class_count_kernel<MASKED>), dim3((unsigned)(items * a.W)), dim3(WB), 0, stream, a);
    SVA_CHECK_LAUNCH("class_count_kernel");
  }
  hipLaunchKernelGGL(class_select_kernel, dim3((unsigned)items), dim3(SB), 0, stream, a);
  SVA_CHECK_LAUNCH("class_select_kernel");
  hipLaunchKernelGGL((class_extract_kernel<MASKED>), dim3((unsigned)(items * a.W)), dim3(WB), 0, stream, a);
  SVA_CHECK_LAUNCH("class_extract_kernel");
  if (a.p.B <= 0) return SVA_OK;
  if (a.fv.out == nullptr) return launch_class_budget_nov(a, items, stream);
  const int kv = a.fv.kv_dtype;
  if (a.fv.D == 64) {
    if (kv == BF16) return launch_class_budget_v64_bf16(a, items, stream);
    if (kv == F16) return launch_class_budget_v64_f16(a, items, stream);
    return launch_class_budget_v64_f32(a, items, stream);
  }
  if (kv == BF16) return launch_class_budget_v128_bf16(a, items, stream);
  if (kv == F16) return launch_class_budget_v128_f16(a, items, stream);
  return launch_class_budget_v128_f32(a, items, stream);
}

}  // namespace

int launch_class(const ClassArgs& a, int64_t items, bool masked, const QueryLaunch* query, hipStream_t stream) {
  return masked ? launch_class_m<true>(a, items, query, stream) : launch_class_m<false>(a, items, query, stream);
}

int launch_class_budget_nov(const ClassArgs& a, int64_t items, hipStream_t stream) {
  return launch_class_budget<0, F32>(a, items, stream);
}

}  // namespace wide
}  // namespace sva
