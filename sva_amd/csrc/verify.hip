// Exact verifier, GQA-aware (sva/llama.py:304-317 and :532-553).
//
// verify_part: one workgroup per (sequence, KV head g, token, slice).  The
// budget lists of the H/G query heads sharing g (ascending key indices) are
// staged in LDS; their concatenation in (head, position) order is cut into
// slices of at most EPW entries.  An entry is processed only by the slice
// holding its first occurrence (the lowest head whose list contains the key,
// found by binary search), so every selected K row and V row is read from HBM
// once per group and scored against every query head whose list holds it.
// Every global load of a phase is issued before any is used: the lists, the
// query rows and the counts together, then every K and V row of the slice.
// Scores are fp32 dot(K[n], q_h) * scaling; per head the slice keeps the
// maximum m, the sum z of exp(score - m) and the exp-weighted V sum.
// verify_combine: one workgroup per query item merges the slices (all loaded
// at once, max-rescaled sums) and stores acc / z in the output dtype.
// Many groups (the prefill shape: thousands of tokens): one workgroup per
// (sequence, KV head, token) walks all its slices in order instead, keeping
// a running maximum, exp-sum and weighted V sum per head (each slice's sums
// rescaled to the new maximum), and stores the output itself: the groups
// alone fill the GPU, and no slice partials go through HBM.
#include <mutex>

#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

constexpr int VB = 256;   // threads per part workgroup: 4 lanes per entry
constexpr int EPW = VB / 4;  // union entries per slice
constexpr int MAX_GRP = 8;
constexpr int MAX_D = 256;
constexpr int CB = 256;   // threads per combine workgroup
constexpr int SEQ_MIN_GROUPS = 2048;  // groups from which one workgroup walks all slices of a group
constexpr int ACC = (MAX_GRP * MAX_D + VB - 1) / VB;  // (head, dim) outputs per thread, walking form

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
  bool kv_vec;  // rows start 8-byte (half types) / 16-byte (fp32) aligned: 4-element vector loads
  const int64_t* offs;
  const int64_t* lens;
  int64_t N;
  const int32_t* fin_idx;
  const int32_t* fin_count;
  int H, G, Q, D, B, split;
  int groups;  // n_seq * G * Q
  float scaling;
  float* part;  // [items, split, D + 2]: m, z, acc[D]
  void* out;
  int out_dtype;
  int64_t o_bs, o_hs, o_ts;
};

// DT: compile-time head_dim (0: runtime p.D, a multiple of 16; -1: any
// head_dim, elementwise).  Each of the 4 lanes of an entry holds D/4
// consecutive dimensions of its K and V rows (every 4th one for DT = -1).
template <int DT, bool SEQ>
__global__ void __launch_bounds__(VB) verify_part_kernel(VerifyParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int D = DT > 0 ? DT : p.D;
  const int grp = p.H / p.G;
  // SEQ: one workgroup per group, head-major group ranges per XCD
  // (xcd_range_item), so one XCD's L2 holds the K/V rows of one or two heads
  const int s = SEQ ? 0 : (int)blockIdx.x;
  const int64_t gx = SEQ ? sva::xcd_range_item((int64_t)blockIdx.x, p.groups) : (int64_t)blockIdx.y;
  if (gx < 0) return;  // block-uniform: past the last group
  const int gi = (int)gx;
  const int t = gi % p.Q;
  const int g = (gi / p.Q) % p.G;
  const int b = gi / (p.Q * p.G);
  const int B = p.B;
  int32_t* lists = (int32_t*)lds;                     // [grp][B]
  float* qv = (float*)(lists + grp * B);              // [grp][D]
  float* vrow = qv + grp * D;                         // [EPW][D + 1] (padded: no bank conflicts)
  float* wt = vrow + EPW * (D + 1);                   // [EPW][MAX_GRP] scores, then weights
  int* cnt = (int*)(wt + EPW * MAX_GRP);              // [MAX_GRP + 1] prefix of list lengths
  float* stat = (float*)(cnt + MAX_GRP + 1);          // [MAX_GRP][2]
  float* run = stat + 2 * MAX_GRP;                    // [MAX_GRP][3] running m, z and rescale factor (SEQ)

  const int64_t len = p.lens ? p.lens[b] : p.N;
  const int64_t off = p.offs ? p.offs[b] : 0;
  const int64_t item0 = ((int64_t)b * p.H + (int64_t)g * grp) * p.Q + t;  // head j: item0 + j * Q
  // phase 1: counts, lists (all B slots) and query rows in one round of loads
  if ((int)threadIdx.x < grp) cnt[threadIdx.x + 1] = max(0, min(p.fin_count[item0 + threadIdx.x * p.Q], B));
  for (int e = threadIdx.x; e < grp * B; e += VB) {
    const int j = e / B;
    lists[e] = p.fin_idx[(item0 + (int64_t)j * p.Q) * B + (e - j * B)];
  }
  for (int e = threadIdx.x; e < grp * D; e += VB) {
    const int j = e / D;
    const int64_t qb = (int64_t)b * p.q_bs + (int64_t)(g * grp + j) * p.q_hs + (int64_t)t * p.q_ts;
    qv[e] = load_elem(p.q, qb + (e - j * D), p.q_dtype);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    cnt[0] = 0;
    for (int j = 0; j < grp; ++j) cnt[j + 1] += cnt[j];
  }
  __syncthreads();
  const int M = cnt[grp];
  constexpr int NACC = !SEQ ? 1 : (DT > 0 ? (MAX_GRP * DT + VB - 1) / VB : ACC);
  float acc_run[NACC];
#pragma unroll
  for (int k = 0; k < NACC; ++k) acc_run[k] = 0.0f;
  if (SEQ && (int)threadIdx.x < grp) {
    run[3 * threadIdx.x] = -INFINITY;
    run[3 * threadIdx.x + 1] = 0.0f;
  }
  const int n_slices = SEQ ? (M + EPW - 1) / EPW : 1;
  for (int sl = 0; sl < n_slices; ++sl) {
  const int e0 = SEQ ? sl * EPW : (int)((int64_t)s * M / p.split);
  const int n = SEQ ? min(EPW, M - e0) : (int)((int64_t)(s + 1) * M / p.split) - e0;  // <= EPW
  // phase 2: first occurrences of the slice and the heads holding each; the
  // 4 lanes of an entry search lists qt and qt + 4.  The 4 lanes of an entry
  // share a wave, so the entry state stays in registers.
  {
    const int r = threadIdx.x >> 2;
    const int qt = threadIdx.x & 3;
    const int dq = D / 4;
    int j = 0;
    int32_t x = -1;
    if (r < n) {
      const int e = e0 + r;
      while (j + 1 < grp && e >= cnt[j + 1]) ++j;
      x = lists[j * B + (e - cnt[j])];
    }
    const bool valid = r < n && x >= 0 && (int64_t)x < len;
    uint32_t found = 0u;
    if (valid) {
      for (int jj = qt; jj < grp; jj += 4)
        if (jj == j || bsearch_i32(lists + jj * B, cnt[jj + 1] - cnt[jj], x) >= 0) found |= 1u << jj;
    }
    found |= __shfl_xor(found, 1, 4);
    found |= __shfl_xor(found, 2, 4);
    const bool own = valid && (found & ((1u << j) - 1u)) == 0u;  // no lower head holds the key
    const uint32_t mem = own ? found : 0u;
    // phase 3: every owned K and V row of the slice, 4 lanes per row
    float dot[MAX_GRP];
#pragma unroll
    for (int jj = 0; jj < MAX_GRP; ++jj) dot[jj] = 0.0f;
    if (DT < 0) {
      // any head_dim: lane qt takes dimensions qt, qt + 4, ...
      if (mem != 0u) {
        const int64_t rowb = (int64_t)g * p.kv_hs + (off + x) * p.kv_rs;
        for (int d = qt; d < D; d += 4) {
          const float kk = load_elem(p.keys, rowb + d, p.kv_dtype);
          vrow[r * (D + 1) + d] = load_elem(p.values, rowb + d, p.kv_dtype);
#pragma unroll
          for (int jj = 0; jj < MAX_GRP; ++jj)
            if (jj < grp) dot[jj] = __builtin_fmaf(kk, qv[jj * D + d], dot[jj]);
        }
      } else if (r < n) {
        for (int d = qt; d < D; d += 4) vrow[r * (D + 1) + d] = 0.0f;  // weight 0 must not meet NaN
      }
    } else if (mem != 0u) {
      const int64_t rowe = (int64_t)g * p.kv_hs + (off + x) * p.kv_rs + qt * dq;
      constexpr int NCH = (DT > 0 ? DT : MAX_D) / 16;  // 4-element chunks per lane (DT >= 0)
      float kv[NCH][4], vv[NCH][4];
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (DT > 0 || 4 * c < dq) {
          load4(p.keys, rowe + 4 * c, p.kv_dtype, p.kv_vec, kv[c]);
          load4(p.values, rowe + 4 * c, p.kv_dtype, p.kv_vec, vv[c]);
        }
      }
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (DT > 0 || 4 * c < dq) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int d = qt * dq + 4 * c + k;
            vrow[r * (D + 1) + d] = vv[c][k];
#pragma unroll
            for (int jj = 0; jj < MAX_GRP; ++jj)
              if (jj < grp) dot[jj] = __builtin_fmaf(kv[c][k], qv[jj * D + d], dot[jj]);
          }
        }
      }
    } else if (r < n) {
      for (int d = qt * dq; d < (qt + 1) * dq; ++d) vrow[r * (D + 1) + d] = 0.0f;  // weight 0 must not meet NaN
    }
#pragma unroll
    for (int jj = 0; jj < MAX_GRP; ++jj) {
      if (jj < grp) {
        float v = dot[jj];
        v += __shfl_xor(v, 1, 4);
        v += __shfl_xor(v, 2, 4);
        if (qt == 0) wt[r * MAX_GRP + jj] = ((mem >> jj) & 1u) ? v * p.scaling : -INFINITY;
      }
    }
  }
  __syncthreads();
  // phase 4: per head, max and exp-sum over the slice (one wave per head);
  // walking all slices, the maximum is the running one and the running sums
  // are rescaled to it
  const int wid = threadIdx.x / WAVE;
  for (int j = wid; j < grp; j += VB / WAVE) {
    const int r = lane_id();
    const float sc = r < n ? wt[r * MAX_GRP + j] : -INFINITY;
    const float m_old = SEQ ? run[3 * j] : -INFINITY;
    const float m = fmaxf(wave_max(sc), m_old);
    const float e = (m == -INFINITY || sc == -INFINITY) ? 0.0f : expf(sc - m);
    wt[r * MAX_GRP + j] = e;
    const float z = wave_sum(e);
    if (r == 0) {
      if (SEQ) {
        const float f = m_old == -INFINITY ? 0.0f : expf(m_old - m);
        run[3 * j] = m;
        run[3 * j + 1] = run[3 * j + 1] * f + z;
        run[3 * j + 2] = f;
      } else {
        stat[2 * j] = m;
        stat[2 * j + 1] = z;
      }
    }
  }
  __syncthreads();
  // phase 5: exp-weighted V sums, one (head, dim) per thread
  if (SEQ) {
#pragma unroll
    for (int k = 0; k < NACC; ++k) {
      const int e = (int)threadIdx.x + k * VB;
      if (e < grp * D) {
        const int j = e / D, d = e - j * D;
        float acc = 0.0f;
        for (int r = 0; r < n; ++r) acc = acc + wt[r * MAX_GRP + j] * vrow[r * (D + 1) + d];
        acc_run[k] = acc_run[k] * run[3 * j + 2] + acc;
      }
    }
    __syncthreads();  // the next slice overwrites the rows and weights
  } else {
    for (int e = threadIdx.x; e < grp * D; e += VB) {
      const int j = e / D, d = e - j * D;
      float acc = 0.0f;
      for (int r = 0; r < n; ++r) acc = acc + wt[r * MAX_GRP + j] * vrow[r * (D + 1) + d];
      float* dst = p.part + ((item0 + (int64_t)j * p.Q) * p.split + s) * (D + 2);
      dst[2 + d] = acc;
      if (d == 0) {
        dst[0] = stat[2 * j];
        dst[1] = stat[2 * j + 1];
      }
    }
  }
  }  // slices
  if (SEQ) {
#pragma unroll
    for (int k = 0; k < NACC; ++k) {
      const int e = (int)threadIdx.x + k * VB;
      if (e < grp * D) {
        const int j = e / D, d = e - j * D;
        const float m = run[3 * j], z = run[3 * j + 1];
        const float v = (m > -INFINITY && z > 0.0f) ? acc_run[k] / z : 0.0f;
        const int64_t o = (int64_t)b * p.o_bs + (int64_t)(g * grp + j) * p.o_hs + (int64_t)t * p.o_ts + d;
        store_elem(p.out, o, p.out_dtype, v);
      }
    }
  }
}

__global__ void __launch_bounds__(CB) verify_combine_kernel(VerifyParams p) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  float* fs = (float*)lds;  // [split] rescale factor of each slice
  __shared__ float red[CB / WAVE];
  const int item = blockIdx.x;
  const int t = item % p.Q;
  const int h = (item / p.Q) % p.H;
  const int b = item / (p.Q * p.H);
  const int D = p.D;
  const int split = p.split;
  const float* src = p.part + (int64_t)item * split * (D + 2);
  // maximum over slices
  float m = -INFINITY;
  for (int s = threadIdx.x; s < split; s += CB) m = fmaxf(m, src[(int64_t)s * (D + 2)]);
  m = wave_max(m);
  if (lane_id() == 0) red[threadIdx.x / WAVE] = m;
  __syncthreads();
  float M = red[0];
  for (int w = 1; w < CB / WAVE; ++w) M = fmaxf(M, red[w]);
  __syncthreads();
  // per-slice factors and the total exp-sum
  float z = 0.0f;
  for (int s = threadIdx.x; s < split; s += CB) {
    const float ms = src[(int64_t)s * (D + 2)];
    const float f = (ms == -INFINITY) ? 0.0f : expf(ms - M);
    fs[s] = f;
    z = z + f * src[(int64_t)s * (D + 2) + 1];
  }
  z = wave_sum(z);
  if (lane_id() == 0) red[threadIdx.x / WAVE] = z;
  __syncthreads();
  float Z = 0.0f;
  for (int w = 0; w < CB / WAVE; ++w) Z = Z + red[w];
  for (int d = threadIdx.x; d < D; d += CB) {
    float acc = 0.0f;
    int s = 0;
    for (; s + 8 <= split; s += 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = src[(int64_t)(s + k) * (D + 2) + 2 + d];
#pragma unroll
      for (int k = 0; k < 8; ++k) acc = acc + fs[s + k] * v[k];
    }
    for (; s < split; ++s) acc = acc + fs[s] * src[(int64_t)s * (D + 2) + 2 + d];
    const float v = (M > -INFINITY && Z > 0.0f) ? acc / Z : 0.0f;
    const int64_t o = (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)t * p.o_ts + d;
    store_elem(p.out, o, p.out_dtype, v);
  }
}

// ---------------------------------------------------------------------------
// Row-streaming verifier.  WPI = 1 (many items: the prefill): one wave per
// query item walks its own budget list with an online softmax, no barriers,
// four items per workgroup.  WPI > 1 (few items: a decode step, a ragged
// batch): one workgroup of WPI waves per item, wave w taking the item's
// octet rounds w, w + WPI, ..., so a decode head's 512 rows are one round of
// loads per wave; the waves' partials merge through LDS.  Lane octet o takes
// entry 8 r + o of round r; lane c of an octet holds elements
// [c * D/8, (c + 1) * D/8) of the query, of each K and V row it reads and of
// its accumulator, so a row is the octet's coalesced 16-byte loads and a
// score is one octet sum.  A wave's eight octets merge by cross-lane sums.
// A row that several heads of a KV group choose is read once per head:
// items run in head-major ranges per XCD, so the group's K and V stay in
// that XCD's L2.
constexpr int RB = 256;   // threads per workgroup at WPI = 1: 4 items
constexpr int RWPI = 16;  // waves per item of the few-item form

template <int D, int KV, int WPI>
__global__ void __launch_bounds__(WPI == 1 ? RB : WPI * WAVE)
    verify_rows_kernel(VerifyParams p, int64_t items, int64_t blocks) {
#pragma clang fp contract(off)
  constexpr int DL = D / 8;                             // elements per lane
  constexpr int ES = KV == F32 ? 4 : 2;                 // element bytes
  constexpr int NV = DL * ES / 16;                      // 16-byte loads per lane and row
  constexpr int U = NV == 1 ? 4 : (NV == 2 ? 2 : 1);    // entries per octet in flight
  static_assert(NV >= 1 && NV * 16 == DL * ES, "rows of whole 16-byte lane slices");
  __shared__ float part[WPI > 1 ? WPI : 1][D + 2];      // WPI > 1: each wave's m, z and sums
  const int64_t blk = xcd_range_item((int64_t)blockIdx.x, blocks);
  const int wid = (int)threadIdx.x / WAVE;
  const int64_t item = WPI > 1 ? blk : blk * (RB / WAVE) + wid;
  const int w = WPI > 1 ? wid : 0;  // this wave's share of the item's rounds
  if (blk < 0 || item >= items) return;  // uniform per workgroup (WPI > 1) or wave (WPI = 1)
  const int lane = lane_id(), oc = lane >> 3, c = lane & 7;
  const int t = (int)(item % p.Q);
  const int hq = (int)((item / p.Q) % p.H);
  const int b = (int)(item / ((int64_t)p.Q * p.H));
  const int g = hq / (p.H / p.G);
  const int64_t len = p.lens ? p.lens[b] : p.N;
  const int64_t off = p.offs ? p.offs[b] : 0;
  // no entry is valid in an empty sequence (row 0 then need not exist)
  const int cnt = len > 0 ? max(0, min(p.fin_count[item], p.B)) : 0;
  float q[DL];
  const int64_t qb = (int64_t)b * p.q_bs + (int64_t)hq * p.q_hs + (int64_t)t * p.q_ts + c * DL;
#pragma unroll
  for (int i = 0; i < DL; ++i) q[i] = load_elem(p.q, qb + i, p.q_dtype);
  const int32_t* list = p.fin_idx + item * p.B;
  const int64_t lane0 = (int64_t)g * p.kv_hs + off * p.kv_rs + c * DL;  // element offset of row 0's slice
  const uint4* kb = reinterpret_cast<const uint4*>((const char*)p.keys + lane0 * ES);
  const uint4* vb = reinterpret_cast<const uint4*>((const char*)p.values + lane0 * ES);
  const int64_t rs4 = p.kv_rs * ES / 16;  // row stride in 16-byte words
  float m = -INFINITY, z = 0.0f, acc[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) acc[i] = 0.0f;
  auto unpack = [](const uint4 (&w)[NV], float (&x)[DL]) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const uint32_t u[4] = {w[v].x, w[v].y, w[v].z, w[v].w};
      if constexpr (KV == F32) {
#pragma unroll
        for (int k = 0; k < 4; ++k) x[4 * v + k] = __uint_as_float(u[k]);
      } else if constexpr (KV == BF16) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          x[8 * v + 2 * k] = __uint_as_float(u[k] << 16);
          x[8 * v + 2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          x[8 * v + 2 * k] = __half2float(__ushort_as_half((unsigned short)(u[k] & 0xFFFFu)));
          x[8 * v + 2 * k + 1] = __half2float(__ushort_as_half((unsigned short)(u[k] >> 16)));
        }
      }
    }
  };
  // this wave's rounds r = w + WPI j hold entries 8 r + o (octet o); lane
  // 8 k + o holds the entry of round j0 + k, position o, of the current
  // block of eight rounds
  const int rounds = (cnt + 7) / 8;
  const int mine = rounds > w ? (rounds - w + WPI - 1) / WPI : 0;
  auto entry = [&](int j, int o) { return 8 * (w + WPI * j) + o; };
  int nxt = (lane >> 3) < mine && entry(lane >> 3, lane & 7) < cnt ? list[entry(lane >> 3, lane & 7)] : -1;
  for (int j0 = 0; j0 < mine; j0 += 8) {
    const int cur = nxt;  // the entry of round j0 + l / 8, position l % 8, in lane l; -1 past the count
    {
      const int jn = j0 + 8 + (lane >> 3);
      nxt = jn < mine && entry(jn, lane & 7) < cnt ? list[entry(jn, lane & 7)] : -1;
    }
    const int nk = min(8, mine - j0);          // rounds of this block
    for (int k0 = 0; k0 < nk; k0 += U) {       // k0 + u < 8: U divides 8
      uint4 kw[U][NV], vw[U][NV];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int x = __shfl(cur, 8 * (k0 + u) + oc, WAVE);
        ok[u] = x >= 0 && (int64_t)x < len;
        const int64_t ro = (int64_t)(ok[u] ? x : 0) * rs4;  // an invalid entry reads row 0, weight 0
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          kw[u][v] = kb[ro + v];
          vw[u][v] = vb[ro + v];
        }
      }
      float sc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float k[DL];
        unpack(kw[u], k);
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < DL; ++i) d = __builtin_fmaf(k[i], q[i], d);
        d = octet_sum(d);
        sc[u] = ok[u] ? d * p.scaling : -INFINITY;
      }
      float mn = m;
#pragma unroll
      for (int u = 0; u < U; ++u) mn = fmaxf(mn, sc[u]);
      const float corr = mn == -INFINITY ? 1.0f : __expf(m - mn);
      z = z * corr;
#pragma unroll
      for (int i = 0; i < DL; ++i) acc[i] = acc[i] * corr;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float w = sc[u] == -INFINITY ? 0.0f : __expf(sc[u] - mn);
        float v[DL];
        unpack(vw[u], v);
        z = z + w;
#pragma unroll
        for (int i = 0; i < DL; ++i) acc[i] = __builtin_fmaf(w, ok[u] ? v[i] : 0.0f, acc[i]);  // weight 0 meets no NaN
      }
      m = mn;
    }
  }
  // merge the eight octets: the wave maximum, then the rescaled sums
  float M = m;
  M = fmaxf(M, __shfl_xor(M, 8, WAVE));
  M = fmaxf(M, __shfl_xor(M, 16, WAVE));
  M = fmaxf(M, __shfl_xor(M, 32, WAVE));
  const float f = m == -INFINITY ? 0.0f : __expf(m - M);
  float Z = z * f;
  Z = Z + __shfl_xor(Z, 8, WAVE);
  Z = Z + __shfl_xor(Z, 16, WAVE);
  Z = Z + __shfl_xor(Z, 32, WAVE);
  const int64_t ob = (int64_t)b * p.o_bs + (int64_t)hq * p.o_hs + (int64_t)t * p.o_ts;
#pragma unroll
  for (int i = 0; i < DL; ++i) {
    float a = acc[i] * f;
    a = a + __shfl_xor(a, 8, WAVE);
    a = a + __shfl_xor(a, 16, WAVE);
    a = a + __shfl_xor(a, 32, WAVE);
    if constexpr (WPI == 1) {
      if (oc == 0) store_elem(p.out, ob + c * DL + i, p.out_dtype, (M > -INFINITY && Z > 0.0f) ? a / Z : 0.0f);
    } else {
      if (oc == 0) part[w][2 + c * DL + i] = a;
    }
  }
  if constexpr (WPI > 1) {
    // the waves' partials: the item's maximum, then the rescaled sums
    if (lane == 0) {
      part[w][0] = M;
      part[w][1] = Z;
    }
    __syncthreads();
    const int d = (int)threadIdx.x;
    if (d < D) {
      float Mi = -INFINITY;
#pragma unroll
      for (int v = 0; v < WPI; ++v) Mi = fmaxf(Mi, part[v][0]);
      float Zi = 0.0f, a = 0.0f;
#pragma unroll
      for (int v = 0; v < WPI; ++v) {
        const float fv = part[v][0] == -INFINITY ? 0.0f : __expf(part[v][0] - Mi);
        Zi = Zi + part[v][1] * fv;
        a = a + part[v][2 + d] * fv;
      }
      store_elem(p.out, ob + d, p.out_dtype, (Mi > -INFINITY && Zi > 0.0f) ? a / Zi : 0.0f);
    }
  }
}

// The many-item verifier takes D = 64 or 128 with K and V rows whose lane
// slices are whole aligned 16-byte words.
bool verify_rows_eligible(const void* keys, const void* values, int kv_dtype, int64_t kv_head_stride,
                          int64_t kv_row_stride, int64_t D) {
  if (D != 64 && D != 128) return false;
  const int64_t es = kv_dtype == F32 ? 4 : 2;
  return (((uintptr_t)keys | (uintptr_t)values) & 15u) == 0 && (kv_head_stride * es) % 16 == 0 &&
         (kv_row_stride * es) % 16 == 0;
}

template <int D, int KV, int WPI>
int launch_rows(const VerifyParams& p, int64_t items, hipStream_t stream) {
  const int64_t blocks = WPI > 1 ? items : (items + RB / WAVE - 1) / (RB / WAVE);
  hipLaunchKernelGGL((verify_rows_kernel<D, KV, WPI>), dim3((unsigned)xcd_range_grid(blocks)),
                     dim3(WPI > 1 ? WPI * WAVE : RB), 0, stream, p, items, blocks);
  SVA_CHECK_LAUNCH("verify_rows_kernel");
  return SVA_OK;
}

template <int WPI>
int launch_rows_any(const VerifyParams& p, int64_t items, hipStream_t stream) {
  if (p.D == 64) {
    if (p.kv_dtype == BF16) return launch_rows<64, BF16, WPI>(p, items, stream);
    if (p.kv_dtype == F16) return launch_rows<64, F16, WPI>(p, items, stream);
    return launch_rows<64, F32, WPI>(p, items, stream);
  }
  if (p.kv_dtype == BF16) return launch_rows<128, BF16, WPI>(p, items, stream);
  if (p.kv_dtype == F16) return launch_rows<128, F16, WPI>(p, items, stream);
  return launch_rows<128, F32, WPI>(p, items, stream);
}

int verify_split(int64_t grp, int64_t B) {
  const int64_t m = grp * B;
  return (int)std::max<int64_t>(1, (m + EPW - 1) / EPW);
}

size_t verify_lds_bytes(int64_t grp, int64_t B, int64_t D) {
  return sizeof(int32_t) * grp * B + sizeof(float) * grp * D + sizeof(float) * EPW * (D + 1) +
         sizeof(float) * EPW * MAX_GRP + sizeof(int) * (MAX_GRP + 1) +
         sizeof(float) * 5 * MAX_GRP + 16;
}

template <int DT, bool SEQ>
int launch_part(const VerifyParams& p, dim3 grid, size_t lds, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((verify_part_kernel<DT, SEQ>), sva::kMaxLds, "hipFuncSetAttribute(verify_part_kernel)");
  hipLaunchKernelGGL((verify_part_kernel<DT, SEQ>), grid, dim3(VB), lds, stream, p);
  SVA_CHECK_LAUNCH("verify_part_kernel");
  return SVA_OK;
}

template <bool SEQ>
int launch_part_dim(const VerifyParams& p, dim3 grid, size_t lds, hipStream_t stream) {
  if (p.D == 64) return launch_part<64, SEQ>(p, grid, lds, stream);
  if (p.D == 128) return launch_part<128, SEQ>(p, grid, lds, stream);
  if (p.D % 16 == 0) return launch_part<0, SEQ>(p, grid, lds, stream);
  return launch_part<-1, SEQ>(p, grid, lds, stream);
}

bool verify_walks_slices(int64_t n_seq, int64_t G, int64_t Q) { return n_seq * G * Q >= SEQ_MIN_GROUPS; }

// Slice partials of sva_verify_noalloc: a static device array, one copy per
// GPU the library runs on, held until the process ends.  Host code never
// passes the array's name to a kernel (on the host it is only a stand-in
// symbol): each device's address comes from hipGetSymbolAddress, taken once
// with that device current, and is used wherever host code needs the array.
static __device__ __align__(256) unsigned char scratch[SVA_VERIFY_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices];

// Address of the current device's scratch (set up on its first call).
int current_device_scratch(void** out) {
  int dev = -1;
  SVA_CHECK_HIP(hipGetDevice(&dev), "sva_verify_noalloc: hipGetDevice");
  SVA_UNSUPPORTED(dev >= 0 && dev < kMaxScratchDevices, "sva_verify_noalloc: device %d beyond the %d supported", dev,
                  kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    SVA_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "sva_verify_noalloc: hipGetSymbolAddress(scratch)");
    SVA_REQUIRE(ptr != nullptr && ((uintptr_t)ptr & 255u) == 0, "sva_verify_noalloc: scratch address unusable");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SVA_OK;
}

}  // namespace

extern "C" size_t sva_verify_workspace_bytes(int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D, int64_t B) {
  if (n_seq <= 0 || H <= 0 || G <= 0 || Q <= 0 || D <= 0 || B <= 0 || H % G != 0) return 0;
  if (verify_walks_slices(n_seq, G, Q)) return 256;  // no slice partials
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
  SVA_REQUIRE(D > 0 && D <= MAX_D, "sva_verify: head_dim %lld out of range (at most %d)", (long long)D, MAX_D);
  SVA_REQUIRE(q_dtype >= 0 && q_dtype <= 2 && kv_dtype >= 0 && kv_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
              "sva_verify: bad dtype");
  const int64_t grp = H / G;
  const size_t lds = verify_lds_bytes(grp, B, D);
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_verify: budget %lld with %lld heads per KV head exceeds LDS",
                  (long long)B, (long long)grp);
  const size_t need = sva_verify_workspace_bytes(n_seq, H, G, Q, D, B);
  SVA_REQUIRE(workspace != nullptr && workspace_bytes >= need, "sva_verify: workspace of %zu bytes required", need);
  const int split = verify_split(grp, B);
  SVA_REQUIRE(n_seq * G * Q < (1ll << 31) && n_seq * H * Q < (1ll << 31), "sva_verify: too many items");
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
  const uintptr_t kv_align = kv_dtype == 0 ? 15u : 7u;
  p.kv_vec = (((uintptr_t)keys | (uintptr_t)values) & kv_align) == 0 && kv_head_stride % 4 == 0 &&
             kv_row_stride % 4 == 0;
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
  p.groups = (int)(n_seq * G * Q);
  p.scaling = scaling;
  p.part = (float*)workspace;
  p.out = out;
  p.out_dtype = out_dtype;
  p.o_bs = out_seq_stride;
  p.o_hs = out_head_stride;
  p.o_ts = out_tok_stride;
  const bool rows = verify_rows_eligible(keys, values, kv_dtype, kv_head_stride, kv_row_stride, D);
  if (verify_walks_slices(n_seq, G, Q)) {
    if (rows) return launch_rows_any<1>(p, n_seq * H * Q, (hipStream_t)stream);
    return launch_part_dim<true>(p, dim3((unsigned)sva::xcd_range_grid(n_seq * G * Q)), lds, (hipStream_t)stream);
  }
  // few items with budgets of up to 2048 rows: one workgroup per item
  // (RWPI waves take at most four rounds of loads each); longer budgets
  // spread over the slice-split form's workgroups
  if (rows && B <= 2048) return launch_rows_any<RWPI>(p, n_seq * H * Q, (hipStream_t)stream);
  int rc = launch_part_dim<false>(p, dim3((unsigned)split, (unsigned)(n_seq * G * Q)), lds, (hipStream_t)stream);
  if (rc != SVA_OK) return rc;
  hipLaunchKernelGGL(verify_combine_kernel, dim3((unsigned)(n_seq * H * Q)), dim3(CB), sizeof(float) * (size_t)split,
                     (hipStream_t)stream, p);
  SVA_CHECK_LAUNCH("verify_combine_kernel");
  return SVA_OK;
}

extern "C" int sva_verify_noalloc(const void* q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride,
                                  int64_t q_tok_stride, const void* keys, const void* values, int kv_dtype,
                                  int64_t kv_head_stride, int64_t kv_row_stride, const int64_t* seq_offsets,
                                  const int64_t* seq_lens, int64_t n_keys, const int32_t* fin_idx,
                                  const int32_t* fin_count, int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D,
                                  int64_t B, float scaling, void* out, int out_dtype, int64_t out_seq_stride,
                                  int64_t out_head_stride, int64_t out_tok_stride, void* stream) {
  sva::clear_error();
  const size_t need = sva_verify_workspace_bytes(n_seq, H, G, Q, D, B);
  SVA_REQUIRE(need > 0, "sva_verify_noalloc: bad sizes");
  SVA_UNSUPPORTED(need <= (size_t)SVA_VERIFY_NOALLOC_SCRATCH_BYTES,
                  "sva_verify_noalloc: this call needs %zu bytes of slice partials, more than the %zu-byte static "
                  "scratch; use sva_verify with a workspace",
                  need, (size_t)SVA_VERIFY_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = current_device_scratch(&ws);
  if (rc != SVA_OK) return rc;
  return sva_verify(q, q_dtype, q_seq_stride, q_head_stride, q_tok_stride, keys, values, kv_dtype, kv_head_stride,
                    kv_row_stride, seq_offsets, seq_lens, n_keys, fin_idx, fin_count, n_seq, H, G, Q, D, B, scaling,
                    out, out_dtype, out_seq_stride, out_head_stride, out_tok_stride, ws,
                    (size_t)SVA_VERIFY_NOALLOC_SCRATCH_BYTES, stream);
}
