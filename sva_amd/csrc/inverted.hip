// Inverted-index summon (q = 1 decode): postings, candidates, unique refill
// selection with margin-adaptive budgets (sva/llama.py:330-425, :427-576,
// :626-693, :83-116).
//
// sva_postings_build   CSR postings per (head, subspace): offsets [C + 1] and
//                      key ids ascending within each cell (a stable counting
//                      sort; the reference's dense [.., max_bucket] table holds
//                      the same ids per cell, sva/llama.py:626-657).
// sva_inverted_candidates
//                      per head: the top `cells` cells of every subspace by
//                      LUT / sqrt(R) (ties: lower cell index), the posting
//                      lists of those cells (a key listed in several chosen
//                      cells appears once per list, as in the reference), the
//                      tail rows past the postings (static: all of them;
//                      adaptive: those whose code falls in a chosen cell) and
//                      one extra slot (static: the current row when there is
//                      no tail; adaptive: the current row, or the last allowed
//                      row as a fallback).  Every entry is rank-scored,
//                      (k_low . q_low) / sqrt(R) in torch's sum order, masked
//                      by the attention mask, and stored as a 64-bit composite
//                      (score key, key index).
// sva_unique_refill_select
//                      per head: refill window of the best min(width,
//                      max(B, factor B)) entries counted with multiplicity,
//                      first occurrence of each key, the margin-adaptive budget
//                      and the chosen keys (ascending) for sva_verify.
#include <cfloat>
#include <cmath>

#include "capi_internal.h"
#include "common.cuh"
#include "summon.h"

using namespace sva;

namespace {

// ---------------------------------------------------------------------------
// postings

constexpr int PB = 1024;
constexpr int PNW = PB / WAVE;
constexpr int kMaxPostingCells = 1024;

// One workgroup per (sequence b, head h, subspace s): the first n_rows rows of
// the sequence (rows_of[b] of a ragged batch), which start at packed row
// row0[b] (0 without one); ids hold sequence-local key indices at the
// sequence's own packed rows of the [H, S, ids_rows] table.
__global__ void __launch_bounds__(PB)
    postings_build_kernel(const void* __restrict__ codes, int ctype, int64_t code_hs, int H, int S, int n_rows, int C,
                          const int64_t* __restrict__ row0, const int64_t* __restrict__ rows_of, int64_t ids_rows,
                          int32_t* __restrict__ offsets, int32_t* __restrict__ ids, int32_t* __restrict__ max_count) {
  extern __shared__ __align__(16) unsigned char lds[];
  uint32_t* hist = (uint32_t*)lds;        // [C]
  uint32_t* cursor = hist + C;            // [C]
  uint32_t* wcnt = cursor + C;            // [PNW][C]
  uint32_t* scratch = wcnt + PNW * C;     // [PNW + 2]
  const int b = blockIdx.x / (H * S);
  const int hs = blockIdx.x - b * (H * S);
  const int h = hs / S, s = hs - h * S;
  const int64_t r0 = row0 ? row0[b] : 0;
  if (rows_of) n_rows = (int)rows_of[b];
  const int64_t cbase = (int64_t)h * code_hs + r0 * S + s;
  auto code_at = [&](int n) {
    int64_t c = load_code(codes, cbase + (int64_t)n * S, ctype);
    return (int)(c < 0 ? 0 : (c >= C ? C - 1 : c));
  };
  for (int c = threadIdx.x; c < C; c += PB) hist[c] = 0u;
  __syncthreads();
  for (int n = threadIdx.x; n < n_rows; n += PB) atomicAdd(&hist[code_at(n)], 1u);
  __syncthreads();
  int32_t* off = offsets + (int64_t)blockIdx.x * (C + 1);
  {
    uint32_t carry = 0, mx = 0;
    for (int c0 = 0; c0 < C; c0 += PB) {
      const int c = c0 + (int)threadIdx.x;
      const uint32_t v = c < C ? hist[c] : 0u;
      uint32_t tot;
      const uint32_t ex = block_excl_scan<PB>(v, scratch, &tot);
      if (c < C) {
        off[c] = (int32_t)(carry + ex);
        cursor[c] = carry + ex;
        mx = max(mx, v);
      }
      carry += tot;
    }
    if (threadIdx.x == 0) {
      off[C] = n_rows;
      scratch[PNW] = 0u;
    }
    __syncthreads();
    atomicMax(&scratch[PNW], mx);
    __syncthreads();
    if (threadIdx.x == 0) max_count[blockIdx.x] = (int32_t)scratch[PNW];
    __syncthreads();
  }
  int bits = 0;
  while ((1 << bits) < C) ++bits;
  const int wid = threadIdx.x / WAVE;
  int32_t* out = ids + (int64_t)hs * ids_rows + r0;
  for (int base = 0; base < n_rows; base += PB) {
    for (int i = threadIdx.x; i < PNW * C; i += PB) wcnt[i] = 0u;
    __syncthreads();
    const int n = base + (int)threadIdx.x;
    const bool valid = n < n_rows;
    const int c = valid ? code_at(n) : 0;
    // lanes of this wave holding the same code
    uint64_t same = __builtin_amdgcn_ballot_w64(valid);
    for (int b = 0; b < bits; ++b) {
      const bool bit = (c >> b) & 1;
      const uint64_t m = __builtin_amdgcn_ballot_w64(bit);
      same &= bit ? m : ~m;
    }
    const uint64_t below = same & ((1ull << lane_id()) - 1ull);
    if (valid && below == 0ull) wcnt[wid * C + c] = (uint32_t)__popcll(same);  // the first lane of its code
    __syncthreads();
    for (int cc = threadIdx.x; cc < C; cc += PB) {
      uint32_t run = 0;
      for (int w = 0; w < PNW; ++w) {
        const uint32_t v = wcnt[w * C + cc];
        wcnt[w * C + cc] = run;
        run += v;
      }
      hist[cc] = run;  // this chunk's count of code cc
    }
    __syncthreads();
    if (valid) out[cursor[c] + wcnt[wid * C + c] + (uint32_t)__popcll(below)] = n;
    __syncthreads();
    for (int cc = threadIdx.x; cc < C; cc += PB) cursor[cc] += hist[cc];
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// candidates

constexpr int CT = 256;          // threads per candidate workgroup
constexpr int TAIL_ROWS = 256;   // tail rows per workgroup
constexpr int SCORE_U = 4;       // entries in flight per 16-lane group while scoring (2 per octet)
constexpr int kMaxCells = 64;
constexpr int kMaxSub = 16;

struct CandParams {
  const float* lut;  // [H, S, C]
  const float* q_low;  // [H, R]
  const float* k_low;
  int64_t klow_hs;
  const void* codes;
  int ctype;
  int64_t code_hs;
  const int32_t* offsets;  // [H, S, C + 1]
  const int32_t* ids;      // [H, S, postings_len]
  int postings_len;
  int tail_start;
  int k_len;
  int H, S, C, R, cells;
  float sqrt_r;
  const void* mask;  // allowed iff mask[n] > -1e4 (MASK_* types), or NULL: every row
  int mask_type;
  int adaptive;
  int W;                     // slots per item
  uint64_t* comp;            // [items, W]; 0 = empty slot
  uint8_t* flag;             // [items, W]: bit 0 valid, bit 1 fallback entry
  // ragged batches (static mode): item b * H + h; sequence b starts at
  // packed row seq_offs[b], its postings cover its first plens[b] rows, its
  // tail is [plens[b], klens[b]); lists take S * postings_len slots and the
  // tail tail_cap slots.  NULL for one sequence (the scalars above).
  const int64_t* seq_offs;
  const int64_t* plens;
  const int64_t* klens;
  int tail_cap;
  int64_t ids_rows;  // row dimension of ids: [H, S, ids_rows]
  int32_t* nlist;    // ragged: [items] list entries of each item (list slots past them are left as they are)
};

SVA_DEV bool row_allowed(const CandParams& p, int n) {
  return p.mask == nullptr || mask_allows(p.mask, n, p.mask_type);
}

// Item geometry: the packed row of key 0, the postings length, the tail start
// and the key count of the item's sequence.
struct ItemRows {
  int64_t r0;
  int plen, tail_start, k_len;
};

SVA_DEV ItemRows item_rows(const CandParams& p, int b) {
  if (p.seq_offs == nullptr) return ItemRows{0, p.postings_len, p.tail_start, p.k_len};
  const int plen = (int)p.plens[b];
  return ItemRows{p.seq_offs[b], plen, plen, (int)p.klens[b]};
}

// Rank score of key n (16 lanes), torch's order, then / sqrt(R).  R == 64
// splits the row over the 16 lanes; other ranks are summed by the group's
// first lane.
SVA_DEV float rank_score16(const CandParams& p, int h, int item, int64_t r0, int n) {
#pragma clang fp contract(off)
  const float* row = p.k_low + (int64_t)h * p.klow_hs + (r0 + n) * p.R;
  const float* q = p.q_low + (int64_t)item * p.R;
  if (p.R != 64) {
    float t = 0.0f;
    if ((lane_id() & 15) == 0) t = torch_order_dot(row, q, p.R);
    return __shfl(t, 0, 16) / p.sqrt_r;
  }
  const int j = lane_id() & 15;
  const float4 r = reinterpret_cast<const float4*>(row)[j];
  const float4 qq = reinterpret_cast<const float4*>(q)[j];
  const float p0 = r.x * qq.x, p1 = r.y * qq.y, p2 = r.z * qq.z, p3 = r.w * qq.w;
  const float a0 = (0.0f + p0) + __shfl_down(p0, 8, 16);
  const float a1 = (0.0f + p1) + __shfl_down(p1, 8, 16);
  const float a2 = (0.0f + p2) + __shfl_down(p2, 8, 16);
  const float a3 = (0.0f + p3) + __shfl_down(p3, 8, 16);
  const float v0 = ((a0 + __shfl_down(a0, 2, 16)) + __shfl_down(a0, 4, 16)) + __shfl_down(a0, 6, 16);
  const float v1 = ((a1 + __shfl_down(a1, 2, 16)) + __shfl_down(a1, 4, 16)) + __shfl_down(a1, 6, 16);
  const float v2 = ((a2 + __shfl_down(a2, 2, 16)) + __shfl_down(a2, 4, 16)) + __shfl_down(a2, 6, 16);
  const float v3 = ((a3 + __shfl_down(a3, 2, 16)) + __shfl_down(a3, 4, 16)) + __shfl_down(a3, 6, 16);
  const float w0 = __shfl_down(v0, 1, 16), w1 = __shfl_down(v1, 1, 16);
  const float w2 = __shfl_down(v2, 1, 16), w3 = __shfl_down(v3, 1, 16);
  const float t = (((((((0.0f + v0) + v1) + v2) + v3) + w0) + w1) + w2) + w3;
  return __shfl(t, 0, 16) / p.sqrt_r;
}

SVA_DEV uint64_t entry_comp(bool valid, float score, int n) {
  return composite(f2key(valid ? score : -FLT_MAX), (uint32_t)n);
}

// Scores the entries [0, count) (16 lanes per entry, 4 entries per lane
// group in flight) and stores them; key_at(i) gives entry i's key, or -1 for
// a slot left empty.
template <typename KeyAt>
SVA_DEV void score_entries(const CandParams& p, int h, int item, int64_t r0, int count, KeyAt key_at, uint64_t* comp,
                           uint8_t* flag, uint8_t extra_flag) {
#pragma clang fp contract(off)
  constexpr int GROUPS = CT / 16;
  constexpr int U = SCORE_U;
  const int g = threadIdx.x >> 4;
  const int j = lane_id() & 15;
  auto store = [&](int i, int n, float sc) {
    if (n >= 0) {
      const bool ok = row_allowed(p, n);
      comp[i] = entry_comp(ok, sc, n);
      flag[i] = (uint8_t)((ok ? 1 : 0) | extra_flag);
    } else {
      comp[i] = 0ull;
      flag[i] = 0;
    }
  };
  if (p.R == 64) {
    const float* klow = p.k_low + (int64_t)h * p.klow_hs;
    const float4 qq = reinterpret_cast<const float4*>(p.q_low + (int64_t)item * 64)[j];
    for (int b0 = 0; b0 < count; b0 += GROUPS * U) {
      int n[U];
      float4 rv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = b0 + g + u * GROUPS;
        n[u] = i < count ? key_at(i) : -1;
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        rv[u] = n[u] >= 0 ? reinterpret_cast<const float4*>(klow + (r0 + n[u]) * 64)[j]
                          : float4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float dot = rank_dot64_row16(rv[u], qq);  // valid in the row's first lane
        const int i = b0 + g + u * GROUPS;
        if (i < count && j == 0) store(i, n[u], dot / p.sqrt_r);
      }
    }
    return;
  }
  for (int b = 0; b < count; b += GROUPS) {
    const int i = b + g;
    const bool live = i < count;
    const int n = live ? key_at(i) : -1;
    const float sc = rank_score16(p, h, item, r0, n >= 0 ? n : 0);
    if (live && j == 0) store(i, n, sc);
  }
}

// Whether key n's code falls in a chosen cell of one of the subspaces [0, s_end)
// (code_base: the head's codes at the sequence's first row).
SVA_DEV bool in_chosen_cells(const CandParams& p, const uint32_t* member, int64_t code_base, int n, int s_end) {
  for (int s = 0; s < s_end; ++s) {
    int64_t c = load_code(p.codes, code_base + (int64_t)n * p.S + s, p.ctype);
    c = c < 0 ? 0 : (c >= p.C ? p.C - 1 : c);
    if ((member[s * 8 + (c >> 5)] >> (c & 31)) & 1u) return true;
  }
  return false;
}

// The chosen lists of an item: the top `cells` cells of every subspace by
// LUT / sqrt(R) (ties: lower cell index) in topc (rank order), their cells
// as bits in member, and lbase[j] = the slot of list j's first entry
// (lbase[S * cells] = all list entries).  Every thread of the block calls it.
SVA_DEV void choose_lists(const CandParams& p, int item, float* score, int* topc, uint32_t* member, int* lbase,
                          uint32_t* scan_scratch) {
#pragma clang fp contract(off)
  const int S = p.S, C = p.C, cells = p.cells;
  // top cells of every subspace by LUT / sqrt(R), ties to the lower cell
  const float* item_lut = p.lut + (int64_t)item * S * C;
  for (int e = threadIdx.x; e < S * 8; e += CT) member[e] = 0u;
  for (int e = threadIdx.x; e < S * cells; e += CT) topc[e] = 0;
  if (cells <= 16) {
    // one wave per subspace: `cells` rounds of a wave arg-max over composite
    // keys (score key, cell), 4 cells per lane
    __syncthreads();
    const int lane = lane_id();
    for (int s = (int)threadIdx.x / WAVE; s < S; s += CT / WAVE) {
      uint64_t k[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = lane + WAVE * q;
        k[q] = c < C ? composite(f2key(item_lut[s * C + c] / p.sqrt_r), (uint32_t)c) : 0ull;
      }
      for (int r = 0; r < cells; ++r) {
        uint64_t m = k[0];
#pragma unroll
        for (int q = 1; q < 4; ++q) m = k[q] > m ? k[q] : m;
        m = wave_max_u64(m);
        const uint32_t c = composite_index(m);
        if (lane == 0) {
          topc[s * cells + r] = (int)c;
          atomicOr(&member[s * 8 + (c >> 5)], 1u << (c & 31));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (k[q] == m) k[q] = 0ull;
      }
    }
  } else {
    // rank of each cell among its subspace
    for (int e = threadIdx.x; e < S * C; e += CT) score[e] = item_lut[e] / p.sqrt_r;
    __syncthreads();
    for (int e = threadIdx.x; e < S * C; e += CT) {
      const int s = e / C, c = e - s * C;
      const float v = score[e];
      int rank = 0;
      for (int o = 0; o < C; ++o) {
        const float u = score[s * C + o];
        rank += (u > v) || (u == v && o < c);
      }
      if (rank < cells) {
        topc[s * cells + rank] = c;
        if (c < 256) atomicOr(&member[s * 8 + (c >> 5)], 1u << (c & 31));
      }
    }
  }
  __syncthreads();
  const int nlists = S * cells;
  const int32_t* item_off = p.offsets + (int64_t)item * S * (C + 1);  // [S, C + 1] of this item
  {
    // list sizes, all loaded at once, and their prefix
    uint32_t carry = 0;
    for (int j0 = 0; j0 < nlists; j0 += CT) {
      const int jj = j0 + (int)threadIdx.x;
      uint32_t sz = 0;
      if (jj < nlists) {
        const int32_t* off = item_off + (jj / cells) * (C + 1);
        const int c = min(max(topc[jj], 0), C - 1);
        sz = (uint32_t)max(0, off[c + 1] - off[c]);
      }
      uint32_t tot;
      const uint32_t ex = block_excl_scan<CT>(sz, scan_scratch, &tot);
      if (jj < nlists) lbase[jj] = (int)(carry + ex);
      carry += tot;
    }
    if (threadIdx.x == 0) lbase[nlists] = (int)carry;
  }
  __syncthreads();
}

__global__ void __launch_bounds__(CT) inverted_candidates_kernel(CandParams p) {
#pragma clang fp contract(off)
  extern __shared__ float score[];  // [S * C] for the ranking path (cells > 16) only
  __shared__ int topc[kMaxSub * kMaxCells];
  __shared__ uint32_t member[kMaxSub * 8];  // bit c of subspace s: cell c chosen (C <= 256)
  __shared__ int lbase[kMaxSub * kMaxCells + 1];
  __shared__ uint32_t scan_scratch[CT / WAVE + 1];
  const int item = blockIdx.y;
  const int h = item % p.H;
  const ItemRows ir = item_rows(p, item / p.H);
  choose_lists(p, item, score, topc, member, lbase, scan_scratch);
  const int S = p.S, C = p.C, cells = p.cells;
  const int nlists = S * cells;
  const int32_t* item_off = p.offsets + (int64_t)item * S * (C + 1);  // [S, C + 1] of this item
  uint64_t* comp = p.comp + (int64_t)item * p.W;
  uint8_t* flag = p.flag + (int64_t)item * p.W;
  const int tail_len = max(0, ir.k_len - ir.tail_start);
  const int tail_wgs = (p.tail_cap + TAIL_ROWS - 1) / TAIL_ROWS;
  const int j = blockIdx.x;
  const int64_t cb = (int64_t)h * p.code_hs + ir.r0 * S;  // the head's codes at the sequence's first row
  // slots: [lists (S * postings_len at most)] [tail (tail_cap)] [extra]
  const int tail_slot0 = S * p.postings_len;
  const int extra_slot = p.W - 1;
  if (j < nlists) {
    const int s = j / cells;
    const int32_t* off = item_off + s * (C + 1);
    const int c = min(max(topc[j], 0), C - 1);
    const int o0 = off[c];
    // lists fill at most S * postings_len slots; the clamp keeps a batch whose
    // lengths exceed the stated maxima inside its row of slots
    const int count = max(0, min(off[c + 1] - o0, tail_slot0 - lbase[j]));
    const int32_t* lst = p.ids + ((int64_t)h * S + s) * p.ids_rows + ir.r0 + o0;
    score_entries(
        p, h, item, ir.r0, count,
        [&](int i) {
          const int n = (int)lst[i];
          // adaptive: distinct keys, each kept by its lowest chosen subspace
          if (p.adaptive && in_chosen_cells(p, member, cb, n, s)) return -1;
          return n;
        },
        comp + lbase[j], flag + lbase[j], 0);
  } else if (j < nlists + tail_wgs) {
    const int t0 = (j - nlists) * TAIL_ROWS;
    const int count = min(TAIL_ROWS, p.tail_cap - t0);  // slots past this item's tail are cleared
    score_entries(
        p, h, item, ir.r0, count,
        [&](int i) {
          if (t0 + i >= tail_len) return -1;
          const int n = ir.tail_start + t0 + i;
          if (!p.adaptive) return n;
          return in_chosen_cells(p, member, cb, n, S) ? n : -1;
        },
        comp + tail_slot0 + t0, flag + tail_slot0 + t0, 0);
  } else {
    // the extra slot, and the list slots past the lists' total: cleared, or
    // (ragged) their count recorded so that the selection skips them
    if (p.nlist != nullptr) {
      if (threadIdx.x == 0) p.nlist[item] = min(lbase[nlists], tail_slot0);
    } else {
      for (int i = min(lbase[nlists], tail_slot0) + (int)threadIdx.x; i < tail_slot0; i += CT) comp[i] = 0ull, flag[i] = 0;
    }
    int n = -1;
    uint8_t extra = 0;
    if (!p.adaptive) {
      if (tail_len == 0) n = ir.k_len - 1;
    } else {
      n = ir.k_len - 1;
      if (row_allowed(p, n)) {
        // the current row joins the candidates unless it is one already
        if (in_chosen_cells(p, member, cb, n, S)) n = -1;
      } else {
        // fallback: the last allowed row, used only when nothing else is
        for (n = ir.k_len - 1; n >= 0 && !row_allowed(p, n); --n) {
        }
        extra = 2;
      }
    }
    score_entries(p, h, item, ir.r0, 1, [&](int) { return n; }, comp + extra_slot, flag + extra_slot, extra);
  }
}

// Ragged static batches, two launches balanced over the items' entries:
//   prep:  one workgroup per item chooses its lists (choose_lists), records
//          the item's list entries in nlist[item] and copies the lists' keys
//          into the item's list slots (coalesced runs of ids);
//   score: a fixed grid splits the live slots of all items (list entries,
//          tail slots, the extra slot) evenly over its workgroups, so one
//          oversized cell is scored by many CUs; each slot gets its
//          composite and flag as in inverted_candidates_kernel.
__global__ void __launch_bounds__(CT) ragged_cand_prep_kernel(CandParams p) {
  __shared__ int topc[kMaxSub * kMaxCells];
  __shared__ uint32_t member[kMaxSub * 8];
  __shared__ int lbase[kMaxSub * kMaxCells + 1];
  __shared__ uint32_t scan_scratch[CT / WAVE + 1];
  extern __shared__ float score[];
  const int item = blockIdx.x;
  const int h = item % p.H;
  const ItemRows ir = item_rows(p, item / p.H);
  choose_lists(p, item, score, topc, member, lbase, scan_scratch);
  const int S = p.S, C = p.C, cells = p.cells;
  const int nlists = S * cells;
  const int tail_slot0 = S * p.postings_len;
  const int32_t* item_off = p.offsets + (int64_t)item * S * (C + 1);
  uint64_t* comp = p.comp + (int64_t)item * p.W;
  for (int j = 0; j < nlists; ++j) {
    const int s = j / cells;
    const int c = min(max(topc[j], 0), C - 1);
    const int o0 = item_off[s * (C + 1) + c];
    const int count = max(0, min(lbase[j + 1] - lbase[j], tail_slot0 - lbase[j]));
    const int32_t* lst = p.ids + ((int64_t)h * S + s) * p.ids_rows + ir.r0 + o0;
    for (int i = threadIdx.x; i < count; i += CT) comp[lbase[j] + i] = (uint64_t)(uint32_t)lst[i];
  }
  if (threadIdx.x == 0) p.nlist[item] = min(lbase[nlists], tail_slot0);
}

constexpr int MAX_RAGGED_ITEMS = 8192;  // items of a ragged launch (the score kernel's prefix in LDS)

__global__ void __launch_bounds__(CT) ragged_cand_score_kernel(CandParams p, int items) {
#pragma clang fp contract(off)
  extern __shared__ int pre[];  // [items + 1] first live entry of each item
  __shared__ uint32_t scan_scratch[CT / WAVE + 1];
  const int live_extra = p.tail_cap + 1;  // tail slots and the extra slot of every item
  {
    uint32_t carry = 0;
    for (int i0 = 0; i0 < items; i0 += CT) {
      const int it = i0 + (int)threadIdx.x;
      const uint32_t v = it < items ? (uint32_t)(max(p.nlist[it], 0) + live_extra) : 0u;
      uint32_t tot;
      const uint32_t ex = block_excl_scan<CT>(v, scan_scratch, &tot);
      if (it < items) pre[it] = (int)(carry + ex);
      carry += tot;
    }
    if (threadIdx.x == 0) pre[items] = (int)carry;
  }
  __syncthreads();
  constexpr int GROUPS = CT / 8;  // lane octets, one entry each per round
  constexpr int U = SCORE_U / 2;  // entries in flight per octet
  const int total = pre[items];
  const int per = ((total + (int)gridDim.x - 1) / (int)gridDim.x + GROUPS * U - 1) / (GROUPS * U) * (GROUPS * U);
  const int e_begin = (int)blockIdx.x * per, e_end = min(total, e_begin + per);
  const int g = threadIdx.x >> 3;
  const int j = lane_id() & 7;
  const int tail_slot0 = p.S * p.postings_len;
  for (int b0 = e_begin; b0 < e_end; b0 += GROUPS * U) {
    int it[U], slot[U], n[U];
    int64_t r0[U];
    float4 ra[U], rb[U], qa[U], qb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = b0 + g + u * GROUPS;
      it[u] = -1;
      n[u] = -1;
      slot[u] = 0;
      r0[u] = 0;
      if (e < e_end) {
        int lo = 0, hi = items;  // last item whose first entry is <= e
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (pre[mid] <= e) lo = mid;
          else hi = mid;
        }
        it[u] = lo;
        const ItemRows ir = item_rows(p, lo / p.H);
        r0[u] = ir.r0;
        const int i = e - pre[lo];
        const int nl = pre[lo + 1] - pre[lo] - live_extra;
        const int tail_len = max(0, ir.k_len - ir.tail_start);
        if (i < nl) {
          slot[u] = i;
          n[u] = (int)(uint32_t)p.comp[(int64_t)lo * p.W + i];
        } else if (i < nl + p.tail_cap) {
          const int t = i - nl;
          slot[u] = tail_slot0 + t;
          n[u] = t < tail_len ? ir.tail_start + t : -1;
        } else {
          slot[u] = p.W - 1;
          n[u] = tail_len == 0 ? ir.k_len - 1 : -1;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = n[u] >= 0;
      const int hh = live ? it[u] % p.H : 0;
      const float4 zero = float4{0.0f, 0.0f, 0.0f, 0.0f};
      const float4* row = reinterpret_cast<const float4*>(p.k_low + (int64_t)hh * p.klow_hs + (r0[u] + n[u]) * 64);
      const float4* qrow = reinterpret_cast<const float4*>(p.q_low + (int64_t)it[u] * 64);
      ra[u] = live ? row[j] : zero;
      rb[u] = live ? row[8 + j] : zero;
      qa[u] = live ? qrow[j] : zero;
      qb[u] = live ? qrow[8 + j] : zero;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float dot = rank_dot64_oct8(ra[u], rb[u], qa[u], qb[u]);  // valid in the octet's first lane
      if (it[u] >= 0 && j == 0) {
        uint64_t* comp = p.comp + (int64_t)it[u] * p.W;
        uint8_t* flag = p.flag + (int64_t)it[u] * p.W;
        if (n[u] >= 0) {
          comp[slot[u]] = entry_comp(true, dot / p.sqrt_r, n[u]);
          flag[slot[u]] = 1;
        } else {
          comp[slot[u]] = 0ull;
          flag[slot[u]] = 0;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// unique refill select

constexpr int UB = 1024;
constexpr int UNW = UB / WAVE;
constexpr uint32_t EMPTY = 0xFFFFFFFFu;

struct SelParams {
  const uint64_t* comp;
  const uint8_t* flag;
  int W;
  int mode;  // 0 static decode, 1 adaptive decode, 2 plain top-unique
  int B, min_budget, mid_budget;
  float low_f, high_f;     // fp32 thresholds (static: tensor comparison)
  double low_d, high_d;    // fp64 thresholds (adaptive: Python float comparison)
  int64_t width;           // plain mode: candidate width
  const int32_t* max_count;  // static: per (head, subspace) largest cell of the postings
  int n_max;
  int64_t lists;           // static: S * cells
  int64_t tail_extra;      // static: tail rows, or 1 (the current row) without a tail
  int refill_factor;
  int win_cap;
  int hash;                // key table slots: a power of 2 >= 2 * win_cap
  uint64_t* win;           // [H, win_cap] workspace
  int32_t* fin_idx;        // [H, B] ascending (modes 0, 1)
  int32_t* fin_count;      // [H]
  float* stats;            // [H, 4]: summoned, refill_pool, verified, rank_count
  int32_t* sel_idx;        // mode 2: [H, sel_cap] by score desc
  float* sel_score;
  uint8_t* sel_valid;
  int sel_cap;
  // ragged static batches: row b * H + h of sequence b; its budgets follow
  // from B (the largest), amin / amid (0: the defaults) and klens[b] as in
  // sva/llama.py:443-445, its tail is [plens[b], klens[b]), its postings
  // maxima are max_count[b * n_max, (b + 1) * n_max).  NULL: the scalars.
  const int64_t* plens;
  const int64_t* klens;
  int H;
  int amin, amid;
  const int32_t* nlist;  // ragged: live slots are [0, nlist[row]) and [tail_slot0, W)
  int tail_slot0;
};

SVA_DEV uint32_t hash_key(uint32_t n, int hash) { return (n * 2654435761u) & (uint32_t)(hash - 1); }

__global__ void __launch_bounds__(UB, 8) unique_select_kernel(SelParams p) {  // 8 waves per SIMD: two workgroups per CU
  extern __shared__ __align__(16) unsigned char lds[];
  const int HASH = p.hash;
  uint64_t* hcomp = (uint64_t*)lds;                        // [HASH] best composite per key
  uint64_t* sel = hcomp + HASH;                            // [max(B, sel_cap), even] chosen composites
  uint64_t* shared64 = sel + ((max(p.B, p.sel_cap) + 1) & ~1);  // [4]; whist after it 16-byte aligned
  uint32_t(*whist)[256] = (uint32_t(*)[256])(shared64 + 4);  // [UNW][256]
  uint32_t* hkey = (uint32_t*)(whist + UNW);               // [HASH]
  uint32_t* hpos = hkey + HASH;                            // [HASH] first window position of the best
  uint32_t* scratch = hpos + HASH;                         // [UNW + 1]
  uint32_t* shared = scratch + UNW + 1;                    // [8]
  const int h = blockIdx.x;
  const uint64_t* comp = p.comp + (int64_t)h * p.W;
  const uint8_t* flag = p.flag + (int64_t)h * p.W;
  uint64_t* win = p.win + (int64_t)h * p.win_cap;
  const int W = p.W;
  // live slots in slot order: every slot, or (ragged) the row's list entries,
  // then its tail slots and the extra slot
  const int nl = p.nlist != nullptr ? min(max(p.nlist[h], 0), p.tail_slot0) : 0;
  const int WL = p.nlist != nullptr ? nl + (W - p.tail_slot0) : W;
  auto at = [&](int i) { return (p.nlist != nullptr && i >= nl) ? p.tail_slot0 + (i - nl) : i; };
  int Bi = p.B, min_b = p.min_budget, mid_b = p.mid_budget;
  int64_t tail_extra = p.tail_extra;
  const int32_t* mc = p.max_count;
  if (p.klens != nullptr) {
    const int b = h / p.H;
    const int64_t kl = p.klens[b], pl = p.plens[b];
    const int64_t cap = std::min<int64_t>(p.B, kl);
    Bi = (int)cap;
    min_b = (int)std::min<int64_t>(p.amin > 0 ? p.amin : p.B, cap);
    mid_b = (int)std::min<int64_t>(p.amid > 0 ? p.amid : std::max<int64_t>(min_b, p.B / 2), cap);
    tail_extra = kl - pl > 0 ? kl - pl : 1;
    mc = p.max_count + (int64_t)b * p.n_max;
  }
  // counts: real entries, valid entries; bounds of the real entries
  uint32_t real = 0, nvalid = 0;
  uint64_t ror = 0ull, rand_ = ~0ull;
  for (int i = threadIdx.x; i < WL; i += UB) {
    const int j = at(i);
    const uint64_t c = comp[j];
    const uint8_t f = flag[j];
    const bool is_real = c != 0ull && !(f & 2);
    real += is_real;
    nvalid += is_real && (f & 1);
    if (is_real) {
      ror |= c;
      rand_ &= c;
    }
  }
  uint32_t Real, Valid;
  block_excl_scan<UB>(real, scratch, &Real);
  block_excl_scan<UB>(nvalid, scratch, &Valid);
  // refill window
  int64_t width = p.width;
  if (p.mode == 0) {
    // the reference's padded layout: S * cells lists of the largest cell's
    // length, then the tail (or the current row)
    int mb = 0;
    for (int i = 0; i < p.n_max; ++i) mb = max(mb, (int)mc[i]);
    width = p.lists * (int64_t)max(1, mb) + tail_extra;
  }
  int64_t refill;
  if (p.mode == 1) refill = Real;
  else refill = min(width, (int64_t)max(Bi, Bi * p.refill_factor));
  auto visit_real = [&](auto&& f) {
    for (int i = threadIdx.x; i < WL; i += UB) {
      const int j = at(i);
      const uint64_t c = comp[j];
      if (c != 0ull && !(flag[j] & 2)) f(c);
    }
  };
  // adaptive mode: the candidates are distinct keys already, so U is read
  // straight from them; otherwise a refill window and a key table in LDS
  const bool direct = p.mode == 1;
  if (threadIdx.x == 0) shared[4] = 0u;
  if (!direct) {
    uint64_t X1 = 1ull;
    if (refill > 0 && (int64_t)Real > refill)
      X1 = select_largest12<UB>(visit_real, (int)refill, ror, rand_, &whist[0][0], scratch, shared64, shared);
    if (refill <= 0) X1 = ~0ull;
    // window entries in slot order, with their valid flag in bit 0 of the stored word
    for (int i = threadIdx.x; i < HASH; i += UB) {
      hkey[i] = EMPTY;
      hcomp[i] = 0ull;
      hpos[i] = EMPTY;
    }
    __syncthreads();
    {
      const int per = (WL + UB - 1) / UB;
      const int i0 = min(WL, (int)threadIdx.x * per), i1 = min(WL, i0 + per);
      uint32_t cnt = 0;
      for (int i = i0; i < i1; ++i) {
        const int j = at(i);
        const uint64_t c = comp[j];
        cnt += c != 0ull && !(flag[j] & 2) && c >= X1;
      }
      uint32_t tot;
      uint32_t o = block_excl_scan<UB>(cnt, scratch, &tot);
      for (int i = i0; i < i1; ++i) {
        const int j = at(i);
        const uint64_t c = comp[j];
        if (c != 0ull && !(flag[j] & 2) && c >= X1) {
          if (o < (uint32_t)p.win_cap) {
            win[o] = c;
            // key table: best composite per key, then first window position of it
            const uint32_t n = composite_index(c);
            uint32_t slot = hash_key(n, HASH);
            while (true) {
              const uint32_t prev = atomicCAS(&hkey[slot], EMPTY, n);
              if (prev == EMPTY || prev == n) break;
              slot = (slot + 1) & (HASH - 1);
            }
            atomicMax((unsigned long long*)&hcomp[slot], (unsigned long long)c);
          }
          ++o;
        }
      }
      if (threadIdx.x == 0) shared[4] = min(tot, (uint32_t)p.win_cap);
    }
    __syncthreads();
    // first window position of each key's best copy (copies of a key carry
    // the same mask value, so the masked score tells validity)
    const int wn = (int)shared[4];
    for (int i = threadIdx.x; i < wn; i += UB) {
      const uint64_t c = win[i];
      uint32_t slot = hash_key(composite_index(c), HASH);
      while (hkey[slot] != composite_index(c)) slot = (slot + 1) & (HASH - 1);
      if (hcomp[slot] == c) atomicMin(&hpos[slot], (uint32_t)i);
    }
  }
  __syncthreads();
  const int nwin = (int)shared[4];
  const int ndom = direct ? W : nwin;
  auto dom = [&](int i) -> uint64_t { return direct ? comp[i] : win[i]; };
  auto slot_of = [&](uint32_t n) {
    uint32_t slot = hash_key(n, HASH);
    while (hkey[slot] != n) slot = (slot + 1) & (HASH - 1);
    return slot;
  };
  // U: allowed distinct keys (the first window position of a key's best copy)
  auto in_u = [&](int i, uint64_t c) -> bool {
    if (direct) return c != 0ull && (flag[i] & 3) == 1;
    const uint32_t slot = slot_of(composite_index(c));
    return hcomp[slot] == c && hpos[slot] == (uint32_t)i && composite_key(c) != f2key(-FLT_MAX);
  };
  // a domain of at most UR * UB entries (the usual one) puts U's elements in
  // registers, slot j of thread t holding entry t + j UB, and selects over
  // them with 12-bit passes that rank the last bucket directly
  // (select_top_regs), instead of 8-bit passes that probe the key table for
  // every element; the selections are the same (unique composites)
  constexpr int UR = 2;
  const bool regs = ndom <= UR * UB;  // block-uniform
  const int uslots = (ndom + UB - 1) / UB;
  uint64_t ue[UR];
  uint64_t uor = 0ull, uand = ~0ull;
  uint32_t ucount = 0;
  if (regs) {
#pragma unroll
    for (int j = 0; j < UR; ++j) {
      const int i = (int)threadIdx.x + j * UB;
      ue[j] = 0ull;
      if (i < ndom) {
        const uint64_t c = dom(i);
        if (in_u(i, c)) {
          ue[j] = c;
          uor |= c;
          uand &= c;
          ++ucount;
        }
      }
    }
  } else {
    for (int i = threadIdx.x; i < ndom; i += UB) ucount += in_u(i, dom(i));
  }
  uint32_t U;
  block_excl_scan<UB>(ucount, scratch, &U);
  // the register selects' LDS: the wave histograms as one 4096-bin histogram,
  // the key table's composites (no longer probed) as the last bucket
  const TopLds tl{&whist[0][0], hcomp, scratch, shared, shared64};
  // rank count (selected slots) and the budget
  const int64_t rank_count = p.mode == 1 ? min((int64_t)Bi, (int64_t)U) : min((int64_t)Bi, refill);
  auto visit_u = [&](auto&& f) {
    for (int i = threadIdx.x; i < ndom; i += UB) {
      const uint64_t c = dom(i);
      if (in_u(i, c)) f(c);
    }
  };
  int budget = (int)rank_count;
  if (p.mode != 2 && rank_count > 1) {
    // best and (min_budget)-th best scores of the selected slots; slots past
    // U hold the masked minimum
    const int mref = (int)min((int64_t)min_b, rank_count) - 1;
    uint64_t best = 0ull;
    if (regs) {
#pragma unroll
      for (int j = 0; j < UR; ++j) best = ue[j] > best ? ue[j] : best;
    } else {
      visit_u([&](uint64_t c) { best = c > best ? c : best; });
    }
    for (int off = 1; off < WAVE; off <<= 1) {
      const uint64_t o = __shfl_xor(best, off, WAVE);
      best = o > best ? o : best;
    }
    if (threadIdx.x == 0) {
      shared64[2] = 0ull;
      shared64[3] = ~0ull;
    }
    __syncthreads();
    if (lane_id() == 0) atomicMax((unsigned long long*)&shared64[2], (unsigned long long)best);
    __syncthreads();
    const float s0 = U > 0 ? key2f(composite_key(shared64[2])) : -FLT_MAX;
    float sref = -FLT_MAX;
    if ((int64_t)U > mref) {
      const uint64_t Xr = regs ? select_top_regs<UB, UR>(ue, mref + 1, uor, uand, tl, uslots)
                               : select_largest<UB>(visit_u, mref + 1, whist, scratch, shared64, shared);
      // the (mref+1)-th largest element is the smallest one >= Xr
      uint64_t mn = ~0ull;
      if (regs) {
#pragma unroll
        for (int j = 0; j < UR; ++j) mn = (ue[j] != 0ull && ue[j] >= Xr && ue[j] < mn) ? ue[j] : mn;
      } else {
        visit_u([&](uint64_t c) { mn = (c >= Xr && c < mn) ? c : mn; });
      }
      for (int off = 1; off < WAVE; off <<= 1) {
        const uint64_t o = __shfl_xor(mn, off, WAVE);
        mn = o < mn ? o : mn;
      }
      if (lane_id() == 0) atomicMin((unsigned long long*)&shared64[3], (unsigned long long)mn);
      __syncthreads();
      sref = key2f(composite_key(shared64[3]));
    }
    const float margin = s0 - sref;
    if (p.mode == 1) {
      const double md = (double)margin;
      budget = md >= p.high_d ? (int)min((int64_t)min_b, rank_count)
                              : (md >= p.low_d ? (int)min((int64_t)mid_b, rank_count) : (int)rank_count);
    } else {
      budget = margin >= p.high_f ? min_b : (margin >= p.low_f ? mid_b : Bi);
      budget = (int)min((int64_t)budget, rank_count);
    }
  } else if (p.mode == 0) {
    budget = 1;
  }
  const int k3 = (int)min((int64_t)budget, (int64_t)U);
  uint64_t X3 = 1ull;
  if (k3 > 0 && (int)U > k3)
    X3 = regs ? select_top_regs<UB, UR>(ue, k3, uor, uand, tl, uslots)
              : select_largest<UB>(visit_u, k3, whist, scratch, shared64, shared);
  // chosen keys (composites): any order, the outputs below order them
  if (k3 > 0 && regs) {
    if (threadIdx.x == 0) shared[5] = 0u;
    __syncthreads();
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < UR; ++j) {
      const bool take = ue[j] != 0ull && ue[j] >= X3;
      const uint64_t m = __builtin_amdgcn_ballot_w64(take);
      if (m != 0ull) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&shared[5], (uint32_t)__popcll(m));
        base = __shfl(base, 0, WAVE);
        const uint32_t o = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (take && o < (uint32_t)k3) sel[o] = ue[j];
      }
    }
  } else if (k3 > 0) {  // in window order
    const int per = (ndom + UB - 1) / UB;
    const int i0 = min(ndom, (int)threadIdx.x * per), i1 = min(ndom, i0 + per);
    uint32_t cnt = 0;
    for (int i = i0; i < i1; ++i) cnt += in_u(i, dom(i)) && dom(i) >= X3;
    uint32_t tot;
    uint32_t o = block_excl_scan<UB>(cnt, scratch, &tot);
    for (int i = i0; i < i1; ++i) {
      const uint64_t c = dom(i);
      if (in_u(i, c) && c >= X3 && o < (uint32_t)k3) sel[o++] = c;
    }
  }
  __syncthreads();
  if (p.mode == 2) {
    // the selected slots by score desc (key asc on ties), then invalid slots
    const int slots = (int)min((int64_t)p.sel_cap, rank_count);
    int32_t* oi = p.sel_idx + (int64_t)h * p.sel_cap;
    float* os = p.sel_score + (int64_t)h * p.sel_cap;
    uint8_t* ov = p.sel_valid + (int64_t)h * p.sel_cap;
    for (int i = threadIdx.x; i < k3; i += UB) {
      const uint64_t v = sel[i];
      int r = 0;
      for (int j = 0; j < k3; ++j) r += sel[j] > v;
      oi[r] = (int32_t)composite_index(v);
      os[r] = key2f(composite_key(v));
      ov[r] = 1;
    }
    for (int r = k3 + (int)threadIdx.x; r < slots; r += UB) {
      oi[r] = 0;
      os[r] = -FLT_MAX;
      ov[r] = 0;
    }
    if (threadIdx.x == 0) {
      p.fin_count[h] = slots;
      p.stats[(int64_t)h * 4 + 1] = (float)refill;
    }
    return;
  }
  int32_t* out = p.fin_idx + (int64_t)h * p.B;
  int kfin = k3;
  if (p.mode == 1 && U == 0) {
    // no allowed candidate: the last allowed row, when there is one
    if (threadIdx.x == 0) shared[6] = EMPTY;
    __syncthreads();
    for (int i = threadIdx.x; i < W; i += UB)
      if ((flag[i] & 2) && comp[i] != 0ull) shared[6] = composite_index(comp[i]);
    __syncthreads();
    kfin = shared[6] == EMPTY ? 0 : 1;
    if (threadIdx.x == 0 && kfin) out[0] = (int32_t)shared[6];
  } else {
    for (int i = threadIdx.x; i < k3; i += UB) {
      const uint32_t v = composite_index(sel[i]);
      int r = 0;
      for (int j = 0; j < k3; ++j) r += composite_index(sel[j]) < v;
      out[r] = (int32_t)v;
    }
  }
  if (threadIdx.x == 0) {
    p.fin_count[h] = kfin;
    float* st = p.stats + (int64_t)h * 4;
    st[0] = p.mode == 1 ? (float)max((uint32_t)kfin, U) : (float)Valid;
    st[1] = p.mode == 1 ? 0.0f : (float)refill;
    st[2] = (float)kfin;
    st[3] = (float)rank_count;
  }
}

// Generic entries (key, score, valid) -> composites for the plain top-unique
// selection; the masked score of an invalid entry is -FLT_MAX (finfo.min).
__global__ void pack_entries_kernel(const int64_t* __restrict__ idx, const float* __restrict__ score,
                                    const uint8_t* __restrict__ valid, int64_t total, uint64_t* __restrict__ comp,
                                    uint8_t* __restrict__ flag) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const bool ok = valid[i] != 0;
  comp[i] = composite(f2key(ok ? score[i] : -FLT_MAX), (uint32_t)idx[i]);
  flag[i] = ok ? 1 : 0;
}

size_t select_lds_bytes(int64_t B, int64_t hash) {
  return sizeof(uint64_t) * (size_t)(hash + ((B + 1) & ~1ll) + 4) +
         sizeof(uint32_t) * (size_t)(UNW * 256 + 2 * hash + UNW + 1 + 8);
}

int hash_slots(int win_cap) {
  int h = 256;
  while (h < 2 * win_cap) h <<= 1;
  return h;
}

int win_cap_for(int64_t B, int refill_factor, int64_t W) {
  // the window holds the best `refill` entries plus the copies of the
  // boundary key (at most one per list and the tail)
  return (int)std::min<int64_t>(W, std::max<int64_t>(B, B * refill_factor) + 64);
}

int launch_select(const SelParams& p, int64_t H, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE(unique_select_kernel, sva::kMaxLds, "hipFuncSetAttribute(unique_select_kernel)");
  hipLaunchKernelGGL(unique_select_kernel, dim3((unsigned)H), dim3(UB),
                     select_lds_bytes(std::max(p.B, p.sel_cap), p.hash), stream, p);
  SVA_CHECK_LAUNCH("unique_select_kernel");
  return SVA_OK;
}

}  // namespace

extern "C" int sva_postings_build(const void* codes, int code_type, int64_t code_head_stride, int64_t H,
                                  int64_t n_rows, int64_t S, int64_t C, int32_t* offsets, int32_t* ids,
                                  int32_t* max_count, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(codes && offsets && ids && max_count, "sva_postings_build: null pointer");
  SVA_REQUIRE(H > 0 && S > 0 && n_rows >= 0 && n_rows < (1ll << 31) && H * S < (1ll << 31),
              "sva_postings_build: bad sizes");
  SVA_REQUIRE(code_type >= 0 && code_type <= 3, "sva_postings_build: bad code type");
  SVA_UNSUPPORTED(C > 0 && C <= kMaxPostingCells, "sva_postings_build: %lld codewords (at most %d)", (long long)C,
                  kMaxPostingCells);
  SVA_SET_MAX_LDS_ONCE(postings_build_kernel, sva::kMaxLds, "hipFuncSetAttribute(postings_build)");
  const size_t lds = sizeof(uint32_t) * (size_t)(2 * C + PNW * C + PNW + 2);
  hipLaunchKernelGGL(postings_build_kernel, dim3((unsigned)(H * S)), dim3(PB), lds, (hipStream_t)stream, codes,
                     code_type, code_head_stride, (int)H, (int)S, (int)n_rows, (int)C, nullptr, nullptr, n_rows,
                     offsets, ids, max_count);
  SVA_CHECK_LAUNCH("postings_build_kernel");
  return SVA_OK;
}

extern "C" int sva_postings_build_ragged(const void* codes, int code_type, int64_t code_head_stride,
                                         const int64_t* seq_offsets, const int64_t* postings_lens, int64_t n_seq,
                                         int64_t H, int64_t rows, int64_t S, int64_t C, int32_t* offsets, int32_t* ids,
                                         int32_t* max_count, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(codes && seq_offsets && postings_lens && offsets && ids && max_count,
              "sva_postings_build_ragged: null pointer");
  SVA_REQUIRE(n_seq > 0 && H > 0 && S > 0 && rows > 0 && rows < (1ll << 31) && n_seq * H * S < (1ll << 31),
              "sva_postings_build_ragged: bad sizes");
  SVA_REQUIRE(code_type >= 0 && code_type <= 3, "sva_postings_build_ragged: bad code type");
  SVA_UNSUPPORTED(C > 0 && C <= kMaxPostingCells, "sva_postings_build_ragged: %lld codewords (at most %d)",
                  (long long)C, kMaxPostingCells);
  SVA_SET_MAX_LDS_ONCE(postings_build_kernel, sva::kMaxLds, "hipFuncSetAttribute(postings_build)");
  const size_t lds = sizeof(uint32_t) * (size_t)(2 * C + PNW * C + PNW + 2);
  hipLaunchKernelGGL(postings_build_kernel, dim3((unsigned)(n_seq * H * S)), dim3(PB), lds, (hipStream_t)stream, codes,
                     code_type, code_head_stride, (int)H, (int)S, 0, (int)C, seq_offsets, postings_lens, rows,
                     offsets, ids, max_count);
  SVA_CHECK_LAUNCH("postings_build_kernel");
  return SVA_OK;
}

extern "C" int64_t sva_inverted_slots(int64_t S, int64_t postings_len, int64_t k_len, int64_t tail_start) {
  return S * postings_len + std::max<int64_t>(0, k_len - tail_start) + 1;
}

extern "C" int sva_inverted_candidates(const float* lut, const float* q_low, const float* k_low,
                                       int64_t k_low_head_stride, const void* codes, int code_type,
                                       int64_t code_head_stride, const int32_t* offsets, const int32_t* ids,
                                       int64_t postings_len, int64_t tail_start, int64_t k_len, int64_t H, int64_t S,
                                       int64_t C, int64_t R, int64_t cells, const void* mask, int mask_type,
                                       int adaptive, uint64_t* comp, uint8_t* flag, int64_t slots, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(lut && q_low && k_low && codes && offsets && ids && comp && flag, "sva_inverted_candidates: null pointer");
  SVA_REQUIRE(H > 0 && H <= 65535 && k_len > 0 && k_len < (1ll << 31) && postings_len >= 0 &&
                  postings_len <= k_len && tail_start >= 0 && tail_start <= k_len,
              "sva_inverted_candidates: bad sizes");
  SVA_UNSUPPORTED(R > 0 && R <= 511, "sva_inverted_candidates: rank %lld unsupported", (long long)R);
  SVA_UNSUPPORTED(S > 0 && S <= kMaxSub && C > 0 && C <= 256 && cells > 0 && cells <= std::min<int64_t>(C, kMaxCells),
                  "sva_inverted_candidates: layout %lldx%lld with %lld cells unsupported", (long long)S, (long long)C,
                  (long long)cells);
  SVA_REQUIRE(R != 64 || ((((uintptr_t)k_low | (uintptr_t)q_low) & 15u) == 0 && k_low_head_stride % 4 == 0),
              "sva_inverted_candidates: k_low / q_low must be 16-byte aligned");
  SVA_REQUIRE(slots == sva_inverted_slots(S, postings_len, k_len, tail_start),
              "sva_inverted_candidates: slots must be sva_inverted_slots(...)");
  SVA_REQUIRE(mask_type >= 0 && mask_type <= 4 && (mask_type == 0 || mask_type == 4 || mask != nullptr),
              "sva_inverted_candidates: bad mask");
  CandParams p;
  p.lut = lut;
  p.q_low = q_low;
  p.k_low = k_low;
  p.klow_hs = k_low_head_stride;
  p.codes = codes;
  p.ctype = code_type;
  p.code_hs = code_head_stride;
  p.offsets = offsets;
  p.ids = ids;
  p.postings_len = (int)postings_len;
  p.tail_start = (int)tail_start;
  p.k_len = (int)k_len;
  p.H = (int)H;
  p.S = (int)S;
  p.C = (int)C;
  p.R = (int)R;
  p.cells = (int)cells;
  p.sqrt_r = (float)std::sqrt((double)R);
  p.mask = (mask_type == 1 || mask_type == 2 || mask_type == 3) ? mask : nullptr;
  p.mask_type = mask_type;
  p.adaptive = adaptive ? 1 : 0;
  p.W = (int)slots;
  p.comp = comp;
  p.flag = flag;
  const int64_t tail_len = k_len - tail_start;
  p.seq_offs = nullptr;
  p.plens = nullptr;
  p.klens = nullptr;
  p.tail_cap = (int)tail_len;
  p.ids_rows = postings_len;
  p.nlist = nullptr;
  const int64_t wgs = S * cells + (tail_len + TAIL_ROWS - 1) / TAIL_ROWS + 1;
  SVA_REQUIRE(wgs < (1ll << 31) && slots < (1ll << 31), "sva_inverted_candidates: too many rows");
  hipLaunchKernelGGL(inverted_candidates_kernel, dim3((unsigned)wgs, (unsigned)H), dim3(CT),
                     cells > 16 ? sizeof(float) * (size_t)(S * C) : 0, (hipStream_t)stream, p);
  SVA_CHECK_LAUNCH("inverted_candidates_kernel");
  return SVA_OK;
}

extern "C" int64_t sva_inverted_slots_ragged(int64_t S, int64_t max_postings_len, int64_t max_tail) {
  return S * max_postings_len + std::max<int64_t>(0, max_tail) + 1;
}

extern "C" int sva_inverted_candidates_ragged(const float* lut, const float* q_low, const float* k_low,
                                              int64_t k_low_head_stride, const void* codes, int code_type,
                                              int64_t code_head_stride, const int32_t* offsets, const int32_t* ids,
                                              int64_t rows, const int64_t* seq_offsets, const int64_t* postings_lens,
                                              const int64_t* k_lens, int64_t n_seq, int64_t max_postings_len,
                                              int64_t max_tail, int64_t H, int64_t S, int64_t C, int64_t R,
                                              int64_t cells, uint64_t* comp, uint8_t* flag, int32_t* list_counts,
                                              int64_t slots, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(lut && q_low && k_low && codes && offsets && ids && seq_offsets && postings_lens && k_lens && comp &&
                  flag && list_counts,
              "sva_inverted_candidates_ragged: null pointer");
  SVA_REQUIRE(n_seq > 0 && H > 0 && n_seq * H <= 65535 && rows > 0 && rows < (1ll << 31) && max_postings_len >= 0 &&
                  max_postings_len <= rows && max_tail >= 0 && max_tail <= rows,
              "sva_inverted_candidates_ragged: bad sizes");
  SVA_UNSUPPORTED(R > 0 && R <= 511, "sva_inverted_candidates_ragged: rank %lld unsupported", (long long)R);
  SVA_UNSUPPORTED(S > 0 && S <= kMaxSub && C > 0 && C <= 256 && cells > 0 && cells <= std::min<int64_t>(C, kMaxCells),
                  "sva_inverted_candidates_ragged: layout %lldx%lld with %lld cells unsupported", (long long)S,
                  (long long)C, (long long)cells);
  SVA_REQUIRE(R != 64 || ((((uintptr_t)k_low | (uintptr_t)q_low) & 15u) == 0 && k_low_head_stride % 4 == 0),
              "sva_inverted_candidates_ragged: k_low / q_low must be 16-byte aligned");
  SVA_REQUIRE(slots == sva_inverted_slots_ragged(S, max_postings_len, max_tail),
              "sva_inverted_candidates_ragged: slots must be sva_inverted_slots_ragged(...)");
  CandParams p;
  p.lut = lut;
  p.q_low = q_low;
  p.k_low = k_low;
  p.klow_hs = k_low_head_stride;
  p.codes = codes;
  p.ctype = code_type;
  p.code_hs = code_head_stride;
  p.offsets = offsets;
  p.ids = ids;
  p.postings_len = (int)max_postings_len;
  p.tail_start = 0;
  p.k_len = 0;
  p.H = (int)H;
  p.S = (int)S;
  p.C = (int)C;
  p.R = (int)R;
  p.cells = (int)cells;
  p.sqrt_r = (float)std::sqrt((double)R);
  p.mask = nullptr;
  p.mask_type = 0;
  p.adaptive = 0;
  p.W = (int)slots;
  p.comp = comp;
  p.flag = flag;
  p.seq_offs = seq_offsets;
  p.plens = postings_lens;
  p.klens = k_lens;
  p.tail_cap = (int)max_tail;
  p.ids_rows = rows;
  p.nlist = list_counts;
  const int64_t items = n_seq * H;
  SVA_UNSUPPORTED(items <= MAX_RAGGED_ITEMS, "sva_inverted_candidates_ragged: %lld items (at most %d)",
                  (long long)items, MAX_RAGGED_ITEMS);
  SVA_UNSUPPORTED(R == 64, "sva_inverted_candidates_ragged: rank %lld (64 only)", (long long)R);
  SVA_REQUIRE(slots < (1ll << 31) && items * slots < (1ll << 40), "sva_inverted_candidates_ragged: too many rows");
  hipLaunchKernelGGL(ragged_cand_prep_kernel, dim3((unsigned)items), dim3(CT),
                     cells > 16 ? sizeof(float) * (size_t)(S * C) : 0, (hipStream_t)stream, p);
  SVA_CHECK_LAUNCH("ragged_cand_prep_kernel");
  const int score_wgs = 4 * sva::device_cu_count();
  hipLaunchKernelGGL(ragged_cand_score_kernel, dim3((unsigned)score_wgs), dim3(CT), sizeof(int) * (size_t)(items + 1),
                     (hipStream_t)stream, p, (int)items);
  SVA_CHECK_LAUNCH("ragged_cand_score_kernel");
  return SVA_OK;
}

extern "C" size_t sva_unique_select_workspace_bytes(int64_t H, int64_t B, int64_t refill_factor, int64_t slots) {
  if (H <= 0 || B <= 0 || slots <= 0) return 256;
  return sizeof(uint64_t) * (size_t)H * (size_t)win_cap_for(B, (int)std::max<int64_t>(1, refill_factor), slots) + 256;
}

extern "C" int sva_unique_refill_select(const uint64_t* comp, const uint8_t* flag, int64_t slots, int64_t H, int mode,
                                        int64_t B, int64_t min_budget, int64_t mid_budget, double low_margin,
                                        double high_margin, int64_t refill_factor, const int32_t* max_count,
                                        int64_t S, int64_t cells, int64_t tail_len, int32_t* fin_idx,
                                        int32_t* fin_count, float* stats, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  sva::clear_error();
  SVA_REQUIRE(comp && flag && fin_idx && fin_count && stats && workspace, "sva_unique_refill_select: null pointer");
  SVA_REQUIRE(mode == 0 || mode == 1, "sva_unique_refill_select: mode 0 (static) or 1 (adaptive)");
  SVA_REQUIRE(mode == 1 || max_count != nullptr, "sva_unique_refill_select: static mode needs the postings maxima");
  SVA_REQUIRE(H > 0 && H < (1ll << 31) && slots > 0 && slots < (1ll << 31) && B > 0 && min_budget > 0 &&
                  mid_budget > 0 && min_budget <= B && mid_budget <= B && refill_factor >= 1,
              "sva_unique_refill_select: bad sizes");
  const int win_cap = win_cap_for(B, (int)refill_factor, slots);
  const int hash = hash_slots(win_cap);
  const size_t lds = select_lds_bytes(B, hash);
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_unique_refill_select: budget %lld needs %zu bytes of LDS",
                  (long long)B, lds);
  SVA_REQUIRE(workspace_bytes >= sva_unique_select_workspace_bytes(H, B, refill_factor, slots),
              "sva_unique_refill_select: workspace too small");
  SelParams p{};
  p.comp = comp;
  p.flag = flag;
  p.W = (int)slots;
  p.mode = mode;
  p.B = (int)B;
  p.min_budget = (int)min_budget;
  p.mid_budget = (int)mid_budget;
  p.low_f = (float)low_margin;
  p.high_f = (float)high_margin;
  p.low_d = low_margin;
  p.high_d = high_margin;
  p.width = slots;
  p.max_count = max_count;
  p.n_max = (int)(H * S);
  p.lists = S * cells;
  p.tail_extra = tail_len > 0 ? tail_len : 1;
  p.refill_factor = (int)refill_factor;
  p.win_cap = win_cap;
  p.hash = hash;
  p.win = (uint64_t*)workspace;
  p.fin_idx = fin_idx;
  p.fin_count = fin_count;
  p.stats = stats;
  p.sel_cap = 0;
  return launch_select(p, H, (hipStream_t)stream);
}

extern "C" int sva_unique_refill_select_ragged(const uint64_t* comp, const uint8_t* flag, int64_t slots, int64_t n_seq,
                                               int64_t H, int64_t budget, int64_t adaptive_min_budget,
                                               int64_t adaptive_mid_budget, double low_margin, double high_margin,
                                               int64_t refill_factor, const int32_t* max_count, int64_t S,
                                               int64_t cells, const int64_t* postings_lens, const int64_t* k_lens,
                                               const int32_t* list_counts, int64_t max_postings_len, int32_t* fin_idx,
                                               int32_t* fin_count, float* stats, void* workspace,
                                               size_t workspace_bytes, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(comp && flag && max_count && postings_lens && k_lens && list_counts && fin_idx && fin_count && stats &&
                  workspace,
              "sva_unique_refill_select_ragged: null pointer");
  SVA_REQUIRE(max_postings_len >= 0 && S * max_postings_len < slots,
              "sva_unique_refill_select_ragged: slots must be sva_inverted_slots_ragged(...)");
  SVA_REQUIRE(n_seq > 0 && H > 0 && n_seq * H < (1ll << 31) && slots > 0 && slots < (1ll << 31) && budget > 0 &&
                  adaptive_min_budget >= 0 && adaptive_mid_budget >= 0 && refill_factor >= 1 && S > 0 && cells > 0,
              "sva_unique_refill_select_ragged: bad sizes");
  const int win_cap = win_cap_for(budget, (int)refill_factor, slots);
  const int hash = hash_slots(win_cap);
  const size_t lds = select_lds_bytes(budget, hash);
  SVA_UNSUPPORTED(lds <= (size_t)sva::kMaxLds, "sva_unique_refill_select_ragged: budget %lld needs %zu bytes of LDS",
                  (long long)budget, lds);
  SVA_REQUIRE(workspace_bytes >= sva_unique_select_workspace_bytes(n_seq * H, budget, refill_factor, slots),
              "sva_unique_refill_select_ragged: workspace too small");
  SelParams p{};
  p.comp = comp;
  p.flag = flag;
  p.W = (int)slots;
  p.mode = 0;
  p.B = (int)budget;
  p.min_budget = (int)budget;
  p.mid_budget = (int)budget;
  p.low_f = (float)low_margin;
  p.high_f = (float)high_margin;
  p.low_d = low_margin;
  p.high_d = high_margin;
  p.width = slots;
  p.max_count = max_count;
  p.n_max = (int)(H * S);
  p.lists = S * cells;
  p.tail_extra = 1;
  p.refill_factor = (int)refill_factor;
  p.win_cap = win_cap;
  p.hash = hash;
  p.win = (uint64_t*)workspace;
  p.fin_idx = fin_idx;
  p.fin_count = fin_count;
  p.stats = stats;
  p.sel_cap = 0;
  p.plens = postings_lens;
  p.klens = k_lens;
  p.H = (int)H;
  p.amin = (int)std::min<int64_t>(adaptive_min_budget, budget);
  p.amid = (int)std::min<int64_t>(adaptive_mid_budget, budget);
  p.nlist = list_counts;
  p.tail_slot0 = (int)(S * max_postings_len);
  return launch_select(p, n_seq * H, (hipStream_t)stream);
}

extern "C" size_t sva_top_unique_workspace_bytes(int64_t H, int64_t W, int64_t budget, int64_t refill_factor) {
  if (H <= 0 || W <= 0 || budget <= 0) return 256;
  const size_t n = (size_t)H * (size_t)W;
  return 2 * ((sizeof(uint64_t) * n + 255) & ~(size_t)255) + ((n + 255) & ~(size_t)255) +
         sizeof(float) * 4 * (size_t)H + sizeof(int32_t) * (size_t)H + 512;
}

extern "C" int sva_top_unique(const int64_t* idx, const float* scores, const uint8_t* valid, int64_t H, int64_t W,
                              int64_t budget, int64_t refill_factor, int32_t* sel_idx, float* sel_scores,
                              uint8_t* sel_valid, void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(idx && scores && valid && sel_idx && sel_scores && sel_valid && workspace, "sva_top_unique: null pointer");
  SVA_REQUIRE(H > 0 && H < (1ll << 31) && W > 0 && W < (1ll << 31) && budget > 0 && refill_factor >= 1,
              "sva_top_unique: bad sizes");
  SVA_REQUIRE(workspace_bytes >= sva_top_unique_workspace_bytes(H, W, budget, refill_factor),
              "sva_top_unique: workspace too small");
  const int64_t refill = std::min<int64_t>(W, std::max<int64_t>(budget, budget * refill_factor));
  const int64_t cap = std::min<int64_t>(budget, refill);
  // arbitrary entries may repeat one key any number of times: the window
  // holds every entry at or above the refill threshold
  const int win_cap = (int)W;
  const int hash = hash_slots(win_cap);
  SVA_UNSUPPORTED(select_lds_bytes(std::max<int64_t>(budget, cap), hash) <= (size_t)sva::kMaxLds,
                  "sva_top_unique: %lld entries per row too many", (long long)W);
  char* ws = (char*)workspace;
  const size_t n = (size_t)H * (size_t)W;
  uint64_t* comp = (uint64_t*)ws;
  ws += (sizeof(uint64_t) * n + 255) & ~(size_t)255;
  uint8_t* flag = (uint8_t*)ws;
  ws += (n + 255) & ~(size_t)255;
  uint64_t* win = (uint64_t*)ws;
  ws += (sizeof(uint64_t) * n + 255) & ~(size_t)255;
  float* stats = (float*)ws;
  int32_t* counts = (int32_t*)(stats + 4 * H);
  const int64_t blocks = ((int64_t)n + 255) / 256;
  hipLaunchKernelGGL(pack_entries_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, idx, scores, valid,
                     (int64_t)n, comp, flag);
  SVA_CHECK_LAUNCH("pack_entries_kernel");
  SelParams p{};
  p.comp = comp;
  p.flag = flag;
  p.W = (int)W;
  p.mode = 2;
  p.B = (int)budget;
  p.min_budget = (int)budget;
  p.mid_budget = (int)budget;
  p.width = W;
  p.refill_factor = (int)refill_factor;
  p.win_cap = win_cap;
  p.hash = hash;
  p.win = win;
  p.fin_idx = sel_idx;
  p.fin_count = counts;
  p.stats = stats;
  p.sel_idx = sel_idx;
  p.sel_score = sel_scores;
  p.sel_valid = sel_valid;
  p.sel_cap = (int)cap;
  return launch_select(p, H, (hipStream_t)stream);
}
