// Summon: PQ scan over the cached codes, exact shortlist selection and the
// low-rank rescore of the shortlist (sva/llama.py:270-292, sva/ops.py:50-71).
//
// Item path (this file, summon_item_kernel): one workgroup per query item
// (sequence, head, token).  The LUT sits in LDS; every allowed key's score is
// turned into an order-preserving key; an LDS radix select finds the L-th
// largest key T and how many keys equal to T to take (lowest key indices
// first); a compaction in key-index order writes the shortlist; each
// shortlisted key is rescored against q_low in torch's summation order.
// Keys live in LDS when they fit, otherwise they are recomputed per pass.
//
// Fused item path (summon_regs_kernel): caches of up to 16K keys with a
// budget run shortlist, rescore and budget in one workgroup per item from
// registers (the prefill shape).
//
// The long-context q=1 path (many workgroups per item) is in summon_wide.hip.
#include <type_traits>

#include "capi_internal.h"
#include "common.cuh"
#include "query.h"
#include "summon.h"
#include "summon_regs.cuh"
#include "write_few.cuh"

using namespace sva;

namespace {

struct ItemLds {
  // offsets (bytes) of the dynamic LDS regions
  int tab, ql, hist, scratch, shared, slidx, keys, total;
};

// idx16: shortlist slots as uint16 (every key index below 65536), which
// leaves room for the keys of caches of about 35K keys at L = 8192.
__host__ __device__ inline ItemLds item_lds_layout(int S, int C, int R, int L, int64_t N, bool keys_in_lds,
                                                   bool idx16) {
  ItemLds l;
  int o = 0;
  l.tab = o;
  o = align16(o + 4 * S * C);
  l.ql = o;
  o = align16(o + 4 * R);
  l.hist = o;
  o = align16(o + 4 * 256);
  l.scratch = o;
  o = align16(o + 4 * (ITEM_BLOCK / WAVE + 1));
  l.shared = o;
  o = align16(o + 4 * 4);
  l.slidx = o;
  o = align16(o + (idx16 ? 2 : 4) * L);
  l.keys = o;
  if (keys_in_lds) o = align16(o + (int)(4 * N));
  l.total = o;
  return l;
}

// flags: bit 0 the keys sit in LDS, bit 1 the shortlist slots are uint16
// (item_lds_layout's idx16; the host sets both from the largest length).
__global__ void __launch_bounds__(ITEM_BLOCK) summon_item_kernel(SummonParams p, int flags) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) unsigned char lds[];
  const int item = blockIdx.x;
  const int t = item % p.Q;
  const int h = (item / p.Q) % p.H;
  const int b = item / (p.Q * p.H);
  const int64_t len = p.lens ? p.lens[b] : p.N;
  const int64_t off = p.offs ? p.offs[b] : 0;
  const bool keys_in_lds = (flags & 1) != 0, idx16 = (flags & 2) != 0;
  const ItemLds L = item_lds_layout(p.S, p.C, p.R, p.L, len, keys_in_lds, idx16);
  float* tab = (float*)(lds + L.tab);
  float* ql = (float*)(lds + L.ql);
  uint32_t* hist = (uint32_t*)(lds + L.hist);
  uint32_t* scratch = (uint32_t*)(lds + L.scratch);
  uint32_t* shared = (uint32_t*)(lds + L.shared);
  int32_t* slidx32 = (int32_t*)(lds + L.slidx);
  uint16_t* slidx16 = (uint16_t*)(lds + L.slidx);
  auto set_slot = [&](uint32_t j, int64_t n) {
    if (idx16) slidx16[j] = (uint16_t)n;
    else slidx32[j] = (int32_t)n;
  };
  auto slot = [&](int j) -> int64_t { return idx16 ? (int64_t)slidx16[j] : (int64_t)slidx32[j]; };
  uint32_t* keys = (uint32_t*)(lds + L.keys);

  const int SC = p.S * p.C;
  const float* lsrc = p.lut + (int64_t)item * SC;
  for (int e = threadIdx.x; e < SC; e += ITEM_BLOCK) tab[e] = lsrc[e];
  const float* qsrc = p.q_low + (int64_t)item * p.R;
  for (int r = threadIdx.x; r < p.R; r += ITEM_BLOCK) ql[r] = qsrc[r];
  __syncthreads();

  const int64_t code_base = (int64_t)h * p.code_hs + off * p.S;
  const int64_t causal_last = len - p.Q + t;  // last allowed key without a mask
  const char* mrow = p.mask ? (const char*)p.mask : nullptr;
  const int S = p.S, C = p.C;
  const float sqrt_r = p.sqrt_r;
  const bool r64 = p.R == 64;  // x / 8 is x * 0.125 exactly

  auto compute_key = [&](int64_t n) -> uint32_t {
    const bool allowed =
        p.mask_type == MASK_NONE ? n <= causal_last : mask_allows(mrow, (int64_t)t * p.mask_ts + n, p.mask_type);
    if (!allowed) return 0u;
    float acc = 0.0f;
    const int64_t row = code_base + n * S;
    for (int s = 0; s < S; ++s) {
      int64_t c = load_code(p.codes, row + s, p.ctype);
      c = c < 0 ? 0 : (c >= C ? C - 1 : c);
      acc = acc + tab[s * C + c];
    }
    return f2key(r64 ? acc * 0.125f : acc / sqrt_r);
  };

  uint32_t cnt = 0;
  const bool u8w = p.ctype == CODE_U8 && (S == 1 || S == 2 || S == 4) && code_base % S == 0 &&
                   ((uintptr_t)p.codes % (uintptr_t)S) == 0;
  if (keys_in_lds && u8w) {
    // uint8 codes of 1, 2 or 4 subspaces: one load per key, U keys' loads
    // issued (clamped to the last key) before any is used; the same sums as
    // compute_key
    constexpr int U = 8;
    const uint8_t* c8 = (const uint8_t*)p.codes + code_base;
    for (int64_t n0 = threadIdx.x; n0 < len; n0 += (int64_t)U * ITEM_BLOCK) {
      uint32_t w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t n = min(n0 + (int64_t)u * ITEM_BLOCK, len - 1);
        w[u] = S == 4   ? *reinterpret_cast<const uint32_t*>(c8 + n * 4)
               : S == 2 ? (uint32_t)*reinterpret_cast<const uint16_t*>(c8 + n * 2)
                        : (uint32_t)c8[n];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t n = n0 + (int64_t)u * ITEM_BLOCK;
        if (n < len) {
          const bool allowed = p.mask_type == MASK_NONE ? n <= causal_last
                                                        : mask_allows(mrow, (int64_t)t * p.mask_ts + n, p.mask_type);
          uint32_t k = 0u;
          if (allowed) {
            float acc = 0.0f;
            for (int s = 0; s < S; ++s) {
              const int c = (int)((w[u] >> (8 * s)) & 0xFFu);
              acc = acc + tab[s * C + (c >= C ? C - 1 : c)];
            }
            k = f2key(r64 ? acc * 0.125f : acc / sqrt_r);
          }
          cnt += k != 0u;
          keys[n] = k;
        }
      }
    }
  } else {
    for (int64_t n = threadIdx.x; n < len; n += ITEM_BLOCK) {
      const uint32_t k = compute_key(n);
      cnt += k != 0u;
      if (keys_in_lds) keys[n] = k;
    }
  }
  uint32_t allowed_total;
  block_excl_scan<ITEM_BLOCK>(cnt, scratch, &allowed_total);
  const int leff = (int)min((int64_t)p.L, (int64_t)allowed_total);
  if (leff == 0) {
    if (threadIdx.x == 0) p.sl_count[item] = 0;
    return;
  }

  auto get_key = [&](int64_t n) -> uint32_t { return keys_in_lds ? keys[n] : compute_key(n); };

  uint32_t T;
  int keq;
  radix_select_u32<ITEM_BLOCK>([&](int i) { return get_key(i); }, (int)len, leff, hist, scratch, shared, &T, &keq);

  // compaction in key-index order over thread-contiguous segments
  const int64_t seg = (len + ITEM_BLOCK - 1) / ITEM_BLOCK;
  const int64_t lo = min((int64_t)threadIdx.x * seg, len);
  const int64_t hi = min(lo + seg, len);
  uint32_t gt = 0, eq = 0;
  for (int64_t n = lo; n < hi; ++n) {
    const uint32_t k = get_key(n);
    gt += k > T;
    eq += k == T;
  }
  const uint32_t eq_before = block_excl_scan<ITEM_BLOCK>(eq, scratch, nullptr);
  const int take_eq = max(0, min((int)eq, keq - (int)eq_before));
  uint32_t pos = block_excl_scan<ITEM_BLOCK>(gt + (uint32_t)take_eq, scratch, nullptr);
  int taken = 0;
  for (int64_t n = lo; n < hi; ++n) {
    const uint32_t k = get_key(n);
    if (k > T) {
      set_slot(pos++, n);
    } else if (k == T && taken < take_eq) {
      set_slot(pos++, n);
      ++taken;
    }
  }
  __syncthreads();

  // exact low-rank rescore of the shortlist (torch's sum order)
  const float* kl = p.k_low + (int64_t)h * p.klow_hs + off * p.R;
  int32_t* out_idx = p.sl_idx + (int64_t)item * p.L;
  float* out_rank = p.sl_rank + (int64_t)item * p.L;
  if (r64 && ((uintptr_t)kl & 15u) == 0) {  // block-uniform
    // lane octet o takes shortlist entries o, o + 128, ...: eight lanes per
    // row, two 16-byte loads each (a row's two 128-byte lines), REG_OCT
    // rows in flight; rank_dot64_oct8 sums in torch_order_dot64's order
    const int oct = (int)threadIdx.x >> 3, c = (int)threadIdx.x & 7;
    const float4 q0 = reinterpret_cast<const float4*>(ql)[c], q1 = reinterpret_cast<const float4*>(ql)[8 + c];
    const float4* kl4 = reinterpret_cast<const float4*>(kl);
    for (int j0 = 0; j0 < leff; j0 += REG_OCT * (ITEM_BLOCK / 8)) {
      float4 r0[REG_OCT], r1[REG_OCT];
#pragma unroll
      for (int u = 0; u < REG_OCT; ++u) {
        const int j = j0 + u * (ITEM_BLOCK / 8) + oct;
        const int64_t n = slot(j < leff ? j : 0);
        r0[u] = kl4[n * 16 + c];
        r1[u] = kl4[n * 16 + 8 + c];
      }
#pragma unroll
      for (int u = 0; u < REG_OCT; ++u) {
        const int j = j0 + u * (ITEM_BLOCK / 8) + oct;
        const float dot = rank_dot64_oct8(r0[u], r1[u], q0, q1);
        if (c == 0 && j < leff) out_rank[j] = dot * 0.125f;
      }
    }
    for (int j = threadIdx.x; j < leff; j += ITEM_BLOCK) out_idx[j] = (int32_t)slot(j);
  } else {
    for (int j = threadIdx.x; j < leff; j += ITEM_BLOCK) {
      const int64_t n = slot(j);
      const float* row = kl + n * p.R;
      const float dot = p.R == 64 ? torch_order_dot64(row, ql) : torch_order_dot(row, ql, p.R);
      out_idx[j] = (int32_t)n;
      out_rank[j] = r64 ? dot * 0.125f : dot / sqrt_r;
    }
  }
  if (threadIdx.x == 0) p.sl_count[item] = leff;
}


// items: n_seq * H * Q; workgroups take head-major item ranges per XCD
// (xcd_range_item), so one XCD's L2 holds the k_low rows of one or two heads.
template <int NPT, int SB>
__global__ void __launch_bounds__(ITEM_BLOCK, NPT <= 8 ? 8 : 4) summon_regs_kernel(SummonParams p, int64_t items) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int64_t item = xcd_range_item((int64_t)blockIdx.x, items);
  if (item < 0) return;  // block-uniform: past the last item
  regs_item<NPT, SB>(p, (int)item, lds);
}

template <int NPT, int SB>
int launch_regs(const SummonParams& p, int64_t items, size_t lds, hipStream_t stream) {
  SVA_SET_MAX_LDS_ONCE((summon_regs_kernel<NPT, SB>), kMaxLds, "hipFuncSetAttribute(summon_regs_kernel)");
  hipLaunchKernelGGL((summon_regs_kernel<NPT, SB>), dim3((unsigned)xcd_range_grid(items)), dim3(ITEM_BLOCK), lds,
                     stream, p, items);
  SVA_CHECK_LAUNCH("summon_regs_kernel");
  return SVA_OK;
}

template <int NPT>
int launch_regs_codes(const SummonParams& p, int64_t items, size_t lds, hipStream_t stream) {
  // one load per key for uint8 codes of 1, 2 or 4 subspaces at aligned rows
  const int64_t S = p.S;
  const bool u8 = p.ctype == CODE_U8 && (S == 1 || S == 2 || S == 4) && p.code_hs % S == 0 &&
                  ((uintptr_t)p.codes % (uintptr_t)S) == 0;
  if (u8 && S == 1) return launch_regs<NPT, 1>(p, items, lds, stream);
  if (u8 && S == 2) return launch_regs<NPT, 2>(p, items, lds, stream);
  if (u8 && S == 4) return launch_regs<NPT, 4>(p, items, lds, stream);
  return launch_regs<NPT, 0>(p, items, lds, stream);
}
}  // namespace

namespace sva {

bool summon_regs_eligible(const SummonParams& p) {
  if (p.B <= 0 || p.R != 64 || p.L > REG_MAX_L || p.N > 16 * ITEM_BLOCK) return false;
  if (((uintptr_t)p.k_low & 15u) != 0 || p.klow_hs % 4 != 0 || ((uintptr_t)p.q_low & 15u) != 0) return false;
  return reg_lds_layout(p.S, p.C, p.L, 16).total <= kMaxLds;
}

int summon_regs_path(const SummonParams& p, int64_t items, hipStream_t stream) {
  const int npt = p.N <= 4 * ITEM_BLOCK ? 4 : (p.N <= 8 * ITEM_BLOCK ? 8 : 16);
  const size_t lds = (size_t)reg_lds_layout(p.S, p.C, p.L, npt).total;
  if (npt == 4) return launch_regs_codes<4>(p, items, lds, stream);
  if (npt == 8) return launch_regs_codes<8>(p, items, lds, stream);
  return launch_regs_codes<16>(p, items, lds, stream);
}

int summon_item_path(const SummonParams& p, int64_t items, hipStream_t stream) {
  const bool idx16 = p.N <= 65536;  // every sequence's length is at most N
  const bool keys_fit = item_lds_layout(p.S, p.C, p.R, p.L, p.N, true, idx16).total <= kMaxLds;
  const ItemLds layout = item_lds_layout(p.S, p.C, p.R, p.L, p.N, keys_fit, idx16);
  SVA_UNSUPPORTED(layout.total <= kMaxLds, "sva_summon: shortlist %d with %dx%d codes exceeds LDS", p.L, p.S, p.C);
  SVA_SET_MAX_LDS_ONCE(summon_item_kernel, kMaxLds, "hipFuncSetAttribute(summon_item_kernel)");
  hipLaunchKernelGGL(summon_item_kernel, dim3((unsigned)items), dim3(ITEM_BLOCK), (size_t)layout.total, stream, p,
                     (keys_fit ? 1 : 0) | (idx16 ? 2 : 0));
  SVA_CHECK_LAUNCH("summon_item_kernel");
  return SVA_OK;
}

}  // namespace sva

extern "C" int sva_summon_strategy(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t R, int64_t S,
                                   int64_t C, int64_t L, int code_type, int mask_type) {
  sva::SummonParams p{};
  alignas(16) static const float dummy[4] = {0, 0, 0, 0};
  p.codes = dummy;
  p.ctype = code_type;
  p.code_hs = 0;
  p.offs = n_seq == 1 ? nullptr : (const int64_t*)dummy;
  p.H = (int)H;
  p.Q = (int)Q;
  p.N = n_keys;
  p.R = (int)R;
  p.S = (int)S;
  p.C = (int)C;
  p.L = (int)L;
  p.mask = dummy;
  p.mask_type = mask_type;
  if (sva::summon_class_eligible(p, n_seq * H * Q)) return 2;
  if (sva::summon_wide_eligible(p, n_seq * H * Q)) return 1;
  p.B = 1;
  return sva::summon_regs_eligible(p) ? 3 : 0;
}

extern "C" size_t sva_summon_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t L) {
  return sva::summon_wide_workspace_bytes(n_seq, H, Q, n_keys, L);
}

namespace {

int summon_impl(const char* fn, const float* lut, const float* score_range, const float* q_low, const void* codes,
                int code_type, int64_t code_head_stride, const float* k_low, int64_t k_low_head_stride,
                const int64_t* seq_offsets, const int64_t* seq_lens, int64_t n_seq, int64_t H, int64_t Q,
                int64_t n_keys, int64_t R, int64_t S, int64_t C, int64_t L, const void* mask, int mask_type,
                int64_t mask_tok_stride, int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B,
                int32_t* fin_idx, int32_t* fin_count, void* workspace, size_t workspace_bytes, void* stream,
                const sva::FusedVerify* fv = nullptr, bool* fused = nullptr, int32_t* overshoot = nullptr,
                const sva::QueryLaunch* query = nullptr, unsigned long long* stats = nullptr,
                const sva::WriteParams* append = nullptr) {
  if (fused != nullptr) *fused = false;
  SVA_REQUIRE(lut && score_range && q_low && codes && k_low && sl_count, "%s: null pointer", fn);
  SVA_REQUIRE((sl_idx == nullptr) == (sl_rank == nullptr), "%s: shortlist indices and ranks go together", fn);
  SVA_REQUIRE((seq_offsets == nullptr) == (seq_lens == nullptr), "%s: offsets and lengths go together", fn);
  SVA_REQUIRE(n_seq > 0 && H > 0 && Q > 0 && n_keys >= 0, "%s: bad sizes", fn);
  SVA_REQUIRE(n_keys < (1ll << 31), "%s: at most 2^31-1 keys per sequence", fn);
  SVA_REQUIRE(R > 0 && R <= 511 && S > 0 && R % S == 0 && C > 0 && S * C <= 16384,
              "%s: bad rank/PQ layout R=%lld S=%lld C=%lld", fn, (long long)R, (long long)S, (long long)C);
  SVA_REQUIRE(L > 0 && L <= 16384, "%s: shortlist %lld out of range (1..16384)", fn, (long long)L);
  SVA_REQUIRE(code_type >= 0 && code_type <= 3, "%s: bad code type", fn);
  SVA_REQUIRE(mask_type >= 0 && mask_type <= 4, "%s: bad mask type", fn);
  SVA_REQUIRE(mask_type == SVA_MASK_NONE || mask_type == SVA_MASK_BOOL || mask != nullptr,
              "%s: mask type given without a mask", fn);
  SVA_REQUIRE(R != 64 || (((uintptr_t)k_low & 15u) == 0 && k_low_head_stride % 4 == 0),
              "%s: k_low must be 16-byte aligned", fn);
  const int64_t items = n_seq * H * Q;
  SVA_REQUIRE(items < (1ll << 31), "%s: too many query items", fn);
  sva::SummonParams p;
  p.lut = lut;
  p.range = score_range;
  p.q_low = q_low;
  p.codes = codes;
  p.ctype = code_type;
  p.code_hs = code_head_stride;
  p.k_low = k_low;
  p.klow_hs = k_low_head_stride;
  p.offs = seq_offsets;
  p.lens = seq_lens;
  p.H = (int)H;
  p.Q = (int)Q;
  p.N = n_keys;
  p.R = (int)R;
  p.S = (int)S;
  p.C = (int)C;
  p.L = (int)L;
  p.mask = mask;
  p.mask_type = mask_type;
  p.mask_ts = mask_tok_stride;
  p.sqrt_r = (float)sqrt((double)R);
  p.sl_idx = sl_idx;
  p.sl_rank = sl_rank;
  p.sl_count = sl_count;
  p.B = (int)B;
  p.fin_idx = fin_idx;
  p.fin_count = fin_count;
  p.stats = stats;
  // a prepared query launch (the tables this call reads): the code-class
  // path runs its decode form in one grid with the code counts; every other
  // path launches it first
  const bool class_path = n_keys > 0 && sva::summon_class_eligible(p, items);
  SVA_REQUIRE(stats == nullptr || (n_keys > 0 && !class_path && !sva::summon_wide_eligible(p, items) &&
                                   sva::summon_regs_eligible(p)),
              "%s: a statistics row is added on the per-item register path only", fn);
  // without shortlist outputs only the fused per-item path (strategy 3) runs
  SVA_UNSUPPORTED(sl_idx != nullptr || n_keys == 0 ||
                      (B > 0 && !class_path && !sva::summon_wide_eligible(p, items) && sva::summon_regs_eligible(p)),
                  "%s: these shapes keep the shortlist in memory; pass shortlist outputs", fn);
  // one token of one sequence on the per-item register path with the
  // verifier: the query, the summon and the verifier in one launch, with a
  // decode step's catalog append in front where that launch can take it
  const bool item_one_launch = fv != nullptr && fused != nullptr && query != nullptr && n_keys > 0 && !class_path &&
                               !sva::summon_wide_eligible(p, items);
  if (append != nullptr && !(item_one_launch && sva::item_fused_eligible(p, *query, *fv, append))) {
    // the catalog's new rows on their own, before anything reads them
    const int rc = sva::write_encode_launch(*append, (hipStream_t)stream);
    if (rc != SVA_OK) return rc;
    append = nullptr;
  }
  if (item_one_launch && sva::item_fused_eligible(p, *query, *fv, append)) {
    const int rc = sva::item_lookup_verify_path(*query, p, *fv, append, overshoot, (hipStream_t)stream);
    if (rc == SVA_OK) *fused = true;
    return rc;
  }
  if (query != nullptr && !(class_path && query->form == sva::QUERY_DECODE_1_256)) {
    const int rc = sva::query_lut_launch(*query, (hipStream_t)stream);
    if (rc != SVA_OK) return rc;
    query = nullptr;
  }
  if (n_keys == 0) {
    int rc = sva::fill_i32(sl_count, items, 0, (hipStream_t)stream);
    if (rc == SVA_OK && B > 0) rc = sva::fill_i32(fin_count, items, 0, (hipStream_t)stream);
    return rc;
  }
  if (class_path) {
    const bool with_fv = fv != nullptr && sva::fused_verify_eligible(p, items, *fv);
    const int rc = sva::summon_class_path(p, workspace, workspace_bytes, (hipStream_t)stream, with_fv ? fv : nullptr,
                                          overshoot, query);
    if (rc == SVA_OK && fused != nullptr) *fused = with_fv;
    return rc;
  }
  if (sva::summon_wide_eligible(p, items)) {
    const bool with_fv = fv != nullptr && sva::fused_verify_eligible(p, items, *fv);
    const int rc = sva::summon_wide_path(p, workspace, workspace_bytes, (hipStream_t)stream, with_fv ? fv : nullptr,
                                         overshoot);
    if (rc == SVA_OK && fused != nullptr) *fused = with_fv;
    return rc;
  }
  if (overshoot != nullptr) {  // the per-item paths use no sampled floor
    const int rc = sva::fill_i32(overshoot, items, 0, (hipStream_t)stream);
    if (rc != SVA_OK) return rc;
  }
  if (sva::summon_regs_eligible(p)) return sva::summon_regs_path(p, items, (hipStream_t)stream);
  int rc = sva::summon_item_path(p, items, (hipStream_t)stream);
  if (rc == SVA_OK && B > 0)
    rc = sva::budget_select_launch(sl_idx, sl_rank, sl_count, items, L, B, fin_idx, fin_count, true,
                                   (hipStream_t)stream);  // the item kernel's shortlists ascend
  return rc;
}

}  // namespace

extern "C" int sva_summon(const float* lut, const float* score_range, const float* q_low, const void* codes,
                          int code_type, int64_t code_head_stride, const float* k_low, int64_t k_low_head_stride,
                          const int64_t* seq_offsets, const int64_t* seq_lens, int64_t n_seq, int64_t H, int64_t Q,
                          int64_t n_keys, int64_t R, int64_t S, int64_t C, int64_t L, const void* mask, int mask_type,
                          int64_t mask_tok_stride, int32_t* sl_idx, float* sl_rank, int32_t* sl_count,
                          void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  return summon_impl("sva_summon", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                     k_low_head_stride, seq_offsets, seq_lens, n_seq, H, Q, n_keys, R, S, C, L, mask, mask_type,
                     mask_tok_stride, sl_idx, sl_rank, sl_count, 0, nullptr, nullptr, workspace, workspace_bytes,
                     stream);
}

extern "C" int sva_summon_select(const float* lut, const float* score_range, const float* q_low, const void* codes,
                                 int code_type, int64_t code_head_stride, const float* k_low,
                                 int64_t k_low_head_stride, const int64_t* seq_offsets, const int64_t* seq_lens,
                                 int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t R, int64_t S, int64_t C,
                                 int64_t L, const void* mask, int mask_type, int64_t mask_tok_stride, int32_t* sl_idx,
                                 float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx, int32_t* fin_count,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(fin_idx && fin_count, "sva_summon_select: null pointer");
  SVA_REQUIRE(B > 0 && B <= 8192, "sva_summon_select: budget %lld out of range (1..8192)", (long long)B);
  return summon_impl("sva_summon_select", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                     k_low_head_stride, seq_offsets, seq_lens, n_seq, H, Q, n_keys, R, S, C, L, mask, mask_type,
                     mask_tok_stride, sl_idx, sl_rank, sl_count, B, fin_idx, fin_count, workspace, workspace_bytes,
                     stream);
}

extern "C" int sva_lookup_select(const void* q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R,
                                 int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                                 const void* codes, int code_type, int64_t code_head_stride, const float* k_low,
                                 int64_t k_low_head_stride, int64_t n_keys, int64_t L, const void* mask, int mask_type,
                                 int64_t mask_tok_stride, float* q_low, float* lut, float* score_range,
                                 int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx,
                                 int32_t* fin_count, void* workspace, size_t workspace_bytes, void* stream) {
  sva::clear_error();
  SVA_REQUIRE(q && q_proj && scale && codebooks && codes && q_low && lut && score_range,
              "sva_lookup_select: null pointer");
  SVA_REQUIRE(fin_idx && fin_count, "sva_lookup_select: null pointer");
  SVA_REQUIRE(B > 0 && B <= 8192, "sva_lookup_select: budget %lld out of range (1..8192)", (long long)B);
  SVA_REQUIRE(H > 0 && n_keys >= 0 && L > 0, "sva_lookup_select: bad sizes");
  sva::QueryLaunch ql;
  const int rc = sva::query_lut_setup(q, q_dtype, 0, q_head_stride, 0, 1, H, 1, D, R, S, C, q_proj, scale, codebooks,
                                      codes, code_type, code_head_stride, n_keys, L, q_low, lut, score_range, &ql);
  if (rc != SVA_OK) return rc;
  return summon_impl("sva_lookup_select", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                     k_low_head_stride, nullptr, nullptr, 1, H, 1, n_keys, R, S, C, L, mask, mask_type,
                     mask_tok_stride, sl_idx, sl_rank, sl_count, B, fin_idx, fin_count, workspace, workspace_bytes,
                     stream, nullptr, nullptr, nullptr, &ql);
}

namespace sva {

// sva_lookup_verify with an optional statistics row (see SummonParams::stats;
// the per-item register path only).  The caller clears the error state.
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
                       void* stream, unsigned long long* stats, const WriteParams* append) {
  SVA_REQUIRE(q && q_proj && scale && codebooks && codes && q_low && lut && score_range,
              "sva_lookup_verify: null pointer");
  SVA_REQUIRE(fin_idx && fin_count && keys && values && out, "sva_lookup_verify: null pointer");
  SVA_REQUIRE(B > 0 && B <= 8192, "sva_lookup_verify: budget %lld out of range (1..8192)", (long long)B);
  SVA_REQUIRE(H > 0 && G > 0 && H % G == 0 && n_keys > 0 && L > 0, "sva_lookup_verify: bad sizes");
  SVA_REQUIRE(q_dtype >= 0 && q_dtype <= 2 && kv_dtype >= 0 && kv_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2,
              "sva_lookup_verify: bad dtype");
  sva::QueryLaunch ql;
  int rc = sva::query_lut_setup(q, q_dtype, 0, q_head_stride, 0, 1, H, 1, D, R, S, C, q_proj, scale, codebooks, codes,
                                code_type, code_head_stride, n_keys, L, q_low, lut, score_range, &ql);
  if (rc != SVA_OK) return rc;
  sva::FusedVerify fv{};
  fv.q = q;
  fv.q_dtype = q_dtype;
  fv.q_hs = q_head_stride;
  fv.keys = keys;
  fv.values = values;
  fv.kv_dtype = kv_dtype;
  fv.kv_hs = kv_head_stride;
  fv.kv_rs = kv_row_stride;
  const uintptr_t kv_align = kv_dtype == 0 ? 15u : 7u;
  fv.kv_vec = (((uintptr_t)keys | (uintptr_t)values) & kv_align) == 0 && kv_head_stride % 4 == 0 &&
              kv_row_stride % 4 == 0;
  fv.G = (int)G;
  fv.D = (int)D;
  fv.scaling = scaling;
  fv.out = out;
  fv.out_dtype = out_dtype;
  fv.o_hs = out_head_stride;
  bool fused = false;
  rc = summon_impl("sva_lookup_verify", lut, score_range, q_low, codes, code_type, code_head_stride, k_low,
                   k_low_head_stride, nullptr, nullptr, 1, H, 1, n_keys, R, S, C, L, mask, mask_type, mask_tok_stride,
                   sl_idx, sl_rank, sl_count, B, fin_idx, fin_count, workspace, workspace_bytes, stream, &fv, &fused,
                   floor_overshoot, &ql, stats, append);
  if (rc != SVA_OK || fused) return rc;
  return sva_verify(q, q_dtype, 0, q_head_stride, 0, keys, values, kv_dtype, kv_head_stride, kv_row_stride, nullptr,
                    nullptr, n_keys, fin_idx, fin_count, 1, H, G, 1, D, B, scaling, out, out_dtype, 0, out_head_stride,
                    0, verify_workspace, verify_workspace_bytes, stream);
}

}  // namespace sva

extern "C" int sva_lookup_verify(const void* q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R,
                                 int64_t S, int64_t C, const float* q_proj, const float* scale, const float* codebooks,
                                 const void* codes, int code_type, int64_t code_head_stride, const float* k_low,
                                 int64_t k_low_head_stride, int64_t n_keys, int64_t L, const void* mask, int mask_type,
                                 int64_t mask_tok_stride, float* q_low, float* lut, float* score_range,
                                 int32_t* sl_idx, float* sl_rank, int32_t* sl_count, int64_t B, int32_t* fin_idx,
                                 int32_t* fin_count, void* workspace, size_t workspace_bytes, const void* keys,
                                 const void* values, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                                 int64_t G, float scaling, void* out, int out_dtype, int64_t out_head_stride,
                                 void* verify_workspace, size_t verify_workspace_bytes, int32_t* floor_overshoot,
                                 void* stream) {
  sva::clear_error();
  return sva::lookup_verify_impl(q, q_dtype, q_head_stride, H, D, R, S, C, q_proj, scale, codebooks, codes, code_type,
                                 code_head_stride, k_low, k_low_head_stride, n_keys, L, mask, mask_type,
                                 mask_tok_stride, q_low, lut, score_range, sl_idx, sl_rank, sl_count, B, fin_idx,
                                 fin_count, workspace, workspace_bytes, keys, values, kv_dtype, kv_head_stride,
                                 kv_row_stride, G, scaling, out, out_dtype, out_head_stride, verify_workspace,
                                 verify_workspace_bytes, floor_overshoot, stream, nullptr);
}
