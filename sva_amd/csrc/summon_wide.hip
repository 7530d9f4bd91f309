// Host side of the long-context summon: eligibility, workspace layout and the
// launches (device code in summon_wide.cuh, kernels in summon_wide_*.hip).
#include "summon_wide.cuh"

namespace sva {

using namespace wide;

namespace {

int launch_finish_any(const WideArgs& a, int64_t items, hipStream_t stream) {
  if (a.fv.out == nullptr) return launch_finish_nov(a, items, stream);
  const int kv = a.fv.kv_dtype;
  if (a.fv.D == 64) {
    if (kv == BF16) return launch_finish_v64_bf16(a, items, stream);
    if (kv == F16) return launch_finish_v64_f16(a, items, stream);
    return launch_finish_v64_f32(a, items, stream);
  }
  if (kv == BF16) return launch_finish_v128_bf16(a, items, stream);
  if (kv == F16) return launch_finish_v128_f16(a, items, stream);
  return launch_finish_v128_f32(a, items, stream);
}

}  // namespace

bool summon_wide_eligible(const SummonParams& p, int64_t items) {
  if (p.Q != 1 || p.offs != nullptr || p.ctype != CODE_U8 || p.C > 256) return false;
  if (p.S != 1 && p.S != 2 && p.S != 4 && p.S != 8) return false;
  if (p.R != 64 || p.N < kWideMinKeys || p.N >= (1ll << 30) || items > kMaxWideItems) return false;
  if (p.L > FIN_MAX_L) return false;
  if (((uintptr_t)p.codes & 15u) != 0 || p.code_hs % 16 != 0) return false;
  if (((uintptr_t)p.k_low & 15u) != 0 || p.klow_hs % 4 != 0 || ((uintptr_t)p.q_low & 15u) != 0) return false;
  if (p.mask_type != MASK_NONE && p.mask_type != MASK_BOOL && p.mask == nullptr) return false;
  return true;
}

size_t summon_wide_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t L) {
  const int64_t items = n_seq * H * Q;
  if (n_seq != 1 || Q != 1 || n_keys < kWideMinKeys || items > kMaxWideItems) return 256;
  const int64_t W = (n_keys + CHUNK - 1) / CHUNK;
  return counters_bytes(items, W) + align256((size_t)items * (size_t)W * CHUNK * (sizeof(uint64_t) + sizeof(float))) +
         over_bytes(items, std::max<int64_t>(L, 1));
}

bool summon_class_eligible(const SummonParams& p, int64_t items) {
  if (!summon_wide_eligible(p, items) || !class_shape(p.S, p.C, p.L)) return false;
  return (p.N + CLASS_CHUNK - 1) / CLASS_CHUNK <= CLASS_MAX_W;
}

int summon_class_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream,
                      const FusedVerify* fv, int32_t* overshoot, const QueryLaunch* query) {
  const int64_t items = (int64_t)p.H;  // one sequence, q = 1
  const int64_t W = (p.N + CLASS_CHUNK - 1) / CLASS_CHUNK;
  const size_t counts = align256((size_t)(items * W * 256) * sizeof(uint32_t));
  const size_t bound = align256((size_t)(items * 4) * sizeof(uint32_t));
  const size_t need = counts + bound + align256((size_t)(items * W * 2) * sizeof(uint32_t));
  SVA_REQUIRE(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace & 255u) == 0,
              "sva_summon: workspace of %zu bytes (256-byte aligned) required, got %zu", need, workspace_bytes);
  ClassArgs a;
  a.p = p;
  a.W = (int)W;
  a.overshoot = overshoot;
  a.fv = FusedVerify{};
  a.fv.out = nullptr;
  if (fv != nullptr) {
    SVA_REQUIRE(fused_verify_eligible(p, items, *fv), "summon_class_path: the fused verifier does not fit these sizes");
    a.fv = *fv;
  }
  char* ws = (char*)workspace;
  a.counts = (uint32_t*)ws;
  a.bound = (uint32_t*)(ws + counts);
  a.woff = (uint32_t*)(ws + counts + bound);
  const bool masked = p.mask_type == MASK_F32 || p.mask_type == MASK_BF16 || p.mask_type == MASK_F16;
  return launch_class(a, items, masked, query, stream);
}

bool fused_verify_eligible(const SummonParams& p, int64_t items, const FusedVerify& fv) {
  if (!summon_wide_eligible(p, items) || p.offs != nullptr || items != p.H || p.B <= 0) return false;
  if (fv.D != 64 && fv.D != 128) return false;
  if (fv.G <= 0 || p.H % fv.G != 0) return false;
  if (fv.q_dtype < 0 || fv.q_dtype > 2 || fv.kv_dtype < 0 || fv.kv_dtype > 2 || fv.out_dtype < 0 || fv.out_dtype > 2)
    return false;
  return verify_item_lds(p.B, fv.D) <= kFinLds;
}

int summon_wide_path(const SummonParams& p, void* workspace, size_t workspace_bytes, hipStream_t stream,
                     const FusedVerify* fv, int32_t* overshoot) {
  const int64_t items = (int64_t)p.H;  // one sequence, q = 1
  const size_t need = summon_wide_workspace_bytes(1, p.H, 1, p.N, p.L);
  SVA_REQUIRE(workspace != nullptr && workspace_bytes >= need && ((uintptr_t)workspace & 255u) == 0,
              "sva_summon: workspace of %zu bytes (256-byte aligned) required, got %zu", need, workspace_bytes);
  WideArgs a;
  a.p = p;
  a.W = (int)((p.N + CHUNK - 1) / CHUNK);
  a.overshoot = overshoot;
  a.fv = FusedVerify{};
  a.fv.out = nullptr;
  if (fv != nullptr) {
    SVA_REQUIRE(fused_verify_eligible(p, items, *fv), "summon_wide_path: the fused verifier does not fit these sizes");
    a.fv = *fv;
  }
  char* ws = (char*)workspace;
  a.ncand = (uint32_t*)ws;
  a.nallow = a.ncand + items * a.W * NW;
  a.wg_count = (uint32_t*)(ws + align256((size_t)(2 * items * a.W * NW) * sizeof(uint32_t)));
  a.wg_cand = (uint64_t*)((char*)a.wg_count + align256((size_t)(2 * items * a.W) * sizeof(uint32_t)));
  a.wg_rank = (float*)(a.wg_cand + items * a.W * WG_CAP);
  a.cand = (uint64_t*)(ws + counters_bytes(items, a.W));
  a.cand_rank = (float*)(ws + counters_bytes(items, a.W) + (size_t)items * (size_t)a.W * CHUNK * sizeof(uint64_t));
  a.items = (int)items;
  a.K = over_slices(items);
  char* over = ws + counters_bytes(items, a.W) +
               align256((size_t)items * (size_t)a.W * CHUNK * (sizeof(uint64_t) + sizeof(float)));
  a.arrive = (uint32_t*)over;
  a.slice_n = (uint32_t*)(over + align256((size_t)items * sizeof(uint32_t)));
  a.slice_list = (uint64_t*)(over + align256((size_t)items * sizeof(uint32_t)) +
                             align256((size_t)(items * a.K) * sizeof(uint32_t)));
  // a bool mask allows every key (the reference's `mask > -1e4` rule)
  const bool masked = p.mask_type == MASK_F32 || p.mask_type == MASK_BF16 || p.mask_type == MASK_F16;
  const int rc = launch_scan(a, items, masked, stream);
  if (rc != SVA_OK) return rc;
  return launch_finish_any(a, items, stream);
}

}  // namespace sva
