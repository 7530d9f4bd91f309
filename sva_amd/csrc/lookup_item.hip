// Host side of the fused one-token lookup on the per-item register path
// (device code in lookup_item.cuh, one translation unit per verifier variant).
#include "lookup_item.cuh"

namespace sva {

bool item_fused_eligible(const SummonParams& p, const QueryLaunch& ql, const FusedVerify& fv) {
  const int form_s = ql.form == QUERY_DECODE_4_64    ? 4
                     : ql.form == QUERY_DECODE_2_256 ? 2
                     : ql.form == QUERY_DECODE_1_256 ? 1
                                                     : 0;
  if (form_s == 0 || form_s != p.S || ql.blocks != p.H) return false;
  if (p.Q != 1 || p.offs != nullptr || p.N <= 0 || p.B <= 0 || p.ctype != CODE_U8) return false;
  // the register path's one load per key of S code bytes
  if (p.code_hs % p.S != 0 || ((uintptr_t)p.codes % (uintptr_t)p.S) != 0) return false;
  if (!summon_regs_eligible(p)) return false;
  // head_dim 64: the decode query's (its form requires D = R = 64)
  if (fv.out == nullptr || fv.D != 64 || fv.G <= 0 || p.H % fv.G != 0) return false;
  if (fv.q_dtype < 0 || fv.q_dtype > 2 || fv.kv_dtype < 0 || fv.kv_dtype > 2 || fv.out_dtype < 0 || fv.out_dtype > 2)
    return false;
  return item_lookup::item_lds(p, fv.D) <= item_lookup::kDynLds;
}

int item_lookup_verify_path(const QueryLaunch& ql, const SummonParams& p, const FusedVerify& fv, int32_t* overshoot,
                            hipStream_t stream) {
  using namespace item_lookup;
  SVA_REQUIRE(fv.D == 64, "item_lookup_verify: head_dim %d", fv.D);
  if (fv.kv_dtype == BF16) return launch_v64_bf16(ql.p, p, fv, overshoot, stream);
  if (fv.kv_dtype == F16) return launch_v64_f16(ql.p, p, fv, overshoot, stream);
  return launch_v64_f32(ql.p, p, fv, overshoot, stream);
}

}  // namespace sva
