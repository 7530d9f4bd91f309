// Host side of the fused one-token lookup on the per-item register path
// (device code in lookup_item.cuh, one translation unit per verifier variant).
#include "lookup_item.cuh"

namespace sva {

bool item_fused_eligible(const SummonParams& p, const QueryLaunch& ql, const FusedVerify& fv,
                         const WriteParams* append) {
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
  if (append != nullptr) {  // the append writes this lookup's catalog, in the form compiled in
    if (fv.kv_dtype == F32) return false;  // the fp32 K / V variants carry no append
    const WriteParams& w = *append;
    const int form = write_few_form(w);
    if (form < 0 || (p.S > 1 && form != 64 / p.S) || w.n_seq != 1 || w.codes == nullptr || w.codes != p.codes || w.k_low != p.k_low ||
        w.code_hs != p.code_hs || w.klow_hs != p.klow_hs || w.ctype != p.ctype || w.H != p.H || w.G != fv.G ||
        w.R != p.R || w.S != p.S || w.C != p.C || w.D != fv.D || w.row0 + w.n_rows > p.N)
      return false;
  }
  return item_lookup::item_lds(p, fv.D) <= item_lookup::kDynLds;
}

int item_lookup_verify_path(const QueryLaunch& ql, const SummonParams& p, const FusedVerify& fv,
                            const WriteParams* append, int32_t* overshoot, hipStream_t stream) {
  using namespace item_lookup;
  SVA_REQUIRE(fv.D == 64, "item_lookup_verify: head_dim %d", fv.D);
  WriteParams none{};
  none.n_rows = 0;
  const WriteParams& wp = append != nullptr ? *append : none;
  if (fv.kv_dtype == BF16) return launch_v64_bf16(ql.p, p, fv, wp, overshoot, stream);
  if (fv.kv_dtype == F16) return launch_v64_f16(ql.p, p, fv, wp, overshoot, stream);
  return launch_v64_f32(ql.p, p, fv, wp, overshoot, stream);
}

}  // namespace sva
