// Dispatch of the MFMA flash-attention family (kernels in sdpa_mfma.h, one translation unit per
// pass so they compile in parallel).

#include "sdpa_mfma.h"

namespace limn {

bool mfma_supports(int dtype, int64_t hd, int64_t hd_v) {
  return (dtype == LIMN_HIP_BFLOAT16 || dtype == LIMN_HIP_FLOAT16) && hd == hd_v && (hd == 64 || hd == 128);
}

bool mfma_fits(int64_t t_q, int64_t t_k, int64_t hd) {
  // per-head byte offsets are 32-bit inside the kernels (buffer resources included)
  const int64_t limit = ((int64_t)1 << 31) - 1;
  return t_q * hd * 2 < limit && t_k * hd * 2 < limit;
}

int launch_sdpa_mfma(SdpaPass pass, const SdpaArgs& a) {
  if (pass == SDPA_FWD) return launch_mfma_fwd(a);
  if (pass == SDPA_BWD_Q) return launch_mfma_bwd_q(a);
  return launch_mfma_bwd_kv(a);
}

int64_t mfma_bwd_workspace(const SdpaArgs& a) {
  if (!mfma_supports(a.dtype, a.hd, a.hd_v) || !mfma_fits(a.t_q, a.t_k, a.hd) || a.hd != 128 || a.mask != nullptr) return 0;
  // keys past t_k inside a block are not masked by the unmasked dK/dV pass; causal calls mask them
  // on the diagonal tiles, other calls need whole blocks
  if (!a.causal && a.t_k % 128 != 0) return 0;
  return a.batch * DsLayout::of(a.t_q, a.t_k, a.causal).units_per_head() * DS_UNIT;
}

}  // namespace limn
