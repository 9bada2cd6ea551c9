// Both backward passes through the dS hand-off: the pipelined dK/dV pass storing dS, then the
// dQ pass reading it (sdpa_mfma.h).

#include "sdpa_mfma.h"

namespace limn {

int launch_mfma_bwd(const SdpaArgs& a, void* ws, int passes) {
  if (a.dtype == LIMN_HIP_BFLOAT16)
    return a.causal ? launch_bwd_ds<BF16, true>(a, ws, passes) : launch_bwd_ds<BF16, false>(a, ws, passes);
  return a.causal ? launch_bwd_ds<F16, true>(a, ws, passes) : launch_bwd_ds<F16, false>(a, ws, passes);
}

}  // namespace limn
