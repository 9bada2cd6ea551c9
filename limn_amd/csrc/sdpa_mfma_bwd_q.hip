// The MFMA flash-attention bwd_q pass at every dtype, head dim, causality and masking.

#include "sdpa_mfma.h"

namespace limn {

int launch_mfma_bwd_q(const SdpaArgs& a) { return launch_pass<SDPA_BWD_Q>(a); }

}  // namespace limn
