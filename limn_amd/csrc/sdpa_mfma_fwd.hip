// The MFMA flash-attention fwd pass at every dtype, head dim, causality and masking.

#include "sdpa_mfma.h"

namespace limn {

int launch_mfma_fwd(const SdpaArgs& a) { return launch_pass<SDPA_FWD>(a); }

}  // namespace limn
