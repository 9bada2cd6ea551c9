// The MFMA flash-attention bwd_kv pass at every dtype, head dim, causality and masking.

#include "sdpa_mfma.h"

namespace limn {

int launch_mfma_bwd_kv(const SdpaArgs& a) { return launch_pass<SDPA_BWD_KV>(a); }

}  // namespace limn
