// Internal launch interface between the C ABI (capi.hip) and the attention kernel families.
#pragma once

#include "common.h"

namespace limn {

// One fused-attention call, already validated by the C ABI layer.
struct SdpaArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  const void* lse;    // output of the forward, input of both backward passes
  const void* delta;  // rowsum(dout * out), input of both backward passes
  const void* mask;   // (batch, t_k) of the storage dtype, or nullptr
  void* out0;         // out / dq / dk
  void* out1;         // lse (forward) / dv (bwd_kv)
  int dtype;
  int64_t batch, t_q, t_k, hd, hd_v;
  bool causal;
  double scale;
  hipStream_t stream;
  void* out2 = nullptr;  // dv of the fused backward (out0 = dq, out1 = dk there)
};

enum SdpaPass { SDPA_FWD = 0, SDPA_BWD_Q = 1, SDPA_BWD_KV = 2 };

// MFMA flash kernels: bf16/f16, hd == hd_v in {64, 128}.
bool mfma_supports(int dtype, int64_t hd, int64_t hd_v);
bool mfma_fits(int64_t t_q, int64_t t_k, int64_t hd);
int launch_sdpa_mfma(SdpaPass pass, const SdpaArgs& a);
// one pass each, in its own translation unit (sdpa_mfma_fwd/bwd_q/bwd_kv.hip)
int launch_mfma_fwd(const SdpaArgs& a);
int launch_mfma_bwd_q(const SdpaArgs& a);
int launch_mfma_bwd_kv(const SdpaArgs& a);
// Both backward passes through the dS hand-off (sdpa_mfma_bwd.hip): the workspace bytes it needs
// for this call, 0 when the call has no such route (only D = 128 without a key mask, keys in whole
// 128-row blocks unless causal); and the launch, out0 = dq, out1 = dk, out2 = dv.
int64_t mfma_bwd_workspace(const SdpaArgs& a);
int launch_mfma_bwd(const SdpaArgs& a, void* ws, int passes);  // LIMN_HIP_BWD_* bits

// General-width kernels: any float dtype, max(hd, hd_v) <= 256.
bool rows_supports(int dtype, int64_t hd, int64_t hd_v);
int launch_sdpa_rows(SdpaPass pass, const SdpaArgs& a);

}  // namespace limn
