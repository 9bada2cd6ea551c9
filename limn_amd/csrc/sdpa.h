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
};

enum SdpaPass { SDPA_FWD = 0, SDPA_BWD_Q = 1, SDPA_BWD_KV = 2 };

// MFMA flash kernels: bf16/f16, hd == hd_v in {64, 128}.
bool mfma_supports(int dtype, int64_t hd, int64_t hd_v);
bool mfma_fits(int64_t t_q, int64_t t_k, int64_t hd);
int launch_sdpa_mfma(SdpaPass pass, const SdpaArgs& a);

// General-width kernels: any float dtype, max(hd, hd_v) <= 256.
bool rows_supports(int dtype, int64_t hd, int64_t hd_v);
int launch_sdpa_rows(SdpaPass pass, const SdpaArgs& a);

}  // namespace limn
