// The C ABI declared in include/limn_hip.h: argument checks, kernel-family dispatch, errors.

#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "matmul.h"
#include "sdpa.h"

namespace limn {

static thread_local char last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(last_error, sizeof last_error, fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(last_error, sizeof last_error, fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t err, const char* doing) {
  if (err == hipSuccess) return LIMN_HIP_OK;
  return fail(LIMN_HIP_ERUNTIME, "hip: %s: %s", doing, hipGetErrorString(err));
}

static const char* pass_name(SdpaPass pass) {
  return pass == SDPA_FWD ? "sdpa" : pass == SDPA_BWD_Q ? "sdpa_bwd_q" : "sdpa_bwd_kv";
}

// The same shape rules as the numpy reference's _validate (reference limn/sdpa.py:64-75),
// on the flattened (batch, t, d) form the device hands over.
static int validate(SdpaPass pass, const SdpaArgs& a) {
  const char* name = pass_name(pass);
  if (a.dtype < LIMN_HIP_FLOAT64 || a.dtype > LIMN_HIP_BFLOAT16)
    return fail(LIMN_HIP_EUNSUPPORTED, "%s: dtype code %d is not a float dtype", name, a.dtype);
  if (a.batch < 1 || a.t_q < 1 || a.t_k < 1 || a.hd < 1 || a.hd_v < 1)
    return fail(LIMN_HIP_EINVAL, "%s: sizes must be positive (batch %lld, t_q %lld, t_k %lld, hd %lld, hd_v %lld)", name,
                (long long)a.batch, (long long)a.t_q, (long long)a.t_k, (long long)a.hd, (long long)a.hd_v);
  if (a.causal && a.t_q != a.t_k)
    return fail(LIMN_HIP_EINVAL, "%s: causal attention needs square keys, got %lld queries and %lld keys", name,
                (long long)a.t_q, (long long)a.t_k);
  if (!isfinite(a.scale)) return fail(LIMN_HIP_EINVAL, "%s: scale must be finite", name);
  if (a.q == nullptr || a.k == nullptr || a.v == nullptr || a.out0 == nullptr)
    return fail(LIMN_HIP_EINVAL, "%s: null buffer", name);
  if (pass == SDPA_FWD && a.out1 == nullptr) return fail(LIMN_HIP_EINVAL, "%s: null lse buffer", name);
  if (pass != SDPA_FWD && (a.dout == nullptr || a.lse == nullptr || a.delta == nullptr))
    return fail(LIMN_HIP_EINVAL, "%s: null dout/lse/delta buffer", name);
  if (pass == SDPA_BWD_KV && a.out1 == nullptr) return fail(LIMN_HIP_EINVAL, "%s: null dv buffer", name);
  const int64_t limit = (int64_t)1 << 40;  // element counts far past any allocation; keeps index math in range
  if (a.t_q > limit / a.batch || a.t_k > limit / a.batch || a.hd > 4096 || a.hd_v > 4096)
    return fail(LIMN_HIP_EUNSUPPORTED, "%s: sizes out of range", name);
  return LIMN_HIP_OK;
}

static int run(SdpaPass pass, const SdpaArgs& a) {
  const int rc = validate(pass, a);
  if (rc != LIMN_HIP_OK) return rc;
  // the MFMA forward keeps each row's running max over raw scores, which orders the scaled scores
  // only for a positive scale; the backward passes use the saved L and take any scale
  const bool mfma_scale = pass != SDPA_FWD || a.scale > 0;
  if (mfma_supports(a.dtype, a.hd, a.hd_v) && mfma_fits(a.t_q, a.t_k, a.hd) && mfma_scale) return launch_sdpa_mfma(pass, a);
  if (rows_supports(a.dtype, a.hd, a.hd_v)) return launch_sdpa_rows(pass, a);
  return fail(LIMN_HIP_EUNSUPPORTED, "%s: no kernel for head dims %lld and %lld (at most 256)", pass_name(pass),
              (long long)a.hd, (long long)a.hd_v);
}

// The argument rules both matmul entry points apply before launching anything.
static int check_matmul(const char* name, const void* a, const void* b, const void* c, int dtype, const MatmulShape& s,
                        int epilogue) {
  if (dtype != LIMN_HIP_BFLOAT16 && dtype != LIMN_HIP_FLOAT16)
    return fail(LIMN_HIP_EUNSUPPORTED, "%s: the MFMA contraction takes bfloat16 or float16, not dtype code %d", name, dtype);
  if (s.batch < 1 || s.M < 1 || s.N < 1 || s.K < 1)
    return fail(LIMN_HIP_EINVAL, "%s: sizes must be positive (batch %lld, M %lld, N %lld, K %lld)", name,
                (long long)s.batch, (long long)s.M, (long long)s.N, (long long)s.K);
  if (a == nullptr || b == nullptr || c == nullptr) return fail(LIMN_HIP_EINVAL, "%s: null buffer", name);
  if (epilogue != MATMUL_EPILOGUE_NONE && epilogue != MATMUL_EPILOGUE_RELU)
    return fail(LIMN_HIP_EINVAL, "%s: unknown epilogue %d", name, epilogue);
  if (!matmul_layout_ok(s))
    return fail(LIMN_HIP_EUNSUPPORTED, "%s: operands must be contiguous along m/n or k with 16-byte aligned rows", name);
  if (((uintptr_t)a | (uintptr_t)b) % 16 != 0) return fail(LIMN_HIP_EUNSUPPORTED, "%s: operands must be 16-byte aligned", name);
  return LIMN_HIP_OK;
}

// The split-k scratch of limn_hip_matmul_noalloc: a static device array, one copy per GPU, held
// until the process ends. In host code `scratch` names a host-side stand-in, not device memory:
// its device address is looked up once per device (hipGetSymbolAddress, that device current)
// and only that address is handed to kernels.
__device__ __align__(256) unsigned char scratch[LIMN_HIP_SCRATCH_BYTES];

constexpr int SCRATCH_DEVICES = 64;
static void* scratch_at[SCRATCH_DEVICES];
static std::mutex scratch_lock;

static int scratch_address(void** out) {
  int device = -1;
  int rc = check_hip(hipGetDevice(&device), "reading the current device");
  if (rc != LIMN_HIP_OK) return rc;
  if (device < 0 || device >= SCRATCH_DEVICES)
    return fail(LIMN_HIP_EUNSUPPORTED, "matmul_noalloc: device %d is past the %d devices the scratch table holds", device,
                SCRATCH_DEVICES);
  std::lock_guard<std::mutex> hold(scratch_lock);
  if (scratch_at[device] == nullptr) {
    void* found = nullptr;
    rc = check_hip(hipGetSymbolAddress(&found, HIP_SYMBOL(scratch)), "finding the static matmul scratch");
    if (rc != LIMN_HIP_OK) return rc;
    scratch_at[device] = found;
  }
  *out = scratch_at[device];
  return LIMN_HIP_OK;
}

}  // namespace limn

using namespace limn;

extern "C" {

int limn_hip_abi_version(void) { return LIMN_HIP_ABI_VERSION; }

const char* limn_hip_last_error(void) { return last_error; }

int limn_hip_device_info(int device, char* arch, int arch_len, int* compute_units, int* clock_khz, int64_t* global_mem) {
  hipDeviceProp_t prop;
  const int rc = check_hip(hipGetDeviceProperties(&prop, device), "reading device properties");
  if (rc != LIMN_HIP_OK) return rc;
  if (arch != nullptr && arch_len > 0) snprintf(arch, (size_t)arch_len, "%s", prop.gcnArchName);
  if (compute_units != nullptr) *compute_units = prop.multiProcessorCount;
  if (clock_khz != nullptr) *clock_khz = prop.clockRate;
  if (global_mem != nullptr) *global_mem = (int64_t)prop.totalGlobalMem;
  return LIMN_HIP_OK;
}

int limn_hip_sdpa_path(int dtype, int64_t hd, int64_t hd_v) {
  if (mfma_supports(dtype, hd, hd_v)) return 1;
  if (rows_supports(dtype, hd, hd_v)) return 0;
  return -1;
}

int limn_hip_sdpa_fwd(const void* q, const void* k, const void* v, const void* key_mask, void* out, void* lse, int dtype,
                      int64_t batch, int64_t t_q, int64_t t_k, int64_t hd, int64_t hd_v, int causal, double scale,
                      void* stream) {
  SdpaArgs a = {q,     k,   v,    nullptr, nullptr, nullptr, key_mask, out,    lse,      dtype,
                batch, t_q, t_k,  hd,      hd_v,    causal != 0, scale, (hipStream_t)stream};
  return run(SDPA_FWD, a);
}

int limn_hip_sdpa_bwd_q(const void* q, const void* k, const void* v, const void* dout, const void* lse, const void* delta,
                        const void* key_mask, void* dq, int dtype, int64_t batch, int64_t t_q, int64_t t_k, int64_t hd,
                        int64_t hd_v, int causal, double scale, void* stream) {
  SdpaArgs a = {q,     k,   v,   dout, lse,  delta,       key_mask, dq,   nullptr, dtype,
                batch, t_q, t_k, hd,   hd_v, causal != 0, scale,    (hipStream_t)stream};
  return run(SDPA_BWD_Q, a);
}

int limn_hip_sdpa_bwd_kv(const void* q, const void* k, const void* v, const void* dout, const void* lse, const void* delta,
                         const void* key_mask, void* dk, void* dv, int dtype, int64_t batch, int64_t t_q, int64_t t_k,
                         int64_t hd, int64_t hd_v, int causal, double scale, void* stream) {
  SdpaArgs a = {q,     k,   v,   dout, lse,  delta,       key_mask, dk,   dv, dtype,
                batch, t_q, t_k, hd,   hd_v, causal != 0, scale,    (hipStream_t)stream};
  return run(SDPA_BWD_KV, a);
}

int64_t limn_hip_sdpa_bwd_workspace(int dtype, int64_t batch, int64_t t_q, int64_t t_k, int64_t hd, int64_t hd_v, int causal,
                                    int masked) {
  static const char one = 0;  // a stand-in key mask: only its presence matters here
  SdpaArgs a = {nullptr, nullptr, nullptr, nullptr,     nullptr, nullptr, masked ? &one : nullptr, nullptr, nullptr, dtype,
                batch,   t_q,     t_k,     hd,          hd_v,    causal != 0, 1.0, nullptr};
  if (batch < 1 || t_q < 1 || t_k < 1 || (causal && t_q != t_k)) return 0;
  return mfma_bwd_workspace(a);
}

int limn_hip_sdpa_bwd(const void* q, const void* k, const void* v, const void* dout, const void* lse, const void* delta,
                      const void* key_mask, void* dq, void* dk, void* dv, int dtype, int64_t batch, int64_t t_q, int64_t t_k,
                      int64_t hd, int64_t hd_v, int causal, double scale, int passes, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  SdpaArgs a = {q,     k,   v,   dout, lse,  delta,       key_mask, dq,   dk, dtype,
                batch, t_q, t_k, hd,   hd_v, causal != 0, scale,    (hipStream_t)stream};
  a.out2 = dv;
  int rc = validate(SDPA_BWD_Q, a);
  if (rc != LIMN_HIP_OK) return rc;
  if (dk == nullptr || dv == nullptr) return fail(LIMN_HIP_EINVAL, "sdpa_bwd: null dk/dv buffer");
  if (workspace_bytes < 0) return fail(LIMN_HIP_EINVAL, "sdpa_bwd: negative workspace size");
  if (passes < LIMN_HIP_BWD_KV_PASS || passes > LIMN_HIP_BWD_BOTH) return fail(LIMN_HIP_EINVAL, "sdpa_bwd: passes must be 1, 2 or 3");
  const int64_t need = mfma_bwd_workspace(a);
  if (need > 0 && workspace != nullptr && workspace_bytes >= need) return launch_mfma_bwd(a, workspace, passes);
  // no hand-off: the two passes as their own entry points run them
  SdpaArgs kv = a;
  kv.out0 = dk;
  kv.out1 = dv;
  rc = passes & LIMN_HIP_BWD_Q_PASS ? run(SDPA_BWD_Q, a) : LIMN_HIP_OK;
  return rc != LIMN_HIP_OK || !(passes & LIMN_HIP_BWD_KV_PASS) ? rc : run(SDPA_BWD_KV, kv);
}

int limn_hip_matmul(const void* a, const void* b, void* c, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                    int64_t a_batch, int64_t a_m, int64_t a_k, int64_t b_batch, int64_t b_k, int64_t b_n, int64_t c_batch,
                    int64_t c_m, int64_t c_n, int epilogue, void* workspace, int64_t workspace_bytes, void* stream) {
  MatmulShape s = {batch, M, N, K, a_batch, a_m, a_k, b_batch, b_k, b_n, c_batch, c_m, c_n};
  const int rc = check_matmul("matmul", a, b, c, dtype, s, epilogue);
  if (rc != LIMN_HIP_OK) return rc;
  if (workspace_bytes < 0) return fail(LIMN_HIP_EINVAL, "matmul: negative workspace size");
  return launch_matmul(a, b, c, dtype, s, epilogue, MatmulAddends{}, workspace, workspace_bytes, (hipStream_t)stream);
}

int limn_hip_matmul_add(const void* a, const void* b, void* c, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                        int64_t a_batch, int64_t a_m, int64_t a_k, int64_t b_batch, int64_t b_k, int64_t b_n,
                        int64_t c_batch, int64_t c_m, int64_t c_n, int epilogue, const void* bias, int bias_dtype,
                        int64_t bias_n, const void* residual, int64_t r_batch, int64_t r_m, int64_t r_n,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  MatmulShape s = {batch, M, N, K, a_batch, a_m, a_k, b_batch, b_k, b_n, c_batch, c_m, c_n};
  const int rc = check_matmul("matmul_add", a, b, c, dtype, s, epilogue);
  if (rc != LIMN_HIP_OK) return rc;
  if (workspace_bytes < 0) return fail(LIMN_HIP_EINVAL, "matmul_add: negative workspace size");
  if (bias != nullptr && bias_dtype != dtype && bias_dtype != LIMN_HIP_FLOAT32)
    return fail(LIMN_HIP_EINVAL, "matmul_add: the bias is of the output type or float32, not dtype %d", bias_dtype);
  const int f32 = bias != nullptr && bias_dtype == LIMN_HIP_FLOAT32;
  if ((uintptr_t)bias % (f32 ? 4 : 2) != 0 || (uintptr_t)residual % 2 != 0)
    return fail(LIMN_HIP_EINVAL, "matmul_add: the bias and residual must be aligned to their element size");
  MatmulAddends add = {bias, f32, bias_n, (const u16*)residual, r_batch, r_m, r_n, 0};
  if (bias != nullptr && bias_n == 1 && (uintptr_t)bias % 16 == 0) add.vec |= 1;
  if (residual != nullptr && r_n == 1 && r_m % 8 == 0 && r_batch % 8 == 0 && (uintptr_t)residual % 16 == 0) add.vec |= 2;
  return launch_matmul(a, b, c, dtype, s, epilogue, add, workspace, workspace_bytes, (hipStream_t)stream);
}

int limn_hip_matmul_noalloc(const void* a, const void* b, void* c, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                            int64_t a_batch, int64_t a_m, int64_t a_k, int64_t b_batch, int64_t b_k, int64_t b_n,
                            int64_t c_batch, int64_t c_m, int64_t c_n, int epilogue, void* stream) {
  MatmulShape s = {batch, M, N, K, a_batch, a_m, a_k, b_batch, b_k, b_n, c_batch, c_m, c_n};
  int rc = check_matmul("matmul_noalloc", a, b, c, dtype, s, epilogue);
  if (rc != LIMN_HIP_OK) return rc;
  const int64_t need = matmul_workspace_bytes(s);
  if (need > (int64_t)LIMN_HIP_SCRATCH_BYTES)
    return fail(LIMN_HIP_EINVAL,
                "matmul_noalloc: this contraction splits k into slices that need %lld bytes of scratch, more than the "
                "%lld-byte static scratch; call limn_hip_matmul with a workspace instead",
                (long long)need, (long long)LIMN_HIP_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0 && (rc = scratch_address(&ws)) != LIMN_HIP_OK) return rc;
  return launch_matmul(a, b, c, dtype, s, epilogue, MatmulAddends{}, ws, need, (hipStream_t)stream);
}

int64_t limn_hip_matmul_workspace(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K) {
  if ((dtype != LIMN_HIP_BFLOAT16 && dtype != LIMN_HIP_FLOAT16) || batch < 1 || M < 1 || N < 1 || K < 1) return 0;
  MatmulShape s = {batch, M, N, K, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  return matmul_workspace_bytes(s);
}

int limn_hip_matmul_supported(int dtype, int64_t M, int64_t N, int64_t K, int64_t a_batch, int64_t a_m, int64_t a_k,
                              int64_t b_batch, int64_t b_k, int64_t b_n) {
  MatmulShape s = {1, M, N, K, a_batch, a_m, a_k, b_batch, b_k, b_n, 0, 0, 0};
  return (dtype == LIMN_HIP_BFLOAT16 || dtype == LIMN_HIP_FLOAT16) && M > 0 && N > 0 && K > 0 && matmul_layout_ok(s);
}

}  // extern "C"
