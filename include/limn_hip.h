/*
 * limn_hip.h - the C ABI of limn's MI355X (gfx950) `hip` device: hand-written CDNA4 kernels
 * behind plain pointers and sizes.
 *
 * limn reaches its GPU kernels through ctypes (reference limn/backend_cuda.py:54-151 binds the
 * CUDA driver and NVRTC the same way). The generated loop-nest kernels go through hipRTC and
 * hipModuleLaunchKernel directly; the three fused-attention CUSTOM kernels and the dense
 * contraction are hand-written and exported here.
 *
 * Conventions for every entry point:
 *  - pointers are device pointers (hipMalloc'd), row-major and contiguous;
 *  - `dtype` is one of LIMN_HIP_FLOAT64/FLOAT32/FLOAT16/BFLOAT16 and names the storage type of
 *    q, k, v, dout, key_mask and the outputs; the per-row statistics (lse, delta) are float32
 *    when dtype is a half width and dtype itself otherwise (limn's accumulate_in);
 *  - `key_mask` may be NULL; else it is (batch, t_k) of `dtype`, and a zero hides that key;
 *  - launches are asynchronous on `stream` (NULL = the null stream); return 0 on success, else
 *    a LIMN_HIP_E* code, with a message from limn_hip_last_error() (thread-local).
 */
#ifndef LIMN_HIP_H
#define LIMN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LIMN_HIP_ABI_VERSION 3

enum {
  LIMN_HIP_FLOAT64 = 0,
  LIMN_HIP_FLOAT32 = 1,
  LIMN_HIP_FLOAT16 = 2,
  LIMN_HIP_BFLOAT16 = 3,
};

enum {
  LIMN_HIP_OK = 0,
  LIMN_HIP_EINVAL = 1,       /* arguments that describe no valid call (limn raises ValueError) */
  LIMN_HIP_EUNSUPPORTED = 2, /* a valid call this library has no kernel for (NotImplementedError) */
  LIMN_HIP_ERUNTIME = 3,     /* the HIP runtime refused (RuntimeError) */
};

/* Which ABI this library speaks: LIMN_HIP_ABI_VERSION at build time. */
int limn_hip_abi_version(void);

/* The message of the last failed call on this thread ("" if none). */
const char* limn_hip_last_error(void);

/* Properties of HIP device `device` that the limn device checks and reports: its gcn arch
 * name (e.g. "gfx950:sramecc+:xnack-") into arch[arch_len], compute-unit count, peak clock in
 * kHz and global memory in bytes. Replaces the capability queries of reference
 * limn/backend_cuda.py:253-293 (pick_arch, cuDeviceGetAttribute). */
int limn_hip_device_info(int device, char* arch, int arch_len, int* compute_units, int* clock_khz,
                         int64_t* global_mem);

/* Which kernel family serves an sdpa call of this shape: 1 = MFMA flash kernels, 0 = the
 * general-width kernels (any float dtype, any head dims up to 256), -1 = none. */
int limn_hip_sdpa_path(int dtype, int64_t hd, int64_t hd_v);

/*
 * Fused attention forward: out = softmax(q k^T * scale [causal: key j <= query i] [key_mask]) v
 * and lse = the per-row logsumexp of the masked scaled scores.
 *   q (batch, t_q, hd), k (batch, t_k, hd), v (batch, t_k, hd_v) -> out (batch, t_q, hd_v),
 *   lse (batch, t_q). A row with every key hidden gives NaN and lse = -inf.
 * Replaces the CUSTOM "sdpa" kernel of reference limn/cuda_emit.py:921-965, launched by
 * limn/backend_cuda.py:352-361 (_sdpa_runner); numpy reference limn/sdpa.py:91-137.
 */
int limn_hip_sdpa_fwd(const void* q, const void* k, const void* v, const void* key_mask, void* out, void* lse, int dtype,
                      int64_t batch, int64_t t_q, int64_t t_k, int64_t hd, int64_t hd_v, int causal, double scale,
                      void* stream);

/*
 * dQ of fused attention, from p = exp(s*scale - lse) and ds = p (dout v^T - delta) scale:
 *   dq (batch, t_q, hd) = sum over keys of ds k. delta (batch, t_q) is rowsum(dout * out).
 * Replaces CUSTOM "sdpa_bwd_q", reference limn/cuda_emit.py:968-1005; numpy reference
 * limn/sdpa.py:140-170.
 */
int limn_hip_sdpa_bwd_q(const void* q, const void* k, const void* v, const void* dout, const void* lse, const void* delta,
                        const void* key_mask, void* dq, int dtype, int64_t batch, int64_t t_q, int64_t t_k, int64_t hd,
                        int64_t hd_v, int causal, double scale, void* stream);

/*
 * dK and dV of fused attention in one pass over queries: dv = sum_i p dout_i, dk = sum_i ds q_i.
 * A hidden key gets zero rows. Replaces CUSTOM "sdpa_bwd_kv", reference
 * limn/cuda_emit.py:1008-1083; numpy reference limn/sdpa.py:173-203.
 */
int limn_hip_sdpa_bwd_kv(const void* q, const void* k, const void* v, const void* dout, const void* lse, const void* delta,
                         const void* key_mask, void* dk, void* dv, int dtype, int64_t batch, int64_t t_q, int64_t t_k,
                         int64_t hd, int64_t hd_v, int causal, double scale, void* stream);

/*
 * Both backward kernels of fused attention in one call: dq as limn_hip_sdpa_bwd_q defines it, dk
 * and dv as limn_hip_sdpa_bwd_kv does. limn's backward issues them as two CUSTOM calls on the same
 * inputs (reference limn/tensor.py:707-712: "sdpa_bwd_q", "sdpa_bwd_kv"; kernels
 * limn/cuda_emit.py:968-1083); the device runs such a pair as this one call. Given a workspace
 * of limn_hip_sdpa_bwd_workspace(...) bytes, the dK/dV pass hands the dS it computes (2 bytes per
 * (query, key) pair it visits) to the dQ pass through the workspace, and the dQ pass reads it
 * instead of recomputing S, dP and the softmax; without one (null, smaller, or a call with no such
 * route) the two passes run as the separate entry points run them. dq may differ between the two
 * routes in rounding; each route is deterministic. `passes` is LIMN_HIP_BWD_BOTH for callers;
 * LIMN_HIP_BWD_KV_PASS and LIMN_HIP_BWD_Q_PASS run one pass each (the dQ pass reads the dS the
 * dK/dV pass of an earlier call on the same workspace left there), so a harness can time each.
 */
enum { LIMN_HIP_BWD_KV_PASS = 1, LIMN_HIP_BWD_Q_PASS = 2, LIMN_HIP_BWD_BOTH = 3 };
int limn_hip_sdpa_bwd(const void* q, const void* k, const void* v, const void* dout, const void* lse, const void* delta,
                      const void* key_mask, void* dq, void* dk, void* dv, int dtype, int64_t batch, int64_t t_q, int64_t t_k,
                      int64_t hd, int64_t hd_v, int causal, double scale, int passes, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* Workspace bytes limn_hip_sdpa_bwd hands dS through for such a call (masked: a key mask is
 * given); 0 when the call has no such route (today: bf16/f16 at hd == hd_v == 128 without a key
 * mask, and keys in whole 128-row blocks unless causal). No counterpart in the reference. */
int64_t limn_hip_sdpa_bwd_workspace(int dtype, int64_t batch, int64_t t_q, int64_t t_k, int64_t hd, int64_t hd_v, int causal,
                                    int masked);

/*
 * Dense contraction on matrix cores: c[b, m, n] = epilogue(sum_k a[b, m, k] * b[b, k, n]), bf16 or
 * f16 operands and result, f32 accumulation. Strides are in elements; each operand must be
 * contiguous along k or along its row (m / n) with the other stride a multiple of 8.
 * epilogue: 0 = none, 1 = relu before the store. Replaces the tiled SIMT matmul the reference
 * emits for a dense contraction nest, limn/cuda_emit.py:376-685 (matmul_shape, emit_tiled).
 * A contraction with too few output tiles to fill the GPU and a long k (a weight gradient: a sum
 * over every batch row) splits k: float32 partial tiles go to `workspace` and a second kernel adds
 * them in a fixed order, so results are deterministic. `workspace` must hold
 * limn_hip_matmul_workspace(...) bytes for that; with a null or smaller workspace the
 * contraction runs unsplit (same result, slower).
 */
int limn_hip_matmul(const void* a, const void* b, void* c, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                    int64_t a_batch, int64_t a_m, int64_t a_k, int64_t b_batch, int64_t b_k, int64_t b_n, int64_t c_batch,
                    int64_t c_m, int64_t c_n, int epilogue, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * limn_hip_matmul with terms added at the store: out[b, m, n] = T(residual[b, m, n] +
 * (T(epilogue(sum)) + T(bias[n]))), computed in float with T the rounding to the output type, either
 * term left out when its pointer is null (bias[n] at bias + n * bias_n, of type bias_dtype: the
 * output's, or LIMN_HIP_FLOAT32 for a float32 bias rounded to the output type first, as a cast
 * would; the residual of the output type at r_batch, r_m, r_n element strides). This is an elementwise reader of the contraction that adds a bias vector
 * (and a residual), which the device evaluates in the contraction's store instead of a launch of
 * its own: the reference emits such a reader as a separate kernel (limn/cuda_emit.py:287-372,
 * emit_elementwise, after the contraction's emit_tiled). Same workspace rules as limn_hip_matmul.
 */
int limn_hip_matmul_add(const void* a, const void* b, void* c, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                        int64_t a_batch, int64_t a_m, int64_t a_k, int64_t b_batch, int64_t b_k, int64_t b_n,
                        int64_t c_batch, int64_t c_m, int64_t c_n, int epilogue, const void* bias, int bias_dtype,
                        int64_t bias_n, const void* residual, int64_t r_batch, int64_t r_m, int64_t r_n,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of workspace limn_hip_matmul uses to split k for this shape; 0 when it does not split. No
 * counterpart in the reference (its contraction kernel never splits). */
int64_t limn_hip_matmul_workspace(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K);

/*
 * limn_hip_matmul without a caller workspace and without allocating: the split-k slices (see
 * above) go to a static device array of LIMN_HIP_SCRATCH_BYTES, one per GPU, held until the process
 * ends. For callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc); no counterpart in the reference. Results equal
 * limn_hip_matmul's with a large enough workspace, bit for bit. Refuses (LIMN_HIP_EINVAL) a
 * contraction whose slices need more than LIMN_HIP_SCRATCH_BYTES (limn_hip_matmul_workspace says
 * how much). Every call on one GPU shares that GPU's array: calls that overlap on one GPU (on two
 * streams, or from two threads) race on it and must be ordered by the caller.
 */
#define LIMN_HIP_SCRATCH_BYTES (128ll << 20)
int limn_hip_matmul_noalloc(const void* a, const void* b, void* c, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                            int64_t a_batch, int64_t a_m, int64_t a_k, int64_t b_batch, int64_t b_k, int64_t b_n,
                            int64_t c_batch, int64_t c_m, int64_t c_n, int epilogue, void* stream);

/* 1 when limn_hip_matmul has a kernel for this dtype and operand layout, else 0 (the device
 * then keeps the contraction on the general reduce kernels). */
int limn_hip_matmul_supported(int dtype, int64_t M, int64_t N, int64_t K, int64_t a_batch, int64_t a_m, int64_t a_k,
                              int64_t b_batch, int64_t b_k, int64_t b_n);

/*
 * A pre-bound launch list: the kernels of one recorded execution of a plan, replayed against new
 * buffers. Each step is one launch: a hipRTC module kernel (`function`, `grid` x `block`
 * threads, its arguments the kernel's parameters in order), a zero fill (pointer, bytes), or one
 * call of limn_hip_matmul (its 20 arguments before `stream`), limn_hip_matmul_add (27),
 * limn_hip_sdpa_fwd (13 before
 * `scale`), limn_hip_sdpa_bwd_q (15), limn_hip_sdpa_bwd_kv (16) or limn_hip_sdpa_bwd (17 before
 * `scale`, then passes, workspace and its size: 20), with `scale` in the step. An
 * argument is `value` when `slot` < 0, else slots[slot] + value: a byte offset into the buffer
 * this replay binds to that slot. Steps run in order on `stream`; the first failing one stops the
 * list and its status is returned. No counterpart in the reference: its capture replays a plan
 * by calling every kernel's runner again (limn/capture.py:152-179).
 */
enum {
  LIMN_HIP_STEP_KERNEL = 0,
  LIMN_HIP_STEP_ZERO = 1,
  LIMN_HIP_STEP_MATMUL = 2,
  LIMN_HIP_STEP_SDPA_FWD = 3,
  LIMN_HIP_STEP_SDPA_BWD_Q = 4,
  LIMN_HIP_STEP_SDPA_BWD_KV = 5,
  LIMN_HIP_STEP_MATMUL_ADD = 6,
  LIMN_HIP_STEP_SDPA_BWD = 7,
};

typedef struct {
  int64_t value;
  int32_t slot;
  int32_t reserved;
} limn_hip_replay_arg;

typedef struct {
  int32_t kind;
  int32_t nargs;
  int64_t first; /* this step's arguments are args[first .. first + nargs) */
  void* function;
  int32_t grid;
  int32_t block;
  double scale;
} limn_hip_replay_step;

int limn_hip_replay(const limn_hip_replay_step* steps, int64_t nsteps, const limn_hip_replay_arg* args, int64_t nargs,
                    const int64_t* slots, int64_t nslots, void* stream);

/*
 * The same list issued as a HIP graph on the null stream: the first call captures the steps,
 * bound to `slots`, into a graph (recorded on a stream made for the capture, not run) and
 * instantiates it; a later call with the same list and the same slot values launches the
 * instantiated graph (one call for every launch of the list), and one with other slots captures
 * again. `*handle` is NULL before the first call; limn_hip_replay_graph_free releases it, once no
 * launch of it is pending. No counterpart in the reference (limn/capture.py:152-179 replays
 * through every runner); for callers that replay one plan many times with the same buffers, such
 * as a training loop.
 */
int limn_hip_replay_graph(const limn_hip_replay_step* steps, int64_t nsteps, const limn_hip_replay_arg* args,
                          int64_t nargs, const int64_t* slots, int64_t nslots, void** handle);
int limn_hip_replay_graph_free(void* handle);

#ifdef __cplusplus
}
#endif

#endif /* LIMN_HIP_H */
