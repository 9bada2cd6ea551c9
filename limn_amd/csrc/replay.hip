// limn_hip_replay: launch a recorded plan's kernels from a pre-bound list (include/limn_hip.h).
//
// A plan the hip device has run before is recorded once as a list of steps (module kernel
// launches, the contraction and attention entry points, zero fills), each argument either a
// constant (a kernel's scratch pointer, a size) or an offset into one of the plan's buffers,
// named by slot. A replay binds the slots to this run's buffers and issues every step in order
// on one stream; nothing is looked up or rebuilt per launch.

#include <stdio.h>

#include "matmul.h"
#include "sdpa.h"

using namespace limn;

namespace {

constexpr int MAX_ARGS = 256;  // a merged launch of up to 16 nests takes at most a few dozen pointers

int64_t bound(const limn_hip_replay_arg& a, const int64_t* slots) { return a.slot < 0 ? a.value : slots[a.slot] + a.value; }

const void* ptr(const limn_hip_replay_arg& a, const int64_t* slots) { return (const void*)(intptr_t)bound(a, slots); }

int expect(const limn_hip_replay_step& s, int64_t i, int n, const char* what) {
  if (s.nargs == n) return LIMN_HIP_OK;
  return fail(LIMN_HIP_EINVAL, "replay step %lld: a %s step takes %d arguments, not %d", (long long)i, what, n, s.nargs);
}

int run_step(const limn_hip_replay_step& s, int64_t i, const limn_hip_replay_arg* a, const int64_t* slots, void* stream) {
  switch (s.kind) {
    case LIMN_HIP_STEP_KERNEL: {
      if (s.nargs < 0 || s.nargs > MAX_ARGS)
        return fail(LIMN_HIP_EINVAL, "replay step %lld: %d kernel arguments (at most %d)", (long long)i, s.nargs, MAX_ARGS);
      int64_t values[MAX_ARGS];
      void* params[MAX_ARGS];
      for (int k = 0; k < s.nargs; k++) {
        values[k] = bound(a[k], slots);
        params[k] = &values[k];
      }
      return check_hip(hipModuleLaunchKernel((hipFunction_t)s.function, (unsigned)s.grid, 1, 1, (unsigned)s.block, 1, 1, 0,
                                             (hipStream_t)stream, params, nullptr),
                       "launching a replayed kernel");
    }
    case LIMN_HIP_STEP_ZERO: {
      int rc = expect(s, i, 2, "zero");
      if (rc != LIMN_HIP_OK) return rc;
      return check_hip(hipMemsetAsync((void*)ptr(a[0], slots), 0, (size_t)bound(a[1], slots), (hipStream_t)stream),
                       "zeroing a replayed output");
    }
    case LIMN_HIP_STEP_MATMUL: {
      int rc = expect(s, i, 20, "matmul");
      if (rc != LIMN_HIP_OK) return rc;
      int64_t v[20];
      for (int k = 0; k < 20; k++) v[k] = bound(a[k], slots);
      return limn_hip_matmul((const void*)(intptr_t)v[0], (const void*)(intptr_t)v[1], (void*)(intptr_t)v[2], (int)v[3], v[4], v[5],
                             v[6], v[7], v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15], v[16], (int)v[17],
                             (void*)(intptr_t)v[18], v[19], stream);
    }
    case LIMN_HIP_STEP_SDPA_FWD: {
      int rc = expect(s, i, 13, "sdpa");
      if (rc != LIMN_HIP_OK) return rc;
      int64_t v[13];
      for (int k = 0; k < 13; k++) v[k] = bound(a[k], slots);
      return limn_hip_sdpa_fwd((const void*)(intptr_t)v[0], (const void*)(intptr_t)v[1], (const void*)(intptr_t)v[2],
                               (const void*)(intptr_t)v[3], (void*)(intptr_t)v[4], (void*)(intptr_t)v[5], (int)v[6], v[7], v[8],
                               v[9], v[10], v[11], (int)v[12], s.scale, stream);
    }
    case LIMN_HIP_STEP_SDPA_BWD_Q: {
      int rc = expect(s, i, 15, "sdpa_bwd_q");
      if (rc != LIMN_HIP_OK) return rc;
      int64_t v[15];
      for (int k = 0; k < 15; k++) v[k] = bound(a[k], slots);
      return limn_hip_sdpa_bwd_q((const void*)(intptr_t)v[0], (const void*)(intptr_t)v[1], (const void*)(intptr_t)v[2],
                                 (const void*)(intptr_t)v[3], (const void*)(intptr_t)v[4], (const void*)(intptr_t)v[5],
                                 (const void*)(intptr_t)v[6], (void*)(intptr_t)v[7], (int)v[8], v[9], v[10], v[11], v[12], v[13],
                                 (int)v[14], s.scale, stream);
    }
    case LIMN_HIP_STEP_SDPA_BWD_KV: {
      int rc = expect(s, i, 16, "sdpa_bwd_kv");
      if (rc != LIMN_HIP_OK) return rc;
      int64_t v[16];
      for (int k = 0; k < 16; k++) v[k] = bound(a[k], slots);
      return limn_hip_sdpa_bwd_kv((const void*)(intptr_t)v[0], (const void*)(intptr_t)v[1], (const void*)(intptr_t)v[2],
                                  (const void*)(intptr_t)v[3], (const void*)(intptr_t)v[4], (const void*)(intptr_t)v[5],
                                  (const void*)(intptr_t)v[6], (void*)(intptr_t)v[7], (void*)(intptr_t)v[8], (int)v[9], v[10],
                                  v[11], v[12], v[13], v[14], (int)v[15], s.scale, stream);
    }
    default:
      return fail(LIMN_HIP_EINVAL, "replay step %lld: unknown kind %d", (long long)i, s.kind);
  }
}

}  // namespace

extern "C" int limn_hip_replay(const limn_hip_replay_step* steps, int64_t nsteps, const limn_hip_replay_arg* args,
                               int64_t nargs, const int64_t* slots, int64_t nslots, void* stream) {
  if (nsteps < 0 || nargs < 0 || nslots < 0 || (nsteps > 0 && (steps == nullptr || args == nullptr)))
    return fail(LIMN_HIP_EINVAL, "replay: bad step or argument list");
  for (int64_t i = 0; i < nsteps; i++) {
    const limn_hip_replay_step& s = steps[i];
    if (s.first < 0 || s.nargs < 0 || s.first + s.nargs > nargs)
      return fail(LIMN_HIP_EINVAL, "replay step %lld: arguments [%lld, %lld) outside the list of %lld", (long long)i,
                  (long long)s.first, (long long)(s.first + s.nargs), (long long)nargs);
    for (int k = 0; k < s.nargs; k++) {
      const int32_t slot = args[s.first + k].slot;
      if (slot >= nslots) return fail(LIMN_HIP_EINVAL, "replay step %lld: slot %d of %lld", (long long)i, slot, (long long)nslots);
    }
    const int rc = run_step(s, i, args + s.first, slots, stream);
    if (rc != LIMN_HIP_OK) return rc;
  }
  return LIMN_HIP_OK;
}
