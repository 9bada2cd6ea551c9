// limn_hip_replay: launch a recorded plan's kernels from a pre-bound list (include/limn_hip.h).
//
// A plan the hip device has run before is recorded once as a list of steps (module kernel
// launches, the contraction and attention entry points, zero fills), each argument either a
// constant (a kernel's scratch pointer, a size) or an offset into one of the plan's buffers,
// named by slot. A replay binds the slots to this run's buffers and issues every step in order
// on one stream; nothing is looked up or rebuilt per launch.

#include <stdio.h>

#include <vector>

#include "matmul.h"
#include "sdpa.h"

using namespace limn;

namespace {

constexpr int MAX_ARGS = 512;  // a merged launch takes at most 400 pointers (the emitter's MERGE_PARAMS)

// A zero fill as a kernel rather than hipMemsetAsync, so the list can be captured into a graph
// (memset nodes of captured graphs have given wrong results on replays after the first): 16-byte
// stores over the aligned body, single bytes at the ends.
__global__ __launch_bounds__(256) void zero_bytes(unsigned char* __restrict__ p, int64_t n) {
  const int64_t head = ((16 - ((uintptr_t)p & 15)) & 15) < n ? (16 - ((uintptr_t)p & 15)) & 15 : n;
  const int64_t chunks = (n - head) / 16, tail = n - head - chunks * 16;
  uint4* body = (uint4*)(p + head);
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * 256)
    body[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0 && threadIdx.x < head) p[threadIdx.x] = 0;
  if (blockIdx.x == 0 && threadIdx.x < tail) p[head + chunks * 16 + threadIdx.x] = 0;
}

int zero_fill(void* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return LIMN_HIP_OK;
  const int64_t blocks = (n / 16 + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 1 ? 1 : blocks > 4096 ? 4096 : blocks);
  hipLaunchKernelGGL(zero_bytes, dim3(grid), dim3(256), 0, stream, (unsigned char*)p, n);
  return check_hip(hipGetLastError(), "launching a replayed zero fill");
}

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
      return zero_fill((void*)ptr(a[0], slots), bound(a[1], slots), (hipStream_t)stream);
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
    case LIMN_HIP_STEP_MATMUL_ADD: {
      int rc = expect(s, i, 27, "matmul_add");
      if (rc != LIMN_HIP_OK) return rc;
      int64_t v[27];
      for (int k = 0; k < 27; k++) v[k] = bound(a[k], slots);
      return limn_hip_matmul_add((const void*)(intptr_t)v[0], (const void*)(intptr_t)v[1], (void*)(intptr_t)v[2], (int)v[3],
                                 v[4], v[5], v[6], v[7], v[8], v[9], v[10], v[11], v[12], v[13], v[14], v[15], v[16],
                                 (int)v[17], (const void*)(intptr_t)v[18], (int)v[19], v[20], (const void*)(intptr_t)v[21],
                                 v[22], v[23], v[24], (void*)(intptr_t)v[25], v[26], stream);
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
    case LIMN_HIP_STEP_SDPA_BWD: {
      int rc = expect(s, i, 20, "sdpa_bwd");
      if (rc != LIMN_HIP_OK) return rc;
      int64_t v[20];
      for (int k = 0; k < 20; k++) v[k] = bound(a[k], slots);
      return limn_hip_sdpa_bwd((const void*)(intptr_t)v[0], (const void*)(intptr_t)v[1], (const void*)(intptr_t)v[2],
                               (const void*)(intptr_t)v[3], (const void*)(intptr_t)v[4], (const void*)(intptr_t)v[5],
                               (const void*)(intptr_t)v[6], (void*)(intptr_t)v[7], (void*)(intptr_t)v[8], (void*)(intptr_t)v[9],
                               (int)v[10], v[11], v[12], v[13], v[14], v[15], (int)v[16], s.scale, (int)v[17], (void*)(intptr_t)v[18],
                               v[19], stream);
    }
    default:
      return fail(LIMN_HIP_EINVAL, "replay step %lld: unknown kind %d", (long long)i, s.kind);
  }
}

int check_list(const limn_hip_replay_step* steps, int64_t nsteps, const limn_hip_replay_arg* args, int64_t nargs,
               const int64_t* slots, int64_t nslots) {
  if (nsteps < 0 || nargs < 0 || nslots < 0 || (nsteps > 0 && (steps == nullptr || args == nullptr)) ||
      (nslots > 0 && slots == nullptr))
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
  }
  return LIMN_HIP_OK;
}

int run_list(const limn_hip_replay_step* steps, int64_t nsteps, const limn_hip_replay_arg* args, const int64_t* slots,
             void* stream) {
  for (int64_t i = 0; i < nsteps; i++) {
    const int rc = run_step(steps[i], i, args + steps[i].first, slots, stream);
    if (rc != LIMN_HIP_OK) return rc;
  }
  return LIMN_HIP_OK;
}

// A list captured as a graph and the binding it was captured with.
struct ReplayGraph {
  hipGraphExec_t exec = nullptr;
  const limn_hip_replay_step* steps = nullptr;
  const limn_hip_replay_arg* args = nullptr;
  int64_t nsteps = 0, nargs = 0;
  std::vector<int64_t> slots;

  void drop_exec() {
    if (exec != nullptr) hipGraphExecDestroy(exec);
    exec = nullptr;
  }

  ~ReplayGraph() { drop_exec(); }

  bool matches(const limn_hip_replay_step* s, int64_t ns, const limn_hip_replay_arg* a, int64_t na, const int64_t* sl,
               int64_t nsl) const {
    if (exec == nullptr || s != steps || ns != nsteps || a != args || na != nargs || (int64_t)slots.size() != nsl) return false;
    for (int64_t i = 0; i < nsl; i++)
      if (slots[(size_t)i] != sl[i]) return false;
    return true;
  }

  // The steps recorded (not run) on a stream made for the capture: non-blocking, so the capture
  // never meets the null stream's implicit synchronisation.
  int capture(const limn_hip_replay_step* s, int64_t ns, const limn_hip_replay_arg* a, int64_t na, const int64_t* sl,
              int64_t nsl) {
    drop_exec();
    hipStream_t stream = nullptr;
    int rc = check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "creating a capture stream");
    if (rc != LIMN_HIP_OK) return rc;
    rc = check_hip(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "starting a replay capture");
    if (rc == LIMN_HIP_OK) {
      const int listed = run_list(s, ns, a, sl, stream);
      hipGraph_t graph = nullptr;
      rc = check_hip(hipStreamEndCapture(stream, &graph), "ending a replay capture");
      if (listed != LIMN_HIP_OK) rc = listed;
      if (rc == LIMN_HIP_OK) rc = check_hip(hipGraphInstantiateWithFlags(&exec, graph, 0), "instantiating a replay graph");
      if (graph != nullptr) hipGraphDestroy(graph);
    }
    hipStreamDestroy(stream);
    if (rc != LIMN_HIP_OK) {
      exec = nullptr;
      return rc;
    }
    steps = s;
    nsteps = ns;
    args = a;
    nargs = na;
    slots.assign(sl, sl + nsl);
    return LIMN_HIP_OK;
  }
};

}  // namespace

extern "C" int limn_hip_replay(const limn_hip_replay_step* steps, int64_t nsteps, const limn_hip_replay_arg* args,
                               int64_t nargs, const int64_t* slots, int64_t nslots, void* stream) {
  const int rc = check_list(steps, nsteps, args, nargs, slots, nslots);
  if (rc != LIMN_HIP_OK) return rc;
  return run_list(steps, nsteps, args, slots, stream);
}

extern "C" int limn_hip_replay_graph(const limn_hip_replay_step* steps, int64_t nsteps, const limn_hip_replay_arg* args,
                                     int64_t nargs, const int64_t* slots, int64_t nslots, void** handle) {
  if (handle == nullptr) return fail(LIMN_HIP_EINVAL, "replay_graph: no handle");
  int rc = check_list(steps, nsteps, args, nargs, slots, nslots);
  if (rc != LIMN_HIP_OK) return rc;
  ReplayGraph* g = (ReplayGraph*)*handle;
  if (g == nullptr) *handle = g = new ReplayGraph();
  if (!g->matches(steps, nsteps, args, nargs, slots, nslots)) {
    rc = g->capture(steps, nsteps, args, nargs, slots, nslots);
    if (rc != LIMN_HIP_OK) return rc;
  }
  // on the null stream, ordered as the steps themselves would be there
  return check_hip(hipGraphLaunch(g->exec, nullptr), "launching a replay graph");
}

extern "C" int limn_hip_replay_graph_free(void* handle) {
  delete (ReplayGraph*)handle;
  return LIMN_HIP_OK;
}
