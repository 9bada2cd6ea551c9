"""The `hip` device: limn's CompiledDevice on one MI355X (gfx950).

It is what reference `limn/backend_cuda.py:272-415` (`CudaDevice`) is for NVIDIA, designed for
this GPU rather than translated:

- memory is hipMalloc'd device buffers recycled through a per-size pool (a training step
  retires one output per kernel; hipMalloc/hipFree per call would dominate it);
- lowered loop nests are rendered by limn_amd/hip/emit.py into gfx950 kernels, compiled by
  hipRTC once per program and launched with hipModuleLaunchKernel on the null stream;
- the CUSTOM attention kernels `sdpa`, `sdpa_bwd_q` and `sdpa_bwd_kv` are the hand-written
  MFMA/LDS kernels of liblimn_hip.so, reached through its C ABI (include/limn_hip.h);
- host arrays handed in are uploaded per batch (`prepare`), and an ASSIGN whose target is a host
  array is written back (`commit`), as the reference device does;
- `finish()` synchronizes once per batch, which pins an asynchronous failure to its batch.
"""

from __future__ import annotations

import collections
import ctypes
import dataclasses
import math
import time
from typing import Any

import numpy as np

from limn_amd.dtypes import ABI_CODE
from limn_amd.hip import replay, runtime
from limn_amd.hip.runtime import DEVICE_TO_DEVICE, DEVICE_TO_HOST, HOST_TO_DEVICE, check, check_limn
from limn_amd.seam import FLOATS, CompiledDevice, LoopNest, Node, Op, Runner, accumulate_in, realized

Buffer = Any

SDPA, SDPA_BWD_Q, SDPA_BWD_KV = "sdpa", "sdpa_bwd_q", "sdpa_bwd_kv"
BWD_BOTH = 3  # LIMN_HIP_BWD_BOTH: limn_hip_sdpa_bwd runs both passes


# One workgroup per table entry (value, target, bytes <= 64 KiB, 16-byte aligned starts): 16-byte
# copies, then the entry's tail byte by byte.
COMMIT_SOURCE = r"""
extern "C" __global__ void limn_commit_batch(const long long* __restrict__ table, long long entries) {
  const long long e = blockIdx.x;
  if (e >= entries) return;
  const char* src = (const char*)table[3 * e];
  char* dst = (char*)table[3 * e + 1];
  const long long n = table[3 * e + 2], whole = n / 16;
  for (long long i = threadIdx.x; i < whole; i += blockDim.x) ((uint4*)dst)[i] = ((const uint4*)src)[i];
  for (long long i = whole * 16 + threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
}
"""


def plan_context(order: list[Node], sinks: list[Node]) -> tuple[set, set]:
    """(kept, custom_inputs) of one plan for the emitter: the nodes whose buffers must hold their
    values (every sink, every CUSTOM src), and the CUSTOM srcs alone."""
    custom_inputs = {realized(src) for n in order if n.op is Op.CUSTOM for src in n.srcs}
    return {realized(s) for s in sinks} | custom_inputs, custom_inputs


class HipBuffer:
    """Device bytes; the pointer returns to its device's pool when the last reference drops."""

    __slots__ = ("ptr", "nbytes", "pool")

    def __init__(self, ptr: int, nbytes: int, pool: dict[int, list[int]]):
        self.ptr = ptr
        self.nbytes = nbytes
        self.pool = pool

    def __del__(self) -> None:
        try:
            self.pool.setdefault(self.nbytes, []).append(self.ptr)
        except Exception:  # interpreter teardown
            pass


class Arena:
    """One allocation holding every output of a replay, kept by its launch list for later
    replays; `live` counts the buffers handed out inside it that are still referenced."""

    __slots__ = ("buf", "live")

    def __init__(self, buf: HipBuffer):
        self.buf = buf
        self.live = 0


class ArenaBuffer:
    """Bytes inside a replay's arena. The arena is free for another replay once every buffer
    inside it has dropped (later launches are ordered after the earlier ones on the stream)."""

    __slots__ = ("ptr", "nbytes", "arena")

    def __init__(self, ptr: int, nbytes: int, arena: Arena):
        self.ptr = ptr
        self.nbytes = nbytes
        self.arena = arena
        arena.live += 1

    def __del__(self) -> None:
        self.arena.live -= 1


class HipDevice(CompiledDevice):
    """Construct through set_device("hip"), which checks the runtime and the GPU first."""

    def __init__(self) -> None:
        self.plan_kept: set | None = None  # set by plan_of for runners(), see there
        self.plan_custom_inputs: set | None = None
        super().__init__()
        api = runtime.hip()
        assert api is not None, "construct via set_device('hip'), which explains what is missing"
        self.api = api
        self.lib = runtime.kernels()
        check(api.hipInit(0), "hipInit")
        check(api.hipSetDevice(0), "selecting device 0")
        arch = ctypes.create_string_buffer(256)
        cus, clock = ctypes.c_int(), ctypes.c_int()
        mem = ctypes.c_int64()
        check_limn(self.lib.limn_hip_device_info(0, arch, 256, ctypes.byref(cus), ctypes.byref(clock), ctypes.byref(mem)))
        self.arch = arch.value.decode()
        self.compute_units = cus.value
        self.clock_khz = clock.value
        self.global_mem = mem.value
        self.pool: dict[int, list[int]] = {}
        # ASSIGN commits to device buffers, queued until finish() copies them in one launch
        self._commits: list[tuple[Buffer, Buffer]] = []
        self._commit_targets: set[int] = set()
        self._committed: list[tuple[Buffer, Buffer]] = []  # launched, kept alive until the barrier
        self._commit_table: tuple[int, int, Buffer] | None = None  # (pinned host ptr, entries, device copy)
        self.custom[SDPA] = self._sdpa_runner
        self.custom[SDPA_BWD_Q] = self._sdpa_runner
        self.custom[SDPA_BWD_KV] = self._sdpa_runner
        # pre-bound launch lists: id(plan) -> [plan, Program or None, refused], least recently
        # run first, at most replay.PLANS_KEPT; `tape` collects the launches of the run that
        # records one (every launch site appends while it is set)
        self.replays: collections.OrderedDict[int, list] = collections.OrderedDict()
        self.replay_graphs = True  # replay through a captured graph (False: launch by launch)
        self.tape: list[replay.Launch] | None = None
        self.issue_seconds = 0.0  # host time replayed runs spent before their barrier, summed

    # ---- Device protocol ----

    def _alloc(self, nb: int) -> HipBuffer:
        free = self.pool.get(nb)
        if free:
            return HipBuffer(free.pop(), nb, self.pool)
        ptr = ctypes.c_void_p()
        status = self.api.hipMalloc(ctypes.byref(ptr), max(nb, 1))
        if status != 0 and self.pool:
            self.trim()
            status = self.api.hipMalloc(ctypes.byref(ptr), max(nb, 1))
        check(status, f"allocating {nb} bytes")
        return HipBuffer(ptr.value, nb, self.pool)

    def trim(self) -> None:
        """Give every pooled buffer, and every launch list's idle arenas, back to the runtime."""
        self.finish()
        for entry in self.replays.values():
            if entry[1] is not None:
                entry[1].arenas = [a for a in entry[1].arenas if a.live]
        for ptrs in self.pool.values():
            for ptr in ptrs:
                self.api.hipFree(ctypes.c_void_p(ptr))
        self.pool.clear()

    def alloc(self, nbytes: int) -> Buffer:
        return self.out_alloc(nbytes, zero=True)

    def copyin(self, buf: Buffer, array: np.ndarray) -> None:
        data = np.ascontiguousarray(array)
        if data.nbytes != buf.nbytes:
            raise ValueError(f"copyin: {data.nbytes} bytes into a {buf.nbytes}-byte buffer")
        check(self.api.hipMemcpy(ctypes.c_void_p(buf.ptr), data.ctypes.data_as(ctypes.c_void_p), data.nbytes, HOST_TO_DEVICE), "uploading bytes")

    def copyout(self, buf: Buffer) -> np.ndarray:
        out = np.empty(buf.nbytes, dtype=np.uint8)
        check(self.api.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(buf.ptr), buf.nbytes, DEVICE_TO_HOST), "downloading bytes")
        return out

    # ---- CompiledDevice hooks ----

    def prepare(self, buf: Buffer) -> Buffer:
        if isinstance(buf, np.ndarray):  # a tensor whose bytes live on the host
            moved = self._alloc(buf.nbytes)
            self.copyin(moved, buf)
            return moved
        return buf

    def out_alloc(self, nb: int, zero: bool) -> Buffer:
        buf = self._alloc(nb)
        if zero:
            check(self.api.hipMemsetAsync(ctypes.c_void_p(buf.ptr), 0, nb, None), "zeroing an allocation")
            if self.tape is not None:
                self.tape.append(replay.Launch(replay.STEP_ZERO, (buf.ptr, nb)))
        return buf

    # ---- execution: hot plans replay from a pre-bound launch list ----

    def run(self, plan, sources):
        """The executor's transaction (every call, then the commits, then one barrier), issued
        one of three ways: a plan's first run call by call; its second also records every launch
        into a launch list (replay.py); later runs allocate fresh outputs, bind them and the
        sources to the list's slots and launch it in one native call, as a graph captured for
        that binding unless `replay_graphs` is off. Results and commits are the same either way;
        a recording whose buffers overlap is refused and the plan keeps running call by call."""
        entry = self.replays.get(id(plan))
        if entry is None or entry[0] is not plan:
            if entry is not None:  # a dead plan's id, reused
                self._drop_replay(id(plan))
            self.replays[id(plan)] = [plan, None, False]
            while len(self.replays) > replay.PLANS_KEPT:
                self._drop_replay(next(iter(self.replays)))
            return super().run(plan, sources)
        self.replays.move_to_end(id(plan))
        if entry[1] is not None:
            return self._replay(plan, entry[1], sources)
        if entry[2]:
            return super().run(plan, sources)
        return self._record(plan, sources, entry)

    def _drop_replay(self, key: int) -> None:
        """Forget one plan's launch list: its graphs are released once the device has finished
        their launches; its arenas and staging buffers go back to the pool as their last
        references drop (a result still held keeps its arena)."""
        entry = self.replays.pop(key)
        if entry[1] is not None:
            self.finish()
            entry[1].release(self.lib)

    def _record(self, plan, sources, entry: list):
        bufs: list = [None] * plan.positions
        slots: list[tuple[int, int, int]] = []
        for p, buf in sources.items():
            bufs[p] = self.prepare(buf)
            slots.append((p, bufs[p].ptr, bufs[p].nbytes))
        outs_all: list = []  # every output of the run, kept alive so no two share bytes
        out_positions: list[tuple[int, int]] = []
        assigns: list[tuple[int, int]] = []
        self.tape = tape = []
        try:
            for call in plan.calls:
                outs = [self.out_alloc(nb, call.zero_fill) for nb in call.out_nbytes]
                base = len(outs_all)
                outs_all += outs
                call.fn([bufs[p] for p in call.inputs], outs)
                for j, (p, out) in enumerate(zip(call.outputs, outs)):
                    if p is not None:
                        bufs[p] = out
                        out_positions.append((base + j, p))
                if call.assign_target is not None:
                    assigns.append((call.assign_target, base))
        finally:
            self.tape = None
        for p, i in assigns:
            self.commit(sources[p], outs_all[i])
            bufs[p] = outs_all[i]
        self.finish()
        slots += [(plan.positions + i, out.ptr, out.nbytes) for i, out in enumerate(outs_all)]
        bound = replay.bind(tape, slots)
        if bound is None:
            entry[2] = True
        else:
            nbytes = tuple(o.nbytes for o in outs_all)
            offsets, total = replay.arena_layout(nbytes)
            entry[1] = replay.Program(bound[0], bound[1], nbytes, tuple(out_positions), tuple(assigns), plan.positions,
                                      offsets, total)
        return [bufs[p] for p in plan.sinks]

    def _replay(self, plan, prog: "replay.Program", sources):
        start = time.perf_counter()
        bufs: list = [None] * plan.positions
        slots = np.zeros(prog.nslots, dtype=np.int64)
        sinks = set(plan.sinks)
        for p, buf in sources.items():
            if isinstance(buf, np.ndarray) and p not in sinks:
                # host bytes go to the list's own buffer for this position (the copy waits for
                # the launches before it), so a loop feeding host batches binds the same buffers
                staged = prog.staging.get(p)
                if staged is None or staged.nbytes != buf.nbytes:
                    staged = prog.staging[p] = self._alloc(buf.nbytes)
                self.copyin(staged, buf)
                bufs[p] = staged
            else:
                bufs[p] = self.prepare(buf)
            slots[p] = bufs[p].ptr
        # the list's own arenas, one not in use: the same few bindings recur step after step
        # whatever else the pool hands out between them (zero fills are steps of the list)
        arena = next((a for a in prog.arenas if a.live == 0), None)
        if arena is None:
            arena = Arena(self._alloc(prog.arena_bytes))
            if len(prog.arenas) < replay.ARENAS_PER_PLAN:
                prog.arenas.append(arena)
        outs = [ArenaBuffer(arena.buf.ptr + off, nb, arena) for off, nb in zip(prog.arena_offsets, prog.out_nbytes)]
        del arena
        for i, out in enumerate(outs):
            slots[prog.positions + i] = out.ptr
        for i, p in prog.out_positions:
            bufs[p] = outs[i]
        check_limn(prog.run(self.lib, slots, self.finish, self.replay_graphs))
        for p, i in prog.assigns:
            self.commit(sources[p], outs[i])
            bufs[p] = outs[i]
        self._flush_commits()
        self.issue_seconds += time.perf_counter() - start
        self.finish()
        return [bufs[p] for p in plan.sinks]

    def commit(self, target: Buffer, value: Buffer) -> None:
        """A device target's copy is queued: finish() runs every commit of the batch as one kernel
        (a training step commits hundreds of parameters and moments, one launch each otherwise;
        reference limn/backend_cuda.py:343-347 issues a cuMemcpyDtoD per commit). A host target is
        written at once."""
        if isinstance(target, np.ndarray):
            check(self.api.hipMemcpy(target.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(value.ptr), target.nbytes, DEVICE_TO_HOST), "committing an assign to host")
            return
        if target.ptr in self._commit_targets:
            self._flush_commits()  # a second commit to one target in a batch: the later one wins
        self._commits.append((target, value))
        self._commit_targets.add(target.ptr)

    COMMIT_CHUNK = 1 << 16  # bytes per workgroup of the commit kernel

    def _flush_commits(self) -> None:
        """Launch the queued commits as one kernel over a (value, target, bytes) table. The queue is
        taken first, so an allocation failure below (whose trim() finishes the batch) finds
        nothing left to flush; a grown table is allocated before the old one is released."""
        if not self._commits:
            return
        commits, self._commits, self._commit_targets = self._commits, [], set()
        entries = []
        for target, value in commits:
            for off in range(0, value.nbytes, self.COMMIT_CHUNK):
                entries.append((value.ptr + off, target.ptr + off, min(self.COMMIT_CHUNK, value.nbytes - off)))
        if self._committed:
            # the pinned table of an earlier launch in this batch may not have been read yet
            check(self.api.hipStreamSynchronize(None), "waiting for a commit table")
        table = np.array(entries, dtype=np.int64)
        host, cap, dev_table = self._commit_table or (0, 0, None)
        if cap < len(entries):
            cap = max(len(entries), 2 * cap, 1024)
            grown = self._alloc(cap * 24)
            ptr = ctypes.c_void_p()
            check(self.api.hipHostMalloc(ctypes.byref(ptr), cap * 24, 0), "allocating a pinned commit table")
            if host:
                check(self.api.hipStreamSynchronize(None), "waiting for a commit table")
                self.api.hipHostFree(ctypes.c_void_p(host))
            host, dev_table = ptr.value, grown
            self._commit_table = (host, cap, dev_table)
        ctypes.memmove(host, table.ctypes.data, table.nbytes)
        check(self.api.hipMemcpyAsync(ctypes.c_void_p(dev_table.ptr), ctypes.c_void_p(host), table.nbytes, HOST_TO_DEVICE, None), "uploading a commit table")
        fn = runtime.load_functions(COMMIT_SOURCE, ["limn_commit_batch"])["limn_commit_batch"]
        args = (ctypes.c_void_p * 2)(ctypes.c_void_p(dev_table.ptr), ctypes.c_void_p(len(entries)))
        params = (ctypes.c_void_p * 2)(*[ctypes.addressof(args) + k * ctypes.sizeof(ctypes.c_void_p) for k in range(2)])
        check(self.api.hipModuleLaunchKernel(fn, len(entries), 1, 1, 256, 1, 1, 0, None, params, None), "launching the commits")
        self._committed += commits

    def finish(self) -> None:
        self._flush_commits()
        check(self.api.hipDeviceSynchronize(), "waiting for the batch")
        self._committed = []

    def plan_of(self, order: list[Node], position: dict[Node, int], sinks: list[Node]):
        """The executor's plan_of, with the buffers that must hold their values recorded for
        runners(): the sinks and every CUSTOM src. runners() sees only the non-CUSTOM nests, and
        a contraction's epilogue may absorb a relu nest only when no one else reads the sum."""
        self.plan_kept, self.plan_custom_inputs = plan_context(order, sinks)
        try:
            plan = super().plan_of(order, position, sinks)
        finally:
            self.plan_kept = None
            self.plan_custom_inputs = None
        return self._pair_backward(plan)

    # the most workspace one backward pair may hold for its dS hand-off
    SDPA_HANDOFF_CAP = 8 << 30

    def _pair_backward(self, plan):
        """Run each sdpa_bwd_q call and the sdpa_bwd_kv call on the same inputs and params as one
        call (limn_hip_sdpa_bwd), at the first one's place: both read only those inputs, so every
        one is ready there. Through one call the dK/dV pass hands its dS to the dQ pass instead of
        the dQ pass recomputing it. Pairs whose call has no hand-off route stay as they are."""
        calls = list(plan.calls)
        tags = [getattr(c.fn, "sdpa_pair", None) for c in calls]
        drop: set[int] = set()
        for i, tag in enumerate(tags):
            if tag is None or tag[0] != SDPA_BWD_Q or i in drop:
                continue
            j = next((j for j, other in enumerate(tags) if other is not None and other[0] == SDPA_BWD_KV
                      and other[1] == tag[1] and calls[j].inputs == calls[i].inputs and j not in drop), None)
            if j is None:
                continue
            fused = tag[2]()
            if fused is None:
                continue
            q_call, kv_call = calls[i], calls[j]
            first = min(i, j)
            calls[first] = dataclasses.replace(q_call, fn=fused, outputs=q_call.outputs + kv_call.outputs,
                                               out_nbytes=q_call.out_nbytes + kv_call.out_nbytes)
            drop.add(max(i, j))
        if not drop:
            return plan
        return dataclasses.replace(plan, calls=tuple(c for k, c in enumerate(calls) if k not in drop))

    def runners(self, nests: list[LoopNest]) -> list[Runner]:
        from limn_amd.hip.emit import nest_runners

        return nest_runners(self, nests)

    # ---- fused attention ----

    def _sdpa_runner(self, node: Node) -> Runner:
        """The three CUSTOM attention kernels, bound to liblimn_hip.so's entry points.

        srcs are (q, k, v[, mask]) for the forward and (q, k, v, dout, lse, delta[, mask]) for
        both backward passes, contiguous, with shared leading (batch) dims; a mask rides last
        (reference `limn/tensor.py:562-567, 707-712`). Shapes are checked here, at plan time.
        """
        name = node.arg.name
        causal, scale = node.arg.params
        q, k, v = node.srcs[:3]
        base = 3 if name == SDPA else 6
        masked = len(node.srcs) == base + 1
        if len(node.srcs) not in (base, base + 1):
            raise ValueError(f"{name}: expected {base} or {base + 1} srcs, got {len(node.srcs)}")
        dtype = q.dtype
        if dtype not in FLOATS or dtype not in ABI_CODE:
            raise NotImplementedError(f"{name}: no kernel for dtype {dtype}")
        if any(s.dtype != dtype for s in (k, v)) or (masked and node.srcs[-1].dtype != dtype):
            raise ValueError(f"{name}: q, k, v and the mask must share a dtype")
        if len(q.shape) < 2 or len(k.shape) != len(q.shape) or len(v.shape) != len(q.shape):
            raise ValueError(f"{name} wants 2D+ inputs of equal rank, got {q.shape}, {k.shape}, {v.shape}")
        lead = q.shape[:-2]
        if k.shape[:-2] != lead or v.shape[:-2] != lead or k.shape[-2] != v.shape[-2] or q.shape[-1] != k.shape[-1]:
            raise ValueError(f"{name} shape mismatch: {q.shape}, {k.shape}, {v.shape}")
        batch, t_q, hd = math.prod(lead), q.shape[-2], q.shape[-1]
        t_k, hd_v = k.shape[-2], v.shape[-1]
        if causal and t_q != t_k:
            raise ValueError(f"causal {name} needs square keys, got {t_q} queries and {t_k} keys")
        if masked and node.srcs[-1].shape != lead + (t_k,):
            raise ValueError(f"{name} key mask must be {lead + (t_k,)}, got {node.srcs[-1].shape}")
        if name != SDPA:
            stat = accumulate_in(dtype)
            do, lse, delta = node.srcs[3:6]
            if do.shape != lead + (t_q, hd_v) or do.dtype != dtype:
                raise ValueError(f"{name}: dout must be {lead + (t_q, hd_v)} {dtype}, got {do.shape} {do.dtype}")
            for stat_node, what in ((lse, "lse"), (delta, "delta")):
                if stat_node.dtype != stat or math.prod(stat_node.shape) != batch * t_q:
                    raise ValueError(f"{name}: {what} must hold {batch * t_q} {stat} values")
        code = ABI_CODE[dtype]
        if self.lib.limn_hip_sdpa_path(code, hd, hd_v) < 0:
            raise NotImplementedError(f"{name}: no kernel for head dims {hd} and {hd_v}")
        lib, sizes = self.lib, (batch, t_q, t_k, hd, hd_v, int(bool(causal)), float(scale), None)

        ints, scale_f = sizes[:6], sizes[6]

        def call(kind: int, entry, args: tuple) -> None:
            check_limn(entry(*args, code, *sizes))
            if self.tape is not None:
                self.tape.append(replay.Launch(kind, (*args, code, *ints), scale=scale_f))

        if name == SDPA:

            def run(inputs: list[Buffer], outs: list[Buffer]) -> None:
                mask = inputs[3].ptr if masked else None
                call(replay.STEP_SDPA_FWD, lib.limn_hip_sdpa_fwd, (inputs[0].ptr, inputs[1].ptr, inputs[2].ptr, mask, outs[0].ptr, outs[1].ptr))

        elif name == SDPA_BWD_Q:

            def run(inputs: list[Buffer], outs: list[Buffer]) -> None:
                mask = inputs[6].ptr if masked else None
                call(replay.STEP_SDPA_BWD_Q, lib.limn_hip_sdpa_bwd_q, (*[b.ptr for b in inputs[:6]], mask, outs[0].ptr))

        elif name == SDPA_BWD_KV:

            def run(inputs: list[Buffer], outs: list[Buffer]) -> None:
                mask = inputs[6].ptr if masked else None
                call(replay.STEP_SDPA_BWD_KV, lib.limn_hip_sdpa_bwd_kv, (*[b.ptr for b in inputs[:6]], mask, outs[0].ptr, outs[1].ptr))

        else:
            raise NotImplementedError(f"HipDevice has no kernel for custom op {name!r}")
        if name != SDPA:
            # plan_of pairs the two backward calls of one attention through this tag (_pair_backward)
            run.sdpa_pair = (name, (code, *ints, scale_f, masked), lambda: self._fused_backward(code, ints, scale_f, masked))
        return run

    def _fused_backward(self, code: int, ints: tuple, scale: float, masked: bool) -> Runner | None:
        """The runner of a paired backward call (outputs dq, dk, dv) through limn_hip_sdpa_bwd, or
        None when the call has no dS hand-off route or its workspace would pass SDPA_HANDOFF_CAP.
        The workspace is allocated on the first run and kept with the runner, so a replayed or
        graph-captured list sees the same pointer every time."""
        lib = self.lib
        need = int(lib.limn_hip_sdpa_bwd_workspace(code, *ints, int(masked)))
        if need <= 0 or need > self.SDPA_HANDOFF_CAP:
            return None
        held: list = []

        def run(inputs: list[Buffer], outs: list[Buffer]) -> None:
            if not held:
                held.append(self._alloc(need))
            ws = held[0]
            mask = inputs[6].ptr if masked else None
            args = (*[b.ptr for b in inputs[:6]], mask, outs[0].ptr, outs[1].ptr, outs[2].ptr, code, *ints)
            check_limn(lib.limn_hip_sdpa_bwd(*args, scale, BWD_BOTH, ws.ptr, ws.nbytes, None))
            if self.tape is not None:
                self.tape.append(replay.Launch(replay.STEP_SDPA_BWD, (*args, BWD_BOTH, ws.ptr, ws.nbytes), scale=scale))

        return run
