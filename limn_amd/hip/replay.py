"""Pre-bound launch lists: a plan's launches recorded once, replayed by one native call.

The executor runs a plan call by call, and each call's runner rebuilds its launch arguments in
Python (reference `limn/jit.py:159-184`; capture replays through the same `run`,
`limn/capture.py:152-179`). A training step is hundreds of launches, so that host work is
milliseconds per step. The hip device instead records a hot plan's launches once, during an
ordinary run with every buffer of the run kept alive: each launch becomes a step of
`limn_hip_replay` (include/limn_hip.h) and each argument either a constant (a size, a kernel's
own scratch pointer) or an offset into a *slot*: a buffer position of the plan (its sources) or
one of the outputs the run allocated, in call order. A replay takes its outputs from one arena
(fixed offsets in one allocation the list keeps, reused once nothing inside it is referenced, so
the same few bindings recur run after run), binds every
slot to this run's buffer and issues the whole list in one call: as a HIP graph captured for that
binding (one capture serves every later run with the same buffers, and the launches cost the host
one call), or launch by launch.

A recording is refused (the plan keeps running call by call) when two slots share bytes, since a
pointer into them could not be told apart.
"""

from __future__ import annotations

import bisect
import ctypes
from dataclasses import dataclass, field

import numpy as np

(STEP_KERNEL, STEP_ZERO, STEP_MATMUL, STEP_SDPA_FWD, STEP_SDPA_BWD_Q, STEP_SDPA_BWD_KV, STEP_MATMUL_ADD,
 STEP_SDPA_BWD) = range(8)

# which arguments of each step kind are device pointers (the rest are sizes, codes and flags)
POINTER_ARGS = {
    STEP_ZERO: frozenset({0}),
    STEP_MATMUL: frozenset({0, 1, 2, 18}),
    STEP_MATMUL_ADD: frozenset({0, 1, 2, 18, 21, 25}),
    STEP_SDPA_FWD: frozenset(range(6)),
    STEP_SDPA_BWD_Q: frozenset(range(8)),
    STEP_SDPA_BWD_KV: frozenset(range(9)),
    STEP_SDPA_BWD: frozenset(range(10)) | {18},
}

ARG = np.dtype([("value", np.int64), ("slot", np.int32), ("reserved", np.int32)])
STEP = np.dtype([("kind", np.int32), ("nargs", np.int32), ("first", np.int64), ("function", np.uint64),
                 ("grid", np.int32), ("block", np.int32), ("scale", np.float64)])
assert ARG.itemsize == 16 and STEP.itemsize == 40


@dataclass(frozen=True)
class Launch:
    """One recorded launch: its kind, module function (kernels), grid and block, sdpa scale, and
    its arguments as the recording run passed them."""

    kind: int
    args: tuple[int, ...]
    function: int = 0
    grid: int = 0
    block: int = 0
    scale: float = 0.0


@dataclass
class Program:
    steps: np.ndarray
    args: np.ndarray
    out_nbytes: tuple[int, ...]  # the outputs a replay allocates, in call order
    out_positions: tuple[tuple[int, int], ...]  # (output index, plan position) of outputs the plan reads
    assigns: tuple[tuple[int, int], ...]  # (target position, output index) committed after the list
    positions: int  # slots [0, positions) are the plan's buffer positions, then the outputs
    arena_offsets: tuple[int, ...] = ()  # each output's byte offset in the replay's one allocation
    arena_bytes: int = 0
    # captured graphs by binding (slot values), the most recently used last; a training loop that
    # keeps the previous step's result alive while it runs the next alternates two bindings
    graphs: dict[bytes, ctypes.c_void_p] = field(default_factory=dict)
    captures: int = 0  # graphs captured
    arenas: list = field(default_factory=list)  # the device's Arena objects for this list's outputs
    staging: dict = field(default_factory=dict)  # plan position -> the buffer host bytes are copied to
    graph_failure: str | None = None  # why this list stopped using graphs, once it has

    @property
    def nslots(self) -> int:
        return self.positions + len(self.out_nbytes)

    def launch(self, lib, slots: np.ndarray, stream=None) -> int:
        return lib.limn_hip_replay(self.steps.ctypes.data, len(self.steps), self.args.ctypes.data, len(self.args),
                                   slots.ctypes.data, len(slots), stream)

    def launch_graph(self, lib, slots: np.ndarray, finish) -> int:
        """The list as one graph launch on the null stream: the graph captured for this binding,
        or a new capture (the least recently used of GRAPHS_PER_PLAN dropped first, after
        `finish()` has waited for its launches)."""
        key = slots.tobytes()
        handle = self.graphs.pop(key, None)
        if handle is None:
            if len(self.graphs) >= GRAPHS_PER_PLAN:
                finish()
                lib.limn_hip_replay_graph_free(self.graphs.pop(next(iter(self.graphs))))
            handle = ctypes.c_void_p()
            self.captures += 1
        self.graphs[key] = handle
        return lib.limn_hip_replay_graph(self.steps.ctypes.data, len(self.steps), self.args.ctypes.data, len(self.args),
                                         slots.ctypes.data, len(slots), ctypes.byref(handle))

    def run(self, lib, slots: np.ndarray, finish, graphs: bool) -> int:
        """Issue the list for this binding: as a captured graph when `graphs` is set and no graph
        of this list has failed, else launch by launch. A capture, instantiation or graph launch
        that fails does so before any step runs (and the steps only write this replay's own
        outputs), so the list then runs launch by launch, and keeps doing so: its graphs are
        released and the reason kept in `graph_failure`. A list that cannot run launch by launch
        either returns that status."""
        if graphs and self.graph_failure is None:
            status = self.launch_graph(lib, slots, finish)
            if status == 0:
                return 0
            self.graph_failure = lib.limn_hip_last_error().decode() or f"status {status}"
            finish()
            self.release(lib)
        return self.launch(lib, slots)

    def release(self, lib) -> None:
        """Free the captured graphs (after the device has finished every launch of them)."""
        for handle in self.graphs.values():
            if handle.value:
                lib.limn_hip_replay_graph_free(handle)
        self.graphs.clear()


GRAPHS_PER_PLAN = 8
PLANS_KEPT = 64  # launch lists a device keeps, the least recently run dropped first
ARENAS_PER_PLAN = 3  # a list keeps this many output arenas; past that a replay takes a passing one
ARENA_ALIGN = 256  # bytes between the starts of a replay's outputs in its arena


def arena_layout(out_nbytes) -> tuple[tuple[int, ...], int]:
    """Byte offsets of a replay's outputs in one allocation, and its size."""
    offsets, at = [], 0
    for nb in out_nbytes:
        offsets.append(at)
        at += -(-max(nb, 1) // ARENA_ALIGN) * ARENA_ALIGN
    return tuple(offsets), max(at, 1)


def bind(tape: list[Launch], slots: list[tuple[int, int, int]]) -> tuple[np.ndarray, np.ndarray] | None:
    """The recorded launches as (steps, args) arrays. `slots` holds (slot, device pointer, bytes)
    for every buffer of the recording run; a pointer argument inside one becomes that slot plus an
    offset, any other is kept as it is. None when two slots overlap."""
    spans = sorted((ptr, ptr + max(nb, 1), slot) for slot, ptr, nb in slots)
    starts = [s for s, _, _ in spans]
    if any(a[1] > b[0] for a, b in zip(spans, spans[1:])):
        return None
    steps = np.zeros(len(tape), dtype=STEP)
    rows: list[tuple[int, int, int]] = []
    for i, launch in enumerate(tape):
        pointers = POINTER_ARGS.get(launch.kind)
        steps[i] = (launch.kind, len(launch.args), len(rows), launch.function, launch.grid, launch.block, launch.scale)
        for k, value in enumerate(launch.args):
            value = int(value or 0)
            slot = -1
            if (pointers is None or k in pointers) and value:
                j = bisect.bisect_right(starts, value) - 1
                if j >= 0 and value < spans[j][1]:
                    slot, value = spans[j][2], value - spans[j][0]
            rows.append((value, slot, 0))
    return steps, np.array(rows, dtype=ARG) if rows else np.zeros(1, dtype=ARG)
