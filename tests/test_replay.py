"""Pre-bound launch lists (limn_amd/hip/replay.py) without a GPU: how a recorded launch's
arguments bind to slots, the refusals, the fall back from graphs, and the bound on kept lists."""

from __future__ import annotations

import collections
import ctypes

import numpy as np

from limn_amd.hip import replay


def test_pointers_bind_to_slots_and_offsets():
    slots = [(0, 0x1000, 256), (1, 0x2000, 64), (5, 0x9000, 1)]
    tape = [
        replay.Launch(replay.STEP_KERNEL, (0x1000, 0x2010, 0x5000), function=7, grid=3, block=64),
        replay.Launch(replay.STEP_MATMUL, (0x1040, 0x2000, 0x9000, 3, 1, 2048, 4096, 4096, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 0x5000, 4096)),
        replay.Launch(replay.STEP_ZERO, (0x9000, 1)),
    ]
    steps, args = replay.bind(tape, slots)
    assert steps["kind"].tolist() == [replay.STEP_KERNEL, replay.STEP_MATMUL, replay.STEP_ZERO]
    assert steps["first"].tolist() == [0, 3, 23] and steps["nargs"].tolist() == [3, 20, 2]
    assert (int(steps[0]["function"]), int(steps[0]["grid"]), int(steps[0]["block"])) == (7, 3, 64)
    rows = [(int(v), int(s)) for v, s in zip(args["value"], args["slot"])]
    assert rows[:3] == [(0, 0), (0x10, 1), (0x5000, -1)]  # a pointer outside every slot stays constant
    # matmul: a, b, c are pointers; 2048 and 4096 are sizes even though 0x1000 <= 4096 < 0x1100
    assert rows[3:6] == [(0x40, 0), (0, 1), (0, 5)] and rows[3 + 6] == (4096, -1)
    assert rows[3 + 18] == (0x5000, -1) and rows[3 + 19] == (4096, -1)
    assert rows[23:] == [(0, 5), (1, -1)]


def test_overlapping_slots_refuse_the_recording():
    assert replay.bind([], [(0, 0x1000, 256), (1, 0x1000, 256)]) is None
    assert replay.bind([], [(0, 0x1000, 256), (1, 0x10f0, 64)]) is None
    assert replay.bind([], [(0, 0x1000, 256), (1, 0x1100, 64)]) is not None


class StubLib:
    """limn_hip_replay*, as a library whose graph capture fails: counts what was called."""

    def __init__(self, graph_status: int):
        self.graph_status = graph_status
        self.graph_calls = self.list_calls = self.freed = 0

    def limn_hip_replay_graph(self, *args):
        self.graph_calls += 1
        args[-1]._obj.value = 0x1234  # the handle the library would have made
        return self.graph_status

    def limn_hip_replay(self, *args):
        self.list_calls += 1
        return 0

    def limn_hip_replay_graph_free(self, handle):
        self.freed += 1
        return 0

    def limn_hip_last_error(self):
        return b"hip: instantiating a replay graph: operation not supported"


def program() -> replay.Program:
    steps, args = replay.bind([replay.Launch(replay.STEP_ZERO, (0x1000, 16))], [(0, 0x1000, 16)])
    return replay.Program(steps, args, (), (), (), 1)


def test_a_graph_that_fails_falls_back_to_launching_the_list_for_good():
    lib, finished = StubLib(graph_status=3), []
    prog = program()
    slots = np.zeros(1, dtype=np.int64)
    assert prog.run(lib, slots, lambda: finished.append(1), graphs=True) == 0
    assert (lib.graph_calls, lib.list_calls, lib.freed) == (1, 1, 1)  # tried, fell back, released
    assert prog.graph_failure == "hip: instantiating a replay graph: operation not supported"
    assert not prog.graphs and finished
    assert prog.run(lib, slots, lambda: None, graphs=True) == 0
    assert (lib.graph_calls, lib.list_calls) == (1, 2)  # no second capture attempt


def test_a_graph_that_works_is_launched_and_kept():
    lib = StubLib(graph_status=0)
    prog = program()
    assert prog.run(lib, np.zeros(1, dtype=np.int64), lambda: None, graphs=True) == 0
    assert (lib.graph_calls, lib.list_calls, lib.freed) == (1, 0, 0)
    assert len(prog.graphs) == 1 and prog.graph_failure is None


def test_the_device_keeps_a_bounded_number_of_launch_lists(monkeypatch):
    from limn_amd.hip.device import HipDevice
    from limn_amd.seam import Plan

    class Api:
        def hipDeviceSynchronize(self):
            return 0

    lib = StubLib(graph_status=0)
    dev = HipDevice.__new__(HipDevice)
    dev.api, dev.lib, dev.pool = Api(), lib, {}
    dev._commits, dev._commit_targets, dev._committed = [], set(), []
    dev.replays = collections.OrderedDict()
    monkeypatch.setattr(replay, "PLANS_KEPT", 3)
    plans = [Plan(calls=(), buffers=(), sinks=(), positions=0) for _ in range(5)]
    for p in plans[:3]:
        dev.run(p, {})
    dev.replays[id(plans[0])][1] = program()  # the oldest holds a recorded list with a graph
    dev.replays[id(plans[0])][1].graphs[b"k"] = ctypes.c_void_p(0x99)
    dev.run(plans[1], {})  # a second run: recorded now, and the most recently run
    for p in plans[3:]:
        dev.run(p, {})
    assert list(dev.replays) == [id(plans[1]), id(plans[3]), id(plans[4])]
    assert lib.freed == 1  # the evicted list's graph was released
