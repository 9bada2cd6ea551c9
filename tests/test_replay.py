"""Pre-bound launch lists (limn_amd/hip/replay.py) without a GPU: how a recorded launch's
arguments bind to slots, and the refusals."""

from __future__ import annotations

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
