"""Stand-in for limn's `capture` (reference `limn/capture.py`): record the device work of one
training step, then replay it without running the step's Python.

Contract kept from limn:

- `capture(fn)` wraps a function whose tensor arguments (realized buffers) are all that changes
  between calls; everything else it touches is updated in place (parameters, optimizer state);
- the first call runs normally; the second runs recorded and must make the device do the same
  thing (the same plans wired the same way) or capture refuses; later calls replay;
- a replay feeds each recorded plan its buffers: the new arguments', the outputs of an earlier
  plan of the same replay (a value the step realized mid-way), or the bytes it saw while
  recording (in-place state); every replay hands back tensors over its own results, except a
  returned in-place target, which is returned as itself;
- a device that does not compile plans (the numpy oracle) just runs the function every call.

Design here: a recording becomes a list of `Feed`s over one *environment* per replay, a list
that starts as the argument buffers and grows by each replayed plan's outputs; a feed says, for
every buffer position of its plan, which environment entry it reads, or holds the buffer it
read while recording. Replaying is evaluating the feeds in order. How fast the plans replay is
the device's business (`CompiledDevice.run`); the hip device launches a hot plan from a
pre-bound launch list.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

from . import device
from .jit import CompiledDevice, Plan, Recording
from .ops import Node, Op
from .schedule import realized
from .tensor import Tensor


@dataclass(frozen=True, slots=True)
class Feed:
    """One recorded plan: `reads` gives (buffer position, environment index) and `held`
    (buffer position, buffer) for bytes that only change in place."""

    plan: Plan
    reads: tuple[tuple[int, int], ...]
    held: tuple[tuple[int, Any], ...]

    def shape(self) -> tuple:
        return id(self.plan), self.reads, tuple(p for p, _ in self.held)


def _feeds(recordings: list[Recording], args: tuple) -> tuple[list[Feed], dict[int, int]]:
    """The recordings as feeds, and which environment index holds each buffer a recording
    produced (by buffer identity; a later producer of the same buffer wins)."""
    where: dict[int, int] = {}
    for i, t in enumerate(args):
        where.setdefault(id(t.node.arg), i)
    size = len(args)
    feeds = []
    for rec in recordings:
        reads, held = [], []
        for p, buf in zip(rec.plan.buffers, rec.bound):
            (reads.append((p, where[id(buf)])) if id(buf) in where else held.append((p, buf)))
        feeds.append(Feed(rec.plan, tuple(reads), tuple(held)))
        for buf in rec.outs:
            where[id(buf)] = size
            size += 1
    produced = {b: i for b, i in where.items() if i >= len(args)}
    return feeds, produced


class capture:
    def __init__(self, fn: Callable[..., Any]):
        self.fn = fn
        self._dev: CompiledDevice | None = None
        self._trial: tuple | None = None  # the first recorded call's feed shapes
        self._feeds: list[Feed] | None = None
        self._spec: tuple = ()
        self._result: Any = None
        self._served: dict[int, int] = {}  # id of a returned tensor -> environment index

    def __call__(self, *args: Any) -> Any:
        dev = device.active()
        if not isinstance(dev, CompiledDevice):
            return self.fn(*args)
        if not all(isinstance(t, Tensor) and t.node.op is Op.BUFFER for t in args):
            raise ValueError("capture takes realized, buffer-backed tensors as arguments")
        if self._feeds is None:
            return self._record(dev, args)
        return self._replay(dev, args)

    def _record(self, dev: CompiledDevice, args: tuple) -> Any:
        if dev.record is not None:
            raise ValueError("capture does not nest")
        dev.record = recordings = []
        try:
            out = self.fn(*args)
        finally:
            dev.record = None
        if not recordings:
            raise ValueError("the captured function realized nothing, so there is no work to replay")
        feeds, produced = _feeds(recordings, args)
        shape = tuple(f.shape() for f in feeds)
        if self._trial is None:  # the first call may do one-time work; the second is the one kept
            self._trial = shape
            return out
        if shape != self._trial:
            raise ValueError("the captured function built a different graph on its second call; capture needs a fixed graph")
        returned = [out] if isinstance(out, Tensor) else list(out or [])
        for t in returned:
            if not isinstance(t, Tensor):
                raise ValueError(f"a captured function may return tensors only, got {type(t).__name__}")
            if realized(t.node).op is not Op.BUFFER:
                raise ValueError("a captured function must realize what it returns; pass it to Optimizer.step or realize()")
        self._served = {id(t): produced[id(realized(t.node).arg)] for t in returned if id(realized(t.node).arg) in produced}
        for t in returned:
            t.derivation = None  # frees the recorded call's graph; requires_grad stays (a parameter)
        self._dev, self._feeds, self._result = dev, feeds, out
        self._spec = tuple((t.shape, t.dtype) for t in args)
        return out

    def _replay(self, dev: CompiledDevice, args: tuple) -> Any:
        if dev is not self._dev:
            raise ValueError("a capture replays only on the device that recorded it; set_device has replaced that one")
        if dev.record is not None:
            raise ValueError("capture does not nest")
        spec = tuple((t.shape, t.dtype) for t in args)
        if spec != self._spec:
            raise ValueError(f"capture recorded arguments {self._spec}, this call passed {spec}")
        env = [t.node.arg for t in args]
        for feed in self._feeds:
            sources = dict(feed.held)
            sources.update((p, env[i]) for p, i in feed.reads)
            env += dev.run(feed.plan, sources)

        def served(t: Any) -> Any:
            i = self._served.get(id(t))
            return t if i is None else Tensor._made(Node(Op.BUFFER, (), t.dtype, t.shape, env[i]))

        if isinstance(self._result, (tuple, list)):
            return type(self._result)(served(t) for t in self._result)
        return served(self._result)
