"""The plan executor every compiled limn device shares: this is the drop-in boundary.

Restates reference `limn/jit.py:44-242` with the same hooks, plan-cache key, CUSTOM sibling
merge and transaction rule, so the `hip` device (limn_amd/hip/device.py) subclasses exactly
what limn's own `cuda` device subclasses:

- `execute(sinks)` walks the graph, keys it by structure (`graph_key`: op, dtype, shape, arg
  except a BUFFER's bytes, src positions, sink positions) and builds a Plan on a miss;
- a Plan is kernel Calls by buffer position; `run` allocates a fresh output per call (zeroed
  for SCATTER), launches every call, then commits every ASSIGN, then calls `finish()` once;
- CUSTOM nodes that are outputs of one kernel invocation (same name, params and src
  positions) fold into one Call, each taking the first call whose slot for its index is free;
- a backend supplies `runners`, `out_alloc`, `commit`, and optionally `prepare`/`finish`,
  and registers CUSTOM builders by name in `self.custom`.
"""

from __future__ import annotations

import math
from collections.abc import Callable, Mapping
from dataclasses import dataclass, replace
from typing import Any

from .codegen import LoopNest, lower_all
from .ops import Custom, Node, Op, topological
from .schedule import realized, schedule

Buffer = Any
Runner = Callable[[list[Buffer], list[Buffer]], None]


def nbytes(node: Node) -> int:
    return node.dtype.itemsize * math.prod(node.shape)


def graph_key(order: list[Node], position: dict[Node, int], sinks: list[Node]) -> tuple:
    """A hashable key for the graph's structure; equal keys lower to the same program."""
    nodes = tuple(
        (n.op, n.dtype, n.shape, None if n.op is Op.BUFFER else n.arg, tuple(position[s] for s in n.srcs)) for n in order
    )
    return nodes, tuple(position[s] for s in sinks)


@dataclass(frozen=True)
class Call:
    fn: Runner
    inputs: tuple[int, ...]
    outputs: tuple[int | None, ...]
    out_nbytes: tuple[int, ...]
    zero_fill: bool
    assign_target: int | None


@dataclass(frozen=True)
class Plan:
    calls: tuple[Call, ...]
    buffers: tuple[int, ...]
    sinks: tuple[int, ...]
    positions: int


@dataclass(frozen=True)
class Recording:
    plan: Plan
    bound: tuple[Buffer, ...]
    outs: tuple[Buffer, ...]


class CompiledDevice:
    """Plan-cached execution over backend hooks (alloc/copyin/copyout come from the backend)."""

    def __init__(self) -> None:
        self.plans: dict[tuple, Plan] = {}
        self.record: list[Recording] | None = None
        self.custom: dict[str, Callable[[Node], Runner]] = {}

    # ---- backend hooks ----

    def runners(self, nests: list[LoopNest]) -> list[Runner]:
        raise NotImplementedError

    def out_alloc(self, nb: int, zero: bool) -> Buffer:
        raise NotImplementedError

    def commit(self, target: Buffer, value: Buffer) -> None:
        raise NotImplementedError

    def has_custom(self, name: str) -> bool:
        return name in self.custom

    def custom_runner(self, node: Node) -> Runner:
        build = self.custom.get(node.arg.name)
        if build is None:
            raise NotImplementedError(f"{type(self).__name__} has no kernel for custom op {node.arg.name!r}")
        return build(node)

    def prepare(self, buf: Buffer) -> Buffer:
        return buf

    def finish(self) -> None:
        pass

    # ---- shared execution ----

    def execute(self, sinks: list[Node]) -> list[Buffer]:
        order = topological(sinks)
        position = {node: p for p, node in enumerate(order)}
        key = graph_key(order, position, sinks)
        plan = self.plans.get(key)
        if plan is None:
            plan = self.plan_of(order, position, sinks)
            self.plans[key] = plan
        sources = {p: order[p].arg for p in plan.buffers}
        outs = self.run(plan, sources)
        if self.record is not None:
            self.record.append(Recording(plan, tuple(sources.values()), tuple(outs)))
        return outs

    def run(self, plan: Plan, sources: Mapping[int, Buffer]) -> list[Buffer]:
        """One transaction: every call, then the deferred ASSIGN commits, then one barrier."""
        bufs: list[Buffer] = [None] * plan.positions
        for p, buf in sources.items():
            bufs[p] = self.prepare(buf)
        pending: list[tuple[int, Buffer]] = []
        for call in plan.calls:
            outs = [self.out_alloc(nb, call.zero_fill) for nb in call.out_nbytes]
            call.fn([bufs[p] for p in call.inputs], outs)
            for p, out in zip(call.outputs, outs):
                if p is not None:
                    bufs[p] = out
            if call.assign_target is not None:
                pending.append((call.assign_target, outs[0]))
        for p, value in pending:
            self.commit(sources[p], value)
            bufs[p] = value
        self.finish()
        return [bufs[p] for p in plan.sinks]

    def plan_of(self, order: list[Node], position: dict[Node, int], sinks: list[Node]) -> Plan:
        kernels = schedule(sinks, order)
        nests = lower_all(sinks, order, kernels)
        fns = iter(self.runners(nests)) if nests else iter(())
        calls: list[Call] = []
        groups: dict[tuple, list[int]] = {}
        for kernel in kernels:
            root = kernel.ast
            if root.op is Op.CUSTOM:
                arg: Custom = root.arg
                key = (arg.name, arg.params, tuple(position[s] for s in root.srcs))
                group = groups.setdefault(key, [])
                slot = next((c for c in group if calls[c].outputs[arg.index] is None), None)
                if slot is not None:
                    outputs = list(calls[slot].outputs)
                    outputs[arg.index] = position[root]
                    calls[slot] = replace(calls[slot], outputs=tuple(outputs))
                    continue
                group.append(len(calls))
                fn = self.custom_runner(root)
                outputs = tuple(position[root] if k == arg.index else None for k in range(len(arg.outs)))
                sizes = tuple(dtype.itemsize * math.prod(shape) for dtype, shape in arg.outs)
            else:
                fn = next(fns)
                outputs = (position[root],)
                sizes = (nbytes(kernel.target),)
            calls.append(
                Call(
                    fn=fn,
                    inputs=tuple(position[n] for n in kernel.inputs),
                    outputs=outputs,
                    out_nbytes=sizes,
                    zero_fill=root.op is Op.SCATTER,
                    assign_target=position[kernel.target] if root.op is Op.ASSIGN else None,
                )
            )
        return Plan(
            calls=tuple(calls),
            buffers=tuple(p for p, node in enumerate(order) if node.op is Op.BUFFER),
            sinks=tuple(position[realized(s)] for s in sinks),
            positions=len(order),
        )
