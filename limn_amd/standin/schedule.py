"""Kernel cuts: which nodes of a graph land in a buffer of their own.

Restates reference `limn/schedule.py:46-141`; the cut rule decides which kernels a device is
handed, so it is kept exactly:

- CONTIGUOUS, ASSIGN, SUM, MAX, GATHER, SCATTER and CUSTOM always end a kernel (CUT_OPS);
- a node that a VIEW or GATHER *addresses* (its first src) must be bytes, so a computed one is
  cut (an expand of an expression is therefore a cut);
- every sink is cut unless it only aliases a buffer (a reshape of realized bytes);
- everything else (elementwise work, CONST, aliasing views) fuses into its consumer.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

from .ops import Node, Op, topological

CUT_OPS = (Op.CONTIGUOUS, Op.ASSIGN, Op.SUM, Op.MAX, Op.GATHER, Op.SCATTER, Op.CUSTOM)
_ADDRESSING = (Op.VIEW, Op.GATHER)


@dataclass(frozen=True)
class Kernel:
    """One nest's work: `ast` is the root it computes, `body` the fused nodes (sources first),
    `inputs` the realized nodes it loads, in first-load order."""

    ast: Node
    body: tuple[Node, ...]
    inputs: tuple[Node, ...]

    @property
    def target(self) -> Node:
        """Whose buffer the kernel writes: an ASSIGN's target, otherwise the root itself."""
        return self.ast.srcs[0] if self.ast.op is Op.ASSIGN else self.ast


def addressed(node: Node) -> Node | None:
    """The src a VIEW or GATHER indexes into (not a value it reads)."""
    return node.srcs[0] if node.op in _ADDRESSING else None


def reads(node: Node) -> tuple[Node, ...]:
    """The srcs whose values this node consumes: all of them except an addressed buffer or an
    ASSIGN's destination, which for these three ops is always the first src."""
    if node.op in (Op.VIEW, Op.GATHER, Op.ASSIGN):
        return node.srcs[1:]
    return node.srcs


def is_alias(node: Node) -> bool:
    """A VIEW that reads its whole source row-major from element 0: same bytes, new shape."""
    if node.op is not Op.VIEW:
        return False
    view = node.arg
    return view.is_contiguous and view.numel == math.prod(node.srcs[0].shape)


def realized(node: Node) -> Node:
    """The node whose buffer holds `node`'s bytes once realized (peels aliases and ASSIGNs)."""
    while node.op is Op.ASSIGN or is_alias(node):
        node = node.srcs[0]
    return node


def boundaries(sinks: list[Node], order: list[Node]) -> set[Node]:
    """Every node that must end in its own buffer; `order` is topological(sinks)."""
    cuts: set[Node] = {node for node in order if node.op in CUT_OPS}
    for node in order:
        src = addressed(node)
        if src is not None and src.op not in (Op.BUFFER, Op.CONST):
            cuts.add(src)
    for sink in sinks:
        home = realized(sink)
        if home.op is not Op.BUFFER:
            cuts.add(home)
    return cuts


def fuse(root: Node, cuts: set[Node]) -> Kernel:
    """Collect the nodes computed inside `root`'s kernel and the realized nodes it loads.

    Post-order over `reads`, stopping at cuts and BUFFERs (which become inputs, in the order
    first met); then the buffers the body addresses are appended as further inputs.
    """
    body: list[Node] = []
    inputs: list[Node] = []
    seen: set[Node] = {root}
    stack: list[tuple[Node, int]] = [(root, 0)]
    while stack:
        node, k = stack[-1]
        children = reads(node)
        if k < len(children):
            stack[-1] = (node, k + 1)
            child = children[k]
            if child in seen:
                continue
            seen.add(child)
            if child in cuts or child.op is Op.BUFFER:
                inputs.append(child)
            else:
                stack.append((child, 0))
        else:
            stack.pop()
            body.append(node)
    for node in body:
        src = addressed(node)
        if src is not None and src.op is not Op.CONST and src not in seen:
            seen.add(src)
            inputs.append(src)
    return Kernel(root, tuple(body), tuple(inputs))


def schedule(sinks: list[Node], order: list[Node] | None = None) -> list[Kernel]:
    """The kernels that realize `sinks`, in dependency order."""
    if order is None:
        order = topological(sinks)
    cuts = boundaries(sinks, order)
    return [fuse(node, cuts) for node in order if node in cuts]
