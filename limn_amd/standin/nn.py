"""Layers composed from Tensor ops: the callers that put limn's training graphs on the hip device.

Same classes, parameter layouts and initialisations as reference limn/nn.py (Linear stores
(out, in) and draws uniform(+-1/sqrt(in)) like torch; LayerNorm starts at ones/zeros and uses the
biased variance; Embedding draws N(0, 1) rows), so a model written against the reference builds
the same graph here. Conv layers are not part of this build (its hot path has none).
"""

from __future__ import annotations

import math

from .tensor import Tensor

class Linear:
    """y = x @ weight^T + bias (reference limn/nn.py:16-26)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        bound = 1.0 / math.sqrt(in_features)
        self.weight = Tensor.uniform((out_features, in_features), -bound, bound, requires_grad=True)
        self.bias = Tensor.uniform((out_features,), -bound, bound, requires_grad=True) if bias else None

    def __call__(self, x: Tensor) -> Tensor:
        y = x @ self.weight.transpose()
        return y if self.bias is None else y + self.bias


class LayerNorm:
    """Normalise the last dim with its biased variance, then scale and shift (reference
    limn/nn.py:29-38)."""

    def __init__(self, dim: int, eps: float = 1e-5):
        self.weight = Tensor.ones((dim,), requires_grad=True)
        self.bias = Tensor.zeros((dim,), requires_grad=True)
        self.eps = eps

    def __call__(self, x: Tensor) -> Tensor:
        centred = x - x.mean(axis=-1, keepdim=True)
        var = (centred * centred).mean(axis=-1, keepdim=True)
        return centred / (var + self.eps).sqrt() * self.weight + self.bias


class Embedding:
    """Rows of an N(0, 1) table picked by int32 indices (reference limn/nn.py:144-150)."""

    def __init__(self, vocab_size: int, dim: int):
        self.weight = Tensor.randn((vocab_size, dim), requires_grad=True)

    def __call__(self, indices: Tensor) -> Tensor:
        return self.weight.gather_rows(indices)


def parameters(module: object) -> list[Tensor]:
    """Every requires_grad tensor reachable through attributes, lists, tuples and dicts, in
    depth-first order, each once; containers are visited once too, so cycles terminate
    (reference limn/nn.py:153-190)."""
    found: list[Tensor] = []
    seen: set[int] = set()
    stack: list[object] = [module]
    # an explicit stack in reverse child order keeps depth-first, first-seen order
    while stack:
        obj = stack.pop()
        if isinstance(obj, Tensor):
            if obj.requires_grad and id(obj) not in seen:
                seen.add(id(obj))
                found.append(obj)
            continue
        if id(obj) in seen:
            continue
        if isinstance(obj, (list, tuple)):
            children = list(obj)
        elif isinstance(obj, dict):
            children = list(obj.values())
        elif hasattr(obj, "__dict__"):
            children = list(vars(obj).values())
        else:
            continue
        seen.add(id(obj))
        stack.extend(reversed(children))
    return found
