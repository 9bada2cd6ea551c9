"""Optimizers whose steps are ASSIGN graphs, committed in one batch (reference limn/optim.py).

A step builds every update from the pre-step values and realizes all of them together; the
plan executor defers the ASSIGN writes until every kernel of the batch has run, so the order
of the updates cannot matter. Optimizer state is float32 or wider (the parameter's dtype when
that is wider), and the update rounds once into the parameter's own dtype.

AdamW keeps beta1**t and beta2**t in one-element device buffers that each step multiplies in
its own graph: the graph is then identical from step to step, which is what lets one compiled
plan serve a whole run and a captured step replay without host bookkeeping (reference
limn/optim.py:75-120).
"""

from __future__ import annotations

from collections.abc import Iterable

from limn_amd.ops import DType, float32, promote
from limn_amd.tensor import Tensor, no_grad, realize


def state_like(p: Tensor) -> Tensor:
    return Tensor.zeros(p.shape, dtype=promote(p.dtype, float32))


class Optimizer:
    def __init__(self, params: Iterable[Tensor]):
        self.params = [p for p in params if p.requires_grad]
        if not self.params:
            raise ValueError("optimizer got no parameters with requires_grad=True")

    def zero_grad(self) -> None:
        for p in self.params:
            p.grad = None

    def step(self, *also: Tensor) -> None:
        """Commit the step's updates in one batch; tensors passed in (a loss) realize in the
        same batch, reading the pre-step parameters like everything else in it."""
        with no_grad():
            updates = self.updates()
        realize(*[target.assign(value) for target, value in updates], *also)

    def updates(self) -> list[tuple[Tensor, Tensor]]:
        raise NotImplementedError


class SGD(Optimizer):
    """p -= lr * g, or with momentum v = momentum * v + g, p -= lr * v (torch.optim.SGD)."""

    def __init__(self, params: Iterable[Tensor], lr: float, momentum: float = 0.0):
        super().__init__(params)
        self.lr = lr
        self.momentum = momentum
        self.velocity = [state_like(p) if momentum else None for p in self.params]

    def updates(self) -> list[tuple[Tensor, Tensor]]:
        out: list[tuple[Tensor, Tensor]] = []
        for p, v in zip(self.params, self.velocity):
            if p.grad is None:
                continue
            g = p.grad
            if v is not None:
                g = self.momentum * v + g
                out.append((v, g))
            out.append((p, (p - self.lr * g).cast(p.dtype)))
        return out


class AdamW(Optimizer):
    """torch.optim.AdamW: Adam moments with bias correction and weight decay decoupled from the
    gradient (p -= lr * (m_hat / (sqrt(v_hat) + eps) + weight_decay * p))."""

    def __init__(
        self,
        params: Iterable[Tensor],
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 1e-2,
    ):
        super().__init__(params)
        self.lr = lr
        self.beta1, self.beta2 = betas
        self.eps = eps
        self.weight_decay = weight_decay
        self.m = [state_like(p) for p in self.params]
        self.v = [state_like(p) for p in self.params]
        # beta**t per state dtype, so a float64 state is not corrected through float32
        self.powers: dict[DType, tuple[Tensor, Tensor]] = {
            d: (Tensor.ones((1,), dtype=d), Tensor.ones((1,), dtype=d)) for d in {m.dtype for m in self.m}
        }

    def updates(self) -> list[tuple[Tensor, Tensor]]:
        out: list[tuple[Tensor, Tensor]] = []
        corrections: dict[DType, tuple[Tensor, Tensor]] = {}
        for p, m, v in zip(self.params, self.m, self.v):
            if p.grad is None:
                continue
            if m.dtype not in corrections:
                pow1, pow2 = self.powers[m.dtype]
                next1, next2 = pow1 * self.beta1, pow2 * self.beta2
                out += [(pow1, next1), (pow2, next2)]
                # 1 / (1 - beta**t) once per dtype: every parameter multiplies by the same buffer
                corrections[m.dtype] = ((1.0 - next1).reciprocal(), (1.0 - next2).reciprocal())
            inv1, inv2 = corrections[m.dtype]
            g = p.grad
            m_next = self.beta1 * m + (1.0 - self.beta1) * g
            v_next = self.beta2 * v + (1.0 - self.beta2) * (g * g)
            step = (m_next * inv1) / ((v_next * inv2).sqrt() + self.eps) + self.weight_decay * p
            out += [(m, m_next), (v, v_next), (p, (p - self.lr * step).cast(p.dtype))]
        return out
