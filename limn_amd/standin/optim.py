"""Stand-in for limn's optimizers (reference `limn/optim.py`): SGD with momentum and AdamW, each
step one batch of ASSIGNs.

The contract limn's callers rely on: `step(*also)` builds every update against the pre-step
values and realizes them, with `also` (a loss) in the same batch; the device's transaction rule
commits all the writes after every value is computed, so update order cannot matter. State is
kept at the parameter's dtype but never narrower than float32, and a new parameter value is
rounded once, back into the parameter's own dtype.

The update rules are torch's (torch.optim.SGD without dampening or nesterov; torch.optim.AdamW),
written here as lazy graphs. Everything a step changes lives in device buffers, including
AdamW's bias corrections: a step builds the same graph every time, so one compiled plan (and one
captured replay) serves a whole run.
"""

from __future__ import annotations

from collections.abc import Iterable

from .ops import DType, float32, promote
from .tensor import Tensor, no_grad, realize


def _state_for(p: Tensor) -> Tensor:
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
        """Commit this step's writes, and realize `also` in the same batch (it then reads the
        pre-step parameters like every other value of the batch)."""
        with no_grad():
            writes = self.updates()
        realize(*(target.assign(value) for target, value in writes), *also)

    def updates(self) -> list[tuple[Tensor, Tensor]]:
        """(buffer, its new value) for everything this step writes; commits nothing."""
        raise NotImplementedError


class SGD(Optimizer):
    """p -= lr * b, with b = momentum * b + g kept per parameter when momentum is nonzero."""

    def __init__(self, params: Iterable[Tensor], lr: float, momentum: float = 0.0):
        super().__init__(params)
        self.lr, self.momentum = lr, momentum
        self.buffers = {id(p): _state_for(p) for p in self.params} if momentum else {}

    def updates(self) -> list[tuple[Tensor, Tensor]]:
        writes: list[tuple[Tensor, Tensor]] = []
        for p in (p for p in self.params if p.grad is not None):
            width = promote(p.dtype, float32)
            direction = p.grad.cast(width)
            if self.momentum:
                b = self.buffers[id(p)]
                direction = b * self.momentum + direction
                writes.append((b, direction))
            writes.append((p, (p.cast(width) - direction * self.lr).cast(p.dtype)))
        return writes


class AdamW(Optimizer):
    """torch.optim.AdamW: decoupled decay, then an Adam step with bias-corrected moments,

        p <- p (1 - lr wd) - (lr / c1) m / (sqrt(v) / sqrt(c2) + eps),
        m <- b1 m + (1 - b1) g,   v <- b2 v + (1 - b2) g^2,   c_i = 1 - b_i^t.

    c_i is 1 - b_i^t exactly when it is the running average of the constant 1 started at 0,
    c_i <- b_i c_i + (1 - b_i), so each is a one-element state buffer advanced inside the step's
    graph like the moments (one pair per state dtype). The per-dtype factors lr / c1 and
    1 / sqrt(c2) are built once per step and shared by every parameter of that dtype.
    """

    def __init__(
        self,
        params: Iterable[Tensor],
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 1e-2,
    ):
        super().__init__(params)
        self.lr, (self.beta1, self.beta2), self.eps, self.weight_decay = lr, betas, eps, weight_decay
        self.moments = {id(p): (_state_for(p), _state_for(p)) for p in self.params}
        widths = {promote(p.dtype, float32) for p in self.params}
        self.corrections: dict[DType, tuple[Tensor, Tensor]] = {w: (Tensor.zeros((1,), dtype=w), Tensor.zeros((1,), dtype=w)) for w in widths}

    def updates(self) -> list[tuple[Tensor, Tensor]]:
        writes: list[tuple[Tensor, Tensor]] = []
        factors: dict[DType, tuple[Tensor, Tensor]] = {}
        b1, b2 = self.beta1, self.beta2
        for p in (p for p in self.params if p.grad is not None):
            m, v = self.moments[id(p)]
            if m.dtype not in factors:
                c1, c2 = self.corrections[m.dtype]
                c1_next, c2_next = c1 * b1 + (1 - b1), c2 * b2 + (1 - b2)
                writes += [(c1, c1_next), (c2, c2_next)]
                factors[m.dtype] = (c1_next.reciprocal() * self.lr, c2_next.sqrt().reciprocal())
            step_size, unbias2 = factors[m.dtype]
            g, wide = p.grad.cast(m.dtype), p.cast(m.dtype)  # all arithmetic at the state's width
            m_next = m * b1 + g * (1 - b1)
            v_next = v * b2 + g * g * (1 - b2)
            denom = (v_next.sqrt() * unbias2 + self.eps).reciprocal()
            p_next = wide * (1 - self.lr * self.weight_decay) - m_next * step_size * denom
            writes += [(m, m_next), (v, v_next), (p, p_next.cast(p.dtype))]
        return writes
