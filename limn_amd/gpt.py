"""The C5 workload: one training step of a byte-level GPT built from limn's nn layers.

The model follows reference examples/train_stories.py:23-58 (pre-norm blocks: fused qkv Linear,
causal attention through limn's CUSTOM seam, output projection, MLP 4x; token + position
embeddings; a final LayerNorm and an unbiased head) at the size the C5 configuration names:
vocab 256, d_model 512, 8 layers, 8 heads (head dim 64), context 512, batch 32, MLP with tanh
GELU, AdamW (lr 3e-4, weight decay 0.1).

The residual stream (and its gradient) is materialized after every sublayer; see
`materialized`. limn has no GELU (its examples use relu), so `gelu` here composes the tanh
form from primitives.

Everything limn-facing comes through limn_amd.seam: with limn importable this is a model on
limn's own Tensor, nn and AdamW.

Mixed precision, explicit in the graph: parameters (and AdamW's state) stay float32 masters;
each Linear casts its weight and bias to the activation dtype at use, so the products run as
bf16 contractions with float32 totals; LayerNorm statistics and the loss's log-softmax are
computed in float32 and the normalised activations rounded back; the residual stream and
attention are bf16. The backward of each cast hands float32 gradients to the masters. With
`dtype=float32` the same graph is an all-float32 twin (what a device without bf16 runs).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from limn_amd.seam import DType, Node, Op, Tensor, bfloat16, float32, int32, nn, optim

Embedding, LayerNorm, Linear, parameters, AdamW = nn.Embedding, nn.LayerNorm, nn.Linear, nn.parameters, optim.AdamW

GELU_C = math.sqrt(2.0 / math.pi)
GELU_CUBIC = 0.044715
GELU_EXP_LIMIT = 80.0  # exp(80) ~ 5.5e34: finite in float32 and bfloat16


def gelu(x: Tensor) -> Tensor:
    """GELU, tanh form: 0.5 x (1 + tanh(c (x + 0.044715 x^3))), c = sqrt(2/pi). Since
    0.5 (1 + tanh(z)) = 1 / (1 + exp(-2z)), it is x / (1 + exp(-2c (x + 0.044715 x^3))): one
    EXP and one RECIP, no tanh primitive. The exponent is capped at GELU_EXP_LIMIT: past it the
    value (|x| e^-80 < 1e-33) is zero to float precision, and without the cap the exponential
    overflows and the backward multiplies that infinity by zero."""
    inner = ((x + GELU_CUBIC * (x * x * x)) * (-2.0 * GELU_C)).minimum(GELU_EXP_LIMIT)
    return x * (inner.exp() + 1.0).reciprocal()


@dataclass(frozen=True)
class GPTConfig:
    vocab: int = 256
    ctx: int = 512
    dim: int = 512
    layers: int = 8
    heads: int = 8
    batch: int = 32
    dtype: DType = bfloat16

    @property
    def tokens(self) -> int:
        return self.batch * self.ctx

    def matmul_params(self) -> int:
        """Weights that take part in a matmul: 12 d^2 per block plus the head."""
        return self.layers * 12 * self.dim * self.dim + self.dim * self.vocab

    def flops_per_token(self) -> float:
        """6 N for the matmuls (forward 2N, backward 4N) plus causal attention (QK^T and PV
        forward, their 4 backward products, counted as half the square): 3 * 4 * ctx * d / 2
        per layer."""
        return 6.0 * self.matmul_params() + self.layers * 3 * 4 * self.ctx * self.dim / 2


def materialized(x: Tensor) -> Tensor:
    """x written to memory once (a CONTIGUOUS node, a scheduler cut), and in the backward its
    gradient too. The residual stream is read by every later sublayer: left as an expression, the
    scheduler fuses the whole sum into each reader, which then re-reads every term ever added to
    it (traffic quadratic in depth, in the forward and again in the backward)."""
    return Tensor.from_node(Node(Op.CONTIGUOUS, (x.node,), x.dtype, x.shape), (x,), lambda g: (materialized(g),))


def mixed(layer: Linear, x: Tensor) -> Tensor:
    """A Linear with its float32 weight and bias cast to x's dtype at use."""
    y = x @ layer.weight.cast(x.dtype).transpose()
    return y if layer.bias is None else y + layer.bias.cast(x.dtype)


def normed(ln: LayerNorm, x: Tensor) -> Tensor:
    """LayerNorm computed in float32, the result in x's dtype."""
    return ln(x.cast(float32)).cast(x.dtype)


class Block:
    def __init__(self, cfg: GPTConfig):
        d = cfg.dim
        self.heads = cfg.heads
        self.ln1, self.ln2 = LayerNorm(d), LayerNorm(d)
        self.qkv = Linear(d, 3 * d)
        self.proj = Linear(d, d)
        self.up, self.down = Linear(d, 4 * d), Linear(4 * d, d)

    def __call__(self, x: Tensor) -> Tensor:
        b, t, c = x.shape
        hd = c // self.heads
        q, k, v = mixed(self.qkv, normed(self.ln1, x)).reshape(b, t, 3, self.heads, hd).permute(2, 0, 3, 1, 4)
        att = q.attention(k, v, causal=True)
        x = materialized(x + mixed(self.proj, att.permute(0, 2, 1, 3).reshape(b, t, c)))
        return materialized(x + mixed(self.down, gelu(mixed(self.up, normed(self.ln2, x)))))


class GPT:
    def __init__(self, cfg: GPTConfig):
        self.cfg = cfg
        self.tok = Embedding(cfg.vocab, cfg.dim)
        self.pos = Embedding(cfg.ctx, cfg.dim)
        self.blocks = [Block(cfg) for _ in range(cfg.layers)]
        self.ln = LayerNorm(cfg.dim)
        self.head = Linear(cfg.dim, cfg.vocab, bias=False)

    def __call__(self, tokens: Tensor) -> Tensor:
        x = materialized((self.tok(tokens) + self.pos(Tensor.arange(self.cfg.ctx))).cast(self.cfg.dtype))
        for block in self.blocks:
            x = block(x)
        return mixed(self.head, normed(self.ln, x))


def cross_entropy(logits: Tensor, targets: Tensor) -> Tensor:
    """Mean next-token loss, log-softmax in float32 (reference examples/train_stories.py:61-64)."""
    logp = logits.cast(float32).log_softmax(-1)
    vocab = logits.shape[-1]
    onehot = Tensor.arange(vocab).reshape(1, 1, vocab).eq(targets.reshape(*targets.shape, 1))
    return -(logp * onehot).sum() / float(targets.numel)


def synthetic_batch(cfg: GPTConfig, rng: np.random.Generator) -> tuple[Tensor, Tensor]:
    """Tokens uniform in [0, vocab); targets are the next token of the same random stream."""
    stream = rng.integers(0, cfg.vocab, size=(cfg.batch, cfg.ctx + 1)).astype(np.int32)
    return Tensor(stream[:, :-1], dtype=int32), Tensor(stream[:, 1:], dtype=int32)


def make_trainer(cfg: GPTConfig, lr: float = 3e-4, weight_decay: float = 0.1):
    """The model, its optimizer and the (uncaptured) train step: zero_grad, forward, backward,
    AdamW update committed with the loss in one batch, zero_grad again so no gradient graph
    stays attached to the parameters."""
    model = GPT(cfg)
    opt = AdamW(parameters(model), lr=lr, weight_decay=weight_decay)

    def train_step(x: Tensor, y: Tensor) -> Tensor:
        opt.zero_grad()
        loss = cross_entropy(model(x), y)
        loss.backward()
        opt.step(loss)
        opt.zero_grad()
        return loss

    return model, opt, train_step
