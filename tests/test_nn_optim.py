"""The callers of the hot path on the CPU: nn layers, AdamW/SGD, capture/replay and the C5 GPT
(reference tests/test_nn.py, test_optim.py, test_jit.py's capture cases). Numerics are pinned to
torch on the CPU (an independent implementation: torch.nn.functional, torch.optim); capture is
pinned to the uncaptured step, bit for bit, on the C device (a compiled device, so the capture
really replays plans)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from limn_amd.seam import capture, float32, grad, nn, optim, set_seed, Tensor
from limn_amd.seam import device as limn_device
from limn_amd.gpt import GPT, GPTConfig, cross_entropy, gelu, make_trainer, synthetic_batch
from oracle import c_device
from oracle.numpy_device import NumpyDevice

Embedding, LayerNorm, Linear, parameters = nn.Embedding, nn.LayerNorm, nn.Linear, nn.parameters
SGD, AdamW = optim.SGD, optim.AdamW

rng = np.random.default_rng(5)


@pytest.fixture(autouse=True)
def on_numpy():
    limn_device.set_device("numpy")
    set_seed(0)
    yield


def t64(x: Tensor) -> torch.Tensor:
    return torch.tensor(x.numpy(), dtype=torch.float64)


def test_linear_layout_and_init():
    lin = Linear(16, 8)
    assert lin.weight.shape == (8, 16) and lin.bias.shape == (8,)
    w = lin.weight.numpy()
    assert np.abs(w).max() <= 0.25 and np.abs(w).max() > 0.2  # uniform(+-1/sqrt(16))
    x = rng.standard_normal((3, 5, 16)).astype(np.float32)
    got = lin(Tensor(x)).numpy()
    want = F.linear(torch.tensor(x, dtype=torch.float64), t64(lin.weight), t64(lin.bias)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_layer_norm_matches_torch():
    ln = LayerNorm(12)
    ln.weight = Tensor(rng.uniform(0.5, 1.5, 12).astype(np.float32), requires_grad=True)
    ln.bias = Tensor(rng.standard_normal(12).astype(np.float32), requires_grad=True)
    x = rng.standard_normal((4, 12)).astype(np.float32) * 3 + 1
    want = F.layer_norm(torch.tensor(x, dtype=torch.float64), (12,), t64(ln.weight), t64(ln.bias), 1e-5).numpy()
    np.testing.assert_allclose(ln(Tensor(x)).numpy(), want, rtol=1e-5, atol=1e-5)


def test_gelu_is_torch_tanh_gelu_and_finite_everywhere():
    x = np.concatenate([np.linspace(-12, 12, 301), [-1e4, -200.0, 200.0, 1e4]]).astype(np.float32)
    got = gelu(Tensor(x)).numpy()
    want = F.gelu(torch.tensor(x, dtype=torch.float64), approximate="tanh").numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    t = Tensor(x[:301], requires_grad=True)
    (g,) = grad(gelu(t).sum(), [t])
    tx = torch.tensor(x[:301], dtype=torch.float64, requires_grad=True)
    F.gelu(tx, approximate="tanh").sum().backward()
    np.testing.assert_allclose(g.numpy(), tx.grad.numpy(), rtol=1e-4, atol=1e-5)


def test_embedding_rows():
    emb = Embedding(10, 4)
    idx = rng.integers(0, 10, size=(3, 5)).astype(np.int32)
    np.testing.assert_array_equal(emb(Tensor(idx)).numpy(), emb.weight.numpy()[idx])


def test_parameters_walks_depth_first_once_and_survives_cycles():
    class M:
        def __init__(self):
            self.a = Linear(2, 3)
            self.layers = [Linear(3, 3), {"x": Linear(3, 1, bias=False)}]
            self.again = self.a
            self.me = self

    m = M()
    ps = parameters(m)
    want = [m.a.weight, m.a.bias, m.layers[0].weight, m.layers[0].bias, m.layers[1]["x"].weight]
    assert [id(p) for p in ps] == [id(p) for p in want]


def _torch_linear_model(lin: Linear) -> torch.nn.Linear:
    t = torch.nn.Linear(lin.weight.shape[1], lin.weight.shape[0]).double()
    with torch.no_grad():
        t.weight.copy_(t64(lin.weight))
        t.bias.copy_(t64(lin.bias))
    return t


@pytest.mark.parametrize("dev_name", ["numpy", "c"])
def test_adamw_matches_torch(dev_name):
    if dev_name == "c":
        if c_device.compiler() is None:
            pytest.skip("no host C compiler")
        limn_device.active_device = c_device.CDevice()
    lin = Linear(6, 4)
    ref = _torch_linear_model(lin)
    opt = AdamW(parameters(lin), lr=1e-2, betas=(0.8, 0.95), eps=1e-6, weight_decay=0.1)
    topt = torch.optim.AdamW(ref.parameters(), lr=1e-2, betas=(0.8, 0.95), eps=1e-6, weight_decay=0.1)
    for _ in range(4):
        x = rng.standard_normal((5, 6)).astype(np.float32)
        opt.zero_grad()
        loss = (lin(Tensor(x)) * lin(Tensor(x))).mean()
        loss.backward()
        opt.step(loss)
        topt.zero_grad()
        tl = (ref(torch.tensor(x, dtype=torch.float64)) ** 2).mean()
        tl.backward()
        topt.step()
        np.testing.assert_allclose(loss.item(), tl.item(), rtol=1e-5)
    np.testing.assert_allclose(lin.weight.numpy(), ref.weight.detach().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lin.bias.numpy(), ref.bias.detach().numpy(), rtol=1e-5, atol=1e-6)


def test_sgd_momentum_matches_torch():
    lin = Linear(3, 2)
    ref = _torch_linear_model(lin)
    opt = SGD(parameters(lin), lr=0.1, momentum=0.9)
    topt = torch.optim.SGD(ref.parameters(), lr=0.1, momentum=0.9)
    for _ in range(3):
        x = rng.standard_normal((4, 3)).astype(np.float32)
        opt.zero_grad()
        loss = lin(Tensor(x)).sum()
        loss.backward()
        opt.step()
        topt.zero_grad()
        ref(torch.tensor(x, dtype=torch.float64)).sum().backward()
        topt.step()
    np.testing.assert_allclose(lin.weight.numpy(), ref.weight.detach().numpy(), rtol=1e-5, atol=1e-6)


def test_optimizer_needs_parameters():
    with pytest.raises(ValueError):
        AdamW([Tensor(np.zeros(3, np.float32))])


# ---- the GPT, against torch ---------------------------------------------------------------------

TINY = GPTConfig(vocab=32, ctx=8, dim=16, layers=2, heads=2, batch=3, dtype=float32)


def _torch_gpt_loss(model: GPT, tokens: np.ndarray, targets: np.ndarray):
    """The same model written with torch ops from the same float64 weights."""
    P = {id(p): t64(p).requires_grad_() for p in parameters(model)}
    W = lambda p: P[id(p)]  # noqa: E731
    cfg = model.cfg
    x = W(model.tok.weight)[torch.tensor(tokens, dtype=torch.long)] + W(model.pos.weight)[torch.arange(cfg.ctx)]
    for blk in model.blocks:
        b, t, c = x.shape
        h = F.layer_norm(x, (c,), W(blk.ln1.weight), W(blk.ln1.bias), 1e-5)
        qkv = F.linear(h, W(blk.qkv.weight), W(blk.qkv.bias)).reshape(b, t, 3, cfg.heads, c // cfg.heads).permute(2, 0, 3, 1, 4)
        att = F.scaled_dot_product_attention(qkv[0], qkv[1], qkv[2], is_causal=True)
        x = x + F.linear(att.permute(0, 2, 1, 3).reshape(b, t, c), W(blk.proj.weight), W(blk.proj.bias))
        h = F.layer_norm(x, (c,), W(blk.ln2.weight), W(blk.ln2.bias), 1e-5)
        x = x + F.linear(F.gelu(F.linear(h, W(blk.up.weight), W(blk.up.bias)), approximate="tanh"), W(blk.down.weight), W(blk.down.bias))
    logits = F.linear(F.layer_norm(x, (cfg.dim,), W(model.ln.weight), W(model.ln.bias), 1e-5), W(model.head.weight))
    loss = F.cross_entropy(logits.reshape(-1, cfg.vocab), torch.tensor(targets, dtype=torch.long).reshape(-1))
    loss.backward()
    return loss.item(), [P[id(p)].grad.numpy() for p in parameters(model)]


def test_gpt_loss_and_gradients_match_torch():
    model = GPT(TINY)
    x, y = synthetic_batch(TINY, np.random.default_rng(1))
    loss = cross_entropy(model(x), y)
    grads = grad(loss, parameters(model))
    want_loss, want_grads = _torch_gpt_loss(model, x.numpy(), y.numpy())
    np.testing.assert_allclose(loss.item(), want_loss, rtol=1e-5)
    for g, w in zip(grads, want_grads):
        np.testing.assert_allclose(g.numpy(), w, rtol=1e-3, atol=1e-5)


def test_gpt_flop_count_is_the_c5_figure():
    cfg = GPTConfig()
    assert cfg.matmul_params() == 25_296_896
    assert abs(cfg.flops_per_token() - 1.644e8) / 1.644e8 < 1e-3
    assert abs(cfg.flops_per_token() * cfg.tokens - 2.693e12) / 2.693e12 < 1e-3


# ---- capture on a compiled device ---------------------------------------------------------------

needs_cc = pytest.mark.skipif(c_device.compiler() is None, reason="no host C compiler")


def _trained(captured: bool, steps: int = 5):
    limn_device.active_device = c_device.CDevice()
    set_seed(3)
    model, opt, step = make_trainer(TINY, lr=1e-2)
    fn = capture(step) if captured else step
    r = np.random.default_rng(2)
    losses = []
    for _ in range(steps):
        x, y = synthetic_batch(TINY, r)
        losses.append(fn(x, y).item())
    return losses, [p.numpy() for p in parameters(model)], fn


@needs_cc
def test_captured_training_is_bit_identical_to_running_the_step():
    plain_losses, plain_params, _ = _trained(False)
    cap_losses, cap_params, fn = _trained(True)
    assert fn._feeds is not None  # replays really happened
    assert cap_losses == plain_losses
    for a, b in zip(cap_params, plain_params):
        np.testing.assert_array_equal(a, b)


@needs_cc
def test_replays_return_fresh_results_that_do_not_alias():
    limn_device.active_device = c_device.CDevice()
    model, opt, step = make_trainer(TINY, lr=1e-2)
    fn = capture(step)
    r = np.random.default_rng(4)
    batches = [synthetic_batch(TINY, r) for _ in range(4)]
    outs = [fn(x, y) for x, y in batches]
    vals = [o.item() for o in outs]
    assert len({id(o.node.arg) for o in outs[2:]}) == 2 and len(set(vals)) == 4


@needs_cc
def test_capture_refuses_a_changing_graph_and_bad_arguments():
    limn_device.active_device = c_device.CDevice()
    w = Tensor(np.ones(3, np.float32))
    calls = []

    def step(x):
        calls.append(1)
        out = (x * (2.0 if len(calls) == 1 else 3.0) + w).realize()
        return out

    fn = capture(step)
    x = Tensor(np.ones(3, np.float32))
    fn(x)
    with pytest.raises(ValueError, match="different graph"):
        fn(x)
    fn2 = capture(lambda x: (x + 1.0).realize())
    with pytest.raises(ValueError, match="buffer-backed"):
        fn2(x * 2.0)
    with pytest.raises(ValueError, match="realized nothing"):
        capture(lambda x: x + 1.0)(x)

    def unrealized_result(x):
        (x * 2.0).realize()
        return x + 1.0

    fn3 = capture(unrealized_result)
    fn3(x)
    with pytest.raises(ValueError, match="must realize what it returns"):
        fn3(x)


@needs_cc
def test_a_replay_refuses_another_device():
    dev = c_device.CDevice()
    limn_device.active_device = dev
    fn = capture(lambda x: (x * 2.0).realize())
    x = Tensor(np.ones(4, np.float32))
    fn(x), fn(x)
    np.testing.assert_array_equal(fn(x).numpy(), np.full(4, 2.0, np.float32))
    limn_device.active_device = c_device.CDevice()
    with pytest.raises(ValueError, match="device that recorded"):
        fn(Tensor(np.ones(4, np.float32)))


def test_capture_on_an_interpreting_device_just_runs():
    limn_device.active_device = NumpyDevice()
    fn = capture(lambda x: (x + 1.0).realize())
    for k in range(3):
        assert fn(Tensor(np.full(2, float(k), np.float32))).numpy().tolist() == [k + 1.0, k + 1.0]
