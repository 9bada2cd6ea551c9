"""The C5 path on the MI355X: the byte-level GPT's training step through the hip device (every
kernel kind at once: embedding GATHER and SCATTER, the emitted elementwise/reduce nests, MFMA
contractions for the Linears and their gradients, CUSTOM attention forward and backward),
against the numpy oracle on a small configuration, captured and replayed, and at full size."""

from __future__ import annotations

import math

import numpy as np
import pytest

from limn_amd.seam import CompiledDevice, bfloat16, capture, grad, nn, set_seed
from limn_amd.seam import device as limn_device
from limn_amd.gpt import GPT, GPTConfig, cross_entropy, make_trainer, synthetic_batch
from oracle import sdpa as ref
from oracle.numpy_device import NumpyDevice

parameters = nn.parameters

pytestmark = pytest.mark.gpu

SMALL = GPTConfig(vocab=64, ctx=64, dim=128, layers=2, heads=2, batch=2, dtype=bfloat16)


def _loss_and_grads(dev, cfg: GPTConfig, seed: int):
    limn_device.active_device = dev
    set_seed(seed)
    model = GPT(cfg)
    x, y = synthetic_batch(cfg, np.random.default_rng(seed))
    loss = cross_entropy(model(x), y)
    grads = grad(loss, parameters(model))
    return loss.item(), [g.numpy() for g in grads]


def test_small_gpt_step_matches_the_oracle(hipdev):
    """bf16 activations: the oracle rounds every node to bf16, the device keeps fused values in
    float, so the comparison is the normalised max error (reference limn/sdpa.py:251-259) at the
    bf16 tolerance of 3e-2."""
    got_loss, got = _loss_and_grads(hipdev, SMALL, 3)
    want_loss, want = _loss_and_grads(NumpyDevice(), SMALL, 3)
    assert abs(got_loss - want_loss) <= 2e-2 * abs(want_loss)
    for g, w in zip(got, want):
        assert np.isfinite(g).all()
        assert ref.worst(g, w) <= 3e-2, ref.worst(g, w)


def test_small_gpt_training_captured_equals_uncaptured(hipdev):
    """Captured training (the hip device replays its launch lists through HIP graphs) against
    the same steps on a device that runs every plan call by call and never records."""
    from limn_amd.hip.device import HipDevice

    plain = HipDevice()
    plain.run = lambda plan, sources: CompiledDevice.run(plain, plan, sources)

    def run(captured: bool):
        limn_device.active_device = hipdev if captured else plain
        set_seed(4)
        model, opt, step = make_trainer(SMALL, lr=1e-3)
        fn = capture(step) if captured else step
        r = np.random.default_rng(4)
        losses = [fn(*synthetic_batch(SMALL, r)).item() for _ in range(5)]
        return losses, [p.numpy() for p in parameters(model)], fn

    plain_losses, plain_params, _ = run(False)
    cap_losses, cap_params, fn = run(True)
    assert fn._feeds is not None
    assert cap_losses == plain_losses
    for a, b in zip(cap_params, plain_params):
        np.testing.assert_array_equal(a, b)


def test_c5_full_size_steps(hipdev):
    """The C5 configuration itself: three captured steps on one fixed batch; the loss starts near
    ln(256) plus the random init's excess, stays finite, and falls."""
    cfg = GPTConfig()
    limn_device.active_device = hipdev
    set_seed(5)
    model, opt, step = make_trainer(cfg)
    fn = capture(step)
    x, y = synthetic_batch(cfg, np.random.default_rng(5))
    losses = [fn(x, y).item() for _ in range(4)]
    assert all(math.isfinite(v) for v in losses)
    assert math.log(256) - 0.5 < losses[0] < math.log(256) + 3.0
    assert losses[-1] < losses[0]
    for p in parameters(model)[:4]:
        assert np.isfinite(p.numpy()).all()
