"""Pre-bound launch lists on the MI355X: a plan's first run goes call by call, its second also
records every launch, later runs replay the list in one native call (limn_amd/hip/replay.py).
Each case runs one graph structure four times with new inputs and checks every result bit for bit
against a device made to run call by call, covering emitted nests with inlined producers, an
ordered scatter (a zero-filled output), a contraction with its relu epilogue, and attention
forward and backward (CUSTOM calls, merged launches), a bf16 Linear with its bias and a residual
added in the contraction's store, and a contraction whose k is split."""

from __future__ import annotations

import numpy as np
import pytest

from limn_amd.seam import CompiledDevice, Tensor, bfloat16, grad, nn, realize, scatter_rows, set_seed
from limn_amd.seam import device as limn_device

pytestmark = pytest.mark.gpu


def softmax_layernorm(seed):
    x = Tensor(np.random.default_rng(seed).standard_normal((300, 257)).astype(np.float32))
    return [nn.LayerNorm(257)(x.softmax(-1))]


def scatter(seed):
    r = np.random.default_rng(seed)
    values = Tensor(r.standard_normal((600, 40)).astype(np.float32))
    return [scatter_rows(values, Tensor(r.integers(0, 50, 600).astype(np.int32)), (50, 40))]


def matmul_relu(seed):
    r = np.random.default_rng(seed)
    a = Tensor(r.standard_normal((256, 512)).astype(np.float32), dtype=bfloat16)
    b = Tensor(r.standard_normal((512, 384)).astype(np.float32), dtype=bfloat16)
    return [(a @ b).relu()]


def linear_bias_residual(seed):
    """A bf16 Linear with its float32 bias cast at use, added to a residual stream, as the GPT's
    blocks spell it: one contraction with the bias and the residual added at its store."""
    from limn_amd.gpt import mixed

    set_seed(seed)
    layer = nn.Linear(256, 384)
    r = np.random.default_rng(seed)
    x = Tensor(r.standard_normal((4, 128, 256)).astype(np.float32), dtype=bfloat16)
    res = Tensor(r.standard_normal((4, 128, 384)).astype(np.float32), dtype=bfloat16)
    return [res + mixed(layer, x)]


SPLIT_K = (256, 256, 8192)  # (M, N, K): 4 output tiles and a long k, so k splits


def split_k(seed):
    """Few output tiles and a long k: slices of k in float32 partials (a fixed workspace the
    runner holds) folded in slice order by a second kernel."""
    m, n, k = SPLIT_K
    r = np.random.default_rng(seed)
    a = Tensor(r.standard_normal((m, k)).astype(np.float32), dtype=bfloat16)
    b = Tensor(r.standard_normal((k, n)).astype(np.float32), dtype=bfloat16)
    return [a @ b]


def attention(seed):
    r = np.random.default_rng(seed)
    q, k, v = (Tensor(r.standard_normal((2, 2, 200, 64)).astype(np.float32), dtype=bfloat16, requires_grad=True) for _ in range(3))
    w = Tensor(r.standard_normal((2, 2, 200, 64)).astype(np.float32))
    out = q.attention(k, v, causal=True)
    return [out, *grad((out.float() * w).sum(), [q, k, v])]


CASES = {"softmax_layernorm": softmax_layernorm, "scatter": scatter, "matmul_relu": matmul_relu, "attention": attention,
         "linear_bias_residual": linear_bias_residual, "split_k": split_k}


def test_the_split_k_case_splits(hipdev):
    from limn_amd.dtypes import ABI_CODE

    assert hipdev.lib.limn_hip_matmul_workspace(ABI_CODE[bfloat16], 1, *SPLIT_K) > 0


def results(dev, build, seed) -> list[np.ndarray]:
    limn_device.active_device = dev
    tensors = build(seed)
    realize(*tensors)
    return [t.numpy() for t in tensors]


@pytest.mark.parametrize("case", sorted(CASES))
def test_replayed_runs_equal_call_by_call_runs(hipdev, case):
    from limn_amd.hip.device import HipDevice

    plain = HipDevice()
    plain.run = lambda plan, sources: CompiledDevice.run(plain, plan, sources)  # never records
    # the plans that already had a list (held, so no new plan can take one's id); the table is
    # bounded, so a new list may push an old one out and the count alone need not grow
    before = [e[0] for e in hipdev.replays.values() if e[1] is not None]
    for seed in range(4):
        print(f"replay case {case}, run {seed}", flush=True)
        got = results(hipdev, CASES[case], seed)
        want = results(plain, CASES[case], seed)
        for g, w in zip(got, want):
            assert g.dtype == w.dtype and g.shape == w.shape
            np.testing.assert_array_equal(g.view(np.uint8), w.view(np.uint8))
    recorded = [e[0] for e in hipdev.replays.values() if e[1] is not None]
    assert any(all(p is not b for b in before) for p in recorded)  # a list was recorded and replayed


@pytest.mark.parametrize("case", sorted(CASES))
def test_graph_replays_equal_call_by_call_runs(case):
    """The launch list replayed as a captured HIP graph: six runs with new inputs, each checked bit
    for bit against a device running call by call (eager work and its barriers between the
    replays). Runs 3 and 4 keep their results alive, so the next runs get other buffers and the
    graph is captured again for the new binding."""
    from limn_amd.hip.device import HipDevice

    graphs = HipDevice()
    assert graphs.replay_graphs
    plain = HipDevice()
    plain.run = lambda plan, sources: CompiledDevice.run(plain, plan, sources)
    held = []
    for seed in range(6):
        print(f"graph replay case {case}, run {seed}", flush=True)
        limn_device.active_device = graphs
        tensors = CASES[case](seed)
        realize(*tensors)
        got = [t.numpy() for t in tensors]
        if seed in (3, 4):
            held.append(tensors)
        want = results(plain, CASES[case], seed)
        for g, w in zip(got, want):
            assert g.dtype == w.dtype and g.shape == w.shape
            np.testing.assert_array_equal(g.view(np.uint8), w.view(np.uint8))
    progs = [e[1] for e in graphs.replays.values() if e[1] is not None]
    assert any(p.graphs for p in progs)  # graphs were captured and replayed
    assert max(p.captures for p in progs) >= 2  # and captured again for the held runs' successors
