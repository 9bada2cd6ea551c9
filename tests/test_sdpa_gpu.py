"""Fused attention on the MI355X: the three CUSTOM kernels (sdpa, sdpa_bwd_q, sdpa_bwd_kv) run
through the hip device's CompiledDevice boundary and its C ABI, diffed against the oracle on the
same inputs.

Tolerances are the reference's own for its GPU device against the numpy reference
(tests/test_attention.py:250-308 there): forward f32 1e-5, f16 2e-3, bf16 1e-2; backward f32
1e-4, f16 4e-3, bf16 3e-2, as rtol = atol (its conftest.check). Each kernel gets the same
inputs on both sides (the GPU forward's L and delta feed both backward checks), so a failure
names one kernel.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from conftest import DTYPES, download, storage_values, upload
from limn_amd.seam import accumulate_in, bfloat16, custom, float32
from oracle import sdpa as ref

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
FWD_TOL = {"float64": 1e-12, "float32": 1e-5, "float16": 2e-3, "bfloat16": 1e-2}
BWD_TOL = {"float64": 1e-11, "float32": 1e-4, "float16": 4e-3, "bfloat16": 3e-2}


def forward(dev, q, k, v, mask, causal, dtype_name):
    dtype = DTYPES[dtype_name]
    scale = q.shape[-1] ** -0.5
    srcs = [upload(dev, x, dtype) for x in (q, k, v)]
    if mask is not None:
        srcs.append(upload(dev, mask, dtype))
    lead, t_q = q.shape[:-2], q.shape[-2]
    outs = ((dtype, lead + (t_q, v.shape[-1])), (accumulate_in(dtype), lead + (t_q, 1)))
    o, lse = custom("sdpa", tuple(srcs), (causal, scale), outs)
    bo, bl = dev.execute([o, lse])
    return download(dev, bo, dtype, o.shape), download(dev, bl, accumulate_in(dtype), lse.shape)


def backward_nodes(dev, q, k, v, do, lse, delta, mask, causal, dtype_name):
    """The (dq, dk, dv) nodes of limn's backward: two CUSTOM calls on the same inputs."""
    dtype = DTYPES[dtype_name]
    stat = accumulate_in(dtype)
    scale = q.shape[-1] ** -0.5
    srcs = [upload(dev, x, dtype) for x in (q, k, v, do)] + [upload(dev, lse, stat), upload(dev, delta, stat)]
    if mask is not None:
        srcs.append(upload(dev, mask, dtype))
    (dq,) = custom("sdpa_bwd_q", tuple(srcs), (causal, scale), ((dtype, q.shape),))
    dk, dv = custom("sdpa_bwd_kv", tuple(srcs), (causal, scale), ((dtype, k.shape), (dtype, v.shape)))
    return dq, dk, dv


def backward(dev, q, k, v, do, lse, delta, mask, causal, dtype_name):
    """Both backward calls in one execution, as limn's gradients() realizes them: the device may
    run the pair as one call (dS handed from the dK/dV pass to the dQ pass)."""
    nodes = backward_nodes(dev, q, k, v, do, lse, delta, mask, causal, dtype_name)
    bufs = dev.execute(list(nodes))
    return [download(dev, b, DTYPES[dtype_name], n.shape) for b, n in zip(bufs, nodes)]


def backward_separately(dev, q, k, v, do, lse, delta, mask, causal, dtype_name):
    """The two backward calls in two executions, so nothing pairs them: each pass on its own."""
    dq, dk, dv = backward_nodes(dev, q, k, v, do, lse, delta, mask, causal, dtype_name)
    (bq,) = dev.execute([dq])
    bk, bv = dev.execute([dk, dv])
    return [download(dev, b, DTYPES[dtype_name], n.shape) for b, n in zip((bq, bk, bv), (dq, dk, dv))]


def draw(seed, q_shape, k_shape, v_shape, dtype_name, live=None):
    rng = np.random.default_rng(seed)
    dtype = DTYPES[dtype_name]
    q, k, v = (storage_values(rng.standard_normal(s).astype(np.float32), dtype) for s in (q_shape, k_shape, v_shape))
    do = storage_values(rng.standard_normal(q_shape[:-1] + v_shape[-1:]).astype(np.float32), dtype)
    mask = None
    if live is not None:
        mask = np.broadcast_to(np.arange(k_shape[-2]) < live, k_shape[:-1]).astype(np.float32)
    if dtype_name == "float64":
        q, k, v, do = (x.astype(np.float64) for x in (q, k, v, do))
        mask = None if mask is None else mask.astype(np.float64)
    return q, k, v, do, mask


def check_case(dev, seed, shapes, causal, dtype_name, live=None):
    q, k, v, do, mask = draw(seed, *shapes, dtype_name, live)
    scale = q.shape[-1] ** -0.5
    out, lse = forward(dev, q, k, v, mask, causal, dtype_name)
    want_out, want_lse = ref.sdpa(q, k, v, mask, causal=causal, scale=scale, dtype=dtype_name)
    tol = FWD_TOL[dtype_name]
    np.testing.assert_allclose(out, want_out, rtol=tol, atol=tol)
    np.testing.assert_allclose(lse, want_lse, rtol=tol, atol=tol)
    delta = (do.astype(np.float64) * out).sum(axis=-1, keepdims=True).astype(lse.dtype)
    dq, dk, dv = backward(dev, q, k, v, do, lse, delta, mask, causal, dtype_name)
    args = (q, k, v, do, lse, delta, mask)
    want_dq = ref.sdpa_backward_q(*args, causal=causal, scale=scale, dtype=dtype_name)
    want_dk, want_dv = ref.sdpa_backward_kv(*args, causal=causal, scale=scale, dtype=dtype_name)
    tol = BWD_TOL[dtype_name]
    for name, got, want in (("dq", dq, want_dq), ("dk", dk, want_dk), ("dv", dv, want_dv)):
        np.testing.assert_allclose(got, want, rtol=tol, atol=tol, err_msg=name)
    return out, lse, dq, dk, dv


# general-width family: the shapes of the reference's own GPU attention tests
ROWS_CASES = {
    "batched": ((2, 3, 64, 16), (2, 3, 64, 16), (2, 3, 64, 24)),
    "ragged": ((2, 2, 100, 16), (2, 2, 100, 16), (2, 2, 100, 24)),
    "several_chunks": ((300, 16), (300, 16), (300, 24)),
}


@pytest.mark.parametrize("dtype_name", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("case", sorted(ROWS_CASES))
def test_rows_family_matches_the_oracle(hipdev, case, causal, dtype_name):
    check_case(hipdev, 1, ROWS_CASES[case], causal, dtype_name)


@pytest.mark.parametrize(
    "shapes",
    [((70, 60, 16), (70, 60, 16), (70, 60, 16)), ((24, 700, 16), (24, 700, 16), (24, 700, 16)), ((64, 1100, 8), (64, 1100, 8), (64, 1100, 8))],
    ids=["eight-groups", "four-groups", "whole-rows"],
)
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_rows_family_lane_group_splits(hipdev, shapes, causal):
    """The small cases above split each row's keys among 16 lane groups; 70 heads of 60 rows take
    8, 24 heads of 700 rows 4, 64 heads of 1100 rows whole rows per group."""
    check_case(hipdev, 6, shapes, causal, "float32")


def test_rows_family_rectangular_keys(hipdev):
    check_case(hipdev, 2, ((40, 8), (72, 8), (72, 12)), False, "float32")


def test_rows_family_float64(hipdev):
    check_case(hipdev, 3, ((2, 64, 32), (2, 64, 32), (2, 64, 16)), True, "float64")


@pytest.mark.parametrize(
    "shapes,causal,live",
    [(((2, 100, 16), (2, 100, 16), (2, 100, 16)), True, 66), (((4, 1, 32), (4, 96, 32), (4, 96, 48)), False, 64)],
    ids=["ragged_causal", "decode_row"],
)
def test_rows_family_key_mask(hipdev, shapes, causal, live):
    _, _, _, dk, dv = check_case(hipdev, 4, shapes, causal, "float32", live)
    assert (dk[..., live:, :] == 0).all() and (dv[..., live:, :] == 0).all()


# MFMA family: bf16/f16 at D = 64 and 128
MFMA_CASES = {
    "d64_ragged": ((2, 2, 200, 64), (2, 2, 200, 64), (2, 2, 200, 64)),
    # causal D = 64 workgroups take a 128-row block and its mirror: three blocks leave the middle
    # one paired with itself, four are the GPT step's heads (512 rows), five end ragged
    "d64_three_blocks": ((1, 2, 384, 64), (1, 2, 384, 64), (1, 2, 384, 64)),
    "d64_four_blocks": ((2, 1, 512, 64), (2, 1, 512, 64), (2, 1, 512, 64)),
    "d64_five_ragged": ((1, 1, 600, 64), (1, 1, 600, 64), (1, 1, 600, 64)),
    "d128_two_blocks": ((1, 2, 256, 128), (1, 2, 256, 128), (1, 2, 256, 128)),
    "d128_ragged": ((2, 1, 333, 128), (2, 1, 333, 128), (2, 1, 333, 128)),
    # long heads: 10 and 13 query tiles per key block, tile loops unrolled by two with an odd
    # count, a ragged last tile past the diagonal
    "d128_long": ((1, 2, 640, 128), (1, 2, 640, 128), (1, 2, 640, 128)),
    "d128_long_ragged": ((1, 1, 801, 128), (1, 1, 801, 128), (1, 1, 801, 128)),
    # one and two 64-key tiles: the software-pipelined forward's prologue and last step with no
    # steady-state step between them
    "d128_one_tile": ((2, 1, 40, 128), (2, 1, 40, 128), (2, 1, 40, 128)),
    "d128_two_tiles": ((1, 2, 100, 128), (1, 2, 100, 128), (1, 2, 100, 128)),
}


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("case", sorted(MFMA_CASES))
def test_mfma_family_matches_the_oracle(hipdev, case, causal, dtype_name):
    check_case(hipdev, 5, MFMA_CASES[case], causal, dtype_name)


def test_mfma_family_rectangular_keys(hipdev):
    check_case(hipdev, 6, ((3, 70, 64), (3, 190, 64), (3, 190, 64)), False, "bfloat16")


@pytest.mark.parametrize("t_q,t_k", [(70, 390), (390, 70)])
def test_mfma_family_rectangular_d128(hipdev, t_q, t_k):
    check_case(hipdev, 8, ((2, t_q, 128), (2, t_k, 128), (2, t_k, 128)), False, "bfloat16")


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_mfma_family_key_mask(hipdev, causal):
    shapes = ((2, 150, 128), (2, 150, 128), (2, 150, 128))
    _, _, _, dk, dv = check_case(hipdev, 7, shapes, causal, "bfloat16", live=97)
    assert (dk[..., 97:, :] == 0).all() and (dv[..., 97:, :] == 0).all()


@pytest.mark.parametrize("dtype_name,hd", [("bfloat16", 128), ("float32", 64)])
def test_same_bits_twice(hipdev, dtype_name, hd):
    """Every total is owned by one wave and folded in a fixed order: no atomics, same bits."""
    q, k, v, do, _ = draw(8, (2, 2, 300, hd), (2, 2, 300, hd), (2, 2, 300, hd), dtype_name)
    first = forward(hipdev, q, k, v, None, True, dtype_name)
    second = forward(hipdev, q, k, v, None, True, dtype_name)
    for a, b in zip(first, second):
        np.testing.assert_array_equal(a, b)
    out, lse = first
    delta = (do * out).sum(axis=-1, keepdims=True).astype(lse.dtype)
    g1 = backward(hipdev, q, k, v, do, lse, delta, None, True, dtype_name)
    g2 = backward(hipdev, q, k, v, do, lse, delta, None, True, dtype_name)
    for a, b in zip(g1, g2):
        np.testing.assert_array_equal(a, b)


def test_config1_matches_torch_golden(hipdev):
    """BASELINE config 1 end to end: f32 causal B=2 H=4 S=256 D=64 from seed 1, forward and
    backward (delta from the GPU forward), against torch's float64 answer."""
    rng = np.random.default_rng(1)
    shape = (2, 4, 256, 64)
    q, k, v, do = (rng.standard_normal(shape, dtype=np.float32) for _ in range(4))
    out, lse = forward(hipdev, q, k, v, None, True, "float32")
    delta = (do * out).sum(axis=-1, keepdims=True)
    dq, dk, dv = backward(hipdev, q, k, v, do, lse, delta, None, True, "float32")
    g = np.load(GOLDEN / "config1_sdpa.npz")
    for key, val, tol in (("o", out, 1e-5), ("lse", lse, 1e-5), ("dq", dq, 1e-4), ("dk", dk, 1e-4), ("dv", dv, 1e-4)):
        assert ref.worst(val[0, 0], g[f"{key}_slice"]) <= tol, key
        np.testing.assert_allclose(float((val.astype(np.float64) ** 2).sum()), float(g[f"{key}_sumsq"]), rtol=1e-4)


def _poisoned_pool(dev, sizes) -> None:
    """Return buffers of these sizes to the device's pool filled with 0xFF bytes (NaN in bf16 and
    f32): the next outputs of those sizes start as NaN, so a cell a kernel never writes fails
    the finiteness check instead of passing on stale finite bytes."""
    held = [dev._alloc(n) for n in sizes]
    for buf in held:
        dev.copyin(buf, np.full(buf.nbytes, 0xFF, dtype=np.uint8))
    del held


# One head from each of the eight runs head_and_block gives the XCDs (16 consecutive heads each
# at C4), plus the last head; flat index b * H + h.
C4_HEADS = (0, 21, 42, 63, 68, 89, 110, 127)


def test_config4_full_size_every_xcd(hipdev):
    """BASELINE config 4 at its full shape (bf16, causal, B=8 H=16 S=4096 D=128, seed 4).

    Every output starts as NaN bytes and must come back finite (all 128 heads, forward and
    backward). The kernels number workgroups head-major per XCD (each XCD a run of 16 heads), so
    one head of every run is diffed against the oracle, forward and backward."""
    from limn_amd.dtypes import bf16_bits, bf16_values

    B, H, S, D = 8, 16, 4096, 128
    rng = np.random.default_rng(4)

    def rnd():
        return bf16_values(bf16_bits(rng.standard_normal((B, H, S, D), dtype=np.float32)))

    q, k, v, do = rnd(), rnd(), rnd(), rnd()
    scale = D**-0.5
    big, stat = B * H * S * D * 2, B * H * S * 4
    q_n, k_n, v_n, do_n = (upload(hipdev, x, bfloat16) for x in (q, k, v, do))
    print("C4 forward, NaN-poisoned outputs", flush=True)
    _poisoned_pool(hipdev, [big, stat])
    o_node, l_node = custom("sdpa", (q_n, k_n, v_n), (True, scale), ((bfloat16, q.shape), (float32, (B, H, S, 1))))
    bo, bl = hipdev.execute([o_node, l_node])
    out, lse = download(hipdev, bo, bfloat16, q.shape), download(hipdev, bl, float32, (B, H, S, 1))
    assert np.isfinite(out).all() and np.isfinite(lse).all()
    delta = (do * out).sum(axis=-1, keepdims=True).astype(np.float32)
    srcs = (q_n, k_n, v_n, do_n, upload(hipdev, lse, float32), upload(hipdev, delta, float32))
    print("C4 backward, NaN-poisoned outputs", flush=True)
    _poisoned_pool(hipdev, [big, big, big])
    (dq_n,) = custom("sdpa_bwd_q", srcs, (True, scale), ((bfloat16, q.shape),))
    dk_n, dv_n = custom("sdpa_bwd_kv", srcs, (True, scale), ((bfloat16, q.shape), (bfloat16, q.shape)))
    dq, dk, dv = (download(hipdev, b, bfloat16, q.shape) for b in hipdev.execute([dq_n, dk_n, dv_n]))
    for g in (dq, dk, dv):
        assert np.isfinite(g).all()
    for flat in C4_HEADS:
        b, h = divmod(flat, H)
        args = [x[b, h] for x in (q, k, v)]
        want_out, want_lse = ref.sdpa(*args, causal=True, scale=scale, dtype="bfloat16", block_size=256)
        np.testing.assert_allclose(out[b, h], want_out, rtol=1e-2, atol=1e-2, err_msg=f"O head {flat}")
        np.testing.assert_allclose(lse[b, h], want_lse, rtol=1e-2, atol=1e-2, err_msg=f"L head {flat}")
        bargs = (*args, do[b, h], lse[b, h], delta[b, h])
        want_dq = ref.sdpa_backward_q(*bargs, causal=True, scale=scale, dtype="bfloat16", block_size=256)
        want_dk, want_dv = ref.sdpa_backward_kv(*bargs, causal=True, scale=scale, dtype="bfloat16", block_size=256)
        for name, got, want in (("dQ", dq[b, h], want_dq), ("dK", dk[b, h], want_dk), ("dV", dv[b, h], want_dv)):
            np.testing.assert_allclose(got, want, rtol=3e-2, atol=3e-2, err_msg=f"{name} head {flat}")


# The dS hand-off route (limn_hip_sdpa_bwd): D = 128 without a key mask, causal or with whole
# 128-key blocks; ragged query tiles, several key blocks, rectangular non-causal.
HANDOFF_CASES = {
    "causal_ragged": (((2, 1, 333, 128), (2, 1, 333, 128), (2, 1, 333, 128)), True),
    "causal_long": (((1, 2, 640, 128), (1, 2, 640, 128), (1, 2, 640, 128)), True),
    "full_square": (((1, 2, 384, 128), (1, 2, 384, 128), (1, 2, 384, 128)), False),
    "full_ragged_queries": (((2, 200, 128), (2, 256, 128), (2, 256, 128)), False),
}


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16"])
@pytest.mark.parametrize("case", sorted(HANDOFF_CASES))
def test_paired_backward_hands_ds_to_the_dq_pass(hipdev, case, dtype_name):
    """An sdpa_bwd_q / sdpa_bwd_kv pair on the same inputs is one call of the plan, whose dK/dV
    pass hands dS to the dQ pass. It matches the oracle; against the two passes run on their
    own, dK and dV come from the same dK/dV pass (the same bits) and dQ from the other route
    (within the bf16 tolerance); and it gives the same bits twice."""
    from limn_amd.seam import topological

    shapes, causal = HANDOFF_CASES[case]
    q, k, v, do, _ = draw(9, *shapes, dtype_name)
    scale = q.shape[-1] ** -0.5
    out, lse = forward(hipdev, q, k, v, None, causal, dtype_name)
    delta = (do.astype(np.float64) * out).sum(axis=-1, keepdims=True).astype(lse.dtype)
    nodes = backward_nodes(hipdev, q, k, v, do, lse, delta, None, causal, dtype_name)
    order = topological(list(nodes))
    plan = hipdev.plan_of(order, {n: i for i, n in enumerate(order)}, list(nodes))
    assert len(plan.calls) == 1 and len(plan.calls[0].outputs) == 3, "the pair runs as one call"
    paired = backward(hipdev, q, k, v, do, lse, delta, None, causal, dtype_name)
    args = (q, k, v, do, lse, delta, None)
    want = [ref.sdpa_backward_q(*args, causal=causal, scale=scale, dtype=dtype_name),
            *ref.sdpa_backward_kv(*args, causal=causal, scale=scale, dtype=dtype_name)]
    tol = BWD_TOL[dtype_name]
    for name, got, w in zip(("dq", "dk", "dv"), paired, want):
        np.testing.assert_allclose(got, w, rtol=tol, atol=tol, err_msg=name)
    alone = backward_separately(hipdev, q, k, v, do, lse, delta, None, causal, dtype_name)
    np.testing.assert_array_equal(paired[1], alone[1], err_msg="dk")
    np.testing.assert_array_equal(paired[2], alone[2], err_msg="dv")
    np.testing.assert_allclose(paired[0], alone[0], rtol=tol, atol=tol, err_msg="dq")
    again = backward(hipdev, q, k, v, do, lse, delta, None, causal, dtype_name)
    for a, b in zip(paired, again):
        np.testing.assert_array_equal(a, b)


HIDDEN_FAMILIES = {"rows_f32": ("float32", 16), "mfma_d64_bf16": ("bfloat16", 64), "mfma_d128_bf16": ("bfloat16", 128)}


@pytest.mark.parametrize("family", sorted(HIDDEN_FAMILIES))
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_a_batch_row_with_every_key_hidden(hipdev, family, causal):
    """A query row with no visible key gives NaN and L = -inf (reference limn/sdpa.py:110-112,
    126-129). Batch row 0 hides every key, batch row 1 a run of keys. The backward is NaN exactly
    where the numpy reference's is (every probability of a row with L = -inf is
    exp(-inf - (-inf))): all of batch row 0's dQ, dK and dV; batch row 1 matches the reference,
    its hidden keys with exactly zero dK and dV."""
    dtype_name, hd = HIDDEN_FAMILIES[family]
    shape = (2, 150, hd)
    q, k, v, do, _ = draw(10, shape, shape, shape, dtype_name)
    mask = np.ones((2, 150), np.float64 if dtype_name == "float64" else np.float32)
    mask[0] = 0
    mask[1, 40:90] = 0
    scale = hd**-0.5
    out, lse = forward(hipdev, q, k, v, mask, causal, dtype_name)
    want_out, want_lse = ref.sdpa(q, k, v, mask, causal=causal, scale=scale, dtype=dtype_name)
    assert np.isnan(want_out[0]).all() and np.isneginf(want_lse[0]).all()
    assert np.isnan(out[0]).all() and np.isneginf(lse[0]).all()
    tol = FWD_TOL[dtype_name]
    np.testing.assert_allclose(out[1], want_out[1], rtol=tol, atol=tol)
    np.testing.assert_allclose(lse[1], want_lse[1], rtol=tol, atol=tol)
    with np.errstate(invalid="ignore"):
        delta = (do.astype(np.float64) * out).sum(axis=-1, keepdims=True).astype(lse.dtype)
    got = backward(hipdev, q, k, v, do, lse, delta, mask, causal, dtype_name)
    args = (q, k, v, do, lse, delta, mask)
    want = [ref.sdpa_backward_q(*args, causal=causal, scale=scale, dtype=dtype_name),
            *ref.sdpa_backward_kv(*args, causal=causal, scale=scale, dtype=dtype_name)]
    tol = BWD_TOL[dtype_name]
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        assert np.isnan(w[0]).all() and not np.isnan(w[1]).any(), name
        np.testing.assert_array_equal(np.isnan(g), np.isnan(w), err_msg=f"{name}: NaN positions")
        np.testing.assert_allclose(g[1], w[1], rtol=tol, atol=tol, err_msg=name)
    assert (got[1][1, 40:90] == 0).all() and (got[2][1, 40:90] == 0).all()
