"""Pins for the oracle itself (CPU only): before the HIP kernels are diffed against it, it is
held to torch's golden vectors, to the textbook forms at the reference's own check() cases, and
to closed forms a plausible mistake would break."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import bf16
from oracle import sdpa as ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_bf16_round_to_nearest_even_matches_torch():
    data = np.load(GOLDEN / "bf16_rne.npz")
    got = bf16.round_bits(data["x"])
    want = data["bits"]
    nan = np.isnan(data["x"])
    np.testing.assert_array_equal(got[~nan], want[~nan])
    assert np.isnan(bf16.widen(got[nan])).all()


def test_product_bf16_storage_matches_the_oracle():
    """The host-side conversion the product uses to build bfloat16 tensors agrees bit for bit."""
    from limn_amd.dtypes import bf16_bits

    data = np.load(GOLDEN / "bf16_rne.npz")
    x = data["x"]
    nan = np.isnan(x)
    np.testing.assert_array_equal(bf16_bits(x)[~nan], data["bits"][~nan])
    assert np.isnan(bf16.widen(bf16_bits(x)[nan])).all()


def _golden_cases():
    data = np.load(GOLDEN / "sdpa_torch.npz")
    names = sorted({k.split("/")[0] for k in data.files})
    return data, names


@pytest.mark.parametrize("name", _golden_cases()[1])
def test_oracle_matches_torch(name):
    data, _ = _golden_cases()
    g = {k.split("/")[1]: data[k] for k in data.files if k.startswith(name + "/")}
    causal = bool(g["causal"])
    mask = g.get("mask")
    scale = g["q"].shape[-1] ** -0.5
    out, lse = ref.sdpa(g["q"], g["k"], g["v"], mask, causal=causal, scale=scale)
    assert ref.worst(out, g["o"]) <= 1e-5
    assert ref.worst(lse, g["lse"]) <= 1e-5
    delta = (g["do"] * out).sum(axis=-1, keepdims=True)
    dq = ref.sdpa_backward_q(g["q"], g["k"], g["v"], g["do"], lse, delta, mask, causal=causal, scale=scale)
    dk, dv = ref.sdpa_backward_kv(g["q"], g["k"], g["v"], g["do"], lse, delta, mask, causal=causal, scale=scale)
    for got, want in ((dq, g["dq"]), (dk, g["dk"]), (dv, g["dv"])):
        assert ref.worst(got, want) <= 1e-4


def test_config1_golden_against_the_oracle():
    """BASELINE config 1 (f32 causal, B=2 H=4 S=256 D=64, seed 1): the oracle reproduces torch's
    (b=0, h=0) slice and the whole-tensor sums."""
    rng = np.random.default_rng(1)
    shape = (2, 4, 256, 64)
    q, k, v, do = (rng.standard_normal(shape, dtype=np.float32) for _ in range(4))
    g = np.load(GOLDEN / "config1_sdpa.npz")
    out, lse = ref.sdpa(q, k, v, causal=True, scale=0.125)
    delta = (do * out).sum(axis=-1, keepdims=True)
    dq = ref.sdpa_backward_q(q, k, v, do, lse, delta, causal=True, scale=0.125)
    dk, dv = ref.sdpa_backward_kv(q, k, v, do, lse, delta, causal=True, scale=0.125)
    for key, val, tol in (("o", out, 1e-5), ("lse", lse, 1e-5), ("dq", dq, 1e-4), ("dk", dk, 1e-4), ("dv", dv, 1e-4)):
        assert ref.worst(val[0, 0], g[f"{key}_slice"]) <= tol, key
        assert abs(float(val.astype(np.float64).sum()) - float(g[f"{key}_sum"])) <= tol * max(1.0, np.abs(val).sum()) * 1e-1
        np.testing.assert_allclose(float((val.astype(np.float64) ** 2).sum()), float(g[f"{key}_sumsq"]), rtol=1e-4)


def _check_cases():
    """The reference's own self-check cases (limn/sdpa.py:262-285), as shapes and tolerances."""
    rng = np.random.default_rng(0)

    def r(*s, dtype=np.float32):
        return rng.standard_normal(s).astype(dtype)

    q, k, v = r(2, 3, 128, 32), r(2, 3, 128, 32), r(2, 3, 128, 48)
    pad = np.arange(128) < 77
    holes = (rng.random((2, 3, 128)) > 0.3).astype(np.float32)
    return [
        (q, k, v, None, True, 1e-5, "float32"),
        (q, k, v, None, False, 1e-5, "float32"),
        (r(64, 200, 16), r(64, 160, 16), r(64, 160, 48), None, False, 1e-5, "float32"),
        (r(100, 32), r(100, 32), r(100, 32), None, False, 1e-5, "float32"),
        (r(256, 64) * 100.0, r(256, 64), r(256, 64), None, True, 1e-4, "float32"),
        (r(2, 64, 32, dtype=np.float64), r(2, 64, 32, dtype=np.float64), r(2, 64, 16, dtype=np.float64), None, True, 1e-12, "float64"),
        (q, k, v, np.broadcast_to(pad, (2, 3, 128)).astype(np.float32), True, 1e-5, "float32"),
        (q, k, v, holes, False, 1e-5, "float32"),
        (r(4, 1, 32), r(4, 96, 32), r(4, 96, 48), np.broadcast_to(np.arange(96) < 61, (4, 96)).astype(np.float32), False, 1e-5, "float32"),
        # the half widths: inputs rounded to storage, the textbook form run widened on those values
        (*(r(*s).astype(np.float16).astype(np.float32) for s in ((2, 3, 128, 32), (2, 3, 128, 32), (2, 3, 128, 48))), None, True, 2e-3, "float16"),
        (*(bf16.rne(r(*s)) for s in ((2, 3, 128, 32), (2, 3, 128, 32), (2, 3, 128, 48))), None, True, 2e-2, "bfloat16"),
    ]


@pytest.mark.parametrize("case", range(11))
def test_blocked_recurrence_equals_the_textbook_form(case):
    """limn/sdpa.py's check(): every block size (1, 16, t, t+7) lands on the materialized form,
    for all eleven of its cases (f32, f64, f16, bf16, masks, ragged and rectangular shapes)."""
    q, k, v, mask, causal, tol, dtype = _check_cases()[case]
    rng = np.random.default_rng(case)
    scale = q.shape[-1] ** -0.5
    do = rng.standard_normal(q.shape[:-1] + v.shape[-1:]).astype(q.dtype)
    stored_do = ref.store(do, dtype).astype(q.dtype)  # the backward reads dO at the storage width
    want = ref.plain(q, k, v, causal=causal, scale=scale, key_mask=mask)
    want_grads = ref.plain_backward(q, k, v, do, causal=causal, scale=scale, key_mask=mask)
    for block in (1, 16, k.shape[-2], k.shape[-2] + 7):
        out, lse = ref.sdpa(q, k, v, mask, causal=causal, scale=scale, dtype=dtype, block_size=block)
        assert ref.worst(out, want) <= tol
        assert ref.worst(lse, ref.plain_lse(q, k, causal=causal, scale=scale, key_mask=mask)) <= tol
        delta = (do * out).sum(axis=-1, keepdims=True)
        args = (q, k, v, stored_do, lse, delta, mask)
        dq = ref.sdpa_backward_q(*args, causal=causal, scale=scale, dtype=dtype, block_size=block)
        dk, dv = ref.sdpa_backward_kv(*args, causal=causal, scale=scale, dtype=dtype, block_size=block)
        for got, w in zip((dq, dk, dv), want_grads):
            assert ref.worst(got, w) <= tol * 10


def test_closed_form_causal_first_row():
    """Causal row 0 sees only key 0: O[0] = V[0] exactly and L[0] = s00 * scale."""
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((3, 17, 8)) for _ in range(3))
    out, lse = ref.sdpa(q, k, v, causal=True, scale=0.5, dtype="float64")
    np.testing.assert_array_equal(out[:, 0], v[:, 0])
    np.testing.assert_allclose(lse[:, 0, 0], (q[:, 0] * k[:, 0]).sum(-1) * 0.5, rtol=1e-14)


def test_closed_form_uniform_keys():
    """Identical keys give uniform probabilities: O is the mean of V and L = s + log(t_k)."""
    rng = np.random.default_rng(6)
    q = rng.standard_normal((5, 8))
    k = np.tile(rng.standard_normal((1, 8)), (12, 1))
    v = rng.standard_normal((12, 3))
    out, lse = ref.sdpa(q, k, v, causal=False, scale=1.0, dtype="float64")
    np.testing.assert_allclose(out, np.tile(v.mean(0), (5, 1)), rtol=1e-12)
    np.testing.assert_allclose(lse[:, 0], q @ k[0] + np.log(12), rtol=1e-12)


def test_a_hidden_key_gets_exactly_zero_gradient():
    rng = np.random.default_rng(8)
    q, k, v, do = (rng.standard_normal((2, 20, 8)).astype(np.float32) for _ in range(4))
    mask = np.broadcast_to(np.arange(20) < 12, (2, 20)).astype(np.float32)
    out, lse = ref.sdpa(q, k, v, mask, causal=False, scale=8**-0.5)
    delta = (do * out).sum(-1, keepdims=True)
    dk, dv = ref.sdpa_backward_kv(q, k, v, do, lse, delta, mask, causal=False, scale=8**-0.5)
    assert (dk[:, 12:] == 0).all() and (dv[:, 12:] == 0).all()


def test_a_key_mask_equals_slicing_the_keys():
    rng = np.random.default_rng(9)
    q, k, v, do = (rng.standard_normal((2, 24, 8)).astype(np.float32) for _ in range(4))
    mask = np.broadcast_to(np.arange(24) < 15, (2, 24)).astype(np.float32)
    out_m, lse_m = ref.sdpa(q, k, v, mask, causal=False, scale=8**-0.5)
    out_s, lse_s = ref.sdpa(q, k[:, :15], v[:, :15], causal=False, scale=8**-0.5)
    np.testing.assert_allclose(out_m, out_s, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(lse_m, lse_s, rtol=1e-6, atol=1e-6)


def test_a_planted_mistake_is_caught():
    """A dropped scale in the backward (a plausible slip) must fail the textbook comparison."""
    rng = np.random.default_rng(10)
    q, k, v, do = (rng.standard_normal((2, 32, 8)) for _ in range(4))
    out, lse = ref.sdpa(q, k, v, causal=True, scale=0.3, dtype="float64")
    delta = (do * out).sum(-1, keepdims=True)
    wrong = ref.sdpa_backward_q(q, k, v, do, lse, delta, causal=True, scale=1.0, dtype="float64")
    want = ref.plain_backward(q, k, v, do, causal=True, scale=0.3)[0]
    assert ref.worst(wrong, want) > 1e-3
