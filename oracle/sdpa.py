"""Fused attention on the CPU, as the reference's numpy device computes it (TEST INFRASTRUCTURE
ONLY; see oracle/__init__.py).

Restates reference limn/sdpa.py:
  - `sdpa`           limn/sdpa.py:91-137  blocked online softmax over key blocks, returns (O, L);
  - `sdpa_backward_q`  limn/sdpa.py:140-170 dQ over key blocks from p = exp(s*scale - L);
  - `sdpa_backward_kv` limn/sdpa.py:173-203 dK, dV over query blocks;
  - `plain_probs`, `plain`, `plain_backward` limn/sdpa.py:227-248, the textbook forms that
    materialize the t_q x t_k, evaluated here in float64;
  - `worst`          limn/sdpa.py:251-259, max |got - want| / max(1, max |want|).

Dtypes: `dtype` names the storage width ("float64", "float32", "float16", "bfloat16"); inputs
are arrays holding values of that width (bfloat16 values carried in float32 arrays). Half
widths run the recurrence in float32 and round the outputs back once (limn/sdpa.py:48-51,
136); L and the backward statistics stay at the recurrence width.

Pinned by tests/test_oracle.py: the blocked recurrence against the float64 textbook form at
block sizes 1, 16, t and t+7 over the reference's own check() cases (limn/sdpa.py:262-318),
against torch's scaled_dot_product_attention and autograd through tests/golden/sdpa_torch.npz,
and against closed forms (causal row 0 returns v[0] with L = s00*scale; a hidden key's dK and
dV are exactly zero; a key mask equals slicing the keys away).
"""

from __future__ import annotations

import numpy as np

from oracle.bf16 import rne

WORK = {"float64": np.float64, "float32": np.float32, "float16": np.float32, "bfloat16": np.float32}


def store(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round recurrence-width values to the storage dtype (as values a float32 array can hold)."""
    if dtype == "bfloat16":
        return rne(np.asarray(x, dtype=np.float32))
    if dtype == "float16":
        return np.asarray(x).astype(np.float16)
    return np.asarray(x).astype(WORK[dtype])


def _blocks(n: int, size: int):
    return [(a, min(a + size, n)) for a in range(0, n, size)]


def _scores(a, b, rows: range, cols: range, causal: bool, scale: float, keep):
    s = a @ np.swapaxes(b, -1, -2) * scale
    if causal:
        s = np.where(np.arange(cols.start, cols.stop)[None, :] <= np.arange(rows.start, rows.stop)[:, None], s, -np.inf)
    if keep is not None:
        s = np.where(keep, s, -np.inf)
    return s


def _keep(mask, cols):
    return None if mask is None else (mask[..., None, cols] != 0)


def _check(q, k, v, mask, causal):
    if q.ndim < 2 or k.ndim != q.ndim or v.ndim != q.ndim:
        raise ValueError(f"sdpa wants 2D+ inputs of equal rank, got {q.shape}, {k.shape}, {v.shape}")
    if q.shape[:-2] != k.shape[:-2] or q.shape[:-2] != v.shape[:-2] or k.shape[-2] != v.shape[-2]:
        raise ValueError(f"sdpa shape mismatch: {q.shape}, {k.shape}, {v.shape}")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError("sdpa: head dims differ")
    if causal and q.shape[-2] != k.shape[-2]:
        raise ValueError("causal sdpa needs square keys")
    if mask is not None and mask.shape != q.shape[:-2] + k.shape[-2:-1]:
        raise ValueError(f"sdpa key mask must be {q.shape[:-2] + k.shape[-2:-1]}, got {mask.shape}")


def sdpa(q, k, v, key_mask=None, *, causal: bool, scale: float, dtype: str = "float32", block_size: int = 16):
    """(O at the storage dtype, L = logsumexp per row at the recurrence width, shape (..., t_q, 1))."""
    _check(q, k, v, key_mask, causal)
    w = WORK[dtype]
    Q, K, V = (np.asarray(x, dtype=w) for x in (q, k, v))
    t_q, t_k = Q.shape[-2], K.shape[-2]
    lead = Q.shape[:-2]
    acc = np.zeros(lead + (t_q, V.shape[-1]), dtype=w)
    m = np.full(lead + (t_q,), -np.inf, dtype=w)
    l = np.zeros(lead + (t_q,), dtype=w)
    with np.errstate(invalid="ignore", divide="ignore"):
        for a, b in _blocks(t_k, block_size):
            s = _scores(Q, K[..., a:b, :], range(t_q), range(a, b), causal, scale, _keep(key_mask, slice(a, b)))
            m_new = np.maximum(m, s.max(axis=-1))
            base = np.where(np.isneginf(m_new), w(0), m_new)  # a row with nothing seen yet keeps zeros
            alpha = np.exp(m - base)
            p = np.exp(s - base[..., None])
            l = l * alpha + p.sum(axis=-1)
            acc = acc * alpha[..., None] + p @ V[..., a:b, :]
            m = m_new
        lse = (m + np.log(l))[..., None].astype(w)
        out = acc / l[..., None]
    return store(out, dtype), lse


def sdpa_backward_q(q, k, v, do, lse, delta, key_mask=None, *, causal: bool, scale: float, dtype: str = "float32", block_size: int = 16):
    _check(q, k, v, key_mask, causal)
    w = WORK[dtype]
    Q, K, V, DO, L, D = (np.asarray(x, dtype=w) for x in (q, k, v, do, lse, delta))
    t_q, t_k = Q.shape[-2], K.shape[-2]
    dq = np.zeros(Q.shape, dtype=w)
    with np.errstate(invalid="ignore", over="ignore"):
        for a, b in _blocks(t_k, block_size):
            s = _scores(Q, K[..., a:b, :], range(t_q), range(a, b), causal, scale, _keep(key_mask, slice(a, b)))
            p = np.exp(s - L)
            dp = DO @ np.swapaxes(V[..., a:b, :], -1, -2)
            dq += (p * (dp - D) * scale) @ K[..., a:b, :]
    return store(dq, dtype)


def sdpa_backward_kv(q, k, v, do, lse, delta, key_mask=None, *, causal: bool, scale: float, dtype: str = "float32", block_size: int = 16):
    _check(q, k, v, key_mask, causal)
    w = WORK[dtype]
    Q, K, V, DO, L, D = (np.asarray(x, dtype=w) for x in (q, k, v, do, lse, delta))
    t_q, t_k = Q.shape[-2], K.shape[-2]
    dk = np.zeros(K.shape, dtype=w)
    dv = np.zeros(V.shape, dtype=w)
    with np.errstate(invalid="ignore", over="ignore"):
        for a, b in _blocks(t_q, block_size):
            Qi, DOi = Q[..., a:b, :], DO[..., a:b, :]
            s = _scores(Qi, K, range(a, b), range(t_k), causal, scale, _keep(key_mask, slice(None)))
            p = np.exp(s - L[..., a:b, :])
            dv += np.swapaxes(p, -1, -2) @ DOi
            dp = DOi @ np.swapaxes(V, -1, -2)
            dk += np.swapaxes(p * (dp - D[..., a:b, :]) * scale, -1, -2) @ Qi
    return store(dk, dtype), store(dv, dtype)


# ---- textbook forms (float64), the answers the recurrence must land on ----


def plain_probs(q, k, *, causal: bool, scale: float, key_mask=None):
    q, k = np.asarray(q, np.float64), np.asarray(k, np.float64)
    s = _scores(q, k, range(q.shape[-2]), range(k.shape[-2]), causal, scale, _keep(key_mask, slice(None)))
    e = np.exp(s - s.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def plain(q, k, v, *, causal: bool, scale: float, key_mask=None):
    return plain_probs(q, k, causal=causal, scale=scale, key_mask=key_mask) @ np.asarray(v, np.float64)


def plain_lse(q, k, *, causal: bool, scale: float, key_mask=None):
    q, k = np.asarray(q, np.float64), np.asarray(k, np.float64)
    s = _scores(q, k, range(q.shape[-2]), range(k.shape[-2]), causal, scale, _keep(key_mask, slice(None)))
    m = s.max(axis=-1, keepdims=True)
    return m + np.log(np.exp(s - m).sum(axis=-1, keepdims=True))


def plain_backward(q, k, v, do, *, causal: bool, scale: float, key_mask=None):
    """(dQ, dK, dV) of sum(do * attention(q, k, v)), materialized, float64."""
    q, k, v, do = (np.asarray(x, np.float64) for x in (q, k, v, do))
    p = plain_probs(q, k, causal=causal, scale=scale, key_mask=key_mask)
    dp = do @ np.swapaxes(v, -1, -2)
    ds = p * (dp - (dp * p).sum(axis=-1, keepdims=True)) * scale
    return ds @ k, np.swapaxes(ds, -1, -2) @ q, np.swapaxes(p, -1, -2) @ do


def worst(got, want) -> float:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(1.0, float(np.abs(want).max())))
