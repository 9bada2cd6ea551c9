"""Write the golden fixtures under tests/golden/ from torch (CPU) in this container.

torch is an independent implementation of what the oracle restates: its bfloat16 cast for the
oracle's round-to-nearest-even, and F.scaled_dot_product_attention with autograd (evaluated in
float64) for fused attention forward and backward. Every input is drawn from a named seed so
the tests regenerate inputs instead of storing them where that is cheap.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent


def bf16_cases() -> None:
    rng = np.random.default_rng(11)
    specials = np.array(
        [0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-40, -1e-40, 1.17549435e-38, 65504.0],
        dtype=np.float32,
    )
    # exact ties: low 16 bits == 0x8000, with the kept lsb both even and odd
    base = rng.integers(0, 2**15, size=256, dtype=np.uint32) << np.uint32(17)
    ties_even = (base | np.uint32(0x8000)).view(np.float32)
    ties_odd = (base | np.uint32(0x18000)).view(np.float32)
    near = (base | rng.integers(0, 2**16, size=256, dtype=np.uint32)).view(np.float32)
    normal = rng.standard_normal(2048).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 2048).astype(np.float32)
    x = np.concatenate([specials, ties_even, ties_odd, -ties_even, near, normal]).astype(np.float32)
    bits = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(HERE / "bf16_rne.npz", x=x, bits=bits)


def attention(q, k, v, do, causal: bool, mask):
    """O, L, dQ, dK, dV from torch in float64; mask is (..., t_k) of 0/1 or None."""
    tq, tk, tv, tdo = (torch.tensor(a, dtype=torch.float64, requires_grad=i < 3) for i, a in enumerate((q, k, v, do)))
    scale = q.shape[-1] ** -0.5
    attn_mask = None
    if mask is not None:
        keep = torch.tensor(mask != 0)[..., None, :]
        if causal:
            tri = torch.ones(q.shape[-2], k.shape[-2], dtype=torch.bool).tril()
            keep = keep & tri
        attn_mask = keep.expand(*q.shape[:-1], k.shape[-2])
    out = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=attn_mask, is_causal=causal and mask is None, scale=scale)
    (out * tdo).sum().backward()
    s = (tq @ tk.transpose(-1, -2)) * scale
    if attn_mask is not None:
        s = s.masked_fill(~attn_mask, float("-inf"))
    elif causal:
        s = s.masked_fill(~torch.ones_like(s, dtype=torch.bool).tril(), float("-inf"))
    lse = torch.logsumexp(s, dim=-1, keepdim=True)
    return [t.detach().numpy() for t in (out, lse, tq.grad, tk.grad, tv.grad)]


def sdpa_cases() -> None:
    """Small cases covering the shapes the reference's tests hold attention to: batched causal,
    plain 2D, rectangular keys, ragged tails, key masks (padding and holes), hd != hd_v."""
    rng = np.random.default_rng(5)
    cases = {
        "causal_batched": ((2, 3, 64, 16), (2, 3, 64, 16), (2, 3, 64, 24), True, None),
        "full_2d": ((64, 32), (64, 32), (64, 48), False, None),
        "rectangular": ((2, 40, 8), (2, 72, 8), (2, 72, 12), False, None),
        "ragged_causal": ((2, 2, 100, 16), (2, 2, 100, 16), (2, 2, 100, 24), True, None),
        "padded_causal": ((2, 3, 32, 8), (2, 3, 32, 8), (2, 3, 32, 8), True, "pad21"),
        "holes_full": ((2, 48, 16), (2, 48, 16), (2, 48, 16), False, "holes"),
        "decode_row": ((4, 1, 32), (4, 96, 32), (4, 96, 48), False, "pad64"),
        "d64_causal": ((1, 2, 160, 64), (1, 2, 160, 64), (1, 2, 160, 64), True, None),
        "d128_full": ((1, 2, 96, 128), (1, 2, 96, 128), (1, 2, 96, 128), False, None),
    }
    out = {}
    for name, (qs, ks, vs, causal, mask_kind) in cases.items():
        q, k, v = (rng.standard_normal(s).astype(np.float32) for s in (qs, ks, vs))
        do = rng.standard_normal(qs[:-1] + vs[-1:]).astype(np.float32)
        mask = None
        if mask_kind is not None:
            t_k = ks[-2]
            if mask_kind.startswith("pad"):
                mask = np.broadcast_to(np.arange(t_k) < int(mask_kind[3:]), qs[:-2] + (t_k,)).astype(np.float32)
            else:
                mask = (rng.random(qs[:-2] + (t_k,)) > 0.3).astype(np.float32)
                mask[..., 0] = 1.0  # no row may lose every key
        o, lse, dq, dk, dv = attention(q, k, v, do, causal, mask)
        for key, val in (("q", q), ("k", k), ("v", v), ("do", do), ("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
            out[f"{name}/{key}"] = val.astype(np.float32)
        out[f"{name}/causal"] = np.array(causal)
        if mask is not None:
            out[f"{name}/mask"] = np.ascontiguousarray(mask)
    np.savez_compressed(HERE / "sdpa_torch.npz", **out)


def config1() -> None:
    """causal sdpa f32, B=2, H=4, S=256, D=64, inputs N(0,1) from
    default_rng(1) drawn in the order q, k, v, dO. Stored: the (b=0, h=0) slice of each output
    and, per output, the float64 sum and sum of squares over the whole tensor."""
    rng = np.random.default_rng(1)
    shape = (2, 4, 256, 64)
    q, k, v, do = (rng.standard_normal(shape, dtype=np.float32) for _ in range(4))
    o, lse, dq, dk, dv = attention(q, k, v, do, True, None)
    out = {}
    for key, val in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        out[f"{key}_slice"] = val[0, 0].astype(np.float32)
        out[f"{key}_sum"] = np.float64(val.sum())
        out[f"{key}_sumsq"] = np.float64((val * val).sum())
    np.savez_compressed(HERE / "config1_sdpa.npz", **out)


if __name__ == "__main__":
    bf16_cases()
    sdpa_cases()
    config1()
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)
