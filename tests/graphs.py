"""The graph corpus every device is run through (the reference's tests/conftest.py:76-93 set),
and the check that diffs a device against the numpy oracle on the same graph."""

from __future__ import annotations

import numpy as np

from limn_amd.seam import HALF_FLOATS
from limn_amd.seam import device as limn_device
from limn_amd.dtypes import from_storage
from oracle.numpy_device import NumpyDevice

limn_device.DEVICES["numpy"] = NumpyDevice

GRAPHS = {
    "elementwise": lambda a, b: (a + b) * 2.0 - a,
    "relu": lambda a, b: (a * b).relu() + 1.0,
    "unary math": lambda a, b: (a * a + 1.0).log().exp().sqrt(),
    "divide": lambda a, b: a / (b * b + 0.5),
    "where": lambda a, b: (a < b).where(a, b),
    "cast round trip": lambda a, b: (a * 4.0).int().float() + 0.5,
    "sum an axis": lambda a, b: (a + b).sum(axis=1),
    "sum everything": lambda a, b: (a * b).sum(),
    "max keepdim": lambda a, b: (a * b).max(axis=0, keepdim=True),
    "mean": lambda a, b: (a + b).mean(axis=1),
    "matmul": lambda a, b: a @ b.transpose(),
    "softmax": lambda a, b: (a + b).softmax(axis=1),
    "log softmax": lambda a, b: (a * b).log_softmax(axis=0),
    "padded reduce": lambda a, b: a.pad(((1, 1), (0, 2))).sum(axis=1),
    "movement then reduce": lambda a, b: (a.transpose() * 2.0).sum(axis=0),
    "reduce then elementwise": lambda a, b: (a.sum(axis=1, keepdim=True) * b).relu(),
}


def check(dev, t, rtol: float = 1e-5, atol: float = 1e-5, exact: bool = False, worst: float | None = None, bitwise: bool = False) -> None:
    """Realize `t` on `dev` first, then on the numpy oracle (which retires the node), and diff
    (reference tests/conftest.py:52-69). Half widths compare widened to float32. With `worst`,
    the bound is on max|got - want| / max(1, max|want|) instead (reference limn/sdpa.py:251-259):
    for sums whose terms cancel, where no per-element relative bound holds across orders. With
    `bitwise`, the stored bytes must be identical (a -0.0 or a NaN payload counts)."""
    got = from_storage(dev.copyout(dev.execute([t.node])[0]), t.dtype, t.shape)
    saved = limn_device.active_device
    limn_device.active_device = NumpyDevice()
    try:
        want = t.numpy()
    finally:
        limn_device.active_device = saved
    if bitwise:
        assert got.dtype == want.dtype and got.shape == want.shape, (got.dtype, want.dtype, got.shape, want.shape)
        g, w = np.ascontiguousarray(got).reshape(-1), np.ascontiguousarray(want).reshape(-1)
        differ = np.any(g.view(np.uint8).reshape(g.size, -1) != w.view(np.uint8).reshape(w.size, -1), axis=1)
        bad = np.flatnonzero(differ)
        assert bad.size == 0, f"{bad.size} of {g.size} values differ in their bits; first at {bad[:5]}: got {g[bad[:5]]}, want {w[bad[:5]]}"
        return
    if exact:
        np.testing.assert_array_equal(got, want)
        return
    if t.dtype in HALF_FLOATS:
        got, want = got.astype(np.float32), want.astype(np.float32)
    if worst is not None:
        err = float(np.max(np.abs(got.astype(np.float64) - want))) / max(1.0, float(np.max(np.abs(want))))
        assert err <= worst, f"worst error {err:.3g} > {worst:.3g}"
        return
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)
