"""A child-process probe for tests/test_seam.py: builds limn graphs with whatever IR classes
limn_amd.seam bound in this process, then either plans them for the hip device (no GPU) or runs
them on it against the numpy oracle.

    python tests/seam_probe.py plan   -> one JSON line: the binding and each graph's plan summary
    python tests/seam_probe.py run    -> one JSON line: the binding and each graph's max error

The test runs it once with a copy of limn_amd/standin imported under the name `limn` (so every
enum member and class the graphs carry is distinct from the stand-in's) and once bound to the
stand-in, and asks for identical plans and for GPU results within tolerance.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

from limn_amd import seam  # noqa: E402
from limn_amd.gpt import GPTConfig, cross_entropy, make_trainer, synthetic_batch  # noqa: E402
from oracle.numpy_device import NumpyDevice  # noqa: E402
from oracle.sdpa import worst  # noqa: E402

Tensor = seam.Tensor
TINY = GPTConfig(vocab=32, ctx=32, dim=64, layers=1, heads=2, batch=2, dtype=seam.bfloat16)


def draw(seed: int, shape: tuple[int, ...]) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def softmax_layernorm() -> list:
    x = Tensor(draw(1, (64, 96)))
    return [seam.nn.LayerNorm(96)(x.softmax(-1))]


def matmul_relu() -> list:
    a = Tensor(draw(2, (128, 64)), dtype=seam.bfloat16)
    b = Tensor(draw(3, (64, 96)), dtype=seam.bfloat16)
    return [(a @ b).relu()]


def attention() -> list:
    q, k, v = (Tensor(draw(s, (2, 2, 64, 64)), dtype=seam.bfloat16, requires_grad=True) for s in (4, 5, 6))
    w = Tensor(draw(7, (2, 2, 64, 64)))
    out = q.attention(k, v, causal=True)
    loss = (out.cast(seam.float32) * w).sum()
    return [out, *seam.grad(loss, [q, k, v])]


def embedding() -> list:
    table = Tensor(draw(8, (50, 32)), requires_grad=True)
    idx = Tensor(np.random.default_rng(9).integers(0, 50, (4, 16)).astype(np.int32))
    rows = table.gather_rows(idx)
    loss = (rows * rows).sum()
    return [rows, *seam.grad(loss, [table])]


GRAPHS = {"softmax_layernorm": softmax_layernorm, "matmul_relu": matmul_relu, "attention": attention, "embedding": embedding}


def gpt_step_sinks() -> list:
    """One training step's whole graph: forward, backward, the AdamW writes and the loss."""
    seam.set_seed(10)
    model, opt, _ = make_trainer(TINY)
    x, y = synthetic_batch(TINY, np.random.default_rng(10))
    loss = cross_entropy(model(x), y)
    loss.backward()
    with seam.no_grad():
        writes = opt.updates()
    return [t.assign(v) for t, v in writes] + [loss]


def plan_summary(tensors: list) -> dict:
    from limn_amd.hip.device import plan_context
    from limn_amd.hip.emit import plan_program

    sinks = [t.node for t in tensors]
    order = seam.topological(sinks)
    kernels = seam.schedule(sinks, order)
    nests = seam.lower_all(sinks, order, kernels)
    kept, custom_inputs = plan_context(order, sinks)
    prog = plan_program(nests, kept, custom_inputs)
    nest_rows = []
    for k, nest in enumerate(nests):
        plan = prog.plans[k]
        con = plan.contraction
        nest_rows.append([nest.name, prog.role(k), [[l.name, l.grid, l.block, l.args] for l in plan.launches],
                          None if con is None else [con.batch, con.M, con.N, con.K]])
    return {
        "kernels": len(kernels),
        "custom": sorted(k.ast.arg.name for k in kernels if k.ast.op is seam.Op.CUSTOM),
        "nests": nest_rows,
        "source_sha256": hashlib.sha256(prog.source.encode()).hexdigest(),
    }


def plan_mode() -> dict:
    seam.use_device(NumpyDevice())  # the frontend asks the active device which CUSTOM kernels exist
    out = {name: plan_summary(build()) for name, build in GRAPHS.items()}
    out["gpt_step"] = plan_summary(gpt_step_sinks())
    return out


def run_mode() -> dict:
    import limn_amd.hip  # noqa: F401  (registers "hip" in the bound registry)

    seam.set_device("hip")
    hip = seam.active_device()
    oracle = NumpyDevice()
    errors = {}
    for name, build in GRAPHS.items():
        seam.use_device(hip)
        got = [t.numpy().astype(np.float64) for t in build()]
        seam.use_device(oracle)
        want = [t.numpy().astype(np.float64) for t in build()]
        errors[name] = max(worst(g, w) for g, w in zip(got, want))
    losses = {}
    for label, dev in (("hip", hip), ("oracle", oracle)):
        seam.use_device(dev)
        seam.set_seed(11)
        _, _, step = make_trainer(TINY)
        fn = seam.capture(step)
        r = np.random.default_rng(11)
        losses[label] = [fn(*synthetic_batch(TINY, r)).item() for _ in range(4)]
    errors["gpt_steps"] = max(abs(a - b) / abs(b) for a, b in zip(losses["hip"], losses["oracle"]))
    return {"errors": errors, "losses": losses}


def main() -> None:
    mode = sys.argv[1]
    result = plan_mode() if mode == "plan" else run_mode()
    stand_in_ops = __import__("limn_amd.standin.ops", fromlist=["Op"])
    result["binding"] = {
        "package": seam.PACKAGE,
        "op_module": seam.Op.__module__,
        "distinct_from_standin": seam.Op is not stand_in_ops.Op and seam.Opcode.__module__ != "limn_amd.standin.codegen",
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
