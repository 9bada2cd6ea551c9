"""The drop-in boundary: the hip device works on IR objects it did not define.

limn hands the device its own Node/Op/DType/LoopNest/Opcode objects (reference
`limn/jit.py:103-142`, `limn/device.py:182-220`), and the device's checks (`node.op is Op.SUM`)
only hold against those very classes. limn_amd.seam binds them; these tests make a second,
separately imported copy of the IR (limn_amd/standin copied under the name `limn`, so its enums,
dtypes and classes have identities of their own, as limn's will) and check that:

- product code reaches limn's names only through the seam;
- a child process bound to the copy plans softmax/LayerNorm, a bf16 contraction with its relu,
  attention forward and backward, an embedding gradient and a whole GPT training step exactly as
  a process bound to the stand-in does (same roles, launches, contractions, and byte-identical
  kernel source);
- on the GPU, those graphs run through the hip device bound to the copy and match the numpy
  oracle bound to the same copy.
"""

from __future__ import annotations

import ast
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PROBE = Path(__file__).resolve().parent / "seam_probe.py"


def _foreign_limn(tmp: Path) -> Path:
    """A directory holding a package `limn` that is a copy of the stand-in."""
    shutil.copytree(ROOT / "limn_amd" / "standin", tmp / "limn", ignore=shutil.ignore_patterns("__pycache__"))
    return tmp


def _probe(mode: str, bind: str, path: Path | None = None, timeout: int = 300) -> dict:
    env = dict(os.environ, LIMN_AMD_BIND=bind)
    if path is not None:
        env["PYTHONPATH"] = os.pathsep.join([str(path), env.get("PYTHONPATH", "")])
    done = subprocess.run([sys.executable, "-u", str(PROBE), mode], env=env, capture_output=True, text=True, timeout=timeout, cwd=ROOT)
    assert done.returncode == 0, done.stdout[-2000:] + done.stderr[-6000:]
    return json.loads(done.stdout.strip().splitlines()[-1])


def _imports(path: Path) -> list[str]:
    tree = ast.parse(path.read_text())
    found = []
    for node in ast.walk(tree):
        if isinstance(node, ast.Import):
            found += [a.name for a in node.names]
        elif isinstance(node, ast.ImportFrom) and node.module and node.level == 0:
            found.append(node.module)
    return found


def test_product_code_reaches_limn_only_through_the_seam():
    files = [p for p in (ROOT / "limn_amd").rglob("*.py") if "standin" not in p.parts and p.name != "seam.py"]
    files += list((ROOT / "oracle").glob("*.py")) + [ROOT / "bench.py", ROOT / "__graft_entry__.py"]
    files += [p for p in (ROOT / "tests").glob("*.py") if p.name not in ("test_seam.py", "seam_probe.py")]
    offenders = []
    for path in files:
        for module in _imports(path):
            if module == "limn" or module.startswith(("limn.", "limn_amd.standin")):
                offenders.append(f"{path.relative_to(ROOT)} imports {module}")
    assert not offenders, offenders


def test_standin_imports_only_itself():
    """The stand-in must be copyable as `limn`: no absolute import of this package inside it."""
    for path in (ROOT / "limn_amd" / "standin").glob("*.py"):
        assert not [m for m in _imports(path) if m.startswith("limn")], path.name


def test_plans_match_under_a_foreign_ir_copy(tmp_path):
    foreign = _probe("plan", "limn", _foreign_limn(tmp_path))
    native = _probe("plan", "standin")
    assert foreign["binding"] == {"package": "limn", "op_module": "limn.ops", "distinct_from_standin": True}
    assert native["binding"]["package"] == "limn_amd.standin"
    graphs = ("softmax_layernorm", "matmul_relu", "attention", "embedding", "gpt_step")
    for name in graphs:
        assert foreign[name] == native[name], name
    roles = {name: {row[1] for row in foreign[name]["nests"]} for name in graphs}
    assert {"stash", "epilogue"} <= roles["matmul_relu"]  # contraction found, relu fused into its store
    assert "inlined" in roles["softmax_layernorm"]  # the row statistics evaluated in their readers
    assert sorted(set(foreign["attention"]["custom"])) == ["sdpa", "sdpa_bwd_kv", "sdpa_bwd_q"]
    assert {"contraction", "inlined", "merged", "deferred", "launch"} <= roles["gpt_step"]
    assert any("_sort" in launch[0] for row in foreign["embedding"]["nests"] for launch in row[2])  # ordered scatter


@pytest.mark.gpu
def test_foreign_ir_graphs_run_on_the_hip_device(tmp_path):
    print("seam probe: run mode bound to a foreign copy of the IR", flush=True)
    got = _probe("run", "limn", _foreign_limn(tmp_path), timeout=600)
    assert got["binding"]["distinct_from_standin"]
    tol = {"softmax_layernorm": 1e-4, "matmul_relu": 2e-2, "attention": 3e-2, "embedding": 1e-5, "gpt_steps": 3e-2}
    for name, bound in tol.items():
        assert got["errors"][name] <= bound, (name, got["errors"])
