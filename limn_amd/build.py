"""Build the hand-written kernel library (liblimn_hip.so) in-tree with hipcc for gfx950.

`python -m limn_amd.build` compiles every `csrc/*.hip` to an object under `limn_amd/_build/`
(in parallel) and links them into `limn_amd/liblimn_hip.so`, next to the package that loads
it. Objects are rebuilt when their source or a header is newer; the library is always relinked.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
INCLUDE = PACKAGE.parent / "include"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "liblimn_hip.so"
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc would otherwise fuse float pairs into packed-FP32 VALU forms.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", *DEVICE_FLAGS]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the limn HIP library needs ROCm's hipcc to build")
    return path


def _includes(path: Path, seen: set[Path]) -> set[Path]:
    """The quoted #include files `path` reaches (transitively), resolved next to it or in include/."""
    for line in path.read_text().splitlines():
        line = line.strip()
        if not line.startswith('#include "'):
            continue
        name = line.split('"')[1]
        for base in (path.parent, INCLUDE):
            dep = (base / name).resolve()
            if dep.exists():
                if dep not in seen:
                    seen.add(dep)
                    _includes(dep, seen)
                break
    return seen


def _stale(obj: Path, src: Path, headers: list[Path]) -> bool:
    """Whether obj is older than its source or a header the source includes (`headers` bounds the
    search to the project's own headers)."""
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    own = set(headers)
    deps = [h for h in _includes(src, set()) if h in own]
    return any(p.stat().st_mtime > t for p in [src, *deps])


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{done.stderr[-8000:]}")


def build(force: bool = False, verbose: bool = False) -> Path:
    """Compile the kernel library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    headers = sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))
    jobs = [(src, BUILD / (src.stem + ".o")) for src in sources]
    todo = [(s, o) for s, o in jobs if force or _stale(o, s, headers)]
    workers = max(1, min(len(todo), int(os.environ.get("MAX_JOBS", "8")), os.cpu_count() or 1))
    if todo:
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            for src, _ in todo:
                if verbose:
                    print(f"hipcc {src.name}", flush=True)
            list(pool.map(lambda job: _compile(*job), todo))
    tmp = LIBRARY.with_suffix(".so.tmp")
    # every symbol resolved at link time: a kernel whose launch stub the host pass did not emit
    # would otherwise surface only when the library is loaded on the GPU box
    cmd = [hipcc(), *FLAGS, "-shared", "-Wl,--no-undefined", "-o", str(tmp), *(str(o) for _, o in jobs)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"linking liblimn_hip.so failed:\n{done.stderr[-8000:]}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(force="--force" in sys.argv, verbose=True))
