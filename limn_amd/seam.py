"""Where the hip device meets limn: the one module through which this package reaches limn's IR.

The hip device is a plug-in. Its scheduler input, loop nests, CUSTOM nodes and executor base
class are limn's own objects, and it tells them apart by the enum members and dtypes limn
defines (`node.op is Op.SUM`, `instr.opcode is Opcode.LOAD`). Those checks only mean something
against the very classes the nodes were built from. This module binds those classes once:

- `limn` itself when it imports (Python 3.12 with ml_dtypes; `import limn_amd.hip` then adds
  "hip" to `limn.device.DEVICES`, and nothing above the device changes);
- otherwise `limn_amd.standin`, a restatement of limn's IR and frontend under the same module
  names, which is what runs in this build's own container (Python 3.10, no ml_dtypes).

`LIMN_AMD_BIND=standin` forces the stand-in even where limn imports; `LIMN_AMD_BIND=limn`
makes a failed limn import an error instead of a fallback.

Every product module imports limn's names from here and nowhere else (a test scans for direct
imports of the stand-in), so the device, the emitter, the oracle and the stand-in callers agree
on one set of classes whichever package is bound. The emitter's identity checks are then checks
against limn's members when limn is bound.

Reference modules bound (all under `limn/`): ops.py (Node, Op, DType, Custom, custom,
promote, accumulate_in, topological), view.py, schedule.py (Kernel, CUT_OPS, realized,
schedule), codegen.py (LoopNest, Instr, Opcode, Index, Valid, lower_all), jit.py
(CompiledDevice, Plan, Call, Recording), device.py (DEVICES, set_device, HostDevice), and the
callers tensor.py, nn.py, optim.py and capture.py.
"""

from __future__ import annotations

import importlib
import os
from types import ModuleType

STANDIN = "limn_amd.standin"


def _package() -> tuple[str, str | None]:
    """(bound package, why limn was not bound or None)."""
    want = os.environ.get("LIMN_AMD_BIND", "")
    if want == "standin":
        return STANDIN, "LIMN_AMD_BIND=standin"
    try:
        importlib.import_module("limn.jit")
        importlib.import_module("limn.tensor")
    except (ImportError, SyntaxError) as exc:  # absent, or a Python older than limn's 3.12
        if want == "limn":
            raise ImportError(f"LIMN_AMD_BIND=limn but limn does not import: {exc}") from exc
        return STANDIN, f"{type(exc).__name__}: {exc}"
    return "limn", None


PACKAGE, FALLBACK_REASON = _package()


def _module(name: str) -> ModuleType:
    return importlib.import_module(f"{PACKAGE}.{name}")


ops = _module("ops")
view = _module("view")
schedule_module = _module("schedule")
codegen = _module("codegen")
jit = _module("jit")
device = _module("device")
tensor = _module("tensor")
nn = _module("nn")
optim = _module("optim")
capture_module = _module("capture")

# the IR contract (reference limn/ops.py:18-154)
DType, Node, Op, Custom = ops.DType, ops.Node, ops.Op, ops.Custom
custom, topological, promote, accumulate_in = ops.custom, ops.topological, ops.promote, ops.accumulate_in
DTYPES, FLOATS, INTS, HALF_FLOATS = ops.DTYPES, ops.FLOATS, ops.INTS, ops.HALF_FLOATS
float64, float32, float16, bfloat16 = ops.float64, ops.float32, ops.float16, ops.bfloat16
int32, int16, int8 = ops.int32, ops.int16, ops.int8

# the scheduler (reference limn/schedule.py:46-141)
Kernel, CUT_OPS, realized, schedule = schedule_module.Kernel, schedule_module.CUT_OPS, schedule_module.realized, schedule_module.schedule

# the loop-nest IR (reference limn/codegen.py:45-348)
LoopNest, Instr, Opcode, Index, Valid = codegen.LoopNest, codegen.Instr, codegen.Opcode, codegen.Index, codegen.Valid
lower_all, contiguous_index, loop_range = codegen.lower_all, codegen.contiguous_index, codegen.loop_range

# the executor a compiled device subclasses (reference limn/jit.py:64-142)
CompiledDevice, Plan, Call, Recording, Runner = jit.CompiledDevice, jit.Plan, jit.Call, jit.Recording, jit.Runner

# the caller-facing API (reference limn/__init__.py)
Tensor, grad, no_grad, realize, set_seed = tensor.Tensor, tensor.grad, tensor.no_grad, tensor.realize, tensor.set_seed
scatter_rows = tensor.scatter_rows
capture = capture_module.capture
DEVICES, set_device, HostDevice = device.DEVICES, device.set_device, device.HostDevice


def active_device():
    """The device graphs currently run on (limn's `device.active()`)."""
    return device.active()


def use_device(dev) -> None:
    """Make an already constructed device the active one (what set_device does after its
    factory ran); tests and the bench hold their devices and switch between them."""
    device.active_device = dev
