"""A restatement of limn's IR and frontend, bound by `limn_amd.seam` where limn cannot be imported.

The modules carry limn's own names (ops, view, schedule, codegen, jit, device, tensor, nn,
optim, capture) and import each other only relatively, so the package stands in for `limn`
as a whole: the tests copy it under the name `limn` to check that the hip device works against
IR classes it did not define.
"""

from .capture import capture
from .device import set_device
from .ops import bfloat16, float16, float32, float64, int8, int16, int32
from .tensor import Tensor, grad, no_grad, realize, set_seed

__all__ = [
    "Tensor",
    "capture",
    "grad",
    "no_grad",
    "realize",
    "set_device",
    "set_seed",
    "bfloat16",
    "float16",
    "float32",
    "float64",
    "int8",
    "int16",
    "int32",
]
