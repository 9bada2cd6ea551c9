"""The MI355X `hip` device for limn. Importing this package registers it: afterwards
`set_device("hip")` selects it, through limn's own registry when limn is bound
(`limn.device.DEVICES`, reference `limn/device.py:199-220`) or the stand-in's otherwise.

The factory checks the HIP runtime, the kernel library and the GPU first and raises
RuntimeError with the reason, as limn's factories do for their toolchains.
"""

from __future__ import annotations

from limn_amd import seam


def hip_device():
    from limn_amd.hip.device import HipDevice
    from limn_amd.hip.runtime import hip_unavailable

    reason = hip_unavailable()
    if reason is not None:
        raise RuntimeError(f"the 'hip' device is unavailable: {reason}")
    return HipDevice()


seam.DEVICES["hip"] = hip_device
