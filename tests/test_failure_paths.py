"""Failure handling of the hip device, forced from the host on the CPU (no GPU needed).

The reference's CUDA device (limn/backend_cuda.py) reports every failure as RuntimeError with
what it was doing and why (`check`, :154-162), detects a missing toolchain when the device is
selected (`cuda_unavailable`, :165-178; limn/device.py:182-196), trims its buffer pool and retries
an allocation once (:301-306), and raises with the compiler's log when a kernel does not compile
(:202-209). The hip device keeps the same conventions; these tests force each path with a fake
runtime object or a real hipRTC compile (hipRTC needs no GPU).
"""

from __future__ import annotations

import pytest

from limn_amd.hip import runtime
from limn_amd.hip.device import HipDevice


class FakeHip:
    """The few libamdhip64 calls the allocation path makes; hipMalloc fails `failures` times."""

    def __init__(self, failures: int):
        self.failures = failures
        self.freed: list[int] = []
        self.next_ptr = 0x10000

    def hipMalloc(self, ptr_ref, nbytes):
        if self.failures > 0:
            self.failures -= 1
            return 2  # hipErrorOutOfMemory
        ptr_ref._obj.value = self.next_ptr
        self.next_ptr += 0x10000
        return 0

    def hipFree(self, ptr):
        self.freed.append(ptr.value)
        return 0

    def hipDeviceSynchronize(self):
        return 0


def device_on(api: FakeHip) -> HipDevice:
    """A HipDevice whose runtime is `api`: only the state the allocation path touches."""
    dev = HipDevice.__new__(HipDevice)
    dev.api = api
    dev.pool = {}
    dev.replays = {}
    dev._commits = []
    dev._commit_targets = set()
    dev._committed = []
    return dev


def test_a_failed_allocation_trims_the_pool_and_retries_once():
    api = FakeHip(failures=0)
    dev = device_on(api)
    held = [dev._alloc(256), dev._alloc(512)]
    pooled = sorted(b.ptr for b in held)
    del held  # both return to the pool
    assert sorted(p for ptrs in dev.pool.values() for p in ptrs) == pooled
    api.failures = 1
    buf = dev._alloc(1 << 20)  # not in the pool: hipMalloc fails, trim() frees the pool, the retry succeeds
    assert sorted(api.freed) == pooled
    assert dev.pool == {} or all(not v for v in dev.pool.values())
    assert buf.nbytes == 1 << 20 and buf.ptr not in pooled


def test_an_allocation_that_fails_twice_raises_with_what_it_was_doing():
    api = FakeHip(failures=0)
    dev = device_on(api)
    held = dev._alloc(64)
    del held
    api.failures = 2
    with pytest.raises(RuntimeError, match=r"^hip: allocating 4096 bytes: "):
        dev._alloc(4096)


def test_with_an_empty_pool_a_failed_allocation_raises_at_once():
    api = FakeHip(failures=1)
    dev = device_on(api)
    with pytest.raises(RuntimeError, match=r"^hip: allocating 128 bytes"):
        dev._alloc(128)
    assert api.failures == 0 and api.freed == []  # no retry: nothing to trim


def test_a_missing_runtime_library_is_the_reason_set_device_reports(monkeypatch):
    monkeypatch.setattr(runtime, "hip", lambda: None)
    uncached = runtime.hip_unavailable.__wrapped__
    assert uncached() == "libamdhip64 not found (it ships with ROCm)"
    import limn_amd.hip as hip_package

    monkeypatch.setattr(runtime, "hip_unavailable", uncached)
    with pytest.raises(RuntimeError, match="the 'hip' device is unavailable: libamdhip64 not found"):
        hip_package.hip_device()


def test_a_missing_hiprtc_is_reported(monkeypatch):
    monkeypatch.setattr(runtime, "hiprtc", lambda: None)
    assert runtime.hip_unavailable.__wrapped__() == "libhiprtc not found (it ships with ROCm)"
    with pytest.raises(RuntimeError, match="hiprtc: library not found"):
        runtime.compile_source("extern \"C\" __global__ void k() {}", ["k"])


def test_a_missing_kernel_library_says_how_to_build_it(monkeypatch, tmp_path):
    monkeypatch.setattr(runtime, "LIBRARY", tmp_path / "liblimn_hip.so")
    with pytest.raises(RuntimeError, match=r"is missing: build it with `python -m limn_amd.build`"):
        runtime.kernels.__wrapped__()


def test_a_kernel_that_does_not_compile_raises_with_the_compiler_log():
    source = 'extern "C" __global__ void broken(float* out) { out[0] = undeclared_name; }'
    with pytest.raises(RuntimeError) as err:
        runtime.compile_source(source, ["broken"])
    message = str(err.value)
    assert message.startswith("hiprtc failed:")
    assert "undeclared_name" in message and "error" in message


def test_runtime_failures_name_what_was_being_done():
    runtime.check(0, "anything")  # success is silent
    with pytest.raises(RuntimeError, match=r"^hip: copying a tile: "):
        runtime.check(1, "copying a tile")
