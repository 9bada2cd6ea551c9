"""The hip device's pairing of limn's two backward CUSTOM calls, on the CPU.

limn's attention backward issues `sdpa_bwd_q` and `sdpa_bwd_kv` as two calls on the same inputs
(reference limn/tensor.py:707-712). HipDevice._pair_backward (run by its plan_of) replaces such a
pair with one call of three outputs at the first one's place, so the dK/dV pass can hand dS to the
dQ pass. These tests drive it with plans of stub calls: no GPU, no library call.
"""

from __future__ import annotations

from limn_amd.hip.device import SDPA_BWD_KV, SDPA_BWD_Q, HipDevice
from limn_amd.seam import Call, Plan


def stub(name: str | None, key=("bf16", 128, True), fused=True):
    def run(inputs, outs):
        raise AssertionError("stubs never run")

    if name is not None:
        run.sdpa_pair = (name, key, (lambda: paired_runner) if fused else (lambda: None))
    return run


def paired_runner(inputs, outs):
    raise AssertionError("stubs never run")


def call(fn, inputs, outputs, sizes):
    return Call(fn=fn, inputs=inputs, outputs=outputs, out_nbytes=sizes, zero_fill=False, assign_target=None)


def plan(*calls):
    return Plan(calls=tuple(calls), buffers=(0, 1, 2, 3, 4, 5), sinks=(9, 10, 11), positions=12)


def pair(p):
    dev = HipDevice.__new__(HipDevice)  # _pair_backward touches no device state
    return dev._pair_backward(p)


SRCS = (0, 1, 2, 3, 4, 5)


def test_a_pair_on_the_same_inputs_becomes_one_call_at_the_first_place():
    other = call(stub(None), (0,), (8,), (4,))
    q = call(stub(SDPA_BWD_Q), SRCS, (9,), (100,))
    kv = call(stub(SDPA_BWD_KV), SRCS, (10, 11), (200, 300))
    got = pair(plan(other, kv, q))
    assert len(got.calls) == 2
    assert got.calls[0] is other
    merged = got.calls[1]
    assert merged.fn is paired_runner
    assert merged.inputs == SRCS
    assert merged.outputs == (9, 10, 11) and merged.out_nbytes == (100, 200, 300)
    assert got.sinks == (9, 10, 11) and got.positions == 12


def test_calls_on_other_inputs_or_params_stay_apart():
    q = call(stub(SDPA_BWD_Q), SRCS, (9,), (100,))
    kv_other_inputs = call(stub(SDPA_BWD_KV), (0, 1, 2, 3, 4, 6), (10, 11), (200, 300))
    kv_other_params = call(stub(SDPA_BWD_KV, key=("bf16", 128, False)), SRCS, (10, 11), (200, 300))
    p = plan(q, kv_other_inputs, kv_other_params)
    assert pair(p) is p


def test_a_pair_without_a_handoff_route_stays_apart():
    q = call(stub(SDPA_BWD_Q, fused=False), SRCS, (9,), (100,))
    kv = call(stub(SDPA_BWD_KV, fused=False), SRCS, (10, 11), (200, 300))
    p = plan(q, kv)
    assert pair(p) is p


def test_two_attentions_pair_each_with_its_own():
    q1 = call(stub(SDPA_BWD_Q), SRCS, (9,), (1,))
    q2 = call(stub(SDPA_BWD_Q), (6, 1, 2, 3, 4, 5), (12,), (2,))
    kv2 = call(stub(SDPA_BWD_KV), (6, 1, 2, 3, 4, 5), (13, 14), (3, 4))
    kv1 = call(stub(SDPA_BWD_KV), SRCS, (10, 11), (5, 6))
    got = pair(plan(q1, q2, kv2, kv1))
    assert [c.outputs for c in got.calls] == [(9, 10, 11), (12, 13, 14)]
    assert [c.inputs for c in got.calls] == [SRCS, (6, 1, 2, 3, 4, 5)]
