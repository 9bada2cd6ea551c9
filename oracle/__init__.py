"""TEST INFRASTRUCTURE ONLY: the CPU oracle the `hip` device is diffed against.

Nothing in the product (limn_amd/) imports this package. Only tests/, `__graft_entry__.smoke()`
and bench.py's cpu_baseline leg use it, and only as the checker or the reported CPU baseline.

- oracle/sdpa.py     restates the reference's numpy flash attention (limn/sdpa.py:48-203) and its
                     textbook forms (limn/sdpa.py:227-248);
- oracle/bf16.py     an independent bfloat16 round-to-nearest-even, pinned to torch.bfloat16;
- oracle/numpy_device.py restates the reference's NumpyDevice interpreter (limn/device.py:63-175).

What pins each function is listed in that function's module header.
"""
