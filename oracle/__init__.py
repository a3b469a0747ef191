"""CPU oracle for the quantized-weight matmul path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain numpy, the reference (codemk8/fastllm-py)
algorithms of the path: the packers/unpackers, the expert router and the
fp32 dequantize-then-matmul that every kernel is checked against.  Each
function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline — never as the product path.  The product
(``fastllm-py_amd/fastllm_py``) runs exclusively in the HIP library and has
no CPU fallback.

How each function is pinned (beyond retyping the formula) is listed in the
docstring of each module; the pins live in ``tests/test_oracle_*.py``.
"""
