"""fastllm_py quantized-weight matmul path, MI355X (gfx950) HIP implementation.

Import surface mirrors the reference package's hot-path modules:
``fastllm_py.quantizer``, ``fastllm_py.expert_router``, ``fastllm_py.moe``
(packers and the expert FFN) and ``fastllm_py.kernels.{marlin, fp8, moe_int4}``.
"""
