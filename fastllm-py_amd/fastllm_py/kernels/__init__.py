"""Kernel wrappers over native/libfastllm_kernels.so (gfx950 HIP)."""
