"""dwim_amd: an MI355X (gfx950) backend for dwim's inference engine.

The product is the shared library dwim_amd/libdwim_hip.so (HIP kernels and the
C ABI of include/dwim_hip.h).  `dwim_amd.device` mirrors the reference's
`gpu::Device` trait over that ABI; `dwim_amd.model` drives the qwen35
forward pass built on it.
"""
from .device import (BF16, CACHE_BLOCK, CONV_KERNEL, Q4_0, Q4_K, Q6_K, Q8_0, DwimError, Hip,  # noqa: F401
                     Tensor, lib)
