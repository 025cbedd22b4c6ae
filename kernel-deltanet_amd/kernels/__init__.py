"""Reference-named surfaces of the Kernel-DeltaNet prefill path on MI355X (gfx950).

Mirrors the import paths of the reference package ``kernels`` (kernels/__init__.py:5-23) for the
names on the prefill path; every call runs HIP kernels from libkdn.so.
"""
from .fwht import FastWalshHadamardProjection, fast_walsh_hadamard_transform
from .fused_kernel_deltanet import FusedKernelDeltaNet, FusedKernelDeltaNetFunction, fused_chunked_deltanet_forward

__all__ = [
    "FastWalshHadamardProjection",
    "fast_walsh_hadamard_transform",
    "fused_chunked_deltanet_forward",
    "FusedKernelDeltaNet",
    "FusedKernelDeltaNetFunction",
]
