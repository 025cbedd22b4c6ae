"""Reference-named surfaces of the Kernel-DeltaNet prefill path on MI355X (gfx950).

Mirrors the import paths of the reference package ``kernels`` (kernels/__init__.py:5-23) for the
names on the prefill path; every call runs HIP kernels from libkdn.so.
"""
from .factored_kernel_deltanet import (FactoredFastWalshHadamardProjection, FactoredKernelDeltaNet,
                                       factored_chunked_deltanet_forward)
from .fwht import FastWalshHadamardProjection, fast_walsh_hadamard_transform
from .fused_kernel_deltanet import FusedKernelDeltaNet, FusedKernelDeltaNetFunction, fused_chunked_deltanet_forward
from .fused_triton_engine import fused_triton_chunk_scan
from .tiled_triton_engine import streaming_triton_chunk_scan, tiled_triton_chunk_scan

__all__ = [
    "FactoredFastWalshHadamardProjection",
    "FactoredKernelDeltaNet",
    "factored_chunked_deltanet_forward",
    "FastWalshHadamardProjection",
    "fast_walsh_hadamard_transform",
    "fused_chunked_deltanet_forward",
    "FusedKernelDeltaNet",
    "FusedKernelDeltaNetFunction",
    "fused_triton_chunk_scan",
    "tiled_triton_chunk_scan",
    "streaming_triton_chunk_scan",
]
