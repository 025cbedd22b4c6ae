"""Native MI355X (gfx950) backend of the Kernel-DeltaNet prefill path: ctypes binding of libkdn.so.

The reference-named Python surfaces live beside this package (``kernels``, ``layers``); they call
``kdn.ops``, which calls the HIP kernels through the C ABI of include/kdn.h.
"""
from . import ops  # noqa: F401
from ._native import LIB_PATH, NativeLibraryMissing  # noqa: F401
