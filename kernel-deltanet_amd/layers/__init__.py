"""Reference-named layer surface of the prefill path on MI355X (reference layers/__init__.py:5)."""
from .kernel_deltanet_layer import KernelDeltaNetLayer, KernelTTTLayer, MultiHeadRKHSKernel

__all__ = ["KernelDeltaNetLayer", "KernelTTTLayer", "MultiHeadRKHSKernel"]
