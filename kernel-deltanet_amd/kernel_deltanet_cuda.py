"""Drop-in for the reference's native extension module `kernel_deltanet_cuda` on MI355X.

The reference builds `kernel_deltanet_cuda` from kernels/fwht_cuda.cpp (pybind `fwht_forward(input,
rademacher_bits, D_lifted, tau_star_inv=0.35355339f)`, :29-32) and calls it from
FastWalshHadamardProjection.forward (kernels/fwht.py:19-23 import, :119-120 call).  This module has the
same name and function; with `kernel-deltanet_amd/` on sys.path the reference's `import
kernel_deltanet_cuda` picks it up.  It binds libkdn.so's kdn_fwht_lift_bits (include/kdn.h) with ctypes
and nothing else, so it can be copied next to the reference's kernels/fwht.py as it is.

Semantics: the torch branch of the reference's forward (kernels/fwht.py:122-131),
    phi_hat = phi / (||phi|| + 1e-8),   phi = sqrt(2/D) cos(x Omega^T * tau_star_inv + b),
with Omega built on the device from `rademacher_bits`.  That branch adds the module's phases b, which the
reference's CUDA function never receives; pass them as `phase`.  The reference's one call site then reads
    kernel_deltanet_cuda.fwht_forward(x.contiguous(), self.rademacher_bits, self.D, self.tau_star_inv,
                                      phase=self.b)
(kernels/fwht.py:120 with `phase=self.b` added).  Without `phase` the call raises: the reference's CUDA
kernel computes a different feature function (a 4-block transform without phases or renormalisation,
kernels/in_register_fwht.cu:10-93), which this build does not reproduce.

Errors are raised as RuntimeError with the library's status text (the reference raises from TORCH_CHECK).
"""
from __future__ import annotations

import ctypes
import os

import torch

# KDN_LIBRARY names another build of libkdn.so, as for the kdn package (kdn/_native.py), so both load the same
# copy
_LIB_PATH = os.environ.get("KDN_LIBRARY") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "kdn", "libkdn.so")
_L = None
_TAG = {torch.float32: 0, torch.bfloat16: 1}


def _lib():
    global _L
    if _L is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"kernel_deltanet_cuda: {_LIB_PATH} is missing (build libkdn.so for gfx950 first)")
        L = ctypes.CDLL(_LIB_PATH)
        vp, i64, ci, cf = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.kdn_fwht_lift_bits.argtypes = [vp, i64, i64, ci, ci, vp, ci, cf, vp, ci, vp, i64, ci, vp]
        L.kdn_fwht_lift_bits.restype = ci
        L.kdn_strerror.argtypes = [ci]
        L.kdn_strerror.restype = ctypes.c_char_p
        _L = L
    return _L


def fwht_forward(input: torch.Tensor, rademacher_bits: torch.Tensor, D_lifted: int,
                 tau_star_inv: float = 0.35355339, phase: torch.Tensor = None) -> torch.Tensor:
    """(..., 64) -> (..., D_lifted) in input's dtype (float32 or bfloat16), on input's device and current
    stream.  rademacher_bits: the module's (D_lifted / 64, 3) int64 table; phase: its (D_lifted,) b."""
    if not input.is_cuda:
        raise RuntimeError("fwht_forward: input must be a GPU tensor")
    if phase is None:
        raise ValueError("fwht_forward: pass the module's phases, phase=self.b (kernels/fwht.py:120); the lift "
                         "phi = sqrt(2/D) cos(x Omega^T / tau + b) of kernels/fwht.py:122-131 needs them")
    if input.dtype not in _TAG:
        raise TypeError(f"fwht_forward: dtype {input.dtype} is not supported (float32 or bfloat16)")
    dev = input.device
    x = input.reshape(-1, input.shape[-1])
    if x.stride(-1) != 1 or (x.stride(0) * x.element_size()) % 16 or x.data_ptr() % 16:
        x = x.contiguous()
    bits = rademacher_bits.to(device=dev, dtype=torch.int64).contiguous()
    ph = phase.to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty(x.shape[0], int(D_lifted), dtype=input.dtype, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    with torch.cuda.device(dev):
        rc = _lib().kdn_fwht_lift_bits(x.data_ptr(), x.shape[0], x.stride(0), _TAG[x.dtype], x.shape[1],
                                       bits.data_ptr(), int(D_lifted), float(tau_star_inv), ph.data_ptr(), 0,
                                       out.data_ptr(), out.stride(0), _TAG[out.dtype], stream)
    if rc != 0:
        raise RuntimeError(f"fwht_forward: kdn_fwht_lift_bits failed ({_lib().kdn_strerror(rc).decode()})")
    return out.view(*input.shape[:-1], int(D_lifted))
