"""Structured-FWHT random-feature lift -- drop-in for the reference module kernels/fwht.py.

Same public names, constructor arguments, buffers and forward semantics as the reference
(kernels/fwht.py:25-131): FastWalshHadamardProjection(d_k=64, D=512, seed=42) with buffers d1, d2, d3,
rademacher_bits (non-persistent), b and Omega, and forward(x) = phi / (||phi|| + 1e-8) with
phi = sqrt(2/D) cos(x Omega^T / tau* + b), tau* = d_k^(1/4).

The forward runs the gfx950 lift kernel at the reference's native boundary (kdn_fwht_lift_bits, the
replacement of kernel_deltanet_cuda.fwht_forward): every workgroup builds Omega in LDS from the packed
sign table with wave64 butterflies, then projects on MFMA.  The scan's kernels read a resident bf16 copy
of Omega instead, built once per device by the same butterflies (kdn_build_omega).  Device tensors only.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn as nn

from kdn import ops


def fast_walsh_hadamard_transform(x: torch.Tensor) -> torch.Tensor:
    """Unnormalised natural-order Walsh-Hadamard transform along the last dimension (power of two <= 64).

    Reference: kernels/fwht.py:25-45.  Runs the wave64 butterfly kernel kdn_fwht.
    """
    return ops.fwht(x)


class FastWalshHadamardProjection(nn.Module):
    """Maps (..., d_k) -> (..., D) spherically renormalised cosine features over the structured projection
    Omega = concat_m (H D3_m H D2_m H D1_m) / sqrt(d_k).  Reference: kernels/fwht.py:48-131."""

    def __init__(self, d_k: int = 64, D: int = 512, seed: int = 42):
        super().__init__()
        assert D % d_k == 0, f"D ({D}) must be divisible by d_k ({d_k})"
        self.d_k = d_k
        self.D = D
        self.M = D // d_k
        self.scale_norm = 1.0 / math.sqrt(d_k)
        self.tau_star = float(d_k) ** 0.25
        self.tau_star_inv = 1.0 / self.tau_star

        # Seeded draws in the reference order: d1, d2, d3, then the phases b (kernels/fwht.py:66-86).
        gen = torch.Generator().manual_seed(seed)
        d1 = torch.where(torch.rand(self.M, d_k, generator=gen) > 0.5, 1.0, -1.0)
        d2 = torch.where(torch.rand(self.M, d_k, generator=gen) > 0.5, 1.0, -1.0)
        d3 = torch.where(torch.rand(self.M, d_k, generator=gen) > 0.5, 1.0, -1.0)
        b = torch.rand(D, generator=gen) * (2.0 * math.pi)

        # Packed sign table: bit i of word (m, s) set <=> stage s sign i is -1 (kernels/fwht.py:74-83).
        signs = np.stack([d1.numpy(), d2.numpy(), d3.numpy()], axis=1) < 0          # [M, 3, d_k]
        weights = np.left_shift(np.uint64(1), np.arange(min(64, d_k), dtype=np.uint64))
        words = (signs[..., :64].astype(np.uint64) * weights).sum(axis=-1, dtype=np.uint64)
        rad_masks = torch.from_numpy(words.view(np.int64).copy())

        # Explicit Omega (integer arithmetic, then the 1/sqrt(d_k) scale), same values as :94-111.
        H = np.ones((1, 1), dtype=np.int64)
        while H.shape[0] < d_k:
            H = np.block([[H, H], [H, -H]])
        blocks = []
        for m in range(self.M):
            s1, s2, s3 = (t[m].numpy().astype(np.int64) for t in (d1, d2, d3))
            blocks.append(H @ np.diag(s3) @ H @ np.diag(s2) @ H @ np.diag(s1))
        omega_int = np.concatenate(blocks, axis=0)
        Omega = torch.from_numpy(omega_int.astype(np.float32)) * self.scale_norm

        self.register_buffer("d1", d1)
        self.register_buffer("d2", d2)
        self.register_buffer("d3", d3)
        self.register_buffer("rademacher_bits", rad_masks, persistent=False)
        self.register_buffer("b", b)
        self.register_buffer("Omega", Omega)
        # The device kernels hold Omega in bf16; its entries are integer / sqrt(d_k) with few significant
        # bits, so the bf16 copy is exact (checked here for this seed).
        if not bool((Omega.to(torch.bfloat16).to(torch.float32) == Omega).all()):
            raise ValueError(f"seed {seed}: Omega is not exactly representable in bf16; unsupported")
        self._dev_omega = {}
        self._dev_tables = {}

    def device_omega(self, device) -> torch.Tensor:
        """bf16 Omega on `device`, built once per device from the sign table by kdn_build_omega."""
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError(f"device_omega: kernel-deltanet_amd runs on gfx950 device tensors only (got {device})")
        key = (device.type, device.index if device.index is not None else torch.cuda.current_device())
        om = self._dev_omega.get(key)
        if om is None:
            om = ops.build_omega(self.rademacher_bits, self.d_k, self.D, device, torch.bfloat16)
            self._dev_omega[key] = om
        return om

    def _device_table(self, name: str, device, dtype) -> torch.Tensor:
        """Buffer `name` on `device` in `dtype`: the buffer itself when it is already there (the module was
        moved), else a copy kept per device and refreshed only when the buffer changes (load_state_dict
        writes buffers in place, which bumps their version), so that a forward issues no host-to-device
        copy."""
        buf = getattr(self, name)
        device = torch.device(device)
        if buf.device == device or (device.index is None and buf.is_cuda):
            return buf if buf.dtype == dtype else buf.to(dtype)
        key = (name, device.index if device.index is not None else torch.cuda.current_device())
        stamp = (buf.data_ptr(), buf._version)
        hit = self._dev_tables.get(key)
        if hit is None or hit[0] != stamp:
            hit = (stamp, buf.to(device=device, dtype=dtype))
            self._dev_tables[key] = hit
        return hit[1]

    def device_phase(self, device) -> torch.Tensor:
        """The phases b as float32 on `device`."""
        return self._device_table("b", device, torch.float32)

    def device_bits(self, device) -> torch.Tensor:
        """The packed [M, 3] sign table on `device` (the argument of kdn_fwht_lift_bits)."""
        return self._device_table("rademacher_bits", device, torch.int64)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """(..., d_k) -> (..., D) in x's dtype (bfloat16 or float32); fp32 arithmetic inside."""
        ops.require_device(x, "FastWalshHadamardProjection")
        return ops.lift_bits(x, self.device_bits(x.device), self.device_phase(x.device), self.tau_star_inv,
                             normalize=False, out_dtype=x.dtype)
