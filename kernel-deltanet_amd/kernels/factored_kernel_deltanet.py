"""Factored d_k = 128 path -- drop-in for the reference module kernels/factored_kernel_deltanet.py.

Same names and signatures as the reference (kernels/factored_kernel_deltanet.py:42-206):
  FactoredFastWalshHadamardProjection(d_k=128, D=1024, seed=42)   -- two 64 -> 512 lifts (seeds s and
      s + 1000) of the two halves of x, concatenated and renormalised onto S^{D-1} (eps 1e-7)
  factored_chunked_deltanet_forward(q, k, v, beta, decay, factored_proj, chunk_size=64,
                                    initial_state=None) -> (Y, S)
  FactoredKernelDeltaNet(d_k=128, d_v=128, D=1024, chunk_size=64, seed=42)
Layouts as in the reference: q, k (B, T, 128), v (B, T, d_v), beta, decay (B, T), state (B, d_v, D).

The lift is kdn_fwht_lift_factored; the scan is the exact delta rule
S_t = lambda_t S_{t-1} (I - beta_t phi(k_t) phi(k_t)^T) + beta_t v_t phi(k_t)^T with readout
y_t = S_{t-1} phi(q_t) over the 1024 pre-lifted features (kdn_delta_scan_fwd with d_k = D = 1024, the
general-width kernels of csrc/kdn_general.hip), state in fp32; d_v is 64 or 128.  Results do not depend
on chunk_size (the kernels use 64-token chunks; padding past T is an exact no-op).

Gradients (the reference trains this path through torch autograd) flow to q, k, v, beta, decay and
initial_state: kdn_delta_scan_bwd at D = 1024 gives dL/dphi_q, dL/dphi_k, dv, dbeta, dlambda and dS_0,
and kdn_fwht_lift_factored_bwd takes dL/dphi back through the lift to q and k.  The projections' tables
are constants (buffers in the reference).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from kdn import ops

from .fwht import FastWalshHadamardProjection


class FactoredFastWalshHadamardProjection(nn.Module):
    """Reference: kernels/factored_kernel_deltanet.py:42-74."""

    def __init__(self, d_k: int = 128, D: int = 1024, seed: int = 42):
        super().__init__()
        if d_k % 2 or D % 2:
            raise ValueError(f"d_k and D must be even, got {d_k}, {D}")
        if d_k != 128 or D != 1024:
            raise ValueError(f"the factored lift runs d_k = 128 -> D = 1024 (got {d_k} -> {D})")
        self.d_k, self.D = d_k, D
        self.d_k0, self.D0 = d_k // 2, D // 2
        self.proj1 = FastWalshHadamardProjection(d_k=self.d_k0, D=self.D0, seed=seed)
        self.proj2 = FastWalshHadamardProjection(d_k=self.d_k0, D=self.D0, seed=seed + 1000)
        self.tau = d_k ** 0.25  # kept for attribute parity; each half lifts with its own tau* = 64^(1/4)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x (..., 128) -> (..., 1024) on the unit sphere, in x's dtype."""
        ops.require_device(x, "FactoredFastWalshHadamardProjection")
        dev = x.device
        return ops.lift_factored(x, self.proj1.device_omega(dev), self.proj1.device_phase(dev),
                                 self.proj2.device_omega(dev), self.proj2.device_phase(dev), self.proj1.tau_star_inv)


class _FactoredScan(torch.autograd.Function):
    """The factored lift of q and k followed by the D = 1024 scan, with its backward (see the module
    docstring).  Layouts as factored_chunked_deltanet_forward; returns (y (B, T, d_v), S (B, d_v, D) fp32)."""

    @staticmethod
    def forward(ctx, q, k, v, beta, decay, initial_state, proj):
        B, T, _ = k.shape
        d_v = v.shape[-1]
        D = proj.D
        dev = k.device
        phi_q = proj(q)
        phi_k = proj(k)
        init4 = None
        if initial_state is not None:
            init4 = initial_state.to(device=dev, dtype=torch.float32).unsqueeze(1).transpose(2, 3)
        final = torch.empty(B, d_v, D, device=dev, dtype=torch.float32)
        y = torch.empty(B, T, d_v, device=dev, dtype=q.dtype)
        vf = v.to(phi_q.dtype)
        ops.scan(phi_q.unsqueeze(2), phi_k.unsqueeze(2), vf.unsqueeze(2), beta.unsqueeze(-1),
                 None if decay is None else decay.unsqueeze(-1), None, None, 1.0, initial_state=init4,
                 final_state=final.unsqueeze(1).transpose(2, 3), y=y.unsqueeze(2),
                 features=ops.FeatureMap(lifted=True))
        ctx.save_for_backward(q, k, vf, beta, decay, initial_state, phi_q, phi_k)
        ctx.proj = proj
        ctx.v_dtype = v.dtype
        return y, final

    @staticmethod
    def backward(ctx, dy, dfinal):
        q, k, vf, beta, decay, init, phi_q, phi_k = ctx.saved_tensors
        proj = ctx.proj
        need = ctx.needs_input_grad
        dev = q.device
        B, T, _ = q.shape
        d_v = vf.shape[-1]
        D = proj.D
        dy4 = (torch.zeros(B, T, d_v, device=dev, dtype=torch.float32) if dy is None else dy.float()).unsqueeze(2)
        dfin4 = None if dfinal is None else dfinal.float().unsqueeze(1).transpose(2, 3)
        init4 = None if init is None else init.to(device=dev, dtype=torch.float32).unsqueeze(1).transpose(2, 3)
        plan = ops.ScanBackwardPlan(phi_q.unsqueeze(2), phi_k.unsqueeze(2), vf.unsqueeze(2), beta.unsqueeze(-1),
                                    None if decay is None else decay.unsqueeze(-1), None, None, 1.0, dy4, dfin4,
                                    initial_state=init4, need_ddecay=decay is not None and bool(need[4]),
                                    need_dinit=init is not None and bool(need[5]),
                                    features=ops.FeatureMap(lifted=True))
        dphi_q, dphi_k, dv, dbeta, ddecay, dinit = plan.run(concurrent_carries=False)
        p1, p2 = proj.proj1, proj.proj2
        args = (p1.device_omega(dev), p1.device_phase(dev), p2.device_omega(dev), p2.device_phase(dev),
                p1.tau_star_inv)
        dq = ops.lift_factored_backward(q, dphi_q[:, :, 0], *args) if need[0] else None
        dk = ops.lift_factored_backward(k, dphi_k[:, :, 0], *args) if need[1] else None
        return (None if dq is None else dq.to(q.dtype), None if dk is None else dk.to(k.dtype),
                dv[:, :, 0].to(ctx.v_dtype), dbeta[:, :, 0].to(beta.dtype),
                None if ddecay is None else ddecay[:, :, 0].to(decay.dtype),
                None if dinit is None else dinit[:, 0].transpose(1, 2).to(init.dtype), None)


def factored_chunked_deltanet_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    beta: torch.Tensor,
    decay: Optional[torch.Tensor],
    factored_proj: FactoredFastWalshHadamardProjection,
    chunk_size: int = 64,
    initial_state: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Reference: kernels/factored_kernel_deltanet.py:77-183."""
    if chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    if q.dim() != 3 or k.shape != q.shape or v.dim() != 3 or v.shape[:2] != k.shape[:2]:
        raise ValueError(f"expected q, k (B, T, 128) and v (B, T, d_v); got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    B, T, _ = k.shape
    d_v = v.shape[-1]
    D = factored_proj.D
    if beta.shape != (B, T) or (decay is not None and decay.shape != (B, T)):
        raise ValueError("beta and decay must be (B, T)")
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta")):
        ops.require_device(t, f"factored_chunked_deltanet_forward: {nm}")
    if initial_state is not None and tuple(initial_state.shape) != (B, d_v, D):
        raise ValueError(f"initial_state must be (B, d_v, D) = {(B, d_v, D)}")
    if d_v not in (64, 128):
        raise ValueError(f"factored path: d_v must be 64 or 128, got {d_v}")
    Y, S = _FactoredScan.apply(q, k, v, beta, decay, initial_state, factored_proj)
    s_dtype = initial_state.dtype if initial_state is not None else k.dtype
    return Y, (S if s_dtype == torch.float32 else S.to(s_dtype))


class FactoredKernelDeltaNet(nn.Module):
    """Reference: kernels/factored_kernel_deltanet.py:186-206."""

    def __init__(self, d_k: int = 128, d_v: int = 128, D: int = 1024, chunk_size: int = 64, seed: int = 42):
        super().__init__()
        self.d_k, self.d_v, self.D, self.chunk_size = d_k, d_v, D, chunk_size
        self.factored_proj = FactoredFastWalshHadamardProjection(d_k=d_k, D=D, seed=seed)

    def forward(self, q, k, v, beta, decay, initial_state=None):
        return factored_chunked_deltanet_forward(q, k, v, beta, decay, self.factored_proj, self.chunk_size,
                                                 initial_state)
