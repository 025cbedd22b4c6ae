"""Chunked gated delta-rule scan -- drop-in for the reference module kernels/fused_kernel_deltanet.py.

Same names and signatures as the reference (kernels/fused_kernel_deltanet.py:31-209):
  fused_chunked_deltanet_forward(q, k, v, beta, decay, fwht_proj, chunk_size=64, initial_state=None) -> (Y, S)
  FusedKernelDeltaNetFunction (autograd.Function, forward returns Y)
  FusedKernelDeltaNet(d_model=64, d_kernel=512, chunk_size=64)
Layouts as in the reference: q, k (B, T, d_k), v (B, T, d_v), beta, decay (B, T), state (B, d_v, D).
Heads are folded into B by the callers (pipeline/transmute.py:76-80 in the reference).

The computation is the exact delta rule y_t = S_{t-1} phi(q_t),
S_t = lambda_t S_{t-1} (I - beta_t phi(k_t) phi(k_t)^T) + beta_t v_t phi(k_t)^T, run by the gfx950 kernels
kdn_delta_scan_fwd (lift + chunk prep + state scan) with the state carried in fp32.  The WY form is
exact for any chunk length, so results do not depend on chunk_size (the kernels use 64-token chunks;
padding past T is an exact no-op, as with the reference's beta = 0 / lambda = 1 padding, :55-62).
Y is returned in q's dtype; S in the dtype the reference returns (initial_state's, else k's).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from kdn import ops

from .fwht import FastWalshHadamardProjection


def fused_chunked_deltanet_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    beta: torch.Tensor,
    decay: Optional[torch.Tensor],
    fwht_proj: FastWalshHadamardProjection,
    chunk_size: int = 64,
    initial_state: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Reference: kernels/fused_kernel_deltanet.py:31-155."""
    if chunk_size <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk_size}")
    if q.dim() != 3 or k.shape != q.shape or v.dim() != 3 or v.shape[:2] != k.shape[:2]:
        raise ValueError(f"expected q, k (B, T, d_k) and v (B, T, d_v); got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    B, T, d_k = k.shape
    d_v = v.shape[-1]
    D = fwht_proj.D
    if beta.shape != (B, T) or (decay is not None and decay.shape != (B, T)):
        raise ValueError("beta and decay must be (B, T)")
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta")):
        ops.require_device(t, f"fused_chunked_deltanet_forward: {nm}")
    dev = k.device
    inputs = (q, k, v, beta, decay, initial_state)
    if torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in inputs):
        # differentiable path: the scan's autograd node runs kdn_delta_scan_bwd in the backward
        init4 = None
        if initial_state is not None:
            if tuple(initial_state.shape) != (B, d_v, D):
                raise ValueError(f"initial_state must be (B, d_v, D) = {(B, d_v, D)}")
            init4 = initial_state.to(device=dev, dtype=torch.float32).unsqueeze(1).transpose(2, 3)
        y4, f4 = ops.scan_autograd(q.unsqueeze(2), k.unsqueeze(2), v.unsqueeze(2), beta.unsqueeze(-1),
                                   None if decay is None else decay.unsqueeze(-1), fwht_proj.device_omega(dev),
                                   fwht_proj.device_phase(dev), fwht_proj.tau_star_inv, initial_state=init4)
        final = f4.squeeze(1).transpose(1, 2)
        s_dtype = initial_state.dtype if initial_state is not None else k.dtype
        return y4.squeeze(2), (final if s_dtype == torch.float32 else final.to(s_dtype))
    y = torch.empty(B, T, d_v, device=dev, dtype=q.dtype)
    final = torch.empty(B, d_v, D, device=dev, dtype=torch.float32)
    init4 = None
    if initial_state is not None:
        if tuple(initial_state.shape) != (B, d_v, D):
            raise ValueError(f"initial_state must be (B, d_v, D) = {(B, d_v, D)}")
        init4 = initial_state.to(device=dev, dtype=torch.float32).unsqueeze(1).transpose(2, 3)
    ops.scan(q.unsqueeze(2), k.unsqueeze(2), v.unsqueeze(2), beta.unsqueeze(-1),
             None if decay is None else decay.unsqueeze(-1),
             fwht_proj.device_omega(dev), fwht_proj.device_phase(dev), fwht_proj.tau_star_inv,
             normalize=False, initial_state=init4, final_state=final.unsqueeze(1).transpose(2, 3),
             y=y.unsqueeze(2))
    s_dtype = initial_state.dtype if initial_state is not None else k.dtype
    return y, (final if s_dtype == torch.float32 else final.to(s_dtype))


class FusedKernelDeltaNetFunction(torch.autograd.Function):
    """Reference: kernels/fused_kernel_deltanet.py:158-179 (forward returns Y only).  The reference's
    backward re-runs its forward under autograd; here it is kdn_delta_scan_bwd (gradients for q, k, v,
    beta and decay; none for the projection or chunk_size)."""

    @staticmethod
    def forward(ctx, q, k, v, beta, decay, fwht_proj, chunk_size=64):
        with torch.no_grad():
            Y, _ = fused_chunked_deltanet_forward(q, k, v, beta, decay, fwht_proj, chunk_size)
        ctx.save_for_backward(q, k, v, beta, decay)
        ctx.fwht_proj = fwht_proj
        return Y

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, beta, decay = ctx.saved_tensors
        p = ctx.fwht_proj
        dev = q.device
        need = ctx.needs_input_grad
        dq, dk, dv, db, dd, _ = ops.scan_backward(
            q.unsqueeze(2), k.unsqueeze(2), v.unsqueeze(2), beta.unsqueeze(-1),
            None if decay is None else decay.unsqueeze(-1), p.device_omega(dev), p.device_phase(dev),
            p.tau_star_inv, grad_output.unsqueeze(2), need_ddecay=bool(need[4]), need_dinit=False)
        return (dq.squeeze(2).to(q.dtype), dk.squeeze(2).to(k.dtype), dv.squeeze(2).to(v.dtype),
                db.squeeze(-1).to(beta.dtype), None if dd is None else dd.squeeze(-1).to(decay.dtype), None, None)


class FusedKernelDeltaNet(nn.Module):
    """Reference: kernels/fused_kernel_deltanet.py:182-209 (d_model is d_k, d_kernel is D)."""

    def __init__(self, d_model: int = 64, d_kernel: int = 512, chunk_size: int = 64):
        super().__init__()
        self.d_model = d_model
        self.d_kernel = d_kernel
        self.chunk_size = chunk_size
        self.fwht_proj = FastWalshHadamardProjection(d_k=d_model, D=d_kernel)

    def forward(self, q, k, v, beta, decay, initial_state=None):
        return fused_chunked_deltanet_forward(q=q, k=k, v=v, beta=beta, decay=decay, fwht_proj=self.fwht_proj,
                                              chunk_size=self.chunk_size, initial_state=initial_state)
