"""Per-head random-feature Kernel-DeltaNet -- drop-in for the reference module kernels/kernel_deltanet_fused.py.

Same names and signatures as the reference (kernels/kernel_deltanet_fused.py:36-303):
  FusedKernelDeltaNetFunction.apply(q, k, v, omega, b_rff, tau, beta, decay, chunk_size=64) -> (Y, S_final)
  FusedKernelDeltaNet(d_model, num_heads, rkhs_dim=512, chunk_size=64, tau_init=1.0).forward(x, state=None)
Layouts as in the reference: q, k (B, H, T, d_k), v (B, H, T, d_v), omega (H, D, d_k), b_rff (H, D),
tau (H, 1) or a scalar, beta, decay (B, H, T); Y (B, H, T, d_v), state (B, H, d_v, D).

What runs: the gated delta rule with readout before update,
  phi(x) = sqrt(2/D) cos(x_hat Omega_h^T / tau_h + b_h),  x_hat = F.normalize(x, eps=1e-6)   (:85-92, :113-117)
  y_t = S_{t-1} phi(q_t),  S_t = lambda_t S_{t-1} (I - beta_t phi(k_t) phi(k_t)^T) + beta_t v_t phi(k_t)^T,
which is the reference's recurrent branch (:288-300) -- for prefill as well as for steps.  The reference's
chunked branch (:119-192) is not an exact form of that recurrence: its inter-chunk readout applies the
chunk-start state without the erasure by the chunk's earlier keys (:179), its intra-chunk term multiplies
the resolvent elementwise rather than as a matrix product (:187-189), and its carry scales the erasure
by both gamma_C and the in-chunk decays (:147, :170).  Its prefill output therefore differs from its
own recurrent branch; this module returns the recurrence's values in both modes.

On the device: the scan kernels lift q, k in-register with Omega given as two bf16 parts
(hi = bf16(Omega), lo = bf16(Omega - hi), so the projection keeps about 16 significant bits), per-head
phases and 1/tau, no renormalisation of phi; the state is carried in fp32.  Y and S are returned in q's dtype.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from kdn import ops


def split_bf16(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(hi, lo) bf16 parts of a float tensor: hi = bf16(w), lo = bf16(w - hi)."""
    w32 = w.to(torch.float32)
    hi = w32.to(torch.bfloat16)
    lo = (w32 - hi.to(torch.float32)).to(torch.bfloat16)
    return hi.contiguous(), lo.contiguous()


def _head_vector(x, H: int, dev, what: str) -> torch.Tensor:
    t = torch.as_tensor(x, dtype=torch.float32, device=dev).reshape(-1)
    if t.numel() == 1:
        return t.expand(H).contiguous()
    if t.numel() != H:
        raise ValueError(f"{what} must have one value per head (H = {H}) or be a scalar; got {t.numel()} values")
    return t.contiguous()


def kernel_deltanet_scan(q, k, v, omega, b_rff, tau, beta, decay, initial_state=None, y=None):
    """The exact per-head scan over (B, H, T, .) tensors: returns Y (B, H, T, d_v) in q's dtype (written
    into `y` if given, any strides) and the final state (B, H, d_v, D) in float32."""
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"expected q, k (B, H, T, d_k) and v (B, H, T, d_v); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, H, T, d_k = q.shape
    d_v = v.shape[-1]
    if omega.dim() != 3 or omega.shape[0] != H or omega.shape[2] != d_k:
        raise ValueError(f"omega must be (H, D, d_k) = ({H}, D, {d_k}); got {tuple(omega.shape)}")
    D = omega.shape[1]
    if tuple(b_rff.shape) != (H, D):
        raise ValueError(f"b_rff must be (H, D) = {(H, D)}; got {tuple(b_rff.shape)}")
    if tuple(beta.shape) != (B, H, T) or (decay is not None and tuple(decay.shape) != (B, H, T)):
        raise ValueError("beta and decay must be (B, H, T)")
    ops.require_device(q, "FusedKernelDeltaNetFunction: q")
    dev = q.device
    hi, lo = split_bf16(omega.to(dev))
    fm = ops.FeatureMap(omega=hi, phase=b_rff.to(device=dev, dtype=torch.float32), omega_lo=lo,
                        inv_tau_head=1.0 / _head_vector(tau, H, dev, "tau"), no_renorm=True)
    if y is None:
        y = torch.empty(B, H, T, d_v, device=dev, dtype=q.dtype)
    final = torch.empty(B, H, d_v, D, device=dev, dtype=torch.float32)
    init = None
    if initial_state is not None:
        if tuple(initial_state.shape) != (B, H, d_v, D):
            raise ValueError(f"state must be (B, H, d_v, D) = {(B, H, d_v, D)}")
        init = initial_state.to(device=dev, dtype=torch.float32).transpose(2, 3)
    v = v.to(q.dtype)
    ops.scan(q.transpose(1, 2), k.to(q.dtype).transpose(1, 2), v.transpose(1, 2),
             beta.to(torch.float32).transpose(1, 2), None if decay is None else decay.to(torch.float32).transpose(1, 2),
             None, None, 1.0, normalize=True, initial_state=init, final_state=final.transpose(2, 3),
             y=y.transpose(1, 2), features=fm)
    return y, final


def _feature_map(omega, b_rff, inv_tau_head, dev) -> ops.FeatureMap:
    hi, lo = split_bf16(omega.detach().to(dev))
    return ops.FeatureMap(omega=hi, phase=b_rff.detach().to(device=dev, dtype=torch.float32), omega_lo=lo,
                          inv_tau_head=inv_tau_head, no_renorm=True)


class FusedKernelDeltaNetFunction(torch.autograd.Function):
    """Reference: kernels/kernel_deltanet_fused.py:36-178.  Forward returns (Y, S_final).  Backward:
    kdn_delta_scan_bwd with this surface's feature map, gradients for q, k, v, tau, beta and decay
    (omega and b_rff are buffers of the reference module: no gradient)."""

    @staticmethod
    def forward(ctx, q, k, v, omega, b_rff, tau, beta, decay, chunk_size: int = 64):
        if chunk_size <= 0:
            raise ValueError(f"chunk_size must be positive, got {chunk_size}")
        with torch.no_grad():
            y, final = kernel_deltanet_scan(q, k, v, omega, b_rff, tau, beta, decay)
        ctx.save_for_backward(q, k, v, omega, b_rff, tau if isinstance(tau, torch.Tensor) else None, beta, decay)
        ctx.tau = tau
        return y, final.to(k.dtype)

    @staticmethod
    def backward(ctx, dy, dfinal):
        q, k, v, omega, b_rff, tau_t, beta, decay = ctx.saved_tensors
        tau = tau_t if tau_t is not None else ctx.tau
        need = ctx.needs_input_grad
        B, H, T, _ = q.shape
        dev = q.device
        tau_h = _head_vector(tau.detach() if isinstance(tau, torch.Tensor) else tau, H, dev, "tau")
        fm = _feature_map(omega, b_rff, (1.0 / tau_h).contiguous(), dev)
        dt = q.dtype
        plan = ops.ScanBackwardPlan(
            q.transpose(1, 2), k.to(dt).transpose(1, 2), v.to(dt).transpose(1, 2),
            beta.to(torch.float32).transpose(1, 2),
            None if decay is None else decay.to(torch.float32).transpose(1, 2), None, None, 1.0,
            dy.transpose(1, 2), None if dfinal is None else dfinal.to(torch.float32).transpose(2, 3),
            normalize=True, need_ddecay=decay is not None and bool(need[7]), need_dinit=False, features=fm,
            need_dinv_tau=tau_t is not None and bool(need[5]))
        dq, dk, dv, dbeta, ddecay, _ = plan.run()
        dtau = None
        if plan.dinv_tau is not None:
            g = -plan.dinv_tau / (tau_h * tau_h)  # d(1/tau)/dtau = -1/tau^2
            dtau = (g.sum() if tau_t.numel() == 1 else g).reshape(tau_t.shape).to(tau_t.dtype)
        return (dq.transpose(1, 2).to(q.dtype), dk.transpose(1, 2).to(k.dtype), dv.transpose(1, 2).to(v.dtype),
                None, None, dtau, dbeta.transpose(1, 2).to(beta.dtype),
                None if ddecay is None else ddecay.transpose(1, 2).to(decay.dtype), None)


class FusedKernelDeltaNet(nn.Module):
    """Reference: kernels/kernel_deltanet_fused.py:181-303.  Parameters and buffers carry the reference's
    names and shapes (w_q, w_k, w_v, w_out, w_beta, w_decay, raw_tau, omega, b_rff), so state dicts load
    either way.  The device path needs d_model / num_heads = 64 and rkhs_dim 128, 256 or 512."""

    def __init__(self, d_model: int, num_heads: int, rkhs_dim: int = 512, chunk_size: int = 64,
                 tau_init: float = 1.0):
        super().__init__()
        self.d_model = d_model
        self.num_heads = num_heads
        self.d_head = d_model // num_heads
        self.rkhs_dim = rkhs_dim
        self.chunk_size = chunk_size
        self.w_q = nn.Linear(d_model, d_model, bias=False)
        self.w_k = nn.Linear(d_model, d_model, bias=False)
        self.w_v = nn.Linear(d_model, d_model, bias=False)
        self.w_out = nn.Linear(d_model, d_model, bias=False)
        self.w_beta = nn.Linear(d_model, num_heads, bias=False)
        self.w_decay = nn.Linear(d_model, num_heads, bias=False)
        self.raw_tau = nn.Parameter(torch.full((num_heads, 1), float(tau_init)))
        self.register_buffer("omega", self._orthogonal_features())
        self.register_buffer("b_rff", torch.empty(num_heads, rkhs_dim).uniform_(0, 2 * math.pi))

    def _orthogonal_features(self) -> torch.Tensor:
        """Per head: stacked d_head x d_head orthogonal blocks, columns scaled by chi(d_head) radii,
        truncated to rkhs_dim rows (orthogonal random features, :228-237)."""
        d = self.d_head
        n_blocks = -(-self.rkhs_dim // d)
        heads = []
        for _ in range(self.num_heads):
            rows = []
            for _ in range(n_blocks):
                qmat, _ = torch.linalg.qr(torch.randn(d, d))
                radii = torch.randn(d, d).pow(2).sum(dim=0, keepdim=True).sqrt()
                rows.append(qmat * radii)
            heads.append(torch.cat(rows, dim=0)[: self.rkhs_dim])
        return torch.stack(heads, dim=0)

    def get_tau(self) -> torch.Tensor:
        return F.softplus(self.raw_tau) + 1e-4

    def forward(self, x: torch.Tensor, state: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        B, T, _ = x.shape
        H, dh = self.num_heads, self.d_head
        # (B, T, H, d) views of the projections are what the scan reads; no head transposes are made
        q = self.w_q(x).view(B, T, H, dh)
        k = self.w_k(x).view(B, T, H, dh)
        v = self.w_v(x).view(B, T, H, dh)
        beta = torch.sigmoid(self.w_beta(x))
        decay = torch.sigmoid(self.w_decay(x))
        tau = self.get_tau()
        if torch.is_grad_enabled():
            # differentiable end to end: the scan's backward (kdn_delta_scan_bwd) gives q, k, v, beta, decay,
            # the state and 1/tau their gradients, autograd the rest (projections, softplus of raw_tau)
            fm = _feature_map(self.omega, self.b_rff, None, x.device)
            inv_tau = 1.0 / tau.reshape(H).to(torch.float32)
            init = None if state is None else state.to(device=x.device, dtype=torch.float32).transpose(2, 3)
            y, final = ops.feature_scan_autograd(q, k, v, beta.to(torch.float32), decay.to(torch.float32), fm.omega,
                                                 fm.phase, inv_tau, omega_lo=fm.omega_lo, no_renorm=True,
                                                 normalize=True, initial_state=init)
            return self.w_out(y.reshape(B, T, self.d_model)), final.transpose(2, 3).to(x.dtype)
        y = torch.empty(B, T, H, dh, device=x.device, dtype=q.dtype)
        _, final = kernel_deltanet_scan(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), self.omega,
                                        self.b_rff, tau, beta.transpose(1, 2), decay.transpose(1, 2),
                                        initial_state=state, y=y.transpose(1, 2))
        return self.w_out(y.view(B, T, self.d_model)), final.to(x.dtype)
