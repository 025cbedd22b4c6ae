"""Multi-head Kernel-DeltaNet layer -- drop-in for the reference module layers/kernel_deltanet_layer.py.

Same names and signatures as the reference (layers/kernel_deltanet_layer.py:20-147):
  KernelDeltaNetLayer(d_model, num_heads, rkhs_factor=4, chunk_size=64, gamma_init=2.0, initial_decay=0.99,
                      initial_eta=0.5).forward(x (B, T, d_model), state=None) -> (out, None | state)
with the parameters w_q, w_k, w_v, w_out, kernel.log_gamma, kernel.omega, logit_decay, raw_eta.

What runs (the layer's recurrence, core/chunked_scan.py:145-186 of the reference, in both modes):
  q_hat, k_hat = F.normalize(W_q x), F.normalize(W_k x)  per head          (:101-102)
  phi(x) = [cos(a), sin(a)] / sqrt(m),  a = sqrt(2 gamma_h) x Omega_h^T      (core/rkhs_features.py:107-131)
  y_t = S_{t-1} phi(q_t),  S_t = lambda_h S_{t-1} + eta_h v_t phi(k_t)^T        (no erasure term)
with lambda_h = sigmoid(logit_decay_h), eta_h = softplus(raw_eta_h).  The reference's chunked prefill
(core/chunked_scan.py:48-143) is an exact form of the same recurrence, so prefill and step outputs agree.

On the device the scan kernels lift in-register.  [cos(a), sin(a)] / sqrt(m) is written as
sqrt(2/D) cos(x Omega'^T / tau_h + phase) with Omega' = [Omega; Omega] (D = 2m rows, as hi + lo bf16
parts), phase = [0; -pi/2], 1/tau_h = sqrt(2 gamma_h) and no renormalisation; beta = eta_h and
lambda = lambda_h reach the kernels as stride-0 (B, T, H) views, and the update runs as the linear rule
(kdn_scan_args.rule = 1).  The state is carried in fp32.

Differences from the reference, all outside the ranges the layer produces: F.normalize's eps is 1e-6
here (1e-12 there), and lambda is clamped below at 1e-5 (lambda_h < 1e-5 needs logit_decay < -11.5).
The device path needs d_model / num_heads = 64 and rkhs_dim = d_head * rkhs_factor in {128, 256, 512}
(rkhs_factor 2, 4 (the default) or 8); other sizes raise.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from kdn import ops


class MultiHeadRKHSKernel(nn.Module):
    """Random Fourier features with a learnable bandwidth per head (reference core/rkhs_features.py:43-131):
    parameter `log_gamma` (H,) and buffer `omega` (H, m, d_head), m = rkhs_dim / 2.

    The features are never materialised on the device path: `feature_map()` hands the scan kernels the
    equivalent shifted-cosine lift.  Calling the module to materialise phi is not supported here."""

    def __init__(self, num_heads: int, d_head: int, rkhs_dim: int, gamma_init: float = 2.0,
                 orthogonal: bool = True):
        super().__init__()
        if rkhs_dim % 2 != 0:
            raise ValueError("rkhs_dim must be even for the sin/cos features")
        self.num_heads = num_heads
        self.d_head = d_head
        self.rkhs_dim = rkhs_dim
        self.m = rkhs_dim // 2
        self.orthogonal = orthogonal
        if num_heads == 1:
            gammas = torch.tensor([float(gamma_init)])
        else:
            # bandwidths spread log-uniformly from gamma_init / 5 to max(4 gamma_init, 10) (:66-72)
            gammas = torch.logspace(math.log10(gamma_init * 0.2), math.log10(max(gamma_init * 4.0, 10.0)),
                                    steps=num_heads)
        self.log_gamma = nn.Parameter(torch.log(gammas))
        self.register_buffer("omega", self._draw_omega())

    def _draw_omega(self) -> torch.Tensor:
        """Gaussian rows, or orthogonal d_head x d_head blocks with chi(d_head) row radii (:79-101)."""
        if not self.orthogonal:
            return torch.randn(self.num_heads, self.m, self.d_head)
        d = self.d_head
        n_blocks = -(-self.m // d)
        heads = []
        for _ in range(self.num_heads):
            blocks = []
            for _ in range(n_blocks):
                qmat, _ = torch.linalg.qr(torch.randn(d, d))
                radii = torch.randn(d, d).pow(2).sum(dim=-1, keepdim=True).sqrt()
                blocks.append(qmat * radii)
            heads.append(torch.cat(blocks, dim=0)[: self.m])
        return torch.stack(heads, dim=0)

    def get_bandwidths(self) -> torch.Tensor:
        return torch.exp(self.log_gamma)

    def feature_map(self, device) -> ops.FeatureMap:
        """The scan's lift that reproduces [cos(a), sin(a)] / sqrt(m): Omega' = [Omega; Omega] as hi + lo bf16
        parts, phase [0; -pi/2], 1/tau_h = sqrt(2 gamma_h), no renormalisation."""
        with torch.no_grad():
            om = self.omega.to(device=device, dtype=torch.float32)
            om2 = torch.cat([om, om], dim=1)
            hi = om2.to(torch.bfloat16)
            lo = (om2 - hi.to(torch.float32)).to(torch.bfloat16)
            phase = torch.cat([torch.zeros(self.m), torch.full((self.m,), -math.pi / 2)]).to(device)
            inv_tau = torch.sqrt(2.0 * torch.exp(self.log_gamma.detach().to(device=device, dtype=torch.float32)))
        return ops.FeatureMap(omega=hi.contiguous(), phase=phase, omega_lo=lo.contiguous(),
                              inv_tau_head=inv_tau.contiguous(), no_renorm=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError("MultiHeadRKHSKernel: materialised features are not part of the MI355X "
                                  "path; KernelDeltaNetLayer lifts inside the scan kernels")


class KernelDeltaNetLayer(nn.Module):
    """Reference: layers/kernel_deltanet_layer.py:20-143."""

    def __init__(self, d_model: int, num_heads: int, rkhs_factor: int = 4, chunk_size: int = 64,
                 gamma_init: float = 2.0, initial_decay: float = 0.99, initial_eta: float = 0.5):
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError(f"d_model ({d_model}) must be divisible by num_heads ({num_heads})")
        self.d_model = d_model
        self.num_heads = num_heads
        self.d_head = d_model // num_heads
        self.rkhs_factor = rkhs_factor
        self.rkhs_dim = self.d_head * rkhs_factor
        self.chunk_size = chunk_size
        self.w_q = nn.Linear(d_model, d_model, bias=False)
        self.w_k = nn.Linear(d_model, d_model, bias=False)
        self.w_v = nn.Linear(d_model, d_model, bias=False)
        self.w_out = nn.Linear(d_model, d_model, bias=False)
        self.kernel = MultiHeadRKHSKernel(num_heads=num_heads, d_head=self.d_head, rkhs_dim=self.rkhs_dim,
                                          gamma_init=gamma_init, orthogonal=True)
        logit = math.log(initial_decay / (1.0 - initial_decay + 1e-7))
        self.logit_decay = nn.Parameter(torch.full((1, num_heads, 1, 1), float(logit)))
        raw_eta = math.log(math.exp(initial_eta) - 1.0 + 1e-7)
        self.raw_eta = nn.Parameter(torch.full((1, num_heads, 1, 1), float(raw_eta)))

    def get_decay(self) -> torch.Tensor:
        return torch.sigmoid(self.logit_decay)

    def get_eta(self) -> torch.Tensor:
        return F.softplus(self.raw_eta)

    def forward(self, x: torch.Tensor, state: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Prefill (state None, T > 1) returns (out, None); step mode (a state, or T == 1) returns
        (out, new state (B, H, d_head, rkhs_dim)) -- reference :76-143."""
        B, T, d_in = x.shape
        H, dh, D = self.num_heads, self.d_head, self.rkhs_dim
        if dh != 64 or D not in (128, 256, 512):
            raise ValueError(f"KernelDeltaNetLayer on MI355X needs d_head = 64 and rkhs_dim 128, 256 or 512 "
                             f"(rkhs_factor 2, 4 or 8); got d_head = {dh}, rkhs_dim = {D}")
        step_mode = state is not None or T == 1
        q = self.w_q(x).view(B, T, H, dh)
        k = self.w_k(x).view(B, T, H, dh)
        v = self.w_v(x).view(B, T, H, dh)
        lam = self.get_decay().reshape(H)
        eta = self.get_eta().reshape(H)
        if state is not None and tuple(state.shape) != (B, H, dh, D):
            raise ValueError(f"state must be (B, H, d_head, rkhs_dim) = {(B, H, dh, D)}")
        if torch.is_grad_enabled():
            # differentiable end to end: the scan's backward (kdn_delta_scan_bwd, linear rule) gives q, k, v,
            # the per-token eta and lambda (summed over the stride-0 views by autograd), the state and
            # 1/tau_h = sqrt(2 gamma_h) their gradients; autograd the rest (projections, log_gamma, logits)
            fm = self.kernel.feature_map(x.device)
            inv_tau = torch.sqrt(2.0 * torch.exp(self.kernel.log_gamma.to(device=x.device, dtype=torch.float32)))
            beta = eta.to(torch.float32).view(1, 1, H).expand(B, T, H)
            decay = lam.to(torch.float32).view(1, 1, H).expand(B, T, H)
            init = None if state is None else state.to(device=x.device, dtype=torch.float32).transpose(2, 3)
            y, final = ops.feature_scan_autograd(q, k, v, beta, decay, fm.omega, fm.phase, inv_tau,
                                                 omega_lo=fm.omega_lo, no_renorm=True, normalize=True,
                                                 initial_state=init, rule=ops.RULE_LINEAR)
            out = self.w_out(y.reshape(B, T, d_in))
            return out, (final.transpose(2, 3).to(x.dtype) if step_mode else None)
        y = torch.empty(B, T, H, dh, device=x.device, dtype=q.dtype)
        final = torch.empty(B, H, dh, D, device=x.device, dtype=torch.float32)
        init = None if state is None else state.to(device=x.device, dtype=torch.float32).transpose(2, 3)
        beta = eta.to(torch.float32).view(1, 1, H).expand(B, T, H)
        decay = lam.to(torch.float32).view(1, 1, H).expand(B, T, H)
        ops.scan(q, k, v, beta, decay, None, None, 1.0, normalize=True, initial_state=init,
                 final_state=final.transpose(2, 3), y=y, features=self.kernel.feature_map(x.device),
                 rule=ops.RULE_LINEAR)
        out = self.w_out(y.view(B, T, d_in))
        return out, (final.to(x.dtype) if step_mode else None)


# the reference's backwards-compatibility alias (:147)
KernelTTTLayer = KernelDeltaNetLayer
