"""The scan over pre-lifted features shared by the Triton-named entry points (fused_triton_engine,
tiled_triton_engine).  q and k are the features phi(q), phi(k) (B, H, T, D) themselves; the update is the
exact gated delta rule with readout before update, y_t = S_{t-1} q_t,
S_t = lambda_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T, from S_0 = 0, run by the gfx950 scan
kernels in feature mode 1 (kdn_scan_args.feature_mode).  The output is bf16 (B, H, T, d_v), as the
reference's entry points return.
"""
from __future__ import annotations

from typing import Optional

import torch

from kdn import ops


def lifted_delta_scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                      decay: Optional[torch.Tensor], what: str) -> torch.Tensor:
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"{what}: expected q, k (B, H, T, D) and v (B, H, T, d_v); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, H, T, D = q.shape
    if tuple(beta.shape) != (B, H, T) or (decay is not None and tuple(decay.shape) != (B, H, T)):
        raise ValueError(f"{what}: beta and decay must be (B, H, T) = {(B, H, T)}")
    if D != 512:
        raise ValueError(f"{what}: the MI355X scan takes D = 512 features; got D = {D}")
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta")):
        ops.require_device(t, f"{what}: {nm}")
    dt = q.dtype if q.dtype in (torch.bfloat16, torch.float32) else torch.float32
    y = torch.empty(B, H, T, v.shape[-1], device=q.device, dtype=torch.bfloat16)
    with torch.no_grad():
        ops.scan(q.to(dt).transpose(1, 2), k.to(dt).transpose(1, 2), v.to(dt).transpose(1, 2),
                 beta.to(torch.float32).transpose(1, 2),
                 None if decay is None else decay.to(torch.float32).transpose(1, 2),
                 None, None, 1.0, y=y.transpose(1, 2), features=ops.FeatureMap(lifted=True))
    return ops.forward_only(what, (y,), (q, k, v, beta, decay))[0]
