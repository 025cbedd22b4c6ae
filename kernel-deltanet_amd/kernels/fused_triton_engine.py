"""`fused_triton_chunk_scan` -- the reference's entry point (kernels/fused_triton_engine.py:123-169) with
its signature and its T % chunk_size assertion, over pre-lifted features.  No Triton here: it runs the
exact delta-rule scan kernels of libkdn.so (kernels/lifted_scan.py).  The reference kernel behind this
name drops the erasure term and the in-chunk decay (:78-115), so its outputs differ from these by design.
"""
from __future__ import annotations

import torch

from .lifted_scan import lifted_delta_scan


def fused_triton_chunk_scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                            decay: torch.Tensor, chunk_size: int = 64) -> torch.Tensor:
    """q, k (B, H, T, D) features; v (B, H, T, d_v); beta, decay (B, H, T).  Returns bf16 (B, H, T, d_v)."""
    T = q.shape[2]
    assert T % chunk_size == 0, f"Sequence length T={T} must be divisible by chunk_size={chunk_size}"
    return lifted_delta_scan(q, k, v, beta, decay, "fused_triton_chunk_scan")
