"""`tiled_triton_chunk_scan` and `streaming_triton_chunk_scan` -- the reference's entry points
(kernels/tiled_triton_engine.py:109-145 and 228-266) with their signatures, over pre-lifted features.  No
Triton here: both run the exact delta-rule scan kernels of libkdn.so (kernels/lifted_scan.py), whose
state rows are split over workgroups by value components, not by feature tiles, so `block_d` only keeps
the reference's D % block_d check.  The reference kernels behind these names use per-tile partial
products for the erasure term (:101-106), so their outputs differ from these by design.
"""
from __future__ import annotations

import torch

from .lifted_scan import lifted_delta_scan


def tiled_triton_chunk_scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                            decay: torch.Tensor, chunk_size: int = 64, block_d: int = 64) -> torch.Tensor:
    """q, k (B, H, T, D) features; v (B, H, T, d_v); beta, decay (B, H, T).  Returns bf16 (B, H, T, d_v)."""
    D = q.shape[-1]
    assert D % block_d == 0, f"D={D} must be divisible by block_d={block_d}"
    return lifted_delta_scan(q, k, v, beta, decay, "tiled_triton_chunk_scan")


def streaming_triton_chunk_scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                                decay: torch.Tensor, chunk_size: int = 64, block_d: int = 64) -> torch.Tensor:
    """As tiled_triton_chunk_scan (the reference's streaming variant differs only in how it reduces)."""
    return lifted_delta_scan(q, k, v, beta, decay, "streaming_triton_chunk_scan")
