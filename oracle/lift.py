"""Oracle restatement of the structured-FWHT feature lift -- TEST INFRASTRUCTURE ONLY.

Follows the reference file kernels/fwht.py (jatin-yadav-acad/kernel-deltanet):
  make_projection  <- FastWalshHadamardProjection.__init__, kernels/fwht.py:54-111
  fwht_rows        <- fast_walsh_hadamard_transform,       kernels/fwht.py:25-45
  lift             <- FastWalshHadamardProjection.forward,  kernels/fwht.py:122-131 (torch branch)
  rff_features     <- the per-head random-feature lift of the P2 module, kernels/kernel_deltanet_fused.py:85-92,
                      113-117 and 286-287 (spherical normalisation, Omega (H, D, d_k), phases (H, D), tau (H,))
  rkhs_features    <- MultiHeadRKHSKernel.forward, core/rkhs_features.py:107-131 ([cos, sin] / sqrt(m))
"""
from __future__ import annotations

import math

import numpy as np
import torch


def hadamard(n: int) -> np.ndarray:
    """Natural-order (Sylvester) Hadamard matrix, built by the recursion of kernels/fwht.py:97-99."""
    h = np.ones((1, 1), dtype=np.int64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def make_projection(d_k: int = 64, D: int = 512, seed: int = 42) -> dict:
    """Seeded tables of FastWalshHadamardProjection (kernels/fwht.py:54-111).

    Draw order (kernels/fwht.py:66-86): one CPU torch.Generator seeded with `seed`; d1, d2, d3 =
    where(rand(M, d_k) > 0.5, +1, -1) in that order; then b = rand(D) * 2 pi.  The bit table packs
    bit i of column s of row m as (d_s[m, i] < 0) (kernels/fwht.py:74-83), stored as int64 (the
    uint64 pattern reinterpreted).  Omega[D][d_k] = concat_m H D3_m H D2_m H D1_m / sqrt(d_k), computed
    here in exact integer arithmetic (every entry of H D3 H D2 H D1 is an integer).
    """
    assert D % d_k == 0
    M = D // d_k
    gen = torch.Generator().manual_seed(seed)
    d1 = torch.where(torch.rand(M, d_k, generator=gen) > 0.5, 1.0, -1.0)
    d2 = torch.where(torch.rand(M, d_k, generator=gen) > 0.5, 1.0, -1.0)
    d3 = torch.where(torch.rand(M, d_k, generator=gen) > 0.5, 1.0, -1.0)
    b = torch.rand(D, generator=gen) * (2.0 * math.pi)

    signs = [d1.numpy().astype(np.int64), d2.numpy().astype(np.int64), d3.numpy().astype(np.int64)]
    bits = np.zeros((M, 3), dtype=np.uint64)
    for m in range(M):
        for s in range(3):
            word = 0
            for i in range(min(64, d_k)):
                if signs[s][m, i] < 0:
                    word |= 1 << i
            bits[m, s] = np.uint64(word)
    bits_i64 = bits.view(np.int64)

    H = hadamard(d_k)
    blocks = []
    for m in range(M):
        W = H @ np.diag(signs[2][m]) @ H @ np.diag(signs[1][m]) @ H @ np.diag(signs[0][m])
        blocks.append(W)
    omega_int = np.concatenate(blocks, axis=0)  # integer matrix = Omega * sqrt(d_k)
    omega = omega_int.astype(np.float64) / math.sqrt(d_k)
    return {
        "d_k": d_k,
        "D": D,
        "M": M,
        "seed": seed,
        "d1": d1.numpy(),
        "d2": d2.numpy(),
        "d3": d3.numpy(),
        "bits": bits_i64,
        "b": b.numpy().astype(np.float32),
        "omega": omega,
        "omega_int": omega_int,
        "tau_star": float(d_k) ** 0.25,
    }


def fwht_rows(x: np.ndarray) -> np.ndarray:
    """Unnormalised natural-order FWHT along the last axis, strides h = 1, 2, 4, ...

    Butterfly of kernels/fwht.py:35-44: pairs (u, v) at distance h become (u + v, u - v).
    """
    res = np.array(x, dtype=np.float64, copy=True)
    n = res.shape[-1]
    assert n & (n - 1) == 0
    h = 1
    lead = res.shape[:-1]
    while h < n:
        r = res.reshape(*lead, n // (2 * h), 2, h)
        u = r[..., 0, :].copy()
        v = r[..., 1, :].copy()
        r[..., 0, :] = u + v
        r[..., 1, :] = u - v
        res = r.reshape(*lead, n)
        h *= 2
    return res


def omega_by_butterfly(proj: dict) -> np.ndarray:
    """Omega built column by column with the butterfly instead of matrix products (an independent check)."""
    d_k, M = proj["d_k"], proj["M"]
    out = np.zeros((proj["D"], d_k), dtype=np.float64)
    for m in range(M):
        e = np.eye(d_k) * proj["d1"][m][None, :]  # column j = d1[j] e_j, laid out as rows here
        y = fwht_rows(e)
        y = y * proj["d2"][m][None, :]
        y = fwht_rows(y)
        y = y * proj["d3"][m][None, :]
        y = fwht_rows(y)
        out[m * d_k:(m + 1) * d_k, :] = y.T / math.sqrt(d_k)
    return out


def normalize_rows(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """F.normalize(x, p=2, dim=-1, eps) (kernels/kernel_deltanet_fused.py:90-91)."""
    n = np.sqrt(np.sum(np.asarray(x, dtype=np.float64) ** 2, axis=-1, keepdims=True))
    return np.asarray(x, dtype=np.float64) / np.maximum(n, eps)


def lift(x: np.ndarray, proj: dict, normalize: bool = False) -> np.ndarray:
    """phi_hat = phi / (||phi|| + 1e-8), phi = sqrt(2/D) cos(x Omega^T / tau* + b)  (kernels/fwht.py:122-131).

    Float64 throughout.  `normalize` applies F.normalize (eps 1e-6) to x first, as the BASELINE lift
    configuration and kernels/kernel_deltanet_fused.py:90-91 do.
    """
    xx = np.asarray(x, dtype=np.float64)
    if normalize:
        xx = normalize_rows(xx)
    proj_ = xx @ proj["omega"].T
    scaled = proj_ / proj["tau_star"] + proj["b"].astype(np.float64)
    phi = math.sqrt(2.0 / proj["D"]) * np.cos(scaled)
    return phi / (np.linalg.norm(phi, axis=-1, keepdims=True) + 1e-8)


def factored_lift(x: np.ndarray, proj1: dict, proj2: dict) -> np.ndarray:
    """FactoredFastWalshHadamardProjection.forward (kernels/factored_kernel_deltanet.py:62-74), float64:
    the two halves of x lifted by `lift` with the projections of seeds s and s + 1000
    (:57-58), concatenated and divided by (norm + 1e-7)."""
    xx = np.asarray(x, dtype=np.float64)
    d0 = xx.shape[-1] // 2
    phi = np.concatenate([lift(xx[..., :d0], proj1), lift(xx[..., d0:], proj2)], axis=-1)
    return phi / (np.linalg.norm(phi, axis=-1, keepdims=True) + 1e-7)


def rff_features(x: np.ndarray, omega: np.ndarray, phase: np.ndarray, tau, normalize: bool = True,
                 renorm: bool = False) -> np.ndarray:
    """phi = sqrt(2/D) cos(x_hat Omega_h^T / tau_h + b_h), per head; float64.

    x (B, H, T, d_k); omega (H, D, d_k); phase (H, D); tau (H,) or a scalar.  `normalize` applies
    F.normalize (eps 1e-6) to x (kernels/kernel_deltanet_fused.py:90-91, 286-287); the P2 module does not
    renormalise phi (`renorm` adds the division by ||phi|| + 1e-8 of kernels/fwht.py:131).
    """
    xx = np.asarray(x, dtype=np.float64)
    if normalize:
        xx = normalize_rows(xx)
    om = np.asarray(omega, dtype=np.float64)
    H, D, _ = om.shape
    tt = np.broadcast_to(np.asarray(tau, dtype=np.float64).reshape(-1), (H,))
    ang = np.einsum("bhtd,hfd->bhtf", xx, om) / tt[None, :, None, None] \
        + np.asarray(phase, dtype=np.float64)[None, :, None, :]
    phi = math.sqrt(2.0 / D) * np.cos(ang)
    if renorm:
        phi = phi / (np.linalg.norm(phi, axis=-1, keepdims=True) + 1e-8)
    return phi


def rkhs_features(x: np.ndarray, omega: np.ndarray, log_gamma: np.ndarray) -> np.ndarray:
    """MultiHeadRKHSKernel.forward (core/rkhs_features.py:107-131) in float64.

    x (B, H, T, d_head); omega (H, m, d_head); log_gamma (H,).  Returns (B, H, T, 2m):
    [cos(sqrt(2 gamma_h) x Omega_h^T), sin(same)] / sqrt(m).
    """
    xx = np.asarray(x, dtype=np.float64)
    om = np.asarray(omega, dtype=np.float64)
    m = om.shape[1]
    gamma = np.exp(np.asarray(log_gamma, dtype=np.float64))
    ang = np.einsum("bhtd,hmd->bhtm", xx, om) * np.sqrt(2.0 * gamma)[None, :, None, None]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=-1) / math.sqrt(m)
