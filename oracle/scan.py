"""Oracle restatement of the chunked delta-rule scan -- TEST INFRASTRUCTURE ONLY.

  token_recurrence  <- the defining recurrence, readout before update:
                       reference tests/test_fused_kernel.py:53-65 and kernels/kernel_deltanet_fused.py:288-300
  chunked_forward   <- fused_chunked_deltanet_forward, kernels/fused_kernel_deltanet.py:47-155, op for op
                       (torch on the CPU, compute dtype selectable, state carried in the compute dtype)
  delta_rule        <- lift (oracle.lift) followed by token_recurrence, float64: the parity definition.
  linear_recurrence <- recurrent_step of the P4 layer, core/chunked_scan.py:145-186 (no erasure term):
                       y_t = S_{t-1} phi_q(t);  S_t = lambda_t S_{t-1} + beta_t v_t phi_k(t)^T
  linear_chunked    <- chunked_affine_scan, core/chunked_scan.py:48-143 (per-head constant lambda, eta)
  *_torch           <- the same definitions on torch tensors, for autograd (the gradient oracle):
                       token_recurrence_torch, delta_rule_torch (lift of kernels/fwht.py:122-131),
                       linear_recurrence_torch, rff_features_torch (the per-head feature map of the P2
                       module, kernels/kernel_deltanet_fused.py:238-251, and of the P4 layer's shifted
                       [cos, sin] form, core/rkhs_features.py:107-131), factored_lift_torch (the d_k = 128
                       factored lift, kernels/factored_kernel_deltanet.py:60-74)
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

from . import lift as olift


def token_recurrence(phi_q, phi_k, v, beta, decay=None, S0=None) -> Tuple[np.ndarray, np.ndarray]:
    """y_t = S_{t-1} phi_q(t);  S_t = lambda_t (S_{t-1} - beta_t (S_{t-1} phi_k(t)) phi_k(t)^T) + beta_t v_t phi_k(t)^T.

    Shapes: phi_q, phi_k (B, T, D); v (B, T, d_v); beta, decay (B, T); S0 (B, d_v, D).  Float64.
    Follows tests/test_fused_kernel.py:53-65 line for line (batched over B).
    """
    pq = np.asarray(phi_q, dtype=np.float64)
    pk = np.asarray(phi_k, dtype=np.float64)
    vv = np.asarray(v, dtype=np.float64)
    bb = np.asarray(beta, dtype=np.float64)
    B, T, D = pk.shape
    dv = vv.shape[-1]
    ll = np.ones((B, T)) if decay is None else np.asarray(decay, dtype=np.float64)
    S = np.zeros((B, dv, D)) if S0 is None else np.array(S0, dtype=np.float64, copy=True)
    Y = np.zeros((B, T, dv))
    for t in range(T):
        Y[:, t] = np.einsum("bvd,bd->bv", S, pq[:, t])
        s_phi = np.einsum("bvd,bd->bv", S, pk[:, t])
        S = ll[:, t, None, None] * (S - bb[:, t, None, None] * s_phi[:, :, None] * pk[:, t, None, :]) \
            + bb[:, t, None, None] * vv[:, t, :, None] * pk[:, t, None, :]
    return Y, S


def token_recurrence_torch(phi_q: torch.Tensor, phi_k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                           decay: Optional[torch.Tensor] = None, S0: Optional[torch.Tensor] = None
                           ) -> Tuple[torch.Tensor, torch.Tensor]:
    """token_recurrence on torch tensors, so that autograd differentiates the defining rule: the same
    loop (tests/test_fused_kernel.py:53-65), with lambda clamped to [1e-5, 1] as the forward clamps
    log lambda (kernels/fused_kernel_deltanet.py:74).  The gradient oracle of the backward pass, the
    role the reference gives torch autograd over its forward (kernels/fused_kernel_deltanet.py:168-179).
    Shapes as token_recurrence; returns (Y (B, T, d_v), S (B, d_v, D))."""
    B, T, D = phi_k.shape
    dv = v.shape[-1]
    S = torch.zeros(B, dv, D, dtype=phi_k.dtype) if S0 is None else S0
    ys = []
    for t in range(T):
        ys.append(torch.einsum("bvd,bd->bv", S, phi_q[:, t]))
        s_phi = torch.einsum("bvd,bd->bv", S, phi_k[:, t])
        lam = 1.0 if decay is None else decay[:, t].clamp(1e-5, 1.0)[:, None, None]
        b = beta[:, t, None, None]
        S = lam * (S - b * s_phi[:, :, None] * phi_k[:, t, None, :]) + b * v[:, t, :, None] * phi_k[:, t, None, :]
    return torch.stack(ys, 1), S


def linear_recurrence_torch(phi_q: torch.Tensor, phi_k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                            decay: Optional[torch.Tensor] = None, S0: Optional[torch.Tensor] = None
                            ) -> Tuple[torch.Tensor, torch.Tensor]:
    """linear_recurrence on torch tensors (core/chunked_scan.py:145-186 with eta -> beta_t, decay ->
    lambda_t, lambda clamped to [1e-5, 1] as the scan clamps log lambda), for autograd.  Shapes as
    token_recurrence; returns (Y (B, T, d_v), S (B, d_v, D))."""
    B, T, D = phi_k.shape
    dv = v.shape[-1]
    S = torch.zeros(B, dv, D, dtype=phi_k.dtype) if S0 is None else S0
    ys = []
    for t in range(T):
        ys.append(torch.einsum("bvd,bd->bv", S, phi_q[:, t]))
        lam = 1.0 if decay is None else decay[:, t].clamp(1e-5, 1.0)[:, None, None]
        S = lam * S + beta[:, t, None, None] * v[:, t, :, None] * phi_k[:, t, None, :]
    return torch.stack(ys, 1), S


def rff_features_torch(x: torch.Tensor, omega: torch.Tensor, phase: torch.Tensor, inv_tau: torch.Tensor,
                       normalize: bool = True, renorm: bool = False) -> torch.Tensor:
    """oracle.lift.rff_features on torch tensors, with 1/tau as the (differentiable) per-head input:
    phi = sqrt(2/D) cos(x_hat Omega_h^T inv_tau_h + phase_h), optionally renormalised.

    x (B, H, T, d_k); omega (H, D, d_k); phase (H, D); inv_tau (H,).  Returns (B, H, T, D)."""
    if normalize:
        x = F.normalize(x, p=2, dim=-1, eps=1e-6)
    D = omega.shape[1]
    ang = torch.einsum("bhtd,hfd->bhtf", x, omega) * inv_tau[None, :, None, None] + phase[None, :, None, :]
    phi = math.sqrt(2.0 / D) * torch.cos(ang)
    if renorm:
        phi = phi / (torch.norm(phi, dim=-1, keepdim=True) + 1e-8)
    return phi


def delta_rule_torch(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                     decay: Optional[torch.Tensor], proj: dict, initial_state: Optional[torch.Tensor] = None,
                     normalize: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """delta_rule on torch tensors (lift by _torch_lift, then token_recurrence_torch): differentiable
    end to end, in the inputs' dtype (float64 for the gradient oracle)."""
    return token_recurrence_torch(_torch_lift(q, proj, normalize), _torch_lift(k, proj, normalize), v, beta, decay,
                                  initial_state)


def factored_lift_torch(x: torch.Tensor, proj1: dict, proj2: dict) -> torch.Tensor:
    """oracle.lift.factored_lift on torch tensors (FactoredFastWalshHadamardProjection.forward,
    kernels/factored_kernel_deltanet.py:60-74): the halves of x lifted by _torch_lift with the projections
    of seeds s and s + 1000, concatenated and divided by (norm + 1e-7); differentiable."""
    d0 = x.shape[-1] // 2
    phi = torch.cat([_torch_lift(x[..., :d0], proj1, False), _torch_lift(x[..., d0:], proj2, False)], dim=-1)
    return phi / (torch.norm(phi, dim=-1, keepdim=True) + 1e-7)


def delta_rule(q, k, v, beta, decay, proj: dict, initial_state=None, normalize: bool = False):
    """Float64 definition of the whole path: lift q and k, then the token recurrence."""
    return token_recurrence(olift.lift(q, proj, normalize), olift.lift(k, proj, normalize), v, beta, decay,
                            initial_state)


def _torch_lift(x: torch.Tensor, proj: dict, normalize: bool) -> torch.Tensor:
    """kernels/fwht.py:122-131 in the tensor's dtype (CPU)."""
    if normalize:
        x = F.normalize(x, p=2, dim=-1, eps=1e-6)
    omega = torch.as_tensor(proj["omega"], dtype=x.dtype)
    b = torch.as_tensor(proj["b"]).to(x.dtype)
    p = torch.matmul(x, omega.T)
    s = p / proj["tau_star"] + b
    phi = math.sqrt(2.0 / proj["D"]) * torch.cos(s)
    return phi / (torch.norm(phi, dim=-1, keepdim=True) + 1e-8)


def chunked_forward(q, k, v, beta, decay, proj: dict, chunk_size: int = 64,
                    initial_state: Optional[torch.Tensor] = None, dtype=torch.float64,
                    normalize: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Op-for-op CPU restatement of kernels/fused_kernel_deltanet.py:47-155.

    q, k (B, T, d_k); v (B, T, d_v); beta, decay (B, T); initial_state (B, d_v, D).  All arithmetic in
    `dtype` (the reference uses the input dtype for the lift and the state and fp32 for the solves);
    the lift of each chunk is streamed as in :95-96.  Returns Y (B, T, d_v) and S (B, d_v, D).
    """
    q = torch.as_tensor(q).to(dtype)
    k = torch.as_tensor(k).to(dtype)
    v = torch.as_tensor(v).to(dtype)
    beta = torch.as_tensor(beta).to(dtype)
    decay = torch.ones_like(beta) if decay is None else torch.as_tensor(decay).to(dtype)
    B, T, d_k = k.shape
    d_v = v.shape[-1]
    D = proj["D"]
    C = chunk_size
    remainder = T % C                                                       # :55-62
    pad_len = (C - remainder) if remainder != 0 else 0
    if pad_len > 0:
        q = F.pad(q, (0, 0, 0, pad_len))
        k = F.pad(k, (0, 0, 0, pad_len))
        v = F.pad(v, (0, 0, 0, pad_len))
        beta = F.pad(beta, (0, pad_len), value=0.0)
        decay = F.pad(decay, (0, pad_len), value=1.0)
    T_pad = T + pad_len
    nc = T_pad // C
    k_c = k.view(B, nc, C, d_k)                                             # :67-71
    q_c = q.view(B, nc, C, d_k)
    v_c = v.view(B, nc, C, d_v)
    beta_c = beta.view(B, nc, C)
    decay_c = decay.view(B, nc, C)
    log_d = torch.log(torch.clamp(decay_c, min=1e-5, max=1.0))            # :74-77
    cum_log_d = torch.cumsum(log_d, dim=-1)
    log_d_diff = cum_log_d.unsqueeze(-1) - cum_log_d.unsqueeze(-2)
    gamma_pairwise = torch.exp(torch.clamp(log_d_diff, max=0.0))
    upper_mask = torch.triu(torch.ones(C, C, dtype=dtype), 1).view(1, 1, C, C)   # :79-81
    lower_mask = torch.tril(torch.ones(C, C, dtype=dtype), -1).view(1, 1, C, C)
    eye_C = torch.eye(C, dtype=dtype).view(1, 1, C, C)
    if initial_state is not None:                                           # :83-86
        S = torch.as_tensor(initial_state).to(dtype).clone()
    else:
        S = torch.zeros(B, d_v, D, dtype=dtype)
    Y = torch.empty(B, nc, C, d_v, dtype=dtype)
    for c in range(nc):                                                     # :93
        pk = _torch_lift(k_c[:, c], proj, normalize)                        # :95-96
        pq = _torch_lift(q_c[:, c], proj, normalize)
        G_kk = torch.matmul(pk, pk.transpose(-1, -2)).unsqueeze(1)          # :99-100
        G_qk = torch.matmul(pq, pk.transpose(-1, -2)).unsqueeze(1)
        bc = beta_c[:, c:c + 1]                                             # :102-105
        U_bar = -(bc.unsqueeze(-2) * G_kk) * upper_mask
        inv_U = torch.linalg.solve_triangular(eye_C - U_bar, eye_C.expand(B, 1, C, C), upper=True)
        W_tilde = (bc.unsqueeze(-1) * inv_U).squeeze(1)                     # :107
        cum = cum_log_d[:, c:c + 1]                                         # :109-111
        g_i_to_C = torch.exp(cum[:, :, -1:] - cum)
        W_c = ((bc * g_i_to_C).unsqueeze(-1) * inv_U).squeeze(1)
        L_c = -(bc.unsqueeze(-1) * gamma_pairwise[:, c:c + 1] * G_kk) * lower_mask   # :113-116
        V_tilde = torch.linalg.solve_triangular(eye_C - L_c, bc.unsqueeze(-1) * v_c[:, c:c + 1],
                                                upper=False).squeeze(1)
        cum_shift = F.pad(cum[:, :, :-1], (1, 0), value=0.0)               # :119-122
        P_decay = torch.exp(torch.clamp(cum_shift.unsqueeze(-1) - cum.unsqueeze(-2), max=0.0))
        A_intra = (G_qk * P_decay * lower_mask).squeeze(1)
        Y_intra = torch.matmul(A_intra, V_tilde)
        S_K = torch.matmul(S, pk.transpose(-1, -2))                         # :128-141
        S_K_W = torch.matmul(S_K, W_tilde)
        A_corr = (G_qk.squeeze(1) * lower_mask.squeeze(1))
        inter_corr = torch.matmul(A_corr, S_K_W.transpose(-1, -2))
        Q_S = torch.matmul(pq, S.transpose(-1, -2))
        gamma_inter = torch.cat([torch.ones(B, 1, dtype=dtype), torch.exp(cum[:, 0, :-1])], dim=-1).unsqueeze(-1)
        Y[:, c] = Y_intra + gamma_inter * (Q_S - inter_corr)
        V_W = torch.matmul(v_c[:, c].transpose(-1, -2), W_c)               # :144-149
        delta_S = torch.matmul(V_W, pk)
        g0C = torch.exp(cum[:, :, -1:, None]).squeeze(1)
        S = g0C * (S - torch.matmul(S_K_W, pk)) + delta_S
    Yo = Y.view(B, T_pad, d_v)[:, :T]
    return Yo, S


def linear_recurrence(phi_q, phi_k, v, beta, decay=None, S0=None) -> Tuple[np.ndarray, np.ndarray]:
    """y_t = S_{t-1} phi_q(t);  S_t = lambda_t S_{t-1} + beta_t v_t phi_k(t)^T  (float64).

    The recurrent step of core/chunked_scan.py:145-186 with eta -> beta_t and decay -> lambda_t, batched
    over B.  Shapes as token_recurrence.
    """
    pq = np.asarray(phi_q, dtype=np.float64)
    pk = np.asarray(phi_k, dtype=np.float64)
    vv = np.asarray(v, dtype=np.float64)
    bb = np.asarray(beta, dtype=np.float64)
    B, T, D = pk.shape
    dv = vv.shape[-1]
    ll = np.ones((B, T)) if decay is None else np.asarray(decay, dtype=np.float64)
    S = np.zeros((B, dv, D)) if S0 is None else np.array(S0, dtype=np.float64, copy=True)
    Y = np.zeros((B, T, dv))
    for t in range(T):
        Y[:, t] = np.einsum("bvd,bd->bv", S, pq[:, t])
        S = ll[:, t, None, None] * S + bb[:, t, None, None] * vv[:, t, :, None] * pk[:, t, None, :]
    return Y, S


def linear_chunked(phi_q, phi_k, v, decay, eta, chunk_size: int = 64) -> np.ndarray:
    """chunked_affine_scan (core/chunked_scan.py:48-143) in float64: per-head constant lambda and eta.

    phi_q, phi_k (B, H, T, D); v (B, H, T, d_v); decay, eta (H,).  Returns y (B, H, T, d_v).  Intra-chunk
    weights eta lambda^{i-1-j} [i > j] on the q-k Gram, chunk states sum_j lambda^{C-1-j} v_j phi_j^T,
    carried as S <- lambda^C S + eta dS, inter-chunk readout lambda^i (S phi_q).
    """
    pq = np.asarray(phi_q, dtype=np.float64)
    pk = np.asarray(phi_k, dtype=np.float64)
    vv = np.asarray(v, dtype=np.float64)
    B, H, T, D = pk.shape
    dv = vv.shape[-1]
    lam = np.asarray(decay, dtype=np.float64).reshape(H)
    eta = np.asarray(eta, dtype=np.float64).reshape(H)
    C = chunk_size
    pad = (-T) % C
    if pad:
        z = lambda a: np.concatenate([a, np.zeros(a.shape[:2] + (pad, a.shape[-1]))], axis=2)
        pq, pk, vv = z(pq), z(pk), z(vv)
    n = (T + pad) // C
    pqc, pkc, vc = (a.reshape(B, H, n, C, a.shape[-1]) for a in (pq, pk, vv))
    i = np.arange(C)[:, None]
    j = np.arange(C)[None, :]
    powd = np.clip(i - 1 - j, 0, None)
    w = eta[:, None, None] * lam[:, None, None] ** powd[None] * (i > j)[None]   # (H, C, C)
    y_intra = np.einsum("bhnij,hij,bhnjv->bhniv", np.einsum("bhnid,bhnjd->bhnij", pqc, pkc), w, vc)
    tok = lam[:, None] ** (C - 1 - np.arange(C))[None]                           # (H, C)
    dS = np.einsum("bhnjv,hj,bhnjd->bhnvd", vc, tok, pkc)
    S = np.zeros((B, H, dv, D))
    y = np.zeros((B, H, n, C, dv))
    for c in range(n):
        y[:, :, c] = np.einsum("bhid,bhvd->bhiv", pqc[:, :, c], S) * (lam[:, None] ** np.arange(C))[None, :, :, None]
        S = lam[None, :, None, None] ** C * S + eta[None, :, None, None] * dS[:, :, c]
    return (y + y_intra).reshape(B, H, n * C, dv)[:, :, :T]
