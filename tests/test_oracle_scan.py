"""Pins of the oracle scan (oracle/scan.py): brute force, closed forms, invariants, and the reference's
own carry-algebra check (tests/test_inter_woodbury.py:14-84 of the reference).  CPU only."""
import os

import numpy as np
import pytest
import torch

from oracle import lift as ol
from oracle import scan as osc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def proj():
    return ol.make_projection(64, 512, 42)


def _unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def test_token_recurrence_vs_dense_matrices():
    # S_t = lambda_t S_{t-1} (I - beta_t k k^T) + beta_t v k^T written with explicit D x D matrices.
    rng = np.random.default_rng(0)
    B, T, D, dv = 2, 9, 6, 3
    pq, pk = rng.standard_normal((B, T, D)), _unit(rng.standard_normal((B, T, D)))
    v = rng.standard_normal((B, T, dv))
    beta, lam = rng.uniform(0.1, 0.9, (B, T)), rng.uniform(0.5, 1.0, (B, T))
    S0 = rng.standard_normal((B, dv, D))
    Y, S = osc.token_recurrence(pq, pk, v, beta, lam, S0)
    for b in range(B):
        Sb = S0[b].copy()
        for t in range(T):
            np.testing.assert_allclose(Y[b, t], Sb @ pq[b, t], atol=1e-12)
            A = lam[b, t] * (np.eye(D) - beta[b, t] * np.outer(pk[b, t], pk[b, t]))
            Sb = Sb @ A + beta[b, t] * np.outer(v[b, t], pk[b, t])
        np.testing.assert_allclose(S[b], Sb, atol=1e-12)


def test_beta_zero_is_pure_decay():
    rng = np.random.default_rng(1)
    B, T, D, dv = 1, 12, 5, 4
    pq, pk, v = rng.standard_normal((B, T, D)), rng.standard_normal((B, T, D)), rng.standard_normal((B, T, dv))
    lam = rng.uniform(0.9, 1.0, (B, T))
    S0 = rng.standard_normal((B, dv, D))
    Y, S = osc.token_recurrence(pq, pk, v, np.zeros((B, T)), lam, S0)
    g = np.cumprod(lam[0])
    gshift = np.concatenate([[1.0], g[:-1]])
    np.testing.assert_allclose(Y[0], gshift[:, None] * (pq[0] @ S0[0].T), atol=1e-12)
    np.testing.assert_allclose(S[0], g[-1] * S0[0], atol=1e-12)


def test_orthonormal_keys_overwrite():
    # beta = 1, lambda = 1, orthonormal keys: S k_t = v_t for every written key.
    rng = np.random.default_rng(2)
    D, dv, T = 8, 3, 5
    Q, _ = np.linalg.qr(rng.standard_normal((D, D)))
    pk = Q[:T][None]
    v = rng.standard_normal((1, T, dv))
    S0 = rng.standard_normal((1, dv, D))
    _, S = osc.token_recurrence(np.zeros((1, T, D)), pk, v, np.ones((1, T)), None, S0)
    for t in range(T):
        np.testing.assert_allclose(S[0] @ pk[0, t], v[0, t], atol=1e-12)


def test_contractive_transition():
    rng = np.random.default_rng(3)
    D = 16
    for _ in range(50):
        k = _unit(rng.standard_normal(D))
        beta, lam = rng.uniform(0, 1), rng.uniform(0, 1)
        A = lam * (np.eye(D) - beta * np.outer(k, k))
        assert np.linalg.norm(A, 2) <= lam + 1e-12


@pytest.mark.parametrize("C", [16, 32, 64, 128])
@pytest.mark.parametrize("decay_kind", ["none", "sigmoid", "narrow"])
def test_chunked_matches_recurrence(proj, C, decay_kind):
    rng = np.random.default_rng(10 + C)
    B, T, dv = 2, 150, 32
    q, k, v = (rng.standard_normal((B, T, n)) for n in (64, 64, dv))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T))))
    decay = {"none": None, "sigmoid": 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T)))),
             "narrow": rng.uniform(0.94, 0.99, (B, T))}[decay_kind]
    S0 = rng.standard_normal((B, dv, 512)) * 0.1
    Yr, Sr = osc.delta_rule(q, k, v, beta, decay, proj, S0)
    Yc, Sc = osc.chunked_forward(q, k, v, beta, decay, proj, C, torch.tensor(S0))
    assert np.abs(Yc.numpy() - Yr).max() <= 1e-12 * max(1.0, np.abs(Yr).max())
    assert np.abs(Sc.numpy() - Sr).max() <= 1e-12 * max(1.0, np.abs(Sr).max())


def test_reference_carry_algebra():
    # Restates the reference check tests/test_inter_woodbury.py:14-84 (v = 0, non-zero S_start):
    # S_C = gamma_0C (S - S K^T W K),  W = (I + triu(diag(beta) K K^T, 1))^{-1} diag(beta);
    # Y_inter = gamma_inter * (Q S^T - (Q K^T o lower) (S K^T W)^T).  Checked against token_recurrence.
    rng = np.random.default_rng(42)
    T, d, C = 8, 4, 4
    q, k = _unit(rng.standard_normal((T, d))), _unit(rng.standard_normal((T, d)))
    beta = rng.uniform(0.1, 0.5, T)
    decay = rng.uniform(0.94, 0.99, T)
    S_start = rng.standard_normal((d, d))
    Yseq, Sseq = osc.token_recurrence(q[None, :C], k[None, :C], np.zeros((1, C, d)), beta[None, :C],
                                      decay[None, :C], S_start[None])
    K, Q, bc, dc = k[:C], q[:C], beta[:C], decay[:C]
    cum = np.cumsum(np.log(dc))
    g0C = np.exp(cum[-1])
    ginter = np.concatenate([[1.0], np.exp(cum[:-1])])
    G_kk, G_qk = K @ K.T, Q @ K.T
    U = np.triu(np.diag(bc) @ G_kk, 1)
    W = np.linalg.inv(np.eye(C) + U) @ np.diag(bc)
    S_chunk = g0C * (S_start - S_start @ K.T @ W @ K)
    corr = (G_qk * np.tril(np.ones((C, C)), -1)) @ (S_start @ K.T @ W).T
    Y_chunk = ginter[:, None] * (Q @ S_start.T - corr)
    assert np.abs(Sseq[0] - S_chunk).max() < 1e-12
    assert np.abs(Yseq[0] - Y_chunk).max() < 1e-12


def test_padding_is_noop(proj):
    rng = np.random.default_rng(5)
    B, T, dv = 1, 70, 16
    q, k, v = (rng.standard_normal((B, T, n)) for n in (64, 64, dv))
    beta = rng.uniform(0, 1, (B, T))
    Y1, S1 = osc.chunked_forward(q, k, v, beta, None, proj, 64)
    Y2, S2 = osc.chunked_forward(q, k, v, beta, None, proj, 35)
    np.testing.assert_allclose(Y1.numpy(), Y2.numpy(), atol=1e-12)
    np.testing.assert_allclose(S1.numpy(), S2.numpy(), atol=1e-12)


def test_scan_fixture(proj):
    g = np.load(os.path.join(GOLDEN, "scan_kat.npz"))
    Y, S = osc.delta_rule(g["q"], g["k"], g["v"], g["beta"], g["decay"], proj, g["S0"])
    np.testing.assert_allclose(Y, g["y"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(S, g["S"], rtol=0, atol=1e-12)
