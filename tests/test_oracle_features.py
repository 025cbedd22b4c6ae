"""Pins of the oracle's general feature maps and of the linear (no-erasure) rule: closed forms,
invariants and the equivalence checks the reference's own tests make
(tests/test_parallel_vs_recurrent.py:19-80 of the reference).  CPU only."""
import math

import numpy as np
import pytest

from oracle import lift as ol
from oracle import scan as osc


def _rng(seed):
    return np.random.default_rng(seed)


def test_rff_features_reduce_to_structured_lift():
    # With the seed-42 projection, its phases, tau* and renormalisation, rff_features is the pinned lift.
    proj = ol.make_projection(64, 512, 42)
    x = _rng(0).standard_normal((2, 1, 7, 64))
    phi = ol.rff_features(x, proj["omega"][None], proj["b"][None], proj["tau_star"], normalize=True, renorm=True)
    ref = ol.lift(x[:, 0], proj, normalize=True)
    np.testing.assert_allclose(phi[:, 0], ref, atol=1e-12)


def test_rff_features_zero_input_and_per_head_parameters():
    # x = 0 (normalisation keeps it 0): phi = sqrt(2/D) cos(b_h) for every head, whatever Omega and tau.
    rng = _rng(1)
    H, D, dk = 3, 16, 4
    om, b = rng.standard_normal((H, D, dk)), rng.uniform(0, 2 * np.pi, (H, D))
    tau = np.array([0.5, 1.0, 2.0])
    phi = ol.rff_features(np.zeros((1, H, 2, dk)), om, b, tau)
    np.testing.assert_allclose(phi[0, :, 0], math.sqrt(2.0 / D) * np.cos(b), atol=1e-15)
    # head h uses its own Omega, phase and tau: permuting the heads permutes the output
    x = rng.standard_normal((1, H, 3, dk))
    perm = [2, 0, 1]
    a = ol.rff_features(x[:, perm], om[perm], b[perm], tau[perm])
    np.testing.assert_allclose(a, ol.rff_features(x, om, b, tau)[:, perm], atol=1e-14)
    # tau scales the angle: tau_h = 2 equals tau = 1 with Omega / 2
    np.testing.assert_allclose(ol.rff_features(x, om, b, 2.0), ol.rff_features(x, om / 2, b, 1.0), atol=1e-14)


def test_rkhs_features_unit_norm_and_kernel_identity():
    rng = _rng(2)
    H, m, d = 2, 32, 8
    om = rng.standard_normal((H, m, d))
    lg = np.log(np.array([0.7, 3.0]))
    x, y = rng.standard_normal((1, H, 5, d)), rng.standard_normal((1, H, 5, d))
    px, py = ol.rkhs_features(x, om, lg), ol.rkhs_features(y, om, lg)
    assert px.shape == (1, H, 5, 2 * m)
    np.testing.assert_allclose(np.linalg.norm(px, axis=-1), 1.0, atol=1e-14)  # cos^2 + sin^2, / m
    # cos a cos b + sin a sin b = cos(a - b): the Gram is the mean cosine of the projected difference
    g = np.sqrt(2.0 * np.exp(lg))
    want = np.mean(np.cos(np.einsum("htd,hmd->htm", (x - y)[0], om) * g[:, None, None]), axis=-1)
    np.testing.assert_allclose(np.sum(px * py, axis=-1)[0], want, atol=1e-14)
    # gamma enters as sqrt(2 gamma) x: gamma * 4 at x equals gamma at 2x
    np.testing.assert_allclose(ol.rkhs_features(x, om, lg + np.log(4.0)), ol.rkhs_features(2 * x, om, lg),
                               atol=1e-13)


def test_rkhs_features_as_shifted_cosines():
    # [cos(a), sin(a)] / sqrt(m) = sqrt(2/D) cos([a; a] + [0; -pi/2]), D = 2m: the form the scan lifts.
    rng = _rng(3)
    H, m, d = 2, 16, 8
    om = rng.standard_normal((H, m, d))
    lg = np.log(np.array([1.5, 0.4]))
    x = rng.standard_normal((1, H, 4, d))
    om2 = np.concatenate([om, om], axis=1)
    ph = np.concatenate([np.zeros((H, m)), np.full((H, m), -np.pi / 2)], axis=1)
    tau = 1.0 / np.sqrt(2.0 * np.exp(lg))
    np.testing.assert_allclose(ol.rff_features(x, om2, ph, tau, normalize=False), ol.rkhs_features(x, om, lg),
                               atol=1e-14)


def test_linear_recurrence_explicit_sum():
    # y_t = sum_{j<t} beta_j (prod_{j<m<t} lambda_m) (q_t . k_j) v_j + (prod_{m<t} lambda_m) S0 q_t
    rng = _rng(4)
    B, T, D, dv = 2, 11, 5, 3
    pq, pk, v = rng.standard_normal((B, T, D)), rng.standard_normal((B, T, D)), rng.standard_normal((B, T, dv))
    beta, lam = rng.uniform(0.1, 2.0, (B, T)), rng.uniform(0.5, 1.0, (B, T))
    S0 = rng.standard_normal((B, dv, D))
    Y, S = osc.linear_recurrence(pq, pk, v, beta, lam, S0)
    for b in range(B):
        for t in range(T):
            want = np.prod(lam[b, :t]) * (S0[b] @ pq[b, t])
            for j in range(t):
                want = want + beta[b, j] * np.prod(lam[b, j + 1:t]) * (pq[b, t] @ pk[b, j]) * v[b, j]
            np.testing.assert_allclose(Y[b, t], want, atol=1e-12)
        Sf = np.prod(lam[b]) * S0[b]
        for j in range(T):
            Sf = Sf + beta[b, j] * np.prod(lam[b, j + 1:]) * np.outer(v[b, j], pk[b, j])
        np.testing.assert_allclose(S[b], Sf, atol=1e-12)


def test_linear_vs_delta_rule():
    rng = _rng(5)
    T, D, dv = 6, 8, 3
    Q, _ = np.linalg.qr(rng.standard_normal((D, D)))
    pk = Q[:T][None]  # mutually orthogonal keys: the erasure term S_{t-1} k_t is zero
    pq, v = rng.standard_normal((1, T, D)), rng.standard_normal((1, T, dv))
    beta, lam = rng.uniform(0.1, 0.9, (1, T)), rng.uniform(0.5, 1.0, (1, T))
    a = osc.linear_recurrence(pq, pk, v, beta, lam)
    d = osc.token_recurrence(pq, pk, v, beta, lam)
    np.testing.assert_allclose(a[0], d[0], atol=1e-12)
    np.testing.assert_allclose(a[1], d[1], atol=1e-12)
    # a repeated key is erased by the delta rule, not by the linear rule
    pk2 = np.concatenate([pk[:, :1], pk[:, :1]], axis=1)
    y_lin = osc.linear_recurrence(pk2, pk2, v[:, :2], np.ones((1, 2)), None)[1]
    y_del = osc.token_recurrence(pk2, pk2, v[:, :2], np.ones((1, 2)), None)[1]
    np.testing.assert_allclose(y_del[0] @ pk[0, 0], v[0, 1], atol=1e-12)
    np.testing.assert_allclose(y_lin[0] @ pk[0, 0], v[0, 0] + v[0, 1], atol=1e-12)


@pytest.mark.parametrize("T,C", [(64, 64), (100, 32), (37, 8), (5, 64)])
def test_linear_chunked_equals_recurrence(T, C):
    rng = _rng(6 + T)
    B, H, D, dv = 2, 3, 12, 4
    pq, pk = rng.standard_normal((B, H, T, D)), rng.standard_normal((B, H, T, D)) / 3
    v = rng.standard_normal((B, H, T, dv))
    lam, eta = rng.uniform(0.8, 1.0, H), rng.uniform(0.2, 1.5, H)
    y = osc.linear_chunked(pq, pk, v, lam, eta, C)
    for h in range(H):
        ref, _ = osc.linear_recurrence(pq[:, h], pk[:, h], v[:, h], np.full((B, T), eta[h]), np.full((B, T), lam[h]))
        np.testing.assert_allclose(y[:, h], ref, atol=1e-11)
