"""Pins of the gradient oracle (oracle.scan.token_recurrence_torch / delta_rule_torch), CPU only.

The backward pass is checked on the GPU against torch autograd of these functions, so they are pinned
here: their forward equals the numpy definitions (token_recurrence / delta_rule), and
torch.autograd.gradcheck compares autograd with central finite differences for every input -- the
check the reference prescribes for its backward (tests/test_fused_chunk_kernel.py:54-72).  A dropped
term, a wrong sign or a transposed operand in the recurrence or the lift changes the forward (first
test) or the gradient (gradcheck) and fails one of them.
"""
import numpy as np
import torch

from oracle import lift as ol
from oracle import scan as osc


def _inputs(B, T, D, dv, seed):
    g = torch.Generator().manual_seed(seed)
    pq = torch.nn.functional.normalize(torch.randn(B, T, D, generator=g, dtype=torch.float64), dim=-1)
    pk = torch.nn.functional.normalize(torch.randn(B, T, D, generator=g, dtype=torch.float64), dim=-1)
    v = torch.randn(B, T, dv, generator=g, dtype=torch.float64)
    beta = torch.sigmoid(torch.randn(B, T, generator=g, dtype=torch.float64))
    lam = 0.8 + 0.19 * torch.rand(B, T, generator=g, dtype=torch.float64)
    s0 = 0.3 * torch.randn(B, dv, D, generator=g, dtype=torch.float64)
    return pq, pk, v, beta, lam, s0


def test_torch_recurrence_equals_numpy_definition():
    pq, pk, v, beta, lam, s0 = _inputs(2, 37, 16, 5, 0)
    Y, S = osc.token_recurrence_torch(pq, pk, v, beta, lam, s0)
    Yr, Sr = osc.token_recurrence(pq.numpy(), pk.numpy(), v.numpy(), beta.numpy(), lam.numpy(), s0.numpy())
    assert np.abs(Y.numpy() - Yr).max() < 1e-12
    assert np.abs(S.numpy() - Sr).max() < 1e-12


def test_gradcheck_recurrence():
    pq, pk, v, beta, lam, s0 = _inputs(1, 6, 8, 3, 1)
    args = tuple(t.clone().requires_grad_(True) for t in (pq, pk, v, beta, lam, s0))

    def f(*a):
        Y, S = osc.token_recurrence_torch(*a)
        return Y, S

    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-8, rtol=1e-6)


def test_gradcheck_lift_and_normalisation():
    proj = ol.make_projection(8, 16, 42)
    g = torch.Generator().manual_seed(2)
    for normalize in (False, True):
        x = torch.randn(3, 8, generator=g, dtype=torch.float64, requires_grad=True)
        assert torch.autograd.gradcheck(lambda t: osc._torch_lift(t, proj, normalize), (x,), eps=1e-6, atol=1e-8)


def test_delta_rule_torch_matches_numpy_and_gradcheck():
    proj = ol.make_projection(8, 16, 42)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 5, 8, generator=g, dtype=torch.float64)
    k = torch.randn(1, 5, 8, generator=g, dtype=torch.float64)
    v = torch.randn(1, 5, 2, generator=g, dtype=torch.float64)
    beta = torch.sigmoid(torch.randn(1, 5, generator=g, dtype=torch.float64))
    lam = 0.9 + 0.09 * torch.rand(1, 5, generator=g, dtype=torch.float64)
    Y, S = osc.delta_rule_torch(q, k, v, beta, lam, proj, normalize=True)
    Yr, Sr = osc.delta_rule(q.numpy(), k.numpy(), v.numpy(), beta.numpy(), lam.numpy(), proj, normalize=True)
    assert np.abs(Y.numpy() - Yr).max() < 1e-12 and np.abs(S.numpy() - Sr).max() < 1e-12
    args = tuple(t.clone().requires_grad_(True) for t in (q, k, v, beta, lam))
    assert torch.autograd.gradcheck(lambda *a: osc.delta_rule_torch(*a, proj, normalize=True), args, eps=1e-6,
                                    atol=1e-8, rtol=1e-6)


def test_lambda_clamp_blocks_the_gradient():
    # below 1e-5 the forward uses the clamped value, so d/d lambda is 0 there (as the kernel reports)
    pq, pk, v, beta, lam, s0 = _inputs(1, 4, 8, 3, 4)
    lam = lam.clone()
    lam[0, 2] = 1e-7
    lam.requires_grad_(True)
    Y, S = osc.token_recurrence_torch(pq, pk, v, beta, lam, s0)
    (Y.sum() + S.sum()).backward()
    assert float(lam.grad[0, 2]) == 0.0 and float(lam.grad[0, 1]) != 0.0


def test_torch_linear_rule_and_feature_map_equal_numpy_definitions():
    pq, pk, v, beta, lam, s0 = _inputs(2, 29, 16, 5, 3)
    Y, S = osc.linear_recurrence_torch(pq, pk, v, beta, lam, s0)
    Yr, Sr = osc.linear_recurrence(pq.numpy(), pk.numpy(), v.numpy(), beta.numpy(), lam.numpy(), s0.numpy())
    assert np.abs(Y.numpy() - Yr).max() < 1e-12 and np.abs(S.numpy() - Sr).max() < 1e-12
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 3, 7, 8, generator=g, dtype=torch.float64)
    om = torch.randn(3, 12, 8, generator=g, dtype=torch.float64)
    ph = 6.28 * torch.rand(3, 12, generator=g, dtype=torch.float64)
    tau = 0.5 + torch.rand(3, generator=g, dtype=torch.float64)
    for norm, renorm in ((True, False), (False, True)):
        got = osc.rff_features_torch(x, om, ph, 1.0 / tau, normalize=norm, renorm=renorm).numpy()
        ref = ol.rff_features(x.numpy(), om.numpy(), ph.numpy(), tau.numpy(), normalize=norm, renorm=renorm)
        assert np.abs(got - ref).max() < 1e-12
    # the P4 layer's [cos, sin] / sqrt(m) is the same map with Omega stacked twice and phases 0, -pi/2
    lg = torch.log(0.5 + torch.rand(3, generator=g, dtype=torch.float64))
    om6 = om[:, :6]
    shifted = osc.rff_features_torch(x, torch.cat([om6, om6], 1),
                                     torch.cat([torch.zeros(3, 6, dtype=torch.float64),
                                                torch.full((3, 6), -np.pi / 2, dtype=torch.float64)], 1),
                                     torch.sqrt(2 * torch.exp(lg)), normalize=False)
    assert np.abs(shifted.numpy() - ol.rkhs_features(x.numpy(), om6.numpy(), lg.numpy())).max() < 1e-12


def test_gradcheck_feature_map_and_linear_rule():
    # q, k through the per-head feature map (normalised inputs, no renormalisation), then the delta or the
    # linear rule; gradients w.r.t. q, k, v, beta, lambda, S_0 and the per-head 1/tau
    g = torch.Generator().manual_seed(5)
    B, H, T, dk, D, dv = 1, 2, 5, 4, 6, 3
    q = torch.randn(B, H, T, dk, generator=g, dtype=torch.float64)
    k = torch.randn(B, H, T, dk, generator=g, dtype=torch.float64)
    v = torch.randn(B * H, T, dv, generator=g, dtype=torch.float64)
    beta = torch.sigmoid(torch.randn(B * H, T, generator=g, dtype=torch.float64))
    lam = 0.8 + 0.19 * torch.rand(B * H, T, generator=g, dtype=torch.float64)
    s0 = 0.3 * torch.randn(B * H, dv, D, generator=g, dtype=torch.float64)
    itau = 0.5 + torch.rand(H, generator=g, dtype=torch.float64)
    om = torch.randn(H, D, dk, generator=g, dtype=torch.float64)
    ph = 6.28 * torch.rand(H, D, generator=g, dtype=torch.float64)
    for rec in (osc.token_recurrence_torch, osc.linear_recurrence_torch):
        def f(q_, k_, v_, b_, l_, s_, it_):
            pq = osc.rff_features_torch(q_, om, ph, it_, normalize=True).reshape(B * H, T, D)
            pk = osc.rff_features_torch(k_, om, ph, it_, normalize=True).reshape(B * H, T, D)
            return rec(pq, pk, v_, b_, l_, s_)
        args = tuple(t.clone().requires_grad_(True) for t in (q, k, v, beta, lam, s0, itau))
        assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-8, rtol=1e-6)
