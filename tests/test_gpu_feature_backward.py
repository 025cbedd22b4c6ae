"""GPU parity of the backward pass with the per-head feature maps and the linear rule (kdn_delta_scan_bwd,
ABI 1.7), and of the training surfaces built on it: FusedKernelDeltaNetFunction / FusedKernelDeltaNet
(reference kernels/kernel_deltanet_fused.py:36-303) and KernelDeltaNetLayer (layers/kernel_deltanet_layer.py:
20-143).

Oracle: torch autograd in float64 on the CPU of oracle.scan.rff_features_torch (per-head Omega, phases
and 1/tau; pinned against oracle.lift.rff_features / rkhs_features and by gradcheck in
test_oracle_backward.py) followed by token_recurrence_torch (delta rule) or linear_recurrence_torch (the
layer's rule), on the same inputs (bf16 inputs rounded first), for L = sum(y * dy) + sum(S_T * dS).  For
the modules, the same float64 re-implementation of their forward from their own weights, gradients of
every parameter.  Tolerances (relative L2): 1e-4 for fp32, 2e-2 for bf16 inputs, as for the forward.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kdn import ops
from kernels.kernel_deltanet_fused import FusedKernelDeltaNet, FusedKernelDeltaNetFunction, split_bf16
from layers import KernelDeltaNetLayer
from oracle import scan as osc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def rel(a, b):
    a = a.detach().to("cpu", torch.float64).numpy()
    b = b.detach().to("cpu", torch.float64).numpy()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _inputs(B, T, H, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g).to(dtype)
    k = torch.randn(B, T, H, 64, generator=g).to(dtype)
    v = torch.randn(B, T, H, 64, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    lam = 0.9 + 0.1 * torch.rand(B, T, H, generator=g)
    s0 = 0.1 * torch.randn(B, H, 512, 64, generator=g)
    dy = torch.randn(B, T, H, 64, generator=g)
    ds = 0.5 * torch.randn(B, H, 512, 64, generator=g)
    omega = torch.randn(H, 512, 64, generator=g)            # fp32: not exact in bf16, so hi + lo parts
    phase = 2 * math.pi * torch.rand(H, 512, generator=g)
    itau = 0.3 + 0.4 * torch.rand(H, generator=g)
    return q, k, v, beta, lam, s0, dy, ds, omega, phase, itau


def _oracle(rule, q, k, v, beta, lam, s0, dy, ds, omega, phase, itau):
    """Float64 autograd of the features + recurrence; gradients in the kernel layouts."""
    B, T, H, _ = q.shape
    rec = osc.token_recurrence_torch if rule == ops.RULE_DELTA else osc.linear_recurrence_torch
    leaves = [t.double().clone().requires_grad_(True) for t in (q.float(), k.float(), v.float(), beta, lam, s0, itau)]
    qd, kd, vd, bd, ld, sd, itd = leaves
    om, ph = omega.double(), phase.double()
    pq = osc.rff_features_torch(qd.transpose(1, 2), om, ph, itd, normalize=True).reshape(B * H, T, 512)
    pk = osc.rff_features_torch(kd.transpose(1, 2), om, ph, itd, normalize=True).reshape(B * H, T, 512)
    fold = lambda x: x.transpose(1, 2).reshape(B * H, T, *x.shape[3:])
    Y, S = rec(pq, pk, fold(vd), fold(bd), fold(ld), sd.reshape(B * H, 512, 64).transpose(1, 2))
    L = (Y * fold(dy.double())).sum() + (S * ds.double().reshape(B * H, 512, 64).transpose(1, 2)).sum()
    L.backward()
    return [t.grad for t in leaves]


@pytest.mark.parametrize("rule", [ops.RULE_DELTA, ops.RULE_LINEAR])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_feature_map_backward_parity(rule, dtype):
    # per-head Omega (hi + lo), phases and 1/tau, no renormalisation, normalised inputs; T = 200: three full
    # chunks and a partial one; decay, initial state and dL/dS_T present
    q, k, v, beta, lam, s0, dy, ds, omega, phase, itau = _inputs(2, 200, 2, dtype, seed=21 + rule)
    hi, lo = split_bf16(omega)
    fm = ops.FeatureMap(omega=hi.to(DEV), phase=phase.to(DEV), omega_lo=lo.to(DEV), inv_tau_head=itau.to(DEV),
                        no_renorm=True)
    plan = ops.ScanBackwardPlan(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), None, None, 1.0,
                                dy.to(DEV), ds.to(DEV), normalize=True, initial_state=s0.to(DEV), features=fm,
                                rule=rule, need_dinv_tau=True)
    got = list(plan.run()) + [plan.dinv_tau]
    torch.cuda.synchronize()
    ref = _oracle(rule, q, k, v, beta, lam, s0, dy, ds, omega, phase, itau)
    names = ("dq", "dk", "dv", "dbeta", "ddecay", "dinit", "dinv_tau")
    errs = {n: rel(g, r) for n, g, r in zip(names, got, ref)}
    assert all(e < TOL[dtype] for e in errs.values()), errs
    # the schedules agree bit for bit
    again = ops.ScanBackwardPlan(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), None, None, 1.0,
                                 dy.to(DEV), ds.to(DEV), normalize=True, initial_state=s0.to(DEV), features=fm,
                                 rule=rule, need_dinv_tau=True)
    serial = list(again.run(concurrent_carries=False)) + [again.dinv_tau]
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(got, serial))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_p2_function_gradients(dtype):
    g = torch.Generator().manual_seed(31)
    B, H, T = 2, 2, 150
    m = FusedKernelDeltaNet(64 * H, H)  # the module's own ORF Omega and phases
    q = torch.randn(B, H, T, 64, generator=g).to(dtype)
    k = torch.randn(B, H, T, 64, generator=g).to(dtype)
    v = torch.randn(B, H, T, 64, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=g))
    decay = torch.sigmoid(torch.randn(B, H, T, generator=g) + 3.0)
    tau = F.softplus(torch.randn(H, 1, generator=g)) + 0.5
    gy = torch.randn(B, H, T, 64, generator=g)
    gs = 0.3 * torch.randn(B, H, 64, 512, generator=g)
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v, tau, beta, decay)]
    qd, kd, vd, td, bd, dd = leaves
    Y, S = FusedKernelDeltaNetFunction.apply(qd, kd, vd, m.omega.to(DEV), m.b_rff.to(DEV), td, bd, dd, 64)
    ((Y.float() * gy.to(DEV)).sum() + (S.float() * gs.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    # oracle
    ref = [t.float().double().clone().requires_grad_(True) for t in (q, k, v, tau, beta, decay)]
    rq, rk, rv, rt, rb, rd = ref
    om, ph = m.omega.double(), m.b_rff.double()
    pq = osc.rff_features_torch(rq, om, ph, 1.0 / rt.reshape(-1), normalize=True).reshape(B * H, T, 512)
    pk = osc.rff_features_torch(rk, om, ph, 1.0 / rt.reshape(-1), normalize=True).reshape(B * H, T, 512)
    Yr, Sr = osc.token_recurrence_torch(pq, pk, rv.reshape(B * H, T, 64), rb.reshape(B * H, T), rd.reshape(B * H, T))
    ((Yr * gy.double().reshape(B * H, T, 64)).sum() + (Sr * gs.double().reshape(B * H, 64, 512)).sum()).backward()
    errs = {n: rel(a.grad, b.grad) for n, a, b in zip(("q", "k", "v", "tau", "beta", "decay"), leaves, ref)}
    assert all(e < TOL[dtype] for e in errs.values()), errs


def _module_grads(module, x, loss_fn):
    module.zero_grad()
    loss_fn(*module(x)).backward()
    torch.cuda.synchronize()
    return {n: p.grad.detach().cpu().double() for n, p in module.named_parameters()}


def test_p2_module_parameter_gradients():
    torch.manual_seed(41)
    m = FusedKernelDeltaNet(128, 2).to(DEV)
    x = torch.randn(2, 130, 128, device=DEV) * 0.5
    go = torch.randn(2, 130, 128, device=DEV)
    gs = 0.3 * torch.randn(2, 2, 64, 512, device=DEV)
    got = _module_grads(m, x, lambda out, S: (out * go).sum() + (S * gs).sum())
    # float64 re-implementation of the module's forward from its own weights
    W = {n: p.detach().cpu().double().requires_grad_(True) for n, p in m.named_parameters()}
    xd = x.cpu().double()
    B, T, _ = xd.shape
    H, dh = 2, 64
    heads = lambda w: (xd @ W[w].T).view(B, T, H, dh).transpose(1, 2)
    beta = torch.sigmoid(xd @ W["w_beta.weight"].T).transpose(1, 2).reshape(B * H, T)
    decay = torch.sigmoid(xd @ W["w_decay.weight"].T).transpose(1, 2).reshape(B * H, T)
    itau = 1.0 / (F.softplus(W["raw_tau"]) + 1e-4).reshape(-1)
    om, ph = m.omega.cpu().double(), m.b_rff.cpu().double()
    pq = osc.rff_features_torch(heads("w_q.weight"), om, ph, itau, normalize=True).reshape(B * H, T, 512)
    pk = osc.rff_features_torch(heads("w_k.weight"), om, ph, itau, normalize=True).reshape(B * H, T, 512)
    Y, S = osc.token_recurrence_torch(pq, pk, heads("w_v.weight").reshape(B * H, T, dh), beta, decay)
    out = Y.reshape(B, H, T, dh).transpose(1, 2).reshape(B, T, H * dh) @ W["w_out.weight"].T
    ((out * go.cpu().double()).sum() + (S.reshape(B, H, dh, 512) * gs.cpu().double()).sum()).backward()
    errs = {n: rel(got[n], W[n].grad) for n in W}
    assert all(e < TOL[torch.float32] for e in errs.values()), errs


@pytest.mark.parametrize("with_state", [False, True])
def test_layer_parameter_gradients(with_state):
    torch.manual_seed(51)
    layer = KernelDeltaNetLayer(128, 2, rkhs_factor=8).to(DEV)
    B, T, H, dh, D = 2, 140 if not with_state else 70, 2, 64, 512
    x = torch.randn(B, T, 128, device=DEV)
    s0 = 0.1 * torch.randn(B, H, dh, D, device=DEV) if with_state else None
    go = torch.randn(B, T, 128, device=DEV)
    gs = 0.3 * torch.randn(B, H, dh, D, device=DEV)

    def loss(out, S):
        return (out * go).sum() + ((S * gs).sum() if S is not None else 0.0)

    layer.zero_grad()
    loss(*layer(x, s0)).backward()
    torch.cuda.synchronize()
    got = {n: p.grad.detach().cpu().double() for n, p in layer.named_parameters()}
    W = {n: p.detach().cpu().double().requires_grad_(True) for n, p in layer.named_parameters()}
    xd = x.cpu().double()
    heads = lambda w: (xd @ W[w].T).view(B, T, H, dh).transpose(1, 2)
    m = D // 2
    om = layer.kernel.omega.cpu().double()
    om2 = torch.cat([om, om], dim=1)
    ph = torch.cat([torch.zeros(m, dtype=torch.float64), torch.full((m,), -math.pi / 2, dtype=torch.float64)])
    ph = ph.expand(H, D)
    itau = torch.sqrt(2.0 * torch.exp(W["kernel.log_gamma"]))
    pq = osc.rff_features_torch(heads("w_q.weight"), om2, ph, itau, normalize=True).reshape(B * H, T, D)
    pk = osc.rff_features_torch(heads("w_k.weight"), om2, ph, itau, normalize=True).reshape(B * H, T, D)
    lam = torch.sigmoid(W["logit_decay"]).reshape(H)
    eta = F.softplus(W["raw_eta"]).reshape(H)
    beta = eta.view(1, H, 1).expand(B, H, T).reshape(B * H, T)
    decay = lam.view(1, H, 1).expand(B, H, T).reshape(B * H, T)
    S0 = None if s0 is None else s0.cpu().double().reshape(B * H, dh, D)
    Y, S = osc.linear_recurrence_torch(pq, pk, heads("w_v.weight").reshape(B * H, T, dh), beta, decay, S0)
    out = Y.reshape(B, H, T, dh).transpose(1, 2).reshape(B, T, H * dh) @ W["w_out.weight"].T
    L = (out * go.cpu().double()).sum()
    if with_state:
        L = L + (S.reshape(B, H, dh, D) * gs.cpu().double()).sum()
    L.backward()
    errs = {n: rel(got[n], W[n].grad) for n in W}
    assert all(e < TOL[torch.float32] for e in errs.values()), errs
