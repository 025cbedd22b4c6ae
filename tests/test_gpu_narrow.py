"""GPU parity of the D = 128 and 256 lifts: kdn_delta_scan_fwd and kdn_delta_scan_bwd run them on the
D = 512 kernels with Omega and the phases replicated 512 / D times (the products are those of the D-wide
scan; the 512-wide state folds back to D columns), and the reference-default surfaces that need them:
FusedKernelDeltaNet(d_kernel=256) (reference kernels/fused_kernel_deltanet.py:182-209, kernels/fwht.py:54-59)
and KernelDeltaNetLayer with its default rkhs_factor = 4 (layers/kernel_deltanet_layer.py:26-42).

Oracles (float64, CPU): oracle.lift.lift + token_recurrence for the structured-FWHT lift and the delta rule;
rkhs_features + linear_recurrence for the layer; torch autograd of oracle.scan.delta_rule_torch /
rff_features_torch + linear_recurrence_torch for the gradients.  Tolerances (relative L2) as every scan
test: 1e-4 for fp32 inputs, 2e-2 for bf16 inputs.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kdn import ops
from kernels import FastWalshHadamardProjection, FusedKernelDeltaNet
from layers import KernelDeltaNetLayer
from oracle import lift as ol
from oracle import scan as osc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def rel(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, dtype=np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def inputs(B, T, H, D, dv, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g).to(dtype)
    k = torch.randn(B, T, H, 64, generator=g).to(dtype)
    v = torch.randn(B, T, H, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    lam = 0.9 + 0.1 * torch.rand(B, T, H, generator=g)
    s0 = 0.1 * torch.randn(B, H, D, dv, generator=g)
    dy = torch.randn(B, T, H, dv, generator=g)
    ds = 0.5 * torch.randn(B, H, D, dv, generator=g)
    return q, k, v, beta, lam, s0, dy, ds


def oracle_forward(q, k, v, beta, lam, s0, oproj):
    """Y (B, T, H, d_v) and S (B, H, D, d_v) from the float64 lift and token recurrence."""
    B, T, H, _ = q.shape
    Y = np.zeros((B, T, H, v.shape[-1]))
    S = np.zeros(s0.shape)
    for h in range(H):
        pq = np.stack([ol.lift(q[b, :, h].float().numpy(), oproj) for b in range(B)])
        pk = np.stack([ol.lift(k[b, :, h].float().numpy(), oproj) for b in range(B)])
        y, s = osc.token_recurrence(pq, pk, v[:, :, h].double().numpy(), beta[:, :, h].double().numpy(),
                                    lam[:, :, h].double().numpy(), s0[:, h].double().numpy().transpose(0, 2, 1))
        Y[:, :, h], S[:, h] = y, s.transpose(0, 2, 1)
    return Y, S


@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_forward_matches_oracle(D, dtype):
    proj, oproj = FastWalshHadamardProjection(64, D, 42), ol.make_projection(64, D, 42)
    q, k, v, beta, lam, s0, _, _ = inputs(2, 200, 3, D, 64, dtype, seed=D + (dtype == torch.bfloat16))
    d = lambda t: t.to(DEV)
    y, S = ops.scan(d(q), d(k), d(v), d(beta), d(lam), proj.device_omega(DEV), proj.device_phase(DEV),
                    proj.tau_star_inv, initial_state=d(s0))
    torch.cuda.synchronize()
    assert tuple(S.shape) == (2, 3, D, 64)
    Yr, Sr = oracle_forward(q, k, v, beta, lam, s0, oproj)
    assert rel(y.float(), Yr) < TOL[dtype]
    assert rel(S, Sr) < TOL[dtype]


@pytest.mark.parametrize("D", [128, 256])
def test_scan_pipelined_equals_serial_and_in_place_state(D):
    proj = FastWalshHadamardProjection(64, D, 7)
    q, k, v, beta, lam, s0, _, _ = inputs(1, 64 * 20 + 5, 2, D, 32, torch.bfloat16, seed=3)
    d = lambda t: t.to(DEV)
    outs = []
    for pipelined in (False, True):
        outs.append(ops.scan(d(q), d(k), d(v), d(beta), d(lam), proj.device_omega(DEV), proj.device_phase(DEV),
                             proj.tau_star_inv, initial_state=d(s0), segment_chunks=4, pipelined=pipelined))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    # final_state aliasing initial_state (the continuing-prefill pattern)
    st = d(s0).clone()
    y, _ = ops.scan(d(q), d(k), d(v), d(beta), d(lam), proj.device_omega(DEV), proj.device_phase(DEV),
                    proj.tau_star_inv, initial_state=st, final_state=st, segment_chunks=4)
    torch.cuda.synchronize()
    assert torch.equal(y, outs[0][0]) and torch.equal(st, outs[0][1])


def oracle_grads(q, k, v, beta, lam, s0, dy, ds, oproj):
    B, T, H, _ = q.shape
    D, dv = s0.shape[-2], s0.shape[-1]

    def fold(x):
        x = x.double()
        if x.dim() == 4:
            return x.permute(0, 2, 1, 3).reshape(B * H, T, -1).clone()
        return x.permute(0, 2, 1).reshape(B * H, T).clone()

    def unfold(x):
        if x.dim() == 3:
            return x.reshape(B, H, T, -1).permute(0, 2, 1, 3)
        return x.reshape(B, H, T).permute(0, 2, 1)

    qf, kf, vf, bf, lf = (fold(t).requires_grad_(True) for t in (q.float(), k.float(), v.float(), beta, lam))
    sf = s0.double().reshape(B * H, D, dv).transpose(1, 2).clone().requires_grad_(True)
    Y, S = osc.delta_rule_torch(qf, kf, vf, bf, lf, oproj, sf, False)
    L = (Y * fold(dy)).sum() + (S * ds.double().reshape(B * H, D, dv).transpose(1, 2)).sum()
    L.backward()
    return {"dq": unfold(qf.grad), "dk": unfold(kf.grad), "dv": unfold(vf.grad), "dbeta": unfold(bf.grad),
            "ddecay": unfold(lf.grad), "dinit": sf.grad.transpose(1, 2).reshape(B, H, D, dv)}


@pytest.mark.parametrize("D,dv", [(256, 64), (128, 64), (256, 32)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_backward_matches_float64_autograd(D, dv, dtype):
    proj, oproj = FastWalshHadamardProjection(64, D, 42), ol.make_projection(64, D, 42)
    q, k, v, beta, lam, s0, dy, ds = inputs(1, 200, 2, D, dv, dtype, seed=D + dv)
    d = lambda t: t.to(DEV)
    dq, dk, dvv, db, dd, di = ops.scan_backward(d(q), d(k), d(v), d(beta), d(lam), proj.device_omega(DEV),
                                                proj.device_phase(DEV), proj.tau_star_inv, d(dy), d(ds),
                                                initial_state=d(s0))
    torch.cuda.synchronize()
    got = {"dq": dq, "dk": dk, "dv": dvv, "dbeta": db, "ddecay": dd, "dinit": di}
    ref = oracle_grads(q, k, v, beta, lam, s0, dy, ds, oproj)
    errs = {n: rel(got[n], ref[n]) for n in ref}
    assert all(e < TOL[dtype] for e in errs.values()), errs


def test_fused_module_d_kernel_256():
    """FusedKernelDeltaNet(d_kernel=256): forward against the float64 lift + token recurrence, and every
    input's gradient against float64 autograd."""
    m = FusedKernelDeltaNet(d_model=64, d_kernel=256).to(DEV)
    oproj = ol.make_projection(64, 256, 42)
    g = torch.Generator().manual_seed(8)
    B, T = 2, 150
    q, k, v = torch.randn(B, T, 64, generator=g), torch.randn(B, T, 64, generator=g), torch.randn(B, T, 64, generator=g)
    beta, decay = torch.sigmoid(torch.randn(B, T, generator=g)), torch.sigmoid(torch.randn(B, T, generator=g) + 2)
    dy = torch.randn(B, T, 64, generator=g)
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v, beta, decay)]
    y, S = m(*leaves)
    (y * dy.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    pq = np.stack([ol.lift(q[b].numpy(), oproj) for b in range(B)])
    pk = np.stack([ol.lift(k[b].numpy(), oproj) for b in range(B)])
    Yr, Sr = osc.token_recurrence(pq, pk, v.double().numpy(), beta.double().numpy(), decay.double().numpy())
    assert rel(y, Yr) < TOL[torch.float32]
    assert tuple(S.shape) == (B, 64, 256) and rel(S, Sr) < TOL[torch.float32]
    ref = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, decay)]
    yo, _ = osc.delta_rule_torch(ref[0], ref[1], ref[2], ref[3], ref[4], oproj)
    (yo * dy.double()).sum().backward()
    errs = [rel(a.grad, r.grad) for a, r in zip(leaves, ref)]
    assert max(errs) < TOL[torch.float32], errs


def np64(t):
    return t.detach().to("cpu", torch.float64).numpy()


def layer_reference(layer, x, state=None):
    """The layer's forward in float64 from the projections the module computed, through
    oracle.lift.rkhs_features and linear_recurrence (as the D = 512 layer test)."""
    B, T, _ = x.shape
    H, dh = layer.num_heads, layer.d_head
    W = {n: p.detach().cpu().double() for n, p in layer.named_parameters()}

    def heads(lin, norm):
        with torch.no_grad():
            h = lin(x).detach().cpu().double().view(B, T, H, dh).transpose(1, 2)
        return (F.normalize(h, dim=-1) if norm else h).numpy()

    om, lg = np64(layer.kernel.omega), W["kernel.log_gamma"].numpy()
    pq = ol.rkhs_features(heads(layer.w_q, True), om, lg)
    pk = ol.rkhs_features(heads(layer.w_k, True), om, lg)
    lam = np64(layer.get_decay()).reshape(H)
    eta = np64(layer.get_eta()).reshape(H)
    Y = np.zeros((B, H, T, dh))
    S = np.zeros((B, H, dh, layer.rkhs_dim))
    for h in range(H):
        s0 = None if state is None else np64(state)[:, h]
        Y[:, h], S[:, h] = osc.linear_recurrence(pq[:, h], pk[:, h], heads(layer.w_v, False)[:, h],
                                                 np.full((B, T), eta[h]), np.full((B, T), lam[h]), s0)
    out = torch.from_numpy(Y).transpose(1, 2).reshape(B, T, H * dh) @ W["w_out.weight"].T
    return out.numpy(), S


def test_layer_default_rkhs_factor():
    """KernelDeltaNetLayer(d_model=256, num_heads=4) with the reference's default rkhs_factor = 4 (rkhs_dim
    256): prefill and step modes against the oracle, and prefill == steps."""
    torch.manual_seed(12)
    layer = KernelDeltaNetLayer(256, 4).to(DEV)
    assert layer.rkhs_dim == 256
    x = torch.randn(2, 150, 256, device=DEV)
    with torch.no_grad():
        out, none_state = layer(x)
    assert none_state is None
    ref_out, ref_S = layer_reference(layer, x)
    assert rel(out, ref_out) < TOL[torch.float32]
    with torch.no_grad():
        zero = torch.zeros(2, 4, 64, 256, device=DEV)
        o_a, s_a = layer(x[:, :70], zero)
        o_b, s_b = layer(x[:, 70:], s_a)
    assert rel(torch.cat([o_a, o_b], 1), out) < 1e-5
    assert rel(s_b, ref_S) < TOL[torch.float32]


def test_layer_rkhs_factor_2_parameter_gradients():
    """rkhs_factor = 2 (rkhs_dim 128) with a given state: gradients of every parameter against float64
    autograd of the module's forward through rff_features_torch + linear_recurrence_torch."""
    torch.manual_seed(13)
    layer = KernelDeltaNetLayer(128, 2, rkhs_factor=2).to(DEV)
    B, T, H, dh, D = 2, 90, 2, 64, 128
    x = torch.randn(B, T, 128, device=DEV)
    s0 = 0.1 * torch.randn(B, H, dh, D, device=DEV)
    go = torch.randn(B, T, 128, device=DEV)
    gs = 0.3 * torch.randn(B, H, dh, D, device=DEV)
    layer.zero_grad()
    out, S = layer(x, s0)
    ((out * go).sum() + (S * gs).sum()).backward()
    torch.cuda.synchronize()
    got = {n: p.grad.detach().cpu().double() for n, p in layer.named_parameters()}
    W = {n: p.detach().cpu().double().requires_grad_(True) for n, p in layer.named_parameters()}
    xd = x.cpu().double()
    heads = lambda w: (xd @ W[w].T).view(B, T, H, dh).transpose(1, 2)
    m = D // 2
    om = layer.kernel.omega.cpu().double()
    om2 = torch.cat([om, om], dim=1)
    ph = torch.cat([torch.zeros(m, dtype=torch.float64), torch.full((m,), -math.pi / 2, dtype=torch.float64)])
    itau = torch.sqrt(2.0 * torch.exp(W["kernel.log_gamma"]))
    pq = osc.rff_features_torch(heads("w_q.weight"), om2, ph.expand(H, D), itau, normalize=True).reshape(B * H, T, D)
    pk = osc.rff_features_torch(heads("w_k.weight"), om2, ph.expand(H, D), itau, normalize=True).reshape(B * H, T, D)
    lam = torch.sigmoid(W["logit_decay"]).reshape(H)
    eta = F.softplus(W["raw_eta"]).reshape(H)
    beta = eta.view(1, H, 1).expand(B, H, T).reshape(B * H, T)
    decay = lam.view(1, H, 1).expand(B, H, T).reshape(B * H, T)
    Y, Sr = osc.linear_recurrence_torch(pq, pk, heads("w_v.weight").reshape(B * H, T, dh), beta, decay,
                                        s0.cpu().double().reshape(B * H, dh, D))
    o = Y.reshape(B, H, T, dh).transpose(1, 2).reshape(B, T, H * dh) @ W["w_out.weight"].T
    ((o * go.cpu().double()).sum() + (Sr.reshape(B, H, dh, D) * gs.cpu().double()).sum()).backward()
    errs = {n: rel(got[n], W[n].grad) for n in W}
    assert all(e < TOL[torch.float32] for e in errs.values()), errs
