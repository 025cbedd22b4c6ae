"""GPU parity of the factored d_k = 128 path: kdn_fwht_lift_factored and the D = 1024 scan.

Oracles: oracle.lift.factored_lift (float64; pinned in test_oracle_factored.py) for the lift, and the
float64 token recurrence (oracle.scan.token_recurrence) over the oracle's factored features for the scan
-- the reference's own acceptance check (tests/test_factored_kernel.py:25-60, 82-118: chunked scan vs
the unrolled recurrence, B = 2, T = 256, d_k = 128, d_v = 128, decay in [0.9, 1]).  Tolerances (relative
L2): lift 1e-5 (fp32) / 1e-2 (bf16 outputs); scan 1e-4 for fp32 inputs, 2e-2 for bf16 inputs.  Unit
norms to 1e-5 as the reference checks them (tests/test_factored_kernel.py:65-78).
"""
import numpy as np
import pytest
import torch

from kdn import ops
from kernels import FactoredFastWalshHadamardProjection, FactoredKernelDeltaNet, factored_chunked_deltanet_forward
from oracle import lift as ol
from oracle import scan as osc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def fproj():
    return FactoredFastWalshHadamardProjection(128, 1024, 42)


@pytest.fixture(scope="module")
def oprojs():
    return ol.make_projection(64, 512, 42), ol.make_projection(64, 512, 1042)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_factored_lift(fproj, oprojs, dtype, tol):
    x = torch.randn(4, 32, 128, generator=torch.Generator().manual_seed(0)).to(dtype)
    phi = fproj(x.to(DEV))
    torch.cuda.synchronize()
    assert phi.shape == (4, 32, 1024) and phi.dtype == dtype
    ref = ol.factored_lift(x.float().numpy(), *oprojs)
    assert rel(phi.float().cpu().numpy(), ref) < tol
    norms = torch.linalg.vector_norm(phi.float(), dim=-1).cpu()
    assert torch.allclose(norms, torch.ones_like(norms), atol=1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("rows", [1, 37, 70001])
def test_factored_lift_one_pass_bf16_inputs(fproj, oprojs, rows):
    """bf16 inputs take the one-pass kernel (both halves and the renormalisation per workgroup, persistent
    over 4-tile groups): fp32 outputs against the oracle at the fp32 tolerance (x is exact in bf16 and
    nothing is rounded to bf16 on the way), bf16 outputs equal to those rounded within one bf16 step, at
    row counts that leave partial tiles, idle waves in the last group and several groups per workgroup."""
    x = torch.randn(rows, 128, generator=torch.Generator().manual_seed(rows)).to(torch.bfloat16)
    p1, p2 = fproj.proj1, fproj.proj2
    args = (p1.device_omega(DEV), p1.device_phase(DEV), p2.device_omega(DEV), p2.device_phase(DEV), p1.tau_star_inv)
    xd = x.to(DEV)
    y32 = ops.lift_factored(xd, *args, out_dtype=torch.float32)
    y16 = ops.lift_factored(xd, *args)
    torch.cuda.synchronize()
    assert y32.dtype == torch.float32 and y16.dtype == torch.bfloat16 and y32.shape == (rows, 1024)
    idx = np.unique(np.linspace(0, rows - 1, min(rows, 512)).astype(np.int64))
    ref = ol.factored_lift(x.float().numpy()[idx], *oprojs)
    assert rel(y32.cpu().numpy()[idx], ref) < 1e-5
    norms = torch.linalg.vector_norm(y32, dim=-1).cpu()
    assert torch.allclose(norms, torch.ones_like(norms), atol=1e-5)
    # the bf16 path rounds each half and then the renormalised value: within 2^-7 relative of fp32
    assert torch.allclose(y16.float(), y32, rtol=2 ** -7, atol=1e-6)


def oracle_scan(q, k, v, beta, decay, oprojs, s0=None):
    pq = ol.factored_lift(q.float().numpy(), *oprojs)
    pk = ol.factored_lift(k.float().numpy(), *oprojs)
    return osc.token_recurrence(pq, pk, v.double().numpy(), beta.double().numpy(),
                                None if decay is None else decay.double().numpy(),
                                None if s0 is None else s0.double().numpy())


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_factored_scan_matches_the_recurrence(fproj, oprojs, dtype, tol):
    g = torch.Generator().manual_seed(42)
    B, T, dv = 2, 256, 128
    q = torch.randn(B, T, 128, generator=g).to(dtype)
    k = torch.randn(B, T, 128, generator=g).to(dtype)
    v = torch.randn(B, T, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    decay = torch.sigmoid(torch.randn(B, T, generator=g)) * 0.1 + 0.9
    Y, S = factored_chunked_deltanet_forward(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), decay.to(DEV), fproj)
    torch.cuda.synchronize()
    Yr, Sr = oracle_scan(q, k, v, beta, decay, oprojs)
    assert Y.shape == (B, T, dv) and S.shape == (B, dv, 1024)
    assert rel(Y.float().cpu().numpy(), Yr) < tol
    assert rel(S.float().cpu().numpy(), Sr) < tol


def test_factored_scan_partial_chunk_initial_state_dv64(fproj, oprojs):
    g = torch.Generator().manual_seed(7)
    B, T, dv = 1, 200, 64
    q, k = torch.randn(B, T, 128, generator=g), torch.randn(B, T, 128, generator=g)
    v = torch.randn(B, T, dv, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    s0 = 0.1 * torch.randn(B, dv, 1024, generator=g)
    model = FactoredKernelDeltaNet(d_k=128, d_v=dv, D=1024)
    Y, S = model(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), None, s0.to(DEV))
    torch.cuda.synchronize()
    Yr, Sr = oracle_scan(q, k, v, beta, None, oprojs, s0)
    assert rel(Y.cpu().numpy(), Yr) < 1e-4
    assert rel(S.cpu().numpy(), Sr) < 1e-4


def test_factored_scan_continues_across_calls(fproj):
    # two calls chained through the state equal one call over the concatenation
    g = torch.Generator().manual_seed(8)
    T1, T2 = 130, 70
    q, k = torch.randn(1, T1 + T2, 128, generator=g), torch.randn(1, T1 + T2, 128, generator=g)
    v = torch.randn(1, T1 + T2, 128, generator=g)
    beta = torch.sigmoid(torch.randn(1, T1 + T2, generator=g))
    dec = 0.95 + 0.05 * torch.rand(1, T1 + T2, generator=g)
    a = [t.to(DEV) for t in (q, k, v, beta, dec)]
    Y1, S1 = factored_chunked_deltanet_forward(*(t[:, :T1] for t in a), fproj)
    Y2, S2 = factored_chunked_deltanet_forward(*(t[:, T1:] for t in a), fproj, initial_state=S1)
    Y, S = factored_chunked_deltanet_forward(*a, fproj)
    torch.cuda.synchronize()
    assert rel(torch.cat([Y1, Y2], 1).cpu().numpy(), Y.cpu().numpy()) < 1e-5
    assert rel(S2.cpu().numpy(), S.cpu().numpy()) < 1e-5


def test_factored_scan_single_partial_chunk(fproj, oprojs):
    g = torch.Generator().manual_seed(9)
    q, k = torch.randn(1, 5, 128, generator=g), torch.randn(1, 5, 128, generator=g)
    v = torch.randn(1, 5, 128, generator=g)
    beta = torch.sigmoid(torch.randn(1, 5, generator=g))
    dec = 0.9 + 0.1 * torch.rand(1, 5, generator=g)
    Y, S = factored_chunked_deltanet_forward(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), dec.to(DEV), fproj)
    torch.cuda.synchronize()
    Yr, Sr = oracle_scan(q, k, v, beta, dec, oprojs)
    assert rel(Y.cpu().numpy(), Yr) < 1e-4
    assert rel(S.cpu().numpy(), Sr) < 1e-4


# ------------------------------------------------------------------------------------------------ backward
# Gradient oracle: torch autograd in float64 of oracle.scan.factored_lift_torch (equal to the numpy
# factored-lift oracle, gradcheck-pinned in test_oracle_factored.py) and oracle.scan.token_recurrence_torch
# (gradcheck-pinned in test_oracle_backward.py) -- the role the reference gives torch autograd over its
# chunked forward.  Tolerances (relative L2): 1e-4 for fp32 inputs, 2e-2 for bf16 inputs; the lift's
# backward alone 1e-5 for fp32 inputs and 5e-3 for bf16 inputs (whose dL/dtheta is rounded to bf16 for
# the product with Omega, the bf16 policy of every feature contraction of the backward).

def _t64(x):
    return torch.as_tensor(np.asarray(x, dtype=np.float64))


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 5e-3)])
def test_factored_lift_backward(fproj, oprojs, dtype, tol):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(3, 20, 128, generator=g).to(dtype)
    dphi = torch.randn(3, 20, 1024, generator=g)
    p1, p2 = fproj.proj1, fproj.proj2
    dx = ops.lift_factored_backward(x.to(DEV), dphi.to(DEV), p1.device_omega(DEV), p1.device_phase(DEV),
                                    p2.device_omega(DEV), p2.device_phase(DEV), p1.tau_star_inv)
    torch.cuda.synchronize()
    xr = x.double().requires_grad_(True)
    (osc.factored_lift_torch(xr, *oprojs) * dphi.double()).sum().backward()
    assert dx.shape == x.shape and dx.dtype == torch.float32
    assert rel(dx.cpu().numpy(), xr.grad.numpy()) < tol


def _prelifted_case(B, T, dv, dtype, oprojs, seed):
    g = torch.Generator().manual_seed(seed)
    pq = torch.from_numpy(ol.factored_lift(torch.randn(B, T, 128, generator=g).numpy(), *oprojs)).to(dtype)
    pk = torch.from_numpy(ol.factored_lift(torch.randn(B, T, 128, generator=g).numpy(), *oprojs)).to(dtype)
    v = torch.randn(B, T, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    decay = 0.9 + 0.1 * torch.rand(B, T, generator=g)
    s0 = 0.1 * torch.randn(B, dv, 1024, generator=g)
    dy = torch.randn(B, T, dv, generator=g)
    ds = torch.randn(B, dv, 1024, generator=g)
    return pq, pk, v, beta, decay, s0, dy, ds


def _oracle_scan_grads(pq, pk, v, beta, decay, s0, dy, ds):
    leaves = [t.double().requires_grad_(True) for t in (pq, pk, v, beta, decay, s0)]
    Y, S = osc.token_recurrence_torch(*leaves)
    ((Y * dy.double()).sum() + (S * ds.double()).sum()).backward()
    return [t.grad.numpy() for t in leaves]


@pytest.mark.parametrize("dtype,dv,T", [(torch.float32, 128, 200), (torch.bfloat16, 128, 200),
                                        (torch.float32, 64, 700)])
def test_d1024_scan_backward(oprojs, dtype, dv, T):
    # kdn_delta_scan_bwd at D = 1024 over pre-lifted features: every gradient, with decay, an initial
    # state, dL/dS_T and a partial last chunk
    B = 2
    pq, pk, v, beta, decay, s0, dy, ds = _prelifted_case(B, T, dv, dtype, oprojs, 5)
    d = lambda t: t.to(DEV)
    plan = ops.ScanBackwardPlan(d(pq).unsqueeze(2), d(pk).unsqueeze(2), d(v).unsqueeze(2), d(beta).unsqueeze(-1),
                                d(decay).unsqueeze(-1), None, None, 1.0, d(dy).unsqueeze(2),
                                d(ds).unsqueeze(1).transpose(2, 3), initial_state=d(s0).unsqueeze(1).transpose(2, 3),
                                features=ops.FeatureMap(lifted=True))
    assert plan.segments == 1
    dq, dk, dvv, dbeta, ddecay, dinit = plan.run(concurrent_carries=False)
    torch.cuda.synchronize()
    ref = _oracle_scan_grads(pq, pk, v, beta, decay, s0, dy, ds)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    got = [dq[:, :, 0], dk[:, :, 0], dvv[:, :, 0], dbeta[:, :, 0], ddecay[:, :, 0], dinit[:, 0].transpose(1, 2)]
    for name, a, r in zip(("dphi_q", "dphi_k", "dv", "dbeta", "ddecay", "dS0"), got, ref):
        assert rel(a.cpu().numpy(), r) < tol, name


@pytest.mark.parametrize("dtype,dv", [(torch.float32, 64), (torch.bfloat16, 128)])
def test_d1024_scan_backward_segments(oprojs, dtype, dv):
    # the segmented backward (checkpoint pass, then segments last first with dL/dS carried between them):
    # 11 chunks in segments of 3 give every gradient bit for bit as one segment does, and match the oracle
    B, T = 2, 700
    pq, pk, v, beta, decay, s0, dy, ds = _prelifted_case(B, T, dv, dtype, oprojs, 8)
    d = lambda t: t.to(DEV)
    outs = []
    for seg in (0, 3):
        plan = ops.ScanBackwardPlan(d(pq).unsqueeze(2), d(pk).unsqueeze(2), d(v).unsqueeze(2),
                                    d(beta).unsqueeze(-1), d(decay).unsqueeze(-1), None, None, 1.0,
                                    d(dy).unsqueeze(2), d(ds).unsqueeze(1).transpose(2, 3),
                                    initial_state=d(s0).unsqueeze(1).transpose(2, 3), segment_chunks=seg,
                                    features=ops.FeatureMap(lifted=True))
        assert plan.segments == (1 if seg == 0 else 4)
        outs.append([t.clone() for t in plan.run()])
    torch.cuda.synchronize()
    for name, a, b in zip(("dphi_q", "dphi_k", "dv", "dbeta", "ddecay", "dS0"), *outs):
        assert torch.equal(a, b), name
    ref = _oracle_scan_grads(pq, pk, v, beta, decay, s0, dy, ds)
    dq, dk, dvv, dbeta, ddecay, dinit = outs[1]
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    got = [dq[:, :, 0], dk[:, :, 0], dvv[:, :, 0], dbeta[:, :, 0], ddecay[:, :, 0], dinit[:, 0].transpose(1, 2)]
    for name, a, r in zip(("dphi_q", "dphi_k", "dv", "dbeta", "ddecay", "dS0"), got, ref):
        assert rel(a.cpu().numpy(), r) < tol, name


def test_d1024_scan_backward_is_deterministic(oprojs):
    pq, pk, v, beta, decay, s0, dy, ds = _prelifted_case(1, 300, 128, torch.bfloat16, oprojs, 6)
    d = lambda t: t.to(DEV)
    outs = []
    for _ in range(2):
        plan = ops.ScanBackwardPlan(d(pq).unsqueeze(2), d(pk).unsqueeze(2), d(v).unsqueeze(2),
                                    d(beta).unsqueeze(-1), d(decay).unsqueeze(-1), None, None, 1.0,
                                    d(dy).unsqueeze(2), None, features=ops.FeatureMap(lifted=True))
        outs.append([t.clone() for t in plan.run() if t is not None])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_factored_module_gradients(fproj, oprojs, dtype):
    # autograd through factored_chunked_deltanet_forward (the reference's training path for d_k = 128):
    # gradients of q, k, v, beta, decay and the initial state
    g = torch.Generator().manual_seed(12)
    B, T, dv = 2, 150, 128
    q, k = torch.randn(B, T, 128, generator=g).to(dtype), torch.randn(B, T, 128, generator=g).to(dtype)
    v = torch.randn(B, T, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    decay = 0.9 + 0.1 * torch.rand(B, T, generator=g)
    s0 = 0.1 * torch.randn(B, dv, 1024, generator=g)
    dy, ds = torch.randn(B, T, dv, generator=g), torch.randn(B, dv, 1024, generator=g)
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v, beta, decay, s0)]
    Y, S = factored_chunked_deltanet_forward(*leaves[:5], fproj, initial_state=leaves[5])
    ((Y.float() * dy.to(DEV)).sum() + (S.float() * ds.to(DEV)).sum()).backward()
    torch.cuda.synchronize()
    refs = [t.double().requires_grad_(True) for t in (q, k, v, beta, decay, s0)]
    Yr, Sr = osc.token_recurrence_torch(osc.factored_lift_torch(refs[0], *oprojs),
                                        osc.factored_lift_torch(refs[1], *oprojs), *refs[2:])
    ((Yr * dy.double()).sum() + (Sr * ds.double()).sum()).backward()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for name, a, r in zip(("dq", "dk", "dv", "dbeta", "ddecay", "dS0"), leaves, refs):
        assert a.grad is not None and a.grad.dtype == a.dtype, name
        assert rel(a.grad.float().cpu().numpy(), r.grad.numpy()) < tol, name


def test_d1024_scan_backward_two_heads_without_decay(oprojs):
    # head indexing of every record and gradient (H = 2 in the (B, T, H, .) layout), no decay, no initial
    # state and no dL/dS_T (their NULL paths), a partial last chunk
    g = torch.Generator().manual_seed(21)
    B, T, H, dv = 1, 130, 2, 64
    pq = torch.from_numpy(ol.factored_lift(torch.randn(B, T, H, 128, generator=g).numpy(), *oprojs)).float()
    pk = torch.from_numpy(ol.factored_lift(torch.randn(B, T, H, 128, generator=g).numpy(), *oprojs)).float()
    v = torch.randn(B, T, H, dv, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    dy = torch.randn(B, T, H, dv, generator=g)
    plan = ops.ScanBackwardPlan(pq.to(DEV), pk.to(DEV), v.to(DEV), beta.to(DEV), None, None, None, 1.0, dy.to(DEV),
                                need_dinit=False, features=ops.FeatureMap(lifted=True))
    dq, dk, dvv, dbeta, ddecay, dinit = plan.run()
    torch.cuda.synchronize()
    assert ddecay is None and dinit is None
    for h in range(H):
        leaves = [t[:, :, h].double().requires_grad_(True) for t in (pq, pk, v, beta)]
        Y, _ = osc.token_recurrence_torch(*leaves)
        (Y * dy[:, :, h].double()).sum().backward()
        for name, a, r in zip(("dphi_q", "dphi_k", "dv", "dbeta"), (dq, dk, dvv, dbeta), leaves):
            assert rel(a[:, :, h].cpu().numpy(), r.grad.numpy()) < 1e-4, (h, name)
