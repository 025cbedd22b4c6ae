"""GPU parity of the D = 512 backward at d_v = 16, 32 and 128 (kdn_delta_scan_bwd: the 64-wide backward
over the value columns, split in two halves for d_v = 128 and zero-padded for d_v < 64).

Oracle: torch autograd in float64 on the CPU of oracle.scan.delta_rule_torch (the token recurrence over
the lift, gradcheck-pinned in test_oracle_backward.py) for L = sum(y * dy) + sum(S_T * dS).  Tolerances
(relative L2): 1e-4 for fp32 inputs, 2e-2 for bf16 inputs, as every backward test.  Cases: every
gradient with decay, initial state and dL/dS_T at T = 200 (a partial last chunk); the reference's own test
shape (tests/test_fused_kernel.py:70-107: B = 2, d_v = 128, D = 512, chunk_size = 32) through the
differentiable P1 surface; the two streams' schedule bit-identical to the one-stream schedule.
"""
import numpy as np
import pytest
import torch

from kdn import ops
from kernels import FastWalshHadamardProjection, fused_chunked_deltanet_forward
from oracle import lift as ol
from oracle import scan as osc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


@pytest.fixture(scope="module")
def proj():
    return FastWalshHadamardProjection(64, 512, 42)


@pytest.fixture(scope="module")
def oproj():
    return ol.make_projection(64, 512, 42)


def rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def make(B, T, H, dv, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g).to(dtype)
    k = torch.randn(B, T, H, 64, generator=g).to(dtype)
    v = torch.randn(B, T, H, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    lam = 0.9 + 0.1 * torch.rand(B, T, H, generator=g)
    s0 = 0.1 * torch.randn(B, H, 512, dv, generator=g)
    dy = torch.randn(B, T, H, dv, generator=g)
    ds = 0.5 * torch.randn(B, H, 512, dv, generator=g)
    return q, k, v, beta, lam, s0, dy, ds


def oracle_grads(q, k, v, beta, lam, s0, dy, ds, oproj):
    B, T, H, _ = q.shape
    dv = v.shape[-1]

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
    sf = s0.double().reshape(B * H, 512, dv).transpose(1, 2).clone().requires_grad_(True)
    Y, S = osc.delta_rule_torch(qf, kf, vf, bf, lf, oproj, sf, False)
    L = (Y * fold(dy)).sum() + (S * ds.double().reshape(B * H, 512, dv).transpose(1, 2)).sum()
    L.backward()
    return {"dq": unfold(qf.grad), "dk": unfold(kf.grad), "dv": unfold(vf.grad), "dbeta": unfold(bf.grad),
            "ddecay": unfold(lf.grad), "dinit": sf.grad.transpose(1, 2).reshape(B, H, 512, dv)}


def gpu_grads(proj, q, k, v, beta, lam, s0, dy, ds):
    dq, dk, dv, db, dd, di = ops.scan_backward(
        q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), proj.device_omega(DEV), proj.device_phase(DEV),
        proj.tau_star_inv, dy.to(DEV), ds.to(DEV), initial_state=s0.to(DEV))
    torch.cuda.synchronize()
    return {"dq": dq.cpu(), "dk": dk.cpu(), "dv": dv.cpu(), "dbeta": db.cpu(), "ddecay": dd.cpu(), "dinit": di.cpu()}


@pytest.mark.parametrize("dv", [16, 32, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_other_dv_matches_float64_autograd(proj, oproj, dv, dtype):
    q, k, v, beta, lam, s0, dy, ds = make(1, 200, 2, dv, dtype, seed=dv + (dtype == torch.bfloat16))
    got = gpu_grads(proj, q, k, v, beta, lam, s0, dy, ds)
    ref = oracle_grads(q, k, v, beta, lam, s0, dy, ds, oproj)
    errs = {n: rel(got[n].numpy(), ref[n].detach().numpy()) for n in ref}
    assert all(e < TOL[dtype] for e in errs.values()), errs


def test_reference_test_shape_through_the_surface(proj, oproj):
    """tests/test_fused_kernel.py:70-107 of the reference: B = 2, d_v = 128, D = 512, chunk_size = 32, fp32,
    gradients of every input through fused_chunked_deltanet_forward."""
    g = torch.Generator().manual_seed(42)
    B, T, dv = 2, 96, 128
    q, k, v = torch.randn(B, T, 64, generator=g), torch.randn(B, T, 64, generator=g), torch.randn(B, T, dv, generator=g)
    beta, decay = torch.sigmoid(torch.randn(B, T, generator=g)), torch.sigmoid(torch.randn(B, T, generator=g))
    dy = torch.randn(B, T, dv, generator=g)
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v, beta, decay)]
    y, _ = fused_chunked_deltanet_forward(*leaves, proj.to(DEV), chunk_size=32)
    (y * dy.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    ref = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, decay)]
    yo, _ = osc.delta_rule_torch(ref[0], ref[1], ref[2], ref[3], ref[4], oproj)
    (yo * dy.double()).sum().backward()
    errs = [rel(a.grad.cpu().numpy(), r.grad.numpy()) for a, r in zip(leaves, ref)]
    assert max(errs) < TOL[torch.float32], errs


def test_two_streams_equal_one_stream_dv128(proj):
    q, k, v, beta, lam, s0, dy, ds = make(1, 64 * 9 + 5, 2, 128, torch.bfloat16, seed=7)
    d = lambda t: t.to(DEV)
    outs = []
    for concurrent in (False, True):
        plan = ops.ScanBackwardPlan(d(q), d(k), d(v), d(beta), d(lam), proj.device_omega(DEV), proj.device_phase(DEV),
                                    proj.tau_star_inv, d(dy), d(ds), initial_state=d(s0), need_ddecay=True,
                                    need_dinit=True, segment_chunks=4)
        outs.append([t.clone() for t in plan.run(concurrent_carries=concurrent) if t is not None])
        torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
