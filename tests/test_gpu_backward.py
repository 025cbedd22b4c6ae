"""GPU parity of the scan's backward pass (kdn_delta_scan_bwd) and of the differentiable surfaces.

Oracle: torch autograd, in float64 on the CPU, of oracle.scan.delta_rule_torch (the token recurrence over
the lift, pinned by gradcheck in test_oracle_backward.py) on the same inputs (bf16 inputs rounded
first), for L = sum(y * dy) + sum(S_T * dS).  Tolerances (relative L2), as for the forward: 1e-4 for
fp32 inputs (every product in fp32), 2e-2 for bf16 inputs (the 512-feature contractions take bf16
operands with fp32 accumulation, the forward's bf16 policy).  At sizes the oracle cannot afford:
exactness of the gradient of the (bilinear) v-direction against the forward kernel, and linearity of
the backward in (dy, dS).
"""
import numpy as np
import pytest
import torch

from kdn import ops
from kernels import FastWalshHadamardProjection, FusedKernelDeltaNetFunction, fused_chunked_deltanet_forward
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
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def make(B, T, H, dtype, seed, decay=True, init=True, dfinal=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g).to(dtype)
    k = torch.randn(B, T, H, 64, generator=g).to(dtype)
    v = torch.randn(B, T, H, 64, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    lam = (0.9 + 0.1 * torch.rand(B, T, H, generator=g)) if decay else None
    s0 = 0.1 * torch.randn(B, H, 512, 64, generator=g) if init else None
    dy = torch.randn(B, T, H, 64, generator=g)
    ds = 0.5 * torch.randn(B, H, 512, 64, generator=g) if dfinal else None
    return q, k, v, beta, lam, s0, dy, ds


def oracle_grads(q, k, v, beta, lam, s0, dy, ds, oproj, normalize=False):
    """Float64 autograd of the token recurrence; gradients returned in the kernel layouts."""
    B, T, H, _ = q.shape

    def fold(x):  # (B, T, H, d) -> (B*H, T, d); (B, T, H) -> (B*H, T)
        x = x.double()
        if x.dim() == 4:
            return x.permute(0, 2, 1, 3).reshape(B * H, T, -1).clone()
        return x.permute(0, 2, 1).reshape(B * H, T).clone()

    def unfold(x):
        if x.dim() == 3:
            return x.reshape(B, H, T, -1).permute(0, 2, 1, 3)
        return x.reshape(B, H, T).permute(0, 2, 1)

    qf, kf, vf, bf = (fold(t).requires_grad_(True) for t in (q.float(), k.float(), v.float(), beta))
    lf = fold(lam).requires_grad_(True) if lam is not None else None
    sf = s0.double().reshape(B * H, 512, 64).transpose(1, 2).clone().requires_grad_(True) if s0 is not None else None
    Y, S = osc.delta_rule_torch(qf, kf, vf, bf, lf, oproj, sf, normalize)
    L = (Y * fold(dy)).sum()
    if ds is not None:
        L = L + (S * ds.double().reshape(B * H, 512, 64).transpose(1, 2)).sum()
    L.backward()
    out = {"dq": unfold(qf.grad), "dk": unfold(kf.grad), "dv": unfold(vf.grad), "dbeta": unfold(bf.grad)}
    if lf is not None:
        out["ddecay"] = unfold(lf.grad)
    if sf is not None:
        out["dinit"] = sf.grad.transpose(1, 2).reshape(B, H, 512, 64)
    return out


def gpu_grads(proj, q, k, v, beta, lam, s0, dy, ds, normalize=False):
    dq, dk, dv, db, dd, di = ops.scan_backward(
        q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), None if lam is None else lam.to(DEV), proj.device_omega(DEV),
        proj.device_phase(DEV), proj.tau_star_inv, dy.to(DEV), None if ds is None else ds.to(DEV),
        normalize=normalize, initial_state=None if s0 is None else s0.to(DEV))
    torch.cuda.synchronize()
    out = {"dq": dq.cpu(), "dk": dk.cpu(), "dv": dv.cpu(), "dbeta": db.cpu()}
    if dd is not None:
        out["ddecay"] = dd.cpu()
    if s0 is not None:
        out["dinit"] = di.cpu()
    return out


def check(got, ref, tol=TOL[torch.float32]):
    assert set(got) == set(ref), (sorted(got), sorted(ref))
    errs = {k: rel(got[k].numpy(), ref[k].detach().numpy()) for k in ref}
    assert all(e < tol for e in errs.values()), errs


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_parity(proj, oproj, dtype):
    # T = 200: three full chunks and a partial one; decay, initial state and dL/dS_T all present
    args = make(1, 200, 2, dtype, seed=11)
    check(gpu_grads(proj, *args), oracle_grads(*args, oproj), TOL[dtype])


def test_backward_normalised_inputs(proj, oproj):
    args = make(1, 130, 2, torch.float32, seed=12)
    check(gpu_grads(proj, *args, normalize=True), oracle_grads(*args, oproj, normalize=True))


def test_backward_without_decay_state_or_final_gradient(proj, oproj):
    args = make(2, 70, 1, torch.float32, seed=13, decay=False, init=False, dfinal=False)
    check(gpu_grads(proj, *args), oracle_grads(*args, oproj))


def test_backward_single_partial_chunk(proj, oproj):
    args = make(1, 5, 1, torch.float32, seed=14)
    check(gpu_grads(proj, *args), oracle_grads(*args, oproj))


def test_backward_is_linear_in_the_output_gradients(proj):
    # large enough for many chunks and a 32-workgroup chain grid: bwd(a dy1 + b dy2) = a bwd(dy1) + b bwd(dy2)
    q, k, v, beta, lam, s0, dy1, ds1 = make(2, 1500, 4, torch.float32, seed=15)
    g = torch.Generator().manual_seed(16)
    dy2, ds2 = torch.randn(dy1.shape, generator=g), torch.randn(ds1.shape, generator=g)
    g1 = gpu_grads(proj, q, k, v, beta, lam, s0, dy1, ds1)
    g2 = gpu_grads(proj, q, k, v, beta, lam, s0, dy2, ds2)
    g12 = gpu_grads(proj, q, k, v, beta, lam, s0, 2.0 * dy1 - 0.5 * dy2, 2.0 * ds1 - 0.5 * ds2)
    for key in g1:
        assert rel(g12[key].numpy(), (2.0 * g1[key] - 0.5 * g2[key]).numpy()) < 1e-5, key


def test_value_gradient_matches_the_forward_at_length(proj):
    # L is bilinear in v and dy: L(v + d) - L(v - d) = 2 <dL/dv, d> exactly, through the forward kernel
    q, k, v, beta, lam, s0, dy, ds = make(1, 4096, 2, torch.float32, seed=17)
    d = torch.randn(v.shape, generator=torch.Generator().manual_seed(18))
    omega, phase = proj.device_omega(DEV), proj.device_phase(DEV)

    def loss(vv):
        y, S = ops.scan(q.to(DEV), k.to(DEV), vv.to(DEV), beta.to(DEV), lam.to(DEV), omega, phase, proj.tau_star_inv,
                        initial_state=s0.to(DEV))
        return float((y.double() * dy.to(DEV).double()).sum() + (S.double() * ds.to(DEV).double()).sum())

    fd = (loss(v + d) - loss(v - d)) / 2.0
    gv = gpu_grads(proj, q, k, v, beta, lam, s0, dy, ds)["dv"]
    an = float((gv.double() * d.double()).sum())
    assert abs(fd - an) <= 1e-4 * max(abs(an), 1.0), (fd, an)


def test_p1_surface_autograd(proj, oproj):
    # fused_chunked_deltanet_forward with requires_grad records the scan's autograd node
    q, k, v, beta, lam, s0, dy, ds = make(2, 90, 1, torch.float32, seed=19)
    leaves = [t.squeeze(2).to(DEV).requires_grad_(True) for t in (q, k, v)] + \
             [beta.squeeze(-1).to(DEV).requires_grad_(True), lam.squeeze(-1).to(DEV).requires_grad_(True)]
    init = s0.squeeze(1).transpose(1, 2).contiguous().to(DEV).requires_grad_(True)  # (B, d_v, D)
    Y, S = fused_chunked_deltanet_forward(*leaves, proj, 64, init)
    L = (Y * dy.squeeze(2).to(DEV)).sum() + (S * ds.squeeze(1).transpose(1, 2).to(DEV)).sum()
    L.backward()
    ref = oracle_grads(q, k, v, beta, lam, s0, dy, ds, oproj)
    got = {"dq": leaves[0].grad.unsqueeze(2).cpu(), "dk": leaves[1].grad.unsqueeze(2).cpu(),
           "dv": leaves[2].grad.unsqueeze(2).cpu(), "dbeta": leaves[3].grad.unsqueeze(-1).cpu(),
           "ddecay": leaves[4].grad.unsqueeze(-1).cpu(), "dinit": init.grad.transpose(1, 2).unsqueeze(1).cpu()}
    check(got, ref)


def test_function_apply_backward(proj, oproj):
    q, k, v, beta, lam, _, dy, _ = make(3, 64, 1, torch.float32, seed=20, init=False, dfinal=False)
    leaves = [t.squeeze(2).to(DEV).requires_grad_(True) for t in (q, k, v)] + \
             [beta.squeeze(-1).to(DEV).requires_grad_(True), lam.squeeze(-1).to(DEV).requires_grad_(True)]
    Y = FusedKernelDeltaNetFunction.apply(*leaves, proj, 64)
    (Y * dy.squeeze(2).to(DEV)).sum().backward()
    ref = oracle_grads(q, k, v, beta, lam, None, dy, None, oproj)
    got = {"dq": leaves[0].grad.unsqueeze(2).cpu(), "dk": leaves[1].grad.unsqueeze(2).cpu(),
           "dv": leaves[2].grad.unsqueeze(2).cpu(), "dbeta": leaves[3].grad.unsqueeze(-1).cpu(),
           "ddecay": leaves[4].grad.unsqueeze(-1).cpu()}
    check(got, ref)


def test_backward_rejects_unsupported_shapes(proj):
    q = torch.randn(1, 64, 1, 64, device=DEV)
    v = torch.randn(1, 64, 1, 48, device=DEV)   # d_v outside {16, 32, 64, 128}
    beta = torch.rand(1, 64, 1, device=DEV)
    with pytest.raises(ValueError, match="unsupported"):
        ops.scan_backward(q, q, v, beta, None, proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv,
                          torch.randn(1, 64, 1, 48, device=DEV))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_two_streams_equal_one_stream_bit_for_bit(proj, dtype):
    # kdn_delta_scan_bwd_streams runs the reverse carries on the launch stream and everything else on an
    # auxiliary stream; every reduction has a fixed order, so its results equal kdn_delta_scan_bwd's bit
    # for bit, and two runs on one stream agree bit for bit.  Segments of 4 chunks (6 segments over three
    # rotating record buffers); issued twice back to back so that the second call's recompute overwrites
    # records only after the first call's readers are done.
    q, k, v, beta, lam, s0, dy, ds = make(2, 1500, 4, dtype, seed=21)
    plan = ops.ScanBackwardPlan(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), proj.device_omega(DEV),
                                proj.device_phase(DEV), proj.tau_star_inv, dy.to(DEV), ds.to(DEV),
                                initial_state=s0.to(DEV), segment_chunks=4)
    assert plan.segments == 6 and plan.segment_chunks == 4
    ref = [t.clone() for t in plan.run(concurrent_carries=False)]
    again = [t.clone() for t in plan.run(concurrent_carries=False)]
    for _ in range(2):
        got = plan.run(concurrent_carries=True)
    torch.cuda.synchronize()
    names = ("dq", "dk", "dv", "dbeta", "ddecay", "dinit")
    for n, g, a, r in zip(names, got, again, ref):
        assert torch.equal(a, r), n
        assert torch.equal(g, r), n


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_parity_segmented(proj, oproj, dtype):
    # one (batch, head) at T = 1500 (24 chunks, the last partial) in segments of 5 chunks (4 full segments
    # and one of 4): the checkpoint pass, the carried dL/dS and the segment-local chunk indexing all count
    args = make(1, 1500, 1, dtype, seed=22)
    q, k, v, beta, lam, s0, dy, ds = args
    dq, dk, dv, db, dd, di = ops.scan_backward(
        q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), proj.device_omega(DEV), proj.device_phase(DEV),
        proj.tau_star_inv, dy.to(DEV), ds.to(DEV), initial_state=s0.to(DEV), segment_chunks=5)
    got = {"dq": dq.cpu(), "dk": dk.cpu(), "dv": dv.cpu(), "dbeta": db.cpu(), "ddecay": dd.cpu(), "dinit": di.cpu()}
    check(got, oracle_grads(*args, oproj), TOL[dtype])


def test_segment_length_changes_only_rounding(proj):
    # the same gradients in one segment and in segments of 3 chunks (fp32: rounding only)
    q, k, v, beta, lam, s0, dy, ds = make(2, 1500, 2, torch.float32, seed=23)
    runs = []
    for seg in (0, 3):
        dq, dk, dv, db, dd, di = ops.scan_backward(
            q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), proj.device_omega(DEV),
            proj.device_phase(DEV), proj.tau_star_inv, dy.to(DEV), ds.to(DEV), initial_state=s0.to(DEV),
            segment_chunks=seg)
        runs.append([t.cpu() for t in (dq, dk, dv, db, dd, di)])
    for n, a, b in zip(("dq", "dk", "dv", "dbeta", "ddecay", "dinit"), *runs):
        assert rel(a.numpy(), b.numpy()) < 1e-5, n


def test_backward_config4_shape(proj):
    # B = 32, H = 16, T = 16384 (bf16, decay, initial state, dL/dS_T): the workspace is bounded by the
    # segment (default 8 chunks at B*H = 512), every gradient is finite, and one (batch, head) equals bit
    # for bit the backward of that head alone with the same segments (no kernel mixes heads), which the
    # segmented parity test above pins to the float64 oracle
    B, T, H = 32, 16384, 16
    g = torch.Generator(device=DEV).manual_seed(24)
    q = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device=DEV))
    lam = 0.95 + 0.05 * torch.rand(B, T, H, generator=g, device=DEV)
    s0 = 0.1 * torch.randn(B, H, 512, 64, generator=g, device=DEV)
    dy = torch.randn(B, T, H, 64, generator=g, device=DEV)
    ds = 0.5 * torch.randn(B, H, 512, 64, generator=g, device=DEV)
    omega, phase = proj.device_omega(DEV), proj.device_phase(DEV)
    plan = ops.ScanBackwardPlan(q, k, v, beta, lam, omega, phase, proj.tau_star_inv, dy, ds, initial_state=s0)
    assert plan.segment_chunks == 8 and plan.segments == 32
    # the records of three 8-chunk segments, 31 segment-start states and the carry, the checkpoint
    # pass's two buffers and the table: about 18 GB, against 163 GB for records of every chunk
    print("workspace bytes", plan.workspace.numel(), flush=True)
    assert plan.workspace.numel() < 19 * 10**9
    full = [t.clone() for t in plan.run()]
    torch.cuda.synchronize()
    for n, t in zip(("dq", "dk", "dv", "dbeta", "ddecay", "dinit"), full):
        assert bool(torch.isfinite(t).all()), n
    del plan
    b, h = 5, 7
    one = ops.scan_backward(q[b:b + 1, :, h:h + 1], k[b:b + 1, :, h:h + 1], v[b:b + 1, :, h:h + 1],
                            beta[b:b + 1, :, h:h + 1], lam[b:b + 1, :, h:h + 1], omega, phase, proj.tau_star_inv,
                            dy[b:b + 1, :, h:h + 1], ds[b:b + 1, h:h + 1].contiguous(),
                            initial_state=s0[b:b + 1, h:h + 1].contiguous(), segment_chunks=8)
    torch.cuda.synchronize()
    for n, f, o in zip(("dq", "dk", "dv", "dbeta", "ddecay"), full, one):
        assert torch.equal(f[b:b + 1, :, h:h + 1], o), n
    assert torch.equal(full[5][b:b + 1, h:h + 1], one[5]), "dinit"


def test_backward_config3_default_segments(proj):
    # B = 1, H = 16, T = 65536 (bf16, decay, initial state, dL/dS_T): the default segment is 256 chunks,
    # so each of the three segment buffers of records spans 4.5 GB and the last heads' records lie past
    # 2^31 bytes into their buffer; every gradient is finite and that head equals bit for bit the backward
    # of the head alone with the same segments
    B, T, H = 1, 65536, 16
    g = torch.Generator(device=DEV).manual_seed(25)
    q = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device=DEV))
    lam = 0.95 + 0.05 * torch.rand(B, T, H, generator=g, device=DEV)
    s0 = 0.1 * torch.randn(B, H, 512, 64, generator=g, device=DEV)
    dy = torch.randn(B, T, H, 64, generator=g, device=DEV)
    ds = 0.5 * torch.randn(B, H, 512, 64, generator=g, device=DEV)
    omega, phase = proj.device_omega(DEV), proj.device_phase(DEV)
    plan = ops.ScanBackwardPlan(q, k, v, beta, lam, omega, phase, proj.tau_star_inv, dy, ds, initial_state=s0)
    assert plan.segment_chunks == 256 and plan.segments == 4
    print("workspace bytes", plan.workspace.numel(), flush=True)
    assert plan.workspace.numel() < 16 * 10**9
    full = [t.clone() for t in plan.run()]
    torch.cuda.synchronize()
    for n, t in zip(("dq", "dk", "dv", "dbeta", "ddecay", "dinit"), full):
        assert bool(torch.isfinite(t).all()), n
    del plan
    h = 15
    one = ops.scan_backward(q[:, :, h:h + 1], k[:, :, h:h + 1], v[:, :, h:h + 1], beta[:, :, h:h + 1],
                            lam[:, :, h:h + 1], omega, phase, proj.tau_star_inv, dy[:, :, h:h + 1],
                            ds[:, h:h + 1].contiguous(), initial_state=s0[:, h:h + 1].contiguous(),
                            segment_chunks=256)
    torch.cuda.synchronize()
    for n, f, o in zip(("dq", "dk", "dv", "dbeta", "ddecay"), full, one):
        assert torch.equal(f[:, :, h:h + 1], o), n
    assert torch.equal(full[5][:, h:h + 1], one[5]), "dinit"
