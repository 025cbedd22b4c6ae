"""GPU parity at the BASELINE workloads that fill the GPU (configs 4 and 5) and of the P1 module surface.

- Config 4 (B=32, H=16, D=512, d_v=64, bf16): at T=4096 every output is finite, all 512 heads' first 512
  tokens and three sampled (b, h) over the whole sequence match the float64 chunked oracle; at T=16384
  three (b, h) over the whole sequence match it; at T=65536
  the prefill split in two halves equals the single call bit for bit and one (b, h) over the full length
  matches the oracle.
- Config 5 (bench.py's step: 224 decodes + 32 prefills of U[512, 8192] tokens, seed 1234, H=16): every
  decode sequence and 4 prefill sequences x 2 heads over their full length match the float64 oracle,
  continuing from their slot states; slots no sequence uses come back bit-identical.
- a7: FusedKernelDeltaNet(...).forward (kernels/fused_kernel_deltanet.py:182-209 of the reference) with
  and without initial_state, and a backward through it, against the oracle and float64 autograd.
Tolerances (relative L2): 2e-2 for bf16 inputs with the fp32 state, 1e-4 for fp32.
"""
import numpy as np
import pytest
import torch

from kdn import ops
from kernels import FastWalshHadamardProjection, FusedKernelDeltaNet
from oracle import lift as ol
from oracle import scan as osc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL_BF16 = 2e-2


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.fixture(scope="module")
def proj():
    return FastWalshHadamardProjection(64, 512, 42)


@pytest.fixture(scope="module")
def oproj():
    return ol.make_projection(64, 512, 42)


def device_inputs(B, T, H, seed=1234):
    """q, k, v ~ N(0,1) (bf16) and beta = sigmoid(N(0,1)) (fp32) drawn on the device (bench.py's order)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, T, H, 64, generator=g, device=DEV).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device=DEV))
    return q, k, v, beta


def oracle_head(q, k, v, beta, b, h, oproj, T=None, S0=None):
    """Float64 chunked oracle of one (b, h) stream over its first T tokens (all when None)."""
    sl = slice(None, T)
    f = lambda t: t[b:b + 1, sl, h].float().cpu().double()
    s0 = None if S0 is None else S0.double()[None]
    y, S = osc.chunked_forward(f(q), f(k), f(v), beta[b:b + 1, sl, h].cpu().double(), None, oproj, 64, s0,
                               torch.float64)
    return y[0].numpy(), S[0].numpy()   # (T, dv), (dv, D)


def run(proj, q, k, v, beta, **kw):
    return ops.scan(q, k, v, beta, None, proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv, **kw)


def test_config4_T4096(proj, oproj):
    B, T, H = 32, 4096, 16
    q, k, v, beta = device_inputs(B, T, H)
    y, S = run(proj, q, k, v, beta)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(S).all()
    # every head over its first 512 tokens (8 chunks of each of the 512 streams)
    n0 = 512
    f = lambda t: t[:, :n0].float().cpu().permute(0, 2, 1, 3).reshape(B * H, n0, -1).double()
    fb = beta[:, :n0].cpu().permute(0, 2, 1).reshape(B * H, n0).double()
    yr, _ = osc.chunked_forward(f(q), f(k), f(v), fb, None, oproj, 64, None, torch.float64)
    yr = yr.numpy().reshape(B, H, n0, 64).transpose(0, 2, 1, 3)
    assert rel_l2(y[:, :n0].float().cpu().numpy(), yr) < TOL_BF16
    # three streams over the whole sequence
    for b, h in ((0, 0), (17, 9), (31, 15)):
        yh, Sh = oracle_head(q, k, v, beta, b, h, oproj)
        assert rel_l2(y[b, :, h].float().cpu().numpy(), yh) < TOL_BF16, (b, h)
        assert rel_l2(S[b, h].t().cpu().numpy(), Sh) < TOL_BF16, (b, h)


def test_config4_T16384(proj, oproj):
    """The config-4 sweep point T = 16384 (the fused schedule by default at B*H = 512): three (b, h) streams
    over the whole sequence against the float64 oracle, every output finite."""
    B, T, H = 32, 16384, 16
    q, k, v, beta = device_inputs(B, T, H, seed=16384)
    y, S = run(proj, q, k, v, beta)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(S).all()
    for b, h in ((0, 3), (13, 0), (31, 15)):
        yh, Sh = oracle_head(q, k, v, beta, b, h, oproj)
        assert rel_l2(y[b, :, h].float().cpu().numpy(), yh) < TOL_BF16, (b, h)
        assert rel_l2(S[b, h].t().cpu().numpy(), Sh) < TOL_BF16, (b, h)


def test_config4_T65536(proj, oproj):
    B, T, H = 32, 65536, 16
    q, k, v, beta = device_inputs(B, T, H)
    y, S = run(proj, q, k, v, beta)
    torch.cuda.synchronize()
    assert torch.isfinite(S).all()
    half = T // 2
    ya, Sa = run(proj, q[:, :half], k[:, :half], v[:, :half], beta[:, :half])
    yb, Sb = run(proj, q[:, half:], k[:, half:], v[:, half:], beta[:, half:], initial_state=Sa)
    torch.cuda.synchronize()
    assert torch.equal(ya, y[:, :half]) and torch.equal(yb, y[:, half:])
    assert torch.equal(Sb, S)
    del ya, yb, Sa, Sb
    b, h = 23, 6
    yh, Sh = oracle_head(q, k, v, beta, b, h, oproj)
    assert rel_l2(y[b, :, h].float().cpu().numpy(), yh) < TOL_BF16
    assert rel_l2(S[b, h].t().cpu().numpy(), Sh) < TOL_BF16


def config5_step(n_slots):
    """bench.py's config-5 step (bench_serving): 224 one-token decodes then 32 prefills with lengths
    U[512, 8192] (CPU generator seeded 1234), q/k/v/beta drawn on the device (seed 1234), states
    N(0,1) * 0.01 in a slab of n_slots slots; the 256 sequences use a random subset of the slots."""
    H, n_dec, n_pre = 16, 224, 32
    g = torch.Generator().manual_seed(1234)
    pre_lens = torch.randint(512, 8193, (n_pre,), generator=g)
    lens = torch.cat([torch.ones(n_dec, dtype=torch.int64), pre_lens])
    T = int(lens.sum())
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(lens, 0)])
    gd = torch.Generator(device=DEV).manual_seed(1234)
    q = torch.randn(T, H, 64, generator=gd, device=DEV).to(torch.bfloat16)
    k = torch.randn(T, H, 64, generator=gd, device=DEV).to(torch.bfloat16)
    v = torch.randn(T, H, 64, generator=gd, device=DEV).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(T, H, generator=gd, device=DEV))
    states = torch.randn(n_slots, H, 512, 64, generator=gd, device=DEV) * 0.01
    slots = torch.randperm(n_slots, generator=g)[: n_dec + n_pre].to(torch.int32)
    return q, k, v, beta, cu, slots, states, n_dec


def test_config5_step(proj, oproj):
    n_slots = 300
    q, k, v, beta, cu, slots, states, n_dec = config5_step(n_slots)
    before = states.clone()
    cu_d, slots_d = cu.to(DEV), slots.to(DEV)
    y = ops.ragged_step(q, k, v, beta, None, cu, slots_d, states, proj.device_omega(DEV), proj.device_phase(DEV),
                        proj.tau_star_inv, cu_seqlens_device=cu_d)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    H = q.shape[1]
    # every decode sequence, all heads: y = S_0 phi(q), S_1 = S_0 + beta phi(k) (v - S_0^T phi(k))^T
    rows = cu[:n_dec].numpy()
    qd, kd, vd = (t[rows].float().cpu().double().numpy() for t in (q, k, v))
    bd = beta[rows].cpu().double().numpy()
    pq = ol.lift(qd.reshape(-1, 64), oproj).reshape(n_dec, H, 512)
    pk = ol.lift(kd.reshape(-1, 64), oproj).reshape(n_dec, H, 512)
    s_idx = slots[:n_dec].long()
    S0 = before[s_idx.to(DEV)].cpu().double().numpy()            # (n_dec, H, D, dv)
    y_ref = np.einsum("nhdj,nhd->nhj", S0, pq)
    u = np.einsum("nhdj,nhd->nhj", S0, pk)
    S1 = S0 + np.einsum("nhd,nhj->nhdj", pk, bd[..., None] * (vd - u))
    assert rel_l2(y[rows].float().cpu().numpy(), y_ref) < TOL_BF16
    assert rel_l2(states[s_idx.to(DEV)].cpu().numpy(), S1) < TOL_BF16
    for i in range(n_dec):   # per sequence too, so that one bad sequence cannot hide in the total
        assert rel_l2(y[rows[i]].float().cpu().numpy(), y_ref[i]) < TOL_BF16, i
    # four prefill sequences (the shortest, the longest and two others), two heads each, full length
    pre = list(range(n_dec, n_dec + 32))
    lens = (cu[1:] - cu[:-1]).numpy()
    pick = sorted({min(pre, key=lambda i: lens[i]), max(pre, key=lambda i: lens[i]), pre[5], pre[20]})
    for i in pick:
        lo, hi, s = int(cu[i]), int(cu[i + 1]), int(slots[i])
        for h in (0, 13):
            f = lambda t: t[lo:hi, h].float().cpu().double()[None]
            yr, Sr = osc.chunked_forward(f(q), f(k), f(v), beta[lo:hi, h].cpu().double()[None], None, oproj, 64,
                                         before[s, h].t().cpu().double()[None], torch.float64)
            assert rel_l2(y[lo:hi, h].float().cpu().numpy(), yr[0].numpy()) < TOL_BF16, (i, h)
            assert rel_l2(states[s, h].t().cpu().numpy(), Sr[0].numpy()) < TOL_BF16, (i, h)
    used = set(slots.tolist())
    unused = torch.tensor([s for s in range(n_slots) if s not in used], device=DEV)
    assert unused.numel() == n_slots - 256
    assert torch.equal(states[unused], before[unused])


@pytest.mark.parametrize("with_init", [False, True])
def test_p1_module_forward_and_backward(oproj, with_init):
    """FusedKernelDeltaNet (kernels/fused_kernel_deltanet.py:182-209 of the reference): d_model is d_k,
    forward(q, k, v, beta, decay, initial_state) -> (Y, S) with S in the reference's (B, d_v, D) layout;
    gradients through it against float64 autograd of the oracle's token recurrence."""
    m = FusedKernelDeltaNet(d_model=64, d_kernel=512, chunk_size=64).to(DEV)
    g = torch.Generator().manual_seed(77)
    B, T = 3, 200
    q, k, v = (torch.randn(B, T, 64, generator=g) for _ in range(3))
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    decay = 0.9 + 0.1 * torch.rand(B, T, generator=g)
    s0 = 0.1 * torch.randn(B, 64, 512, generator=g) if with_init else None
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, k, v, beta, decay)]
    init = s0.to(DEV).requires_grad_(True) if with_init else None
    Y, S = m(*leaves, initial_state=init)
    assert Y.shape == (B, T, 64) and S.shape == (B, 64, 512)
    yr, Sr = osc.chunked_forward(q.double(), k.double(), v.double(), beta.double(), decay.double(), oproj, 64,
                                 None if s0 is None else s0.double(), torch.float64)
    assert rel_l2(Y.detach().cpu().numpy(), yr.numpy()) < 1e-4
    assert rel_l2(S.detach().cpu().numpy(), Sr.numpy()) < 1e-4
    dy = torch.randn(B, T, 64, generator=g)
    dS = 0.3 * torch.randn(B, 64, 512, generator=g)
    ((Y * dy.to(DEV)).sum() + (S * dS.to(DEV)).sum()).backward()
    ref = [t.double().clone().requires_grad_(True) for t in (q, k, v, beta, decay)]
    rs0 = s0.double().clone().requires_grad_(True) if with_init else None
    yo, So = osc.delta_rule_torch(ref[0], ref[1], ref[2], ref[3], ref[4], oproj, rs0)
    ((yo * dy.double()).sum() + (So * dS.double()).sum()).backward()
    for got, want in zip(leaves, ref):
        assert rel_l2(got.grad.cpu().numpy(), want.grad.numpy()) < 1e-4
    if with_init:
        assert rel_l2(init.grad.cpu().numpy(), rs0.grad.numpy()) < 1e-4
