"""GPU parity of the fused schedule (prep + the fused chain of kdn_chain.hip, no output kernel), forced with
KDN_SCAN_SCHEDULE=fused whatever the head count (by default it runs only when the split schedule's state
workgroups would fill the GPU).

Checks: against the float64 oracle (relative L2 2e-2 for bf16 inputs, as every bf16 scan test); against
the split schedule, whose state kernel forms the same products in the same order, so the final state is
bit-identical and y differs only by the summation order of Q S^T over the four feature quarters (fp32,
then rounded to bf16: relative L2 below 5e-3); pipelined = serial and segment lengths bit for bit; a
prefill in two calls equal to one; the ragged serving step against its oracle.
"""
import numpy as np
import pytest
import torch

from kdn import ops
from kernels import FastWalshHadamardProjection
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


def make_inputs(B, T, H, dv, decay_kind="none", seed=1234):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(B, T, H, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, H, dv, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    if decay_kind == "none":
        decay = None
    elif decay_kind == "sigmoid":
        decay = torch.sigmoid(torch.randn(B, T, H, generator=g))
    else:
        decay = 0.94 + 0.05 * torch.rand(B, T, H, generator=g)
    return q, k, v, beta, decay


def oracle_bthd(q, k, v, beta, decay, oproj, S0=None):
    B, T, H, _ = q.shape
    dv = v.shape[-1]
    f = lambda t: t.float().permute(0, 2, 1, 3).reshape(B * H, T, -1).double()
    fb = lambda t: None if t is None else t.float().permute(0, 2, 1).reshape(B * H, T).double()
    s0 = None if S0 is None else S0.float().reshape(B * H, 512, dv).transpose(1, 2).double()
    y, S = osc.chunked_forward(f(q), f(k), f(v), fb(beta), fb(decay), oproj, 64, s0, torch.float64)
    return (y.numpy().reshape(B, H, T, dv).transpose(0, 2, 1, 3), S.numpy().reshape(B, H, dv, 512).transpose(0, 1, 3, 2))


def run(proj, schedule, monkeypatch, q, k, v, beta, decay, **kw):
    monkeypatch.setenv("KDN_SCAN_SCHEDULE", schedule)
    d = lambda t: None if t is None else t.to(DEV)
    y, S = ops.scan(d(q), d(k), d(v), d(beta), d(decay), proj.device_omega(DEV), proj.device_phase(DEV),
                    proj.tau_star_inv, **kw)
    torch.cuda.synchronize()
    return y, S


@pytest.mark.parametrize("dv,decay_kind", [(64, "none"), (64, "sigmoid"), (16, "narrow"), (32, "sigmoid"),
                                           (128, "none")])
def test_fused_matches_oracle_and_split(proj, oproj, monkeypatch, dv, decay_kind):
    B, T, H = 2, 64 * 5 + 17, 3
    q, k, v, beta, decay = make_inputs(B, T, H, dv, decay_kind, seed=dv)
    S0 = 0.05 * torch.randn(B, H, 512, dv, generator=torch.Generator().manual_seed(5))
    yf, Sf = run(proj, "fused", monkeypatch, q, k, v, beta, decay, initial_state=S0, segment_chunks=2)
    ys, Ss = run(proj, "split", monkeypatch, q, k, v, beta, decay, initial_state=S0, segment_chunks=2)
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj, S0)
    assert rel_l2(yf.float().cpu().numpy(), yr) < TOL_BF16
    assert rel_l2(Sf.cpu().numpy(), Sr) < TOL_BF16
    assert torch.equal(Sf, Ss)
    assert rel_l2(yf.float().cpu().numpy(), ys.float().cpu().numpy()) < 5e-3


@pytest.mark.parametrize("seg,decay_kind", [(4, "none"), (7, "sigmoid")])
def test_fused_pipelined_equals_serial(proj, monkeypatch, seg, decay_kind):
    q, k, v, beta, decay = make_inputs(1, 64 * 40 + 17, 3, 64, decay_kind, seed=seg)
    y1, S1 = run(proj, "fused", monkeypatch, q, k, v, beta, decay, segment_chunks=seg, pipelined=True)
    y2, S2 = run(proj, "fused", monkeypatch, q, k, v, beta, decay, segment_chunks=seg, pipelined=False)
    y3, S3 = run(proj, "fused", monkeypatch, q, k, v, beta, decay, segment_chunks=1, pipelined=False)
    assert torch.equal(y1, y2) and torch.equal(S1, S2)
    assert torch.equal(y1, y3) and torch.equal(S1, S3)


def test_fused_two_calls_equal_one(proj, oproj, monkeypatch):
    B, T, H = 2, 64 * 9, 4
    q, k, v, beta, decay = make_inputs(B, T, H, 64, "sigmoid", seed=9)
    y, S = run(proj, "fused", monkeypatch, q, k, v, beta, decay)
    cut = 64 * 4  # a chunk boundary: the two calls then run the same chunks as one
    ya, Sa = run(proj, "fused", monkeypatch, q[:, :cut], k[:, :cut], v[:, :cut], beta[:, :cut], decay[:, :cut])
    yb, Sb = run(proj, "fused", monkeypatch, q[:, cut:], k[:, cut:], v[:, cut:], beta[:, cut:], decay[:, cut:],
                 initial_state=Sa)
    assert torch.equal(torch.cat([ya, yb], 1), y) and torch.equal(Sb, S)
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj)
    assert rel_l2(y.float().cpu().numpy(), yr) < TOL_BF16


def test_fused_fp32_out(proj, oproj, monkeypatch):
    """bf16 inputs with an fp32 y (out_dtype): the chain stores rows of fp32."""
    q, k, v, beta, decay = make_inputs(1, 200, 2, 64, "sigmoid", seed=4)
    y, S = run(proj, "fused", monkeypatch, q, k, v, beta, decay, out_dtype=torch.float32)
    assert y.dtype == torch.float32
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_BF16


def test_fused_serving_step(proj, oproj, monkeypatch):
    """The ragged mixed step (decode sequences, prefills of several lengths, an empty sequence) with its
    prefill on the fused chain: every sequence against the float64 token recurrence from its slot state,
    untouched slots bit-identical."""
    monkeypatch.setenv("KDN_SCAN_SCHEDULE", "fused")
    lens = [1, 37, 0, 200, 1, 64, 130]
    H, dv, n_slots = 2, 64, 12
    g = torch.Generator().manual_seed(3)
    T = int(sum(lens))
    q = torch.randn(T, H, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(T, H, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(T, H, dv, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(T, H, generator=g))
    lam = 0.9 + 0.1 * torch.rand(T, H, generator=g)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int64)
    slots = torch.randperm(n_slots, generator=g)[: len(lens)].to(torch.int32)
    states = 0.05 * torch.randn(n_slots, H, 512, dv, generator=g)
    sd = states.to(DEV)
    y = ops.ragged_step(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), cu, slots, sd,
                        proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv)
    torch.cuda.synchronize()
    y, S = y.float().cpu().numpy(), sd.cpu()
    used = set(int(s) for s in slots)
    for s in range(n_slots):
        if s not in used:
            assert torch.equal(S[s], states[s]), s
    for i, ln in enumerate(lens):
        lo, hi, s = int(cu[i]), int(cu[i + 1]), int(slots[i])
        if hi == lo:
            assert torch.equal(S[s], states[s])
            continue
        for h in range(H):
            pq = ol.lift(q[lo:hi, h].float().numpy(), oproj)
            pk = ol.lift(k[lo:hi, h].float().numpy(), oproj)
            yr, Sr = osc.token_recurrence(pq[None], pk[None], v[lo:hi, h].double().numpy()[None],
                                          beta[lo:hi, h].double().numpy()[None], lam[lo:hi, h].double().numpy()[None],
                                          states[s, h].double().numpy().T[None])
            assert rel_l2(y[lo:hi, h], yr[0]) < TOL_BF16, (i, h)
            assert rel_l2(S[s, h].numpy(), Sr[0].T) < TOL_BF16, (i, h)
