"""GPU parity of the chunked delta-rule scan (kdn_delta_scan_fwd) against the CPU oracle.

Tolerances (relative L2 over the whole tensor): 1e-4 for fp32 inputs, 2e-2 for bf16 inputs with the
fp32 state; the bf16 oracle runs in float64 on the bf16-rounded inputs."""
import numpy as np
import pytest
import torch

from kdn import ops
from kernels import FastWalshHadamardProjection, fused_chunked_deltanet_forward
from oracle import lift as ol
from oracle import scan as osc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL_F32 = 1e-4
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


def make_inputs(B, T, H, dv, dtype, decay_kind="none", seed=1234):
    """q, k, v ~ N(0,1), beta = sigmoid(N(0,1)) in (B, T, H, .) layout from one seeded CPU generator."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g)
    k = torch.randn(B, T, H, 64, generator=g)
    v = torch.randn(B, T, H, dv, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    if decay_kind == "none":
        decay = None
    elif decay_kind == "sigmoid":
        decay = torch.sigmoid(torch.randn(B, T, H, generator=g))
    else:
        decay = 0.94 + 0.05 * torch.rand(B, T, H, generator=g)
    return q.to(dtype), k.to(dtype), v.to(dtype), beta, decay


def oracle_bthd(q, k, v, beta, decay, oproj, S0=None, normalize=False):
    """Float64 oracle over (B, T, H, .) inputs; returns y (B, T, H, dv) and S (B, H, D, dv)."""
    B, T, H, _ = q.shape
    dv = v.shape[-1]
    # The chunked float64 restatement equals the token recurrence to 1e-12 (tests/test_oracle_scan.py)
    # and is much faster at these lengths.
    f = lambda t: t.float().permute(0, 2, 1, 3).reshape(B * H, T, -1).double()
    fb = lambda t: None if t is None else t.float().permute(0, 2, 1).reshape(B * H, T).double()
    s0 = None if S0 is None else S0.float().reshape(B * H, 512, dv).transpose(1, 2).double()
    y, S = osc.chunked_forward(f(q), f(k), f(v), fb(beta), fb(decay), oproj, 64, s0, torch.float64, normalize)
    y, S = y.numpy(), S.numpy()
    return (y.reshape(B, H, T, dv).transpose(0, 2, 1, 3), S.reshape(B, H, dv, 512).transpose(0, 1, 3, 2))


def run(proj, q, k, v, beta, decay, **kw):
    d = lambda t: None if t is None else t.to(DEV)
    return ops.scan(d(q), d(k), d(v), d(beta), d(decay), proj.device_omega(DEV), proj.device_phase(DEV),
                    proj.tau_star_inv, **kw)


@pytest.mark.parametrize("decay_kind", ["none", "sigmoid", "narrow"])
def test_config1_fp32(proj, oproj, decay_kind):
    """B=1, H=4, T=1024, d_k=64 -> D=512, d_v=64, fp32."""
    q, k, v, beta, decay = make_inputs(1, 1024, 4, 64, torch.float32, decay_kind)
    y, S = run(proj, q, k, v, beta, decay)
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_F32


def test_reference_test_shape_surface(proj, oproj):
    """Shape of the reference's own precision test (tests/test_fused_kernel.py:76): B=2, T=32, d_v=128,
    C=32, fp32, sigmoid decay, through fused_chunked_deltanet_forward."""
    g = torch.Generator().manual_seed(42)
    B, T, dv = 2, 32, 128
    q, k, v = torch.randn(B, T, 64, generator=g), torch.randn(B, T, 64, generator=g), torch.randn(B, T, dv, generator=g)
    beta, decay = torch.sigmoid(torch.randn(B, T, generator=g)), torch.sigmoid(torch.randn(B, T, generator=g))
    y, S = fused_chunked_deltanet_forward(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), decay.to(DEV),
                                          proj.to(DEV), chunk_size=32)
    yr, Sr = osc.delta_rule(q.numpy(), k.numpy(), v.numpy(), beta.numpy(), decay.numpy(), oproj)
    assert y.shape == (B, T, dv) and S.shape == (B, dv, 512)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_F32


@pytest.mark.parametrize("decay_kind", ["none", "sigmoid"])
def test_bf16_16_heads(proj, oproj, decay_kind):
    """bf16 q/k/v, fp32 beta and state, H=16 (the headline layer), T=2048."""
    q, k, v, beta, decay = make_inputs(1, 2048, 16, 64, torch.bfloat16, decay_kind)
    y, S = run(proj, q, k, v, beta, decay)
    assert y.dtype == torch.bfloat16
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj)
    assert rel_l2(y.float().cpu().numpy(), yr) < TOL_BF16
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_BF16


@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 100, 130])
def test_ragged_lengths(proj, oproj, T):
    q, k, v, beta, decay = make_inputs(2, T, 3, 32, torch.float32, "narrow", seed=T)
    y, S = run(proj, q, k, v, beta, decay)
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_F32


@pytest.mark.parametrize("dv", [16, 32, 128])
def test_value_widths(proj, oproj, dv):
    q, k, v, beta, decay = make_inputs(1, 200, 2, dv, torch.float32, "sigmoid", seed=dv)
    y, S = run(proj, q, k, v, beta, decay)
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_F32


def test_initial_state_and_continuation(proj, oproj):
    q, k, v, beta, decay = make_inputs(1, 300, 2, 64, torch.float32, "narrow", seed=5)
    g = torch.Generator().manual_seed(9)
    S0 = 0.1 * torch.randn(1, 2, 512, 64, generator=g)
    y, S = run(proj, q, k, v, beta, decay, initial_state=S0.to(DEV))
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj, S0)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_F32
    # prefill in two pieces (split inside a chunk) == one prefill
    cut = 130
    y1, S1 = run(proj, q[:, :cut], k[:, :cut], v[:, :cut], beta[:, :cut], decay[:, :cut], initial_state=S0.to(DEV))
    y2, S2 = run(proj, q[:, cut:], k[:, cut:], v[:, cut:], beta[:, cut:], decay[:, cut:], initial_state=S1)
    assert rel_l2(torch.cat([y1, y2], 1).cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S2.cpu().numpy(), Sr) < TOL_F32


def test_normalize_input(proj, oproj):
    q, k, v, beta, decay = make_inputs(1, 256, 2, 64, torch.float32, "sigmoid", seed=11)
    y, S = run(proj, q, k, v, beta, decay, normalize=True)
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj, normalize=True)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_F32


def test_segments_and_determinism(proj):
    q, k, v, beta, decay = make_inputs(1, 1000, 4, 64, torch.bfloat16, "sigmoid", seed=3)
    y0, S0 = run(proj, q, k, v, beta, decay)
    y1, S1 = run(proj, q, k, v, beta, decay, segment_chunks=1)
    y2, S2 = run(proj, q, k, v, beta, decay, segment_chunks=5)
    y3, S3 = run(proj, q, k, v, beta, decay)
    for yy, SS in ((y1, S1), (y2, S2), (y3, S3)):
        assert torch.equal(yy, y0) and torch.equal(SS, S0)


def test_layouts_agree(proj):
    """(B, T, H, d), (B, H, T, d) strided views and the reference (B*H, T, d) surface give identical bits."""
    B, T, H, dv = 2, 256, 3, 64
    q, k, v, beta, decay = make_inputs(B, T, H, dv, torch.bfloat16, "sigmoid", seed=21)
    y0, S0 = run(proj, q, k, v, beta, decay)
    # (B, H, T, d) storage viewed as (B, T, H, d)
    tr = lambda t: t.transpose(1, 2).contiguous().transpose(1, 2)
    y1, S1 = run(proj, tr(q), tr(k), tr(v), beta.transpose(1, 2).contiguous().transpose(1, 2),
                 decay.transpose(1, 2).contiguous().transpose(1, 2))
    assert torch.equal(y1, y0) and torch.equal(S1, S0)
    fold = lambda t: t.permute(0, 2, 1, 3).reshape(B * H, T, -1)
    foldb = lambda t: t.permute(0, 2, 1).reshape(B * H, T)
    y2, S2 = fused_chunked_deltanet_forward(fold(q).to(DEV), fold(k).to(DEV), fold(v).to(DEV), foldb(beta).to(DEV),
                                            foldb(decay).to(DEV), proj.to(DEV))
    assert torch.equal(y2.view(B, H, T, dv).permute(0, 2, 1, 3).cpu(), y0.cpu())
    assert S2.dtype == torch.bfloat16  # the reference returns S in the input dtype
    assert torch.equal(S2.view(B, H, dv, 512).transpose(2, 3).cpu(), S0.to(torch.bfloat16).cpu())


def test_config3_full_length(proj, oproj):
    """BASELINE config 3 shape: B=1, H=16, T=65536, bf16.  Checks: all finite; the first 2048 tokens of all
    heads and the whole sequence of two heads against the oracle (chunked fp64 CPU restatement); the
    prefill split in two halves equals the single call."""
    B, T, H, dv = 1, 65536, 16, 64
    q, k, v, beta, decay = make_inputs(B, T, H, dv, torch.bfloat16, "none", seed=1234)
    y, S = run(proj, q, k, v, beta, decay)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(S).all()
    n0 = 2048
    yr0, _ = oracle_bthd(q[:, :n0], k[:, :n0], v[:, :n0], beta[:, :n0], None, oproj)
    assert rel_l2(y[:, :n0].float().cpu().numpy(), yr0) < TOL_BF16
    for h in (0, 11):
        f = lambda t: t[:, :, h].float()
        yh, Sh = osc.chunked_forward(f(q), f(k), f(v), beta[:, :, h], None, oproj, 64, None, torch.float64)
        assert rel_l2(y[:, :, h].float().cpu().numpy(), yh.numpy()) < TOL_BF16
        assert rel_l2(S[:, h].transpose(1, 2).cpu().numpy(), Sh.numpy()) < TOL_BF16
    half = T // 2
    ya, Sa = run(proj, q[:, :half], k[:, :half], v[:, :half], beta[:, :half], None)
    yb, Sb = run(proj, q[:, half:], k[:, half:], v[:, half:], beta[:, half:], None, initial_state=Sa)
    assert torch.equal(torch.cat([ya, yb], 1), y)
    assert torch.equal(Sb, S)


@pytest.mark.parametrize("seg,decay_kind", [(4, "none"), (16, "sigmoid"), (7, "narrow")])
def test_pipelined_equals_serial(proj, seg, decay_kind):
    """kdn_delta_scan_fwd_streams (prep and output on two auxiliary streams, segments rotating through up
    to three workspace buffers) runs the same kernels as the serial schedule: results are bit-identical."""
    q, k, v, beta, decay = make_inputs(1, 64 * 40 + 17, 3, 64, torch.bfloat16, decay_kind, seed=seg)
    S0 = 0.1 * torch.randn(1, 3, 512, 64, generator=torch.Generator().manual_seed(7))
    y1, S1 = run(proj, q, k, v, beta, decay, initial_state=S0, segment_chunks=seg, pipelined=True)
    y2, S2 = run(proj, q, k, v, beta, decay, initial_state=S0, segment_chunks=seg, pipelined=False)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(S1, S2)


def test_pipelined_without_spare_cus_equals_serial(proj):
    # 4 sequences x 16 heads x 4 value tiles fill every CU with state workgroups: the pipelined schedule
    # then keeps q's lifted features in the workspace (prep stores them, the output kernel reads them);
    # with one sequence (above) the output kernel lifts q again.  Both equal the serial schedule bit for bit.
    q, k, v, beta, decay = make_inputs(4, 64 * 6 + 9, 16, 64, torch.bfloat16, "sigmoid", seed=3)
    y1, S1 = run(proj, q, k, v, beta, decay, segment_chunks=2, pipelined=True)
    y2, S2 = run(proj, q, k, v, beta, decay, segment_chunks=2, pipelined=False)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(S1, S2)


def test_two_stream_pipeline_equals_serial(proj):
    """kdn_delta_scan_fwd_pipelined (prep and output sharing one auxiliary stream) is bit-identical too."""
    import ctypes
    from kdn import _native as N
    q, k, v, beta, decay = make_inputs(1, 64 * 23 + 9, 2, 64, torch.bfloat16, "sigmoid", seed=21)
    qd, kd, vd, bd, dd = (t.to(DEV) for t in (q, k, v, beta, decay))
    om, ph = proj.device_omega(DEV), proj.device_phase(DEV)
    ws = torch.empty(ops.scan_workspace_bytes(qd, vd, om, 5, pipelined=True), dtype=torch.uint8, device=DEV)
    y = torch.empty(1, qd.shape[1], 2, 64, device=DEV, dtype=torch.bfloat16)
    S = torch.empty(1, 2, 512, 64, device=DEV)
    a = ops.scan_args(qd, kd, vd, bd, dd, om, ph, proj.tau_star_inv, False, None, S, y, ws, 5)
    aux = torch.cuda.Stream()
    st = torch.cuda.current_stream()
    N.check(N.lib().kdn_delta_scan_fwd_pipelined(ctypes.byref(a), ctypes.c_void_p(st.cuda_stream),
                                                 ctypes.c_void_p(aux.cuda_stream)), "pipelined")
    y2, S2 = ops.scan(qd, kd, vd, bd, dd, om, ph, proj.tau_star_inv, segment_chunks=5, pipelined=False)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    assert torch.equal(S, S2)


def test_pipelined_two_buffers_parity(proj, oproj):
    """Workspace for two segment buffers only; checked against the float64 oracle."""
    q, k, v, beta, decay = make_inputs(2, 64 * 12 + 5, 2, 32, torch.float32, "sigmoid", seed=11)
    qd, kd, vd, bd, dd = (t.to(DEV) for t in (q, k, v, beta, decay))
    om, ph = proj.device_omega(DEV), proj.device_phase(DEV)
    one = ops.scan_workspace_bytes(qd, vd, om, 3, pipelined=False)
    ws = torch.empty(2 * one, dtype=torch.uint8, device=DEV)
    y, S = ops.scan(qd, kd, vd, bd, dd, om, ph, proj.tau_star_inv, workspace=ws, segment_chunks=3, pipelined=True)
    yr, Sr = oracle_bthd(q, k, v, beta, decay, oproj)
    assert rel_l2(y.cpu().numpy(), yr) < TOL_F32
    assert rel_l2(S.cpu().numpy(), Sr) < TOL_F32
