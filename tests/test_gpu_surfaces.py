"""GPU parity of the per-head, layer and pre-lifted surfaces (reference kernels/kernel_deltanet_fused.py,
layers/kernel_deltanet_layer.py, kernels/fused_triton_engine.py, kernels/tiled_triton_engine.py) against the
float64 oracle on the same inputs: oracle.lift.rff_features / rkhs_features for the features, then
oracle.scan.token_recurrence (delta rule) or linear_recurrence (the layer's rule without erasure).

Tolerances (relative L2): 1e-4 for fp32 inputs; 2e-2 for bf16 inputs or bf16 outputs (the oracle runs
on the bf16-rounded inputs; the residual is the bf16 rounding of the normalised inputs, the features
and Y inside the kernels).  The reference's own acceptance check between its prefill and step modes is
1e-5 (tests/test_parallel_vs_recurrent.py:80); here both modes run the same kernels and agree to 1e-5.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kdn import ops
from kernels import (FastWalshHadamardProjection, fused_triton_chunk_scan, streaming_triton_chunk_scan,
                     tiled_triton_chunk_scan)
from kernels.kernel_deltanet_fused import FusedKernelDeltaNet, FusedKernelDeltaNetFunction
from layers import KernelDeltaNetLayer
from oracle import lift as ol
from oracle import scan as osc

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 2e-2
DEV = "cuda:0"


@pytest.fixture(scope="module")
def proj():
    return FastWalshHadamardProjection(64, 512, 42)


@pytest.fixture(scope="module")
def oproj():
    return ol.make_projection(64, 512, 42)


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def per_head(rule, phi_q, phi_k, v, beta, decay, S0=None):
    """Run the oracle recurrence per (b, h) over (B, H, T, .) arrays; returns Y (B, H, T, d_v), S (B, H, d_v, D)."""
    fn = osc.token_recurrence if rule == "delta" else osc.linear_recurrence
    B, H = phi_q.shape[:2]
    Y = np.zeros(phi_q.shape[:3] + (v.shape[-1],))
    S = np.zeros((B, H, v.shape[-1], phi_k.shape[-1]))
    for h in range(H):
        s0 = None if S0 is None else S0[:, h]
        Y[:, h], S[:, h] = fn(phi_q[:, h], phi_k[:, h], v[:, h], beta[:, h], None if decay is None else decay[:, h], s0)
    return Y, S


def np64(t):
    return t.detach().to("cpu", torch.float64).numpy()


# ------------------------------------------------------------------------------------------------ P2


def _p2_inputs(dtype, B=2, H=2, T=150, seed=0):
    g = torch.Generator().manual_seed(seed)
    m = FusedKernelDeltaNet(64 * H, H)  # ORF Omega (H, 512, 64) and phases from the module's own init
    q = torch.randn(B, H, T, 64, generator=g).to(dtype)
    k = torch.randn(B, H, T, 64, generator=g).to(dtype)
    v = torch.randn(B, H, T, 64, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=g))
    decay = torch.sigmoid(torch.randn(B, H, T, generator=g) + 3.0)
    tau = F.softplus(torch.randn(H, 1, generator=g)) + 0.5
    return q, k, v, m.omega, m.b_rff, tau, beta, decay


@pytest.mark.parametrize("dtype,tol", [(torch.float32, TOL_F32), (torch.bfloat16, TOL_BF16)])
def test_p2_function_parity(dtype, tol):
    q, k, v, omega, b, tau, beta, decay = _p2_inputs(dtype)
    args = [t.to(DEV) for t in (q, k, v, omega, b, tau, beta, decay)]
    Y, S = FusedKernelDeltaNetFunction.apply(*args, 64)
    torch.cuda.synchronize()
    assert Y.dtype == dtype and S.dtype == dtype
    assert Y.shape == (2, 2, 150, 64) and S.shape == (2, 2, 64, 512)
    pq = ol.rff_features(np64(q), np64(omega), np64(b), np64(tau).reshape(-1), normalize=True)
    pk = ol.rff_features(np64(k), np64(omega), np64(b), np64(tau).reshape(-1), normalize=True)
    Yr, Sr = per_head("delta", pq, pk, np64(v), np64(beta), np64(decay))
    assert rel_l2(np64(Y), Yr) < tol
    assert rel_l2(np64(S), Sr) < tol


def test_p2_scalar_tau_and_no_decay_shapes():
    q, k, v, omega, b, _, beta, decay = _p2_inputs(torch.float32, B=1, H=2, T=64, seed=1)
    tau = torch.tensor(1.7)
    Y, S = FusedKernelDeltaNetFunction.apply(*[t.to(DEV) for t in (q, k, v, omega, b, tau, beta, decay)])
    pq = ol.rff_features(np64(q), np64(omega), np64(b), 1.7, normalize=True)
    pk = ol.rff_features(np64(k), np64(omega), np64(b), 1.7, normalize=True)
    Yr, Sr = per_head("delta", pq, pk, np64(v), np64(beta), np64(decay))
    assert rel_l2(np64(Y), Yr) < TOL_F32
    assert rel_l2(np64(S), Sr) < TOL_F32


def _p2_module_reference(m, x):
    """The module's forward in float64 on the CPU from the projections the module computed (the scan's
    inputs), through the oracle's features and recurrence."""
    B, T, _ = x.shape
    H, dh = m.num_heads, m.d_head
    W = {n: p.detach().cpu().double() for n, p in m.named_parameters()}

    def lin(layer):
        with torch.no_grad():
            return layer(x).detach().cpu().double()

    def heads(layer):
        return lin(layer).view(B, T, H, dh).transpose(1, 2).numpy()

    beta = torch.sigmoid(lin(m.w_beta)).transpose(1, 2).numpy()
    decay = torch.sigmoid(lin(m.w_decay)).transpose(1, 2).numpy()
    tau = (F.softplus(W["raw_tau"]) + 1e-4).numpy().reshape(-1)
    om, b = np64(m.omega), np64(m.b_rff)
    pq = ol.rff_features(heads(m.w_q), om, b, tau, normalize=True)
    pk = ol.rff_features(heads(m.w_k), om, b, tau, normalize=True)
    Y, S = per_head("delta", pq, pk, heads(m.w_v), beta, decay)
    out = torch.from_numpy(Y).transpose(1, 2).reshape(B, T, H * dh) @ W["w_out.weight"].T
    return out.numpy(), S


def test_p2_module_prefill_and_steps():
    torch.manual_seed(3)
    m = FusedKernelDeltaNet(128, 2).to(DEV)
    x = torch.randn(2, 130, 128, device=DEV) * 0.5
    with torch.no_grad():
        out, S = m(x)
    ref_out, ref_S = _p2_module_reference(m, x)
    assert rel_l2(np64(out), ref_out) < TOL_F32
    assert rel_l2(np64(S), ref_S) < TOL_F32
    # step mode: the first token alone (T == 1), then the rest from the returned state in two pieces
    with torch.no_grad():
        o1, s1 = m(x[:, :1])
        o2, s2 = m(x[:, 1:70], s1)
        o3, s3 = m(x[:, 70:], s2)
    steps = torch.cat([o1, o2, o3], dim=1)
    assert rel_l2(np64(steps), np64(out)) < 1e-5
    assert rel_l2(np64(s3), np64(S)) < 1e-5


# ------------------------------------------------------------------------------------------------ P4 layer


def _layer_reference(layer, x, state=None):
    """The layer's forward in float64 on the CPU from the projections the module computed (the scan's
    inputs), through the oracle's features and recurrence."""
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
    # lambda and eta as the module computes them (in its parameter dtype, as the reference's recurrent
    # step casts them, core/chunked_scan.py:175-176): the scan's inputs
    lam = np64(layer.get_decay()).reshape(H)
    eta = np64(layer.get_eta()).reshape(H)
    beta = np.broadcast_to(eta[None, :, None], (B, H, T))
    decay = np.broadcast_to(lam[None, :, None], (B, H, T))
    Y, S = per_head("linear", pq, pk, heads(layer.w_v, False), beta, decay,
                    None if state is None else np64(state))
    out = torch.from_numpy(Y).transpose(1, 2).reshape(B, T, H * dh) @ W["w_out.weight"].T
    return out.numpy(), S


def test_layer_prefill_parity_and_dual_mode():
    torch.manual_seed(4)
    layer = KernelDeltaNetLayer(128, 2, rkhs_factor=8).to(DEV)
    x = torch.randn(2, 140, 128, device=DEV)
    with torch.no_grad():
        out, none_state = layer(x)
    assert none_state is None
    ref_out, ref_S = _layer_reference(layer, x)
    assert rel_l2(np64(out), ref_out) < TOL_F32
    # step mode from a zero state returns the same outputs and the final state
    with torch.no_grad():
        zero = torch.zeros(2, 2, 64, 512, device=DEV)
        o_a, s_a = layer(x[:, :65], zero)
        o_b, s_b = layer(x[:, 65:], s_a)
    assert rel_l2(np64(torch.cat([o_a, o_b], 1)), np64(out)) < 1e-5
    assert rel_l2(np64(s_b), ref_S) < TOL_F32


def test_layer_steps_from_given_state():
    torch.manual_seed(5)
    layer = KernelDeltaNetLayer(128, 2, rkhs_factor=8, initial_decay=0.9, initial_eta=1.3).to(DEV)
    x = torch.randn(1, 9, 128, device=DEV)
    S0 = torch.randn(1, 2, 64, 512, device=DEV) * 0.1
    with torch.no_grad():
        out, S = layer(x, S0)
    ref_out, ref_S = _layer_reference(layer, x, S0)
    assert rel_l2(np64(out), ref_out) < TOL_F32
    assert rel_l2(np64(S), ref_S) < TOL_F32
    with torch.no_grad():
        o1, s1 = layer(x[:, :1])  # T == 1 without a state: one step from zero
    r1, rs1 = _layer_reference(layer, x[:, :1])
    assert rel_l2(np64(o1), r1) < TOL_F32 or np.linalg.norm(r1) == 0.0
    assert rel_l2(np64(s1), rs1) < TOL_F32


def test_layer_bf16():
    torch.manual_seed(6)
    layer = KernelDeltaNetLayer(128, 2, rkhs_factor=8).to(DEV).to(torch.bfloat16)
    x = torch.randn(1, 200, 128, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        out, _ = layer(x)
    ref_out, _ = _layer_reference(layer, x)
    assert out.dtype == torch.bfloat16
    assert rel_l2(np64(out), ref_out) < TOL_BF16


def test_forward_only_surfaces_raise_on_backward():
    # the pre-lifted (Triton-named) surfaces have no backward: a training step fails loudly instead of
    # skipping the scan's gradient (the layer and the P2 surfaces differentiate: test_gpu_feature_backward)
    g = torch.Generator().manual_seed(9)
    phi = F.normalize(torch.randn(1, 2, 64, 512, generator=g), dim=-1).to(DEV).requires_grad_(True)
    v = torch.randn(1, 2, 64, 64, generator=g).to(DEV)
    beta, decay = torch.full((1, 2, 64), 0.5, device=DEV), torch.full((1, 2, 64), 0.99, device=DEV)
    y = fused_triton_chunk_scan(phi, phi, v, beta, decay)
    with pytest.raises(NotImplementedError):
        y.float().sum().backward()


# ------------------------------------------------------------------------------------------------ linear rule


def test_linear_rule_structured_features(proj, oproj):
    g = torch.Generator().manual_seed(7)
    B, T, H = 1, 333, 2
    q, k = torch.randn(B, T, H, 64, generator=g), torch.randn(B, T, H, 64, generator=g)
    v = torch.randn(B, T, H, 64, generator=g)
    beta = torch.rand(B, T, H, generator=g) * 1.5
    decay = 0.9 + 0.1 * torch.rand(B, T, H, generator=g)
    y, S = ops.scan(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), decay.to(DEV), proj.device_omega(DEV),
                    proj.device_phase(DEV), proj.tau_star_inv, rule=ops.RULE_LINEAR)
    for h in range(H):
        Yr, Sr = osc.linear_recurrence(ol.lift(q[:, :, h].numpy(), oproj), ol.lift(k[:, :, h].numpy(), oproj),
                                       v[:, :, h].numpy(), beta[:, :, h].numpy(), decay[:, :, h].numpy())
        assert rel_l2(np64(y[:, :, h]), Yr) < TOL_F32
        assert rel_l2(np64(S[:, h].transpose(1, 2)), Sr) < TOL_F32


# ------------------------------------------------------------------------------------------------ pre-lifted


def _lifted_inputs(T, seed=8, B=1, H=2):
    rng = np.random.default_rng(seed)
    proj = ol.make_projection(64, 512, 42)
    fq = ol.lift(rng.standard_normal((B * H * T, 64)), proj).reshape(B, H, T, 512)
    fk = ol.lift(rng.standard_normal((B * H * T, 64)), proj).reshape(B, H, T, 512)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    q, k = to(fq), to(fk)
    v = to(rng.standard_normal((B, H, T, 64)))
    beta = to(1.0 / (1.0 + np.exp(-rng.standard_normal((B, H, T)))))
    decay = to(1.0 / (1.0 + np.exp(-rng.standard_normal((B, H, T)) - 3.0)))
    return q, k, v, beta, decay


@pytest.mark.parametrize("fn", [fused_triton_chunk_scan, tiled_triton_chunk_scan, streaming_triton_chunk_scan])
def test_prelifted_surfaces(fn):
    q, k, v, beta, decay = _lifted_inputs(192)
    y = fn(*(t.to(DEV) for t in (q, k, v, beta, decay)), chunk_size=64)
    assert y.dtype == torch.bfloat16 and y.shape == (1, 2, 192, 64)
    Yr, _ = per_head("delta", np64(q), np64(k), np64(v), np64(beta), np64(decay))
    assert rel_l2(np64(y), Yr) < TOL_BF16


def test_prelifted_fp32_and_ragged():
    q, k, v, beta, decay = _lifted_inputs(100, seed=9)
    y = streaming_triton_chunk_scan(*(t.float().to(DEV) for t in (q, k, v, beta, decay)))
    Yr, _ = per_head("delta", np64(q), np64(k), np64(v), np64(beta), np64(decay))
    # fp32 arithmetic throughout; only the bf16 output rounding remains
    assert rel_l2(np64(y), Yr) < 4e-3
