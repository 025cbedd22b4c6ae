"""Host-side logic of the reference-named surfaces (no GPU): projection tables equal the oracle's,
device-only enforcement (no CPU fallback), argument checking."""
import numpy as np
import pytest
import torch

from kernels import FastWalshHadamardProjection, FusedKernelDeltaNet, fused_chunked_deltanet_forward
from oracle import lift as ol


def test_projection_buffers_match_oracle():
    p = FastWalshHadamardProjection(64, 512, 42)
    o = ol.make_projection(64, 512, 42)
    np.testing.assert_array_equal(p.d1.numpy(), o["d1"])
    np.testing.assert_array_equal(p.d2.numpy(), o["d2"])
    np.testing.assert_array_equal(p.d3.numpy(), o["d3"])
    np.testing.assert_array_equal(p.rademacher_bits.numpy(), o["bits"])
    np.testing.assert_array_equal(p.b.numpy(), o["b"])
    np.testing.assert_array_equal(p.Omega.numpy(), o["omega"].astype(np.float32))
    assert p.tau_star == pytest.approx(64 ** 0.25)
    names = dict(p.named_buffers())
    assert set(names) == {"d1", "d2", "d3", "rademacher_bits", "b", "Omega"}
    assert "rademacher_bits" not in p.state_dict()


@pytest.mark.parametrize("seed", [0, 7, 1042])
def test_other_seeds_and_sizes(seed):
    for D in (128, 256, 512):
        p = FastWalshHadamardProjection(64, D, seed)
        o = ol.make_projection(64, D, seed)
        np.testing.assert_array_equal(p.rademacher_bits.numpy(), o["bits"])
        np.testing.assert_array_equal(p.Omega.numpy(), o["omega"].astype(np.float32))


def test_no_cpu_fallback_lift():
    p = FastWalshHadamardProjection()
    with pytest.raises(RuntimeError, match="device tensors only"):
        p(torch.randn(3, 64))


def test_no_cpu_fallback_scan():
    p = FastWalshHadamardProjection()
    B, T = 1, 8
    q = torch.randn(B, T, 64)
    with pytest.raises(RuntimeError, match="device tensors only"):
        fused_chunked_deltanet_forward(q, q, torch.randn(B, T, 64), torch.rand(B, T), torch.rand(B, T), p)


def test_scan_argument_checks():
    p = FastWalshHadamardProjection()
    q = torch.randn(1, 8, 64)
    with pytest.raises(ValueError):
        fused_chunked_deltanet_forward(q, q, torch.randn(1, 8, 64), torch.rand(1, 8), torch.rand(1, 8), p, chunk_size=0)
    with pytest.raises(ValueError):
        fused_chunked_deltanet_forward(q, q, torch.randn(1, 8, 64), torch.rand(1, 9), torch.rand(1, 8), p)


def test_host_slot_checks():
    """Slots known on the host are checked before anything is launched: in range of the slab, one
    sequence per slot; negative slots are padding (skipped on the device)."""
    from kdn import ops
    from serving.vllm_kernel_deltanet_op import sequences_from_slot_mapping

    ops.check_host_slots([0, 3, -1, 5, -1], 6)
    with pytest.raises(ValueError, match="outside"):
        ops.check_host_slots([0, 6], 6)
    with pytest.raises(ValueError, match="share"):
        ops.check_host_slots(torch.tensor([2, 1, 2], dtype=torch.int32), 6)
    cu, slots = sequences_from_slot_mapping(torch.tensor([4, 4, 4, 1, -1, -1, 0, 0]), 5)
    assert cu.tolist() == [0, 3, 4, 6, 8] and slots.tolist() == [4, 1, -1, 0]
    with pytest.raises(ValueError, match="two separate runs"):
        sequences_from_slot_mapping(torch.tensor([1, 1, 2, 1]), 5)
    with pytest.raises(ValueError, match="outside"):
        sequences_from_slot_mapping(torch.tensor([1, 1, 7]), 5)


def test_module_surface():
    m = FusedKernelDeltaNet(d_model=64, d_kernel=512, chunk_size=64)
    assert m.fwht_proj.D == 512 and m.chunk_size == 64


def test_feature_map_argument_fill():
    # kdn_scan_args fields for per-head hi + lo Omega, shared phases, per-head 1/tau and the linear rule
    from kdn import ops
    B, T, H = 1, 70, 3
    q = torch.zeros(B, T, H, 64)
    v = torch.zeros(B, T, H, 64)
    beta = torch.zeros(B, T, H)
    hi = torch.zeros(H, 512, 64, dtype=torch.bfloat16)
    fm = ops.FeatureMap(omega=hi, phase=torch.zeros(512), omega_lo=hi.clone(), inv_tau_head=torch.ones(H),
                        no_renorm=True)
    y = torch.zeros(B, T, H, 64)
    fin = torch.zeros(B, H, 512, 64)
    a = ops.scan_args(q, q, v, beta, None, None, None, 1.0, True, None, fin, y, features=fm, rule=ops.RULE_LINEAR)
    assert (a.D, a.d_k, a.feature_mode, a.no_renorm, a.rule) == (512, 64, 0, 1, 1)
    assert a.omega_head_stride == 512 * 64 and a.phase_head_stride == 0
    assert a.omega_lo == fm.omega_lo.data_ptr() and a.inv_tau_head == fm.inv_tau_head.data_ptr()
    # pre-lifted features: d_k = D, no Omega
    ql = torch.zeros(B, T, H, 512)
    a = ops.scan_args(ql, ql, v, beta, None, None, None, 1.0, False, None, fin, y,
                      features=ops.FeatureMap(lifted=True))
    assert (a.D, a.d_k, a.feature_mode, a.rule) == (512, 512, 1, 0)
    assert not a.omega_bf16 and not a.phase and not a.omega_lo
    assert ops.scan_workspace_bytes(ql, v, None, 0, False, ops.FeatureMap(lifted=True)) > 0
    assert ops.scan_workspace_bytes(q, v, None, 0, False, ops.FeatureMap(lifted=True)) == 0  # d_k != D


def test_surface_argument_checks_on_host():
    from kernels import fused_triton_chunk_scan, tiled_triton_chunk_scan
    from layers import KernelDeltaNetLayer
    x = torch.zeros(1, 2, 100, 512)
    with pytest.raises(AssertionError):
        fused_triton_chunk_scan(x, x, torch.zeros(1, 2, 100, 64), torch.zeros(1, 2, 100), torch.zeros(1, 2, 100))
    with pytest.raises(AssertionError):
        tiled_triton_chunk_scan(x, x, torch.zeros(1, 2, 100, 64), torch.zeros(1, 2, 100), torch.zeros(1, 2, 100),
                                block_d=48)
    layer = KernelDeltaNetLayer(64, 4)  # reference default rkhs_factor = 4: d_head 16, rkhs_dim 64
    with pytest.raises(ValueError, match="d_head = 64 and rkhs_dim 128, 256 or 512"):
        layer(torch.zeros(1, 8, 64))
    sd = KernelDeltaNetLayer(128, 2, rkhs_factor=8).state_dict()
    assert set(sd) == {"w_q.weight", "w_k.weight", "w_v.weight", "w_out.weight", "kernel.log_gamma",
                       "kernel.omega", "logit_decay", "raw_eta"}
    assert sd["kernel.omega"].shape == (2, 256, 64) and sd["logit_decay"].shape == (1, 2, 1, 1)


def test_forward_only_guard_on_host():
    from kdn import ops
    a = torch.ones(3)
    w = torch.ones(3, requires_grad=True)
    (out,) = ops.forward_only("probe", (a,), (w,))
    assert out.requires_grad
    with pytest.raises(NotImplementedError, match="probe"):
        (out * w).sum().backward()
    with torch.no_grad():
        (plain,) = ops.forward_only("probe", (a,), (w,))
    assert plain is a
