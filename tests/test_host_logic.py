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


def test_module_surface():
    m = FusedKernelDeltaNet(d_model=64, d_kernel=512, chunk_size=64)
    assert m.fwht_proj.D == 512 and m.chunk_size == 64
