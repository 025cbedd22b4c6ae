"""GPU parity of the lift kernels (kdn_build_omega, kdn_fwht, kdn_fwht_lift) against the CPU oracle."""
import numpy as np
import pytest
import torch

import ctypes

from kdn import _native as N
from kdn import ops
from kernels import FastWalshHadamardProjection, fast_walsh_hadamard_transform
from oracle import lift as ol

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.fixture(scope="module")
def proj():
    return FastWalshHadamardProjection(64, 512, 42)


@pytest.fixture(scope="module")
def oproj():
    return ol.make_projection(64, 512, 42)


@pytest.mark.parametrize("D", [128, 256, 512, 1024])
@pytest.mark.parametrize("seed", [42, 3])
def test_build_omega_bit_exact(D, seed):
    o = ol.make_projection(64, D, seed)
    bits = torch.tensor(o["bits"])
    for dt in (torch.float32, torch.bfloat16):
        om = ops.build_omega(bits, 64, D, DEV, dt).float().cpu().numpy()
        np.testing.assert_array_equal(om, o["omega"].astype(np.float32))


@pytest.mark.parametrize("n", [1, 2, 4, 8, 16, 32, 64])
def test_fwht_rows(n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(37, n, generator=g)
    ref = ol.fwht_rows(x.numpy())
    out = fast_walsh_hadamard_transform(x.to(DEV)).cpu().numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    xb = x.to(torch.bfloat16)
    outb = fast_walsh_hadamard_transform(xb.to(DEV)).float().cpu().numpy()
    refb = ol.fwht_rows(xb.float().numpy())
    assert rel_l2(outb, refb) < 1e-2


@pytest.mark.parametrize("rows", [1, 15, 16, 17, 1000, 4099])
@pytest.mark.parametrize("normalize", [False, True])
def test_lift_fp32(proj, oproj, rows, normalize):
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, 64, generator=g) * 1.5
    out = ops.lift(x.to(DEV), proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv, normalize)
    ref = ol.lift(x.numpy(), oproj, normalize)
    assert out.dtype == torch.float32 and out.shape == (rows, 512)
    assert rel_l2(out.cpu().numpy(), ref) < 1e-5
    assert np.abs(out.cpu().numpy() - ref).max() < 2e-5


def test_lift_module_forward_shapes(proj, oproj):
    x = torch.randn(2, 3, 5, 64)
    out = proj.to(DEV)(x.to(DEV))
    assert out.shape == (2, 3, 5, 512)
    ref = ol.lift(x.numpy().reshape(-1, 64), oproj).reshape(2, 3, 5, 512)
    assert rel_l2(out.cpu().numpy(), ref) < 1e-5


def test_lift_strided_rows(proj, oproj):
    big = torch.randn(50, 128)
    x = big[:, 32:96]  # row stride 128, 16-byte aligned start
    out = ops.lift(x.to(DEV), proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv)
    assert rel_l2(out.cpu().numpy(), ol.lift(x.numpy(), oproj)) < 1e-5


@pytest.mark.parametrize("D", [128, 256, 512])
def test_lift_padded_output_rows_and_ragged_tile(proj, D):
    # output rows wider than D (the kernel writes only the first D of each) and a row count that
    # leaves the last 16-row tile partial
    from kernels import FastWalshHadamardProjection
    p = FastWalshHadamardProjection(64, D, 42)
    op = ol.make_projection(64, D, 42)
    x = torch.randn(37, 64)
    om, ph = p.device_omega(DEV), p.device_phase(DEV)
    out = torch.full((37, D + 64), 7.0, dtype=torch.bfloat16, device=DEV)
    xd = x.to(DEV).to(torch.bfloat16)
    N.check(N.lib().kdn_fwht_lift(ctypes.c_void_p(xd.data_ptr()), 37, 64, 1, 0, ctypes.c_void_p(om.data_ptr()),
                                  ctypes.c_void_p(ph.data_ptr()), 64, D, p.tau_star_inv,
                                  ctypes.c_void_p(out.data_ptr()), D + 64, 1,
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), "kdn_fwht_lift")
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert (o[:, D:] == 7.0).all()
    assert rel_l2(o[:, :D], ol.lift(xd.float().cpu().numpy(), op)) < 1e-2


@pytest.mark.parametrize("normalize", [False, True])
def test_lift_bf16(proj, oproj, normalize):
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(3000, 64, generator=g).to(torch.bfloat16)
    out = ops.lift(x.to(DEV), proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv, normalize)
    assert out.dtype == torch.bfloat16
    xr = x.float().numpy()
    if normalize:  # F.normalize on a bf16 tensor returns bf16
        xr = torch.nn.functional.normalize(x.float(), dim=-1, eps=1e-6).to(torch.bfloat16).float().numpy()
    ref = ol.lift(xr, oproj)
    o = out.float().cpu().numpy()
    assert rel_l2(o, ref) < 1e-2
    assert np.abs(o - ref).max() <= 1e-2 * np.abs(ref).max()


def test_lift_config2_properties(proj, oproj):
    """Standalone lift at the BASELINE config-2 size: 2,097,152 rows (B=8, T=16384, H=16), bf16,
    L2-normalised rows.  Size-independent checks on all rows (unit norm), oracle parity on a sample and
    every element within the per-element bound of a float32 restatement."""
    rows = 8 * 16384 * 16
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(rows, 64, generator=g).to(torch.bfloat16)
    xd = x.to(DEV)
    out = ops.lift(xd, proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv, normalize=True)
    norms = out.float().norm(dim=-1)
    assert torch.isfinite(out.float()).all()
    assert float((norms - 1).abs().max()) < 1e-2
    idx = torch.randint(0, rows, (2048,), generator=g)
    xs = torch.nn.functional.normalize(x[idx].float(), dim=-1, eps=1e-6).to(torch.bfloat16).float().numpy()
    ref = ol.lift(xs, oproj)
    assert rel_l2(out[idx.to(DEV)].float().cpu().numpy(), ref) < 1e-2

    # Every element of all rows against a float32 restatement of the lift on the GPU (the bf16 normalised
    # rows times the bf16-exact Omega, cos with the phases, renormalised), with the per-element bound of
    # the 3,000-row test, the restatement pinned to the oracle on the sample above.  The inputs are the
    # rows normalised and rounded to bf16 on the host, lifted without in-kernel normalisation: with it, the
    # bf16 rounding of a normalised element can fall on the other side of a tie than F.normalize's (the
    # norm is summed in another order), which moves one angle by |Omega_fk| ulp(x_k) (measured: one element
    # in 10^9 off by 1.7 % of the peak, the 99.999th percentile at 0.4 %).
    om, ph = proj.device_omega(DEV).float(), proj.device_phase(DEV).float()

    def torch_lift(xn):
        c = torch.cos((xn.float() @ om.t()) * proj.tau_star_inv + ph) * (2.0 / 512) ** 0.5
        return c / (c.norm(dim=-1, keepdim=True) + 1e-8)

    xn = torch.nn.functional.normalize(xd.float(), dim=-1, eps=1e-6).to(torch.bfloat16)
    assert rel_l2(torch_lift(xn[idx.to(DEV)]).cpu().numpy(), ref) < 1e-4
    del out
    out = ops.lift(xn, proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv, normalize=False)
    worst, peak = 0.0, 0.0
    for r0 in range(0, rows, 1 << 18):
        tr = torch_lift(xn[r0:r0 + (1 << 18)])
        worst = max(worst, float((out[r0:r0 + (1 << 18)].float() - tr).abs().max()))
        peak = max(peak, float(tr.abs().max()))
    assert worst <= 1e-2 * peak, (worst, peak)


@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("seed", [42, 7])
@pytest.mark.parametrize("dtype,normalize", [(torch.float32, False), (torch.bfloat16, False), (torch.bfloat16, True)])
def test_lift_bits_equals_table_lift(D, seed, dtype, normalize):
    """kdn_fwht_lift_bits builds Omega in LDS from the sign table; with the same Omega values the lift does
    the same arithmetic as kdn_fwht_lift, so the outputs are equal bit for bit (this pins the in-kernel
    build, element by element, to kdn_build_omega, which is bit-exact against the oracle), and both match
    the oracle."""
    p = FastWalshHadamardProjection(64, D, seed)
    op = ol.make_projection(64, D, seed)
    g = torch.Generator().manual_seed(seed + D)
    x = (torch.randn(1037, 64, generator=g) * 1.3).to(dtype)
    xd = x.to(DEV)
    a = ops.lift_bits(xd, p.device_bits(DEV), p.device_phase(DEV), p.tau_star_inv, normalize)
    b = ops.lift(xd, p.device_omega(DEV), p.device_phase(DEV), p.tau_star_inv, normalize)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    xr = x.float()
    if normalize:
        xr = torch.nn.functional.normalize(xr, dim=-1, eps=1e-6).to(dtype).float()
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_l2(a.float().cpu().numpy(), ol.lift(xr.numpy(), op)) < tol


def test_reference_call_site_shim(proj, oproj):
    """The drop-in for the reference's extension module: kernel_deltanet_cuda.fwht_forward called with the
    reference's argument list (kernels/fwht.py:120) plus phase=self.b, no Omega."""
    import kernel_deltanet_cuda

    p = FastWalshHadamardProjection(64, 512, 42).to(DEV)   # the reference moves the module to the GPU
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 300, 64, generator=g)
    xd = x.to(DEV)
    out = kernel_deltanet_cuda.fwht_forward(xd.contiguous(), p.rademacher_bits, p.D, p.tau_star_inv, phase=p.b)
    assert out.shape == (2, 300, 512) and out.dtype == torch.float32
    ref = ol.lift(x.reshape(-1, 64).numpy(), oproj).reshape(2, 300, 512)
    assert rel_l2(out.cpu().numpy(), ref) < 1e-5
    # host-side tables (a module left on the CPU) are copied to the input's device
    cpu_p = FastWalshHadamardProjection(64, 512, 42)
    out2 = kernel_deltanet_cuda.fwht_forward(xd, cpu_p.rademacher_bits, 512, cpu_p.tau_star_inv, phase=cpu_p.b)
    assert torch.equal(out, out2)
    with pytest.raises(ValueError, match="phase=self.b"):
        kernel_deltanet_cuda.fwht_forward(xd.contiguous(), p.rademacher_bits, p.D, p.tau_star_inv)


def test_lift_bits_config2_equals_table_lift(proj):
    """At config 2's full size (2,097,152 bf16 rows, normalised inputs) the sign-table lift equals the
    table lift bit for bit (the latter is checked against the oracle above)."""
    rows = 8 * 16384 * 16
    g = torch.Generator(device=DEV).manual_seed(99)
    x = torch.randn(rows, 64, generator=g, device=DEV).to(torch.bfloat16)
    a = ops.lift_bits(x, proj.device_bits(DEV), proj.device_phase(DEV), proj.tau_star_inv, normalize=True)
    b = ops.lift(x, proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv, normalize=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("dtype,normalize", [(torch.float32, False), (torch.float32, True), (torch.bfloat16, False),
                                             (torch.bfloat16, True)])
def test_lift_bits_butterfly_matches_oracle(D, dtype, normalize):
    """kdn_fwht_lift_bits_butterfly (in-register wave64 butterflies, no Omega table) against the oracle, and
    against the MFMA-projection lift: the same function up to fp32 summation order (bf16 outputs may
    differ by one rounding step)."""
    p = FastWalshHadamardProjection(64, D, 11)
    op = ol.make_projection(64, D, 11)
    g = torch.Generator().manual_seed(D + 1)
    x = (torch.randn(2051, 64, generator=g) * 1.3).to(dtype)
    xd = x.to(DEV)
    a = ops.lift_bits(xd, p.device_bits(DEV), p.device_phase(DEV), p.tau_star_inv, normalize, butterfly=True)
    b = ops.lift_bits(xd, p.device_bits(DEV), p.device_phase(DEV), p.tau_star_inv, normalize)
    torch.cuda.synchronize()
    assert a.dtype == dtype and a.shape == (2051, D)
    xr = x.float()
    if normalize:
        xr = torch.nn.functional.normalize(xr, dim=-1, eps=1e-6).to(dtype).float()
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    ref = ol.lift(xr.numpy(), op)
    assert rel_l2(a.float().cpu().numpy(), ref) < tol
    assert rel_l2(a.float().cpu().numpy(), b.float().cpu().numpy()) < tol
