"""Pins of the oracle lift (oracle/lift.py) against closed forms, library routines and the reference's
own construction rules (kernels/fwht.py:25-131).  CPU only."""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import lift as ol

GOLDEN = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def proj():
    return ol.make_projection(64, 512, 42)


def test_seeded_uniform_stream_known_values():
    # torch's CPU MT19937 stream for seed 42 (the library routine behind kernels/fwht.py:66-86).
    g = torch.Generator().manual_seed(42)
    u = torch.rand(10, generator=g).numpy()
    known = np.array([0.8823, 0.9150, 0.3829, 0.9593, 0.3904, 0.6009, 0.2566, 0.7936, 0.9408, 0.1332])
    np.testing.assert_allclose(u, known, atol=6e-5)


def test_draw_order_stream_positions(proj):
    """d1, d2, d3 and b take consecutive blocks of the seed-42 stream in that order (kernels/fwht.py:66-86:
    three rand(M, d_k) draws, then rand(D)): with M * d_k = 512, d1 = u[0:512], d2 = u[512:1024],
    d3 = u[1024:1536] (+1 iff u > 0.5) and b = 2 pi u[1536:2048] of one rand(2048) draw.  Known values of
    the stream at each block start pin the positions themselves; a swap of d2 / d3 (equal in only about
    half of their entries) or of the signs and b fails here."""
    g = torch.Generator().manual_seed(42)
    u = torch.rand(2048, generator=g)
    starts = {0: [0.882269, 0.915004, 0.382864, 0.959306], 512: [0.655622, 0.118564, 0.183628, 0.084309],
              1024: [0.778491, 0.42534, 0.712356, 0.206497], 1536: [0.572927, 0.346504, 0.241869, 0.339226]}
    for s, vals in starts.items():
        np.testing.assert_allclose(u[s:s + 4].numpy(), vals, atol=1e-6)
    signs = lambda a: np.where(a.numpy() > 0.5, 1.0, -1.0).reshape(8, 64)
    np.testing.assert_array_equal(proj["d1"], signs(u[0:512]))
    np.testing.assert_array_equal(proj["d2"], signs(u[512:1024]))
    np.testing.assert_array_equal(proj["d3"], signs(u[1024:1536]))
    np.testing.assert_array_equal(np.asarray(proj["b"], np.float32), (u[1536:] * (2 * math.pi)).numpy())
    assert 0.3 < (proj["d2"] == proj["d3"]).mean() < 0.7


def test_first_signs_follow_rand_gt_half(proj):
    # d1 row 0 comes from the first 64 uniforms: +1 iff u > 0.5 (kernels/fwht.py:69).
    assert list(proj["d1"][0, :10]) == [1, 1, -1, 1, -1, 1, -1, 1, 1, -1]


def test_bit_table_encodes_minus_signs(proj):
    bits = proj["bits"].view(np.uint64)
    for m in range(proj["M"]):
        for s, d in enumerate((proj["d1"], proj["d2"], proj["d3"])):
            for i in range(64):
                assert ((int(bits[m, s]) >> i) & 1) == (1 if d[m, i] < 0 else 0)


def test_sylvester_matches_scipy():
    np.testing.assert_array_equal(ol.hadamard(64), scipy.linalg.hadamard(64))


def test_omega_blocks_orthogonal(proj):
    om = proj["omega"]
    for m in range(8):
        blk = om[64 * m:64 * (m + 1)]
        np.testing.assert_allclose(blk.T @ blk, 4096.0 * np.eye(64), atol=1e-9)
        np.testing.assert_allclose(blk @ blk.T, 4096.0 * np.eye(64), atol=1e-9)


def test_omega_matches_butterfly_construction(proj):
    np.testing.assert_array_equal(ol.omega_by_butterfly(proj), proj["omega"])


def test_omega_is_integer_over_8_and_bf16_exact(proj):
    o8 = proj["omega"] * 8.0
    np.testing.assert_array_equal(o8, np.round(o8))
    t = torch.tensor(proj["omega"], dtype=torch.float32)
    assert bool((t.to(torch.bfloat16).float() == t).all())


def test_fwht_rows_equals_hadamard_product():
    rng = np.random.default_rng(1)
    for n in (1, 2, 4, 8, 16, 32, 64):
        x = rng.standard_normal((5, n))
        np.testing.assert_allclose(ol.fwht_rows(x), x @ ol.hadamard(n), atol=1e-12)
        np.testing.assert_allclose(ol.fwht_rows(ol.fwht_rows(x)), n * x, atol=1e-10)


def test_fwht_rows_brute_force_n4():
    x = np.array([[1.0, 2.0, 3.0, 4.0]])
    # butterflies h=1: (3,-1,7,-1); h=2: (10,-2,-4,0)
    np.testing.assert_array_equal(ol.fwht_rows(x), [[10.0, -2.0, -4.0, 0.0]])


def test_lift_unit_norm_and_zero_input(proj):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 64))
    phi = ol.lift(x, proj)
    np.testing.assert_allclose(np.linalg.norm(phi, axis=-1), 1.0, atol=1e-12)
    z = ol.lift(np.zeros((1, 64)), proj)
    c = np.cos(proj["b"].astype(np.float64))
    np.testing.assert_allclose(z[0], c / (np.linalg.norm(c) + 1e-8 / math.sqrt(2 / 512)), atol=1e-12)


def test_lift_projection_via_butterfly(proj):
    # Omega x evaluated block by block with butterflies instead of the explicit matrix.
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 64))
    via = []
    for m in range(8):
        y = ol.fwht_rows(x * proj["d1"][m])
        y = ol.fwht_rows(y * proj["d2"][m])
        y = ol.fwht_rows(y * proj["d3"][m])
        via.append(y / 8.0)
    np.testing.assert_allclose(np.concatenate(via, axis=-1), x @ proj["omega"].T, atol=1e-9)


def test_lift_normalize_matches_torch_normalize(proj):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 64)) * 5
    xn = torch.nn.functional.normalize(torch.tensor(x), p=2, dim=-1, eps=1e-6).numpy()
    np.testing.assert_allclose(ol.lift(x, proj, normalize=True), ol.lift(xn, proj), atol=1e-12)


def test_projection_fixture(proj):
    g = np.load(f"{GOLDEN}/projection_seed42.npz")
    np.testing.assert_array_equal(g["bits"], proj["bits"])
    np.testing.assert_array_equal(g["b"], proj["b"])
    np.testing.assert_array_equal(g["omega_int"], proj["omega_int"])


def test_lift_fixture(proj):
    g = np.load(f"{GOLDEN}/lift_kat.npz")
    np.testing.assert_allclose(ol.lift(g["x"], proj), g["phi"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(ol.lift(g["x"], proj, normalize=True), g["phi_normalized"], rtol=0, atol=1e-12)
