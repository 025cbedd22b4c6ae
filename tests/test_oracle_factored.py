"""Pins of the factored-lift oracle (oracle.lift.factored_lift), CPU only.

Reference: kernels/factored_kernel_deltanet.py:42-74 (two 64 -> 512 lifts of the halves of x, seeds s and
s + 1000, concatenated and renormalised with eps 1e-7) and tests/test_factored_kernel.py:65-78 (unit norm).
"""
import math

import numpy as np

from oracle import lift as ol


def test_unit_norm_and_shape():
    p1, p2 = ol.make_projection(64, 512, 42), ol.make_projection(64, 512, 1042)
    x = np.random.default_rng(0).standard_normal((4, 32, 128))
    phi = ol.factored_lift(x, p1, p2)
    assert phi.shape == (4, 32, 1024)
    assert np.abs(np.linalg.norm(phi, axis=-1) - 1.0).max() < 1e-6


def test_closed_form_at_zero():
    p1, p2 = ol.make_projection(64, 512, 42), ol.make_projection(64, 512, 1042)
    # x = 0: each half is sqrt(2/D) cos(b) / (|.| + 1e-8), the concatenation divided by (|.| + 1e-7)
    phi = ol.factored_lift(np.zeros((1, 128)), p1, p2)[0]

    def half(p):
        f = math.sqrt(2.0 / 512) * np.cos(p["b"].astype(np.float64))
        return f / (np.linalg.norm(f) + 1e-8)

    c = np.concatenate([half(p1), half(p2)])
    assert np.abs(phi - c / (np.linalg.norm(c) + 1e-7)).max() < 1e-15


def test_equal_halves_reduce_to_the_single_lift():
    p = ol.make_projection(64, 512, 42)
    xh = np.random.default_rng(1).standard_normal((5, 64))
    phi = ol.factored_lift(np.concatenate([xh, xh], axis=-1), p, p)
    single = ol.lift(xh, p)
    assert np.abs(phi[:, :512] - single / math.sqrt(2.0)).max() < 1e-6
    assert np.array_equal(phi[:, :512], phi[:, 512:])


def test_second_projection_uses_seed_plus_1000():
    p1, p2 = ol.make_projection(64, 512, 42), ol.make_projection(64, 512, 1042)
    assert not np.array_equal(p1["omega"], p2["omega"])
    x = np.random.default_rng(2).standard_normal((3, 128))
    phi = ol.factored_lift(x, p1, p2)
    # the second half is the seed-1042 lift of the second half of x, up to the common scale
    h2 = ol.lift(x[:, 64:], p2)
    ratio = phi[:, 512:] / h2
    assert np.abs(ratio - ratio[:, :1]).max() < 1e-9


def test_torch_factored_lift_equals_the_numpy_oracle_and_passes_gradcheck():
    # oracle.scan.factored_lift_torch (the gradient oracle of the factored backward) restates
    # oracle.lift.factored_lift on torch tensors: equal in float64, and its autograd gradient agrees with
    # central differences (torch.autograd.gradcheck)
    import torch
    from oracle import scan as osc
    p1, p2 = ol.make_projection(64, 512, 42), ol.make_projection(64, 512, 1042)
    x = np.random.default_rng(3).standard_normal((3, 128))
    got = osc.factored_lift_torch(torch.from_numpy(x), p1, p2).numpy()
    assert np.abs(got - ol.factored_lift(x, p1, p2)).max() < 1e-13
    xt = torch.from_numpy(x[:2]).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: osc.factored_lift_torch(t, p1, p2), (xt,), eps=1e-6, atol=1e-7)
