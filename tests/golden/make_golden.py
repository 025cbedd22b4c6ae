"""Writes the small golden fixtures of tests/golden from the CPU oracle (run from the repo root).

  projection_seed42.npz  packed sign table, phases b, integer Omega*sqrt(d_k) for d_k=64, D=512, seed=42
  lift_kat.npz           8 input rows -> lifted features (plain and with input normalisation), float64
  scan_kat.npz           B=2, T=80, d_v=16 delta-rule inputs with decay and an initial state -> y, S, float64
The fixtures pin the oracle against regressions; the oracle itself is pinned by the closed-form tests.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import lift as ol  # noqa: E402
from oracle import scan as osc  # noqa: E402


def main():
    proj = ol.make_projection(64, 512, 42)
    np.savez(os.path.join(HERE, "projection_seed42.npz"), bits=proj["bits"], b=proj["b"],
             omega_int=proj["omega_int"].astype(np.int32))
    rng = np.random.default_rng(20241201)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    np.savez(os.path.join(HERE, "lift_kat.npz"), x=x, phi=ol.lift(x, proj),
             phi_normalized=ol.lift(x, proj, normalize=True))
    B, T, dv = 2, 80, 16
    q = rng.standard_normal((B, T, 64)).astype(np.float32)
    k = rng.standard_normal((B, T, 64)).astype(np.float32)
    v = rng.standard_normal((B, T, dv)).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, T))))).astype(np.float32)
    decay = rng.uniform(0.94, 0.99, (B, T)).astype(np.float32)
    S0 = (0.1 * rng.standard_normal((B, dv, 512))).astype(np.float32)
    y, S = osc.delta_rule(q, k, v, beta, decay, proj, S0)
    np.savez(os.path.join(HERE, "scan_kat.npz"), q=q, k=k, v=v, beta=beta, decay=decay, S0=S0, y=y, S=S)


if __name__ == "__main__":
    main()
