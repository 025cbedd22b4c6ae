"""GPU parity of the factored d_k = 128 path: kdn_fwht_lift_factored and the D = 1024 scan.

Oracles: oracle.lift.factored_lift (float64; pinned in test_oracle_factored.py) for the lift, and the
float64 token recurrence (oracle.scan.token_recurrence) over the oracle's factored features for the scan
-- the reference's own acceptance check (tests/test_factored_kernel.py:25-60, 82-118: chunked scan vs
the unrolled recurrence, B = 2, T = 256, d_k = 128, d_v = 128, decay in [0.9, 1]).  Tolerances (relative
L2): lift 1e-5 (fp32) / 1e-2 (bf16 outputs); scan 1e-4 for fp32 inputs, 2e-2 for bf16 inputs.  Unit
norms to 1e-5 as the reference checks them (tests/test_factored_kernel.py:65-78).
"""
import numpy as np
import pytest
import torch

from kdn import ops
from kernels import FactoredFastWalshHadamardProjection, FactoredKernelDeltaNet, factored_chunked_deltanet_forward
from oracle import lift as ol
from oracle import scan as osc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def fproj():
    return FactoredFastWalshHadamardProjection(128, 1024, 42)


@pytest.fixture(scope="module")
def oprojs():
    return ol.make_projection(64, 512, 42), ol.make_projection(64, 512, 1042)


def rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_factored_lift(fproj, oprojs, dtype, tol):
    x = torch.randn(4, 32, 128, generator=torch.Generator().manual_seed(0)).to(dtype)
    phi = fproj(x.to(DEV))
    torch.cuda.synchronize()
    assert phi.shape == (4, 32, 1024) and phi.dtype == dtype
    ref = ol.factored_lift(x.float().numpy(), *oprojs)
    assert rel(phi.float().cpu().numpy(), ref) < tol
    norms = torch.linalg.vector_norm(phi.float(), dim=-1).cpu()
    assert torch.allclose(norms, torch.ones_like(norms), atol=1e-5 if dtype == torch.float32 else 1e-2)


def oracle_scan(q, k, v, beta, decay, oprojs, s0=None):
    pq = ol.factored_lift(q.float().numpy(), *oprojs)
    pk = ol.factored_lift(k.float().numpy(), *oprojs)
    return osc.token_recurrence(pq, pk, v.double().numpy(), beta.double().numpy(),
                                None if decay is None else decay.double().numpy(),
                                None if s0 is None else s0.double().numpy())


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_factored_scan_matches_the_recurrence(fproj, oprojs, dtype, tol):
    g = torch.Generator().manual_seed(42)
    B, T, dv = 2, 256, 128
    q = torch.randn(B, T, 128, generator=g).to(dtype)
    k = torch.randn(B, T, 128, generator=g).to(dtype)
    v = torch.randn(B, T, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    decay = torch.sigmoid(torch.randn(B, T, generator=g)) * 0.1 + 0.9
    Y, S = factored_chunked_deltanet_forward(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), decay.to(DEV), fproj)
    torch.cuda.synchronize()
    Yr, Sr = oracle_scan(q, k, v, beta, decay, oprojs)
    assert Y.shape == (B, T, dv) and S.shape == (B, dv, 1024)
    assert rel(Y.float().cpu().numpy(), Yr) < tol
    assert rel(S.float().cpu().numpy(), Sr) < tol


def test_factored_scan_partial_chunk_initial_state_dv64(fproj, oprojs):
    g = torch.Generator().manual_seed(7)
    B, T, dv = 1, 200, 64
    q, k = torch.randn(B, T, 128, generator=g), torch.randn(B, T, 128, generator=g)
    v = torch.randn(B, T, dv, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, generator=g))
    s0 = 0.1 * torch.randn(B, dv, 1024, generator=g)
    model = FactoredKernelDeltaNet(d_k=128, d_v=dv, D=1024)
    Y, S = model(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), None, s0.to(DEV))
    torch.cuda.synchronize()
    Yr, Sr = oracle_scan(q, k, v, beta, None, oprojs, s0)
    assert rel(Y.cpu().numpy(), Yr) < 1e-4
    assert rel(S.cpu().numpy(), Sr) < 1e-4


def test_factored_scan_continues_across_calls(fproj):
    # two calls chained through the state equal one call over the concatenation
    g = torch.Generator().manual_seed(8)
    T1, T2 = 130, 70
    q, k = torch.randn(1, T1 + T2, 128, generator=g), torch.randn(1, T1 + T2, 128, generator=g)
    v = torch.randn(1, T1 + T2, 128, generator=g)
    beta = torch.sigmoid(torch.randn(1, T1 + T2, generator=g))
    dec = 0.95 + 0.05 * torch.rand(1, T1 + T2, generator=g)
    a = [t.to(DEV) for t in (q, k, v, beta, dec)]
    Y1, S1 = factored_chunked_deltanet_forward(*(t[:, :T1] for t in a), fproj)
    Y2, S2 = factored_chunked_deltanet_forward(*(t[:, T1:] for t in a), fproj, initial_state=S1)
    Y, S = factored_chunked_deltanet_forward(*a, fproj)
    torch.cuda.synchronize()
    assert rel(torch.cat([Y1, Y2], 1).cpu().numpy(), Y.cpu().numpy()) < 1e-5
    assert rel(S2.cpu().numpy(), S.cpu().numpy()) < 1e-5


def test_factored_scan_single_partial_chunk(fproj, oprojs):
    g = torch.Generator().manual_seed(9)
    q, k = torch.randn(1, 5, 128, generator=g), torch.randn(1, 5, 128, generator=g)
    v = torch.randn(1, 5, 128, generator=g)
    beta = torch.sigmoid(torch.randn(1, 5, generator=g))
    dec = 0.9 + 0.1 * torch.rand(1, 5, generator=g)
    Y, S = factored_chunked_deltanet_forward(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), dec.to(DEV), fproj)
    torch.cuda.synchronize()
    Yr, Sr = oracle_scan(q, k, v, beta, dec, oprojs)
    assert rel(Y.cpu().numpy(), Yr) < 1e-4
    assert rel(S.cpu().numpy(), Sr) < 1e-4
