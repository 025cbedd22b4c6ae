"""The allocation-free scan entry point kdn_delta_scan_fwd_noalloc (its workspace is the library's fixed
device array) against kdn_delta_scan_fwd with a caller workspace, through the C ABI: equal bit for bit
(the scan's results do not depend on how the chunks are cut into segments), on two calls in a row, the
second with a smaller input, so that the second call runs over the array the first one left filled.
A request too large for the array is refused before anything is launched."""
import ctypes

import pytest
import torch

from kdn import _native as N
from kdn import ops
from kernels import FastWalshHadamardProjection

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(B, T, H, dv, dtype, decay, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 64, generator=g).to(dtype)
    k = torch.randn(B, T, H, 64, generator=g).to(dtype)
    v = torch.randn(B, T, H, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    lam = torch.sigmoid(torch.randn(B, T, H, generator=g)) if decay else None
    s0 = 0.1 * torch.randn(B, H, 512, dv, generator=g)
    return [None if t is None else t.to(DEV) for t in (q, k, v, beta, lam, s0)]


def _run(name, proj, q, k, v, beta, lam, s0, workspace):
    B, T, H, _ = q.shape
    dv = v.shape[-1]
    y = torch.full((B, T, H, dv), float("nan"), device=DEV, dtype=q.dtype)
    S = torch.full((B, H, 512, dv), float("nan"), device=DEV)
    a = ops.scan_args(q, k, v, beta, lam, proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv,
                      False, s0, S, y, workspace, 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    N.check(getattr(N.lib(), name)(ctypes.byref(a), stream), name)
    return y, S


def test_noalloc_equals_workspace_entry_point():
    proj = FastWalshHadamardProjection(64, 512, 42)
    cases = [(2, 64 * 37 + 5, 8, 64, torch.bfloat16, True, 1),   # 16 heads, 38 chunks, decay, initial state
             (1, 64 * 3 + 1, 3, 32, torch.float32, False, 2)]    # then a smaller call, another layout
    for B, T, H, dv, dtype, decay, seed in cases:
        print(f"noalloc case B={B} T={T} H={H} dv={dv} {dtype} decay={decay}", flush=True)
        q, k, v, beta, lam, s0 = _inputs(B, T, H, dv, dtype, decay, seed)
        ws = torch.empty(ops.scan_workspace_bytes(q, v, proj.device_omega(DEV)), dtype=torch.uint8, device=DEV)
        y1, S1 = _run("kdn_delta_scan_fwd", proj, q, k, v, beta, lam, s0, ws)
        y2, S2 = _run("kdn_delta_scan_fwd_noalloc", proj, q, k, v, beta, lam, s0, None)
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)
        assert torch.equal(S1, S2)


def test_noalloc_refuses_requests_beyond_the_array():
    # 600 heads need 600 * 2 records of 238,592 bytes (bf16, d_v = 64) > 256 MiB: refused on the host
    a = N.ScanArgs()
    a.B, a.T, a.H, a.d_k, a.D, a.d_v = 1, 4096, 600, 64, 512, 64
    a.in_dtype = a.out_dtype = N.KDN_DTYPE_BF16
    a.inv_tau = 0.35355339
    assert 600 * 2 * 238592 > N.NOALLOC_SCRATCH_BYTES
    assert N.lib().kdn_delta_scan_fwd_noalloc(ctypes.byref(a), None) == N.KDN_ERR_WORKSPACE_TOO_SMALL
    a.d_k, a.D, a.feature_mode = 1024, 1024, 1     # the pre-lifted D = 1024 path has no segment form
    assert N.lib().kdn_delta_scan_fwd_noalloc(ctypes.byref(a), None) == -2
