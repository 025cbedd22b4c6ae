"""C ABI checks that need no GPU: the library loads, exports exactly what include/kdn.h declares, the
ctypes mirror of kdn_scan_args matches the C layout, and argument errors come back as status codes
before anything is launched."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from kdn import _native as N
from kdn.build import build_native

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "kdn.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(N.LIB_PATH):
        build_native()
    return N.lib()


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|void|const char\*)\s+(kdn_\w+)\s*\(", text, re.M)))


def test_header_declares_exported_set():
    assert _declared() == sorted(N.EXPORTED)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", N.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s+(kdn_\w+)$", out, re.M))
    for name in _declared():
        assert name in exported, name
        assert hasattr(lib, name)


@pytest.mark.parametrize("cname,pystruct", [("kdn_scan_args", N.ScanArgs), ("kdn_ragged_args", N.RaggedArgs),
                                            ("kdn_scan_bwd_args", N.ScanBwdArgs)])
def test_args_layout_matches_c(cname, pystruct):
    fields = [f[0] for f in pystruct._fields_]
    src = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){",
           f'printf("%zu\\n", sizeof({cname}));']
    src += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    src += ["return 0;}"]
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        open(c, "w").write("\n".join(src))
        subprocess.run(["gcc", "-std=c99", "-o", exe, c], check=True)
        vals = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(pystruct)
    for f, off in zip(fields, vals[1:]):
        assert getattr(pystruct, f).offset == off, f


def test_strerror_and_version(lib):
    for code in (0, -1, -2, -3, -4, -5, -99):
        assert len(lib.kdn_strerror(code)) > 0
    assert lib.kdn_abi_version() == (2 << 16) | 3


def _args(**kw):
    a = N.ScanArgs()
    a.B, a.T, a.H, a.d_k, a.D, a.d_v = 1, 65536, 16, 64, 512, 64
    a.in_dtype = a.out_dtype = N.KDN_DTYPE_BF16
    a.inv_tau = 0.35355339
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_workspace_bytes(lib):
    # one 64-token chunk record of one head = 238592 bytes for bf16 inputs, D = 512, d_v = 64; a segment
    # of n chunks uses n + 1 records per head (the last is the state kernel's scratch record)
    a = _args(segment_chunks=1)
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(a)) == 16 * 2 * 238592
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(d_k=32))) == 0
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(d_v=48))) == 0
    a = _args(segment_chunks=100000)  # clamped to the number of chunks
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(a)) == 16 * 1025 * 238592
    # D = 256 runs the 512-wide scan on replicated tables: its workspace (4 + 1 records of 2 heads), then
    # the replicated Omega (512 x 64 bf16) and phases (512 fp32) and two 512-wide fp32 states; per-head
    # Omega with low parts: 2 x 2 tables
    a = _args(T=256, H=2, D=256)
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(a)) == 5 * 2 * 238592 + 65536 + 2048 + 2 * 2 * 512 * 64 * 4
    assert lib.kdn_scan_segment_chunks(ctypes.byref(a), 0) == 4
    a.omega_lo, a.omega_head_stride, a.phase_head_stride = 0x7D0000000000, 256 * 64, 256
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(a)) == \
        5 * 2 * 238592 + 2 * 2 * 65536 + 2 * 2048 + 2 * 2 * 512 * 64 * 4
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(T=256, H=2, D=128))) == \
        5 * 2 * 238592 + 65536 + 2048 + 2 * 2 * 512 * 64 * 4
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(T=256, H=2, D=384))) == 0


def _fake_ptrs(a, base=0x7F0000000000):
    for i, f in enumerate(("q", "k", "v", "beta", "omega_bf16", "phase", "final_state", "y", "workspace")):
        setattr(a, f, base + 0x100000 * i)
    a.q_stride = N._i64x3(64 * 65536 * 16, 64 * 16, 64)
    a.k_stride = N._i64x3(64 * 65536 * 16, 64 * 16, 64)
    a.v_stride = N._i64x3(64 * 65536 * 16, 64 * 16, 64)
    return a


def test_scan_argument_errors_need_no_device(lib):
    run = lambda a: lib.kdn_delta_scan_fwd(ctypes.byref(a), None)
    assert lib.kdn_delta_scan_fwd(None, None) == -1
    assert run(_fake_ptrs(_args(d_k=32))) == -2
    assert run(_fake_ptrs(_args(D=384))) == -2
    assert run(_fake_ptrs(_args(D=256))) == -3                            # supported; workspace too small
    a = _fake_ptrs(_args(D=256))
    a.workspace_bytes = 1 << 40
    assert lib.kdn_scan_prep(ctypes.byref(a), 0, 1, None) == -2           # no phase entry points below 512
    assert lib.kdn_delta_scan_fwd_noalloc(ctypes.byref(a), None) == -2
    a.state_slots = 0x7A0000000000                                       # uniform batches only
    assert run(a) == -2
    assert run(_fake_ptrs(_args(T=0))) == -1
    assert run(_fake_ptrs(_args(in_dtype=7))) == -1
    a = _fake_ptrs(_args())
    a.q = None
    assert run(a) == -1
    a = _fake_ptrs(_args())
    a.q = a.q + 2
    assert run(a) == -4
    a = _fake_ptrs(_args())
    a.v_stride = N._i64x3(1, 3, 1)
    assert run(a) == -4
    a = _fake_ptrs(_args())
    a.workspace_bytes = 1024
    assert run(a) == -3


def test_lift_fwht_omega_argument_errors_need_no_device(lib):
    p = 0x7F0000000000
    assert lib.kdn_fwht_lift(p, 10, 64, 1, 0, p, p, 32, 512, 0.35, p, 512, 1, None) == -2
    assert lib.kdn_fwht_lift(p, 10, 64, 1, 0, p, p, 64, 384, 0.35, p, 512, 1, None) == -2
    assert lib.kdn_fwht_lift(p + 2, 10, 64, 1, 0, p, p, 64, 512, 0.35, p, 512, 1, None) == -4
    assert lib.kdn_fwht_lift(None, 10, 64, 1, 0, p, p, 64, 512, 0.35, p, 512, 1, None) == -1
    assert lib.kdn_fwht_lift(p, 0, 64, 1, 0, p, p, 64, 512, 0.35, p, 512, 1, None) == 0
    # bf16 output rows must be 16-byte multiples (the kernel stores whole 16-byte pieces of rows)
    assert lib.kdn_fwht_lift(p, 10, 64, 1, 0, p, p, 64, 512, 0.35, p, 516, 1, None) == -4
    assert lib.kdn_fwht(p, 4, 3, 3, 0, p, 3, None) == -2
    assert lib.kdn_fwht(p, 0, 64, 64, 0, p, 64, None) == 0
    assert lib.kdn_build_omega(p, 32, 512, p, 1, None) == -2
    assert lib.kdn_build_omega(None, 64, 512, p, 1, None) == -1
    # the sign-table lift (the reference's fwht_forward boundary): (x, rows, stride, dtype, d_k, bits, D, 1/tau,
    # phase, normalize, out, out stride, out dtype, stream)
    for lb in (lib.kdn_fwht_lift_bits, lib.kdn_fwht_lift_bits_butterfly):
        _lift_bits_errors(lb, p)


def _lift_bits_errors(lb, p):
    assert lb(p, 10, 64, 0, 64, None, 512, 0.35, p, 0, p, 512, 0, None) == -1     # no table
    assert lb(p, 10, 64, 0, 64, p, 512, 0.35, None, 0, p, 512, 0, None) == -1     # no phase
    assert lb(p, 10, 64, 0, 128, p, 512, 0.35, p, 0, p, 512, 0, None) == -2      # d_k 128
    assert lb(p, 10, 64, 0, 64, p, 1024, 0.35, p, 0, p, 1024, 0, None) == -2     # D 1024
    assert lb(p, 10, 64, 0, 64, p + 4, 512, 0.35, p, 0, p, 512, 0, None) == -4   # table not 8-byte aligned
    assert lb(p, 10, 64, 0, 64, p, 512, 0.35, p + 8, 0, p, 512, 0, None) == -4   # phase not 16-byte aligned
    assert lb(p, 10, 64, 0, 64, p, 512, float("nan"), p, 0, p, 512, 0, None) == -1
    assert lb(p, 0, 64, 0, 64, p, 512, 0.35, p, 0, p, 512, 0, None) == 0         # no rows: nothing launched


def test_general_width_requests_need_no_device(lib):
    # D = 1024 (the factored d_k = 128 path): pre-lifted features only, d_v 64 or 128, the delta rule; one
    # fp32 record per (batch, head, chunk): 286,848 floats at d_v = 128, 213,120 at d_v = 64
    a = _args(T=256, H=2, d_k=1024, D=1024, d_v=128, feature_mode=1)
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(a)) == 2 * 4 * 286848 * 4
    assert lib.kdn_scan_workspace_bytes_pipelined(ctypes.byref(a)) == 2 * 4 * 286848 * 4
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(T=256, d_k=1024, D=1024, d_v=64, feature_mode=1))) \
        == 16 * 4 * 213120 * 4
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(d_k=64, D=1024, feature_mode=0))) == 0
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(d_k=1024, D=1024, d_v=32, feature_mode=1))) == 0
    assert lib.kdn_scan_workspace_bytes(ctypes.byref(_args(d_k=1024, D=1024, feature_mode=1, rule=1))) == 0
    # the general-width scan has no phase entry points: rejected on the host before anything is enqueued
    a = _fake_ptrs(_args(T=256, H=2, d_k=1024, D=1024, d_v=128, feature_mode=1))
    a.workspace_bytes = 1 << 40
    assert lib.kdn_scan_prep(ctypes.byref(a), 0, 1, None) == -2
    assert lib.kdn_scan_state(ctypes.byref(a), 0, 1, None) == -2
    a.workspace_bytes = 1024
    assert lib.kdn_delta_scan_fwd(ctypes.byref(a), None) == -3


def test_schedule_query_and_fused_phases_need_no_device(lib, monkeypatch):
    """kdn_scan_schedule: the pre-lifted D = 1024 scan is its own schedule, fp32 inputs always run the split
    kernels, and KDN_SCAN_SCHEDULE (read per call) forces the bf16 choice; the fused schedule's phase entry
    points reject what the fused chain does not implement before anything is enqueued."""
    monkeypatch.delenv("KDN_SCAN_SCHEDULE", raising=False)
    assert lib.kdn_scan_schedule(ctypes.byref(_args(d_k=1024, D=1024, d_v=64, feature_mode=1))) == 2
    f32 = _args(in_dtype=N.KDN_DTYPE_F32, out_dtype=N.KDN_DTYPE_F32)
    assert lib.kdn_scan_schedule(ctypes.byref(f32)) == 0
    monkeypatch.setenv("KDN_SCAN_SCHEDULE", "fused")
    assert lib.kdn_scan_schedule(ctypes.byref(_args())) == 1
    assert lib.kdn_scan_schedule(ctypes.byref(f32)) == 0
    monkeypatch.setenv("KDN_SCAN_SCHEDULE", "split")
    assert lib.kdn_scan_schedule(ctypes.byref(_args())) == 0
    assert lib.kdn_scan_schedule(ctypes.byref(_args(d_v=48))) == -2
    a = _fake_ptrs(_args(T=256, H=2, in_dtype=N.KDN_DTYPE_F32, out_dtype=N.KDN_DTYPE_F32))
    a.workspace_bytes = 1 << 40
    assert lib.kdn_scan_prep_fused(ctypes.byref(a), 0, 1, None) == -2
    assert lib.kdn_scan_chain(ctypes.byref(a), 0, 1, None) == -2
    g = _fake_ptrs(_args(T=256, H=2, d_k=1024, D=1024, d_v=128, feature_mode=1))
    g.workspace_bytes = 1 << 40
    assert lib.kdn_scan_chain(ctypes.byref(g), 0, 1, None) == -2
    b = _fake_ptrs(_args(T=256, H=2))
    b.workspace_bytes = 1024
    assert lib.kdn_scan_chain(ctypes.byref(b), 0, 1, None) == -3


def test_backward_workspace_and_errors_need_no_device(lib):
    f = _fake_ptrs(_args(T=256, H=2))
    g = N.ScanBwdArgs()
    g.fwd = ctypes.addressof(f)
    for i, nm in enumerate(("dy", "dq", "dk", "dv", "dbeta", "workspace")):
        setattr(g, nm, 0x7E0000000000 + 0x100000 * i)
    # one segment (the default at this size): its 4 chunk records per head and the Omega^T table
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 4 * 1099776 + 65536
    seg = ctypes.c_int64(0)
    assert lib.kdn_scan_bwd_segments(ctypes.byref(g), ctypes.byref(seg)) == 1 and seg.value == 4
    # segments of one chunk: three rotating record buffers, three segment-start states and the carried
    # dL/dS (2 heads x 512 x 64 fp32 each), two buffers of the forward scan's records for the checkpoint
    # pass (2 records of 238,592 bytes per head), the table
    f.segment_chunks = 1
    assert lib.kdn_scan_bwd_segments(ctypes.byref(g), ctypes.byref(seg)) == 4 and seg.value == 1
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == \
        3 * 2 * 1099776 + 4 * 2 * 512 * 64 * 4 + 2 * 2 * 2 * 238592 + 65536
    g.workspace_bytes = 1 << 40
    assert lib.kdn_scan_bwd_phase(ctypes.byref(g), 5, 0, None) == -1
    assert lib.kdn_scan_bwd_phase(ctypes.byref(g), 1, 4, None) == -1   # segments 0 .. 3
    assert lib.kdn_scan_bwd_phase(ctypes.byref(g), 2, -1, None) == -1
    f.segment_chunks = 0
    g.workspace_bytes = 1024
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -3
    assert lib.kdn_scan_bwd_phase(ctypes.byref(g), 1, 0, None) == -3
    f2 = _fake_ptrs(_args(T=256, H=2, d_v=48))                         # d_v outside {16, 32, 64, 128}
    g.fwd = ctypes.addressof(f2)
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 0
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -2
    # d_v = 32 runs the 64-wide backward on zero-padded copies: its workspace, then (256-byte aligned) the
    # padded v (512 rows x 64 bf16), dy and dv (512 x 64 fp32 each); no phase entry points
    f2.d_v = 32
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 4 * 1099776 + 65536 + 512 * 64 * (2 + 4 + 4)
    seg = ctypes.c_int64(0)
    assert lib.kdn_scan_bwd_segments(ctypes.byref(g), ctypes.byref(seg)) == 1 and seg.value == 4
    g.workspace_bytes = 1 << 40
    assert lib.kdn_scan_bwd_phase(ctypes.byref(g), 1, 0, None) == -2
    g.workspace_bytes = 1024
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -3
    # d_v = 128: two 64-wide passes; the second pass's dq, dk (512 x 64 fp32) and dbeta (512 fp32) go to
    # the workspace before they are added into the outputs
    f2.d_v = 128
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 4 * 1099776 + 65536 + 2 * 512 * 64 * 4 + 2048
    # D = 256: the 512-wide backward's workspace, the replicated tables, three 512-wide fp32 states
    f2.d_v, f2.D = 64, 256
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == \
        2 * 4 * 1099776 + 65536 + 65536 + 2048 + 3 * 2 * 512 * 64 * 4
    assert lib.kdn_scan_bwd_segments(ctypes.byref(g), ctypes.byref(seg)) == 1 and seg.value == 4
    assert lib.kdn_scan_bwd_phase(ctypes.byref(g), 1, 0, None) == -2
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -3
    f2.D = 512
    g.fwd = ctypes.addressof(f)
    # per-head Omega with low parts (the P2 / P4 feature maps, ABI 1.7): one Omega^T table per head and
    # part; dL/d(1/tau) adds one fp32 partial per (batch, head, chunk), rounded up to 256 bytes
    f3 = _fake_ptrs(_args(T=256, H=2, rule=1, no_renorm=1))
    f3.omega_lo, f3.omega_head_stride, f3.phase_head_stride = 0x7D0000000000, 512 * 64, 512
    g.fwd = ctypes.addressof(f3)
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 4 * 1099776 + 2 * 2 * 65536
    g.dinv_tau = 0x7C0000000000
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 4 * 1099776 + 2 * 2 * 65536 + 256
    f3.phase_head_stride = 510                                          # per-head phases must stay 16-byte aligned
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -4
    f3.feature_mode, f3.d_k = 1, 512                                    # pre-lifted features: no backward
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 0
    g.dinv_tau = None
    g.fwd = ctypes.addressof(f)
    g.dy = None
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -1


def test_general_width_backward_needs_no_device(lib):
    # D = 1024 over pre-lifted features (ABI 1.8): one record per (batch, head, chunk) of a segment
    # (753,792 floats at d_v = 128, 454,784 at d_v = 64) plus the forward carry's final state
    f = _fake_ptrs(_args(T=256, H=2, d_k=1024, D=1024, d_v=128, feature_mode=1))
    g = N.ScanBwdArgs()
    g.fwd = ctypes.addressof(f)
    for i, nm in enumerate(("dy", "dq", "dk", "dv", "dbeta", "workspace")):
        setattr(g, nm, 0x7E0000000000 + 0x100000 * i)
    rec128, rec64 = 753792 * 4, 454784 * 4
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 4 * rec128 + 2 * 1024 * 128 * 4
    seg = ctypes.c_int64(0)
    assert lib.kdn_scan_bwd_segments(ctypes.byref(g), ctypes.byref(seg)) == 1 and seg.value == 4
    f.d_v = 64
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 4 * rec64 + 2 * 1024 * 64 * 4
    g.workspace_bytes = 1 << 40
    assert lib.kdn_scan_bwd_phase(ctypes.byref(g), 1, 0, None) == -2   # no phase entry points at D = 1024
    g.workspace_bytes = 1024
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -3
    f.H = 70000                                                        # beyond the chunk launches' grid limit
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 0
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -2
    f.H = 2
    # segments: the records of one segment plus a state per segment boundary, the carried dL/dS and the
    # forward carry's final state; the default segment is the largest power of two up to 256 chunks whose
    # records fit 12 GiB (2 heads x 3,015,168 bytes per chunk: 256), so the workspace stops growing with T
    f.d_v = 128
    st = 2 * 1024 * 128 * 4
    f.segment_chunks = 3                                               # 4 chunks in segments of 3 and 1
    assert lib.kdn_scan_bwd_segments(ctypes.byref(g), ctypes.byref(seg)) == 2 and seg.value == 3
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 3 * rec128 + 3 * st
    f.segment_chunks, f.T = 0, 64 * 1000                               # 1000 chunks: 4 segments of 256
    assert lib.kdn_scan_bwd_segments(ctypes.byref(g), ctypes.byref(seg)) == 4 and seg.value == 256
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 256 * rec128 + (3 + 1 + 1) * st
    f.T = 64 * 100000                                                  # 100,000 chunks: the same records
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 2 * 256 * rec128 + (391 + 1) * st
    f.T = 256
    g.dinv_tau = 0x7C0000000000                                        # no temperature to differentiate
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 0
    g.dinv_tau = None
    f.d_v = 32
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 0
    f.d_v, f.rule = 64, 1
    assert lib.kdn_scan_bwd_workspace_bytes(ctypes.byref(g)) == 0
    f.rule = 0
    g.ddecay = 0x7B0000000000                                          # ddecay without a forward decay
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -1
    g.ddecay = None
    g.dk = None
    assert lib.kdn_delta_scan_bwd(ctypes.byref(g), None) == -1


def test_factored_lift_backward_errors_need_no_device(lib):
    fb = lib.kdn_fwht_lift_factored_bwd
    p = 0x7F0000000000
    ok = (p, 10, 128, 1, p, p, p, p, 0.35, p, 1024, p, 128, None)
    assert fb(*ok[:1], 0, *ok[2:]) == 0                                  # no rows: nothing launched
    assert fb(None, *ok[1:]) == -1
    assert fb(*ok[:1], -1, *ok[2:]) == -1
    assert fb(*ok[:2], 64, *ok[3:]) == -1                                # x rows of 128
    assert fb(*ok[:3], 7, *ok[4:]) == -1                                 # dtype
    assert fb(*ok[:4], p + 4, *ok[5:]) == -4                             # Omega 8-byte aligned
    assert fb(*ok[:5], p + 8, *ok[6:]) == -4                             # phases 16-byte aligned
    assert fb(*ok[:10], 1026, *ok[11:]) == -4                            # dout rows of 16-byte multiples
    assert fb(*ok[:8], float("nan"), *ok[9:]) == -1
    assert fb(*ok[:10], 512, *ok[11:]) == -1                             # dout rows of 1024
    assert fb(*ok[:9], p + 2, *ok[10:]) == -4                            # fp32 dout


def test_slot_step_workspace_and_errors_need_no_device(lib):
    # the serving step from a slot map: every size from num_tokens and num_slots.  1000 tokens, 10 slots:
    # at most 21 runs (and prefills), 16 + 2 * 21 = 58 packed slots: one window of 64; the small arrays
    # (run counts of one 2048-token block, runs, lists, layout: 2816 bytes) and one window buffer of
    # 2 heads x 65 records of 238,592 bytes
    a = N.SlotStepArgs()
    a.num_tokens, a.H, a.d_k, a.D, a.d_v = 1000, 2, 64, 512, 64
    a.in_dtype = a.out_dtype = N.KDN_DTYPE_BF16
    a.inv_tau, a.slot_bytes, a.num_slots = 0.35355339, 8, 10
    assert lib.kdn_slot_step_workspace_bytes(ctypes.byref(a)) == 2816 + 2 * 65 * 238592
    a.num_tokens = 1 << 20    # 16384 + 2 * 21 slots: windows of 1024 (the most), three buffers of 1025 records;
    # 512 run-count blocks of 2048 tokens
    assert lib.kdn_slot_step_workspace_bytes(ctypes.byref(a)) == 2560 + 512 * 8 + 3 * 2 * 1025 * 238592
    a.num_tokens = 1                          # one token: a decode at most, no prefill window
    assert lib.kdn_slot_step_workspace_bytes(ctypes.byref(a)) == 11 * 256
    a.num_tokens = 1000
    a.slot_bytes = 2
    assert lib.kdn_slot_step_workspace_bytes(ctypes.byref(a)) == 0
    a.slot_bytes, a.D = 4, 256
    assert lib.kdn_slot_step_workspace_bytes(ctypes.byref(a)) == 0   # D = 512 only
    a.D = 512
    assert lib.kdn_slot_step(ctypes.byref(a), None, None) == -1       # no pointers
    for i, f in enumerate(("slot_mapping", "q", "k", "v", "beta", "omega_bf16", "phase", "states", "y", "workspace")):
        setattr(a, f, 0x7F0000000000 + 0x100000 * i)
    a.workspace_bytes = 1024
    assert lib.kdn_slot_step(ctypes.byref(a), None, None) == -3
