"""Tensor-level entry points over the C ABI (include/kdn.h).

torch supplies device memory and the current HIP stream; every computation is a HIP kernel in
libkdn.so.  Inputs must be gfx950 device tensors -- there is no CPU path.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _native as N

_DTYPE_TAG = {torch.float32: N.KDN_DTYPE_F32, torch.bfloat16: N.KDN_DTYPE_BF16}


def _tag(dt: torch.dtype, what: str) -> int:
    try:
        return _DTYPE_TAG[dt]
    except KeyError:
        raise TypeError(f"{what}: dtype {dt} is not supported (bfloat16 or float32)") from None


def require_device(t: torch.Tensor, what: str) -> None:
    """Raise unless `t` lives on a GPU: there is no CPU implementation of any entry point."""
    if not t.is_cuda:
        raise RuntimeError(f"{what}: kernel-deltanet_amd runs on gfx950 device tensors only (got {t.device})")


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _rows(x: torch.Tensor, n: int) -> torch.Tensor:
    """(..., n) -> a (rows, n) view with contiguous rows (copies only if no such view exists)."""
    if x.dim() == 1:
        x = x.unsqueeze(0)
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    return x2


def build_omega(sign_bits: torch.Tensor, d_k: int, D: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    """Omega[D][d_k] built on `device` from the packed [M][3] Rademacher table (kdn_build_omega)."""
    device = torch.device(device)
    bits = sign_bits.to(device=device, dtype=torch.int64).contiguous()
    require_device(bits, "build_omega")
    out = torch.empty(D, d_k, dtype=dtype, device=device)
    with torch.cuda.device(device):
        N.check(N.lib().kdn_build_omega(ctypes.c_void_p(bits.data_ptr()), d_k, D, ctypes.c_void_p(out.data_ptr()),
                                        _tag(dtype, "build_omega"), ctypes.c_void_p(_stream(device))),
                "kdn_build_omega")
    return out


def fwht(x: torch.Tensor) -> torch.Tensor:
    """Unnormalised natural-order FWHT along the last dimension (kdn_fwht)."""
    require_device(x, "fwht")
    n = x.shape[-1]
    x2 = _rows(x, n)
    out = torch.empty_like(x2)
    with torch.cuda.device(x.device):
        N.check(N.lib().kdn_fwht(ctypes.c_void_p(x2.data_ptr()), x2.shape[0], x2.stride(0), n,
                                 _tag(x.dtype, "fwht"), ctypes.c_void_p(out.data_ptr()), out.stride(0),
                                 ctypes.c_void_p(_stream(x.device))), "kdn_fwht")
    return out.view(x.shape)


def lift(x: torch.Tensor, omega_bf16: torch.Tensor, phase: torch.Tensor, inv_tau: float,
         normalize: bool = False, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """(..., d_k) -> (..., D) feature lift (kdn_fwht_lift)."""
    require_device(x, "lift")
    D, d_k = omega_bf16.shape
    if x.shape[-1] != d_k:
        raise ValueError(f"lift: last dimension {x.shape[-1]} != d_k {d_k}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    x2 = _rows(x, d_k)
    if (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    ph = phase.to(device=x.device, dtype=torch.float32).contiguous()
    om = omega_bf16.to(device=x.device).contiguous()
    out = torch.empty(x2.shape[0], D, dtype=out_dtype, device=x.device)
    with torch.cuda.device(x.device):
        N.check(N.lib().kdn_fwht_lift(ctypes.c_void_p(x2.data_ptr()), x2.shape[0], x2.stride(0),
                                      _tag(x.dtype, "lift"), 1 if normalize else 0,
                                      ctypes.c_void_p(om.data_ptr()), ctypes.c_void_p(ph.data_ptr()),
                                      d_k, D, float(inv_tau), ctypes.c_void_p(out.data_ptr()), out.stride(0),
                                      _tag(out_dtype, "lift output"), ctypes.c_void_p(_stream(x.device))),
                "kdn_fwht_lift")
    return out.view(*x.shape[:-1], D)


def lift_bits(x: torch.Tensor, rademacher_bits: torch.Tensor, phase: torch.Tensor, inv_tau: float,
              normalize: bool = False, out_dtype: Optional[torch.dtype] = None,
              butterfly: bool = False) -> torch.Tensor:
    """(..., 64) -> (..., D) feature lift from the packed [D/64, 3] sign table (kdn_fwht_lift_bits): each
    workgroup builds Omega in LDS with wave64 butterflies, then lifts as `lift`.  D = 64 * rows of the
    table; phase is the (D,) phase vector b.  butterfly=True projects every row by in-register wave64
    butterflies instead (kdn_fwht_lift_bits_butterfly, the reference's P3 design; slower)."""
    require_device(x, "lift_bits")
    d_k = x.shape[-1]
    D = 64 * rademacher_bits.shape[0]
    if rademacher_bits.dim() != 2 or rademacher_bits.shape[1] != 3 or phase.numel() != D:
        raise ValueError(f"lift_bits: expects rademacher_bits (D/64, 3) and phase (D,); got "
                         f"{tuple(rademacher_bits.shape)}, {tuple(phase.shape)}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    x2 = _rows(x, d_k)
    if (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    bits = rademacher_bits.to(device=x.device, dtype=torch.int64).contiguous()
    ph = phase.to(device=x.device, dtype=torch.float32).contiguous()
    out = torch.empty(x2.shape[0], D, dtype=out_dtype, device=x.device)
    name = "kdn_fwht_lift_bits_butterfly" if butterfly else "kdn_fwht_lift_bits"
    with torch.cuda.device(x.device):
        N.check(getattr(N.lib(), name)(ctypes.c_void_p(x2.data_ptr()), x2.shape[0], x2.stride(0),
                                       _tag(x.dtype, "lift_bits"), d_k, ctypes.c_void_p(bits.data_ptr()), D,
                                       float(inv_tau), ctypes.c_void_p(ph.data_ptr()), 1 if normalize else 0,
                                       ctypes.c_void_p(out.data_ptr()), out.stride(0),
                                       _tag(out_dtype, "lift_bits output"), ctypes.c_void_p(_stream(x.device))),
                name)
    return out.view(*x.shape[:-1], D)


def lift_factored(x: torch.Tensor, omega1: torch.Tensor, phase1: torch.Tensor, omega2: torch.Tensor,
                  phase2: torch.Tensor, inv_tau: float, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """(..., 128) -> (..., 1024) factored lift (kdn_fwht_lift_factored): the two halves of x lifted by the
    two 64 -> 512 projections, concatenated and renormalised (eps 1e-7)."""
    require_device(x, "lift_factored")
    if x.shape[-1] != 128 or tuple(omega1.shape) != (512, 64) or tuple(omega2.shape) != (512, 64):
        raise ValueError(f"lift_factored: expects x (..., 128) and two (512, 64) projections; got {tuple(x.shape)}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    x2 = _rows(x, 128)
    if (x2.stride(0) * x2.element_size()) % 16 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    dev = x.device
    o1, o2 = omega1.to(device=dev).contiguous(), omega2.to(device=dev).contiguous()
    p1 = phase1.to(device=dev, dtype=torch.float32).contiguous()
    p2 = phase2.to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty(x2.shape[0], 1024, dtype=out_dtype, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().kdn_fwht_lift_factored(
            ctypes.c_void_p(x2.data_ptr()), x2.shape[0], x2.stride(0), _tag(x.dtype, "lift_factored"),
            ctypes.c_void_p(o1.data_ptr()), ctypes.c_void_p(p1.data_ptr()), ctypes.c_void_p(o2.data_ptr()),
            ctypes.c_void_p(p2.data_ptr()), float(inv_tau), ctypes.c_void_p(out.data_ptr()), out.stride(0),
            _tag(out_dtype, "lift_factored output"), ctypes.c_void_p(_stream(dev))), "kdn_fwht_lift_factored")
    return out.view(*x.shape[:-1], 1024)


def lift_factored_backward(x: torch.Tensor, dphi: torch.Tensor, omega1: torch.Tensor, phase1: torch.Tensor,
                           omega2: torch.Tensor, phase2: torch.Tensor, inv_tau: float) -> torch.Tensor:
    """dL/dx (float32, x's shape) of lift_factored(x, ...) for dL/d(out) = dphi (..., 1024)
    (kdn_fwht_lift_factored_bwd; the lift is recomputed in fp32 from x)."""
    require_device(x, "lift_factored_backward")
    if x.shape[-1] != 128 or dphi.shape != (*x.shape[:-1], 1024):
        raise ValueError(f"lift_factored_backward: expects x (..., 128) and dphi (..., 1024); got {tuple(x.shape)}, "
                         f"{tuple(dphi.shape)}")
    dev = x.device
    x2 = _rows(x, 128)
    g2 = _rows(dphi.to(device=dev, dtype=torch.float32), 1024)
    if g2.data_ptr() % 16 or g2.stride(0) % 4:
        g2 = g2.contiguous()
    o1, o2 = omega1.to(device=dev).contiguous(), omega2.to(device=dev).contiguous()
    p1 = phase1.to(device=dev, dtype=torch.float32).contiguous()
    p2 = phase2.to(device=dev, dtype=torch.float32).contiguous()
    dx = torch.empty(x2.shape[0], 128, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        N.check(N.lib().kdn_fwht_lift_factored_bwd(
            ctypes.c_void_p(x2.data_ptr()), x2.shape[0], x2.stride(0), _tag(x.dtype, "lift_factored_backward"),
            ctypes.c_void_p(o1.data_ptr()), ctypes.c_void_p(p1.data_ptr()), ctypes.c_void_p(o2.data_ptr()),
            ctypes.c_void_p(p2.data_ptr()), float(inv_tau), ctypes.c_void_p(g2.data_ptr()), g2.stride(0),
            ctypes.c_void_p(dx.data_ptr()), dx.stride(0), ctypes.c_void_p(_stream(dev))), "kdn_fwht_lift_factored_bwd")
    return dx.view(*x.shape)


def _last_contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


# Update rules (kdn_scan_args.rule): the gated delta rule, and gated linear attention (no erasure term).
RULE_DELTA, RULE_LINEAR = 0, 1


class FeatureMap:
    """How the scan maps q, k to features (the feature-map fields of kdn_scan_args).

    - lifted=False (default): phi = sqrt(2/D) cos(x Omega_h^T inv_tau_h + phase_h), renormalised unless
      no_renorm.  Omega is `omega` (+ `omega_lo` when a bf16 Omega is not exact), either (D, d_k) shared
      by every head or (H, D, d_k) per head; phase is (D,) or (H, D); inv_tau_head is an optional (H,)
      float32 tensor overriding the scalar inv_tau.
    - lifted=True: q and k already are the (B, T, H, D) features; Omega and the phases are unused.
    """

    def __init__(self, omega=None, phase=None, omega_lo=None, inv_tau_head=None, no_renorm=False,
                 lifted=False):
        self.omega, self.phase, self.omega_lo = omega, phase, omega_lo
        self.inv_tau_head, self.no_renorm, self.lifted = inv_tau_head, bool(no_renorm), bool(lifted)

    def dim(self, q: torch.Tensor) -> int:
        return q.shape[-1] if self.lifted else self.omega.shape[-2]

    def keep(self):
        return (self.omega, self.phase, self.omega_lo, self.inv_tau_head)


def _head_stride(t: Optional[torch.Tensor], ndim_shared: int) -> int:
    return 0 if t is None or t.dim() == ndim_shared else t.stride(0)


def _fill_features(a: N.ScanArgs, fm: FeatureMap) -> None:
    a.feature_mode = 1 if fm.lifted else 0
    a.no_renorm = 1 if fm.no_renorm else 0
    if fm.lifted:
        a.omega_bf16, a.phase, a.omega_lo = None, None, None
        a.omega_head_stride = a.phase_head_stride = 0
    else:
        a.omega_bf16, a.phase = fm.omega.data_ptr(), fm.phase.data_ptr()
        a.omega_lo = fm.omega_lo.data_ptr() if fm.omega_lo is not None else None
        a.omega_head_stride = _head_stride(fm.omega, 2)
        a.phase_head_stride = _head_stride(fm.phase, 1)
    a.inv_tau_head = fm.inv_tau_head.data_ptr() if fm.inv_tau_head is not None else None


def scan_args(q, k, v, beta, decay, omega_bf16, phase, inv_tau, normalize, initial_state, final_state, y,
              workspace=None, segment_chunks: int = 0, features: Optional[FeatureMap] = None,
              rule: int = RULE_DELTA) -> N.ScanArgs:
    """Fill struct kdn_scan_args from (B, T, H, .) views.  `features` (if given) replaces
    omega_bf16/phase; `rule` is RULE_DELTA or RULE_LINEAR."""
    fm = features if features is not None else FeatureMap(omega_bf16, phase)
    B, T, H, d_k = q.shape
    d_v = v.shape[-1]
    a = N.ScanArgs()
    a.B, a.T, a.H = B, T, H
    a.d_k, a.D, a.d_v = d_k, fm.dim(q), d_v
    a.in_dtype = _tag(q.dtype, "scan inputs")
    a.out_dtype = _tag(y.dtype, "scan output")
    a.normalize_input = 1 if normalize else 0
    a.inv_tau = float(inv_tau)
    a.q, a.q_stride = q.data_ptr(), N._i64x3(*q.stride()[:3])
    a.k, a.k_stride = k.data_ptr(), N._i64x3(*k.stride()[:3])
    a.v, a.v_stride = v.data_ptr(), N._i64x3(*v.stride()[:3])
    a.beta, a.beta_stride = beta.data_ptr(), N._i64x3(*beta.stride())
    if decay is not None:
        a.decay, a.decay_stride = decay.data_ptr(), N._i64x3(*decay.stride())
    else:
        a.decay, a.decay_stride = None, N._i64x3(0, 0, 0)
    _fill_features(a, fm)
    if initial_state is not None:
        a.initial_state, a.init_stride = initial_state.data_ptr(), N._i64x4(*initial_state.stride())
    else:
        a.initial_state, a.init_stride = None, N._i64x4(0, 0, 0, 0)
    a.final_state, a.final_stride = final_state.data_ptr(), N._i64x4(*final_state.stride())
    a.y, a.y_stride = y.data_ptr(), N._i64x3(*y.stride()[:3])
    a.segment_chunks = int(segment_chunks)
    a.rule = int(rule)
    if workspace is not None:
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    else:
        a.workspace, a.workspace_bytes = None, 0
    return a


def scan_workspace_bytes(q, v, omega_bf16, segment_chunks: int = 0, pipelined: bool = False,
                         features: Optional[FeatureMap] = None) -> int:
    B, T, H, d_k = q.shape
    a = N.ScanArgs()
    D = features.dim(q) if features is not None else omega_bf16.shape[-2]
    a.B, a.T, a.H, a.d_k, a.D, a.d_v = B, T, H, d_k, D, v.shape[-1]
    a.feature_mode = 1 if (features is not None and features.lifted) else 0
    if features is not None:
        _fill_features(a, features)  # D < 512: the replicated tables' size follows the heads and low parts
    a.in_dtype = _tag(q.dtype, "scan inputs")
    a.out_dtype = a.in_dtype
    a.inv_tau = 1.0
    a.segment_chunks = int(segment_chunks)
    fn = N.lib().kdn_scan_workspace_bytes_pipelined if pipelined else N.lib().kdn_scan_workspace_bytes
    return int(fn(ctypes.byref(a)))


_AUX_STREAMS = {}


def aux_stream(dev: torch.device, which: int = 0) -> torch.cuda.Stream:
    """Auxiliary stream `which` of a device (0: prep kernels, 1: output kernels of the pipelined scan),
    created once, default priority."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _AUX_STREAMS.get((idx, which))
    if st is None:
        st = torch.cuda.Stream(device=idx)
        _AUX_STREAMS[(idx, which)] = st
    return st


def _launch_scan(a, dev: torch.device, pipelined: bool, keep=()):
    """kdn_delta_scan_fwd, or the pipelined three-stream variant (kdn_delta_scan_fwd_streams: prep and
    output on two auxiliary streams).  Tensors the auxiliary streams read or write are marked with
    record_stream so the caching allocator does not hand their memory out again before that work ends."""
    st = torch.cuda.current_stream(dev)
    if pipelined:
        aux_p, aux_o = aux_stream(dev, 0), aux_stream(dev, 1)
        for t in keep:
            if t is not None:
                t.record_stream(aux_p)
                t.record_stream(aux_o)
        N.check(N.lib().kdn_delta_scan_fwd_streams(ctypes.byref(a), ctypes.c_void_p(st.cuda_stream),
                                                   ctypes.c_void_p(aux_p.cuda_stream),
                                                   ctypes.c_void_p(aux_o.cuda_stream)), "kdn_delta_scan_fwd_streams")
    else:
        N.check(N.lib().kdn_delta_scan_fwd(ctypes.byref(a), ctypes.c_void_p(st.cuda_stream)), "kdn_delta_scan_fwd")


def scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, decay: Optional[torch.Tensor],
         omega_bf16: torch.Tensor, phase: torch.Tensor, inv_tau: float, normalize: bool = False,
         initial_state: Optional[torch.Tensor] = None, final_state: Optional[torch.Tensor] = None,
         y: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
         workspace: Optional[torch.Tensor] = None, segment_chunks: int = 0,
         pipelined: bool = True, features: Optional[FeatureMap] = None,
         rule: int = RULE_DELTA) -> Tuple[torch.Tensor, torch.Tensor]:
    """Chunked delta-rule prefill over (B, T, H, d) views (kdn_delta_scan_fwd_streams: the state chain on
    the current stream, prep and output on two auxiliary streams; kdn_delta_scan_fwd with pipelined=False).

    q, k (B, T, H, d_k) and v (B, T, H, d_v) share a dtype; beta, decay (B, T, H) are float32 (decay may
    be None for lambda = 1); initial_state/final_state are (B, H, D, d_v) float32 views with any strides.
    `features` selects another feature map (per-head or hi + lo Omega, no renormalisation, pre-lifted
    q, k); omega_bf16/phase are then ignored.  rule=RULE_LINEAR drops the erasure term
    (S_t = lambda_t S_{t-1} + beta_t v_t phi_k^T).  Returns (y (B, T, H, d_v), final_state).
    """
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta")):
        require_device(t, nm)
    dev = q.device
    if q.dim() != 4 or k.shape != q.shape or v.shape[:3] != q.shape[:3] or beta.shape != q.shape[:3]:
        raise ValueError(f"scan: shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} beta{tuple(beta.shape)}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("scan: q, k and v must share a dtype")
    q, k, v = _last_contig(q), _last_contig(k), _last_contig(v)
    beta = beta.to(torch.float32)
    if decay is not None:
        if decay.shape != beta.shape:
            raise ValueError("scan: decay must have the shape of beta")
        decay = decay.to(device=dev, dtype=torch.float32)
    B, T, H, _ = q.shape
    if features is None:
        features = FeatureMap(omega_bf16, phase)
    features = _features_on(features, dev, H)
    D = features.dim(q)
    d_v = v.shape[-1]
    if initial_state is not None:
        if tuple(initial_state.shape) != (B, H, D, d_v):
            raise ValueError(f"scan: initial_state must be (B, H, D, d_v) = {(B, H, D, d_v)}")
        initial_state = initial_state.to(device=dev, dtype=torch.float32)
    if final_state is None:
        final_state = torch.empty(B, H, D, d_v, device=dev, dtype=torch.float32)
    if y is None:
        y = torch.empty(B, T, H, d_v, device=dev, dtype=q.dtype if out_dtype is None else out_dtype)
    if workspace is None:
        nbytes = scan_workspace_bytes(q, v, None, segment_chunks, pipelined, features)
        if nbytes == 0:
            raise ValueError("scan: unsupported shape (kdn_scan_workspace_bytes returned 0)")
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    a = scan_args(q, k, v, beta, decay, None, None, inv_tau, normalize, initial_state, final_state, y,
                  workspace, segment_chunks, features, rule)
    with torch.cuda.device(dev):
        _launch_scan(a, dev, pipelined, (q, k, v, beta, decay, initial_state, final_state, y, workspace)
                     + features.keep())
    return y, final_state


class ScanBackwardPlan:
    """One backward call of the scan (kdn_delta_scan_bwd) with its arguments, outputs and workspace
    prepared once: run() issues the whole backward; phase(0) the start of a call (the checkpoint pass)
    and phase(i, s) for i = 1 .. 4 one launch of segment s (1 per-chunk recompute, 2 forward carry,
    3 reverse carry, 4 gradients), e.g. for timing: phase 0, then for s from segments - 1 down to 0
    phases 1, 2, 3, 4.

    Same layouts as `scan`: q, k (B, T, H, 64), v and dy (B, T, H, 64), beta and decay (B, T, H), states
    (B, H, 512, 64); dL/dy = dy, dL/d(final state) = d_final_state (None: zero).  `outputs` holds the
    float32 gradients (dq, dk, dv, dbeta, ddecay or None, d_initial_state or None).  The feature map is
    one shared Omega (omega_bf16, phase, inv_tau) or `features` (per-head Omega with low parts, phases and
    1/tau, no renormalisation; not pre-lifted features); `rule` is RULE_DELTA or RULE_LINEAR.  With
    need_dinv_tau, `dinv_tau` holds dL/d(1/tau) per head (H,) in float32.  segment_chunks (0: the
    library's default) sets the backward's segment length in 64-token chunks; `segments` and
    `segment_chunks` hold the schedule."""

    def __init__(self, q, k, v, beta, decay, omega_bf16, phase, inv_tau, dy, d_final_state=None,
                 normalize: bool = False, initial_state=None, need_ddecay: bool = True, need_dinit: bool = True,
                 workspace: Optional[torch.Tensor] = None, segment_chunks: int = 0,
                 features: Optional[FeatureMap] = None, rule: int = RULE_DELTA, need_dinv_tau: bool = False):
        for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta"), (dy, "dy")):
            require_device(t, f"scan_backward: {nm}")
        dev = q.device
        if q.dim() != 4 or k.shape != q.shape or v.shape[:3] != q.shape[:3] or beta.shape != q.shape[:3] \
                or dy.shape != v.shape:
            raise ValueError(f"scan_backward: shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} "
                             f"beta{tuple(beta.shape)} dy{tuple(dy.shape)}")
        if k.dtype != q.dtype or v.dtype != q.dtype:
            raise TypeError("scan_backward: q, k and v must share a dtype")
        q, k, v = _last_contig(q), _last_contig(k), _last_contig(v)
        beta = beta.to(torch.float32)
        if decay is not None:
            decay = decay.to(device=dev, dtype=torch.float32)
        dy = _last_contig(dy.to(torch.float32))
        B, T, H, d_k = q.shape
        d_v = v.shape[-1]
        fm = _features_on(features if features is not None else FeatureMap(omega_bf16, phase), dev, H)
        if fm.lifted and d_k != 1024:
            raise ValueError("scan_backward: pre-lifted features have a backward at D = 1024 only (the factored path)")
        D = fm.dim(q)
        if initial_state is not None:
            if tuple(initial_state.shape) != (B, H, D, d_v):
                raise ValueError(f"scan_backward: initial_state must be (B, H, D, d_v) = {(B, H, D, d_v)}")
            initial_state = initial_state.to(device=dev, dtype=torch.float32)
        if d_final_state is not None:
            d_final_state = d_final_state.to(device=dev, dtype=torch.float32)
            if tuple(d_final_state.shape) != (B, H, D, d_v):
                raise ValueError(f"scan_backward: d_final_state must be (B, H, D, d_v) = {(B, H, D, d_v)}")
        unused = torch.empty(1, device=dev, dtype=torch.float32).expand(B, H, D, d_v)  # fwd.final_state (ignored)
        if segment_chunks < 0:
            raise ValueError("scan_backward: segment_chunks must be >= 0")
        self._fa = scan_args(q, k, v, beta, decay, None, None, inv_tau, normalize, initial_state, unused, dy, None,
                             segment_chunks, fm, rule)
        f32 = dict(device=dev, dtype=torch.float32)
        dq, dk = torch.empty(B, T, H, d_k, **f32), torch.empty(B, T, H, d_k, **f32)
        dv, dbeta = torch.empty(B, T, H, d_v, **f32), torch.empty(B, T, H, **f32)
        ddecay = torch.empty(B, T, H, **f32) if (decay is not None and need_ddecay) else None
        dinit = torch.empty(B, H, D, d_v, **f32) if need_dinit else None
        a = N.ScanBwdArgs()
        a.fwd = ctypes.addressof(self._fa)
        a.dy, a.dy_stride = dy.data_ptr(), N._i64x3(*dy.stride()[:3])
        if d_final_state is not None:
            a.d_final_state, a.dfinal_stride = d_final_state.data_ptr(), N._i64x4(*d_final_state.stride())
        for nm, t in (("dq", dq), ("dk", dk), ("dv", dv)):
            setattr(a, nm, t.data_ptr())
            setattr(a, nm + "_stride", N._i64x3(*t.stride()[:3]))
        a.dbeta, a.dbeta_stride = dbeta.data_ptr(), N._i64x3(*dbeta.stride())
        if ddecay is not None:
            a.ddecay, a.ddecay_stride = ddecay.data_ptr(), N._i64x3(*ddecay.stride())
        if dinit is not None:
            a.d_initial_state, a.dinit_stride = dinit.data_ptr(), N._i64x4(*dinit.stride())
        self.dinv_tau = torch.empty(H, **f32) if need_dinv_tau else None
        if self.dinv_tau is not None:
            a.dinv_tau = self.dinv_tau.data_ptr()
        nbytes = N.lib().kdn_scan_bwd_workspace_bytes(ctypes.byref(a))
        if nbytes == 0:
            raise ValueError("scan_backward: unsupported request (kdn_scan_bwd_workspace_bytes returned 0; the "
                             "backward covers d_k = 64, D = 512, d_v 16, 32, 64 or 128 with lifted features and D = 1024 "
                             "pre-lifted features with d_v 64 or 128)")
        if workspace is None or workspace.numel() * workspace.element_size() < nbytes:
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        seg = ctypes.c_int64(0)
        self.segments = int(N.lib().kdn_scan_bwd_segments(ctypes.byref(a), ctypes.byref(seg)))
        self.segment_chunks = int(seg.value)
        self.args, self.device, self.workspace = a, dev, workspace
        self.outputs = (dq, dk, dv, dbeta, ddecay, dinit)
        self.shape = (B, T, H)
        self._keep = (q, k, v, beta, decay, dy, d_final_state, initial_state, unused, fm.keep(), self.dinv_tau)

    def _st(self, stream):
        return stream if stream is not None else torch.cuda.current_stream(self.device)

    def _tensors(self):
        out, todo = [], [self._keep, self.outputs, self.workspace]
        while todo:
            t = todo.pop()
            if isinstance(t, torch.Tensor):
                out.append(t)
            elif isinstance(t, (tuple, list)):
                todo.extend(t)
        return out

    def run(self, stream=None, concurrent_carries: bool = True):
        """Issues the whole backward on `stream` (default: the current stream).  With
        concurrent_carries the reverse carries run back to back on `stream` while the device's auxiliary
        stream 0 runs the other launches around them (kdn_delta_scan_bwd_streams), else every launch runs
        in order on `stream` (kdn_delta_scan_bwd).  The results are the same bit for bit."""
        st = self._st(stream)
        with torch.cuda.device(self.device):
            if concurrent_carries:
                aux = aux_stream(self.device, 0)
                for t in self._tensors():
                    t.record_stream(aux)
                N.check(N.lib().kdn_delta_scan_bwd_streams(ctypes.byref(self.args), ctypes.c_void_p(st.cuda_stream),
                                                           ctypes.c_void_p(aux.cuda_stream)),
                        "kdn_delta_scan_bwd_streams")
            else:
                N.check(N.lib().kdn_delta_scan_bwd(ctypes.byref(self.args), ctypes.c_void_p(st.cuda_stream)),
                        "kdn_delta_scan_bwd")
        return self.outputs

    def phase(self, i: int, segment: int = 0, stream=None):
        st = self._st(stream)
        with torch.cuda.device(self.device):
            N.check(N.lib().kdn_scan_bwd_phase(ctypes.byref(self.args), int(i), int(segment),
                                               ctypes.c_void_p(st.cuda_stream)), "kdn_scan_bwd_phase")


def scan_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                  decay: Optional[torch.Tensor], omega_bf16: torch.Tensor, phase: torch.Tensor, inv_tau: float,
                  dy: torch.Tensor, d_final_state: Optional[torch.Tensor] = None, normalize: bool = False,
                  initial_state: Optional[torch.Tensor] = None, need_ddecay: bool = True,
                  need_dinit: bool = True, workspace: Optional[torch.Tensor] = None, segment_chunks: int = 0,
                  concurrent_carries: bool = True):
    """Gradients of `scan` (kdn_delta_scan_bwd) for the loss with dL/dy = dy and dL/d(final state) =
    d_final_state (None: zero); see ScanBackwardPlan for layouts and segment_chunks.  Returns float32
    (dq, dk, dv, dbeta, ddecay or None, d_initial_state or None)."""
    return ScanBackwardPlan(q, k, v, beta, decay, omega_bf16, phase, inv_tau, dy, d_final_state, normalize,
                            initial_state, need_ddecay, need_dinit, workspace,
                            segment_chunks).run(concurrent_carries=concurrent_carries)


class _Scan(torch.autograd.Function):
    """`scan` with its backward (kdn_delta_scan_bwd); the autograd node of the differentiable surfaces."""

    @staticmethod
    def forward(ctx, q, k, v, beta, decay, initial_state, omega_bf16, phase, inv_tau, normalize):
        y, final = scan(q, k, v, beta, decay, omega_bf16, phase, inv_tau, normalize=normalize,
                        initial_state=initial_state)
        ctx.save_for_backward(q, k, v, beta, decay, initial_state, omega_bf16, phase)
        ctx.inv_tau, ctx.normalize = inv_tau, normalize
        return y, final

    @staticmethod
    def backward(ctx, dy, dfinal):
        q, k, v, beta, decay, init, omega_bf16, phase = ctx.saved_tensors
        need = ctx.needs_input_grad
        dq, dk, dv, dbeta, ddecay, dinit = scan_backward(
            q, k, v, beta, decay, omega_bf16, phase, ctx.inv_tau, dy, dfinal, normalize=ctx.normalize,
            initial_state=init, need_ddecay=bool(need[4]), need_dinit=bool(need[5]))
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dbeta.to(beta.dtype),
                None if ddecay is None else ddecay.to(decay.dtype),
                None if dinit is None or init is None else dinit.to(init.dtype), None, None, None, None)


def scan_autograd(q, k, v, beta, decay, omega_bf16, phase, inv_tau, normalize: bool = False,
                  initial_state: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """`scan` (default schedule) recorded for autograd: gradients flow to q, k, v, beta, decay and
    initial_state through kdn_delta_scan_bwd.  Returns (y (B, T, H, d_v), final_state (B, H, D, d_v)).
    The backward covers d_k = 64, D in {128, 256, 512}, d_v in {16, 32, 64, 128}; other shapes are rejected
    here, before the forward runs, rather than inside .backward()."""
    d_k, D, d_v = q.shape[-1], omega_bf16.shape[-2], v.shape[-1]
    if d_k != 64 or D not in (128, 256, 512) or d_v not in (16, 32, 64, 128):
        raise ValueError(f"scan with gradients: the backward supports d_k = 64, D in 128, 256, 512, d_v in 16, 32, "
                         f"64, 128 "
                         f"(got d_k = {d_k}, D = {D}, d_v = {d_v}); run the forward under torch.no_grad() or detach "
                         f"the inputs")
    return _Scan.apply(q, k, v, beta, decay, initial_state, omega_bf16, phase, inv_tau, normalize)


class _FeatureScan(torch.autograd.Function):
    """`scan` with a per-head feature map and its backward (kdn_delta_scan_bwd): gradients flow to q, k,
    v, beta, decay, initial_state and the per-head 1/tau; Omega, its low parts and the phases are
    constants (buffers on the reference's surfaces)."""

    @staticmethod
    def forward(ctx, q, k, v, beta, decay, initial_state, inv_tau_head, omega, omega_lo, phase, no_renorm,
                normalize, rule):
        fm = FeatureMap(omega=omega, phase=phase, omega_lo=omega_lo, inv_tau_head=inv_tau_head.detach(),
                        no_renorm=no_renorm)
        y, final = scan(q, k, v, beta, decay, None, None, 1.0, normalize=normalize, initial_state=initial_state,
                        features=fm, rule=rule)
        ctx.save_for_backward(q, k, v, beta, decay, initial_state, inv_tau_head, omega, omega_lo, phase)
        ctx.flags = (no_renorm, normalize, rule)
        return y, final

    @staticmethod
    def backward(ctx, dy, dfinal):
        q, k, v, beta, decay, init, itau, omega, omega_lo, phase = ctx.saved_tensors
        no_renorm, normalize, rule = ctx.flags
        need = ctx.needs_input_grad
        fm = FeatureMap(omega=omega, phase=phase, omega_lo=omega_lo, inv_tau_head=itau.detach(), no_renorm=no_renorm)
        plan = ScanBackwardPlan(q, k, v, beta, decay, None, None, 1.0, dy, dfinal, normalize=normalize,
                                initial_state=init, need_ddecay=decay is not None and bool(need[4]),
                                need_dinit=init is not None and bool(need[5]), features=fm, rule=rule,
                                need_dinv_tau=bool(need[6]))
        dq, dk, dv, dbeta, ddecay, dinit = plan.run()
        ditau = None if plan.dinv_tau is None else plan.dinv_tau.to(itau.dtype)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dbeta.to(beta.dtype),
                None if ddecay is None else ddecay.to(decay.dtype),
                None if dinit is None else dinit.to(init.dtype), ditau, None, None, None, None, None, None)


def feature_scan_autograd(q, k, v, beta, decay, omega, phase, inv_tau_head, omega_lo=None, no_renorm: bool = False,
                          normalize: bool = False, initial_state=None, rule: int = RULE_DELTA
                          ) -> Tuple[torch.Tensor, torch.Tensor]:
    """`scan` over (B, T, H, .) views with a per-head feature map, recorded for autograd (gradients through
    kdn_delta_scan_bwd to q, k, v, beta, decay, initial_state and inv_tau_head (H,)).  omega (H, D, 64)
    bf16 with optional bf16 low parts, phase (H, D), the delta or the linear rule; d_k = 64, D in {128, 256,
    512}, d_v in {16, 32, 64, 128}.  Returns (y (B, T, H, d_v), final_state (B, H, D, d_v))."""
    d_k, D, d_v = q.shape[-1], omega.shape[-2], v.shape[-1]
    if d_k != 64 or D not in (128, 256, 512) or d_v not in (16, 32, 64, 128):
        raise ValueError(f"scan with gradients: the backward supports d_k = 64, D in 128, 256, 512, d_v in 16, 32, "
                         f"64, 128 "
                         f"(got d_k = {d_k}, D = {D}, d_v = {d_v}); run the forward under torch.no_grad() or detach "
                         f"the inputs")
    return _FeatureScan.apply(q, k, v, beta, decay, initial_state, inv_tau_head, omega, omega_lo, phase,
                              bool(no_renorm), bool(normalize), int(rule))


def _features_on(fm: FeatureMap, dev: torch.device, H: int) -> FeatureMap:
    """The feature map with its tensors on `dev` in the layouts the library reads (bf16 Omega rows
    and float32 phases / 1/tau, innermost dimension contiguous), shapes checked."""
    if fm.lifted:
        return FeatureMap(inv_tau_head=None, lifted=True)

    def per_head(t, ndim, what):
        if t.dim() == ndim + 1 and t.shape[0] != H:
            raise ValueError(f"scan: per-head {what} must have H = {H} rows, got {tuple(t.shape)}")
        if t.dim() not in (ndim, ndim + 1):
            raise ValueError(f"scan: {what} has shape {tuple(t.shape)}")

    for t, nm in ((fm.omega, "omega"), (fm.omega_lo, "omega_lo")):
        if t is not None:
            per_head(t, 2, nm)
            if t.dtype != torch.bfloat16:
                raise TypeError(f"scan: {nm} must be bfloat16")
    per_head(fm.phase, 1, "phase")
    if fm.omega_lo is not None and fm.omega_lo.shape != fm.omega.shape:
        raise ValueError("scan: omega_lo must have the shape of omega")
    itau = fm.inv_tau_head
    if itau is not None and tuple(itau.shape) != (H,):
        raise ValueError(f"scan: inv_tau_head must be ({H},)")
    return FeatureMap(fm.omega.to(dev).contiguous(), fm.phase.to(device=dev, dtype=torch.float32).contiguous(),
                      None if fm.omega_lo is None else fm.omega_lo.to(dev).contiguous(),
                      None if itau is None else itau.to(device=dev, dtype=torch.float32).contiguous(),
                      fm.no_renorm, False)


SCHEDULE_SPLIT, SCHEDULE_FUSED, SCHEDULE_GENERAL = 0, 1, 2  # kdn_scan_schedule (include/kdn.h)


class ScanPlan:
    """Reusable launch description for repeated prefills of one shape (benchmarks, serving loops).

    Holds the filled kdn_scan_args, the workspace for one segment of `segment_chunks` chunks and the
    tensors the arguments point into, so each run is only the native calls.  `run()` is
    kdn_delta_scan_fwd (or the pipelined variant); `schedule` is the schedule it runs (kdn_scan_schedule:
    SCHEDULE_SPLIT or SCHEDULE_FUSED) and `prep()` / `state()` / `output()` (split) or `prep_fused()` /
    `chain()` (fused) launch that schedule's phases of one segment.
    """

    def __init__(self, q, k, v, beta, decay, omega_bf16, phase, inv_tau, normalize=False, initial_state=None,
                 out_dtype=None, segment_chunks: int = 0, pipelined: bool = False):
        dev = q.device
        B, T, H, _ = q.shape
        D, d_v = omega_bf16.shape[0], v.shape[-1]
        self.nchunks = (T + 63) // 64
        self.pipelined = pipelined
        self.q, self.k, self.v = _last_contig(q), _last_contig(k), _last_contig(v)
        self.beta = beta.to(torch.float32)
        self.decay = None if decay is None else decay.to(torch.float32)
        self.omega = omega_bf16.to(dev).contiguous()
        self.phase = phase.to(device=dev, dtype=torch.float32).contiguous()
        self.initial_state = initial_state
        self.final_state = torch.empty(B, H, D, d_v, device=dev, dtype=torch.float32)
        self.y = torch.empty(B, T, H, d_v, device=dev, dtype=q.dtype if out_dtype is None else out_dtype)
        # the library's segment length for this shape (its default when segment_chunks is 0)
        probe = scan_args(self.q, self.k, self.v, self.beta, self.decay, self.omega, self.phase, inv_tau, normalize,
                          initial_state, self.final_state, self.y, None, segment_chunks)
        with torch.cuda.device(dev):
            self.segment_chunks = int(N.lib().kdn_scan_segment_chunks(ctypes.byref(probe), 1 if pipelined else 0))
            self.schedule = int(N.lib().kdn_scan_schedule(ctypes.byref(probe)))
        if self.segment_chunks <= 0 or self.schedule < 0:
            raise ValueError("ScanPlan: unsupported shape")
        nbytes = scan_workspace_bytes(self.q, self.v, self.omega, self.segment_chunks, pipelined)
        if nbytes == 0:
            raise ValueError("ScanPlan: unsupported shape")
        self.seg_bytes = scan_workspace_bytes(self.q, self.v, self.omega, self.segment_chunks, False)
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        self.args = scan_args(self.q, self.k, self.v, self.beta, self.decay, self.omega, self.phase, inv_tau,
                              normalize, initial_state, self.final_state, self.y, self.workspace, self.segment_chunks)
        self.device = dev

    def _stream(self):
        return ctypes.c_void_p(_stream(self.device))

    def run(self):
        _launch_scan(self.args, self.device, self.pipelined)
        return self.y, self.final_state

    def segment_args(self, s: int) -> N.ScanArgs:
        """Arguments whose workspace is buffer (s mod nbuf) of the pipelined layout (for phase-by-phase
        scheduling of segment s)."""
        a = N.ScanArgs.from_buffer_copy(self.args)
        nbuf = max(1, self.workspace.numel() // self.seg_bytes)
        a.workspace = self.workspace.data_ptr() + (s % nbuf) * self.seg_bytes
        a.workspace_bytes = self.seg_bytes
        return a

    def prep(self, chunk0: int, nchunks: int, args: Optional[N.ScanArgs] = None, stream=None):
        self._phase("kdn_scan_prep", chunk0, nchunks, args, stream)

    def state(self, chunk0: int, nchunks: int, args: Optional[N.ScanArgs] = None, stream=None):
        self._phase("kdn_scan_state", chunk0, nchunks, args, stream)

    def output(self, chunk0: int, nchunks: int, args: Optional[N.ScanArgs] = None, stream=None):
        self._phase("kdn_scan_output", chunk0, nchunks, args, stream)

    def prep_fused(self, chunk0: int, nchunks: int, args: Optional[N.ScanArgs] = None, stream=None):
        self._phase("kdn_scan_prep_fused", chunk0, nchunks, args, stream)

    def chain(self, chunk0: int, nchunks: int, args: Optional[N.ScanArgs] = None, stream=None):
        self._phase("kdn_scan_chain", chunk0, nchunks, args, stream)

    def _phase(self, name, chunk0, nchunks, args, stream):
        a = self.args if args is None else args
        st = self._stream() if stream is None else ctypes.c_void_p(stream.cuda_stream)
        N.check(getattr(N.lib(), name)(ctypes.byref(a), chunk0, nchunks, st), name)



class _ForwardOnly(torch.autograd.Function):
    """Identity on the scan outputs that ties them to the inputs' autograd graph; its backward raises,
    so a training step fails loudly instead of computing gradients that skip the scan."""

    @staticmethod
    def forward(ctx, what, n_out, *tensors):
        ctx.what = what
        return tuple(t.view_as(t) for t in tensors[:n_out])

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(f"{ctx.what}: the backward pass of the scan is not implemented on MI355X "
                                  "(forward/prefill only)")


def forward_only(what: str, outputs, inputs):
    """`outputs` unchanged when no input needs a gradient; otherwise views of them whose backward raises."""
    if not torch.is_grad_enabled() or not any(isinstance(t, torch.Tensor) and t.requires_grad for t in inputs):
        return tuple(outputs)
    grads = [t for t in inputs if isinstance(t, torch.Tensor) and t.requires_grad]
    return _ForwardOnly.apply(what, len(outputs), *outputs, *grads)


# ------------------------------------------------------------------------------------------------ serving


def check_host_slots(slots, n_slots: int) -> None:
    """Rejects per-sequence state slots given on the host that the step must not run with: a slot at or
    above n_slots, or a slot shared by two sequences (they would race).  Negative slots are padding.
    (Device slots are not checked here, which would synchronise; the kernels skip out-of-range ones.)"""
    sl = torch.as_tensor(slots, dtype=torch.int64).reshape(-1)
    if sl.numel() and int(sl.max()) >= n_slots:
        raise ValueError(f"ragged_step: slot {int(sl.max())} is outside the {n_slots} state slots")
    live = sl[sl >= 0]
    if torch.unique(live).numel() != live.numel():
        raise ValueError("ragged_step: two sequences of one step share a state slot")


def _ragged_args(q, k, v, beta, decay, cu_seqlens, slots, states, omega_bf16, phase, inv_tau, normalize, rule, y,
                 out_dtype, cu_seqlens_device):
    """Checks the arguments of a ragged step and fills kdn_ragged_args; returns (args, tensors it points to)."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta"), (states, "states")):
        require_device(t, f"ragged_step: {nm}")
    dev = q.device
    if q.dim() != 3 or k.shape != q.shape or v.dim() != 3 or v.shape[:2] != q.shape[:2] or beta.shape != q.shape[:2]:
        raise ValueError(f"ragged_step: shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} beta{tuple(beta.shape)}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("ragged_step: q, k and v must share a dtype")
    if states.dtype != torch.float32 or states.dim() != 4:
        raise TypeError("ragged_step: states must be a float32 (slots, H, D, d_v) tensor")
    cu_host = torch.as_tensor(cu_seqlens, dtype=torch.int64).cpu().contiguous()
    n = cu_host.numel() - 1
    if n < 0 or int(cu_host[-1]) > q.shape[0]:
        raise ValueError("ragged_step: cu_seqlens must hold num_seqs + 1 offsets within the token count")
    n_slots = states.shape[0]
    if not (isinstance(slots, torch.Tensor) and slots.is_cuda):
        check_host_slots(slots, n_slots)
    slots_d = torch.as_tensor(slots).to(device=dev, dtype=torch.int32).contiguous()
    if slots_d.numel() != n:
        raise ValueError("ragged_step: one slot per sequence")
    if cu_seqlens_device is not None:
        if cu_seqlens_device.device != dev or cu_seqlens_device.dtype != torch.int64 or cu_seqlens_device.numel() != n + 1:
            raise ValueError("ragged_step: cu_seqlens_device must be the int64 offsets on the inputs' device")
        cu_d = cu_seqlens_device.contiguous()
    else:
        cu_d = cu_host.to(dev)
    q, k, v = _last_contig(q), _last_contig(k), _last_contig(v)
    beta = beta.to(torch.float32)
    if decay is not None:
        decay = decay.to(device=dev, dtype=torch.float32)
    T, H = q.shape[:2]
    d_v = v.shape[-1]
    if y is None:
        y = torch.empty(T, H, d_v, device=dev, dtype=q.dtype if out_dtype is None else out_dtype)
    om = omega_bf16.to(dev).contiguous()
    ph = phase.to(device=dev, dtype=torch.float32).contiguous()
    a = N.RaggedArgs()
    a.num_seqs, a.H = n, H
    a.d_k, a.D, a.d_v = q.shape[-1], om.shape[0], d_v
    a.in_dtype, a.out_dtype = _tag(q.dtype, "ragged inputs"), _tag(y.dtype, "ragged output")
    a.normalize_input, a.rule, a.inv_tau = 1 if normalize else 0, int(rule), float(inv_tau)
    a.cu_seqlens, a.cu_seqlens_host, a.slots = cu_d.data_ptr(), cu_host.data_ptr(), slots_d.data_ptr()
    a.q, a.q_stride = q.data_ptr(), N._i64x2(*q.stride()[:2])
    a.k, a.k_stride = k.data_ptr(), N._i64x2(*k.stride()[:2])
    a.v, a.v_stride = v.data_ptr(), N._i64x2(*v.stride()[:2])
    a.beta, a.beta_stride = beta.data_ptr(), N._i64x2(*beta.stride())
    if decay is not None:
        a.decay, a.decay_stride = decay.data_ptr(), N._i64x2(*decay.stride())
    a.omega_bf16, a.phase = om.data_ptr(), ph.data_ptr()
    a.states, a.state_stride = states.data_ptr(), N._i64x4(*states.stride())
    a.y, a.y_stride = y.data_ptr(), N._i64x2(*y.stride()[:2])
    a.num_slots = n_slots
    return a, (q, k, v, beta, decay, om, ph, states, y, cu_d, slots_d, cu_host)


def ragged_workspace_bytes(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                           decay: Optional[torch.Tensor], cu_seqlens, slots: torch.Tensor, states: torch.Tensor,
                           omega_bf16: torch.Tensor, phase: torch.Tensor, inv_tau: float, normalize: bool = False,
                           rule: int = RULE_DELTA, y: Optional[torch.Tensor] = None,
                           out_dtype: Optional[torch.dtype] = None,
                           cu_seqlens_device: Optional[torch.Tensor] = None) -> int:
    """Bytes of workspace that ragged_step needs for these arguments (kdn_ragged_workspace_bytes).  A serving
    loop allocates it once for its largest step and passes it as ragged_step(workspace=...), so that no
    call allocates device memory."""
    a, _ = _ragged_args(q, k, v, beta, decay, cu_seqlens, slots, states, omega_bf16, phase, inv_tau, normalize, rule,
                        y, out_dtype, cu_seqlens_device)
    need = int(N.lib().kdn_ragged_workspace_bytes(ctypes.byref(a)))
    if need == 0:
        raise ValueError("ragged_step: unsupported shape (kdn_ragged_workspace_bytes returned 0)")
    return need


def ragged_step(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, decay: Optional[torch.Tensor],
                cu_seqlens, slots: torch.Tensor, states: torch.Tensor, omega_bf16: torch.Tensor, phase: torch.Tensor,
                inv_tau: float, normalize: bool = False, rule: int = RULE_DELTA, y: Optional[torch.Tensor] = None,
                out_dtype: Optional[torch.dtype] = None, workspace: Optional[torch.Tensor] = None,
                pipelined: bool = True, cu_seqlens_device: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One ragged mixed prefill + decode step (kdn_ragged_step).

    q, k (tokens, H, d_k) and v (tokens, H, d_v) share a dtype; beta, decay (tokens, H) float32 (decay may
    be None); cu_seqlens: num_seqs + 1 token offsets (host list/array or tensor); slots (num_seqs,) the
    distinct state slots; states (slots_total, H, D, d_v) float32, any strides, updated in place.
    A negative slot marks a padding sequence: it is skipped (no state touched, its y rows left as they
    are).  Slots given on the host are checked (range, distinctness) before anything is launched.
    A serving loop that keeps its batch metadata on the device passes slots as a device int32 tensor and
    cu_seqlens_device (the same offsets as cu_seqlens, device int64); nothing is then copied to the device
    per call, and the kernels skip any sequence whose slot is outside the slab instead of checking on the
    host (which would synchronise).
    Without `workspace` each call allocates one (ragged_workspace_bytes; several GB for long prefills)
    from torch's caching allocator; a loop passes one buffer instead.
    Returns y (tokens, H, d_v).
    """
    a, keep = _ragged_args(q, k, v, beta, decay, cu_seqlens, slots, states, omega_bf16, phase, inv_tau, normalize,
                           rule, y, out_dtype, cu_seqlens_device)
    dev = q.device
    y = keep[8]
    need = int(N.lib().kdn_ragged_workspace_bytes(ctypes.byref(a)))
    if need == 0:
        raise ValueError("ragged_step: unsupported shape (kdn_ragged_workspace_bytes returned 0)")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    st = torch.cuda.current_stream(dev)
    with torch.cuda.device(dev):
        aux = None
        if pipelined:
            aux = aux_stream(dev)
            for t in keep[:11] + (workspace,):
                if t is not None:
                    t.record_stream(aux)
        N.check(N.lib().kdn_ragged_step(ctypes.byref(a), ctypes.c_void_p(st.cuda_stream),
                                        ctypes.c_void_p(aux.cuda_stream) if aux is not None else None),
                "kdn_ragged_step")
    return y


def slot_step(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, decay: Optional[torch.Tensor],
              slot_mapping: torch.Tensor, states: torch.Tensor, omega_bf16: torch.Tensor, phase: torch.Tensor,
              inv_tau: float, normalize: bool = False, rule: int = RULE_DELTA, y: Optional[torch.Tensor] = None,
              out_dtype: Optional[torch.dtype] = None, workspace: Optional[torch.Tensor] = None,
              pipelined: bool = True, status: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The ragged step described by a token -> slot map alone (kdn_slot_step): nothing is read back to the
    host.  q, k (tokens, H, d_k), v (tokens, H, d_v), beta, decay (tokens, H); slot_mapping (tokens,) int32
    or int64 on the device, a sequence being a run of equal consecutive slots (negative: padding);
    states (slots, H, D, d_v) float32 updated in place.  Distinct runs must have distinct slots (not
    checked); `status` (device int32 (1,), optional) is set to 1 when the map has more runs than
    2 * slots + 1 (then nothing runs).  Returns y (tokens, H, d_v)."""
    for t, nm in ((q, "q"), (k, "k"), (v, "v"), (beta, "beta"), (states, "states"), (slot_mapping, "slot_mapping")):
        require_device(t, f"slot_step: {nm}")
    dev = q.device
    if q.dim() != 3 or k.shape != q.shape or v.dim() != 3 or v.shape[:2] != q.shape[:2] or beta.shape != q.shape[:2]:
        raise ValueError(f"slot_step: shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} beta{tuple(beta.shape)}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("slot_step: q, k and v must share a dtype")
    if states.dtype != torch.float32 or states.dim() != 4:
        raise TypeError("slot_step: states must be a float32 (slots, H, D, d_v) tensor")
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != q.shape[0] or slot_mapping.dtype not in (torch.int32, torch.int64):
        raise ValueError("slot_step: slot_mapping must be an int32 or int64 (tokens,) tensor")
    sm = slot_mapping.contiguous()
    q, k, v = _last_contig(q), _last_contig(k), _last_contig(v)
    beta = beta.to(torch.float32)
    if decay is not None:
        decay = decay.to(device=dev, dtype=torch.float32)
    T, H = q.shape[:2]
    d_v = v.shape[-1]
    if y is None:
        y = torch.empty(T, H, d_v, device=dev, dtype=q.dtype if out_dtype is None else out_dtype)
    om = omega_bf16.to(dev).contiguous()
    ph = phase.to(device=dev, dtype=torch.float32).contiguous()
    a = N.SlotStepArgs()
    a.num_tokens, a.H = T, H
    a.d_k, a.D, a.d_v = q.shape[-1], om.shape[0], d_v
    a.in_dtype, a.out_dtype = _tag(q.dtype, "slot step inputs"), _tag(y.dtype, "slot step output")
    a.normalize_input, a.rule, a.inv_tau = 1 if normalize else 0, int(rule), float(inv_tau)
    a.slot_mapping, a.slot_bytes = sm.data_ptr(), sm.element_size()
    a.q, a.q_stride = q.data_ptr(), N._i64x2(*q.stride()[:2])
    a.k, a.k_stride = k.data_ptr(), N._i64x2(*k.stride()[:2])
    a.v, a.v_stride = v.data_ptr(), N._i64x2(*v.stride()[:2])
    a.beta, a.beta_stride = beta.data_ptr(), N._i64x2(*beta.stride())
    if decay is not None:
        a.decay, a.decay_stride = decay.data_ptr(), N._i64x2(*decay.stride())
    a.omega_bf16, a.phase = om.data_ptr(), ph.data_ptr()
    a.states, a.state_stride = states.data_ptr(), N._i64x4(*states.stride())
    a.num_slots = states.shape[0]
    a.y, a.y_stride = y.data_ptr(), N._i64x2(*y.stride()[:2])
    a.status = status.data_ptr() if status is not None else None
    need = int(N.lib().kdn_slot_step_workspace_bytes(ctypes.byref(a)))
    if need == 0:
        raise ValueError("slot_step: unsupported shape (kdn_slot_step_workspace_bytes returned 0)")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    st = torch.cuda.current_stream(dev)
    with torch.cuda.device(dev):
        aux = None
        if pipelined:
            aux = aux_stream(dev)
            for t in (q, k, v, beta, decay, om, ph, states, y, sm, workspace, status):
                if t is not None:
                    t.record_stream(aux)
        N.check(N.lib().kdn_slot_step(ctypes.byref(a), ctypes.c_void_p(st.cuda_stream),
                                      ctypes.c_void_p(aux.cuda_stream) if aux is not None else None),
                "kdn_slot_step")
    return y


class StatePool:
    """Slab state pool (kdn_pool_*): `max_slots` fp32 slots of shape (layers, H, D, d_v) in one device
    tensor, with slot bookkeeping in the native library.  New slots are zeroed; fork copies a slot."""

    def __init__(self, max_slots: int, layers: int, heads: int, D: int = 512, d_v: int = 64, device="cuda:0",
                 slab: Optional[torch.Tensor] = None):
        self.shape = (max_slots, layers, heads, D, d_v)
        self.device = torch.device(device)
        self.slab = slab if slab is not None else torch.empty(self.shape, dtype=torch.float32, device=self.device)
        if tuple(self.slab.shape) != self.shape or not self.slab.is_contiguous() or self.slab.dtype != torch.float32:
            raise ValueError("StatePool: slab must be a contiguous float32 tensor of shape (slots, layers, H, D, d_v)")
        self.slot_bytes = layers * heads * D * d_v * 4
        h = ctypes.c_void_p()
        N.check(N.lib().kdn_pool_create(max_slots, self.slot_bytes, ctypes.byref(h)), "kdn_pool_create")
        self._h = h

    def _slab_ptr(self):
        return ctypes.c_void_p(self.slab.data_ptr()) if self.slab.is_cuda else None

    def _stream(self):
        return ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream) if self.slab.is_cuda else None

    def allocate(self) -> int:
        rc = N.lib().kdn_pool_allocate(self._h, self._slab_ptr(), self._stream())
        if rc == N.KDN_ERR_CAPACITY:
            return -1
        N.check(rc if rc < 0 else 0, "kdn_pool_allocate")
        return rc

    def fork(self, parent: int) -> int:
        rc = N.lib().kdn_pool_fork(self._h, int(parent), self._slab_ptr(), self._stream())
        if rc == N.KDN_ERR_CAPACITY:
            return -1
        N.check(rc if rc < 0 else 0, "kdn_pool_fork")
        return rc

    def release(self, slot: int) -> None:
        N.check(N.lib().kdn_pool_release(self._h, int(slot)), "kdn_pool_release")

    @property
    def active(self) -> int:
        return int(N.lib().kdn_pool_active(self._h))

    def allocated_bytes(self) -> int:
        return int(N.lib().kdn_pool_allocated_bytes(self._h))

    def free_bytes(self) -> int:
        return int(N.lib().kdn_pool_free_bytes(self._h))

    def layer_states(self, layer: int) -> torch.Tensor:
        """(slots, H, D, d_v) view of one layer's states, the `states` argument of ragged_step."""
        return self.slab[:, layer]

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                N.lib().kdn_pool_destroy(h)
            except Exception:
                pass
            self._h = None
