#!/usr/bin/env python
"""Benchmark of the Kernel-DeltaNet prefill hot path on one MI355X.

Workload (the one the headline metric is quoted on): one Kernel-DeltaNet layer
prefill, B=1, H=16, T=65536, d_k=64 lifted to D=512, d_v=64, 64-token chunks, bf16 q/k/v ~ N(0,1),
beta = sigmoid(N(0,1)) fp32, lambda = 1, fp32 state [16, 512, 64].  A step = the whole path over that
batch: per segment of chunks, the prep, state and output kernels.

Prints one JSON line.  `value` is prefill tokens/s (B*T tokens per step) with inputs resident in HBM.
`roofline` is for the dominant kernel, its average duration measured here with HIP events on the
launch stream; `traffic` comes from the committed rocprofv3 PMC summary when present.
`cpu_baseline` times the oracle's fp32 chunked restatement of the reference (torch on the host
cores) on the first tokens of the same inputs.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "kernel-deltanet_amd")
for _p in (REPO, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

C = 64
HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_BF16_PEAK = 2.5e15    # FLOP/s, MI355X dense bf16


def flops_per_chunk(D: int, dv: int) -> dict:
    """Algorithmic FLOPs per (head, 64-token chunk), split by kernel (terms of the reference algebra,
    kernels/fused_kernel_deltanet.py:99-149; total 4C^2D + 6CDdv + 9C^2dv + (2/3)C^3).  The fused
    schedule's chain forms the state kernel's and the output kernel's products."""
    prep = 4 * C * C * D + 5 * C * C * dv + (2.0 / 3.0) * C ** 3     # Grams, resolvents, U~, W~ factor
    state = 4 * C * D * dv + 2 * C * C * dv                           # K S^T, the update; E
    output = 2 * C * D * dv + 2 * C * C * dv                          # Q S^T; P E
    return {"prep": prep, "state": state, "output": output, "chain": state + output,
            "total": prep + state + output}


def path_bytes(B: int, T: int, H: int, D: int, dv: int, in_bytes: int = 2, out_bytes: int = 2) -> float:
    """Minimal HBM I/O of the path: q, k, v, beta, y per head-token plus the final fp32 state."""
    per_ht = 2 * 64 * in_bytes + dv * in_bytes + 4 + dv * out_bytes
    return B * T * H * per_ht + B * H * D * dv * 4


def read_pmc(path: str) -> dict:
    """key = value lines of a committed PMC summary (profiles/*.txt)."""
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        line = line.strip()
        if line and not line.startswith("#") and "=" in line:
            k, v = line.split("=", 1)
            try:
                out[k.strip()] = float(v.strip())
            except ValueError:
                pass
    return out


def cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as "Model name"), from /proc/cpuinfo."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(q, k, v, beta, T_sample: int, decay=None, runs: int = 3) -> dict:
    """Oracle fp32 chunked restatement (heads folded into batch) on the first T_sample tokens; the median
    of `runs` timed runs after a one-chunk warm-up."""
    from oracle import lift as ol
    from oracle import scan as osc

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    B, T, H, _ = q.shape
    f = lambda t: t[:, :T_sample].float().permute(0, 2, 1, 3).reshape(B * H, T_sample, -1).contiguous()
    fb = lambda t: None if t is None else t[:, :T_sample].float().permute(0, 2, 1).reshape(B * H, T_sample).contiguous()
    proj = ol.make_projection(64, 512, 42)
    args = (f(q), f(k), f(v), fb(beta), fb(decay), proj, C, None, torch.float32)
    osc.chunked_forward(*[a[:, :C] if isinstance(a, torch.Tensor) else a for a in args])  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        osc.chunked_forward(*args)
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[len(times) // 2]
    return {"value": B * T_sample / dt, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": cpu_model(), "runs_s": [round(t, 3) for t in times],
            "sample": f"oracle fp32 chunked restatement (torch CPU, heads folded into batch) on the first "
                      f"{T_sample} tokens of the same B={B}, H={H} inputs; median of {runs} runs, {dt:.2f} s"}


def synthetic_inputs(B: int, T: int, H: int, dv: int, dev, decay: str = "none") -> tuple:
    """q, k, v ~ N(0,1) (bf16), beta = sigmoid(N(0,1)) (fp32) and, with decay "sigmoid", lambda =
    sigmoid(N(0,1)) (fp32) from one generator seeded 1234, drawn in that order; on the host for up to 2^24
    head-tokens, on the device beyond (config 4).  decay "none" is lambda = 1 (returned as None)."""
    big = B * T * H > (1 << 24)
    where = dev if big else "cpu"
    g = torch.Generator(device=where).manual_seed(1234)
    q = torch.randn(B, T, H, 64, generator=g, device=where).to(torch.bfloat16)
    k = torch.randn(B, T, H, 64, generator=g, device=where).to(torch.bfloat16)
    v = torch.randn(B, T, H, dv, generator=g, device=where).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device=where))
    lam = torch.sigmoid(torch.randn(B, T, H, generator=g, device=where)) if decay == "sigmoid" else None
    return q, k, v, beta, lam


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=(2, 3, 4, 5),
                    help="3: one layer B=1 H=16 T=64k (default, the headline); 4: B=32 streams (use --T for "
                         "the sweep 4096/16384/65536); 2: the standalone lift of 2,097,152 rows; 5: the ragged "
                         "mixed step, 224 decode + 32 prefill sequences over resident states")
    ap.add_argument("--B", type=int, default=None)
    ap.add_argument("--H", type=int, default=16)
    ap.add_argument("--T", type=int, default=None)
    ap.add_argument("--dv", type=int, default=64)
    ap.add_argument("--segment-chunks", type=int, default=0,
                    help="chunks per segment (0 = the library default)")
    ap.add_argument("--serial", action="store_true",
                    help="serial schedule (kdn_delta_scan_fwd) instead of the pipelined one")
    ap.add_argument("--decay", default="none", choices=("none", "sigmoid"),
                    help="decay lambda: none (lambda = 1, the headline) or sigmoid(N(0,1)) per head-token "
                         "(the decay variant reported separately; configs 3 and 4)")
    ap.add_argument("--cpu-tokens", type=int, default=65536, help="tokens in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of known size (for PMC byte-counter calibration)")
    ap.add_argument("--pmc", default=None)
    ap.add_argument("--lift-variant", default="table", choices=("table", "bits", "butterfly"),
                    help="config 2: kdn_fwht_lift (resident Omega table), kdn_fwht_lift_bits (Omega built from the "
                         "sign table per workgroup) or kdn_fwht_lift_bits_butterfly (in-register butterflies)")
    ap.add_argument("--factored", action="store_true",
                    help="time the factored d_k = 128 path (two 64 -> 512 lifts, D = 1024 scan, d_v = 128) on a "
                         "B=1, H=32, T=16384 layer instead of config 3 (with --backward: its backward)")
    ap.add_argument("--backward", action="store_true",
                    help="time the backward pass (kdn_delta_scan_bwd: gradients of q, k, v, beta) on the config "
                         "3 shape instead of the forward")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; --gpus above 1 is not supported "
              "(the path shards over independent heads with no communication inside the scan)", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = 256 << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_dispatch_each_way": n}), flush=True)
        return
    if args.backward and args.factored:
        return bench_factored_backward(args, dev)
    if args.backward:
        return bench_backward(args, dev)
    if args.factored:
        return bench_factored(args, dev)
    if args.config == 2:
        return bench_lift(args, dev)
    if args.config == 5:
        return bench_serving(args, dev)
    return bench_scan(args, dev)


def bench_scan(args, dev):
    from kdn import ops
    from kernels import FastWalshHadamardProjection

    cfg = args.config
    B = args.B if args.B is not None else (32 if cfg == 4 else 1)
    T = args.T if args.T is not None else 65536
    H, dv, D = args.H, args.dv, 512
    q, k, v, beta, lam = synthetic_inputs(B, T, H, dv, dev, args.decay)
    proj = FastWalshHadamardProjection(64, D, 42)
    qd, kd, vd, bd = q.to(dev), k.to(dev), v.to(dev), beta.to(dev)
    ld = None if lam is None else lam.to(dev)
    plan = ops.ScanPlan(qd, kd, vd, bd, ld, proj.device_omega(dev), proj.device_phase(dev), proj.tau_star_inv,
                        segment_chunks=args.segment_chunks, pipelined=not args.serial)
    nchunks, seg = plan.nchunks, plan.segment_chunks
    stream = torch.cuda.current_stream(dev)

    for _ in range(args.warmup):
        plan.run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        plan.run()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps

    # Per-kernel durations: the same step issued phase by phase from here, in the order of the library's
    # schedule (split: prep, state, output; fused: prep, chain), with HIP events around each launch on the
    # stream it is launched on.
    fused = plan.schedule == ops.SCHEDULE_FUSED
    kinds = ("prep_fused", "chain") if fused else ("prep", "state", "output")
    segs = [(c0, min(seg, nchunks - c0)) for c0 in range(0, nchunks, seg)]
    timed = {kd: [] for kd in kinds}

    def launch(kind, s, st):
        c0, nc = segs[s]
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(st)
        getattr(plan, kind)(c0, nc, args=plan.segment_args(s), stream=st)
        a1.record(st)
        timed[kind].append((a0, a1))

    nbuf = max(1, plan.workspace.numel() // plan.seg_bytes)
    for _ in range(args.steps):
        if plan.pipelined and fused:
            # the library's fused schedule: the chain on the launch stream, prep on an auxiliary stream;
            # prep into a reused buffer waits for that buffer's last chain
            aux = ops.aux_stream(dev, 0)
            ev_in = torch.cuda.Event()
            ev_in.record(stream)
            aux.wait_event(ev_in)
            ev_p = [torch.cuda.Event() for _ in segs]
            ev_c = [torch.cuda.Event() for _ in segs]
            launch("prep_fused", 0, aux)
            ev_p[0].record(aux)
            for s_ in range(len(segs)):
                stream.wait_event(ev_p[s_])
                launch("chain", s_, stream)
                ev_c[s_].record(stream)
                if s_ + 1 < len(segs):
                    if s_ + 1 >= nbuf:
                        aux.wait_event(ev_c[s_ + 1 - nbuf])
                    launch("prep_fused", s_ + 1, aux)
                    ev_p[s_ + 1].record(aux)
        elif plan.pipelined:
            # the library's split schedule: state on the launch stream, prep and output on two auxiliary
            # streams; prep into a reused buffer waits for that buffer's last output
            aux, aux_o = ops.aux_stream(dev, 0), ops.aux_stream(dev, 1)
            ev_in = torch.cuda.Event()
            ev_in.record(stream)
            aux.wait_event(ev_in)
            aux_o.wait_event(ev_in)
            ev_p = [torch.cuda.Event() for _ in segs]
            ev_s = [torch.cuda.Event() for _ in segs]
            ev_o = [torch.cuda.Event() for _ in segs]
            launch("prep", 0, aux)
            ev_p[0].record(aux)
            for s_ in range(len(segs)):
                stream.wait_event(ev_p[s_])
                launch("state", s_, stream)
                ev_s[s_].record(stream)
                if s_ + 1 < len(segs):
                    if s_ + 1 >= nbuf:
                        aux.wait_event(ev_o[s_ + 1 - nbuf])
                    launch("prep", s_ + 1, aux)
                    ev_p[s_ + 1].record(aux)
                aux_o.wait_event(ev_s[s_])
                launch("output", s_, aux_o)
                ev_o[s_].record(aux_o)
            ev_out = torch.cuda.Event()
            ev_out.record(aux_o)
            stream.wait_event(ev_out)
        else:
            for s_ in range(len(segs)):
                for kind in kinds:
                    launch(kind, s_, stream)
    torch.cuda.synchronize()
    ms_kernel = {(k if k != "prep_fused" else "prep"): sum(x.elapsed_time(y) for x, y in v) / args.steps
                 for k, v in timed.items()}
    launches = {(k if k != "prep_fused" else "prep"): len(v) / args.steps for k, v in timed.items()}

    fl = flops_per_chunk(D, dv)
    units = B * H * nchunks
    tokens = B * T
    phases = {k: {"ms": ms_kernel[k], "launches": launches[k], "avg_launch_ms": ms_kernel[k] / launches[k],
                  "alg_flops": fl[k] * units, "tflops": fl[k] * units / ms_kernel[k] / 1e9}
              for k in ms_kernel}
    # The dominant kernel: in the split schedule with fewer state workgroups than CUs (config 3) the state
    # kernel is the sequential chain that prep and output run beside, so it bounds the step even when
    # concurrency stretches the others' launches; otherwise the kernels compete for CUs and the one with
    # the most launch time dominates.
    if plan.pipelined and not fused:
        dom = "state"
    else:
        dom = max(phases, key=lambda p: phases[p]["ms"])
    achieved = phases[dom]["tflops"]
    # Counter summaries committed under profiles/ for the measured shapes (rocprofv3 --pmc runs of this
    # script): HBM bytes (FETCH_SIZE / WRITE_SIZE) and MFMA busy % (MfmaUtil) of the dominant kernel.
    std = dv == 64 and H == 16 and args.decay == "none" and ((cfg == 3 and B == 1 and T == 65536) or
                                                            (cfg == 4 and B == 32))
    stem = f"pmc_config3" if cfg == 3 else f"pmc_config4_T{T}"
    pmc = read_pmc(args.pmc) if args.pmc else (read_pmc(os.path.join(REPO, "profiles", stem + ".txt")) if std else {})
    pmc_mfma = read_pmc(os.path.join(REPO, "profiles", stem + "_mfma.txt")) if std else {}
    key = dom
    traffic = None
    if f"{key}_fetch_kib" in pmc and f"{key}_write_kib" in pmc and "copy_fetch_kib" in pmc and "copy_write_kib" in pmc:
        copy_bytes = pmc.get("copy_bytes", 256 << 20)
        f_fac = copy_bytes / (pmc["copy_fetch_kib"] * 1024.0)
        w_fac = copy_bytes / (pmc["copy_write_kib"] * 1024.0)
        traffic = pmc[f"{key}_fetch_kib"] * 1024.0 * f_fac + pmc[f"{key}_write_kib"] * 1024.0 * w_fac
    mfma_util = pmc_mfma.get(f"{key}_mfma_util_pct")
    path_flops = fl["total"] * units
    name = ("config3: one Kernel-DeltaNet layer prefill" if cfg == 3 else
            "config4: batched long-context prefill (concurrent streams)")
    out = {
        "metric": "prefill tokens/s + ms/layer at T=64k, D=512 on 1 GPU; % of MFMA/HBM roofline",
        "value": tokens / (ms_per_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, sigmoid(N(0,1)) beta; projection seed 42)",
        "config": {"workload": f"{name}, B={B}, H={H}, T={T}, d_k=64->D={D}, "
                               f"d_v={dv}, chunk 64, bf16 q/k/v, fp32 beta and state, "
                               + ("lambda=1" if lam is None else "lambda=sigmoid(N(0,1)) fp32 (decay variant)"),
                   "decay": args.decay,
                   "B": B, "H": H, "T": T, "D": D, "d_v": dv, "chunk": C, "segment_chunks": seg,
                   "schedule": ("fused (prep on an auxiliary stream beside the fused chain, which writes y)"
                                if fused else "split (state chain on the launch stream, prep and output on two "
                                              "auxiliary streams)") + ("" if plan.pipelined else ", serial"),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": achieved / (MFMA_BF16_PEAK / 1e12), "traffic": traffic, "kernel": dom,
                     "mfma_util": mfma_util,
                     "mfma_util_source": (f"profiles/{stem}_mfma.txt ({key}_mfma_util_pct: rocprofv3 MfmaUtil, % "
                                          "of the GPU's MFMA cycles over the dispatch run alone)")
                     if mfma_util is not None else None},
        "phases": phases,
        "path": {"alg_flops": path_flops, "alg_bytes": path_bytes(B, T, H, D, dv),
                 "tflops": path_flops / ms_per_step / 1e9,
                 "mfma_frac": path_flops / (ms_per_step / 1e3) / MFMA_BF16_PEAK},
    }
    if args.cpu_tokens > 0:
        Ts = min(args.cpu_tokens, T)
        Bs = 1 if cfg == 4 else B
        out["cpu_baseline"] = cpu_baseline(q[:Bs, :Ts].cpu(), k[:Bs, :Ts].cpu(), v[:Bs, :Ts].cpu(),
                                           beta[:Bs, :Ts].cpu(), Ts, None if lam is None else lam[:Bs, :Ts].cpu())
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


def bwd_flops_per_chunk(D: int, dv: int, dk: int = 64) -> dict:
    """Algorithmic FLOPs per (head, 64-token chunk) of the closed-form chunk backward, split by launch:
    the matrix products the gradient needs (2 m n k each), as the kernels form them.
      prep   lift of q and k (2 C D dk each), K K^T and Q K^T (2 C^2 D each), H = Q^T (a o dY) (2 D C dv),
             U~ and R (2 C^2 dv each), the triangular inverse (2/3 C^3)
      carry  K Sigma and K^T Z (2 C D dv each), W or Tp^T dW (2 C^2 dv)   -- forward and reverse alike
      grad   Q S^T (2 C D dv); dQ^T: S^T (a o dY)^T, K^T N^T; dK^T: Gamma (kappa o W)^T, S^T Zn^T, Q^T N,
             K^T (M + M^T) (2 D C dv or 2 D C^2 each); lift recompute and dx^ for q and k (2 C D dk each);
             the 64 x 64 algebra T^T dW, dW X_K^T, dW V^T, dY W^T, dT T^T, Tp^T dW, T^T Y1 (2 C^2 dv or 2 C^3)
    The checkpoint pass (the forward scan's prep and state kernels, once per chunk) counts as the forward
    scan's prep (lift of q and k, K K^T and Q K^T, the inverse, U~ = T (beta o V)) and state (K S^T,
    K^T E, Tp X_K) products.
    """
    prep = 4 * C * D * dk + 4 * C * C * D + 2 * D * C * dv + 4 * C * C * dv + (2.0 / 3.0) * C ** 3
    carry = 4 * C * D * dv + 2 * C * C * dv
    grad = (2 * C * D * dv + (2 * D * dv * C + 2 * D * C * C) + (4 * D * dv * C + 4 * D * C * C)
            + 8 * C * D * dk + (5 * 2 * C * C * dv + 2 * 2 * C ** 3))
    ckpt = (4 * C * D * dk + 4 * C * C * D + (2.0 / 3.0) * C ** 3 + 2 * C * C * dv) + carry
    return {"checkpoint": ckpt, "prep": prep, "carry_fwd": carry, "carry_rev": carry, "grad": grad,
            "total": ckpt + prep + 2 * carry + grad}


def cpu_backward_baseline(q, k, v, beta, dy, T_sample: int, H: int) -> dict:
    """Float64 autograd of the oracle's token recurrence over the lift (one head, first T_sample tokens)."""
    from oracle import lift as ol
    from oracle import scan as osc

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    proj = ol.make_projection(64, 512, 42)
    qf = q[:1, :T_sample, 0].double().clone().requires_grad_(True)
    kf = k[:1, :T_sample, 0].double().clone().requires_grad_(True)
    vf = v[:1, :T_sample, 0].double().clone().requires_grad_(True)
    bf = beta[:1, :T_sample, 0].double().clone().requires_grad_(True)
    t0 = time.perf_counter()
    Y, S = osc.delta_rule_torch(qf, kf, vf, bf, None, proj)
    (Y * dy[:1, :T_sample, 0].double()).sum().backward()
    sec = time.perf_counter() - t0
    return {"value": T_sample / (sec * H), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"float64 torch autograd of the oracle token recurrence (forward + backward) over one "
                      f"head's first {T_sample} tokens; value scaled to all {H} heads ({sec:.2f} s measured)"}


def bench_backward(args, dev):
    """The backward pass on the config 3 shape (B=1, H=16, T=65536, bf16 q/k/v, fp32 beta, lambda = 1,
    dL/dy ~ N(0,1)): kdn_delta_scan_bwd computing dq, dk, dv, dbeta.  A step = one whole backward."""
    from kdn import ops
    from kernels import FastWalshHadamardProjection

    B = args.B if args.B is not None else 1
    T = args.T if args.T is not None else 65536
    H, dv, D = args.H, args.dv, 512
    q, k, v, beta, _ = synthetic_inputs(B, T, H, dv, dev)
    qd, kd, vd, bd = q.to(dev), k.to(dev), v.to(dev), beta.to(dev)
    gd = torch.Generator(device=dev).manual_seed(4321)
    dy = torch.randn(B, T, H, dv, generator=gd, device=dev)
    proj = FastWalshHadamardProjection(64, D, 42)
    plan = ops.ScanBackwardPlan(qd, kd, vd, bd, None, proj.device_omega(dev), proj.device_phase(dev),
                                proj.tau_star_inv, dy, need_dinit=False, segment_chunks=args.segment_chunks)
    stream = torch.cuda.current_stream(dev)
    for _ in range(args.warmup):
        plan.run(concurrent_carries=not args.serial)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        plan.run(concurrent_carries=not args.serial)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    # one phase at a time, on one stream: the checkpoint pass, then per segment (last first) the four
    # launches of the segment
    names = ("checkpoint", "prep", "carry_fwd", "carry_rev", "grad")
    timed = {n: [] for n in names}

    def timed_phase(n, i, s):
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        plan.phase(i, s)
        a1.record(stream)
        timed[n].append((a0, a1))

    for _ in range(args.steps):
        timed_phase("checkpoint", 0, 0)
        for s in reversed(range(plan.segments)):
            for i in range(1, 5):
                timed_phase(names[i], i, s)
    torch.cuda.synchronize()
    fl = bwd_flops_per_chunk(D, dv)
    nch = (T + C - 1) // C
    units = B * H * nch
    phases = {}
    for n in names:
        pm = sum(x.elapsed_time(y) for x, y in timed[n]) / args.steps
        launches = 1 if n == "checkpoint" else plan.segments
        phases[n] = {"ms": pm, "launches": launches, "avg_launch_ms": pm / launches, "alg_flops": fl[n] * units,
                     "tflops": fl[n] * units / pm / 1e9}
    dom = max(phases, key=lambda x: phases[x]["ms"])
    achieved = phases[dom]["tflops"]
    out = {
        "metric": "backward (gradients of q, k, v, beta) tokens/s at T=64k, D=512 on 1 GPU; % of MFMA roofline",
        "value": B * T / (ms / 1e3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, sigmoid(N(0,1)) beta, N(0,1) dL/dy; projection seed 42)",
        "config": {"workload": f"backward of config3 (one layer, B={B}, H={H}, T={T}, d_k=64->D={D}, d_v={dv}, "
                               f"bf16 q/k/v, fp32 beta, lambda=1)", "B": B, "H": H, "T": T, "D": D, "d_v": dv,
                   "workspace_bytes": plan.workspace.numel(), "parallelism": "single GPU",
                   "segments": plan.segments, "segment_chunks": plan.segment_chunks,
                   "schedule": "checkpoint pass (forward prep + state kernels, prep on an auxiliary stream), "
                               "then per segment, last first, the reverse carries back to back on the launch "
                               "stream while the auxiliary stream recomputes, carries forward and writes the "
                               "gradients of the segments around them (kdn_delta_scan_bwd_streams); the "
                               "per-phase times below are measured one phase at a time on one stream"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": achieved / (MFMA_BF16_PEAK / 1e12), "traffic": None, "kernel": dom},
        "phases": phases,
        "path": {"alg_flops": fl["total"] * units, "tflops": fl["total"] * units / ms / 1e9},
    }
    if args.cpu_tokens > 0:
        out["cpu_baseline"] = cpu_backward_baseline(q.cpu(), k.cpu(), v.cpu(), beta.cpu(), dy.cpu(),
                                                    min(args.cpu_tokens, 4096), H)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


def bench_factored(args, dev):
    """The factored d_k = 128 path (reference kernels/factored_kernel_deltanet.py): q, k (B, T, H, 128) bf16
    lifted to D = 1024 by kdn_fwht_lift_factored, then the D = 1024 delta-rule scan (d_v = 128, fp32 state,
    lambda = 1).  A step = both lifts and the scan."""
    from kdn import ops
    from kernels import FactoredFastWalshHadamardProjection

    B = args.B if args.B is not None else 1
    T = args.T if args.T is not None else 16384
    H = 32 if args.H == 16 else args.H
    D, dv, dk = 1024, 128, 128
    g = torch.Generator(device=dev).manual_seed(1234)
    q = torch.randn(B, T, H, dk, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, T, H, dk, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, T, H, dv, generator=g, device=dev).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device=dev))
    fp = FactoredFastWalshHadamardProjection(dk, D, 42)
    o1, p1 = fp.proj1.device_omega(dev), fp.proj1.device_phase(dev)
    o2, p2 = fp.proj2.device_omega(dev), fp.proj2.device_phase(dev)
    inv_tau = fp.proj1.tau_star_inv
    fm = ops.FeatureMap(lifted=True)
    final = torch.empty(B, H, D, dv, device=dev)
    y = torch.empty(B, T, H, dv, device=dev, dtype=torch.bfloat16)
    pq = ops.lift_factored(q, o1, p1, o2, p2, inv_tau)
    ws = torch.empty(ops.scan_workspace_bytes(pq, v, None, 0, True, fm), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step(times=None):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)] if times is not None else None
        if ev:
            ev[0].record(stream)
        fq = ops.lift_factored(q, o1, p1, o2, p2, inv_tau)
        fk = ops.lift_factored(k, o1, p1, o2, p2, inv_tau)
        if ev:
            ev[1].record(stream)
        ops.scan(fq, fk, v, beta, None, None, None, 1.0, final_state=final, y=y, workspace=ws, features=fm)
        if ev:
            ev[2].record(stream)
            times.append(ev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    times = []
    for _ in range(args.steps):
        step(times)
    torch.cuda.synchronize()
    lift_ms = sum(a.elapsed_time(b) for a, b, _ in times) / args.steps
    scan_ms = sum(b.elapsed_time(c) for _, b, c in times) / args.steps
    nch = (T + C - 1) // C
    units = B * H * nch
    f_chunk = 4 * C * C * D + 6 * C * D * dv + 9 * C * C * dv + (2.0 / 3.0) * C ** 3
    achieved = f_chunk * units / scan_ms / 1e9
    lift_bytes = 2 * B * T * H * (dk + D) * 2  # q and k: bf16 rows in, bf16 features out
    out = {
        "metric": "factored d_k=128 prefill tokens/s (lift + D=1024 scan) on 1 GPU; % of MFMA roofline",
        "value": B * T / (ms / 1e3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, sigmoid(N(0,1)) beta; projection seeds 42 and 1042)",
        "config": {"workload": f"factored d_k=128 layer, B={B}, H={H}, T={T}, d_k=128->D={D} (2 x 64->512), "
                               f"d_v={dv}, bf16 q/k/v, fp32 beta and state, lambda=1",
                   "B": B, "H": H, "T": T, "D": D, "d_v": dv, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": achieved / (MFMA_BF16_PEAK / 1e12), "traffic": None, "kernel": "scan (3 launches)"},
        "phases": {"lift": {"ms": lift_ms, "alg_bytes": lift_bytes, "gbps": lift_bytes / lift_ms / 1e6},
                   "scan": {"ms": scan_ms, "alg_flops": f_chunk * units, "tflops": achieved}},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_factored_backward(args, dev):
    """The backward of the factored d_k = 128 layer of bench_factored (B=1, H=32, T=16384, bf16, d_v = 128,
    lambda = 1, dL/dy ~ N(0,1)): kdn_delta_scan_bwd at D = 1024 over the lifted features (dL/dphi_q,
    dL/dphi_k, dv, dbeta), then kdn_fwht_lift_factored_bwd for q and k.  A step = the whole backward."""
    from kdn import ops
    from kernels import FactoredFastWalshHadamardProjection

    B = args.B if args.B is not None else 1
    T = args.T if args.T is not None else 16384
    H = 32 if args.H == 16 else args.H
    D, dv, dk = 1024, 128, 128
    g = torch.Generator(device=dev).manual_seed(1234)
    q = torch.randn(B, T, H, dk, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, T, H, dk, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, T, H, dv, generator=g, device=dev).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device=dev))
    dy = torch.randn(B, T, H, dv, generator=g, device=dev)
    fp = FactoredFastWalshHadamardProjection(dk, D, 42)
    lift_args = (fp.proj1.device_omega(dev), fp.proj1.device_phase(dev), fp.proj2.device_omega(dev),
                 fp.proj2.device_phase(dev), fp.proj1.tau_star_inv)
    fq, fk = ops.lift_factored(q, *lift_args), ops.lift_factored(k, *lift_args)
    plan = ops.ScanBackwardPlan(fq, fk, v, beta, None, None, None, 1.0, dy, need_dinit=False,
                                features=ops.FeatureMap(lifted=True), segment_chunks=args.segment_chunks)
    stream = torch.cuda.current_stream(dev)

    def step(times=None):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)] if times is not None else None
        if ev:
            ev[0].record(stream)
        dpq, dpk = plan.run(concurrent_carries=False)[:2]
        if ev:
            ev[1].record(stream)
        ops.lift_factored_backward(q, dpq, *lift_args)
        ops.lift_factored_backward(k, dpk, *lift_args)
        if ev:
            ev[2].record(stream)
            times.append(ev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    times = []
    for _ in range(args.steps):
        step(times)
    torch.cuda.synchronize()
    scan_ms = sum(a.elapsed_time(b) for a, b, _ in times) / args.steps
    lift_ms = sum(b.elapsed_time(c) for _, b, c in times) / args.steps
    nch = (T + C - 1) // C
    units = B * H * nch
    # per chunk: the recompute's Grams and carry (4 C^2 D + 4 C D d_v), R and H (2 C D d_v), the reverse
    # carry (4 C D d_v), Q S^T (2 C D d_v) and the feature gradients (6 C D d_v + 6 C^2 D), plus the
    # 64 x 64 algebra (~16 C^2 d_v + 6 C^3)
    f_chunk = 10 * C * C * D + 18 * C * D * dv + 16 * C * C * dv + 6 * C ** 3
    achieved = f_chunk * units / scan_ms / 1e9
    out = {
        "metric": "factored d_k=128 backward tokens/s (D=1024 scan backward + lift backward) on 1 GPU; "
                  "% of MFMA roofline",
        "value": B * T / (ms / 1e3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, sigmoid(N(0,1)) beta, N(0,1) dL/dy; projection seeds 42, 1042)",
        "config": {"workload": f"backward of the factored d_k=128 layer, B={B}, H={H}, T={T}, d_k=128->D={D}, "
                               f"d_v={dv}, bf16 q/k/v, fp32 beta, lambda=1",
                   "B": B, "H": H, "T": T, "D": D, "d_v": dv, "workspace_bytes": plan.workspace.numel(),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                     "frac": achieved / (MFMA_BF16_PEAK / 1e12), "traffic": None, "kernel": "scan backward (6 launches)"},
        "phases": {"scan_backward": {"ms": scan_ms, "alg_flops": f_chunk * units, "tflops": achieved},
                   "lift_backward": {"ms": lift_ms}},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def _slot_args_probe(T, H, dv, n_slots):
    """kdn_slot_step_args with the shape fields the workspace size reads (bf16, D = 512)."""
    from kdn import _native as N
    a = N.SlotStepArgs()
    a.num_tokens, a.H, a.d_k, a.D, a.d_v = T, H, 64, 512, dv
    a.in_dtype = a.out_dtype = N.KDN_DTYPE_BF16
    a.inv_tau, a.slot_bytes, a.num_slots = 1.0, 8, n_slots
    return a


def bench_serving(args, dev):
    """Config 5: one ragged mixed step over 256 sequences, 224 single-token decodes (rank-1 update of a
    resident [16, 512, 64] fp32 state in a slab pool) and 32 prefills with lengths uniform in
    [512, 8192]; H=16, D=512, d_v=64, bf16 q/k/v ~ N(0,1), beta = sigmoid(N(0,1)), lambda = 1."""
    from kdn import ops
    from kernels import FastWalshHadamardProjection

    H, D, dv, n_dec, n_pre = args.H, 512, args.dv, 224, 32
    g = torch.Generator().manual_seed(1234)
    pre_lens = torch.randint(512, 8193, (n_pre,), generator=g)
    lens = torch.cat([torch.ones(n_dec, dtype=torch.int64), pre_lens])
    T = int(lens.sum())
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(lens, 0)])
    gd = torch.Generator(device=dev).manual_seed(1234)
    q = torch.randn(T, H, 64, generator=gd, device=dev).to(torch.bfloat16)
    k = torch.randn(T, H, 64, generator=gd, device=dev).to(torch.bfloat16)
    v = torch.randn(T, H, dv, generator=gd, device=dev).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(T, H, generator=gd, device=dev))
    pool = ops.StatePool(n_dec + n_pre, 1, H, D, dv, device=dev)
    slots = torch.tensor([pool.allocate() for _ in range(n_dec + n_pre)], dtype=torch.int32)
    pool.slab.normal_(generator=gd).mul_(0.01)
    states = pool.layer_states(0)
    proj = FastWalshHadamardProjection(64, D, 42)
    om, ph = proj.device_omega(dev), proj.device_phase(dev)
    y = torch.empty(T, H, dv, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(dev)

    def timed(cu_, slots_, q_, k_, v_, b_, y_, steps):
        # batch metadata staged on the device and the workspace allocated once, as a serving loop keeps them
        cu_d, slots_d = cu_.to(dev), slots_.to(dev)
        ws = torch.empty(ops.ragged_workspace_bytes(q_, k_, v_, b_, None, cu_, slots_d, states, om, ph,
                                                    proj.tau_star_inv, y=y_, cu_seqlens_device=cu_d),
                         dtype=torch.uint8, device=dev)
        call = lambda: ops.ragged_step(q_, k_, v_, b_, None, cu_, slots_d, states, om, ph, proj.tau_star_inv, y=y_,
                                       workspace=ws, cu_seqlens_device=cu_d)
        for _ in range(args.warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms = timed(cu, slots, q, k, v, beta, y, args.steps)
    # the same step described by the token -> slot map alone (kdn_slot_step: no host offsets, launches sized
    # from the token and slot counts), workspace allocated once
    import ctypes
    from kdn import _native as N
    slot_map = torch.repeat_interleave(slots.to(torch.int64), lens).to(dev)
    ws_slot = torch.empty(int(N.lib().kdn_slot_step_workspace_bytes(ctypes.byref(_slot_args_probe(
        T, H, dv, states.shape[0])))), dtype=torch.uint8, device=dev)
    for _ in range(args.warmup):
        ops.slot_step(q, k, v, beta, None, slot_map, states, om, ph, proj.tau_star_inv, y=y, workspace=ws_slot)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        ops.slot_step(q, k, v, beta, None, slot_map, states, om, ph, proj.tau_star_inv, y=y, workspace=ws_slot)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_slot = e0.elapsed_time(e1) / args.steps
    # the two parts alone: the decode tokens (rows 0..223) and the prefill tokens (rows 224..)
    ms_dec = timed(cu[: n_dec + 1], slots[:n_dec], q, k, v, beta, y, args.steps)
    cu_pre = cu[n_dec:] - n_dec
    ms_pre = timed(cu_pre, slots[n_dec:], q[n_dec:], k[n_dec:], v[n_dec:], beta[n_dec:], y[n_dec:], args.steps)
    dec_bytes = n_dec * H * (2 * D * dv * 4 + (2 * 64 + 2 * dv) * 2 + 4)
    dec_gbs = dec_bytes / (ms_dec / 1e3) / 1e9
    pre_tokens = int(pre_lens.sum())
    fl = flops_per_chunk(D, dv)
    pre_flops = sum(((int(L) + C - 1) // C) for L in pre_lens) * H * fl["total"]
    pre_tflops = pre_flops / (ms_pre / 1e3) / 1e12
    out = {
        "metric": "ragged mixed prefill+decode step tokens/s (config 5); % of HBM (decode) / MFMA (prefill) roofline",
        "value": T / (ms / 1e3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": f"synthetic (seeded N(0,1) q/k/v, sigmoid(N(0,1)) beta, N(0,1)*0.01 resident states; prefill "
                f"lengths U[512, 8192], {pre_tokens} prefill tokens)",
        "config": {"workload": f"config5: ragged mixed step, {n_dec} decode + {n_pre} prefill sequences, H={H}, D={D}, "
                               f"d_v={dv}, fp32 states in a slab pool, lambda=1", "tokens": T, "parallelism": "single GPU"},
        "roofline": ({"bound": "mfma", "achieved": pre_tflops, "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                      "frac": pre_tflops * 1e12 / MFMA_BF16_PEAK, "traffic": None, "kernel": "prefill (scan)"}
                     if ms_pre >= ms_dec else
                     {"bound": "hbm", "achieved": dec_gbs, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                      "frac": dec_gbs * 1e9 / HBM_PEAK, "traffic": None, "kernel": "decode"}),
        "parts": {"decode": {"ms": ms_dec, "sequences": n_dec, "alg_bytes": dec_bytes, "GBps": dec_gbs,
                             "hbm_frac": dec_gbs * 1e9 / HBM_PEAK},
                  "prefill": {"ms": ms_pre, "sequences": n_pre, "tokens": pre_tokens, "alg_flops": pre_flops,
                              "tflops": pre_tflops, "mfma_frac": pre_tflops * 1e12 / MFMA_BF16_PEAK},
                  "slot_map_step": {"ms": ms_slot, "note": "the whole step from slot_mapping alone (kdn_slot_step, "
                                                           "no host offsets)"}},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_lift(args, dev):
    """Config 2: the standalone lift (kdn_fwht_lift) of x [B*T*H, 64] bf16 ~ N(0,1), B=8, T=16384, H=16,
    L2-normalised per row, to D=512 bf16.  HBM-bound: algorithmic bytes = rows * (64 + 512) * 2."""
    from kdn import ops
    from kernels import FastWalshHadamardProjection

    B = args.B if args.B is not None else 8
    T = args.T if args.T is not None else 16384
    rows, D = B * T * args.H, 512
    g = torch.Generator(device=dev).manual_seed(1234)
    x = torch.randn(rows, 64, generator=g, device=dev).to(torch.bfloat16)
    proj = FastWalshHadamardProjection(64, D, 42)
    om, ph, bits = proj.device_omega(dev), proj.device_phase(dev), proj.device_bits(dev)
    stream = torch.cuda.current_stream(dev)
    variant = args.lift_variant

    def lift_once():
        if variant == "table":     # kdn_fwht_lift: Omega from the resident bf16 table, MFMA projection
            return ops.lift(x, om, ph, proj.tau_star_inv, normalize=True)
        # kdn_fwht_lift_bits (Omega built in LDS per workgroup, MFMA projection) or
        # kdn_fwht_lift_bits_butterfly (in-register wave64 butterflies, no Omega)
        return ops.lift_bits(x, bits, ph, proj.tau_star_inv, normalize=True, butterfly=variant == "butterfly")

    # At least 40 untimed lifts (~25 ms): for the first few dozen launches after the GPU leaves idle the
    # per-launch time swings by up to 40 % (510 -> 683 -> 590 us) before it settles near 460 us
    warmup = max(args.warmup, 40)
    for _ in range(warmup):
        y = lift_once()
    torch.cuda.synchronize()
    # K lifts back to back between two events (the GPU never waits for the host between them), as the
    # other configs time their steps
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        y = lift_once()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    alg_bytes = rows * (64 + D) * 2
    achieved = alg_bytes / (ms / 1e3) / 1e9
    std = rows == 2097152 and variant == "table"
    pmc = read_pmc(args.pmc) if args.pmc else (read_pmc(os.path.join(REPO, "profiles", "pmc_config2.txt")) if std else {})
    pmc_mfma = read_pmc(os.path.join(REPO, "profiles", "pmc_config2_mfma.txt")) if std else {}
    traffic = None
    if all(k in pmc for k in ("lift_fetch_kib", "lift_write_kib", "copy_fetch_kib", "copy_write_kib")):
        copy_bytes = pmc.get("copy_bytes", 256 << 20)
        traffic = (pmc["lift_fetch_kib"] * copy_bytes / pmc["copy_fetch_kib"]
                   + pmc["lift_write_kib"] * copy_bytes / pmc["copy_write_kib"])
    out = {
        "metric": "standalone lift rows/s (config 2); % of HBM roofline",
        "value": rows / (ms / 1e3), "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) x; projection seed 42)",
        "config": {"workload": f"config2: standalone lift, x [{rows}, 64] bf16 L2-normalised -> [{rows}, 512] bf16 "
                               f"(B={B}, T={T}, H={args.H})", "rows": rows, "D": D, "parallelism": "single GPU",
                   "lift_variant": variant},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": achieved * 1e9 / HBM_PEAK, "traffic": traffic,
                     "kernel": "lift" if variant != "butterfly" else "lift_butterfly",
                     "mfma_util": pmc_mfma.get("lift_mfma_util_pct"),
                     "mfma_util_source": "profiles/pmc_config2_mfma.txt (lift_mfma_util_pct)" if pmc_mfma else None},
    }
    if args.cpu_tokens > 0:
        from oracle import lift as ol
        n = min(args.cpu_tokens * 4, rows)
        xs = x[:n].float().cpu().numpy()
        op = ol.make_projection(64, D, 42)
        t0 = time.perf_counter()
        ol.lift(xs, op, normalize=True)
        dt = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": n / dt, "unit": "rows/s", "cores": 1, "kind": "port",
                               "sample": f"oracle float64 lift (numpy) of the first {n} rows; {dt:.2f} s"}
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
