#!/usr/bin/env python
"""Benchmark of the selective-SSM path on one GPU.

Default workload (the one the headline metric is quoted on): the fused
multihead DIAG chunked scan at B=8 L=4096 H=16 P=N=64, chunk 128, bf16
x/B/C/y, fp32 dt and state, ZOH discretization fused into the load stage.
``--workload`` selects the other measured workloads:

  mamba1_small   Mamba-1 selective scan B=2 L=256 D=16 N=16 fp32
  interp_mamba1  interpolation + Mamba-1 scan B=16 T=2048 F=256 N=16 fp32
  ssd_long       SSD scan B=1 L=262144 H=8 P=64 N=16 bf16, chunk 256
  ssd_config1    SSD scan on the headline shapes B=8 L=4096 H=16 P=N=64 bf16
  ssd_n64_long   SSD scan B=1 L=65536 H=8 P=N=64 bf16 (time-segmented one-pass kernel)
  ssd_stream     streaming SSD step, 4096 streams H=32 P=64 N=128 fp32 state
  dtproj         Mamba-1 scan B=16 L=2048 D=256 N=16 fp32 with dt = clamp(softplus(
                 dt_raw W + bias)) formed inside the scan's passes (rank 16)
  dtproj_two_launch  the same as dt_project_softplus_kernel + the scan
  bcproj         Mamba-1 scan B=16 L=2048 D=256 N=16 fp32 with B, C = x W formed inside
                 the scan's first pass
  bcproj_two_launch  the same as matmuls producing B and C, then the scan
  xproj          Mamba-1 scan B=16 L=2048 D=256 N=16 fp32 with the whole input
                 projection x -> (dt, B, C) formed inside the scan (rank 16)
  xproj_unfused  the same as the x_proj matmul, column copies and the dt-producing scan
  rows           every drop-in kernel at a config-sized shape (one JSON line, "rows" list)

A step is one pass of the path over one batch of seeded synthetic input that
is already resident in HBM.  Input sets are rotated where memory allows so
consecutive steps do not hit in the 256 MB Infinity Cache.  Prints ONE JSON
line with the metric, the roofline of the dominant kernel (algorithmic bytes
/ average launch duration: HIP events on the launch stream around the timed
region of back-to-back launches) and the C
restatement timed on the host cores (rank 0, N=1, bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "triton-ssm_amd"))
sys.path.insert(0, str(ROOT))

PEAK_GBS = 8000.0
# VALU roofline of the vector-bound workloads: MI355X's published fp32 rate
# without packed math, 78.6 TFLOP/s = 39.3 T fused multiply-adds (lane
# operations) per second; an exp2 occupies the issue of 2.31 of them (measured
# on gfx950: independent v_exp_f32 at 3.51 ns and v_fma_f32 at 1.52 ns per
# wave instruction per SIMD).
PEAK_VALU_TLANE = 39.3
EXP2_SLOTS = 2.31
HEADLINE_METRIC = "scan elements/sec + achieved HBM GB/s (% of peak), B=8 L=4096 H=16 P=64 N=64"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _np32(t):
    import numpy as np
    return np.ascontiguousarray(t.float().numpy())


# The CPU baseline runs a workload at least ``--cpu-reps`` times and until
# ``--cpu-seconds`` of CPU work have been timed (a bounded sample of about ten
# seconds); the sample notes say how many runs that took.
CPU_SECONDS = 10.0
_cpu_runs = [0, 0.0]   # runs and total seconds of the last _timed_cpu


def _timed_cpu(fn, reps):
    fn()   # warm
    times = []
    while len(times) < reps or (sum(times) < CPU_SECONDS and len(times) < 100000):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    _cpu_runs[0], _cpu_runs[1] = len(times), sum(times)
    return statistics.median(times)


def _runs_note():
    return f"median of {_cpu_runs[0]} runs ({_cpu_runs[1]:.1f} s of CPU work)"


# ------------------------------------------------------------------ workloads
def wl_multihead(args, dev):
    import torch
    from tssm import multihead_ssm_forward, workloads
    B, L, H, P = 8, 4096, 16, 64
    w = workloads.multihead(B=B, L=L, H=H, P=P)
    a_key = "A_log" if args.a_per_channel else "A_log_h"
    base = {k: w[k].to(dev) for k in ("u", "B", "C", "dt")}
    if args.a_log_const is not None:
        # a slowly decaying input of the same shape: every decay exp(-e^c dt)
        w = dict(w)
        w[a_key] = torch.full_like(w[a_key], args.a_log_const)
    A_log = w[a_key].to(dev)
    sets = []
    for i in range(args.sets):
        s = {k: torch.roll(v, shifts=i, dims=0).contiguous() for k, v in base.items()}
        s["y"] = torch.empty_like(s["u"])
        sets.append(s)

    def step(i):
        s = sets[i % len(sets)]
        multihead_ssm_forward(s["u"], A_log, s["B"], s["C"], s["dt"], None, disc=args.disc,
                              chunk=128, out=s["y"])

    def cpu():
        from oracle import cport
        arrs = [_np32(w[k]) for k in ("u", a_key, "B", "C", "dt")]
        med = _timed_cpu(lambda: cport.multihead_scan(*arrs, None, disc=args.disc, prepared=True),
                         args.cpu_reps)
        return {"value": B * L * H * P / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"whole workload, {_runs_note()}, "
                                          f"{med:.3f} s each"}

    n = B * L * H * P
    nbytes = workloads.multihead_bytes(B, L, H, P, io_bytes=2) - H * P * 4 + A_log.numel() * 4
    cfg = {"workload": "fused multihead DIAG chunked scan, B=8 L=4096 H=16 P=N=64, chunk 128, "
                       f"bf16 x/B/C/y, fp32 dt/state, {args.disc.upper()} discretization",
           "B": B, "L": L, "H": H, "P": P, "N": P, "chunk": 128, "disc": args.disc,
           "io_dtype": "bf16", "state_dtype": "f32",
           "a_log": "per channel [H, P]" if args.a_per_channel else "per head [H]"}
    if args.a_log_const is not None:
        cfg["a_log_const"] = args.a_log_const
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, kernel="mh_scan_fused_kernel",
                dtype="bf16", metric=HEADLINE_METRIC, unit="elements/s", config=cfg,
                traffic="mh_scan_fused_traffic.json")


def wl_ssd_config1(args, dev):
    """The SSD form (state P x N per head) on the headline shapes: the same seeded
    x, B, C, dt and per-head A_log as the DIAG workload, x read as [B, L, H, P]."""
    import torch
    from tssm import ssd_scan_forward, workloads
    B, L, H, P = 8, 4096, 16, 64
    w = workloads.multihead(B=B, L=L, H=H, P=P)
    base = {"x": w["u"].view(B, L, H, P), "B": w["B"], "C": w["C"], "dt": w["dt"]}
    base = {k: v.to(dev) for k, v in base.items()}
    A_log = w["A_log_h"].to(dev)
    N = base["B"].shape[-1]
    sets = []
    for i in range(args.sets):
        s = {k: torch.roll(v, shifts=i, dims=0).contiguous() for k, v in base.items()}
        s["y"] = torch.empty_like(s["x"])
        sets.append(s)

    def step(i):
        s = sets[i % len(sets)]
        ssd_scan_forward(s["x"], s["dt"], A_log, s["B"], s["C"], None, chunk=args.ssd_chunk,
                         disc=args.disc, out=s["y"])

    def cpu():
        from oracle import cport
        Bs = 1
        arrs = [_np32(w["u"][:Bs].view(Bs, L, H, P)), _np32(w["dt"][:Bs]), _np32(w["A_log_h"]),
                _np32(w["B"][:Bs]), _np32(w["C"][:Bs])]
        med = _timed_cpu(lambda: cport.ssd_scan(*arrs, None, None, disc=args.disc), args.cpu_reps)
        return {"value": Bs * L * H * P / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"batch 0 of {B}, {_runs_note()}, "
                                          f"{med:.3f} s each"}

    n = B * L * H * P
    nbytes = 2 * (2 * n + 2 * B * L * H * N) + 4 * B * L * H + 4 * H
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes,
                kernel="ssd_seq_kernel", traffic="ssd_seq_traffic.json", dtype="bf16",
                metric="SSD scan elements/sec on the headline shapes, B=8 L=4096 H=16 P=N=64 bf16",
                unit="elements/s",
                config={"workload": "SSD scan (decay per head, P x N state) on the DIAG headline "
                                    f"shapes, B=8 L=4096 H=16 P=N=64, chunk {args.ssd_chunk}, "
                                    f"bf16 I/O, fp32 state, {args.disc.upper()}",
                        "B": B, "L": L, "H": H, "P": P, "N": N, "chunk": args.ssd_chunk})


def wl_mamba1_small(args, dev):
    from tssm import selective_scan_forward, workloads
    w = workloads.mamba1_small()
    d = {k: v.to(dev) for k, v in w.items()}
    B, L, Dc = d["x"].shape
    N = d["A_log"].shape[1]

    def step(i):
        selective_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None, disc=args.disc)

    def cpu():
        from oracle import cport
        arrs = [_np32(w[k]) for k in ("x", "dt", "A_log", "B", "C")]
        reps = 2000
        med = _timed_cpu(lambda: [cport.selective_scan(*arrs, None, disc=args.disc)
                                  for _ in range(reps)], 3) / reps
        return {"value": B * L * Dc / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port",
                "sample": f"whole workload x{reps}, {_runs_note()}, {med * 1e6:.1f} us each"}

    n = B * L * Dc
    nbytes = 4 * (2 * n + B * L + Dc * N + 2 * B * L * N)
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, kernel="mh_scan_fused_kernel",
                metric="Mamba-1 selective scan elements/sec, B=2 L=256 D=16 N=16 fp32",
                unit="elements/s",
                config={"workload": "Mamba-1 selective scan (lanes d x n), B=2 L=256 D=16 N=16, "
                                    f"fp32, {args.disc.upper()}, dt per (b,t)",
                        "B": B, "L": L, "D": Dc, "N": N})


def wl_interp_mamba1(args, dev):
    from tssm import fused_interp_ssm_forward, workloads
    import torch
    w = workloads.interp_mamba1()
    base = {k: v.to(dev) for k, v in w.items()}
    B, T, F = base["V"].shape
    N = base["A_log"].shape[1]
    # rotated input sets (batch rolled): one set's 139 MB would otherwise stay
    # in the 256 MB last-level cache from one step to the next
    sets = []
    for i in range(max(args.sets, 3)):
        s = {k: (v if k == "A_log" else torch.roll(v, shifts=i, dims=0).contiguous())
             for k, v in base.items()}
        sets.append(s)

    def step(i):
        d = sets[i % len(sets)]
        fused_interp_ssm_forward(d["V"], d["M"], d["tau"], d["A_log"], d["B"], d["C"],
                                 K=10, FTILE=128, disc=args.disc, chunk=args.scan_chunk)

    def cpu():
        import numpy as np
        from oracle import cport
        V, M, tau = (_np32(w[k]) for k in ("V", "M", "tau"))
        rest = [_np32(w[k]) for k in ("A_log", "B", "C")]

        def run():
            vhat = cport.time_aware_interp(V, M, tau, 10, 128)
            dt = np.diff(tau, axis=1, prepend=0.0).astype(np.float32)
            cport.selective_scan(vhat, dt, *rest, None, disc=args.disc)
        med = _timed_cpu(run, args.cpu_reps)
        return {"value": B * T * F / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"whole workload, {_runs_note()}, "
                                          f"{med:.3f} s each"}

    n = B * T * F
    nbytes = 4 * (4 * n + B * T + F * N + 2 * B * T * N)   # V, M in; Vhat, y out
    # VALU floor per lane update (b, t, d, n) of the three-pass ZOH scan: the
    # update (dt a, exp2, -1, B x, two fmas) and the readout fma in pass 1, the
    # carried share (a cum, exp2, C S, fma) in pass 3: 9 ops and 2 exp2
    valu = {"lane_updates": n * N, "ops_per_update": 9, "exp2_per_update": 2}
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, valu=valu,
                kernel="whole step: sel_interp_state_kernel (interpolation in pass 1), "
                       "sel_carry_kernel, sel_output_kernel",
                metric="interp + Mamba-1 scan elements/sec, B=16 T=2048 F=256 N=16 fp32",
                unit="elements/s",
                config={"workload": "time-aware interpolation (K=10, FTILE=128, 30% missing) + "
                                    f"Mamba-1 scan, B=16 T=2048 F=256 N=16 fp32, {args.disc.upper()}",
                        "B": B, "T": T, "F": F, "N": N, "K": 10, "FTILE": 128})


def _wl_dtproj(args, dev, fused):
    """Mamba-1 scan with dt from the rank-16 projection, B=16 L=2048 D=256 N=16
    fp32: fused into the scan's load stage, or as two launches
    (dt_project_softplus_kernel writing dt [B,L,D], then the scan reading it)."""
    import torch
    import discretize_kernel as dk
    from tssm import selective_scan_forward, workloads
    w = workloads.dtproj_mamba1()
    base = {k: v.to(dev) for k, v in w.items() if isinstance(v, torch.Tensor)}
    B, L, Dc = base["x"].shape
    N = base["A_log"].shape[1]
    R = base["dt_raw"].shape[2]
    sets = []
    for i in range(max(args.sets, 3)):
        st = {k: (v if k in ("W", "bias", "A_log") else torch.roll(v, shifts=i, dims=0).contiguous())
              for k, v in base.items()}
        st["y"] = torch.empty_like(st["x"])
        st["dt"] = torch.empty(B, L, Dc, device=dev)
        sets.append(st)
    lo, hi = w["DT_MIN"], w["DT_MAX"]

    def step(i):
        d = sets[i % len(sets)]
        if fused:
            selective_scan_forward(d["x"], d["dt_raw"], d["A_log"], d["B"], d["C"], None,
                                   chunk=args.scan_chunk, disc=args.disc, out=d["y"],
                                   dt_proj=(d["W"], d["bias"], lo, hi))
        else:
            dk.dt_project_softplus_kernel[(B, L, Dc // 256)](
                d["dt_raw"], d["W"], d["bias"], d["dt"], B, L, Dc, R, *d["dt_raw"].stride(),
                *d["W"].stride(), *d["dt"].stride(), DT_MIN=lo, DT_MAX=hi, BLOCK_H=256,
                BLOCK_R=16)
            selective_scan_forward(d["x"], d["dt"], d["A_log"], d["B"], d["C"], None,
                                   chunk=args.scan_chunk, disc=args.disc, out=d["y"])

    def cpu():
        import numpy as np
        from oracle import cport
        raw, W, bias = (_np32(w[k]) for k in ("dt_raw", "W", "bias"))
        rest = [_np32(w[k]) for k in ("A_log", "B", "C")]
        x = _np32(w["x"])

        def run():
            dt = np.clip(np.logaddexp(0.0, raw @ W + bias), lo, hi).astype(np.float32)
            cport.selective_scan(x, dt, *rest, None, disc=args.disc)
        med = _timed_cpu(run, args.cpu_reps)
        return {"value": B * L * Dc / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"whole workload, {_runs_note()}, "
                                          f"{med:.3f} s each (projection in numpy)"}

    n = B * L * Dc
    nbytes = 4 * (2 * n + B * L * R + R * Dc + Dc + Dc * N + 2 * B * L * N)
    if not fused:
        nbytes += 2 * 4 * n      # dt written by the projection and read by the scan
    how = "fused into the scan's load stage" if fused else "two launches through dt [B,L,D]"
    # the same VALU floor per lane update as the interpolation workload's scan
    valu = {"lane_updates": n * N, "ops_per_update": 9, "exp2_per_update": 2}
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, valu=valu,
                kernel="sel_chunk_state_kernel (dt formed on the matrix cores) + "
                       "sel_carry_kernel + sel_output_kernel" if fused
                else "dt_project_mfma_kernel + sel_chunk_state_kernel + sel_carry_kernel + "
                     "sel_output_kernel",
                metric=f"Mamba-1 scan with dt projection ({how}) elements/sec, B=16 L=2048 "
                       "D=256 N=16 rank 16 fp32",
                unit="elements/s",
                config={"workload": f"dt = clamp(softplus(dt_raw W + bias)) {how} + Mamba-1 "
                                    f"scan, B=16 L=2048 D=256 N=16 rank 16 fp32, "
                                    f"{args.disc.upper()}",
                        "B": B, "L": L, "D": Dc, "N": N, "rank": R})


def wl_dtproj(args, dev):
    return _wl_dtproj(args, dev, True)


def wl_dtproj_two_launch(args, dev):
    return _wl_dtproj(args, dev, False)


def _wl_bcproj(args, dev, fused):
    """Mamba-1 scan with B and C from x: B_t = x_t W_B, C_t = x_t W_C, at the
    interpolation workload's scan shape (B=16 L=2048 D=256 N=16 fp32, dt from
    sorted timestamps): formed inside the scan (bc_proj=), or as a matmul
    producing B and C followed by the scan."""
    import torch
    from tssm import selective_scan_forward, workloads
    w = workloads.interp_mamba1()
    g = torch.Generator().manual_seed(1006)
    B, L, Dc = w["V"].shape
    N = w["A_log"].shape[1]
    x0 = torch.randn(B, L, Dc, generator=g)
    W_bc = (torch.randn(Dc, 2 * N, generator=g) / Dc ** 0.5).to(dev)
    A_log = w["A_log"].to(dev)
    sets = []
    for i in range(max(args.sets, 3)):
        st = {"x": torch.roll(x0, shifts=i, dims=0).contiguous().to(dev),
              "tau": torch.roll(w["tau"], shifts=i, dims=0).contiguous().to(dev)}
        st["y"] = torch.empty_like(st["x"])
        st["Bm"] = torch.empty(B, L, N, device=dev)
        st["Cm"] = torch.empty(B, L, N, device=dev)
        sets.append(st)

    def step(i):
        d = sets[i % len(sets)]
        if fused:
            selective_scan_forward(d["x"], d["tau"], A_log, None, None, None, disc=args.disc,
                                   dt_is_tau=True, out=d["y"], bc_proj=W_bc)
        else:
            torch.matmul(d["x"], W_bc[:, :N], out=d["Bm"])
            torch.matmul(d["x"], W_bc[:, N:], out=d["Cm"])
            selective_scan_forward(d["x"], d["tau"], A_log, d["Bm"], d["Cm"], None,
                                   disc=args.disc, dt_is_tau=True, out=d["y"])

    def cpu():
        import numpy as np
        from oracle import cport
        x = _np32(x0)
        Wn = _np32(W_bc.cpu())
        tau = _np32(w["tau"])
        Al = _np32(w["A_log"])

        def run():
            Bm = np.ascontiguousarray(x @ Wn[:, :N])
            Cm = np.ascontiguousarray(x @ Wn[:, N:])
            dt = np.diff(tau, axis=1, prepend=0.0).astype(np.float32)
            cport.selective_scan(x, dt, Al, Bm, Cm, None, disc=args.disc)
        med = _timed_cpu(run, args.cpu_reps)
        return {"value": B * L * Dc / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"whole workload, {_runs_note()}, "
                                          f"{med:.3f} s each"}

    n = B * L * Dc
    nbytes = 4 * (2 * n + B * L + Dc * N + Dc * 2 * N)   # x, y, tau, A_log, W
    how = "formed in the scan" if fused else "matmul, then the scan"
    valu = {"lane_updates": n * N, "ops_per_update": 9, "exp2_per_update": 2}
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, valu=valu,
                kernel="sel_bcproj_state_kernel + sel_carry_kernel + sel_output_kernel" if fused
                else "matmul (B), matmul (C), sel_chunk_state_kernel, sel_carry_kernel, "
                     "sel_output_kernel",
                metric=f"Mamba-1 scan with B, C = x W ({how}) elements/sec, B=16 L=2048 D=256 "
                       "N=16 fp32",
                unit="elements/s",
                config={"workload": f"B_t = x_t W_B, C_t = x_t W_C ({how}) + Mamba-1 scan, "
                                    f"B=16 L=2048 D=256 N=16 fp32, dt from timestamps, "
                                    f"{args.disc.upper()}",
                        "B": B, "L": L, "D": Dc, "N": N})


def _wl_xproj(args, dev, fused):
    """Mamba-1 scan with the whole input projection x -> (dt, B, C): x_dbl =
    x W_x split into dt_raw (rank 16), B and C, dt = clamp(softplus(dt_raw W_dt
    + bias)), at B=16 L=2048 D=256 N=16 fp32: formed inside the scan
    (x_proj=), or as a matmul producing x_dbl, then the scan with the dt
    projection (dt_proj=) reading the dt_raw columns and B/C copied out."""
    import math
    import torch
    from tssm import selective_scan_forward, workloads
    w = workloads.interp_mamba1()
    g = torch.Generator().manual_seed(1007)
    B, L, Dc = w["V"].shape
    N = w["A_log"].shape[1]
    R = 16
    x0 = torch.randn(B, L, Dc, generator=g)
    W_x = (torch.randn(Dc, R + 2 * N, generator=g) / Dc ** 0.5).to(dev)
    W_dt = (torch.randn(R, Dc, generator=g) * (0.5 / R ** 0.5)).to(dev)
    bias = (math.log(math.expm1(0.05)) + torch.empty(Dc).uniform_(-0.5, 0.5, generator=g)).to(dev)
    dmin, dmax = 1e-3, 0.5
    A_log = w["A_log"].to(dev)
    sets = []
    for i in range(max(args.sets, 3)):
        st = {"x": torch.roll(x0, shifts=i, dims=0).contiguous().to(dev)}
        st["y"] = torch.empty_like(st["x"])
        st["xdbl"] = torch.empty(B, L, R + 2 * N, device=dev)
        st["raw"] = torch.empty(B, L, R, device=dev)
        st["Bm"] = torch.empty(B, L, N, device=dev)
        st["Cm"] = torch.empty(B, L, N, device=dev)
        sets.append(st)

    def step(i):
        d = sets[i % len(sets)]
        if fused:
            selective_scan_forward(d["x"], None, A_log, None, None, None, disc=args.disc,
                                   out=d["y"], x_proj=(W_x, W_dt, bias, dmin, dmax))
        else:
            torch.matmul(d["x"], W_x, out=d["xdbl"])
            d["raw"].copy_(d["xdbl"][..., :R])
            d["Bm"].copy_(d["xdbl"][..., R:R + N])
            d["Cm"].copy_(d["xdbl"][..., R + N:])
            selective_scan_forward(d["x"], d["raw"], A_log, d["Bm"], d["Cm"], None,
                                   disc=args.disc, out=d["y"],
                                   dt_proj=(W_dt, bias, dmin, dmax))

    def cpu():
        import numpy as np
        from oracle import cport
        x = _np32(x0)
        Wn, Wd, bn = _np32(W_x.cpu()), _np32(W_dt.cpu()), _np32(bias.cpu())
        Al = _np32(w["A_log"])

        def run():
            xd = x @ Wn
            acc = xd[..., :R] @ Wd + bn
            dt = np.clip(np.logaddexp(0.0, acc), dmin, dmax).astype(np.float32)
            cport.selective_scan(x, dt, Al, np.ascontiguousarray(xd[..., R:R + N]),
                                 np.ascontiguousarray(xd[..., R + N:]), None, disc=args.disc)
        med = _timed_cpu(run, args.cpu_reps)
        return {"value": B * L * Dc / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"whole workload, {_runs_note()}, "
                                          f"{med:.3f} s each"}

    n = B * L * Dc
    nbytes = 4 * (2 * n + Dc * N + Dc * (R + 2 * N) + R * Dc + Dc)  # x, y, A_log, W_x, W_dt, bias
    how = "formed in the scan" if fused else "matmul, then the scan with the dt projection"
    valu = {"lane_updates": n * N, "ops_per_update": 9, "exp2_per_update": 2}
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, valu=valu,
                kernel="sel_bcproj_state_kernel (x -> dt, B, C) + sel_carry_kernel + "
                       "sel_output_kernel" if fused
                else "matmul (x_dbl), copies, sel_chunk_state_kernel (dt projected), "
                     "sel_carry_kernel, sel_output_kernel",
                metric=f"Mamba-1 scan with dt, B, C from x ({how}) elements/sec, B=16 L=2048 "
                       "D=256 N=16 R=16 fp32",
                unit="elements/s",
                config={"workload": f"x_dbl = x W_x -> dt_raw, B, C; dt = clamp(softplus(dt_raw "
                                    f"W_dt + bias)) ({how}) + Mamba-1 scan, B=16 L=2048 D=256 "
                                    f"N=16 R=16 fp32, {args.disc.upper()}",
                        "B": B, "L": L, "D": Dc, "N": N, "R": R})


def wl_xproj(args, dev):
    return _wl_xproj(args, dev, True)


def wl_xproj_unfused(args, dev):
    return _wl_xproj(args, dev, False)


def wl_bcproj(args, dev):
    return _wl_bcproj(args, dev, True)


def wl_bcproj_two_launch(args, dev):
    return _wl_bcproj(args, dev, False)


def wl_ssd_long(args, dev):
    import torch
    from tssm import ssd_scan_forward, workloads
    w = workloads.ssd_long()
    base = {k: w[k].to(dev) for k in ("x", "dt", "B", "C")}
    A_log = w["A_log"].to(dev)
    B, L, H, P = base["x"].shape
    N = base["B"].shape[-1]
    sets = []
    for i in range(min(args.sets, 2)):
        s = {k: torch.roll(v, shifts=i * 997, dims=1).contiguous() for k, v in base.items()}
        s["y"] = torch.empty_like(s["x"])
        sets.append(s)

    def step(i):
        s = sets[i % len(sets)]
        ssd_scan_forward(s["x"], s["dt"], A_log, s["B"], s["C"], None, chunk=args.ssd_chunk,
                         disc=args.disc, out=s["y"])

    def cpu():
        from oracle import cport
        Ls = 32768
        arrs = [_np32(w[k][:, :Ls]) for k in ("x", "dt")] + [_np32(w["A_log"])] + \
               [_np32(w[k][:, :Ls]) for k in ("B", "C")]
        med = _timed_cpu(lambda: cport.ssd_scan(*arrs, None, None, disc=args.disc), args.cpu_reps)
        return {"value": B * Ls * H * P / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"first {Ls} of {L} steps (8 heads), {_runs_note()}, "
                                          f"{med:.3f} s each"}

    n = B * L * H * P
    nbytes = 2 * (2 * n + 2 * B * L * H * N) + 4 * B * L * H + 4 * H
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes,
                kernel="ssd_fused_wave_kernel",
                traffic="ssd_long_traffic.json",
                dtype="bf16",
                metric="SSD long-sequence scan elements/sec, B=1 L=262144 H=8 P=64 N=16 bf16",
                unit="elements/s",
                config={"workload": "SSD scan (decay per head, P x N state), B=1 L=262144 H=8 "
                                    f"P=64 N=16, chunk {args.ssd_chunk}, bf16 I/O, fp32 state, "
                                    f"{args.disc.upper()}",
                        "B": B, "L": L, "H": H, "P": P, "N": N, "chunk": args.ssd_chunk})


def wl_ssd_n64_long(args, dev):
    """bf16 N = 64 with one row per head and a long sequence (B=1 L=65536 H=8
    P=N=64): 16 (row, channel block) units, so the one-pass kernel runs 16
    time segments after the segment end-state and prefix passes."""
    import torch
    from tssm import ssd_scan_forward, workloads
    w = workloads.ssd_long(L=65536, N=64)
    base = {k: w[k].to(dev) for k in ("x", "dt", "B", "C")}
    A_log = w["A_log"].to(dev)
    B, L, H, P = base["x"].shape
    N = base["B"].shape[-1]
    sets = []
    for i in range(min(args.sets, 2)):
        s = {k: torch.roll(v, shifts=i * 997, dims=1).contiguous() for k, v in base.items()}
        s["y"] = torch.empty_like(s["x"])
        sets.append(s)

    def step(i):
        s = sets[i % len(sets)]
        ssd_scan_forward(s["x"], s["dt"], A_log, s["B"], s["C"], None, chunk=args.ssd_chunk,
                         disc=args.disc, out=s["y"])

    def cpu():
        from oracle import cport
        arrs = [_np32(w[k]) for k in ("x", "dt")] + [_np32(w["A_log"])] + \
               [_np32(w[k]) for k in ("B", "C")]
        med = _timed_cpu(lambda: cport.ssd_scan(*arrs, None, None, disc=args.disc), args.cpu_reps)
        return {"value": B * L * H * P / med, "unit": "elements/s", "cores": cport.threads(),
                "kind": "port", "sample": f"whole workload, {_runs_note()}, "
                                          f"{med:.3f} s each"}

    n = B * L * H * P
    nbytes = 2 * (2 * n + 2 * B * L * H * N) + 4 * B * L * H + 4 * H
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes,
                kernel="ssd_seg_state_kernel + ssd_seg_prefix_kernel + ssd_seq_kernel",
                traffic="ssd_n64_long_traffic.json",
                dtype="bf16",
                metric="SSD long-sequence scan elements/sec, B=1 L=65536 H=8 P=N=64 bf16",
                unit="elements/s",
                config={"workload": "SSD scan (decay per head, P x N state), B=1 L=65536 H=8 "
                                    f"P=N=64, chunk {args.ssd_chunk}, bf16 I/O, fp32 state, "
                                    f"{args.disc.upper()}, time-segmented one-pass kernel",
                        "B": B, "L": L, "H": H, "P": P, "N": N, "chunk": args.ssd_chunk})


def wl_ssd_stream(args, dev):
    import torch
    from tssm import ssd_stream_step, workloads
    w = workloads.ssd_stream()
    S, H, P, N = w["S"], w["H"], w["P"], w["N"]
    A_log = w["A_log"].to(dev)
    pool = [{k: v.to(dev) for k, v in st.items()} for st in w["steps"]]
    state = torch.zeros(S, H, P, N, device=dev)
    ys = [torch.empty(S, H, P, device=dev) for _ in range(2)]

    def step(i):
        s = pool[i % len(pool)]
        ssd_stream_step(s["x"], s["dt"], A_log, s["B"], s["C"], None, state, disc=args.disc,
                        out=ys[i % 2])

    def cpu():
        import numpy as np
        from oracle import cport
        Ss = 256
        st = np.zeros((Ss, H, P, N), np.float32)
        steps = [[_np32(p[k][:Ss]) for k in ("x", "dt", "B", "C")] for p in w["steps"][:4]]
        t0 = time.perf_counter()
        for xs, dts, Bs, Cs in steps:
            cport.ssd_stream_step(xs, dts, _np32(w["A_log"]), Bs, Cs, None, st, disc=args.disc)
        el = (time.perf_counter() - t0) / len(steps)
        return {"value": Ss / el, "unit": "stream-steps/s", "cores": cport.threads(),
                "kind": "port", "sample": f"{Ss} of {S} streams, {len(steps)} steps, "
                                          f"{el * 1e3:.2f} ms per step"}

    nbytes = 2 * S * H * P * N * 4 + 4 * (2 * S * H * P + 2 * S * H * N + S) + 4 * H
    return dict(step=step, cpu=cpu, elements=S, bytes=nbytes, kernel="ssd_stream_step_kernel",
                metric="streaming SSD step: stream-steps/sec and p50 step latency, 4096 streams "
                       "H=32 P=64 N=128 fp32 state",
                unit="stream-steps/s",
                config={"workload": "streaming SSD step, state [4096,32,64,128] fp32 resident in "
                                    f"HBM, per-stream dt, {args.disc.upper()}",
                        "S": S, "H": H, "P": P, "N": N})


# ------------------------------------------------------------------ per-row sweep
def rows_sweep(args, dev):
    """Each drop-in kernel of the path (and its model-layer neighbours) at a
    config-sized shape: average launch time over back-to-back launches (HIP
    events on the launch stream), algorithmic bytes (inputs read once, outputs
    written once, in the dtypes used) and the fraction of 8 TB/s.  Prints one
    JSON line with a "rows" list; the table goes to stderr."""
    import math
    import torch
    import discretize_kernel as dk
    import fused_interp_kernel as fi
    import fused_ssm_interp as fs
    import multihead_ssm_kernel as mk
    import ssm_scan as ss
    import streaming_inference_kernel as sk
    g = torch.Generator(device=dev).manual_seed(7)
    rnd = lambda *shape, dtype=torch.float32: torch.randn(*shape, generator=g, device=dev).to(dtype)  # noqa: E731
    uni = lambda lo, hi, *shape: torch.empty(*shape, device=dev).uniform_(lo, hi, generator=g)  # noqa: E731
    stream = torch.cuda.current_stream(dev)
    reps = max(5, min(args.steps, 50))
    rows = []

    # Every timed launch starts from a cold last-level cache: reading 512 MB
    # (outside the timed events) replaces the 256 MB Infinity Cache with clean
    # lines, so a row's inputs are never served from the previous repetition
    # (a write would leave dirty lines that drain to HBM during the timed
    # launch).  Each launch is bracketed by its own events; the row's time is
    # the median.
    flush = torch.zeros(128 << 20, dtype=torch.float32, device=dev)

    def median_us(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        for e0, e1 in ev:
            flush.sum()
            e0.record(stream)
            fn()
            e1.record(stream)
        torch.cuda.synchronize()
        return statistics.median(e0.elapsed_time(e1) for e0, e1 in ev) * 1e3

    # A device copy (torch's copy_) that reads and writes the row's bytes in
    # total, timed the same way: what one launch moving those bytes costs
    # here, launch latency and the cold cache included.
    copy_cache = {}

    def copy_us(nbytes):
        key = max(1, int(nbytes) >> 20)
        if key not in copy_cache:
            src = torch.empty(max(1024, int(nbytes) // 8), device=dev).uniform_()
            dst = torch.empty_like(src)
            copy_cache[key] = median_us(lambda: dst.copy_(src))
            del src, dst
        return copy_cache[key]

    def timeit(name, shape, nbytes, fn):
        us = median_us(fn)
        cus = copy_us(nbytes)
        gbps = nbytes / (us * 1e-6) / 1e9
        rows.append({"row": name, "shape": shape, "us": round(us, 2), "bytes": int(nbytes),
                     "gbps": round(gbps, 1), "frac": round(gbps / 8000.0, 4),
                     "copy_us": round(cus, 2), "vs_copy": round(cus / us, 3)})
        log(f"{name:52s} {shape:34s} {us:9.1f} us {gbps:8.0f} GB/s {100 * gbps / 8000:5.1f}%"
            f"  (copy of the same bytes {cus:7.1f} us)")

    B, T, H = 8, 4096, 1024          # lanes of the headline config
    n = B * T * H
    # a1/a2 ZOH discretize, a19 its backward
    A = uni(math.log(0.5), math.log(5.0), H)
    dt = torch.exp(uni(-6.0, 0.5, B, T))
    for dtype, kern, tag in ((torch.float32, dk.zoh_discretize_diag_kernel, "fp32"),
                             (torch.bfloat16, dk.zoh_discretize_diag_bf16_kernel, "bf16")):
        Bm = rnd(B, T, H, dtype=dtype)
        Ab, Bb = torch.empty_like(Bm), torch.empty_like(Bm)
        es = Bm.element_size()
        timeit(f"a1/a2 zoh_discretize_diag ({tag})", f"B={B} T={T} H={H}", n * 3 * es + B * T * 4,
               lambda: kern[(B, T, H // 256)](A, Bm, dt, Ab, Bb, B, T, H, *Bm.stride(),
                                              *dt.stride(), *Ab.stride(), *Bb.stride(),
                                              BLOCK_H=256))
        if dtype == torch.float32:
            dAb, dBb, dB = rnd(B, T, H), rnd(B, T, H), torch.empty_like(Bm)
            dA, ddt = torch.zeros(H, device=dev), torch.empty(B, T, device=dev)
            timeit("a19 zoh_discretize_bwd (fp32)", f"B={B} T={T} H={H}", n * 5 * 4 + B * T * 8,
                   lambda: dk.zoh_discretize_bwd_kernel[(B, T, H // 256)](
                       A, Bm, dt, Ab, dAb, dBb, dA, dB, ddt, B, T, H, *Bm.stride(),
                       *dt.stride(), *Ab.stride(), *dBb.stride(), BLOCK_H=256))
        del Bm, Ab, Bb
    # a21 dt projection (Mamba-1 shape: D = 256 channels, rank 16)
    Bd, Td, Hd, R = 16, 2048, 256, 16
    raw, W, bias = rnd(Bd, Td, R), rnd(R, Hd) / 4, rnd(Hd)
    dto = torch.empty(Bd, Td, Hd, device=dev)
    timeit("a21 dt_project_softplus", f"B={Bd} T={Td} H={Hd} R={R}",
           4 * (Bd * Td * (R + Hd) + R * Hd + Hd),
           lambda: dk.dt_project_softplus_kernel[(Bd, Td, 1)](
               raw, W, bias, dto, Bd, Td, Hd, R, *raw.stride(), *W.stride(), *dto.stride(),
               DT_MIN=1e-3, DT_MAX=0.1, BLOCK_H=256, BLOCK_R=16))
    del raw, dto
    # a4-a8 elementwise scan (ssm_forward), a20 ssm_backward
    u, Bm, Cm = rnd(B, T, H), rnd(B, T, H), rnd(B, T, H)
    Am = uni(0.5, 1.0, B, T, H)
    Dv = rnd(H)
    out = {}
    timeit("a4-a8 ssm_forward (single pass)", f"B={B} L={T} H={H}", n * 6 * 4,
           lambda: out.update(r=ss.ssm_forward(u, Am, Bm, Cm, Dv, BLK=256)))
    y_, h_ = out["r"]
    dY = rnd(B, T, H)
    timeit("a20 ssm_backward (single pass)", f"B={B} L={T} H={H}", n * 10 * 4,
           lambda: ss.ssm_backward(u, Am, Bm, Cm, h_, dY, BLK=256))
    del u, Bm, Cm, Am, y_, h_, dY, out
    # a9-a11 multihead phase-exact kernels (reference layouts, fp32)
    nh, hd, BLK = 16, 64, 128
    from tssm import workloads
    w = workloads.multihead(B=B, L=T, H=nh, P=hd, dtype=torch.float32)
    u, Bm, Cm, dtm = (w[k].to(dev) for k in ("u", "B", "C", "dt"))
    A_log = w["A_log"].to(dev)
    Dm = rnd(nh * hd)
    nblk = 1 << (((T + BLK - 1) // BLK) - 1).bit_length()
    loc_a = torch.empty(B, T, nh, hd, device=dev)
    loc_x = torch.empty_like(loc_a)
    carry = torch.empty(2 * B * nh * hd * nblk, device=dev)
    y = torch.empty(B, T, nh * hd, device=dev)
    # reads u and B (C is a parameter the local phase does not read), writes loc_a, loc_x
    timeit("a9 multihead_ssm_fwd_local", f"B={B} L={T} nh={nh} hd={hd}", n * 4 * 4 + B * T * nh * 4,
           lambda: mk.multihead_ssm_fwd_local_kernel[(B * nh, nblk)](
               u, A_log, Bm, Cm, dtm, loc_a, loc_x, carry, B, T, nh * hd, nh, hd, *u.stride(),
               *A_log.stride(), *Bm.stride(), *Cm.stride(), *dtm.stride(), BLK_L=BLK, NBLK=nblk,
               HEAD_DIM=hd))
    timeit("a10 multihead_ssm_carry_scan", f"{B * nh * hd} lanes x {nblk} chunks",
           2 * 2 * B * nh * hd * nblk * 4,
           lambda: mk.multihead_ssm_carry_scan_kernel[(B * nh * hd,)](carry, B * nh * hd, nblk))
    timeit("a11 multihead_ssm_output", f"B={B} L={T} nh={nh} hd={hd}", n * 5 * 4,
           lambda: mk.multihead_ssm_output_kernel[(B * nh, nblk)](
               loc_a, loc_x, carry, Cm, Dm, u, y, B, T, nh * hd, nh, hd, *u.stride(),
               *Cm.stride(), BLK_L=BLK, NBLK=nblk, HEAD_DIM=hd))
    del u, Bm, Cm, dtm, loc_a, loc_x, carry, y, w
    # a12 time-aware interpolation at B=16 T=2048 F=256 (the interpolation + Mamba-1 workload shape)
    wi = workloads.interp_mamba1()
    V, M, tau = (wi[k].to(dev) for k in ("V", "M", "tau"))
    Bi, Ti, Fi = V.shape
    Vh = torch.empty_like(V)
    timeit("a12 fused_time_aware_interp (fp32)", f"B={Bi} T={Ti} F={Fi} K=10 FTILE=128",
           Bi * Ti * Fi * 12 + Bi * Ti * 4,
           lambda: fi.fused_time_aware_interp_kernel[(Bi, Ti, Fi // 128)](
               V, M, tau, Vh, Bi, Ti, Fi, *V.stride(), *M.stride(), *tau.stride(), *Vh.stride(),
               K=10, FTILE=128))
    # opt-in corrected interpolation (per-feature neighbours), same shape
    from tssm import time_aware_interp_corrected
    timeit("f4 interp corrected (fp32)", f"B={Bi} T={Ti} F={Fi} K=10", Bi * Ti * Fi * 12 + Bi * Ti * 4,
           lambda: time_aware_interp_corrected(V, M, tau, K=10, out=Vh))
    # a15 interp + SSM step at one t_cur (per-step launch of the reference loop)
    Ab1, Bb1 = torch.rand(Fi, device=dev), rnd(Fi)
    h_in, h_out = rnd(Bi, Fi), torch.empty(Bi, Fi, device=dev)
    timeit("a15 fused_interp_ssm_step (one step)", f"B={Bi} F={Fi} K=10 t=1000",
           Bi * Fi * 4 * (2 * 21 + 3) + Bi * 21 * 4,
           lambda: fs.fused_interp_ssm_step_kernel[(Bi, Fi // 128)](
               V, M, tau, Ab1, Bb1, h_in, Vh, h_out, Bi, Ti, Fi, *V.stride(), *M.stride(),
               *tau.stride(), *Vh.stride(), *h_in.stride(), *h_out.stride(), 1000, K=10,
               FTILE=128))
    del V, M, tau, Vh, wi
    # a16/a17 streaming in-place step, a18 ring interp + step
    S, Hs = 4096, 1024
    for dtype, kern, tag in ((torch.float32, sk.streaming_ssm_inplace_kernel, "fp32"),
                             (torch.bfloat16, sk.streaming_ssm_inplace_bf16_kernel, "bf16")):
        v, hs, Cs = rnd(S, Hs, dtype=dtype), rnd(S, Hs, dtype=dtype), rnd(S, Hs, dtype=dtype)
        Abs, Bbs, Ds = (torch.rand(Hs, device=dev).to(dtype) for _ in range(3))
        ys = torch.empty_like(v)
        es = v.element_size()
        timeit(f"a16/a17 streaming_ssm_inplace ({tag})", f"S={S} H={Hs}", S * Hs * 5 * es,
               lambda: kern[(S, Hs // 256)](v, hs, Abs, Bbs, Cs, Ds, ys, S, Hs, *v.stride(),
                                            *hs.stride(), *Cs.stride(), BLOCK_H=256))
    Sr, Hr, KR = 4096, 1024, 11
    ring_V, ring_M = rnd(Sr, KR, Hr), (torch.rand(Sr, KR, Hr, device=dev) < 0.3).float()
    ring_tau = torch.arange(KR, device=dev, dtype=torch.float32).repeat(Sr, 1)
    head = torch.zeros(Sr, dtype=torch.int32, device=dev)
    vn, mn = rnd(Sr, Hr), (torch.rand(Sr, Hr, device=dev) < 0.3).float()
    tn = torch.full((Sr,), 20.0, device=dev)
    hr, Cr, yr = rnd(Sr, Hr), rnd(Sr, Hr), torch.empty(Sr, Hr, device=dev)
    Abr, Bbr, Dr = (torch.rand(Hr, device=dev) for _ in range(3))
    timeit("a18 streaming_interp_then_ssm (ring)", f"S={Sr} H={Hr} KRING={KR}", Sr * Hr * 4 * 8,
           lambda: sk.streaming_interp_then_ssm_kernel[(Sr, Hr // 128)](
               ring_V, ring_M, ring_tau, head, vn, mn, tn, hr, Abr, Bbr, Cr, Dr, yr, Sr, Hr,
               KR - 1, *ring_V.stride(), *vn.stride(), *hr.stride(), *Cr.stride(), BLOCK_H=128,
               KRING=KR))
    # opt-in corrected interpolation (per-feature neighbours), same shapes
    from tssm import streaming_interp_step_corrected
    timeit("f4 streaming corrected (ring)", f"S={Sr} H={Hr} KRING={KR}", Sr * Hr * 4 * 8,
           lambda: streaming_interp_step_corrected(ring_V, ring_M, ring_tau, head, vn, mn, tn, hr,
                                                   Abr, Bbr, Cr, Dr, yr))
    # model layers (fp32, headline lane count)
    x, dout = rnd(B, T, H), rnd(B, T, H)
    wv, bv = rnd(H), rnd(H)
    o1, o2 = torch.empty_like(x), torch.empty_like(x)
    dw, db = torch.zeros(H, device=dev), torch.zeros(H, device=dev)
    timeit("layernorm_kernel", f"B={B} L={T} H={H}", n * 8,
           lambda: fs.layernorm_kernel[(B, T)](x, wv, bv, o1, B, T, H, *x.stride(), EPS=1e-5,
                                               BLOCK_H=H))
    timeit("layernorm_bwd_kernel", f"B={B} L={T} H={H}", n * 12,
           lambda: fs.layernorm_bwd_kernel[(B, T)](dout, x, wv, o1, dw, db, B, T, H,
                                                   x.stride(0), x.stride(1), EPS=1e-5, BLOCK_H=H))
    timeit("swiglu_kernel", f"B={B} L={T} H={H}", n * 12,
           lambda: fs.swiglu_kernel[(B, T)](x, dout, o1, B, T, H, x.stride(0), x.stride(1),
                                            BLOCK_H=H))
    o3 = torch.empty_like(x)
    timeit("swiglu_bwd_kernel", f"B={B} L={T} H={H}", n * 20,
           lambda: fs.swiglu_bwd_kernel[(B, T)](dout, x, o3, o1, o2, B, T, H, x.stride(0),
                                                x.stride(1), BLOCK_H=H))
    del o3
    keep = (torch.rand(n, device=dev) < 0.9).to(torch.uint8)
    xf, rf, of = x.view(-1), dout.view(-1), o1.view(-1)
    timeit("residual_add_kernel", f"N={n}", n * 12,
           lambda: mk.residual_add_kernel[(n // 1024,)](xf, rf, of, n, BLOCK=1024))
    timeit("dropout_residual_kernel", f"N={n}", n * 13,
           lambda: mk.dropout_residual_kernel[(n // 1024,)](xf, rf, keep, of, n, 0.9, BLOCK=1024))
    mask = (torch.rand(B, T, device=dev) < 0.8).to(torch.uint8)
    timeit("masked_fill_zero_kernel", f"B={B} T={T} H={H}", n * 8 + B * T,
           lambda: sk.masked_fill_zero_kernel[(n // 1024,)](x, mask, o1, B, T, H, BLOCK=1024))
    lo = torch.empty(B, device=dev)
    b1 = torch.zeros(1, device=dev)
    timeit("mean_pool_logit_kernel", f"B={B} T={T} H={H}", n * 4,
           lambda: sk.mean_pool_logit_kernel[(B,)](x, wv, b1, lo, B, T, H, *x.stride(),
                                                   BLOCK_H=256, BLOCK_T=16))
    gm = math.exp(sum(math.log(max(r["frac"], 1e-6)) for r in rows) / len(rows))
    gmc = math.exp(sum(math.log(max(r["vs_copy"], 1e-6)) for r in rows) / len(rows))
    print(json.dumps({"metric": "per-row kernel HBM bandwidth (algorithmic bytes / launch time)",
                      "value": round(gm, 4), "unit": "geometric-mean fraction of 8 TB/s",
                      "vs_copy_geomean": round(gmc, 4),
                      "n_gpus": 1, "steps": reps, "warmup": 3, "higher_is_better": True,
                      "dtype": "f32", "data": "synthetic", "config": {"workload": "row sweep"},
                      "rows": rows}))


WORKLOADS = {"bcproj": wl_bcproj, "bcproj_two_launch": wl_bcproj_two_launch,
             "xproj": wl_xproj, "xproj_unfused": wl_xproj_unfused,
             "multihead": wl_multihead, "mamba1_small": wl_mamba1_small,
             "interp_mamba1": wl_interp_mamba1, "ssd_long": wl_ssd_long,
             "ssd_config1": wl_ssd_config1, "ssd_n64_long": wl_ssd_n64_long,
             "ssd_stream": wl_ssd_stream, "dtproj": wl_dtproj,
             "dtproj_two_launch": wl_dtproj_two_launch}


def traffic_from_profile(name):
    if not name:
        return None
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("hbm_bytes_per_launch")
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 50; 10000 for ssd_stream, the streaming run length)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["rows"], default="multihead")
    ap.add_argument("--disc", choices=["zoh", "euler"], default="zoh")
    ap.add_argument("--a-log-const", type=float, default=None,
                    help="multihead: every A_log entry set to this value (e.g. -4.6 = log 0.01, "
                         "a slowly decaying input of the headline shape)")
    ap.add_argument("--a-per-channel", action="store_true",
                    help="multihead: pass A_log as [H, P] (the reference kernel's layout, the "
                         "per-head value repeated) instead of [H] (one decay per head)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run torch copies of a 256 MiB buffer (scales rocprof "
                         "FETCH_SIZE/WRITE_SIZE to bytes); prints nothing else")
    ap.add_argument("--sets", type=int, default=3)
    ap.add_argument("--scan-chunk", type=int, default=256,
                    help="interp_mamba1: steps per chunk of the selective scan")
    ap.add_argument("--ssd-chunk", type=int, default=256,
                    help="steps per chunk of the SSD scan passes (multiple of 64, <= 1024)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="time the CPU baseline until this much CPU work has run")
    args = ap.parse_args()
    global CPU_SECONDS
    CPU_SECONDS = args.cpu_seconds
    if args.steps is None:
        args.steps = 10000 if args.workload == "ssd_stream" else 50
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every workload is data-parallel over rows or "
              "streams, and the benchmark runs on a single MI355X; run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        src = torch.ones(64 * 2**20, dtype=torch.float32, device=dev)   # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copied 256 MiB x5")
        return

    if args.workload == "rows":
        return rows_sweep(args, dev)
    log(f"workload {args.workload}: generating inputs ...")
    wl = WORKLOADS[args.workload](args, dev)
    step = wl["step"]
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)

    def timed(per_step_events):
        """Time ``args.steps`` steps.  A GPU sleep queued first keeps the device
        busy while the host enqueues every launch, so kernels run back to back
        and the events time the GPU, not the host."""
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)] if per_step_events else []
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(int(2e8))
        t0.record(stream)
        for i in range(args.steps):
            if per_step_events:
                ev[i][0].record(stream)
            step(i)
            if per_step_events:
                ev[i][1].record(stream)
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1), [a.elapsed_time(b) for a, b in ev]

    total_ms, _ = timed(False)        # the measured K steps, back to back
    _, per = timed(True)              # per-step events: p50 latency only
    import tssm
    tssm.check()   # raises if a bounded look-back wait expired in any run above
    ms_per_step = total_ms / args.steps
    # Roofline: the kernels of a step run back to back on the launch stream,
    # so the timed region's average is their average launch duration (an
    # event pair around every launch adds ~2 us and is used for p50 only).
    kern_ms = ms_per_step
    achieved = wl["bytes"] / (kern_ms * 1e-3) / 1e9
    log(f"{ms_per_step * 1e3:.1f} us/step over the timed region, {achieved:.0f} GB/s; "
        f"per-step events p50 {statistics.median(per) * 1e3:.1f} us, "
        f"min {min(per) * 1e3:.1f} us")

    # A device copy (torch's copy_) moving the same bytes per step (half read,
    # half written), over as many rotated buffer sets and timed the same way:
    # what a plain streaming kernel of this size reaches on this box.
    copy_ref = None
    if not wl.get("valu") and wl["bytes"] <= (2 << 30):
        half = max(1024, int(wl["bytes"]) // 8)
        bufs = [(torch.empty(half, device=dev).uniform_(), torch.empty(half, device=dev))
                for _ in range(max(1, args.sets))]
        real_step = step

        def step(i):  # noqa: F811 -- the copy stands in for the workload's step
            src, dst = bufs[i % len(bufs)]
            dst.copy_(src)

        for i in range(args.warmup):
            step(i)
        copy_total, _ = timed(False)
        step = real_step
        del bufs
        copy_ms = copy_total / args.steps
        copy_gbs = wl["bytes"] / (copy_ms * 1e-3) / 1e9
        copy_ref = {"ms_per_step": copy_ms, "achieved": copy_gbs, "unit": "GB/s",
                    "frac": copy_gbs / PEAK_GBS, "kernel_vs_copy": copy_ms / ms_per_step}
        log(f"device copy of the same bytes: {copy_ms * 1e3:.1f} us/step, {copy_gbs:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        log("timing the CPU baseline ...")
        cpu = wl["cpu"]()

    out = {
        "metric": wl["metric"],
        "value": wl["elements"] / (ms_per_step * 1e-3),
        "unit": wl["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # I/O dtype of x/B/C/y; arithmetic and the state are fp32 in every workload
        "dtype": wl.get("dtype", "f32"),
        "data": "synthetic",
        "config": dict(wl["config"], parallelism="single GPU", arithmetic="f32", state="f32"),
        "roofline": {
            "bound": "hbm",
            "kernel": wl["kernel"],
            "achieved": achieved,
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_GBS,
            "traffic": traffic_from_profile(wl.get("traffic")),
            "algorithmic_bytes_per_launch": wl["bytes"],
            "kernel_avg_us": kern_ms * 1e3,
            "copy_reference": copy_ref,
        },
        "cpu_baseline": cpu,
        "p50_step_ms": statistics.median(per),
    }
    v = wl.get("valu")
    if v:
        # vector-issue bound: the algorithm's floor of lane operations (exp2
        # weighted by its issue cost) over the measured time, against the
        # published lane-op rate; the HBM figures stay as secondary keys
        slots = v["ops_per_update"] + EXP2_SLOTS * v["exp2_per_update"]
        got = v["lane_updates"] * slots / (kern_ms * 1e-3) / 1e12
        hbm = out["roofline"]
        out["roofline"] = {
            "bound": "valu",
            "kernel": wl["kernel"],
            "achieved": got,
            "peak": PEAK_VALU_TLANE,
            "unit": "T lane-ops/s",
            "frac": got / PEAK_VALU_TLANE,
            "traffic": hbm["traffic"],
            "ops_per_lane_update": v["ops_per_update"],
            "exp2_per_lane_update": v["exp2_per_update"],
            "exp2_issue_slots": EXP2_SLOTS,
            "lane_updates_per_launch": v["lane_updates"],
            "hbm_achieved_GBs": hbm["achieved"],
            "hbm_frac": hbm["frac"],
            "algorithmic_bytes_per_launch": wl["bytes"],
            "kernel_avg_us": kern_ms * 1e3,
        }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
