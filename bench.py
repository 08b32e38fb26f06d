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
  ssd_stream     streaming SSD step, 4096 streams H=32 P=64 N=128 fp32 state

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
HEADLINE_METRIC = "scan elements/sec + achieved HBM GB/s (% of peak), B=8 L=4096 H=16 P=64 N=64"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _np32(t):
    import numpy as np
    return np.ascontiguousarray(t.float().numpy())


def _timed_cpu(fn, reps):
    fn()   # warm
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


# ------------------------------------------------------------------ workloads
def wl_multihead(args, dev):
    import torch
    from tssm import multihead_ssm_forward, workloads
    B, L, H, P = 8, 4096, 16, 64
    w = workloads.multihead(B=B, L=L, H=H, P=P)
    a_key = "A_log" if args.a_per_channel else "A_log_h"
    base = {k: w[k].to(dev) for k in ("u", "B", "C", "dt")}
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
                "kind": "port", "sample": f"whole workload, median of {args.cpu_reps} runs, "
                                          f"{med:.3f} s each"}

    n = B * L * H * P
    nbytes = workloads.multihead_bytes(B, L, H, P, io_bytes=2) - H * P * 4 + A_log.numel() * 4
    cfg = {"workload": "fused multihead DIAG chunked scan, B=8 L=4096 H=16 P=N=64, chunk 128, "
                       f"bf16 x/B/C/y, fp32 dt/state, {args.disc.upper()} discretization",
           "B": B, "L": L, "H": H, "P": P, "N": P, "chunk": 128, "disc": args.disc,
           "io_dtype": "bf16", "state_dtype": "f32",
           "a_log": "per channel [H, P]" if args.a_per_channel else "per head [H]"}
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, kernel="mh_scan_fused_kernel",
                metric=HEADLINE_METRIC, unit="elements/s", config=cfg,
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
                "kind": "port", "sample": f"batch 0 of {B}, median of {args.cpu_reps} runs, "
                                          f"{med:.3f} s each"}

    n = B * L * H * P
    nbytes = 2 * (2 * n + 2 * B * L * H * N) + 4 * B * L * H + 4 * H
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes,
                kernel="ssd_state_kernel + ssd_pass_kernel + ssd_out_kernel",
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
                "sample": f"whole workload x{reps}, median of 3, {med * 1e6:.1f} us each"}

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
    w = workloads.interp_mamba1()
    d = {k: v.to(dev) for k, v in w.items()}
    B, T, F = d["V"].shape
    N = d["A_log"].shape[1]

    def step(i):
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
                "kind": "port", "sample": f"whole workload, median of {args.cpu_reps} runs, "
                                          f"{med:.3f} s each"}

    n = B * T * F
    nbytes = 4 * (4 * n + B * T + F * N + 2 * B * T * N)   # V, M in; Vhat, y out
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes, kernel="mh_scan_fused_kernel",
                metric="interp + Mamba-1 scan elements/sec, B=16 T=2048 F=256 N=16 fp32",
                unit="elements/s",
                config={"workload": "time-aware interpolation (K=10, FTILE=128, 30% missing) + "
                                    f"Mamba-1 scan, B=16 T=2048 F=256 N=16 fp32, {args.disc.upper()}",
                        "B": B, "T": T, "F": F, "N": N, "K": 10, "FTILE": 128})


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
                "kind": "port", "sample": f"first {Ls} of {L} steps (8 heads), median of "
                                          f"{args.cpu_reps} runs, {med:.3f} s each"}

    n = B * L * H * P
    nbytes = 2 * (2 * n + 2 * B * L * H * N) + 4 * B * L * H + 4 * H
    return dict(step=step, cpu=cpu, elements=n, bytes=nbytes,
                kernel="ssd_state_kernel + ssd_pass_kernel + ssd_out_kernel",
                metric="SSD long-sequence scan elements/sec, B=1 L=262144 H=8 P=64 N=16 bf16",
                unit="elements/s",
                config={"workload": "SSD scan (decay per head, P x N state), B=1 L=262144 H=8 "
                                    f"P=64 N=16, chunk {args.ssd_chunk}, bf16 I/O, fp32 state, "
                                    f"{args.disc.upper()}",
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


WORKLOADS = {"multihead": wl_multihead, "mamba1_small": wl_mamba1_small,
             "interp_mamba1": wl_interp_mamba1, "ssd_long": wl_ssd_long,
             "ssd_config1": wl_ssd_config1,
             "ssd_stream": wl_ssd_stream}


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
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="multihead")
    ap.add_argument("--disc", choices=["zoh", "euler"], default="zoh")
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
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 10000 if args.workload == "ssd_stream" else 50
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every workload is data-parallel over rows or "
              "streams and this build runs on a single MI355X; run with --gpus 1",
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
    ms_per_step = total_ms / args.steps
    # Roofline: the kernels of a step run back to back on the launch stream,
    # so the timed region's average is their average launch duration (an
    # event pair around every launch adds ~2 us and is used for p50 only).
    kern_ms = ms_per_step
    achieved = wl["bytes"] / (kern_ms * 1e-3) / 1e9
    log(f"{ms_per_step * 1e3:.1f} us/step over the timed region, {achieved:.0f} GB/s; "
        f"per-step events p50 {statistics.median(per) * 1e3:.1f} us, "
        f"min {min(per) * 1e3:.1f} us")

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
        "dtype": "f32",
        "data": "synthetic",
        "config": dict(wl["config"], parallelism="single GPU"),
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
        },
        "cpu_baseline": cpu,
        "p50_step_ms": statistics.median(per),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
