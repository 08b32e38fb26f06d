"""Seeded synthetic inputs for the five measured workloads, and their
algorithmic byte counts.

Every generator draws on the CPU from ``torch.Generator().manual_seed(seed)``
in a fixed order (so the same seed gives the same inputs on any machine) and
returns a dict of CPU tensors; callers move them to the device.  ``scale``
shrinks the sequence/stream axis for quick tests while keeping the
distributions.

  mamba1_small   B=2 L=256 D=16 N=16 fp32, dt ~ Exp(mean 0.05) clamped to
                 [1e-3, 1] per (b,t), A_log [D,N] ~ U(log .5, log 5),
                 B, C [B,L,N] ~ N(0, 1/N), x ~ N(0,1)
  multihead      B=8 L=4096 H=16 P=N=64 chunk 128; x, B, C bf16; dt fp32 =
                 softplus(N(0,1)) per (b,t,h) * Exp(mean 1) gap per (b,t);
                 A_log[h] ~ U(log 1, log 16) per head
  interp_mamba1  B=16 T=2048 F=D=256 N=16 fp32; tau = sorted U(0,100);
                 M ~ Bernoulli(0.7) (1 = observed), V ~ N(0,1) with V=0 where
                 missing; A_log, B, C as mamba1_small; K=10, FTILE=128
  ssd_long       B=1 L=262144 H=8 P=64 N=16 chunk 256; x, B, C bf16; dt ~
                 LogNormal(-3, 1.5) per (t,h); A_log as multihead
  ssd_stream     S=4096 H=32 P=64 N=128 fp32 state; per step x ~ N(0,1),
                 dt ~ Exp(mean 0.1) per stream, B, C ~ N(0, 1/N)
  dtproj_mamba1  the interpolation workload's scan shape with dt produced by a
                 rank-16 projection (dt_raw, W, bias)
"""
from __future__ import annotations

import math

import torch


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _exp(g, shape, mean):
    return torch.empty(shape).exponential_(1.0 / mean, generator=g)


def _unif(g, shape, lo, hi):
    return torch.rand(shape, generator=g) * (hi - lo) + lo


def mamba1_small(seed=1000, B=2, L=256, D=16, N=16):
    g = _gen(seed)
    dt = _exp(g, (B, L), 0.05).clamp_(1e-3, 1.0)
    A_log = _unif(g, (D, N), math.log(0.5), math.log(5.0))
    Bm = torch.randn(B, L, N, generator=g) / math.sqrt(N)
    Cm = torch.randn(B, L, N, generator=g) / math.sqrt(N)
    x = torch.randn(B, L, D, generator=g)
    return {"x": x, "dt": dt, "A_log": A_log, "B": Bm, "C": Cm}


def multihead(seed=1001, B=8, L=4096, H=16, P=64, dtype=torch.bfloat16):
    g = _gen(seed)
    x = torch.randn(B, L, H * P, generator=g).to(dtype)
    Bm = (torch.randn(B, L, H, P, generator=g) / math.sqrt(P)).to(dtype)
    Cm = (torch.randn(B, L, H, P, generator=g) / math.sqrt(P)).to(dtype)
    z = torch.randn(B, L, H, generator=g)
    gap = _exp(g, (B, L, 1), 1.0)
    dt = torch.nn.functional.softplus(z) * gap
    A_log_h = _unif(g, (H,), math.log(1.0), math.log(16.0))
    return {"u": x, "B": Bm, "C": Cm, "dt": dt, "A_log_h": A_log_h,
            "A_log": A_log_h[:, None].expand(H, P).contiguous()}


def interp_mamba1(seed=1002, B=16, T=2048, F=256, N=16):
    g = _gen(seed)
    tau = torch.sort(_unif(g, (B, T), 0.0, 100.0), dim=1).values
    M = (torch.rand(B, T, F, generator=g) < 0.7).float()
    V = torch.randn(B, T, F, generator=g) * M
    A_log = _unif(g, (F, N), math.log(0.5), math.log(5.0))
    Bm = torch.randn(B, T, N, generator=g) / math.sqrt(N)
    Cm = torch.randn(B, T, N, generator=g) / math.sqrt(N)
    return {"V": V, "M": M, "tau": tau, "A_log": A_log, "B": Bm, "C": Cm}


def ssd_long(seed=1003, B=1, L=262144, H=8, P=64, N=16, dtype=torch.bfloat16):
    g = _gen(seed)
    x = torch.randn(B, L, H, P, generator=g).to(dtype)
    Bm = (torch.randn(B, L, H, N, generator=g) / math.sqrt(N)).to(dtype)
    Cm = (torch.randn(B, L, H, N, generator=g) / math.sqrt(N)).to(dtype)
    dt = torch.exp(torch.randn(B, L, H, generator=g) * 1.5 - 3.0)
    A_log = _unif(g, (H,), math.log(1.0), math.log(16.0))
    return {"x": x, "B": Bm, "C": Cm, "dt": dt, "A_log": A_log}


def ssd_stream(seed=1004, S=4096, H=32, P=64, N=128, pool=16):
    """Parameters plus a pool of ``pool`` pre-drawn per-step input sets."""
    g = _gen(seed)
    A_log = _unif(g, (H,), math.log(1.0), math.log(16.0))
    steps = []
    for _ in range(pool):
        steps.append({
            "x": torch.randn(S, H, P, generator=g),
            "dt": _exp(g, (S,), 0.1),
            "B": torch.randn(S, H, N, generator=g) / math.sqrt(N),
            "C": torch.randn(S, H, N, generator=g) / math.sqrt(N),
        })
    return {"A_log": A_log, "steps": steps, "S": S, "H": H, "P": P, "N": N}


def dtproj_mamba1(seed=1005, B=16, L=2048, D=256, N=16, R=16):
    """Mamba-1 scan with dt produced by the rank-R projection, at the
    interpolation workload's scan shape (B=16 L=2048 D=256 N=16 fp32):
    dt_raw ~ N(0,1) [B,L,R], W ~ N(0, 0.25/R) [R,D], bias [D] =
    softplus^-1(0.05) + U(-0.5, 0.5), DT_MIN=1e-3, DT_MAX=1; x, A_log, B, C as
    mamba1_small."""
    g = _gen(seed)
    x = torch.randn(B, L, D, generator=g)
    dt_raw = torch.randn(B, L, R, generator=g)
    W = torch.randn(R, D, generator=g) * (0.5 / math.sqrt(R))
    bias = math.log(math.expm1(0.05)) + _unif(g, (D,), -0.5, 0.5)
    A_log = _unif(g, (D, N), math.log(0.5), math.log(5.0))
    Bm = torch.randn(B, L, N, generator=g) / math.sqrt(N)
    Cm = torch.randn(B, L, N, generator=g) / math.sqrt(N)
    return {"x": x, "dt_raw": dt_raw, "W": W, "bias": bias, "A_log": A_log, "B": Bm, "C": Cm,
            "DT_MIN": 1e-3, "DT_MAX": 1.0}


# ------------------------------------------------------------------ bytes
def multihead_bytes(B, L, H, P, io_bytes=2, with_d=False):
    """Algorithmic HBM bytes of one fused multihead scan: x, B, C and y once
    in the I/O dtype, dt fp32 once, A_log (and D) fp32 once."""
    n = B * L * H * P
    return 4 * n * io_bytes + B * L * H * 4 + H * P * 4 * (2 if with_d else 1)


def multihead_elements(B, L, H, P):
    return B * L * H * P
