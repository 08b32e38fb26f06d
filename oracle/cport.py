"""ctypes loader of the C restatement (``liboracle_c.so``) -- test/bench
infrastructure only.  All arrays are passed as contiguous float32 numpy."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle_c.so"
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_SIGS = {
    "oc_num_threads": ([], _I),
    "oc_multihead_scan": ([_I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L], None),
    "oc_ssd_scan": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L], None),
    "oc_selective_scan": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L], None),
    "oc_ssd_stream_step": ([_I, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L], None),
    "oc_time_aware_interp": ([_P, _P, _P, _P, _L, _L, _L, _L, _L], None),
}


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        cd = ctypes.CDLL(str(LIB))
        for n, (args, ret) in _SIGS.items():
            f = getattr(cd, n)
            f.argtypes, f.restype = args, ret
        _lib = cd
    return _lib


def _f32(x):
    if x is None:
        return None
    try:
        import torch
        if isinstance(x, torch.Tensor):
            x = x.detach().to("cpu", torch.float32).numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.ascontiguousarray(x, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data


def threads() -> int:
    return lib().oc_num_threads()


def multihead_scan(u, A_log, B, C, dt, D=None, disc="euler", prepared=False):
    """Returns (y [Bsz,L,nh*hd], h_last [Bsz,nh,hd]) in float32."""
    arrs = [u, A_log, B, C, dt, D] if prepared else [_f32(v) for v in (u, A_log, B, C, dt, D)]
    u, A_log, B, C, dt, D = arrs
    Bsz, L, nh, hd = B.shape
    y = np.empty_like(u)
    hl = np.empty((Bsz, nh, hd), np.float32)
    lib().oc_multihead_scan(int(disc == "zoh"), int(A_log.ndim == 1), _p(u), _p(A_log), _p(B),
                            _p(C), _p(dt), _p(D), _p(y), _p(hl), Bsz, L, nh, hd)
    return y, hl


def ssd_scan(x, dt, A_log, B, C, D=None, h0=None, disc="zoh"):
    x, dt, A_log, B, C, D, h0 = (_f32(v) for v in (x, dt, A_log, B, C, D, h0))
    Bsz, L, H, P = x.shape
    N = B.shape[-1]
    y = np.empty_like(x)
    hl = np.empty((Bsz, H, P, N), np.float32)
    lib().oc_ssd_scan(int(disc == "zoh"), _p(x), _p(dt), _p(A_log), _p(B), _p(C), _p(D), _p(h0),
                      _p(y), _p(hl), Bsz, L, H, P, N)
    return y, hl


def selective_scan(x, dt, A_log, B, C, D=None, disc="zoh"):
    x, dt, A_log, B, C, D = (_f32(v) for v in (x, dt, A_log, B, C, D))
    Bsz, L, Dc = x.shape
    N = A_log.shape[-1]
    y = np.empty_like(x)
    hl = np.empty((Bsz, Dc, N), np.float32)
    lib().oc_selective_scan(int(disc == "zoh"), _p(x), _p(dt), _p(A_log), _p(B), _p(C), _p(D),
                            _p(y), _p(hl), Bsz, L, Dc, N)
    return y, hl


def ssd_stream_step(x, dt, A_log, B, C, D, state, disc="zoh"):
    """state: contiguous float32 numpy array, updated in place."""
    x, dt, A_log, B, C, D = (_f32(v) for v in (x, dt, A_log, B, C, D))
    S, H, P = x.shape
    N = B.shape[-1]
    y = np.empty_like(x)
    lib().oc_ssd_stream_step(int(disc == "zoh"), _p(x), _p(dt), _p(A_log), _p(B), _p(C), _p(D),
                             _p(state), _p(y), S, H, P, N)
    return y


def time_aware_interp(V, M, tau, K=10, FTILE=128):
    V, M, tau = (_f32(v) for v in (V, M, tau))
    Bsz, T, F = V.shape
    out = np.empty_like(V)
    lib().oc_time_aware_interp(_p(V), _p(M), _p(tau), _p(out), Bsz, T, F, K, FTILE)
    return out
