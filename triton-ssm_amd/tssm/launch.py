"""Launcher objects that accept the reference's Triton launch convention.

``kernel[grid](*args, **kwargs)`` binds the arguments to the reference
kernel's parameter list (same names, same order), and hands the bound
arguments plus the grid to a host function that validates them and calls the
C ABI.  Triton compile options (``num_warps`` ...) are accepted and ignored:
launch geometry is the library's own choice.  A grid may be a tuple or a
callable taking the dict of bound arguments (Triton's ``grid(meta)`` form).
"""
from __future__ import annotations

import torch

from . import _lib

TRITON_OPTIONS = frozenset({
    "num_warps", "num_stages", "num_ctas", "waves_per_eu", "matrix_instr_nonkdim",
    "kpack", "enable_fp_fusion", "maxnreg", "debug", "grid", "warmup",
})


class HipKernel:
    """Drop-in for a ``@triton.jit`` kernel object."""

    def __init__(self, name: str, params: list[str], launch, reference: str = ""):
        self.__name__ = name
        self.fn_name = name
        self.arg_names = list(params)
        self._launch = launch
        self.reference = reference
        self.__doc__ = f"HIP drop-in for `{name}` ({reference}); launch as {name}[grid](...)."

    def __repr__(self):
        return f"<HipKernel {self.__name__} ({self.reference})>"

    def bind(self, args, kwargs) -> dict:
        if len(args) > len(self.arg_names):
            raise TypeError(f"{self.__name__}: expected at most {len(self.arg_names)} "
                            f"positional arguments, got {len(args)}")
        bound = dict(zip(self.arg_names, args))
        for k, v in kwargs.items():
            if k in TRITON_OPTIONS:
                continue
            if k not in self.arg_names:
                raise TypeError(f"{self.__name__}: unexpected argument {k!r}")
            if k in bound:
                raise TypeError(f"{self.__name__}: argument {k!r} given twice")
            bound[k] = v
        missing = [p for p in self.arg_names if p not in bound]
        if missing:
            raise TypeError(f"{self.__name__}: missing arguments {missing}")
        return bound

    def __getitem__(self, grid):
        def run(*args, **kwargs):
            bound = self.bind(args, kwargs)
            g = grid(bound) if callable(grid) else grid
            return self._launch(normalize_grid(g), bound)
        return run

    def __call__(self, *args, **kwargs):
        raise TypeError(f"{self.__name__} is a kernel: launch it as {self.__name__}[grid](...)")


def normalize_grid(g) -> tuple[int, int, int]:
    if isinstance(g, int):
        g = (g,)
    g = tuple(int(x) for x in g)
    if not 1 <= len(g) <= 3 or any(x < 0 for x in g):
        raise ValueError(f"invalid grid {g}")
    return g + (1,) * (3 - len(g))


# ------------------------------------------------------------------ tensors
_DCODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def dcode(t: torch.Tensor, what: str = "tensor") -> int:
    try:
        return _DCODE[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype} (float32/bfloat16/float16)") from None


def need_gpu(t, what: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what}: expected a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{what}: tensor must be on a HIP device, got {t.device}")
    return t


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def as_f32(t: torch.Tensor, what: str) -> torch.Tensor:
    """Small side inputs the kernels read as fp32: convert other float dtypes
    without changing the element layout the caller's strides describe."""
    need_gpu(t, what)
    if t.dtype == torch.float32:
        return t
    if not t.is_floating_point():
        raise TypeError(f"{what}: expected a float tensor, got {t.dtype}")
    if not t.is_non_overlapping_and_dense():
        raise TypeError(f"{what}: a non-fp32 tensor must be dense to be read as fp32")
    return t.to(torch.float32)  # preserve_format keeps strides of dense tensors


def extent(t: torch.Tensor, max_offset: int, what: str) -> None:
    """Raise unless element offsets 0..max_offset from ``t.data_ptr()`` lie
    inside t's storage: the kernels address memory through the caller's
    sizes and strides, so this is checked before every launch."""
    if max_offset < 0:
        return
    avail = t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()
    if max_offset >= avail:
        raise ValueError(f"{what}: the launch would read/write element offset {max_offset} but "
                         f"the tensor's storage holds only {avail} elements from its start")


def span(sizes_strides) -> int:
    """Largest element offset sum((n-1)*s) of an (n, stride) list (-1 if empty)."""
    off = 0
    for n, s in sizes_strides:
        if n <= 0:
            return -1
        if s < 0:
            raise ValueError("negative strides are not supported")
        off += (n - 1) * s
    return off


def stream_handle(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ival(x, what: str) -> int:
    try:
        return int(x)
    except Exception:
        raise TypeError(f"{what}: expected an integer, got {x!r}") from None
