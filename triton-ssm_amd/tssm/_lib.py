"""ctypes binding of libtssm.so.

Function signatures are read from the C header ``include/tssm.h`` (the one
declaration of the ABI), so Python and C cannot drift apart.  Status codes map
to exceptions: negative TSSM_ERR_* -> ``ValueError`` (argument errors detected
before any launch), positive hipError_t -> ``TssmError``.

There is deliberately no CPU fallback: if the library is missing or cannot be
loaded every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import re
import threading
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("TSSM_LIB", _PKG / "libtssm.so"))
HEADER_PATH = Path(os.environ.get("TSSM_HEADER", _PKG.parents[1] / "include" / "tssm.h"))

F32, BF16, F16 = 0, 1, 2
DISC_EULER, DISC_ZOH = 0, 1

ERR_NAMES = {
    -1: "TSSM_ERR_NULL", -2: "TSSM_ERR_SHAPE", -3: "TSSM_ERR_STRIDE", -4: "TSSM_ERR_DTYPE",
    -5: "TSSM_ERR_WORKSPACE", -6: "TSSM_ERR_UNSUPPORTED", -7: "TSSM_ERR_ALIGN",
    -8: "TSSM_ERR_SCRATCH",
}


class TssmError(RuntimeError):
    """A HIP runtime error reported by a tssm entry point."""


_CTYPE = {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float}


def parse_header(text: str) -> dict[str, tuple[str, list[str]]]:
    """Return {name: (restype, [argtype, ...])} for every tssm_* declaration."""
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    out = {}
    for m in re.finditer(r"\b(int64_t|int|const\s+char\s*\*)\s+(tssm_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        types = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                if "*" in p:
                    types.append("ptr")
                else:
                    types.append(p.rsplit(" ", 1)[0].replace("const ", ""))
        out[name] = ("str" if "char" in ret else ret, types)
    return out


def declared_functions() -> dict[str, tuple[str, list[str]]]:
    return parse_header(HEADER_PATH.read_text())


_lock = threading.Lock()
_lib = None


def _bind(cdll) -> None:
    for name, (ret, args) in declared_functions().items():
        fn = getattr(cdll, name)
        fn.restype = ctypes.c_char_p if ret == "str" else _CTYPE[ret]
        fn.argtypes = [ctypes.c_void_p if a == "ptr" else _CTYPE[a] for a in args]


def lib():
    """Load (once) and return the bound library; raises if it is missing."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise ImportError(
                        f"tssm HIP library not found at {LIB_PATH}; build it with "
                        "`python triton-ssm_amd/build.py` (there is no CPU fallback)")
                cdll = ctypes.CDLL(str(LIB_PATH))
                _bind(cdll)
                _lib = cdll
    return _lib


def strerror(code: int) -> str:
    return lib().tssm_strerror(code).decode()


def check(code: int, what: str) -> None:
    if code == 0:
        return
    if code < 0:
        raise ValueError(f"{what}: {ERR_NAMES.get(code, code)} ({strerror(code)})")
    raise TssmError(f"{what}: HIP error {code} ({strerror(code)})")


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise on a nonzero status."""
    check(getattr(lib(), name)(*args), name)
