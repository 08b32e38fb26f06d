"""CPU checks of host-side validation and of the look-back error check.

No GPU compute: every bad argument must raise before any library call, and
``tssm.check`` must turn a set sticky flag into ``TssmError`` (the flag is
faked through the library call it reads it with).
"""
import contextlib

import pytest
import torch

import tssm
from tssm import _lib, workspace


def _stream_args(S=3, H=2, P=8, N=16):
    return dict(x=torch.zeros(S, H, P), dt=torch.zeros(S), A_log=torch.zeros(H),
                B=torch.zeros(S, H, N), C=torch.zeros(S, H, N), D=torch.zeros(H, P),
                state=torch.zeros(S, H, P, N))


def _call_stream(a, **kw):
    return tssm.ssd_stream_step(a["x"], a["dt"], a["A_log"], a["B"], a["C"], a["D"], a["state"],
                                **kw)


@pytest.mark.parametrize("field,bad,match", [
    ("A_log", torch.zeros(5), "A_log must be"),
    ("D", torch.zeros(3, 3), "D must be"),
    ("B", torch.zeros(3, 2, 8), "expected B/C"),
    ("state", torch.zeros(3, 2, 8, 8), "expected B/C"),
    ("dt", torch.zeros(4), "dt must be"),
    ("x", torch.zeros(3, 2, 8, dtype=torch.float64), "float32"),
    ("state", torch.zeros(3, 2, 8, 16, dtype=torch.bfloat16), "float32"),
])
def test_ssd_stream_step_rejects_bad_arguments(field, bad, match):
    a = _stream_args()
    a[field] = bad
    with pytest.raises((ValueError, TypeError), match=match):
        _call_stream(a)


def test_ssd_stream_step_rejects_bad_out():
    a = _stream_args()
    with pytest.raises(ValueError, match="out must be"):
        _call_stream(a, out=torch.zeros(3, 2, 4))
    with pytest.raises(TypeError, match="float32"):
        _call_stream(a, out=torch.zeros(3, 2, 8, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="innermost"):
        _call_stream(a, out=torch.zeros(3, 8, 2).transpose(1, 2))


def test_ssd_stream_step_needs_device_tensors():
    # well-formed host tensors reach the device check, which refuses them
    with pytest.raises(ValueError, match="HIP device"):
        _call_stream(_stream_args())


def test_check_raises_on_a_set_flag(monkeypatch):
    """check() reads every lookback workspace's flag, raises TssmError naming
    the set ones, clears them, and ignores SSD workspaces."""
    flags = {}

    def fake_call(name, buf_ptr, clear, out_ref):
        assert name == "tssm_workspace_error"
        out_ref._obj.value = flags.get(buf_ptr, 0)
        if clear:
            flags[buf_ptr] = 0

    lb = torch.zeros(256, dtype=torch.uint8)
    sd = torch.zeros(256, dtype=torch.uint8)
    monkeypatch.setattr(_lib, "call", fake_call)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda, "device", lambda d: contextlib.nullcontext())
    monkeypatch.setattr(workspace, "_cache", {(0, 7, workspace.LOOKBACK): lb,
                                              (0, 7, workspace.SSD): sd})
    workspace.check()                      # nothing set
    flags[sd.data_ptr()] = 1               # an SSD workspace holds raw data: not read
    workspace.check()
    flags[lb.data_ptr()] = 1
    with pytest.raises(_lib.TssmError, match="look-back wait expired"):
        workspace.check()
    workspace.check()                      # cleared by the failing check
    flags[lb.data_ptr()] = 1
    workspace.check(device=1)              # other device: not read
    with pytest.raises(_lib.TssmError):
        workspace.check(device=0, clear=False)
    with pytest.raises(_lib.TssmError):    # still set: clear=False kept it
        tssm.check()
    flags[None] = 1                        # the no-allocation scratch (workspace NULL)
    with pytest.raises(_lib.TssmError, match="no-allocation scratch"):
        workspace.check()
    workspace.check()


def test_workspace_kinds_are_distinct():
    with pytest.raises(ValueError, match="kind"):
        workspace.get(torch.device("cpu"), 0, 16, kind="other")
