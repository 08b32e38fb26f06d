"""Session save/restore format (CPU): round trips, the wire form, and every
corruption the reader must reject."""
import io
import struct
import zlib

import pytest
import torch

from tssm import session as S


def _tensors():
    g = torch.Generator().manual_seed(5)
    return {
        "h": torch.randn(3, 70, generator=g),
        "ring_V": torch.randn(3, 11, 70, generator=g),
        "hb": torch.randn(4, 9, generator=g).to(torch.bfloat16),
        "hf": torch.randn(5, generator=g).to(torch.float16),
        "head": torch.tensor([0, 3, 10], dtype=torch.int32),
        "mask": (torch.rand(2, 3, generator=g) > 0.5).to(torch.uint8),
        "scalar": torch.tensor(2.5),
        "empty": torch.zeros(0, 4),
        "strided": torch.randn(6, 8, generator=g)[:, ::2],
    }


def test_round_trip_file(tmp_path):
    ts = _tensors()
    p = tmp_path / "s.tssm"
    S.save(p, ts, {"kind": "test", "step": 7})
    out, meta = S.load(p)
    assert meta == {"kind": "test", "step": 7}
    assert set(out) == set(ts)
    for k, t in ts.items():
        assert out[k].dtype == t.dtype and out[k].shape == t.shape
        assert torch.equal(out[k], t), k
    assert not (tmp_path / "s.tssm.tmp").exists()


def test_wire_form_matches_file(tmp_path):
    ts = _tensors()
    data = S.dumps(ts, {"a": 1})
    p = tmp_path / "s.tssm"
    S.save(p, ts, {"a": 1})
    assert p.read_bytes() == data
    out, _ = S.loads(data)
    assert all(torch.equal(out[k], ts[k]) for k in ts)


def test_layout_fields():
    data = S.dumps({"x": torch.arange(6, dtype=torch.int32).reshape(2, 3)}, {})
    magic, ver, n, size, mlen, tcrc = struct.unpack_from("<8sIIQII", data, 0)
    assert (magic, ver, n, size) == (b"TSSMSES1", 1, 1, len(data))
    assert tcrc == zlib.crc32(data[32:32 + 112 + mlen])
    name, code, ndim, *rest = struct.unpack_from("<32sII6qQQII", data, 32)
    shape, (off, nbytes, crc, _) = rest[:6], rest[6:]
    assert name.rstrip(b"\0") == b"x" and code == 3 and ndim == 2 and shape[:2] == [2, 3]
    assert off % 64 == 0 and nbytes == 24
    assert data[off:off + 24] == bytes(torch.arange(6, dtype=torch.int32).numpy().tobytes())
    assert crc == zlib.crc32(data[off:off + 24])


def test_stream_object_with_offset():
    buf = io.BytesIO(b"prefix--")
    buf.seek(0, io.SEEK_END)
    S.save(buf, {"h": torch.ones(3)}, {"k": 1})
    buf.seek(8)
    out, meta = S.load(buf)
    assert torch.equal(out["h"], torch.ones(3)) and meta == {"k": 1}


@pytest.mark.parametrize("where", ["magic", "version", "table", "data", "truncate", "size"])
def test_corruption_rejected(where):
    data = bytearray(S.dumps(_tensors(), {"kind": "x"}))
    if where == "magic":
        data[0] ^= 1
    elif where == "version":
        struct.pack_into("<I", data, 8, 2)
    elif where == "table":
        data[32 + 40] ^= 0xFF
    elif where == "data":
        off = struct.unpack_from("<32sII6qQQII", data, 32)[9]   # first block's offset
        data[off] ^= 0x01
    elif where == "truncate":
        data = data[:-100]
    elif where == "size":
        struct.pack_into("<Q", data, 16, len(data) + 64)
    with pytest.raises(S.SessionFormatError):
        S.loads(bytes(data))


def test_bad_names_and_dtypes():
    with pytest.raises(ValueError):
        S.dumps({"x" * 33: torch.zeros(1)})
    with pytest.raises(TypeError):
        S.dumps({"x": torch.zeros(1, dtype=torch.float64)})
    with pytest.raises(ValueError):
        S.dumps({"x": torch.zeros([1] * 7)})


def test_ring_session_round_trip():
    s = S.RingSession(3, 70, 10, block_h=32)
    g = torch.Generator().manual_seed(1)
    for k in S.RingSession.FIELDS:
        t = getattr(s, k)
        if t.dtype == torch.int32:
            t.copy_(torch.randint(0, 11, t.shape, generator=g, dtype=torch.int32))
        else:
            t.copy_(torch.randn(t.shape, generator=g))
    r = S.RingSession.load(s.dumps())
    assert (r.B, r.H, r.K, r.block_h) == (3, 70, 10, 32)
    for k in S.RingSession.FIELDS:
        assert torch.equal(getattr(r, k), getattr(s, k)), k


def test_ring_session_rejects_inconsistent_state():
    s = S.RingSession(2, 8, 3)
    s.ring_head[0] = 4   # outside [0, K]
    with pytest.raises(S.SessionFormatError):
        S.RingSession.load(s.dumps())
    bad = S.dumps({"h": torch.zeros(2, 8)}, {"kind": "ring", "B": 2, "H": 8, "K": 3, "BLOCK_H": 8})
    with pytest.raises(S.SessionFormatError):
        S.RingSession.load(bad)
    with pytest.raises(S.SessionFormatError):
        S.RingSession.load(S.dumps({}, {"kind": "other"}))
