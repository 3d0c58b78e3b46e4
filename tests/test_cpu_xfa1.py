"""XFA1 flash-attention captures (xqattn.xfa1): the file layout the reference
writes for its first multi-query FLASH_ATTN_EXT node (src/bridge/session.cpp:
493-533), read back and replayed through the oracle.

Pins: the byte offsets of the first record read by hand from the writer's
sequence of fwrite calls (8-byte header, then 3 int32 + 4 int64 + 4 uint64 +
uint64 + char[64] = 148 bytes before each tensor's bytes); ggml_nbytes closed
forms for contiguous, permuted, block-quantized and cache-view tensors; a
capture of every multi-query golden fixture (permuted Q, K/V as views into a
larger cache whose gap rows hold junk) replays through the oracle to the
fixture's expected output bit for bit; malformed files are rejected.
"""
import struct

import numpy as np
import pytest

import golden_io as gio
import oracle
from xqattn import workloads as wl
from xqattn import xfa1

# multi-query fixtures without sinks (the capture holds q, k, v, mask, output only)
CASES = gio.fixture_paths("fa_verify")


def test_record_layout_by_offsets(tmp_path):
    meta, a, (q, k, v, m, out), cap = gio.fa_capture(CASES[0], tmp_path)
    data = cap.read_bytes()
    assert struct.unpack_from("<2I", data, 0) == (0x31414658, 5)
    assert data[0:4] == b"XFA1"
    off = 8
    spans = []
    for i, t in enumerate((q, k, v, m, out)):
        assert struct.unpack_from("<3i", data, off) == (i, [34, 33, 33, 0, 74][i], t.type)
        assert struct.unpack_from("<4q", data, off + 12) == tuple(t.ne)
        assert struct.unpack_from("<4Q", data, off + 44) == tuple(t.nb)
        (nbytes,) = struct.unpack_from("<Q", data, off + 76)
        assert data[off + 84:off + 148].rstrip(b"\0") == [b"q-0", b"cache_k_l3 (view)", b"cache_v_l3 (view)",
                                                        b"attn_inp_kq_mask", b"__fattn__-3"][i]
        assert data[off + 148:off + 148 + nbytes] == t.buf.reshape(-1).view(np.uint8)[:nbytes].tobytes()
        spans.append(nbytes)
        off += 148 + nbytes
    assert off == len(data) == 8 + 5 * 148 + sum(spans)
    B, NQ, H, D = a["q"].shape
    assert spans[0] == spans[4] == B * NQ * H * D * 4


def test_span_bytes_closed_forms():
    D, NQ, H, B = 128, 5, 8, 2
    # permuted Q [D, n_q, H, B] over token-major rows: exactly the rows
    assert xfa1.span_bytes(wl.F32, (D, NQ, H, B), (4, H * D * 4, D * 4, NQ * H * D * 4)) == B * NQ * H * D * 4
    # contiguous f16 mask
    assert xfa1.span_bytes(wl.F16, (70, 8, 1, 1), (2, 140, 1120, 1120)) == 70 * 8 * 2
    # q8_0 cache rows [D=256, L, Hkv=4, 1]: L rows of 4 records of 272 bytes
    rec, L = 272, 1000
    assert xfa1.span_bytes(wl.Q8_0, (256, L, 4, 1), (34, 4 * rec, rec, 4096 * 4 * rec)) == L * 4 * rec
    # two sequences in a cache of capacity C: the gap up to the second sequence counts
    C = 1500
    assert xfa1.span_bytes(wl.Q4_0, (128, L, 2, 2), (18, 2 * 72, 72, C * 2 * 72)) == (C + L) * 2 * 72
    # an empty view spans nothing (ggml_nbytes returns 0 for any ne <= 0)
    assert xfa1.span_bytes(wl.F32, (128, 0, 8, 1), (4, 512, 64, 4096)) == 0


@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_capture_round_trip_replays_through_oracle(path, tmp_path):
    meta, a, tensors, cap = gio.fa_capture(path, tmp_path)
    got = xfa1.read(cap)
    for role, t in zip(xfa1.ROLES, tensors):
        c = got[role]
        assert (c.type, c.ne, c.nb) == (t.type, tuple(t.ne), tuple(t.nb))
        assert np.array_equal(c.raw, t.buf.reshape(-1).view(np.uint8)[:c.raw.size])
    q, k, v, m, o = (got[r].host() for r in xfa1.ROLES)
    want = xfa1.gather_f32(o)
    assert np.array_equal(want, a["out"])
    dst = wl.HostTensor(o.type, o.ne, o.nb, np.zeros(o.buf.size, np.uint8))
    oracle.flash_attn_ext(q, k, v, m, None, dst, meta["scale"], meta["max_bias"], meta["softcap"],
                          oracle.QK_CONSISTENT, True)
    assert np.array_equal(xfa1.gather_f32(dst), want), "oracle on the capture differs from the fixture output"


def _bad(tmp_path, edit):
    _, _, _, cap = gio.fa_capture(CASES[0], tmp_path)
    data = bytearray(cap.read_bytes())
    data = edit(data)
    bad = tmp_path / "bad.xfa1"
    bad.write_bytes(bytes(data))
    return bad


@pytest.mark.parametrize("what,edit,msg", [
    ("magic", lambda d: d[:0] + b"XFA2" + d[4:], "bad magic"),
    ("count", lambda d: d[:4] + struct.pack("<I", 4) + d[8:], "4 tensors"),
    ("truncated", lambda d: d[:-1], "truncated"),
    ("trailing", lambda d: d + b"\0", "trailing"),
    ("index", lambda d: d[:8] + struct.pack("<i", 1) + d[12:], "record 1"),
    ("bytes", lambda d: d[:84] + struct.pack("<Q", struct.unpack_from("<Q", d, 84)[0] - 4) + d[92:], "spans"),
    ("type", lambda d: d[:16] + struct.pack("<i", 39) + d[20:], "unsupported type"),
])
def test_malformed_captures_are_rejected(tmp_path, what, edit, msg):
    with pytest.raises(ValueError, match=msg):
        xfa1.read(_bad(tmp_path, edit))
