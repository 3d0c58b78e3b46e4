"""CPU pins of the oracle's storage codecs and quantizers (no GPU).

Each check is against something outside the oracle's own formula:
  * f32 -> f16: numpy's IEEE round-to-nearest-even cast (plus ggml's NaN
    canonicalisation 0x7e00 | sign, src/bridge ggml_half_bits as restated in
    shaders/rkva/rkva_store_f16.hlsl:27-61), and the reference's own
    f32_to_f16_bits compiled from uwp/rkva/rkva-bulk-fp8.h (oracle/_ref);
  * f32 -> bf16: torch's round-to-nearest-even cast;
  * E5M2: the reference's exhaustive test (tests/rkva_bulk_fp8_cpu.cpp:11-49):
    every finite f16 maps to the nearest code 0..0x7b, ties to the even code,
    plus its two-step rounding known answer 0x3c80 -> 0x3c;
  * q8_0 / q4_0: an independent numpy decoder of the block layouts
    (tests/rkva_range_fmt_opt_model.py:41-47 describes the same records), the
    round-trip bound |x - deq(q(x))| <= d/2, and hand-computed blocks.
"""
import numpy as np
import pytest
import torch

import oracle
from xqattn import workloads as wl


def _numpy_f16_bits(x):
    with np.errstate(over="ignore"):
        h = np.asarray(x, np.float32).astype(np.float16).view(np.uint16).copy()
    nan = np.isnan(np.asarray(x, np.float32))
    sign = (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16) & np.uint16(0x8000)
    h[nan] = (sign[nan] | np.uint16(0x7e00))
    return h


def _sample_f32(n=1 << 18, seed=3):
    u = wl.splitmix64(seed, n)
    bits = (u & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    x = bits.view(np.float32)
    # plus decimals across the f16 range, halfway points and edges
    extra = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 6.1035156e-05, 5.9604645e-08,
                      2.9802322e-08, 2.9802326e-08, np.inf, -np.inf, np.nan, 1.125, np.nextafter(np.float32(1.125), 2)],
                     np.float32)
    dec = (wl.uniform(seed + 1, 1 << 16) * 140000 - 70000).astype(np.float32)
    return np.concatenate([x, extra, dec])


def test_f32_to_f16_matches_numpy_rne():
    x = _sample_f32()
    got = oracle.f32_to_f16(x)
    want = _numpy_f16_bits(x)
    assert np.array_equal(got, want)


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))


def test_f32_to_bf16_matches_torch_rne():
    x = _sample_f32()
    x = x[np.isfinite(x)]
    got = oracle.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def _nearest_e5m2(h):
    """The reference test's brute-force rule, vectorised over finite f16 bits h:
    the nearest code among 0..0x7b by magnitude (finite saturation), ties to the
    even code, sign copied."""
    mag = (h & np.uint16(0x7FFF)).view(np.float16).astype(np.float64)
    codes = np.arange(0x7C, dtype=np.uint16)
    vals = (codes << 8).view(np.float16).astype(np.float64)
    dist = np.abs(mag[:, None] - vals[None, :])
    tie = dist == dist.min(axis=1, keepdims=True)
    even = tie & ((codes & 1) == 0)[None, :]
    best = np.where(even.any(axis=1), even.argmax(axis=1), tie.argmax(axis=1)).astype(np.uint8)
    return best | np.where((h & 0x8000) != 0, 0x80, 0).astype(np.uint8)


def test_e5m2_exhaustive_nearest_even_saturating():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (h & 0x7C00) != 0x7C00
    assert int(finite.sum()) == 63488 and int((~finite).sum()) == 2048
    x = h[finite].view(np.float16).astype(np.float32)  # exact, so f32 -> f16 is the identity
    got = oracle.f32_to_e5m2(x)
    want = _nearest_e5m2(h[finite])
    assert np.array_equal(got, want)
    # the decode is the byte shifted into an f16's high byte
    dec = (got.astype(np.uint16) << 8).view(np.float16).astype(np.float32)
    assert np.all(np.abs(dec) <= 57344.0)


def test_e5m2_two_step_rounding_known_answer():
    above = np.nextafter(np.float32(1.125), np.float32(2.0))
    assert oracle.f32_to_f16(np.array([above], np.float32))[0] == 0x3C80
    assert oracle.f32_to_e5m2(np.array([above], np.float32))[0] == 0x3C


def test_codecs_match_reference_shim():
    ref = oracle.load_ref()
    if ref is None:
        pytest.skip("reference shim not built (no reference checkout)")
    x = _sample_f32(1 << 14, seed=9)
    x = x[~np.isnan(x)]
    got = oracle.f32_to_f16(x)
    want = np.array([ref.xr_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (h & 0x7C00) != 0x7C00
    e_ref = np.array([ref.xr_f16_to_e5m2(int(v)) for v in h[finite]], np.uint8)
    e_got = oracle.f32_to_e5m2(h[finite].view(np.float16).astype(np.float32))
    assert np.array_equal(e_got, e_ref)
    for code in range(256):
        assert ref.xr_e5m2_to_f16(code) == (code << 8)


# ---------------------------------------------------------------- block formats

def _decode_q8_0(raw, k):
    blk = np.dtype([("d", "<f2"), ("qs", "i1", (32,))])
    b = np.frombuffer(raw.tobytes(), blk)
    return (b["d"].astype(np.float32)[:, None] * b["qs"].astype(np.float32)).reshape(-1)[:k]


def _decode_q4_0(raw, k):
    blk = np.dtype([("d", "<f2"), ("qs", "u1", (16,))])
    b = np.frombuffer(raw.tobytes(), blk)
    lo = (b["qs"] & 0x0F).astype(np.int32) - 8
    hi = (b["qs"] >> 4).astype(np.int32) - 8
    vals = np.concatenate([lo, hi], axis=1).astype(np.float32)  # element j<16: low nibble of qs[j]
    return (b["d"].astype(np.float32)[:, None] * vals).reshape(-1)[:k]


@pytest.mark.parametrize("variant", [0, 1])
def test_q8_0_layout_roundtrip_and_bound(variant):
    x = (wl.normal(5, (64, 256)) * np.float32(3.0)).astype(np.float32)
    raw = oracle.quantize(wl.Q8_0, x, q8_variant=variant)
    assert raw.size == 64 * 8 * 34
    dec = oracle.dequant(wl.Q8_0, raw, 256).reshape(-1)
    assert np.array_equal(dec, _decode_q8_0(raw, x.size))
    d = np.frombuffer(raw.tobytes(), np.dtype([("d", "<f2"), ("qs", "i1", (32,))]))["d"].astype(np.float32)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert np.array_equal(d, (amax / 127).astype(np.float16).astype(np.float32))
    err = np.abs(dec - x.reshape(-1)).reshape(-1, 32).max(axis=1)
    # rounding to the f16 scale moves the grid by at most 127 * |d - amax/127|
    assert np.all(err <= d / 2 + 127 * np.abs(d - amax / 127) + 1e-6)


def test_q8_0_variants_known_block():
    # amax 127 -> d = 1, id = 1: exact halves expose the rounding rule
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 3.5, 0.5
    q_x86 = np.frombuffer(oracle.quantize(wl.Q8_0, x[None], 0).tobytes()[2:], np.int8)
    q_ref = np.frombuffer(oracle.quantize(wl.Q8_0, x[None], 1).tobytes()[2:], np.int8)
    # ggml-cpu x86 path: round half to even; ggml reference path: roundf (half away from zero)
    assert q_x86[:5].tolist() == [127, 2, -2, 4, 0]
    assert q_ref[:5].tolist() == [127, 3, -3, 4, 1]


def test_q4_0_layout_and_known_block():
    x = (wl.normal(6, (32, 128)) * np.float32(2.0)).astype(np.float32)
    raw = oracle.quantize(wl.Q4_0, x)
    dec = oracle.dequant(wl.Q4_0, raw, 128).reshape(-1)
    assert np.array_equal(dec, _decode_q4_0(raw, x.size))
    # ggml quantize_row_q4_0_ref: max = signed value of largest |x| (first on ties),
    # d = max / -8, q = min(15, (int8)(x * id + 8.5))
    blk = np.arange(32, dtype=np.float32) - 16.0  # max |x| = 16 at x = -16 -> d = 2
    r = oracle.quantize(wl.Q4_0, blk[None])
    d = np.frombuffer(r.tobytes()[:2], np.float16)[0]
    assert float(d) == 2.0
    q = _decode_q4_0(r, 32) / 2.0 + 8
    want = np.minimum(15, np.floor(blk * 0.5 + 8.5)).astype(np.float32)
    assert np.array_equal(q, want)


@pytest.mark.parametrize("typ", [wl.F16, wl.BF16, wl.E5M2, wl.Q8_0, wl.Q4_0])
def test_kv_store_oracle_equals_row_quantizer(typ):
    n_tok, hkv, d, cap = 7, 4, 128, 16
    src = wl.normal(11, (n_tok, hkv, d))
    pos = np.array([3, 0, 15, 7, 8, 1, 12], np.int32)
    rec = wl.record_bytes(typ, d)
    dst = np.full(cap * hkv * rec, 0xAB, np.uint8)
    oracle.kv_store(src, pos, hkv, d, typ, dst, cap)
    rows = dst.reshape(cap, hkv, rec)
    want = oracle.quantize(typ, src.reshape(n_tok * hkv, d)).reshape(n_tok, hkv, rec)
    for i, p in enumerate(pos):
        assert np.array_equal(rows[p], want[i])
    untouched = np.setdiff1d(np.arange(cap), pos)
    assert np.all(rows[untouched] == 0xAB)
