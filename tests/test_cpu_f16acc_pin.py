"""Pin of the oracle's F16-V path: ggml's one-chunk loop with an f16 value
accumulator (patches/0008-flash-attn-query-consistency.patch:25-38,
patches/README.md:63-64 "keeps the original online softmax and F16 value
accumulator").

An independent step-by-step restatement in Python: per KV row, a new maximum
rescales the f16 accumulator (ggml_vec_scale_f16: y = f16(f32(y) * ms)),
then ggml_vec_mad_f16 adds the row (y = f16(fma(f32(v), vs, f32(y))): the
x86 AVX2+FMA+F16C build converts 8 halves to f32, fuses the multiply-add in f32
and rounds back to f16 with round-to-nearest-even), and S = fma(S, ms, vs)
(GCC contracts S*ms + vs on an FMA target). The fused multiply-adds are formed
exactly with fractions and rounded once to f32. exp is libm's expf, the one
ggml's loop calls. Scores are made exact in f32 in any summation order (Q and
K are small multiples of 1/16, the scale a power of two), so the comparison
isolates the accumulator schedule.

The restatement must equal xo_flash_attn_ext(v_acc_f16=1) bit for bit; the
same restatement with a separate multiply and add (two roundings) and the
oracle's f32-accumulator mode must both differ, so the test tells the
schedules apart.
"""
import ctypes
import ctypes.util
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from fa_cases import dst_array
from xqattn import workloads as wl

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]


def expf(x: np.float32) -> np.float32:
    return np.float32(_libm.expf(float(x)))


def f32_rne(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest binary32 (ties to even)."""
    if x == 0:
        return np.float32(0.0)
    neg = x < 0
    x = -x if neg else x
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    elif Fraction(2) ** (e + 1) <= x:
        e += 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 23)
    q = x / ulp
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = n * ulp
    if v >= Fraction(2) ** 128:
        r = np.float32(np.inf)
    else:
        r = np.float32(float(v))  # exact: v is a binary32 value
    return -r if neg else r


def fma32(a, b, c) -> np.float32:
    return f32_rne(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def muladd32(a, b, c) -> np.float32:
    return np.float32(np.float32(np.float32(a) * np.float32(b)) + np.float32(c))


def restate(q, k, v, mask, scale, fused=True):
    """q [NQ, H, D] f32, k/v [L, Hkv, D] f16, mask [NQ, L] f16 -> out [NQ, H, D] f32."""
    madd = fma32 if fused else muladd32
    NQ, H, D = q.shape
    L, Hkv, _ = k.shape
    G = H // Hkv
    out = np.zeros((NQ, H, D), np.float32)
    for iq in range(NQ):
        for h in range(H):
            kh = h // G
            M, S = np.float32(-np.inf), np.float32(0.0)
            acc = np.zeros(D, np.float16)
            for ic in range(L):
                mv = np.float32(mask[iq, ic])  # slope 1 (no ALiBi)
                if mv == -np.inf:
                    continue
                dot = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(q[iq, h], k[ic, kh].astype(np.float32)))
                s = np.float32(float(dot))  # exact by construction
                assert Fraction(float(s)) == dot
                s = np.float32(s * np.float32(scale))
                s = np.float32(s + mv)
                ms, vs = np.float32(1.0), np.float32(1.0)
                if s > M:
                    Mold, M = M, s
                    ms = expf(np.float32(Mold - M))
                    acc = (acc.astype(np.float32) * ms).astype(np.float16)
                else:
                    vs = expf(np.float32(s - M))
                vf = v[ic, kh].astype(np.float32)
                acc = np.array([madd(vf[d], vs, np.float32(acc[d])) for d in range(D)], np.float32).astype(np.float16)
                S = madd(S, ms, vs)
            inv = np.float32(0.0) if S == 0 else np.float32(np.float32(1.0) / S)
            out[iq, h] = acc.astype(np.float32) * inv
    return out


def _case(seed):
    rng = np.random.default_rng(seed)
    NQ, H, Hkv, D, L = 2, 2, 1, 128, 40
    q = (rng.integers(-32, 33, (NQ, H, D)) / 16.0).astype(np.float32)
    k = (rng.integers(-24, 25, (L, Hkv, D)) / 16.0).astype(np.float16)
    v = (rng.standard_normal((L, Hkv, D)) * 2.0).astype(np.float16)
    mask = np.zeros((NQ, L), np.float16)
    mask[:, rng.integers(0, L, 6)] = -np.inf
    mask[1, L - 3:] = -np.inf
    mask[0, 5] = np.float16(-3.5)  # a finite bias
    scale = 0.125
    return q, k, v, mask, scale


def _oracle(q, k, v, mask, scale, v_acc_f16):
    NQ, H, D = q.shape
    L, Hkv, _ = k.shape
    cfg = wl.FaConfig("pin", NQ, H, Hkv, D, L, 1, wl.F16)
    hq = wl.fa_q_tensor(q[None])
    kv = lambda a: wl.kv_tensor(a.view(np.uint8).reshape(1, L, Hkv, 2 * D), wl.F16, D)
    hm = wl.mask_tensor(mask.view(np.uint16)[None])
    dst = wl.fa_dst_tensor(1, NQ, H, D)
    oracle.flash_attn_ext(hq, kv(k), kv(v), hm, None, dst, scale, 0.0, 0.0, oracle.QK_CONSISTENT, v_acc_f16, 1)
    case = type("C", (), {"dst": dst, "shape": (1, NQ, H, D)})
    return dst_array(case)[0]


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_f16_accumulator_matches_step_by_step_restatement(seed):
    q, k, v, mask, scale = _case(seed)
    want = restate(q, k, v, mask, scale, fused=True)
    got = _oracle(q, k, v, mask, scale, v_acc_f16=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{int(np.sum(got != want))} elements differ from the fused f16-accumulator schedule"


def test_the_pin_tells_the_schedules_apart():
    """Over the pin's cases, the mul+add schedule and the f32 accumulator each
    give different bits somewhere, so the bitwise pin fixes the fused f16 one."""
    differ_muladd = differ_f32 = False
    for seed in (1, 2, 3):
        q, k, v, mask, scale = _case(seed)
        fused = restate(q, k, v, mask, scale, fused=True)
        differ_muladd |= not np.array_equal(fused, restate(q, k, v, mask, scale, fused=False))
        differ_f32 |= not np.array_equal(fused, _oracle(q, k, v, mask, scale, v_acc_f16=False))
    assert differ_muladd, "mul+add and fused schedules agree on every case: the pin cannot tell them apart"
    assert differ_f32, "the f32 accumulator agrees with the f16 one: the pin cannot tell them apart"


def test_f32_rne_against_numpy():
    """The exact rounding helper against numpy's float64 -> float32 cast where
    that cast is a single rounding (values exact in float64)."""
    rng = np.random.default_rng(5)
    for x in rng.standard_normal(2000) * 10.0 ** rng.integers(-30, 30, 2000):
        assert f32_rne(Fraction(float(x))) == np.float32(x)
    assert f32_rne(Fraction(1, 3)) == np.float32(1 / 3)
    tie = Fraction(1) + Fraction(1, 2 ** 24)  # halfway between 1 and 1 + 2^-23: ties to even
    assert f32_rne(tie) == np.float32(1.0)
    assert f32_rne(tie + Fraction(1, 2 ** 23)) == np.float32(1.0 + 2.0 ** -22)
    assert math.isinf(float(f32_rne(Fraction(2) ** 129)))
