"""CPU pins of the flash-attention oracle (the ggml one-chunk loop restated in
oracle/xq_oracle.c) and of the RKVA range pass / reduce restatement.

The pins are independent of the oracle's code: a float64 numpy closed form
softmax(Q K^T * scale + slope * mask) V (tests/rkva_range_q4_opt_model.py:124-137
states the same formula), with ggml's softcap / ALiBi / sinks terms
(patches/0008-... loop structure; ggml's ALiBi slope rule), the all-masked
case (output 0, LSE -inf), query-width invariance, and hand-built partial
states for the reduce's poisoning rules (shaders/rkva/rkva_range_reduce_opt.hlsl:39-56,126-132).
"""
import math

import numpy as np
import pytest

import oracle
from fa_cases import dst_array, make_fa_case, oracle_f64, oracle_fa
from xqattn import workloads as wl


def _dequant_kv(case):
    c = case.cfg
    rec = wl.record_bytes(c.kv_type, c.D)
    kraw = case.k.buf.reshape(c.B, c.L, c.Hkv, rec)
    vraw = case.v.buf.reshape(c.B, c.L, c.Hkv, rec)
    k = oracle.dequant(c.kv_type, kraw, c.D).astype(np.float64)
    v = oracle.dequant(c.kv_type, vraw, c.D).astype(np.float64)
    return k, v


def _q_used(case):
    """Q as the consistent policy uses it: q8_0-quantised for quantised K, f16-rounded
    hi + lo (= f32 exactly) otherwise."""
    c = case.cfg
    q = np.frombuffer(case.q.buf.tobytes(), np.float32).reshape(c.B, c.n_q, c.H, c.D)
    if c.kv_type in (wl.Q8_0, wl.Q4_0):
        raw = oracle.quantize(wl.Q8_0, q)
        return oracle.dequant(wl.Q8_0, raw, c.D).astype(np.float64)
    return q.astype(np.float64)


def _alibi(h, H, max_bias):
    if max_bias <= 0:
        return 1.0
    n = 1 << int(math.floor(math.log2(H)))
    m0 = 2.0 ** (-max_bias / n)
    m1 = 2.0 ** (-(max_bias / 2.0) / n)
    return m0 ** (h + 1) if h < n else m1 ** (2 * (h - n) + 1)


def closed_form(case):
    c = case.cfg
    k, v = _dequant_kv(case)
    q = _q_used(case)
    mask = None
    if case.mask is not None:
        mask = np.frombuffer(case.mask.buf.tobytes(), np.float16).reshape(case.mask.ne[3], case.mask.ne[1],
                                                                          case.mask.ne[0]).astype(np.float64)
    sinks = np.frombuffer(case.sinks.buf.tobytes(), np.float32) if case.sinks is not None else None
    G = c.H // c.Hkv
    out = np.zeros((c.B, c.n_q, c.H, c.D))
    lse = np.full((c.B, c.n_q, c.H), -np.inf)
    for b in range(c.B):
        for i in range(c.n_q):
            for h in range(c.H):
                s = k[b, :, h // G] @ q[b, i, h] * case.scale
                if case.softcap:
                    s = case.softcap * np.tanh(s / case.softcap)
                if mask is not None:
                    s = s + _alibi(h, c.H, case.max_bias) * mask[b % mask.shape[0], i, :c.L]
                logits = s
                if sinks is not None:
                    logits = np.concatenate([s, [float(sinks[h])]])
                M = np.max(logits)
                if not np.isfinite(M):
                    continue
                w = np.exp(logits - M)
                S = w.sum()
                out[b, i, h] = (w[:c.L] @ v[b, :, h // G]) / S
                lse[b, i, h] = M + math.log(S)
    return out, lse


SMALL = [
    ("f16_d128", wl.FaConfig("t_f16", 3, 8, 2, 128, 300, 2, wl.F16, causal_prefix=297)),
    ("q8_d256", wl.FaConfig("t_q8", 2, 6, 1, 256, 260, 1, wl.Q8_0, causal_prefix=258)),
    ("q4_d128", wl.FaConfig("t_q4", 4, 8, 4, 128, 333, 2, wl.Q4_0, causal_prefix=329)),
    ("e5m2_d128", wl.FaConfig("t_e5", 1, 4, 2, 128, 200, 1, wl.E5M2)),
]


@pytest.mark.parametrize("name,cfg", SMALL, ids=[s[0] for s in SMALL])
def test_fa_oracle_vs_numpy_closed_form(name, cfg):
    case = make_fa_case(cfg, seed=31)
    want, wlse = closed_form(case)
    f64, lse64 = oracle_f64(case)
    assert np.max(np.abs(f64 - want)) < 1e-6  # f64 oracle returns f32
    assert np.max(np.abs(lse64 - wlse)) < 1e-5
    # the loop with f32 value accumulation pins the loop's math tightly
    got, glse = oracle_fa(case, v_acc_f16=False)
    assert np.max(np.abs(got - want)) < 2e-5
    assert np.max(np.abs(glse - wlse)) < 1e-4
    if cfg.kv_type == wl.F16:
        # ggml accumulates F16 V in an f16 vector (rounding each step): bounded, not pinned bitwise
        got16, _ = oracle_fa(case, v_acc_f16=True)
        assert np.max(np.abs(got16 - want)) < 1e-2


@pytest.mark.parametrize("kv", [wl.F16, wl.Q8_0, wl.Q4_0])
def test_fa_oracle_sinks_softcap_alibi(kv):
    cfg = wl.FaConfig("t_feat", 3, 12, 4, 128, 250, 2, kv, causal_prefix=247)
    case = make_fa_case(cfg, seed=33, sinks=True, softcap=30.0, max_bias=8.0, mask_per_seq=True)
    want, wlse = closed_form(case)
    f64, lse64 = oracle_f64(case)
    assert np.max(np.abs(f64 - want)) < 1e-6  # f64 oracle returns f32
    assert np.max(np.abs(lse64 - wlse)) < 1e-5
    got, glse = oracle_fa(case, v_acc_f16=False)
    assert np.max(np.abs(got - want)) < 2e-5
    assert np.max(np.abs(glse - wlse)) < 1e-4


def test_fa_oracle_alibi_slopes():
    lib = oracle.load()
    for H in (4, 12, 24, 32):
        for h in range(H):
            assert abs(lib.xo_alibi_slope(8.0, H, h) - _alibi(h, H, 8.0)) < 1e-6 * _alibi(h, H, 8.0)
        assert lib.xo_alibi_slope(0.0, H, 0) == 1.0


def test_fa_oracle_fully_masked_rows():
    cfg = wl.FaConfig("t_pad", 6, 8, 2, 128, 100, 1, wl.Q4_0, causal_prefix=96, n_q_pad=8)
    case = make_fa_case(cfg, seed=34)
    case.mask = wl.mask_tensor(wl.fa_causal_mask(cfg, n_q_rows=4))  # rows 4.. all -inf
    got, lse = oracle_fa(case)
    assert np.all(got[:, 4:] == 0.0) and np.all(np.isneginf(lse[:, 4:]))
    want, wlse = closed_form(case)
    assert np.max(np.abs(got - want)) < 2e-5


def test_fa_oracle_query_width_invariance():
    cfg = wl.FaConfig("t_inv", 4, 8, 2, 128, 150, 1, wl.Q8_0, causal_prefix=147)
    case = make_fa_case(cfg, seed=35)
    batch, _ = oracle_fa(case)
    q = np.frombuffer(case.q.buf.tobytes(), np.float32).reshape(1, 4, 8, 128)
    m = np.frombuffer(case.mask.buf.tobytes(), np.uint16).reshape(1, -1, 150)
    import dataclasses
    for i in range(4):
        one = dataclasses.replace(case, cfg=wl.FaConfig("t_inv1", 1, 8, 2, 128, 150, 1, wl.Q8_0),
                                  q=wl.fa_q_tensor(q[:, i:i + 1].copy()), mask=wl.mask_tensor(m[:, i:i + 1].copy()),
                                  dst=wl.fa_dst_tensor(1, 1, 8, 128))
        o, _ = oracle_fa(one)
        assert np.array_equal(o[:, 0], batch[:, i])


# ---------------------------------------------------------------- range pass + reduce

def _range_case(kv, active, n_q=3, H=8, Hkv=2, D=128, origin=1000, seed=41):
    q = wl.normal(seed, (n_q, H, D))
    kf = wl.normal(seed + 1, (max(active, 1), Hkv, D))
    vf = wl.normal(seed + 2, (max(active, 1), Hkv, D))
    k = oracle.quantize(kv, kf)
    v = oracle.quantize(kv, vf)
    return q, k, v


@pytest.mark.parametrize("kv", [wl.F16, wl.Q8_0, wl.Q4_0])
@pytest.mark.parametrize("active", [0, 1, 2, 64, 257, 300])
def test_range_attention_vs_closed_form(kv, active):
    n_q, H, Hkv, D, origin = 3, 8, 2, 128, 1000
    q, k, v = _range_case(kv, active)
    positions = np.array([origin + active - 1, origin + active // 2, origin - 5], np.int32)  # last query: nothing
    split_k = max(1, -(-active // 256))
    out, lse, _ = oracle.range_attn(q, positions, H, k, v, Hkv, D, kv, origin, active, 1.0 / 16, split_k)
    kd = oracle.dequant(kv, k, D).astype(np.float64)
    vd = oracle.dequant(kv, v, D).astype(np.float64)
    for i in range(n_q):
        lim = min(active, max(0, positions[i] - origin + 1))
        for h in range(H):
            if lim == 0:
                assert np.all(out[i, h] == 0) and np.isneginf(lse[i, h])
                continue
            s = kd[:lim, h // (H // Hkv)] @ q[i, h].astype(np.float64) / 16
            w = np.exp(s - s.max())
            ref = w @ vd[:lim, h // (H // Hkv)] / w.sum()
            assert np.max(np.abs(out[i, h] - ref)) < 2e-5
            assert abs(lse[i, h] - (s.max() + math.log(w.sum()))) < 1e-4


def test_range_reduce_poison_rules():
    D = 4
    base = np.zeros((3, 2, D + 2), np.float32)
    base[:, :, :D] = 1.0
    base[:, :, D] = [[0.0, 0.5], [1.0, 0.25], [0.5, 0.0]]  # running maxima
    base[:, :, D + 1] = [[1.0, 2.0], [3.0, 1.0], [2.0, 0.0]]  # denominators (row 1 split 2 empty)
    out, lse = oracle.range_reduce(base, D, poison=True)
    assert np.all(np.isfinite(out)) and np.all(np.isfinite(lse))
    # float64 merge identity, ascending splits
    for r in range(2):
        m = base[:, r, D].astype(np.float64)
        l = base[:, r, D + 1].astype(np.float64)
        ok = l > 0
        M = m[ok].max()
        L = (l[ok] * np.exp(m[ok] - M)).sum()
        num = (base[ok, r, :D].astype(np.float64) * np.exp(m[ok] - M)[:, None]).sum(axis=0)
        assert np.max(np.abs(out[r] - num / L)) < 1e-6
        assert abs(lse[r] - (M + math.log(L))) < 1e-6
    for bad in ("nan_den", "neg_den", "inf_max", "nan_num"):
        p = base.copy()
        if bad == "nan_den":
            p[1, 0, D + 1] = np.nan
        elif bad == "neg_den":
            p[1, 0, D + 1] = -1.0
        elif bad == "inf_max":
            p[1, 0, D] = np.inf
        else:
            p[1, 0, 2] = np.nan
        out, lse = oracle.range_reduce(p, D, poison=True)
        assert np.all(np.isnan(out[0])) and np.isnan(lse[0]), bad
        assert np.all(np.isfinite(out[1])), bad
    empty = np.zeros((2, 1, D + 2), np.float32)
    empty[:, :, D] = -np.inf
    out, lse = oracle.range_reduce(empty, D, poison=True)
    assert np.all(out == 0) and np.isneginf(lse[0])
