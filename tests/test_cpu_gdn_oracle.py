"""CPU pins of the gated-delta-net oracle (oracle/xq_oracle.c, the host mirror
of shaders/ggml_d3d12_gated_delta_net.hlsl:40-85 in the summation order of
src/bridge/ggml_d3d12.cpp:113-158) against an independent float64 numpy
recurrence written from the shader's per-column algorithm, closed forms, and
the reference selftest's invariants (ggml_d3d12.cpp:222-301, 333-351).
"""
import math

import numpy as np
import pytest

import oracle
from gdn_cases import SENTINEL, _selftest_inputs, make_gdn_case
from xqattn import workloads as wl

SCALE = 1.0 / math.sqrt(128.0)


def numpy_recurrence(q, k, v, g, beta, st, slots):
    """q,k [B,T,16,128]; v [B,T,32,128]; g,beta [B,T,32]; st [B,32,c=128,i=128].
    Returns out [B, T + 128*min(T, slots), 4096] in float64 (snapshot slot j =
    the state j tokens before the end)."""
    B, T = q.shape[:2]
    nsl = min(T, slots)
    out = np.zeros((B, T + 128 * nsl, 4096))
    for b in range(B):
        S = st[b].astype(np.float64).copy()  # [h][c][i]
        snaps = {}
        for t in range(T):
            for h in range(32):
                kh = h % 16  # k-heads broadcast over v-heads by modulo
                kv = k[b, t, kh].astype(np.float64)
                S[h] *= math.exp(float(g[b, t, h]))
                pred = S[h] @ kv
                delta = (v[b, t, h].astype(np.float64) - pred) * float(beta[b, t, h])
                S[h] += delta[:, None] * kv[None, :]
                out[b, t, h * 128:(h + 1) * 128] = (S[h] @ q[b, t, kh].astype(np.float64)) * SCALE
            j = T - 1 - t
            if j < nsl:
                snaps[j] = S.copy()
        for j in range(nsl):
            out[b, T + 128 * j:T + 128 * (j + 1)] = snaps[j].reshape(128, 4096)
    return out


def test_f64_oracle_vs_numpy_recurrence():
    T, slots, B = 3, 5, 2
    q, k, v, g, beta, st = _selftest_inputs(T, B)
    case = make_gdn_case(T, slots, B=B, dist="selftest")
    want = numpy_recurrence(q, k, v, g, beta, st, slots)
    got = case.oracle_f64()
    n = T + 128 * min(T, slots)
    assert np.max(np.abs(got[:, :n] - want)) < 1e-12


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 64])
@pytest.mark.parametrize("slots", [1, 5])
def test_oracle_vs_f64_selftest_matrix(T, slots):
    """The reference selftest's tolerance: relative error <= 1e-4."""
    case = make_gdn_case(T, slots, B=2, dist="selftest", pad=3 if T in (3, 5) else 0)
    got = case.oracle()
    want = case.oracle_f64()
    n = T + 128 * min(T, slots)
    err = np.max(np.abs(got[:, :n] - want[:, :n]))
    scale = np.max(np.abs(want[:, :n]))
    assert err <= 1e-4 * scale
    assert np.all(got[:, n:] == SENTINEL)  # unwritten slots stay untouched


def test_zero_state_single_step_closed_form():
    q, k, v, g, beta, st = wl.gdn_inputs(wl.GdnConfig("z", 1, 1, 1), seed=5)
    st = np.zeros_like(st)
    case = make_gdn_case(1, 1, B=1, seed=5)
    case.state = wl.f32_tensor(st, (128, 128, 32, 1))
    got = case.oracle()
    # S = k (v beta)^T per head (kv = 0), y = (k . q) v beta / sqrt(128)
    for h in range(32):
        kh = h % 16
        kq = float(k[0, 0, kh].astype(np.float64) @ q[0, 0, kh].astype(np.float64))
        y = kq * v[0, 0, h].astype(np.float64) * float(beta[0, 0, h]) * SCALE
        assert np.max(np.abs(got[0, 0, h * 128:(h + 1) * 128] - y)) < 1e-6
        S = np.outer(v[0, 0, h].astype(np.float64) * float(beta[0, 0, h]), k[0, 0, kh])
        assert np.max(np.abs(got[0, 1:129].reshape(32, 128, 128)[h] - S)) < 1e-6


def test_beta_zero_is_pure_decay():
    T = 4
    q, k, v, g, beta, st = wl.gdn_inputs(wl.GdnConfig("d", T, 1, 1), seed=6)
    case = make_gdn_case(T, 1, B=1, seed=6)
    case.beta = wl.f32_tensor(np.zeros_like(beta), (1, 32, T, 1))
    got = case.oracle()
    decay = np.exp(np.cumsum(g[0].astype(np.float64), axis=0))  # [T, 32]
    final = got[0, T:T + 128].reshape(32, 128, 128)
    want = st[0].astype(np.float64) * decay[-1][:, None, None]
    assert np.max(np.abs(final - want)) < 1e-5 * np.max(np.abs(want))
    for t in range(T):
        for h in (0, 17, 31):
            y = (st[0, h].astype(np.float64) * decay[t, h]) @ q[0, t, h % 16].astype(np.float64) * SCALE
            assert np.max(np.abs(got[0, t, h * 128:(h + 1) * 128] - y)) < 1e-5


def test_prefix_invariance_and_snapshot_slots():
    long = make_gdn_case(8, 5, B=1, dist="selftest").oracle()
    for T in (3, 5, 7):
        short = make_gdn_case(T, 1, B=1, dist="selftest").oracle()
        assert np.array_equal(short[0, :T], long[0, :T])  # outputs of the common prefix
        # slot j of the 8-token run holds the state after 8 - j tokens
        j = 8 - T
        if j < 5:
            assert np.array_equal(long[0, 8 + 128 * j:8 + 128 * (j + 1)], short[0, T:T + 128])


def test_head_modulo_broadcast_is_pinned():
    """Swapping k-heads 0 and 1 must move exactly the v-heads h with h % 16 in {0, 1}."""
    T = 2
    q, k, v, g, beta, st = wl.gdn_inputs(wl.GdnConfig("m", T, 1, 1), seed=7)
    base = make_gdn_case(T, 1, B=1, seed=7).oracle()
    k2 = k.copy()
    k2[:, :, [0, 1]] = k2[:, :, [1, 0]]
    case = make_gdn_case(T, 1, B=1, seed=7)
    case.k = wl.f32_tensor(k2, (128, 16, T, 1))
    swapped = case.oracle()
    for h in range(32):
        same = np.array_equal(base[0, :T, h * 128:(h + 1) * 128], swapped[0, :T, h * 128:(h + 1) * 128])
        assert same == (h % 16 not in (0, 1)), h
