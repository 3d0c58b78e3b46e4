"""Merge of position-split range results (oracle/xq_oracle.c xo_lse_merge, the
host side of xq_fa_lse_merge): OUT/LSE pairs of the same (query, head) rows
over disjoint KV ranges combined into the result over their union.

Pins: the merge of range attention over pieces of the KV rows equals range
attention over all of them (uwp/rkva/remote-attn-protocol.h:228-231 semantics
on both sides); a float64 restatement of the weights; a single part is returned
unchanged; empty parts drop out; the reducer's poisoning rules
(shaders/rkva/rkva_range_reduce_opt.hlsl:39-56,126-132).
"""
import ctypes

import numpy as np
import pytest

import oracle
import xqattn
from conftest import assert_close
from xqattn import workloads as wl


def _merge64(parts_out, parts_lse):
    po = parts_out.astype(np.float64)
    pl = parts_lse.astype(np.float64)
    live = pl != -np.inf
    M = np.where(live, pl, -np.inf).max(axis=0)
    with np.errstate(invalid="ignore"):  # rows no part sees: -inf - -inf, masked below
        w = np.where(live, np.exp(np.where(live, pl - M, 0.0)), 0.0)
    s = w.sum(axis=0)
    out = np.where(s[:, None] > 0, (w[:, :, None] * po).sum(axis=0) / np.where(s > 0, s, 1)[:, None], 0.0)
    lse = np.where(s > 0, M + np.log(np.where(s > 0, s, 1)), -np.inf)
    return out, lse


def _range(kv_type, kraw, vraw, q, positions, origin, a, b, n_head, hkv, D, scale=1.0 / 16):
    split_k = int(oracle.load().xo_ref_split_k(b - a))
    out, lse, _ = oracle.range_attn(q, positions, n_head, kraw[a:b], vraw[a:b], hkv, D, kv_type, origin + a,
                                    b - a, scale, split_k)
    return out, lse


@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0])
@pytest.mark.parametrize("cuts", [(0, 150, 300), (0, 64, 65, 300), (0, 10, 200, 299, 300)])
def test_merge_of_pieces_equals_whole_range(kv_type, cuts):
    n_head, hkv, D, origin, active = 8, 2, 128, 4096, 300
    kraw = oracle.quantize(kv_type, wl.normal(61, (active, hkv, D)))
    vraw = oracle.quantize(kv_type, wl.normal(62, (active, hkv, D)))
    # queries: sees all rows, sees a prefix, sees none (before the origin), sees one row
    positions = np.array([origin + active - 1, origin + 120, origin - 3, origin], np.int32)
    q = wl.normal(63, (positions.size, n_head, D))
    whole, wlse = _range(kv_type, kraw, vraw, q, positions, origin, 0, active, n_head, hkv, D)
    parts = [_range(kv_type, kraw, vraw, q, positions, origin, a, b, n_head, hkv, D)
             for a, b in zip(cuts[:-1], cuts[1:])]
    po = np.stack([p[0].reshape(-1, D) for p in parts])
    pl = np.stack([p[1].reshape(-1) for p in parts])
    out, lse = oracle.lse_merge(po, pl)
    assert_close(out, whole.reshape(-1, D), atol=1e-5, rtol=1e-5, what="merged O vs whole range")
    assert_close(lse, wlse.reshape(-1), atol=1e-5, rtol=1e-6, what="merged LSE vs whole range")
    # the query before the origin sees nothing in any piece
    assert np.all(out.reshape(positions.size, n_head, D)[2] == 0) and np.all(np.isneginf(lse.reshape(-1, n_head)[2]))


def test_merge_matches_float64_and_part_order():
    rng = np.random.default_rng(5)
    n_parts, rows, D = 5, 40, 96
    po = rng.standard_normal((n_parts, rows, D)).astype(np.float32)
    pl = (rng.standard_normal((n_parts, rows)) * 20).astype(np.float32)
    pl[1, ::3] = -np.inf                      # empty pieces for some rows
    pl[:, 7] = -np.inf                        # a row no piece sees
    po[1, ::3] = np.inf                       # never read: the piece is empty
    out, lse = oracle.lse_merge(po, pl)
    out64, lse64 = _merge64(np.where(np.isinf(pl)[:, :, None], 0, po), pl)
    assert_close(out, out64, atol=1e-6, rtol=1e-5, what="merge vs float64")
    assert_close(lse, lse64, atol=1e-6, rtol=1e-6, what="merged LSE vs float64")
    assert np.all(out[7] == 0) and np.isneginf(lse[7])


def test_single_part_is_returned_unchanged():
    rng = np.random.default_rng(6)
    po = rng.standard_normal((1, 17, 256)).astype(np.float32)
    pl = rng.standard_normal((1, 17)).astype(np.float32)
    pl[0, 3] = -np.inf
    po[0, 3] = 0.0
    out, lse = oracle.lse_merge(po, pl)
    assert np.array_equal(out, po[0]) and np.array_equal(lse, pl[0])


@pytest.mark.parametrize("bad", ["nan_lse", "inf_lse", "nan_out"])
def test_merge_poisons_rows(bad):
    rng = np.random.default_rng(7)
    po = rng.standard_normal((3, 6, 64)).astype(np.float32)
    pl = rng.standard_normal((3, 6)).astype(np.float32)
    if bad == "nan_lse":
        pl[1, 2] = np.nan
    elif bad == "inf_lse":
        pl[1, 2] = np.inf
    else:
        po[1, 2, 5] = np.nan
    out, lse = oracle.lse_merge(po, pl)
    assert np.all(np.isnan(out[2])) and np.isnan(lse[2])
    keep = [r for r in range(6) if r != 2]
    assert np.all(np.isfinite(out[keep])) and np.all(np.isfinite(lse[keep]))


def test_merge_entry_rejects_bad_arguments_before_device_work():
    lib = xqattn.load()
    P = ctypes.c_void_p
    dummy = P(0x100000)
    assert lib.xq_fa_lse_merge(None, dummy, 2, 4, 128, dummy, dummy, None) == 3          # null
    assert lib.xq_fa_lse_merge(dummy, dummy, 0, 4, 128, dummy, dummy, None) == 3         # no parts
    assert lib.xq_fa_lse_merge(dummy, dummy, 2, 4, 600, dummy, dummy, None) == 1         # head dim
    assert b"head dim" in lib.xq_last_error()
    assert lib.xq_fa_lse_merge(P(0x100002), dummy, 2, 4, 128, dummy, dummy, None) == 1   # alignment
