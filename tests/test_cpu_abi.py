"""The C-ABI library on the host (no GPU calls): it loads, exports every entry
point include/xq_attn.h declares, and its pure host functions (predicates,
workspace sizes, split policy, argument checks) behave as specified.

Split-policy known answers are the reference's own assertions
(tests/rkva_range_profile_cpu.cpp:23-40) restated; the sweep is also compared
with the reference header compiled in oracle/_ref where that is built.
"""
import ctypes
import re

import numpy as np
import pytest

import oracle
import xqattn
from conftest import ROOT
from xqattn import workloads as wl

HEADERS = sorted((ROOT / "include").glob("*.h"))


def lib():
    return xqattn.load()


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(xq_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_loads_and_exports_header():
    l = lib()
    assert [h.name for h in HEADERS] == ["xq_attn.h", "xq_ggml_backend.h"]
    names = declared_functions()
    assert len(names) >= 24
    for n in names:
        assert hasattr(l, n), f"{n} declared in include/ but not exported"
    assert set(xqattn.EXPORTS) == set(names)
    assert l.xq_abi_version() == 1
    assert l.xq_last_error() == b""


def test_split_policy_reference_known_answers():
    sc = xqattn.split_count
    # reference split: clamp(ceil(L/256), 1, 32)
    for L, k in [(0, 1), (1, 1), (256, 1), (257, 2), (28672, 32), (1 << 20, 32)]:
        assert sc(L, xqattn.SPLIT_REFERENCE) == k, L
    # optimized modes at 28672 rows (balanced / fine / coarse)
    assert sc(28672, xqattn.SPLIT_BALANCED) == 128
    assert sc(28672, xqattn.SPLIT_FINE) == 256
    assert sc(28672, xqattn.SPLIT_COARSE) == 56
    assert sc(1, xqattn.SPLIT_BALANCED) == 1
    # the multi-query verify split (tests/rkva_range_profile_cpu.cpp:135-139)
    assert sc(1, xqattn.SPLIT_MQ_BALANCED) == 1
    assert (sc(58128, xqattn.SPLIT_MQ_BALANCED), xqattn.split_rows(58128, xqattn.SPLIT_MQ_BALANCED)) == (114, 512)
    assert (sc(58128, xqattn.SPLIT_MQ_FINE), xqattn.split_rows(58128, xqattn.SPLIT_MQ_FINE)) == (228, 256)


def test_split_policy_length_mode():
    """The length-only mode is AUTO's partition for 16 (sequence x KV head)
    units: 16 x 2048 rows at 32k (the 4-sequence, 4-KV-head decode's own AUTO
    partition), 16 x 256 at 4k, 16 x 1040 at 16392, ceil(L/256) splits of 256
    below 4096 rows, one split up to 256 rows."""
    sc, sr = xqattn.split_count, xqattn.split_rows
    L_ = xqattn.SPLIT_LENGTH
    assert (sc(32768, L_), sr(32768, L_)) == (16, 2048)
    assert (sc(4096, L_), sr(4096, L_)) == (16, 256)
    assert (sc(16392, L_), sr(16392, L_)) == (16, 1040)
    assert (sc(1000, L_), sr(1000, L_)) == (4, 256)
    assert (sc(256, L_), sr(256, L_)) == (1, 256) and (sc(1, L_), sr(1, L_)) == (1, 16)
    for L in (1, 17, 255, 4097, 32768, 131072):
        assert sc(L, L_) <= 16 and sr(L, L_) % 16 == 0 and sr(L, L_) * (sc(L, L_) - 1) < L <= sr(L, L_) * sc(L, L_)


@pytest.mark.parametrize("mode", [xqattn.SPLIT_AUTO, xqattn.SPLIT_REFERENCE, xqattn.SPLIT_BALANCED,
                                  xqattn.SPLIT_FINE, xqattn.SPLIT_COARSE, xqattn.SPLIT_NONE,
                                  xqattn.SPLIT_MQ_BALANCED, xqattn.SPLIT_MQ_FINE, xqattn.SPLIT_LENGTH])
def test_split_policy_covers_every_row(mode):
    for L in [1, 7, 16, 31, 32, 33, 128, 129, 255, 256, 257, 512, 1000, 4096, 4133, 16392, 28672, 32768, 131072]:
        k = xqattn.split_count(L, mode)
        rows = xqattn.split_rows(L, mode)
        assert 1 <= k <= 256
        assert rows * k >= L, (L, k, rows)  # every row is covered
        if mode in (xqattn.SPLIT_AUTO, xqattn.SPLIT_LENGTH):
            assert rows % 16 == 0 and rows * (k - 1) < L  # no empty split
        if L in (1, 31, 32, 33, 128, 129, 512, 4096, 28672, 131072):
            assert rows * (k - 1) < L  # the reference's own assertion for these lengths
        if mode == xqattn.SPLIT_NONE:
            assert k == 1
        if mode in (xqattn.SPLIT_MQ_BALANCED, xqattn.SPLIT_MQ_FINE):
            # whole 64-row tiles, no empty split, never more splits than the mode's
            assert rows % 64 == 0 and rows * (k - 1) < L
            base = xqattn.SPLIT_BALANCED if mode == xqattn.SPLIT_MQ_BALANCED else xqattn.SPLIT_FINE
            assert k <= xqattn.split_count(L, base)


def test_split_policy_matches_reference_header():
    ref = oracle.load_ref()
    if ref is None:
        pytest.skip("reference shim not built")
    modes = {xqattn.SPLIT_BALANCED: 1, xqattn.SPLIT_FINE: 2, xqattn.SPLIT_COARSE: 3}
    for L in list(range(0, 700)) + [1000, 4096, 28672, 58128, 131072]:
        assert xqattn.split_count(L, xqattn.SPLIT_REFERENCE) == ref.xr_reference_split_k(L)
        for m, rm in modes.items():
            k = ref.xr_optimized_split_k(L, rm)
            assert xqattn.split_count(L, m) == k, (L, m)
            if L:
                assert xqattn.split_rows(L, m) == ref.xr_split_rows(L, k), (L, m)
        kk, rr = ctypes.c_uint32(), ctypes.c_uint32()
        for m, rm in {xqattn.SPLIT_MQ_BALANCED: 1, xqattn.SPLIT_MQ_FINE: 2}.items():
            ref.xr_q4_mq_split(L, rm, ctypes.byref(kk), ctypes.byref(rr))
            if L:
                assert (xqattn.split_count(L, m), xqattn.split_rows(L, m)) == (kk.value, rr.value), (L, m)


def _desc(typ, ne, nb=None, esize=None):
    d = xqattn.XqTensor()
    d.type = typ
    esize = esize or wl.TYPE_SIZE[typ]
    if nb is None:
        blk = wl.BLOCK[typ]
        nb = [esize, esize * ne[0] // blk]
        nb.append(nb[1] * ne[1])
        nb.append(nb[2] * ne[2])
    for i in range(4):
        d.ne[i], d.nb[i] = ne[i], nb[i]
    d.data = 0x100000  # never dereferenced by the host checks
    return d


def _fa_descs(kv=wl.Q8_0, D=256, NQ=1, H=24, Hkv=4, L=32768, B=4):
    rec = wl.record_bytes(kv, D)
    q = _desc(wl.F32, (D, NQ, H, B))
    k = _desc(kv, (D, L, Hkv, B), (wl.TYPE_SIZE[kv], Hkv * rec, rec, L * Hkv * rec))
    v = _desc(kv, (D, L, Hkv, B), (wl.TYPE_SIZE[kv], Hkv * rec, rec, L * Hkv * rec))
    m = _desc(wl.F16, (L, NQ, 1, B))
    dst = _desc(wl.F32, (D, H, NQ, B))
    return q, k, v, m, dst


def test_fa_predicate_and_workspace():
    l = lib()
    p = xqattn.fa_params(1.0 / 16)
    for kv in (wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2):
        for D in (128, 256):
            q, k, v, m, dst = _fa_descs(kv=kv, D=D)
            assert l.xq_supports_flash_attn_ext(*(ctypes.byref(x) for x in (q, k, v, m)), None, ctypes.byref(dst),
                                                ctypes.byref(p)) == 1, (kv, D)
            nb = ctypes.c_size_t(0)
            st = l.xq_flash_attn_ext_workspace(*(ctypes.byref(x) for x in (q, k, v, m)), None, ctypes.byref(dst),
                                              ctypes.byref(p), ctypes.byref(nb))
            assert st == 0 and nb.value > 0
    q, k, v, m, dst = _fa_descs(D=64)
    assert l.xq_supports_flash_attn_ext(*(ctypes.byref(x) for x in (q, k, v, m)), None, ctypes.byref(dst),
                                        ctypes.byref(p)) == 0
    assert b"head dim" in l.xq_last_error()
    q, k, v, m, dst = _fa_descs(H=20)  # 20 % 4 == 0 but GQA 5 fine; 21 is not
    q, k, v, m, dst = _fa_descs(H=21)
    assert l.xq_supports_flash_attn_ext(*(ctypes.byref(x) for x in (q, k, v, m)), None, ctypes.byref(dst),
                                        ctypes.byref(p)) == 0


def test_fa_workspace_reserves_mask_relayout():
    """With a mask the workspace holds room for the mask rows re-laid with an
    even element count ([n_q][mask heads][mask sequences] rows of f16, 256-byte
    rounded), used when the rows are not 4-byte aligned."""
    l = lib()
    p = xqattn.fa_params(1.0 / 16)
    for L, NQ, B in ((193, 1, 1), (1001, 4, 2), (32768, 1, 4)):
        q, k, v, m, dst = _fa_descs(kv=wl.Q8_0, D=128, NQ=NQ, H=8, Hkv=2, L=L, B=B)
        with_mask, without = ctypes.c_size_t(0), ctypes.c_size_t(0)
        assert l.xq_flash_attn_ext_workspace(*(ctypes.byref(x) for x in (q, k, v, m)), None, ctypes.byref(dst),
                                             ctypes.byref(p), ctypes.byref(with_mask)) == 0
        assert l.xq_flash_attn_ext_workspace(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), None, None,
                                             ctypes.byref(dst), ctypes.byref(p), ctypes.byref(without)) == 0
        pack = B * NQ * (L + (L & 1)) * 2
        assert with_mask.value - without.value == (pack + 255) // 256 * 256, (L, NQ, B)


def test_fa_entry_rejects_before_any_device_work():
    l = lib()
    q, k, v, m, dst = _fa_descs()
    p = xqattn.fa_params(1.0 / 16)
    st = l.xq_flash_attn_ext(*(ctypes.byref(x) for x in (q, k, v, m)), None, ctypes.byref(dst), None,
                             ctypes.byref(p), None, 0, None)
    assert st == 4  # workspace missing
    assert b"workspace" in l.xq_last_error()
    st = l.xq_flash_attn_ext(*(ctypes.byref(x) for x in (q, k, v, m)), None, ctypes.byref(dst), None, None,
                             None, 0, None)
    assert st == 3  # null params


def test_gdn_predicate():
    l = lib()
    T, B = 1, 8
    q = _desc(wl.F32, (128, 16, T, B))
    k = _desc(wl.F32, (128, 16, T, B))
    v = _desc(wl.F32, (128, 32, T, B))
    g = _desc(wl.F32, (1, 32, T, B))
    beta = _desc(wl.F32, (1, 32, T, B))
    s = _desc(wl.F32, (128, 128, 32, B))
    dst = _desc(wl.F32, (4096, T + 128, B, 1))
    args = [ctypes.byref(x) for x in (q, k, v, g, beta, s, dst)]
    assert l.xq_supports_gated_delta_net(*args, 1, 0) == 1
    assert l.xq_supports_gated_delta_net(*args, 1, 1) == 0  # raw gates are outside the contract
    assert l.xq_supports_gated_delta_net(*args, 0, 0) == 0  # at least one snapshot slot
    v_bad = _desc(wl.F32, (128, 31, T, B))
    assert l.xq_supports_gated_delta_net(args[0], args[1], ctypes.byref(v_bad), *args[3:], 1, 0) == 0


def test_gdn_workspace_query():
    """AUTO runs prefills longer than one chunk on the chunked kernels: one
    workspace record of 27648 bytes per (sequence, v-head, 64-token chunk) of
    the first T - (slots - 1) tokens; the step kernel needs none."""
    l = lib()
    n = ctypes.c_size_t(0)

    def need(T, B, slots, mode, typ=wl.BF16):
        q = _desc(typ, (128, 16, T, B))
        v = _desc(typ, (128, 32, T, B))
        assert l.xq_gated_delta_net_workspace(ctypes.byref(q), ctypes.byref(v), slots, mode, ctypes.byref(n)) == 0
        return n.value

    rec = 2 * 64 * 64 * 2 + 1024 + 10 * 1024  # T (f16 hi, lo), decays and G, the P tiles
    assert need(4096, 1, 1, xqattn.GDN_AUTO, wl.F32) == 32 * 64 * rec  # the same record for f32 rows
    assert need(200, 2, 3, xqattn.GDN_CHUNKED) == 2 * 32 * 4 * rec  # 198 tokens -> 4 chunks
    assert need(4096, 1, 1, xqattn.GDN_AUTO) == 32 * 64 * rec
    assert need(64, 1, 1, xqattn.GDN_AUTO) == 0                     # one chunk: step kernel
    assert need(4096, 1, 1, xqattn.GDN_STEP) == 0
    assert need(3, 1, 5, xqattn.GDN_CHUNKED) == 0                   # every token keeps a snapshot


@pytest.mark.parametrize("typ,d,want", [(wl.F16, 128, 256), (wl.Q8_0, 256, 272), (wl.Q8_0, 128, 136),
                                        (wl.Q4_0, 128, 72), (wl.E5M2, 256, 256), (wl.F32, 128, 512)])
def test_kv_record_bytes(typ, d, want):
    assert lib().xq_kv_record_bytes(typ, d) == want
