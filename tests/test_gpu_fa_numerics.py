"""GPU numerics of GGML_OP_FLASH_ATTN_EXT beyond the N(0,1) configurations:

* the value path's accuracy does not depend on V's magnitude (the 32k q8_0 decode's and the q4_0 verify's geometry,
  V scaled by 1e-1 .. 1e-3, both engines, 1e-5 relative to max|f64|);
* KV dequantisation inside the kernels is bit-exact: with Q = 0 and one visible
  row per (query, head) the output is that row's dequantised V, bit for bit
  (shaders/rkva/rkva_range_attn.hlsl:28-57 decoders, ggml's to_float);
* rows a query does not see never reach it, even when they hold Inf/NaN, and a
  range call turns exactly the rows that see a non-finite record into NaN
  (shaders/rkva/rkva_range_reduce_opt.hlsl:39-56,126-132);
* a non-finite V element or block scale reaches exactly its own dims of the
  queries that see its row, as ggml's per-dim accumulation does, whatever
  queries share the tile;
* a query's bits do not depend on how many queries (n_q 1 / 3 / 8) or, under
  the length-only split modes, how many sequences (B 1 / 4) share the call, at
  the 32k head-dim-256 geometry and at head dim 128 with GQA 2 and 4
  (patches/0008-flash-attn-query-consistency.patch:40-56,
  uwp/rkva/rkva-range-profile.h:99-107);
* the verify configuration at full size with padded and fully masked query rows.
"""
import dataclasses

import numpy as np
import pytest

import oracle
import xqattn
from conftest import assert_close, case_note
from fa_cases import make_fa_case, oracle_f64, oracle_fa, run_fa_gpu
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu

ENGINES = [xqattn.ENGINE_MFMA, xqattn.ENGINE_VALU]
ENGINE_IDS = ["mfma", "valu"]
NAN16, INF16 = 0x7E00, 0x7C00


# ---------------------------------------------------------------------------
# value path vs V's magnitude
# ---------------------------------------------------------------------------

_VCACHE = {}


def _vscale_case(cfg, v_scale):
    key = (cfg.name, v_scale)
    if key not in _VCACHE:
        _VCACHE.clear()  # one full-size case in memory at a time
        case = make_fa_case(cfg, seed=11, v_scale=v_scale)
        ref, _ = oracle_f64(case)
        _VCACHE[key] = (case, ref)
    return _VCACHE[key]


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("v_scale", [1e-1, 1e-2, 1e-3])
@pytest.mark.parametrize("cfg", [wl.FA_C2, wl.FA_C5], ids=lambda c: c.name)
def test_fa_value_path_independent_of_v_scale(torch_gpu, cfg, v_scale, engine):
    """max|gpu - f64| / max|f64| <= 1e-5 whatever V's scale: the weight x block
    scale products keep f32's exponent range and about 22 significant bits on
    both engines (ggml forms them in f32)."""
    case_note(f"v_scale {v_scale} {cfg.name} engine {engine}")
    case, ref = _vscale_case(cfg, v_scale)
    got, _ = run_fa_gpu(case, torch_gpu, engine=engine)
    rel = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
    print(f"{cfg.name} v_scale {v_scale} engine {engine}: max|gpu-f64|/max|f64| = {rel:.2e}")
    assert rel <= 1e-5, rel


# ---------------------------------------------------------------------------
# dequantisation bit-exact
# ---------------------------------------------------------------------------

def _one_row_case(kv_type, D, seed=3):
    B, NQ, H, Hkv, L = 1, 4, 8, 2, 300
    G = H // Hkv
    cfg = wl.FaConfig("one_row", NQ, H, Hkv, D, L, B, kv_type)
    vf = wl.normal(seed, (B, L, Hkv, D)) * np.float32(3.0)
    vf[0, 7, 0, :] = np.float32(1e-6)   # tiny values (f16 subnormal records)
    vraw = oracle.quantize(kv_type, vf)
    kraw = oracle.quantize(kv_type, wl.normal(seed + 1, (B, L, Hkv, D)))
    q = np.zeros((B, NQ, H, D), np.float32)
    rows = np.array([[(37 * iq + 101 * h + 13) % L for h in range(H)] for iq in range(NQ)])
    rows[0, 0] = 7
    m = np.full((1, H, NQ, L), 0xFC00, np.uint16)  # [Bm, H, n_q, L]: per-head mask planes
    for iq in range(NQ):
        for h in range(H):
            m[0, h, iq, rows[iq, h]] = 0
    mask = wl.HostTensor(wl.F16, (L, NQ, H, 1), (2, 2 * L, 2 * L * NQ, 2 * L * NQ * H), m.reshape(-1).view(np.uint8))
    case = dataclasses.replace(
        make_fa_case(cfg, seed=seed, mask=None), q=wl.fa_q_tensor(q), k=wl.kv_tensor(kraw, kv_type, D),
        v=wl.kv_tensor(vraw, kv_type, D), mask=mask)
    deq = oracle.dequant(kv_type, vraw, D)  # [B, L, Hkv, D]
    want = np.empty((B, NQ, H, D), np.float32)
    for iq in range(NQ):
        for h in range(H):
            want[0, iq, h] = deq[0, rows[iq, h], h // G]
    return case, want


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("split_mode", [xqattn.SPLIT_AUTO, xqattn.SPLIT_NONE], ids=["auto", "none"])
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2], ids=lambda t: wl.TYPE_NAME[t])
def test_fa_dequant_bit_exact_one_visible_row(torch_gpu, kv_type, D, split_mode, engine):
    """Q = 0 and one visible row per (query, head): every weight is a power of two
    and the output is the dequantised V row, bit for bit."""
    case_note(f"one visible row {wl.TYPE_NAME[kv_type]} D{D} split {split_mode} engine {engine}")
    case, want = _one_row_case(kv_type, D)
    got, lse = run_fa_gpu(case, torch_gpu, split_mode=split_mode, engine=engine)
    # equal as floats: every nonzero element bit for bit; a zero element may
    # carry either sign (ggml's accumulator also starts at +0, so 0*d with d < 0
    # leaves +0 in its output too)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} elements differ, first {bad[0]}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"
    nz = want != 0
    assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))
    assert np.all(np.abs(lse) < 1e-6)


# scales and elements at the formats' edges: f16 +-65504, +-0, the smallest
# and largest subnormals; int8 -128 and 127; q4_0 nibbles 0 and 15; E5M2's
# largest finite, subnormals and -0 (each quantized row keeps one scale, as a
# row's blocks of a real cache lie within f16's range of one another)
_F16_EDGES = [0x7BFF, 0xFBFF, 0x0001, 0x8001, 0x8000, 0x0000, 0x0400, 0x03FF, 0x83FF, 0x3C00, 0xBC00, 0x7800]
_E5M2_EDGES = [0x7B, 0xFB, 0x01, 0x81, 0x80, 0x00, 0x04, 0x03, 0x3C, 0xBC, 0x78, 0x7A]
_SCALE_EDGES = [0x7BFF, 0xFBFF, 0x0001, 0x8000, 0x03FF, 0x0400]


def _edge_record(kv_type, D, j):
    """Record j of the edge set (bytes) and its values, decoded here with numpy
    from the block layouts (f16 d then int8 qs[32]; f16 d then 16 bytes, element
    i < 16 the low nibble of byte i, element i >= 16 the high nibble of byte i - 16,
    value (nibble - 8) d; E5M2 = the high byte of an f16)."""
    if kv_type == wl.F16:
        bits = np.array([_F16_EDGES[(i + j) % len(_F16_EDGES)] for i in range(D)], np.uint16)
        return bits.view(np.uint8), bits.view(np.float16).astype(np.float32)
    if kv_type == wl.E5M2:
        b = np.array([_E5M2_EDGES[(i + j) % len(_E5M2_EDGES)] for i in range(D)], np.uint8)
        return b, (b.astype(np.uint16) << 8).view(np.float16).astype(np.float32)
    d_bits = np.uint16(_SCALE_EDGES[j % len(_SCALE_EDGES)])
    d = np.float32(np.array([d_bits], np.uint16).view(np.float16)[0])
    raw, vals = [], []
    for blk in range(D // 32):
        if kv_type == wl.Q8_0:
            qs = np.array([(-128 + 8 * i + blk + j) % 256 - 128 if i else -128 for i in range(32)], np.int16)
            qs[31] = 127
            raw.append(np.concatenate([np.array([d_bits], np.uint16).view(np.uint8), qs.astype(np.int8).view(np.uint8)]))
            vals.append(qs.astype(np.float32) * d)
        else:
            lo = np.array([(i + blk + j) % 16 for i in range(16)], np.uint8)
            hi = np.array([15 - (i + blk) % 16 for i in range(16)], np.uint8)
            raw.append(np.concatenate([np.array([d_bits], np.uint16).view(np.uint8), lo | (hi << 4)]))
            vals.append((np.concatenate([lo, hi]).astype(np.float32) - np.float32(8)) * d)
    return np.concatenate(raw), np.concatenate(vals).astype(np.float32)


def _edge_case(kv_type, D):
    """The one-visible-row case with edge records in six rows of both KV heads,
    each seen alone by a (query, head) pair of its own."""
    case, want = _one_row_case(kv_type, D)
    vraw = np.frombuffer(case.v.buf.tobytes(), np.uint8).reshape(1, 300, 2, -1).copy()
    mraw = np.frombuffer(case.mask.buf.tobytes(), np.uint16).reshape(8, 4, 300).copy()  # [H, n_q, L]
    seen = {int(r) for r in np.argwhere(mraw == 0)[:, 2]}  # rows the other pairs see
    edge_rows = [r for r in (50, 123, 211, 260, 299, 1, 2, 3, 4, 5, 6, 8, 9) if r not in seen][:6]
    for j, r in enumerate(edge_rows):
        for hk in range(2):
            rec, vals = _edge_record(kv_type, D, j + 3 * hk)
            vraw[0, r, hk] = rec
        # (query j % 4, head 2 + j // 4) on KV head 0 and (j % 4, 6 + j // 4)
        # on KV head 1 see row r only: a pair of its own for every edge row
        iq = j % 4
        for hk, h in ((0, 2 + j // 4), (1, 6 + j // 4)):
            mraw[h, iq, :] = 0xFC00
            mraw[h, iq, r] = 0
            want[0, iq, h] = _edge_record(kv_type, D, j + 3 * hk)[1]
    case = dataclasses.replace(case, v=wl.kv_tensor(vraw, kv_type, D),
                               mask=wl.HostTensor(wl.F16, case.mask.ne, case.mask.nb, mraw.reshape(-1).view(np.uint8)))
    return case, want


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2], ids=lambda t: wl.TYPE_NAME[t])
def test_fa_dequant_bit_exact_edge_records(torch_gpu, kv_type, D, engine):
    """The one-visible-row output of V records that hold the formats' edge values
    is those values, bit for bit (zeros of either sign), for every query whose
    visible row is an edge record."""
    case_note(f"edge records {wl.TYPE_NAME[kv_type]} D{D} engine {engine}")
    case, want = _edge_case(kv_type, D)
    got, lse = run_fa_gpu(case, torch_gpu, engine=engine)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} elements differ, first {bad[0]}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"
    nz = want != 0
    assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))


# ---------------------------------------------------------------------------
# non-finite records
# ---------------------------------------------------------------------------

def _spoil(raw, kv_type, row, head, what):
    """Make one record of raw [L, Hkv, rec] non-finite: an element (F16, E5M2) or
    the scale of block 1 (q8_0, q4_0)."""
    rec = raw[row, head]
    if kv_type == wl.F16:
        rec[10:12] = np.frombuffer(np.uint16(NAN16 if what == "nan" else INF16).tobytes(), np.uint8)
    elif kv_type == wl.E5M2:
        rec[5] = 0x7F if what == "nan" else 0x7C
    else:
        bb = 34 if kv_type == wl.Q8_0 else 18
        rec[bb:bb + 2] = np.frombuffer(np.uint16(NAN16 if what == "nan" else INF16).tobytes(), np.uint8)


@pytest.mark.parametrize("split_mode", [xqattn.SPLIT_NONE, xqattn.SPLIT_REFERENCE], ids=["one_split", "splits"])
@pytest.mark.parametrize("where,what", [("k", "nan"), ("v", "nan"), ("v", "inf")])
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2], ids=lambda t: wl.TYPE_NAME[t])
def test_fa_range_nonfinite_record_poisons_exactly_the_rows_that_see_it(torch_gpu, kv_type, where, what,
                                                                        split_mode):
    """A NaN/Inf K or V record at row R of KV head 1 makes OUT and LSE NaN for
    exactly the (query, head) rows with head in KV head 1's group whose causal
    limit passes R; every other row stays finite and matches the oracle."""
    torch = torch_gpu
    n_head, hkv, D, origin, active, R = 8, 2, 128, 1000, 700, 400
    G = n_head // hkv
    kraw = oracle.quantize(kv_type, wl.normal(81, (active, hkv, D)))
    vraw = oracle.quantize(kv_type, wl.normal(82, (active, hkv, D)))
    _spoil(kraw if where == "k" else vraw, kv_type, R, 1, what)
    positions = np.array([origin + 300, origin + R, origin + R - 1, origin + 699, origin - 3, origin + 2000],
                         np.int32)
    n_q = positions.size
    q = wl.normal(83, (n_q, n_head, D))
    scale = 1.0 / 16
    limit = np.minimum(active, np.maximum(positions - origin + 1, 0))
    want_nan = np.zeros((n_q, n_head), bool)
    for i in range(n_q):
        for h in range(n_head):
            want_nan[i, h] = h // G == 1 and limit[i] > R
    split_k = xqattn.split_count(active, split_mode)
    want, wlse, _ = oracle.range_attn(q, positions, n_head, kraw, vraw, hkv, D, kv_type, origin, active, scale,
                                      split_k)
    assert np.array_equal(np.isnan(wlse), want_nan), "oracle poisoning pattern"
    case_note(f"range non-finite {wl.TYPE_NAME[kv_type]} {where} {what} split {split_mode}")
    out = torch.empty(n_q * n_head * D, dtype=torch.float32, device="cuda")
    lse = torch.empty(n_q * n_head, dtype=torch.float32, device="cuda")
    xqattn.fa_range(torch.from_numpy(q).cuda(), torch.from_numpy(positions).cuda(), n_head,
                    torch.from_numpy(kraw.reshape(-1)).cuda(), torch.from_numpy(vraw.reshape(-1)).cuda(),
                    hkv, D, kv_type, origin, active, scale, out, lse, split_mode=split_mode)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(n_q, n_head, D)
    glse = lse.cpu().numpy().reshape(n_q, n_head)
    assert np.array_equal(np.isnan(glse), want_nan), f"LSE NaN rows {np.argwhere(np.isnan(glse))}"
    assert np.all(np.isnan(got[want_nan])), "a row that sees the record is not NaN in full"
    assert np.all(np.isfinite(got[~want_nan])), "a row that does not see the record is not finite"
    assert_close(got[~want_nan], want[~want_nan], atol=3e-4, rtol=3e-4, what="finite rows O")
    assert_close(glse[~want_nan], wlse[~want_nan], atol=3e-4, rtol=3e-5, what="finite rows LSE")


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2], ids=lambda t: wl.TYPE_NAME[t])
def test_fa_masked_nonfinite_rows_never_reach_a_query(torch_gpu, kv_type, engine):
    """ggml's loop skips masked rows: NaN K/V records in rows masked for every
    query change nothing (bitwise); a NaN V record in a row only query 2 sees
    makes query 2's rows of that KV head non-finite and leaves queries 0, 1
    bitwise unchanged."""
    cfg = wl.FaConfig("masknan", 3, 16, 4, 128, 500, 2, kv_type, causal_prefix=400)
    case_note(f"masked non-finite rows {wl.TYPE_NAME[kv_type]} engine {engine}")
    case = make_fa_case(cfg, seed=61, mask_per_seq=True)
    clean, clse = run_fa_gpu(case, torch_gpu, engine=engine)
    rec = wl.record_bytes(kv_type, 128)
    k = case.k.buf.reshape(2, 500, 4, rec).copy()
    v = case.v.buf.reshape(2, 500, 4, rec).copy()
    for r in range(450, 461):
        for h in range(4):
            _spoil(k[0], kv_type, r, h, "nan")
            _spoil(v[1], kv_type, r, h, "nan")
    spoiled = dataclasses.replace(case, k=wl.kv_tensor(k, kv_type, 128), v=wl.kv_tensor(v, kv_type, 128))
    got, glse = run_fa_gpu(spoiled, torch_gpu, engine=engine)
    assert np.array_equal(got, clean) and np.array_equal(glse, clse), "masked non-finite rows changed the output"
    # row 402 is visible to query 2 only (query i sees rows <= 400 + i)
    v2 = v.copy()
    _spoil(v2[0], kv_type, 402, 1, "nan")
    spoiled2 = dataclasses.replace(spoiled, v=wl.kv_tensor(v2, kv_type, 128))
    got2, _ = run_fa_gpu(spoiled2, torch_gpu, engine=engine)
    heads1 = slice(4, 8)  # query heads of KV head 1 (GQA 4)
    assert np.array_equal(got2[:, :2], clean[:, :2]), "queries 0, 1 do not see row 402"
    assert np.array_equal(got2[1], clean[1]), "sequence 1 does not read sequence 0's cache"
    assert not np.all(np.isfinite(got2[0, 2, heads1])), "query 2 sees the NaN row"
    assert np.array_equal(got2[0, 2, :4], clean[0, 2, :4]) and np.array_equal(got2[0, 2, 8:], clean[0, 2, 8:])
    # ggml accumulates V per dim: exactly the dims the NaN element (F16, E5M2)
    # or the NaN block scale (q8_0, q4_0: dims 32..63) sits in become NaN
    want2, _ = oracle_fa(spoiled2)
    assert np.array_equal(np.isnan(got2), np.isnan(want2)), \
        f"NaN dims {np.argwhere(np.isnan(got2))[:8]} vs the oracle's {np.argwhere(np.isnan(want2))[:8]}"


def _limit_mask(L, limits):
    """f16 mask [1, n_q, L]: query i sees rows 0 .. limits[i]."""
    m = np.full((1, len(limits), L), 0xFC00, np.uint16)
    for i, lim in enumerate(limits):
        m[0, i, :lim + 1] = 0
    return m


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("what", ["nan", "inf"])
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2], ids=lambda t: wl.TYPE_NAME[t])
def test_fa_nonfinite_v_reaches_only_its_dims_whatever_the_tile(torch_gpu, kv_type, what, engine):
    """A NaN or Inf V element (F16, E5M2) or block scale (q8_0, q4_0) at row 390
    of KV head 1 makes exactly its dims non-finite, with the oracle's NaN / +-Inf
    pattern (ggml's per-dim VKQ += v * vs), in the queries that see the row.
    Query 0 sees rows up to 388 only, so with it in the call the slice of rows
    384..399 holds rows past a query's limit; query 1 (up to 449) gives the same
    bits alone, where every row of that slice is visible to it, and next to
    query 0. Query 0 stays finite and gives the same bits alone."""
    B, NQ, H, Hkv, D, L = 1, 3, 8, 2, 128, 500
    cfg = wl.FaConfig("nonfin_dims", NQ, H, Hkv, D, L, B, kv_type)
    case_note(f"non-finite V dims {wl.TYPE_NAME[kv_type]} {what} engine {engine}")
    case = make_fa_case(cfg, seed=91, mask=None)
    case.mask = wl.mask_tensor(_limit_mask(L, [388, 449, 499]))
    rec = wl.record_bytes(kv_type, D)
    v = case.v.buf.reshape(L, Hkv, rec).copy()
    _spoil(v, kv_type, 390, 1, what)
    case = dataclasses.replace(case, v=wl.kv_tensor(v.reshape(B, L, Hkv, rec), kv_type, D))
    got, _ = run_fa_gpu(case, torch_gpu, engine=engine)
    want, _ = oracle_fa(case)
    assert np.array_equal(np.isnan(got), np.isnan(want)), \
        f"NaN at {np.argwhere(np.isnan(got))[:8]}, oracle {np.argwhere(np.isnan(want))[:8]}"
    assert np.array_equal(np.isposinf(got), np.isposinf(want)) and np.array_equal(np.isneginf(got), np.isneginf(want))
    bad_dims = [5] if kv_type in (wl.F16, wl.E5M2) else list(range(32, 64))
    nonfin = ~np.isfinite(got)
    assert not nonfin[:, 0].any(), "query 0 does not see row 390"
    assert not nonfin[:, :, :4].any(), "heads of KV head 0 do not read KV head 1"
    for iq in (1, 2):
        assert np.array_equal(np.argwhere(nonfin[0, iq, 4:].any(axis=0)).ravel(), np.array(bad_dims)), \
            f"query {iq}: non-finite dims {np.argwhere(nonfin[0, iq, 4:].any(axis=0)).ravel()}"
    assert_close(got[np.isfinite(want)], want[np.isfinite(want)], what="finite elements vs restatement")
    for iq in (0, 1):
        alone, _ = run_fa_gpu(_sub_case(case, iq, 1), torch_gpu, engine=engine)
        a, b = alone[:, 0], got[:, iq]
        assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(np.isinf(a), np.isinf(b))
        fin = np.isfinite(b)
        assert np.array_equal(a[fin].view(np.uint32), b[fin].view(np.uint32)), f"query {iq} alone differs"
        assert np.array_equal(a[~fin & np.isinf(b)], b[~fin & np.isinf(b)])


# ---------------------------------------------------------------------------
# batch-composition invariance at the 32k, head-dim-256 geometry
# ---------------------------------------------------------------------------

_CASES = {}


def _cached_case(cfg, **kw):
    key = (cfg, tuple(sorted(kw.items())))
    if key not in _CASES:
        _CASES.clear()  # one full-size case in memory at a time
        _CASES[key] = make_fa_case(cfg, **kw)
    return _CASES[key]


def _sub_case(case, iq0, n, b_sel=None):
    """The same K/V with queries [iq0, iq0 + n) (and sequences b_sel) only."""
    B, NQ, H, D = case.shape
    L = case.cfg.L
    q_all = np.frombuffer(case.q.buf.tobytes(), np.float32).reshape(B, NQ, H, D)
    m_all = np.frombuffer(case.mask.buf.tobytes(), np.uint16).reshape(case.mask.ne[3], case.mask.ne[1], L)
    kv = case.k, case.v
    if b_sel is not None:
        if m_all.shape[0] == B:
            m_all = m_all[b_sel]
        rec = wl.record_bytes(case.cfg.kv_type, D)
        kv = tuple(wl.kv_tensor(t.buf.reshape(B, L, case.cfg.Hkv, rec)[b_sel].copy(), case.cfg.kv_type, D)
                   for t in kv)
        q_all = q_all[b_sel]
        B = q_all.shape[0]
    cfg = dataclasses.replace(case.cfg, n_q=n, B=B)
    return dataclasses.replace(case, cfg=cfg, q=wl.fa_q_tensor(q_all[:, iq0:iq0 + n].copy()),
                               k=kv[0], v=kv[1], mask=wl.mask_tensor(m_all[:, iq0:iq0 + n].copy()),
                               dst=wl.fa_dst_tensor(B, n, H, D))


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("kv_type", [wl.Q8_0, wl.Q4_0, wl.E5M2], ids=lambda t: wl.TYPE_NAME[t])
def test_fa_query_width_invariance_c2_geometry(torch_gpu, kv_type, engine):
    """n_q = 1, 3 and 8 give the same bits for a query at L = 32768, D = 256,
    GQA 6, B = 4 (2048-row splits: many 16-row slices per wave)."""
    cfg = wl.FaConfig("inv_c2", 8, 24, 4, 256, 32768, 4, kv_type, causal_prefix=32760)
    case_note(f"query width invariance 32k q8_0 decode geometry {wl.TYPE_NAME[kv_type]} engine {engine}")
    case = _cached_case(cfg, seed=5)
    batch, blse = run_fa_gpu(case, torch_gpu, engine=engine)
    for iq0, n in ((0, 1), (3, 1), (7, 1), (2, 3), (5, 3)):
        sub, slse = run_fa_gpu(_sub_case(case, iq0, n), torch_gpu, engine=engine)
        assert np.array_equal(sub, batch[:, iq0:iq0 + n]), f"queries {iq0}..{iq0 + n - 1} differ at n_q={n}"
        assert np.array_equal(slse, blse[:, iq0:iq0 + n])


D128_GEOMS = [
    # (name, n_head, n_head_kv, kv_len, n_seq, kv type): the 4k decode's heads
    # (GQA 2: at most 16 pairs per tile) and the verify's (GQA 4: n_q 1..4 run
    # one 16-pair tile, n_q 5..8 one 32-pair tile, another kernel variant)
    ("c1_f16", 16, 8, 4104, 1, wl.F16),
    ("c1_q8_0", 16, 8, 4104, 1, wl.Q8_0),
    ("c5_q4_0", 32, 8, 16392, 2, wl.Q4_0),
    ("c5_f16", 32, 8, 16392, 2, wl.F16),
    ("c5_e5m2", 32, 8, 16392, 2, wl.E5M2),
]


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("geom", D128_GEOMS, ids=lambda g: g[0])
def test_fa_query_width_invariance_d128(torch_gpu, geom, engine):
    """At head dim 128 the query tile holds up to 32 (query, head) pairs, so the
    tile's kernel variant can change with n_q (GQA 4: one 16-pair tile for n_q
    <= 4, a 32-pair tile above); the wave count, the slice-to-wave assignment
    and every per-pair quantity are the same in both, so n_q = 1, 3 and 8 give
    the same bits for a query."""
    name, H, Hkv, L, B, kv_type = geom
    cfg = wl.FaConfig(f"inv_{name}", 8, H, Hkv, 128, L, B, kv_type, causal_prefix=L - 8)
    case_note(f"query width invariance D128 {name} engine {engine}")
    case = _cached_case(cfg, seed=6)
    batch, blse = run_fa_gpu(case, torch_gpu, engine=engine)
    for iq0, n in ((0, 1), (4, 1), (7, 1), (2, 3), (5, 3)):
        sub, slse = run_fa_gpu(_sub_case(case, iq0, n), torch_gpu, engine=engine)
        assert np.array_equal(sub.view(np.uint32), batch[:, iq0:iq0 + n].view(np.uint32)), \
            f"queries {iq0}..{iq0 + n - 1} differ at n_q={n}"
        assert np.array_equal(slse.view(np.uint32), blse[:, iq0:iq0 + n].view(np.uint32))


@pytest.mark.parametrize("split_mode", [xqattn.SPLIT_REFERENCE, xqattn.SPLIT_BALANCED, xqattn.SPLIT_COARSE],
                         ids=["reference", "balanced", "coarse"])
@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
def test_fa_sequence_batch_invariance_length_only_split_modes(torch_gpu, engine, split_mode):
    """Under split modes that depend on the KV length only, a sequence's output
    is bitwise the same alone (B = 1) or in a batch of four (B = 4)."""
    cfg = wl.FaConfig("inv_b", 2, 24, 4, 256, 32768, 4, wl.Q8_0, causal_prefix=32766)
    case_note(f"sequence batch invariance split {split_mode} engine {engine}")
    case = _cached_case(cfg, seed=8, mask_per_seq=True)
    batch, blse = run_fa_gpu(case, torch_gpu, split_mode=split_mode, engine=engine)
    for b in (0, 2):
        alone, alse = run_fa_gpu(_sub_case(case, 0, 2, b_sel=slice(b, b + 1)), torch_gpu, split_mode=split_mode,
                                 engine=engine)
        assert np.array_equal(alone[0], batch[b]), f"sequence {b} differs between B=1 and B=4"
        assert np.array_equal(alse[0], blse[b])


# ---------------------------------------------------------------------------
# the verify configuration with padded and fully masked query rows
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
def test_fa_verify_full_size_masked_query_rows(torch_gpu, engine):
    """The q4_0 verify at full size (n_q 8, L 16392, B 8) with the mask padded to 16
    rows and queries 6 and 7 fully masked (-inf rows): those give O = 0 and
    LSE = -inf, the others match the oracle."""
    cfg = dataclasses.replace(wl.FA_C5, name="c5_masked_rows", n_q_pad=16)
    case_note(f"q4_0 verify full size masked query rows engine {engine}")
    case = make_fa_case(cfg, seed=12)
    m = wl.fa_causal_mask(cfg, n_q_rows=6)  # rows 6..15 all -inf
    case.mask = wl.mask_tensor(m)
    got, glse = run_fa_gpu(case, torch_gpu, engine=engine)
    assert np.all(got[:, 6:] == 0.0) and np.all(np.isneginf(glse[:, 6:]))
    want, wlse = oracle_fa(case)
    assert_close(got, want, what="q4_0 verify masked query rows vs ggml restatement")
    ref64, lse64 = oracle_f64(case)
    assert_close(got[:, :6], ref64[:, :6], atol=1e-4, rtol=1e-4, what="q4_0 verify vs f64")
    assert_close(glse[:, :6], lse64[:, :6], atol=1e-4, rtol=1e-5, what="q4_0 verify LSE")
