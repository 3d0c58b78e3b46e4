"""The oracle against the committed golden fixtures (tests/golden/*.npz).

Each fixture was written by tests/golden/make_golden.py. Here the oracle is
re-run on the stored inputs and must reproduce the stored outputs bit for bit
(the ggml-loop restatement and the quantizers are deterministic C, row-parallel
only), and the stored outputs must agree with the stored float64 closed form
within the tolerance the GPU is held to, so a fixture cannot drift silently.
"""
import numpy as np
import pytest

import golden_io as gio
import oracle
from conftest import assert_close
from xqattn import workloads as wl

FA = gio.fixture_paths("fa_")
RANGE = gio.fixture_paths("range_")
GDN = gio.fixture_paths("gdn_")


def test_fixture_set_present():
    names = {p.stem for p in gio.GOLDEN.glob("*.npz")}
    assert len(FA) >= 8 and len(RANGE) >= 2 and len(GDN) >= 3 and "kv_store" in names


@pytest.mark.parametrize("path", FA, ids=lambda p: p.stem)
def test_fa_fixture_oracle_bit_exact(path):
    meta, a = gio.load(path)
    q, k, v, m, s, dst = gio.fa_tensors(meta, a)
    lse = oracle.flash_attn_ext(q, k, v, m, s, dst, meta["scale"], meta["max_bias"], meta["softcap"],
                                oracle.QK_CONSISTENT, True, 8)
    out = np.frombuffer(dst.buf.tobytes(), np.float32).reshape(a["out"].shape)
    assert np.array_equal(out, a["out"]), "ggml-loop restatement changed"
    assert np.array_equal(lse, a["lse"])
    out64, lse64 = oracle.flash_attn_f64(q, k, v, m, s, meta["scale"], meta["max_bias"], meta["softcap"],
                                         oracle.QK_CONSISTENT, True, 8)
    assert np.array_equal(out64.astype(np.float32), a["out64"])
    assert np.array_equal(lse64.astype(np.float32), a["lse64"])
    # the stored ggml-loop result and the closed form agree to the parity tolerance
    assert_close(a["out"], a["out64"], what=f"{path.stem}: ggml loop vs float64")


@pytest.mark.parametrize("path", FA, ids=lambda p: p.stem)
def test_fa_fixture_records_decode_as_stored_type(path):
    """The stored KV records are what the oracle's quantizer writes for the
    dequantised values (a re-quantisation round trip is the identity)."""
    meta, a = gio.load(path)
    kt, D = meta["kv_type"], meta["D"]
    for name in ("k", "v"):
        raw = a[name]
        x = oracle.dequant(kt, raw, D)
        if kt in (wl.F16, wl.E5M2):
            assert np.array_equal(oracle.quantize(kt, x), raw), name
        else:  # block formats: d and the codes survive, up to the all-zero-block case
            again = oracle.quantize(kt, x, 1 if kt == wl.Q8_0 else 0)
            assert np.array_equal(oracle.dequant(kt, again, D), x), name


@pytest.mark.parametrize("path", RANGE, ids=lambda p: p.stem)
def test_range_fixture_oracle_bit_exact(path):
    meta, a = gio.load(path)
    assert int(oracle.load().xo_ref_split_k(meta["active"])) == meta["split_k"]
    out, lse, _ = oracle.range_attn(a["q"], a["positions"], meta["n_head"], a["k"], a["v"],
                                    meta["n_head_kv"], meta["D"], meta["kv_type"], meta["origin"],
                                    meta["active"], meta["scale"], meta["split_k"])
    assert np.array_equal(out, a["out"]) and np.array_equal(lse, a["lse"])
    # query 1 sits before the origin: empty range
    assert np.all(a["out"][1] == 0) and np.all(np.isneginf(a["lse"][1]))


def test_kv_store_fixture_oracle_bit_exact():
    meta, a = gio.load(gio.GOLDEN / "kv_store.npz")
    planes = [n for n in a if n.startswith("plane_")]
    assert len(planes) == 7
    for name in planes:
        tname, var = name[len("plane_"):].rsplit("_", 1)
        typ = {v: k for k, v in wl.TYPE_NAME.items()}[tname]
        want = np.zeros_like(a[name])
        oracle.kv_store(a["src"], a["positions"], meta["n_head_kv"], meta["D"], typ, want,
                        meta["capacity"], int(var[1:]))
        assert np.array_equal(want, a[name]), name
        untouched = np.setdiff1d(np.arange(meta["capacity"]), a["positions"])
        assert np.all(a[name][untouched] == 0), f"{name}: rows without a token were written"


@pytest.mark.parametrize("path", GDN, ids=lambda p: p.stem)
def test_gdn_fixture_oracle_bit_exact(path):
    meta, a = gio.load(path)
    (q, k, v, g, beta, st, dst), hashes = gio.gdn_tensors(meta)
    assert hashes == meta["sha256"], "integer-coded inputs regenerate differently"
    oracle.gated_delta_net(q, k, v, g, beta, st, dst, meta["slots"], 8)
    out = np.frombuffer(dst.buf.tobytes(), np.float32).reshape(meta["B"], -1, 4096)
    y, s = gio.gdn_select(meta, out)
    assert np.array_equal(y, a["want_y"]) and np.array_equal(s, a["want_state"])
    assert_close(a["want_y"], a["want64_y"], what=f"{path.stem} y: f32 recurrence vs float64")
    assert_close(a["want_state"], a["want64_state"], what=f"{path.stem} state: f32 vs float64")


def test_gdn_coded_inputs_are_exact_in_bf16():
    q, k, v, g, beta, st = gio.gdn_coded_inputs(901, 3, 1)
    for x in (q, k, v):
        assert np.all((x.view(np.uint32) & np.uint32(0xFFFF)) == 0)
    assert np.all(g < 0) and np.all(g >= -1 / 16) and np.all((beta >= 0) & (beta < 1))
