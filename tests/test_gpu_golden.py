"""GPU library against the committed golden fixtures (tests/golden/*.npz):
the expected outputs were written by the oracle when the fixtures were made,
so these checks need nothing but the fixtures and the C ABI.

Tolerances: attention and GDN outputs within the parity tolerance 2e-3 abs / 1e-2 rel
of the ggml-loop result and of the float64 closed form; LSE within 1e-4 abs +
1e-5 rel of float64; range attention within the reference's GPU bar
(3e-4 + 3e-4|ref| for O, 3e-4 + 3e-5|ref| for LSE); KV append bit-exact.
"""
import numpy as np
import pytest

import golden_io as gio
import xqattn
from conftest import assert_close, case_note
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu

FA = gio.fixture_paths("fa_")
RANGE = gio.fixture_paths("range_")
GDN = gio.fixture_paths("gdn_")


@pytest.mark.parametrize("engine", [xqattn.ENGINE_MFMA, xqattn.ENGINE_VALU], ids=["mfma", "valu"])
@pytest.mark.parametrize("split_mode", [xqattn.SPLIT_AUTO, xqattn.SPLIT_FINE], ids=["auto", "fine"])
@pytest.mark.parametrize("path", FA, ids=lambda p: p.stem)
def test_fa_golden(torch_gpu, path, split_mode, engine):
    torch = torch_gpu
    meta, a = gio.load(path)
    case_note(f"golden {path.stem} split {split_mode} engine {engine}")
    q, k, v, m, s, dst = gio.fa_tensors(meta, a)
    dq, dk, dv = (xqattn.DevTensor.from_host(t) for t in (q, k, v))
    dm = xqattn.DevTensor.from_host(m) if m is not None else None
    ds = xqattn.DevTensor.from_host(s) if s is not None else None
    dd = xqattn.DevTensor.empty_like_host(dst)
    lse = torch.empty(a["lse"].size, dtype=torch.float32, device="cuda")
    p = xqattn.fa_params(meta["scale"], meta["max_bias"], meta["softcap"], xqattn.QK_CONSISTENT, split_mode, engine)
    xqattn.flash_attn_ext(dq, dk, dv, dm, ds, dd, p, lse=lse)
    torch.cuda.synchronize()
    got = np.frombuffer(dd.to_host_bytes().tobytes(), np.float32).reshape(a["out"].shape)
    glse = lse.cpu().numpy().reshape(a["lse"].shape)
    assert_close(got, a["out"], what=f"{path.stem} vs ggml loop")
    assert_close(got, a["out64"], what=f"{path.stem} vs float64")
    assert_close(glse, a["lse64"], atol=1e-4, rtol=1e-5, what=f"{path.stem} LSE")


@pytest.mark.parametrize("split_mode", [xqattn.SPLIT_REFERENCE, xqattn.SPLIT_AUTO], ids=["reference", "auto"])
@pytest.mark.parametrize("path", RANGE, ids=lambda p: p.stem)
def test_range_golden(torch_gpu, path, split_mode):
    torch = torch_gpu
    meta, a = gio.load(path)
    case_note(f"golden {path.stem} split {split_mode}")
    n_q, H, D = a["out"].shape
    out = torch.empty(n_q * H * D, dtype=torch.float32, device="cuda")
    lse = torch.empty(n_q * H, dtype=torch.float32, device="cuda")
    xqattn.fa_range(torch.from_numpy(a["q"]).cuda(), torch.from_numpy(a["positions"]).cuda(), H,
                    torch.from_numpy(a["k"].reshape(-1)).cuda(), torch.from_numpy(a["v"].reshape(-1)).cuda(),
                    meta["n_head_kv"], D, meta["kv_type"], meta["origin"], meta["active"], meta["scale"],
                    out, lse, split_mode=split_mode)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy().reshape(n_q, H, D), a["out"], atol=3e-4, rtol=3e-4, what="range O")
    assert_close(lse.cpu().numpy().reshape(n_q, H), a["lse"], atol=3e-4, rtol=3e-5, what="range LSE")


def test_kv_store_golden(torch_gpu):
    torch = torch_gpu
    meta, a = gio.load(gio.GOLDEN / "kv_store.npz")
    cap, hkv, D = meta["capacity"], meta["n_head_kv"], meta["D"]
    src = torch.from_numpy(a["src"]).cuda()
    pos = torch.from_numpy(a["positions"]).cuda()
    for name in [n for n in a if n.startswith("plane_")]:
        tname, var = name[len("plane_"):].rsplit("_", 1)
        typ = {v: k for k, v in wl.TYPE_NAME.items()}[tname]
        if typ == wl.F32:
            continue  # not a KV cache type of the library
        case_note(f"golden kv_store {name}")
        dst = torch.zeros(a[name].size, dtype=torch.uint8, device="cuda")
        xqattn.kv_store(src, pos, hkv, D, typ, dst, cap, q8_variant=int(var[1:]))
        torch.cuda.synchronize()
        assert np.array_equal(dst.cpu().numpy().reshape(a[name].shape), a[name]), name


@pytest.mark.parametrize("path", GDN, ids=lambda p: p.stem)
def test_gdn_golden(torch_gpu, path):
    torch = torch_gpu
    meta, a = gio.load(path)
    (q, k, v, g, beta, st, dst), hashes = gio.gdn_tensors(meta, pad=3)
    assert hashes == meta["sha256"], "integer-coded inputs regenerate differently"
    modes = [xqattn.GDN_STEP] + ([xqattn.GDN_CHUNKED] if meta["T"] > 64 else [])
    for mode in modes:
        case_note(f"golden {path.stem} mode {mode}")
        dev = [xqattn.DevTensor.from_host(t) for t in (q, k, v, g, beta, st)]
        dd = xqattn.DevTensor.from_host(dst)
        xqattn.gated_delta_net(*dev, dd, meta["slots"], mode=mode)
        torch.cuda.synchronize()
        out = np.frombuffer(dd.to_host_bytes().tobytes(), np.float32).reshape(meta["B"], -1, 4096)
        y, s = gio.gdn_select(meta, out)
        for want, got, what in ((a["want_y"], y, "y"), (a["want_state"], s, "state")):
            assert_close(got, want, what=f"{path.stem} mode {mode} {what} vs f32 recurrence")
        assert_close(y, a["want64_y"], what=f"{path.stem} mode {mode} y vs float64")
        assert_close(s, a["want64_state"], what=f"{path.stem} mode {mode} state vs float64")
        # the reference selftest's bar: max |diff| / max |ref| <= 1e-4
        for got, want in ((y, a["want64_y"]), (s, a["want64_state"])):
            assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max(), f"{path.stem} mode {mode}"
        n_written = meta["T"] + 128 * min(meta["T"], meta["slots"])
        assert np.all(out[:, n_written:] == gio.SENTINEL), "rows past the written slots were touched"
