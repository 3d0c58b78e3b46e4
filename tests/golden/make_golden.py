"""Writes the golden fixtures of this directory from the CPU oracle.

    python tests/golden/make_golden.py        (from the repository root)

Each fixture holds a case's inputs (or, for gated delta net, the integer
recipe that regenerates them with its sha256) and the expected outputs of the
oracle. ``tests/test_cpu_golden.py`` checks that the oracle still reproduces
them bit for bit; ``tests/test_gpu_golden.py`` checks the GPU library against
them. Re-run only when a fixture is added or the oracle's semantics change on
purpose.
"""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (ROOT, ROOT / "xllama-qwen35-xbox_amd", HERE.parent):
    sys.path.insert(0, str(p))

import oracle  # noqa: E402
import golden_io as gio  # noqa: E402
from fa_cases import make_fa_case, oracle_f64, oracle_fa  # noqa: E402
from xqattn import workloads as wl  # noqa: E402

# name, config, case options
FA_CASES = [
    ("fa_decode_f16_d128", wl.FaConfig("g", 1, 8, 2, 128, 193, 1, wl.F16), {}),
    ("fa_decode_q8_0_d128", wl.FaConfig("g", 1, 8, 2, 128, 193, 1, wl.Q8_0), {}),
    ("fa_decode_q4_0_d128", wl.FaConfig("g", 1, 8, 2, 128, 193, 1, wl.Q4_0), {}),
    ("fa_decode_e5m2_d128", wl.FaConfig("g", 1, 8, 2, 128, 193, 1, wl.E5M2), {}),
    ("fa_decode_q8_0_d256_b2", wl.FaConfig("g", 1, 12, 2, 256, 100, 2, wl.Q8_0, scale=1.0 / 16), {}),
    ("fa_verify_q4_0_nq8", wl.FaConfig("g", 8, 8, 2, 128, 136, 2, wl.Q4_0, causal_prefix=128), {}),
    ("fa_features_q8_0_sinks_softcap_alibi",
     wl.FaConfig("g", 3, 4, 2, 128, 150, 1, wl.Q8_0, causal_prefix=147),
     dict(sinks=True, softcap=30.0, max_bias=8.0)),
    ("fa_verify_f16_padded_rows", wl.FaConfig("g", 5, 8, 4, 128, 70, 1, wl.F16, causal_prefix=65, n_q_pad=8), {}),
]

GDN_CASES = [
    # name, T, B, slots, bf16, kept y heads, kept state heads, kept state columns
    ("gdn_step_b2", 1, 2, 1, False, list(range(32)), [0, 5, 17, 31], list(range(0, 128, 8))),
    ("gdn_snapshots_t5", 5, 1, 3, False, list(range(32)), [3, 20], list(range(0, 128, 8))),
    ("gdn_chunked_t130_bf16", 130, 1, 1, True, [0, 13, 31], [0, 17, 31], list(range(0, 128, 4))),
    ("gdn_chunked_t136_f32_fine", 136, 1, 2, False, [2, 30], [6, 25], list(range(0, 128, 4))),
]


def save(name: str, meta: dict, arrays: dict) -> None:
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, meta=np.array(json.dumps(meta, sort_keys=True)), **arrays)
    print(f"{path.name}: {path.stat().st_size} bytes")


def fa_fixture(name, cfg, opts, seed):
    case = make_fa_case(cfg, seed=seed, **opts)  # mask rows past n_q are all -inf
    out, lse = oracle_fa(case)
    out64, lse64 = oracle_f64(case)
    B, NQ, H, D = case.shape
    rec = wl.record_bytes(cfg.kv_type, D)
    arrays = {
        "q": np.frombuffer(case.q.buf.tobytes(), np.float32).reshape(B, NQ, H, D),
        "k": case.k.buf.reshape(B, cfg.L, cfg.Hkv, rec),
        "v": case.v.buf.reshape(B, cfg.L, cfg.Hkv, rec),
        "out": out, "lse": lse, "out64": out64.astype(np.float32), "lse64": lse64.astype(np.float32),
    }
    if case.mask is not None:
        arrays["mask"] = np.frombuffer(case.mask.buf.tobytes(), np.uint16).reshape(-1, case.mask.ne[1], cfg.L)
    if case.sinks is not None:
        arrays["sinks"] = np.frombuffer(case.sinks.buf.tobytes(), np.float32).copy()
    meta = dict(kind="fa", kv_type=cfg.kv_type, D=D, H=H, Hkv=cfg.Hkv, L=cfg.L, n_q=NQ, B=B,
                scale=case.scale, softcap=case.softcap, max_bias=case.max_bias, seed=seed,
                qk_policy="consistent", v_acc="f16" if cfg.kv_type == wl.F16 else "f32")
    save(name, meta, arrays)


def range_fixture(kv_type, seed):
    n_head, hkv, D, origin, active = 8, 2, 128, 102400, 200
    kraw = oracle.quantize(kv_type, wl.normal(seed, (active, hkv, D)))
    vraw = oracle.quantize(kv_type, wl.normal(seed + 1, (active, hkv, D)))
    positions = np.array([origin + active - 1, origin - 5, origin + 100, origin + active + 100, origin],
                         np.int32)
    q = wl.normal(seed + 2, (positions.size, n_head, D))
    scale = 1.0 / 16
    split_k = int(oracle.load().xo_ref_split_k(active))
    out, lse, _ = oracle.range_attn(q, positions, n_head, kraw, vraw, hkv, D, kv_type, origin, active,
                                    scale, split_k)
    meta = dict(kind="range", kv_type=kv_type, n_head=n_head, n_head_kv=hkv, D=D, origin=origin,
                active=active, scale=scale, split_k=split_k, seed=seed)
    save(f"range_{wl.TYPE_NAME[kv_type]}", meta,
         dict(q=q, positions=positions, k=kraw, v=vraw, out=out, lse=lse))


def kv_store_fixture(seed):
    n_tok, hkv, D, cap = 21, 2, 128, 32
    x = wl.normal(seed, (n_tok, hkv, D)) * np.float32(3.0)
    x[0, 0, :6] = [0.0, -0.0, 65504.0, 1e-8, -7.5, 70000.0]
    x[1, 1, :] = 0.0
    x[2, 0, 32:64] = 1e-30
    pos = np.array([(5 * i + 3) % cap for i in range(n_tok)], np.int32)
    pos[-1] = cap + 5  # outside the cache: skipped
    arrays = dict(src=x, positions=pos)
    for typ, variants in ((wl.F32, (0,)), (wl.F16, (0,)), (wl.BF16, (0,)), (wl.E5M2, (0,)), (wl.Q8_0, (0, 1)),
                          (wl.Q4_0, (0,))):
        for var in variants:
            want = np.zeros((cap, hkv, wl.record_bytes(typ, D)), np.uint8)
            oracle.kv_store(x, pos, hkv, D, typ, want, cap, var)
            arrays[f"plane_{wl.TYPE_NAME[typ]}_v{var}"] = want
    save("kv_store", dict(kind="kv_store", n_head_kv=hkv, D=D, capacity=cap, seed=seed), arrays)


def gdn_fixture(name, T, B, slots, bf16, y_heads, st_heads, st_cols, seed):
    fine = name.endswith("_fine")
    meta = dict(kind="gdn", T=T, B=B, slots=slots, bf16=bf16, seed=seed, y_heads=y_heads,
                state_heads=st_heads, state_cols=st_cols, fine=fine,
                recipe=("q,k = c16/2^18" if fine else "q,k = c/1024") +
                ", v = c/64, g = -(c+129)/4096, beta = (c+128)/256, state = c/256")
    (q, k, v, g, beta, st, dst), hashes = gio.gdn_tensors(meta)
    meta["sha256"] = hashes
    oracle.gated_delta_net(q, k, v, g, beta, st, dst, slots, 8)
    out = np.frombuffer(dst.buf.tobytes(), np.float32).reshape(B, -1, 4096)
    out64 = oracle.gated_delta_net_f64(q, k, v, g, beta, st, slots, 8)
    y, s = gio.gdn_select(meta, out)
    y64, s64 = gio.gdn_select(meta, out64)
    save(name, meta, dict(want_y=y, want_state=s, want64_y=y64.astype(np.float32),
                          want64_state=s64.astype(np.float32)))


def main():
    oracle.build(with_ref=False)
    for i, (name, cfg, opts) in enumerate(FA_CASES):
        fa_fixture(name, cfg, opts, seed=500 + 10 * i)
    range_fixture(wl.Q8_0, 700)
    range_fixture(wl.Q4_0, 710)
    kv_store_fixture(800)
    for i, (name, T, B, slots, bf16, yh, sh, sc) in enumerate(GDN_CASES):
        gdn_fixture(name, T, B, slots, bf16, yh, sh, sc, seed=900 + 10 * i)


if __name__ == "__main__":
    main()
