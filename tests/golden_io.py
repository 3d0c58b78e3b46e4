"""Golden fixtures under tests/golden/: loading them as ggml-shaped host tensors.

A fixture is one ``.npz`` holding the inputs of one case and the expected
outputs the oracle produced for them when ``tests/golden/make_golden.py`` ran:

* ``fa_*.npz``: FLASH_ATTN_EXT. Inputs stored as they are handed to the op
  (f32 Q rows, raw KV records, f16 mask bits, sinks); expected ``out``/``lse``
  of the ggml one-chunk loop restatement (consistent query policy, f16 V
  accumulator for F16 V) and ``out64``/``lse64`` of the float64 closed form
  (rounded to f32 for storage).
* ``range_*.npz``: range attention (positions, origin, active rows) with the
  expected OUT and LSE of pass 1 + ordered reduce at the reference split count.
* ``kv_store.npz``: F32 rows and the exact cache planes for every KV type.
* ``gdn_*.npz``: GATED_DELTA_NET. Inputs are integer codes times powers of two
  drawn from splitmix64 (integer arithmetic only, so every host regenerates the
  same bytes; the fixture keeps their sha256), expected outputs of the f32
  recurrence in the reference emulator's order (``want``) and of a float64
  recurrence (``want64``, rounded to f32), in full for the per-token outputs where small and
  for fixed (head, column) subsets of the states.
"""
from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np

from xqattn import workloads as wl
from xqattn import xfa1

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
SENTINEL = np.float32(1e30)


def fixture_paths(prefix: str):
    return sorted(GOLDEN.glob(f"{prefix}*.npz"))


def load(path) -> tuple[dict, dict]:
    with np.load(path, allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files if k != "meta"}
        meta = json.loads(str(z["meta"]))
    return meta, arrays


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---------------------------------------------------------------------------
# flash attention
# ---------------------------------------------------------------------------

def fa_tensors(meta: dict, a: dict):
    """-> (q, k, v, mask | None, sinks | None, dst) host tensors of the fixture."""
    kt, D = meta["kv_type"], meta["D"]
    q = wl.fa_q_tensor(a["q"])
    k = wl.kv_tensor(a["k"], kt, D)
    v = wl.kv_tensor(a["v"], kt, D)
    mask = wl.mask_tensor(a["mask"]) if "mask" in a else None
    sinks = wl.f32_tensor(a["sinks"], (meta["H"], 1, 1, 1)) if "sinks" in a else None
    B, NQ, H, _ = a["q"].shape
    return q, k, v, mask, sinks, wl.fa_dst_tensor(B, NQ, H, D)


def cache_view(raw: np.ndarray, typ: int, d: int, spare: int, seed: int) -> wl.HostTensor:
    """raw records [B, L, Hkv, rec] placed in a cache of L + spare rows per
    sequence (junk in the spare rows) -> the ggml view of the first L rows."""
    B, L, Hkv, rec = raw.shape
    cache = np.random.default_rng(seed).integers(0, 256, (B, L + spare, Hkv, rec), dtype=np.uint8)
    cache[:, :L] = raw
    nb = (wl.TYPE_SIZE[typ], Hkv * rec, rec, (L + spare) * Hkv * rec)
    span = xfa1.span_bytes(typ, (d, L, Hkv, B), nb)
    return wl.HostTensor(typ, (d, L, Hkv, B), nb, cache.reshape(-1)[:span].copy())


def fa_capture(path, out_dir, spare=24):
    """Write a multi-query FA fixture as an XFA1 capture, with ggml-like op ids
    and names -> (meta, arrays, (q, k, v, mask, output) host tensors, file)."""
    meta, a = load(path)
    q, k, v, m, s, dst = fa_tensors(meta, a)
    assert s is None
    kt, D = meta["kv_type"], meta["D"]
    k = cache_view(a["k"], kt, D, spare, 1)
    v = cache_view(a["v"], kt, D, spare, 2)
    out = wl.HostTensor(wl.F32, dst.ne, dst.nb, np.ascontiguousarray(a["out"]).reshape(-1).view(np.uint8))
    cap = pathlib.Path(out_dir) / f"{path.stem}.xfa1"
    xfa1.write(cap, dict(q=q, k=k, v=v, mask=m, output=out),
               ops=dict(q=34, k=33, v=33, mask=0, output=74),
               names=dict(q="q-0", k="cache_k_l3 (view)", v="cache_v_l3 (view)", mask="attn_inp_kq_mask",
                          output="__fattn__-3"))
    return meta, a, (q, k, v, m, out), cap


# ---------------------------------------------------------------------------
# gated delta net: integer-coded inputs
# ---------------------------------------------------------------------------

def int_codes(seed: int, n: int) -> np.ndarray:
    """n integers uniform in [-128, 127]: the top byte of splitmix64 outputs."""
    return (wl.splitmix64(seed, n) >> np.uint64(56)).astype(np.int64) - 128


def gdn_coded_inputs(seed: int, T: int, B: int, fine: bool = False):
    """q, k = c/1024, v = c/64, g = -(c+129)/4096 (in [-1/16, 0)), beta = (c+128)/256,
    state = c/256, each c from its own stream. Exact in f32 and in bf16.
    fine: q, k = c16/2^18 with c16 = 256 c + c' (16-bit codes, same range), exact
    in f32 but not in f16 or bf16."""
    def codes(j, shape, s):
        return (int_codes(seed + j, int(np.prod(shape))) * s).astype(np.float32).reshape(shape)
    if fine:
        def codes16(j, shape):
            n = int(np.prod(shape))
            c = int_codes(seed + j, n) * 256 + int_codes(seed + 100 + j, n) + 128
            return (c * 2.0 ** -18).astype(np.float32).reshape(shape)
        q = codes16(1, (B, T, 16, 128))
        k = codes16(2, (B, T, 16, 128))
    else:
        q = codes(1, (B, T, 16, 128), 2.0 ** -10)
        k = codes(2, (B, T, 16, 128), 2.0 ** -10)
    v = codes(3, (B, T, 32, 128), 2.0 ** -6)
    g = (-(int_codes(seed + 4, B * T * 32) + 129) * 2.0 ** -12).astype(np.float32).reshape(B, T, 32)
    beta = ((int_codes(seed + 5, B * T * 32) + 128) * 2.0 ** -8).astype(np.float32).reshape(B, T, 32)
    state = codes(6, (B, 32, 128, 128), 2.0 ** -8)
    return q, k, v, g, beta, state


def gdn_tensors(meta: dict, pad: int = 0):
    """Host tensors (q, k, v, g, beta, state, dst) of a coded GDN fixture; dst
    filled with a sentinel. Rows of q, k, v may be padded (layout only)."""
    T, B, slots, bf16 = meta["T"], meta["B"], meta["slots"], meta["bf16"]
    q, k, v, g, beta, st = gdn_coded_inputs(meta["seed"], T, B, meta.get("fine", False))
    typ = wl.BF16 if bf16 else wl.F32
    if bf16:  # the codes are exact in bf16: keep the top half of each f32
        q, k, v = ((a.view(np.uint32) >> np.uint32(16)).astype(np.uint16) for a in (q, k, v))
    hashes = {n: sha256(x) for n, x in zip(("q", "k", "v", "g", "beta", "state"), (q, k, v, g, beta, st))}
    qt = wl.padded_rows_tensor(q, typ, pad)
    kt = wl.padded_rows_tensor(k, typ, pad)
    vt = wl.padded_rows_tensor(v, typ, pad)
    gt = wl.f32_tensor(g, (1, 32, T, B))
    bt = wl.f32_tensor(beta, (1, 32, T, B))
    stt = wl.f32_tensor(st, (128, 128, 32, B))
    rows = T + slots * 128
    dst = wl.HostTensor(wl.F32, (4096, rows, B, 1), (4, 16384, 16384 * rows, 16384 * rows * B),
                        np.full(B * rows * 4096, SENTINEL, np.float32).view(np.uint8))
    return (qt, kt, vt, gt, bt, stt, dst), hashes


def gdn_select(meta: dict, out: np.ndarray):
    """The parts of a full output [B, T + slots*128, 4096] a fixture keeps:
    y rows of the kept heads [B, T, nh, 128] and the kept state columns of
    every written slot [B, n_slots, nsh, ncols, 128] (element i fastest)."""
    T, slots = meta["T"], meta["slots"]
    B = out.shape[0]
    y = out[:, :T].reshape(B, T, 32, 128)[:, :, meta["y_heads"]]
    n_slots = min(T, slots)
    st = out[:, T:T + 128 * n_slots].reshape(B, n_slots, 32, 128, 128)
    st = st[:, :, meta["state_heads"]][:, :, :, meta["state_cols"]]
    return y, st
