"""CPU oracle bindings — TEST INFRASTRUCTURE ONLY.

ctypes front-end over ``oracle/_build/libxqoracle.so`` (a plain-C restatement of
the reference's ggml CPU semantics, see ``xq_oracle.h``). Only ``tests/``, the
smoke check and the benchmark's CPU-baseline leg import this module, and only to
check or time the CPU path; the product library never calls it.

``load_ref()`` gives the reference's own header-only codec / split-policy
functions compiled from the reference checkout into ``oracle/_ref`` (present only
where that checkout was available at build time).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = _DIR / "_build" / "libxqoracle.so"
REF_PATH = _DIR / "_ref" / "libxqref.so"
REFERENCE = pathlib.Path(os.environ.get("XQ_REFERENCE", "/root/reference"))

F32, F16, Q4_0, Q8_0, BF16, E5M2 = 0, 1, 2, 8, 30, 0x100
QK_CONSISTENT, QK_NATIVE = 0, 1


class XqTensor(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
        ("data", ctypes.c_void_p),
    ]


def build(with_ref: bool | None = None) -> None:
    """Compile the oracle (and the reference shim when the checkout exists)."""
    subprocess.run(["make", "-s", "-C", str(_DIR), "all"], check=True)
    if with_ref is None:
        with_ref = (REFERENCE / "uwp" / "rkva" / "rkva-kvarn-bulk.h").exists()
    if with_ref:
        subprocess.run(["make", "-s", "-C", str(_DIR), "ref", f"REFERENCE={REFERENCE}"], check=True)


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"oracle library not built: {LIB_PATH} (run oracle.build())")
    lib = ctypes.CDLL(str(LIB_PATH))
    P = ctypes.c_void_p
    T = ctypes.POINTER(XqTensor)
    i32, i64, u32, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_float
    sig = {
        "xo_f32_to_f16": (ctypes.c_uint16, [f32]),
        "xo_f16_to_f32": (f32, [ctypes.c_uint16]),
        "xo_f32_to_bf16": (ctypes.c_uint16, [f32]),
        "xo_f16_to_e5m2": (ctypes.c_uint8, [ctypes.c_uint16]),
        "xo_f32_to_f16_row": (None, [P, P, i64]),
        "xo_f16_to_f32_row": (None, [P, P, i64]),
        "xo_f32_to_bf16_row": (None, [P, P, i64]),
        "xo_bf16_to_f32_row": (None, [P, P, i64]),
        "xo_f32_to_e5m2_row": (None, [P, P, i64]),
        "xo_quantize_row_q8_0": (None, [P, P, i64, ctypes.c_int]),
        "xo_quantize_row_q4_0": (None, [P, P, i64]),
        "xo_dequant_row": (None, [ctypes.c_int, P, P, i64]),
        "xo_row_bytes": (ctypes.c_size_t, [ctypes.c_int, i64]),
        "xo_flash_attn_ext": (ctypes.c_int, [T, T, T, T, T, T, P, f32, f32, f32, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
        "xo_flash_attn_f64": (ctypes.c_int, [T, T, T, T, T, P, P, f32, f32, f32, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
        "xo_alibi_slope": (f32, [f32, ctypes.c_int, ctypes.c_int]),
        "xo_ref_split_k": (i32, [u32]),
        "xo_opt_split_k": (i32, [u32, u32]),
        "xo_split_rows": (u32, [u32, u32]),
        "xo_q4_mq_split": (None, [u32, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]),
        "xo_range_attn_partials": (ctypes.c_int, [P, P, i32, i32, P, P, i32, i32, i32, i32, i32, f32, i32, P]),
        "xo_range_reduce": (ctypes.c_int, [P, i32, i32, i32, i32, P, P]),
        "xo_lse_merge": (ctypes.c_int, [P, P, i32, ctypes.c_int64, i32, P, P]),
        "xo_gated_delta_net": (ctypes.c_int, [T, T, T, T, T, T, T, i32, ctypes.c_int]),
        "xo_gated_delta_net_f64": (ctypes.c_int, [T, T, T, T, T, T, P, i32, ctypes.c_int]),
        "xo_kv_store": (ctypes.c_int, [P, P, i32, i32, i32, i32, i32, P, i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


_ref = None


def load_ref():
    """The compiled reference shim, or None when it was not built here."""
    global _ref
    if _ref is not None:
        return _ref
    if not REF_PATH.exists():
        return None
    lib = ctypes.CDLL(str(REF_PATH))
    u32 = ctypes.c_uint32
    lib.xr_f32_to_f16.restype, lib.xr_f32_to_f16.argtypes = ctypes.c_uint16, [ctypes.c_float]
    lib.xr_f16_to_f32.restype, lib.xr_f16_to_f32.argtypes = ctypes.c_float, [ctypes.c_uint16]
    lib.xr_f16_to_e5m2.restype, lib.xr_f16_to_e5m2.argtypes = ctypes.c_uint8, [ctypes.c_uint16]
    lib.xr_e5m2_to_f16.restype, lib.xr_e5m2_to_f16.argtypes = ctypes.c_uint16, [ctypes.c_uint8]
    lib.xr_reference_split_k.restype, lib.xr_reference_split_k.argtypes = u32, [u32]
    lib.xr_optimized_split_k.restype, lib.xr_optimized_split_k.argtypes = u32, [u32, u32]
    lib.xr_split_rows.restype, lib.xr_split_rows.argtypes = u32, [u32, u32]
    lib.xr_q4_mq_split.restype = None
    lib.xr_q4_mq_split.argtypes = [u32, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]
    _ref = lib
    return lib


# ---------------------------------------------------------------------------
# numpy conveniences
# ---------------------------------------------------------------------------

def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def desc(t) -> XqTensor:
    """XqTensor for an object with .type/.ne/.nb/.buf (host numpy buffer)."""
    if t is None:
        return None
    d = XqTensor()
    d.type = int(t.type)
    for i in range(4):
        d.ne[i] = int(t.ne[i])
        d.nb[i] = int(t.nb[i])
    d.data = _ptr(t.buf)
    return d


def _ref_or_none(d):
    return ctypes.byref(d) if d is not None else None


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    load().xo_f32_to_f16_row(_ptr(x), _ptr(y), x.size)
    return y


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    load().xo_f16_to_f32_row(_ptr(h), _ptr(y), h.size)
    return y


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    load().xo_f32_to_bf16_row(_ptr(x), _ptr(y), x.size)
    return y


def f32_to_e5m2(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint8)
    load().xo_f32_to_e5m2_row(_ptr(x), _ptr(y), x.size)
    return y


def row_bytes(typ: int, k: int) -> int:
    return int(load().xo_row_bytes(typ, k))


def quantize(typ: int, x: np.ndarray, q8_variant: int = 0) -> np.ndarray:
    """Rows of x (last axis = elements) -> raw bytes [..., row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    rb = row_bytes(typ, k)
    out = np.empty(x.shape[:-1] + (rb,), np.uint8)
    n_rows = x.size // k
    lib = load()
    if typ == Q8_0:
        lib.xo_quantize_row_q8_0(_ptr(x), _ptr(out), x.size, q8_variant)
    elif typ == Q4_0:
        lib.xo_quantize_row_q4_0(_ptr(x), _ptr(out), x.size)
    elif typ == F16:
        lib.xo_f32_to_f16_row(_ptr(x), _ptr(out), x.size)
    elif typ == BF16:
        lib.xo_f32_to_bf16_row(_ptr(x), _ptr(out), x.size)
    elif typ == E5M2:
        lib.xo_f32_to_e5m2_row(_ptr(x), _ptr(out), x.size)
    elif typ == F32:
        out = x.view(np.uint8).reshape(x.shape[:-1] + (rb,)).copy()
    else:
        raise ValueError(typ)
    assert out.size == n_rows * rb
    return out


def dequant(typ: int, raw: np.ndarray, k: int) -> np.ndarray:
    """Raw rows [..., row_bytes] -> float32 [..., k]."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    rb = row_bytes(typ, k)
    lead = raw.shape[:-1]
    assert raw.shape[-1] == rb
    y = np.empty(lead + (k,), np.float32)
    n_rows = int(np.prod(lead)) if lead else 1
    load().xo_dequant_row(typ, _ptr(raw), _ptr(y), n_rows * k)
    return y


def flash_attn_ext(q, k, v, mask, sinks, dst, scale, max_bias=0.0, softcap=0.0,
                   policy=QK_CONSISTENT, v_acc_f16=True, n_threads=8, want_lse=True):
    """Run the ggml-CPU restatement; fills dst.buf, returns lse [B, n_q, H] or None."""
    dq, dk, dv, dd = desc(q), desc(k), desc(v), desc(dst)
    dm, ds = desc(mask), desc(sinks)
    B, NQ, H = q.ne[3], q.ne[1], q.ne[2]
    lse = np.empty((B, NQ, H), np.float32) if want_lse else None
    rc = load().xo_flash_attn_ext(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv),
                                  _ref_or_none(dm), _ref_or_none(ds), ctypes.byref(dd),
                                  _ptr(lse) if lse is not None else None,
                                  scale, max_bias, softcap, policy, int(v_acc_f16), n_threads)
    if rc:
        raise ValueError("oracle flash_attn_ext rejected the shapes")
    return lse


def flash_attn_f64(q, k, v, mask, sinks, scale, max_bias=0.0, softcap=0.0,
                   policy=QK_CONSISTENT, q_round=True, n_threads=8):
    """float64 closed form: returns (out [B, n_q, H, D], lse [B, n_q, H])."""
    B, NQ, H, D = q.ne[3], q.ne[1], q.ne[2], v.ne[0]
    out = np.empty((B, NQ, H, D), np.float64)
    lse = np.empty((B, NQ, H), np.float64)
    dq, dk, dv = desc(q), desc(k), desc(v)
    dm, ds = desc(mask), desc(sinks)
    rc = load().xo_flash_attn_f64(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv),
                                  _ref_or_none(dm), _ref_or_none(ds), _ptr(out), _ptr(lse),
                                  scale, max_bias, softcap, policy, int(q_round), n_threads)
    if rc:
        raise ValueError("oracle flash_attn_f64 rejected the shapes")
    return out, lse


def gated_delta_net(q, k, v, g, beta, state, dst, slots, n_threads=8):
    ds = [desc(t) for t in (q, k, v, g, beta, state, dst)]
    rc = load().xo_gated_delta_net(*[ctypes.byref(d) for d in ds], slots, n_threads)
    if rc:
        raise ValueError("oracle gated_delta_net rejected the shapes")


def gated_delta_net_f64(q, k, v, g, beta, state, slots, n_threads=8):
    T, B = v.ne[2], v.ne[3]
    out = np.empty((B, T + slots * 128, 4096), np.float64)
    ds = [desc(t) for t in (q, k, v, g, beta, state)]
    rc = load().xo_gated_delta_net_f64(*[ctypes.byref(d) for d in ds], _ptr(out), slots, n_threads)
    if rc:
        raise ValueError("oracle gated_delta_net_f64 rejected the shapes")
    return out


def range_attn(q, positions, n_head, k, v, n_head_kv, head_dim, kv_type, origin, active,
               kq_scale, split_k, poison=True):
    """RKVA range attention pass 1 + reduce: returns (out [n_q, H, D], lse [n_q, H])."""
    q = np.ascontiguousarray(q, np.float32)
    positions = np.ascontiguousarray(positions, np.int32)
    n_q = positions.size
    parts = np.empty((split_k, n_q * n_head, head_dim + 2), np.float32)
    lib = load()
    rc = lib.xo_range_attn_partials(_ptr(q), _ptr(positions), n_q, n_head, _ptr(k), _ptr(v),
                                    n_head_kv, head_dim, kv_type, origin, active, kq_scale,
                                    split_k, _ptr(parts))
    if rc:
        raise ValueError("oracle range_attn rejected the shapes")
    out = np.empty((n_q * n_head, head_dim), np.float32)
    lse = np.empty((n_q * n_head,), np.float32)
    lib.xo_range_reduce(_ptr(parts), n_q * n_head, head_dim, split_k, int(poison), _ptr(out), _ptr(lse))
    return out.reshape(n_q, n_head, head_dim), lse.reshape(n_q, n_head), parts


def range_reduce(parts: np.ndarray, head_dim: int, poison: bool):
    parts = np.ascontiguousarray(parts, np.float32)
    split_k, n_qh = parts.shape[0], parts.shape[1]
    out = np.empty((n_qh, head_dim), np.float32)
    lse = np.empty((n_qh,), np.float32)
    load().xo_range_reduce(_ptr(parts), n_qh, head_dim, split_k, int(poison), _ptr(out), _ptr(lse))
    return out, lse


def lse_merge(parts_out: np.ndarray, parts_lse: np.ndarray):
    """parts_out [n_parts, rows, D], parts_lse [n_parts, rows] -> (out [rows, D], lse [rows])."""
    parts_out = np.ascontiguousarray(parts_out, np.float32)
    parts_lse = np.ascontiguousarray(parts_lse, np.float32)
    n_parts, rows, D = parts_out.shape
    assert parts_lse.shape == (n_parts, rows)
    out = np.empty((rows, D), np.float32)
    lse = np.empty((rows,), np.float32)
    load().xo_lse_merge(_ptr(parts_out), _ptr(parts_lse), n_parts, rows, D, _ptr(out), _ptr(lse))
    return out, lse


def kv_store(src, positions, n_head_kv, head_dim, kv_type, dst, capacity, q8_variant=0):
    src = np.ascontiguousarray(src, np.float32)
    positions = np.ascontiguousarray(positions, np.int32)
    rc = load().xo_kv_store(_ptr(src), _ptr(positions), positions.size, n_head_kv, head_dim,
                            kv_type, q8_variant, _ptr(dst), capacity)
    if rc:
        raise ValueError("oracle kv_store rejected the type")
