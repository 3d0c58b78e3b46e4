"""Host binding of the MI355X attention + gated-delta-net library (libxqattn.so).

A thin ctypes layer over the C ABI in ``include/xq_attn.h``: it builds ggml-style
tensor descriptors (type, ne, nb, data) over torch device tensors, sizes and
hands over workspaces, passes torch's current HIP stream, and raises
``XqError`` with the library's message on any non-OK status. torch is used only
for device memory and streams; all compute runs in the library's gfx950
kernels. There is no fallback: if the library is missing, importing the
functions below fails loudly.

Mirrors the ggml op interface of the reference path:
  ``flash_attn_ext``   GGML_OP_FLASH_ATTN_EXT (ggml-cpu ops.cpp as patched by
                       patches/0006-… and patches/0008-…)
  ``fa_range``         RemoteAttnEngine::attend_range (uwp/rkva/remote-attn-engine.h:152-154)
  ``gated_delta_net``  GGML_OP_GATED_DELTA_NET (src/bridge/ggml_d3d12.cpp:77-158,1905-1942)
  ``kv_store``         KV append (shaders/rkva/rkva_store_f16.hlsl:63-85, all KV types)
"""
from __future__ import annotations

import ctypes
import dataclasses
import pathlib

from .workloads import (BF16, E5M2, F16, F32, Q4_0, Q8_0, TYPE_SIZE, HostTensor,  # noqa: F401
                        record_bytes)

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libxqattn.so"

XQ_OK = 0
STATUS = {0: "OK", 1: "UNSUPPORTED", 2: "BAD_SHAPE", 3: "BAD_ARG", 4: "WORKSPACE", 5: "HIP"}

QK_CONSISTENT, QK_NATIVE = 0, 1
SPLIT_AUTO, SPLIT_REFERENCE, SPLIT_BALANCED, SPLIT_FINE, SPLIT_COARSE, SPLIT_NONE = range(6)
SPLIT_MQ_BALANCED, SPLIT_MQ_FINE, SPLIT_LENGTH = 6, 7, 8
GDN_AUTO, GDN_STEP, GDN_CHUNKED = 0, 1, 2
ENGINE_AUTO, ENGINE_MFMA, ENGINE_VALU = 0, 1, 2

EXPORTS = (
    "xq_supports_flash_attn_ext", "xq_flash_attn_ext_workspace", "xq_flash_attn_ext",
    "xq_flash_attn_ext_noalloc",
    "xq_fa_range_workspace", "xq_fa_range", "xq_fa_lse_merge", "xq_fa_split_count", "xq_fa_split_rows",
    "xq_fa_params_from_env",
    "xq_supports_gated_delta_net", "xq_gated_delta_net_workspace", "xq_gated_delta_net",
    "xq_kv_store", "xq_kv_record_bytes", "xq_last_error", "xq_abi_version",
    "xq_profile_enable", "xq_profile_reset", "xq_profile_read",
    "xq_ggml_backend_init", "xq_ggml_backend_free", "xq_ggml_backend_name", "xq_ggml_backend_stream",
    "xq_ggml_backend_workspace_bytes", "xq_ggml_supports_op", "xq_ggml_supports_op_params",
    "xq_ggml_graph_compute",
)


class XqError(RuntimeError):
    def __init__(self, status: int, what: str, msg: str):
        super().__init__(f"{what}: {STATUS.get(status, status)}: {msg}")
        self.status = status


class XqTensor(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
        ("data", ctypes.c_void_p),
    ]


class XqFaParams(ctypes.Structure):
    _fields_ = [
        ("scale", ctypes.c_float),
        ("max_bias", ctypes.c_float),
        ("logit_softcap", ctypes.c_float),
        ("qk_policy", ctypes.c_int32),
        ("split_mode", ctypes.c_int32),
        ("engine", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 2),
    ]


GGML_MAX_SRC, GGML_MAX_OP_PARAMS, GGML_FLAG_COMPUTE = 10, 16, 1
OP_NOOP, OP_FLASH_ATTN_EXT, OP_GATED_DELTA_NET, OP_OTHER = 0, 1, 2, 3


class XqGgmlNode(ctypes.Structure):
    """xq_ggml_node: one ggml graph node as a backend binding copies it out."""
    _fields_ = [
        ("op", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("op_params", ctypes.c_int32 * GGML_MAX_OP_PARAMS),
        ("dst", XqTensor),
        ("src", ctypes.POINTER(XqTensor) * GGML_MAX_SRC),
    ]


class XqGgmlBackendParams(ctypes.Structure):
    _fields_ = [
        ("fa_qk_policy", ctypes.c_int32),
        ("fa_split_mode", ctypes.c_int32),
        ("fa_engine", ctypes.c_int32),
        ("gdn_mode", ctypes.c_int32),
        ("gdn_min_tokens", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 3),
    ]


_lib = None


def load() -> ctypes.CDLL:
    """Load libxqattn.so (built by ``xqattn.build``); raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(LIB_PATH))
    T = ctypes.POINTER(XqTensor)
    P = ctypes.c_void_p
    i32, i64, f32, sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
    FP = ctypes.POINTER(XqFaParams)
    sig = {
        "xq_supports_flash_attn_ext": (ctypes.c_int, [T, T, T, T, T, T, FP]),
        "xq_flash_attn_ext_workspace": (i32, [T, T, T, T, T, T, FP, ctypes.POINTER(sz)]),
        "xq_flash_attn_ext": (i32, [T, T, T, T, T, T, P, FP, P, sz, P]),
        "xq_flash_attn_ext_noalloc": (i32, [T, T, T, T, T, T, P, FP, P]),
        "xq_fa_range_workspace": (i32, [i32, i32, i32, i32, i32, i32, i32, ctypes.POINTER(sz)]),
        "xq_fa_range": (i32, [P, P, i32, i32, P, P, i32, i32, i32, i32, i32, f32, i32, P, P, P, sz, P]),
        "xq_fa_lse_merge": (i32, [P, P, i32, i64, i32, P, P, P]),
        "xq_fa_split_count": (i32, [i64, i32]),
        "xq_fa_split_rows": (i64, [i64, i32]),
        "xq_fa_params_from_env": (i32, [FP]),
        "xq_supports_gated_delta_net": (ctypes.c_int, [T, T, T, T, T, T, T, i32, i32]),
        "xq_gated_delta_net_workspace": (i32, [T, T, i32, i32, ctypes.POINTER(sz)]),
        "xq_gated_delta_net": (i32, [T, T, T, T, T, T, T, i32, i32, i32, P, sz, P]),
        "xq_kv_store": (i32, [P, P, i32, i32, i32, i32, i32, P, i32, P]),
        "xq_kv_record_bytes": (sz, [i32, i32]),
        "xq_last_error": (ctypes.c_char_p, []),
        "xq_abi_version": (i32, []),
        "xq_profile_enable": (None, [i32]),
        "xq_profile_reset": (None, []),
        "xq_profile_read": (i32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_int64), i32]),
        "xq_ggml_backend_init": (P, [i32, ctypes.POINTER(XqGgmlBackendParams)]),
        "xq_ggml_backend_free": (None, [P]),
        "xq_ggml_backend_name": (ctypes.c_char_p, [P]),
        "xq_ggml_backend_stream": (P, [P]),
        "xq_ggml_backend_workspace_bytes": (sz, [P]),
        "xq_ggml_supports_op": (ctypes.c_int, [ctypes.POINTER(XqGgmlNode)]),
        "xq_ggml_supports_op_params": (ctypes.c_int, [ctypes.POINTER(XqGgmlNode), ctypes.POINTER(XqGgmlBackendParams)]),
        "xq_ggml_graph_compute": (i32, [P, ctypes.POINTER(XqGgmlNode), i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(st: int, what: str):
    if st != XQ_OK:
        raise XqError(st, what, load().xq_last_error().decode())


# ---------------------------------------------------------------------------
# device tensors
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class DevTensor:
    """A ggml-shaped tensor over a torch device buffer (any dtype; bytes matter)."""
    type: int
    ne: tuple
    nb: tuple
    t: "object"  # torch.Tensor holding the bytes

    def desc(self) -> XqTensor:
        d = XqTensor()
        d.type = int(self.type)
        for i in range(4):
            d.ne[i] = int(self.ne[i])
            d.nb[i] = int(self.nb[i])
        d.data = self.t.data_ptr()
        return d

    @classmethod
    def from_host(cls, h: HostTensor, device="cuda"):
        import torch
        t = torch.from_numpy(h.buf.reshape(-1).view("uint8").copy()).to(device)
        return cls(h.type, tuple(h.ne), tuple(h.nb), t)

    @classmethod
    def empty_like_host(cls, h: HostTensor, device="cuda"):
        import torch
        return cls(h.type, tuple(h.ne), tuple(h.nb), torch.zeros(h.buf.nbytes, dtype=torch.uint8, device=device))

    def to_host_bytes(self):
        return self.t.reshape(-1).view(__import__("torch").uint8).cpu().numpy()


def _d(x):
    return ctypes.byref(x.desc()) if x is not None else None


def _keep(*xs):
    return [x.desc() if x is not None else None for x in xs]


def _stream(stream):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _workspace(nbytes: int, ws=None):
    import torch
    if nbytes == 0:
        return None
    if ws is not None and ws.numel() * ws.element_size() >= nbytes:
        return ws
    return torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")


def _aligned_ptr(ws):
    if ws is None:
        return None, 0
    p = ws.data_ptr()
    off = (-p) % 256
    return p + off, ws.numel() * ws.element_size() - off


# ---------------------------------------------------------------------------
# flash attention
# ---------------------------------------------------------------------------

def fa_params(scale, max_bias=0.0, softcap=0.0, qk_policy=QK_CONSISTENT, split_mode=SPLIT_AUTO,
              engine=ENGINE_AUTO):
    p = XqFaParams()
    p.scale, p.max_bias, p.logit_softcap = scale, max_bias, softcap
    p.qk_policy, p.split_mode, p.engine = qk_policy, split_mode, engine
    return p


def supports_flash_attn_ext(q, k, v, mask, sinks, dst, params) -> bool:
    ds = _keep(q, k, v, mask, sinks, dst)
    refs = [ctypes.byref(x) if x is not None else None for x in ds]
    return bool(load().xq_supports_flash_attn_ext(*refs, ctypes.byref(params)))


def flash_attn_ext_workspace(q, k, v, mask, sinks, dst, params) -> int:
    ds = _keep(q, k, v, mask, sinks, dst)
    refs = [ctypes.byref(x) if x is not None else None for x in ds]
    n = ctypes.c_size_t(0)
    _check(load().xq_flash_attn_ext_workspace(*refs, ctypes.byref(params), ctypes.byref(n)),
           "flash_attn_ext_workspace")
    return n.value + 256


def flash_attn_ext(q: DevTensor, k: DevTensor, v: DevTensor, mask, sinks, dst: DevTensor,
                   params: XqFaParams, lse=None, workspace=None, stream=None):
    """GGML_OP_FLASH_ATTN_EXT into dst (and the optional LSE tensor)."""
    ws = _workspace(flash_attn_ext_workspace(q, k, v, mask, sinks, dst, params), workspace)
    wp, wn = _aligned_ptr(ws)
    ds = _keep(q, k, v, mask, sinks, dst)
    refs = [ctypes.byref(x) if x is not None else None for x in ds]
    _check(load().xq_flash_attn_ext(*refs, ctypes.c_void_p(lse.data_ptr()) if lse is not None else None,
                                    ctypes.byref(params), ctypes.c_void_p(wp), wn, _stream(stream)),
           "flash_attn_ext")
    return ws


def flash_attn_ext_noalloc(q: DevTensor, k: DevTensor, v: DevTensor, mask, sinks, dst: DevTensor,
                           params: XqFaParams, lse=None, stream=None):
    """GGML_OP_FLASH_ATTN_EXT with the library's per-GPU scratch as workspace
    (no allocation on any path)."""
    ds = _keep(q, k, v, mask, sinks, dst)
    refs = [ctypes.byref(x) if x is not None else None for x in ds]
    _check(load().xq_flash_attn_ext_noalloc(*refs, ctypes.c_void_p(lse.data_ptr()) if lse is not None else None,
                                            ctypes.byref(params), _stream(stream)), "flash_attn_ext_noalloc")


def fa_range(q, positions, n_head, k, v, n_head_kv, head_dim, kv_type, origin, active, kq_scale,
             out, lse, split_mode=SPLIT_AUTO, workspace=None, stream=None):
    lib = load()
    n_q = positions.numel()
    n = ctypes.c_size_t(0)
    _check(lib.xq_fa_range_workspace(n_q, n_head, n_head_kv, head_dim, kv_type, active, split_mode,
                                     ctypes.byref(n)), "fa_range_workspace")
    ws = _workspace(n.value + 256, workspace)
    wp, wn = _aligned_ptr(ws)
    _check(lib.xq_fa_range(q.data_ptr(), positions.data_ptr(), n_q, n_head, k.data_ptr(), v.data_ptr(),
                           n_head_kv, head_dim, kv_type, origin, active, kq_scale, split_mode,
                           out.data_ptr(), lse.data_ptr(), ctypes.c_void_p(wp), wn, _stream(stream)),
           "fa_range")
    return ws


def fa_lse_merge(parts_out, parts_lse, out, lse, stream=None):
    """Merge position-split results: parts_out [n_parts, rows, D], parts_lse
    [n_parts, rows] (device tensors) into out [rows, D], lse [rows]."""
    n_parts, rows, d = parts_out.shape
    _check(load().xq_fa_lse_merge(parts_out.data_ptr(), parts_lse.data_ptr(), n_parts, rows, d, out.data_ptr(),
                                  lse.data_ptr(), _stream(stream)), "fa_lse_merge")


def split_count(kv_len: int, split_mode: int = SPLIT_AUTO) -> int:
    return int(load().xq_fa_split_count(kv_len, split_mode))


def fa_params_from_env(params: XqFaParams) -> XqFaParams:
    """Apply the environment's ggml knobs (GGML_FLASH_ATTN_NO_QUERY_TILING,
    GGML_FLASH_ATTN_NO_SPLIT_KV) to params, as xq_fa_params_from_env does."""
    _check(load().xq_fa_params_from_env(ctypes.byref(params)), "fa_params_from_env")
    return params


def split_rows(kv_len: int, split_mode: int = SPLIT_AUTO) -> int:
    return int(load().xq_fa_split_rows(kv_len, split_mode))


# ---------------------------------------------------------------------------
# gated delta net
# ---------------------------------------------------------------------------

def supports_gated_delta_net(q, k, v, g, beta, state, dst, slots, raw_gates=0) -> bool:
    ds = _keep(q, k, v, g, beta, state, dst)
    return bool(load().xq_supports_gated_delta_net(*[ctypes.byref(x) for x in ds], slots, raw_gates))


def gated_delta_net_workspace(q, v, slots, mode=GDN_AUTO) -> int:
    """Device workspace bytes xq_gated_delta_net needs for these shapes and mode."""
    n = ctypes.c_size_t(0)
    dq, dv = q.desc(), v.desc()
    _check(load().xq_gated_delta_net_workspace(ctypes.byref(dq), ctypes.byref(dv), slots, mode,
                                               ctypes.byref(n)), "gated_delta_net_workspace")
    return int(n.value)


def gated_delta_net(q, k, v, g, beta, state, dst, slots, mode=GDN_AUTO, raw_gates=0,
                    workspace=None, stream=None):
    lib = load()
    dq, dv = q.desc(), v.desc()
    n = ctypes.c_size_t(0)
    _check(lib.xq_gated_delta_net_workspace(ctypes.byref(dq), ctypes.byref(dv), slots, mode,
                                            ctypes.byref(n)), "gated_delta_net_workspace")
    ws = _workspace(n.value + 256, workspace) if n.value else None
    wp, wn = _aligned_ptr(ws)
    ds = _keep(q, k, v, g, beta, state, dst)
    _check(lib.xq_gated_delta_net(*[ctypes.byref(x) for x in ds], slots, raw_gates, mode,
                                  ctypes.c_void_p(wp) if wp else None, wn, _stream(stream)),
           "gated_delta_net")
    return ws


# ---------------------------------------------------------------------------
# KV append
# ---------------------------------------------------------------------------

def kv_record_bytes(kv_type: int, head_dim: int) -> int:
    return int(load().xq_kv_record_bytes(kv_type, head_dim))


def kv_store(src, positions, n_head_kv, head_dim, kv_type, dst, capacity, q8_variant=0, stream=None):
    """src float32 [n_tokens, n_head_kv, head_dim] (device) -> dst cache plane."""
    n_tokens = positions.numel()
    _check(load().xq_kv_store(src.data_ptr(), positions.data_ptr(), n_tokens, n_head_kv, head_dim,
                              kv_type, q8_variant, dst.data_ptr(), capacity, _stream(stream)),
           "kv_store")


def abi_version() -> int:
    return int(load().xq_abi_version())


# ---------------------------------------------------------------------------
# per-kernel device timing
# ---------------------------------------------------------------------------

def profile_enable(on: bool = True):
    load().xq_profile_enable(1 if on else 0)


def profile_reset():
    load().xq_profile_reset()


def profile_read(max_entries: int = 32) -> dict:
    """{kernel name: (total device ms, launches)} accumulated since the last reset."""
    names = ctypes.create_string_buffer(32 * max_entries)
    ms = (ctypes.c_double * max_entries)()
    cnt = (ctypes.c_int64 * max_entries)()
    n = load().xq_profile_read(names, ms, cnt, max_entries)
    out = {}
    for i in range(n):
        nm = names.raw[32 * i: 32 * (i + 1)].split(b"\0", 1)[0].decode()
        out[nm] = (ms[i], cnt[i])
    return out


# ---------------------------------------------------------------------------
# ggml backend face (include/xq_ggml_backend.h)
# ---------------------------------------------------------------------------

class GgmlNode:
    """A ggml node for the backend: op kind, op_params words, dst and sources.

    The constructors pack op_params as ggml's own graph constructors do:
    ``ggml_flash_attn_ext`` stores (scale, max_bias, logit_softcap) as float
    bits and ``ggml_flash_attn_ext_set_prec`` the precision in word 3;
    ``ggml_gated_delta_net`` stores the snapshot slots in word 0 and the
    raw-gate flag in word 1 (src/bridge/ggml_d3d12.cpp:77-83)."""

    def __init__(self, op, dst, srcs=(), op_params=(), compute=True):
        self.op, self.dst, self.srcs = op, dst, list(srcs)
        self.op_params = list(op_params) + [0] * (GGML_MAX_OP_PARAMS - len(op_params))
        self.compute = compute
        self._keep = []

    @staticmethod
    def f32_bits(x) -> int:
        import struct
        return struct.unpack("<i", struct.pack("<f", float(x)))[0]

    @classmethod
    def flash_attn_ext(cls, q, k, v, mask, sinks, dst, scale, max_bias=0.0, softcap=0.0, prec=0, compute=True):
        words = [cls.f32_bits(scale), cls.f32_bits(max_bias), cls.f32_bits(softcap), int(prec)]
        return cls(OP_FLASH_ATTN_EXT, dst, [q, k, v, mask, sinks], words, compute)

    @classmethod
    def gated_delta_net(cls, q, k, v, g, beta, state, dst, slots, raw_gates=0, compute=True):
        return cls(OP_GATED_DELTA_NET, dst, [q, k, v, g, beta, state], [int(slots), int(raw_gates)], compute)

    @classmethod
    def noop(cls, dst):
        return cls(OP_NOOP, dst)

    def struct(self) -> XqGgmlNode:
        n = XqGgmlNode()
        n.op = self.op
        n.flags = GGML_FLAG_COMPUTE if self.compute else 0
        for i, w in enumerate(self.op_params):
            n.op_params[i] = w
        n.dst = self.dst.desc() if hasattr(self.dst, "desc") else self.dst
        self._keep = []
        for i, s in enumerate(self.srcs):
            if s is None:
                continue
            d = s.desc() if hasattr(s, "desc") else s
            self._keep.append(d)
            n.src[i] = ctypes.pointer(d)
        return n


def backend_params(fa_qk_policy=QK_CONSISTENT, fa_split_mode=SPLIT_AUTO, fa_engine=ENGINE_AUTO,
                   gdn_mode=GDN_AUTO, gdn_min_tokens=1) -> XqGgmlBackendParams:
    p = XqGgmlBackendParams()
    p.fa_qk_policy, p.fa_split_mode, p.fa_engine = fa_qk_policy, fa_split_mode, fa_engine
    p.gdn_mode, p.gdn_min_tokens = gdn_mode, gdn_min_tokens
    return p


def ggml_supports_op(node: GgmlNode, params: XqGgmlBackendParams | None = None) -> bool:
    """dev_supports_op for a backend with these params (None = the defaults);
    pure, no GPU needed."""
    st = node.struct()
    if params is None:
        return bool(load().xq_ggml_supports_op(ctypes.byref(st)))
    return bool(load().xq_ggml_supports_op_params(ctypes.byref(st), ctypes.byref(params)))


class GgmlBackend:
    """The backend object: its own HIP stream, a grow-only workspace, and a
    synchronous ``graph_compute`` over ``GgmlNode`` lists. ``use_defaults``
    passes NULL params (the defaults, with the environment's ggml
    flash-attention knobs applied at init)."""

    def __init__(self, device=0, fa_qk_policy=QK_CONSISTENT, fa_split_mode=SPLIT_AUTO,
                 fa_engine=ENGINE_AUTO, gdn_mode=GDN_AUTO, gdn_min_tokens=1, use_defaults=False):
        lib = load()
        p = backend_params(fa_qk_policy, fa_split_mode, fa_engine, gdn_mode, gdn_min_tokens)
        self.params = None if use_defaults else p
        self._h = lib.xq_ggml_backend_init(device, None if use_defaults else ctypes.byref(p))
        if not self._h:
            raise XqError(5, "ggml_backend_init", lib.xq_last_error().decode())

    @property
    def name(self) -> str:
        return load().xq_ggml_backend_name(self._h).decode()

    @property
    def workspace_bytes(self) -> int:
        return int(load().xq_ggml_backend_workspace_bytes(self._h))

    def graph_compute(self, nodes):
        arr = (XqGgmlNode * max(1, len(nodes)))()
        for i, n in enumerate(nodes):
            arr[i] = n.struct()
        _check(load().xq_ggml_graph_compute(self._h, arr, len(nodes)), "ggml_graph_compute")

    def free(self):
        if self._h:
            load().xq_ggml_backend_free(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()
