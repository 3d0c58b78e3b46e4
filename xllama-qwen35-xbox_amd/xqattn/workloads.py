"""Synthetic workloads in ggml tensor layouts, with a deterministic generator.

Tensors are described as in ggml: ``ne`` (elements, innermost first) and ``nb``
(byte strides), over a flat byte buffer. The layouts are the ones llama.cpp
hands to the ops:

* FLASH_ATTN_EXT ``q`` is the permuted view ``[D, n_q, H, B]`` of a token-major
  activation (``nb1 = H*D*4`` token stride, ``nb2 = D*4`` head stride);
  ``k``/``v`` are KV-cache views ``[D, L, Hkv, B]`` whose row stride is all KV
  heads of a token (``nb1 = Hkv*record``, ``nb2 = record``); the mask is F16
  ``[L, n_q_pad, 1, B]``; the output is ``[D, H, n_q, B]``.
* GATED_DELTA_NET ``q``/``k`` ``[128, 16, T, B]``, ``v`` ``[128, 32, T, B]``,
  gates ``[1, 32, T, B]``, state ``[128, 128, 32, B]`` with element (i, c) of
  head h at ``h*16384 + c*128 + i``, output ``[4096, T + slots*128, B, 1]``.

The random generator is splitmix64 + Box-Muller in float64 rounded to f32, so
inputs are bit-identical on any host and across library versions.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

F32, F16, Q4_0, Q8_0, BF16, E5M2 = 0, 1, 2, 8, 30, 0x100
TYPE_SIZE = {F32: 4, F16: 2, BF16: 2, Q8_0: 34, Q4_0: 18, E5M2: 1}
BLOCK = {F32: 1, F16: 1, BF16: 1, Q8_0: 32, Q4_0: 32, E5M2: 1}
TYPE_NAME = {F32: "f32", F16: "f16", BF16: "bf16", Q8_0: "q8_0", Q4_0: "q4_0", E5M2: "e5m2"}


def record_bytes(typ: int, d: int) -> int:
    return d // BLOCK[typ] * TYPE_SIZE[typ]


# ---------------------------------------------------------------------------
# deterministic generator
# ---------------------------------------------------------------------------

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset..offset+n-1 of splitmix64 seeded with ``seed``."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """float64 uniforms in (0, 1)."""
    z = splitmix64(seed, n, offset)
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape, chunk: int = 1 << 22) -> np.ndarray:
    """N(0,1) float32 via Box-Muller on consecutive uniform pairs."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, np.float32)
    done = 0
    while done < n:
        m = min(chunk, n - done)
        half = (m + 1) // 2
        u = uniform(seed, 2 * half, 2 * ((done + 1) // 2) if done else 0)
        u1, u2 = u[0::2], u[1::2]
        r = np.sqrt(-2.0 * np.log(u1))
        t = 2.0 * math.pi * u2
        z = np.empty(2 * half, np.float64)
        z[0::2] = r * np.cos(t)
        z[1::2] = r * np.sin(t)
        out[done:done + m] = z[:m].astype(np.float32)
        done += m
    return out.reshape(shape)


# ---------------------------------------------------------------------------
# ggml-shaped host tensors
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class HostTensor:
    """A ggml tensor over host bytes: type id, ne, nb (bytes), flat buffer."""
    type: int
    ne: tuple
    nb: tuple
    buf: np.ndarray  # contiguous uint8 (or typed) array holding the bytes

    @property
    def nbytes(self) -> int:
        return self.buf.nbytes


def _as_bytes(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).reshape(-1).view(np.uint8)


def fa_q_tensor(q: np.ndarray) -> HostTensor:
    """q float32 [B, n_q, H, D] (token-major) -> ggml [D, n_q, H, B] view."""
    B, NQ, H, D = q.shape
    return HostTensor(F32, (D, NQ, H, B), (4, H * D * 4, D * 4, NQ * H * D * 4), _as_bytes(q.astype(np.float32)))


def kv_tensor(raw: np.ndarray, typ: int, d: int) -> HostTensor:
    """raw records uint8 [B, L, Hkv, rec] -> ggml [D, L, Hkv, B] cache view."""
    B, L, Hkv, rec = raw.shape
    assert rec == record_bytes(typ, d)
    return HostTensor(typ, (d, L, Hkv, B), (TYPE_SIZE[typ], Hkv * rec, rec, L * Hkv * rec), _as_bytes(raw))


def mask_tensor(mask_f16: np.ndarray) -> HostTensor:
    """mask uint16 (f16 bits) [Bm, n_q_pad, L] -> ggml [L, n_q_pad, 1, Bm]."""
    Bm, NP, L = mask_f16.shape
    return HostTensor(F16, (L, NP, 1, Bm), (2, L * 2, NP * L * 2, NP * L * 2), _as_bytes(mask_f16.astype(np.uint16)))


def fa_dst_tensor(B: int, NQ: int, H: int, D: int) -> HostTensor:
    """Output [D, H, n_q, B] (ggml's permuted FA result), zero filled."""
    buf = np.zeros(B * NQ * H * D * 4, np.uint8)
    return HostTensor(F32, (D, H, NQ, B), (4, D * 4, H * D * 4, NQ * H * D * 4), buf)


def f32_tensor(a: np.ndarray, ne: tuple) -> HostTensor:
    """Contiguous float32 array whose C order matches ggml ne (reversed)."""
    a = np.ascontiguousarray(a, np.float32)
    nb = [4]
    for i in range(1, 4):
        nb.append(nb[-1] * ne[i - 1])
    return HostTensor(F32, tuple(ne), tuple(nb), _as_bytes(a))


def padded_rows_tensor(a: np.ndarray, typ: int, pad: int) -> HostTensor:
    """[B, T, heads, 128] rows -> ggml [128, heads, T, B] with `pad` extra elements
    between head rows (the reference selftest's padded q/k/v layouts)."""
    B, T, Hh, Dd = a.shape
    es = 4 if typ == F32 else 2
    row = (Dd + pad) * es
    buf = np.zeros(B * T * Hh * row, np.uint8)
    view = buf.reshape(B, T, Hh, row)
    if typ == F32:
        view[..., : Dd * 4] = np.ascontiguousarray(a, np.float32).view(np.uint8).reshape(B, T, Hh, Dd * 4)
    else:
        view[..., : Dd * 2] = np.ascontiguousarray(a, np.uint16).view(np.uint8).reshape(B, T, Hh, Dd * 2)
    return HostTensor(typ, (Dd, Hh, T, B), (es, row, Hh * row, T * Hh * row), buf)


# ---------------------------------------------------------------------------
# the workload configurations
# ---------------------------------------------------------------------------

@dataclasses.dataclass(frozen=True)
class FaConfig:
    name: str
    n_q: int
    H: int
    Hkv: int
    D: int
    L: int
    B: int
    kv_type: int
    causal_prefix: int | None = None   # query i sees rows <= causal_prefix + i
    n_q_pad: int | None = None          # mask rows (>= n_q); extra rows are -inf
    scale: float | None = None

    @property
    def kq_scale(self) -> float:
        return self.scale if self.scale is not None else 1.0 / math.sqrt(self.D)

    def kv_bytes(self) -> int:
        return 2 * self.B * self.L * self.Hkv * record_bytes(self.kv_type, self.D)

    def algorithmic_bytes(self) -> int:
        """K+V read once, Q read once, O written once, mask rows read once."""
        qo = 2 * self.B * self.n_q * self.H * self.D * 4
        mask = self.B * self.n_q * self.L * 2
        return self.kv_bytes() + qo + mask


FA_C1 = FaConfig("fa_decode_f16_h16kv8_d128_L4096", 1, 16, 8, 128, 4096, 1, F16)
FA_C2 = FaConfig("fa_decode_q8_0_h24kv4_d256_L32768_b4", 1, 24, 4, 256, 32768, 4, Q8_0)
# verify: mask padded to 16 rows (rows 8..15 all -inf, never read by the op)
FA_C5 = FaConfig("fa_verify_q4_0_nq8_h32kv8_d128_L16392_b8", 8, 32, 8, 128, 16392, 8, Q4_0,
                 causal_prefix=16384, n_q_pad=16)


@dataclasses.dataclass(frozen=True)
class GdnConfig:
    name: str
    T: int
    B: int
    slots: int = 1
    bf16: bool = False

    def algorithmic_bytes(self) -> int:
        es = 2 if self.bf16 else 4
        qk = 2 * self.B * self.T * 16 * 128 * es
        v = self.B * self.T * 32 * 128 * es
        gb = 2 * self.B * self.T * 32 * 4
        y = self.B * self.T * 32 * 128 * 4
        state_in = self.B * 32 * 128 * 128 * 4
        snaps = min(self.T, self.slots)
        state_out = self.B * snaps * 32 * 128 * 128 * 4
        return qk + v + gb + y + state_in + state_out


GDN_C3 = GdnConfig("gdn_step_hk16_hv32_d128_b8", T=1, B=8, slots=1)
GDN_C4 = GdnConfig("gdn_prefill_T4096_c64_bf16", T=4096, B=1, slots=1, bf16=True)
GDN_C4_B8 = GdnConfig("gdn_prefill_T4096_c64_bf16_b8", T=4096, B=8, slots=1, bf16=True)  # 8 sequences at once


def fa_causal_mask(cfg: FaConfig, n_q_rows: int | None = None) -> np.ndarray:
    """f16-bit mask [1, n_q_pad, L]: 0 visible / -inf hidden, padding rows -inf."""
    n_q_pad = cfg.n_q_pad or cfg.n_q
    rows = n_q_rows if n_q_rows is not None else cfg.n_q
    m = np.full((1, n_q_pad, cfg.L), 0xFC00, np.uint16)  # -inf
    for i in range(min(rows, n_q_pad)):
        end = cfg.L if cfg.causal_prefix is None else min(cfg.L, cfg.causal_prefix + i + 1)
        m[0, i, :end] = 0
    return m


def gdn_inputs(cfg: GdnConfig, seed: int = 1234, state_scale: float = 0.1):
    """The model's GDN input distributions: q, k L2-normalised N(0,1) per (token, head);
    v ~ N(0,1); beta = sigmoid(N(0,1)); g = -softplus(N(0,1)); S0 ~ 0.1*N(0,1).
    Returns float32 arrays q, k [B,T,16,128], v [B,T,32,128], g, beta [B,T,32],
    state [B,32,128,128]."""
    B, T = cfg.B, cfg.T
    q = normal(seed + 1, (B, T, 16, 128))
    k = normal(seed + 2, (B, T, 16, 128))
    q = (q / np.linalg.norm(q.astype(np.float64), axis=-1, keepdims=True)).astype(np.float32)
    k = (k / np.linalg.norm(k.astype(np.float64), axis=-1, keepdims=True)).astype(np.float32)
    v = normal(seed + 3, (B, T, 32, 128))
    z = normal(seed + 4, (B, T, 32)).astype(np.float64)
    beta = (1.0 / (1.0 + np.exp(-z))).astype(np.float32)
    z = normal(seed + 5, (B, T, 32)).astype(np.float64)
    g = (-np.log1p(np.exp(z))).astype(np.float32)
    state = (normal(seed + 6, (B, 32, 128, 128)) * np.float32(state_scale)).astype(np.float32)
    return q, k, v, g, beta, state
