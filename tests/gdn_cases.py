"""Host-side construction of GATED_DELTA_NET cases (CPU and GPU tests)."""
from __future__ import annotations

import dataclasses

import numpy as np

import oracle
from xqattn import workloads as wl

SENTINEL = np.float32(1e30)


@dataclasses.dataclass
class GdnCase:
    T: int
    slots: int
    B: int
    q: wl.HostTensor
    k: wl.HostTensor
    v: wl.HostTensor
    g: wl.HostTensor
    beta: wl.HostTensor
    state: wl.HostTensor
    dst: wl.HostTensor

    def oracle(self, threads=16):
        dst = wl.HostTensor(wl.F32, self.dst.ne, self.dst.nb, self.dst.buf.copy())
        oracle.gated_delta_net(self.q, self.k, self.v, self.g, self.beta, self.state, dst, self.slots, threads)
        return np.frombuffer(dst.buf.tobytes(), np.float32).reshape(self.B, -1, 4096)

    def oracle_f64(self, threads=16):
        out = oracle.gated_delta_net_f64(self.q, self.k, self.v, self.g, self.beta, self.state, self.slots, threads)
        sent = np.frombuffer(self.dst.buf.tobytes(), np.float32).reshape(self.B, -1, 4096).astype(np.float64)
        valid = self.T + 128 * min(self.T, self.slots)
        sent[:, :valid] = out[:, :valid]
        return sent


def _selftest_inputs(T, B, seed=1701):
    """The reference selftest's recipe (src/bridge/ggml_d3d12.cpp:222-239):
    uniform(-0.05, 0.05) per tensor, g = -0.3 - |u|, beta = u + 0.5; one
    generator stream per tensor, independent of T/K/padding (so prefixes agree)."""
    def uni(j, shape):
        # per-token streams make the first t tokens identical for every T
        n_per = int(np.prod(shape[2:])) if len(shape) > 2 else 1
        out = np.empty(shape, np.float32)
        for b in range(shape[0]):
            for t in range(shape[1]):
                u = wl.uniform(seed + j, n_per, offset=(b * 4096 + t) * n_per)
                out[b, t] = (u * 0.1 - 0.05).astype(np.float32).reshape(shape[2:])
        return out
    q = uni(0, (B, T, 16, 128))
    k = uni(1, (B, T, 16, 128))
    v = uni(2, (B, T, 32, 128))
    g = (-0.3 - np.abs(uni(3, (B, T, 32)))).astype(np.float32)
    beta = (uni(4, (B, T, 32)) + np.float32(0.5)).astype(np.float32)
    st = np.empty((B, 32, 128, 128), np.float32)
    for b in range(B):
        st[b] = (wl.uniform(seed + 5, 32 * 128 * 128, offset=b * 524288) * 0.1 - 0.05).astype(np.float32).reshape(32, 128, 128)
    return q, k, v, g, beta, st


def make_gdn_case(T, slots, B=1, dist="model", seed=1234, pad=0, bf16=False, v_scale=1.0,
                  qk_edit=None, vs_edit=None, gb_edit=None) -> GdnCase:
    """v_scale multiplies v and the initial state (the recurrence is linear in
    them); qk_edit(q, k) edits the f32 q [B,T,16,128] and k rows, vs_edit(v,
    st) the f32 v [B,T,32,128] and the initial state [B,32,128 (c),128 (i)],
    gb_edit(g, beta) the decays and betas [B,T,32], in place before they are
    stored."""
    if dist == "selftest":
        q, k, v, g, beta, st = _selftest_inputs(T, B)
    else:
        q, k, v, g, beta, st = wl.gdn_inputs(wl.GdnConfig("case", T, B, slots, bf16), seed=seed)
    if v_scale != 1.0:
        v = (v * np.float32(v_scale)).astype(np.float32)
        st = (st * np.float32(v_scale)).astype(np.float32)
    if qk_edit is not None:
        qk_edit(q, k)
    if vs_edit is not None:
        vs_edit(v, st)
    if gb_edit is not None:
        gb_edit(g, beta)
    typ = wl.BF16 if bf16 else wl.F32
    if bf16:
        q, k, v = (oracle.f32_to_bf16(a) for a in (q, k, v))
    pads = (pad, pad + 2 if pad else 0, pad + 4 if pad else 0)
    qt = wl.padded_rows_tensor(q, typ, pads[0])
    kt = wl.padded_rows_tensor(k, typ, pads[1])
    vt = wl.padded_rows_tensor(v, typ, pads[2])
    gt = wl.f32_tensor(g, (1, 32, T, B))
    bt = wl.f32_tensor(beta, (1, 32, T, B))
    stt = wl.f32_tensor(st, (128, 128, 32, B))
    rows = T + slots * 128
    dst = wl.HostTensor(wl.F32, (4096, rows, B, 1), (4, 16384, 16384 * rows, 16384 * rows * B),
                        np.full(B * rows * 4096, SENTINEL, np.float32).view(np.uint8))
    return GdnCase(T, slots, B, qt, kt, vt, gt, bt, stt, dst)


def out_array(case: GdnCase, raw) -> np.ndarray:
    return np.frombuffer(raw.tobytes(), np.float32).reshape(case.B, -1, 4096)
