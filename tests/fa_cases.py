"""Host-side construction of flash-attention cases shared by the CPU and GPU tests."""
from __future__ import annotations

import dataclasses

import numpy as np

import oracle
from xqattn import workloads as wl


@dataclasses.dataclass
class FaCase:
    cfg: wl.FaConfig
    q: wl.HostTensor
    k: wl.HostTensor
    v: wl.HostTensor
    mask: wl.HostTensor | None
    sinks: wl.HostTensor | None
    dst: wl.HostTensor
    scale: float
    softcap: float = 0.0
    max_bias: float = 0.0

    @property
    def shape(self):
        c = self.cfg
        return (c.B, c.n_q, c.H, c.D)


def make_fa_case(cfg: wl.FaConfig, seed: int = 7, mask: str | None = "causal", sinks=False,
                 softcap=0.0, max_bias=0.0, q8_variant=0, kv_scale=1.0, q_scale=1.0,
                 mask_per_seq=False, v_scale=1.0) -> FaCase:
    """Q/K/V ~ N(0,1) from the splitmix generator; K/V quantised by the oracle's
    ggml quantizers (or rounded to f16 / E5M2). kv_scale multiplies K and V,
    v_scale V alone (the score distribution stays the same)."""
    B, NQ, H, Hkv, D, L = cfg.B, cfg.n_q, cfg.H, cfg.Hkv, cfg.D, cfg.L
    q = wl.normal(seed, (B, NQ, H, D)) * np.float32(q_scale)
    kf = wl.normal(seed + 1, (B, L, Hkv, D)) * np.float32(kv_scale)
    vf = wl.normal(seed + 2, (B, L, Hkv, D)) * np.float32(kv_scale * v_scale)
    kraw = oracle.quantize(cfg.kv_type, kf, q8_variant)
    vraw = oracle.quantize(cfg.kv_type, vf, q8_variant)
    del kf, vf
    mt = None
    if mask == "causal":
        m = wl.fa_causal_mask(cfg)
        if mask_per_seq:
            m = np.repeat(m, B, axis=0)
        mt = wl.mask_tensor(m)
    elif mask is not None:
        raise ValueError(mask)
    st = None
    if sinks:
        s = wl.normal(seed + 3, (H,)) * np.float32(2.0)
        st = wl.f32_tensor(s, (H, 1, 1, 1))
    return FaCase(cfg, wl.fa_q_tensor(q), wl.kv_tensor(kraw, cfg.kv_type, D),
                  wl.kv_tensor(vraw, cfg.kv_type, D), mt, st, wl.fa_dst_tensor(B, NQ, H, D),
                  cfg.kq_scale, softcap, max_bias)


def dst_array(case: FaCase, raw: np.ndarray | None = None) -> np.ndarray:
    """dst bytes -> float32 [B, n_q, H, D]."""
    b = case.dst.buf if raw is None else raw
    B, NQ, H, D = case.shape
    return np.frombuffer(b.tobytes(), np.float32).reshape(B, NQ, H, D)


def oracle_fa(case: FaCase, policy=oracle.QK_CONSISTENT, v_acc_f16=True, threads=16):
    """The ggml-CPU restatement: returns (out [B,n_q,H,D], lse [B,n_q,H])."""
    dst = wl.fa_dst_tensor(*case.shape[:1], case.cfg.n_q, case.cfg.H, case.cfg.D)
    lse = oracle.flash_attn_ext(case.q, case.k, case.v, case.mask, case.sinks, dst, case.scale,
                                case.max_bias, case.softcap, policy, v_acc_f16, threads)
    B, NQ, H, D = case.shape
    return np.frombuffer(dst.buf.tobytes(), np.float32).reshape(B, NQ, H, D).copy(), lse


def oracle_f64(case: FaCase, policy=oracle.QK_CONSISTENT, q_round=True, threads=16):
    return oracle.flash_attn_f64(case.q, case.k, case.v, case.mask, case.sinks, case.scale,
                                 case.max_bias, case.softcap, policy, q_round, threads)


def run_fa_gpu(case: FaCase, torch, qk_policy=None, split_mode=None, want_lse=True, engine=None):
    """xq_flash_attn_ext on the GPU: returns (out [B,n_q,H,D], lse [B,n_q,H] or None)."""
    import xqattn
    qk_policy = xqattn.QK_CONSISTENT if qk_policy is None else qk_policy
    split_mode = xqattn.SPLIT_AUTO if split_mode is None else split_mode
    engine = xqattn.ENGINE_AUTO if engine is None else engine
    q = xqattn.DevTensor.from_host(case.q)
    k = xqattn.DevTensor.from_host(case.k)
    v = xqattn.DevTensor.from_host(case.v)
    m = xqattn.DevTensor.from_host(case.mask) if case.mask is not None else None
    s = xqattn.DevTensor.from_host(case.sinks) if case.sinks is not None else None
    d = xqattn.DevTensor.empty_like_host(case.dst)
    B, NQ, H, D = case.shape
    lse = torch.empty(B * NQ * H, dtype=torch.float32, device="cuda") if want_lse else None
    p = xqattn.fa_params(case.scale, case.max_bias, case.softcap, qk_policy, split_mode, engine)
    xqattn.flash_attn_ext(q, k, v, m, s, d, p, lse=lse)
    torch.cuda.synchronize()
    out = dst_array(case, d.to_host_bytes())
    return out, (lse.cpu().numpy().reshape(B, NQ, H) if want_lse else None)
