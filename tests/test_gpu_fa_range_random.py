"""GPU parity of RKVA range attention (`xq_fa_range`: pass 1 + the ascending
split reduce, OUT + LSE) over seeded random shapes: KV type, head dim, GQA
group, KV heads, query count, active rows (down to none and one), origin,
query positions before, inside and past the active rows, and split mode, each
case against the oracle's restatement of the reference's range pass and
reducer (uwp/rkva/remote-attn-engine.cpp:2774-3251,
shaders/rkva/rkva_range_reduce_opt.hlsl) and a float64 closed form.

A query at position p sees the rows r < min(p - origin + 1, active); one that
sees none has O = 0 and LSE = -inf (uwp/rkva/remote-attn-protocol.h:228-231).

Tolerance: the reference's range-probe bar against the restatement, O within
3e-4 + 3e-4|ref| and LSE within 3e-4 + 3e-5|ref| (tests/rkva_range_probe.py:139,148);
against float64, relative to the largest output, 1e-5 for every KV type, and
LSE within 1e-4 + 1e-5|ref|.
"""
import numpy as np
import pytest

import oracle
import xqattn
from conftest import assert_close, case_note
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu

N_CASES = 24
KV_TYPES = [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2]
SPLITS = [xqattn.SPLIT_AUTO, xqattn.SPLIT_REFERENCE, xqattn.SPLIT_FINE, xqattn.SPLIT_NONE,
          xqattn.SPLIT_MQ_BALANCED]


def draw_case(i):
    r = np.random.default_rng(990 + 13 * i)
    kv = KV_TYPES[i % len(KV_TYPES)]
    D = int(r.choice([128, 256]))
    hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 3, 4, 6, 8]))
    n_q = int(r.integers(1, 9))
    active = int(r.choice([0, 1, 15, 16, 17, int(r.integers(18, 700)), int(r.integers(700, 4000))]))
    origin = int(r.integers(0, 200000))
    # positions: before the origin, inside the rows, at the last row, past them
    kinds = r.integers(0, 4, n_q)
    pos = []
    for k in kinds:
        if k == 0:
            pos.append(origin - int(r.integers(1, 50)))
        elif k == 1 and active > 0:
            pos.append(origin + int(r.integers(0, active)))
        elif k == 2:
            pos.append(origin + active - 1)
        else:
            pos.append(origin + active + int(r.integers(0, 300)))
    split = SPLITS[int(r.integers(0, len(SPLITS)))]
    return kv, D, hkv, G, n_q, active, origin, np.array(pos, np.int32), split


def range_f64(q, positions, n_head, kf, vf, hkv, origin, active, scale):
    """Closed form in float64 over the dequantized rows: (O [n_q, H, D], LSE [n_q, H])."""
    n_q, _, D = q.shape
    G = n_head // hkv
    out = np.zeros((n_q, n_head, D))
    lse = np.full((n_q, n_head), -np.inf)
    for i, p in enumerate(positions):
        lim = 0 if p < origin else min(int(p) - origin + 1, active)
        if lim <= 0:
            continue
        for h in range(n_head):
            g = h // G
            s = kf[:lim, g, :].astype(np.float64) @ q[i, h].astype(np.float64) * scale
            m = s.max()
            w = np.exp(s - m)
            out[i, h] = w @ vf[:lim, g, :].astype(np.float64) / w.sum()
            lse[i, h] = m + np.log(w.sum())
    return out, lse


@pytest.mark.parametrize("i", range(N_CASES))
def test_fa_range_random_shapes(torch_gpu, i):
    torch = torch_gpu
    kv, D, hkv, G, n_q, active, origin, positions, split = draw_case(i)
    n_head = hkv * G
    note = (f"range case {i}: kv {wl.TYPE_NAME[kv]} D {D} H {n_head} Hkv {hkv} n_q {n_q} active {active} "
            f"origin {origin} positions {positions.tolist()} split {split}")
    case_note(note)
    cap = max(active, 1)
    kraw = oracle.quantize(kv, wl.normal(4000 + i, (cap, hkv, D)))
    vraw = oracle.quantize(kv, wl.normal(5000 + i, (cap, hkv, D)))
    q = wl.normal(6000 + i, (n_q, n_head, D))
    scale = float(1.0 / np.sqrt(D))
    split_k = oracle.load().xo_ref_split_k(active) if active > 0 else 1
    want, wlse, _ = oracle.range_attn(q, positions, n_head, kraw, vraw, hkv, D, kv, origin, active, scale, split_k)

    out = torch.empty(n_q * n_head * D, dtype=torch.float32, device="cuda")
    lse = torch.empty(n_q * n_head, dtype=torch.float32, device="cuda")
    xqattn.fa_range(torch.from_numpy(q).cuda(), torch.from_numpy(positions).cuda(), n_head,
                    torch.from_numpy(kraw.reshape(-1)).cuda(), torch.from_numpy(vraw.reshape(-1)).cuda(),
                    hkv, D, kv, origin, active, scale, out, lse, split_mode=split)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(n_q, n_head, D)
    glse = lse.cpu().numpy().reshape(n_q, n_head)

    # empty queries: O = 0, LSE = -inf, exactly
    lims = np.array([0 if p < origin else min(int(p) - origin + 1, active) for p in positions])
    empty = lims <= 0
    assert np.all(got[empty] == 0.0), f"{note}: an empty query's O is not 0"
    assert np.all(np.isneginf(glse[empty])), f"{note}: an empty query's LSE is not -inf"

    assert_close(got, want, atol=3e-4, rtol=3e-4, what=f"{note} O vs restatement")
    fin = np.isfinite(wlse)
    assert np.array_equal(np.isfinite(glse), fin), f"{note}: LSE finiteness"
    assert_close(glse[fin], wlse[fin], atol=3e-4, rtol=3e-5, what=f"{note} LSE vs restatement")

    kf = oracle.dequant(kv, kraw.reshape(-1, kraw.shape[-1]), D).reshape(cap, hkv, D)
    vf = oracle.dequant(kv, vraw.reshape(-1, vraw.shape[-1]), D).reshape(cap, hkv, D)
    ref64, lse64 = range_f64(q, positions, n_head, kf, vf, hkv, origin, active, scale)
    if np.any(~empty):
        err = float(np.abs(got - ref64).max())
        rel = err / max(float(np.abs(ref64).max()), 1e-30)
        assert rel < 1e-5, (note, rel)
        assert_close(glse[~empty], lse64[~empty], atol=1e-4, rtol=1e-5, what=f"{note} LSE vs float64")
        print(f"{note}: max|gpu-f64| / max|f64| {rel:.2e}")
