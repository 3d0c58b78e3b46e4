"""GPU parity of GGML_OP_FLASH_ATTN_EXT over seeded random shapes: KV type, head
dim, GQA group, KV heads, queries, sequences, KV length (down to a single row),
causal prefix, mask padding rows, sinks, softcap, ALiBi and split mode drawn
from a fixed-seed generator, each case checked against the ggml-CPU
restatement in oracle/ and the float64 closed form.

The shapes between the benchmark configurations are where the kernels' tile
and split boundaries fall differently (ragged last slices, splits shorter than
a slice, query tiles with idle pairs, GQA groups that do not divide 16).

Tolerance (the ops' parity bar): max-abs 2e-3 / rel 1e-2 elementwise against the
restatement and against float64. Relative to the largest output, the outputs
stay within 1e-5 of float64 for every KV type: the value products keep about
22 significant bits (f16 hi + lo operands) and accumulate in f32, so even short
KV lengths, where roundings do not average out, stay at f32-class precision.
"""
import numpy as np
import pytest

import xqattn
from conftest import assert_close, case_note
from fa_cases import make_fa_case, oracle_f64, oracle_fa, run_fa_gpu
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu

N_CASES = 40
KV_TYPES = [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2]
SPLITS = [xqattn.SPLIT_AUTO, xqattn.SPLIT_REFERENCE, xqattn.SPLIT_FINE, xqattn.SPLIT_NONE]


def draw_case(i):
    """Case i of the fixed sequence: (FaConfig, make_fa_case kwargs, split mode)."""
    r = np.random.default_rng(20261202 + i)
    kv = KV_TYPES[i % len(KV_TYPES)]
    D = int(r.choice([128, 256]))
    Hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 3, 4, 5, 6, 8]))
    n_q = int(r.integers(1, 9))
    B = int(r.integers(1, 4))
    L = int(r.choice([1, 2, 15, 16, 17, 33, int(r.integers(18, 700)), int(r.integers(700, 3000)),
                      int(r.integers(700, 3000)), int(r.integers(3000, 5000))]))
    L = max(L, n_q)
    causal = bool(r.integers(0, 2)) or n_q > 1
    pad = int(r.choice([0, 0, 3, 8])) if causal else 0
    cfg = wl.FaConfig(f"rand{i}", n_q, G * Hkv, Hkv, D, L, B, kv,
                      causal_prefix=(L - n_q) if causal else None,
                      n_q_pad=(n_q + pad) if pad else None)
    kw = dict(seed=1000 + 17 * i, mask="causal" if causal else None,
              sinks=bool(r.integers(0, 4) == 0),
              softcap=float(r.choice([0.0, 0.0, 0.0, 20.0])),
              max_bias=float(r.choice([0.0, 0.0, 0.0, 8.0])) if causal else 0.0)
    split = SPLITS[int(r.integers(0, len(SPLITS)))]
    return cfg, kw, split


@pytest.mark.parametrize("i", range(N_CASES))
def test_fa_random_shapes(torch_gpu, i):
    cfg, kw, split = draw_case(i)
    note = (f"random case {i}: kv {wl.TYPE_NAME[cfg.kv_type]} D {cfg.D} H {cfg.H} Hkv {cfg.Hkv} "
            f"n_q {cfg.n_q} (pad {cfg.n_q_pad}) B {cfg.B} L {cfg.L} split {split} "
            f"sinks {kw['sinks']} softcap {kw['softcap']} max_bias {kw['max_bias']}")
    case_note(note)
    case = make_fa_case(cfg, **kw)
    got, glse = run_fa_gpu(case, torch_gpu, split_mode=split)
    want, _ = oracle_fa(case)
    assert_close(got, want, what=f"{note} vs ggml-CPU restatement")
    ref64, lse64 = oracle_f64(case)
    err64 = assert_close(got, ref64, what=f"{note} vs float64")
    fin = np.isfinite(lse64)
    assert np.array_equal(np.isfinite(glse), fin), f"{note}: LSE finiteness"
    assert_close(glse[fin], lse64[fin], atol=1e-4, rtol=1e-5, what=f"{note} LSE")
    # against float64, relative to the largest output: the value products
    # (quantized V's weight x block scale, F16 / E5M2 V's weight) enter the
    # matrix cores as f16 hi + lo, about 22 significant bits, and accumulate in
    # f32, as ggml's f32 products w * (q * d) do
    scale = max(float(np.abs(ref64).max()), 1e-30)
    assert err64 / scale < 1e-5, (note, err64 / scale)
    print(f"{note}: max|gpu-f64| {err64:.2e}, / max|f64| {err64 / scale:.2e}")
