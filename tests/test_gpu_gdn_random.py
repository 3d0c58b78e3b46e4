"""GPU parity of GGML_OP_GATED_DELTA_NET over seeded random shapes: token count
(1 to 500, so chunked runs end in ragged chunks), snapshot slots (1 to 17),
sequences, row padding, f32 or bf16 q/k/v, and the step / chunked / AUTO
modes, each case against the float64 recurrence (outputs, every kept snapshot
and the untouched slots).

Tolerance (the ops' parity bar): max-abs 2e-3 / rel 1e-2 elementwise, and the reference
selftest's max|gpu - want| / max|want| <= 1e-4 (src/bridge/ggml_d3d12.cpp:285-301).
"""
import numpy as np
import pytest

import xqattn
from conftest import assert_close, case_note
from gdn_cases import SENTINEL, make_gdn_case
from test_gpu_gdn import run_gpu

pytestmark = pytest.mark.gpu

N_CASES = 18
MODES = [xqattn.GDN_AUTO, xqattn.GDN_STEP, xqattn.GDN_CHUNKED]


def draw_case(i):
    r = np.random.default_rng(777 + 31 * i)
    T = int(r.choice([1, 2, 63, 64, 65, int(r.integers(3, 200)), int(r.integers(200, 500))]))
    slots = int(r.choice([1, 1, 2, 5, 17]))
    B = int(r.integers(1, 3))
    pad = int(r.choice([0, 0, 0, 3, 8]))
    bf16 = bool(r.integers(0, 2))
    mode = MODES[i % len(MODES)]
    return T, slots, B, pad, bf16, mode


@pytest.mark.parametrize("i", range(N_CASES))
def test_gdn_random_shapes(torch_gpu, i):
    T, slots, B, pad, bf16, mode = draw_case(i)
    note = f"gdn random case {i}: T {T} slots {slots} B {B} pad {pad} bf16 {bf16} mode {mode}"
    case_note(note)
    case = make_gdn_case(T, slots, B=B, dist="model", seed=4000 + i, pad=pad, bf16=bf16)
    got = run_gpu(case, torch_gpu, mode=mode)
    want = case.oracle_f64()
    valid = T + 128 * min(T, slots)
    assert np.all(got[:, valid:] == SENTINEL), f"{note}: an unwritten snapshot slot was overwritten"
    err = assert_close(got[:, :valid], want[:, :valid], what=f"{note} vs float64")
    rel = err / max(float(np.abs(want[:, :valid]).max()), 1e-30)
    print(f"{note}: max|gpu-f64| {err:.2e} rel {rel:.2e}")
    assert rel <= 1e-4, (note, rel)
