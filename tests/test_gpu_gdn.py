"""GPU parity of GGML_OP_GATED_DELTA_NET (gfx950 kernels through the C ABI)
against the CPU restatement of the reference's recurrence (the eight-lane order
of d3d12_gdn_emulate, src/bridge/ggml_d3d12.cpp:113-158) and a float64
recurrence, with the reference selftest's matrix of T, slots and padded q/k/v
rows (src/bridge/ggml_d3d12.cpp:310-369).

Tolerance (the ops' parity bar): outputs and states within max-abs 2e-3 / rel 1e-2.
"""
import numpy as np
import pytest

import oracle
import xqattn
from conftest import assert_close, case_note
from gdn_cases import make_gdn_case, out_array
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(1e30)


def run_gpu(case, torch, mode=xqattn.GDN_AUTO):
    dev = {n: xqattn.DevTensor.from_host(getattr(case, n)) for n in ("q", "k", "v", "g", "beta", "state")}
    dst = xqattn.DevTensor.from_host(case.dst)  # keeps the sentinel fill
    xqattn.gated_delta_net(dev["q"], dev["k"], dev["v"], dev["g"], dev["beta"], dev["state"], dst,
                           case.slots, mode=mode)
    torch.cuda.synchronize()
    after = {n: d.to_host_bytes() for n, d in dev.items()}
    for n, d in after.items():
        assert np.array_equal(d, getattr(case, n).buf.reshape(-1).view(np.uint8)), f"input {n} was written"
    return np.frombuffer(dst.to_host_bytes().tobytes(), np.float32).reshape(case.B, -1, 4096)


def test_gdn_step_c3(torch_gpu):
    cfg = wl.GDN_C3
    case_note(f"gated_delta_net {cfg.name}")
    case = make_gdn_case(cfg.T, cfg.slots, B=cfg.B, dist="model", seed=99)
    got = run_gpu(case, torch_gpu)
    want = case.oracle()
    err = assert_close(got, want, what="8-sequence step vs restated recurrence")
    ref64 = case.oracle_f64()
    err64 = assert_close(got, ref64, atol=1e-5, rtol=1e-4, what="8-sequence step vs float64")
    print(f"8-sequence step: max|gpu-oracle|={err:.2e} max|gpu-f64|={err64:.2e}")


@pytest.mark.parametrize("slots", [5, 1])
@pytest.mark.parametrize("T", [5, 1, 2, 3, 4, 64])
def test_gdn_selftest_matrix(torch_gpu, T, slots):
    """The reference's selftest cases: rel_err <= 1e-4 against the CPU op,
    unwritten snapshot slots untouched, inputs untouched."""
    case_note(f"gdn selftest T={T} K={slots}")
    case = make_gdn_case(T, slots, B=1, dist="selftest", pad=0)
    got = run_gpu(case, torch_gpu)
    want = case.oracle()
    valid = 4096 * T + 524288 * min(T, slots)
    g, w = got.reshape(-1), want.reshape(-1)
    rel = np.abs(g[:valid] - w[:valid]).max() / np.abs(w[:valid]).max()
    assert rel <= 1e-4, rel
    assert np.all(g[valid:] == SENTINEL), "an unwritten snapshot slot was overwritten"


@pytest.mark.parametrize("T,pad", [(3, 3), (4, 3), (6, 5), (2, 7)])
def test_gdn_padded_rows(torch_gpu, T, pad):
    case = make_gdn_case(T, 5, B=1, dist="selftest", pad=pad)
    got = run_gpu(case, torch_gpu)
    assert_close(got, case.oracle(), atol=1e-6, rtol=1e-4, what=f"padded q/k/v pad={pad}")


def test_gdn_prefix_invariance(torch_gpu):
    """Outputs of the first t tokens and the snapshots agree across T and K
    (src/bridge/ggml_d3d12.cpp:333-351)."""
    base = run_gpu(make_gdn_case(5, 5, B=1, dist="selftest"), torch_gpu).reshape(-1)
    for T in (1, 2, 3, 4):
        for slots in (5, 1):
            got = run_gpu(make_gdn_case(T, slots, B=1, dist="selftest"), torch_gpu).reshape(-1)
            assert np.array_equal(got[:4096 * T], base[:4096 * T])
            for j in range(min(T, slots)):
                st = 5 - T if slots == 1 else 5 - T + j
                a = got[4096 * T + 524288 * j: 4096 * T + 524288 * (j + 1)]
                b = base[4096 * 5 + 524288 * st: 4096 * 5 + 524288 * (st + 1)]
                assert np.array_equal(a, b), (T, slots, j)


@pytest.mark.parametrize("B", [1, 3, 8])
def test_gdn_bf16_inputs(torch_gpu, B):
    case = make_gdn_case(7, 2, B=B, dist="model", bf16=True, seed=5)
    got = run_gpu(case, torch_gpu)
    assert_close(got, case.oracle(), what=f"bf16 q/k/v B={B}")


def test_gdn_long_sequence_step(torch_gpu):
    """T = 512 through the token-sequential kernel against the f64 recurrence."""
    case = make_gdn_case(512, 1, B=1, dist="model", bf16=True, seed=8)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_STEP)
    assert_close(got, case.oracle_f64(), what="T=512 step vs f64")
