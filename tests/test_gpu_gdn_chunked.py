"""GPU parity of the chunked GATED_DELTA_NET prefill (64-token WY/UT chunks on
the matrix cores) against the token-sequential recurrence: the CPU restatement
of the reference's op (src/bridge/ggml_d3d12.cpp:113-158) and a float64
recurrence.

Covers the full prefill (4096 bf16 tokens), partial last chunks, snapshot slots
(the last slots - 1 tokens run on the step kernel from the chunked part's
state), f32 and bf16 inputs, padded q/k/v rows and several sequences.

Tolerance (the ops' parity bar): outputs and states within max-abs 2e-3 / rel 1e-2.
"""
import numpy as np
import pytest

import xqattn
from conftest import assert_close, case_note
from gdn_cases import SENTINEL, make_gdn_case
from test_gpu_gdn import run_gpu
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu


def _valid_rows(case):
    return case.T + 128 * min(case.T, case.slots)


def _check(case, got, want, what):
    v = _valid_rows(case)
    err = assert_close(got[:, :v], want[:, :v], what=what)
    assert np.all(got[:, v:] == SENTINEL), f"{what}: an unwritten snapshot slot was overwritten"
    return err


def test_gdn_chunked_prefill_4096_bf16(torch_gpu):
    cfg = wl.GDN_C4
    case_note(f"gated_delta_net chunked {cfg.name}")
    case = make_gdn_case(cfg.T, cfg.slots, B=cfg.B, dist="model", bf16=cfg.bf16, seed=77)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    err = _check(case, got, case.oracle(), "4096-token prefill vs restated recurrence")
    err64 = _check(case, got, case.oracle_f64(), "4096-token prefill vs float64")
    print(f"4096-token prefill: max|gpu-oracle|={err:.2e} max|gpu-f64|={err64:.2e}")


def test_gdn_chunked_prefill_8_sequences(torch_gpu):
    """8 bf16 sequences of 1089 tokens at once (2048 scan workgroups, several per
    CU, and a one-token last chunk) against the restated recurrence."""
    case_note("gated_delta_net chunked T=1089 B=8 bf16")
    case = make_gdn_case(1089, 1, B=8, dist="model", bf16=True, seed=78)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    err = _check(case, got, case.oracle(), "chunked x8 vs restated recurrence")
    print(f"T=1089 B=8: max|gpu-oracle|={err:.2e}")


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("T,slots,B", [(65, 1, 1), (100, 1, 2), (128, 1, 1), (130, 3, 1),
                                       (200, 17, 1), (257, 5, 2), (64, 1, 1), (7, 2, 1)])
def test_gdn_chunked_shapes(torch_gpu, T, slots, B, bf16):
    case_note(f"gdn chunked T={T} slots={slots} B={B} bf16={bf16}")
    case = make_gdn_case(T, slots, B=B, dist="model", bf16=bf16, seed=T + 31 * slots)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    err = _check(case, got, case.oracle_f64(), f"chunked T={T} K={slots} B={B}")
    print(f"T={T} K={slots} B={B} bf16={bf16}: max|gpu-f64|={err:.2e}")


@pytest.mark.parametrize("T,slots", [(5, 5), (5, 1), (3, 5), (64, 5), (70, 5), (70, 1)])
def test_gdn_chunked_selftest_inputs(torch_gpu, T, slots):
    """The reference selftest's input recipe through the chunked mode (with
    T < slots every token keeps a snapshot and the step kernel runs alone)."""
    case_note(f"gdn chunked selftest T={T} K={slots}")
    case = make_gdn_case(T, slots, B=1, dist="selftest")
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    _check(case, got, case.oracle(), f"chunked selftest T={T} K={slots}")


@pytest.mark.parametrize("pad", [3, 8])
def test_gdn_chunked_padded_rows(torch_gpu, pad):
    case = make_gdn_case(150, 2, B=2, dist="model", pad=pad, seed=3)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    _check(case, got, case.oracle_f64(), f"chunked padded rows pad={pad}")


def test_gdn_chunked_matches_step_kernel(torch_gpu):
    """Both kernels compute the same recurrence; AUTO picks the chunked one
    for prefills longer than one chunk."""
    case = make_gdn_case(300, 1, B=2, dist="model", bf16=True, seed=12)
    a = run_gpu(case, torch_gpu, mode=xqattn.GDN_STEP)
    b = run_gpu(case, torch_gpu, mode=xqattn.GDN_AUTO)
    c = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    assert np.array_equal(b, c)
    _check(case, c, a, "chunked vs step kernel")


@pytest.mark.parametrize("bf16", [True, False])
def test_gdn_chunked_meets_reference_selftest_bar(torch_gpu, bf16):
    """max|gpu - want| / max|want| <= 1e-4 over the outputs and the state, the
    reference selftest's criterion (src/bridge/ggml_d3d12.cpp:285-301), against
    the float64 recurrence, at 300 tokens (4 full chunks + tail). f32 rows
    enter the matrix products as f16 hi + lo, bf16 rows exactly."""
    case_note(f"gdn chunked selftest bar bf16={bf16}")
    case = make_gdn_case(300, 1, B=2, dist="model", bf16=bf16, seed=99)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    want = case.oracle_f64()
    v = _valid_rows(case)
    rel = np.abs(got[:, :v] - want[:, :v]).max() / np.abs(want[:, :v]).max()
    print(f"bf16={bf16}: rel {rel:.2e}")
    assert rel <= 1e-4, rel


def test_gdn_chunked_strong_decay(torch_gpu):
    """Decays that underflow within a chunk (g = -40 per token) keep every
    factor in [0, 1] and the result finite."""
    case = make_gdn_case(192, 1, B=1, dist="model", seed=21)
    g = np.frombuffer(case.g.buf.tobytes(), np.float32).copy()
    g[::3] = -40.0
    case.g.buf[:] = g.view(np.uint8)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    _check(case, got, case.oracle_f64(), "chunked strong decay")



def _q_large(q, k):
    q[:, 100:110, 3] *= np.float32(1e5)  # |q| |k| per element far above 256: f16 P tiles would overflow


def _k_large(q, k):
    k[:, 200, 5] *= np.float32(100.0)  # |k| above 16


def _k_nan(q, k):
    k[:, 150, 2, 7] = np.float32(np.nan)


@pytest.mark.parametrize("pad", [0, 3])
@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("edit", [_q_large, _k_large, _k_nan], ids=["q_large", "k_large", "k_nan"])
def test_gdn_chunked_out_of_range_qk_runs_the_sequential_recurrence(torch_gpu, edit, bf16, pad):
    """q / k rows outside the range the chunked form's f16 operands hold (the
    prep's per-chunk check: |k| < 16, |q| < 2^15, |q| |k| < 256, finite) send
    their (sequence, v-head) through the token-by-token f32 recurrence, so the
    result is the sequential form's: within the reference selftest's 1e-4 of
    the float64 recurrence (relative to the largest output) for large rows,
    and NaN exactly where the restated recurrence has it for a NaN k element
    (every later token and the final state of the two v-heads on that k-head)."""
    case_note(f"gdn chunked out-of-range {edit.__name__} bf16={bf16} pad={pad}")
    case = make_gdn_case(300, 1, B=2, dist="model", bf16=bf16, seed=5, pad=pad, qk_edit=edit)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    v = _valid_rows(case)
    if edit is _k_nan:
        want = case.oracle()
        assert np.array_equal(np.isnan(got[:, :v]), np.isnan(want[:, :v])), "NaN pattern differs"
        assert np.isnan(want[:, 150:300, 2 * 128:3 * 128]).all() and not np.isnan(want[:, :150]).any()
        _check(case, got, want, "NaN k vs restated recurrence")
        return
    want = case.oracle_f64()
    assert np.all(np.isfinite(got[:, :v]))
    # per v-head (outputs and state of each head apart): the enlarged rows
    # dominate their own heads' magnitudes only
    def heads(x):  # [B, 32, ...]: each head's outputs and final state
        T = case.T
        y = x[:, :T].reshape(case.B, T, 32, 128).transpose(0, 2, 1, 3).reshape(case.B, 32, -1)
        st = x[:, T:v].reshape(case.B, 32, -1)  # state (i, c) of head h at h * 16384 + c * 128 + i
        return np.concatenate([y, st], axis=2)
    gh, wh = heads(got), heads(want)
    rel = (np.abs(gh - wh).max(axis=(0, 2)) / np.abs(wh).max(axis=(0, 2))).max()
    print(f"{edit.__name__} bf16={bf16} pad={pad}: largest per-head rel {rel:.2e}")
    assert rel <= 1e-4, rel


def _v_nan(v, st):
    v[0, 150, 2, 7] = np.float32(np.nan)


def _v_inf(v, st):
    v[1, 70, 9, 100] = np.float32(np.inf)


def _state_nan(v, st):
    st[0, 20, 33, 5] = np.float32(np.nan)  # head 20, column 33, key dim 5


def _state_inf(v, st):
    st[1, 30, 3, 1] = np.float32(-np.inf)


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("edit", [_v_nan, _v_inf, _state_nan, _state_inf],
                         ids=["v_nan", "v_inf", "state_nan", "state_inf"])
def test_gdn_chunked_nonfinite_v_or_state_runs_the_sequential_recurrence(torch_gpu, edit, bf16):
    """An Inf or NaN in v or in the entering state reaches exactly the outputs
    the token recurrence gives it (its column from its token on; with the state,
    the whole column): in the chunk products a zero of T or of the causal P
    times it would be NaN in earlier tokens of its chunk, so the column block
    that holds it runs token by token. The finite outputs stay within the
    parity tolerance of the restated recurrence, the non-finite ones match its
    NaN / Inf pattern."""
    case_note(f"gdn chunked non-finite {edit.__name__} bf16={bf16}")
    case = make_gdn_case(300, 1, B=2, dist="model", bf16=bf16, seed=6, vs_edit=edit)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    want = case.oracle()
    v = _valid_rows(case)
    bad = ~np.isfinite(want[:, :v])
    assert bad.any() and not bad.all()
    if edit is _v_nan:  # column 2 * 128 + 7 of sequence 0 from token 150 on, not before
        assert np.isnan(want[0, 150:300, 2 * 128 + 7]).all() and np.isfinite(want[0, :150]).all()
    _check(case, got, want, f"{edit.__name__} vs restated recurrence")


def _g_positive(g, beta):
    g[0, 100, 4] = np.float32(0.5)


def _g_nan(g, beta):
    g[1, 200, 17] = np.float32(np.nan)


def _beta_inf(g, beta):
    beta[0, 10, 31] = np.float32(np.inf)


@pytest.mark.parametrize("edit", [_g_positive, _g_nan, _beta_inf], ids=["g_positive", "g_nan", "beta_inf"])
def test_gdn_chunked_decay_outside_0_1_runs_the_sequential_recurrence(torch_gpu, edit):
    """A g that is not finite or above 0 (a decay e^g outside [0, 1]) or a beta
    that is not finite sends its (sequence, v-head) through the token
    recurrence: the result is the restated recurrence's, non-finite pattern
    included, and a growing decay stays within the parity tolerance."""
    case_note(f"gdn chunked {edit.__name__}")
    case = make_gdn_case(300, 1, B=2, dist="model", bf16=True, seed=8, gb_edit=edit)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    _check(case, got, case.oracle(), f"{edit.__name__} vs restated recurrence")
    if edit is _g_positive:
        _check(case, got, case.oracle_f64(), "positive g vs float64")


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("v_scale", [1e-6, 1e-3, 1e3, 1e6])
def test_gdn_chunked_magnitude_sweep(torch_gpu, v_scale, bf16):
    """v and the initial state scaled by 1e-6 .. 1e6 (q, k L2-normalised, as the
    model gives them): the per-column-block power of two keeps the f16 operands
    in range, so the reference selftest's bar max|gpu - want| / max|want| <= 1e-4
    holds against the float64 recurrence at every scale."""
    case_note(f"gdn chunked magnitude v_scale={v_scale} bf16={bf16}")
    case = make_gdn_case(200, 1, B=1, dist="model", bf16=bf16, seed=41, v_scale=v_scale)
    got = run_gpu(case, torch_gpu, mode=xqattn.GDN_CHUNKED)
    want = case.oracle_f64()
    v = _valid_rows(case)
    assert np.all(np.isfinite(got[:, :v]))
    rel = np.abs(got[:, :v] - want[:, :v]).max() / np.abs(want[:, :v]).max()
    print(f"v_scale={v_scale} bf16={bf16}: rel {rel:.2e}")
    assert rel <= 1e-4, rel


@pytest.mark.parametrize("mode,T", [(xqattn.GDN_STEP, 3), (xqattn.GDN_CHUNKED, 200)], ids=["step", "chunked"])
def test_gdn_graph_replays_match_eager(torch_gpu, mode, T):
    """A captured call (the step kernel, or the prep and scan launches of the
    chunked prefill, as the bench replays them) replays bit-identically, with
    the output cleared before each replay and eager calls between the replays."""
    torch = torch_gpu
    case_note(f"gdn graph replays mode {mode} T {T}")
    case = make_gdn_case(T, 3, B=2, dist="model", seed=23, bf16=True)
    dev = {n: xqattn.DevTensor.from_host(getattr(case, n)) for n in ("q", "k", "v", "g", "beta", "state")}
    dst = xqattn.DevTensor.from_host(case.dst)
    n_ws = xqattn.gated_delta_net_workspace(dev["q"], dev["v"], case.slots, mode)
    ws = torch.zeros(max(n_ws, 1) + 256, dtype=torch.uint8, device="cuda")

    def call():
        xqattn.gated_delta_net(dev["q"], dev["k"], dev["v"], dev["g"], dev["beta"], dev["state"], dst,
                               case.slots, mode=mode, workspace=ws)

    call()
    torch.cuda.synchronize()
    eager = dst.to_host_bytes().copy()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call()
    for rep in range(4):
        dst.t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dst.to_host_bytes(), eager), f"replay {rep} differs"
        call()  # eager work between the replays
        torch.cuda.synchronize()
    got = np.frombuffer(eager.tobytes(), np.float32).reshape(case.B, -1, 4096)
    want = case.oracle_f64()
    valid = T + 128 * min(T, case.slots)
    assert_close(got[:, :valid], want[:, :valid], what=f"graph case vs float64 (mode {mode})")
