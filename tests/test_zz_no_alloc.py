"""xq_flash_attn_ext_noalloc: the flash-attention entry point that allocates
nothing (its workspace is the library's per-GPU scratch array). It must give
xq_flash_attn_ext's results bit for bit, on consecutive calls that reuse the
scratch (the second smaller than the first), and reject a call whose workspace
exceeds the scratch before launching anything. Its callers capture HIP graphs:
the process's first call (which looks the scratch address up) is made under
capture, and the graph's replays equal the workspace entry's result bit for
bit, with eager calls between the replays. The capture test comes first in
this file so that it makes the first call of its process.
"""
import ctypes

import numpy as np
import pytest

import xqattn
from conftest import case_note
from fa_cases import dst_array, make_fa_case, run_fa_gpu
from test_cpu_abi import _fa_descs
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _run_noalloc(case, torch, split_mode, engine):
    q, k, v = (xqattn.DevTensor.from_host(t) for t in (case.q, case.k, case.v))
    m = xqattn.DevTensor.from_host(case.mask) if case.mask is not None else None
    d = xqattn.DevTensor.empty_like_host(case.dst)
    B, NQ, H, D = case.shape
    lse = torch.empty(B * NQ * H, dtype=torch.float32, device="cuda")
    p = xqattn.fa_params(case.scale, split_mode=split_mode, engine=engine)
    xqattn.flash_attn_ext_noalloc(q, k, v, m, None, d, p, lse=lse)
    torch.cuda.synchronize()
    return dst_array(case, d.to_host_bytes()), lse.cpu().numpy().reshape(B, NQ, H)


def test_fa_noalloc_first_call_under_graph_capture_replays_bit_exact(torch_gpu):
    torch = torch_gpu
    cfg = wl.FaConfig("na_graph", 2, 24, 4, 256, 5000, 2, wl.Q8_0, causal_prefix=4998)
    case_note("no-alloc call under graph capture")
    case = make_fa_case(cfg, seed=19)
    want, wlse = run_fa_gpu(case, torch, split_mode=xqattn.SPLIT_AUTO, engine=xqattn.ENGINE_AUTO)
    q, k, v = (xqattn.DevTensor.from_host(t) for t in (case.q, case.k, case.v))
    m = xqattn.DevTensor.from_host(case.mask)
    d = xqattn.DevTensor.empty_like_host(case.dst)
    B, NQ, H, D = case.shape
    lse = torch.empty(B * NQ * H, dtype=torch.float32, device="cuda")
    p = xqattn.fa_params(case.scale)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        xqattn.flash_attn_ext_noalloc(q, k, v, m, None, d, p, lse=lse, stream=s)
    for rep in range(4):
        d.t.zero_()
        lse.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = dst_array(case, d.to_host_bytes())
        glse = lse.cpu().numpy().reshape(B, NQ, H)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}: output differs"
        assert np.array_equal(glse.view(np.uint32), wlse.view(np.uint32)), f"replay {rep}: LSE differs"
        xqattn.flash_attn_ext_noalloc(q, k, v, m, None, d, p, lse=lse)  # eager work on the same scratch
        torch.cuda.synchronize()


CALLS = [
    # (config, split mode, engine): the first call's workspace is the largest
    (wl.FaConfig("na_q8", 3, 24, 4, 256, 6000, 2, wl.Q8_0, causal_prefix=5997), xqattn.SPLIT_FINE,
     xqattn.ENGINE_MFMA),
    (wl.FaConfig("na_f16_odd", 1, 16, 8, 128, 1001, 1, wl.F16), xqattn.SPLIT_AUTO, xqattn.ENGINE_MFMA),
    (wl.FaConfig("na_q4_valu", 2, 8, 2, 128, 700, 1, wl.Q4_0, causal_prefix=698), xqattn.SPLIT_REFERENCE,
     xqattn.ENGINE_VALU),
]


def test_fa_noalloc_matches_workspace_entry_on_consecutive_calls(torch_gpu):
    sizes = []
    for i, (cfg, split_mode, engine) in enumerate(CALLS):
        case_note(f"no-alloc call {i}: {cfg.name} split {split_mode} engine {engine}")
        case = make_fa_case(cfg, seed=50 + i)
        q, k, v = (xqattn.DevTensor.from_host(t) for t in (case.q, case.k, case.v))
        m = xqattn.DevTensor.from_host(case.mask) if case.mask is not None else None
        d = xqattn.DevTensor.empty_like_host(case.dst)
        sizes.append(xqattn.flash_attn_ext_workspace(q, k, v, m, None, d,
                                                     xqattn.fa_params(case.scale, split_mode=split_mode,
                                                                      engine=engine)))
        want, wlse = run_fa_gpu(case, torch_gpu, split_mode=split_mode, engine=engine)
        got, glse = _run_noalloc(case, torch_gpu, split_mode, engine)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {i}: output differs"
        assert np.array_equal(glse.view(np.uint32), wlse.view(np.uint32)), f"call {i}: LSE differs"
    assert sizes[0] > sizes[1] and sizes[0] > sizes[2], sizes  # later calls reuse a part of the scratch


def test_fa_noalloc_rejects_a_workspace_beyond_the_scratch(torch_gpu):
    """256 (query, head) rows x 256 splits x 256 dims of f32 partials is 64 MiB:
    the call is refused with XQ_ERR_WORKSPACE before any launch."""
    q, k, v, m, dst = _fa_descs(kv=wl.Q8_0, D=256, NQ=8, H=32, Hkv=8, L=16384, B=1)
    p = xqattn.fa_params(1 / 16, split_mode=xqattn.SPLIT_FINE)
    lib = xqattn.load()
    refs = [ctypes.byref(x) for x in (q, k, v, m)]
    n = ctypes.c_size_t(0)
    assert lib.xq_flash_attn_ext_workspace(*refs, None, ctypes.byref(dst), ctypes.byref(p), ctypes.byref(n)) == 0
    assert n.value > SCRATCH_BYTES
    st = lib.xq_flash_attn_ext_noalloc(*refs, None, ctypes.byref(dst), None, ctypes.byref(p), None)
    assert st == 4 and b"scratch" in lib.xq_last_error()
