"""GPU tests of the ggml-backend face (include/xq_ggml_backend.h): graphs of
FLASH_ATTN_EXT and GATED_DELTA_NET nodes run through xq_ggml_graph_compute in
graph order on the backend's stream, with the synchronous contract of the
reference backend (src/bridge/ggml_d3d12.cpp:1836-1942, synchronize = nullptr).

Each node's result must equal the direct C-ABI call on the same inputs bit for
bit (same kernels, same policy), and the oracle within the parity
tolerance (2e-3 abs / 1e-2 rel). A later node reads an earlier node's output
(the GDN state carried through a view of the first node's snapshot rows), a
node without the compute flag is skipped, and an unsupported node fails the
graph before anything is launched.
"""
import numpy as np
import pytest

import xqattn
from conftest import assert_close, case_note
from fa_cases import dst_array, make_fa_case, oracle_fa
from gdn_cases import SENTINEL, make_gdn_case, out_array
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu

FA_SMALL = wl.FaConfig("fa_verify_q4_0_nq8_h8kv2_d128_L1000_b2", 8, 8, 2, 128, 1000, 2, wl.Q4_0,
                       causal_prefix=992)


def _run(be, nodes, torch):
    # inputs were filled on torch's stream; the backend runs on its own
    torch.cuda.synchronize()
    be.graph_compute(nodes)


def _dev_gdn(case):
    return {n: xqattn.DevTensor.from_host(getattr(case, n)) for n in ("q", "k", "v", "g", "beta", "state")}


def _gdn_node(dev, dst, slots, compute=True):
    return xqattn.GgmlNode.gated_delta_net(dev["q"], dev["k"], dev["v"], dev["g"], dev["beta"], dev["state"],
                                           dst, slots, compute=compute)


def test_graph_fa_and_gdn_match_direct_calls(torch_gpu):
    case_note(f"ggml graph: noop + {FA_SMALL.name} + gdn step B=2")
    fa = make_fa_case(FA_SMALL, seed=31)
    q, k, v, m = (xqattn.DevTensor.from_host(t) for t in (fa.q, fa.k, fa.v, fa.mask))
    d_graph = xqattn.DevTensor.empty_like_host(fa.dst)
    d_direct = xqattn.DevTensor.empty_like_host(fa.dst)
    gdn = make_gdn_case(1, 1, B=2, dist="model", seed=5)
    dev = _dev_gdn(gdn)
    g_graph = xqattn.DevTensor.from_host(gdn.dst)
    g_direct = xqattn.DevTensor.from_host(gdn.dst)

    nodes = [xqattn.GgmlNode.noop(d_graph),
             xqattn.GgmlNode.flash_attn_ext(q, k, v, m, None, d_graph, fa.scale),
             _gdn_node(dev, g_graph, 1)]
    assert all(xqattn.ggml_supports_op(n) for n in nodes)
    with xqattn.GgmlBackend() as be:
        assert be.name == "XQ-MI355X"
        _run(be, nodes, torch_gpu)  # returns after completion: read without a sync
        got_fa = dst_array(fa, d_graph.to_host_bytes())
        got_gdn = out_array(gdn, g_graph.to_host_bytes())

    # the backend's consistent default runs the length-only split
    xqattn.flash_attn_ext(q, k, v, m, None, d_direct, xqattn.fa_params(fa.scale, split_mode=xqattn.SPLIT_LENGTH))
    xqattn.gated_delta_net(dev["q"], dev["k"], dev["v"], dev["g"], dev["beta"], dev["state"], g_direct, 1)
    torch_gpu.cuda.synchronize()
    assert np.array_equal(got_fa, dst_array(fa, d_direct.to_host_bytes()))
    assert np.array_equal(got_gdn, out_array(gdn, g_direct.to_host_bytes()))
    want_fa, _ = oracle_fa(fa)
    assert_close(got_fa, want_fa, what="graph FA vs oracle")
    assert_close(got_gdn, gdn.oracle(), what="graph GDN vs oracle")


def test_graph_orders_dependent_nodes(torch_gpu):
    """Two one-token GDN nodes, the second reading its state from the first
    node's final-state rows, equal one two-token node."""
    case_note("ggml graph: chained gdn steps T=1 -> T=1 vs T=2")
    two = make_gdn_case(2, 1, B=1, dist="model", seed=11)
    full = _dev_gdn(two)
    d_two = xqattn.DevTensor.from_host(two.dst)

    def token(t):  # token t of the two-token inputs as a one-token tensor (a view)
        out = {}
        for n in ("q", "k", "v", "g", "beta"):
            d = full[n]
            out[n] = xqattn.DevTensor(d.type, (d.ne[0], d.ne[1], 1, 1), (d.nb[0], d.nb[1], d.nb[2], d.nb[2]),
                                      d.t[t * d.nb[2]:(t + 1) * d.nb[2]])
        return out

    rows = 1 + 128
    first, second = token(0), token(1)
    first["state"] = full["state"]
    dst1 = xqattn.DevTensor(wl.F32, (4096, rows, 1, 1), (4, 16384, 16384 * rows, 16384 * rows),
                            torch_gpu.full((rows * 4096,), float(SENTINEL), device="cuda").view(torch_gpu.uint8))
    # the first node's final state (rows 1 .. 128) as the second node's state source
    second["state"] = xqattn.DevTensor(wl.F32, (128, 128, 32, 1), (4, 512, 65536, 2097152),
                                       dst1.t[16384:16384 + 2097152])
    dst2 = xqattn.DevTensor(wl.F32, (4096, rows, 1, 1), dst1.nb,
                            torch_gpu.full((rows * 4096,), float(SENTINEL), device="cuda").view(torch_gpu.uint8))
    with xqattn.GgmlBackend(gdn_mode=xqattn.GDN_STEP) as be:
        _run(be, [_gdn_node(first, dst1, 1), _gdn_node(second, dst2, 1), _gdn_node(full, d_two, 1)],
             torch_gpu)
    y1 = np.frombuffer(dst1.to_host_bytes().tobytes(), np.float32).reshape(rows, 4096)
    y2 = np.frombuffer(dst2.to_host_bytes().tobytes(), np.float32).reshape(rows, 4096)
    ref = out_array(two, d_two.to_host_bytes())[0]  # rows: y(t0), y(t1), final state
    assert np.array_equal(y1[0], ref[0])
    assert np.array_equal(y2[0], ref[1])
    assert np.array_equal(y2[1:], ref[2:])
    assert_close(ref[None], two.oracle(), what="T=2 vs oracle")


def test_graph_skips_non_compute_and_rejects_unsupported_before_launch(torch_gpu):
    case_note("ggml graph: skipped and rejected nodes")
    gdn = make_gdn_case(1, 1, B=1, dist="model", seed=17)
    dev = _dev_gdn(gdn)
    dst = xqattn.DevTensor.from_host(gdn.dst)
    sentinel = dst.to_host_bytes().copy()
    with xqattn.GgmlBackend() as be:
        _run(be, [_gdn_node(dev, dst, 1, compute=False)], torch_gpu)
        assert np.array_equal(dst.to_host_bytes(), sentinel)  # skipped
        with pytest.raises(xqattn.XqError) as e:
            _run(be, [_gdn_node(dev, dst, 1), xqattn.GgmlNode(xqattn.OP_OTHER, dst)], torch_gpu)
        assert e.value.status == 1 and "node 1" in str(e.value)
        assert np.array_equal(dst.to_host_bytes(), sentinel)  # nothing ran
        with pytest.raises(xqattn.XqError):
            _run(be, [xqattn.GgmlNode.gated_delta_net(dev["q"], dev["k"], dev["v"], dev["g"], dev["beta"],
                                                      dev["state"], dst, 1, raw_gates=1)], torch_gpu)
        assert np.array_equal(dst.to_host_bytes(), sentinel)
        _run(be, [_gdn_node(dev, dst, 1)], torch_gpu)
        assert_close(out_array(gdn, dst.to_host_bytes()), gdn.oracle(), what="after rejections")


def test_graph_workspace_grows_once(torch_gpu):
    """A chunked prefill node grows the backend's workspace to its need; a
    later graph that needs less runs in the same workspace."""
    case_note("ggml graph: chunked gdn T=130 then step")
    pre = make_gdn_case(130, 1, B=1, dist="model", seed=23, bf16=True)
    dev = _dev_gdn(pre)
    dst = xqattn.DevTensor.from_host(pre.dst)
    need = xqattn.gated_delta_net_workspace(dev["q"], dev["v"], 1)
    assert need > 0
    with xqattn.GgmlBackend() as be:
        assert be.workspace_bytes == 0
        _run(be, [_gdn_node(dev, dst, 1)], torch_gpu)
        assert be.workspace_bytes == need
        assert_close(out_array(pre, dst.to_host_bytes()), pre.oracle(), what="chunked node vs oracle")
        step = make_gdn_case(1, 1, B=2, dist="model", seed=29)
        sdev = _dev_gdn(step)
        sdst = xqattn.DevTensor.from_host(step.dst)
        _run(be, [_gdn_node(sdev, sdst, 1)], torch_gpu)
        assert be.workspace_bytes == need
        assert_close(out_array(step, sdst.to_host_bytes()), step.oracle(), what="step node vs oracle")


def test_graph_consistent_default_is_batch_invariant(torch_gpu):
    """Under the backend's defaults (consistent query policy, automatic split)
    a sequence's FA output is bitwise the same alone and in a batch of four:
    the split is the length-only partition (at 32k rows with 4 KV heads the
    batch-sized AUTO partition would give the lone sequence 64 splits and the
    batch 16)."""
    cfg = wl.FaConfig("fa_bi_q4_0_h16kv4_d128_L32768_b4", 2, 16, 4, 128, 32768, 4, wl.Q4_0, causal_prefix=32766)
    case_note(f"ggml graph: batch invariance {cfg.name}")
    assert xqattn.split_count(32768, xqattn.SPLIT_LENGTH) == 16
    fa = make_fa_case(cfg, seed=41, mask_per_seq=True)
    B, NQ, H, D = fa.shape
    rec = wl.record_bytes(wl.Q4_0, D)
    q, k, v, m = (xqattn.DevTensor.from_host(t) for t in (fa.q, fa.k, fa.v, fa.mask))
    d4 = xqattn.DevTensor.empty_like_host(fa.dst)
    b = 2
    q_all = np.frombuffer(fa.q.buf.tobytes(), np.float32).reshape(B, NQ, H, D)
    m_all = np.frombuffer(fa.mask.buf.tobytes(), np.uint16).reshape(B, fa.mask.ne[1], cfg.L)
    q1 = xqattn.DevTensor.from_host(wl.fa_q_tensor(q_all[b:b + 1].copy()))
    k1, v1 = (xqattn.DevTensor.from_host(wl.kv_tensor(t.buf.reshape(B, cfg.L, cfg.Hkv, rec)[b:b + 1].copy(),
                                                       wl.Q4_0, D)) for t in (fa.k, fa.v))
    m1 = xqattn.DevTensor.from_host(wl.mask_tensor(m_all[b:b + 1].copy()))
    d1 = xqattn.DevTensor.empty_like_host(wl.fa_dst_tensor(1, NQ, H, D))
    with xqattn.GgmlBackend() as be:
        _run(be, [xqattn.GgmlNode.flash_attn_ext(q, k, v, m, None, d4, fa.scale),
                  xqattn.GgmlNode.flash_attn_ext(q1, k1, v1, m1, None, d1, fa.scale)], torch_gpu)
    got4 = np.frombuffer(d4.to_host_bytes().tobytes(), np.float32).reshape(B, NQ, H, D)
    got1 = np.frombuffer(d1.to_host_bytes().tobytes(), np.float32).reshape(1, NQ, H, D)
    assert np.array_equal(got1[0].view(np.uint32), got4[b].view(np.uint32)), "sequence 2 alone differs"


def test_graph_gdn_min_tokens_two_leaves_single_token_nodes_to_the_cpu(torch_gpu):
    """With gdn_min_tokens = 2 (the reference's d3d12gdn.txt=2 hybrid) a
    single-token GDN node is outside the backend's contract: the graph fails
    before any launch; a two-token node runs."""
    case_note("ggml graph: gdn_min_tokens 2")
    one = make_gdn_case(1, 1, B=1, dist="model", seed=43)
    two = make_gdn_case(2, 1, B=1, dist="model", seed=44)
    d1, d2 = _dev_gdn(one), _dev_gdn(two)
    o1, o2 = xqattn.DevTensor.from_host(one.dst), xqattn.DevTensor.from_host(two.dst)
    sentinel = o1.to_host_bytes().copy()
    p = xqattn.backend_params(gdn_min_tokens=2)
    assert not xqattn.ggml_supports_op(_gdn_node(d1, o1, 1), p) and xqattn.ggml_supports_op(_gdn_node(d2, o2, 1), p)
    with xqattn.GgmlBackend(gdn_min_tokens=2) as be:
        with pytest.raises(xqattn.XqError) as e:
            _run(be, [_gdn_node(d2, o2, 1), _gdn_node(d1, o1, 1)], torch_gpu)
        assert e.value.status == 1 and "node 1" in str(e.value)
        assert np.array_equal(o1.to_host_bytes(), sentinel)
        _run(be, [_gdn_node(d2, o2, 1)], torch_gpu)
    assert_close(out_array(two, o2.to_host_bytes()), two.oracle(), what="T=2 node with min tokens 2")
