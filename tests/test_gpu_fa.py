"""GPU parity of GGML_OP_FLASH_ATTN_EXT (gfx950 kernels through the C ABI) against
the ggml-CPU restatement in oracle/, at the benchmark configurations' full sizes.

Tolerance (the ops' parity bar): max-abs 2e-3 / rel 1e-2 elementwise, f32 accumulation
on the GPU; ggml's CPU path accumulates F16 V in an f16 vector, so the F16
config is also compared with the float64 closed form as the tie-break.
"""
import dataclasses

import numpy as np
import pytest

import oracle
import xqattn
from conftest import assert_close, case_note
from fa_cases import dst_array, make_fa_case, oracle_f64, oracle_fa, run_fa_gpu
from xqattn import workloads as wl

pytestmark = pytest.mark.gpu


ENGINES = [xqattn.ENGINE_MFMA, xqattn.ENGINE_VALU]
ENGINE_IDS = ["mfma", "valu"]


def run_gpu(case, torch, qk_policy=xqattn.QK_CONSISTENT, split_mode=xqattn.SPLIT_AUTO, want_lse=True,
            engine=xqattn.ENGINE_AUTO):
    return run_fa_gpu(case, torch, qk_policy, split_mode, want_lse, engine)


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("cfg", [wl.FA_C1, wl.FA_C2, wl.FA_C5], ids=lambda c: c.name)
def test_fa_config_parity(torch_gpu, cfg, engine):
    case_note(f"flash_attn_ext {cfg.name} engine {engine}")
    case = make_fa_case(cfg, seed=11)
    got, glse = run_gpu(case, torch_gpu, engine=engine)
    want, wlse = oracle_fa(case)
    err = assert_close(got, want, what=f"{cfg.name} vs ggml-CPU restatement")
    ref64, lse64 = oracle_f64(case)
    err64 = assert_close(got, ref64, what=f"{cfg.name} vs float64 closed form")
    assert_close(glse, lse64, atol=1e-4, rtol=1e-5, what=f"{cfg.name} LSE")
    # f32 accumulation on both engines; the matrix-core engine's value
    # operands (weight, or weight x block scale) carry about 22 significant
    # bits as f16 hi + lo
    rel64 = err64 / float(np.abs(ref64).max())
    print(f"{cfg.name} engine {engine}: max|gpu-ggml|={err:.2e} max|gpu-f64|={err64:.2e} "
          f"(/ max|f64| {rel64:.2e})")
    assert rel64 < 1e-5, rel64


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("split_mode", [xqattn.SPLIT_REFERENCE, xqattn.SPLIT_FINE, xqattn.SPLIT_NONE,
                                        xqattn.SPLIT_BALANCED, xqattn.SPLIT_COARSE, xqattn.SPLIT_MQ_BALANCED,
                                        xqattn.SPLIT_MQ_FINE])
def test_fa_split_modes(torch_gpu, split_mode, engine):
    cfg = wl.FaConfig("q8_split", 1, 24, 4, 256, 5000, 2, wl.Q8_0)
    case_note(f"split mode {split_mode} engine {engine}")
    case = make_fa_case(cfg, seed=3)
    got, _ = run_gpu(case, torch_gpu, split_mode=split_mode, engine=engine)
    ref64, _ = oracle_f64(case)
    assert_close(got, ref64, atol=1e-4, rtol=1e-4, what=f"split {split_mode}")
    again, _ = run_gpu(case, torch_gpu, split_mode=split_mode, engine=engine)
    assert np.array_equal(got, again), "not deterministic"


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2])
@pytest.mark.parametrize("D,H,Hkv", [(128, 32, 8), (256, 24, 4), (128, 16, 16)])
def test_fa_query_width_invariance(torch_gpu, kv_type, D, H, Hkv, engine):
    """A query's result is bitwise the same alone (n_q = 1) or inside an n_q <= 8 batch."""
    cfg = wl.FaConfig("inv", 8, H, Hkv, D, 1000, 2, kv_type, causal_prefix=992)
    case_note(f"invariance {wl.TYPE_NAME[kv_type]} D{D} H{H}/{Hkv}")
    case = make_fa_case(cfg, seed=5)
    batch, _ = run_gpu(case, torch_gpu, engine=engine)
    q_all = np.frombuffer(case.q.buf.tobytes(), np.float32).reshape(2, 8, H, D)
    m_all = np.frombuffer(case.mask.buf.tobytes(), np.uint16).reshape(1, 8, 1000)
    cfg1 = wl.FaConfig("inv1", 1, H, Hkv, D, 1000, 2, kv_type)
    for i in (0, 3, 7):
        single = dataclasses.replace(case, cfg=cfg1, q=wl.fa_q_tensor(q_all[:, i:i + 1].copy()),
                                     mask=wl.mask_tensor(m_all[:, i:i + 1].copy()),
                                     dst=wl.fa_dst_tensor(2, 1, H, D))
        one, _ = run_gpu(single, torch_gpu, engine=engine)
        assert np.array_equal(one[:, 0], batch[:, i]), f"query {i} differs between n_q=1 and n_q=8"


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
def test_fa_padding_rows_and_fully_masked(torch_gpu, engine):
    """Extra query rows whose mask rows are all -inf produce 0 and LSE -inf."""
    cfg = wl.FaConfig("pad", 10, 32, 8, 128, 700, 2, wl.Q4_0, causal_prefix=692, n_q_pad=16)
    case = make_fa_case(cfg, seed=9)
    m = wl.fa_causal_mask(cfg, n_q_rows=8)  # rows 8..15 all -inf
    case.mask = wl.mask_tensor(m)
    got, lse = run_gpu(case, torch_gpu, engine=engine)
    want, wlse = oracle_fa(case)
    assert np.all(got[:, 8:] == 0.0)
    assert np.all(np.isneginf(lse[:, 8:]))
    assert_close(got, want, what="padded verify")


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2])
def test_fa_sinks_softcap_alibi(torch_gpu, kv_type, engine):
    cfg = wl.FaConfig("feat", 3, 12, 4, 128, 900, 2, kv_type, causal_prefix=897)
    case = make_fa_case(cfg, seed=21, sinks=True, softcap=30.0, max_bias=8.0, mask_per_seq=True)
    got, glse = run_gpu(case, torch_gpu, engine=engine)
    want, wlse = oracle_fa(case)
    assert_close(got, want, what="sinks+softcap+alibi vs ggml restatement")
    ref64, lse64 = oracle_f64(case)
    assert_close(got, ref64, what="sinks+softcap+alibi vs f64")
    assert_close(glse, lse64, atol=1e-4, rtol=1e-5, what="lse")


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
def test_fa_native_policy_f16(torch_gpu, engine):
    cfg = wl.FaConfig("native", 2, 16, 8, 128, 1500, 1, wl.F16, causal_prefix=1498)
    case = make_fa_case(cfg, seed=4)
    got, _ = run_gpu(case, torch_gpu, qk_policy=xqattn.QK_NATIVE, engine=engine)
    want, _ = oracle_fa(case, policy=oracle.QK_NATIVE)
    assert_close(got, want, what="native f16 policy")
    ref64, _ = oracle_f64(case, policy=oracle.QK_NATIVE, q_round=True)
    tol = 1e-5 if engine == xqattn.ENGINE_VALU else 5e-4
    assert_close(got, ref64, atol=tol, rtol=1e-4, what="native f16 vs f64 (f16-rounded Q)")


@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2])
@pytest.mark.parametrize("D", [128, 256])
def test_kv_store_bit_exact(torch_gpu, kv_type, D):
    """GPU KV append quantizers are bit-identical to ggml's (oracle restatement)."""
    torch = torch_gpu
    n_tok, hkv, cap = 37, 4, 64
    x = wl.normal(77, (n_tok, hkv, D)) * np.float32(3.0)
    x[0, 0, :5] = [0.0, -0.0, 65504.0, 1e-8, -7.5]       # edge values
    x[1, 1, :] = 0.0                                        # all-zero block -> d = 0
    pos = np.array([(5 * i + 3) % cap for i in range(n_tok)], np.int32)
    pos[-1] = cap + 5                                        # out of range: skipped
    rec = wl.record_bytes(kv_type, D)
    for variant in (0, 1) if kv_type == wl.Q8_0 else (0,):
        want = np.zeros((cap, hkv, rec), np.uint8)
        oracle.kv_store(x, pos, hkv, D, kv_type, want, cap, variant)
        dst = torch.zeros(cap * hkv * rec, dtype=torch.uint8, device="cuda")
        xqattn.kv_store(torch.from_numpy(x).cuda(), torch.from_numpy(pos).cuda(), hkv, D, kv_type, dst, cap,
                        q8_variant=variant)
        torch.cuda.synchronize()
        got = dst.cpu().numpy().reshape(cap, hkv, rec)
        assert np.array_equal(got, want), f"kv_store {wl.TYPE_NAME[kv_type]} D{D} variant {variant}"


@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0])
@pytest.mark.parametrize("active", [0, 1, 64, 257, 4096])
def test_fa_range_vs_reference_semantics(torch_gpu, kv_type, active):
    """attend_range: causal limits from positions/origin, empty -> O=0, LSE=-inf."""
    torch = torch_gpu
    n_head, hkv, D, origin = 24, 4, 256, 102400
    cap = max(active, 1)
    kf = wl.normal(31, (cap, hkv, D))
    vf = wl.normal(32, (cap, hkv, D))
    kraw = oracle.quantize(kv_type, kf)
    vraw = oracle.quantize(kv_type, vf)
    positions = np.array([origin + active - 1, origin - 5, origin + active // 2, origin + active + 100], np.int32)
    q = wl.normal(33, (4, n_head, D))
    scale = 1.0 / 16
    split_k = oracle.load().xo_ref_split_k(active)
    want, wlse, _ = oracle.range_attn(q, positions, n_head, kraw, vraw, hkv, D, kv_type, origin, active, scale, split_k)
    out = torch.empty(4 * n_head * D, dtype=torch.float32, device="cuda")
    lse = torch.empty(4 * n_head, dtype=torch.float32, device="cuda")
    xqattn.fa_range(torch.from_numpy(q).cuda(), torch.from_numpy(positions).cuda(), n_head,
                    torch.from_numpy(kraw.reshape(-1)).cuda(), torch.from_numpy(vraw.reshape(-1)).cuda(),
                    hkv, D, kv_type, origin, active, scale, out, lse)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(4, n_head, D)
    glse = lse.cpu().numpy().reshape(4, n_head)
    # reference GPU tolerance: 3e-4 + 3e-4|ref| (O), 3e-4 + 3e-5|ref| (LSE)
    assert_close(got, want, atol=3e-4, rtol=3e-4, what="range O")
    assert_close(glse, wlse, atol=3e-4, rtol=3e-5, what="range LSE")
    assert np.all(got[1] == 0.0) and np.all(np.isneginf(glse[1])), "query before origin must be empty"


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0])
def test_fa_mask_rows_2byte_aligned(torch_gpu, kv_type, engine):
    """An odd KV length gives mask rows of 2 (mod 4) bytes; a mask view may also
    start 2 bytes into its buffer. Both run (the matrix-core engine re-lays such
    a mask in the workspace first) and give the aligned layout's result."""
    torch = torch_gpu
    cfg = wl.FaConfig("odd", 4, 16, 4, 128, 1001, 2, kv_type, causal_prefix=997)
    case_note(f"odd mask rows {wl.TYPE_NAME[kv_type]} engine {engine}")
    case = make_fa_case(cfg, seed=41, mask_per_seq=True)
    assert case.mask.nb[1] % 4 == 2
    got, glse = run_gpu(case, torch, engine=engine)
    want, _ = oracle_fa(case)
    assert_close(got, want, what="odd-length mask vs ggml restatement")
    ref64, lse64 = oracle_f64(case)
    assert_close(glse, lse64, atol=1e-4, rtol=1e-5, what="odd-length mask LSE")

    cfg2 = wl.FaConfig("even", 4, 16, 4, 128, 1000, 2, kv_type, causal_prefix=996)
    case2 = make_fa_case(cfg2, seed=43)
    aligned, _ = run_gpu(case2, torch, engine=engine)
    q, k, v = (xqattn.DevTensor.from_host(t) for t in (case2.q, case2.k, case2.v))
    raw = np.concatenate([np.zeros(2, np.uint8), case2.mask.buf.reshape(-1)])
    m = xqattn.DevTensor(case2.mask.type, case2.mask.ne, case2.mask.nb, torch.from_numpy(raw).cuda()[2:])
    assert m.t.data_ptr() % 4 == 2
    d = xqattn.DevTensor.empty_like_host(case2.dst)
    xqattn.flash_attn_ext(q, k, v, m, None, d, xqattn.fa_params(case2.scale, engine=engine))
    torch.cuda.synchronize()
    assert np.array_equal(dst_array(case2, d.to_host_bytes()), aligned), "mask pointer offset changed the result"


@pytest.mark.parametrize("engine", ENGINES, ids=ENGINE_IDS)
def test_fa_empty_trailing_split(torch_gpu, engine):
    """The reference's fine mode keeps 256 splits at 10200 rows (40 rows each), so
    the last split is empty; its partial state must merge as nothing."""
    assert xqattn.split_count(10200, xqattn.SPLIT_FINE) == 256
    assert xqattn.split_rows(10200, xqattn.SPLIT_FINE) * 255 >= 10200
    cfg = wl.FaConfig("q8_empty_split", 1, 8, 2, 128, 10200, 1, wl.Q8_0)
    case_note(f"empty trailing split engine {engine}")
    case = make_fa_case(cfg, seed=13)
    got, glse = run_gpu(case, torch_gpu, split_mode=xqattn.SPLIT_FINE, engine=engine)
    ref64, lse64 = oracle_f64(case)
    assert_close(got, ref64, atol=5e-4, rtol=5e-4, what="empty trailing split")
    assert_close(glse, lse64, atol=1e-4, rtol=1e-5, what="empty trailing split LSE")


def test_fa_graph_replays_match_eager(torch_gpu):
    """A captured multi-split call (pass 1, then the split merge on the same
    stream) replays bit-identically, with eager calls between the replays."""
    torch = torch_gpu
    cfg = wl.FaConfig("q8_graph", 1, 24, 4, 256, 6000, 2, wl.Q8_0)
    case_note("graph replays")
    case = make_fa_case(cfg, seed=17)
    q, k, v = (xqattn.DevTensor.from_host(t) for t in (case.q, case.k, case.v))
    m = xqattn.DevTensor.from_host(case.mask)
    d = xqattn.DevTensor.empty_like_host(case.dst)
    p = xqattn.fa_params(case.scale)
    ws = torch.zeros(xqattn.flash_attn_ext_workspace(q, k, v, m, None, d, p) + 256, dtype=torch.uint8,
                     device="cuda")
    xqattn.flash_attn_ext(q, k, v, m, None, d, p, workspace=ws)
    torch.cuda.synchronize()
    eager = d.to_host_bytes().copy()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        xqattn.flash_attn_ext(q, k, v, m, None, d, p, workspace=ws)
    for rep in range(4):
        d.t.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(d.to_host_bytes(), eager), f"replay {rep} differs"
        xqattn.flash_attn_ext(q, k, v, m, None, d, p, workspace=ws)  # eager work between replays
        torch.cuda.synchronize()


def test_lse_merge_matches_oracle(torch_gpu):
    """xq_fa_lse_merge against the oracle's merge: empty pieces (LSE -inf, their
    O never read), a row no piece sees, and poisoned rows (NaN LSE, NaN value)."""
    torch = torch_gpu
    rng = np.random.default_rng(11)
    n_parts, rows, D = 6, 200, 256
    po = rng.standard_normal((n_parts, rows, D)).astype(np.float32)
    pl = (rng.standard_normal((n_parts, rows)) * 10).astype(np.float32)
    pl[2, ::4] = -np.inf
    po[2, ::4] = np.inf
    pl[:, 9] = -np.inf
    pl[3, 11] = np.nan
    po[4, 13, 7] = np.nan
    want, wlse = oracle.lse_merge(po, pl)
    case_note("lse merge vs oracle")
    out = torch.empty(rows, D, dtype=torch.float32, device="cuda")
    lse = torch.empty(rows, dtype=torch.float32, device="cuda")
    xqattn.fa_lse_merge(torch.from_numpy(po).cuda(), torch.from_numpy(pl).cuda(), out, lse)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, atol=1e-6, rtol=1e-6, what="merged O")
    assert_close(lse.cpu().numpy(), wlse, atol=1e-6, rtol=1e-6, what="merged LSE")


@pytest.mark.parametrize("kv_type", [wl.F16, wl.Q8_0, wl.Q4_0])
def test_range_pieces_merged_equal_whole_range(torch_gpu, kv_type):
    """Range attention over two pieces of the KV rows (the second with its origin
    moved by the cut), merged with xq_fa_lse_merge, equals range attention over
    all rows: the exchange a split of the KV rows across devices needs."""
    torch = torch_gpu
    n_head, hkv, D, origin, active, cut = 24, 4, 256, 102400, 5000, 1777
    kraw = oracle.quantize(kv_type, wl.normal(71, (active, hkv, D)))
    vraw = oracle.quantize(kv_type, wl.normal(72, (active, hkv, D)))
    positions = np.array([origin + active - 1, origin + 1000, origin - 5, origin + 3000], np.int32)
    q = wl.normal(73, (positions.size, n_head, D))
    n_q = positions.size
    dq, dpos = torch.from_numpy(q).cuda(), torch.from_numpy(positions).cuda()
    kd, vd = torch.from_numpy(kraw).cuda(), torch.from_numpy(vraw).cuda()

    def run(a, b):
        out = torch.empty(n_q * n_head * D, dtype=torch.float32, device="cuda")
        lse = torch.empty(n_q * n_head, dtype=torch.float32, device="cuda")
        xqattn.fa_range(dq, dpos, n_head, kd[a:b].contiguous().reshape(-1), vd[a:b].contiguous().reshape(-1),
                        hkv, D, kv_type, origin + a, b - a, 1.0 / 16, out, lse)
        return out.reshape(n_q * n_head, D), lse

    case_note(f"range pieces + merge {wl.TYPE_NAME[kv_type]}")
    whole, wlse = run(0, active)
    p0, l0 = run(0, cut)
    p1, l1 = run(cut, active)
    out = torch.empty(n_q * n_head, D, dtype=torch.float32, device="cuda")
    lse = torch.empty(n_q * n_head, dtype=torch.float32, device="cuda")
    xqattn.fa_lse_merge(torch.stack([p0, p1]), torch.stack([l0, l1]), out, lse)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), whole.cpu().numpy(), atol=1e-4, rtol=1e-4, what="merged pieces vs whole")
    assert_close(lse.cpu().numpy(), wlse.cpu().numpy(), atol=1e-5, rtol=1e-6, what="merged LSE vs whole")
