"""The ggml-backend face of the library on the host (no GPU calls): the node
descriptor's layout, op_params packing as ggml's graph constructors write it,
and the pure supports_op predicate (src/bridge/ggml_d3d12.cpp:2331-2353 for
the predicate's role, :77-109 for the GDN operand rules)."""
import ctypes
import struct

import pytest

import xqattn
from test_cpu_abi import _desc, _fa_descs
from xqattn import workloads as wl


def test_node_struct_layout():
    # int32 op, int32 flags, 16 int32 op_params, xq_tensor dst (80 bytes), 10 pointers
    assert ctypes.sizeof(xqattn.XqTensor) == 4 + 4 + 32 + 32 + 8
    assert xqattn.XqGgmlNode.dst.offset == 4 + 4 + 64
    assert xqattn.XqGgmlNode.src.offset == 72 + 80
    assert ctypes.sizeof(xqattn.XqGgmlNode) == 72 + 80 + 80
    assert ctypes.sizeof(xqattn.XqGgmlBackendParams) == 32


def test_fa_op_params_are_ggml_float_bits():
    q, k, v, m, dst = _fa_descs()
    n = xqattn.GgmlNode.flash_attn_ext(q, k, v, m, None, dst, 1 / 16, max_bias=8.0, softcap=30.0, prec=10)
    st = n.struct()
    words = list(st.op_params)
    assert words[:4] == [struct.unpack("<i", struct.pack("<f", x))[0] for x in (1 / 16, 8.0, 30.0)] + [10]
    assert words[4:] == [0] * 12
    assert st.op == xqattn.OP_FLASH_ATTN_EXT and st.flags == xqattn.GGML_FLAG_COMPUTE
    assert bool(st.src[3]) and not bool(st.src[4]) and not bool(st.src[5])
    assert st.src[1].contents.type == wl.Q8_0 and st.src[1].contents.ne[1] == 32768


@pytest.mark.parametrize("kv", [wl.F16, wl.Q8_0, wl.Q4_0, wl.E5M2])
def test_supports_op_fa_matches_direct_predicate(kv):
    for D in (128, 256):
        q, k, v, m, dst = _fa_descs(kv=kv, D=D)
        node = xqattn.GgmlNode.flash_attn_ext(q, k, v, m, None, dst, 1 / 16)
        assert xqattn.ggml_supports_op(node)
        # a sixth source is not part of FLASH_ATTN_EXT's contract
        node.srcs.append(m)
        assert not xqattn.ggml_supports_op(node)
    q, k, v, m, dst = _fa_descs(D=64)  # head dim outside the kernels
    assert not xqattn.ggml_supports_op(xqattn.GgmlNode.flash_attn_ext(q, k, v, m, None, dst, 0.125))
    q, k, v, m, dst = _fa_descs()
    assert not xqattn.ggml_supports_op(xqattn.GgmlNode.flash_attn_ext(None, k, v, m, None, dst, 0.125))


def _gdn_descs(T=1, B=8, slots=1):
    q = _desc(wl.F32, (128, 16, T, B))
    k = _desc(wl.F32, (128, 16, T, B))
    v = _desc(wl.F32, (128, 32, T, B))
    g = _desc(wl.F32, (1, 32, T, B))
    beta = _desc(wl.F32, (1, 32, T, B))
    s = _desc(wl.F32, (128, 128, 32, B))
    dst = _desc(wl.F32, (4096, T + slots * 128, B, 1))
    return q, k, v, g, beta, s, dst


def test_supports_op_gdn_contract():
    q, k, v, g, beta, s, dst = _gdn_descs()
    ok = xqattn.GgmlNode.gated_delta_net(q, k, v, g, beta, s, dst, 1)
    assert xqattn.ggml_supports_op(ok)
    assert list(ok.struct().op_params[:2]) == [1, 0]
    assert not xqattn.ggml_supports_op(xqattn.GgmlNode.gated_delta_net(q, k, v, g, beta, s, dst, 1, raw_gates=1))
    q5, k5, v5, g5, b5, s5, d5 = _gdn_descs(T=5, B=1, slots=5)
    assert xqattn.ggml_supports_op(xqattn.GgmlNode.gated_delta_net(q5, k5, v5, g5, b5, s5, d5, 5))
    q18, k18, v18, g18, b18, s18, d18 = _gdn_descs(T=1, B=1, slots=18)
    assert not xqattn.ggml_supports_op(xqattn.GgmlNode.gated_delta_net(q18, k18, v18, g18, b18, s18, d18, 18))
    # the rows-indexed mode (src[6..8]) is outside the contract
    rows = xqattn.GgmlNode.gated_delta_net(q, k, v, g, beta, s, dst, 1)
    rows.srcs += [q]
    assert not xqattn.ggml_supports_op(rows)
    missing = xqattn.GgmlNode.gated_delta_net(q, k, v, g, beta, None, dst, 1)
    assert not xqattn.ggml_supports_op(missing)


def test_supports_op_noop_and_other_kinds():
    dst = _desc(wl.F32, (4096, 1, 1, 1))
    assert xqattn.ggml_supports_op(xqattn.GgmlNode.noop(dst))
    assert not xqattn.ggml_supports_op(xqattn.GgmlNode(xqattn.OP_OTHER, dst))
    assert not xqattn.ggml_supports_op(xqattn.GgmlNode(7, dst))
    assert xqattn.load().xq_ggml_supports_op(None) == 0


def test_c_header_layout_matches_ctypes(tmp_path):
    """The C declarations of include/xq_ggml_backend.h, compiled by the host C
    compiler, have the field offsets the ctypes mirror uses."""
    import shutil
    import subprocess
    from conftest import ROOT
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    src = tmp_path / "layout.c"
    src.write_text("""
#include <stddef.h>
#include <stdio.h>
#include "xq_ggml_backend.h"
int main(void) {
    printf("%zu %zu %zu %zu %zu %zu %zu\\n", sizeof(xq_tensor), offsetof(xq_ggml_node, op_params),
           offsetof(xq_ggml_node, dst), offsetof(xq_ggml_node, src), sizeof(xq_ggml_node),
           sizeof(xq_ggml_backend_params), sizeof(xq_fa_params));
    return 0;
}
""")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [ctypes.sizeof(xqattn.XqTensor), xqattn.XqGgmlNode.op_params.offset, xqattn.XqGgmlNode.dst.offset,
            xqattn.XqGgmlNode.src.offset, ctypes.sizeof(xqattn.XqGgmlNode),
            ctypes.sizeof(xqattn.XqGgmlBackendParams), ctypes.sizeof(xqattn.XqFaParams)]
    assert got == want


def test_gdn_contract_flips_of_the_reference_test():
    """The reference's own flip sequence on one T = 3, slots = 5 node
    (tests/test_ggml_d3d12.cpp:238-271), each flip undone before the next:
    rows-indexed src[6], raw gates, 18 slots, the KDA vector gate
    g->ne[0] = 128, F16 q, a q row stride that is not float-aligned, and a
    sequence count that differs between operands; the restored node is
    supported again. Each flip is checked through the ggml face and, where it is
    an operand flip, through the direct predicate."""
    T, slots = 3, 5
    q, k, v, g, beta, s, dst = _gdn_descs(T=T, B=1, slots=slots)
    assert (dst.ne[0], dst.ne[1]) == (4096, T + slots * 128)

    def node(**kw):
        return xqattn.GgmlNode.gated_delta_net(q, k, v, g, beta, s, dst, kw.get("slots", slots),
                                               raw_gates=kw.get("raw", 0))

    def direct(sl=slots, raw=0):
        return bool(xqattn.load().xq_supports_gated_delta_net(
            *(ctypes.byref(x) for x in (q, k, v, g, beta, s, dst)), sl, raw))

    assert xqattn.ggml_supports_op(node()) and direct()
    n = node()
    n.srcs += [q]  # src[6]: rows-indexed mode
    assert not xqattn.ggml_supports_op(n)
    assert not xqattn.ggml_supports_op(node(raw=1)) and not direct(raw=1)
    assert not direct(sl=18)
    g.ne[0] = 128  # KDA vector gate
    assert not xqattn.ggml_supports_op(node()) and not direct()
    g.ne[0] = 1
    q.type = wl.F16
    assert not xqattn.ggml_supports_op(node()) and not direct()
    q.type = wl.F32
    q.nb[1] += 1  # cannot be expressed in float indices
    assert not xqattn.ggml_supports_op(node()) and not direct()
    q.nb[1] -= 1
    v.ne[3] = 2
    assert not xqattn.ggml_supports_op(node()) and not direct()
    v.ne[3] = 1
    assert xqattn.ggml_supports_op(node()) and direct()


def test_gdn_min_tokens_hybrid_cpu_t1_gpu_t2():
    """The reference's width cases (tests/test_ggml_d3d12.cpp:273-285): T = 1 and
    T = 2 nodes (5 slots) both satisfy the full contract with the default
    minimum; with gdn_min_tokens = 2 (d3d12_set_gdn_enabled(true, 2), the
    d3d12gdn.txt=2 hybrid) only T = 2 runs here and T = 1 stays on the CPU.
    Values other than 2 mean 1, as the reference's setter maps them."""
    for tokens in (1, 2):
        q, k, v, g, beta, s, dst = _gdn_descs(T=tokens, B=1, slots=5)
        node = xqattn.GgmlNode.gated_delta_net(q, k, v, g, beta, s, dst, 5)
        assert xqattn.ggml_supports_op(node)
        assert xqattn.ggml_supports_op(node, xqattn.backend_params(gdn_min_tokens=1))
        assert xqattn.ggml_supports_op(node, xqattn.backend_params(gdn_min_tokens=2)) == (tokens == 2)
        for other in (0, 3, -1):
            assert xqattn.ggml_supports_op(node, xqattn.backend_params(gdn_min_tokens=other))


def test_supports_op_params_rejects_bad_params():
    q, k, v, g, beta, s, dst = _gdn_descs(T=2, B=1, slots=1)
    node = xqattn.GgmlNode.gated_delta_net(q, k, v, g, beta, s, dst, 1)
    assert xqattn.ggml_supports_op(node, xqattn.backend_params())
    assert not xqattn.ggml_supports_op(node, xqattn.backend_params(gdn_mode=7))
    assert not xqattn.ggml_supports_op(node, xqattn.backend_params(fa_split_mode=9))


@pytest.mark.parametrize("env,want", [
    ({}, (xqattn.QK_NATIVE, xqattn.SPLIT_BALANCED)),  # absent: unchanged
    ({"GGML_FLASH_ATTN_NO_QUERY_TILING": "4"}, (xqattn.QK_CONSISTENT, xqattn.SPLIT_BALANCED)),
    ({"GGML_FLASH_ATTN_NO_QUERY_TILING": "1"}, (xqattn.QK_NATIVE, xqattn.SPLIT_BALANCED)),
    ({"GGML_FLASH_ATTN_NO_QUERY_TILING": "4 "}, (xqattn.QK_NATIVE, xqattn.SPLIT_BALANCED)),  # exact values only
    ({"GGML_FLASH_ATTN_NO_SPLIT_KV": "1"}, (xqattn.QK_NATIVE, xqattn.SPLIT_LENGTH)),
    ({"GGML_FLASH_ATTN_NO_SPLIT_KV": "0"}, (xqattn.QK_NATIVE, xqattn.SPLIT_BALANCED)),
    ({"GGML_FLASH_ATTN_NO_SPLIT_KV": "11"}, (xqattn.QK_NATIVE, xqattn.SPLIT_BALANCED)),
    # flashattn.txt=2 (uwp/inference-bridge.cpp:887-893) sets both
    ({"GGML_FLASH_ATTN_NO_QUERY_TILING": "4", "GGML_FLASH_ATTN_NO_SPLIT_KV": "1"},
     (xqattn.QK_CONSISTENT, xqattn.SPLIT_LENGTH)),
])
def test_fa_params_from_env_knob_semantics(monkeypatch, env, want):
    """ggml's strict parse of the two knobs (patches/0006-…:9-10,
    patches/0008-…:7-8,46-50): exactly "4" / "1" and exactly "1"."""
    for name in ("GGML_FLASH_ATTN_NO_QUERY_TILING", "GGML_FLASH_ATTN_NO_SPLIT_KV"):
        monkeypatch.delenv(name, raising=False)
    for name, val in env.items():
        monkeypatch.setenv(name, val)
    p = xqattn.fa_params(1 / 16, qk_policy=xqattn.QK_NATIVE, split_mode=xqattn.SPLIT_BALANCED)
    xqattn.fa_params_from_env(p)
    assert (p.qk_policy, p.split_mode) == want
    assert p.scale == pytest.approx(1 / 16) and p.engine == xqattn.ENGINE_AUTO
