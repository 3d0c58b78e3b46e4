"""XFA1 capture replay on the GPU: a capture of each multi-query golden fixture
(permuted Q, K/V as views into a larger cache with junk in the gap rows) run
through xq_flash_attn_ext via xqattn.xfa1.replay, against the captured output
(the oracle's ggml-loop result) and the float64 closed form, at the parity
tolerance 2e-3 abs / 1e-2 rel.
"""
import pytest

import golden_io as gio
import xqattn
from conftest import assert_close, case_note
from xqattn import xfa1

pytestmark = pytest.mark.gpu

CASES = gio.fixture_paths("fa_verify")


@pytest.mark.parametrize("engine", [xqattn.ENGINE_MFMA, xqattn.ENGINE_VALU], ids=["mfma", "valu"])
@pytest.mark.parametrize("path", CASES, ids=lambda p: p.stem)
def test_capture_replay_matches_captured_output(torch_gpu, path, engine, tmp_path):
    meta, a, _, cap = gio.fa_capture(path, tmp_path)
    case_note(f"xfa1 replay {path.stem} engine {engine}")
    got, want = xfa1.replay(cap, meta["scale"], meta["max_bias"], meta["softcap"], engine=engine)
    assert got.shape == want.shape == a["out"].shape
    assert_close(got, want, what=f"{path.stem} replay vs captured output")
    assert_close(got, a["out64"], what=f"{path.stem} replay vs float64")
