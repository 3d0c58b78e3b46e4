"""The library's C ABI called from plain C (tests/c_abi/xq_c_caller.c): no
Python binding and no torch, only the HIP runtime for device memory. The
program runs a q8_0 flash-attention decode and a 5-token gated-delta-net
prefill with two snapshot slots (step kernel and chunked form) and checks each
against the CPU oracle within the parity tolerance (2e-3 abs + 1e-2 rel); it is
built with the library (the repository's build entry point runs its Makefile).
"""
import pathlib
import subprocess

import pytest

from conftest import case_note

pytestmark = pytest.mark.gpu

BIN = pathlib.Path(__file__).resolve().parent / "c_abi" / "_build" / "xq_c_caller"


def test_c_caller_matches_the_oracle(torch_gpu):
    case_note("plain-C caller: q8_0 decode, gdn prefill (step, chunked)")
    assert BIN.exists(), f"{BIN} is not built (run the build entry point)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, f"exit {r.returncode}: {r.stdout}{r.stderr}"
    assert "all checks passed" in r.stdout
    assert r.stdout.count("outside the tolerance") == 3
