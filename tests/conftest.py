"""Shared fixtures. GPU tests carry @pytest.mark.gpu; everything else runs on CPU.

The product package lives in ``xllama-qwen35-xbox_amd/xqattn``; the CPU oracle
(test infrastructure) in ``oracle/``. Both are imported from the repository root.
"""
import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "xllama-qwen35-xbox_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402
import xqattn  # noqa: E402
from xqattn import workloads as wl  # noqa: E402

# parity tolerance for attention outputs and GDN outputs/state (f32 accumulation)
ATOL, RTOL = 2e-3, 1e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the gfx950 kernels)")


@pytest.fixture(scope="session", autouse=True)
def _built_oracle():
    if not oracle.LIB_PATH.exists():
        oracle.build()
    oracle.load()


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    xqattn.load()  # fails loudly when the library is missing
    return torch


def assert_close(got, want, atol=ATOL, rtol=RTOL, what=""):
    """|got - want| <= atol + rtol*|want| elementwise (the parity tolerance)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin), f"{what}: finiteness differs"
    assert np.array_equal(got[~fin], want[~fin]) or np.all(np.isnan(got[~fin]) == np.isnan(want[~fin])), what
    err = np.abs(got[fin] - want[fin])
    lim = atol + rtol * np.abs(want[fin])
    bad = err > lim
    if bad.any():
        i = int(np.argmax(err - lim))
        raise AssertionError(f"{what}: {int(bad.sum())} of {err.size} outside tolerance; "
                             f"worst |d|={err[i]:.3e} at want={want[fin][i]:.4e} (max abs err {err.max():.3e})")
    return float(err.max()) if err.size else 0.0


def case_note(msg: str):
    """Name the case on stdout before a GPU step (flushed)."""
    print(f"[case] {msg}", flush=True)
