"""Test configuration: import paths, the `gpu` marker and shared helpers."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "aicasgc-2026_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

# Per-kernel parity bar: max |out - ref| <= 2e-3 * max |ref| against fp32 math.
REL_TOL = 2e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from qwen3vl_hip import _lib

    _lib.lib()  # raises if the library is not built: GPU tests never run without it
    return torch.device("cuda:0")


def assert_close_rel(out, ref, rel: float = REL_TOL, what: str = ""):
    """max |out - ref| <= rel * max |ref| (ref is fp32/fp64 math on the CPU)."""
    import torch

    o = out.detach().to("cpu", torch.float64)
    r = ref.detach().to("cpu", torch.float64)
    assert o.shape == r.shape, f"{what}: shape {tuple(o.shape)} != {tuple(r.shape)}"
    assert torch.isfinite(o).all(), f"{what}: non-finite output"
    err = (o - r).abs().max().item()
    scale = r.abs().max().item()
    print(f"[parity] {what}: max_abs_err={err:.3e} max|ref|={scale:.3e} ratio={err / max(scale, 1e-30):.2e}",
          flush=True)
    assert err <= rel * scale, f"{what}: max abs err {err:.3e} > {rel} * {scale:.3e}"
