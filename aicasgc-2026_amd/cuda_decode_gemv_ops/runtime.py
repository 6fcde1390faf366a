"""Runtime side of the decode GEMV wrappers: library handle and shared checks.

Mirrors the reference module of the same name (cuda_decode_gemv_ops/runtime.py)
whose ``_load_ext`` (:168-193) built and imported a pybind11 CUDA extension.
Here ``_load_ext`` returns the ctypes handle of the prebuilt gfx950 C-ABI
library and raises RuntimeError if it is absent: there is no fallback path.

The reference's profile-slot tables (:23-140) name %globaltimer stamps of its
NVIDIA profiling kernels; those kernels are not part of this build (rocprofv3
counters replace them), so the tables are exported empty for import
compatibility.
"""

from __future__ import annotations

import torch

from qwen3vl_hip import _lib

NOSPLIT_PROFILE_SLOT_NAMES: tuple = ()
NOSPLIT_XWARP_DETAIL_SLOT_NAMES: tuple = ()
FULL_LAYER_PROFILE_SLOT_NAMES: tuple = ()
SOFTSYNC_PROFILE_SLOT_NAMES: tuple = ()
PERSISTENT_PROFILE_SLOT_NAMES: tuple = ()
OPROJ_MLP_PROFILE_SLOT_NAMES: tuple = ()
GRIDSYNC_PROFILE_SLOT_NAMES: tuple = ()
DUALCOPY_ROUTE_MODES: dict = {}

# Variant names accepted by nosplit_matvec_half_variant.  Every name maps to
# the same gfx950 GEMV (the A800-specific kernel choices do not apply).
NOSPLIT_VARIANTS = (
    "auto",
    "k6144_row4",
    "k6144_n8k1024_async",
    "k6144_n8k1024_xw_async",
    "k6144_n8k1024_xwarp_w_async",
    "k6144_n8k1024_xwarp_w_async_sms2",
    "k6144_n8k1024_xwarp_w_async_sms2_balanced",
)


def _load_ext():
    """The C-ABI library handle (raises RuntimeError when it is not built)."""
    return _lib.lib()


def _stream(t: torch.Tensor):
    return _lib.stream(t.device)


def _p(t: torch.Tensor | None):
    return _lib.ptr(t)


def _check(status: int, what: str) -> None:
    _lib.check(status, what)


def _require_decode_half(name: str, *tensors: torch.Tensor, x: torch.Tensor | None = None) -> None:
    """The reference's guard: fp16 GPU tensors, single-token decode shape."""
    for t in tensors:
        if t.device.type != "cuda" or t.dtype != torch.float16:
            raise RuntimeError(f"{name} expects fp16 CUDA single-token decode tensors")
    if x is not None and (x.ndim < 2 or x.shape[-2] != 1):
        raise RuntimeError(f"{name} expects fp16 CUDA single-token decode tensors")


def _contig_weight(w: torch.Tensor, name: str) -> torch.Tensor:
    if w.ndim != 2:
        raise RuntimeError(f"{name}: weight must be 2-D [N, K]")
    return w if w.is_contiguous() else w.contiguous()


def _reuse(workspace: dict | None, kind: str, key: str, shape: tuple, dtype, device) -> torch.Tensor:
    """Workspace reuse with the reference's dict convention (fused.py:294-318)."""
    if (workspace is not None and workspace.get("type") == kind and key in workspace
            and tuple(workspace[key].shape) == shape and workspace[key].dtype == dtype
            and workspace[key].device == device):
        return workspace[key]
    return torch.empty(shape, dtype=dtype, device=device)
