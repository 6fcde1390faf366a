"""Decode GEMV entry points (batch 1, fp16) backed by the gfx950 GEMV kernels.

Same names, arguments and return conventions as the reference's
cuda_decode_gemv_ops/matvec.py; every variant the reference exposes for A800
kernel experiments routes to the single MI355X GEMV family
(``qd_matvec_f16`` / ``qd_splitk_matvec_f16``).
"""

from __future__ import annotations

import torch

from qwen3vl_hip import _lib

from .runtime import NOSPLIT_VARIANTS, _check, _contig_weight, _load_ext, _p, _require_decode_half, _reuse, _stream

__all__ = [
    "splitk_matvec", "splitk_matvec_row4", "splitk_matvec_row8_shared", "splitk_matvec_row4_shared_vec_half",
    "splitk_matvec_row4_shared_vec_half_v2", "persistent_matvec_half", "nosplit_matvec_half",
    "nosplit_hfma2_matvec_half", "nosplit_matvec_half_variant", "weight_stream_read_half",
    "weight_stream_read_dual_half", "l2_8kb_pointer_chase_pair", "l2_sequential_pointer_chase_trace",
    "nosplit_weight_only_half_variant", "nosplit_matvec_half_dualcopy_routed", "nosplit_matvec_half_partition",
    "nosplit_matvec_half_partition_v2",
]


def _matvec(name: str, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
            out_vec: torch.Tensor | None = None) -> torch.Tensor:
    _require_decode_half(name, x, weight, x=x)
    if bias is not None:
        _require_decode_half(name, bias)
    w = _contig_weight(weight, name)
    n, k = w.shape
    x_vec = x.reshape(-1).contiguous()
    if x_vec.numel() != k:
        raise RuntimeError(f"{name}: x has {x_vec.numel()} elements, weight expects K={k}")
    if out_vec is None:
        out_vec = torch.empty((n,), dtype=x.dtype, device=x.device)
    b = bias.reshape(-1).contiguous() if bias is not None else None
    _check(_load_ext().qd_matvec_f16(_p(x_vec), _p(w), _p(b), _p(out_vec), n, k, _stream(x)), name)
    return out_vec.view(*x.shape[:-1], n)


def nosplit_matvec_half(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                        workspace: dict | None = None) -> torch.Tensor:
    """y = W x (+ b) for one decode token (reference matvec.py:274-321)."""
    n = weight.shape[0]
    out = _reuse(workspace, "nosplit", "out", (n,), x.dtype, x.device) if workspace is not None else None
    return _matvec("nosplit_matvec_half", x, weight, bias, out)


def nosplit_hfma2_matvec_half(x, weight, bias, workspace: dict | None = None):
    """Reference matvec.py:324-: same product; the gfx950 kernel accumulates in fp32."""
    return nosplit_matvec_half(x, weight, bias, workspace)


def nosplit_matvec_half_variant(x, weight, bias, variant: str):
    """Reference matvec.py variant dispatcher: every known variant name maps to the gfx950 GEMV."""
    if variant not in NOSPLIT_VARIANTS:
        raise RuntimeError(f"unknown nosplit variant {variant!r}; known: {', '.join(NOSPLIT_VARIANTS)}")
    return _matvec("nosplit_matvec_half_variant", x, weight, bias)


def persistent_matvec_half(x, weight, bias, workspace: dict | None = None):
    return nosplit_matvec_half(x, weight, bias, workspace)


def splitk_matvec(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, split_k: int,
                  workspace: dict | None = None) -> torch.Tensor:
    """Split-K GEMV (reference matvec.py:10-51).

    The K dimension is cut into ``split_k`` slices; fp32 partials [split_k, N]
    are reduced in slice order (deterministic) with the bias.  ``workspace``
    may carry ``{"split_k", "scratch" (fp32 [split_k*N]), "out"}``.
    """
    if x.device.type != "cuda" or weight.device.type != "cuda" or x.ndim < 2 or x.shape[-2] != 1 or split_k <= 0:
        raise RuntimeError("splitk_matvec expects CUDA single-token decode tensors")
    _require_decode_half("splitk_matvec", x, weight, x=x)
    w = _contig_weight(weight, "splitk_matvec")
    n, k = w.shape
    x_vec = x.reshape(-1).contiguous()
    if (workspace is not None and workspace.get("split_k") == split_k
            and tuple(workspace["scratch"].shape) == (split_k * n,) and workspace["scratch"].device == x.device
            and workspace["out"].dtype == x.dtype and tuple(workspace["out"].shape) == (n,)):
        scratch, out_vec = workspace["scratch"], workspace["out"]
    else:
        scratch = torch.empty((split_k * n,), dtype=torch.float32, device=x.device)
        out_vec = torch.empty((n,), dtype=x.dtype, device=x.device)
    b = bias.reshape(-1).contiguous() if bias is not None else None
    _check(_load_ext().qd_splitk_matvec_f16(_p(x_vec), _p(w), _p(b), _p(scratch), _p(out_vec), n, k,
                                            int(split_k), _stream(x)), "splitk_matvec")
    return out_vec.view(*x.shape[:-1], n)


def splitk_matvec_row4(x, weight, bias, split_k, workspace=None):
    return splitk_matvec(x, weight, bias, split_k, workspace)


def splitk_matvec_row8_shared(x, weight, bias, split_k, workspace=None):
    return splitk_matvec(x, weight, bias, split_k, workspace)


def splitk_matvec_row4_shared_vec_half(x, weight, bias, split_k, workspace=None):
    return splitk_matvec(x, weight, bias, split_k, workspace)


def splitk_matvec_row4_shared_vec_half_v2(x, weight, bias, split_k, workspace=None):
    return splitk_matvec(x, weight, bias, split_k, workspace)


def _a800_research(name: str):
    def fn(*args, **kwargs):
        raise NotImplementedError(
            f"{name} is an A800 memory-system probe / partition experiment of the reference; "
            "it has no MI355X counterpart in this build")
    fn.__name__ = name
    return fn


weight_stream_read_half = _a800_research("weight_stream_read_half")
weight_stream_read_dual_half = _a800_research("weight_stream_read_dual_half")
l2_8kb_pointer_chase_pair = _a800_research("l2_8kb_pointer_chase_pair")
l2_sequential_pointer_chase_trace = _a800_research("l2_sequential_pointer_chase_trace")
nosplit_weight_only_half_variant = _a800_research("nosplit_weight_only_half_variant")
nosplit_matvec_half_dualcopy_routed = _a800_research("nosplit_matvec_half_dualcopy_routed")
nosplit_matvec_half_partition = _a800_research("nosplit_matvec_half_partition")
nosplit_matvec_half_partition_v2 = _a800_research("nosplit_matvec_half_partition_v2")

_ = _lib  # the library module is the only native dependency
