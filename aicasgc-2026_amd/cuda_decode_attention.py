#!/usr/bin/env python3
"""Decode-attention entry points backed by the gfx950 split-KV kernels.

Same names, arguments and return conventions as the reference's
cuda_decode_attention.py: inputs are q [1, Hq, 1, D] (any row stride),
static K/V caches [1, Hkv, T, D] and a device ``cache_position`` [1]; the
valid length is min(cache_position + 1, T); the result is returned as a
[1, 1, Hq, D] view, or ``None`` when the inputs are outside what the kernels
support (the caller then falls back, optimized_layer.py:2404-2458).

All variants compute the same softmax(q K^T * scale) V.  On MI355X one kernel
serves them: each workgroup owns a (kv head, KV split) and serves all q heads
of the group, so K/V is read once; splits are merged from (normalised output,
LSE) partials either by the last-arriving workgroup (``*_fused`` and
``*_cta_*`` names) or by a separate merge launch (``decode_attn_v4_splitkv``).
``split_k`` is honoured as a minimum split count; the kernel may use more
splits to fill 256 CUs (results do not depend on the split count).
"""

from __future__ import annotations

import torch

from qwen3vl_hip import _lib

_WS_KEY = "_qd_attention_ws"


def _load_ext():
    return _lib.lib()


def _supported(q, k, v, num_key_value_groups, cache_position) -> bool:
    return not (
        q.device.type != "cuda" or k.device.type != "cuda" or v.device.type != "cuda"
        or cache_position.device.type != "cuda"
        or q.dtype != torch.float16 or k.dtype != torch.float16 or v.dtype != torch.float16
        or q.ndim != 4 or k.ndim != 4 or v.ndim != 4
        or q.shape[0] != 1 or q.shape[2] != 1 or q.shape[-1] != 128
        or k.shape[0] != 1 or k.shape != v.shape or k.shape[-1] != 128
        or k.shape[1] * num_key_value_groups != q.shape[1]
        or num_key_value_groups not in (1, 2, 4)
        or q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1
        or k.stride(1) != v.stride(1) or k.stride(2) != v.stride(2)
        or q.stride(1) % 8 != 0 or k.stride(1) % 8 != 0 or k.stride(2) % 8 != 0
        or q.data_ptr() % 16 != 0 or k.data_ptr() % 16 != 0 or v.data_ptr() % 16 != 0
        or cache_position.dtype != torch.long or cache_position.numel() != 1
    )


def _splits(seq_len: int, split_k: int | None) -> int:
    s = int(_load_ext().qd_attention_default_splits(int(seq_len)))
    return max(s, int(split_k)) if split_k else s


def _out_buffer(workspace, q) -> torch.Tensor:
    hq, d = q.shape[1], q.shape[-1]
    if (workspace is not None and "out" in workspace and tuple(workspace["out"].shape) == (1, hq, d)
            and workspace["out"].dtype == q.dtype and workspace["out"].device == q.device):
        return workspace["out"]
    return torch.empty((1, hq, d), dtype=q.dtype, device=q.device)


def _ws_buffer(workspace, q, n_bytes: int) -> torch.Tensor:
    """Graph-stable kernel workspace; zero-initialised once (its counters self-reset)."""
    if workspace is not None:
        t = workspace.get(_WS_KEY)
        if t is not None and t.numel() >= n_bytes and t.device == q.device:
            return t
    t = torch.zeros(n_bytes, dtype=torch.uint8, device=q.device)
    if workspace is not None:
        workspace[_WS_KEY] = t
    return t


def _run_fused(q, k, v, scaling, num_key_value_groups, cache_position, split_k, workspace):
    if not _supported(q, k, v, num_key_value_groups, cache_position):
        return None
    lib = _load_ext()
    hq, hkv, T = q.shape[1], k.shape[1], k.shape[2]
    n_split = _splits(T, split_k)
    out = _out_buffer(workspace, q)
    ws = _ws_buffer(workspace, q, int(lib.qd_attention_workspace_bytes(hq, hkv, n_split)))
    _lib.check(lib.qd_attention_decode(
        _lib.ptr(q), _lib.QD_F16, q.stride(1), _lib.ptr(k), _lib.ptr(v), k.stride(1), k.stride(2), T,
        _lib.ptr(cache_position), float(scaling), _lib.ptr(out), _lib.QD_F16, hq, hkv, n_split, _lib.ptr(ws),
        _lib.stream(q.device)), "qd_attention_decode")
    return out.unsqueeze(2).transpose(1, 2)


def _qkv_rope_attention(qkv, q_weight, k_weight, eps: float, cos, sin, k_cache, v_cache, scaling, cache_position,
                        split_k: int = 4, workspace: dict | None = None):
    """q/k head RMSNorm + RoPE (the caller's cos / sin), the new K/V row written
    to the caches at ``cache_position`` and split-KV attention, in one launch
    (qd_attention_qkv_decode_f16): the pair fused_q_rope_kv_cache_update +
    decode_attn_v4_cta_qhead_splitkv_fused that the decoder layer calls back to
    back.  qkv [1, 1, (Hq + 2 Hkv) * 128] fp16; returns [1, 1, Hq, 128], or
    None when the inputs are outside what the kernel supports."""
    if qkv.device.type != "cuda" or qkv.dtype != torch.float16 or not qkv.is_contiguous():
        return None
    if k_cache.ndim != 4 or k_cache.shape[0] != 1 or k_cache.shape[-1] != 128 or k_cache.shape != v_cache.shape:
        return None
    hkv, T = k_cache.shape[1], k_cache.shape[2]
    hq = qkv.shape[-1] // 128 - 2 * hkv
    if (hq != 2 * hkv or qkv.numel() != (hq + 2 * hkv) * 128 or k_cache.dtype != torch.float16
            or v_cache.dtype != torch.float16 or k_cache.stride(-1) != 1 or k_cache.stride() != v_cache.stride()
            or k_cache.stride(1) % 8 or k_cache.stride(2) % 8 or k_cache.data_ptr() % 16 or v_cache.data_ptr() % 16
            or qkv.data_ptr() % 16):
        return None
    if not (cache_position.device.type == "cuda" and cache_position.dtype == torch.long
            and cache_position.numel() == 1):
        return None
    norms = (q_weight, k_weight)
    if any(t.dtype != torch.float16 or t.numel() != 128 or t.device != qkv.device for t in norms):
        return None
    if any(t.dtype != torch.float16 or t.numel() != 128 or t.device != qkv.device for t in (cos, sin)):
        return None
    lib = _load_ext()
    n_split = _splits(T, split_k)
    out = _out_buffer(workspace, qkv.view(1, hq + 2 * hkv, 1, 128)[:, :hq])
    ws = _ws_buffer(workspace, qkv, int(lib.qd_attention_workspace_bytes(hq, hkv, n_split)))
    qw, kw = q_weight.contiguous(), k_weight.contiguous()   # held until the launch is enqueued
    cs, sn, cp = cos.contiguous(), sin.contiguous(), cache_position.contiguous()
    _lib.check(lib.qd_attention_qkv_decode_f16(
        _lib.ptr(qkv), _lib.ptr(qw), _lib.ptr(kw), float(eps), _lib.ptr(cs), _lib.ptr(sn), _lib.ptr(k_cache),
        _lib.ptr(v_cache), k_cache.stride(1), k_cache.stride(2), T, _lib.ptr(cp), float(scaling), _lib.ptr(out),
        hq, hkv, n_split, _lib.ptr(ws), _lib.stream(qkv.device)), "qd_attention_qkv_decode_f16")
    return out.unsqueeze(2).transpose(1, 2)


def decode_attn_v4_cta_qhead_splitkv_fused(q, k, v, scaling, num_key_value_groups, cache_position, split_k: int = 4,
                                           workspace: dict | None = None):
    """Reference cuda_decode_attention.py:489-558 (default decode attention)."""
    if split_k <= 1:
        return None
    return _run_fused(q, k, v, scaling, num_key_value_groups, cache_position, split_k, workspace)


def decode_attn_v4_fused(q, k, v, scaling, num_key_value_groups, cache_position, split_k: int | None = None,
                         workspace: dict | None = None, prefetch_weight=None, prefetch_blocks: int = 0):
    """Reference cuda_decode_attention.py:305-392.  The o_proj L2-prefetch
    sidecar is an A800 experiment and is ignored."""
    del prefetch_weight, prefetch_blocks
    return _run_fused(q, k, v, scaling, num_key_value_groups, cache_position, split_k, workspace)


def decode_attn_v4_cta_local(q, k, v, scaling, num_key_value_groups, cache_position, out=None):
    """Reference cuda_decode_attention.py:395-432."""
    ws = {"out": out} if out is not None else None
    return _run_fused(q, k, v, scaling, num_key_value_groups, cache_position, None, ws)


def decode_attn_v4_cta_qhead(q, k, v, scaling, num_key_value_groups, cache_position, warps_per_cta: int = 4,
                             lane_layout: int = 0, prefetch_mode: int = 0, merge_mode: int = 0, out=None):
    """Reference cuda_decode_attention.py:435-486 (A800 lane-layout knobs ignored)."""
    del warps_per_cta, lane_layout, prefetch_mode, merge_mode
    ws = {"out": out} if out is not None else None
    return _run_fused(q, k, v, scaling, num_key_value_groups, cache_position, None, ws)


def decode_attn_v4_splitkv(q, k, v, scaling, num_key_value_groups, cache_position, split_k: int | None = None,
                           workspace: dict | None = None, prefetch_weight=None, prefetch_blocks: int = 0):
    """Reference cuda_decode_attention.py:226-302: partials then a merge launch.

    ``workspace`` may hold fp32 ``partial_acc`` [Hq, S, 128] and ``lse`` [Hq, S]."""
    del prefetch_weight, prefetch_blocks
    if not _supported(q, k, v, num_key_value_groups, cache_position):
        return None
    lib = _load_ext()
    hq, hkv, T = q.shape[1], k.shape[1], k.shape[2]
    n_split = _splits(T, split_k)
    if (workspace is not None and "partial_acc" in workspace and "lse" in workspace
            and tuple(workspace["partial_acc"].shape) == (hq, n_split, 128)
            and tuple(workspace["lse"].shape) == (hq, n_split)):
        o_part, lse = workspace["partial_acc"], workspace["lse"]
    else:
        o_part = torch.empty((hq, n_split, 128), dtype=torch.float32, device=q.device)
        lse = torch.empty((hq, n_split), dtype=torch.float32, device=q.device)
    out = _out_buffer(workspace, q)
    st = _lib.stream(q.device)
    _lib.check(lib.qd_attention_partial(
        _lib.ptr(q), _lib.QD_F16, q.stride(1), _lib.ptr(k), _lib.ptr(v), k.stride(1), k.stride(2), T,
        _lib.ptr(cache_position), float(scaling), _lib.ptr(o_part), _lib.ptr(lse), hq, hkv, n_split, st),
        "qd_attention_partial")
    _lib.check(lib.qd_attention_merge(_lib.ptr(o_part), _lib.ptr(lse), _lib.ptr(out), _lib.QD_F16, hq, n_split, st),
               "qd_attention_merge")
    return out.unsqueeze(2).transpose(1, 2)


def grouped_prefix_cachepos_splitkv(q, k, v, scaling, num_key_value_groups, cache_position, split_k: int,
                                    workspace: dict | None = None):
    """Reference cuda_decode_attention.py:90-150 (older kernel family)."""
    if split_k <= 1:
        return None
    return _run_fused(q, k, v, scaling, num_key_value_groups, cache_position, split_k, workspace)


def grouped_prefix_cachepos_splitkv_qhead(q, k, v, scaling, num_key_value_groups, cache_position, split_k: int,
                                          workspace: dict | None = None):
    if split_k <= 1:
        return None
    return _run_fused(q, k, v, scaling, num_key_value_groups, cache_position, split_k, workspace)
