#!/usr/bin/env python3
"""Small fused decode ops backed by gfx950 kernels.

Same names, arguments, checks (RuntimeError on a bad dtype/shape) and return
conventions as the reference's cuda_decode_small_ops.py.
"""

from __future__ import annotations

import torch

from qwen3vl_hip import _lib


def _load_ext():
    return _lib.lib()


def _all_cuda_half(*ts) -> bool:
    return all(t.device.type == "cuda" and t.dtype == torch.float16 for t in ts)


def fused_qk_rms_norm_rope(q, k, q_weight, k_weight, eps: float, cos, sin):
    """Per-head RMSNorm + rotate-half RoPE of q [B,S,Hq,128] and k [B,S,Hkv,128]
    with cos/sin [B,S,128] (reference cuda_decode_small_ops.py:70-133)."""
    if not _all_cuda_half(q, k, q_weight, k_weight, cos, sin):
        raise RuntimeError("fused_qk_rms_norm_rope: every tensor must be fp16 on the GPU")
    if q.ndim != 4 or k.ndim != 4:
        raise RuntimeError("fused_qk_rms_norm_rope: q and k must be 4-D [batch, seq, heads, 128]")
    if q.shape[:2] != k.shape[:2]:
        raise RuntimeError("fused_qk_rms_norm_rope: q and k disagree on batch or sequence length")
    if q.shape[-1] != 128 or k.shape[-1] != 128:
        raise RuntimeError("fused_qk_rms_norm_rope: head size must be 128")
    if q.shape[2] != k.shape[2] * 2:
        raise RuntimeError("fused_qk_rms_norm_rope: need twice as many q heads as k heads")
    if q_weight.numel() != 128 or k_weight.numel() != 128:
        raise RuntimeError("fused_qk_rms_norm_rope: q/k norm weights must hold 128 values")
    q_in, k_in = q.contiguous(), k.contiguous()
    cos_in, sin_in = cos.contiguous(), sin.contiguous()
    if cos_in.shape != q_in.shape[:2] + (128,) or sin_in.shape != q_in.shape[:2] + (128,):
        raise RuntimeError("fused_qk_rms_norm_rope: cos/sin must be [batch, seq, 128]")
    m = q_in.shape[0] * q_in.shape[1]
    q_out, k_out = torch.empty_like(q_in), torch.empty_like(k_in)
    qw, kw = q_weight.contiguous(), k_weight.contiguous()   # held until the launch is enqueued
    _lib.check(_load_ext().qd_qk_norm_rope_f16(
        _lib.ptr(q_in), _lib.ptr(k_in), _lib.ptr(qw), _lib.ptr(kw),
        _lib.ptr(cos_in), _lib.ptr(sin_in), _lib.ptr(q_out), _lib.ptr(k_out), m, q_in.shape[2], k_in.shape[2],
        float(eps), _lib.stream(q.device)), "fused_qk_rms_norm_rope")
    return q_out, k_out


def fused_q_rope_kv_cache_update(q, k, v, q_weight, k_weight, eps: float, cos, sin, k_cache, v_cache,
                                 cache_position):
    """q/k per-head RMSNorm + RoPE; K_rot and V written at cache_position;
    returns the rotated q [1,1,Hq,128] (reference cuda_decode_small_ops.py:136-225)."""
    if not (_all_cuda_half(q, k, v, q_weight, k_weight, cos, sin, k_cache, v_cache)
            and cache_position.device.type == "cuda" and cache_position.dtype == torch.long):
        raise RuntimeError("fused_q_rope_kv_cache_update: tensors must be fp16 on the GPU, cache_position int64 on the GPU")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise RuntimeError("fused_q_rope_kv_cache_update: q, k and v must be 4-D [batch, seq, heads, 128]")
    if q.shape[:2] != k.shape[:2] or k.shape != v.shape:
        raise RuntimeError("fused_q_rope_kv_cache_update: k and v shapes differ, or q disagrees with them")
    if q.shape[0] != 1 or q.shape[1] != 1 or k.shape[0] != 1 or k.shape[1] != 1:
        raise RuntimeError("fused_q_rope_kv_cache_update: one token per call (batch 1, seq 1)")
    if q.shape[-1] != 128 or k.shape[-1] != 128 or v.shape[-1] != 128:
        raise RuntimeError("fused_q_rope_kv_cache_update: head size must be 128")
    if q.shape[2] != k.shape[2] * 2:
        raise RuntimeError("fused_q_rope_kv_cache_update: need twice as many q heads as kv heads")
    if q_weight.numel() != 128 or k_weight.numel() != 128:
        raise RuntimeError("fused_q_rope_kv_cache_update: q/k norm weights must hold 128 values")
    if cos.shape != q.shape[:2] + (128,) or sin.shape != q.shape[:2] + (128,):
        raise RuntimeError("fused_q_rope_kv_cache_update: cos/sin must be [batch, seq, 128]")
    if k_cache.ndim != 4 or v_cache.ndim != 4:
        raise RuntimeError("fused_q_rope_kv_cache_update: caches must be 4-D [batch, kv heads, rows, 128]")
    if k_cache.shape[0] != 1 or v_cache.shape[0] != 1:
        raise RuntimeError("fused_q_rope_kv_cache_update: caches must have batch 1")
    if k_cache.shape[1] != k.shape[2] or v_cache.shape[1] != v.shape[2]:
        raise RuntimeError("fused_q_rope_kv_cache_update: cache and k have different kv head counts")
    if k_cache.shape[-1] != 128 or v_cache.shape[-1] != 128:
        raise RuntimeError("fused_q_rope_kv_cache_update: cache rows are not 128 wide")
    if cache_position.ndim != 1 or cache_position.numel() != 1:
        raise RuntimeError("fused_q_rope_kv_cache_update: cache_position must hold exactly one position")
    if (k_cache.stride(-1) != 1 or v_cache.stride(-1) != 1 or k_cache.stride(1) != v_cache.stride(1)
            or k_cache.stride(2) != v_cache.stride(2) or k_cache.shape != v_cache.shape):
        raise RuntimeError("fused_q_rope_kv_cache_update: k_cache and v_cache need the same strides and contiguous rows")
    # contiguous copies are bound to locals so they outlive the asynchronous launch's enqueue
    q_in, k_in, v_in = q.contiguous(), k.contiguous(), v.contiguous()
    qw, kw = q_weight.contiguous(), k_weight.contiguous()
    cos_in, sin_in, cp = cos.contiguous(), sin.contiguous(), cache_position.contiguous()
    q_out = torch.empty((1, 1, q.shape[2], 128), dtype=q.dtype, device=q.device)
    _lib.check(_load_ext().qd_q_rope_kv_update(
        _lib.ptr(q_in), _lib.ptr(k_in), _lib.ptr(v_in), _lib.QD_F16, 128, 128, 128,
        _lib.ptr(qw), _lib.ptr(kw), float(eps), _lib.ptr(cos_in), _lib.ptr(sin_in), None, None, 24, 20, 20,
        _lib.ptr(q_out), _lib.QD_F16, _lib.ptr(k_cache), _lib.ptr(v_cache), k_cache.stride(1), k_cache.stride(2),
        k_cache.shape[2], _lib.ptr(cp), q.shape[2], k.shape[2], _lib.stream(q.device)),
        "fused_q_rope_kv_cache_update")
    return q_out


def fused_silu_mul(gate, up):
    """silu(gate) * up (reference cuda_decode_small_ops.py:228-247)."""
    if not _all_cuda_half(gate, up):
        raise RuntimeError("fused_silu_mul: gate and up must be fp16 on the GPU")
    if gate.shape != up.shape:
        raise RuntimeError("fused_silu_mul: gate and up shapes differ")
    g, u = gate.contiguous(), up.contiguous()
    out = torch.empty_like(g)
    _lib.check(_load_ext().qd_silu_mul_f16(_lib.ptr(g), _lib.ptr(u), _lib.ptr(out), g.numel(),
                                           _lib.stream(g.device)), "fused_silu_mul")
    return out


def fused_add_rms_norm(residual, x, weight, eps: float):
    """(residual + x, rmsnorm(residual + x) * weight) (reference cuda_decode_small_ops.py:250-287)."""
    if not _all_cuda_half(residual, x, weight):
        raise RuntimeError("fused_add_rms_norm: every tensor must be fp16 on the GPU")
    if residual.shape != x.shape:
        raise RuntimeError("fused_add_rms_norm: residual and x shapes differ")
    if residual.shape[-1] != weight.numel():
        raise RuntimeError("fused_add_rms_norm: weight length differs from the last dimension")
    r, xi = residual.contiguous(), x.contiguous()
    cols = r.shape[-1]
    rows = r.numel() // cols
    out_sum, out_norm = torch.empty_like(r), torch.empty_like(r)
    wc = weight.contiguous()
    _lib.check(_load_ext().qd_add_rmsnorm_f16(_lib.ptr(r), _lib.ptr(xi), _lib.ptr(wc),
                                              _lib.ptr(out_sum), _lib.ptr(out_norm), rows, cols, float(eps),
                                              _lib.stream(r.device)), "fused_add_rms_norm")
    return out_sum, out_norm


def rms_norm(x, weight, eps: float):
    """rmsnorm(x) * weight over the last dim (reference cuda_decode_small_ops.py:290-317)."""
    if not _all_cuda_half(x, weight):
        raise RuntimeError("rms_norm: x and weight must be fp16 on the GPU")
    if x.shape[-1] != weight.numel():
        raise RuntimeError("rms_norm: weight length differs from the last dimension")
    xi = x.contiguous()
    cols = xi.shape[-1]
    out = torch.empty_like(xi)
    wc = weight.contiguous()
    _lib.check(_load_ext().qd_rmsnorm_f16(_lib.ptr(xi), _lib.ptr(wc), _lib.ptr(out),
                                          xi.numel() // cols, cols, float(eps), _lib.stream(xi.device)), "rms_norm")
    return out


def add(a, b):
    """a + b (reference cuda_decode_small_ops.py:320-339)."""
    if not _all_cuda_half(a, b):
        raise RuntimeError("add: both operands must be fp16 on the GPU")
    if a.shape != b.shape:
        raise RuntimeError("add: operand shapes differ")
    ai, bi = a.contiguous(), b.contiguous()
    out = torch.empty_like(ai)
    _lib.check(_load_ext().qd_add_f16(_lib.ptr(ai), _lib.ptr(bi), _lib.ptr(out), ai.numel(),
                                      _lib.stream(ai.device)), "add")
    return out
