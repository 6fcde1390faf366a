"""Fused decode GEMV entry points (batch 1, fp16) backed by gfx950 kernels.

Same names, arguments and return conventions as the reference's
cuda_decode_gemv_ops/fused.py.  The reference ships several launch strategies
for the same math (persistent, softsync, gridsync, mega); each name maps to
the MI355X kernel that computes that math, so callers selecting any of them
get identical results.
"""

from __future__ import annotations

import ctypes

import torch

from qwen3vl_hip import _lib

from .matvec import nosplit_matvec_half
from .runtime import _check, _contig_weight, _load_ext, _p, _require_decode_half, _reuse, _stream

__all__ = [
    "fused_add_rmsnorm_gateup_half", "fused_rmsnorm_qkv_half", "fused_silu_downproj_half",
    "fused_gateup_silu_downproj_half", "fused_post_attn_mlp_persistent_half", "fused_post_attn_mlp_softsync_half",
    "fused_o_proj_post_attn_mlp_persistent_half", "fused_o_proj_post_attn_mlp_softsync_half",
    "fused_decode_full_layer_softsync_half", "fused_gateup_silu_downproj_mega_half",
    "fused_gateup_silu_downproj_mega_partial_half", "fused_gateup_silu_downproj_softsync_half",
    "fused_gateup_silu_downproj_gridsync_half", "fused_gateup_silu_downproj_persistent_half",
    "decode_attn_persistent_half",
]


def _vec(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1).contiguous()


def fused_rmsnorm_qkv_half(x: torch.Tensor, norm_weight: torch.Tensor, weight: torch.Tensor,
                           bias: torch.Tensor | None, eps: float) -> torch.Tensor:
    """out = W (rmsnorm(x) * gamma) (+ b)  (reference fused.py:71-105)."""
    name = "fused_rmsnorm_qkv_half"
    _require_decode_half(name, x, norm_weight, weight, x=x)
    w = _contig_weight(weight, name)
    n, k = w.shape
    x_vec, g = _vec(x), _vec(norm_weight)
    if x_vec.numel() != k or g.numel() != k:
        raise RuntimeError(f"{name}: x/norm_weight must have K={k} elements")
    out = torch.empty((n,), dtype=x.dtype, device=x.device)
    b = _vec(bias) if bias is not None else None
    _check(_load_ext().qd_rmsnorm_matvec_f16(_p(x_vec), _p(g), _p(w), _p(b), _p(out), n, k, float(eps),
                                             _stream(x)), name)
    return out.view(*x.shape[:-1], n)


def fused_add_rmsnorm_gateup_half(residual: torch.Tensor, x: torch.Tensor, norm_weight: torch.Tensor,
                                  weight: torch.Tensor, bias: torch.Tensor | None, eps: float,
                                  workspace: dict | None = None):
    """(residual + x, W rmsnorm(residual + x)) (reference fused.py:12-68)."""
    name = "fused_add_rmsnorm_gateup_half"
    _require_decode_half(name, residual, x, norm_weight, weight, x=residual)
    if residual.shape != x.shape:
        raise RuntimeError(f"{name}: residual/x shapes differ")
    w = _contig_weight(weight, name)
    n, k = w.shape
    res_out = _reuse(workspace, "fused_add_rmsnorm_gateup", "residual_out", (k,), residual.dtype, residual.device)
    out = _reuse(workspace, "fused_add_rmsnorm_gateup", "out", (n,), residual.dtype, residual.device)
    b = _vec(bias) if bias is not None else None
    rv, xv, gv = _vec(residual), _vec(x), _vec(norm_weight)   # held until the launch is enqueued
    _check(_load_ext().qd_add_rmsnorm_matvec_f16(_p(rv), _p(xv), _p(gv), _p(w), _p(b), _p(res_out), _p(out), n, k,
                                                 float(eps), _stream(x)), name)
    return res_out.view_as(residual), out.view(*residual.shape[:-1], n)


def fused_silu_downproj_half(gate_up: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                             workspace: dict | None = None) -> torch.Tensor:
    """W (silu(gate) * up) (+ b) for gate_up = [gate; up] (reference fused.py:108-145)."""
    name = "fused_silu_downproj_half"
    _require_decode_half(name, gate_up, weight, x=gate_up)
    w = _contig_weight(weight, name)
    n, k = w.shape
    gu = _vec(gate_up)
    if gu.numel() != 2 * k:
        raise RuntimeError(f"{name}: gate_up must have 2*K = {2 * k} elements")
    out = _reuse(workspace, "fused_silu_downproj", "out", (n,), gate_up.dtype, gate_up.device)
    b = _vec(bias) if bias is not None else None
    _check(_load_ext().qd_silu_matvec_f16(_p(gu), _p(w), _p(b), _p(out), n, k, _stream(gate_up)), name)
    return out.view(*gate_up.shape[:-1], n)


def _gateup_silu_down(name: str, x, gate_up_weight, down_proj_weight, bias, workspace, kind):
    _require_decode_half(name, x, gate_up_weight, down_proj_weight, x=x)
    wgu = _contig_weight(gate_up_weight, name)
    wd = _contig_weight(down_proj_weight, name)
    two_i, h = wgu.shape
    n, i = wd.shape
    if two_i != 2 * i or _vec(x).numel() != h:
        raise RuntimeError(f"{name}: inconsistent shapes gate_up {tuple(wgu.shape)} down {tuple(wd.shape)}")
    hidden = _reuse(workspace, kind, "hidden_out", (i,), x.dtype, x.device)
    out = _reuse(workspace, kind, "out", (n,), x.dtype, x.device)
    b = _vec(bias) if bias is not None else None
    xv = _vec(x)
    _check(_load_ext().qd_gateup_silu_down_f16(_p(xv), _p(wgu), _p(wd), _p(b), _p(hidden), _p(out), h, i,
                                               _stream(x)), name)
    return hidden.view(*x.shape[:-1], i), out.view(*x.shape[:-1], n)


def fused_gateup_silu_downproj_half(x, gate_up_weight, down_proj_weight, bias, workspace=None):
    """(silu(W_g x) * W_u x, W_d of it (+ b)) (reference fused.py:148-197)."""
    return _gateup_silu_down("fused_gateup_silu_downproj_half", x, gate_up_weight, down_proj_weight, bias,
                             workspace, "fused_gateup_silu_downproj")


def fused_gateup_silu_downproj_persistent_half(x, gate_up_weight, down_proj_weight, workspace=None):
    return _gateup_silu_down("fused_gateup_silu_downproj_persistent_half", x, gate_up_weight, down_proj_weight,
                             None, workspace, "fused_gateup_silu_downproj_persistent")


def fused_gateup_silu_downproj_softsync_half(x, gate_up_weight, down_proj_weight, workspace=None):
    return _gateup_silu_down("fused_gateup_silu_downproj_softsync_half", x, gate_up_weight, down_proj_weight,
                             None, workspace, "fused_gateup_silu_downproj_softsync")


def fused_gateup_silu_downproj_gridsync_half(x, gate_up_weight, down_proj_weight, workspace=None):
    return _gateup_silu_down("fused_gateup_silu_downproj_gridsync_half", x, gate_up_weight, down_proj_weight,
                             None, workspace, "fused_gateup_silu_downproj_gridsync")


def fused_gateup_silu_downproj_mega_half(x, gate_up_weight, down_proj_weight, workspace=None):
    return _gateup_silu_down("fused_gateup_silu_downproj_mega_half", x, gate_up_weight, down_proj_weight,
                             None, workspace, "fused_gateup_silu_downproj_mega")


def fused_gateup_silu_downproj_mega_partial_half(x, gate_up_weight, down_proj_weight, workspace=None):
    return _gateup_silu_down("fused_gateup_silu_downproj_mega_partial_half", x, gate_up_weight,
                             down_proj_weight, None, workspace, "fused_gateup_silu_downproj_mega_partial")


def _post_attn_mlp(name, residual, attn_output, norm_weight, gate_up_weight, down_proj_weight, bias, eps, workspace,
                   kind, next_position=None):
    """next_position: optional (position, length) int64 device words; the last
    kernel then also writes length = position + 1."""
    _require_decode_half(name, residual, attn_output, norm_weight, gate_up_weight, down_proj_weight, x=residual)
    if residual.shape != attn_output.shape:
        raise RuntimeError(f"{name} expects fp16 CUDA single-token decode tensors")
    if bias is not None:
        _require_decode_half(name, bias)
    wgu = _contig_weight(gate_up_weight, name)
    wd = _contig_weight(down_proj_weight, name)
    two_i, h = wgu.shape
    n, i = wd.shape
    if two_i != 2 * i or n != h or residual.shape[-1] != h:
        raise RuntimeError(f"{name}: inconsistent shapes")
    hidden = _reuse(workspace, kind, "hidden_out", (i,), residual.dtype, residual.device)
    out = _reuse(workspace, kind, "out", (n,), residual.dtype, residual.device)
    b = _vec(bias) if bias is not None else None
    rv, av, gv = _vec(residual), _vec(attn_output), _vec(norm_weight)   # held until the launch is enqueued
    if next_position is None:
        _check(_load_ext().qd_post_attn_mlp_f16(_p(rv), _p(av), _p(gv), _p(wgu), _p(wd), _p(b), _p(hidden), _p(out),
                                                h, i, float(eps), _stream(residual)), name)
    else:
        pos, length = next_position
        if not all(t.device == residual.device and t.dtype == torch.int64 and t.numel() == 1 for t in (pos, length)):
            raise RuntimeError(f"{name}: position and length must be single int64 words on the GPU")
        _check(_load_ext().qd_post_attn_mlp_next_f16(_p(rv), _p(av), _p(gv), _p(wgu), _p(wd), _p(b), _p(hidden),
                                                     _p(out), h, i, float(eps), _p(pos), _p(length),
                                                     _stream(residual)), name)
    return hidden.view(*residual.shape[:-1], i), out.view(*residual.shape[:-1], n)


def fused_post_attn_mlp_softsync_half(residual, attn_output, norm_weight, gate_up_weight, down_proj_weight, bias,
                                      eps, workspace=None, threads_per_block: int = 1024, launch_blocks=None):
    """Post-attention MLP of a layer (reference fused.py:261-337):
    r = residual + attn; hidden = silu(W_g x) * W_u x with x = rmsnorm(r) * gamma;
    out = W_d hidden + r (+ b).  Returns (hidden [.., I], out [.., H]).
    ``threads_per_block`` / ``launch_blocks`` tuned the A800 launch and are
    accepted for compatibility."""
    del threads_per_block, launch_blocks
    return _post_attn_mlp("fused_post_attn_mlp_softsync_half", residual, attn_output, norm_weight, gate_up_weight,
                          down_proj_weight, bias, eps, workspace, "fused_post_attn_mlp_softsync")


def fused_post_attn_mlp_persistent_half(residual, attn_output, norm_weight, gate_up_weight, down_proj_weight, bias,
                                        eps, workspace=None):
    return _post_attn_mlp("fused_post_attn_mlp_persistent_half", residual, attn_output, norm_weight,
                          gate_up_weight, down_proj_weight, bias, eps, workspace, "fused_post_attn_mlp_persistent")


def _o_proj_post_attn_mlp(name, residual, attn_input, o_proj_weight, o_proj_bias, norm_weight, gate_up_weight,
                          down_proj_weight, down_proj_bias, eps, workspace):
    o = nosplit_matvec_half(attn_input, o_proj_weight, o_proj_bias)
    return _post_attn_mlp(name, residual, o.view_as(residual), norm_weight, gate_up_weight, down_proj_weight,
                          down_proj_bias, eps, workspace, name)


def fused_o_proj_post_attn_mlp_persistent_half(residual, attn_input, o_proj_weight, o_proj_bias, norm_weight,
                                               gate_up_weight, down_proj_weight, down_proj_bias, eps, workspace=None):
    """o_proj followed by the post-attention MLP (reference fused.py:340-409)."""
    return _o_proj_post_attn_mlp("fused_o_proj_post_attn_mlp_persistent_half", residual, attn_input, o_proj_weight,
                                 o_proj_bias, norm_weight, gate_up_weight, down_proj_weight, down_proj_bias, eps,
                                 workspace)


def fused_o_proj_post_attn_mlp_softsync_half(residual, attn_input, o_proj_weight, o_proj_bias, norm_weight,
                                             gate_up_weight, down_proj_weight, down_proj_bias, eps, workspace=None,
                                             gate_up_active_sms: int = 0):
    del gate_up_active_sms
    return _o_proj_post_attn_mlp("fused_o_proj_post_attn_mlp_softsync_half", residual, attn_input, o_proj_weight,
                                 o_proj_bias, norm_weight, gate_up_weight, down_proj_weight, down_proj_bias, eps,
                                 workspace)


_FULL_LAYER_KIND = "fused_decode_full_layer_softsync"
_PERSISTENT_DEVICE_OK: dict = {}   # device index -> the one-layer persistent launch runs there


def _persistent_layer_device_ok(device: torch.device) -> bool:
    """Whether the one-layer persistent launch runs on ``device``.  The first
    call per device (outside stream capture) allocates the device's persistent
    hand-off area (qd_persistent_prepare); under capture before that, False."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ok = _PERSISTENT_DEVICE_OK.get(idx)
    if ok is None:
        if torch.cuda.is_current_stream_capturing():
            return False
        st = _load_ext().qd_persistent_prepare(_lib.stream(device))
        if st not in (0, _lib.QD_ERR_SHAPE):
            _check(st, "qd_persistent_prepare")
        ok = _PERSISTENT_DEVICE_OK[idx] = st == 0
    return ok


def _full_layer_eligible(h, qkv_weight, input_layernorm_weight, q_norm_weight, k_norm_weight, cos, sin, k_cache,
                         v_cache, cache_position, o_proj_weight, o_proj_bias, post_attn_norm_weight, gate_up_weight,
                         down_proj_weight, down_proj_bias, length=None) -> bool:
    """The reference's eligibility of its one-launch layer (optimized_layer.py:1511-1600:
    fp16 GPU tensors at the 2B shapes, contiguous last dims, static [1, 8, T, 128]
    caches, one cache position) with no biases, contiguous 16-byte aligned
    weights, norms and caches and 8-byte aligned input and position words."""
    if not (h.device.type == "cuda" and h.dtype == torch.float16 and h.numel() == 2048 and h.shape[-1] == 2048
            and o_proj_bias is None and down_proj_bias is None):
        return False
    mats = ((qkv_weight, (4096, 2048)), (o_proj_weight, (2048, 2048)), (gate_up_weight, (12288, 2048)),
            (down_proj_weight, (2048, 6144)))
    vecs = ((input_layernorm_weight, 2048), (post_attn_norm_weight, 2048), (q_norm_weight, 128),
            (k_norm_weight, 128), (cos, 128), (sin, 128))
    if not all(t.device == h.device and t.dtype == torch.float16 and tuple(t.shape) == shp and t.is_contiguous()
               for t, shp in mats):
        return False
    if not all(t.device == h.device and t.dtype == torch.float16 and t.numel() == n and t.is_contiguous()
               for t, n in vecs):
        return False
    if not all(c.device == h.device and c.dtype == torch.float16 and c.ndim == 4 and c.shape[0] == 1
               and c.shape[1] == 8 and c.shape[3] == 128 and c.is_contiguous() for c in (k_cache, v_cache)):
        return False
    if k_cache.shape != v_cache.shape or not (cache_position.device == h.device and cache_position.numel() == 1
                                              and cache_position.dtype == torch.int64):
        return False
    if length is not None and not (length.device == h.device and length.dtype == torch.int64
                                   and length.numel() == 1):
        return False
    # the launch reads weights, norms and caches as 16-byte vectors and the
    # input as 8-byte slices: offset views take the kernel chain instead
    if any(t.data_ptr() % 16 for t in (qkv_weight, o_proj_weight, gate_up_weight, down_proj_weight,
                                       input_layernorm_weight, post_attn_norm_weight, k_cache, v_cache)):
        return False
    return not (h.data_ptr() % 8 or cache_position.data_ptr() % 8)


def _full_layer_persistent(hidden_states, qkv_weight, input_layernorm_weight, q_norm_weight, k_norm_weight, cos,
                           sin, k_cache, v_cache, cache_position, o_proj_weight, o_proj_bias, post_attn_norm_weight,
                           gate_up_weight, down_proj_weight, down_proj_bias, eps, attn_scale, workspace=None,
                           length=None):
    """One Qwen3-VL-2B decoder layer as one persistent launch
    (qd_decoder_layer_persistent_f16), or None where it does not apply
    (_full_layer_eligible, and a device that keeps the grid resident).
    ``length``: the cache's running-length word, set to position + 1 by the
    launch.  The output and the status word live in ``workspace`` (stable
    addresses for graph capture)."""
    h = hidden_states
    if not _full_layer_eligible(h, qkv_weight, input_layernorm_weight, q_norm_weight, k_norm_weight, cos, sin,
                                k_cache, v_cache, cache_position, o_proj_weight, o_proj_bias, post_attn_norm_weight,
                                gate_up_weight, down_proj_weight, down_proj_bias, length):
        return None
    with torch.cuda.device(h.device):   # the persistent hand-off area is per device: the current one
        return _full_layer_launch(h, qkv_weight, input_layernorm_weight, q_norm_weight, k_norm_weight, cos, sin,
                                  k_cache, v_cache, cache_position, o_proj_weight, post_attn_norm_weight,
                                  gate_up_weight, down_proj_weight, eps, attn_scale, workspace, length)


def _layer_stack_launch(h, layers, cos, sin, cache_position, lengths, out, status, eps, attn_scale) -> bool:
    """Consecutive decoder layers as one persistent launch
    (qd_decoder_layers_persistent_f16): ``layers`` holds per layer the tuple
    (qkv, o_proj, gate_up, down, input_norm, post_norm, q_norm, k_norm,
    k_cache, v_cache), each layer already checked with _full_layer_eligible
    and all caches of one capacity; ``lengths`` per layer a running-length
    word or None; ``out`` fp16 [n, 2048] receives every layer's output.
    False when the device cannot keep the grid resident."""
    with torch.cuda.device(h.device):
        if not _persistent_layer_device_ok(h.device):
            return False
        n = len(layers)
        descs = (_lib.LayerDesc * n)()
        for d, t in zip(descs, layers):
            (d.qkv, d.o_proj, d.gate_up, d.down, d.input_norm, d.post_norm, d.q_norm, d.k_norm, d.k_cache,
             d.v_cache) = (x.data_ptr() for x in t)
        lens = (ctypes.c_void_p * n)(*[(L.data_ptr() if L is not None else None) for L in lengths])
        _check(_load_ext().qd_decoder_layers_persistent_f16(
            _p(h.reshape(-1)), ctypes.cast(descs, ctypes.c_void_p), n, int(layers[0][8].shape[2]),
            _p(cache_position), _p(cos), _p(sin), float(eps), float(attn_scale), _p(out),
            ctypes.cast(lens, ctypes.c_void_p), _p(status), _stream(h)), "qd_decoder_layers_persistent_f16")
        return True


def _full_layer_launch(h, qkv_weight, input_layernorm_weight, q_norm_weight, k_norm_weight, cos, sin, k_cache,
                       v_cache, cache_position, o_proj_weight, post_attn_norm_weight, gate_up_weight,
                       down_proj_weight, eps, attn_scale, workspace, length):
    if not _persistent_layer_device_ok(h.device):
        return None
    ws = workspace if workspace is not None else {}
    if not (ws.get("type") == _FULL_LAYER_KIND and "out" in ws and "status" in ws and ws["out"].device == h.device):
        ws.clear()
        ws.update(type=_FULL_LAYER_KIND, out=torch.empty(2048, dtype=torch.float16, device=h.device),
                  status=torch.zeros(1, dtype=torch.int32, device=h.device))
    out = ws["out"]
    x = h.reshape(-1)
    w = _lib.LayerDesc(qkv=qkv_weight.data_ptr(), o_proj=o_proj_weight.data_ptr(), gate_up=gate_up_weight.data_ptr(),
                       down=down_proj_weight.data_ptr(), input_norm=input_layernorm_weight.data_ptr(),
                       post_norm=post_attn_norm_weight.data_ptr(), q_norm=q_norm_weight.data_ptr(),
                       k_norm=k_norm_weight.data_ptr(), k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr())
    _check(_load_ext().qd_decoder_layer_persistent_f16(
        _p(x), ctypes.byref(w), int(k_cache.shape[2]), _p(cache_position), _p(cos), _p(sin), float(eps),
        float(attn_scale), _p(out), _p(length), _p(ws["status"]), _stream(h)), "fused_decode_full_layer_softsync_half")
    return out.view(*h.shape[:-1], 2048)


def fused_decode_full_layer_softsync_half(hidden_states, qkv_weight, input_layernorm_weight, q_norm_weight,
                                          k_norm_weight, cos, sin, k_cache, v_cache, cache_position, o_proj_weight,
                                          o_proj_bias, post_attn_norm_weight, gate_up_weight, down_proj_weight,
                                          down_proj_bias, eps, attn_scale, workspace=None, launch_blocks=None):
    """One full decoder layer for one token (reference fused.py:498-665): QKV,
    q/k norm + RoPE + KV write, attention, o_proj and MLP.  At the Qwen3-VL-2B
    shapes this is one persistent launch (the reference's one-launch soft-sync
    layer); elsewhere the layer chain of the separate kernels."""
    import cuda_decode_attention
    import cuda_decode_small_ops

    del launch_blocks
    name = "fused_decode_full_layer_softsync_half"
    _require_decode_half(name, hidden_states, qkv_weight, x=hidden_states)
    out = _full_layer_persistent(hidden_states, qkv_weight, input_layernorm_weight, q_norm_weight, k_norm_weight,
                                 cos, sin, k_cache, v_cache, cache_position, o_proj_weight, o_proj_bias,
                                 post_attn_norm_weight, gate_up_weight, down_proj_weight, down_proj_bias, eps,
                                 attn_scale, workspace)
    if out is not None:
        return out
    hkv, d = k_cache.shape[1], k_cache.shape[3]
    hq = (qkv_weight.shape[0] - 2 * hkv * d) // d
    qkv = fused_rmsnorm_qkv_half(hidden_states, input_layernorm_weight, qkv_weight, None, eps).reshape(-1)
    q = qkv[: hq * d].view(1, 1, hq, d)
    k = qkv[hq * d: (hq + hkv) * d].view(1, 1, hkv, d)
    v = qkv[(hq + hkv) * d:].view(1, 1, hkv, d)
    q_rot = cuda_decode_small_ops.fused_q_rope_kv_cache_update(q, k, v, q_norm_weight, k_norm_weight, eps, cos, sin,
                                                               k_cache, v_cache, cache_position)
    attn = cuda_decode_attention.decode_attn_v4_cta_qhead_splitkv_fused(
        q_rot.transpose(1, 2), k_cache, v_cache, attn_scale, hq // hkv, cache_position)
    if attn is None:
        raise RuntimeError(f"{name}: unsupported attention shape")
    attn = attn.reshape(*hidden_states.shape[:-1], hq * d)
    _hidden, out = fused_o_proj_post_attn_mlp_persistent_half(hidden_states, attn, o_proj_weight, o_proj_bias,
                                                              post_attn_norm_weight, gate_up_weight,
                                                              down_proj_weight, down_proj_bias, eps, workspace)
    return out


def decode_attn_persistent_half(q, k_cache, v_cache, cache_position, scale, workspace=None):
    """Decode attention returning [1, Hq, 1, D] (reference fused.py:895-965)."""
    import cuda_decode_attention

    if (q.device.type != "cuda" or k_cache.device.type != "cuda" or v_cache.device.type != "cuda"
            or q.dtype != torch.float16 or k_cache.dtype != torch.float16 or v_cache.dtype != torch.float16):
        raise RuntimeError("decode_attn_persistent_half expects fp16 CUDA tensors")
    if q.ndim == 4:
        hq, d = q.shape[1], q.shape[3]
    elif q.ndim == 3:
        hq, d = q.shape[1], q.shape[2]
    else:
        raise RuntimeError("q must be 3D or 4D")
    q4 = q.reshape(1, hq, 1, d)
    out = cuda_decode_attention.decode_attn_v4_fused(q4, k_cache, v_cache, scale, hq // k_cache.shape[1],
                                                     cache_position)
    if out is None:
        raise RuntimeError("decode_attn_persistent_half: unsupported shape")
    return out.reshape(1, hq, 1, d)
