"""Small fused ops parity on the GPU: q/k head RMSNorm + RoPE + static-KV
write, add+RMSNorm, RMSNorm, SiLU*mul, add (against the CPU oracle)."""

from __future__ import annotations

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu


def _qkv(seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, 1, 16, 128, generator=g).half()
    k = torch.randn(1, 1, 8, 128, generator=g).half()
    v = torch.randn(1, 1, 8, 128, generator=g).half()
    qw = (1 + 0.02 * torch.randn(128, generator=g)).half()
    kw = (1 + 0.02 * torch.randn(128, generator=g)).half()
    return q, k, v, qw, kw


def _cos_sin_fp16(pos: int):
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), pos, dtype=torch.int64))
    return cos.half().view(1, 1, 128), sin.half().view(1, 1, 128)


@pytest.mark.parametrize("pos,T", [(512, 513), (0, 64), (4095, 4096), (700, 1024)])
def test_fused_q_rope_kv_cache_update(cuda, pos, T):
    import cuda_decode_small_ops as S

    q, k, v, qw, kw = _qkv(pos)
    cos, sin = _cos_sin_fp16(pos)
    kc = torch.randn(1, 8, T, 128, generator=torch.Generator().manual_seed(1)).half()
    vc = torch.randn(1, 8, T, 128, generator=torch.Generator().manual_seed(2)).half()
    kc_d, vc_d = kc.to(cuda), vc.to(cuda)
    cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
    print(f"case q_rope_kv pos={pos} T={T}", flush=True)
    q_out = S.fused_q_rope_kv_cache_update(q.to(cuda), k.to(cuda), v.to(cuda), qw.to(cuda), kw.to(cuda), 1e-6,
                                           cos.to(cuda), sin.to(cuda), kc_d, vc_d, cp)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q_ref = O.q_rope_kv_update(q.reshape(16, 128), k.reshape(8, 128), v.reshape(8, 128), qw, kw, 1e-6,
                               cos.reshape(128), sin.reshape(128), kc_ref, vc_ref, pos)
    assert q_out.shape == (1, 1, 16, 128)
    assert_close_rel(q_out.reshape(16, 128), q_ref, what="q_rot")
    kc_got, vc_got = kc_d.cpu(), vc_d.cpu()
    assert_close_rel(kc_got[0, :, pos], kc_ref[0, :, pos].float(), what="k row")
    assert torch.equal(vc_got[0, :, pos], v.reshape(8, 128))            # V is copied bit-exactly
    mask = torch.ones(T, dtype=torch.bool)
    mask[pos] = False
    assert torch.equal(kc_got[0, :, mask], kc[0, :, mask])              # nothing else touched
    assert torch.equal(vc_got[0, :, mask], vc[0, :, mask])


def test_q_rope_out_of_range_position_writes_nothing(cuda):
    import cuda_decode_small_ops as S

    q, k, v, qw, kw = _qkv(3)
    cos, sin = _cos_sin_fp16(10)
    kc = torch.zeros(1, 8, 16, 128, dtype=torch.float16, device=cuda)
    vc = torch.zeros_like(kc)
    cp = torch.tensor([16], dtype=torch.int64, device=cuda)
    S.fused_q_rope_kv_cache_update(q.to(cuda), k.to(cuda), v.to(cuda), qw.to(cuda), kw.to(cuda), 1e-6,
                                   cos.to(cuda), sin.to(cuda), kc, vc, cp)
    assert kc.abs().sum().item() == 0 and vc.abs().sum().item() == 0


def test_q_rope_position_mode_fp32(cuda):
    """Device-side M-RoPE from (T, H, W) positions with fp32 q/k/v (the decode
    engine's form), including distinct H/W streams."""
    from qwen3vl_hip import _lib
    from qwen3vl_hip.engine import rope_inv_freq

    q, k, v, qw, kw = _qkv(9)
    pos3 = torch.tensor([1234, 57, 981], dtype=torch.int64)
    cos, sin = O.mrope_cos_sin(pos3.view(3, 1))
    T, cpos = 2048, 1500
    qkv = torch.cat([q.reshape(-1), k.reshape(-1), v.reshape(-1)]).float().to(cuda)
    kc = torch.zeros(1, 8, T, 128, dtype=torch.float16, device=cuda)
    vc = torch.zeros_like(kc)
    q_out = torch.empty(16, 128, dtype=torch.float32, device=cuda)
    inv = rope_inv_freq().to(cuda)
    rp, cp = pos3.to(cuda), torch.tensor([cpos], device=cuda)
    qw_d, kw_d = qw.to(cuda), kw.to(cuda)   # device copies stay referenced across the launch
    _lib.check(_lib.lib().qd_q_rope_kv_update(
        _lib.ptr(qkv), _lib.ptr(qkv[2048:]), _lib.ptr(qkv[3072:]), _lib.QD_F32, 128, 128, 128, _lib.ptr(qw_d),
        _lib.ptr(kw_d), 1e-6, None, None, _lib.ptr(rp), _lib.ptr(inv), 24, 20, 20, _lib.ptr(q_out),
        _lib.QD_F32, _lib.ptr(kc), _lib.ptr(vc), T * 128, 128, T, _lib.ptr(cp), 16, 8, _lib.stream()), "rope")
    kc_ref = torch.zeros(1, 8, T, 128, dtype=torch.float16)
    vc_ref = torch.zeros_like(kc_ref)
    q_ref = O.q_rope_kv_update(q.reshape(16, 128), k.reshape(8, 128), v.reshape(8, 128), qw, kw, 1e-6, cos[0],
                               sin[0], kc_ref, vc_ref, cpos)
    assert_close_rel(q_out, q_ref, rel=1e-4, what="q_rot position mode")
    assert_close_rel(kc[0, :, cpos], kc_ref[0, :, cpos].float(), what="k row position mode")


def test_fused_qk_rms_norm_rope(cuda):
    import cuda_decode_small_ops as S

    g = torch.Generator().manual_seed(4)
    M = 5
    q = torch.randn(1, M, 16, 128, generator=g).half()
    k = torch.randn(1, M, 8, 128, generator=g).half()
    qw = (1 + 0.02 * torch.randn(128, generator=g)).half()
    kw = (1 + 0.02 * torch.randn(128, generator=g)).half()
    cos, sin = O.mrope_cos_sin(torch.arange(100, 100 + M).view(1, M).expand(3, M))
    cos16, sin16 = cos.half().view(1, M, 128), sin.half().view(1, M, 128)
    qo, ko = S.fused_qk_rms_norm_rope(q.to(cuda), k.to(cuda), qw.to(cuda), kw.to(cuda), 1e-6, cos16.to(cuda),
                                      sin16.to(cuda))
    c, s = cos16.float().view(M, 1, 128), sin16.float().view(M, 1, 128)
    q_ref = O.apply_rope(O.rms_norm(q.view(M, 16, 128), qw, 1e-6), c, s)
    k_ref = O.apply_rope(O.rms_norm(k.view(M, 8, 128), kw, 1e-6), c, s)
    assert_close_rel(qo.view(M, 16, 128), q_ref, what="qk_norm_rope q")
    assert_close_rel(ko.view(M, 8, 128), k_ref, what="qk_norm_rope k")


@pytest.mark.parametrize("rows,cols", [(1, 2048), (3, 2048), (2, 1000)])
def test_add_rms_norm_and_rms_norm(cuda, rows, cols):
    import cuda_decode_small_ops as S

    g = torch.Generator().manual_seed(rows * cols)
    r = torch.randn(rows, cols, generator=g).half()
    x = torch.randn(rows, cols, generator=g).half()
    w = (1 + 0.02 * torch.randn(cols, generator=g)).half()
    s_sum, s_norm = S.fused_add_rms_norm(r.to(cuda), x.to(cuda), w.to(cuda), 1e-6)
    ref_sum = r.float() + x.float()
    assert_close_rel(s_sum, ref_sum, what="add_rms_norm sum")
    assert_close_rel(s_norm, O.rms_norm(ref_sum, w, 1e-6), what="add_rms_norm norm")
    n = S.rms_norm(x.to(cuda), w.to(cuda), 1e-6)
    assert_close_rel(n, O.rms_norm(x, w, 1e-6), what="rms_norm")


def test_silu_mul_and_add(cuda):
    import cuda_decode_small_ops as S

    g = torch.Generator().manual_seed(8)
    a = torch.randn(6144, generator=g).half()
    b = torch.randn(6144, generator=g).half()
    assert_close_rel(S.fused_silu_mul(a.to(cuda), b.to(cuda)), O.silu_mul(a, b), what="silu_mul")
    assert_close_rel(S.add(a.to(cuda), b.to(cuda)), a.float() + b.float(), what="add")


def test_small_ops_reject_bad_dtype(cuda):
    import cuda_decode_small_ops as S

    with pytest.raises(RuntimeError):
        S.add(torch.randn(8, device=cuda), torch.randn(8, device=cuda))
    with pytest.raises(RuntimeError):
        S.rms_norm(torch.randn(2, 8, device=cuda).half(), torch.ones(4, device=cuda).half(), 1e-6)
