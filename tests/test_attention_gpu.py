"""Split-KV GQA decode attention parity on the GPU (config 2) against the
CPU oracle's fp32 softmax attention.

Bar: max |gpu - oracle| <= 2e-3 * max |oracle|.
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _run(fn, q, kc, vc, pos, cuda, **kw):
    qd = q.to(cuda)
    cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
    out = fn(qd, kc.to(cuda), vc.to(cuda), SCALE, 2, cp, **kw)
    assert out is not None
    assert out.shape == (1, 1, 16, 128)
    return out.reshape(16, 128)


@pytest.mark.parametrize("L", [256, 1024, 4096, 8192, 32768])   # config 2, and a 32K context
@pytest.mark.parametrize("stale", [False, True])
def test_attention_config2(cuda, L, stale):
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    cap = L + 320 if stale else L
    q, kc, vc, pos = syn.attention_inputs(L, capacity=cap)
    print(f"case attention L={L} T={cap}", flush=True)
    out = _run(A.decode_attn_v4_cta_qhead_splitkv_fused, q, kc, vc, pos, cuda)
    ref = O.decode_attention(q.reshape(16, 128), kc, vc, pos, SCALE)
    assert_close_rel(out, ref, what=f"attention L={L} T={cap}")


@pytest.mark.parametrize("split_k", [2, 4, 16, 64, 200])
def test_attention_split_count_invariance(cuda, split_k):
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    q, kc, vc, pos = syn.attention_inputs(1024, capacity=1100)
    ref = O.decode_attention(q.reshape(16, 128), kc, vc, pos, SCALE)
    out = _run(A.decode_attn_v4_fused, q, kc, vc, pos, cuda, split_k=split_k)
    assert_close_rel(out, ref, what=f"split_k={split_k}")


@pytest.mark.parametrize("L", [1024, 4096, 8192])   # 8 / 16 / 16 default splits
def test_attention_partial_merge_matches_fused(cuda, L):
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    q, kc, vc, pos = syn.attention_inputs(L)
    fused = _run(A.decode_attn_v4_fused, q, kc, vc, pos, cuda)
    two = _run(A.decode_attn_v4_splitkv, q, kc, vc, pos, cuda)
    # same partials; the in-kernel merge (last split of a kv head) and the merge
    # kernel sum the splits in different orders, so the fp16 outputs may differ
    # by one rounding step: at most 2^-10 of the largest output
    assert_close_rel(fused.cpu(), two.cpu(), rel=2.0 ** -10, what="one-launch vs two-launch merge")


def test_attention_length_one_returns_v0(cuda):
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    q, kc, vc, _ = syn.attention_inputs(256, capacity=512)
    out = _run(A.decode_attn_v4_cta_qhead_splitkv_fused, q, kc, vc, 0, cuda).cpu()
    expect = vc[0, :, 0, :].repeat_interleave(2, 0)
    assert torch.equal(out, expect)


def test_attention_equal_keys_give_mean_of_values(cuda):
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    q, kc, vc, pos = syn.attention_inputs(1024)
    kc[:] = kc[:, :, :1, :]  # every key identical -> uniform softmax
    out = _run(A.decode_attn_v4_cta_qhead_splitkv_fused, q, kc, vc, pos, cuda)
    expect = vc[0].float().mean(1).repeat_interleave(2, 0)
    assert_close_rel(out, expect, what="equal keys")


@pytest.mark.parametrize("T,split_k", [(1024, 4), (2048, 32)])   # one launch (arrival counters); two launches
def test_attention_graph_replay_self_resets(cuda, T, split_k):
    """Capture once, replay at several cache positions: the arrival counters
    reset themselves, so every replay matches the eager result and the oracle."""
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    q, kc, vc, _ = syn.attention_inputs(T)
    qd, kd, vd = q.to(cuda), kc.to(cuda), vc.to(cuda)
    cp = torch.tensor([100], dtype=torch.int64, device=cuda)
    ws: dict = {}
    A.decode_attn_v4_cta_qhead_splitkv_fused(qd, kd, vd, SCALE, 2, cp, split_k=split_k, workspace=ws)  # warm-up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = A.decode_attn_v4_cta_qhead_splitkv_fused(qd, kd, vd, SCALE, 2, cp, split_k=split_k, workspace=ws)
    for pos in (100, T - 1, 5, T // 2 - 1, T + 100):
        cp.fill_(pos)
        g.replay()
        torch.cuda.synchronize()
        got = out.reshape(16, 128).clone()
        eager = A.decode_attn_v4_cta_qhead_splitkv_fused(qd, kd, vd, SCALE, 2, cp, split_k=split_k,
                                                         workspace={})
        torch.cuda.synchronize()
        assert torch.equal(got, eager.reshape(16, 128))
        assert_close_rel(got, O.decode_attention(q.reshape(16, 128), kc, vc, pos, SCALE), what=f"replay pos={pos}")


@pytest.mark.parametrize("pos,cap", [(0, 64), (700, 1024), (4095, 4096)])
def test_qkv_rope_attention_matches_the_two_call_sequence(cuda, pos, cap):
    """The one-launch q/k norm + RoPE + K/V write + attention of the drop-in
    layer against the reference's two calls (fused_q_rope_kv_cache_update,
    then decode attention) on the same inputs: identical cache rows (V exact,
    K within one fp16 step), attention within the bar (the one-launch form
    keeps the rotated q in fp32), and against the oracle."""
    import cuda_decode_attention as A
    import cuda_decode_small_ops as S
    from qwen3vl_hip import synthetic as syn

    print(f"case qkv attention pos={pos} cap={cap}", flush=True)
    lw = syn.layer_weights(4, 0)
    qkv = syn.normal(4, ("x", pos), (1, 1, 4096)).to(cuda)
    cos, sin = O.mrope_cos_sin(torch.tensor([[pos + 9], [pos + 3], [pos + 5]]))
    cos16, sin16 = cos.half().reshape(128).to(cuda), sin.half().reshape(128).to(cuda)
    kc = syn.normal(4, ("k", pos), (1, 8, cap, 128))
    vc = syn.normal(4, ("v", pos), (1, 8, cap, 128))
    kc[:, :, pos:] = 7.0   # stale rows at and after the new position
    vc[:, :, pos:] = -7.0
    cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
    qn, kn = lw.q_norm_weight.to(cuda), lw.k_norm_weight.to(cuda)
    k1, v1 = kc.to(cuda), vc.to(cuda)
    one = A._qkv_rope_attention(qkv, qn, kn, 1e-6, cos16, sin16, k1, v1, SCALE, cp, workspace={})
    assert one is not None and one.shape == (1, 1, 16, 128)
    k2, v2 = kc.to(cuda), vc.to(cuda)
    q, k, v = qkv.split([2048, 1024, 1024], dim=-1)
    q_rot = S.fused_q_rope_kv_cache_update(q.view(1, 1, 16, 128), k.view(1, 1, 8, 128), v.view(1, 1, 8, 128),
                                           qn, kn, 1e-6, cos16.view(1, 1, 128), sin16.view(1, 1, 128), k2, v2, cp)
    two = A.decode_attn_v4_cta_qhead_splitkv_fused(q_rot.transpose(1, 2), k2, v2, SCALE, 2, cp, workspace={})
    torch.cuda.synchronize()
    assert torch.equal(v1.cpu(), v2.cpu())
    assert torch.equal(k1[:, :, :pos].cpu(), k2[:, :, :pos].cpu()) and torch.equal(k1[:, :, pos + 1:].cpu(),
                                                                                  k2[:, :, pos + 1:].cpu())
    assert_close_rel(k1[0, :, pos].float().cpu(), k2[0, :, pos].float().cpu(), rel=2.0 ** -10, what="new K row")
    assert_close_rel(one.reshape(16, 128).float().cpu(), two.reshape(16, 128).float().cpu(), what="one vs two calls")
    ref = O.decode_attention(q_rot.reshape(16, 128).float().cpu(), k2.cpu(), v2.cpu(), pos, SCALE)
    assert_close_rel(one.reshape(16, 128).float().cpu(), ref, what="one launch vs oracle")


def test_attention_unsupported_returns_none(cuda):
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    q, kc, vc, pos = syn.attention_inputs(256)
    cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
    # head_dim 64 is not supported -> None (caller falls back)
    assert A.decode_attn_v4_fused(q[..., :64].contiguous().to(cuda), kc[..., :64].contiguous().to(cuda),
                                  vc[..., :64].contiguous().to(cuda), SCALE, 2, cp) is None


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 4), (32, 8)])       # GQA groups 1, 4, 4
@pytest.mark.parametrize("L,split_k", [(700, 4), (5000, 40)])          # merge in the partial kernel / merge kernel
def test_attention_other_gqa_groups(cuda, hq, hkv, L, split_k):
    """Group sizes 1 and 4, which the entry points accept besides Qwen3-VL's 2,
    against the oracle; one length merged by the last split of each kv head,
    one with enough splits for the separate merge launch, a stale tail."""
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    cap = L + 64
    q = syn.normal(11, ("q", hq, hkv, L), (1, hq, 1, 128))
    kc = syn.normal(11, ("k_cache", hq, hkv, L), (1, hkv, cap, 128))
    vc = syn.normal(11, ("v_cache", hq, hkv, L), (1, hkv, cap, 128))
    kc[:, :, L:] = 60000.0
    vc[:, :, L:] = 60000.0
    pos = L - 1
    print(f"case attention Hq={hq} Hkv={hkv} L={L} split_k={split_k}", flush=True)
    cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
    ref = O.decode_attention(q.reshape(hq, 128), kc, vc, pos, SCALE)
    for fn in (A.decode_attn_v4_cta_qhead_splitkv_fused, A.decode_attn_v4_splitkv):
        out = fn(q.to(cuda), kc.to(cuda), vc.to(cuda), SCALE, hq // hkv, cp, split_k=split_k)
        assert out is not None and out.shape == (1, 1, hq, 128)
        assert_close_rel(out.reshape(hq, 128), ref, what=f"{fn.__name__} Hq={hq} Hkv={hkv} L={L}")


def test_grouped_prefix_entry_points(cuda):
    """The reference's older split-KV entry points (cuda_decode_attention.py:90-215)
    give the same attention, and decline a split count of 1 as the reference does."""
    import cuda_decode_attention as A
    from qwen3vl_hip import synthetic as syn

    q, kc, vc, pos = syn.attention_inputs(1500, capacity=1600)
    ref = O.decode_attention(q.reshape(16, 128), kc, vc, pos, SCALE)
    for fn in (A.grouped_prefix_cachepos_splitkv, A.grouped_prefix_cachepos_splitkv_qhead):
        print(f"case {fn.__name__}", flush=True)
        cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
        assert fn(q.to(cuda), kc.to(cuda), vc.to(cuda), SCALE, 2, cp, 1) is None
        out = fn(q.to(cuda), kc.to(cuda), vc.to(cuda), SCALE, 2, cp, 8)
        assert out is not None
        assert_close_rel(out.reshape(16, 128), ref, what=fn.__name__)
