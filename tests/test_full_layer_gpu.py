"""The one-launch decoder layer (qd_decoder_layer_persistent_f16 behind
cuda_decode_gemv.fused_decode_full_layer_softsync_half, reference
cuda_decode_gemv_ops/fused.py:498-665) on the GPU against the CPU oracle's
layer, the kernel chain, and itself under graph capture.

Bar: max |gpu - oracle| <= 2e-3 * max |oracle|; the new
K row within one fp16 step of the oracle's, rows other than the new one
untouched.
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _inputs(seed, pos, cap):
    from qwen3vl_hip import synthetic as syn

    inp = syn.layer_step_inputs(seed=seed, cache_position=pos, capacity=cap)
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), pos + 7, dtype=torch.int64))
    return inp, cos.half().reshape(128), sin.half().reshape(128)


def _call(lw, hidden, cos16, sin16, kc, vc, cp, workspace=None):
    import cuda_decode_gemv

    return cuda_decode_gemv.fused_decode_full_layer_softsync_half(
        hidden, lw.qkv_weight, lw.input_layernorm_weight, lw.q_norm_weight, lw.k_norm_weight, cos16, sin16, kc, vc,
        cp, lw.o_proj_weight, None, lw.post_attn_layernorm_weight, lw.gate_up_weight, lw.down_proj_weight, None,
        1e-6, SCALE, workspace=workspace)


@pytest.mark.parametrize("pos,cap", [(0, 64), (512, 640), (4095, 4096), (8000, 8192), (30000, 32768)])
def test_full_layer_matches_oracle(cuda, pos, cap):
    """The layer output, the K/V row written at the position and the rest of
    the cache against the oracle's decoder layer on the same fp16 inputs."""
    print(f"case full layer pos={pos} cap={cap}", flush=True)
    inp, cos16, sin16 = _inputs(5, pos, cap)
    lw = inp.weights.to(cuda)
    kc, vc = inp.k_cache.to(cuda), inp.v_cache.to(cuda)
    cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
    ws: dict = {}
    out = _call(lw, inp.hidden.to(cuda), cos16.to(cuda), sin16.to(cuda), kc, vc, cp, ws)
    torch.cuda.synchronize()
    assert out.shape == (1, 1, 2048) and out.dtype == torch.float16
    assert int(ws["status"].item()) == 0, "a hand-off wait ran out of its polling budget"
    kc_ref, vc_ref = inp.k_cache.clone(), inp.v_cache.clone()
    ref = O.decode_layer(inp.weights.tensors(), inp.hidden.reshape(-1), kc_ref, vc_ref, pos, cos16.float(),
                         sin16.float())
    assert_close_rel(out.reshape(-1).float().cpu(), ref, what=f"one-launch layer pos={pos}")
    assert_close_rel(kc[0, :, pos].float().cpu(), kc_ref[0, :, pos].float(), rel=2.0 ** -10, what="new K row")
    assert_close_rel(vc[0, :, pos].float().cpu(), vc_ref[0, :, pos].float(), rel=2.0 ** -10, what="new V row")
    others = torch.ones(cap, dtype=torch.bool)
    others[pos] = False
    assert torch.equal(kc[0][:, others].cpu(), inp.k_cache[0][:, others])
    assert torch.equal(vc[0][:, others].cpu(), inp.v_cache[0][:, others])


def test_full_layer_agrees_with_the_chain(cuda):
    """The swapped layer's two decode paths (one launch; the kernel chain with
    the full_layer_softsync fusion flag off) on the same state."""
    import types

    import optimized_layer
    from test_layer_gpu import _hf_layer

    inp, cos16, sin16 = _inputs(6, 1500, 2048)
    layer = optimized_layer.OptimizedDecoderLayer(_hf_layer(inp.weights)).to(cuda).half()
    outs = {}
    for one_launch in (True, False):
        prev = optimized_layer.set_cuda_mlp_fusion_flags(full_layer_softsync=one_launch)
        try:
            kc, vc = inp.k_cache.to(cuda), inp.v_cache.to(cuda)
            cache = types.SimpleNamespace(layers=[types.SimpleNamespace(keys=kc, values=vc, is_initialized=True,
                                                                        max_cache_len=kc.shape[2])])
            cp = torch.tensor([1500], dtype=torch.int64, device=cuda)
            outs[one_launch] = layer(inp.hidden.to(cuda), (cos16.view(1, 1, 128).to(cuda),
                                                           sin16.view(1, 1, 128).to(cuda)),
                                     past_key_values=cache, cache_position=cp).float().cpu()
        finally:
            optimized_layer.set_cuda_mlp_fusion_flags(full_layer_softsync=prev[1])
    assert layer._full_layer_workspace.get("out") is not None, "the one-launch path did not run"
    assert_close_rel(outs[True].reshape(-1), outs[False].reshape(-1), what="one launch vs chain")


@pytest.mark.parametrize("same_word", [False, True])
def test_full_layer_advances_the_running_length(cuda, same_word):
    """length_out = cache_position + 1 after the launch, also when it is the
    cache_position word itself (a static cache's running length used as the
    write row); the output is the one without the advance."""
    import cuda_decode_gemv_ops.fused as F

    inp, cos16, sin16 = _inputs(7, 300, 512)
    lw = inp.weights.to(cuda)
    h = inp.hidden.to(cuda)
    args = lambda kc, vc, cp, ws, length: F._full_layer_persistent(  # noqa: E731
        h, lw.qkv_weight, lw.input_layernorm_weight, lw.q_norm_weight, lw.k_norm_weight, cos16.to(cuda),
        sin16.to(cuda), kc, vc, cp, lw.o_proj_weight, None, lw.post_attn_layernorm_weight, lw.gate_up_weight,
        lw.down_proj_weight, None, 1e-6, SCALE, ws, length=length)
    cp0 = torch.tensor([300], dtype=torch.int64, device=cuda)
    plain = args(inp.k_cache.to(cuda), inp.v_cache.to(cuda), cp0, {}, None).clone()
    cp = torch.tensor([300], dtype=torch.int64, device=cuda)
    length = cp if same_word else torch.tensor([17], dtype=torch.int64, device=cuda)
    out = args(inp.k_cache.to(cuda), inp.v_cache.to(cuda), cp, {}, length)
    torch.cuda.synchronize()
    assert int(length.item()) == 301
    assert torch.equal(out, plain)


def test_full_layer_graph_replay(cuda):
    """One captured launch replayed at several cache positions (the position
    word rewritten between replays): every replay equals an eager call at that
    position bit for bit, and the oracle."""
    inp, _, _ = _inputs(8, 100, 1024)
    lw = inp.weights.to(cuda)
    h = inp.hidden.to(cuda)
    kc, vc = inp.k_cache.to(cuda), inp.v_cache.to(cuda)
    cp = torch.tensor([100], dtype=torch.int64, device=cuda)
    cos_d = torch.empty(128, dtype=torch.float16, device=cuda)
    sin_d = torch.empty_like(cos_d)
    ws: dict = {}
    _call(lw, h, cos_d.fill_(1.0), sin_d.zero_(), kc, vc, cp, ws)   # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = _call(lw, h, cos_d, sin_d, kc, vc, cp, ws)
    for pos in (100, 1023, 5, 511):
        print(f"case graph replay pos={pos}", flush=True)
        cos, sin = O.mrope_cos_sin(torch.full((3, 1), pos, dtype=torch.int64))
        cos16, sin16 = cos.half().reshape(128), sin.half().reshape(128)
        cos_d.copy_(cos16)
        sin_d.copy_(sin16)
        cp.fill_(pos)
        kc.copy_(inp.k_cache)
        vc.copy_(inp.v_cache)
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        k_got = kc[0, :, pos].clone()
        kc.copy_(inp.k_cache)
        vc.copy_(inp.v_cache)
        eager = _call(lw, h, cos_d, sin_d, kc, vc, cp, {})
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay at {pos} differs from the eager call"
        assert torch.equal(k_got, kc[0, :, pos])
        kc_ref, vc_ref = inp.k_cache.clone(), inp.v_cache.clone()
        ref = O.decode_layer(inp.weights.tensors(), inp.hidden.reshape(-1), kc_ref, vc_ref, pos, cos16.float(),
                             sin16.float())
        assert_close_rel(got.reshape(-1).float().cpu(), ref, what=f"replay pos={pos}")
    assert int(ws["status"].item()) == 0


def test_full_layer_declines_inputs_it_does_not_take(cuda):
    """The one-launch layer returns None (the caller then runs the kernel
    chain, as the reference's optimized_layer.py:1511-1600 falls back) for a
    projection bias, non-contiguous cos / sin, a non-contiguous cache or a
    non-int64 position; on its own inputs it runs."""
    import cuda_decode_gemv_ops.fused as F

    inp, cos16, sin16 = _inputs(9, 40, 64)
    lw = inp.weights.to(cuda)
    h = inp.hidden.to(cuda)
    kc, vc = inp.k_cache.to(cuda), inp.v_cache.to(cuda)
    cp = torch.tensor([40], dtype=torch.int64, device=cuda)
    cos_d, sin_d = cos16.to(cuda), sin16.to(cuda)

    def call(**kw):
        args = dict(o_proj_bias=None, down_proj_bias=None, cos=cos_d, sin=sin_d, k_cache=kc, v_cache=vc,
                    cache_position=cp)
        args.update(kw)
        return F._full_layer_persistent(h, lw.qkv_weight, lw.input_layernorm_weight, lw.q_norm_weight,
                                        lw.k_norm_weight, args["cos"], args["sin"], args["k_cache"],
                                        args["v_cache"], args["cache_position"], lw.o_proj_weight,
                                        args["o_proj_bias"], lw.post_attn_layernorm_weight, lw.gate_up_weight,
                                        lw.down_proj_weight, args["down_proj_bias"], 1e-6, SCALE, {})

    bias = torch.zeros(2048, dtype=torch.float16, device=cuda)
    assert call(o_proj_bias=bias) is None
    assert call(down_proj_bias=bias) is None
    strided = torch.stack([cos_d, cos_d], dim=1)[:, 0]          # 128 values, stride 2
    assert not strided.is_contiguous() and call(cos=strided) is None
    wide = torch.zeros(1, 8, 64, 256, dtype=torch.float16, device=cuda)[..., :128]
    assert call(k_cache=wide) is None
    assert call(cache_position=cp.to(torch.int32)) is None
    # contiguous but 8 bytes off a 16-byte boundary: the launch reads 16-byte rows
    shifted = torch.zeros(8 * 64 * 128 + 4, dtype=torch.float16, device=cuda)[4:].view(1, 8, 64, 128)
    assert shifted.is_contiguous() and shifted.data_ptr() % 16 == 8 and call(k_cache=shifted) is None
    out = call()
    torch.cuda.synchronize()
    assert out is not None and out.shape == (1, 1, 2048)


def test_full_layer_exhausted_polling_budget_is_reported(cuda):
    """The one-launch layer with a one-poll budget (forced from the host)
    finishes and sets bit 0 of its status word; with the default budget again
    the next launch reports nothing and equals the oracle's layer."""
    from qwen3vl_hip import _lib

    inp, cos16, sin16 = _inputs(10, 300, 512)
    lw = inp.weights.to(cuda)
    h = inp.hidden.to(cuda)
    cp = torch.tensor([300], dtype=torch.int64, device=cuda)
    lib = _lib.lib()
    print("case one-launch layer with a one-poll budget", flush=True)
    _lib.check(lib.qd_persistent_set_spin_limit(1), "qd_persistent_set_spin_limit")
    try:
        ws: dict = {}
        _call(lw, h, cos16.to(cuda), sin16.to(cuda), inp.k_cache.to(cuda), inp.v_cache.to(cuda), cp, ws)
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.qd_persistent_set_spin_limit(0), "qd_persistent_set_spin_limit")
    assert int(ws["status"].item()) & 1, "a launch with a one-poll budget reported no exhausted wait"
    # a wait that gave up hands its readers NaN, which reaches the output
    assert torch.isnan(ws["out"].float()).any(), "the output of a failed launch looks valid"
    ws = {}
    out = _call(lw, h, cos16.to(cuda), sin16.to(cuda), inp.k_cache.to(cuda), inp.v_cache.to(cuda), cp, ws)
    torch.cuda.synchronize()
    assert int(ws["status"].item()) == 0
    ref = O.decode_layer(inp.weights.tensors(), inp.hidden.reshape(-1), inp.k_cache.clone(), inp.v_cache.clone(), 300,
                         cos16.float(), sin16.float())
    assert_close_rel(out.reshape(-1).float().cpu(), ref, what="one-launch layer after an exhausted budget")


def test_dropin_layer_status_check_reports_an_exhausted_budget(cuda):
    """The swapped layer's one-launch decode step under a one-poll budget:
    optimized_layer.check_decode_status raises (naming the layer) and clears
    the word; with the default budget the next step checks clean."""
    import optimized_layer
    from qwen3vl_hip import _lib
    from test_layer_gpu import _hf_layer

    inp, cos16, sin16 = _inputs(12, 200, 512)
    layer = optimized_layer.OptimizedDecoderLayer(_hf_layer(inp.weights)).to(cuda).half()
    model = torch.nn.Module()
    model.layers = torch.nn.ModuleList([layer])
    kc, vc = inp.k_cache.to(cuda), inp.v_cache.to(cuda)
    cp = torch.tensor([200], dtype=torch.int64, device=cuda)
    pe = (cos16.to(cuda).reshape(1, 1, 128), sin16.to(cuda).reshape(1, 1, 128))

    import types

    cache = types.SimpleNamespace(layers=[types.SimpleNamespace(keys=kc, values=vc, is_initialized=True,
                                                                max_cache_len=kc.shape[2])])

    def step():
        return layer(inp.hidden.to(cuda).reshape(1, 1, 2048), pe, past_key_values=cache, cache_position=cp)

    lib = _lib.lib()
    step()
    torch.cuda.synchronize()
    optimized_layer.check_decode_status(model)            # clean
    print("case drop-in layer with a one-poll budget", flush=True)
    _lib.check(lib.qd_persistent_set_spin_limit(1), "qd_persistent_set_spin_limit")
    try:
        out = step()
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.qd_persistent_set_spin_limit(0), "qd_persistent_set_spin_limit")
    assert torch.isnan(out.float()).any()
    with pytest.raises(RuntimeError, match="layer 0"):
        optimized_layer.check_decode_status(model)
    optimized_layer.check_decode_status(model)            # the word was cleared
    out = step()
    torch.cuda.synchronize()
    optimized_layer.check_decode_status(model)
    assert not torch.isnan(out.float()).any()
