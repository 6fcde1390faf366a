"""One decoder layer, one decode step (config 0) on the GPU against the oracle.

Two product paths are checked: the drop-in ``OptimizedDecoderLayer`` built
from a transformers ``Qwen3VLTextDecoderLayer`` (fp16 activations between
kernels, HF fp16 cos/sin; on a stand-in cache and on transformers' own
``StaticCache`` over consecutive steps), and the native decode step of the
engine (fp32 activations between kernels, device-side M-RoPE) on a 1-layer
model.
"""

from __future__ import annotations

import types

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu


def _hf_layer(lw):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextDecoderLayer

    cfg = Qwen3VLTextConfig(hidden_size=2048, intermediate_size=6144, num_attention_heads=16,
                            num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, num_hidden_layers=1,
                            vocab_size=1024)
    cfg._attn_implementation = "sdpa"
    layer = Qwen3VLTextDecoderLayer(cfg, 0)
    a, m = layer.self_attn, layer.mlp
    with torch.no_grad():
        a.q_proj.weight.copy_(lw.qkv_weight[:2048].float())
        a.k_proj.weight.copy_(lw.qkv_weight[2048:3072].float())
        a.v_proj.weight.copy_(lw.qkv_weight[3072:].float())
        a.o_proj.weight.copy_(lw.o_proj_weight.float())
        a.q_norm.weight.copy_(lw.q_norm_weight.float())
        a.k_norm.weight.copy_(lw.k_norm_weight.float())
        m.gate_proj.weight.copy_(lw.gate_up_weight[:6144].float())
        m.up_proj.weight.copy_(lw.gate_up_weight[6144:].float())
        m.down_proj.weight.copy_(lw.down_proj_weight.float())
        layer.input_layernorm.weight.copy_(lw.input_layernorm_weight.float())
        layer.post_attention_layernorm.weight.copy_(lw.post_attn_layernorm_weight.float())
    return layer


@pytest.fixture(params=[True, False], ids=["one_launch", "chain"])
def layer_path(request):
    """The swapped layer's two decode paths: the one-launch persistent layer
    (default) and the kernel chain (full_layer_softsync fusion flag off)."""
    import optimized_layer

    prev = optimized_layer.set_cuda_mlp_fusion_flags(full_layer_softsync=request.param)
    yield request.param
    optimized_layer.set_cuda_mlp_fusion_flags(full_layer_softsync=prev[1])


def test_optimized_decoder_layer_config0(cuda, layer_path):
    import optimized_layer
    from qwen3vl_hip import synthetic as syn

    inp = syn.layer_step_inputs(seed=0, cache_position=512, capacity=640)
    lw = inp.weights
    layer = optimized_layer.OptimizedDecoderLayer(_hf_layer(lw)).to(cuda).half()
    kc, vc = inp.k_cache.to(cuda), inp.v_cache.to(cuda)
    cache = types.SimpleNamespace(layers=[types.SimpleNamespace(keys=kc, values=vc, is_initialized=True,
                                                                max_cache_len=kc.shape[2])])
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), inp.rope_position, dtype=torch.int64))
    cos16, sin16 = cos.half().view(1, 1, 128), sin.half().view(1, 1, 128)
    cp = torch.tensor([inp.cache_position], dtype=torch.int64, device=cuda)
    out = layer(inp.hidden.to(cuda), (cos16.to(cuda), sin16.to(cuda)), past_key_values=cache, cache_position=cp)
    assert out.shape == (1, 1, 2048) and out.dtype == torch.float16
    kc_ref, vc_ref = inp.k_cache.clone(), inp.v_cache.clone()
    ref = O.decode_layer(lw.tensors(), inp.hidden.reshape(-1), kc_ref, vc_ref, inp.cache_position,
                         cos16.float().reshape(128), sin16.float().reshape(128))
    assert_close_rel(out.reshape(-1), ref, what="OptimizedDecoderLayer decode step")
    assert_close_rel(kc[0, :, 512].cpu(), kc_ref[0, :, 512].float(), what="layer K write")
    assert torch.equal(kc[0, :, :512].cpu(), inp.k_cache[0, :, :512])


def test_optimized_decoder_layer_with_transformers_static_cache(cuda, layer_path):
    """The drop-in layer on transformers' own StaticCache (lazily initialised by
    the layer on its first call): three consecutive decode steps, each reading
    the K/V rows the previous ones wrote, against the oracle step by step."""
    from transformers.cache_utils import StaticCache
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig

    import optimized_layer
    from qwen3vl_hip import synthetic as syn

    inp = syn.layer_step_inputs(seed=3, cache_position=0, capacity=64)
    lw = inp.weights
    layer = optimized_layer.OptimizedDecoderLayer(_hf_layer(lw)).to(cuda).half()
    cfg = Qwen3VLTextConfig(hidden_size=2048, intermediate_size=6144, num_attention_heads=16,
                            num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, num_hidden_layers=1,
                            vocab_size=1024)
    cache = StaticCache(config=cfg, max_cache_len=64)
    kc_ref = torch.zeros(1, 8, 64, 128, dtype=torch.float16)
    vc_ref = torch.zeros_like(kc_ref)
    for pos in range(3):
        h = syn.normal(3, ("x", 100 + pos), (1, 1, 2048))
        cos, sin = O.mrope_cos_sin(torch.full((3, 1), pos, dtype=torch.int64))
        cos16, sin16 = cos.half().view(1, 1, 128), sin.half().view(1, 1, 128)
        cp = torch.tensor([pos], dtype=torch.int64, device=cuda)
        out = layer(h.to(cuda), (cos16.to(cuda), sin16.to(cuda)), past_key_values=cache, cache_position=cp)
        ref = O.decode_layer(lw.tensors(), h.reshape(-1), kc_ref, vc_ref, pos, cos16.float().reshape(128),
                             sin16.float().reshape(128))
        assert_close_rel(out.reshape(-1), ref, what=f"drop-in layer on StaticCache, step at {pos}")
    keys = cache.layers[0].keys
    assert keys.device.type == "cuda" and keys.shape == (1, 8, 64, 128)
    assert_close_rel(keys[0, :, :3].cpu(), kc_ref[0, :, :3].float(), what="StaticCache K rows 0..2")
    assert torch.count_nonzero(keys[0, :, 3:]) == 0   # rows past the last step untouched


def test_engine_phases_match_oracle_intermediates(cuda):
    """Each phase of the native step, run alone, against the oracle's value of
    the vector that phase produces (fp32 buffers, so the bar is tighter)."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import DecodeEngine

    w = syn.model_weights(0, num_layers=1)
    eng = DecodeEngine(w, capacity=640)
    inp = syn.layer_step_inputs(seed=0, cache_position=512, capacity=640)
    eng.k_caches[0].copy_(inp.k_cache)
    eng.v_caches[0].copy_(inp.v_cache)
    token = 4242
    eng.set_state(token, 512, 512)
    lw = w.layers[0].tensors()
    x0 = w.embed_tokens[token].float()
    qkv = O.gemv(O.rms_norm(x0, lw["input_layernorm_weight"], 1e-6), lw["qkv_weight"])
    kc, vc = inp.k_cache.clone(), inp.v_cache.clone()
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), 512, dtype=torch.int64))
    q_rot = O.q_rope_kv_update(qkv[:2048].view(16, 128), qkv[2048:3072].view(8, 128), qkv[3072:].view(8, 128),
                               lw["q_norm_weight"], lw["k_norm_weight"], 1e-6, cos[0], sin[0], kc, vc, 512)
    attn = O.decode_attention(q_rot, kc, vc, 512, 128 ** -0.5)
    hid, out, r = O.post_attn_mlp(x0, O.gemv(attn.reshape(-1), lw["o_proj_weight"]),
                                  lw["post_attn_layernorm_weight"], lw["gate_up_weight"], lw["down_proj_weight"],
                                  None, 1e-6)
    b = eng.buffers()
    expect = [("embed", "x", x0), ("qkv", "qkv", qkv), ("attn", "q_rot", q_rot.reshape(-1)),
              ("attn_merge", "attn", attn.reshape(-1)), ("o_proj", "r", r), ("gate_up", "hidden", hid),
              ("down", "x", out)]
    for phase, buf, ref in expect:
        print(f"case engine phase {phase}", flush=True)
        eng.run_phases([phase])
        torch.cuda.synchronize()
        assert_close_rel(b[buf].cpu(), ref, rel=1e-4 if phase in ("embed", "qkv") else REL_ENGINE,
                         what=f"engine phase {phase}")
        if phase == "attn":
            # fp32 K/V rounded to the fp16 cache: equal up to one fp16 rounding step
            assert_close_rel(eng.k_caches[0][0, :, 512].cpu(), kc[0, :, 512].float(), what="engine K row")
            assert_close_rel(eng.v_caches[0][0, :, 512].cpu(), vc[0, :, 512].float(), what="engine V row")
            mask = torch.ones(640, dtype=torch.bool)
            mask[512] = False
            assert torch.equal(eng.k_caches[0][0, :, mask].cpu(), inp.k_cache[0, :, mask])


REL_ENGINE = 2e-3


def test_engine_one_layer_step_config0(cuda):
    """Native step on a 1-layer model: logits and argmax against the oracle."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import DecodeEngine

    w = syn.model_weights(0, num_layers=1)
    eng = DecodeEngine(w, capacity=640, keep_logits=True)
    inp = syn.layer_step_inputs(seed=0, cache_position=512, capacity=640)
    eng.k_caches[0].copy_(inp.k_cache)
    eng.v_caches[0].copy_(inp.v_cache)
    token = 4242
    toks = eng.decode(token, 512, 0, 1, use_graph=False)
    kc_ref, vc_ref = inp.k_cache.clone(), inp.v_cache.clone()
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), 512, dtype=torch.int64))
    h = O.decode_layer(w.layers[0].tensors(), w.embed_tokens[token], kc_ref, vc_ref, 512, cos[0], sin[0])
    logits, tok = O.lm_head_argmax(h, w.final_norm_weight, w.embed_tokens, 1e-6)
    assert_close_rel(eng.logits.cpu(), logits, what="engine 1-layer logits")
    assert_close_rel(eng.k_caches[0][0, :, 512].cpu(), kc_ref[0, :, 512].float(), what="engine K write")
    print(f"engine token {toks[0]} oracle {tok} margin {O.top2_margin(logits):.4g}", flush=True)
    assert toks[0] == tok


@pytest.mark.parametrize("step_mode,splits,pos,poison", [
    ("chain", 0, 512, "nan"),     # 10 splits of 52 rows: the split holding pos clamps to the poisoned row
    ("chain", 2, 600, "inf"),     # 301 rows per split: three trips of the K/V loop, the new row in the third
    ("chain", 2, 600, None),
    ("chain", 1, 700, "nan"),     # one split of 701 rows (six loop trips)
    ("chain", 24, 600, "nan"),    # more than 16 splits: the merge kernel after the partials
    ("chain", 80, 1000, "inf"),   # more than 64 splits: the merge kernel's second chunk
    ("persistent", 0, 600, "nan"),
])
def test_engine_step_long_splits_and_poisoned_new_row(cuda, step_mode, splits, pos, poison):
    """Native step (1 layer) whose attention splits walk several batches of K/V
    rows, with the cache row of the new position (and every row after it)
    holding inf or NaN before the step, as a reused cache can.  The step must
    write the new row and never let the stale values reach the output: logits,
    token and the written K/V row against the oracle, and the rows after the
    new one untouched."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import DecodeEngine

    w = syn.model_weights(0, num_layers=1)
    cap = 1024
    eng = DecodeEngine(w, capacity=cap, keep_logits=True, attn_splits=splits, step_mode=step_mode)
    assert eng.step_mode == step_mode
    kc = syn.normal(7, ("k_cache", pos), (1, 8, cap, 128))
    vc = syn.normal(7, ("v_cache", pos), (1, 8, cap, 128))
    if poison is not None:
        bad = float(poison)
        kc[:, :, pos:] = bad
        vc[:, :, pos:] = bad
    eng.k_caches[0].copy_(kc)
    eng.v_caches[0].copy_(vc)
    token = 777
    print(f"case {step_mode} splits={splits} pos={pos} poison={poison}", flush=True)
    toks = eng.decode(token, pos, 0, 1, use_graph=False)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), pos, dtype=torch.int64))
    h = O.decode_layer(w.layers[0].tensors(), w.embed_tokens[token], kc_ref, vc_ref, pos, cos[0], sin[0])
    logits, tok = O.lm_head_argmax(h, w.final_norm_weight, w.embed_tokens, 1e-6)
    assert_close_rel(eng.logits.cpu(), logits, what=f"logits ({step_mode}, splits {splits}, pos {pos})")
    assert toks[0] == tok
    # V comes out of an fp32 GEMV whose summation order differs from the
    # oracle's, so its fp16 rounding may differ by an ulp: same bar as K
    assert_close_rel(eng.k_caches[0][0, :, pos].cpu(), kc_ref[0, :, pos].float(), what="K row written")
    assert_close_rel(eng.v_caches[0][0, :, pos].cpu(), vc_ref[0, :, pos].float(), what="V row written")
    if poison == "nan":   # NaN != NaN: check the rows are still all NaN
        assert torch.isnan(eng.k_caches[0][0, :, pos + 1:]).all() and torch.isnan(eng.v_caches[0][0, :, pos + 1:]).all()
    else:
        assert torch.equal(eng.k_caches[0][0, :, pos + 1:].cpu(), kc[0, :, pos + 1:])
        assert torch.equal(eng.v_caches[0][0, :, pos + 1:].cpu(), vc[0, :, pos + 1:])
    if step_mode == "persistent":
        assert eng.status() == 0
