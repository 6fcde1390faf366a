"""The drop-in at the model level: transformers' ``Qwen3VLTextModel`` (2 layers
at the real Qwen3-VL-2B layer shapes) with every decoder layer swapped by
``optimized_layer.replace_decoder_layers`` (reference optimized_layer.py:3848),
run on the GPU in fp16 on a ``StaticCache``, against the same model unswapped
in fp32 on the CPU.

The prompt is prefilled by the CPU model only (its K/V rows are copied into the
GPU model's StaticCache), so the GPU runs transformers' own decode glue
(embedding lookup, M-RoPE cos/sin, causal mask) around the swapped layers, which
take their HIP decode path.  Each greedy decode step's logits are compared.
"""

from __future__ import annotations

import copy

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu

VOCAB = 2048
# End to end through two layers the GPU model keeps fp16 activations between
# kernels (the drop-in path's I/O dtype, as in the reference) and transformers
# runs its final RMSNorm in fp16; each kernel alone meets 2e-3 in its own test.
MODEL_REL = 5e-3
# The rows a layer writes to the cache are its rotated keys, computed from the
# fp16 residual stream of the layers below (layer 1: 4.7e-3 in one run); a wrong
# row, position or rotation shows as an O(1) error.
KV_ROW_REL = 1e-2


def _hf_model(w, shape):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    cfg = Qwen3VLTextConfig(hidden_size=shape.hidden, intermediate_size=shape.intermediate,
                            num_attention_heads=shape.num_heads, num_key_value_heads=shape.num_kv_heads,
                            head_dim=shape.head_dim, num_hidden_layers=shape.num_layers, vocab_size=shape.vocab,
                            rms_norm_eps=shape.rms_eps,
                            rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta,
                                             "mrope_section": list(shape.mrope_section)})
    cfg._attn_implementation = "sdpa"
    m = Qwen3VLTextModel(cfg).float().eval()
    q, kv, i = shape.q_size, shape.kv_size, shape.intermediate
    with torch.no_grad():
        m.embed_tokens.weight.copy_(w.embed_tokens.float())
        m.norm.weight.copy_(w.final_norm_weight.float())
        for lw, L in zip(w.layers, m.layers):
            a = L.self_attn
            a.q_proj.weight.copy_(lw.qkv_weight[:q].float())
            a.k_proj.weight.copy_(lw.qkv_weight[q:q + kv].float())
            a.v_proj.weight.copy_(lw.qkv_weight[q + kv:].float())
            a.o_proj.weight.copy_(lw.o_proj_weight.float())
            a.q_norm.weight.copy_(lw.q_norm_weight.float())
            a.k_norm.weight.copy_(lw.k_norm_weight.float())
            L.mlp.gate_proj.weight.copy_(lw.gate_up_weight[:i].float())
            L.mlp.up_proj.weight.copy_(lw.gate_up_weight[i:].float())
            L.mlp.down_proj.weight.copy_(lw.down_proj_weight.float())
            L.input_layernorm.weight.copy_(lw.input_layernorm_weight.float())
            L.post_attention_layernorm.weight.copy_(lw.post_attn_layernorm_weight.float())
    return m


def test_replace_decoder_layers_decode_matches_transformers(cuda):
    from transformers.cache_utils import DynamicCache, StaticCache

    import optimized_layer
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.config import Qwen3VLTextShape

    shape = Qwen3VLTextShape(num_layers=2, vocab=VOCAB)
    w = syn.model_weights(23, shape=shape)
    ref = _hf_model(w, shape)
    gpu = copy.deepcopy(ref).half().to(cuda)
    assert optimized_layer.replace_decoder_layers(gpu) == 2
    assert all(isinstance(L, optimized_layer.OptimizedDecoderLayer) for L in gpu.layers)

    prompt = syn.multimodal_prompt(23, grid_h=4, grid_w=8, n_text=16, shape=shape)
    S, n_steps = prompt.length, 6
    emb = O.embed_prompt(w, prompt, torch.float32)
    cache_ref = DynamicCache(config=ref.config)
    with torch.no_grad():
        out = ref(inputs_embeds=emb[None], position_ids=prompt.position_ids[:, None, :], past_key_values=cache_ref,
                  use_cache=True)
    logits = out.last_hidden_state[0, -1] @ w.embed_tokens.float().T
    tok = int(torch.argmax(logits))

    # the GPU model's static cache holds the CPU prefill's K/V rows
    cache_gpu = StaticCache(config=gpu.config, max_cache_len=S + n_steps + 2)
    like = torch.empty(1, shape.num_kv_heads, 1, shape.head_dim, dtype=torch.float16, device=cuda)
    for li in range(shape.num_layers):
        layer = cache_gpu.layers[li]
        if not layer.is_initialized:
            layer.lazy_initialization(like, like)
        layer.keys[:, :, :S].copy_(cache_ref.layers[li].keys.half())
        layer.values[:, :, :S].copy_(cache_ref.layers[li].values.half())
        # transformers' own StaticLayer.update writes at this running length; the
        # swapped layers write at cache_position (as the reference's kernels do)
        layer.cumulative_length = torch.tensor(S)

    emb_gpu = w.embed_tokens.to(cuda)
    for step in range(n_steps):
        p = S + step
        rp = torch.full((3, 1, 1), p + prompt.rope_delta)
        with torch.no_grad():
            out_ref = ref(inputs_embeds=w.embed_tokens[tok].float().view(1, 1, -1), position_ids=rp,
                          past_key_values=cache_ref, use_cache=True)
            out_gpu = gpu(inputs_embeds=emb_gpu[tok].view(1, 1, -1), position_ids=rp.to(cuda),
                          past_key_values=cache_gpu, use_cache=True,
                          cache_position=torch.tensor([p], device=cuda))
        h_ref = out_ref.last_hidden_state[0, -1]
        h_gpu = out_gpu.last_hidden_state[0, -1].float().cpu()
        assert_close_rel(h_gpu, h_ref, rel=MODEL_REL, what=f"final hidden state, decode step {step}")
        l_ref = h_ref @ w.embed_tokens.float().T
        l_gpu = h_gpu @ w.embed_tokens.float().T
        assert_close_rel(l_gpu, l_ref, rel=MODEL_REL, what=f"logits, decode step {step}")
        margin = O.top2_margin(l_ref)
        print(f"step {step}: ref token {int(torch.argmax(l_ref))} gpu {int(torch.argmax(l_gpu))} "
              f"margin {margin:.4g}", flush=True)
        if margin > 1e-2:   # a closer top-2 may legitimately swap under fp16 activations
            assert int(torch.argmax(l_gpu)) == int(torch.argmax(l_ref))
        tok = int(torch.argmax(l_ref))
    # the new rows the swapped layers wrote match the reference cache's
    for li in range(shape.num_layers):
        assert_close_rel(cache_gpu.layers[li].keys[0, :, S:S + n_steps].float().cpu(),
                         cache_ref.layers[li].keys[0, :, S:S + n_steps], rel=KV_ROW_REL,
                         what=f"layer {li} new K rows")
