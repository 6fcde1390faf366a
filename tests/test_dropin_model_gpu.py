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
    # the new rows the swapped layers wrote match the reference cache's, and
    # each StaticLayer's running length follows the explicit cache positions
    for li in range(shape.num_layers):
        assert_close_rel(cache_gpu.layers[li].keys[0, :, S:S + n_steps].float().cpu(),
                         cache_ref.layers[li].keys[0, :, S:S + n_steps], rel=KV_ROW_REL,
                         what=f"layer {li} new K rows")
        assert int(cache_gpu.layers[li].cumulative_length) == S + n_steps


def test_dropin_decodes_at_the_static_layers_running_length(cuda):
    """The transformers 5.x calling convention without explicit positions: the
    swapped GPU model prefills its own StaticCache (transformers' layer math on
    the GPU, StaticLayer.update advances cumulative_length), then decodes passing
    neither position_ids nor cache_position.  transformers derives the rope
    positions from the cache's running length and the swapped layers must write
    K/V at that row and advance it on the device.  Checked against the unswapped
    model in fp32 on the CPU, decoding the same way: logits every step, the K/V
    rows written, and the running length after each step."""
    from transformers.cache_utils import DynamicCache, StaticCache

    import optimized_layer
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.config import Qwen3VLTextShape

    shape = Qwen3VLTextShape(num_layers=2, vocab=VOCAB)
    w = syn.model_weights(24, shape=shape)
    ref = _hf_model(w, shape)
    gpu = copy.deepcopy(ref).half().to(cuda)
    optimized_layer.replace_decoder_layers(gpu)
    prompt = syn.multimodal_prompt(24, grid_h=4, grid_w=8, n_text=16, shape=shape)
    S, n_steps = prompt.length, 5
    emb = O.embed_prompt(w, prompt, torch.float32)
    cache_ref = DynamicCache(config=ref.config)
    cache_gpu = StaticCache(config=gpu.config, max_cache_len=S + n_steps + 3)
    with torch.no_grad():
        out_ref = ref(inputs_embeds=emb[None], position_ids=prompt.position_ids[:, None, :],
                      past_key_values=cache_ref, use_cache=True)
        out_gpu = gpu(inputs_embeds=emb[None].half().to(cuda), position_ids=prompt.position_ids[:, None, :].to(cuda),
                      past_key_values=cache_gpu, use_cache=True)
    assert all(int(cache_gpu.layers[li].cumulative_length) == S for li in range(shape.num_layers))
    tok = int(torch.argmax(out_ref.last_hidden_state[0, -1] @ w.embed_tokens.float().T))
    emb_gpu = w.embed_tokens.to(cuda)
    for step in range(n_steps):
        with torch.no_grad():
            out_ref = ref(inputs_embeds=w.embed_tokens[tok].float().view(1, 1, -1), past_key_values=cache_ref,
                          use_cache=True)
            out_gpu = gpu(inputs_embeds=emb_gpu[tok].view(1, 1, -1), past_key_values=cache_gpu, use_cache=True)
        l_ref = out_ref.last_hidden_state[0, -1] @ w.embed_tokens.float().T
        l_gpu = out_gpu.last_hidden_state[0, -1].float().cpu() @ w.embed_tokens.float().T
        assert_close_rel(l_gpu, l_ref, rel=MODEL_REL, what=f"logits, decode step {step} (no explicit positions)")
        for li in range(shape.num_layers):
            assert int(cache_gpu.layers[li].cumulative_length) == S + step + 1
        tok = int(torch.argmax(l_ref))
    for li in range(shape.num_layers):
        assert_close_rel(cache_gpu.layers[li].keys[0, :, S:S + n_steps].float().cpu(),
                         cache_ref.layers[li].keys[0, :, S:S + n_steps], rel=KV_ROW_REL,
                         what=f"layer {li} new K rows (no explicit positions)")
        assert_close_rel(cache_gpu.layers[li].values[0, :, S:S + n_steps].float().cpu(),
                         cache_ref.layers[li].values[0, :, S:S + n_steps], rel=KV_ROW_REL,
                         what=f"layer {li} new V rows (no explicit positions)")
        # nothing written past the decoded rows
        assert cache_gpu.layers[li].keys[0, :, S + n_steps:].abs().max() == 0


class _GraphStep:
    """One decode step of a transformers text model captured in a HIP graph,
    with the reference's static input buffers (DecodeCudaGraphRunner,
    evaluation_wrapper.py:864-904 prebuild, :941-952 _run_step, :954-960
    _write_inputs): input ids [1,1], cache_position [1], position_ids [3,1,1]
    (cache position + rope delta on all three streams), the boolean attention
    mask over the static cache, and the next token written by an on-device
    argmax over the tied lm_head."""

    def __init__(self, model, cache, emb, max_len, device):
        self.model, self.cache, self.emb = model, cache, emb
        self.ids = torch.zeros(1, 1, dtype=torch.int64, device=device)
        self.cache_position = torch.zeros(1, dtype=torch.int64, device=device)
        self.position_ids = torch.zeros(3, 1, 1, dtype=torch.int64, device=device)
        self.mask = torch.zeros(1, max_len, dtype=torch.int64, device=device)
        self.next_token = torch.zeros(1, 1, dtype=torch.int64, device=device)
        self.logits = torch.zeros(1, emb.shape[0], dtype=torch.float16, device=device)
        self.graph = None

    def write_inputs(self, token: int, position: int, rope_delta: int) -> None:
        self.ids.fill_(token)
        self.cache_position.fill_(position)
        self.position_ids.fill_(position + rope_delta)
        self.mask[:, : position + 1] = 1

    def run(self) -> None:
        out = self.model(input_ids=self.ids, attention_mask=self.mask, position_ids=self.position_ids,
                         past_key_values=self.cache, use_cache=True, cache_position=self.cache_position)
        self.logits.copy_(out.last_hidden_state[:, -1] @ self.emb.T)
        self.next_token.copy_(torch.argmax(self.logits, dim=-1, keepdim=True))

    def capture(self) -> None:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            self.run()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.run()
        torch.cuda.synchronize()


def _prefilled_static_cache(ref, gpu, w, prompt, shape, max_len, cuda):
    """CPU fp32 prefill of the prompt; its K/V rows copied into a GPU StaticCache."""
    from transformers.cache_utils import DynamicCache, StaticCache

    emb = O.embed_prompt(w, prompt, torch.float32)
    cache_ref = DynamicCache(config=ref.config)
    with torch.no_grad():
        out = ref(inputs_embeds=emb[None], position_ids=prompt.position_ids[:, None, :], past_key_values=cache_ref,
                  use_cache=True)
    first = int(torch.argmax(out.last_hidden_state[0, -1] @ w.embed_tokens.float().T))
    cache = StaticCache(config=gpu.config, max_cache_len=max_len)
    like = torch.empty(1, shape.num_kv_heads, 1, shape.head_dim, dtype=torch.float16, device=cuda)
    S = prompt.length
    for li in range(shape.num_layers):
        layer = cache.layers[li]
        if not layer.is_initialized:
            layer.lazy_initialization(like, like)
        layer.keys[:, :, :S].copy_(cache_ref.layers[li].keys.half())
        layer.values[:, :, :S].copy_(cache_ref.layers[li].values.half())
    return cache, cache_ref, first


def test_dropin_model_step_captured_in_a_hip_graph(cuda):
    """The reference's graph runner over the swapped model: one decode step of
    transformers' Qwen3VLTextModel (2 layers at the real shapes) with every
    layer replaced, captured once in a HIP graph and replayed at successive
    positions with the static buffers rewritten between replays.  Every
    replay's logits and token equal an eager run of the same swapped model from
    the same state (same kernels: bit-identical), the logits are within the
    model-level bar of the unswapped model in fp32 on the CPU, and the cache
    rows written by the replays equal the eager run's."""
    import optimized_layer
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.config import Qwen3VLTextShape

    shape = Qwen3VLTextShape(num_layers=2, vocab=VOCAB)
    w = syn.model_weights(25, shape=shape)
    ref = _hf_model(w, shape)
    gpu = copy.deepcopy(ref).half().to(cuda)
    optimized_layer.replace_decoder_layers(gpu)
    prompt = syn.multimodal_prompt(25, grid_h=4, grid_w=8, n_text=16, shape=shape)
    S, n_steps = prompt.length, 4
    max_len = S + n_steps + 4
    emb_gpu = w.embed_tokens.to(cuda)

    # eager swapped model from the prefilled state
    cache_e, cache_ref, first = _prefilled_static_cache(ref, gpu, w, prompt, shape, max_len, cuda)
    eager = _GraphStep(gpu, cache_e, emb_gpu, max_len, cuda)
    tok, eager_logits, eager_tokens = first, [], []
    for step in range(n_steps):
        eager.write_inputs(tok, S + step, prompt.rope_delta)
        with torch.no_grad():
            eager.run()
        eager_logits.append(eager.logits.clone())
        tok = int(eager.next_token.item())
        eager_tokens.append(tok)

    # the same steps as replays of one captured step
    cache_g, _, first_g = _prefilled_static_cache(ref, gpu, w, prompt, shape, max_len, cuda)
    assert first_g == first
    g = _GraphStep(gpu, cache_g, emb_gpu, max_len, cuda)
    g.write_inputs(first, S, prompt.rope_delta)
    g.capture()
    tok, graph_tokens = first, []
    for step in range(n_steps):
        g.write_inputs(tok, S + step, prompt.rope_delta)
        g.graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g.logits, eager_logits[step]), f"replay {step} differs from the eager step"
        tok = int(g.next_token.item())
        graph_tokens.append(tok)
    assert graph_tokens == eager_tokens
    for li in range(shape.num_layers):
        assert torch.equal(cache_g.layers[li].keys[:, :, :S + n_steps], cache_e.layers[li].keys[:, :, :S + n_steps])
        assert torch.equal(cache_g.layers[li].values[:, :, :S + n_steps],
                           cache_e.layers[li].values[:, :, :S + n_steps])
        assert int(cache_g.layers[li].cumulative_length) == S + n_steps

    # and the unswapped fp32 model on the CPU, fed the same tokens
    tok = first
    for step in range(n_steps):
        p = S + step
        with torch.no_grad():
            out_ref = ref(inputs_embeds=w.embed_tokens[tok].float().view(1, 1, -1),
                          position_ids=torch.full((3, 1, 1), p + prompt.rope_delta), past_key_values=cache_ref,
                          use_cache=True)
        l_ref = out_ref.last_hidden_state[0, -1] @ w.embed_tokens.float().T
        assert_close_rel(eager_logits[step][0].float().cpu(), l_ref, rel=MODEL_REL,
                         what=f"graph-replayed drop-in logits, step {step}")
        tok = eager_tokens[step]
