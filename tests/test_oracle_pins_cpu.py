"""Pins for the CPU oracle (no GPU).  Each oracle function is checked against
something independent of its own formula: a PyTorch library routine,
transformers' Qwen3-VL modules (the third-party library the reference runs on,
transformers 5.15.0 in this image), a closed form, an invariant, or brute
force on a tiny input — chosen so that a dropped term, a wrong sign, a wrong
index or a transposed operand fails."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import qwen3vl_oracle as O

D64 = torch.float64


# ----------------------------------------------------------------- RMSNorm

def test_rms_norm_matches_torch_functional():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 2048, generator=g, dtype=D64)
    w = 1 + 0.02 * torch.randn(2048, generator=g, dtype=D64)
    ref = F.rms_norm(x, (2048,), w, eps=1e-6)
    assert torch.allclose(O.rms_norm(x, w, 1e-6, D64), ref, rtol=1e-12, atol=1e-12)


def test_rms_norm_invariants():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2048, generator=g, dtype=D64)
    w = 1 + 0.02 * torch.randn(2048, generator=g, dtype=D64)
    # scale invariance (up to eps) and a constant input maps to +-w
    assert torch.allclose(O.rms_norm(37.0 * x, w, 0.0, D64), O.rms_norm(x, w, 0.0, D64), rtol=1e-12)
    c = torch.full((2048,), -3.0, dtype=D64)
    assert torch.allclose(O.rms_norm(c, w, 0.0, D64), -w, rtol=1e-12)
    # unit RMS output before the weight
    y = O.rms_norm(x, torch.ones(2048, dtype=D64), 0.0, D64)
    assert abs(float(y.pow(2).mean()) - 1.0) < 1e-12


# ----------------------------------------------------------------- RoPE / M-RoPE

def test_mrope_slot_map_has_24_20_20_sections():
    m = O.mrope_stream_of_slot()
    assert len(m) == 64 and m.count(0) == 24 and m.count(1) == 20 and m.count(2) == 20
    assert m[:6] == [0, 1, 2, 0, 1, 2] and m[60:] == [0, 0, 0, 0]


def test_mrope_cos_sin_match_transformers_rotary():
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextRotaryEmbedding

    cfg = Qwen3VLTextConfig(head_dim=128, hidden_size=2048, num_attention_heads=16,
                            rope_parameters={"rope_type": "default", "rope_theta": 5_000_000.0,
                                             "mrope_section": [24, 20, 20]})
    rot = Qwen3VLTextRotaryEmbedding(cfg)
    g = torch.Generator().manual_seed(2)
    pos = torch.randint(0, 5000, (3, 1, 40), generator=g)      # distinct T/H/W streams
    cos_hf, sin_hf = rot(torch.zeros(1, 40, 2048), pos)
    cos, sin = O.mrope_cos_sin(pos[:, 0, :])
    assert torch.allclose(cos, cos_hf[0], atol=2e-6) and torch.allclose(sin, sin_hf[0], atol=2e-6)


def test_rope_identity_at_position_zero_and_pair_norms():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, 128, generator=g, dtype=D64)
    cos, sin = O.mrope_cos_sin(torch.zeros(3, 1, dtype=torch.int64), dtype=D64)
    assert torch.equal(O.apply_rope(x, cos[0], sin[0]), x)
    cos, sin = O.mrope_cos_sin(torch.tensor([[777], [12], [300]]), dtype=D64, exact=True)
    y = O.apply_rope(x, cos[0], sin[0])
    pn = lambda t: t[:, :64] ** 2 + t[:, 64:] ** 2   # noqa: E731
    assert torch.allclose(pn(y), pn(x), rtol=1e-12)


def test_rope_equals_complex_rotation_when_streams_agree():
    """At decode T = H = W, so interleaved M-RoPE is textbook 1-D RoPE: the pair
    (x_j, x_{j+64}) is the complex number x_j + i x_{j+64} times e^{i p f_j}."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(8, 128, generator=g, dtype=D64)
    p = 1234
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), p), dtype=D64, exact=True)
    y = O.apply_rope(x, cos[0], sin[0])
    f = 1.0 / (5e6 ** (torch.arange(0, 128, 2, dtype=D64) / 128))
    z = torch.complex(x[:, :64], x[:, 64:]) * torch.polar(torch.ones(64, dtype=D64), p * f)
    assert torch.allclose(y[:, :64], z.real, atol=1e-9) and torch.allclose(y[:, 64:], z.imag, atol=1e-9)


# ----------------------------------------------------------------- attention

def _attn_inputs(seed, L, T):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(16, 128, generator=g, dtype=D64)
    k = torch.randn(1, 8, T, 128, generator=g, dtype=D64)
    v = torch.randn(1, 8, T, 128, generator=g, dtype=D64)
    return q, k, v


def test_attention_matches_sdpa_with_gqa():
    q, k, v = _attn_inputs(5, 300, 300)
    ref = F.scaled_dot_product_attention(q.view(1, 16, 1, 128), k, v, scale=128 ** -0.5, enable_gqa=True)
    assert torch.allclose(O.decode_attention(q, k, v, 299, 128 ** -0.5, dtype=D64), ref.view(16, 128), atol=1e-12)


def test_attention_brute_force_tiny():
    q, k, v = _attn_inputs(6, 5, 7)
    out = O.decode_attention(q, k, v, 4, 0.3, dtype=D64)
    for h in range(16):
        kv = h // 2
        s = [0.3 * float(q[h] @ k[0, kv, t]) for t in range(5)]
        mx = max(s)
        w = [math.exp(si - mx) for si in s]
        ref = sum(wi * v[0, kv, t] for t, wi in enumerate(w)) / sum(w)
        assert torch.allclose(out[h], ref, atol=1e-12)


def test_attention_valid_prefix_and_special_cases():
    q, k, v = _attn_inputs(7, 64, 100)
    base = O.decode_attention(q, k, v, 63, 0.1, dtype=D64)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 64:] = 1e4
    v2[:, :, 64:] = -1e4
    assert torch.equal(O.decode_attention(q, k2, v2, 63, 0.1, dtype=D64), base)   # stale tail ignored
    one = O.decode_attention(q, k, v, 0, 0.1, dtype=D64)                           # L = 1 -> V[0]
    assert torch.allclose(one, v[0, :, 0].repeat_interleave(2, 0), atol=1e-14)
    keq = k[:, :, :1].expand(-1, -1, 100, -1)
    mean = O.decode_attention(q, keq, v, 63, 0.1, dtype=D64)                        # equal keys -> mean of V
    assert torch.allclose(mean, v[0, :, :64].mean(1).repeat_interleave(2, 0), atol=1e-12)
    # position past the capacity attends the whole cache
    assert torch.equal(O.decode_attention(q, k, v, 10_000, 0.1, dtype=D64),
                       O.decode_attention(q, k, v, 99, 0.1, dtype=D64))


def test_split_lse_merge_reproduces_full_attention():
    """The split-KV merge used by the kernels: out = sum_s e^{lse_s} o_s / sum_s e^{lse_s}."""
    q, k, v = _attn_inputs(8, 1000, 1000)
    full = O.decode_attention(q, k, v, 999, 0.09, dtype=D64)
    outs, lses = [], []
    for a, b in ((0, 137), (137, 600), (600, 1000)):
        ks, vs = k[:, :, a:b], v[:, :, a:b]
        outs.append(O.decode_attention(q, ks, vs, b - a - 1, 0.09, dtype=D64))
        lses.append(O.decode_attention_lse(q, ks, vs, b - a - 1, 0.09))
    lse = torch.stack(lses)                    # [S, Hq]
    w = torch.softmax(lse, 0)
    merged = sum(w[s][:, None] * outs[s] for s in range(3))
    assert torch.allclose(merged, full, atol=1e-12)
    assert torch.allclose(torch.logsumexp(lse, 0), O.decode_attention_lse(q, k, v, 999, 0.09), atol=1e-12)


def test_q_rope_kv_update_writes_only_its_row():
    g = torch.Generator().manual_seed(9)
    q, k, v = torch.randn(16, 128, generator=g), torch.randn(8, 128, generator=g), torch.randn(8, 128, generator=g)
    kc = torch.randn(1, 8, 20, 128, generator=g).half()
    vc = torch.randn(1, 8, 20, 128, generator=g).half()
    kc0, vc0 = kc.clone(), vc.clone()
    cos, sin = O.mrope_cos_sin(torch.full((3, 1), 5))
    O.q_rope_kv_update(q, k, v, torch.ones(128), torch.ones(128), 1e-6, cos[0], sin[0], kc, vc, 5)
    others = [i for i in range(20) if i != 5]
    assert torch.equal(kc[:, :, others], kc0[:, :, others]) and torch.equal(vc[:, :, others], vc0[:, :, others])
    assert torch.equal(vc[0, :, 5], v.half())
    O.q_rope_kv_update(q, k, v, torch.ones(128), torch.ones(128), 1e-6, cos[0], sin[0], kc0, vc0, 20)  # out of range
    assert torch.equal(kc0[:, :, 5], kc[:, :, 5] * 0 + kc0[:, :, 5])


# ----------------------------------------------------------------- GEMV / MLP / argmax

def test_gemv_one_hot_and_fp64():
    g = torch.Generator().manual_seed(10)
    w = torch.randn(300, 512, generator=g).half()
    x = torch.zeros(512)
    x[77] = 1.0
    assert torch.equal(O.gemv(x, w), w[:, 77].float())
    xr = torch.randn(512, generator=g)
    assert torch.allclose(O.gemv(xr, w, dtype=D64), w.double() @ xr.double(), rtol=1e-12)


def test_post_attn_mlp_matches_transformers_modules():
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextMLP, Qwen3VLTextRMSNorm

    cfg = Qwen3VLTextConfig(hidden_size=256, intermediate_size=512, hidden_act="silu")
    mlp = Qwen3VLTextMLP(cfg).double()
    norm = Qwen3VLTextRMSNorm(256, eps=1e-6).double()
    g = torch.Generator().manual_seed(11)
    with torch.no_grad():
        # every parameter set explicitly: module construction may leave them
        # uninitialised when an earlier test disabled transformers' weight init
        for lin in (mlp.gate_proj, mlp.up_proj, mlp.down_proj):
            lin.weight.copy_(0.05 * torch.randn(lin.weight.shape, generator=g, dtype=D64))
        norm.weight.copy_(1 + 0.02 * torch.randn(256, generator=g))
    res, att = torch.randn(256, generator=g, dtype=D64), torch.randn(256, generator=g, dtype=D64)
    gu = torch.cat([mlp.gate_proj.weight, mlp.up_proj.weight], 0).detach()
    hid, out, r = O.post_attn_mlp(res, att, norm.weight.detach(), gu, mlp.down_proj.weight.detach(), None, 1e-6, D64)
    with torch.no_grad():
        # transformers' MLP module on an fp64 RMSNorm: exact to fp64 rounding
        ref = (res + att) + mlp(F.rms_norm(res + att, (256,), norm.weight, eps=1e-6))
        # transformers' own RMSNorm module normalises in fp32 (relative error ~6e-8)
        ref_hf = (res + att) + mlp(norm(res + att))
    assert torch.allclose(out, ref, rtol=1e-12, atol=1e-12) and torch.equal(r, res + att)
    assert torch.allclose(out, ref_hf, rtol=0, atol=1e-6 * float(ref_hf.abs().max()))
    assert float((out - (res + att)).abs().max()) > 0.1   # the MLP term is present, not zero


def test_lm_head_argmax_takes_first_maximum():
    w = torch.zeros(10, 4)
    w[3, 0] = w[7, 0] = 2.0
    logits, tok = O.lm_head_argmax(torch.tensor([1.0, 0, 0, 0]), torch.ones(4), w, 1e-6)
    assert tok == 3 and logits[3] == logits[7]


# ----------------------------------------------------------------- whole model vs transformers

def _tiny():
    from qwen3vl_hip.config import Qwen3VLTextShape

    shape = Qwen3VLTextShape(hidden=128, num_heads=4, num_kv_heads=2, head_dim=32, intermediate=256, num_layers=2,
                             vocab=97, mrope_section=(6, 5, 5))
    oshape = O.OracleShape(hidden=128, num_heads=4, num_kv_heads=2, head_dim=32, intermediate=256, num_layers=2,
                           vocab=97, mrope_section=(6, 5, 5))
    return shape, oshape


def _hf_tiny_model(w, shape):
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel

    cfg = Qwen3VLTextConfig(hidden_size=shape.hidden, intermediate_size=shape.intermediate,
                            num_attention_heads=shape.num_heads, num_key_value_heads=shape.num_kv_heads,
                            head_dim=shape.head_dim, num_hidden_layers=shape.num_layers, vocab_size=shape.vocab,
                            rms_norm_eps=shape.rms_eps,
                            rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta,
                                             "mrope_section": list(shape.mrope_section)})
    # sdpa keeps the softmax in the model dtype (the eager path rounds it through fp32)
    cfg._attn_implementation = "sdpa"
    m = Qwen3VLTextModel(cfg).float().eval()
    q, kv = shape.q_size, shape.kv_size
    with torch.no_grad():
        m.embed_tokens.weight.copy_(w.embed_tokens.double())
        m.norm.weight.copy_(w.final_norm_weight.double())
        for lw, L in zip(w.layers, m.layers):
            a = L.self_attn
            a.q_proj.weight.copy_(lw.qkv_weight[:q].double())
            a.k_proj.weight.copy_(lw.qkv_weight[q:q + kv].double())
            a.v_proj.weight.copy_(lw.qkv_weight[q + kv:].double())
            a.o_proj.weight.copy_(lw.o_proj_weight.double())
            a.q_norm.weight.copy_(lw.q_norm_weight.double())
            a.k_norm.weight.copy_(lw.k_norm_weight.double())
            L.mlp.gate_proj.weight.copy_(lw.gate_up_weight[:shape.intermediate].double())
            L.mlp.up_proj.weight.copy_(lw.gate_up_weight[shape.intermediate:].double())
            L.mlp.down_proj.weight.copy_(lw.down_proj_weight.double())
            L.input_layernorm.weight.copy_(lw.input_layernorm_weight.double())
            L.post_attention_layernorm.weight.copy_(lw.post_attn_layernorm_weight.double())
    return m


def test_oracle_prefill_and_decode_match_transformers_text_model():
    """Tiny Qwen3-VL text model (2 layers, 4/2 heads, d 32, M-RoPE sections 6/5/5)
    with a multimodal-shaped prompt: the oracle's prefill logits and each cached
    decode step's logits equal transformers' Qwen3VLTextModel.  Both run in fp32
    (transformers' RMSNorm and rotary always round through fp32, so an fp64 run
    would differ at 1e-7 by construction); the bar is set by fp32 summation order."""
    from transformers.cache_utils import DynamicCache

    from qwen3vl_hip import synthetic as syn

    shape, oshape = _tiny()
    w = syn.model_weights(13, shape)
    prompt = syn.multimodal_prompt(13, grid_h=3, grid_w=4, n_text=5, shape=shape)
    hf = _hf_tiny_model(w, shape)
    S = prompt.length
    F32 = torch.float32
    emb = O.embed_prompt(w, prompt, F32)
    with torch.no_grad():
        cache = DynamicCache(config=hf.config)
        out = hf(inputs_embeds=emb[None], position_ids=prompt.position_ids[:, None, :], past_key_values=cache,
                 use_cache=True)
        logits_hf = out.last_hidden_state[0, -1] @ w.embed_tokens.float().T
    caches = [(torch.zeros(1, 2, S + 8, 32, dtype=F32), torch.zeros(1, 2, S + 8, 32, dtype=F32)) for _ in range(2)]
    h_last = O.prefill(w, emb, prompt.position_ids, caches, oshape, F32)
    logits, tok = O.lm_head_argmax(h_last, w.final_norm_weight, w.embed_tokens, shape.rms_eps, F32)
    assert (logits - logits_hf).abs().max() < 2e-5 * logits_hf.abs().max()
    assert tok == int(torch.argmax(logits_hf))
    # cached decode steps at position p with rope position p + delta on all streams
    for step in range(4):
        p = S + step
        rp = p + prompt.rope_delta
        with torch.no_grad():
            out = hf(inputs_embeds=w.embed_tokens[tok].float().view(1, 1, -1),
                     position_ids=torch.full((3, 1, 1), rp), past_key_values=cache, use_cache=True)
            lhf = out.last_hidden_state[0, -1] @ w.embed_tokens.float().T
        cos, sin = O.mrope_cos_sin(torch.full((3, 1), rp), oshape, F32)
        h = w.embed_tokens[tok].float()
        for li, lw in enumerate(w.layers):
            h = O.decode_layer(lw.tensors(), h, caches[li][0], caches[li][1], p, cos[0], sin[0], oshape, F32)
        logits, tok = O.lm_head_argmax(h, w.final_norm_weight, w.embed_tokens, shape.rms_eps, F32)
        assert (logits - lhf).abs().max() < 2e-5 * lhf.abs().max(), f"decode step {step}"
        assert tok == int(torch.argmax(lhf))


def _hf_tiny_vl_model(w, shape):
    """transformers' full Qwen3-VL model (tiny vision tower, spatial merge 2) with
    the text decoder and the tied lm_head set to ``w``: its get_rope_index and
    compute_3d_position_ids are the reference's position rules (the reference
    decodes through this model, evaluation_wrapper.py:206-209, :941-950)."""
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLForConditionalGeneration

    text = dict(hidden_size=shape.hidden, intermediate_size=shape.intermediate, num_attention_heads=shape.num_heads,
                num_key_value_heads=shape.num_kv_heads, head_dim=shape.head_dim, num_hidden_layers=shape.num_layers,
                vocab_size=shape.vocab, rms_norm_eps=shape.rms_eps,
                rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta,
                                 "mrope_section": list(shape.mrope_section)})
    vision = dict(depth=1, hidden_size=32, intermediate_size=64, num_heads=2, out_hidden_size=shape.hidden,
                  spatial_merge_size=2, patch_size=16, temporal_patch_size=2, deepstack_visual_indexes=[])
    cfg = Qwen3VLConfig(text_config=text, vision_config=vision, image_token_id=shape.vocab - 7,
                        video_token_id=shape.vocab - 6, vision_start_token_id=shape.vocab - 5,
                        tie_word_embeddings=True)
    cfg.text_config._attn_implementation = "sdpa"
    m = Qwen3VLForConditionalGeneration(cfg).float().eval()
    lm = _hf_tiny_model(w, shape)
    m.model.language_model.load_state_dict(lm.state_dict())
    with torch.no_grad():
        m.lm_head.weight.copy_(w.embed_tokens.double())
    return m


@pytest.mark.parametrize("grid", [(1, 3, 4, 5), (1, 24, 32, 256), (3, 2, 2, 5), (5, 2, 3, 4), (2, 4, 3, 1)])
def test_multimodal_prompt_positions_match_transformers_get_rope_index(grid):
    """The synthetic prompt's [3, S] M-RoPE positions and rope_delta equal
    transformers' Qwen3VLModel.get_rope_index (HF:932-1023) for the same token
    layout: one image (LLM grid t x h x w after the 2x2 spatial merge, so
    image_grid_thw = [t, 2h, 2w]) followed by text, with image placeholder ids
    and mm_token_type_ids as the processor emits them.  Covers the config-3
    grid 1x24x32, the tiny grid, and temporal grids t > 1 (one where t exceeds
    h and w, so a rule that advances text past max(t, h, w) would differ)."""
    from qwen3vl_hip import synthetic as syn

    t, h, w_, n_text = grid
    shape, _ = _tiny()
    weights = syn.model_weights(16, shape, num_layers=1)
    model = _hf_tiny_vl_model(weights, dataclasses_replace(shape, num_layers=1))
    prompt = syn.multimodal_prompt(16, grid_t=t, grid_h=h, grid_w=w_, n_text=n_text, shape=shape)
    n_vis = t * h * w_
    ids = torch.cat([torch.full((n_vis,), model.config.image_token_id), prompt.text_ids]).view(1, -1)
    types = torch.cat([torch.ones(n_vis, dtype=torch.int32), torch.zeros(n_text, dtype=torch.int32)]).view(1, -1)
    pos, delta = model.model.get_rope_index(ids, types, image_grid_thw=torch.tensor([[t, 2 * h, 2 * w_]]))
    assert torch.equal(prompt.position_ids, pos[:, 0, :])
    assert prompt.rope_delta == int(delta)


def dataclasses_replace(obj, **kw):
    import dataclasses

    return dataclasses.replace(obj, **kw)


def test_greedy_generate_matches_transformers_generation_loop():
    """The oracle's greedy loop against transformers' own: prefill the
    multimodal-shaped prompt through Qwen3VLForConditionalGeneration with the
    positions of its get_rope_index (vision rows as inputs_embeds, text rows
    through its embedding table), then decode token by token passing only
    input_ids and the cache, so transformers derives every decode position
    itself from the cached length and its stored rope_deltas
    (compute_3d_position_ids, HF:1098-1145).  Tokens must be identical and
    logits equal at fp32 summation-order level for every step; a wrong rope
    delta, a position off by one or a stale cache row changes the logits far
    beyond that bar.  transformers' cache here is fp32, so the oracle runs with
    an fp32 cache for the tight comparison; with its default fp16 cache (the
    reference's StaticCache dtype) the tokens must still agree.  A rope delta
    planted one position off in the oracle must miss the bar by far."""
    from transformers.cache_utils import DynamicCache

    from qwen3vl_hip import synthetic as syn

    shape, oshape = _tiny()
    w = syn.model_weights(17, shape)
    prompt = syn.multimodal_prompt(17, grid_h=3, grid_w=4, n_text=5, shape=shape)
    assert prompt.rope_delta != 0
    n = 10
    logits_o, logits_16, logits_bad = [], [], []
    toks, _, _ = O.greedy_generate(w, prompt, n, prompt.length + n, oshape, logits_out=logits_o,
                                   cache_dtype=torch.float32)
    toks16, _, _ = O.greedy_generate(w, prompt, n, prompt.length + n, oshape, logits_out=logits_16)
    O.greedy_generate(w, prompt, 3, prompt.length + n, oshape, logits_out=logits_bad, cache_dtype=torch.float32,
                      rope_delta=prompt.rope_delta + 1)

    model = _hf_tiny_vl_model(w, shape)
    n_vis = prompt.vision_embeds.shape[0]
    ids = torch.cat([torch.full((n_vis,), model.config.image_token_id), prompt.text_ids]).view(1, -1)
    types = torch.cat([torch.ones(n_vis, dtype=torch.int32), torch.zeros(prompt.text_ids.numel(), dtype=torch.int32)])
    emb = O.embed_prompt(w, prompt, torch.float32)[None]
    with torch.no_grad():
        pos, delta = model.model.get_rope_index(ids, types.view(1, -1), image_grid_thw=torch.tensor([[1, 6, 8]]))
        model.model.rope_deltas = delta
        cache = DynamicCache(config=model.config.text_config)
        out = model(inputs_embeds=emb, position_ids=pos, past_key_values=cache, use_cache=True)
        logits_hf = [out.logits[0, -1]]
        tok = int(torch.argmax(logits_hf[-1]))
        toks_hf = [tok]
        for _ in range(n - 1):
            out = model(input_ids=torch.tensor([[tok]]), past_key_values=cache, use_cache=True)
            logits_hf.append(out.logits[0, -1])
            tok = int(torch.argmax(logits_hf[-1]))
            toks_hf.append(tok)
    assert toks == toks_hf and toks16 == toks_hf
    for i, (a, b) in enumerate(zip(logits_o, logits_hf)):
        assert (a - b).abs().max() < 2e-5 * b.abs().max(), f"step {i}"
    for i, (a, b) in enumerate(zip(logits_16, logits_hf)):
        assert (a - b).abs().max() < 2e-3 * b.abs().max(), f"fp16 cache, step {i}"
    # the planted off-by-one delta: identical prefill, decode steps far off
    assert (logits_bad[0] - logits_hf[0]).abs().max() < 2e-5 * logits_hf[0].abs().max()
    for a, b in zip(logits_bad[1:], logits_hf[1:3]):
        assert (a - b).abs().max() > 100 * 2e-5 * b.abs().max()


def test_greedy_generate_matches_step_by_step_decoding():
    from qwen3vl_hip import synthetic as syn

    shape, oshape = _tiny()
    w = syn.model_weights(14, shape)
    prompt = syn.multimodal_prompt(14, grid_h=3, grid_w=4, n_text=5, shape=shape)
    toks, margins, caches = O.greedy_generate(w, prompt, 6, prompt.length + 8, oshape)
    assert len(toks) == 6 and all(0 <= t < 97 for t in toks) and all(m >= 0 for m in margins)
    # continuing from the returned state reproduces the tail
    toks2, _, _ = O.greedy_generate(w, prompt, 6, prompt.length + 8, oshape)
    assert toks2 == toks


def test_oracle_batch_step_matches_transformers_per_sequence():
    """Batch decode step (config 4 semantics): three sequences with different
    cache lengths and rope positions share one call; each sequence's logits equal
    transformers' Qwen3VLTextModel decoding that sequence alone after its own
    prefill, so a mixed-up sequence index, position or cache row fails."""
    from transformers.cache_utils import DynamicCache

    from qwen3vl_hip import synthetic as syn

    shape, oshape = _tiny()
    w = syn.model_weights(15, shape)
    hf = _hf_tiny_model(w, shape)
    F32 = torch.float32
    lengths, T = [5, 9, 2], 12
    g = torch.Generator().manual_seed(15)
    caches = [(torch.zeros(3, 2, T, 32, dtype=F32), torch.zeros(3, 2, T, 32, dtype=F32)) for _ in range(2)]
    tokens, rope, ref = [], [], []
    for b, L in enumerate(lengths):
        ids = torch.randint(0, shape.vocab, (L,), generator=g)
        pos = torch.arange(L).view(1, L).expand(3, L)
        tok = int(torch.randint(0, shape.vocab, (1,), generator=g))
        rp = L + 3 * b                                   # rope position differs from the cache position
        with torch.no_grad():
            cache = DynamicCache(config=hf.config)
            hf(inputs_embeds=w.embed_tokens[ids].float()[None], position_ids=pos[:, None, :], past_key_values=cache,
               use_cache=True)
            out = hf(inputs_embeds=w.embed_tokens[tok].float().view(1, 1, -1), position_ids=torch.full((3, 1, 1), rp),
                     past_key_values=cache, use_cache=True)
            ref.append(out.last_hidden_state[0, -1] @ w.embed_tokens.float().T)
        O.prefill(w, w.embed_tokens[ids].float(), pos, [(k[b:b + 1], v[b:b + 1]) for k, v in caches], oshape, F32)
        tokens.append(tok)
        rope.append(rp)
    logits, toks = O.decode_step_batch(w, tokens, caches, lengths, rope, oshape, F32)
    for b in range(3):
        assert (logits[b] - ref[b]).abs().max() < 2e-5 * ref[b].abs().max(), f"sequence {b}"
        assert toks[b] == int(torch.argmax(ref[b]))


@pytest.mark.parametrize("L", [0, 4096])
def test_step_roofline_bytes(L):
    assert O.roofline_bytes_step(L) == 3_441_154_048 + 114_688 * L
