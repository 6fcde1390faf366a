"""CPU oracle for the Qwen3-VL-2B batch-1 decode step (TEST INFRASTRUCTURE ONLY).

This module restates, in plain PyTorch on the CPU, the arithmetic of the
reference decode path.  It is the checker for the HIP kernels: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it, and only to compute expected values or the CPU baseline.  The product path
(the `aicasgc-2026_amd` package and its C-ABI library) never calls it.

Math is fp32 by default (``dtype=torch.float64`` is accepted everywhere for
closed-form checks).  Weights are the fp16 tensors upcast exactly.  The static
KV cache keeps the dtype of the tensor handed in (fp16 for every benchmark
configuration), so the cache write rounds exactly as the reference's cache does.

What each function follows (reference = /root/reference, HF = transformers
5.15.0 models/qwen3_vl/modeling_qwen3_vl.py, the third-party library the
reference runs on):

* ``rms_norm``            HF:391-408 (Qwen3VLTextRMSNorm); fused variants
                          decode_gemv_kernel_fused.cuh:99-185 (rmsnorm+qkv).
* ``rope_inv_freq``       HF:326-343 (compute_default_rope_parameters).
* ``mrope_cos_sin``       HF:345-389 (rotary forward + apply_interleaved_mrope).
* ``apply_rope``          HF:138-143 (rotate_half), HF:412-435.
* ``gemv``                F.linear as called at optimized_layer.py:180-182, :362, :461;
                          evaluation_wrapper.py:1238 (lm_head).
* ``q_rope_kv_update``    decode_small_ops_kernel.cu:115-182 and its wrapper
                          cuda_decode_small_ops.py:136-225 (q/k per-head RMSNorm,
                          rotate-half RoPE, K/V written at cache_position).
* ``decode_attention``    decode_attention_v4_kernel.cu:646-910 (valid length
                          min(pos+1, T) at :679) and HF eager attention HF:171-193
                          (fp32 softmax, GQA repeat_kv).
* ``post_attn_mlp``       decode_gemv_kernel_fused.cuh:856-1076 via
                          cuda_decode_gemv_ops/fused.py:261-337: r = residual + attn,
                          x = rmsnorm(r), hidden = silu(gate) * up, out = down(hidden) + r.
* ``decode_layer``        optimized_layer.py:108-469 (decode op order) == HF:526-568.
* ``lm_head_argmax``      evaluation_wrapper.py:1227-1238 and :952 (first maximal index).
* ``prefill`` / ``greedy_generate``  HF:769-852 (text model loop, final norm),
                          evaluation_wrapper.py:149-315, :507-539 (decode position =
                          cache_position + rope_delta on all three M-RoPE streams).

Parity pins for every function live in tests/test_oracle_*.py (library routines
such as F.rms_norm / F.scaled_dot_product_attention / torch.polar, transformers'
own Qwen3-VL modules, closed forms and invariants, brute force on tiny inputs).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

# ----------------------------------------------------------------- shapes


@dataclass(frozen=True)
class OracleShape:
    hidden: int = 2048
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    num_layers: int = 28
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 5_000_000.0
    mrope_section: tuple = (24, 20, 20)

    @property
    def q_size(self):
        return self.num_heads * self.head_dim

    @property
    def kv_size(self):
        return self.num_kv_heads * self.head_dim


SHAPE = OracleShape()


def _f(t: torch.Tensor, dtype) -> torch.Tensor:
    return t.to(dtype)


# ----------------------------------------------------------------- norms


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, dtype=torch.float32) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * weight over the last dim (HF:400-405)."""
    xf = _f(x, dtype)
    var = xf.pow(2).mean(-1, keepdim=True)
    return xf * torch.rsqrt(var + eps) * _f(weight, dtype)


# ----------------------------------------------------------------- RoPE


def rope_inv_freq(shape: OracleShape = SHAPE, dtype=torch.float32) -> torch.Tensor:
    """inv_freq[j] = theta^(-2j/d), j < d/2 (HF:340-342), evaluated in ``dtype``
    (fp32 reproduces HF's own fp32 expression bit for bit)."""
    d = shape.head_dim
    return 1.0 / (shape.rope_theta ** (torch.arange(0, d, 2, dtype=dtype) / d))


def mrope_stream_of_slot(shape: OracleShape = SHAPE) -> list:
    """Which position stream (0=T, 1=H, 2=W) drives frequency slot j (HF:372-389).

    Slots j with j % 3 == 1 and j < 3*sec[1] take H, j % 3 == 2 and j < 3*sec[2]
    take W, all others keep T.
    """
    half = shape.head_dim // 2
    out = [0] * half
    for dim, offset in ((1, 1), (2, 2)):
        for j in range(offset, shape.mrope_section[dim] * 3, 3):
            out[j] = dim
    return out


def mrope_cos_sin(position_ids: torch.Tensor, shape: OracleShape = SHAPE, dtype=torch.float32,
                  exact: bool = False):
    """cos/sin [S, d] for position ids [3, S] (T, H, W streams), HF:352-370.

    freqs[s, j] = pos[stream(j), s] * inv_freq[j]; emb = cat(freqs, freqs).
    HF evaluates the angles and cos/sin in fp32 whatever the model dtype
    (HF:363-368) and casts the result; that is the default here.  ``exact``
    evaluates them in ``dtype`` instead (closed-form checks in fp64).
    """
    work = dtype if exact else torch.float32
    pos = position_ids.to(work)
    inv = rope_inv_freq(shape, work)
    streams = torch.tensor(mrope_stream_of_slot(shape))
    p = pos[streams, :].T                      # [S, d/2]: position of the stream owning slot j
    freqs = p * inv[None, :]
    emb = torch.cat([freqs, freqs], -1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], -1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin (HF:432-434); cos/sin broadcast over heads."""
    return x * cos + rotate_half(x) * sin


# ----------------------------------------------------------------- linear


def gemv(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, dtype=torch.float32):
    """y = W x (+ b) for x [..., K], W [N, K]."""
    y = _f(x, dtype) @ _f(weight, dtype).T
    if bias is not None:
        y = y + _f(bias, dtype)
    return y


# ----------------------------------------------------------------- attention sub-ops


def q_rope_kv_update(q, k, v, q_weight, k_weight, eps, cos, sin, k_cache, v_cache, cache_position,
                     dtype=torch.float32):
    """Decode-step q/k per-head RMSNorm + RoPE; K_rot and V written into the cache.

    q [Hq, D], k/v [Hkv, D]; cos/sin [D]; caches [1, Hkv, T, D] are written in
    place at row ``cache_position`` (rounded to the cache dtype).  Returns the
    rotated q [Hq, D] in ``dtype``.  A position outside [0, T) writes nothing.
    """
    qn = rms_norm(q, q_weight, eps, dtype)
    kn = rms_norm(k, k_weight, eps, dtype)
    c, s = _f(cos, dtype), _f(sin, dtype)
    q_rot = apply_rope(qn, c, s)
    k_rot = apply_rope(kn, c, s)
    pos = int(cache_position)
    if 0 <= pos < k_cache.shape[2]:
        k_cache[0, :, pos, :] = k_rot.to(k_cache.dtype)
        v_cache[0, :, pos, :] = _f(v, dtype).to(v_cache.dtype)
    return q_rot


def decode_attention(q, k_cache, v_cache, cache_position, scaling, groups=None, dtype=torch.float32):
    """Single-token GQA attention over the valid cache prefix.

    q [Hq, D]; caches [1, Hkv, T, D].  L = min(cache_position + 1, T);
    q head h reads kv head h // (Hq / Hkv).  Softmax in ``dtype``.
    Returns [Hq, D].
    """
    hq = q.shape[0]
    hkv, t = k_cache.shape[1], k_cache.shape[2]
    g = hq // hkv if groups is None else groups
    L = min(int(cache_position) + 1, t)
    kk = _f(k_cache[0, :, :L, :], dtype).repeat_interleave(g, 0)    # [Hq, L, D]
    vv = _f(v_cache[0, :, :L, :], dtype).repeat_interleave(g, 0)
    scores = torch.einsum("hd,hld->hl", _f(q, dtype), kk) * scaling
    p = torch.softmax(scores, -1)
    return torch.einsum("hl,hld->hd", p, vv)


def decode_attention_lse(q, k_cache, v_cache, cache_position, scaling, dtype=torch.float64):
    """Per-head log-sum-exp of the scaled scores (for the split-KV merge checks)."""
    hq = q.shape[0]
    hkv, t = k_cache.shape[1], k_cache.shape[2]
    L = min(int(cache_position) + 1, t)
    kk = _f(k_cache[0, :, :L, :], dtype).repeat_interleave(hq // hkv, 0)
    scores = torch.einsum("hd,hld->hl", _f(q, dtype), kk) * scaling
    return torch.logsumexp(scores, -1)


def silu_mul(gate, up, dtype=torch.float32):
    g = _f(gate, dtype)
    return g * torch.sigmoid(g) * _f(up, dtype)


def post_attn_mlp(residual, attn_out, norm_weight, gate_up_weight, down_weight, bias, eps,
                  dtype=torch.float32):
    """Returns (hidden [I], out [H], r [H]) with r = residual + attn_out,
    hidden = silu(W_g x) * (W_u x) for x = rmsnorm(r), out = W_d hidden + r (+ bias)."""
    r = _f(residual, dtype) + _f(attn_out, dtype)
    x = rms_norm(r, norm_weight, eps, dtype)
    gu = gemv(x, gate_up_weight, None, dtype)
    i = gate_up_weight.shape[0] // 2
    hidden = silu_mul(gu[..., :i], gu[..., i:], dtype)
    out = gemv(hidden, down_weight, bias, dtype) + r
    return hidden, out, r


# ----------------------------------------------------------------- layer / model


def decode_layer(w: dict, hidden, k_cache, v_cache, cache_position, cos, sin,
                 shape: OracleShape = SHAPE, dtype=torch.float32):
    """One decoder layer for one token (optimized_layer.py:108-469 op order).

    ``w`` holds the fused layout (qkv_weight, o_proj_weight, gate_up_weight,
    down_proj_weight, input_layernorm_weight, post_attn_layernorm_weight,
    q_norm_weight, k_norm_weight).  hidden [H]; cos/sin [D]; caches are
    written at ``cache_position``.  Returns the layer output [H] in ``dtype``.
    """
    x = _f(hidden, dtype)
    xn = rms_norm(x, w["input_layernorm_weight"], shape.rms_eps, dtype)
    qkv = gemv(xn, w["qkv_weight"], None, dtype)
    q = qkv[: shape.q_size].view(shape.num_heads, shape.head_dim)
    k = qkv[shape.q_size: shape.q_size + shape.kv_size].view(shape.num_kv_heads, shape.head_dim)
    v = qkv[shape.q_size + shape.kv_size:].view(shape.num_kv_heads, shape.head_dim)
    q_rot = q_rope_kv_update(q, k, v, w["q_norm_weight"], w["k_norm_weight"], shape.rms_eps,
                             cos, sin, k_cache, v_cache, cache_position, dtype)
    attn = decode_attention(q_rot, k_cache, v_cache, cache_position, shape.head_dim ** -0.5, dtype=dtype)
    o = gemv(attn.reshape(-1), w["o_proj_weight"], None, dtype)
    _, out, _ = post_attn_mlp(x, o, w["post_attn_layernorm_weight"], w["gate_up_weight"],
                              w["down_proj_weight"], None, shape.rms_eps, dtype)
    return out


def lm_head_argmax(hidden, final_norm_weight, lm_head_weight, eps, dtype=torch.float32):
    """Final RMSNorm, tied lm_head, argmax with the first maximal index winning."""
    hn = rms_norm(hidden, final_norm_weight, eps, dtype)
    logits = gemv(hn, lm_head_weight, None, dtype)
    return logits, int(torch.argmax(logits, -1))


def top2_margin(logits: torch.Tensor) -> float:
    v = torch.topk(logits.to(torch.float64), 2).values
    return float(v[0] - v[1])


def _layer_dict(lw) -> dict:
    return lw if isinstance(lw, dict) else lw.tensors()


def prefill(weights, embeds: torch.Tensor, position_ids: torch.Tensor, caches,
            shape: OracleShape = SHAPE, dtype=torch.float32, layer_chunk: int | None = None):
    """Causal prefill over S prompt rows (HF:769-852 loop; HF:526-568 layer).

    embeds [S, H]; position_ids [3, S]; caches: list of (k_cache, v_cache)
    [1, Hkv, T, D] written at rows 0..S-1.  Returns the last row's hidden state
    before the final norm.
    """
    S = embeds.shape[0]
    cos, sin = mrope_cos_sin(position_ids, shape, dtype)          # [S, D]
    h = _f(embeds, dtype)
    causal = torch.ones(S, S, dtype=torch.bool).tril()
    for li, lw in enumerate(weights.layers):
        w = _layer_dict(lw)
        xn = rms_norm(h, w["input_layernorm_weight"], shape.rms_eps, dtype)
        qkv = xn @ _f(w["qkv_weight"], dtype).T
        q = qkv[:, : shape.q_size].view(S, shape.num_heads, shape.head_dim)
        k = qkv[:, shape.q_size: shape.q_size + shape.kv_size].view(S, shape.num_kv_heads, shape.head_dim)
        v = qkv[:, shape.q_size + shape.kv_size:].view(S, shape.num_kv_heads, shape.head_dim)
        q = apply_rope(rms_norm(q, w["q_norm_weight"], shape.rms_eps, dtype), cos[:, None], sin[:, None])
        k = apply_rope(rms_norm(k, w["k_norm_weight"], shape.rms_eps, dtype), cos[:, None], sin[:, None])
        kc, vc = caches[li]
        kc[0, :, :S] = k.transpose(0, 1).to(kc.dtype)
        vc[0, :, :S] = v.transpose(0, 1).to(vc.dtype)
        qh = q.transpose(0, 1)                                     # [Hq, S, D]
        kh = k.transpose(0, 1).repeat_interleave(shape.num_heads // shape.num_kv_heads, 0)
        vh = v.transpose(0, 1).repeat_interleave(shape.num_heads // shape.num_kv_heads, 0)
        attn = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=causal, scale=shape.head_dim ** -0.5)
        o = attn.transpose(0, 1).reshape(S, shape.q_size) @ _f(w["o_proj_weight"], dtype).T
        r = h + o
        xn2 = rms_norm(r, w["post_attn_layernorm_weight"], shape.rms_eps, dtype)
        gu = xn2 @ _f(w["gate_up_weight"], dtype).T
        i = shape.intermediate
        hid = silu_mul(gu[:, :i], gu[:, i:], dtype)
        h = r + hid @ _f(w["down_proj_weight"], dtype).T
    return h[-1]


def embed_prompt(weights, prompt, dtype=torch.float32) -> torch.Tensor:
    """Rows: vision embeddings as given, then embedding-table rows of the text ids."""
    txt = weights.embed_tokens[prompt.text_ids]
    return torch.cat([_f(prompt.vision_embeds, dtype), _f(txt, dtype)], 0)


def greedy_generate(weights, prompt, n_tokens: int, capacity: int, shape: OracleShape = SHAPE,
                    dtype=torch.float32, caches=None, first_token: int | None = None,
                    start_position: int | None = None, log=None, logits_out: list | None = None,
                    cache_dtype=torch.float16, rope_delta: int | None = None):
    """Greedy decoding after a prefill (evaluation_wrapper.py:149-315 semantics).

    Returns (tokens [n_tokens], margins [n_tokens]) where tokens[0] is the
    prefill's argmax and tokens[i] the i-th decode step's argmax.  The decode
    step at cache position p uses rope position p + rope_delta on all three
    streams (evaluation_wrapper.py:507-511, :954-960).  When ``caches``,
    ``first_token`` and ``start_position`` are given the prefill is skipped and
    decoding continues from that state.  ``logits_out``, when given, receives
    the logits of every generated token (prefill first).  The static cache is
    fp16 as the reference's (``cache_dtype`` changes it for comparisons with
    an fp32 cache); ``rope_delta`` overrides the prompt's (tests plant a wrong
    one to show the checks see it).
    """
    delta = prompt.rope_delta if rope_delta is None else int(rope_delta)
    tokens, margins = [], []
    if caches is None:
        caches = [(torch.zeros(1, shape.num_kv_heads, capacity, shape.head_dim, dtype=cache_dtype),
                   torch.zeros(1, shape.num_kv_heads, capacity, shape.head_dim, dtype=cache_dtype))
                  for _ in weights.layers]
        h_last = prefill(weights, embed_prompt(weights, prompt, dtype), prompt.position_ids, caches, shape, dtype)
        logits, tok = lm_head_argmax(h_last, weights.final_norm_weight, weights.embed_tokens, shape.rms_eps, dtype)
        tokens.append(tok)
        margins.append(top2_margin(logits))
        if logits_out is not None:
            logits_out.append(logits)
        pos = prompt.length
    else:
        tokens.append(int(first_token))
        margins.append(float("nan"))
        pos = int(start_position)
    inv_cache = {}
    while len(tokens) < n_tokens:
        rp = pos + delta
        if rp not in inv_cache:
            cos, sin = mrope_cos_sin(torch.full((3, 1), rp, dtype=torch.int64), shape, dtype)
            inv_cache[rp] = (cos[0], sin[0])
        cos, sin = inv_cache[rp]
        h = _f(weights.embed_tokens[tokens[-1]], dtype)
        for li, lw in enumerate(weights.layers):
            kc, vc = caches[li]
            h = decode_layer(_layer_dict(lw), h, kc, vc, pos, cos, sin, shape, dtype)
        logits, tok = lm_head_argmax(h, weights.final_norm_weight, weights.embed_tokens, shape.rms_eps, dtype)
        tokens.append(tok)
        margins.append(top2_margin(logits))
        if logits_out is not None:
            logits_out.append(logits)
        if log is not None:
            log(len(tokens), tok, margins[-1])
        pos += 1
    return tokens, margins, caches


def decode_step_batch(weights, token_ids, caches, cache_positions, rope_positions,
                      shape: OracleShape = SHAPE, dtype=torch.float32):
    """Batch-B decode step with per-sequence cache positions (config 4).

    caches[l] = (k [B, Hkv, T, D], v [B, Hkv, T, D]).  Each sequence is the
    batch-1 step on its own cache rows.  Returns (logits [B, V], tokens [B]).
    """
    B = len(token_ids)
    outs_logits, outs_tok = [], []
    for b in range(B):
        cos, sin = mrope_cos_sin(torch.full((3, 1), int(rope_positions[b]), dtype=torch.int64), shape, dtype)
        h = _f(weights.embed_tokens[int(token_ids[b])], dtype)
        for li, lw in enumerate(weights.layers):
            kc, vc = caches[li]
            h = decode_layer(_layer_dict(lw), h, kc[b:b + 1], vc[b:b + 1], int(cache_positions[b]),
                             cos[0], sin[0], shape, dtype)
        logits, tok = lm_head_argmax(h, weights.final_norm_weight, weights.embed_tokens, shape.rms_eps, dtype)
        outs_logits.append(logits)
        outs_tok.append(tok)
    return torch.stack(outs_logits), outs_tok


def roofline_bytes_step(context_len: int, shape: OracleShape = SHAPE) -> int:
    """Algorithmic HBM bytes of one batch-1 decode step at KV length L (each weight,
    K/V element and activation counted once)."""
    h, i, d = shape.hidden, shape.intermediate, shape.head_dim
    layer_w = 2 * ((shape.q_size + 2 * shape.kv_size) * h + h * shape.q_size + 3 * i * h) + 2 * (2 * h + 2 * d)
    kv = 2 * 2 * shape.num_kv_heads * d * context_len
    return shape.num_layers * (layer_w + kv) + 2 * shape.vocab * h + 2 * h + 2 * h

