"""Qwen3-VL decoder layer whose batch-1 decode step runs on gfx950 HIP kernels.

Drop-in for the reference's optimized_layer.py: ``OptimizedDecoderLayer``
wraps an HF ``Qwen3VLTextDecoderLayer`` (same constructor, same forward
signature, fused qkv / gate_up weights as at optimized_layer.py:60-84), and
``replace_decoder_layers`` swaps it into a model.

Decode step (one token, batch 1, fp16, GPU, static KV cache; optimized_layer.py:108-469).
At the Qwen3-VL-2B shapes the whole layer is one persistent launch, the
reference's one-launch layer fused_decode_full_layer_softsync_half (tried
first, :127-154); otherwise, or with the ``full_layer_softsync`` fusion flag
off, the chain:

    fused_rmsnorm_qkv_half            RMSNorm + QKV GEMV        (HIP)
    fused_q_rope_kv_cache_update      q/k norm + RoPE + KV write (HIP)
    decode_attn_v4_cta_qhead_splitkv_fused  split-KV attention  (HIP)
    nosplit_matvec_half               o_proj GEMV               (HIP)
    fused_post_attn_mlp_softsync_half add+RMSNorm, gate_up+SiLU, down+residual (HIP)

If the HIP library is missing these raise RuntimeError.  Other inputs
(prefill with several tokens) take the HF layer math with PyTorch-ROCm ops,
like the reference's own non-decode path.  CPU tensors are rejected: the
CPU restatement of this math lives in the test oracle, not in the product.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

import cuda_decode_attention
import cuda_decode_gemv
import cuda_decode_small_ops
from cuda_decode_gemv_ops import fused as fused_ops


@dataclass(slots=True)
class PrefillFastpathContext:
    """Kept for import compatibility with the reference (optimized_layer.py:22-27)."""

    position_embeddings: tuple
    past_key_values: object
    cache_position: torch.Tensor
    cache_kwargs: dict | None


class OptimizedDecoderLayer(nn.Module):
    """Drop-in replacement for Qwen3VLTextDecoderLayer (reference optimized_layer.py:30-469)."""

    def __init__(self, orig_layer):
        super().__init__()
        attn = orig_layer.self_attn
        mlp = orig_layer.mlp
        self.hidden_size = orig_layer.hidden_size
        self.head_dim = attn.head_dim
        self.num_heads = attn.config.num_attention_heads
        self.num_kv_heads = attn.config.num_key_value_heads
        self.num_key_value_groups = attn.num_key_value_groups
        self.scaling = attn.scaling
        self.is_causal = attn.is_causal
        self.layer_idx = attn.layer_idx
        self.attention_dropout = attn.attention_dropout
        self.rms_norm_eps = attn.config.rms_norm_eps

        self.input_layernorm_weight = orig_layer.input_layernorm.weight
        self.post_attn_layernorm_weight = orig_layer.post_attention_layernorm.weight
        self.q_norm_weight = attn.q_norm.weight
        self.k_norm_weight = attn.k_norm.weight

        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_weight = nn.Parameter(
            torch.cat([attn.q_proj.weight.data, attn.k_proj.weight.data, attn.v_proj.weight.data], 0).contiguous(),
            requires_grad=False)
        self.qkv_bias = None
        if getattr(attn.q_proj, "bias", None) is not None:
            self.qkv_bias = torch.cat([attn.q_proj.bias.data, attn.k_proj.bias.data, attn.v_proj.bias.data], 0)
        self.o_proj = attn.o_proj
        self.o_proj_weight = attn.o_proj.weight
        self.o_proj_bias = attn.o_proj.bias

        self.intermediate_size = mlp.intermediate_size
        self.gate_up_weight = nn.Parameter(
            torch.cat([mlp.gate_proj.weight.data, mlp.up_proj.weight.data], 0).contiguous(), requires_grad=False)
        self.down_proj = mlp.down_proj
        self.down_proj_weight = mlp.down_proj.weight
        self.down_proj_bias = mlp.down_proj.bias

        self.config = attn.config
        self._attn_implementation = getattr(attn.config, "_attn_implementation", "sdpa")
        self._prefer_small_decode_triton = False
        # graph-stable workspaces of the decode kernels
        self._attention_workspace: dict = {}
        self._post_attn_mlp_workspace: dict = {"type": "fused_post_attn_mlp_softsync"}
        self._o_proj_workspace: dict = {"type": "nosplit"}
        self._full_layer_workspace: dict = {}
        self._stack: _LayerStack | None = None   # set by replace_decoder_layers
        self._stack_index = -1

    # ------------------------------------------------------------ dispatch
    def _static_layer(self, past_key_values, k_like: torch.Tensor):
        """The StaticLayer of this layer when its K/V tensors suit the HIP decode step."""
        if past_key_values is None:
            return None
        layers = getattr(past_key_values, "layers", None)
        if layers is None or self.layer_idx >= len(layers):
            return None
        layer = layers[self.layer_idx]
        if not getattr(layer, "is_initialized", True) and hasattr(layer, "lazy_initialization"):
            layer.lazy_initialization(k_like, k_like)
        kc, vc = getattr(layer, "keys", None), getattr(layer, "values", None)
        if kc is None or vc is None or kc.ndim != 4 or kc.shape[0] != 1 or kc.device != k_like.device:
            return None
        if getattr(layer, "max_cache_len", kc.shape[2]) != kc.shape[2]:
            return None
        return layer

    @staticmethod
    def _decode_position(layer, cache_position, device):
        """Cache row of the new token: ``cache_position`` when the caller gives
        it (the reference's graph runner does, evaluation_wrapper.py:941-960),
        else the StaticLayer's running length ``cumulative_length``, which is
        where transformers' own StaticLayer.update writes (cache_utils.py
        StaticLayer.update).  Both stay on the device (no host sync)."""
        if cache_position is not None:
            if cache_position.device.type == "cuda" and cache_position.numel() == 1:
                return cache_position.reshape(1)
            return None
        cl = getattr(layer, "cumulative_length", None)
        if torch.is_tensor(cl) and cl.device == device and cl.numel() == 1 and cl.dtype == torch.int64:
            return cl.reshape(1)
        return None

    @staticmethod
    def _length_word(layer, pos: torch.Tensor):
        """The StaticLayer's running length when it is one int64 word beside
        ``pos`` on the device: the layer's last kernel then advances it."""
        cl = getattr(layer, "cumulative_length", None)
        if torch.is_tensor(cl) and cl.device == pos.device and cl.dtype == torch.int64 and cl.numel() == 1 \
                and cl.is_contiguous():
            return cl
        return None

    @staticmethod
    def _advance_length(layer, pos: torch.Tensor) -> None:
        """Keep the StaticLayer's running length at pos + 1 after the HIP step
        wrote row ``pos``, as StaticLayer.update would: transformers reads it
        for default position ids and the next write row.  In place on the
        device, so it is also replayed inside a captured graph."""
        cl = getattr(layer, "cumulative_length", None)
        if torch.is_tensor(cl) and cl.device == pos.device:
            cl.copy_((pos + 1).reshape(cl.shape))
        elif cl is not None and not torch.cuda.is_current_stream_capturing():
            layer.cumulative_length = (pos + 1).reshape(())

    def _decode_ok(self, hidden_states, position_embeddings) -> bool:
        cos, sin = position_embeddings
        return (hidden_states.device.type == "cuda" and hidden_states.dtype == torch.float16
                and hidden_states.ndim == 3 and hidden_states.shape[0] == 1 and hidden_states.shape[1] == 1
                and self.head_dim == 128
                and self.num_heads == 2 * self.num_kv_heads and cos.dtype == torch.float16
                and cos.numel() == 128 and sin.numel() == 128 and self.qkv_bias is None)

    def forward(self, hidden_states: torch.Tensor, position_embeddings: tuple, attention_mask=None,
                position_ids=None, past_key_values=None, use_cache=False, cache_position=None,
                **kwargs) -> torch.Tensor:
        if hidden_states.device.type != "cuda":
            raise RuntimeError("OptimizedDecoderLayer runs on a ROCm GPU (got a CPU tensor)")
        kwargs.pop("prefill_static_cache_no_mask", None)
        if self._decode_ok(hidden_states, position_embeddings):
            layer = self._static_layer(past_key_values,
                                       hidden_states.new_empty(1, self.num_kv_heads, 1, self.head_dim))
            pos = self._decode_position(layer, cache_position, hidden_states.device) if layer is not None else None
            if pos is not None:
                length = self._length_word(layer, pos)
                if _LOOKAHEAD[0] and self._stack is not None:
                    out = self._stack.step(self, hidden_states, position_embeddings, past_key_values, pos)
                    if out is not None:
                        return out
                out = self._decode_step(hidden_states, position_embeddings, (layer.keys, layer.values), pos, length)
                if length is None:
                    self._advance_length(layer, pos)
                return out
        return self._general_forward(hidden_states, position_embeddings, attention_mask, position_ids,
                                     past_key_values, use_cache, cache_position, **kwargs)

    # ------------------------------------------------------------ HIP decode chain
    def _decode_step(self, hidden_states, position_embeddings, kv, cache_position, length=None):
        """The HIP decode step of one layer; with ``length`` (the cache's
        running-length word) its last kernel also sets length = position + 1."""
        cos, sin = position_embeddings
        k_cache, v_cache = kv
        eps = self.rms_norm_eps
        if _FUSION_FLAGS["full_layer_softsync"]:
            out = fused_ops._full_layer_persistent(
                hidden_states, self.qkv_weight, self.input_layernorm_weight, self.q_norm_weight, self.k_norm_weight,
                cos, sin, k_cache, v_cache, cache_position, self.o_proj_weight, self.o_proj_bias,
                self.post_attn_layernorm_weight, self.gate_up_weight, self.down_proj_weight, self.down_proj_bias,
                eps, self.scaling, self._full_layer_workspace, length=length)
            if out is not None:
                return out
        qkv = cuda_decode_gemv.fused_rmsnorm_qkv_half(hidden_states, self.input_layernorm_weight, self.qkv_weight,
                                                      None, eps)
        # q/k norm + RoPE + K/V write + attention in one launch; the two-call
        # form (the reference's own sequence) where that kernel does not apply
        attn = cuda_decode_attention._qkv_rope_attention(
            qkv, self.q_norm_weight, self.k_norm_weight, eps, cos.reshape(128), sin.reshape(128), k_cache, v_cache,
            self.scaling, cache_position, split_k=4, workspace=self._attention_workspace)
        if attn is None:
            q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
            q_rot = cuda_decode_small_ops.fused_q_rope_kv_cache_update(
                q.view(1, 1, self.num_heads, self.head_dim), k.view(1, 1, self.num_kv_heads, self.head_dim),
                v.view(1, 1, self.num_kv_heads, self.head_dim), self.q_norm_weight, self.k_norm_weight, eps,
                cos.reshape(1, 1, 128), sin.reshape(1, 1, 128), k_cache, v_cache, cache_position)
            attn = cuda_decode_attention.decode_attn_v4_cta_qhead_splitkv_fused(
                q_rot.transpose(1, 2), k_cache, v_cache, self.scaling, self.num_key_value_groups, cache_position,
                split_k=4, workspace=self._attention_workspace)
        if attn is None:
            raise RuntimeError("decode attention inputs unsupported by the HIP kernel")
        attn = attn.reshape(1, 1, self.q_size)
        o = cuda_decode_gemv.nosplit_matvec_half(attn, self.o_proj_weight, self.o_proj_bias,
                                                 workspace=self._o_proj_workspace)
        _hidden, out = fused_ops._post_attn_mlp(
            "fused_post_attn_mlp_softsync_half", hidden_states, o, self.post_attn_layernorm_weight,
            self.gate_up_weight, self.down_proj_weight, self.down_proj_bias, eps, self._post_attn_mlp_workspace,
            "fused_post_attn_mlp_softsync",
            next_position=None if length is None else (cache_position, length))
        return out

    # ------------------------------------------------------------ general (prefill) path
    def _general_forward(self, hidden_states, position_embeddings, attention_mask, position_ids, past_key_values,
                         use_cache, cache_position, **kwargs):
        """HF Qwen3VLTextDecoderLayer math (transformers modeling_qwen3_vl.py:526-568) on PyTorch-ROCm."""
        from transformers.models.qwen3_vl.modeling_qwen3_vl import apply_rotary_pos_emb, eager_attention_forward
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

        residual = hidden_states
        input_shape = hidden_states.shape[:-1]
        x = _rms_norm(hidden_states, self.input_layernorm_weight, self.rms_norm_eps)
        qkv = F.linear(x, self.qkv_weight, self.qkv_bias)
        q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
        q = _rms_norm(q.view(*input_shape, -1, self.head_dim), self.q_norm_weight, self.rms_norm_eps).transpose(1, 2)
        k = _rms_norm(k.view(*input_shape, -1, self.head_dim), self.k_norm_weight, self.rms_norm_eps).transpose(1, 2)
        v = v.view(*input_shape, -1, self.head_dim).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        if past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx, {"sin": sin, "cos": cos,
                                                                  "cache_position": cache_position})
        interface = ALL_ATTENTION_FUNCTIONS.get_interface(self._attn_implementation, eager_attention_forward)
        attn, _ = interface(self, q, k, v, attention_mask, dropout=0.0, scaling=self.scaling, **kwargs)
        attn = attn.reshape(*input_shape, -1).contiguous()
        h = residual + F.linear(attn, self.o_proj_weight, self.o_proj_bias)
        x2 = _rms_norm(h, self.post_attn_layernorm_weight, self.rms_norm_eps)
        gu = F.linear(x2, self.gate_up_weight)
        gate, up = gu.split([self.intermediate_size, self.intermediate_size], dim=-1)
        return h + F.linear(F.silu(gate) * up, self.down_proj_weight, self.down_proj_bias)


_LOOKAHEAD = [os.environ.get("QD_DECODE_LAYER_LOOKAHEAD", "0") == "1"]


def set_decode_layer_lookahead(enabled: bool) -> bool:
    """Opt-in look-ahead of the swapped layers' decode step (off by default;
    also QD_DECODE_LAYER_LOOKAHEAD=1): the first swapped layer of a step runs
    every swapped layer in one persistent launch when all of them qualify for
    the one-launch layer and carry no hooks, and each later layer returns its
    row of that launch's output when its input is the previous layer's row,
    untouched.  Each row is bit for bit what the layer's own launch would
    return (the launch hands fp16 outputs from layer to layer).  In any other
    case a layer runs its own launch.  Returns the previous setting."""
    prev = _LOOKAHEAD[0]
    _LOOKAHEAD[0] = bool(enabled)
    return prev


_STACK_MAX_LAYERS = 32   # layers one persistent launch takes (kPersistMaxLayers, csrc/qd_kernels.h)


class _LayerStack:
    """The swapped decoder layers of one model, in order (replace_decoder_layers
    makes one per model), and the state of a look-ahead launch in flight: its
    output rows [n, 2048] (a stable buffer, so a captured graph keeps reading
    it), its status word, the next layer allowed to take its row and the
    rows' version when they were written."""

    def __init__(self, layers):
        self.layers = layers            # the model's own layer list
        self.out = None
        self.status = None
        self.next = -1
        self.version = -1

    def _members(self):
        ls = list(self.layers)
        ok = all(isinstance(L, OptimizedDecoderLayer) and L._stack is self and L._stack_index == i
                 for i, L in enumerate(ls))
        return ls if ok else None

    @staticmethod
    def _hook_free(layer) -> bool:
        from torch.nn.modules import module as _m

        return not (layer._forward_hooks or layer._forward_pre_hooks or getattr(layer, "_backward_hooks", None)
                    or _m._global_forward_hooks or _m._global_forward_pre_hooks)

    def step(self, layer, hidden_states, position_embeddings, past_key_values, pos):
        i = layer._stack_index
        if i > 0:
            out = self.out
            if (self.next == i and out is not None and hidden_states.shape == (1, 1, 2048)
                    and hidden_states.data_ptr() == out[i - 1].data_ptr()
                    and hidden_states._version == self.version):
                self.next = i + 1 if i + 1 < out.shape[0] else -1
                return out[i].view(1, 1, 2048)
            self.next = -1
            return None
        self.next = -1
        return self._launch(hidden_states, position_embeddings, past_key_values, pos)

    def _launch(self, h, position_embeddings, past_key_values, pos):
        members = self._members()
        if (members is None or not 2 <= len(members) <= _STACK_MAX_LAYERS
                or not _FUSION_FLAGS["full_layer_softsync"]):
            return None
        cos, sin = position_embeddings
        cos, sin = cos.reshape(-1), sin.reshape(-1)
        rows, lengths, statics = [], [], []
        cap = None
        for L in members:
            if not self._hook_free(L) or not L._decode_ok(h, position_embeddings):
                return None
            st = L._static_layer(past_key_values, h.new_empty(1, L.num_kv_heads, 1, L.head_dim))
            if st is None:
                return None
            kc, vc = st.keys, st.values
            length = L._length_word(st, pos)
            if cap is None:
                cap = kc.shape[2]
            if kc.shape[2] != cap or not fused_ops._full_layer_eligible(
                    h, L.qkv_weight, L.input_layernorm_weight, L.q_norm_weight, L.k_norm_weight, cos, sin, kc, vc,
                    pos, L.o_proj_weight, L.o_proj_bias, L.post_attn_layernorm_weight, L.gate_up_weight,
                    L.down_proj_weight, L.down_proj_bias, length):
                return None
            rows.append((L.qkv_weight, L.o_proj_weight, L.gate_up_weight, L.down_proj_weight,
                         L.input_layernorm_weight, L.post_attn_layernorm_weight, L.q_norm_weight, L.k_norm_weight,
                         kc, vc))
            lengths.append(length)
            statics.append(st)
        n = len(members)
        if self.out is None or self.out.shape[0] != n or self.out.device != h.device:
            if torch.cuda.is_current_stream_capturing():
                return None            # the buffers are allocated outside capture
            self.out = torch.empty(n, 2048, dtype=torch.float16, device=h.device)
            self.status = torch.zeros(1, dtype=torch.int32, device=h.device)
        eps, scale = members[0].rms_norm_eps, members[0].scaling
        if any(L.rms_norm_eps != eps or L.scaling != scale for L in members):
            return None
        if not fused_ops._layer_stack_launch(h, rows, cos, sin, pos, lengths, self.out, self.status, eps, scale):
            return None
        for st, length in zip(statics, lengths):
            if length is None:
                OptimizedDecoderLayer._advance_length(st, pos)
        self.version = self.out._version
        self.next = 1
        return self.out[0].view(1, 1, 2048)


def _rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """HF Qwen3VLTextRMSNorm (modeling_qwen3_vl.py:400-405)."""
    dt = x.dtype
    xf = x.to(torch.float32)
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(dt)


def _decoder_layers(model):
    for path in ("model.language_model.layers", "language_model.layers", "model.layers", "layers"):
        obj = model
        try:
            for part in path.split("."):
                obj = getattr(obj, part)
        except AttributeError:
            continue
        return obj
    raise RuntimeError("could not find the decoder layer list on this model")


def replace_decoder_layers(model) -> int:
    """Swap every text decoder layer for OptimizedDecoderLayer (reference
    optimized_layer.py:3848-3858); the new layers are put in eval mode when
    the model is, as there."""
    layers = _decoder_layers(model)
    is_eval = not getattr(model, "training", False)
    n = 0
    for i, layer in enumerate(layers):
        if not isinstance(layer, OptimizedDecoderLayer):
            layers[i] = OptimizedDecoderLayer(layer)
            if is_eval:
                layers[i].eval()
            n += 1
    # the model's swapped layers in order, for the opt-in look-ahead launch
    stack = _LayerStack(layers)
    for i, layer in enumerate(layers):
        if isinstance(layer, OptimizedDecoderLayer):
            layer._stack = stack
            layer._stack_index = i
    return n


def check_decode_status(model, reset: bool = True) -> None:
    """Raise RuntimeError if a swapped layer's one-launch decode step ran out of
    its hand-off polling budget since the last check (bit 0 of the layer's
    status word; the launch then also wrote NaN into the outputs it could not
    compute).  That happens only when the launch's 256 workgroups could not all
    stay resident, e.g. other work occupied CUs.  Reads every status word (one
    device synchronisation); call it outside stream capture, e.g. after a
    generation.  ``reset`` clears the words that were set."""
    bad = []
    stacks = []
    for i, layer in enumerate(_decoder_layers(model)):
        st = getattr(layer, "_full_layer_workspace", {}).get("status") if isinstance(
            layer, OptimizedDecoderLayer) else None
        if st is not None and int(st.item()) != 0:
            bad.append(str(i))
            if reset:
                st.zero_()
        stack = getattr(layer, "_stack", None)
        if stack is not None and stack not in stacks:
            stacks.append(stack)
    for stack in stacks:
        if stack.status is not None and int(stack.status.item()) != 0:
            bad.append("stack (look-ahead launch)")
            if reset:
                stack.status.zero_()
    if bad:
        raise RuntimeError("one-launch decoder layer: a hand-off wait ran out of its polling budget in layer "
                           + ", ".join(bad) + " (its outputs are NaN)")


def set_small_decode_triton_enabled(model, enabled: bool) -> bool:
    """Reference optimized_layer.py:3861-3873 toggled the graph-only fast paths.

    The HIP decode chain is used whenever inputs qualify, so the flag is only
    recorded on each layer.  Returns the previous value of the first layer."""
    layers = _decoder_layers(model)
    prev = bool(getattr(layers[0], "_prefer_small_decode_triton", False)) if len(layers) else False
    for layer in layers:
        if isinstance(layer, OptimizedDecoderLayer):
            layer._prefer_small_decode_triton = bool(enabled)
    return prev


_FUSION_FLAG_NAMES = ("add_rmsnorm_gateup", "full_layer_softsync", "post_attn_mlp_persistent",
                      "o_proj_post_attn_mlp_persistent", "o_proj_post_attn_mlp_softsync", "silu_downproj",
                      "gateup_silu_downproj", "gateup_silu_downproj_mega")
# full_layer_softsync: the swapped layer's decode step is one persistent launch
# where the shapes allow (on by default here: on MI355X it is faster than the
# kernel chain; the reference's A800 default was off)
_FUSION_FLAGS = {n: n in ("post_attn_mlp_persistent", "full_layer_softsync") for n in _FUSION_FLAG_NAMES}
# The reference reads its choices from the environment at import
# (optimized_layer.py:837-921).  A variable that is set explicitly is honoured
# here too ("1" on, anything else off); an unset one keeps the default above.
_FUSION_FLAG_ENV = {n: "ENABLE_CUDA_FUSED_" + n.upper() for n in _FUSION_FLAG_NAMES}
for _n, _var in _FUSION_FLAG_ENV.items():
    if os.environ.get(_var) is not None:
        _FUSION_FLAGS[_n] = os.environ[_var] == "1"


def set_cuda_mlp_fusion_flags(*, add_rmsnorm_gateup: bool | None = None, full_layer_softsync: bool | None = None,
                              post_attn_mlp_persistent: bool | None = None,
                              o_proj_post_attn_mlp_persistent: bool | None = None,
                              o_proj_post_attn_mlp_softsync: bool | None = None, silu_downproj: bool | None = None,
                              gateup_silu_downproj: bool | None = None,
                              gateup_silu_downproj_mega: bool | None = None) -> tuple:
    """Reference optimized_layer.py:3876-3921: sets the MLP fusion choices and
    returns the previous 8-tuple.  ``full_layer_softsync`` selects the
    one-launch layer (on by default) or the kernel chain; the other choices
    compute the same math on gfx950 and are recorded for callers that read
    them back."""
    prev = tuple(_FUSION_FLAGS[n] for n in _FUSION_FLAG_NAMES)
    new = dict(add_rmsnorm_gateup=add_rmsnorm_gateup, full_layer_softsync=full_layer_softsync,
               post_attn_mlp_persistent=post_attn_mlp_persistent,
               o_proj_post_attn_mlp_persistent=o_proj_post_attn_mlp_persistent,
               o_proj_post_attn_mlp_softsync=o_proj_post_attn_mlp_softsync, silu_downproj=silu_downproj,
               gateup_silu_downproj=gateup_silu_downproj, gateup_silu_downproj_mega=gateup_silu_downproj_mega)
    for n, v in new.items():
        if v is not None:
            _FUSION_FLAGS[n] = bool(v)
    return prev


def fused_vision_rope(*args, **kwargs):
    """The reference's vision-tower RoPE kernel (optimized_layer.py:3268) belongs to the
    prefill path, which this build does not provide."""
    raise NotImplementedError("fused_vision_rope is part of the vision prefill path (out of scope)")
