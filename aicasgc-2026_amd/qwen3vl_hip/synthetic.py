"""Seeded synthetic inputs for the decode-path configurations.

Every tensor is drawn from its own numpy PCG64 stream keyed by
``(seed, *key)`` so that a tensor does not depend on which other tensors were
generated before it, and generation can run on several threads.  numpy's
PCG64 + ziggurat normal sampler is integer/float arithmetic only, so the same
key produces the same bits on every x86 host running this image (the build
container and the GPU box both generate the weights on the CPU).

Distributions follow the benchmark configurations: projection weights
N(0, 0.02) fp16, norm weights 1 + N(0, 0.02) fp16, activations N(0, 1),
KV-cache prefixes N(0, 1) fp16.
"""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np
import torch

from .config import QWEN3VL_2B, Qwen3VLTextShape

# Stable integer ids for tensor names inside a seed key.
_NAME_IDS = {
    "q_proj": 1, "k_proj": 2, "v_proj": 3, "o_proj": 4,
    "gate_proj": 5, "up_proj": 6, "down_proj": 7,
    "input_layernorm": 8, "post_attention_layernorm": 9, "q_norm": 10, "k_norm": 11,
    "embed_tokens": 20, "final_norm": 21,
    "x": 30, "W": 31, "q": 32, "k_cache": 33, "v_cache": 34, "k": 35, "v": 36,
    "vision_embeds": 40, "text_ids": 41, "kv_len": 42, "residual": 43, "attn": 44,
}


def _rng(seed: int, key: tuple) -> np.random.Generator:
    ints = [int(seed)] + [(_NAME_IDS[k] if isinstance(k, str) else int(k)) for k in key]
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence(ints)))


def normal(seed: int, key: tuple, shape, std: float = 1.0, mean: float = 0.0,
           dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """N(mean, std^2) tensor of ``shape``; drawn in fp32, then rounded to ``dtype``."""
    n = int(np.prod(shape))
    a = _rng(seed, key).standard_normal(n, dtype=np.float32)
    if std != 1.0:
        a *= np.float32(std)
    if mean != 0.0:
        a += np.float32(mean)
    t = torch.from_numpy(a.reshape(shape))
    return t.to(dtype) if dtype != torch.float32 else t


def randint(seed: int, key: tuple, shape, low: int, high: int) -> torch.Tensor:
    a = _rng(seed, key).integers(low, high, size=shape, dtype=np.int64)
    return torch.from_numpy(a)


def _pool_workers() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(16, n))


@dataclass
class LayerWeights:
    """One decoder layer in the fused layout of `optimized_layer.py:60-84`.

    qkv_weight = cat(q_proj, k_proj, v_proj) [4096, 2048];
    gate_up_weight = cat(gate_proj, up_proj) [12288, 2048];
    o_proj_weight [2048, 2048]; down_proj_weight [2048, 6144];
    four norm vectors.  All fp16, row-major, contiguous.
    """

    qkv_weight: torch.Tensor
    o_proj_weight: torch.Tensor
    gate_up_weight: torch.Tensor
    down_proj_weight: torch.Tensor
    input_layernorm_weight: torch.Tensor
    post_attn_layernorm_weight: torch.Tensor
    q_norm_weight: torch.Tensor
    k_norm_weight: torch.Tensor

    def tensors(self) -> dict:
        return dict(self.__dict__)

    def to(self, device) -> "LayerWeights":
        return LayerWeights(**{k: v.to(device) for k, v in self.__dict__.items()})


def layer_weights(seed: int, layer: int, shape: Qwen3VLTextShape = QWEN3VL_2B,
                  pool: ThreadPoolExecutor | None = None) -> LayerWeights:
    h, d, i = shape.hidden, shape.head_dim, shape.intermediate
    specs = {
        "q_proj": ((shape.q_size, h), 0.02, 0.0),
        "k_proj": ((shape.kv_size, h), 0.02, 0.0),
        "v_proj": ((shape.kv_size, h), 0.02, 0.0),
        "o_proj": ((h, shape.q_size), 0.02, 0.0),
        "gate_proj": ((i, h), 0.02, 0.0),
        "up_proj": ((i, h), 0.02, 0.0),
        "down_proj": ((h, i), 0.02, 0.0),
        "input_layernorm": ((h,), 0.02, 1.0),
        "post_attention_layernorm": ((h,), 0.02, 1.0),
        "q_norm": ((d,), 0.02, 1.0),
        "k_norm": ((d,), 0.02, 1.0),
    }

    def make(name):
        shp, std, mean = specs[name]
        return name, normal(seed, (layer, name), shp, std=std, mean=mean)

    if pool is not None:
        t = dict(pool.map(make, specs))
    else:
        t = dict(make(n) for n in specs)
    return LayerWeights(
        qkv_weight=torch.cat([t["q_proj"], t["k_proj"], t["v_proj"]], 0).contiguous(),
        o_proj_weight=t["o_proj"],
        gate_up_weight=torch.cat([t["gate_proj"], t["up_proj"]], 0).contiguous(),
        down_proj_weight=t["down_proj"],
        input_layernorm_weight=t["input_layernorm"],
        post_attn_layernorm_weight=t["post_attention_layernorm"],
        q_norm_weight=t["q_norm"],
        k_norm_weight=t["k_norm"],
    )


@dataclass
class ModelWeights:
    layers: list
    embed_tokens: torch.Tensor      # [V, H]; also the tied lm_head weight
    final_norm_weight: torch.Tensor  # [H]
    shape: Qwen3VLTextShape = QWEN3VL_2B

    def to(self, device) -> "ModelWeights":
        return ModelWeights([lw.to(device) for lw in self.layers],
                            self.embed_tokens.to(device), self.final_norm_weight.to(device), self.shape)


def model_weights(seed: int, shape: Qwen3VLTextShape = QWEN3VL_2B, num_layers: int | None = None,
                  device=None) -> ModelWeights:
    """Random-init fp16 weights for the text decoder + tied lm_head.

    When ``device`` is given each layer is moved there as soon as it is made, so
    host memory holds at most a few layers at a time.
    """
    n_layers = shape.num_layers if num_layers is None else num_layers
    with ThreadPoolExecutor(_pool_workers()) as pool:
        emb_f = pool.submit(normal, seed, ("embed_tokens",), (shape.vocab, shape.hidden), 0.02)
        layers = []
        for li in range(n_layers):
            lw = layer_weights(seed, li, shape, pool)
            layers.append(lw.to(device) if device is not None else lw)
        emb = emb_f.result()
    fnorm = normal(seed, ("final_norm",), (shape.hidden,), std=0.02, mean=1.0)
    if device is not None:
        emb, fnorm = emb.to(device), fnorm.to(device)
    return ModelWeights(layers, emb, fnorm, shape)


# ---------------------------------------------------------------- configurations

@dataclass
class LayerStepInputs:
    """Config 0: one decoder layer, one decode step at batch 1."""

    weights: LayerWeights
    hidden: torch.Tensor          # [1, 1, H] fp16
    k_cache: torch.Tensor         # [1, KVH, T, D] fp16, positions < cache_position filled
    v_cache: torch.Tensor
    cache_position: int
    rope_position: int


def layer_step_inputs(seed: int = 0, cache_position: int = 512, capacity: int | None = None,
                      shape: Qwen3VLTextShape = QWEN3VL_2B) -> LayerStepInputs:
    cap = cache_position + 1 if capacity is None else capacity
    w = layer_weights(seed, 0, shape)
    x = normal(seed, ("x",), (1, 1, shape.hidden))
    kc = torch.zeros(1, shape.num_kv_heads, cap, shape.head_dim, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    kc[:, :, :cache_position] = normal(seed, ("k_cache",), (1, shape.num_kv_heads, cache_position, shape.head_dim))
    vc[:, :, :cache_position] = normal(seed, ("v_cache",), (1, shape.num_kv_heads, cache_position, shape.head_dim))
    return LayerStepInputs(w, x, kc, vc, cache_position, cache_position)


GEMV_SHAPES = {
    # name: (N, K) — batch-1 decode GEMVs of the model (config 1)
    "qkv": (4096, 2048),
    "o_proj": (2048, 2048),
    "gate_up": (12288, 2048),
    "down_proj": (2048, 6144),
    "lm_head": (151936, 2048),
}


def gemv_inputs(name: str, seed: int = 1):
    n, k = GEMV_SHAPES[name]
    sid = list(GEMV_SHAPES).index(name)
    x = normal(seed, ("x", sid), (1, 1, k))
    w = normal(seed, ("W", sid), (n, k), std=0.02)
    return x, w


def attention_inputs(kv_len: int, seed: int = 2, capacity: int | None = None,
                     shape: Qwen3VLTextShape = QWEN3VL_2B, stale_fill: float | None = None):
    """Config 2: q [1, 16, 1, 128], K/V caches [1, 8, T, 128]; valid prefix = kv_len.

    ``cache_position`` is kv_len - 1.  When ``capacity`` exceeds kv_len the tail
    beyond the valid prefix is filled with ``stale_fill`` (default: large
    values) so any read past the valid prefix changes the result.
    """
    cap = kv_len if capacity is None else capacity
    q = normal(seed, ("q", kv_len), (1, shape.num_heads, 1, shape.head_dim))
    kc = normal(seed, ("k_cache", kv_len), (1, shape.num_kv_heads, cap, shape.head_dim))
    vc = normal(seed, ("v_cache", kv_len), (1, shape.num_kv_heads, cap, shape.head_dim))
    if cap > kv_len:
        fill = 60000.0 if stale_fill is None else stale_fill
        kc[:, :, kv_len:] = fill
        vc[:, :, kv_len:] = fill
    return q, kc, vc, kv_len - 1


@dataclass
class MultimodalPrompt:
    """Config 3 prompt: 768 vision rows on a 1x24x32 grid, then 256 text ids."""

    vision_embeds: torch.Tensor   # [768, H] fp16 ~ N(0,1)
    text_ids: torch.Tensor        # [256] int64, uniform in [0, V)
    position_ids: torch.Tensor    # [3, 1024] int64 (T, H, W streams)
    rope_delta: int               # max position + 1 - prompt length

    @property
    def length(self) -> int:
        return self.vision_embeds.shape[0] + self.text_ids.shape[0]


def multimodal_prompt(seed: int = 3, grid_t: int = 1, grid_h: int = 24, grid_w: int = 32,
                      n_text: int = 256, shape: Qwen3VLTextShape = QWEN3VL_2B) -> MultimodalPrompt:
    """Positions follow HF Qwen3-VL `get_rope_index` / `get_vision_position_ids`
    (transformers 5.15 modeling_qwen3_vl.py:880-1023) for one image whose LLM
    grid (after the 2x2 spatial merge) is grid_t x grid_h x grid_w, followed by
    text: vision T = t, H = h, W = w (start 0); text continues at
    max(grid_h, grid_w) on all three streams."""
    n_vis = grid_t * grid_h * grid_w
    vis = normal(seed, ("vision_embeds",), (n_vis, shape.hidden))
    ids = randint(seed, ("text_ids",), (n_text,), 0, shape.vocab)
    tt, hh, ww = torch.meshgrid(torch.arange(grid_t), torch.arange(grid_h), torch.arange(grid_w), indexing="ij")
    vis_pos = torch.stack([tt, hh, ww]).reshape(3, -1)
    start = max(grid_h, grid_w)
    text_pos = (torch.arange(n_text) + start).view(1, -1).expand(3, -1)
    pos = torch.cat([vis_pos, text_pos], 1).to(torch.int64)
    delta = int(pos.max()) + 1 - (n_vis + n_text)
    return MultimodalPrompt(vis, ids, pos, delta)


def batch8_kv_lengths(seed: int = 4, batch: int = 8, low: int = 2048, high: int = 4096) -> torch.Tensor:
    """Config 4: per-sequence valid KV lengths ~ U[low, high]."""
    return randint(seed, ("kv_len",), (batch,), low, high + 1)
