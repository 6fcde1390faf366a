"""Qwen3-VL-2B text-decoder shape constants used by the decode path.

The values are those of the Qwen3-VL-2B-Instruct text config that the reference
decode path is specialised for (hidden 2048, 16 q heads / 8 kv heads, head_dim
128, SwiGLU 6144, 28 layers, tied vocab 151936, eps 1e-6, interleaved M-RoPE with
theta 5e6 and sections [24, 20, 20]).  The reference hard-codes the same numbers
in its kernels and dispatch guards, e.g. `optimized_layer.py:1650-1654`
(2048 / 12288x2048 / 2048x6144) and `cuda_decode_small_ops.py:98-103` (head_dim
128, q_heads == 2 * kv_heads).
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class Qwen3VLTextShape:
    hidden: int = 2048
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    num_layers: int = 28
    vocab: int = 151936
    rms_eps: float = 1e-6
    rope_theta: float = 5_000_000.0
    mrope_section: tuple = field(default=(24, 20, 20))

    @property
    def q_size(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def qkv_rows(self) -> int:
        return self.q_size + 2 * self.kv_size

    @property
    def groups(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def scaling(self) -> float:
        return self.head_dim ** -0.5

    def layer_weight_bytes(self) -> int:
        """fp16 bytes of one layer's weights (7 projections + 4 norm vectors)."""
        h, i, d = self.hidden, self.intermediate, self.head_dim
        proj = self.qkv_rows * h + h * self.q_size + 2 * i * h + h * i
        norms = 2 * h + 2 * d
        return 2 * (proj + norms)


QWEN3VL_2B = Qwen3VLTextShape()
