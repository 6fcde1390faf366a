"""CPU checks of the drop-in boundary: the C-ABI library loads and exports every
declared entry point, the Python surface matches the reference's names, and
the product path refuses CPU tensors instead of falling back."""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "qwen3vl_decode.h"


def _declared() -> set:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(qd_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    from qwen3vl_hip import _lib

    handle = _lib.lib()
    declared = _declared()
    assert declared, "no declarations parsed"
    missing = sorted(n for n in declared if not hasattr(handle, n))
    assert not missing, f"declared but not exported: {missing}"
    assert set(_lib.EXPORTED) == declared, "ctypes signature table out of sync with the header"


def test_library_host_only_calls():
    from qwen3vl_hip import _lib

    lib = _lib.lib()
    assert lib.qd_version() >= 1
    assert lib.qd_attention_default_splits(256) == 4
    assert lib.qd_attention_default_splits(1024) == 8
    assert lib.qd_attention_default_splits(2048) == 16
    assert lib.qd_attention_default_splits(3072) == 24
    assert lib.qd_attention_default_splits(4096) == 32
    assert lib.qd_attention_default_splits(8192) == 32
    assert lib.qd_attention_default_splits(1 << 20) == 32
    assert lib.qd_attention_workspace_bytes(16, 8, 4) >= 16 * 4 * 128 * 4
    assert lib.qd_lm_head_workspace_bytes(151936) > 0
    # argument errors are reported without touching a device
    assert lib.qd_matvec_f16(None, None, None, None, 8, 8, None) == -1
    assert b"null" in lib.qd_last_error()
    assert lib.qd_attention_merge(None, None, None, 0, 16, 4, None) == -1
    assert lib.qd_decoder_layer_persistent_f16(None, None, 64, None, None, None, 1e-6, 0.088, None, None, None,
                                               None) == -1
    # the persistent launches' polling budget is host state only
    assert lib.qd_persistent_set_spin_limit(0) == 0


def test_one_launch_layer_rejects_misaligned_pointers():
    """qd_decoder_layer_persistent_f16 reads weights, norms and caches as 16-byte
    vectors and the input as 8-byte slices: misaligned addresses are an
    argument error reported before any device work (the addresses below are
    never dereferenced)."""
    import ctypes

    from qwen3vl_hip import _lib

    lib = _lib.lib()
    good = dict(qkv=0x10000, o_proj=0x20000, gate_up=0x30000, down=0x40000, input_norm=0x50000,
                post_norm=0x50400, q_norm=0x50800, k_norm=0x50900, k_cache=0x60000, v_cache=0x70000)

    def call(hidden_in=0x80000, pos=0x90000, length=0x90010, **over):
        w = _lib.LayerDesc(**{**good, **over})
        return lib.qd_decoder_layer_persistent_f16(
            ctypes.c_void_p(hidden_in), ctypes.byref(w), 64, ctypes.c_void_p(pos), ctypes.c_void_p(0xa0000),
            ctypes.c_void_p(0xa0100), 1e-6, 0.088, ctypes.c_void_p(0xb0000), ctypes.c_void_p(length),
            ctypes.c_void_p(0xc0000), None)

    for over in (dict(qkv=0x10008), dict(gate_up=0x30002), dict(input_norm=0x50004), dict(v_cache=0x70008),
                 dict(hidden_in=0x80004), dict(pos=0x90004), dict(length=0x90014)):
        assert call(**over) == -1, over
        assert b"aligned" in lib.qd_last_error(), over


def test_gemv_facade_exports_reference_names():
    import cuda_decode_gemv

    expected = {
        "nosplit_matvec_half", "splitk_matvec", "fused_rmsnorm_qkv_half", "fused_post_attn_mlp_softsync_half",
        "fused_post_attn_mlp_persistent_half", "fused_gateup_silu_downproj_persistent_half",
        "fused_add_rmsnorm_gateup_half", "fused_silu_downproj_half", "fused_decode_full_layer_softsync_half",
        "decode_attn_persistent_half", "NOSPLIT_VARIANTS", "nosplit_matvec_half_profile",
    }
    assert expected <= set(cuda_decode_gemv.__all__)
    assert len(cuda_decode_gemv.__all__) == 54   # the reference's 45 functions + 9 constants
    for name in cuda_decode_gemv.__all__:
        assert hasattr(cuda_decode_gemv, name), name


def test_attention_and_small_ops_names():
    import cuda_decode_attention as A
    import cuda_decode_small_ops as S

    for n in ("decode_attn_v4_cta_qhead_splitkv_fused", "decode_attn_v4_fused", "decode_attn_v4_splitkv",
              "decode_attn_v4_cta_qhead", "decode_attn_v4_cta_local"):
        assert callable(getattr(A, n))
    for n in ("fused_q_rope_kv_cache_update", "fused_qk_rms_norm_rope", "fused_add_rms_norm", "rms_norm",
              "fused_silu_mul", "add"):
        assert callable(getattr(S, n))


def test_cpu_tensors_are_rejected():
    import cuda_decode_attention as A
    import cuda_decode_gemv as G
    import cuda_decode_small_ops as S

    x = torch.randn(1, 1, 2048).half()
    w = torch.randn(64, 2048).half()
    with pytest.raises(RuntimeError):
        G.nosplit_matvec_half(x, w, None)
    with pytest.raises(RuntimeError):
        G.fused_rmsnorm_qkv_half(x, torch.ones(2048).half(), w, None, 1e-6)
    with pytest.raises(RuntimeError):
        S.add(x, x)
    q = torch.randn(1, 16, 1, 128).half()
    kc = torch.randn(1, 8, 64, 128).half()
    assert A.decode_attn_v4_fused(q, kc, kc, 0.088, 2, torch.tensor([5])) is None


def test_optimized_layer_refuses_cpu():
    import optimized_layer
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextDecoderLayer

    cfg = Qwen3VLTextConfig(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=2,
                            head_dim=64, num_hidden_layers=1, vocab_size=97)
    layer = optimized_layer.OptimizedDecoderLayer(Qwen3VLTextDecoderLayer(cfg, 0))
    assert layer.qkv_weight.shape == (4 * 64 + 2 * 2 * 64, 256)
    assert layer.gate_up_weight.shape == (1024, 256)
    with pytest.raises(RuntimeError):
        layer(torch.randn(1, 1, 256), (torch.ones(1, 1, 64), torch.zeros(1, 1, 64)))
    prev = optimized_layer.set_cuda_mlp_fusion_flags(post_attn_mlp_persistent=False)
    assert len(prev) == 8
    assert optimized_layer.set_cuda_mlp_fusion_flags(post_attn_mlp_persistent=prev[2])[2] is False


def test_engine_needs_gpu():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.config import Qwen3VLTextShape
    from qwen3vl_hip.engine import DecodeEngine

    shape = Qwen3VLTextShape(hidden=512, intermediate=512, num_layers=1, vocab=64)
    w = syn.model_weights(0, shape)
    with pytest.raises(RuntimeError):
        DecodeEngine(w, capacity=8)


def test_synthetic_streams_are_keyed_and_deterministic():
    from qwen3vl_hip import synthetic as syn

    a = syn.normal(3, ("x", 1), (1000,))
    b = syn.normal(3, ("x", 1), (1000,))
    c = syn.normal(3, ("x", 2), (1000,))
    assert torch.equal(a, b) and not torch.equal(a, c)
    lw = syn.layer_weights(0, 0)
    assert lw.qkv_weight.shape == (4096, 2048) and lw.gate_up_weight.shape == (12288, 2048)
    assert lw.down_proj_weight.shape == (2048, 6144) and lw.qkv_weight.dtype == torch.float16
    assert abs(float(lw.qkv_weight.float().std()) - 0.02) < 1e-3
    assert abs(float(lw.input_layernorm_weight.float().mean()) - 1.0) < 5e-3


def test_multimodal_prompt_positions_and_delta():
    """Positions of HF get_rope_index for one 1x24x32 image then 256 text tokens."""
    from qwen3vl_hip import synthetic as syn

    p = syn.multimodal_prompt(3)
    assert p.length == 1024 and p.rope_delta == 288 - 1024
    pos = p.position_ids
    assert pos.shape == (3, 1024)
    assert pos[0, :768].eq(0).all()
    assert pos[1, :768].view(24, 32)[:, 0].tolist() == list(range(24))
    assert pos[2, :768].view(24, 32)[0].tolist() == list(range(32))
    assert pos[:, 768:].eq(torch.arange(32, 288)).all()


def test_roofline_bytes_match_the_stated_figures():
    from oracle import qwen3vl_oracle as O
    from qwen3vl_hip.config import QWEN3VL_2B
    from qwen3vl_hip.engine import roofline_bytes_step

    assert QWEN3VL_2B.layer_weight_bytes() == 100_672_000
    assert roofline_bytes_step(0) == 3_441_154_048
    assert roofline_bytes_step(4096) == 3_910_916_096
    assert roofline_bytes_step(4096) == O.roofline_bytes_step(4096)


def test_bench_refuses_more_than_one_gpu():
    """The bench measures one GPU; asking for more exits with status 2 and a
    message, before anything touches a device."""
    import subprocess
    import sys

    repo = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(repo / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_bench_batch8_and_config_bytes_are_consistent():
    """The batch-8 step bytes and the one-layer bytes bench.py reports follow
    the same per-weight / per-K/V-row accounting as the batch-1 step."""
    import dataclasses

    import bench
    from qwen3vl_hip.config import QWEN3VL_2B
    from qwen3vl_hip.engine import roofline_bytes_batch_step, roofline_bytes_step

    one = dataclasses.replace(QWEN3VL_2B, num_layers=1)
    # one layer at cache position 512: weights + norms, K/V rows 0..512, embedding row + fp32 hidden
    assert bench.persistent_launch_bytes(513, one) == 100_672_000 + 4096 * 513 + 2 * 2048 + 4 * 2048
    # a batch of one sequence reads what the batch-1 step reads
    assert roofline_bytes_batch_step([4096]) == roofline_bytes_step(4096)


def test_fusion_flags_follow_the_reference_environment():
    """The reference reads ENABLE_CUDA_FUSED_* at import
    (optimized_layer.py:837-921): an explicitly set variable selects the path,
    an unset one keeps this build's default (one-launch layer on)."""
    import os
    import subprocess
    import sys

    code = ("import optimized_layer as m; print(m.set_cuda_mlp_fusion_flags()[1], m.set_cuda_mlp_fusion_flags()[0])")
    env = {k: v for k, v in os.environ.items() if not k.startswith("ENABLE_CUDA_FUSED_")}
    env["PYTHONPATH"] = str(REPO / "aicasgc-2026_amd")
    out = {}
    for val in (None, "0", "1"):
        e = dict(env)
        if val is not None:
            e["ENABLE_CUDA_FUSED_FULL_LAYER_SOFTSYNC"] = val
            e["ENABLE_CUDA_FUSED_ADD_RMSNORM_GATEUP"] = val
        res = subprocess.run([sys.executable, "-c", code], env=e, capture_output=True, text=True, timeout=300)
        assert res.returncode == 0, res.stderr
        out[val] = res.stdout.split()
    assert out[None] == ["True", "False"]
    assert out["0"] == ["False", "False"]
    assert out["1"] == ["True", "True"]


def test_batch_tile_order_layout():
    """The batch GEMVs' tile order (qd_model_desc.batch_tiled_weights): the
    library's row-group sizes for the 2B shapes, and the positions the header
    states for both layouts, checked element by element on small matrices."""
    import torch

    from qwen3vl_hip import _lib
    from qwen3vl_hip.engine import batch_tile_order

    lib = _lib.lib()
    assert lib.qd_batch_tile_rows(4096, 2048, 0) == 16     # qkv
    assert lib.qd_batch_tile_rows(2048, 2048, 0) == 8      # o_proj
    assert lib.qd_batch_tile_rows(6144, 2048, 1) == 8      # gate_up
    assert lib.qd_batch_tile_rows(2048, 6144, 0) == 16     # down
    assert lib.qd_batch_tile_rows(0, 2048, 0) == 0
    rows, K = 32, 256
    w = torch.arange(rows * K, dtype=torch.float32).reshape(rows, K)
    t16 = batch_tile_order(w, 16).reshape(-1)
    t8 = batch_tile_order(w, 8).reshape(-1)
    for r in range(rows):
        for k in range(K):
            o16 = ((r // 16) * (K // 8) + k // 8) * 128 + (r % 16) * 8 + k % 8
            o8 = ((r // 8) * (K // 64) + k // 64) * 512 + ((k % 64) // 8 % 4) * 128 + ((k % 64) // 32) * 64 \
                + (r % 8) * 8 + k % 8
            assert t16[o16] == w[r, k] and t8[o8] == w[r, k]
