"""The reference's variant and alias entry points of the GEMV family on the GPU.

The reference keeps several kernels per operation (A800 tuning variants:
row4 / row8 split-K GEMVs, hfma2 and persistent matvecs, softsync / gridsync /
mega gate_up-SiLU-down, persistent / softsync o_proj + MLP).  On MI355X each
name runs the one gfx950 kernel of its operation; these tests call every name
with the reference's signature and check the result against the oracle, so a
caller that picks any of them gets the operation's value.
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu


def _mlp_weights(seed: int):
    from qwen3vl_hip import synthetic as syn

    inp = syn.layer_step_inputs(seed=seed, cache_position=4, capacity=8)
    return inp.weights, inp.hidden


@pytest.mark.parametrize("name", ["nosplit_hfma2_matvec_half", "persistent_matvec_half"])
def test_matvec_aliases(cuda, name):
    import cuda_decode_gemv
    from qwen3vl_hip import synthetic as syn

    x, w = syn.gemv_inputs("o_proj")
    b = syn.normal(1, ("o_proj", 7), (2048,), std=0.1)
    print(f"case {name}", flush=True)
    y = getattr(cuda_decode_gemv, name)(x.to(cuda), w.to(cuda), b.to(cuda))
    assert y.shape == (1, 1, 2048) and y.dtype == torch.float16
    assert_close_rel(y.reshape(-1), O.gemv(x.reshape(-1), w, b), what=name)


def test_matvec_variant_dispatcher(cuda):
    import cuda_decode_gemv
    from cuda_decode_gemv_ops.runtime import NOSPLIT_VARIANTS
    from qwen3vl_hip import synthetic as syn

    x, w = syn.gemv_inputs("down_proj")
    ref = O.gemv(x.reshape(-1), w)
    for variant in (NOSPLIT_VARIANTS[0], NOSPLIT_VARIANTS[-1]):
        print(f"case nosplit variant {variant}", flush=True)
        y = cuda_decode_gemv.nosplit_matvec_half_variant(x.to(cuda), w.to(cuda), None, variant)
        assert_close_rel(y.reshape(-1), ref, what=f"nosplit_matvec_half_variant {variant}")
    with pytest.raises(RuntimeError, match="unknown nosplit variant"):
        cuda_decode_gemv.nosplit_matvec_half_variant(x.to(cuda), w.to(cuda), None, "no_such_variant")


@pytest.mark.parametrize("name", ["splitk_matvec_row4", "splitk_matvec_row8_shared",
                                  "splitk_matvec_row4_shared_vec_half", "splitk_matvec_row4_shared_vec_half_v2"])
def test_splitk_aliases(cuda, name):
    import cuda_decode_gemv
    from qwen3vl_hip import synthetic as syn

    x, w = syn.gemv_inputs("qkv")
    print(f"case {name}", flush=True)
    y = getattr(cuda_decode_gemv, name)(x.to(cuda), w.to(cuda), None, 4)
    assert y.shape[-1] == 4096
    assert_close_rel(y.reshape(-1), O.gemv(x.reshape(-1), w), what=name)


@pytest.mark.parametrize("name", ["fused_gateup_silu_downproj_softsync_half", "fused_gateup_silu_downproj_gridsync_half",
                                  "fused_gateup_silu_downproj_mega_half",
                                  "fused_gateup_silu_downproj_mega_partial_half"])
def test_gateup_silu_down_variants(cuda, name):
    import cuda_decode_gemv

    lw, x = _mlp_weights(12)
    print(f"case {name}", flush=True)
    hidden, out = getattr(cuda_decode_gemv, name)(x.to(cuda), lw.gate_up_weight.to(cuda),
                                                  lw.down_proj_weight.to(cuda))
    gu = O.gemv(x.reshape(-1), lw.gate_up_weight)
    h_ref = O.silu_mul(gu[:6144], gu[6144:])
    assert hidden.shape == (1, 1, 6144) and out.shape == (1, 1, 2048)
    assert_close_rel(hidden.reshape(-1), h_ref, what=f"{name}: hidden")
    assert_close_rel(out.reshape(-1), O.gemv(h_ref, lw.down_proj_weight), what=f"{name}: out")


@pytest.mark.parametrize("name", ["fused_o_proj_post_attn_mlp_persistent_half",
                                  "fused_o_proj_post_attn_mlp_softsync_half"])
def test_o_proj_post_attn_mlp_variants(cuda, name):
    import cuda_decode_gemv
    from qwen3vl_hip import synthetic as syn

    lw, residual = _mlp_weights(13)
    attn = syn.normal(13, ("attn", 2), (1, 1, 2048))
    print(f"case {name}", flush=True)
    hidden, out = getattr(cuda_decode_gemv, name)(
        residual.to(cuda), attn.to(cuda), lw.o_proj_weight.to(cuda), None, lw.post_attn_layernorm_weight.to(cuda),
        lw.gate_up_weight.to(cuda), lw.down_proj_weight.to(cuda), None, 1e-6)
    o = O.gemv(attn.reshape(-1), lw.o_proj_weight)
    h_ref, o_ref, _ = O.post_attn_mlp(residual.reshape(-1), o, lw.post_attn_layernorm_weight, lw.gate_up_weight,
                                      lw.down_proj_weight, None, 1e-6)
    assert_close_rel(hidden.reshape(-1), h_ref, what=f"{name}: hidden")
    assert_close_rel(out.reshape(-1), o_ref, what=f"{name}: out")
