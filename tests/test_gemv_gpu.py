"""GEMV family parity on the GPU (config 1) against the CPU oracle in fp32.

Bar: max |gpu - oracle| <= 2e-3 * max |oracle| for every fp16 output.
"""

from __future__ import annotations

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu

SHAPES = ["qkv", "o_proj", "gate_up", "down_proj", "lm_head"]


def _inputs(name):
    from qwen3vl_hip import synthetic as syn

    return syn.gemv_inputs(name)


@pytest.mark.parametrize("name", SHAPES)
def test_nosplit_matvec_config1(cuda, name):
    import cuda_decode_gemv as g

    x, w = _inputs(name)
    print(f"case nosplit {name} N={w.shape[0]} K={w.shape[1]}", flush=True)
    y = g.nosplit_matvec_half(x.to(cuda), w.to(cuda), None)
    assert y.shape == (1, 1, w.shape[0]) and y.dtype == torch.float16
    assert_close_rel(y.reshape(-1), O.gemv(x.reshape(-1), w), what=f"nosplit {name}")


@pytest.mark.parametrize("name,split_k", [("qkv", 2), ("qkv", 4), ("lm_head", 2), ("lm_head", 4), ("down_proj", 2),
                                          ("down_proj", 3), ("o_proj", 1)])
def test_splitk_matvec(cuda, name, split_k):
    import cuda_decode_gemv as g

    x, w = _inputs(name)
    print(f"case splitk {name} split_k={split_k}", flush=True)
    b = torch.randn(w.shape[0], generator=torch.Generator().manual_seed(7)).half()
    y = g.splitk_matvec(x.to(cuda), w.to(cuda), b.to(cuda), split_k)
    assert_close_rel(y.reshape(-1), O.gemv(x.reshape(-1), w, b), what=f"splitk {name}/{split_k}")


def test_splitk_independent_of_split_count(cuda):
    import cuda_decode_gemv as g

    x, w = _inputs("qkv")
    xs, ws = x.to(cuda), w.to(cuda)
    ys = [g.splitk_matvec(xs, ws, None, s).float().cpu() for s in (1, 2, 4)]
    ref = O.gemv(x.reshape(-1), w)
    for y in ys:
        assert_close_rel(y.reshape(-1), ref, what="splitk count invariance")
    # every split count stays within fp16 rounding of the others
    assert (ys[0] - ys[2]).abs().max().item() <= 2e-3 * ref.abs().max().item()


@pytest.mark.parametrize("n,k", [(2049, 2048), (4097, 2048), (7, 6144), (300, 1000), (33, 8)])
def test_matvec_ragged_shapes(cuda, n, k):
    """Row counts that are not multiples of the rows per wave, and K outside the
    register-resident set (generic kernel)."""
    import cuda_decode_gemv as g

    gen = torch.Generator().manual_seed(n * 31 + k)
    x = torch.randn(1, 1, k, generator=gen).half()
    w = (torch.randn(n, k, generator=gen) * 0.02).half()
    b = torch.randn(n, generator=gen).half()
    print(f"case ragged n={n} k={k}", flush=True)
    y = g.nosplit_matvec_half(x.to(cuda), w.to(cuda), b.to(cuda))
    assert_close_rel(y.reshape(-1), O.gemv(x.reshape(-1), w, b), what=f"ragged {n}x{k}")


def test_matvec_one_hot_selects_column(cuda):
    import cuda_decode_gemv as g

    _, w = _inputs("o_proj")
    x = torch.zeros(1, 1, 2048, dtype=torch.float16)
    x[0, 0, 1234] = 1.0
    y = g.nosplit_matvec_half(x.to(cuda), w.to(cuda), None).reshape(-1).cpu()
    assert torch.equal(y, w[:, 1234])


def test_fused_rmsnorm_qkv(cuda):
    import cuda_decode_gemv as g
    from qwen3vl_hip import synthetic as syn

    lw = syn.layer_weights(0, 0)
    x = syn.normal(0, ("x",), (1, 1, 2048))
    y = g.fused_rmsnorm_qkv_half(x.to(cuda), lw.input_layernorm_weight.to(cuda), lw.qkv_weight.to(cuda), None, 1e-6)
    ref = O.gemv(O.rms_norm(x.reshape(-1), lw.input_layernorm_weight, 1e-6), lw.qkv_weight)
    assert_close_rel(y.reshape(-1), ref, what="fused_rmsnorm_qkv")


def test_fused_post_attn_mlp(cuda):
    import cuda_decode_gemv as g
    from qwen3vl_hip import synthetic as syn

    lw = syn.layer_weights(0, 0)
    res = syn.normal(0, ("residual",), (1, 1, 2048))
    att = syn.normal(0, ("attn",), (1, 1, 2048))
    for fn in (g.fused_post_attn_mlp_softsync_half, g.fused_post_attn_mlp_persistent_half):
        hid, out = fn(res.to(cuda), att.to(cuda), lw.post_attn_layernorm_weight.to(cuda),
                      lw.gate_up_weight.to(cuda), lw.down_proj_weight.to(cuda), None, 1e-6)
        rh, ro, _ = O.post_attn_mlp(res.reshape(-1), att.reshape(-1), lw.post_attn_layernorm_weight,
                                    lw.gate_up_weight, lw.down_proj_weight, None, 1e-6)
        assert hid.shape == (1, 1, 6144) and out.shape == (1, 1, 2048)
        assert_close_rel(hid.reshape(-1), rh, what=f"{fn.__name__} hidden")
        assert_close_rel(out.reshape(-1), ro, what=f"{fn.__name__} out")


def test_post_attn_mlp_advances_the_running_length(cuda):
    """qd_post_attn_mlp_next_f16: the same outputs as qd_post_attn_mlp_f16
    (bit for bit) plus length = position + 1, also when both are one word (the
    StaticLayer's cumulative_length read and advanced in place)."""
    from cuda_decode_gemv_ops import fused
    from qwen3vl_hip import synthetic as syn

    lw = syn.layer_weights(0, 0)
    args = (syn.normal(0, ("residual",), (1, 1, 2048)).to(cuda), syn.normal(0, ("attn",), (1, 1, 2048)).to(cuda),
            lw.post_attn_layernorm_weight.to(cuda), lw.gate_up_weight.to(cuda), lw.down_proj_weight.to(cuda), None,
            1e-6)
    hid0, out0 = fused._post_attn_mlp("post_attn_mlp", *args, None, "plain")
    pos = torch.tensor([777], dtype=torch.int64, device=cuda)
    length = torch.tensor(-5, dtype=torch.int64, device=cuda)
    hid1, out1 = fused._post_attn_mlp("post_attn_mlp", *args, None, "next", next_position=(pos, length))
    assert torch.equal(hid0, hid1) and torch.equal(out0, out1)
    assert int(length) == 778 and int(pos) == 777
    _, out2 = fused._post_attn_mlp("post_attn_mlp", *args, None, "same", next_position=(length, length))
    assert torch.equal(out0, out2) and int(length) == 779


def test_post_attn_mlp_advance_at_an_unspecialised_intermediate_size(cuda):
    """I = 1536 has no fixed-K kernel for down_proj (the generic GEMV runs it):
    the running-length advance must still happen, and the outputs must still
    match the oracle."""
    from cuda_decode_gemv_ops import fused

    g = torch.Generator().manual_seed(11)
    H, I = 2048, 1536
    res = torch.randn(1, 1, H, generator=g).half()
    att = torch.randn(1, 1, H, generator=g).half()
    gamma = (1 + 0.02 * torch.randn(H, generator=g)).half()
    w_gu = (0.02 * torch.randn(2 * I, H, generator=g)).half()
    w_d = (0.02 * torch.randn(H, I, generator=g)).half()
    pos = torch.tensor([41], dtype=torch.int64, device=cuda)
    length = torch.tensor(0, dtype=torch.int64, device=cuda)
    hid, out = fused._post_attn_mlp("post_attn_mlp", res.to(cuda), att.to(cuda), gamma.to(cuda), w_gu.to(cuda),
                                    w_d.to(cuda), None, 1e-6, None, "next", next_position=(pos, length))
    torch.cuda.synchronize()
    assert int(length) == 42 and int(pos) == 41
    rh, ro, _ = O.post_attn_mlp(res.reshape(-1), att.reshape(-1), gamma, w_gu, w_d, None, 1e-6)
    assert_close_rel(hid.reshape(-1), rh, what="I=1536 hidden")
    assert_close_rel(out.reshape(-1), ro, what="I=1536 out")


def test_fused_post_attn_mlp_bias_and_workspace_reuse(cuda):
    import cuda_decode_gemv as g
    from qwen3vl_hip import synthetic as syn

    lw = syn.layer_weights(0, 0)
    res = syn.normal(0, ("residual",), (1, 1, 2048))
    att = syn.normal(0, ("attn",), (1, 1, 2048))
    bias = syn.normal(5, ("x",), (2048,))
    ws = {"type": "fused_post_attn_mlp_softsync"}
    args = (res.to(cuda), att.to(cuda), lw.post_attn_layernorm_weight.to(cuda), lw.gate_up_weight.to(cuda),
            lw.down_proj_weight.to(cuda), bias.to(cuda), 1e-6)
    _, out1 = g.fused_post_attn_mlp_softsync_half(*args, workspace=ws)
    ws["hidden_out"], ws["out"] = torch.empty(6144, dtype=torch.float16, device=cuda), out1.reshape(-1).clone()
    _, out2 = g.fused_post_attn_mlp_softsync_half(*args, workspace=ws)
    assert out2.data_ptr() == ws["out"].data_ptr()
    _, ro, _ = O.post_attn_mlp(res.reshape(-1), att.reshape(-1), lw.post_attn_layernorm_weight, lw.gate_up_weight,
                               lw.down_proj_weight, bias, 1e-6)
    assert_close_rel(out2.reshape(-1), ro, what="post_attn_mlp + bias")


def test_fused_add_rmsnorm_gateup_and_silu_down(cuda):
    import cuda_decode_gemv as g
    from qwen3vl_hip import synthetic as syn

    lw = syn.layer_weights(0, 0)
    res = syn.normal(0, ("residual",), (1, 1, 2048))
    att = syn.normal(0, ("attn",), (1, 1, 2048))
    r_out, gu = g.fused_add_rmsnorm_gateup_half(res.to(cuda), att.to(cuda), lw.post_attn_layernorm_weight.to(cuda),
                                                lw.gate_up_weight.to(cuda), None, 1e-6)
    r = res.float() + att.float()
    assert_close_rel(r_out.reshape(-1), r.reshape(-1), what="add_rmsnorm_gateup residual")
    ref_gu = O.gemv(O.rms_norm(r.reshape(-1), lw.post_attn_layernorm_weight, 1e-6), lw.gate_up_weight)
    assert_close_rel(gu.reshape(-1), ref_gu, what="add_rmsnorm_gateup")
    down = g.fused_silu_downproj_half(gu, lw.down_proj_weight.to(cuda), None)
    ref_down = O.gemv(O.silu_mul(gu.reshape(-1)[:6144].cpu(), gu.reshape(-1)[6144:].cpu()), lw.down_proj_weight)
    assert_close_rel(down.reshape(-1), ref_down, what="silu_downproj")
    hid, out = g.fused_gateup_silu_downproj_half(att.to(cuda), lw.gate_up_weight.to(cuda),
                                                 lw.down_proj_weight.to(cuda), None)
    gu2 = O.gemv(att.reshape(-1), lw.gate_up_weight)
    h2 = O.silu_mul(gu2[:6144], gu2[6144:])
    assert_close_rel(hid.reshape(-1), h2, what="gateup_silu_downproj hidden")
    assert_close_rel(out.reshape(-1), O.gemv(h2, lw.down_proj_weight), what="gateup_silu_downproj out")


def test_lm_head_argmax_config1(cuda):
    from qwen3vl_hip import _lib

    x, w = _inputs("lm_head")
    g = torch.ones(2048, dtype=torch.float16) + 0.02 * torch.randn(2048, generator=torch.Generator().manual_seed(3)).half()
    xs, ws_, gs = x.reshape(-1).to(cuda), w.to(cuda), g.to(cuda)
    logits = torch.empty(w.shape[0], dtype=torch.float16, device=cuda)
    tok = torch.empty(1, dtype=torch.int64, device=cuda)
    lib = _lib.lib()
    wsp = torch.zeros(int(lib.qd_lm_head_workspace_bytes(w.shape[0])), dtype=torch.uint8, device=cuda)
    for _ in range(3):  # the arrival counter must self-reset between launches
        tok.fill_(-1)   # a launch whose last block never reduces would leave this
        _lib.check(lib.qd_lm_head_argmax(_lib.ptr(xs), _lib.QD_F16, _lib.ptr(gs), 1e-6, _lib.ptr(ws_), w.shape[0],
                                         2048, _lib.ptr(logits), _lib.ptr(tok), _lib.ptr(wsp), _lib.stream()),
                   "lm_head")
        torch.cuda.synchronize()
        ref_logits, ref_tok = O.lm_head_argmax(x.reshape(-1), g, w, 1e-6)
        assert_close_rel(logits, ref_logits, what="lm_head logits")
        print(f"lm_head margin {O.top2_margin(ref_logits):.4g}", flush=True)
        assert int(tok.item()) == ref_tok


def test_lm_head_argmax_tie_takes_first_index(cuda):
    """torch.argmax semantics: with duplicated maximal rows the lowest index wins."""
    from qwen3vl_hip import _lib

    V, H = 50000, 2048
    gen = torch.Generator().manual_seed(11)
    w = (torch.randn(V, H, generator=gen) * 0.02).half()
    x = w[31337].float() / w[31337].float().norm()
    for j in (40000, 45001, 49999, 31338):
        w[j] = w[31337]
    xs, wd = x.half().to(cuda), w.to(cuda)   # device copies stay referenced across the launch
    tok = torch.empty(1, dtype=torch.int64, device=cuda)
    lib = _lib.lib()
    wsp = torch.zeros(int(lib.qd_lm_head_workspace_bytes(V)), dtype=torch.uint8, device=cuda)
    _lib.check(lib.qd_lm_head_argmax(_lib.ptr(xs), _lib.QD_F16, None, 1e-6, _lib.ptr(wd), V, H, None,
                                     _lib.ptr(tok), _lib.ptr(wsp), _lib.stream()), "lm_head")
    assert int(tok.item()) == 31337
    assert int(torch.argmax(x.half().float() @ w.float().T)) == 31337


def test_bad_inputs_raise(cuda):
    import cuda_decode_gemv as g

    x = torch.randn(1, 1, 2048, device=cuda)  # fp32: rejected like the reference
    w = torch.randn(64, 2048, device=cuda).half()
    with pytest.raises(RuntimeError):
        g.nosplit_matvec_half(x, w, None)
    with pytest.raises(RuntimeError):
        g.nosplit_matvec_half(torch.randn(1, 2, 2048, device=cuda).half(), w, None)
    with pytest.raises(RuntimeError):
        g.splitk_matvec(x.half(), w, None, 3)  # 2048 / 3 is not an integer slice


@pytest.mark.parametrize("f16", [False, True])
def test_lm_head_argmax_logits_within_one_fp16_ulp(cuda, f16):
    """Two logits that differ by less than one fp16 ulp, the larger fp32 value
    at the higher index.  Default (fp32 comparison, the oracle's argmax): the
    higher index.  argmax_f16_logits (the reference's FastLmHead returns fp16
    logits and takes torch.argmax, evaluation_wrapper.py:952, :1233-1238): the
    two round to the same fp16 value and the first index wins.  The fp16 logits
    written out are equal either way."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.config import Qwen3VLTextShape
    from qwen3vl_hip.engine import DecodeEngine

    w = syn.model_weights(26, shape=Qwen3VLTextShape(num_layers=1, vocab=4096))
    emb = torch.zeros(4096, 2048, dtype=torch.float16)
    emb[3, 0] = 1.0
    emb[7, 0] = 1.0
    emb[7, 1] = 2.0 ** -12          # logit 7 = logit 3 * (1 + 2^-12): below half an fp16 ulp at 1.0
    w.embed_tokens = emb
    w.final_norm_weight = torch.ones(2048, dtype=torch.float16)
    eng = DecodeEngine(w, capacity=64, step_mode="chain", keep_logits=True, argmax_f16_logits=f16)
    eng.buffers()["x"].fill_(1.0)
    eng.run_phases(["lm_head"], n_layers=0)
    torch.cuda.synchronize()
    tok = int(eng.token.item())
    assert eng.logits[3].item() == eng.logits[7].item() == 1.0
    _, tok_oracle = O.lm_head_argmax(torch.ones(2048), w.final_norm_weight, emb, 1e-6)
    assert tok_oracle == 7
    assert tok == (3 if f16 else 7)
    # the same through torch's own argmax over the fp16 logits (reference semantics)
    assert int(torch.argmax(eng.logits)) == 3
