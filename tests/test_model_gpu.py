"""Greedy decoding of the full model on the GPU (config 3) against the oracle.

* a 2-layer model with the real vocabulary and a small multimodal prompt,
  checked against the oracle run live on the CPU (prefill K/V, tokens, and
  graph replay == eager);
* the full 28-layer model with the 1024-position prompt: the first 64 greedy
  tokens must equal the oracle's tokens in tests/golden/config3_tokens.json.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "config3_tokens.json"


@pytest.mark.parametrize("step_mode", ["chain", "persistent"])
def test_two_layer_model_greedy_matches_oracle(cuda, step_mode):
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import DecodeEngine

    w = syn.model_weights(21, num_layers=2)
    prompt = syn.multimodal_prompt(21, grid_h=4, grid_w=8, n_text=16)
    n = 24
    cap = prompt.length + n + 8
    eng = DecodeEngine(w, capacity=cap, step_mode=step_mode)
    toks = eng.generate(prompt, n, use_graph=True)
    # prefill K/V against the oracle's prefill
    caches = [(torch.zeros(1, 8, cap, 128, dtype=torch.float16), torch.zeros(1, 8, cap, 128, dtype=torch.float16))
              for _ in range(2)]
    O.prefill(w, O.embed_prompt(w, prompt), prompt.position_ids, caches)
    for li in range(2):
        assert_close_rel(eng.k_caches[li][0, :, :prompt.length].cpu(), caches[li][0][0, :, :prompt.length].float(),
                         what=f"prefill K layer {li}")
    ref, margins, _ = O.greedy_generate(w, prompt, n, cap)
    print(f"gpu {toks}\noracle {ref}\nmin margin {min(margins):.4g}", flush=True)
    assert toks == ref
    # eager decode from the same state gives the same tokens as graph replay,
    # with the position advance as its own launch instead of fused into the lm_head
    eng2 = DecodeEngine(w.to(cuda), capacity=cap, step_mode=step_mode, fuse_advance=False)
    first = eng2.prefill(prompt)
    assert eng2.decode(first, prompt.length, prompt.rope_delta, n - 1, use_graph=False) == toks[1:]
    # one graph per step instead of several (steps_per_graph=1), fused advance
    eng3 = DecodeEngine(w.to(cuda), capacity=cap, step_mode=step_mode, steps_per_graph=1)
    first = eng3.prefill(prompt)
    assert eng3.decode(first, prompt.length, prompt.rope_delta, n - 1, use_graph=True) == toks[1:]
    assert int(eng3.step_counter.item()) == n - 1
    assert int(eng3.cache_position.item()) == prompt.length + n - 1


@pytest.fixture(scope="module")
def config3_weights(cuda):
    from qwen3vl_hip import synthetic as syn

    gold = json.loads(GOLDEN.read_text())
    return syn.model_weights(gold["weight_seed"], device=cuda)


@pytest.mark.parametrize("step_mode", ["persistent", "chain"])
def test_full_model_config3_first_64_tokens(cuda, config3_weights, step_mode):
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import DecodeEngine

    gold = json.loads(GOLDEN.read_text())
    w = config3_weights
    fp = {
        "embed_sum": float(w.embed_tokens[:64].double().sum()),
        "layer0_qkv_sum": float(w.layers[0].qkv_weight[:64].double().sum()),
        "layer27_down_sum": float(w.layers[-1].down_proj_weight[:, :64].double().sum()),
        "final_norm_sum": float(w.final_norm_weight.double().sum()),
    }
    for k, v in gold["weight_fingerprint"].items():
        assert abs(fp[k] - v) <= 1e-9 * max(1.0, abs(v)), f"synthetic weight stream differs on this host: {k}"
    prompt = syn.multimodal_prompt(gold["prompt_seed"])
    assert prompt.length == gold["prompt_length"] and prompt.rope_delta == gold["rope_delta"]
    n = 64
    eng = DecodeEngine(w, capacity=prompt.length + 256, step_mode=step_mode)
    toks = eng.generate(prompt, n, use_graph=True)
    if step_mode == "persistent":
        assert eng.status() == 0
    ref = gold["tokens"][:n]
    first_bad = next((i for i, (a, b) in enumerate(zip(toks, ref)) if a != b), None)
    print(f"first mismatch: {first_bad}; margins there: "
          f"{gold['margins'][first_bad] if first_bad is not None else None}", flush=True)
    assert toks == ref
