"""Write the oracle's greedy tokens for the full-model configuration (config 3).

Runs the CPU oracle (fp32 math, fp16 static KV cache) on the seeded synthetic
28-layer Qwen3-VL-2B text decoder with the 1024-position multimodal-shaped
prompt, and records the first N greedy tokens with each step's top-1/top-2
logit margin.  The GPU test regenerates the same weights from the same seeds
and compares its tokens against this file.

    python tests/golden/make_config3_tokens.py [--tokens 64] [--out tests/golden/config3_tokens.json]
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(REPO), str(REPO / "aicasgc-2026_amd")]

from oracle import qwen3vl_oracle as O  # noqa: E402
from qwen3vl_hip import synthetic as syn  # noqa: E402

WEIGHT_SEED = 3
PROMPT_SEED = 3


def weight_fingerprint(w) -> dict:
    """A few exact sums that detect a different weight stream on another host."""
    return {
        "embed_sum": float(w.embed_tokens[:64].double().sum()),
        "layer0_qkv_sum": float(w.layers[0].qkv_weight[:64].double().sum()),
        "layer27_down_sum": float(w.layers[-1].down_proj_weight[:, :64].double().sum()),
        "final_norm_sum": float(w.final_norm_weight.double().sum()),
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--out", default=str(REPO / "tests" / "golden" / "config3_tokens.json"))
    args = ap.parse_args()
    t0 = time.time()
    w = syn.model_weights(WEIGHT_SEED)
    fp = weight_fingerprint(w)
    # upcast once so the oracle does not convert per call
    for lw in w.layers:
        for k, v in lw.__dict__.items():
            setattr(lw, k, v.float())
    w.embed_tokens = w.embed_tokens.float()
    w.final_norm_weight = w.final_norm_weight.float()
    prompt = syn.multimodal_prompt(PROMPT_SEED)
    print(f"weights ready in {time.time() - t0:.1f}s", flush=True)
    capacity = prompt.length + args.tokens
    tokens, margins, _ = O.greedy_generate(
        w, prompt, args.tokens, capacity,
        log=lambda i, t, m: print(f"step {i}: token {t} margin {m:.4f}  ({time.time() - t0:.0f}s)", flush=True))
    out = {
        "config": "config 3: 28-layer Qwen3-VL-2B text decoder, tied lm_head, batch 1, greedy",
        "weight_seed": WEIGHT_SEED,
        "prompt_seed": PROMPT_SEED,
        "prompt_length": prompt.length,
        "rope_delta": prompt.rope_delta,
        "tokens": tokens,
        "margins": margins,
        "weight_fingerprint": fp,
        "oracle": "oracle/qwen3vl_oracle.py greedy_generate, fp32 math, fp16 KV cache",
    }
    Path(args.out).write_text(json.dumps(out, indent=1))
    print(f"wrote {args.out} in {time.time() - t0:.1f}s; min margin {min(margins):.4g}")


if __name__ == "__main__":
    torch.set_num_threads(max(1, torch.get_num_threads()))
    main()
