#!/usr/bin/env python3
"""Batch-1 decode benchmark of the Qwen3-VL-2B text decoder on one MI355X.

Workload: the full 28-layer text decoder + tied lm_head
(vocab 151936) with random-init fp16 weights, batch 1, greedy decoding after a
1024-position multimodal-shaped prompt (768 vision rows on a 1x24x32 M-RoPE
grid + 256 random text ids), 256 generated tokens.  One "step" is one decode
token: the whole 28-layer step (embedding row, 28 x {RMSNorm+QKV, q/k norm +
M-RoPE + KV write, split-KV attention, o_proj+residual, RMSNorm+gate_up+SiLU,
down+residual}, final norm + lm_head + argmax, position advance) captured in a
HIP graph; the engine replays graphs that hold 8 consecutive steps (each step
reads the token and positions the previous one advanced on the device).
Weights and the KV cache are resident in HBM when the timed region starts.

Prints one JSON line: ms/token over the timed steps (value), tokens/s, the
step's achieved HBM GB/s (algorithmic bytes: weights + K/V[0:L] + activations,
each once), the same at a 4096-token context, the dominant kernel's roofline
entry and the CPU baseline (the fp32 PyTorch restatement of the reference path
on this host's cores); beside it the batch-8 workload (config 4) and configs
0-2 (one layer step, the five GEMVs, attention at L = 256..8192), each timed on
cold operands against its roofline with the CPU time of the same call.

The run checks itself and exits non-zero instead of printing a number when a
check fails: the timed config-3 tokens must match the oracle's golden stream
(tests/golden/config3_tokens.json) for at least the first 64 (all of them when
fewer are generated), the persistent step's status word must be clear after the
timed replays and after the 4096-context run, and the batch-8 step's first
tokens must equal the oracle's on a copy of the same caches.

    python bench.py [--gpus 1] [--steps 250] [--warmup 5]
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import platform
import sys
import time
import types
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "aicasgc-2026_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

GOLDEN = REPO / "tests" / "golden" / "config3_tokens.json"
PEAK_HBM_GBPS = 8000.0
PEAK_FP16_TFLOPS = 2500.0   # dense fp16 MFMA
WEIGHT_SEED = 3
PROMPT_SEED = 3


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gate_up_launch_bytes(shape) -> int:
    """Algorithmic bytes of one gate_up launch: 2NK + 2K + 2N with N = 2I rows, K = H."""
    n, k = 2 * shape.intermediate, shape.hidden
    return 2 * n * k + 2 * k + 2 * n


def persistent_launch_bytes(context_len: int, shape) -> int:
    """Algorithmic bytes of one persistent launch at cache position context_len - 1:
    every layer's weights and norms once, K/V rows [0, context_len) once per
    layer (the new row counted as its write), the fp16 embedding row read and
    the fp32 hidden state written for the lm_head."""
    h, i, d = shape.hidden, shape.intermediate, shape.head_dim
    layer_w = 2 * ((shape.q_size + 2 * shape.kv_size) * h + h * shape.q_size + 3 * i * h) + 2 * (2 * h + 2 * d)
    kv = 2 * 2 * shape.num_kv_heads * d * context_len
    return shape.num_layers * (layer_w + kv) + 2 * h + 4 * h


def bench_batch8(w, steps: int, warmup: int = 4, cpu: bool = True) -> dict:
    """Config 4: batch 8, per-sequence valid lengths L_i ~ U[2048, 4096]
    (seeded), seeded random K/V prefixes, greedy steps as HIP-graph replays (4
    steps per graph; MFMA batch GEMVs, per-sequence split-KV attention with the
    merge fused in, per-sequence argmax).

    The first step's 8 tokens are checked against the oracle's batch step on a
    host copy of the same caches (raises on a mismatch that is not a tie of
    the oracle's logits); that oracle call is also the CPU baseline's sample."""
    import torch

    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import BatchDecodeEngine, roofline_bytes_batch_step

    lens = [int(v) for v in syn.batch8_kv_lengths()]
    n = warmup + steps
    eng = BatchDecodeEngine(w, batch=8, capacity=max(lens) + n + 1)
    gen = torch.Generator(device=eng.device).manual_seed(44)   # the same caches whatever ran before
    for k, v in zip(eng.k_caches, eng.v_caches):
        k.normal_(generator=gen)
        v.normal_(generator=gen)
    host_caches = [(k.cpu(), v.cpu()) for k, v in zip(eng.k_caches, eng.v_caches)]
    tokens = [int(t) for t in syn.randint(4, ("text_ids",), (8,), 0, w.shape.vocab)]
    eng.reserve_tokens(n)
    eng.set_state(tokens, lens, lens)
    eng.step_counter.zero_()
    eng.capture()
    eng.warm_graphs()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    eng.replay_steps(warmup)   # enqueued right before the timed steps (no idle gap)
    e0.record()
    eng.replay_steps(steps)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    per_step = [roofline_bytes_batch_step([L + warmup + i + 1 for L in lens], w.shape) for i in range(steps)]
    nbytes = sum(per_step) / steps
    gbps = nbytes / (ms * 1e-3) / 1e9
    first_gpu = eng.out_tokens[0].tolist()
    final_pos = eng.cache_position.tolist()
    counter = int(eng.step_counter.item())
    status = eng.status()
    del eng
    if status != 0:
        raise RuntimeError(f"batch8: a qkv hand-off wait ran out of its polling budget (status {status})")
    if counter != n or final_pos != [L + n for L in lens]:
        raise RuntimeError(f"batch8: device positions did not advance {n} steps: counter {counter}, {final_pos}")
    check = batch8_first_step_check(w, tokens, lens, host_caches, first_gpu)
    del host_caches
    # GEMV flops on MFMA (2 per weight and sequence; attention runs on the VALU)
    s = w.shape
    gemv_params = s.num_layers * (s.qkv_rows * s.hidden + s.hidden * s.q_size + 3 * s.intermediate * s.hidden) \
        + s.vocab * s.hidden
    mfma_tflops = 2 * 8 * gemv_params / (ms * 1e-3) / 1e12
    return {"workload": "config4: 8 sequences, valid KV lengths U[2048,4096] (seeded), greedy, 4 steps per HIP graph",
            "kv_lengths": lens, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
            "first_step_tokens_match_oracle": not check["ties_within_tolerance"],
            "first_step_ties_within_tolerance": check["ties_within_tolerance"],
            "first_step_min_top2_margin": check["min_margin"],
            "cpu_baseline": check["cpu_baseline"] if cpu else None,
            "tokens_per_s": round(8 * 1000.0 / ms, 1), "step_bytes": int(nbytes), "achieved_GBps": round(gbps, 1),
            "roofline_frac": round(gbps / PEAK_HBM_GBPS, 4),
            "roofline_ms": round(nbytes / (PEAK_HBM_GBPS * 1e9) * 1e3, 4),
            "mfma": {"gflop_per_step": round(2 * 8 * gemv_params / 1e9, 2), "achieved_TFLOPs": round(mfma_tflops, 2),
                     "peak_TFLOPs": PEAK_FP16_TFLOPS, "frac": round(mfma_tflops / PEAK_FP16_TFLOPS, 5)}}


def batch8_first_step_check(weights_gpu, tokens, lens, host_caches, gpu_tokens) -> dict:
    """Config 4 on the host: the oracle's batch step (each sequence its own
    fp32 step on its own cache rows) on a copy of the GPU engine's caches taken
    before its first step.  Its tokens must equal the GPU's first-step tokens,
    except where the oracle's own logits tie within 2e-3 * max|logit| (raises
    otherwise); its time is the batch-8 CPU baseline sample."""
    import torch

    from oracle import qwen3vl_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    f32 = types.SimpleNamespace(
        embed_tokens=weights_gpu.embed_tokens.detach().to("cpu", torch.float32),
        final_norm_weight=weights_gpu.final_norm_weight.detach().to("cpu", torch.float32),
        layers=[{k: v.detach().to("cpu", torch.float32) for k, v in lw.tensors().items()}
                for lw in weights_gpu.layers])
    t0 = time.perf_counter()
    logits, toks = O.decode_step_batch(f32, tokens, host_caches, lens, lens)
    dt = time.perf_counter() - t0
    margins = [O.top2_margin(row) for row in logits]
    # A GPU token that differs from the oracle's must be a tie within the
    # logits' tolerance (2e-3 * max|logit| of the sequence, the bar of the GPU
    # tests): the oracle's logit at the GPU's token that close to its maximum.
    ties = []
    for b, (t_ref, t_gpu) in enumerate(zip(toks, gpu_tokens)):
        if int(t_ref) == int(t_gpu):
            continue
        row = logits[b].to(torch.float64)
        gap = float(row.max() - row[int(t_gpu)])
        if not gap <= 2e-3 * float(row.abs().max()):
            raise RuntimeError(f"batch8 first step: GPU tokens {gpu_tokens} != oracle {list(toks)} "
                               f"(top-2 margins {margins})")
        ties.append({"sequence": b, "oracle": int(t_ref), "gpu": int(t_gpu), "logit_gap": gap})
    return {"min_margin": round(min(margins), 6), "ties_within_tolerance": ties,
            "cpu_baseline": {"value": round(1000.0 * dt, 1), "unit": "ms/step", "cores": cores, "kind": "port",
                             "sample": "one batch-8 step of the oracle's fp32 restatement at the KV lengths above "
                                       "(the step whose tokens check the GPU's first step)"}}


ROTATE_BYTES = 512 << 20   # cold caches: every call reads a different copy (MALL: 256 MB)


def _graph_us(fns, reps: int) -> float:
    """Average microseconds per call of ``fns`` (each enqueues one call on the
    current stream): one HIP graph holds every call once, events bracket
    ``reps`` replays."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:   # lazy initialisation outside the capture
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / (reps * len(fns))


def _cpu_ms(fn, n: int, warmup: int = 2) -> float:
    times = []
    for i in range(warmup + n):
        t0 = time.perf_counter()
        fn()
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    times.sort()
    return round(1000.0 * times[len(times) // 2], 3)


def bench_configs012(w, cpu: bool, reps: int = 5) -> dict:
    """Configs 0-2 (one layer step, the five GEMVs, attention at four lengths)
    against their HBM rooflines, each call on a cold copy of its operands
    (copies rotated through >= 512 MB), with the oracle's fp32 time on this
    host beside each (``cpu``)."""
    import ctypes

    import torch

    from oracle import qwen3vl_oracle as O
    from qwen3vl_hip import _lib
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import DecodeEngine

    lib = _lib.lib()
    dev = torch.device("cuda:0")
    shape = w.shape
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gen = torch.Generator(device=dev).manual_seed(20)
    out = {"method": ("GPU: HIP events around replays of one HIP graph that calls the kernel once per operand "
                      f"copy (copies rotated through >= {ROTATE_BYTES >> 20} MiB, above the 256 MB MALL), "
                      f"{reps} replays; roofline = algorithmic bytes / 8 TB/s.  CPU: the oracle's fp32 PyTorch "
                      f"restatement, median of N calls after 2 warm-up, torch threads={cores}")}

    # ---- config 0: one decoder layer, cache_position 512 (K/V rows 0..511 filled)
    nl = max(4, -(-ROTATE_BYTES // 100_672_000))
    engines = []
    for i in range(nl):
        one = syn.ModelWeights([w.layers[i]], w.embed_tokens, w.final_norm_weight, shape)
        e = DecodeEngine(one, capacity=640)
        e.k_caches[0][:, :, :512].normal_(generator=gen)
        e.v_caches[0][:, :, :512].normal_(generator=gen)
        e.set_state(4242, 512, 512)
        engines.append(e)
    c0 = {"bytes": persistent_launch_bytes(513, dataclasses.replace(shape, num_layers=1))}
    if engines[0].step_mode == "persistent":
        c0["persistent_us"] = round(_graph_us([e.layers_persistent for e in engines], reps), 2)
        if any(e.status() for e in engines):
            raise RuntimeError("persistent one-layer step reported a failed hand-off")
    chain = ["qkv", "attn", "attn_merge", "o_proj", "gate_up", "down"]
    c0["chain_us"] = round(_graph_us([lambda e=e: e.run_phases(chain, 0, 1) for e in engines], reps), 2)
    # the drop-in layer's one launch (cuda_decode_gemv.fused_decode_full_layer_softsync_half) on
    # config 0's own input: a hidden state x ~ N(0, 1) and the rotation of position 512
    from cuda_decode_gemv_ops import fused as fused_ops

    f = engines[0].inv_freq * 512.0
    cos = torch.cat([f, f]).cos().half()
    sin = torch.cat([f, f]).sin().half()
    cp = torch.full((1,), 512, dtype=torch.int64, device=dev)
    xs = [torch.randn(1, 1, shape.hidden, generator=gen, device=dev).half() for _ in engines]
    wss = [{} for _ in engines]

    def one_launch(i):
        lw, e = w.layers[i], engines[i]
        if fused_ops._full_layer_persistent(
                xs[i], lw.qkv_weight, lw.input_layernorm_weight, lw.q_norm_weight, lw.k_norm_weight, cos, sin,
                e.k_caches[0], e.v_caches[0], cp, lw.o_proj_weight, None, lw.post_attn_layernorm_weight,
                lw.gate_up_weight, lw.down_proj_weight, None, shape.rms_eps, shape.head_dim ** -0.5, wss[i]) is None:
            raise RuntimeError("the one-launch decoder layer does not apply here")

    if engines[0].step_mode == "persistent":
        c0["dropin_one_launch_us"] = round(_graph_us([lambda i=i: one_launch(i) for i in range(len(engines))], reps), 2)
        if any(int(ws["status"].item()) for ws in wss):
            raise RuntimeError("one-launch decoder layer reported a failed hand-off")
    best = min(v for k, v in c0.items() if k.endswith("_us"))
    c0.update(roofline_us=round(c0["bytes"] / (PEAK_HBM_GBPS * 1e3), 2), frac=round(c0["bytes"] / (best * 1e-6) /
                                                                                        1e9 / PEAK_HBM_GBPS, 4))
    del engines
    if cpu:
        lw = {k: v.detach().to("cpu", torch.float32) for k, v in w.layers[0].tensors().items()}
        kc = syn.normal(5, ("k",), (1, shape.num_kv_heads, 513, shape.head_dim))
        vc = syn.normal(5, ("v",), (1, shape.num_kv_heads, 513, shape.head_dim))
        x = syn.normal(5, ("x",), (shape.hidden,)).float()
        cos, sin = O.mrope_cos_sin(torch.full((3, 1), 512, dtype=torch.int64))
        c0["cpu_ms"] = _cpu_ms(lambda: O.decode_layer(lw, x, kc, vc, 512, cos[0], sin[0]), 10)
        del lw
    out["config0_layer_step"] = c0

    # ---- config 1: the decode GEMVs (plain y = W x, fp16 in and out)
    c1 = {}
    for name, (n, k) in syn.GEMV_SHAPES.items():
        copies = max(4, -(-ROTATE_BYTES // (2 * n * k)))
        ws = [torch.randn(n, k, generator=gen, device=dev, dtype=torch.float16).mul_(0.02) for _ in range(copies)]
        xs = [torch.randn(k, generator=gen, device=dev, dtype=torch.float16) for _ in range(copies)]
        ys = [torch.empty(n, device=dev, dtype=torch.float16) for _ in range(copies)]

        def call(i, n=n, k=k, ws=ws, xs=xs, ys=ys):
            _lib.check(lib.qd_matvec_f16(_lib.ptr(xs[i]), _lib.ptr(ws[i]), None, _lib.ptr(ys[i]), n, k,
                                         _lib.stream()), "qd_matvec_f16")

        us = _graph_us([lambda i=i: call(i) for i in range(copies)], reps)
        nbytes = 2 * n * k + 2 * k + 2 * n
        r = {"shape": [n, k], "us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
             "roofline_us": round(nbytes / (PEAK_HBM_GBPS * 1e3), 2),
             "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
        if cpu:
            wc, xc = ws[0].float().cpu(), xs[0].float().cpu()
            r["cpu_ms"] = _cpu_ms(lambda: O.gemv(xc, wc), 20 if n * k < 1e8 else 5)
            del wc
        c1[name] = r
        del ws, xs, ys
    out["config1_gemv"] = c1

    # ---- config 2: split-KV attention, valid length L = T (cache_position L - 1)
    c2 = {}
    hq, hkv, d = shape.num_heads, shape.num_kv_heads, shape.head_dim
    scale = 1.0 / (d ** 0.5)
    for L in (256, 1024, 4096, 8192):
        kv = 2 * 2 * hkv * L * d
        copies = min(512, max(4, -(-ROTATE_BYTES // kv)))
        ks = [torch.randn(hkv, L, d, generator=gen, device=dev, dtype=torch.float16) for _ in range(copies)]
        vs = [torch.randn(hkv, L, d, generator=gen, device=dev, dtype=torch.float16) for _ in range(copies)]
        q = torch.randn(hq, d, generator=gen, device=dev, dtype=torch.float16)
        o = torch.empty(hq, d, device=dev, dtype=torch.float16)
        cp = torch.full((1,), L - 1, dtype=torch.int64, device=dev)
        n_split = int(lib.qd_attention_default_splits(L))
        wsb = torch.zeros(int(lib.qd_attention_workspace_bytes(hq, hkv, n_split)), dtype=torch.uint8, device=dev)

        def acall(i, L=L, ks=ks, vs=vs, q=q, o=o, cp=cp, n_split=n_split, wsb=wsb):
            _lib.check(lib.qd_attention_decode(
                _lib.ptr(q), _lib.QD_F16, d, _lib.ptr(ks[i]), _lib.ptr(vs[i]), L * d, d, L, _lib.ptr(cp),
                ctypes.c_float(scale), _lib.ptr(o), _lib.QD_F16, hq, hkv, n_split, _lib.ptr(wsb), _lib.stream()),
                "qd_attention_decode")

        us = _graph_us([lambda i=i: acall(i) for i in range(copies)], reps)
        nbytes = kv + 2 * 2 * hq * d
        r = {"us": round(us, 2), "splits": n_split, "bytes": nbytes, "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
             "roofline_us": round(nbytes / (PEAK_HBM_GBPS * 1e3), 3),
             "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
        if cpu:
            qc = q.float().cpu()
            kc, vc = ks[0].cpu().unsqueeze(0), vs[0].cpu().unsqueeze(0)
            r["cpu_ms"] = _cpu_ms(lambda: O.decode_attention(qc, kc, vc, L - 1, scale), 20)
        c2[f"L{L}"] = r
        del ks, vs
    out["config2_attention"] = c2
    torch.cuda.empty_cache()
    return out


def dropin_text_model(w, device):
    """transformers' Qwen3VLTextModel at the Qwen3-VL-2B text shape holding the
    synthetic fp16 weights, every decoder layer swapped by
    optimized_layer.replace_decoder_layers (reference optimized_layer.py:3848).
    Built on the meta device and materialised on the GPU (the rotary buffers
    are recomputed there, in fp32)."""
    import torch
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLTextConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLTextModel, Qwen3VLTextRotaryEmbedding

    import optimized_layer

    s = w.shape
    cfg = Qwen3VLTextConfig(hidden_size=s.hidden, intermediate_size=s.intermediate, num_attention_heads=s.num_heads,
                            num_key_value_heads=s.num_kv_heads, head_dim=s.head_dim, num_hidden_layers=s.num_layers,
                            vocab_size=s.vocab, rms_norm_eps=s.rms_eps,
                            rope_parameters={"rope_type": "default", "rope_theta": s.rope_theta,
                                             "mrope_section": list(s.mrope_section)})
    cfg._attn_implementation = "sdpa"
    with torch.device("meta"):
        m = Qwen3VLTextModel(cfg)
    m = m.to_empty(device=device).half().eval()
    with torch.device(device):
        m.rotary_emb = Qwen3VLTextRotaryEmbedding(cfg)
    q, kv, i = s.q_size, s.kv_size, s.intermediate
    with torch.no_grad():
        m.embed_tokens.weight.copy_(w.embed_tokens)
        m.norm.weight.copy_(w.final_norm_weight)
        for lw, L in zip(w.layers, m.layers):
            a = L.self_attn
            a.q_proj.weight.copy_(lw.qkv_weight[:q])
            a.k_proj.weight.copy_(lw.qkv_weight[q:q + kv])
            a.v_proj.weight.copy_(lw.qkv_weight[q + kv:])
            a.o_proj.weight.copy_(lw.o_proj_weight)
            a.q_norm.weight.copy_(lw.q_norm_weight)
            a.k_norm.weight.copy_(lw.k_norm_weight)
            L.mlp.gate_proj.weight.copy_(lw.gate_up_weight[:i])
            L.mlp.up_proj.weight.copy_(lw.gate_up_weight[i:])
            L.mlp.down_proj.weight.copy_(lw.down_proj_weight)
            L.input_layernorm.weight.copy_(lw.input_layernorm_weight)
            L.post_attention_layernorm.weight.copy_(lw.post_attn_layernorm_weight)
    optimized_layer.replace_decoder_layers(m)
    return m, cfg


def bench_dropin(w, prompt, k_caches, v_caches, first: int, steps: int, warmup: int, golden) -> dict:
    """The reference's own decode loop over the drop-in layers: one step of the
    swapped transformers model (embedding, M-RoPE cos/sin, 28 swapped layers,
    final norm, the tied lm_head through the drop-in nosplit_matvec_half as the
    reference's FastLmHead does, argmax) captured in a HIP graph and
    replayed with the static input buffers rewritten on the device between
    replays (DecodeCudaGraphRunner, evaluation_wrapper.py:864-904, :941-960).
    It continues from the native engine's prefilled K/V rows, so its tokens are
    compared with the golden stream (reported, not required: this path keeps
    fp16 activations between kernels, as the reference does)."""
    import torch
    from transformers.cache_utils import StaticCache

    import cuda_decode_gemv

    dev = k_caches[0].device
    model, cfg = dropin_text_model(w, dev)
    S = prompt.length
    n = warmup + steps
    max_len = S + n + 2
    cache = StaticCache(config=cfg, max_cache_len=max_len)
    like = torch.empty(1, w.shape.num_kv_heads, 1, w.shape.head_dim, dtype=torch.float16, device=dev)
    for li, layer in enumerate(cache.layers):
        if not layer.is_initialized:
            layer.lazy_initialization(like, like)
        layer.keys[:, :, :S].copy_(k_caches[li][:, :, :S])
        layer.values[:, :, :S].copy_(v_caches[li][:, :, :S])
    ids = torch.zeros(1, 1, dtype=torch.int64, device=dev)
    cache_position = torch.zeros(1, dtype=torch.int64, device=dev)
    position_ids = torch.zeros(3, 1, 1, dtype=torch.int64, device=dev)
    mask = torch.zeros(1, max_len, dtype=torch.int64, device=dev)
    mask[:, :S] = 1
    next_token = torch.zeros(1, 1, dtype=torch.int64, device=dev)
    out_tokens = torch.zeros(n, dtype=torch.int64, device=dev)
    emb = w.embed_tokens
    lm_head_ws = {"type": "nosplit", "out": torch.empty(emb.shape[0], dtype=emb.dtype, device=dev)}

    def run():
        out = model(input_ids=ids, attention_mask=mask, position_ids=position_ids, past_key_values=cache,
                    use_cache=True, cache_position=cache_position)
        # the reference's FastLmHead (evaluation_wrapper.py:1210-1238): the tied lm_head as one
        # cuda_decode_gemv.nosplit_matvec_half into a workspace output, then torch.argmax (:952)
        logits = cuda_decode_gemv.nosplit_matvec_half(out.last_hidden_state, emb, None, workspace=lm_head_ws)
        next_token.copy_(torch.argmax(logits[:, -1, :], dim=-1, keepdim=True))

    def write_inputs(p):   # the runner's _write_inputs: device-side copies and fills, no host sync
        ids.copy_(next_token)
        cache_position.fill_(p)
        position_ids.fill_(p + prompt.rope_delta)
        mask[:, p] = 1

    def timed(one_launch: bool, lookahead: bool = False):
        """Capture the step with the swapped layers on one decode path (the
        one-launch persistent layer, or the kernel chain; with ``lookahead``
        the first swapped layer launches the whole stack) and time its replays
        from the prompt's end; returns (ms per token, tokens)."""
        import optimized_layer

        prev = optimized_layer.set_cuda_mlp_fusion_flags(full_layer_softsync=one_launch)
        prev_la = optimized_layer.set_decode_layer_lookahead(lookahead)
        try:
            next_token.fill_(first)
            write_inputs(S)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side), torch.no_grad():
                run()                      # warm-up of lazy initialisation, outside the capture
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            next_token.fill_(first)
            write_inputs(S)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph), torch.no_grad():
                run()
        finally:
            optimized_layer.set_cuda_mlp_fusion_flags(full_layer_softsync=prev[1])
            optimized_layer.set_decode_layer_lookahead(prev_la)
        next_token.fill_(first)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for i in range(n):
            if i == warmup:
                e0.record()
            write_inputs(S + i)
            graph.replay()
            out_tokens[i].copy_(next_token[0, 0])
        e1.record()
        torch.cuda.synchronize()
        del graph
        return e0.elapsed_time(e1) / steps, out_tokens.tolist()

    gold = golden["tokens"][1:1 + n]
    res = {}
    toks_by = {}
    for label, one_launch, la in (("one_launch", True, False), ("chain", False, False), ("lookahead", True, True)):
        ms, toks = timed(one_launch, la)
        match = next((i for i, (a, b) in enumerate(zip(toks, gold)) if a != b), min(len(toks), len(gold)))
        res[label] = (ms, match, min(len(toks), len(gold)))
        toks_by[label] = toks
    import optimized_layer

    optimized_layer.check_decode_status(model)
    fused_layers = sum(1 for L in model.layers if L._full_layer_workspace.get("out") is not None)
    del model, cache
    torch.cuda.empty_cache()
    ms, match, n_cmp = res["one_launch"]
    return {"method": "transformers Qwen3VLTextModel with every decoder layer swapped by "
                      "optimized_layer.replace_decoder_layers, one step captured in a HIP graph, static input "
                      "buffers rewritten on the device between replays (the reference's DecodeCudaGraphRunner); "
                      "tied lm_head through cuda_decode_gemv.nosplit_matvec_half (the reference's FastLmHead) + "
                      "torch.argmax in the graph; HIP events over the timed steps",
            "layer_path": "one persistent launch per swapped layer (fused_decode_full_layer_softsync_half)",
            "layers_on_one_launch_path": fused_layers,
            "ms_per_token": round(ms, 4), "tokens_per_s": round(1000.0 / ms, 1), "steps": steps, "warmup": warmup,
            "context_start": S, "tokens_match_golden_prefix": match, "tokens_compared": n_cmp,
            "chain": {"layer_path": "kernel chain per swapped layer (full_layer_softsync fusion flag off)",
                      "ms_per_token": round(res["chain"][0], 4),
                      "tokens_match_golden_prefix": res["chain"][1], "tokens_compared": res["chain"][2]},
            "lookahead": {"layer_path": "opt-in look-ahead (optimized_layer.set_decode_layer_lookahead): the first "
                                        "swapped layer launches all 28 in one persistent launch, the others "
                                        "return their rows",
                          "ms_per_token": round(res["lookahead"][0], 4),
                          "tokens_match_golden_prefix": res["lookahead"][1], "tokens_compared": res["lookahead"][2],
                          "tokens_equal_one_launch": toks_by["lookahead"] == toks_by["one_launch"]}}


def phase_trace(contexts) -> list:
    """Per-link timeline of the persistent step (qwen3vl_hip.phase_trace) in a
    child process that loads the traced library, so this process's numbers come
    from the regular one."""
    import subprocess

    from qwen3vl_hip import _lib

    if not _lib.TRACE_LIB_PATH.exists():
        raise RuntimeError(f"{_lib.TRACE_LIB_PATH} is not built (__graft_entry__.build() makes it)")
    env = dict(os.environ, QD_LIB_PATH=str(_lib.TRACE_LIB_PATH),
               PYTHONPATH=os.pathsep.join([str(REPO / "aicasgc-2026_amd"), os.environ.get("PYTHONPATH", "")]))
    cmd = [sys.executable, "-u", "-m", "qwen3vl_hip.phase_trace"] + [a for c in contexts for a in ("--ctx", str(c))]
    r = subprocess.run(cmd, env=env, stdout=subprocess.PIPE, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"phase trace failed with status {r.returncode}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(weights_gpu, prompt_len: int, n_steps: int, warmup: int = 2) -> dict:
    """The oracle's fp32 decode step (the reference's CPU PyTorch path restated)
    on this host, timed on a bounded sample: ``n_steps`` decode tokens at a
    ~prompt_len context with a random K/V prefix."""
    import torch

    from oracle import qwen3vl_oracle as O
    from qwen3vl_hip import synthetic as syn

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    s = weights_gpu.shape
    layers = [{k: v.detach().to("cpu", torch.float32) for k, v in lw.tensors().items()} for lw in weights_gpu.layers]
    emb = weights_gpu.embed_tokens.detach().to("cpu", torch.float32)
    fnorm = weights_gpu.final_norm_weight.detach().to("cpu", torch.float32)
    cap = prompt_len + warmup + n_steps + 1
    caches = []
    for li in range(s.num_layers):
        k = syn.normal(99, ("k_cache", li), (1, s.num_kv_heads, cap, s.head_dim))
        v = syn.normal(99, ("v_cache", li), (1, s.num_kv_heads, cap, s.head_dim))
        caches.append((k, v))
    tok = 1234
    times = []
    for i in range(warmup + n_steps):
        pos = prompt_len + i
        cos, sin = O.mrope_cos_sin(torch.full((3, 1), pos - 736, dtype=torch.int64))
        t0 = time.perf_counter()
        h = emb[tok]
        for li, w in enumerate(layers):
            h = O.decode_layer(w, h, caches[li][0], caches[li][1], pos, cos[0], sin[0])
        _, tok = O.lm_head_argmax(h, fnorm, emb, s.rms_eps)
        dt = time.perf_counter() - t0
        if i >= warmup:
            times.append(dt)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(1000.0 * med, 2),
        "unit": "ms/token",
        "cores": cores,
        "kind": "port",
        "sample": (f"median of {n_steps} decode steps (after {warmup} warm-up) of the oracle's fp32 PyTorch "
                   f"restatement of the 28-layer step + lm_head at context ~{prompt_len}, random K/V prefix, "
                   f"torch threads={cores}, cpu={_cpu_model()}"),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=250)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ctx-steps", type=int, default=64, help="decode steps timed around a 4096 context")
    ap.add_argument("--kernel-reps", type=int, default=10, help="repetitions of the gate_up timing (x28 launches)")
    ap.add_argument("--cpu-steps", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--attn-splits", type=int, default=0)
    ap.add_argument("--step-mode", choices=["auto", "chain", "persistent"], default="auto")
    ap.add_argument("--batch8-steps", type=int, default=64,
                    help="timed steps of the batch-8 workload (config 4); 0 skips it")
    ap.add_argument("--no-configs012", action="store_true",
                    help="skip configs 0-2 (one layer, the GEMVs, attention) against their rooflines")
    ap.add_argument("--dropin-steps", type=int, default=32,
                    help="timed steps of the graph-captured drop-in path (transformers model + swapped layers); "
                         "0 skips it")
    ap.add_argument("--phase-trace", type=int, action="append", metavar="CTX",
                    help="also report the persistent step's per-link timeline at this context (repeatable), from "
                         "the -DQD_TRACE library run in a child process (qwen3vl_hip.phase_trace)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build's decode path runs on a single MI355X "
              "(no collectives / multi-GPU sharding); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import DecodeEngine, roofline_bytes_step

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t_start = time.time()
    w = syn.model_weights(WEIGHT_SEED, device=dev)
    prompt = syn.multimodal_prompt(PROMPT_SEED)
    shape = w.shape
    log(f"weights ready ({time.time() - t_start:.1f}s)")

    n_dec = args.warmup + args.steps
    cap = prompt.length + n_dec + 1
    eng = DecodeEngine(w, capacity=cap, attn_splits=args.attn_splits, step_mode=args.step_mode)
    eng_steps_per_graph = eng.steps_per_graph
    first = eng.prefill(prompt)
    eng.reserve_tokens(n_dec)
    eng.set_state(first, prompt.length, prompt.length + prompt.rope_delta)
    eng.step_counter.zero_()
    eng.capture()
    torch.cuda.synchronize()
    log(f"prefill + capture done ({time.time() - t_start:.1f}s)")

    # every captured graph (the single step and the multi-step one) is replayed
    # once before the timed region, state restored, so no first replay is timed
    eng.warm_graphs()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # the W untimed warm-up steps are enqueued right before the timed ones, so
    # the GPU goes from warm-up into the timed steps without an idle gap (an
    # idle GPU after a host sync runs its next steps slower)
    eng.replay_steps(args.warmup)
    ev0.record()
    eng.replay_steps(args.steps)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    tokens = [first] + eng.out_tokens[:n_dec].tolist()
    # the timed run must be a valid one: every hand-off completed, the tokens
    # are the oracle's (the first 64 identical)
    if eng.step_mode == "persistent" and eng.status() != 0:
        log("FAIL: a persistent-step hand-off timed out during the timed replays")
        return 1
    gold = json.loads(GOLDEN.read_text())
    n_chk = min(len(tokens), len(gold["tokens"]))
    match = next((i for i in range(n_chk) if tokens[i] != gold["tokens"][i]), n_chk)
    if match < min(64, n_chk):
        log(f"FAIL: token {match} differs from the oracle's golden stream ({tokens[match]} vs "
            f"{gold['tokens'][match]})")
        return 1
    # K/V length read by timed step i (cache position p reads p + 1 rows)
    lens = [prompt.length + args.warmup + i + 1 for i in range(args.steps)]
    step_bytes = sum(roofline_bytes_step(L, shape) for L in lens) / len(lens)
    gbps = step_bytes / (ms * 1e-3) / 1e9
    log(f"config3: {ms:.4f} ms/token, {gbps:.1f} GB/s ({time.time() - t_start:.1f}s)")

    # ---- the same step around a 4096-token context (the target point)
    half = args.ctx_steps // 2
    eng4 = DecodeEngine(w, capacity=4096 + half + 1, attn_splits=args.attn_splits, step_mode=args.step_mode)
    for k, v in zip(eng4.k_caches, eng4.v_caches):
        k.normal_()
        v.normal_()
    w4 = 4   # untimed warm-up steps, enqueued right before the timed ones
    eng4.reserve_tokens(args.ctx_steps + w4)
    eng4.set_state(first, 4096 - half - w4, 4096 - half - w4 + prompt.rope_delta)
    eng4.step_counter.zero_()
    eng4.capture()
    eng4.warm_graphs()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    eng4.replay_steps(w4)
    e0.record()
    eng4.replay_steps(args.ctx_steps)
    e1.record()
    torch.cuda.synchronize()
    ms4 = e0.elapsed_time(e1) / args.ctx_steps
    lens4 = [4096 - half + i + 1 for i in range(args.ctx_steps)]
    bytes4 = sum(roofline_bytes_step(L, shape) for L in lens4) / len(lens4)
    gbps4 = bytes4 / (ms4 * 1e-3) / 1e9
    if eng4.step_mode == "persistent" and eng4.status() != 0:
        log("FAIL: a persistent-step hand-off timed out in the 4096-context run")
        return 1
    if int(eng4.step_counter.item()) != args.ctx_steps + w4:
        log("FAIL: the 4096-context run did not advance every step")
        return 1
    del eng4
    log(f"ctx4096: {ms4:.4f} ms/token, {gbps4:.1f} GB/s")

    # ---- dominant kernel.  Persistent step: the one launch that runs all 28
    # layers (algorithmic bytes = every layer weight + K/V[0:L] once, the
    # embedding row, the fp32 hidden it leaves for the lm_head).  Kernel chain:
    # the gate_up GEMV (RMSNorm prologue, SiLU*up epilogue), 28 distinct weights
    # per pass.  Timed with events on the stream the kernels are launched on.
    stream = torch.cuda.current_stream()
    mode = eng.step_mode
    if mode == "persistent":
        # fixed context (cache position prompt_len + 4), the one the committed
        # PMC traffic figures in profiles/persistent_traffic.json were taken at
        ctx = min(prompt.length + 5, cap)
        eng.set_state(first, ctx - 1, ctx - 1 + prompt.rope_delta)
        eng.layers_persistent()
        torch.cuda.synchronize()
        k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        k0.record(stream)
        for _ in range(args.kernel_reps):
            eng.layers_persistent()
        k1.record(stream)
        torch.cuda.synchronize()
        if eng.status() != 0:
            raise RuntimeError("persistent step reported a failed hand-off")
        n_launch = args.kernel_reps
        kbytes = persistent_launch_bytes(ctx, shape)
        kname = "decode_persistent_kernel (embedding + 28 layers, one launch)"
        kunits = f"one decode step's 28 layers at context {ctx}"
    else:
        eng.run_phases(["gate_up"])
        torch.cuda.synchronize()
        k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        k0.record(stream)
        for _ in range(args.kernel_reps):
            eng.run_phases(["gate_up"])
        k1.record(stream)
        torch.cuda.synchronize()
        n_launch = args.kernel_reps * shape.num_layers
        kbytes = gate_up_launch_bytes(shape)
        kname = "gemv_kernel<4,4,PRO_RMSNORM,EPI_SILU,f32,f32> (gate_up)"
        kunits = "one layer's gate_up rows (2I x H)"
    us_launch = k0.elapsed_time(k1) * 1000.0 / n_launch
    k_gbps = kbytes / (us_launch * 1e-6) / 1e9
    log(f"{kname}: {us_launch:.2f} us/launch, {k_gbps:.1f} GB/s")

    # ---- the lm_head + argmax phase (second largest; same stream, events)
    eng.run_phases(["lm_head"], n_layers=0)
    torch.cuda.synchronize()
    h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h0.record(stream)
    for _ in range(args.kernel_reps):
        eng.run_phases(["lm_head"], n_layers=0)
    h1.record(stream)
    torch.cuda.synchronize()
    us_head = h0.elapsed_time(h1) * 1000.0 / args.kernel_reps
    head_bytes = 2 * shape.vocab * shape.hidden + 2 * shape.hidden + 4 * shape.hidden
    log(f"lm_head+argmax: {us_head:.2f} us, {head_bytes / (us_head * 1e-6) / 1e9:.1f} GB/s")

    # ---- the drop-in path at config 3 (the reference user's own decode loop)
    dropin = None
    if args.dropin_steps > 0:
        dropin = bench_dropin(w, prompt, eng.k_caches, eng.v_caches, first, args.dropin_steps, 4, gold)
        log(f"drop-in (transformers model + swapped layers, HIP graph): {dropin['ms_per_token']:.4f} ms/token "
            f"one launch per layer ({dropin['layers_on_one_launch_path']} layers), "
            f"{dropin['lookahead']['ms_per_token']:.4f} ms/token with the look-ahead (tokens equal: "
            f"{dropin['lookahead']['tokens_equal_one_launch']}), "
            f"{dropin['chain']['ms_per_token']:.4f} ms/token kernel chain; golden prefix "
            f"{dropin['tokens_match_golden_prefix']} / {dropin['chain']['tokens_match_golden_prefix']} of "
            f"{dropin['tokens_compared']}")

    # ---- config 4: 8 sequences, ragged contexts L_i ~ U[2048, 4096]
    b8 = None
    if args.batch8_steps > 0:
        b8 = bench_batch8(w, args.batch8_steps, cpu=not args.no_cpu)
        log(f"batch8: {b8['ms_per_step']:.4f} ms/step, {b8['tokens_per_s']:.0f} tok/s, {b8['achieved_GBps']:.1f} GB/s")

    # ---- configs 0-2 against their rooflines (cold operands), CPU beside them
    c012 = None
    if not args.no_configs012:
        c012 = bench_configs012(w, cpu=not args.no_cpu)
        c0 = c012["config0_layer_step"]
        log("config0 one layer: " + ", ".join(f"{k} {v}" for k, v in c0.items()))
        log("config1 GEMV us: " + ", ".join(f"{n} {r['us']} ({r['frac']:.2f})" for n, r in c012["config1_gemv"].items()))
        log("config2 attention us: " + ", ".join(f"{n} {r['us']} ({r['frac']:.2f})"
                                                 for n, r in c012["config2_attention"].items()))

    # ---- reference stream: a plain 256 MiB device copy (known bytes; also the
    # scale for the PMC FETCH_SIZE / WRITE_SIZE counters in profiles/)
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(4):
        dst.copy_(src)
    c1.record()
    torch.cuda.synchronize()
    copy_gbps = 2 * src.numel() / (c0.elapsed_time(c1) / 4 * 1e-3) / 1e9
    del src, dst
    log(f"256 MiB device copy: {copy_gbps:.1f} GB/s (read + write)")

    traffic = None
    tfile = REPO / "profiles" / ("persistent_traffic.json" if mode == "persistent" else "gate_up_traffic.json")
    if tfile.exists():
        try:
            tj = json.loads(tfile.read_text())
            if mode != "persistent" or tj.get("context_rows") == ctx:
                traffic = tj.get("bytes_per_launch")
        except (ValueError, OSError):
            traffic = None

    traced = None
    if args.phase_trace:
        log(f"phase trace at contexts {args.phase_trace} ...")
        traced = phase_trace(args.phase_trace)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline(w, prompt.length, args.cpu_steps)
        log(f"cpu baseline {cpu['value']} ms/token on {cpu['cores']} cores")
        if b8 is not None:
            log(f"cpu baseline batch8 {b8['cpu_baseline']['value']} ms/step")

    out = {
        "metric": "bs1 decode ms/token, Qwen3-VL-2B fp16; achieved HBM GB/s vs 8 TB/s peak",
        "value": round(ms, 4),
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded random-init weights, multimodal-shaped prompt)",
        "config": {
            "workload": "config3: 28-layer Qwen3-VL-2B text decoder + tied lm_head, batch 1, greedy, "
                        "1024-position prompt (768 vision rows on 1x24x32 M-RoPE grid + 256 text ids), "
                        f"{1 + n_dec} generated tokens, whole step in one HIP graph, "
                        f"{eng_steps_per_graph} steps per graph replay",
            "prompt_len": prompt.length,
            "generated_tokens": 1 + n_dec,
            "mean_context": round(sum(lens) / len(lens), 1),
            "attn_splits": int(eng.desc.attn_splits) or None,
            "step_mode": eng.step_mode,
        },
        "tokens_per_s": round(1000.0 / ms, 1),
        "achieved_GBps": round(gbps, 1),
        "step_roofline_frac": round(gbps / PEAK_HBM_GBPS, 4),
        "step_bytes": int(step_bytes),
        "ctx4096": {"ms_per_token": round(ms4, 4), "tokens_per_s": round(1000.0 / ms4, 1),
                    "achieved_GBps": round(gbps4, 1), "roofline_frac": round(gbps4 / PEAK_HBM_GBPS, 4),
                    "step_bytes": int(bytes4), "roofline_ms": round(bytes4 / (PEAK_HBM_GBPS * 1e9) * 1e3, 4)},
        "roofline": {"bound": "hbm", "kernel": kname, "units_per_launch": kunits,
                     "achieved": round(k_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(k_gbps / PEAK_HBM_GBPS, 4), "traffic": traffic,
                     "us_per_launch": round(us_launch, 3), "bytes_per_launch": kbytes},
        "lm_head": {"us_per_launch": round(us_head, 3), "bytes_per_launch": head_bytes,
                    "achieved_GBps": round(head_bytes / (us_head * 1e-6) / 1e9, 1)},
        # what a graph-replayed step costs beyond its two kernels (launch gaps,
        # the graph's own work): the step minus the persistent launch and the
        # lm_head, each timed on its own (the launch at context ctx)
        "step_tail_us": (round(ms * 1000.0 - us_launch - us_head, 1) if mode == "persistent" else None),
        "cpu_baseline": cpu,
        "device_copy_GBps": round(copy_gbps, 1),
        "tokens_head": tokens[:8],
        "tokens_checked": n_chk,
        "tokens_match_golden_prefix": match,
        "batch8": b8,
        "configs012": c012,
        "phase_trace": traced,
        "dropin": dropin,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
