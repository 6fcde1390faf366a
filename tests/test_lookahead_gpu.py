"""The swapped layers' opt-in look-ahead (optimized_layer.set_decode_layer_lookahead):
the first swapped layer of a decode step runs every swapped layer in one
persistent launch (qd_decoder_layers_persistent_f16) and the later layers
return their rows.  Each row must equal, bit for bit, what the layer's own
one-layer launch returns, so the model's outputs, the K/V rows every layer
writes and the caches' running lengths are compared for equality with the
look-ahead off, in eager steps and in a captured graph replayed over several
positions; a layer with a hook, or an input that is not the previous row,
falls back to its own launch.
"""

from __future__ import annotations

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

N_LAYERS = 3


def _model_and_cache(cuda, S, extra):
    from transformers.cache_utils import StaticCache

    import optimized_layer
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.config import Qwen3VLTextShape
    from test_dropin_model_gpu import _hf_model

    shape = Qwen3VLTextShape(num_layers=N_LAYERS, vocab=1024)
    w = syn.model_weights(31, shape=shape)
    gpu = copy.deepcopy(_hf_model(w, shape)).half().to(cuda)
    assert optimized_layer.replace_decoder_layers(gpu) == N_LAYERS
    cache = StaticCache(config=gpu.config, max_cache_len=S + extra)
    like = torch.empty(1, shape.num_kv_heads, 1, shape.head_dim, dtype=torch.float16, device=cuda)
    g = torch.Generator(device=cuda).manual_seed(5)
    for layer in cache.layers:
        if not layer.is_initialized:
            layer.lazy_initialization(like, like)
        layer.keys.normal_(generator=g)
        layer.values.normal_(generator=g)
    return gpu, cache, w.embed_tokens.to(cuda)


def _snapshot(cache):
    return [(L.keys.clone(), L.values.clone()) for L in cache.layers]


def _restore(cache, snap):
    for L, (k, v) in zip(cache.layers, snap):
        L.keys.copy_(k)
        L.values.copy_(v)


def _step(gpu, cache, emb, tok, p, delta=-5):
    rp = torch.full((3, 1, 1), p + delta, device=emb.device)
    with torch.no_grad():
        out = gpu(inputs_embeds=emb[tok].view(1, 1, -1), position_ids=rp, past_key_values=cache, use_cache=True,
                  cache_position=torch.tensor([p], device=emb.device))
    return out.last_hidden_state.clone()


def _run(gpu, cache, emb, S, n, lookahead):
    import optimized_layer

    prev = optimized_layer.set_decode_layer_lookahead(lookahead)
    try:
        outs = [_step(gpu, cache, emb, 7 + i, S + i) for i in range(n)]
    finally:
        optimized_layer.set_decode_layer_lookahead(prev)
    torch.cuda.synchronize()
    return outs


def test_lookahead_equals_per_layer_launches_eager(cuda):
    import optimized_layer

    S, n = 700, 4
    gpu, cache, emb = _model_and_cache(cuda, S, n + 2)
    snap = _snapshot(cache)
    ref = _run(gpu, cache, emb, S, n, lookahead=False)
    ref_rows = [(L.keys[:, :, S:S + n].clone(), L.values[:, :, S:S + n].clone()) for L in cache.layers]
    _restore(cache, snap)
    for L in gpu.layers:
        L._full_layer_workspace.clear()
    got = _run(gpu, cache, emb, S, n, lookahead=True)
    stack = gpu.layers[0]._stack
    assert stack.out is not None and stack.out.shape == (N_LAYERS, 2048)
    # the later layers never launched on their own
    assert all("out" not in L._full_layer_workspace for L in gpu.layers[1:])
    for i, (a, b) in enumerate(zip(ref, got)):
        assert torch.equal(a, b), f"step {i}: look-ahead output differs from per-layer launches"
    for li, (L, (k, v)) in enumerate(zip(cache.layers, ref_rows)):
        assert torch.equal(L.keys[:, :, S:S + n], k) and torch.equal(L.values[:, :, S:S + n], v), f"layer {li}"
        assert int(L.cumulative_length) == S + n
    optimized_layer.check_decode_status(gpu)


def test_lookahead_falls_back_with_a_hook(cuda):
    S, n = 300, 2
    gpu, cache, emb = _model_and_cache(cuda, S, n + 2)
    snap = _snapshot(cache)
    ref = _run(gpu, cache, emb, S, n, lookahead=False)
    _restore(cache, snap)
    seen = []
    handle = gpu.layers[1].register_forward_hook(lambda mod, args, out: seen.append(1))
    try:
        for L in gpu.layers:
            L._full_layer_workspace.clear()
        got = _run(gpu, cache, emb, S, n, lookahead=True)
    finally:
        handle.remove()
    assert len(seen) == n
    # no stack launch: every layer ran its own
    assert all("out" in L._full_layer_workspace for L in gpu.layers)
    for a, b in zip(ref, got):
        assert torch.equal(a, b)


def test_lookahead_in_a_captured_graph(cuda):
    """One decode step with the look-ahead on, captured and replayed at four
    positions with the static inputs rewritten on the device: every replay's
    output and K/V rows equal the eager per-layer launches' at that position."""
    import optimized_layer

    S, n = 1100, 4
    gpu, cache, emb = _model_and_cache(cuda, S, n + 2)
    snap = _snapshot(cache)
    ref = _run(gpu, cache, emb, S, n, lookahead=False)
    ref_rows = [(L.keys[:, :, S:S + n].clone(), L.values[:, :, S:S + n].clone()) for L in cache.layers]
    _restore(cache, snap)

    x = torch.empty(1, 1, 2048, dtype=torch.float16, device=cuda)
    rp = torch.empty(3, 1, 1, dtype=torch.int64, device=cuda)
    cp = torch.empty(1, dtype=torch.int64, device=cuda)

    def write(i):
        x.copy_(emb[7 + i].view(1, 1, -1))
        rp.fill_(S + i - 5)
        cp.fill_(S + i)

    def run():
        with torch.no_grad():
            return gpu(inputs_embeds=x, position_ids=rp, past_key_values=cache, use_cache=True,
                       cache_position=cp).last_hidden_state

    prev = optimized_layer.set_decode_layer_lookahead(True)
    try:
        write(0)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            run()                      # lazy initialisation (buffers, the hand-off area) outside capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        _restore(cache, snap)
        write(0)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = run()
        _restore(cache, snap)
        for i in range(n):
            write(i)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref[i]), f"graph replay {i} differs from per-layer launches"
    finally:
        optimized_layer.set_decode_layer_lookahead(prev)
    for li, (L, (k, v)) in enumerate(zip(cache.layers, ref_rows)):
        assert torch.equal(L.keys[:, :, S:S + n], k) and torch.equal(L.values[:, :, S:S + n], v), f"layer {li}"
    optimized_layer.check_decode_status(gpu)
