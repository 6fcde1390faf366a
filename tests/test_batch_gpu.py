"""Batch decoding (config 4 shape: up to 8 sequences, ragged cache positions)
on the GPU against the oracle.

* the MFMA batch GEMV (qkv / o_proj / gate_up / down shapes, RMSNorm prologue,
  residual and SiLU*up epilogues, 8 and 5 live sequences) against the oracle's
  fp32 GEMV per sequence;
* a 2-layer batch step (real vocabulary tail cut to 8192) with ragged cache
  positions: logits, greedy tokens and the written K/V rows against the
  oracle's per-sequence batch-1 steps, eager and as graph replays;
* the full 28-layer model, 8 sequences, two steps: tokens and logits against
  the oracle.
"""

from __future__ import annotations

import types

import pytest
import torch

from conftest import assert_close_rel
from oracle import qwen3vl_oracle as O

pytestmark = pytest.mark.gpu


def _gemv(x, W, gamma, residual, nseq, epi, up_offset, cuda):
    from qwen3vl_hip import _lib

    N = up_offset if epi == 1 else W.shape[0]
    K = W.shape[1]
    xd = x.to(cuda).contiguous()
    Wd = W.to(cuda).contiguous()
    gd = gamma.to(cuda).contiguous() if gamma is not None else None
    rd = residual.to(cuda).contiguous() if residual is not None else None
    y = torch.full((8, N), float("nan"), dtype=torch.float32, device=cuda)
    nws = _lib.lib().qd_batch_gemv_workspace_bytes(N, K)
    ws = torch.zeros(nws, dtype=torch.uint8, device=cuda)
    for _ in range(2):   # the second call runs on counters the first one reset
        _lib.check(_lib.lib().qd_batch_gemv(
            _lib.ptr(xd), K, _lib.ptr(gd), ctypes_float(1e-6), _lib.ptr(Wd), K, N, K, up_offset, _lib.ptr(rd),
            N, _lib.ptr(y), N, nseq, epi, _lib.ptr(ws), nws, _lib.stream()), "qd_batch_gemv")
    torch.cuda.synchronize()
    return y.cpu()


def ctypes_float(v):
    import ctypes

    return ctypes.c_float(v)


@pytest.mark.parametrize("name,N,K,norm,resid,silu", [
    ("qkv", 4096, 2048, True, False, False),
    ("o_proj", 2048, 2048, False, True, False),
    ("gate_up", 6144, 2048, True, False, True),
    ("down", 2048, 6144, False, True, False),
])
@pytest.mark.parametrize("nseq", [8, 5])
def test_batch_gemv_matches_oracle(cuda, name, N, K, norm, resid, silu, nseq):
    from qwen3vl_hip import synthetic as syn

    print(f"case batch gemv {name} nseq={nseq}", flush=True)
    rows = 2 * N if silu else N
    sid = {"qkv": 1, "o_proj": 2, "gate_up": 3, "down": 4}[name]
    W = syn.normal(31, ("W", sid), (rows, K), std=0.02)
    x = syn.normal(31, ("x", sid), (8, K), dtype=torch.float32)
    x[3] *= 40.0      # a row with large values: the rounding residual must carry it
    gamma = syn.normal(31, ("input_layernorm", sid), (K,), std=0.02, mean=1.0) if norm else None
    residual = syn.normal(31, ("residual", sid), (8, N), dtype=torch.float32) if resid else None
    y = _gemv(x, W, gamma, residual, nseq, 1 if silu else 0, N if silu else 0, cuda)
    for b in range(8):
        if b >= nseq:
            assert torch.isnan(y[b]).all(), "rows beyond nseq must not be written"
            continue
        xb = O.rms_norm(x[b], gamma, 1e-6) if norm else x[b]
        ref = O.gemv(xb, W)
        if silu:
            ref = O.silu_mul(ref[:N], ref[N:])
        if resid:
            ref = ref + residual[b]
        assert_close_rel(y[b], ref, rel=1e-4, what=f"batch gemv {name} seq {b}")


def test_batch_gemv_rejects_bad_shapes(cuda):
    from qwen3vl_hip import _lib

    z = torch.zeros(8, 1024, device=cuda)
    W = torch.zeros(64, 1024, dtype=torch.float16, device=cuda)
    y = torch.zeros(8, 64, device=cuda)
    nws = _lib.lib().qd_batch_gemv_workspace_bytes(64, 2048)
    ws = torch.zeros(nws, dtype=torch.uint8, device=cuda)
    st = _lib.lib().qd_batch_gemv(_lib.ptr(z), 1024, None, ctypes_float(1e-6), _lib.ptr(W), 1024, 64, 1024, 0, None,
                                  64, _lib.ptr(y), 64, 8, 0, _lib.ptr(ws), nws, _lib.stream())
    assert st != 0 and "K in" in _lib.last_error()
    st = _lib.lib().qd_batch_gemv(_lib.ptr(z), 1024, None, ctypes_float(1e-6), _lib.ptr(W), 1024, 64, 2048, 0, None,
                                  64, _lib.ptr(y), 64, 9, 0, _lib.ptr(ws), nws, _lib.stream())
    assert st != 0 and "nseq" in _lib.last_error()
    st = _lib.lib().qd_batch_gemv(_lib.ptr(z), 1024, None, ctypes_float(1e-6), _lib.ptr(W), 1024, 64, 2048, 0, None,
                                  64, _lib.ptr(y), 64, 8, 0, _lib.ptr(ws), 256, _lib.stream())
    assert st != 0 and "workspace" in _lib.last_error()


VOCAB = 8192


@pytest.fixture(scope="module")
def two_layer_weights():
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.config import Qwen3VLTextShape

    return syn.model_weights(17, shape=Qwen3VLTextShape(num_layers=2, vocab=VOCAB))


def _fill_caches(eng, positions, seed):
    from qwen3vl_hip import synthetic as syn

    cap = eng.capacity
    caches = []
    for li, (kc, vc) in enumerate(zip(eng.k_caches, eng.v_caches)):
        k = torch.full((eng.batch, 8, cap, 128), 3.0, dtype=torch.float16)
        v = torch.full((eng.batch, 8, cap, 128), -3.0, dtype=torch.float16)
        for b, p in enumerate(positions):
            if p:
                k[b, :, :p] = syn.normal(seed, ("k", li, b), (8, p, 128))
                v[b, :, :p] = syn.normal(seed, ("v", li, b), (8, p, 128))
        kc.copy_(k)
        vc.copy_(v)
        caches.append((k, v))
    return caches


@pytest.mark.parametrize("positions", [[5, 17, 0, 63, 100, 33, 1, 77],
                                       [127, 0, 126, 64, 1, 2, 120, 31]])   # last cache row, empty prefix
def test_batch_step_two_layers_matches_oracle(cuda, two_layer_weights, positions):
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    rope = [p + 11 for p in positions]
    tokens = [123, 4000, 7, 8191, 55, 1024, 2048, 3]
    eng = BatchDecodeEngine(w, batch=8, capacity=128, keep_logits=True)
    caches = _fill_caches(eng, positions, 19)
    out = eng.decode(tokens, positions, rope, 1, use_graph=False)
    ref_caches = [(k.clone(), v.clone()) for k, v in caches]
    logits, toks = O.decode_step_batch(w, tokens, ref_caches, positions, rope, shape=O.OracleShape(num_layers=2,
                                                                                                    vocab=VOCAB))
    assert_close_rel(eng.logits.cpu(), logits, what="batch step logits")
    for li in range(2):
        for b, p in enumerate(positions):
            assert_close_rel(eng.k_caches[li][b, :, p].cpu(), ref_caches[li][0][b, :, p].float(),
                             what=f"K row layer {li} seq {b}")
            mask = torch.ones(128, dtype=torch.bool)
            mask[p] = False
            assert torch.equal(eng.k_caches[li][b, :, mask].cpu(), caches[li][0][b, :, mask])
    print(f"gpu {out[0]} oracle {toks}", flush=True)
    assert out[0] == toks


@pytest.mark.parametrize("fuse_advance", [True, False])
def test_batch_graph_generation_matches_oracle(cuda, two_layer_weights, fuse_advance):
    """Graph replays of 12 steps; the advance fused into the argmax reduction
    or run as qd_decode_advance_batch after it."""
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    positions = [40, 3, 90, 12, 64, 27, 100, 8]
    tokens = [11, 22, 33, 44, 55, 66, 77, 88]
    n = 12
    eng = BatchDecodeEngine(w, batch=8, capacity=128, fuse_advance=fuse_advance)
    caches = _fill_caches(eng, positions, 23)
    got = eng.decode(tokens, positions, positions, n, use_graph=True)
    assert eng.cache_position.tolist() == [p + n for p in positions]
    assert eng.rope_position.tolist() == [[p + n] * 3 for p in positions]
    assert int(eng.step_counter.item()) == n
    ref_caches = [(k.clone(), v.clone()) for k, v in caches]
    cur, pos, ref = list(tokens), list(positions), []
    for _ in range(n):
        _, cur = O.decode_step_batch(w, cur, ref_caches, pos, pos, shape=O.OracleShape(num_layers=2, vocab=VOCAB))
        ref.append(list(cur))
        pos = [p + 1 for p in pos]
    print(f"gpu {got}\noracle {ref}", flush=True)
    assert got == ref


def test_batch_step_partial_batch(cuda, two_layer_weights):
    """Batch 3: only three sequences are stepped."""
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    positions = [7, 50, 21]
    tokens = [100, 200, 300]
    eng = BatchDecodeEngine(w, batch=3, capacity=64, keep_logits=True)
    caches = _fill_caches(eng, positions, 29)
    out = eng.decode(tokens, positions, positions, 1, use_graph=False)
    ref_caches = [(k.clone(), v.clone()) for k, v in caches]
    logits, toks = O.decode_step_batch(w, tokens, ref_caches, positions, positions,
                                       shape=O.OracleShape(num_layers=2, vocab=VOCAB))
    assert_close_rel(eng.logits.cpu(), logits, what="batch-3 logits")
    assert out[0] == toks


def test_batch_full_model_two_steps(cuda):
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = syn.model_weights(3, device=cuda)
    positions = [150, 37, 220, 96, 5, 180, 64, 128]
    tokens = [99327, 74931, 74000, 12, 98789, 41501, 65727, 146052]
    eng = BatchDecodeEngine(w, batch=8, capacity=256, keep_logits=True)
    caches = _fill_caches(eng, positions, 31)
    got = eng.decode(tokens, positions, positions, 2, use_graph=True)
    gpu_logits = eng.logits.cpu()
    f32 = types.SimpleNamespace(
        embed_tokens=w.embed_tokens.float().cpu(), final_norm_weight=w.final_norm_weight.float().cpu(),
        layers=[{k: v.float().cpu() for k, v in lw.tensors().items()} for lw in w.layers])
    ref_caches = [(k.clone(), v.clone()) for k, v in caches]
    cur, pos, ref, logits = list(tokens), list(positions), [], None
    for _ in range(2):
        logits, cur = O.decode_step_batch(f32, cur, ref_caches, pos, pos)
        ref.append(list(cur))
        pos = [p + 1 for p in pos]
    assert_close_rel(gpu_logits, logits, what="28-layer batch logits (second step)")
    print(f"gpu {got}\noracle {ref}", flush=True)
    assert got == ref


def _fill_caches_device(eng, positions, seed):
    """Random K/V prefixes [0, p) drawn on the device (seeded), stale rows past
    them set to +-3 (an over-read changes the result); returns host copies."""
    gen = torch.Generator(device=eng.device).manual_seed(seed)
    caches = []
    for kc, vc in zip(eng.k_caches, eng.v_caches):
        kc.fill_(3.0)
        vc.fill_(-3.0)
        for b, p in enumerate(positions):
            kc[b, :, :p].normal_(generator=gen)
            vc[b, :, :p].normal_(generator=gen)
        caches.append((kc.cpu(), vc.cpu()))
    return caches


def test_batch_two_layers_config4_lengths(cuda, two_layer_weights):
    """Config-4 KV lengths (the seeded U[2048, 4096] draw, 2273..4067) on a
    2-layer model: 8 splits per kv head of up to 509 rows, so every split walks
    four batches of K/V rows (two loop trips), each sequence at its own
    position.  Two graph-replayed steps: tokens of both, the second step's
    logits, and the K/V rows both steps wrote."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    positions = [int(v) for v in syn.batch8_kv_lengths()]
    assert min(positions) >= 2048 and max(positions) <= 4096
    tokens = [17, 4000, 8191, 2, 555, 1234, 6000, 42]
    cap = max(positions) + 4
    eng = BatchDecodeEngine(w, batch=8, capacity=cap, keep_logits=True)
    caches = _fill_caches_device(eng, positions, 41)
    got = eng.decode(tokens, positions, positions, 2, use_graph=True)
    ref_caches = [(k.clone(), v.clone()) for k, v in caches]
    cur, pos, ref, logits = list(tokens), list(positions), [], None
    shape = O.OracleShape(num_layers=2, vocab=VOCAB)
    for _ in range(2):
        logits, cur = O.decode_step_batch(w, cur, ref_caches, pos, pos, shape=shape)
        ref.append(list(cur))
        pos = [p + 1 for p in pos]
    assert_close_rel(eng.logits.cpu(), logits, what="2-layer batch logits at config-4 lengths (second step)")
    for li in range(2):
        for b, p in enumerate(positions):
            assert_close_rel(eng.k_caches[li][b, :, p:p + 2].cpu(), ref_caches[li][0][b, :, p:p + 2].float(),
                             what=f"K rows layer {li} seq {b}")
            assert torch.equal(eng.k_caches[li][b, :, p + 2:].cpu(), caches[li][0][b, :, p + 2:])
    print(f"gpu {got}\noracle {ref}", flush=True)
    assert got == ref


def test_batch_full_model_config4_lengths(cuda):
    """Config 4 at its own workload: the full 28-layer model, 8 sequences at the
    seeded config-4 KV lengths (2273..4067) with random K/V prefixes, eight
    graph-replayed steps (two replays of the 4-step graph) against the
    oracle's batch step (which is pinned per sequence against transformers):
    every step's tokens and the last step's logits (bar 2e-3 * max|ref|)."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = syn.model_weights(3, device=cuda)
    positions = [int(v) for v in syn.batch8_kv_lengths()]
    tokens = [int(t) for t in syn.randint(4, ("text_ids",), (8,), 0, w.shape.vocab)]
    n_steps = 8
    eng = BatchDecodeEngine(w, batch=8, capacity=max(positions) + n_steps + 2, keep_logits=True)
    caches = _fill_caches_device(eng, positions, 43)
    print("case config4 28 layers: GPU steps", flush=True)
    got = eng.decode(tokens, positions, positions, n_steps, use_graph=True)
    gpu_logits = eng.logits.cpu()
    del eng
    f32 = types.SimpleNamespace(
        embed_tokens=w.embed_tokens.float().cpu(), final_norm_weight=w.final_norm_weight.float().cpu(),
        layers=[{k: v.float().cpu() for k, v in lw.tensors().items()} for lw in w.layers])
    cur, pos, ref, logits, margins = list(tokens), list(positions), [], None, []
    for step in range(n_steps):
        print(f"case config4 28 layers: oracle step {step}", flush=True)
        logits, cur = O.decode_step_batch(f32, cur, caches, pos, pos)
        ref.append(list(cur))
        margins.append([round(O.top2_margin(r), 5) for r in logits])
        pos = [p + 1 for p in pos]
    print(f"gpu {got}\noracle {ref}\nmargins {margins}", flush=True)
    assert_close_rel(gpu_logits, logits, what=f"28-layer batch logits at config-4 lengths (step {n_steps - 1})")
    assert got == ref


@pytest.mark.parametrize("batch", [8, 3])
def test_batch_qkv_in_attention_launch_equals_two_launches(cuda, two_layer_weights, batch):
    """The batch step's qkv GEMV inside the attention launch (the default,
    parity-tagged hand-off to the attention workgroups) against the same step
    with the GEMV as a launch of its own, at config-4 lengths: three
    graph-replayed steps, tokens equal, logits and written K/V rows within the
    kernels' tolerance, status word clear.  Batch 3 (19 splits per sequence,
    456 workgroups) leaves the producers' rows of sequences 3..7 unwritten."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    positions = [int(v) for v in syn.batch8_kv_lengths()][:batch]
    tokens = [17, 4000, 8191, 2, 555, 1234, 6000, 42][:batch]
    cap = max(positions) + 8
    res = {}
    for fuse in (True, False):
        print(f"case batch {batch} qkv fusion={fuse}", flush=True)
        eng = BatchDecodeEngine(w, batch=batch, capacity=cap, keep_logits=True, fuse_qkv=fuse)
        _fill_caches_device(eng, positions, 43)
        got = eng.decode(tokens, positions, positions, 3, use_graph=True)
        rows = [(eng.k_caches[li][:, :, min(positions):max(positions) + 3].cpu(),
                 eng.v_caches[li][:, :, min(positions):max(positions) + 3].cpu()) for li in range(2)]
        res[fuse] = (got, eng.logits.cpu(), rows, eng.status())
        del eng
    (g1, l1, r1, s1), (g0, l0, r0, s0) = res[True], res[False]
    assert s1 == 0 and s0 == 0
    print(f"fused {g1}\ntwo launches {g0}", flush=True)
    assert_close_rel(l1, l0, what="batch logits, qkv in the attention launch vs its own launch")
    for li in range(2):
        assert_close_rel(r1[li][0].float(), r0[li][0].float(), what=f"K rows layer {li}")
        assert_close_rel(r1[li][1].float(), r0[li][1].float(), what=f"V rows layer {li}")
    assert g1 == g0


def test_batch_partial_batch_qkv_in_attention_launch_matches_oracle(cuda, two_layer_weights):
    """Batch 3 at the first three config-4 lengths, qkv GEMV inside the
    attention launch (456 workgroups): one step against the oracle's."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    positions = [int(v) for v in syn.batch8_kv_lengths()][:3]
    tokens = [100, 8000, 300]
    eng = BatchDecodeEngine(w, batch=3, capacity=max(positions) + 8, keep_logits=True)
    caches = _fill_caches_device(eng, positions, 31)
    print(f"case batch 3 fused qkv at {positions}", flush=True)
    out = eng.decode(tokens, positions, positions, 1, use_graph=False)
    assert eng.status() == 0
    logits, toks = O.decode_step_batch(w, tokens, caches, positions, positions,
                                       shape=O.OracleShape(num_layers=2, vocab=VOCAB))
    assert_close_rel(eng.logits.cpu(), logits, what="batch-3 logits, qkv in the attention launch")
    assert out[0] == toks


@pytest.mark.parametrize("batch,capacity", [(8, 128), (3, 4096)])
def test_batch_qkv_hand_off_exhausted_wait_is_reported(cuda, two_layer_weights, batch, capacity):
    """With a one-poll budget the qkv hand-off's waits run out: the status word
    reports it (which also shows that the step ran the hand-off: at batch 8 and
    128 rows the grid has 256 workgroups, at batch 3 and 4096 rows 504), and
    the next step with the default budget is unaffected."""
    from qwen3vl_hip import _lib
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    positions = [5, 17, 0, 63, 100, 33, 1, 77][:batch]
    tokens = [123, 4000, 7, 8191, 55, 1024, 2048, 3][:batch]
    eng = BatchDecodeEngine(w, batch=batch, capacity=capacity, keep_logits=True)

    def run():
        _fill_caches(eng, positions, 19)
        eng.decode(tokens, positions, positions, 1, use_graph=False)
        torch.cuda.synchronize()
        return eng.logits.cpu().clone(), eng.status()

    ref, st = run()
    assert st == 0
    lib = _lib.lib()
    print("case batch step with a one-poll budget", flush=True)
    _lib.check(lib.qd_persistent_set_spin_limit(1), "qd_persistent_set_spin_limit")
    try:
        _, st_bad = run()
    finally:
        _lib.check(lib.qd_persistent_set_spin_limit(0), "qd_persistent_set_spin_limit")
    assert st_bad & 1, "a batch step with a one-poll budget reported no exhausted wait"
    again, st = run()
    assert st == 0
    assert torch.equal(again, ref)


@pytest.mark.parametrize("fuse", [True, False])
def test_batch_tile_ordered_weights_equal_row_major(cuda, two_layer_weights, fuse):
    """qkv, o_proj, gate_up and down read from tile-ordered copies (the default)
    against the row-major weights: the MFMA operands are the same values in
    the same order, so logits, tokens and written K/V rows are bit-equal
    (three graph-replayed steps at config-4 lengths; both qkv forms)."""
    from qwen3vl_hip import synthetic as syn
    from qwen3vl_hip.engine import BatchDecodeEngine

    w = two_layer_weights
    positions = [int(v) for v in syn.batch8_kv_lengths()]
    tokens = [17, 4000, 8191, 2, 555, 1234, 6000, 42]
    cap = max(positions) + 8
    res = {}
    for tiled in (True, False):
        print(f"case batch tile-ordered weights={tiled} fuse_qkv={fuse}", flush=True)
        eng = BatchDecodeEngine(w, batch=8, capacity=cap, keep_logits=True, fuse_qkv=fuse, tiled_weights=tiled)
        assert bool(eng.tiled) == tiled
        _fill_caches_device(eng, positions, 47)
        got = eng.decode(tokens, positions, positions, 3, use_graph=True)
        rows = [eng.k_caches[li][:, :, min(positions):max(positions) + 3].cpu() for li in range(2)]
        res[tiled] = (got, eng.logits.cpu(), rows, eng.status())
        del eng
    (g1, l1, r1, s1), (g0, l0, r0, s0) = res[True], res[False]
    assert s1 == 0 and s0 == 0
    assert g1 == g0
    assert torch.equal(l1, l0)
    for a, b in zip(r1, r0):
        assert torch.equal(a, b)
