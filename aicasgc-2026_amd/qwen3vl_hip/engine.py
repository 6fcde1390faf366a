"""Batch-1 greedy decode engine for the Qwen3-VL-2B text decoder on one MI355X.

The hot path is one call of the native ``qd_decode_step`` (embedding row,
28 layers of HIP kernels, final norm, lm_head + argmax) followed by
``qd_decode_advance`` (append the token, advance cache/rope positions on the
device).  Both are captured once into a HIP graph (``torch.cuda.CUDAGraph``),
and 2, 4 and 8 consecutive steps into further graphs; generation is a loop of
graph replays with no host writes in between.

Mirrors the reference's decode engine: GreedyDecodeEngine.generate
(evaluation_wrapper.py:149-315) and DecodeCudaGraphRunner
(evaluation_wrapper.py:747-1005: static input buffers, graph prebuild and
replay).  The prefill that fills the static KV cache
(evaluation_wrapper.py:218-228, a full HF forward in the reference) runs here
as plain PyTorch-ROCm ops in fp32; it is not part of the decode step.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .config import QWEN3VL_2B, Qwen3VLTextShape
from .synthetic import ModelWeights, MultimodalPrompt


def rope_inv_freq(shape: Qwen3VLTextShape = QWEN3VL_2B) -> torch.Tensor:
    """inv_freq[j] = 1 / theta^(2j/d) in fp32, the same expression HF evaluates
    (transformers modeling_qwen3_vl.py:340-342)."""
    d = shape.head_dim
    return 1.0 / (shape.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))


class _CapturedSteps:
    """HIP-graph capture shared by the engines: one step (``step_eager``:
    decode + advance) in one graph, and k consecutive steps in one graph for
    every power of two k up to ``steps_per_graph``.  Each step reads the token
    and positions the previous step's advance wrote on the device, so k steps
    replay as one graph launch; n steps take one replay per set bit of n (at
    most steps_per_graph steps per replay), and each replay's launch gap (a
    single-step replay costs ~8 us more than a step inside a longer graph) is
    paid once per replay."""

    def _state_tensors(self):
        return (self.token, self.cache_position, self.rope_position, self.step_counter)

    def capture(self) -> None:
        # Warm up once on a side stream so lazy initialisation is not captured,
        # restoring the device state (positions, counter, the cache rows the
        # warm-up step wrote) afterwards.
        saved = [t.clone() for t in self._state_tensors()]
        snap = self._snapshot()
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.step_eager()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        for t, v in zip(self._state_tensors(), saved):
            t.copy_(v)
        self._restore(snap)
        self.graphs = {}
        k = 1
        while k <= self.steps_per_graph:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(k):
                    self.step_eager()
            torch.cuda.synchronize(self.device)
            self.graphs[k] = g
            k *= 2
        self.graph = self.graphs[1]
        top = max(self.graphs)
        self.graph_multi = self.graphs[top] if top > 1 else None

    def warm_graphs(self, rounds: int = 6) -> None:
        """Replay every captured graph once, then the longest one ``rounds`` - 1
        more times, each time putting the step state (token, positions, step
        counter) back, so later timed replays start warm: on MI355X the first
        ~40 ms of decoding after an idle host sync run ~2% slower per step
        (clocks ramping up).  The K/V rows those steps wrote lie at or after the
        current position, and each is rewritten by its own step before any
        step reads it."""
        if self.graph is None:
            self.capture()
        saved = [t.clone() for t in self._state_tensors()]
        order = list(self.graphs.values()) + [self.graphs[max(self.graphs)]] * max(0, rounds - 1)
        for g in order:
            g.replay()
            for t, v in zip(self._state_tensors(), saved):
                t.copy_(v)
        torch.cuda.synchronize(self.device)

    def replay_steps(self, n: int) -> None:
        """Enqueue n captured steps: replays of the largest graph, then one
        replay per remaining set bit of n (20 = 8 + 8 + 4)."""
        if self.graph is None:
            self.capture()
        while n > 0:
            k = max(k for k in self.graphs if k <= n)
            self.graphs[k].replay()
            n -= k


class DecodeEngine(_CapturedSteps):
    """Owns device weights, the static KV cache and the captured decode step."""

    STEP_MODES = {"auto": _lib.STEP_AUTO, "chain": _lib.STEP_CHAIN, "persistent": _lib.STEP_PERSISTENT}

    def __init__(self, weights: ModelWeights, capacity: int, device="cuda", attn_splits: int = 0,
                 keep_logits: bool = False, step_mode: str = "auto", steps_per_graph: int = 8,
                 fuse_advance: bool = True, argmax_f16_logits: bool = False):
        if not torch.cuda.is_available():
            raise RuntimeError("DecodeEngine needs a ROCm GPU")
        if steps_per_graph < 1:
            raise ValueError("steps_per_graph must be >= 1")
        self.steps_per_graph = int(steps_per_graph)
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.shape = weights.shape
        s = self.shape
        self.capacity = int(capacity)
        self.w = weights if weights.embed_tokens.device == self.device else weights.to(self.device)
        self.k_caches = [torch.zeros(1, s.num_kv_heads, self.capacity, s.head_dim, dtype=torch.float16,
                                     device=self.device) for _ in self.w.layers]
        self.v_caches = [torch.zeros_like(k) for k in self.k_caches]
        dev = self.device
        self.token = torch.zeros(1, dtype=torch.int64, device=dev)
        self.cache_position = torch.zeros(1, dtype=torch.int64, device=dev)
        self.rope_position = torch.zeros(3, dtype=torch.int64, device=dev)
        self.step_counter = torch.zeros(1, dtype=torch.int64, device=dev)
        self.out_tokens = torch.zeros(1, dtype=torch.int64, device=dev)
        self.inv_freq = rope_inv_freq(s).to(dev)
        self.logits = torch.empty(s.vocab, dtype=torch.float16, device=dev) if keep_logits else None

        layers = (_lib.LayerDesc * len(self.w.layers))()
        for i, lw in enumerate(self.w.layers):
            L = layers[i]
            L.qkv = lw.qkv_weight.data_ptr()
            L.o_proj = lw.o_proj_weight.data_ptr()
            L.gate_up = lw.gate_up_weight.data_ptr()
            L.down = lw.down_proj_weight.data_ptr()
            L.input_norm = lw.input_layernorm_weight.data_ptr()
            L.post_norm = lw.post_attn_layernorm_weight.data_ptr()
            L.q_norm = lw.q_norm_weight.data_ptr()
            L.k_norm = lw.k_norm_weight.data_ptr()
            L.k_cache = self.k_caches[i].data_ptr()
            L.v_cache = self.v_caches[i].data_ptr()
        self._layers = layers
        d = _lib.ModelDesc()
        d.num_layers = len(self.w.layers)
        d.hidden, d.num_heads, d.num_kv_heads = s.hidden, s.num_heads, s.num_kv_heads
        d.head_dim, d.intermediate, d.vocab = s.head_dim, s.intermediate, s.vocab
        d.capacity = self.capacity
        d.eps = s.rms_eps
        d.sec_t, d.sec_h, d.sec_w = s.mrope_section
        d.inv_freq = self.inv_freq.data_ptr()
        d.layers = ctypes.cast(layers, ctypes.POINTER(_lib.LayerDesc))
        d.embed = self.w.embed_tokens.data_ptr()
        d.final_norm = self.w.final_norm_weight.data_ptr()
        d.token = self.token.data_ptr()
        d.cache_position = self.cache_position.data_ptr()
        d.rope_position = self.rope_position.data_ptr()
        d.logits_out = self.logits.data_ptr() if self.logits is not None else None
        d.attn_splits = int(attn_splits)
        d.step_mode = self.STEP_MODES[step_mode]
        d.argmax_f16_logits = int(bool(argmax_f16_logits))
        nbytes = _lib.lib().qd_decode_workspace_bytes(ctypes.byref(d))
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        d.workspace = self.workspace.data_ptr()
        self.desc = d
        self.graph = None
        self.graph_multi = None
        self.graphs = {}
        self._graph_max_tokens = 0
        if fuse_advance:
            self._bind_advance()

    @property
    def step_mode(self) -> str:
        """The mode qd_decode_step runs in on this device ("chain" or "persistent")."""
        with torch.cuda.device(self.device):   # the library's per-device state follows the current device
            m = _lib.lib().qd_decode_step_mode(ctypes.byref(self.desc))
        if m < 0:
            _lib.check(m, "qd_decode_step_mode")
        return "persistent" if m == _lib.STEP_PERSISTENT else "chain"

    def status(self, reset: bool = True) -> int:
        """Persistent-step status word (0: every hand-off completed)."""
        v = ctypes.c_uint(0)
        _lib.check(_lib.lib().qd_decode_status(ctypes.byref(self.desc), ctypes.byref(v), int(reset)),
                   "qd_decode_status")
        return int(v.value)

    def layers_persistent(self) -> None:
        """Enqueue embedding + all layers as one persistent launch (x left in buffers()["x"])."""
        st = torch.cuda.current_stream(self.device).cuda_stream
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().qd_decode_layers_persistent(ctypes.byref(self.desc), ctypes.c_void_p(st)),
                       "qd_decode_layers_persistent")

    # ------------------------------------------------------------ state
    def set_state(self, token: int, cache_position: int, rope_position: int) -> None:
        self.token.fill_(int(token))
        self.cache_position.fill_(int(cache_position))
        self.rope_position.fill_(int(rope_position))

    def reserve_tokens(self, n: int) -> None:
        if self.out_tokens.numel() < n:
            self.out_tokens = torch.zeros(n, dtype=torch.int64, device=self.device)
            self.graph = None  # the captured advance points at the old buffer
            self.graph_multi = None
            self.graphs = {}
            self._bind_advance()

    def _bind_advance(self) -> None:
        """The step ends with the position advance, fused into its last kernel."""
        d = self.desc
        d.advance_out_tokens = self.out_tokens.data_ptr()
        d.advance_counter = self.step_counter.data_ptr()
        d.advance_max_tokens = int(self.out_tokens.numel())

    # ------------------------------------------------------------ step
    def step_eager(self) -> None:
        """Enqueue one decode step + advance on the current stream."""
        st = torch.cuda.current_stream(self.device).cuda_stream
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().qd_decode_step(ctypes.byref(self.desc), ctypes.c_void_p(st)), "qd_decode_step")
        if self.desc.advance_counter:
            return
        _lib.check(_lib.lib().qd_decode_advance(
            ctypes.c_void_p(self.token.data_ptr()), ctypes.c_void_p(self.out_tokens.data_ptr()),
            ctypes.c_void_p(self.step_counter.data_ptr()), ctypes.c_void_p(self.cache_position.data_ptr()),
            ctypes.c_void_p(self.rope_position.data_ptr()), int(self.out_tokens.numel()),
            ctypes.c_void_p(st)), "qd_decode_advance")

    def run_phases(self, phases, first_layer: int = 0, n_layers: int | None = None) -> None:
        """Enqueue only the named phases of the step (timing / profiling one kernel)."""
        mask = 0
        for p in phases:
            mask |= _lib.PHASE[p]
        n = len(self.w.layers) if n_layers is None else n_layers
        st = torch.cuda.current_stream(self.device).cuda_stream
        _lib.check(_lib.lib().qd_decode_step_phases(ctypes.byref(self.desc), int(first_layer), int(n), mask,
                                                    ctypes.c_void_p(st)), "qd_decode_step_phases")

    def buffers(self) -> dict:
        """fp32 views of the activation vectors the step hands between kernels."""
        offs = (ctypes.c_size_t * 6)()
        _lib.lib().qd_decode_workspace_layout(ctypes.byref(self.desc), offs, 6)
        s = self.shape
        sizes = {"x": s.hidden, "qkv": s.qkv_rows, "q_rot": s.q_size, "attn": s.q_size, "r": s.hidden,
                 "hidden": s.intermediate}
        return {name: self.workspace[o: o + 4 * n].view(torch.float32)
                for (name, n), o in zip(sizes.items(), offs)}

    def _snapshot(self):
        pos = int(self.cache_position.item())
        if not (0 <= pos < self.capacity):
            return None
        return pos, [(k[:, :, pos].clone(), v[:, :, pos].clone()) for k, v in zip(self.k_caches, self.v_caches)]

    def _restore(self, snap) -> None:
        if snap is None:
            return
        pos, rows = snap
        for (k, v), (kr, vr) in zip(zip(self.k_caches, self.v_caches), rows):
            k[:, :, pos].copy_(kr)
            v[:, :, pos].copy_(vr)

    def replay(self) -> None:
        if self.graph is None:
            self.capture()
        self.graph.replay()

    # ------------------------------------------------------------ generation
    def decode(self, first_token: int, start_position: int, rope_delta: int, n_steps: int,
               use_graph: bool = True, eos_token_ids=None, eos_window: int = 2) -> list:
        """Greedy decode n_steps tokens after ``first_token`` at cache row start_position.

        With ``eos_token_ids`` generation stops at the first of them (included in
        the result), detected without stalling the device: after every graph
        replay the new tokens are copied to pinned host memory behind an event,
        the host checks copies whose event has completed and blocks only when
        ``eos_window`` copies are outstanding (the reference's async EOS poll,
        evaluation_wrapper.py:317-463, :906-939).  Steps already enqueued when
        the EOS is seen still run; their tokens are dropped.
        """
        if start_position + n_steps > self.capacity:
            raise ValueError("static cache too small for the requested generation")
        self.reserve_tokens(n_steps)
        self.set_state(first_token, start_position, start_position + rope_delta)
        self.step_counter.zero_()
        if eos_token_ids is not None and n_steps > 0:
            n_out = self._decode_until_eos(n_steps, use_graph, set(int(t) for t in eos_token_ids),
                                           max(1, int(eos_window)))
            self._check_status()
            return self._host_tokens[:n_out].tolist()
        if use_graph:
            self.replay_steps(n_steps)
        else:
            for _ in range(n_steps):
                self.step_eager()
        torch.cuda.synchronize(self.device)
        self._check_status()
        return self.out_tokens[:n_steps].tolist()

    def _decode_until_eos(self, n_steps: int, use_graph: bool, eos: set, window: int) -> int:
        """Enqueue steps in chunks (one graph replay each), staging each chunk's
        tokens to pinned host memory; returns how many tokens to keep."""
        from collections import deque

        if getattr(self, "_host_tokens", None) is None or self._host_tokens.numel() < n_steps:
            self._host_tokens = torch.zeros(max(n_steps, 64), dtype=torch.int64, pin_memory=True)
        host = self._host_tokens
        if use_graph and self.graph is None:
            self.capture()
        k = self.steps_per_graph if (use_graph and self.graph_multi is not None) else 1
        stream = torch.cuda.current_stream(self.device)
        pending, done, found = deque(), 0, None
        while done < n_steps and found is None:
            chunk = min(k, n_steps - done)
            if use_graph:
                self.replay_steps(chunk)
            else:
                for _ in range(chunk):
                    self.step_eager()
            host[done:done + chunk].copy_(self.out_tokens[done:done + chunk], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(stream)
            pending.append((ev, done, chunk))
            done += chunk
            while pending and found is None and (len(pending) >= window or pending[0][0].query()):
                ev0, s0, c0 = pending.popleft()
                ev0.synchronize()
                for i in range(s0, s0 + c0):
                    if int(host[i]) in eos:
                        found = i
                        break
        torch.cuda.synchronize(self.device)
        if found is None:
            for i in range(done):
                if int(host[i]) in eos:
                    found = i
                    break
        return found + 1 if found is not None else done

    def _check_status(self) -> None:
        if self.step_mode == "persistent" and self.status(reset=True) != 0:
            # a hand-off wait ran out of its polling budget (e.g. the grid was not
            # co-resident because another process held CUs): the tokens are invalid
            raise RuntimeError("persistent decode step: a workgroup hand-off timed out; results are invalid")

    # ------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, prompt: MultimodalPrompt) -> int:
        """Causal prefill of the prompt into the static cache (fp32 PyTorch-ROCm ops).

        Follows the text-model loop of transformers Qwen3VLTextModel
        (modeling_qwen3_vl.py:769-852) with M-RoPE positions [3, S]; returns
        the argmax token of the last position.
        """
        s = self.shape
        dev = self.device
        S = prompt.length
        if S > self.capacity:
            raise ValueError("prompt longer than the static cache")
        ids = prompt.text_ids
        if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= s.vocab):
            raise ValueError(f"prompt token ids outside the vocabulary [0, {s.vocab})")
        emb = torch.cat([prompt.vision_embeds.to(dev).float(),
                         self.w.embed_tokens[prompt.text_ids.to(dev)].float()], 0)
        pos = prompt.position_ids.to(dev)
        inv = self.inv_freq
        slot_stream = torch.zeros(s.head_dim // 2, dtype=torch.long)
        for dim, off in ((1, 1), (2, 2)):
            slot_stream[off: s.mrope_section[dim] * 3: 3] = dim
        p = pos[slot_stream.to(dev), :].T.float()              # [S, d/2]
        freqs = p * inv[None, :]
        emb_f = torch.cat([freqs, freqs], -1)
        cos, sin = emb_f.cos()[:, None, :], emb_f.sin()[:, None, :]
        g = s.num_heads // s.num_kv_heads
        causal = torch.full((S, S), float("-inf"), device=dev).triu(1)
        h = emb
        for li, lw in enumerate(self.w.layers):
            xn = _rms(h, lw.input_layernorm_weight, s.rms_eps)
            qkv = xn @ lw.qkv_weight.float().T
            q = qkv[:, : s.q_size].view(S, s.num_heads, s.head_dim)
            k = qkv[:, s.q_size: s.q_size + s.kv_size].view(S, s.num_kv_heads, s.head_dim)
            v = qkv[:, s.q_size + s.kv_size:].view(S, s.num_kv_heads, s.head_dim)
            q = _rope(_rms(q, lw.q_norm_weight, s.rms_eps), cos, sin)
            k = _rope(_rms(k, lw.k_norm_weight, s.rms_eps), cos, sin)
            self.k_caches[li][0, :, :S] = k.transpose(0, 1).half()
            self.v_caches[li][0, :, :S] = v.transpose(0, 1).half()
            qh = q.transpose(0, 1).contiguous()                                      # [Hq, S, D]
            kh = k.transpose(0, 1).repeat_interleave(g, 0).contiguous()
            vh = v.transpose(0, 1).repeat_interleave(g, 0).contiguous()
            sc = torch.matmul(qh, kh.transpose(1, 2).contiguous()) * (s.head_dim ** -0.5) + causal
            attn = torch.matmul(torch.softmax(sc, -1), vh)
            o = attn.transpose(0, 1).reshape(S, s.q_size) @ lw.o_proj_weight.float().T
            r = h + o
            xn2 = _rms(r, lw.post_attn_layernorm_weight, s.rms_eps)
            gu = xn2 @ lw.gate_up_weight.float().T
            gate, up = gu[:, : s.intermediate], gu[:, s.intermediate:]
            h = r + (torch.nn.functional.silu(gate) * up) @ lw.down_proj_weight.float().T
        hn = _rms(h[-1], self.w.final_norm_weight, s.rms_eps)
        logits = hn @ self.w.embed_tokens.float().T
        return int(torch.argmax(logits))

    def generate(self, prompt: MultimodalPrompt, n_tokens: int, use_graph: bool = True, eos_token_ids=None,
                 eos_window: int = 2) -> list:
        """Prefill + greedy decode; returns n_tokens ids (the first from the
        prefill), or fewer when ``eos_token_ids`` is given and one of them is
        generated (the EOS token is the last one returned)."""
        first = self.prefill(prompt)
        if eos_token_ids is not None and first in set(int(t) for t in eos_token_ids):
            return [first]
        rest = self.decode(first, prompt.length, prompt.rope_delta, n_tokens - 1, use_graph, eos_token_ids,
                           eos_window) if n_tokens > 1 else []
        return [first] + rest


class BatchDecodeEngine(_CapturedSteps):
    """Greedy decoding of B (2..8) independent sequences per step (config 4).

    Every sequence has its own static cache rows ``[B, Hkv, T, D]`` per layer
    and its own cache / rope position, so ragged lengths need no padding.  The
    step is ``qd_decode_step`` with ``batch = B`` (MFMA batch GEMVs, per-sequence
    split-KV attention, per-sequence argmax) followed by the advance of
    ``qd_decode_advance_batch`` (done by the argmax reduction itself unless
    ``fuse_advance`` is False), captured once into a HIP graph.  With
    ``fuse_qkv`` (default) each layer's qkv GEMV runs inside its attention
    launch where the library allows it (``QD_STEP_AUTO``); False keeps two
    launches.  With ``tiled_weights`` (default) the engine keeps copies of every
    layer's qkv, o_proj, gate_up and down in the batch GEMVs' MFMA tile order
    (``qd_model_desc.batch_tiled_weights``; 101 MB per layer of the 2B model):
    each wave load is then one contiguous 1 KB that is already the MFMA
    operand, with the same results bit for bit.  The reference has no batch
    decode path (it rejects batch != 1, evaluation_wrapper.py:110-111).
    """

    def __init__(self, weights: ModelWeights, batch: int, capacity: int, device="cuda", attn_splits: int = 0,
                 keep_logits: bool = False, steps_per_graph: int = 4, fuse_advance: bool = True,
                 fuse_qkv: bool = True, tiled_weights: bool = True):
        if not torch.cuda.is_available():
            raise RuntimeError("BatchDecodeEngine needs a ROCm GPU")
        if steps_per_graph < 1:
            raise ValueError("steps_per_graph must be >= 1")
        self.steps_per_graph = int(steps_per_graph)
        if not 2 <= batch <= 8:
            raise ValueError("batch must be 2..8")
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.shape = s = weights.shape
        self.batch = B = int(batch)
        self.capacity = int(capacity)
        self.w = weights if weights.embed_tokens.device == self.device else weights.to(self.device)
        dev = self.device
        self.k_caches = [torch.zeros(B, s.num_kv_heads, self.capacity, s.head_dim, dtype=torch.float16, device=dev)
                         for _ in self.w.layers]
        self.v_caches = [torch.zeros_like(k) for k in self.k_caches]
        self.token = torch.zeros(B, dtype=torch.int64, device=dev)
        self.cache_position = torch.zeros(B, dtype=torch.int64, device=dev)
        self.rope_position = torch.zeros(B, 3, dtype=torch.int64, device=dev)
        self.step_counter = torch.zeros(1, dtype=torch.int64, device=dev)
        self.out_tokens = torch.zeros(1, B, dtype=torch.int64, device=dev)
        self.inv_freq = rope_inv_freq(s).to(dev)
        self.logits = torch.empty(B, s.vocab, dtype=torch.float32, device=dev) if keep_logits else None
        layers = (_lib.LayerDesc * len(self.w.layers))()
        self.tiled = []   # per layer (qkv, o_proj, gate_up, down) in tile order, or empty
        if tiled_weights:
            lib = _lib.lib()
            qs = s.num_heads * s.head_dim
            r_q = int(lib.qd_batch_tile_rows(qs + 2 * s.num_kv_heads * s.head_dim, s.hidden, 0))
            r_o = int(lib.qd_batch_tile_rows(s.hidden, qs, 0))
            r_gu = int(lib.qd_batch_tile_rows(s.intermediate, s.hidden, 1))
            r_d = int(lib.qd_batch_tile_rows(s.hidden, s.intermediate, 0))
            self.tiled = [(batch_tile_order(lw.qkv_weight, r_q), batch_tile_order(lw.o_proj_weight, r_o),
                           batch_tile_order(lw.gate_up_weight, r_gu), batch_tile_order(lw.down_proj_weight, r_d))
                          for lw in self.w.layers]
        for i, lw in enumerate(self.w.layers):
            L = layers[i]
            L.qkv, L.o_proj = lw.qkv_weight.data_ptr(), lw.o_proj_weight.data_ptr()
            L.gate_up, L.down = lw.gate_up_weight.data_ptr(), lw.down_proj_weight.data_ptr()
            if self.tiled:
                L.qkv, L.o_proj, L.gate_up, L.down = (x.data_ptr() for x in self.tiled[i])
            L.input_norm, L.post_norm = lw.input_layernorm_weight.data_ptr(), lw.post_attn_layernorm_weight.data_ptr()
            L.q_norm, L.k_norm = lw.q_norm_weight.data_ptr(), lw.k_norm_weight.data_ptr()
            L.k_cache, L.v_cache = self.k_caches[i].data_ptr(), self.v_caches[i].data_ptr()
        self._layers = layers
        d = _lib.ModelDesc()
        d.num_layers = len(self.w.layers)
        d.hidden, d.num_heads, d.num_kv_heads = s.hidden, s.num_heads, s.num_kv_heads
        d.head_dim, d.intermediate, d.vocab = s.head_dim, s.intermediate, s.vocab
        d.capacity = self.capacity
        d.eps = s.rms_eps
        d.sec_t, d.sec_h, d.sec_w = s.mrope_section
        d.inv_freq = self.inv_freq.data_ptr()
        d.layers = ctypes.cast(layers, ctypes.POINTER(_lib.LayerDesc))
        d.embed = self.w.embed_tokens.data_ptr()
        d.final_norm = self.w.final_norm_weight.data_ptr()
        d.token = self.token.data_ptr()
        d.cache_position = self.cache_position.data_ptr()
        d.rope_position = self.rope_position.data_ptr()
        d.logits_out = self.logits.data_ptr() if self.logits is not None else None
        d.attn_splits = int(attn_splits)
        # AUTO: each layer's qkv GEMV runs inside its attention launch where the
        # device allows it; CHAIN: two launches
        d.step_mode = _lib.STEP_AUTO if fuse_qkv else _lib.STEP_CHAIN
        d.batch = B
        d.batch_tiled_weights = 1 if self.tiled else 0
        nbytes = _lib.lib().qd_decode_workspace_bytes(ctypes.byref(d))
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        d.workspace = self.workspace.data_ptr()
        self.desc = d
        self.graph = None
        self.graph_multi = None
        self.graphs = {}
        if fuse_advance:
            self._bind_advance()

    def _bind_advance(self) -> None:
        """The step ends with the per-sequence advance, fused into its argmax reduction."""
        d = self.desc
        d.advance_out_tokens = self.out_tokens.data_ptr()
        d.advance_counter = self.step_counter.data_ptr()
        d.advance_max_tokens = int(self.out_tokens.shape[0])

    def set_state(self, tokens, cache_positions, rope_positions) -> None:
        self.token.copy_(torch.as_tensor(tokens, dtype=torch.int64))
        self.cache_position.copy_(torch.as_tensor(cache_positions, dtype=torch.int64))
        rp = torch.as_tensor(rope_positions, dtype=torch.int64).view(-1, 1).expand(self.batch, 3)
        self.rope_position.copy_(rp)

    def reserve_tokens(self, n: int) -> None:
        if self.out_tokens.shape[0] < n:
            self.out_tokens = torch.zeros(n, self.batch, dtype=torch.int64, device=self.device)
            self.graph = None
            self.graph_multi = None
            self.graphs = {}
            if self.desc.advance_counter:
                self._bind_advance()

    def step_eager(self) -> None:
        st = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        _lib.check(_lib.lib().qd_decode_step(ctypes.byref(self.desc), st), "qd_decode_step (batch)")
        if self.desc.advance_counter:
            return
        _lib.check(_lib.lib().qd_decode_advance_batch(
            ctypes.c_void_p(self.token.data_ptr()), ctypes.c_void_p(self.out_tokens.data_ptr()),
            ctypes.c_void_p(self.step_counter.data_ptr()), ctypes.c_void_p(self.cache_position.data_ptr()),
            ctypes.c_void_p(self.rope_position.data_ptr()), int(self.out_tokens.shape[0]), self.batch, st),
            "qd_decode_advance_batch")

    def status(self, reset: bool = True) -> int:
        """Status word of the batch step's hand-offs (0: every wait completed)."""
        v = ctypes.c_uint(0)
        _lib.check(_lib.lib().qd_decode_status(ctypes.byref(self.desc), ctypes.byref(v), int(reset)),
                   "qd_decode_status")
        return int(v.value)

    def _snapshot(self):
        pos = self.cache_position.tolist()
        snap = []
        for k, v in zip(self.k_caches, self.v_caches):
            snap.append([(k[b, :, p].clone(), v[b, :, p].clone()) if 0 <= p < self.capacity else None
                         for b, p in enumerate(pos)])
        return pos, snap

    def _restore(self, rows) -> None:
        pos, snap = rows
        for (k, v), per in zip(zip(self.k_caches, self.v_caches), snap):
            for b, (p, kv) in enumerate(zip(pos, per)):
                if kv is not None:
                    k[b, :, p].copy_(kv[0])
                    v[b, :, p].copy_(kv[1])

    def decode(self, first_tokens, start_positions, rope_positions, n_steps: int, use_graph: bool = True):
        """n_steps greedy steps; returns a [n_steps][B] list of token ids."""
        if max(int(p) for p in start_positions) + n_steps > self.capacity:
            raise ValueError("static cache too small for the requested generation")
        if min(int(t) for t in first_tokens) < 0 or max(int(t) for t in first_tokens) >= self.shape.vocab:
            raise ValueError("token ids outside the vocabulary")
        self.reserve_tokens(n_steps)
        self.set_state(first_tokens, start_positions, rope_positions)
        self.step_counter.zero_()
        if use_graph:
            self.replay_steps(n_steps)
        else:
            for _ in range(n_steps):
                self.step_eager()
        torch.cuda.synchronize(self.device)
        return self.out_tokens[:n_steps].tolist()


def batch_tile_order(w: torch.Tensor, rows_per_group: int) -> torch.Tensor:
    """A copy of the row-major fp16 matrix ``w`` [rows, K] in the batch GEMVs'
    MFMA tile order for row groups of ``rows_per_group`` (qd_batch_tile_rows):
    16: [rows/16][K/8][16][8]; 8: [rows/8][K/64][4][2][8][8] with element
    (g, p, c, h, r, e) = w[8 g + r][64 p + 32 h + 8 c + e]."""
    n, k = w.shape
    if rows_per_group == 16:
        return w.reshape(n // 16, 16, k // 8, 8).permute(0, 2, 1, 3).contiguous()
    if rows_per_group == 8:
        return w.reshape(n // 8, 8, k // 64, 2, 4, 8).permute(0, 2, 4, 3, 1, 5).contiguous()
    raise ValueError(f"rows per group {rows_per_group}")


def roofline_bytes_batch_step(context_lens, shape: Qwen3VLTextShape = QWEN3VL_2B) -> int:
    """Algorithmic HBM bytes of one batch decode step: every weight once (shared
    by the batch), K/V[0:L_b] of every layer once per sequence, B embedding rows."""
    h, i, d = shape.hidden, shape.intermediate, shape.head_dim
    layer_w = 2 * ((shape.q_size + 2 * shape.kv_size) * h + h * shape.q_size + 3 * i * h) + 2 * (2 * h + 2 * d)
    kv = 2 * 2 * shape.num_kv_heads * d * int(sum(int(x) for x in context_lens))
    return shape.num_layers * layer_w + kv * shape.num_layers + 2 * shape.vocab * h + 2 * h + 2 * h * len(context_lens)


def _rms(x, w, eps):
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def _rope(x, cos, sin):
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], -1)
    return x * cos + rot * sin


def roofline_bytes_step(context_len: int, shape: Qwen3VLTextShape = QWEN3VL_2B) -> int:
    """Algorithmic HBM bytes of one batch-1 decode step at KV length L: every
    weight once, K/V[0:L] of every layer once, the embedding row and final norm."""
    h, i, d = shape.hidden, shape.intermediate, shape.head_dim
    layer_w = 2 * (shape.qkv_rows * h + h * shape.q_size + 3 * i * h) + 2 * (2 * h + 2 * d)
    kv = 2 * 2 * shape.num_kv_heads * d * context_len
    return shape.num_layers * (layer_w + kv) + 2 * shape.vocab * h + 2 * h + 2 * h


__all__ = ["DecodeEngine", "rope_inv_freq", "roofline_bytes_step"]
