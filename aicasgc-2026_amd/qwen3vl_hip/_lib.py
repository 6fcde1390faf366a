"""ctypes binding of ``libqwen3vl_decode.so`` (the C ABI in include/qwen3vl_decode.h).

The library is loaded from the package directory (built in-tree by
``qwen3vl_hip.build``).  There is no fallback: if the library is missing or a
call reports a non-zero status, a RuntimeError is raised.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int64, c_long, c_size_t, c_void_p
from functools import lru_cache
from pathlib import Path

import torch

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("QD_LIB_PATH", PKG_ROOT / "libqwen3vl_decode.so"))
TRACE_LIB_PATH = PKG_ROOT / "libqwen3vl_decode_trace.so"   # -DQD_TRACE build (phase timestamps)

QD_F16 = 0
QD_F32 = 1

# decode-step phase bits (QD_PHASE_* in include/qwen3vl_decode.h)
PHASE = {"embed": 0x01, "qkv": 0x02, "attn": 0x04, "attn_merge": 0x08, "o_proj": 0x10, "gate_up": 0x20,
         "down": 0x40, "lm_head": 0x80}
PHASE_ALL = 0xFF
STEP_AUTO, STEP_CHAIN, STEP_PERSISTENT = 0, 1, 2
QD_ERR_ARG, QD_ERR_SHAPE = -1, -2

P = c_void_p

# name -> (restype, argtypes)
_SIGS = {
    "qd_version": (c_int, []),
    "qd_last_error": (ctypes.c_char_p, []),
    "qd_device_cu_count": (c_int, []),
    "qd_matvec_f16": (c_int, [P, P, P, P, c_int, c_int, P]),
    "qd_splitk_matvec_f16": (c_int, [P, P, P, P, P, c_int, c_int, c_int, P]),
    "qd_rmsnorm_matvec_f16": (c_int, [P, P, P, P, P, c_int, c_int, c_float, P]),
    "qd_post_attn_mlp_f16": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_float, P]),
    "qd_post_attn_mlp_next_f16": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_float, P, P, P]),
    "qd_gateup_silu_down_f16": (c_int, [P, P, P, P, P, P, c_int, c_int, P]),
    "qd_add_rmsnorm_matvec_f16": (c_int, [P, P, P, P, P, P, P, c_int, c_int, c_float, P]),
    "qd_silu_matvec_f16": (c_int, [P, P, P, P, c_int, c_int, P]),
    "qd_lm_head_workspace_bytes": (c_size_t, [c_int]),
    "qd_lm_head_argmax": (c_int, [P, c_int, P, c_float, P, c_int, c_int, P, P, P, P]),
    "qd_q_rope_kv_update": (c_int, [P, P, P, c_int, c_long, c_long, c_long, P, P, c_float, P, P, P, P,
                                    c_int, c_int, c_int, P, c_int, P, P, c_long, c_long, c_int, P,
                                    c_int, c_int, P]),
    "qd_qk_norm_rope_f16": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_float, P]),
    "qd_add_rmsnorm_f16": (c_int, [P, P, P, P, P, c_int, c_int, c_float, P]),
    "qd_rmsnorm_f16": (c_int, [P, P, P, c_int, c_int, c_float, P]),
    "qd_silu_mul_f16": (c_int, [P, P, P, c_long, P]),
    "qd_add_f16": (c_int, [P, P, P, c_long, P]),
    "qd_attention_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "qd_attention_decode": (c_int, [P, c_int, c_long, P, P, c_long, c_long, c_int, P, c_float, P, c_int,
                                    c_int, c_int, c_int, P, P]),
    "qd_attention_qkv_decode_f16": (c_int, [P, P, P, c_float, P, P, P, P, c_long, c_long, c_int, P, c_float, P,
                                            c_int, c_int, c_int, P, P]),
    "qd_attention_decode_noalloc": (c_int, [P, c_int, c_long, P, P, c_long, c_long, c_int, P, c_float, P,
                                            c_int, c_int, c_int, c_int, P]),
    "qd_attention_partial": (c_int, [P, c_int, c_long, P, P, c_long, c_long, c_int, P, c_float, P, P,
                                     c_int, c_int, c_int, P]),
    "qd_attention_merge": (c_int, [P, P, P, c_int, c_int, c_int, P]),
    "qd_attention_default_splits": (c_int, [c_int]),
    "qd_decode_workspace_bytes": (c_size_t, [P]),
    "qd_decode_workspace_layout": (c_int, [P, POINTER(c_size_t), c_int]),
    "qd_decode_step": (c_int, [P, P]),
    "qd_decode_step_phases": (c_int, [P, c_int, c_int, ctypes.c_uint, P]),
    "qd_decode_advance": (c_int, [P, P, P, P, P, c_int, P]),
    "qd_decode_step_mode": (c_int, [P]),
    "qd_decode_layers_persistent": (c_int, [P, P]),
    "qd_decoder_layer_persistent_f16": (c_int, [P, P, c_int, P, P, P, c_float, c_float, P, P, P, P]),
    "qd_decoder_layers_persistent_f16": (c_int, [P, P, c_int, c_int, P, P, P, c_float, c_float, P, P, P, P]),
    "qd_persistent_prepare": (c_int, [P]),
    "qd_persistent_set_spin_limit": (c_int, [ctypes.c_uint]),
    "qd_decode_status": (c_int, [P, POINTER(ctypes.c_uint), c_int]),
    "qd_persistent_trace_read": (c_int, [P, c_size_t, POINTER(c_int)]),
    "qd_batch_gemv_workspace_bytes": (ctypes.c_size_t, [c_long, c_long]),
    "qd_batch_tile_rows": (c_int, [c_long, c_long, c_int]),
    "qd_batch_gemv": (c_int, [P, c_long, P, c_float, P, c_long, c_long, c_long, c_long, P, c_long, P, c_long, c_int,
                              c_int, P, ctypes.c_size_t, P]),
    "qd_decode_advance_batch": (c_int, [P, P, P, P, P, c_int, c_int, P]),
}

EXPORTED = tuple(_SIGS)


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"HIP decode library not found at {LIB_PATH}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (or python -m qwen3vl_hip.build)")
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGS.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def last_error() -> str:
    msg = lib().qd_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed with status {status}: {last_error()}")


def ptr(t: torch.Tensor | None):
    return None if t is None else c_void_p(t.data_ptr())


def stream(device: torch.device | None = None):
    return c_void_p(torch.cuda.current_stream(device).cuda_stream)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


class ModelDesc(ctypes.Structure):
    pass


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("qkv", "o_proj", "gate_up", "down", "input_norm", "post_norm",
                                         "q_norm", "k_norm", "k_cache", "v_cache")]


ModelDesc._fields_ = [
    ("num_layers", c_int), ("hidden", c_int), ("num_heads", c_int), ("num_kv_heads", c_int),
    ("head_dim", c_int), ("intermediate", c_int), ("vocab", c_int),
    ("capacity", c_int),
    ("eps", c_float),
    ("sec_t", c_int), ("sec_h", c_int), ("sec_w", c_int),
    ("inv_freq", c_void_p),
    ("layers", POINTER(LayerDesc)),
    ("embed", c_void_p),
    ("final_norm", c_void_p),
    ("token", c_void_p),
    ("cache_position", c_void_p),
    ("rope_position", c_void_p),
    ("logits_out", c_void_p),
    ("workspace", c_void_p),
    ("attn_splits", c_int), ("step_mode", c_int), ("batch", c_int),
    ("advance_out_tokens", c_void_p), ("advance_counter", c_void_p), ("advance_max_tokens", c_int),
    ("argmax_f16_logits", c_int),
    ("batch_tiled_weights", c_int),
]

__all__ = ["lib", "check", "ptr", "stream", "call", "QD_F16", "QD_F32", "ModelDesc", "LayerDesc", "EXPORTED",
           "LIB_PATH", "c_int64"]
