"""Profiling entry points of the reference (cuda_decode_gemv_ops/profile.py).

The reference stamps %globaltimer / clock64 / %smid values from inside its
CUDA kernels into trace buffers.  That instrumentation is NVIDIA-specific and
is not part of this build: per-kernel time, HBM bytes and occupancy on MI355X
come from rocprofv3 (kernel trace and PMC counters).  The names stay
importable and raise NotImplementedError with that explanation.
"""

from __future__ import annotations

_NAMES = (
    "fused_decode_full_layer_softsync_profile_half",
    "fused_o_proj_post_attn_mlp_persistent_profile_half",
    "fused_o_proj_post_attn_mlp_softsync_profile_half",
    "fused_gateup_silu_downproj_softsync_profile_half",
    "fused_gateup_silu_downproj_gridsync_profile_half",
    "fused_gateup_silu_downproj_persistent_profile_half",
    "nosplit_matvec_half_profile",
    "nosplit_matvec_half_profile_variant",
    "nosplit_matvec_half_profile_xwarp_detail",
    "nosplit_xwarp_wait_sync_calibration",
    "nosplit_matvec_half_profile_xwarp_detail_with_smid",
    "nosplit_matvec_half_profile_xwarp_sms2_cta_trace",
    "nosplit_matvec_half_profile_xwarp_sms2_balanced_cta_trace",
)


def _unavailable(name: str):
    def fn(*args, **kwargs):
        raise NotImplementedError(
            f"{name}: in-kernel timer tracing is not provided on MI355X; profile with "
            "`rocprofv3 --kernel-trace --stats` and `rocprofv3 --pmc ...` instead")
    fn.__name__ = name
    return fn


for _n in _NAMES:
    globals()[_n] = _unavailable(_n)

__all__ = list(_NAMES)
