"""Decode GEMV operator wrappers re-exported as one public surface.

Same module layout and public names as the reference package
cuda_decode_gemv_ops (__init__.py:22-74), backed by the gfx950 C-ABI library.
"""

from .runtime import (
    DUALCOPY_ROUTE_MODES,
    FULL_LAYER_PROFILE_SLOT_NAMES,
    GRIDSYNC_PROFILE_SLOT_NAMES,
    NOSPLIT_PROFILE_SLOT_NAMES,
    NOSPLIT_VARIANTS,
    NOSPLIT_XWARP_DETAIL_SLOT_NAMES,
    OPROJ_MLP_PROFILE_SLOT_NAMES,
    PERSISTENT_PROFILE_SLOT_NAMES,
    SOFTSYNC_PROFILE_SLOT_NAMES,
)
from .fused import *  # noqa: F401,F403
from .matvec import *  # noqa: F401,F403
from .profile import *  # noqa: F401,F403
from . import fused as _fused, matvec as _matvec, profile as _profile

__all__ = [
    "NOSPLIT_PROFILE_SLOT_NAMES",
    "NOSPLIT_XWARP_DETAIL_SLOT_NAMES",
    "NOSPLIT_VARIANTS",
    "DUALCOPY_ROUTE_MODES",
    "FULL_LAYER_PROFILE_SLOT_NAMES",
    "SOFTSYNC_PROFILE_SLOT_NAMES",
    "PERSISTENT_PROFILE_SLOT_NAMES",
    "OPROJ_MLP_PROFILE_SLOT_NAMES",
    "GRIDSYNC_PROFILE_SLOT_NAMES",
    *_matvec.__all__,
    *_fused.__all__,
    *_profile.__all__,
]
