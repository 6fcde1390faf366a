"""Native MI355X (gfx950) decode path for the Qwen3-VL-2B text decoder.

``_lib`` binds the C-ABI library (libqwen3vl_decode.so); ``engine`` drives the
captured 28-layer decode step; ``synthetic`` makes the seeded benchmark inputs.
"""

from .config import QWEN3VL_2B, Qwen3VLTextShape  # noqa: F401
