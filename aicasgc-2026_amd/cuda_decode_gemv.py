#!/usr/bin/env python3
"""Facade for the decode GEMV entry points (reference cuda_decode_gemv.py:1-5)."""

from cuda_decode_gemv_ops import *  # noqa: F401,F403
from cuda_decode_gemv_ops import __all__  # noqa: F401
