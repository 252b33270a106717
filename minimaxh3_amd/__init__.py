"""MI355X (gfx950) native FP8 hot path of a video+audio DiT server.

``minimaxh3_amd.kernels`` mirrors the reference's ``kernels`` package (fp8_linear,
fp8_attention, attention_router); ``install_as_kernels()`` makes ``import kernels...``
resolve to it so that an unchanged runtime picks up this implementation.
"""
from __future__ import annotations

import sys

__version__ = "0.1.0"


def install_as_kernels() -> None:
    """Alias this package's ``kernels`` modules as the top-level ``kernels`` package."""
    from . import kernels
    from .kernels import attention_router, fp8_attention, fp8_linear

    sys.modules["kernels"] = kernels
    sys.modules["kernels.fp8_linear"] = fp8_linear
    sys.modules["kernels.fp8_attention"] = fp8_attention
    sys.modules["kernels.attention_router"] = attention_router
