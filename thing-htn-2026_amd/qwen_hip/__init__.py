"""MI355X kernels for the Qwen3-4B decode path, behind the reference's operator API.

``qwen_hip.ops`` exposes the operators of the reference's ``self.ops`` table
(``engine/engine.py:257-263``) with the same names, argument meaning and
error behaviour (``AssertionError`` on shape/dtype preconditions,
``RuntimeError`` when the native library is unavailable), plus the fused
projections and the LM-head argmax. Every op runs a hand-written HIP kernel
from ``libqwen_hip.so`` through ctypes; there is no CPU or torch fallback.
"""

from . import _lib  # noqa: F401
from .ops import (  # noqa: F401
    TiledWeight,
    add_rms_norm,
    attn_decode,
    choose_num_splits,
    embed,
    fused_linear,
    lm_head_argmax,
    qk_norm_rope_cache,
    rms_norm,
    silu_mul,
    tile_weight,
)
