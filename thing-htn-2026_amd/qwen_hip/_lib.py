"""ctypes binding of libqwen_hip.so (declarations: ``include/qwen_hip.h``).

The library is loaded lazily on first use. A missing library raises
``RuntimeError`` (the product path has no fallback). Every call checks the
returned status and raises ``RuntimeError`` naming the entry point.
"""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqwen_hip.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_ll = ctypes.c_longlong
_f = ctypes.c_float
_pi = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); the order matches include/qwen_hip.h.
SIGNATURES = {
    "qwen_rms_norm": (_i, [_p, _p, _p, _i, _i, _f, _p]),
    "qwen_add_rms_norm": (_i, [_p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "qwen_silu_mul": (_i, [_p, _p, _i, _i, _p]),
    "qwen_qk_norm_rope_cache": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _f, _p]),
    "qwen_attn_workspace_bytes": (_ll, [_i, _i, _i, _i, _i, _i]),
    "qwen_attn_decode": (_i, [_p, _p, _p, _p, _i, _p, _p, _ll, _i, _i, _i, _i, _i, _i, _f, _i, _i, _p]),
    "qwen_attn_decode_fused": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _ll, _i, _i, _i, _i, _i, _i, _i, _f,
                                    _f, _i, _i, _p]),
    "qwen_attn_mfma_workspace_bytes": (_ll, [_i, _i, _i, _i]),
    "qwen_attn_decode_mfma": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _ll, _i, _i, _i, _i, _i, _i, _i, _f,
                                   _f, _i, _i, _p]),
    "qwen_attn_decode_mfma_ex": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _ll, _i, _i, _i, _i, _i, _i, _i,
                                      _f, _f, _i, _i, _i, _p]),
    "qwen_attn_decode_mfma_noalloc": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _f, _f,
                                           _i, _i, _i, _p]),
    "qwen_sumsq16": (_i, [_p, _p, _i, _i, _p]),
    "qwen_linear_workspace_bytes": (_ll, [_i, _i, _i, _i]),
    "qwen_linear": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _p, _f, _p, _p, _i, _i, _i, _i, _p, _ll, _p]),
    "qwen_linear_rect": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _p, _f, _p, _p, _i, _i, _i, _i, _i, _p, _ll, _p]),
    "qwen_gemv_lds_bytes": (_ll, [_i, _i, _i, _i, _i, _i]),
    "qwen_gemv": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _f, _p, _i, _p, _i, _i, _p]),
    "qwen_gemv_rowmap": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _f, _p, _i, _p, _p, _i, _i, _p]),
    "qwen_lm_head_argmax": (_i, [_p, _p, _p, _f, _p, _i, _i, _i, _p, _p, _i, _i, _p]),
    "qwen_argmax_extract": (_i, [_p, _i, _p, _p]),
    "qwen_embed": (_i, [_p, _p, _p, _i, _p, _p, _p, _i, _ll, _i, _p]),
    "qwen_decode_finish": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _ll, _i, _p]),
    "qwen_spec_draft": (_i, [_p, _p, _i, _i, _i, _i, _p, _p]),
    "qwen_spec_accept": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _p, _p, _p, _p, _p, _ll, _i, _p]),
    "qwen_gemm": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _i, _p]),
    "qwen_attn_prefill": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _f, _p]),
    "qwen_tile_weight": (_i, [_p, _p, _ll, _i, _i, _p]),
    "qwen_init_weight": (_i, [_p, _ll, _i, _i, _i, _pi, _pi, _i, ctypes.c_ulonglong, _f, _p]),
}

_STATUS = {1001: "bad size/shape argument", 1002: "null pointer", 1003: "workspace too small",
           1004: "request exceeds the allocation-free entry point's fixed scratch"}

_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and type the native library; RuntimeError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950) first")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke entry point ``name``; raise RuntimeError on a nonzero status."""
    status = getattr(load(), name)(*args)
    if status != 0:
        raise RuntimeError(f"{name} failed with status {status} ({_STATUS.get(status, 'hipError_t')})")


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))
