"""Independent numpy restatement of the per-op formulas (cross-check of ``ref_torch``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

bf16 tensors are float32 arrays whose values are bf16-representable; ``rb``
rounds fp32 to the nearest bf16 (ties to even) by bit manipulation, so this
module shares no rounding code with torch. Rounding points follow
``engine/kernels/torch_ref.py:16-29``; GEMMs accumulate in float64 and round
once (the exact sum, which any fp32 accumulation order approximates).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def rb(x) -> np.ndarray:
    """Round float32 values to bf16 (RNE), returned as float32."""
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = ((u + np.uint32(0x7FFF) + lsb) & np.uint32(0xFFFF0000)).view(F32)
    return np.where(np.isnan(x), np.float32(np.nan), r).astype(F32)


def rms_norm(x, w, eps):
    """``torch_ref.py:47-58``: bf16(x * rsqrt(mean(x^2) + eps)), then * gain, rounded; the mean is
    the fp32 sum times fp32(1/N) (``engine/kernels/rmsnorm.py:87-88``)."""
    x = np.asarray(x, F32)
    var = (np.sum(x * x, axis=-1, keepdims=True, dtype=F32) * F32(1.0 / x.shape[-1])).astype(F32)
    r = (F32(1.0) / np.sqrt(var + F32(eps))).astype(F32)
    return rb(np.asarray(w, F32) * rb(x * r))


def add_rms_norm(x, r, w, eps):
    h = rb(np.asarray(x, F32) + np.asarray(r, F32))
    return h, rms_norm(h, w, eps)


def silu_mul(gu):
    """``torch_ref.py:74-88``: bf16(silu_f32(g)), then bf16(s * u)."""
    gu = np.asarray(gu, F32)
    i = gu.shape[-1] // 2
    g, u = gu[..., :i], gu[..., i:]
    s = rb(g / (F32(1.0) + np.exp(-g)))
    return rb(s * u)


def linear(x, w):
    """bf16(x @ w.T), exact (float64) accumulation, one rounding."""
    return rb((np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(F32))


def rope(x, cos, sin):
    """``torch_ref.py:94-104``: bf16(bf16(x*cos) + bf16(rotate_half(x)*sin))."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return rb(rb(x * cos) + rb(rot * sin))


def attn_decode(q, k_cache, v_cache, lengths, scale):
    """``torch_ref.py:168-227`` in float64 except the bf16 rounding of P and of the output."""
    B, T, Nq, D = q.shape
    Nkv = k_cache.shape[1]
    G = Nq // Nkv
    out = np.zeros((B, T, Nq, D), F32)
    for b in range(B):
        for t in range(T):
            lim = int(lengths[b]) - (T - 1 - t)
            for h in range(Nq):
                kv = h // G
                s = (k_cache[b, kv, :lim].astype(np.float64) @ q[b, t, h].astype(np.float64)) * scale
                e = np.exp(s - s.max())
                p = rb(e.astype(F32)).astype(np.float64)
                out[b, t, h] = (p @ v_cache[b, kv, :lim].astype(np.float64)) / e.sum()
    return rb(out).reshape(B, T, Nq * D)


def argmax_lowest(logits):
    return np.argmax(logits, axis=-1)
