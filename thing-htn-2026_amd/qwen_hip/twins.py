"""Device-side torch twins of the decode-step operators, used only to certify the HIP kernels.

The reference keeps a pure-torch twin of every fused kernel and, at warmup, runs each kernel
on the production shapes against its twin (``engine/kernels/torch_ref.py:1-40``,
``engine/engine.py:407-486``). These are this engine's twins: the same formulas and bf16
rounding points, written for device tensors (fp32 arithmetic, explicit roundings), and sized
for one certification pass. They never produce an output of the engine; the decode step is
HIP kernels only.

Rounding points (``bf16(.)`` is round-to-nearest-even):

* RMSNorm: ``y = w * bf16(x * rsqrt(sum(x^2) * (1/N) + eps))``, the product rounded once.
* residual: ``h = bf16(x + r)``.
* projections: fp32 accumulation, one rounding; the fused epilogues round the product first
  (``bf16(res + bf16(acc))``, ``bf16(bf16(silu(bf16(g))) * bf16(u))``).
* RoPE: ``bf16(bf16(y * cos) + bf16(rotate_half(y) * sin))``.
* attention: fp32 scores times scale, un-normalised probabilities rounded to bf16 before the
  value product, fp32 row sum, one rounding of ``acc / l``.
"""

from __future__ import annotations

import torch

BF16 = torch.bfloat16
F32 = torch.float32


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3 RMSNorm over the last dim (``engine/kernels/torch_ref.py:47-58``); the mean is the
    fp32 sum times fp32(1/N) (``engine/kernels/rmsnorm.py:87-88``)."""
    xf = x.to(F32)
    var = xf.square().sum(-1, keepdim=True) * torch.tensor(1.0 / x.shape[-1], dtype=F32, device=x.device)
    n = (xf * torch.rsqrt(var + eps)).to(BF16)
    return (n.to(F32) * w.to(F32)).to(BF16)


def add(x: torch.Tensor, r: torch.Tensor) -> torch.Tensor:
    """Residual add, one rounding (``engine/kernels/torch_ref.py:61-68``)."""
    return (x.to(F32) + r.to(F32)).to(BF16)


def linear(x: torch.Tensor, w: torch.Tensor, rows: int = 32768) -> torch.Tensor:
    """``bf16(x @ w.T)`` with fp32 products and sums (``engine/engine.py:341-350``); the weight is
    widened ``rows`` output rows at a time to bound the fp32 copy."""
    xf = x.to(F32)
    out = torch.empty((x.shape[0], w.shape[0]), dtype=BF16, device=x.device)
    for r0 in range(0, w.shape[0], rows):
        out[:, r0:r0 + rows] = (xf @ w[r0:r0 + rows].to(F32).t()).to(BF16)
    return out


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """SwiGLU of a fused ``[..., 2I]`` gate|up output (``engine/kernels/torch_ref.py:74-88``):
    ``bf16(bf16(g / (1 + exp(-g))) * u)``."""
    inter = gu.shape[-1] // 2
    g = gu[..., :inter].to(F32)
    s = (g / (1.0 + torch.exp(-g))).to(BF16)
    return (s.to(F32) * gu[..., inter:].to(F32)).to(BF16)


def rope(y: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """RoPE with three roundings (``engine/kernels/torch_ref.py:94-104``)."""
    yf = y.to(F32)
    half = yf.shape[-1] // 2
    rot = torch.cat((-yf[..., half:], yf[..., :half]), dim=-1)
    a = (yf * cos.to(F32)).to(BF16).to(F32)
    b = (rot * sin.to(F32)).to(BF16).to(F32)
    return (a + b).to(BF16)


def qk_norm_rope(qkv, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, positions, T, Nkv):
    """Per-head q/k RMSNorm + RoPE at ``positions[b] + t`` and the raw V rows
    (``engine/kernels/torch_ref.py:107-162`` without the cache write).

    Returns ``q [B, T, Nq, D]``, ``k [B, T, Nkv, D]``, ``v [B, T, Nkv, D]`` bf16."""
    M, width = qkv.shape
    B = M // T
    D = q_norm_w.shape[0]
    Nq = width // D - 2 * Nkv
    q = qkv[:, :Nq * D].reshape(B, T, Nq, D)
    k = qkv[:, Nq * D:(Nq + Nkv) * D].reshape(B, T, Nkv, D)
    v = qkv[:, (Nq + Nkv) * D:].reshape(B, T, Nkv, D)
    pos = positions.to(torch.int64)[:, None] + torch.arange(T, device=qkv.device)[None, :]
    cos, sin = cos_tab[pos].unsqueeze(2), sin_tab[pos].unsqueeze(2)
    return rope(rms_norm(q, q_norm_w, eps), cos, sin), rope(rms_norm(k, k_norm_w, eps), cos, sin), v


def attention(q, k_cache, v_cache, lengths, scale):
    """Causal GQA decode attention (``engine/kernels/torch_ref.py:168-227``).

    ``q [B, T, Nq, D]``; caches ``[B, Nkv, CAP, D]``; query ``t`` of row ``b`` sees key ``j`` iff
    ``j < lengths[b] - (T - 1 - t)``; head ``h`` reads KV head ``h // (Nq / Nkv)``. Only the
    first ``max(lengths)`` cache slots are read; slots at or past a row's length are zeroed
    before the value product. Returns ``[B, T, Nq * D]`` bf16."""
    B, T, Nq, D = q.shape
    Nkv = k_cache.shape[1]
    G = Nq // Nkv
    Lmax = int(lengths.max())
    kf = k_cache[:, :, :Lmax].to(F32)
    vf = v_cache[:, :, :Lmax].to(F32)
    len64 = lengths.to(torch.int64)
    j = torch.arange(Lmax, device=q.device)
    vf = vf.masked_fill(~(j[None, :] < len64[:, None])[:, None, :, None], 0.0)
    qf = q.to(F32).reshape(B, T, Nkv, G, D).permute(0, 2, 3, 1, 4).reshape(B, Nkv, G * T, D)
    limit = len64[:, None] - (T - 1 - torch.arange(T, device=q.device))[None, :]
    vis = (j[None, None, :] < limit[:, :, None])[:, None, None].expand(B, 1, G, T, Lmax).reshape(B, 1, G * T, Lmax)
    s = (qf @ kf.transpose(-1, -2)) * scale
    s = s.masked_fill(~vis, float("-inf"))
    e = torch.exp(s - s.amax(dim=-1, keepdim=True))
    out = (e.to(BF16).to(F32) @ vf) / e.sum(dim=-1, keepdim=True)
    return out.reshape(B, Nkv, G, T, D).permute(0, 3, 1, 2, 4).to(BF16).reshape(B, T, Nq * D)


def close(a: torch.Tensor, b: torch.Tensor, atol: float = 1e-2, rtol: float = 1.0 / 64) -> bool:
    """The reference's certification predicate (``engine/engine.py:425-429``): same shape and
    dtype, ``a`` finite, ``|a - b| <= atol + rtol * |b|`` everywhere."""
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    af, bf = a.to(F32), b.to(F32)
    return bool(torch.isfinite(af).all()) and bool(((af - bf).abs() <= atol + rtol * bf.abs()).all())


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at ``|x|`` (8 significant bits), for fp32 ``x``."""
    _, e = torch.frexp(x.abs().clamp_min(2.0 ** -126))
    return torch.ldexp(torch.ones_like(x), (e - 8).to(torch.int32))


def argmax_ok(tokens: torch.Tensor, logits: torch.Tensor) -> bool:
    """Greedy tokens against bf16 logits ``[M, V]``: each token is in range and its logit lies
    within two bf16 ulps of the row maximum. The kernel's fp32 sums differ from the twin's in
    order only, so each of the two competing logits may round one ulp the other way; the
    reference's argmax takes the lowest index among equal logits."""
    M, V = logits.shape
    t = tokens.to(torch.int64).reshape(-1)
    if t.numel() != M or bool(((t < 0) | (t >= V)).any()):
        return False
    lf = logits.to(F32)
    top = lf.max(dim=-1).values
    got = lf.gather(1, t[:, None])[:, 0]
    return bool(torch.isfinite(top).all()) and bool((top - got <= 2 * bf16_ulp(top)).all())
