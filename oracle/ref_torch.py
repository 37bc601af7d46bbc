"""torch-CPU restatement of the reference's decode-path arithmetic (primary oracle).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every function keeps the reference's formula and every bf16 rounding point;
the reference states them in ``engine/kernels/torch_ref.py:16-29`` and the
Transformers Qwen3 module they mirror is
``transformers/models/qwen3/modeling_qwen3.py:59-64`` (RMSNorm), ``:81-83``
(MLP), ``:86-170`` (rotary), ``:211-280`` (attention), ``:283-322`` (decoder
layer). On CPU a bf16 binary op is computed in fp32 and rounded once, so
``a * b`` on bf16 tensors is ``bf16(f32(a) * f32(b))``; the code relies on
that exactly as the reference does.

Shapes follow the reference's operator boundary (``engine/engine.py:257-263``):
activations are ``[M, width]`` with ``M = B * T`` and row ``m = b * T + t``;
KV caches are ``[B, Nkv, CAP, D]``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16
F32 = torch.float32


# --------------------------------------------------------------------- norms

def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3 RMSNorm over the last dim. Restates ``engine/kernels/torch_ref.py:47-58``.

    fp32 sum of squares times the fp32 reciprocal ``1/N`` (the reference's
    mean: ``engine/kernels/rmsnorm.py:87-88`` passes ``inv_n = 1 / n_cols``,
    and torch's GPU ``mean`` multiplies by that factor; torch's CPU ``mean``
    divides by ``N`` instead, up to 1 fp32 ulp away), ``rsqrt(var + eps)``;
    the normalised value is rounded to bf16 first and only then multiplied by
    the bf16 gain (that product rounded once).
    """
    xf = x.to(F32)
    var = xf.pow(2).sum(-1, keepdim=True) * torch.tensor(1.0 / x.shape[-1], dtype=F32)
    n = (xf * torch.rsqrt(var + eps)).to(x.dtype)
    return w * n


def add_rms_norm(x: torch.Tensor, r: torch.Tensor, w: torch.Tensor, eps: float):
    """Residual add then RMSNorm of the ROUNDED sum. Restates ``torch_ref.py:61-68``.

    Returns ``(h, y)`` with ``h = bf16(f32(x) + f32(r))`` and ``y = rms_norm(h)``.
    """
    h = (x.to(F32) + r.to(F32)).to(x.dtype)
    return h, rms_norm(h, w, eps)


# ----------------------------------------------------------------------- mlp

def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """SwiGLU on the fused gate/up output. Restates ``torch_ref.py:74-88``.

    ``gu [..., 2I]``: gate = columns ``[0, I)``, up = ``[I, 2I)``.
    ``s = bf16(silu_f32(g))`` then ``bf16(f32(s) * f32(u))``.
    """
    inter = gu.shape[-1] // 2
    g = gu[..., :inter].contiguous()
    u = gu[..., inter:]
    s = F.silu(g)
    return (s.to(F32) * u.to(F32)).to(gu.dtype)


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``x @ w.T`` in bf16 with fp32 accumulation and one rounding.

    The reference's projections are ``F.linear`` / cuBLAS calls
    (``engine/engine.py:341-350``; ``gemm.py:12-15`` states the one-rounding rule).
    """
    return F.linear(x, w)


# ---------------------------------------------------------------------- rope

def rope_tables(P: int, theta: float, D: int):
    """cos/sin tables ``[P, D]`` bf16, op for op as ``engine/engine.py:232-251``.

    ``inv_freq = 1 / theta ** (arange(0, D, 2) / D)`` in fp32, the K=1 fp32
    matmul with the positions, ``emb = cat(freqs, freqs)``, fp32 cos/sin,
    rounded to bf16 (``modeling_qwen3.py:86-137`` computes the same).
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.int64).to(F32) / D))
    pos = torch.arange(P, dtype=F32)[None, :]
    freqs = (inv_freq[None, :, None].float().expand(1, -1, 1) @ pos[:, None, :].float()).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos()[0].to(BF16).contiguous(), emb.sin()[0].to(BF16).contiguous()


def rope_bf16(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``apply_rotary_pos_emb`` with its three bf16 roundings. Restates ``torch_ref.py:94-104``.

    ``out = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin))`` with
    ``rotate_half(x) = cat(-x[D/2:], x[:D/2])``.
    """
    xf = x.to(F32)
    half = xf.shape[-1] // 2
    rot = torch.cat((-xf[..., half:], xf[..., :half]), dim=-1)
    a = (xf * cos.to(F32)).to(x.dtype)
    b = (rot * sin.to(F32)).to(x.dtype)
    return (a.to(F32) + b.to(F32)).to(x.dtype)


def qk_norm_rope_cache(qkv, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, positions, T, k_cache, v_cache):
    """Per-head QK RMSNorm + RoPE + KV-cache write. Restates ``torch_ref.py:107-162``.

    ``qkv [M, (Nq + 2 Nkv) D]`` (q heads, then k heads, then v heads);
    token ``t`` of sequence ``b`` sits at position ``positions[b] + t``.
    Writes ``k_cache[b, :, pos]`` (normed + rotated K) and ``v_cache[b, :, pos]``
    (raw V) in place and returns q ``[B, T, Nq, D]``.
    """
    M, width = qkv.shape
    B = M // T
    D = q_norm_w.shape[0]
    Nkv = k_cache.shape[1]
    Nq = width // D - 2 * Nkv
    q = qkv[:, : Nq * D].reshape(B, T, Nq, D)
    k = qkv[:, Nq * D: (Nq + Nkv) * D].reshape(B, T, Nkv, D)
    v = qkv[:, (Nq + Nkv) * D:].reshape(B, T, Nkv, D)
    pos = positions.to(torch.int64)[:, None] + torch.arange(T, dtype=torch.int64)[None, :]
    cos = cos_tab[pos].unsqueeze(2)
    sin = sin_tab[pos].unsqueeze(2)
    q_out = rope_bf16(rms_norm(q, q_norm_w, eps), cos, sin)
    k_out = rope_bf16(rms_norm(k, k_norm_w, eps), cos, sin)
    for b in range(B):
        for t in range(T):
            p = int(pos[b, t])
            k_cache[b, :, p, :] = k_out[b, t]
            v_cache[b, :, p, :] = v[b, t]
    return q_out.contiguous()


# ----------------------------------------------------------------- attention

def attn_decode(q, k_cache, v_cache, lengths, scale):
    """Causal GQA decode attention over a static cache. Restates ``torch_ref.py:168-227``.

    Query ``t`` of sequence ``b`` sees key ``j`` iff ``j < lengths[b] - (T-1-t)``;
    query head ``h`` reads KV head ``h // (Nq/Nkv)``. fp32 scores scaled after the
    dot; un-normalised ``P = exp(s - max)`` rounded to bf16 for the PV product;
    fp32 row sum; one division and one bf16 rounding at the end. Slots at or
    beyond ``lengths[b]`` are ignored even if they hold NaN/Inf.
    Returns ``[B, T, Nq * D]`` bf16.
    """
    B, T, Nq, D = q.shape
    Nkv, CAP = k_cache.shape[1], k_cache.shape[2]
    G = Nq // Nkv
    qf = q.to(F32).reshape(B, T, Nkv, G, D).permute(0, 2, 3, 1, 4).reshape(B, Nkv, G * T, D)
    kf = k_cache.to(F32)
    vf = v_cache.to(F32)
    keys = torch.arange(CAP, dtype=torch.int64)
    lens = lengths.to(torch.int64)
    limit = lens[:, None] - (T - 1 - torch.arange(T, dtype=torch.int64))[None, :]      # [B, T]
    vis = keys[None, None, :] < limit[:, :, None]                                          # [B, T, CAP]
    vis = vis[:, None, None].expand(B, 1, G, T, CAP).reshape(B, 1, G * T, CAP)
    valid = keys[None, :] < lens[:, None]
    vf = vf.masked_fill(~valid[:, None, :, None], 0.0)
    kf = kf.masked_fill(~valid[:, None, :, None], 0.0)
    s = torch.matmul(qf, kf.transpose(-1, -2)) * scale
    s = s.masked_fill(~vis, float("-inf"))
    m = s.amax(dim=-1, keepdim=True)
    e = torch.exp(s - m)
    l = e.sum(dim=-1, keepdim=True)
    o = torch.matmul(e.to(BF16).to(F32), vf) / l
    o = o.reshape(B, Nkv, G, T, D).permute(0, 3, 1, 2, 4)
    return o.to(BF16).reshape(B, T, Nq * D).contiguous()


FLASH_BLOCK_N = 64        # keys per block of the reference's Triton kernel (attention.py:80)
FLASH_NEG = -1e30         # its finite stand-in for -inf (attention.py:84-87)


def choose_num_splits(B: int, Nkv: int) -> int:
    """The reference's split count (``engine/kernels/attention.py:94-110``): the smallest power of
    two ``S`` with ``B * Nkv * S >= 264``, at most 32."""
    bh, s = max(1, B * Nkv), 1
    while bh * s < 264 and s < 32:
        s *= 2
    return s


def reference_schedule(num_splits: int, block_n: int = FLASH_BLOCK_N):
    """The key blocks of the reference's Triton decode attention (``attention.py:139-214``) as a
    schedule ``f(length, T) -> lanes``: split ``s`` covers ``[s * chunk, min((s + 1) * chunk, length))``
    with ``chunk = cdiv(length, S)`` rounded up to whole blocks, walked in blocks of ``block_n``."""
    def lanes(length: int, T: int):
        chunk = -(-length // num_splits)
        chunk = -(-chunk // block_n) * block_n
        out = []
        for s in range(num_splits):
            start, end = s * chunk, min(s * chunk + chunk, length)
            out.append([(n0, min(n0 + block_n, end)) for n0 in range(start, end, block_n)])
        return out
    return lanes


def attn_decode_flash(q, k_cache, v_cache, lengths, scale, schedule=None):
    """Decode attention with the reference kernel's online softmax. Restates
    ``engine/kernels/attention.py:115-275`` (``_attn_partial_kernel`` + ``_attn_reduce_kernel``).

    Same visibility, scale and rounding points as ``attn_decode``, but the un-normalised
    probabilities of a block are ``exp(s - m)`` against the running maximum ``m`` of its lane
    (the keys seen so far), rounded to bf16 for the PV product; earlier blocks are rescaled by
    ``exp(m_old - m_new)`` in fp32 (``attention.py:199-214``); the lanes' ``(m, l, acc)`` merge by
    log-sum-exp and one division, rounded to bf16 once (``attention.py:253-275``). ``attn_decode``
    instead rounds every probability against the row's global maximum, so the two differ in the
    last bf16 bit of many P values.

    ``schedule(length, T) -> lanes``: per lane, the key ranges ``[k0, k1)`` it walks in order
    (default: ``reference_schedule(choose_num_splits(B, Nkv))``, the reference kernel's), or a list
    of such, one per sequence. A key beyond a query's limit ``length - (T - 1 - t)`` is masked.
    Returns ``[B, T, Nq * D]`` bf16."""
    B, T, Nq, D = q.shape
    Nkv = k_cache.shape[1]
    G = Nq // Nkv
    if schedule is None:
        schedule = reference_schedule(choose_num_splits(B, Nkv))
    schedules = schedule if isinstance(schedule, (list, tuple)) else [schedule] * B
    out = torch.empty((B, T, Nkv, G, D), dtype=BF16)
    neg = torch.tensor(FLASH_NEG, dtype=F32)
    for b in range(B):
        schedule = schedules[b]
        L = int(lengths[b])
        qf = q[b].to(F32).reshape(T, Nkv, G, D).permute(1, 0, 2, 3).reshape(Nkv, T * G, D)   # row t*G + g
        limit = L - (T - 1 - torch.arange(T * G) // G)                                       # [T*G]
        parts = []
        for lane in schedule(L, T):
            m = torch.full((Nkv, T * G), FLASH_NEG, dtype=F32)
            l = torch.zeros((Nkv, T * G), dtype=F32)
            acc = torch.zeros((Nkv, T * G, D), dtype=F32)
            for k0, k1 in lane:
                n = torch.arange(k0, k1)
                kf = k_cache[b, :, k0:k1].to(F32)
                vf = v_cache[b, :, k0:k1].to(F32)
                vis = (n[None, :] < limit[:, None])[None]                                    # [1, R, n]
                s = torch.where(vis, torch.matmul(qf, kf.transpose(-1, -2)) * scale, neg)
                m_new = torch.maximum(m, s.amax(-1))
                alpha = torch.exp(m - m_new)
                p = torch.where(vis, torch.exp(s - m_new[..., None]), torch.zeros((), dtype=F32))
                l = l * alpha + p.sum(-1)
                acc = acc * alpha[..., None] + torch.matmul(p.to(BF16).to(F32), vf)
                m = m_new
            parts.append((m, l, acc))
        ms = torch.stack([p[0] for p in parts])
        mx = ms.amax(0)
        w = torch.exp(ms - mx)
        lt = (w * torch.stack([p[1] for p in parts])).sum(0)
        at = (w[..., None] * torch.stack([p[2] for p in parts])).sum(0)
        o = (at / lt[..., None]).reshape(Nkv, T, G, D).permute(1, 0, 2, 3)
        out[b] = o.to(BF16)
    return out.reshape(B, T, Nq * D).contiguous()


def causal_prefill_attention_flash(q, k, v, scale, block_n: int = FLASH_BLOCK_N):
    """``causal_prefill_attention`` with the online softmax of flash attention, as the reference's
    prefill SDPA computes it on the GPU (``engine/engine.py:1123-1179``): every query walks the keys
    in blocks of ``block_n`` from key 0, rounding P to bf16 against its running maximum
    (``attn_decode_flash`` with one lane)."""
    B, S = q.shape[0], q.shape[1]
    lengths = torch.full((B,), S, dtype=torch.int32)
    one_lane = reference_schedule(1, block_n)
    return attn_decode_flash(q, k, v, lengths, scale, one_lane).reshape(B * S, -1)


def causal_prefill_attention(q, k, v, scale):
    """Prompt attention for one batch slice: ``q [B, S, Nq, D]``, ``k/v [B, Nkv, S, D]``.

    The reference prefill runs SDPA with ``is_causal`` (``engine/engine.py:1123-1179``);
    causal attention over the first ``S`` cache slots is exactly ``attn_decode`` with
    ``T = S`` and ``lengths = S``, which is how this oracle computes it.
    """
    B, S = q.shape[0], q.shape[1]
    lengths = torch.full((B,), S, dtype=torch.int32)
    return attn_decode(q, k, v, lengths, scale).reshape(B * S, -1)


# -------------------------------------------------------------------- argmax

def argmax_lowest(logits: torch.Tensor) -> torch.Tensor:
    """First index of the maximum (``torch.argmax`` semantics, ``OPTIMIZATION_GUIDE.md:213``)."""
    return logits.argmax(dim=-1)


# ------------------------------------------------------- speculative drafting

def spec_draft(hist: torch.Tensor, L: torch.Tensor, k: int, n: int) -> torch.Tensor:
    """Prompt-lookup draft, restating ``engine/engine.py:955-977``.

    For each row: find the latest start ``i`` with ``i < L - n`` such that
    ``hist[i:i+n] == hist[L-n:L]``; draft = ``hist[i+n : i+n+k]`` with indices
    clamped to ``[0, L-1]`` (``i = -1`` on a miss). Returns ``[B, k+1]`` =
    ``[hist[L-1], draft...]``.
    """
    B, W = hist.shape
    out = torch.empty((B, k + 1), dtype=hist.dtype)
    for b in range(B):
        Lb = int(L[b])
        suffix = [int(hist[b, max(0, Lb - n + j)]) for j in range(n)]
        best = -1
        for i in range(0, W - n + 1):
            if i >= Lb - n:
                break
            if all(int(hist[b, i + j]) == suffix[j] for j in range(n)):
                best = i
        out[b, 0] = hist[b, Lb - 1]
        for j in range(k):
            src = max(0, best + n + j)
            src = min(src, Lb - 1)
            out[b, 1 + j] = hist[b, src]
    return out


def spec_accept(nxt: torch.Tensor, tok: torch.Tensor, done: torch.Tensor) -> torch.Tensor:
    """Accepted length per row, restating ``engine/engine.py:994-997``.

    ``nxt [B, T]`` greedy outputs, ``tok [B, T]`` fed tokens (``tok[:, 1:]`` are
    drafts): ``adv = 1 + (number of leading drafts equal to the model's output)``,
    or 0 for rows already finished.
    """
    k = tok.shape[1] - 1
    eq = (nxt[:, :k] == tok[:, 1:]).to(torch.int64)
    acc = torch.cumprod(eq, dim=1).sum(dim=1) if k else torch.zeros(nxt.shape[0], dtype=torch.int64)
    return torch.where(done, torch.zeros_like(acc), acc + 1)
