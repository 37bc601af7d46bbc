"""Operator wrappers over libqwen_hip.so, mirroring the reference's operator boundary.

Names, argument order and meaning follow ``engine/engine.py:257-263`` (the
``self.ops`` table) and the Triton wrappers they dispatch to
(``engine/kernels/rmsnorm.py:141-207``, ``rope.py:169-226``,
``attention.py:278-348``, ``silu.py:95-125``, ``gemm_fused.py:136-173``).
Like the reference, each op allocates and returns its output (``torch.empty``,
so under graph capture it comes from the graph's private pool), mutates only
the caches it is documented to write, asserts its shape/dtype preconditions
and raises ``RuntimeError`` if the native library is missing or a launch fails.
All tensors must be on the GPU: there is no CPU path.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

BF16 = torch.bfloat16
EPI_STORE, EPI_RES, EPI_SWIGLU = 0, 1, 2


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _gpu(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("qwen_hip ops run on the GPU only; got a tensor on " + str(t.device))


def _nullable(t):
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------- norms

def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """``Qwen3RMSNorm`` over the last dim (``rmsnorm.py:141-167``)."""
    _gpu(x, w)
    assert x.dtype == BF16 and w.dtype == BF16, "rms_norm expects bf16"
    N = x.shape[-1]
    assert w.numel() == N and w.is_contiguous()
    x = x.contiguous()
    y = torch.empty_like(x)
    _lib.call("qwen_rms_norm", x.data_ptr(), w.data_ptr(), y.data_ptr(), x.numel() // N, N, float(eps), _stream())
    return y


def add_rms_norm(x: torch.Tensor, r: torch.Tensor, w: torch.Tensor, eps: float):
    """``h = bf16(x + r)``, ``y = rms_norm(h)``; returns ``(h, y)`` (``rmsnorm.py:170-207``)."""
    _gpu(x, r, w)
    assert x.dtype == BF16 and r.dtype == BF16 and w.dtype == BF16, "add_rms_norm expects bf16"
    assert x.shape == r.shape, "add_rms_norm: x and r shapes differ"
    N = x.shape[-1]
    assert w.numel() == N and w.is_contiguous()
    x, r = x.contiguous(), r.contiguous()
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    _lib.call("qwen_add_rms_norm", x.data_ptr(), r.data_ptr(), w.data_ptr(), h.data_ptr(), y.data_ptr(),
              x.numel() // N, N, float(eps), _stream())
    return h, y


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """``bf16(bf16(silu(gate)) * up)`` for ``gu [..., 2I]`` (``silu.py:95-125``)."""
    _gpu(gu)
    assert gu.dtype == BF16 and gu.shape[-1] % 2 == 0, "silu_mul expects bf16 [..., 2I]"
    gu = gu.contiguous()
    inter = gu.shape[-1] // 2
    out = torch.empty((*gu.shape[:-1], inter), dtype=BF16, device=gu.device)
    _lib.call("qwen_silu_mul", gu.data_ptr(), out.data_ptr(), gu.numel() // gu.shape[-1], inter, _stream())
    return out


# ------------------------------------------------------------ rope + cache

def qk_norm_rope_cache(qkv, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, positions, T, k_cache, v_cache,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """q/k RMSNorm + RoPE, K/V cache write; returns q ``[B, T, Nq, D]`` (``rope.py:169-226``)."""
    _gpu(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache)
    B, Nkv, CAP, D = k_cache.shape
    M, W = qkv.shape
    assert D == 128, f"head_dim must be 128, got {D}"
    assert W % D == 0 and W // D > 2 * Nkv, f"qkv width {W} does not hold Nq + 2*{Nkv} heads of {D}"
    Nq = W // D - 2 * Nkv
    assert M == B * T, f"qkv has {M} rows but B*T = {B}*{T}"
    assert qkv.dtype == BF16 and qkv.is_contiguous()
    assert k_cache.is_contiguous() and v_cache.is_contiguous() and v_cache.shape == k_cache.shape
    assert k_cache.dtype == BF16 and v_cache.dtype == BF16
    assert q_norm_w.numel() == D and k_norm_w.numel() == D
    assert cos_tab.dim() == 2 and cos_tab.shape[1] == D and cos_tab.is_contiguous() and sin_tab.shape == cos_tab.shape
    assert cos_tab.dtype == BF16 and sin_tab.dtype == BF16
    assert positions.dtype == torch.int32 and positions.numel() == B and positions.is_contiguous()
    q = out if out is not None else torch.empty((B, T, Nq, D), dtype=BF16, device=qkv.device)
    for t in (qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, q, k_cache, v_cache):
        assert t.data_ptr() % 16 == 0, "qk_norm_rope_cache reads and writes 16-byte pieces: tensors must be 16-byte aligned"
    _lib.call("qwen_qk_norm_rope_cache", qkv.data_ptr(), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
              cos_tab.data_ptr(), sin_tab.data_ptr(), positions.data_ptr(), q.data_ptr(), k_cache.data_ptr(),
              v_cache.data_ptr(), B, T, Nq, Nkv, D, CAP, cos_tab.shape[0], float(eps), _stream())
    return q


# --------------------------------------------------------------- attention

def choose_num_splits(B: int, Nkv: int, cap: int, T: int = 1) -> int:
    """Context splits per (sequence, KV head, query) for a decode shape.

    Targets about 256 workgroups (one per CU) while keeping at least 128 cache
    slots per split; power of two in [1, 64]. Fixed per captured graph, as in
    the reference (``attention.py:94-110``), where the target was 264 programs.
    """
    if B * Nkv * T <= 8:   # one sequence: the cross-workgroup merge costs more than it saves (measured)
        return 1
    want = max(1, math.ceil(256 / max(1, B * Nkv * T)))
    limit = max(1, cap // 128)
    s = 1
    while s * 2 <= min(want, limit, 64):
        s *= 2
    return s


def attn_waves(B: int, T: int) -> int:
    """Wavefronts per attention workgroup (measured on MI355X at B = 1, 8, 32): 4 up to eight
    query rows, 8 once the context stream dominates."""
    return 8 if B * T >= 16 and T == 1 else 4



ATTN_WAVES = 8   # wavefronts per attention workgroup


def attn_workspace_bytes(B, T, Nq, Nkv, D, num_splits) -> int:
    return _lib.query("qwen_attn_workspace_bytes", B, T, Nq, Nkv, D, num_splits)


def attn_workspace(B, T, Nq, Nkv, D, num_splits, device) -> torch.Tensor:
    """Zeroed workspace for ``num_splits > 1`` (split partials + arrival counters that
    every launch re-arms to zero, so one allocation serves any number of launches)."""
    return torch.zeros(max(16, attn_workspace_bytes(B, T, Nq, Nkv, D, num_splits)), dtype=torch.uint8,
                       device=device)


def attn_decode(q, k_cache, v_cache, lengths, scale, num_splits, *, len_add: int = 0,
                out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                waves: int = ATTN_WAVES) -> torch.Tensor:
    """Causal decode attention of ``T`` new queries over the cache (``attention.py:278-348``).

    ``lengths [B]`` int32 counts valid slots including the ``T`` new ones
    (plus ``len_add``); returns ``[B, T, Nq * D]`` bf16.
    """
    _gpu(q, k_cache, v_cache, lengths)
    B, T, Nq, D = q.shape
    Bk, Nkv, CAP, Dk = k_cache.shape
    assert Bk == B and Dk == D and v_cache.shape == k_cache.shape, "q / cache shape mismatch"
    assert q.dtype == BF16 and k_cache.dtype == BF16 and v_cache.dtype == BF16
    assert k_cache.is_contiguous() and v_cache.is_contiguous(), "KV cache must be contiguous"
    assert lengths.dtype == torch.int32 and lengths.numel() == B and lengths.is_contiguous()
    assert Nq == 4 * Nkv and D == 128 and 1 <= T <= 16, "kernel supports G = 4, D = 128, T <= 16"
    S = int(num_splits)
    assert S >= 1
    q = q.contiguous()
    if workspace is None:
        workspace = attn_workspace(B, T, Nq, Nkv, D, S, q.device)
    o = out if out is not None else torch.empty((B, T, Nq * D), dtype=BF16, device=q.device)
    _lib.call("qwen_attn_decode", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), lengths.data_ptr(),
              int(len_add), o.data_ptr(), workspace.data_ptr(), workspace.numel(), B, T, Nq, Nkv, D, CAP,
              float(scale), S, int(waves), _stream())
    return o


def attn_decode_fused(qkv, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, positions, T, k_cache, v_cache, scale,
                      num_splits, *, out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                      waves: int = ATTN_WAVES) -> torch.Tensor:
    """``qk_norm_rope_cache`` followed by ``attn_decode`` in one launch (decode step).

    Same arguments and effects as the two reference ops in sequence
    (``rope.py:169-226``, ``attention.py:278-348``): K/V of tokens
    ``positions[b] + t`` are written to the caches, and the attention output of
    the T new queries (lengths ``positions + T``) is returned as ``[B, T, Nq*D]``.
    """
    _gpu(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache)
    B, Nkv, CAP, D = k_cache.shape
    M, W = qkv.shape
    assert D == 128 and W % D == 0 and W // D > 2 * Nkv, f"qkv width {W} vs {Nkv} KV heads of {D}"
    Nq = W // D - 2 * Nkv
    assert Nq == 4 * Nkv and M == B * T and 1 <= T <= 16, "G = 4, rows = B*T, T <= 16"
    assert qkv.dtype == BF16 and qkv.is_contiguous()
    assert k_cache.is_contiguous() and v_cache.is_contiguous() and v_cache.shape == k_cache.shape
    assert k_cache.dtype == BF16 and v_cache.dtype == BF16
    assert q_norm_w.numel() == D and k_norm_w.numel() == D and q_norm_w.is_contiguous() and k_norm_w.is_contiguous()
    assert cos_tab.dim() == 2 and cos_tab.shape[1] == D and cos_tab.is_contiguous() and sin_tab.shape == cos_tab.shape
    assert cos_tab.dtype == BF16 and sin_tab.dtype == BF16
    assert positions.dtype == torch.int32 and positions.numel() == B and positions.is_contiguous()
    S = int(num_splits)
    assert S >= 1
    if workspace is None:
        workspace = attn_workspace(B, T, Nq, Nkv, D, S, qkv.device)
    o = out if out is not None else torch.empty((B, T, Nq * D), dtype=BF16, device=qkv.device)
    _lib.call("qwen_attn_decode_fused", qkv.data_ptr(), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
              cos_tab.data_ptr(), sin_tab.data_ptr(), positions.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              o.data_ptr(), workspace.data_ptr(), workspace.numel(), B, T, Nq, Nkv, D, CAP, cos_tab.shape[0],
              float(eps), float(scale), S, int(waves), _stream())
    return o


MFMA_MAX_T = 8
MFMA_MAX_SPLITS = 8
MFMA_WAVES = 8
ATTN_KV_CACHED = 1   # qwen_attn_decode_mfma_ex flag: cache-allocating K/V loads


def choose_mfma_splits(B: int, Nkv: int, cap: int) -> int:
    """Context splits of ``attn_decode_mfma`` for a decode shape: about 256 workgroups (one
    per CU, each serving every query row of its KV head), at most 8, at least 512 cache slots
    per split (a split merge costs about what 512 keys of one workgroup's stream do).
    Measured on MI355X: B = 1 at context 300 one split 10.0 us, two 11.2; B = 1 at 4096
    eight splits 16 us, one 43; B = 8 at 2300 four; B = 32 at 8300 one; B = 4, T = 5 at
    4150 eight."""
    want = max(1, 256 // max(1, B * Nkv))
    return max(1, min(want, MFMA_MAX_SPLITS, max(1, cap // 512)))


def attn_mfma_workspace(B, T, Nkv, num_splits, device) -> torch.Tensor:
    """Zeroed workspace of ``attn_decode_mfma`` (split partials + re-armed arrival counters)."""
    return torch.zeros(max(16, _lib.query("qwen_attn_mfma_workspace_bytes", B, T, Nkv, num_splits)),
                       dtype=torch.uint8, device=device)


def attn_decode_mfma(qkv, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, positions, T, k_cache, v_cache, scale,
                     num_splits, *, out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                     waves: int = 4, kv_cached: bool = False) -> torch.Tensor:
    """``attn_decode_fused`` on the matrix cores (``T <= 8``, ``num_splits <= 8``).

    Same operator as the reference's ``qk_norm_rope_cache`` + ``attn_decode``
    (``rope.py:169-226``, ``attention.py:278-348``); one workgroup per (sequence,
    KV head, split) serves the ``4 T`` query rows of a KV head. ``kv_cached``: read the cached
    K/V with cache-allocating loads (for a KV cache that fits the Infinity Cache).
    """
    _gpu(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache)
    B, Nkv, CAP, D = k_cache.shape
    M, W = qkv.shape
    assert D == 128 and W % D == 0 and W // D > 2 * Nkv, f"qkv width {W} vs {Nkv} KV heads of {D}"
    Nq = W // D - 2 * Nkv
    assert Nq == 4 * Nkv and M == B * T and 1 <= T <= MFMA_MAX_T, "G = 4, rows = B*T, T <= 8"
    assert qkv.dtype == BF16 and qkv.is_contiguous()
    assert k_cache.is_contiguous() and v_cache.is_contiguous() and v_cache.shape == k_cache.shape
    assert k_cache.dtype == BF16 and v_cache.dtype == BF16
    assert q_norm_w.numel() == D and k_norm_w.numel() == D and q_norm_w.is_contiguous() and k_norm_w.is_contiguous()
    assert cos_tab.dim() == 2 and cos_tab.shape[1] == D and cos_tab.is_contiguous() and sin_tab.shape == cos_tab.shape
    assert cos_tab.dtype == BF16 and sin_tab.dtype == BF16
    assert positions.dtype == torch.int32 and positions.numel() == B and positions.is_contiguous()
    S = int(num_splits)
    assert 1 <= S <= MFMA_MAX_SPLITS and waves in (4, 8)
    if workspace is None:
        workspace = attn_mfma_workspace(B, T, Nkv, S, qkv.device)
    o = out if out is not None else torch.empty((B, T, Nq * D), dtype=BF16, device=qkv.device)
    assert o.is_contiguous() and o.numel() == B * T * Nq * D and o.dtype == BF16
    _lib.call("qwen_attn_decode_mfma_ex", qkv.data_ptr(), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
              cos_tab.data_ptr(), sin_tab.data_ptr(), positions.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              o.data_ptr(), workspace.data_ptr(), workspace.numel(), B, T, Nq, Nkv, D, CAP, cos_tab.shape[0],
              float(eps), float(scale), S, int(waves), ATTN_KV_CACHED if kv_cached else 0, _stream())
    return o


ATTN_NOALLOC_SCRATCH_BYTES = 8 << 20   # qwen_attn_decode_mfma_noalloc's fixed scratch per GPU


def attn_decode_mfma_noalloc(qkv, q_norm_w, k_norm_w, eps, cos_tab, sin_tab, positions, T, k_cache, v_cache, scale,
                             num_splits, *, out: torch.Tensor, waves: int = 4, kv_cached: bool = False) -> torch.Tensor:
    """``attn_decode_mfma`` through the allocation-free entry point: the split partials live in
    the library's fixed per-GPU scratch (``ATTN_NOALLOC_SCRATCH_BYTES``), ``out`` is the caller's.
    Raises ``RuntimeError`` (status 1004) when the shape needs more scratch than that."""
    _gpu(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out)
    B, Nkv, CAP, D = k_cache.shape
    M, W = qkv.shape
    Nq = W // D - 2 * Nkv
    assert M == B * T and qkv.dtype == BF16 and qkv.is_contiguous() and k_cache.is_contiguous()
    assert v_cache.is_contiguous() and v_cache.shape == k_cache.shape and positions.dtype == torch.int32
    assert cos_tab.shape == sin_tab.shape and cos_tab.is_contiguous() and sin_tab.is_contiguous()
    assert out.is_contiguous() and out.numel() == B * T * Nq * D and out.dtype == BF16
    _lib.call("qwen_attn_decode_mfma_noalloc", qkv.data_ptr(), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
              cos_tab.data_ptr(), sin_tab.data_ptr(), positions.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
              out.data_ptr(), B, T, Nq, Nkv, D, CAP, cos_tab.shape[0], float(eps), float(scale), int(num_splits),
              int(waves), ATTN_KV_CACHED if kv_cached else 0, _stream())
    return out


# ------------------------------------------------------- weights + GEMMs

class TiledWeight:
    """A projection weight ``[N, K]`` stored in MFMA-B tiles (see ``include/qwen_hip.h``).

    ``pair`` marks a gate|up weight whose 16-row tiles are interleaved
    (gate tile p, up tile p) for the SwiGLU epilogue.
    """

    __slots__ = ("data", "N", "K", "pair")

    def __init__(self, data: torch.Tensor, N: int, K: int, pair: bool = False):
        assert data.dtype == BF16 and data.numel() == N * K and data.is_contiguous()
        assert N % 16 == 0 and K % 32 == 0
        self.data, self.N, self.K, self.pair = data, int(N), int(K), bool(pair)

    @property
    def nbytes(self) -> int:
        return self.data.numel() * 2

    @classmethod
    def empty(cls, N: int, K: int, device, pair: bool = False):
        return cls(torch.empty(N * K, dtype=BF16, device=device), N, K, pair)

    @classmethod
    def random(cls, N, K, seg_start, seg_tid, seed, scale, device, pair=False):
        """Fill from the counter-based generator (``qwen_init_weight``)."""
        t = cls.empty(N, K, device, pair)
        init_weight(t.data, N, K, True, pair, seg_start, seg_tid, seed, scale)
        return t


def init_weight(dst: torch.Tensor, N, K, tiled, pair, seg_start, seg_tid, seed, scale) -> None:
    _gpu(dst)
    n = len(seg_start)
    assert n == len(seg_tid) and 1 <= n <= 4
    starts = (ctypes.c_int * n)(*[int(v) for v in seg_start])
    tids = (ctypes.c_int * n)(*[int(v) for v in seg_tid])
    _lib.call("qwen_init_weight", dst.data_ptr(), int(N), int(K), int(bool(tiled)), int(bool(pair)), starts, tids,
              n, int(seed), float(scale), _stream())


def tile_weight(w: torch.Tensor, pair: bool = False) -> TiledWeight:
    """Re-lay a row-major ``[N, K]`` bf16 weight into MFMA-B tiles."""
    _gpu(w)
    assert w.dtype == BF16 and w.dim() == 2
    w = w.contiguous()
    N, K = w.shape
    t = TiledWeight.empty(N, K, w.device, pair)
    _lib.call("qwen_tile_weight", w.data_ptr(), t.data.data_ptr(), N, K, int(pair), _stream())
    return t


# Measured launch shapes (ntw, waves, ksplit) for the Qwen3-4B projections on
# MI355X (graph-replayed, 36 weight copies rotated), keyed by (N, K, SwiGLU
# pair) and by M == 1, M <= 16 (one A fragment) or M <= 32 (two).
_TUNED = {   # per M class: 1, <= 16, <= 24, <= 32 rows
    (6144, 2560, False): {1: (2, 8, 1), 16: (2, 8, 1), 24: (2, 4, 1), 32: (4, 4, 2)},                  # QKV
    (2560, 4096, False): {1: (1, 8, 1), 16: (1, 8, 1), 24: (2, 8, 3), 32: (2, 4, 3)},                  # O
    (19456, 2560, True): {1: (2, 8, 1), 16: (2, 8, 1), 24: (2, 16, 256, 1), 32: (2, 16, 256, 1)},      # gate/up
    (2560, 9728, False): {1: (1, 16, 1), 16: (2, 4, 3), 24: (2, 4, 3), 32: (2, 4, 3)},                 # down
}


def gemm_config(M: int, N: int, K: int, silu_pair: bool = False) -> tuple:
    """Launch shape for ``x[M, K] @ W[N, K]^T``: ``(ntw, waves, ksplit)`` for ``qwen_linear``
    or ``(ntw, waves, gn, gk)`` for the rectangle launch ``qwen_linear_rect``.

    ``ksplit == 0`` selects the stream-K launch (one workgroup of 8 wavefronts
    per CU, equal weight bytes per CU). Known Qwen3-4B shapes use the measured
    table (MI355X, graph-replayed over rotated weight copies: the rectangle launch wins
    only for gate/up at M > 16, 25.5 vs 31.5 us at M = 32; QKV's 384 and O / down's 160
    n-tiles cannot be spread evenly over 256 CUs without a split-K merge that costs as
    much as the imbalance; down at M = 20 / 32 takes 17.3 / 18.8 us with three k-splits
    against 19.1 / 21.0 with two); otherwise: 8 wavefronts per
    workgroup and enough workgroups (n-tile groups x k-splits) to give about
    four per CU on 256 CUs, keeping at least 4 k-steps (4 KB of weight per
    n-tile) per wavefront.
    """
    tuned = _TUNED.get((N, K, bool(silu_pair)))
    if tuned is not None:
        return tuned[1 if M == 1 else (16 if M <= 16 else (24 if M <= 24 else 32))]
    ntw = 2 if silu_pair else 1
    waves = 8 if K // 32 >= 32 else 4
    units = N // (16 * ntw)
    KT = K // 32
    ks = 1
    while ks < 64 and units * ks < 1024 and KT // (ks * 2 * waves) >= 4:
        ks *= 2
    return ntw, waves, ks


def linear_workspace_bytes(M: int, N: int, ntw: int, ks: int) -> int:
    return _lib.query("qwen_linear_workspace_bytes", M, N, ntw, ks)


def gemm_workspace_bytes(M: int, N: int, cfg) -> int:
    """Split-K workspace bytes of a ``gemm_config`` launch shape (either form)."""
    if len(cfg) == 4:
        ntw, _, _, gk = cfg
        return linear_workspace_bytes(M, N, ntw, gk) if gk > 1 else 0
    ntw, _, ks = cfg
    return linear_workspace_bytes(M, N, ntw, ks)


def gemm_kernel_name(M: int, cfg, norm: bool, epi: int) -> str:
    """Kernel symbol (as rocprofv3 prints it) that ``fused_linear`` launches for ``cfg``."""
    mt = 2 if M > 16 else 1
    flag = "true" if norm else "false"
    if len(cfg) == 4:
        return f"rect_gemm_kernel<{mt}, {cfg[0]}, {cfg[1]}, {flag}, {epi}>"
    if cfg[2] == 0:
        return f"sk_gemm_kernel<{mt}, {cfg[0]}, {flag}, {epi}>"
    return f"skinny_gemm_kernel<{mt}, {cfg[0]}, {cfg[1]}, {flag}, {epi}>"


def linear_workspace(nbytes: int, device) -> torch.Tensor:
    """Zeroed split-K workspace (partials + arrival counters; every launch re-arms the
    counters, so one allocation serves any sequence of launches on one stream)."""
    return torch.zeros(max(256, int(nbytes)), dtype=torch.uint8, device=device)


def sumsq16(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-16-column partial sums of squares ``[M, K/16]`` fp32 (the RMSNorm statistics)."""
    _gpu(x)
    assert x.dtype == BF16 and x.dim() == 2 and x.is_contiguous() and x.shape[1] % 16 == 0
    M, K = x.shape
    if out is None:
        out = torch.empty((M, K // 16), dtype=torch.float32, device=x.device)
    _lib.call("qwen_sumsq16", x.data_ptr(), out.data_ptr(), M, K, _stream())
    return out


def fused_linear(x: torch.Tensor, w: TiledWeight, cfg=None, *, norm_w=None, eps: float = 0.0, residual=None,
                 silu_pair: bool = False, out: torch.Tensor | None = None, psq_in: torch.Tensor | None = None,
                 psq_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ w.T`` with optional RMSNorm prologue and residual / SwiGLU epilogue (``gemm_fused.py:136-173``).

    ``x [M <= 32, K]`` bf16; ``w`` tiled ``[N, K]`` (for ``silu_pair`` a pair-
    interleaved ``cat(gate, up)`` and the output is ``[M, N/2]``); ``norm_w [K]``;
    ``residual [M, N]`` (may be the same tensor as ``out``). ``cfg`` is
    ``(ntw, waves, ksplit)`` or ``None`` for ``gemm_config``. ``psq_in`` are x's
    ``sumsq16`` partials (computed here when omitted); ``psq_out`` receives the
    partials of a residual output. ``workspace``: a zeroed buffer of at least
    ``linear_workspace_bytes`` (allocated here when omitted and needed).
    """
    _gpu(x, norm_w, residual, out, psq_in, psq_out, workspace)
    assert x.dtype == BF16 and x.dim() == 2 and x.is_contiguous()
    M, K = x.shape
    assert K == w.K and 1 <= M <= 32, f"x [{M}, {K}] vs weight K={w.K}; M must be in [1, 32]"
    assert not (silu_pair and residual is not None)
    assert silu_pair == w.pair, "silu_pair requires a pair-interleaved weight (and only then)"
    if norm_w is not None:
        assert norm_w.dtype == BF16 and norm_w.numel() == K and norm_w.is_contiguous()
        if psq_in is None:
            psq_in = sumsq16(x)
        assert psq_in.dtype == torch.float32 and psq_in.shape == (M, K // 16) and psq_in.is_contiguous()
    ncols = w.N // 2 if silu_pair else w.N
    if residual is not None:
        assert residual.shape == (M, ncols) and residual.dtype == BF16 and residual.is_contiguous()
    if psq_out is not None:
        assert residual is not None and psq_out.shape == (M, ncols // 16) and psq_out.dtype == torch.float32
    if out is None:
        out = torch.empty((M, ncols), dtype=BF16, device=x.device)
    assert out.shape == (M, ncols) and out.is_contiguous()
    if cfg is None:
        cfg = gemm_config(M, w.N, K, silu_pair)
    epi = EPI_SWIGLU if silu_pair else (EPI_RES if residual is not None else EPI_STORE)
    if len(cfg) == 4:   # rectangle decomposition (ntw, waves, gn, gk)
        ntw, waves, gn, gk = cfg
        need = linear_workspace_bytes(M, w.N, ntw, gk) if gk > 1 else 0
        if need and workspace is None:
            workspace = linear_workspace(need, x.device)
        _lib.call("qwen_linear_rect", x.data_ptr(), w.data.data_ptr(), out.data_ptr(), M, w.N, K, ncols,
                  _nullable(norm_w), _nullable(psq_in), float(eps), _nullable(residual), _nullable(psq_out), epi,
                  ntw, waves, gn, gk, _nullable(workspace), 0 if workspace is None else workspace.numel(), _stream())
        return out
    ntw, waves, ks = cfg
    need = linear_workspace_bytes(M, w.N, ntw, ks)
    if need and workspace is None:
        workspace = linear_workspace(need, x.device)
    _lib.call("qwen_linear", x.data_ptr(), w.data.data_ptr(), out.data_ptr(), M, w.N, K, ncols, _nullable(norm_w),
              _nullable(psq_in), float(eps), _nullable(residual), _nullable(psq_out), epi, ntw, waves, ks,
              _nullable(workspace), 0 if workspace is None else workspace.numel(), _stream())
    return out


RECT_LDS_MAX = 160 * 1024


def rect_fits(M: int, N: int, K: int, ntw: int, waves: int, gn: int, gk: int, norm: bool = True) -> bool:
    """Host mirror of the library's admission rule for a rectangle launch."""
    if not (1 <= M <= 32 and K % 32 == 0 and ntw in (1, 2) and waves in (8, 16) and N % (16 * ntw) == 0):
        return False
    NU, KT = N // (16 * ntw), K // 32
    if not (1 <= gn <= NU and gk >= 1 and KT % (4 * gk) == 0):
        return False
    kc = KT // gk
    if kc * 4 > 64 * 5 or M > 2 * waves or (norm and K // 16 > 64 * 4) or -(-NU // gn) > waves:
        return False
    MT = 2 if M > 16 else 1
    rows = M + 1 if M < 16 * MT else M   # the zero row that padding rows of the 16-row tiles read
    return max(rows * kc * 64, waves * 2 * MT * ntw * 64 * 16) <= RECT_LDS_MAX


def rect_config(M: int, N: int, K: int, silu_pair: bool = False, cus: int = 256, waves: int = 16,
                norm: bool = True):
    """(ntw, waves, gn, gk) of the rectangle launch: gn * gk = the CU count (or twice it), the
    split of the (unit, k-step) plane whose largest rectangle is closest to the average, with a
    small charge per k-group for the split-K partials; None if no split fits."""
    ntw = 2 if silu_pair else 1
    NU, KT = N // (16 * ntw), K // 32
    MT = 2 if M > 16 else 1
    best, best_cost = None, None
    for mult in (1, 2):
        G = cus * mult
        for gk in range(1, min(KT // 4, 64) + 1):
            if G % gk:
                continue
            gn = G // gk
            if not rect_fits(M, N, K, ntw, waves, gn, gk, norm):
                continue
            if mult > 1 and waves == 16:   # a CU holds one 16-wavefront workgroup: two rounds
                continue
            imbalance = (-(-NU // gn)) * (-(-KT // gk)) / (NU * KT / G)
            # a split-K merge (store, count, re-load) costs about a quarter of a small GEMM
            cost = imbalance + (0.25 if gk > 1 else 0.0) + 0.02 * (mult - 1)
            if best_cost is None or cost < best_cost - 1e-9:
                best, best_cost = (ntw, waves, gn, gk), cost
    return best


# ----------------------------------------------------------- prompt forward

PF_BN, PF_BK = 128, 64   # qwen_gemm: N must be a multiple of PF_BN, K of PF_BK


def gemm(x: torch.Tensor, w: TiledWeight, *, residual: torch.Tensor | None = None, silu_pair: bool = False,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ w.T`` for any number of rows over a tiled weight (the prompt forward's projections,
    ``engine/engine.py:1191-1221``), fp32 accumulation and one rounding, with the fused epilogues of
    ``gemm_fused.py:136-173``: ``residual`` -> ``bf16(residual + bf16(acc))`` (``out`` may be the
    residual itself); ``silu_pair`` (pair-interleaved gate|up weight) -> the SwiGLU product
    ``[M, N/2]``."""
    _gpu(x, residual, out)
    assert x.dtype == BF16 and x.dim() == 2 and x.is_contiguous()
    M, K = x.shape
    assert K == w.K and w.N % PF_BN == 0 and K % PF_BK == 0, f"gemm: x [{M}, {K}] vs weight [{w.N}, {w.K}]"
    assert silu_pair == w.pair and not (silu_pair and residual is not None)
    ncols = w.N // 2 if silu_pair else w.N
    if residual is not None:
        assert residual.shape == (M, ncols) and residual.dtype == BF16 and residual.is_contiguous()
    if out is None:
        out = torch.empty((M, ncols), dtype=BF16, device=x.device)
    assert out.shape == (M, ncols) and out.dtype == BF16 and out.is_contiguous()
    epi = EPI_SWIGLU if silu_pair else (EPI_RES if residual is not None else EPI_STORE)
    _lib.call("qwen_gemm", x.data_ptr(), w.data.data_ptr(), out.data_ptr(), M, w.N, K, ncols, _nullable(residual),
              epi, _stream())
    return out


def attn_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, p0: int, scale: float,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal attention of a prompt chunk: ``q [B, T, Nq, D]`` holds the (normed, rotated) queries
    of positions ``p0 .. p0 + T - 1`` of every sequence, whose keys and values are already in the
    caches ``[B, Nkv, CAP, D]``; query ``t`` sees slots ``[0, p0 + t]``. Returns
    ``[B, T, Nq * D]`` bf16 (``engine/engine.py:1123-1179``)."""
    _gpu(q, k_cache, v_cache, out)
    B, T, Nq, D = q.shape
    Bk, Nkv, CAP, Dk = k_cache.shape
    assert Bk == B and Dk == D and v_cache.shape == k_cache.shape and Nq == 4 * Nkv and D == 128
    assert q.dtype == BF16 and q.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous()
    assert 0 <= p0 and p0 + T <= CAP
    if out is None:
        out = torch.empty((B, T, Nq * D), dtype=BF16, device=q.device)
    assert out.shape == (B, T, Nq * D) and out.is_contiguous()
    _lib.call("qwen_attn_prefill", q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(), B, T, Nq,
              Nkv, D, CAP, int(p0), float(scale), _stream())
    return out


GEMV_MAX_M = 2   # rows handled by the balanced row-major GEMV (qwen_gemv)
GEPI_STORE, GEPI_RES, GEPI_SWIGLU, GEPI_ARGMAX = 0, 1, 2, 3


def cu_count(device=None) -> int:
    return torch.cuda.get_device_properties(device if device is not None else 0).multi_processor_count


def gemv_config(M: int, N: int, K: int, epi: int, device=None) -> tuple[int, int]:
    """(grid, waves) for qwen_gemv (measured on MI355X, graph-replayed over 36 layers): one
    workgroup of 8 wavefronts per CU, so every CU streams the same bytes; the SwiGLU projection
    (the largest) runs two workgroups per CU."""
    cus = cu_count(device)
    return (2 * cus if epi == GEPI_SWIGLU else cus), 8


def gemv(x: torch.Tensor, w: torch.Tensor, *, norm_w=None, eps: float = 0.0, residual=None, silu_pair: bool = False,
         out: torch.Tensor | None = None, amax: torch.Tensor | None = None, cfg=None,
         row_map: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ w.T`` for ``x [M <= 2, K]`` over a row-major ``w [N, K]`` (``gemm_fused.py:136-173``
    semantics): optional RMSNorm prologue (``norm_w``), residual or SwiGLU epilogue
    (``silu_pair``: ``w = cat(gate, up)`` rows, output ``[M, N/2]``), or, with ``amax``, the
    first-index argmax of the bf16 logits folded into the packed int64 keys (LM head).
    ``row_map`` (store epilogue only; int32 ``[N]``, a permutation): weight row ``i``'s output
    goes to column ``row_map[i]``.
    """
    _gpu(x, w, norm_w, residual, out, amax)
    assert x.dtype == BF16 and x.dim() == 2 and x.is_contiguous()
    assert w.dtype == BF16 and w.dim() == 2 and w.is_contiguous()
    M, K = x.shape
    assert 1 <= M <= GEMV_MAX_M and w.shape[1] == K and K % 512 == 0, f"gemv: x [{M}, {K}], w {tuple(w.shape)}"
    if amax is not None:
        epi = GEPI_ARGMAX
        assert norm_w is not None and residual is None and not silu_pair
        assert amax.dtype == torch.int64 and amax.numel() >= argmax_keys_count(M) and amax.is_contiguous()
    elif silu_pair:
        epi = GEPI_SWIGLU
        assert norm_w is not None and residual is None and w.shape[0] % 2 == 0
    elif residual is not None:
        epi = GEPI_RES
        assert norm_w is None
    else:
        epi = GEPI_STORE
    N = w.shape[0] // 2 if silu_pair else w.shape[0]
    if norm_w is not None:
        assert norm_w.dtype == BF16 and norm_w.numel() == K and norm_w.is_contiguous()
    if epi != GEPI_ARGMAX:
        if residual is not None:
            assert residual.shape == (M, N) and residual.dtype == BF16 and residual.is_contiguous()
        if out is None:
            out = torch.empty((M, N), dtype=BF16, device=x.device)
        assert out.shape == (M, N) and out.is_contiguous() and out.dtype == BF16
    grid, waves = cfg if cfg is not None else gemv_config(M, N, K, epi, x.device)
    if row_map is None:
        _lib.call("qwen_gemv", x.data_ptr(), w.data_ptr(), _nullable(out) if epi != GEPI_ARGMAX else None, M, N, K,
                  N, _nullable(norm_w), float(eps), _nullable(residual), epi, _nullable(amax), int(grid), int(waves),
                  _stream())
    else:
        _gpu(row_map)
        assert epi == GEPI_STORE and row_map.dtype == torch.int32 and row_map.numel() == N and row_map.is_contiguous()
        _lib.call("qwen_gemv_rowmap", x.data_ptr(), w.data_ptr(), out.data_ptr(), M, N, K, N, _nullable(norm_w),
                  float(eps), None, epi, None, row_map.data_ptr(), int(grid), int(waves), _stream())
    return amax if epi == GEPI_ARGMAX else out


def lm_head_config(M: int, N: int, K: int) -> tuple[int, int]:
    """(ntw, waves) for the LM head: the vocabulary gives thousands of workgroups already, so
    each workgroup takes the widest unit (up to 8 n-tiles) that divides N and shares each
    activation load and normalisation over it. Measured on MI355X (N = 151936, graph of 20
    launches): M = 32 194 us at (8, 4) vs 257 at (4, 8); M = 20 176 vs 198; M = 8 144 vs 168."""
    if M == 1:
        return (2, 8)
    for ntw in (8, 4, 2, 1):
        if N % (16 * ntw) == 0:
            return (ntw, 4) if ntw == 8 else (ntw, 8)
    return (1, 8)


ARGMAX_SLOTS = 8   # QWEN_ARGMAX_SLOTS: key slots per row (atomics of the LM head spread over them)


def argmax_keys_count(M: int) -> int:
    """Words of an M-row key buffer (``QWEN_ARGMAX_KEYS``): slot s of row m at s * ld + m."""
    return ARGMAX_SLOTS * ((M + 15) // 16 * 16)


def argmax_keys(M: int, device) -> torch.Tensor:
    """Packed (logit, index) argmax keys of M rows, zeroed; every consumer re-arms them."""
    return torch.zeros((argmax_keys_count(M),), dtype=torch.int64, device=device)


def lm_head_argmax(x: torch.Tensor, norm_w: torch.Tensor, eps: float, w: TiledWeight, *, cfg=None,
                   out: torch.Tensor | None = None, keys: torch.Tensor | None = None,
                   psq_in: torch.Tensor | None = None, extract: bool = True) -> torch.Tensor:
    """Final RMSNorm + tied LM head + first-index argmax over bf16 logits -> int64 ``[M]``.

    ``keys``: zeroed int64 ``[M]`` packed-argmax buffer (allocated when omitted).
    With ``extract=False`` the tokens stay in ``keys`` for ``decode_finish``.
    """
    _gpu(x, norm_w, out, keys, psq_in)
    assert x.dtype == BF16 and x.dim() == 2 and x.is_contiguous()
    M, K = x.shape
    assert K == w.K and 1 <= M <= 32 and not w.pair
    if psq_in is None:
        psq_in = sumsq16(x)
    ntw, waves = cfg if cfg is not None else lm_head_config(M, w.N, K)
    if keys is None:
        keys = argmax_keys(M, x.device)
    assert keys.dtype == torch.int64 and keys.numel() >= argmax_keys_count(M) and keys.is_contiguous()
    if extract and out is None:
        out = torch.empty((M,), dtype=torch.int64, device=x.device)
    _lib.call("qwen_lm_head_argmax", x.data_ptr(), norm_w.data_ptr(), psq_in.data_ptr(), float(eps),
              w.data.data_ptr(), M, w.N, K, keys.data_ptr(), out.data_ptr() if extract else None, ntw, waves,
              _stream())
    return out if extract else keys


def argmax_extract(keys: torch.Tensor, M: int, out: torch.Tensor) -> torch.Tensor:
    """Tokens of packed argmax keys (re-arms the keys to zero)."""
    assert keys.dtype == torch.int64 and keys.numel() >= argmax_keys_count(M) and keys.is_contiguous()
    _lib.call("qwen_argmax_extract", keys.data_ptr(), int(M), out.data_ptr(), _stream())
    return out


def decode_finish(keys, nxt, hist, pos, s_buf, ntarget, w: TiledWeight, h, psq) -> None:
    """Step tail (``engine/engine.py:941-953``) + next step's embedding: token from the
    argmax keys, history / position update, ``h = W[hist[pos]]`` and its statistics."""
    B, cap = hist.shape
    assert keys.dtype == torch.int64 and keys.numel() >= argmax_keys_count(B) and keys.is_contiguous()
    _lib.call("qwen_decode_finish", keys.data_ptr(), nxt.data_ptr(), hist.data_ptr(), pos.data_ptr(),
              s_buf.data_ptr(), ntarget.data_ptr(), w.data.data_ptr(), h.data_ptr(), psq.data_ptr(), B, cap, w.N,
              w.K, _stream())


def spec_draft(hist: torch.Tensor, pos: torch.Tensor, k: int, n: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """Prompt-lookup drafts ``[B, k+1]`` = ``[hist[L-1], draft...]`` (``engine/engine.py:955-977``)."""
    _gpu(hist, pos, out)
    B, cap = hist.shape
    assert hist.dtype == torch.int64 and hist.is_contiguous()
    assert pos.dtype == torch.int32 and pos.numel() == B and pos.is_contiguous()
    if out is None:
        out = torch.empty((B, k + 1), dtype=torch.int64, device=hist.device)
    assert out.shape == (B, k + 1) and out.dtype == torch.int64 and out.is_contiguous()
    _lib.call("qwen_spec_draft", hist.data_ptr(), pos.data_ptr(), B, cap, int(k), int(n), out.data_ptr(), _stream())
    return out


def spec_accept(nxt, tok, hist, pos, s_buf, ntarget, w: TiledWeight, h, psq, out_t, adv) -> None:
    """Verify-step acceptance (``engine/engine.py:994-1003``): history scatter, position advance,
    ``out_t [T, B]`` / ``adv [B]`` for the host, and the next plain step's input row."""
    B, cap = hist.shape
    T = tok.shape[1]
    assert nxt.numel() == B * T and tok.shape == (B, T) and out_t.shape == (T, B) and adv.numel() == B
    _lib.call("qwen_spec_accept", nxt.data_ptr(), tok.data_ptr(), hist.data_ptr(), pos.data_ptr(), s_buf.data_ptr(),
              ntarget.data_ptr(), B, cap, T, out_t.data_ptr(), adv.data_ptr(), w.data.data_ptr(), h.data_ptr(),
              psq.data_ptr(), w.N, w.K, _stream())


def embed(tok: torch.Tensor, w: TiledWeight, out: torch.Tensor | None = None,
          psq_out: torch.Tensor | None = None) -> torch.Tensor:
    """``F.embedding(tok, W)`` from the tiled tied table; ``tok`` int64 ``[M]``."""
    _gpu(tok, psq_out)
    assert tok.dtype == torch.int64 and tok.is_contiguous()
    M = tok.numel()
    if out is None:
        out = torch.empty((M, w.K), dtype=BF16, device=tok.device)
    _lib.call("qwen_embed", tok.data_ptr(), None, None, 0, w.data.data_ptr(), out.data_ptr(), _nullable(psq_out),
              M, w.N, w.K, _stream())
    return out


def embed_hist(hist: torch.Tensor, pos: torch.Tensor, w: TiledWeight, out: torch.Tensor,
               psq_out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode-step embedding of ``hist[b, pos[b]]`` for every row ``b`` (``engine/engine.py:941-946``)."""
    B, cap = hist.shape
    _lib.call("qwen_embed", None, hist.data_ptr(), pos.data_ptr(), cap, w.data.data_ptr(), out.data_ptr(),
              _nullable(psq_out), B, w.N, w.K, _stream())
    return out
