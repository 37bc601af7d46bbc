"""GPU parity of the matrix-core decode attention (``qwen_attn_decode_mfma``).

Same operator as ``attn_decode_fused``: the reference's ``qk_norm_rope_cache``
(``engine/kernels/rope.py:169-226``) followed by ``attn_decode``
(``engine/kernels/attention.py:278-348``), checked against the CPU oracle on the
same seeded inputs with the fused test's bar (the reference's attention
tolerance, ``tests/test_torch_ref.py:421``), plus the cache writes, the slots it
must leave untouched, key blocks that straddle the context end, empty splits,
re-armed split counters and run-to-run determinism.
"""

import pytest
import torch

from helpers import assert_close
from oracle import ref_torch as R

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda:0"
EPS = 1e-6
NQ, NKV, D = 32, 8, 128


def _bf16(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * scale).to(BF16)


def _gain(n, gen):
    return (1.0 + 0.5 * torch.randn(n, generator=gen)).to(BF16)


@pytest.fixture(scope="module")
def qops():
    from qwen_hip import ops
    return ops


@pytest.fixture(scope="module")
def tables():
    cos, sin = R.rope_tables(8192, 5e6, D)
    return cos, sin, cos.to(DEV), sin.to(DEV)


def _case(B, T, positions, CAP, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = _bf16(B * T, (NQ + 2 * NKV) * D, gen=g, scale=2.0)
    kc, vc = _bf16(B, NKV, CAP, D, gen=g), _bf16(B, NKV, CAP, D, gen=g)
    qw, kw = _gain(D, g), _gain(D, g)
    return qkv, kc, vc, qw, kw, torch.tensor(positions, dtype=torch.int32)


def _check(got, want, kd, vd, kc, kc_ref, vc_ref, positions, T, what):
    # Bar of the fused kernel's test: RoPE's bf16(p1 + p2) can cancel, so a one-ulp change of
    # a normed input moves a few q/k elements by several ulps; at most 0.1% of the outputs
    # may sit outside atol 2e-2.
    assert_close(got, want, 2e-2, 2e-2, what)
    assert float(((got.float() - want.float()).abs() > 2e-2).float().mean()) <= 1e-3, what
    assert_close(kd, kc_ref, 1e-2, 1 / 64, "k_cache " + what)
    assert float((kd != kc_ref).float().mean()) <= 1e-2
    assert torch.equal(vd, vc_ref)     # V copied raw
    B, CAP = kc.shape[0], kc.shape[2]
    untouched = torch.ones(B, CAP, dtype=torch.bool)
    for b, p0 in enumerate(positions):
        untouched[b, p0:p0 + T] = False
    assert torch.equal(kd.permute(0, 2, 1, 3)[untouched], kc.permute(0, 2, 1, 3)[untouched])


@pytest.mark.parametrize("B,T,positions,splits,waves", [
    (1, 1, [0], 1, 4),                       # no cached key: the new-key block alone
    (1, 1, [1], 1, 8),
    (1, 1, [383], 1, 4),                     # 12 blocks minus one key: a ragged last block
    (1, 1, [4095], 8, 8),
    (2, 1, [5, 900], 8, 4),                  # sequence 0 has fewer blocks than splits: empty splits
    (4, 5, [4096, 100, 7, 0], 4, 8),         # T = 5: two 16-row tiles
    (3, 8, [16, 200, 1000], 2, 4),           # T = 8: 32 query rows, new keys 0..7 causal
    (2, 4, [31, 33], 3, 8),                  # split count that does not divide the blocks
    (8, 1, [2304, 1, 77, 2048, 999, 1500, 64, 65], 8, 8),
    (2, 2, [4000, 3000], 5, 4),
    (1, 6, [128], 1, 8),
    (3, 3, [63, 64, 65], 7, 4),
])
def test_attn_decode_mfma_matches_rope_then_attention(qops, tables, B, T, positions, splits, waves):
    cos, sin, cos_d, sin_d = tables
    CAP = 4160
    qkv, kc, vc, qw, kw, pos = _case(B, T, positions, CAP, 91 + 7 * B + T)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    q_ref = R.qk_norm_rope_cache(qkv, qw, kw, EPS, cos, sin, pos, T, kc_ref, vc_ref)
    want = R.attn_decode(q_ref, kc_ref, vc_ref, pos + T, D ** -0.5)
    kd, vd = kc.to(DEV), vc.to(DEV)
    got = qops.attn_decode_mfma(qkv.to(DEV), qw.to(DEV), kw.to(DEV), EPS, cos_d, sin_d, pos.to(DEV), T, kd, vd,
                                D ** -0.5, splits, waves=waves).cpu()
    assert got.shape == (B, T, NQ * D)
    _check(got, want, kd.cpu(), vd.cpu(), kc, kc_ref, vc_ref, positions, T, f"T={T} S={splits} W={waves}")


@pytest.mark.parametrize("T,splits,waves", [(1, 4, 8), (5, 8, 4), (8, 2, 8)])
def test_attn_decode_mfma_relaunch_and_determinism(qops, tables, T, splits, waves):
    """Several launches on one workspace (the split counters re-arm themselves) give bit-identical
    outputs, and they equal the fused CUDA-core kernel's result to the attention bar."""
    _, _, cos_d, sin_d = tables
    B, CAP = 3, 2048
    positions = [1500, 20, 777]
    qkv, kc, vc, qw, kw, pos = _case(B, T, positions, CAP, 5 + T)
    args = (qkv.to(DEV), qw.to(DEV), kw.to(DEV), EPS, cos_d, sin_d, pos.to(DEV), T)
    ws = qops.attn_mfma_workspace(B, T, NKV, splits, DEV)
    outs = []
    for _ in range(3):
        kd, vd = kc.to(DEV), vc.to(DEV)
        outs.append(qops.attn_decode_mfma(*args, kd, vd, D ** -0.5, splits, workspace=ws, waves=waves).cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    kd, vd = kc.to(DEV), vc.to(DEV)
    fused = qops.attn_decode_fused(*args, kd, vd, D ** -0.5, 1).cpu()
    assert_close(outs[0], fused, 2e-2, 2e-2, "mfma vs fused")


def test_attn_decode_mfma_rejects_bad_shapes(qops, tables):
    _, _, cos_d, sin_d = tables
    B, T, CAP = 1, 9, 256
    qkv, kc, vc, qw, kw, pos = _case(B, T, [10], CAP, 1)
    with pytest.raises(AssertionError):
        qops.attn_decode_mfma(qkv.to(DEV), qw.to(DEV), kw.to(DEV), EPS, cos_d, sin_d, pos.to(DEV), T, kc.to(DEV),
                              vc.to(DEV), D ** -0.5, 1)
    from qwen_hip import _lib
    with pytest.raises(RuntimeError, match="qwen_attn_decode_mfma failed"):   # T = 9 refused by the library too
        _lib.call("qwen_attn_decode_mfma", 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, B, T, NQ, NKV, D, CAP, 8192, EPS,
                  D ** -0.5, 1, 4, 0)


@pytest.mark.parametrize("B,T,pos,CAP,splits", [(1, 1, [300], 448, 1), (2, 5, [40, 1000], 1088, 2), (1, 2, [4090], 4160, 8)])
def test_attn_decode_mfma_kv_cached_loads_change_nothing(qops, tables, B, T, pos, CAP, splits):
    """The cache-allocating K/V load policy gives the same output and cache writes, bit for bit."""
    _, _, cos_d, sin_d = tables
    qkv, kc, vc, qw, kw, p = _case(B, T, pos, CAP, 21 + B + T)
    args = (qkv.to(DEV), qw.to(DEV), kw.to(DEV), EPS, cos_d, sin_d, p.to(DEV), T)
    res = []
    for cached in (False, True):
        kd, vd = kc.to(DEV), vc.to(DEV)
        ws = qops.attn_mfma_workspace(B, T, NKV, splits, DEV)
        o = qops.attn_decode_mfma(*args, kd, vd, D ** -0.5, splits, workspace=ws, waves=8, kv_cached=cached)
        torch.cuda.synchronize()
        res.append((o.cpu(), kd.cpu(), vd.cpu()))
    for a, b in zip(res[0], res[1]):
        assert torch.equal(a, b)


def test_attn_decode_mfma_ex_rejects_unknown_flags(qops):
    from qwen_hip import _lib
    with pytest.raises(RuntimeError, match="qwen_attn_decode_mfma_ex failed"):
        _lib.call("qwen_attn_decode_mfma_ex", 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, 1, 1, NQ, NKV, D, 256, 8192, EPS,
                  D ** -0.5, 1, 8, 2, 0)
