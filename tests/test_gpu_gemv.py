"""GPU parity of the balanced row-major GEMV (``qwen_gemv``, M <= 2) against the CPU oracle.

Bars as for the MFMA projections: the reference's certification tolerance
(atol 1e-2, rtol 1/64, ``engine/engine.py:425-429``) on random inputs, bit-exact
on two-hot weights (every output is an exact sum in any order), and the argmax
identical to the oracle's first-index argmax except inside a one-ulp top-2 tie.
Shapes are the Qwen3-4B projections plus grids that leave workgroups with one
row, with rows split between wavefronts, or with no rows at all.
"""

import math

import pytest
import torch

from helpers import assert_close
from oracle import ref_torch as R

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda:0"
EPS = 1e-6


def _bf16(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * scale).to(BF16)


def _gain(n, gen):
    return (1.0 + 0.5 * torch.randn(n, generator=gen)).to(BF16)


@pytest.fixture(scope="module")
def qops():
    from qwen_hip import ops
    return ops


def _case(qops, M, N, K, kind, gen, cfg=None):
    """kind: plain | norm | res | silu (silu: N output columns, W = cat(gate, up) [2N, K])."""
    x = _bf16(M, K, gen=gen)
    rows = 2 * N if kind == "silu" else N
    w = _bf16(rows, K, gen=gen, scale=0.03)
    nw = _gain(K, gen) if kind in ("norm", "silu") else None
    resid = _bf16(M, N, gen=gen) if kind == "res" else None
    xin = R.rms_norm(x, nw, EPS) if nw is not None else x
    y = R.linear(xin, w)
    want = R.silu_mul(y) if kind == "silu" else y
    if resid is not None:
        want = (resid.float() + want.float()).to(BF16)
    r = None if resid is None else resid.to(DEV)
    got = qops.gemv(x.to(DEV), w.to(DEV), norm_w=None if nw is None else nw.to(DEV), eps=EPS, residual=r, out=r,
                    silu_pair=kind == "silu", cfg=cfg).cpu()
    return got, want


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("kind,N,K", [("norm", 6144, 2560), ("res", 2560, 4096), ("silu", 9728, 2560),
                                      ("res", 2560, 9728), ("plain", 1024, 512)])
def test_gemv_qwen_shapes(qops, M, kind, N, K):
    g = torch.Generator().manual_seed(7 + M + N + K)
    got, want = _case(qops, M, N, K, kind, g)
    assert_close(got, want, 1e-2, 1 / 64, f"{kind} {N}x{K} M={M}")


@pytest.mark.parametrize("grid,waves", [(1, 16), (7, 8), (100, 16), (300, 16), (513, 8)])
@pytest.mark.parametrize("kind", ["norm", "res", "silu"])
def test_gemv_grids(qops, grid, waves, kind):
    """Workgroups with many rows (grid 1), rows split across wavefronts, one row per
    workgroup, and workgroups without rows (grid > N)."""
    g = torch.Generator().manual_seed(grid * 3 + waves)
    N, K = 300, 1536
    got, want = _case(qops, 2, N, K, kind, g, cfg=(grid, waves))
    assert_close(got, want, 1e-2, 1 / 64, f"{kind} grid={grid} waves={waves}")


def test_gemv_two_hot_exact(qops):
    """Two exactly representable products per output: the bf16 bits are closed-form."""
    M, N, K = 2, 640, 1024
    g = torch.Generator().manual_seed(17)
    x = torch.randint(-8, 9, (M, K), generator=g).to(BF16)
    w = torch.zeros(N, K, dtype=BF16)
    cols = torch.randint(0, K, (N, 2), generator=g)
    for n in range(N):
        w[n, cols[n, 0]] += 0.5
        w[n, cols[n, 1]] += 0.25
    want = (x.double() @ w.double().T).to(BF16)
    for cfg in [(256, 16), (3, 8), (1000, 16)]:
        got = qops.gemv(x.to(DEV), w.to(DEV), cfg=cfg).cpu()
        assert torch.equal(got, want), cfg


def test_gemv_matches_mfma_kernel(qops):
    """The GEMV and the MFMA-tile kernel compute the same operator (different fp32 orders)."""
    g = torch.Generator().manual_seed(5)
    x = _bf16(1, 2560, gen=g)
    w = _bf16(6144, 2560, gen=g, scale=0.02)
    nw = _gain(2560, g)
    a = qops.gemv(x.to(DEV), w.to(DEV), norm_w=nw.to(DEV), eps=EPS).cpu()
    b = qops.fused_linear(x.to(DEV), qops.tile_weight(w.to(DEV)), norm_w=nw.to(DEV), eps=EPS).cpu()
    assert_close(a, b, 1e-2, 1 / 64, "gemv vs fused_linear")


def test_gemv_argmax_one_hot_exact(qops):
    """Rows of W are one-hot: every logit value repeats, so the first-index rule decides."""
    M, V, K = 2, 4096, 512
    g = torch.Generator().manual_seed(21)
    x = _bf16(M, K, gen=g)
    nw = torch.ones(K, dtype=BF16)
    w = torch.zeros(V, K, dtype=BF16)
    w[torch.arange(V), torch.arange(V) % K] = 1.0
    want = R.linear(R.rms_norm(x, nw, EPS), w).argmax(-1)
    assert bool((want < K).all())
    for cfg in [(256, 16), (5, 8), (4096, 16)]:
        keys = qops.argmax_keys(M, DEV)
        qops.gemv(x.to(DEV), w.to(DEV), norm_w=nw.to(DEV), eps=EPS, amax=keys, cfg=cfg)
        out = torch.empty(M, dtype=torch.int64, device=DEV)
        qops.argmax_extract(keys, M, out)
        assert torch.equal(out.cpu(), want), cfg


@pytest.mark.parametrize("M", [1, 2])
def test_gemv_argmax_lm_head(qops, M):
    V, K = 151936, 2560
    g = torch.Generator().manual_seed(31 + M)
    x = _bf16(M, K, gen=g)
    nw = _gain(K, g)
    w = _bf16(V, K, gen=g, scale=0.02)
    logits = R.linear(R.rms_norm(x, nw, EPS), w).float()
    keys = qops.argmax_keys(M, DEV)
    qops.gemv(x.to(DEV), w.to(DEV), norm_w=nw.to(DEV), eps=EPS, amax=keys)
    got = torch.empty(M, dtype=torch.int64, device=DEV)
    qops.argmax_extract(keys, M, got)
    got = got.cpu()
    top = logits.max(-1).values
    chosen = logits.gather(-1, got[:, None])[:, 0]
    ulp = torch.tensor([2.0 ** (math.floor(math.log2(abs(float(t)))) - 7) for t in top])
    assert bool(((top - chosen) <= ulp).all())
    exact = (top - logits.topk(2, -1).values[:, 1]) > 2 * ulp
    assert torch.equal(got[exact], logits.argmax(-1)[exact])


def test_gemv_rejects_bad_shapes(qops):
    x = torch.zeros(1, 520, dtype=BF16, device=DEV)
    w = torch.zeros(64, 520, dtype=BF16, device=DEV)
    with pytest.raises(AssertionError):          # K % 512 != 0
        qops.gemv(x, w)
    x = torch.zeros(1, 512, dtype=BF16, device=DEV)
    w = torch.zeros(64, 512, dtype=BF16, device=DEV)
    with pytest.raises(RuntimeError, match="bad size/shape"):   # 12 wavefronts: not built
        qops.gemv(x, w, cfg=(4, 12))


@pytest.mark.parametrize("M,N,K,grid", [(1, 6144, 2560, 256), (2, 6144, 2560, 256), (1, 300, 1536, 7)])
def test_gemv_row_map(qops, M, N, K, grid):
    """``qwen_gemv_rowmap``: with the weight's rows permuted and the inverse order as the row
    map, the output lands in its natural columns and matches the oracle at the GEMV bar; the
    two-hot case is bit-exact."""
    g = torch.Generator().manual_seed(31 + M + N)
    x = _bf16(M, K, gen=g)
    w = _bf16(N, K, gen=g, scale=0.03)
    nw = _gain(K, g)
    perm = torch.randperm(N, generator=g)
    want = R.linear(R.rms_norm(x, nw, EPS), w)
    got = qops.gemv(x.to(DEV), w[perm].contiguous().to(DEV), norm_w=nw.to(DEV), eps=EPS, cfg=(grid, 8),
                    row_map=perm.to(torch.int32).to(DEV)).cpu()
    assert_close(got, want, 1e-2, 1 / 64, f"row map {N}x{K} M={M}")
    xi = torch.randint(-8, 9, (M, K), generator=g).to(BF16)
    w2 = torch.zeros(N, K, dtype=BF16)
    cols = torch.randint(0, K, (N, 2), generator=g)
    for n in range(N):
        w2[n, cols[n, 0]] += 0.5
        w2[n, cols[n, 1]] += 0.25
    exact = (xi.double() @ w2.double().T).to(BF16)
    got2 = qops.gemv(xi.to(DEV), w2[perm].contiguous().to(DEV), cfg=(grid, 8), row_map=perm.to(torch.int32).to(DEV))
    assert torch.equal(got2.cpu(), exact)


def test_gemv_row_map_only_with_store(qops):
    from qwen_hip import _lib
    with pytest.raises(RuntimeError, match="qwen_gemv_rowmap failed"):   # residual epilogue + map: refused
        _lib.call("qwen_gemv_rowmap", 1, 1, 1, 1, 512, 512, 512, None, EPS, 1, 1, None, 1, 8, 8, 0)
