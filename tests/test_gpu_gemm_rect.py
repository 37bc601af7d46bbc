"""GPU parity of the rectangle-decomposed projection GEMM (``qwen_linear_rect``).

Same operator as ``fused_linear`` (``engine/kernels/gemm_fused.py:136-173``:
RMSNorm prologue, store / residual / SwiGLU epilogues, one bf16 rounding),
checked against the CPU oracle at the bar of the reference's op certification
(``engine/engine.py:425-429``: atol 1e-2, rtol 1/64), on the Qwen3-4B
projection shapes and on small shapes that exercise empty wavefront pieces,
pieces that straddle two units, uneven rectangles and split-K merges, each
launched twice on one workspace (re-armed counters, bit-identical results).
"""

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


def _run(qops, kind, M, N, K, cfg, seed):
    g = torch.Generator().manual_seed(seed)
    x = _bf16(M, K, gen=g)
    w = _bf16(N, K, gen=g, scale=0.03)
    nw = _gain(K, g) if kind in ("norm", "silu") else None
    ncol = N // 2 if kind == "silu" else N
    resid = _bf16(M, ncol, gen=g) if kind == "res" else None
    xin = R.rms_norm(x, nw, EPS) if nw is not None else x
    y = R.linear(xin, w)
    want = R.silu_mul(y) if kind == "silu" else y
    if resid is not None:
        want = (resid.float() + want.float()).to(BF16)
    t = qops.tile_weight(w.to(DEV), pair=kind == "silu")
    ntw, waves, gn, gk = cfg
    ws = qops.linear_workspace(qops.linear_workspace_bytes(M, N, ntw, gk) if gk > 1 else 256, DEV)
    outs = []
    for _ in range(2):
        r = None if resid is None else resid.to(DEV)
        psq = torch.empty((M, ncol // 16), dtype=torch.float32, device=DEV) if kind == "res" else None
        out = qops.fused_linear(x.to(DEV), t, cfg, norm_w=None if nw is None else nw.to(DEV), eps=EPS, residual=r,
                                out=r, psq_out=psq, silu_pair=kind == "silu", workspace=ws)
        outs.append(out.cpu())
        if psq is not None:   # the epilogue's statistics are those of the rounded output rows
            assert_close(psq.cpu(), qops.sumsq16(out).cpu(), 1e-5, 1e-6, "psq_out")
    assert_close(outs[0], want, 1e-2, 1 / 64, f"{kind} {N}x{K} M={M} cfg={cfg}")
    assert torch.equal(outs[0], outs[1])
    assert int(ws[:65536].count_nonzero()) == 0, "split-K arrival counters not re-armed"


@pytest.mark.parametrize("M", [3, 8, 17, 20, 32])
@pytest.mark.parametrize("kind,N,K", [("norm", 6144, 2560), ("res", 2560, 4096), ("silu", 19456, 2560),
                                      ("res", 2560, 9728)])
def test_rect_qwen_shapes(qops, M, kind, N, K):
    cfg = qops.rect_config(M, N, K, kind == "silu", norm=kind != "res")
    assert cfg is not None
    _run(qops, kind, M, N, K, cfg, 2000 + M + N + K)


@pytest.mark.parametrize("kind,M,N,K,cfg", [
    ("plain", 5, 32, 128, (1, 16, 1, 1)),     # 8 tiles over 16 wavefronts: empty pieces
    ("plain", 16, 48, 256, (1, 8, 2, 2)),     # uneven rectangles (units 1 / 2), 16 rows on 8 wavefronts
    ("norm", 9, 160, 1536, (1, 8, 4, 3)),     # k-ranges of 16 steps: pieces straddle units
    ("res", 31, 256, 1024, (1, 16, 16, 8)),
    ("silu", 12, 320, 512, (2, 8, 5, 4)),
    ("silu", 32, 640, 1280, (2, 16, 7, 5)),   # unit counts 2 / 3 per rectangle
    ("norm", 1, 512, 2560, (1, 8, 16, 4)),
    ("res", 2, 128, 4096, (1, 8, 8, 32)),
])
def test_rect_small_shapes(qops, kind, M, N, K, cfg):
    _run(qops, kind, M, N, K, cfg, 31 * M + N)


def test_rect_rejects_unfit_shapes(qops):
    g = torch.Generator().manual_seed(1)
    x = _bf16(4, 256, gen=g)
    t = qops.tile_weight(_bf16(512, 256, gen=g).to(DEV))
    assert not qops.rect_fits(4, 512, 256, 1, 8, 2, 1)        # 16 units per rectangle > 8 wavefronts
    with pytest.raises(RuntimeError, match="qwen_linear_rect failed"):
        qops.fused_linear(x.to(DEV), t, (1, 8, 2, 1))
    with pytest.raises(RuntimeError, match="qwen_linear_rect failed"):
        qops.fused_linear(x.to(DEV), t, (1, 8, 32, 4))        # k-ranges of 2 k-steps (not a multiple of 4)
    assert not qops.rect_fits(20, 512, 256, 1, 8, 32, 1)      # 20 rows > 2 staged rows x 8 wavefronts
