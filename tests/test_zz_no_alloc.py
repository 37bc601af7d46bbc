"""The allocation-free decode attention (``qwen_attn_decode_mfma_noalloc``) against the workspace
entry point it mirrors (``qwen_attn_decode_mfma``), through the C ABI.

Both run the same kernels on the same inputs, so the bar is bit-exact: the attention output and
the K/V slots the call writes. Two calls in a row on the shared scratch (the second with a
smaller input, so stale partials and counters of the first would show); the first call of the
process recorded into a HIP graph and replayed; a shape that needs more than the fixed scratch is
refused with status 1004 before anything is launched.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda:0"


@pytest.fixture(scope="module")
def qops():
    from qwen_hip import ops
    return ops


def _case(B, T, CAP, Nkv, seed):
    g = torch.Generator().manual_seed(seed)
    D, Nq = 128, 4 * Nkv
    qkv = torch.randn(B * T, (Nq + 2 * Nkv) * D, generator=g).to(BF16)
    kc = torch.randn(B, Nkv, CAP, D, generator=g).to(BF16)
    vc = torch.randn(B, Nkv, CAP, D, generator=g).to(BF16)
    pos = torch.randint(CAP // 2, CAP - T, (B,), generator=g, dtype=torch.int32)
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    return qkv, kc, vc, pos, qn, kn


def _tables(P, D=128):
    from oracle import ref_torch as R
    return R.rope_tables(P, 5e6, D)


def test_noalloc_first_call_recorded_in_a_graph(qops):
    """The process's first call of the entry point on the device (its scratch-address lookup
    included) is recorded into a HIP graph (``torch.cuda.CUDAGraph``); every replay, with eager
    work and synchronisations between them, gives the workspace entry point's output and cache
    writes bit for bit. Defined first in this module so it is that first call."""
    cos, sin = _tables(4096)
    cos, sin = cos.to(DEV), sin.to(DEV)
    scale = 128 ** -0.5
    B, T, CAP, Nkv, S = 8, 1, 2304, 8, 4
    qkv, kc, vc, pos, qn, kn = _case(B, T, CAP, Nkv, 71)
    args = (qkv.to(DEV), qn.to(DEV), kn.to(DEV), 1e-6, cos, sin, pos.to(DEV), T)
    kc_g, vc_g = kc.to(DEV), vc.to(DEV)
    out = torch.empty(B, T, 4 * Nkv * 128, dtype=BF16, device=DEV)
    torch.cuda.synchronize()
    # recorded under inference mode, as the engine records its step graphs (the process's graph
    # generator state is created by the first recording, in whichever mode that ran)
    with torch.inference_mode():
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            qops.attn_decode_mfma_noalloc(*args, kc_g, vc_g, scale, S, out=out, waves=8)
        kc1, vc1 = kc.to(DEV), vc.to(DEV)
        ws = qops.attn_mfma_workspace(B, T, Nkv, S, DEV)
        want = qops.attn_decode_mfma(*args, kc1, vc1, scale, S, workspace=ws, waves=8)
        for r in range(3):
            out.zero_()
            kc_g.copy_(kc)
            vc_g.copy_(vc)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want), f"replay {r}: outputs differ"
            assert torch.equal(kc_g, kc1) and torch.equal(vc_g, vc1), f"replay {r}: cache writes differ"
            qops.attn_decode_mfma(*args, kc1, vc1, scale, S, workspace=ws, waves=8)   # eager work between replays
            torch.cuda.synchronize()
        del graph


@pytest.mark.parametrize("order", ["big_then_small"])
def test_noalloc_matches_workspace_entry_point(qops, order):
    cos, sin = _tables(8192)
    cos, sin = cos.to(DEV), sin.to(DEV)
    scale = 128 ** -0.5
    # (B, T, CAP, Nkv, splits): c3-like (4 splits, 2.1 MB of scratch), then a smaller verify shape
    for B, T, CAP, Nkv, S in [(8, 1, 2304, 8, 4), (2, 5, 1200, 8, 3)]:
        qkv, kc, vc, pos, qn, kn = _case(B, T, CAP, Nkv, B * 100 + T)
        need = qops._lib.query("qwen_attn_mfma_workspace_bytes", B, T, Nkv, S)
        assert 0 < need <= qops.ATTN_NOALLOC_SCRATCH_BYTES
        args = (qkv.to(DEV), qn.to(DEV), kn.to(DEV), 1e-6, cos, sin, pos.to(DEV), T)
        kc1, vc1, kc2, vc2 = kc.to(DEV), vc.to(DEV), kc.to(DEV), vc.to(DEV)
        ws = qops.attn_mfma_workspace(B, T, Nkv, S, DEV)
        want = qops.attn_decode_mfma(*args, kc1, vc1, scale, S, workspace=ws, waves=8)
        out = torch.empty_like(want)
        got = qops.attn_decode_mfma_noalloc(*args, kc2, vc2, scale, S, out=out, waves=8)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"B={B} T={T} S={S}: outputs differ"
        assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1), f"B={B} T={T}: cache writes differ"


def test_noalloc_refuses_oversized_request(qops):
    B, T, Nkv, S = 32, 8, 8, 8        # 256 (sequence, KV head) pairs x 8 splits x 32 rows: 34 MB > 8 MB
    need = qops._lib.query("qwen_attn_mfma_workspace_bytes", B, T, Nkv, S)
    assert need > qops.ATTN_NOALLOC_SCRATCH_BYTES
    qkv, kc, vc, pos, qn, kn = _case(B, T, 64, Nkv, 5)
    cos, sin = _tables(1024)
    out = torch.empty(B, T, 4 * Nkv * 128, dtype=BF16, device=DEV)
    with pytest.raises(RuntimeError, match="fixed scratch"):
        qops.attn_decode_mfma_noalloc(qkv.to(DEV), qn.to(DEV), kn.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV),
                                      pos.to(DEV), T, kc.to(DEV), vc.to(DEV), 128 ** -0.5, S, out=out, waves=8)
