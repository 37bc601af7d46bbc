"""The single-launch QKV projection + decode attention (``qwen_qkv_attn_decode``) against the two
launches it replaces, through the C ABI: ``qwen_gemv_rowmap`` (RMSNorm prologue, store epilogue,
8 row groups, the same 256 - na workgroups) then ``qwen_attn_decode_mfma`` (T = 1, 8 wavefronts).
Both run the same kernel bodies on the same inputs, so the bar is bit-exact: the qkv rows, the
attention output and the K/V slots written. Covered: B = 1 and 2, one and several context splits
(the split merge inside the same launch), three launches in a row on one workspace (every
generation flag ends at 3, the split counters re-armed), replays of a HIP graph with eager work
between them, and shapes the entry point refuses before launching. Parity with the oracle comes through the engine's tests, where every
M <= 2 plain decode step takes this form.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda:0"
H, NQ, NKV, D = 2560, 32, 8, 128
N = (NQ + 2 * NKV) * D
EPS = 1e-6


@pytest.fixture(scope="module")
def qops():
    from qwen_hip import ops
    return ops


def _head_major(Nq=NQ, Nkv=NKV, D=D):
    """Head-major row order: block h holds KV head group h's q rows, k row, v row."""
    qd, grp = Nq // Nkv * D, Nq // Nkv * D + 2 * D
    p = torch.arange((Nq + 2 * Nkv) * D)
    h, i = p // grp, p % grp
    return torch.where(i < qd, h * qd + i, torch.where(i < qd + D, Nq * D + h * D + (i - qd),
                                                       (Nq + Nkv) * D + h * D + (i - qd - D)))


def _case(B, CAP, seed):
    from oracle import ref_torch as R
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, H, generator=g) * 2).to(BF16)
    w = (torch.randn(N, H, generator=g) * 0.03).to(BF16)
    ln1 = (1 + 0.2 * torch.randn(H, generator=g)).to(BF16)
    qn = (1 + 0.2 * torch.randn(D, generator=g)).to(BF16)
    kn = (1 + 0.2 * torch.randn(D, generator=g)).to(BF16)
    kc = torch.randn(B, NKV, CAP, D, generator=g).to(BF16)
    vc = torch.randn(B, NKV, CAP, D, generator=g).to(BF16)
    pos = torch.randint(CAP // 2, CAP - 1, (B,), generator=g, dtype=torch.int32)
    cos, sin = R.rope_tables(max(1024, 1 << (CAP - 1).bit_length()), 5e6, D)
    perm = _head_major()
    dev = lambda t: t.to(DEV)
    return dict(x=dev(x), w_rows=dev(w[perm].contiguous()), ln1=dev(ln1), row_map=dev(perm.to(torch.int32)),
                qn=dev(qn), kn=dev(kn), kc=dev(kc), vc=dev(vc), pos=dev(pos), cos=dev(cos), sin=dev(sin))


def _separate(qops, c, S, kc, vc):
    B = c["x"].shape[0]
    na = B * NKV * S
    qkv = qops.gemv(c["x"], c["w_rows"], norm_w=c["ln1"], eps=EPS, cfg=(256 - na, 8), row_map=c["row_map"],
                    groups=8)
    ws = qops.attn_mfma_workspace(B, 1, NKV, S, DEV)
    a = qops.attn_decode_mfma(qkv, c["qn"], c["kn"], EPS, c["cos"], c["sin"], c["pos"], 1, kc, vc, D ** -0.5, S,
                              workspace=ws, waves=8)
    return qkv, a


def _fused(qops, c, S, kc, vc, ws, qkv=None, out=None):
    B = c["x"].shape[0]
    qkv = torch.empty(B, N, dtype=BF16, device=DEV) if qkv is None else qkv
    out = torch.empty(B, 1, NQ * D, dtype=BF16, device=DEV) if out is None else out
    qops.qkv_attn_decode(c["x"], c["w_rows"], c["ln1"], c["row_map"], EPS, qkv, c["qn"], c["kn"], c["cos"], c["sin"],
                         c["pos"], kc, vc, D ** -0.5, S, out=out, workspace=ws)
    return qkv, out


@pytest.mark.parametrize("B,CAP,S", [(1, 512, 1), (1, 4096, 8), (2, 512, 1), (2, 2048, 4), (1, 2048, 2)])
def test_single_launch_matches_two_launches(qops, B, CAP, S):
    c = _case(B, CAP, B * 1000 + CAP + S)
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    qkv_ref, a_ref = _separate(qops, c, S, kc1, vc1)
    ws = qops.qkv_attn_workspace(B, NKV, S, DEV)
    for launch in range(3):                     # generation flags advance, split counters re-arm
        kc2, vc2 = c["kc"].clone(), c["vc"].clone()
        qkv, a = _fused(qops, c, S, kc2, vc2, ws)
        torch.cuda.synchronize()
        assert not qops.qkv_attn_failed(ws), f"launch {launch}: a hand-off wait expired"
        assert torch.equal(qkv, qkv_ref), f"launch {launch}: qkv rows differ"
        assert torch.equal(a, a_ref), f"launch {launch}: attention output differs"
        assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1), f"launch {launch}: cache writes differ"
    flags = ws[-4096:-4096 + 1280].view(torch.int32)
    na = B * NKV * S
    assert torch.equal(flags[:256 - na], torch.full((256 - na,), 3, dtype=torch.int32, device=DEV))
    assert torch.equal(flags[256:256 + na], torch.full((na,), 3, dtype=torch.int32, device=DEV))


def test_single_launch_graph_replays(qops):
    """Recorded into a HIP graph (under inference mode, as the engine records its steps) and
    replayed three times with eager work in between: every replay bit-exact."""
    B, CAP, S = 1, 1024, 2
    c = _case(B, CAP, 77)
    kc1, vc1 = c["kc"].clone(), c["vc"].clone()
    qkv_ref, a_ref = _separate(qops, c, S, kc1, vc1)
    ws = qops.qkv_attn_workspace(B, NKV, S, DEV)
    kc2, vc2 = c["kc"].clone(), c["vc"].clone()
    qkv = torch.empty(B, N, dtype=BF16, device=DEV)
    out = torch.empty(B, 1, NQ * D, dtype=BF16, device=DEV)
    torch.cuda.synchronize()
    with torch.inference_mode():
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _fused(qops, c, S, kc2, vc2, ws, qkv=qkv, out=out)
        for r in range(3):
            qkv.zero_()
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(qkv, qkv_ref) and torch.equal(out, a_ref), f"replay {r} differs"
            assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1), f"replay {r}: cache writes differ"
            _separate(qops, c, S, kc1, vc1)      # eager work between replays
            torch.cuda.synchronize()
        del graph
    assert not qops.qkv_attn_failed(ws)


def test_single_launch_refuses_unsupported_shapes(qops):
    assert not qops.qkv_attn_supported(3, NKV, 1)          # B > 2
    assert not qops.qkv_attn_supported(1, 2, 1)            # not one KV head group per XCD
    assert not qops.qkv_attn_supported(2, NKV, 8)          # 128 attention workgroups > 64
    assert qops.qkv_attn_supported(2, NKV, 4) and qops.qkv_attn_supported(1, NKV, 8)
    c = _case(1, 512, 5)
    ws = qops.qkv_attn_workspace(1, NKV, 1, DEV)
    with pytest.raises(RuntimeError, match="workspace too small"):
        _fused(qops, c, 1, c["kc"], c["vc"], ws[:64])
