"""CPU tests of the certification twins (``qwen_hip.twins``) against the oracle.

The engine certifies its kernels at warmup against these twins (``engine/engine.py:407-486``
in the reference), so the twins must compute the oracle's formulas: each is run on CPU tensors
here and compared with ``oracle.ref_torch`` (itself pinned by the oracle tests), bit-exact
where both use the same operation order and within one bf16 ulp where only a summation order
or an ``exp`` implementation differs. The predicates (``close``, ``argmax_ok``) are checked on
constructed cases at their boundaries.
"""

import pytest
import torch

from oracle import ref_torch as R
from qwen_hip import twins as tw

BF16 = torch.bfloat16


def _bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(BF16)


def _ulps(a, b):
    """Distance in bf16 steps between same-sign bf16 tensors (monotone 16-bit patterns)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs()


def test_rms_norm_and_add_match_oracle():
    x, r, w = _bf((5, 256), 1), _bf((5, 256), 2), _bf((256,), 3)
    assert torch.equal(tw.rms_norm(x, w, 1e-6), R.rms_norm(x, w, 1e-6))
    h, y = R.add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(tw.add(x, r), h)
    assert torch.equal(tw.rms_norm(tw.add(x, r), w, 1e-6), y)


def test_linear_is_the_rounded_fp64_product():
    x, w = _bf((3, 512), 4), _bf((200, 512), 5, 0.05)
    want = (x.double() @ w.double().t()).to(BF16)
    got = tw.linear(x, w, rows=64)            # several row chunks
    assert (_ulps(got, want) <= 1).all()
    assert (got != want).float().mean() < 0.01


def test_silu_mul_matches_oracle():
    gu = _bf((4, 2 * 384), 6, 3.0)
    got, want = tw.silu_mul(gu), R.silu_mul(gu)
    d = (got.float() - want.float()).abs()
    assert float((d > 0).float().mean()) < 0.01
    assert bool((d <= want.float().abs() * 2.0 ** -7 + 1e-30).all())


@pytest.mark.parametrize("B,T", [(1, 1), (3, 2), (2, 5)])
def test_qk_norm_rope_matches_oracle(B, T):
    Nq, Nkv, D, CAP = 8, 2, 128, 64
    qkv = _bf((B * T, (Nq + 2 * Nkv) * D), 7 + B + T)
    qn, kn = _bf((D,), 8), _bf((D,), 9)
    cos, sin = R.rope_tables(128, 5e6, D)
    pos = torch.tensor([3, 17, 40][:B], dtype=torch.int32)
    kc = torch.zeros((B, Nkv, CAP, D), dtype=BF16)
    vc = torch.zeros_like(kc)
    q_o = R.qk_norm_rope_cache(qkv, qn, kn, 1e-6, cos, sin, pos, T, kc, vc)
    q_t, k_t, v_t = tw.qk_norm_rope(qkv, qn, kn, 1e-6, cos, sin, pos, T, Nkv)
    assert torch.equal(q_t, q_o)
    for b in range(B):
        for t in range(T):
            p = int(pos[b]) + t
            assert torch.equal(k_t[b, t], kc[b, :, p])
            assert torch.equal(v_t[b, t], vc[b, :, p])


@pytest.mark.parametrize("B,T,lens", [(1, 1, [9]), (2, 1, [1, 40]), (2, 4, [6, 33]), (3, 5, [5, 12, 64])])
def test_attention_matches_oracle(B, T, lens):
    Nq, Nkv, D, CAP = 8, 2, 128, 64
    q = _bf((B, T, Nq, D), 10 + B)
    kc, vc = _bf((B, Nkv, CAP, D), 11), _bf((B, Nkv, CAP, D), 12)
    lengths = torch.tensor(lens, dtype=torch.int32)
    got = tw.attention(q, kc, vc, lengths, D ** -0.5)
    want = R.attn_decode(q, kc, vc, lengths, D ** -0.5)
    assert got.shape == want.shape
    assert float((got.float() - want.float()).abs().max()) <= 2e-3


def test_attention_ignores_slots_past_the_length():
    B, T, Nq, Nkv, D, CAP = 2, 2, 4, 1, 128, 32
    q = _bf((B, T, Nq, D), 13)
    kc, vc = _bf((B, Nkv, CAP, D), 14), _bf((B, Nkv, CAP, D), 15)
    lengths = torch.tensor([7, 20], dtype=torch.int32)
    base = tw.attention(q, kc, vc, lengths, D ** -0.5)
    kc2, vc2 = kc.clone(), vc.clone()
    kc2[0, :, 7:] = float("nan")
    vc2[0, :, 7:] = float("inf")
    assert torch.equal(tw.attention(q, kc2, vc2, lengths, D ** -0.5), base)


def test_close_predicate():
    b = torch.tensor([1.0, -2.0, 0.0]).to(BF16)
    assert tw.close(b, b)
    assert tw.close((b.float() + torch.tensor([0.02, 0.0, 0.0])).to(BF16), b)        # 1e-2 + 1/64
    assert not tw.close((b.float() + torch.tensor([0.05, 0.0, 0.0])).to(BF16), b)
    assert not tw.close(b.float(), b)                                                 # dtype
    assert not tw.close(b[:2], b)                                                     # shape
    assert not tw.close(torch.tensor([float("nan"), -2.0, 0.0]).to(BF16), b)          # non-finite


def test_bf16_ulp():
    x = torch.tensor([1.0, 1.5, 3.0, 4.0, 0.3])
    assert torch.equal(tw.bf16_ulp(x), torch.tensor([2.0 ** -7, 2.0 ** -7, 2.0 ** -6, 2.0 ** -5, 2.0 ** -9]))


def test_argmax_ok():
    logits = torch.zeros((2, 10))
    logits[0, 3] = 4.0
    logits[1, 7] = 1.0
    logits = logits.to(BF16)
    assert tw.argmax_ok(torch.tensor([3, 7]), logits)
    assert not tw.argmax_ok(torch.tensor([2, 7]), logits)
    assert not tw.argmax_ok(torch.tensor([3, 10]), logits)                            # out of range
    assert not tw.argmax_ok(torch.tensor([3]), logits)                                # wrong count
    near = logits.float().clone()
    near[0, 5] = 4.0 - 2 * 2.0 ** -5                                                  # two ulps below 4.0
    near[1, 2] = 1.0 - 3 * 2.0 ** -7                                                  # three ulps below 1.0
    near = near.to(BF16)
    assert tw.argmax_ok(torch.tensor([5, 7]), near)
    assert not tw.argmax_ok(torch.tensor([3, 2]), near)
