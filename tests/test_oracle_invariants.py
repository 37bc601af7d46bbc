"""Pins of the oracle that do not go through Transformers: closed forms, float64 brute force,
known-answer vectors, invariants the reference's tests state, and an independent numpy
restatement (``oracle/ref_numpy.py``) of every op."""

import math

import numpy as np
import pytest
import torch

from oracle import ref_numpy as N
from oracle import ref_torch as R
from oracle import weights as OW

BF16 = torch.bfloat16
EPS = 1e-6


def _bf16(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * scale).to(BF16)


def _np(t):
    return t.float().numpy()


def _ulps(a, b):
    """bf16 ulp distance between float32 arrays of bf16 values."""
    ai = a.astype(np.float32).view(np.int32) >> 16
    bi = b.astype(np.float32).view(np.int32) >> 16
    ai = np.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFF), bi)
    return np.abs(ai - bi)


# ------------------------------------------------------------- bf16 rounding

def test_bf16_round_to_nearest_even_known_answers():
    cases = {1.0 + 2 ** -8: 1.0,                 # exact tie -> even (down)
             1.0 + 3 * 2 ** -8: 1.0 + 2 ** -6,  # tie -> even (up)
             1.0 + 2 ** -8 + 2 ** -20: 1.0 + 2 ** -7,
             -(1.0 + 2 ** -8): -1.0,
             3.140625: 3.140625}
    for x, want in cases.items():
        assert float(N.rb(np.array([x], np.float32))[0]) == want
        assert float(torch.tensor(x, dtype=torch.float32).to(BF16).float()) == want
    bits = OW.bf16_rne_bits(np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32))
    assert bits.tolist() == [0x3F80, 0x3F82]


# ------------------------------------------------------------- weights generator

def test_splitmix64_known_answers():
    """First outputs of the published SplitMix64 generator seeded with 0."""
    gamma = 0x9E3779B97F4A7C15
    keys = np.array([0, gamma, (2 * gamma) & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
    got = [int(v) for v in OW.splitmix64(keys)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_generator_statistics_and_determinism():
    bits = OW.gen_bits(0, OW.tensor_id(0, "q_proj"), 0, 1 << 20)
    assert np.array_equal(bits, OW.gen_bits(0, OW.tensor_id(0, "q_proj"), 0, 1 << 20))
    v = OW.bits_to_f32(bits).astype(np.float64)
    assert abs(v.mean()) < 1e-4
    assert abs(v.std() - 0.02) < 2e-4
    assert np.abs(v).max() <= 0.02 * math.sqrt(12.0) * 1.01       # Irwin-Hall(4) bound: 2*sqrt(3) sigma
    # chunked generation equals one-shot generation
    a = OW.gen_tensor_bits(0, 5, (64, 96), chunk=1000)
    assert np.array_equal(a.reshape(-1), OW.gen_bits(0, 5, 0, 64 * 96))
    # different tensor ids / seeds give different streams
    assert not np.array_equal(OW.gen_bits(0, 1, 0, 64), OW.gen_bits(0, 2, 0, 64))
    assert not np.array_equal(OW.gen_bits(0, 1, 0, 64), OW.gen_bits(1, 1, 0, 64))


# ------------------------------------------------------------- norms / silu / rope

def test_rms_norm_closed_forms():
    w = (1.0 + torch.arange(256) / 256).to(BF16)
    assert torch.equal(R.rms_norm(torch.zeros(3, 256, dtype=BF16), w, EPS), torch.zeros(3, 256, dtype=BF16))
    # a constant row c normalises to ~1 (exactly 1/sqrt(1 + eps/c^2)), then * gain
    x = torch.full((1, 256), 2.0, dtype=BF16)
    assert torch.equal(R.rms_norm(x, w, EPS), w[None])


@pytest.mark.parametrize("rows,n", [(4, 2560), (9, 128)])
def test_numpy_cross_check_norms(rows, n):
    g = torch.Generator().manual_seed(3)
    x, r = _bf16(rows, n, gen=g, scale=3.0), _bf16(rows, n, gen=g, scale=3.0)
    w = (1.0 + 0.5 * torch.randn(n, generator=g)).to(BF16)
    assert _ulps(_np(R.rms_norm(x, w, EPS)), N.rms_norm(_np(x), _np(w), EPS)).max() <= 1
    h_t, y_t = R.add_rms_norm(x, r, w, EPS)
    h_n, y_n = N.add_rms_norm(_np(x), _np(r), _np(w), EPS)
    assert np.array_equal(_np(h_t), h_n)
    assert _ulps(_np(y_t), y_n).max() <= 1


def test_numpy_cross_check_silu():
    g = torch.Generator().manual_seed(4)
    gu = _bf16(7, 2 * 3072, gen=g, scale=4.0)
    d = _ulps(_np(R.silu_mul(gu)), N.silu_mul(_np(gu)))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_rope_position_zero_is_identity_and_numpy_cross_check():
    cos, sin = R.rope_tables(1024, 5e6, 128)
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
    g = torch.Generator().manual_seed(5)
    y = _bf16(3, 128, gen=g)
    assert torch.equal(R.rope_bf16(y, cos[0], sin[0]), y)
    pos = torch.tensor([1, 77, 1000])
    got = R.rope_bf16(y, cos[pos], sin[pos])
    assert np.array_equal(_np(got), N.rope(_np(y), _np(cos[pos]), _np(sin[pos])))   # 2-term sums: exact
    # theta: the highest frequency is 1 rad/position, the lowest theta^(-126/128)
    assert abs(float(cos[1, 0]) - math.cos(1.0)) < 4e-3
    inv_last = 5e6 ** (-126 / 128)
    assert abs(float(sin[1000, 63]) - math.sin(1000 * inv_last)) < 4e-3


# ------------------------------------------------------------- attention

def _attn_case(B, T, lengths, CAP, seed, NQ=8, NKV=2, D=128):
    g = torch.Generator().manual_seed(seed)
    return (_bf16(B, T, NQ, D, gen=g), _bf16(B, NKV, CAP, D, gen=g), _bf16(B, NKV, CAP, D, gen=g),
            torch.tensor(lengths, dtype=torch.int32))


@pytest.mark.parametrize("B,T,lengths", [(2, 1, [5, 9]), (2, 3, [7, 12]), (1, 5, [5])])
def test_attention_float64_brute_force(B, T, lengths):
    q, kc, vc, lens = _attn_case(B, T, lengths, 16, 11)
    got = R.attn_decode(q, kc, vc, lens, 128 ** -0.5).float().numpy()
    want = N.attn_decode(_np(q), _np(kc), _np(vc), lens.numpy(), 128 ** -0.5)
    assert np.abs(got - want).max() <= 1e-2


def test_attention_single_key_and_uniform_scores():
    q, kc, vc, _ = _attn_case(2, 1, [1, 1], 16, 12)
    out = R.attn_decode(q, kc, vc, torch.tensor([1, 1], dtype=torch.int32), 128 ** -0.5)
    want = vc[:, :, 0, :][:, :, None, :].expand(2, 2, 4, 128).reshape(2, 1, 8 * 128)
    assert torch.equal(out, want)
    # q = 0: every visible key has score 0 and p = 1, so the output is the mean of V rows.
    q0 = torch.zeros_like(q)
    out = R.attn_decode(q0, kc, vc, torch.tensor([6, 11], dtype=torch.int32), 128 ** -0.5).view(2, 8, 128)
    for b, L in enumerate([6, 11]):
        mean = vc[b, :, :L].double().mean(1)                 # [NKV, D]
        for h in range(8):
            assert torch.allclose(out[b, h].double(), mean[h // 4], atol=1e-2)


def test_attention_kv_head_mapping_and_causal_mask():
    kc = torch.zeros(1, 2, 8, 128, dtype=BF16)
    vc = torch.zeros(1, 2, 8, 128, dtype=BF16)
    vc[0, 0], vc[0, 1] = 1.0, 2.0
    out = R.attn_decode(torch.zeros(1, 1, 8, 128, dtype=BF16), kc, vc, torch.tensor([3], dtype=torch.int32), 0.1)
    assert torch.equal(out.view(8, 128)[:, 0], torch.tensor([1, 1, 1, 1, 2, 2, 2, 2], dtype=BF16))
    # T = 3: query t sees keys < len - (2 - t); with V[j] = j and q = 0 the output is the mean index.
    vc = torch.arange(8, dtype=torch.float32)[None, None, :, None].expand(1, 2, 8, 128).to(BF16).contiguous()
    out = R.attn_decode(torch.zeros(1, 3, 8, 128, dtype=BF16), kc, vc, torch.tensor([6], dtype=torch.int32), 0.1)
    assert out.view(3, 8, 128)[:, 0, 0].tolist() == [1.5, 2.0, 2.5]


def test_attention_poisoned_slots_ignored():
    q, kc, vc, lens = _attn_case(2, 3, [7, 12], 16, 13)
    clean = R.attn_decode(q, kc, vc, lens, 128 ** -0.5)
    kc[0, :, 7:], vc[0, :, 7:] = float("nan"), float("inf")
    kc[1, :, 12:], vc[1, :, 12:] = float("nan"), float("inf")
    assert torch.equal(R.attn_decode(q, kc, vc, lens, 128 ** -0.5), clean)


# ------------------------------------------------------------- GEMM / argmax

def test_linear_two_hot_exact_and_float64():
    g = torch.Generator().manual_seed(17)
    x = torch.randint(-8, 9, (3, 256), generator=g).to(BF16)
    w = torch.zeros(64, 256, dtype=BF16)
    cols = torch.randint(0, 256, (64, 2), generator=g)
    for n in range(64):
        w[n, cols[n, 0]] += 0.5
        w[n, cols[n, 1]] += 0.25
    assert torch.equal(R.linear(x, w), (x.double() @ w.double().T).to(BF16))
    x, w = _bf16(4, 2560, gen=g), _bf16(96, 2560, gen=g, scale=0.05)
    d = _ulps(_np(R.linear(x, w)), N.linear(_np(x), _np(w)))
    assert d.max() <= 1 and (d > 0).mean() < 0.05


def test_argmax_lowest_index_on_ties():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0]], dtype=BF16)
    assert R.argmax_lowest(logits).tolist() == [1, 0]


# ------------------------------------------------------------- speculative drafting

def test_spec_draft_prompt_lookup():
    hist = torch.tensor([[1, 2, 3, 4, 5, 1, 2, 3, 0, 0, 0, 0]])
    L = torch.tensor([8])                       # hist[:8] valid; suffix (1, 2, 3) occurred at 0
    out = R.spec_draft(hist, L, 3, 3)
    assert out.tolist() == [[3, 4, 5, 1]]
    # no earlier occurrence: drafts come from the start of the history (i = -1)
    hist = torch.tensor([[7, 8, 9, 10, 11, 0, 0, 0]])
    assert R.spec_draft(hist, torch.tensor([5]), 2, 3).tolist() == [[11, 9, 10]]


def test_spec_draft_latest_of_several_matches_wins():
    """``engine/engine.py:973``: the latest match start (``max`` over candidates) is taken. The
    suffix (1, 2) occurs at 0 and at 3 before the tail: the draft follows the one at 3 (7, 5), not
    the one at 0 (9, 1)."""
    hist = torch.tensor([[1, 2, 9, 1, 2, 7, 5, 1, 2, 0, 0]])
    assert R.spec_draft(hist, torch.tensor([9]), 2, 2).tolist() == [[2, 7, 5]]
    # a match that would overlap the suffix itself (start >= L - n) does not count: with the
    # suffix (4, 4) at 4..5, the starts 0..3 qualify and the latest, 3, drafts hist[5:8] clamped
    # to L - 1 = 5 -> (4, 4, 4); start 4 (the suffix itself) would draft past the history.
    hist = torch.tensor([[4, 4, 4, 4, 4, 4, 0, 0]])
    assert R.spec_draft(hist, torch.tensor([6]), 3, 2).tolist() == [[4, 4, 4, 4]]
    # three occurrences, three rows with different valid lengths: each row's latest qualifying one
    hist = torch.tensor([[5, 6, 1, 5, 6, 2, 5, 6, 3, 5, 6]] * 3)
    L = torch.tensor([11, 8, 5])
    assert R.spec_draft(hist, L, 1, 2).tolist() == [[6, 3], [6, 2], [6, 1]]


def test_spec_accept():
    nxt = torch.tensor([[4, 5, 6, 9], [1, 2, 3, 4]])
    tok = torch.tensor([[0, 4, 5, 7], [0, 9, 9, 9]])
    assert R.spec_accept(nxt, tok, torch.tensor([False, False])).tolist() == [3, 1]
    assert R.spec_accept(nxt, tok, torch.tensor([True, False])).tolist() == [0, 1]
