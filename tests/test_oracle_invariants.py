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

def test_rms_norm_mean_is_sum_times_reciprocal():
    """The mean is ``sum(x^2) * fp32(1/N)`` (``engine/kernels/rmsnorm.py:87-88``), not ``sum / N``:
    on rows whose sum of squares is exact in any order, the two forms round the case element to
    different bf16 values (``helpers.MEAN_FORM_CASES``), and both restatements give the product's."""
    from helpers import mean_form_rows
    x, cols, y_mul, y_div = mean_form_rows()
    w = torch.ones(x.shape[1], dtype=BF16)
    rows = torch.arange(len(cols))
    assert not torch.equal(y_mul, y_div)
    assert torch.equal(R.rms_norm(x, w, EPS)[rows, cols].float(), y_mul)
    assert np.array_equal(N.rms_norm(_np(x), _np(w), EPS)[rows.numpy(), cols.numpy()], y_mul.numpy())
    h, y = R.add_rms_norm(x, torch.zeros_like(x), w, EPS)
    assert torch.equal(h, x) and torch.equal(y[rows, cols].float(), y_mul)
    # the same rows under a division by N (torch's CPU mean) give the other value
    xf = x.float()
    div = (xf * torch.rsqrt(xf.pow(2).sum(-1, keepdim=True) / x.shape[1] + EPS)).to(BF16)
    assert torch.equal(div[rows, cols].float(), y_div)


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


# Known answers of the running-maximum rounding (flash) against the global-maximum rounding (twin):
# 64 keys of score 0 then one key of score a (scale 1); V = e0 for the 64 keys, e1 for the last.
# Output dim 0 is 64 p0 / (64 e + 1), e = exp(-a): p0 = e in fp32 for the flash form (the block's
# P = 1 exactly, rescaled by alpha = e), p0 = bf16(e) for the twin. Closed forms in float64, rounded
# to bf16 (each at least 1.9e-4 from a rounding boundary), found by a scan of bf16 a in [0.5, 4).
FLASH_KAT = [(0.5, 0.9765625, 0.97265625), (0.55859375, 0.97265625, 0.96875), (0.5859375, 0.97265625, 0.96875)]


@pytest.mark.parametrize("a,want_flash,want_twin", FLASH_KAT)
def test_flash_attention_rounds_p_against_the_running_maximum(a, want_flash, want_twin):
    D = 128
    q = torch.zeros(1, 1, 4, D, dtype=BF16)
    q[..., 0] = a
    kc = torch.zeros(1, 1, 80, D, dtype=BF16)
    kc[0, 0, 64, 0] = 1.0
    vc = torch.zeros(1, 1, 80, D, dtype=BF16)
    vc[0, 0, :64, 0] = 1.0
    vc[0, 0, 64, 1] = 1.0
    lens = torch.tensor([65], dtype=torch.int32)
    flash = R.attn_decode_flash(q, kc, vc, lens, 1.0).view(4, D)
    twin = R.attn_decode(q, kc, vc, lens, 1.0).view(4, D)
    assert flash[:, 0].tolist() == [want_flash] * 4 and twin[:, 0].tolist() == [want_twin] * 4
    # one split of two blocks gives the same closed form as two one-block splits (the reference's 32)
    two_blocks = R.attn_decode_flash(q, kc, vc, lens, 1.0, R.reference_schedule(1)).view(4, D)
    assert torch.equal(two_blocks, flash)


def test_flash_schedule_and_split_rule_known_answers():
    assert [R.choose_num_splits(B, 8) for B in (1, 4, 8, 32, 64)] == [32, 16, 8, 2, 1]
    lanes = R.reference_schedule(4)(650, 1)     # chunk = cdiv(650, 4) = 163 -> 192 (whole 64-key blocks)
    assert lanes == [[(0, 64), (64, 128), (128, 192)], [(192, 256), (256, 320), (320, 384)],
                     [(384, 448), (448, 512), (512, 576)], [(576, 640), (640, 650)]]
    assert R.reference_schedule(8)(100, 1)[2:] == [[]] * 6     # splits past the length are empty


@pytest.mark.parametrize("B,T,lengths,CAP", [(2, 1, [5, 200], 256), (2, 3, [70, 12], 128), (1, 5, [650], 700)])
def test_flash_attention_float64_and_twin(B, T, lengths, CAP):
    q, kc, vc, lens = _attn_case(B, T, lengths, CAP, 21)
    scale = 128 ** -0.5
    got = R.attn_decode_flash(q, kc, vc, lens, scale)
    want = N.attn_decode(_np(q), _np(kc), _np(vc), lens.numpy(), scale)
    assert np.abs(got.float().numpy() - want).max() <= 1e-2
    # the twin and the flash form differ only through P's rounding point: within the reference's
    # attention bar (atol 2e-2, tests/test_torch_ref.py:264), and equal up to fp32 summation
    # order when one block spans every key (running maximum = global maximum)
    twin = R.attn_decode(q, kc, vc, lens, scale)
    assert (got.float() - twin.float()).abs().max() <= 2e-2
    one = R.attn_decode_flash(q, kc, vc, lens, scale, lambda L, T: [[(0, L)]])
    d = (one.float() - twin.float()).abs()
    assert float(d.max()) <= 2 ** -7 * float(twin.float().abs().max()) and float((d > 0).float().mean()) <= 2e-3


def test_flash_attention_single_key_and_poison():
    q, kc, vc, _ = _attn_case(2, 1, [1, 1], 16, 12)
    lens = torch.tensor([1, 1], dtype=torch.int32)
    out = R.attn_decode_flash(q, kc, vc, lens, 128 ** -0.5)
    assert torch.equal(out, vc[:, :, 0, :][:, :, None, :].expand(2, 2, 4, 128).reshape(2, 1, 8 * 128))
    q, kc, vc, lens = _attn_case(2, 3, [7, 12], 16, 13)
    clean = R.attn_decode_flash(q, kc, vc, lens, 128 ** -0.5)
    kc[0, :, 7:], vc[0, :, 7:] = float("nan"), float("inf")
    kc[1, :, 12:], vc[1, :, 12:] = float("nan"), float("inf")
    assert torch.equal(R.attn_decode_flash(q, kc, vc, lens, 128 ** -0.5), clean)


def test_flash_prefill_attention():
    """The flash prompt attention (64-key blocks from key 0, one running maximum per query) within
    the attention bar of the twin's, equal to it up to fp32 order while one block holds every key,
    and equal, up to fp32 summation order, to the flash decode attention of each position on its
    own (a causal prefix)."""
    g = torch.Generator().manual_seed(31)
    B, S, NQ, NKV, D = 2, 150, 8, 2, 128
    q, k, v = _bf16(B, S, NQ, D, gen=g), _bf16(B, NKV, S, D, gen=g), _bf16(B, NKV, S, D, gen=g)
    scale = D ** -0.5
    flash = R.causal_prefill_attention_flash(q, k, v, scale)
    twin = R.causal_prefill_attention(q, k, v, scale)
    assert (flash.float() - twin.float()).abs().max() <= 2e-2
    one = R.causal_prefill_attention_flash(q[:, :60], k[:, :, :60], v[:, :, :60], scale)
    d = (one.float() - R.causal_prefill_attention(q[:, :60], k[:, :, :60], v[:, :, :60], scale).float()).abs()
    assert float((d > 0).float().mean()) <= 2e-3
    for p in (0, 63, 64, 149):
        dec = R.attn_decode_flash(q[:, p:p + 1], k, v, torch.full((B,), p + 1, dtype=torch.int32), scale,
                                  R.reference_schedule(1))
        u = _ulps(_np(flash.view(B, S, -1)[:, p]), _np(dec[:, 0]))
        assert u.max() <= 1 and (u > 0).mean() <= 1e-2, p


def test_engine_schedule_covers_every_key_once():
    from helpers import engine_schedule
    for splits, waves, T, L in [(1, 8, 1, 129), (4, 8, 1, 2305), (8, 8, 5, 4101), (1, 4, 1, 40), (3, 8, 2, 7)]:
        lanes = engine_schedule(splits, waves, T)(L, T)
        assert len(lanes) == splits * waves
        keys = sorted(k for lane in lanes for k0, k1 in lane for k in range(k0, k1))
        assert keys == list(range(L)), (splits, waves, T, L)
        last = lanes[-1]
        new = (L - T, L)
        first = (4 * T + 15) // 16 == 1 and waves != 4
        assert last.index(new) == (0 if first else len(last) - 1)
        assert all(k1 - k0 <= 32 for lane in lanes for k0, k1 in lane if (k0, k1) != new)


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
