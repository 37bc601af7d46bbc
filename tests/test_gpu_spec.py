"""GPU tests of exact speculative decoding (``engine/engine.py:955-1003``, ``:1309-1378``).

Kernels: the prompt-lookup draft against the oracle's ``spec_draft`` (bit-exact:
integer work) and the acceptance against ``spec_accept`` plus the history /
position bookkeeping of ``_spec_step``. Engine: periodic prompts (so drafts are
really accepted, as in the reference's ``tests/spec_check.py``) decoded with
speculation on, checked with the judge rule against the CPU oracle, the
generate protocol, and that verify steps were taken and accepted drafts.
"""

import itertools

import pytest
import torch

from __graft_entry__ import write_random_model
from helpers import assert_greedy_parity
from oracle import ref_torch as R
from oracle.model import CpuQwen3

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SMALL = {
    "hidden_size": 512, "intermediate_size": 1024, "vocab_size": 2048, "num_hidden_layers": 3,
    "num_attention_heads": 8, "num_key_value_heads": 2, "head_dim": 128, "rms_norm_eps": 1e-6,
    "rope_theta": 5000000.0, "rope_scaling": None, "tie_word_embeddings": True,
}
STD = 0.05


@pytest.fixture(scope="module")
def qops():
    from qwen_hip import ops
    return ops


def _hist_case(B, cap, seed, period=None):
    g = torch.Generator().manual_seed(seed)
    hist = torch.randint(0, 50, (B, cap), generator=g)
    if period:
        for b in range(B):
            pat = torch.randint(0, 50, (period[b],), generator=g)
            hist[b] = pat.repeat(cap // period[b] + 1)[:cap]
    return hist


@pytest.mark.parametrize("B,cap,k,n,lengths,period", [
    (1, 64, 4, 3, [40], [7]),          # periodic: the latest earlier occurrence wins
    (3, 128, 4, 3, [1, 2, 100], None),  # L < n: suffix indices clamp at 0
    (4, 256, 3, 2, [5, 60, 200, 256], [3, 5, 11, 4]),
    (2, 96, 1, 1, [10, 95], None),
    (2, 512, 15, 8, [300, 511], [9, 16]),
])
def test_spec_draft_matches_oracle(qops, B, cap, k, n, lengths, period):
    hist = _hist_case(B, cap, 11 * B + k, period)
    pos = torch.tensor(lengths, dtype=torch.int32) - 1
    got = qops.spec_draft(hist.to(DEV), pos.to(DEV), k, n).cpu()
    want = R.spec_draft(hist, pos.to(torch.int64) + 1, k, n)
    assert torch.equal(got, want)


def test_spec_draft_no_match_reads_from_the_start(qops):
    hist = torch.arange(100, 164, dtype=torch.int64)[None, :].clone()   # all distinct: no n-gram repeats
    pos = torch.tensor([20], dtype=torch.int32)
    got = qops.spec_draft(hist.to(DEV), pos.to(DEV), 4, 3).cpu()
    assert got.tolist() == [[120, 102, 103, 104, 105]]                 # i = -1 -> hist[n-1+j]


@pytest.mark.parametrize("done_rows", [[], [1]])
def test_spec_accept_bookkeeping(qops, done_rows):
    g = torch.Generator().manual_seed(5)
    B, T, cap, V, K = 3, 5, 64, 256, 128
    table = (torch.randn(V, K, generator=g) * 0.5).to(torch.bfloat16)
    w = qops.tile_weight(table.to(DEV))
    hist = torch.randint(0, V, (B, cap), generator=g)
    pos = torch.tensor([10, 20, 30], dtype=torch.int32)
    tok = torch.randint(0, V, (B, T), generator=g)
    nxt = torch.randint(0, V, (B, T), generator=g)
    nxt[0, :3] = tok[0, 1:4]          # row 0: three drafts accepted, then a miss
    nxt[1, :4] = tok[1, 1:5]          # row 1: all four accepted
    s_buf = torch.tensor([0], dtype=torch.int64)
    ntarget = torch.tensor([1 << 40], dtype=torch.int64)
    done = torch.zeros(B, dtype=torch.bool)
    if done_rows:                     # row 1 already produced its tokens: frozen
        ntarget = torch.tensor([21], dtype=torch.int64)
        done = (pos.to(torch.int64) + 1 - s_buf) >= ntarget
    want_adv = R.spec_accept(nxt, tok, done)
    hd, pd = hist.to(DEV), pos.to(DEV)
    out_t = torch.empty(T, B, dtype=torch.int64, device=DEV)
    adv = torch.empty(B, dtype=torch.int64, device=DEV)
    h = torch.empty(B, K, dtype=torch.bfloat16, device=DEV)
    psq = torch.empty(B, K // 16, dtype=torch.float32, device=DEV)
    qops.spec_accept(nxt.reshape(-1).to(DEV), tok.to(DEV), hd, pd, s_buf.to(DEV), ntarget.to(DEV), w, h, psq, out_t,
                     adv)
    assert torch.equal(adv.cpu(), want_adv)
    assert want_adv.tolist()[0] == 4 and (want_adv.tolist()[1] == (0 if done_rows else 5))
    assert torch.equal(out_t.cpu(), nxt.t())
    want_hist, want_pos = hist.clone(), pos.clone()
    for b in range(B):
        a = int(want_adv[b])
        for j in range(T):
            want_hist[b, int(pos[b]) + 1 + j if j < a else cap - 1] = nxt[b, j]
        want_pos[b] += a
    assert torch.equal(pd.cpu(), want_pos)
    assert torch.equal(hd.cpu()[:, :cap - 1], want_hist[:, :cap - 1])   # the dump slot holds any rejected token
    rows = [int(want_hist[b, int(want_pos[b])]) for b in range(B)]
    assert torch.equal(h.cpu(), table[rows])                            # next plain step's input row
    assert torch.allclose(psq.cpu(), table[rows].float().pow(2).view(B, K // 16, 16).sum(-1), atol=1e-5, rtol=1e-6)


def _periodic(period, S):
    return (period * (S // len(period) + 1))[:S]


@pytest.fixture(scope="module")
def spec_engine(tmp_path_factory):
    import engine as engine_mod
    from engine import Engine
    path = write_random_model(str(tmp_path_factory.mktemp("spec")), SMALL, seed=0, std=STD)
    saved = engine_mod.CONFIG["spec_k"]
    engine_mod.CONFIG["spec_k"] = 4
    try:
        yield Engine(path), CpuQwen3.random_init(SMALL, seed=0, std=STD)
    finally:
        engine_mod.CONFIG["spec_k"] = saved


@pytest.mark.parametrize("graphs", [True, False])
@pytest.mark.parametrize("case", ["periodic_b1", "mixed_b3"])
def test_generate_with_speculation_matches_oracle(spec_engine, monkeypatch, graphs, case):
    import engine as engine_mod
    eng, ref = spec_engine
    monkeypatch.setitem(engine_mod.CONFIG, "graphs", graphs)
    V, N = SMALL["vocab_size"], 24
    g = torch.Generator().manual_seed(3)
    if case == "periodic_b1":
        prompt = [_periodic([11, 220, 3, 500, 77, 9, 42], 64)]
        # keep speculating (the adaptive policy weighs measured step times): the acceptance
        # check below is about the model falling into the cycle, not about the timing
        monkeypatch.setitem(engine_mod.CONFIG, "spec_policy", "always")
    else:
        prompt = [_periodic([1, 2, 3, 4, 5], 48), _periodic([7, 1000, 7, 33], 48),
                  torch.randint(0, V, (48,), generator=g).tolist()]
    before_launch, before_tok = eng.counters["verify"], eng.counters["verify_gain"]
    steps = list(itertools.islice(eng.generate(prompt, N), N + 1))
    assert len(steps) == N and all(len(s) == len(prompt) and all(type(t) is int for t in s) for s in steps)
    assert eng.k_active == 4
    launches = eng.counters["verify"] - before_launch
    assert launches > 0, "no verify step was taken"
    tokens = [[steps[n][b] for n in range(N)] for b in range(len(prompt))]
    assert_greedy_parity(ref, prompt, tokens, f"speculation {case} graphs={graphs}")
    gained = eng.counters["verify_gain"] - before_tok
    print(f"{case} graphs={graphs}: {launches} verify steps, {gained} tokens ({gained / launches:.2f} per step)")
    if case == "periodic_b1":   # the model falls into the prompt's cycle: drafts get accepted
        assert gained > launches, "no draft was accepted"
