"""Pin the oracle (``oracle/ref_torch.py``) against the Transformers Qwen3 modules on CPU.

The reference's own twin tests compare its pure-torch twins with
``Qwen3RMSNorm``, ``Qwen3RotaryEmbedding`` / ``apply_rotary_pos_emb`` and SDPA
(``tests/test_torch_ref.py:71-339``); the same comparisons, with the same
seeds, shapes and tolerances, pin this build's oracle. Transformers is the
third-party library the reference defers to (pinned 4.51.3 in
``requirements.txt:11``; 5.15.0 is installed here, with the same formulas in
``modeling_qwen3.py:59-64`` (RMSNorm), ``:86-170`` (rotary), ``:211-280``
(attention)).
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import ref_torch as R

transformers = pytest.importorskip("transformers")
from transformers.models.qwen3.configuration_qwen3 import Qwen3Config  # noqa: E402
from transformers.models.qwen3.modeling_qwen3 import (  # noqa: E402
    Qwen3RMSNorm,
    Qwen3RotaryEmbedding,
    apply_rotary_pos_emb,
    repeat_kv,
)

BF16 = torch.bfloat16
EPS = 1e-6
D = 128
NQ = 8
NKV = 2
THETA = 5e6


def _bf16(*shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen, dtype=torch.float32) * scale).to(BF16)


def _norm_module(n, gen):
    mod = Qwen3RMSNorm(n, eps=EPS).to(BF16)
    with torch.no_grad():
        mod.weight.copy_((1.0 + 0.5 * torch.randn(n, generator=gen)).to(BF16))
    return mod


def _config():
    return Qwen3Config(vocab_size=1024, hidden_size=NQ * D, intermediate_size=512, num_hidden_layers=1,
                       num_attention_heads=NQ, num_key_value_heads=NKV, head_dim=D, rms_norm_eps=EPS,
                       rope_theta=THETA, max_position_embeddings=4096, tie_word_embeddings=True)


@pytest.mark.parametrize("rows,n", [(1, 128), (6, 2560), (37, 1024), (3, 96)])
def test_rms_norm_bit_exact(rows, n):
    gen = torch.Generator().manual_seed(1234)
    mod = _norm_module(n, gen)
    x = _bf16(rows, n, gen=gen, scale=3.0)
    with torch.no_grad():
        want = mod(x)
    got = R.rms_norm(x, mod.weight.data, EPS)
    assert got.dtype == BF16 and got.shape == x.shape
    assert torch.equal(got, want)


def test_rms_norm_mean_form_differs_from_cpu_module():
    """On the CPU, ``Qwen3RMSNorm``'s ``mean`` divides the sum by N; the reference's kernels and
    torch's GPU ``mean`` multiply it by fp32(1/N) (``engine/kernels/rmsnorm.py:87-88``), which the
    oracle follows. On the discriminating rows of ``helpers.MEAN_FORM_CASES`` the CPU module gives
    the division's value and the oracle the product's; elsewhere they agree bit for bit."""
    from helpers import mean_form_rows
    x, cols, y_mul, y_div = mean_form_rows()
    mod = Qwen3RMSNorm(x.shape[1], eps=EPS).to(BF16)
    rows = torch.arange(len(cols))
    with torch.no_grad():
        want = mod(x)
    got = R.rms_norm(x, mod.weight.data, EPS)
    assert torch.equal(want[rows, cols].float(), y_div) and torch.equal(got[rows, cols].float(), y_mul)


def test_rms_norm_flat_rows_match_3d():
    gen = torch.Generator().manual_seed(1234)
    mod = _norm_module(2560, gen)
    x3 = _bf16(2, 5, 2560, gen=gen, scale=3.0)
    with torch.no_grad():
        want = mod(x3).reshape(10, 2560)
    assert torch.equal(R.rms_norm(x3.reshape(10, 2560), mod.weight.data, EPS), want)


@pytest.mark.parametrize("rows,n", [(1, 128), (6, 2560), (37, 1024)])
def test_add_rms_norm_bit_exact(rows, n):
    gen = torch.Generator().manual_seed(1234)
    mod = _norm_module(n, gen)
    x = _bf16(rows, n, gen=gen, scale=3.0)
    r = _bf16(rows, n, gen=gen, scale=3.0)
    with torch.no_grad():
        h_want = x + r
        y_want = mod(h_want)
    h, y = R.add_rms_norm(x, r, mod.weight.data, EPS)
    assert torch.equal(h, h_want) and torch.equal(y, y_want)


@pytest.mark.parametrize("rows,inter", [(1, 64), (7, 3072), (13, 9728), (5, 300)])
def test_silu_mul_bit_exact(rows, inter):
    gen = torch.Generator().manual_seed(42)
    g = _bf16(rows, inter, gen=gen, scale=4.0)
    u = _bf16(rows, inter, gen=gen, scale=4.0)
    want = F.silu(g) * u   # Qwen3MLP: act_fn(gate_proj(x)) * up_proj(x) on bf16 tensors
    got = R.silu_mul(torch.cat([g, u], dim=-1))
    assert got.shape == (rows, inter) and torch.equal(got, want)


class TestRope:
    P = 256

    def setup_method(self):
        self.gen = torch.Generator().manual_seed(7)
        self.rope = Qwen3RotaryEmbedding(_config())
        self.q_norm = _norm_module(D, self.gen)
        self.k_norm = _norm_module(D, self.gen)
        with torch.no_grad():
            c, s = self.rope(torch.zeros(1, dtype=BF16), torch.arange(self.P)[None, :])
        self.cos_tab, self.sin_tab = c[0].contiguous(), s[0].contiguous()

    def test_table_matches_oracle_table(self):
        cos, sin = R.rope_tables(self.P, THETA, D)
        assert torch.equal(cos, self.cos_tab) and torch.equal(sin, self.sin_tab)
        # cos[:, :64] == cos[:, 64:] (the table repeats the 64 frequencies)
        assert torch.equal(cos[:, :64], cos[:, 64:])

    def test_table_is_gatherable(self):
        position_ids = torch.tensor([[5, 6, 7], [20, 21, 22]])
        with torch.no_grad():
            c, s = self.rope(torch.zeros(1, dtype=BF16), position_ids)
        assert torch.equal(c, self.cos_tab[position_ids]) and torch.equal(s, self.sin_tab[position_ids])

    def _run(self, T, positions, B=2, CAP=64):
        width = (NQ + 2 * NKV) * D
        qkv = _bf16(B * T, width, gen=self.gen, scale=2.0)
        k_cache = _bf16(B, NKV, CAP, D, gen=self.gen)
        v_cache = _bf16(B, NKV, CAP, D, gen=self.gen)
        k_before, v_before, qkv_before = k_cache.clone(), v_cache.clone(), qkv.clone()
        pos_t = torch.tensor(positions, dtype=torch.int32)
        position_ids = pos_t.to(torch.int64)[:, None] + torch.arange(T)[None, :]
        with torch.no_grad():
            cos, sin = self.rope(torch.zeros(1, dtype=BF16), position_ids)
            q_hf = self.q_norm(qkv[:, :NQ * D].contiguous().view(B, T, NQ, D)).transpose(1, 2)
            k_hf = self.k_norm(qkv[:, NQ * D:(NQ + NKV) * D].contiguous().view(B, T, NKV, D)).transpose(1, 2)
            v_hf = qkv[:, (NQ + NKV) * D:].contiguous().view(B, T, NKV, D).transpose(1, 2)
            q_hf, k_hf = apply_rotary_pos_emb(q_hf, k_hf, cos, sin)
        q = R.qk_norm_rope_cache(qkv, self.q_norm.weight.data, self.k_norm.weight.data, EPS, self.cos_tab,
                                 self.sin_tab, pos_t, T, k_cache, v_cache)
        assert q.shape == (B, T, NQ, D) and q.is_contiguous()
        assert torch.equal(qkv, qkv_before)
        assert torch.equal(q, q_hf.transpose(1, 2))
        touched = torch.zeros(B, CAP, dtype=torch.bool)
        for b in range(B):
            for t in range(T):
                p = positions[b] + t
                touched[b, p] = True
                assert torch.equal(k_cache[b, :, p], k_hf[b, :, t])
                assert torch.equal(v_cache[b, :, p], v_hf[b, :, t])
        keep = ~touched[:, None, :, None].expand_as(k_cache)
        assert torch.equal(k_cache[keep], k_before[keep]) and torch.equal(v_cache[keep], v_before[keep])

    def test_t1(self):
        self._run(1, [5, 40])

    def test_t3(self):
        self._run(3, [0, 17])

    def test_prefill_like_from_zero(self):
        self._run(9, [0, 0])


class TestAttention:
    def setup_method(self):
        self.gen = torch.Generator().manual_seed(99)
        self.scale = D ** -0.5

    def _sdpa(self, q, k_cache, v_cache, lengths, T):
        """SDPA over each sequence's valid slice with the causal rule (tests/test_torch_ref.py:234-256)."""
        B, G = q.shape[0], NQ // NKV
        outs = []
        for b in range(B):
            L = int(lengths[b])
            kb = repeat_kv(k_cache[b:b + 1, :, :L], G).float()
            vb = repeat_kv(v_cache[b:b + 1, :, :L], G).float()
            qb = q[b:b + 1].transpose(1, 2).float()
            mask = None if T == 1 else (torch.arange(L)[None, :] < (L - (T - 1 - torch.arange(T)[:, None])))
            o = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask, scale=self.scale)
            outs.append(o.transpose(1, 2).reshape(1, T, NQ * D))
        return torch.cat(outs, 0)

    @pytest.mark.parametrize("T,lengths,poison", [(1, [13, 40], False), (1, [64, 64], False),
                                                  (3, [13, 40], False), (3, [64, 30], False),
                                                  (3, [13, 40], True), (1, [1, 64], True)])
    def test_vs_sdpa(self, T, lengths, poison):
        B, CAP = 2, 64
        q = _bf16(B, T, NQ, D, gen=self.gen)
        k_cache = _bf16(B, NKV, CAP, D, gen=self.gen)
        v_cache = _bf16(B, NKV, CAP, D, gen=self.gen)
        want = self._sdpa(q, k_cache, v_cache, lengths, T)
        if poison:
            for b in range(B):
                k_cache[b, :, lengths[b]:] = float("nan")
                v_cache[b, :, lengths[b]:] = float("inf")
        got = R.attn_decode(q, k_cache, v_cache, torch.tensor(lengths, dtype=torch.int32), self.scale)
        assert got.shape == (B, T, NQ * D) and got.is_contiguous()
        assert torch.isfinite(got.float()).all()
        assert torch.allclose(got.float(), want.float(), atol=2e-2, rtol=0)

    def test_mask_is_load_bearing(self):
        B, T, CAP, G = 2, 3, 64, NQ // NKV
        lengths = [13, 40]
        q = _bf16(B, T, NQ, D, gen=self.gen)
        k_cache = _bf16(B, NKV, CAP, D, gen=self.gen)
        v_cache = _bf16(B, NKV, CAP, D, gen=self.gen)
        got = R.attn_decode(q, k_cache, v_cache, torch.tensor(lengths, dtype=torch.int32), self.scale)
        wrong = []
        for b in range(B):
            L = lengths[b]
            o = F.scaled_dot_product_attention(q[b:b + 1].transpose(1, 2).float(),
                                               repeat_kv(k_cache[b:b + 1, :, :L], G).float(),
                                               repeat_kv(v_cache[b:b + 1, :, :L], G).float(), scale=self.scale)
            wrong.append(o.transpose(1, 2).reshape(1, T, NQ * D))
        wrong = torch.cat(wrong)
        assert torch.allclose(got[:, -1].float(), wrong[:, -1].float(), atol=2e-2, rtol=0)
        assert not torch.allclose(got[:, 0].float(), wrong[:, 0].float(), atol=2e-2, rtol=0)
