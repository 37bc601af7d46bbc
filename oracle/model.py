"""Whole-model CPU restatement of the reference engine's decode path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

``CpuQwen3`` follows ``engine/engine.py`` step for step with the ``ref_torch``
ops: weight fusion (``:209-227``), RoPE tables (``:232-251``), static state
(``:830-863``), ``_step`` (``:1093-1121``), ``_plain_step`` (``:941-953``),
``_spec_step`` (``:979-1003``), ``_prefill_slice`` (``:1191-1221``) and the
``generate`` protocol (``:1225-1250``): exactly ``N`` yields of ``B`` Python
ints, the first from prefill, then ``N - 1`` decode steps.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import ref_torch as R
from .weights import bits_to_f32, gen_tensor_bits, model_shapes, tensor_id

BF16 = torch.bfloat16

QWEN3_4B = {
    "hidden_size": 2560, "intermediate_size": 9728, "vocab_size": 151936,
    "num_hidden_layers": 36, "num_attention_heads": 32, "num_key_value_heads": 8,
    "head_dim": 128, "rms_norm_eps": 1e-6, "rope_theta": 5000000.0, "rope_scaling": None,
    "tie_word_embeddings": True,
}


def _t(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits_to_f32(bits)).to(BF16)


class CpuQwen3:
    """Qwen3 decoder on CPU (bf16 storage, fp32 accumulation), static KV cache."""

    def __init__(self, cfg: dict, weights: dict):
        self.cfg = dict(cfg)
        self.H, self.I, self.V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
        self.L = len(weights["layers"])
        self.Nq, self.Nkv, self.D = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
        self.eps = float(cfg["rms_norm_eps"])
        self.theta = float(cfg.get("rope_theta") or cfg["rope_parameters"]["rope_theta"])
        self.scale = self.D ** -0.5
        self.w = weights
        self.B = self.CAP = 0
        self.cos_tab = self.sin_tab = None
        # the LM head: tied to the embedding unless the weights hold their own (engine/engine.py:225-226)
        self.lm_head = weights.get("lm_head", weights["embed"])
        # decode-step attention ``f(q, k_cache, v_cache, lengths, scale)`` and prompt attention
        # ``f(q, k, v, scale)``: the twin's global-maximum form by default; ``R.attn_decode_flash`` /
        # ``R.causal_prefill_attention_flash`` restate the running maximum of flash attention
        self.attention = R.attn_decode
        self.prefill_attention = R.causal_prefill_attention

    # ------------------------------------------------------------- weights
    @classmethod
    def random_init(cls, cfg: dict, seed: int = 0, std: float = 0.02, layers: int | None = None):
        L = cfg["num_hidden_layers"] if layers is None else layers
        shapes = model_shapes(cfg)
        ones_h = torch.ones(cfg["hidden_size"], dtype=BF16)
        ones_d = torch.ones(cfg["head_dim"], dtype=BF16)
        lw = []
        for l in range(L):
            t = {n: _t(gen_tensor_bits(seed, tensor_id(l, n), s, std)) for n, s in shapes.items()}
            lw.append({
                "ln1": ones_h.clone(), "ln2": ones_h.clone(), "q_norm": ones_d.clone(), "k_norm": ones_d.clone(),
                "w_qkv": torch.cat([t["q_proj"], t["k_proj"], t["v_proj"]], 0).contiguous(),
                "w_o": t["o_proj"], "w_gu": torch.cat([t["gate_proj"], t["up_proj"]], 0).contiguous(),
                "w_down": t["down_proj"],
            })
        embed = _t(gen_tensor_bits(seed, tensor_id(None, "embed"), (cfg["vocab_size"], cfg["hidden_size"]), std))
        return cls(cfg, {"embed": embed, "final_norm": ones_h.clone(), "layers": lw})

    def hf_state_dict(self) -> dict:
        """The same weights under Transformers ``Qwen3ForCausalLM`` parameter names."""
        sd = {"model.embed_tokens.weight": self.w["embed"], "model.norm.weight": self.w["final_norm"],
              "lm_head.weight": self.w["embed"]}
        qn, kn = self.Nq * self.D, self.Nkv * self.D
        for l, w in enumerate(self.w["layers"]):
            p = f"model.layers.{l}."
            sd[p + "input_layernorm.weight"] = w["ln1"]
            sd[p + "post_attention_layernorm.weight"] = w["ln2"]
            sd[p + "self_attn.q_proj.weight"] = w["w_qkv"][:qn]
            sd[p + "self_attn.k_proj.weight"] = w["w_qkv"][qn:qn + kn]
            sd[p + "self_attn.v_proj.weight"] = w["w_qkv"][qn + kn:]
            sd[p + "self_attn.q_norm.weight"] = w["q_norm"]
            sd[p + "self_attn.k_norm.weight"] = w["k_norm"]
            sd[p + "self_attn.o_proj.weight"] = w["w_o"]
            sd[p + "mlp.gate_proj.weight"] = w["w_gu"][: self.I]
            sd[p + "mlp.up_proj.weight"] = w["w_gu"][self.I:]
            sd[p + "mlp.down_proj.weight"] = w["w_down"]
        return sd

    # --------------------------------------------------------------- state
    def prepare(self, B: int, cap: int):
        """Static state as ``engine/engine.py:830-863`` (zeroed caches, history, positions)."""
        P = int(2 ** math.ceil(math.log2(max(cap, 1024))))
        if self.cos_tab is None or self.cos_tab.shape[0] < P:
            self.cos_tab, self.sin_tab = R.rope_tables(P, self.theta, self.D)
        shape = (B, self.Nkv, cap, self.D)
        self.k_cache = [torch.zeros(shape, dtype=BF16) for _ in range(self.L)]
        self.v_cache = [torch.zeros(shape, dtype=BF16) for _ in range(self.L)]
        self.hist = torch.zeros((B, cap), dtype=torch.int64)
        self.pos = torch.zeros((B,), dtype=torch.int32)
        self.B, self.CAP = B, cap

    # ---------------------------------------------------------------- step
    def layer(self, l: int, h, d, pos, T, B, hidden=None):
        """One decoder layer of ``_step`` (``engine/engine.py:1103-1118``); returns ``(h, d)``."""
        w = self.w["layers"][l]
        M = h.shape[0]
        if d is None:
            n = R.rms_norm(h, w["ln1"], self.eps)
        else:
            h, n = R.add_rms_norm(h, d, w["ln1"], self.eps)
        qkv = R.linear(n, w["w_qkv"])
        q = R.qk_norm_rope_cache(qkv, w["q_norm"], w["k_norm"], self.eps, self.cos_tab, self.sin_tab,
                                 pos, T, self.k_cache[l][:B], self.v_cache[l][:B])
        a = self.attention(q, self.k_cache[l][:B], self.v_cache[l][:B], pos + T, self.scale)
        o = R.linear(a.view(M, -1), w["w_o"])
        h, n = R.add_rms_norm(h, o, w["ln2"], self.eps)
        p = R.silu_mul(R.linear(n, w["w_gu"]))
        d = R.linear(p, w["w_down"])
        if hidden is not None:
            hidden.append(R.add_rms_norm(h, d, w["ln1"], self.eps)[0])
        return h, d

    def step(self, tok: torch.Tensor, pos: torch.Tensor, T: int, hidden=None, return_logits=False):
        """``_step``: ``tok [B, T]`` int64, ``pos [B]`` int32 -> greedy ``next [B*T]``."""
        B = tok.shape[0]
        h = self.w["embed"][tok.reshape(-1)]
        d = None
        for l in range(self.L):
            h, d = self.layer(l, h, d, pos, T, B, hidden)
        _, n = R.add_rms_norm(h, d, self.w["final_norm"], self.eps)
        logits = R.linear(n, self.lm_head)
        nxt = R.argmax_lowest(logits)
        return (nxt, logits) if return_logits else nxt

    def plain_step(self):
        """``_plain_step`` (``engine/engine.py:941-953``) without the frozen-row branch."""
        L = self.pos.to(torch.int64) + 1
        tok = self.hist.gather(1, (L - 1)[:, None])
        nxt = self.step(tok, self.pos, 1)
        self.hist.scatter_(1, L[:, None], nxt[:, None])
        self.pos += 1
        return nxt

    def spec_step(self, k: int, n: int = 3):
        """``_spec_step`` (``engine/engine.py:979-1003``): verify ``k`` drafts in one T=k+1 step."""
        B = self.hist.shape[0]
        L = self.pos.to(torch.int64) + 1
        tok = R.spec_draft(self.hist, L, k, n)
        nxt = self.step(tok, self.pos, k + 1).view(B, k + 1)
        adv = R.spec_accept(nxt, tok, torch.zeros(B, dtype=torch.bool))
        for b in range(B):
            for j in range(int(adv[b])):
                self.hist[b, int(L[b]) + j] = nxt[b, j]
        self.pos += adv.to(torch.int32)
        return nxt, adv

    def prefill(self, ids: torch.Tensor, hidden=None, return_logits=False, positions=None):
        """``_prefill_slice`` for the whole batch (``engine/engine.py:1191-1221``).

        Returns the greedy token after the last prompt position (and its bf16 logits with
        ``return_logits``). ``positions`` (a list of prompt positions) instead returns the bf16
        logits ``[B, len(positions), V]`` predicting the token after each of them.
        """
        B, S = ids.shape
        pos = torch.zeros((B,), dtype=torch.int32)
        h = self.w["embed"][ids.reshape(-1)]
        d = None
        for l in range(self.L):
            w = self.w["layers"][l]
            if d is None:
                n = R.rms_norm(h, w["ln1"], self.eps)
            else:
                h, n = R.add_rms_norm(h, d, w["ln1"], self.eps)
            qkv = R.linear(n, w["w_qkv"])
            kc, vc = self.k_cache[l][:B], self.v_cache[l][:B]
            q = R.qk_norm_rope_cache(qkv, w["q_norm"], w["k_norm"], self.eps, self.cos_tab, self.sin_tab,
                                     pos, S, kc, vc)
            a = self.prefill_attention(q, kc[:, :, :S], vc[:, :, :S], self.scale)
            o = R.linear(a, w["w_o"])
            h, n = R.add_rms_norm(h, o, w["ln2"], self.eps)
            d = R.linear(R.silu_mul(R.linear(n, w["w_gu"])), w["w_down"])
            if hidden is not None:
                hidden.append(R.add_rms_norm(h, d, w["ln1"], self.eps)[0])
        if positions is not None:
            rows = (torch.arange(B)[:, None] * S + torch.as_tensor(positions)[None, :]).reshape(-1)
            _, n = R.add_rms_norm(h[rows], d[rows], self.w["final_norm"], self.eps)
            return R.linear(n, self.lm_head).view(B, len(positions), -1)
        last = torch.arange(B) * S + (S - 1)
        _, n = R.add_rms_norm(h[last], d[last], self.w["final_norm"], self.eps)
        logits = R.linear(n, self.lm_head)
        nxt = R.argmax_lowest(logits)
        return (nxt, logits) if return_logits else nxt

    def replay_logits(self, prompt, tokens):
        """bf16 logits ``[B, N, V]`` predicting each emitted token from its own prefix, from ONE
        teacher-forced forward over prompt + emitted tokens, as the reference's judge does
        (``tests/local_check.py:254-272``: logits at positions ``S - 1 .. S + N - 2``)."""
        B, S, N = len(prompt), len(prompt[0]), len(tokens[0])
        ids = torch.tensor([list(prompt[b]) + list(tokens[b][:-1]) for b in range(B)], dtype=torch.int64)
        self.prepare(B, ((S + N + 63) // 64) * 64)
        return self.prefill(ids, positions=list(range(S - 1, S + N - 1)))

    def teacher_forced_logits(self, prompt, tokens):
        """bf16 logits ``[B, N, V]`` predicting each emitted token from its own prefix.

        The reference harness replays the candidate's tokens through the
        Transformers model and checks them (``tests/local_check.py:233-271``);
        this runs the same replay as a prompt forward plus ``N - 1`` decode steps.
        """
        B, S, N = len(prompt), len(prompt[0]), len(tokens[0])
        ids = torch.tensor([list(prompt[b]) + list(tokens[b][:-1]) for b in range(B)], dtype=torch.int64)
        self.prepare(B, ((S + N + 63) // 64) * 64)
        _, lg = self.prefill(ids[:, :S], return_logits=True)
        out = [lg]
        self.pos.fill_(S)
        for n in range(1, N):
            _, lg = self.step(ids[:, S + n - 1:S + n], self.pos, 1, return_logits=True)
            self.pos += 1
            out.append(lg)
        return torch.stack(out, dim=1)

    def judge_gaps(self, prompt, tokens):
        """``max_logit - logit[emitted]`` per (b, n), teacher-forced (0 = the oracle's argmax value)."""
        lg = self.teacher_forced_logits(prompt, tokens).float()
        tok = torch.tensor(tokens, dtype=torch.int64)
        return lg.amax(-1) - lg.gather(-1, tok[..., None])[..., 0]

    # ------------------------------------------------------------ generate
    def generate(self, input_ids, max_new_tokens: int, slack: int = 16):
        """The reference protocol (``engine/engine.py:1225-1250``): N yields of B ints."""
        B, S = len(input_ids), len(input_ids[0])
        N = int(max_new_tokens)
        if N <= 0:
            return
        cap = ((S + N + slack + 63) // 64) * 64
        self.prepare(B, cap)
        ids = torch.tensor(input_ids, dtype=torch.int64)
        first = self.prefill(ids)
        self.hist[:, :S] = ids
        self.hist[:, S] = first
        self.pos.fill_(S)
        yield [int(t) for t in first.tolist()]
        for _ in range(N - 1):
            yield [int(t) for t in self.plain_step().tolist()]
