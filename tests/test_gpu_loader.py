"""GPU tests of the checkpoint loader (``engine/engine.py:184-230``): a Qwen3 directory written with
safetensors (``config.json`` + ``model.safetensors`` under Transformers parameter names) is loaded
by ``Engine(path)`` and decoded, then checked against the CPU oracle on the same weights.

The weights use non-unit RMSNorm gains (input / post-attention / q / k / final norms), so the
loader's placement of every gain is exercised end to end, and both config forms of the RoPE base
(``rope_theta``, and Transformers 5's ``rope_parameters``). The q|k|v and gate|up concatenation
is checked by greedy parity and per-layer hidden states; the untied case gives the LM head its
own matrix.
"""

import json
import os

import pytest
import torch

from helpers import assert_greedy_parity
from oracle.model import CpuQwen3

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
CFG = {
    "hidden_size": 512, "intermediate_size": 1024, "vocab_size": 2048, "num_hidden_layers": 2,
    "num_attention_heads": 8, "num_key_value_heads": 2, "head_dim": 128, "rms_norm_eps": 1e-6,
    "rope_theta": 5000000.0, "rope_scaling": None, "tie_word_embeddings": True,
    "architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3", "torch_dtype": "bfloat16",
}


def _oracle(tied: bool, seed: int = 0) -> CpuQwen3:
    """Random-init oracle weights with non-unit norm gains (and an own LM head when untied)."""
    ref = CpuQwen3.random_init(CFG, seed=seed, std=0.05)
    g = torch.Generator().manual_seed(99)

    def gain(n):
        return (1.0 + 0.2 * torch.randn(n, generator=g)).to(BF16)

    for lw in ref.w["layers"]:
        lw["ln1"], lw["ln2"] = gain(CFG["hidden_size"]), gain(CFG["hidden_size"])
        lw["q_norm"], lw["k_norm"] = gain(CFG["head_dim"]), gain(CFG["head_dim"])
    ref.w["final_norm"] = gain(CFG["hidden_size"])
    if not tied:
        ref.w["lm_head"] = (0.05 * torch.randn(CFG["vocab_size"], CFG["hidden_size"], generator=g)).to(BF16)
        ref.lm_head = ref.w["lm_head"]
    return ref


def _write_checkpoint(path, ref: CpuQwen3, tied: bool, rope_form: str, shards: int = 1):
    from safetensors.torch import save_file
    sd = ref.hf_state_dict()
    if tied:
        sd.pop("lm_head.weight")           # tied: Transformers ties the head to the embedding
    else:
        sd["lm_head.weight"] = ref.w["lm_head"]
    sd = {k: v.contiguous().clone() for k, v in sd.items()}
    keys = sorted(sd)
    for i in range(shards):
        part = {k: sd[k] for k in keys[i::shards]}
        save_file(part, os.path.join(path, f"model-{i + 1:05d}-of-{shards:05d}.safetensors"))
    cfg = dict(CFG, tie_word_embeddings=tied)
    if rope_form == "rope_parameters":
        theta = cfg.pop("rope_theta")
        cfg.pop("rope_scaling")
        cfg["rope_parameters"] = {"rope_type": "default", "rope_theta": theta}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    return str(path)


def _prompt(B, S, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, CFG["vocab_size"], (B, S), generator=g).tolist()


@pytest.mark.parametrize("tied,rope_form,shards", [(True, "rope_theta", 1), (True, "rope_parameters", 2),
                                                    (False, "rope_theta", 3)])
def test_checkpoint_loads_and_decodes(tmp_path, tied, rope_form, shards):
    from engine import Engine
    ref = _oracle(tied)
    eng = Engine(_write_checkpoint(tmp_path, ref, tied, rope_form, shards))
    assert eng.spec.theta == CFG["rope_theta"] and eng.spec.tied == tied
    for B, S, N in [(1, 20, 8), (3, 45, 6)]:
        prompt = _prompt(B, S, B * 31 + S)
        steps = list(eng.generate(prompt, N))
        tokens = [[steps[n][b] for n in range(N)] for b in range(B)]
        assert_greedy_parity(ref, prompt, tokens, f"checkpoint tied={tied} {rope_form} B={B}", engine=eng)
    # per-layer hidden states of one decode step
    prompt = _prompt(2, 16, 7)
    list(eng.generate(prompt, 1))
    tok = torch.tensor(prompt)[:, -1:]
    hidden = eng.step_hidden(tok, [15, 15])
    ref.prepare(2, eng.CAP)
    ref.prefill(torch.tensor(prompt)[:, :15])
    want = []
    ref.step(tok, torch.full((2,), 15, dtype=torch.int32), 1, hidden=want)
    for l, (a, b) in enumerate(zip(hidden, want)):
        rel = float((a.float().cpu() - b.float()).norm() / b.float().norm())
        assert rel <= 2e-2, f"layer {l}: {rel}"


def test_checkpoint_errors(tmp_path):
    from engine import Engine
    ref = _oracle(True)
    path = _write_checkpoint(tmp_path, ref, True, "rope_theta")
    with open(os.path.join(path, "config.json")) as f:
        cfg = json.load(f)
    cfg["rope_scaling"] = {"rope_type": "yarn", "factor": 4.0}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    with pytest.raises(RuntimeError, match="rope scaling"):
        Engine(path)
    cfg["rope_scaling"] = None
    cfg["tie_word_embeddings"] = False         # untied but the checkpoint has no lm_head.weight
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    with pytest.raises(RuntimeError, match="lm_head.weight"):
        Engine(path)
