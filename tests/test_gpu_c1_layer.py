"""BASELINE configs[0] (c1): one Qwen3-4B decoder layer, one decode step, compared per tensor.

Hidden 2560, 32 query / 8 KV heads of 128, MLP 9728, RMSNorm eps 1e-6 with per-head QK-norm,
RoPE theta 5e6, bf16 weights N(0, 0.02) from seed 0 (the oracle's generator, identical on the
device); batch 1, KV cache prefilled with 512 positions of N(0, 1) bf16, input hidden state
N(0, 1). The engine's layer (``Engine._layer``: the fused projections and the matrix-core
attention it runs in every decode step) is compared tensor by tensor with the oracle's
restatement of ``engine/engine.py:1103-1118`` (``oracle/ref_torch.py``) on the same inputs:
qkv and the attention output at the op bars (GEMM: atol 1e-2 / rtol 1/64,
``engine/engine.py:425-429``; attention: 2e-2, ``tests/test_torch_ref.py:264``), the residual
stream after O and down, and the SwiGLU product, by relative error (the hidden-state bar,
2e-2), plus the cache slot the step writes.

Each run prints every stage's relative error twice: accumulated (the oracle's chain from the
layer input) and local (the oracle's stage applied to the engine's own input of that stage), with
the attention also against the reference kernel's arithmetic in the engine's block order
(``R.attn_decode_flash``), which is where the layer's excess over the twin comes from.
"""

import functools

import pytest
import torch

from __graft_entry__ import write_random_model
from helpers import assert_close, engine_schedule
from oracle import ref_torch as R
from oracle.model import QWEN3_4B, CpuQwen3

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
CTX = 512


def _rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).norm() / b.norm())


@pytest.fixture(scope="module")
def c1(tmp_path_factory):
    from engine import Engine
    cfg = dict(QWEN3_4B, num_hidden_layers=1)
    path = write_random_model(str(tmp_path_factory.mktemp("c1")), cfg, seed=0, std=0.02)
    eng = Engine(path)
    ref = CpuQwen3.random_init(cfg, seed=0, std=0.02)
    return eng, ref, cfg


@pytest.mark.parametrize("seed", [0, 1])
def test_c1_single_layer_per_tensor(c1, seed):
    eng, ref, cfg = c1
    eng.prepare(1, CTX, 2)
    g = torch.Generator().manual_seed(100 + seed)
    kv_shape = (1, cfg["num_key_value_heads"], CTX, cfg["head_dim"])
    k_pre = torch.randn(kv_shape, generator=g).to(BF16)
    v_pre = torch.randn(kv_shape, generator=g).to(BF16)
    hidden = torch.randn(1, cfg["hidden_size"], generator=g).to(BF16)
    with torch.inference_mode():       # the engine's state tensors are inference tensors
        eng.state.kcache(0)[:, :, :CTX].copy_(k_pre.to(eng.device))
        eng.state.vcache(0)[:, :, :CTX].copy_(v_pre.to(eng.device))
    got_qkv, got_a, got_h1, got_p, got_h2 = [t.cpu() for t in eng.layer_step(0, hidden, [CTX])]

    # Oracle restatement of the layer (same weights, same cache contents).
    ref.prepare(1, eng.CAP)
    ref.k_cache[0][:, :, :CTX] = k_pre
    ref.v_cache[0][:, :, :CTX] = v_pre
    w = ref.w["layers"][0]
    pos = torch.tensor([CTX], dtype=torch.int32)
    qkv = R.linear(R.rms_norm(hidden, w["ln1"], ref.eps), w["w_qkv"])
    q = R.qk_norm_rope_cache(qkv, w["q_norm"], w["k_norm"], ref.eps, ref.cos_tab, ref.sin_tab, pos, 1,
                             ref.k_cache[0], ref.v_cache[0])
    a = R.attn_decode(q, ref.k_cache[0], ref.v_cache[0], pos + 1, ref.scale)
    h1, n2 = R.add_rms_norm(hidden, R.linear(a.view(1, -1), w["w_o"]), w["ln2"], ref.eps)
    p = R.silu_mul(R.linear(n2, w["w_gu"]))
    h2 = (h1.float() + R.linear(p, w["w_down"]).float()).to(BF16)

    # Per-stage errors: accumulated (oracle chain) and local (oracle stage on the engine's input).
    b = eng.bufs(eng.state.groups[0], 1)
    flash = functools.partial(R.attn_decode_flash, schedule=engine_schedule(b.splits, b.attn_waves, 1))
    kc_e, vc_e = torch.zeros_like(ref.k_cache[0]), torch.zeros_like(ref.v_cache[0])
    kc_e[:, :, :CTX], vc_e[:, :, :CTX] = k_pre, v_pre
    q_l = R.qk_norm_rope_cache(got_qkv, w["q_norm"], w["k_norm"], ref.eps, ref.cos_tab, ref.sin_tab, pos, 1, kc_e, vc_e)
    a_l = R.attn_decode(q_l, kc_e, vc_e, pos + 1, ref.scale)
    a_f = flash(q_l, kc_e, vc_e, pos + 1, ref.scale)
    h1_l, _ = R.add_rms_norm(hidden, R.linear(got_a.view(1, -1), w["w_o"]), w["ln2"], ref.eps)
    p_l = R.silu_mul(R.linear(R.rms_norm(got_h1, w["ln2"], ref.eps), w["w_gu"]))
    h2_l = (got_h1.float() + R.linear(got_p, w["w_down"]).float()).to(BF16)
    rows = [("qkv", _rel(got_qkv, qkv), _rel(got_qkv, qkv)),
            ("attention (twin)", _rel(got_a.view(1, -1), a.view(1, -1)), _rel(got_a.view(1, -1), a_l.view(1, -1))),
            ("attention (engine's block order)", None, _rel(got_a.view(1, -1), a_f.view(1, -1))),
            ("h after O + residual", _rel(got_h1, h1), _rel(got_h1, h1_l)),
            ("SwiGLU product", _rel(got_p, p), _rel(got_p, p_l)),
            ("layer output", _rel(got_h2, h2), _rel(got_h2, h2_l))]
    print(f"\nc1 seed {seed}: relative error per stage (accumulated / local)")
    for name, acc, loc in rows:
        print(f"  {name:34s} {'-' if acc is None else f'{acc:.2e}':>9s} {loc:.2e}")
    assert _rel(got_a.view(1, -1), a_f.view(1, -1)) <= 5e-3, "attention vs the engine's block order"

    assert_close(got_qkv, qkv, 1e-2, 1 / 64, "qkv")
    assert_close(got_a.view(1, -1), a.view(1, -1), 2e-2, 2e-2, "attention output")
    assert _rel(got_h1, h1) <= 2e-2, f"h after O: {_rel(got_h1, h1)}"
    assert _rel(got_p, p) <= 2e-2, f"SwiGLU product: {_rel(got_p, p)}"
    assert _rel(got_h2, h2) <= 2e-2, f"layer output: {_rel(got_h2, h2)}"
    # The step's cache writes: slot CTX holds the normed, rotated key and the raw value.
    kc, vc = eng.state.kcache(0)[0, :, CTX].cpu(), eng.state.vcache(0)[0, :, CTX].cpu()
    assert_close(kc, ref.k_cache[0][0, :, CTX], 1e-2, 1 / 64, "k slot")
    assert torch.equal(vc, ref.v_cache[0][0, :, CTX])
    assert torch.equal(eng.state.kcache(0)[:, :, :CTX].cpu(), k_pre)   # prefilled slots untouched
