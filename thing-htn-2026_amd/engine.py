"""Qwen3-4B greedy-decode engine for one MI355X (gfx950): drop-in for the reference's ``engine/engine.py``.

Public surface as in the reference (``engine/engine.py:109-111``, ``:1225-1250``):
``Engine(model_path)`` loads the model once; ``generate(input_ids, max_new_tokens)`` is a
generator yielding exactly ``max_new_tokens`` lists of ``B`` Python ints, the first from the
prompt forward, then one per decode step. State resets on every call; batch size and prompt
length may change between calls.

Device work is hand-written HIP kernels only (``qwen_hip``, ``libqwen_hip.so``):

* decode step (one HIP graph per step width ``T``, replayed per token), per row group of at
  most 32 sequences::

      36 x [ norm+QKV projection | QK-norm + RoPE + KV write + split attention + merge |
             O projection + residual | norm + gate/up projection + SwiGLU |
             down projection + residual ]
      final norm + LM head + argmax | token / history / position update + next embedding

* prompt forward: the prompt in position chunks of all sequences; per layer RMSNorm, the
  MFMA GEMM over the tiled weights (QKV, O + residual, gate/up + SwiGLU, down + residual),
  QK-norm + RoPE + KV write, and causal flash attention over the cache.

Torch provides device memory, the RoPE tables, graph recording and host <-> device copies.
There is no CPU path: without a GPU or without ``libqwen_hip.so`` the constructor raises.
The host runtime (batch state, graphs, speculation policy, token pump) is in
``decode_runtime.py``.
"""

from __future__ import annotations

import json
import math
import os
import sys
import time
from dataclasses import dataclass

import torch

import decode_runtime as rt
from qwen_hip import ops
from qwen_hip import twins as tw
from qwen_hip.ops import TiledWeight

BF16 = torch.bfloat16

CONFIG = {
    "graphs": True,          # replay one HIP graph per decode step
    "inflight": 4,           # decode steps queued on the device ahead of the consumer
    "prefill_tokens": 65536, # rows (sequences x positions) per prompt-forward chunk
    "cap_round": 256,        # KV capacity granularity (a later call with a smaller need reuses the state)
    "group_rows": 32,        # sequences per decode row group (the kernels take at most 32 rows)
    # Exact speculative decoding (engine/engine.py:79-82): prompt-lookup drafts of spec_k tokens
    # verified in one T = spec_k + 1 step; 0 = off (the reference's default).
    "spec_k": int(os.environ.get("QWEN_ENGINE_SPEC_K", "0")),
    "spec_n": 3,             # n-gram length of the draft lookup
    "spec_max_batch": 8,     # speculate only when B <= this (and B * (spec_k + 1) <= 32)
    "spec_policy": "adaptive",   # or "always"
    "spec_backoff": (16, 256),   # plain steps before re-probing a losing speculation (doubles)
    "spec_probe_len": 4,         # verify steps per probe
    # Run each decode-step shape's kernels against the torch twins once before the first decode
    # of that shape and refuse to decode on a mismatch (engine/engine.py:407-486 falls back instead).
    "certify": os.environ.get("QWEN_ENGINE_CERTIFY", "1") != "0",
    # M <= 2: order the QKV GEMV's weight rows so that each KV head's q / k / v rows are
    # produced on the XCD that runs that head's attention workgroup.
    "xcd_heads": os.environ.get("QWEN_ENGINE_XCD_HEADS", "1") != "0",
    # Whole-KV-cache size up to which the decode attention reads K/V with cache-allocating loads.
    "kv_cached_max_bytes": int(os.environ.get("QWEN_ENGINE_KV_CACHED_MAX", str(128 << 20))),
    "log": True,
}

XCDS = 8   # MI355X: 8 XCDs; workgroup i of a launch runs on XCD i mod 8

# Generator tensor ids of the counter-based random init (one per HF weight).
_PROJ_IDS = {"q_proj": 0, "k_proj": 1, "v_proj": 2, "o_proj": 3, "gate_proj": 4, "up_proj": 5, "down_proj": 6}


def _log(*parts):
    if CONFIG["log"]:
        print("[engine]", *parts, file=sys.stderr, flush=True)


def _tid(layer, name):
    return 0 if name == "embed" else 1 + 16 * layer + _PROJ_IDS[name]


def random_init_scale(std: float) -> float:
    """fp32 multiplier of the centred Irwin-Hall(4) sum of 16-bit fields (sigma^2 = (2^32 - 1) / 3)."""
    import numpy as np
    return float(np.float32(std / math.sqrt((65536.0 * 65536.0 - 1.0) / 3.0)))


@dataclass(frozen=True)
class ModelSpec:
    """Model dimensions from an HF ``config.json`` (``engine/engine.py:128-141``)."""

    H: int
    I: int
    V: int
    L: int
    Nq: int
    Nkv: int
    D: int
    eps: float
    theta: float
    tied: bool

    @classmethod
    def from_config(cls, cfg: dict) -> "ModelSpec":
        rope = cfg.get("rope_parameters") or {}
        theta = cfg.get("rope_theta", rope.get("rope_theta"))
        if theta is None:
            raise RuntimeError("config.json has neither rope_theta nor rope_parameters.rope_theta")
        if cfg.get("rope_scaling") is not None or rope.get("rope_type", "default") != "default":
            raise RuntimeError("rope scaling is not supported by this engine")
        H, Nq = cfg["hidden_size"], cfg["num_attention_heads"]
        spec = cls(H=H, I=cfg["intermediate_size"], V=cfg["vocab_size"], L=cfg["num_hidden_layers"], Nq=Nq,
                   Nkv=cfg["num_key_value_heads"], D=cfg.get("head_dim") or H // Nq,
                   eps=float(cfg["rms_norm_eps"]), theta=float(theta),
                   tied=bool(cfg.get("tie_word_embeddings", False)))
        if spec.D != 128 or spec.Nq != 4 * spec.Nkv:
            raise RuntimeError(f"kernels need head_dim 128 and 4 query heads per KV head (got {spec.D}, "
                               f"{spec.Nq}/{spec.Nkv})")
        if spec.H % 512 or spec.I % 512 or spec.V % 16 or (spec.Nq * spec.D) % 512:
            raise RuntimeError("hidden / intermediate / attention widths must be multiples of 512, vocab of 16")
        return spec

    @property
    def qkv_width(self) -> int:
        return (self.Nq + 2 * self.Nkv) * self.D


class LayerWeights:
    """One decoder layer on the device: RMSNorm gains, the four projections in MFMA-B tiles
    (decode at M > 2 and the prompt forward), and row-major copies for the M <= 2 GEMV."""

    __slots__ = ("ln1", "ln2", "q_norm", "k_norm", "qkv", "o", "gu", "down",
                 "qkv_rows", "o_rows", "gu_rows", "down_rows")


class Weights:
    """Device weights: layers, the embedding table (tiled; the gather reads it), the LM head
    (tiled for M > 2, row-major for the GEMV) and the final norm. With tied embeddings the LM
    head's tiled copy is the embedding table itself (``engine/engine.py:225-226``)."""

    def __init__(self):
        self.layers: list[LayerWeights] = []
        self.embed: TiledWeight | None = None
        self.lm: TiledWeight | None = None
        self.lm_rows: torch.Tensor | None = None
        self.final_norm: torch.Tensor | None = None
        self.qkv_perm: torch.Tensor | None = None   # int64 [N]: row p of qkv_rows is natural row perm[p]
        self.qkv_map: torch.Tensor | None = None    # the same permutation, int32 on the device

    def natural_qkv_rows(self, w: LayerWeights) -> torch.Tensor:
        """The row-major q|k|v weight in the HF order (undoing the XCD row order)."""
        if self.qkv_perm is None:
            return w.qkv_rows
        out = torch.empty_like(w.qkv_rows)
        out.index_copy_(0, self.qkv_perm.to(out.device), w.qkv_rows)
        return out


class StepBuffers:
    """Activation buffers, launch shapes and workspaces of one decode step over one row group
    (``rows`` sequences x ``T`` tokens); reused by every replay of that step."""

    def __init__(self, spec: ModelSpec, rows: int, T: int, cap: int, device):
        M = rows * T
        self.rows, self.T, self.M = rows, T, M
        self.h = torch.zeros((M, spec.H), dtype=BF16, device=device)
        self.psq = torch.zeros((M, spec.H // 16), dtype=torch.float32, device=device)
        self.qkv = torch.empty((M, spec.qkv_width), dtype=BF16, device=device)
        self.a = torch.empty((rows, T, spec.Nq * spec.D), dtype=BF16, device=device)
        self.p = torch.empty((M, spec.I), dtype=BF16, device=device)
        self.nxt = torch.empty((M,), dtype=torch.int64, device=device)
        self.tok = torch.zeros((rows, T), dtype=torch.int64, device=device)      # verify-step input ids
        self.out_t = torch.zeros((T, rows), dtype=torch.int64, device=device)    # verify-step tokens [T, rows]
        self.adv = torch.zeros((rows,), dtype=torch.int64, device=device)        # tokens accepted per row
        self.keys = ops.argmax_keys(M, device)
        self.mfma_attn = T <= ops.MFMA_MAX_T
        self.splits = (ops.choose_mfma_splits(rows, spec.Nkv, cap) if self.mfma_attn
                       else ops.choose_num_splits(rows, spec.Nkv, cap, T))
        self.attn_waves = ops.MFMA_WAVES if self.mfma_attn else ops.attn_waves(rows, T)
        self.attn_ws = (ops.attn_mfma_workspace(rows, T, spec.Nkv, self.splits, device) if self.mfma_attn
                        else ops.attn_workspace(rows, T, spec.Nq, spec.Nkv, spec.D, self.splits, device))
        self.cfg = {
            "qkv": ops.gemm_config(M, spec.qkv_width, spec.H),
            "o": ops.gemm_config(M, spec.H, spec.Nq * spec.D),
            "gu": ops.gemm_config(M, 2 * spec.I, spec.H, True),
            "down": ops.gemm_config(M, spec.H, spec.I),
        }
        widths = {"qkv": spec.qkv_width, "o": spec.H, "gu": 2 * spec.I, "down": spec.H}
        ws = max(ops.gemm_workspace_bytes(M, widths[k], c) for k, c in self.cfg.items())
        self.gemm_ws = ops.linear_workspace(ws, device)
        self.gemv = M <= ops.GEMV_MAX_M
        self.gemv_cfg = {
            "qkv": ops.gemv_config(M, spec.qkv_width, spec.H, ops.GEPI_STORE, device),
            "o": ops.gemv_config(M, spec.H, spec.Nq * spec.D, ops.GEPI_RES, device),
            "gu": ops.gemv_config(M, spec.I, spec.H, ops.GEPI_SWIGLU, device),
            "down": ops.gemv_config(M, spec.H, spec.I, ops.GEPI_RES, device),
            "lm": ops.gemv_config(M, spec.V, spec.H, ops.GEPI_ARGMAX, device),
        } if self.gemv else None
        self.lm_cfg = ops.lm_head_config(M, spec.V, spec.H)


class Engine:
    def __init__(self, model_path: str) -> None:
        """Load the model in ``model_path``: an HF checkpoint directory (``config.json`` +
        ``*.safetensors``) or ``config.json`` + ``random_init.json`` (seeded random weights)."""
        t0 = time.time()
        if not torch.cuda.is_available():
            raise RuntimeError("Engine needs an MI355X GPU (HIP device); there is no CPU path")
        self.device = torch.device("cuda:0")
        with open(os.path.join(model_path, "config.json")) as handle:
            self.cfg = json.load(handle)
        self.spec = ModelSpec.from_config(self.cfg)
        s = self.spec
        self.eps, self.scale = s.eps, s.D ** -0.5
        # The reference's operator table (engine/engine.py:257-263), all HIP kernels.
        self.ops = {"rms_norm": ops.rms_norm, "add_rms_norm": ops.add_rms_norm, "silu_mul": ops.silu_mul,
                    "qk_norm_rope_cache": ops.qk_norm_rope_cache, "attn_decode": ops.attn_decode}
        self.w = Weights()
        if os.path.exists(os.path.join(model_path, "random_init.json")):
            with open(os.path.join(model_path, "random_init.json")) as handle:
                rnd = json.load(handle)
            self._init_random(int(rnd.get("seed", 0)), float(rnd.get("std", 0.02)),
                              norm_std=float(rnd.get("norm_std", 0.0)))
        else:
            self._load_checkpoint(model_path)
        self.state: rt.BatchState | None = None
        self.counters = {"decode": 0, "verify": 0, "verify_gain": 0}
        self.cos_tab = self.sin_tab = None
        self._rope_rows = 0
        self._rope_for(8192)
        torch.cuda.synchronize()
        _log(f"loaded in {rt.log_time(t0)}: L={s.L} H={s.H} V={s.V} tied={s.tied}")

    # ================================================================== weights
    def _qkv_xcd_order(self):
        """Row order of the M <= 2 QKV GEMV's weight in which the workgroups of one XCD produce
        exactly one KV head group (its query heads, key and value rows), or None when the
        shapes do not allow it.

        Workgroup g of a launch runs on XCD g mod 8, the GEMV's workgroup g owns weight rows
        [N g / G, N (g + 1) / G), and the decode attention's workgroup for (sequence b, KV
        head h) is number b * Nkv + h. With Nkv = 8 and each head group exactly G / 8
        workgroups of rows, the order below (outputs still stored at their natural columns)
        leaves head h's q / k / v rows in the L2 of the XCD that runs its attention.
        Returns ``perm [N]``: reordered row p is natural row perm[p]."""
        s = self.spec
        N = s.qkv_width
        G, _ = ops.gemv_config(1, N, s.H, ops.GEPI_STORE, self.device)
        qd = (s.Nq // s.Nkv) * s.D
        grp = qd + 2 * s.D
        if s.Nkv != XCDS or N % G or G % XCDS or grp != (G // XCDS) * (N // G):
            return None
        rows = N // G
        p = torch.arange(N, dtype=torch.int64)
        g, j = p // rows, p % rows
        h, i = g % XCDS, (g // XCDS) * rows + j
        k0, v0 = s.Nq * s.D, (s.Nq + s.Nkv) * s.D
        return torch.where(i < qd, h * qd + i,
                           torch.where(i < qd + s.D, k0 + h * s.D + (i - qd), v0 + h * s.D + (i - qd - s.D)))

    def _finish_layer(self, w: LayerWeights, qkv_rows: torch.Tensor):
        """Store the QKV GEMV copy in the XCD row order (when enabled)."""
        if self.w.qkv_perm is not None:
            w.qkv_rows = qkv_rows.index_select(0, self.w.qkv_perm.to(self.device))
        else:
            w.qkv_rows = qkv_rows

    def _init_random(self, seed: int, std: float, norm_std: float = 0.0):
        """Seeded random weights written on the device by the counter-based generator
        (``qwen_init_weight``): the tiled and row-major copies hold the same values. RMSNorm gains
        are 1 (``Qwen3RMSNorm``'s init) unless ``norm_std > 0``, which draws them as
        ``1 + N(0, norm_std)`` from a seeded torch generator (tests of non-unit gains)."""
        s, dev = self.spec, self.device
        scale = random_init_scale(std)
        self.w.qkv_perm = self._qkv_xcd_order() if CONFIG["xcd_heads"] else None
        if self.w.qkv_perm is not None:
            self.w.qkv_map = self.w.qkv_perm.to(torch.int32).to(dev)
        gen = torch.Generator().manual_seed(seed + 7)

        def gain(n):
            if norm_std <= 0:
                return torch.ones(n, dtype=BF16, device=dev)
            return (1.0 + norm_std * torch.randn(n, generator=gen)).to(BF16).to(dev)

        qkv_seg = [0, s.Nq * s.D, (s.Nq + s.Nkv) * s.D]
        for l in range(s.L):
            w = LayerWeights()
            w.ln1, w.ln2, w.q_norm, w.k_norm = gain(s.H), gain(s.H), gain(s.D), gain(s.D)
            plan = {
                "qkv": (s.qkv_width, s.H, qkv_seg, [_tid(l, "q_proj"), _tid(l, "k_proj"), _tid(l, "v_proj")], False),
                "o": (s.H, s.Nq * s.D, [0], [_tid(l, "o_proj")], False),
                "gu": (2 * s.I, s.H, [0, s.I], [_tid(l, "gate_proj"), _tid(l, "up_proj")], True),
                "down": (s.H, s.I, [0], [_tid(l, "down_proj")], False),
            }
            for name, (N, K, starts, tids, pair) in plan.items():
                setattr(w, name, TiledWeight.random(N, K, starts, tids, seed, scale, dev, pair))
                rows = torch.empty((N, K), dtype=BF16, device=dev)
                ops.init_weight(rows, N, K, False, False, starts, tids, seed, scale)
                if name == "qkv":
                    self._finish_layer(w, rows)
                else:
                    setattr(w, name + "_rows", rows)
            self.w.layers.append(w)
        self.w.embed = TiledWeight.random(s.V, s.H, [0], [_tid(None, "embed")], seed, scale, dev)
        self.w.lm = self.w.embed
        self.w.lm_rows = torch.empty((s.V, s.H), dtype=BF16, device=dev)
        ops.init_weight(self.w.lm_rows, s.V, s.H, False, False, [0], [_tid(None, "embed")], seed, scale)
        self.w.final_norm = gain(s.H)

    def _load_checkpoint(self, model_path: str):
        """HF Qwen3 safetensors checkpoint -> device layouts (``engine/engine.py:184-230``).

        Tensors are read one at a time with the safe loader (no pickle) and moved to the
        device as bf16; q|k|v and gate|up are concatenated along the output dimension in
        the reference's order. The LM head is the embedding when ``tie_word_embeddings`` is
        set (a stored ``lm_head.weight`` is then ignored, as Transformers ties it), else the
        checkpoint's ``lm_head.weight``."""
        from safetensors import safe_open
        s, dev = self.spec, self.device
        files = sorted(f for f in os.listdir(model_path) if f.endswith(".safetensors"))
        if not files:
            raise RuntimeError(f"{model_path}: no *.safetensors weights and no random_init.json")
        where = {}
        handles = [safe_open(os.path.join(model_path, f), framework="pt", device="cpu") for f in files]
        for hnd in handles:
            for key in hnd.keys():
                where[key] = hnd

        def get(name, shape):
            if name not in where:
                raise RuntimeError(f"{model_path}: checkpoint has no tensor {name}")
            t = where[name].get_tensor(name)
            if tuple(t.shape) != tuple(shape):
                raise RuntimeError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
            return t.to(dtype=BF16).to(dev).contiguous()

        self.w.qkv_perm = self._qkv_xcd_order() if CONFIG["xcd_heads"] else None
        if self.w.qkv_perm is not None:
            self.w.qkv_map = self.w.qkv_perm.to(torch.int32).to(dev)
        for l in range(s.L):
            p = f"model.layers.{l}."
            w = LayerWeights()
            w.ln1 = get(p + "input_layernorm.weight", (s.H,))
            w.ln2 = get(p + "post_attention_layernorm.weight", (s.H,))
            w.q_norm = get(p + "self_attn.q_norm.weight", (s.D,))
            w.k_norm = get(p + "self_attn.k_norm.weight", (s.D,))
            qkv = torch.cat([get(p + "self_attn.q_proj.weight", (s.Nq * s.D, s.H)),
                             get(p + "self_attn.k_proj.weight", (s.Nkv * s.D, s.H)),
                             get(p + "self_attn.v_proj.weight", (s.Nkv * s.D, s.H))], 0)
            gu = torch.cat([get(p + "mlp.gate_proj.weight", (s.I, s.H)),
                            get(p + "mlp.up_proj.weight", (s.I, s.H))], 0)
            w.o_rows = get(p + "self_attn.o_proj.weight", (s.H, s.Nq * s.D))
            w.down_rows = get(p + "mlp.down_proj.weight", (s.H, s.I))
            w.gu_rows = gu
            w.qkv = ops.tile_weight(qkv)
            w.o = ops.tile_weight(w.o_rows)
            w.gu = ops.tile_weight(gu, pair=True)
            w.down = ops.tile_weight(w.down_rows)
            self._finish_layer(w, qkv)
            self.w.layers.append(w)
        emb = get("model.embed_tokens.weight", (s.V, s.H))
        self.w.embed = ops.tile_weight(emb)
        if s.tied:
            self.w.lm, self.w.lm_rows = self.w.embed, emb
        else:
            self.w.lm_rows = get("lm_head.weight", (s.V, s.H))
            self.w.lm = ops.tile_weight(self.w.lm_rows)
        self.w.final_norm = get("model.norm.weight", (s.H,))
        del handles, where
        torch.cuda.synchronize()

    def _rope_for(self, positions: int):
        """cos/sin ``[P, D]`` bf16 tables covering ``positions``, P a power of two >= 1024, with the
        reference's op sequence (``engine/engine.py:232-251``) on the host CPU so they are
        bit-identical to the Transformers rotary embedding, then copied to the device. A new
        table invalidates recorded graphs (they hold the old addresses)."""
        if positions <= self._rope_rows:
            return
        s = self.spec
        P = 1 << max(10, math.ceil(math.log2(max(positions, 1))))
        inv = 1.0 / (s.theta ** (torch.arange(0, s.D, 2, dtype=torch.int64).to(torch.float32) / s.D))
        t = torch.arange(P, dtype=torch.float32)[None, :]
        freqs = (inv[None, :, None].float().expand(1, -1, 1) @ t[:, None, :].float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.cos_tab = emb.cos()[0].to(BF16).contiguous().to(self.device)
        self.sin_tab = emb.sin()[0].to(BF16).contiguous().to(self.device)
        self._rope_rows = P
        if self.state is not None:
            self.state.graphs = {}

    # ================================================================== state
    @property
    def B(self) -> int:
        return self.state.B if self.state else 0

    @property
    def CAP(self) -> int:
        return self.state.cap if self.state else 0

    @property
    def k_active(self) -> int:
        return self.state.k if self.state else 0

    def _spec_k_for(self, B: int) -> int:
        k = int(CONFIG["spec_k"])
        ok = 0 < k <= 15 and B <= CONFIG["spec_max_batch"] and B * (k + 1) <= 32
        return k if ok else 0

    @torch.inference_mode()
    def prepare(self, B: int, S: int, N: int) -> rt.BatchState:
        """Batch state for ``B`` prompts of ``S`` tokens and ``N`` outputs: reused when the batch
        size and draft length match and its capacity suffices, else rebuilt. Certifies and
        records the decode steps of the shape (once per state). Runs under inference mode: the
        first graph recording in a process creates generator state that later recordings update
        in place, so all of them must run in the same mode."""
        k = self._spec_k_for(B)
        cap = rt.capacity(S, N, k, CONFIG["cap_round"])
        self._rope_for(cap)
        st = self.state
        if st is None or st.B != B or st.k != k or st.cap < cap:
            self.state = None
            if st is not None:
                del st
                torch.cuda.synchronize()
                torch.cuda.empty_cache()
            st = rt.BatchState(self.spec, B, cap, k, self.device, CONFIG["group_rows"])
            st.kv_cached = st.kv_bytes <= CONFIG["kv_cached_max_bytes"]
            self.state = st
            _log(f"batch state B={B} cap={cap} groups={len(st.groups)} spec_k={k} kv={st.kv_bytes / 2**30:.2f}GiB")
        for T in ((1, k + 1) if k else (1,)):
            if CONFIG["certify"]:
                for g in {st.groups[0].n: st.groups[0], st.groups[-1].n: st.groups[-1]}.values():
                    if (g.n, T) not in st.certified:
                        self.certify(g, T)
            if CONFIG["graphs"] and T not in st.graphs:
                issue = self._issue_plain if T == 1 else (lambda: self._issue_verify())
                st.graphs[T] = rt.StepGraph(issue, st, T).record()
                _log(f"recorded T={T} step graph: {st.graphs[T].ms:.3f} ms/step")
        return st

    def bufs(self, g: rt.RowGroup, T: int) -> StepBuffers:
        st = self.state
        key = (g.index, T)
        if key not in st.bufs:
            st.bufs[key] = StepBuffers(self.spec, g.n, T, st.cap, self.device)
        return st.bufs[key]

    # ================================================================== decode step
    def _layer(self, l: int, g: rt.RowGroup, b: StepBuffers, trace=None):
        """Decoder layer ``l`` (``engine/engine.py:1103-1118``) on the step buffers ``b`` of row
        group ``g``: the residual stream ``h`` (and its RMSNorm statistics ``psq``) is updated in
        place, K/V are written at ``pos + t``. ``trace`` (a list) receives copies of qkv, the
        attention output, h after O, the SwiGLU product and h after down."""
        w, s = self.w.layers[l], self.spec
        kc, vc = g.kv[l]
        keep = (lambda t: trace.append(t.clone())) if trace is not None else (lambda t: None)
        M = b.M
        # M <= 2: balanced row-major GEMVs (statistics computed in-kernel); else MFMA GEMMs over
        # the tiled weights, statistics from psq (left by whoever last wrote h).
        if b.gemv:
            gc = b.gemv_cfg
            ops.gemv(b.h, w.qkv_rows, norm_w=w.ln1, eps=s.eps, out=b.qkv, cfg=gc["qkv"], row_map=self.w.qkv_map)
        else:
            ops.fused_linear(b.h, w.qkv, b.cfg["qkv"], norm_w=w.ln1, eps=s.eps, out=b.qkv, psq_in=b.psq,
                             workspace=b.gemm_ws)
        keep(b.qkv)
        if b.mfma_attn:
            ops.attn_decode_mfma(b.qkv, w.q_norm, w.k_norm, s.eps, self.cos_tab, self.sin_tab, g.pos, b.T, kc, vc,
                                 self.scale, b.splits, out=b.a, workspace=b.attn_ws, waves=b.attn_waves,
                                 kv_cached=self.state.kv_cached)
        else:
            ops.attn_decode_fused(b.qkv, w.q_norm, w.k_norm, s.eps, self.cos_tab, self.sin_tab, g.pos, b.T, kc, vc,
                                  self.scale, b.splits, out=b.a, workspace=b.attn_ws, waves=b.attn_waves)
        keep(b.a)
        a = b.a.view(M, -1)
        if b.gemv:
            gc = b.gemv_cfg
            ops.gemv(a, w.o_rows, residual=b.h, out=b.h, cfg=gc["o"])
            keep(b.h)
            ops.gemv(b.h, w.gu_rows, norm_w=w.ln2, eps=s.eps, silu_pair=True, out=b.p, cfg=gc["gu"])
            keep(b.p)
            ops.gemv(b.p, w.down_rows, residual=b.h, out=b.h, cfg=gc["down"])
        else:
            ops.fused_linear(a, w.o, b.cfg["o"], residual=b.h, out=b.h, psq_out=b.psq, workspace=b.gemm_ws)
            keep(b.h)
            ops.fused_linear(b.h, w.gu, b.cfg["gu"], norm_w=w.ln2, eps=s.eps, silu_pair=True, out=b.p,
                             psq_in=b.psq, workspace=b.gemm_ws)
            keep(b.p)
            ops.fused_linear(b.p, w.down, b.cfg["down"], residual=b.h, out=b.h, psq_out=b.psq, workspace=b.gemm_ws)
        keep(b.h)

    def _lm_head(self, b: StepBuffers, extract: bool):
        """Final RMSNorm + LM head + argmax (``engine/engine.py:1119-1121``): tokens into ``b.nxt``
        with ``extract``, else left in the packed keys for the step tail."""
        if b.gemv:
            ops.gemv(b.h, self.w.lm_rows, norm_w=self.w.final_norm, eps=self.eps, amax=b.keys, cfg=b.gemv_cfg["lm"])
            if extract:
                ops.argmax_extract(b.keys, b.M, b.nxt)
        else:
            ops.lm_head_argmax(b.h, self.w.final_norm, self.eps, self.w.lm, cfg=b.lm_cfg,
                               out=b.nxt if extract else None, keys=b.keys, psq_in=b.psq, extract=extract)

    def _forward_rows(self, g: rt.RowGroup, T: int, tok=None, hidden=None) -> StepBuffers:
        """``_step`` (``engine/engine.py:1093-1121``) for row group ``g``: with ``tok [rows, T]`` the
        ids are embedded and the greedy tokens land in ``b.nxt``; without (T = 1) the input rows
        are already in ``h`` / ``psq`` and the argmax stays in the packed keys."""
        b = self.bufs(g, T)
        if tok is not None:
            ops.embed(tok.reshape(-1), self.w.embed, out=b.h, psq_out=b.psq)
        for l in range(self.spec.L):
            self._layer(l, g, b)
            if hidden is not None:
                hidden.append(b.h.clone())
        self._lm_head(b, extract=tok is not None)
        return b

    def _issue_plain(self):
        """One plain step for every row group (``engine/engine.py:941-953``): each group runs on
        the embedding of ``hist[pos]``; the tail writes the token, ``hist[pos + 1]``, advances
        ``pos`` (frozen rows write the dump slot and stay) and embeds the new ``hist[pos]``."""
        st = self.state
        for g in st.groups:
            b = self._forward_rows(g, 1)
            ops.decode_finish(b.keys, g.nxt, g.hist, g.pos, st.s_mark, st.n_mark, self.w.embed, b.h, b.psq)
        return st.nxt

    def _issue_verify(self):
        """One speculative verify step (``engine/engine.py:955-1003``): prompt-lookup drafts of k
        tokens, one forward over T = k + 1 tokens per row, acceptance of the leading matches
        (history scatter, position advance, next input row). Single row group (B <= 8)."""
        st = self.state
        g = st.groups[0]
        T = st.k + 1
        b = self.bufs(g, T)
        ops.spec_draft(g.hist, g.pos, st.k, CONFIG["spec_n"], out=b.tok)
        self._forward_rows(g, T, tok=b.tok)
        b1 = self.bufs(g, 1)
        ops.spec_accept(b.nxt, b.tok, g.hist, g.pos, st.s_mark, st.n_mark, self.w.embed, b1.h, b1.psq, b.out_t, b.adv)
        return b.out_t, b.adv

    def _plain(self):
        st = self.state
        if CONFIG["graphs"] and 1 in st.graphs:
            return st.graphs[1].launch()
        return self._issue_plain()

    def _verify(self):
        st = self.state
        T = st.k + 1
        if CONFIG["graphs"] and T in st.graphs:
            return st.graphs[T].launch()
        return self._issue_verify()

    # ================================================================== certification
    def certify(self, g: rt.RowGroup, T: int, seed: int = 0) -> dict:
        """Warmup certification (``engine/engine.py:407-486``) of the kernels one decode step of
        row group ``g`` and width ``T`` runs, on that step's own buffers, launch shapes and KV
        capacity.

        Layer 0 and the LM head run through ``_layer`` / ``_lm_head`` on a seeded N(0, 1) residual
        stream, with layer 0's cache prefix filled with N(0, 1) keys and values and ragged
        positions (the prompt forward or a decode step rewrites every slot of it before any step
        reads it). Each stage is compared with its twin (``qwen_hip.twins``) fed the kernels' own
        output of the stage before, so a mismatch names the stage; the operators of the
        reference's ``ops`` table are checked on the same data. Bars: ``atol 1e-2, rtol 1/64``,
        attention ``1e-2 / 1e-2``, the V copy and the residual of ``add_rms_norm`` bit-exact,
        greedy tokens within two bf16 ulps of the twin's maximum logit.

        Unlike the reference, a failing stage is not replaced by its twin (that would put a
        non-HIP computation into the decode step): the engine raises ``RuntimeError`` and the
        shape stays uncertified. Returns the verdict ``{stage: bool}``."""
        st, s, dev, eps = self.state, self.spec, self.device, self.eps
        b = self.bufs(g, T)
        M, rows = b.M, g.n
        w = self.w.layers[0]
        gd = torch.Generator(device=dev).manual_seed(seed)
        gh = torch.Generator().manual_seed(seed)
        pos = torch.randint(0, st.cap - T - 1, (rows,), generator=gh, dtype=torch.int32)
        pos_d = pos.to(dev)
        lengths = pos_d + T
        kc, vc = g.kv[0]
        top = int(pos.max()) + T
        verdict = {}

        def check(name, ok):
            verdict[name] = verdict.get(name, True) and bool(ok)

        saved_pos = g.pos.clone()
        with torch.inference_mode():
            kc[:, :, :top].normal_(generator=gd)
            vc[:, :, :top].normal_(generator=gd)
            h0 = torch.randn((M, s.H), generator=gd, device=dev).to(BF16)
            g.pos.copy_(pos_d)
            b.h.copy_(h0)
            ops.sumsq16(b.h, out=b.psq)
            trace = []
            self._layer(0, g, b, trace=trace)
            self._lm_head(b, extract=True)
            qkv_k, a_k, h1_k, p_k, h2_k = trace
            nxt = b.nxt.clone()
            qkv_w = self.w.natural_qkv_rows(w)
            check("step.norm_qkv", tw.close(qkv_k, tw.linear(tw.rms_norm(h0, w.ln1, eps), qkv_w)))
            q_t, k_t, v_t = tw.qk_norm_rope(qkv_k, w.q_norm, w.k_norm, eps, self.cos_tab, self.sin_tab, pos_d, T,
                                            s.Nkv)
            bi = torch.arange(rows, device=dev)[:, None].expand(rows, T)
            slots = pos_d.to(torch.int64)[:, None] + torch.arange(T, device=dev)[None, :]
            check("step.kv_write", tw.close(kc.transpose(1, 2)[bi, slots], k_t)
                  and torch.equal(vc.transpose(1, 2)[bi, slots], v_t))
            a_t = tw.attention(q_t, kc, vc, lengths, self.scale)
            check("step.attention", tw.close(a_k, a_t, atol=1e-2, rtol=1e-2))
            o_t = tw.linear(a_k.view(M, -1), w.o_rows)
            check("step.o_residual", tw.close(h1_k, tw.add(h0, o_t)))
            gu_t = tw.linear(tw.rms_norm(h1_k, w.ln2, eps), w.gu_rows)
            check("step.norm_gate_up_swiglu", tw.close(p_k, tw.silu_mul(gu_t)))
            check("step.down_residual", tw.close(h2_k, tw.add(h1_k, tw.linear(p_k, w.down_rows))))
            logits = tw.linear(tw.rms_norm(h2_k, self.w.final_norm, eps), self.w.lm_rows)
            check("step.norm_lm_head_argmax", tw.argmax_ok(nxt, logits))
            for name, op in self.ops.items():
                if name == "rms_norm":
                    check(name, tw.close(op(h0, w.ln1, eps), tw.rms_norm(h0, w.ln1, eps)))
                elif name == "add_rms_norm":
                    h_o, y_o = op(h0, o_t, w.ln2, eps)
                    h_t = tw.add(h0, o_t)
                    check(name, torch.equal(h_o, h_t) and tw.close(y_o, tw.rms_norm(h_t, w.ln2, eps)))
                elif name == "silu_mul":
                    check(name, tw.close(op(gu_t), tw.silu_mul(gu_t)))
                elif name == "qk_norm_rope_cache":
                    kc2, vc2 = kc.clone(), vc.clone()
                    q_o = op(qkv_k, w.q_norm, w.k_norm, eps, self.cos_tab, self.sin_tab, pos_d, T, kc2, vc2)
                    check(name, tw.close(q_o, q_t) and tw.close(kc2.transpose(1, 2)[bi, slots], k_t)
                          and torch.equal(vc2.transpose(1, 2)[bi, slots], v_t))
                    del kc2, vc2
                elif name == "attn_decode" and T <= 16:
                    splits = ops.choose_num_splits(rows, s.Nkv, st.cap, T)
                    a_o = op(q_t, kc, vc, lengths.to(torch.int32), self.scale, splits)
                    check(name, tw.close(a_o, a_t, atol=1e-2, rtol=1e-2))
            g.pos.copy_(saved_pos)
        torch.cuda.synchronize()
        _log(f"certified rows={rows} T={T}: {verdict}")
        failed = [k for k, ok in verdict.items() if not ok]
        if failed:
            raise RuntimeError(f"kernel certification failed on rows={rows} T={T} for {failed}; "
                               "the engine has no fallback path")
        st.certified[(rows, T)] = verdict
        return verdict

    # ================================================================== prompt forward
    def _prefill(self, ids: torch.Tensor, hidden=None, probe=None) -> torch.Tensor:
        """Prompt forward (``engine/engine.py:1181-1221``): fills the KV cache for positions
        ``[0, S)`` of every sequence and returns the first greedy token per sequence (``[B]``
        int64). The prompt runs in position chunks ``[p0, p1)`` of all ``B`` sequences
        (``prefill_tokens`` rows each); a chunk's attention reads the keys of earlier chunks
        from the cache. A chunk of more than 16 positions takes the wide attention kernel and
        gives the same bits however the prompt is cut; a shorter last chunk takes the narrow
        kernel, whose exponent and summation order differ (same bar, not the same bits).
        ``hidden`` (a list) receives the residual stream after each layer for the positions of
        the last chunk, ``[B * (p1 - p0), H]`` (row ``b * (p1 - p0) + t``); ``probe(l, p0, p1,
        a, h)`` is called after every layer of every chunk with the attention output ``a [B,
        p1 - p0, Nq * D]`` and the residual stream ``h`` (tests)."""
        st, s, dev = self.state, self.spec, self.device
        B, S = ids.shape
        chunk = max(1, min(S, CONFIG["prefill_tokens"] // B))
        h = None
        for p0 in range(0, S, chunk):
            p1 = min(S, p0 + chunk)
            Tc = p1 - p0
            last = p1 == S
            pos = torch.full((B,), p0, dtype=torch.int32, device=dev)
            h = ops.embed(ids[:, p0:p1].reshape(-1).contiguous(), self.w.embed)
            for l, w in enumerate(self.w.layers):
                kc, vc = st.kcache(l), st.vcache(l)
                n = ops.rms_norm(h, w.ln1, s.eps)
                qkv = ops.gemm(n, w.qkv)
                q = ops.qk_norm_rope_cache(qkv, w.q_norm, w.k_norm, s.eps, self.cos_tab, self.sin_tab, pos, Tc,
                                           kc, vc)
                a = ops.attn_prefill(q, kc, vc, p0, self.scale)
                ops.gemm(a.view(B * Tc, -1), w.o, residual=h, out=h)
                n = ops.rms_norm(h, w.ln2, s.eps)
                p = ops.gemm(n, w.gu, silu_pair=True)
                ops.gemm(p, w.down, residual=h, out=h)
                if hidden is not None and last:
                    hidden.append(h.clone())
                if probe is not None:
                    probe(l, p0, p1, a, h)
        h_last = h.view(B, -1, s.H)[:, -1].contiguous()
        first = torch.empty((B,), dtype=torch.int64, device=dev)
        for r0 in range(0, B, 32):
            r1 = min(B, r0 + 32)
            ops.lm_head_argmax(h_last[r0:r1], self.w.final_norm, s.eps, self.w.lm, out=first[r0:r1])
        return first

    # ================================================================== generate
    def _token_ids(self, input_ids) -> torch.Tensor:
        B = len(input_ids)
        if B == 0:
            raise ValueError("input_ids holds no sequence")
        S = len(input_ids[0])
        if S == 0 or any(len(row) != S for row in input_ids):
            raise ValueError("all prompts must be non-empty and of the same length")
        ids = torch.tensor(input_ids, dtype=torch.int64)
        if int(ids.min()) < 0 or int(ids.max()) >= self.spec.V:
            raise ValueError(f"token ids must lie in [0, {self.spec.V})")
        return ids

    def start(self, input_ids, max_new_tokens: int) -> torch.Tensor:
        """Everything ``generate`` does before its first yield: batch state, prompt forward,
        history and positions, the first decode step's input rows. Returns the first token of
        every sequence (``[B]`` int64 on the device)."""
        ids_cpu = self._token_ids(input_ids)
        B, S = ids_cpu.shape
        N = int(max_new_tokens)
        with torch.inference_mode():
            st = self.prepare(B, S, N)
            ids = ids_cpu.to(self.device)
            first = self._prefill(ids)
            st.hist[:, :S].copy_(ids)
            st.hist[:, S].copy_(first)
            st.pos.fill_(S)
            st.marks[0] = S
            st.marks[1] = N
            for g in st.groups:
                b = self.bufs(g, 1)
                ops.embed_hist(g.hist, g.pos, self.w.embed, b.h, psq_out=b.psq)
        return first

    def generate(self, input_ids: list[list[int]], max_new_tokens: int):
        """Greedy continuation of every sequence (``engine/engine.py:1225-1250``): yields a list of
        one token id per sequence per output position, exactly ``max_new_tokens`` times; never
        stops at an end-of-sequence token."""
        N = int(max_new_tokens)
        if N <= 0:
            return
        first = self.start(input_ids, N)
        st = self.state
        k = st.k
        t_plain = st.graphs[1].ms if 1 in st.graphs else 1.0
        t_verify = st.graphs[k + 1].ms if k and (k + 1) in st.graphs else 1.0
        policy = rt.SpecPolicy(k, t_plain, t_verify, CONFIG["spec_backoff"], CONFIG["spec_probe_len"],
                               CONFIG["spec_policy"])
        pump = rt.TokenPump(st.B, N, first, CONFIG["inflight"], k, self._plain, self._verify, policy,
                            self.counters)
        yield from pump

    # ================================================================== test / bench hooks
    def verify_step(self, tok: torch.Tensor, positions) -> torch.Tensor:
        """Greedy next token at every position of ``tok [B, T]`` (the verify forward of
        ``engine/engine.py:979-993``): token ``t`` of row ``b`` sits at ``positions[b] + t`` and
        its K/V are written there. Needs the prepared batch in one row group. Returns ``[B, T]``
        int64 (synchronises)."""
        B, T = tok.shape
        st = self.state
        assert st is not None and B == st.B and len(st.groups) == 1 and B * T <= 32 and T <= 16
        g = st.groups[0]
        with torch.inference_mode():
            g.pos.copy_(torch.as_tensor(positions, dtype=torch.int32).reshape(B).to(self.device))
            b = self._forward_rows(g, T, tok=tok.to(self.device, torch.int64).contiguous())
            out = b.nxt.view(B, T).clone()
        torch.cuda.synchronize()
        return out

    def step_hidden(self, tok: torch.Tensor, positions) -> list:
        """One eager step of ``tok [B, T]`` (T = 1: a decode step; T > 1: the verify forward, token
        ``t`` of row ``b`` at ``positions[b] + t``) on the prepared batch, one row group; returns
        the residual stream ``[B * T, H]`` after every layer."""
        st = self.state
        g = st.groups[0]
        T = tok.shape[1]
        assert tok.shape[0] == st.B and len(st.groups) == 1 and st.B * T <= 32 and T <= 16
        hidden = []
        with torch.inference_mode():
            g.pos.copy_(torch.as_tensor(positions, dtype=torch.int32).reshape(-1).to(self.device))
            self._forward_rows(g, T, tok=tok.to(self.device, torch.int64).contiguous(), hidden=hidden)
        torch.cuda.synchronize()
        return hidden

    def layer_step(self, l: int, hidden: torch.Tensor, positions, T: int = 1) -> list:
        """One decoder layer on a given residual stream ``hidden [B*T, H]`` at ``positions`` (the
        single-layer case): returns ``_layer``'s trace (qkv, attention
        output, h after O, SwiGLU product, h after down). Prepared batch, one row group."""
        st = self.state
        g = st.groups[0]
        b = self.bufs(g, T)
        assert hidden.shape == (b.M, self.spec.H)
        trace = []
        with torch.inference_mode():
            g.pos.copy_(torch.as_tensor(positions, dtype=torch.int32).reshape(-1).to(self.device))
            b.h.copy_(hidden.to(self.device, BF16))
            ops.sumsq16(b.h, out=b.psq)
            self._layer(l, g, b, trace=trace)
        torch.cuda.synchronize()
        return trace

    def prefill_hidden(self, input_ids, N: int = 1, probe=None):
        """Prompt forward of ``input_ids`` on a fresh batch state; returns ``(first [B], hidden)``
        with the residual stream after each layer (positions of the last prompt chunk);
        ``probe`` as in ``_prefill``."""
        ids = self._token_ids(input_ids)
        hidden = []
        with torch.inference_mode():
            self.prepare(ids.shape[0], ids.shape[1], N)
            first = self._prefill(ids.to(self.device), hidden=hidden, probe=probe)
        torch.cuda.synchronize()
        return first, hidden
