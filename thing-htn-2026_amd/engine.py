"""Qwen3-4B greedy-decode engine for one MI355X (gfx950): drop-in for the reference's ``engine/engine.py``.

Same public surface as the reference (``engine/engine.py:109-111``,
``:1225-1250``): ``Engine(model_path)`` loads the model once; then
``generate(input_ids, max_new_tokens)`` is a generator that yields exactly
``max_new_tokens`` lists of ``B`` Python ints, the first from the prompt
forward, then one per decode step. State resets on every call; batch size and
prompt length may change between calls.

Per decode step the device runs only hand-written HIP kernels from
``qwen_hip`` (libqwen_hip.so), recorded once per batch shape into one HIP
graph (``torch.cuda.CUDAGraph``) and replayed per token:

    36 x [ norm+QKV GEMM |
           QK-norm + RoPE + KV write + split-K attention + merge |
           O GEMM + residual | norm+gate/up GEMM+SwiGLU |
           down GEMM + residual ]                      5 kernels / layer
    final norm + LM head + argmax                      1 kernel
    token / history / position update + next embedding 1 kernel

With ``CONFIG["spec_k"] = k > 0`` (exact speculative decoding, off by default as in
the reference) a second graph verifies k prompt-lookup drafts per sequence in one
T = k + 1 step: draft kernel | the same per-layer kernels over B*T rows | accept
kernel (history scatter, position advance, next input row); the decode loop picks
verify or plain steps adaptively.

Torch is used for device memory, the KV cache, the RoPE tables, graph
capture, host<->device copies and (for now) the prompt forward's large GEMMs
and causal attention (hipBLASLt / SDPA flash), whose norms, RoPE, cache writes
and SwiGLU are the same HIP kernels. There is no CPU fallback: without a GPU
or without libqwen_hip.so the constructor raises.
"""

from __future__ import annotations

import glob
import json
import math
import os
import sys
import time
from collections import deque

import torch
import torch.nn.functional as F

from qwen_hip import ops
from qwen_hip import twins as tw
from qwen_hip.ops import TiledWeight

BF16 = torch.bfloat16

CONFIG = {
    "graphs": True,          # replay one HIP graph per decode step
    "pipeline_depth": 3,     # decode steps in flight ahead of the host yield (engine/engine.py:71)
    "prefill_rows": 32768,   # max B*S rows per prompt-forward batch slice (engine/engine.py:72)
    "cap_align": 64,         # KV-cache capacity alignment (engine/engine.py:73)
    # Exact speculative decoding (engine/engine.py:79-82): prompt-lookup drafts of spec_k tokens
    # verified in one T = spec_k + 1 step; 0 = off (the reference's default).
    "spec_k": int(os.environ.get("QWEN_ENGINE_SPEC_K", "0")),
    "spec_n": 3,             # n-gram length of the draft lookup
    "spec_max_batch": 8,     # speculate only when B <= this (and B * (spec_k + 1) <= 32)
    "spec_probe": (24, 6),   # while speculation loses: plain steps between probes, spec steps per probe
    # Run each decode-step shape's kernels against the torch twins once at warmup and refuse
    # to decode on a mismatch (engine/engine.py:407-486; the reference falls back instead).
    "certify": os.environ.get("QWEN_ENGINE_CERTIFY", "1") != "0",
    # M <= 2: order the QKV GEMV's weight rows so that each KV head's q / k / v rows are
    # produced on the XCD that runs that head's attention workgroup.
    "xcd_heads": os.environ.get("QWEN_ENGINE_XCD_HEADS", "1") != "0",
    # Whole-KV-cache size up to which the decode attention reads K/V with cache-allocating
    # loads (measured on MI355X: c2 527 -> 530 tok/s; non-temporal loads win at c4).
    "kv_cached_max_bytes": int(os.environ.get("QWEN_ENGINE_KV_CACHED_MAX", str(128 << 20))),
    "log": True,
}

XCDS = 8   # MI355X: 8 XCDs, workgroup i of a launch runs on XCD i mod 8

# Tensor ids of the counter-based random-init generator (one per HF weight).
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


class _Layer:
    __slots__ = ("ln1", "w_qkv", "q_norm", "k_norm", "w_o", "ln2", "w_gu", "w_down",
                 "r_qkv", "r_o", "r_gu", "r_down", "g_qkv")


class Engine:
    def __init__(self, model_path: str) -> None:
        """Load the model from ``model_path`` (HF checkpoint dir, or config + random_init.json)."""
        t0 = time.time()
        if not torch.cuda.is_available():
            raise RuntimeError("Engine needs an MI355X GPU (HIP device); there is no CPU path")
        self.device = torch.device("cuda:0")
        torch.backends.cuda.matmul.allow_tf32 = False
        with open(os.path.join(model_path, "config.json")) as handle:
            cfg = json.load(handle)
        self.cfg = cfg
        self.H = cfg["hidden_size"]
        self.I = cfg["intermediate_size"]
        self.V = cfg["vocab_size"]
        self.L = cfg["num_hidden_layers"]
        self.Nq = cfg["num_attention_heads"]
        self.Nkv = cfg["num_key_value_heads"]
        self.D = cfg.get("head_dim") or self.H // self.Nq
        self.eps = float(cfg["rms_norm_eps"])
        theta = cfg.get("rope_theta")
        if theta is None:
            theta = (cfg.get("rope_parameters") or {}).get("rope_theta")
        self.theta = float(theta)
        self.scale = self.D ** -0.5
        rope_params = cfg.get("rope_parameters") or {}
        if cfg.get("rope_scaling") is not None or rope_params.get("rope_type", "default") != "default":
            raise RuntimeError("rope_scaling is not supported by this engine")
        if self.D != 128 or self.Nq != 4 * self.Nkv:
            raise RuntimeError(f"kernels support head_dim 128 and 4 query heads per KV head (got {self.D}, "
                               f"{self.Nq}/{self.Nkv})")
        if self.H % 32 or self.I % 32 or self.V % 16:
            raise RuntimeError("hidden/intermediate sizes must be multiples of 32 and vocab of 16")
        self.ops = {
            "rms_norm": ops.rms_norm,
            "add_rms_norm": ops.add_rms_norm,
            "silu_mul": ops.silu_mul,
            "qk_norm_rope_cache": ops.qk_norm_rope_cache,
            "attn_decode": ops.attn_decode,
        }
        self.B = self.CAP = 0
        self.graphs = {}
        self.certified = {}
        self.kv_cached = False
        self.step_ms = {}
        self.sdpa_mode = None
        self.decode_launches = 0   # decode steps launched since load (benchmarks read it)
        self.spec_launches = 0     # of which speculative verify steps
        self.spec_tokens = 0       # tokens the slowest unfinished row gained from them
        self.k_active = 0          # draft tokens per verify step for the prepared batch (0: plain only)
        self._load_weights(model_path)
        self.qkv_map = None
        if CONFIG["xcd_heads"]:
            order = self._qkv_xcd_order()
            if order is not None:
                self.qkv_map = order.to(torch.int32).to(self.device)
                idx = order.to(self.device)
                for w in self.layers:
                    w.g_qkv = w.r_qkv.index_select(0, idx).contiguous()
        self._rope_max = 0
        self._ensure_rope(8192)
        torch.cuda.synchronize()
        _log(f"loaded in {time.time() - t0:.1f}s: L={self.L} H={self.H} V={self.V}")

    # ------------------------------------------------------------------ weights
    def _qkv_xcd_order(self):
        """Row order of the QKV weight for the M <= 2 GEMV in which the workgroups of one XCD
        produce exactly one KV head group (its query heads, key and value rows), or None when
        the shapes do not allow it.

        Workgroup g of a launch runs on XCD g mod 8, the GEMV's workgroup g owns weight rows
        [N g / G, N (g + 1) / G), and the attention's workgroup for (sequence b, KV head h)
        is number b * Nkv + h. With Nkv = 8 and each head group exactly G / 8 workgroups of
        rows, permuting the rows as below (and storing each output at its natural column)
        leaves head h's q / k / v rows in the L2 of the XCD whose attention workgroup reads
        them. Returns ``orig [N]``: permuted row p is natural row orig[p]."""
        N = (self.Nq + 2 * self.Nkv) * self.D
        G, _ = ops.gemv_config(1, N, self.H, ops.GEPI_STORE, self.device)
        qd = (self.Nq // self.Nkv) * self.D
        grp = qd + 2 * self.D
        if self.Nkv != XCDS or N % G or G % XCDS or grp != (G // XCDS) * (N // G):
            return None
        rows = N // G
        p = torch.arange(N, dtype=torch.int64)
        g, j = p // rows, p % rows
        h, i = g % XCDS, (g // XCDS) * rows + j
        k0, v0 = self.Nq * self.D, (self.Nq + self.Nkv) * self.D
        return torch.where(i < qd, h * qd + i,
                           torch.where(i < qd + self.D, k0 + h * self.D + (i - qd), v0 + h * self.D + (i - qd - self.D)))

    def _load_weights(self, model_path):
        rnd = os.path.join(model_path, "random_init.json")
        if os.path.exists(rnd):
            with open(rnd) as handle:
                spec = json.load(handle)
            self._init_random(int(spec.get("seed", 0)), float(spec.get("std", 0.02)))
        else:
            self._load_safetensors(model_path)

    def _init_random(self, seed: int, std: float):
        """Random-init weights on the device from the counter-based generator (tiled + row-major)."""
        dev, H, I, D, Nq, Nkv = self.device, self.H, self.I, self.D, self.Nq, self.Nkv
        scale = random_init_scale(std)
        ones_h = torch.ones(H, dtype=BF16, device=dev)
        ones_d = torch.ones(D, dtype=BF16, device=dev)
        self.layers = []
        for l in range(self.L):
            w = _Layer()
            w.ln1, w.ln2, w.q_norm, w.k_norm = ones_h.clone(), ones_h.clone(), ones_d.clone(), ones_d.clone()
            qkv_seg = ([0, Nq * D, (Nq + Nkv) * D],
                       [_tid(l, "q_proj"), _tid(l, "k_proj"), _tid(l, "v_proj")])
            gu_seg = ([0, I], [_tid(l, "gate_proj"), _tid(l, "up_proj")])
            shapes = {
                "qkv": ((Nq + 2 * Nkv) * D, H, qkv_seg, False),
                "o": (H, Nq * D, ([0], [_tid(l, "o_proj")]), False),
                "gu": (2 * I, H, gu_seg, True),
                "down": (H, I, ([0], [_tid(l, "down_proj")]), False),
            }
            for name, (N, K, (starts, tids), pair) in shapes.items():
                setattr(w, "w_" + name, TiledWeight.random(N, K, starts, tids, seed, scale, dev, pair))
                row = torch.empty((N, K), dtype=BF16, device=dev)
                ops.init_weight(row, N, K, False, False, starts, tids, seed, scale)
                setattr(w, "r_" + name, row)
            self.layers.append(w)
        self.embed = TiledWeight.random(self.V, H, [0], [_tid(None, "embed")], seed, scale, dev)
        self.embed_rows = torch.empty((self.V, H), dtype=BF16, device=dev)
        ops.init_weight(self.embed_rows, self.V, H, False, False, [0], [_tid(None, "embed")], seed, scale)
        self.final_norm = ones_h.clone()

    def _load_safetensors(self, model_path):
        """HF Qwen3 checkpoint (safetensors, safe loader) -> fused, tiled device weights."""
        from safetensors.torch import safe_open
        files = sorted(glob.glob(os.path.join(model_path, "*.safetensors")))
        if not files:
            raise RuntimeError(f"no safetensors weights and no random_init.json in {model_path}")
        tensors = {}
        for f in files:
            with safe_open(f, framework="pt", device="cpu") as handle:
                for k in handle.keys():
                    tensors[k] = handle.get_tensor(k)

        def get(name):
            return tensors[name].to(device=self.device, dtype=BF16).contiguous()

        self.layers = []
        for l in range(self.L):
            p = f"model.layers.{l}."
            w = _Layer()
            w.ln1 = get(p + "input_layernorm.weight")
            w.ln2 = get(p + "post_attention_layernorm.weight")
            w.q_norm = get(p + "self_attn.q_norm.weight")
            w.k_norm = get(p + "self_attn.k_norm.weight")
            w.r_qkv = torch.cat([get(p + "self_attn.q_proj.weight"), get(p + "self_attn.k_proj.weight"),
                                 get(p + "self_attn.v_proj.weight")], 0).contiguous()
            w.r_o = get(p + "self_attn.o_proj.weight")
            w.r_gu = torch.cat([get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight")], 0).contiguous()
            w.r_down = get(p + "mlp.down_proj.weight")
            w.w_qkv = ops.tile_weight(w.r_qkv)
            w.w_o = ops.tile_weight(w.r_o)
            w.w_gu = ops.tile_weight(w.r_gu, pair=True)
            w.w_down = ops.tile_weight(w.r_down)
            self.layers.append(w)
        emb = get("model.embed_tokens.weight")
        self.embed = ops.tile_weight(emb)
        self.embed_rows = emb          # row-major copy: the M <= 2 LM head streams it
        if "lm_head.weight" in tensors and not self.cfg.get("tie_word_embeddings", True):
            raise RuntimeError("untied LM head is not supported (Qwen3-4B ties it to the embedding)")
        self.final_norm = get("model.norm.weight")
        del tensors

    def _ensure_rope(self, max_pos):
        """cos/sin ``[P, D]`` bf16 with the reference's op sequence (``engine/engine.py:232-251``).

        Computed on the host CPU so the table is bit-identical to the
        Transformers rotary embedding on CPU, then copied to the device.
        """
        if max_pos <= self._rope_max:
            return
        P = int(2 ** math.ceil(math.log2(max(max_pos, 1024))))
        inv_freq = 1.0 / (self.theta ** (torch.arange(0, self.D, 2, dtype=torch.int64).to(torch.float32) / self.D))
        pos = torch.arange(P, dtype=torch.float32)[None, :]
        freqs = (inv_freq[None, :, None].float().expand(1, -1, 1) @ pos[:, None, :].float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        self.cos_tab = emb.cos()[0].to(BF16).contiguous().to(self.device)
        self.sin_tab = emb.sin()[0].to(BF16).contiguous().to(self.device)
        self._rope_max = P
        self.graphs = {}  # captured graphs hold the old table addresses

    # ------------------------------------------------------------------ state
    def _prepare(self, B, S, N):
        """Per-shape state (``engine/engine.py:830-863``): KV cache, history, buffers, graph."""
        if B > 32:
            raise ValueError("this engine decodes at most 32 sequences per call")
        k = int(CONFIG["spec_k"])
        if not (0 < k <= 15 and B <= CONFIG["spec_max_batch"] and B * (k + 1) <= 32):
            k = 0
        slack = (CONFIG["pipeline_depth"] + 3) * (k + 1) + 16
        align = CONFIG["cap_align"]
        cap = ((S + N + slack + align - 1) // align) * align
        self._ensure_rope(cap)
        if B != self.B or cap > self.CAP or k != getattr(self, "k_active", 0):
            torch.cuda.synchronize()
            self.graphs = {}
            self.k_cache = self.v_cache = None
            torch.cuda.empty_cache()
            dev = self.device
            shape = (B, self.Nkv, cap, self.D)
            self.k_cache = [torch.zeros(shape, dtype=BF16, device=dev) for _ in range(self.L)]
            self.v_cache = [torch.zeros(shape, dtype=BF16, device=dev) for _ in range(self.L)]
            self.hist_buf = torch.zeros((B, cap), dtype=torch.int64, device=dev)
            self.pos_buf = torch.zeros((B,), dtype=torch.int32, device=dev)
            self.s_buf = torch.zeros((1,), dtype=torch.int64, device=dev)
            self.ntarget_buf = torch.full((1,), 1 << 40, dtype=torch.int64, device=dev)
            self.B, self.CAP, self.k_active = B, cap, k
            self.certified = {}
            # A KV cache well inside the 256 MB Infinity Cache stays there between steps when it
            # is read with cache-allocating loads; larger ones stream with non-temporal loads.
            kv_bytes = 2 * self.L * B * self.Nkv * cap * self.D * 2
            self.kv_cached = kv_bytes <= CONFIG["kv_cached_max_bytes"]
            self.bufs = {}
            ring = CONFIG["pipeline_depth"] + 2
            self.pin_nxt = [torch.zeros((k + 1, B), dtype=torch.int64, pin_memory=True) for _ in range(ring)]
            self.pin_adv = [torch.zeros((B,), dtype=torch.int64, pin_memory=True) for _ in range(ring)]
            self.events = [torch.cuda.Event() for _ in range(ring)]
            _log(f"state B={B} CAP={cap} spec_k={k} "
                 f"kv={2 * self.L * B * self.Nkv * cap * self.D * 2 / 2**30:.2f}GiB")
        for T in (1, k + 1) if k else (1,):
            if CONFIG["certify"] and (B, T) not in self.certified:
                self._certify(B, T)
            if CONFIG["graphs"] and T not in self.graphs:
                self._capture(T)

    def _buffers(self, B, T):
        """Static activation buffers for a (B, T) step, reused by every replay."""
        key = (B, T)
        if key not in self.bufs:
            M, dev = B * T, self.device
            mfma = T <= ops.MFMA_MAX_T   # matrix-core attention for decode / verify widths
            S = (ops.choose_mfma_splits(B, self.Nkv, self.CAP) if mfma
                 else ops.choose_num_splits(B, self.Nkv, self.CAP, T))
            W_qkv = (self.Nq + 2 * self.Nkv) * self.D
            cfg = {
                "qkv": ops.gemm_config(M, W_qkv, self.H),
                "o": ops.gemm_config(M, self.H, self.Nq * self.D),
                "gu": ops.gemm_config(M, 2 * self.I, self.H, True),
                "down": ops.gemm_config(M, self.H, self.I),
            }
            n_of = {"qkv": W_qkv, "o": self.H, "gu": 2 * self.I, "down": self.H}
            ws = max(ops.gemm_workspace_bytes(M, n_of[k], c) for k, c in cfg.items())
            gemv = M <= ops.GEMV_MAX_M
            gemv_cfg = {
                "qkv": ops.gemv_config(M, W_qkv, self.H, ops.GEPI_STORE, dev),
                "o": ops.gemv_config(M, self.H, self.Nq * self.D, ops.GEPI_RES, dev),
                "gu": ops.gemv_config(M, self.I, self.H, ops.GEPI_SWIGLU, dev),
                "down": ops.gemv_config(M, self.H, self.I, ops.GEPI_RES, dev),
                "lm": ops.gemv_config(M, self.V, self.H, ops.GEPI_ARGMAX, dev),
            } if gemv else None
            self.bufs[key] = {
                "h": torch.zeros((M, self.H), dtype=BF16, device=dev),
                "qkv": torch.empty((M, W_qkv), dtype=BF16, device=dev),
                "a": torch.empty((B, T, self.Nq * self.D), dtype=BF16, device=dev),
                "p": torch.empty((M, self.I), dtype=BF16, device=dev),
                "psq": torch.zeros((M, self.H // 16), dtype=torch.float32, device=dev),
                "next": torch.empty((M,), dtype=torch.int64, device=dev),
                "tok": torch.zeros((B, T), dtype=torch.int64, device=dev),      # verify-step input ids
                "out_t": torch.zeros((T, B), dtype=torch.int64, device=dev),    # verify-step tokens, [T, B]
                "adv": torch.zeros((B,), dtype=torch.int64, device=dev),        # accepted tokens per row
                "keys": ops.argmax_keys(M, dev),
                "attn_mfma": mfma,
                "splits": S,
                "attn_waves": ops.MFMA_WAVES if mfma else ops.attn_waves(B, T),
                "attn_ws": (ops.attn_mfma_workspace(B, T, self.Nkv, S, dev) if mfma
                            else ops.attn_workspace(B, T, self.Nq, self.Nkv, self.D, S, dev)),
                "gemm_ws": ops.linear_workspace(ws, dev),
                "cfg": cfg,
                "gemv": gemv,
                "gemv_cfg": gemv_cfg,
                "lm_cfg": ops.lm_head_config(M, self.V, self.H),
            }
        return self.bufs[key]

    # ------------------------------------------------------------------ decode step
    def _step(self, T, tok=None, hidden=None):
        """One decode step of ``T`` tokens per sequence (``engine/engine.py:1093-1121``).

        With ``tok [B, T]`` int64 the step embeds those ids and returns the
        greedy ``next [B*T]`` int64 buffer. Without it (T = 1, the plain step)
        the input rows are already in ``h`` / ``psq`` (the embedding of
        ``hist[b, pos[b]]``, left there by the previous step's tail or by
        ``_prime``) and the argmax stays in the packed keys for ``decode_finish``.
        Positions are ``pos_buf``; K/V are written at ``pos + t``. Issues only
        HIP kernels and allocates nothing, so it is capturable.
        """
        B = self.B
        M = B * T
        b = self._buffers(B, T)
        h, psq = b["h"], b["psq"]
        # psq holds the per-16-column sums of squares of the current residual
        # stream h: written by whoever last wrote h (embedding, O / down
        # epilogues), read by the next normed projection.
        if tok is not None:
            ops.embed(tok.reshape(-1), self.embed, out=h, psq_out=psq)
        else:
            assert T == 1
        for l in range(self.L):
            self._layer(l, b, T)
            if hidden is not None:
                hidden.append(h.clone())
        self._lm_head(b, M, extract=tok is not None)
        return b["next"]

    def _lm_head(self, b, M, extract):
        """Final RMSNorm + tied LM head + argmax of the step buffers ``b`` (``engine/engine.py:1119-1121``):
        tokens into ``b["next"]`` with ``extract``, else left in the packed keys for ``decode_finish``."""
        if b["gemv_cfg"] is not None:
            ops.gemv(b["h"], self.embed_rows, norm_w=self.final_norm, eps=self.eps, amax=b["keys"],
                     cfg=b["gemv_cfg"]["lm"])
            if extract:
                ops.argmax_extract(b["keys"], M, b["next"])
        else:
            ops.lm_head_argmax(b["h"], self.final_norm, self.eps, self.embed, cfg=b["lm_cfg"],
                               out=b["next"] if extract else None, keys=b["keys"], psq_in=b["psq"], extract=extract)

    def _layer(self, l, b, T, trace=None):
        """Decoder layer ``l`` of ``_step`` (``engine/engine.py:1103-1118``) on the step buffers
        ``b``: the residual stream ``h`` (and its statistics ``psq``) is updated in place, K/V
        are written at ``pos_buf + t``. ``trace`` (a list) receives copies of qkv, the attention
        output, h after the O projection, the SwiGLU product and h after the down projection."""
        M = self.B * T
        w = self.layers[l]
        h, qkv, a, p, psq, cfg, ws = b["h"], b["qkv"], b["a"], b["p"], b["psq"], b["cfg"], b["gemm_ws"]
        gc = b["gemv_cfg"]
        keep = (lambda t: trace.append(t.clone())) if trace is not None else (lambda t: None)
        # M <= 2: balanced row-major GEMVs (RMSNorm statistics computed in-kernel);
        # larger M: MFMA kernels over the tiled weights, statistics from psq.
        if gc is not None:
            if self.qkv_map is not None:   # head h's rows produced on XCD h (see _qkv_xcd_order)
                ops.gemv(h, w.g_qkv, norm_w=w.ln1, eps=self.eps, out=qkv, cfg=gc["qkv"], row_map=self.qkv_map)
            else:
                ops.gemv(h, w.r_qkv, norm_w=w.ln1, eps=self.eps, out=qkv, cfg=gc["qkv"])
        else:
            ops.fused_linear(h, w.w_qkv, cfg["qkv"], norm_w=w.ln1, eps=self.eps, out=qkv, psq_in=psq, workspace=ws)
        keep(qkv)
        if b["attn_mfma"]:
            ops.attn_decode_mfma(qkv, w.q_norm, w.k_norm, self.eps, self.cos_tab, self.sin_tab, self.pos_buf, T,
                                 self.k_cache[l], self.v_cache[l], self.scale, b["splits"], out=a,
                                 workspace=b["attn_ws"], waves=b["attn_waves"], kv_cached=self.kv_cached)
        else:
            ops.attn_decode_fused(qkv, w.q_norm, w.k_norm, self.eps, self.cos_tab, self.sin_tab, self.pos_buf, T,
                                  self.k_cache[l], self.v_cache[l], self.scale, b["splits"], out=a,
                                  workspace=b["attn_ws"], waves=b["attn_waves"])
        keep(a)
        if gc is not None:
            ops.gemv(a.view(M, -1), w.r_o, residual=h, out=h, cfg=gc["o"])
            keep(h)
            ops.gemv(h, w.r_gu, norm_w=w.ln2, eps=self.eps, silu_pair=True, out=p, cfg=gc["gu"])
            keep(p)
            ops.gemv(p, w.r_down, residual=h, out=h, cfg=gc["down"])
        else:
            ops.fused_linear(a.view(M, -1), w.w_o, cfg["o"], residual=h, out=h, psq_out=psq, workspace=ws)
            keep(h)
            ops.fused_linear(h, w.w_gu, cfg["gu"], norm_w=w.ln2, eps=self.eps, silu_pair=True, out=p,
                             psq_in=psq, workspace=ws)
            keep(p)
            ops.fused_linear(p, w.w_down, cfg["down"], residual=h, out=h, psq_out=psq, workspace=ws)
        keep(h)

    def layer_step(self, l: int, hidden: torch.Tensor, positions, T: int = 1) -> list:
        """One decoder layer on a given residual stream ``hidden [B*T, H]`` at ``positions``
        (the reference's single-layer case): returns the per-tensor trace of
        ``_layer`` (qkv, attention output, h after O, SwiGLU product, h after down). Uses the
        prepared batch and caches; eager, synchronous."""
        assert hidden.shape == (self.B * T, self.H)
        b = self._buffers(self.B, T)
        trace = []
        with torch.inference_mode():
            self.pos_buf.copy_(torch.as_tensor(positions, dtype=torch.int32).reshape(-1).to(self.device))
            b["h"].copy_(hidden.to(self.device, BF16))
            ops.sumsq16(b["h"], out=b["psq"])
            self._layer(l, b, T, trace=trace)
        torch.cuda.synchronize()
        return trace

    def _certify(self, B, T, seed=0):
        """Warmup certification (``engine/engine.py:407-486``) of the kernels one decode step of
        ``(B, T)`` runs, on that step's own buffers, launch configurations and KV capacity.

        Layer 0 and the LM head run through ``_layer`` / ``_lm_head`` on a seeded N(0, 1) residual
        stream, with layer 0's cache prefix filled with N(0, 1) keys and values and ragged
        positions (every slot of it is rewritten by the prompt forward or by a decode step before
        any step reads it). Each stage is compared with its twin (``qwen_hip.twins``) fed the
        kernels' own output of the stage before, so a mismatch names the stage; the standalone
        operators of the reference's ``ops`` table are checked on the same data. The bars are the
        reference's: ``atol 1e-2, rtol 1/64``, attention ``1e-2 / 1e-2``, the V-cache copy and
        the residual stream of ``add_rms_norm`` bit-exact, and greedy tokens within two bf16 ulps
        of the twin's maximum logit.

        Unlike the reference, a failed stage is not replaced by its twin (that would put a non-HIP
        computation into the decode step): the engine raises ``RuntimeError`` and the shape stays
        uncertified. Returns the verdict ``{stage: bool}`` (kept in ``self.certified[(B, T)]``).
        """
        M, dev, eps = B * T, self.device, self.eps
        b = self._buffers(B, T)
        w = self.layers[0]
        g = torch.Generator(device=dev).manual_seed(seed)
        gh = torch.Generator().manual_seed(seed)
        pos = torch.randint(0, self.CAP - T, (B,), generator=gh, dtype=torch.int32)
        pos_d = pos.to(dev)
        lengths = pos_d + T
        kc, vc = self.k_cache[0], self.v_cache[0]
        Lmax = int(pos.max()) + T
        verdict = {}

        def check(name, ok):
            verdict[name] = verdict.get(name, True) and bool(ok)

        with torch.inference_mode():
            kc[:, :, :Lmax].normal_(generator=g)
            vc[:, :, :Lmax].normal_(generator=g)
            h0 = torch.randn((M, self.H), generator=g, device=dev).to(BF16)
            self.pos_buf.copy_(pos_d)
            b["h"].copy_(h0)
            ops.sumsq16(b["h"], out=b["psq"])
            trace = []
            self._layer(0, b, T, trace=trace)
            self._lm_head(b, M, extract=True)
            qkv_k, a_k, h1_k, p_k, h2_k = trace
            nxt = b["next"].clone()
            # decode-step stages, each twin fed the kernels' previous stage
            check("step.norm_qkv", tw.close(qkv_k, tw.linear(tw.rms_norm(h0, w.ln1, eps), w.r_qkv)))
            q_t, k_t, v_t = tw.qk_norm_rope(qkv_k, w.q_norm, w.k_norm, eps, self.cos_tab, self.sin_tab, pos_d, T,
                                            self.Nkv)
            bi = torch.arange(B, device=dev)[:, None].expand(B, T)
            slots = pos_d.to(torch.int64)[:, None] + torch.arange(T, device=dev)[None, :]
            check("step.kv_write", tw.close(kc.transpose(1, 2)[bi, slots], k_t)
                  and torch.equal(vc.transpose(1, 2)[bi, slots], v_t))
            a_t = tw.attention(q_t, kc, vc, lengths, self.scale)
            check("step.attention", tw.close(a_k, a_t, atol=1e-2, rtol=1e-2))
            o_t = tw.linear(a_k.view(M, -1), w.r_o)
            check("step.o_residual", tw.close(h1_k, tw.add(h0, o_t)))
            gu_t = tw.linear(tw.rms_norm(h1_k, w.ln2, eps), w.r_gu)
            check("step.norm_gate_up_swiglu", tw.close(p_k, tw.silu_mul(gu_t)))
            check("step.down_residual", tw.close(h2_k, tw.add(h1_k, tw.linear(p_k, w.r_down))))
            logits = tw.linear(tw.rms_norm(h2_k, self.final_norm, eps), self.embed_rows)
            check("step.norm_lm_head_argmax", tw.argmax_ok(nxt, logits))
            # the reference's operator table on the same data
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
                    splits = ops.choose_num_splits(B, self.Nkv, self.CAP, T)
                    a_o = op(q_t, kc, vc, lengths.to(torch.int32), self.scale, splits)
                    check(name, tw.close(a_o, a_t, atol=1e-2, rtol=1e-2))
        torch.cuda.synchronize()
        _log(f"certified on B={B} T={T}: {verdict}")
        failed = [k for k, ok in verdict.items() if not ok]
        if failed:
            raise RuntimeError(f"kernel certification failed on B={B} T={T} for {failed}; "
                               "the engine has no fallback path")
        self.certified[(B, T)] = verdict
        return verdict

    def _plain_step(self):
        """``_plain_step`` (``engine/engine.py:941-953``): step on hist[pos], write hist[pos+1], pos += 1,
        and leave the embedding of the new hist[pos] in ``h`` for the next step."""
        self._step(1)
        b = self._buffers(self.B, 1)
        ops.decode_finish(b["keys"], b["next"], self.hist_buf, self.pos_buf, self.s_buf, self.ntarget_buf, self.embed,
                          b["h"], b["psq"])
        return b["next"]

    def _prime(self):
        """Embed ``hist[b, pos[b]]`` into the plain step's input rows (before the first decode step)."""
        b = self._buffers(self.B, 1)
        ops.embed_hist(self.hist_buf, self.pos_buf, self.embed, b["h"], psq_out=b["psq"])

    def _spec_step(self, k):
        """``_spec_step`` (``engine/engine.py:979-1003``): draft ``k`` tokens per sequence by prompt
        lookup, verify them in one T = k+1 step, accept the leading matches. Returns ``(out_t [T, B],
        adv [B])``; also leaves the embedding of the new ``hist[pos]`` in the plain step's input rows."""
        B, T = self.B, k + 1
        b = self._buffers(B, T)
        b1 = self._buffers(B, 1)
        ops.spec_draft(self.hist_buf, self.pos_buf, k, CONFIG["spec_n"], out=b["tok"])
        nxt = self._step(T, tok=b["tok"])
        ops.spec_accept(nxt, b["tok"], self.hist_buf, self.pos_buf, self.s_buf, self.ntarget_buf, self.embed,
                        b1["h"], b1["psq"], b["out_t"], b["adv"])
        return b["out_t"], b["adv"]

    def verify_step(self, tok: torch.Tensor, positions) -> torch.Tensor:
        """Greedy next token at every position of ``tok [B, T]`` (the speculative verify forward
        of ``engine/engine.py:979-993``): token ``t`` of row ``b`` sits at ``positions[b] + t``;
        K/V are written for those slots. Returns ``[B, T]`` int64 (host sync)."""
        B, T = tok.shape
        assert B == self.B and B * T <= 32 and T <= 16, "verify needs the prepared batch, B*T <= 32, T <= 16"
        with torch.inference_mode():
            pos = torch.as_tensor(positions, dtype=torch.int32).reshape(B)
            self.pos_buf.copy_(pos.to(self.device))
            out = self._step(T, tok=tok.to(self.device, torch.int64).contiguous()).view(B, T).clone()
        return out

    def step_hidden(self, tok: torch.Tensor, positions) -> list:
        """One eager decode step of ``tok [B, 1]`` at ``positions``; returns the residual stream
        after every layer (for per-layer parity checks)."""
        hidden = []
        with torch.inference_mode():
            self.pos_buf.copy_(torch.as_tensor(positions, dtype=torch.int32).reshape(-1).to(self.device))
            self._step(1, tok=tok.to(self.device, torch.int64).contiguous(), hidden=hidden)
        return [h.clone() for h in hidden]

    @torch.inference_mode()
    def _capture(self, T):
        """Record one decode step into a HIP graph (``engine/engine.py:1005-1042``): the plain step
        (T = 1) or the speculative verify step (T = k + 1).

        Always under inference mode: the first capture in a process creates the generator state
        that later captures update in place, so every capture must run in the same mode (the
        engine's own callers capture inside ``generate``)."""
        k = T - 1
        run = self._plain_step if k == 0 else (lambda: self._spec_step(k))
        pos_saved = self.pos_buf.clone()
        hist_saved = self.hist_buf.clone()
        s_saved, n_saved = self.s_buf.clone(), self.ntarget_buf.clone()
        self.s_buf.zero_()
        self.ntarget_buf.fill_(1 << 40)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            self.pos_buf.fill_(1)
            run()                           # warm-up (allocates nothing new)
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        self.pos_buf.fill_(1)
        with torch.cuda.graph(graph):
            out = run()
        torch.cuda.synchronize()
        self.graphs[T] = (graph, out)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        start.record()
        for _ in range(reps):
            self.pos_buf.fill_(1)
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        self.step_ms[T] = start.elapsed_time(end) / reps
        # Capture wrote K/V at slots 1..T and hist[:, 2..T+1]: the prompt forward and the
        # first decode steps overwrite those slots before anything reads them.
        self.pos_buf.copy_(pos_saved)
        self.hist_buf.copy_(hist_saved)
        self.s_buf.copy_(s_saved)
        self.ntarget_buf.copy_(n_saved)
        torch.cuda.synchronize()
        _log(f"captured T={T} graph; replay {self.step_ms[T]:.3f} ms/step")

    # ------------------------------------------------------------------ prompt forward
    def _prefill_attention(self, q, kc, vc, S):
        """Causal attention of the prompt: q ``[Bs, S, Nq, D]``, cache views -> ``[Bs*S, Nq*D]``.

        Uses torch SDPA restricted to its flash / memory-efficient kernels; if
        neither accepts the shape, the decode-attention kernel runs over
        16-token chunks of the prompt (same causal rule).
        """
        Bs = q.shape[0]
        from torch.nn.attention import SDPBackend, sdpa_kernel
        if self.sdpa_mode != "chunked":
            try:
                qt = q.transpose(1, 2)
                rep = self.Nq // self.Nkv
                k = kc[:, :, :S]
                v = vc[:, :, :S]
                with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                    if self.sdpa_mode in (None, "gqa"):
                        try:
                            out = F.scaled_dot_product_attention(qt, k, v, is_causal=True, scale=self.scale,
                                                                 enable_gqa=True)
                            self.sdpa_mode = "gqa"
                            return out.transpose(1, 2).reshape(Bs * S, self.Nq * self.D)
                        except RuntimeError:
                            self.sdpa_mode = "expand"
                    ke = k[:, :, None].expand(Bs, self.Nkv, rep, S, self.D).reshape(Bs, self.Nq, S, self.D)
                    ve = v[:, :, None].expand(Bs, self.Nkv, rep, S, self.D).reshape(Bs, self.Nq, S, self.D)
                    out = F.scaled_dot_product_attention(qt, ke, ve, is_causal=True, scale=self.scale)
                    return out.transpose(1, 2).reshape(Bs * S, self.Nq * self.D)
            except RuntimeError as error:
                _log(f"SDPA flash/efficient unavailable ({error!r}); chunked decode-attention kernel")
                self.sdpa_mode = "chunked"
        out = torch.empty((Bs, S, self.Nq * self.D), dtype=BF16, device=self.device)
        lengths = torch.empty((Bs,), dtype=torch.int32, device=self.device)
        for t0 in range(0, S, 16):
            T = min(16, S - t0)
            lengths.fill_(t0 + T)
            splits = ops.choose_num_splits(Bs, self.Nkv, t0 + T)
            out[:, t0:t0 + T] = ops.attn_decode(q[:, t0:t0 + T].contiguous(), kc, vc, lengths, self.scale, splits)
        return out.reshape(Bs * S, self.Nq * self.D)

    def _prefill(self, ids):
        """Prompt forward (``engine/engine.py:1181-1189``): batch slices of at most prefill_rows rows."""
        B, S = ids.shape
        rows_per = max(1, CONFIG["prefill_rows"] // S)
        firsts = []
        for b0 in range(0, B, rows_per):
            b1 = min(B, b0 + rows_per)
            firsts.append(self._prefill_slice(ids[b0:b1], b0))
        return firsts[0] if len(firsts) == 1 else torch.cat(firsts)

    def _prefill_slice(self, ids, b0, hidden=None):
        """``_prefill_slice`` (``engine/engine.py:1191-1221``) for rows ``b0 .. b0 + Bs``."""
        Bs, S = ids.shape
        b1 = b0 + Bs
        pos = torch.zeros((Bs,), dtype=torch.int32, device=self.device)
        h = ops.embed(ids.reshape(-1).contiguous(), self.embed)
        d = None
        for l, w in enumerate(self.layers):
            kc = self.k_cache[l][b0:b1]
            vc = self.v_cache[l][b0:b1]
            if d is None:
                n = ops.rms_norm(h, w.ln1, self.eps)
            else:
                h, n = ops.add_rms_norm(h, d, w.ln1, self.eps)
            qkv = F.linear(n, w.r_qkv)
            q = ops.qk_norm_rope_cache(qkv, w.q_norm, w.k_norm, self.eps, self.cos_tab, self.sin_tab, pos, S, kc, vc)
            a = self._prefill_attention(q, kc, vc, S)
            o = F.linear(a, w.r_o)
            h, n = ops.add_rms_norm(h, o, w.ln2, self.eps)
            d = F.linear(ops.silu_mul(F.linear(n, w.r_gu)), w.r_down)
            if hidden is not None:
                hidden.append(ops.add_rms_norm(h, d, w.ln1, self.eps)[0])
        last = torch.arange(Bs, device=self.device) * S + (S - 1)
        hl, _ = ops.add_rms_norm(h.index_select(0, last), d.index_select(0, last), self.final_norm, self.eps)
        firsts = []
        for r0 in range(0, Bs, 32):
            firsts.append(ops.lm_head_argmax(hl[r0:r0 + 32].contiguous(), self.final_norm, self.eps, self.embed))
        return firsts[0] if len(firsts) == 1 else torch.cat(firsts)

    # ------------------------------------------------------------------ generate
    def generate(self, input_ids: list[list[int]], max_new_tokens: int):
        """Greedy continuation of every sequence, one step at a time (``engine/engine.py:1225-1250``).

        Yields a list with one token id per sequence for each output step,
        exactly ``max_new_tokens`` times. Never stops at end-of-sequence tokens.
        """
        B, S = len(input_ids), len(input_ids[0])
        N = int(max_new_tokens)
        if N <= 0:
            return
        if any(len(row) != S for row in input_ids):
            raise ValueError("all prompts must have the same length")
        with torch.inference_mode():
            first = self.start(input_ids, N)
            yield from self._decode_loop(first, B, N)

    def start(self, input_ids: list[list[int]], max_new_tokens: int) -> torch.Tensor:
        """The part of ``generate`` before the first yield (``engine/engine.py:1225-1248``): per-shape
        state, prompt forward, history and positions, the first decode step's input row. Returns the
        first token of every sequence (``[B]`` int64 on the device)."""
        B, S, N = len(input_ids), len(input_ids[0]), int(max_new_tokens)
        ids_cpu = torch.tensor(input_ids, dtype=torch.int64)
        if ids_cpu.numel() and (int(ids_cpu.min()) < 0 or int(ids_cpu.max()) >= self.V):
            raise ValueError(f"token ids must lie in [0, {self.V})")
        with torch.inference_mode():
            self._prepare(B, S, N)
            ids = ids_cpu.to(self.device)
            first = self._prefill(ids)
            self.hist_buf[:, :S].copy_(ids)
            self.hist_buf[:, S].copy_(first)
            self.pos_buf.fill_(S)
            self.s_buf.fill_(S)
            self.ntarget_buf.fill_(N)
            self._prime()
        return first

    def _decode_loop(self, first, B, N):
        """Pipelined graph replays with async D2H copies into a pinned ring (``engine/engine.py:1254-1378``).

        At most ``pipeline_depth + 1`` steps are in flight, and no step is launched that could
        not contribute a token (``:1332-1336``). With speculation on, the loop alternates between
        verify steps and plain steps: it speculates while the accepted tokens per verify step
        (moving average of the slowest unfinished row) times the plain step time beat the verify
        step time, and otherwise runs plain steps, probing speculation again every so often
        (``:1319-1372``).
        """
        depth = CONFIG["pipeline_depth"]
        ring = len(self.pin_nxt)
        stream = torch.cuda.current_stream()
        k = self.k_active
        T = k + 1
        graphs = self.graphs

        def launch(slot, mode):
            if mode == "first":
                self.pin_nxt[slot][0].copy_(first, non_blocking=True)
            elif mode == "plain":
                if 1 in graphs:
                    graphs[1][0].replay()
                    out = graphs[1][1]
                else:
                    out = self._plain_step()
                self.decode_launches += 1
                self.pin_nxt[slot][0].copy_(out, non_blocking=True)
            else:
                if T in graphs:
                    graphs[T][0].replay()
                    out_t, adv = graphs[T][1]
                else:
                    out_t, adv = self._spec_step(k)
                self.decode_launches += 1
                self.spec_launches += 1
                self.pin_nxt[slot].copy_(out_t, non_blocking=True)
                self.pin_adv[slot].copy_(adv, non_blocking=True)
            self.events[slot].record(stream)

        t1 = self.step_ms.get(1, 1.0)
        tk = self.step_ms.get(T, 1.0) if k else float("inf")
        mode = "spec" if k else "plain"
        rate = tk / t1 + 0.25 if k else 0.0       # optimistic start: speculate first
        plain_left = probe_left = 0
        probe_plain, probe_spec = CONFIG["spec_probe"]
        losing = lambda: rate * t1 < tk * 1.03   # noqa: E731

        queues = [deque() for _ in range(B)]
        produced = [0] * B
        inflight = deque()
        launch(0, "first")
        inflight.append((0, "first"))
        launched = 1
        potential = 1      # upper bound on the tokens per sequence the in-flight steps can still bring
        yielded = 0
        while yielded < N:
            while len(inflight) <= depth and min(produced) + potential < N:
                slot = launched % ring
                launched += 1
                if k:
                    if mode == "plain":
                        plain_left -= 1
                        if plain_left <= 0:
                            mode, probe_left = "spec", probe_spec
                    elif probe_left > 0:
                        probe_left -= 1
                        if probe_left == 0 and losing():
                            mode, plain_left = "plain", probe_plain
                m = mode
                if m == "spec" and N - min(produced) - potential <= 1:
                    m = "plain"    # one token left: the cheap step wins
                launch(slot, m)
                inflight.append((slot, m))
                potential += T if m == "spec" else 1
            slot, m = inflight.popleft()
            potential -= T if m == "spec" else 1
            self.events[slot].synchronize()
            if m == "spec":
                rows = self.pin_nxt[slot].tolist()          # rows[j][b]
                adv = self.pin_adv[slot].tolist()
                gains = []
                for b in range(B):
                    a = int(adv[b])
                    queues[b].extend(int(rows[j][b]) for j in range(a))
                    produced[b] += a
                    if produced[b] < N:
                        gains.append(a)
                if gains:
                    rate = 0.75 * rate + 0.25 * min(gains)
                    self.spec_tokens += min(gains)
                    if probe_left == 0 and mode == "spec" and losing():
                        mode, plain_left = "plain", probe_plain
            else:
                for b, t in enumerate(self.pin_nxt[slot][0].tolist()):
                    queues[b].append(int(t))
                    produced[b] += 1
            while yielded < N and all(queues):
                yield [q.popleft() for q in queues]
                yielded += 1
