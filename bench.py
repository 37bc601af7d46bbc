"""Decode throughput of the MI355X Qwen3-4B engine (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config default|c2|c3|c4|c5]

BASELINE.json's metric is "decode tok/s at B=1 and B=32 (Qwen3-4B bf16); HBM GB/s as % of peak".
The default run measures both halves in one invocation on random-init Qwen3-4B bf16 weights
(seed 0), greedy decoding through the engine's own ``generate()``:

* ``value`` (B = 1, configs[1] "c2": a 128-token uniform-random prompt, 256 decode steps);
* ``b32`` (B = 32, configs[3] "c4": 8192-token prompts, 256 decode steps, ~37 GiB of KV cache);
* ``c3`` (B = 8, configs[2]) and ``c5`` (the speculative verify step, configs[4]) as further
  blocks of the same line, so that every decode config is timed in the default run.

Each is timed as follows. The batch state is built, certified and its step graph recorded
first (untimed); the prompt forward gives ``ttft_s``; ``W`` warm-up steps run; then exactly
``K`` decode steps of the same ``generate()`` are timed with HIP events on the launch stream
(before the first timed launch, after the last), so ``value`` = B x K tokens / those seconds;
the generation then runs to the config's length untimed. The c5 block of the default run
replays at least its 200 verify steps. The default run times c2, c3 and c5 before c4: right
after c4's 37 GiB batch state is freed, the next batch state measured up to 5 % slower in the
same process (c5 292 against 307.5 verify steps/s; 307.9 again once another state had been
built and freed), while each config run in a process of its own matches its figure here.
Weights and KV cache are resident in HBM; only token ids cross PCIe (8 bytes per sequence per
step).

``roofline`` is for the dominant kernel of the workload, timed live with HIP events on the
stream it runs on: at B = 1 the fused RMSNorm + gate/up GEMV + SwiGLU (44 % of a step's bytes),
rotating over the 36 layers' weights so nothing is served from the 256 MB Infinity Cache; at
B = 32 the decode attention (its KV stream is 83 % of the bytes), over the 36 layers' caches.
``step_roofline``: algorithmic bytes of a whole step (weights + visible KV) over the measured
step time. ``b32.mfma``: MFMA utilisation of the four projections at M = 32 (2 M N K flops per
launch over the measured launch time, against the 2.5 PFLOP/s bf16 dense peak); they are
HBM-bound, so this is a secondary figure. ``cpu_baseline``: the oracle's torch-CPU decode step
over all 36 layers on this host's cores, median of 3 runs (a bounded sample of the c2 decode).

``--config c3|c4`` run one decode config (``roofline``: gate/up at c3, attention at c4, each
that step's largest kernel); ``--config c5`` replays the speculative verify graph
(B = 4, T = 5, context 4096) and reports verify steps/s. ``--profile-sample`` runs only the
dominant kernel (and a copy of known size) for rocprofv3 counter runs.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "thing-htn-2026_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12        # MI355X HBM3E, bytes/s
MFMA_BF16_PEAK = 2.5e15  # MI355X dense bf16 matrix peak, flop/s
CONFIGS = {
    # name: (B, prompt length, decode steps), BASELINE.json configs[1..4]
    "c2": (1, 128, 256),
    "c3": (8, 2048, 512),
    "c4": (32, 8192, 256),
    "c5": (4, 4096, 200),     # speculative verify steps, T = SPEC_T tokens per sequence
}
SPEC_T = 5                    # c5: 1 accepted + 4 draft tokens per verify step
QWEN3_4B = {
    "hidden_size": 2560, "intermediate_size": 9728, "vocab_size": 151936,
    "num_hidden_layers": 36, "num_attention_heads": 32, "num_key_value_heads": 8,
    "head_dim": 128, "rms_norm_eps": 1e-6, "rope_theta": 5000000.0, "rope_scaling": None,
    "tie_word_embeddings": True,
}
DATA = ("synthetic: random-init bf16 weights (counter-based generator, seed 0, std 0.02), "
        "uniform-random prompt ids (torch seed 1)")
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def weight_bytes(cfg) -> int:
    H, I, D, Nq, Nkv, L, V = (cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"],
                              cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["num_hidden_layers"],
                              cfg["vocab_size"])
    per_layer = 2 * (H * (Nq + 2 * Nkv) * D + Nq * D * H + 2 * I * H + I * H)
    norms = 2 * (L * (2 * H + 2 * D) + H)
    return L * per_layer + 2 * V * H + norms


def kv_bytes_per_token(cfg) -> int:
    return cfg["num_hidden_layers"] * 2 * cfg["num_key_value_heads"] * cfg["head_dim"] * 2


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--config", default="default", choices=["default"] + sorted(CONFIGS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--profile-sample", action="store_true",
                   help="run only the dominant kernel of --config (c2: gate/up GEMV, c4: attention) and a plain "
                        "1 GiB device copy, for rocprofv3 --pmc traffic runs; prints one JSON line")
    p.add_argument("--profile-kernel", default="dominant", choices=["dominant", "o", "qkv", "down"],
                   help="with --profile-sample: the dominant kernel, or the O, QKV or down projection")
    return p.parse_args()


def measured_traffic(config: str, kernel: str, nbytes: int | None = None):
    """HBM bytes per launch of ``kernel`` at ``config`` from the committed PMC summary
    (``FETCH_SIZE`` + ``WRITE_SIZE`` scaled by a copy of known size), or None. An entry measured at
    another size (the attention's context grows during decoding) carries its algorithmic bytes, and
    its traffic-to-algorithmic ratio is applied to ``nbytes``."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    entry = rec.get(config)
    if entry is None or entry.get("kernel") != kernel:
        return None
    if nbytes is not None and entry.get("algorithmic_bytes"):
        return int(round(entry["bytes_per_launch"] / entry["algorithmic_bytes"] * nbytes))
    return entry.get("bytes_per_launch")


def _events_time(torch, run, n_outer, stream):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    n = 0
    for _ in range(n_outer):
        n += run()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / n


def time_gate_up(eng, torch, reps=3, T=1):
    """Average launch time of the fused RMSNorm + gate/up + SwiGLU projection at M = B * T, rotating
    over the 36 layers' weights (3.6 GB). Returns (seconds, algorithmic bytes, kernel name)."""
    from qwen_hip import ops
    b = eng.bufs(eng.state.groups[0], T)
    ops.sumsq16(b.h, out=b.psq)

    def one(w):
        if b.gemv:
            ops.gemv(b.h, w.gu_rows, norm_w=w.ln2, eps=eng.eps, silu_pair=True, out=b.p, cfg=b.gemv_cfg["gu"])
        else:
            ops.fused_linear(b.h, w.gu, b.cfg["gu"], norm_w=w.ln2, eps=eng.eps, silu_pair=True, out=b.p,
                             psq_in=b.psq, workspace=b.gemm_ws)

    def sweep():
        for w in eng.w.layers:
            one(w)
        return len(eng.w.layers)

    sweep()
    torch.cuda.synchronize()
    avg = _events_time(torch, sweep, reps, torch.cuda.current_stream())
    w0 = eng.w.layers[0].gu
    M = b.M
    nbytes = w0.nbytes + M * w0.K * 2 + w0.K * 2 + M * (w0.N // 2) * 2
    name = ("gemv_kernel<%d, %d, true, 2>" % (M, b.gemv_cfg["gu"][1]) if b.gemv
            else ops.gemm_kernel_name(M, b.cfg["gu"], True, ops.EPI_SWIGLU))
    return avg, nbytes, name


def time_qkv(eng, torch, reps=3, T=1):
    """Average launch time of the fused RMSNorm + QKV projection at M = B * T, rotating over the 36
    layers' weights. Returns (seconds, algorithmic bytes, kernel name)."""
    from qwen_hip import ops
    b = eng.bufs(eng.state.groups[0], T)
    ops.sumsq16(b.h, out=b.psq)

    def one(w):
        if b.gemv:
            ops.gemv(b.h, w.qkv_rows, norm_w=w.ln1, eps=eng.eps, out=b.qkv, cfg=b.gemv_cfg["qkv"],
                     row_map=eng.w.qkv_map)
        else:
            ops.fused_linear(b.h, w.qkv, b.cfg["qkv"], norm_w=w.ln1, eps=eng.eps, out=b.qkv, psq_in=b.psq,
                             workspace=b.gemm_ws)

    def sweep():
        for w in eng.w.layers:
            one(w)
        return len(eng.w.layers)

    sweep()
    torch.cuda.synchronize()
    avg = _events_time(torch, sweep, reps, torch.cuda.current_stream())
    w0 = eng.w.layers[0].qkv
    M = b.M
    nbytes = w0.nbytes + M * w0.K * 2 + w0.K * 2 + M * w0.N * 2
    name = ("gemv_kernel<%d, %d, true, 0>" % (M, b.gemv_cfg["qkv"][1]) if b.gemv
            else ops.gemm_kernel_name(M, b.cfg["qkv"], True, ops.EPI_STORE))
    return avg, nbytes, name


def time_o_proj(eng, torch, reps=3, T=1):
    """Average launch time of the O projection + residual (M = B * T rows, K = 4096), rotating over the
    36 layers' weights. Returns (seconds, algorithmic bytes, kernel name)."""
    from qwen_hip import ops
    b = eng.bufs(eng.state.groups[0], T)
    a = b.a.view(b.M, -1)
    h2 = b.h.clone()

    def one(w):
        if b.gemv:
            ops.gemv(a, w.o_rows, residual=h2, out=h2, cfg=b.gemv_cfg["o"])
        else:
            ops.fused_linear(a, w.o, b.cfg["o"], residual=h2, out=h2, workspace=b.gemm_ws)

    def sweep():
        for w in eng.w.layers:
            one(w)
        return len(eng.w.layers)

    sweep()
    torch.cuda.synchronize()
    avg = _events_time(torch, sweep, reps, torch.cuda.current_stream())
    w0 = eng.w.layers[0].o
    M = b.M
    nbytes = w0.nbytes + M * w0.K * 2 + 2 * M * w0.N * 2
    name = ("gemv_kernel<%d, %d, false, 1>" % (M, b.gemv_cfg["o"][1]) if b.gemv
            else ops.gemm_kernel_name(M, b.cfg["o"], False, ops.EPI_RES))
    return avg, nbytes, name


def time_down(eng, torch, reps=3, T=1):
    """Average launch time of the down projection + residual (M = B * T rows, K = 9728), rotating
    over the 36 layers' weights. Returns (seconds, algorithmic bytes, kernel name)."""
    from qwen_hip import ops
    b = eng.bufs(eng.state.groups[0], T)
    h2 = b.h.clone()

    def one(w):
        if b.gemv:
            ops.gemv(b.p, w.down_rows, residual=h2, out=h2, cfg=b.gemv_cfg["down"])
        else:
            ops.fused_linear(b.p, w.down, b.cfg["down"], residual=h2, out=h2, workspace=b.gemm_ws)

    def sweep():
        for w in eng.w.layers:
            one(w)
        return len(eng.w.layers)

    sweep()
    torch.cuda.synchronize()
    avg = _events_time(torch, sweep, reps, torch.cuda.current_stream())
    w0 = eng.w.layers[0].down
    M = b.M
    nbytes = w0.nbytes + M * w0.K * 2 + 2 * M * w0.N * 2
    name = ("gemv_kernel<%d, %d, false, 1>" % (M, b.gemv_cfg["down"][1]) if b.gemv
            else ops.gemm_kernel_name(M, b.cfg["down"], False, ops.EPI_RES))
    return avg, nbytes, name


def time_attention(eng, torch, reps=2):
    """Average launch time of the decode attention (QK-norm + RoPE + KV write + attention + merge)
    over the 36 layers' caches at the batch's current positions. Algorithmic bytes: the visible
    K and V rows (B x ctx x Nkv x D x 2 x 2 B) plus the q/k/v rows read and the output written."""
    from qwen_hip import ops
    st = eng.state
    g = st.groups[0]
    b = eng.bufs(g, 1)
    s = eng.spec
    ctx = [int(v) + 1 for v in st.pos.tolist()]

    def sweep():
        for l, w in enumerate(eng.w.layers):
            kc, vc = g.kv[l]
            ops.attn_decode_mfma(b.qkv, w.q_norm, w.k_norm, s.eps, eng.cos_tab, eng.sin_tab, g.pos, 1, kc, vc,
                                 eng.scale, b.splits, out=b.a, workspace=b.attn_ws, waves=b.attn_waves,
                                 kv_cached=st.kv_cached)
        return len(eng.w.layers)

    sweep()
    torch.cuda.synchronize()
    avg = _events_time(torch, sweep, reps, torch.cuda.current_stream())
    nbytes = sum(c * s.Nkv * s.D * 2 * 2 for c in ctx) + b.M * (s.qkv_width + s.Nq * s.D) * 2
    name = f"attn_mfma_kernel<1, {b.attn_waves}, {'true' if st.kv_cached else 'false'}>"
    return avg, nbytes, name


def mfma_utilisation(eng, torch, reps=2):
    """Flops over time of the four projections at the batch's M (MFMA kernels), rotating over layers."""
    from qwen_hip import ops
    b = eng.bufs(eng.state.groups[0], 1)
    s = eng.spec
    M = b.M
    ops.sumsq16(b.h, out=b.psq)
    a = b.a.view(M, -1)
    h2 = b.h.clone()
    kinds = {
        "qkv": (lambda w: ops.fused_linear(b.h, w.qkv, b.cfg["qkv"], norm_w=w.ln1, eps=s.eps, out=b.qkv,
                                           psq_in=b.psq, workspace=b.gemm_ws), s.qkv_width, s.H),
        "o": (lambda w: ops.fused_linear(a, w.o, b.cfg["o"], residual=h2, out=h2, workspace=b.gemm_ws),
              s.H, s.Nq * s.D),
        "gate_up": (lambda w: ops.fused_linear(b.h, w.gu, b.cfg["gu"], norm_w=w.ln2, eps=s.eps, silu_pair=True,
                                               out=b.p, psq_in=b.psq, workspace=b.gemm_ws), 2 * s.I, s.H),
        "down": (lambda w: ops.fused_linear(b.p, w.down, b.cfg["down"], residual=h2, out=h2,
                                            workspace=b.gemm_ws), s.H, s.I),
    }
    out = {}
    total_flops = total_s = 0.0
    for name, (fn, N, K) in kinds.items():
        def sweep(fn=fn):
            for w in eng.w.layers:
                fn(w)
            return len(eng.w.layers)
        sweep()
        torch.cuda.synchronize()
        avg = _events_time(torch, sweep, reps, torch.cuda.current_stream())
        flops = 2.0 * M * N * K
        out[name] = {"avg_us": round(avg * 1e6, 2), "tflops": round(flops / avg / 1e12, 1),
                     "frac": round(flops / avg / MFMA_BF16_PEAK, 4),
                     "hbm_frac": round(N * K * 2 / avg / HBM_PEAK, 4)}
        total_flops += flops
        total_s += avg
    out["all"] = {"tflops": round(total_flops / total_s / 1e12, 1),
                  "frac": round(total_flops / total_s / MFMA_BF16_PEAK, 4),
                  "peak_tflops": MFMA_BF16_PEAK / 1e12, "M": M}
    return out


def run_decode(eng, torch, cfg, B, S, N, K, W):
    """One greedy generate() of the config's N tokens (more if 1 + W + K asks for more) for B prompts
    of S tokens; the W decode steps after the first token are untimed, the next K are timed with HIP
    events recorded on the launch stream just before the (W + 1)-th step launch and just after the
    (W + K)-th (exactly K steps of device time, the token pump's read-back included); the rest of
    the generation runs untimed. ``decode_wall_tok_s``: all decode steps over host wall time."""
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g).tolist()
    total = max(N, 1 + W + K)
    with torch.inference_mode():
        eng.prepare(B, S, total)          # batch state, certification, step graph: untimed
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    launched = [0]
    plain = eng._plain

    def timed_plain():
        launched[0] += 1
        if launched[0] == W + 1:
            ev0.record(stream)
        out = plain()
        if launched[0] == W + K:
            ev1.record(stream)
        return out

    eng._plain = timed_plain               # the token pump calls it once per decode step
    try:
        gen = eng.generate(prompt, total)
        t_pf = time.perf_counter()
        next(gen)                          # prompt forward + first token
        ttft = time.perf_counter() - t_pf
        t0 = time.perf_counter()
        for _ in gen:
            pass
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    finally:
        del eng._plain
    if launched[0] < W + K:
        sys.exit(f"bench.py: only {launched[0]} decode steps were launched (warm-up {W} + timed {K})")
    dt = ev0.elapsed_time(ev1) / 1e3
    ms_step = dt / K * 1e3
    ctx_mid = S + 1 + W + K / 2
    step_bytes = weight_bytes(cfg) + B * ctx_mid * kv_bytes_per_token(cfg)
    return {
        "value": round(K * B / dt, 2), "steps": K, "ms_per_step": round(ms_step, 4), "ttft_s": round(ttft, 3),
        "decode_wall_tok_s": round(launched[0] * B / wall, 2),
        "step_roofline": {"bytes_per_step": int(step_bytes),
                          "achieved_GBps": round(step_bytes / (ms_step / 1e3) / 1e9, 1),
                          "frac": round(step_bytes / (ms_step / 1e3) / HBM_PEAK, 4)},
    }


def roofline(avg, nbytes, name, config, what):
    achieved = nbytes / avg
    return {"bound": "hbm", "kernel": f"{name}: {what}", "achieved": round(achieved / 1e9, 1),
            "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
            "traffic": measured_traffic(config, name, int(nbytes)), "avg_us": round(avg * 1e6, 2),
            "bytes_per_launch": int(nbytes)}


def bench_verify(eng, torch, cfg, B, S, K, W):
    """c5: K speculative verify steps (T = SPEC_T tokens per sequence: the last accepted token and
    SPEC_T - 1 prompt-lookup drafts, which on a uniform-random prompt are effectively random ids),
    each one replay of the recorded verify graph (draft, 36 layers over B*T rows with causal
    multi-query attention, argmax per position, acceptance). ``value`` = verify steps per second."""
    T = SPEC_T
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g).tolist()
    eng.start(prompt, T * (K + W) + 8)
    assert eng.k_active == T - 1 and T in eng.state.graphs, "verify graph not recorded"
    graph = eng.state.graphs[T]
    for _ in range(W):
        graph.launch()
    torch.cuda.synchronize()
    pos0 = int(eng.state.pos[0])
    t0 = time.perf_counter()
    for _ in range(K):
        graph.launch()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ctx_mid = (pos0 + int(eng.state.pos[0])) / 2 + T
    step_bytes = weight_bytes(cfg) + B * ctx_mid * kv_bytes_per_token(cfg)
    avg, nbytes, name = time_gate_up(eng, torch, T=T)
    return {
        "metric": f"spec-verify steps/s at B={B}, T={T}, context {S} (Qwen3-4B bf16)",
        "value": round(K / dt, 2), "unit": "verify steps/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(dt / K * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": DATA + "; drafts by prompt lookup (no repeats: effectively random ids)",
        "config": {"workload": f"c5: Qwen3-4B, B={B}, context {S}, T={T} verify steps",
                   "global_batch": B, "seq_len": S, "verify_tokens": T, "parallelism": "single GPU"},
        "positions_per_s": round(K * B * T / dt, 1),
        "roofline": roofline(avg, nbytes, name, "c5", "RMSNorm + gate/up + SwiGLU (one layer)"),
        "step_roofline": {"bytes_per_step": int(step_bytes),
                          "achieved_GBps": round(step_bytes * K / dt / 1e9, 1),
                          "frac": round(step_bytes * K / dt / HBM_PEAK, 4)},
    }


def cpu_baseline(eng, cfg, S, runs=3, target_s=6.0):
    """The oracle's torch-CPU decode step (oracle/model.py, all 36 layers + LM head) on this host's
    cores, B = 1 at context ~S: median over ``runs`` runs of about ``target_s`` seconds each."""
    import torch
    from oracle.model import CpuQwen3
    w = eng.w
    layers = [{"ln1": lw.ln1.cpu(), "ln2": lw.ln2.cpu(), "q_norm": lw.q_norm.cpu(), "k_norm": lw.k_norm.cpu(),
               "w_qkv": w.natural_qkv_rows(lw).cpu(), "w_o": lw.o_rows.cpu(), "w_gu": lw.gu_rows.cpu(),
               "w_down": lw.down_rows.cpu()} for lw in w.layers]
    ref = CpuQwen3(cfg, {"embed": w.lm_rows.cpu(), "final_norm": w.final_norm.cpu(), "layers": layers})
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, cfg["vocab_size"], (1, S), generator=g)
    rates = []
    with torch.inference_mode():
        ref.prepare(1, ((S + 256 + 63) // 64) * 64)
        # the S context slots hold seeded random K/V in place of the prompt forward (a decode
        # step's work does not depend on the cached values)
        for kc, vc in zip(ref.k_cache, ref.v_cache):
            kc[:, :, :S].copy_(torch.randn(kc[:, :, :S].shape, generator=g).to(kc.dtype))
            vc[:, :, :S].copy_(torch.randn(vc[:, :, :S].shape, generator=g).to(vc.dtype))
        ref.hist[:, :S] = ids
        ref.pos.fill_(S - 1)
        t0 = time.perf_counter()
        ref.plain_step()                   # warm-up, and the per-step estimate
        per = time.perf_counter() - t0
        n = max(2, min(60, int(target_s / max(per, 1e-3))))
        for _ in range(runs):
            ref.pos.fill_(S - 1)
            t0 = time.perf_counter()
            for _ in range(n):
                ref.plain_step()
            rates.append(n / (time.perf_counter() - t0))
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(statistics.median(rates), 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "runs": [round(r, 3) for r in rates],
            "sample": (f"oracle torch-CPU decode step (oracle/model.py), all {cfg['num_hidden_layers']} layers + LM "
                       f"head, B=1 at context {S}..{S + n} (random cached K/V), {n} steps per run, median of "
                       f"{runs} runs; host CPU {cpu}")}


def profile_sample(eng, torch, config, kernel="dominant"):
    """Dominant-kernel (or ``kernel="o"`` / ``"qkv"`` / ``"down"``: that projection) launches at the config's
    step width, plus a copy of known size (the FETCH_SIZE / WRITE_SIZE calibration)."""
    T = SPEC_T if config == "c5" else 1
    if kernel == "o":
        avg, nbytes, name = time_o_proj(eng, torch, reps=1, T=T)
    elif kernel == "down":
        avg, nbytes, name = time_down(eng, torch, reps=1, T=T)
    elif kernel == "qkv":
        avg, nbytes, name = time_qkv(eng, torch, reps=1, T=T)
    elif config == "c4":
        avg, nbytes, name = time_attention(eng, torch, reps=1)
    else:
        avg, nbytes, name = time_gate_up(eng, torch, reps=1, T=SPEC_T if config == "c5" else 1)
    n = 1 << 29                                # 2^29 bf16 = 1 GiB read + 1 GiB written per copy
    src = torch.ones(n, dtype=torch.bfloat16, device=eng.device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"kernel": name, "avg_us": round(avg * 1e6, 2), "bytes_per_launch": nbytes,
            "copy_bytes_each_way": 2 * n, "copies": 3}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box in this build has a single MI355X; sequences "
              f"would shard data-parallel over GPUs, with no exchange while decoding); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import engine as engine_mod
    from __graft_entry__ import write_random_model
    from engine import Engine

    cfg = QWEN3_4B
    W = args.warmup
    if args.config == "c5":
        engine_mod.CONFIG["spec_k"] = SPEC_T - 1
    with tempfile.TemporaryDirectory() as d:
        eng = Engine(write_random_model(d, cfg, seed=0, std=0.02))

    if args.profile_sample:
        name = "c2" if args.config == "default" else args.config
        B, S, N = CONFIGS[name]
        engine_mod.CONFIG["certify"] = False
        if name == "c4":
            eng.start(torch.randint(0, cfg["vocab_size"], (B, S)).tolist(), 8)
        else:
            with torch.inference_mode():
                eng.prepare(B, S, N + W + 1)
        print(json.dumps(profile_sample(eng, torch, name, args.profile_kernel)), flush=True)
        return
    if args.config == "c5":
        B, S, N = CONFIGS["c5"]
        K = args.steps if args.steps is not None else N
        print(json.dumps(bench_verify(eng, torch, cfg, B, S, K, W)), flush=True)
        return

    first = "c2" if args.config == "default" else args.config
    B, S, N = CONFIGS[first]
    K = args.steps if args.steps is not None else N - 1 - W
    res = run_decode(eng, torch, cfg, B, S, N, K, W)
    if first == "c4":  # the KV-bound step: attention is 68 % of its kernel time
        avg, nbytes, name = time_attention(eng, torch)
        what = "QK-norm + RoPE + KV write + GQA attention (one layer)"
    else:
        avg, nbytes, name = time_gate_up(eng, torch)
        what = "RMSNorm + gate/up + SwiGLU (one layer)"
    out = {
        "metric": ("decode tok/s at B=1 and B=32 (Qwen3-4B bf16); HBM GB/s as % of peak" if args.config == "default"
                   else f"decode tok/s at B={B} (Qwen3-4B bf16)"),
        "value": res["value"], "unit": "tok/s", "n_gpus": 1, "steps": res["steps"], "warmup": W,
        "ms_per_step": res["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": DATA,
        "config": {"workload": f"{first}: Qwen3-4B, B={B}, prompt {S}, {N} greedy decode steps",
                   "global_batch": B, "seq_len": S, "decode_steps": N, "parallelism": "single GPU"},
        "roofline": roofline(avg, nbytes, name, first, what),
        "step_roofline": res["step_roofline"],
        "ttft_s": res["ttft_s"],
        "decode_wall_tok_s": res["decode_wall_tok_s"],
        "steps_note": ("exactly `steps` decode steps of one generate() are timed (HIP events around their "
                       "launches, after `warmup` untimed steps); the rest of the generation is untimed"),
    }
    if args.config == "default":
        # c3 and c5 first, then c4 (see the module docstring: a batch state built right after
        # c4's is freed runs slower in the same process).
        B3, S3, N3 = CONFIGS["c3"]
        K3 = args.steps if args.steps is not None else N3 - 1 - W
        r3 = run_decode(eng, torch, cfg, B3, S3, N3, K3, W)
        out["c3"] = {
            "metric": "decode tok/s at B=8 (Qwen3-4B bf16)", "value": r3["value"], "unit": "tok/s",
            "steps": r3["steps"], "ms_per_step": r3["ms_per_step"], "ttft_s": r3["ttft_s"],
            "config": {"workload": f"c3: Qwen3-4B, B={B3}, prompts {S3}, {N3} greedy decode steps",
                       "global_batch": B3, "seq_len": S3, "decode_steps": N3},
            "step_roofline": r3["step_roofline"],
        }
        engine_mod.CONFIG["spec_k"] = SPEC_T - 1
        B5, S5, N5 = CONFIGS["c5"]
        r5 = bench_verify(eng, torch, cfg, B5, S5, max(N5, args.steps or 0), W)   # at least its 200 steps
        engine_mod.CONFIG["spec_k"] = 0
        out["c5"] = {k: r5[k] for k in ("metric", "value", "unit", "steps", "ms_per_step", "positions_per_s",
                                        "config", "roofline", "step_roofline")}
        B4, S4, N4 = CONFIGS["c4"]
        K4 = args.steps if args.steps is not None else N4 - 1 - W
        r4 = run_decode(eng, torch, cfg, B4, S4, N4, K4, W)
        a_avg, a_bytes, a_name = time_attention(eng, torch)
        out["b32"] = {
            "metric": "decode tok/s at B=32 (Qwen3-4B bf16)", "value": r4["value"], "unit": "tok/s",
            "steps": r4["steps"], "ms_per_step": r4["ms_per_step"], "ttft_s": r4["ttft_s"],
            "config": {"workload": f"c4: Qwen3-4B, B={B4}, prompts {S4}, {N4} greedy decode steps",
                       "global_batch": B4, "seq_len": S4, "decode_steps": N4},
            "roofline": roofline(a_avg, a_bytes, a_name, "c4",
                                 "QK-norm + RoPE + KV write + GQA attention (one layer)"),
            "step_roofline": r4["step_roofline"],
            "mfma": mfma_utilisation(eng, torch),
            "vs_b1": round(r4["value"] / res["value"], 3),
        }
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(eng, cfg, CONFIGS["c2"][1])
        except Exception as error:  # noqa: BLE001 - report, do not fail the GPU number
            out["cpu_baseline"] = {"value": None, "error": repr(error)[:200]}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
