"""Decode throughput of the MI355X Qwen3-4B engine (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2|c3|c4|c5]

c5 (speculative verify steps) reports verify steps/s instead of decoded tokens/s.

Default workload is BASELINE.json's configs[1] ("c2"): Qwen3-4B, random-init
bf16 weights (seed 0), batch 1, a 128-token uniform-random prompt, greedy
decoding. The engine's own generate() runs the prompt forward (untimed) and
W warm-up steps, then K decode steps are timed between two device
synchronisations; ``value`` = decoded tokens / wall seconds over the steps
launched inside that window. Inputs and weights are resident in HBM
throughout; only token ids cross PCIe (8 bytes per sequence per step).

Extra fields: ``roofline`` for the dominant kernel (the fused
RMSNorm + gate/up GEMM + SwiGLU, 44% of the bytes of a B=1 step), timed live
with HIP events on the stream it is launched on, rotating over the 36 layers'
weights so that nothing is served from the 256 MB Infinity Cache;
``step_roofline`` for the whole step (algorithmic bytes of weights + visible
KV per step over the measured step time); ``cpu_baseline``: the oracle's
torch-CPU restatement of the same decode step on this host's cores, over a
bounded sample (2 of the 36 layers + the LM head, scaled to 36 layers).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "thing-htn-2026_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12   # MI355X HBM3E, bytes/s
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


def weight_bytes(cfg) -> int:
    H, I, D, Nq, Nkv, L, V = (cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"],
                              cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["num_hidden_layers"],
                              cfg["vocab_size"])
    per_layer = 2 * (H * (Nq + 2 * Nkv) * D + Nq * D * H + 2 * I * H + I * H)
    norms = 2 * (L * (2 * H + 2 * D) + H)
    return L * per_layer + 2 * V * H + norms


def kv_bytes_per_token(cfg) -> int:
    return cfg["num_hidden_layers"] * 2 * cfg["num_key_value_heads"] * cfg["head_dim"] * 2


def eng_pipeline_depth() -> int:
    from engine import CONFIG
    return CONFIG["inflight"]


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-layers", type=int, default=2)
    p.add_argument("--profile-sample", action="store_true",
                   help="run only the dominant kernel (rotating over the layers) and a plain 1 GiB device copy, "
                        "for rocprofv3 --pmc traffic runs; prints one JSON line")
    return p.parse_args()


def profile_sample(eng, torch, T=1):
    """Dominant-kernel launches plus a copy of known size (the FETCH_SIZE / WRITE_SIZE calibration)."""
    avg_s, k_bytes, _ = time_dominant_kernel(eng, torch, reps_per_layer=1, T=T)
    n = 1 << 29                                # 2^29 bf16 = 1 GiB read + 1 GiB written per copy
    src = torch.ones(n, dtype=torch.bfloat16, device=eng.device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"dominant_kernel_avg_us": round(avg_s * 1e6, 2), "dominant_kernel_bytes": k_bytes,
            "copy_bytes_each_way": 2 * n, "copies": 3}


# Measured HBM traffic of the dominant kernel (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE,
# scaled by the same counters' reading for a plain copy of known size); written by
# hand from the committed summary under profiles/ for the workload it names.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gate_up_traffic.json")


def measured_traffic(config: str, kernel: str):
    """Bytes per launch of ``kernel`` at ``config`` from the committed PMC summary (None if absent
    or measured for another kernel)."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    entry = rec.get(config)
    if entry is None or entry.get("kernel") != kernel:
        return None
    return entry.get("bytes_per_launch")


def time_dominant_kernel(eng, torch, reps_per_layer=3, T=1):
    """Average duration of the fused norm + gate/up + SwiGLU GEMM at the bench's M = B * T.

    Timed with HIP events on the stream the kernel is launched on, rotating over
    the 36 layers' weights (3.6 GB) so that nothing is served from cache.
    """
    from qwen_hip import ops
    B = eng.B
    b = eng.bufs(eng.state.groups[0], T)
    h, p, psq, cfg, ws = b.h, b.p, b.psq, b.cfg["gu"], b.gemm_ws
    stream = torch.cuda.current_stream()
    ops.sumsq16(h, out=psq)

    def run(w):
        if b.gemv:    # M <= 2: the balanced row-major GEMV the engine runs
            ops.gemv(h, w.gu_rows, norm_w=w.ln2, eps=eng.eps, silu_pair=True, out=p, cfg=b.gemv_cfg["gu"])
        else:
            ops.fused_linear(h, w.gu, cfg, norm_w=w.ln2, eps=eng.eps, silu_pair=True, out=p, psq_in=psq,
                             workspace=ws)

    for w in eng.w.layers[:2]:
        run(w)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    n = 0
    for _ in range(reps_per_layer):
        for w in eng.w.layers:
            run(w)
            n += 1
    end.record(stream)
    end.synchronize()
    avg_s = start.elapsed_time(end) / 1e3 / n
    w0 = eng.w.layers[0].gu
    M = B * T
    bytes_launch = w0.nbytes + M * w0.K * 2 + w0.K * 2 + M * (w0.N // 2) * 2
    name = ("gemv_kernel<%d, %d, true, 2>" % (M, b.gemv_cfg["gu"][1]) if b.gemv
            else ops.gemm_kernel_name(M, cfg, True, ops.EPI_SWIGLU))
    return avg_s, bytes_launch, name


def bench_verify(eng, torch, cfg, B, S, K, W):
    """c5: K speculative verify steps (T = SPEC_T tokens per sequence: the last accepted token and
    SPEC_T - 1 prompt-lookup drafts, which on a uniform-random prompt are effectively random ids),
    each one replay of the captured verify graph (draft, 36 layers over B*T rows with causal
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
    avg_s, k_bytes, k_name = time_dominant_kernel(eng, torch, T=T)
    achieved = k_bytes / avg_s
    return {
        "metric": f"spec-verify steps/s at B={B}, T={T}, context {S} (Qwen3-4B bf16)",
        "value": round(K / dt, 2), "unit": "verify steps/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(dt / K * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights (counter-based generator, seed 0, std 0.02), uniform-random "
                "prompt ids (torch seed 1); drafts by prompt lookup (no repeats: effectively random ids)",
        "config": {"workload": f"c5: Qwen3-4B, B={B}, context {S}, T={T} verify steps",
                   "global_batch": B, "seq_len": S, "verify_tokens": T, "parallelism": "single GPU"},
        "positions_per_s": round(K * B * T / dt, 1),
        "roofline": {"bound": "hbm", "kernel": f"{k_name}: RMSNorm + gate/up + SwiGLU (one layer)",
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4), "traffic": measured_traffic("c5", k_name),
                     "avg_us": round(avg_s * 1e6, 2), "bytes_per_launch": k_bytes},
        "step_roofline": {"bytes_per_step": int(step_bytes),
                          "achieved_GBps": round(step_bytes * K / dt / 1e9, 1),
                          "frac": round(step_bytes * K / dt / HBM_PEAK, 4)},
    }


def cpu_baseline(eng, cfg, B, S, layers):
    """Time the oracle's torch-CPU decode step on a 2-layer slice of the same weights."""
    import torch
    from oracle.model import CpuQwen3

    lw = []
    for w in eng.w.layers[:layers]:
        lw.append({"ln1": w.ln1.cpu(), "ln2": w.ln2.cpu(), "q_norm": w.q_norm.cpu(), "k_norm": w.k_norm.cpu(),
                   "w_qkv": eng.w.natural_qkv_rows(w).cpu(), "w_o": w.o_rows.cpu(), "w_gu": w.gu_rows.cpu(),
                   "w_down": w.down_rows.cpu()})
    weights = {"embed": eng.w.lm_rows.cpu(), "final_norm": eng.w.final_norm.cpu(), "layers": lw}
    ref = CpuQwen3(dict(cfg, num_hidden_layers=layers), weights)
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    max_steps = 64
    ref.prepare(B, ((S + max_steps + 64) // 64) * 64)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, cfg["vocab_size"], (B, S), generator=g)
    with torch.inference_mode():
        # The S context slots get seeded random K/V in place of the prompt forward: a decode
        # step's work does not depend on the cached values, and the oracle's prefill would hold
        # [B, heads, S, S] fp32 scores (275 GB at B = 32, S = 8192).
        for kc, vc in zip(ref.k_cache, ref.v_cache):
            kc[:, :, :S].copy_(torch.randn(kc[:, :, :S].shape, generator=g).to(kc.dtype))
            vc[:, :, :S].copy_(torch.randn(vc[:, :, :S].shape, generator=g).to(vc.dtype))
        ref.hist[:, :S] = ids
        ref.pos.fill_(S - 1)
        ref.plain_step()                       # warm-up
        t_layers, t_head, steps = 0.0, 0.0, 0
        t_end = time.perf_counter() + 15.0
        while (time.perf_counter() < t_end or steps < 2) and steps < max_steps:
            tok = ref.hist.gather(1, ref.pos.to(torch.int64)[:, None])
            t0 = time.perf_counter()
            h = ref.w["embed"][tok.reshape(-1)]
            d = None
            for l in range(layers):
                h, d = ref.layer(l, h, d, ref.pos, 1, B)
            t1 = time.perf_counter()
            from oracle import ref_torch as R
            _, n = R.add_rms_norm(h, d, ref.w["final_norm"], ref.eps)
            R.argmax_lowest(R.linear(n, ref.w["embed"]))
            t2 = time.perf_counter()
            ref.pos += 1
            t_layers += t1 - t0
            t_head += t2 - t1
            steps += 1
    per_token = (t_layers / steps) * cfg["num_hidden_layers"] / layers + t_head / steps
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(B / per_token, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"oracle torch-CPU decode step (oracle/model.py) on {layers} of "
                       f"{cfg['num_hidden_layers']} layers + LM head, {steps} steps at context ~{S} (B={B}, "
                       f"random cached K/V), scaled to {cfg['num_hidden_layers']} layers; host CPU {cpu}")}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build runs on a single MI355X); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from __graft_entry__ import write_random_model
    from engine import Engine

    B, S, N = CONFIGS[args.config]
    K = args.steps if args.steps is not None else N
    W = args.warmup
    cfg = QWEN3_4B
    if args.config == "c5":
        import engine as engine_mod
        engine_mod.CONFIG["spec_k"] = SPEC_T - 1
    with tempfile.TemporaryDirectory() as d:
        eng = Engine(write_random_model(d, cfg, seed=0, std=0.02))
    if args.config == "c5" and not args.profile_sample:
        print(json.dumps(bench_verify(eng, torch, cfg, B, S, K, W)), flush=True)
        return
    if args.profile_sample:
        # counter calibration only: the warmup certification's KV-sized copies would sit next to
        # the calibration copy in the counter log
        import engine as engine_mod
        engine_mod.CONFIG["certify"] = False
        eng.prepare(B, S, K + W + 1)
        print(json.dumps(profile_sample(eng, torch, T=SPEC_T if args.config == "c5" else 1)), flush=True)
        return
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg["vocab_size"], (B, S), generator=g).tolist()
    total = 1 + W + K
    gen = eng.generate(prompt, total)
    t_pf = time.perf_counter()
    next(gen)                                  # prompt forward + first token
    ttft = time.perf_counter() - t_pf
    for _ in range(W):
        next(gen)
    torch.cuda.synchronize()
    l0 = eng.counters["decode"]
    t0 = time.perf_counter()
    for _ in gen:
        pass
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    steps = eng.counters["decode"] - l0
    if steps <= 0:
        sys.exit(f"bench.py: no decode step was launched inside the timed window (--steps {K} is within the "
                 f"engine's {eng_pipeline_depth()} steps of pipelining); use more steps")
    dt = t1 - t0
    tok_s = steps * B / dt
    ms_step = dt / steps * 1e3

    ctx_mid = S + 1 + W + steps / 2
    step_bytes = weight_bytes(cfg) + B * ctx_mid * kv_bytes_per_token(cfg)
    avg_s, k_bytes, k_name = time_dominant_kernel(eng, torch)
    achieved = k_bytes / avg_s
    out = {
        "metric": "decode tok/s at B=1 (Qwen3-4B bf16)" if B == 1 else f"decode tok/s at B={B} (Qwen3-4B bf16)",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": W,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init bf16 weights (counter-based generator, seed 0, std 0.02), "
                "uniform-random prompt ids (torch seed 1)",
        "config": {"workload": f"{args.config}: Qwen3-4B, B={B}, prompt {S}, {N} greedy decode steps",
                   "global_batch": B, "seq_len": S, "decode_steps": N, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": f"{k_name}: RMSNorm + gate/up + SwiGLU (one layer)",
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4), "traffic": measured_traffic(args.config, k_name),
                     "avg_us": round(avg_s * 1e6, 2), "bytes_per_launch": k_bytes},
        "step_roofline": {"bytes_per_step": int(step_bytes), "achieved_GBps": round(step_bytes / (ms_step / 1e3) / 1e9, 1),
                          "frac": round(step_bytes / (ms_step / 1e3) / HBM_PEAK, 4)},
        "ttft_s": round(ttft, 3),
    }
    if not args.no_cpu_baseline:
        try:
            out["cpu_baseline"] = cpu_baseline(eng, cfg, B, S, args.cpu_layers)
        except Exception as error:  # noqa: BLE001 - report, do not fail the GPU number
            out["cpu_baseline"] = {"value": None, "error": repr(error)[:200]}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
