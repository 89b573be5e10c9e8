"""Benchmark: Qwen3-0.6B-shaped INT8 W8A8 decode on one MI355X.

Workload (the metric's named config): hidden 1024,
28 layers, 16 q / 8 kv heads, head_dim 128, SwiGLU 3072, vocab 151936, tied
embeddings, RMSNorm eps 1e-6, RoPE theta 1e6; weights N(0, 0.02) from the
SplitMix64 seed spec, quantized with the reference's INT8 per-row quantizer;
a 16-token random prompt, then greedy decode.  A "step" is one decode token
(one forward_one + argmax, all on the device, replayed as a HIP graph).

Prints ONE JSON line.  `value` = decode tokens/s.  `roofline` covers the
dominant decode matvec (the tied lm_head, 151936 x 1024 INT8 GEMV) timed per
launch with hipEvents on the model stream, with the Infinity Cache flushed
between launches.  `cpu_baseline` = the oracle (C restatement of the
reference cpu_simd path, single thread) decoding the same model on the host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

QWEN3 = dict(hidden=1024, n_layers=28, n_heads=16, n_kv_heads=8, head_dim=128, inter=3072,
             vocab=151936, eps=1e-6, rope_theta=1e6)
PROMPT = 16
SEED_BASE = 0x5EED0000
PROMPT_SEED = SEED_BASE + 0xFFFF
HBM_PEAK_GBS = 8000.0
REF_DECODE_TOKS = 27.3  # Qwen3-0.6B INT8 decode, reference cpu_simd (Apple Silicon)


def step_weight_bytes(c):
    """Algorithmic bytes per decode token: int8 weights + f32 per-row scales."""
    h, q, kv, i, v, L = (c["hidden"], c["n_heads"] * c["head_dim"],
                         c["n_kv_heads"] * c["head_dim"], c["inter"], c["vocab"], c["n_layers"])
    per_layer = (q * h + 2 * kv * h + h * q + 3 * i * h) + 4 * (q + 2 * kv + h + 2 * i + h)
    return L * per_layer + v * h + 4 * v


def lm_head_bytes(c):
    """One INT8 GEMV: N*K weights + 4N scales + K activation bytes + 4N output."""
    n, k = c["vocab"], c["hidden"]
    return n * k + 4 * n + k + 4 * n


def prompt_ids():
    """Uniform random ids in [0, vocab) from the seed spec (SplitMix64)."""
    s = PROMPT_SEED
    out = []
    M = (1 << 64) - 1
    for _ in range(PROMPT):
        s = (s + 0x9E3779B97F4A7C15) & M
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        out.append(z % QWEN3["vocab"])
    return out


def cpu_baseline(budget_s: float):
    """Oracle decode on the host: 1 thread, same model and prompt."""
    import numpy as np

    import oracle as O
    cfg = dict(QWEN3, max_seq=PROMPT + 256)
    m = O.QuantizedCausalLM(cfg)
    m.init_synthetic(SEED_BASE, 0.02)
    ids = np.array(prompt_ids(), np.uint32)
    t0 = time.perf_counter()
    logits = m.prefill(ids)
    prefill_s = time.perf_counter() - t0
    tok = O.argmax(logits)
    steps = 0
    t0 = time.perf_counter()
    while True:
        logits = m.forward_one(tok)
        tok = O.argmax(logits)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 200:
            break
    m.close()
    return {"value": round(steps / el, 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{steps} greedy decode steps after the {PROMPT}-token prompt "
                      f"({el:.1f} s; prefill {prefill_s:.1f} s), oracle/oracle.c "
                      f"single-threaded on {os.cpu_count()} visible host cores"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--lm-head-iters", type=int, default=20)
    ap.add_argument("--unfused", action="store_true",
                    help="one kernel per reference op instead of the fused decode layer")
    ap.add_argument("--eager", action="store_true",
                    help="launch the decode kernels eagerly instead of replaying a HIP graph "
                         "(for profilers that do not follow graph launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the decode path is single-GPU; "
              "sharding is described in DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from synapse_amd import hip
    hip.init(0)
    cfg = dict(QWEN3, max_seq=PROMPT + args.warmup + args.steps + 1)
    t0 = time.perf_counter()
    model = hip.QuantizedCausalLM(cfg)
    model.init_synthetic(SEED_BASE, 0.02)
    model.set_options(fused=not args.unfused, graph=not args.eager)
    load_s = time.perf_counter() - t0
    import numpy as np
    ids = np.array(prompt_ids(), np.uint32)
    model.prefill(ids)
    if args.warmup:
        model.decode_timed(args.warmup)
    hip.check(hip.lib().syn_hip_synchronize())
    w0 = time.perf_counter()
    ms = model.decode_timed(args.steps)
    hip.check(hip.lib().syn_hip_synchronize())
    wall_ms = (time.perf_counter() - w0) * 1e3
    ms_per_step = ms / args.steps
    toks = 1000.0 / ms_per_step
    step_bytes = step_weight_bytes(QWEN3)

    lm_ms = model.time_lm_head(args.lm_head_iters)
    lm_gbs = lm_head_bytes(QWEN3) / (lm_ms * 1e-3) / 1e9
    model.close()

    line = {
        "metric": "quant GEMV GB/s (% HBM peak) + decode tok/s, Qwen3-0.6B-shape INT8, 1 GPU",
        "value": round(toks, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(toks / REF_DECODE_TOKS, 2),
        "vs_baseline_ref": f"{REF_DECODE_TOKS} tok/s, reference cpu_simd Qwen3-0.6B INT8 decode "
                           "(Apple Silicon, BASELINE.md)",
        "dtype": "int8",
        "data": "synthetic (random N(0,0.02) weights, random prompt ids)",
        "config": {"workload": "qwen3-0.6b-shape int8 w8a8 greedy decode after a 16-token prompt",
                   "hidden": 1024, "layers": 28, "heads": "16q/8kv", "head_dim": 128,
                   "inter": 3072, "vocab": 151936, "positions": [PROMPT + args.warmup,
                                                                 PROMPT + args.warmup + args.steps]},
        "decode_weight_gbs": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "decode_weight_hbm_frac": round(step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_token": step_bytes,
        "wall_ms_timed_region": round(wall_ms, 2),
        "model_load_s": round(load_s, 1),
        "roofline": {"bound": "hbm", "kernel": "k_gemv_w8a8<1> lm_head 151936x1024",
                     "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "avg_launch_us": round(lm_ms * 1e3, 2),
                     "bytes_per_launch": lm_head_bytes(QWEN3)},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
