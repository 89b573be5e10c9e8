"""Benchmark: Qwen3-0.6B-shaped INT8 W8A8 decode on one MI355X.

Workload (the metric's named config): hidden 1024,
28 layers, 16 q / 8 kv heads, head_dim 128, SwiGLU 3072, vocab 151936, tied
embeddings, RMSNorm eps 1e-6, RoPE theta 1e6; weights N(0, 0.02) from the
SplitMix64 seed spec, quantized with the reference's INT8 per-row quantizer;
a 16-token random prompt, then greedy decode.  A "step" is one decode token
(one forward_one + argmax, all on the device, replayed as a HIP graph).

Prints ONE JSON line.  `value` = decode tokens/s.  `roofline` covers the
dominant kernel of the timed step: eager fused steps right after the timed
region launch every kernel with start/stop hipEvents (hipExtLaunchKernelGGL,
the dispatch's own timestamps, on the model stream;
syn_hip_qlm_time_step_kernels), and the kernel kind with the largest time
per step is reported against its algorithmic bytes; `roofline.step` is the
whole graph-replayed step against its weight bytes, `roofline.lm_head` the
lm_head GEMV, and `step_kernels` every kind.  `cpu_baseline` = the oracle (C
restatement of the reference cpu_simd path, single thread) decoding the same
model on the host, with `cpu_baseline.secondary` the same oracle on bounded
samples of configs 2-5.  `secondary` = the other BASELINE configurations
measured on the same GPU (synapse_amd/microbench.py): the config-1 GEMVs
one launch at a time, the config-2 Q4_0 microbench (1000 launches per
matrix), the config-3 K-quant GEMVs and decoder, the config-4 Q8_0 prefill
GEMMs, the INT8 prefill GEMM, and the config-5 Mamba decoder
(--no-secondary skips them).  A secondary that fails is recorded as
{"error": ...} and the line is still printed.
"""
from __future__ import annotations

import argparse
import hashlib
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
# HBM traffic per launch of the fused step's lm_head kernel (k_lmhead_top2),
# from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each
# scaled by what the counter reads for a 256 MiB device copy (FETCH_SIZE reads
# half the copied bytes: factor 2.0; WRITE_SIZE exact: 1.0); commands and
# readings in profiles/lm_head_int8_qwen3_k_lmhead_top2.md
LM_HEAD_FETCH_KIB, LM_HEAD_FETCH_FACTOR = 76301.0, 262144.0 / 131084.7
LM_HEAD_WRITE_KIB, LM_HEAD_WRITE_FACTOR = 816.5, 262144.0 / 262144.0
# HBM traffic per launch of the step's kernels: median FETCH_SIZE and
# WRITE_SIZE (KiB per dispatch) over the 364 dispatches of each kernel in two
# counter runs of eager steps at positions 16-29, scaled as above (readings
# and commands in profiles/qwen3_int8_decode_step_kernels_traffic.md, taken
# on the kernels of this source tree; the attention's traffic grows with the
# position).  These are recorded readings, reported as `traffic` with
# `traffic_source` naming the profile, and only while the step kernels'
# sources hash to STEP_SOURCES_SHA16 (the hash of the build the readings were
# taken on): after a change to those files the field is null until the
# profile's commands are run again and the readings and hash updated here.
TRAFFIC_SOURCE = "profiles/qwen3_int8_decode_step_kernels_traffic.md (recorded rocprofv3 --pmc)"
_STEP_KIB = {"qkv": (2157.1, 68.0), "attention": (377.5, 32.0), "o": (1078.0, 64.0),
             "gate_up": (3206.6, 113.5), "down": (1605.5, 48.0)}
STEP_SOURCES = ("synapse_amd/csrc/decode_fused.hip", "synapse_amd/csrc/fused_dev.hpp",
                "synapse_amd/csrc/qlm.hip")
STEP_SOURCES_SHA16 = "43f9074b6c63b25e"


def step_sources_sha16() -> str:
    h = hashlib.sha256()
    for f in STEP_SOURCES:
        with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


STEP_KERNEL_TRAFFIC = ({k: round(1024 * (f * LM_HEAD_FETCH_FACTOR + w * LM_HEAD_WRITE_FACTOR))
                        for k, (f, w) in _STEP_KIB.items()}
                       if step_sources_sha16() == STEP_SOURCES_SHA16 else {})


def step_weight_bytes(c):
    """Algorithmic bytes per decode token: int8 weights + f32 per-row scales."""
    h, q, kv, i, v, L = (c["hidden"], c["n_heads"] * c["head_dim"],
                         c["n_kv_heads"] * c["head_dim"], c["inter"], c["vocab"], c["n_layers"])
    per_layer = (q * h + 2 * kv * h + h * q + 3 * i * h) + 4 * (q + 2 * kv + h + 2 * i + h)
    return L * per_layer + v * h + 4 * v


def step_kernel_bytes(c, pos):
    """Algorithmic HBM bytes of one launch of each fused-step kernel kind at
    decode position `pos`: a GEMV moves N*K int8 weights + 4N scales + K
    int8 activations + 4N outputs (the per-matvec formula of the metric);
    the attention reads the K and V cache rows of positions 0..pos."""
    h, q, kv, i, v = (c["hidden"], c["n_heads"] * c["head_dim"],
                      c["n_kv_heads"] * c["head_dim"], c["inter"], c["vocab"])
    gemv = lambda n, k: n * k + 8 * n + k
    return {"qkv": gemv(q + 2 * kv, h), "o": gemv(h, q), "gate_up": gemv(2 * i, h),
            "down": gemv(h, i), "lm_head": gemv(v, h),
            "attention": 2 * 4 * kv * (pos + 1)}


STEP_KERNEL_NAMES = {
    "qkv": "k_fused_gemv<0,256,U,false,R> (residual + RMSNorm + quantize + QKV GEMV)",
    "attention": "k_attn_head<false,128> (head norms, RoPE, KV append, attention)",
    "o": "k_fused_gemv<1,512,U,false,R> (quantize + O GEMV)",
    "gate_up": "k_fused_gemv<0,256,U,true,R> (residual + RMSNorm + quantize + gate|up GEMV in "
               "panel pairs, split K, SwiGLU in each pair's last slice)",
    "down": "k_fused_gemv<5,512,U,false,R> (quantize h range + down GEMV)",
    "lm_head": "k_lmhead_top2<8,8> (lm_head GEMV + per-panel top-2)"}


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


LLAMA3B = dict(hidden=3072, n_layers=28, n_heads=24, n_kv_heads=8, head_dim=128, inter=8192,
               vocab=128256, eps=1e-5, rope_theta=5e5)
MAMBA370M = dict(d_model=1024, d_inner=2048, d_state=16, d_conv=4, dt_rank=64, n_layers=48,
                 vocab=50280, eps=1e-5)
# LFM2.5-350M (models/ssm/hybrid/config.rs:132-156): 0 = LIV conv, 1 = GQA
LFM25 = dict(hidden=1024, n_layers=16, vocab=65536, n_heads=16, n_kv_heads=8, head_dim=64,
             inner=1024, conv_kernel=3, inter=6656, eps=1e-5, rope_theta=1e6,
             layer_kinds=[0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 1, 0, 1, 0, 1, 0])


def hybrid_weight_bytes(c):
    """Bytes one decode step streams: the Q4_0 projections (18 bytes per 32
    weights) and the tied f32 lm_head."""
    h, inner, f = c["hidden"], c["inner"], c["inter"]
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    q4 = 0
    for kind in c["layer_kinds"]:
        q4 += (3 * inner * h + h * inner) if kind == 0 else ((qd + 2 * kvd) * h + h * qd)
        q4 += 3 * f * h
    return q4 // 32 * 18 + c["vocab"] * h * 4


def _ids(n, vocab, seed):
    """Uniform random ids in [0, vocab) (SplitMix64, as prompt_ids)."""
    s, out, M = seed, [], (1 << 64) - 1
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        out.append(z % vocab)
    return out


def kquant_weight_bytes(c):
    """Config 3 bytes per decode token: Q4_K q,k,v,o,gate,up; Q6_K down, lm_head."""
    h, q, kv, i, v, L = (c["hidden"], c["n_heads"] * c["head_dim"],
                         c["n_kv_heads"] * c["head_dim"], c["inter"], c["vocab"], c["n_layers"])
    q4k = lambda n, k: n * (k // 256) * 144
    q6k = lambda n, k: n * (k // 256) * 210
    layer = q4k(q, h) + 2 * q4k(kv, h) + q4k(h, q) + 2 * q4k(i, h) + q6k(h, i)
    return L * layer + q6k(v, h)


def guarded(fn, *a):
    """Run one secondary record; a failure is recorded in the line instead of
    ending the run before the headline is printed."""
    try:
        return fn(*a)
    except Exception as e:  # noqa: BLE001 - any failure of a secondary is reported
        import traceback
        traceback.print_exc(file=sys.stderr)
        return {"error": f"{type(e).__name__}: {e}"}


def secondary(hip, np):
    """The other BASELINE configurations, measured on the same GPU."""
    from synapse_amd import microbench as mb
    out = {}
    t0 = time.perf_counter()
    # measured ceilings of this GPU beside the published peaks
    out["measured_peaks"] = {
        "hbm_read_gb_s": round(hip.probe_hbm_read(4 << 30), 1),
        "mfma_f16_32x32x16_tflops": round(hip.probe_mfma(2, 20000), 1),
        "mfma_i8_32x32x32_tops": round(hip.probe_mfma(3, 20000), 1),
        "published": {"hbm_gb_s": 8000.0, "f16_tflops": 2500.0, "i8_tops": 5000.0}}
    out["config1_int8_gemv_qwen3"] = {
        "note": "one launch per GEMV (the decode step fuses them), >= 1 GiB rotated",
        "gemvs": mb.int8_suite()}
    out["config2_q4_0_gemv_llama1b"] = {
        "note": "batch-1 Q4_0 GEMV, f32 activations, 1000 launches per matrix round-robin "
                "over >= 1 GiB of weight copies",
        "gemvs": mb.q4_0_suite()}
    out["ternary_gemv_llama1b_shapes"] = {
        "note": "TernaryLinear batch-1 GEMV (not a BASELINE config; the quantized-linear "
                "format of ternary_linear.rs), >= 1 GiB of weight copies rotated",
        "gemvs": mb.ternary_suite()}
    out["config3_kquant_gemv_llama3b"] = {
        "note": "batch-1 Q4_K / Q6_K GEMV at the LLaMA-3.2-3B shapes, >= 1 GiB rotated",
        "gemvs": mb.kquant_suite()}
    # config 3 decoder: 256-token prompt, 128 greedy decode steps
    cfg = dict(LLAMA3B, max_seq=256 + 128 + 1)
    m = hip.KQuantCausalLM(cfg)
    m.init_synthetic(SEED_BASE, 0.02)
    ids = np.array(_ids(256, cfg["vocab"], PROMPT_SEED), np.uint32)
    pf_ms, dec_ms = m.time(ids, 128)
    # speculative decode with the reference's default draft (first L/3 layers)
    spec = {}
    for name, fn in (("generate", lambda: m.generate(ids, 64)),
                     ("speculative_k4", lambda: m.generate_speculative(ids, 64, 4)),
                     ("speculative_k7", lambda: m.generate_speculative(ids, 64, 7))):
        fn()
        best = float("inf")
        for _ in range(3):
            t = time.perf_counter()
            fn()
            best = min(best, time.perf_counter() - t)
        spec[name] = {"ms": round(best * 1e3, 2), "tok_s": round(64 / best, 1)}
    spec["note"] = ("256-token prompt + 64 greedy tokens per call, best of 3; drafts from the "
                    f"first {LLAMA3B['n_layers'] // 3} of {LLAMA3B['n_layers']} layers "
                    "(forward_one_draft), every draft accepted; k = 7 verifies 8 rows, one "
                    "K-quant GEMV launch per projection")
    m.close()
    wb = kquant_weight_bytes(LLAMA3B)
    out["config3_kquant_decode_llama3b"] = {
        "prefill_256_ms": round(pf_ms, 2), "decode_tok_s": round(128e3 / dec_ms, 1),
        "decode_ms_per_token": round(dec_ms / 128, 3), "weight_bytes_per_token": wb,
        "decode_weight_gbs": round(wb / (dec_ms / 128 * 1e-3) / 1e9, 1),
        "speculative_decode": spec}
    out["config4_q8_0_prefill_mistral7b"] = [mb.q8_0_prefill_suite(512),
                                             mb.q8_0_prefill_suite(2048)]
    out["int8_prefill_gemm"] = [mb.int8_prefill_record(128, 1024, 3072),
                                mb.int8_prefill_record(512, 4096, 4096),
                                mb.int8_prefill_record(2048, 4096, 4096)]
    mam = {}
    for xdt in (False, True):
        mc = dict(MAMBA370M, max_tokens=64 + 128 + 1)
        mm = hip.QuantizedMamba(mc, int8_xdt=xdt)
        mm.init_synthetic(SEED_BASE, 0.02)
        mm.prefill(np.array(_ids(64, mc["vocab"], PROMPT_SEED), np.uint32))
        ms = mm.decode_timed(128)
        mm.close()
        mam["int8_x_dt_proj" if xdt else "reference_semantics"] = {
            "decode_tok_s": round(128e3 / ms, 1), "decode_ms_per_token": round(ms / 128, 3)}
    mam["int8_projection_gemvs"] = [
        mb.gemv_record(hip.FMT_INT8, 4096, 1024, "in_proj 1024->4096"),
        mb.gemv_record(hip.FMT_INT8, 1024, 2048, "out_proj 2048->1024")]
    out["config5_mamba370m"] = mam
    # hybrid LFM2.5-350M Q4 decode (metal/hybrid_gpu_forward.rs's path): not a
    # BASELINE configuration; 8-token prompt, 128 greedy decode steps
    hc = dict(LFM25, max_seq=8 + 128 + 1)
    hm = hip.HybridLM(hc)
    hm.init_synthetic(SEED_BASE, 0.02)
    hm.prefill(np.array(_ids(8, hc["vocab"], PROMPT_SEED), np.uint32))
    ms = hm.decode_timed(128)
    fused = hm.fused_active
    hm.reset()
    hm.set_options(fused=False)
    hm.prefill(np.array(_ids(8, hc["vocab"], PROMPT_SEED), np.uint32))
    ms_op = hm.decode_timed(128)
    hm.close()
    hb = hybrid_weight_bytes(LFM25)
    out["hybrid_lfm25_q4_0_decode"] = {
        "decode_tok_s": round(128e3 / ms, 1), "decode_ms_per_token": round(ms / 128, 4),
        "weight_bytes_per_token": hb, "decode_weight_gbs": round(hb / (ms / 128 * 1e-3) / 1e9, 1),
        "fused": fused, "op_by_op_tok_s": round(128e3 / ms_op, 1),
        "note": "16 layers (10 LIV conv, 6 GQA), Q4_0 projections, tied f32 lm_head (65536 x "
                "1024), graph replay of the fused step, 72 kernels (op_by_op_tok_s: the "
                "op-by-op step)"}
    out["seconds"] = round(time.perf_counter() - t0, 1)
    return out


def speculative_record(model, np, k: int = 4, max_new: int = 64, reps: int = 3):
    """generate vs generate_speculative (speculative_k = k) on the config-1
    model: whole calls (16-token prefill + max_new tokens, tokens read back),
    wall clock, best of `reps`.  The INT8 model drafts with full forward_one
    steps (int8.rs:739), so each round adds a (k+1)-row verify prefill."""
    ids = np.array(prompt_ids(), np.uint32)
    res = {}
    for name, fn in (("generate", lambda: model.generate(ids, max_new)),
                     (f"speculative_k{k}", lambda: model.generate_speculative(ids, max_new, k))):
        fn()
        best = float("inf")
        for _ in range(reps):
            t = time.perf_counter()
            fn()
            best = min(best, time.perf_counter() - t)
        res[name] = {"ms": round(best * 1e3, 2), "tok_s": round(max_new / best, 1)}
    res["note"] = (f"{PROMPT}-token prompt + {max_new} tokens per call, greedy; drafts are full "
                   "forward_one steps (no INT8 draft model in the reference), every draft accepted")
    return res


def _median_s(fn, reps):
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return sorted(ts)[len(ts) // 2]


def cpu_baselines_secondary(np):
    """The oracle single-threaded (the reference's kernels are) on bounded
    samples of configs 2-5, in the units of the GPU records beside them."""
    import oracle as O
    from synapse_amd import microbench as mb
    O.set_threads(1)
    out = {"cores": 1, "kind": "port",
           "note": "oracle/oracle.c, one thread (O.set_threads(1)); the reference's Zig/Rust "
                   "kernels cannot be built in this image"}
    t0 = time.perf_counter()
    # config 2: q4_0GemvRow (qmatmul.zig:276-343) at the five LLaMA-1B shapes
    # (the time does not depend on the values: random nibbles, scale 0.01)
    rng = np.random.default_rng(1)
    rows = []
    for lab, k, n in mb.Q4_0_SHAPES:
        packed = rng.integers(0, 256, size=(n * (k // 32), 18), dtype=np.uint8)
        packed[:, 0:2] = np.array([np.float16(0.01)]).view(np.uint8)
        packed = packed.reshape(-1)
        x = rng.standard_normal(k).astype(np.float32)
        reps = 3 if n * k > 50_000_000 else 7
        s = _median_s(lambda: O.q4_0_gemv(x, packed, n), reps)
        nb = n * (k // 32) * 18 + 4 * k + 4 * n
        rows.append({"matrix": lab, "us": round(s * 1e6, 1), "gb_s": round(nb / s / 1e9, 2)})
    out["config2_q4_0_gemv"] = {"sample": "median of 3-7 calls per matrix", "gemvs": rows}
    # config 3: the f32 CausalLM over Q4_K / Q6_K weights (matmul.zig:223-347
    # per token): one LLaMA-3B-width layer (Q4_K q/k/v/o/gate/up, Q6_K down)
    # with a small vocabulary, and the 128256 x 3072 f32 lm_head GEMV on its
    # own; a token = 28 layers + the lm_head
    cfg = dict(LLAMA3B, n_layers=1, vocab=256, max_seq=32)
    o = kquant_oracle_model(cfg, np)
    o.prefill(np.array(_ids(4, cfg["vocab"], PROMPT_SEED), np.uint32))
    t_layer = _median_s(lambda: o.forward_one(1), 3)
    o.close()
    w_lm = np.full((LLAMA3B["vocab"], LLAMA3B["hidden"]), 0.01, np.float32)
    xh = rng.standard_normal((1, LLAMA3B["hidden"])).astype(np.float32)
    t_lm = _median_s(lambda: O.matmul_t(xh, w_lm), 2)
    del w_lm
    t28 = LLAMA3B["n_layers"] * t_layer + t_lm
    out["config3_kquant_decode"] = {
        "tok_s": round(1.0 / t28, 3), "ms_per_token": round(t28 * 1e3, 1),
        "sample": f"one full-width layer (+ a 256-row head) {t_layer * 1e3:.0f} ms, the "
                  f"lm_head GEMV {t_lm * 1e3:.0f} ms; a token = 28 x layer + lm_head"}
    # config 4: sgemmTiled's GOTO path (matmul.zig:157-183) on dequantized Q8_0
    # weights, the q matrix 4096 -> 4096 at M = 32 (the same code runs M = 512)
    k = n = 4096
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    x = rng.standard_normal((32, k), dtype=np.float32)
    s = _median_s(lambda: O.matmul_t(x, w), 1)
    out["config4_q8_0_prefill_gemm"] = {
        "tflops": round(2.0 * 32 * n * k / s / 1e12, 5), "ms": round(s * 1e3, 1),
        "sample": "q 4096->4096 at M = 32, one call (f32 weights as the reference runs them)"}
    # config 5: the INT8 Mamba decode (int8_mamba.rs:78-109), 370M shape
    mc = dict(MAMBA370M)
    mm = O.QuantizedMamba(mc)
    mm.init_synthetic(SEED_BASE)
    mm.prefill(np.array(_ids(4, mc["vocab"], PROMPT_SEED), np.uint32))
    s = _median_s(lambda: mm.decode_one(1), 5)
    mm.close()
    out["config5_mamba_decode"] = {
        "tok_s": round(1.0 / s, 3), "ms_per_token": round(s * 1e3, 1),
        "sample": "median of 5 decode steps after a 4-token prompt (reference semantics: "
                  "x_proj, dt_proj and lm_head f32)"}
    # hybrid LFM2.5-350M Q4 decode: one-conv, one-GQA and conv+GQA models at
    # full widths give a conv layer, a GQA layer and the head; a token = 10
    # conv + 6 GQA layers + the head
    ts = {}
    for name, kinds in (("c", [0]), ("a", [1]), ("ca", [0, 1])):
        hc = dict(LFM25, n_layers=len(kinds), layer_kinds=kinds, max_seq=16)
        hm = O.HybridLM(hc)
        hm.init_synthetic(SEED_BASE, 0.02)
        hm.decode_one(1)
        ts[name] = _median_s(lambda: hm.decode_one(2), 3)
        hm.close()
    t_conv, t_gqa = ts["ca"] - ts["a"], ts["ca"] - ts["c"]
    t_head = ts["c"] + ts["a"] - ts["ca"]
    nc = sum(1 for k in LFM25["layer_kinds"] if k == 0)
    t_tok = nc * t_conv + (LFM25["n_layers"] - nc) * t_gqa + t_head
    out["hybrid_lfm25_q4_0_decode"] = {
        "tok_s": round(1.0 / t_tok, 3), "ms_per_token": round(t_tok * 1e3, 1),
        "sample": f"median of 3 decode steps of 1- and 2-layer models at full widths: conv "
                  f"layer {t_conv * 1e3:.1f} ms, GQA layer {t_gqa * 1e3:.1f} ms, head "
                  f"{t_head * 1e3:.1f} ms; a token = {nc} conv + {LFM25['n_layers'] - nc} GQA "
                  "layers + head"}
    out["seconds"] = round(time.perf_counter() - t0, 1)
    O.set_threads(16)
    return out


def kquant_oracle_model(cfg, np):
    """The oracle's f32 CausalLM over config 3's block formats (Q4_K attention
    and gate/up, Q6_K down and lm_head), synthetic weights from the seed spec
    encoded by the library's host encoder (the bytes the GPU model loads)."""
    import oracle as O
    from synapse_amd import hip
    h, hd = cfg["hidden"], cfg["head_dim"]
    qd, kvd, inter = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["inter"]
    q4k, q6k = (hip.FMT_Q4_K, "q4_k"), (hip.FMT_Q6_K, "q6_k")
    o = O.CausalLM(cfg, qk_norm=False)
    o.set_embed(O.normal(cfg["vocab"] * h, SEED_BASE, 0.02).reshape(cfg["vocab"], h))
    shapes = [(qd, h, q4k), (kvd, h, q4k), (kvd, h, q4k), (h, qd, q4k), (inter, h, q4k),
              (inter, h, q4k), (h, inter, q6k)]
    for layer in range(cfg["n_layers"]):
        for p, (n, k, (fmt, name)) in enumerate(shapes):
            w = O.normal(n * k, SEED_BASE + 1 + 8 * layer + p, 0.02).reshape(n, k)
            o.set_proj(layer, p, name, hip.kquant_encode(fmt, w))
    w = O.normal(cfg["vocab"] * h, SEED_BASE + 1 + 8 * cfg["n_layers"], 0.02)
    o.set_lm_head("q6_k", hip.kquant_encode(hip.FMT_Q6_K, w.reshape(cfg["vocab"], h)))
    return o


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
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other BASELINE configurations (configs 2-5 and GEMMs)")
    ap.add_argument("--lm-head-iters", type=int, default=20)
    ap.add_argument("--unfused", action="store_true",
                    help="one kernel per reference op instead of the fused decode layer")
    ap.add_argument("--eager", action="store_true",
                    help="launch the decode kernels eagerly instead of replaying a HIP graph "
                         "(for profilers that do not follow graph launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the decode path runs on a single "
              "GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from synapse_amd import hip
    hip.init(0)
    # rows for the timed decode (and the per-kernel timing steps after it) and
    # for the speculative record (k = 4, 64 tokens: a round appends k + 2
    # rows for k + 1 tokens)
    kern_steps = 8
    cfg = dict(QWEN3, max_seq=PROMPT + max(args.warmup + args.steps + kern_steps, 2 * 64 + 8) + 1)
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

    # lm_head kernel as the fused step launches it, back to back over two
    # weight copies (HBM-streamed); the one-kernel-per-op step: single launches
    # with the Infinity Cache flushed in between
    lm_ms = (model.time_lm_head(args.lm_head_iters) if args.unfused
             else model.time_lm_head_rotating(2 * args.lm_head_iters))
    lm_gbs = lm_head_bytes(QWEN3) / (lm_ms * 1e-3) / 1e9
    # every kernel of the step, timed by its own start/stop events in eager
    # steps right after the timed region
    kern = None
    if not args.unfused:
        pos0 = PROMPT + args.warmup + args.steps
        kern = guarded(model.time_step_kernels, kern_steps)
        if "error" not in kern:
            kb = step_kernel_bytes(QWEN3, pos0 + kern_steps // 2)
            for k, rec in kern.items():
                rec["us_per_step"] = round(rec["avg_us"] * rec["launches_per_step"], 2)
                if k in kb:
                    rec["bytes_per_launch"] = kb[k]
                    rec["gb_s"] = round(kb[k] / (rec["avg_us"] * 1e-6) / 1e9, 1)
                    rec["hbm_frac"] = round(rec["gb_s"] / HBM_PEAK_GBS, 4)
    spec = None if args.no_secondary else guarded(speculative_record, model, np)
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
                           "(Apple Silicon, status/benchmark_matrix.md:23)",
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
    }
    lm_rec = {"kernel": ("k_lmhead_top2<8,8>" if not args.unfused else "k_gemv_w8a8<1>")
                        + " lm_head 151936x1024",
              "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
              "frac": round(lm_gbs / HBM_PEAK_GBS, 4),
              "traffic": None if args.unfused else round(
                  1024 * (LM_HEAD_FETCH_KIB * LM_HEAD_FETCH_FACTOR
                          + LM_HEAD_WRITE_KIB * LM_HEAD_WRITE_FACTOR)),
              "traffic_source": None if args.unfused else
                  "profiles/lm_head_int8_qwen3_k_lmhead_top2.md (recorded rocprofv3 --pmc)",
              "avg_launch_us": round(lm_ms * 1e3, 2), "bytes_per_launch": lm_head_bytes(QWEN3),
              "timing": "hipEvent pair around back-to-back launches alternating two weight "
                        "copies (2 x 156 MB > the 256 MB Infinity Cache)"}
    step_rec = {"kernel": "the whole decode step (graph replay)",
                "achieved": line["decode_weight_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": line["decode_weight_hbm_frac"], "bytes_per_step": step_bytes,
                "ms_per_step": round(ms_per_step, 4)}
    if kern and "error" not in kern:
        # the dominant kernel of the step: the largest time per step
        dom = max((k for k in kern if k in STEP_KERNEL_NAMES),
                  key=lambda k: kern[k]["us_per_step"])
        d = kern[dom]
        line["roofline"] = {
            "bound": "hbm", "kernel": STEP_KERNEL_NAMES[dom], "achieved": d["gb_s"],
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": d["hbm_frac"],
            "traffic": STEP_KERNEL_TRAFFIC.get(dom),
            "traffic_source": TRAFFIC_SOURCE if STEP_KERNEL_TRAFFIC else
                "none: the step kernels' sources differ from the build the readings were taken on",
            "avg_launch_us": d["avg_us"],
            "bytes_per_launch": d["bytes_per_launch"],
            "share_of_step": round(d["us_per_step"] / (ms_per_step * 1e3), 4),
            "timing": "start/stop hipEvents of every launch (hipExtLaunchKernelGGL: the "
                      "dispatch's own timestamps) of eager fused steps on the model stream, "
                      f"positions {PROMPT + args.warmup + args.steps}-"
                      f"{PROMPT + args.warmup + args.steps + kern_steps}",
            "step": step_rec, "lm_head": lm_rec}
        line["step_kernels"] = kern
    else:
        line["roofline"] = dict(bound="hbm", **lm_rec)
        line["roofline"]["step"] = step_rec
        if kern:
            line["step_kernels"] = kern
    if not args.no_secondary:
        line["secondary"] = guarded(secondary, hip, np)
        line["secondary"]["config1_speculative_decode"] = spec
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = guarded(cpu_baseline, args.cpu_seconds)
        if not args.no_secondary:
            line["cpu_baseline"]["secondary"] = guarded(cpu_baselines_secondary, np)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
