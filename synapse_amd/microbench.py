"""Kernel-level measurements of the quantized-linear path on one GPU.

Each function builds synthetic weights of the benchmark shapes, uploads them
through the library's C ABI and times back-to-back launches with hipEvents
(syn_hip_qlinear_time_set).  Decode GEMVs at batch 1 are HBM-bound: to
measure HBM and not the 256 MB Infinity Cache, each shape is timed
round-robin over enough copies of its matrix to stream >= 1 GiB per round.

Weight values do not change the kernels' work, so the block bytes are
random with fixed, finite f16 scales (Q4_0 / Q8_0 / Q4_K / Q6_K) and int8
weights are random bytes with random per-row scales.

Algorithmic bytes per GEMV (the roofline numerator) = weight blocks and
scales + activation in + output out; GEMM work = 2*M*N*K flops.
"""
from __future__ import annotations

import math

import numpy as np

from . import hip

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense bf16/f16
MFMA_I8_PEAK_TOPS = 5000.0     # dense int8
F16_SCALE = 0x1E66             # a finite f16 (about 0.0062)

BLOCK = {hip.FMT_Q4_0: (32, 18), hip.FMT_Q8_0: (32, 34), hip.FMT_Q4_K: (256, 144),
         hip.FMT_Q6_K: (256, 210)}
NAMES = {hip.FMT_INT8: "int8", hip.FMT_Q4_0: "q4_0", hip.FMT_Q8_0: "q8_0",
         hip.FMT_Q4_K: "q4_k", hip.FMT_Q6_K: "q6_k", hip.FMT_TERNARY: "ternary"}


def weight_bytes(fmt: int, n: int, k: int) -> int:
    if fmt == hip.FMT_INT8:
        return n * k + 4 * n
    if fmt == hip.FMT_TERNARY:
        return n * ((k + 15) // 16) * 8
    el, b = BLOCK[fmt]
    return n * (k // el) * b


def gemv_bytes(fmt: int, n: int, k: int) -> int:
    """Algorithmic HBM bytes of one batch-1 GEMV launch."""
    act = k if fmt == hip.FMT_INT8 else 4 * k
    return weight_bytes(fmt, n, k) + act + 4 * n


def _blocks(fmt: int, n: int, k: int, rng) -> np.ndarray:
    """Random block bytes of an [n, k] matrix with finite f16 scales."""
    el, b = BLOCK[fmt]
    nb = n * (k // el)
    raw = rng.integers(0, 256, size=(nb, b), dtype=np.uint8)
    f16 = np.array([F16_SCALE & 0xFF, F16_SCALE >> 8], np.uint8)
    if fmt in (hip.FMT_Q4_0, hip.FMT_Q8_0):
        raw[:, 0:2] = f16                      # d at the front
    elif fmt == hip.FMT_Q4_K:
        raw[:, 0:2] = f16                      # d, dmin
        raw[:, 2:4] = f16
    else:
        raw[:, 208:210] = f16                  # Q6_K: d at the end
    return raw.reshape(-1)


def _make(fmt: int, n: int, k: int, rng):
    """One device copy of a synthetic [n, k] matrix in `fmt`."""
    if fmt == hip.FMT_INT8:
        w = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
        sc = (rng.random(n, dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
        return lambda: hip.QLinear.int8(w, sc, hip.LAYOUT_NK)
    if fmt == hip.FMT_TERNARY:
        raw = rng.integers(0, 256, size=(n * ((k + 15) // 16), 8), dtype=np.uint8)
        raw[:, 0:4] = np.frombuffer(np.float32(0.01).tobytes(), np.uint8)  # scale
        tb = raw.reshape(-1)
        return lambda: hip.QLinear.ternary(tb, n, k)
    blocks = _blocks(fmt, n, k, rng)
    if fmt == hip.FMT_Q4_0:
        return lambda: hip.QLinear.q4_0(blocks, n, k)
    return lambda: hip.QLinear.gguf(fmt, blocks, n, k)


def copies_for(nbytes: int, target: int = 1 << 30, cap: int = 512) -> int:
    return max(2, min(cap, math.ceil(target / max(1, nbytes))))


def time_gemv(fmt: int, n: int, k: int, m: int = 1, rounds: int = 4, target: int = 1 << 30,
              seed: int = 0, launches: int = 0):
    """Average launch time (ms) of y[m,n] = x[m,k] W^T over rotating copies
    (`rounds` passes over the copies, or enough for `launches` launches)."""
    rng = np.random.default_rng(seed)
    make = _make(fmt, n, k, rng)
    ncopy = copies_for(weight_bytes(fmt, n, k), target)
    if launches:
        rounds = max(rounds, math.ceil(launches / ncopy))
    lins = [make() for _ in range(ncopy)]
    x = hip.DeviceBuffer(max(4, m * k * 4))
    x.upload(rng.standard_normal(m * k, dtype=np.float32))
    y = hip.DeviceBuffer(max(4, m * n * 4))
    xq = sx = None
    try:
        if fmt == hip.FMT_INT8:
            ldq = (k + 15) // 16 * 16
            xq = hip.DeviceBuffer(m * ldq)
            xq.upload(rng.integers(-127, 128, size=m * ldq, dtype=np.int8))
            sx = hip.DeviceBuffer(4 * m)
            sx.upload(np.full(m, 0.01, np.float32))
            ms = hip.QLinear.time_set(lins, m, d_xq=xq.ptr, ldxq=ldq, d_sx=sx.ptr, d_y=y.ptr,
                                      rounds=rounds)
        else:
            ms = hip.QLinear.time_set(lins, m, d_x=x.ptr, d_y=y.ptr, rounds=rounds)
    finally:
        for l in lins:
            l.close()
        for b in (x, y, xq, sx):
            if b is not None:
                b.close()
    return ms, ncopy


def gemv_record(fmt: int, n: int, k: int, label: str, rounds: int = 4,
                launches: int = 0) -> dict:
    ms, ncopy = time_gemv(fmt, n, k, 1, rounds, launches=launches)
    nbytes = gemv_bytes(fmt, n, k)
    gbs = nbytes / (ms * 1e-3) / 1e9
    rounds = max(rounds, math.ceil(launches / ncopy)) if launches else rounds
    return {"matrix": label, "fmt": NAMES[fmt], "k": k, "n": n, "us": round(ms * 1e3, 2),
            "bytes": nbytes, "gb_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "copies": ncopy, "launches": ncopy * rounds}


def gemm_record(fmt: int, m: int, n: int, k: int, label: str, rounds: int = 3) -> dict:
    ms, ncopy = time_gemv(fmt, n, k, m, rounds, target=256 << 20)
    flops = 2.0 * m * n * k
    tf = flops / (ms * 1e-3) / 1e12
    peak = MFMA_I8_PEAK_TOPS if fmt == hip.FMT_INT8 else MFMA_F16_PEAK_TFLOPS
    return {"matrix": label, "fmt": NAMES[fmt], "m": m, "k": k, "n": n,
            "us": round(ms * 1e3, 1), "tflops": round(tf, 1), "mfma_frac": round(tf / peak, 4),
            "peak_tflops": peak, "copies": ncopy}


# ---- the BASELINE configurations ------------------------------------------
# config 2: Q4_0 GEMV at LLaMA-3.2-1B shapes (K -> N)
Q4_0_SHAPES = [("q/o 2048->2048", 2048, 2048), ("k/v 2048->512", 2048, 512),
               ("gate/up 2048->8192", 2048, 8192), ("down 8192->2048", 8192, 2048),
               ("lm_head 2048->128256", 2048, 128256)]
# config 1: the INT8 W8A8 GEMVs of one Qwen3-0.6B decode step (q|k|v and
# gate|up stacked as the model runs them)
INT8_QWEN3_SHAPES = [("qkv 1024->4096", 1024, 4096), ("o 2048->1024", 2048, 1024),
                     ("gate|up 1024->6144", 1024, 6144), ("down 3072->1024", 3072, 1024),
                     ("lm_head 1024->151936", 1024, 151936)]
# config 3: LLaMA-3.2-3B Q4_K attention and gate/up, Q6_K down and lm_head
KQ_LLAMA3B_SHAPES = [(hip.FMT_Q4_K, "q/o 3072->3072", 3072, 3072),
                     (hip.FMT_Q4_K, "k/v 3072->1024", 3072, 1024),
                     (hip.FMT_Q4_K, "gate/up 3072->8192", 3072, 8192),
                     (hip.FMT_Q6_K, "down 8192->3072", 8192, 3072),
                     (hip.FMT_Q6_K, "lm_head 3072->128256", 3072, 128256)]
# config 4: Mistral-7B Q8_0 prefill GEMMs
Q8_0_MISTRAL = [("q 4096->4096", 4096, 4096, 1), ("k/v 4096->1024", 4096, 1024, 2),
                ("gate/up 4096->14336", 4096, 14336, 2), ("down 14336->4096", 14336, 4096, 1)]


def ternary_suite(rounds: int = 4) -> list:
    """TernaryLinear GEMVs at the LLaMA-3.2-1B shapes of config 2 (0.5 B/weight)."""
    return [gemv_record(hip.FMT_TERNARY, n, k, lab, rounds) for lab, k, n in Q4_0_SHAPES]


def q4_0_suite(rounds: int = 4, launches: int = 1000) -> list:
    """Config 2: each matrix at `launches` launches (1000, the configuration's
    iteration count), round-robin over >= 1 GiB of weight copies."""
    return [gemv_record(hip.FMT_Q4_0, n, k, lab, rounds, launches) for lab, k, n in Q4_0_SHAPES]


def int8_suite(rounds: int = 4) -> list:
    return [gemv_record(hip.FMT_INT8, n, k, lab, rounds) for lab, k, n in INT8_QWEN3_SHAPES]


def kquant_suite(rounds: int = 4) -> list:
    return [gemv_record(f, n, k, lab, rounds) for f, lab, k, n in KQ_LLAMA3B_SHAPES]


def q8_0_prefill_suite(m: int, rounds: int = 3) -> dict:
    """One Mistral-7B matrix set (q, k, v, gate, up, down: 201,326,592 weights) at M
    tokens: per-matrix records and the set's aggregate TFLOP/s."""
    recs = [gemm_record(hip.FMT_Q8_0, m, n, k, lab, rounds) for lab, k, n, _ in Q8_0_MISTRAL]
    total_flops = sum(2.0 * m * r["n"] * r["k"] * cnt
                      for r, (_, _, _, cnt) in zip(recs, Q8_0_MISTRAL))
    total_s = sum(r["us"] * 1e-6 * cnt for r, (_, _, _, cnt) in zip(recs, Q8_0_MISTRAL))
    tf = total_flops / total_s / 1e12
    return {"note": "whole QLinear calls: f32->f16 activation conversion kernel + GEMM kernel",
            "m": m, "gflop": round(total_flops / 1e9, 2), "ms": round(total_s * 1e3, 3),
            "tflops": round(tf, 1), "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
            "matrices": recs}


def int8_prefill_record(m: int = 128, k: int = 1024, n: int = 3072) -> dict:
    """The reference's published INT8 prefill GEMM shape (128x1024 -> 3072)."""
    return gemm_record(hip.FMT_INT8, m, n, k, f"int8 prefill {m}x{k}->{n}")


def copy_calibration(nbytes: int, reps: int = 3) -> float:
    """Device-to-device copies of `nbytes` (the runtime's copy kernel): the
    known traffic that scales FETCH_SIZE / WRITE_SIZE counter readings."""
    src = hip.DeviceBuffer(nbytes)
    dst = hip.DeviceBuffer(nbytes)
    src.zero()
    t = hip.Timer()
    t.start()
    for _ in range(reps):
        hip.check(hip.lib().syn_hip_memcpy_d2d(dst.ptr, src.ptr, nbytes), "d2d")
    t.stop()
    ms = t.ms() / reps
    src.close()
    dst.close()
    return ms


FMT_BY_NAME = {v: k for k, v in NAMES.items()}


def _decoder_run(which: str, steps: int, graph: bool):
    """Prefill + `steps` decode steps of a BASELINE decoder (for profilers:
    graph=False launches the step's kernels eagerly)."""
    import bench  # the configs and prompt ids of the benchmark
    if which == "klm":
        cfg = dict(bench.LLAMA3B, max_seq=256 + steps + 1)
        m = hip.KQuantCausalLM(cfg)
        m.init_synthetic(bench.SEED_BASE, 0.02)
        m.set_options(graph=graph)
        ids = np.array(bench._ids(256, cfg["vocab"], bench.PROMPT_SEED), np.uint32)
        pf, dec = m.time(ids, steps)
        m.close()
        return {"decoder": "klm", "prefill_ms": round(pf, 3), "decode_ms_per_token": round(dec / steps, 4)}
    if which in ("hlm", "hlm-op"):  # the fused step, or the op-by-op one
        hc = dict(bench.LFM25, max_seq=8 + steps + 1)
        hm = hip.HybridLM(hc)
        hm.init_synthetic(bench.SEED_BASE, 0.02)
        hm.set_options(fused=which == "hlm", graph=graph)
        hm.prefill(np.array(bench._ids(8, hc["vocab"], bench.PROMPT_SEED), np.uint32))
        ms = hm.decode_timed(steps)
        fused = hm.fused_active
        hm.close()
        return {"decoder": which, "fused": fused, "decode_ms_per_token": round(ms / steps, 4)}
    xdt = which == "mamba-int8"
    mc = dict(bench.MAMBA370M, max_tokens=64 + steps + 1)
    mm = hip.QuantizedMamba(mc, int8_xdt=xdt)
    mm.init_synthetic(bench.SEED_BASE, 0.02)
    mm.set_options(fused=True, graph=graph)
    mm.prefill(np.array(bench._ids(64, mc["vocab"], bench.PROMPT_SEED), np.uint32))
    ms = mm.decode_timed(steps)
    mm.close()
    return {"decoder": which, "decode_ms_per_token": round(ms / steps, 4)}


# kernel kinds of the decode-step timeline (decode_fused.hip SYN_TL_EXIT ids)
TL_KINDS = {0: "qkv", 1: "o", 5: "down", 2: "down_swiglu", 10: "gate_up", 3: "in_proj",
            6: "x_proj", 20: "attention", 30: "zero", 31: "final_norm", 32: "lm_head",
            33: "select"}


def qwen3_timeline(steps_before: int = 20, graph: bool = True) -> dict:
    """One Qwen3 INT8 decode step after the 16-token prompt and
    `steps_before` steps: for every kernel kind the mean period (start of its
    workgroup (0, 0) to the next kernel's) and workgroup (0, 0)'s time in the
    kernel, from s_memrealtime stamps (the instrumented build:
    `python -m synapse_amd.build --phase-timing`, loaded with
    SYN_HIP_LIBRARY=synapse_amd/libsynapse_hip_pt.so)."""
    import ctypes as C
    import bench
    L = hip.lib()
    if not hasattr(L, "syn_hip_debug_timeline"):
        raise RuntimeError("timeline: load the phase-timing build (SYN_HIP_LIBRARY)")
    L.syn_hip_debug_timeline.restype = C.c_int
    L.syn_hip_debug_phase_ts.restype = C.c_int
    cfg = dict(bench.QWEN3, max_seq=bench.PROMPT + steps_before + 8)
    m = hip.QuantizedCausalLM(cfg)
    m.init_synthetic(bench.SEED_BASE, 0.02)
    m.set_options(fused=True, graph=graph)
    m.prefill(np.array(bench.prompt_ids(), np.uint32))
    m.decode_timed(steps_before)
    buf = (C.c_uint64 * (3 * 8192))()
    n = C.c_int()
    hip.check(L.syn_hip_debug_timeline(buf, 8192, C.byref(n)), "timeline")  # clears the ring
    ms = m.decode_timed(1)
    hip.check(L.syn_hip_debug_timeline(buf, 8192, C.byref(n)), "timeline")
    t = np.array(buf[:3 * n.value], np.int64).reshape(-1, 3)
    t = t[np.argsort(t[:, 1], kind="stable")]
    agg = {}
    for i in range(len(t) - 1):
        k = TL_KINDS.get(int(t[i, 0]), str(int(t[i, 0])))
        a = agg.setdefault(k, [0, 0, 0])
        a[0] += 1
        a[1] += (t[i + 1, 1] - t[i, 1]) * 10  # 100 MHz ticks -> ns
        a[2] += (t[i, 2] - t[i, 1]) * 10
    ph = (C.c_uint64 * 256)()
    hip.check(L.syn_hip_debug_phase_ts(ph, 256), "phase_ts")
    attn = [int(ph[48 + i] - ph[48]) for i in range(12)]  # k_attn_head stamps, core clocks
    m.close()
    return {"position": bench.PROMPT + steps_before, "graph": graph, "step_ms": round(ms, 4),
            "kernels": int(n.value), "span_us": round(float(t[-1, 2] - t[0, 1]) / 100.0, 2),
            "per_kind": {k: {"launches": v[0], "period_us": round(v[1] / v[0] / 1e3, 3),
                             "wg0_us": round(v[2] / v[0] / 1e3, 3)} for k, v in agg.items()},
            "attention_phase_clocks": attn}


if __name__ == "__main__":
    import json
    import sys

    hip.init(0)
    a = sys.argv[1:]
    if len(a) == 2 and a[0] == "copy":
        n = int(a[1])
        ms = copy_calibration(n)
        print(json.dumps({"copy_bytes": n, "ms": round(ms, 4),
                          "gb_s_read_plus_write": round(2 * n / (ms * 1e-3) / 1e9, 1)}))
    elif len(a) == 1 and a[0] == "sync":  # what a dependency level of the step costs
        rec = {"graph_kernel_us": {w: round(hip.probe_graph_floor(140, w), 3)
                                   for w in (32, 256, 512)}}
        for mode in (0, 1, 2, 3):
            for w in (64, 128, 256):
                us, to = hip.probe_grid_barrier(w, mode, 200)
                rec[f"barrier_mode{mode}_{w}wg_us"] = round(us, 3) if not to else f"{to} timeouts"
        print(json.dumps(rec))
    elif len(a) in (1, 2) and a[0] == "timeline":  # the phase-timing build's step timeline
        print(json.dumps(qwen3_timeline(int(a[1]) if len(a) == 2 else 20)))
    elif len(a) == 4 and a[0] == "gemv":  # gemv FMT N K
        print(json.dumps(gemv_record(FMT_BY_NAME[a[1]], int(a[2]), int(a[3]), "gemv")))
    elif len(a) == 5 and a[0] == "gemm":  # gemm FMT M N K
        print(json.dumps(gemm_record(FMT_BY_NAME[a[1]], int(a[2]), int(a[3]), int(a[4]), "gemm")))
    elif len(a) in (2, 3) and a[0] in ("klm", "mamba-ref", "mamba-int8", "hlm", "hlm-op"):  # DECODER STEPS [eager]
        print(json.dumps(_decoder_run(a[0], int(a[1]), graph=not (len(a) == 3 and a[2] == "eager"))))
    else:
        print("usage: python -m synapse_amd.microbench copy NBYTES | sync | timeline [STEPS] | gemv FMT N K | "
              "gemm FMT M N K | {klm,mamba-ref,mamba-int8,hlm,hlm-op} STEPS [eager]", file=sys.stderr)
        sys.exit(2)
