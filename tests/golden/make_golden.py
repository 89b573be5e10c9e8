"""Writes the golden fixtures of the quantized-linear path (tests/golden/*.npz).

The reference's own hot path (Zig cpu_simd kernels + Rust drivers) cannot be
built in this image, so the expected outputs come from the C restatement in
oracle/oracle.c, whose functions are pinned separately against the
reference's known-answer tests (tests/test_oracle.py).  The fixtures freeze
those outputs: the CPU suite checks that the oracle still reproduces them bit
for bit, and the GPU suite checks the HIP path against the same files.

Inputs are either stored (when small) or regenerated from the SplitMix64 /
Box-Muller seed spec (oracle.normal, oracle.token_ids); regenerated inputs
carry a SHA-256 of their bytes, so a change of the generator is detected
instead of silently producing other expectations.

Run from the repository root:  python -m tests.golden.make_golden
"""
from __future__ import annotations

import hashlib
import os

import numpy as np

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
SEED = 0x5EED0000

# tiny model shapes (also used by the tests that read the fixtures)
QWEN3_TINY = dict(hidden=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, inter=128,
                  vocab=256, max_seq=48)
QWEN3_TINY_STD = 0.1  # larger than N(0, 0.02) so the greedy tokens vary
MAMBA_TINY = dict(d_model=64, d_inner=128, d_state=16, d_conv=4, dt_rank=8, n_layers=2,
                  vocab=256)
INT8_SHAPES = [(1, 1024, 1024), (1, 1024, 3072), (16, 1024, 2048), (33, 600, 40)]
F16_SCALE = np.array([0x66, 0x1E], np.uint8)  # a finite f16 (about 0.0062), little endian


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def int8_inputs(m: int, k: int, n: int):
    """Activations N(0,1) quantized per row (A1); weights N(0,0.02) quantized
    per output row into [K,N] (A2)."""
    x = O.normal(m * k, SEED + 10 + m * 7 + k, 1.0).reshape(m, k)
    a, sa = O.quantize_per_channel_int8(x)
    w = O.normal(n * k, SEED + 20 + n * 3 + k, 0.02).reshape(n, k)
    b, sb = O.quantize_weights_int8(w)
    return a, sa, b, sb


def q4_inputs(n: int, k: int):
    w = O.normal(n * k, SEED + 30 + n + k, 0.02).reshape(n, k)
    a = O.normal(k, SEED + 40 + k, 1.0)
    return w, a


def kquant_blocks(fmt: str, n_blocks: int, seed: int) -> np.ndarray:
    """Random block bytes with finite f16 scales (every bit of the quant
    fields exercised): Q8_0 34 B / 32, Q4_K 144 B / 256, Q6_K 210 B / 256."""
    size = {"q8_0": 34, "q4_k": 144, "q6_k": 210}[fmt]
    rng = np.random.Generator(np.random.PCG64(seed))
    raw = rng.integers(0, 256, size=(n_blocks, size), dtype=np.uint8)
    if fmt == "q8_0":
        raw[:, 0:2] = F16_SCALE
    elif fmt == "q4_k":
        raw[:, 0:2] = F16_SCALE
        raw[:, 2:4] = F16_SCALE
    else:
        raw[:, 208:210] = F16_SCALE
    return raw.reshape(-1)


KQ_GEMV = {"q8_0": (8, 512), "q4_k": (8, 512), "q6_k": (8, 512)}  # n, k


def make_quantize():
    x = O.normal(6 * 40, SEED + 1, 3.0).reshape(6, 40)
    x[1] = 0.0                      # zero row: scale 1, q 0
    x[2] = 0.5
    x[2, 0] = 127.0                 # x*inv = 0.5 exactly: round half away from zero
    x[3, 5] = -1e30                 # one huge value dominates the row
    x[4, :] = -x[4, :]              # sign symmetry
    q, s = O.quantize_per_channel_int8(x)
    np.savez(os.path.join(HERE, "quantize_rows.npz"), x=x, q=q, s=s)


def make_int8():
    out = {}
    for m, k, n in INT8_SHAPES:
        a, sa, b, sb = int8_inputs(m, k, n)
        c = O.qgemm_int8(a, b, sa, sb)
        key = f"{m}x{k}x{n}"
        out[f"{key}_inputs_sha"] = np.array(sha(a, sa, b, sb))
        out[f"{key}_c"] = c
    np.savez_compressed(os.path.join(HERE, "int8_gemm.npz"), **out)


def make_q4():
    out = {}
    for n, k in [(16, 64), (64, 2048)]:
        w, a = q4_inputs(n, k)
        packed = O.q4_pack(w)
        key = f"{n}x{k}"
        out[f"{key}_w_sha"] = np.array(sha(w))
        out[f"{key}_packed_sha"] = np.array(sha(packed))
        if packed.size <= 4096:
            out[f"{key}_packed"] = packed
        out[f"{key}_a"] = a
        out[f"{key}_y"] = O.q4_0_gemv(a, packed, n)
    np.savez_compressed(os.path.join(HERE, "q4_0.npz"), **out)


def make_kquant():
    out = {}
    for i, (fmt, (n, k)) in enumerate(KQ_GEMV.items()):
        per = 32 if fmt == "q8_0" else 256
        blocks = kquant_blocks(fmt, n * k // per, SEED + 50 + i)
        w = O.dequant(fmt, blocks, n * k).reshape(n, k)
        x = O.normal(k, SEED + 60 + i, 1.0)
        out[f"{fmt}_blocks"] = blocks
        out[f"{fmt}_dequant"] = w
        out[f"{fmt}_x"] = x
        out[f"{fmt}_y"] = O.matmul_t(x.reshape(1, k), w).reshape(n)
    np.savez_compressed(os.path.join(HERE, "kquant.npz"), **out)


def make_qwen3_tiny():
    o = O.QuantizedCausalLM(QWEN3_TINY)
    o.init_synthetic(SEED, QWEN3_TINY_STD)
    ids = O.token_ids(8, SEED + 0xFFFF, QWEN3_TINY["vocab"])
    logits = o.prefill(ids)
    o.reset()
    toks, margins = o.generate(ids, 16)
    o.close()
    np.savez(os.path.join(HERE, "qwen3_tiny_w8a8.npz"), prompt=ids, prefill_logits=logits,
             tokens=toks, margins=margins)


def make_mamba_tiny():
    o = O.QuantizedMamba(MAMBA_TINY)
    o.init_synthetic(SEED)
    ids = O.token_ids(8, SEED + 0xFFFF, MAMBA_TINY["vocab"])
    logits = o.prefill(ids)
    o.close()
    o = O.QuantizedMamba(MAMBA_TINY)
    o.init_synthetic(SEED)
    toks, margins = o.generate(ids, 12)
    o.close()
    np.savez(os.path.join(HERE, "mamba_tiny_int8.npz"), prompt=ids, prefill_logits=logits,
             tokens=toks, margins=margins)


def main():
    make_quantize()
    make_int8()
    make_q4()
    make_kquant()
    make_qwen3_tiny()
    make_mamba_tiny()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
