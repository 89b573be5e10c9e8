"""CPU oracle (test infrastructure only).

ctypes binding of ``liboracle.so`` — the plain-C restatement of the
reference's quantized-linear path (see ``oracle.c`` for the per-function
reference citations and the list of parity pins).  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package; the HIP product never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

CFLAGS = ["-O3", "-mavx2", "-mfma", "-mf16c", "-ffp-contract=off", "-fno-fast-math",
          "-fopenmp", "-fPIC", "-shared", "-Wall", "-Wextra"]


def build(verbose: bool = False) -> str:
    """Compile oracle.c into liboracle.so (gcc; x86-64-v3 so it runs on the GPU box host)."""
    cmd = ["gcc", *CFLAGS, "-o", LIB_PATH, os.path.join(HERE, "oracle.c"), "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
SZ = C.c_size_t


class LmCfg(C.Structure):
    _fields_ = [("hidden", SZ), ("n_layers", SZ), ("n_heads", SZ), ("n_kv_heads", SZ),
                ("head_dim", SZ), ("inter", SZ), ("vocab", SZ), ("max_seq", SZ),
                ("eps", C.c_float), ("rope_theta", C.c_double)]


class MambaCfg(C.Structure):
    _fields_ = [("d_model", SZ), ("d_inner", SZ), ("d_state", SZ), ("d_conv", SZ),
                ("dt_rank", SZ), ("n_layers", SZ), ("vocab", SZ), ("eps", C.c_float)]


def _declare(L):
    sig = {
        "orc_fill_normal": (None, [P, SZ, C.c_uint64, C.c_float]),
        "orc_fill_token_ids": (None, [P, SZ, C.c_uint64, C.c_uint32]),
        "orc_f32_to_f16_trunc": (C.c_uint16, [C.c_float]),
        "orc_f16_to_f32_zig": (C.c_float, [C.c_uint16]),
        "orc_f16_to_f32_rs": (C.c_float, [C.c_uint16]),
        "orc_quantize_per_channel_int8": (C.c_int, [P, SZ, SZ, P, P]),
        "orc_minmax_scales": (None, [P, SZ, SZ, P]),
        "orc_quantize_weights_int8": (None, [P, P, SZ, SZ, P]),
        "orc_qgemm_int8": (C.c_int, [SZ, SZ, SZ, P, SZ, P, SZ, P, SZ, P, P]),
        "orc_naive_int8_gemm": (None, [SZ, SZ, SZ, P, SZ, P, SZ, P, SZ, P, P]),
        "orc_q4_packed_bytes": (SZ, [SZ, SZ]),
        "orc_q4_from_f32_packed": (None, [P, SZ, SZ, P]),
        "orc_q4_0_gemv": (C.c_int, [SZ, SZ, P, P, P]),
        "orc_dequant_q4_0": (C.c_int, [P, SZ, P]),
        "orc_dequant_q8_0": (C.c_int, [P, SZ, P]),
        "orc_dequant_q4_k": (C.c_int, [P, SZ, P]),
        "orc_dequant_q6_k": (C.c_int, [P, SZ, P]),
        "orc_sgemm": (C.c_int, [SZ, SZ, SZ, P, SZ, C.c_int, P, SZ, C.c_int, P, SZ]),
        "orc_rmsnorm": (None, [P, P, C.c_float, SZ, SZ, P]),
        "orc_rope_tables": (None, [SZ, SZ, C.c_double, P, P]),
        "orc_rope_apply": (None, [P, P, P, SZ, SZ, SZ, SZ]),
        "orc_silu": (C.c_float, [C.c_float]),
        "orc_expf": (C.c_float, [C.c_float]),
        "orc_softmax_slice": (None, [P, SZ]),
        "orc_argmax": (C.c_uint32, [P, SZ]),
        "orc_repetition_penalty": (None, [P, SZ, P, SZ, C.c_float]),
        "orc_softmax_inplace": (None, [P, SZ]),
        "orc_top_k_filter": (None, [P, SZ, SZ]),
        "orc_top_p_filter": (None, [P, SZ, C.c_float]),
        "orc_sample_combined": (C.c_uint32, [P, SZ, P, SZ, C.c_float, SZ, C.c_float, C.c_float,
                                             C.c_float]),
        "orc_chacha_block": (None, [P, C.c_uint64, C.c_uint64, C.c_int, P]),
        "orc_stdrng_f32": (None, [C.c_uint64, SZ, P]),
        "orc_pcg32_step": (C.c_uint64, [C.c_uint64, C.c_uint64]),
        "orc_pcg32_xsh_rr": (C.c_uint32, [C.c_uint64]),
        "orc_ternary_from_f32": (None, [P, SZ, SZ, P]),
        "orc_ternary_forward": (None, [P, SZ, SZ, P, SZ, P]),
        "orc_attention_decode": (None, [P, P, P, SZ, SZ, SZ, SZ, P]),
        "orc_fused_attention": (C.c_int, [SZ, SZ, SZ, P, P, P, P]),
        "orc_qlm_create": (P, [C.POINTER(LmCfg)]),
        "orc_qlm_destroy": (None, [P]),
        "orc_qlm_set_embed": (C.c_int, [P, P]),
        "orc_qlm_set_layer": (C.c_int, [P, SZ, P, P, P, P, P, P, P]),
        "orc_qlm_init_synthetic": (C.c_int, [P, C.c_uint64, C.c_float]),
        "orc_qlm_finalize": (C.c_int, [P]),
        "orc_qlm_set_norms": (C.c_int, [P, SZ, P, P, P, P]),
        "orc_qlm_set_final_norm": (C.c_int, [P, P]),
        "orc_qlm_set_qk_norm": (None, [P, C.c_int]),
        "orc_qlm_set_lm_head": (C.c_int, [P, P]),
        "orc_qlm_reset": (None, [P]),
        "orc_qlm_cur_len": (SZ, [P]),
        "orc_qlm_prefill": (C.c_int, [P, P, SZ, P]),
        "orc_qlm_prefill_append": (C.c_int, [P, P, SZ, P]),
        "orc_qlm_truncate": (None, [P, SZ]),
        "orc_qlm_forward_one": (C.c_int, [P, C.c_uint32, P]),
        "orc_qlm_generate": (C.c_int, [P, P, SZ, SZ, P, P]),
        "orc_qlm_lm_head_weights": (P, [P]),
        "orc_qlm_lm_head_scales": (P, [P]),
        "orc_flm_create": (P, [C.POINTER(LmCfg), C.c_int]),
        "orc_flm_destroy": (None, [P]),
        "orc_flm_set_embed": (C.c_int, [P, P]),
        "orc_flm_set_proj": (C.c_int, [P, SZ, C.c_int, C.c_int, P]),
        "orc_flm_set_lm_head": (C.c_int, [P, C.c_int, P]),
        "orc_flm_reset": (None, [P]),
        "orc_flm_set_norms": (C.c_int, [P, C.c_size_t, P, P, P, P]),
        "orc_flm_set_final_norm": (C.c_int, [P, P]),
        "orc_flm_prefill": (C.c_int, [P, P, SZ, P]),
        "orc_flm_prefill_append": (C.c_int, [P, P, SZ, P]),
        "orc_flm_truncate": (None, [P, SZ]),
        "orc_flm_cur_len": (SZ, [P]),
        "orc_flm_forward_one_draft": (C.c_int, [P, C.c_uint32, SZ, P]),
        "orc_flm_forward_one": (C.c_int, [P, C.c_uint32, P]),
        "orc_flm_generate": (C.c_int, [P, P, SZ, SZ, P, P]),
        "orc_swiglu_fused": (None, [P, P, P, SZ]),
        "orc_mamba_create": (P, [C.POINTER(MambaCfg)]),
        "orc_mamba_destroy": (None, [P]),
        "orc_mamba_init_synthetic": (C.c_int, [P, C.c_uint64]),
        "orc_mamba_init_synthetic_std": (C.c_int, [P, C.c_uint64, C.c_float]),
        "orc_mamba_reset": (None, [P]),
        "orc_mamba_set_int8_xdt": (C.c_int, [P]),
        "orc_mamba_prefill": (C.c_int, [P, P, SZ, P]),
        "orc_mamba_decode_one": (C.c_int, [P, C.c_uint32, P]),
        "orc_mamba_generate": (C.c_int, [P, P, SZ, SZ, P, P]),
        "orc_hlm_create": (P, [P]),
        "orc_hlm_destroy": (None, [P]),
        "orc_hlm_init_synthetic": (C.c_int, [P, C.c_uint64, C.c_float]),
        "orc_hlm_reset": (None, [P]),
        "orc_hlm_pos": (SZ, [P]),
        "orc_hlm_conv_step": (None, [P, SZ, SZ, P, P, P, P]),
        "orc_hlm_decode_one": (C.c_int, [P, C.c_uint32, P]),
        "orc_hlm_generate": (C.c_int, [P, P, SZ, SZ, P, P]),
        "orc_softplus": (C.c_float, [C.c_float]),
        "orc_conv1d_step": (None, [P, P, P, P, SZ, SZ, P]),
        "orc_set_threads": (None, [C.c_int]),
        "orc_get_threads": (C.c_int, []),
        "orc_rmsnorm_seq": (None, [P, P, C.c_float, SZ, P]),
        "orc_selective_scan_step": (None, [P, P, P, P, P, P, P, P, SZ, SZ]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle needs C-contiguous arrays"
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- inputs
def normal(n: int, seed: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(_p(out), n, seed, std)
    return out


def token_ids(n: int, seed: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().orc_fill_token_ids(_p(out), n, seed, vocab)
    return out


# ---------------------------------------------------------------- A1/A2
def quantize_per_channel_int8(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    rc = lib().orc_quantize_per_channel_int8(_p(x), m, k, _p(q), _p(s))
    if rc:
        raise ValueError(f"orc_quantize_per_channel_int8 status {rc}")
    return q, s


def quantize_weights_int8(w: np.ndarray):
    """QuantizedLinear::from_f32: w [N,K] f32 -> (weights_int8 [K,N], scales [N])."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    s = np.empty(n, np.float32)
    q = np.empty((k, n), np.int8)
    lib().orc_minmax_scales(_p(w), n, k, _p(s))
    lib().orc_quantize_weights_int8(_p(w), _p(s), n, k, _p(q))
    return q, s


def qgemm_int8(a: np.ndarray, b_kn: np.ndarray, sa: np.ndarray, sb: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.int8)
    b_kn = np.ascontiguousarray(b_kn, np.int8)
    m, k = a.shape
    k2, n = b_kn.shape
    assert k == k2
    c = np.zeros((m, n), np.float32)
    sa = np.ascontiguousarray(sa, np.float32)
    sb = np.ascontiguousarray(sb, np.float32)
    rc = lib().orc_qgemm_int8(m, n, k, _p(a), k, _p(b_kn), n, _p(c), n, _p(sa), _p(sb))
    if rc:
        raise ValueError(f"orc_qgemm_int8 status {rc}")
    return c


def naive_int8_gemm(a, b_kn, sa, sb):
    a = np.ascontiguousarray(a, np.int8)
    b_kn = np.ascontiguousarray(b_kn, np.int8)
    m, k = a.shape
    n = b_kn.shape[1]
    c = np.zeros((m, n), np.float32)
    sa = np.ascontiguousarray(sa, np.float32)
    sb = np.ascontiguousarray(sb, np.float32)
    lib().orc_naive_int8_gemm(m, n, k, _p(a), k, _p(b_kn), n, _p(c), n, _p(sa), _p(sb))
    return c


# ---------------------------------------------------------------- Q4_0
def q4_pack(w: np.ndarray) -> np.ndarray:
    """Q4Linear::from_f32 + pack_for_zig: w [N,K] -> bytes [N * ceil(K/32) * 18]."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    out = np.empty(lib().orc_q4_packed_bytes(n, k), np.uint8)
    lib().orc_q4_from_f32_packed(_p(w), n, k, _p(out))
    return out


def q4_0_gemv(a: np.ndarray, packed: np.ndarray, n: int) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    packed = np.ascontiguousarray(packed, np.uint8)
    c = np.zeros(n, np.float32)
    rc = lib().orc_q4_0_gemv(n, a.shape[0], _p(a), _p(packed), _p(c))
    if rc:
        raise ValueError(f"orc_q4_0_gemv status {rc}")
    return c


# ---------------------------------------------------------------- GGUF dequant
def dequant(fmt: str, data: np.ndarray, numel: int) -> np.ndarray:
    data = np.ascontiguousarray(data, np.uint8)
    out = np.empty(numel, np.float32)
    fn = {"q4_0": lib().orc_dequant_q4_0, "q8_0": lib().orc_dequant_q8_0,
          "q4_k": lib().orc_dequant_q4_k, "q6_k": lib().orc_dequant_q6_k}[fmt]
    rc = fn(_p(data), numel, _p(out))
    if rc:
        raise ValueError(f"dequant {fmt} status {rc}")
    return out


# ---------------------------------------------------------------- f32 GEMM
def sgemm(a: np.ndarray, b: np.ndarray, trans_a: bool = False, trans_b: bool = False,
          c: np.ndarray = None) -> np.ndarray:
    """syn_sgemm / sgemmTiled (exports.zig:725-761, matmul.zig:125-184)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = (a.shape[1], a.shape[0]) if trans_a else a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    out = np.zeros((m, n), np.float32) if c is None else np.array(c, np.float32, copy=True)
    rc = lib().orc_sgemm(m, n, k, _p(a), a.shape[1], int(trans_a), _p(b), b.shape[1],
                         int(trans_b), _p(out), n)
    if rc:
        raise ValueError(f"orc_sgemm status {rc}")
    return out


def matmul_t(a: np.ndarray, w_nk: np.ndarray) -> np.ndarray:
    """ops/matmul.rs:55-79: a [M,K] x W[N,K]^T via syn_sgemm(trans_b=1)."""
    a = np.ascontiguousarray(a, np.float32)
    w_nk = np.ascontiguousarray(w_nk, np.float32)
    m, k = a.shape
    n = w_nk.shape[0]
    c = np.zeros((m, n), np.float32)
    rc = lib().orc_sgemm(m, n, k, _p(a), k, 0, _p(w_nk), k, 1, _p(c), n)
    if rc:
        raise ValueError(f"orc_sgemm status {rc}")
    return c


# ---------------------------------------------------------------- ops
def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, h = x.shape
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(np.ascontiguousarray(w, np.float32)), eps, rows, h, _p(out))
    return out


def rope_tables(max_pos: int, head_dim: int, base: float):
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_tables(max_pos, head_dim, base, _p(c), _p(s))
    return c, s


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().orc_argmax(_p(x), x.size))


# ---------------------------------------------------------------- sampling
def repetition_penalty(logits: np.ndarray, history, penalty: float) -> np.ndarray:
    x = np.array(logits, np.float32, copy=True)
    h = np.ascontiguousarray(history, np.uint32)
    lib().orc_repetition_penalty(_p(x), x.size, _p(h), h.size, penalty)
    return x


def softmax(logits: np.ndarray) -> np.ndarray:
    x = np.array(logits, np.float32, copy=True)
    lib().orc_softmax_inplace(_p(x), x.size)
    return x


def top_k_filter(logits: np.ndarray, k: int) -> np.ndarray:
    x = np.array(logits, np.float32, copy=True)
    lib().orc_top_k_filter(_p(x), x.size, k)
    return x


def top_p_filter(logits: np.ndarray, p: float) -> np.ndarray:
    x = np.array(logits, np.float32, copy=True)
    lib().orc_top_p_filter(_p(x), x.size, p)
    return x


def sample_combined(logits: np.ndarray, history=(), temperature: float = 1.0, top_k: int = 0,
                    top_p: float = 1.0, repetition_penalty: float = 1.0, u: float = 0.5) -> int:
    """CombinedSampler::sample_with_history with the uniform draw u given."""
    x = np.array(logits, np.float32, copy=True)
    h = np.ascontiguousarray(np.asarray(history, np.uint32).reshape(-1))
    if h.size == 0:
        h = np.zeros(1, np.uint32)
        nh = 0
    else:
        nh = h.size
    return int(lib().orc_sample_combined(_p(x), x.size, _p(h), nh, temperature, top_k, top_p,
                                         repetition_penalty, u))


def chacha_block(key, counter: int, stream: int, rounds: int) -> np.ndarray:
    k = np.ascontiguousarray(key, np.uint32)
    out = np.zeros(16, np.uint32)
    lib().orc_chacha_block(_p(k), counter, stream, rounds, _p(out))
    return out


def pcg32_step(state: int, inc: int) -> int:
    """PCG32's LCG step: state * 6364136223846793005 + inc (mod 2^64)."""
    return int(lib().orc_pcg32_step(state, inc))


def pcg32_xsh_rr(state: int) -> int:
    """PCG32's XSH-RR output of a 64-bit state."""
    return int(lib().orc_pcg32_xsh_rr(state))


def stdrng_f32(seed: int, n: int) -> np.ndarray:
    """The first n draws of StdRng::seed_from_u64(seed).gen::<f32>()."""
    out = np.zeros(n, np.float32)
    lib().orc_stdrng_f32(seed, n, _p(out))
    return out


# ---------------------------------------------------------------- ternary
def ternary_from_f32(w: np.ndarray) -> np.ndarray:
    """TernaryLinear::from_f32: w [N,K] -> blocks [N * ceil(K/16) * 8] bytes
    (f32 scale, then 4 code bytes, per block of 16 weights)."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    out = np.zeros(n * ((k + 15) // 16) * 8, np.uint8)
    lib().orc_ternary_from_f32(_p(w), n, k, _p(out))
    return out


def ternary_forward(blocks: np.ndarray, n: int, k: int, x: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8)
    x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
    y = np.zeros((x.shape[0], n), np.float32)
    lib().orc_ternary_forward(_p(blocks), n, k, _p(x), x.shape[0], _p(y))
    return y


def expf(x: float) -> float:
    return float(lib().orc_expf(x))


def silu(x: float) -> float:
    return float(lib().orc_silu(x))


def fused_attention(q, k, v):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    sq, d = q.shape
    sk = k.shape[0]
    out = np.zeros((sq, d), np.float32)
    lib().orc_fused_attention(sq, sk, d, _p(q), _p(k), _p(v), _p(out))
    return out


def attention_decode(q, kcache, vcache, seq_len, n_heads, n_kv, head_dim):
    q = np.ascontiguousarray(q, np.float32)
    out = np.zeros(n_heads * head_dim, np.float32)
    lib().orc_attention_decode(_p(q), _p(np.ascontiguousarray(kcache, np.float32)),
                               _p(np.ascontiguousarray(vcache, np.float32)), seq_len,
                               n_heads, n_kv, head_dim, _p(out))
    return out


# ---------------------------------------------------------------- A15 model
def set_threads(n: int):
    """OpenMP threads of the oracle's large f32 products (the values do not
    depend on it; 1 times the reference's single-threaded kernels)."""
    lib().orc_set_threads(int(n))


def conv1d_step(x: np.ndarray, w: np.ndarray, bias: np.ndarray, state: np.ndarray) -> np.ndarray:
    """QuantizedMambaBlock::conv1d_step (int8_mamba.rs:43-56); state
    [d_inner, d_conv] is updated in place."""
    d_inner, d_conv = state.shape
    assert state.dtype == np.float32 and state.flags.c_contiguous
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    out = np.empty(d_inner, np.float32)
    lib().orc_conv1d_step(_p(x), _p(w), _p(bias), _p(state), d_inner, d_conv, _p(out))
    return out


def swiglu_fused(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    out = np.empty_like(gate)
    lib().orc_swiglu_fused(_p(out), _p(gate), _p(up), gate.size)
    return out


class QuantizedCausalLM:
    """INT8 W8A8 decoder (quantization/lm/int8.rs) restated in C."""

    def __init__(self, cfg: dict):
        self.cfg = cfg
        c = LmCfg(cfg["hidden"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                  cfg["head_dim"], cfg["inter"], cfg["vocab"], cfg["max_seq"],
                  cfg.get("eps", 1e-6), cfg.get("rope_theta", 1e6))
        self._c = c
        self.h = lib().orc_qlm_create(C.byref(c))
        if not self.h:
            raise MemoryError("orc_qlm_create failed")

    def init_synthetic(self, seed_base: int = 0x5EED0000, std: float = 0.02):
        rc = lib().orc_qlm_init_synthetic(self.h, seed_base, std)
        if rc:
            raise RuntimeError(f"orc_qlm_init_synthetic status {rc}")
        self._check(lib().orc_qlm_finalize(self.h))

    def set_weights(self, embed: np.ndarray, layers: list, final_norm=None, lm_head=None,
                    qk_norm: bool = True):
        self._keep = [embed]
        self._check(lib().orc_qlm_set_embed(self.h, _p(np.ascontiguousarray(embed, np.float32))))
        lib().orc_qlm_set_qk_norm(self.h, int(qk_norm))
        for i, lw in enumerate(layers):
            arrs = [np.ascontiguousarray(lw[n], np.float32)
                    for n in ("q", "k", "v", "o", "gate", "up", "down")]
            self._check(lib().orc_qlm_set_layer(self.h, i, *[_p(a) for a in arrs]))
            gains = [None if lw.get(n) is None else np.ascontiguousarray(lw[n], np.float32)
                     for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm")]
            self._check(lib().orc_qlm_set_norms(self.h, i, *[None if g is None else _p(g)
                                                             for g in gains]))
        if final_norm is not None:
            self._check(lib().orc_qlm_set_final_norm(
                self.h, _p(np.ascontiguousarray(final_norm, np.float32))))
        if lm_head is not None:
            self._check(lib().orc_qlm_set_lm_head(
                self.h, _p(np.ascontiguousarray(lm_head, np.float32))))
        self._check(lib().orc_qlm_finalize(self.h))

    @staticmethod
    def _check(rc):
        if rc:
            raise RuntimeError(f"oracle status {rc}")

    def reset(self):
        lib().orc_qlm_reset(self.h)

    def prefill(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.uint32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        self._check(lib().orc_qlm_prefill(self.h, _p(ids), ids.size, _p(logits)))
        return logits

    def forward_one(self, token: int) -> np.ndarray:
        logits = np.empty(self.cfg["vocab"], np.float32)
        self._check(lib().orc_qlm_forward_one(self.h, int(token), _p(logits)))
        return logits

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        self._check(lib().orc_qlm_generate(self.h, _p(prompt), prompt.size, max_new,
                                           _p(toks), _p(margins)))
        return toks, margins

    def prefill_append(self, ids) -> np.ndarray:
        """forward_prefill into the cache as it stands (int8.rs:593-635 with
        cached_attention_prefill, ops/attention.rs:153-247)."""
        ids = np.ascontiguousarray(ids, np.uint32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        self._check(lib().orc_qlm_prefill_append(self.h, _p(ids), ids.size, _p(logits)))
        return logits

    def truncate(self, new_len: int):
        """KvCache.truncateTo (kvcache.zig:109-113)."""
        lib().orc_qlm_truncate(self.h, new_len)

    def cache_len(self) -> int:
        return int(lib().orc_qlm_cur_len(self.h))

    def generate_speculative(self, prompt, max_new: int, k: int, sampler=None, seed: int = 0):
        """generate_speculative (generation/pipeline.rs:281-395).
        QuantizedCausalLM has no forward_one_draft (int8.rs:739), so the trait
        default (models/traits.rs:64-68) drafts with forward_one."""
        return speculative_loop(self, prompt, max_new, k, self.forward_one, sampler, seed)

    def close(self):
        if self.h:
            lib().orc_qlm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


FMT_CODES = {"q8_0": 3, "q4_k": 4, "q6_k": 5}


class CausalLM:
    """f32 decoder over GGUF-dequantized weights (models/lm/causal_lm.rs)."""

    def __init__(self, cfg: dict, qk_norm: bool = False):
        self.cfg = cfg
        c = LmCfg(cfg["hidden"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                  cfg["head_dim"], cfg["inter"], cfg["vocab"], cfg["max_seq"],
                  cfg.get("eps", 1e-5), cfg.get("rope_theta", 5e5))
        self._c = c
        self.h = lib().orc_flm_create(C.byref(c), 1 if qk_norm else 0)
        if not self.h:
            raise MemoryError("orc_flm_create failed")

    def _check(self, rc):
        if rc:
            raise RuntimeError(f"oracle status {rc}")

    def set_embed(self, embed):
        self._check(lib().orc_flm_set_embed(self.h, _p(np.ascontiguousarray(embed, np.float32))))

    def set_proj(self, layer: int, proj: int, fmt: str, blocks: np.ndarray):
        self._check(lib().orc_flm_set_proj(self.h, layer, proj, FMT_CODES[fmt],
                                           _p(np.ascontiguousarray(blocks, np.uint8))))

    def set_lm_head(self, fmt: str, blocks: np.ndarray):
        self._check(lib().orc_flm_set_lm_head(self.h, FMT_CODES[fmt],
                                              _p(np.ascontiguousarray(blocks, np.uint8))))

    def set_norms(self, layer: int, attn=None, ffn=None, q=None, k=None):
        arrs = [None if a is None else np.ascontiguousarray(a, np.float32)
                for a in (attn, ffn, q, k)]
        self._check(lib().orc_flm_set_norms(self.h, layer,
                                            *[None if a is None else _p(a) for a in arrs]))

    def set_final_norm(self, gain):
        self._check(lib().orc_flm_set_final_norm(self.h,
                                                 _p(np.ascontiguousarray(gain, np.float32))))

    def reset(self):
        lib().orc_flm_reset(self.h)

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32)
        self._check(lib().orc_flm_prefill(self.h, _p(ids), ids.size, _p(out)))
        return out

    def forward_one(self, token: int):
        out = np.empty(self.cfg["vocab"], np.float32)
        self._check(lib().orc_flm_forward_one(self.h, int(token), _p(out)))
        return out

    def forward_one_draft(self, token: int, n_draft: int):
        """CausalLM::forward_one_draft (causal_lm.rs:283-323)."""
        out = np.empty(self.cfg["vocab"], np.float32)
        self._check(lib().orc_flm_forward_one_draft(self.h, int(token), n_draft, _p(out)))
        return out

    def prefill_append(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32)
        self._check(lib().orc_flm_prefill_append(self.h, _p(ids), ids.size, _p(out)))
        return out

    def truncate(self, new_len: int):
        lib().orc_flm_truncate(self.h, new_len)

    def cache_len(self) -> int:
        return int(lib().orc_flm_cur_len(self.h))

    def generate_speculative(self, prompt, max_new: int, k: int, draft_layers: int = 0):
        """generate_speculative (pipeline.rs:281-395), greedy: drafts from the
        first draft_layers layers (0: num_layers / 3, pipeline.rs:28, 295-299)."""
        n = draft_layers if draft_layers > 0 else self.cfg["n_layers"] // 3
        return speculative_loop(self, prompt, max_new, k,
                                lambda t: self.forward_one_draft(t, n))

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        self._check(lib().orc_flm_generate(self.h, _p(prompt), prompt.size, max_new, _p(toks),
                                           _p(margins)))
        return toks, margins

    def close(self):
        if self.h:
            lib().orc_flm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HlmCfg(C.Structure):
    _fields_ = [("hidden", SZ), ("n_layers", SZ), ("vocab", SZ), ("n_heads", SZ),
                ("n_kv_heads", SZ), ("head_dim", SZ), ("inner", SZ), ("conv_kernel", SZ),
                ("inter", SZ), ("max_seq", SZ), ("eps", C.c_float), ("rope_theta", C.c_float),
                ("conv_bias", C.c_int), ("layer_kinds", C.c_uint8 * 64)]


# LFM2.5-350M (models/ssm/hybrid/config.rs:132-156): C = LIV conv (0), A = GQA (1)
LFM25_KINDS = [0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 1, 0, 1, 0, 1, 0]
LFM25_350M = dict(hidden=1024, n_layers=16, vocab=65536, n_heads=16, n_kv_heads=8, head_dim=64,
                  inner=1024, conv_kernel=3, inter=6656, eps=1e-5, rope_theta=1e6,
                  layer_kinds=LFM25_KINDS)


def hlm_cfg(cfg: dict) -> HlmCfg:
    kinds = (C.c_uint8 * 64)(*cfg["layer_kinds"])
    return HlmCfg(cfg["hidden"], cfg["n_layers"], cfg["vocab"], cfg["n_heads"],
                  cfg["n_kv_heads"], cfg["head_dim"], cfg["inner"], cfg["conv_kernel"],
                  cfg["inter"], cfg["max_seq"], cfg.get("eps", 1e-5), cfg.get("rope_theta", 1e6),
                  int(cfg.get("conv_bias", 0)), kinds)


class HybridLM:
    """Hybrid LFM2.5 decoder, Q4 decode path (models/ssm/hybrid) restated in C."""

    def __init__(self, cfg: dict):
        self.cfg = cfg
        self._c = hlm_cfg(cfg)
        self.h = lib().orc_hlm_create(C.byref(self._c))
        if not self.h:
            raise ValueError("orc_hlm_create: unsupported configuration")

    def init_synthetic(self, seed_base: int = 0x5EED0000, std: float = 0.02):
        if lib().orc_hlm_init_synthetic(self.h, seed_base, std):
            raise RuntimeError("orc_hlm_init_synthetic failed")

    def reset(self):
        lib().orc_hlm_reset(self.h)

    @property
    def pos(self) -> int:
        return lib().orc_hlm_pos(self.h)

    def decode_one(self, token: int):
        out = np.empty(self.cfg["vocab"], np.float32)
        if lib().orc_hlm_decode_one(self.h, int(token), _p(out)):
            raise RuntimeError("orc_hlm_decode_one failed (cache full?)")
        return out

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        if lib().orc_hlm_generate(self.h, _p(prompt), prompt.size, max_new, _p(toks),
                                  _p(margins)):
            raise RuntimeError("orc_hlm_generate failed")
        return toks, margins

    def close(self):
        if self.h:
            lib().orc_hlm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def hlm_conv_step(proj, inner: int, ck: int, state, w, bias=None):
    """orc_hlm_conv_step: one LIV double-gated conv step; updates `state` in place."""
    proj = np.ascontiguousarray(proj, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty(inner, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_hlm_conv_step(_p(proj), inner, ck, _p(state), _p(w), None if b is None else _p(b),
                            _p(out))
    return out


class QuantizedMamba:
    """INT8 Mamba (quantization/ssm/int8_mamba.rs) restated in C."""

    def __init__(self, cfg: dict):
        self.cfg = cfg
        c = MambaCfg(cfg["d_model"], cfg["d_inner"], cfg["d_state"], cfg["d_conv"],
                     cfg["dt_rank"], cfg["n_layers"], cfg["vocab"], cfg.get("eps", 1e-5))
        self._c = c
        self.h = lib().orc_mamba_create(C.byref(c))

    def init_synthetic(self, seed_base: int = 0x5EED0000, std: float = 0.02):
        """std: the projections' and conv taps' (the embedding keeps 0.02)"""
        if lib().orc_mamba_init_synthetic_std(self.h, seed_base, std):
            raise RuntimeError("orc_mamba_init_synthetic failed")

    def set_int8_xdt(self):
        """BASELINE config 5's variant: x_proj and dt_proj quantized by
        QuantizedLinear::from_f32 and run through its forward (the reference
        keeps them f32, int8_mamba.rs:33-34)"""
        if lib().orc_mamba_set_int8_xdt(self.h):
            raise RuntimeError("orc_mamba_set_int8_xdt failed")

    def reset(self):
        lib().orc_mamba_reset(self.h)

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32)
        lib().orc_mamba_prefill(self.h, _p(ids), ids.size, _p(out))
        return out

    def decode_one(self, token: int):
        out = np.empty(self.cfg["vocab"], np.float32)
        lib().orc_mamba_decode_one(self.h, int(token), _p(out))
        return out

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        lib().orc_mamba_generate(self.h, _p(prompt), prompt.size, max_new, _p(toks), _p(margins))
        return toks, margins

    def close(self):
        if self.h:
            lib().orc_mamba_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def speculative_loop(model, prompt, max_new: int, k: int, draft, sampler=None, seed: int = 0):
    """TextGenerator::generate_speculative (generation/pipeline.rs:281-395)
    with max_new_tokens as the only stop condition.  model: prefill,
    prefill_append, forward_one, truncate, cache_len; draft(token) -> logits
    is the model's forward_one_draft.  sampler: None (GreedySampler) or
    CombinedSampler settings (sample_combined keywords), fed by
    StdRng::seed_from_u64(seed) one draw per sample call.  Returns (tokens,
    margins): the top1 - top2 logit of each greedy choice (zeros when
    sampling)."""
    k = max(1, k)  # pipeline.rs:294
    draws = stdrng_f32(seed, max_new + k + 1) if sampler is not None else None
    calls = [0]
    margins = []

    def sample(logits, generated):  # pipeline.rs:475-489
        if sampler is None:
            tok = argmax(logits)
            second = np.max(np.delete(logits, tok)) if logits.size > 1 else np.float32(-np.inf)
            margins.append(np.float32(logits[tok] - second))
        else:
            tok = sample_combined(logits, np.array(generated, np.uint32),
                                  u=float(draws[calls[0]]), **sampler)
            margins.append(np.float32(0.0))
        calls[0] += 1
        return int(tok)

    gen, out_margins = [], []
    gen.append(sample(model.prefill(prompt), gen))
    out_margins.append(margins[-1])
    while len(gen) < max_new:  # stopping.rs:39-42
        save = model.cache_len()
        drafts, dmarg = [], []
        last = gen[-1]
        for _ in range(k):
            tok = sample(draft(last), gen)
            drafts.append(tok)
            dmarg.append(margins[-1])
            last = tok
        model.truncate(save)
        model.prefill_append([gen[-1]] + drafts)  # verify; logits unused
        accepted = 0
        for tok, mg in zip(drafts, dmarg):
            gen.append(tok)
            out_margins.append(mg)
            accepted += 1
            if len(gen) >= max_new:
                break
        if accepted == k and len(gen) < max_new:  # bonus token
            gen.append(sample(model.forward_one(gen[-1]), gen))
            out_margins.append(margins[-1])
    return np.array(gen, np.uint32), np.array(out_margins, np.float32)
