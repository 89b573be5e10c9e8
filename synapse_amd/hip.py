"""ctypes binding of libsynapse_hip.so (the C ABI in include/synapse_hip.h).

This module is the Python view of the `hip` backend used by the tests and
the benchmark.  It loads the in-tree library and fails loudly when the
library is missing: there is no CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# SYN_HIP_LIBRARY may name another build of the same sources (the
# instrumented profiling build, `python -m synapse_amd.build --phase-timing`)
LIB_PATH = os.environ.get("SYN_HIP_LIBRARY") or os.path.join(HERE, "libsynapse_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "synapse_hip.h")

SYN_OK = 0
STATUS_NAMES = {0: "OK", 1: "NULL_PTR", 2: "INVALID_ARG", 3: "OUT_OF_MEMORY",
                4: "SHAPE_MISMATCH", 5: "NOT_CONTIGUOUS", 6: "INVALID_AXIS",
                7: "INVALID_DIMENSIONS", 8: "INTERNAL", 100: "NO_DEVICE", 101: "HIP",
                102: "LAUNCH"}
FMT_INT8, FMT_Q4_0, FMT_Q8_0, FMT_Q4_K, FMT_Q6_K, FMT_TERNARY = 1, 2, 3, 4, 5, 6
KQ_BLOCK = {FMT_Q8_0: (32, 34), FMT_Q4_K: (256, 144), FMT_Q6_K: (256, 210)}
LAYOUT_KN, LAYOUT_NK, LAYOUT_GGUF_DEQUANT = 0, 1, 2

P, SZ, ST = C.c_void_p, C.c_size_t, C.c_int32


class SamplerParams(C.Structure):
    """syn_hip_sampler: CombinedSampler (generation/sampler.rs:152-157)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float)]


class LmConfig(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("n_layers", C.c_uint32), ("n_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("inter", C.c_uint32),
                ("vocab", C.c_uint32), ("max_seq", C.c_uint32), ("eps", C.c_float),
                ("rope_theta", C.c_double)]


class KLmConfig(C.Structure):
    _fields_ = [("base", LmConfig), ("fmt_qkv", C.c_int32), ("fmt_o", C.c_int32),
                ("fmt_gate_up", C.c_int32), ("fmt_down", C.c_int32),
                ("fmt_lm_head", C.c_int32), ("qk_norm", C.c_int32)]


class MambaConfig(C.Structure):
    _fields_ = [("d_model", C.c_uint32), ("d_inner", C.c_uint32), ("d_state", C.c_uint32),
                ("d_conv", C.c_uint32), ("dt_rank", C.c_uint32), ("n_layers", C.c_uint32),
                ("vocab", C.c_uint32), ("max_tokens", C.c_uint32), ("eps", C.c_float),
                ("int8_xdt", C.c_int32)]


class HybridConfig(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("n_layers", C.c_uint32), ("vocab", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("inner", C.c_uint32), ("conv_kernel", C.c_uint32), ("inter", C.c_uint32),
                ("max_seq", C.c_uint32), ("eps", C.c_float), ("rope_theta", C.c_float),
                ("conv_bias", C.c_int32), ("layer_kinds", C.c_uint8 * 64)]


SIGNATURES = {
    "syn_quantize_per_channel_int8": (ST, [P, SZ, SZ, P, P]),
    "syn_qgemm_int8": (ST, [SZ, SZ, SZ, P, SZ, P, SZ, P, SZ, P, P]),
    "syn_q4_0_gemv": (ST, [SZ, SZ, P, P, P]),
    "syn_sgemm": (ST, [SZ, SZ, SZ, P, SZ, C.c_int, P, SZ, C.c_int, P, SZ]),
    "syn_hip_quantize_per_channel_int8": (ST, [P, SZ, SZ, P, P]),
    "syn_hip_qgemm_int8": (ST, [SZ, SZ, SZ, P, SZ, P, SZ, P, SZ, P, P]),
    "syn_hip_q4_0_gemv": (ST, [SZ, SZ, P, P, P]),
    "syn_hip_sgemm": (ST, [SZ, SZ, SZ, P, SZ, C.c_int, P, SZ, C.c_int, P, SZ]),
    "syn_hip_init": (ST, [C.c_int]),
    "syn_hip_device_count": (ST, [C.POINTER(C.c_int)]),
    "syn_hip_last_error": (C.c_char_p, []),
    "syn_hip_malloc": (ST, [C.POINTER(P), SZ]),
    "syn_hip_free": (ST, [P]),
    "syn_hip_memcpy_h2d": (ST, [P, P, SZ]),
    "syn_hip_memcpy_d2h": (ST, [P, P, SZ]),
    "syn_hip_memcpy_d2d": (ST, [P, P, SZ]),
    "syn_hip_memset": (ST, [P, C.c_int, SZ]),
    "syn_hip_synchronize": (ST, []),
    "syn_hip_stream_create": (ST, [C.POINTER(P)]),
    "syn_hip_stream_destroy": (ST, [P]),
    "syn_hip_stream_synchronize": (ST, [P]),
    "syn_hip_timer_create": (ST, [C.POINTER(P)]),
    "syn_hip_timer_start": (ST, [P, P]),
    "syn_hip_timer_stop": (ST, [P, P]),
    "syn_hip_timer_elapsed_ms": (ST, [P, C.POINTER(C.c_float)]),
    "syn_hip_timer_destroy": (ST, [P]),
    "syn_hip_quantize_rows": (ST, [P, SZ, SZ, SZ, P, SZ, P, P]),
    "syn_hip_qlinear_create": (ST, [C.c_int, SZ, SZ, P, P, C.c_int, C.POINTER(P)]),
    "syn_hip_qlinear_from_f32": (ST, [C.c_int, SZ, SZ, P, C.POINTER(P)]),
    "syn_hip_qlinear_forward": (ST, [P, SZ, P, P, P]),
    "syn_hip_qlinear_forward_noalloc": (ST, [P, SZ, P, P, P]),
    "syn_hip_qlinear_forward_pre_quantized": (ST, [P, SZ, P, SZ, P, P, P]),
    "syn_hip_qlinear_info": (ST, [P, C.POINTER(SZ), C.POINTER(SZ), C.POINTER(C.c_int),
                                  C.POINTER(SZ)]),
    "syn_hip_qlinear_destroy": (ST, [P]),
    "syn_hip_qlinear_time": (ST, [P, SZ, P, P, SZ, P, P, SZ, C.POINTER(C.c_float)]),
    "syn_hip_qlinear_time_set": (ST, [P, SZ, SZ, P, P, SZ, P, P, SZ, C.POINTER(C.c_float)]),
    "syn_hip_qlm_create": (ST, [C.POINTER(LmConfig), C.POINTER(P)]),
    "syn_hip_qlm_set_embed": (ST, [P, P]),
    "syn_hip_qlm_set_layer": (ST, [P, C.c_uint32, P, P, P, P, P, P, P]),
    "syn_hip_qlm_init_synthetic": (ST, [P, C.c_uint64, C.c_float]),
    "syn_hip_qlm_set_lm_head": (ST, [P, P]),
    "syn_hip_qlm_set_norms": (ST, [P, C.c_uint32, P, P, P, P]),
    "syn_hip_qlm_set_final_norm": (ST, [P, P]),
    "syn_hip_qlm_set_qk_norm": (ST, [P, C.c_int]),
    "syn_hip_qlm_finalize": (ST, [P]),
    "syn_hip_qlm_reset": (ST, [P]),
    "syn_hip_qlm_forward_prefill": (ST, [P, P, SZ, P]),
    "syn_hip_qlm_forward_one": (ST, [P, C.c_uint32, P]),
    "syn_hip_qlm_generate": (ST, [P, P, SZ, SZ, P, P]),
    "syn_hip_qlm_forward_prefill_append": (ST, [P, P, SZ, P]),
    "syn_hip_qlm_truncate": (ST, [P, SZ]),
    "syn_hip_qlm_cache_len": (ST, [P, C.POINTER(SZ)]),
    "syn_hip_qlm_generate_speculative": (ST, [P, P, SZ, SZ, SZ, P, P]),
    "syn_hip_qlm_decode_timed": (ST, [P, SZ, C.POINTER(C.c_float)]),
    "syn_hip_qlm_time_lm_head": (ST, [P, SZ, SZ, C.POINTER(C.c_float)]),
    "syn_hip_qlm_set_options": (ST, [P, C.c_int, C.c_int]),
    "syn_hip_qlm_set_sampler": (ST, [P, C.POINTER(SamplerParams), C.c_uint64]),
    "syn_hip_sample": (ST, [P, SZ, P, SZ, C.POINTER(SamplerParams), C.c_float, P, P, P]),
    "syn_hip_stdrng_f32": (ST, [C.c_uint64, SZ, P]),
    "syn_hip_qlm_time_lm_head_rotating": (ST, [P, SZ, C.POINTER(C.c_float)]),
    "syn_hip_qlm_time_step_kernels": (ST, [P, SZ, P, P]),
    "syn_hip_qlm_destroy": (ST, [P]),
    "syn_hip_klm_create": (ST, [C.POINTER(KLmConfig), C.POINTER(P)]),
    "syn_hip_klm_forward_prefill_append": (ST, [P, P, SZ, P]),
    "syn_hip_klm_truncate": (ST, [P, SZ]),
    "syn_hip_klm_cache_len": (ST, [P, C.POINTER(SZ)]),
    "syn_hip_klm_forward_one_draft": (ST, [P, C.c_uint32, SZ, P]),
    "syn_hip_klm_generate_speculative": (ST, [P, P, SZ, SZ, SZ, SZ, P, P]),
    "syn_hip_klm_set_embed": (ST, [P, P]),
    "syn_hip_klm_set_proj": (ST, [P, C.c_uint32, C.c_int, P]),
    "syn_hip_klm_set_lm_head": (ST, [P, P]),
    "syn_hip_klm_init_synthetic": (ST, [P, C.c_uint64, C.c_float]),
    "syn_hip_klm_finalize": (ST, [P]),
    "syn_hip_klm_reset": (ST, [P]),
    "syn_hip_klm_forward_prefill": (ST, [P, P, SZ, P]),
    "syn_hip_klm_forward_one": (ST, [P, C.c_uint32, P]),
    "syn_hip_klm_generate": (ST, [P, P, SZ, SZ, P, P]),
    "syn_hip_klm_time": (ST, [P, P, SZ, SZ, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    "syn_hip_klm_set_options": (ST, [P, C.c_int, C.c_int]),
    "syn_hip_klm_set_norms": (ST, [P, C.c_uint32, P, P, P, P]),
    "syn_hip_klm_set_final_norm": (ST, [P, P]),
    "syn_hip_klm_load_gguf": (ST, [P, P]),
    "syn_hip_gguf_open": (ST, [C.c_char_p, C.POINTER(P)]),
    "syn_hip_gguf_tensor_count": (ST, [P, C.POINTER(SZ)]),
    "syn_hip_gguf_find": (ST, [P, C.c_char_p, C.POINTER(SZ)]),
    "syn_hip_gguf_tensor_info": (ST, [P, SZ, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32),
                                      C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                      C.POINTER(C.c_uint64), C.POINTER(P)]),
    "syn_hip_gguf_meta_u64": (ST, [P, C.c_char_p, C.POINTER(C.c_uint64)]),
    "syn_hip_gguf_meta_f64": (ST, [P, C.c_char_p, C.POINTER(C.c_double)]),
    "syn_hip_gguf_meta_str": (ST, [P, C.c_char_p, C.POINTER(C.c_char_p)]),
    "syn_hip_gguf_close": (ST, [P]),
    "syn_hip_gguf_to_f32": (ST, [P, SZ, P]),
    "syn_hip_safetensors_open": (ST, [C.c_char_p, C.POINTER(P)]),
    "syn_hip_safetensors_tensor_count": (ST, [P, C.POINTER(SZ)]),
    "syn_hip_safetensors_find": (ST, [P, C.c_char_p, C.POINTER(SZ)]),
    "syn_hip_safetensors_tensor_info": (ST, [P, SZ, C.POINTER(C.c_char_p),
                                             C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                             C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                             C.POINTER(P)]),
    "syn_hip_safetensors_meta": (ST, [P, C.c_char_p, C.POINTER(C.c_char_p)]),
    "syn_hip_safetensors_to_f32": (ST, [P, SZ, P]),
    "syn_hip_safetensors_q4_pack": (ST, [P, C.c_char_p, P, C.POINTER(SZ), C.POINTER(SZ)]),
    "syn_hip_safetensors_close": (ST, [P]),
    "syn_hip_qlinear_from_gguf": (ST, [P, C.c_char_p, C.POINTER(P)]),
    "syn_hip_qlinear_from_safetensors_q4": (ST, [P, C.c_char_p, C.POINTER(P)]),
    "syn_hip_qlm_load_gguf": (ST, [P, P]),
    "syn_hip_qlm_load_safetensors": (ST, [P, P]),
    "syn_hip_klm_destroy": (ST, [P]),
    "syn_hip_mamba_create": (ST, [C.POINTER(MambaConfig), C.POINTER(P)]),
    "syn_hip_mamba_init_synthetic": (ST, [P, C.c_uint64, C.c_float]),
    "syn_hip_mamba_prefill": (ST, [P, P, SZ, P]),
    "syn_hip_mamba_decode_one": (ST, [P, C.c_uint32, P]),
    "syn_hip_mamba_generate": (ST, [P, P, SZ, SZ, P, P]),
    "syn_hip_mamba_decode_timed": (ST, [P, SZ, C.POINTER(C.c_float)]),
    "syn_hip_mamba_set_options": (ST, [P, C.c_int, C.c_int]),
    "syn_hip_mamba_destroy": (ST, [P]),
    "syn_hip_hlm_create": (ST, [C.POINTER(HybridConfig), C.POINTER(P)]),
    "syn_hip_hlm_init_synthetic": (ST, [P, C.c_uint64, C.c_float]),
    "syn_hip_hlm_reset": (ST, [P]),
    "syn_hip_hlm_position": (ST, [P, C.POINTER(SZ)]),
    "syn_hip_hlm_decode_one": (ST, [P, C.c_uint32, P]),
    "syn_hip_hlm_prefill": (ST, [P, P, SZ, P]),
    "syn_hip_hlm_generate": (ST, [P, P, SZ, SZ, P, P]),
    "syn_hip_hlm_decode_timed": (ST, [P, SZ, C.POINTER(C.c_float)]),
    "syn_hip_hlm_set_options": (ST, [P, C.c_int, C.c_int]),
    "syn_hip_hlm_fused_active": (ST, [P, C.POINTER(C.c_int)]),
    "syn_hip_hlm_destroy": (ST, [P]),
    "syn_hip_fill_normal": (ST, [P, SZ, C.c_uint64, C.c_float]),
    "syn_hip_probe_mfma": (ST, [C.c_int, SZ, C.POINTER(C.c_double)]),
    "syn_hip_probe_hbm_read": (ST, [SZ, C.POINTER(C.c_double)]),
    "syn_hip_probe_seq_sum": (ST, [P, SZ, P]),
    "syn_hip_probe_graph_floor": (ST, [C.c_int, C.c_int, C.POINTER(C.c_double)]),
    "syn_hip_probe_grid_barrier": (ST, [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double),
                                        C.POINTER(C.c_int)]),
    "syn_hip_eval_expf": (ST, [P, P, SZ, P]),
    "syn_hip_kquant_encode": (ST, [C.c_int, SZ, SZ, P, P]),
    "syn_hip_kquant_decode": (ST, [C.c_int, SZ, P, P]),
}

_lib = None


class SynapseError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: status {status} ({STATUS_NAMES.get(status, 'Unknown')})"
                         f" {last_error()}")


def lib():
    """Load the in-tree HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "`python -m synapse_amd.build` (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    if _lib is None:
        return ""
    s = _lib.syn_hip_last_error()
    return s.decode() if s else ""


def check(status: int, what: str = "synapse_hip"):
    if status != SYN_OK:
        raise SynapseError(status, what)


def ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def device_count() -> int:
    n = C.c_int(0)
    lib().syn_hip_device_count(C.byref(n))
    return n.value


def init(device: int = 0):
    check(lib().syn_hip_init(device), "syn_hip_init")


class DeviceBuffer:
    """Raw device allocation owned by Python (freed on close / GC)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().syn_hip_malloc(C.byref(p), max(self.nbytes, 1)), "syn_hip_malloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().syn_hip_memcpy_h2d(self.ptr, ptr(a), a.nbytes), "h2d")

    def download(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().syn_hip_memcpy_d2h(ptr(out), self.ptr, out.nbytes), "d2h")
        return out

    def zero(self):
        check(lib().syn_hip_memset(self.ptr, 0, self.nbytes), "memset")

    def close(self):
        if self.ptr:
            lib().syn_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Timer:
    def __init__(self):
        p = C.c_void_p()
        check(lib().syn_hip_timer_create(C.byref(p)), "timer_create")
        self.h = p.value

    def start(self, stream=None):
        check(lib().syn_hip_timer_start(self.h, stream))

    def stop(self, stream=None):
        check(lib().syn_hip_timer_stop(self.h, stream))

    def ms(self) -> float:
        v = C.c_float()
        check(lib().syn_hip_timer_elapsed_ms(self.h, C.byref(v)))
        return v.value

    def __del__(self):
        try:
            lib().syn_hip_timer_destroy(self.h)
        except Exception:
            pass


# ------------------------------------------------------------------ reference-signature calls
def quantize_per_channel_int8(x: np.ndarray):
    """syn_quantize_per_channel_int8 through the HIP library (host pointers)."""
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    check(lib().syn_quantize_per_channel_int8(ptr(x), m, k, ptr(q), ptr(s)),
          "syn_quantize_per_channel_int8")
    return q, s


def qgemm_int8(a, b_kn, sa, sb) -> np.ndarray:
    a = np.ascontiguousarray(a, np.int8)
    b_kn = np.ascontiguousarray(b_kn, np.int8)
    m, k = a.shape
    n = b_kn.shape[1]
    c = np.zeros((m, n), np.float32)
    sa = np.ascontiguousarray(sa, np.float32)
    sb = np.ascontiguousarray(sb, np.float32)
    check(lib().syn_qgemm_int8(m, n, k, ptr(a), k, ptr(b_kn), n, ptr(c), n, ptr(sa), ptr(sb)),
          "syn_qgemm_int8")
    return c


def sgemm(a: np.ndarray, b: np.ndarray, trans_a: bool = False, trans_b: bool = False,
          c: np.ndarray = None) -> np.ndarray:
    """syn_sgemm (synapse.h:176-184): op(A) op(B), accumulated into c (zeros
    if None) on the GOTO path, overwritten on the M <= 16 GEMV path."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = (a.shape[1], a.shape[0]) if trans_a else a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    out = np.zeros((m, n), np.float32) if c is None else np.array(c, np.float32, copy=True)
    check(lib().syn_sgemm(m, n, k, ptr(a), a.shape[1], int(trans_a), ptr(b), b.shape[1],
                          int(trans_b), ptr(out), n), "syn_sgemm")
    return out


def q4_0_gemv(a: np.ndarray, packed: np.ndarray, n: int) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    packed = np.ascontiguousarray(packed, np.uint8)
    c = np.zeros(n, np.float32)
    check(lib().syn_q4_0_gemv(n, a.shape[0], ptr(a), ptr(packed), ptr(c)), "syn_q4_0_gemv")
    return c


# ------------------------------------------------------------------ handles
class QLinear:
    """Device-resident quantized linear (INT8 W8A8 or Q4_0)."""

    def __init__(self, handle, fmt):
        self.h = handle
        self.fmt = fmt
        n, k, f, wb = SZ(), SZ(), C.c_int(), SZ()
        check(lib().syn_hip_qlinear_info(self.h, C.byref(n), C.byref(k), C.byref(f),
                                         C.byref(wb)))
        self.n, self.k, self.weight_bytes = n.value, k.value, wb.value

    @classmethod
    def from_f32(cls, fmt: int, w_nk: np.ndarray) -> "QLinear":
        w_nk = np.ascontiguousarray(w_nk, np.float32)
        h = C.c_void_p()
        check(lib().syn_hip_qlinear_from_f32(fmt, w_nk.shape[0], w_nk.shape[1], ptr(w_nk),
                                             C.byref(h)), "qlinear_from_f32")
        return cls(h.value, fmt)

    @classmethod
    def int8(cls, weights: np.ndarray, scales: np.ndarray, layout: int = LAYOUT_KN) -> "QLinear":
        weights = np.ascontiguousarray(weights, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        if layout == LAYOUT_KN:
            k, n = weights.shape
        else:
            n, k = weights.shape
        h = C.c_void_p()
        check(lib().syn_hip_qlinear_create(FMT_INT8, n, k, ptr(weights), ptr(scales), layout,
                                           C.byref(h)), "qlinear_create")
        return cls(h.value, FMT_INT8)

    @classmethod
    def q4_0(cls, packed: np.ndarray, n: int, k: int, gguf_dequant: bool = False) -> "QLinear":
        """pack_for_zig / GGUF Q4_0 blocks; gguf_dequant reads the block scales
        as the reference's dequantize_q4_0 (subnormals halved)."""
        packed = np.ascontiguousarray(packed, np.uint8)
        h = C.c_void_p()
        check(lib().syn_hip_qlinear_create(FMT_Q4_0, n, k, ptr(packed), None,
                                           LAYOUT_GGUF_DEQUANT if gguf_dequant else 0,
                                           C.byref(h)), "qlinear_create")
        return cls(h.value, FMT_Q4_0)

    @classmethod
    def ternary(cls, blocks: np.ndarray, n: int, k: int) -> "QLinear":
        """TernaryLinear blocks (f32 scale + 4 code bytes per 16 weights) of [n, k]."""
        blocks = np.ascontiguousarray(blocks, np.uint8)
        h = C.c_void_p()
        check(lib().syn_hip_qlinear_create(FMT_TERNARY, n, k, ptr(blocks), None, 0, C.byref(h)),
              "qlinear_create")
        return cls(h.value, FMT_TERNARY)

    @classmethod
    def gguf(cls, fmt: int, blocks: np.ndarray, n: int, k: int) -> "QLinear":
        """Q8_0 / Q4_K / Q6_K block bytes of a row-major [n, k] tensor."""
        blocks = np.ascontiguousarray(blocks, np.uint8)
        h = C.c_void_p()
        check(lib().syn_hip_qlinear_create(fmt, n, k, ptr(blocks), None, 0, C.byref(h)),
              "qlinear_create")
        return cls(h.value, fmt)

    @classmethod
    def from_gguf(cls, gguf: "Gguf", name: str) -> "QLinear":
        """A Q4_0 / Q8_0 / Q4_K / Q6_K GGUF tensor, uploaded as stored."""
        h = C.c_void_p()
        check(lib().syn_hip_qlinear_from_gguf(gguf.h, name.encode(), C.byref(h)),
              "qlinear_from_gguf")
        fmt = {2: FMT_Q4_0, 8: FMT_Q8_0, 12: FMT_Q4_K, 14: FMT_Q6_K}[
            gguf.info(gguf.index(name)).ggml_type]
        return cls(h.value, fmt)

    @classmethod
    def from_safetensors_q4(cls, st: "Safetensors", base: str) -> "QLinear":
        """A safetensors Q4_0 triple, uploaded without dequantizing."""
        h = C.c_void_p()
        check(lib().syn_hip_qlinear_from_safetensors_q4(st.h, base.encode(), C.byref(h)),
              "qlinear_from_safetensors_q4")
        return cls(h.value, FMT_Q4_0)

    def forward_dev(self, m: int, d_x: int, d_y: int, stream=None):
        check(lib().syn_hip_qlinear_forward(self.h, m, d_x, d_y, stream), "qlinear_forward")

    def forward_noalloc_dev(self, m: int, d_x: int, d_y: int, stream=None):
        """INT8: forward with the library's fixed device scratch (no allocation)."""
        check(lib().syn_hip_qlinear_forward_noalloc(self.h, m, d_x, d_y, stream),
              "qlinear_forward_noalloc")

    def forward_pre_quantized_dev(self, m, d_xq, ldxq, d_sx, d_y, stream=None):
        check(lib().syn_hip_qlinear_forward_pre_quantized(self.h, m, d_xq, ldxq, d_sx, d_y,
                                                          stream), "forward_pre_quantized")

    def time(self, m: int, d_x=None, d_xq=None, ldxq=0, d_sx=None, d_y=None,
             iters: int = 20) -> float:
        ms = C.c_float()
        check(lib().syn_hip_qlinear_time(self.h, m, d_x, d_xq, ldxq, d_sx, d_y, iters,
                                         C.byref(ms)), "qlinear_time")
        return ms.value

    @staticmethod
    def time_set(linears, m: int, d_x=None, d_xq=None, ldxq=0, d_sx=None, d_y=None,
                 rounds: int = 10) -> float:
        """Average ms per launch, round-robin over several handles (copies of
        one matrix), so that the working set can exceed the Infinity Cache."""
        arr = (C.c_void_p * len(linears))(*[l.h for l in linears])
        ms = C.c_float()
        check(lib().syn_hip_qlinear_time_set(arr, len(linears), m, d_x, d_xq, ldxq, d_sx, d_y,
                                             rounds, C.byref(ms)), "qlinear_time_set")
        return ms.value

    def forward(self, x: np.ndarray) -> np.ndarray:
        """Host convenience: upload x [m,k], run, download y [m,n]."""
        x = np.ascontiguousarray(x, np.float32)
        m = x.shape[0]
        dx = DeviceBuffer.from_array(x)
        dy = DeviceBuffer(m * self.n * 4)
        self.forward_dev(m, dx.ptr, dy.ptr)
        check(lib().syn_hip_stream_synchronize(None))
        return dy.download((m, self.n), np.float32)

    def close(self):
        if self.h:
            lib().syn_hip_qlinear_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QuantizedCausalLM:
    """Device-resident INT8 W8A8 decoder (mirror of QuantizedCausalLM)."""

    def __init__(self, cfg: dict):
        self.cfg = dict(cfg)
        c = LmConfig(cfg["hidden"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                     cfg["head_dim"], cfg["inter"], cfg["vocab"], cfg["max_seq"],
                     cfg.get("eps", 1e-6), cfg.get("rope_theta", 1e6))
        h = C.c_void_p()
        check(lib().syn_hip_qlm_create(C.byref(c), C.byref(h)), "qlm_create")
        self.h = h.value

    def init_synthetic(self, seed_base: int = 0x5EED0000, std: float = 0.02):
        check(lib().syn_hip_qlm_init_synthetic(self.h, seed_base, std), "qlm_init_synthetic")
        check(lib().syn_hip_qlm_finalize(self.h), "qlm_finalize")

    def set_weights(self, embed: np.ndarray, layers: list, final_norm=None, lm_head=None,
                    qk_norm: bool = True):
        """f32 weights: layers[i] holds q,k,v,o,gate,up,down [out, in] and optionally
        the gains attn_norm, ffn_norm, q_norm, k_norm; lm_head None = tied."""
        check(lib().syn_hip_qlm_set_embed(self.h, ptr(np.ascontiguousarray(embed, np.float32))))
        check(lib().syn_hip_qlm_set_qk_norm(self.h, int(qk_norm)), "set_qk_norm")
        for i, lw in enumerate(layers):
            arrs = [np.ascontiguousarray(lw[n], np.float32)
                    for n in ("q", "k", "v", "o", "gate", "up", "down")]
            check(lib().syn_hip_qlm_set_layer(self.h, i, *[ptr(a) for a in arrs]), "set_layer")
            gains = [None if lw.get(n) is None else np.ascontiguousarray(lw[n], np.float32)
                     for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm")]
            check(lib().syn_hip_qlm_set_norms(self.h, i, *[None if g is None else ptr(g)
                                                           for g in gains]), "set_norms")
        if final_norm is not None:
            check(lib().syn_hip_qlm_set_final_norm(
                self.h, ptr(np.ascontiguousarray(final_norm, np.float32))), "set_final_norm")
        if lm_head is not None:
            check(lib().syn_hip_qlm_set_lm_head(
                self.h, ptr(np.ascontiguousarray(lm_head, np.float32))), "set_lm_head")
        check(lib().syn_hip_qlm_finalize(self.h), "qlm_finalize")

    def load_gguf(self, gguf: "Gguf"):
        """Every weight from a GGUF file (HuggingFace or llama.cpp names), then finalize."""
        check(lib().syn_hip_qlm_load_gguf(self.h, gguf.h), "qlm_load_gguf")
        check(lib().syn_hip_qlm_finalize(self.h), "qlm_finalize")

    def load_safetensors(self, st: "Safetensors"):
        """Every weight from a safetensors file or sharded checkpoint, then finalize."""
        check(lib().syn_hip_qlm_load_safetensors(self.h, st.h), "qlm_load_safetensors")
        check(lib().syn_hip_qlm_finalize(self.h), "qlm_finalize")

    def reset(self):
        check(lib().syn_hip_qlm_reset(self.h))

    def prefill(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.uint32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_qlm_forward_prefill(self.h, ptr(ids), ids.size, ptr(logits)),
              "forward_prefill")
        return logits

    def forward_one(self, token: int) -> np.ndarray:
        logits = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_qlm_forward_one(self.h, int(token), ptr(logits)), "forward_one")
        return logits

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        check(lib().syn_hip_qlm_generate(self.h, ptr(prompt), prompt.size, max_new, ptr(toks),
                                         ptr(margins)), "generate")
        return toks, margins

    def prefill_append(self, ids) -> np.ndarray:
        """forward_prefill into the cache as it stands (rows appended after the
        cached ones, rotated from position 0, attending among themselves)."""
        ids = np.ascontiguousarray(ids, np.uint32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_qlm_forward_prefill_append(self.h, ptr(ids), ids.size, ptr(logits)),
              "forward_prefill_append")
        return logits

    def truncate(self, new_len: int):
        """KVCache::truncate_to: a shorter cache length applies, a longer one is ignored."""
        check(lib().syn_hip_qlm_truncate(self.h, new_len), "truncate")

    def cache_len(self) -> int:
        n = SZ()
        check(lib().syn_hip_qlm_cache_len(self.h, C.byref(n)), "cache_len")
        return n.value

    def generate_speculative(self, prompt, max_new: int, k: int):
        """generate_speculative (pipeline.rs:281-395) with speculative_k = k."""
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        check(lib().syn_hip_qlm_generate_speculative(self.h, ptr(prompt), prompt.size, max_new, k,
                                                     ptr(toks), ptr(margins)),
              "generate_speculative")
        return toks, margins

    def decode_timed(self, steps: int) -> float:
        ms = C.c_float()
        check(lib().syn_hip_qlm_decode_timed(self.h, steps, C.byref(ms)), "decode_timed")
        return ms.value

    def set_options(self, fused: bool = True, graph: bool = True):
        """Decode-step form: fused five-kernel layers or one kernel per op; HIP
        graph replay or eager launches (same results either way)."""
        check(lib().syn_hip_qlm_set_options(self.h, int(fused), int(graph)), "set_options")

    def set_sampler(self, params=None, seed: int = 0):
        """CombinedSampler settings for generate / decode steps (None: greedy),
        with the draws of StdRng::seed_from_u64(seed)."""
        check(lib().syn_hip_qlm_set_sampler(self.h, None if params is None else C.byref(params),
                                            seed), "set_sampler")

    def time_lm_head_rotating(self, iters: int = 40) -> float:
        ms = C.c_float()
        check(lib().syn_hip_qlm_time_lm_head_rotating(self.h, iters, C.byref(ms)),
              "time_lm_head_rotating")
        return ms.value

    STEP_KINDS = ("zero", "qkv", "attention", "o", "gate_up", "down", "final_norm", "lm_head",
                  "select")

    def time_step_kernels(self, steps: int = 8) -> dict:
        """Eager fused steps with a hipEvent pair around every kernel: per kind
        the average us per launch and the launches per step."""
        n = len(self.STEP_KINDS)
        us = (C.c_float * n)()
        cnt = (C.c_uint32 * n)()
        check(lib().syn_hip_qlm_time_step_kernels(self.h, steps, us, cnt), "time_step_kernels")
        return {k: {"avg_us": round(us[i], 3), "launches_per_step": cnt[i] / steps}
                for i, k in enumerate(self.STEP_KINDS) if cnt[i]}

    def time_lm_head(self, iters: int = 20, flush_bytes: int = 512 << 20) -> float:
        ms = C.c_float()
        check(lib().syn_hip_qlm_time_lm_head(self.h, iters, flush_bytes, C.byref(ms)),
              "time_lm_head")
        return ms.value

    def close(self):
        if self.h:
            lib().syn_hip_qlm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KQuantCausalLM:
    """Device-resident f32 decoder over Q8_0/Q4_K/Q6_K weights (CausalLM)."""

    def __init__(self, cfg: dict, fmt_qkv=FMT_Q4_K, fmt_o=FMT_Q4_K, fmt_gate_up=FMT_Q4_K,
                 fmt_down=FMT_Q6_K, fmt_lm_head=FMT_Q6_K, qk_norm=False):
        self.cfg = dict(cfg)
        base = LmConfig(cfg["hidden"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                        cfg["head_dim"], cfg["inter"], cfg["vocab"], cfg["max_seq"],
                        cfg.get("eps", 1e-5), cfg.get("rope_theta", 5e5))
        c = KLmConfig(base, fmt_qkv, fmt_o, fmt_gate_up, fmt_down, fmt_lm_head,
                      1 if qk_norm else 0)
        h = C.c_void_p()
        check(lib().syn_hip_klm_create(C.byref(c), C.byref(h)), "klm_create")
        self.h = h.value

    def init_synthetic(self, seed_base: int = 0x5EED0000, std: float = 0.02):
        check(lib().syn_hip_klm_init_synthetic(self.h, seed_base, std), "klm_init_synthetic")
        check(lib().syn_hip_klm_finalize(self.h), "klm_finalize")

    def set_embed(self, embed):
        check(lib().syn_hip_klm_set_embed(self.h, ptr(np.ascontiguousarray(embed, np.float32))))

    def set_proj(self, layer: int, proj: int, blocks: np.ndarray):
        check(lib().syn_hip_klm_set_proj(self.h, layer, proj,
                                         ptr(np.ascontiguousarray(blocks, np.uint8))), "set_proj")

    def set_lm_head(self, blocks: np.ndarray):
        check(lib().syn_hip_klm_set_lm_head(self.h, ptr(np.ascontiguousarray(blocks, np.uint8))))

    def finalize(self):
        check(lib().syn_hip_klm_finalize(self.h), "klm_finalize")

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_klm_forward_prefill(self.h, ptr(ids), ids.size, ptr(out)), "prefill")
        return out

    def forward_one(self, token: int):
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_klm_forward_one(self.h, int(token), ptr(out)), "forward_one")
        return out

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        check(lib().syn_hip_klm_generate(self.h, ptr(prompt), prompt.size, max_new, ptr(toks),
                                         ptr(margins)), "generate")
        return toks, margins

    def prefill_append(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_klm_forward_prefill_append(self.h, ptr(ids), ids.size, ptr(out)),
              "klm_forward_prefill_append")
        return out

    def truncate(self, new_len: int):
        check(lib().syn_hip_klm_truncate(self.h, new_len), "klm_truncate")

    def cache_len(self) -> int:
        n = SZ()
        check(lib().syn_hip_klm_cache_len(self.h, C.byref(n)), "klm_cache_len")
        return n.value

    def forward_one_draft(self, token: int, n_layers: int):
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_klm_forward_one_draft(self.h, int(token), n_layers, ptr(out)),
              "klm_forward_one_draft")
        return out

    def generate_speculative(self, prompt, max_new: int, k: int, draft_layers: int = 0):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        check(lib().syn_hip_klm_generate_speculative(self.h, ptr(prompt), prompt.size, max_new, k,
                                                     draft_layers, ptr(toks), ptr(margins)),
              "klm_generate_speculative")
        return toks, margins

    def time(self, prompt, steps: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        p, d = C.c_float(), C.c_float()
        check(lib().syn_hip_klm_time(self.h, ptr(prompt), prompt.size, steps, C.byref(p),
                                     C.byref(d)), "klm_time")
        return p.value, d.value

    def set_options(self, fused: bool = True, graph: bool = True):
        """Decode-step form: fused five-kernel layers (tree-ordered sums) or one
        kernel per op; HIP graph replay or eager launches (same results)."""
        check(lib().syn_hip_klm_set_options(self.h, int(fused), int(graph)), "set_options")

    def set_norms(self, layer: int, attn=None, ffn=None, q=None, k=None):
        """RMSNorm gains of one layer (None leaves a gain as it is; all start at 1.0)."""
        arrs = [None if a is None else np.ascontiguousarray(a, np.float32)
                for a in (attn, ffn, q, k)]
        check(lib().syn_hip_klm_set_norms(self.h, layer,
                                          *[None if a is None else ptr(a) for a in arrs]),
              "set_norms")

    def set_final_norm(self, gain):
        check(lib().syn_hip_klm_set_final_norm(self.h,
                                               ptr(np.ascontiguousarray(gain, np.float32))),
              "set_final_norm")

    def load_gguf(self, gguf: "Gguf"):
        """Every weight from a GGUF file (llama.cpp or HuggingFace tensor names), then finalize."""
        check(lib().syn_hip_klm_load_gguf(self.h, gguf.h), "klm_load_gguf")
        check(lib().syn_hip_klm_finalize(self.h), "klm_finalize")

    def close(self):
        if self.h:
            lib().syn_hip_klm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufTensorInfo:
    __slots__ = ("name", "ggml_type", "dims", "nbytes", "data")

    def __init__(self, name, ggml_type, dims, nbytes, data):
        self.name, self.ggml_type, self.dims, self.nbytes, self.data = (
            name, ggml_type, dims, nbytes, data)

    def bytes(self) -> np.ndarray:
        """A copy of the tensor's stored bytes."""
        return np.ctypeslib.as_array((C.c_uint8 * self.nbytes).from_address(self.data)).copy()


class Gguf:
    """Read-only mapping of a GGUF v2/v3 file (host code only, no device use)."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().syn_hip_gguf_open(str(path).encode(), C.byref(h)), "gguf_open")
        self.h = h.value

    def __len__(self):
        n = SZ()
        check(lib().syn_hip_gguf_tensor_count(self.h, C.byref(n)), "gguf_tensor_count")
        return n.value

    def index(self, name: str):
        i = SZ()
        rc = lib().syn_hip_gguf_find(self.h, name.encode(), C.byref(i))
        return i.value if rc == 0 else None

    def info(self, index: int) -> GgufTensorInfo:
        name, t, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        dims, nb, data = (C.c_uint64 * 4)(), C.c_uint64(), C.c_void_p()
        check(lib().syn_hip_gguf_tensor_info(self.h, index, C.byref(name), C.byref(t),
                                             C.byref(nd), dims, C.byref(nb), C.byref(data)),
              "gguf_tensor_info")
        return GgufTensorInfo(name.value.decode(), t.value, tuple(dims[:nd.value]), nb.value,
                              data.value)

    def tensors(self):
        return [self.info(i) for i in range(len(self))]

    def to_f32(self, index: int) -> np.ndarray:
        """f32 values of a tensor as the reference's parse_gguf returns them."""
        t = self.info(index)
        out = np.empty(int(np.prod(t.dims)), np.float32)
        check(lib().syn_hip_gguf_to_f32(self.h, index, ptr(out)), "gguf_to_f32")
        return out

    def meta_u64(self, key: str):
        v = C.c_uint64()
        return v.value if lib().syn_hip_gguf_meta_u64(self.h, key.encode(), C.byref(v)) == 0 \
            else None

    def meta_f64(self, key: str):
        v = C.c_double()
        return v.value if lib().syn_hip_gguf_meta_f64(self.h, key.encode(), C.byref(v)) == 0 \
            else None

    def meta_str(self, key: str):
        v = C.c_char_p()
        return v.value.decode() if lib().syn_hip_gguf_meta_str(self.h, key.encode(),
                                                                C.byref(v)) == 0 else None

    def close(self):
        if self.h:
            lib().syn_hip_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


ST_DTYPES = {0: "F32", 1: "F16", 2: "BF16", 3: "I64", 4: "I32", 5: "U8"}


class SafetensorsTensorInfo(GgufTensorInfo):
    __slots__ = ()

    @property
    def dtype(self) -> str:
        return ST_DTYPES[self.ggml_type]


class Safetensors:
    """Read-only mapping of a safetensors file or sharded checkpoint directory."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().syn_hip_safetensors_open(str(path).encode(), C.byref(h)), "safetensors_open")
        self.h = h.value

    def __len__(self):
        n = SZ()
        check(lib().syn_hip_safetensors_tensor_count(self.h, C.byref(n)), "tensor_count")
        return n.value

    def index(self, name: str):
        i = SZ()
        rc = lib().syn_hip_safetensors_find(self.h, name.encode(), C.byref(i))
        return i.value if rc == 0 else None

    def info(self, index: int) -> SafetensorsTensorInfo:
        name, t, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        dims, nb, data = (C.c_uint64 * 8)(), C.c_uint64(), C.c_void_p()
        check(lib().syn_hip_safetensors_tensor_info(self.h, index, C.byref(name), C.byref(t),
                                                    C.byref(nd), dims, C.byref(nb),
                                                    C.byref(data)), "tensor_info")
        return SafetensorsTensorInfo(name.value.decode(), t.value, tuple(dims[:nd.value]),
                                     nb.value, data.value)

    def names(self):
        return [self.info(i).name for i in range(len(self))]

    def to_f32(self, index: int) -> np.ndarray:
        """f32 values as the reference's parse_safetensors converts them."""
        t = self.info(index)
        out = np.empty(int(np.prod(t.dims, dtype=np.int64)), np.float32)
        check(lib().syn_hip_safetensors_to_f32(self.h, index, ptr(out)), "safetensors_to_f32")
        return out.reshape(t.dims)

    def meta(self, key: str):
        v = C.c_char_p()
        return v.value.decode() if lib().syn_hip_safetensors_meta(self.h, key.encode(),
                                                                   C.byref(v)) == 0 else None

    def q4_pack(self, base: str):
        """A Q4_0 triple (<base>.q4_nibbles/.q4_scales/.q4_orig_cols) as pack_for_zig bytes."""
        r, c = SZ(), SZ()
        check(lib().syn_hip_safetensors_q4_pack(self.h, base.encode(), None, C.byref(r),
                                                C.byref(c)), "q4_pack")
        bpr = self.info(self.index(base + ".q4_nibbles")).dims[1]
        out = np.empty(r.value * bpr * 18, np.uint8)
        check(lib().syn_hip_safetensors_q4_pack(self.h, base.encode(), ptr(out), C.byref(r),
                                                C.byref(c)), "q4_pack")
        return out, r.value, c.value

    def close(self):
        if self.h:
            lib().syn_hip_safetensors_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QuantizedMamba:
    """Device-resident INT8 Mamba (QuantizedMambaModel)."""

    def __init__(self, cfg: dict, int8_xdt: bool = False):
        self.cfg = dict(cfg)
        c = MambaConfig(cfg["d_model"], cfg["d_inner"], cfg["d_state"], cfg["d_conv"],
                        cfg["dt_rank"], cfg["n_layers"], cfg["vocab"], cfg["max_tokens"],
                        cfg.get("eps", 1e-5), 1 if int8_xdt else 0)
        h = C.c_void_p()
        check(lib().syn_hip_mamba_create(C.byref(c), C.byref(h)), "mamba_create")
        self.h = h.value

    def init_synthetic(self, seed_base: int = 0x5EED0000, std: float = 0.02):
        check(lib().syn_hip_mamba_init_synthetic(self.h, seed_base, std), "mamba_init")

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_mamba_prefill(self.h, ptr(ids), ids.size, ptr(out)), "prefill")
        return out

    def decode_one(self, token: int):
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_mamba_decode_one(self.h, int(token), ptr(out)), "decode_one")
        return out

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        check(lib().syn_hip_mamba_generate(self.h, ptr(prompt), prompt.size, max_new, ptr(toks),
                                           ptr(margins)), "generate")
        return toks, margins

    def decode_timed(self, steps: int) -> float:
        ms = C.c_float()
        check(lib().syn_hip_mamba_decode_timed(self.h, steps, C.byref(ms)), "decode_timed")
        return ms.value

    def set_options(self, fused: bool = True, graph: bool = True):
        """Token-step form: fused split-K GEMV kernels or one kernel per op;
        HIP graph replay or eager launches (same results either way)."""
        check(lib().syn_hip_mamba_set_options(self.h, int(fused), int(graph)), "set_options")

    def close(self):
        if self.h:
            lib().syn_hip_mamba_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HybridLM:
    """Device-resident hybrid LFM2.5 decoder, Q4 decode path (models/ssm/hybrid).
    cfg: hidden, n_layers, vocab, n_heads, n_kv_heads, head_dim, inner,
    conv_kernel, inter, max_seq, eps, rope_theta, conv_bias, layer_kinds
    (0 LIV conv, 1 GQA)."""

    def __init__(self, cfg: dict):
        self.cfg = dict(cfg)
        kinds = (C.c_uint8 * 64)(*cfg["layer_kinds"])
        c = HybridConfig(cfg["hidden"], cfg["n_layers"], cfg["vocab"], cfg["n_heads"],
                         cfg["n_kv_heads"], cfg["head_dim"], cfg["inner"], cfg["conv_kernel"],
                         cfg["inter"], cfg["max_seq"], cfg.get("eps", 1e-5),
                         cfg.get("rope_theta", 1e6), int(cfg.get("conv_bias", 0)), kinds)
        h = C.c_void_p()
        check(lib().syn_hip_hlm_create(C.byref(c), C.byref(h)), "hlm_create")
        self.h = h.value

    def init_synthetic(self, seed_base: int = 0x5EED0000, std: float = 0.02):
        check(lib().syn_hip_hlm_init_synthetic(self.h, seed_base, std), "hlm_init")

    def reset(self):
        check(lib().syn_hip_hlm_reset(self.h), "hlm_reset")

    @property
    def pos(self) -> int:
        v = C.c_size_t()
        check(lib().syn_hip_hlm_position(self.h, C.byref(v)), "hlm_position")
        return v.value

    def decode_one(self, token: int):
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_hlm_decode_one(self.h, int(token), ptr(out)), "hlm_decode_one")
        return out

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.uint32)
        out = np.empty(self.cfg["vocab"], np.float32)
        check(lib().syn_hip_hlm_prefill(self.h, ptr(ids), ids.size, ptr(out)), "hlm_prefill")
        return out

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        toks = np.zeros(max_new, np.uint32)
        margins = np.zeros(max_new, np.float32)
        check(lib().syn_hip_hlm_generate(self.h, ptr(prompt), prompt.size, max_new, ptr(toks),
                                         ptr(margins)), "hlm_generate")
        return toks, margins

    def decode_timed(self, steps: int) -> float:
        ms = C.c_float()
        check(lib().syn_hip_hlm_decode_timed(self.h, steps, C.byref(ms)), "hlm_decode_timed")
        return ms.value

    def set_options(self, fused: bool = True, graph: bool = True):
        check(lib().syn_hip_hlm_set_options(self.h, int(fused), int(graph)), "hlm_set_options")

    @property
    def fused_active(self) -> bool:
        v = C.c_int()
        check(lib().syn_hip_hlm_fused_active(self.h, C.byref(v)), "hlm_fused_active")
        return bool(v.value)

    def close(self):
        if self.h:
            lib().syn_hip_hlm_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sampler_params(temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0):
    return SamplerParams(temperature, top_k, top_p, repetition_penalty)


def sample(logits: np.ndarray, history=(), temperature=1.0, top_k=0, top_p=1.0,
           repetition_penalty=1.0, u=0.5):
    """syn_hip_sample on host arrays (uploads, samples on the device, reads the
    token back): CombinedSampler::sample_with_history with the draw u."""
    x = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(np.asarray(history, np.uint32).reshape(-1))
    dx = DeviceBuffer.from_array(x)
    dh = DeviceBuffer.from_array(h if h.size else np.zeros(1, np.uint32))
    dt = DeviceBuffer(4)
    ds = DeviceBuffer(4)
    try:
        prm = sampler_params(temperature, top_k, top_p, repetition_penalty)
        check(lib().syn_hip_sample(dx.ptr, x.size, dh.ptr, h.size, C.byref(prm), u, dt.ptr,
                                   ds.ptr, None), "sample")
        check(lib().syn_hip_stream_synchronize(None))
        tok = int(dt.download(1, np.uint32)[0])
        status = int(ds.download(1, np.int32)[0])
    finally:
        for b in (dx, dh, dt, ds):
            b.close()
    if status:
        raise SynapseError(2, "sample: top-p over more than 4096 candidates")
    return tok


def stdrng_f32(seed: int, n: int) -> np.ndarray:
    out = np.zeros(max(n, 1), np.float32)
    check(lib().syn_hip_stdrng_f32(seed, n, ptr(out)), "stdrng_f32")
    return out[:n]


def kquant_encode(fmt: int, w: np.ndarray) -> np.ndarray:
    """Encode f32 [n, k] into GGUF block bytes (host-side encoder of the library)."""
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    be, bb = KQ_BLOCK[fmt]
    out = np.empty(n * (k // be) * bb, np.uint8)
    check(lib().syn_hip_kquant_encode(fmt, n, k, ptr(w), ptr(out)), "kquant_encode")
    return out


def kquant_decode(fmt: int, blocks: np.ndarray) -> np.ndarray:
    """Host dequantization of Q8_0 / Q4_K / Q6_K block bytes (the reference's values)."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    be, bb = KQ_BLOCK[fmt]
    nb = blocks.size // bb
    out = np.empty(nb * be, np.float32)
    check(lib().syn_hip_kquant_decode(fmt, nb, ptr(blocks), ptr(out)), "kquant_decode")
    return out


def fill_normal(n: int, seed: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib().syn_hip_fill_normal(ptr(out), n, seed, std))
    return out


def probe_mfma(kind: int, iters: int = 20000) -> float:
    """Measured dense MFMA rate: kind 0 = f16 16x16x32, 2 = f16 32x32x16 (TFLOP/s);
    1 = i8 16x16x64, 3 = i8 32x32x32 (TOP/s)."""
    v = C.c_double()
    check(lib().syn_hip_probe_mfma(kind, iters, C.byref(v)), "probe_mfma")
    return v.value


def probe_seq_sum(values):
    """(one-lane chain, wave chain, its clocks, long-row wave chain, its
    clocks) of the device's reference-order sequential sum of `values`
    (float32)."""
    v = np.ascontiguousarray(values, np.float32)
    out = np.zeros(5, np.float32)
    check(lib().syn_hip_probe_seq_sum(ptr(v), v.size, ptr(out)), "probe_seq_sum")
    return tuple(float(o) for o in out)


def probe_graph_floor(n: int = 140, wgs: int = 256) -> float:
    """us per kernel of a graph replay of n dependent tiny kernels"""
    v = C.c_double()
    check(lib().syn_hip_probe_graph_floor(n, wgs, C.byref(v)), "probe_graph_floor")
    return v.value


def probe_grid_barrier(wgs: int, mode: int, nbar: int = 200):
    """(us per grid barrier, timed-out waits) inside one cooperative launch"""
    v, t = C.c_double(), C.c_int()
    check(lib().syn_hip_probe_grid_barrier(wgs, mode, nbar, C.byref(v), C.byref(t)),
          "probe_grid_barrier")
    return v.value, t.value


def probe_hbm_read(nbytes: int = 4 << 30) -> float:
    """Measured streaming-read bandwidth of HBM (GB/s)."""
    v = C.c_double()
    check(lib().syn_hip_probe_hbm_read(nbytes, C.byref(v)), "probe_hbm_read")
    return v.value
