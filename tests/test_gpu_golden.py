"""The HIP path against the committed golden fixtures (tests/golden/*.npz),
through the C ABI: bit-exact for the integer paths and the INT8 decoder,
within the north star's float bars for the GGUF-block GEMVs and Mamba."""
import os

import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests.golden import make_golden as G

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def rel_row(y, r):
    """max_j |y - r| / max_j |r| (the per-row relative error of the north star)"""
    return float(np.abs(y.astype(np.float64) - r).max() / np.abs(r.astype(np.float64)).max())


def test_quantize_rows_golden():
    d = load("quantize_rows.npz")
    q, s = hip.quantize_per_channel_int8(d["x"])
    np.testing.assert_array_equal(q, d["q"])
    np.testing.assert_array_equal(bits(s), bits(d["s"]))


@pytest.mark.parametrize("m,k,n", G.INT8_SHAPES)
def test_int8_gemm_golden(m, k, n):
    d = load("int8_gemm.npz")
    key = f"{m}x{k}x{n}"
    a, sa, b, sb = G.int8_inputs(m, k, n)
    assert G.sha(a, sa, b, sb) == str(d[f"{key}_inputs_sha"])
    np.testing.assert_array_equal(bits(hip.qgemm_int8(a, b, sa, sb)), bits(d[f"{key}_c"]))
    # the device-resident handle ([K,N] weights repacked once) gives the same bits
    lin = hip.QLinear.int8(b, sb, hip.LAYOUT_KN)
    try:
        ldq = (k + 15) // 16 * 16  # activation rows in whole 16-byte chunks
        apad = np.zeros((m, ldq), np.int8)
        apad[:, :k] = a
        xq = hip.DeviceBuffer.from_array(apad)
        xs = hip.DeviceBuffer.from_array(sa)
        y = hip.DeviceBuffer(m * n * 4)
        lin.forward_pre_quantized_dev(m, xq.ptr, ldq, xs.ptr, y.ptr)
        hip.check(hip.lib().syn_hip_synchronize())
        np.testing.assert_array_equal(bits(y.download((m, n), np.float32)), bits(d[f"{key}_c"]))
        for buf in (xq, xs, y):
            buf.close()
    finally:
        lin.close()


@pytest.mark.parametrize("n,k", [(16, 64), (64, 2048)])
def test_q4_0_golden(n, k):
    d = load("q4_0.npz")
    key = f"{n}x{k}"
    w, a = G.q4_inputs(n, k)
    assert G.sha(w) == str(d[f"{key}_w_sha"])
    packed = d[f"{key}_packed"] if f"{key}_packed" in d else O.q4_pack(w)
    assert G.sha(packed) == str(d[f"{key}_packed_sha"])
    y = hip.q4_0_gemv(d[f"{key}_a"], packed, n)
    assert rel_row(y, d[f"{key}_y"]) <= 1e-3
    # the library's own producer (Q4Linear::from_f32 + pack_for_zig) on the device
    lin = hip.QLinear.from_f32(hip.FMT_Q4_0, w)
    try:
        assert rel_row(lin.forward(d[f"{key}_a"].reshape(1, k)).reshape(n), d[f"{key}_y"]) <= 1e-3
    finally:
        lin.close()


@pytest.mark.parametrize("fmt", list(G.KQ_GEMV))
def test_kquant_gemv_golden(fmt):
    d = load("kquant.npz")
    n, k = G.KQ_GEMV[fmt]
    code = {"q8_0": hip.FMT_Q8_0, "q4_k": hip.FMT_Q4_K, "q6_k": hip.FMT_Q6_K}[fmt]
    lin = hip.QLinear.gguf(code, d[f"{fmt}_blocks"], n, k)
    try:
        y = lin.forward(d[f"{fmt}_x"].reshape(1, k)).reshape(n)
    finally:
        lin.close()
    assert rel_row(y, d[f"{fmt}_y"]) <= 1e-3


def test_qwen3_tiny_golden():
    d = load("qwen3_tiny_w8a8.npz")
    g = hip.QuantizedCausalLM(G.QWEN3_TINY)
    try:
        g.init_synthetic(G.SEED, G.QWEN3_TINY_STD)
        np.testing.assert_array_equal(bits(g.prefill(d["prompt"])), bits(d["prefill_logits"]))
        g.reset()
        toks, margins = g.generate(d["prompt"], 16)
    finally:
        g.close()
    np.testing.assert_array_equal(toks, d["tokens"])
    np.testing.assert_array_equal(bits(margins), bits(d["margins"]))


def test_mamba_tiny_golden():
    d = load("mamba_tiny_int8.npz")
    g = hip.QuantizedMamba(dict(G.MAMBA_TINY, max_tokens=32))
    try:
        g.init_synthetic(G.SEED)
        lg = g.prefill(d["prompt"])
    finally:
        g.close()
    r = d["prefill_logits"].astype(np.float64)
    cos = float(lg.astype(np.float64) @ r / (np.linalg.norm(lg) * np.linalg.norm(r)))
    assert cos >= 0.9999
    g = hip.QuantizedMamba(dict(G.MAMBA_TINY, max_tokens=32))
    try:
        g.init_synthetic(G.SEED)
        toks, _ = g.generate(d["prompt"], 12)
    finally:
        g.close()
    # the oracle's top1-top2 margins are all far above float noise (>= 0.9)
    assert d["margins"].min() > 0.1
    np.testing.assert_array_equal(toks, d["tokens"])
