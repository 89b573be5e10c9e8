"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) against the CPU oracle and the library's host
code: every expectation must still be reproduced bit for bit, and the inputs
regenerated from the seed spec must still hash to what the fixtures recorded."""
import os

import numpy as np
import pytest

import oracle as O
from tests.golden import make_golden as G

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_quantize_rows_fixture():
    d = load("quantize_rows.npz")
    q, s = O.quantize_per_channel_int8(d["x"])
    np.testing.assert_array_equal(q, d["q"])
    np.testing.assert_array_equal(bits(s), bits(d["s"]))
    # the planted cases: zero row, exact half rounded away from zero
    assert d["s"][1] == 1.0 and not d["q"][1].any()
    assert d["q"][2, 0] == 127 and (d["q"][2, 1:] == 1).all()
    # negating a row negates its codes and keeps its scale
    qn, sn = O.quantize_per_channel_int8(-d["x"][4:5])
    np.testing.assert_array_equal(qn[0], -d["q"][4])
    assert bits(sn)[0] == bits(d["s"])[4]


@pytest.mark.parametrize("m,k,n", G.INT8_SHAPES)
def test_int8_gemm_fixture(m, k, n):
    d = load("int8_gemm.npz")
    key = f"{m}x{k}x{n}"
    a, sa, b, sb = G.int8_inputs(m, k, n)
    assert G.sha(a, sa, b, sb) == str(d[f"{key}_inputs_sha"])
    c = O.qgemm_int8(a, b, sa, sb)
    np.testing.assert_array_equal(bits(c), bits(d[f"{key}_c"]))
    # independent restatement from int64 products: M <= 16 scales the whole
    # i32 sum once (qmatmul.zig:54-66); M > 16 adds the scaled KC = 512
    # chunk sums in order (qmatmul.zig:68-99)
    kc = k if m <= 16 else 512
    ref = np.zeros((m, n), np.float32)
    for p in range(0, k, kc):
        acc = a[:, p:p + kc].astype(np.int64) @ b[p:p + kc].astype(np.int64)
        t = (acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sb[None, :]
        ref = (ref + t.astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(bits(c), bits(ref))


@pytest.mark.parametrize("n,k", [(16, 64), (64, 2048)])
def test_q4_0_fixture(n, k):
    d = load("q4_0.npz")
    key = f"{n}x{k}"
    w, a = G.q4_inputs(n, k)
    assert G.sha(w) == str(d[f"{key}_w_sha"])
    packed = O.q4_pack(w)
    assert G.sha(packed) == str(d[f"{key}_packed_sha"])
    if f"{key}_packed" in d:
        np.testing.assert_array_equal(packed, d[f"{key}_packed"])
    np.testing.assert_array_equal(bits(O.q4_0_gemv(d[f"{key}_a"], packed, n)),
                                  bits(d[f"{key}_y"]))


@pytest.mark.parametrize("fmt", list(G.KQ_GEMV))
def test_kquant_fixture(fmt):
    d = load("kquant.npz")
    n, k = G.KQ_GEMV[fmt]
    blocks = d[f"{fmt}_blocks"]
    w = O.dequant(fmt, blocks, n * k)
    np.testing.assert_array_equal(bits(w), bits(d[f"{fmt}_dequant"].reshape(-1)))
    y = O.matmul_t(d[f"{fmt}_x"].reshape(1, k), w.reshape(n, k)).reshape(n)
    np.testing.assert_array_equal(bits(y), bits(d[f"{fmt}_y"]))


@pytest.mark.parametrize("fmt", list(G.KQ_GEMV))
def test_kquant_fixture_host_decoder(fmt):
    """The library's host dequantizer (no GPU needed) gives the fixture's values."""
    from synapse_amd import hip
    d = load("kquant.npz")
    code = {"q8_0": hip.FMT_Q8_0, "q4_k": hip.FMT_Q4_K, "q6_k": hip.FMT_Q6_K}[fmt]
    w = hip.kquant_decode(code, d[f"{fmt}_blocks"])
    np.testing.assert_array_equal(bits(w), bits(d[f"{fmt}_dequant"].reshape(-1)))


def test_qwen3_tiny_fixture():
    d = load("qwen3_tiny_w8a8.npz")
    o = O.QuantizedCausalLM(G.QWEN3_TINY)
    o.init_synthetic(G.SEED, G.QWEN3_TINY_STD)
    ids = O.token_ids(8, G.SEED + 0xFFFF, G.QWEN3_TINY["vocab"])
    np.testing.assert_array_equal(ids, d["prompt"])
    np.testing.assert_array_equal(bits(o.prefill(ids)), bits(d["prefill_logits"]))
    o.reset()
    toks, margins = o.generate(ids, 16)
    o.close()
    np.testing.assert_array_equal(toks, d["tokens"])
    np.testing.assert_array_equal(bits(margins), bits(d["margins"]))
    assert len(set(d["tokens"].tolist())) > 1  # a sequence that actually moves


def test_mamba_tiny_fixture():
    d = load("mamba_tiny_int8.npz")
    o = O.QuantizedMamba(G.MAMBA_TINY)
    o.init_synthetic(G.SEED)
    np.testing.assert_array_equal(bits(o.prefill(d["prompt"])), bits(d["prefill_logits"]))
    o.close()
    o = O.QuantizedMamba(G.MAMBA_TINY)
    o.init_synthetic(G.SEED)
    toks, _ = o.generate(d["prompt"], 12)
    o.close()
    np.testing.assert_array_equal(toks, d["tokens"])
