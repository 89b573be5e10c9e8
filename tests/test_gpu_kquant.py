"""Q8_0 / Q4_K / Q6_K on the GPU against the reference semantics: the oracle
dequantizes the same bytes (gguf.rs:255-487) and runs matmul_t
(ops/matmul.rs:55-79, sgemm/f32GemvRow order).  Tolerance: the north star's
max_j|y-r| / max_j|r| <= 1e-3 per output row set."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip

pytestmark = pytest.mark.gpu
TOL = 1e-3
FMTS = {"q8_0": hip.FMT_Q8_0, "q4_k": hip.FMT_Q4_K, "q6_k": hip.FMT_Q6_K}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.mark.parametrize("name", list(FMTS))
def test_encoder_roundtrip_quality(name):
    # the library's encoder writes the reference byte format; the oracle's
    # dequantizer (reference semantics) must give back the weights closely
    n, k = 64, 1024
    w = O.normal(n * k, 11, 0.02).reshape(n, k)
    blocks = hip.kquant_encode(FMTS[name], w)
    deq = O.dequant(name, blocks, n * k).reshape(n, k)
    err = np.abs(deq - w).max() / np.abs(w).max()
    assert err < {"q8_0": 0.01, "q4_k": 0.12, "q6_k": 0.04}[name], err
    # correlation close to 1
    c = float(np.corrcoef(deq.ravel(), w.ravel())[0, 1])
    assert c > {"q8_0": 0.9999, "q4_k": 0.99, "q6_k": 0.999}[name], c


CASES = [("q8_0", 4096, 4096, 1), ("q8_0", 4096, 1024, 3), ("q8_0", 14336, 4096, 1),
         ("q8_0", 96, 100, 4), ("q4_k", 3072, 3072, 1), ("q4_k", 3072, 1024, 2),
         ("q4_k", 3072, 8192, 1), ("q4_k", 512, 67, 5), ("q6_k", 8192, 3072, 1),
         ("q6_k", 3072, 1000, 3), ("q6_k", 256, 65, 7),
         # up to 8 rows run as one launch (a speculative verify of k = 7)
         ("q4_k", 3072, 5120, 8), ("q8_0", 4096, 1024, 6)]


@pytest.mark.parametrize("name,k,n,m", CASES)
def test_kquant_gemv_vs_reference(name, k, n, m):
    w = O.normal(n * k, k + n, 0.02).reshape(n, k)
    blocks = hip.kquant_encode(FMTS[name], w)
    lin = hip.QLinear.gguf(FMTS[name], blocks, n, k)
    x = O.normal(m * k, 7 * m + k, 1.0).reshape(m, k)
    got = lin.forward(x)
    deq = O.dequant(name, blocks, n * k).reshape(n, k)
    want = O.matmul_t(x, deq)
    for i in range(m):
        assert _rel(got[i], want[i]) <= TOL * 0.1, (i, _rel(got[i], want[i]))


@pytest.mark.parametrize("name,m", [("q4_k", 1), ("q6_k", 1), ("q8_0", 3), ("q4_k", 4),
                                    ("q8_0", 6), ("q6_k", 8)])
def test_split_k_slices_on_every_xcd_twice(name, m):
    """Three 64-row panels over a long K: the slices of a panel land on all
    eight XCDs (workgroup id x + 3y), so the one-launch K split's atomics,
    arrival counter and read-back cross XCDs; a second call checks that the
    accumulators and counters were left cleared."""
    n, k = 192, 16384
    w = O.normal(n * k, 5, 0.02).reshape(n, k)
    blocks = hip.kquant_encode(FMTS[name], w)
    lin = hip.QLinear.gguf(FMTS[name], blocks, n, k)
    deq = O.dequant(name, blocks, n * k).reshape(n, k)
    for call in range(2):
        x = O.normal(m * k, 17 + call, 1.0).reshape(m, k)
        got = lin.forward(x)
        want = O.matmul_t(x, deq)
        for i in range(m):
            assert _rel(got[i], want[i]) <= TOL * 0.1, (call, i, _rel(got[i], want[i]))


def test_q6_k_lm_head_shape():
    # LLaMA-3.2-3B lm_head: 128256 x 3072 Q6_K, random blocks
    n, k = 128256, 3072
    rng = np.random.default_rng(5)
    nb = k // 256
    blk = rng.integers(0, 256, (n, nb, 210), dtype=np.uint8)
    blk[:, :, 192:208] = rng.integers(-40, 41, (n, nb, 16), dtype=np.int8).view(np.uint8)
    d = (rng.uniform(1e-5, 3e-5, (n, nb))).astype(np.float16)
    blk[:, :, 208:210] = d.view(np.uint8).reshape(n, nb, 2)
    blk = blk.reshape(-1)
    lin = hip.QLinear.gguf(hip.FMT_Q6_K, blk, n, k)
    x = O.normal(k, 3, 1.0).reshape(1, k)
    got = lin.forward(x)[0]
    deq = O.dequant("q6_k", blk, n * k).reshape(n, k)
    want = O.matmul_t(x, deq)[0]
    assert _rel(got, want) <= TOL * 0.1


def test_subnormal_scale_semantics():
    # converter.rs halves subnormal f16 scales; the device decoder must agree
    n, k = 64, 32
    blk = np.zeros((n, 34), np.uint8)
    blk[:, 0:2] = np.array([0x0200], np.uint16).view(np.uint8)  # subnormal d
    blk[:, 2:] = np.arange(1, 33, dtype=np.int8).view(np.uint8)
    blk = blk.reshape(-1)
    lin = hip.QLinear.gguf(hip.FMT_Q8_0, blk, n, k)
    x = np.ones((1, k), np.float32)
    got = lin.forward(x)[0]
    deq = O.dequant("q8_0", blk, n * k).reshape(n, k)
    np.testing.assert_allclose(got, deq.sum(axis=1), rtol=1e-6)
    assert deq[0, 0] == np.float32(2.0 ** -16)  # half of IEEE 2^-15


def test_kquant_shape_errors():
    w = np.zeros((4, 100), np.float32)
    with pytest.raises(hip.SynapseError):
        hip.QLinear.from_f32(hip.FMT_Q4_K, w)  # k % 256


GEMM_CASES = [("q8_0", 40, 4096, 1024), ("q8_0", 300, 1024, 512), ("q4_k", 64, 3072, 384),
              ("q6_k", 33, 2048, 200), ("q4_k", 9, 512, 130), ("q8_0", 129, 96, 257)]


@pytest.mark.parametrize("name,m,k,n", GEMM_CASES)
def test_kquant_gemm_vs_reference(name, m, k, n):
    # M > 8: f16 MFMA prefill GEMM; reference = dequant + sgemmTiled semantics
    w = O.normal(n * k, 3 * k + n, 0.02).reshape(n, k)
    blocks = hip.kquant_encode(FMTS[name], w)
    lin = hip.QLinear.gguf(FMTS[name], blocks, n, k)
    x = O.normal(m * k, m + k, 1.0).reshape(m, k)
    got = lin.forward(x)
    deq = O.dequant(name, blocks, n * k).reshape(n, k)
    want = O.matmul_t(x, deq)
    worst = max(_rel(got[i], want[i]) for i in range(m))
    print(f"{name} {m}x{k}->{n}: worst per-row rel err {worst:.2e}")
    assert worst <= TOL, worst


def test_kquant_gemm_mistral_shape_sampled_rows():
    # config 4 shape (Q8_0 gate/up 4096 -> 14336, M = 512): check sampled rows in f64
    m, k, n = 512, 4096, 14336
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    blocks = hip.kquant_encode(hip.FMT_Q8_0, w)
    lin = hip.QLinear.gguf(hip.FMT_Q8_0, blocks, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = lin.forward(x)
    deq = O.dequant("q8_0", blocks, n * k).reshape(n, k).astype(np.float64)
    for i in (0, 1, 255, 511):
        want = deq @ x[i].astype(np.float64)
        assert _rel(got[i], want) <= TOL


@pytest.mark.parametrize("name", ["q8_0", "q4_k", "q6_k"])
def test_kquant_gemm_256x256_tiles(name):
    # 8 x 24 tiles of 256 x 256 (the four-wave kernel), ragged M and N
    m, k, n = 2000, 512, 6100
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    blocks = hip.kquant_encode(FMTS[name], w)
    lin = hip.QLinear.gguf(FMTS[name], blocks, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    got = lin.forward(x)
    deq = O.dequant(name, blocks, n * k).reshape(n, k).astype(np.float64)
    for i in (0, 1, 127, 255, 256, 1024, 1999):
        want = deq @ x[i].astype(np.float64)
        assert _rel(got[i], want) <= TOL, i
    # every output column of one row block, against the f64 product
    want = x[1792:1800].astype(np.float64) @ deq.T
    worst = max(_rel(got[1792 + i], want[i]) for i in range(8))
    assert worst <= TOL, worst


# ---------------------------------------------------------------- output range
# The one-launch K split adds per-slice f32 sums in slice order (split_k.hpp),
# so rows keep f32's range: outputs ~1e-7 (activations x 1e-6), ~1e6
# (activations x 1e6) and rows fed a few 1e4 outliers stay within the float
# bar of the reference chain (qmatmul.zig:276-343 for Q4_0, matmul_t over
# the dequantized weights for the GGUF formats).
RANGE_SCALES = [("tiny", 1e-6), ("huge", 1e6), ("outliers", 1.0)]


def _range_rows(m, k, seed, kind, scale):
    x = O.normal(m * k, seed, 1.0).reshape(m, k) * np.float32(scale)
    if kind == "outliers":
        rng = np.random.default_rng(seed)
        for i in range(m):
            idx = rng.choice(k, 3, replace=False)
            x[i, idx] = np.float32(1e4) * rng.choice([-1, 1], 3)
    return np.ascontiguousarray(x, np.float32)


# shapes whose GEMV runs as a K split (k large against n)
RANGE_CASES = [("q8_0", 4096, 1024, 1), ("q8_0", 8192, 512, 3), ("q4_k", 3072, 1024, 1),
               ("q4_k", 8192, 512, 2), ("q6_k", 8192, 1024, 1), ("q6_k", 8192, 300, 3)]


@pytest.mark.parametrize("kind,scale", RANGE_SCALES, ids=[r[0] for r in RANGE_SCALES])
@pytest.mark.parametrize("name,k,n,m", RANGE_CASES)
def test_kquant_gemv_output_range(name, k, n, m, kind, scale):
    print("case", name, k, n, m, kind, flush=True)
    w = O.normal(n * k, k + n + 1, 0.02).reshape(n, k)
    blocks = hip.kquant_encode(FMTS[name], w)
    lin = hip.QLinear.gguf(FMTS[name], blocks, n, k)
    x = _range_rows(m, k, 3 * m + k, kind, scale)
    got = lin.forward(x)
    deq = O.dequant(name, blocks, n * k).reshape(n, k)
    want = O.matmul_t(x, deq)
    assert np.isfinite(got).all()
    for i in range(m):
        assert _rel(got[i], want[i]) <= TOL, (i, _rel(got[i], want[i]))


@pytest.mark.parametrize("kind,scale", RANGE_SCALES, ids=[r[0] for r in RANGE_SCALES])
@pytest.mark.parametrize("name", list(FMTS))
def test_kquant_gemm_output_range(name, kind, scale):
    # M > 8 rows run the f16 MFMA GEMM with power-of-two row scaling
    print("case", name, kind, flush=True)
    n, k, m = 384, 1024, 40
    w = O.normal(n * k, 57, 0.02).reshape(n, k)
    blocks = hip.kquant_encode(FMTS[name], w)
    lin = hip.QLinear.gguf(FMTS[name], blocks, n, k)
    x = _range_rows(m, k, 58, kind, scale)
    got = lin.forward(x)
    assert np.isfinite(got).all()
    deq = O.dequant(name, blocks, n * k).reshape(n, k)
    want = O.matmul_t(x, deq)
    for i in range(m):
        assert _rel(got[i], want[i]) <= TOL, (i, _rel(got[i], want[i]))
