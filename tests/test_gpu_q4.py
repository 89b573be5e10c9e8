"""Q4_0 GEMV parity on the GPU: max_j|y-r| / max_j|r| <= 1e-3 per output row
set (north-star float tolerance) against the oracle's q4_0GemvRow."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip

pytestmark = pytest.mark.gpu

TOL = 1e-3  # north star: max relative error per row, metric max|y-r| / max|r|


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def _random_packed(n, k, seed):
    """Random Q4_0 blocks: nibbles uniform, f16 scales ~ N(0,0.02)/7 magnitudes."""
    rng = np.random.default_rng(seed)
    b = k // 32
    blocks = rng.integers(0, 256, (n, b, 18), dtype=np.uint8)
    sc = (np.abs(rng.standard_normal((n, b))) * 0.006 + 1e-4).astype(np.float16)
    blocks[:, :, 0:2] = sc.view(np.uint8).reshape(n, b, 2)
    return blocks.reshape(-1)


@pytest.mark.parametrize("n,k", [(16, 64), (67, 2048), (5, 32), (3, 96), (64, 128)])
def test_q4_gemv_from_f32_weights(n, k):
    w = O.normal(n * k, n * 3 + k, 0.02).reshape(n, k)
    a = O.normal(k, k + 1, 1.0)
    packed = O.q4_pack(w)
    got = hip.q4_0_gemv(a, packed, n)
    want = O.q4_0_gemv(a, packed, n)
    assert _rel(got, want) <= TOL * 1e-2  # observed ~1e-7; tolerance is 1e-3


# LLaMA-3.2-1B shapes of the Q4_0 microbench (K -> N)
@pytest.mark.parametrize("k,n", [(2048, 2048), (2048, 512), (2048, 8192), (8192, 2048),
                                 (2048, 128256)])
def test_q4_gemv_llama_shapes(k, n):
    packed = _random_packed(n, k, k + n)
    a = O.normal(k, 5, 1.0)
    got = hip.q4_0_gemv(a, packed, n)
    want = O.q4_0_gemv(a, packed, n)
    assert _rel(got, want) <= TOL


def test_q4_handle_multi_row():
    n, k, m = 1000, 2048, 5
    w = O.normal(n * k, 77, 0.02).reshape(n, k)
    x = O.normal(m * k, 78, 1.0).reshape(m, k)
    lin = hip.QLinear.from_f32(hip.FMT_Q4_0, w)
    got = lin.forward(x)
    packed = O.q4_pack(w)
    for i in range(m):
        assert _rel(got[i], O.q4_0_gemv(x[i], packed, n)) <= TOL * 1e-2


@pytest.mark.parametrize("m", [1, 3])
def test_q4_split_k_slices_on_every_xcd_twice(m):
    """Three 64-row panels over a long K: the slices of a panel run on all
    eight XCDs (workgroup id x + 3y), so the one-launch K split's atomics,
    arrival counter and read-back cross XCDs; the second call checks the
    accumulators and counters were left cleared."""
    n, k = 192, 16384
    packed = _random_packed(n, k, 99)
    lin = hip.QLinear.q4_0(packed, n, k)
    for call in range(2):
        x = O.normal(m * k, 40 + call, 1.0).reshape(m, k)
        got = lin.forward(x)
        for i in range(m):
            assert _rel(got[i], O.q4_0_gemv(x[i], packed, n)) <= TOL * 1e-2, (call, i)


def test_q4_errors():
    L = hip.lib()
    a = np.zeros(40, np.float32)
    c = np.zeros(2, np.float32)
    b = np.zeros(100, np.uint8)
    assert L.syn_q4_0_gemv(2, 40, hip.ptr(a), hip.ptr(b), hip.ptr(c)) == 4  # k % 32
    assert L.syn_q4_0_gemv(0, 32, hip.ptr(a), hip.ptr(b), hip.ptr(c)) == 0
    assert L.syn_q4_0_gemv(2, 32, None, hip.ptr(b), hip.ptr(c)) == 1


def test_gguf_q4_0_subnormal_scale_semantics():
    """A Q4_0 block whose f16 delta is subnormal: the reference reads it as the
    Zig Q4 GEMV does (IEEE, qmatmul.zig:346-371) on the raw-block path, and
    halved on the dequantize_q4_0 path (gguf.rs:294-326, converter.rs:12-40);
    a handle created with gguf_dequant follows the latter."""
    n, k = 64, 64
    blk = np.zeros((n, k // 32, 18), np.uint8)
    deltas = np.array([0x0201, 0x0100, 0x3C00, 0x0003], np.uint16)  # 1.0 and three subnormals
    for r in range(n):
        for b in range(k // 32):
            blk[r, b, 0:2] = np.array([deltas[(r + b) % 4]], np.uint16).view(np.uint8)
            blk[r, b, 2:] = ((np.arange(16) * 7 + r + b) % 256).astype(np.uint8)
    packed = blk.reshape(-1)
    x = O.normal(k, 12, 1.0)
    ieee = hip.QLinear.q4_0(packed, n, k).forward(x[None, :])[0]
    np.testing.assert_allclose(ieee, O.q4_0_gemv(x, packed, n), rtol=1e-5)
    halved = hip.QLinear.q4_0(packed, n, k, gguf_dequant=True).forward(x[None, :])[0]
    deq = O.dequant("q4_0", packed, n * k).reshape(n, k).astype(np.float64)
    np.testing.assert_allclose(halved, deq @ x.astype(np.float64), rtol=1e-5, atol=0)
    # the two readings differ exactly by the halving of the subnormal blocks
    assert not np.allclose(ieee, halved)


# ------------------------------------------------------------------ prefill GEMM
# M > 16 rows run the f16 MFMA GEMM (kquant_gemm.hip with the Q4_0 plane
# decoder): weights (nibble - 8) * d and activations rounded once to f16, f32
# accumulation; each row must stay within the per-row tolerance of the
# reference's q4_0GemvRow (the oracle) and of the device GEMV.
@pytest.mark.parametrize("m,n,k", [(17, 96, 64), (40, 200, 96), (256, 2048, 2048),
                                   (512, 512, 2048), (2048, 1024, 2048),
                                   # >= 192 tiles of 256 x 256: the direct-load kernel
                                   (2048, 6144, 96), (2000, 12300, 64), (2048, 8192, 2048)])
def test_q4_gemm_rows_match_gemv_rows(m, n, k):
    packed = _random_packed(n, k, m * 7 + n + k)
    x = O.normal(m * k, m + 3, 1.0).reshape(m, k)
    lin = hip.QLinear.q4_0(packed, n, k)
    got = lin.forward(x)
    rows = sorted(set([0, 1, m // 2, m - 1] + list(range(0, m, max(1, m // 24)))))
    worst = 0.0
    for i in rows:
        want = O.q4_0_gemv(x[i], packed, n)
        worst = max(worst, _rel(got[i], want))
        dev = lin.forward(x[i:i + 1])[0]  # the GEMV kernel for one row
        assert _rel(got[i], dev) <= TOL
    print(f"m={m} n={n} k={k} worst row rel {worst:.2e}")
    assert worst <= TOL


def test_q4_gemm_halved_subnormal_scales_use_the_gemv():
    # gguf_dequant handles whose scales include subnormals keep the GEMV
    # (its scale reading halves them); IEEE handles run the GEMM
    n, k, m = 64, 64, 24
    blk = np.zeros((n, k // 32, 18), np.uint8)
    for r in range(n):
        for b in range(k // 32):
            d = 0x0003 if (r + b) % 3 == 0 else 0x2C00
            blk[r, b, 0:2] = np.array([d], np.uint16).view(np.uint8)
            blk[r, b, 2:] = ((np.arange(16) * 5 + r + 3 * b) % 256).astype(np.uint8)
    packed = blk.reshape(-1)
    x = O.normal(m * k, 31, 1.0).reshape(m, k)
    halved = hip.QLinear.q4_0(packed, n, k, gguf_dequant=True).forward(x)
    deq = O.dequant("q4_0", packed, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T
    # per-row metric: elementwise relative error of near-cancelling dot
    # products says nothing about the scale reading
    assert max(_rel(halved[i], want[i]) for i in range(m)) <= 1e-5
    ieee = hip.QLinear.q4_0(packed, n, k).forward(x)
    for i in (0, m - 1):
        assert _rel(ieee[i], O.q4_0_gemv(x[i], packed, n)) <= TOL


# ---------------------------------------------------------------- output range
# Rows of ~1e-7 and ~1e6, and rows fed a few 1e4 outliers, through the K
# split (split_k.hpp: per-slice f32 slots added in slice order) against
# q4_0GemvRow (qmatmul.zig:276-343), both through the reference-signature
# export and a handle at several rows.
def _range_rows(m, k, seed, kind, scale):
    x = O.normal(m * k, seed, 1.0).reshape(m, k) * np.float32(scale)
    if kind == "outliers":
        rng = np.random.default_rng(seed)
        for i in range(m):
            idx = rng.choice(k, 3, replace=False)
            x[i, idx] = np.float32(1e4) * rng.choice([-1, 1], 3)
    return np.ascontiguousarray(x, np.float32)


@pytest.mark.parametrize("kind,scale", [("tiny", 1e-6), ("huge", 1e6), ("outliers", 1.0)])
@pytest.mark.parametrize("k,n", [(2048, 512), (8192, 2048), (8192, 300)])
def test_q4_gemv_output_range(k, n, kind, scale):
    print("case", k, n, kind, flush=True)
    w = O.normal(n * k, k + n + 2, 0.02).reshape(n, k)
    packed = O.q4_pack(w)
    a = _range_rows(1, k, k + 9, kind, scale)[0]
    got = hip.q4_0_gemv(a, packed, n)
    want = O.q4_0_gemv(a, packed, n)
    assert np.isfinite(got).all()
    assert _rel(got, want) <= TOL, _rel(got, want)
    lin = hip.QLinear.from_f32(hip.FMT_Q4_0, w)
    x = _range_rows(3, k, k + 10, kind, scale)
    got = lin.forward(x)
    for i in range(3):
        want = O.q4_0_gemv(x[i], packed, n)
        assert _rel(got[i], want) <= TOL, (i, _rel(got[i], want))


@pytest.mark.parametrize("kind,scale", [("tiny", 1e-6), ("huge", 1e5), ("outliers", 1.0)])
@pytest.mark.parametrize("m", [20, 300])
def test_q4_gemm_rows_output_range(m, kind, scale):
    # M > 16 rows run the f16 MFMA GEMM; each activation row is scaled by a
    # power of two into f16's range first (|x| ~ 1e5 would round to inf,
    # ~1e-6 to subnormal f16), and the rows still match q4_0GemvRow
    print("case", m, kind, flush=True)
    n, k = 512, 2048
    w = O.normal(n * k, 91, 0.02).reshape(n, k)
    packed = O.q4_pack(w)
    lin = hip.QLinear.from_f32(hip.FMT_Q4_0, w)
    x = _range_rows(m, k, 92 + m, kind, scale)
    got = lin.forward(x)
    assert np.isfinite(got).all()
    for i in sorted({0, 1, m // 2, m - 1}):
        want = O.q4_0_gemv(x[i], packed, n)
        assert _rel(got[i], want) <= TOL, (i, _rel(got[i], want))
