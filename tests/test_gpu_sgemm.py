"""syn_sgemm (synapse.h:176-184, exports.zig:725-761) and the syn_hip_-prefixed
aliases of the reference-signature entry points, through the C ABI, bit for
bit against the oracle's sgemmTiled restatement (matmul.zig:125-184)."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# (m, n, k): the GEMV path (m <= 16) with its 32/8-wide column blocks and
# tails, the GOTO path with partial 8-row panels, a partial 256-row block and
# a partial 4096-column block
SHAPES = [(1, 1000, 300), (5, 77, 33), (16, 40, 9), (17, 300, 40), (33, 19, 70),
          (260, 50, 16), (20, 4100, 12)]


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_matches_reference(m, n, k, ta, tb):
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)  # the GOTO path accumulates
    np.testing.assert_array_equal(_bits(hip.sgemm(a, b, ta, tb, c0)),
                                  _bits(O.sgemm(a, b, ta, tb, c0)))
    # and it is the product (float64 check of the semantics, not the bits)
    want = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    if not (m <= 16 and not ta):
        want += c0
    got = hip.sgemm(a, b, ta, tb, c0)
    assert np.abs(got - want).max() <= 1e-4 * max(1.0, np.abs(want).max())


def test_sgemm_status_codes():
    L = hip.lib()
    f = np.zeros(16, np.float32)
    assert L.syn_sgemm(0, 2, 2, hip.ptr(f), 2, 0, hip.ptr(f), 2, 0, hip.ptr(f), 2) == 0
    assert L.syn_sgemm(2, 2, 2, None, 2, 0, hip.ptr(f), 2, 0, hip.ptr(f), 2) == 1
    assert L.syn_sgemm(2, 2, 2, hip.ptr(f), 2, 0, hip.ptr(f), 2, 0, None, 2) == 1
    # identity KAT (ops/matmul.rs:126-180)
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    np.testing.assert_array_equal(hip.sgemm(a, np.eye(4, dtype=np.float32)), a)


def test_prefixed_aliases_match():
    L = hip.lib()
    rng = np.random.default_rng(3)
    a = rng.standard_normal((20, 64)).astype(np.float32)
    b = rng.standard_normal((64, 30)).astype(np.float32)
    c1 = np.zeros((20, 30), np.float32)
    c2 = np.zeros((20, 30), np.float32)
    hip.check(L.syn_sgemm(20, 30, 64, hip.ptr(a), 64, 0, hip.ptr(b), 30, 0, hip.ptr(c1), 30))
    hip.check(L.syn_hip_sgemm(20, 30, 64, hip.ptr(a), 64, 0, hip.ptr(b), 30, 0, hip.ptr(c2), 30))
    np.testing.assert_array_equal(_bits(c1), _bits(c2))
    x = rng.standard_normal((3, 64)).astype(np.float32)
    q1, s1 = np.zeros((3, 64), np.int8), np.zeros(3, np.float32)
    q2, s2 = np.zeros((3, 64), np.int8), np.zeros(3, np.float32)
    hip.check(L.syn_quantize_per_channel_int8(hip.ptr(x), 3, 64, hip.ptr(q1), hip.ptr(s1)))
    hip.check(L.syn_hip_quantize_per_channel_int8(hip.ptr(x), 3, 64, hip.ptr(q2), hip.ptr(s2)))
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(_bits(s1), _bits(s2))
    bq = rng.integers(-127, 128, (64, 30)).astype(np.int8)
    sb = rng.random(30).astype(np.float32)
    g1, g2 = np.zeros((3, 30), np.float32), np.zeros((3, 30), np.float32)
    hip.check(L.syn_qgemm_int8(3, 30, 64, hip.ptr(q1), 64, hip.ptr(bq), 30, hip.ptr(g1), 30,
                               hip.ptr(s1), hip.ptr(sb)))
    hip.check(L.syn_hip_qgemm_int8(3, 30, 64, hip.ptr(q1), 64, hip.ptr(bq), 30, hip.ptr(g2), 30,
                                   hip.ptr(s1), hip.ptr(sb)))
    np.testing.assert_array_equal(_bits(g1), _bits(g2))
    w = O.normal(30 * 64, 4, 0.02).reshape(30, 64)
    packed = O.q4_pack(w)
    y1, y2 = np.zeros(30, np.float32), np.zeros(30, np.float32)
    hip.check(L.syn_q4_0_gemv(30, 64, hip.ptr(x[0]), hip.ptr(packed), hip.ptr(y1)))
    hip.check(L.syn_hip_q4_0_gemv(30, 64, hip.ptr(x[0]), hip.ptr(packed), hip.ptr(y2)))
    np.testing.assert_array_equal(_bits(y1), _bits(y2))
