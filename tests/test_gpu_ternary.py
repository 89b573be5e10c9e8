"""Ternary linear (ternary.hip) against the oracle's restatement of
TernaryLinear: the device producer gives the reference's block bytes, and
the GEMV gives the reference's forward() bit for bit (same per-block order,
same chain over the blocks)."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests.test_ternary import pseudo_random_vec

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n,k,m", [(8, 32, 4), (64, 1024, 1), (100, 2048, 1), (2048, 2048, 1),
                                   (512, 8192, 2), (37, 1000, 3), (3, 16, 1), (130, 5000, 1)])
def test_ternary_gemv_bit_exact(n, k, m):
    rng = np.random.default_rng(n + k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    blocks = O.ternary_from_f32(w)
    want = O.ternary_forward(blocks, n, k, x)
    lin = hip.QLinear.ternary(blocks, n, k)
    try:
        np.testing.assert_array_equal(bits(lin.forward(x)), bits(want))
    finally:
        lin.close()
    lin = hip.QLinear.from_f32(hip.FMT_TERNARY, w)  # the library's producer
    try:
        np.testing.assert_array_equal(bits(lin.forward(x)), bits(want))
        assert lin.weight_bytes == blocks.size
    finally:
        lin.close()


def test_ternary_reference_test_inputs():
    m, n, k = 4, 8, 32
    x = pseudo_random_vec(m * k, 42).reshape(m, k)
    w = pseudo_random_vec(n * k, 123).reshape(n, k)
    lin = hip.QLinear.from_f32(hip.FMT_TERNARY, w)
    try:
        y = lin.forward(x)
    finally:
        lin.close()
    np.testing.assert_array_equal(bits(y), bits(O.ternary_forward(O.ternary_from_f32(w), n, k, x)))
