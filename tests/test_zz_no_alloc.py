"""syn_hip_qlinear_forward_noalloc (INT8, no allocation: the library's fixed
device scratch) against syn_hip_qlinear_forward and the oracle, bit for bit,
over consecutive calls that shrink (the scratch keeps the previous call's
contents) and across the GEMV (M <= 16, split-K partials) and both GEMM
paths (K a multiple of 128: direct global->LDS loads; other K: register
staging)."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _linear(n, k, seed):
    w = O.normal(n * k, seed, 0.02).reshape(n, k)
    return hip.QLinear.from_f32(hip.FMT_INT8, w), w


def _both(lin, x):
    m = x.shape[0]
    dx = hip.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    y_ref = hip.DeviceBuffer(m * lin.n * 4)
    y_na = hip.DeviceBuffer(m * lin.n * 4)
    lin.forward_dev(m, dx.ptr, y_ref.ptr)
    lin.forward_noalloc_dev(m, dx.ptr, y_na.ptr)
    hip.check(hip.lib().syn_hip_stream_synchronize(None))
    return y_ref.download((m, lin.n), np.float32), y_na.download((m, lin.n), np.float32)


# each case: two calls in a row, the second with a smaller input
# (4096, 1024, 128, 40): M > 16 with K a multiple of 128, the direct-load GEMM
@pytest.mark.parametrize("n,k,m1,m2", [(3072, 1024, 16, 1), (1024, 3072, 16, 3),
                                       (300, 700, 40, 5), (2048 + 17, 1000, 33, 17),
                                       (4096, 1024, 128, 40), (1000, 2048, 64, 17)])
def test_noalloc_matches_forward_on_shrinking_calls(n, k, m1, m2):
    print("case", n, k, m1, m2, flush=True)
    lin, w = _linear(n, k, 7)
    x1 = O.normal(m1 * k, 8, 1.0).reshape(m1, k)
    r1, a1 = _both(lin, x1)
    np.testing.assert_array_equal(_bits(a1), _bits(r1))
    x2 = O.normal(m2 * k, 9, 1.0).reshape(m2, k)
    r2, a2 = _both(lin, x2)
    np.testing.assert_array_equal(_bits(a2), _bits(r2))
    # and the reference: QuantizedLinear::forward (int8_linear.rs:87-117)
    q_kn, s = O.quantize_weights_int8(w)
    xq, sx = O.quantize_per_channel_int8(x2)
    np.testing.assert_array_equal(_bits(a2), _bits(O.qgemm_int8(xq, q_kn, sx, s)))


def test_noalloc_after_a_larger_linear():
    # a smaller linear after a larger one reuses the scratch the larger one left
    big, _ = _linear(1024, 3072, 11)
    small, _ = _linear(512, 96, 12)
    xb = O.normal(16 * 3072, 13, 1.0).reshape(16, 3072)
    r, a = _both(big, xb)
    np.testing.assert_array_equal(_bits(a), _bits(r))
    xs = O.normal(2 * 96, 14, 1.0).reshape(2, 96)
    r, a = _both(small, xs)
    np.testing.assert_array_equal(_bits(a), _bits(r))


def test_noalloc_rejects_more_than_the_scratch():
    lin, _ = _linear(64, 4096, 15)
    m = 1100  # 1100 rows x 4096 bytes > 4 MiB
    dx = hip.DeviceBuffer(m * 4096 * 4)
    dy = hip.DeviceBuffer(m * 64 * 4)
    with pytest.raises(hip.SynapseError):
        lin.forward_noalloc_dev(m, dx.ptr, dy.ptr)
    assert "scratch" in hip.last_error()


def test_noalloc_rejects_other_formats():
    w = O.normal(64 * 64, 16, 0.02).reshape(64, 64)
    lin = hip.QLinear.from_f32(hip.FMT_Q4_0, w)
    dx = hip.DeviceBuffer(64 * 4)
    dy = hip.DeviceBuffer(64 * 4)
    with pytest.raises(hip.SynapseError):
        lin.forward_noalloc_dev(1, dx.ptr, dy.ptr)
