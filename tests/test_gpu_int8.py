"""INT8 W8A8 parity on the GPU through the C ABI: bit-exact against the oracle."""
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


@pytest.mark.parametrize("m,k", [(1, 1024), (1, 2048), (1, 3072), (16, 1024), (5, 33), (3, 1)])
def test_quantize_rows_bit_exact(m, k):
    x = O.normal(m * k, 1000 + m * k, 3.0).reshape(m, k)
    x[0, 0] = 0.0
    if m > 2:
        x[1] = 0.0                         # zero row -> scale 1
        x[2, :] = 0.5
        x[2, 0] = 127.0                    # exact halves: round away from zero
    q, s = hip.quantize_per_channel_int8(x)
    qo, so = O.quantize_per_channel_int8(x)
    np.testing.assert_array_equal(q, qo)
    np.testing.assert_array_equal(_bits(s), _bits(so))


def test_quantize_rows_device_api_strided():
    m, k, ldx, ldq = 4, 1000, 1024, 1008
    x = O.normal(m * ldx, 5, 1.0).reshape(m, ldx)
    dx = hip.DeviceBuffer.from_array(x)
    dq = hip.DeviceBuffer(m * ldq)
    ds = hip.DeviceBuffer(m * 4)
    hip.check(hip.lib().syn_hip_quantize_rows(dx.ptr, m, k, ldx, dq.ptr, ldq, ds.ptr, None))
    hip.check(hip.lib().syn_hip_stream_synchronize(None))
    q = dq.download((m, ldq), np.int8)[:, :k]
    qo, so = O.quantize_per_channel_int8(np.ascontiguousarray(x[:, :k]))
    np.testing.assert_array_equal(q, qo)
    np.testing.assert_array_equal(_bits(ds.download(m, np.float32)), _bits(so))


SHAPES = [(1, 1024, 1024), (1, 1024, 3072), (1, 3072, 1024), (1, 2048, 1024), (1, 1024, 4096),
          (16, 1024, 2048), (2, 1024, 6144), (17, 33, 25), (33, 600, 40), (40, 1100, 130),
          (1, 1, 1), (3, 5000, 7), (1, 17, 65), (64, 1536, 200)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_qgemm_reference_signature_bit_exact(m, k, n):
    rng = np.random.default_rng(m * 131 + k * 7 + n)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    sa = rng.uniform(1e-3, 0.1, m).astype(np.float32)
    sb = rng.uniform(1e-3, 0.1, n).astype(np.float32)
    got = hip.qgemm_int8(a, b, sa, sb)
    want = O.qgemm_int8(a, b, sa, sb)
    np.testing.assert_array_equal(_bits(got), _bits(want))


def test_qgemm_kats_and_edges():
    # crates/synapse-core/src/lib.rs:1541-1573
    c = hip.qgemm_int8(np.array([[1, 2, 3], [4, 5, 6]], np.int8),
                       np.array([[7, 8], [9, 10], [11, 12]], np.int8),
                       np.ones(2, np.float32), np.ones(2, np.float32))
    assert c[0, 0] == 58 and c[0, 1] == 64
    c = hip.qgemm_int8(np.array([[127, 0], [0, 127]], np.int8),
                       np.array([[127, 0], [0, 127]], np.int8),
                       np.array([2.0, 3.0], np.float32), np.array([0.5, 1.0], np.float32))
    assert c[0, 0] == 16129.0
    L = hip.lib()
    dummy = np.zeros(4, np.int8)
    f = np.zeros(4, np.float32)
    # zero dims -> SYN_OK no-op (exports.zig:1331); null pointers -> NULL_PTR
    assert L.syn_qgemm_int8(0, 2, 2, hip.ptr(dummy), 2, hip.ptr(dummy), 2, hip.ptr(f), 2,
                            hip.ptr(f), hip.ptr(f)) == 0
    assert L.syn_qgemm_int8(1, 1, 1, None, 1, hip.ptr(dummy), 1, hip.ptr(f), 1, hip.ptr(f),
                            hip.ptr(f)) == 1
    assert L.syn_quantize_per_channel_int8(hip.ptr(f), 0, 4, hip.ptr(dummy), hip.ptr(f)) == 2


@pytest.mark.parametrize("layout", [hip.LAYOUT_KN, hip.LAYOUT_NK])
def test_qlinear_handle_pre_quantized(layout):
    m, k, n = 3, 1024, 2048 + 17
    w = O.normal(n * k, 42, 0.02).reshape(n, k)
    q_kn, s = O.quantize_weights_int8(w)
    lin = hip.QLinear.int8(q_kn if layout == hip.LAYOUT_KN else np.ascontiguousarray(q_kn.T), s,
                           layout)
    x = O.normal(m * k, 43, 1.0).reshape(m, k)
    xq, sx = O.quantize_per_channel_int8(x)
    ldq = 1024
    dxq = hip.DeviceBuffer.from_array(xq)
    dsx = hip.DeviceBuffer.from_array(sx)
    dy = hip.DeviceBuffer(m * n * 4)
    lin.forward_pre_quantized_dev(m, dxq.ptr, ldq, dsx.ptr, dy.ptr)
    hip.check(hip.lib().syn_hip_stream_synchronize(None))
    got = dy.download((m, n), np.float32)
    np.testing.assert_array_equal(_bits(got), _bits(O.qgemm_int8(xq, q_kn, sx, s)))
    # unaligned activation stride is rejected
    with pytest.raises(hip.SynapseError):
        lin.forward_pre_quantized_dev(m, dxq.ptr, 1000, dsx.ptr, dy.ptr)


@pytest.mark.parametrize("m,k,n", [(1, 1024, 3072), (4, 3072, 1024), (20, 700, 300)])
def test_qlinear_from_f32_forward(m, k, n):
    # QuantizedLinear::from_f32 + forward (int8_linear.rs:35-117)
    w = O.normal(n * k, 7 + n, 0.02).reshape(n, k)
    x = O.normal(m * k, 9 + m, 1.0).reshape(m, k)
    lin = hip.QLinear.from_f32(hip.FMT_INT8, w)
    got = lin.forward(x)
    q_kn, s = O.quantize_weights_int8(w)
    xq, sx = O.quantize_per_channel_int8(x)
    np.testing.assert_array_equal(_bits(got), _bits(O.qgemm_int8(xq, q_kn, sx, s)))


@pytest.mark.parametrize("m", [1, 5])
def test_int8_split_k_slices_on_every_xcd_twice(m):
    """Three 64-row panels over K = 16384: the slices of a panel run on all
    eight XCDs, so the one-launch K split's int32 atomics, arrival counter
    and read-back cross XCDs; bit-exact on two calls in a row."""
    n, k = 192, 16384
    w = O.normal(n * k, 3, 0.02).reshape(n, k)
    lin = hip.QLinear.from_f32(hip.FMT_INT8, w)
    q_kn, s = O.quantize_weights_int8(w)
    for call in range(2):
        x = O.normal(m * k, 50 + call, 1.0).reshape(m, k)
        xq, sx = O.quantize_per_channel_int8(x)
        np.testing.assert_array_equal(_bits(lin.forward(x)), _bits(O.qgemm_int8(xq, q_kn, sx, s)))


def test_lm_head_shape_bit_exact():
    # Qwen3 tied lm_head: 151936 x 1024
    n, k = 151936, 1024
    rng = np.random.default_rng(1)
    q_nk = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s = rng.uniform(1e-4, 1e-3, n).astype(np.float32)
    lin = hip.QLinear.int8(q_nk, s, hip.LAYOUT_NK)
    x = O.normal(k, 3, 1.0).reshape(1, k)
    xq, sx = O.quantize_per_channel_int8(x)
    dxq = hip.DeviceBuffer.from_array(xq)
    dsx = hip.DeviceBuffer.from_array(sx)
    dy = hip.DeviceBuffer(n * 4)
    lin.forward_pre_quantized_dev(1, dxq.ptr, k, dsx.ptr, dy.ptr)
    hip.check(hip.lib().syn_hip_stream_synchronize(None))
    got = dy.download(n, np.float32)
    want = O.qgemm_int8(xq, np.ascontiguousarray(q_nk.T), sx, s)[0]
    np.testing.assert_array_equal(_bits(got), _bits(want))


def test_device_expf_matches_glibc():
    # the expf used by SiLU / softmax must equal glibc's expf bit for bit
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.uniform(-104, 89, 2_000_000).astype(np.float32),
        rng.standard_normal(1_000_000).astype(np.float32) * 5,
        np.array([0.0, -0.0, 1.0, -1.0, 88.72, 88.73, -103.97, -104.0, -87.0, np.inf, -np.inf,
                  1e-30, -1e-30, 0.5], np.float32)])
    dx = hip.DeviceBuffer.from_array(x)
    dy = hip.DeviceBuffer(x.nbytes)
    hip.check(hip.lib().syn_hip_eval_expf(dx.ptr, dy.ptr, x.size, None))
    hip.check(hip.lib().syn_hip_stream_synchronize(None))
    got = dy.download(x.size, np.float32)
    want = np.array([O.expf(float(v)) for v in x[-14:]], np.float32)
    np.testing.assert_array_equal(_bits(got[-14:]), _bits(want))
    # bulk: vectorised glibc expf through the oracle's silu-free path
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    idx = rng.choice(x.size, 200_000, replace=False)
    ref = np.array([libm.expf(float(v)) for v in x[idx]], np.float32)
    np.testing.assert_array_equal(_bits(got[idx]), _bits(ref))


@pytest.mark.parametrize("m,k,n", [(128, 1024, 3072), (300, 2048, 1000), (17, 4096, 513),
                                   (256, 4096, 1024),
                                   # direct-load tiles 256 x 128 and 128 x 128 (a K of 5 and
                                   # 9 steps: a partial last KC chunk), ragged M and N
                                   (300, 640, 16384), (300, 1152, 11000),
                                   # 128 x 64 tiles with eight waves (fewer than 256 tiles
                                   # of 128 x 128, at least 256 of 128 x 64), ragged
                                   (300, 1152, 6000),
                                   # exactly 256 tiles of 128 x 128: three stages (and
                                   # the two accumulator sets over two whole chunks
                                   # and a tail)
                                   (250, 640, 16384), (250, 1152, 16384),
                                   # chunk counts: K of 1 step (no whole KC chunk), 3, 12
                                   # (three whole chunks, no tail) and 14 (three and a tail
                                   # of two), on each direct-load tile shape
                                   (200, 128, 20000), (40, 384, 700), (300, 1536, 9000),
                                   (300, 1792, 11000),
                                   # K not whole 128-byte steps: the register-staged kernel
                                   (40, 1040, 700), (520, 1040, 9000)])
def test_int8_gemm_mfma_bit_exact(m, k, n):
    # M > 16: v_mfma_i32_32x32x32_i8 tiles with the KC=512 chunked epilogue
    rng = np.random.default_rng(m + k + n)
    q_nk = rng.integers(-128, 128, (n, k), dtype=np.int8)
    s = rng.uniform(1e-4, 1e-2, n).astype(np.float32)
    lin = hip.QLinear.int8(q_nk, s, hip.LAYOUT_NK)
    xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    sx = rng.uniform(1e-3, 0.1, m).astype(np.float32)
    dxq = hip.DeviceBuffer.from_array(xq)
    dsx = hip.DeviceBuffer.from_array(sx)
    dy = hip.DeviceBuffer(m * n * 4)
    lin.forward_pre_quantized_dev(m, dxq.ptr, k, dsx.ptr, dy.ptr)
    hip.check(hip.lib().syn_hip_stream_synchronize(None))
    got = dy.download((m, n), np.float32)
    want = O.qgemm_int8(xq, np.ascontiguousarray(q_nk.T), sx, s)
    np.testing.assert_array_equal(_bits(got), _bits(want))
