"""Ternary linear oracle (quantization/primitives/ternary_linear.rs restated in
oracle.c) against the reference's own tests (ternary_linear.rs:264-409, on
the same pseudo-random inputs) and a loop-by-loop Python form of from_f32 and
forward on small shapes."""
import struct

import numpy as np
import pytest

import oracle as O

U64 = (1 << 64) - 1


def u64_to_f32(v: int) -> np.float32:
    """`v as f32` for a u64: round to 24 significant bits, ties to even."""
    if v == 0:
        return np.float32(0.0)
    e = v.bit_length()
    if e <= 24:
        return np.float32(v)
    shift = e - 24
    q, r = divmod(v, 1 << shift)
    half = 1 << (shift - 1)
    if r > half or (r == half and q & 1):
        q += 1
    return np.float32(q * 2.0 ** shift)


def pseudo_random_vec(n, seed):
    """ternary_linear.rs:269-279: xorshift64, (state as f32 / u64::MAX as f32) * 2 - 1."""
    state, out = seed, []
    umax = u64_to_f32(U64)
    for _ in range(n):
        state ^= (state << 13) & U64
        state ^= state >> 7
        state ^= (state << 17) & U64
        out.append(np.float32(u64_to_f32(state) / umax) * np.float32(2.0) - np.float32(1.0))
    return np.array(out, np.float32)


def py_from_f32(w):
    n, k = w.shape
    bpr = (k + 15) // 16
    out = bytearray()
    for r in range(n):
        row = w[r]
        s = np.float32(0.0)
        for v in row:
            s = np.float32(s + np.float32(abs(v)))
        mean_abs = np.float32(s / np.float32(k))
        thr = np.float32(np.float32(0.5) * mean_abs)
        codes = [1] * (bpr * 16)
        nz_sum, nz = np.float32(0.0), 0
        for i, v in enumerate(row):
            if v > thr:
                codes[i] = 2
            elif v < -thr:
                codes[i] = 0
            if codes[i] != 1:
                nz_sum = np.float32(nz_sum + np.float32(abs(v)))
                nz += 1
        scale = np.float32(nz_sum / np.float32(nz)) if nz else mean_abs
        for b in range(bpr):
            out += struct.pack("<f", scale)
            for byte in range(4):
                v = 0
                for j in range(4):
                    v |= codes[b * 16 + byte * 4 + j] << (2 * j)
                out.append(v)
    return np.frombuffer(bytes(out), np.uint8)


def py_forward(blocks, n, k, x):
    bpr = (k + 15) // 16
    blk = blocks.reshape(n, bpr, 8)
    y = np.zeros((x.shape[0], n), np.float32)
    for i in range(x.shape[0]):
        for j in range(n):
            acc = np.float32(0.0)
            for b in range(bpr):
                scale = np.frombuffer(blk[j, b, :4].tobytes(), np.float32)[0]
                bacc = np.float32(0.0)
                for wi in range(16):
                    col = b * 16 + wi
                    if col >= k:
                        continue
                    code = (int(blk[j, b, 4 + wi // 4]) >> (2 * (wi % 4))) & 3
                    if code == 2:
                        bacc = np.float32(bacc + x[i, col])
                    elif code == 0:
                        bacc = np.float32(bacc - x[i, col])
                acc = np.float32(acc + np.float32(bacc * scale))
            y[i, j] = acc
    return y


def dequant(blocks, n, k):
    bpr = (k + 15) // 16
    blk = blocks.reshape(n, bpr, 8)
    out = np.zeros((n, k), np.float32)
    for r in range(n):
        for b in range(bpr):
            scale = np.frombuffer(blk[r, b, :4].tobytes(), np.float32)[0]
            for wi in range(16):
                col = b * 16 + wi
                if col < k:
                    code = (int(blk[r, b, 4 + wi // 4]) >> (2 * (wi % 4))) & 3
                    out[r, col] = {0: -1.0, 2: 1.0}.get(code, 0.0) * scale
    return out


# ---- the reference's own tests ----------------------------------------------
def test_forward_small_reference_inputs():
    m, n, k = 4, 8, 32
    x = pseudo_random_vec(m * k, 42).reshape(m, k)
    w = pseudo_random_vec(n * k, 123).reshape(n, k)
    blocks = O.ternary_from_f32(w)
    y = O.ternary_forward(blocks, n, k, x)
    assert y.shape == (m, n) and np.isfinite(y).all()
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 0.8, rel


def test_dequantize_values_reference_inputs():
    n, k = 4, 32
    w = pseudo_random_vec(n * k, 999).reshape(n, k)
    blocks = O.ternary_from_f32(w)
    dq = dequant(blocks, n, k)
    scales = np.frombuffer(blocks.reshape(-1, 8)[:, :4].tobytes(), np.float32).reshape(n, -1)
    for r in range(n):
        s = scales[r, 0]
        assert set(np.unique(np.abs(dq[r])).tolist()) <= {0.0, float(s)}


def test_memory_compression():
    n, k = 64, 128
    blocks = O.ternary_from_f32(pseudo_random_vec(n * k, 42).reshape(n, k))
    assert blocks.size / (n * k * 4) < 0.25


def test_pseudo_random_vec_is_uniform_in_range():
    v = pseudo_random_vec(1000, 42)
    assert (v >= -1).all() and (v <= 1).all() and abs(float(v.mean())) < 0.1


# ---- loop-by-loop restatement -----------------------------------------------
@pytest.mark.parametrize("n,k,m", [(3, 16, 1), (5, 37, 2), (4, 64, 3), (2, 1, 1)])
def test_against_python_loops(n, k, m):
    rng = np.random.default_rng(n * 100 + k)
    w = rng.standard_normal((n, k)).astype(np.float32)
    w[0, : min(k, 5)] = 0.0
    blocks = O.ternary_from_f32(w)
    np.testing.assert_array_equal(blocks, py_from_f32(w))
    x = rng.standard_normal((m, k)).astype(np.float32)
    np.testing.assert_array_equal(O.ternary_forward(blocks, n, k, x).view(np.uint32),
                                  py_forward(blocks, n, k, x).view(np.uint32))


def test_all_zero_row_uses_mean_abs():
    w = np.zeros((1, 32), np.float32)
    blocks = O.ternary_from_f32(w)
    assert np.frombuffer(blocks[:4].tobytes(), np.float32)[0] == 0.0
    assert (blocks.reshape(-1, 8)[:, 4:] == 0x55).all()  # every code 0b01
