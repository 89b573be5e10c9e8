"""Pin the CPU oracle before trusting it (CPU only).

Each test checks the oracle against something that does not come from the
oracle's own formula: the reference's known-answer tests, IEEE conversions
done by numpy, brute-force integer arithmetic, closed forms, or hand-built
blocks whose expected values were worked out by hand.
"""
import numpy as np
import pytest

import oracle as O


# ---------------------------------------------------------------- A1 quantizer
def test_quantize_clamp_kat():
    # zig/tests/test_quantize.zig:225-246
    x = np.array([[100.0, -100.0, 50.0, -50.0, 0.0, 127.0, -127.0, 1.0]], np.float32)
    q, s = O.quantize_per_channel_int8(x)
    assert s[0] == np.float32(1.0)
    assert q.tolist() == [[100, -100, 50, -50, 0, 127, -127, 1]]


def test_quantize_zero_row_kat():
    # zig/tests/test_quantize.zig:143-170: zero channel -> scale 1.0, all q = 0
    x = np.zeros((2, 16), np.float32)
    x[0] = O.normal(16, 42, 3.0)
    q, s = O.quantize_per_channel_int8(x)
    assert s[0] > 0 and s[1] == 1.0
    assert not q[1].any()


def test_quantize_symmetry():
    # zig/tests/test_quantize.zig:110-137: q(-x) = -q(x)
    x = O.normal(32, 99, 5.0).reshape(1, 32)
    q1, s1 = O.quantize_per_channel_int8(x)
    q2, s2 = O.quantize_per_channel_int8(-x)
    assert s1[0] == s2[0]
    assert (q2 == -q1).all()


def test_quantize_round_half_away_and_bound():
    # max|x| = 127 makes inv_scale exactly 1, so q = round-half-away(x)
    x = np.array([[127.0, 0.5, -0.5, 1.5, -1.5, 2.5, 126.5, -126.5]], np.float32)
    q, s = O.quantize_per_channel_int8(x)
    assert q.tolist() == [[127, 1, -1, 2, -2, 3, 127, -127]]
    # error bound on random data: |x - q*s| <= s/2 (+1 ulp)
    x = O.normal(4096, 7, 2.0).reshape(4, 1024)
    q, s = O.quantize_per_channel_int8(x)
    err = np.abs(x - q.astype(np.float32) * s[:, None])
    assert (err <= s[:, None] * 0.5000001 + 1e-7).all()
    assert np.abs(q).max() == 127


def test_quantize_zero_dims_invalid():
    with pytest.raises(ValueError):
        O.quantize_per_channel_int8(np.zeros((0, 4), np.float32))


# ---------------------------------------------------------------- A2 weight quantizer
def test_weight_quantizer_layout_and_scales():
    w = O.normal(24 * 40, 3, 0.02).reshape(24, 40)
    w[5] = 0.0
    q_kn, s = O.quantize_weights_int8(w)
    assert q_kn.shape == (40, 24)
    assert s[5] == 1.0 and not q_kn[:, 5].any()
    mx = np.abs(w).max(axis=1)
    np.testing.assert_array_equal(s[mx > 0], (mx[mx > 0] / np.float32(127)).astype(np.float32))
    recon = q_kn.T.astype(np.float32) * s[:, None]
    assert (np.abs(recon - w) <= s[:, None] * 0.5000001 + 1e-9).all()


# ---------------------------------------------------------------- A3/A4 INT8 GEMM
def _brute(a, b_kn, sa, sb, chunked):
    acc = a.astype(np.int64) @ b_kn.astype(np.int64)
    if not chunked:
        return (acc.astype(np.float32) * sa[:, None]) * sb[None, :]
    k = a.shape[1]
    c = np.zeros((a.shape[0], b_kn.shape[1]), np.float32)
    for p in range(0, k, 512):
        part = a[:, p:p + 512].astype(np.int64) @ b_kn[p:p + 512].astype(np.int64)
        t = (part.astype(np.float32) * sa[:, None]) * sb[None, :]
        c = (c + t).astype(np.float32)
    return c


def test_qgemm_kats():
    # crates/synapse-core/src/lib.rs:1541-1567
    c = O.qgemm_int8(np.array([[1, 2, 3], [4, 5, 6]], np.int8),
                     np.array([[7, 8], [9, 10], [11, 12]], np.int8),
                     np.ones(2, np.float32), np.ones(2, np.float32))
    assert c[0, 0] == 58 and c[0, 1] == 64
    c = O.qgemm_int8(np.array([[127, 0], [0, 127]], np.int8), np.array([[127, 0], [0, 127]], np.int8),
                     np.array([2.0, 3.0], np.float32), np.array([0.5, 1.0], np.float32))
    assert c[0, 0] == 16129.0


@pytest.mark.parametrize("m,k,n", [(1, 1024, 1024), (1, 1024, 3072), (3, 37, 77), (16, 1024, 130),
                                   (17, 33, 25), (33, 600, 40), (20, 1100, 9), (1, 1, 1)])
def test_qgemm_vs_bruteforce(m, k, n):
    rng = np.random.default_rng(m * 7919 + k * 31 + n)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    sa = rng.uniform(0.001, 0.1, m).astype(np.float32)
    sb = rng.uniform(0.001, 0.1, n).astype(np.float32)
    got = O.qgemm_int8(a, b, sa, sb)
    want = _brute(a, b, sa, sb, chunked=m > 16)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    if m <= 16:  # naive kernel (qmatmul.zig:106-128) agrees with the GEMV path
        np.testing.assert_array_equal(got, O.naive_int8_gemm(a, b, sa, sb))


# ---------------------------------------------------------------- f16
def test_f16_zig_exhaustive_ieee():
    bits = np.arange(65536, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([O.lib().orc_f16_to_f32_zig(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()


def test_f16_rust_converter_halves_subnormals():
    # converter.rs:12-40 starts its shift count at 1: subnormals come out halved
    bits = np.arange(65536, dtype=np.uint32)
    ieee = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([O.lib().orc_f16_to_f32_rs(int(b)) for b in bits], np.float32)
    exp = (bits >> 10) & 0x1F
    sub = (exp == 0) & ((bits & 0x3FF) != 0)
    normal = ~sub & ~np.isnan(ieee)
    np.testing.assert_array_equal(got[normal].view(np.uint32), ieee[normal].view(np.uint32))
    np.testing.assert_array_equal(got[sub], ieee[sub] * np.float32(0.5))


def test_f32_to_f16_truncates():
    x = np.concatenate([O.normal(20000, 5, 3.0), O.normal(2000, 6, 1e-4),
                        np.array([65504.0, 65520.0, 1e6, 6.1e-5, 5.9e-5, 1e-8, 0.0], np.float32)])
    h = np.array([O.lib().orc_f32_to_f16_trunc(float(v)) for v in x], np.uint16)
    back = h.view(np.float16).astype(np.float32)
    ax = np.abs(x)
    normal = (ax >= 2.0 ** -14) & (ax < 65536.0)
    # truncation: |f16| <= |x| < next f16 up, same sign
    nxt = (h[normal] + 1).view(np.float16).astype(np.float32)
    assert (np.abs(back[normal]) <= ax[normal]).all()
    assert (ax[normal] < np.abs(nxt)).all()
    assert (np.sign(back[normal]) == np.sign(x[normal])).all()
    assert (back[ax < 2.0 ** -14] == 0).all()      # subnormal range flushes to 0
    assert np.isinf(back[ax >= 65536.0]).all()     # overflow -> inf


# ---------------------------------------------------------------- Q4_0 / GGUF KATs
def test_gguf_q8_0_kat():
    # weight_loading/gguf.rs:700-721: scale 0x3800 (0.5), q = 1..32 -> 0.5*q
    blk = np.zeros(34, np.uint8)
    blk[0], blk[1] = 0x00, 0x38
    blk[2:] = np.arange(1, 33, dtype=np.int8).view(np.uint8)
    np.testing.assert_array_equal(O.dequant("q8_0", blk, 32), 0.5 * np.arange(1, 33, dtype=np.float32))


def test_gguf_q4_0_kat():
    # weight_loading/gguf.rs:789-820: delta 0x3C00, bytes 0x10 -> (-8, -7) pairs
    blk = np.full(18, 0x10, np.uint8)
    blk[0], blk[1] = 0x00, 0x3C
    out = O.dequant("q4_0", blk, 32)
    assert (out[0::2] == -8).all() and (out[1::2] == -7).all()


def test_q4_pack_format_and_roundtrip():
    w = O.normal(8 * 96, 11, 0.02).reshape(8, 96)
    w[3, 32:64] = 0.0  # all-zero block -> scale 0
    packed = O.q4_pack(w)
    assert packed.size == 8 * 3 * 18
    deq = O.dequant("q4_0", packed, 8 * 96).reshape(8, 96)
    blocks = np.abs(w.reshape(8, 3, 32)).max(axis=2)
    scale = np.repeat(blocks / 7.0, 32, axis=1)
    assert (np.abs(deq - w) <= scale * 0.51 + 1e-6).all()
    assert (deq[3, 32:64] == 0).all()
    # low nibble holds the even element: a block whose element 0 is its max
    v = np.zeros((1, 32), np.float32)
    v[0, 0] = 7.0
    v[0, 1] = -7.0
    p = O.q4_pack(v)
    assert p[2] == ((7 + 8) | ((-7 + 8) << 4))


def test_q4_gemv_vs_f64():
    for n, k in [(16, 64), (67, 2048), (5, 32), (3, 96)]:
        w = O.normal(n * k, n + k, 0.02).reshape(n, k)
        a = O.normal(k, 2 * k + 1, 1.0)
        packed = O.q4_pack(w)
        deq = O.dequant("q4_0", packed, n * k).reshape(n, k).astype(np.float64)
        want = deq @ a.astype(np.float64)
        got = O.q4_0_gemv(a, packed, n)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-6
    with pytest.raises(ValueError):
        O.q4_0_gemv(np.zeros(40, np.float32), np.zeros(100, np.uint8), 2)  # k % 32 != 0


def test_q4_k_handmade_superblock():
    # weight_loading/gguf.rs:375-431.  d = 1.0, dmin = 0.5, scale bytes chosen so
    # every 6-bit/8-bit field is distinct; sc/mn worked out by hand from the
    # bit layout of lines 405-410.
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x38]
    blk[4:16] = [0x41, 0x82, 0xC3, 0x04, 0x25, 0x16, 0x37, 0x58, 0x9A, 0x6B, 0x2C, 0xFD]
    sc = [1, 2, 3, 4, 21, 38, 55, 8]
    mn = [162, 177, 195, 213, 73, 134, 194, 15]
    for s in range(8):
        for i in range(16):
            blk[16 + 16 * s + i] = (i & 0xF) | ((15 - i) << 4)
    out = O.dequant("q4_k", blk, 256)
    for s in range(8):
        for i in range(16):
            assert out[32 * s + 2 * i] == i * sc[s] - 0.5 * mn[s]
            assert out[32 * s + 2 * i + 1] == (15 - i) * sc[s] - 0.5 * mn[s]


def _pack_q6_k(qv, sc, d_bits):
    """Bytes for one Q6_K superblock from 6-bit values (reference layout,
    gguf.rs:459-482: ql nibble idx%2, qh 2-bit field idx%4)."""
    blk = np.zeros(210, np.uint8)
    for idx in range(256):
        lo, hi = qv[idx] & 0xF, qv[idx] >> 4
        blk[idx // 2] |= lo << (4 * (idx % 2))
        blk[128 + idx // 4] |= hi << (2 * (idx % 4))
    blk[192:208] = np.array(sc, np.int8).view(np.uint8)
    blk[208], blk[209] = d_bits & 0xFF, d_bits >> 8
    return blk


def test_q6_k_handmade_superblock():
    # literal bytes: ql[0] = 0x21 -> idx0 lo 1, idx1 lo 2; qh[0] = 0xE4 -> hi 0,1,2,3
    blk = np.zeros(210, np.uint8)
    blk[0] = 0x21
    blk[1] = 0x43
    blk[128] = 0xE4
    blk[192] = 3                      # sc[0] = 3
    blk[208], blk[209] = 0x00, 0x38   # d = 0.5
    out = O.dequant("q6_k", blk, 256)
    # q = lo | hi<<4 : 1, 2|16, 3|32, 4|48 ; value = (q-32) * 3 * 0.5
    np.testing.assert_array_equal(out[:4], np.array([1 - 32, 18 - 32, 35 - 32, 52 - 32], np.float32) * 1.5)
    assert (out[4:16] == -32 * 1.5).all()
    # every index through the reference layout
    qv = [(i * 5 + 3) % 64 for i in range(256)]
    sc = [s - 8 for s in range(16)]
    out = O.dequant("q6_k", _pack_q6_k(qv, sc, 0x3800), 256)
    want = np.array([(qv[i] - 32) * (sc[i // 16] * 0.5) for i in range(256)], np.float32)
    np.testing.assert_array_equal(out, want)


# ---------------------------------------------------------------- A12 f32 GEMM
@pytest.mark.parametrize("m,k,n", [(1, 64, 77), (16, 128, 40), (17, 33, 25), (40, 600, 19), (1, 5, 3)])
def test_sgemm_vs_f64(m, k, n):
    a = O.normal(m * k, m + 3 * k, 1.0).reshape(m, k)
    w = O.normal(n * k, n + 5 * k, 0.1).reshape(n, k)
    got = O.matmul_t(a, w)
    want = a.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - want).max() <= 1e-5 * (np.abs(a).max() * np.abs(w).max() * k)


def test_sgemm_identity_kat():
    # ops/matmul.rs:126-180 style: x @ I^T == x exactly
    x = O.normal(4 * 8, 1, 1.0).reshape(4, 8)
    np.testing.assert_array_equal(O.matmul_t(x, np.eye(8, dtype=np.float32)), x)


# ---------------------------------------------------------------- A14 ops
def test_rmsnorm_unit_rms():
    # ops/norm.rs:103-126: weight 1 -> output RMS 1
    x = O.normal(3 * 1024, 17, 4.0).reshape(3, 1024)
    out = O.rmsnorm(x, np.ones(1024, np.float32), 1e-6)
    rms = np.sqrt((out.astype(np.float64) ** 2).mean(axis=1))
    np.testing.assert_allclose(rms, 1.0, rtol=1e-5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=1e-7)


def test_rope_identity_and_rotation():
    # ops/rope.rs:72-139: position 0 is the identity; rotation keeps pair norms
    cos_t, sin_t = O.rope_tables(8, 16, 10000.0)
    assert (cos_t[0] == 1).all() and (sin_t[0] == 0).all()
    np.testing.assert_allclose(cos_t[3], np.cos(3 / 10000.0 ** (np.arange(8) * 2 / 16)), rtol=1e-6)
    qk = O.normal(2 * 16, 9, 1.0)
    before = qk.copy()
    O.lib().orc_rope_apply(O._p(qk), O._p(cos_t), O._p(sin_t), 1, 2, 16, 5)
    for h in range(2):
        b = before[h * 16:(h + 1) * 16]
        a = qk[h * 16:(h + 1) * 16]
        np.testing.assert_allclose(a[:8] ** 2 + a[8:] ** 2, b[:8] ** 2 + b[8:] ** 2, rtol=1e-5)


def test_argmax_last_max_wins():
    # generation/sampler.rs:217-224: Iterator::max_by returns the last maximum
    assert O.argmax(np.array([1.0, 3.0, 2.0, 3.0, 0.0], np.float32)) == 3
    assert O.argmax(np.array([5.0], np.float32)) == 0


def test_silu_and_expf():
    for x in [0.0, 1.0, -3.5, 20.0, -80.0]:
        assert abs(O.silu(x) - x / (1 + np.exp(-x))) <= 1e-6 * max(1.0, abs(x))
    assert O.expf(0.0) == 1.0 and O.expf(float("-inf")) == 0.0


def test_fused_attention_causal():
    t, d = 40, 16
    q = O.normal(t * d, 1, 1.0).reshape(t, d)
    k = O.normal(t * d, 2, 1.0).reshape(t, d)
    v = O.normal(t * d, 3, 1.0).reshape(t, d)
    got = O.fused_attention(q, k, v)
    np.testing.assert_array_equal(got[0], v[0] * np.float32(1.0))  # row 0 attends to itself
    s = (q.astype(np.float64) @ k.astype(np.float64).T) / np.sqrt(d)
    s[np.triu_indices(t, 1)] = -np.inf
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(got, p @ v.astype(np.float64), rtol=1e-5, atol=1e-5)


def test_attention_decode_paths_agree_with_f64():
    nh, nkv, hd = 4, 2, 16
    for L in (10, 70):  # scalar path and gather+matmul path
        q = O.normal(nh * hd, L, 1.0)
        kc = O.normal(L * nkv * hd, L + 1, 1.0)
        vc = O.normal(L * nkv * hd, L + 2, 1.0)
        got = O.attention_decode(q, kc, vc, L, nh, nkv, hd)
        for h in range(nh):
            kv = h // (nh // nkv)
            K = kc.reshape(L, nkv, hd)[:, kv].astype(np.float64)
            V = vc.reshape(L, nkv, hd)[:, kv].astype(np.float64)
            s = K @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            np.testing.assert_allclose(got[h * hd:(h + 1) * hd], p @ V, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- harness input spec
def test_normal_stream_is_chunk_invariant():
    a = O.normal(10, 0x5EED0000, 1.0)
    b = O.normal(11, 0x5EED0000, 1.0)
    np.testing.assert_array_equal(a, b[:10])
    big = O.normal(1_000_001, 77, 1.0)
    assert abs(big.mean()) < 5e-3 and abs(big.std() - 1.0) < 5e-3


def test_model_prefill_consistency():
    # int8.rs:913-968: prefill logits of the last token == decode of the same
    # prefix (prefill(p[:n-1]) then forward_one(p[n-1])) within 1e-5
    cfg = dict(hidden=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, inter=128,
               vocab=256, max_seq=64)
    m = O.QuantizedCausalLM(cfg)
    m.init_synthetic()
    ids = O.token_ids(9, 5, 256)
    full = m.prefill(ids)
    m.reset()
    m.prefill(ids[:-1])
    one = m.forward_one(ids[-1])
    assert np.abs(full - one).max() <= 1e-5 * max(1.0, np.abs(full).max()) + 1e-3
    toks, margins = m.generate(ids, 8)
    assert toks.shape == (8,) and (margins >= 0).all()


# ---------------------------------------------------------------- Mamba pieces
def test_selective_scan_reference_values():
    # tests/integration/reference_correctness.rs:43-87 (d_state = 2: scalar tail path)
    a_log = np.full(4, -1.0, np.float32)
    d = np.zeros(2, np.float32)
    state = np.zeros(4, np.float32)
    ys = []
    for x, b, c in (([1.0, 2.0], [1.0, 0.5], [1.0, 1.0]), ([0.5, 1.0], [0.5, 1.0], [1.0, 0.5])):
        x = np.array(x, np.float32)
        y = np.zeros(2, np.float32)
        O.lib().orc_selective_scan_step(O._p(x), O._p(np.full(2, 0.5, np.float32)), O._p(a_log),
                                        O._p(np.array(b, np.float32)), O._p(np.array(c, np.float32)),
                                        O._p(d), O._p(state), O._p(y), 2, 2)
        ys += y.tolist()
    assert abs(ys[0] - 0.75) < 1e-5 and abs(ys[1] - 1.5) < 1e-5
    assert abs(ys[2] - 0.76996) < 1e-3 and abs(ys[3] - 1.53993) < 1e-3


def test_selective_scan_vector_path_vs_f64():
    di, ds = 8, 16
    x = O.normal(di, 1, 1.0)
    dt = np.abs(O.normal(di, 2, 0.1)) + 0.01
    al = O.normal(di * ds, 3, 0.5)
    b, c, dd = O.normal(ds, 4, 1.0), O.normal(ds, 5, 1.0), O.normal(di, 6, 1.0)
    st0 = O.normal(di * ds, 7, 1.0)
    st = st0.copy()
    y = np.zeros(di, np.float32)
    O.lib().orc_selective_scan_step(O._p(x), O._p(dt.astype(np.float32)), O._p(al), O._p(b), O._p(c),
                                    O._p(dd), O._p(st), O._p(y), di, ds)
    h = (np.exp(-dt.astype(np.float64)[:, None] * np.exp(al.astype(np.float64).reshape(di, ds)))
         * st0.reshape(di, ds) + (dt[:, None] * x[:, None]) * b[None, :])
    np.testing.assert_allclose(st.reshape(di, ds), h, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(y, h @ c + dd * x, rtol=1e-5, atol=1e-5)


def test_softplus_and_seq_rmsnorm():
    # ops/activation.rs:88-90; pure_rust_ops.rs:96-112
    assert O.lib().orc_softplus(25.0) == 25.0
    assert abs(O.lib().orc_softplus(0.0) - np.log(2.0)) < 1e-7
    x = O.normal(1024, 8, 2.0)
    out = np.empty_like(x)
    O.lib().orc_rmsnorm_seq(O._p(x), O._p(np.ones(1024, np.float32)), 1e-5, 1024, O._p(out))
    np.testing.assert_allclose(np.sqrt((out.astype(np.float64) ** 2).mean()), 1.0, rtol=1e-5)


def test_mamba_prefill_equals_token_loop():
    cfg = dict(d_model=64, d_inner=128, d_state=16, d_conv=4, dt_rank=8, n_layers=2, vocab=256)
    m = O.QuantizedMamba(cfg)
    m.init_synthetic()
    ids = O.token_ids(6, 3, 256)
    full = m.prefill(ids)
    m2 = O.QuantizedMamba(cfg)
    m2.init_synthetic()
    m2.prefill(ids[:3])
    for t in ids[3:5]:
        m2.decode_one(int(t))
    np.testing.assert_array_equal(m2.decode_one(int(ids[5])), full)
