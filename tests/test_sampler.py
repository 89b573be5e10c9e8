"""Sampling oracle (generation/sampler.rs restated in oracle.c) against the
reference's own sampler tests (sampler.rs:332-507), independent numpy forms
of each stage, and the ChaCha block test vector of RFC 8439 for the random
stream (rand 0.8.5 StdRng = rand_chacha 0.3.1 ChaCha12, seeded by rand_core
0.6.4 seed_from_u64; those crates are not vendored in the reference, so the
stream beyond the block function is parity unpinned)."""
import numpy as np
import pytest

import oracle as O

F32_EPS = np.float32(1.1920929e-07)


# ---- the reference's own tests (sampler.rs:332-507) -------------------------
def test_greedy_kat():
    assert O.argmax(np.array([0.1, 0.5, 0.3, 0.9, 0.2], np.float32)) == 3
    assert O.argmax(np.array([1.0, 3.0, 2.0], np.float32)) == 1
    assert O.argmax(np.array([5.0, 1.0, 2.0], np.float32)) == 0
    assert O.argmax(np.array([1.0, 2.0, 5.0], np.float32)) == 2


@pytest.mark.parametrize("kw", [dict(temperature=0.0), dict(top_k=1), dict(top_p=0.0)])
def test_degenerate_settings_equal_greedy(kw):
    base = np.array([1.0, 3.0, 2.0, 5.0, 0.5], np.float32)
    params = dict(temperature=1.0, top_k=0, top_p=1.0)
    params.update(kw)
    for u in O.stdrng_f32(42, 50):
        if "top_p" in kw:  # TopPSampler with p = 0 returns argmax before any stage
            assert O.argmax(base) == 3
            continue
        assert O.sample_combined(base, u=float(u), **params) == O.argmax(base)


def test_temperature_1_has_entropy():
    counts = np.zeros(5, int)
    for u in O.stdrng_f32(42, 1000):
        counts[O.sample_combined(np.ones(5, np.float32), temperature=1.0, u=float(u))] += 1
    assert (counts > 50).all(), counts


def test_repetition_penalty_kats():
    x = np.array([2.0, 3.0, 1.0, 4.0, 0.5], np.float32)
    y = O.repetition_penalty(x, [1, 3], 2.0)
    assert abs(y[1] - x[1] / 2) < F32_EPS and abs(y[3] - x[3] / 2) < F32_EPS
    assert y[0] == x[0] and y[2] == x[2] and y[4] == x[4]
    y = O.repetition_penalty(np.array([-2.0, 3.0], np.float32), [0], 2.0)
    assert abs(y[0] + 4.0) < F32_EPS
    # every occurrence applies again; penalty 1 is a no-op
    y = O.repetition_penalty(np.array([8.0, -1.0], np.float32), [0, 0, 1, 1, 1], 2.0)
    assert y[0] == 2.0 and y[1] == -8.0
    assert (O.repetition_penalty(x, [0, 1], 1.0) == x).all()


def test_softmax_valid_distribution():
    p = O.softmax(np.array([1, 2, 3, 4, 5], np.float32))
    assert (p >= 0).all() and abs(float(p.sum()) - 1.0) < 1e-5


def test_combined_applies_all_stages():
    for u in O.stdrng_f32(42, 20):
        t = O.sample_combined(np.array([1.0, 5.0, 3.0, 2.0, 0.5], np.float32), [1], 1.0, 3, 0.9,
                              1.5, float(u))
        assert t < 5


def test_top_k_filter_kat():
    y = O.top_k_filter(np.array([1.0, 5.0, 3.0, 2.0, 4.0], np.float32), 3)
    assert np.isfinite(y[[1, 4, 2]]).all() and (y[[0, 3]] == -np.inf).all()


# ---- independent numpy forms -------------------------------------------------
def np_softmax(x):
    x = x.astype(np.float32)
    m = np.float32(-np.inf)
    for v in x:
        m = np.fmax(m, v)
    e = np.exp((x - m).astype(np.float32)).astype(np.float32)
    s = np.cumsum(e, dtype=np.float32)[-1]  # a sequential float32 scan
    return (e / s).astype(np.float32) if s > 0 else e


@pytest.mark.parametrize("seed", range(6))
def test_stages_against_numpy(seed):
    rng = np.random.default_rng(seed)
    n = 300
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    x[rng.integers(0, n, 20)] = x[0]  # ties
    k = int(rng.integers(2, 50))
    thr = np.sort(x)[::-1][k - 1]
    np.testing.assert_array_equal(O.top_k_filter(x, k), np.where(x < thr, -np.inf, x).astype(np.float32))
    e = O.softmax(x)
    ref = np_softmax(x)
    assert np.abs(e - ref).max() <= 2e-7 * np.abs(ref).max()
    p = float(rng.uniform(0.1, 0.95))
    order = np.lexsort((np.arange(n), -e))  # probability descending, index ascending
    cum = np.cumsum(e[order], dtype=np.float32)
    cut = int(np.argmax(cum >= np.float32(p))) + 1 if (cum >= np.float32(p)).any() else n
    keep = np.zeros(n, bool)
    keep[order[:cut]] = True
    np.testing.assert_array_equal(O.top_p_filter(x, p), np.where(keep, x, -np.inf).astype(np.float32))


@pytest.mark.parametrize("seed", range(6))
def test_categorical_draw_interval(seed):
    """The drawn token is the first whose cumulative probability exceeds u."""
    rng = np.random.default_rng(100 + seed)
    x = (rng.standard_normal(200) * 2).astype(np.float32)
    for u in O.stdrng_f32(seed, 25):
        t = O.sample_combined(x, temperature=0.7, u=float(u))
        probs = O.softmax((x * np.float32(1.0 / np.float32(0.7))).astype(np.float32))
        cum = np.cumsum(probs, dtype=np.float32)
        assert u < cum[t] and (t == 0 or not u < cum[t - 1])


# ---- the random stream ------------------------------------------------------
def test_chacha20_block_rfc8439():
    """RFC 8439 2.3.2: key 00..1f, nonce 00000009 0000004a 00000000, counter 1,
    in the 64-bit counter / 64-bit stream layout of rand_chacha."""
    key = np.array([int.from_bytes(bytes(range(4 * i, 4 * i + 4)), "little") for i in range(8)],
                   np.uint32)
    out = O.chacha_block(key, 1 | (0x09000000 << 32), 0x4A000000, 20)
    want = [0xE4E7F110, 0x15593BD1, 0x1FDD0F50, 0xC47120A3, 0xC7F4D1C7, 0x0368C033, 0x9AAA2204,
            0x4E6CD4C3, 0x466482D2, 0x09AA9F07, 0x05D7C214, 0xA2028BD9, 0xD19C12B5, 0xB94E16DE,
            0xE883D0CB, 0x4E3C50A2]
    assert out.tolist() == want


def test_pcg32_demo_stream():
    """The seed expansion's PCG32 pieces (the LCG multiplier and the XSH-RR
    output) against the PCG reference implementation's demo stream
    (pcg32_srandom_r(&rng, 42, 54), then pcg32_random_r: the output of the
    state before each step)."""
    inc = (54 << 1) | 1
    state = O.pcg32_step(0, inc)
    state = O.pcg32_step((state + 42) % 2**64, inc)
    got = []
    for _ in range(6):
        got.append(O.pcg32_xsh_rr(state))
        state = O.pcg32_step(state, inc)
    assert got == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_stdrng_stream_shape():
    u = O.stdrng_f32(42, 300)
    assert ((u >= 0) & (u < 1)).all()
    assert (np.round(u * 2**24) == u * 2**24).all()      # 24-bit draws
    assert len(set(u.tolist())) > 290
    np.testing.assert_array_equal(O.stdrng_f32(42, 100), u[:100])  # a prefix of the stream
    assert not np.array_equal(O.stdrng_f32(43, 10), u[:10])


def test_library_host_stream_matches_oracle():
    """The library's host StdRng (which feeds the device sampler) gives the
    oracle's draws."""
    from synapse_amd import hip
    for seed in (0, 42, 2**63 + 5):
        np.testing.assert_array_equal(hip.stdrng_f32(seed, 200), O.stdrng_f32(seed, 200))
