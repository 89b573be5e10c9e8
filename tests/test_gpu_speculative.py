"""Speculative decode on the device INT8 decoder (qlm.hip) against the
oracle's restatement of generate_speculative (generation/pipeline.rs:281-395):
the same tokens (and greedy margins, bit for bit) for greedy and sampled
settings, fused and one-kernel-per-op steps, graph replay and eager launches;
forward_prefill into a non-empty cache and truncate_to against the oracle."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests.golden import make_golden as G

pytestmark = pytest.mark.gpu

TINY = dict(G.QWEN3_TINY)
# hd 32, positions beyond 64 (the attention kernels switch to the reference's
# 32/8-wide f32GemvRow blocks at length 64)
MID = dict(hidden=128, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=32, inter=256,
           vocab=512, max_seq=160)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _pair(cfg, std):
    o = O.QuantizedCausalLM(cfg)
    o.init_synthetic(G.SEED, std)
    g = hip.QuantizedCausalLM(cfg)
    g.init_synthetic(G.SEED, std)
    return o, g


@pytest.fixture(scope="module")
def tiny():
    o, g = _pair(TINY, G.QWEN3_TINY_STD)
    yield o, g
    o.close()
    g.close()


@pytest.fixture(scope="module")
def mid():
    o, g = _pair(MID, 0.15)
    yield o, g
    o.close()
    g.close()


def _ids(cfg, n, salt=0):
    return O.token_ids(n, G.SEED + 0xFFFF + salt, cfg["vocab"])


def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def test_prefill_append_and_truncate(tiny):
    o, g = tiny
    for m in (o, g):
        m.prefill(_ids(TINY, 9, 1))
    a, b = o.prefill_append(_ids(TINY, 5, 2)), g.prefill_append(_ids(TINY, 5, 2))
    np.testing.assert_array_equal(_bits(b), _bits(a))
    assert g.cache_len() == o.cache_len() == 14
    np.testing.assert_array_equal(_bits(g.forward_one(7)), _bits(o.forward_one(7)))
    for m in (o, g):
        m.truncate(40)  # longer: ignored
        m.truncate(11)
    assert g.cache_len() == 11
    np.testing.assert_array_equal(_bits(g.forward_one(3)), _bits(o.forward_one(3)))
    np.testing.assert_array_equal(_bits(g.forward_one(4)), _bits(o.forward_one(4)))


@pytest.mark.parametrize("fused,graph", [(True, True), (False, True), (True, False)])
@pytest.mark.parametrize("max_new,k", [(1, 3), (2, 1), (5, 4), (16, 2), (16, 4), (13, 3)])
def test_greedy_speculative_matches_oracle(tiny, fused, graph, max_new, k):
    o, g = tiny
    ids = _ids(TINY, 8)
    want, wm = o.generate_speculative(ids, max_new, k)
    g.set_options(fused=fused, graph=graph)
    got, gm = g.generate_speculative(ids, max_new, k)
    assert got.tolist() == want.tolist(), (got.tolist(), want.tolist())
    np.testing.assert_array_equal(_bits(gm), _bits(wm))
    assert g.cache_len() == o.cache_len()
    g.set_options()


def test_greedy_speculative_past_64_positions(mid):
    o, g = mid
    ids = _ids(MID, 30, 3)
    want, wm = o.generate_speculative(ids, 60, 4)
    got, gm = g.generate_speculative(ids, 60, 4)
    assert len(set(want.tolist())) > 3
    assert got.tolist() == want.tolist()
    np.testing.assert_array_equal(_bits(gm), _bits(wm))
    assert g.cache_len() == o.cache_len() > 64


def test_sampled_speculative_matches_oracle(tiny):
    o, g = tiny
    params = dict(temperature=0.9, top_k=20, top_p=0.9, repetition_penalty=1.2)
    ids = _ids(TINY, 8)
    try:
        g.set_sampler(hip.sampler_params(**params), 42)
        for fused in (True, False):
            for k in (2, 3):
                want, _ = o.generate_speculative(ids, 16, k, sampler=params, seed=42)
                g.set_options(fused=fused, graph=True)
                got, _ = g.generate_speculative(ids, 16, k)
                assert got.tolist() == want.tolist(), (fused, k, got.tolist(), want.tolist())
        assert len(set(want.tolist())) > 2
    finally:
        g.set_sampler(None)
        g.set_options()


def test_k_zero_is_generate(tiny):
    o, g = tiny
    ids = _ids(TINY, 8)
    got, _ = g.generate_speculative(ids, 10, 0)
    want, _ = o.generate(ids, 10)
    assert got.tolist() == want.tolist()


def test_rows_beyond_max_seq_are_refused(tiny):
    _, g = tiny
    ids = _ids(TINY, 30)
    with pytest.raises(hip.SynapseError):
        g.generate_speculative(ids, 18, 4)  # 30 + 3 rounds x 6 rows > 48


# ---- K-quant decoder: forward_one_draft with the first layers ---------------
from tests.test_gpu_klm import LLAMA_FMTS, build_pair  # noqa: E402

KCFG = dict(hidden=256, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=64, inter=512, vocab=300,
            max_seq=96, eps=1e-5, rope_theta=5e5)


def _cos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


@pytest.fixture(scope="module")
def kpair():
    o, g = build_pair(KCFG, LLAMA_FMTS)
    yield o, g
    o.close()
    g.close()


def test_klm_draft_and_append_track_the_oracle(kpair):
    o, g = kpair
    ids = _ids(KCFG, 7, 5)
    for m in (o, g):
        m.prefill(ids)
    for t, n in ((3, 1), (50, 2), (7, 4)):
        lo, lg = o.forward_one_draft(t, n), g.forward_one_draft(t, n)
        assert _cos(lo, lg) >= 0.9999, (t, n, _cos(lo, lg))
    lo, lg = o.prefill_append(_ids(KCFG, 4, 6)), g.prefill_append(_ids(KCFG, 4, 6))
    assert _cos(lo, lg) >= 0.9999
    for m in (o, g):
        m.truncate(9)
    lo, lg = o.forward_one(11), g.forward_one(11)
    assert _cos(lo, lg) >= 0.9999
    assert o.cache_len() == g.cache_len() == 10


@pytest.mark.parametrize("graph", [True, False])
@pytest.mark.parametrize("k,draft_layers", [(2, 0), (4, 2), (3, 4)])
def test_klm_speculative_matches_oracle(kpair, graph, k, draft_layers):
    o, g = kpair
    ids = _ids(KCFG, 8, 7)
    want, wm = o.generate_speculative(ids, 24, k, draft_layers=draft_layers)
    g.set_options(graph=graph)
    got, _ = g.generate_speculative(ids, 24, k, draft_layers=draft_layers)
    g.set_options()
    # the f32 path sums in another order: tokens agree while the oracle's
    # greedy margin is above float noise
    thin = next((i for i, m in enumerate(wm) if m < 1e-4), len(wm))
    assert thin > 4
    assert got[:thin].tolist() == want[:thin].tolist()
    assert g.cache_len() == o.cache_len()


@pytest.mark.parametrize("n", [1, 17, 64, 100, 150])
def test_long_prefill_and_append_bit_exact(mid, n):
    """Prefill attention over several 64-position chunks and partial 16-row
    blocks, into an empty cache and appended after cached rows."""
    o, g = mid
    ids = _ids(MID, n, 9)
    np.testing.assert_array_equal(_bits(g.prefill(ids)), _bits(o.prefill(ids)))
    if n <= 100:
        extra = _ids(MID, 37, 10)
        np.testing.assert_array_equal(_bits(g.prefill_append(extra)),
                                      _bits(o.prefill_append(extra)))
        np.testing.assert_array_equal(_bits(g.forward_one(5)), _bits(o.forward_one(5)))
