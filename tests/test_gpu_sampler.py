"""Device sampling (sampler.hip) against the oracle's restatement of
generation/sampler.rs: the same token for the same logits, history, settings
and draw, for every stage and their combination, and inside the INT8
decoder's generate loop (graph replay, fused and one-kernel-per-op steps)."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests.golden import make_golden as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def logits_for(seed, n, scale=3.0, ties=True):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    if ties:
        x[rng.integers(0, n, max(4, n // 50))] = x.max()  # ties at the top
        x[rng.integers(0, n, max(4, n // 50))] = x[1]
    return x


CASES = [
    dict(temperature=0.0),                                     # greedy
    dict(temperature=0.8, top_k=1),                            # top-k 1: greedy
    dict(temperature=1.0),                                     # full softmax sample
    dict(temperature=0.7, top_k=40),
    dict(temperature=1.3, top_k=2),
    dict(temperature=0.9, top_k=1000),
    dict(temperature=0.9, top_k=1500),                         # k beyond the block's threads
    dict(temperature=0.8, top_k=50, top_p=0.9),
    dict(temperature=1.0, top_k=300, top_p=0.5),
    dict(temperature=0.6, top_k=40, top_p=0.95, repetition_penalty=1.3),
    dict(temperature=1.0, repetition_penalty=2.0),
]


@pytest.mark.parametrize("n", [5, 1000, 151936])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_sample_matches_oracle(n, case):
    kw = CASES[case]
    x = logits_for(1000 + case, n)
    rng = np.random.default_rng(case)
    hist = rng.integers(0, n, 12).astype(np.uint32)
    hist[3] = hist[0]  # a repeated token is penalised twice
    for u in O.stdrng_f32(7 + case, 6 if n > 5000 else 20):
        want = O.sample_combined(x, hist, u=float(u), **kw)
        got = hip.sample(x, hist, u=float(u), **kw)
        assert got == want, (kw, float(u), got, want)


def test_top_p_without_top_k_small_vocab():
    x = logits_for(5, 3000)
    for u in O.stdrng_f32(3, 20):
        assert hip.sample(x, temperature=1.0, top_p=0.8, u=float(u)) == \
            O.sample_combined(x, temperature=1.0, top_p=0.8, u=float(u))


@pytest.mark.parametrize("n,ties", [(10000, False), (151936, False), (151936, True)])
def test_top_p_without_top_k_large_vocab(n, ties):
    # a nucleus of far more than 4096 candidates (top_p_filter over the whole
    # vocabulary, sampler.rs:279-319): the stable radix sort in global memory
    x = logits_for(6, n, scale=1.0, ties=ties)
    for tp in (0.5, 0.8, 0.95):
        for u in O.stdrng_f32(11, 4):
            want = O.sample_combined(x, temperature=1.0, top_p=tp, u=float(u))
            got = hip.sample(x, temperature=1.0, top_p=tp, u=float(u))
            assert got == want, (n, ties, tp, float(u), got, want)


def test_sampled_generate_matches_oracle():
    params = dict(temperature=0.9, top_k=20, top_p=0.9, repetition_penalty=1.2)
    seed = 42
    o = O.QuantizedCausalLM(G.QWEN3_TINY)
    o.init_synthetic(G.SEED, G.QWEN3_TINY_STD)
    ids = O.token_ids(8, G.SEED + 0xFFFF, G.QWEN3_TINY["vocab"])
    u = O.stdrng_f32(seed, 16)
    logits = o.prefill(ids)
    want = []
    for i in range(16):
        tok = O.sample_combined(logits, np.array(want, np.uint32), u=float(u[i]), **params)
        want.append(tok)
        if i < 15:
            logits = o.forward_one(tok)
    o.close()
    assert len(set(want)) > 2
    g = hip.QuantizedCausalLM(G.QWEN3_TINY)
    try:
        g.init_synthetic(G.SEED, G.QWEN3_TINY_STD)
        g.set_sampler(hip.sampler_params(**params), seed)
        for fused in (True, False):
            g.set_options(fused=fused, graph=True)
            g.reset()
            toks, _ = g.generate(ids, 16)
            assert toks.tolist() == want, (fused, toks.tolist(), want)
        g.set_sampler(None)  # back to greedy
        g.reset()
        toks, _ = g.generate(ids, 16)
        d = np.load(__import__("os").path.join(G.HERE, "qwen3_tiny_w8a8.npz"))
        assert toks.tolist() == d["tokens"].tolist()
    finally:
        g.close()
