"""Speculative decode, oracle side (INT8 decoder and the f32 CausalLM of the
K-quant path, whose forward_one_draft runs the first layers only): forward_prefill into a
non-empty cache (int8.rs:593-635 with cached_attention_prefill,
ops/attention.rs:153-247), KvCache.truncateTo (kvcache.zig:109-113) and
generate_speculative (generation/pipeline.rs:281-395).  The reference has no
test of its own for these; they are pinned by properties the reference code
fixes: an appended prefill rotates from position 0 and attends only among its
own rows (so its logits do not depend on what the cache held), a truncated
row is rewritten by the next step, the first round's drafts are the plain
greedy continuation, and the cache grows by k + 2 rows per full round."""
import numpy as np
import pytest

import oracle as O
from tests.golden import make_golden as G

CFG = dict(G.QWEN3_TINY)


@pytest.fixture(scope="module")
def model():
    o = O.QuantizedCausalLM(CFG)
    o.init_synthetic(G.SEED, G.QWEN3_TINY_STD)
    yield o
    o.close()


def _ids(n, salt=0):
    return O.token_ids(n, G.SEED + 0xFFFF + salt, CFG["vocab"])


def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def test_prefill_append_on_empty_cache_is_prefill(model):
    ids = _ids(7)
    a = model.prefill(ids)
    model.reset()
    b = model.prefill_append(ids)
    np.testing.assert_array_equal(_bits(a), _bits(b))
    assert model.cache_len() == 7


def test_prefill_append_ignores_the_cached_prefix(model):
    """The appended rows rotate from position 0 and attend among themselves:
    their logits equal a fresh prefill of the same ids, whatever came before."""
    fresh = model.prefill(_ids(5, 1))
    for n_prefix in (1, 9, 20):
        model.prefill(_ids(n_prefix, 2))
        got = model.prefill_append(_ids(5, 1))
        np.testing.assert_array_equal(_bits(got), _bits(fresh))
        assert model.cache_len() == n_prefix + 5


def test_appended_rows_feed_later_decode_steps(model):
    """A decode step after an appended prefill attends over every cached row:
    with a different prefix its logits change."""
    model.prefill(_ids(4, 3))
    model.prefill_append(_ids(3, 4))
    a = model.forward_one(5)
    model.prefill(_ids(4, 5))
    model.prefill_append(_ids(3, 4))
    b = model.forward_one(5)
    assert not np.array_equal(a, b)


def test_truncate(model):
    ids = _ids(6, 6)
    model.prefill(ids)
    first = model.forward_one(11)
    second = model.forward_one(12)
    model.truncate(100)  # longer: ignored (kvcache.zig:110)
    assert model.cache_len() == 8
    model.truncate(6)
    assert model.cache_len() == 6
    again = model.forward_one(11)  # rewrites row 6 with the same values
    np.testing.assert_array_equal(_bits(again), _bits(first))
    np.testing.assert_array_equal(_bits(model.forward_one(12)), _bits(second))
    model.truncate(7)
    np.testing.assert_array_equal(_bits(model.forward_one(12)), _bits(second))


@pytest.mark.parametrize("k", [1, 2, 3, 5])
def test_first_round_is_plain_greedy(model, k):
    ids = _ids(6)
    plain, pm = model.generate(ids, 12)
    spec, sm = model.generate_speculative(ids, 12, k)
    assert spec.size == 12
    np.testing.assert_array_equal(spec[:k + 1], plain[:k + 1])
    np.testing.assert_array_equal(_bits(sm[:k + 1]), _bits(pm[:k + 1]))


@pytest.mark.parametrize("max_new", [1, 2, 4])
def test_drafts_only_equals_plain(model, max_new):
    ids = _ids(5, 7)
    plain, _ = model.generate(ids, max_new)
    spec, _ = model.generate_speculative(ids, max_new, 4)
    np.testing.assert_array_equal(spec, plain)


def _rows_after(n_prompt, max_new, k):
    pos, gen = n_prompt, 1
    while gen < max_new:
        acc = min(k, max_new - gen)
        gen += acc
        pos += k + 1
        if acc == k and gen < max_new:
            pos += 1
            gen += 1
    return pos


@pytest.mark.parametrize("max_new,k", [(2, 1), (7, 2), (16, 4), (9, 4), (10, 3)])
def test_cache_rows_per_round(model, max_new, k):
    ids = _ids(6, 8)
    spec, _ = model.generate_speculative(ids, max_new, k)
    assert spec.size == max_new
    assert model.cache_len() == _rows_after(6, max_new, k)


def test_later_rounds_leave_the_plain_path(model):
    """The verify pass re-rotates the drafts from position 0 and the bonus step
    appends the last draft a second time, so the tokens after the first round
    follow another sequence than plain decode (the reference's approximation)."""
    ids = _ids(6)
    plain, _ = model.generate(ids, 24)
    spec, _ = model.generate_speculative(ids, 24, 2)
    assert not np.array_equal(spec, plain)


def test_sampled_zero_temperature_is_greedy(model):
    ids = _ids(6, 9)
    greedy, _ = model.generate_speculative(ids, 10, 3)
    sampled, _ = model.generate_speculative(ids, 10, 3, sampler=dict(temperature=0.0), seed=5)
    np.testing.assert_array_equal(sampled, greedy)


def test_sampled_first_round_matches_plain_sampling(model):
    """Drafts of the first round sample with the history at the round's start
    (the first token only) and draws 1..k of the stream."""
    params = dict(temperature=0.9, top_k=20, top_p=0.9, repetition_penalty=1.2)
    ids = _ids(6, 10)
    k = 3
    spec, _ = model.generate_speculative(ids, 8, k, sampler=params, seed=42)
    u = O.stdrng_f32(42, k + 1)
    logits = model.prefill(ids)
    want = [O.sample_combined(logits, np.zeros(0, np.uint32), u=float(u[0]), **params)]
    last = want[0]
    for i in range(k):
        last = O.sample_combined(model.forward_one(last), np.array(want[:1], np.uint32),
                                 u=float(u[1 + i]), **params)
        want.append(last)
    assert spec[:k + 1].tolist() == want


# ---- the f32 CausalLM (K-quant decoder): a real draft forward ---------------
KCFG = dict(hidden=128, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=32, inter=256, vocab=200,
            max_seq=96, eps=1e-5, rope_theta=5e5)


def _flm(cfg, seed=0x5EED0000):
    """An oracle CausalLM over Q8_0 blocks (layer l's weights depend only on l)."""
    from synapse_amd import hip  # the library's host-side block encoder
    o = O.CausalLM(cfg)
    h, qd = cfg["hidden"], cfg["n_heads"] * cfg["head_dim"]
    kvd, inter = cfg["n_kv_heads"] * cfg["head_dim"], cfg["inter"]
    o.set_embed(O.normal(cfg["vocab"] * h, seed, 0.1).reshape(cfg["vocab"], h))
    shapes = [(qd, h), (kvd, h), (kvd, h), (h, qd), (inter, h), (inter, h), (h, inter)]
    for layer in range(cfg["n_layers"]):
        for p, (n, k) in enumerate(shapes):
            w = O.normal(n * k, seed + 1 + 8 * layer + p, 0.1).reshape(n, k)
            o.set_proj(layer, p, "q8_0", hip.kquant_encode(hip.FMT_Q8_0, w))
    w = O.normal(cfg["vocab"] * h, seed + 1 + 8 * 64, 0.1).reshape(cfg["vocab"], h)
    o.set_lm_head("q8_0", hip.kquant_encode(hip.FMT_Q8_0, w))
    return o


@pytest.fixture(scope="module")
def flm():
    o = _flm(KCFG)
    yield o
    o.close()


def test_draft_with_all_layers_is_forward_one(flm):
    ids = _ids(6, 11)
    flm.prefill(ids)
    a = flm.forward_one(17)
    flm.truncate(6)
    b = flm.forward_one_draft(17, KCFG["n_layers"])
    np.testing.assert_array_equal(_bits(a), _bits(b))


@pytest.mark.parametrize("n", [1, 2])
def test_draft_is_the_shallow_model(flm, n):
    """forward_one_draft with n layers = forward_one of a model built from the
    first n layers alone (same embedding, final norm and lm_head)."""
    small = _flm(dict(KCFG, n_layers=n))
    ids = _ids(5, 12)
    for m in (flm, small):
        m.prefill(ids)
    # the shallow model's prefill fills its n layers as the deep model's first n
    for t in (3, 99, 41):
        np.testing.assert_array_equal(_bits(flm.forward_one_draft(t, n)),
                                      _bits(small.forward_one(t)))
    assert flm.cache_len() == small.cache_len() == 8
    small.close()


def test_draft_pads_the_skipped_layers_with_zero_rows(flm):
    """A 1-layer draft leaves zero K/V rows in layers 1..: the next full step
    then differs from the one after a full step of the same token."""
    ids = _ids(5, 13)
    flm.prefill(ids)
    flm.forward_one_draft(7, 1)
    after_draft = flm.forward_one(9)
    flm.truncate(5)
    flm.forward_one(7)
    after_full = flm.forward_one(9)
    assert not np.array_equal(after_draft, after_full)


@pytest.mark.parametrize("k", [1, 3])
def test_flm_speculative_all_layer_draft_first_round(flm, k):
    ids = _ids(6, 14)
    plain, pm = flm.generate(ids, 10)
    spec, sm = flm.generate_speculative(ids, 10, k, draft_layers=KCFG["n_layers"])
    np.testing.assert_array_equal(spec[:k + 1], plain[:k + 1])
    np.testing.assert_array_equal(_bits(sm[:k + 1]), _bits(pm[:k + 1]))


@pytest.mark.parametrize("max_new,k", [(9, 2), (16, 4)])
def test_flm_speculative_rows_and_default_draft(flm, max_new, k):
    ids = _ids(6, 15)
    a, _ = flm.generate_speculative(ids, max_new, k)  # draft_layers 0: n_layers / 3 = 1
    assert flm.cache_len() == _rows_after(6, max_new, k)
    b, _ = flm.generate_speculative(ids, max_new, k, draft_layers=1)
    np.testing.assert_array_equal(a, b)
