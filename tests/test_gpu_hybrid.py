"""Hybrid LFM2.5 decoder (Q4 decode path) on the GPU against the oracle
(orc_hlm: models/ssm/hybrid layer.rs / model.rs restated in C).

The Q4 GEMVs are held to the float tolerance (their sums run in another
order than q4_0GemvRow's), everything else follows the reference's float
order, so the decoder's logits are compared by tolerance: per step
max|dev - ref| / max|ref| <= 2e-4 and cosine >= 0.99999; greedy tokens must
agree while the reference's top1 - top2 margin exceeds 1e-3.
"""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip

pytestmark = pytest.mark.gpu

TOL, COS = 2e-4, 0.99999

TINY = dict(hidden=64, n_layers=4, vocab=128, n_heads=4, n_kv_heads=2, head_dim=16, inner=64,
            conv_kernel=4, inter=128, max_seq=64, eps=1e-6, rope_theta=1e4,
            layer_kinds=[0, 1, 0, 1])


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _cmp(got, want, tag):
    rel = float(np.abs(got - want).max() / np.abs(want).max())
    cos = float(np.dot(got.astype(np.float64), want) /
                (np.linalg.norm(got.astype(np.float64)) * np.linalg.norm(want.astype(np.float64))))
    assert np.isfinite(got).all(), tag
    assert rel <= TOL and cos >= COS, (tag, rel, cos)
    return rel


def _pair(cfg, seed, std):
    dev = hip.HybridLM(cfg)
    dev.init_synthetic(seed, std)
    ref = O.HybridLM(cfg)
    ref.init_synthetic(seed, std)
    return dev, ref


@pytest.mark.parametrize("variant", ["conv_gqa", "gqa_first", "conv_bias"])
def test_hybrid_tiny_tracks_oracle(variant):
    cfg = dict(TINY)
    if variant == "gqa_first":
        cfg["layer_kinds"] = [1, 0, 0, 1]
    if variant == "conv_bias":
        cfg["conv_bias"] = 1
    dev, ref = _pair(cfg, 0x5EED0000, 0.08)
    toks = O.token_ids(40, 11, cfg["vocab"])
    worst = 0.0
    for t, tok in enumerate(toks):
        worst = max(worst, _cmp(dev.decode_one(int(tok)), ref.decode_one(int(tok)), (variant, t)))
    assert dev.pos == ref.pos == 40
    print(f"{variant}: worst rel {worst:.2e}")


def test_hybrid_reset_and_graph_forms_agree():
    dev = hip.HybridLM(TINY)
    dev.init_synthetic(3, 0.08)
    toks = [5, 9, 100, 7, 7, 42]
    eager = []
    dev.set_options(graph=False)
    for t in toks:
        eager.append(dev.decode_one(t))
    dev.reset()
    assert dev.pos == 0
    dev.set_options(graph=True)
    for t, want in zip(toks, eager):
        np.testing.assert_array_equal(dev.decode_one(t), want)


def test_hybrid_generate_matches_oracle_tokens():
    cfg = dict(TINY, max_seq=96)
    dev, ref = _pair(cfg, 77, 0.1)
    prompt = O.token_ids(12, 5, cfg["vocab"])
    dt, dm = dev.generate(prompt, 48)
    rt, rm = ref.generate(prompt, 48)
    for i in range(48):
        if rm[i] <= 1e-3:
            break
        assert dt[i] == rt[i], (i, dt[:i + 1], rt[:i + 1])
    np.testing.assert_allclose(dm[:8], rm[:8], rtol=1e-3, atol=1e-3)


def test_hybrid_lfm25_widths_track_oracle():
    """LFM2.5-350M widths (hidden 1024, inner 1024, 16/8 heads of 64, FFN 6656,
    vocab 65536, conv kernel 3) with the first four layer kinds."""
    cfg = dict(O.LFM25_350M, n_layers=4, layer_kinds=O.LFM25_KINDS[:4], max_seq=48)
    dev, ref = _pair(cfg, 0x5EED0000, 0.02)
    toks = O.token_ids(24, 3, cfg["vocab"])
    for t, tok in enumerate(toks):
        _cmp(dev.decode_one(int(tok)), ref.decode_one(int(tok)), ("lfm4", t))


def test_hybrid_lfm25_full_depth_properties():
    """All 16 LFM2.5-350M layers: finite logits, greedy generate equal to the
    argmax of a decode_one loop from the same state."""
    cfg = dict(O.LFM25_350M, max_seq=80)
    dev = hip.HybridLM(cfg)
    dev.init_synthetic(0x5EED0000, 0.02)
    prompt = O.token_ids(8, 9, cfg["vocab"])
    toks, margins = dev.generate(prompt, 24)
    assert dev.pos == 8 + 24 - 1
    dev.reset()
    lg = dev.prefill(prompt)
    loop = []
    for _ in range(24):
        assert np.isfinite(lg).all()
        nxt = int(np.flatnonzero(lg == lg.max())[-1])  # last maximum wins
        loop.append(nxt)
        lg = dev.decode_one(nxt)
    np.testing.assert_array_equal(toks, loop)
    assert (margins >= 0).all()
