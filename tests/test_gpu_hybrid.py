"""Hybrid LFM2.5 decoder (Q4 decode path) on the GPU against the oracle
(orc_hlm: models/ssm/hybrid layer.rs / model.rs restated in C).

Both device forms are graded by tolerance: the op-by-op step (Q4 GEMVs
summed in their own order, the small ops in the reference's order except
RMSNorm's tree sum) and the fused step (five kernels per layer: split-K
Q4_0 rows added into fixed-point accumulators, norms, SwiGLU and the
attention combine inside the GEMVs, chunked attention, tree-ordered f32
lm_head).  Per step max|dev - ref| / max|ref| <= 2e-4 and cosine >= 0.99999;
greedy tokens must agree while the reference's top1 - top2 margin exceeds 1e-3.
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


# the smallest shapes the fused step takes (hidden, inner, inter and the q
# width in whole 256s, head_dim 64); 70 steps cross a 64-position chunk
SMALL = dict(hidden=256, n_layers=4, vocab=512, n_heads=4, n_kv_heads=2, head_dim=64, inner=256,
             conv_kernel=3, inter=512, max_seq=96, eps=1e-5, rope_theta=1e4,
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
    assert not dev.fused_active  # hidden 64: the op-by-op step
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


@pytest.mark.parametrize("kinds", [[0, 1, 0, 1], [1, 0, 0, 1], [0, 0, 0, 0]])
def test_hybrid_fused_tracks_oracle(kinds):
    cfg = dict(SMALL, layer_kinds=kinds, conv_bias=int(kinds[0] == 0 and kinds[1] == 0))
    dev, ref = _pair(cfg, 0x5EED0000, 0.08)
    assert dev.fused_active
    toks = O.token_ids(70, 17, cfg["vocab"])
    worst = 0.0
    for t, tok in enumerate(toks):
        worst = max(worst, _cmp(dev.decode_one(int(tok)), ref.decode_one(int(tok)), (kinds, t)))
    assert dev.pos == ref.pos == 70
    print(f"fused {kinds}: worst rel {worst:.2e}")


@pytest.mark.parametrize("hidden,hd,group", [(512, 64, 2), (768, 64, 4), (1536, 128, 2)])
def test_hybrid_fused_other_widths(hidden, hd, group):
    """Head kernel widths NC = 2, 3, 6 (hidden = 256 NC), head_dim 64 and 128,
    GQA groups of 2 and 4."""
    nh = hidden // hd
    cfg = dict(SMALL, hidden=hidden, inner=hidden, inter=2 * hidden, n_heads=nh,
               n_kv_heads=nh // group, head_dim=hd, vocab=700, n_layers=2, layer_kinds=[1, 0],
               max_seq=32)
    dev, ref = _pair(cfg, 0x5EED0000 + hidden, 0.05)
    assert dev.fused_active
    for t, tok in enumerate(O.token_ids(20, hidden, cfg["vocab"])):
        _cmp(dev.decode_one(int(tok)), ref.decode_one(int(tok)), (hidden, t))


def test_hybrid_fused_long_context():
    """330 positions: the chunked attention combines six 64-position chunks,
    and the conv state halves alternate 330 times."""
    cfg = dict(SMALL, n_layers=2, layer_kinds=[0, 1], max_seq=336)
    dev, ref = _pair(cfg, 9, 0.08)
    assert dev.fused_active
    toks = O.token_ids(330, 21, cfg["vocab"])
    worst = 0.0
    for t, tok in enumerate(toks):
        got, want = dev.decode_one(int(tok)), ref.decode_one(int(tok))
        if t % 10 == 0 or t >= 320:
            worst = max(worst, _cmp(got, want, ("long", t)))
    print(f"long context: worst rel {worst:.2e}")


def test_hybrid_fused_graph_eager_and_reset_agree():
    """Fixed-point split-K sums are order-free: graph replay, eager launches
    and a replay after reset give the same logits bit for bit."""
    dev = hip.HybridLM(SMALL)
    dev.init_synthetic(5, 0.08)
    toks = [5, 9, 300, 7, 7, 42, 511, 0]
    dev.set_options(fused=True, graph=False)
    eager = [dev.decode_one(t) for t in toks]
    for graph in (True, True):
        dev.reset()
        dev.set_options(fused=True, graph=graph)
        for t, want in zip(toks, eager):
            np.testing.assert_array_equal(dev.decode_one(t), want)


def test_hybrid_fused_generate_matches_oracle_tokens():
    cfg = dict(SMALL, max_seq=96)
    dev, ref = _pair(cfg, 77, 0.1)
    assert dev.fused_active
    prompt = O.token_ids(12, 5, cfg["vocab"])
    dt, dm = dev.generate(prompt, 72)
    rt, rm = ref.generate(prompt, 72)
    for i in range(72):
        if rm[i] <= 1e-3:
            break
        assert dt[i] == rt[i], (i, dt[:i + 1], rt[:i + 1])
    np.testing.assert_allclose(dm[:8], rm[:8], rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("fused", [True, False])
def test_hybrid_lfm25_widths_track_oracle(fused):
    """LFM2.5-350M widths (hidden 1024, inner 1024, 16/8 heads of 64, FFN 6656,
    vocab 65536, conv kernel 3) with the first four layer kinds."""
    cfg = dict(O.LFM25_350M, n_layers=4, layer_kinds=O.LFM25_KINDS[:4], max_seq=48)
    dev, ref = _pair(cfg, 0x5EED0000, 0.02)
    dev.set_options(fused=fused)
    assert dev.fused_active == fused
    toks = O.token_ids(24, 3, cfg["vocab"])
    for t, tok in enumerate(toks):
        _cmp(dev.decode_one(int(tok)), ref.decode_one(int(tok)), ("lfm4", fused, t))


def test_hybrid_lfm25_full_depth_properties():
    """All 16 LFM2.5-350M layers: finite logits, greedy generate equal to the
    argmax of a decode_one loop from the same state."""
    cfg = dict(O.LFM25_350M, max_seq=80)
    dev = hip.HybridLM(cfg)
    dev.init_synthetic(0x5EED0000, 0.02)
    assert dev.fused_active
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
