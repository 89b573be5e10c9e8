"""Fused decode step (five kernels per layer) vs the oracle and vs the
one-kernel-per-op step: all three must agree bit for bit, with and without
HIP graph replay, across the 64-position attention switch and on ragged
shapes (hidden not a multiple of 4 or 16, head_dim not a multiple of 32,
vocab not a multiple of 64, GQA groups of 1..5)."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip

pytestmark = pytest.mark.gpu

PROMPT_SEED = 0x5EED0000 + 0xFFFF
SMALL = dict(hidden=576, n_layers=2, n_heads=6, n_kv_heads=2, head_dim=96, inter=1152,
             vocab=1000, max_seq=128)
RAGGED = dict(hidden=202, n_layers=3, n_heads=5, n_kv_heads=1, head_dim=50, inter=301,
              vocab=777, max_seq=100)
MHA = dict(hidden=256, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=64, inter=512,
           vocab=4099, max_seq=80)
# head sizes of the one-kernel head attention: positions past 64 (fused
# chains), 128 (second staged V chunk) and 256 (second pass of score lanes)
LONG128 = dict(hidden=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128, inter=512,
               vocab=1000, max_seq=300)
HD32 = dict(hidden=192, n_layers=2, n_heads=6, n_kv_heads=3, head_dim=32, inter=384,
            vocab=700, max_seq=160)
HD16 = dict(hidden=128, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=16, inter=256,
            vocab=500, max_seq=150)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("cfg,cap", [(SMALL, 70), (RAGGED, 70), (MHA, 70), (LONG128, 289),
                                     (HD32, 149), (HD16, 139)],
                         ids=["small", "ragged", "mha", "hd128-long", "hd32", "hd16"])
def test_fused_matches_oracle_and_unfused(cfg, cap):
    print("case", cfg, flush=True)
    o = O.QuantizedCausalLM(cfg)
    o.init_synthetic()
    g = hip.QuantizedCausalLM(cfg)
    g.init_synthetic()
    ids = O.token_ids(12, PROMPT_SEED, cfg["vocab"])
    n_new = min(cap, cfg["max_seq"] - ids.size + 1)
    to, mo = o.generate(ids, n_new)
    runs = {}
    for fused in (True, False):
        for graph in (True, False):
            g.set_options(fused=fused, graph=graph)
            runs[(fused, graph)] = g.generate(ids, n_new)
    for key, (tg, mg) in runs.items():
        np.testing.assert_array_equal(tg, to, err_msg=f"fused,graph={key}")
        np.testing.assert_array_equal(_bits(mg), _bits(mo), err_msg=f"fused,graph={key}")


def test_fused_forward_one_logits_bit_exact():
    cfg = SMALL
    o = O.QuantizedCausalLM(cfg)
    o.init_synthetic()
    g = hip.QuantizedCausalLM(cfg)
    g.init_synthetic()
    g.set_options(fused=True, graph=True)
    ids = O.token_ids(20, PROMPT_SEED, cfg["vocab"])
    lo, lg = o.prefill(ids), g.prefill(ids)
    np.testing.assert_array_equal(_bits(lg), _bits(lo))
    tok = O.argmax(lo)
    for step in range(50):  # positions 20..69 cross the 64-position switch
        lo, lg = o.forward_one(tok), g.forward_one(tok)
        np.testing.assert_array_equal(_bits(lg), _bits(lo), err_msg=f"step {step}")
        tok = O.argmax(lo)


def test_fused_rejects_oversized_attention_row():
    # the fused attention keeps the score row in LDS; a longer cache falls back
    cfg = dict(SMALL, max_seq=20000, n_layers=1)
    g = hip.QuantizedCausalLM(cfg)
    g.init_synthetic()
    with pytest.raises(hip.SynapseError):
        g.set_options(fused=True, graph=True)
    g.set_options(fused=False, graph=True)
    ids = O.token_ids(4, PROMPT_SEED, cfg["vocab"])
    toks, _ = g.generate(ids, 3)
    assert toks.shape == (3,)
