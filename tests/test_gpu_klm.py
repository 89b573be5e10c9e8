"""f32 decoder over Q4_K / Q6_K / Q8_0 weights (config 3 path) vs the oracle's
CausalLM, which dequantizes the same bytes and runs the reference's f32 ops.

The device decodes blocks in registers and sums in a different order (and the
prefill GEMM rounds operands to f16), so the bar is the north star's float
one: logits cosine >= 0.9999 and per-row max relative error small; greedy
tokens are compared where the oracle's top1-top2 margin is not razor thin."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests import gguf_writer as W

pytestmark = pytest.mark.gpu

NAMES = {hip.FMT_Q8_0: "q8_0", hip.FMT_Q4_K: "q4_k", hip.FMT_Q6_K: "q6_k"}


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _cos(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def build_pair(cfg, fmts, seed=0x5EED0000, qk_norm=False):
    """Same f32 weights -> same block bytes -> oracle and device models."""
    fq, fo, fgu, fd, flm = fmts
    o = O.CausalLM(cfg, qk_norm=qk_norm)
    g = hip.KQuantCausalLM(cfg, fq, fo, fgu, fd, flm, qk_norm=qk_norm)
    h, qd = cfg["hidden"], cfg["n_heads"] * cfg["head_dim"]
    kvd, inter = cfg["n_kv_heads"] * cfg["head_dim"], cfg["inter"]
    emb = O.normal(cfg["vocab"] * h, seed, 0.02).reshape(cfg["vocab"], h)
    o.set_embed(emb)
    g.set_embed(emb)
    shapes = [(qd, h, fq), (kvd, h, fq), (kvd, h, fq), (h, qd, fo), (inter, h, fgu),
              (inter, h, fgu), (h, inter, fd)]
    for layer in range(cfg["n_layers"]):
        for p, (n, k, f) in enumerate(shapes):
            w = O.normal(n * k, seed + 1 + 8 * layer + p, 0.02).reshape(n, k)
            b = hip.kquant_encode(f, w)
            o.set_proj(layer, p, NAMES[f], b)
            g.set_proj(layer, p, b)
    w = O.normal(cfg["vocab"] * h, seed + 1 + 8 * cfg["n_layers"], 0.02).reshape(cfg["vocab"], h)
    b = hip.kquant_encode(flm, w)
    o.set_lm_head(NAMES[flm], b)
    g.set_lm_head(b)
    g.finalize()
    return o, g


TINY = dict(hidden=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, inter=512, vocab=300,
            max_seq=96, eps=1e-5, rope_theta=5e5)
LLAMA_FMTS = (hip.FMT_Q4_K, hip.FMT_Q4_K, hip.FMT_Q4_K, hip.FMT_Q6_K, hip.FMT_Q6_K)


@pytest.mark.parametrize("prompt_len", [6, 40])  # GEMV prefill (M <= 8) and MFMA GEMM prefill
def test_tiny_llama_style(prompt_len):
    o, g = build_pair(TINY, LLAMA_FMTS)
    ids = O.token_ids(prompt_len, 0x5EED0000 + 0xFFFF, TINY["vocab"])
    lo, lg = o.prefill(ids), g.prefill(ids)
    assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (_cos(lo, lg), _rel(lg, lo))
    tok = O.argmax(lo)
    for step in range(12):
        lo, lg = o.forward_one(tok), g.forward_one(tok)
        assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (step, _rel(lg, lo))
        tok = O.argmax(lo)


def test_prefill_attention_hd128_row_blocks_and_append():
    # the tolerance-graded prefill attention (32-row blocks, 64-position
    # chunks) at head dim 128 with GQA: a 150-token prompt (five row blocks,
    # three chunks) and a 70-token append at cache offset 150
    cfg = dict(hidden=512, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128, inter=512,
               vocab=300, max_seq=232, eps=1e-5, rope_theta=5e5)
    o, g = build_pair(cfg, LLAMA_FMTS)
    ids = O.token_ids(150, 0x5EED0000 + 0xFFFF, cfg["vocab"])
    lo, lg = o.prefill(ids), g.prefill(ids)
    assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (_cos(lo, lg), _rel(lg, lo))
    extra = O.token_ids(70, 0x5EED0000 + 0x1234, cfg["vocab"])
    lo, lg = o.prefill_append(extra), g.prefill_append(extra)
    assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (_cos(lo, lg), _rel(lg, lo))
    tok = O.argmax(lo)
    for step in range(4):
        lo, lg = o.forward_one(tok), g.forward_one(tok)
        assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (step, _rel(lg, lo))
        tok = O.argmax(lo)


@pytest.mark.parametrize("t", [752, 753])
def test_prefill_attention_hd128_tile_switch_point(t):
    # head dim 128: the tile kernel holds 32 score rows of round_up4(t) + 1
    # floats beside its K / V chunks in 144 KiB of LDS, which fits up to 752
    # tokens; 753 takes the bit-exact row kernel.  Both sides of the switch
    # against the oracle.
    cfg = dict(hidden=256, n_layers=1, n_heads=2, n_kv_heads=1, head_dim=128, inter=256,
               vocab=300, max_seq=760, eps=1e-5, rope_theta=5e5)
    o, g = build_pair(cfg, LLAMA_FMTS)
    ids = O.token_ids(t, 0x5EED0000 + 0xFFFF, cfg["vocab"])
    lo, lg = o.prefill(ids), g.prefill(ids)
    assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (_cos(lo, lg), _rel(lg, lo))
    tok = O.argmax(lo)
    lo, lg = o.forward_one(tok), g.forward_one(tok)
    assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (_cos(lo, lg), _rel(lg, lo))


def test_tiny_q8_0_with_qk_norm_greedy():
    fm = (hip.FMT_Q8_0,) * 5
    o, g = build_pair(TINY, fm, qk_norm=True)
    ids = O.token_ids(8, 0x5EED0000 + 0xFFFF, TINY["vocab"])
    to, mo = o.generate(ids, 32)
    tg, _ = g.generate(ids, 32)
    # identical while the oracle's margin is not below float noise
    first_thin = next((i for i, m in enumerate(mo) if m < 1e-4), len(mo))
    np.testing.assert_array_equal(tg[:first_thin], to[:first_thin])


def test_llama_3b_widths_two_layers():
    # LLaMA-3.2-3B widths and vocab (h 3072, 24q/8kv, hd 128, inter 8192,
    # vocab 128256; Q4_K attn + gate/up, Q6_K down + lm_head), 2 layers
    cfg = dict(hidden=3072, n_layers=2, n_heads=24, n_kv_heads=8, head_dim=128, inter=8192,
               vocab=128256, max_seq=64, eps=1e-5, rope_theta=5e5)
    o, g = build_pair(cfg, LLAMA_FMTS)
    ids = O.token_ids(16, 0x5EED0000 + 0xFFFF, cfg["vocab"])
    lo, lg = o.prefill(ids), g.prefill(ids)
    print("prefill cos", _cos(lo, lg), "rel", _rel(lg, lo))
    assert _cos(lo, lg) >= 0.9999
    tok = O.argmax(lo)
    for step in range(4):
        lo, lg = o.forward_one(tok), g.forward_one(tok)
        print("decode", step, "cos", _cos(lo, lg), "rel", _rel(lg, lo))
        assert _cos(lo, lg) >= 0.9999
        tok = O.argmax(lo)


# ------------------------------------------------------------------ GGUF files
GGML = {hip.FMT_Q8_0: 8, hip.FMT_Q4_K: 12, hip.FMT_Q6_K: 14}
LLAMA_NAMES = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
HF_NAMES = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
            "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]


def _gguf_model(tmp_path, cfg, fmts, qk_norm, hf, tied, seed=0x5EED1000):
    """One set of weights and norm gains written to a GGUF file, set into the
    oracle, and set into a device model through the per-tensor API."""
    fq, fo, fgu, fd, flm = fmts
    h, hd = cfg["hidden"], cfg["head_dim"]
    qd, kvd, inter = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["inter"]
    o = O.CausalLM(cfg, qk_norm=qk_norm)
    api = hip.KQuantCausalLM(cfg, fq, fo, fgu, fd, flm, qk_norm=qk_norm)
    tensors = []

    def gain(n, s):  # f16-representable gains around 1, stored as F16 or F32
        return (1.0 + O.normal(n, s, 0.2)).astype(np.float16).astype(np.float32)

    shapes = [(qd, h, fq), (kvd, h, fq), (kvd, h, fq), (h, qd, fo), (inter, h, fgu),
              (inter, h, fgu), (h, inter, fd)]
    for layer in range(cfg["n_layers"]):
        pre = f"model.layers.{layer}." if hf else f"blk.{layer}."
        for p, (n, k, f) in enumerate(shapes):
            b = hip.kquant_encode(f, O.normal(n * k, seed + 16 * layer + p, 0.02).reshape(n, k))
            o.set_proj(layer, p, NAMES[f], b)
            api.set_proj(layer, p, b)
            nm = HF_NAMES[p] if hf else LLAMA_NAMES[p]
            tensors.append((pre + nm + ".weight", GGML[f], [k, n], b.tobytes()))
        an, fn = gain(h, seed + 16 * layer + 8), gain(h, seed + 16 * layer + 9)
        qn = gain(hd, seed + 16 * layer + 10) if qk_norm else None
        kn = gain(hd, seed + 16 * layer + 11) if qk_norm else None
        o.set_norms(layer, an, fn, qn, kn)
        api.set_norms(layer, an, fn, qn, kn)
        names = (["input_layernorm", "post_attention_layernorm", "self_attn.q_norm",
                  "self_attn.k_norm"] if hf else
                 ["attn_norm", "ffn_norm", "attn_q_norm", "attn_k_norm"])
        tensors.append((pre + names[0] + ".weight", 0, [h], an.tobytes()))
        tensors.append((pre + names[1] + ".weight", 1, [h], fn.astype(np.float16).tobytes()))
        if qk_norm:
            tensors.append((pre + names[2] + ".weight", 1, [hd], qn.astype(np.float16).tobytes()))
            tensors.append((pre + names[3] + ".weight", 0, [hd], kn.tobytes()))
    final = gain(h, seed + 0xF00)
    o.set_final_norm(final)
    api.set_final_norm(final)
    tensors.append(("model.norm.weight" if hf else "output_norm.weight", 0, [h],
                    final.tobytes()))
    vocab = cfg["vocab"]
    wl = O.normal(vocab * h, seed + 0xF01, 0.02).reshape(vocab, h)
    if tied:
        # token_embd in the lm_head format and no output.weight: both use it
        b = hip.kquant_encode(flm, wl)
        emb = O.dequant(NAMES[flm], b, vocab * h).reshape(vocab, h)
        tensors.append(("model.embed_tokens.weight" if hf else "token_embd.weight", GGML[flm],
                        [h, vocab], b.tobytes()))
    else:
        emb = O.normal(vocab * h, seed + 0xF02, 0.02).reshape(vocab, h)
        b = hip.kquant_encode(flm, wl)
        tensors.append(("model.embed_tokens.weight" if hf else "token_embd.weight", 0,
                        [h, vocab], emb.tobytes()))
        tensors.append(("lm_head.weight" if hf else "output.weight", GGML[flm], [h, vocab],
                        b.tobytes()))
    o.set_embed(emb)
    api.set_embed(emb)
    o.set_lm_head(NAMES[flm], b)
    api.set_lm_head(b)
    api.finalize()
    path = W.write_gguf(tmp_path / "model.gguf", tensors,
                        [("general.architecture", W.STRING, "llama")])
    return o, api, path


@pytest.mark.parametrize("hf,tied,qk_norm,fmts", [
    (False, False, False, LLAMA_FMTS),
    (True, True, True, (hip.FMT_Q8_0,) * 5),
    (False, True, True, (hip.FMT_Q4_K, hip.FMT_Q6_K, hip.FMT_Q4_K, hip.FMT_Q6_K, hip.FMT_Q6_K)),
])
def test_load_gguf_matches_api_and_oracle(tmp_path, hf, tied, qk_norm, fmts):
    o, api, path = _gguf_model(tmp_path, TINY, fmts, qk_norm, hf, tied)
    with hip.Gguf(path) as f:
        g = hip.KQuantCausalLM(TINY, *fmts, qk_norm=qk_norm)
        g.load_gguf(f)
    ids = O.token_ids(12, 0x5EED0000 + 0xFFFF, TINY["vocab"])
    lo, la, lg = o.prefill(ids), api.prefill(ids), g.prefill(ids)
    # same bytes and gains through both routes: identical device results
    np.testing.assert_array_equal(lg, la)
    assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (_cos(lo, lg), _rel(lg, lo))
    tok = O.argmax(lo)
    for step in range(8):
        lo, la, lg = o.forward_one(tok), api.forward_one(tok), g.forward_one(tok)
        np.testing.assert_array_equal(lg, la)
        assert _cos(lo, lg) >= 0.9999 and _rel(lg, lo) < 5e-3, (step, _rel(lg, lo))
        tok = O.argmax(lo)


def test_load_gguf_rejects_wrong_format(tmp_path):
    _, _, path = _gguf_model(tmp_path, TINY, LLAMA_FMTS, False, False, False)
    with hip.Gguf(path) as f:
        g = hip.KQuantCausalLM(TINY, *((hip.FMT_Q8_0,) * 5))
        with pytest.raises(hip.SynapseError, match="GGML type"):
            g.load_gguf(f)


# ------------------------------------------------------------------ fused decode step
# The fused step (klm_fused.hip: five kernels per layer, split-K partials
# summed by the consumer, flash-decoding attention over 64-position chunks)
# sums in another order than the op-by-op step, so it is held to the
# oracle's tolerance and to the op-by-op step within rounding; graph replay,
# eager launches and repeated runs of it must agree bit for bit.
FUSED_CASES = [
    # (n_heads, n_kv_heads, head_dim, fmts, qk_norm): GQA group sizes 1..8
    (16, 16, 16, LLAMA_FMTS, False),
    (8, 2, 32, LLAMA_FMTS, True),
    (6, 2, 64, (hip.FMT_Q8_0,) * 5, True),
    (16, 2, 128, LLAMA_FMTS, False),
    (4, 1, 128, (hip.FMT_Q6_K, hip.FMT_Q4_K, hip.FMT_Q8_0, hip.FMT_Q4_K, hip.FMT_Q4_K), False),
]


def _fused_cfg(nh, nkv, hd, max_seq=150):
    # max_seq not a multiple of 64: the last chunk of the cache is partial
    return dict(hidden=512, n_layers=2, n_heads=nh, n_kv_heads=nkv, head_dim=hd, inter=768,
                vocab=520, max_seq=max_seq, eps=1e-5, rope_theta=1e4)


def _teacher_forced(g, ids, toks):
    g.prefill(ids)
    return [g.forward_one(t) for t in toks]


@pytest.mark.parametrize("nh,nkv,hd,fmts,qkn", FUSED_CASES)
def test_fused_step_tracks_oracle_and_op_by_op(nh, nkv, hd, fmts, qkn):
    cfg = _fused_cfg(nh, nkv, hd)
    o, g = build_pair(cfg, fmts, qk_norm=qkn)
    ids = O.token_ids(60, 0x5EED0000 + 0xFFFF, cfg["vocab"])
    # decode from position 60 across the chunk boundary at 64 to 89
    toks = [int(t) for t in O.token_ids(30, 0x5EED0000 + 0x7777, cfg["vocab"])]
    print(f"case nh={nh} nkv={nkv} hd={hd} qk_norm={qkn}", flush=True)
    g.set_options(fused=False, graph=True)
    unf = _teacher_forced(g, ids, toks)
    g.set_options(fused=True, graph=True)
    fus = _teacher_forced(g, ids, toks)
    o.prefill(ids)
    for step, t in enumerate(toks):
        lo = o.forward_one(t)
        assert _cos(lo, fus[step]) >= 0.9999 and _rel(fus[step], lo) < 5e-3, (step,)
        assert _cos(unf[step], fus[step]) >= 0.99999 and _rel(fus[step], unf[step]) < 2e-4, step


@pytest.mark.parametrize("nh,nkv,hd,fmts,qkn", [FUSED_CASES[1], FUSED_CASES[3]])
def test_fused_step_graph_eager_and_reruns_identical(nh, nkv, hd, fmts, qkn):
    cfg = _fused_cfg(nh, nkv, hd)
    _, g = build_pair(cfg, fmts, qk_norm=qkn)
    # an 8-token prompt takes the GEMV prefill (the MFMA prefill GEMM adds
    # split-K tiles with float atomics, whose rounding varies run to run)
    ids = O.token_ids(8, 0x5EED0000 + 0xFFFF, cfg["vocab"])
    outs = []
    for graph in (True, False, True):
        g.set_options(fused=True, graph=graph)
        outs.append(g.generate(ids, 135))  # positions 8 .. 141: chunk boundaries 64, 128
    for toks, margins in outs[1:]:
        np.testing.assert_array_equal(toks, outs[0][0])
        np.testing.assert_array_equal(margins, outs[0][1])


def test_fused_step_fills_the_cache_to_max_seq():
    # the last decode step writes cache row max_seq - 1 (partial last chunk)
    cfg = _fused_cfg(8, 2, 128, max_seq=130)
    o, g = build_pair(cfg, LLAMA_FMTS)
    ids = O.token_ids(100, 0x5EED0000 + 0xFFFF, cfg["vocab"])
    toks = [int(t) for t in O.token_ids(30, 0x5EED0000 + 0x5555, cfg["vocab"])]
    fus = _teacher_forced(g, ids, toks)
    o.prefill(ids)
    for step, t in enumerate(toks):
        lo = o.forward_one(t)
        assert _cos(lo, fus[step]) >= 0.9999 and _rel(fus[step], lo) < 5e-3, step


def test_fused_step_llama_3b_widths():
    # LLaMA-3.2-3B layer widths: the split plans of the benchmark model
    cfg = dict(hidden=3072, n_layers=2, n_heads=24, n_kv_heads=8, head_dim=128, inter=8192,
               vocab=128256, max_seq=200, eps=1e-5, rope_theta=5e5)
    o, g = build_pair(cfg, LLAMA_FMTS)
    ids = O.token_ids(120, 0x5EED0000 + 0xFFFF, cfg["vocab"])
    toks = [int(t) for t in O.token_ids(16, 0x5EED0000 + 0x3333, cfg["vocab"])]
    g.set_options(fused=False, graph=True)
    unf = _teacher_forced(g, ids, toks)
    g.set_options(fused=True, graph=True)
    fus = _teacher_forced(g, ids, toks)
    o.prefill(ids)
    for step, t in enumerate(toks):
        lo = o.forward_one(t)
        print("step", step, "cos", _cos(lo, fus[step]), "rel", _rel(fus[step], lo),
              "vs op-by-op", _rel(fus[step], unf[step]), flush=True)
        assert _cos(lo, fus[step]) >= 0.9999
        assert _cos(unf[step], fus[step]) >= 0.99999 and _rel(fus[step], unf[step]) < 2e-4
