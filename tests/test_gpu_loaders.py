"""Models and linear layers loaded from weight files on the device.

Each file route is compared with the per-tensor API fed the same values (the
device results must be bit-identical: same bytes, same kernels) and with the
oracle (bit-exact for the INT8 decoder, whose whole pipeline is)."""
import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests import gguf_writer as G
from tests import safetensors_writer as S

pytestmark = pytest.mark.gpu

CFG = dict(hidden=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, inter=512, vocab=384,
           max_seq=64, eps=1e-6, rope_theta=1e6)
PROMPT_SEED = 0x5EED0000 + 0xFFFF


@pytest.fixture(scope="module", autouse=True)
def gpu():
    hip.init(0)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _bf16_round(x):
    """values exactly representable in bf16 (truncated), as f32"""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)


def _model_weights(cfg, seed, qk_norm=True, untied=True, bf16=False):
    h, hd = cfg["hidden"], cfg["head_dim"]
    qd, kvd, inter = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["inter"]
    rnd = _bf16_round if bf16 else (lambda x: x)
    shapes = {"q": (qd, h), "k": (kvd, h), "v": (kvd, h), "o": (h, qd), "gate": (inter, h),
              "up": (inter, h), "down": (h, inter)}
    layers = []
    for layer in range(cfg["n_layers"]):
        lw = {n: rnd(O.normal(r * c, seed + 16 * layer + i, 0.05).reshape(r, c))
              for i, (n, (r, c)) in enumerate(shapes.items())}
        lw["attn_norm"] = 1.0 + O.normal(h, seed + 16 * layer + 8, 0.3)
        lw["ffn_norm"] = 1.0 + O.normal(h, seed + 16 * layer + 9, 0.3)
        if qk_norm:
            lw["q_norm"] = 1.0 + O.normal(hd, seed + 16 * layer + 10, 0.3)
            lw["k_norm"] = 1.0 + O.normal(hd, seed + 16 * layer + 11, 0.3)
        layers.append(lw)
    embed = rnd(O.normal(cfg["vocab"] * h, seed + 0xE0, 0.05).reshape(cfg["vocab"], h))
    final = 1.0 + O.normal(h, seed + 0xE1, 0.3)
    lm = rnd(O.normal(cfg["vocab"] * h, seed + 0xE2, 0.05).reshape(cfg["vocab"], h)) \
        if untied else None
    return embed, layers, final, lm


HF = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
      "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
      "down": "mlp.down_proj", "attn_norm": "input_layernorm",
      "ffn_norm": "post_attention_layernorm", "q_norm": "self_attn.q_norm",
      "k_norm": "self_attn.k_norm"}
LLAMA = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate",
         "up": "ffn_up", "down": "ffn_down", "attn_norm": "attn_norm", "ffn_norm": "ffn_norm",
         "q_norm": "attn_q_norm", "k_norm": "attn_k_norm"}


def _st_tensors(embed, layers, final, lm, bf16, fused=False):
    def enc(name, x):
        x = np.ascontiguousarray(x, np.float32)
        if bf16 and x.ndim == 2:
            return (name, "BF16", list(x.shape), S.bf16_bits(x).tobytes())
        return (name, x)

    out = [enc("model.embed_tokens.weight", embed), enc("model.norm.weight", final)]
    if lm is not None:
        out.append(enc("lm_head.weight", lm))
    for l, lw in enumerate(layers):
        pre = f"model.layers.{l}."
        if fused:
            out.append(enc(pre + "self_attn.qkv_proj.weight",
                           np.concatenate([lw["q"], lw["k"], lw["v"]])))
            out.append(enc(pre + "mlp.gate_up_proj.weight",
                           np.concatenate([lw["gate"], lw["up"]])))
        for n, x in lw.items():
            if fused and n in ("q", "k", "v", "gate", "up"):
                continue
            out.append(enc(pre + HF[n] + ".weight", x))
    return out


def _run_pair(cfg, o, g, ids, steps):
    lo, lg = o.prefill(ids), g.prefill(ids)
    np.testing.assert_array_equal(_bits(lg), _bits(lo))
    tok = O.argmax(lo)
    for step in range(steps):
        lo, lg = o.forward_one(tok), g.forward_one(tok)
        np.testing.assert_array_equal(_bits(lg), _bits(lo), err_msg=f"step {step}")
        tok = O.argmax(lo)


@pytest.mark.parametrize("bf16,fused,untied,qk_norm", [
    (True, False, True, True),    # Qwen3-style bf16 checkpoint with an lm_head
    (False, True, False, True),   # fused qkv / gate_up projections, tied head
    (True, False, False, False),  # no head norms (LLaMA-style)
])
def test_int8_decoder_from_safetensors(tmp_path, bf16, fused, untied, qk_norm):
    embed, layers, final, lm = _model_weights(CFG, 0x5EED7000, qk_norm, untied, bf16)
    S.write_st(tmp_path / "model.safetensors",
               _st_tensors(embed, layers, final, lm, bf16, fused), {"format": "pt"})
    o = O.QuantizedCausalLM(CFG)
    o.set_weights(embed, layers, final, lm, qk_norm=qk_norm)
    api = hip.QuantizedCausalLM(CFG)
    api.set_weights(embed, layers, final, lm, qk_norm=qk_norm)
    g = hip.QuantizedCausalLM(CFG)
    with hip.Safetensors(tmp_path / "model.safetensors") as st:
        g.load_safetensors(st)
    ids = O.token_ids(20, PROMPT_SEED, CFG["vocab"])
    np.testing.assert_array_equal(_bits(g.prefill(ids)), _bits(api.prefill(ids)))
    _run_pair(CFG, o, g, ids, 12)
    to, mo = o.generate(ids, 16)
    tg, mg = g.generate(ids, 16)
    np.testing.assert_array_equal(tg, to)
    np.testing.assert_array_equal(_bits(mg), _bits(mo))


def test_int8_decoder_from_sharded_checkpoint(tmp_path):
    embed, layers, final, lm = _model_weights(CFG, 0x5EED7100)
    tensors = _st_tensors(embed, layers, final, lm, True)
    half = len(tensors) // 2
    S.write_st(tmp_path / "model-00001-of-00002.safetensors", tensors[:half])
    S.write_st(tmp_path / "model-00002-of-00002.safetensors", tensors[half:])
    S.write_index(tmp_path, {t[0]: f"model-0000{1 + (i >= half)}-of-00002.safetensors"
                             for i, t in enumerate(tensors)})
    S.write_st(tmp_path / "single.safetensors", tensors)
    a, b = hip.QuantizedCausalLM(CFG), hip.QuantizedCausalLM(CFG)
    with hip.Safetensors(tmp_path) as st:
        a.load_safetensors(st)
    with hip.Safetensors(tmp_path / "single.safetensors") as st:
        b.load_safetensors(st)
    ids = O.token_ids(12, PROMPT_SEED, CFG["vocab"])
    ta, _ = a.generate(ids, 24)
    tb, _ = b.generate(ids, 24)
    np.testing.assert_array_equal(ta, tb)


@pytest.mark.parametrize("wtype", [G.F16, G.Q8_0])
def test_int8_decoder_from_gguf(tmp_path, wtype):
    # llama.cpp names; weights stored F16 or Q8_0, converted as parse_gguf does
    embed, layers, final, lm = _model_weights(CFG, 0x5EED7200)
    tensors = []

    def add(name, x):
        x = np.ascontiguousarray(x, np.float32)
        if x.ndim == 1:
            tensors.append((name, G.F32, [x.size], x.tobytes()))
        elif wtype == G.F16:
            tensors.append((name, G.F16, [x.shape[1], x.shape[0]], x.astype(np.float16).tobytes()))
        else:
            tensors.append((name, G.Q8_0, [x.shape[1], x.shape[0]],
                            hip.kquant_encode(hip.FMT_Q8_0, x).tobytes()))

    add("token_embd.weight", embed)
    add("output_norm.weight", final)
    add("output.weight", lm)
    for l, lw in enumerate(layers):
        for n, x in lw.items():
            add(f"blk.{l}.{LLAMA[n]}.weight", x)
    p = G.write_gguf(tmp_path / "m.gguf", tensors, [("general.architecture", G.STRING, "qwen3")])
    g = hip.QuantizedCausalLM(CFG)
    with hip.Gguf(p) as f:
        g.load_gguf(f)
        # the oracle gets the values the file decodes to
        conv = {f.info(i).name: f.to_f32(i).reshape(tuple(reversed(f.info(i).dims)))
                for i in range(len(f))}
    emb = conv["token_embd.weight"]
    lyr = [{n: conv[f"blk.{l}.{LLAMA[n]}.weight"] for n in lw} for l, lw in enumerate(layers)]
    o = O.QuantizedCausalLM(CFG)
    o.set_weights(emb, lyr, conv["output_norm.weight"], conv["output.weight"])
    _run_pair(CFG, o, g, O.token_ids(16, PROMPT_SEED, CFG["vocab"]), 10)


def test_loader_errors(tmp_path):
    embed, layers, final, lm = _model_weights(CFG, 0x5EED7300)
    tensors = _st_tensors(embed, layers, final, lm, False)
    bad = [t for t in tensors if t[0] != "model.layers.1.mlp.down_proj.weight"]
    S.write_st(tmp_path / "missing.safetensors", bad)
    g = hip.QuantizedCausalLM(CFG)
    with hip.Safetensors(tmp_path / "missing.safetensors") as st:
        with pytest.raises(hip.SynapseError, match="model.layers.1.mlp.down_proj"):
            g.load_safetensors(st)
    wrong = [(n, x.T.copy()) if n == "model.layers.0.mlp.down_proj.weight" else (n, x)
             for n, x in tensors]
    S.write_st(tmp_path / "wrong.safetensors", wrong)
    g = hip.QuantizedCausalLM(CFG)
    with hip.Safetensors(tmp_path / "wrong.safetensors") as st:
        with pytest.raises(hip.SynapseError, match="down_proj.weight is 512x256, the model expects 256x512"):
            g.load_safetensors(st)


# ------------------------------------------------------------------ QLinear
def test_qlinear_from_gguf_block_types(tmp_path):
    n, k = 96, 512
    w = O.normal(n * k, 0x5EED7400, 0.05).reshape(n, k)
    q4 = O.q4_pack(w)
    blocks = {hip.FMT_Q8_0: (G.Q8_0, hip.kquant_encode(hip.FMT_Q8_0, w)),
              hip.FMT_Q4_K: (G.Q4_K, hip.kquant_encode(hip.FMT_Q4_K, w)),
              hip.FMT_Q6_K: (G.Q6_K, hip.kquant_encode(hip.FMT_Q6_K, w))}
    tensors = [("q4", G.Q4_0, [k, n], q4.tobytes())]
    tensors += [(f"t{f}", gt, [k, n], b.tobytes()) for f, (gt, b) in blocks.items()]
    p = G.write_gguf(tmp_path / "m.gguf", tensors)
    x = O.normal(3 * k, 0x5EED7401, 1.0).reshape(3, k)
    with hip.Gguf(p) as g:
        a = hip.QLinear.from_gguf(g, "q4")
        ref = hip.QLinear.q4_0(q4, n, k)
        np.testing.assert_array_equal(_bits(a.forward(x)), _bits(ref.forward(x)))
        want = np.stack([O.q4_0_gemv(x[i], q4, n) for i in range(3)])
        assert np.abs(a.forward(x) - want).max() <= 1e-3 * np.abs(want).max()
        for f, (gt, b) in blocks.items():
            a = hip.QLinear.from_gguf(g, f"t{f}")
            ref = hip.QLinear.gguf(f, b, n, k)
            np.testing.assert_array_equal(_bits(a.forward(x)), _bits(ref.forward(x)))


def test_qlinear_from_safetensors_q4_triple(tmp_path):
    n, k = 70, 256
    w = O.normal(n * k, 0x5EED7500, 0.05).reshape(n, k)
    packed = O.q4_pack(w)
    bpr = k // 32
    blocks = packed.reshape(n, bpr, 18)
    scales = np.ascontiguousarray(blocks[:, :, :2]).view(np.uint16).reshape(n, bpr)
    S.write_st(tmp_path / "q.safetensors", [
        ("enc.w.q4_nibbles", "U8", [n, bpr, 16], np.ascontiguousarray(blocks[:, :, 2:]).tobytes()),
        ("enc.w.q4_scales", "F16", [n, bpr], scales.tobytes()),
        ("enc.w.q4_orig_cols", "I64", [1], np.array([k], np.int64).tobytes())])
    x = O.normal(2 * k, 0x5EED7501, 1.0).reshape(2, k)
    with hip.Safetensors(tmp_path / "q.safetensors") as st:
        a = hip.QLinear.from_safetensors_q4(st, "enc.w")
    ref = hip.QLinear.q4_0(packed, n, k)
    np.testing.assert_array_equal(_bits(a.forward(x)), _bits(ref.forward(x)))
