"""Model-level pins of the oracle's decoders: independent float64 numpy
forwards, written from the reference sources, of a tiny Qwen3-style W8A8
decoder (quantization/lm/int8.rs:170-709), a tiny f32 CausalLM over GGUF
Q8_0 weights (models/lm/causal_lm.rs, decoder_layer.rs) and a tiny INT8
Mamba (quantization/ssm/int8_mamba.rs:43-224, zig/src/ops/selective_scan.zig
:30-90), compared with the oracle's logits.  Each reference is also run with
a planted wiring mistake (a dropped residual add, gate and up swapped,
reversed conv taps, the gate's SiLU on the wrong operand) to show that the
comparison fails for it.  Plus the conv1d impulse response and the fused
SwiGLU against numpy."""
import numpy as np
import pytest

import oracle as O


# ---------------------------------------------------------------- shared pieces
def rha(v):
    """round half away from zero (f32::round)"""
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def q8_rows(x):
    """per-row activation quantizer (quantize.zig:12-47), in float64"""
    x = np.atleast_2d(x)
    m = np.abs(x).max(axis=1)
    q = np.zeros_like(x)
    s = np.ones(x.shape[0])
    nz = m > 0
    q[nz] = np.clip(rha(x[nz] * (127.0 / m[nz])[:, None]), -127, 127)
    s[nz] = m[nz] / 127.0
    return q, s


def quant_weights(w):
    """QuantizedLinear::from_f32 (int8_linear.rs:35-70, calibration.rs:11-24),
    in float32 like the reference: s = max|row|/127 (1 for a zero row),
    q = clamp(round(w * (1/s)), -128, 127); w is [N, K]"""
    w = np.asarray(w, np.float32)
    m = np.abs(w).max(axis=1)
    s = np.where(m == 0, np.float32(1), m / np.float32(127)).astype(np.float32)
    inv = (np.float32(1) / s).astype(np.float32)
    q = np.clip(rha((w * inv[:, None]).astype(np.float32)), -128, 127)
    return q.astype(np.float64), s.astype(np.float64)


def qlinear(x, wq):
    """QuantizedLinear::forward: quantize the rows, exact integer products,
    (acc * sx) * sw"""
    q, s = wq
    xq, sx = q8_rows(x)
    acc = xq.astype(np.int64) @ q.T.astype(np.int64)
    return acc * sx[:, None] * s[None, :]


def rmsnorm(x, g, eps):
    x = np.atleast_2d(x)
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * g


def silu(x):
    return x / (1.0 + np.exp(-x))


def rope(x, pos, theta):
    """rotate-half RoPE, tables as models/lm/builder.rs:88-133 (in float64)"""
    hd = x.shape[-1]
    half = hd // 2
    freq = 1.0 / theta ** (np.arange(half) * 2.0 / hd)
    ang = pos[:, None] * freq[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def causal_attention(q, k, v, nh, nkv):
    """q [T, nh, hd], k/v [T, nkv, hd] -> [T, nh*hd] (ops/attention.rs:24-247)"""
    T, _, hd = q.shape
    g = nh // nkv
    out = np.zeros((T, nh, hd))
    mask = np.triu(np.ones((T, T), bool), 1)
    for h in range(nh):
        sc = q[:, h] @ k[:, h // g].T / np.sqrt(hd)
        sc[mask] = -np.inf
        sc -= sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h] = p @ v[:, h // g]
    return out.reshape(T, nh * hd)


def cmp(a, b):
    """(cosine, max |a - b| / max |b|)"""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    cos = float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))
    return cos, float(np.abs(a - b).max() / np.abs(b).max())


# ---------------------------------------------------------------- decoders
def decoder_ref(cfg, W, ids, quantized, qk_norm, mutate=()):
    """logits of the last position; int8.rs:242-505 / decoder_layer.rs layer order:
    norm -> q,k,v -> head norms -> RoPE -> attention -> o -> +res -> norm ->
    gate, up -> silu(gate)*up -> down -> +res; final norm; lm_head"""
    h, nh, nkv, hd = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    eps, theta = cfg["eps"], cfg["rope_theta"]
    lin = (lambda x, w: qlinear(x, w)) if quantized else (lambda x, w: x @ w.T)
    T = len(ids)
    pos = np.arange(T, dtype=np.float64)
    x = W["embed"][np.asarray(ids)].astype(np.float64)
    for L in W["layers"]:
        n = rmsnorm(x, L["attn_norm"], eps)
        q = lin(n, L["q"]).reshape(T, nh, hd)
        k = lin(n, L["k"]).reshape(T, nkv, hd)
        v = lin(n, L["v"]).reshape(T, nkv, hd)
        if qk_norm:
            q = rmsnorm(q.reshape(-1, hd), L["q_norm"], eps).reshape(T, nh, hd)
            k = rmsnorm(k.reshape(-1, hd), L["k_norm"], eps).reshape(T, nkv, hd)
        q, k = rope(q, pos, theta), rope(k, pos, theta)
        o = lin(causal_attention(q, k, v, nh, nkv), L["o"])
        x = o if "no_attn_residual" in mutate else x + o
        n = rmsnorm(x, L["ffn_norm"], eps)
        g, u = lin(n, L["gate"]), lin(n, L["up"])
        if "swap_gate_up" in mutate:
            g, u = u, g
        d = lin(silu(g) * u, L["down"])
        x = d if "no_ffn_residual" in mutate else x + d
    xf = rmsnorm(x[-1], W["final_norm"], eps)
    return lin(xf, W["lm_head"])[0]


QCFG = dict(hidden=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, inter=128,
            vocab=256, max_seq=32, eps=1e-6, rope_theta=1e6)


# Weights of about 1/sqrt(fan-in) (and a unit-scale embedding), so that every
# sub-layer moves the residual stream as much as the stream itself: with the
# N(0, 0.02) weights of the benchmark shapes a tiny model's logits are the
# embedding's, and a wiring mistake inside a layer would hardly show.
WSTD = 0.15


def _qwen3_weights(seed=11):
    rng = np.random.default_rng(seed)
    c = QCFG
    h, qd, kvd, it = c["hidden"], c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"], c["inter"]
    f = lambda *s: rng.normal(0, WSTD, s).astype(np.float32)
    gain = lambda n: (1.0 + 0.1 * rng.normal(size=n)).astype(np.float32)
    layers = [dict(q=f(qd, h), k=f(kvd, h), v=f(kvd, h), o=f(h, qd), gate=f(it, h), up=f(it, h),
                   down=f(h, it), attn_norm=gain(h), ffn_norm=gain(h),
                   q_norm=gain(c["head_dim"]), k_norm=gain(c["head_dim"]))
              for _ in range(c["n_layers"])]
    return rng.normal(0, 1.0, (c["vocab"], h)).astype(np.float32), layers, gain(h)


def _quantized_view(embed, layers, final_norm):
    W = dict(embed=embed, final_norm=final_norm.astype(np.float64),
             lm_head=quant_weights(embed), layers=[])
    for L in layers:
        d = {k: quant_weights(L[k]) for k in ("q", "k", "v", "o", "gate", "up", "down")}
        d.update({k: L[k].astype(np.float64) for k in ("attn_norm", "ffn_norm", "q_norm", "k_norm")})
        W["layers"].append(d)
    return W


@pytest.fixture(scope="module")
def qwen3():
    embed, layers, fnorm = _qwen3_weights()
    m = O.QuantizedCausalLM(QCFG)
    m.set_weights(embed, layers, final_norm=fnorm, qk_norm=True)
    return m, _quantized_view(embed, layers, fnorm)


QWEN3_TOL = 1e-4  # int8 activation rounding is decided in f64 here, in f32 there


def test_qwen3_w8a8_oracle_matches_float64_forward(qwen3):
    m, W = qwen3
    ids = [3, 77, 190, 5, 42, 250, 9]
    m.reset()
    got = m.prefill(ids)
    cos, rel = cmp(got, decoder_ref(QCFG, W, ids, True, True))
    assert cos > 0.99999 and rel < QWEN3_TOL, (cos, rel)
    # cached decode steps (forward_one) against the stateless forward of the prefix
    seq = list(ids)
    for _ in range(4):
        t = int(np.argmax(got))
        seq.append(t)
        got = m.forward_one(t)
        cos, rel = cmp(got, decoder_ref(QCFG, W, seq, True, True))
        assert cos > 0.99999 and rel < QWEN3_TOL, (len(seq), cos, rel)


@pytest.mark.parametrize("mistake", ["no_attn_residual", "no_ffn_residual", "swap_gate_up"])
def test_qwen3_comparison_catches_wiring_mistakes(qwen3, mistake):
    m, W = qwen3
    ids = [3, 77, 190, 5, 42, 250, 9]
    m.reset()
    got = m.prefill(ids)
    cos, rel = cmp(got, decoder_ref(QCFG, W, ids, True, True, mutate=(mistake,)))
    assert cos < 0.999 or rel > 20 * QWEN3_TOL, (mistake, cos, rel)


# ---------------------------------------------------------------- f32 CausalLM (Q8_0)
FCFG = dict(hidden=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, inter=96,
            vocab=192, max_seq=32, eps=1e-5, rope_theta=5e5)


def q8_0_blocks(w):
    """GGUF Q8_0 blocks of a row-major [n, k] tensor: [d f16][32 x i8] per 32
    elements; returns (bytes, the values gguf.rs:255-288 decodes: f16(d) * q)"""
    w = np.asarray(w, np.float32).reshape(-1, 32)
    amax = np.abs(w).max(axis=1)
    d16 = (amax / 127.0).astype(np.float16)
    d = d16.astype(np.float32)
    q = np.zeros_like(w)
    nz = d > 0
    q[nz] = np.clip(np.rint(w[nz] / d[nz, None]), -127, 127)
    out = np.zeros((w.shape[0], 34), np.uint8)
    out[:, :2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1), (d[:, None].astype(np.float64) * q)


@pytest.fixture(scope="module")
def flm():
    rng = np.random.default_rng(23)
    c = FCFG
    h, qd, kvd, it = c["hidden"], c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"], c["inter"]
    f = lambda *s: rng.normal(0, WSTD, s).astype(np.float32)
    gain = lambda n: (1.0 + 0.1 * rng.normal(size=n)).astype(np.float32)
    m = O.CausalLM(c, qk_norm=False)
    embed = rng.normal(0, 1.0, (c["vocab"], h)).astype(np.float32)
    m.set_embed(embed)
    W = dict(embed=embed, layers=[])
    shapes = [(qd, h), (kvd, h), (kvd, h), (h, qd), (it, h), (it, h), (h, it)]
    names = ("q", "k", "v", "o", "gate", "up", "down")
    for l in range(c["n_layers"]):
        L = {}
        for p, (name, shp) in enumerate(zip(names, shapes)):
            blocks, vals = q8_0_blocks(f(*shp))
            m.set_proj(l, p, "q8_0", blocks)
            L[name] = vals.reshape(shp)
        L["attn_norm"], L["ffn_norm"] = gain(h), gain(h)
        m.set_norms(l, attn=L["attn_norm"], ffn=L["ffn_norm"])
        L["attn_norm"] = L["attn_norm"].astype(np.float64)
        L["ffn_norm"] = L["ffn_norm"].astype(np.float64)
        W["layers"].append(L)
    blocks, vals = q8_0_blocks(f(c["vocab"], h))
    m.set_lm_head("q8_0", blocks)
    W["lm_head"] = vals.reshape(c["vocab"], h)
    fn = gain(h)
    m.set_final_norm(fn)
    W["final_norm"] = fn.astype(np.float64)
    return m, W


FLM_TOL = 1e-4  # f32 chains against float64


def test_f32_causal_lm_oracle_matches_float64_forward(flm):
    m, W = flm
    ids = [1, 150, 33, 8, 91]
    m.reset()
    got = m.prefill(ids)
    cos, rel = cmp(got, decoder_ref(FCFG, W, ids, False, False))
    assert cos > 0.9999999 and rel < FLM_TOL, (cos, rel)
    seq = list(ids)
    for _ in range(3):
        t = int(np.argmax(got))
        seq.append(t)
        got = m.forward_one(t)
        cos, rel = cmp(got, decoder_ref(FCFG, W, seq, False, False))
        assert cos > 0.9999999 and rel < FLM_TOL, (len(seq), cos, rel)


@pytest.mark.parametrize("mistake", ["no_attn_residual", "no_ffn_residual", "swap_gate_up"])
def test_f32_causal_lm_comparison_catches_wiring_mistakes(flm, mistake):
    m, W = flm
    ids = [1, 150, 33, 8, 91]
    m.reset()
    cos, rel = cmp(m.prefill(ids), decoder_ref(FCFG, W, ids, False, False, mutate=(mistake,)))
    assert cos < 0.9999 or rel > 100 * FLM_TOL, (mistake, cos, rel)


# ---------------------------------------------------------------- INT8 Mamba
MCFG = dict(d_model=64, d_inner=128, d_state=16, d_conv=4, dt_rank=8, n_layers=2, vocab=200,
            eps=1e-5)
MSEED = 0x5EED0000


def mamba_weights(c, seed_base, std):
    """the synthetic weights of orc_mamba_init_synthetic (seed spec: embedding
    at seed_base (std 0.02), layer l at seed_base + 1 + 16 l (std `std`):
    in_proj +0, conv1d +1, x_proj +2, dt_proj +3, out_proj +4; conv bias 0,
    dt bias log(expm1(0.01)), a_log[i, s] = log(s + 1), D = 1, norm gains 1;
    lm_head = the embedding)"""
    dm, di, ds, dc, dr = c["d_model"], c["d_inner"], c["d_state"], c["d_conv"], c["dt_rank"]
    W = dict(embed=O.normal(c["vocab"] * dm, seed_base, 0.02).reshape(c["vocab"], dm), layers=[])
    for l in range(c["n_layers"]):
        sb = seed_base + 1 + 16 * l
        W["layers"].append(dict(
            in_proj=quant_weights(O.normal(2 * di * dm, sb + 0, std).reshape(2 * di, dm)),
            conv_w=O.normal(di * dc, sb + 1, std).reshape(di, dc).astype(np.float64),
            x_proj=O.normal((dr + 2 * ds) * di, sb + 2, std).reshape(dr + 2 * ds, di).astype(np.float64),
            dt_proj=O.normal(di * dr, sb + 3, std).reshape(di, dr).astype(np.float64),
            x_i8=quant_weights(O.normal((dr + 2 * ds) * di, sb + 2, std).reshape(dr + 2 * ds, di)),
            dt_i8=quant_weights(O.normal(di * dr, sb + 3, std).reshape(di, dr)),
            out_proj=quant_weights(O.normal(dm * di, sb + 4, std).reshape(dm, di)),
            dt_bias=np.full(di, np.log(np.expm1(0.01))),
            a_log=np.tile(np.log(np.arange(1, ds + 1, dtype=np.float64)), (di, 1))))
    return W


def softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def mamba_ref(c, W, ids, mutate=(), int8_xdt=False):
    """QuantizedMambaModel prefill (int8_mamba.rs:177-203): per token, per block
    forward_one (:78-109), then the final norm and the f32 lm_head.  With
    int8_xdt, x_proj and dt_proj are QuantizedLinears like in_proj (the
    benchmark's config-5 variant; int8_linear.rs:35-117)"""
    di, ds, dc, dr, eps = c["d_inner"], c["d_state"], c["d_conv"], c["dt_rank"], c["eps"]
    conv = [np.zeros((di, dc)) for _ in W["layers"]]
    ssm = [np.zeros((di, ds)) for _ in W["layers"]]
    for tok in ids:
        x = W["embed"][tok].astype(np.float64)
        for l, L in enumerate(W["layers"]):
            n = rmsnorm(x, np.ones(c["d_model"]), eps)
            proj = qlinear(n, L["in_proj"])[0]
            xp, z = proj[:di], proj[di:]
            conv[l] = np.concatenate([conv[l][:, 1:], xp[:, None]], axis=1)  # shift, append
            taps = L["conv_w"][:, ::-1] if "reverse_conv_taps" in mutate else L["conv_w"]
            xa = silu((conv[l] * taps).sum(axis=1))  # conv bias 0
            if int8_xdt:
                xpo = qlinear(xa, L["x_i8"])[0]
                dt, B, C = xpo[:dr], xpo[dr:dr + ds], xpo[dr + ds:]
                if "dt_from_b" in mutate:
                    dt = xpo[ds:dr + ds]
                dtp = qlinear(dt, L["dt_i8"])[0]
            else:
                xpo = L["x_proj"] @ xa
                dt, B, C = xpo[:dr], xpo[dr:dr + ds], xpo[dr + ds:]
                dtp = L["dt_proj"] @ dt
            delta = softplus(dtp + L["dt_bias"])
            a_disc = np.exp(-delta[:, None] * np.exp(L["a_log"]))
            ssm[l] = a_disc * ssm[l] + (delta * xa)[:, None] * B[None, :]
            y = ssm[l] @ C + 1.0 * xa
            gated = z * silu(y) if "gate_silu_on_y" in mutate else silu(z) * y
            o = qlinear(gated, L["out_proj"])[0]
            x = o if "no_residual" in mutate else x + o
    xf = rmsnorm(x, np.ones(c["d_model"]), eps)[0]
    return W["embed"].astype(np.float64) @ xf


MAMBA_TOL = 1e-4
MSTD = 0.3  # projections and conv taps (see WSTD)


@pytest.fixture(scope="module")
def mamba():
    m = O.QuantizedMamba(MCFG)
    m.init_synthetic(MSEED, MSTD)
    return m, mamba_weights(MCFG, MSEED, MSTD)


def test_mamba_oracle_matches_float64_forward(mamba):
    m, W = mamba
    ids = [5, 199, 64, 3, 120, 77]
    cos, rel = cmp(m.prefill(ids), mamba_ref(MCFG, W, ids))
    assert cos > 0.99999 and rel < MAMBA_TOL, (cos, rel)


@pytest.mark.parametrize("mistake", ["reverse_conv_taps", "no_residual", "gate_silu_on_y"])
def test_mamba_comparison_catches_wiring_mistakes(mamba, mistake):
    m, W = mamba
    ids = [5, 199, 64, 3, 120, 77]
    cos, rel = cmp(m.prefill(ids), mamba_ref(MCFG, W, ids, mutate=(mistake,)))
    assert cos < 0.999 or rel > 20 * MAMBA_TOL, (mistake, cos, rel)


@pytest.fixture(scope="module")
def mamba_xdt():
    m = O.QuantizedMamba(MCFG)
    m.init_synthetic(MSEED, MSTD)
    m.set_int8_xdt()
    return m, mamba_weights(MCFG, MSEED, MSTD)


def test_mamba_int8_xdt_oracle_matches_float64_forward(mamba_xdt):
    """the config-5 variant (x_proj and dt_proj through QuantizedLinear) against
    the float64 forward with qlinear on those two projections; the f32 form
    of the same forward does not pass, so the variant is really taken"""
    m, W = mamba_xdt
    ids = [5, 199, 64, 3, 120, 77]
    got = m.prefill(ids)
    cos, rel = cmp(got, mamba_ref(MCFG, W, ids, int8_xdt=True))
    assert cos > 0.99999 and rel < MAMBA_TOL, (cos, rel)
    cos_f, rel_f = cmp(got, mamba_ref(MCFG, W, ids))
    assert rel_f > 20 * MAMBA_TOL, (cos_f, rel_f)


@pytest.mark.parametrize("mistake", ["reverse_conv_taps", "no_residual", "dt_from_b"])
def test_mamba_int8_xdt_comparison_catches_wiring_mistakes(mamba_xdt, mistake):
    m, W = mamba_xdt
    ids = [5, 199, 64, 3, 120, 77]
    cos, rel = cmp(m.prefill(ids), mamba_ref(MCFG, W, ids, mutate=(mistake,), int8_xdt=True))
    assert cos < 0.999 or rel > 20 * MAMBA_TOL, (mistake, cos, rel)


# ---------------------------------------------------------------- pieces
def test_conv1d_step_impulse_response():
    """int8_mamba.rs:43-56: the window shifts left and the new sample enters
    at the end, so an impulse comes out through the taps last to first"""
    w = np.array([[1, 10, 100, 1000], [2, 20, 200, 2000]], np.float32)
    b = np.array([0.5, -0.25], np.float32)
    st = np.zeros((2, 4), np.float32)
    outs = [O.conv1d_step(np.array([1.0 if t == 0 else 0.0, 0.0], np.float32), w, b, st)
            for t in range(5)]
    np.testing.assert_array_equal([o[0] for o in outs], [1000.5, 100.5, 10.5, 1.5, 0.5])
    np.testing.assert_array_equal([o[1] for o in outs], [-0.25] * 5)
    # a ramp: out_t = sum_k window[k] * w[k] with window = last four samples
    st[:] = 0
    xs = [3.0, -1.0, 2.0, 5.0, 7.0]
    for t, v in enumerate(xs):
        o = O.conv1d_step(np.array([0.0, v], np.float32), w, b, st)
        win = ([0.0] * 4 + xs[:t + 1])[-4:]
        assert o[1] == np.float32(np.dot(win, w[1]) + b[1])


def test_swiglu_fused_is_silu_gate_times_up():
    rng = np.random.default_rng(5)
    for n in (1, 3, 4, 37, 1000):
        g = rng.normal(0, 3, n).astype(np.float32)
        u = rng.normal(0, 1, n).astype(np.float32)
        got = O.swiglu_fused(g, u).astype(np.float64)
        want = silu(g.astype(np.float64)) * u
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)
