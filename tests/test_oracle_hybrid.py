"""CPU pins of the hybrid LFM2.5 oracle (models/ssm/hybrid, Q4 decode path).

- the LIV conv step against an impulse known-answer test (shift direction,
  tap order, the B / C / x split of the in_proj output, bias, gating);
- the whole decoder against an independent numpy float64 forward of the
  same synthetic model (dequantized Q4 weights), which fails if a residual
  add, a gate, a norm or a layer kind is miswired.
"""
import numpy as np
import pytest

import oracle as O

TINY = dict(hidden=64, n_layers=4, vocab=128, n_heads=4, n_kv_heads=2, head_dim=16, inner=64,
            conv_kernel=4, inter=128, max_seq=32, eps=1e-6, rope_theta=1e4,
            layer_kinds=[0, 1, 0, 1])


def test_conv_step_impulse_reproduces_the_taps_in_order():
    inner, ck = 2, 3
    w = np.array([[1, 2, 3], [4, 5, 6]], np.float32)  # [channel][tap], tap ck-1 = newest
    bias = np.array([0.5, 0.0], np.float32)
    state = np.zeros(inner * ck, np.float32)

    def step(b, c, x):
        proj = np.array([*b, *c, *x], np.float32)  # [B | C | x]
        return O.hlm_conv_step(proj, inner, ck, state, w, bias)

    # impulse B*x = 1 at t = 0: the newest tap first, then older ones, then bias only
    np.testing.assert_array_equal(step([1, 1], [1, 1], [1, 1]), [3.5, 6.0])
    np.testing.assert_array_equal(step([1, 1], [1, 1], [0, 0]), [2.5, 5.0])
    np.testing.assert_array_equal(step([1, 1], [1, 1], [0, 0]), [1.5, 4.0])
    np.testing.assert_array_equal(step([1, 1], [1, 1], [0, 0]), [0.5, 0.0])
    # the conv input is B * x (pre-gate) and the output C * conv (post-gate)
    np.testing.assert_array_equal(step([3, 1], [2, 1], [2, 0]), [2 * (6 * 3 + 0.5), 0.0])
    np.testing.assert_array_equal(state.reshape(inner, ck), [[0, 0, 6], [0, 0, 0]])


def _dequant_q4(packed, n, k):
    """pack_for_zig bytes -> f64 weights: per 32-block an IEEE f16 scale and
    16 bytes, element 2i the low nibble of byte i, 2i+1 the high; (q - 8) * d."""
    blk = packed.reshape(n, k // 32, 18)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    b = blk[:, :, 2:].astype(np.int64)
    q = np.empty((n, k // 32, 32), np.int64)
    q[:, :, 0::2] = b & 15
    q[:, :, 1::2] = b >> 4
    return ((q - 8) * d[:, :, None]).reshape(n, k)


def _q4(n, k, seed, std):
    return _dequant_q4(O.q4_pack(O.normal(n * k, seed, std).reshape(n, k)), n, k)


def _gain(n, seed):
    return 1.0 + O.normal(n, seed, 0.1).astype(np.float64)


def _rms(x, g, eps):
    return x * g / np.sqrt(np.mean(x * x) + eps)


def _silu(x):
    return x / (1.0 + np.exp(-x))


class NumpyHybrid:
    """float64 restatement of layer.rs LivConv / GQA forward_one and model.rs
    decode_one, weights rebuilt from the synthetic-weight spec."""

    def __init__(self, c, seed, std):
        self.c = c
        H, I, F, hd = c["hidden"], c["inner"], c["inter"], c["head_dim"]
        qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd
        self.embed = O.normal(c["vocab"] * H, seed, std).astype(np.float64).reshape(-1, H)
        self.L = []
        for l, kind in enumerate(c["layer_kinds"]):
            s = seed + 1 + 16 * l
            d = dict(kind=kind, attn=_gain(H, s + 8), ffn=_gain(H, s + 9),
                     gate=_q4(F, H, s + 10, std), up=_q4(F, H, s + 11, std),
                     down=_q4(H, F, s + 12, std))
            if kind == 0:
                d.update(w_in=_q4(3 * I, H, s, std),
                         conv=O.normal(I * c["conv_kernel"], s + 1, std).astype(np.float64)
                         .reshape(I, c["conv_kernel"]),
                         w_out=_q4(H, I, s + 2, std),
                         state=np.zeros((I, c["conv_kernel"])))
            else:
                d.update(wq=_q4(qd, H, s, std), wk=_q4(kvd, H, s + 1, std),
                         wv=_q4(kvd, H, s + 2, std), wo=_q4(H, qd, s + 3, std),
                         qn=_gain(hd, s + 6), kn=_gain(hd, s + 7), K=[], V=[])
            self.L.append(d)
        self.final = _gain(H, seed + 1 + 16 * len(c["layer_kinds"]))
        half = hd // 2
        i = np.arange(half, dtype=np.float32)
        self.freq = (1.0 / np.float32(c["rope_theta"]) ** (2.0 * i / np.float32(hd))).astype(
            np.float64)
        self.pos = 0

    def _ffn(self, d, x):
        n = _rms(x, d["ffn"], self.c["eps"])
        return d["down"] @ (_silu(d["gate"] @ n) * (d["up"] @ n))

    def _rope(self, v):
        half = v.shape[-1] // 2
        ang = self.pos * self.freq
        c, s = np.cos(ang), np.sin(ang)
        a, b = v[..., :half], v[..., half:]
        return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)

    def decode_one(self, token):
        c, eps = self.c, self.c["eps"]
        I, hd, nq, nkv = c["inner"], c["head_dim"], c["n_heads"], c["n_kv_heads"]
        x = self.embed[token].copy()
        for d in self.L:
            n = _rms(x, d["attn"], eps)
            if d["kind"] == 0:
                p = d["w_in"] @ n
                B, C_, X = p[:I], p[I:2 * I], p[2 * I:]
                d["state"] = np.concatenate([d["state"][:, 1:], (B * X)[:, None]], axis=1)
                o = d["w_out"] @ (C_ * np.sum(d["state"] * d["conv"], axis=1))
            else:
                q = (d["wq"] @ n).reshape(nq, hd)
                k = (d["wk"] @ n).reshape(nkv, hd)
                v = (d["wv"] @ n).reshape(nkv, hd)
                q = q * d["qn"] / np.sqrt(np.mean(q * q, axis=1, keepdims=True) + eps)
                k = k * d["kn"] / np.sqrt(np.mean(k * k, axis=1, keepdims=True) + eps)
                d["K"].append(self._rope(k))
                d["V"].append(v)
                K, V = np.stack(d["K"]), np.stack(d["V"])  # [seq][kv][hd]
                q = self._rope(q)
                out = np.empty((nq, hd))
                for h in range(nq):
                    g = h // (nq // nkv)
                    s = K[:, g, :] @ q[h] / np.sqrt(hd)
                    e = np.exp(s - s.max())
                    out[h] = (e / e.sum()) @ V[:, g, :]
                o = d["wo"] @ out.reshape(-1)
            x = x + o
            x = x + self._ffn(d, x)
        self.pos += 1
        return self.embed @ _rms(x, self.final, eps)


@pytest.mark.parametrize("kinds", [[0, 1, 0, 1], [1, 0, 0, 1]])
def test_hybrid_oracle_matches_numpy_float64_forward(kinds):
    cfg = dict(TINY, layer_kinds=kinds)
    seed, std = 0x5EED0000, 0.08
    m = O.HybridLM(cfg)
    m.init_synthetic(seed, std)
    ref = NumpyHybrid(cfg, seed, std)
    for t, tok in enumerate([3, 77, 12, 12, 100, 5, 64, 2]):
        got = m.decode_one(tok)
        want = ref.decode_one(tok)
        rel = np.abs(got - want).max() / np.abs(want).max()
        assert rel < 2e-5, (t, rel)
    assert m.pos == 8


def test_hybrid_oracle_conv_bias_and_reset():
    cfg = dict(TINY, conv_bias=1)
    a, b = O.HybridLM(cfg), O.HybridLM(cfg)
    a.init_synthetic(7, 0.05)
    b.init_synthetic(7, 0.05)
    first = a.decode_one(9)
    a.decode_one(4)
    a.reset()
    np.testing.assert_array_equal(a.decode_one(9), first)
    np.testing.assert_array_equal(b.decode_one(9), first)
    nb = O.HybridLM(TINY)
    nb.init_synthetic(7, 0.05)
    assert not np.array_equal(nb.decode_one(9), first)  # the bias is used
