"""GGUF reader (host code, no GPU): the reference's own GGUF tests
(weight_loading/gguf.rs:680-830) with their golden values, plus the reader's
bounds checks on malformed files.  The reader hands back stored bytes; the
values the reference's parse_gguf returns are recovered with the oracle's
dequantizers, so these tests also pin those against the reference's goldens."""
import struct

import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests import gguf_writer as W


def _open(tmp_path, blob, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    return hip.Gguf(p)


def _f32(t):
    return np.frombuffer(t.bytes().tobytes(), np.float32)


def test_two_f32_tensors_bit_exact(tmp_path):
    # gguf.rs:680-698
    a = np.array([1, 2, 3, 4, 5, 6], np.float32)
    b = np.array([7, 8, 9, 10], np.float32)
    blob = W.gguf_bytes([("tensor_a", W.F32, [2, 3], a.tobytes()),
                         ("tensor_b", W.F32, [4], b.tobytes())])
    with _open(tmp_path, blob) as g:
        assert len(g) == 2
        ta, tb = g.info(g.index("tensor_a")), g.info(g.index("tensor_b"))
        assert ta.dims == (2, 3) and tb.dims == (4,)
        assert ta.ggml_type == W.F32 and ta.nbytes == 24
        np.testing.assert_array_equal(_f32(ta), a)
        np.testing.assert_array_equal(_f32(tb), b)
        assert g.index("tensor_c") is None


def test_q8_0_tensor_golden(tmp_path):
    # gguf.rs:700-721: scale 0.5 (f16 0x3800), quants 1..32 -> 0.5 * q
    quants = np.arange(1, 33, dtype=np.int8)
    block = struct.pack("<H", 0x3800) + quants.tobytes()
    with _open(tmp_path, W.gguf_bytes([("q8_tensor", W.Q8_0, [32], block)])) as g:
        t = g.info(0)
        assert t.dims == (32,) and t.nbytes == 34
        got = O.dequant("q8_0", t.bytes(), 32)
    np.testing.assert_allclose(got, 0.5 * quants.astype(np.float32), atol=1e-4)


def test_q4_0_tensor_golden(tmp_path):
    # gguf.rs:789-820: delta 1.0, bytes 0x10 -> pairs (-8, -7)
    block = struct.pack("<H", 0x3C00) + bytes([0x10] * 16)
    with _open(tmp_path, W.gguf_bytes([("q4_tensor", W.Q4_0, [32], block)])) as g:
        t = g.info(0)
        assert t.nbytes == 18
        got = O.dequant("q4_0", t.bytes(), 32)
    np.testing.assert_allclose(got[0::2], -8.0, atol=1e-3)
    np.testing.assert_allclose(got[1::2], -7.0, atol=1e-3)


def test_bad_magic(tmp_path):
    # gguf.rs:723-730
    blob = struct.pack("<I", 0xDEADBEEF) + bytes(28)
    with pytest.raises(hip.SynapseError):
        _open(tmp_path, blob)


def test_metadata_skipped_and_readable(tmp_path):
    # gguf.rs:732-765, with every value type and nested arrays added
    meta = [("general.name", W.STRING, "test"),
            ("llama.block_count", W.U32, 2),
            ("llama.context_length", W.U64, 4096),
            ("x.i8", W.I8, -3), ("x.i16", W.I16, -300), ("x.u16", W.U16, 60000),
            ("x.i32", W.I32, -70000), ("x.i64", W.I64, -(1 << 40)), ("x.bool", W.BOOL, 1),
            ("llama.rope.freq_base", W.F32V, 500000.0),
            ("llama.attention.layer_norm_rms_epsilon", W.F32V, 1e-5),
            ("x.f64", W.F64, 0.125),
            ("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, ["<s>", "</s>", "hello"])),
            ("tokenizer.ggml.scores", W.ARRAY, (W.F32V, [0.0, -1.0, -2.5])),
            ("x.nested", W.ARRAY, (W.ARRAY, [(W.U8, [1, 2]), (W.STRING, ["a"])]))]
    data = np.array([42.0, 43.0], np.float32)
    blob = W.gguf_bytes([("w", W.F32, [2], data.tobytes())], meta)
    with _open(tmp_path, blob) as g:
        assert len(g) == 1
        np.testing.assert_array_equal(_f32(g.info(0)), data)
        assert g.meta_str("general.name") == "test"
        assert g.meta_u64("llama.block_count") == 2
        assert g.meta_u64("llama.context_length") == 4096
        assert g.meta_u64("x.u16") == 60000
        assert np.uint64(g.meta_u64("x.i64")).view(np.int64) == -(1 << 40)
        assert np.uint64(g.meta_u64("x.i8")).view(np.int64) == -3
        assert g.meta_f64("llama.rope.freq_base") == 500000.0
        assert g.meta_f64("llama.attention.layer_norm_rms_epsilon") == np.float32(1e-5)
        assert g.meta_f64("x.f64") == 0.125
        # wrong kinds and absent keys are reported, not converted
        assert g.meta_u64("general.name") is None
        assert g.meta_str("llama.block_count") is None
        assert g.meta_u64("tokenizer.ggml.tokens") is None
        assert g.meta_f64("nope") is None


def test_unsupported_type(tmp_path):
    # gguf.rs:822-829
    with pytest.raises(hip.SynapseError, match="unsupported GGML type 99"):
        _open(tmp_path, W.gguf_bytes([("bad", 99, [32], bytes(64))]))


@pytest.mark.parametrize("version", [1, 4])
def test_unsupported_version(tmp_path, version):
    blob = W.gguf_bytes([("w", W.F32, [2], bytes(8))], version=version)
    with pytest.raises(hip.SynapseError, match="version"):
        _open(tmp_path, blob)


def test_version_2_reads(tmp_path):
    data = np.arange(8, dtype=np.float32)
    with _open(tmp_path, W.gguf_bytes([("w", W.F32, [8], data.tobytes())], version=2)) as g:
        np.testing.assert_array_equal(_f32(g.info(0)), data)


def test_partial_blocks_rejected(tmp_path):
    with pytest.raises(hip.SynapseError, match="whole blocks"):
        _open(tmp_path, W.gguf_bytes([("w", W.Q4_K, [128], bytes(72))]))


@pytest.mark.parametrize("cut", [10, 23, 40, 60])
def test_truncated_header(tmp_path, cut):
    blob = W.gguf_bytes([("tensor_a", W.F32, [4], bytes(16))],
                        [("general.name", W.STRING, "test")])
    with pytest.raises(hip.SynapseError):
        _open(tmp_path, blob[:cut])


def test_tensor_past_end_of_file(tmp_path):
    blob = W.gguf_bytes([("w", W.F32, [64], bytes(256))])
    with pytest.raises(hip.SynapseError, match="outside the file"):
        _open(tmp_path, blob[:-4])


def test_huge_counts_rejected(tmp_path):
    blob = struct.pack("<IIQQ", W.GGUF_MAGIC, 3, 1 << 60, 0) + bytes(64)
    with pytest.raises(hip.SynapseError, match="header"):
        _open(tmp_path, blob)


def test_huge_string_length_rejected(tmp_path):
    blob = struct.pack("<IIQQ", W.GGUF_MAGIC, 3, 0, 1) + struct.pack("<Q", 1 << 62) + bytes(40)
    with pytest.raises(hip.SynapseError, match="metadata"):
        _open(tmp_path, blob)


def test_missing_file(tmp_path):
    with pytest.raises(hip.SynapseError, match="cannot open"):
        hip.Gguf(tmp_path / "absent.gguf")


def test_alignment_key(tmp_path):
    # llama.cpp's general.alignment: data starts at the next multiple of it
    a = np.arange(3, dtype=np.float32)
    b = np.arange(5, dtype=np.float32) + 10
    blob = W.gguf_bytes([("a", W.F32, [3], a.tobytes()), ("b", W.F32, [5], b.tobytes())],
                        [("general.alignment", W.U32, 256)], alignment=256)
    with _open(tmp_path, blob) as g:
        np.testing.assert_array_equal(_f32(g.info(g.index("a"))), a)
        np.testing.assert_array_equal(_f32(g.info(g.index("b"))), b)
    bad = W.gguf_bytes([("a", W.F32, [3], a.tobytes())], [("general.alignment", W.U32, 48)])
    with pytest.raises(hip.SynapseError, match="power of two"):
        _open(tmp_path, bad, "bad.gguf")


@pytest.mark.parametrize("fmt,ggml", [(hip.FMT_Q8_0, W.Q8_0), (hip.FMT_Q4_K, W.Q4_K),
                                      (hip.FMT_Q6_K, W.Q6_K)])
def test_block_tensor_bytes_round_trip(tmp_path, fmt, ggml):
    # a [N, K] weight is stored with dims {K, N}; its blocks come back as written
    n, k = 6, 512
    w = O.normal(n * k, 0x5EED0000 + ggml, 0.02).reshape(n, k)
    blocks = hip.kquant_encode(fmt, w)
    blob = W.gguf_bytes([("blk.0.attn_q.weight", ggml, [k, n], blocks.tobytes()),
                         ("token_embd.weight", W.F16, [k, n],
                          w.astype(np.float16).tobytes())])
    with _open(tmp_path, blob) as g:
        t = g.info(g.index("blk.0.attn_q.weight"))
        assert t.ggml_type == ggml and t.dims == (k, n) and t.nbytes == blocks.size
        np.testing.assert_array_equal(t.bytes(), blocks)
        e = g.info(g.index("token_embd.weight"))
        assert e.ggml_type == W.F16 and e.nbytes == n * k * 2


@pytest.mark.parametrize("fmt,name", [(hip.FMT_Q8_0, "q8_0"), (hip.FMT_Q4_K, "q4_k"),
                                      (hip.FMT_Q6_K, "q6_k")])
def test_library_host_dequant_matches_oracle(fmt, name):
    # the loader's host dequantizer (embeddings stored in block formats) gives
    # the oracle's values bit for bit, on encoded weights and on random bytes
    # with finite f16 scales
    be, bb = hip.KQ_BLOCK[fmt]
    w = O.normal(4 * 1024, 0x5EED2000 + fmt, 0.05).reshape(4, 1024)
    enc = hip.kquant_encode(fmt, w)
    np.testing.assert_array_equal(hip.kquant_decode(fmt, enc), O.dequant(name, enc, w.size))
    rng = np.random.default_rng(fmt)
    raw = rng.integers(0, 256, 64 * bb, dtype=np.uint8).reshape(64, bb)
    scale_words = {hip.FMT_Q8_0: [0], hip.FMT_Q4_K: [0, 1], hip.FMT_Q6_K: [104]}[fmt]
    for wd in scale_words:  # keep the f16 scales finite (exponent field below 31)
        raw[:, 2 * wd + 1] &= 0x7B
    raw = raw.reshape(-1)
    np.testing.assert_array_equal(hip.kquant_decode(fmt, raw), O.dequant(name, raw, 64 * be))
