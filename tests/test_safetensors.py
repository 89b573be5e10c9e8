"""safetensors reader and the f32 conversions of both containers (host code,
no GPU): the reference's own safetensors tests (safetensors.rs:351-599) with
their golden values, the Q4_0 triple of expand_q4_tensors as pack_for_zig
bytes, and the reader's checks on malformed headers."""
import struct

import numpy as np
import pytest

import oracle as O
from synapse_amd import hip
from tests import gguf_writer as G
from tests import safetensors_writer as S


def _open(tmp_path, blob, name="m.safetensors"):
    p = tmp_path / name
    p.write_bytes(blob)
    return hip.Safetensors(p)


def _f32(x):
    return np.array(x, np.float32)


def test_two_f32_tensors_bit_exact(tmp_path):
    # safetensors.rs:351-374
    a, b = _f32([1, 2, 3, 4, 5, 6]), _f32([7, 8, 9, 10])
    with _open(tmp_path, S.st_bytes([("weight_a", "F32", [2, 3], a.tobytes()),
                                     ("weight_b", "F32", [4], b.tobytes())])) as st:
        assert len(st) == 2
        ia, ib = st.index("weight_a"), st.index("weight_b")
        assert st.info(ia).dims == (2, 3) and st.info(ib).dims == (4,)
        np.testing.assert_array_equal(st.to_f32(ia).ravel(), a)
        np.testing.assert_array_equal(st.to_f32(ib), b)


def test_f16_golden(tmp_path):
    # safetensors.rs:376-388
    raw = np.array([0x3C00, 0x4000, 0x3800], np.uint16).tobytes()
    with _open(tmp_path, S.st_bytes([("w", "F16", [3], raw)])) as st:
        assert st.info(0).dtype == "F16"
        np.testing.assert_array_equal(st.to_f32(0), _f32([1.0, 2.0, 0.5]))


def test_bf16_golden(tmp_path):
    # safetensors.rs:390-401
    raw = np.array([0x3F80, 0x4000, 0xBF80], np.uint16).tobytes()
    with _open(tmp_path, S.st_bytes([("w", "BF16", [3], raw)])) as st:
        np.testing.assert_array_equal(st.to_f32(0), _f32([1.0, 2.0, -1.0]))


def test_unsupported_dtype(tmp_path):
    # safetensors.rs:403-415
    h = b'{"t":{"dtype":"INT4","shape":[2],"data_offsets":[0,1]}}'
    with pytest.raises(hip.SynapseError, match="unsupported dtype INT4"):
        _open(tmp_path, struct.pack("<Q", len(h)) + h + b"\0")


def test_truncated_file(tmp_path):
    # safetensors.rs:417-422
    with pytest.raises(hip.SynapseError, match="too small"):
        _open(tmp_path, bytes(4))


def test_metadata_skipped_and_readable(tmp_path):
    # safetensors.rs:424-441
    blob = S.st_bytes([("w", "F32", [1], _f32([1.0]).tobytes())], metadata={"format": "pt"})
    with _open(tmp_path, blob) as st:
        assert len(st) == 1 and st.names() == ["w"]
        assert st.meta("format") == "pt"
        assert st.meta("absent") is None


def test_f32_values_identical(tmp_path):
    # safetensors.rs:470-486
    x = np.arange(1024, dtype=np.float32) * np.float32(0.001) - np.float32(0.5)
    with _open(tmp_path, S.st_bytes([("w", x)])) as st:
        np.testing.assert_array_equal(st.to_f32(0), x)


def test_integer_dtypes_cast(tmp_path):
    # safetensors.rs:256-289: I64, I32 and U8 cast to f32
    i64 = np.array([0, -3, 51416, 1 << 30], np.int64)
    i32 = np.array([7, -7, 123456], np.int32)
    u8 = np.array([0, 1, 128, 255], np.uint8)
    with _open(tmp_path, S.st_bytes([("a", i64), ("b", i32), ("c", u8)])) as st:
        np.testing.assert_array_equal(st.to_f32(st.index("a")), i64.astype(np.float32))
        np.testing.assert_array_equal(st.to_f32(st.index("b")), i32.astype(np.float32))
        np.testing.assert_array_equal(st.to_f32(st.index("c")), u8.astype(np.float32))


def test_f16_all_bit_patterns_match_reference_converter(tmp_path):
    # converter.rs:12-40 (pinned in the oracle's tests), every f16 bit pattern
    bits = np.arange(65536, dtype=np.uint16)
    want = np.array([O.lib().orc_f16_to_f32_rs(int(b)) for b in bits], np.float32)
    with _open(tmp_path, S.st_bytes([("h", "F16", [65536], bits.tobytes())])) as st:
        got = st.to_f32(0)
    finite = np.isfinite(want)
    np.testing.assert_array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_json_escapes_and_unicode_names(tmp_path):
    name = "layer.é中\U0001F600\"q\\"
    blob = S.st_bytes([(name, _f32([3.0, 4.0])), ("x/y z", _f32([5.0]))],
                      metadata={"k": "v\n\t"})
    with _open(tmp_path, blob) as st:
        assert st.index(name) is not None
        np.testing.assert_array_equal(st.to_f32(st.index(name)), _f32([3.0, 4.0]))
        assert st.meta("k") == "v\n\t"
        assert st.index("x/y z") is not None


@pytest.mark.parametrize("header,msg", [
    (b'{"w":{"dtype":"F32","shape":[2],"data_offsets":[0,16]}}', "exceeds file bounds"),
    (b'{"w":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}', "holds 8 bytes"),
    (b'{"w":{"dtype":"F32","shape":[2],"data_offsets":[8,0]}}', "exceeds file bounds"),
    (b'{"w":{"dtype":"F32","shape":[2]}}', "data_offsets"),
    (b'{"w":{"shape":[2],"data_offsets":[0,8]}}', "dtype"),
    (b'{"w":{"dtype":"F32","shape":[-2],"data_offsets":[0,8]}}', "shape"),
    (b'{"w":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}', "invalid JSON"),
    (b'{"w":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}} x', "invalid JSON"),
    (b'["w"]', "invalid JSON"),
])
def test_malformed_headers(tmp_path, header, msg):
    with pytest.raises(hip.SynapseError, match=msg):
        _open(tmp_path, struct.pack("<Q", len(header)) + header + bytes(8))


def test_header_longer_than_file(tmp_path):
    with pytest.raises(hip.SynapseError, match="header size exceeds"):
        _open(tmp_path, struct.pack("<Q", 1 << 40) + b"{}")


def test_sharded_directory(tmp_path):
    # safetensors.rs:511-558: only the index's tensors, each from its shard
    w1, w2, w3 = _f32([1, 2, 3]), _f32([4, 5]), _f32([6, 7, 8, 9])
    S.write_st(tmp_path / "model-00001-of-00002.safetensors",
               [("tensor_a", w1), ("tensor_b", w2)])
    S.write_st(tmp_path / "model-00002-of-00002.safetensors",
               [("tensor_c", w3), ("extra_tensor", _f32([99]))])
    S.write_index(tmp_path, {"tensor_a": "model-00001-of-00002.safetensors",
                             "tensor_b": "model-00001-of-00002.safetensors",
                             "tensor_c": "model-00002-of-00002.safetensors"}, 100)
    with hip.Safetensors(tmp_path) as st:
        assert sorted(st.names()) == ["tensor_a", "tensor_b", "tensor_c"]
        np.testing.assert_array_equal(st.to_f32(st.index("tensor_a")), w1)
        np.testing.assert_array_equal(st.to_f32(st.index("tensor_b")), w2)
        np.testing.assert_array_equal(st.to_f32(st.index("tensor_c")), w3)
        assert st.info(st.index("tensor_c")).dims == (4,)
        assert st.index("extra_tensor") is None


def test_sharded_missing_shard(tmp_path):
    # safetensors.rs:560-578
    S.write_index(tmp_path, {"tensor_a": "missing-shard.safetensors"}, 100)
    with pytest.raises(hip.SynapseError, match="missing-shard"):
        hip.Safetensors(tmp_path)


def test_sharded_missing_tensor_in_shard(tmp_path):
    # safetensors.rs:580-599: the error names the tensor
    S.write_st(tmp_path / "shard.safetensors", [("actual_tensor", _f32([1.0]))])
    S.write_index(tmp_path, {"claimed_tensor": "shard.safetensors"})
    with pytest.raises(hip.SynapseError, match="claimed_tensor"):
        hip.Safetensors(tmp_path)


def test_directory_with_single_file(tmp_path):
    S.write_st(tmp_path / "model.safetensors", [("w", _f32([1.5]))])
    with hip.Safetensors(tmp_path) as st:
        np.testing.assert_array_equal(st.to_f32(0), _f32([1.5]))
    S.write_st(tmp_path / "other.safetensors", [("w", _f32([2.5]))])
    with pytest.raises(hip.SynapseError, match="2 .safetensors files"):
        hip.Safetensors(tmp_path)


def _q4_triple(packed, rows, bpr, cols):
    blocks = packed.reshape(rows, bpr, 18)
    scales = np.ascontiguousarray(blocks[:, :, :2]).view(np.uint16).reshape(rows, bpr)
    nib = np.ascontiguousarray(blocks[:, :, 2:])
    return [("m.w.q4_nibbles", "U8", [rows, bpr, 16], nib.tobytes()),
            ("m.w.q4_scales", "F16", [rows, bpr], scales.tobytes()),
            ("m.w.q4_orig_cols", "I64", [1], np.array([cols], np.int64).tobytes())]


@pytest.mark.parametrize("cols", [64, 50])
def test_q4_triple_is_pack_for_zig(tmp_path, cols):
    # expand_q4_tensors (safetensors.rs:94-170) decodes the triple exactly as
    # the Q4_0 blocks of pack_for_zig: the reader hands those bytes over
    rows = 3
    w = O.normal(rows * cols, 0x5EED4000, 0.1).reshape(rows, cols)
    packed = O.q4_pack(w)
    bpr = (cols + 31) // 32
    with _open(tmp_path, S.st_bytes(_q4_triple(packed, rows, bpr, cols))) as st:
        got, r, c = st.q4_pack("m.w")
        assert (r, c) == (rows, cols)
        np.testing.assert_array_equal(got, packed)


def test_q4_triple_errors(tmp_path):
    packed = O.q4_pack(O.normal(2 * 32, 1, 0.1).reshape(2, 32))
    t = _q4_triple(packed, 2, 1, 40)  # orig_cols > padded
    with _open(tmp_path, S.st_bytes(t)) as st:
        with pytest.raises(hip.SynapseError, match="padded_cols"):
            st.q4_pack("m.w")
        with pytest.raises(hip.SynapseError, match="q4_nibbles"):
            st.q4_pack("other")


# ------------------------------------------------------------------ GGUF to_f32
@pytest.mark.parametrize("fmt,name,ggml", [(hip.FMT_Q8_0, "q8_0", G.Q8_0),
                                           (hip.FMT_Q4_K, "q4_k", G.Q4_K),
                                           (hip.FMT_Q6_K, "q6_k", G.Q6_K)])
def test_gguf_to_f32_block_types(tmp_path, fmt, name, ggml):
    w = O.normal(4 * 512, 0x5EED5000 + ggml, 0.05).reshape(4, 512)
    b = hip.kquant_encode(fmt, w)
    p = G.write_gguf(tmp_path / "m.gguf", [("w", ggml, [512, 4], b.tobytes())])
    with hip.Gguf(p) as g:
        np.testing.assert_array_equal(g.to_f32(0), O.dequant(name, b, w.size))


def test_gguf_to_f32_q4_0_f16_bf16_q4_1(tmp_path):
    w = O.normal(2 * 64, 0x5EED6000, 0.1).reshape(2, 64)
    q4 = O.q4_pack(w)
    h = np.array([0x3C00, 0x0001, 0x8400, 0x7BFF], np.uint16)  # 1, subnormal, -2^-14, max
    bf = np.array([0x3F80, 0xC000, 0x0001], np.uint16)
    # Q4_1 by hand (gguf.rs:332-373): d = 1.0, m = 0.5, bytes 0x21 -> 1.5, 2.5
    q41 = struct.pack("<HH", 0x3C00, 0x3800) + bytes([0x21] * 16)
    p = G.write_gguf(tmp_path / "m.gguf", [("q4", G.Q4_0, [64, 2], q4.tobytes()),
                                           ("h", G.F16, [4], h.tobytes()),
                                           ("bf", 30, [3], bf.tobytes()),
                                           ("q41", G.Q4_1, [32], q41)])
    with hip.Gguf(p) as g:
        np.testing.assert_array_equal(g.to_f32(g.index("q4")), O.dequant("q4_0", q4, w.size))
        want_h = np.array([O.lib().orc_f16_to_f32_rs(int(b)) for b in h], np.float32)
        np.testing.assert_array_equal(g.to_f32(g.index("h")), want_h)
        np.testing.assert_array_equal(g.to_f32(g.index("bf")),
                                      _f32([1.0, -2.0, np.float32(2.0) ** -133]))
        got = g.to_f32(g.index("q41"))
        np.testing.assert_array_equal(got[0::2], np.full(16, 1.5, np.float32))
        np.testing.assert_array_equal(got[1::2], np.full(16, 2.5, np.float32))
