"""Minimal GGUF v2/v3 writer for tests: the byte layout the reference's own
tests build by hand (weight_loading/gguf.rs:600-680, 768-788) — header, metadata,
tensor infos, padding to the alignment, tensor data — generalised to any
metadata and any number of tensors, each tensor's data padded to the alignment
as llama.cpp writes it."""
import struct

GGUF_MAGIC = 0x46554747

# GGML tensor types
F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K = 0, 1, 2, 3, 8, 12, 14
# metadata value types
U8, I8, U16, I16, U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _str(value)
    if vtype == ARRAY:
        etype, items = value
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, v) for v in items)
    return struct.pack(_SCALAR[vtype], value)


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def gguf_bytes(tensors, meta=(), version=3, alignment=32) -> bytes:
    """tensors: [(name, ggml_type, dims fastest-first, data bytes)];
    meta: [(key, value type, value)], arrays as (key, ARRAY, (elem type, items))."""
    head = struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(meta))
    for key, vtype, value in meta:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
    offset, blobs = 0, []
    for name, ggml_type, dims, data in tensors:
        data = bytes(data)
        head += _str(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ggml_type, offset)
        pad = _align(len(data), alignment) - len(data)
        blobs.append(data + b"\0" * pad)
        offset += len(data) + pad
    head += b"\0" * (_align(len(head), alignment) - len(head))
    return head + b"".join(blobs)


def write_gguf(path, tensors, meta=(), version=3, alignment=32):
    with open(path, "wb") as f:
        f.write(gguf_bytes(tensors, meta, version, alignment))
    return path
