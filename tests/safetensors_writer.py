"""Minimal safetensors writer for tests: the layout the reference's tests
build (safetensors.rs:309-341) — u64 header length, JSON header, data section
— plus the index file of a sharded checkpoint (safetensors.rs:511-558)."""
import json
import struct

import numpy as np

DTYPES = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16",
          np.dtype(np.int64): "I64", np.dtype(np.int32): "I32", np.dtype(np.uint8): "U8"}


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns by truncation (exact for values already bf16)."""
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def st_bytes(tensors, metadata=None) -> bytes:
    """tensors: [(name, dtype string, shape, raw bytes)] or [(name, ndarray)]."""
    header, data = {}, b""
    if metadata is not None:
        header["__metadata__"] = metadata
    for t in tensors:
        if len(t) == 2:
            name, arr = t
            arr = np.ascontiguousarray(arr)
            t = (name, DTYPES[arr.dtype], list(arr.shape), arr.tobytes())
        name, dtype, shape, raw = t
        header[name] = {"dtype": dtype, "shape": list(shape),
                        "data_offsets": [len(data), len(data) + len(raw)]}
        data += bytes(raw)
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


def write_st(path, tensors, metadata=None):
    with open(path, "wb") as f:
        f.write(st_bytes(tensors, metadata))
    return path


def write_index(dir_path, weight_map: dict, total_size: int = 0):
    with open(f"{dir_path}/model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {"total_size": total_size}, "weight_map": weight_map}, f)
