"""Minimal GGUF v3 writer for tests: typed KV pairs, tensor infos, alignment
padding, tensor data. Byte layout per the GGUF v3 format (little-endian):
magic, version, tensor count, KV count, KVs, tensor infos, pad, data."""
import struct

import numpy as np

GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL = range(8)
GGUF_STR, GGUF_ARR, GGUF_U64, GGUF_I64, GGUF_F64 = 8, 9, 10, 11, 12
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30

_FMT = {GGUF_U8: "<B", GGUF_I8: "<b", GGUF_U16: "<H", GGUF_I16: "<h", GGUF_U32: "<I",
        GGUF_I32: "<i", GGUF_F32: "<f", GGUF_BOOL: "<B", GGUF_U64: "<Q", GGUF_I64: "<q",
        GGUF_F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _val(t, v):
    if t == GGUF_STR:
        return _str(v)
    if t == GGUF_ARR:
        at, items = v
        return struct.pack("<IQ", at, len(items)) + b"".join(_val(at, x) for x in items)
    return struct.pack(_FMT[t], v)


def tensor_bytes(arr, ggml_type):
    """numpy array -> payload bytes (bf16 given as uint16 bit patterns)."""
    if ggml_type == GGML_F32:
        return np.ascontiguousarray(arr, np.float32).tobytes()
    if ggml_type == GGML_F16:
        return np.ascontiguousarray(arr, np.float16).tobytes()
    return np.ascontiguousarray(arr, np.uint16).tobytes()


def write(path, kvs, tensors, alignment=256, version=3, magic=b"GGUF", raw_infos=None,
          drop_tail_padding=False):
    """kvs: [(key, gguf_type, value)]; tensors: [(name, dims, ggml_type, payload_bytes)]
    with dims in GGUF order. Offsets are assigned in order, each aligned.
    raw_infos replaces the tensor-info section (for malformed-header tests).
    Returns the list of assigned offsets."""
    head = magic + struct.pack("<IQQ", version, len(tensors) if raw_infos is None else raw_infos[0],
                               len(kvs))
    body = b"".join(_str(k) + struct.pack("<I", t) + _val(t, v) for k, t, v in kvs)
    offs, off = [], 0
    infos = b""
    for name, dims, gt, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        infos += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", gt, off)
        off += len(data)
    if raw_infos is not None:
        infos = raw_infos[1]
    hdr = head + body + infos
    pad = (-len(hdr)) % alignment
    data = b""
    for (name, dims, gt, payload), o in zip(tensors, offs):
        data += b"\0" * (o - len(data)) + payload
    if not drop_tail_padding:
        data += b"\0" * ((-len(data)) % alignment)
    with open(path, "wb") as f:
        f.write(hdr + b"\0" * pad + data)
    return offs
