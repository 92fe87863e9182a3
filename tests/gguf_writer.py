"""Minimal GGUF v3 writer for tests: metadata key/values and tensors laid out as the published GGUF format has them
(magic, version, counts, key/values, tensor infos, data aligned to general.alignment).  Test data only: files written
here feed the engine's reader (rmi_gguf_open) and rmi_engine_create_gguf."""
import struct

import numpy as np

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
        F64: "<d"}

# GGML tensor types and their block geometry (elements, bytes)
GGML = {"F32": (0, 1, 4), "F16": (1, 1, 2), "Q8_0": (8, 32, 34), "Q4_K": (12, 256, 144), "Q5_K": (13, 256, 176),
        "Q6_K": (14, 256, 210)}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_FMT[t], v)


def tensor_bytes(type_name, dims):
    _, per, nb = GGML[type_name]
    elems = int(np.prod(dims))
    assert dims[0] % per == 0
    return elems // per * nb


def write_gguf(path, meta, tensors, alignment=32, version=3):
    """meta: list of (key, type, value); tensors: list of (name, type_name, dims (innermost first), bytes)"""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    kv = b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in meta)
    infos, off, blobs = b"", 0, []
    for name, tname, dims, data in tensors:
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        assert data.size == tensor_bytes(tname, dims), (name, data.size, tensor_bytes(tname, dims))
        infos += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", GGML[tname][0], off)
        blobs.append((off, data))
        off = (off + data.size + alignment - 1) // alignment * alignment
    body = head + kv + infos
    pad = (-len(body)) % alignment
    with open(path, "wb") as f:
        f.write(body + b"\0" * pad)
        pos = 0
        for o, data in blobs:
            f.write(b"\0" * (o - pos))
            f.write(memoryview(data))   # the array's own memory: no copy of a multi-GB tensor
            pos = o + data.size
    return path
