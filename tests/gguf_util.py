"""A small gguf writer for the loader tests (the encoding of the
reference's test/gguf.lua: header, key-values, tensor infos with shapes in
ggml order, data aligned to 32 bytes). Test infrastructure."""
import struct

import numpy as np

U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64 = 4, 5, 6, 7, 8, 9, 10, 11
ALIGN = 32
_FMT = {U32: "<I", I32: "<i", F32V: "<f", BOOL: "<B", U64: "<Q", I64: "<q"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    return struct.pack(_FMT[t], int(v) if t == BOOL else v)


def _pad(b):
    return b + b"\0" * (-len(b) % ALIGN)


def encode(kv, tensors):
    """kv: [(key, type, value)] with type (ARRAY, element type) for lists.
    tensors: [(name, shape in torch order, numpy array of the raw data,
    ggml type)]."""
    out = [b"GGUF", struct.pack("<IQQ", 3, len(tensors), len(kv))]
    for key, t, v in kv:
        out.append(_str(key))
        if isinstance(t, tuple):
            out.append(struct.pack("<IIQ", ARRAY, t[1], len(v)))
            out += [_value(t[1], x) for x in v]
        else:
            out.append(struct.pack("<I", t) + _value(t, v))
    data, off = [], 0
    for name, shape, arr, ty in tensors:
        raw = _pad(np.ascontiguousarray(arr).tobytes())
        out.append(_str(name) + struct.pack("<I", len(shape)))
        out += [struct.pack("<Q", d) for d in reversed(shape)]
        out.append(struct.pack("<IQ", ty, off))
        data.append(raw)
        off += len(raw)
    return _pad(b"".join(out)) + b"".join(data)


def write(path, kv, tensors):
    with open(path, "wb") as f:
        f.write(encode(kv, tensors))
