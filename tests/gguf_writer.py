"""Writes GGUF v2/v3 files for the tests (the container layout the reference
parses: header, key/values, tensor table, aligned data section)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v) -> bytes:
    if vtype == STR:
        return _s(v.encode() if isinstance(v, str) else v)
    if vtype == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_FMT[vtype], v)


def gguf_bytes(kv, tensors, version=3, align=None, pad_to=None):
    """kv: [(key, vtype, value)]; tensors: [(name, dims, ggml_type, data bytes)].
    Tensor data are laid out in order at multiples of the alignment."""
    a = 32 if align is None else align
    kvs = list(kv) + ([("general.alignment", U32, align)] if align is not None else [])
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += _s(k.encode()) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off = (off + len(data) + a - 1) // a * a
    for (name, dims, ty, _), o in zip(tensors, offs):
        nb = name.encode() if isinstance(name, str) else name
        head += _s(nb) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, o)
    data_off = (len(head) + a - 1) // a * a
    body = bytearray(head + b"\0" * (data_off - len(head)))
    for (_, _, _, data), o in zip(tensors, offs):
        body += b"\0" * (data_off + o - len(body))
        body += bytes(data)
    if pad_to is not None and len(body) < pad_to:
        body += b"\0" * (pad_to - len(body))
    return bytes(body), data_off, offs


def write(path, *args, **kw):
    data, data_off, offs = gguf_bytes(*args, **kw)
    with open(path, "wb") as f:
        f.write(data)
    return data, data_off, offs


def random_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()
