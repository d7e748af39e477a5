"""Writes GGUF v2/v3 files for tests (the public GGUF layout, little-endian).

Plays the part of jero-core's create_synthetic_gguf_v3_with_kvs as used by
tests/architecture_certification_gate.rs:82-176 (reference): general.architecture and
general.alignment first, then the given metadata, then one descriptor per tensor in the given
order with offsets packed at the alignment, then the data section.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(arch, kvs, tensors, alignment=32, version=3, offsets=None):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, dims, payload bytes)], dims with the
    row length first.  offsets overrides the computed data offsets (malformed-file tests)."""
    meta = [("general.architecture", STRING, arch), ("general.alignment", U32, alignment)] + list(kvs)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, t, v in meta:
        head += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, pos = [], 0
    for _, _, _, payload in tensors:
        offs.append(pos)
        pos += (len(payload) + alignment - 1) // alignment * alignment
    if offsets is not None:
        offs = offsets
    for (name, q, dims, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", q, off)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    buf = bytearray(head.ljust(data_start, b"\0"))
    for (_, _, _, payload), off in zip(tensors, offs):
        if offsets is not None and off > 1 << 24:  # an overridden offset far past any data: the payload is left out
            continue
        end = data_start + off + len(payload)
        if len(buf) < end:
            buf.extend(b"\0" * (end - len(buf)))
        buf[data_start + off:end] = bytes(payload)
    return bytes(buf)


def as_bytes(arr):
    return np.ascontiguousarray(arr).view(np.uint8).tobytes()
