"""A GGUF writer for tests, written from the GGUF specification (versions 2 and 3, little endian): header, key-values,
tensor infos, padding to general.alignment, then each tensor's bytes at its aligned offset in the data section."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q", I64: "<q",
        F64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vt, v) -> bytes:
    if vt == STRING:
        return _str(v)
    if vt == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def gguf_bytes(kvs, tensors, alignment=32, version=3, offsets=None):
    """kvs: [(key, value type, value)], an array's value being (element type, [items]); tensors: [(name, ggml type,
    ne tuple, data bytes)]. `offsets` overrides the tensors' data offsets (to write broken files). Returns the file's
    bytes and the offset of its data section."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, vt, v in kvs:
        head += _str(k) + struct.pack("<I", vt) + _value(vt, v)
    offs, at = [], 0
    for _, _, _, data in tensors:
        offs.append(at)
        at = (at + len(data) + alignment - 1) // alignment * alignment
    if offsets is not None:
        offs = list(offsets)
    for (name, t, ne, _), off in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", t, off)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(max([o + len(d) for o, (_, _, _, d) in zip(offs, tensors)], default=0))
    for o, (_, _, _, d) in zip(offs, tensors):
        body[o:o + len(d)] = d
    return head + bytes(data_start - len(head)) + bytes(body), data_start


def write_gguf(path, kvs, tensors, **kw) -> int:
    """Writes the file; returns the data section's offset."""
    b, data_start = gguf_bytes(kvs, tensors, **kw)
    path.write_bytes(b)
    return data_start


def as_bytes(a: np.ndarray) -> bytes:
    return np.ascontiguousarray(a).tobytes()
