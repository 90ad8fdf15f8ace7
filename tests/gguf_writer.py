"""Writes small GGUF files for the tests (test infrastructure).

Layout as the GGUF format (v2/v3) defines it and gguf/GGUF.kt reads it: magic,
version, tensor count, metadata count, the metadata key/value pairs, the tensor
infos (name, dims, type id, offset relative to the tensor data), padding to the
alignment, then the tensor data with every tensor at an aligned offset."""
import struct

import numpy as np

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "B", INT8: "b", UINT16: "H", INT16: "h", UINT32: "I", INT32: "i", FLOAT32: "f", UINT64: "Q",
        INT64: "q", FLOAT64: "d"}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vt: int, v) -> bytes:
    if vt in _FMT:
        return struct.pack("<" + _FMT[vt], v)
    if vt == BOOL:
        return struct.pack("<B", 1 if v else 0)
    if vt == STRING:
        return _string(v)
    if vt == ARRAY:
        et, items = v
        out = struct.pack("<iQ", et, len(items))
        return out + b"".join(_value(et, it) for it in items)
    raise ValueError(vt)


def write_gguf(path: str, metadata, tensors, alignment=None, version: int = 3) -> dict:
    """metadata: [(key, value_type, value)] (arrays: (element_type, items));
    tensors: [(name, dims, ggml_type, raw_bytes)].  Returns name -> data offset."""
    al = alignment or 32
    kv = list(metadata)
    if alignment is not None:
        kv.append(("general.alignment", UINT32, alignment))
    head = struct.pack("<IiQQ", 0x46554747, version, len(tensors), len(kv))
    head += b"".join(_string(k) + struct.pack("<i", vt) + _value(vt, v) for k, vt, v in kv)
    offsets, off = {}, 0
    infos = b""
    for name, dims, t, raw in tensors:
        off = (off + al - 1) // al * al
        offsets[name] = off
        infos += _string(name) + struct.pack("<i", len(dims)) + b"".join(struct.pack("<q", d) for d in dims)
        infos += struct.pack("<iq", t, off)
        off += len(np.ascontiguousarray(raw).view(np.uint8).reshape(-1))
    body = head + infos
    body += b"\0" * ((al - len(body) % al) % al)
    data = bytearray(off)
    for name, dims, t, raw in tensors:
        b = np.ascontiguousarray(raw).view(np.uint8).reshape(-1).tobytes()
        data[offsets[name]:offsets[name] + len(b)] = b
    with open(path, "wb") as f:
        f.write(body)
        f.write(bytes(data))
    return offsets
