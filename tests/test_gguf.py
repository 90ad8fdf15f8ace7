"""The GGUF tensor table and load hook of gemma4.kt_amd/gguf.py against the
format: a file assembled byte by byte (known answers), round trips through the
test writer over every metadata value type and tensor type, and the reference's
error behaviour (GGUF.kt, GGMLType.kt:70-76, ModelLoader.kt:281-286)."""
import struct

import numpy as np
import pytest

import gguf
import g4hip
import synth
from gguf_writer import (ARRAY, BOOL, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, STRING, UINT8, UINT16,
                         UINT32, UINT64, write_gguf)


def _s(x: str) -> bytes:
    return struct.pack("<Q", len(x)) + x.encode()


def test_known_answer_file(tmp_path):
    """A v3 file written out by hand: one string and one u32 key, two tensors."""
    b = b"GGUF" + struct.pack("<iqq", 3, 2, 2)
    b += _s("general.name") + struct.pack("<i", 8) + _s("kat")
    b += _s("general.alignment") + struct.pack("<iI", 4, 64)
    b += _s("a.weight") + struct.pack("<iqq", 2, 32, 2) + struct.pack("<iq", 8, 0)     # Q8_0 2x32: 2 blocks
    b += _s("n.weight") + struct.pack("<iq", 1, 4) + struct.pack("<iq", 0, 128)       # F32 [4] at 128
    pad = (64 - len(b) % 64) % 64
    hdr = len(b) + pad
    blocks = bytes(range(68))
    norm = struct.pack("<4f", 1.0, -2.5, 0.0, 3.25)
    data = blocks + b"\0" * (128 - 68) + norm
    p = tmp_path / "kat.gguf"
    p.write_bytes(b + b"\0" * pad + data)
    g = gguf.GGUF.load_model(str(p))
    assert g.version == 3 and g.alignment == 64 and g.tensor_data_offset == hdr
    assert g.metadata == {"general.name": "kat", "general.alignment": 64}
    assert g.tensor_infos["a.weight"] == gguf.GGUFTensorInfo("a.weight", (32, 2), 8, 0)
    assert g.tensor_infos["n.weight"] == gguf.GGUFTensorInfo("n.weight", (4,), 0, 128)
    e = gguf.GGUF.load_tensors(str(p), g.tensor_data_offset, g.tensor_infos)
    assert e["a.weight"].memory_segment.tobytes() == blocks and e["a.weight"].n_elems == 64
    assert list(gguf.ModelLoader.to_float_buffer(e["n.weight"])) == [1.0, -2.5, 0.0, 3.25]


def test_metadata_value_types_round_trip(tmp_path):
    meta = [("u8", UINT8, 200), ("i8", INT8, -5), ("u16", UINT16, 60000), ("i16", INT16, -300),
            ("u32", UINT32, 4000000000), ("i32", INT32, -7), ("f32", FLOAT32, 1.5), ("b", BOOL, True),
            ("s", STRING, "héllo"), ("u64", UINT64, 2 ** 63 + 5), ("i64", INT64, -2 ** 40),
            ("f64", FLOAT64, 0.1), ("ai32", ARRAY, (INT32, [1, -2, 3])), ("af32", ARRAY, (FLOAT32, [0.5, 2.0])),
            ("as", ARRAY, (STRING, ["a", "bc"])), ("ab", ARRAY, (BOOL, [True, False])),
            ("au8", ARRAY, (UINT8, [1, 255])), ("ai16", ARRAY, (INT16, [-1, 7])),
            ("aa", ARRAY, (ARRAY, [(INT32, [1]), (INT32, [2, 3])]))]
    p = tmp_path / "m.gguf"
    write_gguf(str(p), meta, [])
    m = gguf.GGUF.load_model(str(p)).metadata
    # unsigned values come back as the signed type of the same width (readByte/readShort/readInt/readLong)
    assert m["u8"] == -56 and m["i8"] == -5 and m["u16"] == -5536 and m["i16"] == -300
    assert m["u32"] == 4000000000 - 2 ** 32 and m["i32"] == -7 and m["f32"] == 1.5 and m["b"] is True
    assert m["s"] == "héllo" and m["u64"] == 2 ** 63 + 5 - 2 ** 64 and m["i64"] == -2 ** 40
    assert m["f64"] == 0.1
    assert list(m["ai32"]) == [1, -2, 3] and list(m["af32"]) == [0.5, 2.0] and m["as"] == ["a", "bc"]
    assert list(m["ab"]) == [True, False] and m["au8"] == bytes([1, 255]) and list(m["ai16"]) == [-1, 7]
    assert [list(a) for a in m["aa"]] == [[1], [2, 3]]


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_tensors_round_trip(tmp_path, alignment):
    ts = [("q8", (64, 3), 8), ("q4", (32, 5), 2), ("q4k", (256, 2), 12), ("q5k", (256, 1), 13),
          ("q6k", (512, 1), 14), ("f16", (7,), 1), ("bf16", (9,), 30), ("f32", (5,), 0)]
    tensors = []
    for i, (name, dims, t) in enumerate(ts):
        n = int(np.prod(dims))
        tensors.append((name, dims, t, synth.weights(60 + i, name, t, n)))
    p = tmp_path / "t.gguf"
    offs = write_gguf(str(p), [("general.architecture", STRING, "gemma4")], tensors, alignment=alignment)
    g = gguf.GGUF.load_model(str(p))
    al = alignment or 32
    assert g.tensor_data_offset % al == 0
    e = gguf.GGUF.load_tensors(str(p), g.tensor_data_offset, g.tensor_infos)
    for name, dims, t, raw in tensors:
        assert g.tensor_infos[name].offset == offs[name] and offs[name] % al == 0
        assert e[name].ggml_type == t and e[name].shape == dims
        assert e[name].memory_segment.tobytes() == raw.view(np.uint8).tobytes()
        assert e[name].memory_segment.size == gguf.byte_size_for(t, int(np.prod(dims)))


def test_type_table_matches_library():
    for t in g4hip.GGMLType:
        assert gguf.GGML_TYPES[int(t)][0] == t.name
        assert (gguf.GGML_TYPES[int(t)][1], gguf.GGML_TYPES[int(t)][2]) == (t.type_size, t.block_size)
    assert gguf.GGML_TYPES[39] == ("MXFP4", 17, 32) and gguf.GGML_TYPES[3] == ("Q4_1", 20, 32)


def test_errors(tmp_path):
    p = tmp_path / "e.gguf"
    p.write_bytes(b"GGUX" + struct.pack("<iqq", 3, 0, 0))
    with pytest.raises(g4hip.IllegalArgumentException):
        gguf.GGUF.load_model(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<iqq", 1, 0, 0))
    with pytest.raises(g4hip.IllegalArgumentException):
        gguf.GGUF.load_model(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<iqq", 3, 1, 0) + _s("t") + struct.pack("<iqiq", 1, 32, 99, 0))
    with pytest.raises(g4hip.UnsupportedOperationException):
        gguf.GGUF.load_model(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<iqq", 3, 0, 1) + _s("k") + struct.pack("<i", 4))
    with pytest.raises(IOError):
        gguf.GGUF.load_model(str(p))
    write_gguf(str(p), [("x", ARRAY, (UINT64, [1]))], [])
    with pytest.raises(g4hip.UnsupportedOperationException):
        gguf.GGUF.load_model(str(p))
    # a tensor whose bytes run past the end of the file
    write_gguf(str(p), [], [("w", (32,), 8, synth.q8_0(1, "w", 32))])
    g = gguf.GGUF.load_model(str(p))
    g.tensor_infos["w"].dimensions = (64,)
    with pytest.raises(g4hip.IndexOutOfBoundsException):
        gguf.GGUF.load_tensors(str(p), g.tensor_data_offset, g.tensor_infos)
    # toFloatBuffer accepts F32 only
    write_gguf(str(p), [], [("h", (4,), 1, synth.dense(1, "h", 4, 1))])
    g = gguf.GGUF.load_model(str(p))
    e = gguf.GGUF.load_tensors(str(p), g.tensor_data_offset, g.tensor_infos)
    with pytest.raises(g4hip.UnsupportedOperationException):
        gguf.ModelLoader.to_float_buffer(e["h"])
