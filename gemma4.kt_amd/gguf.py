"""GGUF tensor table and the load-time upload hook, mirroring gemma4.kt's gguf package.

Reference paths are relative to lib/src/main/kotlin/io/github/lbenedetto/internal/:
  * gguf/GGUF.kt: the parser (header, metadata key/value pairs, tensor infos,
    alignment padding; :10-185) and loadTensors (:195-212), which memory-maps the
    tensor data and slices one entry per tensor without copying;
  * gguf/GGMLTensorEntry.kt, gguf/GGUFTensorInfo.kt, gguf/MetadataValueType.kt;
  * gguf/ModelLoader.kt:268-286: loadQuantized (every weight matrix goes through
    FloatTensorFactory.create, floattensor/FloatTensorFactory.kt:7-23) and
    toFloatBuffer (norm vectors: F32 only).

The hook: `ModelLoader.load_quantized(ctx, entry)` hands the entry's mapped bytes
to `FloatTensorFactory.create`, which uploads the raw GGUF blocks once to device
memory (g4_upload; no repacking).  Formats the device path does not implement
raise UnsupportedOperationException there; a host keeps its CPU tensor for them.

Scope: this module exists to reach the tensor table (infos, alignment, data
offset) that the upload hook needs.  GGUF stores the tensor infos after the
metadata, and each metadata value's length depends on its type, so the table is
walked and kept as the reference keeps it; nothing here interprets metadata
beyond the alignment, and the model loader above loadQuantized (hyperparameters,
tokenizer) is not built.

Byte order is little-endian throughout (ChannelReader.kt:10).  Values are read
as the reference reads them: UINT8/UINT16/UINT32/UINT64 as the signed type of
the same width (readByte/readShort/readInt/readLong).
"""
from __future__ import annotations

import enum
import mmap
import os
import struct
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

from g4hip import (FloatTensorFactory, IllegalArgumentException, IndexOutOfBoundsException,
                   UnsupportedOperationException)

GGUF_MAGIC = 0x46554747          # "GGUF" read as a little-endian int (GGUF.kt:206)
DEFAULT_ALIGNMENT = 32           # GGUF.kt:207
SUPPORTED_GGUF_VERSIONS = (2, 3)  # GGUF.kt:209

_BIG = 2 ** 31 - 1  # Int.MAX_VALUE: the type size the reference gives formats it cannot read

# GGMLType.kt:16-56: (name, typeSize, blockSize) by id (the enum ordinal).
GGML_TYPES = [
    ("F32", 4, 1), ("F16", 2, 1), ("Q4_0", 18, 32), ("Q4_1", 20, 32), ("UNSUPPORTED_Q4_2", _BIG, 1),
    ("UNSUPPORTED_Q4_3", _BIG, 1), ("Q5_0", _BIG, 1), ("Q5_1", 24, 32), ("Q8_0", 34, 32), ("Q8_1", 40, 32),
    ("Q2_K", _BIG, 1), ("Q3_K", _BIG, 1), ("Q4_K", 144, 256), ("Q5_K", 176, 256), ("Q6_K", 210, 256),
    ("Q8_K", _BIG, 1), ("IQ2_XXS", _BIG, 1), ("IQ2_XS", _BIG, 1), ("IQ3_XXS", _BIG, 1), ("IQ1_S", _BIG, 1),
    ("IQ4_NL", _BIG, 1), ("IQ3_S", _BIG, 1), ("IQ2_S", _BIG, 1), ("IQ4_XS", _BIG, 1), ("I8", 1, 1),
    ("I16", 2, 1), ("I32", 4, 1), ("I64", 8, 1), ("F64", 8, 1), ("IQ1_M", _BIG, 1), ("BF16", 2, 1),
    ("UNSUPPORTED_Q4_0_4_4", _BIG, 1), ("UNSUPPORTED_Q4_0_4_8", _BIG, 1), ("UNSUPPORTED_Q4_0_8_8", _BIG, 1),
    ("TQ1_0", _BIG, 1), ("TQ2_0", _BIG, 1), ("UNSUPPORTED_IQ4_NL_4_4", _BIG, 1),
    ("UNSUPPORTED_IQ4_NL_4_8", _BIG, 1), ("UNSUPPORTED_IQ4_NL_8_8", _BIG, 1), ("MXFP4", 17, 32),
    ("NVFP4", _BIG, 1),
]


def ggml_type_from_id(type_id: int) -> int:
    """GGMLType.fromId (GGMLType.kt:70-76)."""
    if 0 <= type_id < len(GGML_TYPES):
        return type_id
    raise UnsupportedOperationException("Unsupported GGML tensor type id: %d" % type_id)


def ggml_type_name(type_id: int) -> str:
    return GGML_TYPES[type_id][0]


def byte_size_for(type_id: int, n_elems: int) -> int:
    """GGMLType.byteSizeFor (GGMLType.kt:57-61)."""
    _, ts, bs = GGML_TYPES[type_id]
    return n_elems * ts // bs


def number_of_elements(dims) -> int:
    """FloatTensorHelpers.numberOfElementsLong."""
    n = 1
    for d in dims:
        n *= int(d)
    return n


class MetadataValueType(enum.IntEnum):
    """MetadataValueType.kt: the value type index of a metadata entry."""
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


@dataclass
class GGUFTensorInfo:
    """GGUFTensorInfo.kt."""
    name: str
    dimensions: tuple
    ggml_type: int
    offset: int


@dataclass
class GGMLTensorEntry:
    """GGMLTensorEntry.kt: the tensor's bytes are a read-only view into the mapped file."""
    mapped_file: object
    name: str
    ggml_type: int
    shape: tuple
    memory_segment: np.ndarray

    @property
    def n_elems(self) -> int:
        return number_of_elements(self.shape)


class _Reader:
    """Sequential little-endian reads (ChannelReader.kt)."""

    def __init__(self, f):
        self.f = f
        self.pos = 0

    def bytes(self, n: int) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise IOError("Unexpected EOF while reading GGUF metadata")
        self.pos += n
        return b

    def unpack(self, fmt: str):
        return struct.unpack("<" + fmt, self.bytes(struct.calcsize("<" + fmt)))[0]


class GGUF:
    """GGUF.kt: header, metadata, tensor infos and the offset of the tensor data."""

    def __init__(self, f):
        r = _Reader(f)
        self.metadata: Dict[str, object] = {}
        self.metadata_types: Dict[str, MetadataValueType] = {}
        self._read_header(r)
        self.tensor_infos: Dict[str, GGUFTensorInfo] = {}
        for _ in range(self.tensor_count):
            ti = self._read_tensor_info(r)
            self.tensor_infos[ti.name] = ti
        padding = (self.alignment - (r.pos % self.alignment)) % self.alignment
        r.bytes(padding)
        self.tensor_data_offset = r.pos

    @property
    def alignment(self) -> int:
        a = self.metadata.get("general.alignment", DEFAULT_ALIGNMENT)
        if not isinstance(a, int) or isinstance(a, bool):
            raise IllegalArgumentException("general.alignment is not an Int")  # the reference's `as Int` cast
        return a

    # -- parsing (GGUF.kt:42-185)
    def _read_header(self, r: _Reader) -> None:
        magic = r.unpack("i")
        if magic != GGUF_MAGIC:
            raise IllegalArgumentException("unsupported header.magic %d" % magic)
        version = r.unpack("i")
        if version not in SUPPORTED_GGUF_VERSIONS:
            raise IllegalArgumentException("unsupported header.version %d" % version)
        self.version = version
        self.tensor_count = r.unpack("q")
        kv_count = r.unpack("q")
        for _ in range(kv_count):
            key = self._read_string(r)
            vt = self._read_value_type(r)
            self.metadata[key] = self._read_value(vt, r)
            self.metadata_types[key] = vt

    @staticmethod
    def _read_string(r: _Reader) -> str:
        n = r.unpack("q")
        return r.bytes(n).decode("utf-8")

    @staticmethod
    def _read_value_type(r: _Reader) -> MetadataValueType:
        i = r.unpack("i")
        if not 0 <= i < len(MetadataValueType):
            raise IndexOutOfBoundsException("metadata value type %d" % i)
        return MetadataValueType(i)

    _SCALAR = {MetadataValueType.UINT8: "b", MetadataValueType.INT8: "b", MetadataValueType.UINT16: "h",
               MetadataValueType.INT16: "h", MetadataValueType.UINT32: "i", MetadataValueType.INT32: "i",
               MetadataValueType.FLOAT32: "f", MetadataValueType.UINT64: "q", MetadataValueType.INT64: "q",
               MetadataValueType.FLOAT64: "d"}

    def _read_value(self, vt: MetadataValueType, r: _Reader):
        if vt in self._SCALAR:
            return r.unpack(self._SCALAR[vt])
        if vt == MetadataValueType.BOOL:
            return r.unpack("b") != 0
        if vt == MetadataValueType.STRING:
            return self._read_string(r)
        return self._read_array(r)

    def _read_array(self, r: _Reader):
        """GGUF.kt:109-123: 8/16/32-bit integers, float32, bool, string and nested arrays."""
        vt = self._read_value_type(r)
        n = r.unpack("q")
        if vt in (MetadataValueType.UINT8, MetadataValueType.INT8):
            return r.bytes(n)
        if vt in (MetadataValueType.UINT16, MetadataValueType.INT16):
            return np.frombuffer(r.bytes(2 * n), dtype="<i2").copy()
        if vt in (MetadataValueType.UINT32, MetadataValueType.INT32):
            return np.frombuffer(r.bytes(4 * n), dtype="<i4").copy()
        if vt == MetadataValueType.FLOAT32:
            return np.frombuffer(r.bytes(4 * n), dtype="<f4").copy()
        if vt == MetadataValueType.BOOL:
            return np.frombuffer(r.bytes(n), dtype=np.int8) != 0
        if vt == MetadataValueType.STRING:
            return [self._read_string(r) for _ in range(n)]
        if vt == MetadataValueType.ARRAY:
            return [self._read_array(r) for _ in range(n)]
        raise UnsupportedOperationException("read array of %s" % vt.name)

    def _read_tensor_info(self, r: _Reader) -> GGUFTensorInfo:
        name = self._read_string(r)
        nd = r.unpack("i")
        dims = tuple(r.unpack("q") for _ in range(nd))
        for d in dims:
            if not -2 ** 31 <= d < 2 ** 31:
                raise ArithmeticError("integer overflow")  # Math.toIntExact
        t = ggml_type_from_id(r.unpack("i"))
        offset = r.unpack("q")
        return GGUFTensorInfo(name, dims, t, offset)

    # -- GGUF.kt:214-228
    @staticmethod
    def load_model(path: str) -> "GGUF":
        with open(path, "rb") as f:
            return GGUF(f)

    @staticmethod
    def load_tensors(path: str, tensor_data_offset: int,
                     tensor_infos: Dict[str, GGUFTensorInfo]) -> Dict[str, GGMLTensorEntry]:
        """GGUF.kt:195-212: map the tensor data read-only and slice each tensor's
        byteSizeFor(n) bytes at its offset (no copy)."""
        size = os.path.getsize(path)
        if size < tensor_data_offset:
            raise IndexOutOfBoundsException("tensor data offset %d past the end of the file" % tensor_data_offset)
        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size > 0 else b""
        data = np.frombuffer(mm, dtype=np.uint8, offset=tensor_data_offset)
        entries = {}
        for name, ti in tensor_infos.items():
            n = number_of_elements(ti.dimensions)
            nbytes = byte_size_for(ti.ggml_type, n)
            if ti.offset < 0 or nbytes < 0 or ti.offset + nbytes > data.size:
                raise IndexOutOfBoundsException("tensor %s: %d bytes at offset %d exceed the %d bytes of tensor data"
                                                % (name, nbytes, ti.offset, data.size))
            seg = data[ti.offset:ti.offset + nbytes]
            entries[name] = GGMLTensorEntry(mm, name, ti.ggml_type, ti.dimensions, seg)
        return entries


class ModelLoader:
    """The tensor-loading half of ModelLoader.kt: the hook where weights go to the device."""

    @staticmethod
    def load_quantized(ctx, entry: GGMLTensorEntry):
        """ModelLoader.kt:268-271: FloatTensorFactory.create(entry.ggmlType, entry); here
        the factory uploads the entry's raw blocks to ctx's device."""
        return FloatTensorFactory.create(ctx, entry.ggml_type, entry)

    @staticmethod
    def load_array_of_quantized(ctx, size: int, get_entry):
        return [ModelLoader.load_quantized(ctx, get_entry(i)) for i in range(size)]

    @staticmethod
    def to_float_buffer(entry: GGMLTensorEntry) -> np.ndarray:
        """ModelLoader.kt:281-286: an F32 tensor as float32 values (a view of the mapping)."""
        if entry.ggml_type != 0:
            raise UnsupportedOperationException("Conversion to %s" % ggml_type_name(entry.ggml_type))
        return entry.memory_segment.view("<f4")

    @staticmethod
    def load_norm(ctx, entry: GGMLTensorEntry):
        """A norm vector for the device decode step: toFloatBuffer's F32 check, then
        the same upload as any tensor."""
        ModelLoader.to_float_buffer(entry)
        return FloatTensorFactory.create(ctx, entry.ggml_type, entry)


def load_device_tensors(ctx, path: str, names: Optional[list] = None) -> Dict[str, object]:
    """Parse `path`, map its tensor data and upload the named tensors (all when
    names is None) to ctx's device: name -> GpuFloatTensor."""
    g = GGUF.load_model(path)
    entries = GGUF.load_tensors(path, g.tensor_data_offset, g.tensor_infos)
    return {n: ModelLoader.load_quantized(ctx, entries[n]) for n in (names if names is not None else entries)}
