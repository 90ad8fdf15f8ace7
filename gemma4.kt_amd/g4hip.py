"""Python host side of libg4hip.so, mirroring gemma4.kt's tensor layer.

The reference's operator interface for the quantized matrix-vector path is the
Kotlin `FloatTensor` (lib/src/main/kotlin/io/github/lbenedetto/internal/
floattensor/FloatTensor.kt:5-71) created by `FloatTensorFactory.create`
(FloatTensorFactory.kt:7-23).  This module keeps those names and argument
meanings over the C ABI of include/g4hip.h:

  * `FloatTensorFactory.create(ctx, ggml_type, raw, n_elems)` uploads raw GGUF
    blocks once and returns a `GpuFloatTensor`.
  * `GpuFloatTensor.matmul(that, out, dim0, dim1[, this_offset])` computes
    out[i] = dot(this_offset + i*dim1, that, 0, dim1) for i < dim0.
  * `get`, `dot`, `argmax`, plus the batched, LM-head, FFN and MoE entry points.

Errors surface as the reference's exception types (status codes of g4hip.h).
There is no fallback: if libg4hip.so is missing or no device is present, the
calls raise.
"""
from __future__ import annotations

import ctypes
import enum
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libg4hip.so")

# ------------------------------------------------------------------ errors ---


class G4Error(Exception):
    code = 0


class IllegalArgumentException(G4Error, ValueError):
    code = -1


class UnsupportedOperationException(G4Error, NotImplementedError):
    code = -2


class IndexOutOfBoundsException(G4Error, IndexError):
    code = -3


class IllegalStateException(G4Error, RuntimeError):
    code = -4


class DeviceError(IllegalStateException):
    code = -5


class OutOfMemoryError(G4Error, MemoryError):
    code = -6


_ERRORS = {c.code: c for c in (IllegalArgumentException, UnsupportedOperationException,
                               IndexOutOfBoundsException, IllegalStateException, DeviceError,
                               OutOfMemoryError)}

# ---------------------------------------------------------------- library ---

_lib = None
_c_f32p = ctypes.POINTER(ctypes.c_float)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64

# symbol -> argtypes (every symbol declared in include/g4hip.h)
SIGNATURES = {
    "g4_last_error": [],
    "g4_version": [],
    "g4_device_count": [_c_i32p],
    "g4_type_info": [ctypes.c_int, _c_i32p, _c_i32p],
    "g4_byte_size": [ctypes.c_int, _i64, ctypes.POINTER(_i64)],
    "g4_check_matmul": [ctypes.c_int, _i64, _i64, _i32, _i32],
    "g4_open": [ctypes.c_int, ctypes.POINTER(_vp)],
    "g4_close": [_vp],
    "g4_ctx_set_stream": [_vp, _vp],
    "g4_ctx_sync": [_vp],
    "g4_ctx_device": [_vp, _c_i32p],
    "g4_ctx_reserve": [_vp, _i64],
    "g4_ctx_scratch_bytes": [_vp, ctypes.POINTER(_i64)],
    "g4_upload": [_vp, ctypes.c_int, _vp, _i64, _i64, ctypes.POINTER(_vp)],
    "g4_weight_free": [_vp],
    "g4_weight_info": [_vp, _c_i32p, ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    "g4_weight_device_ptr": [_vp, ctypes.POINTER(_vp)],
    "g4_matmul": [_vp, _vp, _i64, _vp, _vp, _i32, _i32],
    "g4_matmul_dev": [_vp, _vp, _i64, _vp, _vp, _i32, _i32],
    "g4_matmul_batch": [_vp, _vp, _i64, _vp, _i32, _vp, _i32, _i32],
    "g4_matmul_batch_dev": [_vp, _vp, _i64, _vp, _i32, _vp, _i32, _i32],
    "g4_matmul_argmax": [_vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32],
    "g4_matmul_argmax_dev": [_vp, _vp, _i64, _vp, _vp, _vp, _i32, _i32],
    "g4_argmax": [_vp, _vp, _i32, _vp],
    "g4_argmax_dev": [_vp, _vp, _i32, _vp],
    "g4_dequant": [_vp, _vp, _i64, _i64, _vp],
    "g4_dequant_dev": [_vp, _vp, _i64, _i64, _vp],
    "g4_ffn": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32],
    "g4_ffn_dev": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32],
    "g4_ffn_gate_up": [_vp, _vp, _vp, _vp, _vp, _i32, _i32],
    "g4_ffn_gate_up_dev": [_vp, _vp, _vp, _vp, _vp, _i32, _i32],
    "g4_moe_route": [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp],
    "g4_moe_route_dev": [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp],
    "g4_moe": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _i32, _vp],
    "g4_moe_dev": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp, _i32, _vp],
    "g4_moe_routed": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp],
    "g4_moe_routed_dev": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp],
    "g4_moe_routed_dev_noalloc": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp],
    "g4_rmsnorm_dev": [_vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, ctypes.c_int],
    "g4_rmsnorm_add_dev": [_vp, _vp, _vp, _vp, _i32, ctypes.c_float],
    "g4_add_dev": [_vp, _vp, _vp, _i32],
    "g4_softcap_dev": [_vp, _vp, _i32, ctypes.c_float],
    "g4_matmul_norm_dev": [_vp, _vp, _i64, _vp, _vp, ctypes.c_float, _vp, _vp, _i32, _i32],
    "g4_ffn_block": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float],
    "g4_ffn_block_dev": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float],
    "g4_lm_head": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, ctypes.c_float],
    "g4_lm_head_dev": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, ctypes.c_float],
    "g4_attention_dev": [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32],
}


def lib(path: Optional[str] = None) -> ctypes.CDLL:
    """Load libg4hip.so once.  Raises OSError if the library was not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise OSError("libg4hip.so not found at %s: run gemma4.kt_amd/build.py (no CPU fallback exists)" % path)
    # The *_dev wrappers take torch's device tensors and streams, so the library
    # must run on torch's HIP runtime.  torch ships its own libamdhip64 and puts
    # it in the process's global symbol scope when imported; a library loaded
    # before torch binds its HIP calls to the system runtime instead, leaving two
    # runtimes in one process whose stream handles and queues are not shared.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p if name == "g4_last_error" else ctypes.c_int
    _lib = L
    return L


def last_error() -> str:
    return lib().g4_last_error().decode(errors="replace")


def check(rc: int) -> None:
    if rc != 0:
        cls = _ERRORS.get(rc, G4Error)
        raise cls(last_error())


def check_matmul(ggml_type: int, n_elems: int, this_offset: int, dim0: int, dim1: int) -> None:
    """Host-only geometry validation (raises what matmul would raise before launching)."""
    check(lib().g4_check_matmul(int(ggml_type), int(n_elems), int(this_offset), int(dim0), int(dim1)))


def device_count() -> int:
    n = ctypes.c_int32(0)
    check(lib().g4_device_count(ctypes.byref(n)))
    return n.value

# ------------------------------------------------------------------ types ---


class GGMLType(enum.IntEnum):
    """GGMLType.kt:16-56 ids of the supported formats."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    BF16 = 30

    @property
    def block_size(self) -> int:
        bs = ctypes.c_int32()
        check(lib().g4_type_info(int(self), ctypes.byref(bs), None))
        return bs.value

    @property
    def type_size(self) -> int:
        ts = ctypes.c_int32()
        check(lib().g4_type_info(int(self), None, ctypes.byref(ts)))
        return ts.value

    def byte_size_for(self, n_elems: int) -> int:
        """GGMLType.kt:58-62 byteSizeFor."""
        out = ctypes.c_int64()
        check(lib().g4_byte_size(int(self), int(n_elems), ctypes.byref(out)))
        return out.value


def _ptr(a) -> int:
    """Address of a contiguous numpy array, or of a torch tensor's storage."""
    if a is None:
        return 0
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise IllegalArgumentException("array must be C-contiguous")
        return a.ctypes.data
    if hasattr(a, "data_ptr"):
        if not a.is_contiguous():
            raise IllegalArgumentException("tensor must be contiguous")
        return a.data_ptr()
    raise IllegalArgumentException("unsupported buffer type %r" % type(a))


def _f32(a, name: str) -> np.ndarray:
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags["C_CONTIGUOUS"]:
        raise IllegalArgumentException("%s must be a C-contiguous float32 numpy array" % name)
    return a


def _dev_f32(t, name: str):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    import torch
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
        raise IllegalArgumentException("%s must be a contiguous float32 device tensor" % name)
    return t


def _dev_i32(t, name: str):
    """A contiguous int32 device tensor (or a raw device address as int)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    import torch
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.int32 and t.is_contiguous()):
        raise IllegalArgumentException("%s must be a contiguous int32 device tensor" % name)
    return t


def _need(a, n: int, what: str) -> None:
    """The reference indexes past the end of a short array with an exception
    (IndexOutOfBoundsException); the C ABI would read or write past it."""
    if a is not None and a.size < n:
        raise IndexOutOfBoundsException("%s holds %d elements, %d needed" % (what, a.size, n))


# ---------------------------------------------------------------- context ---


class Context:
    """A HIP stream plus staging buffers on one device (one thread at a time)."""

    def __init__(self, ordinal: int = 0):
        h = _vp()
        check(lib().g4_open(int(ordinal), ctypes.byref(h)))
        self.handle = h.value
        self.ordinal = ordinal

    def set_stream(self, stream_handle: Optional[int]) -> None:
        """Launch *_dev work on an external hipStream_t (e.g. torch's current stream)."""
        check(lib().g4_ctx_set_stream(self.handle, stream_handle or None))

    def sync(self) -> None:
        check(lib().g4_ctx_sync(self.handle))

    def reserve(self, nbytes: int) -> None:
        """Grow the context's device scratch now (before a HIP graph capture)."""
        check(lib().g4_ctx_reserve(self.handle, int(nbytes)))

    def scratch_bytes(self) -> int:
        v = _i64()
        check(lib().g4_ctx_scratch_bytes(self.handle, ctypes.byref(v)))
        return v.value

    def close(self) -> None:
        if self.handle:
            check(lib().g4_close(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ----------------------------------------------------------------- tensor ---


class FloatTensor:
    """Shape of the reference's FloatTensor interface (FloatTensor.kt:5-71)."""

    size: int

    def get(self, index: int) -> float:
        raise NotImplementedError

    def dot(self, this_offset: int, that: np.ndarray, that_offset: int, size: int) -> float:
        raise NotImplementedError

    def matmul(self, that: np.ndarray, out: np.ndarray, dim0: int, dim1: int, this_offset: int = 0) -> None:
        raise NotImplementedError


class GpuFloatTensor(FloatTensor):
    """Raw GGUF blocks resident in HBM; every matmul runs on the GPU."""

    def __init__(self, ctx: Context, ggml_type: int, raw, n_elems: int):
        self.ctx = ctx
        self.ggml_type = GGMLType(ggml_type) if int(ggml_type) in [t.value for t in GGMLType] else int(ggml_type)
        self.size = int(n_elems)
        buf = np.ascontiguousarray(np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray))
                                   else raw.view(np.uint8).reshape(-1))
        h = _vp()
        check(lib().g4_upload(ctx.handle, int(ggml_type), buf.ctypes.data if buf.size else None,
                              int(buf.size), int(n_elems), ctypes.byref(h)))
        self.handle = h.value
        self.nbytes = int(buf.size)

    def free(self) -> None:
        if getattr(self, "handle", None):
            check(lib().g4_weight_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def device_ptr(self) -> int:
        p = _vp()
        check(lib().g4_weight_device_ptr(self.handle, ctypes.byref(p)))
        return p.value

    # -- get / copyTo (Q8_0FloatTensor.kt:21-28 etc.) --
    def get(self, index: int) -> float:
        return float(self.dequant(index, 1)[0])

    def dequant(self, offset: int, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        check(lib().g4_dequant(self.ctx.handle, self.handle, int(offset), int(n), _ptr(out) if n else None))
        return out

    def dequant_dev(self, offset: int, n: int, out) -> None:
        check(lib().g4_dequant_dev(self.ctx.handle, self.handle, int(offset), int(n), _ptr(_dev_f32(out, "out"))))

    # -- FloatTensor.dot (FloatTensor.kt:14-16): activation offset applied on the host side --
    def dot(self, this_offset: int, that: np.ndarray, that_offset: int, size: int) -> float:
        x = np.ascontiguousarray(_f32(that, "that")[that_offset:that_offset + size])
        out = np.empty(1, dtype=np.float32)
        self.matmul(x, out, 1, size, this_offset)
        return float(out[0])

    # -- FloatTensor.matmul (FloatTensor.kt:18-29) --
    def matmul(self, that: np.ndarray, out: np.ndarray, dim0: int, dim1: int, this_offset: int = 0) -> None:
        _f32(that, "that")
        _f32(out, "out")
        if that.size < dim1 or out.size < dim0:
            raise IndexOutOfBoundsException("that/out shorter than dim1/dim0")
        check(lib().g4_matmul(self.ctx.handle, self.handle, int(this_offset), _ptr(that), _ptr(out),
                              int(dim0), int(dim1)))

    def matmul_dev(self, that, out, dim0: int, dim1: int, this_offset: int = 0) -> None:
        check(lib().g4_matmul_dev(self.ctx.handle, self.handle, int(this_offset), _ptr(_dev_f32(that, "that")),
                                  _ptr(_dev_f32(out, "out")), int(dim0), int(dim1)))

    def matmul_batch(self, X: np.ndarray, dim0: int, dim1: int, this_offset: int = 0) -> np.ndarray:
        X = _f32(np.ascontiguousarray(X, dtype=np.float32), "X")
        M = X.size // dim1 if dim1 else 0
        Y = np.empty((M, dim0), dtype=np.float32)
        check(lib().g4_matmul_batch(self.ctx.handle, self.handle, int(this_offset), _ptr(X), int(M), _ptr(Y),
                                    int(dim0), int(dim1)))
        return Y

    def matmul_batch_dev(self, X, M: int, Y, dim0: int, dim1: int, this_offset: int = 0) -> None:
        check(lib().g4_matmul_batch_dev(self.ctx.handle, self.handle, int(this_offset), _ptr(_dev_f32(X, "X")),
                                        int(M), _ptr(_dev_f32(Y, "Y")), int(dim0), int(dim1)))

    # -- LM head: matmul + FloatTensor.argmax (Llama.kt:402, Sampler ARGMAX) --
    def matmul_argmax(self, that: np.ndarray, dim0: int, dim1: int, this_offset: int = 0,
                      logits: Optional[np.ndarray] = None) -> int:
        _f32(that, "that")
        _need(that, dim1, "that")
        if logits is not None:
            _f32(logits, "logits")
            _need(logits, dim0, "logits")
        idx = np.zeros(1, dtype=np.int32)
        check(lib().g4_matmul_argmax(self.ctx.handle, self.handle, int(this_offset), _ptr(that), _ptr(logits),
                                     _ptr(idx), int(dim0), int(dim1)))
        return int(idx[0])

    def matmul_argmax_dev(self, that, logits, index, dim0: int, dim1: int, this_offset: int = 0) -> None:
        check(lib().g4_matmul_argmax_dev(self.ctx.handle, self.handle, int(this_offset),
                                         _ptr(_dev_f32(that, "that")), _ptr(_dev_f32(logits, "logits")),
                                         _ptr(_dev_i32(index, "index")), int(dim0), int(dim1)))


class FloatTensorFactory:
    """FloatTensorFactory.kt:7-23: one tensor object per GGML type id."""

    @staticmethod
    def create(ctx: Context, ggml_type: int, raw, n_elems: Optional[int] = None) -> GpuFloatTensor:
        """create(ctx, type, raw_bytes, n_elems), or create(ctx, type, entry) with a
        GGMLTensorEntry of gguf.py (n_elems = the product of its shape, as
        FloatTensorFactory.kt:8 computes it; the entry's mapped bytes are uploaded)."""
        if n_elems is None:
            if not hasattr(raw, "memory_segment"):
                raise IllegalArgumentException("n_elems is required for raw bytes")
            n = 1
            for d in raw.shape:
                n *= int(d)
            return GpuFloatTensor(ctx, ggml_type, raw.memory_segment, n)
        return GpuFloatTensor(ctx, ggml_type, raw, n_elems)


# ------------------------------------------------------ free functions ---


def argmax(ctx: Context, v: np.ndarray) -> int:
    """FloatTensor.argmax(0, size) (FloatTensor.kt:53-66)."""
    _f32(v, "v")
    idx = np.zeros(1, dtype=np.int32)
    check(lib().g4_argmax(ctx.handle, _ptr(v), int(v.size), _ptr(idx)))
    return int(idx[0])


def ffn(ctx: Context, gate: GpuFloatTensor, up: GpuFloatTensor, down: GpuFloatTensor, x: np.ndarray,
        dim: int, hidden: int) -> np.ndarray:
    """y = down(gelu(gate x) * up x) (Llama.kt:357-361)."""
    _f32(x, "x")
    _need(x, dim, "x")
    y = np.empty(dim, dtype=np.float32)
    check(lib().g4_ffn(ctx.handle, gate.handle, up.handle, down.handle, _ptr(x), _ptr(y), int(dim), int(hidden)))
    return y


def ffn_dev(ctx: Context, gate, up, down, x, y, dim: int, hidden: int) -> None:
    check(lib().g4_ffn_dev(ctx.handle, gate.handle, up.handle, down.handle, _ptr(_dev_f32(x, "x")),
                           _ptr(_dev_f32(y, "y")), int(dim), int(hidden)))


def ffn_gate_up(ctx: Context, gate: GpuFloatTensor, up: GpuFloatTensor, x: np.ndarray, dim: int,
                hidden: int) -> np.ndarray:
    """h = gelu(gate x) * (up x) (Llama.kt:357-360)."""
    _f32(x, "x")
    _need(x, dim, "x")
    h = np.empty(hidden, dtype=np.float32)
    check(lib().g4_ffn_gate_up(ctx.handle, gate.handle, up.handle, _ptr(x), _ptr(h), int(dim), int(hidden)))
    return h


def ffn_gate_up_dev(ctx: Context, gate, up, x, h, dim: int, hidden: int) -> None:
    check(lib().g4_ffn_gate_up_dev(ctx.handle, gate.handle, up.handle, _ptr(_dev_f32(x, "x")),
                                   _ptr(_dev_f32(h, "h")), int(dim), int(hidden)))


def moe_route(ctx: Context, logits: np.ndarray, k: int, renormalize: bool,
              expert_scale: Optional[np.ndarray] = None):
    """Softmax + top-k routing of Llama.kt:269-293 for logits [T x n_experts]."""
    logits = _f32(np.ascontiguousarray(logits, dtype=np.float32), "logits")
    T, E = logits.shape
    ids = np.zeros((T, k), dtype=np.int32)
    w = np.zeros((T, k), dtype=np.float32)
    if expert_scale is not None:
        _f32(expert_scale, "expert_scale")
        _need(expert_scale, E, "expert_scale")
    check(lib().g4_moe_route(ctx.handle, _ptr(logits), int(T), int(E), int(k), int(bool(renormalize)),
                             _ptr(expert_scale), _ptr(ids), _ptr(w)))
    return ids, w


def moe_route_dev(ctx: Context, logits, T: int, n_experts: int, k: int, renormalize: bool, ids, weights,
                  expert_scale=None) -> None:
    check(lib().g4_moe_route_dev(ctx.handle, _ptr(_dev_f32(logits, "logits")), int(T), int(n_experts), int(k),
                                 int(bool(renormalize)), _ptr(_dev_f32(expert_scale, "expert_scale")),
                                 _ptr(_dev_i32(ids, "ids")), _ptr(_dev_f32(weights, "weights"))))


def moe(ctx: Context, gate_up: GpuFloatTensor, down: GpuFloatTensor, X: np.ndarray, ids: np.ndarray,
        weights: np.ndarray, dim: int, ff: int) -> np.ndarray:
    """Routed expert FFN (Llama.kt:300-337) for X [T x dim], ids/weights [T x k]."""
    X = _f32(np.ascontiguousarray(X, dtype=np.float32), "X")
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = _f32(np.ascontiguousarray(weights, dtype=np.float32), "weights")
    T = X.size // dim
    if X.size != T * dim:
        raise IllegalArgumentException("X holds %d floats, not a whole number of dim %d rows" % (X.size, dim))
    k = ids.size // T if T else 0
    if ids.size != T * k or weights.size != ids.size:
        raise IndexOutOfBoundsException("ids (%d) and weights (%d) must hold T*k entries for T = %d"
                                        % (ids.size, weights.size, T))
    Y = np.empty((T, dim), dtype=np.float32)
    check(lib().g4_moe(ctx.handle, gate_up.handle, down.handle, _ptr(X), int(T), int(dim), int(ff), _ptr(ids),
                       _ptr(weights), int(k), _ptr(Y)))
    return Y


def moe_dev(ctx: Context, gate_up, down, X, T: int, dim: int, ff: int, ids, weights, k: int, Y) -> None:
    check(lib().g4_moe_dev(ctx.handle, gate_up.handle, down.handle, _ptr(_dev_f32(X, "X")), int(T), int(dim),
                           int(ff), _ptr(_dev_i32(ids, "ids")), _ptr(_dev_f32(weights, "weights")), int(k),
                           _ptr(_dev_f32(Y, "Y"))))


def moe_routed(ctx: Context, gate_up: GpuFloatTensor, down: GpuFloatTensor, X: np.ndarray, logits: np.ndarray,
               k: int, renormalize: bool, dim: int, ff: int, expert_scale: Optional[np.ndarray] = None):
    """The MoE block of Llama.kt:269-337 from router logits [T x n_experts]:
    routing, expert FFN and weighted sum in one call.  Returns (Y, ids, weights)."""
    X = _f32(np.ascontiguousarray(X, dtype=np.float32), "X")
    logits = _f32(np.ascontiguousarray(logits, dtype=np.float32), "logits")
    T, E = logits.shape
    if X.size != T * dim:
        raise ValueError("X holds %d floats, %d tokens x dim %d need %d" % (X.size, T, dim, T * dim))
    if expert_scale is not None:
        expert_scale = _f32(np.ascontiguousarray(expert_scale, dtype=np.float32), "expert_scale")
        _need(expert_scale, E, "expert_scale")
    ids = np.zeros((T, k), dtype=np.int32)
    w = np.zeros((T, k), dtype=np.float32)
    Y = np.empty((T, dim), dtype=np.float32)
    check(lib().g4_moe_routed(ctx.handle, gate_up.handle, down.handle, _ptr(X), int(T), int(dim), int(ff),
                              _ptr(logits), int(E), int(k), int(bool(renormalize)), _ptr(expert_scale), _ptr(ids),
                              _ptr(w), _ptr(Y)))
    return Y, ids, w


def moe_routed_dev(ctx: Context, gate_up, down, X, T: int, dim: int, ff: int, logits, n_experts: int, k: int,
                   renormalize: bool, ids, weights, Y, expert_scale=None) -> None:
    check(lib().g4_moe_routed_dev(ctx.handle, gate_up.handle, down.handle, _ptr(_dev_f32(X, "X")), int(T),
                                  int(dim), int(ff), _ptr(_dev_f32(logits, "logits")), int(n_experts), int(k),
                                  int(bool(renormalize)), _ptr(_dev_f32(expert_scale, "expert_scale")),
                                  _ptr(_dev_i32(ids, "ids")),
                                  _ptr(_dev_f32(weights, "weights")), _ptr(_dev_f32(Y, "Y"))))


def moe_routed_dev_noalloc(ctx: Context, gate_up, down, X, T: int, dim: int, ff: int, logits, n_experts: int, k: int,
                           renormalize: bool, ids, weights, Y, expert_scale=None) -> None:
    """moe_routed_dev with its intermediates in the library's fixed per-GPU scratch
    (no device allocation; calls overlapping on one GPU race)."""
    check(lib().g4_moe_routed_dev_noalloc(ctx.handle, gate_up.handle, down.handle, _ptr(_dev_f32(X, "X")), int(T),
                                          int(dim), int(ff), _ptr(_dev_f32(logits, "logits")), int(n_experts), int(k),
                                          int(bool(renormalize)), _ptr(_dev_f32(expert_scale, "expert_scale")),
                                          _ptr(_dev_i32(ids, "ids")), _ptr(_dev_f32(weights, "weights")),
                                          _ptr(_dev_f32(Y, "Y"))))


# ------------------------------------------------------------ decode step ---
# The element-wise work around the matvec (Llama.kt:27-78 rmsnorm,
# MutableFloatTensor.kt:28-37 addInPlace, Llama.kt:403-406 soft-capping) and the
# blocks that keep the activations in device memory.  Norm weights are F32
# tensors uploaded with FloatTensorFactory.create (ModelLoader.kt:281-286).

NORM_WEIGHT_AFTER = 0   # Llama.kt:27-37: w * (s * x)
NORM_WEIGHT_FIRST = 1   # Llama.kt:39-60: w * s * x
NORM_NO_WEIGHT = 2      # Llama.kt:62-78: s * x


def rmsnorm_dev(ctx: Context, weight: Optional[GpuFloatTensor], x, out, n_vec: int, size: int, eps: float,
                form: int = NORM_WEIGHT_AFTER) -> None:
    """n_vec vectors of `size` floats, each normalised on its own (out may be x)."""
    check(lib().g4_rmsnorm_dev(ctx.handle, weight.handle if weight is not None else None, _ptr(_dev_f32(x, "x")),
                               _ptr(_dev_f32(out, "out")), int(n_vec), int(size), float(eps), int(form)))


def rmsnorm_add_dev(ctx: Context, weight: GpuFloatTensor, v, x, size: int, eps: float) -> None:
    """v = rmsnorm(v); x += v (Llama.kt:222-223, 362-363)."""
    check(lib().g4_rmsnorm_add_dev(ctx.handle, weight.handle, _ptr(_dev_f32(v, "v")), _ptr(_dev_f32(x, "x")),
                                   int(size), float(eps)))


def add_dev(ctx: Context, x, that, n: int) -> None:
    """x += that (MutableFloatTensor.kt:28-37)."""
    check(lib().g4_add_dev(ctx.handle, _ptr(_dev_f32(x, "x")), _ptr(_dev_f32(that, "that")), int(n)))


def softcap_dev(ctx: Context, v, n: int, cap: float) -> None:
    """v = cap * tanh(v / cap) (Llama.kt:403-406)."""
    check(lib().g4_softcap_dev(ctx.handle, _ptr(_dev_f32(v, "v")), int(n), float(cap)))


def matmul_norm_dev(ctx: Context, w: GpuFloatTensor, norm: GpuFloatTensor, x, out, dim0: int, dim1: int,
                    eps: float, this_offset: int = 0, xnorm=None) -> None:
    """out = W . rmsnorm(x, norm) with the norm fused into the matvec (Llama.kt:155-158)."""
    check(lib().g4_matmul_norm_dev(ctx.handle, w.handle, int(this_offset), norm.handle, _ptr(_dev_f32(x, "x")),
                                   float(eps), _ptr(_dev_f32(xnorm, "xnorm")), _ptr(_dev_f32(out, "out")),
                                   int(dim0), int(dim1)))


def ffn_block(ctx: Context, gate: GpuFloatTensor, up: GpuFloatTensor, down: GpuFloatTensor,
              norm_pre: GpuFloatTensor, norm_post: GpuFloatTensor, x: np.ndarray, dim: int, hidden: int,
              eps: float) -> np.ndarray:
    """Dense FFN block of Llama.kt:355-363; returns the updated residual stream x."""
    x = _f32(np.array(x, dtype=np.float32, copy=True), "x")
    _need(x, dim, "x")
    check(lib().g4_ffn_block(ctx.handle, gate.handle, up.handle, down.handle, norm_pre.handle, norm_post.handle,
                             _ptr(x), int(dim), int(hidden), float(eps)))
    return x


def ffn_block_dev(ctx: Context, gate, up, down, norm_pre, norm_post, x, dim: int, hidden: int, eps: float) -> None:
    check(lib().g4_ffn_block_dev(ctx.handle, gate.handle, up.handle, down.handle, norm_pre.handle,
                                 norm_post.handle, _ptr(_dev_f32(x, "x")), int(dim), int(hidden), float(eps)))


def lm_head(ctx: Context, w_cls: GpuFloatTensor, norm_final: GpuFloatTensor, x: np.ndarray, vocab: int, dim: int,
            eps: float, softcap: float, want_logits: bool = True):
    """Llama.kt:401-407 then Sampler.ARGMAX: (logits or None, index)."""
    _f32(x, "x")
    _need(x, dim, "x")
    logits = np.empty(vocab, dtype=np.float32) if want_logits else None
    idx = np.zeros(1, dtype=np.int32)
    check(lib().g4_lm_head(ctx.handle, w_cls.handle, norm_final.handle, _ptr(x), _ptr(logits), _ptr(idx),
                           int(vocab), int(dim), float(eps), float(softcap)))
    return logits, int(idx[0])


def lm_head_dev(ctx: Context, w_cls, norm_final, x, logits, index, vocab: int, dim: int, eps: float,
                softcap: float, xnorm=None) -> None:
    check(lib().g4_lm_head_dev(ctx.handle, w_cls.handle, norm_final.handle, _ptr(_dev_f32(x, "x")),
                               _ptr(_dev_f32(xnorm, "xnorm")), _ptr(_dev_f32(logits, "logits")),
                               _ptr(_dev_i32(index, "index")),
                               int(vocab), int(dim), float(eps), float(softcap)))


def attention_dev(ctx: Context, q, key_cache, value_cache, out, n_heads: int, n_kv_heads: int, head_size: int,
                  position: int, att_start: int = 0) -> None:
    """Decode attention over one layer's KV cache (Llama.kt:198-218); device tensors."""
    check(lib().g4_attention_dev(ctx.handle, _ptr(_dev_f32(q, "q")), _ptr(_dev_f32(key_cache, "key_cache")),
                                 _ptr(_dev_f32(value_cache, "value_cache")), _ptr(_dev_f32(out, "out")),
                                 int(n_heads), int(n_kv_heads), int(head_size), int(position), int(att_start)))
