"""ctypes wrapper of liboracle (g4_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker of libg4hip.so.  Only tests/, the smoke
check and the CPU-baseline leg of bench.py load this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libg4oracle.so")

MODE_VECTOR, MODE_SCALAR = 0, 1

_vp, _i32, _i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
_SIG = {
    "or_block_size": ([ctypes.c_int], ctypes.c_int),
    "or_type_size": ([ctypes.c_int], ctypes.c_int),
    "or_fp16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
    "or_fp16_vec_decode": ([ctypes.c_uint16], ctypes.c_float),
    "or_bf16_to_f32": ([ctypes.c_uint16], ctypes.c_float),
    "or_fp16_to_f32_array": ([_vp, _i64, _vp], None),
    "or_fp16_vec_decode_array": ([_vp, _i64, _vp], None),
    "or_get": ([ctypes.c_int, _vp, _i64], ctypes.c_float),
    "or_dequant": ([ctypes.c_int, _vp, _i64, _i64, _vp], None),
    "or_q4k_scale_min": ([ctypes.c_int, _vp, ctypes.c_int], ctypes.c_int),
    "or_scalar_dot": ([ctypes.c_int, _vp, _i64, _vp, _i32], ctypes.c_float),
    "or_vector_dot": ([ctypes.c_int, _vp, _i64, _vp, _i32], ctypes.c_float),
    "or_dot": ([ctypes.c_int, _vp, _i64, _vp, _i32, ctypes.c_int], ctypes.c_float),
    "or_exact_dot": ([ctypes.c_int, _vp, _i64, _vp, _i32, _vp], ctypes.c_double),
    "or_matmul": ([ctypes.c_int, _vp, _i64, _vp, _vp, _i32, _i32, ctypes.c_int, ctypes.c_int], None),
    "or_matmul_exact": ([ctypes.c_int, _vp, _i64, _vp, _vp, _vp, _i32, _i32, ctypes.c_int], None),
    "or_argmax": ([_vp, _i32, _i32], _i32),
    "or_softmax": ([_vp, _i32, _i32], None),
    "or_topk": ([_vp, _i32, _i32, _vp, _vp], None),
    "or_route": ([_vp, _i32, _i32, ctypes.c_int, _vp, _vp, _vp], None),
    "or_gelu": ([ctypes.c_float], ctypes.c_float),
    "or_tanh": ([ctypes.c_double], ctypes.c_double),
    "or_moe": ([ctypes.c_int, _vp, ctypes.c_int, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _i32, _vp, ctypes.c_int,
                ctypes.c_int], None),
    "or_moe_exact": ([ctypes.c_int, _vp, ctypes.c_int, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _i32, _vp, _vp,
                      ctypes.c_int], None),
    "or_rmsnorm": ([_vp, _vp, _vp, _i32, ctypes.c_float, ctypes.c_int], None),
    "or_rmsnorm_exact": ([_vp, _vp, _vp, _i32, ctypes.c_float], None),
    "or_softcap": ([_vp, _i32, ctypes.c_float], None),
    "or_ffn_block": ([ctypes.c_int, _vp, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp, _vp, _vp, _i32, _i32,
                      ctypes.c_float, ctypes.c_int, ctypes.c_int], None),
    "or_ffn_block_exact": ([ctypes.c_int, _vp, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                            _i32, _i32, ctypes.c_float, ctypes.c_int], None),
    "or_lm_head": ([ctypes.c_int, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                    ctypes.c_int], _i32),
    "or_lm_head_exact": ([ctypes.c_int, _vp, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, ctypes.c_float,
                          ctypes.c_int], None),
    "or_attention": ([_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32], None),
    "or_attention_exact": ([_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, ctypes.c_int], None),
}

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIG.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _u8(raw) -> np.ndarray:
    return np.ascontiguousarray(raw).view(np.uint8).reshape(-1)


def _f(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def nthreads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def block_size(t: int) -> int:
    return lib().or_block_size(t)


def type_size(t: int) -> int:
    return lib().or_type_size(t)


def fp16_to_f32(h: int) -> float:
    return lib().or_fp16_to_f32(h)


def fp16_vec_decode(h: int) -> float:
    return lib().or_fp16_vec_decode(h)


def bf16_to_f32(h: int) -> float:
    return lib().or_bf16_to_f32(h)


def fp16_to_f32_array(h) -> np.ndarray:
    hh = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(hh.size, dtype=np.float32)
    lib().or_fp16_to_f32_array(_p(hh), hh.size, _p(out))
    return out


def fp16_vec_decode_array(h) -> np.ndarray:
    hh = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(hh.size, dtype=np.float32)
    lib().or_fp16_vec_decode_array(_p(hh), hh.size, _p(out))
    return out


def get(t: int, raw, index: int) -> float:
    r = _u8(raw)
    return lib().or_get(t, _p(r), index)


def dequant(t: int, raw, offset: int, n: int) -> np.ndarray:
    r = _u8(raw)
    out = np.empty(n, dtype=np.float32)
    lib().or_dequant(t, _p(r), offset, n, _p(out))
    return out


def q4k_scale_min(j: int, scales12, is_min: bool) -> int:
    s = _u8(scales12)
    return lib().or_q4k_scale_min(j, _p(s), int(is_min))


def scalar_dot(t: int, raw, this_offset: int, x, size: int) -> float:
    r, xx = _u8(raw), _f(x)
    return lib().or_scalar_dot(t, _p(r), this_offset, _p(xx), size)


def vector_dot(t: int, raw, this_offset: int, x, size: int) -> float:
    r, xx = _u8(raw), _f(x)
    return lib().or_vector_dot(t, _p(r), this_offset, _p(xx), size)


def exact_dot(t: int, raw, this_offset: int, x, size: int):
    r, xx = _u8(raw), _f(x)
    a = ctypes.c_double()
    v = lib().or_exact_dot(t, _p(r), this_offset, _p(xx), size, ctypes.byref(a))
    return v, a.value


def matmul(t: int, raw, x, dim0: int, dim1: int, this_offset: int = 0, mode: int = MODE_VECTOR,
           threads: int = 0) -> np.ndarray:
    r, xx = _u8(raw), _f(x)
    out = np.empty(dim0, dtype=np.float32)
    lib().or_matmul(t, _p(r), this_offset, _p(xx), _p(out), dim0, dim1, mode, threads or nthreads())
    return out


def matmul_exact(t: int, raw, x, dim0: int, dim1: int, this_offset: int = 0, threads: int = 0):
    r, xx = _u8(raw), _f(x)
    out = np.empty(dim0, dtype=np.float64)
    ab = np.empty(dim0, dtype=np.float64)
    lib().or_matmul_exact(t, _p(r), this_offset, _p(xx), _p(out), _p(ab), dim0, dim1, threads or nthreads())
    return out, ab


def argmax(v, offset: int = 0, size: int = -1) -> int:
    vv = _f(v)
    if size < 0:
        size = vv.size - offset
    return lib().or_argmax(_p(vv), offset, size)


def softmax(v) -> np.ndarray:
    vv = _f(v).copy()
    lib().or_softmax(_p(vv), 0, vv.size)
    return vv


def topk(probs, k: int):
    p = _f(probs).copy()
    idx = np.empty(k, dtype=np.int32)
    val = np.empty(k, dtype=np.float32)
    lib().or_topk(_p(p), p.size, k, _p(idx), _p(val))
    return idx, val, p


def route(logits, k: int, renormalize: bool, expert_scale=None):
    lg = _f(logits)
    T, E = lg.shape
    ids = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    sc = _f(expert_scale) if expert_scale is not None else None
    for t in range(T):
        row = np.ascontiguousarray(lg[t])
        oi = np.empty(k, dtype=np.int32)
        ow = np.empty(k, dtype=np.float32)
        lib().or_route(_p(row), E, k, int(bool(renormalize)), _p(sc) if sc is not None else None, _p(oi), _p(ow))
        ids[t], w[t] = oi, ow
    return ids, w


def gelu(x: float) -> float:
    return lib().or_gelu(x)


def tanh(x: float) -> float:
    """Math.tanh by fdlibm's tanh steps over the C library's expm1 (within 2 ulps of tanh)."""
    return lib().or_tanh(x)


def moe(t_gu: int, gate_up, t_dn: int, down, X, ids, w, dim: int, ff: int, mode: int = MODE_VECTOR,
        threads: int = 0) -> np.ndarray:
    gu, dn, XX = _u8(gate_up), _u8(down), _f(X)
    ii = np.ascontiguousarray(ids, dtype=np.int32)
    ww = _f(w)
    T = XX.size // dim
    k = ii.size // T
    Y = np.empty((T, dim), dtype=np.float32)
    lib().or_moe(t_gu, _p(gu), t_dn, _p(dn), dim, ff, _p(XX), T, _p(ii), _p(ww), k, _p(Y), mode,
                 threads or nthreads())
    return Y


def moe_exact(t_gu: int, gate_up, t_dn: int, down, X, ids, w, dim: int, ff: int, threads: int = 0):
    gu, dn, XX = _u8(gate_up), _u8(down), _f(X)
    ii = np.ascontiguousarray(ids, dtype=np.int32)
    ww = _f(w)
    T = XX.size // dim
    k = ii.size // T
    Y = np.empty((T, dim), dtype=np.float64)
    B = np.empty((T, dim), dtype=np.float64)
    lib().or_moe_exact(t_gu, _p(gu), t_dn, _p(dn), dim, ff, _p(XX), T, _p(ii), _p(ww), k, _p(Y), _p(B),
                       threads or nthreads())
    return Y, B


NORM_WEIGHT_AFTER, NORM_WEIGHT_FIRST, NORM_NO_WEIGHT = 0, 1, 2


def rmsnorm(x, w, eps: float, form: int = NORM_WEIGHT_AFTER) -> np.ndarray:
    """Llama.kt:27-78 over one vector (w may be None for NORM_NO_WEIGHT)."""
    xx = _f(x)
    ww = _f(w) if w is not None else None
    out = np.empty(xx.size, dtype=np.float32)
    lib().or_rmsnorm(_p(out), _p(xx), _p(ww) if ww is not None else None, xx.size, eps, form)
    return out


def rmsnorm_exact(x, w, eps: float) -> np.ndarray:
    xx = _f(x)
    ww = _f(w) if w is not None else None
    out = np.empty(xx.size, dtype=np.float64)
    lib().or_rmsnorm_exact(_p(out), _p(xx), _p(ww) if ww is not None else None, xx.size, eps)
    return out


def softcap(v, cap: float) -> np.ndarray:
    vv = _f(v).copy()
    lib().or_softcap(_p(vv), vv.size, cap)
    return vv


def ffn_block(t_g: int, gate, t_u: int, up, t_d: int, down, norm_pre, norm_post, x, dim: int, hidden: int,
              eps: float, mode: int = MODE_VECTOR, threads: int = 0) -> np.ndarray:
    g, u, d = _u8(gate), _u8(up), _u8(down)
    npre, npost = _f(norm_pre), _f(norm_post)
    xx = _f(x).copy()
    lib().or_ffn_block(t_g, _p(g), t_u, _p(u), t_d, _p(d), _p(npre), _p(npost), _p(xx), dim, hidden, eps, mode,
                       threads or nthreads())
    return xx


def ffn_block_exact(t_g: int, gate, t_u: int, up, t_d: int, down, norm_pre, norm_post, x, dim: int, hidden: int,
                    eps: float, threads: int = 0):
    g, u, d = _u8(gate), _u8(up), _u8(down)
    npre, npost, xx = _f(norm_pre), _f(norm_post), _f(x)
    x64 = np.empty(dim, dtype=np.float64)
    b64 = np.empty(dim, dtype=np.float64)
    lib().or_ffn_block_exact(t_g, _p(g), t_u, _p(u), t_d, _p(d), _p(npre), _p(npost), _p(xx), _p(x64), _p(b64),
                             dim, hidden, eps, threads or nthreads())
    return x64, b64


def lm_head(t: int, raw, norm, x, vocab: int, dim: int, eps: float, cap: float, mode: int = MODE_VECTOR,
            threads: int = 0):
    r, nn, xx = _u8(raw), _f(norm), _f(x)
    logits = np.empty(vocab, dtype=np.float32)
    idx = lib().or_lm_head(t, _p(r), _p(nn), _p(xx), _p(logits), vocab, dim, eps, cap, mode, threads or nthreads())
    return logits, idx


def lm_head_exact(t: int, raw, norm, x, vocab: int, dim: int, eps: float, cap: float, threads: int = 0):
    r, nn, xx = _u8(raw), _f(norm), _f(x)
    l64 = np.empty(vocab, dtype=np.float64)
    b64 = np.empty(vocab, dtype=np.float64)
    lib().or_lm_head_exact(t, _p(r), _p(nn), _p(xx), _p(l64), _p(b64), vocab, dim, eps, cap,
                           threads or nthreads())
    return l64, b64


def attention(q, kc, vc, n_heads: int, n_kv: int, hs: int, position: int, att_start: int = 0) -> np.ndarray:
    """Llama.kt:198-218 for one layer at one position: out [n_heads x hs]."""
    qq, kk, vv = _f(q), _f(kc), _f(vc)
    out = np.empty(n_heads * hs, dtype=np.float32)
    lib().or_attention(_p(qq), _p(kk), _p(vv), _p(out), n_heads, n_kv, hs, position, att_start)
    return out.reshape(n_heads, hs)


def attention_exact(q, kc, vc, n_heads: int, n_kv: int, hs: int, position: int, att_start: int = 0,
                    threads: int = 0):
    qq, kk, vv = _f(q), _f(kc), _f(vc)
    o = np.empty(n_heads * hs, dtype=np.float64)
    b = np.empty(n_heads * hs, dtype=np.float64)
    lib().or_attention_exact(_p(qq), _p(kk), _p(vv), _p(o), _p(b), n_heads, n_kv, hs, position, att_start,
                             threads or nthreads())
    return o.reshape(n_heads, hs), b.reshape(n_heads, hs)
