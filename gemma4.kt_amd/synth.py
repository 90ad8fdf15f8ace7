"""Seeded synthetic GGUF workloads for the quantized matrix-vector path.

Every buffer is a pure function of (seed, tag, index): a counter-based
splitmix64 stream, so any slice of a large tensor can be produced on its own and
two hosts always produce the same bytes.  Normal deviates come from Box-Muller
with log and cos evaluated by fixed polynomials in IEEE basic arithmetic only
(no libm / SIMD-library transcendental), so the result does not depend on the
numpy build or the host CPU.

Block layouts written here are the GGUF ones the reference reads:
  Q8_0  34 B / 32 weights : fp16 d, int8 q[32]          (Q8_0FloatTensor.kt:21-28)
  Q4_0  18 B / 32 weights : fp16 d, 16 B nibbles        (Q4_0FloatTensor.kt:21-39)
  Q4_K 144 B / 256 weights: fp16 d, fp16 dmin, 12 B packed 6-bit scales/mins,
                            128 B nibbles               (Q4_KFloatTensor.kt:23-84)
  Q5_K 176 B / 256 weights: as Q4_K plus 32 B of fifth bits before the nibbles
                                                        (Q5_KFloatTensor.kt:23-50)
  Q6_K 210 B / 256 weights: 128 B low nibbles, 64 B high bit pairs, int8
                            scales[16], fp16 d          (Q6_KFloatTensor.kt:26-75)
"""
from __future__ import annotations

import numpy as np

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_BF16 = 0, 1, 2, 8, 12, 13, 14, 30

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22  # counters generated per numpy pass (bounds temporary memory)


def _mix(z: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser (Steele, Lea, Flood 2014), vectorised, wrapping, in place."""
    z ^= z >> np.uint64(30)
    z *= _M1
    z ^= z >> np.uint64(27)
    z *= _M2
    z ^= z >> np.uint64(31)
    return z


def _tag_hash(tag: str) -> int:
    h = 0xCBF29CE484222325  # FNV-1a 64
    for b in tag.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def u64(seed: int, tag: str, start: int, n: int) -> np.ndarray:
    """Words start .. start+n-1 of the stream (seed, tag)."""
    with np.errstate(over="ignore"):
        base = _mix(np.array([(seed * 0x9E3779B97F4A7C15 ^ _tag_hash(tag)) & 0xFFFFFFFFFFFFFFFF],
                             dtype=np.uint64))[0]
        out = np.empty(n, dtype=np.uint64)
        for s in range(0, n, _CHUNK):
            e = min(n, s + _CHUNK)
            c = np.arange(start + s + 1, start + e + 1, dtype=np.uint64)
            c *= _GOLDEN
            c += base
            out[s:e] = _mix(c)
    return out


def random_bytes(seed: int, tag: str, nbytes: int) -> np.ndarray:
    words = u64(seed, tag, 0, (nbytes + 7) // 8)
    return words.astype("<u8", copy=False).view(np.uint8)[:nbytes].copy()


def _log_unit(u: np.ndarray) -> np.ndarray:
    """ln(u) for u in (0, 1]: frexp split and the atanh series, 16 terms."""
    m, e = np.frexp(u)  # u = m * 2^e, m in [0.5, 1)
    s = (m - 1.0) / (m + 1.0)  # |s| <= 1/3
    s2 = s * s
    acc = np.full_like(s, 1.0 / 31.0)
    for k in range(14, -1, -1):
        acc = acc * s2 + 1.0 / (2 * k + 1)
    return e.astype(np.float64) * 0.6931471805599453 + 2.0 * s * acc


def _cos_coef() -> list:
    out, f = [], 1.0
    facts = [1.0]
    for i in range(1, 41):
        f *= i
        facts.append(f)
    for k in range(20, -1, -1):
        out.append(((-1.0) ** k) / facts[2 * k])
    return out


_COS_COEF = _cos_coef()


def _cos_2pi(u: np.ndarray) -> np.ndarray:
    """cos(2*pi*u) for u in [0, 1): -cos(t) with t = 2*pi*u - pi in [-pi, pi), Taylor in t^2."""
    t = u * 6.283185307179586 - 3.141592653589793
    t2 = t * t
    acc = np.zeros_like(t)
    for c in _COS_COEF:
        acc *= t2
        acc += c
    return -acc


def normal(seed: int, tag: str, n: int) -> np.ndarray:
    """n standard normal deviates (float64), Box-Muller over word pairs."""
    w = u64(seed, tag, 0, 2 * n).reshape(n, 2)
    u1 = ((w[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (w[:, 1] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    return np.sqrt(-2.0 * _log_unit(u1)) * _cos_2pi(u2)


def fp16_bits(v: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float64 -> binary16 bits."""
    return np.asarray(v, dtype=np.float64).astype(np.float16).view(np.uint16)


def bf16_bits(v: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bits (finite inputs)."""
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint16)


def activations(seed: int, tag: str, n: int, scale: float = 1.0) -> np.ndarray:
    return (normal(seed, tag, n) * scale).astype(np.float32)


# ------------------------------------------------------------------ blocks ---

def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Pack 8 six-bit scales and mins per super-block into the 12-byte GGUF
    field read by getScaleMinK4 (Q4_KFloatTensor.kt:70-84).  sc, m: [nsb, 8]."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    s = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    for j in range(4):
        s[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        s[:, j + 4] = (m[:, j] & 63) | ((m[:, j + 4] >> 4) << 6)
        s[:, j + 8] = (sc[:, j + 4] & 0xF) | ((m[:, j + 4] & 0xF) << 4)
    return s


# byte b -> int8 ((b * 255) >> 8) - 127, i.e. uniform over [-127, 127]
_Q8_LUT = (((np.arange(256, dtype=np.int32) * 255) >> 8) - 127).astype(np.int8).view(np.uint8)


def q8_0(seed: int, tag: str, n_elems: int, dscale: float = 0.02) -> np.ndarray:
    """Q8_0 blocks: d = fp16(|N(0,1)| * dscale), q uniform in [-127, 127]."""
    assert n_elems % 32 == 0
    nb = n_elems // 32
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, 0:2] = fp16_bits(np.abs(normal(seed, tag + ".d", nb)) * dscale).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = _Q8_LUT[random_bytes(seed, tag + ".q", nb * 32)].reshape(nb, 32)
    return out.reshape(-1)


def q4_0(seed: int, tag: str, n_elems: int, dscale: float = 0.05) -> np.ndarray:
    """Q4_0 blocks: d = fp16(|N(0,1)| * dscale), nibbles uniform in 0..15."""
    assert n_elems % 32 == 0
    nb = n_elems // 32
    out = np.empty((nb, 18), dtype=np.uint8)
    out[:, 0:2] = fp16_bits(np.abs(normal(seed, tag + ".d", nb)) * dscale).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = random_bytes(seed, tag + ".q", nb * 16).reshape(nb, 16)
    return out.reshape(-1)


def q4_k(seed: int, tag: str, n_elems: int, dscale: float = 0.01) -> np.ndarray:
    """Q4_K super-blocks: d, dmin = fp16(|N(0,1)| * dscale), 6-bit scales and
    mins uniform in 0..63, nibbles uniform in 0..15."""
    assert n_elems % 256 == 0
    nb = n_elems // 256
    out = np.empty((nb, 144), dtype=np.uint8)
    out[:, 0:2] = fp16_bits(np.abs(normal(seed, tag + ".d", nb)) * dscale).view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = fp16_bits(np.abs(normal(seed, tag + ".dmin", nb)) * dscale).view(np.uint8).reshape(nb, 2)
    sm = random_bytes(seed, tag + ".sm", nb * 16).reshape(nb, 16) & 63
    out[:, 4:16] = pack_q4k_scales(sm[:, :8], sm[:, 8:])
    out[:, 16:] = random_bytes(seed, tag + ".q", nb * 128).reshape(nb, 128)
    return out.reshape(-1)


def q5_k(seed: int, tag: str, n_elems: int, dscale: float = 0.01) -> np.ndarray:
    """Q5_K super-blocks (176 B): d, dmin = fp16(|N(0,1)| * dscale), 6-bit
    scales and mins uniform in 0..63 (Q4_K packing), high bits and nibbles uniform."""
    assert n_elems % 256 == 0
    nb = n_elems // 256
    out = np.empty((nb, 176), dtype=np.uint8)
    out[:, 0:2] = fp16_bits(np.abs(normal(seed, tag + ".d", nb)) * dscale).view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = fp16_bits(np.abs(normal(seed, tag + ".dmin", nb)) * dscale).view(np.uint8).reshape(nb, 2)
    sm = random_bytes(seed, tag + ".sm", nb * 16).reshape(nb, 16) & 63
    out[:, 4:16] = pack_q4k_scales(sm[:, :8], sm[:, 8:])
    out[:, 16:] = random_bytes(seed, tag + ".q", nb * 160).reshape(nb, 160)
    return out.reshape(-1)


def q6_k(seed: int, tag: str, n_elems: int, dscale: float = 0.002) -> np.ndarray:
    """Q6_K super-blocks (210 B): 6-bit quants uniform (ql, qh bytes), int8
    scales uniform in -128..127, d = fp16(|N(0,1)| * dscale) at the end."""
    assert n_elems % 256 == 0
    nb = n_elems // 256
    out = np.empty((nb, 210), dtype=np.uint8)
    out[:, 0:208] = random_bytes(seed, tag + ".q", nb * 208).reshape(nb, 208)
    out[:, 208:210] = fp16_bits(np.abs(normal(seed, tag + ".d", nb)) * dscale).view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def dense(seed: int, tag: str, n_elems: int, ggml_type: int, scale: float = 0.05) -> np.ndarray:
    v = normal(seed, tag, n_elems) * scale
    if ggml_type == GGML_F32:
        return v.astype(np.float32).view(np.uint8)
    if ggml_type == GGML_F16:
        return fp16_bits(v).view(np.uint8)
    if ggml_type == GGML_BF16:
        return bf16_bits(v.astype(np.float32)).view(np.uint8)
    raise ValueError(ggml_type)


def weights(seed: int, tag: str, ggml_type: int, n_elems: int) -> np.ndarray:
    if ggml_type == GGML_Q8_0:
        return q8_0(seed, tag, n_elems)
    if ggml_type == GGML_Q4_0:
        return q4_0(seed, tag, n_elems)
    if ggml_type == GGML_Q4_K:
        return q4_k(seed, tag, n_elems)
    if ggml_type == GGML_Q5_K:
        return q5_k(seed, tag, n_elems)
    if ggml_type == GGML_Q6_K:
        return q6_k(seed, tag, n_elems)
    return dense(seed, tag, n_elems, ggml_type)


# ----------------------------------------------------------------- workloads ---
# Seeds are fixed per workload; sizes are the ones the workloads are quoted on.

SEED_Q8_0_MATVEC = 0x51A0
SEED_Q4_0_FFN = 0x51A1
SEED_Q8_0_LM_HEAD = 0x51A2
SEED_Q4_K_BATCHED = 0x51A3
SEED_MOE_Q4_K = 0x51A4


def q8_0_matvec_2048(seed: int = SEED_Q8_0_MATVEC) -> dict:
    """Q8_0 W 2048x2048, x ~ N(0,1)."""
    return dict(w=q8_0(seed, "w", 2048 * 2048), x=activations(seed, "x", 2048), dim0=2048, dim1=2048)


def q4_0_ffn(seed: int = SEED_Q4_0_FFN, dim: int = 2048, hidden: int = 8192) -> dict:
    """Q4_0 FFN of one decode token: gate/up W hidden x dim, down W dim x hidden."""
    return dict(gate=q4_0(seed, "gate", hidden * dim), up=q4_0(seed, "up", hidden * dim),
                down=q4_0(seed, "down", dim * hidden), x=activations(seed, "x", dim), dim=dim, hidden=hidden)


def q8_0_lm_head(seed: int = SEED_Q8_0_LM_HEAD, vocab: int = 262144, dim: int = 2048) -> dict:
    """Q8_0 LM head W vocab x dim, x ~ N(0,1) * 0.5."""
    return dict(w=q8_0(seed, "w", vocab * dim), x=activations(seed, "x", dim, 0.5), dim0=vocab, dim1=dim)


def q4_k_batched(m: int, seed: int = SEED_Q4_K_BATCHED, rows: int = 8192, cols: int = 2048) -> dict:
    """Q4_K W rows x cols and X [m x cols] ~ N(0,1)."""
    return dict(w=q4_k(seed, "w", rows * cols), x=activations(seed, "x%d" % m, m * cols).reshape(m, cols),
                dim0=rows, dim1=cols, m=m)


def norm_weight(seed: int, tag: str, n: int, scale: float = 1.0) -> np.ndarray:
    """An F32 rms-norm weight: scale * (1 + N(0,1) / 4)."""
    return (scale * (1.0 + 0.25 * normal(seed, tag, n))).astype(np.float32)


RMS_EPS = 1e-6        # gemma4.attention.layer_norm_rms_epsilon default (ModelLoader.kt:59)
LOGIT_SOFTCAP = 30.0  # a gemma4.final_logit_softcapping value (ModelLoader.kt:58)


def q4_0_ffn_block(seed: int = SEED_Q4_0_FFN, dim: int = 2048, hidden: int = 8192) -> dict:
    """The Q4_0 FFN above as a whole dense block (Llama.kt:355-363): the same
    weights plus pre/post norm weights, and a residual stream x ~ N(0,1) * 4."""
    d = q4_0_ffn(seed, dim, hidden)
    d.update(norm_pre=norm_weight(seed, "norm_pre", dim), norm_post=norm_weight(seed, "norm_post", dim),
             x=activations(seed, "x_resid", dim, 4.0), eps=RMS_EPS)
    return d


def q8_0_lm_head_block(seed: int = SEED_Q8_0_LM_HEAD, vocab: int = 262144, dim: int = 2048) -> dict:
    """The Q8_0 LM head above behind its final norm and soft-cap (Llama.kt:401-407):
    the same W and x, a final-norm weight of scale 0.05 (logits of standard
    deviation about 3, below the cap of 30)."""
    d = q8_0_lm_head(seed, vocab, dim)
    d.update(norm=norm_weight(seed, "norm_final", dim, 0.05), eps=RMS_EPS, cap=LOGIT_SOFTCAP)
    return d


_MOE_SLABS = {}


def moe_q4_k(tokens: int, seed: int = SEED_MOE_Q4_K, n_experts: int = 128, dim: int = 2048,
             ff: int = 1408, k: int = 8, routing_seed: int = 0) -> dict:
    """128 Q4_K experts (gate_up [E x 2ff x dim], down [E x dim x ff]), router
    logits ~ N(0,1) [tokens x E], X ~ N(0,1) [tokens x dim], top-k routing.
    routing_seed selects one of many independent routings/activations.  The
    expert slabs do not depend on the token count: they are generated once per
    shape and shared by later calls (read-only arrays)."""
    key = (seed, n_experts, dim, ff)
    if key not in _MOE_SLABS:
        gu = q4_k(seed, "gate_up", n_experts * 2 * ff * dim)
        dn = q4_k(seed, "down", n_experts * dim * ff)
        gu.flags.writeable = False
        dn.flags.writeable = False
        _MOE_SLABS.clear()
        _MOE_SLABS[key] = (gu, dn)
    gu, dn = _MOE_SLABS[key]
    return dict(gate_up=gu, down=dn,
                logits=activations(seed, "router%d.%d" % (tokens, routing_seed), tokens * n_experts)
                .reshape(tokens, n_experts),
                x=activations(seed, "x%d.%d" % (tokens, routing_seed), tokens * dim).reshape(tokens, dim),
                n_experts=n_experts, dim=dim, ff=ff, k=k, tokens=tokens)
