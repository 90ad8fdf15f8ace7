"""Independent numpy restatement of the GGUF block decodes (test helper).

Written from the published GGML block layouts, vectorised over whole tensors,
with no code shared with the C oracle: it is the second restatement that the
oracle's get() must agree with bit-for-bit (dequantised weights are unique in
fp32, so two correct restatements cannot differ).

Layouts (ggml, as read by the reference's *FloatTensor.get):
  Q8_0 block (34 B): d fp16 | q int8[32]                      w_i = q_i * d
  Q4_0 block (18 B): d fp16 | qs u8[16]; w_i = (nib_i - 8) * d, nib_i for
                     i < 16 = qs[i] & 15, for i >= 16 = qs[i-16] >> 4
  Q4_K super-block (144 B): d fp16 | dmin fp16 | scales u8[12] | qs u8[128];
                     4 groups of 64: group g reads qs[32g:32g+32], low nibbles
                     are its first 32 weights (sub-block 2g), high nibbles the
                     next 32 (sub-block 2g+1); w = (d*sc)*q - dmin*m.
                     The 12 scale bytes hold eight 6-bit (sc, m) pairs: pairs
                     0..3 in the low 6 bits of bytes 0..3 (sc) and 4..7 (m);
                     pairs 4..7 keep their low 4 bits in bytes 8..11 (sc low
                     nibble, m high nibble) and their top 2 bits in the top
                     2 bits of bytes 0..3 (sc) and 4..7 (m).
  Q5_K super-block (176 B): d fp16 | dmin fp16 | scales u8[12] (as Q4_K) |
                     qh u8[32] | qs u8[128]; group g as Q4_K with the 5th bit
                     of weight l of sub-block s = 2g + h in bit s of qh[l]:
                     w = (d*sc)*(nib + 16*bit) - dmin*m.
  Q6_K super-block (210 B): ql u8[128] | qh u8[64] | scales int8[16] | d fp16;
                     each 128-weight half n reads ql[64n:64n+64], qh[32n:32n+32],
                     scales[8n:8n+8]; for l < 32 its four 32-weight rows are
                     (ql[l] & 15, qh bits 0-1), (ql[l+32] & 15, bits 2-3),
                     (ql[l] >> 4, bits 4-5), (ql[l+32] >> 4, bits 6-7), the
                     6-bit value minus 32, row r, lane l scaled by
                     d * scales[2r + l // 16].
"""
from __future__ import annotations

import numpy as np


def _f16(b2: np.ndarray) -> np.ndarray:
    """[..., 2] uint8 little-endian -> float32 via numpy's float16."""
    return np.ascontiguousarray(b2).view(np.float16)[..., 0].astype(np.float32)


def dequant_q8_0(raw: np.ndarray) -> np.ndarray:
    blk = raw.reshape(-1, 34)
    d = _f16(blk[:, 0:2])
    q = blk[:, 2:].view(np.int8).astype(np.float32)
    return (q * d[:, None]).reshape(-1)


def dequant_q4_0(raw: np.ndarray) -> np.ndarray:
    blk = raw.reshape(-1, 18)
    d = _f16(blk[:, 0:2])
    qs = blk[:, 2:]
    nib = np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.int8) - np.int8(8)
    return (nib.astype(np.float32) * d[:, None]).reshape(-1)


def q4k_unpack_scales(sc12: np.ndarray):
    """[n, 12] -> (sc [n, 8], m [n, 8]) from the bit layout described above."""
    s = sc12.astype(np.int32)
    sc = np.empty((s.shape[0], 8), dtype=np.int32)
    m = np.empty((s.shape[0], 8), dtype=np.int32)
    sc[:, 0:4] = s[:, 0:4] & 0x3F
    m[:, 0:4] = s[:, 4:8] & 0x3F
    sc[:, 4:8] = (s[:, 8:12] & 0x0F) + 16 * (s[:, 0:4] >> 6)
    m[:, 4:8] = (s[:, 8:12] >> 4) + 16 * (s[:, 4:8] >> 6)
    return sc, m


def dequant_q4_k(raw: np.ndarray) -> np.ndarray:
    sb = raw.reshape(-1, 144)
    d = _f16(sb[:, 0:2])
    dmin = _f16(sb[:, 2:4])
    sc, m = q4k_unpack_scales(sb[:, 4:16])
    qs = sb[:, 16:].reshape(-1, 4, 32)
    q = np.empty((sb.shape[0], 4, 2, 32), dtype=np.float32)
    q[:, :, 0, :] = qs & 0x0F
    q[:, :, 1, :] = qs >> 4
    q = q.reshape(-1, 8, 32)
    scale = (d[:, None] * sc.astype(np.float32)).astype(np.float32)       # d*sc exact
    mins = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)      # dmin*m exact
    w = (scale[:, :, None] * q).astype(np.float32) - mins[:, :, None]     # one rounding
    return w.astype(np.float32).reshape(-1)


def dequant_q5_k(raw: np.ndarray) -> np.ndarray:
    sb = raw.reshape(-1, 176)
    n = sb.shape[0]
    d = _f16(sb[:, 0:2])
    dmin = _f16(sb[:, 2:4])
    sc, m = q4k_unpack_scales(sb[:, 4:16])
    qh = sb[:, 16:48].astype(np.int32)
    ql = sb[:, 48:176].reshape(n, 4, 32).astype(np.int32)
    q = np.empty((n, 4, 2, 32), dtype=np.int32)
    for g in range(4):
        q[:, g, 0, :] = (ql[:, g, :] & 0x0F) + 16 * ((qh >> (2 * g)) & 1)
        q[:, g, 1, :] = (ql[:, g, :] >> 4) + 16 * ((qh >> (2 * g + 1)) & 1)
    q = q.reshape(n, 8, 32).astype(np.float32)
    scale = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    mins = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)
    w = (scale[:, :, None] * q).astype(np.float32) - mins[:, :, None]
    return w.astype(np.float32).reshape(-1)


def dequant_q6_k(raw: np.ndarray) -> np.ndarray:
    sb = raw.reshape(-1, 210)
    n = sb.shape[0]
    ql = sb[:, 0:128].reshape(n, 2, 64).astype(np.int32)
    qh = sb[:, 128:192].reshape(n, 2, 32).astype(np.int32)
    sc = np.ascontiguousarray(sb[:, 192:208]).view(np.int8).astype(np.float32).reshape(n, 2, 4, 2)
    d = _f16(sb[:, 208:210])
    q = np.empty((n, 2, 4, 32), dtype=np.int32)
    q[:, :, 0, :] = (ql[:, :, 0:32] & 0x0F) | ((qh & 3) << 4)
    q[:, :, 1, :] = (ql[:, :, 32:64] & 0x0F) | (((qh >> 2) & 3) << 4)
    q[:, :, 2, :] = (ql[:, :, 0:32] >> 4) | (((qh >> 4) & 3) << 4)
    q[:, :, 3, :] = (ql[:, :, 32:64] >> 4) | (((qh >> 6) & 3) << 4)
    ds = (d[:, None, None, None] * sc).astype(np.float32)           # [n, half, row, l // 16]
    w = np.repeat(ds, 16, axis=3) * (q - 32).astype(np.float32)
    return w.astype(np.float32).reshape(-1)


def dequant_f16(raw: np.ndarray) -> np.ndarray:
    return raw.view(np.float16).astype(np.float32)


def dequant_bf16(raw: np.ndarray) -> np.ndarray:
    import torch
    t = torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16)
    return t.to(torch.float32).numpy()


def dequant_f32(raw: np.ndarray) -> np.ndarray:
    return raw.view(np.float32).copy()


def dequant(ggml_type: int, raw: np.ndarray) -> np.ndarray:
    f = {8: dequant_q8_0, 2: dequant_q4_0, 12: dequant_q4_k, 13: dequant_q5_k, 14: dequant_q6_k, 1: dequant_f16,
         30: dequant_bf16, 0: dequant_f32}
    return f[ggml_type](np.ascontiguousarray(raw).view(np.uint8).reshape(-1))


def pack_q4k_scales_quantizer(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Pack (sc, m) [n, 8] the way a Q4_K quantizer writes them: pairs 0..3 go
    straight into bytes j and j+4; pairs 4..7 put their low nibbles in byte j+4
    (j = 4..7, i.e. bytes 8..11) and OR their top two bits into bytes j-4 / j."""
    n = sc.shape[0]
    out = np.zeros((n, 12), dtype=np.int32)
    for j in range(8):
        ls, lm = sc[:, j].astype(np.int32), m[:, j].astype(np.int32)
        if j < 4:
            out[:, j] |= ls
            out[:, j + 4] |= lm
        else:
            out[:, j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            out[:, j - 4] |= (ls >> 4) << 6
            out[:, j] |= (lm >> 4) << 6
    return out.astype(np.uint8)
