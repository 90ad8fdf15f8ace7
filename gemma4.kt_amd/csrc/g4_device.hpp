// g4_device.hpp -- device-side building blocks for gfx950 (CDNA4, wave64).
//
// GGUF block decoders (the per-format get() of the reference) and the 64-element
// "chunk" dot products used by the row-stream matvec kernels.  Reference paths
// are relative to lib/src/main/kotlin/io/github/lbenedetto/internal/.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#define G4_DEV __device__ __forceinline__

namespace g4 {

enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

// Four dwords at 4-byte alignment: one global_load_dwordx4 (gfx950 needs dword alignment only).
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Hide a value from the optimiser so (v >> 8k) & 0xff selects v_cvt_f32_ubyte{k}
// instead of being re-fused with an earlier mask into bfe + ubyte0.
G4_DEV uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// A value rounded to its type and materialised: no fused multiply-add is formed
// across it.  HIP's __fmul_rn / __fadd_rn are plain operators here, and the
// compiler's default contraction (-ffp-contract=fast-honor-pragmas) would fuse
// a*b + c into one rounding where the reference (the JVM, which never fuses)
// rounds the product first.
G4_DEV float rounded(float v) {
  asm volatile("" : "+v"(v));
  return v;
}
G4_DEV double rounded(double v) {
  asm volatile("" : "+v"(v));
  return v;
}

// binary16 -> binary32 (v_cvt_f32_f16; fp16 denormals are preserved in the
// kernels' default float mode, so this is the exact decode of
// FloatTensorHelpers.kt:39-41).
G4_DEV float h2f(uint32_t h16) { return __half2float(__ushort_as_half((unsigned short)(h16 & 0xFFFFu))); }

// F16FloatTensor.kt:59-61: the vector path's bit trick (zero exponent -> +-0,
// exponent 31 -> finite 2^16 * 1.m).
G4_DEV float h2f_vec(uint32_t h16) {
  int32_t b = (int32_t)(int16_t)(uint16_t)h16;
  int32_t mask = (-(b & 0x7C00)) >> 31;
  uint32_t out = ((uint32_t)(b & 0x8000) << 16) | ((((uint32_t)(b & 0x7FFF) + 0x1C000u) << 13) & (uint32_t)mask);
  return __uint_as_float(out);
}

G4_DEV float bf2f(uint32_t h16) { return __uint_as_float((h16 & 0xFFFFu) << 16); }

G4_DEV float sbyte(uint32_t v, int b) { return (float)(int8_t)(v >> (8 * b)); }  // v_cvt_f32_i32_sdwa sext
G4_DEV float ubyte(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }  // v_cvt_f32_ubyte{b}

// f16 bit patterns below 0x0400 are the subnormals k * 2^-24: integers k < 1024
// masked into the two 16-bit halves of a dword are two exact f16 values, and
// v_fma_mix_f32 converts either half inside its fma (op_sel), so one AND
// unpacks two weights and the product with x costs one instruction.  Each
// product and sum is the one with k, scaled by 2^-24 exactly: roundings
// commute with power-of-two scaling while the values stay normal (|x| above
// 2^-102 or so), and the kernels' scales carry the 2^24 back.
G4_DEV float f16lo(uint32_t m) { return (float)__builtin_bit_cast(_Float16, (uint16_t)m); }
G4_DEV float f16hi(uint32_t m) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(m >> 16)); }

// lo + sum over the four bytes b of q, in byte order, of xl[b] * 2^-24 * (the
// low nibble of byte b), and hi + the same of xh[b] * 2^-24 * 16 * (its high
// nibble).  Bytes 0 and 2 come from q, bytes 1 and 3 from q >> 8.  The two
// chains alternate: a v_fma_mix_f32 that reads the result of the one before
// it waits a cycle.
G4_DEV void nib4_fma2(uint32_t q, const float *xl, const float *xh, float &lo, float &hi) {
  const uint32_t c = q >> 8;
  const uint32_t al = opaque(q & 0x000F000Fu), ah = opaque(q & 0x00F000F0u);
  const uint32_t cl = opaque(c & 0x000F000Fu), ch = opaque(c & 0x00F000F0u);
  lo = __builtin_fmaf(f16lo(al), xl[0], lo);
  hi = __builtin_fmaf(f16lo(ah), xh[0], hi);
  lo = __builtin_fmaf(f16lo(cl), xl[1], lo);
  hi = __builtin_fmaf(f16lo(ch), xh[1], hi);
  lo = __builtin_fmaf(f16hi(al), xl[2], lo);
  hi = __builtin_fmaf(f16hi(ah), xh[2], hi);
  lo = __builtin_fmaf(f16hi(cl), xl[3], lo);
  hi = __builtin_fmaf(f16hi(ch), xh[3], hi);
}

G4_DEV uint32_t rd_u8(const uint8_t *p) { return *p; }
G4_DEV uint32_t rd_u16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Q4_KFloatTensor.kt:70-84 getScaleMinK4.
G4_DEV int q4k_scale_min(int j, const uint8_t *s, bool is_min) {
  if (j < 4) return s[is_min ? j + 4 : j] & 63;
  int low = is_min ? (s[j + 4] >> 4) : (s[j + 4] & 0xF);
  int high = (s[is_min ? j : j - 4] >> 6) & 0x3;
  return low | (high << 4);
}

// Per-element get(index), bit-exact restatement of the reference:
// Q8_0FloatTensor.kt:21-28, Q4_0FloatTensor.kt:21-39, Q4_KFloatTensor.kt:23-55,
// Q5_KFloatTensor.kt:23-50, Q6_KFloatTensor.kt:26-75, F16FloatTensor.kt:20-23,
// BF16FloatTensor.kt:20-24, F32FloatTensor.kt:18-20.
// Every product here is exact in fp32 (at most 11 + 8 significant bits, or d*sc
// then *q within 24) or a chain of products, and the one subtraction takes an
// exact dmin*m, so each result is the reference's bit for bit however the
// compiler contracts.
template <int TYPE>
G4_DEV float get_elem(const uint8_t *W, int64_t idx) {
  if constexpr (TYPE == T_Q8_0) {
    const uint8_t *b = W + (idx >> 5) * 34;
    return __fmul_rn((float)(int8_t)b[2 + (idx & 31)], h2f(rd_u16(b)));
  } else if constexpr (TYPE == T_Q4_0) {
    const uint8_t *b = W + (idx >> 5) * 18;
    int mod = (int)(idx & 31);
    int q = (mod < 16) ? (b[2 + mod] & 0xF) : (b[2 + mod - 16] >> 4);
    return __fmul_rn((float)(q - 8), h2f(rd_u16(b)));
  } else if constexpr (TYPE == T_Q4_K) {
    const uint8_t *b = W + (idx >> 8) * 144;
    int within = (int)(idx & 255);
    int group = within >> 6, in_group = within & 63;
    int sub = group * 2 + (in_group >= 32 ? 1 : 0);
    int nib = in_group & 31;
    int sc = q4k_scale_min(sub, b + 4, false);
    int m = q4k_scale_min(sub, b + 4, true);
    int byte = b[16 + group * 32 + nib];
    int q = (in_group >= 32) ? (byte >> 4) : (byte & 0xF);
    float d = h2f(rd_u16(b)), dmin = h2f(rd_u16(b + 2));
    float t = __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
    return __fsub_rn(t, __fmul_rn(dmin, (float)m));
  } else if constexpr (TYPE == T_Q5_K) {
    const uint8_t *b = W + (idx >> 8) * 176;
    int within = (int)(idx & 255);
    int group = within >> 6, high = (within & 63) >= 32 ? 1 : 0, l = within & 31;
    int sub = group * 2 + high;
    int sc = q4k_scale_min(sub, b + 4, false);
    int m = q4k_scale_min(sub, b + 4, true);
    int byte = b[48 + group * 32 + l];
    int q = ((high ? (byte >> 4) : byte) & 0xF) | (((b[16 + l] >> sub) & 1) << 4);
    float d = h2f(rd_u16(b)), dmin = h2f(rd_u16(b + 2));
    float t = __fmul_rn(__fmul_rn(d, (float)sc), (float)q);
    return __fsub_rn(t, __fmul_rn(dmin, (float)m));
  } else if constexpr (TYPE == T_Q6_K) {
    const uint8_t *b = W + (idx >> 8) * 210;
    int within = (int)(idx & 255);
    int half = within >> 7, r = (within & 127) >> 5, l = within & 31;
    int nib = (b[half * 64 + (r & 1) * 32 + l] >> (4 * (r >> 1))) & 0xF;
    int hb = (b[128 + half * 32 + l] >> (2 * r)) & 3;
    int q6 = (nib | (hb << 4)) - 32;
    int sc = (int8_t)b[192 + half * 8 + r * 2 + (l >> 4)];
    float d = h2f(rd_u16(b + 208));
    return __fmul_rn(__fmul_rn(d, (float)sc), (float)q6);
  } else if constexpr (TYPE == T_F16) {
    return h2f(rd_u16(W + idx * 2));
  } else if constexpr (TYPE == T_BF16) {
    return bf2f(rd_u16(W + idx * 2));
  } else {
    return *(const float *)(W + idx * 4);
  }
}

// Element decode used by a dot at row position j of a row of length dim1: the
// F16 vector path decodes with the bit trick up to loopBound(dim1) = dim1 & ~15
// and with the exact decode in the scalar tail (F16FloatTensor.kt:43-77).
template <int TYPE>
G4_DEV float dot_elem(const uint8_t *W, int64_t idx, int j, int dim1) {
  if constexpr (TYPE == T_F16) {
    uint32_t h = rd_u16(W + idx * 2);
    return j < (dim1 & ~15) ? h2f_vec(h) : h2f(h);
  } else {
    return get_elem<TYPE>(W, idx);
  }
}

// ---------------------------------------------------------------------------
// 64-element chunks.  A chunk starts at an element offset e that is a multiple
// of 64 and holds: Q8_0 two blocks (68 B), Q4_0 two blocks (36 B), Q4_K one
// 64-weight group of a super-block (32 B of nibbles + the 16 B super-block
// head), Q5_K the same plus the 32 B of fifth bits, Q6_K a quarter super-block
// (64 B of nibbles shared with the neighbouring chunk, 32 B of bit pairs, 4
// scales, d), F16/BF16 128 B, F32 256 B.  load() issues only dword-aligned
// vector loads (plus 16-bit ones for Q6_K's scales and d); dot() unpacks in
// registers against x[0..64) and the precomputed sums.
// ---------------------------------------------------------------------------

// Q8_0: {fp16 d, int8 q[32]} x 2 = 17 dwords starting dword-aligned (68 * k).
struct FmtQ8_0 {
  static constexpr int TYPE = T_Q8_0, NDW = 17, NS = 0, RT = 2;
  G4_DEV static void load(const uint8_t *W, int64_t e, uint32_t (&D)[NDW]) {
    const uint8_t *p = W + (e >> 6) * 68;
    const u32x4a4 *v = (const u32x4a4 *)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4a4 t = v[i];
      D[4 * i + 0] = t.x; D[4 * i + 1] = t.y; D[4 * i + 2] = t.z; D[4 * i + 3] = t.w;
    }
    D[16] = ((const uint32_t *)p)[16];
  }
  G4_DEV static void sums(const float *x, float *s) { (void)x; (void)s; }
  // per block: (sum_k x_k q_k) * d, the scale applied after the block sum like
  // the reference's fma(s0 + s1, d, acc) (Q8_0FloatTensor.kt:64-78).
  G4_DEV static float dot(const uint32_t (&D)[NDW], const float *x, const float *s, int64_t e) {
    (void)s; (void)e;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t q = __builtin_amdgcn_alignbyte(D[i + 1], D[i], 2);  // bytes 2..33: q of block 0
#pragma unroll
      for (int b = 0; b < 4; ++b) a0 = __builtin_fmaf(x[4 * i + b], sbyte(q, b), a0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t q = D[9 + i];  // bytes 36..67: q of block 1 (dword aligned)
#pragma unroll
      for (int b = 0; b < 4; ++b) a1 = __builtin_fmaf(x[32 + 4 * i + b], sbyte(q, b), a1);
    }
    float d0 = h2f(D[0] & 0xFFFFu), d1 = h2f(D[8] >> 16);
    return __builtin_fmaf(a0, d0, a1 * d1);
  }
};

// Q4_0: {fp16 d, 16 B nibbles} x 2 = 9 dwords (36 * k).  Element k < 16 of a
// block is the low nibble of byte k, element 16 + k the high nibble; value
// (q - 8) * d (Q4_0FloatTensor.kt:21-39).  The high nibble is used in place
// (16 q, exact) and the 1/16 folded into the block sum; -8 enters through the
// precomputed sums of x over each 16 elements.  Those sums run in the same
// order as the weighted sums they are taken from (x[0], x[1], ... from 0), so
// a half block of q = 8 -- weights that are exactly zero, as the reference
// forms them (q - 8 before the product, Q4_0FloatTensor.kt:80-81) -- cancels
// to exactly 0: 8 * x and 128 * x are exact and scale every rounding with them.
struct FmtQ4_0 {
  static constexpr int TYPE = T_Q4_0, NDW = 9, NS = 4, RT = 2;
  G4_DEV static void load(const uint8_t *W, int64_t e, uint32_t (&D)[NDW]) {
    const uint8_t *p = W + (e >> 6) * 36;
    const u32x4a4 *v = (const u32x4a4 *)p;
    u32x4a4 t0 = v[0], t1 = v[1];
    D[0] = t0.x; D[1] = t0.y; D[2] = t0.z; D[3] = t0.w;
    D[4] = t1.x; D[5] = t1.y; D[6] = t1.z; D[7] = t1.w;
    D[8] = ((const uint32_t *)p)[8];
  }
  G4_DEV static void sums(const float *x, float *s) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) t += x[16 * k + i];
      s[k] = t;
    }
  }
  // sl / sh: the sums of x over the block's low / high 16 elements; the result
  // is scaled by 2^-24 (nib4_fma2), as are -8 and -128
  G4_DEV static float block(const uint32_t (&Q)[4], const float *x, float sl, float sh) {
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) nib4_fma2(Q[i], x + 4 * i, x + 16 + 4 * i, lo, hi);
    return __builtin_fmaf(__builtin_fmaf(-0x1p-17f, sh, hi), 0.0625f, __builtin_fmaf(-0x1p-21f, sl, lo));
  }
  G4_DEV static float dot(const uint32_t (&D)[NDW], const float *x, const float *s, int64_t e) {
    (void)e;
    uint32_t Q0[4], Q1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      Q0[i] = __builtin_amdgcn_alignbyte(D[i + 1], D[i], 2);  // bytes 2..17
      Q1[i] = D[5 + i];                                          // bytes 20..35
    }
    float t0 = block(Q0, x, s[0], s[1]);
    float t1 = block(Q1, x + 32, s[2], s[3]);
    return __builtin_fmaf(h2f(D[0] & 0xFFFFu) * 0x1p24f, t0, (h2f(D[4] >> 16) * 0x1p24f) * t1);
  }
};

// Q4_K: super-block {fp16 d, fp16 dmin, scales[12], qs[128]} (144 B).  Group g
// (64 weights) uses qs[32g .. 32g+32): low nibbles are sub-block 2g, high
// nibbles sub-block 2g+1; w = d*sc*q - dmin*m (Q4_KFloatTensor.kt:23-55).
// Per sub-block: d*sc * sum(x q) - dmin*m * sum(x), each product rounded on its
// own.  sum(x) runs in the order of sum(x q), so sum(x q) = q0 sum(x) exactly
// when every q of the sub-block is one power of two q0 (scaling by 2^k commutes
// with every rounding).  A sub-block whose weights the reference forms as
// exactly zero (fma(q, d*sc, -dmin*m) = 0, Q4_KFloatTensor.kt:143-148) gives
// exactly 0 here when d*sc = dmin*m = 0, or when its q are all one power of two
// (such as q = 8 with dmin*m = 8 d*sc) or all 0 with m = 0.  A constant q that is
// not a power of two (q = 3 with dmin*m = 3 d*sc) leaves a residue of the size of
// the rounding of sum(x q): a known limit of the factored form.
struct FmtQ4_K {
  static constexpr int TYPE = T_Q4_K, NDW = 12, NS = 2, RT = 2;
  G4_DEV static void load(const uint8_t *W, int64_t e, uint32_t (&D)[NDW]) {
    int64_t G = e >> 6;
    const uint8_t *sb = W + (G >> 2) * 144;
    const u32x4 *qs = (const u32x4 *)(sb + 16 + 32 * (int)(G & 3));
    u32x4 h = *(const u32x4 *)sb, q0 = qs[0], q1 = qs[1];
    D[0] = q0.x; D[1] = q0.y; D[2] = q0.z; D[3] = q0.w;
    D[4] = q1.x; D[5] = q1.y; D[6] = q1.z; D[7] = q1.w;
    D[8] = h.x; D[9] = h.y; D[10] = h.z; D[11] = h.w;
  }
  G4_DEV static void sums(const float *x, float *s) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) s0 += x[k], s1 += x[32 + k];
    s[0] = s0; s[1] = s1;
  }
  G4_DEV static float dot(const uint32_t (&D)[NDW], const float *x, const float *s, int64_t e) {
    float lo = 0.f, hi = 0.f;  // scaled by 2^-24 (nib4_fma2); d carries 2^24
#pragma unroll
    for (int i = 0; i < 8; ++i) nib4_fma2(D[i], x + 4 * i, x + 32 + 4 * i, lo, hi);
    // getScaleMinK4 (Q4_KFloatTensor.kt:70-84) for sub-blocks 2g and 2g+1: both
    // live in bytes 2(g&1), 2(g&1)+1 of the three scale dwords.
    const int g = (int)((e >> 6) & 3);
    const uint32_t sh = (uint32_t)(g & 1) * 16u;
    const uint32_t y = D[9] >> sh, z = D[10] >> sh, w = D[11] >> sh;
    uint32_t scp, mp;
    if (g < 2) {
      scp = y & 0x3F3Fu;
      mp = z & 0x3F3Fu;
    } else {
      scp = (w & 0x0F0Fu) | ((y >> 2) & 0x3030u);
      mp = ((w >> 4) & 0x0F0Fu) | ((z >> 2) & 0x3030u);
    }
    const float d = h2f(D[8] & 0xFFFFu) * 0x1p24f, dmin = h2f(D[8] >> 16);
    const float d1 = d * ubyte(scp, 0), d2 = d * ubyte(scp, 1) * 0.0625f;
    const float m1 = dmin * ubyte(mp, 0), m2 = dmin * ubyte(mp, 1);
    return k_subblocks(d1, lo, m1, s[0], d2, hi, m2, s[1]);
  }
  // (d1 lo - m1 s0) + (d2 hi - m2 s1), every product and difference rounded once
  G4_DEV static float k_subblocks(float d1, float lo, float m1, float s0, float d2, float hi, float m2, float s1) {
    return (rounded(d1 * lo) - rounded(m1 * s0)) + (rounded(d2 * hi) - rounded(m2 * s1));
  }
  // getScaleMinK4 for group g without a branch: the scale bytes of sub-blocks
  // 2g, 2g+1 are ((w >> sh) & mA) | ((y >> shk) & mB), the mins the same of
  // (w >> sh4) and z, with (y, z, w) the three scale dwords.  g < 2: mA = 0,
  // mB = 0x3F3F, shk = sh; g >= 2: the low nibbles from w, bits 6..7 of y and z
  // on top (mA = 0x0F0F, mB = 0x3030, shk = sh + 2).  For callers whose lanes
  // keep one g over all their rows, so the selector is formed once.
  struct Sel {
    uint32_t sh, shk, sh4, mA, mB;
  };
  G4_DEV static Sel select(int g) {
    const uint32_t sh = (uint32_t)(g & 1) * 16u;
    const bool h = g >= 2;
    return Sel{sh, sh + (h ? 2u : 0u), sh + 4u, h ? 0x0F0Fu : 0u, h ? 0x3030u : 0x3F3Fu};
  }
  // dot() for the group that q selects, the same arithmetic in the same order
  G4_DEV static float dot_sel(const uint32_t (&D)[NDW], const float *x, const float *s, const Sel &q) {
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) nib4_fma2(D[i], x + 4 * i, x + 32 + 4 * i, lo, hi);
    const uint32_t scp = opaque(((D[11] >> q.sh) & q.mA) | ((D[9] >> q.shk) & q.mB));
    const uint32_t mp = opaque(((D[11] >> q.sh4) & q.mA) | ((D[10] >> q.shk) & q.mB));
    const float d = h2f(D[8] & 0xFFFFu) * 0x1p24f, dmin = h2f(D[8] >> 16);
    const float d1 = d * ubyte(scp, 0), d2 = d * ubyte(scp, 1) * 0.0625f;
    const float m1 = dmin * ubyte(mp, 0), m2 = dmin * ubyte(mp, 1);
    return k_subblocks(d1, lo, m1, s[0], d2, hi, m2, s[1]);
  }
};

// Q5_K: super-block {fp16 d, fp16 dmin, scales[12], qh[32], qs[128]} (176 B,
// 16-byte aligned).  Group g as Q4_K, with the fifth bit of weight l of
// sub-block s = 2g + h in bit s of qh[l]: q = nibble + 16 bit, w = d*sc*q -
// dmin*m (Q5_KFloatTensor.kt:23-50).  Per sub-block: d*sc * sum(x q) -
// dmin*m * sum(x), rounded as for Q4_K (exactly 0 for the all-zero sub-blocks
// FmtQ4_K lists: here q0 = 1, 2, 4, 8 or 16).
struct FmtQ5_K {
  static constexpr int TYPE = T_Q5_K, NDW = 20, NS = 2, RT = 2;
  G4_DEV static void load(const uint8_t *W, int64_t e, uint32_t (&D)[NDW]) {
    int64_t G = e >> 6;
    const uint8_t *sb = W + (G >> 2) * 176;
    const u32x4 *qs = (const u32x4 *)(sb + 48 + 32 * (int)(G & 3));
    const u32x4 *qh = (const u32x4 *)(sb + 16);
    u32x4 h = *(const u32x4 *)sb, q0 = qs[0], q1 = qs[1], h0 = qh[0], h1 = qh[1];
    D[0] = q0.x; D[1] = q0.y; D[2] = q0.z; D[3] = q0.w;
    D[4] = q1.x; D[5] = q1.y; D[6] = q1.z; D[7] = q1.w;
    D[8] = h0.x; D[9] = h0.y; D[10] = h0.z; D[11] = h0.w;
    D[12] = h1.x; D[13] = h1.y; D[14] = h1.z; D[15] = h1.w;
    D[16] = h.x; D[17] = h.y; D[18] = h.z; D[19] = h.w;
  }
  G4_DEV static void sums(const float *x, float *s) { FmtQ4_K::sums(x, s); }
  G4_DEV static float dot(const uint32_t (&D)[NDW], const float *x, const float *s, int64_t e) {
    const int g = (int)((e >> 6) & 3);
    const uint32_t lsh = 2u * (uint32_t)g, hsh = lsh + 1u;
    // fifth bits (bit lsh / hsh of each qh byte) rotated onto bit 4 of the same byte
    const uint32_t lrot = (lsh - 4u) & 31u, hrot = (hsh - 4u) & 31u;
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t Q = D[i], H = D[8 + i];
      const uint32_t l = opaque((Q & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(H, H, lrot) & 0x10101010u));
      const uint32_t h = opaque(((Q >> 4) & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(H, H, hrot) & 0x10101010u));
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        lo = __builtin_fmaf(x[4 * i + b], ubyte(l, b), lo);
        hi = __builtin_fmaf(x[32 + 4 * i + b], ubyte(h, b), hi);
      }
    }
    // getScaleMinK4 for sub-blocks 2g, 2g+1 (as FmtQ4_K::dot)
    const uint32_t sh = (uint32_t)(g & 1) * 16u;
    const uint32_t y = D[17] >> sh, z = D[18] >> sh, w = D[19] >> sh;
    uint32_t scp, mp;
    if (g < 2) {
      scp = y & 0x3F3Fu;
      mp = z & 0x3F3Fu;
    } else {
      scp = (w & 0x0F0Fu) | ((y >> 2) & 0x3030u);
      mp = ((w >> 4) & 0x0F0Fu) | ((z >> 2) & 0x3030u);
    }
    const float d = h2f(D[16] & 0xFFFFu), dmin = h2f(D[16] >> 16);
    const float d1 = d * ubyte(scp, 0), d2 = d * ubyte(scp, 1);
    const float m1 = dmin * ubyte(mp, 0), m2 = dmin * ubyte(mp, 1);
    return FmtQ4_K::k_subblocks(d1, lo, m1, s[0], d2, hi, m2, s[1]);
  }
};

// Q6_K: super-block {ql[128], qh[64], int8 scales[16], fp16 d} (210 B, so odd
// super-blocks start at 2 mod 4).  Chunk c = 2n + p (half n, part p) reads
// ql[64n .. 64n+64) -- low nibbles for p = 0, high for p = 1; its first 32
// weights use ql[64n + l], the next 32 ql[64n + 32 + l] -- bit pairs 4p and
// 4p + 2 of qh[32n + l], and scales[8n + 4p + k] for its k-th 16 weights:
// w = d*sc*(q - 32) (Q6_KFloatTensor.kt:26-75).  ql and qh come in as
// dword-aligned loads shifted into place with alignbyte (their windows stay
// inside the super-block and the one before it); scales and d are read as
// 16-bit words.  -32 enters through the sums of x over each 16 weights.
struct FmtQ6_K {
  static constexpr int TYPE = T_Q6_K, NDW = 29, NS = 4, RT = 2;
  G4_DEV static void load(const uint8_t *W, int64_t e, uint32_t (&D)[NDW]) {
    const int64_t sb = e >> 8;
    const int c = (int)((e >> 6) & 3), n = c >> 1, p = c & 1;
    const uint8_t *S = W + sb * 210;
    // dword-aligned windows by pointer arithmetic on W (a pointer rebuilt from an
    // integer loses its global address space and compiles to flat loads)
    const uint8_t *qlb = S + 64 * n, *qhb = S + 128 + 32 * n;
    const u32x4a4 *ql = (const u32x4a4 *)(qlb - ((uintptr_t)qlb & 3));
    const u32x4a4 *qh = (const u32x4a4 *)(qhb - ((uintptr_t)qhb & 3));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4a4 t = ql[i];
      D[4 * i] = t.x; D[4 * i + 1] = t.y; D[4 * i + 2] = t.z; D[4 * i + 3] = t.w;
    }
    D[16] = ((const uint32_t *)ql)[16];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      u32x4a4 t = qh[i];
      D[17 + 4 * i] = t.x; D[18 + 4 * i] = t.y; D[19 + 4 * i] = t.z; D[20 + 4 * i] = t.w;
    }
    D[25] = ((const uint32_t *)qh)[8];
    const uint16_t *sc = (const uint16_t *)(S + 192 + 8 * n + 4 * p);
    D[26] = sc[0];
    D[27] = sc[1];
    D[28] = *(const uint16_t *)(S + 208);
  }
  G4_DEV static void sums(const float *x, float *s) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) t += x[16 * k + i];
      s[k] = t;
    }
  }
  G4_DEV static float dot(const uint32_t (&D)[NDW], const float *x, const float *s, int64_t e) {
    const uint32_t al = (uint32_t)((e >> 8) & 1) * 2u;  // 210 * sb mod 4
    const uint32_t p = (uint32_t)((e >> 6) & 1);
    const uint32_t ns = 4u * p, s0 = 4u * p, s1 = s0 + 2u;
    // bit pairs s0 / s1 of each qh byte rotated onto bits 4..5 of the same byte
    const uint32_t r0 = (s0 - 4u) & 31u, r1 = (s1 - 4u) & 31u;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t qa = __builtin_amdgcn_alignbyte(D[i + 1], D[i], al);           // ql[l], l = 4i..4i+3
      const uint32_t qb = __builtin_amdgcn_alignbyte(D[i + 9], D[i + 8], al);       // ql[32 + l]
      const uint32_t hv = __builtin_amdgcn_alignbyte(D[18 + i], D[17 + i], al);     // qh[l]
      const uint32_t va = opaque(((qa >> ns) & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(hv, hv, r0) & 0x30303030u));
      const uint32_t vb = opaque(((qb >> ns) & 0x0F0F0F0Fu) | (__builtin_amdgcn_alignbit(hv, hv, r1) & 0x30303030u));
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        acc[i >> 2] = __builtin_fmaf(x[4 * i + b], ubyte(va, b), acc[i >> 2]);
        acc[2 + (i >> 2)] = __builtin_fmaf(x[32 + 4 * i + b], ubyte(vb, b), acc[2 + (i >> 2)]);
      }
    }
    const uint32_t sc = D[26] | (D[27] << 16);
    const float d = h2f(D[28]);
    float r = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) r = __builtin_fmaf(d * sbyte(sc, k), __builtin_fmaf(-32.f, s[k], acc[k]), r);
    return r;
  }
};

// F16 / BF16: 64 halves = 32 dwords (16-byte aligned chunks).  F16 uses the
// vector-path decode (the fast path requires dim1 % 64 == 0, so no element is
// in the scalar tail); BF16 is exact.
template <int TYPE_>
struct FmtHalf {
  static constexpr int TYPE = TYPE_, NDW = 32, NS = 0, RT = 2;
  G4_DEV static void load(const uint8_t *W, int64_t e, uint32_t (&D)[NDW]) {
    const u32x4 *v = (const u32x4 *)(W + e * 2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      u32x4 t = v[i];
      D[4 * i + 0] = t.x; D[4 * i + 1] = t.y; D[4 * i + 2] = t.z; D[4 * i + 3] = t.w;
    }
  }
  G4_DEV static void sums(const float *x, float *s) { (void)x; (void)s; }
  G4_DEV static float dot(const uint32_t (&D)[NDW], const float *x, const float *s, int64_t e) {
    (void)s; (void)e;
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      float w0, w1;
      if constexpr (TYPE == T_F16) {
        w0 = h2f_vec(D[i] & 0xFFFFu);
        w1 = h2f_vec(D[i] >> 16);
      } else {
        w0 = __uint_as_float(D[i] << 16);
        w1 = __uint_as_float(D[i] & 0xFFFF0000u);
      }
      a = __builtin_fmaf(w0, x[2 * i], a);
      b = __builtin_fmaf(w1, x[2 * i + 1], b);
    }
    return a + b;
  }
};

// F32: 64 floats = 16 dwordx4.
struct FmtF32 {
  static constexpr int TYPE = T_F32, NDW = 64, NS = 0, RT = 1;
  G4_DEV static void load(const uint8_t *W, int64_t e, uint32_t (&D)[NDW]) {
    const u32x4 *v = (const u32x4 *)(W + e * 4);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      u32x4 t = v[i];
      D[4 * i + 0] = t.x; D[4 * i + 1] = t.y; D[4 * i + 2] = t.z; D[4 * i + 3] = t.w;
    }
  }
  G4_DEV static void sums(const float *x, float *s) { (void)x; (void)s; }
  G4_DEV static float dot(const uint32_t (&D)[NDW], const float *x, const float *s, int64_t e) {
    (void)s; (void)e;
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      a = __builtin_fmaf(__uint_as_float(D[2 * i]), x[2 * i], a);
      b = __builtin_fmaf(__uint_as_float(D[2 * i + 1]), x[2 * i + 1], b);
    }
    return a + b;
  }
};

// ---------------------------------------------------------------------------
// Wave reductions.
// ---------------------------------------------------------------------------

// Partner value for the butterfly step S <= 8 inside a 16-lane row, by DPP:
// S=8 row_ror:8 (lane ^ 8), S=4 row_half_mirror (7 - i within 8 lanes, which
// flips bit 2), S=2 quad_perm [2,3,0,1], S=1 quad_perm [1,0,3,2].  Each is an
// involution whose partner differs in bit S, which is all the butterfly needs.
template <int S>
G4_DEV float dpp_partner(float v) {
  static_assert(S == 8 || S == 4 || S == 2 || S == 1, "row-local step");
  constexpr int ctrl = S == 8 ? 0x128 : S == 4 ? 0x141 : S == 2 ? 0x4E : 0xB1;
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
}

// One transposing butterfly step at distance S: lanes with bit S clear return
// A(self) + A(partner), lanes with bit S set return B(self) + B(partner).
// S = 32 / 16 use the gfx950 permlane swaps (one instruction moves both halves).
template <int S>
G4_DEV float tstep(float A, float B, int lane) {
  if constexpr (S == 32) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(A), __float_as_uint(B), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (S == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(A), __float_as_uint(B), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const bool upper = (lane & S) != 0;
    const float send = upper ? A : B, keep = upper ? B : A;
    return keep + dpp_partner<S>(send);
  }
}

// Plain butterfly step at distance S: every lane gets v(self) + v(partner).
template <int S>
G4_DEV float pstep(float v) {
  if constexpr (S == 32) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (S == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    return v + dpp_partner<S>(v);
  }
}

template <int S, int N, int NV>
G4_DEV void reduce_steps(float (&v)[NV], int lane) {
  if constexpr (S >= 1) {
    if constexpr (N > 1) {
#pragma unroll
      for (int j = 0; j < N / 2; ++j) v[j] = tstep<S>(v[j], v[j + N / 2], lane);
      reduce_steps<S / 2, N / 2>(v, lane);
    } else {
      v[0] = pstep<S>(v[0]);
      reduce_steps<S / 2, 1>(v, lane);
    }
  }
}

// Sum N values over the LPR lanes of each lane group (LPR a power of two, N <= LPR).
// The first log2(N) butterfly steps exchange half of the remaining values
// (a transposing reduction), the rest reduce one value.  On return, lane q of a
// group holds the group total of value index q / (LPR / N).
template <int N, int LPR>
G4_DEV float reduce_transpose(float (&v)[N], int lane) {
  static_assert((N & (N - 1)) == 0 && (LPR & (LPR - 1)) == 0 && N <= LPR, "powers of two");
  reduce_steps<LPR / 2, N>(v, lane);
  return v[0];
}

G4_DEV float wave_sum(float v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, 64);
  return v;
}

// (value, index) ordering of FloatTensor.argmax (FloatTensor.kt:53-66) for a
// parallel reduction: larger value wins, equal values go to the lower index.
// Callers map NaN to -inf (never wins) except at index 0, where it maps to +inf
// (the sequential scan keeps a NaN first element).
// Bitwise, not short-circuit: `||`/`&&` here compiled to a branch per comparison.
G4_DEV bool am_better(float a, int ia, float b, int ib) { return (a > b) | ((a == b) & (ia < ib)); }
G4_DEV float am_key(float v, int64_t idx) { return v != v ? (idx == 0 ? __builtin_inff() : -__builtin_inff()) : v; }

// Value of the butterfly partner at distance S (lane ^ S for S >= 16 and S = 8,
// 2, 1; the half-row mirror for S = 4), without going through LDS.
template <int S>
G4_DEV uint32_t partner_u32(uint32_t v, int lane) {
  if constexpr (S == 32) {
    auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // r[0] = low half, r[1] = high half
    return (lane & 32) ? r[0] : r[1];
  } else if constexpr (S == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // r[0] = even rows, r[1] = odd rows
    return (lane & 16) ? r[0] : r[1];
  } else {
    constexpr int ctrl = S == 8 ? 0x128 : S == 4 ? 0x141 : S == 2 ? 0x4E : 0xB1;
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xF, 0xF, false);
  }
}

template <int S>
G4_DEV void am_step(float &v, int &i, int lane) {
  const float ov = __uint_as_float(partner_u32<S>(__float_as_uint(v), lane));
  const int oi = (int)partner_u32<S>((uint32_t)i, lane);
  if (am_better(ov, oi, v, i)) v = ov, i = oi;
}

// (value, index) arg-max over the 64 lanes of a wave; every lane ends with the result.
G4_DEV void am_wave(float &v, int &i) {
  const int lane = __lane_id();
  am_step<32>(v, i, lane);
  am_step<16>(v, i, lane);
  am_step<8>(v, i, lane);
  am_step<4>(v, i, lane);
  am_step<2>(v, i, lane);
  am_step<1>(v, i, lane);
}


// tanh(x) in double following the steps of fdlibm's s_tanh.c (the algorithm of
// the JDK's StrictMath.tanh): |x| < 2^-55: x (1 + x); |x| < 1: -t / (t + 2) with
// t = expm1(-2|x|); |x| < 22: 1 - 2 / (t + 2) with t = expm1(2|x|); beyond: 1;
// then x's sign.  The expm1 is the device library's, not fdlibm's s_expm1.c, so
// the last double bit can differ from StrictMath.tanh; the JVM's Math.tanh may
// also run an intrinsic of its own.  Bit parity with the reference's tanh is
// therefore not claimed: the result is within 2 ulps of tanh.
// The two middle cases share one expm1 and one division, their operands chosen
// per lane (the same operations on each lane as the branches, without running
// both when the lanes of a wave fall on different sides of |x| = 1).
G4_DEV double tanh_fdlibm(double x) {
  const double ax = fabs(x);
  const bool small = ax < 1.0;
  const double t = expm1(small ? -2.0 * ax : 2.0 * ax);
  const double qt = (small ? -t : 2.0) / (t + 2.0);  // -t / (t + 2), or 2 / (t + 2)
  double z = small ? qt : 1.0 - qt;
  z = ax < 22.0 ? z : 1.0;
  z = __builtin_signbit(x) ? -z : z;
  z = ax < 0x1p-55 ? x * (1.0 + x) : z;
  return x != x ? x + x : z;
}

// Llama.kt:23-25 gelu, evaluated in double like the reference.
G4_DEV float gelu_ref(float xf) {
  double x = (double)xf;
  double inner = 0.7978845608028654 * (x + rounded(0.044715 * (x * x * x)));
  return (float)(0.5 * x * (1.0 + tanh_fdlibm(inner)));
}

// ------------------------------------------------------------ rms norm ----
// The three ways Llama.kt applies the rms scale s to element x with weight w:
// rmsnorm(out, x, weight, size, eps) (Llama.kt:27-37) computes w * (s * x); the
// offset overload (Llama.kt:39-59) computes w * s * x left to right; and
// rmsnormNoWeight (Llama.kt:61-78) computes s * x.
enum : int { NORM_WEIGHT_AFTER = 0, NORM_WEIGHT_FIRST = 1, NORM_NO_WEIGHT = 2 };

G4_DEV float norm_apply(int form, float w, float s, float x) {
  if (form == NORM_WEIGHT_AFTER) return rounded(w * (s * x));
  if (form == NORM_WEIGHT_FIRST) return rounded((w * s) * x);
  return rounded(s * x);
}

// ss = fp32 sum of squares -> s = (float)(1.0 / sqrt((double)(ss / size + eps))),
// each step rounded as in the reference (fp32 divide and add, double sqrt and divide).
G4_DEV float rms_scale(float ss, int32_t size, float eps) {
  const float m = __fadd_rn(__fdiv_rn(ss, (float)size), eps);
  return (float)__ddiv_rn(1.0, __dsqrt_rn((double)m));
}

G4_DEV float sq_acc(float acc, float v) { return __builtin_fmaf(v, v, acc); }

// Sum over a 256-thread workgroup, the same value in every thread: the wave
// butterfly (both partners of a pair add the same two values, so every lane
// ends with identical bits), then the four wave sums in wave order.  `red` is
// four floats of LDS; call once per kernel.  The standalone rms norm and the
// matvec kernels' fused input norm both feed it the same per-thread partials
// (thread t sums 16-byte segments t, t + 256, ... holding elements 4s..4s+3, in
// element order), so fused and standalone norms give identical scales.
G4_DEV float block_sum256(float v, float *red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return __fadd_rn(__fadd_rn(__fadd_rn(red[0], red[1]), red[2]), red[3]);
}

// Llama.kt:403-406 final logit soft-capping: cap * (float)tanh((double)(v / cap)).
G4_DEV float softcap_ref(float v, float cap) {
  return __fmul_rn(cap, (float)tanh_fdlibm((double)__fdiv_rn(v, cap)));
}

}  // namespace g4
