/*
 * g4_oracle.c -- CPU restatement of gemma4.kt's quantized matrix-vector path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Nothing in the product library links
 * or calls this file; tests/, the smoke check and the CPU-baseline leg of the
 * benchmark load it through ctypes.
 *
 * Reference paths are relative to lib/src/main/kotlin/io/github/lbenedetto/internal/.
 * Arithmetic follows the JVM: no fp contraction (built with -ffp-contract=off),
 * explicit fmaf() exactly where the Vector API calls fma, fp32 everywhere the
 * reference keeps Float, double where it converts to Double.
 *
 * Pinning (see tests/test_oracle_pins.py): fp16/bf16 decoders against numpy and
 * torch over all 65536 patterns; get() of every format against an independent
 * numpy restatement and hand-packed blocks with known values; dots against fp64
 * brute force; argmax / softmax / top-k against numpy on constructed cases.
 */
#include "g4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- types ---- */

/* GGMLType.kt:16-30: typeSize/blockSize of the supported ids. */
int or_block_size(int type) {
  switch (type) {
    case OR_F32: return 1;
    case OR_F16: return 1;
    case OR_BF16: return 1;
    case OR_Q4_0: return 32;
    case OR_Q8_0: return 32;
    case OR_Q4_K: return 256;
    case OR_Q5_K: return 256;
    case OR_Q6_K: return 256;
    default: return 0;
  }
}

int or_type_size(int type) {
  switch (type) {
    case OR_F32: return 4;
    case OR_F16: return 2;
    case OR_BF16: return 2;
    case OR_Q4_0: return 2 + 16;          /* Float16.BYTES + 16 bytes */
    case OR_Q8_0: return 2 + 32;          /* Float16.BYTES + 32 bytes */
    case OR_Q4_K: return 2 * 2 + 12 + 128; /* 2*Float16.BYTES + 12 + QK_K/2 */
    case OR_Q5_K: return 2 * 2 + 12 + 32 + 128; /* + QK_K/8 high bits */
    case OR_Q6_K: return 128 + 64 + 16 + 2;     /* QK_K/2 + QK_K/4 + QK_K/16 + Float16.BYTES */
    default: return 0;
  }
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static inline float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* --------------------------------------------------------- 16-bit floats --- */

/* FloatTensorHelpers.kt:39-41 -> Float.float16ToFloat: exact binary16 decode. */
float or_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  if (e == 0x1F) return bits_to_f32(sign | 0x7F800000u | (m << 13)); /* Inf / NaN (payload kept) */
  if (e != 0) return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
  if (m == 0) return bits_to_f32(sign);
  /* subnormal: m * 2^-24, exact in binary32 */
  float v = (float)m * 5.9604644775390625e-08f;
  return sign ? -v : v;
}

/* F16FloatTensor.kt:59-61: bits32 = sext(h); mask = -(bits & 0x7C00) >> 31;
 * bits32 = (bits & 0x8000) << 16 | (((bits & 0x7FFF) + 0x1C000) << 13) & mask. */
float or_fp16_vec_decode(uint16_t h) {
  int32_t b = (int32_t)(int16_t)h;
  int32_t mask = (-(b & 0x7C00)) >> 31;
  uint32_t out = ((uint32_t)(b & 0x8000) << 16) | ((((uint32_t)(b & 0x7FFF) + 0x1C000u) << 13) & (uint32_t)mask);
  return bits_to_f32(out);
}

/* BF16FloatTensor.kt:20-24: Float.fromBits(bits << 16). */
float or_bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

void or_fp16_to_f32_array(const uint16_t *h, int64_t n, float *out) {
  for (int64_t i = 0; i < n; i++) out[i] = or_fp16_to_f32(h[i]);
}

void or_fp16_vec_decode_array(const uint16_t *h, int64_t n, float *out) {
  for (int64_t i = 0; i < n; i++) out[i] = or_fp16_vec_decode(h[i]);
}

/* ------------------------------------------------------------------ get ---- */

/* Q4_KFloatTensor.kt:70-84 getScaleMinK4. */
int or_q4k_scale_min(int j, const uint8_t *s, int is_min) {
  if (j < 4) {
    int idx = is_min ? j + 4 : j;
    return s[idx] & 63;
  }
  int low = is_min ? (s[j + 4] >> 4) : (s[j + 4] & 0xF);
  int high = (s[is_min ? j : j - 4] >> 6) & 0x3;
  return low | (high << 4);
}

float or_get(int type, const uint8_t *raw, int64_t index) {
  switch (type) {
    case OR_Q8_0: { /* Q8_0FloatTensor.kt:21-28 */
      int64_t blk = index / 32, within = index % 32;
      const uint8_t *b = raw + blk * 34;
      int8_t q = (int8_t)b[2 + within];
      float scale = or_fp16_to_f32(rd16(b));
      return (float)q * scale;
    }
    case OR_Q4_0: { /* Q4_0FloatTensor.kt:21-39 */
      int64_t blk = index / 32;
      const uint8_t *b = raw + blk * 18;
      float scale = or_fp16_to_f32(rd16(b));
      int mod = (int)(index % 32);
      int quant = (mod < 16) ? (b[2 + mod] & 0x0F) : ((b[2 + mod - 16] >> 4) & 0x0F);
      int8_t q = (int8_t)(quant - 8);
      return (float)q * scale;
    }
    case OR_Q4_K: { /* Q4_KFloatTensor.kt:23-55 */
      int64_t blk = index / 256;
      int within = (int)(index % 256);
      const uint8_t *b = raw + blk * 144;
      float d = or_fp16_to_f32(rd16(b));
      float dmin = or_fp16_to_f32(rd16(b + 2));
      const uint8_t *scales = b + 4, *qs = b + 16;
      int group = within / 64, in_group = within % 64;
      int sub, nib, high;
      if (in_group < 32) {
        sub = group * 2; nib = in_group; high = 0;
      } else {
        sub = group * 2 + 1; nib = in_group - 32; high = 1;
      }
      int sc = or_q4k_scale_min(sub, scales, 0);
      int m = or_q4k_scale_min(sub, scales, 1);
      int byte = qs[group * 32 + nib];
      int quant = high ? ((byte >> 4) & 0xF) : (byte & 0xF);
      /* d * sc * quant - dmin * m, left to right in fp32 */
      float t = d * (float)sc;
      t = t * (float)quant;
      float u = dmin * (float)m;
      return t - u;
    }
    case OR_Q5_K: { /* Q5_KFloatTensor.kt:23-50 */
      int64_t blk = index / 256;
      int within = (int)(index % 256);
      const uint8_t *b = raw + blk * 176;
      float d = or_fp16_to_f32(rd16(b));
      float dmin = or_fp16_to_f32(rd16(b + 2));
      const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
      int group = within / 64, in_group = within % 64;
      int high = in_group >= 32;
      int l = high ? in_group - 32 : in_group;
      int sub = group * 2 + high;
      int sc = or_q4k_scale_min(sub, scales, 0);
      int m = or_q4k_scale_min(sub, scales, 1);
      int byte = qs[group * 32 + l];
      int nibble = high ? ((byte >> 4) & 0xF) : (byte & 0xF);
      int bit = (qh[l] >> (2 * group + high)) & 1;
      int quant = nibble | (bit << 4);
      /* d * sc * quant - dmin * m, left to right in fp32 */
      float t = d * (float)sc;
      t = t * (float)quant;
      float u = dmin * (float)m;
      return t - u;
    }
    case OR_Q6_K: { /* Q6_KFloatTensor.kt:26-75 */
      int64_t blk = index / 256;
      int within = (int)(index % 256);
      const uint8_t *b = raw + blk * 210;
      const uint8_t *ql = b, *qh = b + 128;
      const int8_t *scales = (const int8_t *)(b + 192);
      float d = or_fp16_to_f32(rd16(b + 208));
      int half = within / 128, rem = within % 128, sub32 = rem / 32, l = rem % 32;
      const uint8_t *qlb = ql + half * 64, *qhb = qh + half * 32;
      int nib;
      switch (sub32) {
        case 0: nib = qlb[l] & 0xF; break;
        case 1: nib = qlb[32 + l] & 0xF; break;
        case 2: nib = (qlb[l] >> 4) & 0xF; break;
        default: nib = (qlb[32 + l] >> 4) & 0xF; break;
      }
      int hb = (qhb[l] >> (2 * sub32)) & 3;
      int q6 = (nib | (hb << 4)) - 32;
      int sc = scales[half * 8 + sub32 * 2 + l / 16];
      /* d * sc * q6, left to right in fp32 */
      float t = d * (float)sc;
      return t * (float)q6;
    }
    case OR_F16: /* F16FloatTensor.kt:20-23 */
      return or_fp16_to_f32(rd16(raw + index * 2));
    case OR_BF16: /* BF16FloatTensor.kt:20-24 */
      return or_bf16_to_f32(rd16(raw + index * 2));
    case OR_F32: { /* F32FloatTensor.kt:18-20 */
      float f;
      memcpy(&f, raw + index * 4, 4);
      return f;
    }
    default:
      return NAN;
  }
}

void or_dequant(int type, const uint8_t *raw, int64_t offset, int64_t n, float *out) {
  for (int64_t i = 0; i < n; i++) out[i] = or_get(type, raw, offset + i);
}

/* ------------------------------------------------------------------ dots --- */

/* FloatTensorHelpers.kt:65-71: result += thiz[i] * that[i], no contraction. */
float or_scalar_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size) {
  float result = 0.0f;
  for (int32_t j = 0; j < size; j++) {
    float p = or_get(type, raw, this_offset + j) * x[j];
    result = result + p;
  }
  return result;
}

/* FloatVector.reduceLanes(ADD) over 16 lanes.  The API leaves the order
 * unspecified; this restatement uses recursive halving (lanes i and i+8, then
 * i and i+4, ...), the shape of the x86 512-bit reduction. */
static float reduce16(const float v[16]) {
  float a[16];
  memcpy(a, v, sizeof(a));
  for (int w = 8; w >= 1; w >>= 1)
    for (int i = 0; i < w; i++) a[i] = a[i] + a[i + w];
  return a[0];
}

/* Q8_0FloatTensor.kt:39-142, 512-bit branch (:64-78). */
static float vdot_q8_0(const uint8_t *raw, int64_t off, const float *x, int32_t size) {
  float result = 0.0f;
  int32_t j = 0;
  int32_t align = (int32_t)((-off) & 31);
  if (align > size) align = size;
  if (align > 0) {
    result += or_scalar_dot(OR_Q8_0, raw, off, x, align);
    j += align;
  }
  float value[16] = {0};
  int64_t block_off = (off + j) / 32 * 34;
  int32_t upper = j + (size - j) / 32 * 32;
  while (j < upper) {
    const uint8_t *b = raw + block_off;
    float d = or_fp16_to_f32(rd16(b));
    for (int l = 0; l < 16; l++) {
      float s0 = x[j + l] * (float)(int8_t)b[2 + l];
      float s1 = x[j + 16 + l] * (float)(int8_t)b[2 + 16 + l];
      value[l] = fmaf(s0 + s1, d, value[l]);
    }
    j += 32;
    block_off += 34;
  }
  result += reduce16(value);
  if (j < size) result += or_scalar_dot(OR_Q8_0, raw, off + j, x + j, size - j);
  return result;
}

/* Q4_0FloatTensor.kt:50-146, 512-bit branch (:83-91). */
static float vdot_q4_0(const uint8_t *raw, int64_t off, const float *x, int32_t size) {
  float result = 0.0f;
  int32_t j = 0;
  int32_t align = (int32_t)((-off) & 31);
  if (align > size) align = size;
  if (align > 0) {
    result += or_scalar_dot(OR_Q4_0, raw, off, x, align);
    j += align;
  }
  float value[16] = {0};
  int64_t block_off = (off + j) / 32 * 18;
  int32_t upper = j + (size - j) / 32 * 32;
  while (j < upper) {
    const uint8_t *b = raw + block_off;
    float d = or_fp16_to_f32(rd16(b));
    for (int l = 0; l < 16; l++) {
      int lo = (int8_t)((b[2 + l] & 0xF) - 8);
      int hi = (int8_t)((b[2 + l] >> 4) - 8);
      float s0 = x[j + l] * (float)lo;
      float s1 = x[j + 16 + l] * (float)hi;
      value[l] = fmaf(s0 + s1, d, value[l]);
    }
    j += 32;
    block_off += 18;
  }
  result += reduce16(value);
  if (j < size) result += or_scalar_dot(OR_Q4_0, raw, off + j, x + j, size - j);
  return result;
}

/* Q4_KFloatTensor.kt:86-207, 512-bit branch (:143-148). */
static float vdot_q4_k(const uint8_t *raw, int64_t off, const float *x, int32_t size) {
  float result = 0.0f;
  int32_t j = 0;
  int32_t align = (int32_t)((-off) & 255);
  if (align > size) align = size;
  if (align > 0) {
    result += or_scalar_dot(OR_Q4_K, raw, off, x, align);
    j += align;
  }
  float value[16] = {0}, val2[16] = {0};
  int64_t block_off = (off + j) / 256 * 144;
  int32_t upper = j + (size - j) / 256 * 256;
  while (j < upper) {
    const uint8_t *b = raw + block_off;
    float d = or_fp16_to_f32(rd16(b));
    float dmin = or_fp16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4, *qs = b + 16;
    for (int g = 0; g < 4; g++) {
      float d1 = d * (float)or_q4k_scale_min(g * 2, sc, 0);
      float negM1 = -(dmin * (float)or_q4k_scale_min(g * 2, sc, 1));
      float d2 = d * (float)or_q4k_scale_min(g * 2 + 1, sc, 0);
      float negM2 = -(dmin * (float)or_q4k_scale_min(g * 2 + 1, sc, 1));
      int32_t lo_base = j + g * 64, hi_base = j + g * 64 + 32;
      for (int c = 0; c < 2; c++) {
        const uint8_t *w = qs + g * 32 + c * 16;
        for (int l = 0; l < 16; l++) {
          float loq = (float)(w[l] & 0xF);
          float hiq = (float)(w[l] >> 4);
          value[l] = fmaf(fmaf(loq, d1, negM1), x[lo_base + c * 16 + l], value[l]);
          val2[l] = fmaf(fmaf(hiq, d2, negM2), x[hi_base + c * 16 + l], val2[l]);
        }
      }
    }
    j += 256;
    block_off += 144;
  }
  float sum[16];
  for (int l = 0; l < 16; l++) sum[l] = value[l] + val2[l];
  result += reduce16(sum);
  if (j < size) result += or_scalar_dot(OR_Q4_K, raw, off + j, x + j, size - j);
  return result;
}

/* Q5_KFloatTensor.kt:64-190, 512-bit branch (:125-131): two accumulators, each
 * element weight fma(q, d*sc, -(dmin*m)) fma'd into its lane. */
static float vdot_q5_k(const uint8_t *raw, int64_t off, const float *x, int32_t size) {
  float result = 0.0f;
  int32_t j = 0;
  int32_t align = (int32_t)((-off) & 255);
  if (align > size) align = size;
  if (align > 0) {
    result += or_scalar_dot(OR_Q5_K, raw, off, x, align);
    j += align;
  }
  float value[16] = {0}, val2[16] = {0};
  int64_t block_off = (off + j) / 256 * 176;
  int32_t upper = j + (size - j) / 256 * 256;
  while (j < upper) {
    const uint8_t *b = raw + block_off;
    float d = or_fp16_to_f32(rd16(b));
    float dmin = or_fp16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
    for (int g = 0; g < 4; g++) {
      float d1 = d * (float)or_q4k_scale_min(g * 2, sc, 0);
      float negM1 = -(dmin * (float)or_q4k_scale_min(g * 2, sc, 1));
      float d2 = d * (float)or_q4k_scale_min(g * 2 + 1, sc, 0);
      float negM2 = -(dmin * (float)or_q4k_scale_min(g * 2 + 1, sc, 1));
      for (int c = 0; c < 2; c++) {
        const uint8_t *w = qs + g * 32 + c * 16, *hb = qh + c * 16;
        int32_t lo_base = j + g * 64 + c * 16, hi_base = j + g * 64 + 32 + c * 16;
        for (int l = 0; l < 16; l++) {
          float loq = (float)((w[l] & 0xF) | (((hb[l] >> (2 * g)) & 1) << 4));
          float hiq = (float)((w[l] >> 4) | (((hb[l] >> (2 * g + 1)) & 1) << 4));
          value[l] = fmaf(fmaf(loq, d1, negM1), x[lo_base + l], value[l]);
          val2[l] = fmaf(fmaf(hiq, d2, negM2), x[hi_base + l], val2[l]);
        }
      }
    }
    j += 256;
    block_off += 176;
  }
  float sum[16];
  for (int l = 0; l < 16; l++) sum[l] = value[l] + val2[l];
  result += reduce16(sum);
  if (j < size) result += or_scalar_dot(OR_Q5_K, raw, off + j, x + j, size - j);
  return result;
}

/* Q6_KFloatTensor.kt:110-250, 512-bit branch (:196-205): per half and 16-lane
 * column c, four 6-bit groups q0..q3 (ql low/high nibbles, qh bit pairs), each
 * weight (float)q * (d*sc) fma'd into one accumulator in q0, q1, q2, q3 order. */
static float vdot_q6_k(const uint8_t *raw, int64_t off, const float *x, int32_t size) {
  float result = 0.0f;
  int32_t j = 0;
  int32_t align = (int32_t)((-off) & 255);
  if (align > size) align = size;
  if (align > 0) {
    result += or_scalar_dot(OR_Q6_K, raw, off, x, align);
    j += align;
  }
  float acc[16] = {0};
  int64_t block_off = (off + j) / 256 * 210;
  int32_t upper = j + (size - j) / 256 * 256;
  while (j < upper) {
    const uint8_t *b = raw + block_off;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = or_fp16_to_f32(rd16(b + 208));
    for (int h = 0; h < 2; h++) {
      const uint8_t *ql = b + h * 64, *qh = b + 128 + h * 32;
      int32_t base = j + h * 128;
      for (int c = 0; c < 2; c++) {
        float ds0 = d * (float)sc[h * 8 + c], ds1 = d * (float)sc[h * 8 + 2 + c];
        float ds2 = d * (float)sc[h * 8 + 4 + c], ds3 = d * (float)sc[h * 8 + 6 + c];
        for (int l = 0; l < 16; l++) {
          int a = ql[c * 16 + l], bb = ql[32 + c * 16 + l], v = qh[c * 16 + l];
          int q0 = ((a & 0xF) | ((v & 3) << 4)) - 32;
          int q1 = ((bb & 0xF) | (((v >> 2) & 3) << 4)) - 32;
          int q2 = ((a >> 4) | (((v >> 4) & 3) << 4)) - 32;
          int q3 = ((bb >> 4) | (((v >> 6) & 3) << 4)) - 32;
          acc[l] = fmaf((float)q0 * ds0, x[base + c * 16 + l], acc[l]);
          acc[l] = fmaf((float)q1 * ds1, x[base + 32 + c * 16 + l], acc[l]);
          acc[l] = fmaf((float)q2 * ds2, x[base + 64 + c * 16 + l], acc[l]);
          acc[l] = fmaf((float)q3 * ds3, x[base + 96 + c * 16 + l], acc[l]);
        }
      }
    }
    j += 256;
    block_off += 210;
  }
  result += reduce16(acc);
  if (j < size) result += or_scalar_dot(OR_Q6_K, raw, off + j, x + j, size - j);
  return result;
}

/* F16FloatTensor.kt:43-77 / BF16FloatTensor.kt:35-73 / F32FloatTensor.kt:37-65:
 * fma over 16 lanes up to loopBound(size), reduceLanes, scalar tail. */
static float vdot_dense(int type, const uint8_t *raw, int64_t off, const float *x, int32_t size) {
  float value[16] = {0};
  int32_t upper = size & ~15;
  for (int32_t i = 0; i < upper; i += 16) {
    for (int l = 0; l < 16; l++) {
      int64_t e = off + i + l;
      float w;
      if (type == OR_F16)
        w = or_fp16_vec_decode(rd16(raw + e * 2));
      else if (type == OR_BF16)
        w = or_bf16_to_f32(rd16(raw + e * 2));
      else
        memcpy(&w, raw + e * 4, 4);
      value[l] = fmaf(w, x[i + l], value[l]);
    }
  }
  float result = reduce16(value);
  if (upper < size) result += or_scalar_dot(type, raw, off + upper, x + upper, size - upper);
  return result;
}

float or_vector_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size) {
  switch (type) {
    case OR_Q8_0: return vdot_q8_0(raw, this_offset, x, size);
    case OR_Q4_0: return vdot_q4_0(raw, this_offset, x, size);
    case OR_Q4_K: return vdot_q4_k(raw, this_offset, x, size);
    case OR_Q5_K: return vdot_q5_k(raw, this_offset, x, size);
    case OR_Q6_K: return vdot_q6_k(raw, this_offset, x, size);
    case OR_F16:
    case OR_BF16:
    case OR_F32: return vdot_dense(type, raw, this_offset, x, size);
    default: return NAN;
  }
}

float or_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size, int mode) {
  return mode == OR_MODE_SCALAR ? or_scalar_dot(type, raw, this_offset, x, size)
                                : or_vector_dot(type, raw, this_offset, x, size);
}

double or_exact_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size,
                    double *abs_sum) {
  double s = 0.0, a = 0.0;
  for (int32_t j = 0; j < size; j++) {
    double p = (double)or_get(type, raw, this_offset + j) * (double)x[j]; /* exact: 24x24 bits */
    s += p;
    a += fabs(p);
  }
  if (abs_sum) *abs_sum = a;
  return s;
}

/* FloatTensor.kt:18-29 matmul over rows (Parallel.kt:5-7 parallelFor). */
void or_matmul(int type, const uint8_t *raw, int64_t this_offset, const float *x, float *out, int32_t dim0,
               int32_t dim1, int mode, int nthreads) {
#ifdef _OPENMP
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
  for (int32_t i = 0; i < dim0; i++)
    out[i] = or_dot(type, raw, this_offset + (int64_t)i * dim1, x, dim1, mode);
  (void)nthreads;
}

void or_matmul_exact(int type, const uint8_t *raw, int64_t this_offset, const float *x, double *out,
                     double *abs_out, int32_t dim0, int32_t dim1, int nthreads) {
#ifdef _OPENMP
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
  for (int32_t i = 0; i < dim0; i++) {
    double a = 0.0;
    out[i] = or_exact_dot(type, raw, this_offset + (int64_t)i * dim1, x, dim1, &a);
    if (abs_out) abs_out[i] = a;
  }
  (void)nthreads;
}

/* ------------------------------------------------------- argmax / routing --- */

/* FloatTensor.kt:53-66. */
int32_t or_argmax(const float *v, int32_t offset, int32_t size) {
  int32_t max_index = offset;
  float max_value = v[max_index];
  for (int32_t i = offset; i < offset + size; i++) {
    float f = v[i];
    if (f > max_value) {
      max_value = f;
      max_index = i;
    }
  }
  return max_index;
}

/* java.lang.Math.max(float, float): NaN if either is NaN; -0.0 < +0.0. */
static float java_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == 0.0f && b == 0.0f) return signbit(a) ? b : a;
  return a >= b ? a : b;
}

/* MutableFloatTensor.kt:54-59 softmaxInPlace; FloatTensor.kt:31-45 reduce/sum/max. */
void or_softmax(float *v, int32_t offset, int32_t size) {
  float max_val = -INFINITY;
  for (int32_t i = 0; i < size; i++) max_val = java_max(max_val, v[offset + i]);
  for (int32_t i = 0; i < size; i++) {
    float diff = v[offset + i] - max_val; /* Float subtraction, then toDouble */
    v[offset + i] = (float)exp((double)diff);
  }
  float sum = 0.0f;
  for (int32_t i = 0; i < size; i++) sum = sum + v[offset + i];
  for (int32_t i = 0; i < size; i++) v[offset + i] = v[offset + i] / sum;
}

/* Llama.kt:275-293. */
void or_topk(float *probs, int32_t n, int32_t k, int32_t *idx_out, float *val_out) {
  for (int32_t ki = 0; ki < k; ki++) {
    int32_t best_idx = 0;
    float best_val = -INFINITY;
    for (int32_t ei = 0; ei < n; ei++) {
      float value = probs[ei];
      if (value > best_val) {
        best_val = value;
        best_idx = ei;
      }
    }
    idx_out[ki] = best_idx;
    val_out[ki] = best_val;
    probs[best_idx] = -INFINITY;
  }
}

void or_route(const float *logits, int32_t n_experts, int32_t k, int renormalize, const float *expert_scale,
              int32_t *ids, float *weights) {
  float *p = (float *)malloc(sizeof(float) * (size_t)n_experts);
  memcpy(p, logits, sizeof(float) * (size_t)n_experts);
  or_softmax(p, 0, n_experts);
  or_topk(p, n_experts, k, ids, weights);
  if (renormalize) {
    float s = 0.0f;
    for (int32_t i = 0; i < k; i++) s = s + weights[i];
    for (int32_t i = 0; i < k; i++) weights[i] = weights[i] / s;
  }
  if (expert_scale)
    for (int32_t i = 0; i < k; i++) weights[i] = weights[i] * expert_scale[ids[i]];
  free(p);
}

/* kotlin.math.tanh = java.lang.Math.tanh (Llama.kt:23-25 gelu, :403-406 soft-cap).
   Restated with the steps of fdlibm's s_tanh.c (the algorithm of the JDK's
   StrictMath.tanh): |x| < 2^-55: x * (1 + x); |x| < 1: -t / (t + 2),
   t = expm1(-2|x|); |x| < 22: 1 - 2 / (t + 2), t = expm1(2|x|); beyond: 1; then
   x's sign.  expm1 is the C library's, not fdlibm's s_expm1.c, and the JVM may
   run an intrinsic for Math.tanh, so bit parity with the reference's tanh is
   unpinned; the function is pinned to within 2 ulps of tanh. */
double or_tanh(double x) {
  const double ax = fabs(x);
  double z = 1.0;
  if (isnan(x)) return x + x;
  if (ax < 0x1p-55) return x * (1.0 + x);
  if (ax < 1.0) {
    const double t = expm1(-2.0 * ax);
    z = -t / (t + 2.0);
  } else if (ax < 22.0) {
    const double t = expm1(2.0 * ax);
    z = 1.0 - 2.0 / (t + 2.0);
  }
  return signbit(x) ? -z : z;
}

/* Llama.kt:23-25: (0.5 * x * (1 + tanh(sqrt(2/PI) * (x + 0.044715 * x^3)))).toFloat(). */
float or_gelu(float xf) {
  double x = (double)xf;
  double inner = sqrt(2.0 / 3.141592653589793) * (x + 0.044715 * pow(x, 3.0));
  return (float)(0.5 * x * (1.0 + or_tanh(inner)));
}

/* ---------------------------------------------------------------- MoE ---- */

/* Llama.kt:300-337 for each token: for ki in topK order, gate_up matmul at
 * offset e*2*ff*dim, gelu(gate)*up, down matmul at offset e*dim*ff,
 * moeOutput = saxpy(finalWeight, expertDown). */
void or_moe(int type_gu, const uint8_t *gate_up, int type_dn, const uint8_t *down, int32_t dim, int32_t ff,
            const float *X, int32_t T, const int32_t *ids, const float *w, int32_t k, float *Y, int mode,
            int nthreads) {
  float *gu = (float *)malloc(sizeof(float) * 2 * (size_t)ff);
  float *dn = (float *)malloc(sizeof(float) * (size_t)dim);
  for (int32_t t = 0; t < T; t++) {
    float *out = Y + (size_t)t * dim;
    for (int32_t i = 0; i < dim; i++) out[i] = 0.0f;
    for (int32_t ki = 0; ki < k; ki++) {
      int64_t e = ids[(size_t)t * k + ki];
      or_matmul(type_gu, gate_up, e * 2 * ff * (int64_t)dim, X + (size_t)t * dim, gu, 2 * ff, dim, mode, nthreads);
      for (int32_t i = 0; i < ff; i++) gu[i] = or_gelu(gu[i]);
      for (int32_t i = 0; i < ff; i++) gu[i] = gu[i] * gu[ff + i];
      or_matmul(type_dn, down, e * (int64_t)dim * ff, gu, dn, dim, ff, mode, nthreads);
      float a = w[(size_t)t * k + ki];
      for (int32_t i = 0; i < dim; i++) out[i] = a * dn[i] + out[i];
    }
  }
  free(gu);
  free(dn);
}

/* fp64 version plus an error scale per output: every dot may be off by 1e-5 of
 * its sum |w*x|; that error is carried through gelu (|gelu'| < 1.2) and the
 * product with up, then through the down projection and the gate weights.
 * A tolerance check uses |Y - Y64| <= 1e-5 * bound64. */
void or_moe_exact(int type_gu, const uint8_t *gate_up, int type_dn, const uint8_t *down, int32_t dim,
                  int32_t ff, const float *X, int32_t T, const int32_t *ids, const float *w, int32_t k,
                  double *Y64, double *bound64, int nthreads) {
  double *gu = (double *)malloc(sizeof(double) * 2 * (size_t)ff);
  double *gua = (double *)malloc(sizeof(double) * 2 * (size_t)ff);
  double *h = (double *)malloc(sizeof(double) * (size_t)ff);
  double *hb = (double *)malloc(sizeof(double) * (size_t)ff);
  for (int32_t t = 0; t < T; t++) {
    double *out = Y64 + (size_t)t * dim;
    double *bnd = bound64 + (size_t)t * dim;
    for (int32_t i = 0; i < dim; i++) out[i] = 0.0, bnd[i] = 0.0;
    for (int32_t ki = 0; ki < k; ki++) {
      int64_t e = ids[(size_t)t * k + ki];
      or_matmul_exact(type_gu, gate_up, e * 2 * ff * (int64_t)dim, X + (size_t)t * dim, gu, gua, 2 * ff, dim,
                      nthreads);
      for (int32_t i = 0; i < ff; i++) {
        double g = gu[i], u = gu[ff + i];
        double gl = 0.5 * g * (1.0 + or_tanh(sqrt(2.0 / 3.141592653589793) * (g + 0.044715 * g * g * g)));
        h[i] = gl * u;
        /* error scale of h in units of 1e-5: 1.2*Sg*(|u| + 1e-5*Su) + |gelu(g)|*Su, plus fp32 rounding of h */
        hb[i] = 1.2 * gua[i] * (fabs(u) + 1e-5 * gua[ff + i]) + fabs(gl) * gua[ff + i] + fabs(h[i]) * 0.05;
      }
      double a = (double)w[(size_t)t * k + ki];
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
      for (int32_t r = 0; r < dim; r++) {
        double s = 0.0, sa = 0.0, sh = 0.0;
        int64_t base = e * (int64_t)dim * ff + (int64_t)r * ff;
        for (int32_t i = 0; i < ff; i++) {
          double wd = (double)or_get(type_dn, down, base + i);
          s += wd * h[i];
          sa += fabs(wd * h[i]);
          sh += fabs(wd) * hb[i];
        }
        out[r] += a * s;
        bnd[r] += fabs(a) * (sa + sh) + fabs(a * s) * 0.05;
      }
    }
  }
  free(gu);
  free(gua);
  free(h);
  free(hb);
}

/* ---------------------------------------------------------- decode step --- */

/* Llama.kt:27-78, the three rmsnorm forms.  ss is the sequential fp32 sum of
 * x*x (FloatTensor.kt:31-37 reduce in the first form, an explicit loop in the
 * others: the same roundings), then ss /= size, ss += eps and
 * s = (float)(1.0 / sqrt((double)ss)).  out may alias x. */
void or_rmsnorm(float *out, const float *x, const float *w, int32_t size, float eps, int form) {
  float ss = 0.0f;
  for (int32_t i = 0; i < size; i++) {
    float xi = x[i];
    ss = ss + xi * xi;
  }
  ss = ss / (float)size;
  ss = ss + eps;
  float s = (float)(1.0 / sqrt((double)ss));
  for (int32_t i = 0; i < size; i++) {
    if (form == OR_NORM_WEIGHT_AFTER) out[i] = w[i] * (s * x[i]); /* Llama.kt:33-36 */
    else if (form == OR_NORM_WEIGHT_FIRST) out[i] = w[i] * s * x[i]; /* Llama.kt:56-58 */
    else out[i] = s * x[i]; /* Llama.kt:75-77 */
  }
}

/* fp64: s = 1/sqrt(sum x^2 / size + eps), out = w * s * x (w NULL: 1). */
void or_rmsnorm_exact(double *out, const float *x, const float *w, int32_t size, float eps) {
  double ss = 0.0;
  for (int32_t i = 0; i < size; i++) ss += (double)x[i] * (double)x[i];
  double s = 1.0 / sqrt(ss / (double)size + (double)eps);
  for (int32_t i = 0; i < size; i++) out[i] = (w ? (double)w[i] : 1.0) * s * (double)x[i];
}

/* Llama.kt:403-406: cap * tanh((v / cap).toDouble()).toFloat(). */
void or_softcap(float *v, int32_t n, float cap) {
  for (int32_t i = 0; i < n; i++) {
    float q = v[i] / cap;
    float t = (float)or_tanh((double)q);
    v[i] = cap * t;
  }
}

/* Llama.kt:355-363 dense FFN block, in place on x. */
void or_ffn_block(int type_g, const uint8_t *gate, int type_u, const uint8_t *up, int type_d, const uint8_t *down,
                  const float *norm_pre, const float *norm_post, float *x, int32_t dim, int32_t hidden, float eps,
                  int mode, int nthreads) {
  float *xb = (float *)malloc(sizeof(float) * (size_t)dim);
  float *hb = (float *)malloc(sizeof(float) * (size_t)hidden);
  float *hb2 = (float *)malloc(sizeof(float) * (size_t)hidden);
  or_rmsnorm(xb, x, norm_pre, dim, eps, OR_NORM_WEIGHT_AFTER);
  or_matmul(type_g, gate, 0, xb, hb, hidden, dim, mode, nthreads);
  or_matmul(type_u, up, 0, xb, hb2, hidden, dim, mode, nthreads);
  for (int32_t i = 0; i < hidden; i++) hb[i] = or_gelu(hb[i]);
  for (int32_t i = 0; i < hidden; i++) hb[i] = hb[i] * hb2[i];
  or_matmul(type_d, down, 0, hb, xb, dim, hidden, mode, nthreads);
  or_rmsnorm(xb, xb, norm_post, dim, eps, OR_NORM_WEIGHT_AFTER);
  for (int32_t i = 0; i < dim; i++) x[i] = x[i] + xb[i];
  free(xb);
  free(hb);
  free(hb2);
}

/* y = W x over fp64 inputs, with ya = sum |w x| and (bx != NULL) yb = sum |w| bx. */
static void mv_exact64(int type, const uint8_t *raw, const double *x, const double *bx, double *y, double *ya,
                       double *yb, int32_t dim0, int32_t dim1, int nthreads) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (int32_t i = 0; i < dim0; i++) {
    double s = 0.0, sa = 0.0, sb = 0.0;
    const int64_t base = (int64_t)i * dim1;
    for (int32_t j = 0; j < dim1; j++) {
      double wv = (double)or_get(type, raw, base + j);
      double p = wv * x[j];
      s += p;
      sa += fabs(p);
      if (bx) sb += fabs(wv) * bx[j];
    }
    y[i] = s;
    ya[i] = sa;
    if (yb) yb[i] = sb;
  }
  (void)nthreads;
}

/* fp64 FFN block plus an error scale in units of 1e-5 (a check uses
 * |x - x64| <= 1e-5 * bound64).  Budget: each rms scale is off by at most 1e-5
 * relative, each dot by 1e-5 of its sum |w x|; the errors are carried through
 * gelu (|gelu'| < 1.2), the product, the down projection, the post-norm (whose
 * scale moves by sum |y| dy / (sum y^2 + dim eps)) and the residual add. */
void or_ffn_block_exact(int type_g, const uint8_t *gate, int type_u, const uint8_t *up, int type_d,
                        const uint8_t *down, const float *norm_pre, const float *norm_post, const float *x,
                        double *x64, double *bound64, int32_t dim, int32_t hidden, float eps, int nthreads) {
  double *xb = (double *)malloc(sizeof(double) * (size_t)dim);
  double *bxb = (double *)malloc(sizeof(double) * (size_t)dim);
  double *g = (double *)malloc(sizeof(double) * (size_t)hidden), *ag = (double *)malloc(sizeof(double) * (size_t)hidden);
  double *u = (double *)malloc(sizeof(double) * (size_t)hidden), *au = (double *)malloc(sizeof(double) * (size_t)hidden);
  double *h = (double *)malloc(sizeof(double) * (size_t)hidden), *bh = (double *)malloc(sizeof(double) * (size_t)hidden);
  double *y = (double *)malloc(sizeof(double) * (size_t)dim), *ay = (double *)malloc(sizeof(double) * (size_t)dim);
  double *by = (double *)malloc(sizeof(double) * (size_t)dim);
  or_rmsnorm_exact(xb, x, norm_pre, dim, eps);
  for (int32_t j = 0; j < dim; j++) bxb[j] = fabs(xb[j]);
  mv_exact64(type_g, gate, xb, NULL, g, ag, NULL, hidden, dim, nthreads);
  mv_exact64(type_u, up, xb, NULL, u, au, NULL, hidden, dim, nthreads);
  for (int32_t i = 0; i < hidden; i++) {
    double gi = g[i];
    double gl = 0.5 * gi * (1.0 + or_tanh(sqrt(2.0 / 3.141592653589793) * (gi + 0.044715 * gi * gi * gi)));
    h[i] = gl * u[i];
    /* g and u are off by their dot error plus the carried norm error: 2 * sum |w xb| */
    double bg = 2.0 * ag[i], bu = 2.0 * au[i];
    bh[i] = 1.2 * bg * (fabs(u[i]) + 1e-5 * bu) + fabs(gl) * bu + 0.05 * fabs(h[i]);
  }
  mv_exact64(type_d, down, h, bh, y, ay, by, dim, hidden, nthreads);
  double ss = 0.0, sdy = 0.0;
  for (int32_t r = 0; r < dim; r++) {
    by[r] += ay[r];
    ss += y[r] * y[r];
    sdy += fabs(y[r]) * by[r];
  }
  double s = 1.0 / sqrt(ss / (double)dim + (double)eps);
  double rel_s = sdy / (ss + (double)dim * (double)eps) + 1.0;
  for (int32_t r = 0; r < dim; r++) {
    double z = (double)norm_post[r] * s * y[r];
    double bz = fabs((double)norm_post[r]) * s * by[r] + fabs(z) * (rel_s + 0.05);
    x64[r] = (double)x[r] + z;
    bound64[r] = bz + 0.01 * fabs(x64[r]);
  }
  free(xb); free(bxb); free(g); free(ag); free(u); free(au); free(h); free(bh); free(y); free(ay); free(by);
}

/* Llama.kt:401-407 then Sampler.ARGMAX (FloatTensor.kt:53-66): logits =
 * softcap(W rmsnorm(x)) (no cap when cap <= 0); returns the arg-max.  x is not
 * modified (the reference normalises it in place). */
int32_t or_lm_head(int type, const uint8_t *w, const float *norm, const float *x, float *logits, int32_t vocab,
                   int32_t dim, float eps, float cap, int mode, int nthreads) {
  float *xb = (float *)malloc(sizeof(float) * (size_t)dim);
  or_rmsnorm(xb, x, norm, dim, eps, OR_NORM_WEIGHT_AFTER);
  or_matmul(type, w, 0, xb, logits, vocab, dim, mode, nthreads);
  if (cap > 0.0f) or_softcap(logits, vocab, cap);
  free(xb);
  return or_argmax(logits, 0, vocab);
}

/* fp64 logits plus error scale (units of 1e-5): the dot error plus the carried
 * norm error (2 sum |w xb|); the cap has slope <= 1 and adds its roundings. */
void or_lm_head_exact(int type, const uint8_t *w, const float *norm, const float *x, double *logits64,
                      double *bound64, int32_t vocab, int32_t dim, float eps, float cap, int nthreads) {
  double *xb = (double *)malloc(sizeof(double) * (size_t)dim);
  or_rmsnorm_exact(xb, x, norm, dim, eps);
  mv_exact64(type, w, xb, NULL, logits64, bound64, NULL, vocab, dim, nthreads);
  for (int32_t i = 0; i < vocab; i++) {
    bound64[i] *= 2.0;
    if (cap > 0.0f) logits64[i] = (double)cap * or_tanh(logits64[i] / (double)cap);
    bound64[i] += 0.05 * fabs(logits64[i]);
  }
  free(xb);
}

/* ------------------------------------------------------------ attention --- */

/* ArrayFloatTensor.kt:66-88 vectorDot of two float arrays (512-bit species):
 * 16-lane fma accumulation, reduceLanes, then the scalar tail. */
static float array_vdot(const float *a, const float *b, int32_t n) {
  float acc[16] = {0};
  int32_t ub = n & ~15;
  for (int32_t i = 0; i < ub; i += 16)
    for (int l = 0; l < 16; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
  float r = reduce16(acc);
  for (int32_t i = ub; i < n; i++) r += a[i] * b[i];
  return r;
}

/* Llama.kt:198-218 for every head of one layer at one position: scores
 * q_h . K[t] (scale 1) for t in att_start..position, softmaxInPlace, then
 * out_h = sum_t a_t V[t] as saxpyInPlace in t order.  Head h reads kv head
 * h / (n_heads / n_kv); row t of a cache starts at t * n_kv * hs. */
void or_attention(const float *q, const float *kc, const float *vc, float *out, int32_t n_heads, int32_t n_kv,
                  int32_t hs, int32_t position, int32_t att_start) {
  const int32_t kv_dim = n_kv * hs, kv_mul = n_heads / n_kv, L = position - att_start + 1;
  float *att = (float *)malloc(sizeof(float) * (size_t)(L > 0 ? L : 1));
  for (int32_t h = 0; h < n_heads; h++) {
    const int32_t kvh = h / kv_mul;
    for (int32_t t = att_start; t <= position; t++)
      att[t - att_start] = array_vdot(q + (size_t)h * hs, kc + (size_t)t * kv_dim + (size_t)kvh * hs, hs);
    or_softmax(att, 0, L);
    float *o = out + (size_t)h * hs;
    for (int32_t i = 0; i < hs; i++) o[i] = 0.0f;
    for (int32_t t = att_start; t <= position; t++) {
      const float a = att[t - att_start];
      const float *v = vc + (size_t)t * kv_dim + (size_t)kvh * hs;
      for (int32_t i = 0; i < hs; i++) o[i] = a * v[i] + o[i];
    }
  }
  free(att);
}

/* fp64 attention plus an error scale in units of 1e-5 (|out - out64| <= 1e-5 *
 * bound64): each score may be off by 1e-5 of its sum |q k|, which moves each
 * softmax weight by at most 2 max_t(error) of itself; the weighted sums add
 * rounding of a few units of 1e-5 of sum a |v|. */
void or_attention_exact(const float *q, const float *kc, const float *vc, double *out64, double *bound64,
                        int32_t n_heads, int32_t n_kv, int32_t hs, int32_t position, int32_t att_start,
                        int nthreads) {
  const int32_t kv_dim = n_kv * hs, kv_mul = n_heads / n_kv, L = position - att_start + 1;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
  for (int32_t h = 0; h < n_heads; h++) {
    const int32_t kvh = h / kv_mul;
    double *s = (double *)malloc(sizeof(double) * (size_t)L);
    double smax = -INFINITY, amax = 0.0;
    for (int32_t t = 0; t < L; t++) {
      const float *k = kc + (size_t)(att_start + t) * kv_dim + (size_t)kvh * hs;
      double d = 0.0, a = 0.0;
      for (int32_t i = 0; i < hs; i++) {
        double p = (double)q[(size_t)h * hs + i] * (double)k[i];
        d += p;
        a += fabs(p);
      }
      s[t] = d;
      if (d > smax) smax = d;
      if (a > amax) amax = a;
    }
    double sum = 0.0;
    for (int32_t t = 0; t < L; t++) {
      s[t] = exp(s[t] - smax);
      sum += s[t];
    }
    for (int32_t i = 0; i < hs; i++) {
      double o = 0.0, oa = 0.0;
      for (int32_t t = 0; t < L; t++) {
        const double v = (double)vc[(size_t)(att_start + t) * kv_dim + (size_t)kvh * hs + i];
        o += s[t] * v;
        oa += s[t] * fabs(v);
      }
      out64[(size_t)h * hs + i] = o / sum;
      bound64[(size_t)h * hs + i] = (2.0 * amax + 5.0) * oa / sum;
    }
    free(s);
  }
  (void)nthreads;
}
