/*
 * g4_oracle.h -- CPU restatement of gemma4.kt's quantized matrix-vector path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * library (libg4hip.so).  Only the test suite, the smoke check and the CPU
 * baseline leg of the benchmark may load it; the product never calls it.
 *
 * Every function cites the Kotlin reference it restates (paths relative to
 * lib/src/main/kotlin/io/github/lbenedetto/internal/).  How each function is
 * pinned (closed forms, independent numpy restatements, fp64 brute force) is
 * listed in the test files under tests/test_oracle_*.py.
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (gguf/GGMLType.kt:16-56: id = enum ordinal). */
enum {
  OR_F32 = 0,
  OR_F16 = 1,
  OR_Q4_0 = 2,
  OR_Q8_0 = 8,
  OR_Q4_K = 12,
  OR_Q5_K = 13,
  OR_Q6_K = 14,
  OR_BF16 = 30
};

/* Dot-product modes of or_matmul. */
enum {
  OR_MODE_VECTOR = 0, /* 512-bit vectorDot restatement (the JIT path on AVX-512) */
  OR_MODE_SCALAR = 1  /* FloatTensorHelpers.scalarDot (-Dllama.VectorBitSize=0) */
};

/* GGMLType.kt:16-56 blockSize / typeSize; 0 for unsupported ids. */
int or_block_size(int type);
int or_type_size(int type);

/* FloatTensorHelpers.kt:39-41 readFloat16 -> java.lang.Float.float16ToFloat
 * (IEEE binary16 -> binary32, exact, subnormals kept). */
float or_fp16_to_f32(uint16_t h);
/* F16FloatTensor.kt:59-61: the bit trick of the vector path (zero exponent
 * flushes to +-0, exponent 31 maps to the finite 2^16 * 1.m). */
float or_fp16_vec_decode(uint16_t h);
/* BF16FloatTensor.kt:20-24: bits << 16. */
float or_bf16_to_f32(uint16_t h);
/* Array forms (keep signalling-NaN bit patterns, which a scalar return through
 * a foreign-function layer may quiet). */
void or_fp16_to_f32_array(const uint16_t *h, int64_t n, float *out);
void or_fp16_vec_decode_array(const uint16_t *h, int64_t n, float *out);

/* Per-format get(index) (dequantization of one element).
 * Q8_0FloatTensor.kt:21-28, Q4_0FloatTensor.kt:21-39, Q4_KFloatTensor.kt:23-55,
 * Q5_KFloatTensor.kt:23-50, Q6_KFloatTensor.kt:26-75,
 * F16FloatTensor.kt:20-23, BF16FloatTensor.kt:20-24, F32FloatTensor.kt:18-20. */
float or_get(int type, const uint8_t *raw, int64_t index);
void or_dequant(int type, const uint8_t *raw, int64_t offset, int64_t n, float *out);

/* Q4_KFloatTensor.kt:70-84 getScaleMinK4. */
int or_q4k_scale_min(int j, const uint8_t *scales12, int is_min);

/* FloatTensorHelpers.kt:65-71 scalarDot: sequential fp32 sum of get(i)*x[i]. */
float or_scalar_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size);

/* Lane-order restatement of the 512-bit branch of each vectorDot, including the
 * scalar head and tail.  Q8_0FloatTensor.kt:39-142, Q4_0FloatTensor.kt:50-146,
 * Q4_KFloatTensor.kt:86-207, F16FloatTensor.kt:43-77, BF16FloatTensor.kt:35-73,
 * F32FloatTensor.kt:37-65. */
float or_vector_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size);

/* The dot the reference's dispatch picks (FloatTensor.dot overrides): vector or scalar. */
float or_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size, int mode);

/* Exact reference value: sum of (double)get(i) * (double)x[i] in fp64, and the
 * tolerance scale sum |get(i) * x[i]| (fp64). */
double or_exact_dot(int type, const uint8_t *raw, int64_t this_offset, const float *x, int32_t size,
                    double *abs_sum);

/* FloatTensor.kt:18-29 matmul: out[i] = dot(this_offset + i*dim1, x, 0, dim1).
 * nthreads > 1 parallelises over rows like Parallel.kt:5-7. */
void or_matmul(int type, const uint8_t *raw, int64_t this_offset, const float *x, float *out,
               int32_t dim0, int32_t dim1, int mode, int nthreads);
/* fp64 exact matmul plus per-row sum |w*x| (tolerance scale). */
void or_matmul_exact(int type, const uint8_t *raw, int64_t this_offset, const float *x, double *out,
                     double *abs_out, int32_t dim0, int32_t dim1, int nthreads);

/* FloatTensor.kt:53-66 argmax: first index of the maximum (strict >). */
int32_t or_argmax(const float *v, int32_t offset, int32_t size);

/* MutableFloatTensor.kt:54-59 softmaxInPlace (exp in double, fp32 sum). */
void or_softmax(float *v, int32_t offset, int32_t size);
/* Llama.kt:275-293 top-k by repeated strict-> scans with -inf masking.
 * probs is modified (chosen entries set to -inf), as in the reference. */
void or_topk(float *probs, int32_t n, int32_t k, int32_t *idx_out, float *val_out);
/* Routing of one token: softmax, top-k, then (renormalize != 0) w_k = p_k / sum_j p_j
 * with the sum in fp32 in k order, else w_k = p_k; times expert_scale[e] if given
 * (Llama.kt:300-304 finalWeight = prob * downScale). */
void or_route(const float *logits, int32_t n_experts, int32_t k, int renormalize,
              const float *expert_scale, int32_t *ids, float *weights);
/* Math.tanh as StrictMath.tanh computes it (fdlibm's algorithm, the C library's expm1). */
double or_tanh(double x);
/* Llama.kt:23-25 gelu (tanh form, evaluated in double). */
float or_gelu(float x);

/* Llama.kt:300-337: routed expert FFN of T tokens with given expert ids and gate weights.
 * gate_up: [n_experts x 2*ff x dim], down: [n_experts x dim x ff].  Y[t] = sum_k w_tk * down_e(gelu(g)*u),
 * accumulated in k order like saxpyInPlace (MutableFloatTensor.kt:61-66).  mode as or_matmul.
 * With exact != 0 everything is done in fp64 (out64 used, may be NULL otherwise) and
 * bound64[t*dim+r] receives an error scale for the tolerance check. */
void or_moe(int type_gu, const uint8_t *gate_up, int type_dn, const uint8_t *down, int32_t dim, int32_t ff,
            const float *X, int32_t T, const int32_t *ids, const float *w, int32_t k, float *Y, int mode,
            int nthreads);
void or_moe_exact(int type_gu, const uint8_t *gate_up, int type_dn, const uint8_t *down, int32_t dim,
                  int32_t ff, const float *X, int32_t T, const int32_t *ids, const float *w, int32_t k,
                  double *Y64, double *bound64, int nthreads);

/* ---- decode step ---- */
/* rmsnorm forms: Llama.kt:27-37 w * (s * x); Llama.kt:39-60 w * s * x; Llama.kt:62-78 s * x. */
enum { OR_NORM_WEIGHT_AFTER = 0, OR_NORM_WEIGHT_FIRST = 1, OR_NORM_NO_WEIGHT = 2 };
/* s = (float)(1.0 / sqrt((double)(ss / size + eps))), ss the sequential fp32 sum of x*x.  out may alias x. */
void or_rmsnorm(float *out, const float *x, const float *w, int32_t size, float eps, int form);
/* fp64 rms norm (w NULL: no weight). */
void or_rmsnorm_exact(double *out, const float *x, const float *w, int32_t size, float eps);
/* Llama.kt:403-406 logit soft-capping in place. */
void or_softcap(float *v, int32_t n, float cap);
/* Llama.kt:355-363 dense FFN block in place on x (weights at offset 0). */
void or_ffn_block(int type_g, const uint8_t *gate, int type_u, const uint8_t *up, int type_d, const uint8_t *down,
                  const float *norm_pre, const float *norm_post, float *x, int32_t dim, int32_t hidden, float eps,
                  int mode, int nthreads);
/* fp64 FFN block and an error scale: a check uses |x - x64| <= 1e-5 * bound64. */
void or_ffn_block_exact(int type_g, const uint8_t *gate, int type_u, const uint8_t *up, int type_d,
                        const uint8_t *down, const float *norm_pre, const float *norm_post, const float *x,
                        double *x64, double *bound64, int32_t dim, int32_t hidden, float eps, int nthreads);
/* Llama.kt:401-407 + FloatTensor.kt:53-66: logits = softcap(W rmsnorm(x)) (cap <= 0: none); returns the arg-max. */
int32_t or_lm_head(int type, const uint8_t *w, const float *norm, const float *x, float *logits, int32_t vocab,
                   int32_t dim, float eps, float cap, int mode, int nthreads);
/* fp64 logits and error scale (|logit - l64| <= 1e-5 * bound64). */
void or_lm_head_exact(int type, const uint8_t *w, const float *norm, const float *x, double *logits64,
                      double *bound64, int32_t vocab, int32_t dim, float eps, float cap, int nthreads);

/* Llama.kt:198-218: decode attention of every head over the KV cache rows
 * att_start..position (scale 1, head h reads kv head h / (n_heads / n_kv), row t
 * of a cache at t * n_kv * hs). */
void or_attention(const float *q, const float *kc, const float *vc, float *out, int32_t n_heads, int32_t n_kv,
                  int32_t hs, int32_t position, int32_t att_start);
/* fp64 attention and error scale (|out - out64| <= 1e-5 * bound64). */
void or_attention_exact(const float *q, const float *kc, const float *vc, double *out64, double *bound64,
                        int32_t n_heads, int32_t n_kv, int32_t hs, int32_t position, int32_t att_start,
                        int nthreads);

#ifdef __cplusplus
}
#endif
#endif
