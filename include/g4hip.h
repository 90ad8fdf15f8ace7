/*
 * g4hip.h -- C ABI of the MI355X (gfx950) quantized matrix-vector library.
 *
 * Drop-in boundary for gemma4.kt's tensor layer.  Reference paths are relative to
 * lib/src/main/kotlin/io/github/lbenedetto/internal/.  The Kotlin side binds these
 * symbols with java.lang.foreign (FFM); a Kotlin FloatTensor implementation
 * overrides both matmul overloads and forwards here.
 *
 * Conventions
 *  - Every function returns an int status: G4_OK (0) or a negative G4_ERR_*.
 *    g4_last_error() returns a thread-local message for the last failure.
 *  - Weights are raw GGUF blocks uploaded once (no repacking) and stay in HBM
 *    until g4_weight_free; a weight is read-only and may be shared by every
 *    context on its device.
 *  - A g4_ctx owns a HIP stream and staging buffers.  One thread uses a context
 *    at a time (the reference runs one generation thread per LlamaState); open one
 *    context per thread for concurrency.
 *  - Host-pointer entry points are synchronous: outputs are complete on return,
 *    like FloatTensor.matmul.  *_dev entry points take device pointers and are
 *    asynchronous on the context's stream (g4_ctx_set_stream can point it at a
 *    caller's stream; g4_ctx_sync waits).
 *  - Element offsets are int64 (the reference's Int offsets overflow past 2^31).
 */
#ifndef G4HIP_H
#define G4HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes and the Kotlin exception each maps to. */
#define G4_OK 0
#define G4_ERR_INVALID_ARGUMENT (-1) /* IllegalArgumentException (null pointer, bad size, bad dims) */
#define G4_ERR_UNSUPPORTED (-2)      /* UnsupportedOperationException (GGML type id), FloatTensorFactory.kt:21 */
#define G4_ERR_OUT_OF_RANGE (-3)     /* IndexOutOfBoundsException (offset/rows past the tensor) */
#define G4_ERR_NO_DEVICE (-4)        /* IllegalStateException: no HIP device */
#define G4_ERR_DEVICE (-5)           /* IllegalStateException: HIP runtime failure */
#define G4_ERR_OUT_OF_MEMORY (-6)    /* OutOfMemoryError: device allocation failed */

/* GGML type ids accepted by g4_upload (GGMLType.kt:16-56, id = ordinal). */
#define G4_TYPE_F32 0
#define G4_TYPE_F16 1
#define G4_TYPE_Q4_0 2
#define G4_TYPE_Q8_0 8
#define G4_TYPE_Q4_K 12
#define G4_TYPE_Q5_K 13
#define G4_TYPE_Q6_K 14
#define G4_TYPE_BF16 30

typedef struct g4_ctx g4_ctx;
typedef struct g4_weight g4_weight;

/* Thread-local message of the last failing call on this thread ("" if none). */
const char *g4_last_error(void);

/* Library version, (major << 16) | minor. */
int g4_version(void);

/* Number of visible HIP devices (0 and G4_OK when there is none). */
int g4_device_count(int *count);

/* GGMLType.kt:16-30 blockSize/typeSize and byteSizeFor (:58-62) for a type id.
 * Returns G4_ERR_UNSUPPORTED for ids outside the supported set. */
int g4_type_info(int ggml_type, int *block_size, int *type_size);
int g4_byte_size(int ggml_type, int64_t n_elems, int64_t *nbytes);

/* Host-only validation of a matmul geometry against a tensor of `n_elems`
 * elements of `ggml_type`: the status g4_matmul would return before launching
 * (FloatTensor.kt:18-29 rows this_offset + i*dim1 .. +dim1, i < dim0, must lie
 * inside the tensor).  Needs no device. */
int g4_check_matmul(int ggml_type, int64_t n_elems, int64_t this_offset, int32_t dim0, int32_t dim1);

/* Open / close a context on device `ordinal` (creates the context's stream). */
int g4_open(int ordinal, g4_ctx **out);
int g4_close(g4_ctx *ctx);
/* Launch subsequent *_dev work on `stream` (a hipStream_t; NULL = the context's own). */
int g4_ctx_set_stream(g4_ctx *ctx, void *stream);
int g4_ctx_sync(g4_ctx *ctx);
int g4_ctx_device(const g4_ctx *ctx, int *ordinal);
/* Scratch for HIP graph capture.  *_dev calls keep intermediates (MoE hidden
 * vectors, attention and column-split partials, a standalone norm) in a
 * per-context device buffer that grows on demand.  A graph captured over such a
 * call keeps that buffer's address, so:
 *  - g4_ctx_reserve grows the buffer to `bytes` now (call it, or run the largest
 *    shapes once eagerly, before capturing);
 *  - a call that needs more than is reserved while its stream is capturing
 *    returns G4_ERR_INVALID_ARGUMENT and records nothing;
 *  - once any call on the context has been captured, an outgrown buffer is kept
 *    allocated (graphs may still replay into it) until g4_close.
 * Host-pointer calls synchronise and return G4_ERR_INVALID_ARGUMENT under capture.
 * No counterpart in the reference (its matmul is synchronous CPU code). */
int g4_ctx_reserve(g4_ctx *ctx, int64_t bytes);
int g4_ctx_scratch_bytes(const g4_ctx *ctx, int64_t *bytes);

/* FloatTensorFactory.kt:7-23 create(ggmlType, entry) + the GGUF slice of
 * GGUF.kt:195-212: copy `nbytes` raw GGUF bytes holding `n_elems` elements to HBM.
 * nbytes must equal byteSizeFor(n_elems) (GGMLType.kt:58-62). */
int g4_upload(g4_ctx *ctx, int ggml_type, const void *raw, int64_t nbytes, int64_t n_elems, g4_weight **out);
int g4_weight_free(g4_weight *w);
int g4_weight_info(const g4_weight *w, int *ggml_type, int64_t *n_elems, int64_t *nbytes);
/* Device address of the uploaded blocks (read-only; for callers that launch on it). */
int g4_weight_device_ptr(const g4_weight *w, const void **dptr);

/* FloatTensor.matmul(that, out, dim0, dim1, thisOffset), FloatTensor.kt:18-29:
 *   out[i] = dot(this_offset + i*dim1, that, 0, dim1) for i in [0, dim0).
 * that: host float[dim1], out: host float[dim0].  Synchronous. */
int g4_matmul(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *that, float *out,
              int32_t dim0, int32_t dim1);
int g4_matmul_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *d_that, float *d_out,
                  int32_t dim0, int32_t dim1);

/* M independent activations (rows of X, row-major [M x dim1]) against the same
 * weight: Y[m*dim0 + i] = dot(this_offset + i*dim1, X[m], 0, dim1).  The reference
 * has no batched call; this is what M calls of matmul compute (Llama.kt:435-436). */
int g4_matmul_batch(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *X, int32_t M, float *Y,
                    int32_t dim0, int32_t dim1);
int g4_matmul_batch_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *d_X, int32_t M,
                        float *d_Y, int32_t dim0, int32_t dim1);

/* LM head: logits = matmul(...) (Llama.kt:402) and *index = argmax(logits)
 * (FloatTensor.kt:53-66: first index of the maximum; a NaN at index 0 wins,
 * NaN elsewhere never does).  logits may be NULL when only the index is wanted. */
int g4_matmul_argmax(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *that, float *logits,
                     int32_t *index, int32_t dim0, int32_t dim1);
int g4_matmul_argmax_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *d_that,
                         float *d_logits, int32_t *d_index, int32_t dim0, int32_t dim1);

/* FloatTensor.argmax(offset=0, size=n) of a float vector (FloatTensor.kt:53-66). */
int g4_argmax(g4_ctx *ctx, const float *v, int32_t n, int32_t *index);
int g4_argmax_dev(g4_ctx *ctx, const float *d_v, int32_t n, int32_t *d_index);

/* Per-element get() of every format (Q8_0FloatTensor.kt:21-28, Q4_0FloatTensor.kt:21-39,
 * Q4_KFloatTensor.kt:23-55, F16FloatTensor.kt:20-23, BF16FloatTensor.kt:20-24,
 * F32FloatTensor.kt:18-20): out[i] = get(offset + i), bit-exact; the embedding
 * lookup copyTo of Llama.kt:112. */
int g4_dequant(g4_ctx *ctx, const g4_weight *w, int64_t offset, int64_t n, float *out);
int g4_dequant_dev(g4_ctx *ctx, const g4_weight *w, int64_t offset, int64_t n, float *d_out);

/* FFN of one token (Llama.kt:357-361, MoE shared MLP :232-236):
 *   h = gelu(w_gate x) * (w_up x)  (gelu of Llama.kt:23-25),  y = w_down h.
 * w_gate, w_up: [hidden x dim], w_down: [dim x hidden]; x: float[dim], y: float[dim]. */
int g4_ffn(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down, const float *x,
           float *y, int32_t dim, int32_t hidden);
int g4_ffn_dev(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down,
               const float *d_x, float *d_y, int32_t dim, int32_t hidden);
/* The first half of that FFN (Llama.kt:357-360): h = gelu(w_gate x) * (w_up x),
 * h: float[hidden].  One fused launch; g4_ffn is this plus g4_matmul of w_down. */
int g4_ffn_gate_up(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const float *x, float *h,
                   int32_t dim, int32_t hidden);
int g4_ffn_gate_up_dev(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const float *d_x, float *d_h,
                       int32_t dim, int32_t hidden);

/* MoE routing of T tokens (Llama.kt:269-293): per token softmax over n_experts
 * router logits (MutableFloatTensor.kt:54-59, exp in double), top-k by repeated
 * strict-> scans (ties to the lowest index).  weights[t*k+j] = p (renormalize = 0,
 * the reference) or p / sum of the k chosen p in fp32, j order (renormalize = 1);
 * then times expert_scale[e] when expert_scale != NULL (ffn_down_exps_scale,
 * Llama.kt:302,334).  logits [T x n_experts]; ids, weights [T x k]. */
int g4_moe_route(g4_ctx *ctx, const float *logits, int32_t T, int32_t n_experts, int32_t k, int32_t renormalize,
                 const float *expert_scale, int32_t *ids, float *weights);
int g4_moe_route_dev(g4_ctx *ctx, const float *d_logits, int32_t T, int32_t n_experts, int32_t k,
                     int32_t renormalize, const float *d_expert_scale, int32_t *d_ids, float *d_weights);

/* Routed expert FFN (Llama.kt:300-337) for T tokens:
 *   Y[t] = sum_j weights[t,j] * down_e( gelu(gate_e X[t]) * up_e X[t] ),  e = ids[t,j]
 * w_gate_up: [n_experts x 2*ff x dim] (gate rows first, then up rows, per expert,
 * slab offset e*2*ff*dim); w_down: [n_experts x dim x ff] (offset e*dim*ff).
 * X [T x dim], ids/weights [T x k], Y [T x dim].
 * g4_moe checks every id against the experts the weights hold
 * (G4_ERR_OUT_OF_RANGE).  g4_moe_dev cannot (the ids are device memory): a slot
 * whose id lies outside [0, n_experts) contributes nothing (its hidden vector
 * and down rows are zero), so Y is the weighted sum over the valid slots.
 * Calls of 41 or more tokens with Q4_K weights (dim and ff multiples of 128 up
 * to 3072, at most 4096 (token, slot) pairs) run the experts grouped by expert
 * on the matrix cores: every dot within the same bound, but rounded differently
 * from the same tokens in smaller calls. */
int g4_moe(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *X, int32_t T,
           int32_t dim, int32_t ff, const int32_t *ids, const float *weights, int32_t k, float *Y);
int g4_moe_dev(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *d_X, int32_t T,
               int32_t dim, int32_t ff, const int32_t *d_ids, const float *d_weights, int32_t k, float *d_Y);

/* The routed MoE block of Llama.kt:269-337 from the router logits, in one call:
 * the routing of g4_moe_route (softmax, top-k, renormalize, expert_scale) and the
 * expert FFN and weighted sum of g4_moe.  logits [T x n_experts] (n_experts at
 * most the experts the weights hold); the routing is also returned in ids and
 * weights [T x k].  Up to 256 experts the routing runs inside the gate+up launch
 * (each workgroup routes its own token); above that, and for the calls that run
 * the experts grouped (see g4_moe), in a launch of its own.
 * Results are identical to g4_moe_route followed by g4_moe. */
int g4_moe_routed(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *X, int32_t T,
                  int32_t dim, int32_t ff, const float *logits, int32_t n_experts, int32_t k, int32_t renormalize,
                  const float *expert_scale, int32_t *ids, float *weights, float *Y);
int g4_moe_routed_dev(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *d_X, int32_t T,
                      int32_t dim, int32_t ff, const float *d_logits, int32_t n_experts, int32_t k,
                      int32_t renormalize, const float *d_expert_scale, int32_t *d_ids, float *d_weights,
                      float *d_Y);

/* g4_moe_routed_dev without any device allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same arguments, results
 * and bits as g4_moe_routed_dev; its intermediates live in a fixed 16 MiB device
 * array per GPU (held until the process ends) instead of the context's scratch,
 * so 4 * T * k * (3 * ff + dim) bytes (each part rounded up to 256) must fit:
 * larger calls return G4_ERR_INVALID_ARGUMENT.  Every call on one GPU shares
 * that array: calls that overlap on one GPU (other threads, other streams or
 * contexts) race and must be serialised by the caller. */
int g4_moe_routed_dev_noalloc(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *d_X,
                              int32_t T, int32_t dim, int32_t ff, const float *d_logits, int32_t n_experts, int32_t k,
                              int32_t renormalize, const float *d_expert_scale, int32_t *d_ids, float *d_weights,
                              float *d_Y);

/* ---- Decode step around the matvec: the activations stay in device memory. ----
 * Norm weights are uploaded F32 tensors (ModelLoader.kt:281-286 reads norms as
 * FloatBuffers and throws UnsupportedOperationException for any other type).
 * s = (float)(1.0 / sqrt((double)(ss / size + eps))), ss = fp32 sum of x*x. */
#define G4_NORM_WEIGHT_AFTER 0 /* Llama.kt:27-37 rmsnorm(out, x, weight, size, eps): w * (s * x) */
#define G4_NORM_WEIGHT_FIRST 1 /* Llama.kt:39-60 rmsnorm(out, outOffset, x, xOffset, ...): w * s * x */
#define G4_NORM_NO_WEIGHT 2    /* Llama.kt:62-78 rmsnormNoWeight: s * x */

/* rms norm of n_vec vectors of `size` floats (vector v at d_x + v*size; the per-head
 * q/k/v norms of Llama.kt:161-163, 185-188), each with its own scale and the shared
 * weight (NULL for G4_NORM_NO_WEIGHT).  d_out may be d_x (in place). */
int g4_rmsnorm_dev(g4_ctx *ctx, const g4_weight *weight, const float *d_x, float *d_out, int32_t n_vec, int32_t size,
                   float eps, int form);
/* Post-norm plus residual (Llama.kt:222-223, 362-363): v = rmsnorm(v) (the
 * G4_NORM_WEIGHT_AFTER form, in place), then x += v.  One launch. */
int g4_rmsnorm_add_dev(g4_ctx *ctx, const g4_weight *weight, float *d_v, float *d_x, int32_t size, float eps);
/* MutableFloatTensor.kt:28-37 addInPlace: x[i] = x[i] + that[i]. */
int g4_add_dev(g4_ctx *ctx, float *d_x, const float *d_that, int32_t n);
/* Llama.kt:403-406 final logit soft-capping in place: v = cap * (float)tanh((double)(v / cap)), cap > 0. */
int g4_softcap_dev(g4_ctx *ctx, float *d_v, int32_t n, float cap);
/* Norm then matmul (Llama.kt:155-158: xb = rmsnorm(x, weight); W.matmul(xb, out, dim0, dim1)):
 * out = W . rmsnorm(x) with the G4_NORM_WEIGHT_AFTER form fused into the matvec's
 * staging of x.  d_xnorm (NULL, or not overlapping d_x) receives rmsnorm(x). */
int g4_matmul_norm_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const g4_weight *norm, const float *d_x,
                       float eps, float *d_xnorm, float *d_out, int32_t dim0, int32_t dim1);
/* Dense FFN block of one token, in place on x (Llama.kt:355-363):
 *   xb = rmsnorm(x, norm_pre); h = gelu(w_gate xb) * (w_up xb); xb = rmsnorm(w_down h, norm_post); x += xb.
 * Three launches: gate/up with the fused pre-norm, down, post-norm plus residual. */
int g4_ffn_block(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down,
                 const g4_weight *norm_pre, const g4_weight *norm_post, float *x, int32_t dim, int32_t hidden,
                 float eps);
int g4_ffn_block_dev(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down,
                     const g4_weight *norm_pre, const g4_weight *norm_post, float *d_x, int32_t dim, int32_t hidden,
                     float eps);
/* Final norm, logits and greedy pick (Llama.kt:401-407, then Sampler.ARGMAX =
 * FloatTensor.argmax, FloatTensor.kt:53-66):
 *   logits = W_cls . rmsnorm(x, norm_final); if softcap > 0: logits = softcap(logits); index = argmax(logits).
 * logits may be NULL; d_xnorm (device form, NULL or not overlapping d_x) receives
 * rmsnorm(x), which the reference leaves in x. */
int g4_lm_head(g4_ctx *ctx, const g4_weight *w_cls, const g4_weight *norm_final, const float *x, float *logits,
               int32_t *index, int32_t vocab, int32_t dim, float eps, float softcap);
int g4_lm_head_dev(g4_ctx *ctx, const g4_weight *w_cls, const g4_weight *norm_final, const float *d_x, float *d_xnorm,
                   float *d_logits, int32_t *d_index, int32_t vocab, int32_t dim, float eps, float softcap);

/* Decode attention of one token over one layer's KV cache (Llama.kt:198-218):
 *   for each query head h (kv head h / (n_heads / n_kv_heads)), scores
 *   s_t = q_h . K[t] with scale 1 for t = att_start..position, softmax
 *   (MutableFloatTensor.kt:54-59: max, exp in double), out_h = sum_t a_t V[t].
 * d_q, d_out: [n_heads x head_size]; d_key_cache, d_value_cache: fp32 rows of
 * kv_dim = n_kv_heads * head_size floats, row t at t * kv_dim, holding at least
 * position + 1 rows.  att_start = max(0, position - window + 1) on sliding-window
 * layers, 0 otherwise (Llama.kt:197).  Head sizes 64/128/256/512 with 16-byte
 * aligned buffers take the split-sequence kernel (two launches); any other shape
 * takes a one-workgroup-per-head kernel. */
int g4_attention_dev(g4_ctx *ctx, const float *d_q, const float *d_key_cache, const float *d_value_cache,
                     float *d_out, int32_t n_heads, int32_t n_kv_heads, int32_t head_size, int32_t position,
                     int32_t att_start);

#ifdef __cplusplus
}
#endif
#endif
