// g4_internal.hpp -- launcher interface between the C ABI (g4_api.hip) and the
// kernels (g4_kernels.hip).  Host-side only types; no torch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace g4 {

enum Epi : int { EPI_STORE = 0, EPI_ARGMAX = 1, EPI_GELU_PAIR = 2 };

// One "rows" launch: logical rows of one or two matrices dotted against x.
// Segment s (blockIdx.y) uses expert ids[s] (when ids != null), activation
// x + (s / x_div) * x_stride and output y + s * y_stride.  Matrix m row r of
// segment s starts at element base_m + ids[s] * expert_stride + r * row_stride.
struct RowsArgs {
  const uint8_t *W0;
  const uint8_t *W1;
  int64_t base0;
  int64_t base1;
  int64_t row_stride;
  int64_t expert_stride;
  const int32_t *ids;
  int32_t expert_count;  // ids outside [0, expert_count) give zero rows
  int32_t rows;
  int32_t dim1;
  const float *x;
  int64_t x_stride;
  int32_t x_div;
  float *y;
  int64_t y_stride;
  // EPI_ARGMAX: per-block partials (max_argmax_blocks() slots) and the result index
  float *am_val;
  int32_t *am_idx;
  int32_t *am_out;
  // EPI_ARGMAX: logits are soft-capped (Llama.kt:403-406) before the store and the
  // arg-max when softcap > 0
  float softcap;
  // Input rms norm (Llama.kt:27-37) fused into the x staging when norm_w != null:
  // every workgroup computes the scale of x and stages norm_w[j] * (s * x[j]); the
  // first workgroup also stores the normalised x to norm_out (when not null, and
  // not aliasing x).  Single-segment, single-pass launches only (rows_norm_ok).
  const float *norm_w;
  float norm_eps;
  float *norm_out;
  // MoE routing in the gate+up launch (EPI_GELU_PAIR) when route_logits != null:
  // segment s is (token s / x_div, slot s % x_div), k = x_div.  Every workgroup
  // routes its token from route_logits[token * route_e ...] (Llama.kt:269-293)
  // and takes its slot's expert; the workgroups with blockIdx.x == 0 store the
  // slot's expert id and weight to route_ids / route_w for the later launches.
  // ids is unused then.
  const float *route_logits;
  const float *route_scale;
  int32_t route_e;
  int32_t route_renorm;
  int32_t *route_ids;
  float *route_w;
};

// Device facts used for launch sizing.
struct DevInfo {
  int cu_count;
};

// True when rows of (type, offsets, dim1) take the 64-element chunk kernels.
bool rows_fast_ok(int type, const RowsArgs &a, bool paired);
// True when such a launch can also take the fused input norm (one column pass).
bool rows_norm_ok(int type, const RowsArgs &a, bool paired);

// Launch the matvec engine over `segments` segments.  For EPI_GELU_PAIR the
// launch writes h[r] = gelu(W0 row r . x) * (W1 row r . x); on the generic path
// that needs `scratch` of 2 * rows * segments floats.  For EPI_ARGMAX, segments
// must be 1 and am_val/am_idx hold max_argmax_blocks() partials (a second, one-block
// launch reduces them into *am_out).
hipError_t launch_rows(int type, int epi, const RowsArgs &a, int segments, const DevInfo &dev, float *scratch,
                       hipStream_t stream);
int max_argmax_blocks(const DevInfo &dev);

// Multi-token matmul on the matrix cores: y[m * y_stride + r] = W row r . x_m for
// m < M, row r starting at element base + r * row_stride, x_m = x + m * x_stride.
struct TokArgs {
  const uint8_t *W;
  int64_t base;
  int64_t row_stride;
  int32_t rows;
  int32_t dim1;
  const float *x;
  int64_t x_stride;
  int32_t M;
  float *y;
  int64_t y_stride;
  float *part;  // tok_scratch_floats() floats of column-split partial sums (null when that is 0)
};

// True when (type, offsets, dim1) take the matrix-core kernel (Q4_K, 64-element aligned rows).
bool tok_ok(int type, const TokArgs &a);
// Scratch the launch needs for partial sums (0: one column split, y written directly).
int64_t tok_scratch_floats(const TokArgs &a, const DevInfo &dev);
hipError_t launch_tok(int type, const TokArgs &a, const DevInfo &dev, hipStream_t stream);

// Routed experts of a multi-token MoE call on the matrix cores, grouped by
// expert (Q4_K): pair p = (token p / x_div, slot p % x_div) with expert ids[p]
// reads x + (p / x_div) * x_stride and writes y + p * y_stride.  gate_up: rows
// r < rows of the gate (base0) and up (base1) matrices, y[r] = gelu(gate) * up;
// otherwise rows r < rows from base0, y[r] = row r . x.  Expert e's matrices
// start expert_stride elements after expert e - 1's.  Pairs whose id is outside
// [0, n_experts) get zero rows.
struct MoeGrpArgs {
  const uint8_t *W;
  int64_t base0;
  int64_t base1;
  int64_t row_stride;
  int64_t expert_stride;
  const int32_t *ids;
  int32_t S;  // (token, slot) pairs
  int32_t n_experts;
  int32_t rows;
  int32_t dim1;
  const float *x;
  int64_t x_stride;
  int32_t x_div;
  float *y;
  int64_t y_stride;
  // gate+up launch: S x 2 rows floats for the gate and up rows of every pair
  // before gelu (the 16-pair tiles write them here, then k_gelu_mul forms y)
  float *gu;
};
bool moe_grp_ok(int type, const MoeGrpArgs &a);
// Grants the grouped kernels their largest dynamic LDS size on the current
// device; called once per device before any launch (g4_open).
hipError_t moe_grp_init_device();
hipError_t launch_moe_grp(int type, bool gate_up, const MoeGrpArgs &a, const DevInfo &dev, hipStream_t stream);
// h[s * h_stride + r] = gelu(gu[s][r]) * gu[s][rows + r] for rows x segments
// (gu: segments x 2 rows floats, gate then up)
hipError_t launch_gelu_mul(const float *gu, int32_t rows, int32_t segments, float *h, int64_t h_stride,
                           hipStream_t stream);

// Plain matvec of rows of 65..256 chunks (g4_wide.hip): the columns split over
// the waves of a workgroup.  wide_ok: the launch takes it (EPI_STORE, no ids,
// no fused norm or routing, 64-element aligned rows of the row-stream formats).
bool wide_ok(int type, const RowsArgs &a, int epi);
hipError_t launch_wide(int type, const RowsArgs &a, int segments, hipStream_t stream);

hipError_t launch_dequant(int type, const uint8_t *W, int64_t offset, int64_t n, float *out, hipStream_t stream);
hipError_t launch_argmax(const float *v, int32_t n, float *part_val, int32_t *part_idx, int32_t *out,
                         const DevInfo &dev, hipStream_t stream);
// launch_route takes up to this many experts per token.
constexpr int ROUTE_LAUNCH_MAX_E = 1024;
hipError_t launch_route(const float *logits, int32_t T, int32_t n_experts, int32_t k, int32_t renorm,
                        const float *expert_scale, int32_t *ids, float *weights, hipStream_t stream);
// Down projection and weighted sum of the routed experts in one launch (k =
// 1..8, one column pass of at most 2048 columns, rows on the 64-element fast
// path; one token, or rows of 17..24 chunks for more); hipErrorNotSupported
// otherwise (the caller then uses launch_rows + launch_moe_combine).
hipError_t launch_moe_down(int type, const RowsArgs &a, const float *gw, int32_t T, int32_t K, const DevInfo &dev,
                           hipStream_t s);
// Gate+up (EPI_GELU_PAIR, routing inside when a.route_logits) of T >= 2 tokens
// with one wave per slot (a.x_div = k <= 8) and one workgroup per (row block,
// token), for Q8_0/Q4_0/Q4_K/Q5_K/Q6_K rows of 17..32 chunks on the fast path;
// hipErrorNotSupported otherwise (the caller then uses launch_rows).
hipError_t launch_moe_gate_up(int type, const RowsArgs &a, int32_t T, const DevInfo &dev, hipStream_t s);
// dst = src for `bytes` (a multiple of 4; both ends 16-byte aligned), by a kernel.
hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s);
// dst[0 .. bytes) = 0 by a kernel (any alignment and size).
hipError_t launch_zero(void *dst, size_t bytes, hipStream_t s);
hipError_t launch_moe_combine(const float *ys, const float *weights, int32_t T, int32_t k, int32_t dim, float *Y,
                              hipStream_t stream);

// Decode-step element-wise work.  rms norm of n_vec vectors of `size` floats
// (vector v at x + v * size; w shared, null for NORM_NO_WEIGHT); out may alias
// x; when resid != null also resid += out.
hipError_t launch_rmsnorm(const float *x, const float *w, float *out, float *resid, int32_t n_vec, int32_t size,
                          float eps, int form, hipStream_t stream);
hipError_t launch_add(float *x, const float *that, int64_t n, hipStream_t stream);
hipError_t launch_softcap(float *v, int64_t n, float cap, hipStream_t stream);

// Decode attention over a layer's KV cache (Llama.kt:198-218).  Rows row0 ..
// row0 + rows - 1 of the caches; head h reads kv head h / kv_mul.  attention_plan
// fills kv_mul, n_groups, ch and n_chunks; the launch needs
// attention_scratch_floats() floats of scratch (16-byte aligned).
struct AttArgs {
  const float *q;
  const float *kc;
  const float *vc;
  float *out;
  float *part;
  float *ml;
  int32_t n_heads;
  int32_t n_kv;
  int32_t hs;
  int32_t kv_mul;
  int32_t n_groups;
  int32_t row0;
  int32_t rows;
  int32_t ch;
  int32_t n_chunks;
  int32_t generic;  // 1: one workgroup per head (any head size or alignment); set before attention_plan
};
bool attention_fast_ok(int32_t hs);
void attention_plan(AttArgs &a, const DevInfo &dev);
int64_t attention_scratch_floats(const AttArgs &a);
hipError_t launch_attention(AttArgs a, float *scratch, hipStream_t stream);

}  // namespace g4
