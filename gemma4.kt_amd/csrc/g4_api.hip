// g4_api.hip -- the C ABI declared in include/g4hip.h.
//
// Host-side argument validation (the error conventions of the reference's
// tensor layer mapped to status codes), contexts, weight upload and the
// dispatch of each entry point onto the kernels of g4_kernels.hip.  Reference
// paths are relative to lib/src/main/kotlin/io/github/lbenedetto/internal/.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/g4hip.h"
#include "g4_internal.hpp"

// A result of a host-pointer call waiting in pinned memory for the call's end.
struct G4PendingOut {
  void *dst;
  const char *src;
  size_t bytes;
};

struct g4_ctx {
  int device;
  hipStream_t own_stream;
  hipStream_t stream;
  g4::DevInfo dev;
  char *scratch;  // grow-only device buffer for staging and intermediates
  size_t scratch_bytes;
  // Stream capture: a captured graph keeps the scratch addresses it was recorded
  // with, so once any call on this context has been captured, a buffer that is
  // outgrown is retired (kept until g4_close) instead of freed, and no call may
  // grow the scratch while its stream is capturing (hipMalloc is not capturable).
  bool capturing;  // the current call's stream is capturing
  bool captured;   // some call on this context was captured
  char *retired[32];
  int n_retired;
  float *am_val;  // per-block argmax partials and a result slot
  int32_t *am_idx;
  int32_t *am_out;
  // Host-pointer calls: activations and results pass through pinned host memory
  // (grow-only), moved by a copy kernel; results reach the caller's arrays when
  // the call ends (finish).
  char *pin;
  size_t pin_bytes;
  size_t pin_used;
  G4PendingOut outs[8];
  int n_outs;
};

struct g4_weight {
  int device;
  int type;
  int64_t n_elems;
  int64_t nbytes;
  uint8_t *d;
};

// Scratch of g4_moe_routed_dev_noalloc: a fixed device array, one copy per GPU
// that loads the library, held until the process ends.  Host code never uses
// the array's name as an address (on the host it is only a stand-in): each
// device's own address comes from hipGetSymbolAddress in g4_open and is kept in
// g_noalloc_scratch.
constexpr size_t G4_NOALLOC_SCRATCH_BYTES = size_t(16) << 20;
static __device__ __align__(256) unsigned char noalloc_scratch[G4_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int G4_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;  // serialises the one-time per-device set-up in g4_open
std::atomic<char *> g_noalloc_scratch[G4_MAX_DEVICES];  // device address of noalloc_scratch per ordinal
bool g_dev_ready[G4_MAX_DEVICES];  // kernel attributes set (under g_noalloc_mu)

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() { return G4_OK; }

int hip_fail(hipError_t e, const char *what) {
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    return fail(G4_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
  return fail(G4_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define G4_HIP(call, what)                 \
  do {                                     \
    hipError_t _e = (call);                \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

// GGMLType.kt:16-32 for the supported ids.
bool type_info(int t, int *bs, int *ts) {
  switch (t) {
    case G4_TYPE_F32: *bs = 1; *ts = 4; return true;
    case G4_TYPE_F16: *bs = 1; *ts = 2; return true;
    case G4_TYPE_BF16: *bs = 1; *ts = 2; return true;
    case G4_TYPE_Q4_0: *bs = 32; *ts = 18; return true;
    case G4_TYPE_Q8_0: *bs = 32; *ts = 34; return true;
    case G4_TYPE_Q4_K: *bs = 256; *ts = 144; return true;
    case G4_TYPE_Q5_K: *bs = 256; *ts = 176; return true;
    case G4_TYPE_Q6_K: *bs = 256; *ts = 210; return true;
    default: return false;
  }
}

constexpr size_t ALIGN = 256;
size_t up(size_t n) { return (n + ALIGN - 1) & ~(ALIGN - 1); }

int use_device(g4_ctx *ctx) {
  G4_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  G4_HIP(hipStreamIsCapturing(ctx->stream, &st), "hipStreamIsCapturing");
  ctx->capturing = st != hipStreamCaptureStatusNone;
  if (ctx->capturing) ctx->captured = true;
  // a host-pointer call that failed part way leaves staged results behind: they
  // are dropped (the call reported its error) once its queued work is done
  if (ctx->pin_used || ctx->n_outs) {
    if (ctx->capturing)
      return fail(G4_ERR_INVALID_ARGUMENT, "a failed host-pointer call left work queued: synchronise before capturing");
    G4_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    ctx->pin_used = 0;
    ctx->n_outs = 0;
  }
  return G4_OK;
}

// Host-pointer entry points copy through pinned memory and synchronise, which a
// stream capture cannot record.
int use_host(g4_ctx *ctx) {
  const int rc = use_device(ctx);
  if (rc != G4_OK) return rc;
  if (ctx->capturing)
    return fail(G4_ERR_INVALID_ARGUMENT,
                "host-pointer calls synchronise and cannot run under stream capture (use the *_dev entry points)");
  return G4_OK;
}

// Make sure the context's scratch holds `bytes`.  Before any capture: waits for
// queued work, frees the old buffer and allocates the new one.  After a capture:
// the old buffer stays allocated (a graph may still replay into it) until
// g4_close.  During a capture: an error, since the allocation cannot be captured.
int ensure_scratch(g4_ctx *ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return G4_OK;
  if (ctx->capturing)
    return fail(G4_ERR_INVALID_ARGUMENT,
                "the call needs %zu bytes of context scratch, %zu are reserved, and its stream is being captured: "
                "reserve them before the capture (g4_ctx_reserve)", bytes, ctx->scratch_bytes);
  size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
  if (ctx->captured) {
    if (ctx->n_retired == (int)(sizeof(ctx->retired) / sizeof(ctx->retired[0])))
      return fail(G4_ERR_OUT_OF_MEMORY, "context scratch regrown too often after a capture");
    if (want < 2 * ctx->scratch_bytes) want = 2 * ctx->scratch_bytes;  // few retirements
    void *p = nullptr;
    G4_HIP(hipMalloc(&p, want), "hipMalloc(scratch)");
    if (ctx->scratch) ctx->retired[ctx->n_retired++] = ctx->scratch;
    ctx->scratch = (char *)p;
    ctx->scratch_bytes = want;
    return G4_OK;
  }
  G4_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (ctx->scratch) G4_HIP(hipFree(ctx->scratch), "hipFree");
  ctx->scratch = nullptr;
  ctx->scratch_bytes = 0;
  void *p = nullptr;
  G4_HIP(hipMalloc(&p, want), "hipMalloc(scratch)");
  ctx->scratch = (char *)p;
  ctx->scratch_bytes = want;
  return G4_OK;
}

// Zero `bytes` of device memory by a kernel (a memset node in a captured graph
// is avoided: the degenerate shapes below may run under capture).
int zero_dev(g4_ctx *ctx, void *p, size_t bytes) {
  G4_HIP(g4::launch_zero(p, bytes, ctx->stream), "zero fill");
  return G4_OK;
}

// Bump allocator over the scratch: layout computed first, then carved.
struct Carve {
  size_t off = 0;
  size_t add(size_t bytes) {
    size_t o = off;
    off += up(bytes);
    return o;
  }
};

int check_ctx(const g4_ctx *ctx) {
  if (!ctx) return fail(G4_ERR_INVALID_ARGUMENT, "context is null");
  return G4_OK;
}

int check_weight(const g4_ctx *ctx, const g4_weight *w, const char *name) {
  if (!w) return fail(G4_ERR_INVALID_ARGUMENT, "%s is null", name);
  if (w->device != ctx->device)
    return fail(G4_ERR_INVALID_ARGUMENT, "%s lives on device %d, context on device %d", name, w->device,
                ctx->device);
  return G4_OK;
}

// FloatTensor.kt:18-29: rows this_offset + i*dim1 .. + dim1 for i < dim0 must lie in the tensor.
int check_geometry(int64_t n_elems, int64_t this_offset, int32_t dim0, int32_t dim1) {
  if (dim0 < 0 || dim1 < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative dims (%d, %d)", dim0, dim1);
  if (this_offset < 0) return fail(G4_ERR_OUT_OF_RANGE, "negative offset %lld", (long long)this_offset);
  const int64_t need = this_offset + (int64_t)dim0 * dim1;
  if (need > n_elems)
    return fail(G4_ERR_OUT_OF_RANGE, "offset %lld + %d x %d elements exceeds the tensor's %lld",
                (long long)this_offset, dim0, dim1, (long long)n_elems);
  return G4_OK;
}

int check_rows(const g4_weight *w, int64_t this_offset, int32_t dim0, int32_t dim1) {
  return check_geometry(w->n_elems, this_offset, dim0, dim1);
}

g4::RowsArgs plain_rows(const g4_weight *w, int64_t this_offset, const float *x, float *y, int32_t dim0,
                        int32_t dim1) {
  g4::RowsArgs a;
  memset(&a, 0, sizeof(a));
  a.W0 = a.W1 = w->d;
  a.base0 = a.base1 = this_offset;
  a.row_stride = dim1;
  a.expert_stride = 0;
  a.ids = nullptr;
  a.expert_count = 1;
  a.rows = dim0;
  a.dim1 = dim1;
  a.x = x;
  a.x_stride = 0;
  a.x_div = 1;
  a.y = y;
  a.y_stride = 0;
  return a;
}

int launch_status(hipError_t e, const char *what) {
  if (e == hipErrorInvalidValue) return fail(G4_ERR_INVALID_ARGUMENT, "%s: unsupported launch shape", what);
  if (e != hipSuccess) return hip_fail(e, what);
  return G4_OK;
}

// Activations up to this size go through pinned memory and the copy kernel;
// larger ones take the DMA engines.
constexpr size_t PIN_MAX_COPY = size_t(256) << 10;

void flush_outs(g4_ctx *ctx) {
  for (int i = 0; i < ctx->n_outs; ++i) memcpy(ctx->outs[i].dst, ctx->outs[i].src, ctx->outs[i].bytes);
  ctx->n_outs = 0;
}

// A pinned region of `bytes` for the current call.  When the call's regions no
// longer fit, its queued work is waited for, the results staged so far are
// delivered, and the buffer regrows.
int pin_take(g4_ctx *ctx, size_t bytes, char **out) {
  if (ctx->pin_used + up(bytes) > ctx->pin_bytes || ctx->n_outs == 8) {
    G4_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    flush_outs(ctx);
    ctx->pin_used = 0;
    if (up(bytes) > ctx->pin_bytes) {
      if (ctx->pin) G4_HIP(hipHostFree(ctx->pin), "hipHostFree");
      ctx->pin = nullptr;
      ctx->pin_bytes = 0;
      size_t want = up(bytes) < (size_t(1) << 20) ? (size_t(1) << 20) : up(bytes);
      void *p = nullptr;
      G4_HIP(hipHostMalloc(&p, want, hipHostMallocDefault), "hipHostMalloc");
      ctx->pin = (char *)p;
      ctx->pin_bytes = want;
    }
  }
  *out = ctx->pin + ctx->pin_used;
  ctx->pin_used += up(bytes);
  return G4_OK;
}

int copy_in(g4_ctx *ctx, void *dst, const void *src, size_t bytes) {
  if (!bytes) return G4_OK;
  if (bytes > PIN_MAX_COPY || (bytes & 3) || ((uintptr_t)dst & 15)) {
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync(H2D)");
    return G4_OK;
  }
  char *p = nullptr;
  const int rc = pin_take(ctx, bytes, &p);
  if (rc != G4_OK) return rc;
  memcpy(p, src, bytes);
  G4_HIP(g4::launch_copy(dst, p, bytes, ctx->stream), "copy in");
  return G4_OK;
}

int copy_out(g4_ctx *ctx, void *dst, const void *src, size_t bytes) {
  if (!bytes) return G4_OK;
  if (bytes > PIN_MAX_COPY || (bytes & 3) || ((uintptr_t)src & 15)) {
    G4_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(D2H)");
    return G4_OK;
  }
  char *p = nullptr;
  const int rc = pin_take(ctx, bytes, &p);
  if (rc != G4_OK) return rc;
  G4_HIP(g4::launch_copy(p, src, bytes, ctx->stream), "copy out");
  ctx->outs[ctx->n_outs++] = G4PendingOut{dst, p, bytes};
  return G4_OK;
}

// Where a host-pointer call's kernels write a result meant for `dst`: a small
// result straight into pinned host memory (the kernels store across the bus, no
// copy launch) that reaches `dst` when the call ends; a larger one into
// `fallback` in device memory, for copy_out.  *direct tells which.  A call
// stages its inputs first and its direct outputs last, right before the kernels
// that write them: a later pin_take could otherwise wait, deliver the region
// before it is written and reuse it.
int stage_out(g4_ctx *ctx, void *dst, size_t bytes, void *fallback, void **dev, bool *direct) {
  *dev = fallback;
  *direct = false;
  if (!bytes || bytes > PIN_MAX_COPY || (bytes & 3)) return G4_OK;
  char *p = nullptr;
  const int rc = pin_take(ctx, bytes, &p);
  if (rc != G4_OK) return rc;
  ctx->outs[ctx->n_outs++] = G4PendingOut{dst, p, bytes};
  *dev = p;
  *direct = true;
  return G4_OK;
}

// End of a host-pointer call: wait, then hand the staged results to the caller.
int finish(g4_ctx *ctx) {
  G4_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  flush_outs(ctx);
  ctx->pin_used = 0;
  return G4_OK;
}

#define G4_TRY(expr)        \
  do {                      \
    int _rc = (expr);       \
    if (_rc != G4_OK) return _rc; \
  } while (0)

// --- shared bodies of host and device entry points ---

int matmul_dev(g4_ctx *ctx, const g4_weight *w, int64_t off, const float *d_x, float *d_y, int32_t dim0,
               int32_t dim1) {
  if (dim0 == 0) return G4_OK;
  if (dim1 == 0) {
    G4_TRY(zero_dev(ctx, d_y, sizeof(float) * (size_t)dim0));
    return G4_OK;
  }
  g4::RowsArgs a = plain_rows(w, off, d_x, d_y, dim0, dim1);
  return launch_status(g4::launch_rows(w->type, g4::EPI_STORE, a, 1, ctx->dev, nullptr, ctx->stream), "matmul");
}

g4::TokArgs tok_args(const g4_weight *w, int64_t off, const float *d_X, int32_t M, float *d_Y, int32_t dim0,
                     int32_t dim1) {
  g4::TokArgs t;
  t.W = w->d;
  t.base = off;
  t.row_stride = dim1;
  t.rows = dim0;
  t.dim1 = dim1;
  t.x = d_X;
  t.x_stride = dim1;
  t.M = M;
  t.y = d_Y;
  t.y_stride = dim0;
  t.part = nullptr;
  return t;
}

// Scratch floats batch_dev needs for partial sums (carved by the caller).
int64_t batch_part_floats(const g4_ctx *ctx, const g4_weight *w, int64_t off, int32_t M, int32_t dim0,
                          int32_t dim1) {
  if (M < 3 || dim0 == 0 || dim1 == 0) return 0;
  const g4::TokArgs t = tok_args(w, off, nullptr, M, nullptr, dim0, dim1);
  return g4::tok_ok(w->type, t) ? g4::tok_scratch_floats(t, ctx->dev) : 0;
}

int batch_dev(g4_ctx *ctx, const g4_weight *w, int64_t off, const float *d_X, int32_t M, float *d_Y, int32_t dim0,
              int32_t dim1, float *d_part) {
  if (dim0 == 0 || M == 0) return G4_OK;
  if (dim1 == 0) {
    G4_TRY(zero_dev(ctx, d_Y, sizeof(float) * (size_t)dim0 * M));
    return G4_OK;
  }
  // several tokens: the matrix-core kernel unpacks each weight once for all of
  // them.  Two tokens stay on the row engine (one segment each): measured on
  // 8192 x 2048, 6.5 us against 8.9 us for the matrix cores; from three on the
  // matrix cores are as fast or faster (9.1 / 9.3 us at M = 3, 9.6 / 14.4 at M = 8).
  if (M >= 3) {
    g4::TokArgs t = tok_args(w, off, d_X, M, d_Y, dim0, dim1);
    if (g4::tok_ok(w->type, t)) {
      t.part = d_part;
      return launch_status(g4::launch_tok(w->type, t, ctx->dev, ctx->stream), "matmul_batch");
    }
  }
  g4::RowsArgs a = plain_rows(w, off, d_X, d_Y, dim0, dim1);
  a.x_stride = dim1;
  a.y_stride = dim0;
  return launch_status(g4::launch_rows(w->type, g4::EPI_STORE, a, M, ctx->dev, nullptr, ctx->stream),
                       "matmul_batch");
}

int argmax_rows_dev(g4_ctx *ctx, const g4_weight *w, int64_t off, const float *d_x, float *d_logits,
                    int32_t *d_index, int32_t dim0, int32_t dim1) {
  g4::RowsArgs a = plain_rows(w, off, d_x, d_logits, dim0, dim1);
  a.am_val = ctx->am_val;
  a.am_idx = ctx->am_idx;
  a.am_out = d_index;
  return launch_status(g4::launch_rows(w->type, g4::EPI_ARGMAX, a, 1, ctx->dev, nullptr, ctx->stream),
                       "matmul_argmax");
}

// h = gelu(W_gate x) * (W_up x): one paired launch (d_gu: 2*hidden floats, used by the generic path only).
int gate_up_dev(g4_ctx *ctx, const g4_weight *wg, const g4_weight *wu, const float *d_x, float *d_h, float *d_gu,
                int32_t dim, int32_t hidden) {
  g4::RowsArgs a = plain_rows(wg, 0, d_x, d_h, hidden, dim);
  a.W1 = wu->d;
  return launch_status(g4::launch_rows(wg->type, g4::EPI_GELU_PAIR, a, 1, ctx->dev, d_gu, ctx->stream), "ffn");
}

int ffn_dev(g4_ctx *ctx, const g4_weight *wg, const g4_weight *wu, const g4_weight *wd, const float *d_x,
            float *d_y, float *d_h, float *d_gu, int32_t dim, int32_t hidden) {
  G4_TRY(gate_up_dev(ctx, wg, wu, d_x, d_h, d_gu, dim, hidden));
  g4::RowsArgs b = plain_rows(wd, 0, d_h, d_y, dim, hidden);
  return launch_status(g4::launch_rows(wd->type, g4::EPI_STORE, b, 1, ctx->dev, nullptr, ctx->stream), "ffn");
}

// w_down may be null (gate/up half only).
int check_ffn(g4_ctx *ctx, const g4_weight *wg, const g4_weight *wu, const g4_weight *wd, int32_t dim,
              int32_t hidden) {
  G4_TRY(check_weight(ctx, wg, "w_gate"));
  G4_TRY(check_weight(ctx, wu, "w_up"));
  if (wd) G4_TRY(check_weight(ctx, wd, "w_down"));
  if (dim <= 0 || hidden <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "ffn dims must be positive (%d, %d)", dim, hidden);
  G4_TRY(check_rows(wg, 0, hidden, dim));
  G4_TRY(check_rows(wu, 0, hidden, dim));
  if (wd) G4_TRY(check_rows(wd, 0, dim, hidden));
  if (wg->type != wu->type) return fail(G4_ERR_UNSUPPORTED, "ffn: gate and up weights must share one GGML type");
  return G4_OK;
}

int check_moe(g4_ctx *ctx, const g4_weight *wgu, const g4_weight *wdn, int32_t T, int32_t dim, int32_t ff,
              int32_t k, int32_t *n_experts) {
  G4_TRY(check_weight(ctx, wgu, "w_gate_up"));
  G4_TRY(check_weight(ctx, wdn, "w_down"));
  if (T < 0 || k < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative T or k (%d, %d)", T, k);
  // one launch row of workgroups per (token, slot) pair
  if ((int64_t)T * k > 65535)
    return fail(G4_ERR_INVALID_ARGUMENT, "T*k = %lld (token, slot) pairs exceed 65535 per call", (long long)T * k);
  if (dim <= 0 || ff <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "moe dims must be positive (%d, %d)", dim, ff);
  const int64_t per_gu = 2 * (int64_t)ff * dim, per_dn = (int64_t)dim * ff;
  if (wgu->n_elems % per_gu != 0)
    return fail(G4_ERR_INVALID_ARGUMENT, "w_gate_up holds %lld elements, not a multiple of 2*ff*dim = %lld",
                (long long)wgu->n_elems, (long long)per_gu);
  const int64_t ne = wgu->n_elems / per_gu;
  if (wdn->n_elems < ne * per_dn)
    return fail(G4_ERR_OUT_OF_RANGE, "w_down holds %lld elements, %lld experts need %lld", (long long)wdn->n_elems,
                (long long)ne, (long long)(ne * per_dn));
  if (ne > 0x7fffffff) return fail(G4_ERR_INVALID_ARGUMENT, "too many experts");
  *n_experts = (int32_t)ne;
  return G4_OK;
}

// Routing done inside the gate+up launch (g4_moe_routed*): the router logits in,
// the ids and weights it stores out.
// Calls of at least this many tokens run the experts grouped (launch_moe_grp):
// measured on the 128-expert top-8 shape (alternating runs, one box), the grouped
// launches take 231, 233, 235, 239 and 288 us at 33, 40, 48, 64 and 128 tokens
// against 201, 233, 275, 332 and 723 us for the per-pair ones, and about 222-230
// us from 16 to 32 tokens, where the per-pair ones take 101-180 us.
constexpr int32_t MOE_GROUPED_MIN_T = 41;

struct MoeRoute {
  const float *d_logits;
  int32_t n_experts;
  int32_t renormalize;
  const float *d_scale;
};

int moe_dev(g4_ctx *ctx, const g4_weight *wgu, const g4_weight *wdn, int32_t n_experts, const float *d_X, int32_t T,
            int32_t dim, int32_t ff, const int32_t *d_ids, const float *d_w, int32_t k, float *d_Y, float *d_h,
            float *d_ys, float *d_gu, const MoeRoute *route = nullptr) {
  const int32_t S = T * k;  // (token, slot) pairs
  if (S == 0) {
    if (T > 0) G4_TRY(zero_dev(ctx, d_Y, sizeof(float) * (size_t)T * dim));
    return G4_OK;
  }
  if (T >= MOE_GROUPED_MIN_T) {
    // many tokens: the experts grouped on the matrix cores (each expert's
    // weights read once for all of its pairs), after a routing launch when the
    // call routes
    g4::MoeGrpArgs gu;
    memset(&gu, 0, sizeof(gu));
    gu.W = wgu->d;
    gu.base0 = 0;
    gu.base1 = (int64_t)ff * dim;
    gu.row_stride = dim;
    gu.expert_stride = 2 * (int64_t)ff * dim;
    gu.ids = d_ids;
    gu.S = S;
    gu.n_experts = n_experts;
    gu.rows = ff;
    gu.dim1 = dim;
    gu.x = d_X;
    gu.x_stride = dim;
    gu.x_div = k;
    gu.y = d_h;
    gu.y_stride = ff;
    gu.gu = d_gu;
    g4::MoeGrpArgs dn = gu;
    dn.gu = nullptr;
    dn.W = wdn->d;
    dn.base1 = 0;
    dn.row_stride = ff;
    dn.expert_stride = (int64_t)dim * ff;
    dn.rows = dim;
    dn.dim1 = ff;
    dn.x = d_h;
    dn.x_stride = ff;
    dn.x_div = 1;
    dn.y = d_ys;
    dn.y_stride = dim;
    if (g4::moe_grp_ok(wgu->type, gu) && g4::moe_grp_ok(wdn->type, dn) && n_experts < 65535 &&
        (!route || route->n_experts <= g4::ROUTE_LAUNCH_MAX_E)) {
      if (route)
        G4_TRY(launch_status(g4::launch_route(route->d_logits, T, route->n_experts, k, route->renormalize,
                                              route->d_scale, const_cast<int32_t *>(d_ids), const_cast<float *>(d_w),
                                              ctx->stream),
                             "moe"));
      G4_TRY(launch_status(g4::launch_moe_grp(wgu->type, true, gu, ctx->dev, ctx->stream), "moe"));
      G4_TRY(launch_status(g4::launch_moe_grp(wdn->type, false, dn, ctx->dev, ctx->stream), "moe"));
      return launch_status(g4::launch_moe_combine(d_ys, d_w, T, k, dim, d_Y, ctx->stream), "moe");
    }
  }
  g4::RowsArgs a;
  memset(&a, 0, sizeof(a));
  if (route) {
    // d_ids / d_w are the outputs of the routing then
    a.route_logits = route->d_logits;
    a.route_scale = route->d_scale;
    a.route_e = route->n_experts;
    a.route_renorm = route->renormalize;
    a.route_ids = const_cast<int32_t *>(d_ids);
    a.route_w = const_cast<float *>(d_w);
  }
  a.W0 = a.W1 = wgu->d;
  a.base0 = 0;
  a.base1 = (int64_t)ff * dim;
  a.row_stride = dim;
  a.expert_stride = 2 * (int64_t)ff * dim;
  a.ids = route ? nullptr : d_ids;
  a.expert_count = n_experts;
  a.rows = ff;
  a.dim1 = dim;
  a.x = d_X;
  a.x_stride = dim;
  a.x_div = k;
  a.y = d_h;
  a.y_stride = ff;
  // several tokens: one wave per slot, so a token's x and routing serve its k slots
  hipError_t egu = g4::launch_moe_gate_up(wgu->type, a, T, ctx->dev, ctx->stream);
  if (egu == hipErrorNotSupported) egu = g4::launch_rows(wgu->type, g4::EPI_GELU_PAIR, a, S, ctx->dev, d_gu, ctx->stream);
  G4_TRY(launch_status(egu, "moe"));
  g4::RowsArgs b;
  memset(&b, 0, sizeof(b));
  b.W0 = b.W1 = wdn->d;
  b.row_stride = ff;
  b.expert_stride = (int64_t)dim * ff;
  b.ids = d_ids;
  b.expert_count = n_experts;
  b.rows = dim;
  b.dim1 = ff;
  b.x = d_h;
  b.x_stride = ff;
  b.x_div = 1;
  // down and the weighted sum in one launch where the shape allows
  g4::RowsArgs c = b;
  c.y = d_Y;
  c.y_stride = dim;
  const hipError_t e = g4::launch_moe_down(wdn->type, c, d_w, T, k, ctx->dev, ctx->stream);
  if (e != hipErrorNotSupported) return launch_status(e, "moe");
  b.y = d_ys;
  b.y_stride = dim;
  G4_TRY(launch_status(g4::launch_rows(wdn->type, g4::EPI_STORE, b, S, ctx->dev, nullptr, ctx->stream), "moe"));
  return launch_status(g4::launch_moe_combine(d_ys, d_w, T, k, dim, d_Y, ctx->stream), "moe");
}

size_t moe_scratch(int32_t T, int32_t dim, int32_t ff, int32_t k, Carve &c, size_t *h, size_t *ys, size_t *gu) {
  const size_t S = (size_t)T * k;
  *h = c.add(sizeof(float) * S * ff);
  *ys = c.add(sizeof(float) * S * dim);
  *gu = c.add(sizeof(float) * S * 2 * ff);
  return c.off;
}

// --- decode step ---

// Norm weights are F32 tensors of at least `size` elements (ModelLoader.kt:281-286
// reads them as FloatBuffers and rejects any other type).
int check_norm(const g4_ctx *ctx, const g4_weight *w, int32_t size, const char *name) {
  G4_TRY(check_weight(ctx, w, name));
  if (w->type != G4_TYPE_F32) return fail(G4_ERR_UNSUPPORTED, "%s: Conversion to type %d (norm weights are F32)", name, w->type);
  if (w->n_elems < size)
    return fail(G4_ERR_OUT_OF_RANGE, "%s holds %lld elements, the norm needs %d", name, (long long)w->n_elems, size);
  return G4_OK;
}

int check_eps_cap(float eps, float cap) {
  if (!(eps >= 0.f) || eps == __builtin_inff()) return fail(G4_ERR_INVALID_ARGUMENT, "rms norm eps must be finite and >= 0");
  if (cap != cap) return fail(G4_ERR_INVALID_ARGUMENT, "softcap is NaN");
  return G4_OK;
}

bool ranges_overlap(const void *a, size_t an, const void *b, size_t bn) {
  const char *pa = (const char *)a, *pb = (const char *)b;
  return pa < pb + bn && pb < pa + an;
}

// out = W . rmsnorm(x): the norm fused into the matvec's x staging when the
// launch takes it, else a standalone norm into `xn` (dim1 floats) first.  Both
// give identical bits (the same scale computation, the same element formula).
int matmul_norm_dev(g4_ctx *ctx, const g4_weight *w, int64_t off, const g4_weight *norm, const float *d_x, float eps,
                    float *d_xnorm, float *d_out, int32_t dim0, int32_t dim1, int epi, const g4_weight *w_pair,
                    float *xn, float *d_gu, int32_t *d_index, float softcap) {
  g4::RowsArgs a = plain_rows(w, off, d_x, d_out, dim0, dim1);
  if (w_pair) a.W1 = w_pair->d;
  a.am_val = ctx->am_val;
  a.am_idx = ctx->am_idx;
  a.am_out = d_index;
  a.softcap = softcap;
  a.norm_w = (const float *)norm->d;
  a.norm_eps = eps;
  a.norm_out = d_xnorm;
  if (!g4::rows_norm_ok(w->type, a, epi == g4::EPI_GELU_PAIR)) {
    float *dst = d_xnorm ? d_xnorm : xn;
    G4_TRY(launch_status(g4::launch_rmsnorm(d_x, (const float *)norm->d, dst, nullptr, 1, dim1, eps,
                                            G4_NORM_WEIGHT_AFTER, ctx->stream), "rmsnorm"));
    a.x = dst;
    a.norm_w = nullptr;
    a.norm_out = nullptr;
  }
  return launch_status(g4::launch_rows(w->type, epi, a, 1, ctx->dev, d_gu, ctx->stream), "matmul_norm");
}

// Scratch floats matmul_norm_dev may need for the standalone norm.
int64_t norm_scratch_floats(const g4_weight *w, int64_t off, int32_t dim0, int32_t dim1, bool paired) {
  g4::RowsArgs a = plain_rows(w, off, nullptr, nullptr, dim0, dim1);
  a.norm_w = (const float *)1;
  return g4::rows_norm_ok(w->type, a, paired) ? 0 : dim1;
}

// Llama.kt:355-363 (dense FFN block), in place on d_x.
int ffn_block_dev(g4_ctx *ctx, const g4_weight *wg, const g4_weight *wu, const g4_weight *wd, const g4_weight *n_pre,
                  const g4_weight *n_post, float *d_x, int32_t dim, int32_t hidden, float eps, float *d_h, float *d_y,
                  float *d_gu, float *xn) {
  // xb = rmsnorm(x, rmsFfnWeight); h = gelu(w1 xb) * (w3 xb)
  G4_TRY(matmul_norm_dev(ctx, wg, 0, n_pre, d_x, eps, nullptr, d_h, hidden, dim, g4::EPI_GELU_PAIR, wu, xn, d_gu,
                         nullptr, 0.f));
  // xb = w2 h
  g4::RowsArgs b = plain_rows(wd, 0, d_h, d_y, dim, hidden);
  G4_TRY(launch_status(g4::launch_rows(wd->type, g4::EPI_STORE, b, 1, ctx->dev, nullptr, ctx->stream), "ffn_block"));
  // xb = rmsnorm(xb, postFfwNorm); x += xb
  return launch_status(g4::launch_rmsnorm(d_y, (const float *)n_post->d, d_y, d_x, 1, dim, eps, G4_NORM_WEIGHT_AFTER,
                                          ctx->stream), "ffn_block");
}

void ffn_block_scratch(const g4_weight *wg, int32_t dim, int32_t hidden, Carve &c, size_t *h, size_t *y, size_t *gu,
                       size_t *xn) {
  *h = c.add(sizeof(float) * (size_t)hidden);
  *y = c.add(sizeof(float) * (size_t)dim);
  *gu = c.add(sizeof(float) * 2 * (size_t)hidden);
  *xn = c.add(sizeof(float) * (size_t)norm_scratch_floats(wg, 0, hidden, dim, true));
}

int check_ffn_block(g4_ctx *ctx, const g4_weight *wg, const g4_weight *wu, const g4_weight *wd, const g4_weight *n_pre,
                    const g4_weight *n_post, int32_t dim, int32_t hidden, float eps) {
  G4_TRY(check_ffn(ctx, wg, wu, wd, dim, hidden));
  G4_TRY(check_norm(ctx, n_pre, dim, "norm_pre"));
  G4_TRY(check_norm(ctx, n_post, dim, "norm_post"));
  return check_eps_cap(eps, 0.f);
}

int check_lm_head(g4_ctx *ctx, const g4_weight *w, const g4_weight *norm, int32_t vocab, int32_t dim, float eps,
                  float cap) {
  G4_TRY(check_weight(ctx, w, "w_cls"));
  if (vocab <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "argmax needs vocab > 0 (FloatTensor.kt:54)");
  if (dim <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "dim must be positive (%d)", dim);
  G4_TRY(check_rows(w, 0, vocab, dim));
  G4_TRY(check_norm(ctx, norm, dim, "norm_final"));
  return check_eps_cap(eps, cap);
}

}  // namespace

// =============================================================== C ABI ====

extern "C" {

const char *g4_last_error(void) { return g_last_error.c_str(); }

int g4_version(void) { return (0 << 16) | 1; }

int g4_device_count(int *count) {
  if (!count) return fail(G4_ERR_INVALID_ARGUMENT, "count is null");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice || e == hipErrorInsufficientDriver || e == hipErrorInitializationError) n = 0;
  else if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  *count = n;
  (void)hipGetLastError();
  return G4_OK;
}

int g4_type_info(int ggml_type, int *block_size, int *type_size) {
  int bs, ts;
  if (!type_info(ggml_type, &bs, &ts)) return fail(G4_ERR_UNSUPPORTED, "Quantization format %d", ggml_type);
  if (block_size) *block_size = bs;
  if (type_size) *type_size = ts;
  return G4_OK;
}

int g4_byte_size(int ggml_type, int64_t n_elems, int64_t *nbytes) {
  int bs, ts;
  if (!type_info(ggml_type, &bs, &ts)) return fail(G4_ERR_UNSUPPORTED, "Quantization format %d", ggml_type);
  if (!nbytes) return fail(G4_ERR_INVALID_ARGUMENT, "nbytes is null");
  if (n_elems < 0 || n_elems % bs != 0)
    return fail(G4_ERR_INVALID_ARGUMENT, "%lld elements is not a whole number of %d-element blocks",
                (long long)n_elems, bs);
  *nbytes = n_elems / bs * ts;
  return G4_OK;
}

int g4_check_matmul(int ggml_type, int64_t n_elems, int64_t this_offset, int32_t dim0, int32_t dim1) {
  int bs, ts;
  if (!type_info(ggml_type, &bs, &ts)) return fail(G4_ERR_UNSUPPORTED, "Quantization format %d", ggml_type);
  if (n_elems < 0 || n_elems % bs != 0)
    return fail(G4_ERR_INVALID_ARGUMENT, "%lld elements is not a whole number of %d-element blocks",
                (long long)n_elems, bs);
  return check_geometry(n_elems, this_offset, dim0, dim1);
}

int g4_open(int ordinal, g4_ctx **out) {
  if (!out) return fail(G4_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  int n = 0;
  G4_TRY(g4_device_count(&n));
  if (n == 0) return fail(G4_ERR_NO_DEVICE, "no HIP device is present");
  if (ordinal < 0 || ordinal >= n) return fail(G4_ERR_NO_DEVICE, "device %d does not exist (%d present)", ordinal, n);
  G4_HIP(hipSetDevice(ordinal), "hipSetDevice");
  g4_ctx *c = new g4_ctx();
  memset(c, 0, sizeof(*c));
  c->device = ordinal;
  int cu = 0;
  hipError_t e = hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, ordinal);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipDeviceGetAttribute");
  }
  c->dev.cu_count = cu > 0 ? cu : 1;
  e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipStreamCreate");
  }
  c->stream = c->own_stream;
  {
    // once per device, with the device current: kernel attributes (never set
    // during a stream capture, since no call sets them)
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (ordinal >= G4_MAX_DEVICES || !g_dev_ready[ordinal]) {
      e = g4::moe_grp_init_device();
      if (e != hipSuccess) {
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return hip_fail(e, "hipFuncSetAttribute");
      }
      if (ordinal < G4_MAX_DEVICES) g_dev_ready[ordinal] = true;
    }
  }
  if (ordinal < G4_MAX_DEVICES) {
    // once per device, with the device current: the address of its copy of the
    // allocation-free entry point's scratch
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_scratch[ordinal].load(std::memory_order_acquire)) {
      void *sp = nullptr;
      e = hipGetSymbolAddress(&sp, HIP_SYMBOL(noalloc_scratch));
      if (e != hipSuccess) {
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return hip_fail(e, "hipGetSymbolAddress(noalloc_scratch)");
      }
      g_noalloc_scratch[ordinal].store((char *)sp, std::memory_order_release);
    }
  }
  const int nb = g4::max_argmax_blocks(c->dev);
  void *p = nullptr;
  size_t bytes = up(sizeof(float) * nb) + up(sizeof(int32_t) * nb) + up(sizeof(int32_t));
  e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(c->own_stream);
    delete c;
    return hip_fail(e, "hipMalloc(argmax)");
  }
  char *b = (char *)p;
  c->am_val = (float *)b;
  c->am_idx = (int32_t *)(b + up(sizeof(float) * nb));
  c->am_out = (int32_t *)(b + up(sizeof(float) * nb) + up(sizeof(int32_t) * nb));
  e = hipMemset(p, 0, bytes);
  if (e != hipSuccess) {
    (void)hipFree(p);
    (void)hipStreamDestroy(c->own_stream);
    delete c;
    return hip_fail(e, "hipMemset");
  }
  *out = c;
  return G4_OK;
}

int g4_close(g4_ctx *ctx) {
  G4_TRY(check_ctx(ctx));
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipStreamSynchronize(ctx->own_stream);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  for (int i = 0; i < ctx->n_retired; ++i) (void)hipFree(ctx->retired[i]);
  if (ctx->am_val) (void)hipFree(ctx->am_val);
  if (ctx->pin) (void)hipHostFree(ctx->pin);
  (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
  return G4_OK;
}

int g4_ctx_set_stream(g4_ctx *ctx, void *stream) {
  G4_TRY(check_ctx(ctx));
  ctx->stream = stream ? (hipStream_t)stream : ctx->own_stream;
  return G4_OK;
}

int g4_ctx_sync(g4_ctx *ctx) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(use_host(ctx));
  return finish(ctx);
}

int g4_ctx_reserve(g4_ctx *ctx, int64_t bytes) {
  G4_TRY(check_ctx(ctx));
  if (bytes < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative reservation %lld", (long long)bytes);
  G4_TRY(use_device(ctx));
  return ensure_scratch(ctx, (size_t)bytes);
}

int g4_ctx_scratch_bytes(const g4_ctx *ctx, int64_t *bytes) {
  G4_TRY(check_ctx(ctx));
  if (!bytes) return fail(G4_ERR_INVALID_ARGUMENT, "bytes is null");
  *bytes = (int64_t)ctx->scratch_bytes;
  return G4_OK;
}

int g4_ctx_device(const g4_ctx *ctx, int *ordinal) {
  G4_TRY(check_ctx(ctx));
  if (!ordinal) return fail(G4_ERR_INVALID_ARGUMENT, "ordinal is null");
  *ordinal = ctx->device;
  return G4_OK;
}

int g4_upload(g4_ctx *ctx, int ggml_type, const void *raw, int64_t nbytes, int64_t n_elems, g4_weight **out) {
  G4_TRY(check_ctx(ctx));
  if (!out) return fail(G4_ERR_INVALID_ARGUMENT, "out is null");
  *out = nullptr;
  int bs, ts;
  if (!type_info(ggml_type, &bs, &ts)) return fail(G4_ERR_UNSUPPORTED, "Quantization format %d", ggml_type);
  if (n_elems < 0 || n_elems % bs != 0)
    return fail(G4_ERR_INVALID_ARGUMENT, "%lld elements is not a whole number of %d-element blocks",
                (long long)n_elems, bs);
  const int64_t want = n_elems / bs * ts;
  if (nbytes != want)
    return fail(G4_ERR_INVALID_ARGUMENT, "nbytes %lld != byteSizeFor(%lld) = %lld", (long long)nbytes,
                (long long)n_elems, (long long)want);
  if (!raw && nbytes > 0) return fail(G4_ERR_INVALID_ARGUMENT, "raw is null");
  G4_TRY(use_host(ctx));
  void *d = nullptr;
  const size_t alloc = (size_t)nbytes + ALIGN;  // zeroed tail: no load ever reads past a block, kept as margin
  G4_HIP(hipMalloc(&d, alloc), "hipMalloc(weight)");
  hipError_t e = hipMemsetAsync((char *)d + nbytes, 0, ALIGN, ctx->stream);
  if (e == hipSuccess && nbytes > 0) e = hipMemcpyAsync(d, raw, (size_t)nbytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return hip_fail(e, "upload");
  }
  g4_weight *w = new g4_weight();
  w->device = ctx->device;
  w->type = ggml_type;
  w->n_elems = n_elems;
  w->nbytes = nbytes;
  w->d = (uint8_t *)d;
  *out = w;
  return G4_OK;
}

int g4_weight_free(g4_weight *w) {
  if (!w) return fail(G4_ERR_INVALID_ARGUMENT, "weight is null");
  int cur = 0;
  (void)hipGetDevice(&cur);
  (void)hipSetDevice(w->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(w->d);
  (void)hipSetDevice(cur);
  delete w;
  return G4_OK;
}

int g4_weight_info(const g4_weight *w, int *ggml_type, int64_t *n_elems, int64_t *nbytes) {
  if (!w) return fail(G4_ERR_INVALID_ARGUMENT, "weight is null");
  if (ggml_type) *ggml_type = w->type;
  if (n_elems) *n_elems = w->n_elems;
  if (nbytes) *nbytes = w->nbytes;
  return G4_OK;
}

int g4_weight_device_ptr(const g4_weight *w, const void **dptr) {
  if (!w || !dptr) return fail(G4_ERR_INVALID_ARGUMENT, "null argument");
  *dptr = w->d;
  return G4_OK;
}

// ---------------------------------------------------------------- matmul ----

int g4_matmul(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *that, float *out, int32_t dim0,
              int32_t dim1) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  G4_TRY(check_rows(w, this_offset, dim0, dim1));
  if ((!that && dim1 > 0) || (!out && dim0 > 0)) return fail(G4_ERR_INVALID_ARGUMENT, "that/out is null");
  if (dim0 == 0) return ok();
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)dim1), oy = c.add(sizeof(float) * (size_t)dim0);
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dx = (float *)(ctx->scratch + ox);
  void *dy = nullptr;
  bool direct = false;
  G4_TRY(copy_in(ctx, dx, that, sizeof(float) * (size_t)dim1));
  G4_TRY(stage_out(ctx, out, sizeof(float) * (size_t)dim0, ctx->scratch + oy, &dy, &direct));
  G4_TRY(matmul_dev(ctx, w, this_offset, dx, (float *)dy, dim0, dim1));
  if (!direct) G4_TRY(copy_out(ctx, out, dy, sizeof(float) * (size_t)dim0));
  return finish(ctx);
}

int g4_matmul_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *d_that, float *d_out,
                  int32_t dim0, int32_t dim1) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  G4_TRY(check_rows(w, this_offset, dim0, dim1));
  if ((!d_that && dim1 > 0) || (!d_out && dim0 > 0)) return fail(G4_ERR_INVALID_ARGUMENT, "that/out is null");
  G4_TRY(use_device(ctx));
  return matmul_dev(ctx, w, this_offset, d_that, d_out, dim0, dim1);
}

int g4_matmul_batch(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *X, int32_t M, float *Y,
                    int32_t dim0, int32_t dim1) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  G4_TRY(check_rows(w, this_offset, dim0, dim1));
  if (M < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative M %d", M);
  if (M > 65535) return fail(G4_ERR_INVALID_ARGUMENT, "M %d exceeds 65535", M);
  if ((!X && M > 0 && dim1 > 0) || (!Y && M > 0 && dim0 > 0)) return fail(G4_ERR_INVALID_ARGUMENT, "X/Y is null");
  if (M == 0 || dim0 == 0) return ok();
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)dim1 * M), oy = c.add(sizeof(float) * (size_t)dim0 * M);
  size_t op = c.add(sizeof(float) * (size_t)batch_part_floats(ctx, w, this_offset, M, dim0, dim1));
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dx = (float *)(ctx->scratch + ox), *dy = (float *)(ctx->scratch + oy), *dp = (float *)(ctx->scratch + op);
  G4_TRY(copy_in(ctx, dx, X, sizeof(float) * (size_t)dim1 * M));
  G4_TRY(batch_dev(ctx, w, this_offset, dx, M, dy, dim0, dim1, dp));
  G4_TRY(copy_out(ctx, Y, dy, sizeof(float) * (size_t)dim0 * M));
  return finish(ctx);
}

int g4_matmul_batch_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *d_X, int32_t M,
                        float *d_Y, int32_t dim0, int32_t dim1) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  G4_TRY(check_rows(w, this_offset, dim0, dim1));
  if (M < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative M %d", M);
  if (M > 65535) return fail(G4_ERR_INVALID_ARGUMENT, "M %d exceeds 65535", M);
  if ((!d_X && M > 0 && dim1 > 0) || (!d_Y && M > 0 && dim0 > 0))
    return fail(G4_ERR_INVALID_ARGUMENT, "X/Y is null");
  G4_TRY(use_device(ctx));
  const int64_t pf = batch_part_floats(ctx, w, this_offset, M, dim0, dim1);
  if (pf > 0) G4_TRY(ensure_scratch(ctx, sizeof(float) * (size_t)pf));
  return batch_dev(ctx, w, this_offset, d_X, M, d_Y, dim0, dim1, pf > 0 ? (float *)ctx->scratch : nullptr);
}

// -------------------------------------------------------------- argmax ----

int g4_matmul_argmax(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *that, float *logits,
                     int32_t *index, int32_t dim0, int32_t dim1) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  G4_TRY(check_rows(w, this_offset, dim0, dim1));
  if (dim0 <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "argmax needs dim0 > 0 (FloatTensor.kt:54)");
  if ((!that && dim1 > 0) || !index) return fail(G4_ERR_INVALID_ARGUMENT, "that/index is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)dim1), oy = c.add(sizeof(float) * (size_t)dim0),
         oi = c.add(sizeof(int32_t));
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dx = (float *)(ctx->scratch + ox), *dy = (float *)(ctx->scratch + oy);
  int32_t *di = (int32_t *)(ctx->scratch + oi);
  G4_TRY(copy_in(ctx, dx, that, sizeof(float) * (size_t)dim1));
  if (dim1 == 0) {
    G4_TRY(zero_dev(ctx, dy, sizeof(float) * (size_t)dim0));
    G4_TRY(launch_status(g4::launch_argmax(dy, dim0, ctx->am_val, ctx->am_idx, di, ctx->dev,
                                           ctx->stream), "argmax"));
  } else {
    G4_TRY(argmax_rows_dev(ctx, w, this_offset, dx, dy, di, dim0, dim1));
  }
  if (logits) G4_TRY(copy_out(ctx, logits, dy, sizeof(float) * (size_t)dim0));
  G4_TRY(copy_out(ctx, index, di, sizeof(int32_t)));
  return finish(ctx);
}

int g4_matmul_argmax_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const float *d_that,
                         float *d_logits, int32_t *d_index, int32_t dim0, int32_t dim1) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  G4_TRY(check_rows(w, this_offset, dim0, dim1));
  if (dim0 <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "argmax needs dim0 > 0 (FloatTensor.kt:54)");
  if ((!d_that && dim1 > 0) || !d_index) return fail(G4_ERR_INVALID_ARGUMENT, "that/index is null");
  G4_TRY(use_device(ctx));
  float *dy = d_logits;
  if (!dy) {
    Carve c;
    size_t oy = c.add(sizeof(float) * (size_t)dim0);
    G4_TRY(ensure_scratch(ctx, c.off));
    dy = (float *)(ctx->scratch + oy);
  }
  if (dim1 == 0) {
    G4_TRY(zero_dev(ctx, dy, sizeof(float) * (size_t)dim0));
    return launch_status(g4::launch_argmax(dy, dim0, ctx->am_val, ctx->am_idx, d_index, ctx->dev,
                                           ctx->stream), "argmax");
  }
  return argmax_rows_dev(ctx, w, this_offset, d_that, dy, d_index, dim0, dim1);
}

int g4_argmax(g4_ctx *ctx, const float *v, int32_t n, int32_t *index) {
  G4_TRY(check_ctx(ctx));
  if (n <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "argmax needs size > 0 (FloatTensor.kt:54)");
  if (!v || !index) return fail(G4_ERR_INVALID_ARGUMENT, "v/index is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ov = c.add(sizeof(float) * (size_t)n), oi = c.add(sizeof(int32_t));
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dv = (float *)(ctx->scratch + ov);
  int32_t *di = (int32_t *)(ctx->scratch + oi);
  G4_TRY(copy_in(ctx, dv, v, sizeof(float) * (size_t)n));
  G4_TRY(launch_status(
      g4::launch_argmax(dv, n, ctx->am_val, ctx->am_idx, di, ctx->dev, ctx->stream), "argmax"));
  G4_TRY(copy_out(ctx, index, di, sizeof(int32_t)));
  return finish(ctx);
}

int g4_argmax_dev(g4_ctx *ctx, const float *d_v, int32_t n, int32_t *d_index) {
  G4_TRY(check_ctx(ctx));
  if (n <= 0) return fail(G4_ERR_INVALID_ARGUMENT, "argmax needs size > 0 (FloatTensor.kt:54)");
  if (!d_v || !d_index) return fail(G4_ERR_INVALID_ARGUMENT, "v/index is null");
  G4_TRY(use_device(ctx));
  return launch_status(
      g4::launch_argmax(d_v, n, ctx->am_val, ctx->am_idx, d_index, ctx->dev, ctx->stream), "argmax");
}

// ------------------------------------------------------------- dequant ----

int g4_dequant(g4_ctx *ctx, const g4_weight *w, int64_t offset, int64_t n, float *out) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  if (n < 0 || offset < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative offset or count");
  if (offset + n > w->n_elems)
    return fail(G4_ERR_OUT_OF_RANGE, "elements %lld..%lld exceed the tensor's %lld", (long long)offset,
                (long long)(offset + n), (long long)w->n_elems);
  if (!out && n > 0) return fail(G4_ERR_INVALID_ARGUMENT, "out is null");
  if (n == 0) return ok();
  G4_TRY(use_host(ctx));
  Carve c;
  size_t oo = c.add(sizeof(float) * (size_t)n);
  G4_TRY(ensure_scratch(ctx, c.off));
  float *d = (float *)(ctx->scratch + oo);
  G4_TRY(launch_status(g4::launch_dequant(w->type, w->d, offset, n, d, ctx->stream), "dequant"));
  G4_TRY(copy_out(ctx, out, d, sizeof(float) * (size_t)n));
  return finish(ctx);
}

int g4_dequant_dev(g4_ctx *ctx, const g4_weight *w, int64_t offset, int64_t n, float *d_out) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  if (n < 0 || offset < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative offset or count");
  if (offset + n > w->n_elems)
    return fail(G4_ERR_OUT_OF_RANGE, "elements %lld..%lld exceed the tensor's %lld", (long long)offset,
                (long long)(offset + n), (long long)w->n_elems);
  if (!d_out && n > 0) return fail(G4_ERR_INVALID_ARGUMENT, "out is null");
  if (n == 0) return ok();
  G4_TRY(use_device(ctx));
  return launch_status(g4::launch_dequant(w->type, w->d, offset, n, d_out, ctx->stream), "dequant");
}

// ------------------------------------------------------------------ ffn ----

int g4_ffn(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down, const float *x,
           float *y, int32_t dim, int32_t hidden) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_ffn(ctx, w_gate, w_up, w_down, dim, hidden));
  if (!x || !y) return fail(G4_ERR_INVALID_ARGUMENT, "x/y is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)dim), oy = c.add(sizeof(float) * (size_t)dim),
         oh = c.add(sizeof(float) * (size_t)hidden), og = c.add(sizeof(float) * 2 * (size_t)hidden);
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dx = (float *)(ctx->scratch + ox), *dy = (float *)(ctx->scratch + oy);
  float *dh = (float *)(ctx->scratch + oh), *dg = (float *)(ctx->scratch + og);
  G4_TRY(copy_in(ctx, dx, x, sizeof(float) * (size_t)dim));
  G4_TRY(ffn_dev(ctx, w_gate, w_up, w_down, dx, dy, dh, dg, dim, hidden));
  G4_TRY(copy_out(ctx, y, dy, sizeof(float) * (size_t)dim));
  return finish(ctx);
}

int g4_ffn_dev(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down,
               const float *d_x, float *d_y, int32_t dim, int32_t hidden) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_ffn(ctx, w_gate, w_up, w_down, dim, hidden));
  if (!d_x || !d_y) return fail(G4_ERR_INVALID_ARGUMENT, "x/y is null");
  G4_TRY(use_device(ctx));
  Carve c;
  size_t oh = c.add(sizeof(float) * (size_t)hidden), og = c.add(sizeof(float) * 2 * (size_t)hidden);
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dh = (float *)(ctx->scratch + oh), *dg = (float *)(ctx->scratch + og);
  return ffn_dev(ctx, w_gate, w_up, w_down, d_x, d_y, dh, dg, dim, hidden);
}

int g4_ffn_gate_up(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const float *x, float *h,
                   int32_t dim, int32_t hidden) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_ffn(ctx, w_gate, w_up, nullptr, dim, hidden));
  if (!x || !h) return fail(G4_ERR_INVALID_ARGUMENT, "x/h is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)dim), oh = c.add(sizeof(float) * (size_t)hidden),
         og = c.add(sizeof(float) * 2 * (size_t)hidden);
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dx = (float *)(ctx->scratch + ox), *dh = (float *)(ctx->scratch + oh), *dg = (float *)(ctx->scratch + og);
  G4_TRY(copy_in(ctx, dx, x, sizeof(float) * (size_t)dim));
  G4_TRY(gate_up_dev(ctx, w_gate, w_up, dx, dh, dg, dim, hidden));
  G4_TRY(copy_out(ctx, h, dh, sizeof(float) * (size_t)hidden));
  return finish(ctx);
}

int g4_ffn_gate_up_dev(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const float *d_x, float *d_h,
                       int32_t dim, int32_t hidden) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_ffn(ctx, w_gate, w_up, nullptr, dim, hidden));
  if (!d_x || !d_h) return fail(G4_ERR_INVALID_ARGUMENT, "x/h is null");
  G4_TRY(use_device(ctx));
  float *dg = nullptr;
  g4::RowsArgs a = plain_rows(w_gate, 0, d_x, d_h, hidden, dim);
  a.W1 = w_up->d;
  if (!g4::rows_fast_ok(w_gate->type, a, true)) {
    Carve c;
    size_t og = c.add(sizeof(float) * 2 * (size_t)hidden);
    G4_TRY(ensure_scratch(ctx, c.off));
    dg = (float *)(ctx->scratch + og);
  }
  return gate_up_dev(ctx, w_gate, w_up, d_x, d_h, dg, dim, hidden);
}

// ------------------------------------------------------------------ moe ----

static int check_route(int32_t T, int32_t n_experts, int32_t k) {
  if (T < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative T %d", T);
  if (n_experts <= 0 || n_experts > 1024)
    return fail(G4_ERR_INVALID_ARGUMENT, "n_experts %d outside 1..1024", n_experts);
  if (k < 0 || k > n_experts) return fail(G4_ERR_INVALID_ARGUMENT, "k %d outside 0..n_experts", k);
  return G4_OK;
}

int g4_moe_route(g4_ctx *ctx, const float *logits, int32_t T, int32_t n_experts, int32_t k, int32_t renormalize,
                 const float *expert_scale, int32_t *ids, float *weights) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_route(T, n_experts, k));
  if (T == 0 || k == 0) return ok();
  if (!logits || !ids || !weights) return fail(G4_ERR_INVALID_ARGUMENT, "logits/ids/weights is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ol = c.add(sizeof(float) * (size_t)T * n_experts), os = c.add(sizeof(float) * (size_t)n_experts),
         oi = c.add(sizeof(int32_t) * (size_t)T * k), ow = c.add(sizeof(float) * (size_t)T * k);
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dl = (float *)(ctx->scratch + ol), *ds = (float *)(ctx->scratch + os);
  int32_t *di = (int32_t *)(ctx->scratch + oi);
  float *dw = (float *)(ctx->scratch + ow);
  G4_TRY(copy_in(ctx, dl, logits, sizeof(float) * (size_t)T * n_experts));
  if (expert_scale) G4_TRY(copy_in(ctx, ds, expert_scale, sizeof(float) * (size_t)n_experts));
  G4_TRY(launch_status(g4::launch_route(dl, T, n_experts, k, renormalize, expert_scale ? ds : nullptr, di, dw,
                                        ctx->stream), "moe_route"));
  G4_TRY(copy_out(ctx, ids, di, sizeof(int32_t) * (size_t)T * k));
  G4_TRY(copy_out(ctx, weights, dw, sizeof(float) * (size_t)T * k));
  return finish(ctx);
}

int g4_moe_route_dev(g4_ctx *ctx, const float *d_logits, int32_t T, int32_t n_experts, int32_t k,
                     int32_t renormalize, const float *d_expert_scale, int32_t *d_ids, float *d_weights) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_route(T, n_experts, k));
  if (T == 0 || k == 0) return ok();
  if (!d_logits || !d_ids || !d_weights) return fail(G4_ERR_INVALID_ARGUMENT, "logits/ids/weights is null");
  G4_TRY(use_device(ctx));
  return launch_status(
      g4::launch_route(d_logits, T, n_experts, k, renormalize, d_expert_scale, d_ids, d_weights, ctx->stream),
      "moe_route");
}

int g4_moe(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *X, int32_t T, int32_t dim,
           int32_t ff, const int32_t *ids, const float *weights, int32_t k, float *Y) {
  G4_TRY(check_ctx(ctx));
  int32_t ne = 0;
  G4_TRY(check_moe(ctx, w_gate_up, w_down, T, dim, ff, k, &ne));
  if (T == 0) return ok();
  if (!X || !Y || (k > 0 && (!ids || !weights))) return fail(G4_ERR_INVALID_ARGUMENT, "X/Y/ids/weights is null");
  for (int64_t i = 0; i < (int64_t)T * k; ++i)
    if (ids[i] < 0 || ids[i] >= ne)
      return fail(G4_ERR_OUT_OF_RANGE, "expert id %d at %lld outside 0..%d", ids[i], (long long)i, ne - 1);
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)T * dim), oi = c.add(sizeof(int32_t) * (size_t)T * k),
         ow = c.add(sizeof(float) * (size_t)T * k), oy = c.add(sizeof(float) * (size_t)T * dim);
  size_t oh, oys, ogu;
  moe_scratch(T, dim, ff, k, c, &oh, &oys, &ogu);
  G4_TRY(ensure_scratch(ctx, c.off));
  char *s = ctx->scratch;
  G4_TRY(copy_in(ctx, s + ox, X, sizeof(float) * (size_t)T * dim));
  if (k > 0) {
    G4_TRY(copy_in(ctx, s + oi, ids, sizeof(int32_t) * (size_t)T * k));
    G4_TRY(copy_in(ctx, s + ow, weights, sizeof(float) * (size_t)T * k));
  }
  G4_TRY(moe_dev(ctx, w_gate_up, w_down, ne, (const float *)(s + ox), T, dim, ff, (const int32_t *)(s + oi),
                 (const float *)(s + ow), k, (float *)(s + oy), (float *)(s + oh), (float *)(s + oys),
                 (float *)(s + ogu)));
  G4_TRY(copy_out(ctx, Y, s + oy, sizeof(float) * (size_t)T * dim));
  return finish(ctx);
}

int g4_moe_dev(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *d_X, int32_t T,
               int32_t dim, int32_t ff, const int32_t *d_ids, const float *d_weights, int32_t k, float *d_Y) {
  G4_TRY(check_ctx(ctx));
  int32_t ne = 0;
  G4_TRY(check_moe(ctx, w_gate_up, w_down, T, dim, ff, k, &ne));
  if (T == 0) return ok();
  if (!d_X || !d_Y || (k > 0 && (!d_ids || !d_weights)))
    return fail(G4_ERR_INVALID_ARGUMENT, "X/Y/ids/weights is null");
  G4_TRY(use_device(ctx));
  Carve c;
  size_t oh, oys, ogu;
  moe_scratch(T, dim, ff, k, c, &oh, &oys, &ogu);
  G4_TRY(ensure_scratch(ctx, c.off));
  char *s = ctx->scratch;
  return moe_dev(ctx, w_gate_up, w_down, ne, d_X, T, dim, ff, d_ids, d_weights, k, d_Y, (float *)(s + oh),
                 (float *)(s + oys), (float *)(s + ogu));
}

static int check_moe_routed(int32_t n_experts_weights, int32_t n_experts, int32_t k) {
  if (n_experts <= 0 || n_experts > 1024)
    return fail(G4_ERR_INVALID_ARGUMENT, "n_experts %d outside 1..1024", n_experts);
  if (n_experts > n_experts_weights)
    return fail(G4_ERR_OUT_OF_RANGE, "%d router logits per token, the weights hold %d experts", n_experts,
                n_experts_weights);
  if (k < 0 || k > n_experts) return fail(G4_ERR_INVALID_ARGUMENT, "k %d outside 0..n_experts", k);
  return G4_OK;
}

int g4_moe_routed(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *X, int32_t T,
                  int32_t dim, int32_t ff, const float *logits, int32_t n_experts, int32_t k, int32_t renormalize,
                  const float *expert_scale, int32_t *ids, float *weights, float *Y) {
  G4_TRY(check_ctx(ctx));
  int32_t ne = 0;
  G4_TRY(check_moe(ctx, w_gate_up, w_down, T, dim, ff, k, &ne));
  G4_TRY(check_moe_routed(ne, n_experts, k));
  if (T == 0) return ok();
  if (!X || !Y || !logits || (k > 0 && (!ids || !weights)))
    return fail(G4_ERR_INVALID_ARGUMENT, "X/Y/logits/ids/weights is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)T * dim), ol = c.add(sizeof(float) * (size_t)T * n_experts),
         os = c.add(sizeof(float) * (size_t)n_experts), oi = c.add(sizeof(int32_t) * (size_t)T * k),
         ow = c.add(sizeof(float) * (size_t)T * k), oy = c.add(sizeof(float) * (size_t)T * dim);
  size_t oh, oys, ogu;
  moe_scratch(T, dim, ff, k, c, &oh, &oys, &ogu);
  G4_TRY(ensure_scratch(ctx, c.off));
  char *s = ctx->scratch;
  G4_TRY(copy_in(ctx, s + ox, X, sizeof(float) * (size_t)T * dim));
  G4_TRY(copy_in(ctx, s + ol, logits, sizeof(float) * (size_t)T * n_experts));
  if (expert_scale) G4_TRY(copy_in(ctx, s + os, expert_scale, sizeof(float) * (size_t)n_experts));
  const MoeRoute route = {(const float *)(s + ol), n_experts, renormalize, expert_scale ? (const float *)(s + os) : nullptr};
  G4_TRY(moe_dev(ctx, w_gate_up, w_down, ne, (const float *)(s + ox), T, dim, ff, (const int32_t *)(s + oi),
                 (const float *)(s + ow), k, (float *)(s + oy), (float *)(s + oh), (float *)(s + oys),
                 (float *)(s + ogu), &route));
  G4_TRY(copy_out(ctx, Y, s + oy, sizeof(float) * (size_t)T * dim));
  if (k > 0) {
    G4_TRY(copy_out(ctx, ids, s + oi, sizeof(int32_t) * (size_t)T * k));
    G4_TRY(copy_out(ctx, weights, s + ow, sizeof(float) * (size_t)T * k));
  }
  return finish(ctx);
}

int g4_moe_routed_dev(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *d_X, int32_t T,
                      int32_t dim, int32_t ff, const float *d_logits, int32_t n_experts, int32_t k,
                      int32_t renormalize, const float *d_expert_scale, int32_t *d_ids, float *d_weights,
                      float *d_Y) {
  G4_TRY(check_ctx(ctx));
  int32_t ne = 0;
  G4_TRY(check_moe(ctx, w_gate_up, w_down, T, dim, ff, k, &ne));
  G4_TRY(check_moe_routed(ne, n_experts, k));
  if (T == 0) return ok();
  if (!d_X || !d_Y || !d_logits || (k > 0 && (!d_ids || !d_weights)))
    return fail(G4_ERR_INVALID_ARGUMENT, "X/Y/logits/ids/weights is null");
  G4_TRY(use_device(ctx));
  Carve c;
  size_t oh, oys, ogu;
  moe_scratch(T, dim, ff, k, c, &oh, &oys, &ogu);
  G4_TRY(ensure_scratch(ctx, c.off));
  char *s = ctx->scratch;
  const MoeRoute route = {d_logits, n_experts, renormalize, d_expert_scale};
  return moe_dev(ctx, w_gate_up, w_down, ne, d_X, T, dim, ff, d_ids, d_weights, k, d_Y, (float *)(s + oh),
                 (float *)(s + oys), (float *)(s + ogu), &route);
}

int g4_moe_routed_dev_noalloc(g4_ctx *ctx, const g4_weight *w_gate_up, const g4_weight *w_down, const float *d_X,
                              int32_t T, int32_t dim, int32_t ff, const float *d_logits, int32_t n_experts, int32_t k,
                              int32_t renormalize, const float *d_expert_scale, int32_t *d_ids, float *d_weights,
                              float *d_Y) {
  G4_TRY(check_ctx(ctx));
  int32_t ne = 0;
  G4_TRY(check_moe(ctx, w_gate_up, w_down, T, dim, ff, k, &ne));
  G4_TRY(check_moe_routed(ne, n_experts, k));
  if (T == 0) return ok();
  if (!d_X || !d_Y || !d_logits || (k > 0 && (!d_ids || !d_weights)))
    return fail(G4_ERR_INVALID_ARGUMENT, "X/Y/logits/ids/weights is null");
  Carve c;
  size_t oh, oys, ogu;
  moe_scratch(T, dim, ff, k, c, &oh, &oys, &ogu);
  if (c.off > G4_NOALLOC_SCRATCH_BYTES)
    return fail(G4_ERR_INVALID_ARGUMENT,
                "%d tokens x %d slots need %zu bytes of scratch (4 * T * k * (3 * ff + dim), rounded up); "
                "the allocation-free entry point holds %zu",
                T, k, c.off, G4_NOALLOC_SCRATCH_BYTES);
  char *s = ctx->device < G4_MAX_DEVICES ? g_noalloc_scratch[ctx->device].load(std::memory_order_acquire) : nullptr;
  if (!s) return fail(G4_ERR_DEVICE, "no static scratch for device %d", ctx->device);
  G4_TRY(use_device(ctx));
  const MoeRoute route = {d_logits, n_experts, renormalize, d_expert_scale};
  return moe_dev(ctx, w_gate_up, w_down, ne, d_X, T, dim, ff, d_ids, d_weights, k, d_Y, (float *)(s + oh),
                 (float *)(s + oys), (float *)(s + ogu), &route);
}

// ---------------------------------------------------------- decode step ----

int g4_rmsnorm_dev(g4_ctx *ctx, const g4_weight *weight, const float *d_x, float *d_out, int32_t n_vec, int32_t size,
                   float eps, int form) {
  G4_TRY(check_ctx(ctx));
  if (form != G4_NORM_WEIGHT_AFTER && form != G4_NORM_WEIGHT_FIRST && form != G4_NORM_NO_WEIGHT)
    return fail(G4_ERR_INVALID_ARGUMENT, "unknown norm form %d", form);
  if (n_vec < 0 || size < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative n_vec or size (%d, %d)", n_vec, size);
  G4_TRY(check_eps_cap(eps, 0.f));
  if (form != G4_NORM_NO_WEIGHT) G4_TRY(check_norm(ctx, weight, size, "weight"));
  if (n_vec == 0 || size == 0) return ok();
  if (!d_x || !d_out) return fail(G4_ERR_INVALID_ARGUMENT, "x/out is null");
  const size_t bytes = sizeof(float) * (size_t)n_vec * size;
  if (d_x != d_out && ranges_overlap(d_x, bytes, d_out, bytes))
    return fail(G4_ERR_INVALID_ARGUMENT, "out overlaps x without being x");
  G4_TRY(use_device(ctx));
  const float *w = form == G4_NORM_NO_WEIGHT ? nullptr : (const float *)weight->d;
  return launch_status(g4::launch_rmsnorm(d_x, w, d_out, nullptr, n_vec, size, eps, form, ctx->stream), "rmsnorm");
}

int g4_rmsnorm_add_dev(g4_ctx *ctx, const g4_weight *weight, float *d_v, float *d_x, int32_t size, float eps) {
  G4_TRY(check_ctx(ctx));
  if (size < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative size %d", size);
  G4_TRY(check_eps_cap(eps, 0.f));
  G4_TRY(check_norm(ctx, weight, size, "weight"));
  if (size == 0) return ok();
  if (!d_v || !d_x) return fail(G4_ERR_INVALID_ARGUMENT, "v/x is null");
  const size_t bytes = sizeof(float) * (size_t)size;
  if (ranges_overlap(d_v, bytes, d_x, bytes)) return fail(G4_ERR_INVALID_ARGUMENT, "v overlaps x");
  G4_TRY(use_device(ctx));
  return launch_status(g4::launch_rmsnorm(d_v, (const float *)weight->d, d_v, d_x, 1, size, eps,
                                          G4_NORM_WEIGHT_AFTER, ctx->stream), "rmsnorm_add");
}

int g4_add_dev(g4_ctx *ctx, float *d_x, const float *d_that, int32_t n) {
  G4_TRY(check_ctx(ctx));
  if (n < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative size %d", n);
  if (n == 0) return ok();
  if (!d_x || !d_that) return fail(G4_ERR_INVALID_ARGUMENT, "x/that is null");
  G4_TRY(use_device(ctx));
  return launch_status(g4::launch_add(d_x, d_that, n, ctx->stream), "add");
}

int g4_softcap_dev(g4_ctx *ctx, float *d_v, int32_t n, float cap) {
  G4_TRY(check_ctx(ctx));
  if (n < 0) return fail(G4_ERR_INVALID_ARGUMENT, "negative size %d", n);
  if (!(cap > 0.f) || cap == __builtin_inff()) return fail(G4_ERR_INVALID_ARGUMENT, "softcap must be finite and > 0");
  if (n == 0) return ok();
  if (!d_v) return fail(G4_ERR_INVALID_ARGUMENT, "v is null");
  G4_TRY(use_device(ctx));
  return launch_status(g4::launch_softcap(d_v, n, cap, ctx->stream), "softcap");
}

int g4_matmul_norm_dev(g4_ctx *ctx, const g4_weight *w, int64_t this_offset, const g4_weight *norm, const float *d_x,
                       float eps, float *d_xnorm, float *d_out, int32_t dim0, int32_t dim1) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_weight(ctx, w, "weight"));
  G4_TRY(check_rows(w, this_offset, dim0, dim1));
  G4_TRY(check_norm(ctx, norm, dim1, "norm"));
  G4_TRY(check_eps_cap(eps, 0.f));
  if ((!d_x && dim1 > 0) || (!d_out && dim0 > 0)) return fail(G4_ERR_INVALID_ARGUMENT, "x/out is null");
  if (d_xnorm && dim1 > 0 && ranges_overlap(d_xnorm, sizeof(float) * (size_t)dim1, d_x, sizeof(float) * (size_t)dim1))
    return fail(G4_ERR_INVALID_ARGUMENT, "xnorm overlaps x");
  G4_TRY(use_device(ctx));
  if (dim1 == 0) {
    if (dim0 > 0) G4_TRY(zero_dev(ctx, d_out, sizeof(float) * (size_t)dim0));
    return ok();
  }
  if (dim0 == 0) {
    if (!d_xnorm) return ok();
    return launch_status(g4::launch_rmsnorm(d_x, (const float *)norm->d, d_xnorm, nullptr, 1, dim1, eps,
                                            G4_NORM_WEIGHT_AFTER, ctx->stream), "rmsnorm");
  }
  // launches that cannot take the fused norm (rows not 64-aligned, several
  // column passes) normalise into scratch first
  float *xn = nullptr;
  if (!d_xnorm && norm_scratch_floats(w, this_offset, dim0, dim1, false) > 0) {
    Carve c;
    size_t o = c.add(sizeof(float) * (size_t)dim1);
    G4_TRY(ensure_scratch(ctx, c.off));
    xn = (float *)(ctx->scratch + o);
  }
  return matmul_norm_dev(ctx, w, this_offset, norm, d_x, eps, d_xnorm, d_out, dim0, dim1, g4::EPI_STORE, nullptr, xn,
                         nullptr, nullptr, 0.f);
}

int g4_ffn_block(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down,
                 const g4_weight *norm_pre, const g4_weight *norm_post, float *x, int32_t dim, int32_t hidden,
                 float eps) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_ffn_block(ctx, w_gate, w_up, w_down, norm_pre, norm_post, dim, hidden, eps));
  if (!x) return fail(G4_ERR_INVALID_ARGUMENT, "x is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)dim), oh, oy, og, on;
  ffn_block_scratch(w_gate, dim, hidden, c, &oh, &oy, &og, &on);
  G4_TRY(ensure_scratch(ctx, c.off));
  char *s = ctx->scratch;
  G4_TRY(copy_in(ctx, s + ox, x, sizeof(float) * (size_t)dim));
  G4_TRY(ffn_block_dev(ctx, w_gate, w_up, w_down, norm_pre, norm_post, (float *)(s + ox), dim, hidden, eps,
                       (float *)(s + oh), (float *)(s + oy), (float *)(s + og), (float *)(s + on)));
  G4_TRY(copy_out(ctx, x, s + ox, sizeof(float) * (size_t)dim));
  return finish(ctx);
}

int g4_ffn_block_dev(g4_ctx *ctx, const g4_weight *w_gate, const g4_weight *w_up, const g4_weight *w_down,
                     const g4_weight *norm_pre, const g4_weight *norm_post, float *d_x, int32_t dim, int32_t hidden,
                     float eps) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_ffn_block(ctx, w_gate, w_up, w_down, norm_pre, norm_post, dim, hidden, eps));
  if (!d_x) return fail(G4_ERR_INVALID_ARGUMENT, "x is null");
  G4_TRY(use_device(ctx));
  Carve c;
  size_t oh, oy, og, on;
  ffn_block_scratch(w_gate, dim, hidden, c, &oh, &oy, &og, &on);
  G4_TRY(ensure_scratch(ctx, c.off));
  char *s = ctx->scratch;
  return ffn_block_dev(ctx, w_gate, w_up, w_down, norm_pre, norm_post, d_x, dim, hidden, eps, (float *)(s + oh),
                       (float *)(s + oy), (float *)(s + og), (float *)(s + on));
}

int g4_lm_head(g4_ctx *ctx, const g4_weight *w_cls, const g4_weight *norm_final, const float *x, float *logits,
               int32_t *index, int32_t vocab, int32_t dim, float eps, float softcap) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_lm_head(ctx, w_cls, norm_final, vocab, dim, eps, softcap));
  if (!x || !index) return fail(G4_ERR_INVALID_ARGUMENT, "x/index is null");
  G4_TRY(use_host(ctx));
  Carve c;
  size_t ox = c.add(sizeof(float) * (size_t)dim), on = c.add(sizeof(float) * (size_t)dim),
         oy = c.add(sizeof(float) * (size_t)vocab), oi = c.add(sizeof(int32_t));
  G4_TRY(ensure_scratch(ctx, c.off));
  char *s = ctx->scratch;
  G4_TRY(copy_in(ctx, s + ox, x, sizeof(float) * (size_t)dim));
  G4_TRY(matmul_norm_dev(ctx, w_cls, 0, norm_final, (const float *)(s + ox), eps, nullptr, (float *)(s + oy), vocab,
                         dim, g4::EPI_ARGMAX, nullptr, (float *)(s + on), nullptr, (int32_t *)(s + oi), softcap));
  if (logits) G4_TRY(copy_out(ctx, logits, s + oy, sizeof(float) * (size_t)vocab));
  G4_TRY(copy_out(ctx, index, s + oi, sizeof(int32_t)));
  return finish(ctx);
}

int g4_lm_head_dev(g4_ctx *ctx, const g4_weight *w_cls, const g4_weight *norm_final, const float *d_x, float *d_xnorm,
                   float *d_logits, int32_t *d_index, int32_t vocab, int32_t dim, float eps, float softcap) {
  G4_TRY(check_ctx(ctx));
  G4_TRY(check_lm_head(ctx, w_cls, norm_final, vocab, dim, eps, softcap));
  if (!d_x || !d_index) return fail(G4_ERR_INVALID_ARGUMENT, "x/index is null");
  if (d_xnorm && ranges_overlap(d_xnorm, sizeof(float) * (size_t)dim, d_x, sizeof(float) * (size_t)dim))
    return fail(G4_ERR_INVALID_ARGUMENT, "xnorm overlaps x");
  G4_TRY(use_device(ctx));
  Carve c;
  size_t oy = c.add(d_logits ? 0 : sizeof(float) * (size_t)vocab), on = c.add(sizeof(float) * (size_t)dim);
  G4_TRY(ensure_scratch(ctx, c.off));
  float *dy = d_logits ? d_logits : (float *)(ctx->scratch + oy);
  return matmul_norm_dev(ctx, w_cls, 0, norm_final, d_x, eps, d_xnorm, dy, vocab, dim, g4::EPI_ARGMAX, nullptr,
                         (float *)(ctx->scratch + on), nullptr, d_index, softcap);
}

// ------------------------------------------------------------ attention ----

int g4_attention_dev(g4_ctx *ctx, const float *d_q, const float *d_key_cache, const float *d_value_cache,
                     float *d_out, int32_t n_heads, int32_t n_kv_heads, int32_t head_size, int32_t position,
                     int32_t att_start) {
  G4_TRY(check_ctx(ctx));
  if (n_heads <= 0 || n_kv_heads <= 0 || head_size <= 0)
    return fail(G4_ERR_INVALID_ARGUMENT, "heads and head size must be positive (%d, %d, %d)", n_heads, n_kv_heads,
                head_size);
  if (n_heads % n_kv_heads != 0)
    return fail(G4_ERR_INVALID_ARGUMENT, "n_heads %d is not a multiple of n_kv_heads %d", n_heads, n_kv_heads);
  if (att_start < 0 || position < att_start)
    return fail(G4_ERR_OUT_OF_RANGE, "positions %d..%d", att_start, position);
  if ((int64_t)n_kv_heads * head_size > 0x7fffffff) return fail(G4_ERR_INVALID_ARGUMENT, "kv_dim too large");
  if (!d_q || !d_key_cache || !d_value_cache || !d_out) return fail(G4_ERR_INVALID_ARGUMENT, "null pointer");
  G4_TRY(use_device(ctx));
  g4::AttArgs a;
  memset(&a, 0, sizeof(a));
  a.q = d_q;
  a.kc = d_key_cache;
  a.vc = d_value_cache;
  a.out = d_out;
  a.n_heads = n_heads;
  a.n_kv = n_kv_heads;
  a.hs = head_size;
  a.row0 = att_start;
  a.rows = position - att_start + 1;
  // the vector kernel reads 16-byte words: caches, q and out must be 16-byte aligned
  a.generic = ((uintptr_t)d_q | (uintptr_t)d_key_cache | (uintptr_t)d_value_cache | (uintptr_t)d_out) % 16 != 0;
  g4::attention_plan(a, ctx->dev);
  Carve c;
  size_t o = c.add(sizeof(float) * (size_t)g4::attention_scratch_floats(a));
  G4_TRY(ensure_scratch(ctx, c.off));
  return launch_status(g4::launch_attention(a, (float *)(ctx->scratch + o), ctx->stream), "attention");
}

}  // extern "C"
