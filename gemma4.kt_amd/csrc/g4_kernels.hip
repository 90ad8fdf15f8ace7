// g4_kernels.hip -- gfx950 kernels of the quantized matrix-vector path.
//
// Row-stream matvec engine (k_rows): a wave owns a contiguous range of rows and
// keeps its 64-column slice of x in registers across them.  Lanes split each
// row into 64-element chunks (two Q8_0/Q4_0 blocks, one Q4_K group), load them
// with dword-aligned 128-bit loads, unpack in registers and reduce the row
// partial sums across the lane group with a transposing butterfly.  x is staged
// once per workgroup in LDS (XOR-swizzled so the per-lane 256-byte reads are
// bank-conflict free).  Rows that do not start on a 64-element boundary go to
// k_rows_generic, a per-element restatement of the reference's get()-based dot.
//
// Reference paths are relative to lib/src/main/kotlin/io/github/lbenedetto/internal/.
#include <float.h>
#include <limits.h>

#include "g4_device.hpp"
#include "g4_internal.hpp"

namespace g4 {

// --------------------------------------------------------------- engine ----

template <class F, int LPR, int EPI>
__global__ __launch_bounds__(256) void k_rows(RowsArgs a) {
  constexpr int RT = F::RT;
  constexpr int RPW = 64 / LPR;                  // rows in flight per step (one per lane group)
  constexpr int TR = RT * RPW;                   // physical rows per tile
  constexpr int LRT = (EPI == EPI_GELU_PAIR) ? TR / 2 : TR;  // logical rows per tile
  constexpr int PX = LPR * 64;                   // columns per pass
  static_assert(EPI != EPI_GELU_PAIR || RT >= 2, "paired tiles need two steps");

  __shared__ float4 xl[PX / 4];
  __shared__ float red_v[4];
  __shared__ int red_i[4];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int gi = lane / LPR, q = lane % LPR;
  const int seg = blockIdx.y;
  const int expert = a.ids ? a.ids[seg] : 0;
  const bool bad_expert = a.ids && (expert < 0 || expert >= a.expert_count);
  const int64_t ebase = bad_expert ? 0 : (int64_t)expert * a.expert_stride;
  const float *x = a.x + (int64_t)(seg / a.x_div) * a.x_stride;
  float *y = a.y ? a.y + (int64_t)seg * a.y_stride : nullptr;

  const int n_tiles = (a.rows + LRT - 1) / LRT;
  const int nwv = gridDim.x * 4, wv = blockIdx.x * 4 + wid;
  const int tpw = (n_tiles + nwv - 1) / nwv;
  const int t0 = wv * tpw, t1 = min(n_tiles, t0 + tpw);
  const int C = a.dim1 >> 6;
  const int passes = (C + LPR - 1) / LPR;

  float best_v = -__builtin_inff();
  int best_i = INT_MAX;

  for (int pass = 0; pass < passes; ++pass) {
    __syncthreads();
    for (int f4 = tid; f4 < PX / 4; f4 += 256) {
      const int col = pass * PX + f4 * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (col < a.dim1) v = make_float4(x[col], x[col + 1], x[col + 2], x[col + 3]);
      const int qq = f4 >> 4, i = f4 & 15;
      xl[qq * 16 + (i ^ (qq & 15))] = v;
    }
    __syncthreads();

    float xv[64];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float4 t = xl[q * 16 + (i ^ (q & 15))];
      xv[4 * i] = t.x; xv[4 * i + 1] = t.y; xv[4 * i + 2] = t.z; xv[4 * i + 3] = t.w;
    }
    float xs[F::NS > 0 ? F::NS : 1];
    F::sums(xv, xs);

    const int c = pass * LPR + q;
    const bool active = c < C;
    const int64_t ecol = (int64_t)c * 64;
    const bool last_pass = pass == passes - 1;

    for (int t = t0; t < t1; ++t) {
      uint32_t D[RT][F::NDW];
      int64_t E[RT];
      bool ok[RT];
#pragma unroll
      for (int k = 0; k < RT; ++k) {
        int lr;
        const uint8_t *W;
        int64_t base;
        if constexpr (EPI == EPI_GELU_PAIR) {
          lr = t * LRT + (k % (RT / 2)) * RPW + gi;
          W = k < RT / 2 ? a.W0 : a.W1;
          base = k < RT / 2 ? a.base0 : a.base1;
        } else {
          lr = t * LRT + k * RPW + gi;
          W = a.W0;
          base = a.base0;
        }
        ok[k] = active && lr < a.rows && !bad_expert;
        E[k] = base + ebase + (int64_t)lr * a.row_stride + ecol;
        if (ok[k]) {
          F::load(W, E[k], D[k]);
        } else {
#pragma unroll
          for (int i = 0; i < F::NDW; ++i) D[k][i] = 0u;
        }
      }
      float v[RT];
#pragma unroll
      for (int k = 0; k < RT; ++k) {
        float r = F::dot(D[k], xv, xs, E[k]);
        v[k] = ok[k] ? r : 0.f;
      }
      const float r = reduce_transpose<RT, LPR>(v, lane);
      const int k = q / (LPR / RT);
      const bool writer = (q % (LPR / RT)) == 0;

      if constexpr (EPI == EPI_GELU_PAIR) {
        const float up = __shfl_xor(r, LPR / 2, 64);
        const int lr = t * LRT + (k % (RT / 2)) * RPW + gi;
        if (writer && k < RT / 2 && lr < a.rows) y[lr] = gelu_ref(r) * up;
      } else {
        const int lr = t * LRT + k * RPW + gi;
        if (writer && lr < a.rows) {
          float val = r;
          if (y) {
            if (pass > 0) val += y[lr];
            y[lr] = val;
          }
          if constexpr (EPI == EPI_ARGMAX) {
            if (last_pass) {
              const float key = am_key(val, lr);
              if (am_better(key, lr, best_v, best_i)) best_v = key, best_i = lr;
            }
          }
        }
      }
    }
  }

  if constexpr (EPI == EPI_ARGMAX) {
    am_wave(best_v, best_i);
    if (lane == 0) red_v[wid] = best_v, red_i[wid] = best_i;
    __syncthreads();
    __shared__ bool is_last;
    if (tid == 0) {
      float bv = red_v[0];
      int bi = red_i[0];
      for (int w = 1; w < 4; ++w)
        if (am_better(red_v[w], red_i[w], bv, bi)) bv = red_v[w], bi = red_i[w];
      a.am_val[blockIdx.x] = bv;
      a.am_idx[blockIdx.x] = bi;
      __threadfence();
      const uint32_t prev = atomicAdd(a.am_counter, 1u);
      is_last = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (is_last) {
      __threadfence();
      float bv = -__builtin_inff();
      int bi = INT_MAX;
      const volatile float *pv = a.am_val;
      const volatile int32_t *pi = a.am_idx;
      for (int b = tid; b < (int)gridDim.x; b += 256) {
        const float v = pv[b];
        const int i = pi[b];
        if (am_better(v, i, bv, bi)) bv = v, bi = i;
      }
      am_wave(bv, bi);
      if (lane == 0) red_v[wid] = bv, red_i[wid] = bi;
      __syncthreads();
      if (tid == 0) {
        bv = red_v[0];
        bi = red_i[0];
        for (int w = 1; w < 4; ++w)
          if (am_better(red_v[w], red_i[w], bv, bi)) bv = red_v[w], bi = red_i[w];
        *a.am_out = bi;
        *a.am_counter = 0u;
      }
    }
  }
}

// ------------------------------------------------------- generic rows ----
// Any offset / row length: one wave per physical row, lanes stride over the
// elements with the per-element decode (FloatTensorHelpers.kt:65-71 computes the
// same sum sequentially).  Output y[seg * y_stride + m * rows + r] for matrix m.
template <int TYPE>
__global__ __launch_bounds__(256) void k_rows_generic(RowsArgs a, int nmat) {
  const int lane = threadIdx.x & 63;
  const int seg = blockIdx.y;
  const int expert = a.ids ? a.ids[seg] : 0;
  const bool bad_expert = a.ids && (expert < 0 || expert >= a.expert_count);
  const int64_t ebase = bad_expert ? 0 : (int64_t)expert * a.expert_stride;
  const float *x = a.x + (int64_t)(seg / a.x_div) * a.x_stride;
  float *y = a.y + (int64_t)seg * a.y_stride;
  const int total = nmat * a.rows;
  const int nwv = gridDim.x * 4;
  for (int pr = blockIdx.x * 4 + (threadIdx.x >> 6); pr < total; pr += nwv) {
    const int m = pr / a.rows, r = pr % a.rows;
    const uint8_t *W = m == 0 ? a.W0 : a.W1;
    const int64_t off = (m == 0 ? a.base0 : a.base1) + ebase + (int64_t)r * a.row_stride;
    float acc = 0.f;
    if (!bad_expert)
      for (int j = lane; j < a.dim1; j += 64) acc = __builtin_fmaf(dot_elem<TYPE>(W, off + j, j, a.dim1), x[j], acc);
    acc = wave_sum(acc);
    if (lane == 0) y[pr] = acc;
  }
}

// h[s*rows + i] = gelu(gu[s*2rows + i]) * gu[s*2rows + rows + i]   (Llama.kt:357-361)
__global__ void k_gelu_mul(const float *gu, int32_t rows, int32_t segments, float *h, int64_t h_stride) {
  const int64_t n = (int64_t)rows * segments;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t s = i / rows, r = i % rows;
    h[s * h_stride + r] = gelu_ref(gu[s * 2 * rows + r]) * gu[s * 2 * rows + rows + r];
  }
}

// ---------------------------------------------------------------- dequant ----
template <int TYPE>
__global__ void k_dequant(const uint8_t *W, int64_t offset, int64_t n, float *out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = get_elem<TYPE>(W, offset + i);
}

// ----------------------------------------------------------------- argmax ----
// FloatTensor.kt:53-66 over v[0..n): per-block partials, the last block to
// arrive reduces them in block order and resets the counter.
__global__ __launch_bounds__(256) void k_argmax(const float *v, int32_t n, float *part_val, int32_t *part_idx,
                                                uint32_t *counter, int32_t *out) {
  __shared__ float rv[4];
  __shared__ int ri[4];
  __shared__ bool is_last;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  float bv = -__builtin_inff();
  int bi = INT_MAX;
  for (int i = blockIdx.x * 256 + tid; i < n; i += gridDim.x * 256) {
    const float k = am_key(v[i], i);
    if (am_better(k, i, bv, bi)) bv = k, bi = i;
  }
  am_wave(bv, bi);
  if (lane == 0) rv[wid] = bv, ri[wid] = bi;
  __syncthreads();
  if (tid == 0) {
    bv = rv[0];
    bi = ri[0];
    for (int w = 1; w < 4; ++w)
      if (am_better(rv[w], ri[w], bv, bi)) bv = rv[w], bi = ri[w];
    part_val[blockIdx.x] = bv;
    part_idx[blockIdx.x] = bi;
    __threadfence();
    is_last = atomicAdd(counter, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  bv = -__builtin_inff();
  bi = INT_MAX;
  const volatile float *pv = part_val;
  const volatile int32_t *pi = part_idx;
  for (int b = tid; b < (int)gridDim.x; b += 256) {
    const float vv = pv[b];
    const int ii = pi[b];
    if (am_better(vv, ii, bv, bi)) bv = vv, bi = ii;
  }
  am_wave(bv, bi);
  __syncthreads();
  if (lane == 0) rv[wid] = bv, ri[wid] = bi;
  __syncthreads();
  if (tid == 0) {
    bv = rv[0];
    bi = ri[0];
    for (int w = 1; w < 4; ++w)
      if (am_better(rv[w], ri[w], bv, bi)) bv = rv[w], bi = ri[w];
    *out = bi;
    *counter = 0u;
  }
}

// ------------------------------------------------------------------ route ----
// One 64-lane block per token.  Softmax of MutableFloatTensor.kt:54-59 (max with
// java.lang.Math.max semantics, exp in double, fp32 sum in index order, fp32
// divide), top-k of Llama.kt:275-293 (strict >, ties to the lowest index,
// chosen entries masked to -inf), optional renormalisation (fp32 sum in k
// order) and expert scale.
constexpr int ROUTE_MAX_E = 1024;

G4_DEV float java_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == 0.f && b == 0.f) return __builtin_signbit(a) ? b : a;
  return a >= b ? a : b;
}

__global__ __launch_bounds__(64) void k_route(const float *logits, int32_t E, int32_t K, int32_t renorm,
                                              const float *expert_scale, int32_t *ids, float *weights) {
  __shared__ float p[ROUTE_MAX_E];
  __shared__ float sum_s;
  const int t = blockIdx.x, lane = threadIdx.x;
  const float *lg = logits + (int64_t)t * E;
  float m = -__builtin_inff();
  for (int i = lane; i < E; i += 64) m = java_max(m, lg[i]);
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) m = java_max(m, __shfl_xor(m, s, 64));
  for (int i = lane; i < E; i += 64) p[i] = (float)exp((double)__fsub_rn(lg[i], m));
  __syncthreads();
  if (lane == 0) {
    float s = 0.f;
    for (int i = 0; i < E; ++i) s = __fadd_rn(s, p[i]);
    sum_s = s;
  }
  __syncthreads();
  const float sum = sum_s;
  for (int i = lane; i < E; i += 64) p[i] = __fdiv_rn(p[i], sum);
  __syncthreads();
  float renorm_sum = 0.f;
  for (int j = 0; j < K; ++j) {
    float bv = -__builtin_inff();
    int bi = INT_MAX;
    for (int i = lane; i < E; i += 64) {
      const float v = p[i] != p[i] ? -__builtin_inff() : p[i];
      if (am_better(v, i, bv, bi)) bv = v, bi = i;
    }
    am_wave(bv, bi);
    if (bv == -__builtin_inff()) bi = 0;  // no entry beats the initial -inf: the scan keeps index 0
    __syncthreads();
    if (lane == 0) {
      ids[(int64_t)t * K + j] = bi;
      weights[(int64_t)t * K + j] = bv;
      p[bi] = -__builtin_inff();
      renorm_sum = __fadd_rn(renorm_sum, bv);
    }
    __syncthreads();
  }
  if (lane == 0) {
    for (int j = 0; j < K; ++j) {
      float w = weights[(int64_t)t * K + j];
      if (renorm) w = __fdiv_rn(w, renorm_sum);
      if (expert_scale) w = __fmul_rn(w, expert_scale[ids[(int64_t)t * K + j]]);
      weights[(int64_t)t * K + j] = w;
    }
  }
}

// Y[t*dim + r] = sum_j w[t,j] * ys[(t*K + j)*dim + r] in j order, a*d + out like
// saxpyInPlace (MutableFloatTensor.kt:61-66).
__global__ void k_moe_combine(const float *ys, const float *w, int32_t T, int32_t K, int32_t dim, float *Y) {
  const int64_t n = (int64_t)T * dim;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / dim, r = i % dim;
    float out = 0.f;
    for (int j = 0; j < K; ++j)
      out = __fadd_rn(__fmul_rn(w[t * K + j], ys[(t * K + j) * dim + r]), out);
    Y[i] = out;
  }
}

// ---------------------------------------------------------------- launchers ----

bool rows_fast_ok(int type, const RowsArgs &a, bool paired) {
  if (a.dim1 <= 0 || (a.dim1 % 64) != 0) return false;
  if ((a.base0 % 64) != 0 || (a.row_stride % 64) != 0 || (a.expert_stride % 64) != 0) return false;
  if (paired && (a.base1 % 64) != 0) return false;
  if (paired && (a.dim1 / 64) > 64) return false;  // paired epilogue needs a single column pass
  switch (type) {
    case T_Q8_0: case T_Q4_0: case T_Q4_K: case T_F16: case T_BF16: case T_F32: return true;
    default: return false;
  }
}

int max_argmax_blocks(const DevInfo &dev) { return dev.cu_count * 2; }

template <class F, int LPR>
static hipError_t launch_fast_lpr(int epi, const RowsArgs &a, int segments, const DevInfo &dev, hipStream_t s) {
  constexpr int RT = F::RT, RPW = 64 / LPR, TR = RT * RPW;
  const int lrt = epi == EPI_GELU_PAIR ? TR / 2 : TR;
  const int n_tiles = (a.rows + lrt - 1) / lrt;
  // target ~8 waves (two per SIMD) per CU over the whole launch
  int max_blocks = dev.cu_count * 2 / (segments > 0 ? segments : 1);
  if (max_blocks < 1) max_blocks = 1;
  if (epi == EPI_ARGMAX) max_blocks = max_argmax_blocks(dev);
  int blocks = (n_tiles + 3) / 4;
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  dim3 grid(blocks, segments);
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((k_rows<F, LPR, EPI_STORE>), grid, dim3(256), 0, s, a); break;
    case EPI_ARGMAX: hipLaunchKernelGGL((k_rows<F, LPR, EPI_ARGMAX>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((k_rows<F, LPR, EPI_GELU_PAIR>), grid, dim3(256), 0, s, a); break;
  }
  return hipGetLastError();
}

template <class F>
static hipError_t launch_fast(int epi, const RowsArgs &a, int segments, const DevInfo &dev, hipStream_t s) {
  const int C = a.dim1 / 64;
  if (C > 32) return launch_fast_lpr<F, 64>(epi, a, segments, dev, s);
  if (C > 16) return launch_fast_lpr<F, 32>(epi, a, segments, dev, s);
  return launch_fast_lpr<F, 16>(epi, a, segments, dev, s);
}

template <int TYPE>
static hipError_t launch_generic_t(const RowsArgs &a, int nmat, int segments, const DevInfo &dev, hipStream_t s) {
  const int total = nmat * a.rows;
  int blocks = (total + 3) / 4;
  const int cap = dev.cu_count * 4;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((k_rows_generic<TYPE>), dim3(blocks, segments), dim3(256), 0, s, a, nmat);
  return hipGetLastError();
}

static hipError_t launch_generic(int type, const RowsArgs &a, int nmat, int segments, const DevInfo &dev,
                                 hipStream_t s) {
  switch (type) {
    case T_Q8_0: return launch_generic_t<T_Q8_0>(a, nmat, segments, dev, s);
    case T_Q4_0: return launch_generic_t<T_Q4_0>(a, nmat, segments, dev, s);
    case T_Q4_K: return launch_generic_t<T_Q4_K>(a, nmat, segments, dev, s);
    case T_F16: return launch_generic_t<T_F16>(a, nmat, segments, dev, s);
    case T_BF16: return launch_generic_t<T_BF16>(a, nmat, segments, dev, s);
    case T_F32: return launch_generic_t<T_F32>(a, nmat, segments, dev, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rows(int type, int epi, const RowsArgs &a, int segments, const DevInfo &dev, float *scratch,
                       hipStream_t s) {
  if (rows_fast_ok(type, a, epi == EPI_GELU_PAIR)) {
    switch (type) {
      case T_Q8_0: return launch_fast<FmtQ8_0>(epi, a, segments, dev, s);
      case T_Q4_0: return launch_fast<FmtQ4_0>(epi, a, segments, dev, s);
      case T_Q4_K: return launch_fast<FmtQ4_K>(epi, a, segments, dev, s);
      case T_F16: return launch_fast<FmtHalf<T_F16>>(epi, a, segments, dev, s);
      case T_BF16: return launch_fast<FmtHalf<T_BF16>>(epi, a, segments, dev, s);
      case T_F32: return launch_fast<FmtF32>(epi, a, segments, dev, s);
      default: return hipErrorInvalidValue;
    }
  }
  // generic path
  if (epi == EPI_GELU_PAIR) {
    RowsArgs g = a;
    g.y = scratch;
    g.y_stride = 2 * (int64_t)a.rows;
    hipError_t e = launch_generic(type, g, 2, segments, dev, s);
    if (e != hipSuccess) return e;
    const int64_t n = (int64_t)a.rows * segments;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_gelu_mul, dim3(blocks), dim3(256), 0, s, (const float *)scratch, a.rows, segments, a.y,
                       a.y_stride);
    return hipGetLastError();
  }
  hipError_t e = launch_generic(type, a, 1, segments, dev, s);
  if (e != hipSuccess || epi != EPI_ARGMAX) return e;
  return launch_argmax(a.y, a.rows, a.am_val, a.am_idx, a.am_counter, a.am_out, dev, s);
}

hipError_t launch_dequant(int type, const uint8_t *W, int64_t offset, int64_t n, float *out, hipStream_t s) {
  int64_t b = (n + 255) / 256;
  int blocks = (int)(b > 8192 ? 8192 : (b < 1 ? 1 : b));
  switch (type) {
    case T_Q8_0: hipLaunchKernelGGL(k_dequant<T_Q8_0>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_Q4_0: hipLaunchKernelGGL(k_dequant<T_Q4_0>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_Q4_K: hipLaunchKernelGGL(k_dequant<T_Q4_K>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_F16: hipLaunchKernelGGL(k_dequant<T_F16>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_BF16: hipLaunchKernelGGL(k_dequant<T_BF16>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_F32: hipLaunchKernelGGL(k_dequant<T_F32>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_argmax(const float *v, int32_t n, float *part_val, int32_t *part_idx, uint32_t *counter,
                         int32_t *out, const DevInfo &dev, hipStream_t s) {
  int blocks = (n + 255) / 256;
  const int cap = max_argmax_blocks(dev);
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_argmax, dim3(blocks), dim3(256), 0, s, v, n, part_val, part_idx, counter, out);
  return hipGetLastError();
}

hipError_t launch_route(const float *logits, int32_t T, int32_t n_experts, int32_t k, int32_t renorm,
                        const float *expert_scale, int32_t *ids, float *weights, hipStream_t s) {
  if (n_experts > ROUTE_MAX_E) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_route, dim3(T), dim3(64), 0, s, logits, n_experts, k, renorm, expert_scale, ids, weights);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const float *ys, const float *weights, int32_t T, int32_t k, int32_t dim, float *Y,
                              hipStream_t s) {
  const int64_t n = (int64_t)T * dim;
  int blocks = (int)((n + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_moe_combine, dim3(blocks), dim3(256), 0, s, ys, weights, T, k, dim, Y);
  return hipGetLastError();
}

}  // namespace g4
