// g4_tok.hip -- multi-token Q4_K matmul on the gfx950 matrix cores.
//
// Y[m][r] = sum_c W[r][c] X[m][c] for M tokens (FloatTensor.matmul applied to M
// activation rows, FloatTensor.kt:18-29; Q4_K blocks of Q4_KFloatTensor.kt:23-55).
//
// Exactness.  The matrix cores multiply bf16 operands into fp32 sums, and both
// operands here are exact in bf16:
//   * weights: a Q4_K weight is d*sc*q - dmin*m with q in 0..15 per 32-weight
//     sub-block; q (or 16 q for the high nibbles) is an exact bf16 and the
//     sub-block's d*sc and dmin*m are applied in fp32 after the product, as
//     d*sc * sum(q x) - dmin*m * sum(x) (the row engine's factorisation);
//   * activations: an fp32 x has 24 significant bits and splits exactly into
//     x1 + x2 + x3, three round-to-nearest bf16 parts of 8 bits each, so three
//     MFMAs give sum(q x) with exact products and fp32 accumulation.
//
// Work split.  v_mfma_f32_16x16x32_bf16 with A = x parts (16 tokens x 32
// columns), B = weight nibbles (32 columns x 16 rows), C = 16 tokens x 16 rows:
// lane l holds A row l%16 / B column l%16 at columns 8(l/16)..+8, and C column
// l%16 (a weight row) at tokens 4(l/16)..+4, so the lane that unpacks weight row
// n also owns that row's outputs and scales.  A workgroup is 8 waves; in each
// column pass (2048 columns) wave w owns columns [256 w, 256 w + 256) and keeps
// that slice of x, split into bf16 parts, in registers while the workgroup
// walks its 16-row tiles.  The 8 per-wave partial tiles are summed in wave
// order through LDS (deterministic), then stored (later passes add to y).
#include "g4_device.hpp"
#include "g4_internal.hpp"

namespace g4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

constexpr int TOK_WAVES = 8;                   // column slices per workgroup
constexpr int TOK_GPW = 4;                     // 64-column groups per wave per pass
constexpr int TOK_PASS = TOK_WAVES * TOK_GPW;  // groups per pass (2048 columns)

// x = p1 + p2 + p3 exactly (each residual is exact in fp32; the third has at
// most 8 significant bits).  Infinite or NaN x stay in p1 with zero residuals.
G4_DEV void split3(const float (&v)[8], bf16x8 &p1, bf16x8 &p2, bf16x8 &p3) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 b1 = (__bf16)v[e];
    const float f1 = (float)b1;
    const float r1 = __builtin_isfinite(f1) ? v[e] - f1 : 0.f;
    const __bf16 b2 = (__bf16)r1;
    const float r2 = r1 - (float)b2;
    p1[e] = b1;
    p2[e] = b2;
    p3[e] = (__bf16)r2;
  }
}

// bf16 of the 8 nibble values of one K-slice: low nibbles give q, high nibbles
// (masked in place) give 16 q; both exact.
G4_DEV bf16x8 nibbles_bf16(uint32_t w0, uint32_t w1) {
  bf16x8 r;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    r[b] = (__bf16)ubyte(w0, b);
    r[4 + b] = (__bf16)ubyte(w1, b);
  }
  return r;
}

template <bool MULTI>
__global__ __launch_bounds__(512) void k_tok_q4k(TokArgs a) {
  __shared__ f32x4 red[2][TOK_WAVES][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, j = lane >> 4;
  const int tt = blockIdx.y;
  const int tok = tt * 16 + n;  // A row (token) of this lane
  const bool tok_ok = tok < a.M;
  const float *xt = a.x + (int64_t)(tok_ok ? tok : 0) * a.x_stride;
  const int C = a.dim1 >> 6;
  const int passes = MULTI ? (C + TOK_PASS - 1) / TOK_PASS : 1;
  const int n_rt = (a.rows + 15) >> 4;
  const int rpb = (n_rt + gridDim.x - 1) / gridDim.x;
  const int rt0 = min(n_rt, (int)blockIdx.x * rpb), rt1 = min(n_rt, rt0 + rpb);
  int buf = 0;

  for (int pass = 0; pass < passes; ++pass) {
    const int g0 = pass * TOK_PASS + wid * TOK_GPW;  // first group of this wave's slice
    const int ng = max(0, min(TOK_GPW, C - g0));     // wave-uniform

    // weight group gi of row tile rt, this lane's row (B column n) and K-slice j:
    // 8 nibble bytes at qs[32 g + 8 j] and the super-block head
    auto load_w = [&](int rt, bool live, u32x2a4 (&Q)[TOK_GPW], u32x4 (&H)[TOK_GPW], int (&gs)[TOK_GPW]) {
      const int r = rt * 16 + n;
      const bool rok = live && r < a.rows;
#pragma unroll
      for (int gi = 0; gi < TOK_GPW; ++gi) {
        // rows past the end and groups past the slice read the first group of
        // the tensor (in bounds; never stored / never multiplied)
        const int64_t e = (rok && gi < ng) ? a.base + (int64_t)r * a.row_stride + (int64_t)(g0 + gi) * 64 : 0;
        const int64_t G = e >> 6;
        const uint8_t *sb = a.W + (G >> 2) * 144;
        gs[gi] = (int)(G & 3);
        H[gi] = *(const u32x4 *)sb;
        Q[gi] = *(const u32x2a4 *)(sb + 16 + 32 * (G & 3) + 8 * j);
      }
    };

    // x slice: token tok, columns 64 g + 32 h + 8 j .. +8 for g in the slice
    u32x4a4 xr[TOK_GPW][2][2];
#pragma unroll
    for (int gi = 0; gi < TOK_GPW; ++gi)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int g = gi < ng ? g0 + gi : 0;
        const u32x4a4 *p = (const u32x4a4 *)(xt + (int64_t)g * 64 + 32 * h + 8 * j);
        xr[gi][h][0] = p[0];
        xr[gi][h][1] = p[1];
      }

    u32x2a4 QA[TOK_GPW], QB[TOK_GPW];
    u32x4 HA[TOK_GPW], HB[TOK_GPW];
    int GA[TOK_GPW], GB[TOK_GPW];
    // the first tile's weight loads go out behind the x loads and before any
    // use of x (vmcnt retires in order: the split below waits for x only)
    __builtin_amdgcn_sched_barrier(0);
    load_w(rt0, rt0 < rt1, QA, HA, GA);
    __builtin_amdgcn_sched_barrier(0);

    float xv[TOK_GPW][2][8];
#pragma unroll
    for (int gi = 0; gi < TOK_GPW; ++gi)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t m = opaque((tok_ok && gi < ng) ? ~0u : 0u);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          xv[gi][h][4 * u] = __uint_as_float(xr[gi][h][u].x & m);
          xv[gi][h][4 * u + 1] = __uint_as_float(xr[gi][h][u].y & m);
          xv[gi][h][4 * u + 2] = __uint_as_float(xr[gi][h][u].z & m);
          xv[gi][h][4 * u + 3] = __uint_as_float(xr[gi][h][u].w & m);
        }
      }

    // bf16 parts (A operands) and per-sub-block sums of x, the latter on the
    // matrix cores as parts x ones: the result lands in the C layout (token
    // 4 j + i of the tile, any column), fp32-accumulated like the products
    bf16x8 A[TOK_GPW][2][3];
    float xs[TOK_GPW][2][4];
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (__bf16)1.0f;
#pragma unroll
    for (int gi = 0; gi < TOK_GPW; ++gi)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        split3(xv[gi][h], A[gi][h][0], A[gi][h][1], A[gi][h][2]);
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < 3; ++p) s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[gi][h][p], ones, s, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[gi][h][i] = s[i];
      }

    auto tile = [&](int rt, const u32x2a4 (&Q)[TOK_GPW], const u32x4 (&H)[TOK_GPW], const int (&gs)[TOK_GPW]) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int gi = 0; gi < TOK_GPW; ++gi) {
        if (gi < ng) {  // wave-uniform
          const uint32_t w0 = Q[gi].x, w1 = Q[gi].y;
          const bf16x8 bl = nibbles_bf16(opaque(w0 & 0x0F0F0F0Fu), opaque(w1 & 0x0F0F0F0Fu));
          const bf16x8 bh = nibbles_bf16(opaque(w0 & 0xF0F0F0F0u), opaque(w1 & 0xF0F0F0F0u));
          // getScaleMinK4 (Q4_KFloatTensor.kt:70-84) for sub-blocks 2g, 2g+1 of
          // this lane's row: bytes 2(g&1), 2(g&1)+1 of the three scale dwords
          const int g = gs[gi];
          const uint32_t sh = (uint32_t)(g & 1) * 16u;
          const uint32_t y = H[gi].y >> sh, z = H[gi].z >> sh, w = H[gi].w >> sh;
          const uint32_t scp = g < 2 ? (y & 0x3F3Fu) : ((w & 0x0F0Fu) | ((y >> 2) & 0x3030u));
          const uint32_t mp = g < 2 ? (z & 0x3F3Fu) : (((w >> 4) & 0x0F0Fu) | ((z >> 2) & 0x3030u));
          const float d = h2f(H[gi].x & 0xFFFFu), dmin = h2f(H[gi].x >> 16);
          const float d1 = d * ubyte(scp, 0), d2 = d * ubyte(scp, 1) * 0.0625f;
          const float m1 = dmin * ubyte(mp, 0), m2 = dmin * ubyte(mp, 1);
          f32x4 pl = {0.f, 0.f, 0.f, 0.f}, ph = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int p = 0; p < 3; ++p) {
            pl = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[gi][0][p], bl, pl, 0, 0, 0);
            ph = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[gi][1][p], bh, ph, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = __builtin_fmaf(d1, pl[i], -(m1 * xs[gi][0][i]));
            acc[i] += __builtin_fmaf(d2, ph[i], __builtin_fmaf(-m2, xs[gi][1][i], v));
          }
        }
      }
      red[buf][wid][lane] = acc;
      __syncthreads();
      if (wid == 0) {
        f32x4 s = red[buf][0][lane];
#pragma unroll
        for (int w = 1; w < TOK_WAVES; ++w) s += red[buf][w][lane];
        const int r = rt * 16 + n;
        if (r < a.rows) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = tt * 16 + 4 * j + i;
            if (m < a.M) {
              float *yp = a.y + (int64_t)m * a.y_stride + r;
              float v = s[i];
              if constexpr (MULTI) {
                if (pass > 0) v += *yp;
              }
              *yp = v;
            }
          }
        }
      }
      buf ^= 1;
    };

    // two row tiles in flight: tile t+1 loads while tile t multiplies
    for (int rt = rt0; rt < rt1; rt += 2) {
      load_w(rt + 1, rt + 1 < rt1, QB, HB, GB);
      __builtin_amdgcn_sched_barrier(0);
      tile(rt, QA, HA, GA);
      __builtin_amdgcn_sched_barrier(0);
      load_w(rt + 2, rt + 2 < rt1, QA, HA, GA);
      __builtin_amdgcn_sched_barrier(0);
      if (rt + 1 < rt1) tile(rt + 1, QB, HB, GB);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

bool tok_ok(int type, const TokArgs &a) {
  if (type != T_Q4_K) return false;
  if (a.dim1 <= 0 || (a.dim1 % 64) != 0) return false;
  if ((a.base % 64) != 0 || (a.row_stride % 64) != 0) return false;
  return a.M >= 1 && a.rows >= 1;
}

hipError_t launch_tok(int type, const TokArgs &a, const DevInfo &dev, hipStream_t s) {
  if (!tok_ok(type, a)) return hipErrorInvalidValue;
  const int C = a.dim1 / 64;
  const bool multi = C > TOK_PASS;
  const int n_tt = (a.M + 15) / 16;
  const int n_rt = (a.rows + 15) / 16;
  // one 8-wave workgroup per CU at a time: spread the row tiles of every token
  // tile over cu / n_tt workgroups (each walks its tiles with one in flight)
  int64_t gx = (dev.cu_count + n_tt - 1) / n_tt;
  if (gx > n_rt) gx = n_rt;
  if (gx < 1) gx = 1;
  if (multi)
    hipLaunchKernelGGL(k_tok_q4k<true>, dim3((unsigned)gx, (unsigned)n_tt), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(k_tok_q4k<false>, dim3((unsigned)gx, (unsigned)n_tt), dim3(512), 0, s, a);
  return hipGetLastError();
}

}  // namespace g4
