// g4_kernels.hip -- gfx950 kernels of the quantized matrix-vector path.
//
// Row-stream matvec engine (k_rows): a wave owns a contiguous range of rows and
// keeps its 64-column slice of x in registers across them.  Lanes split each
// row into 64-element chunks (two Q8_0/Q4_0 blocks, one Q4_K/Q5_K group, a quarter
// Q6_K super-block), load them
// with dword-aligned 128-bit loads, unpack in registers and reduce the row
// partial sums across the lane group with a transposing butterfly.  x is staged
// once per workgroup in LDS (XOR-swizzled so the per-lane 256-byte reads are
// bank-conflict free).  Rows that do not start on a 64-element boundary go to
// k_rows_generic, a per-element restatement of the reference's get()-based dot.
//
// Reference paths are relative to lib/src/main/kotlin/io/github/lbenedetto/internal/.
#include <float.h>
#include <limits.h>

#include <atomic>

#include "../../include/g4hip.h"
#include "g4_device.hpp"
#include "g4_internal.hpp"

// Target tiles per wave of a row launch (one computing while the next is in flight).
#ifndef G4_TILES_PER_WAVE
#define G4_TILES_PER_WAVE 2
#endif

namespace g4 {

static_assert(NORM_WEIGHT_AFTER == G4_NORM_WEIGHT_AFTER && NORM_WEIGHT_FIRST == G4_NORM_WEIGHT_FIRST &&
                  NORM_NO_WEIGHT == G4_NORM_NO_WEIGHT,
              "norm forms of the C ABI");

// ------------------------------------------------------------ arg-max ----
// Cross-block (value, index) reduction in two launches.  Inside one launch a
// block-to-block handoff needs device-scope release/acquire fences, which on a
// multi-XCD part write back / invalidate the per-XCD L2 (the L2s do not snoop
// each other): measured at tens of microseconds for a few hundred blocks behind
// 1 MB of freshly written logits.  So each block stores its partial with a plain
// store and k_argmax_final (one block) reduces them after the kernel boundary.

// (value, index) of the block in thread 0 (all threads call, uniform control
// flow; blocks of up to 16 waves).
__device__ void am_block(float &v, int &i) {
  __shared__ float rv[16];
  __shared__ int ri[16];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, wpb = blockDim.x >> 6;
  am_wave(v, i);
  __syncthreads();
  if (lane == 0) rv[wid] = v, ri[wid] = i;
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < wpb; ++w)
      if (am_better(rv[w], ri[w], v, i)) v = rv[w], i = ri[w];
}

__device__ void am_partial(float v, int i, float *pv, int32_t *pi) {
  am_block(v, i);
  if (threadIdx.x == 0) pv[blockIdx.x] = v, pi[blockIdx.x] = i;
}

// One 256-thread block: best of n block partials -> *out.  The first 2048
// partials are loaded before any comparison (one round trip to memory).
__global__ __launch_bounds__(256) void k_argmax_final(const float *pv, const int32_t *pi, int n, int32_t *out) {
  constexpr int U = 8;
  float v = -__builtin_inff();
  int i = INT_MAX;
  float cv[U];
  int ci[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int b = threadIdx.x + 256 * u;
    cv[u] = pv[b < n ? b : 0];
    ci[u] = pi[b < n ? b : 0];
  }
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (threadIdx.x + 256 * u < n && am_better(cv[u], ci[u], v, i)) v = cv[u], i = ci[u];
  for (int b = threadIdx.x + 256 * U; b < n; b += 256)
    if (am_better(pv[b], pi[b], v, i)) v = pv[b], i = pi[b];
  am_block(v, i);
  if (threadIdx.x == 0) *out = i;
}

// ------------------------------------------------------------------ route ----
// Routing of one token by one 256-thread block: softmax of MutableFloatTensor.kt:54-59
// (max with java.lang.Math.max semantics, exp in double, fp32 sum in index order,
// fp32 divide), top-k of Llama.kt:275-293 (strict >, ties to the lowest index,
// chosen entries masked to -inf), optional renormalisation (fp32 sum in k
// order) and expert scale.  Used by k_route and by the routed gate+up launch.
constexpr int ROUTE_MAX_E = ROUTE_LAUNCH_MAX_E;  // k_route
constexpr int ROUTE_FUSED_MAX_E = 256;  // routing inside the gate+up launch
constexpr int ROUTE_FILTER_MAX_K = 32;  // top-k through the candidate filter up to this k

G4_DEV float java_max(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  if (a == 0.f && b == 0.f) return __builtin_signbit(a) ? b : a;
  return a >= b ? a : b;
}

template <int MAXE>
struct RouteLds {
  float p[MAXE];
  float es[MAXE];
  uint64_t key[MAXE];
  float pick_w[MAXE];
  int32_t pick_i[MAXE];
  float w_out[MAXE];
  uint32_t gmax[ROUTE_FILTER_MAX_K];
  int32_t n_cand;
  float wm[8];
};

// Leaves pick k's expert in r.pick_i[k] and its final weight in r.w_out[k],
// visible to every thread of the block on return (E <= MAXE, K <= E; every
// thread calls, uniform control flow).  Written for 256 threads; a 512-thread
// block may call it when E <= 256 (threads from 256 on then hold no logits and
// take no element in any loop).
template <int MAXE>
G4_DEV void route_token(const float *lg, int E, int K, int renorm, const float *expert_scale, RouteLds<MAXE> &r) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const bool filter = K >= 1 && K <= ROUTE_FILTER_MAX_K;
  if (tid < ROUTE_FILTER_MAX_K) r.gmax[tid] = 0u;
  if (tid == 0) r.n_cand = 0;
  // thread tid's logits (and expert scales) in registers, all loads issued at
  // once; lanes past E load element 0 and do not use it
  constexpr int PER = (MAXE + 255) / 256;
  float lv[PER], sv[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid + 256 * u;
    lv[u] = lg[i < E ? i : 0];
    sv[u] = expert_scale ? expert_scale[i < E ? i : 0] : 0.f;
  }
  // max with Math.max semantics (order-independent: NaN wins, +0 over -0)
  float m = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (tid + 256 * u < E) m = java_max(m, lv[u]);
  // over the wave without LDS (permlane swaps, then DPP; the half-row mirror at
  // distance 4 pairs lanes of the two halves of every 8, which serves a maximum)
  m = java_max(m, __uint_as_float(partner_u32<32>(__float_as_uint(m), lane)));
  m = java_max(m, __uint_as_float(partner_u32<16>(__float_as_uint(m), lane)));
  m = java_max(m, __uint_as_float(partner_u32<8>(__float_as_uint(m), lane)));
  m = java_max(m, __uint_as_float(partner_u32<4>(__float_as_uint(m), lane)));
  m = java_max(m, __uint_as_float(partner_u32<2>(__float_as_uint(m), lane)));
  m = java_max(m, __uint_as_float(partner_u32<1>(__float_as_uint(m), lane)));
  if (lane == 0) r.wm[wid] = m;
  __syncthreads();
  m = java_max(java_max(r.wm[0], r.wm[1]), java_max(r.wm[2], r.wm[3]));
  if (blockDim.x > 256) m = java_max(m, java_max(java_max(r.wm[4], r.wm[5]), java_max(r.wm[6], r.wm[7])));
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = tid + 256 * u;
    if (i < E) {
      r.p[i] = (float)exp((double)__fsub_rn(lv[u], m));
      r.es[i] = sv[u];
    }
  }
  __syncthreads();
  // fp32 sum in index order: every thread adds the same sequence (LDS broadcast
  // reads), so the sum needs no second barrier.  64 reads go out before their adds.
  float sum = 0.f;
  int i0 = 0;
  for (; i0 + 64 <= E; i0 += 64) {
    float v[64];
#pragma unroll
    for (int j = 0; j < 64; ++j) v[j] = r.p[i0 + j];
#pragma unroll
    for (int j = 0; j < 64; ++j) sum = __fadd_rn(sum, v[j]);
  }
  for (; i0 + 16 <= E; i0 += 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = r.p[i0 + j];
#pragma unroll
    for (int j = 0; j < 16; ++j) sum = __fadd_rn(sum, v[j]);
  }
  for (; i0 < E; ++i0) sum = __fadd_rn(sum, r.p[i0]);
  __syncthreads();
  bool nan = false;
  for (int i = tid; i < E; i += 256) {
    const float q = __fdiv_rn(r.p[i], sum);
    r.p[i] = q;
    nan |= q != q;
    // group maxima (group i % K) of the probability bits, for the candidate filter
    if (filter & (q == q)) atomicMax(&r.gmax[i % K], __float_as_uint(q));
  }
  // Top-k of Llama.kt:275-293 (K scans with strict >, the winner masked to -inf).
  // Without NaN every probability is finite and >= 0, and those scans pick the
  // elements in order of (larger value, then lower index): element i's rank is
  // the number of elements that beat it, computed by every thread for its own
  // elements at once.  (value, index) is one 64-bit key: the bits of p >= 0
  // order as an unsigned integer, and the low word ranks lower indices higher.
  // With a NaN present the scans themselves run (a NaN never wins; once nothing
  // beats -inf the scan keeps index 0).
  const bool any_nan = __syncthreads_or(nan);
  if (!any_nan && filter) {
    // The smallest of the K group maxima is at most the K-th largest probability
    // (K distinct elements reach it), so the top K are among the elements at or
    // above it, and every element that beats a candidate is a candidate too: a
    // candidate's rank among the candidates is its rank among all E.
    uint32_t t = 0xFFFFFFFFu;
    for (int g = 0; g < K; ++g) t = min(t, r.gmax[g]);
    for (int i = tid; i < E; i += 256) {
      const uint32_t b = __float_as_uint(r.p[i]);
      if (b >= t) r.key[atomicAdd(&r.n_cand, 1)] = ((uint64_t)b << 32) | (uint32_t)(~i);
    }
    __syncthreads();
    const int n = r.n_cand;
    for (int c = tid; c < n; c += 256) {
      const uint64_t kc = r.key[c];
      int r0 = 0, r1 = 0;
      int d = 0;
      for (; d + 8 <= n; d += 8) {
        uint64_t kk[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) kk[u] = r.key[d + u];
#pragma unroll
        for (int u = 0; u < 8; u += 2) {
          r0 += (int)(kk[u] > kc);
          r1 += (int)(kk[u + 1] > kc);
        }
      }
      for (; d < n; ++d) r0 += (int)(r.key[d] > kc);
      const int rank = r0 + r1;
      if (rank < K) r.pick_w[rank] = __uint_as_float((uint32_t)(kc >> 32)), r.pick_i[rank] = (int)~(uint32_t)kc;
    }
  } else if (!any_nan) {
    for (int i = tid; i < E; i += 256) r.key[i] = ((uint64_t)__float_as_uint(r.p[i]) << 32) | (uint32_t)(~i);
    __syncthreads();
    // element i's rank = number of keys above key[i]; `parts` threads share one
    // element's scan, four independent counters each
    int parts = 1;  // a power of two <= 64 with parts * E <= 256
    while (parts < 64 && 2 * parts * E <= 256) parts *= 2;
    const int part = tid % parts;
    for (int i = tid / parts; i < E; i += 256 / parts) {
      const uint64_t ki = r.key[i];
      int r0 = 0, r1 = 0, r2 = 0, r3 = 0;
      const int j0 = part * E / parts, j1 = (part + 1) * E / parts;
      int j = j0;
      // 16 keys per LDS round trip: their reads go out before the compares
      for (; j + 16 <= j1; j += 16) {
        uint64_t kk[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) kk[u] = r.key[j + u];
#pragma unroll
        for (int u = 0; u < 16; u += 4) {
          r0 += (int)(kk[u] > ki);
          r1 += (int)(kk[u + 1] > ki);
          r2 += (int)(kk[u + 2] > ki);
          r3 += (int)(kk[u + 3] > ki);
        }
      }
      for (; j < j1; ++j) r0 += (int)(r.key[j] > ki);
      int rank = (r0 + r1) + (r2 + r3);
      // the parts of one element are adjacent lanes of one wave (parts is a power
      // of two, wave-uniform): sums over 2, 4, 8, ... lanes, without LDS (at
      // distance 4 the half-row mirror pairs the two quads of every 8 lanes,
      // which after the steps at 1 and 2 gives the same sum as lane ^ 4)
      if (parts > 1) rank += (int)partner_u32<1>((uint32_t)rank, lane);
      if (parts > 2) rank += (int)partner_u32<2>((uint32_t)rank, lane);
      if (parts > 4) rank += (int)partner_u32<4>((uint32_t)rank, lane);
      if (parts > 8) rank += (int)partner_u32<8>((uint32_t)rank, lane);
      if (parts > 16) rank += (int)partner_u32<16>((uint32_t)rank, lane);
      if (parts > 32) rank += (int)partner_u32<32>((uint32_t)rank, lane);
      if (part == 0 && rank < K) r.pick_w[rank] = r.p[i], r.pick_i[rank] = i;
    }
  } else {
    for (int j = 0; j < K; ++j) {
      float bv = -__builtin_inff();
      int bi = INT_MAX;
      for (int i = tid; i < E; i += 256) {
        const float v = r.p[i] != r.p[i] ? -__builtin_inff() : r.p[i];
        if (am_better(v, i, bv, bi)) bv = v, bi = i;
      }
      am_block(bv, bi);  // thread 0 holds the winner
      if (tid == 0) {
        if (bv == -__builtin_inff()) bi = 0;
        r.pick_i[j] = bi;
        r.pick_w[j] = bv;
        r.p[bi] = -__builtin_inff();
      }
      __syncthreads();
    }
  }
  __syncthreads();
  // renormalisation sum in k order, the same in every thread
  float renorm_sum = 0.f;
  if (renorm)
    for (int j = 0; j < K; ++j) renorm_sum = __fadd_rn(renorm_sum, r.pick_w[j]);
  for (int j = tid; j < K; j += 256) {
    float w = r.pick_w[j];
    if (renorm) w = __fdiv_rn(w, renorm_sum);
    if (expert_scale) w = __fmul_rn(w, r.es[r.pick_i[j]]);
    r.w_out[j] = w;
  }
  __syncthreads();
}

// --------------------------------------------------------------- engine ----

template <class F, int LPR, int CPL, int EPI, bool MULTI, bool NORM, bool ROUTE = false, bool XL = false, int WPB = 4,
          bool SLOTW = false, bool KSEL = false>
__global__ __launch_bounds__(64 * WPB) void k_rows(RowsArgs a) {
  constexpr int NT = 64 * WPB;                   // threads per workgroup (WPB waves)
  constexpr int RT = F::RT / CPL > 0 ? F::RT / CPL : 1;  // row steps per tile (about F::RT chunk loads per lane)
  constexpr int RPW = 64 / LPR;                  // rows in flight per step (one per lane group)
  constexpr int TR = RT * RPW;                   // physical rows per tile
  constexpr int LRT = (EPI == EPI_GELU_PAIR) ? TR / 2 : TR;  // logical rows per tile
  constexpr int NDW = F::NDW;
  constexpr int NCH = LPR * CPL;                 // x chunks of one column pass
  constexpr int XSEG = (NCH * 16 + NT - 1) / NT;  // 16-byte x segments each thread stages
  constexpr bool XFULL = NCH * 16 % NT == 0;      // every thread's last segment is one of the pass's
  static_assert(RT >= 1, "tile");
  static_assert(EPI != EPI_GELU_PAIR || (RT >= 2 && CPL == 1), "paired tiles: gate and up steps, one pass");
  static_assert(XSEG >= 1 && (XFULL || (!NORM && !MULTI)), "x staging");
  static_assert(!(NORM && MULTI), "the fused norm needs all of x in one pass");
  static_assert(!NORM || WPB == 4, "the fused norm uses the 256-thread element map of k_rmsnorm");
  static_assert(WPB == 4 || WPB == 8, "workgroup of 4 or 8 waves");
  static_assert(!ROUTE || (EPI == EPI_GELU_PAIR && !MULTI && !NORM), "routing: gate+up launches");
  // XL: each chunk's x is read from LDS when its weights are dotted instead of
  // living in VGPRs for the whole launch, so a lane can take CPL = 3 chunks
  // (rows of 17..24 chunks, e.g. 1408 columns, keep 22 of 24 lanes busy rather
  // than 22 of 32); the block sums of x are computed once into LDS
  static_assert(!XL || (EPI == EPI_STORE && !MULTI && !NORM && !ROUTE), "x at use: plain single-pass launches");
  // SLOTW (MoE gate+up of several tokens): workgroup (row block, token), wave j
  // takes slot j's expert over the block's rows; the token's x is staged and
  // routed once for its K <= 8 slots, and a row block's workgroups of every
  // token run side by side (with a grid x extent that is a multiple of 8, on one
  // XCD), so tokens that share an expert read its rows through one L2
  static_assert(!SLOTW || (EPI == EPI_GELU_PAIR && !MULTI && !NORM && !XL && WPB == 8), "slot per wave: gate+up");
  // KSEL (Q4_K with every base and stride on whole super-blocks): chunk c of
  // any row is group c & 3 of its super-block, and every chunk a lane takes has
  // c = q (mod 4), so the lane's scale selector is formed once
  static_assert(!KSEL || (F::TYPE == T_Q4_K && LPR % 4 == 0), "KSEL: Q4_K rows");
  constexpr int NSX = F::NS > 0 ? F::NS : 1;
  // x layout in LDS (16-byte slots): chunk ch's segment i sits at slot
  // ch * 16 + (i ^ (ch & 15)) -- the 8 lanes one LDS cycle serves read 8
  // different bank groups; with XL at ch * 17 + i instead (the same spread, and
  // the 16 reads of a chunk share one address register and immediate offsets)
  constexpr int XCS = XL ? 17 : 16;
  auto xslot = [](int ch, int i) { return XL ? ch * 17 + i : ch * 16 + (i ^ (ch & 15)); };
  __shared__ u32x4 xl[NCH * XCS];
  __shared__ float xsl[XL ? NCH : 1][NSX];
  __shared__ float red[4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: tile loop control stays scalar
  constexpr int wpb = WPB;
  const int gi = lane / LPR, q = lane % LPR;
  const FmtQ4_K::Sel ksel = FmtQ4_K::select(q & 3);  // KSEL
  const int seg = blockIdx.y;
  const int C = a.dim1 >> 6;
  const float *x = a.x + (int64_t)(SLOTW ? seg : seg / a.x_div) * a.x_stride;
  // x of a column pass, staged once per workgroup: each thread fetches XSEG
  // 16-byte segments (coalesced); with the fused norm also the norm weights
  u32x4a4 xr[XSEG];
  u32x4a4 wr[NORM ? XSEG : 1];
  auto load_x = [&](int pass) {
#pragma unroll
    for (int j = 0; j < XSEG; ++j) {
      const int s = j * NT + tid, c = pass * NCH + (s >> 4);
      // dword alignment is all a caller's x guarantees; gfx950 takes 128-bit loads at that alignment
      xr[j] = ((const u32x4a4 *)(x + (int64_t)(c < C ? c : 0) * 64))[s & 15];
      if constexpr (NORM) wr[j] = ((const u32x4a4 *)(a.norm_w + (int64_t)(c < C ? c : 0) * 64))[s & 15];
    }
  };
  // the routed launch has one column pass: its x is in flight while the token is routed
  if constexpr (ROUTE) load_x(0);
  int expert = 0;
  if constexpr (ROUTE) {
    // the token's routing, computed by every workgroup of its segments (the
    // logits are 4 bytes per expert; a separate launch would cost more)
    __shared__ RouteLds<ROUTE_FUSED_MAX_E> rl;
    const int tok = SLOTW ? seg : seg / a.x_div, slot = SLOTW ? min(wid, a.x_div - 1) : seg % a.x_div;
    route_token(a.route_logits + (int64_t)tok * a.route_e, a.route_e, a.x_div, a.route_renorm, a.route_scale, rl);
    expert = __builtin_amdgcn_readfirstlane(rl.pick_i[slot]);
    if constexpr (SLOTW) {
      if (blockIdx.x == 0 && lane == 0 && wid < a.x_div)
        a.route_ids[tok * a.x_div + wid] = expert, a.route_w[tok * a.x_div + wid] = rl.w_out[wid];
    } else {
      if (blockIdx.x == 0 && tid == 0) a.route_ids[seg] = expert, a.route_w[seg] = rl.w_out[slot];
    }
  } else if (a.ids) {
    expert = a.ids[SLOTW ? seg * a.x_div + min(wid, a.x_div - 1) : seg];
  }
  const bool bad_expert = (ROUTE || a.ids) && (expert < 0 || expert >= a.expert_count);
  const int64_t ebase = bad_expert ? 0 : (int64_t)expert * a.expert_stride;
  float *y = a.y ? a.y + (int64_t)(SLOTW ? seg * a.x_div + wid : seg) * a.y_stride : nullptr;

  const int n_tiles = (a.rows + LRT - 1) / LRT;
  // wave wid of block b is virtual wave wid * blocks + b: when there are fewer
  // tiles than waves, every workgroup (so every CU) still gets some.  SLOTW:
  // every wave of block b takes block b's tiles (for its own slot); waves past
  // the token's K slots take none
  const int nwv = SLOTW ? gridDim.x : gridDim.x * wpb, wv = SLOTW ? blockIdx.x : wid * gridDim.x + blockIdx.x;
  const int tpw = (n_tiles + nwv - 1) / nwv;
  const int t0 = min(n_tiles, wv * tpw), t1 = SLOTW && wid >= a.x_div ? t0 : min(n_tiles, t0 + tpw);
  const int passes = MULTI ? (C + LPR * CPL - 1) / (LPR * CPL) : 1;

  // row (logical index, matrix, base) of tile t, step k for this lane's group
  auto row_of = [&](int t, int k, int &lr, const uint8_t *&W, int64_t &base) {
    if constexpr (EPI == EPI_GELU_PAIR) {
      lr = t * LRT + (k % (RT / 2)) * RPW + gi;
      W = k < RT / 2 ? a.W0 : a.W1;
      base = k < RT / 2 ? a.base0 : a.base1;
    } else {
      lr = t * LRT + k * RPW + gi;
      W = a.W0;
      base = a.base0;
    }
  };

  // `live` false: a prefetch past the wave's last tile (issued anyway so every
  // path through the loop has the same number of loads in flight).
  // SADDR (KSEL with a slot per wave, a launch bound by vector-ALU issue): a
  // chunk's bytes sit at a wave-uniform row address (the step's first row) plus
  // a lane offset fixed for the launch (its row in the step, its super-block),
  // so a tile's addresses cost scalar arithmetic and one select per chunk
  constexpr bool SADDR = KSEL && SLOTW;
  const int64_t rbytes = (a.row_stride >> 8) * 144;  // SADDR: bytes per row
  uint32_t lane_off[CPL];
#pragma unroll
  for (int u = 0; u < CPL; ++u) lane_off[u] = (uint32_t)(gi * rbytes + ((u * LPR + q) >> 2) * 144);
  const uint32_t q_off = 16u + 32u * (uint32_t)(q & 3);
  auto load_tile = [&](int t, int pass, bool live, uint32_t (&D)[RT][CPL][NDW], bool (&ok)[RT][CPL],
                       int64_t (&E)[RT][CPL]) {
#pragma unroll
    for (int k = 0; k < RT; ++k) {
      int lr;
      const uint8_t *W;
      int64_t base;
      row_of(t, k, lr, W, base);
      if constexpr (SADDR) {
        // the step's first row (uniform); past the last row or tile: the matrix's first row
        const int lr0 = lr - gi;
        const bool in = live && lr0 < a.rows;
        const uint8_t *wrow = W + ((base + ebase) >> 8) * 144 + (in ? (int64_t)lr0 * rbytes : 0);
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
          const int c = (pass * CPL + u) * LPR + q;
          ok[k][u] = live && c < C && lr < a.rows && !bad_expert;
          // a masked chunk reads the row's first super-block
          const uint32_t o = ok[k][u] ? lane_off[u] : 0u;
          const u32x4 h = *(const u32x4 *)(wrow + o);
          const u32x4 *qs = (const u32x4 *)(wrow + (o + q_off));
          const u32x4 q0 = qs[0], q1 = qs[1];
          uint32_t(&Du)[NDW] = D[k][u];
          Du[0] = q0.x; Du[1] = q0.y; Du[2] = q0.z; Du[3] = q0.w;
          Du[4] = q1.x; Du[5] = q1.y; Du[6] = q1.z; Du[7] = q1.w;
          Du[8] = h.x; Du[9] = h.y; Du[10] = h.z; Du[11] = h.w;
        }
        continue;
      }
#pragma unroll
      for (int u = 0; u < CPL; ++u) {
        const int c = (pass * CPL + u) * LPR + q;
        ok[k][u] = live && c < C && lr < a.rows && !bad_expert;
        E[k][u] = base + ebase + (int64_t)lr * a.row_stride + (int64_t)c * 64;
        // Unconditional load (lanes past the row or the tile read the tensor's first
        // chunk, always in bounds, and their result is masked): no branch around a
        // load, so the compiler can count outstanding loads and wait for this tile only.
        F::load(W, ok[k][u] ? E[k][u] : 0, D[k][u]);
      }
    }
  };

  float best_v = -__builtin_inff();
  int best_i = INT_MAX;

  // EPI_GELU_PAIR: the (gate, up) pair of each finished row waits in a per-wave
  // LDS queue, and gelu (in double, like the reference) runs once per 64 rows
  // with every lane busy rather than once per tile with one lane per row.  The
  // queued rows are contiguous because a wave finishes its tiles in order.
  __shared__ float2 gq[EPI == EPI_GELU_PAIR ? WPB : 1][64];
  int gq_n = 0, gq_row = t0 * LRT;
  auto gq_flush = [&]() {
    if (lane < gq_n) {
      const float2 p = gq[EPI == EPI_GELU_PAIR ? wid : 0][lane];
      const int lr = gq_row + lane;
      if (lr < a.rows) y[lr] = gelu_ref(p.x) * p.y;
    }
    gq_row += gq_n;
    gq_n = 0;
  };

  // EPI_ARGMAX (one column pass): the same kind of queue for the logits, so the
  // soft-cap's double tanh, the store and the arg-max update run once per 64
  // rows with every lane busy (coalesced stores), not once per tile.
  constexpr bool AQ = EPI == EPI_ARGMAX && !MULTI;
  __shared__ float aq[AQ ? WPB : 1][64];
  int aq_n = 0, aq_row = t0 * LRT;
  auto aq_flush = [&]() {
    if (lane < aq_n) {
      const int lr = aq_row + lane;
      float val = aq[AQ ? wid : 0][lane];
      if (a.softcap > 0.f) val = softcap_ref(val, a.softcap);
      if (lr < a.rows) {
        if (y) y[lr] = val;
        const float key = am_key(val, lr);
        if (am_better(key, lr, best_v, best_i)) best_v = key, best_i = lr;
      }
    }
    aq_row += aq_n;
    aq_n = 0;
  };

  auto read_x = [&](int ch, float (&xu)[64]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u32x4 t = xl[xslot(ch, i)];
      xu[4 * i] = __uint_as_float(t.x);
      xu[4 * i + 1] = __uint_as_float(t.y);
      xu[4 * i + 2] = __uint_as_float(t.z);
      xu[4 * i + 3] = __uint_as_float(t.w);
    }
  };
  constexpr int CX = XL ? 1 : CPL;  // chunks of x held in VGPRs
  auto finish_tile = [&](int t, int pass, const uint32_t (&D)[RT][CPL][NDW], const bool (&ok)[RT][CPL],
                         const int64_t (&E)[RT][CPL], const float (&xv)[CX][64], const float (&xs)[CX][NSX]) {
    float v[RT];
#pragma unroll
    for (int k = 0; k < RT; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < CPL; ++u) {
        float r;
        if constexpr (XL) {
          float xu[64], su[NSX];
          // an opaque chunk index: the reads are the same for every tile, and
          // hoisting them out of the tile loop would hold every chunk's x in VGPRs
          const int ch = (int)opaque((uint32_t)(u * LPR + q));
          read_x(ch, xu);
#pragma unroll
          for (int j = 0; j < NSX; ++j) su[j] = xsl[ch][j];
          if constexpr (KSEL) r = FmtQ4_K::dot_sel(D[k][u], xu, su, ksel);
          else r = F::dot(D[k][u], xu, su, E[k][u]);
          // one chunk's x in VGPRs at a time: this chunk's dot is done before
          // the next chunk's LDS reads are issued
          asm volatile("" : "+v"(r)::"memory");
        } else if constexpr (KSEL) {
          r = FmtQ4_K::dot_sel(D[k][u], xv[u], xs[u], ksel);
        } else {
          r = F::dot(D[k][u], xv[u], xs[u], E[k][u]);
        }
        acc += ok[k][u] ? r : 0.f;
      }
      v[k] = acc;
    }
    const float r = reduce_transpose<RT, LPR>(v, lane);
    const int k = q / (LPR / RT);
    const bool writer = (q % (LPR / RT)) == 0;
    if constexpr (EPI == EPI_GELU_PAIR) {
      // the up row's value from lane ^ LPR/2: a permlane swap or DPP for 32, 16
      // and 8 (exact xor partners), an LDS shuffle below
      float up;
      if constexpr (LPR / 2 == 32 || LPR / 2 == 16 || LPR / 2 == 8)
        up = __uint_as_float(partner_u32<LPR / 2>(__float_as_uint(r), lane));
      else
        up = __shfl_xor(r, LPR / 2, 64);
      if (writer && k < RT / 2) gq[wid][gq_n + (k % (RT / 2)) * RPW + gi] = make_float2(r, up);
      gq_n += LRT;
      if (gq_n + LRT > 64) gq_flush();
    } else if constexpr (AQ) {
      if (writer) aq[wid][aq_n + k * RPW + gi] = r;
      aq_n += LRT;
      if (aq_n + LRT > 64) aq_flush();
    } else {
      const int lr = t * LRT + k * RPW + gi;
      if (writer && lr < a.rows) {
        float val = r;
        // only the multi-pass kernels read back (a load here would make every
        // single-pass tile wait for the prefetched one: vmcnt retires in order)
        if constexpr (MULTI) {
          if (y && pass > 0) val += y[lr];
        }
        if constexpr (EPI == EPI_ARGMAX) {
          if (!MULTI || pass == passes - 1) {
            if (a.softcap > 0.f) val = softcap_ref(val, a.softcap);
            const float key = am_key(val, lr);
            if (am_better(key, lr, best_v, best_i)) best_v = key, best_i = lr;
          }
        }
        if (y) y[lr] = val;
      }
    }
  };

  for (int pass = 0; pass < passes; ++pass) {
    uint32_t DA[RT][CPL][NDW], DB[RT][CPL][NDW];
    bool okA[RT][CPL], okB[RT][CPL];
    int64_t EA[RT][CPL], EB[RT][CPL];
    // x of this pass goes out first, then the first weight tile, and only then
    // does the thread wait for x (vmcnt retires in issue order, so that wait
    // never covers the weight latency; the barrier waits on LDS only)
    if (!ROUTE) load_x(pass);
    load_tile(t0, pass, t0 < t1, DA, okA, EA);
    if (MULTI && pass > 0) __syncthreads();  // every wave has read the previous pass's x
    if constexpr (NORM) {
      // Llama.kt:27-37 on the staged x: thread tid holds 16-byte segments
      // tid + 256 j (elements 4s..4s+3), the element map of k_rmsnorm, so the
      // scale is bit-identical to the standalone norm's
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < XSEG; ++j) {
        const int s = j * 256 + tid, c = s >> 4;
        const uint32_t m = opaque(c < C ? ~0u : 0u);
        xr[j] = u32x4a4{xr[j].x & m, xr[j].y & m, xr[j].z & m, xr[j].w & m};
        acc = sq_acc(acc, __uint_as_float(xr[j].x));
        acc = sq_acc(acc, __uint_as_float(xr[j].y));
        acc = sq_acc(acc, __uint_as_float(xr[j].z));
        acc = sq_acc(acc, __uint_as_float(xr[j].w));
      }
      const float sc = rms_scale(block_sum256(acc, red), a.dim1, a.norm_eps);
      const bool keep = a.norm_out && blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
      for (int j = 0; j < XSEG; ++j) {
        const int s = j * 256 + tid, c = s >> 4;
        xr[j].x = __float_as_uint(norm_apply(NORM_WEIGHT_AFTER, __uint_as_float(wr[j].x), sc, __uint_as_float(xr[j].x)));
        xr[j].y = __float_as_uint(norm_apply(NORM_WEIGHT_AFTER, __uint_as_float(wr[j].y), sc, __uint_as_float(xr[j].y)));
        xr[j].z = __float_as_uint(norm_apply(NORM_WEIGHT_AFTER, __uint_as_float(wr[j].z), sc, __uint_as_float(xr[j].z)));
        xr[j].w = __float_as_uint(norm_apply(NORM_WEIGHT_AFTER, __uint_as_float(wr[j].w), sc, __uint_as_float(xr[j].w)));
        if (keep && c < C) ((u32x4a4 *)(a.norm_out + (int64_t)c * 64))[s & 15] = xr[j];
      }
    }
#pragma unroll
    for (int j = 0; j < XSEG; ++j) {
      const int s = j * NT + tid, ch = s >> 4, c = pass * NCH + ch;
      // zeroed by a mask, not a select: a select lets the compiler sink the
      // load into a branch, whose wait would then cover the weight loads too
      const uint32_t m = opaque(c < C ? ~0u : 0u);
      if (XFULL || ch < NCH) xl[xslot(ch, s & 15)] = u32x4{xr[j].x & m, xr[j].y & m, xr[j].z & m, xr[j].w & m};
    }
    __syncthreads();
    float xv[CX][64];
    float xs[CX][NSX];
    if constexpr (XL) {
      if constexpr (F::NS > 0) {
        // one thread per chunk (NCH <= 256) sums its blocks once for the workgroup
        if (tid < NCH) {
          float xu[64], su[NSX];
          read_x(tid, xu);
          F::sums(xu, su);
#pragma unroll
          for (int j = 0; j < NSX; ++j) xsl[tid][j] = su[j];
        }
        __syncthreads();
      }
    } else {
#pragma unroll
      for (int u = 0; u < CPL; ++u) read_x(u * LPR + q, xv[u]);
#pragma unroll
      for (int u = 0; u < CPL; ++u) F::sums(xv[u], xs[u]);
    }

    // software pipeline: tile t+1 is in flight while tile t is unpacked and
    // reduced (only the first tile goes out with x: issuing the second one too
    // delays every wave's first tile behind the others' second, measured
    // slower).  The scheduling barriers keep the compiler from sinking the next
    // tile's loads into the current tile's arithmetic.
    for (int t = t0; t < t1; t += 2) {
      load_tile(t + 1, pass, t + 1 < t1, DB, okB, EB);
      __builtin_amdgcn_sched_barrier(0);
      finish_tile(t, pass, DA, okA, EA, xv, xs);
      __builtin_amdgcn_sched_barrier(0);
      load_tile(t + 2, pass, t + 2 < t1, DA, okA, EA);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < t1) finish_tile(t + 1, pass, DB, okB, EB, xv, xs);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if constexpr (SLOTW) {
    gq_flush();  // every wave writes its own slot's rows
  } else if constexpr (EPI == EPI_GELU_PAIR) {
    // The rows still queued when the tiles run out: when the four waves' rows
    // fit in 64 lanes, one wave evaluates them all (one double-precision gelu
    // pass per workgroup instead of one per wave at the kernel's tail).
    __shared__ int gq_meta[WPB][2];
    if (lane == 0) gq_meta[wid][0] = gq_n, gq_meta[wid][1] = gq_row;
    __syncthreads();
    int tot = 0;
#pragma unroll
    for (int w = 0; w < WPB; ++w) tot += gq_meta[w][0];
    if (tot <= 64) {
      if (wid == 0 && lane < tot) {
        int w = 0, k = lane;
        while (k >= gq_meta[w][0]) k -= gq_meta[w][0], ++w;
        const float2 p = gq[w][k];
        const int lr = gq_meta[w][1] + k;
        if (lr < a.rows) y[lr] = gelu_ref(p.x) * p.y;
      }
    } else {
      gq_flush();
    }
  }
  if constexpr (AQ) aq_flush();
  if constexpr (EPI == EPI_ARGMAX) am_partial(best_v, best_i, a.am_val, a.am_idx);
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

// k_gelu_mul for rows in fours (16-byte aligned): workgroup (row block, segment),
// four rows per thread, no index division
__global__ __launch_bounds__(256) void k_gelu_mul4(const float *gu, int32_t rows, float *h, int64_t h_stride) {
  const int r = (blockIdx.x * 256 + threadIdx.x) * 4, sg = blockIdx.y;
  if (r >= rows) return;
  const float4 g = *(const float4 *)(gu + (int64_t)sg * 2 * rows + r);
  const float4 u = *(const float4 *)(gu + (int64_t)sg * 2 * rows + rows + r);
  float4 o;
  o.x = gelu_ref(g.x) * u.x;
  o.y = gelu_ref(g.y) * u.y;
  o.z = gelu_ref(g.z) * u.z;
  o.w = gelu_ref(g.w) * u.w;
  *(float4 *)(h + (int64_t)sg * h_stride + r) = o;
}

hipError_t launch_gelu_mul(const float *gu, int32_t rows, int32_t segments, float *h, int64_t h_stride,
                           hipStream_t s) {
  if (rows > 0 && segments > 0 && segments <= 65535 && rows % 4 == 0 && h_stride % 4 == 0 &&
      ((uintptr_t)gu & 15) == 0 && ((uintptr_t)h & 15) == 0) {
    hipLaunchKernelGGL(k_gelu_mul4, dim3((unsigned)((rows / 4 + 255) / 256), (unsigned)segments), dim3(256), 0, s,
                       gu, rows, h, h_stride);
    return hipGetLastError();
  }
  const int64_t n = (int64_t)rows * segments;
  int blocks = (int)((n + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) return hipSuccess;
  hipLaunchKernelGGL(k_gelu_mul, dim3(blocks), dim3(256), 0, s, gu, rows, segments, h, h_stride);
  return hipGetLastError();
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
__global__ __launch_bounds__(256) void k_argmax(const float *v, int32_t n, float *part_val, int32_t *part_idx) {
  float bv = -__builtin_inff();
  int bi = INT_MAX;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const float k = am_key(v[i], i);
    if (am_better(k, i, bv, bi)) bv = k, bi = i;
  }
  am_partial(bv, bi, part_val, part_idx);
}

// ------------------------------------------------------------------ route ----
// One 256-thread block per token (route_token).
__global__ __launch_bounds__(256) void k_route(const float *logits, int32_t E, int32_t K, int32_t renorm,
                                               const float *expert_scale, int32_t *ids, float *weights) {
  __shared__ RouteLds<ROUTE_MAX_E> r;
  const int t = blockIdx.x;
  route_token(logits + (int64_t)t * E, E, K, renorm, expert_scale, r);
  for (int j = threadIdx.x; j < K; j += 256) {
    ids[(int64_t)t * K + j] = r.pick_i[j];
    weights[(int64_t)t * K + j] = r.w_out[j];
  }
}

// ------------------------------------------------------- MoE down + sum ----
// Down projection and weighted sum of the routed experts in one launch
// (Llama.kt:300-337: the down matmul of each slot, then saxpyInPlace in slot
// order), for few tokens.  Workgroup (b, t) owns rows b*TR .. b*TR+TR-1 of token
// t; wave w computes those rows for slots w and w + 4 (expert ids[t*K + j], x =
// the h of slot t*K + j; every slot's h is staged once per workgroup).  The K
// row values wait in LDS and are summed in slot order, out = w_j * y_j + out
// (each product and sum rounded once, as k_moe_combine does), so Y is
// bit-identical to the down launch followed by k_moe_combine.  One column pass:
// dim1 <= 64 * LPR.
constexpr int MOE_DOWN_MAX_K = 8;

// WPB waves: wave w takes slots w and w + WPB (WPB = 4: two slots; WPB = 8: one)
// over RT = F::RT * WPB / 4 row steps, so a wave always holds 2 * F::RT chunks
// in flight and the 8-wave shape covers twice the rows per workgroup: every
// workgroup stages all K slots' x, so rows per workgroup set the x traffic.
template <class F, int LPR, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_moe_down(RowsArgs a, const float *gw, int32_t K) {
  static_assert(WPB == 4 || WPB == 8, "4 or 8 waves");
  constexpr int NT = 64 * WPB;
  constexpr int RT = F::RT * WPB / 4, RPW = 64 / LPR, TR = RT * RPW, NDW = F::NDW;
  constexpr int XS = LPR * 16;                          // 16-byte x segments of one slot
  constexpr int XSEG = MOE_DOWN_MAX_K * XS / NT;        // staged by each thread
  static_assert(XSEG * NT == MOE_DOWN_MAX_K * XS, "x staging");
  __shared__ u32x4 xl[MOE_DOWN_MAX_K][XS];
  __shared__ float cb[MOE_DOWN_MAX_K][TR];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = lane / LPR, q = lane % LPR;
  const int tok = blockIdx.y;
  const int C = a.dim1 >> 6;
  const int row0 = blockIdx.x * TR;

  // every slot's x segments, masked past K and past the row (loads never branch)
  u32x4a4 xr[XSEG];
#pragma unroll
  for (int u = 0; u < XSEG; ++u) {
    const int g = u * NT + tid, j = g / XS, c = (g % XS) >> 4;
    const bool in = (j < K) & (c < C);
    const float *xp = a.x + (int64_t)(tok * K + (in ? j : 0)) * a.x_stride + (int64_t)(in ? c : 0) * 64;
    xr[u] = ((const u32x4a4 *)xp)[g & 15];
  }
  float w_slot[MOE_DOWN_MAX_K];
  if (tid < TR) {
#pragma unroll
    for (int j = 0; j < MOE_DOWN_MAX_K; ++j) w_slot[j] = gw[tok * K + (j < K ? j : 0)];
  }

  // slot j's rows (slots past K load the tensor's first chunk, masked)
  auto load = [&](int j, uint32_t (&D)[RT][NDW], bool (&ok)[RT], int64_t (&E)[RT]) {
    const int expert = a.ids[tok * K + (j < K ? j : 0)];
    const bool bad = (j >= K) | (expert < 0) | (expert >= a.expert_count);
    const int64_t ebase = bad ? 0 : (int64_t)expert * a.expert_stride;
#pragma unroll
    for (int k = 0; k < RT; ++k) {
      const int lr = row0 + k * RPW + gi;
      ok[k] = !bad && q < C && lr < a.rows;
      E[k] = a.base0 + ebase + (int64_t)lr * a.row_stride + (int64_t)q * 64;
      F::load(a.W0, ok[k] ? E[k] : 0, D[k]);
    }
  };
  auto finish = [&](int j, const uint32_t (&D)[RT][NDW], const bool (&ok)[RT], const int64_t (&E)[RT]) {
    float xv[64];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u32x4 t = xl[j][q * 16 + (i ^ (q & 15))];
      xv[4 * i] = __uint_as_float(t.x);
      xv[4 * i + 1] = __uint_as_float(t.y);
      xv[4 * i + 2] = __uint_as_float(t.z);
      xv[4 * i + 3] = __uint_as_float(t.w);
    }
    float xs[F::NS > 0 ? F::NS : 1];
    F::sums(xv, xs);
    float v[RT];
#pragma unroll
    for (int k = 0; k < RT; ++k) {
      const float r = F::dot(D[k], xv, xs, E[k]);
      float acc = 0.f;  // the row engine's one-pass accumulation, bit for bit
      acc += ok[k] ? r : 0.f;
      v[k] = acc;
    }
    const float r = reduce_transpose<RT, LPR>(v, lane);
    const int k = q / (LPR / RT);
    if ((q % (LPR / RT)) == 0) cb[j][k * RPW + gi] = r;
  };

  uint32_t DA[RT][NDW], DB[RT][NDW];
  bool okA[RT], okB[RT];
  int64_t EA[RT], EB[RT];
  // both slots' weights go out before the x staging waits (one token's step:
  // 21.6 -> 21.3 us against issuing the second slot after the barrier)
  load(wid, DA, okA, EA);
  if constexpr (WPB == 4) load(wid + 4, DB, okB, EB);
#pragma unroll
  for (int u = 0; u < XSEG; ++u) {
    const int g = u * NT + tid, j = g / XS, c = (g % XS) >> 4;
    const uint32_t m = opaque(((j < K) & (c < C)) ? ~0u : 0u);
    xl[j][c * 16 + ((g & 15) ^ (c & 15))] = u32x4{xr[u].x & m, xr[u].y & m, xr[u].z & m, xr[u].w & m};
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  if (wid < K) finish(wid, DA, okA, EA);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (WPB == 4) {
    if (wid + 4 < K) finish(wid + 4, DB, okB, EB);
  }
  __syncthreads();
  if (tid < TR && row0 + tid < a.rows) {
    float out = 0.f;
    for (int j = 0; j < K; ++j) out = rounded(w_slot[j] * cb[j][tid]) + out;
    a.y[(int64_t)tok * a.y_stride + row0 + tid] = out;
  }
}

// The same in the 8-wave shape for rows of 17..24 chunks (the MoE's 1408-column
// down rows are 22): 8 lanes x 3 chunks per row, so 22 of 24 lanes work against
// 22 of 32 with one chunk per lane, one row step of 8 rows per wave and slot.
// Each chunk's x is read from LDS right before its dot and the Q-format block
// sums of x are formed once per (slot, chunk), as k_rows' x-read-at-use form
// does: every dot has the bits of the per-pair XL launch, and the k row values
// are summed in slot order as k_moe_combine does.
template <class F>
__global__ __launch_bounds__(512) void k_moe_down_xl(RowsArgs a, const float *gw, int32_t K) {
  constexpr int NT = 512, LPR = 8, CPL = 3, NCH = LPR * CPL, RPW = 64 / LPR, TR = RPW, NDW = F::NDW;
  constexpr int NSX = F::NS > 0 ? F::NS : 1;
  constexpr int XS = NCH * 16;                    // 16-byte x segments of one slot
  constexpr int XSEG = MOE_DOWN_MAX_K * XS / NT;  // staged by each thread
  static_assert(XSEG * NT == MOE_DOWN_MAX_K * XS, "x staging");
  static_assert(MOE_DOWN_MAX_K * NCH <= NT, "one thread per (slot, chunk) for the block sums");
  // chunk ch's segment i at slot ch * 17 + i (a chunk's 16 reads share one
  // address; the 8 chunks one LDS cycle serves land in different bank groups)
  __shared__ u32x4 xl[MOE_DOWN_MAX_K][NCH * 17];
  __shared__ float xsl[MOE_DOWN_MAX_K][NCH][NSX];
  __shared__ float cb[MOE_DOWN_MAX_K][TR];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = lane / LPR, q = lane % LPR;
  const int tok = blockIdx.y;
  const int C = a.dim1 >> 6;
  const int row0 = blockIdx.x * TR;

  // every slot's x segments, masked past K and past the row (loads never branch)
  u32x4a4 xr[XSEG];
#pragma unroll
  for (int u = 0; u < XSEG; ++u) {
    const int g = u * NT + tid, j = g / XS, c = (g % XS) >> 4;
    const bool in = (j < K) & (c < C);
    const float *xp = a.x + (int64_t)(tok * K + (in ? j : 0)) * a.x_stride + (int64_t)(in ? c : 0) * 64;
    xr[u] = ((const u32x4a4 *)xp)[g & 15];
  }
  float w_slot[MOE_DOWN_MAX_K];
  if (tid < TR) {
#pragma unroll
    for (int j = 0; j < MOE_DOWN_MAX_K; ++j) w_slot[j] = gw[tok * K + (j < K ? j : 0)];
  }
  // wave wid's slot: its row step's weights (a slot past K loads the tensor's
  // first chunk, masked)
  uint32_t D[CPL][NDW];
  bool ok[CPL];
  int64_t E[CPL];
  {
    const int j = wid;
    const int expert = a.ids[tok * K + (j < K ? j : 0)];
    const bool bad = (j >= K) | (expert < 0) | (expert >= a.expert_count);
    const int64_t ebase = bad ? 0 : (int64_t)expert * a.expert_stride;
    const int lr = row0 + gi;
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      const int c = u * LPR + q;
      ok[u] = !bad && c < C && lr < a.rows;
      E[u] = a.base0 + ebase + (int64_t)lr * a.row_stride + (int64_t)c * 64;
      F::load(a.W0, ok[u] ? E[u] : 0, D[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < XSEG; ++u) {
    const int g = u * NT + tid, j = g / XS, c = (g % XS) >> 4;
    const uint32_t m = opaque(((j < K) & (c < C)) ? ~0u : 0u);
    xl[j][c * 17 + (g & 15)] = u32x4{xr[u].x & m, xr[u].y & m, xr[u].z & m, xr[u].w & m};
  }
  __syncthreads();
  auto read_x = [&](int j, int ch, float (&xu)[64]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u32x4 t = xl[j][ch * 17 + i];
      xu[4 * i] = __uint_as_float(t.x);
      xu[4 * i + 1] = __uint_as_float(t.y);
      xu[4 * i + 2] = __uint_as_float(t.z);
      xu[4 * i + 3] = __uint_as_float(t.w);
    }
  };
  if constexpr (F::NS > 0) {
    if (tid < MOE_DOWN_MAX_K * NCH) {
      const int j = tid / NCH, ch = tid % NCH;
      float xu[64], su[NSX];
      read_x(j, ch, xu);
      F::sums(xu, su);
#pragma unroll
      for (int i = 0; i < NSX; ++i) xsl[j][ch][i] = su[i];
    }
    __syncthreads();
  }
  __builtin_amdgcn_sched_barrier(0);
  if (wid < K) {
    float acc = 0.f;  // the per-pair launch's accumulation, bit for bit
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      float xu[64], su[NSX];
      const int ch = (int)opaque((uint32_t)(u * LPR + q));
      read_x(wid, ch, xu);
#pragma unroll
      for (int i = 0; i < NSX; ++i) su[i] = xsl[wid][ch][i];
      float r = F::dot(D[u], xu, su, E[u]);
      // one chunk's x in VGPRs at a time
      asm volatile("" : "+v"(r)::"memory");
      acc += ok[u] ? r : 0.f;
    }
    float v[1] = {acc};
    const float r = reduce_transpose<1, LPR>(v, lane);
    if (q == 0) cb[wid][gi] = r;
  }
  __syncthreads();
  if (tid < TR && row0 + tid < a.rows) {
    float out = 0.f;
    for (int j = 0; j < K; ++j) out = rounded(w_slot[j] * cb[j][tid]) + out;
    a.y[(int64_t)tok * a.y_stride + row0 + tid] = out;
  }
}

// k_moe_down_xl for several tokens: workgroup (row block, token), wave j =
// slot j, nrt row steps of 8 rows per wave (tile t+1's weights in flight while
// tile t is dotted), so the workgroups cover the rows of every token with one
// per CU and all K slots' x is staged once per nrt * 8 rows.  With a grid x
// extent that is a multiple of 8 (16 tokens of 2048 rows: 16 blocks) a block's
// rows sit on one XCD for every token, so tokens that share an expert read its
// rows through the same L2.  Every dot has the bits of the per-pair XL launch
// and the k row values are summed in slot order as k_moe_combine does.
constexpr int MOE_DOWN_T_MAX_ROWS = 512;  // rows per workgroup (nrt <= 64)
//
// STEP (Q4_K only; row strides of whole super-blocks per 8 rows, expert bases on
// super-blocks, experts under 2 GiB): a lane's chunks keep their group g on
// every row step, so each chunk's super-block offset advances by one uniform
// byte count from a wave-uniform expert base and its scale selector
// (FmtQ4_K::select) is formed once.
template <class F, bool STEP>
__global__ __launch_bounds__(512) void k_moe_down_xlt(RowsArgs a, const float *gw, int32_t K, int32_t nrt) {
  static_assert(!STEP || F::TYPE == T_Q4_K, "STEP takes the Q4_K layout");
  constexpr int NT = 512, LPR = 8, CPL = 3, NCH = LPR * CPL, RPW = 64 / LPR, NDW = F::NDW;
  constexpr int NSX = F::NS > 0 ? F::NS : 1;
  constexpr int XS = NCH * 16;                    // 16-byte x segments of one slot
  constexpr int XSEG = MOE_DOWN_MAX_K * XS / NT;  // staged by each thread
  static_assert(XSEG * NT == MOE_DOWN_MAX_K * XS, "x staging");
  static_assert(MOE_DOWN_MAX_K * NCH <= NT, "one thread per (slot, chunk) for the block sums");
  __shared__ u32x4 xl[MOE_DOWN_MAX_K][NCH * 17];
  __shared__ float xsl[MOE_DOWN_MAX_K][NCH][NSX];
  __shared__ float cb[MOE_DOWN_MAX_K][MOE_DOWN_T_MAX_ROWS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = lane / LPR, q = lane % LPR;
  const int tok = blockIdx.y;
  const int C = a.dim1 >> 6;
  const int row0 = blockIdx.x * nrt * RPW;

  u32x4a4 xr[XSEG];
#pragma unroll
  for (int u = 0; u < XSEG; ++u) {
    const int g = u * NT + tid, j = g / XS, c = (g % XS) >> 4;
    const bool in = (j < K) & (c < C);
    const float *xp = a.x + (int64_t)(tok * K + (in ? j : 0)) * a.x_stride + (int64_t)(in ? c : 0) * 64;
    xr[u] = ((const u32x4a4 *)xp)[g & 15];
  }
  // wave wid's slot (a slot past K loads the tensor's first chunk, masked)
  const int expert = a.ids[tok * K + (wid < K ? wid : 0)];
  const bool bad = (wid >= K) | (expert < 0) | (expert >= a.expert_count);
  const int64_t ebase = bad ? 0 : (int64_t)expert * a.expert_stride;
  const uint8_t *wb = a.W0 + ((a.base0 + ebase) >> 8) * 144;  // STEP: the expert's first super-block
  const uint32_t step = (uint32_t)(a.row_stride >> 5) * 144u;   // STEP: bytes per 8 rows
  uint32_t off0[CPL], qo[CPL];
  FmtQ4_K::Sel sel[CPL];
  if constexpr (STEP) {
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      const int64_t e0 = (int64_t)(row0 + gi) * a.row_stride + (int64_t)(u * LPR + q) * 64;
      const int g = (int)((e0 >> 6) & 3);
      off0[u] = (uint32_t)((e0 >> 8) * 144);
      qo[u] = 16u + 32u * (uint32_t)g;
      sel[u] = FmtQ4_K::select(g);
    }
  }
  auto load = [&](int t, uint32_t (&D)[CPL][NDW], bool (&ok)[CPL], int64_t (&E)[CPL]) {
    const int lr = row0 + t * RPW + gi;
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      const int c = u * LPR + q;
      ok[u] = !bad && t < nrt && c < C && lr < a.rows;
      if constexpr (STEP) {
        // a masked chunk reads the expert's first super-block
        const uint32_t o = ok[u] ? off0[u] + (uint32_t)t * step : 0u;
        const u32x4 h = *(const u32x4 *)(wb + o);
        const u32x4 *qs = (const u32x4 *)(wb + (o + qo[u]));
        const u32x4 q0 = qs[0], q1 = qs[1];
        D[u][0] = q0.x; D[u][1] = q0.y; D[u][2] = q0.z; D[u][3] = q0.w;
        D[u][4] = q1.x; D[u][5] = q1.y; D[u][6] = q1.z; D[u][7] = q1.w;
        D[u][8] = h.x; D[u][9] = h.y; D[u][10] = h.z; D[u][11] = h.w;
      } else {
        E[u] = a.base0 + ebase + (int64_t)lr * a.row_stride + (int64_t)c * 64;
        F::load(a.W0, ok[u] ? E[u] : 0, D[u]);
      }
    }
  };
  uint32_t DA[CPL][NDW], DB[CPL][NDW];
  bool okA[CPL], okB[CPL];
  int64_t EA[CPL], EB[CPL];
  load(0, DA, okA, EA);
#pragma unroll
  for (int u = 0; u < XSEG; ++u) {
    const int g = u * NT + tid, j = g / XS, c = (g % XS) >> 4;
    const uint32_t m = opaque(((j < K) & (c < C)) ? ~0u : 0u);
    xl[j][c * 17 + (g & 15)] = u32x4{xr[u].x & m, xr[u].y & m, xr[u].z & m, xr[u].w & m};
  }
  __syncthreads();
  auto read_x = [&](int j, int ch, float (&xu)[64]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u32x4 t = xl[j][ch * 17 + i];
      xu[4 * i] = __uint_as_float(t.x);
      xu[4 * i + 1] = __uint_as_float(t.y);
      xu[4 * i + 2] = __uint_as_float(t.z);
      xu[4 * i + 3] = __uint_as_float(t.w);
    }
  };
  if constexpr (F::NS > 0) {
    if (tid < MOE_DOWN_MAX_K * NCH) {
      const int j = tid / NCH, ch = tid % NCH;
      float xu[64], su[NSX];
      read_x(j, ch, xu);
      F::sums(xu, su);
#pragma unroll
      for (int i = 0; i < NSX; ++i) xsl[j][ch][i] = su[i];
    }
    __syncthreads();
  }
  auto finish = [&](int t, const uint32_t (&D)[CPL][NDW], const bool (&ok)[CPL], const int64_t (&E)[CPL]) {
    float acc = 0.f;  // the per-pair launch's accumulation, bit for bit
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
      float xu[64], su[NSX];
      const int ch = (int)opaque((uint32_t)(u * LPR + q));
      read_x(wid, ch, xu);
#pragma unroll
      for (int i = 0; i < NSX; ++i) su[i] = xsl[wid][ch][i];
      float r;
      if constexpr (STEP) r = FmtQ4_K::dot_sel(D[u], xu, su, sel[u]);
      else r = F::dot(D[u], xu, su, E[u]);
      // one chunk's x in VGPRs at a time
      asm volatile("" : "+v"(r)::"memory");
      acc += ok[u] ? r : 0.f;
    }
    float v[1] = {acc};
    const float r = reduce_transpose<1, LPR>(v, lane);
    if (q == 0) cb[wid][t * RPW + gi] = r;
  };
  if (wid < K) {  // wave-uniform
    for (int t = 0; t < nrt; t += 2) {
      load(t + 1, DB, okB, EB);
      __builtin_amdgcn_sched_barrier(0);
      finish(t, DA, okA, EA);
      __builtin_amdgcn_sched_barrier(0);
      load(t + 2, DA, okA, EA);
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < nrt) finish(t + 1, DB, okB, EB);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
  for (int r = tid; r < nrt * RPW; r += NT) {
    const int row = row0 + r;
    if (row < a.rows) {
      float out = 0.f;
      for (int j = 0; j < K; ++j) out = rounded(gw[tok * K + j] * cb[j][r]) + out;
      a.y[(int64_t)tok * a.y_stride + row] = out;
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
    // eight slots' loads go out before their ordered adds
    for (int j0 = 0; j0 < K; j0 += 8) {
      float a[8], v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u < K ? j0 + u : K - 1;
        a[u] = w[t * K + j];
        v[u] = ys[(t * K + j) * dim + r];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (j0 + u < K) out = rounded(a[u] * v[u]) + out;
    }
    Y[i] = out;
  }
}

// --------------------------------------------------------- decode step ----
// rms norm of vector blockIdx.x (x + v * size, `size` floats), one workgroup each:
// rmsnorm / offset rmsnorm / rmsnormNoWeight of Llama.kt:27-78 by `form`.  The
// sum of squares uses block_sum256's element map; out may alias x (every
// element is read before the scale's barrier and rewritten by its reader);
// resid != null: resid += out (addInPlace, MutableFloatTensor.kt:28-37).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *x, const float *w, float *out, float *resid,
                                                 int32_t size, float eps, int form) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * size;
  const float *xv = x + base;
  float acc = 0.f;
  for (int64_t s = threadIdx.x; s * 4 < size; s += 256)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int64_t i = 4 * s + c;
      acc = sq_acc(acc, i < size ? xv[i] : 0.f);
    }
  const float sc = rms_scale(block_sum256(acc, red), size, eps);
  for (int i = threadIdx.x; i < size; i += 256) {
    const float o = norm_apply(form, form == NORM_NO_WEIGHT ? 1.f : w[i], sc, xv[i]);
    out[base + i] = o;
    if (resid) resid[base + i] = __fadd_rn(resid[base + i], o);
  }
}

// The same for sizes that are a multiple of 4 up to 1024 * VPT: every load
// (x, weight, residual; 16-byte segments tid + 256 j) is issued up front and the
// vector stays in registers, so the kernel makes one round trip to memory.
// Null weight / residual pointers read x instead (no branch around a load).
template <int VPT>
__global__ __launch_bounds__(256) void k_rmsnorm_v(const float *x, const float *w, float *out, float *resid,
                                                   int32_t size, float eps, int form) {
  __shared__ float red[4];
  const int64_t base = (int64_t)blockIdx.x * size;
  const int tid = threadIdx.x;
  const float *wp = w ? w : x + base;
  const float *rp = resid ? resid + base : x + base;
  u32x4a4 xv[VPT], wv[VPT], rv[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int s = j * 256 + tid;
    const int64_t e = 4 * s < size ? 4 * s : 0;
    xv[j] = *(const u32x4a4 *)(x + base + e);
    wv[j] = *(const u32x4a4 *)(wp + e);
    rv[j] = *(const u32x4a4 *)(rp + e);
  }
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint32_t m = opaque(4 * (j * 256 + tid) < size ? ~0u : 0u);
    xv[j] = u32x4a4{xv[j].x & m, xv[j].y & m, xv[j].z & m, xv[j].w & m};
    acc = sq_acc(acc, __uint_as_float(xv[j].x));
    acc = sq_acc(acc, __uint_as_float(xv[j].y));
    acc = sq_acc(acc, __uint_as_float(xv[j].z));
    acc = sq_acc(acc, __uint_as_float(xv[j].w));
  }
  const float sc = rms_scale(block_sum256(acc, red), size, eps);
  const bool nw = form == NORM_NO_WEIGHT;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int s = j * 256 + tid;
    if (4 * s >= size) continue;
    float o[4];
    const float xs[4] = {__uint_as_float(xv[j].x), __uint_as_float(xv[j].y), __uint_as_float(xv[j].z),
                         __uint_as_float(xv[j].w)};
    const float ws[4] = {__uint_as_float(wv[j].x), __uint_as_float(wv[j].y), __uint_as_float(wv[j].z),
                         __uint_as_float(wv[j].w)};
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = norm_apply(form, nw ? 1.f : ws[c], sc, xs[c]);
    *(u32x4a4 *)(out + base + 4 * s) = u32x4a4{__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                               __float_as_uint(o[3])};
    if (resid) {
      const float rs[4] = {__uint_as_float(rv[j].x), __uint_as_float(rv[j].y), __uint_as_float(rv[j].z),
                           __uint_as_float(rv[j].w)};
      *(u32x4a4 *)(resid + base + 4 * s) =
          u32x4a4{__float_as_uint(__fadd_rn(rs[0], o[0])), __float_as_uint(__fadd_rn(rs[1], o[1])),
                  __float_as_uint(__fadd_rn(rs[2], o[2])), __float_as_uint(__fadd_rn(rs[3], o[3]))};
    }
  }
}

// x[i] = x[i] + that[i] (MutableFloatTensor.kt:28-37).
__global__ void k_add(float *x, const float *that, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    x[i] = __fadd_rn(x[i], that[i]);
}

// Llama.kt:403-406 soft-capping in place.
__global__ void k_softcap(float *v, int64_t n, float cap) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    v[i] = softcap_ref(v[i], cap);
}

// ---------------------------------------------------------------- launchers ----

bool rows_fast_ok(int type, const RowsArgs &a, bool paired) {
  if (a.dim1 <= 0 || (a.dim1 % 64) != 0) return false;
  if ((a.base0 % 64) != 0 || (a.row_stride % 64) != 0 || (a.expert_stride % 64) != 0) return false;
  if (paired && (a.base1 % 64) != 0) return false;
  if (paired && (a.dim1 / 64) > 64) return false;  // paired epilogue needs a single column pass
  if (paired && type == T_F32) return false;         // one row step per F32 tile: no room for the pair
  switch (type) {
    case T_Q8_0: case T_Q4_0: case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_F16: case T_BF16: case T_F32:
      return true;
    default: return false;
  }
}

bool rows_norm_ok(int type, const RowsArgs &a, bool paired) {
  if (!rows_fast_ok(type, a, paired)) return false;
  // one column pass: up to 64 lanes x 2 chunks per row (x 1 for the paired kernel)
  return (a.dim1 / 64) <= (paired ? 64 : 128);
}

int max_argmax_blocks(const DevInfo &dev) { return dev.cu_count * 8; }

// Q4_K rows whose chunks sit on fixed super-block groups (the KSEL kernels):
// every base and stride a whole number of 256-element super-blocks.
static bool q4k_groups_fixed(const RowsArgs &a) {
  return a.base0 % 256 == 0 && a.base1 % 256 == 0 && a.row_stride % 256 == 0 && a.expert_stride % 256 == 0;
}

// A format's tiles with one row step (F::RT = 1): more, smaller tiles.
template <class F>
struct OneStep : F {
  static constexpr int RT = 1;
};

template <class F, int LPR, int CPL, bool XL = false, int WPB = 4>
static hipError_t launch_fast_cfg(int epi, const RowsArgs &a, int segments, const DevInfo &dev, hipStream_t s) {
  constexpr int RT = F::RT / CPL > 0 ? F::RT / CPL : 1, RPW = 64 / LPR, TR = RT * RPW;
  typedef void (*Kernel)(RowsArgs);
  const bool multi = (a.dim1 / 64) > LPR * CPL;
  const bool norm = a.norm_w != nullptr;
  const bool route = a.route_logits != nullptr;
  // the fused norm and the routing prologue use 256-thread reductions
  if constexpr (WPB != 4)
    if (norm || route) return launch_fast_cfg<F, LPR, CPL, XL, 4>(epi, a, segments, dev, s);
  if (norm && (multi || segments != 1)) return hipErrorInvalidValue;
  if (route && (epi != EPI_GELU_PAIR || multi)) return hipErrorInvalidValue;
  Kernel k = nullptr;
  if constexpr (XL) {
    if (epi == EPI_STORE && !norm && !route && !multi)
      k = k_rows<F, LPR, CPL, EPI_STORE, false, false, false, true, WPB>;
  } else if constexpr (WPB != 4) {
    if (epi == EPI_STORE) k = k_rows<F, LPR, CPL, EPI_STORE, false, false, false, false, WPB>;
    else if (epi == EPI_ARGMAX) k = k_rows<F, LPR, CPL, EPI_ARGMAX, false, false, false, false, WPB>;
    else if constexpr (CPL == 1 && F::RT >= 2) k = k_rows<F, LPR, 1, EPI_GELU_PAIR, false, false, false, false, WPB>;
    if constexpr (LPR == 64 && CPL == 2) {
      if (multi && epi == EPI_STORE) k = k_rows<F, LPR, CPL, EPI_STORE, true, false, false, false, WPB>;
      if (multi && epi == EPI_ARGMAX) k = k_rows<F, LPR, CPL, EPI_ARGMAX, true, false, false, false, WPB>;
    }
  } else if (epi == EPI_STORE) {
    k = norm ? k_rows<F, LPR, CPL, EPI_STORE, false, true> : k_rows<F, LPR, CPL, EPI_STORE, false, false>;
    if constexpr (LPR == 64 && CPL == 2)
      if (multi) k = k_rows<F, LPR, CPL, EPI_STORE, true, false>;
  } else if (epi == EPI_ARGMAX) {
    k = norm ? k_rows<F, LPR, CPL, EPI_ARGMAX, false, true> : k_rows<F, LPR, CPL, EPI_ARGMAX, false, false>;
    if constexpr (LPR == 64 && CPL == 2)
      if (multi) k = k_rows<F, LPR, CPL, EPI_ARGMAX, true, false>;
  } else {
    if constexpr (CPL == 1 && F::RT >= 2) {
      if (route) k = norm ? nullptr : k_rows<F, LPR, 1, EPI_GELU_PAIR, false, false, true>;
      else k = norm ? k_rows<F, LPR, 1, EPI_GELU_PAIR, false, true> : k_rows<F, LPR, 1, EPI_GELU_PAIR, false, false>;
    }
  }
  // Q4_K matvecs and gate+up launches (single pass, no fused norm) with each
  // lane's scale selector formed once (the same results)
  bool ksel = false;
  if constexpr (F::TYPE == T_Q4_K && LPR % 4 == 0 && !XL) {
    if (k && q4k_groups_fixed(a) && !multi && !norm) {
      if (epi == EPI_STORE) {
        k = k_rows<F, LPR, CPL, EPI_STORE, false, false, false, false, WPB, false, true>;
        ksel = true;
      }
      if constexpr (WPB == 4 && CPL == 1 && F::RT >= 2) {
        if (epi == EPI_GELU_PAIR) {
          k = route ? k_rows<F, LPR, 1, EPI_GELU_PAIR, false, false, true, false, 4, false, true>
                    : k_rows<F, LPR, 1, EPI_GELU_PAIR, false, false, false, false, 4, false, true>;
          ksel = true;
        }
      }
    }
  }
  if (!k) return hipErrorInvalidValue;
  if (multi && !(LPR == 64 && CPL == 2)) return hipErrorInvalidValue;

  // Resident 256-thread workgroups per CU for this kernel (register-limited);
  // the launch fills exactly that many waves when there are tiles enough.
  // Looked up once per kernel; contexts on other threads may race to store the
  // same value, hence relaxed atomics.
  static std::atomic<int> resident[3][2][2][2][2];
  std::atomic<int> &slot = resident[epi][multi ? 1 : 0][norm ? 1 : 0][route ? 1 : 0][ksel ? 1 : 0];
  int res = slot.load(std::memory_order_relaxed);
  if (res == 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, 64 * WPB, 0) != hipSuccess || nb < 1) nb = 8 / WPB;
    res = nb;
    slot.store(res, std::memory_order_relaxed);
  }
  const int lrt = epi == EPI_GELU_PAIR ? TR / 2 : TR;
  const int64_t n_tiles = (a.rows + lrt - 1) / lrt;
  const int64_t segs = segments > 0 ? segments : 1;
  const int64_t cu = dev.cu_count;
  // WPB-wave workgroups sharing one LDS copy of x.  About two tiles per wave
  // (one computing while the next is in flight), rounded up to whole rounds of
  // one workgroup per CU over all segments (a partial round leaves CUs with
  // half the work of the others), at most what is resident at once, never more
  // workgroups than tiles (idle waves only help stage x).
  int64_t blocks = (n_tiles + WPB * G4_TILES_PER_WAVE - 1) / (WPB * G4_TILES_PER_WAVE);
  blocks = ((blocks * segs + cu - 1) / cu * cu + segs - 1) / segs;
  // at most eight resident waves per CU: with more requests in flight a long
  // stream (the 570 MB LM head) was measured slower, and the small launches
  // never reach the cap
  constexpr int WG_CAP = 8 / WPB;
  const int64_t slots = cu * (res < WG_CAP ? res : WG_CAP);
  int64_t cap = slots / segs;
  // When the segments do not divide the resident workgroups evenly, more
  // workgroups per segment can even out the CUs: b workgroups per segment leave
  // the busiest CU ceil(b * segs / cu) of them, 1/b segment each (320 MoE pairs
  // on 256 CUs: two whole segments on some CUs at b = 1, 1.25 at b = 4).  The
  // smallest b up to four times the resident share that loads the busiest CU
  // least.
  if (cap >= 1 && slots % segs != 0) {
    auto busiest = [&](int64_t b) { return (double)((b * segs + cu - 1) / cu) / (double)b; };
    int64_t best = cap;
    for (int64_t b = cap + 1; b <= 4 * cap && b <= blocks; ++b)
      if (busiest(b) < busiest(best)) best = b;
    cap = best;
  }
  if (blocks > cap) blocks = cap;
  if (blocks > n_tiles) blocks = n_tiles;
  if (blocks < 1) blocks = 1;
  if (epi == EPI_ARGMAX && blocks > max_argmax_blocks(dev)) blocks = max_argmax_blocks(dev);
  hipLaunchKernelGGL(k, dim3((unsigned)blocks, (unsigned)segments), dim3(64 * WPB), 0, s, a);
  if (epi == EPI_ARGMAX) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, (const float *)a.am_val, (const int32_t *)a.am_idx,
                       (int)blocks, a.am_out);
  }
  return hipGetLastError();
}

template <class F>
static hipError_t launch_fast(int epi, const RowsArgs &a, int segments, const DevInfo &dev, hipStream_t s) {
  const int C = a.dim1 / 64;
  // single column pass up to 64 lanes x 2 chunks = 8192 columns; passes beyond that
  if (C > 64 && epi != EPI_GELU_PAIR) return launch_fast_cfg<F, 64, 2>(epi, a, segments, dev, s);
  // Q8_0 and Q6_K (the formats with the widest chunks, 17 and 29 dwords) take
  // one row step per tile up to 16384 rows: measured 4.55 -> 4.30 us on the
  // 2048-row Q8_0 matvec and 7.4 -> 6.6 us on the 8192-row Q6_K one, while
  // Q4_K got slower and the 262144-row LM head lost 1.4 us with it
  if constexpr (F::RT >= 2 && (F::TYPE == T_Q8_0 || F::TYPE == T_Q6_K)) {
    if (epi == EPI_STORE && (int64_t)a.rows * segments <= 16384) {
      if (C > 32) return launch_fast_cfg<OneStep<F>, 64, 1>(epi, a, segments, dev, s);
      if (C > 16) return launch_fast_cfg<OneStep<F>, 32, 1>(epi, a, segments, dev, s);
      return launch_fast_cfg<OneStep<F>, 16, 1>(epi, a, segments, dev, s);
    }
  }
  // The arg-max matvec over a vocabulary (no fused norm) takes one 8-wave
  // workgroup per CU instead of two 4-wave ones: the 262144-row Q8_0 LM head
  // measured 100.3 -> 98.9 us (the small matvecs lost 0.5-1 us that way)
  if (epi == EPI_ARGMAX && !a.norm_w && (int64_t)a.rows * segments >= 65536 && C <= 64) {
    if (C > 32) return launch_fast_cfg<F, 64, 1, false, 8>(epi, a, segments, dev, s);
    if (C > 16) return launch_fast_cfg<F, 32, 1, false, 8>(epi, a, segments, dev, s);
    return launch_fast_cfg<F, 16, 1, false, 8>(epi, a, segments, dev, s);
  }
  if (C > 32) return launch_fast_cfg<F, 64, 1>(epi, a, segments, dev, s);
  // rows of 17..24 chunks (the MoE down projection's 1408 columns are 22): 8
  // lanes x 3 chunks with x read at use keep 22 of 24 lanes busy, against 22 of
  // 32 with one chunk per lane (16 tokens of 128-expert top-8 MoE: 127 -> 117 us
  // per step); for the formats whose three chunk buffers fit the VGPRs
  if constexpr (F::NDW <= 20)
    if (C > 16 && C <= 24 && epi == EPI_STORE && !a.norm_w)
      return launch_fast_cfg<F, 8, 3, true>(epi, a, segments, dev, s);
  if (C > 16) return launch_fast_cfg<F, 32, 1>(epi, a, segments, dev, s);
  return launch_fast_cfg<F, 16, 1>(epi, a, segments, dev, s);
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
    case T_Q5_K: return launch_generic_t<T_Q5_K>(a, nmat, segments, dev, s);
    case T_Q6_K: return launch_generic_t<T_Q6_K>(a, nmat, segments, dev, s);
    case T_F16: return launch_generic_t<T_F16>(a, nmat, segments, dev, s);
    case T_BF16: return launch_generic_t<T_BF16>(a, nmat, segments, dev, s);
    case T_F32: return launch_generic_t<T_F32>(a, nmat, segments, dev, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_rows(int type, int epi, const RowsArgs &a, int segments, const DevInfo &dev, float *scratch,
                       hipStream_t s) {
  if (a.route_logits) {
    if (epi != EPI_GELU_PAIR || a.norm_w || a.x_div <= 0 || segments % a.x_div != 0) return hipErrorInvalidValue;
    if (!rows_fast_ok(type, a, true) || a.route_e > ROUTE_FUSED_MAX_E) {
      // routing in its own launch; the expert rows then read the ids it stores
      hipError_t e = launch_route(a.route_logits, segments / a.x_div, a.route_e, a.x_div, a.route_renorm,
                                  a.route_scale, a.route_ids, a.route_w, s);
      if (e != hipSuccess) return e;
      RowsArgs b = a;
      b.route_logits = nullptr;
      b.ids = a.route_ids;
      return launch_rows(type, epi, b, segments, dev, scratch, s);
    }
  }
  if (wide_ok(type, a, epi)) return launch_wide(type, a, segments, s);
  if (rows_fast_ok(type, a, epi == EPI_GELU_PAIR)) {
    switch (type) {
      case T_Q8_0: return launch_fast<FmtQ8_0>(epi, a, segments, dev, s);
      case T_Q4_0: return launch_fast<FmtQ4_0>(epi, a, segments, dev, s);
      case T_Q4_K: return launch_fast<FmtQ4_K>(epi, a, segments, dev, s);
      case T_Q5_K: return launch_fast<FmtQ5_K>(epi, a, segments, dev, s);
      case T_Q6_K: return launch_fast<FmtQ6_K>(epi, a, segments, dev, s);
      case T_F16: return launch_fast<FmtHalf<T_F16>>(epi, a, segments, dev, s);
      case T_BF16: return launch_fast<FmtHalf<T_BF16>>(epi, a, segments, dev, s);
      case T_F32: return launch_fast<FmtF32>(epi, a, segments, dev, s);
      default: return hipErrorInvalidValue;
    }
  }
  // generic path
  if (epi == EPI_GELU_PAIR) {
    if (a.norm_w) return hipErrorInvalidValue;
    RowsArgs g = a;
    g.y = scratch;
    g.y_stride = 2 * (int64_t)a.rows;
    hipError_t e = launch_generic(type, g, 2, segments, dev, s);
    if (e != hipSuccess) return e;
    return launch_gelu_mul(scratch, a.rows, segments, a.y, a.y_stride, s);
  }
  if (a.norm_w) return hipErrorInvalidValue;  // callers normalise x first when rows_norm_ok fails
  hipError_t e = launch_generic(type, a, 1, segments, dev, s);
  if (e != hipSuccess || epi != EPI_ARGMAX) return e;
  if (a.softcap > 0.f) {
    e = launch_softcap(a.y, a.rows, a.softcap, s);
    if (e != hipSuccess) return e;
  }
  return launch_argmax(a.y, a.rows, a.am_val, a.am_idx, a.am_out, dev, s);
}

hipError_t launch_dequant(int type, const uint8_t *W, int64_t offset, int64_t n, float *out, hipStream_t s) {
  int64_t b = (n + 255) / 256;
  int blocks = (int)(b > 8192 ? 8192 : (b < 1 ? 1 : b));
  switch (type) {
    case T_Q8_0: hipLaunchKernelGGL(k_dequant<T_Q8_0>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_Q4_0: hipLaunchKernelGGL(k_dequant<T_Q4_0>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_Q4_K: hipLaunchKernelGGL(k_dequant<T_Q4_K>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_Q5_K: hipLaunchKernelGGL(k_dequant<T_Q5_K>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_Q6_K: hipLaunchKernelGGL(k_dequant<T_Q6_K>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_F16: hipLaunchKernelGGL(k_dequant<T_F16>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_BF16: hipLaunchKernelGGL(k_dequant<T_BF16>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    case T_F32: hipLaunchKernelGGL(k_dequant<T_F32>, dim3(blocks), dim3(256), 0, s, W, offset, n, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_argmax(const float *v, int32_t n, float *part_val, int32_t *part_idx, int32_t *out,
                         const DevInfo &dev, hipStream_t s) {
  int blocks = (n + 255) / 256;
  const int cap = max_argmax_blocks(dev);
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_argmax, dim3(blocks), dim3(256), 0, s, v, n, part_val, part_idx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, (const float *)part_val, (const int32_t *)part_idx,
                     blocks, out);
  return hipGetLastError();
}

hipError_t launch_route(const float *logits, int32_t T, int32_t n_experts, int32_t k, int32_t renorm,
                        const float *expert_scale, int32_t *ids, float *weights, hipStream_t s) {
  if (n_experts > ROUTE_MAX_E) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_route, dim3(T), dim3(256), 0, s, logits, n_experts, k, renorm, expert_scale, ids, weights);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *w, float *out, float *resid, int32_t n_vec, int32_t size,
                          float eps, int form, hipStream_t s) {
  if (n_vec <= 0 || size <= 0) return hipSuccess;
  if (form < NORM_WEIGHT_AFTER || form > NORM_NO_WEIGHT || (form != NORM_NO_WEIGHT && !w)) return hipErrorInvalidValue;
  if (form == NORM_NO_WEIGHT) w = nullptr;
  if (size % 4 == 0 && size <= 8192) {
    const int vpt = (size + 1023) / 1024;
    if (vpt == 1) hipLaunchKernelGGL(k_rmsnorm_v<1>, dim3(n_vec), dim3(256), 0, s, x, w, out, resid, size, eps, form);
    else if (vpt == 2) hipLaunchKernelGGL(k_rmsnorm_v<2>, dim3(n_vec), dim3(256), 0, s, x, w, out, resid, size, eps, form);
    else if (vpt <= 4) hipLaunchKernelGGL(k_rmsnorm_v<4>, dim3(n_vec), dim3(256), 0, s, x, w, out, resid, size, eps, form);
    else hipLaunchKernelGGL(k_rmsnorm_v<8>, dim3(n_vec), dim3(256), 0, s, x, w, out, resid, size, eps, form);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(k_rmsnorm, dim3(n_vec), dim3(256), 0, s, x, w, out, resid, size, eps, form);
  return hipGetLastError();
}

static int elementwise_blocks(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (int)(b > 4096 ? 4096 : (b < 1 ? 1 : b));
}

hipError_t launch_add(float *x, const float *that, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_add, dim3(elementwise_blocks(n)), dim3(256), 0, s, x, that, n);
  return hipGetLastError();
}

hipError_t launch_softcap(float *v, int64_t n, float cap, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_softcap, dim3(elementwise_blocks(n)), dim3(256), 0, s, v, n, cap);
  return hipGetLastError();
}

// k_moe_down for a.rows rows of T tokens: a.x = h [T*K slots x dim1], a.ids = the
// slots' experts, a.y = Y with row stride a.y_stride.  hipErrorNotSupported when
// the shape needs the separate down and combine launches.
// One row tile per workgroup.  Only while the (tile, token) workgroups fit two
// per CU: each stages every slot's h, and with more tokens the separate down
// launch (one slot per workgroup, its x staged once per row range) and
// k_moe_combine were measured faster (16 tokens: 120 against 137 us per step).
template <class F, int LPR>
static hipError_t launch_moe_down_cfg(const RowsArgs &a, const float *gw, int32_t T, int32_t K, const DevInfo &dev,
                                      hipStream_t s) {
  // 8-wave workgroups (twice the rows, half the x staging per row) while one
  // per CU covers the rows; else 4-wave ones, up to two per CU
  constexpr int TR8 = 2 * F::RT * (64 / LPR), TR4 = F::RT * (64 / LPR);
  const int64_t n8 = (a.rows + TR8 - 1) / TR8, n4 = (a.rows + TR4 - 1) / TR4;
  if (n8 * T <= (int64_t)dev.cu_count) {
    // rows of 17..24 chunks: 8 lanes x 3 chunks (the same 8 rows per workgroup
    // when LPR is 32), for the formats whose three chunk buffers fit the VGPRs
    if constexpr (F::NDW <= 20 && LPR == 32 && TR8 == 8) {
      if (a.dim1 <= 24 * 64) {
        hipLaunchKernelGGL(k_moe_down_xl<F>, dim3((unsigned)n8, T), dim3(512), 0, s, a, gw, K);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((k_moe_down<F, LPR, 8>), dim3((unsigned)n8, T), dim3(512), 0, s, a, gw, K);
    return hipGetLastError();
  }
  if (n4 * T <= 2 * (int64_t)dev.cu_count) {
    hipLaunchKernelGGL((k_moe_down<F, LPR, 4>), dim3((unsigned)n4, T), dim3(256), 0, s, a, gw, K);
    return hipGetLastError();
  }
  // more tokens, rows of 17..24 chunks: row steps of 8 rows looped per wave,
  // about one workgroup per CU over all tokens
  if constexpr (F::NDW <= 20) {
    if (a.dim1 > 16 * 64 && a.dim1 <= 24 * 64) {
      // at most one workgroup per CU over all tokens (one is resident per CU,
      // and a partial second round would double the launch)
      const int64_t steps = (a.rows + 7) / 8;
      int64_t nbm = dev.cu_count / T;
      if (nbm < 1) nbm = 1;
      const int64_t nrt = (steps + nbm - 1) / nbm;
      if (nrt * 8 <= MOE_DOWN_T_MAX_ROWS) {
        const int64_t nb = (steps + nrt - 1) / nrt;
        if constexpr (F::TYPE == T_Q4_K) {
          if (a.row_stride % 32 == 0 && a.base0 % 256 == 0 && a.expert_stride % 256 == 0 &&
              (int64_t)a.rows * a.row_stride / 256 * 144 + 256 < (1ll << 31)) {
            hipLaunchKernelGGL((k_moe_down_xlt<F, true>), dim3((unsigned)nb, T), dim3(512), 0, s, a, gw, K, (int32_t)nrt);
            return hipGetLastError();
          }
        }
        hipLaunchKernelGGL((k_moe_down_xlt<F, false>), dim3((unsigned)nb, T), dim3(512), 0, s, a, gw, K, (int32_t)nrt);
        return hipGetLastError();
      }
    }
  }
  return hipErrorNotSupported;
}

template <class F>
static hipError_t launch_moe_down_t(const RowsArgs &a, const float *gw, int32_t T, int32_t K, const DevInfo &dev,
                                    hipStream_t s) {
  const int C = a.dim1 / 64;
  if (C <= 16) return launch_moe_down_cfg<F, 16>(a, gw, T, K, dev, s);
  if (C <= 32) return launch_moe_down_cfg<F, 32>(a, gw, T, K, dev, s);
  return hipErrorNotSupported;
}

hipError_t launch_moe_down(int type, const RowsArgs &a, const float *gw, int32_t T, int32_t K, const DevInfo &dev,
                           hipStream_t s) {
  if (K < 1 || K > MOE_DOWN_MAX_K || T < 1 || a.rows < 1 || !rows_fast_ok(type, a, false)) return hipErrorNotSupported;
  switch (type) {
    case T_Q8_0: return launch_moe_down_t<FmtQ8_0>(a, gw, T, K, dev, s);
    case T_Q4_0: return launch_moe_down_t<FmtQ4_0>(a, gw, T, K, dev, s);
    case T_Q4_K: return launch_moe_down_t<FmtQ4_K>(a, gw, T, K, dev, s);
    case T_Q5_K: return launch_moe_down_t<FmtQ5_K>(a, gw, T, K, dev, s);
    case T_Q6_K: return launch_moe_down_t<FmtQ6_K>(a, gw, T, K, dev, s);
    case T_F16: return launch_moe_down_t<FmtHalf<T_F16>>(a, gw, T, K, dev, s);
    case T_BF16: return launch_moe_down_t<FmtHalf<T_BF16>>(a, gw, T, K, dev, s);
    case T_F32: return launch_moe_down_t<FmtF32>(a, gw, T, K, dev, s);
    default: return hipErrorNotSupported;
  }
}

template <class F>
static hipError_t launch_moe_gate_up_t(const RowsArgs &a, int32_t T, const DevInfo &dev, hipStream_t s) {
  constexpr int LRT = F::RT;  // logical rows per paired tile at 32 lanes per row
  const int64_t n_tiles = (a.rows + LRT - 1) / LRT;
  // one 8-wave workgroup per CU over all tokens
  int64_t nb = dev.cu_count / T;
  if (nb > n_tiles) nb = n_tiles;
  if (nb < 1) nb = 1;
  if constexpr (F::TYPE == T_Q4_K) {
    if (q4k_groups_fixed(a)) {
      if (a.route_logits)
        hipLaunchKernelGGL((k_rows<F, 32, 1, EPI_GELU_PAIR, false, false, true, false, 8, true, true>),
                           dim3((unsigned)nb, T), dim3(512), 0, s, a);
      else
        hipLaunchKernelGGL((k_rows<F, 32, 1, EPI_GELU_PAIR, false, false, false, false, 8, true, true>),
                           dim3((unsigned)nb, T), dim3(512), 0, s, a);
      return hipGetLastError();
    }
  }
  if (a.route_logits)
    hipLaunchKernelGGL((k_rows<F, 32, 1, EPI_GELU_PAIR, false, false, true, false, 8, true>), dim3((unsigned)nb, T),
                       dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((k_rows<F, 32, 1, EPI_GELU_PAIR, false, false, false, false, 8, true>), dim3((unsigned)nb, T),
                       dim3(512), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_moe_gate_up(int type, const RowsArgs &a, int32_t T, const DevInfo &dev, hipStream_t s) {
  const int C = a.dim1 / 64;
  if (T < 2 || a.x_div < 1 || a.x_div > 8 || a.norm_w || C <= 16 || C > 32 || !rows_fast_ok(type, a, true))
    return hipErrorNotSupported;
  if (a.route_logits && a.route_e > ROUTE_FUSED_MAX_E) return hipErrorNotSupported;
  switch (type) {
    case T_Q8_0: return launch_moe_gate_up_t<FmtQ8_0>(a, T, dev, s);
    case T_Q4_0: return launch_moe_gate_up_t<FmtQ4_0>(a, T, dev, s);
    case T_Q4_K: return launch_moe_gate_up_t<FmtQ4_K>(a, T, dev, s);
    case T_Q5_K: return launch_moe_gate_up_t<FmtQ5_K>(a, T, dev, s);
    case T_Q6_K: return launch_moe_gate_up_t<FmtQ6_K>(a, T, dev, s);
    default: return hipErrorNotSupported;
  }
}

// dst[0 .. bytes) = src[0 .. bytes): bytes a multiple of 4, both ends 16-byte
// aligned.  Moves the host-pointer entry points' activations between pinned host
// memory and the device without a DMA command (the copy engines' start-up cost
// more than these few kilobytes).
__global__ __launch_bounds__(256) void k_copy(uint32_t *dst, const uint32_t *src, int64_t words) {
  const int64_t n4 = words >> 2;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4; i += step)
    ((u32x4 *)dst)[i] = ((const u32x4 *)src)[i];
  for (int64_t i = 4 * n4 + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < words; i += step) dst[i] = src[i];
}

hipError_t launch_copy(void *dst, const void *src, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  if ((bytes & 3) || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15)) return hipErrorInvalidValue;
  const int64_t words = (int64_t)(bytes >> 2);
  int64_t blocks = (words / 4 + 255) / 256;
  if (blocks > 256) blocks = 256;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_copy, dim3((unsigned)blocks), dim3(256), 0, s, (uint32_t *)dst, (const uint32_t *)src, words);
  return hipGetLastError();
}

// dst[0 .. bytes) = 0, bytewise (the degenerate-shape outputs it serves are small).
__global__ __launch_bounds__(256) void k_zero(uint8_t *dst, int64_t bytes) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < bytes; i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = 0;
}

hipError_t launch_zero(void *dst, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  int64_t blocks = ((int64_t)bytes + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(k_zero, dim3((unsigned)blocks), dim3(256), 0, s, (uint8_t *)dst, (int64_t)bytes);
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
