// g4_wide.hip -- matvec of rows wider than one wave's 64 chunks (more than 4096
// columns), e.g. the FFN's down projection W_down [dim x hidden] of
// Llama.kt:357-361 at hidden = 8192 (FloatTensor.kt:18-29).
//
// The row engine (k_rows) gives each row one wave and stages all of x in LDS per
// workgroup: with 128 chunks per row, a wave then holds two rows at most and
// every wave waits at the staging barrier before it computes.  Here the columns
// are split over the WPB waves of a workgroup instead: wave w owns chunks
// w*LPR .. w*LPR+LPR-1 of every row of the workgroup's row range, loads its own
// slice of x straight into registers (no barrier before the first tile), and
// streams RT-step row tiles through a two-deep pipeline like the row engine.
// Each wave's per-row partial sums meet in LDS and are added in wave order
// (deterministic) once every wave is done.
#include "g4_device.hpp"
#include "g4_internal.hpp"

namespace g4 {

constexpr int WIDE_MAX_ROWS = 64;  // rows per workgroup held in LDS
// 8 rows per workgroup in tiles of two row steps (two tiles per wave).  On the
// 2048 x 8192 Q4_0 down projection: 4 rows per workgroup took 8.2 us (twice the
// workgroups, each fetching all of x), 8 rows 5.5 us, 16 rows 7.1-8.1 us (half
// the CUs idle), 32 rows 10 us; one row step per tile 5.7 us.
constexpr int WIDE_ROWS = 8;
constexpr int WIDE_RT = 2;

template <class F, int LPR, int WPB, int RT>
__global__ __launch_bounds__(64 * WPB) void k_wide(RowsArgs a, int rows_per_wg) {
  constexpr int RPW = 64 / LPR;  // rows per step (one per lane group)
  constexpr int TR = RT * RPW;   // rows per tile
  constexpr int NDW = F::NDW;
  constexpr int NSX = F::NS > 0 ? F::NS : 1;
  __shared__ float part[WPB][WIDE_MAX_ROWS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gi = lane / LPR, q = lane % LPR;
  const int C = a.dim1 >> 6;
  const int seg = blockIdx.y;
  const int c = wid * LPR + q;  // this lane's chunk of every row
  const bool cok = c < C;
  const float *x = a.x + (int64_t)(seg / a.x_div) * a.x_stride;
  float *y = a.y + (int64_t)seg * a.y_stride;
  const int r0 = blockIdx.x * rows_per_wg;
  const int nr = min(rows_per_wg, a.rows - r0);
  const int n_tiles = (nr + TR - 1) / TR;

  auto load_tile = [&](int t, bool live, uint32_t (&D)[RT][NDW], bool (&ok)[RT], int64_t (&E)[RT]) {
#pragma unroll
    for (int k = 0; k < RT; ++k) {
      const int lr = t * TR + k * RPW + gi;
      ok[k] = live && cok && lr < nr;
      E[k] = a.base0 + (int64_t)(r0 + lr) * a.row_stride + (int64_t)c * 64;
      // lanes past the rows or the columns read the tensor's first chunk (in
      // bounds) and mask it: no branch around a load
      F::load(a.W0, ok[k] ? E[k] : 0, D[k]);
    }
  };

  // x of the wave's 32 chunks, loaded first, then the first tile, and only then
  // waited for (vmcnt retires in issue order): x's arrival, not the weights',
  // gates the first tile (the 32 KB vector goes to every workgroup).  Read so
  // that adjacent lanes take adjacent 16-byte pieces (instruction i: lane l takes
  // piece l % 16 of chunk 4 i + l / 16; reading by chunk put 64 chunks 256 bytes
  // apart in every instruction) and staged in the wave's own LDS rows (chunks
  // padded to XC floats, conflict-free below), a wave reading only what it
  // wrote.  Lanes l and l ^ 32 hold the same chunk (LPR = 32): each reads half
  // of its 16 words back and v_permlane32_swap hands each half the other's.
  static_assert(LPR == 32, "two lane groups share each chunk of x");
  constexpr int XC = 68;
  __shared__ __attribute__((aligned(16))) float xst[WPB][LPR * XC];
  const int xh = lane >> 5;
  u32x4a4 xg[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int cc = wid * LPR + 4 * i + (lane >> 4);  // chunks past the row read chunk 0 (in bounds, masked)
    xg[i] = *(const u32x4a4 *)(x + (int64_t)(cc < C ? cc : 0) * 64 + 4 * (lane & 15));
  }
  uint32_t DA[RT][NDW], DB[RT][NDW];
  bool okA[RT], okB[RT];
  int64_t EA[RT], EB[RT];
  __builtin_amdgcn_sched_barrier(0);
  load_tile(0, 0 < n_tiles, DA, okA, EA);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 8; ++i) *(u32x4 *)&xst[wid][(4 * i + (lane >> 4)) * XC + 4 * (lane & 15)] = xg[i];
  u32x4 xr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xr[i] = *(const u32x4 *)&xst[wid][q * XC + 32 * xh + 4 * i];
  float xv[64];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w4[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // r[0]: the lower half's word in every lane (x word 4 i + j), r[1]: the upper half's (word 32 + 4 i + j)
      const auto r = __builtin_amdgcn_permlane32_swap(w4[j], w4[j], false, false);
      xv[4 * i + j] = __uint_as_float(r[0]);
      xv[32 + 4 * i + j] = __uint_as_float(r[1]);
    }
  }
  float xs[NSX];
  F::sums(xv, xs);

  auto finish_tile = [&](int t, const uint32_t (&D)[RT][NDW], const bool (&ok)[RT], const int64_t (&E)[RT]) {
    float v[RT];
#pragma unroll
    for (int k = 0; k < RT; ++k) {
      const float r = F::dot(D[k], xv, xs, E[k]);
      float acc = 0.f;
      acc += ok[k] ? r : 0.f;
      v[k] = acc;
    }
    const float r = reduce_transpose<RT, LPR>(v, lane);
    const int k = q / (LPR / RT);
    if ((q % (LPR / RT)) == 0) {
      const int lr = t * TR + k * RPW + gi;
      if (lr < nr) part[wid][lr] = r;
    }
  };

  for (int t = 0; t < n_tiles; t += 2) {
    load_tile(t + 1, t + 1 < n_tiles, DB, okB, EB);
    __builtin_amdgcn_sched_barrier(0);
    finish_tile(t, DA, okA, EA);
    __builtin_amdgcn_sched_barrier(0);
    load_tile(t + 2, t + 2 < n_tiles, DA, okA, EA);
    __builtin_amdgcn_sched_barrier(0);
    if (t + 1 < n_tiles) finish_tile(t + 1, DB, okB, EB);
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();
  for (int i = tid; i < nr; i += 64 * WPB) {
    float s = part[0][i];
#pragma unroll
    for (int w = 1; w < WPB; ++w) s += part[w][i];
    y[r0 + i] = s;
  }
}

template <class F, int LPR, int WPB, int RT>
static hipError_t launch_wide_cfg(const RowsArgs &a, int segments, hipStream_t s) {
  constexpr int TR = RT * (64 / LPR);
  int rpw = WIDE_ROWS;
  rpw = (rpw + TR - 1) / TR * TR;
  if (rpw > WIDE_MAX_ROWS) rpw = WIDE_MAX_ROWS / TR * TR;
  const int blocks = (a.rows + rpw - 1) / rpw;
  hipLaunchKernelGGL((k_wide<F, LPR, WPB, RT>), dim3((unsigned)blocks, (unsigned)segments), dim3(64 * WPB), 0, s,
                     a, rpw);
  return hipGetLastError();
}

template <class F>
static hipError_t launch_wide_t(const RowsArgs &a, int segments, hipStream_t s) {
  const int C = a.dim1 / 64;
  if (C <= 128) return launch_wide_cfg<F, 32, 4, WIDE_RT>(a, segments, s);
  return launch_wide_cfg<F, 32, 8, WIDE_RT>(a, segments, s);
}

bool wide_ok(int type, const RowsArgs &a, int epi) {
  const int C = a.dim1 / 64;
  if (epi != EPI_STORE || a.norm_w || a.route_logits || a.ids) return false;
  if (C <= 64 || C > 256) return false;
  if (!rows_fast_ok(type, a, false)) return false;
  return type == T_Q4_0 || type == T_Q8_0 || type == T_Q4_K || type == T_Q5_K;
}

hipError_t launch_wide(int type, const RowsArgs &a, int segments, hipStream_t s) {
  switch (type) {
    case T_Q4_0: return launch_wide_t<FmtQ4_0>(a, segments, s);
    case T_Q8_0: return launch_wide_t<FmtQ8_0>(a, segments, s);
    case T_Q4_K: return launch_wide_t<FmtQ4_K>(a, segments, s);
    case T_Q5_K: return launch_wide_t<FmtQ5_K>(a, segments, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace g4
