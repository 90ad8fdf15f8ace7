// g4_tok.hip -- multi-token Q4_K matmul on the gfx950 matrix cores.
//
// Y[m][r] = sum_c W[r][c] X[m][c] for M tokens (FloatTensor.matmul applied to M
// activation rows, FloatTensor.kt:18-29; Q4_K blocks of Q4_KFloatTensor.kt:23-55).
//
// Exactness.  The matrix cores multiply bf16 operands into fp32 sums, and both
// operands here are exact in bf16:
//   * weights: a Q4_K weight is d*sc*q - dmin*m with q in 0..15 per 32-weight
//     sub-block, written here as (d*sc/16) * 16(q - 8) + (8 d*sc - dmin*m):
//     16(q - 8) in -128..112 is an exact bf16, and the sub-block's two fp32
//     coefficients are applied after the products, as
//     (d*sc/16) * sum(16(q - 8) x) + (8 d*sc - dmin*m) * sum(x).  8 d*sc is
//     exact, so a sub-block of weights that are all exactly zero contributes
//     exactly 0, as in the reference, whose fma(q, d*sc, -dmin*m) forms each
//     weight first (Q4_KFloatTensor.kt:143-148), when q = 8 and 8 d*sc =
//     dmin*m, or d*sc = dmin*m = 0.  Other all-zero sub-blocks (a constant
//     q0 != 8 with dmin*m = q0 d*sc) leave a residue of the size of the
//     rounding of the two sums: a known limit.  The rounding of the sums scales
//     with |q - 8| rather than with q.
//     Calls of at most 8 tokens and workgroups of four or more row tiles (more
//     than 16 tokens at 8192 rows) form sum(16(q - 8) x) as
//     sum(16 q x) - sum(128 x) instead: 16 q comes
//     from the nibble as an e4m3 code (two weights per conversion instead of a
//     convert per weight and a pack per two), and sum(128 x) is formed once per
//     wave by the same MFMAs with the weight operand of an all-8 sub-block, so
//     for q = 8 the two sums are equal bit for bit and their difference, taken
//     before the scale, is exactly 0.  The rounding of these sums scales with q
//     and 8 rather than |q - 8|;
//   * activations: an fp32 x has 24 significant bits and splits exactly into
//     x1 + x2 + x3, three bf16 parts of 8 significant bits each, so three
//     MFMAs give sum(q x) with exact products and fp32 accumulation.
//
// Work split.  v_mfma_f32_16x16x32_bf16 with A = x parts (16 tokens x 32
// columns), B = weight nibbles (32 columns x 16 rows), C = 16 tokens x 16 rows:
// lane l holds A row l%16 / B column l%16 at columns 8(l/16)..+8, and C column
// l%16 (a weight row) at tokens 4(l/16)..+4, so the lane that unpacks weight row
// n also owns that row's outputs and scales.  Each wave keeps TT x GPW (token
// tile, 64-column group) pairs of x split into bf16 parts in registers and
// walks the workgroup's 16-row tiles, unpacking each weight once for its token
// tiles.  The WPB per-wave partial tiles are summed in wave order through LDS
// (deterministic).  When the columns need more than one workgroup (more than
// WPB x GPW groups) the column splits store partial sums that k_tok_reduce
// adds in split order.  Splitting the columns this way keeps the x each
// workgroup loads and splits to its own share, so the split work does not grow
// with the number of workgroups.
#include "g4_device.hpp"
#include "g4_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace g4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

constexpr int TOK_SLOTS = 4;  // (token tile, 64-column group) pairs a wave can keep split in registers

// x = p1 + p2 + p3 exactly: p1 and p2 are the bf16 truncations of x and of
// x - p1 (their top 8 significant bits), x - p1 - p2 has at most 8 significant
// bits, and both differences are exact in fp32.  Truncation keeps every part of
// a finite x finite.  GUARD: an infinite x stays in p1 with zero residuals;
// without it x - p1 is NaN there, which the caller detects.  A NaN x gives NaN
// parts either way.
template <bool GUARD>
G4_DEV void split3(const float (&v)[8], bf16x8 &p1, bf16x8 &p2, bf16x8 &p3) {
  uint32_t t1[8], t2[8], t3[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    t1[e] = __float_as_uint(v[e]) & 0xFFFF0000u;
    float r1 = v[e] - __uint_as_float(t1[e]);
    if (GUARD) r1 = __builtin_isinf(v[e]) ? 0.f : r1;
    t2[e] = __float_as_uint(r1) & 0xFFFF0000u;
    t3[e] = __float_as_uint(r1 - __uint_as_float(t2[e]));
  }
  // two values' upper halves per dword (v_perm_b32)
  u32x4 a, b, c;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a[k] = __builtin_amdgcn_perm(t1[2 * k + 1], t1[2 * k], 0x07060302u);
    b[k] = __builtin_amdgcn_perm(t2[2 * k + 1], t2[2 * k], 0x07060302u);
    c[k] = __builtin_amdgcn_perm(t3[2 * k + 1], t3[2 * k], 0x07060302u);
  }
  p1 = __builtin_bit_cast(bf16x8, a);
  p2 = __builtin_bit_cast(bf16x8, b);
  p3 = __builtin_bit_cast(bf16x8, c);
}

// split3 for four values: parts p = 0, 1, 2 as two dwords each (values 0, 1
// and 2, 3 in the low and high halves), the same parts as split3 gives
template <bool GUARD>
G4_DEV void split3_4(const float (&v)[4], u32x2a4 (&pt)[3]) {
  uint32_t t1[4], t2[4], t3[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    t1[e] = __float_as_uint(v[e]) & 0xFFFF0000u;
    float r1 = v[e] - __uint_as_float(t1[e]);
    if (GUARD) r1 = __builtin_isinf(v[e]) ? 0.f : r1;
    t2[e] = __float_as_uint(r1) & 0xFFFF0000u;
    t3[e] = __float_as_uint(r1 - __uint_as_float(t2[e]));
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    pt[0][k] = __builtin_amdgcn_perm(t1[2 * k + 1], t1[2 * k], 0x07060302u);
    pt[1][k] = __builtin_amdgcn_perm(t2[2 * k + 1], t2[2 * k], 0x07060302u);
    pt[2][k] = __builtin_amdgcn_perm(t3[2 * k + 1], t3[2 * k], 0x07060302u);
  }
}

// bf16 of 16(q - 8) for the 8 nibbles of one K-slice.  A nibble q moved to the
// top of its byte and xored with 0x80 is the signed byte 16(q - 8); it converts
// to float with one sign-extending byte select and to bf16 exactly.
G4_DEV uint32_t lo_nibbles_s16(uint32_t w) { return ((w << 4) & 0xF0F0F0F0u) ^ 0x80808080u; }
G4_DEV uint32_t hi_nibbles_s16(uint32_t w) { return (w & 0xF0F0F0F0u) ^ 0x80808080u; }
G4_DEV bf16x8 nibbles_bf16(uint32_t v0, uint32_t v1) {
  bf16x8 r;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    r[b] = (__bf16)sbyte(v0, b);
    r[4 + b] = (__bf16)sbyte(v1, b);
  }
  return r;
}

// bf16 of 16 q for the 8 nibbles of one K-slice, two per instruction: a nibble
// byte q (0..15) is the e4m3 code of q * 2^-9 (the subnormal codes and the
// first normal binade are exactly linear in the code), converted with the scale
// 2^13.  c0, c1: four nibble bytes each, in column order.
G4_DEV bf16x8 codes_bf16_16q(uint32_t c0, uint32_t c1) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c0, 8192.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c0, 8192.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c1, 8192.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c1, 8192.0f, true);
  return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// sc and m of sub-blocks 2(g & 3) and 2(g & 3) + 1 of a super-block head, in
// bytes 0 and 1 (getScaleMinK4, Q4_KFloatTensor.kt:70-84)
G4_DEV void scale_min_pair(const u32x4 &H, int g, uint32_t &scp, uint32_t &mp) {
  const uint32_t sh = (uint32_t)(g & 1) * 16u;
  const uint32_t y = H.y >> sh, z = H.z >> sh, w = H.w >> sh;
  scp = g < 2 ? (y & 0x3F3Fu) : ((w & 0x0F0Fu) | ((y >> 2) & 0x3030u));
  mp = g < 2 ? (z & 0x3F3Fu) : (((w >> 4) & 0x0F0Fu) | ((z >> 2) & 0x3030u));
}

// sc and m of sub-blocks 4 hq .. 4 hq + 3 (hq = 0, 1), in bytes 0..3
G4_DEV void scale_min_quad(const u32x4 &H, int hq, uint32_t &scq, uint32_t &mq) {
  if (hq == 0) {
    scq = H.y & 0x3F3F3F3Fu;
    mq = H.z & 0x3F3F3F3Fu;
  } else {
    scq = (H.w & 0x0F0F0F0Fu) | ((H.y >> 2) & 0x30303030u);
    mq = ((H.w >> 4) & 0x0F0F0F0Fu) | ((H.z >> 2) & 0x30303030u);
  }
}

// Two 64-column groups per wave: four 32-weight sub-blocks, the K of one
// v_mfma_f32_16x16x4_f32, which adds each sub-block's (8 d*sc - dmin*m) sum(x)
// term for the 16 tokens and 16 rows of a tile in one instruction.
constexpr int TOK_GPW = 2;

// TT token tiles per wave: a workgroup of WPB waves covers WPB * TOK_GPW groups
// (its column split, blockIdx.y) for TT token tiles (token group blockIdx.z)
// over a range of 16-row tiles (blockIdx.x).  A wave unpacks each weight once
// for its TT token tiles.
// Per tile, lane (j, n) = (lane / 16, lane % 16) computes the scale of all four
// of the wave's sub-blocks for its row n (the products it owns are row n's) but
// the sum(x) coefficient only for sub-block j (the fp32 MFMA's B operand is
// coefficient[sub-block j][row n]); its A operand, the sum of x over sub-block
// j for token n, is formed once per wave.
// AL: base and row_stride are multiples of 256 (whole super-blocks per row, the
// usual case) and the groups come in pairs: a lane's weight address then moves
// by a fixed stride per row tile, and the wave's two groups lie in one
// super-block, whose head is loaded once and whose four sub-blocks' scales
// take wave-uniform byte positions.
// SUB8: the weight operand is 16 q from e4m3 codes (two per instruction), with
// sum(128 x) formed once per wave and subtracted per sub-block; else 16 (q - 8)
// from signed bytes (9 to 16 tokens in workgroups of few row tiles, where the
// per-wave sum(128 x) does not repay; with at most 8 tokens it does, its MFMAs
// running while the first tile's weights are in flight).
// FULL (with AL): every wave's column slice is whole and the row tiles are
// whole, so the slice and row checks drop out, and the output offsets within
// 16 tokens fit 32 bits.
template <int TT, int WPB, bool AL, bool HALF, bool SUB8, bool FULL>
__global__ __launch_bounds__(WPB * 64) void k_tok_q4k(TokArgs a) {
  static_assert(!FULL || AL, "FULL takes the AL layout");
  constexpr int GPW = TOK_GPW, NH = AL ? 1 : GPW;
  static_assert(TT * GPW <= TOK_SLOTS && WPB >= TT && WPB % TT == 0, "tile shape");
  static_assert(!HALF || TT == 1, "HALF: one token tile of at most 8 tokens");
  // LDS: first each wave's x slice (16 tokens x 128 columns, rows padded to
  // XROW floats so the reads below are conflict-free), then, after a barrier,
  // the cross-wave partial tiles
  // (and with AL each wave's staged weight tile, 16 rows x 80 bytes)
  constexpr int XROW = 132, WROW = 80;
  constexpr size_t RED_BYTES = sizeof(f32x4) * 2 * TT * WPB * 64, XST_BYTES = sizeof(float) * WPB * 16 * XROW;
  constexpr size_t WST_BYTES = AL ? (size_t)WPB * 16 * WROW : 0;
  __shared__ __attribute__((aligned(16))) unsigned char
      lds[RED_BYTES + WST_BYTES > XST_BYTES ? RED_BYTES + WST_BYTES : XST_BYTES];
  f32x4(*red)[TT][WPB][64] = (f32x4(*)[TT][WPB][64])lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, j = lane >> 4;
  const int C = a.dim1 >> 6;
  const int g0 = ((int)blockIdx.y * WPB + wid) * GPW;  // first group of this wave's slice (even)
  const int ng = FULL ? GPW : max(0, min(GPW, C - g0));      // wave-uniform
  const int tt0 = (int)blockIdx.z * TT;                      // first token tile
  const int n_rt = (a.rows + 15) >> 4;
  const int rpb = (n_rt + gridDim.x - 1) / gridDim.x;
  const int rt0 = min(n_rt, (int)blockIdx.x * rpb), rt1 = min(n_rt, rt0 + rpb);
  // one column split: y directly; several: this split's partial sums
  float *out = gridDim.y == 1 ? a.y : a.part + (int64_t)blockIdx.y * a.M * a.rows;
  const int64_t out_stride = gridDim.y == 1 ? a.y_stride : a.rows;
  int buf = 0;

  // weight group gi of row tile rt, this lane's row (B column n) and K-slice j:
  // 8 nibble bytes at qs[32 g + 8 j] and the super-block head
  // AL: super-block of row rt0 * 16 + n and the per-tile byte stride
  const int64_t rs_sb = a.row_stride >> 8;
  const uint8_t *w_row0 = a.W + ((a.base >> 8) + (int64_t)(rt0 * 16 + n) * rs_sb) * 144;
  const int64_t w_step = 16 * rs_sb * 144;
  auto load_w = [&](int rt, bool live, u32x2a4 (&Q)[GPW], u32x4 (&H)[NH], int (&gs)[GPW]) {
    const int r = rt * 16 + n;
    const bool rok = live && r < a.rows;
    if constexpr (AL) {
      // rows past the end read the tensor's first super-block
      const uint8_t *sb = rok && ng > 0 ? w_row0 + (int64_t)(rt - rt0) * w_step + (g0 >> 2) * 144 : a.W;
      H[0] = *(const u32x4 *)sb;
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi) {
        gs[gi] = (g0 + gi) & 3;  // wave-uniform
        Q[gi] = *(const u32x2a4 *)(sb + 16 + 32 * ((g0 + gi) & 3) + 8 * j);
      }
      return;
    }
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
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

  // AL: a tile's weights for this wave, 16 rows x (head + the wave's two
  // groups), read by four adjacent lanes per row (row lane / 4: bytes
  // 16 (lane % 4) of the 64 group bytes and dword lane % 4 of the head, where
  // loading them by row n = lane % 16 would put 16 rows 1152 bytes apart in
  // every instruction) and staged in the wave's own LDS rows, from where each
  // lane takes its row's head and its K-slice of both groups
  unsigned char *wst = lds + RED_BYTES + (size_t)wid * 16 * WROW;
  const uint8_t *w_tile0 = a.W + ((a.base >> 8) + (int64_t)(rt0 * 16 + (lane >> 2)) * rs_sb + (g0 >> 2)) * 144;
  const uint32_t lane_h = (uint32_t)((lane >> 2) * rs_sb * 144) + 4u * (lane & 3);
  const uint32_t lane_w = lane_h + 16u + 32u * (g0 & 3) + 12u * (lane & 3);
  auto load_raw = [&](int rt, bool live, u32x4 &QR, uint32_t &HR) {
    if constexpr (FULL && HALF) {
      // a wave-uniform tile base and this lane's 32-bit offset in it; a tile past
      // the end reads the matrix's first 16 rows.  (With more tokens this form
      // measured slower: 32 and 64 tokens 10.3/14.3 -> 10.5/15.1 us.)
      const uint8_t *tb = a.W + ((a.base >> 8) + (int64_t)((live ? rt : 0) * 16) * rs_sb + (g0 >> 2)) * 144;
      QR = *(const u32x4 *)(tb + lane_w);
      HR = *(const uint32_t *)(tb + lane_h);
      return;
    }
    // rows past the end read the tensor's first super-block
    const bool ok = live && ng > 0 && rt * 16 + (lane >> 2) < a.rows;
    const uint8_t *sb = ok ? w_tile0 + (int64_t)(rt - rt0) * w_step : a.W;
    QR = *(const u32x4 *)(sb + 16 + 32 * (g0 & 3) + 16 * (lane & 3));
    HR = *(const uint32_t *)(sb + 4 * (lane & 3));
  };
  auto stage = [&](const u32x4 &QR, uint32_t HR, u32x2a4 (&Q)[GPW], u32x4 (&H)[NH]) {
    unsigned char *wr = wst + (lane >> 2) * WROW;
    *(u32x4 *)(wr + 16 + 16 * (lane & 3)) = QR;
    *(uint32_t *)(wr + 4 * (lane & 3)) = HR;
    const unsigned char *rd = wst + n * WROW;
    H[0] = *(const u32x4 *)rd;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) Q[gi] = *(const u32x2a4 *)(rd + 16 + 32 * gi + 8 * j);
  };

  // x slice: 16 tokens x the wave's 128 columns, read so that adjacent lanes
  // take adjacent 16-byte pieces (each instruction two tokens' 512 contiguous
  // bytes: lane l takes piece l % 32 of token 2q + l / 32) and staged in LDS;
  // columns of groups past the slice come from group 0 (in bounds, never used);
  // HALF (at most 8 tokens): tokens 8..15 are not read but staged as zeros, so
  // the wave issues half the x loads
  u32x4a4 xg[TT][8];
#pragma unroll
  for (int ti = 0; ti < TT; ++ti)
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int tok = (tt0 + ti) * 16 + 2 * q + (lane >> 5), c = lane & 31, gi = c >> 4;
      const float *p = a.x + (int64_t)(tok < a.M ? tok : 0) * a.x_stride + (int64_t)(gi < ng ? g0 + gi : 0) * 64 + 4 * (c & 15);
      xg[ti][q] = (HALF && q >= 4) ? u32x4a4{0u, 0u, 0u, 0u} : *(const u32x4a4 *)p;
    }
  u32x2a4 QA[GPW], QB[GPW];
  u32x4 HA[NH], HB[NH];
  int GA[GPW], GB[GPW];
  u32x4 QRA, QRB;
  uint32_t HRA, HRB;
  // the first tile's weight loads go out behind the x loads and before any
  // use of x (vmcnt retires in order: the split below waits for x only)
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (AL)
    load_raw(rt0, rt0 < rt1, QRA, HRA);
  else
    load_w(rt0, rt0 < rt1, QA, HA, GA);
  __builtin_amdgcn_sched_barrier(0);

  float xsT[TT];
  bf16x8 A[TT][GPW][2][3];
  if constexpr (HALF) {
    // At most 8 tokens: the bf16 parts and the sub-block sums are formed from
    // the x the lanes loaded (tokens 0..7, four columns per lane), so no lane
    // works on the zero tokens 8..15, then staged in the wave's LDS as
    // [part][row][128 columns] (rows 0..7 the tokens, row 8 zeros for lanes
    // 8..15 of the MFMA layout) and read back in that layout.
    constexpr int XB = 272;                        // one row: 128 bf16 and 16 bytes of padding
    constexpr int XW = 3 * 9 * XB + 9 * 4 * 4;     // a wave's region: parts, then the sums [9][4]
    static_assert((size_t)WPB * XW <= XST_BYTES, "x staging");
    unsigned char *xp = lds + (size_t)wid * XW;
    float *sxt = (float *)(xp + 3 * 9 * XB);
    if (lane < 48) *(u32x4 *)(xp + (lane >> 4) * 9 * XB + 8 * XB + 16 * (lane & 15)) = u32x4{0u, 0u, 0u, 0u};
    if (lane == 48) *(u32x4 *)(sxt + 8 * 4) = u32x4{0u, 0u, 0u, 0u};
    // lane l holds columns 4c .. 4c + 3 (c = l % 32) of token 2q + l / 32: sub-block
    // c / 8, whose sum is over the 8 lanes of the group (every lane ends with it)
    const int c = lane & 31;
    bool bq = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float t = __uint_as_float(xg[0][q].x);
      t += __uint_as_float(xg[0][q].y);
      t += __uint_as_float(xg[0][q].z);
      t += __uint_as_float(xg[0][q].w);
      t = pstep<1>(t);
      t = pstep<2>(t);
      t = pstep<4>(t);
      if ((lane & 7) == 0) sxt[(2 * q + (lane >> 5)) * 4 + (c >> 3)] = t;
      bq |= !__builtin_isfinite(t);
    }
    // the split without the infinity guard runs unless some sum in the wave is
    // infinite or NaN (wave-uniform)
    auto split_store = [&](auto guard) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v[4] = {__uint_as_float(xg[0][q].x), __uint_as_float(xg[0][q].y), __uint_as_float(xg[0][q].z),
                            __uint_as_float(xg[0][q].w)};
        u32x2a4 pt[3];
        split3_4<decltype(guard)::value>(v, pt);
#pragma unroll
        for (int p = 0; p < 3; ++p) *(u32x2a4 *)(xp + p * 9 * XB + (2 * q + (lane >> 5)) * XB + 8 * c) = pt[p];
      }
    };
    if (__builtin_amdgcn_ballot_w64(bq) != 0)
      split_store(std::true_type());
    else
      split_store(std::false_type());
    const int row = n < 8 ? n : 8;
    xsT[0] = sxt[row * 4 + j];
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int p = 0; p < 3; ++p)
          A[0][gi][h][p] = *(const bf16x8 *)(xp + p * 9 * XB + row * XB + 2 * (64 * gi + 32 * h + 8 * j));
    __syncthreads();  // every wave has its x: the LDS now holds the partial tiles
  } else {
    // back from LDS in the MFMA layout: lane (j, n) takes token n, columns
    // 64 gi + 32 h + 8 j .. +8 of the slice (the K-slice j of sub-block (gi, h));
    // a wave reads only what it wrote, and LDS operations of a wave run in order
    u32x4a4 xr[TT][GPW][2][2];
    float *xst = (float *)lds + wid * 16 * XROW;
#pragma unroll
    for (int ti = 0; ti < TT; ++ti) {
#pragma unroll
      for (int q = 0; q < 8; ++q) *(u32x4 *)(xst + (2 * q + (lane >> 5)) * XROW + 4 * (lane & 31)) = xg[ti][q];
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int u = 0; u < 2; ++u) xr[ti][gi][h][u] = *(const u32x4 *)(xst + n * XROW + 64 * gi + 32 * h + 8 * j + 4 * u);
    }
    __syncthreads();  // every wave has its x: the LDS now holds the partial tiles

    // Per token tile, the sum of x over sub-block j (group j / 2, half j % 2) for
    // token n, the fp32 MFMA's A operand: each lane adds its 8 values of each
    // sub-block, and a transposing butterfly over the four K-slice lanes of the
    // token leaves sub-block j's sum in row j.  x is not masked: the tokens past M
    // (token 0's x) only reach their own output rows, which are never stored, and
    // groups past the slice are never multiplied and get no coefficient.
    bool bad = false;
#pragma unroll
    for (int ti = 0; ti < TT; ++ti) {
      float ps[2 * GPW];
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float t = __uint_as_float(xr[ti][gi][h][0].x);
          t += __uint_as_float(xr[ti][gi][h][0].y);
          t += __uint_as_float(xr[ti][gi][h][0].z);
          t += __uint_as_float(xr[ti][gi][h][0].w);
          t += __uint_as_float(xr[ti][gi][h][1].x);
          t += __uint_as_float(xr[ti][gi][h][1].y);
          t += __uint_as_float(xr[ti][gi][h][1].z);
          t += __uint_as_float(xr[ti][gi][h][1].w);
          ps[2 * gi + h] = t;
        }
      static_assert(GPW == 2, "four sub-blocks per wave");
      const float t02 = tstep<32>(ps[0], ps[2], lane), t13 = tstep<32>(ps[1], ps[3], lane);
      xsT[ti] = tstep<16>(t02, t13, lane);
      bad |= !__builtin_isfinite(xsT[ti]);
    }
    // bf16 parts (A operands).  The split without the infinity guard runs unless
    // some sum in the wave is infinite or NaN (an activation is, or a sum
    // overflowed): wave-uniform
    auto split_all = [&](auto guard) {
#pragma unroll
      for (int ti = 0; ti < TT; ++ti)
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              v[4 * u] = __uint_as_float(xr[ti][gi][h][u].x);
              v[4 * u + 1] = __uint_as_float(xr[ti][gi][h][u].y);
              v[4 * u + 2] = __uint_as_float(xr[ti][gi][h][u].z);
              v[4 * u + 3] = __uint_as_float(xr[ti][gi][h][u].w);
            }
            split3<decltype(guard)::value>(v, A[ti][gi][h][0], A[ti][gi][h][1], A[ti][gi][h][2]);
          }
    };
    if (__builtin_amdgcn_ballot_w64(bad) != 0)
      split_all(std::true_type());
    else
      split_all(std::false_type());
  }
#pragma unroll
  for (int ti = 0; ti < TT; ++ti)
    if ((j >> 1) >= ng) xsT[ti] = 0.f;  // a group past the slice
  // SUB8: sum(128 x) of each sub-block with the MFMAs the tiles use (B = 128 is
  // the weight operand of an all-8 sub-block, bit for bit), subtracted from
  // each tile's sum(16 q x) before its scale
  f32x4 S8[SUB8 ? TT : 1][SUB8 ? GPW : 1][2];
  if constexpr (SUB8) {
    bf16x8 b128;
#pragma unroll
    for (int e = 0; e < 8; ++e) b128[e] = (__bf16)128.0f;
#pragma unroll
    for (int ti = 0; ti < TT; ++ti)
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          S8[ti][gi][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int p = 0; p < 3; ++p)
            S8[ti][gi][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[ti][gi][h][p], b128, S8[ti][gi][h], 0, 0, 0);
        }
  }

  // mid() runs between the partial tile's LDS store and the barrier
  auto tile = [&](int rt, const u32x2a4 (&Q)[GPW], const u32x4 (&H)[NH], const int (&gs)[GPW], auto &&mid) {
    f32x4 acc[TT];
#pragma unroll
    for (int ti = 0; ti < TT; ++ti) acc[ti] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (ng > 0) {  // wave-uniform
      // d*sc/16 of the four sub-blocks s (group s / 2, half s % 2) of row n, and
      // 8 d*sc - dmin*m of sub-block j; d*sc is exact (11 x 6 bits), so is
      // 8 d*sc = 128 (d*sc/16)
      float d1[2 * GPW], cj;
      if constexpr (AL) {
        const float dq = h2f(H[0].x & 0xFFFFu) * 0.0625f, dmin = h2f(H[0].x >> 16);
        uint32_t scq, mq;
        scale_min_quad(H[0], (g0 & 3) >> 1, scq, mq);
#pragma unroll
        for (int s = 0; s < 4; ++s) d1[s] = dq * ubyte(scq, s);
        const float scj = (float)((scq >> (8 * j)) & 0xFFu), mj = (float)((mq >> (8 * j)) & 0xFFu);
        cj = __builtin_fmaf(128.f, dq * scj, -(dmin * mj));
      } else {
        float cc[GPW][2];
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
          uint32_t scp, mp;
          scale_min_pair(H[gi], gs[gi], scp, mp);
          const float dq = h2f(H[gi].x & 0xFFFFu) * 0.0625f, dmin = h2f(H[gi].x >> 16);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            d1[2 * gi + h] = dq * ubyte(scp, h);
            cc[gi][h] = __builtin_fmaf(128.f, d1[2 * gi + h], -(dmin * ubyte(mp, h)));
          }
        }
        const float c0 = (j & 1) ? cc[0][1] : cc[0][0], c1 = (j & 1) ? cc[1][1] : cc[1][0];
        // a group past the slice has the tensor's first head: no coefficient
        cj = (j >> 1) >= ng ? 0.f : ((j >> 1) ? c1 : c0);
      }
      // every product first, then the fp32 MFMA of the sum(x) terms, then the
      // scales: the matrix core works through the independent chains
      f32x4 P[TT][GPW][2];
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi) {
        if (gi < ng) {  // wave-uniform
          const uint32_t w0 = Q[gi].x, w1 = Q[gi].y;
          bf16x8 bl, bh;
          if constexpr (SUB8) {
            bl = codes_bf16_16q(opaque(w0 & 0x0F0F0F0Fu), opaque(w1 & 0x0F0F0F0Fu));
            bh = codes_bf16_16q(opaque((w0 >> 4) & 0x0F0F0F0Fu), opaque((w1 >> 4) & 0x0F0F0F0Fu));
          } else {
            bl = nibbles_bf16(opaque(lo_nibbles_s16(w0)), opaque(lo_nibbles_s16(w1)));
            bh = nibbles_bf16(opaque(hi_nibbles_s16(w0)), opaque(hi_nibbles_s16(w1)));
          }
#pragma unroll
          for (int ti = 0; ti < TT; ++ti) P[ti][gi][0] = P[ti][gi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int ti = 0; ti < TT; ++ti) {
              P[ti][gi][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[ti][gi][0][p], bl, P[ti][gi][0], 0, 0, 0);
              P[ti][gi][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[ti][gi][1][p], bh, P[ti][gi][1], 0, 0, 0);
            }
        }
      }
#pragma unroll
      for (int ti = 0; ti < TT; ++ti) acc[ti] = __builtin_amdgcn_mfma_f32_16x16x4f32(xsT[ti], cj, acc[ti], 0, 0, 0);
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi)
        if (gi < ng)
#pragma unroll
          for (int ti = 0; ti < TT; ++ti)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if constexpr (SUB8) {
                acc[ti][i] = __builtin_fmaf(d1[2 * gi], P[ti][gi][0][i] - S8[ti][gi][0][i], acc[ti][i]);
                acc[ti][i] = __builtin_fmaf(d1[2 * gi + 1], P[ti][gi][1][i] - S8[ti][gi][1][i], acc[ti][i]);
              } else {
                acc[ti][i] = __builtin_fmaf(d1[2 * gi], P[ti][gi][0][i], acc[ti][i]);
                acc[ti][i] = __builtin_fmaf(d1[2 * gi + 1], P[ti][gi][1][i], acc[ti][i]);
              }
            }
    }
    // the WPB column slices are summed in wave order (deterministic), the work
    // spread over the waves: wave w takes token tile w / (WPB / TT)'s components
    // i = c, c + WPB/TT, ... of every lane's 4 outputs (c = w % (WPB / TT))
#pragma unroll
    for (int ti = 0; ti < TT; ++ti) red[buf][ti][wid][lane] = acc[ti];
    mid();
    __syncthreads();
    {
      constexpr int WPT = WPB / TT;  // waves per token tile
      const int ti = wid / WPT, c = wid % WPT;
      const int r = rt * 16 + n;
      if constexpr (FULL && WPT >= 4) {
        if (c < 4) {  // wave-uniform: component c of every lane's four outputs
          const float *rp = (const float *)&red[buf][ti][0][lane] + c;
          float s = rp[0];
#pragma unroll
          for (int w = 1; w < WPB; ++w) s += rp[w * 64 * 4];
          const int m = (tt0 + ti) * 16 + 4 * j + c;
          float *ob = out + ((int64_t)((tt0 + ti) * 16 + c) * out_stride + rt * 16);
          if (m < a.M) ob[(uint32_t)(4 * j * out_stride + n)] = s;
        }
      } else
      for (int i = c; i < 4; i += WPT) {  // wave-uniform: one component per read, no selects
        const float *rp = (const float *)&red[buf][ti][0][lane] + i;
        float s = rp[0];
#pragma unroll
        for (int w = 1; w < WPB; ++w) s += rp[w * 64 * 4];
        const int m = (tt0 + ti) * 16 + 4 * j + i;
        if (r < a.rows && m < a.M) out[(int64_t)m * out_stride + r] = s;
      }
    }
    buf ^= 1;
  };

  if constexpr (AL) {
    // tile t+1's weights load while tile t multiplies, and are staged between
    // tile t's partial store and its barrier
    stage(QRA, HRA, QA, HA);
    for (int rt = rt0; rt < rt1; rt += 2) {
      load_raw(rt + 1, rt + 1 < rt1, QRB, HRB);
      __builtin_amdgcn_sched_barrier(0);
      tile(rt, QA, HA, GA, [&] { stage(QRB, HRB, QA, HA); });
      __builtin_amdgcn_sched_barrier(0);
      load_raw(rt + 2, rt + 2 < rt1, QRA, HRA);
      __builtin_amdgcn_sched_barrier(0);
      if (rt + 1 < rt1) tile(rt + 1, QA, HA, GA, [&] { stage(QRA, HRA, QA, HA); });
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    // two row tiles in flight: tile t+1 loads while tile t multiplies
    for (int rt = rt0; rt < rt1; rt += 2) {
      load_w(rt + 1, rt + 1 < rt1, QB, HB, GB);
      __builtin_amdgcn_sched_barrier(0);
      tile(rt, QA, HA, GA, [] {});
      __builtin_amdgcn_sched_barrier(0);
      load_w(rt + 2, rt + 2 < rt1, QA, HA, GA);
      __builtin_amdgcn_sched_barrier(0);
      if (rt + 1 < rt1) tile(rt + 1, QB, HB, GB, [] {});
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// y[m * y_stride + r] = sum over the column splits, in split order, of their
// partial sums.  Thread t of workgroup (bx, m) covers V consecutive rows from
// V * (256 bx + t) of token m; the loads of up to 8 splits are all in flight
// before the first add.
template <int V>
__global__ __launch_bounds__(256) void k_tok_reduce(const float *part, int splits, int32_t M, int32_t rows, float *y,
                                                    int64_t y_stride) {
  typedef float fv __attribute__((ext_vector_type(V)));
  const int r = (blockIdx.x * 256 + threadIdx.x) * V, m = blockIdx.y;
  if (r >= rows) return;
  const int64_t n = (int64_t)M * rows, i = (int64_t)m * rows + r;
  fv s = *(const fv *)(part + i);
  for (int k0 = 1; k0 < splits; k0 += 8) {
    fv v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = *(const fv *)(part + (int64_t)min(k0 + k, splits - 1) * n + i);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (k0 + k < splits) s += v[k];
  }
  *(fv *)(y + (int64_t)m * y_stride + r) = s;
}

// Launch shape: one 16-token tile and two 64-column groups per wave, 16
// waves per workgroup (four per SIMD at <= 128 VGPRs), one workgroup per CU:
// a workgroup covers 2048 columns.  Measured over 1/2/4 token tiles, 1/2/4
// groups and 4/8/16 waves for M = 8..64 at 8192 x 2048, this shape was the
// fastest or within 2% at every M, and it needs no column split up to 2048
// columns.
constexpr int TOK_TT = 1, TOK_WPB = 16;

struct TokShape {
  int splits, tgroups, gx;
};

static TokShape tok_shape(const TokArgs &a, const DevInfo &dev) {
  TokShape sh;
  const int C = a.dim1 / 64;
  const int ntt = (a.M + 15) / 16;
  const int gps = TOK_WPB * TOK_GPW;  // groups per column split
  sh.splits = (C + gps - 1) / gps;
  sh.tgroups = (ntt + TOK_TT - 1) / TOK_TT;
  // one workgroup per CU at a time, spread over every (split, token group)
  const int n_rt = (a.rows + 15) / 16;
  int64_t gx = (int64_t)dev.cu_count / ((int64_t)sh.splits * sh.tgroups);
  if (gx > n_rt) gx = n_rt;
  if (gx < 1) gx = 1;
  sh.gx = (int)gx;
  return sh;
}

bool tok_ok(int type, const TokArgs &a) {
  if (type != T_Q4_K) return false;
  if (a.dim1 <= 0 || (a.dim1 % 64) != 0) return false;
  if ((a.base % 64) != 0 || (a.row_stride % 64) != 0) return false;
  return a.M >= 1 && a.rows >= 1;
}

int64_t tok_scratch_floats(const TokArgs &a, const DevInfo &dev) {
  const TokShape sh = tok_shape(a, dev);
  return sh.splits > 1 ? (int64_t)sh.splits * a.M * a.rows : 0;
}

hipError_t launch_tok(int type, const TokArgs &a, const DevInfo &dev, hipStream_t s) {
  if (!tok_ok(type, a)) return hipErrorInvalidValue;
  const TokShape sh = tok_shape(a, dev);
  if (sh.splits > 1 && !a.part) return hipErrorInvalidValue;
  const dim3 grid((unsigned)sh.gx, (unsigned)sh.splits, (unsigned)sh.tgroups);
  // whole super-blocks per row and an even number of groups: every wave's two
  // groups lie in one super-block
  // at most 8 tokens: the x loads of tokens 8..15 are left out
  const bool al = (a.base % 256) == 0 && (a.row_stride % 256) == 0 && (a.dim1 % 128) == 0, half = a.M <= 8;
  // the 16 q operand from four row tiles per workgroup on (8192 x 2048: 32 and 64
  // tokens 10.58/15.23 -> 10.42/14.73 us; 16 tokens, two tiles, 8.27 -> 8.35),
  // and with at most 8 tokens (7.13 -> 6.86 us)
  const int n_rt = (a.rows + 15) / 16, rpb = (n_rt + sh.gx - 1) / sh.gx;
  const bool sub8 = half || rpb >= 4;
  // FULL: whole slices and row tiles, 32-bit offsets within a tile and within 16
  // tokens of the output (8 / 32 / 64 tokens 6.86 / 10.49 / 14.75 -> 6.77 / 10.24 /
  // 14.29 us)
  const int64_t ost = sh.splits == 1 ? a.y_stride : a.rows;
  const bool full = al && (a.dim1 % (64 * TOK_GPW * TOK_WPB)) == 0 && (a.rows % 16) == 0 &&
                    16 * (a.row_stride / 256) * 144 < (1ll << 31) && 16 * ost < (1ll << 29);
  if (full && half)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, true, true, true, true>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else if (full && sub8)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, true, false, true, true>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else if (full)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, true, false, false, true>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else if (al && half)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, true, true, true, false>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else if (al && sub8)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, true, false, true, false>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else if (al)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, true, false, false, false>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else if (half)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, false, true, true, false>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else if (sub8)
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, false, false, true, false>), grid, dim3(TOK_WPB * 64), 0, s, a);
  else
    hipLaunchKernelGGL((k_tok_q4k<TOK_TT, TOK_WPB, false, false, false, false>), grid, dim3(TOK_WPB * 64), 0, s, a);
  if (sh.splits == 1) return hipGetLastError();
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // four rows per thread when every row quad and its output are 16-byte aligned
  // (the scratch is; y depends on the caller)
  if ((a.rows % 4) == 0 && (a.y_stride % 4) == 0 && ((uintptr_t)a.y & 15) == 0)
    hipLaunchKernelGGL(k_tok_reduce<4>, dim3((unsigned)((a.rows / 4 + 255) / 256), (unsigned)a.M), dim3(256), 0, s,
                       (const float *)a.part, sh.splits, a.M, a.rows, a.y, a.y_stride);
  else
    hipLaunchKernelGGL(k_tok_reduce<1>, dim3((unsigned)((a.rows + 255) / 256), (unsigned)a.M), dim3(256), 0, s,
                       (const float *)a.part, sh.splits, a.M, a.rows, a.y, a.y_stride);
  return hipGetLastError();
}

// ------------------------------------------------------------ grouped MoE ----
// The routed experts of a multi-token MoE call (Llama.kt:300-337 runs expert
// ids[p] on the x of token p / K for every (token, slot) pair p), grouped by
// expert: each expert's Q4_K weights are read and unpacked once for all of its
// pairs, on the matrix cores with the exact 3 x bf16 products of k_tok_q4k.
//
// Workgroup (x, e) takes expert e's pairs (ids[p] == e, in pair order) eight at
// a time.  Their x rows are split into bf16 parts once, into LDS, in the MFMA
// operand layout.  Pair slot t fills A rows 2t and 2t + 1 (the same x twice),
// so C rows 4j and 4j + 2, outputs 0 and 2 of the four lane (j, n) holds, are
// pair slots 2j and 2j + 1: every lane ends with two outputs per weight row, with
// no shuffle.
// Each wave walks units of two 16-row tiles (the gate and the up tile of the
// same rows, or two consecutive tiles) over all the columns, 128 at a time
// (four 32-weight sub-blocks, one fp32 MFMA for their (8 d*sc - dmin*m) sum(x)
// terms).  The sums stay in registers, so there is no cross-wave reduction.
// Workgroups (x, n_experts) write the zero rows of pairs whose id is out of
// range.
constexpr int MG_TOK = 8;        // pairs per pass (MFMA rows 16 / MG_TOK per pair)
constexpr int MG_RPS = 16 / MG_TOK, MG_NOUT = MG_TOK / 4;  // A rows per pair, outputs per lane
constexpr int MG_SBS = 3 * 4 * MG_TOK;  // 16-byte LDS operands per sub-block: parts x K-slices x pairs
constexpr int MG_WPB = 8;        // waves per workgroup
constexpr int MG_UPW = 2;        // units per wave
constexpr int MG_DEPTH = 2;      // chunks of weights in registers (MG_DEPTH - 1 in flight)
constexpr int MG_MAX_S = 4096;   // pairs every workgroup scans
constexpr int MG_MAX_DIM1 = 3072;  // columns: the LDS operands of eight pairs fit in 150 KB

// sc and m of sub-blocks 4 hq .. 4 hq + 3 for a per-lane hq, in bytes 0..3
G4_DEV void scale_min_quad_sel(const u32x4 &H, int hq, uint32_t &scq, uint32_t &mq) {
  const uint32_t s0 = H.y & 0x3F3F3F3Fu, m0 = H.z & 0x3F3F3F3Fu;
  const uint32_t s1 = (H.w & 0x0F0F0F0Fu) | ((H.y >> 2) & 0x30303030u);
  const uint32_t m1 = ((H.w >> 4) & 0x0F0F0F0Fu) | ((H.z >> 2) & 0x30303030u);
  scq = hq ? s1 : s0;
  mq = hq ? m1 : m0;
}

static size_t mg_lds_bytes(int dim1) {
  const size_t nsb = (size_t)(dim1 >> 5);
  return nsb * MG_SBS * sizeof(u32x4) + nsb * MG_TOK * sizeof(float);
}

template <bool GU>
__global__ __launch_bounds__(MG_WPB * 64) void k_moe_grp(MoeGrpArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char mg_lds[];
  __shared__ int pl[MG_TOK];     // the pass's pairs (-1: none)
  __shared__ int wcnt[MG_WPB];   // matches per wave in a scan step
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, j = lane >> 4;
  const int e = blockIdx.y;
  const bool zero_rows = e == a.n_experts;
  const int NSB = a.dim1 >> 5, NCH = a.dim1 >> 7;
  u32x4 *xp = (u32x4 *)mg_lds;                                       // [NSB][3 parts][4 K-slices][MG_TOK slots]
  float *xs = (float *)(mg_lds + (size_t)NSB * MG_SBS * sizeof(u32x4));  // [NSB][MG_TOK slots]
  constexpr int UR = GU ? 16 : 32;  // rows per unit
  const int units = (a.rows + UR - 1) / UR;
  const int u_lo = (int)blockIdx.x * MG_UPW * MG_WPB, u_hi = min(units, u_lo + MG_UPW * MG_WPB);
  const int64_t eoff = zero_rows ? 0 : (int64_t)e * a.expert_stride;

  // pairs of rank MG_TOK pass .. MG_TOK (pass + 1) - 1 among this workgroup's into pl; returns
  // the number of its pairs (the same in every thread)
  auto scan = [&](int pass) {
    if (tid < MG_TOK) pl[tid] = -1;
    int total = 0;
    for (int p0 = 0; p0 < a.S; p0 += MG_WPB * 64) {
      const int p = p0 + tid;
      bool m = false;
      if (p < a.S) {
        const int id = a.ids[p];
        m = zero_rows ? (id < 0 || id >= a.n_experts) : id == e;
      }
      const uint64_t b = __builtin_amdgcn_ballot_w64(m);
      if (lane == 0) wcnt[wid] = __builtin_popcountll(b);
      __syncthreads();
      int before = total, all = 0;
#pragma unroll
      for (int w = 0; w < MG_WPB; ++w) {
        before += w < wid ? wcnt[w] : 0;
        all += wcnt[w];
      }
      const int rank = before + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
      if (m && rank >= MG_TOK * pass && rank < MG_TOK * (pass + 1)) pl[rank - MG_TOK * pass] = p;
      total += all;
      __syncthreads();  // wcnt is rewritten next step; pl is complete after the last
    }
    return total;
  };

  for (int pass = 0;; ++pass) {
    if (pass > 0) __syncthreads();  // every wave has stored the previous pass's rows
    const int total = scan(pass);
    const int cnt = min(MG_TOK, total - MG_TOK * pass);
    if (cnt <= 0) return;
    if (zero_rows) {
      for (int i = tid; i < cnt * (u_hi - u_lo) * UR; i += MG_WPB * 64) {
        const int t = i / ((u_hi - u_lo) * UR), r = u_lo * UR + i % ((u_hi - u_lo) * UR);
        if (r < a.rows) a.y[(int64_t)pl[t] * a.y_stride + r] = 0.f;
      }
      continue;
    }

    // x of the pass's pairs in 8-column pieces (slot t, sub-block s, K-slice q):
    // the three bf16 parts (with the infinity guard) and, over the four
    // K-slices of a sub-block (four adjacent lanes), the sub-block's sum
    for (int o = tid; o < 4 * MG_TOK * NSB; o += MG_WPB * 64) {
      const int t = o / (4 * NSB), rem = o - t * 4 * NSB, s = rem >> 2, q = rem & 3;
      const int p = pl[t];
      float v[8];
      if (p >= 0) {
        const u32x4a4 *src = (const u32x4a4 *)(a.x + (int64_t)(p / a.x_div) * a.x_stride + 32 * s + 8 * q);
        const u32x4a4 lo = src[0], hi = src[1];
        v[0] = __uint_as_float(lo.x), v[1] = __uint_as_float(lo.y), v[2] = __uint_as_float(lo.z);
        v[3] = __uint_as_float(lo.w), v[4] = __uint_as_float(hi.x), v[5] = __uint_as_float(hi.y);
        v[6] = __uint_as_float(hi.z), v[7] = __uint_as_float(hi.w);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.f;
      }
      bf16x8 p1, p2, p3;
      split3<true>(v, p1, p2, p3);
      u32x4 *d = xp + (size_t)s * MG_SBS + q * MG_TOK + t;
      d[0] = __builtin_bit_cast(u32x4, p1);
      d[4 * MG_TOK] = __builtin_bit_cast(u32x4, p2);
      d[8 * MG_TOK] = __builtin_bit_cast(u32x4, p3);
      float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
      sum = pstep<1>(sum);
      sum = pstep<2>(sum);
      if (q == 0) xs[s * MG_TOK + t] = sum;
    }
    __syncthreads();

    const int slot = n / MG_RPS;  // the pair slot whose x this lane's A rows carry
    int pj[MG_NOUT];              // the pairs of this lane's outputs (-1: none)
#pragma unroll
    for (int v = 0; v < MG_NOUT; ++v) pj[v] = pl[j * MG_NOUT + v];
    for (int k = 0; k < MG_UPW; ++k) {
      const int u = u_lo + k * MG_WPB + wid;
      if (u >= u_hi) break;  // wave-uniform
      // this lane's row of the two tiles; rows past the end read the tensor's
      // first super-blocks (in bounds, never stored)
      const int r0 = u * UR + n, r1 = GU ? r0 : r0 + 16;
      const bool ok0 = r0 < a.rows, ok1 = r1 < a.rows;
      const int64_t E0 = ok0 ? eoff + a.base0 + (int64_t)r0 * a.row_stride : 0;
      const int64_t E1 = ok1 ? eoff + (GU ? a.base1 : a.base0) + (int64_t)r1 * a.row_stride : 0;
      const uint8_t *sb0 = a.W + (E0 >> 8) * 144, *sb1 = a.W + (E1 >> 8) * 144;
      const int h0 = (int)(E0 >> 7) & 1, h1 = (int)(E1 >> 7) & 1;
      // chunk c of a row starting at half h: super-block (h + c) / 2, half (h + c) % 2
      auto load = [&](int c, const uint8_t *sb, int h, u32x4 &H, u32x2a4 &Q0, u32x2a4 &Q1) {
        const uint8_t *b = sb + ((h + c) >> 1) * 144;
        const int hq = (h + c) & 1;
        H = *(const u32x4 *)b;
        Q0 = *(const u32x2a4 *)(b + 16 + 64 * hq + 8 * j);
        Q1 = *(const u32x2a4 *)(b + 48 + 64 * hq + 8 * j);
      };
      // the weights of MG_DEPTH chunks: MG_DEPTH - 1 load while one multiplies
      struct Wt {
        u32x4 H0, H1;
        u32x2a4 Q0[2], Q1[2];
      };
      auto load2 = [&](int c, Wt &w) {
        c = min(c, NCH - 1);  // past the end: the last chunk again (in bounds, unused)
        load(c, sb0, h0, w.H0, w.Q0[0], w.Q0[1]);
        load(c, sb1, h1, w.H1, w.Q1[0], w.Q1[1]);
      };
      Wt W[MG_DEPTH];
#pragma unroll
      for (int i = 0; i + 1 < MG_DEPTH; ++i) load2(i, W[i]);
      f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};

      // one tile's four sub-blocks of chunk c: scales, unpacked nibbles and products
      auto tile = [&](int c, int h, const u32x4 &H, const u32x2a4 (&Q)[2], const bf16x8 (&A)[4][3], float xsA,
                      f32x4 &acc) {
        const int hq = (h + c) & 1;
        uint32_t scq, mq;
        scale_min_quad_sel(H, hq, scq, mq);
        const float dq = h2f(H.x & 0xFFFFu) * 0.0625f, dmin = h2f(H.x >> 16);
        const float scj = (float)((scq >> (8 * j)) & 0xFFu), mj = (float)((mq >> (8 * j)) & 0xFFu);
        const float cj = __builtin_fmaf(128.f, dq * scj, -(dmin * mj));
        f32x4 P[4];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const uint32_t w0 = Q[g].x, w1 = Q[g].y;
          const bf16x8 bl = nibbles_bf16(opaque(lo_nibbles_s16(w0)), opaque(lo_nibbles_s16(w1)));
          const bf16x8 bh = nibbles_bf16(opaque(hi_nibbles_s16(w0)), opaque(hi_nibbles_s16(w1)));
          P[2 * g] = P[2 * g + 1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int p = 0; p < 3; ++p) {
            P[2 * g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2 * g][p], bl, P[2 * g], 0, 0, 0);
            P[2 * g + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[2 * g + 1][p], bh, P[2 * g + 1], 0, 0, 0);
          }
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xsA, cj, acc, 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float d1 = dq * ubyte(scq, s);
#pragma unroll
          for (int v = 0; v < MG_NOUT; ++v) acc[v * MG_RPS] = __builtin_fmaf(d1, P[s][v * MG_RPS], acc[v * MG_RPS]);
        }
      };

      // chunk c's products for both tiles (the x operands read once)
      auto chunk = [&](int c, const Wt &w) {
        bf16x8 A[4][3];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int p = 0; p < 3; ++p)
            A[s][p] = __builtin_bit_cast(bf16x8, xp[(size_t)(4 * c + s) * MG_SBS + (p * 4 + j) * MG_TOK + slot]);
        const float xsA = xs[(4 * c + j) * MG_TOK + slot];
        tile(c, h0, w.H0, w.Q0, A, xsA, acc0);
        tile(c, h1, w.H1, w.Q1, A, xsA, acc1);
      };
      // unrolled by the ring size, so every buffer index is a constant
      for (int c0 = 0; c0 < NCH; c0 += MG_DEPTH) {
#pragma unroll
        for (int i = 0; i < MG_DEPTH; ++i) {
          if (c0 + i >= NCH) break;  // wave-uniform
          load2(c0 + i + MG_DEPTH - 1, W[(i + MG_DEPTH - 1) % MG_DEPTH]);
          chunk(c0 + i, W[i]);
        }
      }
#pragma unroll
      for (int v = 0; v < MG_NOUT; ++v) {
        if (pj[v] < 0) continue;
        float *yp = a.y + (int64_t)pj[v] * a.y_stride;
        if constexpr (GU) {
          if (ok0) yp[r0] = gelu_ref(acc0[v * MG_RPS]) * acc1[v * MG_RPS];
        } else {
          if (ok0) yp[r0] = acc0[v * MG_RPS];
          if (ok1) yp[r1] = acc1[v * MG_RPS];
        }
      }
    }
  }
}

// -------------------------------------------- grouped MoE, 16-pair tiles ----
// The experts of a multi-token MoE call on k_tok_q4k's tiles.  Workgroup (row
// block, expert e) takes e's (token, slot) pairs sixteen at a time in pair order
// (a pass): pair slot t is MFMA row t, its token's x split into bf16 parts in the
// waves' registers as a 16-token tile (wave w: columns 128 w .. 128 w + 127), and
// the workgroup walks its 16-row tiles with the 16 q weight operands, each weight
// read once per pass.  Row r of pair p goes to y[p * y_stride + r]; the gate+up
// launch runs the expert's gate and up rows as one matrix of 2 ff rows (its two
// halves adjacent in the slab) and k_gelu_mul forms h.  Workgroups (x,
// n_experts) write the zero rows of pairs whose id is out of range.  Rows of up
// to 2048 columns: one column split, no partial sums.
constexpr int GT_WPB = 16;
// row blocks per expert: this many per CU share of the experts (with 128 experts
// on 256 CUs, two; measured at 128 tokens equal with four, at 40-64 tokens 7%
// faster than four and 8-20% faster than eight)
constexpr int GT_GX_PER_CU = 1;

template <bool AL>
__global__ __launch_bounds__(GT_WPB * 64) void k_grp_q4k(MoeGrpArgs a) {
  constexpr int WPB = GT_WPB, GPW = TOK_GPW, NH = AL ? 1 : GPW;
  constexpr int XROW = 132, WROW = 80;
  constexpr size_t RED_BYTES = sizeof(f32x4) * 2 * WPB * 64, XST_BYTES = sizeof(float) * WPB * 16 * XROW;
  constexpr size_t WST_BYTES = AL ? (size_t)WPB * 16 * WROW : 0;
  __shared__ __attribute__((aligned(16))) unsigned char
      lds[RED_BYTES + WST_BYTES > XST_BYTES ? RED_BYTES + WST_BYTES : XST_BYTES];
  __shared__ int pl[16];      // the pass's pairs (-1: none)
  __shared__ int tl[16];      // their tokens (empty slots: the first pair's)
  __shared__ int wcnt[WPB];   // matches per wave in a scan step
  f32x4(*red)[WPB][64] = (f32x4(*)[WPB][64])lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, j = lane >> 4;
  const int C = a.dim1 >> 6;
  const int g0 = wid * GPW;                     // first group of this wave's slice (even)
  const int ng = max(0, min(GPW, C - g0));      // wave-uniform
  const int e = blockIdx.y;
  const bool zero_rows = e == a.n_experts;
  const int n_rt = (a.rows + 15) >> 4;
  const int rpb = (n_rt + gridDim.x - 1) / gridDim.x;
  const int rt0 = min(n_rt, (int)blockIdx.x * rpb), rt1 = min(n_rt, rt0 + rpb);
  if (rt0 >= rt1) return;  // the whole workgroup
  const int64_t base = (zero_rows ? 0 : (int64_t)e * a.expert_stride) + a.base0;

  // pairs of rank 16 pass .. 16 pass + 15 among this expert's into pl; returns
  // the number of its pairs (the same in every thread)
  auto scan = [&](int pass) {
    if (tid < 16) pl[tid] = -1;
    int total = 0;
    for (int p0 = 0; p0 < a.S; p0 += WPB * 64) {
      const int p = p0 + tid;
      bool m = false;
      if (p < a.S) {
        const int id = a.ids[p];
        m = zero_rows ? (id < 0 || id >= a.n_experts) : id == e;
      }
      const uint64_t b = __builtin_amdgcn_ballot_w64(m);
      if (lane == 0) wcnt[wid] = __builtin_popcountll(b);
      __syncthreads();
      int before = total, all = 0;
#pragma unroll
      for (int w = 0; w < WPB; ++w) {
        before += w < wid ? wcnt[w] : 0;
        all += wcnt[w];
      }
      const int rank = before + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
      if (m && rank >= 16 * pass && rank < 16 * (pass + 1)) pl[rank - 16 * pass] = p;
      total += all;
      __syncthreads();  // wcnt is rewritten next step; pl is complete after the last
    }
    if (tid < 16) tl[tid] = (pl[tid] >= 0 ? pl[tid] : pl[0]) / a.x_div;
    __syncthreads();
    return total;
  };

  const int64_t w_step = (16 * a.row_stride >> 8) * 144;  // 16 rows: whole super-blocks
  // weight group gi of row tile rt, this lane's row (B column n) and K-slice j
  auto load_w = [&](int rt, bool live, u32x2a4 (&Q)[GPW], u32x4 (&H)[NH], int (&gs)[GPW]) {
    const int r = rt * 16 + n;
    const bool rok = live && r < a.rows;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      // rows past the end and groups past the slice read the first group of
      // the tensor (in bounds; never stored / never multiplied)
      const int64_t el = (rok && gi < ng) ? base + (int64_t)r * a.row_stride + (int64_t)(g0 + gi) * 64 : 0;
      const int64_t G = el >> 6;
      const uint8_t *sb = a.W + (G >> 2) * 144;
      gs[gi] = (int)(G & 3);
      H[gi] = *(const u32x4 *)sb;
      Q[gi] = *(const u32x2a4 *)(sb + 16 + 32 * (G & 3) + 8 * j);
    }
  };
  // AL: a tile's 16 rows x (head + the wave's two groups) read by four adjacent
  // lanes per row and staged in the wave's own LDS rows (as k_tok_q4k does).
  // Rows start on a group pair (row_stride a multiple of 128: the MoE down
  // rows of 1408 columns start every second one half way into a super-block),
  // so a wave's two groups lie in one super-block, at a row-dependent position
  // that repeats every 16 rows (16 rows are whole super-blocks)
  unsigned char *wst = lds + RED_BYTES + (size_t)wid * 16 * WROW;
  const int64_t e_st = base + (int64_t)(rt0 * 16 + (lane >> 2)) * a.row_stride + (int64_t)g0 * 64;
  const uint8_t *w_tile0 = a.W + (e_st >> 8) * 144;
  const int q_st = 16 + 32 * (int)((e_st >> 6) & 3) + 16 * (lane & 3);
  // which half of its super-block row n's groups are in (the scales' byte positions)
  const int hq_n = (int)((((int64_t)n * a.row_stride + (int64_t)g0 * 64 + base) >> 7) & 1);
  auto load_raw = [&](int rt, bool live, u32x4 &QR, uint32_t &HR) {
    // rows past the end read the tensor's first super-block
    const bool ok = live && ng > 0 && rt * 16 + (lane >> 2) < a.rows;
    const uint8_t *sb = ok ? w_tile0 + (int64_t)(rt - rt0) * w_step : a.W;
    QR = *(const u32x4 *)(sb + (ok ? q_st : 16));
    HR = *(const uint32_t *)(sb + 4 * (lane & 3));
  };
  auto stage = [&](const u32x4 &QR, uint32_t HR, u32x2a4 (&Q)[GPW], u32x4 (&H)[NH]) {
    unsigned char *wr = wst + (lane >> 2) * WROW;
    *(u32x4 *)(wr + 16 + 16 * (lane & 3)) = QR;
    *(uint32_t *)(wr + 4 * (lane & 3)) = HR;
    const unsigned char *rd = wst + n * WROW;
    H[0] = *(const u32x4 *)rd;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) Q[gi] = *(const u32x2a4 *)(rd + 16 + 32 * gi + 8 * j);
  };

  for (int pass = 0;; ++pass) {
    if (pass > 0) __syncthreads();  // every wave is done with the previous pass's LDS
    const int total = scan(pass);
    const int cnt = min(16, total - 16 * pass);
    if (cnt <= 0) return;
    if (zero_rows) {
      const int r0 = rt0 * 16, nr = min(a.rows, rt1 * 16) - r0;
      for (int i = tid; i < cnt * nr; i += WPB * 64) {
        const int t = i / nr, r = r0 + i % nr;
        a.y[(int64_t)pl[t] * a.y_stride + r] = 0.f;
      }
      continue;
    }
    // the pair of the outputs this lane stores (component wid of its four, waves 0..3)
    const int pj = pl[4 * j + (wid & 3)];

    // x of the 16 pair slots x the wave's 128 columns, adjacent lanes on adjacent
    // 16-byte pieces (lane l: piece l % 32 of slot 2q + l / 32); empty slots read
    // the first pair's token (never stored), groups past the slice group 0
    u32x4a4 xg[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int slot = 2 * q + (lane >> 5), c = lane & 31, gi = c >> 4;
      const float *src = a.x + (int64_t)tl[slot] * a.x_stride + (int64_t)(gi < ng ? g0 + gi : 0) * 64 + 4 * (c & 15);
      xg[q] = *(const u32x4a4 *)src;
    }
    u32x2a4 QA[GPW], QB[GPW];
    u32x4 HA[NH], HB[NH];
    int GA[GPW], GB[GPW];
    u32x4 QRA, QRB;
    uint32_t HRA, HRB;
    // the first tile's weight loads go out behind the x loads
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (AL)
      load_raw(rt0, true, QRA, HRA);
    else
      load_w(rt0, true, QA, HA, GA);
    __builtin_amdgcn_sched_barrier(0);

    // back from LDS in the MFMA layout: lane (j, n) takes slot n, columns
    // 64 gi + 32 h + 8 j .. +8 of the slice
    u32x4a4 xr[GPW][2][2];
    float *xst = (float *)lds + wid * 16 * XROW;
#pragma unroll
    for (int q = 0; q < 8; ++q) *(u32x4 *)(xst + (2 * q + (lane >> 5)) * XROW + 4 * (lane & 31)) = xg[q];
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int u = 0; u < 2; ++u) xr[gi][h][u] = *(const u32x4 *)(xst + n * XROW + 64 * gi + 32 * h + 8 * j + 4 * u);
    __syncthreads();  // every wave has its x: the LDS now holds the partial tiles

    // the sum of x over sub-block j for slot n (the fp32 MFMA's A operand)
    float ps[2 * GPW];
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float t = __uint_as_float(xr[gi][h][0].x);
        t += __uint_as_float(xr[gi][h][0].y);
        t += __uint_as_float(xr[gi][h][0].z);
        t += __uint_as_float(xr[gi][h][0].w);
        t += __uint_as_float(xr[gi][h][1].x);
        t += __uint_as_float(xr[gi][h][1].y);
        t += __uint_as_float(xr[gi][h][1].z);
        t += __uint_as_float(xr[gi][h][1].w);
        ps[2 * gi + h] = t;
      }
    const float t02 = tstep<32>(ps[0], ps[2], lane), t13 = tstep<32>(ps[1], ps[3], lane);
    float xsT = tstep<16>(t02, t13, lane);
    const bool bad = !__builtin_isfinite(xsT);
    bf16x8 A[GPW][2][3];
    auto split_all = [&](auto guard) {
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float v[8];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            v[4 * u] = __uint_as_float(xr[gi][h][u].x);
            v[4 * u + 1] = __uint_as_float(xr[gi][h][u].y);
            v[4 * u + 2] = __uint_as_float(xr[gi][h][u].z);
            v[4 * u + 3] = __uint_as_float(xr[gi][h][u].w);
          }
          split3<decltype(guard)::value>(v, A[gi][h][0], A[gi][h][1], A[gi][h][2]);
        }
    };
    if (__builtin_amdgcn_ballot_w64(bad) != 0)
      split_all(std::true_type());
    else
      split_all(std::false_type());
    if ((j >> 1) >= ng) xsT = 0.f;  // a group past the slice
    // sum(128 x) of each sub-block by the tiles' MFMAs (the all-8 operand)
    f32x4 S8[GPW][2];
    {
      bf16x8 b128;
#pragma unroll
      for (int i = 0; i < 8; ++i) b128[i] = (__bf16)128.0f;
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          S8[gi][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int p = 0; p < 3; ++p)
            S8[gi][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[gi][h][p], b128, S8[gi][h], 0, 0, 0);
        }
    }

    int buf = 0;
    // mid() runs between the partial tile's LDS store and the barrier
    auto tile = [&](int rt, const u32x2a4 (&Q)[GPW], const u32x4 (&H)[NH], const int (&gs)[GPW], auto &&mid) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
      if (ng > 0) {  // wave-uniform
        float d1[2 * GPW], cj;
        if constexpr (AL) {
          const float dq = h2f(H[0].x & 0xFFFFu) * 0.0625f, dmin = h2f(H[0].x >> 16);
          uint32_t scq, mq;
          scale_min_quad_sel(H[0], hq_n, scq, mq);
#pragma unroll
          for (int s = 0; s < 4; ++s) d1[s] = dq * ubyte(scq, s);
          const float scj = (float)((scq >> (8 * j)) & 0xFFu), mj = (float)((mq >> (8 * j)) & 0xFFu);
          cj = __builtin_fmaf(128.f, dq * scj, -(dmin * mj));
        } else {
          float cc[GPW][2];
#pragma unroll
          for (int gi = 0; gi < GPW; ++gi) {
            uint32_t scp, mp;
            scale_min_pair(H[gi], gs[gi], scp, mp);
            const float dq = h2f(H[gi].x & 0xFFFFu) * 0.0625f, dmin = h2f(H[gi].x >> 16);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              d1[2 * gi + h] = dq * ubyte(scp, h);
              cc[gi][h] = __builtin_fmaf(128.f, d1[2 * gi + h], -(dmin * ubyte(mp, h)));
            }
          }
          const float c0 = (j & 1) ? cc[0][1] : cc[0][0], c1 = (j & 1) ? cc[1][1] : cc[1][0];
          // a group past the slice has the tensor's first head: no coefficient
          cj = (j >> 1) >= ng ? 0.f : ((j >> 1) ? c1 : c0);
        }
        f32x4 P[GPW][2];
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
          if (gi < ng) {  // wave-uniform
            const uint32_t w0 = Q[gi].x, w1 = Q[gi].y;
            const bf16x8 bl = codes_bf16_16q(opaque(w0 & 0x0F0F0F0Fu), opaque(w1 & 0x0F0F0F0Fu));
            const bf16x8 bh = codes_bf16_16q(opaque((w0 >> 4) & 0x0F0F0F0Fu), opaque((w1 >> 4) & 0x0F0F0F0Fu));
            P[gi][0] = P[gi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < 3; ++p) {
              P[gi][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[gi][0][p], bl, P[gi][0], 0, 0, 0);
              P[gi][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[gi][1][p], bh, P[gi][1], 0, 0, 0);
            }
          }
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xsT, cj, acc, 0, 0, 0);
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi)
          if (gi < ng)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[i] = __builtin_fmaf(d1[2 * gi], P[gi][0][i] - S8[gi][0][i], acc[i]);
              acc[i] = __builtin_fmaf(d1[2 * gi + 1], P[gi][1][i] - S8[gi][1][i], acc[i]);
            }
      }
      // the 16 column slices summed in wave order (deterministic): wave c < 4
      // takes component c of every lane's four outputs
      red[buf][wid][lane] = acc;
      mid();
      __syncthreads();
      if (wid < 4) {
        const float *rp = (const float *)&red[buf][0][lane] + wid;
        float s = rp[0];
#pragma unroll
        for (int w = 1; w < WPB; ++w) s += rp[w * 64 * 4];
        const int r = rt * 16 + n;
        if (pj >= 0 && r < a.rows) a.y[(int64_t)pj * a.y_stride + r] = s;
      }
      buf ^= 1;
    };

    if constexpr (AL) {
      // tile t+1's weights load while tile t multiplies, and are staged between
      // tile t's partial store and its barrier
      stage(QRA, HRA, QA, HA);
      for (int rt = rt0; rt < rt1; rt += 2) {
        load_raw(rt + 1, rt + 1 < rt1, QRB, HRB);
        __builtin_amdgcn_sched_barrier(0);
        tile(rt, QA, HA, GA, [&] { stage(QRB, HRB, QA, HA); });
        __builtin_amdgcn_sched_barrier(0);
        load_raw(rt + 2, rt + 2 < rt1, QRA, HRA);
        __builtin_amdgcn_sched_barrier(0);
        if (rt + 1 < rt1) tile(rt + 1, QA, HA, GA, [&] { stage(QRA, HRA, QA, HA); });
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      // two row tiles in flight: tile t+1 loads while tile t multiplies
      for (int rt = rt0; rt < rt1; rt += 2) {
        load_w(rt + 1, rt + 1 < rt1, QB, HB, GB);
        __builtin_amdgcn_sched_barrier(0);
        tile(rt, QA, HA, GA, [] {});
        __builtin_amdgcn_sched_barrier(0);
        load_w(rt + 2, rt + 2 < rt1, QA, HA, GA);
        __builtin_amdgcn_sched_barrier(0);
        if (rt + 1 < rt1) tile(rt + 1, QB, HB, GB, [] {});
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

// True when the 16-pair tiles take a grouped launch: Q4_K rows of at most 2048
// columns in 64-column groups; the gate+up launch's gate and up halves adjacent.
static bool grp_tok_ok(bool gate_up, const MoeGrpArgs &a) {
  if (a.dim1 <= 0 || a.dim1 > GT_WPB * TOK_GPW * 64 || a.dim1 % 64 != 0) return false;
  if (a.base0 % 64 != 0 || a.row_stride % 64 != 0 || a.expert_stride % 64 != 0) return false;
  if (gate_up && (a.gu == nullptr || a.base1 != a.base0 + (int64_t)a.rows * a.row_stride)) return false;
  return a.S >= 1 && a.rows >= 1 && a.x_div >= 1 && a.n_experts >= 1;
}

bool moe_grp_ok(int type, const MoeGrpArgs &a) {
  if (type != T_Q4_K) return false;
  if (a.dim1 <= 0 || a.dim1 % 128 != 0 || a.dim1 > MG_MAX_DIM1) return false;
  if (a.base0 % 128 != 0 || a.base1 % 128 != 0 || a.row_stride % 128 != 0 || a.expert_stride % 128 != 0)
    return false;
  return a.S >= 1 && a.S <= MG_MAX_S && a.rows >= 1 && a.x_div >= 1 && a.n_experts >= 1;
}

hipError_t moe_grp_init_device() {
  // the largest LDS operand set (MG_MAX_DIM1 columns), granted once per device
  const int lds = (int)mg_lds_bytes(MG_MAX_DIM1);
  hipError_t e = hipFuncSetAttribute((const void *)k_moe_grp<true>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute((const void *)k_moe_grp<false>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
}

hipError_t launch_moe_grp(int type, bool gate_up, const MoeGrpArgs &a, const DevInfo &dev, hipStream_t s) {
  if (!moe_grp_ok(type, a)) return hipErrorNotSupported;
  if (grp_tok_ok(gate_up, a)) {
    // 16-pair tiles: the gate+up launch writes the gate and up rows (2 rows per
    // pair) and k_gelu_mul forms h; row blocks per expert so that the experts'
    // workgroups about fill the CUs
    MoeGrpArgs b = a;
    if (gate_up) {
      b.rows = 2 * a.rows;
      b.y = a.gu;
      b.y_stride = 2 * (int64_t)a.rows;
    }
    const int n_rt = (b.rows + 15) / 16;
    const int gx = std::max(1, std::min(n_rt, GT_GX_PER_CU * dev.cu_count / std::max(1, b.n_experts)));
    const dim3 grid((unsigned)gx, (unsigned)b.n_experts + 1);
    // rows starting on a group pair and whole 128-column slices: the coalesced,
    // LDS-staged weight tiles
    const bool al = b.base0 % 128 == 0 && b.row_stride % 128 == 0 && b.expert_stride % 128 == 0 && b.dim1 % 128 == 0;
    if (al)
      hipLaunchKernelGGL(k_grp_q4k<true>, grid, dim3(GT_WPB * 64), 0, s, b);
    else
      hipLaunchKernelGGL(k_grp_q4k<false>, grid, dim3(GT_WPB * 64), 0, s, b);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !gate_up) return e;
    return launch_gelu_mul(a.gu, a.rows, a.S, a.y, a.y_stride, s);
  }
  const int ur = gate_up ? 16 : 32;
  const int units = (a.rows + ur - 1) / ur;
  const dim3 grid((unsigned)((units + MG_UPW * MG_WPB - 1) / (MG_UPW * MG_WPB)), (unsigned)a.n_experts + 1);
  // up to mg_lds_bytes(MG_MAX_DIM1) of dynamic LDS: granted by moe_grp_init_device
  // when the context opened (a host-side attribute, never set during a capture)
  const size_t lds = mg_lds_bytes(a.dim1);
  if (gate_up)
    hipLaunchKernelGGL(k_moe_grp<true>, grid, dim3(MG_WPB * 64), lds, s, a);
  else
    hipLaunchKernelGGL(k_moe_grp<false>, grid, dim3(MG_WPB * 64), lds, s, a);
  return hipGetLastError();
}

}  // namespace g4
