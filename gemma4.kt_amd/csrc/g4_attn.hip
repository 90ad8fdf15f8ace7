// g4_attn.hip -- decode attention of one token over a layer's KV cache
// (Llama.kt:198-218): for every query head h, scores q_h . K[t] (scale 1) over
// positions att_start..position, softmax (MutableFloatTensor.kt:54-59: max, exp in
// double, fp32 sum, divide), then out_h = sum_t a_t V[t].  Head h reads kv head
// h / kv_mul; row t of a cache starts at t * n_kv * head_size floats.
//
// Split over positions (the sequence is the long axis at decode): workgroup
// (chunk, kv head, head group) computes the scores of up to 4 query heads that
// share a kv head against its chunk of K rows (each K row read once for all of
// them) into LDS, the chunk's max and exp(s - max) in double, then the exp-weighted
// sum of its V rows.  k_att_combine rescales the chunks to the global max
// (exp(m_c - M), double) and divides by the total sum.  K and V each stream from
// HBM once; the partials are n_chunks * n_heads * (head_size + 2) floats.
#include <float.h>

#include "g4_device.hpp"
#include "g4_internal.hpp"

namespace g4 {

constexpr int ATT_CHMAX = 512;    // rows per chunk (scores in LDS)
constexpr int ATT_MAXCHUNKS = 1024;

G4_DEV float jmax(float a, float b) {  // java.lang.Math.max(float, float)
  if (a != a) return a;
  if (b != b) return b;
  if (a == 0.f && b == 0.f) return __builtin_signbit(a) ? b : a;
  return a >= b ? a : b;
}

// Sum over the wave in every lane, without LDS (permlane swaps at distances 32
// and 16, DPP below; each step adds a lane's value and its partner's, the same
// bits in either order, so every lane ends with the same sum).
G4_DEV float wave_fsum(float v) {
  v = pstep<32>(v);
  v = pstep<16>(v);
  v = pstep<8>(v);
  v = pstep<4>(v);
  v = pstep<2>(v);
  return pstep<1>(v);
}

// Sum over each aligned group of N lanes (N a power of two), without LDS:
// partners at distances 1, 2, 4, ... (DPP quad permutes; at 4 the half-row
// mirror, which after the steps at 1 and 2 pairs the two quads of every 8
// lanes; row_ror:8; then permlane swaps), every lane of a group ending with its
// group's sum.
template <int N>
G4_DEV float group_sum(float s, int lane) {
  if constexpr (N > 1) s += __uint_as_float(partner_u32<1>(__float_as_uint(s), lane));
  if constexpr (N > 2) s += __uint_as_float(partner_u32<2>(__float_as_uint(s), lane));
  if constexpr (N > 4) s += __uint_as_float(partner_u32<4>(__float_as_uint(s), lane));
  if constexpr (N > 8) s += __uint_as_float(partner_u32<8>(__float_as_uint(s), lane));
  if constexpr (N > 16) s += __uint_as_float(partner_u32<16>(__float_as_uint(s), lane));
  if constexpr (N > 32) s += __uint_as_float(partner_u32<32>(__float_as_uint(s), lane));
  return s;
}

G4_DEV float wave_jmax(float v) {  // every lane: the wave's maximum (butterfly without LDS)
  const int lane = threadIdx.x & 63;
  v = jmax(v, __uint_as_float(partner_u32<32>(__float_as_uint(v), lane)));
  v = jmax(v, __uint_as_float(partner_u32<16>(__float_as_uint(v), lane)));
  v = jmax(v, __uint_as_float(partner_u32<8>(__float_as_uint(v), lane)));
  v = jmax(v, __uint_as_float(partner_u32<4>(__float_as_uint(v), lane)));
  v = jmax(v, __uint_as_float(partner_u32<2>(__float_as_uint(v), lane)));
  return jmax(v, __uint_as_float(partner_u32<1>(__float_as_uint(v), lane)));
}

template <int HS, int GT>
__global__ __launch_bounds__(256) void k_att_part(AttArgs a) {
  constexpr int LS = HS / 16, RS = 64 / LS;         // scores: 16 floats per lane, LS lanes per row
  constexpr int VPL = HS > 256 ? HS / 256 : 1;      // values: float4s per lane
  constexpr int LV = HS / (4 * VPL), RV = 64 / LV;  // lanes per V row, rows per step
  static_assert(LS >= 1 && LS <= 64 && LV >= 1 && LV <= 64, "head size");
  __shared__ float sc[ATT_CHMAX][GT];
  __shared__ float mls[2][GT];
  __shared__ float4 red[4][GT][HS / 4];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int chunk = blockIdx.x;
  const int kvh = blockIdx.y / a.n_groups, grp = blockIdx.y % a.n_groups;
  const int64_t kv_dim = (int64_t)a.n_kv * HS;
  const int r_begin = chunk * a.ch;
  const int nr = min(a.rows - r_begin, a.ch);  // valid rows of this chunk (>= 1)
  const int per_wave = a.ch >> 2;              // a.ch is a multiple of 4 * max(RS, RV)
  const int w_begin = wid * per_wave;
  const float *kbase = a.kc + (int64_t)(a.row0 + r_begin) * kv_dim + (int64_t)kvh * HS;
  const float *vbase = a.vc + (int64_t)(a.row0 + r_begin) * kv_dim + (int64_t)kvh * HS;

  int head[GT];
  bool hok[GT];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const int hg = grp * GT + g;
    hok[g] = hg < a.kv_mul;
    head[g] = kvh * a.kv_mul + (hok[g] ? hg : 0);
  }

  // ---- scores: lane (rl, ql) dots 16 floats of row w_begin + st + rl
  const int ql = lane % LS, rl = lane / LS;
  float qv[GT][16];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const float4 *qp = (const float4 *)(a.q + (int64_t)head[g] * HS + 16 * ql);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 t = qp[j];
      qv[g][4 * j] = t.x, qv[g][4 * j + 1] = t.y, qv[g][4 * j + 2] = t.z, qv[g][4 * j + 3] = t.w;
    }
  }
  constexpr int US = 4;  // score steps in flight per lane
  for (int st0 = 0; st0 < per_wave; st0 += US * RS) {
    float4 kk[US][4];
    bool ok[US];
    int rr[US];
#pragma unroll
    for (int u = 0; u < US; ++u) {
      rr[u] = w_begin + st0 + u * RS + rl;
      ok[u] = rr[u] < nr && st0 + u * RS < per_wave;
      const float4 *kp = (const float4 *)(kbase + (int64_t)(ok[u] ? rr[u] : 0) * kv_dim + 16 * ql);
#pragma unroll
      for (int j = 0; j < 4; ++j) kk[u][j] = kp[j];
    }
#pragma unroll
    for (int u = 0; u < US; ++u) {
      if (st0 + u * RS >= per_wave) break;  // wave-uniform
      float d[GT];
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s = __builtin_fmaf(qv[g][4 * j], kk[u][j].x, s);
          s = __builtin_fmaf(qv[g][4 * j + 1], kk[u][j].y, s);
          s = __builtin_fmaf(qv[g][4 * j + 2], kk[u][j].z, s);
          s = __builtin_fmaf(qv[g][4 * j + 3], kk[u][j].w, s);
        }
        d[g] = group_sum<LS>(s, lane);
      }
      if (ql == 0)
#pragma unroll
        for (int g = 0; g < GT; ++g) sc[rr[u]][g] = ok[u] ? d[g] : -__builtin_inff();
    }
  }

  // the first V rows go out now: they do not depend on the scores
  const int vl = lane % LV, vr = lane / LV;
  constexpr int U = 8;  // V rows in flight per lane
  float4 vv[U][VPL];
  bool vok[U];
  int vrr[U];
  auto load_v = [&](int st) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      vrr[u] = w_begin + st + u * RV + vr;
      vok[u] = vrr[u] < nr && st + u * RV < per_wave;
      const float4 *vp = (const float4 *)(vbase + (int64_t)(vok[u] ? vrr[u] : 0) * kv_dim) + VPL * vl;
#pragma unroll
      for (int j = 0; j < VPL; ++j) vv[u][j] = vp[j];
    }
  };
  load_v(0);
  __syncthreads();

  // ---- chunk max, exp(s - max) in double, chunk sum (wave g owns head g)
  if (wid < GT) {
    float m = -__builtin_inff();
    for (int r = lane; r < nr; r += 64) m = jmax(m, sc[r][wid]);
    m = wave_jmax(m);
    if (lane == 0) mls[0][wid] = m;
  }
  __syncthreads();
  for (int i = tid; i < a.ch * GT; i += 256) {
    const int r = i / GT, g = i % GT;
    sc[r][g] = r < nr ? (float)exp((double)__fsub_rn(sc[r][g], mls[0][g])) : 0.f;
  }
  __syncthreads();
  if (wid < GT) {
    float l = 0.f;
    for (int r = lane; r < nr; r += 64) l += sc[r][wid];
    l = wave_fsum(l);
    if (lane == 0) mls[1][wid] = l;
  }

  // ---- values: lane (vr, vl) accumulates VPL float4s of row w_begin + st + vr
  float4 acc[GT][VPL];
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int j = 0; j < VPL; ++j) acc[g][j] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int st = 0; st < per_wave; st += U * RV) {
    if (st > 0) load_v(st);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!vok[u]) continue;
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        const float e = sc[vrr[u]][g];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          acc[g][j].x = __builtin_fmaf(e, vv[u][j].x, acc[g][j].x);
          acc[g][j].y = __builtin_fmaf(e, vv[u][j].y, acc[g][j].y);
          acc[g][j].z = __builtin_fmaf(e, vv[u][j].z, acc[g][j].z);
          acc[g][j].w = __builtin_fmaf(e, vv[u][j].w, acc[g][j].w);
        }
      }
    }
  }
  // rows of one step sit in lane groups vr: add them (lane bits above LV)
#pragma unroll
  for (int m = LV; m < 64; m <<= 1)
#pragma unroll
    for (int g = 0; g < GT; ++g)
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        acc[g][j].x += __shfl_xor(acc[g][j].x, m, 64);
        acc[g][j].y += __shfl_xor(acc[g][j].y, m, 64);
        acc[g][j].z += __shfl_xor(acc[g][j].z, m, 64);
        acc[g][j].w += __shfl_xor(acc[g][j].w, m, 64);
      }
  if (vr == 0)
#pragma unroll
    for (int g = 0; g < GT; ++g)
#pragma unroll
      for (int j = 0; j < VPL; ++j) red[wid][g][VPL * vl + j] = acc[g][j];
  __syncthreads();
  // the four waves' partials in wave order, then the chunk's (max, sum)
  for (int f = tid; f < GT * (HS / 4); f += 256) {
    const int g = f / (HS / 4), e = f % (HS / 4);
    float4 s = red[0][g][e];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float4 t = red[w][g][e];
      s.x += t.x, s.y += t.y, s.z += t.z, s.w += t.w;
    }
    const int hg = grp * GT + g;
    if (hg < a.kv_mul) {
      const int h = kvh * a.kv_mul + hg;
      ((float4 *)(a.part + ((int64_t)chunk * a.n_heads + h) * HS))[e] = s;
    }
  }
  if (tid < GT && grp * GT + tid < a.kv_mul) {
    const int h = kvh * a.kv_mul + grp * GT + tid;
    a.ml[((int64_t)chunk * a.n_heads + h) * 2] = mls[0][tid];
    a.ml[((int64_t)chunk * a.n_heads + h) * 2 + 1] = mls[1][tid];
  }
}

// Per head: M = max of the chunk maxima, w_c = exp(m_c - M) (double), sum =
// sum_c w_c l_c and out = sum_c w_c o_c / sum.  Workgroup (head, 64-element
// slice): wave w takes chunks w, w + 4, ...; the four wave sums are added in wave
// order.  PRE: up to 128 chunks, every partial is loaded at the start (they do not
// depend on the maxima), so the kernel makes one round trip to memory, and each
// wave forms M, the weights and the sum itself (no block-wide reduction).
template <bool PRE>
__global__ __launch_bounds__(256) void k_att_combine(const float *part, const float *ml, int32_t n_chunks,
                                                     int32_t n_heads, int32_t hs, float *out) {
  __shared__ float ws[4][64];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int e = blockIdx.y * 64 + lane;
  const bool live = e < hs;
  const int64_t col = (int64_t)h * hs + (live ? e : 0);
  float o = 0.f, tot;
  if constexpr (PRE) {
    // up to 128 chunks: every partial goes out at the start, and every wave
    // forms the chunk weights itself (lane i: chunks i and i + 64), so the only
    // barrier is the cross-wave sum at the end
    constexpr int NP = 32;
    float p[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int c = wid + 4 * k;
      p[k] = part[(int64_t)(c < n_chunks ? c : 0) * n_heads * hs + col];
    }
    float mc[2], lc[2], w[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int c = lane + 64 * q;
      const bool in = c < n_chunks;
      mc[q] = ml[((int64_t)(in ? c : 0) * n_heads + h) * 2];
      lc[q] = ml[((int64_t)(in ? c : 0) * n_heads + h) * 2 + 1];
      if (!in) mc[q] = -__builtin_inff();
    }
    const float M = wave_jmax(jmax(mc[0], mc[1]));
    float l = 0.f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      w[q] = lane + 64 * q < n_chunks ? (float)exp((double)__fsub_rn(mc[q], M)) : 0.f;
      l = __builtin_fmaf(w[q], lc[q], l);
    }
    tot = wave_fsum(l);
#pragma unroll
    for (int k = 0; k < NP; ++k) {
      const int c = wid + 4 * k;  // wave-uniform; chunk c's weight sits in lane c % 64 of w[c / 64]
      const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[k < 16 ? 0 : 1]), c & 63));
      if (c < n_chunks) o = __builtin_fmaf(wc, p[k], o);
    }
  } else {
    __shared__ float wc[ATT_MAXCHUNKS];
    __shared__ float red[4];
    __shared__ float bm;
    float m = -__builtin_inff(), lc[ATT_MAXCHUNKS / 256];
#pragma unroll
    for (int k = 0; k < ATT_MAXCHUNKS / 256; ++k) {
      const int c = tid + 256 * k;
      const bool in = c < n_chunks;
      const float mc = ml[((int64_t)(in ? c : 0) * n_heads + h) * 2];
      lc[k] = ml[((int64_t)(in ? c : 0) * n_heads + h) * 2 + 1];
      if (in) wc[c] = mc, m = jmax(m, mc);
    }
    m = wave_jmax(m);
    if (lane == 0) red[wid] = m;
    __syncthreads();
    if (tid == 0) bm = jmax(jmax(jmax(red[0], red[1]), red[2]), red[3]);
    __syncthreads();
    const float M = bm;
    float l = 0.f;
#pragma unroll
    for (int k = 0; k < ATT_MAXCHUNKS / 256; ++k) {
      const int c = tid + 256 * k;
      if (c < n_chunks) {
        const float w = (float)exp((double)__fsub_rn(wc[c], M));
        wc[c] = w;
        l = __builtin_fmaf(w, lc[k], l);
      }
    }
    __syncthreads();  // red[] reused, every weight stored
    tot = block_sum256(l, red);
    constexpr int UC = 8;
    for (int c0 = wid; c0 < n_chunks; c0 += 4 * UC) {
      float q[UC];
#pragma unroll
      for (int u = 0; u < UC; ++u) {
        const int c = c0 + 4 * u;
        q[u] = part[(int64_t)(c < n_chunks ? c : 0) * n_heads * hs + col];
      }
#pragma unroll
      for (int u = 0; u < UC; ++u)
        if (c0 + 4 * u < n_chunks) o = __builtin_fmaf(wc[c0 + 4 * u], q[u], o);
    }
  }
  ws[wid][lane] = o;
  __syncthreads();
  if (wid == 0 && live) {
    const float s = ((ws[0][lane] + ws[1][lane]) + ws[2][lane]) + ws[3][lane];
    out[(int64_t)h * hs + e] = __fdiv_rn(s, tot);
  }
}

// Any head size: one workgroup per head, scores in `att` (n_heads * rows floats).
__global__ __launch_bounds__(256) void k_att_generic(AttArgs a) {
  __shared__ float red[4];
  __shared__ float bm;
  const int h = blockIdx.x, tid = threadIdx.x, hs = a.hs;
  const int64_t kv_dim = (int64_t)a.n_kv * hs;
  const int kvh = h / a.kv_mul;
  const float *q = a.q + (int64_t)h * hs;
  float *att = a.part + (int64_t)h * a.rows;
  float m = -__builtin_inff();
  for (int t = tid; t < a.rows; t += 256) {
    const float *k = a.kc + (int64_t)(a.row0 + t) * kv_dim + (int64_t)kvh * hs;
    float s = 0.f;
    for (int i = 0; i < hs; ++i) s = __builtin_fmaf(q[i], k[i], s);
    att[t] = s;
    m = jmax(m, s);
  }
  m = wave_jmax(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) bm = jmax(jmax(jmax(red[0], red[1]), red[2]), red[3]);
  __syncthreads();
  const float M = bm;
  float l = 0.f;
  for (int t = tid; t < a.rows; t += 256) {
    const float e = (float)exp((double)__fsub_rn(att[t], M));
    att[t] = e;
    l += e;
  }
  __syncthreads();  // red[] reused
  const float L = block_sum256(l, red);
  __syncthreads();  // every exp is stored
  for (int i = tid; i < hs; i += 256) {
    float o = 0.f;
    for (int t = 0; t < a.rows; ++t)
      o = __builtin_fmaf(att[t], a.vc[(int64_t)(a.row0 + t) * kv_dim + (int64_t)kvh * hs + i], o);
    a.out[(int64_t)h * hs + i] = __fdiv_rn(o, L);
  }
}

// ------------------------------------------------------------- launcher ----

static int att_unit(int hs) {
  const int LS = hs / 16, RS = 64 / LS, VPL = hs > 256 ? hs / 256 : 1, LV = hs / (4 * VPL), RV = 64 / LV;
  return 4 * (RS > RV ? RS : RV);
}

bool attention_fast_ok(int32_t hs) { return hs == 64 || hs == 128 || hs == 256 || hs == 512; }

void attention_plan(AttArgs &a, const DevInfo &dev) {
  a.kv_mul = a.n_heads / a.n_kv;
  if (!attention_fast_ok(a.hs)) a.generic = 1;
  if (a.generic) {
    a.n_groups = 1;
    a.ch = a.rows;
    a.n_chunks = 1;
    return;
  }
  const int gt = a.kv_mul >= 4 ? 4 : (a.kv_mul >= 2 ? 2 : 1);
  a.n_groups = (a.kv_mul + gt - 1) / gt;
  const int unit = att_unit(a.hs);
  const int64_t per = (int64_t)a.n_kv * a.n_groups;
  // Two workgroups per CU when that leaves chunks of at least 128 rows, else one
  // (measured on 16 heads over 8 kv heads of 256, 512 to 32768 positions, 1 to
  // 16 workgroups per CU: 8192 positions 34.8 us at four per CU, 29.9 at two,
  // 31.7 at one; 2048 positions 15.7 at two, 14.6 at one)
  auto chunk_rows = [&](int64_t per_cu) {
    int64_t chunks = (per_cu * dev.cu_count + per - 1) / per;
    if (chunks < 1) chunks = 1;
    return (a.rows + chunks - 1) / chunks;
  };
  int64_t ch = chunk_rows(2);
  if (ch < 128) ch = chunk_rows(1);
  ch = (ch + unit - 1) / unit * unit;
  if (ch > ATT_CHMAX) ch = ATT_CHMAX;
  a.ch = (int32_t)ch;
  a.n_chunks = (int32_t)((a.rows + ch - 1) / ch);
}

int64_t attention_scratch_floats(const AttArgs &a) {
  if (a.generic) return (int64_t)a.n_heads * a.rows;
  return (int64_t)a.n_chunks * a.n_heads * (a.hs + 2);
}

template <int HS>
static void launch_part(const AttArgs &a, int gt, hipStream_t s) {
  const dim3 grid(a.n_chunks, a.n_kv * a.n_groups);
  if (gt == 4) hipLaunchKernelGGL((k_att_part<HS, 4>), grid, dim3(256), 0, s, a);
  else if (gt == 2) hipLaunchKernelGGL((k_att_part<HS, 2>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((k_att_part<HS, 1>), grid, dim3(256), 0, s, a);
}

hipError_t launch_attention(AttArgs a, float *scratch, hipStream_t s) {
  if (a.generic) {
    a.part = scratch;
    hipLaunchKernelGGL(k_att_generic, dim3(a.n_heads), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  if (a.n_chunks > ATT_MAXCHUNKS || a.ch % att_unit(a.hs) != 0) return hipErrorInvalidValue;
  a.part = scratch;
  a.ml = scratch + (int64_t)a.n_chunks * a.n_heads * a.hs;
  const int gt = a.kv_mul >= 4 ? 4 : (a.kv_mul >= 2 ? 2 : 1);
  switch (a.hs) {
    case 64: launch_part<64>(a, gt, s); break;
    case 128: launch_part<128>(a, gt, s); break;
    case 256: launch_part<256>(a, gt, s); break;
    default: launch_part<512>(a, gt, s); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 cg(a.n_heads, (a.hs + 63) / 64);
  if (a.n_chunks <= 128)
    hipLaunchKernelGGL(k_att_combine<true>, cg, dim3(256), 0, s, (const float *)a.part, (const float *)a.ml,
                       a.n_chunks, a.n_heads, a.hs, a.out);
  else
    hipLaunchKernelGGL(k_att_combine<false>, cg, dim3(256), 0, s, (const float *)a.part, (const float *)a.ml,
                       a.n_chunks, a.n_heads, a.hs, a.out);
  return hipGetLastError();
}

}  // namespace g4
