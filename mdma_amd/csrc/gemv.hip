// Decode GEMV for GGUF Q4_K / Q6_K / Q8_0 (and F32 / F16) weights on gfx950.
//
// y[t, r] = sum_i deq(W)[r, i] * x[t, i]   (reference Backend::qmatmul,
// /root/reference/src/backend.rs:469; CPU oracle src/backend/cpu.rs:335-368)
//
// Design (wave64, CDNA4):
//  - One wave owns R output rows of one weight; its 64 lanes stride over the
//    row's 16-byte "units" of packed quants, so every load of a wave covers
//    contiguous bytes of R rows. A Q4_K unit is 16 quant bytes = 32 weights
//    (16 low nibbles of sub-block 2p, 16 high nibbles of sub-block 2p+1);
//    a Q6_K unit is 8 columns of one 128-half across its 4 quarters; a Q8_0
//    unit is half a block. Eight units per 256 weights for the K-quants.
//  - f32 mode factorises the dequantisation: sum (d*sc*q - dmin*m) * x =
//    d*sc * sum(q*x) - dmin*m * sum(x), so per weight the VALU does one byte
//    -> float conversion and one FMA; scales are decoded once per unit.
//    Unit partial sums are f32; the per-lane accumulator across units and the
//    cross-lane reduction are f64 (full rate on CDNA), which keeps the result
//    closer to the exact dot product than the CPU's sequential f32 sum.
//  - int8 mode (activations quantized per 256 with an f32 scale, see
//    quant.hip) does the integer dot with v_dot4_i32_i8 and keeps exact int32
//    per-sub-block sums; the float epilogue runs once per unit.
//  - Fused QKV: up to three jobs (same dtype) in one launch; waves are dealt
//    out to jobs in order. Gated: the wave computes R rows of gate AND up,
//    then writes silu(g) * u.
#include <algorithm>

#include "kernels.h"

namespace mdma {
namespace {

// Launch shape (tuned on MI355X; overridable at build time for sweeps).
#ifndef MDMA_GEMV_R_F32
#define MDMA_GEMV_R_F32 4
#endif
#ifndef MDMA_GEMV_R_I8
#define MDMA_GEMV_R_I8 2
#endif
constexpr int WAVES = 4;                // waves per workgroup
constexpr int R_F32 = MDMA_GEMV_R_F32;  // rows per wave, f32-activation kernels
constexpr int R_I8 = MDMA_GEMV_R_I8;    // rows per wave, int8-activation kernels

struct Job {
  const uint8_t *w;
  float *y;
  uint32_t n_out, n_in, waves;
};
struct JobSet {
  Job j[3];
  int n;
};

__device__ __forceinline__ float ub(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xffu); }
__device__ __forceinline__ float sb(uint32_t v, int k) { return (float)(int8_t)((v >> (8 * k)) & 0xffu); }

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Locate this wave's job and first row (R rows per wave); false when the
// wave has no rows. The wave index goes through readfirstlane so the job
// choice and every job field stay in scalar registers: a per-lane index
// into the kernel-argument struct would turn each use into a dependent
// memory load in front of every weight load.
template <int R>
__device__ __forceinline__ bool locate(const JobSet &js, bool gated, Job &J, const uint8_t *&wu, uint32_t &row0) {
  uint32_t gw = blockIdx.x * WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t w0 = js.j[0].waves, w1 = js.n > 1 ? js.j[1].waves : 0;
  int ji = 0;
  if (js.n > 1 && gw >= w0) {
    gw -= w0;
    ji = 1;
    if (js.n > 2 && gw >= w1) {
      gw -= w1;
      ji = 2;
    }
  }
  J = ji == 0 ? js.j[0] : (ji == 1 ? js.j[1] : js.j[2]);
  if (gw >= J.waves) return false;
  wu = gated ? js.j[1].w : J.w;
  row0 = gw * R;
  return true;
}

// ---------------------------------------------------------------- Q4_K ----

// Six-bit (scale, min) pairs of sub-blocks 2p and 2p+1 from the 12 scale
// bytes (get_scale_min_k4 of reference kernels.hip:19-27, evaluated for four
// sub-blocks at once in packed bytes).
__device__ __forceinline__ void q4k_scales(uint4 hd, int p, float &sca, float &scb, float &ma, float &mb) {
  uint32_t s0 = hd.y, s1 = hd.z, s2 = hd.w;
  uint32_t scw = p < 2 ? (s0 & 0x3F3F3F3Fu) : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
  uint32_t mw = p < 2 ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
  int sh = (p & 1) * 16;
  sca = ub(scw >> sh, 0);
  scb = ub(scw >> sh, 1);
  ma = ub(mw >> sh, 0);
  mb = ub(mw >> sh, 1);
}

// Integer part of an int8-mode Q4_K unit: dots of the 16 low nibbles with
// qa (16 int8) and of the 16 high nibbles with qb.
__device__ __forceinline__ void q4k_unit_isum(uint4 qs, uint4 qa, uint4 qb, int &ia, int &ib) {
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
  const uint32_t a[4] = {qa.x, qa.y, qa.z, qa.w};
  const uint32_t b[4] = {qb.x, qb.y, qb.z, qb.w};
  ia = 0;
  ib = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    ia = __builtin_amdgcn_sdot4((int)(w[k] & 0x0F0F0F0Fu), (int)a[k], ia, false);
    ib = __builtin_amdgcn_sdot4((int)((w[k] >> 4) & 0x0F0F0F0Fu), (int)b[k], ib, false);
  }
}

// ---------------------------------------------------------------- Q6_K ----

struct Q6Unit {
  uint32_t qa[2], qb[2], qh[2];  // ql[l0..+8], ql[32+l0..+8], qh[l0..+8] of one half
  uint32_t sc;                   // 4 sub-scales (quarters 0..3) as bytes
  uint32_t d;                    // f16 bits
};

// Unit c in 0..7 of a block: half n = c>>2, column group g = c&3 (l0 = 8g).
__device__ __forceinline__ Q6Unit q6_load(const uint8_t *blk, int c) {
  const int n = c >> 2, g = c & 3, l0 = 8 * g;
  Q6Unit u;
  const uint8_t *ql = blk + 64 * n + l0, *qh = blk + 128 + 32 * n + l0;
  u.qa[0] = ld2x16(ql);
  u.qa[1] = ld2x16(ql + 4);
  u.qb[0] = ld2x16(ql + 32);
  u.qb[1] = ld2x16(ql + 36);
  u.qh[0] = ld2x16(qh);
  u.qh[1] = ld2x16(qh + 4);
  // sc[8n + g/2 + 2r], r = 0..3: byte (g>>1) of the halfwords at 192+8n+2r.
  const uint8_t *s = blk + 192 + 8 * n;
  const int sh = (g >> 1) * 8;
  u.sc = ((ldu16(s) >> sh) & 0xff) | (((ldu16(s + 2) >> sh) & 0xff) << 8) |
         (((ldu16(s + 4) >> sh) & 0xff) << 16) | (((ldu16(s + 6) >> sh) & 0xff) << 24);
  u.d = ldu16(blk + 208);
  return u;
}

// Six-bit unsigned quants (0..63) of quarter r, word k (4 columns).
__device__ __forceinline__ uint32_t q6_u(const Q6Unit &u, int r, int k) {
  const uint32_t h = u.qh[k];
  switch (r) {
    case 0: return (u.qa[k] & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
    case 1: return (u.qb[k] & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
    case 2: return ((u.qa[k] >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
    default: return ((u.qb[k] >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
  }
}

// Integer dot of quarter r's 8 quants (q = u - 32) with 8 int8 activations.
__device__ __forceinline__ int q6_quarter_isum(const Q6Unit &u, int r, uint32_t x0, uint32_t x1) {
  int acc = __builtin_amdgcn_sdot4((int)q6_u(u, r, 0), (int)x0, 0, false);
  acc = __builtin_amdgcn_sdot4((int)q6_u(u, r, 1), (int)x1, acc, false);
  int sx = __builtin_amdgcn_sdot4((int)x0, 0x01010101, 0, false);
  sx = __builtin_amdgcn_sdot4((int)x1, 0x01010101, sx, false);
  return acc - 32 * sx;
}

// ---------------------------------------------------------------- Q8_0 ----

struct Q8Unit {
  uint32_t q[4];  // 16 int8 quants
  uint32_t d;
};
// Unit c in 0..1 of a 34-byte block: quants [16c, 16c+16).
__device__ __forceinline__ Q8Unit q8_load(const uint8_t *blk, int c) {
  Q8Unit u;
  const uint8_t *q = blk + 2 + 16 * c;
#pragma unroll
  for (int k = 0; k < 4; k++) u.q[k] = ld2x16(q + 4 * k);
  u.d = ldu16(blk);
  return u;
}

// ------------------------------------------------------- f32 mode kernel ----
//
// Exact products: a quant byte b (0..255) placed by one v_perm_b32 into
// mantissa bits 40..47 of an f64 whose exponent is fixed gives the double
// 2 + b/2048 with no conversion instruction. Its product with an activation
// (converted once to f64 and reused by every row of the wave) is exact, and
// the unit's 16- or 8-term chains accumulate in f64, so
//     sum(q*x) = 2048*acc - (4096 + 2048*bias)*X,  X = sum(x)
// where q = b - bias. Each weight costs one perm and one f64 FMA; the
// result is the exact dot product up to f64 rounding, then one f32 rounding.

template <int DT>
struct F32Fmt;

// Q4_K unit c (0..7): 16 quant bytes; low nibbles are columns 64p+16h+[0,16)
// of sub-block 2p, high nibbles the same columns +32 of sub-block 2p+1.
template <>
struct F32Fmt<DT_Q4_K> {
  static constexpr uint32_t ELEMS = 256, BYTES = 144, UNITS = 8, NX = 32, NG = 2;
  struct W {
    uint4 hd, qs;
  };
  __device__ static W load(const uint8_t *blk, int c) { return W{ld16(blk), ld16(blk + 16 + 16 * c)}; }
  __device__ static W zero() { return W{make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)}; }
  // x index i (0..31) -> column in the block; group of i.
  __device__ static int col(int c, int i) { return ((c >> 1) << 6) + ((c & 1) << 4) + (i & 15) + ((i >> 4) << 5); }
  __device__ static double dot(const W &w, int c, const double *xd, const double *X) {
    const uint32_t q[4] = {w.qs.x, w.qs.y, w.qs.z, w.qs.w};
    double aa = 0.0, ab = 0.0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      aa = fma4(q[k] & 0x0F0F0F0Fu, xd + 4 * k, aa);
      ab = fma4((q[k] >> 4) & 0x0F0F0F0Fu, xd + 16 + 4 * k, ab);
    }
    float sca, scb, ma, mb;
    q4k_scales(w.hd, c >> 1, sca, scb, ma, mb);
    const float d = h2f(w.hd.x), dmin = h2f(w.hd.x >> 16);
    const double dsa = (double)(d * sca), dsb = (double)(d * scb);
    const double dma = (double)(dmin * ma), dmb = (double)(dmin * mb);
    // dsa*(2048*aa - 4096*Xa) - dma*Xa, likewise for b.
    double r = fma(2048.0 * dsa, aa, -fma(4096.0, dsa, dma) * X[0]);
    r += fma(2048.0 * dsb, ab, -fma(4096.0, dsb, dmb) * X[1]);
    return r;
  }
};

// Q6_K unit c (0..7): half n = c>>2, columns 8g..8g+7 (g = c&3) of each of
// the 4 quarters r (columns 128n + 32r + 8g + [0,8)); six-bit quants u, q = u - 32.
template <>
struct F32Fmt<DT_Q6_K> {
  static constexpr uint32_t ELEMS = 256, BYTES = 210, UNITS = 8, NX = 32, NG = 4;
  using W = Q6Unit;
  __device__ static W load(const uint8_t *blk, int c) { return q6_load(blk, c); }
  __device__ static W zero() { return Q6Unit{{0, 0}, {0, 0}, {0, 0}, 0, 0}; }
  __device__ static int col(int c, int i) { return 128 * (c >> 2) + 32 * (i >> 3) + 8 * (c & 3) + (i & 7); }
  __device__ static double dot(const W &w, int c, const double *xd, const double *X) {
    double r = 0.0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      double a = fma4(q6_u(w, q, 0), xd + 8 * q, 0.0);
      a = fma4(q6_u(w, q, 1), xd + 8 * q + 4, a);
      const double s = (double)(int8_t)((w.sc >> (8 * q)) & 0xff);
      r = fma(s, fma(2048.0, a, -4128.0 * X[q]), r);
    }
    return (double)h2f(w.d) * r;
  }
};

// Q8_0 unit c (0..1): quants 16c..16c+15 of a 34-byte block; bytes biased by
// 128 so b = q + 128.
template <>
struct F32Fmt<DT_Q8_0> {
  static constexpr uint32_t ELEMS = 32, BYTES = 34, UNITS = 2, NX = 16, NG = 1;
  using W = Q8Unit;
  __device__ static W load(const uint8_t *blk, int c) { return q8_load(blk, c); }
  __device__ static W zero() { return Q8Unit{{0, 0, 0, 0}, 0}; }
  __device__ static int col(int c, int i) { return 16 * c + i; }
  __device__ static double dot(const W &w, int, const double *xd, const double *X) {
    double a = 0.0;
#pragma unroll
    for (int k = 0; k < 4; k++) a = fma4(w.q[k] ^ 0x80808080u, xd + 4 * k, a);
    return (double)h2f(w.d) * fma(2048.0, a, -4224.0 * X[0]);
  }
};

// One wave owns R rows (2R when gated: gate then up) of one job; lanes stride
// over the row's units, x is read from global memory (L2-resident) per unit.
template <class F, int R, int TT, bool GATED>
__global__ __launch_bounds__(256) void gemv_f32(JobSet js, const float *__restrict__ x, uint32_t T,
                                                float *__restrict__ ygated) {
  Job J;
  const uint8_t *wu;
  uint32_t row0;
  if (!locate<R>(js, GATED, J, wu, row0)) return;
  const int lane = threadIdx.x & 63;
  const uint32_t n_in = J.n_in, nb = n_in / F::ELEMS, units = nb * F::UNITS;
  const size_t rb = (size_t)nb * F::BYTES;
  constexpr int NR = GATED ? 2 * R : R;
  double acc[NR][TT];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = 0.0;

  for (uint32_t u = lane; u < units; u += 64) {
    const uint32_t b = u / F::UNITS;
    const int c = u % F::UNITS;
    typename F::W wd[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const uint32_t row = row0 + (r % R);
      const uint8_t *base = (r < R ? J.w : wu);
      wd[r] = row < J.n_out ? F::load(base + row * rb + (size_t)b * F::BYTES, c) : F::zero();
    }
#pragma unroll
    for (int t = 0; t < TT; t++) {
      if (t >= (int)T) break;
      const float *xt = x + (size_t)t * n_in + (size_t)b * F::ELEMS;
      double xd[F::NX];
#pragma unroll
      for (int i = 0; i < (int)F::NX; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(xt + F::col(c, i));
        xd[i] = v.x, xd[i + 1] = v.y, xd[i + 2] = v.z, xd[i + 3] = v.w;
      }
      double X[F::NG];
#pragma unroll
      for (int g = 0; g < (int)F::NG; g++) {
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < (int)(F::NX / F::NG); i++) s += xd[g * (F::NX / F::NG) + i];
        X[g] = s;
      }
#pragma unroll
      for (int r = 0; r < NR; r++) acc[r][t] += F::dot(wd[r], c, xd, X);
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = wave_sum(acc[r][t]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = row0 + r;
      if (row >= J.n_out) break;
#pragma unroll
      for (int t = 0; t < TT; t++) {
        if (t >= (int)T) break;
        if (GATED) {
          const float g = (float)acc[r][t], up = (float)acc[R + r][t];
          ygated[(size_t)t * J.n_out + row] = g / (1.0f + expf(-g)) * up;
        } else {
          J.y[(size_t)t * J.n_out + row] = (float)acc[r][t];
        }
      }
    }
  }
}

// F32 / F16 weights: plain strided dot with exact f64 products (not a hot
// path; kept for the trait's full dtype set). One wave per row.
template <int DT, bool GATED>
__global__ __launch_bounds__(256) void gemv_plain(JobSet js, const float *__restrict__ x, uint32_t T,
                                                  float *__restrict__ ygated) {
  Job J;
  const uint8_t *wu;
  uint32_t row;
  if (!locate<1>(js, GATED, J, wu, row)) return;
  const int lane = threadIdx.x & 63;
  const uint32_t n_in = J.n_in;
  for (uint32_t t = 0; t < T; t++) {
    double a = 0.0, b = 0.0;
    for (uint32_t i = lane; i < n_in; i += 64) {
      float wv, uv = 0.f;
      if (DT == DT_F32) {
        wv = reinterpret_cast<const float *>(J.w)[(size_t)row * n_in + i];
        if (GATED) uv = reinterpret_cast<const float *>(wu)[(size_t)row * n_in + i];
      } else {
        wv = h2f(reinterpret_cast<const uint16_t *>(J.w)[(size_t)row * n_in + i]);
        if (GATED) uv = h2f(reinterpret_cast<const uint16_t *>(wu)[(size_t)row * n_in + i]);
      }
      const double xv = (double)x[(size_t)t * n_in + i];
      a = fma((double)wv, xv, a);
      if (GATED) b = fma((double)uv, xv, b);
    }
    a = wave_sum(a);
    if (GATED) b = wave_sum(b);
    if (lane == 0) {
      if (GATED) {
        const float g = (float)a, up = (float)b;
        ygated[(size_t)t * J.n_out + row] = g / (1.0f + expf(-g)) * up;
      } else {
        J.y[(size_t)t * J.n_out + row] = (float)a;
      }
    }
  }
}


// ------------------------------------------------------ int8 mode kernel ----
// qx: int8 [T, n_in]; dx: f32 [T, n_in/256]; s16: i32 [T, n_in/16].

template <int TT, bool GATED>
__global__ __launch_bounds__(256) void gemv_q4k_i8(JobSet js, const int8_t *__restrict__ qx,
                                                   const float *__restrict__ dx, const int32_t *__restrict__ s16,
                                                   uint32_t T, float *__restrict__ ygated) {
  Job J;
  const uint8_t *wu;
  uint32_t row0;
  constexpr int R = R_I8;
  if (!locate<R>(js, GATED, J, wu, row0)) return;
  const int lane = threadIdx.x & 63;
  const uint32_t n_in = J.n_in, nb = n_in >> 8, units = nb * 8;
  const size_t rb = (size_t)nb * 144;
  constexpr int NR = GATED ? 2 * R : R;
  double acc[NR][TT];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = 0.0;
  for (uint32_t u = lane; u < units; u += 64) {
    const uint32_t b = u >> 3;
    const int c = u & 7, p = c >> 1;
    uint4 hd[NR], qs[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const uint32_t row = row0 + (r % R);
      const uint8_t *base = (r < R ? J.w : wu);
      if (row < J.n_out) {
        const uint8_t *blk = base + row * rb + (size_t)b * 144;
        hd[r] = ld16(blk);
        qs[r] = ld16(blk + 16 + 16 * c);
      } else {
        hd[r] = make_uint4(0, 0, 0, 0);
        qs[r] = make_uint4(0, 0, 0, 0);
      }
    }
    const uint32_t ca = b * 256 + (p << 6) + ((c & 1) << 4);
#pragma unroll
    for (int t = 0; t < TT; t++) {
      if (t >= (int)T) break;
      const int8_t *xt = qx + (size_t)t * n_in;
      const uint4 qa = *reinterpret_cast<const uint4 *>(xt + ca);
      const uint4 qb = *reinterpret_cast<const uint4 *>(xt + ca + 32);
      const int sa = s16[(size_t)t * (n_in >> 4) + (ca >> 4)];
      const int sbb = s16[(size_t)t * (n_in >> 4) + ((ca + 32) >> 4)];
      const float d8 = dx[(size_t)t * nb + b];
#pragma unroll
      for (int r = 0; r < NR; r++) {
        int ia, ib;
        q4k_unit_isum(qs[r], qa, qb, ia, ib);
        float sca, scb, ma, mb;
        q4k_scales(hd[r], p, sca, scb, ma, mb);
        const int A = (int)sca * ia + (int)scb * ib;
        const int B = (int)ma * sa + (int)mb * sbb;
        const float d = h2f(hd[r].x), dmin = h2f(hd[r].x >> 16);
        acc[r][t] += (double)(d8 * fmaf(d, (float)A, -dmin * (float)B));
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = wave_sum(acc[r][t]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = row0 + r;
      if (row >= J.n_out) break;
#pragma unroll
      for (int t = 0; t < TT; t++) {
        if (t >= (int)T) break;
        if (GATED) {
          const float g = (float)acc[r][t], up = (float)acc[R + r][t];
          ygated[(size_t)t * J.n_out + row] = g / (1.0f + expf(-g)) * up;
        } else {
          J.y[(size_t)t * J.n_out + row] = (float)acc[r][t];
        }
      }
    }
  }
}

template <int TT, bool GATED>
__global__ __launch_bounds__(256) void gemv_q6k_i8(JobSet js, const int8_t *__restrict__ qx,
                                                   const float *__restrict__ dx, const int32_t *__restrict__ s16,
                                                   uint32_t T, float *__restrict__ ygated) {
  Job J;
  const uint8_t *wu;
  uint32_t row0;
  constexpr int R = R_I8;
  if (!locate<R>(js, GATED, J, wu, row0)) return;
  const int lane = threadIdx.x & 63;
  const uint32_t n_in = J.n_in, nb = n_in >> 8, units = nb * 8;
  const size_t rb = (size_t)nb * 210;
  constexpr int NR = GATED ? 2 * R : R;
  double acc[NR][TT];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = 0.0;
  for (uint32_t u = lane; u < units; u += 64) {
    const uint32_t b = u >> 3;
    const int c = u & 7;
    Q6Unit wd[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const uint32_t row = row0 + (r % R);
      const uint8_t *base = (r < R ? J.w : wu);
      if (row < J.n_out)
        wd[r] = q6_load(base + row * rb + (size_t)b * 210, c);
      else
        wd[r] = Q6Unit{{0, 0}, {0, 0}, {0, 0}, 0, 0};
    }
#pragma unroll
    for (int t = 0; t < TT; t++) {
      if (t >= (int)T) break;
      const int8_t *xt = qx + (size_t)t * n_in + (size_t)b * 256;
      uint32_t xq[4][2];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint2 v = *reinterpret_cast<const uint2 *>(xt + 128 * (c >> 2) + 32 * q + 8 * (c & 3));
        xq[q][0] = v.x;
        xq[q][1] = v.y;
      }
      const float d8 = dx[(size_t)t * nb + b];
#pragma unroll
      for (int r = 0; r < NR; r++) {
        int A = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) A += (int)(int8_t)((wd[r].sc >> (8 * q)) & 0xff) *
                                         q6_quarter_isum(wd[r], q, xq[q][0], xq[q][1]);
        acc[r][t] += (double)(d8 * (h2f(wd[r].d) * (float)A));
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = wave_sum(acc[r][t]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = row0 + r;
      if (row >= J.n_out) break;
#pragma unroll
      for (int t = 0; t < TT; t++) {
        if (t >= (int)T) break;
        if (GATED) {
          const float g = (float)acc[r][t], up = (float)acc[R + r][t];
          ygated[(size_t)t * J.n_out + row] = g / (1.0f + expf(-g)) * up;
        } else {
          J.y[(size_t)t * J.n_out + row] = (float)acc[r][t];
        }
      }
    }
  }
}

template <int TT, bool GATED>
__global__ __launch_bounds__(256) void gemv_q8_i8(JobSet js, const int8_t *__restrict__ qx,
                                                  const float *__restrict__ dx, const int32_t *__restrict__ s16,
                                                  uint32_t T, float *__restrict__ ygated) {
  Job J;
  const uint8_t *wu;
  uint32_t row0;
  constexpr int R = R_I8;
  if (!locate<R>(js, GATED, J, wu, row0)) return;
  const int lane = threadIdx.x & 63;
  const uint32_t n_in = J.n_in, nb = n_in >> 5, units = nb * 2;
  const size_t rb = (size_t)nb * 34;
  constexpr int NR = GATED ? 2 * R : R;
  double acc[NR][TT];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = 0.0;
  for (uint32_t u = lane; u < units; u += 64) {
    const uint32_t b = u >> 1;
    const int c = u & 1;
    Q8Unit wd[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const uint32_t row = row0 + (r % R);
      const uint8_t *base = (r < R ? J.w : wu);
      if (row < J.n_out)
        wd[r] = q8_load(base + row * rb + (size_t)b * 34, c);
      else
        wd[r] = Q8Unit{{0, 0, 0, 0}, 0};
    }
    const uint32_t e0 = b * 32 + 16 * c;
#pragma unroll
    for (int t = 0; t < TT; t++) {
      if (t >= (int)T) break;
      const uint4 xv = *reinterpret_cast<const uint4 *>(qx + (size_t)t * n_in + e0);
      const float d8 = dx[(size_t)t * (n_in >> 8) + (e0 >> 8)];
#pragma unroll
      for (int r = 0; r < NR; r++) {
        int s = __builtin_amdgcn_sdot4((int)wd[r].q[0], (int)xv.x, 0, false);
        s = __builtin_amdgcn_sdot4((int)wd[r].q[1], (int)xv.y, s, false);
        s = __builtin_amdgcn_sdot4((int)wd[r].q[2], (int)xv.z, s, false);
        s = __builtin_amdgcn_sdot4((int)wd[r].q[3], (int)xv.w, s, false);
        acc[r][t] += (double)(d8 * (h2f(wd[r].d) * (float)s));
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int t = 0; t < TT; t++) acc[r][t] = wave_sum(acc[r][t]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t row = row0 + r;
      if (row >= J.n_out) break;
#pragma unroll
      for (int t = 0; t < TT; t++) {
        if (t >= (int)T) break;
        if (GATED) {
          const float g = (float)acc[r][t], up = (float)acc[R + r][t];
          ygated[(size_t)t * J.n_out + row] = g / (1.0f + expf(-g)) * up;
        } else {
          J.y[(size_t)t * J.n_out + row] = (float)acc[r][t];
        }
      }
    }
  }
}

// --------------------------------------------------- int8 quantizer -------
// Groups of G values (32 or 256) get amax, d = amax/127 and
// q = round-half-away(x * 127/amax); exact sums of every 16 quants are kept.
// A lane quantizes 4 consecutive values, so a wave covers 256 values: one
// group of 256 or eight groups of 32 (G/4 lanes each).
template <int G>
__global__ __launch_bounds__(256) void quantize_act_kernel(const float *__restrict__ x, uint64_t n,
                                                           int8_t *__restrict__ q, float *__restrict__ d,
                                                           int32_t *__restrict__ s16) {
  constexpr int LPG = G / 4;  // lanes per group
  const uint64_t base = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const bool live = base < n;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (live) {
    const float4 t = *reinterpret_cast<const float4 *>(x + base);
    v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
  }
  static_assert(LPG == 8 || LPG == 64, "groups of 32 or 256");
  // Group maxima and 16-column sums through DPP lane moves (every lane of
  // the group gets the result).
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  if constexpr (LPG == 64) {
    amax = wave_max_all(amax);
  } else {
    amax = dpp_max<0xB1, 0xF>(amax);
    amax = dpp_max<0x4E, 0xF>(amax);
    amax = dpp_max<0x141, 0xF>(amax);  // half-row mirror: 8 lanes
  }
  const float inv = amax == 0.f ? 0.f : 127.0f / amax;
  int qi[4], sum = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    qi[k] = q8_quant(v[k], inv);
    sum += qi[k];
  }
  sum += (int)dpp_u32<0xB1, 0xF>((uint32_t)sum);  // 16 values = 4 lanes
  sum += (int)dpp_u32<0x4E, 0xF>((uint32_t)sum);
  if (!live) return;
  *reinterpret_cast<uint32_t *>(q + base) = pack4_i8(qi[0], qi[1], qi[2], qi[3]);
  const int lane = threadIdx.x & 63;
  if ((lane & 3) == 0) s16[base / 16] = sum;
  if ((lane & (LPG - 1)) == 0) d[base / G] = amax / 127.0f;
}

// --------------------------------------------------- block-dot debug ------
// out[t][row][s] for sub-blocks of 32 (Q4_K, Q8_0) or 16 (Q6_K), through the
// same unit functions the int8 GEMV uses.
__global__ __launch_bounds__(256) void block_dot_kernel(int32_t dtype, const uint8_t *__restrict__ w,
                                                        uint32_t n_out, uint32_t n_in, const int8_t *__restrict__ qx,
                                                        uint32_t T, int32_t *__restrict__ out) {
  const uint32_t sub = dtype == DT_Q6_K ? 16 : 32, nsub = n_in / sub;
  const size_t total = (size_t)T * n_out * nsub;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const uint32_t s = idx % nsub, row = (idx / nsub) % n_out, t = idx / ((size_t)nsub * n_out);
  const int8_t *xt = qx + (size_t)t * n_in;
  int32_t v = 0;
  if (dtype == DT_Q4_K) {
    // Sub-block s = 8b + j; units 2p, 2p+1 with p = j/2 hold its two halves,
    // low nibbles for even j and high for odd j.
    const uint32_t b = s / 8, j = s % 8, p = j / 2;
    const uint8_t *blk = w + (size_t)row * (n_in / 256) * 144 + (size_t)b * 144;
    for (int h = 0; h < 2; h++) {
      const int c = 2 * p + h;
      const uint32_t ca = b * 256 + (p << 6) + (h << 4);
      int ia, ib;
      q4k_unit_isum(ld16(blk + 16 + 16 * c), *reinterpret_cast<const uint4 *>(xt + ca),
                    *reinterpret_cast<const uint4 *>(xt + ca + 32), ia, ib);
      v += (j & 1) ? ib : ia;
    }
  } else if (dtype == DT_Q6_K) {
    // Sub-block s = 16b + 8n + 2r + k2 covers l in [16 k2, 16 k2 + 16) of
    // quarter r of half n: units with g = 2 k2 and 2 k2 + 1.
    const uint32_t b = s / 16, i = s % 16, n = i / 8, r = (i % 8) / 2, k2 = i % 2;
    const uint8_t *blk = w + (size_t)row * (n_in / 256) * 210 + (size_t)b * 210;
    for (int gg = 0; gg < 2; gg++) {
      const int g = 2 * k2 + gg, c = 4 * n + g;
      Q6Unit u = q6_load(blk, c);
      const uint2 xv = *reinterpret_cast<const uint2 *>(xt + b * 256 + 128 * n + 32 * r + 8 * g);
      v += q6_quarter_isum(u, r, xv.x, xv.y);
    }
  } else {
    const uint8_t *blk = w + (size_t)row * (n_in / 32) * 34 + (size_t)s * 34;
    for (int c = 0; c < 2; c++) {
      Q8Unit u = q8_load(blk, c);
      const uint4 xv = *reinterpret_cast<const uint4 *>(xt + s * 32 + 16 * c);
      v = __builtin_amdgcn_sdot4((int)u.q[0], (int)xv.x, v, false);
      v = __builtin_amdgcn_sdot4((int)u.q[1], (int)xv.y, v, false);
      v = __builtin_amdgcn_sdot4((int)u.q[2], (int)xv.z, v, false);
      v = __builtin_amdgcn_sdot4((int)u.q[3], (int)xv.w, v, false);
    }
  }
  out[idx] = v;
}

// ------------------------------------------------------------ launchers ----

uint32_t waves_for(int32_t dtype, uint64_t n_out, int rows_per_wave) {
  if (dtype == DT_F32 || dtype == DT_F16) return (uint32_t)n_out;
  return (uint32_t)((n_out + rows_per_wave - 1) / rows_per_wave);
}

JobSet make_set(const GemvJob *jobs, int n, int rows_per_wave) {
  JobSet js{};
  js.n = n;
  for (int i = 0; i < n; i++) {
    js.j[i].w = jobs[i].w;
    js.j[i].y = jobs[i].y;
    js.j[i].n_out = (uint32_t)jobs[i].n_out;
    js.j[i].n_in = (uint32_t)jobs[i].n_in;
    js.j[i].waves = waves_for(jobs[i].dtype, jobs[i].n_out, rows_per_wave);
  }
  return js;
}

uint32_t grid_of(const JobSet &js) {
  uint64_t w = 0;
  for (int i = 0; i < js.n; i++) w += js.j[i].waves;
  return (uint32_t)((w + WAVES - 1) / WAVES);
}

template <bool GATED>
void dispatch_f32(mdma_ctx *ctx, int32_t dt, const JobSet &js, const float *x, uint32_t T, float *yg) {
  const dim3 grid(grid_of(js)), block(64 * WAVES);
#define MDMA_F32_CASE(TT)                                                                                          \
  switch (dt) {                                                                                                    \
    case DT_Q4_K: gemv_f32<F32Fmt<DT_Q4_K>, R_F32, TT, GATED><<<grid, block, 0, ctx->stream>>>(js, x, T, yg); break; \
    case DT_Q6_K: gemv_f32<F32Fmt<DT_Q6_K>, R_F32, TT, GATED><<<grid, block, 0, ctx->stream>>>(js, x, T, yg); break; \
    case DT_Q8_0: gemv_f32<F32Fmt<DT_Q8_0>, R_F32, TT, GATED><<<grid, block, 0, ctx->stream>>>(js, x, T, yg); break; \
    case DT_F32: gemv_plain<DT_F32, GATED><<<grid, block, 0, ctx->stream>>>(js, x, T, yg); break;                  \
    case DT_F16: gemv_plain<DT_F16, GATED><<<grid, block, 0, ctx->stream>>>(js, x, T, yg); break;                  \
    default: fail(MDMA_ERR_NOT_IMPLEMENTED, "gemv: dtype");                                                        \
  }
  if (T <= 1) { MDMA_F32_CASE(1) }
  else if (T <= 2) { MDMA_F32_CASE(2) }
  else if (T <= 4) { MDMA_F32_CASE(4) }
  else { MDMA_F32_CASE(8) }
#undef MDMA_F32_CASE
  hip_check(hipGetLastError(), "gemv f32 launch");
}

template <bool GATED>
void dispatch_i8(mdma_ctx *ctx, int32_t dt, const JobSet &js, const int8_t *qx, const float *dx,
                 const int32_t *s16, uint32_t T, float *yg) {
  const dim3 grid(grid_of(js)), block(64 * WAVES);
#define MDMA_I8_CASE(TT)                                                                                   \
  switch (dt) {                                                                                            \
    case DT_Q4_K: gemv_q4k_i8<TT, GATED><<<grid, block, 0, ctx->stream>>>(js, qx, dx, s16, T, yg); break; \
    case DT_Q6_K: gemv_q6k_i8<TT, GATED><<<grid, block, 0, ctx->stream>>>(js, qx, dx, s16, T, yg); break; \
    case DT_Q8_0: gemv_q8_i8<TT, GATED><<<grid, block, 0, ctx->stream>>>(js, qx, dx, s16, T, yg); break;  \
    default: fail(MDMA_ERR_NOT_IMPLEMENTED, "gemv i8: dtype");                                             \
  }
  if (T <= 1) { MDMA_I8_CASE(1) }
  else if (T <= 2) { MDMA_I8_CASE(2) }
  else if (T <= 4) { MDMA_I8_CASE(4) }
  else { MDMA_I8_CASE(8) }
#undef MDMA_I8_CASE
  hip_check(hipGetLastError(), "gemv i8 launch");
}

bool same_dtype(const GemvJob *jobs, int n) {
  for (int i = 1; i < n; i++)
    if (jobs[i].dtype != jobs[0].dtype || jobs[i].n_in != jobs[0].n_in) return false;
  return true;
}

// Token chunks of at most 8 per launch.
template <class F>
void by_chunks(uint64_t T, F &&f) {
  for (uint64_t t0 = 0; t0 < T; t0 += 8) f(t0, T - t0 < 8 ? T - t0 : 8);
}

GemvJob offset_job(const GemvJob &j, uint64_t t0) {
  GemvJob o = j;
  if (o.y) o.y += t0 * j.n_out;
  if (o.dots) o.dots += t0 * j.n_out * dot_subs(j.dtype, j.n_in);
  return o;
}

bool is_i8_dtype(int32_t dt) { return dt == DT_Q4_K || dt == DT_Q6_K || dt == DT_Q8_0; }

}  // namespace

// The int8 activations of x [T, n_in] in the context's activation buffer,
// quantized now unless that buffer already holds exactly this x (same
// pointer and shape, no write since; see q8_invalidate).
uint64_t q8_slot_bytes(uint64_t n) {
  return (n + 255) / 256 * 256 + (n / 256 * 4 + 255) / 256 * 256 + n / 16 * 4 + 256;
}

uint64_t gemm_input_bytes(uint64_t n) {
  return (n + 255) / 256 * 256 + (n / 32 * 4 + 255) / 256 * 256 + (n / 16 * 4 + 255) / 256 * 256;
}

void q8_slots(mdma_ctx *ctx, uint64_t T, uint64_t n_in, int8_t **qx, float **dx, int32_t **s16) {
  const uint64_t n = T * n_in;
  const uint64_t qb = (n + 255) / 256 * 256, db = (n / 256 * 4 + 255) / 256 * 256;
  char *s;
  if (ctx->fixed_scratch) {  // an allocation-free call: its fixed buffer
    if (q8_slot_bytes(n) > ctx->fixed_cap) fail(MDMA_ERR_BUFFER_BUDGET, "int8 activations exceed the fixed scratch");
    s = ctx->fixed_scratch;
  } else {
    s = q8_buffer(ctx, q8_slot_bytes(n));
  }
  *qx = reinterpret_cast<int8_t *>(s);
  *dx = reinterpret_cast<float *>(s + qb);
  *s16 = reinterpret_cast<int32_t *>(s + qb + db);
}

void q8_mark(mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in) {
  ctx->q8_valid = true;
  ctx->q8_x = x;
  ctx->q8_n = T * n_in;
  ctx->q8_n_in = n_in;
}

bool q8_holds(mdma_ctx *ctx, const float *x, uint64_t n) {
  return ctx->q8_valid && ctx->q8_x == x && ctx->q8_n == n && ctx->q8_n_in == n;
}

void quantize_into_scratch(mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in, int8_t **qx, float **dx,
                           int32_t **s16) {
  q8_slots(ctx, T, n_in, qx, dx, s16);
  const uint64_t n = T * n_in;
  if (ctx->q8_valid && ctx->q8_x == x && ctx->q8_n == n && ctx->q8_n_in == n_in) return;
  launch_quantize_act(ctx, x, n, 256, *qx, *dx, *s16);
  q8_mark(ctx, x, T, n_in);
}


// BATCH_MIN_TOKENS: below it int8-mode GEMVs of prepared rows run the
// row-team kernels, which keep each token's activations in registers. At
// Llama-3-8B shapes the batch kernel's ring is faster from 3 tokens on every
// weight (gate/up 16.2 us against 28.9 us at 3 tokens); at 2 the row teams
// still win on the Q6_K down and head.

// Prepared-layout jobs go to the row-team kernels; a mix of layouts or
// dtypes runs job by job; raw GGUF jobs use the kernels above.
static bool any_prepared(const GemvJob *jobs, int n) {
  for (int i = 0; i < n; i++)
    if (jobs[i].layout == MDMA_LAYOUT_GFX950) return true;
  return false;
}

void launch_gemv_f32(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t T) {
  if (team_layout_ok(jobs, n_jobs)) {
    launch_gemv_team(ctx, MDMA_ACT_F32, jobs, n_jobs, false, x, T, nullptr);
    return;
  }
  if (!same_dtype(jobs, n_jobs) || any_prepared(jobs, n_jobs)) {
    for (int i = 0; i < n_jobs; i++) launch_gemv_f32(ctx, jobs + i, 1, x, T);
    return;
  }
  by_chunks(T, [&](uint64_t t0, uint64_t tn) {
    GemvJob js[3];
    for (int i = 0; i < n_jobs; i++) js[i] = offset_job(jobs[i], t0);
    dispatch_f32<false>(ctx, jobs[0].dtype, make_set(js, n_jobs, R_F32), x + t0 * jobs[0].n_in, (uint32_t)tn, nullptr);
  });
}

void launch_gemv_f32_gated(mdma_ctx *ctx, const GemvJob &gate, const GemvJob &up, const float *x, uint64_t T,
                           float *y) {
  const GemvJob gu[2] = {gate, up};
  if (team_layout_ok(gu, 2)) {
    launch_gemv_team(ctx, MDMA_ACT_F32, gu, 2, true, x, T, y);
    return;
  }
  if (gate.dtype != up.dtype || any_prepared(gu, 2)) {
    launch_gemv_f32(ctx, &gate, 1, x, T);
    launch_gemv_f32(ctx, &up, 1, x, T);
    launch_silu_mul(ctx, gate.y, up.y, y, T * gate.n_out);
    return;
  }
  by_chunks(T, [&](uint64_t t0, uint64_t tn) {
    GemvJob js[2] = {offset_job(gate, t0), offset_job(up, t0)};
    JobSet set = make_set(js, 2, R_F32);
    set.n = 1;  // waves cover the gate rows; each also reads up
    dispatch_f32<true>(ctx, gate.dtype, set, x + t0 * gate.n_in, (uint32_t)tn, y + t0 * gate.n_out);
  });
}

// Prefill-sized int8 calls (T >= GEMM_MIN_TOKENS) on prepared Q8_0 / Q4_K /
// Q6_K weights run an MFMA GEMM with activations quantized per 32
// (quantized once for every job sharing x). Returns false when a job is not
// covered. Q4_K and Q6_K jobs take the f16-path GEMM unless the context asks
// for the int8 one, or its inputs do not fit where they must go (a
// capture's fixed-size scratch, an allocation-free call's buffer). glu_y:
// a gated call whose two jobs (gate, up) run as one gated launch writing
// silu(gate) * up there.
static bool try_gemm_f16(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t T,
                         float *glu_y = nullptr) {
  // x's f32 rows never stored (a16_noy): this call must take the record.
  const bool noy = ctx->a16_noy && a16_holds(ctx, x, T, jobs[0].n_in);
  auto decline = [&]() {
    if (noy) fail(MDMA_ERR_BACKEND, "GEMM input without its f32 rows cannot serve this call");
    return false;
  };
  if (ctx->prefill_kernel != MDMA_PREFILL_AUTO) return decline();
  for (int i = 0; i < n_jobs; i++)
    if (!gemm_f16_supported(jobs[i].dtype, jobs[i].layout, jobs[i].n_in, jobs[i].n_out) ||
        jobs[i].n_in != jobs[0].n_in || (jobs[i].dtype == DT_Q6_K && jobs[i].dots))
      return decline();  // (Q6_K block-dot capture: the int8 GEMM's per-16 dots)
  // x's input already written by a fused rmsnorm (launch_rmsnorm_a16)?
  bool pre = !ctx->fixed_scratch && a16_holds(ctx, x, T, jobs[0].n_in);
  for (int i = 0; i < n_jobs && pre; i++)
    if (jobs[i].dtype == DT_Q4_K && !ctx->a16_p) pre = false;  // the min term reads P
  if (!pre) decline();
  const uint64_t need = pre ? 0 : (gemm_f16_input_bytes(T, jobs[0].n_in) + 255) / 256 * 256;
  // Split-K partials (launches run one after another and share them).
  uint64_t nc = 0, pb = gemm_f16_split_bytes(ctx, jobs, n_jobs, T, &nc);
  char *s;
  if (ctx->fixed_scratch) {  // an allocation-free call: unsplit, inputs in its fixed buffer
    if (need > ctx->fixed_cap) return false;
    s = ctx->fixed_scratch;
    pb = 0;
  } else {
    if (ctx->capturing && need > ctx->scratch_cap) return false;
    if (ctx->capturing && need + pb > ctx->scratch_cap) pb = 0;  // under capture the scratch cannot grow
    s = scratch(ctx, need + pb);
  }
  uint32_t *cnt = pb && nc ? gemm_counters(ctx, nc) : nullptr;
  launch_gemm_f16(ctx, jobs, n_jobs, x, T, pre ? ctx->a16_buf : s, cnt ? reinterpret_cast<float *>(s + need) : nullptr,
                  cnt ? pb : 0, cnt, cnt ? nc : 0, glu_y, pre);
  return true;
}

static bool try_gemm_i8(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t T) {
  if (T < GEMM_MIN_TOKENS) return false;
  if (try_gemm_f16(ctx, jobs, n_jobs, x, T)) return true;
  for (int i = 0; i < n_jobs; i++)
    if (!gemm_i8_supported(jobs[i].dtype, jobs[i].layout, jobs[i].n_in, jobs[i].n_out) ||
        jobs[i].n_in != jobs[0].n_in)
      return false;
  const uint64_t n_in = jobs[0].n_in, n = T * n_in;
  const uint64_t qb = (n + 255) / 256 * 256, db = (n / 32 * 4 + 255) / 256 * 256,
                 sb = (n / 16 * 4 + 255) / 256 * 256;
  // Split-K partials (the jobs run one after another and share them).
  uint64_t pd = 0, nc = 0;
  for (int i = 0; i < n_jobs; i++) {
    uint64_t p, c;
    gemm_i8_split_need(ctx, jobs[i], T, &p, &c);
    pd = p > pd ? p : pd;
    nc = c > nc ? c : nc;
  }
  // Under stream capture the scratch cannot grow: past its size, unsplit.
  if (ctx->capturing && qb + db + sb + pd * 8 > ctx->scratch_cap) pd = 0;
  char *s;
  if (ctx->fixed_scratch) {  // an allocation-free call: unsplit, inputs in its fixed buffer
    pd = 0;
    if (qb + db + sb > ctx->fixed_cap) fail(MDMA_ERR_BUFFER_BUDGET, "GEMM inputs exceed the fixed scratch");
    s = ctx->fixed_scratch;
  } else {
    s = scratch(ctx, qb + db + sb + pd * 8);
  }
  int8_t *qx = reinterpret_cast<int8_t *>(s);
  float *dx = reinterpret_cast<float *>(s + qb);
  int32_t *s16 = reinterpret_cast<int32_t *>(s + qb + db);
  double *part = pd ? reinterpret_cast<double *>(s + qb + db + sb) : nullptr;
  uint32_t *cnt = pd && nc ? gemm_counters(ctx, nc) : nullptr;
  launch_quantize_act(ctx, x, n, 32, qx, dx, s16);
  for (int i = 0; i < n_jobs; i++) launch_gemm_i8(ctx, jobs[i], qx, dx, s16, T, jobs[i].y, part, pd, cnt, nc);
  return true;
}

void launch_gemv_i8(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t T) {
  if (try_gemm_i8(ctx, jobs, n_jobs, x, T)) return;
  for (int i = 0; i < n_jobs; i++)
    if (!is_i8_dtype(jobs[i].dtype) || jobs[i].n_in % 256) {
      // No int8 kernel for float weights (or rows that are not whole 256-groups):
      // those run in f32 mode.
      launch_gemv_f32(ctx, jobs, n_jobs, x, T);
      return;
    }
  if (T == 1 && !q8_holds(ctx, x, n_jobs ? jobs[0].n_in : 0)) {
    // One token: quantized in the GEMV's own prologue (one launch).
    if (launch_gemv_i8_x(ctx, jobs, n_jobs, false, x, nullptr)) return;
  }
  if (T >= BATCH_MIN_TOKENS && gemv_batch_ok(jobs, n_jobs, 16)) {
    // Up to 16 tokens per matrix-core launch (a short remainder: row teams).
    for (uint64_t t0 = 0; t0 < T; t0 += 16) {
      const uint64_t tn = T - t0 < 16 ? T - t0 : 16;
      GemvJob js[3];
      for (int i = 0; i < n_jobs; i++) js[i] = offset_job(jobs[i], t0);
      if (tn < BATCH_MIN_TOKENS)
        launch_gemv_team(ctx, MDMA_ACT_I8, js, n_jobs, false, x + t0 * jobs[0].n_in, tn, nullptr);
      else
        launch_gemv_batch(ctx, js, n_jobs, false, x + t0 * jobs[0].n_in, tn, nullptr);
    }
    return;
  }
  if (team_layout_ok(jobs, n_jobs)) {
    launch_gemv_team(ctx, MDMA_ACT_I8, jobs, n_jobs, false, x, T, nullptr);
    return;
  }
  if (!same_dtype(jobs, n_jobs) || any_prepared(jobs, n_jobs)) {
    for (int i = 0; i < n_jobs; i++) launch_gemv_i8(ctx, jobs + i, 1, x, T);
    return;
  }
  const uint64_t n_in = jobs[0].n_in;
  int8_t *qx;
  float *dx;
  int32_t *s16;
  quantize_into_scratch(ctx, x, T, n_in, &qx, &dx, &s16);
  by_chunks(T, [&](uint64_t t0, uint64_t tn) {
    GemvJob js[3];
    for (int i = 0; i < n_jobs; i++) js[i] = offset_job(jobs[i], t0);
    dispatch_i8<false>(ctx, jobs[0].dtype, make_set(js, n_jobs, R_I8), qx + t0 * n_in, dx + t0 * (n_in / 256),
                       s16 + t0 * (n_in / 16), (uint32_t)tn, nullptr);
  });
}

void launch_gemv_i8_gated(mdma_ctx *ctx, const GemvJob &gate, const GemvJob &up, const float *x, uint64_t T,
                          float *y) {
  const GemvJob gu[2] = {gate, up};
  // Q4_K gate and up on the f16-path GEMM: the SiLU product in its epilogue.
  if (T >= GEMM_MIN_TOKENS && gemm_f16_glu_ok(gate, up) && try_gemm_f16(ctx, gu, 2, x, T, y)) return;
  if (try_gemm_i8(ctx, gu, 2, x, T)) {
    launch_silu_mul(ctx, gate.y, up.y, y, T * gate.n_out);
    return;
  }
  if (T == 1 && !q8_holds(ctx, x, gate.n_in)) {
    if (launch_gemv_i8_x(ctx, gu, 2, true, x, y)) return;
  }
  if (T >= BATCH_MIN_TOKENS && gemv_batch_ok(gu, 2, 16)) {
    for (uint64_t t0 = 0; t0 < T; t0 += 16) {
      const uint64_t tn = T - t0 < 16 ? T - t0 : 16;
      const GemvJob js[2] = {offset_job(gate, t0), offset_job(up, t0)};
      const float *xt = x + t0 * gate.n_in;
      float *yt = y + t0 * gate.n_out;
      if (tn < BATCH_MIN_TOKENS)
        launch_gemv_team(ctx, MDMA_ACT_I8, js, 2, true, xt, tn, yt);
      else
        launch_gemv_batch(ctx, js, 2, true, xt, tn, yt);
    }
    return;
  }
  if (team_layout_ok(gu, 2) && gate.n_in % 256 == 0) {
    launch_gemv_team(ctx, MDMA_ACT_I8, gu, 2, true, x, T, y);
    return;
  }
  if (gate.dtype != up.dtype || !is_i8_dtype(gate.dtype) || gate.n_in % 256 || any_prepared(gu, 2)) {
    GemvJob js[2] = {gate, up};
    launch_gemv_i8(ctx, js, 1, x, T);
    launch_gemv_i8(ctx, js + 1, 1, x, T);
    launch_silu_mul(ctx, gate.y, up.y, y, T * gate.n_out);
    return;
  }
  const uint64_t n_in = gate.n_in;
  int8_t *qx;
  float *dx;
  int32_t *s16;
  quantize_into_scratch(ctx, x, T, n_in, &qx, &dx, &s16);
  by_chunks(T, [&](uint64_t t0, uint64_t tn) {
    GemvJob js[2] = {offset_job(gate, t0), offset_job(up, t0)};
    JobSet set = make_set(js, 2, R_I8);
    set.n = 1;
    dispatch_i8<true>(ctx, gate.dtype, set, qx + t0 * n_in, dx + t0 * (n_in / 256), s16 + t0 * (n_in / 16),
                      (uint32_t)tn, y + t0 * gate.n_out);
  });
}

void launch_quantize_act(mdma_ctx *ctx, const float *x, uint64_t n, uint64_t group, int8_t *q, float *d,
                         int32_t *s16) {
  const dim3 grid((uint32_t)((n + 1023) / 1024)), block(256);
  if (group == 32)
    quantize_act_kernel<32><<<grid, block, 0, ctx->stream>>>(x, n, q, d, s16);
  else
    quantize_act_kernel<256><<<grid, block, 0, ctx->stream>>>(x, n, q, d, s16);
  hip_check(hipGetLastError(), "quantize_act launch");
}

void launch_block_dot(mdma_ctx *ctx, const GemvJob &w, const int8_t *qx, uint64_t T, int32_t *out) {
  if (w.layout == MDMA_LAYOUT_GFX950) {
    launch_block_dot_prepared(ctx, w, qx, T, out);
    return;
  }
  const uint64_t sub = w.dtype == DT_Q6_K ? 16 : 32, total = T * w.n_out * (w.n_in / sub);
  if (!total) return;
  block_dot_kernel<<<dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, ctx->stream>>>(
      w.dtype, w.w, (uint32_t)w.n_out, (uint32_t)w.n_in, qx, (uint32_t)T, out);
  hip_check(hipGetLastError(), "block_dot launch");
}

}  // namespace mdma
