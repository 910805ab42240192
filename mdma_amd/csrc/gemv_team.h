// Decode GEMV on gfx950 over the prepared weight layouts (layout.cpp): the
// streaming "row team" kernels, in the int8-activation and the
// f32-activation mode, for 1..8 tokens. Instantiated per format and mode by
// gemv_team_{q4,q6,q8}_{i8,f32}.hip; host entry points in gemv_team.hip.
//
// y[t, r] = sum_i deq(W)[r, i] * x[t, i]   (reference Backend::qmatmul,
// /root/reference/src/backend.rs:469; CPU oracle src/backend/cpu.rs:335-368)
//
// Layout of the work:
//  - A lane owns fixed "units" of K (64 columns; 32 for Q8_0). The prepared
//    layout stores each row as planes indexed by unit, so lane i of every
//    16-byte load instruction reads bytes [16i, 16i+16) of a plane: a wave
//    load is 1 KiB of contiguous HBM.
//  - The lane's activations for its units stay in registers for the whole
//    kernel (int8 values, their exact sub-block sums and the per-256 scale;
//    or, in the f32 mode of one token, the f32 values and their f64 sums).
//  - A team of TW waves (64*TW lanes) covers all units of a row, PL units
//    per lane. A team owns a contiguous run of rows of one weight and walks
//    it R rows at a time, loading the next R rows while it computes the
//    current ones (NBUF rotating register buffers).
//  - Lanes reduce with DPP moves; multi-wave teams add the waves' sums in LDS.
//  - Fused QKV: up to three weights share x; teams are dealt out in order.
//    Gated (ffn gate/up + SiLU): a team computes R rows of gate and the same
//    rows of up and writes silu(g) * u.
// Arithmetic per mode:
//  - int8: exact int32 dot per sub-block with v_dot4_i32_i8, scales applied
//    as in the reference's int8 decode (src/backend/rocm/kernels/decode.hip:47-108):
//    Q4_K d_x*(d*sum sc*isum - dmin*sum m*xsum), Q6_K d_x*d*sum sc*isum,
//    Q8_0 d_x*d*isum; f32 partial sums.
//  - f32: exact products (byte_f64) accumulated in f64, one f32 rounding at
//    the end.
#pragma once

#include <hip/hip_ext.h>

#include <type_traits>

#include "kernels.h"

namespace mdma {
namespace {

constexpr int WG = 256;  // threads per workgroup

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ uint32_t ld16b(const uint8_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
}
// The value of another lane of the quad (DPP quad_perm).
template <int PERM>
__device__ __forceinline__ uint32_t quad_perm_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, PERM, 0xF, 0xF, false);
}
// Dword k of the quad (lanes 4j..4j+3 hold the four dwords of one header).
template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K * 0x55, 0xF, 0xF, false);
}
__device__ __forceinline__ void f4(const float *p, float *o) {
  const float4 v = *reinterpret_cast<const float4 *>(p);
  o[0] = v.x, o[1] = v.y, o[2] = v.z, o[3] = v.w;
}
__device__ __forceinline__ double sum_f64(const float *v, int n) {
  double s = 0.0;
  for (int i = 0; i < n; i++) s += (double)v[i];
  return s;
}
// acc += sum_k (2 + byte_k(w)/2048) * x[k] with f32 x converted on use.
__device__ __forceinline__ double fma4f(uint32_t w, const float *x, double acc) {
  acc = fma(byte_f64<0>(w), (double)x[0], acc);
  acc = fma(byte_f64<1>(w), (double)x[1], acc);
  acc = fma(byte_f64<2>(w), (double)x[2], acc);
  acc = fma(byte_f64<3>(w), (double)x[3], acc);
  return acc;
}

// ---------------------------------------------------------------- Q4_K ----
// Unit u = sub-block pair p = u%4 of block u/4: 32 quant bytes (A, B planes)
// whose low nibbles are columns 64u..64u+31 and high nibbles 64u+32..+63;
// the 16-byte block header is spread over the quad (dword u%4 per lane).
struct Q4G {
  static constexpr uint32_t UCOLS = 64;
  struct W {
    uint4 a, b;
    uint32_t h;
  };
  struct XI {
    uint4 a0, a1, b0, b1;
    int sa, sb;
    float d8;
  };
  struct XF {
    float xa[32], xb[32];
    double sa, sb;
  };
  __device__ static uint32_t units(uint32_t n_in) { return n_in / 64; }
  __device__ static size_t row_bytes(uint32_t n_in) { return (size_t)(n_in / 256) * 144; }
  __device__ static W load(const uint8_t *row, uint32_t u, uint32_t U) {
    return W{ld16(row + 16 * (size_t)u), ld16(row + 16 * (size_t)(U + u)), ld32(row + 32 * (size_t)U + 4 * u)};
  }
  __device__ static uint4 header(uint32_t h) {
    return make_uint4(quad_bcast<0>(h), quad_bcast<1>(h), quad_bcast<2>(h), quad_bcast<3>(h));
  }
  // First column of chunk c (16 columns) of unit u, and the activations of
  // a unit from its four chunks (int8 bytes, their sums) and its scale.
  __device__ static uint32_t chunk_col(uint32_t u, int c) { return 64 * u + 16 * c; }
  __device__ static XI make_xi(const uint4 *q, const int *s, float d8) {
    return XI{q[0], q[1], q[2], q[3], s[0] + s[1], s[2] + s[3], d8};
  }
  __device__ static XI loadxi(const int8_t *qx, const float *dx, const int32_t *s16, uint32_t u) {
    const int8_t *xt = qx + 64 * (size_t)u;
    const int4 s = *reinterpret_cast<const int4 *>(s16 + 4 * (size_t)u);
    return XI{ldx16(xt), ldx16(xt + 16), ldx16(xt + 32), ldx16(xt + 48), s.x + s.y, s.z + s.w, dx[u >> 2]};
  }
  __device__ static XF loadxf(const float *x, uint32_t u) {
    XF r;
#pragma unroll
    for (int k = 0; k < 32; k += 4) {
      f4(x + 64 * (size_t)u + k, r.xa + k);
      f4(x + 64 * (size_t)u + 32 + k, r.xb + k);
    }
    r.sa = sum_f64(r.xa, 32);
    r.sb = sum_f64(r.xb, 32);
    return r;
  }
  // dots: the unit's int32 sub-block dots (sum q * x of sub-blocks 2(u%4)
  // and 2(u%4)+1), for the block-dot capture.
  __device__ static float dot_i8(const W &w, const XI &x, uint32_t u, int (&dots)[4]) {
    const uint4 hd = header(w.h);
    const uint32_t q[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
    const uint32_t xa[8] = {x.a0.x, x.a0.y, x.a0.z, x.a0.w, x.a1.x, x.a1.y, x.a1.z, x.a1.w};
    const uint32_t xb[8] = {x.b0.x, x.b0.y, x.b0.z, x.b0.w, x.b1.x, x.b1.y, x.b1.z, x.b1.w};
    int ia = 0, ib = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      ia = __builtin_amdgcn_sdot4((int)(q[k] & 0x0F0F0F0Fu), (int)xa[k], ia, false);
      ib = __builtin_amdgcn_sdot4((int)((q[k] >> 4) & 0x0F0F0F0Fu), (int)xb[k], ib, false);
    }
    dots[0] = ia, dots[1] = ib;
    int sca, scb, ma, mb;
    q4k_scales_i(hd, u & 3, sca, scb, ma, mb);
    // 24-bit multiplies (full rate): |isum| <= 15*127*32, |xsum| <= 127*32.
    const int A = __mul24(sca, ia) + __mul24(scb, ib);
    const int B = __mul24(ma, x.sa) + __mul24(mb, x.sb);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    return x.d8 * fmaf(d, (float)A, -dmin * (float)B);
  }
  __device__ static uint32_t n_sub(uint32_t n_in) { return n_in / 32; }
  __device__ static void put_dots(int32_t *o, const int (&dots)[4], uint32_t u) {
    o[2 * u] = dots[0];
    o[2 * u + 1] = dots[1];
  }
  __device__ static double dot_f32(const W &w, const XF &x, uint32_t u) {
    const uint4 hd = header(w.h);
    const uint32_t q[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
    double aa = 0.0, ab = 0.0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      aa = fma4f(q[k] & 0x0F0F0F0Fu, x.xa + 4 * k, aa);
      ab = fma4f((q[k] >> 4) & 0x0F0F0F0Fu, x.xb + 4 * k, ab);
    }
    int sca, scb, ma, mb;
    q4k_scales_i(hd, u & 3, sca, scb, ma, mb);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    const double dsa = (double)(d * (float)sca), dsb = (double)(d * (float)scb);
    const double dma = (double)(dmin * (float)ma), dmb = (double)(dmin * (float)mb);
    // sum (d*sc*q - dmin*m) * x with sum q*x = 2048*acc - 4096*X.
    double r = fma(2048.0 * dsa, aa, -fma(4096.0, dsa, dma) * x.sa);
    r += fma(2048.0 * dsb, ab, -fma(4096.0, dsb, dmb) * x.sb);
    return r;
  }
};

// ---------------------------------------------------------------- Q6_K ----
// Unit u = (half n, column group h) of block u/4 (u%4 = 2n+h): columns
// 128n + 32r + 16h + [0,16) of quarters r = 0..3 (16 six-bit quants each,
// q = u6 - 32), with sub-scales sc[8n + 2r + h] and the block's f16 d.
struct Q6G {
  static constexpr uint32_t UCOLS = 64;
  struct W {
    uint4 a, b, q;
    uint32_t sc, d;
  };
  struct XI {
    uint4 xq[4];
    int sq[4];
    float d8;
  };
  struct XF {
    float x[4][16];
    double s[4];
  };
  __device__ static uint32_t units(uint32_t n_in) { return n_in / 64; }
  __device__ static size_t row_bytes(uint32_t n_in) { return ((size_t)(n_in / 256) * 210 + 15) / 16 * 16; }
  __device__ static W load(const uint8_t *row, uint32_t u, uint32_t U) {
    return W{ld16(row + 16 * (size_t)u), ld16(row + 16 * (size_t)(U + u)), ld16(row + 16 * (size_t)(2 * U + u)),
             ld32(row + 48 * (size_t)U + 4 * u), ld16b(row + 52 * (size_t)U + 2 * (u >> 2))};
  }
  // First column of quarter r of unit u.
  __device__ static uint32_t col(uint32_t u, int r) {
    return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * r + 16 * (u & 1);
  }
  __device__ static uint32_t chunk_col(uint32_t u, int c) { return col(u, c); }
  __device__ static XI make_xi(const uint4 *q, const int *s, float d8) {
    return XI{{q[0], q[1], q[2], q[3]}, {s[0], s[1], s[2], s[3]}, d8};
  }
  __device__ static XI loadxi(const int8_t *qx, const float *dx, const int32_t *s16, uint32_t u) {
    XI r;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      r.xq[q] = ldx16(qx + col(u, q));
      r.sq[q] = s16[col(u, q) / 16];
    }
    r.d8 = dx[u >> 2];
    return r;
  }
  __device__ static XF loadxf(const float *x, uint32_t u) {
    XF r;
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
      for (int k = 0; k < 16; k += 4) f4(x + col(u, q) + k, r.x[q] + k);
      r.s[q] = sum_f64(r.x[q], 16);
    }
    return r;
  }
  // Six-bit quants of quarter r, dword k (4 columns).
  __device__ static uint32_t u6(const W &w, int r, int k) {
    const uint32_t qa = k == 0 ? w.a.x : k == 1 ? w.a.y : k == 2 ? w.a.z : w.a.w;
    const uint32_t qb = k == 0 ? w.b.x : k == 1 ? w.b.y : k == 2 ? w.b.z : w.b.w;
    const uint32_t h = k == 0 ? w.q.x : k == 1 ? w.q.y : k == 2 ? w.q.z : w.q.w;
    switch (r) {
      case 0: return (qa & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
      case 1: return (qb & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
      case 2: return ((qa >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
      default: return ((qb >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    }
  }
  // dots: the unit's four 16-column dots sum (q - 32) * x (quarters r).
  __device__ static float dot_i8(const W &w, const XI &x, uint32_t, int (&dots)[4]) {
    int A = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t xv[4] = {x.xq[r].x, x.xq[r].y, x.xq[r].z, x.xq[r].w};
      int s = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) s = __builtin_amdgcn_sdot4((int)u6(w, r, k), (int)xv[k], s, false);
      // 24-bit multiply (full rate): |s - 32*xsum| <= 63*127*16 + 32*127*16.
      dots[r] = s - 32 * x.sq[r];
      A += __mul24((int)(int8_t)((w.sc >> (8 * r)) & 0xff), dots[r]);
    }
    return x.d8 * (h2f(w.d) * (float)A);
  }
  __device__ static uint32_t n_sub(uint32_t n_in) { return n_in / 16; }
  __device__ static void put_dots(int32_t *o, const int (&dots)[4], uint32_t u) {
#pragma unroll
    for (int r = 0; r < 4; r++) o[col(u, r) / 16] = dots[r];
  }
  __device__ static double dot_f32(const W &w, const XF &x, uint32_t) {
    double r = 0.0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      double a = 0.0;
#pragma unroll
      for (int k = 0; k < 4; k++) a = fma4f(u6(w, q, k), x.x[q] + 4 * k, a);
      const double s = (double)(int8_t)((w.sc >> (8 * q)) & 0xff);
      r = fma(s, fma(2048.0, a, -4128.0 * x.s[q]), r);
    }
    return (double)h2f(w.d) * r;
  }
};

// ---------------------------------------------------------------- Q8_0 ----
// Unit u = block u: 32 int8 quants (A, B planes) and the f16 d.
struct Q8G {
  static constexpr uint32_t UCOLS = 32;
  struct W {
    uint4 a, b;
    uint32_t d;
  };
  struct XI {
    uint4 x0, x1;
    float d8;
  };
  struct XF {
    float x[32];
    double s;
  };
  __device__ static uint32_t units(uint32_t n_in) { return n_in / 32; }
  __device__ static size_t row_bytes(uint32_t n_in) { return ((size_t)(n_in / 32) * 34 + 15) / 16 * 16; }
  __device__ static W load(const uint8_t *row, uint32_t u, uint32_t U) {
    return W{ld16(row + 16 * (size_t)u), ld16(row + 16 * (size_t)(U + u)), ld16b(row + 32 * (size_t)U + 2 * u)};
  }
  __device__ static XI loadxi(const int8_t *qx, const float *dx, const int32_t *, uint32_t u) {
    return XI{ldx16(qx + 32 * (size_t)u), ldx16(qx + 32 * (size_t)u + 16), dx[u >> 3]};
  }
  __device__ static XF loadxf(const float *x, uint32_t u) {
    XF r;
#pragma unroll
    for (int k = 0; k < 32; k += 4) f4(x + 32 * (size_t)u + k, r.x + k);
    r.s = sum_f64(r.x, 32);
    return r;
  }
  __device__ static float dot_i8(const W &w, const XI &x, uint32_t, int (&dots)[4]) {
    int s = __builtin_amdgcn_sdot4((int)w.a.x, (int)x.x0.x, 0, false);
    s = __builtin_amdgcn_sdot4((int)w.a.y, (int)x.x0.y, s, false);
    s = __builtin_amdgcn_sdot4((int)w.a.z, (int)x.x0.z, s, false);
    s = __builtin_amdgcn_sdot4((int)w.a.w, (int)x.x0.w, s, false);
    s = __builtin_amdgcn_sdot4((int)w.b.x, (int)x.x1.x, s, false);
    s = __builtin_amdgcn_sdot4((int)w.b.y, (int)x.x1.y, s, false);
    s = __builtin_amdgcn_sdot4((int)w.b.z, (int)x.x1.z, s, false);
    s = __builtin_amdgcn_sdot4((int)w.b.w, (int)x.x1.w, s, false);
    dots[0] = s;
    return x.d8 * (h2f(w.d) * (float)s);
  }
  __device__ static uint32_t n_sub(uint32_t n_in) { return n_in / 32; }
  __device__ static void put_dots(int32_t *o, const int (&dots)[4], uint32_t u) { o[u] = dots[0]; }
  __device__ static double dot_f32(const W &w, const XF &x, uint32_t) {
    const uint32_t q[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
    double a = 0.0;
#pragma unroll
    for (int k = 0; k < 8; k++) a = fma4f(q[k] ^ 0x80808080u, x.x + 4 * k, a);
    // bytes biased by 128: sum q*x = 2048*acc - (4096 + 128)*X.
    return (double)h2f(w.d) * fma(2048.0, a, -4224.0 * x.s);
  }
};

// ----------------------------------------------------------- prologue ----
// The int8 activations of unit u quantized from f32 x inside the GEMV, per
// 256 columns (the four units of a quad): the arithmetic of
// quantize_act_kernel, bit for bit. Split into the loads of x and the
// quantization, so the first weight loads can be issued between them.
template <class F>
__device__ void prologue_load(const float *__restrict__ x, uint32_t u, bool ok, float (&v)[4][16]) {
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t col = F::chunk_col(u, c);
#pragma unroll
    for (int k = 0; k < 16; k += 4) {
      const float4 xv = ok ? *reinterpret_cast<const float4 *>(x + col + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      v[c][k] = xv.x, v[c][k + 1] = xv.y, v[c][k + 2] = xv.z, v[c][k + 3] = xv.w;
    }
  }
}
template <class F>
__device__ typename F::XI prologue_quant(const float (&v)[4][16]) {
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < 4; c++)
#pragma unroll
    for (int k = 0; k < 16; k++) amax = fmaxf(amax, fabsf(v[c][k]));
  amax = fmaxf(amax, __builtin_bit_cast(float, quad_perm_u32<0xB1>(__builtin_bit_cast(uint32_t, amax))));
  amax = fmaxf(amax, __builtin_bit_cast(float, quad_perm_u32<0x4E>(__builtin_bit_cast(uint32_t, amax))));
  const float inv = amax == 0.f ? 0.f : 127.0f / amax;
  uint4 q[4];
  int sums[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint32_t w4[4];
    int sm = 0;
#pragma unroll
    for (int k = 0; k < 16; k += 4) {
      const int q0 = q8_quant(v[c][k], inv), q1 = q8_quant(v[c][k + 1], inv);
      const int q2 = q8_quant(v[c][k + 2], inv), q3 = q8_quant(v[c][k + 3], inv);
      sm += (q0 + q1) + (q2 + q3);
      w4[k >> 2] = pack4_i8(q0, q1, q2, q3);
    }
    q[c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    sums[c] = sm;
  }
  return F::make_xi(q, sums, amax / 127.0f);
}

// The same int8 activations, quantized once per workgroup: with one-wave
// teams every wave of a workgroup needs all of x, so its 256 threads
// quantize the (at most 64) units together into LDS, four threads per unit
// (16 columns each, a 256-column group on 16 lanes of one wave), and every
// lane then reads its own unit u back. The same arithmetic, bit for bit.
template <class F>
__device__ void prologue_wg_load(const float *__restrict__ x, uint32_t U, float (&v)[16]) {
  const uint32_t t = threadIdx.x, qu = t >> 2, c = t & 3;
  const bool live = qu < U;
  const uint32_t col = F::chunk_col(live ? qu : 0, c);
#pragma unroll
  for (int k = 0; k < 16; k += 4) {
    const float4 xv = live ? *reinterpret_cast<const float4 *>(x + col + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    v[k] = xv.x, v[k + 1] = xv.y, v[k + 2] = xv.z, v[k + 3] = xv.w;
  }
}
// Called by all threads of the workgroup (it has a barrier).
template <class F>
__device__ typename F::XI prologue_wg_quant(const float (&v)[16], uint32_t U, uint32_t u, uint4 (*lq)[4],
                                            int (*ls)[4], float *ld) {
  const uint32_t t = threadIdx.x, qu = t >> 2, c = t & 3;
  const bool live = qu < U;
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < 16; k++) amax = fmaxf(amax, fabsf(v[k]));
  // Max over the quad (one unit), then over the 16-lane row (four units).
  amax = fmaxf(amax, __builtin_bit_cast(float, quad_perm_u32<0xB1>(__builtin_bit_cast(uint32_t, amax))));
  amax = fmaxf(amax, __builtin_bit_cast(float, quad_perm_u32<0x4E>(__builtin_bit_cast(uint32_t, amax))));
  amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, amax), 0x124, 0xF,
                                                                          0xF, false)));  // row_ror:4
  amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, amax), 0x128, 0xF,
                                                                          0xF, false)));  // row_ror:8
  const float inv = amax == 0.f ? 0.f : 127.0f / amax;
  uint32_t w4[4];
  int sm = 0;
#pragma unroll
  for (int k = 0; k < 16; k += 4) {
    const int q0 = q8_quant(v[k], inv), q1 = q8_quant(v[k + 1], inv);
    const int q2 = q8_quant(v[k + 2], inv), q3 = q8_quant(v[k + 3], inv);
    sm += (q0 + q1) + (q2 + q3);
    w4[k >> 2] = pack4_i8(q0, q1, q2, q3);
  }
  if (live) {
    lq[qu][c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    ls[qu][c] = sm;
    if ((t & 15) == 0) ld[qu >> 2] = amax / 127.0f;
  }
  lds_barrier();  // LDS only: the weight loads already issued stay in flight
  const uint4 q[4] = {lq[u][0], lq[u][1], lq[u][2], lq[u][3]};
  const int sums[4] = {ls[u][0], ls[u][1], ls[u][2], ls[u][3]};
  return F::make_xi(q, sums, ld[u >> 2]);
}

// ------------------------------------------------------------- kernel ----

struct TeamJob {
  const uint8_t *w;
  float *y;
  uint32_t n_out, teams;
  int32_t *dots;  // block-dot capture (GemvJob::dots) or null
};
struct TeamSet {
  TeamJob j[3];
  int n;
  uint32_t n_in, rpt;  // shared row length; rows per team (a multiple of R)
  bool pro;            // one token, int8: x (f32) quantized in the prologue
  // One token, the residual stream of a Llama layer: with res set, a plain
  // launch stores y = res + W x and each workgroup the sum of squares of its
  // rows of y (f32 squares added in f64) in ssq[workgroup].
  const float *res;
  double *ssq;
  uint32_t ssq_cap;  // entries of ssq; a grid past it is not launched
  // One token, PRO 5: x = rmsnorm(nsum) * nw, the sum of squares of nsum
  // being the n_part partials npart that its producer stored.
  const float *nsum, *nw;
  const double *npart;
  uint32_t n_part;
  float eps;
};

// Row groups in flight per wave (loads issued NBUF-1 groups ahead): three
// for one-wave teams in the int8 mode, whose short compute leaves the loads
// exposed; two elsewhere, where a third costs occupancy or registers.
template <bool F32, int TW>
constexpr int nbuf() {
#ifdef MDMA_TEAM_NBUF
  return MDMA_TEAM_NBUF;
#else
  return !F32 && TW == 1 ? 3 : 2;
#endif
}

// PRO: how a one-token int8 launch gets its activations (each a separate
// instantiation: the prologue's registers would otherwise lower every
// launch's occupancy). 0 = every lane loads its units of the quantized-x
// buffers. The kernel quantizes f32 x itself: 1 = each wave its own units
// (multi-wave teams, whose waves hold different units), 2 = once per
// workgroup in LDS (one-wave teams, whose waves all hold every unit).
// 3 = the quantized-x buffers staged once per workgroup in LDS (one-wave
// teams of the fused gate/up and of Q4_K). 5 = x computed as the rmsnorm of
// the residual stream (TeamSet::nsum) and quantized once per workgroup in
// LDS (one-wave teams; the norm fused into the GEMV that reads it).
// 4 = f32 x quantized once per workgroup of
// MDMA_PRO4_TEAMS multi-wave teams into LDS (rows of up to 16384 columns):
// each team needs all of x, so sharing it divides the f32 reads of x and the
// quantization work by the teams per workgroup.
// Teams of a multi-wave workgroup quantizing x once for all of them (PRO 4).
#ifndef MDMA_PRO4_TEAMS
#define MDMA_PRO4_TEAMS 2
#endif
// Threads of a workgroup staging quantized x (PRO 3): its waves share one
// staged copy.
#ifndef MDMA_PRO3_WG
#define MDMA_PRO3_WG 256
#endif
constexpr int team_wg(int pro, int tw) {
  return pro == 4 ? 64 * tw * MDMA_PRO4_TEAMS : (pro == 3 ? MDMA_PRO3_WG : WG);
}

// CAP: the block-dot capture instantiation (TeamJob::dots set), which also
// stores each int32 sub-block dot; the production instantiations have none
// of its code.
template <class F, bool F32, int R, int ITERS, int TW, int PL, int TT, bool GATED, int PRO = 0, bool CAP = false>
__global__ __launch_bounds__(team_wg(PRO, TW)) void gemv_team(TeamSet ts, const float *__restrict__ xf,
                                                const int8_t *__restrict__ qx, const float *__restrict__ dx,
                                                const int32_t *__restrict__ s16, uint32_t T,
                                                float *__restrict__ ygated) {
  // A lane's partial (at most PL unit terms) is f32 in the int8 mode and f64
  // in the f32 mode; lane and wave partials are added in f64, so outputs
  // that cancel (|y| << sum |w*x|) keep their relative accuracy.
  using Acc = typename std::conditional<F32, double, float>::type;
  constexpr int TPW = team_wg(PRO, TW) / 64 / TW;  // teams per workgroup
  constexpr int NR = GATED ? 2 * R : R;
  constexpr int NBUF = nbuf<F32, TW>();
  // Multi-wave teams: each wave's per-row totals for the whole run, added
  // across the team's waves once, after the run (one barrier per kernel).
  __shared__ double red[TW > 1 ? TPW : 1][TW > 1 ? TW : 1][TW > 1 ? ITERS * NR * TT : 1];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int tw = wave % TW, slot = wave / TW;
  // Team -> job, branch-free: every field is read up front, so the
  // kernel-argument loads form one batch before the first weight load, and
  // every job field stays in SGPRs.
  // Every kernel argument this variant reads, pinned in SGPRs before any
  // other work: the scalar loads of the argument segment then go out
  // together and are waited for once, instead of in a chain of round trips
  // as each value's first use (some inside branches) comes up.
  sgpr_ready(ts.n, ts.n_in, ts.rpt, ts.j[0].w, ts.j[0].y, ts.j[0].n_out, ts.j[0].teams, ts.j[1].w, ts.j[1].y,
             ts.j[1].n_out, ts.j[1].teams, ts.j[2].w, ts.j[2].y, ts.j[2].n_out, ts.j[2].teams);
  if constexpr (PRO == 1 || PRO == 2 || PRO == 4) sgpr_ready(xf);
  else if constexpr (PRO == 5) sgpr_ready(ts.nsum, ts.nw, ts.npart, ts.n_part, ts.eps);
  else if constexpr (!F32) sgpr_ready(qx, dx, s16);
  else sgpr_ready(xf);
  if constexpr (GATED) sgpr_ready(ygated);
  else if constexpr (!F32 && TT == 1) sgpr_ready(ts.res, ts.ssq);
  uint32_t team = blockIdx.x * TPW + slot;
  const uint32_t t0 = ts.j[0].teams, t1 = ts.j[1].teams;
  const bool in1 = ts.n > 1 && team >= t0, in2 = ts.n > 2 && team >= t0 + t1;
  team -= in2 ? t0 + t1 : (in1 ? t0 : 0u);
  TeamJob J;
  J.w = in2 ? ts.j[2].w : (in1 ? ts.j[1].w : ts.j[0].w);
  J.y = in2 ? ts.j[2].y : (in1 ? ts.j[1].y : ts.j[0].y);
  J.n_out = in2 ? ts.j[2].n_out : (in1 ? ts.j[1].n_out : ts.j[0].n_out);
  J.teams = in2 ? ts.j[2].teams : (in1 ? t1 : t0);
  J.dots = in2 ? ts.j[2].dots : (in1 ? ts.j[1].dots : ts.j[0].dots);
  // A team past its job's end (the grid's last workgroup) runs the loop for
  // the barriers of its workgroup but stores nothing.
  const bool team_live = team < J.teams;
  const uint32_t n_in = ts.n_in, U = F::units(n_in), n_out = J.n_out;
  const size_t rb = F::row_bytes(n_in);
  const uint8_t *w_main = J.w, *w_up = GATED ? ts.j[1].w : J.w;
  const uint32_t r_begin = min(team, J.teams - 1) * ts.rpt;
  const uint32_t r_last = min(r_begin + ts.rpt, n_out) - 1;

  uint32_t uid[PL];
  bool uok[PL];
#pragma unroll
  for (int p = 0; p < PL; p++) {
    const uint32_t u = (uint32_t)(p * TW + tw) * 64 + lane;
    uok[p] = u < U;
    uid[p] = uok[p] ? u : U - 1;
  }
  typename F::XI xi[F32 ? 1 : PL][F32 ? 1 : TT];
  typename F::XF xr[F32 && TT == 1 ? PL : 1];
  // Rows past the weight's end (last team of a job) re-read its last row;
  // their sums are not stored.
  typename F::W buf[NBUF][PL][NR];  // rotating row-group buffers
  auto load = [&](typename F::W(&w)[PL][NR], uint32_t r0) {
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const uint32_t row = min(r0 + (r % R), r_last);
      const uint8_t *rp = (r < R ? w_main : w_up) + row * rb;
#pragma unroll
      for (int p = 0; p < PL; p++) w[p][r] = F::load(rp, uid[p], U);
    }
  };
  double ssq_lane = 0.0;  // residual mode: this lane's stored rows' squares
  // Multi-wave teams, one token, residual mode: the residual value of the row
  // this lane of wave 0 stores at the end (row r_begin + lane), loaded now so
  // its latency is not at the kernel's tail. Unconditional and clamped (a load
  // under a branch waits for every load in flight); without res the output
  // itself is read and the value unused.
  float res_pre = 0.f;
  if constexpr (TW > 1 && !GATED && TT == 1 && !F32) {
    const float *rp = ts.res ? ts.res : J.y;
    res_pre = rp[min(r_begin + (uint32_t)lane, r_last)];
  }
  auto consume = [&](const typename F::W(&w)[PL][NR], int it) {
    const uint32_t r0 = r_begin + it * R;
    Acc s[NR][TT];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
      for (int t = 0; t < TT; t++) s[r][t] = 0;
#pragma unroll
    for (int p = 0; p < PL; p++) {
      if constexpr (!F32) {
#pragma unroll
        for (int t = 0; t < TT; t++) {
          if (t >= (int)T) break;
#pragma unroll
          for (int r = 0; r < NR; r++) {
            int dots[4];
            const float v = F::dot_i8(w[p][r], xi[p][t], uid[p], dots);
            s[r][t] += uok[p] ? v : 0.f;
            if constexpr (CAP) {
              int32_t *dcap = r < R ? J.dots : ts.j[1].dots;  // the gated kernel's up rows: job 1
              if (team_live && uok[p]) {
                const uint32_t row = min(r0 + (r % R), r_last);
                F::put_dots(dcap + ((size_t)t * n_out + row) * F::n_sub(n_in), dots, uid[p]);
              }
            }
          }
        }
      } else if constexpr (TT == 1) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
          const double v = F::dot_f32(w[p][r], xr[p], uid[p]);
          s[r][0] += uok[p] ? v : 0.0;
        }
      } else {
#pragma unroll
        for (int t = 0; t < TT; t++) {
          if (t >= (int)T) break;
          const typename F::XF xt = F::loadxf(xf + (size_t)t * n_in, uid[p]);
#pragma unroll
          for (int r = 0; r < NR; r++) {
            const double v = F::dot_f32(w[p][r], xt, uid[p]);
            s[r][t] += uok[p] ? v : 0.0;
          }
        }
      }
    }
    double tot[NR][TT];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
      for (int t = 0; t < TT; t++) tot[r][t] = (t < (int)T) ? wave_total63((double)s[r][t]) : 0.0;
    if constexpr (TW > 1) {
      if (lane == 63)
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
          for (int t = 0; t < TT; t++) red[slot][tw][(it * NR + r) * TT + t] = tot[r][t];
    } else if (team_live && lane == 63) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t row = r0 + r;
        if (row > r_last) break;
#pragma unroll
        for (int t = 0; t < TT; t++) {
          if (t >= (int)T) break;
          if (GATED) {
            const float g = (float)tot[r][t], up = (float)tot[R + r][t];
            ygated[(size_t)t * n_out + row] = g / (1.0f + expf(-g)) * up;
          } else {
            float yv = (float)tot[r][t];
            if (ts.res) {  // uniform; one token
              yv = ts.res[row] + yv;
              ssq_lane += (double)(yv * yv);
            }
            J.y[(size_t)t * n_out + row] = yv;
          }
        }
      }
    }
  };

  auto first_loads = [&]() {
#pragma unroll
    for (int it = 0; it < NBUF - 1 && it < ITERS; it++) load(buf[it], r_begin + it * R);
  };
  // Activations of the lane's units, loaded once. With an int8 x already
  // in memory the first rows' weights go out before it (the weights come
  // from HBM, x from L2); x that the kernel quantizes or stages through LDS
  // goes out first, so the waits for it let the weight loads stay in flight
  // (loads complete in order).
  if constexpr (PRO == 2) {
    static_assert(TW == 1 && PL == 1 && TT == 1, "workgroup prologue: one-wave teams, one unit per lane");
    __shared__ uint4 pq[64][4];
    __shared__ int ps[64][4];
    __shared__ float pd[16];
    float v[16];
    prologue_wg_load<F>(xf, U, v);
    first_loads();
    xi[0][0] = prologue_wg_quant<F>(v, U, uid[0], pq, ps, pd);
  } else if constexpr (PRO == 5) {
    // x = rmsnorm(nsum) * nw (the arithmetic of rmsnorm_row_kernel: f32
    // squares added in f64, mean in f32, scale 1/sqrtf(mean + eps), x =
    // (v * scale) * w), then quantized once per workgroup into LDS as PRO 2
    // does. The sum of squares comes from the producer's per-workgroup f64
    // partials: another order of the f64 additions moves the total by a
    // few f64 ulps, far below the f32 rounding of the mean.
    static_assert(TW == 1 && PL == 1 && TT == 1, "normalizing prologue: one-wave teams, one unit per lane");
    __shared__ uint4 pq[64][4];
    __shared__ int ps[64][4];
    __shared__ float pd[16];
    __shared__ double ptot[WG / 64];
    float v[16], wn[16];
    prologue_wg_load<F>(ts.nsum, U, v);
    prologue_wg_load<F>(ts.nw, U, wn);
    double pt = threadIdx.x < ts.n_part ? ts.npart[threadIdx.x] : 0.0;  // n_part <= WG
    first_loads();
    pt = wave_total63(pt);
    if (lane == 63) ptot[wave] = pt;
    lds_barrier();
    double tot = 0.0;
#pragma unroll
    for (int k = 0; k < WG / 64; k++) tot += ptot[k];
    const float mean_sq = (float)tot / (float)n_in;
    const float scale = 1.0f / sqrtf(mean_sq + ts.eps);
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int k = 0; k < 16; k++) v[k] = (v[k] * scale) * wn[k];
    }
    xi[0][0] = prologue_wg_quant<F>(v, U, uid[0], pq, ps, pd);
  } else if constexpr (PRO == 3) {
    // int8 x staged once per workgroup in LDS (one-wave teams: every wave
    // of the workgroup reads all of it): one load per thread instead of
    // six per lane.
    static_assert(TW == 1 && PL == 1 && TT == 1, "workgroup x staging: one-wave teams, one unit per lane");
    __shared__ uint4 sq[WG];
    __shared__ int32_t ss[WG];
    __shared__ float sd[WG / 16];
    const uint32_t t = threadIdx.x;
    const bool lq = t < n_in / 16, ld = t < n_in / 256;  // n_in <= 64 * 64 (one-wave teams)
    const uint4 vq = lq ? ldx16(qx + 16 * (size_t)t) : make_uint4(0, 0, 0, 0);
    const int32_t vs = lq ? s16[t] : 0;
    const float vd = ld ? dx[t] : 0.f;
    first_loads();
    if (lq) sq[t] = vq, ss[t] = vs;
    if (ld) sd[t] = vd;
    lds_barrier();
    xi[0][0] = F::loadxi(reinterpret_cast<const int8_t *>(sq), sd, ss, uid[0]);
  } else if constexpr (PRO == 4) {
    static_assert(TW > 1 && PL == 1 && TT == 1, "workgroup-shared quantization: multi-wave teams, one unit per lane");
    constexpr int NT = team_wg(4, TW);
    constexpr int NP = (16384 / 16 + NT - 1) / NT;  // passes of 16-column chunks
    __shared__ uint4 xq4[16384 / 16];
    __shared__ int32_t xs4[16384 / 16];
    __shared__ float xd4[16384 / 256];
    // Chunk c = 16 columns; the 16 chunks of a 256-group sit on one DPP row
    // of 16 lanes (NT is a multiple of 64).
    const uint32_t nch = n_in / 16;
    float v[NP][16];
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const uint32_t c = threadIdx.x + NT * p;
#pragma unroll
      for (int k = 0; k < 16; k += 4) {
        const float4 xv = c < nch ? *reinterpret_cast<const float4 *>(xf + 16 * c + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        v[p][k] = xv.x, v[p][k + 1] = xv.y, v[p][k + 2] = xv.z, v[p][k + 3] = xv.w;
      }
    }
    first_loads();
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const uint32_t c = threadIdx.x + NT * p;
      float amax = 0.f;
#pragma unroll
      for (int k = 0; k < 16; k++) amax = fmaxf(amax, fabsf(v[p][k]));
      amax = fmaxf(amax, __builtin_bit_cast(float, quad_perm_u32<0xB1>(__builtin_bit_cast(uint32_t, amax))));
      amax = fmaxf(amax, __builtin_bit_cast(float, quad_perm_u32<0x4E>(__builtin_bit_cast(uint32_t, amax))));
      amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, amax), 0x124, 0xF,
                                                                              0xF, false)));  // row_ror:4
      amax = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, amax), 0x128, 0xF,
                                                                              0xF, false)));  // row_ror:8
      const float inv = amax == 0.f ? 0.f : 127.0f / amax;
      uint32_t w4[4];
      int sm = 0;
#pragma unroll
      for (int k = 0; k < 16; k += 4) {
        const int q0 = q8_quant(v[p][k], inv), q1 = q8_quant(v[p][k + 1], inv);
        const int q2 = q8_quant(v[p][k + 2], inv), q3 = q8_quant(v[p][k + 3], inv);
        sm += (q0 + q1) + (q2 + q3);
        w4[k >> 2] = pack4_i8(q0, q1, q2, q3);
      }
      if (c < nch) {
        xq4[c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        xs4[c] = sm;
        if ((c & 15) == 0) xd4[c >> 4] = amax / 127.0f;
      }
    }
    lds_barrier();  // LDS only: the weight loads already issued stay in flight
    xi[0][0] = F::loadxi(reinterpret_cast<const int8_t *>(xq4), xd4, xs4, uid[0]);
  } else if constexpr (PRO == 1) {
    float v[PL][4][16];
#pragma unroll
    for (int p = 0; p < PL; p++) prologue_load<F>(xf, uid[p], uok[p], v[p]);
    first_loads();
#pragma unroll
    for (int p = 0; p < PL; p++) xi[p][0] = prologue_quant<F>(v[p]);
  } else if constexpr (!F32) {
    first_loads();
#pragma unroll
    for (int p = 0; p < PL; p++)
#pragma unroll
      for (int t = 0; t < TT; t++) {
        const uint32_t tc = t < (int)T ? t : 0;  // rows past T are never used
        xi[p][t] = F::loadxi(qx + (size_t)tc * n_in, dx + (size_t)tc * (n_in / 256),
                             s16 + (size_t)tc * (n_in / 16), uid[p]);
      }
  } else if constexpr (TT == 1) {
    first_loads();
#pragma unroll
    for (int p = 0; p < PL; p++) xr[p] = F::loadxf(xf, uid[p]);
  } else {
    first_loads();
  }

  // The team's run is ITERS row groups, fully unrolled: straight-line code
  // gives the compiler exact wait counts (each group waits only for its own
  // loads while the next NBUF-1 groups' are in flight) and nothing is loaded
  // past the run.
#pragma unroll
  for (int it = 0; it < ITERS; it++) {
    if (it + NBUF - 1 < ITERS) load(buf[(it + NBUF - 1) % NBUF], r_begin + (it + NBUF - 1) * R);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
    consume(buf[it % NBUF], it);
  }
  if constexpr (TW > 1) {
    __syncthreads();
    // Wave 0 of the team adds the waves' totals and stores the run's rows.
    if (team_live && tw == 0) {
      for (int i = lane; i < ITERS * R * TT; i += 64) {
        const int it = i / (R * TT), r = (i / TT) % R, t = i % TT;
        const uint32_t row = r_begin + it * R + r;
        if (row > r_last || t >= (int)T) continue;
        double g = 0.0, u = 0.0;
#pragma unroll
        for (int k = 0; k < TW; k++) {
          g += red[slot][k][(it * NR + r) * TT + t];
          if (GATED) u += red[slot][k][(it * NR + R + r) * TT + t];
        }
        if (GATED) {
          const float gf = (float)g, uf = (float)u;
          ygated[(size_t)t * n_out + row] = gf / (1.0f + expf(-gf)) * uf;
        } else {
          float yv = (float)g;
          if (ts.res) {  // uniform; one token
            // i == lane here (ITERS * R <= 64 rows per team at one token)
            yv = ((TT == 1 && !F32 && ITERS * R <= 64) ? res_pre : ts.res[row]) + yv;
            ssq_lane += (double)(yv * yv);
          }
          J.y[(size_t)t * n_out + row] = yv;
        }
      }
    }
  }
  if constexpr (!GATED) {
    if (ts.res) {
      // The workgroup's sum of squares: each wave's lanes, then the waves in
      // order (f32 squares added in f64, as the separate rmsnorm adds them).
      __shared__ double ssq_w[team_wg(PRO, TW) / 64];
      const double v = wave_total63(ssq_lane);
      if (lane == 63) ssq_w[wave] = v;
      __syncthreads();
      if (threadIdx.x == 0) {
        double tsum = 0.0;
        for (int k = 0; k < team_wg(PRO, TW) / 64; k++) tsum += ssq_w[k];
        ts.ssq[blockIdx.x] = tsum;
      }
    }
  }
}

// ----------------------------------------------------------- launcher ----

#ifndef MDMA_TEAM_R
#define MDMA_TEAM_R 2
#endif
#ifndef MDMA_TEAM_RG
#define MDMA_TEAM_RG 1
#endif
#ifndef MDMA_TEAM_WAVES_PER_CU
#define MDMA_TEAM_WAVES_PER_CU 12
#endif
#ifndef MDMA_NORM_WAVES_PER_CU
#define MDMA_NORM_WAVES_PER_CU 3
#endif

template <class F, bool F32, int R, int ITERS, int TT, bool GATED>
void launch_iters(mdma_ctx *ctx, TeamSet ts, int tw, int pl, const float *xf, const int8_t *qx, const float *dx,
                  const int32_t *s16, uint32_t T, float *yg) {
  ts.rpt = ITERS * R;
  uint64_t teams = 0;
  for (int i = 0; i < ts.n; i++) {
    ts.j[i].teams = (ts.j[i].n_out + ts.rpt - 1) / ts.rpt;
    teams += ts.j[i].teams;
  }
  constexpr bool PRO_OK = !F32 && TT == 1 && !std::is_same<F, Q8G>::value;
  const bool pro4 = PRO_OK && ts.pro && tw > 1 && pl == 1;
  // Staging x (PRO 3) pays for the fused gate/up and for Q4_K rows; the
  // Q6_K one-wave launches measured faster with per-lane loads.
  constexpr bool STAGE_OK = !F32 && TT == 1 && ITERS == 1 && (GATED || std::is_same<F, Q4G>::value);
  const bool pro3 = STAGE_OK && !(PRO_OK && ts.pro) && !ts.nsum && tw == 1 && pl == 1;
  const int wg = pro4 ? 64 * tw * MDMA_PRO4_TEAMS : (pro3 ? MDMA_PRO3_WG : WG), tpw = wg / 64 / tw;
  const dim3 grid((uint32_t)((teams + tpw - 1) / tpw)), block(wg);
  if (ts.ssq && grid.x > ts.ssq_cap) {  // one sum-of-squares partial per workgroup: no room, no launch
    ctx->team_grid = 0;
    return;
  }
  ctx->team_grid = grid.x;
  // With timing events set, the dispatch itself timestamps them (kernel-only
  // duration, as a profiler measures it); they apply to one launch.
  hipEvent_t t0 = ctx->time_start, t1 = ctx->time_stop;
  ctx->time_start = ctx->time_stop = nullptr;
  constexpr bool NORM_OK = !F32 && TT == 1 && !GATED && !std::is_same<F, Q8G>::value;
#define MDMA_TEAM_GO(TW_, PL_, PRO_)                                                                              \
  do {                                                                                                            \
    if constexpr (!F32) {                                                                                         \
      if (ts.j[0].dots) {                                                                                         \
        gemv_team<F, F32, R, ITERS, TW_, PL_, TT, GATED, PRO_, true><<<grid, block, 0, ctx->stream>>>(          \
            ts, xf, qx, dx, s16, T, yg);                                                                          \
        break;                                                                                                    \
      }                                                                                                           \
    }                                                                                                             \
    if (t0 || t1)                                                                                                 \
      hipExtLaunchKernelGGL(gemv_team<F, F32, R, ITERS, TW_, PL_, TT, GATED, PRO_>, grid, block, 0, ctx->stream,  \
                            t0, t1, 0, ts, xf, qx, dx, s16, T, yg);                                               \
    else                                                                                                          \
      gemv_team<F, F32, R, ITERS, TW_, PL_, TT, GATED, PRO_><<<grid, block, 0, ctx->stream>>>(ts, xf, qx, dx,   \
                                                                                              s16, T, yg);      \
  } while (0)
#define MDMA_TEAM_LAUNCH(TW_, PL_)                                      \
  do {                                                                  \
    if constexpr (PRO_OK) {                                             \
      if (ts.pro) {                                                     \
        if constexpr (TW_ > 1 && PL_ == 1) MDMA_TEAM_GO(TW_, PL_, 4);   \
        else MDMA_TEAM_GO(TW_, PL_, TW_ == 1 ? 2 : 1);                  \
        break;                                                          \
      }                                                                 \
    }                                                                   \
    if constexpr (NORM_OK && TW_ == 1 && PL_ == 1) {                    \
      if (ts.nsum) {                                                    \
        MDMA_TEAM_GO(TW_, PL_, 5);                                      \
        break;                                                          \
      }                                                                 \
    }                                                                   \
    if (ts.nsum) fail(MDMA_ERR_BACKEND, "normalizing GEMV: no variant for this shape"); \
    if constexpr (STAGE_OK && TW_ == 1 && PL_ == 1) MDMA_TEAM_GO(TW_, PL_, 3); \
    else MDMA_TEAM_GO(TW_, PL_, 0);                                     \
  } while (0)
  if (tw == 1) MDMA_TEAM_LAUNCH(1, 1);
  else if (tw == 2) MDMA_TEAM_LAUNCH(2, 1);
  else if (pl == 1) MDMA_TEAM_LAUNCH(4, 1);
  else if (pl == 2) MDMA_TEAM_LAUNCH(4, 2);
  else MDMA_TEAM_LAUNCH(4, 4);
#undef MDMA_TEAM_LAUNCH
#undef MDMA_TEAM_GO
  hip_check(hipGetLastError(), "gemv team launch");
}

template <class F, bool F32, int R, int TT, bool GATED>
void launch_fmt(mdma_ctx *ctx, TeamSet ts, const float *xf, const int8_t *qx, const float *dx, const int32_t *s16,
                uint32_t T, float *yg) {
  const uint32_t units = ts.n_in / F::UCOLS;
  int tw, pl;
  if (units <= 64) tw = 1, pl = 1;
  else if (units <= 128) tw = 2, pl = 1;
  else if (units <= 256) tw = 4, pl = 1;
  else if (units <= 512) tw = 4, pl = 2;
  else tw = 4, pl = 4;
  // Row groups per team: enough teams for MDMA_TEAM_WAVES_PER_CU waves per
  // CU, rounded up to a power of two (at most 16; batched: 4).
  uint64_t rows = 0;
  for (int i = 0; i < ts.n; i++) rows += ts.j[i].n_out;
  // A normalizing prologue reads 32 KB of f32 per workgroup: fewer, longer
  // teams read it fewer times (at Llama-3-8B's QKV, 3 waves per CU: four
  // row groups per team, measured best against 1, 2, 6 and 12).
  const uint64_t want = (uint64_t)ctx->cu_count * (ts.nsum ? MDMA_NORM_WAVES_PER_CU : MDMA_TEAM_WAVES_PER_CU) / tw;
  const uint64_t groups = ((rows + want - 1) / want + R - 1) / R;
  if constexpr (TT > 1) {
    launch_iters<F, F32, R, 4, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
  } else if (!F32 && !std::is_same<F, Q8G>::value && ts.pro && tw > 1 && pl == 1) {
    // x quantized once per workgroup of MDMA_PRO4_TEAMS teams: about one
    // workgroup per CU.
    const uint64_t per = (uint64_t)ctx->cu_count * MDMA_PRO4_TEAMS;
    const uint64_t g4 = ((rows + per - 1) / per + R - 1) / R;
    if (g4 <= 1) launch_iters<F, F32, R, 1, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else if (g4 <= 2) launch_iters<F, F32, R, 2, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else if (g4 <= 4) launch_iters<F, F32, R, 4, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else if (g4 <= 8) launch_iters<F, F32, R, 8, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else launch_iters<F, F32, R, 16, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
  } else if (GATED && !F32 && !ts.pro && tw == 1) {
    // The fused gate/up reading a quantized x: one row of gate and up per
    // wave (the most waves, each with all its loads issued at once), x
    // staged through LDS once per workgroup.
    launch_iters<F, F32, R, 1, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
  } else {
    if (groups <= 1) launch_iters<F, F32, R, 1, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else if (groups <= 2) launch_iters<F, F32, R, 2, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else if (groups <= 4) launch_iters<F, F32, R, 4, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else if (groups <= 8) launch_iters<F, F32, R, 8, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
    else launch_iters<F, F32, R, 16, TT, GATED>(ctx, ts, tw, pl, xf, qx, dx, s16, T, yg);
  }
}

// One format and activation mode: the launch for 1..8 tokens.
template <class F, bool F32>
void launch_mode(mdma_ctx *ctx, bool gated, const TeamSet &ts, const float *xf, const int8_t *qx, const float *dx,
                 const int32_t *s16, uint32_t T, float *yg) {
  constexpr int RP = MDMA_TEAM_R, RG = MDMA_TEAM_RG;
#define MDMA_TEAM_T(TT_)                                                      \
  do {                                                                        \
    if (gated)                                                                \
      launch_fmt<F, F32, RG, TT_, true>(ctx, ts, xf, qx, dx, s16, T, yg);    \
    else                                                                      \
      launch_fmt<F, F32, RP, TT_, false>(ctx, ts, xf, qx, dx, s16, T, yg);   \
  } while (0)
  if (T <= 1) MDMA_TEAM_T(1);
  else if (T <= 2) MDMA_TEAM_T(2);
  else if (T <= 4) MDMA_TEAM_T(4);
  else MDMA_TEAM_T(8);
#undef MDMA_TEAM_T
}

}  // namespace
}  // namespace mdma

namespace mdma {

// Arguments of one row-team launch (ts: the launching unit's TeamSet).
struct TeamSetArgs {
  const void *ts;
  const float *xf;
  const int8_t *qx;
  const float *dx;
  const int32_t *s16;
  uint32_t T;
  float *yg;
};
void team_launch_q4_i8(mdma_ctx *ctx, bool gated, const TeamSetArgs &a);
void team_launch_q4_f32(mdma_ctx *ctx, bool gated, const TeamSetArgs &a);
void team_launch_q6_i8(mdma_ctx *ctx, bool gated, const TeamSetArgs &a);
void team_launch_q6_f32(mdma_ctx *ctx, bool gated, const TeamSetArgs &a);
void team_launch_q8_i8(mdma_ctx *ctx, bool gated, const TeamSetArgs &a);
void team_launch_q8_f32(mdma_ctx *ctx, bool gated, const TeamSetArgs &a);

}  // namespace mdma
