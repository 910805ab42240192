// expf with the results of the C library's expf, for the device (and the
// host, where a test compares it with the C library on every f32 input).
//
// The CPU backend's softmax and SiLU (/root/reference/src/backend/cpu.rs:
// 50-60, 447-458) call Rust's f32::exp, which on x86-64 Linux is the C
// library's expf. glibc (2.28 on; 2.35 in this image) computes it with the
// method of the expf in ARM's optimized-routines (Szabolcs Nagy, MIT
// licence), in double precision:
//   x * 32/ln2 = k + r, k the nearest integer (the 0x1.8p52 shift trick),
//   2^(k/32) = the table entry 2^((k mod 32)/32) with k/32 added to its
//   exponent field,
//   2^(r/32) ~ C0 r^3 + C1 r^2 + C2 r + 1 (the routine's published
//   coefficients: the minimax cubic for 2^r on [-1/2, 1/2] scaled by
//   32^-3, 32^-2, 32^-1),
// and the double result rounded once to f32. On CPUs with FMA (the MI355X
// box's EPYC and the build container's Xeon) glibc selects its FMA build of
// the routine, in which the compiler fused each multiply-add: the shift
// add, the reduction r = x * 32/ln2 - k and the three polynomial steps.
// This function performs exactly those IEEE double operations, which the
// GPU rounds as the CPU does, so its results equal the C library's expf;
// tests/test_libm_expf.py checks all 2^32 inputs against the C library on
// the CPU.
#pragma once

#include <stdint.h>
#include <string.h>

#ifndef __HIPCC__
#include <math.h>
#define MDMA_HD inline
#else
#define MDMA_HD __host__ __device__ __forceinline__
#endif

namespace mdma {

// 2^(i/32) rounded to the nearest double, minus i << 47 (so adding k << 47
// for k = 32 q + i gives 2^(q + i/32)); checked against exp2l on the CPU.
#define MDMA_EXP2_TABLE                                                                            \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,     \
   0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,     \
   0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,     \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,     \
   0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,     \
   0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,     \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,     \
   0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

MDMA_HD uint64_t exp2_table(uint32_t i) {
  const uint64_t t[32] = MDMA_EXP2_TABLE;
  return t[i];
}

MDMA_HD float libm_expf(float x) {
#pragma clang fp contract(off)
  uint32_t ux;
  memcpy(&ux, &x, 4);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {                   // |x| >= 88, or x is NaN or infinite
    if (ux == 0xff800000u) return 0.0f;    // -inf
    if (abstop >= 0x7f8) return x + x;     // NaN or +inf
    if (x > 0x1.62e42ep6f) return __builtin_inff();  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;            // underflow
  }
  const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
               c2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  double kd = __builtin_fma(inv_ln2_32, xd, shift);
  uint64_t ki;
  memcpy(&ki, &kd, 8);
  kd -= shift;
  const double r = __builtin_fma(inv_ln2_32, xd, -kd);
  uint64_t t = exp2_table((uint32_t)(ki % 32));
  t += ki << 47;
  double s;
  memcpy(&s, &t, 8);
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

}  // namespace mdma
