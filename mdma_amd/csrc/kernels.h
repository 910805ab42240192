// Device helpers shared by the gfx950 GEMV kernels: f16 conversion, 16-byte
// streaming loads, DPP wave reductions and the Q4_K block pieces.
#pragma once

#include "internal.h"

namespace mdma {
namespace {

// Values made ready in SGPRs at this point (kernel arguments: their scalar
// loads are issued here, together).
template <class A>
__device__ __forceinline__ int sgpr_ready1(const A &a) {
  asm volatile("" ::"s"(a));
  return 0;
}
template <class... A>
__device__ __forceinline__ void sgpr_ready(const A &...a) {
  const int order[] = {sgpr_ready1(a)...};  // in argument order
  (void)order;
}
// Workgroup barrier ordering LDS only: unlike __syncthreads it does not wait
// for this wave's global loads, so a prefetch stays in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Global memory straight into LDS (global_load_lds): each lane of the wave
// moves 16 (or 4) bytes from base + off to LDS address lds + 16 (4) * lane.
// Issued as inline assembly so that the compiler does not track it: its own
// LDS-DMA tracking cannot tell runtime-indexed LDS buffers apart and would
// wait for these loads before every LDS read of the other buffer. The
// kernel waits for them itself (lds_wait_dma) before reading what they
// wrote or publishing it at a barrier.
// The statement sets M0, a register the compiler reserves: clang does not
// honour M0 in a clobber list, so nothing here tells it that M0 changed.
// That is safe only while the kernels that use these helpers contain no
// other M0 use; tests/test_m0_usage.py compiles them and checks that every
// M0 write is one of these statements, directly followed by its DMA, and
// that no other instruction reads or writes M0.
__device__ __forceinline__ uint32_t lds_addr(const void *lds) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);  // the LDS offset: low bits of the address
}
__device__ __forceinline__ void lds_dma16(const void *base, uint32_t off, const void *lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_addr(lds))
               : "memory");
}
__device__ __forceinline__ void lds_dma4(const void *base, uint32_t off, const void *lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds_addr(lds))
               : "memory");
}
__device__ __forceinline__ void lds_wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// A GEMM workgroup's output tile (column tile x, token tile y) on a grid of
// nx column tiles by ny token tiles. Workgroups go to the 8 XCDs, each with
// its own L2, round-robin by dispatch index d = y * nx + x (the same for
// every split z when nx * ny is a multiple of 8). XCD j = d % 8 takes the
// tiles [j P, (j + 1) P), P = nx ny / 8, of an order that walks gt token
// tiles for each column tile, so the workgroups on one XCD share a few token
// tiles' activations instead of reading every token tile once per column
// tile they hold. Grids whose tile count is not a multiple of 8 keep the
// dispatch order.
struct GridTile {
  uint32_t x, y;
};
__device__ __forceinline__ GridTile grid_tile(uint32_t gt) {
  const uint32_t nx = gridDim.x, ny = gridDim.y, n = nx * ny;
  if (gt == 0 || ny < 2 || n % 8) return GridTile{blockIdx.x, blockIdx.y};
  const uint32_t d = blockIdx.y * nx + blockIdx.x, l = (d % 8) * (n / 8) + d / 8;
  const uint32_t g = l / (gt * nx), y0 = g * gt, gn = min(gt, ny - y0), r = l - y0 * nx;
  return GridTile{r / gn, y0 + r % gn};
}

typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// silu_mul of one element (cpu.rs:447-458): (g / (1 + exp(-g))) * u, each
// operation rounded on its own (no contraction), the device expf. The
// elementwise kernel and the prefill GEMM's fused gate/up epilogue share it,
// so both give the same bits.
__device__ __forceinline__ float silu_mul1(float g, float u) {
#pragma clang fp contract(off)
  const float s = g / (1.0f + expf(-g));
  return s * u;
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xffff));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Streaming 16-byte weight load (nontemporal: weights are read once per token).
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
// Plain 16-byte load (activations: re-read by many waves, keep them cached).
__device__ __forceinline__ uint4 ldx16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ uint32_t ldu16(const uint8_t *p) {
  return *reinterpret_cast<const uint16_t *>(p);
}
// A dword made of two 2-byte-aligned halves (raw Q6_K / Q8_0 blocks are only
// 2-byte aligned inside a row).
__device__ __forceinline__ uint32_t ld2x16(const uint8_t *p) { return ldu16(p) | (ldu16(p + 2) << 16); }

// Four Q6_K values (bytes 0..63) as the signed int8 bytes v - 32. With bit 7
// set first every byte is at least 0x80, so subtracting 0x20 per byte never
// borrows from the next; clearing bit 7 again leaves (v - 32) mod 256. Three
// full-rate operations (a sign-fill of bit 5 instead compiles to a
// quarter-rate multiply by 6).
__device__ __forceinline__ uint32_t q6_centre4(uint32_t v) {
  return ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

// The int8 of activation v at scale inv = 127/amax: v * inv rounded half
// away from zero, clamped to [-127, 127] (a NaN gives -127, as
// fminf(fmaxf(NaN, -127), 127) does). trunc(r + copysign(0.5 - 2^-25, r))
// equals roundf(r) for every float |r| < 2^22: a tie k + 0.5 sums to
// k + 1 - 2^-25, which rounds to k + 1; below a tie the sum stays more than
// half an ulp under k + 1; above it the sum is at least k + 1. (Adding 0.5
// itself fails at 0.5 - 2^-25, whose sum rounds up to 1.) Five instructions
// instead of roundf's seven plus the clamp. The product is rounded to f32
// before the addition, as the CPU computes it: contraction into one FMA
// (which HIP's default fp-contract allows across statements) would skip
// that rounding and move rare values across a tie.
__device__ __forceinline__ int q8_quant(float v, float inv) {
#pragma clang fp contract(off)
  const float r = v * inv;
  const float t = r + __builtin_copysignf(0x1.fffffep-2f, r);
  return (int)fminf(fmaxf(t, -127.f), 127.f);
}
// Bytes 0 of four ints packed into one dword (q0 lowest).
__device__ __forceinline__ uint32_t pack4_i8(int q0, int q1, int q2, int q3) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x04000c0cu);
  return lo | hi;
}

// Wave-wide sum through DPP lane moves (no LDS round trips): xor 1, xor 2,
// half-row mirror, row mirror (16-lane sums in every lane), then row
// broadcasts 15 and 31. The total is valid in lane 63 only.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_step(float v) {
  return v + __builtin_bit_cast(float, dpp_u32<CTRL, ROWS>(__builtin_bit_cast(uint32_t, v)));
}
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_step(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_u32<CTRL, ROWS>((uint32_t)b), hi = dpp_u32<CTRL, ROWS>((uint32_t)(b >> 32));
  return v + __builtin_bit_cast(double, (hi << 32) | lo);
}
template <class V>
__device__ __forceinline__ V wave_total63(V v) {
  v = dpp_step<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v = dpp_step<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v = dpp_step<0x141, 0xF>(v);  // row_half_mirror
  v = dpp_step<0x140, 0xF>(v);  // row_mirror
  v = dpp_step<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_step<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_max(float v) {
  const float o = __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -INFINITY), __builtin_bit_cast(int, v), CTRL, ROWS,
                                         0xF, false));
  return fmaxf(v, o);
}
// Max / sum over the 64 lanes, the result in every lane.
__device__ __forceinline__ float wave_max_all(float v) {
  v = dpp_max<0xB1, 0xF>(v);
  v = dpp_max<0x4E, 0xF>(v);
  v = dpp_max<0x141, 0xF>(v);
  v = dpp_max<0x140, 0xF>(v);
  v = dpp_max<0x142, 0xA>(v);
  v = dpp_max<0x143, 0xC>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum_all(float v) {
  v = wave_total63(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Six-bit (scale, min) of Q4_K sub-blocks 2p and 2p+1 from the header's
// 12 scale bytes (hd.y, hd.z, hd.w): get_scale_min_k4 of
// /root/reference/src/backend/rocm/kernels/kernels.hip:19-27, evaluated for
// two sub-blocks at once in packed bytes.
__device__ __forceinline__ void q4k_scales_i(uint4 hd, int p, int &sca, int &scb, int &ma, int &mb) {
  const uint32_t s0 = hd.y, s1 = hd.z, s2 = hd.w;
  const uint32_t scw = p < 2 ? (s0 & 0x3F3F3F3Fu) : ((s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u));
  const uint32_t mw = p < 2 ? (s1 & 0x3F3F3F3Fu) : (((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u));
  const int sh = (p & 1) * 16;
  sca = (scw >> sh) & 0xff;
  scb = (scw >> (sh + 8)) & 0xff;
  ma = (mw >> sh) & 0xff;
  mb = (mw >> (sh + 8)) & 0xff;
}

// Exact products: a quant byte b (0..255) placed by one v_perm_b32 into
// mantissa bits 40..47 of an f64 whose exponent is fixed gives the double
// 2 + b/2048 with no conversion instruction. Its product with an activation
// converted to f64 is exact, and short chains accumulate in f64, so
//     sum(q*x) = 2048*acc - (4096 + 2048*bias)*X,  X = sum(x)
// where q = b - bias.
constexpr uint32_t F64_HI_TWO = 0x40000000u;  // high dword of 2.0

// f64 value 2 + byte_k(w)/2048 (k compile-time).
template <int K>
__device__ __forceinline__ double byte_f64(uint32_t w) {
  constexpr uint32_t sel = 0x070C000Cu | ((uint32_t)K << 8);
  const uint32_t hi = __builtin_amdgcn_perm(F64_HI_TWO, w, sel);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32));
}

// acc += sum_k (2 + byte_k(w)/2048) * x[k] over the 4 bytes of w.
__device__ __forceinline__ double fma4(uint32_t w, const double *x, double acc) {
  acc = fma(byte_f64<0>(w), x[0], acc);
  acc = fma(byte_f64<1>(w), x[1], acc);
  acc = fma(byte_f64<2>(w), x[2], acc);
  acc = fma(byte_f64<3>(w), x[3], acc);
  return acc;
}

// Interleaved-pair rotation (apply_rope, cpu.rs:68-84) of one pair.
__device__ __forceinline__ void rot(float &x0, float &x1, float c, float s) {
#pragma clang fp contract(off)
  const float a = x0 * c, bb = x1 * s, cc = x0 * s, d = x1 * c;
  x0 = a - bb;
  x1 = cc + d;
}

}  // namespace
}  // namespace mdma
