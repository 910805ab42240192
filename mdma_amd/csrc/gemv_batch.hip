// Decode GEMV for 2..16 tokens (batched decode, short prefill chunks) in the
// int8-activation mode, on the int8 matrix cores of gfx950, over the
// prepared weight layouts (layout.cpp).
//
// y[t, r] = sum_i deq(W)[r, i] * x[t, i]   (reference Backend::qmatmul,
// /root/reference/src/backend.rs:469; int8 decode arithmetic of
// src/backend/rocm/kernels/decode.hip:47-108)
//
// With one token a row's weights are used once and the row-team kernels
// stream them at HBM speed with v_dot4; with T tokens every weight byte
// meets T activations and v_dot4 work grows T-fold, so from a few tokens up
// the products run on v_mfma_i32_16x16x32_i8 instead:
//  - A tile is 16 rows of one weight. Lane l supplies the weight bytes of
//    row l%16 and the activations of token l%16 (zero past T), both for
//    k-group g = l/16 (8 bytes each); result register j of lane l is the
//    int32 dot of token 4*(l/16) + j with row l%16.
//  - Every MFMA result has a single weight scale: for Q4_K the four
//    k-groups are the 32 columns of one sub-block (low nibbles of a unit's
//    32 bytes, then the high nibbles); for Q8_0 one 32-column block; for
//    Q6_K (scale groups of 16) lanes g = 0,1 carry a group of one unit and
//    lanes g = 2,3 the same group of the next unit, and each MFMA zeroes the
//    other pair's activations. Integer results are scaled in int32 per 256
//    columns as the reference sums sub-blocks:
//      Q4_K  d*sum(sc*isum) - dmin*sum(m*xsum), with m*xsum as an MFMA of x
//            against m repeated in every byte;
//      Q6_K  d*sum(sc*isum) with q - 32 fed as signed bytes;
//      Q8_0  sum(d*isum) per 32-column block;
//    then times the token's per-256 activation scale, accumulated in f32
//    (a handful of registers per result instead of twice that: the kernel's
//    speed is set by how many waves its registers let a SIMD hold).
//  - TW waves split a tile's columns in fixed chunks whose sums meet in LDS
//    (wave 0 adds them in a fixed order and stores, so results do not
//    depend on TW or on what else shares the launch).
//  - Weight bytes are read once per launch, 8 bytes per lane: a row plane's
//    16 contiguous bytes per unit go to two lanes, and the next units
//    continue the same 128-byte lines.
#include <hip/hip_ext.h>

#include "kernels.h"

namespace mdma {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t TROWS = 16;  // rows per tile

// Plain (cached) loads: a block reads half of each 128-byte line of a row
// plane and the next block the other half.
__device__ __forceinline__ uint64_t ldw8(const uint8_t *p) { return *reinterpret_cast<const uint64_t *>(p); }
__device__ __forceinline__ uint32_t ldw4(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
// A byte value (0..255) in all eight bytes: one byte permute (a multiply by
// 0x01010101 is quarter rate).
__device__ __forceinline__ uint64_t bytes8(int v) {
  const uint64_t r = __builtin_amdgcn_perm(0u, (uint32_t)v, 0u);
  return r | (r << 32);
}
__device__ __forceinline__ v4i mma(uint64_t x, uint64_t w, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x, (long)w, c, 0, 0, 0);
}

// Block-dot capture (GemvJob::dots): the row's slots for the block being
// computed (p: null when off), tokens stride apart, the first T live.
struct Dots {
  int32_t *p;
  size_t stride;
  uint32_t T;
  __device__ void put(uint32_t tok, uint32_t s, int v) const {
    if (tok < T) p[tok * stride + s] = v;
  }
};

// Activation bytes of the lane's token at column col.
struct XRow {
  const int8_t *p;
  __device__ uint64_t operator()(uint32_t col) const { return *reinterpret_cast<const uint64_t *>(p + col); }
};

// The weights of a wave's 16-row tile come in per 256-column block with
// 16-byte loads, four lanes per row reading 64 contiguous bytes of a row
// plane (plus one 16-byte per-row piece: Q4_K header, Q6_K scales, Q8_0
// scales), are staged in the wave's own LDS region, and are read back in
// the MFMA operand layout. Each format: Raw = one block's loads of a lane;
// gload issues them (prow: the lane's row for plane loads, row l/4; hrow:
// row l%16 for the per-row piece); lstore writes them to the wave's LDS;
// compute reads the operands back and returns the block's contributions
// c[j] (before the activation scale) for row l%16 and tokens 4*(l/16)+j.

// Q4_K: unit u = 64 columns, 32 quant bytes (16 in plane A, 16 in plane B);
// LDS per row: 4 units x [A 16 | B 16]; lane group g reads bytes 8g..8g+7:
// low nibbles are columns 64u + 8g + [0,8) (sub-block 2(u%4)), high
// nibbles 64u + 32 + 8g + [0,8).
struct BQ4 {
  static constexpr uint32_t UCOLS = 64;
  static constexpr uint32_t RS = 144;                 // LDS row stride (128 + pad)
  static constexpr uint32_t LDS = 16 * RS + 16 * 16;  // + headers
  __device__ static size_t row_bytes(uint32_t n_in) { return (size_t)(n_in / 256) * 144; }
  struct Raw {
    uint4 a, b, h;
  };
  struct X {
    uint64_t lo[4], hi[4];
  };
  __device__ static void gload(const uint8_t *prow, const uint8_t *hrow, uint32_t U, uint32_t b, uint32_t l,
                               Raw &r) {
    const size_t o = 16 * (size_t)(4 * b + (l & 3));
    r.a = ld16(prow + o);
    r.b = ld16(prow + 16 * (size_t)U + o);
    r.h = ld16(hrow + 32 * (size_t)U + 16 * (size_t)b);
  }
  __device__ static void lstore(const Raw &r, uint8_t *lds, uint32_t l) {
    uint8_t *p = lds + (l >> 2) * RS + 32 * (l & 3);
    *reinterpret_cast<uint4 *>(p) = r.a;
    *reinterpret_cast<uint4 *>(p + 16) = r.b;
    if (l < 16) *reinterpret_cast<uint4 *>(lds + 16 * RS + 16 * l) = r.h;
  }
  __device__ static void loadx(const XRow &xr, uint32_t b, uint32_t g, X &x) {
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t col = 256 * b + 64 * p + 8 * g;
      x.lo[p] = xr(col);
      x.hi[p] = xr(col + 32);
    }
  }
  static constexpr uint32_t SUBS = 8;  // capture slots per 256-column block
  __device__ static void compute(const uint8_t *lds, const X &x, uint32_t l, float *c, const Dots &dc) {
    const uint32_t n = l & 15, g = l >> 4;
    const uint4 h = *reinterpret_cast<const uint4 *>(lds + 16 * RS + 16 * n);
    constexpr uint64_t M4 = 0x0F0F0F0F0F0F0F0Full;
    v4i ai = {}, dm = {};
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint64_t w = *reinterpret_cast<const uint64_t *>(lds + n * RS + 32 * p + 8 * g);
      const v4i z = {};
      const v4i da = mma(x.lo[p], w & M4, z);
      const v4i db = mma(x.hi[p], (w >> 4) & M4, z);
      if (dc.p)
#pragma unroll
        for (int j = 0; j < 4; j++) dc.put(4 * g + j, 2 * p, da[j]), dc.put(4 * g + j, 2 * p + 1, db[j]);
      int sca, scb, ma, mb;
      q4k_scales_i(h, p, sca, scb, ma, mb);
      // 24-bit multiplies (full rate): |isum| <= 15*127*32.
#pragma unroll
      for (int j = 0; j < 4; j++) ai[j] += __mul24(sca, da[j]) + __mul24(scb, db[j]);
      dm = mma(x.lo[p], bytes8(ma), dm);
      dm = mma(x.hi[p], bytes8(mb), dm);
    }
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = d * (float)ai[j] - dmin * (float)dm[j];
  }
};

// Q6_K: unit u = (half n, group column h) of block u/4, quarters r = 0..3
// of 16 columns each (col below), one int8 scale per quarter. LDS per row:
// 4 units x [A 16 | B 16 | high bits 16], then the 16 scale bytes and d.
// Lanes g and g+2 (g = 0,1) take dwords 2g, 2g+1 of units 2v and 2v+1:
// columns col(u, r) + 8g + [0,8); each MFMA zeroes the other pair's x.
struct BQ6 {
  static constexpr uint32_t UCOLS = 64;
  static constexpr uint32_t RS = 208;  // 192 + pad
  static constexpr uint32_t LDS = 16 * RS + 16 * 16 + 16 * 4;
  __device__ static size_t row_bytes(uint32_t n_in) { return ((size_t)(n_in / 256) * 210 + 15) / 16 * 16; }
  __device__ static uint32_t u6(uint32_t a, uint32_t b, uint32_t h, int r) {
    switch (r) {
      case 0: return (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
      case 1: return (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
      case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
      default: return ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    }
  }
  __device__ static uint32_t col(uint32_t u, int r) {
    return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * r + 16 * (u & 1);
  }
  struct Raw {
    uint4 a, b, q, s;
    uint32_t d;    // the f16 d of blocks 2(b/2) and 2(b/2)+1 (one aligned word)
    uint32_t dsh;  // 16 * (b % 2): d's half
  };
  struct X {
    uint64_t q[2][4];  // [unit pair][quarter]
  };
  __device__ static void gload(const uint8_t *prow, const uint8_t *hrow, uint32_t U, uint32_t b, uint32_t l,
                               Raw &r) {
    const size_t o = 16 * (size_t)(4 * b + (l & 3));
    r.a = ld16(prow + o);
    r.b = ld16(prow + 16 * (size_t)U + o);
    r.q = ld16(prow + 32 * (size_t)U + o);
    r.s = ld16(hrow + 48 * (size_t)U + 16 * (size_t)b);
    // A 32-bit load: the f16 is taken out of it after the LDS round trip
    // (a 16-bit load's value would be re-masked where the compiler chooses,
    // possibly at the loop's latch, which then waits for the prefetch). The
    // row's padding covers the word's second half for the last odd block.
    r.d = ldw4(hrow + 52 * (size_t)U + 4 * (size_t)(b >> 1));
    r.dsh = 16 * (b & 1);
  }
  __device__ static void lstore(const Raw &r, uint8_t *lds, uint32_t l) {
    uint8_t *p = lds + (l >> 2) * RS + 48 * (l & 3);
    *reinterpret_cast<uint4 *>(p) = r.a;
    *reinterpret_cast<uint4 *>(p + 16) = r.b;
    *reinterpret_cast<uint4 *>(p + 32) = r.q;
    if (l < 16) {
      *reinterpret_cast<uint4 *>(lds + 16 * RS + 16 * l) = r.s;
      // d's word goes to LDS as loaded; its half is taken after the read back.
      *reinterpret_cast<uint32_t *>(lds + 16 * RS + 256 + 4 * l) = r.d >> r.dsh;
    }
  }
  __device__ static void loadx(const XRow &xr, uint32_t b, uint32_t g, X &x) {
#pragma unroll
    for (int v = 0; v < 2; v++)
#pragma unroll
      for (int r = 0; r < 4; r++) x.q[v][r] = xr(col(4 * b + 2 * v + (g >> 1), r) + 8 * (g & 1));
  }
  static constexpr uint32_t SUBS = 16;
  __device__ static void compute(const uint8_t *lds, const X &x, uint32_t l, float *c, const Dots &dc) {
    const uint32_t n = l & 15, g = l >> 4;
    const uint4 sc4 = *reinterpret_cast<const uint4 *>(lds + 16 * RS + 16 * n);
    const uint32_t scw[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
    v4i ai = {};
#pragma unroll
    for (int v = 0; v < 2; v++) {
      const uint8_t *p = lds + n * RS + 48 * (2 * v + (g >> 1)) + 8 * (g & 1);
      const uint64_t wa = *reinterpret_cast<const uint64_t *>(p);
      const uint64_t wb = *reinterpret_cast<const uint64_t *>(p + 16);
      const uint64_t wq = *reinterpret_cast<const uint64_t *>(p + 32);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t lo = q6_centre4(u6((uint32_t)wa, (uint32_t)wb, (uint32_t)wq, r));
        const uint32_t hi = q6_centre4(u6((uint32_t)(wa >> 32), (uint32_t)(wb >> 32), (uint32_t)(wq >> 32), r));
        const uint64_t wv = (uint64_t)lo | ((uint64_t)hi << 32);
        // Unit 2v: lanes g < 2; unit 2v+1: lanes g >= 2.
        const v4i z = {};
        const v4i d0 = mma(g < 2 ? x.q[v][r] : 0ull, wv, z);
        const v4i d1 = mma(g < 2 ? 0ull : x.q[v][r], wv, z);
        // Sub-block (16 columns) of unit 4b + 2v + e, quarter r: 8v + 2r + e.
        if (dc.p)
#pragma unroll
          for (int j = 0; j < 4; j++) dc.put(4 * g + j, 8 * v + 2 * r, d0[j]), dc.put(4 * g + j, 8 * v + 2 * r + 1, d1[j]);
        const int s0 = (int)(int8_t)((scw[2 * v] >> (8 * r)) & 0xff);
        const int s1 = (int)(int8_t)((scw[2 * v + 1] >> (8 * r)) & 0xff);
        // 24-bit multiplies (full rate): |isum| <= 32*127*16.
#pragma unroll
        for (int j = 0; j < 4; j++) ai[j] += __mul24(s0, d0[j]) + __mul24(s1, d1[j]);
      }
    }
    const float d = h2f((uint16_t)*reinterpret_cast<const uint32_t *>(lds + 16 * RS + 256 + 4 * n));
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = d * (float)ai[j];
  }
};

// Q8_0: 32-column blocks (U = n_in/32 units), 16 bytes in plane A and 16 in
// plane B; LDS per row: 8 units x [A 16 | B 16], then the 8 f16 scales.
// Lane group g reads bytes 8g..8g+7 of A|B = columns 32u + 8g + [0,8).
struct BQ8 {
  static constexpr uint32_t UCOLS = 32;
  static constexpr uint32_t RS = 272;  // 256 + pad
  static constexpr uint32_t LDS = 16 * RS + 16 * 16;
  __device__ static size_t row_bytes(uint32_t n_in) { return ((size_t)(n_in / 32) * 34 + 15) / 16 * 16; }
  struct Raw {
    uint4 a[2], b[2], d;
  };
  struct X {
    uint64_t q[8];
  };
  __device__ static void gload(const uint8_t *prow, const uint8_t *hrow, uint32_t U, uint32_t b, uint32_t l,
                               Raw &r) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const size_t o = 16 * (size_t)(8 * b + (l & 3) + 4 * i);
      r.a[i] = ld16(prow + o);
      r.b[i] = ld16(prow + 16 * (size_t)U + o);
    }
    r.d = ld16(hrow + 32 * (size_t)U + 16 * (size_t)b);
  }
  __device__ static void lstore(const Raw &r, uint8_t *lds, uint32_t l) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      uint8_t *p = lds + (l >> 2) * RS + 32 * ((l & 3) + 4 * i);
      *reinterpret_cast<uint4 *>(p) = r.a[i];
      *reinterpret_cast<uint4 *>(p + 16) = r.b[i];
    }
    if (l < 16) *reinterpret_cast<uint4 *>(lds + 16 * RS + 16 * l) = r.d;
  }
  __device__ static void loadx(const XRow &xr, uint32_t b, uint32_t g, X &x) {
#pragma unroll
    for (int i = 0; i < 8; i++) x.q[i] = xr(256 * b + 32 * i + 8 * g);
  }
  static constexpr uint32_t SUBS = 8;
  __device__ static void compute(const uint8_t *lds, const X &x, uint32_t l, float *c, const Dots &dc) {
    const uint32_t n = l & 15, g = l >> 4;
    const uint4 d4 = *reinterpret_cast<const uint4 *>(lds + 16 * RS + 16 * n);
    const uint32_t dw[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint64_t w = *reinterpret_cast<const uint64_t *>(lds + n * RS + 32 * i + 8 * g);
      const v4i z = {};
      const v4i dq = mma(x.q[i], w, z);
      if (dc.p)
#pragma unroll
        for (int j = 0; j < 4; j++) dc.put(4 * g + j, i, dq[j]);
      const float d = h2f(dw[i >> 1] >> (16 * (i & 1)));
#pragma unroll
      for (int j = 0; j < 4; j++) c[j] = fmaf(d, (float)dq[j], c[j]);
    }
  }
};

struct BatchJob {
  const uint8_t *w;
  float *y;
  uint32_t n_out, tiles;
  int32_t *dots;  // block-dot capture or null
};
struct BatchSet {
  BatchJob j[3];
  int n;
  uint32_t n_in;
};

// One workgroup = one tile of 16 rows (of gate and up when GATED), TW
// waves splitting its columns. The 256-column blocks form NCH = min(8, nb)
// fixed chunks; wave 0 adds every chunk's partial sums to its running total
// in chunk order (the other waves' chunks through LDS), so a row's result
// does not depend on TW (fused and separate calls, whatever their tile
// counts, give identical bits).
constexpr int NCHMAX = 8;
#ifndef MDMA_BATCH_NS
#define MDMA_BATCH_NS 2
#endif
// CAP: the block-dot capture instantiation (BatchJob::dots set).
template <class F, int TW, bool GATED, int NS, bool CAP = false>
__global__ __launch_bounds__(64 * TW) void gemv_batch(BatchSet bs, const int8_t *__restrict__ qx,
                                                      const float *__restrict__ dx, uint32_t T,
                                                      float *__restrict__ ygated) {
  constexpr int NR = GATED ? 2 : 1;
  __shared__ float red[TW > 1 ? NCHMAX : 1][NR][4][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  uint32_t tile = blockIdx.x;
  int ji = 0;
  if (bs.n > 1 && tile >= bs.j[0].tiles) {
    tile -= bs.j[0].tiles;
    ji = 1;
    if (bs.n > 2 && tile >= bs.j[1].tiles) {
      tile -= bs.j[1].tiles;
      ji = 2;
    }
  }
  const BatchJob J = ji == 0 ? bs.j[0] : (ji == 1 ? bs.j[1] : bs.j[2]);
  const uint32_t n_in = bs.n_in, nb = n_in / 256, n_out = J.n_out, U = n_in / F::UCOLS;
  const uint32_t nch = nb < NCHMAX ? nb : NCHMAX;
  const uint32_t g = lane >> 4, r_lane = tile * TROWS + (lane & 15);
  const size_t rb = F::row_bytes(n_in);
  // Rows read by the lane: l/4 for the plane loads, l%16 for the per-row
  // piece (rows past the end re-read the last row; their sums are not stored).
  const uint32_t prow_i = min(tile * TROWS + (lane >> 2), n_out - 1), hrow_i = min(r_lane, n_out - 1);
  const uint8_t *prow[NR], *hrow[NR];
  prow[0] = J.w + prow_i * rb, hrow[0] = J.w + hrow_i * rb;
  if (GATED) prow[NR - 1] = bs.j[1].w + prow_i * rb, hrow[NR - 1] = bs.j[1].w + hrow_i * rb;
  __shared__ __attribute__((aligned(16))) uint8_t stage[TW][NR][F::LDS];
  // Token rows past T read row T-1 again: their results are never stored.
  const uint32_t tok = min((uint32_t)(lane & 15), T - 1);
  const XRow xr{qx + (size_t)tok * n_in};
  // Token of result slot j.
  constexpr int NJ = 4;
  uint32_t tj[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) tj[j] = 4 * (lane >> 4) + j;
  // Scale loads are unconditional (a token past T reads token T-1's scale;
  // its results are never stored): a load under a branch leaves the
  // compiler unsure how many loads are in flight, and it then waits for all.
  uint32_t tj_c[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) tj_c[j] = min(tj[j], T - 1);
  float acc[NR][NJ], tot[NR][NJ];
  // A block's loads in flight: the weights (to be staged) and the lane's x.
  struct Slot {
    typename F::Raw w[NR];
    typename F::X x;
    float s[NJ];
    uint32_t b;
  };
  // Block-dot capture: the lane's row (of gate, of up), one slot per
  // sub-block; tokens n_out * n_sub apart.
  const uint32_t nsub = n_in / (256 / F::SUBS);
  int32_t *dcap[NR];
  dcap[0] = J.dots;
  if (GATED) dcap[NR - 1] = bs.j[1].dots;
  auto fill = [&](Slot &sl, uint32_t b) {
    sl.b = b;
#pragma unroll
    for (int r = 0; r < NR; r++) F::gload(prow[r], hrow[r], U, b, lane, sl.w[r]);
    F::loadx(xr, b, g, sl.x);
#pragma unroll
    for (int j = 0; j < NJ; j++) sl.s[j] = dx[(size_t)tj_c[j] * nb + b];
  };
  // Stage the weights in the wave's LDS, read them back as operands. The
  // LDS-only waits order the stores before the reads (and the previous
  // block's reads before the stores) without waiting for loads in flight.
  auto use = [&](const Slot &sl) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int r = 0; r < NR; r++) F::lstore(sl.w[r], stage[wave][r], lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int r = 0; r < NR; r++) {
      float c[NJ];
      Dots dc{nullptr, (size_t)n_out * nsub, T};
      if constexpr (CAP) {
        if (r_lane < n_out) dc.p = dcap[r] + (size_t)r_lane * nsub + F::SUBS * sl.b;
      }
      F::compute(stage[wave][r], sl.x, lane, c, dc);
#pragma unroll
      for (int j = 0; j < NJ; j++) acc[r][j] = fmaf(sl.s[j], c[j], acc[r][j]);
    }
  };
  // The wave's chunks and their blocks.
  const uint32_t c0 = wave * nch / TW, c1 = (wave + 1) * nch / TW;
  const uint32_t b0 = c0 * nb / nch, b1 = c1 * nb / nch;
  uint32_t ch = c0, ch_end = (c0 + 1) * nb / nch;
  // After block b: a finished chunk is added to wave 0's running total
  // (0 + c is exact, so the first chunk starts it) or stored for wave 0.
  auto chunk_done = [&](uint32_t b) {
    if (b + 1 == ch_end) {
#pragma unroll
      for (int r = 0; r < NR; r++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          if (wave == 0) tot[r][j] += acc[r][j];
          else red[ch][r][j][lane] = acc[r][j];
          acc[r][j] = 0.0;
        }
      ch++;
      ch_end = (ch + 1) * nb / nch;
    }
  };
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[r][j] = tot[r][j] = 0.0;
  // NS slots in rotation, each refilled right after its block is computed:
  // while a block is computed the NS-1 blocks after it are in flight (loads
  // clamped to the wave's last block: in bounds, fixed wait counts).
  if (b0 < b1) {
    Slot sl[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) {
      fill(sl[i], min(b0 + i, b1 - 1));
      __builtin_amdgcn_sched_barrier(0);  // slots issued in order (see below)
    }
    for (uint32_t b = b0; b < b1; b += NS) {
#pragma unroll
      for (int i = 0; i < NS; i++) {
        use(sl[i]);
        chunk_done(b + i);
        if (b + i + 1 >= b1) break;
        fill(sl[i], min(b + i + NS, b1 - 1));
        // Keep the refill's loads here: sunk past the next block's compute
        // they would be the newest in flight, and the in-order wait for the
        // next block would then wait for them too.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  if constexpr (TW > 1) {
    __syncthreads();
    if (wave > 0) return;
    for (uint32_t k = c1; k < nch; k++)
#pragma unroll
      for (int r = 0; r < NR; r++)
#pragma unroll
        for (int j = 0; j < NJ; j++) tot[r][j] += red[k][r][j][lane];
  }
  if (r_lane >= n_out) return;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    if (tj[j] >= T) continue;
    if (GATED) {
      const float gv = (float)tot[0][j], uv = (float)tot[NR - 1][j];
      ygated[(size_t)tj[j] * n_out + r_lane] = gv / (1.0f + expf(-gv)) * uv;
    } else {
      J.y[(size_t)tj[j] * n_out + r_lane] = (float)tot[0][j];
    }
  }
}

template <class F, int TW, int NS>
void launch_tw(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, bool gated, const int8_t *qx, const float *dx,
               uint32_t T, float *yg) {
  hipEvent_t t0 = ctx->time_start, t1 = ctx->time_stop;
  ctx->time_start = ctx->time_stop = nullptr;
  const dim3 grid(tiles), block(64 * TW);
  if (bs.j[0].dots) {
    if (gated) gemv_batch<F, TW, true, NS, true><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
    else gemv_batch<F, TW, false, NS, true><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
  } else if (gated) {
    if (t0 || t1)
      hipExtLaunchKernelGGL(gemv_batch<F, TW, true, NS>, grid, block, 0, ctx->stream, t0, t1, 0, bs, qx, dx, T, yg);
    else
      gemv_batch<F, TW, true, NS><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
  } else {
    if (t0 || t1)
      hipExtLaunchKernelGGL(gemv_batch<F, TW, false, NS>, grid, block, 0, ctx->stream, t0, t1, 0, bs, qx, dx, T,
                            yg);
    else
      gemv_batch<F, TW, false, NS><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
  }
  hip_check(hipGetLastError(), "gemv batch launch");
}

template <class F>
void launch_fmt(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, bool gated, const int8_t *qx, const float *dx,
                uint32_t T, float *yg) {
  // Waves per tile: enough for about 8 waves per CU, at most one per chunk
  // and at most 4 (longer chains per wave beat more, shorter ones here).
  const uint32_t nb = bs.n_in / 256, nch = nb < NCHMAX ? nb : NCHMAX;
  uint32_t tw = 1;
  while (tw < 4 && 2 * tw <= nch && (uint64_t)tiles * tw < (uint64_t)ctx->cu_count * 8) tw *= 2;
  // Two slots per wave: three or four (all loads of a short run in flight)
  // measured slower at every shape, the extra registers costing a wave.
  switch (tw) {
    case 1: launch_tw<F, 1, MDMA_BATCH_NS>(ctx, bs, tiles, gated, qx, dx, T, yg); break;
    case 2: launch_tw<F, 2, MDMA_BATCH_NS>(ctx, bs, tiles, gated, qx, dx, T, yg); break;
    default: launch_tw<F, 4, MDMA_BATCH_NS>(ctx, bs, tiles, gated, qx, dx, T, yg); break;
  }
}

}  // namespace

bool gemv_batch_ok(const GemvJob *jobs, int n_jobs, uint64_t T) {
  if (T < 2 || T > 16 || n_jobs < 1 || n_jobs > 3) return false;
  for (int i = 0; i < n_jobs; i++) {
    const GemvJob &j = jobs[i];
    if (j.layout != MDMA_LAYOUT_GFX950 || j.dtype != jobs[0].dtype || j.n_in != jobs[0].n_in) return false;
    if (j.dtype != DT_Q4_K && j.dtype != DT_Q6_K && j.dtype != DT_Q8_0) return false;
  }
  return jobs[0].n_in % 256 == 0 && jobs[0].n_in > 0;
}

void launch_gemv_batch(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, bool gated, const float *x, uint64_t T,
                       float *ygated) {
  const uint64_t n_in = jobs[0].n_in;
  int8_t *qx;
  float *dx;
  int32_t *s16;
  quantize_into_scratch(ctx, x, T, n_in, &qx, &dx, &s16);
  BatchSet bs{};
  bs.n = gated ? 1 : n_jobs;  // gated: tiles cover the gate rows and also read up
  bs.n_in = (uint32_t)n_in;
  uint32_t tiles = 0;
  for (int i = 0; i < (gated ? 2 : n_jobs); i++) {
    bs.j[i].w = jobs[i].w;
    bs.j[i].y = jobs[i].y;
    bs.j[i].dots = jobs[i].dots;
    bs.j[i].n_out = (uint32_t)jobs[i].n_out;
    bs.j[i].tiles = (uint32_t)((jobs[i].n_out + TROWS - 1) / TROWS);
    if (i < bs.n) tiles += bs.j[i].tiles;
  }
  if (!tiles) return;
  const uint32_t t = (uint32_t)T;
  const int32_t dt = jobs[0].dtype;
  if (dt == DT_Q4_K) launch_fmt<BQ4>(ctx, bs, tiles, gated, qx, dx, t, ygated);
  else if (dt == DT_Q6_K) launch_fmt<BQ6>(ctx, bs, tiles, gated, qx, dx, t, ygated);
  else launch_fmt<BQ8>(ctx, bs, tiles, gated, qx, dx, t, ygated);
}

}  // namespace mdma
