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
  // Operands of the staged kernel: the tile in the wave's LDS, x in registers.
  struct Staged {
    const uint8_t *lds;
    uint32_t n, g;
    const X &x;
    __device__ uint4 hdr() const { return *reinterpret_cast<const uint4 *>(lds + 16 * RS + 16 * n); }
    __device__ uint64_t w(int p) const { return *reinterpret_cast<const uint64_t *>(lds + n * RS + 32 * p + 8 * g); }
    __device__ uint64_t xg(int j) const { return j & 1 ? x.hi[j >> 1] : x.lo[j >> 1]; }
  };
  // The block's contributions c[j] (before the activation scale) for row
  // l%16 and tokens 4*(l/16)+j, from the operand source op: hdr() the row's
  // 16-byte header, w(p) the lane's 8 quant bytes of unit p, xg(j) the
  // lane's 8 activation bytes of the block's 32-column group j.
  template <class Op>
  __device__ static void compute(const Op &op, float *c, const Dots &dc, uint32_t g) {
    const uint4 h = op.hdr();
    constexpr uint64_t M4 = 0x0F0F0F0F0F0F0F0Full;
    v4i ai = {}, dm = {};
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint64_t w = op.w(p);
      const uint64_t xlo = op.xg(2 * p), xhi = op.xg(2 * p + 1);
      const v4i z = {};
      const v4i da = mma(xlo, w & M4, z);
      const v4i db = mma(xhi, (w >> 4) & M4, z);
      if (dc.p)
#pragma unroll
        for (int j = 0; j < 4; j++) dc.put(4 * g + j, 2 * p, da[j]), dc.put(4 * g + j, 2 * p + 1, db[j]);
      int sca, scb, ma, mb;
      q4k_scales_i(h, p, sca, scb, ma, mb);
      // 24-bit multiplies (full rate): |isum| <= 15*127*32.
#pragma unroll
      for (int j = 0; j < 4; j++) ai[j] += __mul24(sca, da[j]) + __mul24(scb, db[j]);
      dm = mma(xlo, bytes8(ma), dm);
      dm = mma(xhi, bytes8(mb), dm);
    }
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = d * (float)ai[j] - dmin * (float)dm[j];
  }
  __device__ static void compute(const uint8_t *lds, const X &x, uint32_t l, float *c, const Dots &dc) {
    compute(Staged{lds, l & 15, l >> 4, x}, c, dc, l >> 4);
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
  struct Staged {
    const uint8_t *lds;
    uint32_t n, g;
    const X &x;
    __device__ uint4 sc() const { return *reinterpret_cast<const uint4 *>(lds + 16 * RS + 16 * n); }
    __device__ float d() const {
      return h2f((uint16_t)*reinterpret_cast<const uint32_t *>(lds + 16 * RS + 256 + 4 * n));
    }
    // Plane k (A, B, high bits) of the lane's unit of pair v.
    __device__ uint64_t w(int v, int k) const {
      return *reinterpret_cast<const uint64_t *>(lds + n * RS + 48 * (2 * v + (g >> 1)) + 8 * (g & 1) + 16 * k);
    }
    __device__ uint64_t xg(int j) const { return x.q[j >> 2][j & 3]; }
  };
  // As BQ4::compute: sc() the row's 16 scale bytes, d() its d, w(v, k)
  // plane k's 8 bytes of the lane's unit of pair v, xg(4v + r) the lane's
  // activations of quarter r of pair v (the block's 32-column group 4v+r).
  template <class Op>
  __device__ static void compute(const Op &op, float *c, const Dots &dc, uint32_t g) {
    const uint4 sc4 = op.sc();
    const uint32_t scw[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
    v4i ai = {};
#pragma unroll
    for (int v = 0; v < 2; v++) {
      const uint64_t wa = op.w(v, 0), wb = op.w(v, 1), wq = op.w(v, 2);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t lo = q6_centre4(u6((uint32_t)wa, (uint32_t)wb, (uint32_t)wq, r));
        const uint32_t hi = q6_centre4(u6((uint32_t)(wa >> 32), (uint32_t)(wb >> 32), (uint32_t)(wq >> 32), r));
        const uint64_t wv = (uint64_t)lo | ((uint64_t)hi << 32);
        const uint64_t xq = op.xg(4 * v + r);
        // Unit 2v: lanes g < 2; unit 2v+1: lanes g >= 2.
        const v4i z = {};
        const v4i d0 = mma(g < 2 ? xq : 0ull, wv, z);
        const v4i d1 = mma(g < 2 ? 0ull : xq, wv, z);
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
    const float d = op.d();
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = d * (float)ai[j];
  }
  // compute for at most 8 tokens, with half the MFMAs and scale products:
  // token slots 8..15 of the MFMA carry tokens 0..7 again, so one MFMA forms
  // both sub-blocks of a 32-column group. Lane l supplies x of slot n = l%16
  // at k-group g = l/16, kept where the slot's half matches the k-group's
  // unit (slots 0..7: unit 2v, k-groups 0, 1; slots 8..15: unit 2v+1,
  // k-groups 2, 3) and zero elsewhere. Results: lanes with g < 2 hold unit
  // 2v's dots of tokens 4g+j, lanes with g >= 2 unit 2v+1's of tokens
  // 4(g-2)+j; each lane scales by its own sub-block's scale, and the two
  // halves' int32 sums meet across lanes l and l^32 once per block: c[j] is
  // compute's integer total, so the results are the same bits.
  template <class Op>
  __device__ static void compute_paired(const Op &op, float *c, const Dots &dc, uint32_t g, uint32_t n) {
    const uint4 sc4 = op.sc();
    const bool hi = g >= 2;
    const uint32_t scl[2] = {hi ? sc4.y : sc4.x, hi ? sc4.w : sc4.z};
    const bool keep = (n >= 8) == hi;
    v4i ai = {};
#pragma unroll
    for (int v = 0; v < 2; v++) {
      const uint64_t wa = op.w(v, 0), wb = op.w(v, 1), wq = op.w(v, 2);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t lo = q6_centre4(u6((uint32_t)wa, (uint32_t)wb, (uint32_t)wq, r));
        const uint32_t hw = q6_centre4(u6((uint32_t)(wa >> 32), (uint32_t)(wb >> 32), (uint32_t)(wq >> 32), r));
        const uint64_t wv = (uint64_t)lo | ((uint64_t)hw << 32);
        const v4i z = {};
        const v4i dd = mma(keep ? op.xg(4 * v + r) : 0ull, wv, z);
        if (dc.p)
#pragma unroll
          for (int j = 0; j < 4; j++) dc.put(4 * (g & 1) + j, 8 * v + 2 * r + (g >> 1), dd[j]);
        const int s = (int)(int8_t)((scl[v] >> (8 * r)) & 0xff);
#pragma unroll
        for (int j = 0; j < 4; j++) ai[j] += __mul24(s, dd[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const auto p = __builtin_amdgcn_permlane32_swap(ai[j], ai[j], false, false);
      ai[j] = (int)(p[0] + p[1]);
    }
    const float d = op.d();
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = d * (float)ai[j];
  }
  __device__ static void compute(const uint8_t *lds, const X &x, uint32_t l, float *c, const Dots &dc) {
    compute(Staged{lds, l & 15, l >> 4, x}, c, dc, l >> 4);
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
  struct Staged {
    const uint8_t *lds;
    uint32_t n, g;
    const X &x;
    __device__ uint4 sc() const { return *reinterpret_cast<const uint4 *>(lds + 16 * RS + 16 * n); }
    __device__ uint64_t w(int i) const { return *reinterpret_cast<const uint64_t *>(lds + n * RS + 32 * i + 8 * g); }
    __device__ uint64_t xg(int i) const { return x.q[i]; }
  };
  // As BQ4::compute: sc() the row's eight f16 scales, w(i) the lane's 8
  // quant bytes of block i, xg(i) the lane's activations of block i.
  template <class Op>
  __device__ static void compute(const Op &op, float *c, const Dots &dc, uint32_t g) {
    const uint4 d4 = op.sc();
    const uint32_t dw[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint64_t w = op.w(i);
      const v4i z = {};
      const v4i dq = mma(op.xg(i), w, z);
      if (dc.p)
#pragma unroll
        for (int j = 0; j < 4; j++) dc.put(4 * g + j, i, dq[j]);
      const float d = h2f(dw[i >> 1] >> (16 * (i & 1)));
#pragma unroll
      for (int j = 0; j < 4; j++) c[j] = fmaf(d, (float)dq[j], c[j]);
    }
  }
  __device__ static void compute(const uint8_t *lds, const X &x, uint32_t l, float *c, const Dots &dc) {
    compute(Staged{lds, l & 15, l >> 4, x}, c, dc, l >> 4);
  }
};

struct BatchJob {
  const uint8_t *w;
  const uint8_t *wt;  // the weight's tile image (tile_repack_q6) or null
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


// ---------------------------------------------------------------------------
// The DMA-ring kernel (the default): gemv_batch's products and summation
// order (its results are equal bit for bit), with every byte a block needs
// moved by global_load_lds straight into a ring of two LDS slots per wave:
// one pair of 256-column blocks is computed while the next pair lands. The
// wave holds no registers for the loads in flight and waits for a pair
// with an exact count (s_waitcnt vmcnt) rather than the compiler's, which
// drains every load in flight. A pair makes each row's plane read a whole
// 128-byte line: one request, where one block's 64 bytes take one each.
//
// A slot (the pair's 512 columns of the wave's tile):
//   x      a 512-byte row per token (XN = 8 or 16 rows); the 16-byte chunk
//          k of token t at position k ^ t, so 16 tokens reading the same
//          32-column group hit distinct banks. Tokens past T repeat T-1.
//   scale  the pair's per-256 activation scales, [block][token] (f32).
//   w      per weight: each plane as 16 rows x RB bytes (RB: the row's
//          plane bytes for the pair), the 16-byte chunk c of row n at
//          position c ^ (n * RB / 256), so 16 rows reading one chunk hit
//          distinct banks; then the per-row pieces, [row][block] 16 bytes.
// An operand read is one XOR of the lane's base offset with 16c (weight
// chunk c) or 32j (x group j of the pair's 16).

// A plane of RB bytes per row in the slot (64 lanes x 16 bytes per DMA).
template <uint32_t RB>
struct Plane {
  static constexpr uint32_t CH = RB / 16;      // 16-byte chunks per row
  static constexpr uint32_t ROWS = 64 / CH;    // rows per DMA
  static constexpr uint32_t NDMA = 16 / ROWS;  // DMAs per plane
  static constexpr uint32_t BYTES = 16 * RB;
  __device__ static uint32_t f(uint32_t n) { return (n * RB) >> 8; }
  __device__ static uint32_t row(uint32_t L, int k) { return ROWS * k + L / CH; }
  __device__ static uint32_t chunk(uint32_t L, int k) { return (L % CH) ^ f(row(L, k)); }
  // Read base of lane (row n, k-group g) before the chunk's XOR.
  __device__ static uint32_t base(uint32_t n, uint32_t g) { return RB * n + 8 * (g & 1) + 16 * f(n); }
  template <int NP>
  __device__ static void src(size_t rb, uint32_t row0, uint32_t n_out, uint32_t L, uint32_t (&o)[NDMA]) {
#pragma unroll
    for (int k = 0; k < (int)NDMA; k++) o[k] = (uint32_t)(min(row0 + row(L, k), n_out - 1) * rb) + 16 * chunk(L, k);
  }
  // Plane DMAs of pair s: the plane starts at pl in the row.
  __device__ static void issue(const uint8_t *w, const uint32_t (&o)[NDMA], uint32_t pl, uint32_t s, uint8_t *dst) {
#pragma unroll
    for (int k = 0; k < (int)NDMA; k++) lds_dma16(w, o[k] + pl + RB * s, dst + 1024 * k);
  }
};
// Source of lane L for a 16-byte-per-row-per-block piece at off in the
// row: lanes 0..31 load rows L/2, halves L%2 (the pair's two blocks).
__device__ __forceinline__ uint32_t pair_piece(size_t rb, uint32_t row0, uint32_t n_out, uint32_t L, uint32_t off) {
  return (uint32_t)(min(row0 + ((L >> 1) & 15), n_out - 1) * rb) + off + 16 * (L & 1);
}
__device__ __forceinline__ void issue_piece(const uint8_t *w, uint32_t o, uint32_t s, uint8_t *dst, uint32_t L) {
  if (L < 32) lds_dma16(w, o + 32 * s, dst);
}

// Q4_K: planes A | B, then the headers.
struct RQ4 {
  using B = BQ4;
  static constexpr bool PAIRED = false;  // B::compute_paired (at most 8 tokens)
  // A tile image (issue_tile) measured no faster than the row planes for
  // Q4_K (gate/up at 8 tokens 16.6 against 16.1-16.6 us).
  static constexpr bool TILED = false;
  using P = Plane<128>;
  static constexpr uint32_t WB = 2 * P::BYTES + 512;
  static constexpr int NDMA = 2 * P::NDMA + 1;
  static constexpr int NDMA_T = NDMA;
  struct Src {
    uint32_t pl[P::NDMA], hd, U;
  };
  __device__ static Src src(size_t rb, uint32_t n_in, uint32_t row0, uint32_t n_out, uint32_t L) {
    Src s;
    s.U = n_in / 64;
    P::src<2>(rb, row0, n_out, L, s.pl);
    s.hd = pair_piece(rb, row0, n_out, L, 32 * s.U);
    return s;
  }
  __device__ static void issue(const uint8_t *w, const Src &s, uint32_t sp, uint8_t *slot, uint32_t L) {
    P::issue(w, s.pl, 0, sp, slot);
    P::issue(w, s.pl, 16 * s.U, sp, slot + P::BYTES);
    issue_piece(w, s.hd, sp, slot + 2 * P::BYTES, L);
  }
  __device__ static uint32_t wofs(uint32_t n, uint32_t g) { return P::base(n, g) + P::BYTES * (g >> 1); }
  // Block bi's operands of lane (row n, base wo), read from the slot
  // ahead of its products; x: the lane's eight activation groups.
  struct Op {
    uint4 h;
    uint64_t q[4];
    const uint64_t *x;
    __device__ uint4 hdr() const { return h; }
    __device__ uint64_t w(int p) const { return q[p]; }
    __device__ uint64_t xg(int j) const { return x[j]; }
  };
  __device__ static Op load(const uint8_t *ws, const uint64_t *x, uint32_t wo, uint32_t n, uint32_t bi) {
    Op o;
    o.h = *reinterpret_cast<const uint4 *>(ws + 2 * P::BYTES + 32 * n + 16 * bi);
#pragma unroll
    for (int p = 0; p < 4; p++) o.q[p] = *reinterpret_cast<const uint64_t *>(ws + (wo ^ (16 * (4 * bi + p))));
    o.x = x;
    return o;
  }
};

// Q6_K: planes A | B | high bits, the scale bytes, then d: the word of
// lane n (at 4n) holds row n's f16 d of the pair's two blocks.
struct RQ6 {
  using B = BQ6;
  static constexpr bool PAIRED = true;
  static constexpr bool TILED = true;
  using P = Plane<128>;
  static constexpr uint32_t WB = 3 * P::BYTES + 512 + 256;
  static constexpr int NDMA = 3 * P::NDMA + 2;
  // The tile image of a (tile, pair): the slot's weight bytes as issue()
  // leaves them (planes A, B, high bits, the scale bytes, then the 16 rows'
  // d words), IMG bytes in a row: six 1 KiB DMAs and one of 36 lanes.
  static constexpr uint32_t IMG = 3 * P::BYTES + 512 + 64;
  static constexpr int NDMA_T = (IMG + 1023) / 1024;
  static_assert(IMG % 16 == 0 && IMG <= WB, "the image fits the slot");
  // o: the pair's image offset in the tile's images plus 16 * L.
  __device__ static void issue_tile(const uint8_t *wt, uint32_t o, uint8_t *slot, uint32_t L) {
#pragma unroll
    for (int i = 0; i < NDMA_T - 1; i++) lds_dma16(wt, o + 1024 * i, slot + 1024 * i);
    if (L < (IMG - 1024 * (NDMA_T - 1)) / 16) lds_dma16(wt, o + 1024 * (NDMA_T - 1), slot + 1024 * (NDMA_T - 1));
  }
  struct Src {
    uint32_t pl[P::NDMA], sc, d, U;
  };
  __device__ static Src src(size_t rb, uint32_t n_in, uint32_t row0, uint32_t n_out, uint32_t L) {
    Src s;
    s.U = n_in / 64;
    P::src<3>(rb, row0, n_out, L, s.pl);
    s.sc = pair_piece(rb, row0, n_out, L, 48 * s.U);
    s.d = (uint32_t)(min(row0 + (L & 15), n_out - 1) * rb) + 52 * s.U;
    return s;
  }
  __device__ static void issue(const uint8_t *w, const Src &s, uint32_t sp, uint8_t *slot, uint32_t L) {
#pragma unroll
    for (int k = 0; k < 3; k++) P::issue(w, s.pl, 16 * k * s.U, sp, slot + k * P::BYTES);
    issue_piece(w, s.sc, sp, slot + 3 * P::BYTES, L);
    lds_dma4(w, s.d + 4 * sp, slot + 3 * P::BYTES + 512);
  }
  // The lane's unit half g/2 is bit 0 of its chunks: folded into the base.
  __device__ static uint32_t wofs(uint32_t n, uint32_t g) { return P::base(n, g) ^ (16 * (g >> 1)); }
  struct Op {
    uint4 s;
    uint32_t dw, dsh;
    uint64_t q[2][3];
    const uint64_t *x;
    __device__ uint4 sc() const { return s; }
    __device__ float d() const { return h2f(dw >> dsh); }
    __device__ uint64_t w(int v, int k) const { return q[v][k]; }
    __device__ uint64_t xg(int j) const { return x[j]; }
  };
  __device__ static Op load(const uint8_t *ws, const uint64_t *x, uint32_t wo, uint32_t n, uint32_t bi) {
    Op o;
    o.s = *reinterpret_cast<const uint4 *>(ws + 3 * P::BYTES + 32 * n + 16 * bi);
    o.dw = *reinterpret_cast<const uint32_t *>(ws + 3 * P::BYTES + 512 + 4 * n);
    o.dsh = 16 * bi;
#pragma unroll
    for (int v = 0; v < 2; v++)
#pragma unroll
      for (int k = 0; k < 3; k++)
        o.q[v][k] = *reinterpret_cast<const uint64_t *>(ws + P::BYTES * k + (wo ^ (16 * (4 * bi + 2 * v))));
    o.x = x;
    return o;
  }
};

// Q8_0: planes A | B (a block's eight units are 128 bytes per plane), then
// the scales.
struct RQ8 {
  using B = BQ8;
  static constexpr bool PAIRED = false;
  static constexpr bool TILED = false;
  using P = Plane<256>;
  static constexpr uint32_t WB = 2 * P::BYTES + 512;
  static constexpr int NDMA = 2 * P::NDMA + 1;
  static constexpr int NDMA_T = NDMA;
  struct Src {
    uint32_t pl[P::NDMA], hd, U;
  };
  __device__ static Src src(size_t rb, uint32_t n_in, uint32_t row0, uint32_t n_out, uint32_t L) {
    Src s;
    s.U = n_in / 32;
    P::src<2>(rb, row0, n_out, L, s.pl);
    s.hd = pair_piece(rb, row0, n_out, L, 32 * s.U);
    return s;
  }
  __device__ static void issue(const uint8_t *w, const Src &s, uint32_t sp, uint8_t *slot, uint32_t L) {
    P::issue(w, s.pl, 0, sp, slot);
    P::issue(w, s.pl, 16 * s.U, sp, slot + P::BYTES);
    issue_piece(w, s.hd, sp, slot + 2 * P::BYTES, L);
  }
  __device__ static uint32_t wofs(uint32_t n, uint32_t g) { return P::base(n, g) + P::BYTES * (g >> 1); }
  struct Op {
    uint4 s;
    uint64_t q[8];
    const uint64_t *x;
    __device__ uint4 sc() const { return s; }
    __device__ uint64_t w(int i) const { return q[i]; }
    __device__ uint64_t xg(int i) const { return x[i]; }
  };
  __device__ static Op load(const uint8_t *ws, const uint64_t *x, uint32_t wo, uint32_t n, uint32_t bi) {
    Op o;
    o.s = *reinterpret_cast<const uint4 *>(ws + 2 * P::BYTES + 32 * n + 16 * bi);
#pragma unroll
    for (int i = 0; i < 8; i++) o.q[i] = *reinterpret_cast<const uint64_t *>(ws + (wo ^ (16 * (8 * bi + i))));
    o.x = x;
    return o;
  }
};

// Bytes of a slot: per wave (W == 1) or shared by W waves on W tiles.
template <class R, bool GATED, int XN, int W = 1>
constexpr uint32_t ring_slot() {
  return 512 * XN + 256 + W * (GATED ? 2 : 1) * R::WB;
}
constexpr uint32_t RING_LDS_MAX = 160 * 1024;
template <class R, int TW, int W, bool GATED, int XN>
constexpr bool ring_fits() {
  return TW * 2 * ring_slot<R, GATED, XN, W>() <= RING_LDS_MAX;
}

// XN: token rows staged per pair (8 for T <= 8, else 16). Either TW waves
// split one tile's columns (W = 1), or W waves take W consecutive tiles in
// lockstep (TW = 1), sharing the pair's activations and scales: one staged
// copy per workgroup instead of one per tile. SPLIT (gated, W = 2): the two
// waves take the same tile, one gate's rows and one up's, in lockstep on
// the shared activations: twice the waves for the same LDS.
template <class R, int TW, int W, bool GATED, int XN, bool CAP = false, bool SPLIT = false, bool TL = false>
__global__ __launch_bounds__(64 * TW * W) void gemv_ring(BatchSet bs, const int8_t *__restrict__ qx,
                                                         const float *__restrict__ dx, uint32_t T,
                                                         float *__restrict__ ygated) {
  static_assert(W == 1 || TW == 1, "waves split a tile's columns or take tiles of their own");
  static_assert(!SPLIT || (GATED && W == 2 && TW == 1), "gate and up split over a pair of waves");
  using F = typename R::B;
  constexpr int NR = GATED && !SPLIT ? 2 : 1;  // weights per wave
  constexpr uint32_t XB = 512 * XN, WS = NR * R::WB, SLOT = XB + 256 + W * WS;
  static_assert(!TL || (R::TILED && !CAP), "tile images: the formats that have them, no capture");
  constexpr int PB = XN / 2 + 1 + NR * (TL ? R::NDMA_T : R::NDMA);  // DMA instructions per pair (W == 1)
  static_assert(PB <= 63, "wait count beyond vmcnt's range");
  static_assert(TW == 1 || TW * 2 * SLOT >= NCHMAX * NR * 4 * 64 * sizeof(float), "chunk sums fit the ring");
  static_assert(TW * 2 * SLOT <= RING_LDS_MAX, "ring beyond the LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[TW][2][SLOT];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63;
  // W > 1: the last workgroup's waves past the last tile take part in the
  // barriers on the last tile's bytes and store nothing.
  const uint32_t all_tiles = bs.j[0].tiles + (bs.n > 1 ? bs.j[1].tiles : 0) + (bs.n > 2 ? bs.j[2].tiles : 0);
  const uint32_t tile_w = W == 1 || SPLIT ? blockIdx.x : blockIdx.x * W + wave;
  const bool live = tile_w < all_tiles;
  uint32_t tile = live ? tile_w : all_tiles - 1;
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
  const uint32_t n_in = bs.n_in, nb = n_in / 256, n_out = J.n_out;
  const uint32_t nch = nb < NCHMAX ? nb : NCHMAX;
  // Lane l: weight row l%16 and token l%16 of the MFMA operands, k-group l/16.
  const uint32_t n = lane & 15, g = lane >> 4, r_lane = tile * TROWS + n;
  const size_t rb = F::row_bytes(n_in);
  const uint8_t *wbase[NR];
  wbase[0] = SPLIT && wave == 1 ? bs.j[1].w : J.w;
  if (GATED && !SPLIT) wbase[NR - 1] = bs.j[1].w;
  // DMA sources (the same rows of gate and up).
  const typename R::Src src = R::src(rb, n_in, tile * TROWS, n_out, lane);
  // TL: the tile's images instead, IMG bytes per pair (the same tile of
  // gate and up).
  const uint8_t *tbase[NR];
  if constexpr (TL) {
    const size_t timg = (size_t)tile * (nb / 2) * R::IMG;
    tbase[0] = (SPLIT && wave == 1 ? bs.j[1].wt : J.wt) + timg;
    if (GATED && !SPLIT) tbase[NR - 1] = bs.j[1].wt + timg;
  }
  // The activation DMAs this wave issues (W > 1: its share of them).
  constexpr int XD = XN / 2 / W;
  const int xd0 = W == 1 ? 0 : wave * XD;
  uint32_t xsrc[XD];
#pragma unroll
  for (int i = 0; i < XD; i++) {
    const uint32_t t = 2 * (xd0 + i) + (lane >> 5);
    xsrc[i] = min(t, T - 1) * n_in + 16 * ((lane & 31) ^ t);
  }
  const uint32_t ssrc = (min(lane & 15, T - 1) * nb + ((lane >> 4) & 1)) * 4;
  // Operand reads: x of token n (rows past the slot's tokens read its last).
  // Paired formats at most 8 tokens: slots 8..15 read tokens 0..7 again.
  constexpr bool PAIR = R::PAIRED && XN == 8;
  const uint32_t tr = PAIR ? (n & 7) : min(n, (uint32_t)XN - 1);
  const uint32_t xo = 512 * tr + 8 * (g & 1) + 16 * ((g >> 1) ^ tr), wo = R::wofs(n, g);
  const int rw = W == 1 ? wave : 0;                    // the wave's ring
  const uint32_t wofs_w = XB + 256 + (W == 1 ? 0 : wave * WS);  // its weights in a slot
  auto issue = [&](int s, uint32_t sp) {
    uint8_t *sl = ring[rw][s];
#pragma unroll
    for (int i = 0; i < XD; i++) lds_dma16(qx, xsrc[i] + 512 * sp, sl + 1024 * (xd0 + i));
    if (W == 1 || wave == 0) lds_dma4(dx, ssrc + 8 * sp, sl + XB);
#pragma unroll
    for (int r = 0; r < NR; r++) {
      if constexpr (TL)
        R::issue_tile(tbase[r], sp * R::IMG + 16 * lane, sl + wofs_w + r * R::WB, lane);
      else
        R::issue(wbase[r], src, sp, sl + wofs_w + r * R::WB, lane);
    }
  };
  constexpr int NJ = 4;
  float acc[NR][NJ], tot[NR][NJ];
  // Sums of this wave's finished chunks (waves > 0; wave 0 adds its own to
  // tot as they finish).
  constexpr int CPW = TW > 1 ? (NCHMAX + TW - 1) / TW : 1;
  float part[CPW][NR][NJ];
#pragma unroll
  for (int r = 0; r < NR; r++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[r][j] = tot[r][j] = 0.f;
  const uint32_t nsub = n_in / (256 / F::SUBS);
  int32_t *dcap[NR];
  dcap[0] = SPLIT && wave == 1 ? bs.j[1].dots : J.dots;
  if (GATED && !SPLIT) dcap[NR - 1] = bs.j[1].dots;
  const int ks = W == 1 ? wave : 0;  // the wave's share of the columns
  const uint32_t c0 = ks * nch / TW, c1 = (ks + 1) * nch / TW;
  const uint32_t b0 = c0 * nb / nch, b1 = c1 * nb / nch;
  uint32_t ch = c0, ch_end = (c0 + 1) * nb / nch;
  auto chunk_done = [&](uint32_t b) {
    if (b + 1 == ch_end) {
      if (ks == 0) {
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
          for (int j = 0; j < NJ; j++) tot[r][j] += acc[r][j];
      } else {
        const uint32_t k = ch - c0;
#pragma unroll
        for (int kk = 0; kk < CPW; kk++)
          if (k == (uint32_t)kk)
#pragma unroll
            for (int r = 0; r < NR; r++)
#pragma unroll
              for (int j = 0; j < NJ; j++) part[kk][r][j] = acc[r][j];
      }
#pragma unroll
      for (int r = 0; r < NR; r++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[r][j] = 0.f;
      ch++;
      ch_end = (ch + 1) * nb / nch;
    }
  };
  // Blocks 2sp + bi of the slot that are the wave's, in order. Every
  // operand of the pair is read first (both blocks, every weight), so the
  // reads overlap instead of each block waiting for its own.
  auto use = [&](int s, uint32_t sp) {
    const uint8_t *sl = ring[rw][s];
    uint64_t xv[2][8];
    float4 sv[2];
    typename R::Op op[2][NR];
#pragma unroll
    for (int bi = 0; bi < 2; bi++) {
      sv[bi] = *reinterpret_cast<const float4 *>(sl + XB + 64 * bi + 16 * g);
#pragma unroll
      for (int j = 0; j < 8; j++) xv[bi][j] = *reinterpret_cast<const uint64_t *>(sl + (xo ^ (32 * (8 * bi + j))));
#pragma unroll
      for (int r = 0; r < NR; r++) op[bi][r] = R::load(sl + wofs_w + r * R::WB, xv[bi], wo, n, bi);
    }
#pragma unroll
    for (int bi = 0; bi < 2; bi++) {
      const uint32_t bb = 2 * sp + bi;
      if (bb < b0 || bb >= b1) continue;
      const float sj[NJ] = {sv[bi].x, sv[bi].y, sv[bi].z, sv[bi].w};
#pragma unroll
      for (int r = 0; r < NR; r++) {
        float c[NJ];
        Dots dc{nullptr, (size_t)n_out * nsub, T};
        if constexpr (CAP) {
          if (live && r_lane < n_out) dc.p = dcap[r] + (size_t)r_lane * nsub + F::SUBS * bb;
        }
        if constexpr (PAIR)
          F::compute_paired(op[bi][r], c, dc, g, n);
        else
          F::compute(op[bi][r], c, dc, g);
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[r][j] = fmaf(sj[j], c[j], acc[r][j]);
      }
      chunk_done(bb);
    }
  };
  const uint32_t s0 = b0 >> 1, s1 = (b1 + 1) >> 1;
  issue(0, s0);
  if constexpr (W == 1) {
    // The pairs holding the wave's blocks; a pair past its last is loaded
    // as its last again (in bounds; every pair issues the same DMAs, so the
    // wait count is fixed). (A third slot, two pairs in flight, measured
    // slower at every shape: the 4096x14336 Q6_K at 8 tokens 15.2 -> 16.2
    // us.)
    for (uint32_t sp = s0; sp < s1; sp += 2) {
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t cur = sp + i;
        if (cur >= s1) break;
        // The slot refilled now was read by the previous pair: its reads
        // are complete before the DMAs overwrite it.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(i ^ 1, min(cur + 1, s1 - 1));
        // Pair cur's DMAs done: only the pair issued after it remains.
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PB) : "memory");
        use(i, cur);
      }
    }
    lds_wait_dma();  // the repeated last pair lands before the ring is reused
  } else {
    // Lockstep over every pair (all waves run the same count): each waits
    // for its own DMAs of pair cur, the barrier publishes them all and
    // retires every read of the other slot, then the next pair is issued
    // into it and pair cur computed.
    for (uint32_t sp = s0; sp < s1; sp += 2) {
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t cur = sp + i;
        if (cur >= s1) break;
        lds_wait_dma();
        lds_barrier();
        if (cur + 1 < s1) issue(i ^ 1, cur + 1);
        use(i, cur);
      }
    }
  }
  if constexpr (TW > 1) {
    // Chunk sums of waves > 0 through the (now idle) ring, added by wave 0
    // in chunk order.
    float *red = reinterpret_cast<float *>(&ring[0][0][0]);  // [chunk][r][j][lane]
    __syncthreads();
    if (wave > 0) {
#pragma unroll
      for (int kk = 0; kk < CPW; kk++)
        if (c0 + kk < c1)
#pragma unroll
          for (int r = 0; r < NR; r++)
#pragma unroll
            for (int j = 0; j < NJ; j++) red[(((c0 + kk) * NR + r) * NJ + j) * 64 + lane] = part[kk][r][j];
    }
    __syncthreads();
    if (wave > 0) return;
    for (uint32_t k = c1; k < nch; k++)
#pragma unroll
      for (int r = 0; r < NR; r++)
#pragma unroll
        for (int j = 0; j < NJ; j++) tot[r][j] += red[((k * NR + r) * NJ + j) * 64 + lane];
  }
  float uv_split[NJ] = {};
  if constexpr (SPLIT) {
    // Up's sums (wave 1) to gate's wave through the idle ring.
    float *red = reinterpret_cast<float *>(&ring[0][0][0]);  // [j][lane]
    __syncthreads();
    if (wave == 1)
#pragma unroll
      for (int j = 0; j < NJ; j++) red[j * 64 + lane] = tot[0][j];
    __syncthreads();
    if (wave == 1) return;
#pragma unroll
    for (int j = 0; j < NJ; j++) uv_split[j] = red[j * 64 + lane];
  }
  if (!live || r_lane >= n_out) return;
  const uint32_t t0 = 4 * g;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    if (t0 + j >= T) continue;
    if (GATED) {
      const float gv = tot[0][j], uv = SPLIT ? uv_split[j] : tot[NR - 1][j];
      ygated[(size_t)(t0 + j) * n_out + r_lane] = gv / (1.0f + expf(-gv)) * uv;
    } else {
      J.y[(size_t)(t0 + j) * n_out + r_lane] = tot[0][j];
    }
  }
}

struct RingShape {
  uint32_t tw, w;
};
template <class R, bool GATED, int XN>
RingShape ring_shape(mdma_ctx *ctx, uint32_t tiles, uint32_t nch) {
  // Many tiles (at least 1.5 workgroups per CU of 4): 4 tiles per
  // workgroup share the activations (the 128256-row head: 101.7 us against
  // 113.7 us with a tile per workgroup; 896 tiles two per workgroup measured
  // slower than one, 24.4 us against 18.5 us: the lockstep costs more than
  // the activations it saves there). Otherwise waves per tile: up to 4 (at
  // most one per chunk) while the launch keeps to about one wave per SIMD
  // (4 per CU): more waves splitting the same tiles measured slower (896
  // tiles: one wave each 19.1 us, two 21.0 us; 256 tiles of 56 blocks: four
  // waves each 18.1 us, one 40.7 us).
  const uint64_t cus = ctx->cu_count;
  if (ring_fits<R, 1, 4, GATED, XN>() && (uint64_t)tiles * 2 >= 4 * 3 * cus) return {1, 4};
  uint32_t tw = 1;
  while (tw < 4 && 2 * tw <= nch && (uint64_t)tiles * 2 * tw <= cus * 4 &&
         2 * tw * 2 * ring_slot<R, GATED, XN>() <= RING_LDS_MAX)
    tw *= 2;
  return {tw, 1};
}

template <class R, int TW, int W, bool GATED, int XN, bool SPLIT = false, bool TL = false>
void ring_launch(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, const int8_t *qx, const float *dx, uint32_t T,
                 float *yg) {
  hipEvent_t t0 = ctx->time_start, t1 = ctx->time_stop;
  ctx->time_start = ctx->time_stop = nullptr;
  const dim3 grid(SPLIT ? tiles : (tiles + W - 1) / W), block(64 * TW * W);
  if (bs.j[0].dots) {
    // ring_fmt sized the shape for the 16 token rows the capture stages.
    if constexpr (SPLIT || ring_fits<R, TW, W, GATED, 16>())
      gemv_ring<R, TW, W, GATED, 16, true, SPLIT><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
  } else if (t0 || t1) {
    hipExtLaunchKernelGGL(gemv_ring<R, TW, W, GATED, XN, false, SPLIT, TL>, grid, block, 0, ctx->stream, t0, t1, 0, bs,
                          qx, dx, T, yg);
  } else {
    gemv_ring<R, TW, W, GATED, XN, false, SPLIT, TL><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
  }
  hip_check(hipGetLastError(), "gemv ring launch");
}

template <class R, bool GATED, int XN, bool TL>
void ring_fmt(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, const int8_t *qx, const float *dx, uint32_t T,
              float *yg) {
  const uint32_t nb = bs.n_in / 256, nch = nb < NCHMAX ? nb : NCHMAX;
  // The capture instantiation stages 16 token rows (any T): shape it for that.
  const RingShape sh = bs.j[0].dots ? ring_shape<R, GATED, 16>(ctx, tiles, nch) : ring_shape<R, GATED, XN>(ctx, tiles, nch);
  // (ring_shape only picks shapes whose ring fits; the guards keep the
  // instantiations that would not out of the build.)
  if (sh.w == 4) {
    if constexpr (ring_fits<R, 1, 4, GATED, XN>()) return ring_launch<R, 1, 4, GATED, XN, false, TL>(ctx, bs, tiles, qx, dx, T, yg);
  } else if (GATED && sh.tw == 1) {
    // One wave per tile would hold gate and up alone: split them over a
    // pair (the same LDS as gate and up in one wave).
    if constexpr (GATED) return ring_launch<R, 1, 2, GATED, XN, true, TL>(ctx, bs, tiles, qx, dx, T, yg);
  } else if (sh.tw == 4) {
    if constexpr (ring_fits<R, 4, 1, GATED, XN>()) return ring_launch<R, 4, 1, GATED, XN, false, TL>(ctx, bs, tiles, qx, dx, T, yg);
  } else if (sh.tw == 2) {
    if constexpr (ring_fits<R, 2, 1, GATED, XN>()) return ring_launch<R, 2, 1, GATED, XN, false, TL>(ctx, bs, tiles, qx, dx, T, yg);
  }
  ring_launch<R, 1, 1, GATED, XN, false, TL>(ctx, bs, tiles, qx, dx, T, yg);
}

template <class R, bool TL>
void ring_dispatch_tl(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, bool gated, const int8_t *qx, const float *dx,
                      uint32_t T, float *yg) {
  if (gated) {
    if (T <= 8) ring_fmt<R, true, 8, TL>(ctx, bs, tiles, qx, dx, T, yg);
    else ring_fmt<R, true, 16, TL>(ctx, bs, tiles, qx, dx, T, yg);
  } else {
    if (T <= 8) ring_fmt<R, false, 8, TL>(ctx, bs, tiles, qx, dx, T, yg);
    else ring_fmt<R, false, 16, TL>(ctx, bs, tiles, qx, dx, T, yg);
  }
}
// tl: every job's tile image is there (formats that have one).
template <class R>
void ring_dispatch(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, bool gated, bool tl, const int8_t *qx,
                   const float *dx, uint32_t T, float *yg) {
  if constexpr (R::TILED) {
    if (tl && !bs.j[0].dots) return ring_dispatch_tl<R, true>(ctx, bs, tiles, gated, qx, dx, T, yg);
  }
  ring_dispatch_tl<R, false>(ctx, bs, tiles, gated, qx, dx, T, yg);
}

// The Q6_K tile images of a prepared weight: for tile t (rows 16t..16t+15,
// rows past the last repeating it, as the ring's clamped row-plane DMAs
// read them) and block pair s, RQ6::IMG bytes at (t * pairs + s) * IMG
// holding what RQ6::issue places in a slot: per plane (A, B, high bits)
// byte 1024k + 16L is chunk ((L % 8) ^ (r / 2)) of row r = 8k + L / 8's 128
// bytes of the pair, then byte 16L (L < 32) of the scale piece is row L / 2's
// 16 scale bytes of block 2s + L % 2, then row n's d word (the f16 d of
// blocks 2s and 2s + 1) at 4n. One thread per 16 bytes of image.
__global__ __launch_bounds__(256) void tile_repack_q6_kernel(const uint8_t *__restrict__ w, uint8_t *__restrict__ out,
                                                             uint32_t n_out, uint32_t n_in, uint64_t chunks) {
  constexpr uint32_t CPI = RQ6::IMG / 16;  // 16-byte chunks per image
  const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= chunks) return;
  const uint32_t pairs = n_in / 512, U = n_in / 64, c = (uint32_t)(idx % CPI);
  const uint64_t img = idx / CPI;
  const uint32_t t = (uint32_t)(img / pairs), sp = (uint32_t)(img % pairs);
  const size_t rb = BQ6::row_bytes(n_in);
  auto row = [&](uint32_t r) { return w + (size_t)min(16 * t + r, n_out - 1) * rb; };
  uint4 v;
  if (c < 3 * 128) {
    const uint32_t pl = c / 128, k = (c % 128) / 64, L = c % 64, r = 8 * k + L / 8;
    v = *reinterpret_cast<const uint4 *>(row(r) + 16 * U * pl + 128 * sp + 16 * ((L % 8) ^ (r / 2)));
  } else if (c < 3 * 128 + 32) {
    const uint32_t L = c - 3 * 128;
    v = *reinterpret_cast<const uint4 *>(row(L >> 1) + 48 * U + 32 * sp + 16 * (L & 1));
  } else {
    const uint32_t j = c - (3 * 128 + 32);  // rows 4j..4j+3
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; q++) d[q] = *reinterpret_cast<const uint32_t *>(row(4 * j + q) + 52 * U + 4 * sp);
    v = make_uint4(d[0], d[1], d[2], d[3]);
  }
  *reinterpret_cast<uint4 *>(out + 16 * idx) = v;
}

}  // namespace

uint64_t batch_tile_bytes(int32_t dtype, uint64_t n_out, uint64_t n_in) {
  if (dtype != DT_Q6_K || !n_out || !n_in || n_in % 512) return 0;
  return (n_out + TROWS - 1) / TROWS * (n_in / 512) * RQ6::IMG;
}

void launch_tile_repack(mdma_ctx *ctx, int32_t dtype, uint64_t n_out, uint64_t n_in, const uint8_t *w,
                        uint8_t *out) {
  const uint64_t chunks = batch_tile_bytes(dtype, n_out, n_in) / 16;
  if (!chunks) return;
  tile_repack_q6_kernel<<<dim3((uint32_t)((chunks + 255) / 256)), dim3(256), 0, ctx->stream>>>(
      w, out, (uint32_t)n_out, (uint32_t)n_in, chunks);
  hip_check(hipGetLastError(), "tile repack launch");
}

// Prepared-layout row bytes (the formats' row_bytes, on the host).
static uint64_t batch_row_bytes(int32_t dt, uint64_t n_in) {
  if (dt == DT_Q4_K) return n_in / 256 * 144;
  if (dt == DT_Q6_K) return (n_in / 256 * 210 + 15) / 16 * 16;
  return (n_in / 32 * 34 + 15) / 16 * 16;
}

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
    bs.j[i].wt = nullptr;
    bs.j[i].y = jobs[i].y;
    bs.j[i].dots = jobs[i].dots;
    bs.j[i].n_out = (uint32_t)jobs[i].n_out;
    bs.j[i].tiles = (uint32_t)((jobs[i].n_out + TROWS - 1) / TROWS);
    if (i < bs.n) tiles += bs.j[i].tiles;
  }
  if (!tiles) return;
  const uint32_t t = (uint32_t)T;
  const int32_t dt = jobs[0].dtype;
  // The ring kernel addresses a weight with 32-bit offsets.
  // (and pairs of 256-column blocks).
  bool ring = ctx->batch_kernel == MDMA_BATCH_AUTO && (n_in / 256) % 2 == 0;
  for (int i = 0; i < (gated ? 2 : n_jobs); i++)
    ring = ring && jobs[i].n_out * batch_row_bytes(dt, n_in) < (1ull << 32);
  if (ring) {
    // Q6_K weights' tile images (made here at a weight's first such call
    // when the context asks for them): contiguous DMA per pair instead of
    // 128-byte row pieces (the 4096x14336 Q6_K at 8 tokens 15.3 -> 12.6 us).
    bool tl = dt == DT_Q6_K && !jobs[0].dots;
    for (int i = 0; tl && i < (gated ? 2 : n_jobs); i++) {
      bs.j[i].wt = batch_tile(ctx, jobs[i]);
      tl = bs.j[i].wt != nullptr;
    }
    if (dt == DT_Q4_K) ring_dispatch<RQ4>(ctx, bs, tiles, gated, false, qx, dx, t, ygated);
    else if (dt == DT_Q6_K) ring_dispatch<RQ6>(ctx, bs, tiles, gated, tl, qx, dx, t, ygated);
    else ring_dispatch<RQ8>(ctx, bs, tiles, gated, false, qx, dx, t, ygated);
    return;
  }
  if (dt == DT_Q4_K) launch_fmt<BQ4>(ctx, bs, tiles, gated, qx, dx, t, ygated);
  else if (dt == DT_Q6_K) launch_fmt<BQ6>(ctx, bs, tiles, gated, qx, dx, t, ygated);
  else launch_fmt<BQ8>(ctx, bs, tiles, gated, qx, dx, t, ygated);
}

}  // namespace mdma
