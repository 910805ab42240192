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
//    then times the token's per-256 activation scale, accumulated in f64.
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
__device__ __forceinline__ uint32_t ldw2(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }
__device__ __forceinline__ v4i mma(uint64_t x, uint64_t w, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x, (long)w, c, 0, 0, 0);
}

// Activation bytes of the lane's token at column col (zero rows past T).
struct XRow {
  const int8_t *p;
  __device__ uint64_t operator()(uint32_t col) const {
    return p ? *reinterpret_cast<const uint64_t *>(p + col) : 0ull;
  }
};

// Each format: W = the weight bytes of one row's 256-column block for the
// lane, X = the lane's activation bytes for that block; load / loadx issue
// the loads, compute turns them into the block's contributions c[j]
// (before the activation scale) for the lane's row and tokens.

// Q4_K: unit u = 64 columns, 32 quant bytes (16 in plane A, 16 in plane B);
// lane group g takes bytes 8g..8g+7 of A|B: low nibbles are columns
// 64u + 8g + [0,8) (sub-block 2(u%4)), high nibbles 64u + 32 + 8g + [0,8).
struct BQ4 {
  static constexpr uint32_t UCOLS = 64;
  __device__ static size_t row_bytes(uint32_t n_in) { return (size_t)(n_in / 256) * 144; }
  struct W {
    uint4 h;
    uint64_t q[4];
  };
  struct X {
    uint64_t lo[4], hi[4];
  };
  __device__ static void load(const uint8_t *row, uint32_t U, uint32_t b, uint32_t g, W &w) {
    const uint8_t *plane = row + (g < 2 ? 0 : 16 * (size_t)U) + 8 * (g & 1);
#pragma unroll
    for (int p = 0; p < 4; p++) w.q[p] = ldw8(plane + 16 * (size_t)(4 * b + p));
    w.h = *reinterpret_cast<const uint4 *>(row + 32 * (size_t)U + 16 * (size_t)b);
  }
  __device__ static void loadx(const XRow &xr, uint32_t b, uint32_t g, X &x) {
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const uint32_t col = 256 * b + 64 * p + 8 * g;
      x.lo[p] = xr(col);
      x.hi[p] = xr(col + 32);
    }
  }
  __device__ static void compute(const W &w, const X &x, uint32_t, double *c) {
    constexpr uint64_t M4 = 0x0F0F0F0F0F0F0F0Full, ONES = 0x0101010101010101ull;
    v4i ai = {}, dm = {};
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const v4i z = {};
      const v4i da = mma(x.lo[p], w.q[p] & M4, z);
      const v4i db = mma(x.hi[p], (w.q[p] >> 4) & M4, z);
      int sca, scb, ma, mb;
      q4k_scales_i(w.h, p, sca, scb, ma, mb);
      // 24-bit multiplies (full rate): |isum| <= 15*127*32.
#pragma unroll
      for (int j = 0; j < 4; j++) ai[j] += __mul24(sca, da[j]) + __mul24(scb, db[j]);
      dm = mma(x.lo[p], (uint64_t)ma * ONES, dm);
      dm = mma(x.hi[p], (uint64_t)mb * ONES, dm);
    }
    const double d = (double)h2f(w.h.x), dmin = (double)h2f(w.h.x >> 16);
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = d * (double)ai[j] - dmin * (double)dm[j];
  }
};

// Q6_K: unit u = (half n, group column h) of block u/4, quarters r = 0..3
// of 16 columns each (col below), one int8 scale per quarter. Lanes g and
// g+2 (g = 0,1) hold dwords 2g, 2g+1 of the A, B and high-bit planes of
// units 2v and 2v+1: columns col(u, r) + 8g + [0,8).
struct BQ6 {
  static constexpr uint32_t UCOLS = 64;
  __device__ static size_t row_bytes(uint32_t n_in) { return ((size_t)(n_in / 256) * 210 + 15) / 16 * 16; }
  __device__ static uint32_t u6(uint32_t a, uint32_t b, uint32_t h, int r) {
    switch (r) {
      case 0: return (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
      case 1: return (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
      case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
      default: return ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
    }
  }
  // Bytes u6 (0..63) to the signed int8 u6 - 32.
  __device__ static uint32_t centred(uint32_t v) {
    const uint32_t s = ~v & 0x20202020u;
    return (v ^ 0x20202020u) | (s << 1) | (s << 2);
  }
  __device__ static uint32_t col(uint32_t u, int r) {
    return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * r + 16 * (u & 1);
  }
  struct W {
    uint64_t a[2], b[2], q[2];
    uint32_t sc[2][2];
    uint32_t d;
  };
  struct X {
    uint64_t q[2][4];  // [unit pair][quarter]
  };
  __device__ static void load(const uint8_t *row, uint32_t U, uint32_t b, uint32_t g, W &w) {
#pragma unroll
    for (int v = 0; v < 2; v++) {
      const uint32_t u = 4 * b + 2 * v + (g >> 1);
      const size_t o = 16 * (size_t)u + 8 * (g & 1);
      w.a[v] = ldw8(row + o);
      w.b[v] = ldw8(row + 16 * (size_t)U + o);
      w.q[v] = ldw8(row + 32 * (size_t)U + o);
      // Scales of both units of the pair (each lane pair multiplies by its own).
      w.sc[v][0] = ldw4(row + 48 * (size_t)U + 4 * (size_t)(4 * b + 2 * v));
      w.sc[v][1] = ldw4(row + 48 * (size_t)U + 4 * (size_t)(4 * b + 2 * v + 1));
    }
    w.d = ldw2(row + 52 * (size_t)U + 2 * (size_t)b);
  }
  __device__ static void loadx(const XRow &xr, uint32_t b, uint32_t g, X &x) {
#pragma unroll
    for (int v = 0; v < 2; v++)
#pragma unroll
      for (int r = 0; r < 4; r++) x.q[v][r] = xr(col(4 * b + 2 * v + (g >> 1), r) + 8 * (g & 1));
  }
  __device__ static void compute(const W &w, const X &x, uint32_t g, double *c) {
    v4i ai = {};
#pragma unroll
    for (int v = 0; v < 2; v++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t lo = centred(u6((uint32_t)w.a[v], (uint32_t)w.b[v], (uint32_t)w.q[v], r));
        const uint32_t hi =
            centred(u6((uint32_t)(w.a[v] >> 32), (uint32_t)(w.b[v] >> 32), (uint32_t)(w.q[v] >> 32), r));
        const uint64_t wv = (uint64_t)lo | ((uint64_t)hi << 32);
        // Unit 2v: lanes g < 2; unit 2v+1: lanes g >= 2.
        const v4i z = {};
        const v4i d0 = mma(g < 2 ? x.q[v][r] : 0ull, wv, z);
        const v4i d1 = mma(g < 2 ? 0ull : x.q[v][r], wv, z);
        const int s0 = (int)(int8_t)((w.sc[v][0] >> (8 * r)) & 0xff);
        const int s1 = (int)(int8_t)((w.sc[v][1] >> (8 * r)) & 0xff);
        // 24-bit multiplies (full rate): |isum| <= 32*127*16.
#pragma unroll
        for (int j = 0; j < 4; j++) ai[j] += __mul24(s0, d0[j]) + __mul24(s1, d1[j]);
      }
    }
    const double d = (double)h2f(w.d);
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = d * (double)ai[j];
  }
};

// Q8_0: 32-column blocks (U = n_in/32 units), 16 bytes in plane A and 16 in
// plane B; lane group g takes bytes 8g..8g+7 of A|B = columns 32u + 8g + [0,8).
struct BQ8 {
  static constexpr uint32_t UCOLS = 32;
  __device__ static size_t row_bytes(uint32_t n_in) { return ((size_t)(n_in / 32) * 34 + 15) / 16 * 16; }
  struct W {
    uint64_t q[8];
    uint32_t d[8];
  };
  struct X {
    uint64_t q[8];
  };
  __device__ static void load(const uint8_t *row, uint32_t U, uint32_t b, uint32_t g, W &w) {
    const uint8_t *plane = row + (g < 2 ? 0 : 16 * (size_t)U) + 8 * (g & 1);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      w.q[i] = ldw8(plane + 16 * (size_t)(8 * b + i));
      w.d[i] = ldw2(row + 32 * (size_t)U + 2 * (size_t)(8 * b + i));
    }
  }
  __device__ static void loadx(const XRow &xr, uint32_t b, uint32_t g, X &x) {
#pragma unroll
    for (int i = 0; i < 8; i++) x.q[i] = xr(256 * b + 32 * i + 8 * g);
  }
  __device__ static void compute(const W &w, const X &x, uint32_t, double *c) {
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = 0.0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const v4i z = {};
      const v4i dq = mma(x.q[i], w.q[i], z);
      const double d = (double)h2f(w.d[i]);
#pragma unroll
      for (int j = 0; j < 4; j++) c[j] = fma(d, (double)dq[j], c[j]);
    }
  }
};

struct BatchJob {
  const uint8_t *w;
  float *y;
  uint32_t n_out, tiles;
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
template <class F, int TW, bool GATED>
__global__ __launch_bounds__(64 * TW) void gemv_batch(BatchSet bs, const int8_t *__restrict__ qx,
                                                      const float *__restrict__ dx, uint32_t T,
                                                      float *__restrict__ ygated) {
  constexpr int NR = GATED ? 2 : 1;
  __shared__ double red[TW > 1 ? NCHMAX : 1][NR][4][64];
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
  const uint32_t row = min(r_lane, n_out - 1);  // rows past the end re-read the last row, not stored
  const size_t rb = F::row_bytes(n_in);
  const uint8_t *wrow[NR];
  wrow[0] = J.w + row * rb;
  if (GATED) wrow[NR - 1] = bs.j[1].w + row * rb;
  const uint32_t tok = lane & 15;
  const XRow xr{tok < T ? qx + (size_t)tok * n_in : nullptr};
  // Token of result slot j.
  constexpr int NJ = 4;
  uint32_t tj[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) tj[j] = 4 * (lane >> 4) + j;
  double acc[NR][NJ], tot[NR][NJ];
  // Ping-pong slots: the next block's loads go out before a block is
  // computed (clamped to the wave's last block, so every load is in bounds
  // and the wait counts are fixed).
  struct Slot {
    typename F::X x;
    typename F::W w[NR];
    float s[NJ];
  };
  auto fill = [&](Slot &sl, uint32_t b) {
#pragma unroll
    for (int r = 0; r < NR; r++) F::load(wrow[r], U, b, g, sl.w[r]);
    F::loadx(xr, b, g, sl.x);
#pragma unroll
    for (int j = 0; j < NJ; j++) sl.s[j] = tj[j] < T ? dx[(size_t)tj[j] * nb + b] : 0.f;
  };
  auto use = [&](const Slot &sl) {
#pragma unroll
    for (int r = 0; r < NR; r++) {
      double c[NJ];
      F::compute(sl.w[r], sl.x, g, c);
#pragma unroll
      for (int j = 0; j < NJ; j++) acc[r][j] = fma((double)sl.s[j], c[j], acc[r][j]);
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
  if (b0 < b1) {
    Slot sa, sb;
    fill(sa, b0);
    for (uint32_t b = b0; b < b1; b += 2) {
      fill(sb, min(b + 1, b1 - 1));
      use(sa);
      chunk_done(b);
      if (b + 1 >= b1) break;
      fill(sa, min(b + 2, b1 - 1));
      use(sb);
      chunk_done(b + 1);
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

template <class F, int TW>
void launch_tw(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, bool gated, const int8_t *qx, const float *dx,
               uint32_t T, float *yg) {
  hipEvent_t t0 = ctx->time_start, t1 = ctx->time_stop;
  ctx->time_start = ctx->time_stop = nullptr;
  const dim3 grid(tiles), block(64 * TW);
  if (gated) {
    if (t0 || t1)
      hipExtLaunchKernelGGL(gemv_batch<F, TW, true>, grid, block, 0, ctx->stream, t0, t1, 0, bs, qx, dx, T, yg);
    else
      gemv_batch<F, TW, true><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
  } else {
    if (t0 || t1)
      hipExtLaunchKernelGGL(gemv_batch<F, TW, false>, grid, block, 0, ctx->stream, t0, t1, 0, bs, qx, dx, T,
                            yg);
    else
      gemv_batch<F, TW, false><<<grid, block, 0, ctx->stream>>>(bs, qx, dx, T, yg);
  }
  hip_check(hipGetLastError(), "gemv batch launch");
}

template <class F>
void launch_fmt(mdma_ctx *ctx, const BatchSet &bs, uint32_t tiles, bool gated, const int8_t *qx, const float *dx,
                uint32_t T, float *yg) {
  // Waves per tile: enough for about 8 waves per CU, at most one per chunk.
  const uint32_t nb = bs.n_in / 256, nch = nb < NCHMAX ? nb : NCHMAX;
  uint32_t tw = 1;
  while (tw < 8 && 2 * tw <= nch && (uint64_t)tiles * tw < (uint64_t)ctx->cu_count * 8) tw *= 2;
  switch (tw) {
    case 1: launch_tw<F, 1>(ctx, bs, tiles, gated, qx, dx, T, yg); break;
    case 2: launch_tw<F, 2>(ctx, bs, tiles, gated, qx, dx, T, yg); break;
    case 4: launch_tw<F, 4>(ctx, bs, tiles, gated, qx, dx, T, yg); break;
    default: launch_tw<F, 8>(ctx, bs, tiles, gated, qx, dx, T, yg); break;
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
