// Prefill GEMM on gfx950: int8 MFMA over Q8_0 / Q4_K / Q6_K weights in the
// prepared layout, activations quantized per 32 to int8 with an f32 scale.
//
// Y[m, n] = sum_k X[m, k] * deq(W)[n, k]   (reference HipBackend::qmatmul_i8,
// /root/reference/src/backend/rocm.rs:1759-1918, the WMMA prefill of
// src/backend/rocm/kernels/kernels.hip:1158-2806; CPU oracle
// src/backend/cpu.rs:335-368 on the requantized activations)
//
// Each 32-wide K block is one v_mfma_i32_32x32x32_i8 per 32x32 output tile
// (Q6_K: two v_mfma_i32_32x32x16_i8, one per 16-column sub-block, whose
// int8 scales differ): the exact int32 block dots of int8 weights and int8
// activations. The epilogue applies that block's scales in f32 over the
// stage's four blocks and adds each stage's partial into an f64 total, so
// outputs that cancel across K keep their accuracy while the per-block work
// stays f32:
//   Q8_0: part += (s_x[m] * d_w[n]) * I
//   Q4_K: part += (s_x[m] * d*sc[n]) * I - (dmin*m[n]) * (s_x[m] * sum_k qx[m, k])
//   Q6_K: part += s_x[m] * (sc_lo[n] * I_lo + sc_hi[n] * I_hi)   (exact int32)
//   per stage: acc += part (Q6_K: acc += d[n] * part; a stage is 128 columns
//   of one super-block, so d is constant over it)
// Weights are unpacked to int8 (Q4_K nibbles 0..15, Q6_K values centred to
// -32..31) in LDS with their block scales; activation rows and their scales
// are staged beside them.
//
// Tiling: a 256-thread workgroup computes a 64x128 tile of Y; each of its 4
// waves owns 32x64 (1x2 MFMA tiles). K advances 128 columns (4 blocks) per
// stage; the next stage's global loads are in registers while the current
// stage computes. LDS rows of 32 bytes are padded to 48 so that the 16-byte
// operand reads of 16 lanes hit all 64 banks once.
#include <hip/hip_ext.h>

#include "kernels.h"

namespace mdma {
namespace {

constexpr int BM = 64, BN = 128, BK = 128, KB = BK / 32, LDR = 48;
// Token tiles walked per column tile in the XCD-aware tile order.
#ifndef MDMA_I8_GT
#define MDMA_I8_GT 16
#endif

// Q6_K: the 6-bit values of quarter r (0..3) of a unit from its ql bytes a
// (quarters 0, 2), b (quarters 1, 3) and qh bytes h, four per dword, and
// those values (0..63) as signed int8 v - 32.
__device__ __forceinline__ uint32_t q6_bytes(uint32_t a, uint32_t b, uint32_t h, int r) {
  switch (r) {
    case 0: return (a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
    case 1: return (b & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
    case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
    default: return ((b >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
  }
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const int8_t *qx;    // [M, K] int8
  const float *sx;     // [M, K/32] per-32 activation scales
  const int32_t *s16;  // [M, K/16] exact sums of 16 activations
  const uint8_t *w;    // prepared rows, row_bytes apart
  float *y;            // [M, N]
  double *part;        // split-K: [tile][split][BM*BN] partial sums
  uint32_t *cnt;       // split-K: one zeroed arrival counter per tile
  uint32_t M, N, K;
  uint32_t ks;         // columns per split (a multiple of BK)
  uint64_t row_bytes;
  int32_t *dots;       // block-dot capture [M, N, n_sub] or null
};

// CAP: the block-dot capture instantiation (GemmArgs::dots set).
template <int DT, bool CAP = false>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) int8_t xs[KB][BM][LDR];
  __shared__ __attribute__((aligned(16))) int8_t ws[KB][BN][LDR];
  __shared__ __attribute__((aligned(16))) float sxs[KB][BM];   // s_x
  __shared__ __attribute__((aligned(16))) float sws[KB][BN];   // d_w (Q8_0) or d*sc (Q4_K)
  __shared__ __attribute__((aligned(16))) float sbs[KB][BM];   // Q4_K: s_x * sum of the block's 32 activations
  __shared__ __attribute__((aligned(16))) float dms[KB][BN];   // Q4_K: dmin*m
  __shared__ __attribute__((aligned(16))) int2 s6[KB][BN];      // Q6_K: the two 16-column scales
  __shared__ __attribute__((aligned(16))) float d6[BN];         // Q6_K: d

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const GridTile tl = grid_tile(MDMA_I8_GT);
  const uint32_t bm = tl.y * BM, bn = tl.x * BN;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 64;
  const uint32_t K = a.K, nk32 = K / 32;
  // This workgroup's columns: split blockIdx.z of the K range.
  const uint32_t kbeg = blockIdx.z * a.ks, kend = min(kbeg + a.ks, K);

  // Per-thread byte offsets of the rows this thread stages, fixed over the
  // K loop (32-bit: the launcher keeps X and W below 2^31 / 2^32 bytes);
  // each stage adds its own uniform column offset.
  uint32_t xo[2], wo[4] = {0, 0, 0, 0}, ho = 0, so;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int c = tid + 256 * i, row = c >> 3, part = c & 7;
    xo[i] = min(bm + row, a.M - 1) * K + 16 * part;
  }
  so = min(bm + (tid >> 2), a.M - 1) * nk32 + (tid & 3);  // sx index; Q4_K s16 index = 2*so
  {
    const uint32_t rb = (uint32_t)a.row_bytes;
    if (DT == DT_Q8_0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int c = tid + 256 * i, row = c >> 3, blk = (c >> 1) & 3, half = c & 1;
        wo[i] = min(bn + row, a.N - 1) * rb + 16 * ((half ? nk32 : 0) + blk);
      }
      ho = min(bn + (tid >> 1), a.N - 1) * rb + 32 * nk32 + 4 * (tid & 1);
    } else if (DT == DT_Q6_K) {
      wo[0] = min(bn + (tid >> 1), a.N - 1) * rb + 16 * (tid & 1);
      ho = min(bn + (tid & 127), a.N - 1) * rb;
    } else {
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int c = tid + 256 * i, row = c >> 2, unit = (c >> 1) & 1, plane = c & 1;
        wo[i] = min(bn + row, a.N - 1) * rb + 16 * ((plane ? K / 64 : 0) + unit);
      }
      ho = min(bn + (tid & 127), a.N - 1) * rb + 32 * (K / 64);
    }
  }

  // ---- global -> register staging of one K stage ----
  // X: 64 rows x 128 bytes = 512 chunks of 16 B, 2 per thread.
  // W: Q8_0 128 rows x 4 blocks x 2 halves; Q4_K 128 rows x 2 pair units x 2 planes.
  // Two register sets: stage s+2 is loaded while stage s computes.
  struct Stage {
    uint4 rx[2], rw[4];
    // Q8_0 d (2 x f16 per dword) / Q4_K header dwords / Q6_K scale dwords and d
    uint32_t rh, rh2, rh3, rh4;
    float rsx;
    int rsb;
  };
  Stage s0{}, s1{};
  auto gload = [&](Stage &S, uint32_t k0) {
    uint4(&rx)[2] = S.rx;
    uint4(&rw)[4] = S.rw;
    uint32_t &rh = S.rh, &rh2 = S.rh2, &rh3 = S.rh3, &rh4 = S.rh4;
    float &rsx = S.rsx;
    int &rsb = S.rsb;
#pragma unroll
    for (int i = 0; i < 2; i++) rx[i] = ldx16(a.qx + (xo[i] + k0));
    // scales: 64 rows x 4 blocks = 256, 1 per thread
    rsx = a.sx[so + k0 / 32];
    if (DT == DT_Q4_K) {
      const int2 s = *reinterpret_cast<const int2 *>(a.s16 + (2 * so + k0 / 16));
      rsb = s.x + s.y;
    }
    if (DT == DT_Q8_0) {
      // 128 rows x 4 blocks x 2 halves; d: 128 rows x 4 blocks x 2 B = 256
      // dwords (two blocks per dword), 1 per thread.
#pragma unroll
      for (int i = 0; i < 4; i++) rw[i] = ld16(a.w + (wo[i] + k0 / 2));
      rh = *reinterpret_cast<const uint32_t *>(a.w + (ho + k0 / 16));
    } else if (DT == DT_Q6_K) {
      // The stage is half hn of super-block sb: units u = 4*sb + 2*hn + h =
      // 2*(k0/128) + h (h = 0, 1), each with planes A, B, Q; thread = (row,
      // h), one chunk per plane. Threads 0..127 (one row each) load S of
      // both units (8 bytes) and d.
      const uint32_t U = K / 64, st = k0 / 128;
#pragma unroll
      for (int p = 0; p < 3; p++) rw[p] = ld16(a.w + (wo[0] + 16 * (p * U + 2 * st)));
      if (tid < 128) {
        const uint2 sc = *reinterpret_cast<const uint2 *>(a.w + (ho + 48 * U + 8 * st));
        rh = sc.x, rh2 = sc.y;
        rh3 = *reinterpret_cast<const uint16_t *>(a.w + (ho + 52 * U + 2 * (k0 / 256)));
      }
    } else {
      // 128 rows x 2 pair units x 2 planes = 512 chunks; the header of the
      // stage's block: 128 rows x 16 B, threads 0..127 one each.
#pragma unroll
      for (int i = 0; i < 2; i++) rw[i] = ld16(a.w + (wo[i] + k0 / 4));
      if (tid < 128) {
        const uint4 hd = ldx16(a.w + (ho + 16 * (k0 / 256)));
        rh = hd.x, rh2 = hd.y, rh3 = hd.z, rh4 = hd.w;
      }
    }
  };
  // ---- register -> LDS ----
  auto lstore = [&](const Stage &S, uint32_t k0) {
    const uint4(&rx)[2] = S.rx;
    const uint4(&rw)[4] = S.rw;
    const uint32_t rh = S.rh, rh2 = S.rh2, rh3 = S.rh3, rh4 = S.rh4;
    const float rsx = S.rsx;
    const int rsb = S.rsb;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int c = tid + 256 * i, row = c >> 3, part = c & 7;
      *reinterpret_cast<uint4 *>(&xs[part >> 1][row][16 * (part & 1)]) = rx[i];
    }
    {
      const int row = tid >> 2, kb = tid & 3;
      sxs[kb][row] = rsx;
      if (DT == DT_Q4_K) sbs[kb][row] = rsx * (float)rsb;  // |sum| <= 127*32: exact in f32
    }
    if (DT == DT_Q8_0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int c = tid + 256 * i, row = c >> 3, blk = (c >> 1) & 3, half = c & 1;
        *reinterpret_cast<uint4 *>(&ws[blk][row][16 * half]) = rw[i];
      }
      const int row = tid >> 1, pairb = tid & 1;
      sws[2 * pairb][row] = h2f(rh);
      sws[2 * pairb + 1][row] = h2f(rh >> 16);
    } else if (DT == DT_Q6_K) {
      // Quarter r of unit h is columns [16h, 16h+16) of the stage's block r.
      const int row = tid >> 1, h = tid & 1;
      const uint4 A = rw[0], B = rw[1], Q = rw[2];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint4 v = make_uint4(q6_centre4(q6_bytes(A.x, B.x, Q.x, r)), q6_centre4(q6_bytes(A.y, B.y, Q.y, r)),
                                   q6_centre4(q6_bytes(A.z, B.z, Q.z, r)), q6_centre4(q6_bytes(A.w, B.w, Q.w, r)));
        *reinterpret_cast<uint4 *>(&ws[r][row][16 * h]) = v;
      }
      if (tid < 128) {
#pragma unroll
        for (int r = 0; r < 4; r++)
          s6[r][tid] = make_int2((int)(int8_t)(rh >> (8 * r)), (int)(int8_t)(rh2 >> (8 * r)));
        d6[tid] = h2f(rh3);
      }
    } else {
      // Pair unit (within the stage) -> sub-blocks 2*unit (low nibbles) and
      // 2*unit+1 (high nibbles); plane -> bytes [16*plane, 16*plane+16).
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int c = tid + 256 * i, row = c >> 2, unit = (c >> 1) & 1, plane = c & 1;
        const uint4 q = rw[i];
        const uint4 lo = make_uint4(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu);
        const uint4 hi = make_uint4((q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, (q.z >> 4) & 0x0F0F0F0Fu,
                                    (q.w >> 4) & 0x0F0F0F0Fu);
        *reinterpret_cast<uint4 *>(&ws[2 * unit][row][16 * plane]) = lo;
        *reinterpret_cast<uint4 *>(&ws[2 * unit + 1][row][16 * plane]) = hi;
      }
      if (tid < 128) {
        const uint4 hd = make_uint4(rh, rh2, rh3, rh4);
        const float d = h2f(rh), dmin = h2f(rh >> 16);
        const int p0 = (k0 % 256) / 64;  // first pair of this stage in its block
#pragma unroll
        for (int u = 0; u < 2; u++) {
          int sca, scb, ma, mb;
          q4k_scales_i(hd, p0 + u, sca, scb, ma, mb);
          sws[2 * u][tid] = d * (float)sca;
          sws[2 * u + 1][tid] = d * (float)scb;
          dms[2 * u][tid] = dmin * (float)ma;
          dms[2 * u + 1][tid] = dmin * (float)mb;
        }
      }
    }
  };

  double acc[2][16];
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[j][r] = 0.0;

  const int lr = lane & 31, lk = lane >> 5;  // operand row/column, K half
  // Block-dot capture: result register r of tile j holds token row
  // (r&3) + 4*lk + 8*(r>>2) of the wave's 32 and weight row 32 j + lane%32.
  const uint32_t nsub = DT == DT_Q6_K ? K / 16 : K / 32;
  auto capture = [&](int j, int r, uint32_t sub, int v) {
    const uint32_t m = bm + wm + (r & 3) + 4 * lk + 8 * (r >> 2), n = bn + wn + 32 * j + lr;
    if (m < a.M && n < a.N) a.dots[((size_t)m * a.N + n) * nsub + sub] = v;
  };
  // The barriers order LDS only: the prefetched stages' global loads stay in
  // flight across them (a full __syncthreads would wait for them).
  auto stage = [&](Stage &S, uint32_t k0) {
    lds_barrier();  // the previous stage's reads of LDS are done
    lstore(S, k0);
    lds_barrier();
    // Always loaded (the last two stages reload the last stage, unused), so
    // the number of loads in flight is fixed and each stage waits only for
    // its own set.
    gload(S, min(k0 + 2 * BK, kend - BK));
    float part[2][16];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) part[j][r] = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      if (DT == DT_Q6_K) {
        float sx[16];
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4 s4 = *reinterpret_cast<const float4 *>(&sxs[kb][wm + 8 * g + 4 * lk]);
          sx[4 * g] = s4.x, sx[4 * g + 1] = s4.y, sx[4 * g + 2] = s4.z, sx[4 * g + 3] = s4.w;
        }
        // K = 16 operands: lane l holds k = 8*(l/32) .. +8 of row l%32.
        const long a0 = *reinterpret_cast<const long *>(&xs[kb][wm + lr][8 * lk]);
        const long a1 = *reinterpret_cast<const long *>(&xs[kb][wm + lr][16 + 8 * lk]);
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const int8_t *wr = &ws[kb][wn + 32 * j + lr][0];
          const v16i c0 =
              __builtin_amdgcn_mfma_i32_32x32x16_i8(a0, *reinterpret_cast<const long *>(wr + 8 * lk), v16i{}, 0, 0, 0);
          const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(
              a1, *reinterpret_cast<const long *>(wr + 16 + 8 * lk), v16i{}, 0, 0, 0);
          if constexpr (CAP) {
            const uint32_t sub = (k0 + 32 * kb) / 16;
#pragma unroll
            for (int r = 0; r < 16; r++) capture(j, r, sub, c0[r]), capture(j, r, sub + 1, c1[r]);
          }
          const int2 sc = s6[kb][wn + 32 * j + lr];
#pragma unroll
          for (int r = 0; r < 16; r++) {
            // |I_lo|, |I_hi| <= 16*127*32 and |sc| <= 128: 24-bit multiplies
            // are exact, and so is the sum (< 2^24) as an f32.
            const int isum = __mul24(sc.x, c0[r]) + __mul24(sc.y, c1[r]);
            part[j][r] = fmaf(sx[r], (float)isum, part[j][r]);
          }
        }
        continue;
      }
      const uint4 t = *reinterpret_cast<const uint4 *>(&xs[kb][wm + lr][16 * lk]);
      const v4i av = v4i{(int)t.x, (int)t.y, (int)t.z, (int)t.w};
      v4i bv[2];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const uint4 u = *reinterpret_cast<const uint4 *>(&ws[kb][wn + 32 * j + lr][16 * lk]);
        bv[j] = v4i{(int)u.x, (int)u.y, (int)u.z, (int)u.w};
      }
      // Rows of result register r: (r&3) + 4*lk + 8*(r>>2) of the tile.
      float sx[16], sb[16];
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 s4 = *reinterpret_cast<const float4 *>(&sxs[kb][wm + 8 * g + 4 * lk]);
        sx[4 * g] = s4.x, sx[4 * g + 1] = s4.y, sx[4 * g + 2] = s4.z, sx[4 * g + 3] = s4.w;
        if (DT == DT_Q4_K) {
          const float4 b4 = *reinterpret_cast<const float4 *>(&sbs[kb][wm + 8 * g + 4 * lk]);
          sb[4 * g] = b4.x, sb[4 * g + 1] = b4.y, sb[4 * g + 2] = b4.z, sb[4 * g + 3] = b4.w;
        }
      }
#pragma unroll
      for (int j = 0; j < 2; j++) {
        v16i c = {};
        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[j], c, 0, 0, 0);
        if constexpr (CAP) {
#pragma unroll
          for (int r = 0; r < 16; r++) capture(j, r, (k0 + 32 * kb) / 32, c[r]);
        }
        const float sw = sws[kb][wn + 32 * j + lr];
        const float dm = DT == DT_Q4_K ? dms[kb][wn + 32 * j + lr] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          part[j][r] = fmaf(sx[r] * sw, (float)c[r], part[j][r]);
          if (DT == DT_Q4_K) part[j][r] = fmaf(-dm, sb[r], part[j][r]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const double dd = DT == DT_Q6_K ? (double)d6[wn + 32 * j + lr] : 1.0;
#pragma unroll
      for (int r = 0; r < 16; r++) acc[j][r] = fma((double)part[j][r], dd, acc[j][r]);
    }
  };
  gload(s0, kbeg);
  gload(s1, min(kbeg + BK, kend - BK));
  for (uint32_t k0 = kbeg; k0 < kend; k0 += 2 * BK) {
    stage(s0, k0);
    if (k0 + BK < kend) stage(s1, k0 + BK);
  }
  if (gridDim.z > 1) {
    // Split K: every split stores its f64 partial tile; the split that
    // arrives last adds them in split order (the same sums whatever the
    // arrival order) and stores Y. Partials move between workgroups only
    // through device-scope stores and loads (coherent across the XCDs'
    // L2s); each wave waits for its stores before the barrier that precedes
    // the counter's device-scope add.
    __shared__ uint32_t last;
    const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x, S = gridDim.z;
    double *pt = a.part + (size_t)tile * S * (BM * BN);
    // Element (m, n) of the tile at m*BN + n; rows past M are neither stored
    // nor read.
    auto at = [&](int j, int r) { return (uint32_t)((wm + (r & 3) + 4 * lk + 8 * (r >> 2)) * BN + wn + 32 * j + lr); };
    auto row_ok = [&](int r) { return bm + wm + (r & 3) + 4 * lk + 8 * (r >> 2) < a.M; };
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        if (row_ok(r))
          __hip_atomic_store(pt + (size_t)blockIdx.z * (BM * BN) + at(j, r), acc[j][r], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev =
          __hip_atomic_fetch_add(a.cnt + tile * CNT_STRIDE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == S - 1;
      if (last) __hip_atomic_store(a.cnt + tile * CNT_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    double red[2][16];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) red[j][r] = 0.0;
    for (uint32_t z = 0; z < S; z++) {  // split order; this split's own sums from registers
      const double *pz = pt + (size_t)z * (BM * BN);
      const bool own = z == blockIdx.z;
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          red[j][r] += own ? acc[j][r]
                           : (row_ok(r) ? __hip_atomic_load(pz + at(j, r), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                        : 0.0);
    }
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[j][r] = red[j][r];
  }
  // ---- store ----
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const uint32_t n = bn + wn + 32 * j + lr;
    if (n >= a.N) continue;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const uint32_t m = bm + wm + (r & 3) + 4 * lk + 8 * (r >> 2);
      if (m < a.M) a.y[(size_t)m * a.N + n] = (float)acc[j][r];
    }
  }
}

}  // namespace

bool gemm_i8_supported(int32_t dtype, int layout, uint64_t n_in, uint64_t n_out) {
  if (layout != MDMA_LAYOUT_GFX950) return false;
  // Weight offsets are 32-bit inside the kernel.
  if (n_out * gfx950_row_bytes(dtype, n_in) >= (1ull << 32)) return false;
  if (dtype == DT_Q8_0) return n_in % BK == 0;
  if (dtype == DT_Q4_K || dtype == DT_Q6_K) return n_in % 256 == 0;
  return false;
}

namespace {

// Activation rows per launch: their int8 offsets are 32-bit inside the kernel.
uint64_t gemm_rows_per_launch(uint64_t K) { return ((1ull << 31) / K) / BM * BM; }

// Splits of K per output tile. A tile's workgroup runs its stages one after
// another (each about 2.5 us when a CU holds one or two such workgroups), so
// a launch of few tiles (few tokens, or few output rows) is latency-bound
// and splitting K divides that time; the splits' f64 partial tiles then cost
// a write and a read each, and the last split a round trip per split. The
// plan minimises that estimate over 1..16 splits of at least 4 stages.
struct Split {
  uint32_t S, ks;
};
Split plan_split(const mdma_ctx *ctx, uint64_t M, uint64_t N, uint64_t K) {
  const uint64_t tiles = (N + BN - 1) / BN * ((M + BM - 1) / BM), nst = K / BK;
  const uint64_t slots = 2 * (ctx->cu_count ? ctx->cu_count : 256);  // two workgroups per CU
  const double stage_us = 2.5, hbm_bytes_per_us = 4.0e6;
  Split best{1, (uint32_t)K};
  double best_us = (double)((tiles + slots - 1) / slots) * nst * stage_us;
  for (uint64_t S = 2; S <= 16 && nst / S >= 4; S++) {
    const uint64_t per = (nst + S - 1) / S, splits = (nst + per - 1) / per;
    const double part_bytes = (double)(M < BM ? M : ((M + BM - 1) / BM) * BM) * N * 8.0 * splits;
    const double us = (double)((tiles * splits + slots - 1) / slots) * per * stage_us + 1.0 * splits +
                      2.0 * part_bytes / hbm_bytes_per_us;
    if (us < best_us) best_us = us, best = Split{(uint32_t)splits, (uint32_t)(per * BK)};
  }
  return best;
}

}  // namespace

void gemm_i8_split_need(const mdma_ctx *ctx, const GemvJob &w, uint64_t M, uint64_t *part_doubles,
                        uint64_t *counters) {
  const uint64_t Mc = M < gemm_rows_per_launch(w.n_in) ? M : gemm_rows_per_launch(w.n_in);
  const Split sp = plan_split(ctx, Mc, w.n_out, w.n_in);
  const uint64_t tiles = (w.n_out + BN - 1) / BN * ((Mc + BM - 1) / BM);
  *part_doubles = sp.S > 1 ? tiles * sp.S * (uint64_t)(BM * BN) : 0;
  *counters = sp.S > 1 ? tiles : 0;
}

void launch_gemm_i8(mdma_ctx *ctx, const GemvJob &w, const int8_t *qx, const float *sx, const int32_t *s16,
                    uint64_t M, float *y, double *part, uint64_t part_doubles, uint32_t *cnt, uint64_t counters) {
  const uint64_t K = w.n_in, N = w.n_out, rows = gemm_rows_per_launch(K);
  hipEvent_t t0 = ctx->time_start, t1 = ctx->time_stop;
  ctx->time_start = ctx->time_stop = nullptr;
  for (uint64_t m0 = 0; m0 < M; m0 += rows) {
    const uint64_t Mc = M - m0 < rows ? M - m0 : rows;
    Split sp = plan_split(ctx, Mc, N, K);
    const uint64_t tiles = (N + BN - 1) / BN * ((Mc + BM - 1) / BM);
    if (sp.S > 1 && (!part || !cnt || tiles * sp.S * (uint64_t)(BM * BN) > part_doubles || tiles > counters))
      sp = Split{1, (uint32_t)K};
    GemmArgs a{qx + m0 * K, sx + m0 * (K / 32), s16 + m0 * (K / 16), w.w, y + m0 * N,
               sp.S > 1 ? part : nullptr, sp.S > 1 ? cnt : nullptr, (uint32_t)Mc, (uint32_t)N, (uint32_t)K,
               sp.ks, gfx950_row_bytes(w.dtype, K), w.dots ? w.dots + m0 * N * dot_subs(w.dtype, K) : nullptr};
    const dim3 grid((uint32_t)((N + BN - 1) / BN), (uint32_t)((Mc + BM - 1) / BM), sp.S), block(256);
    // Timing events (one launch) bracket the first chunk.
    const hipEvent_t e0 = m0 == 0 ? t0 : nullptr, e1 = m0 + Mc >= M ? t1 : nullptr;
    if (a.dots) {
      if (w.dtype == DT_Q8_0) gemm_i8_kernel<DT_Q8_0, true><<<grid, block, 0, ctx->stream>>>(a);
      else if (w.dtype == DT_Q6_K) gemm_i8_kernel<DT_Q6_K, true><<<grid, block, 0, ctx->stream>>>(a);
      else gemm_i8_kernel<DT_Q4_K, true><<<grid, block, 0, ctx->stream>>>(a);
    } else if (w.dtype == DT_Q8_0) {
      if (e0 || e1) hipExtLaunchKernelGGL(gemm_i8_kernel<DT_Q8_0>, grid, block, 0, ctx->stream, e0, e1, 0, a);
      else gemm_i8_kernel<DT_Q8_0><<<grid, block, 0, ctx->stream>>>(a);
    } else if (w.dtype == DT_Q6_K) {
      if (e0 || e1) hipExtLaunchKernelGGL(gemm_i8_kernel<DT_Q6_K>, grid, block, 0, ctx->stream, e0, e1, 0, a);
      else gemm_i8_kernel<DT_Q6_K><<<grid, block, 0, ctx->stream>>>(a);
    } else {
      if (e0 || e1) hipExtLaunchKernelGGL(gemm_i8_kernel<DT_Q4_K>, grid, block, 0, ctx->stream, e0, e1, 0, a);
      else gemm_i8_kernel<DT_Q4_K><<<grid, block, 0, ctx->stream>>>(a);
    }
    hip_check(hipGetLastError(), "gemm i8 launch");
  }
}

}  // namespace mdma
