// Prefill GEMM on gfx950 with the int8 activations and integer weight
// values carried on the f16 matrix path.
//
// Y[m, n] = sum_k X[m, k] * deq(W)[n, k]   (reference HipBackend::qmatmul_i8,
// /root/reference/src/backend/rocm.rs:1759-1918; CPU oracle
// src/backend/cpu.rs:335-368 on the requantized activations)
//
// Activations are quantized per 32 columns to int8 with an f32 scale (the
// int8 mode's prefill configuration, the arithmetic of quantize_act_kernel
// bit for bit). Every int8 value is an exact f16 (|q| <= 127 < 2^11), and so
// is every Q4_K weight value q * sc (q <= 15, sc <= 63: at most 945): each
// product of the f16 MFMA is exact and each 32-column block's dot product,
// at most 2^23 in magnitude, is summed exactly in its f32 accumulator. So
// v_mfma_f32_16x16x32_f16 computes the same integer block dots as an int8
// MFMA, but hands them over as exact f32 with the 6-bit sub-scale already
// applied: the float epilogue is one FMA per output and block,
//   part += s_x[m, b] * C_b[n, m]
// where the i32 MFMA would need a conversion, the sub-scale and the
// activation scale on the VALU (3 to 4 operations per output and block;
// without packed FP32 that caps it near 15% of the int8 peak).
//
// Q4_K, per super-block sb (256 columns, 8 blocks):
//   Y += d[n] * part - dmin[n] * sum_b m[n, b] * P[m, b]
// with P[m, b] = s_x[m, b] * sum_{k in b} q_x[m, k]. The min term is one
// more MFMA per super-block: its 16 columns pair the 8 six-bit mins m[n, b]
// (exact) with P[m, b] split into two f16 (hi + lo, 22 bits), P scaled per
// token row by a power of two 2^e[m] that keeps it in f16 range (divided
// out in the epilogue). The weight operand is q * sc itself, not an offset
// form: an offset (1024 + q*sc, the plain bit-pattern conversion) would add
// 1024 * sum_b P to part, a term several times larger than the result that
// the epilogue would have to subtract again, losing its low bits.
//
// Rounding: part and Y are f32 sums of terms at the scale of the dot
// product's partial sums, so each output is within about u * sum_k |x_k w_k|
// (u = 2^-24) of the exact product of the quantized operands.
//
// Tiling: a 256-thread workgroup computes 128 weight rows x 128 tokens; each
// of its 4 waves 64 x 64 (4 x 4 MFMA tiles of 16 x 16, one 16x16x32 MFMA per
// tile and 32-column block). The weight rows are
// the MFMA's first operand, so each lane holds one token's column of a tile:
// the activation scale s_x is a per-lane scalar, and each output of a lane
// is one weight row. K advances 64 columns (one Q4_K sub-block pair) per
// stage through two LDS buffers: while a stage computes from one, the next
// is converted into the other and the one after is in flight from global
// memory, with one barrier per stage. About 80 KB of LDS: two workgroups
// per CU.
#include <hip/hip_ext.h>

#include <algorithm>

#include <type_traits>

#include "kernels.h"

namespace mdma {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int TN = 128, TM = 128, SK = 64, MAX_BLOCKS = 16384 / 32;

// ---------------------------------------------------------- prologue ----
// One workgroup per token row: q = round(x * 127 / amax) per 32 columns (the
// quantize_act_kernel arithmetic), written as f16; s_x = amax / 127. With P
// (Q4_K): P = s_x * sum q per block, stored as f16 hi + lo of P * 2^e where
// 2^e brings the row's largest |P| into [512, 1024); inv[m] = 2^-e.
__global__ __launch_bounds__(256) void gemm_act_kernel(const float *__restrict__ x, uint32_t K,
                                                       _Float16 *__restrict__ xh, float *__restrict__ sx,
                                                       _Float16 *__restrict__ ph, _Float16 *__restrict__ pl,
                                                       float *__restrict__ inv) {
#pragma clang fp contract(off)
  __shared__ float bs[MAX_BLOCKS], bp[MAX_BLOCKS];
  __shared__ float wmax[4];
  const uint32_t m = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const float *xr = x + (size_t)m * K;
  const uint32_t nch = K / 4, nb = K / 32;
  float pmax = 0.f;
  for (uint32_t c0 = 0; c0 < nch; c0 += 256) {
    // Chunks of 4 columns; the 8 chunks of a block sit on 8 consecutive
    // lanes, all live or all past the row (K is whole blocks).
    const uint32_t c = c0 + tid;
    const bool live = c < nch;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (live) {
      const float4 t = *reinterpret_cast<const float4 *>(xr + 4 * (size_t)c);
      v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
    }
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = dpp_max<0xB1, 0xF>(amax);
    amax = dpp_max<0x4E, 0xF>(amax);
    amax = dpp_max<0x141, 0xF>(amax);  // half-row mirror: the 8 lanes of the block
    const float iv = amax == 0.f ? 0.f : 127.0f / amax;
    int qi[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      qi[k] = q8_quant(v[k], iv);
      sum += qi[k];
    }
    sum += (int)dpp_u32<0xB1, 0xF>((uint32_t)sum);
    sum += (int)dpp_u32<0x4E, 0xF>((uint32_t)sum);
    sum += (int)dpp_u32<0x141, 0xF>((uint32_t)sum);
    const float s = amax / 127.0f, p = s * (float)sum;
    if (live) {
      const v4h h = {(_Float16)(float)qi[0], (_Float16)(float)qi[1], (_Float16)(float)qi[2], (_Float16)(float)qi[3]};
      *reinterpret_cast<v4h *>(xh + (size_t)m * K + 4 * (size_t)c) = h;
      if ((lane & 7) == 0) {
        bs[c >> 3] = s;
        bp[c >> 3] = p;
      }
      pmax = fmaxf(pmax, fabsf(p));
    }
  }
  pmax = wave_max_all(pmax);
  if (lane == 0) wmax[tid >> 6] = pmax;
  __syncthreads();
  const float pm = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  int e = 0;
  if (pm > 0.f) {
    int ex;
    frexpf(pm, &ex);  // pm = f * 2^ex, f in [0.5, 1)
    e = min(max(10 - ex, -100), 100);
  }
  for (uint32_t b = tid; b < nb; b += 256) {
    sx[(size_t)m * nb + b] = bs[b];
    if (ph) {
      const float p = ldexpf(bp[b], e);
      const _Float16 hi = (_Float16)p;
      ph[(size_t)m * nb + b] = hi;
      pl[(size_t)m * nb + b] = (_Float16)(p - (float)hi);
    }
  }
  if (tid == 0 && inv) inv[m] = ldexpf(1.0f, -e);
}

// ------------------------------------------------------------- GEMM ----

struct F16Args {
  const _Float16 *xh;  // [M, K] int8 values as f16
  const float *sx;     // [M, K/32]
  const _Float16 *p;   // [M, K/32] Q4_K: P * 2^e, hi; the lo array p_lo elements further
  uint32_t p_lo;
  const float *inv;    // [M] Q4_K: 2^-e
  const uint8_t *w;    // prepared rows, row_bytes apart
  float *y;            // [M, N]
  uint32_t M, N, K;
  uint64_t row_bytes;
  int32_t *dots;       // block-dot capture [M, N, K/32] (sc * block dot) or null
  // Split K (gridDim.z splits of sb_split super-blocks each): f32 partial
  // tiles [tile][split][TM * TN] and one zeroed arrival counter per tile.
  float *part;
  uint32_t *cnt;
  uint32_t sb_split;
  // Up to 3 weights sharing x in one launch (fused QKV): weight j takes the
  // column tiles from jt[j]; w, y and N above are replaced by its own.
  uint32_t n_jobs;
  const uint8_t *jw[3];
  float *jy[3];
  uint32_t jn[3], jt[3];
  // Gated launch (gemm_f16_kernel's GLU instantiation): jw[0] gate, jw[1]
  // up, both N rows; glu_y [M, N] receives silu(gate) * up. glu_in.xh set:
  // the epilogue also writes the f16-path GEMM input of that output for a
  // GEMM that reads no min-term sums (Q6_K): per 32 columns the int8
  // values as f16 and the scale (xh, sx; gemm_act_kernel's arithmetic).
  float *glu_y;
  F16In glu_in;
  uint32_t glu_no_y;  // with glu_in: glu_y's f32 rows are not stored
  // Fused QKV of a prompt (rope.tab set; the Q6_K wide kernel): q (job 0)
  // rotated before its store, k (job 1) rotated and v (job 2) stored as f16
  // cache rows of token m at m * kv_stride, position pos + m (rope_kv_kernel's
  // arithmetic), in place of k's and v's f32 outputs.
  struct {
    const float *tab;  // [position][hd / 2] (cos, sin)
    uint16_t *dk, *dv;
    uint32_t pos, hd;
    uint64_t kv_stride;
  } rope;
};

// The workgroup's weight of a fused launch (static indices: the values
// stay uniform, in SGPRs) and its first weight row.
struct F16Job {
  const uint8_t *w;
  float *y;
  uint32_t N, bn;
};
__device__ __forceinline__ F16Job f16_job(const F16Args &a, uint32_t bx) {
  if (a.n_jobs > 2 && bx >= a.jt[2]) return F16Job{a.jw[2], a.jy[2], a.jn[2], (bx - a.jt[2]) * TN};
  if (a.n_jobs > 1 && bx >= a.jt[1]) return F16Job{a.jw[1], a.jy[1], a.jn[1], (bx - a.jt[1]) * TN};
  return F16Job{a.w, a.y, a.N, bx * TN};
}

// Token tiles walked per column tile in the XCD-aware tile order.
#ifndef MDMA_F16_GT
#define MDMA_F16_GT 4
#endif

typedef _Float16 h2 __attribute__((ext_vector_type(2)));


// Physical 16-byte chunk of logical chunk c (0..7) of LDS row r: rows are
// 128 bytes, so 16 lanes reading one chunk of 16 consecutive rows would hit
// the same 4 banks every second row; XOR-ing the chunk with bits 1..3 of the
// row spreads them over all 64 banks.
__device__ __forceinline__ int swz(int r, int c) { return (c ^ (r >> 1)) & 7; }

// Eight 4-bit quants q (one dword: bytes b, low nibble then high nibble)
// times a sub-block scale, as f16 pairs: v_perm_b32 puts each nibble under
// the exponent byte 0x64 (the f16 1024 + q), and one packed f16 FMA forms
// (1024 + q) * sc - 1024 * sc = q * sc, exact (the FMA rounds once, and
// q * sc <= 945 is an f16 integer).
__device__ __forceinline__ void q4_f16(uint32_t q, h2 sa, h2 na, h2 sb, h2 nb_, uint32_t lo[2], uint32_t hi[2]) {
  const uint32_t t = q & 0x0F0F0F0Fu, u = (q >> 4) & 0x0F0F0F0Fu;
  const uint32_t c = 0x64646464u;
  auto f = [](uint32_t bits, h2 s, h2 n) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, bits), s, n));
  };
  lo[0] = f(__builtin_amdgcn_perm(c, t, 0x04010400u), sa, na);  // quants 0, 1
  lo[1] = f(__builtin_amdgcn_perm(c, t, 0x04030402u), sa, na);  // quants 2, 3
  hi[0] = f(__builtin_amdgcn_perm(c, u, 0x04010400u), sb, nb_);
  hi[1] = f(__builtin_amdgcn_perm(c, u, 0x04030402u), sb, nb_);
}

// Split K: every split stores its f32 partial tile; the split that arrives
// last adds them in split order (the same sums whatever the arrival order)
// into acc and goes on to store Y; the others return false. A tile's
// partial is [value k of a thread][thread], so each store and load of a
// wave covers 256 consecutive bytes. Partials move between workgroups
// (possibly on different XCDs, whose L2s are not coherent with each other)
// only through device-scope stores and loads; each wave waits for its
// stores before the barrier that precedes the counter's device-scope add.
// NT: the workgroup's threads (a tile of NT * 64 outputs).
template <int NT = 256>
__device__ bool f16_split_merge(float (&acc)[4][4][4], const F16Args &a) {
  __shared__ uint32_t last;
  constexpr uint32_t TILE = NT * 64;
  const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x, S = gridDim.z, z = blockIdx.z, tid = threadIdx.x;
  float *pt = a.part + (size_t)tile * S * TILE + tid;
#pragma unroll
  for (int k = 0; k < 64; k++)
    __hip_atomic_store(pt + (size_t)z * TILE + NT * k, acc[k >> 4][(k >> 2) & 3][k & 3], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(a.cnt + tile * CNT_STRIDE, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last = prev == S - 1;
    if (last) __hip_atomic_store(a.cnt + tile * CNT_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return false;
  // Split by split, a split's 64 loads in flight together. The f32 sums in
  // split order round as often as the unsplit kernel's chain over the same
  // super-blocks does (one addition per super-block).
  float sum[64];
#pragma unroll
  for (int k = 0; k < 64; k++) sum[k] = 0.f;
  for (uint32_t y = 0; y < S; y++) {
    const float *py = pt + (size_t)y * TILE;
#pragma unroll
    for (int k = 0; k < 64; k++)
      sum[k] += y == z ? acc[k >> 4][(k >> 2) & 3][k & 3]
                       : __hip_atomic_load(py + NT * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int k = 0; k < 64; k++) acc[k >> 4][(k >> 2) & 3][k & 3] = sum[k];
  return true;
}

// CAP: the block-dot capture instantiation (F16Args::dots set).
// GLU: the gated instantiation. A workgroup takes 64 rows of gate and the
// same 64 rows of up (tile rows 32 w .. 32 w + 31 of wave w: gate for even
// w, up for odd, rows bn + 32 (w / 2) + ..), so each lane holds a gate
// output and its up output in acc[i] and acc[i + 2], and the epilogue
// writes silu(gate) * up: the same per-output arithmetic as two separate
// tiles, the same bits as the elementwise silu_mul of their outputs.
template <int DT, bool CAP = false, bool GLU = false>
__global__ __launch_bounds__(256, 2) void gemm_f16_kernel(F16Args a) {
  __shared__ __attribute__((aligned(16))) _Float16 ws[2][TN][SK];  // weights, f16 q * sc
  __shared__ __attribute__((aligned(16))) _Float16 xs[2][TM][SK];  // activations, f16 int8 values
  __shared__ __attribute__((aligned(16))) uint8_t wraw[TN][32];    // the stage's quant bytes (planes A, B)
  __shared__ __attribute__((aligned(16))) uint8_t whd[TN][16];     // the super-block's row headers
  __shared__ __attribute__((aligned(16))) float sxs[2][2][TM];      // s_x of the stage's two blocks
  __shared__ __attribute__((aligned(16))) _Float16 xmin[2][TM][8];  // P hi / lo of the super-block
  __shared__ __attribute__((aligned(16))) _Float16 wmin[TN][8];     // the rows' 8 mins
  __shared__ __attribute__((aligned(16))) float dvs[TN], dms[TN];
  __shared__ float invs[TM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const GridTile tl = grid_tile(MDMA_F16_GT);
  const F16Job J = f16_job(a, tl.x);
  const uint32_t bn = GLU ? tl.x * (TN / 2) : J.bn, bm = tl.y * TM, N = GLU ? a.N : J.N;
  const int wn = (wave & 1) * 64, wm = (wave >> 1) * 64;
  // 16 x 16 MFMA tiles: lane l holds column l % 16 (a token) and K chunk
  // l / 16 of its operands, and rows 4 (l / 16) .. + 3 of its result.
  const int l16 = lane & 15, lq = lane >> 4;
  const uint32_t K = a.K, nb = K / 32, nst = K / SK, U = K / 64, rb = (uint32_t)a.row_bytes;
  // Weight row of tile row r, and the weight this wave's loads read (its
  // tile rows are 32 wave .. 32 wave + 31).
  auto trow = [&](uint32_t r) { return GLU ? bn + 32 * (r >> 6) + (r & 31) : bn + r; };
  const uint8_t *wsrc = J.w;
  if constexpr (GLU) {
    // The wave index made uniform first, so the choice is a scalar select
    // of two kernel arguments (no per-lane pointer to rebuild).
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    wsrc = (wv & 1) ? a.jw[1] : a.jw[0];
  }

  // Byte offsets of each lane's DMA sources (32-bit: the launcher keeps the
  // activations below 2^31 elements and the weights below 2^32 bytes).
  // X: the wave's i-th load fills rows 32 wave + 8 i + l / 8, physical chunk
  // l % 8 (LDS byte 16 l), with the logical chunk the swizzle places there.
  uint32_t xo[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = 32 * wave + 8 * i + (lane >> 3);
    xo[i] = 2 * (min(bm + row, a.M - 1) * K + 8 * swz(row, lane & 7));
  }
  // Per thread (LDS byte 16 tid or 4 tid): token s_tok's block s_blk (s_x)
  // or hi / lo half (P); weight row w_row's plane w_plane.
  const int s_tok = tid & 127, s_blk = tid >> 7;
  const uint32_t s_row = min(bm + s_tok, a.M - 1);
  const uint32_t so = 4 * (s_row * nb + s_blk), po = 2 * (s_row * nb + (s_blk ? a.p_lo : 0));
  const int w_row = tid >> 1, w_plane = tid & 1;
  const uint32_t wrow = min(trow(w_row), N - 1) * rb;
  const uint32_t wo = wrow + 16 * (w_plane ? U : 0);
  // Headers: lanes 0..31 of wave w load rows 32 w + lane (the rows of the
  // wave's own threads).
  const uint32_t ho = min(trow(32 * wave + (lane & 31)), N - 1) * rb + 32 * U;
  if (tid < TM) invs[tid] = a.inv[min(bm + tid, a.M - 1)];

  // Stage st's operands into LDS: X into xs[st & 1], s_x into sxs[st & 1],
  // the quant bytes into wraw; at a super-block's first stage its headers.
  auto gload = [&](uint32_t st) {
#pragma unroll
    for (int i = 0; i < 4; i++) lds_dma16(a.xh, xo[i] + 128 * st, &xs[st & 1][32 * wave + 8 * i][0]);
    lds_dma4(a.sx, so + 8 * st, &sxs[st & 1][0][64 * wave]);
    lds_dma16(wsrc, wo + 16 * st, &wraw[32 * wave][0]);
    if (st % 4 == 0 && lane < 32) lds_dma16(wsrc, ho + 4 * st, &whd[32 * wave][0]);
  };
  // P of super-block sb into xmin (its previous contents, the last
  // super-block's, are read by that super-block's epilogue: issued after it).
  auto pload = [&](uint32_t sb) { lds_dma16(a.p, po + 16 * sb, &xmin[0][0][0] + 512 * wave); };
  // The stage's weights into ws[st & 1] as f16 q * sc (each thread converts
  // the 16 bytes it loaded).
  auto wstore = [&](uint32_t st) {
    const uint4 gq = *reinterpret_cast<const uint4 *>(&wraw[w_row][16 * w_plane]);
    const uint4 hd = *reinterpret_cast<const uint4 *>(&whd[w_row][0]);
    int sca, scb, ma, mb;
    q4k_scales_i(hd, st & 3, sca, scb, ma, mb);
    const _Float16 fa = (_Float16)(float)sca, fb = (_Float16)(float)scb;
    const h2 sa = {fa, fa}, sb = {fb, fb};
    const h2 na = {(_Float16)(-1024.0f * (float)sca), (_Float16)(-1024.0f * (float)sca)};
    const h2 nbv = {(_Float16)(-1024.0f * (float)scb), (_Float16)(-1024.0f * (float)scb)};
    // 16 bytes: low nibbles -> sub-block 2p columns [16*plane, +16),
    // high nibbles -> sub-block 2p+1 columns [32 + 16*plane, +16).
    const uint32_t qw[4] = {gq.x, gq.y, gq.z, gq.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int d = 0; d < 4; d++) q4_f16(qw[d], sa, na, sb, nbv, &lo[2 * d], &hi[2 * d]);
    _Float16 *wr = &ws[st & 1][w_row][0];
    *reinterpret_cast<uint4 *>(wr + 8 * swz(w_row, 2 * w_plane)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<uint4 *>(wr + 8 * swz(w_row, 2 * w_plane + 1)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
    *reinterpret_cast<uint4 *>(wr + 8 * swz(w_row, 4 + 2 * w_plane)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4 *>(wr + 8 * swz(w_row, 5 + 2 * w_plane)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
  };
  // The super-block's epilogue operands from its headers: the 8 mins of each
  // row (f16), d and dmin.
  auto hstore = [&]() {
    const uint4 hd = *reinterpret_cast<const uint4 *>(&whd[w_row][0]);
    if (w_plane == 0) {
      int mn[8], sc;
#pragma unroll
      for (int j = 0; j < 4; j++) q4k_scales_i(hd, j, sc, sc, mn[2 * j], mn[2 * j + 1]);
      const v8h mv = {(_Float16)(float)mn[0], (_Float16)(float)mn[1], (_Float16)(float)mn[2], (_Float16)(float)mn[3],
                      (_Float16)(float)mn[4], (_Float16)(float)mn[5], (_Float16)(float)mn[6], (_Float16)(float)mn[7]};
      *reinterpret_cast<v8h *>(&wmin[w_row][0]) = mv;
      dvs[w_row] = h2f(hd.x);
    } else {
      dms[w_row] = h2f(hd.x >> 16);
    }
  };

  // part: the super-block's sum of s_x * block dot; acc: the outputs.
  float acc[4][4][4], part[4][4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.f, part[i][j][r] = 0.f;

  // This split's stages (whole super-blocks).
  const uint32_t st0 = blockIdx.z * a.sb_split * 4, st1 = min(st0 + a.sb_split * 4, nst);
  gload(st0);
  pload(st0 / 4);
  lds_wait_dma();
  wstore(st0);
  hstore();
  lds_barrier();
  for (uint32_t st = st0; st < st1; st++) {
    // Stage st + 1's loads in flight over this stage's MFMAs, into the other
    // buffers (last read by stage st - 1, before the barrier). A
    // super-block's P goes in at its second stage, after the previous
    // super-block's epilogue.
    if (st + 1 < st1) gload(st + 1);
    if (st % 4 == 0 && st > st0) pload(st / 4);
    const int buf = st & 1;
    // One block (h) of the stage: one 16x16x32 MFMA per tile, then
    // part += s_x * dot. FIRST (a super-block's first block): part = s_x * dot.
    auto block = [&](int h, auto first) {
      v8h A[4], B[4];
      float s[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = wn + 16 * i + l16;
        A[i] = *reinterpret_cast<const v8h *>(&ws[buf][r][8 * swz(r, 4 * h + lq)]);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int r = wm + 16 * j + l16;
        B[j] = *reinterpret_cast<const v8h *>(&xs[buf][r][8 * swz(r, 4 * h + lq)]);
        s[j] = sxs[buf][h][r];
      }
      // Software-pipelined two tiles deep: tile t + 2's MFMA is issued before
      // tile t's FMAs, whose MFMA result is then long complete, so the
      // matrix core and the VALU overlap.
      v4f c[3];
      c[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], B[0], v4f{}, 0, 0, 0);
      c[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], B[1], v4f{}, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 16; t++) {
        if (t + 2 < 16)
          c[(t + 2) % 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[(t + 2) >> 2], B[(t + 2) & 3], v4f{}, 0, 0, 0);
        const int i = t >> 2, j = t & 3;
        if constexpr (CAP) {  // block-dot capture: the exact integer sc * dot of each output's block
          const uint32_t m = bm + wm + 16 * j + l16;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const uint32_t n = bn + wn + 16 * i + 4 * lq + r;
            if (m < a.M && n < J.N) a.dots[((size_t)m * J.N + n) * nb + 2 * st + h] = (int)c[t % 3][r];
          }
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
          part[i][j][r] = first ? s[j] * c[t % 3][r] : fmaf(s[j], c[t % 3][r], part[i][j][r]);
      }
    };
    if (st % 4 == 0) block(0, std::true_type{});
    else block(0, std::false_type{});
    block(1, std::false_type{});
    if (st % 4 == 3) {  // the super-block's last stage: d and the min term
      // Min MFMA (16x16x16): K chunk lq of 4 columns; chunks 0, 1 pair the
      // 8 mins with P hi, chunks 2, 3 the same mins with P lo.
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int rw = wn + 16 * i;
        const v4h Am = *reinterpret_cast<const v4h *>(&wmin[rw + l16][4 * (lq & 1)]);
        const float4 d4 = *reinterpret_cast<const float4 *>(&dvs[rw + 4 * lq]);
        const float4 m4 = *reinterpret_cast<const float4 *>(&dms[rw + 4 * lq]);
        const float dv[4] = {d4.x, d4.y, d4.z, d4.w}, dm[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int t = wm + 16 * j + l16;
          const v4h Bm = *reinterpret_cast<const v4h *>(&xmin[lq >> 1][t][4 * (lq & 1)]);
          const v4f cm = __builtin_amdgcn_mfma_f32_16x16x16f16(Am, Bm, v4f{}, 0, 0, 0);
          const float iv = invs[t];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            acc[i][j][r] = fmaf(dv[r], part[i][j][r], acc[i][j][r]);
            acc[i][j][r] = fmaf(-dm[r] * iv, cm[r], acc[i][j][r]);
          }
        }
      }
    }
    lds_wait_dma();
    if (st + 1 < st1) wstore(st + 1);
    // A super-block's epilogue operands go to LDS once the previous
    // super-block's epilogue (stage st - 1) has passed the barrier.
    if (st % 4 == 0 && st > st0) hstore();
    lds_barrier();
  }
  if (gridDim.z > 1 && !f16_split_merge(acc, a)) return;
  if constexpr (GLU) {  // silu(gate) * up; the launcher keeps N a multiple of 128
    // A token's (lane l16's) 32 columns bn + wn / 2 + [0, 32) are one
    // quantization block: 8 values in each of the lanes l16 + 16 lq.
    const bool q = a.glu_in.xh != nullptr;  // uniform
    const uint32_t n0 = bn + (wn >> 1);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t m = bm + wm + 16 * j + l16;
      float h[2][4];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t n = n0 + 16 * i + 4 * lq;
#pragma unroll
        for (int r = 0; r < 4; r++) h[i][r] = silu_mul1(acc[i][j][r], acc[i + 2][j][r]);
        if (m < a.M && !a.glu_no_y)
          *reinterpret_cast<float4 *>(a.glu_y + (size_t)m * N + n) = make_float4(h[i][0], h[i][1], h[i][2], h[i][3]);
      }
      if (q) {
#pragma clang fp contract(off)
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
          for (int r = 0; r < 4; r++) am = fmaxf(am, fabsf(h[i][r]));
        am = fmaxf(am, __shfl_xor(am, 16));
        am = fmaxf(am, __shfl_xor(am, 32));
        const float iv = am == 0.f ? 0.f : 127.0f / am;
        if (m < a.M) {
#pragma unroll
          for (int i = 0; i < 2; i++) {
            const v4h hv = {(_Float16)(float)q8_quant(h[i][0], iv), (_Float16)(float)q8_quant(h[i][1], iv),
                            (_Float16)(float)q8_quant(h[i][2], iv), (_Float16)(float)q8_quant(h[i][3], iv)};
            *reinterpret_cast<v4h *>(a.glu_in.xh + (size_t)m * N + n0 + 16 * i + 4 * lq) = hv;
          }
          if (lq == 0) a.glu_in.sx[(size_t)m * (N / 32) + n0 / 32] = am / 127.0f;
        }
      }
    }
    return;
  }
  // ---- store: lane = token; a tile's 4 outputs are 4 consecutive rows ----
  const bool vec = (J.N & 3) == 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t m = bm + wm + 16 * j + l16;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t n = bn + wn + 16 * i + 4 * lq;
      float *yp = J.y + (size_t)m * J.N + n;
      if (vec && n + 3 < J.N) {
        *reinterpret_cast<float4 *>(yp) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int t = 0; t < 4; t++)
          if (n + t < J.N) yp[t] = acc[i][j][t];
      }
    }
  }
}

// Q6_K on the f16 path (same tiling and stages as gemm_f16_kernel). The
// weight value w = sc * q (sc in [-128, 127], q in [-32, 31]) passes 2048,
// past which f16 holds only even integers, so the operand is split exactly:
// A1 = f16(w), the f16 product of the exact f16 operands q and sc, rounded
// once, and A2 = w - A1 in {-1, 0, 1}, a fused multiply-add of the same
// operands (exact). |A1| <= 4096 and |A2| <= 1, so a block's partial sums
// stay below 32 * 127 * 4097 < 2^24 and the MFMA adds them exactly: the
// f32 block dot is the integer sum_k q_x * sc * q. A stage whose A2 is zero
// across the workgroup (no |sc| above 64 meets an odd product past 2048)
// skips the A2 MFMAs. d multiplies each super-block's part as Q4_K's does;
// Q6_K has no min term.
// Stage st is columns [64 st, 64 st + 64) = quarters 2 qp and 2 qp + 1 (qp =
// st % 2, blocks 0 and 1) of half n = st / 2 % 2 of super-block st / 4: the
// prepared units 2 (st / 2) + h' (h' = 0, 1) hold columns [16 h', 16 h' + 16)
// of every quarter (planes A, B: ql of quarters 0/2 and 1/3; Q: qh).
// The converted operands are single-buffered (a second barrier per stage)
// so that two workgroups fit a CU's LDS.
__device__ __forceinline__ void q6_pair_f16(uint32_t v, h2 sc2, uint32_t &a1, uint32_t &a2, int k) {
  const h2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
  const h2 q = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, k ? 0x04030402u : 0x04010400u)) + off;
  const h2 p = q * sc2;
  a1 = __builtin_bit_cast(uint32_t, p);
  a2 = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, sc2, -p));
}

__global__ __launch_bounds__(256, 2) void gemm_f16_q6_kernel(F16Args a) {
  __shared__ __attribute__((aligned(16))) _Float16 ws[TN][SK];      // A1
  __shared__ __attribute__((aligned(16))) _Float16 ws2[TN][SK];     // A2
  __shared__ __attribute__((aligned(16))) _Float16 xs[2][TM][SK];   // activations, f16 int8 values
  __shared__ __attribute__((aligned(16))) uint8_t wraw[3][256][16];  // planes A, B, Q of thread (row, h')
  __shared__ __attribute__((aligned(16))) uint32_t wsc[256];        // the unit's 4 scales
  __shared__ __attribute__((aligned(16))) uint32_t dvr[TN];         // the dword holding d, then d (f32)
  __shared__ __attribute__((aligned(16))) float sxs[2][2][TM];
  __shared__ uint32_t need2[2];  // per stage parity: some A2 of the stage is not zero

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const GridTile tl = grid_tile(MDMA_F16_GT);
  const F16Job J = f16_job(a, tl.x);
  const uint32_t bn = J.bn, bm = tl.y * TM;
  const int wn = (wave & 1) * 64, wm = (wave >> 1) * 64;
  const int l16 = lane & 15, lq = lane >> 4;
  const uint32_t K = a.K, nb = K / 32, nst = K / SK, U = K / 64, rb = (uint32_t)a.row_bytes;

  uint32_t xo[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = 32 * wave + 8 * i + (lane >> 3);
    xo[i] = 2 * (min(bm + row, a.M - 1) * K + 8 * swz(row, lane & 7));
  }
  const int s_tok = tid & 127, s_blk = tid >> 7;
  const uint32_t so = 4 * (min(bm + s_tok, a.M - 1) * nb + s_blk);
  // Quant planes: thread = (row tid / 2, unit h' = tid % 2).
  const int w_row = tid >> 1, w_h = tid & 1;
  const uint32_t wrow = min(bn + w_row, J.N - 1) * rb;
  // d: lanes 0..31 of wave w take rows 32 w + lane.
  const uint32_t drow = min(bn + 32 * wave + (lane & 31), J.N - 1) * rb + 52 * U;

  auto gload = [&](uint32_t st) {
#pragma unroll
    for (int i = 0; i < 4; i++) lds_dma16(a.xh, xo[i] + 128 * st, &xs[st & 1][32 * wave + 8 * i][0]);
    lds_dma4(a.sx, so + 8 * st, &sxs[st & 1][0][64 * wave]);
    if (st % 2 == 0) {  // the half super-block's planes serve both its stages
      const uint32_t u = 2 * (st / 2) + w_h;
#pragma unroll
      for (int p = 0; p < 3; p++) lds_dma16(J.w, wrow + 16 * (p * U + u), &wraw[p][64 * wave][0]);
      lds_dma4(J.w, wrow + 48 * U + 4 * u, &wsc[64 * wave]);
    }
    // A super-block's d goes in with its second stage (the previous
    // super-block's epilogue, at its last stage, has read dvr by then).
    if (st % 4 == 1 && lane < 32) lds_dma4(J.w, (drow + 2 * (st / 4)) & ~3u, &dvr[32 * wave]);
  };
  // Stage st's operands: this thread's 16 columns of each of the two blocks.
  auto wstore = [&](uint32_t st) {
    const uint4 A = *reinterpret_cast<const uint4 *>(&wraw[0][tid][0]);
    const uint4 B = *reinterpret_cast<const uint4 *>(&wraw[1][tid][0]);
    const uint4 Q = *reinterpret_cast<const uint4 *>(&wraw[2][tid][0]);
    const uint32_t sc4 = wsc[tid];
    const int qp = st & 1;
    const uint32_t av[4] = {A.x, A.y, A.z, A.w}, bv[4] = {B.x, B.y, B.z, B.w}, hv[4] = {Q.x, Q.y, Q.z, Q.w};
    uint32_t any = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int qq = 2 * qp + h;
      const _Float16 fs = (_Float16)(float)(int8_t)(sc4 >> (8 * qq));
      const h2 sc2 = {fs, fs};
      const int c0 = 4 * h + 2 * w_h;
#pragma unroll
      for (int d = 0; d < 4; d++) {  // columns 4d..4d+3 of the thread's 16: half of chunk c0 + d / 2
        const uint32_t nd = h ? bv[d] : av[d];
        const uint32_t nib = qp ? (nd >> 4) & 0x0F0F0F0Fu : nd & 0x0F0F0F0Fu;
        const uint32_t v = nib | (((hv[d] >> (2 * qq)) & 0x03030303u) << 4);
        uint32_t a1[2], a2[2];
        q6_pair_f16(v, sc2, a1[0], a2[0], 0);
        q6_pair_f16(v, sc2, a1[1], a2[1], 1);
        any |= (a2[0] | a2[1]) & 0x7FFF7FFFu;
        const int col = 8 * swz(w_row, c0 + (d >> 1)) + 4 * (d & 1);
        *reinterpret_cast<uint2 *>(&ws[w_row][col]) = make_uint2(a1[0], a1[1]);
        *reinterpret_cast<uint2 *>(&ws2[w_row][col]) = make_uint2(a2[0], a2[1]);
      }
    }
    if (__builtin_amdgcn_ballot_w64(any != 0) != 0 && lane == 0) atomicOr(&need2[st & 1], 1u);
  };
  // Super-block sb's d (the half of the aligned dword holding it) as f32,
  // in place, rows 0..127.
  auto hstore = [&](uint32_t sb) {
    if (tid < TN) {
      const uint32_t w = dvr[tid];
      dvr[tid] = __builtin_bit_cast(uint32_t, h2f(sb & 1 ? w >> 16 : w));
    }
  };

  float acc[4][4][4], part[4][4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.f, part[i][j][r] = 0.f;

  if (tid < 2) need2[tid] = 0u;
  lds_barrier();
  const uint32_t st0 = blockIdx.z * a.sb_split * 4, st1 = min(st0 + a.sb_split * 4, nst);
  gload(st0);
  lds_wait_dma();
  lds_barrier();
  wstore(st0);
  lds_barrier();
  for (uint32_t st = st0; st < st1; st++) {
    if (st + 1 < st1) gload(st + 1);
    const int buf = st & 1;
    const bool n2 = need2[buf] != 0u;
    auto block = [&](int h, auto first) {
      v8h A[4], A2[4], B[4];
      float s[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = wn + 16 * i + l16;
        A[i] = *reinterpret_cast<const v8h *>(&ws[r][8 * swz(r, 4 * h + lq)]);
        if (n2) A2[i] = *reinterpret_cast<const v8h *>(&ws2[r][8 * swz(r, 4 * h + lq)]);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int r = wm + 16 * j + l16;
        B[j] = *reinterpret_cast<const v8h *>(&xs[buf][r][8 * swz(r, 4 * h + lq)]);
        s[j] = sxs[buf][h][r];
      }
      auto dot = [&](int t) {
        v4f c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t >> 2], B[t & 3], v4f{}, 0, 0, 0);
        if (n2) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A2[t >> 2], B[t & 3], c, 0, 0, 0);
        return c;
      };
      v4f c[3];
      c[0] = dot(0);
      c[1] = dot(1);
#pragma unroll
      for (int t = 0; t < 16; t++) {
        if (t + 2 < 16) c[(t + 2) % 3] = dot(t + 2);
        const int i = t >> 2, j = t & 3;
#pragma unroll
        for (int r = 0; r < 4; r++)
          part[i][j][r] = first ? s[j] * c[t % 3][r] : fmaf(s[j], c[t % 3][r], part[i][j][r]);
      }
    };
    if (st % 4 == 0) block(0, std::true_type{});
    else block(0, std::false_type{});
    block(1, std::false_type{});
    if (st % 4 == 3) {  // the super-block's last stage: acc += d * part
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float4 d4 = *reinterpret_cast<const float4 *>(&dvr[wn + 16 * i + 4 * lq]);
        const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(dv[r], part[i][j][r], acc[i][j][r]);
      }
    }
    lds_wait_dma();
    lds_barrier();  // every wave is done with the stage's operands and flag
    if (tid == 0) need2[buf] = 0u;  // next written by the stage after next
    if (st + 1 < st1) {
      wstore(st + 1);
      if ((st + 1) % 4 == 1) hstore((st + 1) / 4);
    }
    lds_barrier();
  }
  if (gridDim.z > 1 && !f16_split_merge(acc, a)) return;
  const bool vec = (J.N & 3) == 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t m = bm + wm + 16 * j + l16;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t n = bn + wn + 16 * i + 4 * lq;
      float *yp = J.y + (size_t)m * J.N + n;
      if (vec && n + 3 < J.N) {
        *reinterpret_cast<float4 *>(yp) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int t = 0; t < 4; t++)
          if (n + t < J.N) yp[t] = acc[i][j][t];
      }
    }
  }
}

// Q6_K with 256 tokens per workgroup: 512 threads (8 waves of 64 rows x 64
// tokens), one workgroup per CU (148 KB of LDS). The same arithmetic per
// output as gemm_f16_q6_kernel; what changes is the schedule: the operands
// A1 / A2 are double-buffered like gemm_f16_kernel's (one barrier per
// stage: stage st + 1 is converted while stage st's MFMAs run), each
// stage's weight conversion serves 256 tokens instead of 128, and it is
// split over all 8 waves (block 0 of the stage on waves 0-3, block 1 on
// waves 4-7). Between a wave's wait for its own DMAs and the barrier it
// reads only what it loaded itself: waves 0-3 load plane A, waves 4-7
// plane B, each half its own copy of plane Q and of the scales, and waves
// 0-1 the d of the rows they convert.
constexpr int TMW = 256;

__global__ __launch_bounds__(512, 1) void gemm_f16_q6w_kernel(F16Args a) {
  __shared__ __attribute__((aligned(16))) _Float16 ws[2][TN][SK];    // A1, by stage parity
  __shared__ __attribute__((aligned(16))) _Float16 ws2[2][TN][SK];   // A2
  __shared__ __attribute__((aligned(16))) _Float16 xs[2][TMW][SK];   // activations, f16 int8 values
  // Planes A and B, then plane Q twice (for waves 0-3 and 4-7), of thread
  // (row, h'); the scales twice.
  __shared__ __attribute__((aligned(16))) uint8_t wraw[4][256][16];
  __shared__ __attribute__((aligned(16))) uint32_t wsc[2][256];     // the unit's 4 scales
  __shared__ __attribute__((aligned(16))) uint32_t dvr[TN];          // the dword holding d, then d (f32)
  __shared__ __attribute__((aligned(16))) float sxs[2][2][TMW];
  // Per stage parity and wave: some A2 of the wave's conversion is not zero
  // (each wave writes its own byte, so nothing needs clearing).
  __shared__ __attribute__((aligned(8))) uint8_t need2w[2][8];

  const int tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const GridTile tl = grid_tile(MDMA_F16_GT);
  const F16Job J = f16_job(a, tl.x);
  const uint32_t bn = J.bn, bm = tl.y * TMW;
  const int wn = (wave & 1) * 64, wm = (wave >> 1) * 64;
  const int l16 = lane & 15, lq = lane >> 4;
  const uint32_t K = a.K, nb = K / 32, nst = K / SK, U = K / 64, rb = (uint32_t)a.row_bytes;

  uint32_t xo[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = 32 * wave + 8 * i + (lane >> 3);
    xo[i] = 2 * (min(bm + row, a.M - 1) * K + 8 * swz(row, lane & 7));
  }
  const int s_tok = tid & (TMW - 1), s_blk = tid >> 8;
  const uint32_t so = 4 * (min(bm + s_tok, a.M - 1) * nb + s_blk);
  // Quant planes: thread pt = tid % 256 = (row pt / 2, unit h' = pt % 2)
  // converts the stage's block wh = tid / 256 from plane wh and plane Q.
  const int pt = tid & 255, w_row = pt >> 1, w_h = pt & 1, wh = tid >> 8;
  const uint32_t wrow = min(bn + w_row, J.N - 1) * rb;
  // d: waves 0 and 1 load and convert rows 64 w + lane.
  const uint32_t drow = min(bn + 64 * (wave & 1) + lane, J.N - 1) * rb + 52 * U;
  const uint32_t whs = wave >> 2;  // the wave's half: planes A or B (uniform)

  auto gload = [&](uint32_t st) {
#pragma unroll
    for (int i = 0; i < 4; i++) lds_dma16(a.xh, xo[i] + 128 * st, &xs[st & 1][32 * wave + 8 * i][0]);
    lds_dma4(a.sx, so + 8 * st, &sxs[st & 1][0][64 * wave]);
    if (st % 2 == 0) {  // the half super-block's planes serve both its stages
      const uint32_t u = 2 * (st / 2) + w_h, q = 64 * (wave & 3);
      lds_dma16(J.w, wrow + 16 * (whs * U + u), &wraw[whs][q][0]);
      lds_dma16(J.w, wrow + 16 * (2 * U + u), &wraw[2 + whs][q][0]);
      lds_dma4(J.w, wrow + 48 * U + 4 * u, &wsc[whs][q]);
    }
    // A super-block's d goes in with its second stage (the previous
    // super-block's epilogue, at its last stage, has read dvr by then).
    if (st % 4 == 1 && wave < 2) lds_dma4(J.w, (drow + 2 * (st / 4)) & ~3u, &dvr[64 * wave]);
  };
  // Stage st's operands into buffer st % 2: this thread's 16 columns of
  // block wh.
  auto wstore = [&](uint32_t st) {
    const uint4 P = *reinterpret_cast<const uint4 *>(&wraw[wh][pt][0]);
    const uint4 Q = *reinterpret_cast<const uint4 *>(&wraw[2 + wh][pt][0]);
    const uint32_t sc4 = wsc[wh][pt];
    const int qp = st & 1, qq = 2 * qp + wh, b = st & 1;
    const uint32_t pv[4] = {P.x, P.y, P.z, P.w}, hv[4] = {Q.x, Q.y, Q.z, Q.w};
    const _Float16 fs = (_Float16)(float)(int8_t)(sc4 >> (8 * qq));
    const h2 sc2 = {fs, fs};
    const int c0 = 4 * wh + 2 * w_h;
    uint32_t any = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) {  // columns 4d..4d+3 of the thread's 16: half of chunk c0 + d / 2
      const uint32_t nib = qp ? (pv[d] >> 4) & 0x0F0F0F0Fu : pv[d] & 0x0F0F0F0Fu;
      const uint32_t v = nib | (((hv[d] >> (2 * qq)) & 0x03030303u) << 4);
      uint32_t a1[2], a2[2];
      q6_pair_f16(v, sc2, a1[0], a2[0], 0);
      q6_pair_f16(v, sc2, a1[1], a2[1], 1);
      any |= (a2[0] | a2[1]) & 0x7FFF7FFFu;
      const int col = 8 * swz(w_row, c0 + (d >> 1)) + 4 * (d & 1);
      *reinterpret_cast<uint2 *>(&ws[b][w_row][col]) = make_uint2(a1[0], a1[1]);
      *reinterpret_cast<uint2 *>(&ws2[b][w_row][col]) = make_uint2(a2[0], a2[1]);
    }
    const bool nz = __builtin_amdgcn_ballot_w64(any != 0) != 0;
    if (lane == 0) need2w[b][wave] = nz ? 1 : 0;
  };
  // Super-block sb's d (the half of the aligned dword holding it) as f32,
  // in place, rows 0..127 (threads 0..127: waves 0 and 1, which loaded them).
  auto hstore = [&](uint32_t sb) {
    if (tid < TN) {
      const uint32_t w = dvr[tid];
      dvr[tid] = __builtin_bit_cast(uint32_t, h2f(sb & 1 ? w >> 16 : w));
    }
  };

  float acc[4][4][4], part[4][4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.f, part[i][j][r] = 0.f;

  const uint32_t st0 = blockIdx.z * a.sb_split * 4, st1 = min(st0 + a.sb_split * 4, nst);
  gload(st0);
  lds_wait_dma();
  lds_barrier();
  wstore(st0);
  lds_barrier();
  for (uint32_t st = st0; st < st1; st++) {
    // Stage st + 1's loads in flight over this stage's MFMAs, into buffers
    // last read by stage st - 1 (before the barrier). Each wave waits for
    // its own before converting what they brought (lds_wait_dma below).
    if (st + 1 < st1) gload(st + 1);
    const int buf = st & 1;
    const bool n2 = *reinterpret_cast<const uint64_t *>(&need2w[buf][0]) != 0;
    auto block = [&](int h, auto first) {
      v8h A[4], A2[4], B[4];
      float s[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = wn + 16 * i + l16;
        A[i] = *reinterpret_cast<const v8h *>(&ws[buf][r][8 * swz(r, 4 * h + lq)]);
        if (n2) A2[i] = *reinterpret_cast<const v8h *>(&ws2[buf][r][8 * swz(r, 4 * h + lq)]);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int r = wm + 16 * j + l16;
        B[j] = *reinterpret_cast<const v8h *>(&xs[buf][r][8 * swz(r, 4 * h + lq)]);
        s[j] = sxs[buf][h][r];
      }
      auto dot = [&](int t) {
        v4f c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t >> 2], B[t & 3], v4f{}, 0, 0, 0);
        if (n2) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A2[t >> 2], B[t & 3], c, 0, 0, 0);
        return c;
      };
      v4f c[3];
      c[0] = dot(0);
      c[1] = dot(1);
#pragma unroll
      for (int t = 0; t < 16; t++) {
        if (t + 2 < 16) c[(t + 2) % 3] = dot(t + 2);
        const int i = t >> 2, j = t & 3;
#pragma unroll
        for (int r = 0; r < 4; r++)
          part[i][j][r] = first ? s[j] * c[t % 3][r] : fmaf(s[j], c[t % 3][r], part[i][j][r]);
      }
    };
    if (st % 4 == 0) block(0, std::true_type{});
    else block(0, std::false_type{});
    block(1, std::false_type{});
    if (st % 4 == 3) {  // the super-block's last stage: acc += d * part
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float4 d4 = *reinterpret_cast<const float4 *>(&dvr[wn + 16 * i + 4 * lq]);
        const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int r = 0; r < 4; r++) acc[i][j][r] = fmaf(dv[r], part[i][j][r], acc[i][j][r]);
      }
    }
    lds_wait_dma();
    if (st + 1 < st1) {
      wstore(st + 1);
      if ((st + 1) % 4 == 1) hstore((st + 1) / 4);
    }
    lds_barrier();
  }
  if (gridDim.z > 1 && !f16_split_merge<512>(acc, a)) return;
  const bool vec = (J.N & 3) == 0;
  // The rope epilogue's job: 0 q, 1 k, 2 v; 3 none (uniform).
  const uint32_t rj = !a.rope.tab ? 3 : J.y == a.jy[0] ? 0 : J.y == a.jy[1] ? 1 : 2;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t m = bm + wm + 16 * j + l16;
    if (m >= a.M) continue;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t n = bn + wn + 16 * i + 4 * lq;
      float *yp = J.y + (size_t)m * J.N + n;
      if (rj < 3) {  // N a multiple of hd, hd of 4: the 4 columns are 2 pairs of one head
        if (n >= J.N) continue;
        float r[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        if (rj < 2) {
          const uint32_t half = a.rope.hd / 2;
          const float4 cs =
              *reinterpret_cast<const float4 *>(a.rope.tab + 2 * ((size_t)(a.rope.pos + m) * half + (n % a.rope.hd) / 2));
          rot(r[0], r[1], cs.x, cs.y);
          rot(r[2], r[3], cs.z, cs.w);
        }
        if (rj == 0) {
          *reinterpret_cast<float4 *>(yp) = make_float4(r[0], r[1], r[2], r[3]);
        } else {
          uint16_t *d = (rj == 1 ? a.rope.dk : a.rope.dv) + (size_t)m * a.rope.kv_stride + n;
          const v4h h = {(_Float16)r[0], (_Float16)r[1], (_Float16)r[2], (_Float16)r[3]};
          *reinterpret_cast<v4h *>(d) = h;
        }
        continue;
      }
      if (vec && n + 3 < J.N) {
        *reinterpret_cast<float4 *>(yp) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
#pragma unroll
        for (int t = 0; t < 4; t++)
          if (n + t < J.N) yp[t] = acc[i][j][t];
      }
    }
  }
}

}  // namespace

bool gemm_f16_supported(int32_t dtype, int layout, uint64_t n_in, uint64_t n_out) {
  if (layout != MDMA_LAYOUT_GFX950 || (dtype != DT_Q4_K && dtype != DT_Q6_K)) return false;
  if (n_in % 256 || n_in > 32 * (uint64_t)MAX_BLOCKS) return false;
  // Weight offsets are 32-bit inside the kernel.
  return n_out * gfx950_row_bytes(dtype, n_in) < (1ull << 32);
}

namespace {
uint64_t r256(uint64_t b) { return (b + 255) / 256 * 256; }
}  // namespace

uint64_t gemm_f16_input_bytes(uint64_t M, uint64_t K) {
  return r256(M * K * 2) + r256(M * (K / 32) * 4) + 2 * r256(M * (K / 32) * 2) + r256(M * 4);
}

F16In gemm_f16_input_at(char *s, uint64_t M, uint64_t K) {
  const uint64_t nb = K / 32;
  F16In in;
  in.xh = reinterpret_cast<_Float16 *>(s);
  s += r256(M * K * 2);
  in.sx = reinterpret_cast<float *>(s);
  s += r256(M * nb * 4);
  in.ph = reinterpret_cast<_Float16 *>(s);
  s += r256(M * nb * 2);
  in.pl = reinterpret_cast<_Float16 *>(s);
  s += r256(M * nb * 2);
  in.inv = reinterpret_cast<float *>(s);
  return in;
}

void a16_mark(mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in, char *buf, bool with_p) {
  ctx->a16_valid = true;
  ctx->a16_p = with_p;
  ctx->a16_noy = false;
  ctx->a16_x = x;
  ctx->a16_buf = buf;
  ctx->a16_n = T * n_in;
  ctx->a16_n_in = n_in;
}

bool a16_holds(const mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in) {
  return ctx->a16_valid && ctx->a16_x == x && ctx->a16_n == T * n_in && ctx->a16_n_in == n_in;
}

namespace {
// Splits of K for a launch of few output tiles (few weight rows): enough
// workgroups for two per CU, whole super-blocks, at least two per split.
struct F16Split {
  uint32_t S, sbs;
};
F16Split f16_plan(const mdma_ctx *ctx, uint64_t tiles, uint64_t K) {
  const uint64_t cus = ctx->cu_count ? ctx->cu_count : 256, nsb = K / 256;
  if (tiles >= cus || nsb < 4) return F16Split{1, (uint32_t)nsb};
  const uint64_t S = std::min<uint64_t>(std::min<uint64_t>((2 * cus + tiles - 1) / tiles, nsb / 2), 16);
  const uint64_t sbs = (nsb + S - 1) / S;
  return F16Split{(uint32_t)((nsb + sbs - 1) / sbs), (uint32_t)sbs};
}
uint64_t rows_per_launch(uint64_t K) { return ((1ull << 31) / K) / TM * TM; }

// A launch's kernel: the wide Q6_K kernel (256 tokens per workgroup, one
// workgroup per CU) for Q6_K over more than 128 tokens, else 128 x 128
// tiles, two workgroups per CU.
struct F16Shape {
  bool wide;
  uint64_t tm;
};
F16Shape f16_shape(const GemvJob &w, uint64_t Mc) {
  const bool wide = w.dtype == DT_Q6_K && !w.dots && Mc > (uint64_t)TM;
  return F16Shape{wide, wide ? (uint64_t)TMW : (uint64_t)TM};
}
// The wide kernel's splits: its launches have half the tiles with one
// resident workgroup per CU, so the count keeps the launch's length lowest
// -- rounds of workgroups times a workgroup's super-blocks, plus one for a
// split's partial tile and merge, the fewer splits on a tie (3 splits of
// 96 tiles would be 288 workgroups on 256 CUs: a second round as long as
// the first).
F16Split f16_plan_for(const mdma_ctx *ctx, bool wide, uint64_t tiles, uint64_t K) {
  if (!wide) return f16_plan(ctx, tiles, K);
  const uint64_t cus = ctx->cu_count ? ctx->cu_count : 256, nsb = K / 256;
  F16Split best{1, (uint32_t)nsb};
  if (tiles >= cus || nsb < 4) return best;
  uint64_t best_cost = (tiles + cus - 1) / cus * nsb;
  for (uint64_t s = 2; s <= std::min<uint64_t>(nsb / 2, 16); s++) {
    const uint64_t sbs = (nsb + s - 1) / s, S = (nsb + sbs - 1) / sbs;
    const uint64_t cost = (tiles * S + cus - 1) / cus * (sbs + 1);
    if (cost < best_cost) best_cost = cost, best = F16Split{(uint32_t)S, (uint32_t)sbs};
  }
  return best;
}
}  // namespace

namespace {
// One launch's weights: the jobs fused into it (same type and shape of x, no
// block-dot capture), or the one job.
bool f16_fusable(const GemvJob *jobs, int n_jobs) {
  if (n_jobs < 2 || n_jobs > 3) return false;
  for (int i = 0; i < n_jobs; i++)
    if (jobs[i].dtype != jobs[0].dtype || jobs[i].n_in != jobs[0].n_in || jobs[i].dots) return false;
  return true;
}
uint64_t col_tiles(const GemvJob *jobs, int n) {
  uint64_t t = 0;
  for (int i = 0; i < n; i++) t += (jobs[i].n_out + TN - 1) / TN;
  return t;
}
}  // namespace

uint64_t gemm_f16_split_bytes(const mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, uint64_t M, uint64_t *tiles) {
  const uint64_t K = jobs[0].n_in, Mc = std::min(M, rows_per_launch(K));
  const int groups = f16_fusable(jobs, n_jobs) ? 1 : n_jobs;
  uint64_t bytes = 0;
  *tiles = 0;
  for (int g = 0; g < groups; g++) {
    const GemvJob *gj = groups == 1 ? jobs : jobs + g;
    const F16Shape sh = f16_shape(gj[0], Mc);
    const uint64_t t = col_tiles(gj, groups == 1 ? n_jobs : 1) * ((Mc + sh.tm - 1) / sh.tm);
    const F16Split sp = f16_plan_for(ctx, sh.wide, t, K);
    if (sp.S > 1) {
      bytes = std::max(bytes, t * sp.S * sh.tm * TN * 4);
      *tiles = std::max(*tiles, t);
    }
  }
  return bytes;
}

bool gemm_f16_glu_ok(const GemvJob &gate, const GemvJob &up) {
  const GemvJob gu[2] = {gate, up};
  return gate.dtype == DT_Q4_K && up.dtype == DT_Q4_K && gate.n_out == up.n_out && gate.n_out % TN == 0 &&
         f16_fusable(gu, 2);
}

void launch_gemm_f16(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t M, char *s,
                     float *part, uint64_t part_bytes, uint32_t *cnt, uint64_t counters, float *glu_y,
                     bool have_input) {
  const uint64_t K = jobs[0].n_in, nb = K / 32;
  const F16In in = gemm_f16_input_at(s, M, K);
  _Float16 *xh = in.xh, *ph = in.ph, *pl = in.pl;
  float *sx = in.sx, *inv = in.inv;
  if (!have_input) {
    gemm_act_kernel<<<dim3((uint32_t)M), dim3(256), 0, ctx->stream>>>(x, (uint32_t)K, xh, sx, ph, pl, inv);
    hip_check(hipGetLastError(), "gemm activation launch");
  }
  // Token rows per launch: activation offsets are 32-bit inside the kernel.
  const uint64_t rows = rows_per_launch(K);
  hipEvent_t t0 = ctx->time_start, t1 = ctx->time_stop;
  ctx->time_start = ctx->time_stop = nullptr;
  const bool fused = f16_fusable(jobs, n_jobs);
  const int groups = fused ? 1 : n_jobs;
  const bool glu = glu_y != nullptr;
  if (glu && (n_jobs != 2 || !gemm_f16_glu_ok(jobs[0], jobs[1]))) fail(MDMA_ERR_BACKEND, "gated GEMM: jobs not fusable");
  // A request (a16_want) for the gated output's GEMM input (no min-term
  // sums) in the caller's buffer.
  const bool want = glu && ctx->a16_want_y == glu_y && ctx->a16_want_bytes >= gemm_f16_input_bytes(M, jobs[0].n_out);
  const F16In want_in = want ? gemm_f16_input_at(ctx->a16_want_buf, M, jobs[0].n_out) : F16In{};
  // A request (rope_want) for RoPE and the K/V cache write in the fused QKV
  // launch: Q6_K q, k, v in one wide launch per row chunk.
  const uint32_t rhd = ctx->rope_want_hd;
  bool rope = fused && n_jobs == 3 && ctx->rope_want_q == jobs[0].y && rhd && rhd % 4 == 0 &&
              ctx->rope_want_stride % 4 == 0 && jobs[1].n_out == jobs[2].n_out && jobs[1].n_out <= ctx->rope_want_stride;
  for (int j = 0; rope && j < 3; j++)
    rope = jobs[j].dtype == DT_Q6_K && !jobs[j].dots && jobs[j].n_out % rhd == 0;
  for (uint64_t m0 = 0; rope && m0 < M; m0 += rows) rope = f16_shape(jobs[0], std::min(M - m0, rows)).wide;
  for (int g = 0; g < groups; g++) {
    const GemvJob *gj = fused ? jobs : jobs + g;
    const int nj = fused ? n_jobs : 1;
    const GemvJob &w = gj[0];
    for (uint64_t m0 = 0; m0 < M; m0 += rows) {
      const uint64_t Mc = M - m0 < rows ? M - m0 : rows;
      // Split K when the launch has few tiles and the partials fit (not for
      // the block-dot capture, whose dots are stored by the one split).
      const F16Shape sh = f16_shape(w, Mc);
      const uint64_t ct = col_tiles(gj, nj), mt = (Mc + sh.tm - 1) / sh.tm, tiles = ct * mt;
      F16Split sp = f16_plan_for(ctx, sh.wide, tiles, K);
      if (sp.S > 1 && (w.dots || !part || !cnt || tiles > counters || tiles * sp.S * sh.tm * TN * 4 > part_bytes))
        sp = F16Split{1, (uint32_t)(K / 256)};
      F16Args a{xh + m0 * K, sx + m0 * nb, ph + m0 * nb, (uint32_t)(pl - ph), inv + m0, w.w, w.y + m0 * w.n_out,
                (uint32_t)Mc, (uint32_t)w.n_out, (uint32_t)K, gfx950_row_bytes(w.dtype, K),
                w.dots ? w.dots + m0 * w.n_out * (K / 32) : nullptr, sp.S > 1 ? part : nullptr,
                sp.S > 1 ? cnt : nullptr, sp.sbs, (uint32_t)nj, {}, {}, {}, {}, glu ? glu_y + m0 * w.n_out : nullptr};
      if (rope) {
        a.rope.tab = ctx->rope_want_tab;
        a.rope.dk = ctx->rope_want_dk + m0 * ctx->rope_want_stride;
        a.rope.dv = ctx->rope_want_dv + m0 * ctx->rope_want_stride;
        a.rope.pos = ctx->rope_want_pos + (uint32_t)m0;
        a.rope.hd = rhd;
        a.rope.kv_stride = ctx->rope_want_stride;
      }
      if (glu && want) {
        a.glu_no_y = ctx->a16_want_input_only;
        a.glu_in = want_in;
        a.glu_in.xh += m0 * w.n_out;
        a.glu_in.sx += m0 * (w.n_out / 32);
      }
      uint32_t first = 0;
      for (int j = 0; j < nj; j++) {
        a.jw[j] = gj[j].w;
        a.jy[j] = gj[j].y + m0 * gj[j].n_out;
        a.jn[j] = (uint32_t)gj[j].n_out;
        a.jt[j] = first;
        first += (uint32_t)((gj[j].n_out + TN - 1) / TN);
      }
      // (A gated launch has the same number of column tiles: 64 rows of
      // both weights each, N a multiple of 128.)
      const dim3 grid((uint32_t)ct, (uint32_t)mt, sp.S), block(sh.wide ? 512 : 256);
      // Timing events bracket the calls' GEMM launches (not the prologue).
      const hipEvent_t e0 = g == 0 && m0 == 0 ? t0 : nullptr, e1 = g == groups - 1 && m0 + Mc >= M ? t1 : nullptr;
      if (w.dtype == DT_Q6_K && sh.wide) {
        if (e0 || e1) hipExtLaunchKernelGGL(gemm_f16_q6w_kernel, grid, block, 0, ctx->stream, e0, e1, 0, a);
        else gemm_f16_q6w_kernel<<<grid, block, 0, ctx->stream>>>(a);
      } else if (w.dtype == DT_Q6_K) {
        if (e0 || e1) hipExtLaunchKernelGGL(gemm_f16_q6_kernel, grid, block, 0, ctx->stream, e0, e1, 0, a);
        else gemm_f16_q6_kernel<<<grid, block, 0, ctx->stream>>>(a);
      } else if (glu) {
        if (e0 || e1) hipExtLaunchKernelGGL(gemm_f16_kernel<DT_Q4_K, false, true>, grid, block, 0, ctx->stream, e0, e1, 0, a);
        else gemm_f16_kernel<DT_Q4_K, false, true><<<grid, block, 0, ctx->stream>>>(a);
      } else if (a.dots) gemm_f16_kernel<DT_Q4_K, true><<<grid, block, 0, ctx->stream>>>(a);
      else if (e0 || e1) hipExtLaunchKernelGGL(gemm_f16_kernel<DT_Q4_K>, grid, block, 0, ctx->stream, e0, e1, 0, a);
      else gemm_f16_kernel<DT_Q4_K><<<grid, block, 0, ctx->stream>>>(a);
      hip_check(hipGetLastError(), "gemm f16 launch");
    }
  }
  if (want) {
    a16_mark(ctx, glu_y, M, jobs[0].n_out, ctx->a16_want_buf, false);
    ctx->a16_noy = ctx->a16_want_input_only;
  }
  if (rope) ctx->rope_done = true;
}

}  // namespace mdma
