// gfx950 prepared weight layouts: a lossless re-arrangement of GGUF
// Q4_K / Q6_K / Q8_0 rows so that every 16-byte load instruction of a wave
// reads 64 consecutive 16-byte chunks (lane i at byte 16*i of a plane).
//
// This is the backend-private layout hook of the reference
// (WeightLayout, /root/reference/src/cache/layout.rs:10-38, and
// Backend::upload_weight, src/backend.rs:228-237), whose ROCm backend keeps
// its own Q4_K plane layout (pack_q4k, src/cache/layout.rs:40-79). The
// layout here is designed for wave64 streaming instead: a row is split into
// planes indexed by 64-column "units" (32 for Q8_0), the unit a lane owns.
//
// Rows follow one another, each padded to a multiple of 16 bytes:
//   Q4_K (nb blocks, U = 4 nb units, unit u = sub-block pair p = u%4 of
//         block b = u/4):
//         A[U][16]  quant bytes [32p, 32p+16) of block b
//         B[U][16]  quant bytes [32p+16, 32p+32)
//         H[nb][16] the block header (f16 d, f16 dmin, 12 scale bytes)
//   Q6_K (U = 4 nb units, unit u = (half n, column group h), u%4 = 2n+h):
//         A[U][16]  ql[64n + 16h .. +16]        (quarters 0 and 2)
//         B[U][16]  ql[64n + 32 + 16h .. +16]   (quarters 1 and 3)
//         Q[U][16]  qh[32n + 16h .. +16]
//         S[U][4]   sc[8n + 2r + h], r = 0..3
//         D[nb][2]  f16 d
//   Q8_0 (U = nb units of one block):
//         A[nb][16] quants [0, 16), B[nb][16] quants [16, 32), D[nb][2] f16 d
// Every block keeps its byte count (144, 210, 34); only the row padding is
// added (none when the row is already a multiple of 16 bytes, as at every
// Llama-3-8B shape).
#include <hip/hip_runtime.h>

#include <cstring>

#include "internal.h"

namespace mdma {

uint64_t gfx950_row_bytes(int32_t dtype, uint64_t cols) {
  const uint64_t bs = block_size(dtype);
  if (!bs || cols % bs) return 0;
  const uint64_t raw = cols / bs * type_size(dtype);
  return (raw + 15) / 16 * 16;
}

bool gfx950_layout_dtype(int32_t dtype) { return dtype == DT_Q4_K || dtype == DT_Q6_K || dtype == DT_Q8_0; }

void pack_gfx950(int32_t dtype, uint64_t rows, uint64_t cols, const uint8_t *src, uint8_t *dst) {
  const uint64_t nb = cols / block_size(dtype), ts = type_size(dtype), rbp = gfx950_row_bytes(dtype, cols);
  for (uint64_t r = 0; r < rows; r++) {
    const uint8_t *s = src + r * nb * ts;
    uint8_t *d = dst + r * rbp;
    std::memset(d + nb * ts, 0, rbp - nb * ts);
    if (dtype == DT_Q4_K) {
      const uint64_t U = 4 * nb;
      for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = s + b * 144;
        for (int p = 0; p < 4; p++) {
          std::memcpy(d + 16 * (4 * b + p), blk + 16 + 32 * p, 16);
          std::memcpy(d + 16 * (U + 4 * b + p), blk + 32 + 32 * p, 16);
        }
        std::memcpy(d + 32 * U + 16 * b, blk, 16);
      }
    } else if (dtype == DT_Q6_K) {
      const uint64_t U = 4 * nb;
      for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = s + b * 210, *ql = blk, *qh = blk + 128, *sc = blk + 192;
        for (int k = 0; k < 4; k++) {
          const int n = k >> 1, h = k & 1;
          const uint64_t u = 4 * b + k;
          std::memcpy(d + 16 * u, ql + 64 * n + 16 * h, 16);
          std::memcpy(d + 16 * (U + u), ql + 64 * n + 32 + 16 * h, 16);
          std::memcpy(d + 16 * (2 * U + u), qh + 32 * n + 16 * h, 16);
          for (int q = 0; q < 4; q++) d[48 * U + 4 * u + q] = sc[8 * n + 2 * q + h];
        }
        std::memcpy(d + 52 * U + 2 * b, blk + 208, 2);
      }
    } else {  // Q8_0
      for (uint64_t b = 0; b < nb; b++) {
        const uint8_t *blk = s + b * 34;
        std::memcpy(d + 16 * b, blk + 2, 16);
        std::memcpy(d + 16 * (nb + b), blk + 18, 16);
        std::memcpy(d + 32 * nb + 2 * b, blk, 2);
      }
    }
  }
}

namespace {

__device__ __forceinline__ void copy_bytes(uint8_t *d, const uint8_t *s, int n) {
  for (int i = 0; i < n; i++) d[i] = s[i];
}

// pack_gfx950's byte moves for one (row, block), one thread each; the
// thread of a row's block 0 also clears the row's padding.
__global__ __launch_bounds__(256) void repack_kernel(int32_t dtype, uint64_t rows, uint64_t nb, uint32_t ts,
                                                     uint64_t rbp, const uint8_t *__restrict__ src,
                                                     uint8_t *__restrict__ dst) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nb) return;
  const uint64_t r = i / nb, b = i % nb;
  const uint8_t *blk = src + i * ts;
  uint8_t *d = dst + r * rbp;
  if (b == 0)
    for (uint64_t k = nb * ts; k < rbp; k++) d[k] = 0;
  if (dtype == DT_Q4_K) {
    const uint64_t U = 4 * nb;
    for (int p = 0; p < 4; p++) {
      copy_bytes(d + 16 * (4 * b + p), blk + 16 + 32 * p, 16);
      copy_bytes(d + 16 * (U + 4 * b + p), blk + 32 + 32 * p, 16);
    }
    copy_bytes(d + 32 * U + 16 * b, blk, 16);
  } else if (dtype == DT_Q6_K) {
    const uint64_t U = 4 * nb;
    const uint8_t *ql = blk, *qh = blk + 128, *sc = blk + 192;
    for (int k = 0; k < 4; k++) {
      const int n = k >> 1, h = k & 1;
      const uint64_t u = 4 * b + k;
      copy_bytes(d + 16 * u, ql + 64 * n + 16 * h, 16);
      copy_bytes(d + 16 * (U + u), ql + 64 * n + 32 + 16 * h, 16);
      copy_bytes(d + 16 * (2 * U + u), qh + 32 * n + 16 * h, 16);
      for (int q = 0; q < 4; q++) d[48 * U + 4 * u + q] = sc[8 * n + 2 * q + h];
    }
    copy_bytes(d + 52 * U + 2 * b, blk + 208, 2);
  } else {
    copy_bytes(d + 16 * b, blk + 2, 16);
    copy_bytes(d + 16 * (nb + b), blk + 18, 16);
    copy_bytes(d + 32 * nb + 2 * b, blk, 2);
  }
}

}  // namespace

void launch_repack(mdma_ctx *ctx, int32_t dtype, uint64_t rows, uint64_t cols, const uint8_t *src, uint8_t *dst) {
  const uint64_t nb = cols / block_size(dtype), total = rows * nb;
  if (!total) return;
  repack_kernel<<<dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, ctx->stream>>>(
      dtype, rows, nb, (uint32_t)type_size(dtype), gfx950_row_bytes(dtype, cols), src, dst);
  hip_check(hipGetLastError(), "repack launch");
}

void unpack_gfx950(int32_t dtype, uint64_t rows, uint64_t cols, const uint8_t *src, uint8_t *dst) {
  const uint64_t nb = cols / block_size(dtype), ts = type_size(dtype), rbp = gfx950_row_bytes(dtype, cols);
  for (uint64_t r = 0; r < rows; r++) {
    const uint8_t *s = src + r * rbp;
    uint8_t *d = dst + r * nb * ts;
    if (dtype == DT_Q4_K) {
      const uint64_t U = 4 * nb;
      for (uint64_t b = 0; b < nb; b++) {
        uint8_t *blk = d + b * 144;
        for (int p = 0; p < 4; p++) {
          std::memcpy(blk + 16 + 32 * p, s + 16 * (4 * b + p), 16);
          std::memcpy(blk + 32 + 32 * p, s + 16 * (U + 4 * b + p), 16);
        }
        std::memcpy(blk, s + 32 * U + 16 * b, 16);
      }
    } else if (dtype == DT_Q6_K) {
      const uint64_t U = 4 * nb;
      for (uint64_t b = 0; b < nb; b++) {
        uint8_t *blk = d + b * 210, *ql = blk, *qh = blk + 128, *sc = blk + 192;
        for (int k = 0; k < 4; k++) {
          const int n = k >> 1, h = k & 1;
          const uint64_t u = 4 * b + k;
          std::memcpy(ql + 64 * n + 16 * h, s + 16 * u, 16);
          std::memcpy(ql + 64 * n + 32 + 16 * h, s + 16 * (U + u), 16);
          std::memcpy(qh + 32 * n + 16 * h, s + 16 * (2 * U + u), 16);
          for (int q = 0; q < 4; q++) sc[8 * n + 2 * q + h] = s[48 * U + 4 * u + q];
        }
        std::memcpy(blk + 208, s + 52 * U + 2 * b, 2);
      }
    } else {
      for (uint64_t b = 0; b < nb; b++) {
        uint8_t *blk = d + b * 34;
        std::memcpy(blk + 2, s + 16 * b, 16);
        std::memcpy(blk + 18, s + 16 * (nb + b), 16);
        std::memcpy(blk, s + 32 * nb + 2 * b, 2);
      }
    }
  }
}

}  // namespace mdma
