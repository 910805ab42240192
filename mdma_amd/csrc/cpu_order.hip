// The CPU-order mode (MDMA_ACT_F32_CPU): the quantized matmul and the ops
// around it computed in the reference CPU backend's arithmetic order, so
// their results are the CPU backend's bit for bit.
//
// CpuBackend::qmatmul (/root/reference/src/backend/cpu.rs:46-48,335-368):
// each row is dequantized to f32 (candle's to_float, called from
// src/backend/cpu/dequant.rs:36) and every output is a sequential f32 sum,
// starting from -0.0, of the f32-rounded products w_i * x_i, never fused
// into an FMA. A sum in that order is one dependent chain, so here one lane
// owns one output row (and up to 8 tokens' chains of it); rows run in
// parallel, the columns of a row in order.
//
// The dequantized weights are exact products (the values match candle's in
// any evaluation order): Q8_0 q * d has 8 + 11 significant bits; Q6_K
// (d * sc) * q at most 11 + 7 + 5 < 24; Q4_K d * sc and dmin * m have at most
// 17 bits and (d * sc) * q 21, so only the final subtraction d*sc*q - dmin*m
// rounds, once.
//
// rmsnorm (cpu.rs:388-402), silu_mul (:447-458) and attention (:530-590,
// softmax_inplace :50-60) follow the CPU's sequence of roundings too:
// sequential sums, correctly rounded division and square root (formed in
// double and rounded once to f32, which for one operation on f32 operands
// gives the correctly rounded f32 result), and the C library's expf
// (libm_expf.h). The file is compiled with `fp contract(off)`: no f32
// multiply-add is fused.
#include <algorithm>

#include "internal.h"
#include "kernels.h"
#include "libm_expf.h"

// No f32 multiply and add in this file is fused into an FMA.
#pragma clang fp contract(off)

namespace mdma {
namespace {

// Correctly rounded f32 division and square root.
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }
__device__ __forceinline__ float sqrt_rn(float a) { return (float)__builtin_sqrt((double)a); }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 0xffu; }

// One group of a row's weights in registers, in GGUF byte order whatever
// the buffer's layout (layout.cpp's planes are gathered back), and its
// dequantized element e. GC: columns per group.
template <int DT>
struct Group;

template <>
struct Group<DT_Q4_K> {
  static constexpr int GC = 256;
  uint4 hd;       // f16 d, f16 dmin, 12 scale bytes
  uint32_t q[32];  // 128 quant bytes
  float d1[8], m1[8];
  __device__ __forceinline__ void load(const uint8_t *wr, uint32_t nb, uint32_t b, bool prepared) {
    if (prepared) {
      const uint32_t U = 4 * nb;
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint4 a = ldx16(wr + 16 * (4 * b + p)), c = ldx16(wr + 16 * (U + 4 * b + p));
        q[8 * p + 0] = a.x, q[8 * p + 1] = a.y, q[8 * p + 2] = a.z, q[8 * p + 3] = a.w;
        q[8 * p + 4] = c.x, q[8 * p + 5] = c.y, q[8 * p + 6] = c.z, q[8 * p + 7] = c.w;
      }
      hd = ldx16(wr + 32 * U + 16 * b);
    } else {
      const uint8_t *blk = wr + 144 * (size_t)b;
      hd = ldx16(blk);
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const uint4 a = ldx16(blk + 16 + 16 * k);
        q[4 * k + 0] = a.x, q[4 * k + 1] = a.y, q[4 * k + 2] = a.z, q[4 * k + 3] = a.w;
      }
    }
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
#pragma unroll
    for (int p = 0; p < 4; p++) {
      int sca, scb, ma, mb;
      q4k_scales_i(hd, p, sca, scb, ma, mb);
      d1[2 * p] = d * (float)sca, m1[2 * p] = dmin * (float)ma;
      d1[2 * p + 1] = d * (float)scb, m1[2 * p + 1] = dmin * (float)mb;
    }
  }
  // Column e: sub-block s = e / 32, pair j = e / 64, byte 32 j + e % 32,
  // the low nibble for even s, the high one for odd.
  __device__ __forceinline__ float deq(int e) const {
#pragma clang fp contract(off)
    const int s = e / 32, j = e / 64, byte = 32 * j + e % 32;
    const uint32_t qv = (byte_of(q[byte / 4], byte % 4) >> (4 * (s & 1))) & 0xF;
    const float t = d1[s] * (float)qv;
    return t - m1[s];
  }
};

template <>
struct Group<DT_Q6_K> {
  static constexpr int GC = 256;
  uint32_t ql[32], qh[16];
  uint32_t scw[2][2];  // scw[n][h] byte r: the scale of quarter r, columns 128 n + 32 r + 16 h ..
  float d;
  __device__ __forceinline__ void load(const uint8_t *wr, uint32_t nb, uint32_t b, bool prepared) {
    if (prepared) {
      const uint32_t U = 4 * nb;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int n = k >> 1, h = k & 1;
        const uint32_t u = 4 * b + k;
        const uint4 a = ldx16(wr + 16 * u), c = ldx16(wr + 16 * (U + u)), e = ldx16(wr + 16 * (2 * U + u));
        const int qa = 16 * n + 4 * h, qb = 16 * n + 8 + 4 * h, hh = 8 * n + 4 * h;
        ql[qa] = a.x, ql[qa + 1] = a.y, ql[qa + 2] = a.z, ql[qa + 3] = a.w;
        ql[qb] = c.x, ql[qb + 1] = c.y, ql[qb + 2] = c.z, ql[qb + 3] = c.w;
        qh[hh] = e.x, qh[hh + 1] = e.y, qh[hh + 2] = e.z, qh[hh + 3] = e.w;
        scw[n][h] = *reinterpret_cast<const uint32_t *>(wr + 48 * U + 4 * u);
      }
      d = h2f(ldu16(wr + 52 * U + 2 * b));
    } else {
      const uint8_t *blk = wr + 210 * (size_t)b;  // 2-byte aligned
#pragma unroll
      for (int k = 0; k < 32; k++) ql[k] = ld2x16(blk + 4 * k);
#pragma unroll
      for (int k = 0; k < 16; k++) qh[k] = ld2x16(blk + 128 + 4 * k);
      uint32_t sc[4];
#pragma unroll
      for (int k = 0; k < 4; k++) sc[k] = ld2x16(blk + 192 + 4 * k);
      // scw[n][h] byte r = sc[8 n + 2 r + h]
#pragma unroll
      for (int n = 0; n < 2; n++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          uint32_t w = 0;
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int i = 8 * n + 2 * r + h;
            w |= byte_of(sc[i / 4], i % 4) << (8 * r);
          }
          scw[n][h] = w;
        }
      d = h2f(ldu16(blk + 208));
    }
  }
  // Column e = 128 n + 32 r + l: low 4 bits from ql[64 n + 32 (r & 1) + l]
  // (low nibble for r < 2), high 2 bits from qh[32 n + l] >> 2 r, scale
  // sc[8 n + 2 r + l / 16]; the value (d * sc) * (q - 32).
  __device__ __forceinline__ float deq(int e) const {
#pragma clang fp contract(off)
    const int n = e / 128, r = (e % 128) / 32, l = e % 32, h = l / 16;
    const int lb = 64 * n + 32 * (r & 1) + l, hb = 32 * n + l;
    const uint32_t low = (byte_of(ql[lb / 4], lb % 4) >> (r < 2 ? 0 : 4)) & 0xF;
    const uint32_t high = (byte_of(qh[hb / 4], hb % 4) >> (2 * r)) & 3;
    const int qv = (int)(low | (high << 4)) - 32;
    const int sc = (int)(int8_t)byte_of(scw[n][h], r);
    const float ds = d * (float)sc;
    return ds * (float)qv;
  }
};

template <>
struct Group<DT_Q8_0> {
  static constexpr int GC = 32;
  uint32_t q[8];
  float d;
  __device__ __forceinline__ void load(const uint8_t *wr, uint32_t nb, uint32_t b, bool prepared) {
    if (prepared) {
      const uint4 a = ldx16(wr + 16 * b), c = ldx16(wr + 16 * (nb + b));
      q[0] = a.x, q[1] = a.y, q[2] = a.z, q[3] = a.w, q[4] = c.x, q[5] = c.y, q[6] = c.z, q[7] = c.w;
      d = h2f(ldu16(wr + 32 * nb + 2 * b));
    } else {
      const uint8_t *blk = wr + 34 * (size_t)b;  // 2-byte aligned
#pragma unroll
      for (int k = 0; k < 8; k++) q[k] = ld2x16(blk + 2 + 4 * k);
      d = h2f(ldu16(blk));
    }
  }
  __device__ __forceinline__ float deq(int e) const {
#pragma clang fp contract(off)
    const int qv = (int)(int8_t)byte_of(q[e / 4], e % 4);
    return (float)qv * d;
  }
};

constexpr int SEQ_TT = 8;  // token chains per lane for calls of more than one token

// y[t, row] for rows blockIdx.x * 64 + lane and tokens blockIdx.y * TT ..:
// the sequential sums. x is staged one group at a time into LDS (every lane
// then reads the same word: a broadcast).
template <int DT, int TT>
__global__ __launch_bounds__(64) void gemv_seq_kernel(const uint8_t *__restrict__ w, uint64_t row_bytes,
                                                      uint32_t n_out, uint32_t n_in, bool prepared,
                                                      const float *__restrict__ x, uint32_t T,
                                                      float *__restrict__ y) {
#pragma clang fp contract(off)
  constexpr int GC = Group<DT>::GC;
  __shared__ __attribute__((aligned(16))) float xs[TT][GC];
  const uint32_t lane = threadIdx.x, row = blockIdx.x * 64 + lane, t0 = blockIdx.y * TT;
  const uint8_t *wr = w + (size_t)min(row, n_out - 1) * row_bytes;
  const uint32_t ng = n_in / GC;
  float s[TT];
#pragma unroll
  for (int k = 0; k < TT; k++) s[k] = -0.0f;
  for (uint32_t g = 0; g < ng; g++) {
    Group<DT> grp;
    grp.load(wr, ng, g, prepared);
    __syncthreads();  // the previous group's reads of xs are done
    for (uint32_t i = lane; i < TT * GC / 4; i += 64) {
      const uint32_t k = i / (GC / 4), c = i % (GC / 4), t = min(t0 + k, T - 1);
      *reinterpret_cast<float4 *>(&xs[k][4 * c]) =
          *reinterpret_cast<const float4 *>(x + (size_t)t * n_in + (size_t)g * GC + 4 * c);
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < GC; e++) {
      const float wv = grp.deq(e);
#pragma unroll
      for (int k = 0; k < TT; k++) {
        const float p = wv * xs[k][e];
        s[k] = s[k] + p;
      }
    }
  }
  if (row < n_out) {
#pragma unroll
    for (int k = 0; k < TT; k++)
      if (t0 + k < T) y[(size_t)(t0 + k) * n_out + row] = s[k];
  }
}

// Float weights (F32, F16): the row read element by element, x from global
// memory (uniform addresses).
template <int DT, int TT>
__global__ __launch_bounds__(64) void gemv_seq_float_kernel(const uint8_t *__restrict__ w, uint32_t n_out,
                                                            uint32_t n_in, const float *__restrict__ x, uint32_t T,
                                                            float *__restrict__ y) {
#pragma clang fp contract(off)
  const uint32_t lane = threadIdx.x, row = blockIdx.x * 64 + lane, t0 = blockIdx.y * TT;
  const size_t r = min(row, n_out - 1);
  float s[TT];
  const float *xr[TT];
#pragma unroll
  for (int k = 0; k < TT; k++) s[k] = -0.0f, xr[k] = x + (size_t)min(t0 + k, T - 1) * n_in;
  for (uint32_t i = 0; i < n_in; i++) {
    const float wv = DT == DT_F32 ? reinterpret_cast<const float *>(w)[r * n_in + i]
                                  : h2f(reinterpret_cast<const uint16_t *>(w)[r * n_in + i]);
#pragma unroll
    for (int k = 0; k < TT; k++) {
      const float p = wv * xr[k][i];
      s[k] = s[k] + p;
    }
  }
  if (row < n_out) {
#pragma unroll
    for (int k = 0; k < TT; k++)
      if (t0 + k < T) y[(size_t)(t0 + k) * n_out + row] = s[k];
  }
}

// rmsnorm (cpu.rs:388-402) of one row per workgroup, optionally after the
// residual add (Backend::add_rmsnorm default, src/backend.rs:502-513: sum =
// a + b, then rmsnorm of the sum): lane 0 forms the sequential sum of
// squares (dot(row, row), from -0.0), then every lane its outputs
// (row[i] * scale) * w[i] with scale = 1 / sqrt(mean + eps).
__global__ __launch_bounds__(256) void rmsnorm_seq_kernel(const float *__restrict__ w, uint32_t dim,
                                                          const float *__restrict__ a, const float *__restrict__ b,
                                                          float *__restrict__ sum, float *__restrict__ y, float eps) {
#pragma clang fp contract(off)
  __shared__ float scale_sh;
  const size_t base = (size_t)blockIdx.x * dim;
  const float *ar = a + base, *br = b ? b + base : nullptr;
  if (threadIdx.x == 0) {
    float ss = -0.0f;
    for (uint32_t i = 0; i < dim; i++) {
      const float v = br ? ar[i] + br[i] : ar[i];
      const float p = v * v;
      ss = ss + p;
    }
    const float mean = div_rn(ss, (float)dim);
    scale_sh = div_rn(1.0f, sqrt_rn(mean + eps));
  }
  __syncthreads();
  const float scale = scale_sh;
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) {
    const float v = br ? ar[i] + br[i] : ar[i];
    if (sum) sum[base + i] = v;
    const float t = v * scale;
    y[base + i] = t * w[i];
  }
}

// silu_mul (cpu.rs:447-458): y = (g / (1 + exp(-g))) * u.
__global__ void silu_mul_seq_kernel(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ y,
                                    size_t n) {
#pragma clang fp contract(off)
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float gv = g[i];
    const float den = 1.0f + libm_expf(-gv);
    const float s = div_rn(gv, den);
    y[i] = s * u[i];
  }
}

// Attention (cpu.rs:437-445,530-590 with softmax_inplace :50-60) of one
// (query, query head) per workgroup over the f16 cache (its values widen to
// f32 exactly): scores[t] = dot(q, k_t) * scale (sequential over head_dim,
// from -0.0); mx = max over the scores from -inf (a maximum in any order);
// e_t = expf(s_t - mx); their sum from +0.0 in key order (one lane); p_t =
// e_t / sum; o[d] = the sequential sum from +0.0 of p_t * v_t[d] in key
// order (one lane per dim). The scores live in `sc`, a slice of kv_cap
// floats per (query, head). pos_dev (a captured decode step): one query per
// sequence at position *pos_dev, which sees keys [0, *pos_dev].
__global__ __launch_bounds__(256) void attn_seq_kernel(const float *__restrict__ q, const uint16_t *__restrict__ K,
                                                       const uint16_t *__restrict__ V, float *__restrict__ o,
                                                       float *__restrict__ sc, uint32_t kv_cap, uint32_t prefix,
                                                       uint32_t hd, uint32_t n_q_heads, uint32_t n_kv_heads,
                                                       float scale, uint64_t seq_stride,
                                                       const uint32_t *__restrict__ pos_dev) {
#pragma clang fp contract(off)
  __shared__ float qs[256];
  __shared__ float red[4];
  __shared__ float sum_sh;
  const uint32_t qh = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
  if (pos_dev) prefix = *pos_dev;
  const uint32_t kvh = qh / (n_q_heads / n_kv_heads), kv_row = n_kv_heads * hd;
  const uint32_t visible = seq_stride ? prefix + 1 : prefix + i + 1;
  K += (size_t)i * seq_stride + (size_t)kvh * hd;
  V += (size_t)i * seq_stride + (size_t)kvh * hd;
  float *s = sc + ((size_t)i * n_q_heads + qh) * kv_cap;
  const float *qv = q + ((size_t)i * n_q_heads + qh) * hd;
  for (uint32_t d = tid; d < hd; d += 256) qs[d] = qv[d];
  __syncthreads();
  float mx = -INFINITY;
  for (uint32_t t = tid; t < visible; t += 256) {
    const uint16_t *kr = K + (size_t)t * kv_row;
    float acc = -0.0f;
    for (uint32_t d = 0; d < hd; d++) {
      const float p = qs[d] * h2f(kr[d]);
      acc = acc + p;
    }
    const float v = acc * scale;
    s[t] = v;
    mx = fmaxf(mx, v);
  }
  // The maximum over the block (fmaxf is exact and ignores NaN in any order).
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  for (uint32_t t = tid; t < visible; t += 256) s[t] = libm_expf(s[t] - mx);
  __syncthreads();
  if (tid == 0) {
    float total = 0.0f;
    for (uint32_t t = 0; t < visible; t++) total = total + s[t];
    sum_sh = total;
  }
  __syncthreads();
  const float total = sum_sh;
  for (uint32_t t = tid; t < visible; t += 256) s[t] = div_rn(s[t], total);
  __syncthreads();
  for (uint32_t d = tid; d < hd; d += 256) {
    float acc = 0.0f;
    for (uint32_t t = 0; t < visible; t++) {
      const float p = s[t] * h2f(V[(size_t)t * kv_row + d]);
      acc = acc + p;
    }
    o[((size_t)i * n_q_heads + qh) * hd + d] = acc;
  }
}

}  // namespace

void launch_gemv_seq(mdma_ctx *ctx, const GemvJob &j, const float *x, uint64_t T) {
  if (!T || !j.n_out) return;
  if (j.n_out > 0xffffffffull || j.n_in > 0xffffffffull || T > 0xffffffffull)
    shape_fail("qmatmul (cpu order): dimensions past 32 bits");
  const bool prepared = j.layout == MDMA_LAYOUT_GFX950;
  const uint64_t row_bytes = prepared ? gfx950_row_bytes(j.dtype, j.n_in)
                                      : j.n_in / block_size(j.dtype) * type_size(j.dtype);
  const uint32_t gx = (uint32_t)((j.n_out + 63) / 64);
  const uint32_t n_out = (uint32_t)j.n_out, n_in = (uint32_t)j.n_in, t = (uint32_t)T;
#define MDMA_SEQ_GO(KERNEL, TT, ...)                                                                          \
  KERNEL<<<dim3(gx, (uint32_t)((T + TT - 1) / TT)), dim3(64), 0, ctx->stream>>>(__VA_ARGS__)
#define MDMA_SEQ_Q(DT)                                                                                     \
  do {                                                                                                     \
    if ((DT == DT_Q8_0 ? j.n_in % 32 : j.n_in % 256) || (j.n_in % 4))                                     \
      shape_fail("qmatmul (cpu order): rows must be whole blocks");                                        \
    if (T == 1) MDMA_SEQ_GO((gemv_seq_kernel<DT, 1>), 1, j.w, row_bytes, n_out, n_in, prepared, x, t, j.y); \
    else MDMA_SEQ_GO((gemv_seq_kernel<DT, SEQ_TT>), SEQ_TT, j.w, row_bytes, n_out, n_in, prepared, x, t, j.y); \
  } while (0)
  switch (j.dtype) {
    case DT_Q4_K: MDMA_SEQ_Q(DT_Q4_K); break;
    case DT_Q6_K: MDMA_SEQ_Q(DT_Q6_K); break;
    case DT_Q8_0: MDMA_SEQ_Q(DT_Q8_0); break;
    case DT_F32:
      if (T == 1) MDMA_SEQ_GO((gemv_seq_float_kernel<DT_F32, 1>), 1, j.w, n_out, n_in, x, t, j.y);
      else MDMA_SEQ_GO((gemv_seq_float_kernel<DT_F32, SEQ_TT>), SEQ_TT, j.w, n_out, n_in, x, t, j.y);
      break;
    case DT_F16:
      if (T == 1) MDMA_SEQ_GO((gemv_seq_float_kernel<DT_F16, 1>), 1, j.w, n_out, n_in, x, t, j.y);
      else MDMA_SEQ_GO((gemv_seq_float_kernel<DT_F16, SEQ_TT>), SEQ_TT, j.w, n_out, n_in, x, t, j.y);
      break;
    default: fail(MDMA_ERR_NOT_IMPLEMENTED, "qmatmul (cpu order): unsupported weight dtype");
  }
#undef MDMA_SEQ_Q
#undef MDMA_SEQ_GO
  hip_check(hipGetLastError(), "gemv_seq launch");
}

void launch_rmsnorm_seq(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                        float *y, uint64_t rows, float eps) {
  if (!rows) return;
  rmsnorm_seq_kernel<<<dim3((uint32_t)rows), dim3(256), 0, ctx->stream>>>(w, (uint32_t)dim, a, b, sum, y, eps);
  hip_check(hipGetLastError(), "rmsnorm_seq launch");
}

void launch_silu_mul_seq(mdma_ctx *ctx, const float *g, const float *u, float *y, uint64_t n) {
  if (!n) return;
  const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 65536);
  silu_mul_seq_kernel<<<dim3((uint32_t)blocks), dim3(256), 0, ctx->stream>>>(g, u, y, n);
  hip_check(hipGetLastError(), "silu_mul_seq launch");
}

void launch_attn_seq(mdma_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t n_q,
                     uint64_t kv_len, uint64_t hd, uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride,
                     const uint32_t *pos_dev) {
  if (!n_q) return;
  if (hd > 256 || n_q > 65535 || n_q_heads > 0xffffffffull || kv_len > 0xffffffffull)
    shape_fail("attn (cpu order): head_dim past 256 or too many queries");
  float *sc = reinterpret_cast<float *>(scratch(ctx, n_q * n_q_heads * kv_len * 4));
  const float scale = 1.0f / sqrtf((float)hd);
  const uint32_t prefix = (uint32_t)(seq_stride ? kv_len - 1 : kv_len - n_q);
  attn_seq_kernel<<<dim3((uint32_t)n_q_heads, (uint32_t)n_q), dim3(256), 0, ctx->stream>>>(
      q, k, v, o, sc, (uint32_t)kv_len, prefix, (uint32_t)hd, (uint32_t)n_q_heads, (uint32_t)n_kv_heads, scale,
      seq_stride, pos_dev);
  hip_check(hipGetLastError(), "attn_seq launch");
}

}  // namespace mdma
