// Per-token Llama ops on gfx950: embedding gather, RMSNorm (optionally fused
// with the residual add), elementwise add and SiLU-gate, interleaved RoPE from
// a host-built angle table, f16 KV writes, causal GQA attention over the f16
// cache, and greedy argmax. Semantics follow the reference CPU backend
// (/root/reference/src/backend/cpu.rs) op for op; these are simple, correct
// kernels, not the hot path.
#include <algorithm>

#include "internal.h"
#include "kernels.h"

namespace mdma {
namespace {

__device__ __forceinline__ float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Row dequantization with the CPU's exact rounding sequence (no contraction):
// Q8_0 q*d; Q4_K (d*sc)*q - dmin*m; Q6_K (d*sc)*q.
__device__ float deq_elem(int32_t dt, const uint8_t *row, uint32_t i) {
#pragma clang fp contract(off)
  if (dt == DT_F32) return reinterpret_cast<const float *>(row)[i];
  if (dt == DT_F16) return h2f(reinterpret_cast<const uint16_t *>(row)[i]);
  if (dt == DT_Q8_0) {
    const uint8_t *b = row + (i / 32) * 34;
    const float d = h2f((uint16_t)(b[0] | (b[1] << 8)));
    return (float)(int8_t)b[2 + i % 32] * d;
  }
  if (dt == DT_Q4_K) {
    const uint8_t *b = row + (i / 256) * 144;
    const uint32_t e = i % 256, j = e / 32, pr = e / 64, l = e % 32;
    const float d = h2f((uint16_t)(b[0] | (b[1] << 8))), dmin = h2f((uint16_t)(b[2] | (b[3] << 8)));
    const uint8_t *s = b + 4;
    uint32_t sc, m;
    if (j < 4) {
      sc = s[j] & 63;
      m = s[j + 4] & 63;
    } else {
      sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
      m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    const uint8_t qb = b[16 + 32 * pr + l];
    const uint32_t q = (j & 1) ? (qb >> 4) : (qb & 0xF);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const float t = d1 * (float)q;
    return t - m1;
  }
  // Q6_K
  const uint8_t *b = row + (i / 256) * 210;
  const uint32_t e = i % 256, n = e / 128, r = (e % 128) / 32, l = e % 32;
  const uint8_t lq = b[64 * n + l + 32 * (r & 1)];
  const int low = (r < 2) ? (lq & 0xF) : (lq >> 4);
  const int high = (b[128 + 32 * n + l] >> (2 * r)) & 3;
  const int q = (low | (high << 4)) - 32;
  const int8_t sc = (int8_t)b[192 + 8 * n + l / 16 + 2 * r];
  const float d = h2f((uint16_t)(b[208] | (b[209] << 8)));
  const float ds = d * (float)sc;
  return ds * (float)q;
}

// The same element from a prepared row (layout.cpp): the same bytes, found
// at their plane positions, with the same rounding sequence.
__device__ float deq_elem_prepared(int32_t dt, const uint8_t *row, uint32_t i, uint32_t n_embd) {
#pragma clang fp contract(off)
  if (dt == DT_Q8_0) {
    const uint32_t nb = n_embd / 32, b = i / 32, l = i % 32;
    const float d = h2f((uint16_t)(row[32 * nb + 2 * b] | (row[32 * nb + 2 * b + 1] << 8)));
    return (float)(int8_t)row[16 * (l < 16 ? b : nb + b) + l % 16] * d;
  }
  const uint32_t nb = n_embd / 256, U = 4 * nb, b = i / 256, e = i % 256;
  if (dt == DT_Q4_K) {
    const uint8_t *hd = row + 32 * U + 16 * b;
    const uint32_t j = e / 32, p = e / 64, l = e % 32, u = 4 * b + p;
    const float d = h2f((uint16_t)(hd[0] | (hd[1] << 8))), dmin = h2f((uint16_t)(hd[2] | (hd[3] << 8)));
    const uint8_t *s = hd + 4;
    uint32_t sc, m;
    if (j < 4) {
      sc = s[j] & 63;
      m = s[j + 4] & 63;
    } else {
      sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
      m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    const uint8_t qb = row[16 * (l < 16 ? u : U + u) + l % 16];
    const uint32_t q = (j & 1) ? (qb >> 4) : (qb & 0xF);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const float t = d1 * (float)q;
    return t - m1;
  }
  // Q6_K
  const uint32_t n = e / 128, r = (e % 128) / 32, l = e % 32, u = 4 * b + 2 * n + l / 16, ll = l % 16;
  const uint8_t lq = row[16 * ((r & 1) ? U + u : u) + ll];
  const int low = (r < 2) ? (lq & 0xF) : (lq >> 4);
  const int high = (row[16 * (2 * U + u) + ll] >> (2 * r)) & 3;
  const int q = (low | (high << 4)) - 32;
  const int8_t sc = (int8_t)row[48 * U + 4 * u + r];
  const float d = h2f((uint16_t)(row[52 * U + 2 * b] | (row[52 * U + 2 * b + 1] << 8)));
  const float ds = d * (float)sc;
  return ds * (float)q;
}

__global__ __launch_bounds__(256) void embed_kernel(int32_t dt, int prepared, const uint8_t *__restrict__ table,
                                                    uint32_t n_embd, size_t row_bytes,
                                                    const uint32_t *__restrict__ ids, float *__restrict__ out) {
  const uint32_t t = blockIdx.y;
  const uint8_t *row = table + (size_t)ids[t] * row_bytes;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n_embd; i += gridDim.x * 256)
    out[(size_t)t * n_embd + i] = prepared ? deq_elem_prepared(dt, row, i, n_embd) : deq_elem(dt, row, i);
}

// Block-wide f64 sum (256 threads).
__device__ double block_sum(double v, double *sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  return sh[0] + sh[1] + sh[2] + sh[3];
}

// rmsnorm (cpu.rs:388-402): scale = 1/sqrt(sum(x^2)/dim + eps); y = (x*scale)*w.
// With b: sum = a + b is written and normalised (add_rmsnorm, backend.rs:502-513).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ w, uint32_t dim,
                                                      const float *__restrict__ a, const float *__restrict__ b,
                                                      float *__restrict__ sum, float *__restrict__ y, float eps) {
#pragma clang fp contract(off)
  __shared__ double sh[4];
  const size_t base = (size_t)blockIdx.x * dim;
  double ss = 0.0;
  for (uint32_t i = threadIdx.x; i < dim; i += 256) {
    float v = a[base + i];
    if (b) {
      v = v + b[base + i];
      sum[base + i] = v;
    }
    const float sq = v * v;
    ss += (double)sq;
  }
  ss = block_sum(ss, sh);
  const float mean_sq = (float)ss / (float)dim;
  const float scale = 1.0f / sqrtf(mean_sq + eps);
  for (uint32_t i = threadIdx.x; i < dim; i += 256) {
    const float v = b ? sum[base + i] : a[base + i];
    const float t = v * scale;
    y[base + i] = t * w[i];
  }
}

// rmsnorm for rows of up to 16384 values (dim % 4 == 0), one 1024-thread
// workgroup per row with the row held in registers (a single pass over
// memory); same arithmetic as rmsnorm_kernel: f32 squares summed in f64,
// scale = 1/sqrt(mean + eps) in f32, y = (x*scale)*w. With QUANT (dim % 256
// == 0) it also writes y's int8 form for the int8-activation GEMV: groups of
// 256 (one wave each), d = amax/127, q = round-half-away(y*127/amax), exact
// sums of 16 -- the arithmetic of quantize_act_kernel, so the result is the
// same bit for bit. With A16 (dim % 32 == 0) it writes instead the f16-path
// GEMM's input for y, with gemm_act_kernel's arithmetic (the same bits): per
// 32 columns (8 lanes) the int8 values as f16 and s = amax/127, and P = s *
// their sum as f16 halves scaled by 2^e, e from the row's largest |P|.
template <bool QUANT, bool A16 = false>
__global__ __launch_bounds__(1024) void rmsnorm_row_kernel(const float *__restrict__ w, uint32_t dim,
                                                           const float *__restrict__ a, const float *__restrict__ b,
                                                           float *__restrict__ sum, float *__restrict__ y, float eps,
                                                           int8_t *__restrict__ q, float *__restrict__ qd,
                                                           int32_t *__restrict__ qs16, F16In in = {}) {
#pragma clang fp contract(off)
  __shared__ double sh[16];
  const size_t base = (size_t)blockIdx.x * dim;
  const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
  float v[4][4];
  float4 wv[4];
  double ss = 0.0;
  float pc[4] = {0.f, 0.f, 0.f, 0.f}, pmax = 0.f;  // A16: each block's P, their maximum |P|
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t i = 4 * t + 4096 * c;
    if (i >= dim) break;
    wv[c] = *reinterpret_cast<const float4 *>(w + i);
    float4 av = *reinterpret_cast<const float4 *>(a + base + i);
    if (b) {
      const float4 bv = *reinterpret_cast<const float4 *>(b + base + i);
      av.x = av.x + bv.x, av.y = av.y + bv.y, av.z = av.z + bv.z, av.w = av.w + bv.w;
      *reinterpret_cast<float4 *>(sum + base + i) = av;
    }
    v[c][0] = av.x, v[c][1] = av.y, v[c][2] = av.z, v[c][3] = av.w;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float sq = v[c][k] * v[c][k];
      ss += (double)sq;
    }
  }
  // Wave sums through DPP lane moves (no LDS round trips), then the waves'
  // in order.
  ss = wave_total63(ss);
  if (lane == 63) sh[wave] = ss;
  __syncthreads();
  double tot = 0.0;
  for (int k = 0; k < 16; k++) tot += sh[k];
  const float mean_sq = (float)tot / (float)dim;
  const float scale = 1.0f / sqrtf(mean_sq + eps);
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t i = 4 * t + 4096 * c;
    if (i >= dim) break;
    const float wk[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
    float r[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float s1 = v[c][k] * scale;
      r[k] = s1 * wk[k];
    }
    *reinterpret_cast<float4 *>(y + base + i) = make_float4(r[0], r[1], r[2], r[3]);
    if (QUANT) {
      // A wave's 4 x 64 values are one 256-group.
      const float amax = wave_max_all(fmaxf(fmaxf(fabsf(r[0]), fabsf(r[1])), fmaxf(fabsf(r[2]), fabsf(r[3]))));
      const float inv = amax == 0.f ? 0.f : 127.0f / amax;
      int qi[4], sm = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        qi[k] = q8_quant(r[k], inv);
        sm += qi[k];
      }
      // sums of 16 columns: the quad of lanes, every lane of it
      sm += (int)dpp_u32<0xB1, 0xF>((uint32_t)sm);
      sm += (int)dpp_u32<0x4E, 0xF>((uint32_t)sm);
      *reinterpret_cast<uint32_t *>(q + base + i) = pack4_i8(qi[0], qi[1], qi[2], qi[3]);
      if ((lane & 3) == 0) qs16[(base + i) / 16] = sm;
      if (lane == 0) qd[(base + i) / 256] = amax / 127.0f;
    }
    if (A16) {  // 8 lanes hold a 32-column block
      float am = fmaxf(fmaxf(fabsf(r[0]), fabsf(r[1])), fmaxf(fabsf(r[2]), fabsf(r[3])));
      am = dpp_max<0xB1, 0xF>(am);
      am = dpp_max<0x4E, 0xF>(am);
      am = dpp_max<0x141, 0xF>(am);
      const float iv = am == 0.f ? 0.f : 127.0f / am;
      int qi[4], sm = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        qi[k] = q8_quant(r[k], iv);
        sm += qi[k];
      }
      sm += (int)dpp_u32<0xB1, 0xF>((uint32_t)sm);
      sm += (int)dpp_u32<0x4E, 0xF>((uint32_t)sm);
      sm += (int)dpp_u32<0x141, 0xF>((uint32_t)sm);
      const float s = am / 127.0f;
      pc[c] = s * (float)sm;
      pmax = fmaxf(pmax, fabsf(pc[c]));
      const v4h h = {(_Float16)(float)qi[0], (_Float16)(float)qi[1], (_Float16)(float)qi[2], (_Float16)(float)qi[3]};
      *reinterpret_cast<v4h *>(in.xh + base + i) = h;
      if ((lane & 7) == 0) in.sx[(base + i) / 32] = s;
    }
  }
  if (A16) {
    // e brings the row's largest |P| into [512, 1024).
    __shared__ float pw[16];
    pmax = wave_max_all(pmax);
    if (lane == 0) pw[wave] = pmax;
    __syncthreads();
    float pm = 0.f;
    for (int k = 0; k < 16; k++) pm = fmaxf(pm, pw[k]);
    int e = 0;
    if (pm > 0.f) {
      int ex;
      frexpf(pm, &ex);
      e = min(max(10 - ex, -100), 100);
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const uint32_t i = 4 * t + 4096 * c;
      if (i >= dim) break;
      if ((lane & 7) == 0) {
        const float pe = ldexpf(pc[c], e);
        const _Float16 hi = (_Float16)pe;
        in.ph[(base + i) / 32] = hi;
        in.pl[(base + i) / 32] = (_Float16)(pe - (float)hi);
      }
    }
    if (t == 0) in.inv[blockIdx.x] = ldexpf(1.0f, -e);
  }
}

__global__ void add_kernel(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ y, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    y[i] = a[i] + b[i];
}

// silu_mul (cpu.rs:447-458): y = (g / (1 + exp(-g))) * u.
__global__ void silu_mul_kernel(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ y,
                                size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    y[i] = silu_mul1(g[i], u[i]);
}

// x: [n_tokens, heads, hd]; tab: [pos][hd/2] (cos, sin). pos_dev (a
// captured decode step): the position is read from there.
__global__ void rope_kernel(float *__restrict__ x, uint32_t heads, uint32_t hd, uint64_t pairs,
                            const float *__restrict__ tab, uint32_t pos, const uint32_t *__restrict__ pos_dev) {
  const uint32_t half = hd / 2;
  if (pos_dev) pos = *pos_dev;
  for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs; p += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t t = p / ((uint64_t)heads * half);
    const uint32_t i = p % half;
    const float2 cs = reinterpret_cast<const float2 *>(tab)[(pos + t) * half + i];
    float x0 = x[2 * p], x1 = x[2 * p + 1];
    rot(x0, x1, cs.x, cs.y);
    x[2 * p] = x0;
    x[2 * p + 1] = x1;
  }
}

// pos_dev (a captured decode step): the rows start *pos_dev * n elements
// after dk / dv.
__global__ void kv_write_kernel(const float *__restrict__ k, const float *__restrict__ v, uint16_t *__restrict__ dk,
                                uint16_t *__restrict__ dv, size_t n, const uint32_t *__restrict__ pos_dev) {
  if (pos_dev) {
    dk += (size_t)*pos_dev * n;
    dv += (size_t)*pos_dev * n;
  }
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    dk[i] = f2h(k[i]);
    dv[i] = f2h(v[i]);
  }
}

// Fused rope_kv_write (backend.rs:452-467): q rotated in place; k rotated and
// stored with v as f16 rows. Token t sits at position pos + t*pos_step and
// its cache row starts kv_stride elements after token t-1's (kv_stride =
// the row width for one sequence; a cache-to-cache stride when each token
// is a different sequence of a batch, with pos_step 0). pos_dev (a captured
// decode step): the position is read from there, and the rows of position
// p start p * pos_row elements after dk / dv.
__global__ void rope_kv_kernel(float *__restrict__ q, uint64_t q_pairs, uint32_t q_heads, const float *__restrict__ k,
                               const float *__restrict__ v, uint64_t k_pairs, uint32_t kv_heads, uint32_t hd,
                               const float *__restrict__ tab, uint32_t pos, uint32_t pos_step, uint64_t kv_stride,
                               uint16_t *__restrict__ dk, uint16_t *__restrict__ dv,
                               const uint32_t *__restrict__ pos_dev, uint64_t pos_row) {
  const uint32_t half = hd / 2;
  if (pos_dev) {
    pos = *pos_dev;
    dk += (size_t)pos * pos_row;
    dv += (size_t)pos * pos_row;
  }
  for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < q_pairs + k_pairs;
       p += (uint64_t)gridDim.x * blockDim.x) {
    if (p < q_pairs) {
      const uint64_t t = p / ((uint64_t)q_heads * half);
      const uint32_t i = p % half;
      const float2 cs = reinterpret_cast<const float2 *>(tab)[(pos + t * pos_step) * half + i];
      float x0 = q[2 * p], x1 = q[2 * p + 1];
      rot(x0, x1, cs.x, cs.y);
      q[2 * p] = x0;
      q[2 * p + 1] = x1;
    } else {
      const uint64_t kp = p - q_pairs;
      const uint64_t per_tok = (uint64_t)kv_heads * half;
      const uint64_t t = kp / per_tok;
      const uint32_t i = kp % half;
      const float2 cs = reinterpret_cast<const float2 *>(tab)[(pos + t * pos_step) * half + i];
      float x0 = k[2 * kp], x1 = k[2 * kp + 1];
      rot(x0, x1, cs.x, cs.y);
      const uint64_t dst = t * kv_stride + 2 * (kp - t * per_tok);
      dk[dst] = f2h(x0);
      dk[dst + 1] = f2h(x1);
      dv[dst] = f2h(v[2 * kp]);
      dv[dst + 1] = f2h(v[2 * kp + 1]);
    }
  }
}

constexpr uint32_t ATT_CHUNK = 1024;

__device__ float block_max(float v, float *sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
}
__device__ float block_sumf(float v, float *sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  return (sh[0] + sh[1]) + (sh[2] + sh[3]);
}

// Causal GQA attention (cpu.rs:530-590) over an f16 cache: one workgroup per
// (query token, q head). Keys are processed in chunks with an online softmax
// (exact single pass when the visible keys fit one chunk). With seq_stride
// 0, query i sees keys [0, prefix + i]; otherwise query i is the single
// decode query of sequence i, whose cache starts seq_stride elements after
// sequence i-1's, and sees keys [0, prefix].
__global__ __launch_bounds__(256) void attn_kernel(const float *__restrict__ q, const uint16_t *__restrict__ K,
                                                   const uint16_t *__restrict__ V, float *__restrict__ o,
                                                   uint32_t prefix, uint32_t hd, uint32_t n_q_heads,
                                                   uint32_t n_kv_heads, float scale, uint64_t seq_stride,
                                                   const uint32_t *__restrict__ pos_dev) {
  __shared__ float qs[256];
  __shared__ float sc[ATT_CHUNK];
  __shared__ float red[4];
  const uint32_t qh = blockIdx.x, i = blockIdx.y;
  if (pos_dev) prefix = *pos_dev;  // a captured decode step: one query per sequence at *pos_dev
  const uint32_t kvh = qh / (n_q_heads / n_kv_heads), kv_row = n_kv_heads * hd;
  const uint32_t visible = seq_stride ? prefix + 1 : prefix + i + 1;
  K += (size_t)i * seq_stride;
  V += (size_t)i * seq_stride;
  const float *qv = q + ((size_t)i * n_q_heads + qh) * hd;
  for (uint32_t d = threadIdx.x; d < hd; d += 256) qs[d] = qv[d];
  __syncthreads();
  float m = -INFINITY, l = 0.f;
  float acc = 0.f;  // thread d < hd owns output dim d
  for (uint32_t c0 = 0; c0 < visible; c0 += ATT_CHUNK) {
    const uint32_t cn = min(ATT_CHUNK, visible - c0);
    for (uint32_t j = threadIdx.x; j < cn; j += 256) {
      const uint16_t *kr = K + (size_t)(c0 + j) * kv_row + (size_t)kvh * hd;
      float s = 0.f;
      for (uint32_t d = 0; d < hd; d++) s = fmaf(qs[d], h2f(kr[d]), s);
      sc[j] = s * scale;
    }
    __syncthreads();
    float cm = -INFINITY;
    for (uint32_t j = threadIdx.x; j < cn; j += 256) cm = fmaxf(cm, sc[j]);
    cm = block_max(cm, red);
    const float nm = fmaxf(m, cm);
    float cs = 0.f;
    for (uint32_t j = threadIdx.x; j < cn; j += 256) {
      const float p = expf(sc[j] - nm);
      sc[j] = p;
      cs += p;
    }
    cs = block_sumf(cs, red);
    const float alpha = expf(m - nm);  // 0 on the first chunk (m = -inf)
    l = l * alpha + cs;
    if (threadIdx.x < hd) {
      float a = acc * alpha;
      const uint16_t *vc = V + (size_t)c0 * kv_row + (size_t)kvh * hd + threadIdx.x;
      for (uint32_t j = 0; j < cn; j++) a = fmaf(sc[j], h2f(vc[(size_t)j * kv_row]), a);
      acc = a;
    }
    m = nm;
    __syncthreads();
  }
  if (threadIdx.x < hd) o[((size_t)i * n_q_heads + qh) * hd + threadIdx.x] = acc / l;
}

// Causal GQA attention for a prompt (one sequence, seq_stride 0: query i
// sees keys [0, prefix + i]; at least ATT_PREFILL_MIN queries) on the matrix
// cores, flash-attention style. A workgroup takes 64 rows, 64/G queries
// times the G query heads of one KV head; wave w owns rows 16w..16w+15.
// Per tile of 64 keys:
//   S = Q K^T on v_mfma_f32_16x16x32_f16. The f16 keys are exact operands;
//     q is split exactly into three f16 parts (hi = f16(q), mid = f16(q -
//     hi), lo = q - hi - mid: 11 + 11 + 2 of its 24 bits), three MFMAs of
//     exact products added in f32, as the f32 kernels' dot products are;
//   an online softmax per row: the row's 64 scores sit on the 16 lanes of
//     one DPP row (4 per lane, one per 16-key block), max and sum by DPP;
//   O += P V on the same MFMA, P (f32, through a per-wave LDS tile of rows x
//     keys) split into f16 hi and lo as it is read; V goes to LDS
//     transposed (dims x keys), so an operand's 8 keys are one 16-byte read.
// s = (q.k) * scale and p = expf(s - m) in f32, the output O / l.
// Key chunks (ct > 0): a query block's tiles are split into chunks of ct
// tiles, one workgroup each (blockIdx.z), so the long blocks at the end of
// a causal prompt no longer set the launch's length alone and more
// workgroups share each CU. Each chunk leaves its rows' (m, l, O) in part
// [slot][value][thread]; the chunk that arrives last at the block's
// counter merges all chunks in chunk order (the same result whatever the
// arrival order) and writes O / l. Chunk 0 holds key 0, which every row
// sees, so the merged maximum is finite; a later chunk's fully masked row
// contributes nothing.
// in.xh set: the writer of O / l also writes the output projection's
// f16-path input (per 32 dims of a row the int8 values as f16 and
// amax / 127, the gemm_f16 quantization pass's arithmetic), no P halves.
constexpr uint32_t ATT_PREFILL_MIN = 64;

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dpp_row_op_max(float v) {
  return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -INFINITY),
                                                                         __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                         false)));
}
template <int CTRL>
__device__ __forceinline__ float dpp_row_op_sum(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                    false));
}
// Max / sum over the 16 lanes of this lane's DPP row, in every lane of it.
__device__ __forceinline__ float row16_max(float v) {
  v = dpp_row_op_max<0xB1>(v);
  v = dpp_row_op_max<0x4E>(v);
  v = dpp_row_op_max<0x141>(v);
  return dpp_row_op_max<0x140>(v);
}
__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_row_op_sum<0xB1>(v);
  v = dpp_row_op_sum<0x4E>(v);
  v = dpp_row_op_sum<0x141>(v);
  return dpp_row_op_sum<0x140>(v);
}

template <int G, int HD>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const float *__restrict__ q, const uint16_t *__restrict__ K,
                                                           const uint16_t *__restrict__ V, float *__restrict__ o,
                                                           uint32_t n_q, uint32_t prefix, uint32_t n_q_heads,
                                                           uint32_t n_kv_heads, float scale, uint32_t ct,
                                                           float *__restrict__ part, uint32_t *__restrict__ cnt,
                                                           F16In in) {
  constexpr int QT = 64 / G;             // queries per workgroup
  constexpr int NC = HD / 32;            // 32-dim K steps of S
  constexpr int ND = HD / 16;            // 16-dim blocks of O
  constexpr int KCH = HD / 8;            // 16-byte chunks of a key row
  constexpr int LPT = 64 * KCH / 256;    // chunks of K (and of V) per thread per tile
  constexpr int VP = 64 + 8;             // padded row of the transposed V tile (f16)
  constexpr int PP = 64 + 4;             // padded row of the P tiles (f32)
  __shared__ __attribute__((aligned(16))) uint16_t ks[64 * HD];        // keys x dims, chunks swizzled
  __shared__ __attribute__((aligned(16))) uint16_t vt[HD * VP];        // dims x keys
  __shared__ __attribute__((aligned(16))) float pw[4][16 * PP];         // per wave: P, rows x keys
  sgpr_ready(q, K, V, o, n_q, prefix, n_q_heads, n_kv_heads, scale);
  const uint32_t kvh = blockIdx.x, q0 = blockIdx.y * QT;
  const uint32_t tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lq = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t kv_row = n_kv_heads * HD, kv_last = prefix + n_q - 1;
  const uint16_t *Kh = K + (size_t)kvh * HD, *Vh = V + (size_t)kvh * HD;

  // Tile t's K and V chunks into registers (rows clamped to the cache).
  // Item i of a thread: keys 2 kp, 2 kp + 1 (kp = lane % 32) of chunk
  // lane / 32 + 2 (wave + 4 i): the two keys' V values pair up into 32-bit
  // words of the transposed tile, and a wave's 32-bit writes for one dim
  // fall on 64 different banks (lanes 32..63 write the rows 8 dims on).
  constexpr int IT = LPT / 2;  // items per thread
  uint4 kr[IT][2], vr[IT][2];
  auto item_ch = [&](int i) { return (lane >> 5) + 2 * (wave + 4 * i); };
  const uint32_t kp = lane & 31;
  auto gload = [&](uint32_t t) {
#pragma unroll
    for (int i = 0; i < IT; i++) {
      const uint32_t ch = item_ch(i);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const size_t row = (size_t)min(64 * t + 2 * kp + e, kv_last) * kv_row + 8 * ch;
        kr[i][e] = *reinterpret_cast<const uint4 *>(Kh + row);
        vr[i][e] = *reinterpret_cast<const uint4 *>(Vh + row);
      }
    }
  };
  // This workgroup's tiles: all of the block's, or chunk blockIdx.z of ct.
  const uint32_t n_tiles = (prefix + min(q0 + QT, n_q) - 1) / 64 + 1;
  const uint32_t n_ch = ct ? (n_tiles + ct - 1) / ct : 1, ch = blockIdx.z;
  if (ch >= n_ch) return;  // (uniform: this block has fewer chunks)
  const uint32_t t_begin = ct ? ch * ct : 0, t_end = ct ? min(t_begin + ct, n_tiles) : n_tiles;
  gload(t_begin);

  // This lane's Q operand row (16 wave + l16) as f16 hi + mid + lo, dims
  // 32c + 8lq (each remainder is exact in f32).
  v8h_t qhi[NC], qmid[NC], qlo[NC];
  {
    const uint32_t r = 16 * wave + l16, qi = min(q0 + r / G, n_q - 1), h = kvh * G + r % G;
    const float *qr = q + ((size_t)qi * n_q_heads + h) * HD + 8 * lq;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const float4 a = *reinterpret_cast<const float4 *>(qr + 32 * c);
      const float4 b = *reinterpret_cast<const float4 *>(qr + 32 * c + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const _Float16 hi = (_Float16)x[e];
        const float r1 = x[e] - (float)hi;
        const _Float16 mid = (_Float16)r1;
        qhi[c][e] = hi;
        qmid[c][e] = mid;
        qlo[c][e] = (_Float16)(r1 - (float)mid);
      }
    }
  }
  // Output rows of this lane: 16 wave + 4 lq + j; the last key each sees.
  uint32_t vis[4];
#pragma unroll
  for (int j = 0; j < 4; j++) vis[j] = prefix + q0 + (16 * wave + 4 * lq + j) / G;
  float m[4], l[4];
  v4f_t O[ND];
#pragma unroll
  for (int j = 0; j < 4; j++) m[j] = -INFINITY, l[j] = 0.f;
#pragma unroll
  for (int n = 0; n < ND; n++) O[n] = v4f_t{0.f, 0.f, 0.f, 0.f};
  float *pwf = pw[wave];

  for (uint32_t t = t_begin; t < t_end; t++) {
    lds_barrier();  // the previous tile's reads of ks and vt are done
#pragma unroll
    for (int i = 0; i < IT; i++) {
      const uint32_t ch = item_ch(i);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const uint32_t key = 2 * kp + e;
        *reinterpret_cast<uint4 *>(&ks[key * HD + 8 * (ch ^ (key & (KCH - 1)))]) = kr[i][e];
      }
      const uint32_t a[4] = {vr[i][0].x, vr[i][0].y, vr[i][0].z, vr[i][0].w};
      const uint32_t b[4] = {vr[i][1].x, vr[i][1].y, vr[i][1].z, vr[i][1].w};
#pragma unroll
      for (int d = 0; d < 8; d++) {
        // dim 8 ch + d of keys 2 kp (low half) and 2 kp + 1 (high half)
        const uint32_t w = __builtin_amdgcn_perm(b[d >> 1], a[d >> 1], (d & 1) ? 0x07060302u : 0x05040100u);
        *reinterpret_cast<uint32_t *>(&vt[(8 * ch + d) * VP + 2 * kp]) = w;
      }
    }
    lds_barrier();
    if (t + 1 < t_end) gload(t + 1);  // in flight over this tile's arithmetic

    // ---- S = Q K^T: 16 rows x 64 keys per wave ----
    v4f_t S[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) S[kb] = v4f_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; c++) {
      v8h_t B[4];
#pragma unroll
      for (int kb = 0; kb < 4; kb++) {
        const uint32_t key = 16 * kb + l16;
        B[kb] = *reinterpret_cast<const v8h_t *>(&ks[key * HD + 8 * ((4 * c + lq) ^ (key & (KCH - 1)))]);
      }
#pragma unroll
      for (int kb = 0; kb < 4; kb++) S[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qlo[c], B[kb], S[kb], 0, 0, 0);
#pragma unroll
      for (int kb = 0; kb < 4; kb++) S[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qmid[c], B[kb], S[kb], 0, 0, 0);
#pragma unroll
      for (int kb = 0; kb < 4; kb++) S[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi[c], B[kb], S[kb], 0, 0, 0);
    }
    // ---- online softmax; P to this wave's LDS tile ----
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float s[4], mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; kb++) {
        const uint32_t key = 64 * t + 16 * kb + l16;
        s[kb] = key <= vis[j] ? S[kb][j] * scale : -INFINITY;
        mx = fmaxf(mx, s[kb]);
      }
      // mn is finite once a visible key has been seen (the first tile of
      // chunk 0 holds key 0); a later chunk's row may see none yet.
      const float mn = fmaxf(m[j], row16_max(mx));
      const float alpha = mn == -INFINITY ? 1.f : expf(m[j] - mn);  // 0 on the first visible tile (m = -inf)
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; kb++) {
        const float p = s[kb] == -INFINITY ? 0.f : expf(s[kb] - mn);  // 0 for masked keys
        ps += p;
        pwf[(4 * lq + j) * PP + 16 * kb + l16] = p;
      }
      l[j] = l[j] * alpha + row16_sum(ps);
      m[j] = mn;
#pragma unroll
      for (int n = 0; n < ND; n++) O[n][j] *= alpha;
    }
    // ---- O += P V (the wave reads back only its own P tile) ----
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const float4 p0 = *reinterpret_cast<const float4 *>(&pwf[l16 * PP + 32 * c + 8 * lq]);
      const float4 p1 = *reinterpret_cast<const float4 *>(&pwf[l16 * PP + 32 * c + 8 * lq + 4]);
      const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
      v8h_t Ah, Al;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const _Float16 hi = (_Float16)pv[e];
        Ah[e] = hi;
        Al[e] = (_Float16)(pv[e] - (float)hi);
      }
      v8h_t B[ND];
#pragma unroll
      for (int n = 0; n < ND; n++) B[n] = *reinterpret_cast<const v8h_t *>(&vt[(16 * n + l16) * VP + 32 * c + 8 * lq]);
#pragma unroll
      for (int n = 0; n < ND; n++) O[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, B[n], O[n], 0, 0, 0);
#pragma unroll
      for (int n = 0; n < ND; n++) O[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, B[n], O[n], 0, 0, 0);
    }
  }
  if (n_ch > 1) {
    // Leave this chunk's (m, l, O), then the last chunk to arrive merges.
    constexpr int NV = 8 + 4 * ND;
    __shared__ uint32_t last;
    const size_t blk = (size_t)kvh * gridDim.y + blockIdx.y;
    float *pb = part + blk * gridDim.z * (NV * 256) + tid;
    {
      float *pc = pb + (size_t)ch * (NV * 256);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        __hip_atomic_store(pc + 256 * j, m[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pc + 256 * (4 + j), l[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int n = 0; n < ND; n++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          __hip_atomic_store(pc + 256 * (8 + 4 * n + j), O[n][j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(cnt + blk * CNT_STRIDE, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      last = prev == n_ch - 1;
      if (last) __hip_atomic_store(cnt + blk * CNT_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    float M[4], L[4];
    v4f_t OA[ND];
    for (uint32_t c = 0; c < n_ch; c++) {
      const float *pc = pb + (size_t)c * (NV * 256);
      float mc[4], lc[4];
      v4f_t Oc[ND];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        mc[j] = c == ch ? m[j] : __hip_atomic_load(pc + 256 * j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lc[j] = c == ch ? l[j] : __hip_atomic_load(pc + 256 * (4 + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int n = 0; n < ND; n++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          Oc[n][j] = c == ch ? O[n][j]
                             : __hip_atomic_load(pc + 256 * (8 + 4 * n + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (c == 0) {
#pragma unroll
        for (int j = 0; j < 4; j++) M[j] = mc[j], L[j] = lc[j];
#pragma unroll
        for (int n = 0; n < ND; n++) OA[n] = Oc[n];
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float mn = fmaxf(M[j], mc[j]);  // finite: chunk 0's M is
          const float a = expf(M[j] - mn), b = mc[j] == -INFINITY ? 0.f : expf(mc[j] - mn);
          L[j] = L[j] * a + lc[j] * b;
#pragma unroll
          for (int n = 0; n < ND; n++) OA[n][j] = OA[n][j] * a + Oc[n][j] * b;
          M[j] = mn;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) l[j] = L[j];
#pragma unroll
    for (int n = 0; n < ND; n++) O[n] = OA[n];
  }
  const bool qo = in.xh != nullptr;  // uniform
  const uint32_t KO = n_q_heads * HD;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t r = 16 * wave + 4 * lq + j, qi = q0 + r / G, h = kvh * G + r % G;
    float val[ND];
#pragma unroll
    for (int n = 0; n < ND; n++) val[n] = O[n][j] / l[j];
    if (qo) {
      // The output projection's f16-path input (gemm_act_kernel's arithmetic):
      // dims 32 b + [0, 32) of row (qi, h) are one quantization block, dims
      // 2 b and 2 b + 1 of the 16 lanes that hold the row. Lane pairs swap
      // halves so that each lane stores one pair of adjacent dims: an even
      // lane dims l16, l16 + 1, an odd lane dims 15 + l16, 16 + l16.
#pragma unroll
      for (int b = 0; b < ND / 2; b++) {
        const float am = row16_max(fmaxf(fabsf(val[2 * b]), fabsf(val[2 * b + 1])));
        const float iv = am == 0.f ? 0.f : 127.0f / am;
        const uint32_t ha = __builtin_bit_cast(uint16_t, (_Float16)(float)q8_quant(val[2 * b], iv));
        const uint32_t hb = __builtin_bit_cast(uint16_t, (_Float16)(float)q8_quant(val[2 * b + 1], iv));
        const uint32_t na = dpp_u32<0xB1, 0xF>(ha), nb = dpp_u32<0xB1, 0xF>(hb);  // lane l16 ^ 1's
        if (qi < n_q) {
          const bool ev = (l16 & 1) == 0;
          _Float16 *xr = in.xh + (size_t)qi * KO + h * HD + 32 * b + (ev ? l16 : 15 + l16);
          *reinterpret_cast<uint32_t *>(xr) = ev ? ha | na << 16 : nb | hb << 16;
          if (l16 == 0) in.sx[(size_t)qi * (KO / 32) + h * (HD / 32) + b] = am / 127.0f;
        }
      }
    }
    if (qi >= n_q) continue;
    float *orow = o + ((size_t)qi * n_q_heads + h) * HD + l16;
#pragma unroll
    for (int n = 0; n < ND; n++) orow[16 * n] = val[n];
  }
}

// Split-key attention (flash-decoding). A workgroup takes one query, one KV
// head with all G query heads of its group (each f16 K/V row is read once
// for the group) and a run of `tpw` tiles of ATT_TILE keys, with an online
// softmax across its tiles and the next tile's K/V loaded while the current
// one is computed. Scores: a quad of lanes per key, each lane 8-wide 16-byte
// slices 32 apart, summed over the quad with DPP. P.V: each lane owns two
// adjacent dims of a 128-wide slice over 16 keys per wave, so no cross-lane
// sums; the four waves' partial outputs meet in LDS. A run leaves, per query
// head, its max m, its sum l of exp(s - m) and its unnormalised output in
// part [query][q head][split][hd + 2]; the run that arrives last for its
// (query, KV head) -- a device-scope counter, reset by that run -- merges
// them (weights exp(m_s - M)). A single run writes o directly. Scores and
// exponentials are f32: s = (q.k) * scale, p = expf(s - m).
// With QUANT (G*hd a multiple of 256) the finishing workgroup also writes
// the int8 form of its G heads' output (groups of 256, the arithmetic of
// quantize_act_kernel) into q8 at the output's element offsets.
constexpr uint32_t ATT_TILE = 64;
constexpr uint32_t ATT_MAX_RUNS = 16;  // runs merged per (query, KV head)
#ifndef MDMA_ATT_WG_TARGET
#define MDMA_ATT_WG_TARGET 1024
#endif
struct AttnQ8 {
  int8_t *q;
  float *d;
  int32_t *s16;
};

// Decode with the query's RoPE and the new token's cache write folded in:
// q, k, v are the projections before rotation ([n_q, heads, hd] f32); every
// query's new key sits at its last visible position, rope position pos.
struct AttnRope {
  const float *k, *v, *tab;
  uint32_t pos;
  // Set in a captured decode step: the position is read from here (written
  // before each replay), and the launch's grid is sized for the whole cache.
  const uint32_t *pos_dev;
  // With pos_dev: the host's run count before it meets the key count,
  // min(ceil(MDMA_ATT_WG_TARGET / pairs), ATT_MAX_RUNS); the kernel splits
  // the live keys as the host would (runs min(runs0, tiles), each
  // ceil(tiles / runs) tiles).
  uint32_t runs0;
};

// Device-scope (all XCDs) coherent store and load of one float.
__device__ __forceinline__ void store_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int C>
struct AttnTile {
  uint4 k[4 * C];     // K slices of this lane's key
  uint32_t v[16][C];  // V dim pairs of this wave's 16 keys
};

// One tile's K slices and V pairs. Every load is unconditional, its row
// clamped to visible - 1 and its dims to the head: a load under a branch
// becomes a register copy after it, which waits for every load in flight.
// The values of rows past visible and dims past hd are never used (their
// scores are masked, their P.V terms zeroed, their dims not stored).
template <int C>
__device__ __forceinline__ void attn_load(AttnTile<C> &t, const uint16_t *__restrict__ K,
                                          const uint16_t *__restrict__ V, uint32_t tile, uint32_t visible,
                                          uint32_t kv_row, uint32_t hd, uint32_t lane, uint32_t wave) {
  // 32-bit element offsets from the (uniform) cache bases, and V rows
  // uniform per wave: addresses stay in SGPRs plus one VGPR offset.
  const uint32_t jk = min(tile * ATT_TILE + wave * 16 + (lane >> 2), visible - 1), l4 = lane & 3;
#pragma unroll
  for (int m = 0; m < 4 * C; m++) {
    const uint32_t d0 = min(8 * l4 + 32 * m, hd - 8);
    t.k[m] = *reinterpret_cast<const uint4 *>(K + (jk * kv_row + d0));
  }
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const uint32_t jv = min(tile * ATT_TILE + wave * 16 + r, visible - 1);
    const uint16_t *vrow = V + jv * kv_row;
#pragma unroll
    for (int c = 0; c < C; c++) {
      const uint32_t d = min(2 * lane + 128 * c, hd - 2);
      t.v[r][c] = *reinterpret_cast<const uint32_t *>(vrow + d);
    }
  }
}

// ONE: one tile buffer, each tile of a run loaded after the previous one is
// computed (the host's choice whenever every run is one tile, or the grid
// has more workgroups than two per CU): 92 VGPRs instead of 181 at G = 4,
// so five workgroups fit a CU instead of two (batch-8 decode at 768-key
// caches: 640 workgroups in one wave of the chip). The same tiles in the
// same order as the two-buffer loop: the same bits.
template <int G, int C, bool QUANT, bool ROPE, bool ONE = false>
__global__ __launch_bounds__(256) void attn_split_kernel(const float *__restrict__ q, uint16_t *__restrict__ K,
                                                         uint16_t *__restrict__ V, float *__restrict__ o,
                                                         float *__restrict__ part, uint32_t *__restrict__ cnt,
                                                         uint32_t prefix, uint32_t hd, uint32_t n_q_heads,
                                                         uint32_t n_kv_heads, float scale, uint64_t seq_stride,
                                                         uint32_t tpw, AttnQ8 q8, AttnRope rp) {
  __shared__ float qs[G][128 * C];
  __shared__ float sc[G][ATT_TILE];
  __shared__ float mrun[G], lrun[G], alph[G];
  __shared__ float red[4][G][128 * C];
  __shared__ float gmax[(G * 128 * C + 255) / 256][4];
  __shared__ float wml[G][ATT_MAX_RUNS][2];
  __shared__ uint32_t last;
  __shared__ __attribute__((aligned(16))) uint32_t knew[ROPE ? 64 * C : 4];  // the new row's f16 pairs
  __shared__ uint32_t vnew[ROPE ? 64 * C : 1];
  // The arguments' scalar loads in one batch (one wait, not a chain).
  sgpr_ready(q, K, V, o, part, cnt, prefix, hd, n_q_heads, n_kv_heads, scale, seq_stride, tpw);
  if constexpr (QUANT) sgpr_ready(q8.q, q8.d, q8.s16);
  if constexpr (ROPE) sgpr_ready(rp.k, rp.v, rp.tab, rp.pos, rp.pos_dev);
  // sub workgroups per KV head (the grid's x is n_kv_heads * sub), each with
  // G of the head's query heads: the first query head is blockIdx.x * G.
  const uint32_t sub = gridDim.x / n_kv_heads, kvh = blockIdx.x / sub;
  const uint32_t split = blockIdx.y, i = blockIdx.z, n_splits = gridDim.y;
  // The new row's position and the tiles per run. From device memory in a
  // captured step: the runs are those the host chooses for this length
  // (attn_impl: min(runs0, tiles) runs of ceil(tiles / runs) tiles each),
  // so a replay computes the same partials, merged in the same order, as
  // the eager launch. The grid's n_splits, min(runs0, tiles of the whole
  // cache), is at least that many runs.
  uint32_t rpos = ROPE ? rp.pos : 0;
  if (rp.pos_dev) {
    rpos = *rp.pos_dev;
    prefix = rpos;  // one new query per sequence at rpos: visible = rpos + 1
    const uint32_t tl = (rpos + ATT_TILE) / ATT_TILE, runs = min(rp.runs0, tl);
    tpw = (tl + runs - 1) / runs;
  }
  const uint32_t visible = seq_stride ? prefix + 1 : prefix + i + 1;
  const uint32_t tiles = (visible + ATT_TILE - 1) / ATT_TILE, t0 = split * tpw;
  if (t0 >= tiles) return;  // this query's keys end before the run
  const uint32_t t1 = min(t0 + tpw, tiles), live = (tiles + tpw - 1) / tpw;
  const uint32_t kv_row = n_kv_heads * hd, qh0 = blockIdx.x * G;
  const uint32_t tid = threadIdx.x, lane = tid & 63, l4 = lane & 3;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  K += (size_t)i * seq_stride + (size_t)kvh * hd;
  V += (size_t)i * seq_stride + (size_t)kvh * hd;
  // Loads in the order they are needed: q's pairs (and with ROPE the new
  // key's and value's pairs and their rotation), then the first tile. Every
  // load is unconditional (indices clamped), so each wait below is for the
  // loads it needs and not for the tile behind them.
  const float *qv = q + ((size_t)i * n_q_heads + qh0) * hd;
  constexpr int QP = (G * 64 * C + 255) / 256;  // q pairs per thread
  const uint32_t hp = hd / 2, n_qp = G * hp;
  float2 qx[QP], qcs[QP];
#pragma unroll
  for (int k = 0; k < QP; k++) {
    const uint32_t p = min(tid + 256 * k, n_qp - 1), h = p / hp, e = p % hp;
    qx[k] = *reinterpret_cast<const float2 *>(qv + h * hd + 2 * e);
    if (ROPE) qcs[k] = reinterpret_cast<const float2 *>(rp.tab)[(size_t)rpos * hp + e];
  }
  // The new key (ROPE: position visible - 1) is not read from the cache: it
  // is rotated from rp.k and rounded to f16 exactly as the cache stores it
  // (rope_kv_kernel's values), kept in LDS with the new value, substituted
  // where the scores and P.V meet that row, and written to the cache by the
  // run that holds it.
  const uint32_t jn = visible - 1, en = min(tid, hp - 1);
  float2 kn2, vn2, cn2;
  if (ROPE) {
    kn2 = reinterpret_cast<const float2 *>(rp.k + ((size_t)i * n_kv_heads + kvh) * hd)[en];
    vn2 = reinterpret_cast<const float2 *>(rp.v + ((size_t)i * n_kv_heads + kvh) * hd)[en];
    cn2 = reinterpret_cast<const float2 *>(rp.tab)[(size_t)rpos * hp + en];
  }
  // Ping-pong tile buffers: the loads for tile+1 go out before tile is
  // computed (clamped to the run's last tile, so every load is in bounds and
  // the wait counts are fixed).
  AttnTile<C> ta, tb;
  __builtin_amdgcn_sched_barrier(0);  // q and the new row's loads go out first
  attn_load<C>(ta, K, V, t0, visible, kv_row, hd, lane, wave);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < QP; k++) {
    const uint32_t p = tid + 256 * k;
    if (p < n_qp) {
      const uint32_t h = p / hp, e = p % hp;
      float x0 = qx[k].x, x1 = qx[k].y;
      if (ROPE) rot(x0, x1, qcs[k].x, qcs[k].y);  // interleaved pairs, as rope_kv_kernel rotates q
      qs[h][2 * e] = x0;
      qs[h][2 * e + 1] = x1;
    }
  }
  if (ROPE && tid < hp) {
    float x0 = kn2.x, x1 = kn2.y;
    rot(x0, x1, cn2.x, cn2.y);
    const uint32_t kw = (uint32_t)f2h(x0) | ((uint32_t)f2h(x1) << 16);
    const uint32_t vw = (uint32_t)f2h(vn2.x) | ((uint32_t)f2h(vn2.y) << 16);
    knew[tid] = kw;
    vnew[tid] = vw;
    if (jn / ATT_TILE >= t0 && jn / ATT_TILE < t1 && blockIdx.x % sub == 0) {
      *reinterpret_cast<uint32_t *>(K + (size_t)jn * kv_row + 2 * tid) = kw;
      *reinterpret_cast<uint32_t *>(V + (size_t)jn * kv_row + 2 * tid) = vw;
    }
  }
  if (tid < G) mrun[tid] = -INFINITY, lrun[tid] = 0.f;
  float acc[G][C][2];
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int c = 0; c < C; c++) acc[h][c][0] = acc[h][c][1] = 0.f;
  lds_barrier();
  auto process = [&](const AttnTile<C> &cur, uint32_t tile) {
    // The tile holding the new row takes its K and V from LDS.
    const bool has_new = ROPE && tile == jn / ATT_TILE;
    const bool key_new = has_new && tile * ATT_TILE + wave * 16 + (lane >> 2) == jn;
    float s[G];
#pragma unroll
    for (int h = 0; h < G; h++) s[h] = 0.f;
#pragma unroll
    for (int m = 0; m < 4 * C; m++) {
      const uint32_t d0 = 8 * l4 + 32 * m;
      if (d0 < hd) {
        uint4 k4 = cur.k[m];
        if (has_new) {
          const uint4 nk = *reinterpret_cast<const uint4 *>(&knew[d0 / 2]);
          if (key_new) k4 = nk;
        }
        const uint32_t kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float kf = h2f((uint16_t)(kk[e >> 1] >> (16 * (e & 1))));
#pragma unroll
          for (int h = 0; h < G; h++) s[h] = fmaf(qs[h][d0 + e], kf, s[h]);
        }
      }
    }
    const uint32_t jl = wave * 16 + (lane >> 2);
#pragma unroll
    for (int h = 0; h < G; h++) {
      float v = dpp_step<0xB1, 0xF>(s[h]);
      v = dpp_step<0x4E, 0xF>(v);
      if (l4 == 0) sc[h][jl] = tile * ATT_TILE + jl < visible ? v * scale : -INFINITY;
    }
    lds_barrier();
    for (int h = wave; h < G; h += 4) {
      const float v = sc[h][lane];
      const float mo = mrun[h], mn = fmaxf(mo, wave_max_all(v));
      const float pj = expf(v - mn);  // 0 for masked keys (v = -inf)
      const float l = wave_sum_all(pj);
      sc[h][lane] = pj;
      if (lane == 0) {
        const float a = expf(mo - mn);  // 0 on the first tile (mo = -inf)
        lrun[h] = lrun[h] * a + l;
        mrun[h] = mn;
        alph[h] = a;
      }
    }
    lds_barrier();
#pragma unroll
    for (int h = 0; h < G; h++) {
      const float a = alph[h];
#pragma unroll
      for (int c = 0; c < C; c++) acc[h][c][0] *= a, acc[h][c][1] *= a;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
      // wave-uniform: row r of this wave past visible (its value may be
      // anything, even NaN: zeroed, not weighted by 0), or the new row
      const uint32_t jr = tile * ATT_TILE + wave * 16 + r;
      uint32_t vr[C];
#pragma unroll
      for (int c = 0; c < C; c++) {
        vr[c] = jr < visible ? cur.v[r][c] : 0u;
        if (has_new && jr == jn && 2 * lane + 128 * c < hd) vr[c] = vnew[lane + 64 * c];
      }
#pragma unroll
      for (int h = 0; h < G; h++) {
        const float ph = sc[h][wave * 16 + r];
#pragma unroll
        for (int c = 0; c < C; c++) {
          acc[h][c][0] = fmaf(ph, h2f(vr[c] & 0xffffu), acc[h][c][0]);
          acc[h][c][1] = fmaf(ph, h2f(vr[c] >> 16), acc[h][c][1]);
        }
      }
    }
    lds_barrier();  // sc is rewritten by the next tile
  };
  if (ONE) {
    // One tile buffer: a run of several tiles loads each after the previous
    // one is computed (no prefetch, half the registers).
    for (uint32_t tile = t0; tile < t1; tile++) {
      if (tile > t0) attn_load<C>(ta, K, V, tile, visible, kv_row, hd, lane, wave);
      process(ta, tile);
    }
  } else if (t1 - t0 == 1) {
    process(ta, t0);
  } else {
    for (uint32_t tile = t0; tile < t1; tile += 2) {
      attn_load<C>(tb, K, V, min(tile + 1, t1 - 1), visible, kv_row, hd, lane, wave);
      process(ta, tile);
      if (tile + 1 >= t1) break;
      attn_load<C>(ta, K, V, min(tile + 2, t1 - 1), visible, kv_row, hd, lane, wave);
      process(tb, tile + 1);
    }
  }
#pragma unroll
  for (int c = 0; c < C; c++) {
    const uint32_t d = 2 * lane + 128 * c;
    if (d < hd) {
#pragma unroll
      for (int h = 0; h < G; h++) red[wave][h][d] = acc[h][c][0], red[wave][h][d + 1] = acc[h][c][1];
    }
  }
  lds_barrier();
  // Outputs t = tid + 256*k of the group's G*hd values (heads contiguous).
  constexpr int NO = (G * 128 * C + 255) / 256;
  float out[NO];
  const size_t orow = ((size_t)i * n_q_heads + qh0) * hd;
  if (live == 1) {  // one run (always so when the grid has one split): no partials
#pragma unroll
    for (int k = 0; k < NO; k++) {
      const uint32_t t = tid + 256 * k;
      if (t < G * hd) {
        const uint32_t h = t / hd, d = t % hd;
        out[k] = (((red[0][h][d] + red[1][h][d]) + red[2][h][d]) + red[3][h][d]) / lrun[h];
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < NO; k++) {
      const uint32_t t = tid + 256 * k;
      if (t < G * hd) {
        const uint32_t h = t / hd, d = t % hd;
        store_dev(part + ((orow / hd + h) * n_splits + split) * (hd + 2) + d,
                  ((red[0][h][d] + red[1][h][d]) + red[2][h][d]) + red[3][h][d]);
      }
    }
    if (tid < G) {
      float *pp = part + ((orow / hd + tid) * n_splits + split) * (hd + 2) + hd;
      store_dev(pp, mrun[tid]);
      store_dev(pp + 1, lrun[tid]);
    }
    // Partials move between workgroups (possibly on different XCDs, whose
    // L2s are not coherent with each other) only through device-scope
    // stores and loads, which write through and read from the coherence
    // point. Each wave waits for its stores to be acknowledged before the
    // barrier; the counter's device-scope add comes after the barrier, so a
    // run that sees every other run's add also sees their partials. This
    // avoids the whole-L2 write-back and invalidate of a device-scope fence.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      uint32_t *c = cnt + ((size_t)i * gridDim.x + blockIdx.x) * CNT_STRIDE;
      const uint32_t prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == live - 1;
      // every run of this (query, KV head) has arrived: ready for the next call
      if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // Merge weights w[h][s] = exp(m_s - M) / L with M = max m_s and
    // L = sum l_s exp(m_s - M); then out = sum_s w[h][s] * partial_s.
    // The partial vectors are loaded first, so both loads overlap.
    // Every load unconditional (indices clamped; the terms of runs past
    // live are not used), the (m, l) pairs first: one wait for all of them.
    static_assert(G * ATT_MAX_RUNS <= 256, "one (m, l) pair per thread");
    float ml[2] = {0.f, 0.f};
    const uint32_t e_ml = min(tid, G * live - 1), h_ml = e_ml / live, s_ml = e_ml % live;
    {
      const float *pp = part + ((orow / hd + h_ml) * n_splits + s_ml) * (hd + 2) + hd;
      ml[0] = load_dev(pp);
      ml[1] = load_dev(pp + 1);
    }
    float pv[NO][ATT_MAX_RUNS];
#pragma unroll
    for (int k = 0; k < NO; k++) {
      const uint32_t t = min(tid + 256 * k, G * hd - 1);
      const uint32_t h = t / hd, d = t % hd;
      const float *pb = part + (orow / hd + h) * n_splits * (hd + 2) + d;
#pragma unroll
      for (uint32_t s2 = 0; s2 < ATT_MAX_RUNS; s2++) pv[k][s2] = load_dev(pb + min(s2, live - 1) * (hd + 2));
    }
    if (tid < G * live) wml[h_ml][s_ml][0] = ml[0], wml[h_ml][s_ml][1] = ml[1];
    __syncthreads();
    if (tid < G) {
      float M = -INFINITY;
      for (uint32_t s2 = 0; s2 < live; s2++) M = fmaxf(M, wml[tid][s2][0]);
      float L = 0.f;
      for (uint32_t s2 = 0; s2 < live; s2++) {
        const float w = expf(wml[tid][s2][0] - M);
        wml[tid][s2][0] = w;
        L = fmaf(wml[tid][s2][1], w, L);
      }
      lrun[tid] = L;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NO; k++) {
      const uint32_t t = tid + 256 * k;
      if (t < G * hd) {
        const uint32_t h = t / hd;
        float a = 0.f;
#pragma unroll
        for (uint32_t s2 = 0; s2 < ATT_MAX_RUNS; s2++)
          if (s2 < live) a = fmaf(pv[k][s2], wml[h][s2][0], a);
        out[k] = a / lrun[h];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NO; k++) {
    const uint32_t t = tid + 256 * k;
    if (t < G * hd) o[orow + t] = out[k];
  }
  if (QUANT) {
    // G*hd is whole groups of 256: output k of every thread is group k. The
    // waves' maxima of every group meet in LDS behind one barrier.
#pragma unroll
    for (int k = 0; k < NO; k++) {
      if (256 * k >= G * hd) break;
      const float wm = wave_max_all(fabsf(out[k]));
      if (lane == 0) gmax[k][wave] = wm;
    }
    lds_barrier();
#pragma unroll
    for (int k = 0; k < NO; k++) {
      if (256 * k >= G * hd) break;
      const float amax = fmaxf(fmaxf(gmax[k][0], gmax[k][1]), fmaxf(gmax[k][2], gmax[k][3]));
      const float inv = amax == 0.f ? 0.f : 127.0f / amax;
      const int qi = q8_quant(out[k], inv);
      // sum of 16 columns: quads, then half rows and rows (every lane)
      int sm = qi;
      sm += (int)dpp_u32<0xB1, 0xF>((uint32_t)sm);
      sm += (int)dpp_u32<0x4E, 0xF>((uint32_t)sm);
      sm += (int)dpp_u32<0x141, 0xF>((uint32_t)sm);
      sm += (int)dpp_u32<0x140, 0xF>((uint32_t)sm);
      const size_t e = orow + tid + 256 * k;
      q8.q[e] = (int8_t)qi;
      if ((lane & 15) == 0) q8.s16[e / 16] = sm;
      if (tid == 0) q8.d[e / 256] = amax / 127.0f;
    }
  }
}

// Greedy argmax (sampler.rs:64-74): largest by the total order of floats,
// ties to the last index; non-finite logits are flagged.
__device__ __forceinline__ int32_t total_key(float f) {
  const int32_t b = __builtin_bit_cast(int32_t, f);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

// Greedy argmax in two passes: argmax_part_kernel reduces chunks of
// ARGMAX_CHUNK logits of each row to (key, index, non-finite flag), argmax_final_kernel
// the chunks of a row; ties go to the larger index (max_by keeps the last
// maximum, src/sampler.rs:64-74) at both levels.
// Chunks of 1024 logits: four per thread, loaded together (a latency-bound
// pass: the chain per thread is what it costs).
constexpr uint32_t ARGMAX_CHUNK = 1024;
struct ArgPart {
  int32_t key;
  uint32_t idx, bad;
};
__global__ __launch_bounds__(256) void argmax_part_kernel(const float *__restrict__ x, uint64_t n,
                                                          ArgPart *__restrict__ part) {
  __shared__ ArgPart sp[4];
  const uint32_t chunk = blockIdx.x, row = blockIdx.y, nchunks = gridDim.x;
  const float *xr = x + (size_t)row * n;
  const uint64_t c0 = (uint64_t)chunk * ARGMAX_CHUNK, c1 = min(c0 + ARGMAX_CHUNK, n);
  int32_t bk = INT32_MIN;
  uint32_t bi = 0, bad = 0;
  bool have = false;
  constexpr int PER = ARGMAX_CHUNK / 256;
  float v[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) v[j] = xr[min(c0 + threadIdx.x + 256 * j, n - 1)];  // clamped, unconditional
#pragma unroll
  for (int j = 0; j < PER; j++) {  // increasing index: ties go to the later one
    const uint64_t i = c0 + threadIdx.x + 256 * j;
    if (i >= c1) break;
    bad |= !isfinite(v[j]);
    const int32_t k = total_key(v[j]);
    if (!have || k >= bk) {
      bk = k;
      bi = (uint32_t)i;
      have = true;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const int32_t ok = __shfl_xor(bk, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    const int oh = __shfl_xor((int)have, o, 64);
    if (oh && (!have || ok > bk || (ok == bk && oi > bi))) {
      bk = ok;
      bi = oi;
      have = true;
    }
    bad |= __shfl_xor(bad, o, 64);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sp[w] = ArgPart{have ? bk : INT32_MIN, have ? bi : 0u, bad | (have ? 0u : 2u)};
  __syncthreads();
  if (threadIdx.x == 0) {
    ArgPart r = sp[0];
    for (int j = 1; j < 4; j++) {
      const ArgPart &c = sp[j];
      const bool rh = !(r.bad & 2u), ch = !(c.bad & 2u);
      if (ch && (!rh || c.key > r.key || (c.key == r.key && c.idx > r.idx))) r = ArgPart{c.key, c.idx, r.bad & 1u};
      r.bad = (r.bad & 2u ? (ch ? 0u : 2u) : 0u) | ((r.bad | c.bad) & 1u);
    }
    part[(size_t)row * nchunks + chunk] = r;
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const ArgPart *__restrict__ part, uint32_t nchunks,
                                                          uint32_t *__restrict__ idx, uint32_t *__restrict__ flag) {
  const uint32_t row = blockIdx.x;
  ArgPart r{INT32_MIN, 0, 2u};
  for (uint32_t c = threadIdx.x; c < nchunks; c += 64) {
    const ArgPart p = part[(size_t)row * nchunks + c];
    const bool rh = !(r.bad & 2u), ph = !(p.bad & 2u);
    const uint32_t nb = (r.bad | p.bad) & 1u;
    if (ph && (!rh || p.key > r.key || (p.key == r.key && p.idx > r.idx))) r = ArgPart{p.key, p.idx, nb};
    else r.bad = (r.bad & 2u) | nb;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const int32_t ok = __shfl_xor(r.key, o, 64);
    const uint32_t oi = __shfl_xor(r.idx, o, 64), ob = __shfl_xor(r.bad, o, 64);
    const bool rh = !(r.bad & 2u), oh = !(ob & 2u);
    const uint32_t nb = (r.bad | ob) & 1u;
    if (oh && (!rh || ok > r.key || (ok == r.key && oi > r.idx))) r = ArgPart{ok, oi, nb};
    else r.bad = (r.bad & 2u) | nb;
  }
  if (threadIdx.x == 0) {
    idx[row] = r.idx;
    flag[row] = (r.bad & 1u) || (r.bad & 2u) ? 1u : 0u;  // non-finite, or an empty row
  }
}

// One workgroup per row of x [rows, n]; the index goes to idx[row], the
// non-finite flag to flag[row].
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float *__restrict__ x, uint64_t n,
                                                           uint32_t *__restrict__ idx, uint32_t *__restrict__ flag) {
  __shared__ int32_t sk[16];
  __shared__ uint32_t si[16];
  __shared__ uint32_t sbad[16];
  x += (size_t)blockIdx.x * n;
  int32_t bk = INT32_MIN;
  uint32_t bi = 0, bad = 0;
  bool have = false;
  for (uint64_t i = threadIdx.x; i < n; i += 1024) {
    const float v = x[i];
    bad |= !isfinite(v);
    const int32_t k = total_key(v);
    if (!have || k >= bk) {
      bk = k;
      bi = (uint32_t)i;
      have = true;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    const int32_t ok = __shfl_xor(bk, o, 64);
    const uint32_t oi = __shfl_xor(bi, o, 64);
    const int oh = __shfl_xor((int)have, o, 64);
    if (oh && (!have || ok > bk || (ok == bk && oi > bi))) {
      bk = ok;
      bi = oi;
      have = true;
    }
    bad |= __shfl_xor(bad, o, 64);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sk[w] = have ? bk : INT32_MIN;
    si[w] = have ? bi : 0;
    sbad[w] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t k = sk[0];
    uint32_t best = si[0], fl = sbad[0];
    for (int j = 1; j < 16; j++) {
      fl |= sbad[j];
      if ((uint64_t)j * 64 >= n) continue;
      if (sk[j] > k || (sk[j] == k && si[j] > best)) {
        k = sk[j];
        best = si[j];
      }
    }
    idx[blockIdx.x] = best;
    flag[blockIdx.x] = fl;
  }
}

uint32_t grid1d(uint64_t n, uint32_t per = 256) {
  uint64_t g = (n + per - 1) / per;
  if (g > 65536) g = 65536;
  return (uint32_t)(g ? g : 1);
}

}  // namespace

void launch_embed(mdma_ctx *ctx, int32_t dtype, int layout, const uint8_t *table, uint64_t n_embd,
                  const uint32_t *ids, uint64_t n_ids, float *out) {
  const bool prepared = layout == MDMA_LAYOUT_GFX950;
  const size_t rb = prepared ? gfx950_row_bytes(dtype, n_embd) : n_embd / block_size(dtype) * type_size(dtype);
  embed_kernel<<<dim3(grid1d(n_embd), (uint32_t)n_ids), dim3(256), 0, ctx->stream>>>(
      dtype, prepared ? 1 : 0, table, (uint32_t)n_embd, rb, ids, out);
  hip_check(hipGetLastError(), "embed launch");
}

void launch_rmsnorm(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                    float *y, uint64_t rows, float eps) {
  if (dim % 4 == 0 && dim <= 16384)
    rmsnorm_row_kernel<false><<<dim3((uint32_t)rows), dim3(1024), 0, ctx->stream>>>(w, (uint32_t)dim, a, b, sum, y,
                                                                                     eps, nullptr, nullptr, nullptr);
  else
    rmsnorm_kernel<<<dim3((uint32_t)rows), dim3(256), 0, ctx->stream>>>(w, (uint32_t)dim, a, b, sum, y, eps);
  hip_check(hipGetLastError(), "rmsnorm launch");
}

bool launch_rmsnorm_a16(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                        float *y, uint64_t rows, float eps, char *buf, uint64_t buf_bytes) {
  if (dim % 32 || dim > 16384 || !buf || buf_bytes < gemm_f16_input_bytes(rows, dim)) return false;
  const F16In in = gemm_f16_input_at(buf, rows, dim);
  rmsnorm_row_kernel<false, true><<<dim3((uint32_t)rows), dim3(1024), 0, ctx->stream>>>(
      w, (uint32_t)dim, a, b, sum, y, eps, nullptr, nullptr, nullptr, in);
  hip_check(hipGetLastError(), "rmsnorm launch");
  a16_mark(ctx, y, rows, dim, buf, true);
  return true;
}

bool launch_rmsnorm_q8(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                       float *y, uint64_t rows, float eps) {
  if (dim % 256 || dim > 16384) return false;
  int8_t *q;
  float *d;
  int32_t *s16;
  q8_slots(ctx, rows, dim, &q, &d, &s16);
  rmsnorm_row_kernel<true><<<dim3((uint32_t)rows), dim3(1024), 0, ctx->stream>>>(w, (uint32_t)dim, a, b, sum, y,
                                                                                  eps, q, d, s16);
  hip_check(hipGetLastError(), "rmsnorm launch");
  q8_mark(ctx, y, rows, dim);
  return true;
}

void launch_add(mdma_ctx *ctx, const float *a, const float *b, float *y, uint64_t n) {
  if (!n) return;
  add_kernel<<<dim3(grid1d(n)), dim3(256), 0, ctx->stream>>>(a, b, y, n);
  hip_check(hipGetLastError(), "add launch");
}

void launch_silu_mul(mdma_ctx *ctx, const float *g, const float *u, float *y, uint64_t n) {
  if (!n) return;
  silu_mul_kernel<<<dim3(grid1d(n)), dim3(256), 0, ctx->stream>>>(g, u, y, n);
  hip_check(hipGetLastError(), "silu_mul launch");
}

void launch_rope(mdma_ctx *ctx, float *x, uint64_t n_tokens, uint64_t heads, uint64_t hd, const float *tab,
                 uint32_t pos, const uint32_t *pos_dev) {
  const uint64_t pairs = n_tokens * heads * (hd / 2);
  if (!pairs) return;
  rope_kernel<<<dim3(grid1d(pairs)), dim3(256), 0, ctx->stream>>>(x, (uint32_t)heads, (uint32_t)hd, pairs, tab, pos,
                                                                  pos_dev);
  hip_check(hipGetLastError(), "rope launch");
}

void launch_kv_write(mdma_ctx *ctx, const float *k, const float *v, uint16_t *dk, uint16_t *dv, uint64_t n,
                     const uint32_t *pos_dev) {
  kv_write_kernel<<<dim3(grid1d(n)), dim3(256), 0, ctx->stream>>>(k, v, dk, dv, n, pos_dev);
  hip_check(hipGetLastError(), "kv_write launch");
}

void launch_rope_kv_write(mdma_ctx *ctx, float *q, uint64_t q_heads, const float *k, const float *v,
                          uint64_t kv_heads, uint64_t hd, uint64_t n_tokens, const float *tab, uint32_t pos,
                          uint16_t *dk, uint16_t *dv, uint64_t kv_stride, uint32_t pos_step, const uint32_t *pos_dev) {
  const uint64_t qp = n_tokens * q_heads * (hd / 2), kp = n_tokens * kv_heads * (hd / 2);
  if (!qp && !kp) return;
  if (!kv_stride) kv_stride = kv_heads * hd;
  rope_kv_kernel<<<dim3(grid1d(qp + kp)), dim3(256), 0, ctx->stream>>>(
      q, qp, (uint32_t)q_heads, k, v, kp, (uint32_t)kv_heads, (uint32_t)hd, tab, pos, pos_step, kv_stride, dk, dv,
      pos_dev, kv_heads * hd);
  hip_check(hipGetLastError(), "rope_kv_write launch");
}

namespace {
// rope: RoPE and the new key's cache write folded in (decode only); the
// cache is written only then. A rope with no k only carries pos_dev (a
// captured decode step reading its position from device memory, kv_len the
// cache capacity): attention alone. False, launching nothing, when q8 or
// rope is asked for a shape without that variant.
bool attn_impl(mdma_ctx *ctx, const float *q, const uint16_t *kc, const uint16_t *vc, float *o, uint64_t n_q,
               uint64_t kv_len, uint64_t hd, uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride,
               const AttnQ8 *q8, const AttnRope *rope_in = nullptr) {
  uint16_t *k = const_cast<uint16_t *>(kc), *v = const_cast<uint16_t *>(vc);
  const uint32_t *pos_dev = rope_in ? rope_in->pos_dev : nullptr;
  const uint64_t GP = n_kv_heads ? n_q_heads / n_kv_heads : 0;
  if (!rope_in && !q8 && !seq_stride && n_q >= ATT_PREFILL_MIN && kv_len >= n_q && (hd == 64 || hd == 128) &&
      n_kv_heads && GP * n_kv_heads == n_q_heads && (GP == 1 || GP == 2 || GP == 4 || GP == 8) &&
      kv_len * n_kv_heads * hd < (1ull << 32) && n_kv_heads < 65536) {
    // A prompt's causal attention on the matrix cores (attn_prefill_kernel).
    const uint64_t QT = 64 / GP, nqb = (n_q + QT - 1) / QT;
    const float sc = 1.0f / sqrtf((float)hd);
    const uint32_t pre = (uint32_t)(kv_len - n_q);
    // Key chunks of ct tiles: about two workgroups per CU (what stays
    // resident) over the prompt's tile work, at least two tiles each; none
    // when no block has more than ct tiles, under stream capture or in a
    // fixed scratch.
    uint64_t units = 0, max_t = 0;
    for (uint64_t b = 0; b < nqb; b++) {
      const uint64_t t = (pre + std::min((b + 1) * QT, n_q) - 1) / 64 + 1;
      units += t;
      max_t = std::max(max_t, t);
    }
    units *= n_kv_heads;
    const uint64_t cus = ctx->cu_count ? ctx->cu_count : 256;
    uint64_t ct = std::max<uint64_t>(2, (units + 2 * cus - 1) / (2 * cus)), n_ch = (max_t + ct - 1) / ct;
    const uint64_t NV = 8 + 4 * (hd / 16), pbytes = n_kv_heads * nqb * n_ch * NV * 256 * 4;
    if (n_ch < 2 || ctx->capturing || ctx->fixed_scratch || pbytes > (256ull << 20)) ct = 0, n_ch = 1;
    float *part = ct ? reinterpret_cast<float *>(scratch(ctx, pbytes)) : nullptr;
    uint32_t *cnt = ct ? attn_counters(ctx, n_kv_heads * nqb) : nullptr;
    // Asked for (a16_want_y == o): also the output projection's f16-path
    // input, into the caller's buffer.
    const uint64_t KO = n_q_heads * hd;
    const bool want = ctx->a16_want_y == o && ctx->a16_want_bytes >= gemm_f16_input_bytes(n_q, KO);
    const F16In fin = want ? gemm_f16_input_at(ctx->a16_want_buf, n_q, KO) : F16In{};
    const dim3 grid((uint32_t)n_kv_heads, (uint32_t)nqb, (uint32_t)n_ch);
#define MDMA_ATTP(GG, HH)                                                                                          \
  attn_prefill_kernel<GG, HH><<<grid, dim3(256), 0, ctx->stream>>>(q, k, v, o, (uint32_t)n_q, pre, (uint32_t)n_q_heads, \
                                                                   (uint32_t)n_kv_heads, sc, (uint32_t)ct, part, cnt, \
                                                                   fin)
    if (hd == 128) {
      if (GP == 1) MDMA_ATTP(1, 128);
      else if (GP == 2) MDMA_ATTP(2, 128);
      else if (GP == 4) MDMA_ATTP(4, 128);
      else MDMA_ATTP(8, 128);
    } else {
      if (GP == 1) MDMA_ATTP(1, 64);
      else if (GP == 2) MDMA_ATTP(2, 64);
      else if (GP == 4) MDMA_ATTP(4, 64);
      else MDMA_ATTP(8, 64);
    }
#undef MDMA_ATTP
    hip_check(hipGetLastError(), "attn prefill launch");
    if (want) a16_mark(ctx, o, n_q, KO, ctx->a16_want_buf, false);
    return true;
  }
  const AttnRope *rope = rope_in && rope_in->k ? rope_in : nullptr;
  if (pos_dev && !(seq_stride || n_q == 1)) return false;
  const float scale = 1.0f / sqrtf((float)hd);
  const uint32_t prefix = (uint32_t)(seq_stride ? kv_len - 1 : kv_len - n_q);
  const uint64_t GQ = n_kv_heads ? n_q_heads / n_kv_heads : 0, C = (hd + 127) / 128;
  // Runs of tiles per (query, KV head): enough workgroups to cover the chip
  // (about MDMA_ATT_WG_TARGET), at least one tile and at most ATT_MAX_RUNS
  // runs each; long prompts use one run per query.
  // A captured step (rope->pos_dev) sizes the grid for the whole cache and
  // the kernel recomputes the runs for the live length with these rules.
  const uint64_t tiles = (kv_len + ATT_TILE - 1) / ATT_TILE, pairs = n_q * n_kv_heads;
  const uint64_t runs0 = std::min<uint64_t>(pairs ? (MDMA_ATT_WG_TARGET + pairs - 1) / pairs : 1, ATT_MAX_RUNS);
  uint64_t n_splits = std::max<uint64_t>(std::min(runs0, tiles), 1);
  const uint64_t tpw = (tiles + n_splits - 1) / n_splits;
  if (!pos_dev) n_splits = tiles ? (tiles + tpw - 1) / tpw : 1;
  // Few workgroups (short contexts, few queries): a KV head's query heads
  // split over MDMA_ATT_SUB workgroups, each reading the same K/V tiles with
  // a share of the heads (less work per workgroup on the critical path).
#ifndef MDMA_ATT_SUB
#define MDMA_ATT_SUB 2
#endif
#ifndef MDMA_ATT_SUB_WG_PER_CU
#define MDMA_ATT_SUB_WG_PER_CU 2
#endif
  uint64_t sub = 1;
  if (MDMA_ATT_SUB > 1 && GQ % MDMA_ATT_SUB == 0 && (!q8 || (GQ / MDMA_ATT_SUB * hd) % 256 == 0) &&
      pairs * n_splits * MDMA_ATT_SUB <= MDMA_ATT_SUB_WG_PER_CU * (uint64_t)ctx->cu_count)
    sub = MDMA_ATT_SUB;
  const uint64_t G = GQ / sub;
  const uint64_t part_bytes = n_splits > 1 ? n_q * n_q_heads * n_splits * (hd + 2) * 4 : 0;
  const bool split_ok = hd % 8 == 0 && hd <= 256 && (G == 1 || G == 2 || G == 4 || G == 8) && G * C <= 8 &&
                        n_splits < 65536 && n_q < 65536 && part_bytes <= (256ull << 20);
  if (q8 && !(split_ok && (G * hd) % 256 == 0)) return false;
  if (rope && !(split_ok && n_q && kv_len && hd % 8 == 0 && (seq_stride || n_q == 1))) return false;
  if (split_ok && n_q && kv_len) {
    float *part = part_bytes ? reinterpret_cast<float *>(scratch(ctx, part_bytes)) : nullptr;
    // Counters for the most sub-groups any launch of this shape may take (a
    // captured step and the eager one may choose differently).
    uint32_t *cnt = part_bytes ? attn_counters(ctx, n_q * n_kv_heads * MDMA_ATT_SUB) : nullptr;
    const AttnQ8 a8 = q8 ? *q8 : AttnQ8{nullptr, nullptr, nullptr};
    AttnRope ar = rope ? *rope : AttnRope{nullptr, nullptr, nullptr, 0, pos_dev, 0};
    ar.runs0 = (uint32_t)runs0;
    const dim3 grid((uint32_t)(n_kv_heads * sub), (uint32_t)n_splits, (uint32_t)n_q);
    // One tile buffer when every run is one tile, or when more workgroups
    // than the two-buffer kernel keeps resident (two per CU) share the chip:
    // a captured step sized for a long cache runs one-tile runs at short
    // lengths, and there occupancy counts more than the prefetch.
    const bool one = tpw == 1 || (uint64_t)grid.x * grid.y * grid.z > 2 * (uint64_t)ctx->cu_count;
#define MDMA_ATT_GO1(GG, CC, QQ, RR, OO)                                                                       \
  attn_split_kernel<GG, CC, QQ, RR, OO><<<grid, dim3(256), 0, ctx->stream>>>(                                  \
      q, k, v, o, part, cnt, prefix, (uint32_t)hd, (uint32_t)n_q_heads, (uint32_t)n_kv_heads, scale, seq_stride, \
      (uint32_t)tpw, a8, ar)
#define MDMA_ATT_GO(GG, CC, QQ, RR)          \
  do {                                       \
    if (one) MDMA_ATT_GO1(GG, CC, QQ, RR, true);  \
    else MDMA_ATT_GO1(GG, CC, QQ, RR, false); \
  } while (0)
#define MDMA_ATT(GG, CC)                                \
  do {                                                  \
    if (q8 && rope) MDMA_ATT_GO(GG, CC, true, true);    \
    else if (q8) MDMA_ATT_GO(GG, CC, true, false);      \
    else if (rope) MDMA_ATT_GO(GG, CC, false, true);    \
    else MDMA_ATT_GO(GG, CC, false, false);             \
  } while (0)
    if (C == 1) {
      if (G == 1) MDMA_ATT(1, 1);
      else if (G == 2) MDMA_ATT(2, 1);
      else if (G == 4) MDMA_ATT(4, 1);
      else MDMA_ATT(8, 1);
    } else {
      if (G == 1) MDMA_ATT(1, 2);
      else if (G == 2) MDMA_ATT(2, 2);
      else MDMA_ATT(4, 2);
    }
#undef MDMA_ATT
#undef MDMA_ATT_GO
#undef MDMA_ATT_GO1
    hip_check(hipGetLastError(), "attn launch");
    return true;
  }
  attn_kernel<<<dim3((uint32_t)n_q_heads, (uint32_t)n_q), dim3(256), 0, ctx->stream>>>(
      q, k, v, o, prefix, (uint32_t)hd, (uint32_t)n_q_heads, (uint32_t)n_kv_heads, scale, seq_stride, pos_dev);
  hip_check(hipGetLastError(), "attn launch");
  return true;
}
}  // namespace

void launch_attn(mdma_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t n_q,
                 uint64_t kv_len, uint64_t hd, uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride,
                 const uint32_t *pos_dev) {
  const AttnRope pd{nullptr, nullptr, nullptr, 0, pos_dev, 0};
  if (!attn_impl(ctx, q, k, v, o, n_q, kv_len, hd, n_q_heads, n_kv_heads, seq_stride, nullptr,
                 pos_dev ? &pd : nullptr))
    fail(MDMA_ERR_BACKEND, "attn: no launch reads the position from device memory for this shape");
}

bool launch_attn_q8(mdma_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t n_q,
                    uint64_t kv_len, uint64_t hd, uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride,
                    const uint32_t *pos_dev) {
  const uint64_t n_in = n_q_heads * hd;
  if (!n_q || !kv_len || n_in % 256) return false;
  AttnQ8 a8;
  q8_slots(ctx, n_q, n_in, &a8.q, &a8.d, &a8.s16);
  const AttnRope pd{nullptr, nullptr, nullptr, 0, pos_dev, 0};
  if (!attn_impl(ctx, q, k, v, o, n_q, kv_len, hd, n_q_heads, n_kv_heads, seq_stride, &a8, pos_dev ? &pd : nullptr))
    return false;
  q8_mark(ctx, o, n_q, n_in);
  return true;
}

bool launch_attn_rope(mdma_ctx *ctx, const float *q, const float *k, const float *v, const float *tab, uint32_t pos,
                      uint16_t *kc, uint16_t *vc, float *o, uint64_t n_q, uint64_t kv_len, uint64_t hd,
                      uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride, bool int8_out,
                      const uint32_t *pos_dev) {
  if (!n_q || !kv_len || (!pos_dev && pos != kv_len - 1)) return false;
  const AttnRope rp{k, v, tab, pos, pos_dev, 0};
  if (!int8_out)
    return attn_impl(ctx, q, kc, vc, o, n_q, kv_len, hd, n_q_heads, n_kv_heads, seq_stride, nullptr, &rp);
  const uint64_t n_in = n_q_heads * hd;
  if (n_in % 256) return false;
  AttnQ8 a8;
  q8_slots(ctx, n_q, n_in, &a8.q, &a8.d, &a8.s16);
  if (!attn_impl(ctx, q, kc, vc, o, n_q, kv_len, hd, n_q_heads, n_kv_heads, seq_stride, &a8, &rp)) return false;
  q8_mark(ctx, o, n_q, n_in);
  return true;
}

namespace {
struct U32x4 {
  uint32_t v[4];
};
__global__ void set_u32_kernel(uint32_t *p, U32x4 vals, int n) {
  for (int i = 0; i < n; i++) p[i] = vals.v[i];
}
__global__ __launch_bounds__(1024) void step_record_kernel(uint32_t *params, const uint32_t *cur,
                                                           const uint32_t *cur_flag, uint32_t *hist,
                                                           uint32_t *hist_flag, uint32_t B) {
  const uint32_t step = params[1];
  for (uint32_t b = threadIdx.x; b < B; b += blockDim.x) {
    hist[(size_t)step * B + b] = cur[b];
    hist_flag[(size_t)step * B + b] = cur_flag[b];
  }
  __syncthreads();  // every thread has read the step before it advances
  if (threadIdx.x == 0) {
    params[0] += 1;
    params[1] += 1;
  }
}
}  // namespace

void launch_set_u32(mdma_ctx *ctx, uint32_t *p, const uint32_t *vals, int n) {
  if (n < 1 || n > 4) fail(MDMA_ERR_BACKEND, "set_u32: 1 to 4 values");
  U32x4 v{};
  for (int i = 0; i < n; i++) v.v[i] = vals[i];
  set_u32_kernel<<<dim3(1), dim3(1), 0, ctx->stream>>>(p, v, n);
  hip_check(hipGetLastError(), "set_u32 launch");
}

void launch_step_record(mdma_ctx *ctx, uint32_t *params, const uint32_t *cur, const uint32_t *cur_flag,
                        uint32_t *hist, uint32_t *hist_flag, uint32_t B) {
  step_record_kernel<<<dim3(1), dim3(B < 1024 ? (B + 63) / 64 * 64 : 1024), 0, ctx->stream>>>(
      params, cur, cur_flag, hist, hist_flag, B);
  hip_check(hipGetLastError(), "step_record launch");
}

void launch_argmax_rows(mdma_ctx *ctx, const float *x, uint64_t rows, uint64_t n, uint32_t *idx, uint32_t *flag) {
  const uint32_t nchunks = (uint32_t)((n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK);
  if (nchunks <= 1 || rows > 65535) {
    argmax_rows_kernel<<<dim3((uint32_t)rows), dim3(1024), 0, ctx->stream>>>(x, n, idx, flag);
  } else {
    ArgPart *part = reinterpret_cast<ArgPart *>(argmax_parts(ctx, rows * nchunks));
    argmax_part_kernel<<<dim3(nchunks, (uint32_t)rows), dim3(256), 0, ctx->stream>>>(x, n, part);
    argmax_final_kernel<<<dim3((uint32_t)rows), dim3(64), 0, ctx->stream>>>(part, nchunks, idx, flag);
  }
  hip_check(hipGetLastError(), "argmax_rows launch");
}

}  // namespace mdma
