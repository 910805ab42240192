// Per-token Llama ops on gfx950: embedding gather, RMSNorm (optionally fused
// with the residual add), elementwise add and SiLU-gate, interleaved RoPE from
// a host-built angle table, f16 KV writes, causal GQA attention over the f16
// cache, and greedy argmax. Semantics follow the reference CPU backend
// (/root/reference/src/backend/cpu.rs) op for op; these are simple, correct
// kernels, not the hot path.
#include "internal.h"

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

__global__ void add_kernel(const float *__restrict__ a, const float *__restrict__ b, float *__restrict__ y, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    y[i] = a[i] + b[i];
}

// silu_mul (cpu.rs:447-458): y = (g / (1 + exp(-g))) * u.
__global__ void silu_mul_kernel(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ y,
                                size_t n) {
#pragma clang fp contract(off)
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float gv = g[i];
    const float s = gv / (1.0f + expf(-gv));
    y[i] = s * u[i];
  }
}

// Interleaved-pair rotation (apply_rope, cpu.rs:68-84) of one pair.
__device__ __forceinline__ void rot(float &x0, float &x1, float c, float s) {
#pragma clang fp contract(off)
  const float a = x0 * c, bb = x1 * s, cc = x0 * s, d = x1 * c;
  x0 = a - bb;
  x1 = cc + d;
}

// x: [n_tokens, heads, hd]; tab: [pos][hd/2] (cos, sin).
__global__ void rope_kernel(float *__restrict__ x, uint32_t heads, uint32_t hd, uint64_t pairs,
                            const float *__restrict__ tab, uint32_t pos) {
  const uint32_t half = hd / 2;
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

__global__ void kv_write_kernel(const float *__restrict__ k, const float *__restrict__ v, uint16_t *__restrict__ dk,
                                uint16_t *__restrict__ dv, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    dk[i] = f2h(k[i]);
    dv[i] = f2h(v[i]);
  }
}

// Fused rope_kv_write (backend.rs:452-467): q rotated in place; k rotated and
// stored with v as f16 rows. Token t sits at position pos + t*pos_step and
// its cache row starts kv_stride elements after token t-1's (kv_stride =
// the row width for one sequence; a cache-to-cache stride when each token
// is a different sequence of a batch, with pos_step 0).
__global__ void rope_kv_kernel(float *__restrict__ q, uint64_t q_pairs, uint32_t q_heads, const float *__restrict__ k,
                               const float *__restrict__ v, uint64_t k_pairs, uint32_t kv_heads, uint32_t hd,
                               const float *__restrict__ tab, uint32_t pos, uint32_t pos_step, uint64_t kv_stride,
                               uint16_t *__restrict__ dk, uint16_t *__restrict__ dv) {
  const uint32_t half = hd / 2;
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
                                                   uint32_t n_kv_heads, float scale, uint64_t seq_stride) {
  __shared__ float qs[256];
  __shared__ float sc[ATT_CHUNK];
  __shared__ float red[4];
  const uint32_t qh = blockIdx.x, i = blockIdx.y;
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

// Greedy argmax (sampler.rs:64-74): largest by total order, ties to the last
// index; out[1] flags any non-finite logit.
__device__ __forceinline__ int32_t total_key(float f) {
  const int32_t b = __builtin_bit_cast(int32_t, f);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
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

__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ x, uint64_t n, uint32_t *out) {
  __shared__ int32_t sk[16];
  __shared__ uint32_t si[16];
  __shared__ uint32_t sbad[16];
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
  // Reduce (key, index): larger key wins; equal keys keep the larger index.
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
    uint32_t idx = si[0], fl = sbad[0];
    for (int j = 1; j < 16; j++) {
      fl |= sbad[j];
      if ((uint64_t)j * 64 >= n) continue;
      if (sk[j] > k || (sk[j] == k && si[j] > idx)) {
        k = sk[j];
        idx = si[j];
      }
    }
    out[0] = idx;
    out[1] = fl;
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
  rmsnorm_kernel<<<dim3((uint32_t)rows), dim3(256), 0, ctx->stream>>>(w, (uint32_t)dim, a, b, sum, y, eps);
  hip_check(hipGetLastError(), "rmsnorm launch");
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
                 uint32_t pos) {
  const uint64_t pairs = n_tokens * heads * (hd / 2);
  if (!pairs) return;
  rope_kernel<<<dim3(grid1d(pairs)), dim3(256), 0, ctx->stream>>>(x, (uint32_t)heads, (uint32_t)hd, pairs, tab, pos);
  hip_check(hipGetLastError(), "rope launch");
}

void launch_kv_write(mdma_ctx *ctx, const float *k, const float *v, uint16_t *dk, uint16_t *dv, uint64_t n) {
  kv_write_kernel<<<dim3(grid1d(n)), dim3(256), 0, ctx->stream>>>(k, v, dk, dv, n);
  hip_check(hipGetLastError(), "kv_write launch");
}

void launch_rope_kv_write(mdma_ctx *ctx, float *q, uint64_t q_heads, const float *k, const float *v,
                          uint64_t kv_heads, uint64_t hd, uint64_t n_tokens, const float *tab, uint32_t pos,
                          uint16_t *dk, uint16_t *dv, uint64_t kv_stride, uint32_t pos_step) {
  const uint64_t qp = n_tokens * q_heads * (hd / 2), kp = n_tokens * kv_heads * (hd / 2);
  if (!qp && !kp) return;
  if (!kv_stride) kv_stride = kv_heads * hd;
  rope_kv_kernel<<<dim3(grid1d(qp + kp)), dim3(256), 0, ctx->stream>>>(
      q, qp, (uint32_t)q_heads, k, v, kp, (uint32_t)kv_heads, (uint32_t)hd, tab, pos, pos_step, kv_stride, dk, dv);
  hip_check(hipGetLastError(), "rope_kv_write launch");
}

void launch_attn(mdma_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t n_q,
                 uint64_t kv_len, uint64_t hd, uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride) {
  const float scale = 1.0f / sqrtf((float)hd);
  const uint32_t prefix = (uint32_t)(seq_stride ? kv_len - 1 : kv_len - n_q);
  attn_kernel<<<dim3((uint32_t)n_q_heads, (uint32_t)n_q), dim3(256), 0, ctx->stream>>>(
      q, k, v, o, prefix, (uint32_t)hd, (uint32_t)n_q_heads, (uint32_t)n_kv_heads, scale, seq_stride);
  hip_check(hipGetLastError(), "attn launch");
}

void launch_argmax(mdma_ctx *ctx, const float *x, uint64_t n, uint32_t *out_dev) {
  argmax_kernel<<<dim3(1), dim3(1024), 0, ctx->stream>>>(x, n, out_dev);
  hip_check(hipGetLastError(), "argmax launch");
}

void launch_argmax_rows(mdma_ctx *ctx, const float *x, uint64_t rows, uint64_t n, uint32_t *idx, uint32_t *flag) {
  argmax_rows_kernel<<<dim3((uint32_t)rows), dim3(1024), 0, ctx->stream>>>(x, n, idx, flag);
  hip_check(hipGetLastError(), "argmax_rows launch");
}

}  // namespace mdma
