/*
 * CPU oracle for the quantized-weight path: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of mdma's CPU backend, the reference's own parity
 * oracle. Citations are path:line inside the reference checkout
 * (/root/reference). It must be compiled with -ffp-contract=off and without
 * fast-math: Rust never contracts a*b+c into an FMA, and every reduction
 * below runs in the reference's sequential order.
 *
 * The block decoders follow candle-core 0.11.0's GgmlType::to_float
 * (Cargo.lock:465-468; called from src/backend/cpu/dequant.rs:36), which is
 * not vendored in the reference. Their formulas are pinned by the reference's
 * own known-answer test (src/cache/layout/tests.rs:8-55, restated in
 * tests/test_oracle.py) and by closed forms checked in tests/test_oracle.py.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library. The product library (mdma_amd/) never links or calls it.
 */
#include "oracle.h"

#include <math.h>
#include <time.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

enum { OK = 0, SHAPE = 2 };

/* ---- f16 <-> f32 (the `half` crate, Cargo.lock:1535: exact widening, RNE narrowing) ---- */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xff;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) /* inf / NaN (NaN keeps a quiet payload bit) */
        return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0));
    int e = (int)exp - 127 + 15;
    if (e >= 31)
        return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) { /* subnormal or zero in f16 */
        if (e < -10)
            return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1)))
            half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1)))
        half++; /* may carry into the exponent, which is the correct rounding */
    return (uint16_t)half;
}

static float ld_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ---- block geometry (src/backend/dtype_code.rs:45-52; GGUF block formats) ---- */

size_t orc_block_size(int dtype) {
    switch (dtype) {
    case ORC_F32:
    case ORC_F16:
        return 1;
    case ORC_Q8_0:
        return 32;
    case ORC_Q4_K:
    case ORC_Q6_K:
        return 256;
    default:
        return 0;
    }
}

size_t orc_type_size(int dtype) {
    switch (dtype) {
    case ORC_F32:
        return 4;
    case ORC_F16:
        return 2;
    case ORC_Q8_0:
        return 34;
    case ORC_Q4_K:
        return 144;
    case ORC_Q6_K:
        return 210;
    default:
        return 0;
    }
}

/* get_scale_min_k4 as restated in src/backend/rocm/kernels/kernels.hip:19-27. */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Q8_0: y = q * d (one rounding). GGUF block {f16 d; i8 qs[32]}. */
static void deq_q8_0(const uint8_t *b, float *y) {
    float d = ld_f16(b);
    const int8_t *qs = (const int8_t *)(b + 2);
    for (int j = 0; j < 32; j++)
        y[j] = (float)qs[j] * d;
}

/* Q4_K: y = (d*sc)*q - dmin*m, sub-block pairs of 64 share 32 quant bytes
 * (low nibbles first). Block {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}.
 * Order of roundings as src/backend/rocm/kernels/kernels.hip:44-68. */
static void deq_q4_k(const uint8_t *b, float *y) {
    float d = ld_f16(b), dmin = ld_f16(b + 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    for (int j = 0; j < 4; j++) {
        uint8_t sc, m;
        scale_min_k4(2 * j, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        scale_min_k4(2 * j + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = dmin * (float)m;
        const uint8_t *q = qs + 32 * j;
        for (int l = 0; l < 32; l++)
            y[64 * j + l] = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; l++)
            y[64 * j + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
    }
}

/* Q6_K: y = (d*sc)*q with q in [-32, 31] from 4 low bits (ql) and 2 high
 * bits (qh). Block {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}.
 * Layout as src/backend/rocm/kernels/kernels.hip:82-122. */
static void deq_q6_k(const uint8_t *b, float *y) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = ld_f16(b + 208);
    /* Column 128n + 32r + l: quarter r of half n takes the low (r < 2) or high
     * nibble of ql[64n + 32(r & 1) + l], bits 2r..2r+1 of qh[32n + l], and the
     * scale sc[8n + 2r + l/16]. Written quarter by quarter, 16 columns of one
     * scale at a time, so the compiler vectorizes the inner loop. */
    for (int n = 0; n < 2; n++)
        for (int r = 0; r < 4; r++) {
            const uint8_t *l8 = ql + 64 * n + 32 * (r & 1), *h8 = qh + 32 * n;
            const int sl = 4 * (r >> 1), sh = 2 * r;
            for (int h = 0; h < 2; h++) {
                float ds = d * (float)sc[8 * n + 2 * r + h];
                float *yy = y + 128 * n + 32 * r + 16 * h;
                for (int l = 0; l < 16; l++) {
                    int q = (int)(((l8[16 * h + l] >> sl) & 0xF) | (((h8[16 * h + l] >> sh) & 3) << 4)) - 32;
                    yy[l] = ds * (float)q;
                }
            }
        }
}

/* dequantize_row: src/backend/cpu/dequant.rs:13-58 (whole blocks only). */
int orc_dequantize_row(int dtype, const uint8_t *bytes, size_t n_bytes, float *out, size_t n) {
    size_t bs = orc_block_size(dtype), ts = orc_type_size(dtype);
    if (!bs || n % bs || n_bytes != (n / bs) * ts)
        return SHAPE;
    size_t nb = n / bs;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = bytes + i * ts;
        switch (dtype) {
        case ORC_F32:
            memcpy(out + i, b, 4);
            break;
        case ORC_F16:
            out[i] = ld_f16(b);
            break;
        case ORC_Q8_0:
            deq_q8_0(b, out + 32 * i);
            break;
        case ORC_Q4_K:
            deq_q4_k(b, out + 256 * i);
            break;
        case ORC_Q6_K:
            deq_q6_k(b, out + 256 * i);
            break;
        }
    }
    return OK;
}

/* dot: src/backend/cpu.rs:46-48. `iter().map(a*b).sum()` folds from -0.0 in
 * iteration order; each product is rounded before the add (no FMA). */
static float dot(const float *a, const float *b, size_t n) {
    float s = -0.0f;
    for (size_t i = 0; i < n; i++) {
        float p = a[i] * b[i];
        s = s + p;
    }
    return s;
}

/* shape::matmul (src/backend/shape.rs:51-73) + kquant_aligned (:76-84). */
static int matmul_shape(int dtype, size_t n_out, size_t n_in, size_t x_elems, size_t y_elems,
                        size_t *n_tokens) {
    if (!n_out || !n_in)
        return SHAPE;
    if (!x_elems || x_elems % n_in)
        return SHAPE;
    size_t bs = orc_block_size(dtype);
    if (!bs || n_in % bs)
        return SHAPE;
    *n_tokens = x_elems / n_in;
    if (y_elems < *n_tokens * n_out)
        return SHAPE;
    return OK;
}

typedef struct {
    int dtype;
    const uint8_t *w;
    size_t row_bytes, n_out, n_in, n_tokens, r0, r1;
    const float *x;
    float *y;
    int status;
} qm_job;

/* Eight rows' dots with one token at once: lane k of the vectors is row k's
 * own sequential sum (from -0.0, each product rounded, no FMA), so every
 * output equals dot(row_k, x, n) bit for bit; the independent chains only
 * run side by side (eight rows per vector, four tokens per pass), which
 * also reads x once per eight rows instead of once per row. wt holds the
 * eight dequantized rows interleaved, [n][8]. */
typedef float orc_v8 __attribute__((vector_size(32)));

static void dots_8rows(const orc_v8 *wt, size_t n, const float *const *x, int nt, orc_v8 *out) {
    const orc_v8 z = {-0.0f, -0.0f, -0.0f, -0.0f, -0.0f, -0.0f, -0.0f, -0.0f};
    orc_v8 s0 = z, s1 = z, s2 = z, s3 = z;
    if (nt == 4) {
        for (size_t i = 0; i < n; i++) {
            orc_v8 p0 = wt[i] * x[0][i], p1 = wt[i] * x[1][i], p2 = wt[i] * x[2][i], p3 = wt[i] * x[3][i];
            s0 = s0 + p0;
            s1 = s1 + p1;
            s2 = s2 + p2;
            s3 = s3 + p3;
        }
    } else {
        for (size_t i = 0; i < n; i++) {
            orc_v8 p0 = wt[i] * x[0][i];
            s0 = s0 + p0;
        }
    }
    out[0] = s0, out[1] = s1, out[2] = s2, out[3] = s3;
}

static void *qm_worker(void *arg) {
    qm_job *j = (qm_job *)arg;
    float *row = (float *)malloc(j->n_in * sizeof(float));
    orc_v8 *wt = (orc_v8 *)aligned_alloc(32, j->n_in * sizeof(orc_v8));
    if (!row || !wt) {
        free(row);
        free(wt);
        j->status = SHAPE;
        return NULL;
    }
    for (size_t r0 = j->r0; r0 < j->r1; r0 += 8) {
        size_t nr = j->r1 - r0 < 8 ? j->r1 - r0 : 8;
        for (size_t k = 0; k < 8; k++) { /* rows past the block's end repeat its last row */
            size_t r = r0 + (k < nr ? k : nr - 1);
            if (orc_dequantize_row(j->dtype, j->w + r * j->row_bytes, j->row_bytes, row, j->n_in)) {
                j->status = SHAPE;
                goto done;
            }
            for (size_t i = 0; i < j->n_in; i++)
                wt[i][k] = row[i];
        }
        for (size_t t = 0; t < j->n_tokens;) {
            int nt = j->n_tokens - t >= 4 ? 4 : 1;
            const float *xs[4];
            for (int q = 0; q < 4; q++)
                xs[q] = j->x + (t + (size_t)(q < nt ? q : 0)) * j->n_in;
            orc_v8 o[4];
            dots_8rows(wt, j->n_in, xs, nt, o);
            for (int q = 0; q < nt; q++)
                for (size_t k = 0; k < nr; k++)
                    j->y[(t + (size_t)q) * j->n_out + r0 + k] = o[q][k];
            t += (size_t)nt;
        }
    }
done:
    free(row);
    free(wt);
    return NULL;
}

/* CpuBackend::qmatmul: src/backend/cpu.rs:335-368. Rows are independent
 * (dequantized once, dotted against each token in order), so splitting rows
 * across threads does not change any element. */
int orc_qmatmul(int dtype, const uint8_t *w, size_t w_bytes, size_t n_out, size_t n_in,
                const float *x, size_t x_elems, float *y, size_t y_elems, int n_threads) {
    size_t T;
    if (matmul_shape(dtype, n_out, n_in, x_elems, y_elems, &T))
        return SHAPE;
    size_t row_bytes = orc_type_size(dtype) * (n_in / orc_block_size(dtype));
    if (w_bytes < row_bytes * n_out)
        return SHAPE;
    if (n_threads < 1)
        n_threads = 1;
    if ((size_t)n_threads > n_out)
        n_threads = (int)n_out;
    qm_job *jobs = (qm_job *)calloc((size_t)n_threads, sizeof(qm_job));
    pthread_t *th = (pthread_t *)calloc((size_t)n_threads, sizeof(pthread_t));
    size_t per = (n_out + (size_t)n_threads - 1) / (size_t)n_threads;
    per = (per + 7) / 8 * 8; /* whole blocks of eight rows per thread */
    for (int i = 0; i < n_threads; i++) {
        qm_job *j = &jobs[i];
        j->dtype = dtype;
        j->w = w;
        j->row_bytes = row_bytes;
        j->n_out = n_out;
        j->n_in = n_in;
        j->n_tokens = T;
        j->x = x;
        j->y = y;
        j->r0 = (size_t)i * per;
        j->r1 = j->r0 + per < n_out ? j->r0 + per : n_out;
        if (j->r0 > n_out)
            j->r0 = n_out;
    }
    for (int i = 1; i < n_threads; i++)
        pthread_create(&th[i], NULL, qm_worker, &jobs[i]);
    qm_worker(&jobs[0]);
    int st = jobs[0].status;
    for (int i = 1; i < n_threads; i++) {
        pthread_join(th[i], NULL);
        st |= jobs[i].status;
    }
    free(jobs);
    free(th);
    return st ? SHAPE : OK;
}

/* CpuBackend::embed: src/backend/cpu.rs:370-384 with shape::embed (:92). */
int orc_embed(int dtype, const uint8_t *table, size_t table_bytes, size_t vocab, size_t n_embd,
              const uint32_t *ids, size_t n_ids, float *out, size_t out_elems) {
    size_t bs = orc_block_size(dtype);
    if (!vocab || !n_embd || !n_ids || out_elems < n_ids * n_embd || !bs || n_embd % bs)
        return SHAPE;
    size_t row_bytes = orc_type_size(dtype) * (n_embd / bs);
    for (size_t t = 0; t < n_ids; t++) {
        if (ids[t] >= vocab || (ids[t] + 1) * row_bytes > table_bytes)
            return SHAPE;
        orc_dequantize_row(dtype, table + ids[t] * row_bytes, row_bytes, out + t * n_embd, n_embd);
    }
    return OK;
}

/* CpuBackend::rmsnorm: src/backend/cpu.rs:388-402; shape::rows (shape.rs:113). */
int orc_rmsnorm(const float *w, size_t dim, const float *x, size_t x_elems, float *y,
                size_t y_elems, float eps) {
    if (!dim || !x_elems || x_elems % dim || y_elems < x_elems)
        return SHAPE;
    for (size_t r = 0; r < x_elems / dim; r++) {
        const float *row = x + r * dim;
        float *o = y + r * dim;
        float mean_sq = dot(row, row, dim) / (float)dim;
        float scale = 1.0f / sqrtf(mean_sq + eps);
        for (size_t i = 0; i < dim; i++) {
            float t = row[i] * scale;
            o[i] = t * w[i];
        }
    }
    return OK;
}

/* CpuBackend::add: src/backend/cpu.rs:420-429. */
int orc_add(const float *a, const float *b, size_t n, float *y) {
    for (size_t i = 0; i < n; i++)
        y[i] = a[i] + b[i];
    return OK;
}

/* Backend::add_rmsnorm default: src/backend.rs:502-513 (add, then rmsnorm of the sum). */
int orc_add_rmsnorm(const float *w, size_t dim, const float *a, const float *b, size_t n,
                    float *sum, float *y, float eps) {
    orc_add(a, b, n, sum);
    return orc_rmsnorm(w, dim, sum, n, y, n, eps);
}

/* CpuBackend::silu_mul: src/backend/cpu.rs:447-458. */
int orc_silu_mul(const float *gate, const float *up, size_t n, float *y) {
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float silu = g / (1.0f + expf(-g));
        y[i] = silu * up[i];
    }
    return OK;
}

/* The angle table of apply_rope (src/backend/cpu.rs:68-84) at one position:
 * freq_i = theta^(-2i/head_dim) by powf, (sin, cos) of pos*freq_i. */
void orc_rope_cos_sin(uint32_t pos, size_t head_dim, float theta, float *cos_out, float *sin_out) {
    size_t half = head_dim / 2;
    for (size_t i = 0; i < half; i++) {
        float ex = -2.0f * (float)i / (float)head_dim;
        float freq = powf(theta, ex);
        float a = (float)pos * freq;
        sin_out[i] = sinf(a);
        cos_out[i] = cosf(a);
    }
}

static void apply_rope(float *buf, size_t elems, uint32_t pos, size_t n_tokens, size_t hd,
                       float theta) {
    size_t stride = elems / n_tokens, half = hd / 2;
    float *cs = (float *)malloc(half * sizeof(float)), *sn = (float *)malloc(half * sizeof(float));
    for (size_t t = 0; t < n_tokens; t++) {
        orc_rope_cos_sin(pos + (uint32_t)t, hd, theta, cs, sn);
        for (size_t h = 0; h < stride / hd; h++) {
            float *head = buf + t * stride + h * hd;
            for (size_t i = 0; i < half; i++) {
                float x0 = head[2 * i], x1 = head[2 * i + 1];
                float a = x0 * cs[i], b = x1 * sn[i];
                float c = x0 * sn[i], d = x1 * cs[i];
                head[2 * i] = a - b;
                head[2 * i + 1] = c + d;
            }
        }
    }
    free(cs);
    free(sn);
}

/* CpuBackend::rope: src/backend/cpu.rs:404-418 with shape::rope (shape.rs:146). */
int orc_rope(float *q, size_t q_elems, float *k, size_t k_elems, uint32_t pos, size_t n_tokens,
             size_t head_dim, float theta) {
    if (!n_tokens || q_elems % n_tokens || k_elems % n_tokens)
        return SHAPE;
    size_t qs = q_elems / n_tokens, ks = k_elems / n_tokens;
    if (!head_dim || head_dim % 2 || qs % head_dim || ks % head_dim)
        return SHAPE;
    apply_rope(q, q_elems, pos, n_tokens, head_dim, theta);
    apply_rope(k, k_elems, pos, n_tokens, head_dim, theta);
    return OK;
}

/* softmax_inplace: src/backend/cpu.rs:50-60. */
static void softmax_inplace(float *xs, size_t n) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++)
        mx = fmaxf(mx, xs[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        xs[i] = expf(xs[i] - mx);
        sum += xs[i];
    }
    for (size_t i = 0; i < n; i++)
        xs[i] /= sum;
}

/* CpuBackend::attention with window 0 and scale 1/sqrt(head_dim):
 * src/backend/cpu.rs:437-445, 530-590; shape::attn (shape.rs:291). */
int orc_attention(const float *q, size_t q_elems, const float *k, const float *v, size_t kv_elems,
                  size_t kv_len, size_t hd, size_t n_q_heads, size_t n_kv_heads, float *o,
                  size_t o_elems) {
    size_t per = n_q_heads * hd;
    if (!per || !q_elems || q_elems % per)
        return SHAPE;
    if (!n_kv_heads || n_q_heads % n_kv_heads)
        return SHAPE;
    size_t n_q = q_elems / per;
    if (n_q > kv_len)
        return SHAPE;
    size_t kv_row = n_kv_heads * hd;
    if (kv_elems < kv_len * kv_row || o_elems < q_elems)
        return SHAPE;
    size_t prefix = kv_len - n_q, group = n_q_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)hd);
    float *scores = (float *)malloc((kv_len ? kv_len : 1) * sizeof(float));
    memset(o, 0, n_q * per * sizeof(float));
    for (size_t i = 0; i < n_q; i++) {
        size_t visible = prefix + i + 1;
        for (size_t qh = 0; qh < n_q_heads; qh++) {
            size_t kvh = qh / group;
            const float *qv = q + (i * n_q_heads + qh) * hd;
            for (size_t t = 0; t < visible; t++)
                scores[t] = dot(qv, k + t * kv_row + kvh * hd, hd) * scale;
            softmax_inplace(scores, visible);
            float *ov = o + (i * n_q_heads + qh) * hd;
            for (size_t t = 0; t < visible; t++) {
                const float *vv = v + t * kv_row + kvh * hd;
                for (size_t e = 0; e < hd; e++) {
                    float p = scores[t] * vv[e];
                    ov[e] = ov[e] + p;
                }
            }
        }
    }
    free(scores);
    return OK;
}

/* greedy / argmax: src/sampler.rs:64-74. Iterator::max_by with total_cmp
 * returns the LAST of equal maxima; an empty slice gives 0. */
static int32_t total_key(float f) {
    int32_t b;
    memcpy(&b, &f, 4);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

uint32_t orc_greedy(const float *logits, size_t n) {
    if (!n)
        return 0;
    size_t best = 0;
    int32_t bk = total_key(logits[0]);
    for (size_t i = 1; i < n; i++) {
        int32_t k = total_key(logits[i]);
        if (k >= bk) {
            bk = k;
            best = i;
        }
    }
    return (uint32_t)best;
}

/* ---- int8 activation mode ----
 * The reference quantizes activations per 32 with an f16 scale (Q8_1,
 * src/backend/rocm/kernels/kernels.hip:1102-1133; host restatement
 * src/backend/rocm/decode/tests.rs:68-77): amax from a fold starting at 0,
 * inv = 127/amax (0 for an all-zero block), q = round-half-away(x*inv).
 * The gfx950 mode keeps that rule with an f32 scale d = amax/127 per `group`
 * values (256 for decode GEMV, 32 for prefill GEMM), and records the exact
 * sum of every 16 quants for the K-quant min/offset terms. */
int orc_quantize_act(const float *x, size_t n, size_t group, int8_t *q, float *d, int32_t *sum16) {
    if (!group || group % 16 || n % group)
        return SHAPE;
    for (size_t g = 0; g < n / group; g++) {
        const float *xs = x + g * group;
        float amax = 0.0f;
        for (size_t i = 0; i < group; i++)
            amax = fmaxf(amax, fabsf(xs[i]));
        d[g] = amax / 127.0f;
        float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
        for (size_t i = 0; i < group; i++) {
            float r = roundf(xs[i] * inv);
            if (r > 127.0f)
                r = 127.0f;
            if (r < -127.0f)
                r = -127.0f;
            q[g * group + i] = (int8_t)r;
        }
    }
    if (sum16)
        for (size_t s = 0; s < n / 16; s++) {
            int32_t acc = 0;
            for (int i = 0; i < 16; i++)
                acc += q[16 * s + i];
            sum16[s] = acc;
        }
    return OK;
}

/* Integer quant of weight element e of a block, as the block decoders above
 * read it (Q4_K: 0..15, Q6_K: -32..31, Q8_0: -128..127). */
static int wq_int(int dtype, const uint8_t *b, int e) {
    if (dtype == ORC_Q8_0)
        return ((const int8_t *)(b + 2))[e];
    if (dtype == ORC_Q4_K) {
        int j = e / 64, l = e % 32, hi = (e % 64) >= 32;
        uint8_t byte = b[16 + 32 * j + l];
        return hi ? byte >> 4 : byte & 0xF;
    }
    /* Q6_K */
    int n = e / 128, r = (e % 128) / 32, l = e % 32;
    uint8_t lq = b[64 * n + l + 32 * (r & 1)];
    int low = (r < 2) ? (lq & 0xF) : (lq >> 4);
    int high = (b[128 + 32 * n + l] >> (2 * r)) & 3;
    return (low | (high << 4)) - 32;
}

/* Per-(token, row, sub-block) int32 dot of weight quants with activation
 * quants: the integer accumulator the int8-mode kernels keep per block.
 * Sub-blocks are 32 wide for Q4_K and Q8_0 and 16 wide for Q6_K.
 * out is [n_tokens][n_out][n_in / sub]. */
int orc_block_dot_i32(int dtype, const uint8_t *w, size_t w_bytes, size_t n_out, size_t n_in,
                      const int8_t *qx, size_t n_tokens, int32_t *out) {
    size_t bs = orc_block_size(dtype), ts = orc_type_size(dtype);
    if (dtype != ORC_Q8_0 && dtype != ORC_Q4_K && dtype != ORC_Q6_K)
        return SHAPE;
    if (!n_in || n_in % bs || w_bytes < n_out * (n_in / bs) * ts)
        return SHAPE;
    size_t sub = dtype == ORC_Q6_K ? 16 : 32, nsub = n_in / sub, row_bytes = (n_in / bs) * ts;
    for (size_t t = 0; t < n_tokens; t++)
        for (size_t r = 0; r < n_out; r++)
            for (size_t s = 0; s < nsub; s++) {
                int32_t acc = 0;
                for (size_t i = 0; i < sub; i++) {
                    size_t e = s * sub + i;
                    const uint8_t *b = w + r * row_bytes + (e / bs) * ts;
                    acc += wq_int(dtype, b, (int)(e % bs)) * qx[t * n_in + e];
                }
                out[(t * n_out + r) * nsub + s] = acc;
            }
    return OK;
}

/* ---- Llama decode ---- */

typedef struct {
    float *x, *x_alt, *normed, *q, *k, *v, *attn_out, *proj, *gate, *up, *act;
} orc_ws;

/* Activation group of the device's int8 mode for one GEMV of T tokens: 32
 * where it runs the prefill GEMM (T >= 64 on Q8_0 rows of whole 128-column
 * tiles or Q4_K / Q6_K rows of whole 256-column blocks, weights below 4 GiB),
 * 256 where it runs a decode GEMV (quantized weights, whole 256-column
 * groups), 0 where it keeps f32 activations (float weights, other widths). */
size_t orc_i8_group(int dtype, size_t n_out, size_t n_in, size_t T) {
    int quant = dtype == ORC_Q8_0 || dtype == ORC_Q4_K || dtype == ORC_Q6_K;
    if (!quant)
        return 0;
    size_t bs = orc_block_size(dtype), ts = orc_type_size(dtype);
    size_t row = (n_in / bs * ts + 15) / 16 * 16; /* prepared row bytes */
    int gemm_w = dtype == ORC_Q8_0 ? n_in % 128 == 0 : n_in % 256 == 0;
    if (T >= ORC_GEMM_MIN_TOKENS && gemm_w && (unsigned long long)n_out * row < (1ull << 32))
        return 32;
    return n_in % 256 == 0 ? 256 : 0;
}

/* "Requantize, then CPU qmatmul" (src/backend/rocm/decode/tests.rs:68-77):
 * in the int8 mode every token row of x is quantized per group and the CPU
 * qmatmul runs on the dequantized values q*d. */
static int qm_kind(const orc_model *m, int kind, const orc_weight *w, const float *x, size_t T, float *y) {
    size_t row_bytes = orc_type_size(w->dtype) * (w->n_in / orc_block_size(w->dtype));
    size_t g = (m->act_i8 & kind) ? orc_i8_group(w->dtype, w->n_out, w->n_in, T) : 0;
    if (!g)
        return orc_qmatmul(w->dtype, w->data, row_bytes * w->n_out, w->n_out, w->n_in, x,
                           T * w->n_in, y, T * w->n_out, m->n_threads);
    size_t n = T * w->n_in;
    int8_t *q = (int8_t *)malloc(n);
    float *d = (float *)malloc(n / g * sizeof(float)), *xh = (float *)malloc(n * sizeof(float));
    orc_quantize_act(x, n, g, q, d, NULL);
    for (size_t i = 0; i < n; i++)
        xh[i] = (float)q[i] * d[i / g];
    int st = orc_qmatmul(w->dtype, w->data, row_bytes * w->n_out, w->n_out, w->n_in, xh, n, y,
                         T * w->n_out, m->n_threads);
    free(q);
    free(d);
    free(xh);
    return st;
}

static int qm(const orc_model *m, const orc_weight *w, const float *x, size_t T, float *y) {
    int kind = w == &m->output ? ORC_I8_HEAD : ORC_I8_QKV;
    for (size_t i = 0; i < m->n_layers; i++) {
        const orc_layer *L = &m->layers[i];
        if (w == &L->wo)
            kind = ORC_I8_O;
        else if (w == &L->w_gate || w == &L->w_up)
            kind = ORC_I8_GATE_UP;
        else if (w == &L->w_down)
            kind = ORC_I8_DOWN;
    }
    return qm_kind(m, kind, w, x, T, y);
}

static void swap(float **a, float **b) {
    float *t = *a;
    *a = *b;
    *b = t;
}

/* Llama::run (src/model/arch/llama.rs:136-155) + run_layers (:158-246),
 * with KvCache::rope_write (src/kv_cache.rs:212-244) and the default
 * Backend::rope_kv_write (src/backend.rs:452-467). Leaves the final-normed
 * rows in ws->normed. */
static int run(const orc_model *m, orc_ws *ws, float **kc, float **vc, const uint32_t *tokens,
               size_t T, uint32_t pos) {
    size_t E = m->n_embd, hd = m->head_dim, kvw = m->n_kv_heads * hd, qw = m->n_heads * hd;
    size_t row_bytes =
        orc_type_size(m->token_embd.dtype) * (E / orc_block_size(m->token_embd.dtype));
    if (orc_embed(m->token_embd.dtype, m->token_embd.data, row_bytes * m->vocab, m->vocab, E,
                  tokens, T, ws->x, T * E))
        return SHAPE;
    for (size_t i = 0; i < m->n_layers; i++) {
        const orc_layer *L = &m->layers[i];
        if (i == 0) {
            orc_rmsnorm(L->attn_norm, E, ws->x, T * E, ws->normed, T * E, m->rms_eps);
        } else {
            orc_add_rmsnorm(L->attn_norm, E, ws->x, ws->proj, T * E, ws->x_alt, ws->normed,
                            m->rms_eps);
            swap(&ws->x, &ws->x_alt);
        }
        if (qm(m, &L->wq, ws->normed, T, ws->q) || qm(m, &L->wk, ws->normed, T, ws->k) ||
            qm(m, &L->wv, ws->normed, T, ws->v))
            return SHAPE;
        orc_rope(ws->q, T * qw, ws->k, T * kvw, pos, T, hd, m->rope_theta);
        for (size_t e = 0; e < T * kvw; e++) {
            float kk = ws->k[e], vv = ws->v[e];
            if (m->kv_f16) {
                kk = orc_f16_to_f32(orc_f32_to_f16(kk));
                vv = orc_f16_to_f32(orc_f32_to_f16(vv));
            }
            kc[i][pos * kvw + e] = kk;
            vc[i][pos * kvw + e] = vv;
        }
        size_t len = pos + T;
        orc_attention(ws->q, T * qw, kc[i], vc[i], len * kvw, len, hd, m->n_heads, m->n_kv_heads,
                      ws->attn_out, T * qw);
        if (qm(m, &L->wo, ws->attn_out, T, ws->proj))
            return SHAPE;
        orc_add_rmsnorm(L->ffn_norm, E, ws->x, ws->proj, T * E, ws->x_alt, ws->normed, m->rms_eps);
        swap(&ws->x, &ws->x_alt);
        if (qm(m, &L->w_gate, ws->normed, T, ws->gate) || qm(m, &L->w_up, ws->normed, T, ws->up))
            return SHAPE;
        orc_silu_mul(ws->gate, ws->up, T * m->n_ff, ws->act);
        if (qm(m, &L->w_down, ws->act, T, ws->proj))
            return SHAPE;
    }
    orc_add_rmsnorm(m->output_norm, E, ws->x, ws->proj, T * E, ws->x_alt, ws->normed, m->rms_eps);
    swap(&ws->x, &ws->x_alt);
    return OK;
}

static int nonfinite(const float *v, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(v[i]))
            return 1;
    return 0;
}

/* Model::prefill (src/model.rs:398-468), then the greedy loop of
 * inference::sample (src/inference.rs:102-124) without EOS: n_gen tokens,
 * n_gen - 1 Model::forward calls (src/model.rs:326-387). With `forced`
 * non-null, step i + 1 is fed forced[i] instead of the greedy token of step
 * i (teacher forcing: every step's logits are then those of one fixed token
 * sequence); out_tokens still receives each step's greedy token.
 * step_logits (nullable) receives the logits of every step, [n_gen][vocab]. */
static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int orc_llama_run(const orc_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                  const uint32_t *forced, uint32_t *out_tokens, float *step_logits) {
    return orc_llama_run_timed(m, prompt, n_prompt, n_gen, forced, out_tokens, step_logits, NULL);
}

/* orc_llama_run that also records wall seconds per step (nullable): [0] the
 * prefill and its head, [i] decode step i (forward + head); the CPU
 * baseline's timing. */
int orc_llama_run_timed(const orc_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                        const uint32_t *forced, uint32_t *out_tokens, float *step_logits,
                        double *step_seconds) {
    if (!n_prompt || !n_gen || n_prompt + n_gen > m->n_ctx)
        return 1; /* ContextLimit */
    size_t E = m->n_embd, kvw = m->n_kv_heads * m->head_dim, qw = m->n_heads * m->head_dim;
    size_t T = n_prompt, F = m->n_ff;
    orc_ws ws;
    float **kc = (float **)calloc(m->n_layers, sizeof(float *));
    float **vc = (float **)calloc(m->n_layers, sizeof(float *));
    for (size_t i = 0; i < m->n_layers; i++) {
        kc[i] = (float *)calloc((n_prompt + n_gen) * kvw, sizeof(float));
        vc[i] = (float *)calloc((n_prompt + n_gen) * kvw, sizeof(float));
    }
    ws.x = (float *)calloc(T * E, 4);
    ws.x_alt = (float *)calloc(T * E, 4);
    ws.normed = (float *)calloc(T * E, 4);
    ws.q = (float *)calloc(T * qw, 4);
    ws.k = (float *)calloc(T * kvw, 4);
    ws.v = (float *)calloc(T * kvw, 4);
    ws.attn_out = (float *)calloc(T * qw, 4);
    ws.proj = (float *)calloc(T * E, 4);
    ws.gate = (float *)calloc(T * F, 4);
    ws.up = (float *)calloc(T * F, 4);
    ws.act = (float *)calloc(T * F, 4);
    float *logits = (float *)calloc(m->vocab, 4);
    double t0 = now_s();
    int st = run(m, &ws, kc, vc, prompt, T, 0);
    if (!st)
        st = qm(m, &m->output, ws.normed + (T - 1) * E, 1, logits);
    if (step_seconds)
        step_seconds[0] = now_s() - t0;
    for (size_t i = 0; !st && i < n_gen; i++) {
        if (nonfinite(logits, m->vocab)) {
            st = 10; /* Backend("empty or nonfinite logits") */
            break;
        }
        if (step_logits)
            memcpy(step_logits + i * m->vocab, logits, m->vocab * 4);
        uint32_t tok = orc_greedy(logits, m->vocab);
        out_tokens[i] = tok;
        if (i + 1 < n_gen) {
            uint32_t feed = forced ? forced[i] : tok;
            if (feed >= m->vocab) {
                st = 2;
                break;
            }
            t0 = now_s();
            st = run(m, &ws, kc, vc, &feed, 1, (uint32_t)(n_prompt + i));
            if (!st)
                st = qm(m, &m->output, ws.normed, 1, logits);
            if (step_seconds)
                step_seconds[i + 1] = now_s() - t0;
        }
    }
    for (size_t i = 0; i < m->n_layers; i++) {
        free(kc[i]);
        free(vc[i]);
    }
    free(kc);
    free(vc);
    free(ws.x);
    free(ws.x_alt);
    free(ws.normed);
    free(ws.q);
    free(ws.k);
    free(ws.v);
    free(ws.attn_out);
    free(ws.proj);
    free(ws.gate);
    free(ws.up);
    free(ws.act);
    free(logits);
    return st;
}

int orc_llama_generate(const orc_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                       uint32_t *out_tokens, float *last_logits) {
    float *all = last_logits ? (float *)malloc(n_gen * m->vocab * 4) : NULL;
    if (last_logits && !all)
        return 8;
    int st = orc_llama_run(m, prompt, n_prompt, n_gen, NULL, out_tokens, all);
    if (!st && last_logits)
        memcpy(last_logits, all + (n_gen - 1) * m->vocab, m->vocab * 4);
    free(all);
    return st;
}
