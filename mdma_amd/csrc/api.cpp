// C-ABI entry points of the gfx950 backend: the Backend trait contract
// (/root/reference/src/backend.rs:190-601) with the shared geometry rules of
// src/backend/shape.rs restated before any launch, so a malformed call is
// rejected on the host and never reaches a kernel.
#include <cmath>
#include <cstdarg>
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>

#include "internal.h"

using namespace mdma;

namespace {
thread_local std::string g_last_error;

template <class F>
int guarded(F &&f) {
  try {
    f();
    return MDMA_OK;
  } catch (const Error &e) {
    g_last_error = e.msg;
    return e.code;
  } catch (const std::bad_alloc &) {
    g_last_error = "host allocation failed";
    return MDMA_ERR_OUT_OF_MEMORY;
  } catch (...) {
    g_last_error = "unknown failure";
    return MDMA_ERR_BACKEND;
  }
}

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
  char b[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(b, sizeof b, f, ap);
  va_end(ap);
  return b;
}

void need(const void *p, const char *what) {
  if (!p) shape_fail(fmt("%s: null argument", what));
}

uint64_t f32_elems(const char *op, const mdma_buf *b) {
  need(b, op);
  if (b->len % 4) shape_fail(fmt("%s: %llu bytes is not whole f32s", op, (unsigned long long)b->len));
  return b->len / 4;
}

// shape::range (shape.rs:25-33).
void range(const char *op, uint64_t off, uint64_t len, uint64_t cap) {
  if (off + len < off || off + len > cap)
    shape_fail(fmt("%s: %llu bytes at offset %llu exceeds %llu byte buffer", op,
                   (unsigned long long)len, (unsigned long long)off, (unsigned long long)cap));
}

void same_ctx(mdma_ctx *ctx, const mdma_buf *b, const char *op) {
  if (b && b->ctx != ctx) shape_fail(fmt("%s: buffer belongs to another context", op));
}

// A weight's row bytes, with the dtype / K-quant alignment rules
// (shape.rs:76-84; dtype_code.rs:11-29, widened to Q8_0).
uint64_t weight_row_bytes(const mdma_qweight *w, const char *op) {
  need(w, op);
  need(w->buf, op);
  uint64_t bs = block_size(w->dtype);
  if (!bs) fail(MDMA_ERR_NOT_IMPLEMENTED, fmt("%s: weight dtype %d", op, w->dtype));
  if (!w->rows || !w->cols) shape_fail(fmt("%s: empty weight [%llu, %llu]", op,
                                           (unsigned long long)w->rows, (unsigned long long)w->cols));
  if (w->cols % bs)
    shape_fail(fmt("%s: width %llu is not a multiple of block size %llu", op,
                   (unsigned long long)w->cols, (unsigned long long)bs));
  const bool prepared = w->buf->layout == MDMA_LAYOUT_GFX950;
  if (prepared && !gfx950_layout_dtype(w->dtype))
    shape_fail(fmt("%s: buffer holds a prepared layout, weight dtype %d has none", op, w->dtype));
  uint64_t rb = prepared ? gfx950_row_bytes(w->dtype, w->cols) : w->cols / bs * type_size(w->dtype);
  if (w->buf->len < rb * w->rows)
    shape_fail(fmt("%s: weight buffer %llu bytes, needs %llu", op, (unsigned long long)w->buf->len,
                   (unsigned long long)(rb * w->rows)));
  return rb;
}

// shape::matmul (shape.rs:51-73): n_tokens from x, y only large enough.
uint64_t matmul_tokens(const mdma_qweight *w, const mdma_buf *x, const mdma_buf *y, const char *op) {
  weight_row_bytes(w, op);
  uint64_t xe = f32_elems(op, x), ye = f32_elems(op, y);
  if (!xe || xe % w->cols)
    shape_fail(fmt("%s: x has %llu elems, not whole rows of n_in %llu", op, (unsigned long long)xe,
                   (unsigned long long)w->cols));
  uint64_t T = xe / w->cols;
  if (ye < T * w->rows)
    shape_fail(fmt("%s: y has %llu elems, needs %llu", op, (unsigned long long)ye,
                   (unsigned long long)(T * w->rows)));
  // The kernels read x and the weight blocks with 16-byte vector loads;
  // buffers from alloc are 256-byte aligned, views must keep 16.
  if (reinterpret_cast<uintptr_t>(x->ptr) % 16 || reinterpret_cast<uintptr_t>(w->buf->ptr) % 16)
    shape_fail(fmt("%s: x and weight buffers must be 16-byte aligned", op));
  if (reinterpret_cast<uintptr_t>(y->ptr) % 4) shape_fail(fmt("%s: y must be 4-byte aligned", op));
  return T;
}

GemvJob job_of(const mdma_qweight *w, mdma_buf *y) {
  GemvJob j{w->dtype, reinterpret_cast<const uint8_t *>(w->buf->ptr), w->rows, w->cols,
            reinterpret_cast<float *>(y->ptr), w->buf->layout};
  j.src = const_cast<mdma_buf *>(w->buf);  // the weight itself is not written; its tile images may be made
  return j;
}

// Block-dot capture: the jobs' slots, one region after another.
void attach_dots(mdma_ctx *ctx, GemvJob *jobs, int n, uint64_t T) {
  if (!ctx->dots) return;
  uint64_t off = 0;
  for (int i = 0; i < n; i++) {
    const uint64_t need = T * jobs[i].n_out * dot_subs(jobs[i].dtype, jobs[i].n_in);
    if (off + need > ctx->dots_cap) shape_fail("block-dot capture: the call's dots exceed the capture buffer");
    jobs[i].dots = ctx->dots + off;
    off += need;
  }
}

void run_gemv(mdma_ctx *ctx, int mode, const GemvJob *jobs, int n, const float *x, uint64_t T) {
  if (mode == MDMA_ACT_I8)
    launch_gemv_i8(ctx, jobs, n, x, T);
  else if (mode == MDMA_ACT_F32_CPU)
    for (int i = 0; i < n; i++) launch_gemv_seq(ctx, jobs[i], x, T);
  else
    launch_gemv_f32(ctx, jobs, n, x, T);
}

int qmatmul_mode(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y, int mode) {
  return guarded([&] { qmatmul_run(ctx, w, x, y, mode); });
}

// rope angle table on the host with the CPU backend's formula (apply_rope,
// src/backend/cpu.rs:68-84): freq = theta^(-2i/hd) by powf, then sin/cos of
// pos*freq in f32 with the C library, so the device rotation uses the very
// angles the CPU uses.
void fill_rope(float *tab, uint64_t p0, uint64_t p1, uint64_t hd, float theta) {
  uint64_t half = hd / 2;
  std::vector<float> freq(half);
  for (uint64_t i = 0; i < half; i++)
    freq[i] = powf(theta, -2.0f * (float)i / (float)hd);
  for (uint64_t p = p0; p < p1; p++)
    for (uint64_t i = 0; i < half; i++) {
      volatile float a = (float)p * freq[i];
      tab[(p * half + i) * 2 + 0] = cosf(a);
      tab[(p * half + i) * 2 + 1] = sinf(a);
    }
}

// A setting that selects kernels: a graph captured under the old value
// would replay the old kernels, so a change bumps the buffer epoch and such
// graphs refuse to replay (a decoder then captures again).
template <class T>
void set_kernel_choice(mdma_ctx *ctx, T &field, T value) {
  if (field == value) return;
  field = value;
  ctx->buf_epoch++;
}

// The device position of a replayed decode step (params[1]), or null outside
// replay; a replayed step has one token.
const uint32_t *replay_pos(const mdma_ctx *ctx, uint64_t n_tokens, const char *op) {
  if (!ctx->replay) return nullptr;
  if (n_tokens != 1) shape_fail(fmt("%s: a replayed decode step has one token", op));
  return ctx->replay + 1;
}

void check_rope(const mdma_rope_spec *spec, uint64_t qe, uint64_t ke, uint64_t n_tokens,
                uint64_t *qh, uint64_t *kh) {
  need(spec, "rope");
  // shape::rope (shape.rs:146-168).
  if (!n_tokens || qe % n_tokens || ke % n_tokens)
    shape_fail(fmt("rope: q %llu k %llu elems are not whole tokens of n_tokens %llu",
                   (unsigned long long)qe, (unsigned long long)ke, (unsigned long long)n_tokens));
  uint64_t qs = qe / n_tokens, ks = ke / n_tokens, hd = spec->head_dim;
  if (!hd || hd % 2 || qs % hd || ks % hd)
    shape_fail(fmt("rope: token strides %llu/%llu are not whole even heads of %llu",
                   (unsigned long long)qs, (unsigned long long)ks, (unsigned long long)hd));
  if (!std::isfinite(spec->theta) || spec->theta <= 0.f) shape_fail("rope: theta must be positive");
  *qh = qs / hd;
  *kh = ks / hd;
}

}  // namespace

namespace mdma {

void qmatmul_run(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y, int mode) {
  need(ctx, "qmatmul");
  std::lock_guard<std::recursive_mutex> g(ctx->lock);
  prepare_weight(ctx, w);
  uint64_t T = matmul_tokens(w, x, y, "qmatmul");
  same_ctx(ctx, w->buf, "qmatmul");
  same_ctx(ctx, x, "qmatmul");
  same_ctx(ctx, y, "qmatmul");
  GemvJob j = job_of(w, y);
  attach_dots(ctx, &j, 1, T);
  run_gemv(ctx, mode < 0 ? ctx->act_mode : mode, &j, 1, reinterpret_cast<const float *>(x->ptr), T);
  q8_invalidate_range(ctx, y->ptr, y->len);
}

void prepare_weight(mdma_ctx *ctx, const mdma_qweight *w) {
  if (!w || !w->buf || !w->buf->repack_pending) return;
  mdma_buf *b = const_cast<mdma_buf *>(w->buf);  // the representation changes, not the weight
  if (!b->owner || b->ctx != ctx || !gfx950_layout_dtype(w->dtype)) return;
  const uint64_t bs = block_size(w->dtype);
  if (!w->rows || !w->cols || w->cols % bs || b->len != w->rows * (w->cols / bs) * type_size(w->dtype))
    return;  // not this weight's raw bytes: the shape rules report it
  if (ctx->capturing || ctx->fixed_scratch) return;  // no allocation now: the raw kernels read it
  const uint64_t n = w->rows * gfx950_row_bytes(w->dtype, w->cols);
  mdma_buf *p = nullptr;
  if (mdma_gfx950_alloc(ctx, n, MDMA_POOL_WEIGHTS, &p)) return;  // no room in the budget or on the device: stays raw
  try {
    launch_repack(ctx, w->dtype, w->rows, w->cols, reinterpret_cast<const uint8_t *>(b->ptr),
                  reinterpret_cast<uint8_t *>(p->ptr));
  } catch (...) {
    mdma_gfx950_free(p);
    throw;
  }
  // The prepared copy takes the raw buffer's place (free drains the stream
  // first, so the repack has finished reading the raw bytes). A graph
  // captured while the weight was raw holds the freed address: the epoch
  // makes it refuse to replay.
  ctx->buf_epoch++;
  std::swap(b->ptr, p->ptr);
  std::swap(b->len, p->len);
  std::swap(b->charged, p->charged);
  b->layout = MDMA_LAYOUT_GFX950;
  b->repack_pending = false;
  p->repack_pending = false;
  int st = mdma_gfx950_free(p);
  if (st) fail(st, g_last_error);
}

const uint8_t *batch_tile(mdma_ctx *ctx, const GemvJob &j) {
  mdma_buf *b = j.src;
  if (!b || !b->owner || b->ctx != ctx || b->ptr != reinterpret_cast<const char *>(j.w) ||
      j.layout != MDMA_LAYOUT_GFX950)
    return nullptr;
  if (b->tile && b->tile_stale && !ctx->capturing && !ctx->fixed_scratch) free_tile(ctx, b);
  if (b->tile) return b->tile_stale ? nullptr : reinterpret_cast<const uint8_t *>(b->tile);
  // Made outside capture and outside allocation-free calls only; without
  // room in the budget or on the device the row planes serve.
  if (!ctx->batch_layout || ctx->capturing || ctx->fixed_scratch) return nullptr;
  const uint64_t n = batch_tile_bytes(j.dtype, j.n_out, j.n_in);
  if (!n || b->len < j.n_out * gfx950_row_bytes(j.dtype, j.n_in)) return nullptr;
  Ledger &l = ctx->budget[MDMA_DOMAIN_DEVICE];
  if (l.used + n < l.used || l.used + n > l.limit) return nullptr;
  void *d = nullptr;
  if (hipMalloc(&d, n) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  l.used += n;
  try {
    launch_tile_repack(ctx, j.dtype, j.n_out, j.n_in, j.w, static_cast<uint8_t *>(d));
  } catch (...) {
    (void)hipFree(d);
    l.used -= n;
    throw;
  }
  b->tile = static_cast<char *>(d);
  b->tile_charged = n;
  ctx->tiled.push_back(b);
  return reinterpret_cast<const uint8_t *>(b->tile);
}

// Throws nothing (it runs where outputs are retired): a failed free keeps
// the charge, as a failed buffer free does.
void free_tile(mdma_ctx *ctx, mdma_buf *b) {
  if (!b->tile) return;
  (void)hipStreamSynchronize(ctx->stream);
  if (hipFree(b->tile) == hipSuccess) budget_refund(ctx, MDMA_DOMAIN_DEVICE, b->tile_charged);
  else (void)hipGetLastError();
  b->tile = nullptr;
  b->tile_charged = 0;
  b->tile_stale = false;
  auto &v = ctx->tiled;
  v.erase(std::remove(v.begin(), v.end(), b), v.end());
  ctx->buf_epoch++;  // a captured graph may read the images
}

void drop_tiles(mdma_ctx *ctx, const void *p, uint64_t bytes) {
  const char *a = static_cast<const char *>(p);
  for (size_t i = ctx->tiled.size(); i-- > 0;) {
    mdma_buf *b = ctx->tiled[i];
    if (!(a < b->ptr + b->len && b->ptr < a + bytes)) continue;
    // Under capture (or in an allocation-free call) nothing is freed: the
    // images are set aside and freed by the next call that may.
    if (ctx->capturing || ctx->fixed_scratch) b->tile_stale = true;
    else free_tile(ctx, b);
  }
}

void fail(int code, const std::string &msg) { throw Error{code, msg}; }

void set_last_error(const std::string &msg) { g_last_error = msg; }

void hip_check(hipError_t e, const char *what) {
  if (e == hipSuccess) return;
  int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? MDMA_ERR_OUT_OF_MEMORY
                                                                          : MDMA_ERR_BACKEND;
  fail(code, std::string(what) + ": " + hipGetErrorString(e));
}

void no_capture(mdma_ctx *ctx, const char *what) {
  if (ctx->capturing) fail(MDMA_ERR_BACKEND, std::string(what) + " synchronizes and cannot run under graph capture");
  if (ctx->fixed_scratch) fail(MDMA_ERR_BACKEND, std::string(what) + " would allocate inside an allocation-free call");
}

void budget_charge(mdma_ctx *ctx, int domain, uint64_t bytes, const char *what) {
  Ledger &l = ctx->budget[domain];
  if (l.used + bytes < l.used || l.used + bytes > l.limit)
    fail(MDMA_ERR_BUFFER_BUDGET,
         fmt("%s: %s buffer budget exhausted: requested %llu bytes, used %llu, limit %llu", what,
             domain == MDMA_DOMAIN_DEVICE ? "device" : "host", (unsigned long long)bytes,
             (unsigned long long)l.used, (unsigned long long)l.limit));
  l.used += bytes;
}

void budget_refund(mdma_ctx *ctx, int domain, uint64_t bytes) { ctx->budget[domain].used -= bytes; }

// Replace a context-owned device buffer (buf, cap units of `unit` bytes)
// by one of new_cap units: charged to the device budget first
// (BufferBudget::allocate; a refusal leaves the old buffer as it was), the
// stream drained so no queued kernel still reads the old memory, the old
// buffer freed (its charge refunded only when the free succeeds), and the
// context's buffer epoch bumped (graphs captured before refuse to replay).
template <class T>
static T *regrow(mdma_ctx *ctx, T *&buf, uint64_t &cap, uint64_t new_cap, uint64_t unit, const char *what) {
  no_capture(ctx, what);
  const uint64_t new_bytes = new_cap * unit;
  budget_charge(ctx, MDMA_DOMAIN_DEVICE, new_bytes, what);
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    budget_refund(ctx, MDMA_DOMAIN_DEVICE, new_bytes);
    hip_check(e, what);
  }
  if (buf) {
    ctx->buf_epoch++;
    e = hipFree(buf);
    if (e == hipSuccess) budget_refund(ctx, MDMA_DOMAIN_DEVICE, cap * unit);  // else: the charge stays
    buf = nullptr;
    cap = 0;
    if (e != hipSuccess) {
      budget_refund(ctx, MDMA_DOMAIN_DEVICE, new_bytes);
      hip_check(e, what);
    }
  }
  void *p = nullptr;
  e = hipMalloc(&p, new_bytes);
  if (e != hipSuccess) {
    budget_refund(ctx, MDMA_DOMAIN_DEVICE, new_bytes);
    hip_check(e, what);
  }
  buf = static_cast<T *>(p);
  cap = new_cap;
  return buf;
}

char *scratch(mdma_ctx *ctx, uint64_t bytes) {
  if (bytes <= ctx->scratch_cap) return ctx->scratch;
  const uint64_t cap = bytes < (1u << 20) ? (1u << 20) : bytes + bytes / 4;
  return regrow(ctx, ctx->scratch, ctx->scratch_cap, cap, 1, "scratch growth");
}

char *q8_buffer(mdma_ctx *ctx, uint64_t bytes) {
  if (bytes <= ctx->q8_cap) return ctx->q8;
  const uint64_t cap = bytes < (1u << 20) ? (1u << 20) : bytes + bytes / 4;
  ctx->q8_valid = false;
  return regrow(ctx, ctx->q8, ctx->q8_cap, cap, 1, "int8 activation buffer growth");
}

char *argmax_parts(mdma_ctx *ctx, uint64_t chunks) {
  if (chunks <= ctx->argmax_part_cap) return ctx->argmax_part;
  const uint64_t cap = chunks < 4096 ? 4096 : chunks + chunks / 4;
  return regrow(ctx, ctx->argmax_part, ctx->argmax_part_cap, cap, 12, "argmax buffer growth");
}

double *ssq_parts(mdma_ctx *ctx, uint64_t n) {
  if (n <= ctx->ssq_cap) return ctx->ssq;
  const uint64_t cap = n < 4096 ? 4096 : n + n / 4;
  return regrow(ctx, ctx->ssq, ctx->ssq_cap, cap, 8, "norm partials growth");
}

// A zeroed uint32 buffer of at least n entries (grown outside capture only).
static uint32_t *zeroed_counters(mdma_ctx *ctx, uint32_t *&buf, uint64_t &cap_, uint64_t n, const char *what) {
  if (n <= cap_) return buf;
  const uint64_t cap = n < 4096 ? 4096 : n + n / 4;
  regrow(ctx, buf, cap_, cap, 4, what);
  // On the context's stream (non-blocking: it does not wait for work on the
  // null stream), so the launches that use the counters follow the clear.
  hip_check(hipMemsetAsync(buf, 0, cap * 4, ctx->stream), "counter clear");
  return buf;
}

uint32_t *attn_counters(mdma_ctx *ctx, uint64_t n) {
  return zeroed_counters(ctx, ctx->attn_cnt, ctx->attn_cnt_cap, n * CNT_STRIDE, "attention counter growth");
}

uint32_t *gemm_counters(mdma_ctx *ctx, uint64_t n) {
  if (ctx->capturing && n * CNT_STRIDE > ctx->gemm_cnt_cap) return nullptr;
  return zeroed_counters(ctx, ctx->gemm_cnt, ctx->gemm_cnt_cap, n * CNT_STRIDE, "GEMM counter growth");
}

void q8_invalidate_range(mdma_ctx *ctx, const void *p, uint64_t bytes) {
  if (!ctx->tiled.empty()) drop_tiles(ctx, p, bytes);  // an op output over a weight's bytes
  const char *a = static_cast<const char *>(p);
  auto over = [&](const void *q, uint64_t n) {
    const char *b = static_cast<const char *>(q);
    return a < b + n && b < a + bytes;
  };
  if (ctx->q8_valid && over(ctx->q8_x, ctx->q8_n * 4)) ctx->q8_valid = false;
  if (ctx->a16_valid && (over(ctx->a16_x, ctx->a16_n * 4) ||
                         over(ctx->a16_buf, gemm_f16_input_bytes(ctx->a16_n / ctx->a16_n_in, ctx->a16_n_in))))
    ctx->a16_valid = false;
}

const float *rope_table(mdma_ctx *ctx, uint64_t max_pos, uint64_t hd, float theta) {
  uint64_t need_pos = max_pos + 1;
  if (ctx->rope_tab && ctx->rope_hd == hd && ctx->rope_theta == theta && need_pos <= ctx->rope_positions)
    return ctx->rope_tab;
  no_capture(ctx, "RoPE table growth");
  uint64_t positions = need_pos < 4096 ? 4096 : need_pos + need_pos / 2;
  std::vector<float> host(positions * hd);
  fill_rope(host.data(), 0, positions, hd, theta);
  ctx->rope_positions = 0;
  regrow(ctx, ctx->rope_tab, ctx->rope_bytes, host.size() * 4, 1, "RoPE table growth");
  void *p = ctx->rope_tab;
  hip_check(hipMemcpy(p, host.data(), host.size() * 4, hipMemcpyHostToDevice), "rope table upload");
  ctx->rope_positions = positions;
  ctx->rope_hd = hd;
  ctx->rope_theta = theta;
  return ctx->rope_tab;
}

}  // namespace mdma

extern "C" {

const char *mdma_gfx950_last_error(void) { return g_last_error.c_str(); }

int mdma_gfx950_create(int device, mdma_ctx **out) {
  return guarded([&] {
    need(out, "create");
    *out = nullptr;
    int n = 0;
    hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (device < 0 || device >= n) fail(MDMA_ERR_BACKEND, fmt("no HIP device %d (%d present)", device, n));
    hip_check(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      fail(MDMA_ERR_BACKEND, fmt("device %d is %s; this library is built for gfx950 only", device,
                                 prop.gcnArchName));
    auto *c = new mdma_ctx();
    c->device = device;
    c->label = std::string(prop.name[0] ? prop.name : "AMD Instinct (gfx950)") + " [" + prop.gcnArchName + ", " +
               std::to_string(prop.multiProcessorCount) + " CUs]";
    c->total_bytes = prop.totalGlobalMem;
    c->cu_count = prop.multiProcessorCount;
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete c;
      hip_check(e, "hipStreamCreate");
    }
    void *h = nullptr;
    e = hipHostMalloc(&h, 4096 * sizeof(uint32_t), hipHostMallocDefault);
    if (e != hipSuccess) {
      (void)hipStreamDestroy(c->stream);
      delete c;
      hip_check(e, "hipHostMalloc");
    }
    c->host_ids = static_cast<uint32_t *>(h);
    c->host_ids_cap = 4096;
    try {
      noalloc_setup(c);
    } catch (...) {
      (void)hipHostFree(c->host_ids);
      (void)hipStreamDestroy(c->stream);
      delete c;
      throw;
    }
    *out = c;
  });
}

void mdma_gfx950_destroy(mdma_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  for (mdma_buf *b : ctx->tiled) {  // buffers the caller did not free
    (void)hipFree(b->tile);
    b->tile = nullptr;
  }
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->q8) (void)hipFree(ctx->q8);
  if (ctx->argmax_part) (void)hipFree(ctx->argmax_part);
  if (ctx->attn_cnt) (void)hipFree(ctx->attn_cnt);
  if (ctx->gemm_cnt) (void)hipFree(ctx->gemm_cnt);
  if (ctx->ssq) (void)hipFree(ctx->ssq);
  if (ctx->rope_tab) (void)hipFree(ctx->rope_tab);
  if (ctx->host_ids) (void)hipHostFree(ctx->host_ids);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

int mdma_gfx950_device_label(mdma_ctx *ctx, char *out, size_t cap) {
  return guarded([&] {
    need(ctx, "device_label");
    need(out, "device_label");
    if (!cap) shape_fail("device_label: zero capacity");
    std::snprintf(out, cap, "%s", ctx->label.c_str());
  });
}

uint64_t mdma_gfx950_total_device_bytes(mdma_ctx *ctx) { return ctx ? ctx->total_bytes : 0; }

int mdma_gfx950_available_device_bytes(mdma_ctx *ctx, uint64_t *out) {
  return guarded([&] {
    need(ctx, "available_device_bytes");
    need(out, "available_device_bytes");
    size_t fr = 0, tot = 0;
    hip_check(hipSetDevice(ctx->device), "hipSetDevice");
    hip_check(hipMemGetInfo(&fr, &tot), "hipMemGetInfo");
    *out = fr;
  });
}

int mdma_gfx950_supports_weight_dtype(mdma_ctx *, int32_t dtype) { return block_size(dtype) != 0; }

uint64_t mdma_gfx950_max_head_dim(mdma_ctx *) { return 256; }

uint64_t mdma_gfx950_kv_elem_bytes(mdma_ctx *) { return 2; }

int mdma_gfx950_join_execution(mdma_ctx *ctx) {
  return guarded([&] {
    need(ctx, "join_execution");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    no_capture(ctx, "join_execution");
    hip_check(hipStreamSynchronize(ctx->stream), "join_execution");
  });
}

int mdma_gfx950_set_buffer_budget(mdma_ctx *ctx, uint64_t device_bytes, uint64_t host_bytes) {
  return guarded([&] {
    need(ctx, "set_buffer_budget");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    // BufferBudget::replace (src/memory/buffers.rs:61-70): only an unused ledger.
    if (ctx->budget[MDMA_DOMAIN_DEVICE].used || ctx->budget[MDMA_DOMAIN_HOST].used)
      fail(MDMA_ERR_BACKEND, "buffer budget must be installed before allocations or sharing");
    ctx->budget[MDMA_DOMAIN_DEVICE].limit = device_bytes;
    ctx->budget[MDMA_DOMAIN_HOST].limit = host_bytes;
  });
}

int mdma_gfx950_buffer_usage(mdma_ctx *ctx, int domain, uint64_t *used, uint64_t *limit) {
  return guarded([&] {
    need(ctx, "buffer_usage");
    if (domain != MDMA_DOMAIN_DEVICE && domain != MDMA_DOMAIN_HOST) shape_fail("buffer_usage: unknown domain");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    if (used) *used = ctx->budget[domain].used;
    if (limit) *limit = ctx->budget[domain].limit;
  });
}

int mdma_gfx950_set_act_mode(mdma_ctx *ctx, int mode) {
  return guarded([&] {
    need(ctx, "set_act_mode");
    if (mode != MDMA_ACT_F32 && mode != MDMA_ACT_I8 && mode != MDMA_ACT_F32_CPU)
      shape_fail("set_act_mode: unknown mode");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    set_kernel_choice(ctx, ctx->act_mode, mode);
  });
}

int mdma_gfx950_capture_block_dots(mdma_ctx *ctx, mdma_buf *out) {
  return guarded([&] {
    need(ctx, "capture_block_dots");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    if (out) {
      same_ctx(ctx, out, "capture_block_dots");
      if (reinterpret_cast<uintptr_t>(out->ptr) % 4) shape_fail("capture_block_dots: buffer must be 4-byte aligned");
    }
    ctx->dots = out ? reinterpret_cast<int32_t *>(out->ptr) : nullptr;
    ctx->dots_cap = out ? out->len / 4 : 0;
  });
}

int mdma_gfx950_set_graph_decode(mdma_ctx *ctx, int on) {
  return guarded([&] {
    need(ctx, "set_graph_decode");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    ctx->graph_decode = on != 0;
  });
}

int mdma_gfx950_set_prefill_kernel(mdma_ctx *ctx, int kind) {
  return guarded([&] {
    need(ctx, "set_prefill_kernel");
    if (kind != MDMA_PREFILL_AUTO && kind != MDMA_PREFILL_I8) shape_fail("set_prefill_kernel: unknown kind");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    set_kernel_choice(ctx, ctx->prefill_kernel, kind);
  });
}

int mdma_gfx950_set_batch_kernel(mdma_ctx *ctx, int kind) {
  return guarded([&] {
    need(ctx, "set_batch_kernel");
    if (kind != MDMA_BATCH_AUTO && kind != MDMA_BATCH_STAGED) shape_fail("set_batch_kernel: unknown kind");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    set_kernel_choice(ctx, ctx->batch_kernel, kind);
  });
}

int mdma_gfx950_set_batch_layout(mdma_ctx *ctx, int on) {
  return guarded([&] {
    need(ctx, "set_batch_layout");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    set_kernel_choice(ctx, ctx->batch_layout, on != 0);
  });
}

int mdma_gfx950_set_norm_fusion(mdma_ctx *ctx, int on) {
  return guarded([&] {
    need(ctx, "set_norm_fusion");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    set_kernel_choice(ctx, ctx->norm_fusion, on != 0);
  });
}

void *mdma_gfx950_stream(mdma_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int mdma_gfx950_alloc(mdma_ctx *ctx, uint64_t bytes, int pool, mdma_buf **out) {
  return guarded([&] {
    need(ctx, "alloc");
    need(out, "alloc");
    *out = nullptr;
    if (pool < 0 || pool > 2) shape_fail("alloc: pool out of range");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    // Allocations are rounded to 256 bytes so 16-byte vector loads of a
    // buffer's last element never cross the allocation's end; the budget is
    // charged the requested bytes (at least one), as the reference's HIP
    // buffers are (src/backend/rocm.rs:534-541, src/memory/buffers.rs:52-53).
    const uint64_t charged = bytes ? bytes : 1;
    const uint64_t rounded = (charged + 255) / 256 * 256;
    if (rounded < charged) fail(MDMA_ERR_SIZE_OVERFLOW, "alloc: size overflows");
    budget_charge(ctx, MDMA_DOMAIN_DEVICE, charged, "alloc");
    void *d = nullptr;
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc(&d, rounded);
    if (e != hipSuccess) {
      budget_refund(ctx, MDMA_DOMAIN_DEVICE, charged);
      hip_check(e, "hipMalloc");
    }
    auto *b = new mdma_buf();
    b->ctx = ctx;
    b->ptr = static_cast<char *>(d);
    b->len = bytes;
    b->charged = charged;
    b->pool = pool;
    *out = b;
  });
}

int mdma_gfx950_free(mdma_buf *buf) {
  return guarded([&] {
    if (!buf) return;
    if (!buf->owner) {
      delete buf;
      return;
    }
    mdma_ctx *ctx = buf->ctx;
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    no_capture(ctx, "free");
    // Kernels queued on the stream may still read the buffer.
    hip_check(hipStreamSynchronize(ctx->stream), "free: stream sync");
    free_tile(ctx, buf);
    if (buf->ptr) {
      hipError_t e = hipFree(buf->ptr);
      if (e != hipSuccess) {
        // Keep the charge: the memory may still be allocated
        // (src/backend/rocm/memory.rs:36-55).
        delete buf;
        hip_check(e, "hipFree");
      }
    }
    budget_refund(ctx, MDMA_DOMAIN_DEVICE, buf->charged);
    delete buf;
  });
}

uint64_t mdma_gfx950_buf_len(const mdma_buf *buf) { return buf ? buf->len : 0; }

int mdma_gfx950_buf_view(mdma_buf *parent, uint64_t offset, uint64_t len, mdma_buf **out) {
  return guarded([&] {
    need(parent, "buf_view");
    need(out, "buf_view");
    range("buf_view", offset, len, parent->len);
    auto *b = new mdma_buf();
    b->ctx = parent->ctx;
    b->ptr = parent->ptr + offset;
    b->len = len;
    b->charged = 0;
    b->pool = parent->pool;
    b->layout = parent->layout;
    b->owner = false;
    b->repack_pending = false;  // a window of raw bytes is read by the raw kernels
    // The view points into the parent's raw bytes: the parent stays raw (its
    // repack would free them under the view) and the raw kernels read it.
    parent->repack_pending = false;
    *out = b;
  });
}

int mdma_gfx950_upload(mdma_ctx *ctx, mdma_buf *dst, uint64_t offset, const void *src, uint64_t len) {
  return guarded([&] {
    need(ctx, "upload");
    need(dst, "upload");
    same_ctx(ctx, dst, "upload");
    range("upload", offset, len, dst->len);
    if (!len) return;
    need(src, "upload");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    no_capture(ctx, "upload");
    drop_tiles(ctx, dst->ptr + offset, len);
    hip_check(hipMemcpyAsync(dst->ptr + offset, src, len, hipMemcpyHostToDevice, ctx->stream), "upload");
    hip_check(hipStreamSynchronize(ctx->stream), "upload sync");
  });
}

int mdma_gfx950_download(mdma_ctx *ctx, const mdma_buf *src, uint64_t offset, void *dst, uint64_t len) {
  return guarded([&] {
    need(ctx, "download");
    need(src, "download");
    same_ctx(ctx, src, "download");
    range("download", offset, len, src->len);
    if (!len) return;
    need(dst, "download");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    no_capture(ctx, "download");
    hip_check(hipMemcpyAsync(dst, src->ptr + offset, len, hipMemcpyDeviceToHost, ctx->stream), "download");
    hip_check(hipStreamSynchronize(ctx->stream), "download sync");
  });
}

int mdma_gfx950_copy(mdma_ctx *ctx, const mdma_buf *src, uint64_t src_off, mdma_buf *dst,
                     uint64_t dst_off, uint64_t len) {
  return guarded([&] {
    need(ctx, "copy");
    need(src, "copy");
    need(dst, "copy");
    same_ctx(ctx, src, "copy");
    same_ctx(ctx, dst, "copy");
    range("copy", src_off, len, src->len);
    range("copy", dst_off, len, dst->len);
    if (!len) return;
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    hip_check(hipMemcpyAsync(dst->ptr + dst_off, src->ptr + src_off, len, hipMemcpyDeviceToDevice,
                             ctx->stream), "copy");
  });
}

int mdma_gfx950_upload_weight(mdma_ctx *ctx, const void *bytes, uint64_t len, int layout, mdma_buf **out) {
  return guarded([&] {
    need(ctx, "upload_weight");
    need(out, "upload_weight");
    *out = nullptr;
    // The trait's default stores GGUF bytes and refuses other layouts
    // (src/backend.rs:228-237); this backend also takes its own prepared
    // layout as it is. The reference ROCm backend's packed Q4_K is not read.
    if (layout == MDMA_LAYOUT_ROCM_Q4K_V3)
      fail(MDMA_ERR_NOT_IMPLEMENTED, "prepared weight layout for this backend");
    if (layout != MDMA_LAYOUT_GGUF && layout != MDMA_LAYOUT_GFX950)
      fail(MDMA_ERR_NOT_IMPLEMENTED, "upload_weight: unknown weight layout");
    if (len) need(bytes, "upload_weight");
    mdma_buf *b = nullptr;
    int st = mdma_gfx950_alloc(ctx, len, MDMA_POOL_WEIGHTS, &b);
    if (st) fail(st, g_last_error);
    st = mdma_gfx950_upload(ctx, b, 0, bytes, len);
    if (st) {
      std::string m = g_last_error;
      mdma_gfx950_free(b);
      fail(st, m);
    }
    b->layout = layout;
    b->repack_pending = layout == MDMA_LAYOUT_GGUF;
    *out = b;
  });
}

int mdma_gfx950_upload_weight_typed(mdma_ctx *ctx, const void *bytes, uint64_t len, int layout, int32_t dtype,
                                    uint64_t rows, uint64_t cols, mdma_buf **out) {
  return guarded([&] {
    need(ctx, "upload_weight_typed");
    need(out, "upload_weight_typed");
    *out = nullptr;
    if (layout != MDMA_LAYOUT_GGUF && layout != MDMA_LAYOUT_GFX950)
      fail(MDMA_ERR_NOT_IMPLEMENTED, "upload_weight_typed: unknown weight layout");
    uint64_t bs = block_size(dtype);
    if (!bs) fail(MDMA_ERR_NOT_IMPLEMENTED, fmt("upload_weight_typed: dtype %d", dtype));
    if (layout == MDMA_LAYOUT_GFX950 && !gfx950_layout_dtype(dtype))
      fail(MDMA_ERR_NOT_IMPLEMENTED, fmt("upload_weight_typed: dtype %d has no prepared layout", dtype));
    const uint64_t raw = cols % bs ? 0 : rows * (cols / bs) * type_size(dtype);
    const uint64_t want = layout == MDMA_LAYOUT_GFX950 ? rows * gfx950_row_bytes(dtype, cols) : raw;
    if (cols % bs || len != want)
      shape_fail(fmt("upload_weight_typed: %llu bytes do not hold a [%llu, %llu] weight", (unsigned long long)len,
                     (unsigned long long)rows, (unsigned long long)cols));
    if (len) need(bytes, "upload_weight_typed");
    // GGUF Q4_K / Q6_K / Q8_0 rows are stored in the prepared layout, which
    // every op on this backend reads; other dtypes keep their bytes.
    const bool pack = layout == MDMA_LAYOUT_GGUF && gfx950_layout_dtype(dtype);
    std::vector<uint8_t> packed;
    const void *src = bytes;
    uint64_t n = len;
    if (pack) {
      n = rows * gfx950_row_bytes(dtype, cols);
      packed.resize(n);
      pack_gfx950(dtype, rows, cols, static_cast<const uint8_t *>(bytes), packed.data());
      src = packed.data();
    }
    mdma_buf *b = nullptr;
    int st = mdma_gfx950_alloc(ctx, n, MDMA_POOL_WEIGHTS, &b);
    if (st) fail(st, g_last_error);
    st = mdma_gfx950_upload(ctx, b, 0, src, n);
    if (st) {
      std::string m = g_last_error;
      mdma_gfx950_free(b);
      fail(st, m);
    }
    b->layout = (pack || layout == MDMA_LAYOUT_GFX950) ? MDMA_LAYOUT_GFX950 : MDMA_LAYOUT_GGUF;
    *out = b;
  });
}

int mdma_gfx950_buf_layout(const mdma_buf *buf) { return buf ? buf->layout : -1; }

int mdma_gfx950_qmatmul(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y) {
  return qmatmul_mode(ctx, w, x, y, -1);
}

int mdma_gfx950_qmatmul_f32(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y) {
  return qmatmul_mode(ctx, w, x, y, MDMA_ACT_F32);
}

int mdma_gfx950_qmatmul_i8(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y) {
  return qmatmul_mode(ctx, w, x, y, MDMA_ACT_I8);
}

int mdma_gfx950_qmatmul_qkv(mdma_ctx *ctx, const mdma_qweight *wq, const mdma_qweight *wk,
                            const mdma_qweight *wv, const mdma_buf *x, mdma_buf *q, mdma_buf *k,
                            mdma_buf *v) {
  return guarded([&] {
    need(ctx, "qmatmul_qkv");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    for (const mdma_qweight *w : {wq, wk, wv}) prepare_weight(ctx, w);
    uint64_t T = matmul_tokens(wq, x, q, "qmatmul_qkv");
    if (matmul_tokens(wk, x, k, "qmatmul_qkv") != T || matmul_tokens(wv, x, v, "qmatmul_qkv") != T)
      shape_fail("qmatmul_qkv: projections disagree on n_tokens");
    for (const mdma_buf *b : {wq->buf, wk->buf, wv->buf, x, (const mdma_buf *)q, (const mdma_buf *)k,
                              (const mdma_buf *)v})
      same_ctx(ctx, b, "qmatmul_qkv");
    GemvJob jobs[3] = {job_of(wq, q), job_of(wk, k), job_of(wv, v)};
    attach_dots(ctx, jobs, 3, T);
    run_gemv(ctx, ctx->act_mode, jobs, 3, reinterpret_cast<const float *>(x->ptr), T);
    for (const mdma_buf *o : {(const mdma_buf *)q, (const mdma_buf *)k, (const mdma_buf *)v})
      q8_invalidate_range(ctx, o->ptr, o->len);
  });
}

int mdma_gfx950_ffn_gate_up(mdma_ctx *ctx, const mdma_qweight *gate, const mdma_qweight *up,
                            const mdma_buf *x, mdma_buf *gate_scratch, mdma_buf *up_scratch,
                            mdma_buf *y) {
  return guarded([&] {
    need(ctx, "ffn_gate_up");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    prepare_weight(ctx, gate);
    prepare_weight(ctx, up);
    need(gate, "ffn_gate_up");
    need(up, "ffn_gate_up");
    if (gate->rows != up->rows || gate->cols != up->cols)
      shape_fail("ffn gate/up weight shapes must match");
    uint64_t T = matmul_tokens(gate, x, gate_scratch, "ffn_gate_up");
    matmul_tokens(up, x, up_scratch, "ffn_gate_up");
    uint64_t ye = f32_elems("ffn_gate_up", y);
    // silu_mul's shape::elementwise: y must hold the gate output's elements.
    if (ye < f32_elems("ffn_gate_up", gate_scratch))
      shape_fail("ffn_gate_up: y cannot hold the gate/up output");
    for (const mdma_buf *b : {gate->buf, up->buf, x, (const mdma_buf *)gate_scratch,
                              (const mdma_buf *)up_scratch, (const mdma_buf *)y})
      same_ctx(ctx, b, "ffn_gate_up");
    GemvJob gu_jobs[2] = {job_of(gate, gate_scratch), job_of(up, up_scratch)};
    attach_dots(ctx, gu_jobs, 2, T);
    GemvJob gj = gu_jobs[0], uj = gu_jobs[1];
    const float *xp = reinterpret_cast<const float *>(x->ptr);
    float *yp = reinterpret_cast<float *>(y->ptr);
    struct Inval {  // runs when the call returns, after the launches below
      mdma_ctx *c;
      const mdma_buf *bs[3];
      ~Inval() {
        for (const mdma_buf *b : bs) q8_invalidate_range(c, b->ptr, b->len);
      }
    } inval{ctx, {gate_scratch, up_scratch, y}};
    // The fused kernel writes only y; the scratch buffers stay unspecified,
    // as the trait allows. When the scratch is larger than T*n_out (the
    // default impl would then run silu_mul over the whole scratch length),
    // fall back to that exact sequence so the contract holds bit for bit.
    // The CPU-order mode runs that sequence too (its SiLU is the CPU's).
    uint64_t gse = f32_elems("ffn_gate_up", gate_scratch), use = f32_elems("ffn_gate_up", up_scratch);
    if (gse != T * gate->rows || use != gse || ctx->act_mode == MDMA_ACT_F32_CPU) {
      if (use != gse) shape_fail("silu_mul: input lengths differ");
      run_gemv(ctx, ctx->act_mode, &gj, 1, xp, T);
      run_gemv(ctx, ctx->act_mode, &uj, 1, xp, T);
      const float *gp = reinterpret_cast<const float *>(gate_scratch->ptr),
                  *up_p = reinterpret_cast<const float *>(up_scratch->ptr);
      if (ctx->act_mode == MDMA_ACT_F32_CPU)
        launch_silu_mul_seq(ctx, gp, up_p, yp, gse);
      else
        launch_silu_mul(ctx, gp, up_p, yp, gse);
      return;
    }
    if (ctx->act_mode == MDMA_ACT_I8)
      launch_gemv_i8_gated(ctx, gj, uj, xp, T, yp);
    else
      launch_gemv_f32_gated(ctx, gj, uj, xp, T, yp);
  });
}

int mdma_gfx950_embed(mdma_ctx *ctx, const mdma_qweight *table, const uint32_t *ids, uint64_t n_ids,
                      mdma_buf *out) {
  return guarded([&] {
    need(ctx, "embed");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    prepare_weight(ctx, table);
    weight_row_bytes(table, "embed");
    uint64_t oe = f32_elems("embed", out);
    // shape::embed (shape.rs:92-110).
    if (!n_ids) shape_fail("embed: no tokens");
    if (oe < n_ids * table->cols)
      shape_fail(fmt("embed: out has %llu elems, needs %llu", (unsigned long long)oe,
                     (unsigned long long)(n_ids * table->cols)));
    same_ctx(ctx, table->buf, "embed");
    same_ctx(ctx, out, "embed");
    if (ctx->replay) {
      // Graph replay: the token id is read from params[0] when the kernel
      // runs (embed_gather_graph, src/backend/rocm/kernels/kernels.hip:385).
      if (n_ids != 1) shape_fail("embed: a replayed decode step embeds one token");
      launch_embed(ctx, table->dtype, table->buf->layout, reinterpret_cast<const uint8_t *>(table->buf->ptr),
                   table->cols, ctx->replay, 1, reinterpret_cast<float *>(out->ptr));
      return;
    }
    need(ids, "embed");
    for (uint64_t i = 0; i < n_ids; i++)
      if (ids[i] >= table->rows)
        shape_fail(fmt("embed: token_id %u out of range (vocab %llu)", ids[i],
                       (unsigned long long)table->rows));
    no_capture(ctx, "embed");
    uint32_t *dev_ids = reinterpret_cast<uint32_t *>(scratch(ctx, n_ids * 4));
    hip_check(hipMemcpyAsync(dev_ids, ids, n_ids * 4, hipMemcpyHostToDevice, ctx->stream), "embed ids");
    launch_embed(ctx, table->dtype, table->buf->layout, reinterpret_cast<const uint8_t *>(table->buf->ptr), table->cols,
                 dev_ids, n_ids, reinterpret_cast<float *>(out->ptr));
    // The ids live in scratch that a later call may overwrite.
    hip_check(hipStreamSynchronize(ctx->stream), "embed sync");
  });
}

// In the int8 mode, decode-sized rows also leave their int8 form in the
// activation cache, so a qmatmul that reads y next does not quantize again
// (the same values bit for bit as quantizing y there).
static void rmsnorm_rows(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                         float *y, uint64_t rows, float eps) {
  if (ctx->act_mode == MDMA_ACT_F32_CPU) return launch_rmsnorm_seq(ctx, w, dim, a, b, sum, y, rows, eps);
  if (ctx->act_mode == MDMA_ACT_I8 && rows < GEMM_MIN_TOKENS && launch_rmsnorm_q8(ctx, w, dim, a, b, sum, y, rows, eps))
    return;
  launch_rmsnorm(ctx, w, dim, a, b, sum, y, rows, eps);
}

int mdma_gfx950_rmsnorm(mdma_ctx *ctx, const mdma_buf *w, const mdma_buf *x, mdma_buf *y, float eps) {
  return guarded([&] {
    need(ctx, "rmsnorm");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    uint64_t dim = f32_elems("rmsnorm", w), xe = f32_elems("rmsnorm", x), ye = f32_elems("rmsnorm", y);
    // shape::rows (shape.rs:113-124).
    if (!dim || !xe || xe % dim) shape_fail(fmt("rmsnorm: x has %llu elems, not whole rows of %llu",
                                                (unsigned long long)xe, (unsigned long long)dim));
    if (ye < xe) shape_fail("rmsnorm: y too small");
    rmsnorm_rows(ctx, reinterpret_cast<const float *>(w->ptr), dim, reinterpret_cast<const float *>(x->ptr),
                 nullptr, nullptr, reinterpret_cast<float *>(y->ptr), xe / dim, eps);
  });
}

int mdma_gfx950_add_rmsnorm(mdma_ctx *ctx, const mdma_buf *w, const mdma_buf *a, const mdma_buf *b,
                            mdma_buf *sum, mdma_buf *y, float eps) {
  return guarded([&] {
    need(ctx, "add_rmsnorm");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    uint64_t dim = f32_elems("add_rmsnorm", w), ae = f32_elems("add_rmsnorm", a),
             be = f32_elems("add_rmsnorm", b), se = f32_elems("add_rmsnorm", sum),
             ye = f32_elems("add_rmsnorm", y);
    // add's shape::elementwise, then rmsnorm's shape::rows over `sum`.
    if (ae != be) shape_fail("add: input lengths differ");
    if (se < ae) shape_fail("add: output too small");
    if (!dim || !se || se % dim) shape_fail("rmsnorm: sum is not whole rows");
    if (ye < se) shape_fail("rmsnorm: y too small");
    if (se != ae) {
      // The default composition normalizes the whole `sum` buffer; keep that
      // exact behaviour when sum is longer than a + b.
      launch_add(ctx, reinterpret_cast<const float *>(a->ptr), reinterpret_cast<const float *>(b->ptr),
                 reinterpret_cast<float *>(sum->ptr), ae);
      if (ctx->act_mode == MDMA_ACT_F32_CPU)
        launch_rmsnorm_seq(ctx, reinterpret_cast<const float *>(w->ptr), dim, reinterpret_cast<const float *>(sum->ptr),
                           nullptr, nullptr, reinterpret_cast<float *>(y->ptr), se / dim, eps);
      else
        launch_rmsnorm(ctx, reinterpret_cast<const float *>(w->ptr), dim,
                       reinterpret_cast<const float *>(sum->ptr), nullptr, nullptr,
                       reinterpret_cast<float *>(y->ptr), se / dim, eps);
      return;
    }
    rmsnorm_rows(ctx, reinterpret_cast<const float *>(w->ptr), dim, reinterpret_cast<const float *>(a->ptr),
                 reinterpret_cast<const float *>(b->ptr), reinterpret_cast<float *>(sum->ptr),
                 reinterpret_cast<float *>(y->ptr), se / dim, eps);
  });
}

int mdma_gfx950_add(mdma_ctx *ctx, const mdma_buf *a, const mdma_buf *b, mdma_buf *y) {
  return guarded([&] {
    need(ctx, "add");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    uint64_t ae = f32_elems("add", a), be = f32_elems("add", b), ye = f32_elems("add", y);
    if (ae != be) shape_fail("add: input lengths differ");
    if (ye < ae) shape_fail("add: output too small");
    launch_add(ctx, reinterpret_cast<const float *>(a->ptr), reinterpret_cast<const float *>(b->ptr),
               reinterpret_cast<float *>(y->ptr), ae);
  });
}

int mdma_gfx950_silu_mul(mdma_ctx *ctx, const mdma_buf *gate, const mdma_buf *up, mdma_buf *y) {
  return guarded([&] {
    need(ctx, "silu_mul");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    uint64_t ge = f32_elems("silu_mul", gate), ue = f32_elems("silu_mul", up), ye = f32_elems("silu_mul", y);
    if (ge != ue) shape_fail("silu_mul: input lengths differ");
    if (ye < ge) shape_fail("silu_mul: output too small");
    if (ctx->act_mode == MDMA_ACT_F32_CPU)
      launch_silu_mul_seq(ctx, reinterpret_cast<const float *>(gate->ptr), reinterpret_cast<const float *>(up->ptr),
                          reinterpret_cast<float *>(y->ptr), ge);
    else
      launch_silu_mul(ctx, reinterpret_cast<const float *>(gate->ptr), reinterpret_cast<const float *>(up->ptr),
                      reinterpret_cast<float *>(y->ptr), ge);
  });
}

int mdma_gfx950_rope(mdma_ctx *ctx, mdma_buf *q, mdma_buf *k, uint32_t pos, uint64_t n_tokens,
                     const mdma_rope_spec *spec) {
  return guarded([&] {
    need(ctx, "rope");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    uint64_t qh, kh;
    check_rope(spec, f32_elems("rope", q), f32_elems("rope", k), n_tokens, &qh, &kh);
    // Graph replay: position params[1], the table covering the capacity.
    const uint32_t *pd = replay_pos(ctx, n_tokens, "rope");
    const float *tab = rope_table(ctx, pd ? ctx->replay_cap - 1 : pos + n_tokens - 1, spec->head_dim, spec->theta);
    launch_rope(ctx, reinterpret_cast<float *>(q->ptr), n_tokens, qh, spec->head_dim, tab, pos, pd);
    launch_rope(ctx, reinterpret_cast<float *>(k->ptr), n_tokens, kh, spec->head_dim, tab, pos, pd);
  });
}

int mdma_gfx950_kv_write(mdma_ctx *ctx, const mdma_buf *k, const mdma_buf *v, mdma_buf *dst_k,
                         mdma_buf *dst_v, uint64_t elem_offset, uint64_t n_elems) {
  return guarded([&] {
    need(ctx, "kv_write");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    // The default impl's two copies: n_elems f32 from offset 0 of k/v to
    // element elem_offset of the caches (2-byte elements here).
    range("kv_write", 0, n_elems * 4, f32_elems("kv_write", k) * 4);
    range("kv_write", 0, n_elems * 4, f32_elems("kv_write", v) * 4);
    need(dst_k, "kv_write");
    need(dst_v, "kv_write");
    if (ctx->replay) {
      // Graph replay (kv_write_graph, src/backend/rocm/kernels/kernels.hip:404):
      // the row at element params[1] * n_elems; the caches hold the capacity.
      range("kv_write", 0, n_elems * 2 * ctx->replay_cap, dst_k->len);
      range("kv_write", 0, n_elems * 2 * ctx->replay_cap, dst_v->len);
      if (!n_elems) return;
      launch_kv_write(ctx, reinterpret_cast<const float *>(k->ptr), reinterpret_cast<const float *>(v->ptr),
                      reinterpret_cast<uint16_t *>(dst_k->ptr), reinterpret_cast<uint16_t *>(dst_v->ptr), n_elems,
                      ctx->replay + 1);
      return;
    }
    range("kv_write", elem_offset * 2, n_elems * 2, dst_k->len);
    range("kv_write", elem_offset * 2, n_elems * 2, dst_v->len);
    if (!n_elems) return;
    launch_kv_write(ctx, reinterpret_cast<const float *>(k->ptr), reinterpret_cast<const float *>(v->ptr),
                    reinterpret_cast<uint16_t *>(dst_k->ptr) + elem_offset,
                    reinterpret_cast<uint16_t *>(dst_v->ptr) + elem_offset, n_elems);
  });
}

int mdma_gfx950_rope_kv_write(mdma_ctx *ctx, mdma_buf *q, mdma_buf *k, const mdma_buf *v,
                              mdma_buf *dst_k, mdma_buf *dst_v, uint64_t elem_offset, uint32_t pos,
                              uint64_t n_tokens, const mdma_rope_spec *spec, uint64_t n_elems) {
  return guarded([&] {
    need(ctx, "rope_kv_write");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    uint64_t qh, kh, ke = f32_elems("rope_kv_write", k);
    check_rope(spec, f32_elems("rope_kv_write", q), ke, n_tokens, &qh, &kh);
    range("kv_write", 0, n_elems * 4, ke * 4);
    range("kv_write", 0, n_elems * 4, f32_elems("rope_kv_write", v) * 4);
    need(dst_k, "rope_kv_write");
    need(dst_v, "rope_kv_write");
    const uint32_t *pd = replay_pos(ctx, n_tokens, "rope_kv_write");
    if (pd) {
      // Graph replay (rope_kv_graph, src/backend/rocm/kernels/kernels.hip:620):
      // position params[1], rows at element params[1] * k's width; the
      // caches hold the capacity.
      if (n_elems != ke || f32_elems("rope_kv_write", v) != ke)
        shape_fail("rope_kv_write: a replayed decode step writes k and v whole");
      range("kv_write", 0, n_elems * 2 * ctx->replay_cap, dst_k->len);
      range("kv_write", 0, n_elems * 2 * ctx->replay_cap, dst_v->len);
      const float *tab = rope_table(ctx, ctx->replay_cap - 1, spec->head_dim, spec->theta);
      launch_rope_kv_write(ctx, reinterpret_cast<float *>(q->ptr), qh, reinterpret_cast<const float *>(k->ptr),
                           reinterpret_cast<const float *>(v->ptr), kh, spec->head_dim, 1, tab, 0,
                           reinterpret_cast<uint16_t *>(dst_k->ptr), reinterpret_cast<uint16_t *>(dst_v->ptr), 0, 1,
                           pd);
      return;
    }
    range("kv_write", elem_offset * 2, n_elems * 2, dst_k->len);
    range("kv_write", elem_offset * 2, n_elems * 2, dst_v->len);
    const float *tab = rope_table(ctx, pos + n_tokens - 1, spec->head_dim, spec->theta);
    if (n_elems != ke || f32_elems("rope_kv_write", v) != ke) {
      // General composition of the default impl: rope q/k fully, then copy
      // the first n_elems of k and v.
      launch_rope(ctx, reinterpret_cast<float *>(q->ptr), n_tokens, qh, spec->head_dim, tab, pos);
      launch_rope(ctx, reinterpret_cast<float *>(k->ptr), n_tokens, kh, spec->head_dim, tab, pos);
      if (n_elems)
        launch_kv_write(ctx, reinterpret_cast<const float *>(k->ptr), reinterpret_cast<const float *>(v->ptr),
                        reinterpret_cast<uint16_t *>(dst_k->ptr) + elem_offset,
                        reinterpret_cast<uint16_t *>(dst_v->ptr) + elem_offset, n_elems);
      return;
    }
    launch_rope_kv_write(ctx, reinterpret_cast<float *>(q->ptr), qh, reinterpret_cast<const float *>(k->ptr),
                         reinterpret_cast<const float *>(v->ptr), kh, spec->head_dim, n_tokens, tab, pos,
                         reinterpret_cast<uint16_t *>(dst_k->ptr) + elem_offset,
                         reinterpret_cast<uint16_t *>(dst_v->ptr) + elem_offset);
  });
}

int mdma_gfx950_attn(mdma_ctx *ctx, const mdma_buf *q, const mdma_kv_view *kv, const mdma_attn_spec *spec,
                     mdma_buf *o) {
  return guarded([&] {
    need(ctx, "attn");
    need(kv, "attn");
    need(spec, "attn");
    need(kv->k, "attn");
    need(kv->v, "attn");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    // shape::attn (shape.rs:291-330); K/V elements counted at 2 bytes.
    uint64_t per = spec->n_q_heads * spec->head_dim, qe = f32_elems("attn", q), oe = f32_elems("attn", o);
    if (!per || !qe || qe % per) shape_fail("attn: q is not whole tokens of n_q_heads*head_dim");
    if (!spec->n_kv_heads || spec->n_q_heads % spec->n_kv_heads)
      shape_fail("attn: q heads are not a multiple of KV heads");
    if (spec->head_dim > 256) shape_fail("attn: head_dim above max_head_dim 256");
    uint64_t n_q = qe / per;
    // Graph replay (attn_decode_graph, src/backend/rocm/kernels/kernels.hip:695):
    // params[1] + 1 keys, the launch sized for the capacity.
    const uint32_t *pd = replay_pos(ctx, n_q, "attn");
    const uint64_t len = pd ? ctx->replay_cap : kv->len;
    if (n_q > len) shape_fail("attn: n_q exceeds kv.len");
    uint64_t need_e = len * spec->n_kv_heads * spec->head_dim;
    if (kv->k->len / 2 < need_e || kv->v->len / 2 < need_e) shape_fail("attn: K/V too short for kv.len");
    if (oe < qe) shape_fail("attn: o too small");
    const float *qp = reinterpret_cast<const float *>(q->ptr);
    const uint16_t *kp = reinterpret_cast<const uint16_t *>(kv->k->ptr), *vp = reinterpret_cast<const uint16_t *>(kv->v->ptr);
    float *op = reinterpret_cast<float *>(o->ptr);
    if (ctx->act_mode == MDMA_ACT_F32_CPU) {
      launch_attn_seq(ctx, qp, kp, vp, op, n_q, len, spec->head_dim, spec->n_q_heads, spec->n_kv_heads, 0, pd);
      return;
    }
    // In the int8 mode, decode-sized outputs also leave their int8 form in
    // the activation cache for a qmatmul that reads o next.
    if (ctx->act_mode == MDMA_ACT_I8 && n_q < GEMM_MIN_TOKENS &&
        launch_attn_q8(ctx, qp, kp, vp, op, n_q, len, spec->head_dim, spec->n_q_heads, spec->n_kv_heads, 0, pd))
      return;
    launch_attn(ctx, qp, kp, vp, op, n_q, len, spec->head_dim, spec->n_q_heads, spec->n_kv_heads, 0, pd);
  });
}

int mdma_gfx950_greedy(mdma_ctx *ctx, const mdma_buf *logits, uint64_t offset, uint64_t n, uint32_t *out) {
  return guarded([&] {
    need(ctx, "greedy");
    need(out, "greedy");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    range("greedy", offset * 4, n * 4, f32_elems("greedy", logits) * 4);
    no_capture(ctx, "greedy");
    if (!n) {
      *out = 0;
      return;
    }
    uint32_t *dev = reinterpret_cast<uint32_t *>(scratch(ctx, 256));
    launch_argmax_rows(ctx, reinterpret_cast<const float *>(logits->ptr) + offset, 1, n, dev, dev + 1);
    hip_check(hipMemcpyAsync(ctx->host_ids, dev, 8, hipMemcpyDeviceToHost, ctx->stream), "greedy d2h");
    hip_check(hipStreamSynchronize(ctx->stream), "greedy sync");
    if (ctx->host_ids[1]) fail(MDMA_ERR_BACKEND, "empty or nonfinite logits");
    *out = ctx->host_ids[0];
  });
}

int mdma_gfx950_quantize_act(mdma_ctx *ctx, const mdma_buf *x, uint64_t group, mdma_buf *q, mdma_buf *d,
                             mdma_buf *sum16) {
  return guarded([&] {
    need(ctx, "quantize_act");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    uint64_t n = f32_elems("quantize_act", x);
    if (group != 256 && group != 32) shape_fail("quantize_act: group must be 32 or 256");
    if (!n || n % group) shape_fail("quantize_act: x is not whole groups");
    need(q, "quantize_act");
    need(d, "quantize_act");
    need(sum16, "quantize_act");
    if (q->len < n || d->len < n / group * 4 || sum16->len < n / 16 * 4)
      shape_fail("quantize_act: output too small");
    launch_quantize_act(ctx, reinterpret_cast<const float *>(x->ptr), n, group,
                        reinterpret_cast<int8_t *>(q->ptr), reinterpret_cast<float *>(d->ptr),
                        reinterpret_cast<int32_t *>(sum16->ptr));
  });
}

int mdma_gfx950_block_dot_i32(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *qx, mdma_buf *out) {
  return guarded([&] {
    need(ctx, "block_dot_i32");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    prepare_weight(ctx, w);
    weight_row_bytes(w, "block_dot_i32");
    if (w->dtype != DT_Q4_K && w->dtype != DT_Q6_K && w->dtype != DT_Q8_0)
      fail(MDMA_ERR_NOT_IMPLEMENTED, "block_dot_i32: quantized dtypes only");
    need(qx, "block_dot_i32");
    need(out, "block_dot_i32");
    if (!qx->len || qx->len % w->cols) shape_fail("block_dot_i32: qx is not whole rows");
    uint64_t T = qx->len / w->cols, sub = w->dtype == DT_Q6_K ? 16 : 32;
    if (out->len < T * w->rows * (w->cols / sub) * 4) shape_fail("block_dot_i32: out too small");
    GemvJob j{w->dtype, reinterpret_cast<const uint8_t *>(w->buf->ptr), w->rows, w->cols, nullptr, w->buf->layout};
    launch_block_dot(ctx, j, reinterpret_cast<const int8_t *>(qx->ptr), T,
                     reinterpret_cast<int32_t *>(out->ptr));
  });
}

uint64_t mdma_gfx950_prepared_bytes(int32_t dtype, uint64_t rows, uint64_t cols) {
  if (!gfx950_layout_dtype(dtype)) return 0;
  const uint64_t rb = gfx950_row_bytes(dtype, cols);
  return rb && rows <= UINT64_MAX / rb ? rows * rb : 0;
}

int mdma_gfx950_pack_weight(int32_t dtype, uint64_t rows, uint64_t cols, const void *gguf, uint64_t len, void *out,
                            uint64_t out_len) {
  return guarded([&] {
    if (!gfx950_layout_dtype(dtype)) fail(MDMA_ERR_NOT_IMPLEMENTED, fmt("pack_weight: dtype %d has no prepared layout", dtype));
    const uint64_t bs = block_size(dtype);
    if (!rows || !cols || cols % bs || len != rows * (cols / bs) * type_size(dtype))
      shape_fail("pack_weight: bytes do not hold a [rows, cols] GGUF weight");
    if (out_len != mdma_gfx950_prepared_bytes(dtype, rows, cols)) shape_fail("pack_weight: output size");
    need(gguf, "pack_weight");
    need(out, "pack_weight");
    pack_gfx950(dtype, rows, cols, static_cast<const uint8_t *>(gguf), static_cast<uint8_t *>(out));
  });
}

int mdma_gfx950_unpack_weight(int32_t dtype, uint64_t rows, uint64_t cols, const void *prepared, uint64_t len,
                              void *out, uint64_t out_len) {
  return guarded([&] {
    if (!gfx950_layout_dtype(dtype)) fail(MDMA_ERR_NOT_IMPLEMENTED, fmt("unpack_weight: dtype %d has no prepared layout", dtype));
    const uint64_t bs = block_size(dtype);
    if (!rows || !cols || cols % bs || out_len != rows * (cols / bs) * type_size(dtype))
      shape_fail("unpack_weight: output does not hold a [rows, cols] GGUF weight");
    if (len != mdma_gfx950_prepared_bytes(dtype, rows, cols)) shape_fail("unpack_weight: input size");
    need(prepared, "unpack_weight");
    need(out, "unpack_weight");
    unpack_gfx950(dtype, rows, cols, static_cast<const uint8_t *>(prepared), static_cast<uint8_t *>(out));
  });
}

int mdma_gfx950_graph_begin(mdma_ctx *ctx) {
  return guarded([&] {
    need(ctx, "graph_begin");
    ctx->lock.lock();  // held until graph_end: no other thread may launch meanwhile
    if (ctx->capturing) {
      ctx->lock.unlock();
      fail(MDMA_ERR_BACKEND, "graph_begin: capture already in progress");
    }
    // A captured GEMV must not rely on int8 activations an earlier call left
    // in the cache: a replay would read whatever the buffer then holds.
    q8_invalidate(ctx);
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
      ctx->lock.unlock();
      hip_check(e, "hipStreamBeginCapture");
    }
    ctx->capturing = true;
  });
}

int mdma_gfx950_graph_end(mdma_ctx *ctx, mdma_graph **out) {
  return guarded([&] {
    need(ctx, "graph_end");
    need(out, "graph_end");
    *out = nullptr;
    if (!ctx->capturing) fail(MDMA_ERR_BACKEND, "graph_end: no capture in progress");
    ctx->capturing = false;
    hipGraph_t gr = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &gr);
    ctx->lock.unlock();
    hip_check(e, "hipStreamEndCapture");
    auto *g = new mdma_graph();
    g->graph = gr;
    g->ctx = ctx;
    g->epoch = ctx->buf_epoch;
    e = hipGraphInstantiate(&g->exec, gr, nullptr, nullptr, 0);
    if (e != hipSuccess) {
      (void)hipGraphDestroy(gr);
      delete g;
      hip_check(e, "hipGraphInstantiate");
    }
    *out = g;
  });
}

int mdma_gfx950_graph_launch(mdma_ctx *ctx, mdma_graph *graph) {
  return guarded([&] {
    need(ctx, "graph_launch");
    need(graph, "graph_launch");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    q8_invalidate(ctx);
    no_capture(ctx, "graph_launch");
    if (graph->ctx != ctx) fail(MDMA_ERR_BACKEND, "graph_launch: graph was captured on another context");
    // The graph holds addresses of context buffers as they were at capture.
    if (graph->epoch != ctx->buf_epoch)
      fail(MDMA_ERR_BACKEND, "graph_launch: context buffers were reallocated since capture (reserve_scratch "
                             "before capturing); capture again");
    hip_check(hipGraphLaunch(graph->exec, ctx->stream), "hipGraphLaunch");
  });
}

void mdma_gfx950_graph_destroy(mdma_graph *graph) {
  if (!graph) return;
  if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
  if (graph->graph) (void)hipGraphDestroy(graph->graph);
  delete graph;
}

int mdma_gfx950_time_next_gemv(mdma_ctx *ctx, void *start_event, void *stop_event) {
  return guarded([&] {
    need(ctx, "time_next_gemv");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    no_capture(ctx, "time_next_gemv");
    ctx->time_start = static_cast<hipEvent_t>(start_event);
    ctx->time_stop = static_cast<hipEvent_t>(stop_event);
  });
}

int mdma_gfx950_set_replay_params(mdma_ctx *ctx, const mdma_buf *params, uint64_t capacity) {
  return guarded([&] {
    need(ctx, "set_replay_params");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    if (!params) {
      ctx->replay = nullptr;
      ctx->replay_cap = 0;
      return;
    }
    same_ctx(ctx, params, "set_replay_params");
    if (params->len < 8) shape_fail("set_replay_params: params must hold two uint32 (token, position)");
    if (reinterpret_cast<uintptr_t>(params->ptr) % 4) shape_fail("set_replay_params: params must be 4-byte aligned");
    if (!capacity || capacity > 0xffffffffull) shape_fail("set_replay_params: capacity out of range");
    ctx->replay = reinterpret_cast<const uint32_t *>(params->ptr);
    ctx->replay_cap = capacity;
  });
}

int mdma_gfx950_reserve_scratch(mdma_ctx *ctx, uint64_t bytes) {
  return guarded([&] {
    need(ctx, "reserve_scratch");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    scratch(ctx, bytes);
    q8_buffer(ctx, bytes);
  });
}

}  // extern "C"
