// Llama decoding on the gfx950 backend: the caller of the quantized-weight
// hot path.
//
// Restates, on top of this library's kernels:
//  - GGUF reading (/root/reference/src/gguf.rs:30-231): header, typed
//    metadata, tensor descriptors with dims reversed to [rows, cols];
//  - Llama preflight and config (src/model/arch/llama.rs:16-38,
//    src/model/arch/llama/preflight.rs:48-143);
//  - memory planning (src/model/memory.rs:16-63, src/memory.rs:39-97,
//    headroom src/registry.rs:37): weights, KV and workspace are reserved
//    against the budget and the device before anything is allocated;
//  - Llama::run_layers (src/model/arch/llama.rs:158-246), Model::prefill /
//    forward (src/model.rs:326-468) and the greedy loop of inference::sample
//    (src/inference.rs:102-124).
// Decoding stays on the device: argmax writes each token id to device
// memory, where the next step's embedding reads it, so a whole generation
// is queued without a host round trip per token.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "internal.h"

using namespace mdma;

namespace {

// ------------------------------------------------------------------ GGUF --

struct GgufTensor {
  int32_t dtype = 0;
  uint64_t rows = 1, cols = 0, offset = 0, bytes = 0;
};

struct Gguf {
  FILE *f = nullptr;
  std::map<std::string, double> num;
  std::map<std::string, std::string> str;
  std::map<std::string, GgufTensor> tensors;
  ~Gguf() {
    if (f) fclose(f);
  }
  void rd(void *p, size_t n) {
    if (fread(p, 1, n, f) != n) fail(MDMA_ERR_IO, "gguf: truncated file");
  }
  template <class T>
  T get() {
    T v;
    rd(&v, sizeof v);
    return v;
  }
  std::string gstr() {
    uint64_t n = get<uint64_t>();
    if (n > (1u << 24)) fail(MDMA_ERR_IO, "gguf: string too long");
    std::string s(n, '\0');
    if (n) rd(&s[0], n);
    return s;
  }
  // Read one value of type t; numeric values land in *out when given.
  void value(uint32_t t, double *out, std::string *sout) {
    double v = 0;
    switch (t) {
      case 0: v = get<uint8_t>(); break;
      case 1: v = get<int8_t>(); break;
      case 2: v = get<uint16_t>(); break;
      case 3: v = get<int16_t>(); break;
      case 4: v = get<uint32_t>(); break;
      case 5: v = get<int32_t>(); break;
      case 6: v = get<float>(); break;
      case 7: v = get<uint8_t>(); break;
      case 8: {
        std::string s = gstr();
        if (sout) *sout = s;
        return;
      }
      case 9: {
        uint32_t et = get<uint32_t>();
        uint64_t n = get<uint64_t>();
        for (uint64_t i = 0; i < n; i++) value(et, nullptr, nullptr);
        return;
      }
      case 10: v = (double)get<uint64_t>(); break;
      case 11: v = (double)get<int64_t>(); break;
      case 12: v = get<double>(); break;
      default: fail(MDMA_ERR_IO, "gguf: unknown metadata type");
    }
    if (out) *out = v;
  }
  void open(const char *path) {
    f = fopen(path, "rb");
    if (!f) fail(MDMA_ERR_IO, std::string("gguf: cannot open ") + path);
    char magic[4];
    rd(magic, 4);
    if (memcmp(magic, "GGUF", 4)) fail(MDMA_ERR_UNSUPPORTED_MODEL, "gguf: bad magic");
    uint32_t version = get<uint32_t>();
    if (version != 2 && version != 3) fail(MDMA_ERR_UNSUPPORTED_MODEL, "gguf: unsupported version");
    uint64_t n_t = get<uint64_t>(), n_kv = get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; i++) {
      std::string key = gstr();
      uint32_t t = get<uint32_t>();
      double v = 0;
      std::string s;
      value(t, &v, &s);
      if (t == 8)
        str[key] = s;
      else if (t != 9)
        num[key] = v;
    }
    std::vector<std::pair<std::string, GgufTensor>> raw;
    for (uint64_t i = 0; i < n_t; i++) {
      std::string name = gstr();
      uint32_t nd = get<uint32_t>();
      if (nd == 0 || nd > 4) fail(MDMA_ERR_UNSUPPORTED_MODEL, "gguf: tensor rank");
      // tensor_n_bytes (src/gguf.rs): element and byte counts without
      // overflow, whole blocks only; errors name the tensor.
      GgufTensor t;
      bool over = false;
      for (uint32_t d = 0; d < nd; d++) {
        uint64_t dim = get<uint64_t>();
        if (d == 0) {
          t.cols = dim;  // ne0: the contiguous (column) dimension
        } else {
          over |= dim && t.rows > UINT64_MAX / dim;
          t.rows *= dim;
        }
      }
      t.dtype = (int32_t)get<uint32_t>();
      t.offset = get<uint64_t>();
      uint64_t bs = block_size(t.dtype), ts = type_size(t.dtype);
      if (!bs || t.cols % bs) fail(MDMA_ERR_UNSUPPORTED_MODEL, "gguf: " + name + " has an unsupported dtype or width");
      const uint64_t blocks = t.cols / bs;
      over |= t.rows && blocks > UINT64_MAX / t.rows;
      over |= !over && ts && t.rows * blocks > UINT64_MAX / ts;
      if (over) fail(MDMA_ERR_UNSUPPORTED_MODEL, "gguf: " + name + " byte size overflows");
      t.bytes = t.rows * blocks * ts;
      raw.push_back({name, t});
    }
    uint64_t align = num.count("general.alignment") ? (uint64_t)num["general.alignment"] : 32;
    if (!align) fail(MDMA_ERR_UNSUPPORTED_MODEL, "gguf: zero alignment");
    long pos = ftell(f);
    uint64_t data = ((uint64_t)pos + align - 1) / align * align;
    if (fseeko(f, 0, SEEK_END)) fail(MDMA_ERR_IO, "gguf: seek");
    const uint64_t file_len = (uint64_t)ftello(f);
    for (auto &kv : raw) {
      // tensor_start (src/gguf.rs): data + offset + bytes within the file,
      // without overflow.
      GgufTensor &t = kv.second;
      if (t.offset > UINT64_MAX - data || t.bytes > UINT64_MAX - (data + t.offset) ||
          data + t.offset + t.bytes > file_len)
        fail(MDMA_ERR_UNSUPPORTED_MODEL, "gguf: " + kv.first + " extends past the end of the file");
      t.offset += data;
      tensors[kv.first] = t;
    }
  }
  void read(const GgufTensor &t, std::vector<uint8_t> &buf) {
    buf.resize(t.bytes);
    if (fseeko(f, (off_t)t.offset, SEEK_SET)) fail(MDMA_ERR_IO, "gguf: seek");
    rd(buf.data(), t.bytes);
  }
};

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
  char b[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(b, sizeof b, f, ap);
  va_end(ap);
  return b;
}

constexpr uint64_t DEVICE_HEADROOM = 256ull << 20;  // src/registry.rs:37

struct Weight {
  int32_t dtype = 0;
  uint64_t rows = 0, cols = 0;
  mdma_buf *buf = nullptr;
  GemvJob job(float *y) const {
    GemvJob j{dtype, reinterpret_cast<const uint8_t *>(buf->ptr), rows, cols, y, buf->layout};
    j.src = buf;
    return j;
  }
};

struct Layer {
  mdma_buf *attn_norm = nullptr, *ffn_norm = nullptr;
  Weight wq, wk, wv, wo, gate, up, down;
};

const float *fp(const mdma_buf *b) { return reinterpret_cast<const float *>(b->ptr); }
float *fp(mdma_buf *b) { return reinterpret_cast<float *>(b->ptr); }

}  // namespace

struct mdma_model {
  mdma_ctx *ctx = nullptr;
  mdma_model_config cfg{};
  Weight token_embd, output;
  mdma_buf *output_norm = nullptr;
  std::vector<Layer> layers;
  uint64_t weight_bytes = 0;
  // The batch GEMV's tile images of the Q6_K matrices (made at their first
  // batched call once a session of BATCH_MIN_TOKENS sequences or more
  // turns the context's batch layout on); reserved by that session.
  uint64_t tile_bytes = 0;
  bool tiles_reserved = false;
  uint64_t budget = 0;  // 0 = unlimited (NativeMemoryBudget limit)
  uint64_t reserved = 0;
  std::vector<mdma_buf *> owned;
  ~mdma_model() {
    for (mdma_buf *b : owned) mdma_gfx950_free(b);
  }
};

struct mdma_session {
  mdma_model *m = nullptr;
  uint64_t capacity = 0, batch = 0, rows = 0;  // rows: workspace token rows
  std::vector<mdma_buf *> kc, vc;              // per layer: [batch][capacity][kv_w] f16
  mdma_buf *x = nullptr, *x_alt = nullptr, *normed = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
           *attn_out = nullptr, *proj = nullptr, *gate = nullptr, *up = nullptr, *act = nullptr,
           *logits = nullptr, *ids = nullptr, *flags = nullptr;
  std::vector<uint64_t> len;  // KV positions written, per sequence
  uint64_t reserved = 0;
  std::vector<mdma_buf *> owned;
  ~mdma_session() {
    for (mdma_buf *b : owned) mdma_gfx950_free(b);
    if (m) m->reserved -= reserved;
  }
};

namespace {

mdma_buf *alloc_or_throw(mdma_ctx *ctx, uint64_t bytes, int pool, std::vector<mdma_buf *> &owned) {
  mdma_buf *b = nullptr;
  int st = mdma_gfx950_alloc(ctx, bytes ? bytes : 4, pool, &b);
  if (st) fail(st, mdma_gfx950_last_error());
  owned.push_back(b);
  return b;
}

// Workspace bytes for `rows` token rows (src/model/memory.rs:39-63) plus the
// batch logits and the device token/flag buffers of the decode loop.
uint64_t workspace_bytes(const mdma_model_config &c, uint64_t rows, uint64_t batch, uint64_t n_ids) {
  const uint64_t e = c.n_embd * rows * 4, qb = c.n_heads * c.head_dim * rows * 4,
                 kb = c.n_kv_heads * c.head_dim * rows * 4, f = c.n_ff * rows * 4;
  return 3 * e + qb + 2 * kb + qb + e + 3 * f + c.vocab * (batch ? batch : 1) * 4 + 2 * n_ids * 4;
}

uint64_t kv_bytes(const mdma_model_config &c, uint64_t capacity, uint64_t batch) {
  return c.n_layers * 2 * batch * capacity * c.n_kv_heads * c.head_dim * 2;
}

// Reserve before allocating: the budget first (MemoryBudget), then the device
// with headroom (InsufficientMemory).
void reserve(mdma_model *m, uint64_t bytes) {
  if (m->budget && m->reserved + bytes > m->budget)
    throw Error{MDMA_ERR_MEMORY_BUDGET, fmt("native tensor memory budget exhausted: requested %llu bytes, "
                                            "used/reserved %llu, limit %llu", (unsigned long long)bytes,
                                            (unsigned long long)m->reserved, (unsigned long long)m->budget)};
  uint64_t avail = 0;
  int st = mdma_gfx950_available_device_bytes(m->ctx, &avail);
  if (st) fail(st, mdma_gfx950_last_error());
  if (bytes + DEVICE_HEADROOM > avail)
    throw Error{MDMA_ERR_INSUFFICIENT_MEMORY,
                fmt("insufficient device memory: requested %llu bytes including headroom, available %llu",
                    (unsigned long long)(bytes + DEVICE_HEADROOM), (unsigned long long)avail)};
  m->reserved += bytes;
}

void check_weight(const Gguf &g, const std::string &name, uint64_t rows, uint64_t cols) {
  auto it = g.tensors.find(name);
  if (it == g.tensors.end()) shape_fail("missing tensor " + name);
  const GgufTensor &t = it->second;
  if (t.rows != rows || t.cols != cols)
    shape_fail(fmt("%s: shape [%llu, %llu], expected [%llu, %llu]", name.c_str(), (unsigned long long)t.rows,
                   (unsigned long long)t.cols, (unsigned long long)rows, (unsigned long long)cols));
  if (t.dtype != DT_F32 && t.dtype != DT_F16 && t.dtype != DT_Q8_0 && t.dtype != DT_Q4_K && t.dtype != DT_Q6_K)
    fail(MDMA_ERR_UNSUPPORTED_MODEL, fmt("%s: dtype %d is not supported on gfx950", name.c_str(), t.dtype));
}

void check_norm(const Gguf &g, const std::string &name, uint64_t n) {
  auto it = g.tensors.find(name);
  if (it == g.tensors.end()) shape_fail("missing tensor " + name);
  if (it->second.dtype != DT_F32) shape_fail(name + ": expected F32 norm weight");
  if (it->second.rows * it->second.cols != n) shape_fail(name + ": wrong length");
}

// Llama config and preflight (src/model/arch/llama.rs:16-38; preflight.rs:48-143).
mdma_model_config preflight(const Gguf &g) {
  auto sit = g.str.find("general.architecture");
  if (sit == g.str.end()) fail(MDMA_ERR_UNSUPPORTED_MODEL, "missing general.architecture");
  const std::string arch = sit->second;
  if (arch != "llama") fail(MDMA_ERR_UNSUPPORTED_MODEL, "unsupported architecture " + arch);
  auto key = [&](const char *k, bool required, double def) -> double {
    auto it = g.num.find(arch + "." + k);
    if (it == g.num.end()) {
      if (required) fail(MDMA_ERR_UNSUPPORTED_MODEL, std::string("missing metadata ") + arch + "." + k);
      return def;
    }
    return it->second;
  };
  mdma_model_config c{};
  c.n_embd = (uint64_t)key("embedding_length", true, 0);
  c.n_heads = (uint64_t)key("attention.head_count", true, 0);
  c.n_layers = (uint64_t)key("block_count", true, 0);
  c.n_ff = (uint64_t)key("feed_forward_length", true, 0);
  c.n_kv_heads = (uint64_t)key("attention.head_count_kv", false, (double)c.n_heads);
  c.rope_theta = (float)key("rope.freq_base", false, 10000.0);
  c.rms_eps = (float)key("attention.layer_norm_rms_epsilon", true, 0);
  c.n_ctx = (uint64_t)key("context_length", true, 0);
  if (!c.n_heads || !c.n_embd || c.n_embd % c.n_heads) fail(MDMA_ERR_UNSUPPORTED_MODEL, "n_embd % n_heads");
  c.head_dim = c.n_embd / c.n_heads;
  if (!c.n_kv_heads || c.n_heads % c.n_kv_heads) fail(MDMA_ERR_UNSUPPORTED_MODEL, "n_heads % n_kv_heads");
  if (c.head_dim % 2 || c.head_dim > 256) fail(MDMA_ERR_UNSUPPORTED_MODEL, "head_dim must be even and <= 256");
  if (!c.n_layers || !c.n_ff || !c.n_ctx) fail(MDMA_ERR_UNSUPPORTED_MODEL, "empty geometry");
  auto te = g.tensors.find("token_embd.weight");
  if (te == g.tensors.end()) shape_fail("missing tensor token_embd.weight");
  c.vocab = te->second.rows;
  const uint64_t qd = c.n_heads * c.head_dim, kd = c.n_kv_heads * c.head_dim;
  check_weight(g, "token_embd.weight", c.vocab, c.n_embd);
  check_weight(g, "output.weight", c.vocab, c.n_embd);
  check_norm(g, "output_norm.weight", c.n_embd);
  for (uint64_t i = 0; i < c.n_layers; i++) {
    const std::string p = "blk." + std::to_string(i) + ".";
    check_norm(g, p + "attn_norm.weight", c.n_embd);
    check_norm(g, p + "ffn_norm.weight", c.n_embd);
    check_weight(g, p + "attn_q.weight", qd, c.n_embd);
    check_weight(g, p + "attn_k.weight", kd, c.n_embd);
    check_weight(g, p + "attn_v.weight", kd, c.n_embd);
    check_weight(g, p + "attn_output.weight", c.n_embd, qd);
    check_weight(g, p + "ffn_gate.weight", c.n_ff, c.n_embd);
    check_weight(g, p + "ffn_up.weight", c.n_ff, c.n_embd);
    check_weight(g, p + "ffn_down.weight", c.n_embd, c.n_ff);
  }
  return c;
}

Weight load_weight(mdma_model *m, Gguf &g, const std::string &name, std::vector<uint8_t> &tmp) {
  const GgufTensor &t = g.tensors.at(name);
  g.read(t, tmp);
  Weight w;
  w.dtype = t.dtype;
  w.rows = t.rows;
  w.cols = t.cols;
  int st = mdma_gfx950_upload_weight_typed(m->ctx, tmp.data(), t.bytes, MDMA_LAYOUT_GGUF, t.dtype, t.rows, t.cols,
                                           &w.buf);
  if (st) fail(st, mdma_gfx950_last_error());
  m->owned.push_back(w.buf);
  return w;
}

mdma_buf *load_norm(mdma_model *m, Gguf &g, const std::string &name, std::vector<uint8_t> &tmp) {
  const GgufTensor &t = g.tensors.at(name);
  g.read(t, tmp);
  mdma_buf *b = alloc_or_throw(m->ctx, t.bytes, MDMA_POOL_WEIGHTS, m->owned);
  int st = mdma_gfx950_upload(m->ctx, b, 0, tmp.data(), t.bytes);
  if (st) fail(st, mdma_gfx950_last_error());
  return b;
}

// fresh: x's int8 form was just written by launch_rmsnorm_q8 (kept);
// otherwise inputs here are rewritten between calls without passing through
// the C entry points, so cached int8 activations are not reused.
void gemv(mdma_ctx *ctx, const GemvJob *jobs, int n, const float *x, uint64_t T, bool fresh = false) {
  if (!fresh) q8_invalidate(ctx);
  if (ctx->act_mode == MDMA_ACT_I8)
    launch_gemv_i8(ctx, jobs, n, x, T);
  else if (ctx->act_mode == MDMA_ACT_F32_CPU)
    for (int i = 0; i < n; i++) launch_gemv_seq(ctx, jobs[i], x, T);
  else
    launch_gemv_f32(ctx, jobs, n, x, T);
}

// The CPU-order mode runs the trait's default ffn_gate_up (backend.rs:472-489):
// gate and up into their buffers, then silu_mul.
void gemv_gated(mdma_ctx *ctx, const GemvJob &g, const GemvJob &u, const float *x, uint64_t T, float *y,
                bool fresh = false) {
  if (!fresh) q8_invalidate(ctx);
  if (ctx->act_mode == MDMA_ACT_I8) {
    launch_gemv_i8_gated(ctx, g, u, x, T, y);
  } else if (ctx->act_mode == MDMA_ACT_F32_CPU) {
    launch_gemv_seq(ctx, g, x, T);
    launch_gemv_seq(ctx, u, x, T);
    launch_silu_mul_seq(ctx, g.y, u.y, y, T * g.n_out);
  } else {
    launch_gemv_f32_gated(ctx, g, u, x, T, y);
  }
}

void rmsnorm(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum, float *y,
             uint64_t rows, float eps) {
  if (ctx->act_mode == MDMA_ACT_F32_CPU)
    launch_rmsnorm_seq(ctx, w, dim, a, b, sum, y, rows, eps);
  else
    launch_rmsnorm(ctx, w, dim, a, b, sum, y, rows, eps);
}

// Llama::run_layers (src/model/arch/llama.rs:158-246) for T token rows in
// s->x. seq_stride = 0: one sequence `seq`, rows at positions pos..pos+T-1
// (prefill or decode). seq_stride > 0: row t is the single decode token of
// sequence t, all at position pos (batched decode). Leaves the final-normed
// rows in s->normed.
// pos_dev (a captured decode step, T new tokens of one position): the
// position is read from device memory at run time and pos is unused; the
// RoPE table then covers the whole cache, and a shape whose attention has no
// such launch fails instead of falling back.
void run_layers(mdma_session *s, uint64_t T, uint32_t pos, uint64_t seq, bool batched,
                const uint32_t *pos_dev = nullptr) {
  mdma_model *m = s->m;
  mdma_ctx *ctx = m->ctx;
  const mdma_model_config &c = m->cfg;
  const uint64_t E = c.n_embd, hd = c.head_dim, kvw = c.n_kv_heads * hd;
  const float *tab = rope_table(ctx, pos_dev ? s->capacity - 1 : pos + (batched ? 0 : T - 1), hd, c.rope_theta);
  mdma_buf *x = s->x, *x_alt = s->x_alt;
  const uint64_t cache_stride = s->capacity * kvw;
  // In the int8 mode, decode-sized rows get their int8 form from the
  // rmsnorm that produces them (prefill-sized ones go to the int8 GEMM,
  // which quantizes per 32 itself).
  const bool fuse_q8 = ctx->act_mode == MDMA_ACT_I8 && T < GEMM_MIN_TOKENS;
  // Prefill rows in the int8 mode whose GEMMs (cons) run on the f16 path:
  // the rmsnorm also writes those GEMMs' input, into attn_out (not in use
  // from the norm to the GEMMs that read it), and the GEMMs skip their own
  // quantization pass.
  auto a16_for = [&](const GemvJob *cons, int n) {
    if (!cons || !ctx->norm_fusion || ctx->act_mode != MDMA_ACT_I8 || ctx->prefill_kernel != MDMA_PREFILL_AUTO ||
        T < GEMM_MIN_TOKENS || ctx->fixed_scratch || ctx->capturing)
      return false;
    for (int i = 0; i < n; i++)
      if (!gemm_f16_supported(cons[i].dtype, cons[i].layout, cons[i].n_in, cons[i].n_out)) return false;
    return true;
  };
  auto norm = [&](const mdma_buf *w, const float *a, const float *b, float *sum, const GemvJob *cons = nullptr,
                  int n_cons = 0) {
    q8_invalidate(ctx);
    if (fuse_q8 && launch_rmsnorm_q8(ctx, fp(w), E, a, b, sum, fp(s->normed), T, c.rms_eps)) return true;
    if (a16_for(cons, n_cons) && launch_rmsnorm_a16(ctx, fp(w), E, a, b, sum, fp(s->normed), T, c.rms_eps,
                                                    s->attn_out->ptr, s->attn_out->len))
      return true;
    rmsnorm(ctx, fp(w), E, a, b, sum, fp(s->normed), T, c.rms_eps);
    return false;
  };
  bool fresh = false;
  auto attend = [&](const uint16_t *kc, const uint16_t *vc, uint64_t n_q, uint64_t kv_len, uint64_t stride) {
    q8_invalidate(ctx);
    fresh = fuse_q8 && launch_attn_q8(ctx, fp(s->q), kc, vc, fp(s->attn_out), n_q, kv_len, hd, c.n_heads,
                                      c.n_kv_heads, stride);
    if (!fresh) launch_attn(ctx, fp(s->q), kc, vc, fp(s->attn_out), n_q, kv_len, hd, c.n_heads, c.n_kv_heads, stride);
  };
  // One new token per sequence (a decode step): RoPE, the K/V cache write
  // and attention in one launch.
  // The int8 output form first (when this mode wants it), else f32 output.
  auto decode_attend = [&](uint16_t *kc, uint16_t *vc, uint64_t stride) {
    q8_invalidate(ctx);
    for (bool q8 : {fuse_q8, false}) {
      if (launch_attn_rope(ctx, fp(s->q), fp(s->k), fp(s->v), tab, (uint32_t)pos, kc, vc, fp(s->attn_out), T,
                           pos_dev ? s->capacity : pos + 1, hd, c.n_heads, c.n_kv_heads, stride, q8, pos_dev)) {
        fresh = q8;
        return true;
      }
      if (!q8) break;
    }
    if (pos_dev) fail(MDMA_ERR_BACKEND, "graph decode: no captured attention launch for this shape");
    return false;
  };
  // One token per step (decode of one sequence): the attention rmsnorm of
  // layers after the first is fused into the GEMVs around it. The previous
  // layer's down projection stores the residual stream x + W act and
  // per-workgroup sums of squares; the QKV GEMV normalizes x in its prologue.
  // n_part > 0: x already holds the residual stream and the partials wait.
  const bool fuse_norm = ctx->norm_fusion && fuse_q8 && T == 1 && !batched;
  const bool cpu_order = ctx->act_mode == MDMA_ACT_F32_CPU;
  uint32_t n_part = 0;
  for (uint64_t i = 0; i < c.n_layers; i++) {
    const Layer &L = m->layers[i];
    GemvJob qkv[3] = {L.wq.job(fp(s->q)), L.wk.job(fp(s->k)), L.wv.job(fp(s->v))};
    bool qkv_done = false;
    if (i == 0) {
      fresh = norm(L.attn_norm, fp(x), nullptr, nullptr, qkv, 3);
    } else if (n_part) {
      q8_invalidate(ctx);
      qkv_done = launch_gemv_i8_normed(ctx, qkv, 3, fp(x), fp(L.attn_norm), n_part, c.rms_eps);
      if (!qkv_done) fresh = norm(L.attn_norm, fp(x), nullptr, nullptr, qkv, 3);
    } else {
      fresh = norm(L.attn_norm, fp(x), fp(s->proj), fp(x_alt), qkv, 3);
      std::swap(x, x_alt);
    }
    // KvCache::rope_write (src/kv_cache.rs:212-244): rotate q, store rotated k and v.
    uint16_t *kb = reinterpret_cast<uint16_t *>(s->kc[i]->ptr), *vb = reinterpret_cast<uint16_t *>(s->vc[i]->ptr);
    // A prompt's fused QKV GEMM can do that in its epilogue (rope_done).
    ctx->rope_done = false;
    if (!qkv_done && !batched && !cpu_order && !pos_dev && T > 1 && a16_for(qkv, 3)) {
      ctx->rope_want_q = fp(s->q);
      ctx->rope_want_tab = tab;
      ctx->rope_want_dk = kb + seq * cache_stride + pos * kvw;
      ctx->rope_want_dv = vb + seq * cache_stride + pos * kvw;
      ctx->rope_want_pos = pos;
      ctx->rope_want_hd = (uint32_t)hd;
      ctx->rope_want_stride = kvw;
    }
    if (!qkv_done) gemv(ctx, qkv, 3, fp(s->normed), T, fresh);
    ctx->rope_want_q = nullptr;
    if (cpu_order) {
      // The CPU's order: RoPE and the cache write, then attention; a
      // captured step reads the position from device memory in both.
      uint16_t *ks = batched ? kb : kb + seq * cache_stride, *vs = batched ? vb : vb + seq * cache_stride;
      const uint64_t at = pos_dev ? 0 : (uint64_t)pos * kvw;
      launch_rope_kv_write(ctx, fp(s->q), c.n_heads, fp(s->k), fp(s->v), c.n_kv_heads, hd, T, tab, pos, ks + at,
                           vs + at, batched ? cache_stride : 0, batched ? 0 : 1, pos_dev);
      launch_attn_seq(ctx, fp(s->q), ks, vs, fp(s->attn_out), T, pos_dev ? s->capacity : pos + (batched ? 1 : T), hd,
                      c.n_heads, c.n_kv_heads, batched ? cache_stride : 0, pos_dev);
    } else if ((batched || T == 1) && decode_attend(batched ? kb : kb + seq * cache_stride,
                                             batched ? vb : vb + seq * cache_stride, batched ? cache_stride : 0)) {
      // RoPE, the cache write and attention in one launch.
    } else if (batched) {
      launch_rope_kv_write(ctx, fp(s->q), c.n_heads, fp(s->k), fp(s->v), c.n_kv_heads, hd, T, tab, pos,
                           kb + pos * kvw, vb + pos * kvw, cache_stride, 0);
      attend(kb, vb, T, pos + 1, cache_stride);
    } else {
      uint16_t *ks = kb + seq * cache_stride, *vs = vb + seq * cache_stride;
      if (!ctx->rope_done)
        launch_rope_kv_write(ctx, fp(s->q), c.n_heads, fp(s->k), fp(s->v), c.n_kv_heads, hd, T, tab, pos,
                             ks + pos * kvw, vs + pos * kvw);
      // A prompt's attention can also write a Q6_K output projection's
      // f16-path input, into up (free until the gate/up GEMM).
      const GemvJob wo_in = L.wo.job(fp(s->proj));
      if (a16_for(&wo_in, 1) && wo_in.dtype == DT_Q6_K) {
        ctx->a16_want_y = fp(s->attn_out);
        ctx->a16_want_buf = s->up->ptr;
        ctx->a16_want_bytes = s->up->len;
      }
      attend(ks, vs, T, pos + T, 0);
      ctx->a16_want_y = nullptr;
    }
    GemvJob wo = L.wo.job(fp(s->proj));
    gemv(ctx, &wo, 1, fp(s->attn_out), T, fresh || a16_holds(ctx, fp(s->attn_out), T, c.n_heads * hd));
    const GemvJob gu[2] = {L.gate.job(fp(s->gate)), L.up.job(fp(s->up))};
    fresh = norm(L.ffn_norm, fp(x), fp(s->proj), fp(x_alt), gu, 2);
    std::swap(x, x_alt);
    // A Q6_K down projection on the f16 path: the gated GEMM also writes its
    // input, into the gate buffer (the gated launch does not write it).
    const GemvJob dn_next = L.down.job(fp(s->proj));
    if (a16_for(&dn_next, 1) && dn_next.dtype == DT_Q6_K) {
      ctx->a16_want_y = fp(s->act);
      ctx->a16_want_buf = s->gate->ptr;
      ctx->a16_want_bytes = s->gate->len;
      // The down GEMM below reads act only through that input.
      ctx->a16_want_input_only = !dn_next.dots;
    }
    gemv_gated(ctx, gu[0], gu[1], fp(s->normed), T, fp(s->act), fresh);
    ctx->a16_want_y = nullptr;
    ctx->a16_want_input_only = false;
    n_part = 0;
    if (fuse_norm) {
      // y = x + W act into the other residual buffer (the new stream).
      q8_invalidate(ctx);
      n_part = launch_gemv_i8_residual(ctx, L.down.job(fp(x_alt)), fp(s->act), fp(x));
      if (n_part) std::swap(x, x_alt);
    }
    if (!n_part) {
      GemvJob dn = L.down.job(fp(s->proj));
      gemv(ctx, &dn, 1, fp(s->act), T, a16_holds(ctx, fp(s->act), T, c.n_ff));
    }
  }
  // The head GEMV quantizes the final-normed rows itself when it needs
  // them (only the rows it reads, which may be a subset).
  if (n_part) {
    launch_rmsnorm(ctx, fp(m->output_norm), E, fp(x), nullptr, nullptr, fp(s->normed), T, c.rms_eps);
  } else {
    rmsnorm(ctx, fp(m->output_norm), E, fp(x), fp(s->proj), fp(x_alt), fp(s->normed), T, c.rms_eps);
    std::swap(x, x_alt);
  }
  // Keep s->x as the buffer holding the residual stream.
  if (x != s->x) std::swap(s->x, s->x_alt);
}

void embed_dev(mdma_session *s, const uint32_t *ids_dev, uint64_t n) {
  const Weight &te = s->m->token_embd;
  launch_embed(s->m->ctx, te.dtype, te.buf->layout, reinterpret_cast<const uint8_t *>(te.buf->ptr), te.cols, ids_dev, n,
               fp(s->x));
}

// Output head on `rows` rows starting at row r0 of normed, logits to logits + out_row*vocab.
void head(mdma_session *s, uint64_t r0, uint64_t rows, uint64_t out_row) {
  const mdma_model_config &c = s->m->cfg;
  GemvJob h = s->m->output.job(fp(s->logits) + out_row * c.vocab);
  gemv(s->m->ctx, &h, 1, fp(s->normed) + r0 * c.n_embd, rows);
}

void check_tokens(const mdma_model *m, const uint32_t *ids, uint64_t n) {
  for (uint64_t i = 0; i < n; i++)
    if (ids[i] >= m->cfg.vocab) shape_fail("prefill token outside vocabulary");
}

void prefill_seq(mdma_session *s, uint64_t seq, const uint32_t *tokens, uint64_t n, uint32_t pos) {
  if (!n) shape_fail("prefill: tokens must be non-empty");
  if (n > s->rows) shape_fail("prefill: more tokens than the session workspace holds");
  if (seq >= s->batch) shape_fail("prefill: sequence out of range");
  if (pos > s->len[seq] || pos + n > s->capacity)
    shape_fail("prefill requires a resumable KV prefix within capacity");
  check_tokens(s->m, tokens, n);
  mdma_ctx *ctx = s->m->ctx;
  uint32_t *ids = reinterpret_cast<uint32_t *>(s->ids->ptr);
  hip_check(hipMemcpyAsync(ids, tokens, n * 4, hipMemcpyHostToDevice, ctx->stream), "prefill ids");
  embed_dev(s, ids, n);
  run_layers(s, n, pos, seq, false);
  s->len[seq] = pos + n;
}

template <class F>
int guarded(F &&f) {
  try {
    f();
    return MDMA_OK;
  } catch (const Error &e) {
    set_last_error(e.msg);
    return e.code;
  } catch (const std::bad_alloc &) {
    set_last_error("host allocation failed");
    return MDMA_ERR_OUT_OF_MEMORY;
  } catch (...) {
    set_last_error("unknown failure");
    return MDMA_ERR_BACKEND;
  }
}

}  // namespace

extern "C" {

int mdma_gfx950_model_load(mdma_ctx *ctx, const char *path, uint64_t budget_bytes, mdma_model **out) {
  return guarded([&] {
    if (!ctx || !path || !out) shape_fail("model_load: null argument");
    *out = nullptr;
    Gguf g;
    g.open(path);
    auto m = std::make_unique<mdma_model>();
    m->ctx = ctx;
    m->cfg = preflight(g);
    m->budget = budget_bytes;
    // Device bytes as allocated: Q4_K / Q6_K / Q8_0 matrices in the prepared
    // layout (rows padded to 16 bytes), every buffer rounded to 256 bytes.
    for (auto &kv : g.tensors) {
      const GgufTensor &t = kv.second;
      const uint64_t n = gfx950_layout_dtype(t.dtype) ? t.rows * gfx950_row_bytes(t.dtype, t.cols) : t.bytes;
      m->weight_bytes += (n + 255) / 256 * 256;
      if (kv.first != "token_embd.weight") m->tile_bytes += batch_tile_bytes(t.dtype, t.rows, t.cols);
    }
    reserve(m.get(), m->weight_bytes);  // Model::load_reserved: before any upload
    std::vector<uint8_t> tmp;
    m->token_embd = load_weight(m.get(), g, "token_embd.weight", tmp);
    m->layers.resize(m->cfg.n_layers);
    for (uint64_t i = 0; i < m->cfg.n_layers; i++) {
      const std::string p = "blk." + std::to_string(i) + ".";
      Layer &L = m->layers[i];
      L.attn_norm = load_norm(m.get(), g, p + "attn_norm.weight", tmp);
      L.wq = load_weight(m.get(), g, p + "attn_q.weight", tmp);
      L.wk = load_weight(m.get(), g, p + "attn_k.weight", tmp);
      L.wv = load_weight(m.get(), g, p + "attn_v.weight", tmp);
      L.wo = load_weight(m.get(), g, p + "attn_output.weight", tmp);
      L.ffn_norm = load_norm(m.get(), g, p + "ffn_norm.weight", tmp);
      L.gate = load_weight(m.get(), g, p + "ffn_gate.weight", tmp);
      L.up = load_weight(m.get(), g, p + "ffn_up.weight", tmp);
      L.down = load_weight(m.get(), g, p + "ffn_down.weight", tmp);
    }
    m->output_norm = load_norm(m.get(), g, "output_norm.weight", tmp);
    m->output = load_weight(m.get(), g, "output.weight", tmp);
    // RoPE angles for the whole context, built once.
    {
      std::lock_guard<std::recursive_mutex> lk(ctx->lock);
      rope_table(ctx, m->cfg.n_ctx - 1, m->cfg.head_dim, m->cfg.rope_theta);
    }
    *out = m.release();
  });
}

void mdma_gfx950_model_free(mdma_model *m) { delete m; }

int mdma_gfx950_model_config(const mdma_model *m, mdma_model_config *out) {
  return guarded([&] {
    if (!m || !out) shape_fail("model_config: null argument");
    *out = m->cfg;
  });
}

int mdma_gfx950_model_plan(const mdma_model *m, uint64_t capacity, uint64_t batch, uint64_t tokens,
                           mdma_memory_plan *out) {
  return guarded([&] {
    if (!m || !out) shape_fail("model_plan: null argument");
    if (!batch) batch = 1;
    mdma_memory_plan p{};
    p.weight_bytes = m->weight_bytes + (batch >= BATCH_MIN_TOKENS ? m->tile_bytes : 0);
    p.kv_bytes = kv_bytes(m->cfg, capacity, batch);
    p.workspace_bytes = workspace_bytes(m->cfg, tokens > batch ? tokens : batch, batch, capacity * batch);
    p.headroom_bytes = DEVICE_HEADROOM;
    p.total_bytes = p.weight_bytes + p.kv_bytes + p.workspace_bytes + p.headroom_bytes;
    p.device_bytes = m->ctx->total_bytes;
    uint64_t avail = 0;
    int st = mdma_gfx950_available_device_bytes(m->ctx, &avail);
    if (st) fail(st, mdma_gfx950_last_error());
    p.available_bytes = avail;
    // Positions that fit beside what this model already holds on the device.
    const uint64_t per_pos = kv_bytes(m->cfg, 1, batch) + 8 * batch;
    const uint64_t fixed = p.workspace_bytes + DEVICE_HEADROOM;
    p.max_context = avail > fixed ? (avail - fixed) / per_pos : 0;
    if (p.max_context > m->cfg.n_ctx) p.max_context = m->cfg.n_ctx;
    *out = p;
  });
}

int mdma_gfx950_session_new(mdma_model *m, uint64_t capacity, uint64_t batch, uint64_t max_tokens,
                            mdma_session **out) {
  return guarded([&] {
    if (!m || !out) shape_fail("session_new: null argument");
    *out = nullptr;
    if (!batch) shape_fail("session_new: batch must be positive");
    if (!capacity || capacity > m->cfg.n_ctx)
      throw Error{MDMA_ERR_CONTEXT_LIMIT, fmt("session capacity %llu must fit the %llu-token model context",
                                              (unsigned long long)capacity, (unsigned long long)m->cfg.n_ctx)};
    auto s = std::make_unique<mdma_session>();
    s->m = m;
    s->capacity = capacity;
    s->batch = batch;
    s->rows = max_tokens > batch ? max_tokens : batch;
    const mdma_model_config &c = m->cfg;
    const uint64_t n_ids = capacity * batch;
    const uint64_t bytes = kv_bytes(c, capacity, batch) + workspace_bytes(c, s->rows, batch, n_ids);
    // Batched sessions read the Q6_K matrices' tile images (reserved once
    // for the model; the images themselves follow at their first use).
    const uint64_t tiles = batch >= BATCH_MIN_TOKENS && !m->tiles_reserved ? m->tile_bytes : 0;
    std::lock_guard<std::recursive_mutex> lk(m->ctx->lock);
    reserve(m, bytes + tiles);
    s->reserved = bytes;
    if (batch >= BATCH_MIN_TOKENS) {
      m->tiles_reserved = true;
      m->ctx->batch_layout = true;
    }
    const uint64_t kvw = c.n_kv_heads * c.head_dim;
    for (uint64_t i = 0; i < c.n_layers; i++) {
      s->kc.push_back(alloc_or_throw(m->ctx, batch * capacity * kvw * 2, MDMA_POOL_KV, s->owned));
      s->vc.push_back(alloc_or_throw(m->ctx, batch * capacity * kvw * 2, MDMA_POOL_KV, s->owned));
    }
    const uint64_t R = s->rows;
    auto ws = [&](uint64_t b) { return alloc_or_throw(m->ctx, b, MDMA_POOL_SCRATCH, s->owned); };
    s->x = ws(R * c.n_embd * 4);
    s->x_alt = ws(R * c.n_embd * 4);
    s->normed = ws(R * c.n_embd * 4);
    s->q = ws(R * c.n_heads * c.head_dim * 4);
    s->k = ws(R * kvw * 4);
    s->v = ws(R * kvw * 4);
    s->attn_out = ws(R * c.n_heads * c.head_dim * 4);
    s->proj = ws(R * c.n_embd * 4);
    s->gate = ws(R * c.n_ff * 4);
    s->up = ws(R * c.n_ff * 4);
    s->act = ws(R * c.n_ff * 4);
    s->logits = ws(batch * c.vocab * 4);
    s->ids = ws(n_ids * 4);
    s->flags = ws(n_ids * 4);
    s->len.assign(batch, 0);
    *out = s.release();
  });
}

void mdma_gfx950_session_free(mdma_session *s) {
  if (!s) return;
  std::lock_guard<std::recursive_mutex> lk(s->m->ctx->lock);
  delete s;
}

int mdma_gfx950_session_reset(mdma_session *s) {
  return guarded([&] {
    if (!s) shape_fail("session_reset: null argument");
    s->len.assign(s->batch, 0);  // KvCache::set_len(0)
  });
}

int mdma_gfx950_prefill(mdma_session *s, uint64_t seq, const uint32_t *tokens, uint64_t n, uint32_t pos,
                        float *logits) {
  return guarded([&] {
    if (!s || (n && !tokens)) shape_fail("prefill: null argument");
    mdma_ctx *ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->lock);
    prefill_seq(s, seq, tokens, n, pos);
    // Model::prefill: only the last row goes through the output head.
    head(s, n - 1, 1, seq);
    if (logits) {
      hip_check(hipMemcpyAsync(logits, fp(s->logits) + seq * s->m->cfg.vocab, s->m->cfg.vocab * 4,
                               hipMemcpyDeviceToHost, ctx->stream), "prefill logits");
      hip_check(hipStreamSynchronize(ctx->stream), "prefill sync");
    }
    q8_invalidate(ctx);
  });
}

int mdma_gfx950_forward(mdma_session *s, uint64_t seq, uint32_t token, uint32_t pos, float *logits) {
  return guarded([&] {
    if (!s) shape_fail("forward: null argument");
    // Model::validate_decode (src/model.rs:338-353).
    if (token >= s->m->cfg.vocab || seq >= s->batch || pos >= s->capacity || pos > s->len[seq])
      shape_fail("decode requires a valid token and resumable KV prefix within capacity");
    mdma_ctx *ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->lock);
    uint32_t *ids = reinterpret_cast<uint32_t *>(s->ids->ptr);
    hip_check(hipMemcpyAsync(ids, &token, 4, hipMemcpyHostToDevice, ctx->stream), "forward id");
    embed_dev(s, ids, 1);
    run_layers(s, 1, pos, seq, false);
    s->len[seq] = pos + 1;
    head(s, 0, 1, seq);
    if (logits) {
      hip_check(hipMemcpyAsync(logits, fp(s->logits) + seq * s->m->cfg.vocab, s->m->cfg.vocab * 4,
                               hipMemcpyDeviceToHost, ctx->stream), "forward logits");
      hip_check(hipStreamSynchronize(ctx->stream), "forward sync");
    }
    q8_invalidate(ctx);
  });
}

}  // extern "C"

// The graph decode executor's state: the session's sequence, the device
// parameters [token, position] of the captured step, and its graph.
struct mdma_decoder {
  mdma_session *s = nullptr;
  uint64_t seq = 0;
  mdma_buf *params = nullptr;
  mdma_graph *graph = nullptr;
  bool replayed = false;
  ~mdma_decoder() {
    if (graph) {
      (void)hipStreamSynchronize(s->m->ctx->stream);  // a replay may still run
      mdma_gfx950_graph_destroy(graph);
    }
    if (params) mdma_gfx950_free(params);
  }
};

namespace {

// Captures step() on the context's stream into a graph (nullptr when the
// step cannot be captured, e.g. a buffer it needs would have to grow; the
// stream is back to eager launches either way).
mdma_graph *capture_step(mdma_ctx *ctx, const std::function<void()> &step) {
  if (mdma_gfx950_graph_begin(ctx)) return nullptr;
  bool ok = true;
  try {
    step();
  } catch (...) {
    ok = false;
  }
  mdma_graph *g = nullptr;
  if (mdma_gfx950_graph_end(ctx, &g) || !ok) {
    if (g) mdma_gfx950_graph_destroy(g);
    return nullptr;
  }
  return g;
}

}  // namespace

extern "C" {

int mdma_gfx950_decoder_new(mdma_session *s, uint64_t seq, mdma_decoder **out) {
  return guarded([&] {
    if (!s || !out) shape_fail("decoder_new: null argument");
    if (seq >= s->batch) shape_fail("decoder_new: no such sequence");
    auto d = std::make_unique<mdma_decoder>();
    d->s = s;
    d->seq = seq;
    int st = mdma_gfx950_alloc(s->m->ctx, 16, MDMA_POOL_SCRATCH, &d->params);
    if (st) fail(st, mdma_gfx950_last_error());
    *out = d.release();
  });
}

int mdma_gfx950_decoder_forward(mdma_decoder *d, uint32_t token, uint32_t pos, float *logits) {
  return guarded([&] {
    if (!d) shape_fail("decoder_forward: null argument");
    mdma_session *s = d->s;
    const uint64_t seq = d->seq;
    // Model::validate_decode (src/model.rs:338-353).
    if (token >= s->m->cfg.vocab || pos >= s->capacity || pos > s->len[seq])
      shape_fail("decode requires a valid token and resumable KV prefix within capacity");
    mdma_ctx *ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->lock);
    uint32_t *prm = reinterpret_cast<uint32_t *>(d->params->ptr);
    auto step = [&]() {
      embed_dev(s, prm, 1);
      run_layers(s, 1, 0, seq, false, prm + 1);
      head(s, 0, 1, seq);
    };
    const uint32_t vals[2] = {token, pos};
    launch_set_u32(ctx, prm, vals, 2);
    d->replayed = false;
    if (d->graph) {
      if (mdma_gfx950_graph_launch(ctx, d->graph) == 0) {
        d->replayed = true;
      } else {  // the context replaced a buffer the graph captured
        mdma_gfx950_graph_destroy(d->graph);
        d->graph = nullptr;
      }
    }
    if (!d->replayed) {
      step();  // eagerly: sizes every context buffer the step uses
      d->graph = capture_step(ctx, step);
    }
    s->len[seq] = pos + 1;
    q8_invalidate(ctx);
    if (logits) {
      hip_check(hipMemcpyAsync(logits, fp(s->logits) + seq * s->m->cfg.vocab, s->m->cfg.vocab * 4,
                               hipMemcpyDeviceToHost, ctx->stream), "decoder logits");
      hip_check(hipStreamSynchronize(ctx->stream), "decoder sync");
    }
  });
}

int mdma_gfx950_decoder_replayed(const mdma_decoder *d) { return d && d->replayed ? 1 : 0; }

void mdma_gfx950_decoder_free(mdma_decoder *d) { delete d; }

int mdma_gfx950_generate(mdma_session *s, const uint32_t *prompts, uint64_t n_prompt, uint64_t n_gen,
                         uint32_t *out_tokens, double *step_seconds) {
  return guarded([&] {
    if (!s || !prompts || !out_tokens) shape_fail("generate: null argument");
    const uint64_t B = s->batch;
    const mdma_model_config &c = s->m->cfg;
    // inference::generate_impl's ContextLimit (src/inference.rs:60-67).
    if (!n_prompt || !n_gen || n_prompt + n_gen > s->capacity || n_prompt > s->rows)
      throw Error{MDMA_ERR_CONTEXT_LIMIT, fmt("prompt of %llu tokens must fit the %llu-token session context with "
                                              "room for output", (unsigned long long)n_prompt,
                                              (unsigned long long)s->capacity)};
    check_tokens(s->m, prompts, n_prompt * B);
    mdma_ctx *ctx = s->m->ctx;
    std::lock_guard<std::recursive_mutex> lk(ctx->lock);
    uint32_t *tok = reinterpret_cast<uint32_t *>(s->ids->ptr) + n_prompt;  // after the prompt ids
    uint32_t *flag = reinterpret_cast<uint32_t *>(s->flags->ptr);
    if (n_prompt + n_gen * B > s->capacity * B) shape_fail("generate: token buffer too small");
    std::vector<hipEvent_t> ev(n_gen + 1);
    for (auto &e : ev) hip_check(hipEventCreate(&e), "event");
    struct Events {
      std::vector<hipEvent_t> &v;
      ~Events() {
        for (auto e : v) (void)hipEventDestroy(e);
      }
    } guard{ev};
    hip_check(hipEventRecord(ev[0], ctx->stream), "event");
    // Prefill every sequence, then its first greedy token.
    for (uint64_t b = 0; b < B; b++) {
      prefill_seq(s, b, prompts + b * n_prompt, n_prompt, 0);
      head(s, n_prompt - 1, 1, b);
    }
    launch_argmax_rows(ctx, fp(s->logits), B, c.vocab, tok, flag);
    hip_check(hipEventRecord(ev[1], ctx->stream), "event");
    if (ctx->graph_decode && n_gen > 2) {
      // Decode with one captured step, replayed (src/backend/rocm/graph.rs):
      // the step reads the position and its tokens from device memory and
      // ends by recording its tokens and advancing the position, so every
      // replay is the next step. Step 1 runs eagerly (it sizes the context's
      // buffers), then the graph runs steps 2.. (eagerly again if the step
      // cannot be captured).
      mdma_buf *gpb = alloc_or_throw(ctx, (2 + 2 * B) * 4, MDMA_POOL_SCRATCH, s->owned);
      struct Release {
        mdma_session *s;
        mdma_buf *b;
        ~Release() {
          s->owned.erase(std::find(s->owned.begin(), s->owned.end(), b));
          mdma_gfx950_free(b);
        }
      } release{s, gpb};
      uint32_t *gp = reinterpret_cast<uint32_t *>(gpb->ptr), *cur = gp + 2, *cur_flag = gp + 2 + B;
      hip_check(hipMemcpyAsync(cur, tok, B * 4, hipMemcpyDeviceToDevice, ctx->stream), "decode tokens");
      const uint32_t start[2] = {(uint32_t)n_prompt, 1u};
      launch_set_u32(ctx, gp, start, 2);
      auto step = [&]() {
        embed_dev(s, cur, B);
        run_layers(s, B, 0, 0, B > 1, gp);
        head(s, 0, B, 0);
        launch_argmax_rows(ctx, fp(s->logits), B, c.vocab, cur, cur_flag);
        launch_step_record(ctx, gp, cur, cur_flag, tok, flag, (uint32_t)B);
      };
      step();
      if (step_seconds) hip_check(hipEventRecord(ev[2], ctx->stream), "event");
      mdma_graph *g = capture_step(ctx, step);
      for (uint64_t i = 2; i < n_gen; i++) {
        if (!g) step();
        else if (mdma_gfx950_graph_launch(ctx, g)) fail(MDMA_ERR_BACKEND, "decode graph launch failed");
        if (step_seconds) hip_check(hipEventRecord(ev[i + 1], ctx->stream), "event");
      }
      if (g) {
        hip_check(hipStreamSynchronize(ctx->stream), "decode graph sync");
        mdma_gfx950_graph_destroy(g);
      }
    } else {
      // Decode: step i embeds the tokens of step i-1 straight from device memory.
      for (uint64_t i = 1; i < n_gen; i++) {
        const uint32_t pos = (uint32_t)(n_prompt + i - 1);
        embed_dev(s, tok + (i - 1) * B, B);
        if (B == 1)
          run_layers(s, 1, pos, 0, false);
        else
          run_layers(s, B, pos, 0, true);
        head(s, 0, B, 0);
        launch_argmax_rows(ctx, fp(s->logits), B, c.vocab, tok + i * B, flag + i * B);
        if (step_seconds) hip_check(hipEventRecord(ev[i + 1], ctx->stream), "event");
      }
    }
    for (uint64_t b = 0; b < B; b++) s->len[b] = n_prompt + n_gen - 1;
    std::vector<uint32_t> toks(n_gen * B), flags(n_gen * B);
    hip_check(hipMemcpyAsync(toks.data(), tok, n_gen * B * 4, hipMemcpyDeviceToHost, ctx->stream), "tokens");
    hip_check(hipMemcpyAsync(flags.data(), flag, n_gen * B * 4, hipMemcpyDeviceToHost, ctx->stream), "flags");
    hip_check(hipStreamSynchronize(ctx->stream), "generate sync");
    q8_invalidate(ctx);
    for (uint64_t i = 0; i < n_gen; i++)
      for (uint64_t b = 0; b < B; b++) {
        if (flags[i * B + b]) fail(MDMA_ERR_BACKEND, "empty or nonfinite logits");
        out_tokens[b * n_gen + i] = toks[i * B + b];
      }
    if (step_seconds) {
      for (uint64_t i = 0; i < n_gen; i++) {
        float ms = 0;
        hip_check(hipEventElapsedTime(&ms, ev[i], ev[i + 1]), "elapsed");
        step_seconds[i] = ms * 1e-3;
      }
    }
  });
}

}  // extern "C"
