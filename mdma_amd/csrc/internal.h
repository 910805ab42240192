// Internal declarations shared by the gfx950 backend's host and kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mdma_gfx950.h"

namespace mdma {

enum : int32_t { DT_F32 = 0, DT_F16 = 1, DT_Q8_0 = 8, DT_Q4_K = 12, DT_Q6_K = 14 };

inline uint64_t block_size(int32_t dt) {
  switch (dt) {
    case DT_F32: case DT_F16: return 1;
    case DT_Q8_0: return 32;
    case DT_Q4_K: case DT_Q6_K: return 256;
    default: return 0;
  }
}
inline uint64_t type_size(int32_t dt) {
  switch (dt) {
    case DT_F32: return 4;
    case DT_F16: return 2;
    case DT_Q8_0: return 34;
    case DT_Q4_K: return 144;
    case DT_Q6_K: return 210;
    default: return 0;
  }
}

// Status with message; thrown inside the library and turned into a status
// code at the C boundary.
struct Error {
  int code;
  std::string msg;
};
[[noreturn]] void fail(int code, const std::string &msg);
[[noreturn]] inline void shape_fail(const std::string &msg) { fail(MDMA_ERR_SHAPE_MISMATCH, msg); }
void hip_check(hipError_t e, const char *what);
// The thread-local message mdma_gfx950_last_error() returns.
void set_last_error(const std::string &msg);

// One domain of a BufferBudget (src/memory/buffers.rs:32-99): requested
// bytes of live buffers against an optional quota.
struct Ledger {
  uint64_t used = 0;
  uint64_t limit = UINT64_MAX;
};

}  // namespace mdma

struct mdma_buf {
  mdma_ctx *ctx = nullptr;
  char *ptr = nullptr;     // device address of element 0
  uint64_t len = 0;        // bytes visible to ops
  uint64_t charged = 0;    // bytes charged to the device budget (0 for views)
  int pool = MDMA_POOL_SCRATCH;
  int layout = MDMA_LAYOUT_GGUF;
  bool owner = true;       // false for views
  // Weight bytes from the trait-shaped upload_weight: raw GGUF blocks whose
  // dtype and shape the first op that reads them supplies; that op repacks
  // them into the prepared layout (see prepare_weight).
  bool repack_pending = false;
  // A Q6_K weight's tile images for the batch GEMV (gemv_batch.hip), made
  // at its first batch call when the context's batch layout is on; freed
  // with the buffer or when its bytes are written again.
  char *tile = nullptr;
  uint64_t tile_charged = 0;
  bool tile_stale = false;  // its bytes were written since (set aside under capture)
};

struct mdma_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::recursive_mutex lock;
  mdma::Ledger budget[2];  // MDMA_DOMAIN_DEVICE, MDMA_DOMAIN_HOST
  int act_mode = MDMA_ACT_F32;
  bool norm_fusion = true;  // one-token int8 decode: attention rmsnorm fused into the GEMVs around it
  bool batch_layout = false;  // mdma_gfx950_set_batch_layout
  std::vector<mdma_buf *> tiled;  // buffers holding tile images
  std::string label;
  uint64_t total_bytes = 0;
  int cu_count = 0;
  // Scratch owned by the context (int8 activations, partial sums, RoPE tables).
  char *scratch = nullptr;
  uint64_t scratch_cap = 0;
  // int8 activations of the last quantized x (int8 mode), reused while valid.
  char *q8 = nullptr;
  uint64_t q8_cap = 0;
  bool q8_valid = false;
  const float *q8_x = nullptr;
  uint64_t q8_n = 0, q8_n_in = 0;
  // The f16-path GEMM's input for x [a16_n / a16_n_in, a16_n_in], written by
  // a fused prefill rmsnorm into a16_buf (a caller's buffer), while valid.
  // a16_p: with the Q4_K min term's P halves and row exponents.
  bool a16_valid = false, a16_p = false;
  const float *a16_x = nullptr;
  char *a16_buf = nullptr;
  uint64_t a16_n = 0, a16_n_in = 0;
  // A request to the gated prefill GEMM producing a16_want_y: also write
  // its output's input for a Q6_K GEMM into a16_want_buf (and record it).
  const float *a16_want_y = nullptr;
  char *a16_want_buf = nullptr;
  uint64_t a16_want_bytes = 0;
  // With the request: the caller reads a16_want_y only through that input,
  // so its f32 rows are not stored (a16_noy marks such a record).
  bool a16_want_input_only = false, a16_noy = false;
  // A request to the fused QKV GEMM of a prompt writing q into rope_want_q:
  // RoPE on q and k and the k / v cache rows in its epilogue (rope_done set
  // when a launch took it).
  const float *rope_want_q = nullptr;
  const float *rope_want_tab = nullptr;
  uint16_t *rope_want_dk = nullptr, *rope_want_dv = nullptr;
  uint32_t rope_want_pos = 0, rope_want_hd = 0;
  uint64_t rope_want_stride = 0;
  bool rope_done = false;
  // Device RoPE cos/sin table: [positions][head_dim/2] for one (head_dim, theta).
  float *rope_tab = nullptr;
  uint64_t rope_bytes = 0;
  uint64_t rope_positions = 0, rope_hd = 0;
  float rope_theta = 0.f;
  uint32_t *host_ids = nullptr;  // pinned staging for token ids / argmax result
  uint64_t host_ids_cap = 0;
  bool capturing = false;        // stream capture in progress: no synchronizing calls
  int prefill_kernel = MDMA_PREFILL_AUTO;  // mdma_gfx950_set_prefill_kernel
  int batch_kernel = MDMA_BATCH_AUTO;      // mdma_gfx950_set_batch_kernel
  bool graph_decode = true;                // mdma_gfx950_set_graph_decode
  // Block-dot capture (mdma_gfx950_capture_block_dots): int32 slots or null.
  int32_t *dots = nullptr;
  uint64_t dots_cap = 0;
  // Events the next GEMV kernel's dispatch timestamps (mdma_gfx950_time_next_gemv).
  hipEvent_t time_start = nullptr, time_stop = nullptr;
  // Per-chunk partial results of the two-pass argmax (12 bytes per chunk).
  char *argmax_part = nullptr;
  uint64_t argmax_part_cap = 0;  // chunks
  uint32_t *attn_cnt = nullptr;
  uint64_t attn_cnt_cap = 0;
  uint32_t *gemm_cnt = nullptr;  // split-K GEMM arrival counters (zero between launches)
  uint64_t gemm_cnt_cap = 0;
  double *ssq = nullptr;  // per-workgroup sums of squares of a residual-stream GEMV (norm fusion)
  uint64_t ssq_cap = 0;
  uint32_t team_grid = 0;  // workgroups of the last row-team launch
  // Bumped whenever a context buffer a captured graph may point into is
  // freed or replaced (scratch, int8 activations, counters, partials, RoPE
  // table); a graph captured under another epoch refuses to replay.
  uint64_t buf_epoch = 0;
  // Graph replay parameters (mdma_gfx950_set_replay_params): device words
  // [token, position] the trait-level decode ops read, and the KV capacity
  // their launches are sized for; null when not set.
  const uint32_t *replay = nullptr;
  uint64_t replay_cap = 0;
  // This device's copy of the library's static scratch array (noalloc.hip),
  // from hipGetSymbolAddress at create.
  char *static_scratch = nullptr;
  // Set only for the duration of an allocation-free call: the int8
  // activations and GEMM inputs go to this fixed buffer, and any growth of
  // a context buffer fails instead of allocating.
  char *fixed_scratch = nullptr;
  uint64_t fixed_cap = 0;
};

struct mdma_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  mdma_ctx *ctx = nullptr;
  uint64_t epoch = 0;  // the context's buf_epoch at capture
};

namespace mdma {

// Backend::qmatmul with its shape rules, in activation mode `mode` (-1: the
// context's); throws Error. The lock is taken inside.
void qmatmul_run(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y, int mode);
// Charge / refund requested bytes to a budget domain of the context
// (MDMA_ERR_BUFFER_BUDGET past its quota).
void budget_charge(mdma_ctx *ctx, int domain, uint64_t bytes, const char *what);
void budget_refund(mdma_ctx *ctx, int domain, uint64_t bytes);
// A weight uploaded through the trait-shaped upload_weight holds raw GGUF
// blocks until the first op that reads it with a Q4_K / Q6_K / Q8_0 QWeight
// of matching size: that op repacks it on the device into the prepared
// layout (a new buffer in place of the raw one). Under graph capture or in
// an allocation-free call, or when the budget has no room, the weight stays
// raw for now and the raw-layout kernels read it.
void prepare_weight(mdma_ctx *ctx, const mdma_qweight *w);
// Device repack of raw GGUF rows into the prepared layout (layout.cpp).
void launch_repack(mdma_ctx *ctx, int32_t dtype, uint64_t rows, uint64_t cols, const uint8_t *src, uint8_t *dst);
// Per-device set-up of the allocation-free entry point (noalloc.hip): the
// device address of this device's static scratch, kept in ctx.
void noalloc_setup(mdma_ctx *ctx);
// Bytes of int8 activation slots (per-256 scales, sums of 16) for n values.
uint64_t q8_slot_bytes(uint64_t n);
// Bytes of the prefill GEMM's per-32 activations for n values (unsplit).
uint64_t gemm_input_bytes(uint64_t n);

// Scratch space of at least `bytes` on the context's device; growing it
// synchronizes the stream (callers hold the context lock).
char *scratch(mdma_ctx *ctx, uint64_t bytes);
// The int8-activation buffer (grown like scratch; growth drops the cached x).
char *q8_buffer(mdma_ctx *ctx, uint64_t bytes);
// Device space for `chunks` partial results of the two-pass argmax (grown
// like scratch).
char *argmax_parts(mdma_ctx *ctx, uint64_t chunks);
// Arrival counters that workgroups of one launch update concurrently sit one
// per CNT_STRIDE entries (256 bytes): device-scope atomics on one cache line
// are served one at a time, so counters sharing a line would serialize the
// arrivals of unrelated workgroups.
constexpr uint32_t CNT_STRIDE = 64;
// Zeroed arrival counters for split attention, n counters at CNT_STRIDE
// apart; each launch leaves the counters it used at zero.
uint32_t *attn_counters(mdma_ctx *ctx, uint64_t n);
// Split-K GEMM arrival counters (n at CNT_STRIDE apart), zeroed at allocation
// (each launch leaves them zero); nullptr when n exceeds what is allocated
// during stream capture.
uint32_t *gemm_counters(mdma_ctx *ctx, uint64_t n);
// Forget the cached int8 activations: every entry point that writes device
// memory calls this (a qmatmul only when its output overlaps the cached x).
inline void q8_invalidate(mdma_ctx *ctx) { ctx->q8_valid = ctx->a16_valid = false; }
void q8_invalidate_range(mdma_ctx *ctx, const void *p, uint64_t bytes);
// Device pointer to a cos/sin table covering positions [0, max_pos] for (hd, theta).
const float *rope_table(mdma_ctx *ctx, uint64_t max_pos, uint64_t hd, float theta);

// ---- kernel launchers (gemv.hip / quant.hip / ops.hip) ----
struct GemvJob {
  int32_t dtype;
  const uint8_t *w;
  uint64_t n_out, n_in;
  float *y;        // [T, n_out], row stride n_out
  int layout = MDMA_LAYOUT_GGUF;  // MDMA_LAYOUT_GFX950: prepared rows (layout.cpp)
  // Block-dot capture (mdma_gfx950_capture_block_dots): when set, the int8
  // kernels over prepared rows also store every int32 sub-block dot they
  // form, dots[(t * n_out + row) * n_sub + s] (n_sub = n_in / 16 for Q6_K,
  // n_in / 32 otherwise); the f16-path GEMM stores its block dot times the
  // Q4_K sub-block scale, the integer it forms.
  int32_t *dots = nullptr;
  // The weight's buffer (for its batch tile images), or null.
  mdma_buf *src = nullptr;
};
// Sub-blocks per row in the block-dot capture layout.
inline uint64_t dot_subs(int32_t dtype, uint64_t n_in) { return dtype == DT_Q6_K ? n_in / 16 : n_in / 32; }

// ---- prepared weight layout (layout.cpp) ----
// Bytes of one prepared row (0 if cols is not whole blocks).
uint64_t gfx950_row_bytes(int32_t dtype, uint64_t cols);
bool gfx950_layout_dtype(int32_t dtype);
void pack_gfx950(int32_t dtype, uint64_t rows, uint64_t cols, const uint8_t *src, uint8_t *dst);
void unpack_gfx950(int32_t dtype, uint64_t rows, uint64_t cols, const uint8_t *src, uint8_t *dst);
// f32-activation GEMV for up to 3 independent weights sharing x (fused QKV).
void launch_gemv_f32(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t T);
// gate/up fused with SiLU: y = silu(gate x) * (up x); f32 activations.
void launch_gemv_f32_gated(mdma_ctx *ctx, const GemvJob &gate, const GemvJob &up, const float *x,
                           uint64_t T, float *y);
// int8 mode: quantize x per 256 then integer dots; same job conventions.
void launch_gemv_i8(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t T);
void launch_gemv_i8_gated(mdma_ctx *ctx, const GemvJob &gate, const GemvJob &up, const float *x,
                          uint64_t T, float *y);
// Row-team GEMV over prepared layouts (gemv_team.hip): whether the jobs can
// share one launch (all prepared, same dtype and n_in), and the launch in
// mode MDMA_ACT_F32 or MDMA_ACT_I8 (I8 needs n_in % 256 == 0). Gated: jobs =
// {gate, up}, output silu(gate x) * (up x) into ygated.
bool team_layout_ok(const GemvJob *jobs, int n_jobs);
// One token, int8 mode, prepared Q4_K / Q6_K rows: the GEMV quantizes f32 x
// itself in its prologue (per 256, as launch_quantize_act, bit for bit) --
// one launch instead of two. False (nothing launched) where that variant is
// not available or not faster (rows of at most 4096 columns, fewer than
// 65536 rows).
bool launch_gemv_i8_x(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, bool gated, const float *x, float *ygated);

// Batched decode (2..16 tokens, int8 mode) on the matrix cores for prepared
// Q4_K / Q6_K / Q8_0 rows of whole 256-column groups (gemv_batch.hip).
bool gemv_batch_ok(const GemvJob *jobs, int n_jobs, uint64_t T);
void launch_gemv_batch(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, bool gated, const float *x, uint64_t T,
                       float *ygated);
// Tokens from which int8-mode GEMVs of prepared rows go to the batch kernel.
constexpr uint64_t BATCH_MIN_TOKENS = 3;
// The batch kernel's tile images of a prepared weight (Q6_K, rows of whole
// 512-column pairs; 0 bytes otherwise), the kernel that writes them, and
// the job's images (made now when the context's batch layout is on and the
// call may allocate; null if the job has none).
uint64_t batch_tile_bytes(int32_t dtype, uint64_t n_out, uint64_t n_in);
void launch_tile_repack(mdma_ctx *ctx, int32_t dtype, uint64_t n_out, uint64_t n_in, const uint8_t *w, uint8_t *out);
const uint8_t *batch_tile(mdma_ctx *ctx, const GemvJob &job);
// Frees the tile images of every buffer whose bytes overlap [p, p + bytes).
void drop_tiles(mdma_ctx *ctx, const void *p, uint64_t bytes);
void free_tile(mdma_ctx *ctx, mdma_buf *b);
// pro: one token in the int8 mode, x quantized by the GEMV's prologue.
// The rmsnorm of a Llama layer's residual stream fused into the GEMVs on
// either side of it (one token, int8 mode): res/ssq for the GEMV that
// produces the stream (it stores y = res + W x and per-workgroup sums of
// squares of y), nsum/nw/npart/n_part/eps for the GEMV that reads the norm
// (its x = rmsnorm(nsum) * nw, quantized in its prologue).
struct TeamNorm {
  const float *res = nullptr;
  double *ssq = nullptr;
  uint32_t ssq_cap = 0;  // partials ssq holds: a launch of more workgroups is not made
  const float *nsum = nullptr, *nw = nullptr;
  const double *npart = nullptr;
  uint32_t n_part = 0;
  float eps = 0.f;
};
void launch_gemv_team(mdma_ctx *ctx, int mode, const GemvJob *jobs, int n_jobs, bool gated, const float *x,
                      uint64_t T, float *ygated, bool pro = false, const TeamNorm *nm = nullptr);
// Space for n per-workgroup sums of squares (grown outside capture).
double *ssq_parts(mdma_ctx *ctx, uint64_t n);
// One token, int8 mode: y = res + W x for one prepared weight, leaving the
// workgroups' sums of squares of y in ssq_parts; returns how many (0: not
// done, nothing launched).
uint32_t launch_gemv_i8_residual(mdma_ctx *ctx, const GemvJob &job, const float *x, const float *res);
// One token, int8 mode: the jobs (one-wave rows, whole 256-column groups)
// over x = rmsnorm(nsum) * nw, the sum of squares of nsum being the n_part
// partials in ssq_parts; false (nothing launched) when the shape does not
// allow it.
bool launch_gemv_i8_normed(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *nsum, const float *nw,
                           uint32_t n_part, float eps);
// The int8 activations of x [T, n_in] (per-256 f32 scales, per-16 sums) in
// the context's activation buffer, quantized now unless it already holds
// exactly this x.
// Slots of the int8-activation buffer for x [T, n_in] (int8 values, per-256
// scales, sums of 16), and marking them as holding x's quantization.
void q8_slots(mdma_ctx *ctx, uint64_t T, uint64_t n_in, int8_t **qx, float **dx, int32_t **s16);
void q8_mark(mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in);
// The buffer holds the int8 form of the one row x of n values.
bool q8_holds(mdma_ctx *ctx, const float *x, uint64_t n);
void quantize_into_scratch(mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in, int8_t **qx, float **dx,
                           int32_t **s16);
// Prefill int8 MFMA GEMM (gemm_i8.hip) over prepared Q8_0 / Q4_K / Q6_K
// weights: whether it covers (dtype, layout, n_in, n_out); the split-K
// partial storage (doubles) and counters a launch for M tokens asks for
// (zero when it runs unsplit); and the launch with activations quantized per
// 32 (qx [M, K], sx [M, K/32], s16 [M, K/16]). With part or cnt null, or
// smaller than asked, the launch runs unsplit.
bool gemm_i8_supported(int32_t dtype, int layout, uint64_t n_in, uint64_t n_out);
void gemm_i8_split_need(const mdma_ctx *ctx, const GemvJob &w, uint64_t M, uint64_t *part_doubles,
                        uint64_t *counters);
void launch_gemm_i8(mdma_ctx *ctx, const GemvJob &w, const int8_t *qx, const float *sx, const int32_t *s16,
                    uint64_t M, float *y, double *part, uint64_t part_doubles, uint32_t *cnt, uint64_t counters);
// Token count from which the int8 mode runs the MFMA GEMM instead of the
// GEMV (activations per 32 instead of per 256). Below it the batch GEMV takes
// up to 16 tokens per launch: on the MI355X at Llama-3-8B shapes the GEMMs
// cost about the same at 16 as at 64 tokens (gate/up 170 us, 14336x4096
// Q4_K 86 us, 4096x14336 Q6_K 60 us) against 18.5, 12.0 and 18.3 us for 16
// tokens of the batch GEMV; at 64 tokens the four batch launches of the
// 4096x14336 Q6_K match its GEMM.
constexpr uint64_t GEMM_MIN_TOKENS = 64;
// Prefill GEMM on the f16 matrix path (gemm_f16.hip): the same per-32 int8
// activations, carried as exact f16 integers with the Q4_K weights' 6-bit
// sub-scales folded into the weight operand. Whether it covers (dtype,
// layout, n_in, n_out); the scratch bytes its inputs take for M tokens; the
// launch (quantization prologue, then each job's GEMM) with that scratch.
bool gemm_f16_supported(int32_t dtype, int layout, uint64_t n_in, uint64_t n_out);
uint64_t gemm_f16_input_bytes(uint64_t M, uint64_t K);
// The input's parts in gemm_f16_input_bytes(M, K) bytes at s: the int8
// values as f16 [M, K], per-32 scales [M, K/32], P's f16 halves [M, K/32]
// each, and each row's 2^-e [M].
struct F16In {
  _Float16 *xh;
  float *sx;
  _Float16 *ph, *pl;
  float *inv;
};
F16In gemm_f16_input_at(char *s, uint64_t M, uint64_t K);
// The context's record of a fused rmsnorm's f16-path GEMM input for x, and
// whether it holds x [T, n_in].
void a16_mark(mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in, char *buf, bool with_p);
bool a16_holds(const mdma_ctx *ctx, const float *x, uint64_t T, uint64_t n_in);
// Split-K partials the f16-path launches of these jobs over M tokens take
// (bytes; 0 = unsplit) and the arrival counters they need (*tiles).
uint64_t gemm_f16_split_bytes(const mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, uint64_t M, uint64_t *tiles);
// glu_y: jobs are (gate, up) passing gemm_f16_glu_ok; one gated launch
// writes silu(gate) * up to glu_y (the jobs' own outputs are not written).
bool gemm_f16_glu_ok(const GemvJob &gate, const GemvJob &up);
// have_input: scratch already holds x's input (gemm_f16_input_at), so the
// quantization prologue is not launched.
void launch_gemm_f16(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *x, uint64_t M, char *scratch,
                     float *part, uint64_t part_bytes, uint32_t *cnt, uint64_t counters, float *glu_y = nullptr,
                     bool have_input = false);
void launch_quantize_act(mdma_ctx *ctx, const float *x, uint64_t n, uint64_t group, int8_t *q,
                         float *d, int32_t *sum16);
void launch_block_dot(mdma_ctx *ctx, const GemvJob &w, const int8_t *qx, uint64_t T, int32_t *out);
void launch_block_dot_prepared(mdma_ctx *ctx, const GemvJob &w, const int8_t *qx, uint64_t T, int32_t *out);

void launch_embed(mdma_ctx *ctx, int32_t dtype, int layout, const uint8_t *table, uint64_t n_embd,
                  const uint32_t *ids_dev, uint64_t n_ids, float *out);
void launch_rmsnorm(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b,
                    float *sum, float *y, uint64_t rows, float eps);
// rmsnorm that also leaves y's int8 per-256 quantization in the
// int8-activation buffer, marked as holding y (so the int8 GEMV that reads y
// next does not quantize it again). False, launching nothing, when dim is not
// whole groups of 256 or exceeds 16384.
bool launch_rmsnorm_q8(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                       float *y, uint64_t rows, float eps);
// rmsnorm that also writes the f16-path GEMM's input for y (the bits its
// quantization prologue would write) into buf and records it, so the GEMM
// that reads y next skips that prologue. False, launching nothing, when dim
// is not whole blocks of 32, exceeds 16384, or buf is smaller than
// gemm_f16_input_bytes(rows, dim).
bool launch_rmsnorm_a16(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                        float *y, uint64_t rows, float eps, char *buf, uint64_t buf_bytes);
void launch_add(mdma_ctx *ctx, const float *a, const float *b, float *y, uint64_t n);
void launch_silu_mul(mdma_ctx *ctx, const float *g, const float *u, float *y, uint64_t n);
// pos_dev (a captured decode step, one position): the position is read from
// device memory when the kernel runs, pos is not used, and kv_write's and
// rope_kv_write's rows go to that position's row of dk / dv (which then
// point at the cache's position 0).
void launch_rope(mdma_ctx *ctx, float *x, uint64_t n_tokens, uint64_t heads, uint64_t hd,
                 const float *tab, uint32_t pos, const uint32_t *pos_dev = nullptr);
void launch_kv_write(mdma_ctx *ctx, const float *k, const float *v, uint16_t *dk, uint16_t *dv,
                     uint64_t n, const uint32_t *pos_dev = nullptr);
// kv_stride: elements between consecutive tokens' cache rows (0 = kv_heads*hd,
// contiguous); pos_step: position increment per token (1 in a sequence, 0
// across the sequences of a decode batch).
void launch_rope_kv_write(mdma_ctx *ctx, float *q, uint64_t q_heads, const float *k,
                          const float *v, uint64_t kv_heads, uint64_t hd, uint64_t n_tokens,
                          const float *tab, uint32_t pos, uint16_t *dk, uint16_t *dv,
                          uint64_t kv_stride = 0, uint32_t pos_step = 1, const uint32_t *pos_dev = nullptr);
// seq_stride 0: causal over one sequence. Otherwise query i is sequence i's
// single decode query over its own cache at k + i*seq_stride, kv_len keys.
// pos_dev (a captured decode step, one query per sequence): the position is
// read from device memory when the kernel runs and kv_len is the cache
// capacity the launch is sized for; the results equal a launch with that
// position as the last key, bit for bit.
void launch_attn(mdma_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v, float *o,
                 uint64_t n_q, uint64_t kv_len, uint64_t hd, uint64_t n_q_heads,
                 uint64_t n_kv_heads, uint64_t seq_stride = 0, const uint32_t *pos_dev = nullptr);
// The CPU-order mode (cpu_order.hip): the CPU backend's arithmetic order,
// bit for bit. qmatmul of one job (any layout of Q4_K / Q6_K / Q8_0, or F32
// / F16 rows); rmsnorm with the optional residual add (b, sum nullable);
// silu_mul; causal GQA attention (seq_stride and pos_dev as launch_attn /
// launch_attn_rope; kv_len is then the cache capacity).
void launch_gemv_seq(mdma_ctx *ctx, const GemvJob &j, const float *x, uint64_t T);
void launch_rmsnorm_seq(mdma_ctx *ctx, const float *w, uint64_t dim, const float *a, const float *b, float *sum,
                        float *y, uint64_t rows, float eps);
void launch_silu_mul_seq(mdma_ctx *ctx, const float *g, const float *u, float *y, uint64_t n);
void launch_attn_seq(mdma_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t n_q,
                     uint64_t kv_len, uint64_t hd, uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride = 0,
                     const uint32_t *pos_dev = nullptr);
// Greedy argmax of each row of x [rows, n] into idx[row]; flag[row] = any non-finite.
// launch_attn that also leaves the int8 form of o (per 256) in the
// int8-activation buffer, marked as holding o. False, launching nothing, when
// the shape has no such variant (needs hd % 8 == 0, hd <= 256, a power-of-two
// group of at most 8 query heads per KV head, group outputs whole 256s).
bool launch_attn_q8(mdma_ctx *ctx, const float *q, const uint16_t *k, const uint16_t *v, float *o, uint64_t n_q,
                    uint64_t kv_len, uint64_t hd, uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride = 0,
                    const uint32_t *pos_dev = nullptr);
// Decode attention with launch_rope_kv_write folded in: q, k, v are the
// unrotated projections of n_q queries, each the single new token of its
// sequence (seq_stride apart in kc / vc; or one query over one sequence,
// seq_stride 0), all at rope position pos = kv_len - 1. The rotated key and
// the value are written to the caches at that position, with the values
// launch_rope_kv_write writes. int8_out: as launch_attn_q8. False, launching
// nothing, when the shape has no such variant. pos_dev (a captured decode
// step): the kernel reads the position from device memory instead, and
// kv_len is the cache capacity the launch is sized for; the results equal a
// launch with that position and kv_len = position + 1, bit for bit.
bool launch_attn_rope(mdma_ctx *ctx, const float *q, const float *k, const float *v, const float *tab, uint32_t pos,
                      uint16_t *kc, uint16_t *vc, float *o, uint64_t n_q, uint64_t kv_len, uint64_t hd,
                      uint64_t n_q_heads, uint64_t n_kv_heads, uint64_t seq_stride, bool int8_out,
                      const uint32_t *pos_dev = nullptr);
// A captured decode step's device parameters: p[0..n) = vals (one thread).
void launch_set_u32(mdma_ctx *ctx, uint32_t *p, const uint32_t *vals, int n);
// After a captured generate step: hist[step * B + b] = cur[b] and
// hist_flag[...] = cur_flag[b] for the step in params[1]; then the position
// params[0] and step params[1] advance by one.
void launch_step_record(mdma_ctx *ctx, uint32_t *params, const uint32_t *cur, const uint32_t *cur_flag,
                        uint32_t *hist, uint32_t *hist_flag, uint32_t B);
void launch_argmax_rows(mdma_ctx *ctx, const float *x, uint64_t rows, uint64_t n, uint32_t *idx,
                        uint32_t *flag);

}  // namespace mdma
