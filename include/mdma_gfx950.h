/*
 * mdma_gfx950 — MI355X (gfx950, CDNA4) backend for mdma's quantized-weight path.
 *
 * A C ABI that carries the reference's `trait Backend`
 * (/root/reference/src/backend.rs:190-601) one method per entry point, so a
 * Rust `impl Backend for Gfx950Backend` can wrap it without glue logic.
 * Citations are path:line inside the reference checkout.
 *
 * Conventions
 *  - Every entry point returns an mdma_status; on failure the message is
 *    readable from mdma_gfx950_last_error() on the same thread.
 *  - Buffers are opaque handles owned by the caller and sized in bytes; a
 *    buffer's length defines the shape an op infers (token counts come from
 *    x's length, as src/backend/shape.rs does). Inputs must be whole rows;
 *    outputs only need to be large enough and are never written past the
 *    result (src/backend/shape.rs:1-10).
 *  - Kernels run asynchronously in stream order on one non-blocking stream
 *    per context; upload/download synchronize before returning
 *    (src/backend/rocm.rs:543-599). The context is internally locked.
 *  - Weight dtypes use GGML type ids: F32 0, F16 1, Q8_0 8, Q4_K 12, Q6_K 14.
 */
#ifndef MDMA_GFX950_H
#define MDMA_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* backend::Error variants, src/backend.rs:52-93, in declaration order. */
typedef enum {
    MDMA_OK = 0,
    MDMA_ERR_CONTEXT_LIMIT = 1,
    MDMA_ERR_SHAPE_MISMATCH = 2,
    MDMA_ERR_NOT_IMPLEMENTED = 3,
    MDMA_ERR_UNSUPPORTED_MODEL = 4,
    MDMA_ERR_MEMORY_BUDGET = 5,
    MDMA_ERR_BUFFER_BUDGET = 6,
    MDMA_ERR_INSUFFICIENT_MEMORY = 7,
    MDMA_ERR_OUT_OF_MEMORY = 8,
    MDMA_ERR_SIZE_OVERFLOW = 9,
    MDMA_ERR_BACKEND = 10,
    MDMA_ERR_IO = 11
} mdma_status;

/* Pool, src/backend.rs:108-113. */
typedef enum { MDMA_POOL_WEIGHTS = 0, MDMA_POOL_KV = 1, MDMA_POOL_SCRATCH = 2 } mdma_pool;

/* WeightLayout (src/cache/layout.rs:10-38): raw GGUF blocks, or this
 * backend's prepared layout (MDMA_LAYOUT_GFX950): Q4_K / Q6_K / Q8_0 rows
 * rearranged losslessly into 16-byte planes indexed by the 64-column unit
 * (32 for Q8_0) a lane owns, so every wave load reads 1 KiB of contiguous
 * memory. Each block keeps its byte count; rows are padded to 16 bytes. */
typedef enum { MDMA_LAYOUT_GGUF = 0, MDMA_LAYOUT_GFX950 = 1, MDMA_LAYOUT_ROCM_Q4K_V3 = 2 } mdma_layout;

/* MemoryDomain (src/memory/buffers.rs:5-10): the two ledgers of a BufferBudget. */
typedef enum { MDMA_DOMAIN_DEVICE = 0, MDMA_DOMAIN_HOST = 1 } mdma_memory_domain;

/* Activation mode of the quantized matmuls and the ops around them:
 *  - MDMA_ACT_F32: f32 activations; every output the dot product rounded once
 *    to f32 (closer to exact than the CPU's sequential sum);
 *  - MDMA_ACT_I8: int8 activations quantized per 256 (decode) or per 32
 *    (prefill GEMM) with an f32 scale;
 *  - MDMA_ACT_F32_CPU: f32 activations in the CPU backend's arithmetic
 *    order, bit-identical to it: each qmatmul output the sequential f32 sum,
 *    from -0.0, of f32-rounded products of the dequantized row
 *    (CpuBackend::qmatmul, src/backend/cpu.rs:46-48,335-368), and rmsnorm,
 *    add_rmsnorm, silu_mul, ffn_gate_up and attn in the CPU's order with the
 *    C library's expf (cpu.rs:50-60,388-402,447-458,530-590). A parity mode:
 *    its sums are sequential chains, one lane per output row.
 * The reference's counterpart is the MDMA_HIP_F32 switch
 * (src/backend/select.rs:49). */
typedef enum { MDMA_ACT_F32 = 0, MDMA_ACT_I8 = 1, MDMA_ACT_F32_CPU = 2 } mdma_act_mode;

typedef struct mdma_ctx mdma_ctx;
typedef struct mdma_buf mdma_buf;

/* QWeight (src/backend.rs:114-118): dtype + rank-2 shape [rows=n_out, cols=n_in]. */
typedef struct {
    int32_t dtype;
    uint64_t rows;
    uint64_t cols;
    const mdma_buf *buf;
} mdma_qweight;

/* RopeSpec (src/backend.rs:120-123). */
typedef struct {
    uint64_t head_dim;
    float theta;
} mdma_rope_spec;

/* AttnSpec (src/backend.rs:132-137). */
typedef struct {
    uint64_t head_dim;
    uint64_t n_q_heads;
    uint64_t n_kv_heads;
} mdma_attn_spec;

/* KvView (src/backend.rs:125-129). */
typedef struct {
    const mdma_buf *k;
    const mdma_buf *v;
    uint64_t len;
} mdma_kv_view;

/* ---- lifecycle and capability queries ---- */

/* HipBackend::new / create (src/backend/rocm.rs:165-223). */
int mdma_gfx950_create(int device, mdma_ctx **out);
void mdma_gfx950_destroy(mdma_ctx *ctx);
/* Thread-local message of the last failed call on this thread. */
const char *mdma_gfx950_last_error(void);
/* Backend::device_label (src/backend.rs:206). */
int mdma_gfx950_device_label(mdma_ctx *ctx, char *out, size_t cap);
/* Backend::total_device_bytes (:219) / available_device_bytes (:214). */
uint64_t mdma_gfx950_total_device_bytes(mdma_ctx *ctx);
int mdma_gfx950_available_device_bytes(mdma_ctx *ctx, uint64_t *out);
/* Backend::supports_weight_dtype (:363). Q8_0, Q4_K, Q6_K, F32 and F16. */
int mdma_gfx950_supports_weight_dtype(mdma_ctx *ctx, int32_t dtype);
/* Backend::max_head_dim (:368). */
uint64_t mdma_gfx950_max_head_dim(mdma_ctx *ctx);
/* Backend::kv_elem_bytes (:427): 2, the cache stores f16. */
uint64_t mdma_gfx950_kv_elem_bytes(mdma_ctx *ctx);
/* Backend::join_execution (:197): wait for all queued device work. */
int mdma_gfx950_join_execution(mdma_ctx *ctx);
/* Backend::set_buffer_budget (:352) with a BufferBudget (src/memory/buffers.rs:32-99):
 * quotas for the device and host domains, UINT64_MAX for none (BufferBudget::new's
 * None), 0 to forbid a domain. Installed only while nothing is charged to the
 * context's ledger (MDMA_ERR_BACKEND otherwise, as BufferBudget::replace). Charged
 * to the device domain: every buffer from alloc / upload_weight (the requested
 * bytes, at least one) and the context's own device scratch (int8 activations,
 * partial results, counters, the RoPE table) as it grows; a charge that would
 * pass the quota fails with MDMA_ERR_BUFFER_BUDGET before anything is allocated,
 * and a buffer whose hipFree fails stays charged. The library allocates no host
 * buffers after create, so the host domain stays at zero. */
int mdma_gfx950_set_buffer_budget(mdma_ctx *ctx, uint64_t device_bytes, uint64_t host_bytes);
/* BufferBudget::used / limit of one domain (mdma_memory_domain). */
int mdma_gfx950_buffer_usage(mdma_ctx *ctx, int domain, uint64_t *used, uint64_t *limit);
/* Extra: select the arithmetic of the GEMVs, GEMMs and per-token ops that
 * follow (a mdma_act_mode; default MDMA_ACT_F32). MDMA_ACT_F32_CPU also switches
 * rmsnorm, silu_mul and attention to the CPU backend's evaluation order. After a
 * mode change, graphs captured before it refuse to launch (mdma_gfx950_graph_launch
 * fails; the library's decoder recaptures its step). */
int mdma_gfx950_set_act_mode(mdma_ctx *ctx, int mode);
/* Extra: in the int8 mode's one-token decode, fuse each layer's attention
 * RMSNorm into the GEMVs around it (the down projection stores the residual
 * stream and sums of squares, the QKV GEMV normalizes in its prologue); in
 * the Llama driver's prefill (64 tokens and up), have the RMSNorms ahead of
 * the QKV and gate/up GEMMs, the gated GEMM ahead of a Q6_K down projection
 * and the attention ahead of a Q6_K output projection, write those GEMMs'
 * input, so the GEMMs skip their own quantization pass, and have a Q6_K QKV
 * GEMM apply RoPE and write the K/V cache rows (the same bits). Default on;
 * off runs the separate
 * kernels (for A/B measurement and the parity tests of the fused paths). */
int mdma_gfx950_set_norm_fusion(mdma_ctx *ctx, int on);
/* Extra: the int8 mode's prefill GEMM kernel (calls of 64 or more tokens).
 * AUTO (default) takes the f16-path GEMM where it covers the weight (Q4_K
 * and Q6_K rows of whole 256-column blocks; a Q4_K gate/up pair as one
 * launch with the SiLU product in its epilogue) and the int8 MFMA GEMM
 * elsewhere (Q8_0); I8 forces the int8 MFMA GEMM (for A/B measurement and
 * parity of both).
 * Both compute the per-32-quantized product of the reference's
 * qmatmul_i8 (src/backend/rocm.rs:1759-1918). */
typedef enum { MDMA_PREFILL_AUTO = 0, MDMA_PREFILL_I8 = 1 } mdma_prefill_kernel;
int mdma_gfx950_set_prefill_kernel(mdma_ctx *ctx, int kind);
/* Extra: the int8 mode's batched decode GEMV kernel (calls of 3 tokens or
 * more on prepared-layout weights that the prefill GEMM does not take (3 to
 * 63 tokens), up to 16 tokens per launch). AUTO (default) streams each block of
 * the weight tile, activations and scales through a per-wave LDS ring by
 * DMA; STAGED loads them into registers and stages the weights in LDS (for
 * A/B measurement and the equality test: both give the same bits). */
typedef enum { MDMA_BATCH_AUTO = 0, MDMA_BATCH_STAGED = 1 } mdma_batch_kernel;
int mdma_gfx950_set_batch_kernel(mdma_ctx *ctx, int kind);
/* Extra (no counterpart in the reference): with on != 0, the AUTO batch
 * kernel reads a second, tile-major copy of each prepared Q6_K weight (its
 * size again in device memory, charged to the device budget), made at the
 * weight's first batch call outside graph capture; each 16-row tile's bytes
 * for a 512-column pair are then one contiguous stream instead of 128-byte
 * pieces of 16 rows. Same bits as without. Rewriting the weight's bytes
 * (upload, or an op's output over them) frees the copy. Off by default; the
 * Llama driver turns it on for sessions of 3 sequences or more. */
int mdma_gfx950_set_batch_layout(mdma_ctx *ctx, int on);
/* Extra (for tests; the reference pins its int8 matrix-core fragments the
 * same way, src/backend/rocm/tests.rs:1861-1925): block-dot capture. With
 * out set (NULL: off), every later int8-mode qmatmul, qmatmul_qkv and
 * ffn_gate_up on prepared-layout Q4_K / Q6_K / Q8_0 weights also stores
 * the int32 sub-block dots its production kernels form, for each weight of
 * the call in order: [T][rows][n_sub], n_sub = cols/16 for Q6_K (sum of
 * (q - 32) * x over 16 columns) and cols/32 otherwise (sum of q * x; Q4_K q
 * the 4-bit value). The f16-path prefill GEMM stores sc * dot, the integer
 * it forms with the Q4_K sub-block scale folded in. A call whose slots
 * exceed out fails with MDMA_ERR_SHAPE_MISMATCH; f32-mode calls and raw
 * GGUF-layout weights store nothing. */
int mdma_gfx950_capture_block_dots(mdma_ctx *ctx, mdma_buf *out);
/* Extra: the HIP stream (hipStream_t) every launch of this context uses. */
void *mdma_gfx950_stream(mdma_ctx *ctx);

/* ---- buffers: Backend::alloc/upload/download/copy (src/backend.rs:383-399) ---- */

int mdma_gfx950_alloc(mdma_ctx *ctx, uint64_t bytes, int pool, mdma_buf **out);
/* Drop of a buffer; a failed hipFree keeps its budget charge (src/backend/rocm/memory.rs:36-55). */
int mdma_gfx950_free(mdma_buf *buf);
uint64_t mdma_gfx950_buf_len(const mdma_buf *buf);
/* Extra: a non-owning window [offset, offset+len) of a buffer (freed with mdma_gfx950_free). */
int mdma_gfx950_buf_view(mdma_buf *parent, uint64_t offset, uint64_t len, mdma_buf **out);
int mdma_gfx950_upload(mdma_ctx *ctx, mdma_buf *dst, uint64_t offset, const void *src, uint64_t len);
int mdma_gfx950_download(mdma_ctx *ctx, const mdma_buf *src, uint64_t offset, void *dst, uint64_t len);
int mdma_gfx950_copy(mdma_ctx *ctx, const mdma_buf *src, uint64_t src_off, mdma_buf *dst,
                     uint64_t dst_off, uint64_t len);
/* Backend::upload_weight (src/backend.rs:228-237): the trait's (bytes, layout).
 * MDMA_LAYOUT_GGUF bytes are stored raw and marked for repacking: the first op
 * that reads the buffer as a Q4_K / Q6_K / Q8_0 QWeight of matching size
 * repacks it on the device into the prepared layout, in place of the raw bytes
 * (a buffer the reference's HIP backend uploads with its packed flag is read
 * the same way, src/backend/rocm.rs:401-412). Until then, and where that op
 * may not allocate (graph capture, the allocation-free call, a full budget),
 * the raw-layout kernels read it. MDMA_LAYOUT_GFX950 bytes (from
 * mdma_gfx950_pack_weight, e.g. a model cache) are stored as they are.
 * MDMA_LAYOUT_ROCM_Q4K_V3 (the reference ROCm backend's packed Q4_K,
 * src/cache/layout.rs:10-38) fails with MDMA_ERR_NOT_IMPLEMENTED, as the
 * trait's default does for layouts a backend does not read. */
int mdma_gfx950_upload_weight(mdma_ctx *ctx, const void *bytes, uint64_t len, int layout, mdma_buf **out);
/* Extra, for loaders that know the tensor: upload_weight with the dtype and
 * [rows, cols] given, so GGUF Q4_K / Q6_K / Q8_0 bytes are packed into the
 * prepared layout on the host before the upload (no raw copy on the device). */
int mdma_gfx950_upload_weight_typed(mdma_ctx *ctx, const void *bytes, uint64_t len, int layout,
                                    int32_t dtype, uint64_t rows, uint64_t cols, mdma_buf **out);
/* Extra: the layout a buffer holds now (mdma_layout), -1 for a null buffer. */
int mdma_gfx950_buf_layout(const mdma_buf *buf);
/* Host-side packing into / out of the prepared layout (pack_q4k of
 * src/cache/layout.rs:40-79 is the reference's counterpart): bytes of a
 * prepared [rows, cols] weight (0 if the dtype has no prepared layout), and
 * the lossless conversions. Run on the CPU; no context needed. */
uint64_t mdma_gfx950_prepared_bytes(int32_t dtype, uint64_t rows, uint64_t cols);
int mdma_gfx950_pack_weight(int32_t dtype, uint64_t rows, uint64_t cols, const void *gguf, uint64_t len,
                            void *out, uint64_t out_len);
int mdma_gfx950_unpack_weight(int32_t dtype, uint64_t rows, uint64_t cols, const void *prepared, uint64_t len,
                              void *out, uint64_t out_len);

/* ---- the quantized-weight hot path ---- */

/* Backend::qmatmul (src/backend.rs:469): y[t, r] = sum_i deq(W)[r, i] * x[t, i].
 * x is [T, n_in] f32 (T inferred), y is [T, n_out] f32. */
int mdma_gfx950_qmatmul(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y);
/* Backend::qmatmul_qkv (src/backend.rs:409-422): three projections of one x. */
int mdma_gfx950_qmatmul_qkv(mdma_ctx *ctx, const mdma_qweight *wq, const mdma_qweight *wk,
                            const mdma_qweight *wv, const mdma_buf *x, mdma_buf *q, mdma_buf *k,
                            mdma_buf *v);
/* Backend::ffn_gate_up (src/backend.rs:472-489): y = silu(gate*x) * (up*x).
 * The scratch buffers have the output shape; their final contents are unspecified. */
int mdma_gfx950_ffn_gate_up(mdma_ctx *ctx, const mdma_qweight *gate, const mdma_qweight *up,
                            const mdma_buf *x, mdma_buf *gate_scratch, mdma_buf *up_scratch,
                            mdma_buf *y);

/* ---- per-token ops ---- */

/* Backend::embed (src/backend.rs:494): dequantized rows of a [vocab, n_embd] table. */
int mdma_gfx950_embed(mdma_ctx *ctx, const mdma_qweight *table, const uint32_t *ids, uint64_t n_ids,
                      mdma_buf *out);
/* Backend::rmsnorm (:500); rows of w's length. */
int mdma_gfx950_rmsnorm(mdma_ctx *ctx, const mdma_buf *w, const mdma_buf *x, mdma_buf *y, float eps);
/* Backend::add_rmsnorm (:502-513): sum = a + b; y = rmsnorm(sum) * w. */
int mdma_gfx950_add_rmsnorm(mdma_ctx *ctx, const mdma_buf *w, const mdma_buf *a, const mdma_buf *b,
                            mdma_buf *sum, mdma_buf *y, float eps);
/* Backend::add (:515). */
int mdma_gfx950_add(mdma_ctx *ctx, const mdma_buf *a, const mdma_buf *b, mdma_buf *y);
/* Backend::silu_mul (:540). */
int mdma_gfx950_silu_mul(mdma_ctx *ctx, const mdma_buf *gate, const mdma_buf *up, mdma_buf *y);
/* Backend::rope (:518-526): interleaved pairs; token t at position pos + t. */
int mdma_gfx950_rope(mdma_ctx *ctx, mdma_buf *q, mdma_buf *k, uint32_t pos, uint64_t n_tokens,
                     const mdma_rope_spec *spec);
/* Backend::kv_write (:434-445): f32 rows into the f16 caches at element elem_offset. */
int mdma_gfx950_kv_write(mdma_ctx *ctx, const mdma_buf *k, const mdma_buf *v, mdma_buf *dst_k,
                         mdma_buf *dst_v, uint64_t elem_offset, uint64_t n_elems);
/* Backend::rope_kv_write (:452-467), fused: q rotated in place; rotated k and v stored. */
int mdma_gfx950_rope_kv_write(mdma_ctx *ctx, mdma_buf *q, mdma_buf *k, const mdma_buf *v,
                              mdma_buf *dst_k, mdma_buf *dst_v, uint64_t elem_offset, uint32_t pos,
                              uint64_t n_tokens, const mdma_rope_spec *spec, uint64_t n_elems);
/* Backend::attn (:527-539): causal GQA over the f16 cache, scale 1/sqrt(head_dim). */
int mdma_gfx950_attn(mdma_ctx *ctx, const mdma_buf *q, const mdma_kv_view *kv,
                     const mdma_attn_spec *spec, mdma_buf *o);

/* ---- extras beside the trait ---- */

/* Argmax with ties to the LAST index (sampler::greedy, src/sampler.rs:64-74)
 * of n f32 logits at element offset `offset`; the id is written to host *out. */
int mdma_gfx950_greedy(mdma_ctx *ctx, const mdma_buf *logits, uint64_t offset, uint64_t n,
                       uint32_t *out);
/* Int8 activation quantizer (the Q8_1 rule of src/backend/rocm/kernels/kernels.hip:1102-1133
 * with an f32 scale): q int8 [n], d f32 [n/group], sum16 i32 [n/16]. group is 256 or 32. */
int mdma_gfx950_quantize_act(mdma_ctx *ctx, const mdma_buf *x, uint64_t group, mdma_buf *q,
                             mdma_buf *d, mdma_buf *sum16);
/* Debug: int32 dot per (token, row, sub-block) of weight quants with int8
 * activations qx [T, n_in]; sub-blocks are 32 wide (Q4_K, Q8_0) or 16 (Q6_K).
 * out is int32 [T][n_out][n_in/sub]. */
int mdma_gfx950_block_dot_i32(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *qx,
                              mdma_buf *out);
/* Explicit-mode GEMVs, independent of the context's mode. */
int mdma_gfx950_qmatmul_f32(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y);
int mdma_gfx950_qmatmul_i8(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): mdma_gfx950_qmatmul_i8 with the scratch its int8 routes
 * take -- x's per-256 int8 form, or the prefill GEMM's per-32 inputs (the
 * GEMM then runs unsplit) -- in the library's static device array of 8 MiB
 * per GPU instead of the context's buffers. It calls no hipMalloc or
 * hipFree; an x needing more than 8 MiB of scratch (about 6.1 million
 * values) fails with MDMA_ERR_BUFFER_BUDGET before anything runs. Calls
 * through one context run in its stream's order; calls from several
 * contexts on one GPU share the array and are ordered by an event per GPU
 * (each call's stream waits for the previous call's kernels), except under
 * stream capture, where a captured call races with other contexts' calls
 * that run while its graph replays. */
int mdma_gfx950_qmatmul_i8_noalloc(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x, mdma_buf *y);

/* Stream capture into a replayable HIP graph (the reference's graph decode
 * executor, src/backend/rocm/graph.rs:105-262, captures forward_device the
 * same way). Between begin and end, launches are recorded, not run; calls
 * that must synchronize (upload, download, scratch growth) fail with
 * MDMA_ERR_BACKEND instead. A graph holds the device addresses its launches
 * used: graph_launch fails with MDMA_ERR_BACKEND once the context has
 * replaced any buffer of its own since the capture (scratch growth, the
 * repack of a weight from the trait-shaped upload_weight); reserve_scratch
 * before capturing and capture again after. Buffers the caller frees must
 * outlive the graphs that use them. */
typedef struct mdma_graph mdma_graph;
int mdma_gfx950_graph_begin(mdma_ctx *ctx);
int mdma_gfx950_graph_end(mdma_ctx *ctx, mdma_graph **out);
int mdma_gfx950_graph_launch(mdma_ctx *ctx, mdma_graph *graph);
void mdma_gfx950_graph_destroy(mdma_graph *graph);
/* Pre-size the context scratch and int8-activation buffers so a later capture needs no growth. */
int mdma_gfx950_reserve_scratch(mdma_ctx *ctx, uint64_t bytes);
/* Graph replay parameters (ReplayParams, src/backend/rocm/graph.rs:12-15,
 * read by the reference's *_graph kernels, src/backend/rocm/kernels/
 * kernels.hip:385-410,620-640 and attention.hip:70-74): with params set (a
 * device buffer of two uint32: token, position) the trait-level ops whose
 * arguments change from one decode step to the next read them from device
 * memory when they run, so one captured forward_device replays every step:
 *  - embed reads its single token id from params[0] (n_ids must be 1; the
 *    host ids are not read);
 *  - rope, rope_kv_write and kv_write rotate at position params[1] and write
 *    the cache rows at element params[1] * row width (the pos and
 *    elem_offset arguments are not read; n_tokens must be 1);
 *  - attn attends to params[1] + 1 keys (kv->len is not read; its launch is
 *    sized for `capacity` keys, which the caches must hold, and n_q must be 1).
 * Set while capturing a decode step, then cleared (params NULL); a graph
 * launch replays the step for the values params holds at that time. */
int mdma_gfx950_set_replay_params(mdma_ctx *ctx, const mdma_buf *params, uint64_t capacity);
/* Extra (no counterpart in the reference; for benchmarks and profiling):
 * the next GEMV kernel this context launches on prepared weights is
 * dispatched with these hipEvent_t handles (either may be NULL), which its
 * dispatch packet timestamps at kernel start and end (hipExtLaunchKernel).
 * Applies to one launch; not allowed during graph capture. */
int mdma_gfx950_time_next_gemv(mdma_ctx *ctx, void *start_event, void *stop_event);

/* ---- Llama decoding: the hot path's caller ----
 * Model / KvCache / Workspace / inference::generate (src/model.rs:41-468,
 * src/kv_cache.rs:16-301, src/inference.rs:44-124). A session owns the f16 KV
 * caches of `batch` sequences of up to `capacity` positions and a workspace
 * of max(max_tokens, batch) token rows. */
typedef struct mdma_model mdma_model;
typedef struct mdma_session mdma_session;

/* ModelConfig (src/model.rs:19-29) plus the vocabulary size. */
typedef struct {
    uint64_t n_layers, n_embd, n_ff, n_heads, n_kv_heads, head_dim, n_ctx, vocab;
    float rope_theta, rms_eps;
} mdma_model_config;

/* Memory plan (src/model/memory.rs:16-63; headroom src/registry.rs:37):
 * device bytes of the weights, of a KV cache for `batch` sequences of
 * `capacity` positions and of a workspace, the headroom kept free, and the
 * longest context the device still has room for at that batch. */
typedef struct {
    uint64_t weight_bytes, kv_bytes, workspace_bytes, headroom_bytes, total_bytes;
    uint64_t device_bytes, available_bytes, max_context;
} mdma_memory_plan;

/* Model::load_with_budget (src/model.rs:141-149): preflight, reserve the
 * weight bytes (budget_bytes = 0: unlimited; MDMA_ERR_MEMORY_BUDGET past it,
 * MDMA_ERR_INSUFFICIENT_MEMORY past the device's free bytes less headroom),
 * then upload every tensor of a llama GGUF file. */
int mdma_gfx950_model_load(mdma_ctx *ctx, const char *gguf_path, uint64_t budget_bytes, mdma_model **out);
void mdma_gfx950_model_free(mdma_model *m);
int mdma_gfx950_model_config(const mdma_model *m, mdma_model_config *out);
int mdma_gfx950_model_plan(const mdma_model *m, uint64_t capacity, uint64_t batch, uint64_t tokens,
                           mdma_memory_plan *out);
/* KvCache::new + Model::alloc_workspace, reserved like the weights. */
int mdma_gfx950_session_new(mdma_model *m, uint64_t capacity, uint64_t batch, uint64_t max_tokens,
                            mdma_session **out);
void mdma_gfx950_session_free(mdma_session *s);
/* KvCache::set_len(0) for every sequence. */
int mdma_gfx950_session_reset(mdma_session *s);
/* Model::prefill (src/model.rs:398-468) of sequence `seq`: n tokens at pos;
 * the last row's logits (vocab f32) to host `logits` when non-null. */
int mdma_gfx950_prefill(mdma_session *s, uint64_t seq, const uint32_t *tokens, uint64_t n, uint32_t pos,
                        float *logits);
/* Model::forward (src/model.rs:326-393): one decode step of sequence `seq`. */
int mdma_gfx950_forward(mdma_session *s, uint64_t seq, uint32_t token, uint32_t pos, float *logits);
/* Prefill + greedy decode of every sequence (inference::sample without EOS,
 * src/inference.rs:102-124): prompts [batch][n_prompt], out_tokens
 * [batch][n_gen]. With batch > 1 each decode step runs the batch's tokens
 * through the weights together (one GEMV per matrix for all sequences).
 * step_seconds[n_gen] (nullable): [0] = prefill of all sequences and the
 * first token, [i] = decode step i. Non-finite logits fail with
 * MDMA_ERR_BACKEND. */
int mdma_gfx950_generate(mdma_session *s, const uint32_t *prompts, uint64_t n_prompt, uint64_t n_gen,
                         uint32_t *out_tokens, double *step_seconds);

/* Graph decode executor (HipDecoder / Decoder::forward,
 * src/backend/rocm/graph.rs:105-262): one decode step of sequence `seq`
 * captured into a HIP graph whose token and position are read from device
 * memory, replayed by every later forward. Its logits equal
 * mdma_gfx950_forward's bit for bit, with the same validation
 * (Model::validate_decode) and the same KV update. A forward after the
 * context replaced a buffer the graph captured (scratch growth, a prefill
 * of more tokens) runs that step eagerly and captures again. Free the
 * decoder before its session. */
typedef struct mdma_decoder mdma_decoder;
int mdma_gfx950_decoder_new(mdma_session *s, uint64_t seq, mdma_decoder **out);
int mdma_gfx950_decoder_forward(mdma_decoder *d, uint32_t token, uint32_t pos, float *logits);
/* Whether the decoder's last forward replayed its graph (1) or ran eagerly (0). */
int mdma_gfx950_decoder_replayed(const mdma_decoder *d);
void mdma_gfx950_decoder_free(mdma_decoder *d);
/* Extra: whether generate captures its decode step into a HIP graph and
 * replays it (default on; off runs every step eagerly, for A/B measurement
 * and the test that both give the same tokens). */
int mdma_gfx950_set_graph_decode(mdma_ctx *ctx, int on);

#ifdef __cplusplus
}
#endif
#endif
