/*
 * CPU oracle for the quantized-weight path: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of mdma's CPU backend (the reference's parity oracle,
 * /root/reference/src/backend/cpu.rs) for the operations the gfx950 library
 * implements. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker or the timed CPU baseline; the
 * product library never links or calls it.
 *
 * Every function is exported with C linkage and plain pointers so ctypes can
 * call it. Status codes match include/mdma_gfx950.h (0 = OK, 2 = shape mismatch).
 */
#ifndef MDMA_ORACLE_H
#define MDMA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (GGUF on-disk numbering). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14 };

float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

size_t orc_block_size(int dtype);
size_t orc_type_size(int dtype);

int orc_dequantize_row(int dtype, const uint8_t *bytes, size_t n_bytes, float *out, size_t n);
int orc_qmatmul(int dtype, const uint8_t *w, size_t w_bytes, size_t n_out, size_t n_in,
                const float *x, size_t x_elems, float *y, size_t y_elems, int n_threads);
int orc_embed(int dtype, const uint8_t *table, size_t table_bytes, size_t vocab, size_t n_embd,
              const uint32_t *ids, size_t n_ids, float *out, size_t out_elems);
int orc_rmsnorm(const float *w, size_t dim, const float *x, size_t x_elems, float *y,
                size_t y_elems, float eps);
int orc_add(const float *a, const float *b, size_t n, float *y);
int orc_add_rmsnorm(const float *w, size_t dim, const float *a, const float *b, size_t n,
                    float *sum, float *y, float eps);
int orc_silu_mul(const float *gate, const float *up, size_t n, float *y);
int orc_rope(float *q, size_t q_elems, float *k, size_t k_elems, uint32_t pos, size_t n_tokens,
             size_t head_dim, float theta);
void orc_rope_cos_sin(uint32_t pos, size_t head_dim, float theta, float *cos_out, float *sin_out);
int orc_attention(const float *q, size_t q_elems, const float *k, const float *v, size_t kv_elems,
                  size_t kv_len, size_t head_dim, size_t n_q_heads, size_t n_kv_heads,
                  float *o, size_t o_elems);
uint32_t orc_greedy(const float *logits, size_t n);

/* Int8 activation mode: groups of 256 (decode) or 32 (prefill) with an f32
 * scale, rounded by the Q8_1 rule of the reference. */
int orc_quantize_act(const float *x, size_t n, size_t group, int8_t *q, float *d, int32_t *sum16);
int orc_block_dot_i32(int dtype, const uint8_t *w, size_t w_bytes, size_t n_out, size_t n_in,
                      const int8_t *qx, size_t n_tokens, int32_t *out);

/* Llama decode (reference src/model/arch/llama.rs:158-246, src/model.rs:326-468). */
typedef struct {
    int dtype;
    size_t n_out, n_in;
    const uint8_t *data;
} orc_weight;

typedef struct {
    orc_weight wq, wk, wv, wo, w_gate, w_up, w_down;
    const float *attn_norm, *ffn_norm;
} orc_layer;

typedef struct {
    size_t n_layers, n_embd, n_ff, n_heads, n_kv_heads, head_dim, n_ctx, vocab;
    float rope_theta, rms_eps;
    orc_weight token_embd, output;
    const float *output_norm;
    const orc_layer *layers;
    int kv_f16; /* round K/V through f16 on store, as an f16 KV cache does */
    int n_threads;
    int act_i8; /* int8 activation mode: bits of the GEMVs whose x is requantized (orc_i8_group) */
} orc_model;

/* orc_model.act_i8 bits: which GEMVs of the int8 mode requantize x. */
enum { ORC_I8_QKV = 1, ORC_I8_O = 2, ORC_I8_GATE_UP = 4, ORC_I8_DOWN = 8, ORC_I8_HEAD = 16, ORC_I8_ALL = 31 };

/* Token count from which the device's int8 mode runs its prefill GEMM
 * (activations per 32) rather than a GEMV (per 256). */
enum { ORC_GEMM_MIN_TOKENS = 64 };
size_t orc_i8_group(int dtype, size_t n_out, size_t n_in, size_t T);
int orc_llama_run(const orc_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                  const uint32_t *forced, uint32_t *out_tokens, float *step_logits);
int orc_llama_run_timed(const orc_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                        const uint32_t *forced, uint32_t *out_tokens, float *step_logits,
                        double *step_seconds);
int orc_llama_generate(const orc_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                       uint32_t *out_tokens, float *last_logits);

#ifdef __cplusplus
}
#endif
#endif
