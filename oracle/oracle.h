/*
 * CPU oracle: a C restatement of the reference's CPU device (dwim `gpu/cpu.rs`),
 * its quantization helpers (`gpu/quant.rs`, `gpu/float.rs`, `inference/quants.rs`)
 * and the forward pass that calls them (`inference/qwen35/mod.rs`).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (`dwim_amd/`, `include/`)
 * links, loads or calls this library; only `tests/`, `__graft_entry__.smoke()`
 * and `bench.py`'s `cpu_baseline` leg use it, as the checker or as the timed
 * CPU baseline.
 *
 * Arithmetic follows the reference expression by expression: no fused
 * multiply-adds (the library is built with -ffp-contract=off, as rustc never
 * contracts), the same summation order (8-lane partial sums where the
 * reference has them, sequential folds elsewhere) and the same libm calls
 * (expf, logf, sqrtf, powf, sinf/cosf), so on x86-64 glibc its results are the
 * reference's bit for bit.  Q4_K and Q6_K dot products and the two quantizers
 * for them have no counterpart in the reference (it has no Q4_K at all and
 * requantizes Q6_K to Q8_0): they are defined here from the published ggml
 * block layouts and pinned by the known-answer tests in tests/.
 *
 * Parallelism (OpenMP over rows / heads, as rayon in the reference) never
 * changes per-row arithmetic.
 */
#ifndef DWIM_ORACLE_H
#define DWIM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- gpu/float.rs ---- */
float or_bf16(uint16_t bits);
uint16_t or_to_f16(float x);
uint16_t or_to_bf16(float x);
float or_from_f16(uint16_t bits);

/* ---- gpu/tests.rs:45-54 LCG ---- */
typedef struct { uint64_t s; } or_rng;
float or_rng_next(or_rng *r);
void or_rng_floats(uint64_t *state, float *out, size_t n);
/* Rng::bf16 (gpu/tests.rs:60-68): top halves of successive values. */
void or_rng_bf16(uint64_t *state, uint16_t *out, size_t n);

/* ---- gpu/quant.rs ---- */
void or_quantize(const float *block, uint16_t *scale, int8_t *q);            /* :161-180 */
void or_quantize_q8_0_row(const float *x, size_t cols, uint16_t *scales, int8_t *quants);
void or_dequantize_q8_0_row(const uint16_t *scales, const int8_t *quants, size_t cols, float *out);
float or_dot_q8_0(const uint16_t *scales, const int8_t *quants, const float *x, size_t cols);
void or_quantize_q4_0_row(const float *x, size_t cols, uint16_t *scales, uint8_t *quants);
void or_dequantize_q4_0_row(const uint16_t *scales, const uint8_t *quants, size_t cols, float *out);
float or_dot_q4_0(const uint16_t *scales, const uint8_t *quants, const float *x, size_t cols);
float or_dot_bf16(const uint16_t *w, const float *x, size_t cols);             /* cpu.rs:370-386 */

/* ---- inference/quants.rs (file-block formats) ---- */
void or_dequantize_q4_1_file(const uint8_t *row, size_t cols, float *out);
void or_dequantize_q6_k_file(const uint8_t *row, size_t cols, float *out);

/* ---- Q4_K (ggml block_q4_K, 144 bytes / 256 weights), no reference counterpart ---- */
void or_q4_k_scale_min(int j, const uint8_t *scales12, uint8_t *sc, uint8_t *m);
void or_quantize_q4_k_row(const float *x, size_t cols, uint8_t *blocks);
void or_dequantize_q4_k_row(const uint8_t *blocks, size_t cols, float *out);
float or_dot_q4_k(const uint8_t *blocks, const float *x, size_t cols);

/* ---- Q6_K (ggml block_q6_K, 210 bytes / 256 weights) ---- */
void or_quantize_q6_k_row(const float *x, size_t cols, uint8_t *blocks);
float or_dot_q6_k(const uint8_t *blocks, const float *x, size_t cols);

/* ---- gpu/cpu.rs device ops ---- */
enum { OR_BF16 = 0, OR_Q4_0 = 1, OR_Q8_0 = 2, OR_Q4_K = 3, OR_Q6_K = 4 };
typedef struct {
    int fmt;
    size_t rows, cols;
    const void *quants;       /* bf16 bits, Q4_0 nibbles, Q8_0 int8, Q4_K/Q6_K file blocks */
    const uint16_t *scales;   /* Q4_0 / Q8_0 block scales (f16 bits); unused otherwise */
} or_weight;

void or_matmul(float *out, const or_weight *w, const float *x, size_t n);
void or_add(float *x, const float *y, size_t len);
void or_rmsnorm(float *x, size_t len, const float *weight, size_t dim, float eps);
void or_l2norm(float *x, size_t len, size_t dim, float eps);
void or_rope(float *x, size_t len, const float *table, size_t pos, size_t n_heads,
             size_t head_dim, size_t rot_dim);
void or_store(int8_t *cache_q, uint16_t *cache_s, size_t offset, const float *src, size_t len);
void or_store_f16(uint16_t *cache, size_t offset, const float *src, size_t len);
void or_attention_f16(float *out, const float *q, size_t n, const uint16_t *kc, const uint16_t *vc, size_t pos,
                      size_t n_heads, size_t head_dim, size_t n_kv_heads);
void or_attention(float *out, const float *q, size_t n, const int8_t *kq, const uint16_t *ks,
                  const int8_t *vq, const uint16_t *vs, size_t pos, size_t n_heads,
                  size_t head_dim, size_t n_kv_heads);
void or_silu_mul(float *gate, const float *up, size_t len);
void or_sigmoid_mul(float *x, const float *gate, size_t len);
void or_conv(float *q, size_t q_dim, float *k, size_t k_dim, float *v, size_t v_dim,
             float *state_out, const float *x, size_t n, const float *state, const float *weight);
void or_delta_net(float *out, const float *q, const float *k, const float *v,
                  const float *gates, const float *decay, float *state, size_t n,
                  size_t n_k_heads, size_t n_v_heads, size_t head_dim);
uint32_t or_argmax(const float *logits, size_t len);

/* The token sampler (sampler.c; dwim inference/sampler.rs) */
typedef struct {
    float temperature;
    size_t top_k;
    float top_p, min_p;
    uint64_t rng;
} or_sampler;
float or_xorshift_next(uint64_t *state);
void or_sampler_init(or_sampler *s, float temperature, size_t top_k, float top_p, float min_p, uint64_t seed);
size_t or_sampler_candidates(const or_sampler *s, const float *logits, size_t len, uint32_t *tokens, float *probs,
                             float *total);
uint32_t or_sample(or_sampler *s, const float *logits, size_t len);
uint32_t or_sampler_verify(or_sampler *s, const float *logits, size_t len, uint32_t draft, int *accepted);
void or_rope_table(float *table, size_t max_len, size_t rot_dim, float theta);

int or_threads(void);

/* ---- the qwen35 forward pass (inference/qwen35/mod.rs), for the random model
 * the product builds with dwim_model_synthetic (same tensor names and streams) ---- */
typedef struct {
    size_t hidden, intermediate, layers;
    size_t heads, kv_heads, head_dim, rot_dim;
    float rope_theta;
    size_t full_attention_interval;
    size_t k_heads, v_heads, state_dim;
    float eps;
    size_t vocab;
    int drafter;
} or_qwen35_config;
typedef struct or_model or_model;
#define OR_MAX_DRAFTS 8  /* qwen35 MAX_DRAFTS (inference/qwen35/mod.rs:26) */
void or_synthetic_values(uint64_t seed, uint64_t first, size_t n, float sigma, float *out);
or_model *or_model_synthetic(const or_qwen35_config *cfg, uint64_t seed, int body_fmt, int head_fmt,
                             size_t max_len, size_t batch);
void or_model_free(or_model *m);
void or_model_forward(or_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits);
size_t or_model_draft(or_model *m, uint32_t token, size_t pos, size_t k, uint32_t *drafts);
void or_model_last_logits(const or_model *m, float *out);
void or_model_verify(or_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits);
void or_model_rewind(or_model *m, size_t keep);
void or_model_mark(or_model *m);
int or_model_rewind_to_mark(or_model *m);
void or_model_reset(or_model *m);
void or_model_zero_residual_writes(or_model *m);
size_t or_model_save(or_model *m, size_t len, uint8_t *out);
int or_model_restore(or_model *m, const uint8_t *state, size_t bytes, size_t *len);

#ifdef __cplusplus
}
#endif
#endif
