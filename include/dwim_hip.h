/*
 * dwim_hip.h — the C ABI of the MI355X (gfx950) backend for dwim's inference
 * engine.  It is the `gpu::Device` trait of the reference (dwim `gpu/mod.rs:
 * 176-401`) as plain C: one function per trait method, opaque handles for the
 * trait's three associated types (`Buffer`, `Weight`, `Cache`), plain pointers
 * and sizes, no C++ or torch types.  A Rust `gpu/hip` module binds it with
 * `extern "C"` declarations; this repository's own C++
 * host (the qwen35 forward pass) and its Python tests call it directly.
 *
 * Conventions (those of the reference's `Device`):
 *  - Every function that can fail returns 0 on success and a nonzero status
 *    otherwise, with a message from dwim_last_error().  The reference's ops
 *    panic on contract violations (`gpu/cpu.rs:51-56` "a buffer of {cap}
 *    activations can't hold {len}") and on launch failures; a binding turns a
 *    nonzero status into that panic.  Only dwim_open's failure is a plain
 *    error (the reference's `open` returns `Result`, `gpu/cuda/mod.rs:210`).
 *  - Lengths count f32 activations.  Operations over rows of activations take
 *    a buffer's length as a whole number of rows.
 *  - Operations are queued on the device's one stream, in order; dwim_read and
 *    dwim_read_cache wait for everything queued before them
 *    (`gpu/mod.rs:174-175`).  A device is used from one thread at a time.
 *  - A buffer has a length and the capacity it was allocated with;
 *    dwim_resize changes only the length (`gpu/mod.rs:216-219`).
 */
#ifndef DWIM_HIP_H
#define DWIM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dwim_dev dwim_dev;       /* the device: one GPU, one stream          */
typedef struct dwim_buf dwim_buf;       /* Device::Buffer: f32 activations          */
typedef struct dwim_weight dwim_weight; /* Device::Weight: a weight matrix          */
typedef struct dwim_cache dwim_cache;   /* Device::Cache: Q8 key or value cache     */

/* Weight formats (`Tensor`, gpu/mod.rs:46-61, plus the two K-quant formats the
 * reference has no device form of). */
enum dwim_format {
    DWIM_BF16 = 0, /* quants: u16 bf16 bits [rows][cols]; scales: NULL                        */
    DWIM_Q4_0 = 1, /* quants: u8 [rows][cols/2], element j low / j+16 high nibble of byte j;
                      scales: f16 bits [rows][cols/32]  (gpu/quant.rs:1-12)                     */
    DWIM_Q8_0 = 2, /* quants: i8 [rows][cols]; scales: f16 bits [rows][cols/32]                */
    DWIM_Q4_K = 3, /* quants: ggml block_q4_K, 144 B per 256 weights, row-major; scales: NULL  */
    DWIM_Q6_K = 4  /* quants: ggml block_q6_K, 210 B per 256 weights, row-major; scales: NULL
                      (the file layout of inference/quants.rs:79-104)                          */
};

/* The message of the last failure on this thread ("" if none). */
const char *dwim_last_error(void);

/* ---- the device (gpu/cuda/mod.rs:210-306 `open`; gpu/mod.rs:188-204) ---- */

/* Opens GPU `index` (a gfx950 device), with one in-order stream. */
int dwim_open(int index, dwim_dev **out);
void dwim_close(dwim_dev *dev);
/* Device::name: the GPU's name, NUL-terminated, truncated to `cap` bytes. */
int dwim_name(dwim_dev *dev, char *out, size_t cap);
/* Device::memory: bytes of device memory free. */
int dwim_memory(dwim_dev *dev, uint64_t *free_bytes);
/* Device::batch: most tokens a forward pass should run through at once. */
size_t dwim_batch(dwim_dev *dev);
/* Waits for every operation queued on the device. */
int dwim_sync(dwim_dev *dev);
/* The device's stream (a hipStream_t), for timing with HIP events. */
void *dwim_stream(dwim_dev *dev);

/* ---- memory (gpu/mod.rs:206-249) ---- */

/* Device::upload: copies a weight matrix to the device, which may lay it out
 * anew.  `quants`/`scales` as enum dwim_format says; `cols` a whole number of
 * the format's blocks (32, or 256 for the K formats; any multiple of 8 for bf16). */
int dwim_upload(dwim_dev *dev, int format, size_t rows, size_t cols, const void *quants,
                const uint16_t *scales, dwim_weight **out);
void dwim_free_weight(dwim_weight *w);
/* Device::alloc: a zeroed buffer of `len` activations. */
int dwim_alloc(dwim_dev *dev, size_t len, dwim_buf **out);
void dwim_free_buffer(dwim_buf *buf);
/* Device::alloc_cache: a zeroed cache of `len` activations, whole blocks of 32. */
int dwim_alloc_cache(dwim_dev *dev, size_t len, dwim_cache **out);
void dwim_free_cache(dwim_cache *cache);
/* Device::resize: sets the length, up to the capacity. */
int dwim_resize(dwim_dev *dev, dwim_buf *buf, size_t len);
size_t dwim_len(const dwim_buf *buf);
/* Device::read: copies the buffer's `len` activations out; `len` must equal
 * its length.  Waits for the operations before it. */
int dwim_read(dwim_dev *dev, const dwim_buf *buf, float *out, size_t len);
/* Device::write: copies `len` activations in; `len` must equal its length. */
int dwim_write(dwim_dev *dev, dwim_buf *buf, const float *data, size_t len);
/* Device::copy: dst[dst_offset..][..len] = src[src_offset..][..len]. */
int dwim_copy(dwim_dev *dev, dwim_buf *dst, size_t dst_offset, const dwim_buf *src,
              size_t src_offset, size_t len);
/* Device::store: quantizes `src` into the cache from `offset` on, a block of
 * 32 at a time as gpu/quant.rs:161-180 does; offset and length whole blocks. */
int dwim_store(dwim_dev *dev, dwim_cache *cache, size_t offset, const dwim_buf *src);
/* Device::read_cache: the first `len` activations as stored, `len` int8 then
 * len/32 little-endian f16 scales (an f16 cache: 2·len bytes of f16), that is
 * dwim_cache_bytes_of(cache, len) bytes, into `out`, which holds `out_bytes`;
 * a smaller `out` is refused (status 1) with nothing written. */
int dwim_read_cache(dwim_dev *dev, const dwim_cache *cache, size_t len, uint8_t *out, size_t out_bytes);
/* Device::write_cache: sets the first activations from bytes as read_cache gives them. */
int dwim_write_cache(dwim_dev *dev, dwim_cache *cache, const uint8_t *data, size_t bytes);
/* gpu/mod.rs:404-407: the bytes of `len` activations of a Q8 cache */
size_t dwim_cache_bytes(size_t len);
/* The bytes read_cache gives for `len` activations of this cache, of either
 * format (Q8: dwim_cache_bytes(len); f16: 2·len). */
size_t dwim_cache_bytes_of(const dwim_cache *cache, size_t len);
/* An f16 key/value cache of `len` activations (the f16 KV-cache mode; the
 * reference has only Q8, gpu/mod.rs:39-41,183-186): dwim_store rounds each
 * value to the nearest f16 (ties to even), dwim_read_cache / dwim_write_cache
 * move 2·len bytes of little-endian f16, and dwim_attention reads the values
 * as they are.  Freed with dwim_free_cache. */
int dwim_alloc_cache_f16(dwim_dev *dev, size_t len, dwim_cache **out);

/* ---- operations (gpu/mod.rs:251-400) ---- */

/* Device::matmul (gpu/mod.rs:254): out[t] = w · x[t] for each token row of x. */
int dwim_matmul(dwim_dev *dev, dwim_buf *out, const dwim_weight *w, const dwim_buf *x);
/* Device::matmul_add (gpu/mod.rs:259-268): x += w · input (scratch as long as x, left undefined). */
int dwim_matmul_add(dwim_dev *dev, dwim_buf *x, const dwim_weight *w, const dwim_buf *input,
                    dwim_buf *scratch);
/* Device::swiglu (gpu/mod.rs:274-285): out = silu(gate · x) * (up · x) (scratch as long as out,
 * left undefined). */
int dwim_swiglu(dwim_dev *dev, dwim_buf *out, const dwim_weight *gate, const dwim_weight *up,
                const dwim_buf *x, dwim_buf *scratch);
/* Device::add (gpu/mod.rs:288): x += y */
int dwim_add(dwim_dev *dev, dwim_buf *x, const dwim_buf *y);
/* Device::normalize (gpu/mod.rs:295-305): out = rmsnorm(x[..len]) * weight, rows of weight's length. */
int dwim_normalize(dwim_dev *dev, dwim_buf *out, const dwim_buf *x, const dwim_buf *weight,
                   size_t len, float eps);
/* Device::rmsnorm (gpu/mod.rs:309): each weight-long row of x normalized by its root mean square,
 * times weight. */
int dwim_rmsnorm(dwim_dev *dev, dwim_buf *x, const dwim_buf *weight, float eps);
/* Device::l2norm (gpu/mod.rs:312): each dim-long row of x to unit length. */
int dwim_l2norm(dwim_dev *dev, dwim_buf *x, size_t dim, float eps);
/* Device::rope (gpu/mod.rs:321-336): rotary embeddings: pair (i, i + rot/2) of each head at position p rotated by
 * table[(p*rot/2 + i)*2 ..][..2] = (cos, sin); the first token at `pos`. */
int dwim_rope(dwim_dev *dev, dwim_buf *x, const dwim_buf *table, size_t pos, size_t n_heads,
              size_t head_dim, size_t rot_dim);
/* Device::attention (gpu/mod.rs:338-349): causal GQA over the caches, the first token at `pos`. */
int dwim_attention(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_cache *k_cache,
                   const dwim_cache *v_cache, size_t pos, size_t n_heads, size_t head_dim,
                   size_t n_kv_heads);
/* No counterpart in the reference: dwim_attention for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The same kernels and results as
 * dwim_attention, but the decode path's partial results (fewer than 16
 * tokens) or a batch's expanded key/value cache (16 tokens or more, head_dim
 * 256) live in a file-scope device array of 64 MiB per GPU (held until the
 * process ends) instead of a buffer the library grows: no hipMalloc or
 * hipFree is called.  Fails with a clear error when they exceed it: the
 * partials are n·n_heads·ceil((pos + n)/64)·(head_dim + 2) floats (one token
 * of 24 heads of 256 reaches past 170 000 positions), the expanded cache
 * 64 KiB per 32 positions and key/value head (8192 positions at 4 key/value
 * heads).  Calls that overlap on one GPU share the array and race. */
int dwim_attention_noalloc(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_cache *k_cache,
                           const dwim_cache *v_cache, size_t pos, size_t n_heads, size_t head_dim,
                           size_t n_kv_heads);
/* No counterpart in the reference; measurement only: reads `bytes` (a
 * multiple of 16) at p on the device's stream and nothing else, over `blocks`
 * workgroups of 256 (16 bytes a lane, eight loads in flight a lane; `sink`, 4
 * bytes of device memory, is written only if the folded words equal a fixed
 * value).  The HBM streaming floor the decode products are read against. */
int dwim_measure_stream(dwim_dev *dev, const void *p, size_t bytes, unsigned *sink, unsigned blocks);
/* Device::silu_mul (gpu/mod.rs:351): gate = silu(gate) * up */
int dwim_silu_mul(dwim_dev *dev, dwim_buf *gate, const dwim_buf *up);
/* Device::sigmoid_mul (gpu/mod.rs:354): x *= sigmoid(gate) */
int dwim_sigmoid_mul(dwim_dev *dev, dwim_buf *x, const dwim_buf *gate);
/* Device::conv (gpu/mod.rs:365-386): the causal 4-tap convolution of linear attention, SiLU,
 * split into q|k|v. */
int dwim_conv(dwim_dev *dev, dwim_buf *q, dwim_buf *k, dwim_buf *v, dwim_buf *state_out,
              const dwim_buf *x, const dwim_buf *state, const dwim_buf *weight);
/* Device::delta_net (gpu/mod.rs:388-400): the gated delta rule, token after token, state
 * [n_v_heads][head_dim][head_dim]; any keys. */
int dwim_delta_net(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_buf *k,
                   const dwim_buf *v, const dwim_buf *gates, const dwim_buf *decay,
                   dwim_buf *state, size_t n_k_heads, size_t n_v_heads, size_t head_dim);

/* ---- beyond the trait ---- */

/* Device::delta_net for keys of unit length, as qwen35's layer makes them
 * (l2norm after the conv, inference/qwen35/mod.rs:612-617): from 64 tokens on,
 * the chunked (WY) form on the fp32 matrix cores, whose triangular solve is
 * well conditioned only for unit keys and decays below 1; fewer tokens, the
 * token loop.  Other keys belong to dwim_delta_net. */
int dwim_delta_net_unit_keys(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_buf *k,
                             const dwim_buf *v, const dwim_buf *gates, const dwim_buf *decay,
                             dwim_buf *state, size_t n_k_heads, size_t n_v_heads, size_t head_dim);
/* Device::conv followed by Device::l2norm of q and of k, rows of `dim`, as
 * qwen35's linear layer calls them (inference/qwen35/mod.rs:612-617), in one
 * launch (16 tokens a block for batches); dim a multiple of 64, at most 256. */
int dwim_conv_l2norm(dwim_dev *dev, dwim_buf *q, dwim_buf *k, dwim_buf *v, dwim_buf *state_out,
                     const dwim_buf *x, const dwim_buf *state, const dwim_buf *weight, size_t dim, float eps);

/* The greedy token of each of `rows` rows of logits: the first index of the
 * largest value (qwen35::argmax, inference/qwen35/mod.rs:702-710), on the
 * device, so that a token's 1 MB of logits need not be read back.  Writes
 * `rows` indices to `out` (host memory) and waits. */
int dwim_argmax(dwim_dev *dev, const dwim_buf *logits, size_t rows, uint32_t *out);

/* The token sampler on the device (inference/sampler.rs:7-146, which
 * inference/local.rs:305-312 calls as `pick`): from the top_k most likely
 * tokens of a row of logits, the smallest set reaching top_p, none less than
 * min_p times as likely as the most likely, at `temperature` (0: the most
 * likely, certain), drawn with the sampler's xorshift64* generator seeded
 * with max(seed, 1), as Sampler::new makes it.  The generator's state stays
 * on the device; each call reads back only its token.  A sampler holds a
 * reference on its device.  dwim_sampler_open fails for a negative
 * temperature, top_p <= 0 or min_p > 1 (settings that keep no token, with
 * which the reference's sampler would fail at its first pick). */
typedef struct dwim_sampler dwim_sampler;
int dwim_sampler_open(dwim_dev *dev, float temperature, size_t top_k, float top_p, float min_p, uint64_t seed,
                      dwim_sampler **out);
void dwim_sampler_free(dwim_sampler *s);
/* The generator's state (waits for the device). */
int dwim_sampler_rng(dwim_sampler *s, uint64_t *rng);
/* Sampler::sample (sampler.rs:40-51) of row `row` of `logits` ([rows][vocab]):
 * the token to *token; waits. */
int dwim_sample(dwim_sampler *s, const dwim_buf *logits, size_t row, size_t vocab, uint32_t *token);
/* Sampler::verify (sampler.rs:53-81) of `draft` against row `row`: the draft
 * kept with the probability dwim_sample would pick it, else another kept token
 * in proportion to the rest; the token to *token, *accepted 1 when it is the
 * draft; waits. */
int dwim_sample_verify(dwim_sampler *s, const dwim_buf *logits, size_t row, size_t vocab, uint32_t draft,
                       uint32_t *token, int *accepted);

/* One activation vector for several Q4_K matrices: dwim_prepare converts the
 * `cols` activations of x (one token) into the device's int8 planes, which
 * dwim_matmul_prepared then multiplies by a Q4_K weight of that many columns,
 * out = w · x, as dwim_matmul does for one token.  The planes are the
 * device's: the next dwim_prepare, or a one-token Q4_K dwim_matmul,
 * dwim_matmul_add or dwim_swiglu, replaces them. */
int dwim_prepare(dwim_dev *dev, const dwim_buf *x);
int dwim_matmul_prepared(dwim_dev *dev, dwim_buf *out, const dwim_weight *w);
/* Device::swiglu for one prepared token (gpu/mod.rs:274-285): out =
 * silu(gate · x) * (up · x), gate and up Q4_K, in the one launch the decode
 * step makes for a layer's feed-forward pair, which also writes the result's
 * planes into the device's second planes area (replacing the planes of any
 * other one-token product's output held there). */
int dwim_swiglu_prepared(dwim_dev *dev, dwim_buf *out, const dwim_weight *gate, const dwim_weight *up);

/* out[t] = row tokens[t] of `table` (a rows×cols weight of any format),
 * dequantized: the embedding lookup, which the reference does on the host from
 * the mapped GGUF (qwen35::Pass::embed, inference/qwen35/mod.rs:526-535), on
 * the device so that no embedding table stays on the host.  `tokens` is host
 * memory; out must hold n·cols activations. */
int dwim_embed(dwim_dev *dev, dwim_buf *out, const dwim_weight *table, const uint32_t *tokens,
               size_t n);

/* ---- the qwen35 model (inference/qwen35/mod.rs) on this device ----
 * A C++ restatement of the reference's `Model<D: Device>` over the operations
 * above, in the reference's order, for a random-initialised model built on
 * the device (no GGUF file: see dwim_model_synthetic). */
typedef struct dwim_model dwim_model;

/* qwen35::Config (inference/qwen35/mod.rs:29-56) */
typedef struct {
    size_t hidden, intermediate, layers;
    size_t heads, kv_heads, head_dim, rot_dim;
    float rope_theta;
    size_t full_attention_interval;
    size_t k_heads, v_heads, state_dim;
    float eps;
    size_t vocab;
    int drafter; /* the layer that predicts the token after the next */
} dwim_qwen35_config;

/* A model with every tensor drawn from `seed` (stream per tensor name, values
 * as dwim_synthetic_values makes them), matrices in `body_format` (the output
 * head in `head_format`), state for sequences of up to max_len tokens. */
int dwim_model_synthetic(dwim_dev *dev, const dwim_qwen35_config *cfg, uint64_t seed,
                         int body_format, int head_format, size_t max_len, dwim_model **out);
void dwim_model_free(dwim_model *m);
/* Device::batch as the model uses it: most tokens per forward batch. */
size_t dwim_model_batch(const dwim_model *m);
/* LanguageModel::forward (qwen35/mod.rs:1021-1038): runs the tokens from
 * position `pos` in batches; writes the logits after the last token (vocab
 * floats) to `logits` unless it is NULL. */
int dwim_model_forward(dwim_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits);
/* forward, then the greedy next token (first maximum, qwen35::argmax) taken on
 * the device: only 4 bytes come back. */
int dwim_model_forward_greedy(dwim_model *m, const uint32_t *tokens, size_t n, size_t pos,
                              uint32_t *next);
/* Greedy decoding of `steps` tokens, the reply loop's step (feed the token
 * picked, inference/local.rs:162-240) without the host between steps: from
 * `token` at position `pos`, out[i] = the greedy pick after step i, which is
 * step i+1's token.  The picks stay on the device until all steps are queued;
 * the same tokens as `steps` calls of dwim_model_forward_greedy. */
int dwim_model_decode_greedy(dwim_model *m, uint32_t token, size_t pos, size_t steps, uint32_t *out);
/* LanguageModel::reset (qwen35/mod.rs:1230-1246). */
int dwim_model_reset(dwim_model *m);
/* LanguageModel::draft (qwen35/mod.rs:1045-1071): up to k (at most 8, and as
 * many as the cache has room to verify) tokens the drafter predicts after
 * `token` at `pos`, each the head's first maximum; *count is how many (0
 * without a drafter, before any batch, or while one is being verified).
 * `drafts` holds k tokens. */
int dwim_model_draft(dwim_model *m, uint32_t token, size_t pos, size_t k, uint32_t *drafts,
                     size_t *count);
/* LanguageModel::verify (qwen35/mod.rs:1073-1091): runs 1..=9 tokens from
 * `pos` without committing the linear layers' states; writes the logits after
 * every token (n·vocab floats) to `logits` and/or each row's first maximum
 * (n tokens) to `greedy`, either of which may be NULL. */
int dwim_model_verify(dwim_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits,
                      uint32_t *greedy);
/* LanguageModel::rewind (qwen35/mod.rs:1099-1169): commits the first `keep`
 * (1..=n) tokens of the batch being verified. */
int dwim_model_rewind(dwim_model *m, size_t keep);
/* The model's logits on the device, as its last dwim_model_forward (the row
 * after the last token, also when its `logits` was NULL) or
 * dwim_model_verify (a row after every token) left them: the rows a
 * dwim_sampler picks from (inference/local.rs:305-312) without reading them
 * back.  The buffer stays the model's (not to be freed) and holds them until
 * the model's next call. */
int dwim_model_logits(dwim_model *m, const dwim_buf **out);
/* LanguageModel::mark / rewind_to_mark (qwen35/mod.rs:1176-1228): copies the
 * running sequence's linear-layer states aside on the device, and back; the
 * one mark belongs to the sequence that made it (error from another). */
int dwim_model_mark(dwim_model *m);
int dwim_model_rewind_to_mark(dwim_model *m);
/* LanguageModel::add_sequence / select_sequence (qwen35/mod.rs:1258-1290):
 * another sequence, as before any token, of the first one's length; and a
 * switch of the running sequence (nothing copied; error while verifying). */
int dwim_model_add_sequence(dwim_model *m, size_t *id);
int dwim_model_select_sequence(dwim_model *m, size_t id);
/* LanguageModel::save (inference/qwen35/mod.rs:905-947): the state after `len`
 * positions in the reference's "dwimstat" layout, version 3 (header; each key
 * cache then each value cache as read_cache gives it; per linear layer its conv
 * and recurrent state as f32; the drafter's carried hidden state).  With
 * `out` null, *bytes is the size needed; else up to `cap` bytes are written.
 * *bytes = 0 means no state to save (the reference's None): a batch is being
 * verified, or a drafter has nothing carried over. */
int dwim_model_save(dwim_model *m, size_t len, uint8_t *out, size_t cap, size_t *bytes);
/* LanguageModel::restore (inference/qwen35/mod.rs:949-1017): the current
 * sequence from a saved state; *len = its positions.  Fails with the
 * reference's messages on another layout, version or model. */
int dwim_model_restore(dwim_model *m, const uint8_t *state, size_t bytes, size_t *len);

/* Host-side quantizers, the product's own (gpu/quant.rs restated for the host
 * loader, plus the K formats).  `x` holds `cols` weights. */
void dwim_quantize_q4_0_row(const float *x, size_t cols, uint16_t *scales, uint8_t *quants);
void dwim_quantize_q8_0_row(const float *x, size_t cols, uint16_t *scales, int8_t *quants);
void dwim_quantize_q4_k_row(const float *x, size_t cols, uint8_t *blocks);
void dwim_quantize_q6_k_row(const float *x, size_t cols, uint8_t *blocks);
/* The cache quantizer for one block of 32 (gpu/quant.rs:161-180). */
void dwim_quantize_block(const float *block, uint16_t *scale, int8_t *q);
uint16_t dwim_to_f16(float x);
float dwim_from_f16(uint16_t bits);

/* Synthetic weights for a random-init model: value i of stream `seed` is an
 * approximately normal N(0, sigma) draw (the centred sum of four 16-bit
 * uniforms of a SplitMix64 hash of (seed, i), times sigma·sqrt(3)/65536), a
 * computation with integer steps and one f32 multiply, so that host and device
 * produce the same bits.  dwim_synthetic_values fills `n` values from index
 * `first` on the host; dwim_upload_synthetic builds a rows×cols weight of the
 * format directly on the device, row r's values being indices r*cols.. of the
 * stream, quantized exactly as the host quantizers above do. */
void dwim_synthetic_values(uint64_t seed, uint64_t first, size_t n, float sigma, float *out);
int dwim_upload_synthetic(dwim_dev *dev, int format, size_t rows, size_t cols, uint64_t seed,
                          float sigma, dwim_weight **out);

#ifdef __cplusplus
}
#endif
#endif
