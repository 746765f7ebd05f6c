/*
 * Oracle: the reference's CPU device operations (dwim `gpu/cpu.rs`), restated
 * in C expression by expression.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int or_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static inline float sum_seq(const float *v, size_t n) {
    float t = -0.0f;
    for (size_t i = 0; i < n; i++) t += v[i];
    return t;
}

/* gpu/cpu.rs:425-427 */
static inline float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
/* gpu/cpu.rs:430-432 */
static inline float softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

static float row_dot(const or_weight *w, size_t r, const float *x) {
    size_t cols = w->cols;
    switch (w->fmt) {
    case OR_BF16:
        return or_dot_bf16((const uint16_t *)w->quants + r * cols, x, cols);
    case OR_Q4_0:
        return or_dot_q4_0(w->scales + r * (cols / 32), (const uint8_t *)w->quants + r * cols / 2, x,
                           cols);
    case OR_Q8_0:
        return or_dot_q8_0(w->scales + r * (cols / 32), (const int8_t *)w->quants + r * cols, x,
                           cols);
    case OR_Q4_K:
        return or_dot_q4_k((const uint8_t *)w->quants + r * (cols / 256) * 144, x, cols);
    case OR_Q6_K:
        return or_dot_q6_k((const uint8_t *)w->quants + r * (cols / 256) * 210, x, cols);
    }
    abort();
}

/* or_dot_q4_k for many tokens at once, with the same arithmetic for every
 * (row, token) pair: the row's nibbles are converted to floats once per tile
 * of tokens, and each sub-block's Σx, which does not depend on the row, once
 * per token.  The 8 lanes of a sub-block's Σq·x are one vector, summed in the
 * same order (4 steps of 8 from zero, then sum8 from -0.0), and the total
 * folds in d1·Σqx − m1·Σx sub-block after sub-block as or_dot_q4_k does. */

static void matmul_q4_k(float *out, const or_weight *w, const float *x, size_t n) {
    size_t rows = w->rows, cols = w->cols, subs = cols / 32;
    const uint8_t *quants = (const uint8_t *)w->quants;
    float *sx = (float *)malloc(n * subs * sizeof(float));
#pragma omp parallel for schedule(static)
    for (size_t t = 0; t < n; t++)
        for (size_t s = 0; s < subs; s++) {
            const float *xs = x + t * cols + 32 * s;
            float l[8] = {0};
            for (int c = 0; c < 4; c++)
                for (int i = 0; i < 8; i++) l[i] += xs[8 * c + i];
            float v = -0.0f;
            for (int i = 0; i < 8; i++) v += l[i];
            sx[t * subs + s] = v;
        }
    const size_t tile = 16;
    for (size_t t0 = 0; t0 < n; t0 += tile) {
        size_t t1 = t0 + tile < n ? t0 + tile : n;
#pragma omp parallel
        {
            float *qf = (float *)aligned_alloc(32, cols * sizeof(float));
            float *d1 = (float *)malloc(subs * sizeof(float)), *m1 = (float *)malloc(subs * sizeof(float));
#pragma omp for schedule(static)
            for (size_t r = 0; r < rows; r++) {
                const uint8_t *row = quants + r * (cols / 256) * 144;
                for (size_t b = 0; b < cols / 256; b++) {
                    const uint8_t *blk = row + 144 * b;
                    float d = or_from_f16((uint16_t)(blk[0] | blk[1] << 8));
                    float dmin = or_from_f16((uint16_t)(blk[2] | blk[3] << 8));
                    for (int j = 0; j < 8; j++) {
                        uint8_t sc, m;
                        or_q4_k_scale_min(j, blk + 4, &sc, &m);
                        d1[8 * b + j] = d * (float)sc;
                        m1[8 * b + j] = dmin * (float)m;
                        for (int l = 0; l < 32; l++) {
                            uint8_t byte = blk[16 + 32 * (j / 2) + l];
                            qf[256 * b + 32 * j + l] = (float)((j % 2) ? (byte >> 4) : (byte & 0xf));
                        }
                    }
                }
                for (size_t t = t0; t < t1; t++) {
                    const float *xt = x + t * cols;
                    const float *st = sx + t * subs;
                    float acc = 0.0f;
                    for (size_t s0 = 0; s0 < subs; s0 += 8) {
                        __m256 sq[8];
                        for (int k = 0; k < 8; k++) {
                            const float *qs = qf + 32 * (s0 + k), *xs = xt + 32 * (s0 + k);
                            __m256 v = _mm256_setzero_ps();
                            for (int c = 0; c < 4; c++)
                                v = _mm256_add_ps(v, _mm256_mul_ps(_mm256_load_ps(qs + 8 * c), _mm256_loadu_ps(xs + 8 * c)));
                            sq[k] = v;
                        }
                        /* transpose: lane i of sq[k] to lane k of tr[i], so that
                         * -0.0 + tr[0] + ... + tr[7] is sum8 of each sub-block in order */
                        __m256 a0 = _mm256_unpacklo_ps(sq[0], sq[1]), a1 = _mm256_unpackhi_ps(sq[0], sq[1]);
                        __m256 a2 = _mm256_unpacklo_ps(sq[2], sq[3]), a3 = _mm256_unpackhi_ps(sq[2], sq[3]);
                        __m256 a4 = _mm256_unpacklo_ps(sq[4], sq[5]), a5 = _mm256_unpackhi_ps(sq[4], sq[5]);
                        __m256 a6 = _mm256_unpacklo_ps(sq[6], sq[7]), a7 = _mm256_unpackhi_ps(sq[6], sq[7]);
                        __m256 b0 = _mm256_shuffle_ps(a0, a2, 0x44), b1 = _mm256_shuffle_ps(a0, a2, 0xee);
                        __m256 b2 = _mm256_shuffle_ps(a1, a3, 0x44), b3 = _mm256_shuffle_ps(a1, a3, 0xee);
                        __m256 b4 = _mm256_shuffle_ps(a4, a6, 0x44), b5 = _mm256_shuffle_ps(a4, a6, 0xee);
                        __m256 b6 = _mm256_shuffle_ps(a5, a7, 0x44), b7 = _mm256_shuffle_ps(a5, a7, 0xee);
                        __m256 tr[8] = {
                            _mm256_permute2f128_ps(b0, b4, 0x20), _mm256_permute2f128_ps(b1, b5, 0x20),
                            _mm256_permute2f128_ps(b2, b6, 0x20), _mm256_permute2f128_ps(b3, b7, 0x20),
                            _mm256_permute2f128_ps(b0, b4, 0x31), _mm256_permute2f128_ps(b1, b5, 0x31),
                            _mm256_permute2f128_ps(b2, b6, 0x31), _mm256_permute2f128_ps(b3, b7, 0x31)};
                        __m256 sum = _mm256_set1_ps(-0.0f);
                        for (int i = 0; i < 8; i++) sum = _mm256_add_ps(sum, tr[i]);
                        __m256 term = _mm256_sub_ps(_mm256_mul_ps(_mm256_loadu_ps(d1 + s0), sum),
                                                    _mm256_mul_ps(_mm256_loadu_ps(m1 + s0), _mm256_loadu_ps(st + s0)));
                        float tv[8];
                        _mm256_storeu_ps(tv, term);
                        for (int k = 0; k < 8; k++) acc += tv[k];
                    }
                    out[t * rows + r] = acc;
                }
            }
            free(qf);
            free(d1);
            free(m1);
        }
    }
    free(sx);
}

/* gpu/cpu.rs:110-149: out[t][r] = w[r]·x[t], rows in parallel. */
void or_matmul(float *out, const or_weight *w, const float *x, size_t n) {
    size_t rows = w->rows, cols = w->cols;
    if (w->fmt == OR_Q4_K) {
        matmul_q4_k(out, w, x, n);
        return;
    }
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; r++)
        for (size_t t = 0; t < n; t++) out[t * rows + r] = row_dot(w, r, x + t * cols);
}

/* gpu/cpu.rs:151-155 */
void or_add(float *x, const float *y, size_t len) {
    for (size_t i = 0; i < len; i++) x[i] += y[i];
}

/* gpu/cpu.rs:157-166 */
void or_rmsnorm(float *x, size_t len, const float *weight, size_t dim, float eps) {
    for (size_t r = 0; r + dim <= len; r += dim) {
        float *row = x + r;
        float ms = -0.0f;
        for (size_t i = 0; i < dim; i++) ms += row[i] * row[i];
        ms = ms / (float)dim;
        float scale = 1.0f / sqrtf(ms + eps);
        for (size_t i = 0; i < dim; i++) row[i] *= scale * weight[i];
    }
}

/* gpu/cpu.rs:168-175 */
void or_l2norm(float *x, size_t len, size_t dim, float eps) {
    for (size_t r = 0; r + dim <= len; r += dim) {
        float *row = x + r;
        float ss = -0.0f;
        for (size_t i = 0; i < dim; i++) ss += row[i] * row[i];
        float scale = 1.0f / sqrtf(ss + eps);
        for (size_t i = 0; i < dim; i++) row[i] *= scale;
    }
}

/* gpu/cpu.rs:177-200: pair (i, i + rot/2) of each head rotated by
 * table[(pos + t)·rot + 2i .. +2] = (cos, sin). */
void or_rope(float *x, size_t len, const float *table, size_t pos, size_t n_heads, size_t head_dim,
             size_t rot_dim) {
    size_t half = rot_dim / 2, width = n_heads * head_dim;
    for (size_t t = 0; t * width < len; t++) {
        const float *angles = table + (pos + t) * rot_dim;
        for (size_t h = 0; h < n_heads; h++) {
            float *head = x + t * width + h * head_dim;
            for (size_t i = 0; i < half; i++) {
                float c = angles[2 * i], s = angles[2 * i + 1];
                float a = head[i], b = head[i + half];
                head[i] = a * c - b * s;
                head[i + half] = b * c + a * s;
            }
        }
    }
}

/* gpu/cpu.rs:78-87 */
void or_store(int8_t *cache_q, uint16_t *cache_s, size_t offset, const float *src, size_t len) {
    for (size_t b = 0; b < len / 32; b++)
        or_quantize(src + 32 * b, cache_s + offset / 32 + b, cache_q + offset + 32 * b);
}

/* gpu/cpu.rs:388-399 */
static float dot_q8(const float *a, size_t len, const int8_t *cq, const uint16_t *cs, size_t offset) {
    float total = -0.0f;
    for (size_t b = 0; b < len / 32; b++) {
        float dot = -0.0f;
        for (int i = 0; i < 32; i++) dot += a[32 * b + i] * (float)cq[offset + 32 * b + i];
        total += dot * or_from_f16(cs[offset / 32 + b]);
    }
    return total;
}

/* gpu/cpu.rs:402-411 */
static void add_scaled_q8(float *out, size_t len, float scale, const int8_t *cq, const uint16_t *cs,
                          size_t offset) {
    for (size_t b = 0; b < len / 32; b++) {
        float s = scale * or_from_f16(cs[offset / 32 + b]);
        for (int i = 0; i < 32; i++) out[32 * b + i] += s * (float)cq[offset + 32 * b + i];
    }
}

/* gpu/cpu.rs:413-423 */
static void softmax(float *x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* gpu/cpu.rs:202-236: causal GQA over the Q8 caches, (token, head) pairs in parallel. */
void or_attention(float *out, const float *q, size_t n, const int8_t *kq, const uint16_t *ks,
                  const int8_t *vq, const uint16_t *vs, size_t pos, size_t n_heads, size_t head_dim,
                  size_t n_kv_heads) {
    size_t group = n_heads / n_kv_heads, kv_dim = n_kv_heads * head_dim;
    float scale = 1.0f / sqrtf((float)head_dim);
    size_t items = n * n_heads;
#pragma omp parallel
    {
        float *scores = (float *)malloc((pos + n) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (size_t i = 0; i < items; i++) {
            size_t token = i / n_heads, head = i % n_heads;
            size_t len = pos + token + 1;
            size_t kv = head / group * head_dim;
            const float *qh = q + i * head_dim;
            float *o = out + i * head_dim;
            for (size_t t = 0; t < len; t++)
                scores[t] = scale * dot_q8(qh, head_dim, kq, ks, t * kv_dim + kv);
            softmax(scores, len);
            memset(o, 0, head_dim * sizeof(float));
            for (size_t t = 0; t < len; t++) add_scaled_q8(o, head_dim, scores[t], vq, vs, t * kv_dim + kv);
        }
        free(scores);
    }
}

/* The f16 KV-cache mode (no reference: the reference's caches are Q8): a
 * cache of f16 values, each the nearest f16 of the value stored (ties to
 * even), and Cpu::attention (gpu/cpu.rs:202-236) over it, the dot products
 * and weighted sums in the same order as over the Q8 cache with every block
 * scale 1 (dot_q8 and add_scaled_q8, :388-411). */
void or_store_f16(uint16_t *cache, size_t offset, const float *src, size_t len) {
    for (size_t i = 0; i < len; i++) cache[offset + i] = or_to_f16(src[i]);
}

static float dot_f16(const float *a, size_t len, const uint16_t *c, size_t offset) {
    float total = -0.0f;
    for (size_t b = 0; b < len / 32; b++) {
        float dot = -0.0f;
        for (int i = 0; i < 32; i++) dot += a[32 * b + i] * or_from_f16(c[offset + 32 * b + i]);
        total += dot;
    }
    return total;
}

static void add_scaled_f16(float *out, size_t len, float scale, const uint16_t *c, size_t offset) {
    for (size_t i = 0; i < len; i++) out[i] += scale * or_from_f16(c[offset + i]);
}

void or_attention_f16(float *out, const float *q, size_t n, const uint16_t *kc, const uint16_t *vc, size_t pos,
                      size_t n_heads, size_t head_dim, size_t n_kv_heads) {
    size_t group = n_heads / n_kv_heads, kv_dim = n_kv_heads * head_dim;
    float scale = 1.0f / sqrtf((float)head_dim);
    size_t items = n * n_heads;
#pragma omp parallel
    {
        float *scores = (float *)malloc((pos + n) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (size_t i = 0; i < items; i++) {
            size_t token = i / n_heads, head = i % n_heads;
            size_t len = pos + token + 1;
            size_t kv = head / group * head_dim;
            const float *qh = q + i * head_dim;
            float *o = out + i * head_dim;
            for (size_t t = 0; t < len; t++) scores[t] = scale * dot_f16(qh, head_dim, kc, t * kv_dim + kv);
            softmax(scores, len);
            memset(o, 0, head_dim * sizeof(float));
            for (size_t t = 0; t < len; t++) add_scaled_f16(o, head_dim, scores[t], vc, t * kv_dim + kv);
        }
        free(scores);
    }
}

/* gpu/cpu.rs:238-242 */
void or_silu_mul(float *gate, const float *up, size_t len) {
    for (size_t i = 0; i < len; i++) gate[i] = gate[i] * sigmoid(gate[i]) * up[i];
}

/* gpu/cpu.rs:244-248 */
void or_sigmoid_mul(float *x, const float *gate, size_t len) {
    for (size_t i = 0; i < len; i++) x[i] *= sigmoid(gate[i]);
}

/* gpu/cpu.rs:250-296: causal depthwise convolution of 4 taps, SiLU, split into
 * q | k | v; state_out gets the last 3 input rows. */
void or_conv(float *q, size_t q_dim, float *k, size_t k_dim, float *v, size_t v_dim, float *state_out,
             const float *x, size_t n, const float *state, const float *weight) {
    size_t ch = q_dim + k_dim + v_dim;
#define INPUT(t, c) ((t) < 0 ? state[(size_t)((t) + 3) * ch + (c)] : x[(size_t)(t) * ch + (c)])
    for (size_t t = 0; t < n; t++)
        for (size_t c = 0; c < ch; c++) {
            float acc = 0.0f;
            for (int j = 0; j < 4; j++) {
                long tt = (long)t + j + 1 - 4;
                acc += weight[c * 4 + j] * INPUT(tt, c);
            }
            float y = acc * sigmoid(acc);
            if (c < q_dim)
                q[t * q_dim + c] = y;
            else if (c < q_dim + k_dim)
                k[t * k_dim + c - q_dim] = y;
            else
                v[t * v_dim + c - q_dim - k_dim] = y;
        }
    for (size_t s = 0; s < 3; s++)
        for (size_t c = 0; c < ch; c++) {
            long tt = (long)n + (long)s + 1 - 4;
            state_out[s * ch + c] = INPUT(tt, c);
        }
#undef INPUT
}

/* gpu/cpu.rs:298-363: the gated delta rule, token after token, heads in
 * parallel; the state of head h is s[key][value]. */
void or_delta_net(float *out, const float *q, const float *k, const float *v, const float *gates,
                  const float *decay, float *state, size_t n, size_t n_k_heads, size_t n_v_heads,
                  size_t d) {
    size_t group = n_v_heads / n_k_heads;
    float scale = 1.0f / sqrtf((float)d);
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t h = 0; h < n_v_heads; h++) {
        float *s = state + h * d * d;
        size_t kh = h / group;
        float *kv = (float *)malloc(d * sizeof(float));
        for (size_t t = 0; t < n; t++) {
            const float *qt = q + (t * n_k_heads + kh) * d;
            const float *kt = k + (t * n_k_heads + kh) * d;
            const float *vt = v + (t * n_v_heads + h) * d;
            float alpha = gates[t * 2 * n_v_heads + h];
            float beta = sigmoid(gates[t * 2 * n_v_heads + n_v_heads + h]);
            float g = expf(decay[h] * softplus(alpha + decay[n_v_heads + h]));
            for (size_t e = 0; e < d * d; e++) s[e] *= g;
            for (size_t j = 0; j < d; j++) kv[j] = 0.0f;
            for (size_t i = 0; i < d; i++)
                for (size_t j = 0; j < d; j++) kv[j] += s[i * d + j] * kt[i];
            for (size_t i = 0; i < d; i++)
                for (size_t j = 0; j < d; j++) s[i * d + j] += kt[i] * (vt[j] - kv[j]) * beta;
            float *o = out + (t * n_v_heads + h) * d;
            for (size_t j = 0; j < d; j++) o[j] = 0.0f;
            for (size_t i = 0; i < d; i++)
                for (size_t j = 0; j < d; j++) o[j] += s[i * d + j] * qt[i] * scale;
        }
        free(kv);
    }
}

/* inference/qwen35/mod.rs:702-710: the first index of the largest logit. */
uint32_t or_argmax(const float *logits, size_t len) {
    size_t best = 0;
    for (size_t i = 0; i < len; i++)
        if (logits[i] > logits[best]) best = i;
    return (uint32_t)best;
}

/* inference/qwen35/mod.rs:1504-1515 */
void or_rope_table(float *table, size_t max_len, size_t rot_dim, float theta) {
    size_t half = rot_dim / 2;
    for (size_t pos = 0; pos < max_len; pos++)
        for (size_t i = 0; i < half; i++) {
            float freq = 1.0f / powf(theta, (float)(2 * i) / (float)rot_dim);
            float a = (float)pos * freq;
            table[(pos * half + i) * 2] = cosf(a);
            table[(pos * half + i) * 2 + 1] = sinf(a);
        }
}
