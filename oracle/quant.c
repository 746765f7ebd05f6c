/*
 * Oracle: half floats, block quantization and the dot products the CPU
 * reference multiplies with.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Reference files restated here, as text:
 *   gpu/float.rs        (bf16, to_f16, to_bf16, from_f16)
 *   gpu/quant.rs:34-180 (Q8_0, Q4_0, the cache quantizer)
 *   gpu/cpu.rs:370-386  (the bf16 row dot)
 *   inference/quants.rs:44-104 (Q4_1 and Q6_K file blocks)
 * and, without a reference counterpart, the Q4_K and Q6_K block formats of
 * ggml (llama.cpp `ggml-common.h` block_q4_K / block_q6_K, and the
 * `get_scale_min_k4` packing of `ggml-quants.c`), whose dequantization the
 * tests pin with hand-built blocks.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

static inline uint32_t bits_of(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float of_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* gpu/float.rs:6-8 */
float or_bf16(uint16_t bits) { return of_bits((uint32_t)bits << 16); }

#define F16_MAX 65504.0f

/* gpu/float.rs:15-29: nearest half, ties to even, clamped to the largest finite one. */
uint16_t or_to_f16(float x) {
    uint16_t sign = (uint16_t)((bits_of(x) >> 16) & 0x8000);
    float a = fminf(fabsf(x), F16_MAX);
    if (a < of_bits((uint32_t)(127 - 14) << 23)) {
        return sign | (uint16_t)rintf(a * (float)(1u << 24));
    }
    int e = (int)((bits_of(a) >> 23) & 0xff) - 127;
    uint32_t m = (uint32_t)rintf(a * of_bits((uint32_t)(127 + 10 - e) << 23));
    if (m == 2048) { e += 1; m = 1024; }
    return sign | (uint16_t)((e + 15) << 10) | (uint16_t)(m - 1024);
}

/* gpu/float.rs:32-36 */
uint16_t or_to_bf16(float x) {
    uint32_t b = bits_of(x);
    uint32_t round = 0x7fff + ((b >> 16) & 1);
    return (uint16_t)((b + round) >> 16);
}

/* gpu/float.rs:39-48 */
float or_from_f16(uint16_t h) {
    uint32_t bits = h, sign = h & 0x8000;
    uint32_t exp = (bits >> 10) & 0x1f;
    uint32_t mant = (bits & 0x3ff) | ((uint32_t)(exp != 0) << 10);
    float scale = of_bits(((exp > 1 ? exp : 1) + 127 - 25) << 23);
    float mag = (float)mant * scale;
    return of_bits(bits_of(mag) | (sign << 16));
}

/* gpu/tests.rs:45-54: s = s*6364136223846793005 + 1442695040888963407,
 * value = (s >> 40) / 2^24 * 2 - 1. */
float or_rng_next(or_rng *r) {
    r->s = r->s * 6364136223846793005ull + 1442695040888963407ull;
    return ((float)(r->s >> 40) / (float)(1ull << 24)) * 2.0f - 1.0f;
}

void or_rng_floats(uint64_t *state, float *out, size_t n) {
    or_rng r = {*state};
    for (size_t i = 0; i < n; i++) out[i] = or_rng_next(&r);
    *state = r.s;
}

/* gpu/tests.rs:60-68: the top half of each value's bits (truncation). */
void or_rng_bf16(uint64_t *state, uint16_t *out, size_t n) {
    or_rng r = {*state};
    for (size_t i = 0; i < n; i++) out[i] = (uint16_t)(bits_of(or_rng_next(&r)) >> 16);
    *state = r.s;
}

/* gpu/quant.rs:161-180: the cache quantizer, scale = f16(amax/127), each value
 * the nearest multiple, ties away from zero, settled against exact midpoints. */
void or_quantize(const float *block, uint16_t *scale, int8_t *q) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(block[i]));
    uint16_t bits = or_to_f16(amax * (1.0f / 127.0f));
    float d = or_from_f16(bits);
    for (int i = 0; i < 32; i++) q[i] = 0;
    if (d > 0.0f) {
        for (int i = 0; i < 32; i++) {
            float x = block[i];
            float a = fabsf(x);
            float n = fminf(roundf(a / d), 128.0f);
            if (a >= (n + 0.5f) * d) {
                n += 1.0f;
            } else if (n > 0.0f && a < (n - 0.5f) * d) {
                n -= 1.0f;
            }
            int8_t v = (int8_t)fminf(n, 127.0f);
            q[i] = (int8_t)(v * (x < 0.0f ? -1 : 1));
        }
    }
    *scale = bits;
}

/* gpu/quant.rs:34-46 */
void or_quantize_q8_0_row(const float *x, size_t cols, uint16_t *scales, int8_t *quants) {
    for (size_t b = 0; b < cols / 32; b++) or_quantize(x + 32 * b, scales + b, quants + 32 * b);
}

/* gpu/quant.rs:49-62 */
void or_dequantize_q8_0_row(const uint16_t *scales, const int8_t *quants, size_t cols, float *out) {
    for (size_t b = 0; b < cols / 32; b++) {
        float d = or_from_f16(scales[b]);
        for (int i = 0; i < 32; i++) out[32 * b + i] = (float)quants[32 * b + i] * d;
    }
}

/* Rust's `Sum` for f32 folds from -0.0. */
static inline float sum8(const float *s) {
    float t = -0.0f;
    for (int i = 0; i < 8; i++) t += s[i];
    return t;
}

/* gpu/quant.rs:65-83: 8 lanes per block, the block's scale applied to their sum. */
float or_dot_q8_0(const uint16_t *scales, const int8_t *quants, const float *x, size_t cols) {
    float acc = 0.0f;
    for (size_t b = 0; b < cols / 32; b++) {
        float sum[8] = {0};
        const int8_t *q = quants + 32 * b;
        const float *xb = x + 32 * b;
        for (int c = 0; c < 4; c++)
            for (int i = 0; i < 8; i++) sum[i] += (float)q[8 * c + i] * xb[8 * c + i];
        acc += or_from_f16(scales[b]) * sum8(sum);
    }
    return acc;
}

/* gpu/quant.rs:89-109: scale = the weight of largest magnitude over -8. */
void or_quantize_q4_0_row(const float *x, size_t cols, uint16_t *scales, uint8_t *quants) {
    for (size_t b = 0; b < cols / 32; b++) {
        const float *blk = x + 32 * b;
        float max = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(blk[i]) > fabsf(max)) max = blk[i];
        float d = max / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        scales[b] = or_to_f16(d);
        for (int j = 0; j < 16; j++) {
            float lo = fminf(fmaxf(blk[j] * id + 8.5f, 0.0f), 15.0f);
            float hi = fminf(fmaxf(blk[j + 16] * id + 8.5f, 0.0f), 15.0f);
            quants[16 * b + j] = (uint8_t)((uint8_t)lo | ((uint8_t)hi << 4));
        }
    }
}

/* gpu/quant.rs:112-126 */
void or_dequantize_q4_0_row(const uint16_t *scales, const uint8_t *quants, size_t cols, float *out) {
    for (size_t b = 0; b < cols / 32; b++) {
        float d = or_from_f16(scales[b]);
        for (int j = 0; j < 16; j++) {
            uint8_t q = quants[16 * b + j];
            out[32 * b + j] = ((float)(q & 0xf) - 8.0f) * d;
            out[32 * b + j + 16] = ((float)(q >> 4) - 8.0f) * d;
        }
    }
}

/* gpu/quant.rs:129-152 */
float or_dot_q4_0(const uint16_t *scales, const uint8_t *quants, const float *x, size_t cols) {
    float acc = 0.0f;
    for (size_t b = 0; b < cols / 32; b++) {
        const uint8_t *q = quants + 16 * b;
        const float *lo = x + 32 * b, *hi = x + 32 * b + 16;
        float sum[8] = {0};
        for (int c = 0; c < 2; c++)
            for (int i = 0; i < 8; i++) {
                uint8_t v = q[8 * c + i];
                sum[i] += ((float)(v & 0xf) - 8.0f) * lo[8 * c + i] +
                          ((float)(v >> 4) - 8.0f) * hi[8 * c + i];
            }
        acc += or_from_f16(scales[b]) * sum8(sum);
    }
    return acc;
}

/* gpu/cpu.rs:370-386: 8 independent sums, then the tail. */
float or_dot_bf16(const uint16_t *w, const float *x, size_t cols) {
    float acc[8] = {0};
    size_t done = cols / 8 * 8;
    for (size_t c = 0; c < done; c += 8)
        for (int i = 0; i < 8; i++) acc[i] += or_bf16(w[c + i]) * x[c + i];
    float rest = -0.0f;
    for (size_t c = done; c < cols; c++) rest += or_bf16(w[c]) * x[c];
    return sum8(acc) + rest;
}

/* inference/quants.rs:44-57 */
void or_dequantize_q4_1_file(const uint8_t *row, size_t cols, float *out) {
    for (size_t b = 0; b < cols / 32; b++) {
        const uint8_t *blk = row + 20 * b;
        float d = or_from_f16((uint16_t)(blk[0] | blk[1] << 8));
        float m = or_from_f16((uint16_t)(blk[2] | blk[3] << 8));
        for (int j = 0; j < 16; j++) {
            uint8_t q = blk[4 + j];
            out[32 * b + j] = (float)(q & 0xf) * d + m;
            out[32 * b + j + 16] = (float)(q >> 4) * d + m;
        }
    }
}

/* inference/quants.rs:79-104: ql[128] | qh[64] | scales i8[16] | d f16.  Weight
 * l + 32k of a half comes from nibble k/2 of low byte l + 32(k%2), bits 2k..2k+1
 * of high byte l, scale 2k + l/16. */
void or_dequantize_q6_k_file(const uint8_t *row, size_t cols, float *out) {
    for (size_t b = 0; b < cols / 256; b++) {
        const uint8_t *blk = row + 210 * b;
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = or_from_f16((uint16_t)(blk[208] | blk[209] << 8));
        for (int half = 0; half < 2; half++) {
            float *o = out + 256 * b + 128 * half;
            for (int l = 0; l < 32; l++)
                for (int k = 0; k < 4; k++) {
                    int low = (ql[64 * half + l + 32 * (k % 2)] >> (4 * (k / 2))) & 0xf;
                    int high = (qh[32 * half + l] >> (2 * k)) & 3;
                    int q = (low | high << 4) - 32;
                    o[l + 32 * k] = d * (float)sc[8 * half + 2 * k + l / 16] * (float)q;
                }
        }
    }
}

/* Q6_K, 16 weights per scale: group s of a block is weights 16s..16s+15 (the
 * layout above makes each scale's 16 weights consecutive). */
static inline int q6_k_value(const uint8_t *blk, int i) {
    int half = i / 128, r = i % 128, k = r / 32, l = r % 32;
    int low = (blk[64 * half + l + 32 * (k % 2)] >> (4 * (k / 2))) & 0xf;
    int high = (blk[128 + 32 * half + l] >> (2 * k)) & 3;
    return (low | high << 4) - 32;
}

/* Dot of a Q6_K row with f32 activations, shaped as dot_q4_0 is: per scale
 * group, 8-lane sums of q·x, then (d·scale)·sum added to the total. */
float or_dot_q6_k(const uint8_t *blocks, const float *x, size_t cols) {
    float acc = 0.0f;
    for (size_t b = 0; b < cols / 256; b++) {
        const uint8_t *blk = blocks + 210 * b;
        const int8_t *sc = (const int8_t *)(blk + 192);
        float d = or_from_f16((uint16_t)(blk[208] | blk[209] << 8));
        for (int s = 0; s < 16; s++) {
            float sum[8] = {0};
            for (int c = 0; c < 2; c++)
                for (int i = 0; i < 8; i++) {
                    int w = 16 * s + 8 * c + i;
                    sum[i] += (float)q6_k_value(blk, w) * x[256 * b + w];
                }
            acc += d * (float)sc[s] * sum8(sum);
        }
    }
    return acc;
}

/* Q6_K quantizer: each group of 16 takes the weight of largest magnitude,
 * sign and all, to -32 of its scale (as Q4_0 takes its to -8); the block's d
 * is the largest group scale over 127 in f16, each group's scale the integer
 * multiple of d next away from zero (so the group still fits), and each weight the nearest multiple of d·scale in
 * [-32, 31]. */
void or_quantize_q6_k_row(const float *x, size_t cols, uint8_t *blocks) {
    for (size_t b = 0; b < cols / 256; b++) {
        const float *xb = x + 256 * b;
        uint8_t *blk = blocks + 210 * b;
        memset(blk, 0, 210);
        float gs[16];
        float amax = 0.0f;
        for (int s = 0; s < 16; s++) {
            float max = 0.0f;
            for (int i = 0; i < 16; i++)
                if (fabsf(xb[16 * s + i]) > fabsf(max)) max = xb[16 * s + i];
            gs[s] = max / -32.0f;
            amax = fmaxf(amax, fabsf(gs[s]));
        }
        uint16_t dbits = or_to_f16(amax / 127.0f);
        if (or_from_f16(dbits) * 127.0f < amax) dbits++; /* next half up: 127·d covers amax */
        float d = or_from_f16(dbits);
        blk[208] = (uint8_t)(dbits & 0xff);
        blk[209] = (uint8_t)(dbits >> 8);
        for (int s = 0; s < 16; s++) {
            int sc = 0;
            if (d > 0.0f) {
                /* rounded away from zero, so that d·scale covers the group */
                float r = ceilf(fabsf(gs[s]) / d);
                sc = (int)fminf(r, 127.0f) * (gs[s] < 0.0f ? -1 : 1);
            }
            blk[192 + s] = (uint8_t)(int8_t)sc;
            float ds = d * (float)sc;
            for (int i = 0; i < 16; i++) {
                int w = 16 * s + i;
                int q = 0;
                if (ds != 0.0f) {
                    float r = rintf(xb[w] / ds);
                    q = (int)fminf(fmaxf(r, -32.0f), 31.0f);
                }
                int u = q + 32;
                int half = w / 128, rr = w % 128, k = rr / 32, l = rr % 32;
                blk[64 * half + l + 32 * (k % 2)] |= (uint8_t)((u & 0xf) << (4 * (k / 2)));
                blk[128 + 32 * half + l] |= (uint8_t)(((u >> 4) & 3) << (2 * k));
            }
        }
    }
}

/* ggml get_scale_min_k4: sub-blocks 0-3 keep 6-bit scale and min in bytes j and
 * j+4; sub-blocks 4-7 keep their low 4 bits in byte j+4 (scale low nibble, min
 * high nibble) and their top 2 bits in the top bits of bytes j-4 and j. */
void or_q4_k_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* block_q4_K: d f16 | dmin f16 | scales[12] | qs[128]; weight 32j+l of the
 * block is nibble (j%2) of qs[32(j/2)+l], and equals d·sc_j·q − dmin·m_j. */
void or_dequantize_q4_k_row(const uint8_t *blocks, size_t cols, float *out) {
    for (size_t b = 0; b < cols / 256; b++) {
        const uint8_t *blk = blocks + 144 * b;
        float d = or_from_f16((uint16_t)(blk[0] | blk[1] << 8));
        float dmin = or_from_f16((uint16_t)(blk[2] | blk[3] << 8));
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            or_q4_k_scale_min(j, blk + 4, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            for (int l = 0; l < 32; l++) {
                uint8_t byte = blk[16 + 32 * (j / 2) + l];
                int q = (j % 2) ? (byte >> 4) : (byte & 0xf);
                out[256 * b + 32 * j + l] = d1 * (float)q - m1;
            }
        }
    }
}

/* Dot of a Q4_K row with f32 activations: per sub-block of 32, 8-lane sums of
 * q·x and of x, then d1·Σqx − m1·Σx added to the total (the min folded out of
 * the sum, as dot_q4_0 folds its scale out). */
float or_dot_q4_k(const uint8_t *blocks, const float *x, size_t cols) {
    float acc = 0.0f;
    for (size_t b = 0; b < cols / 256; b++) {
        const uint8_t *blk = blocks + 144 * b;
        float d = or_from_f16((uint16_t)(blk[0] | blk[1] << 8));
        float dmin = or_from_f16((uint16_t)(blk[2] | blk[3] << 8));
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            or_q4_k_scale_min(j, blk + 4, &sc, &m);
            float d1 = d * (float)sc, m1 = dmin * (float)m;
            const float *xs = x + 256 * b + 32 * j;
            float sq[8] = {0}, sx[8] = {0};
            for (int c = 0; c < 4; c++)
                for (int i = 0; i < 8; i++) {
                    int l = 8 * c + i;
                    uint8_t byte = blk[16 + 32 * (j / 2) + l];
                    int q = (j % 2) ? (byte >> 4) : (byte & 0xf);
                    sq[i] += (float)q * xs[l];
                    sx[i] += xs[l];
                }
            acc += d1 * sum8(sq) - m1 * sum8(sx);
        }
    }
    return acc;
}

/* Q4_K quantizer: each sub-block of 32 maps [min(0, lo), hi] onto 0..15, so its
 * scale is (hi − min(0, lo))/15 and its min −min(0, lo); the block's d and dmin
 * are the largest of these over 63, in f16, each sub-block's 6-bit multiple of
 * them the nearest (ties to even), and each weight q = nearest((x + m1)/d1) in
 * 0..15 for the d1, m1 the block decodes to. */
void or_quantize_q4_k_row(const float *x, size_t cols, uint8_t *blocks) {
    for (size_t b = 0; b < cols / 256; b++) {
        const float *xb = x + 256 * b;
        uint8_t *blk = blocks + 144 * b;
        memset(blk, 0, 144);
        float scale[8], mins[8], max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = xb[32 * j];
            for (int l = 0; l < 32; l++) {
                lo = fminf(lo, xb[32 * j + l]);
                hi = fmaxf(hi, xb[32 * j + l]);
            }
            scale[j] = (hi - lo) / 15.0f;
            mins[j] = 0.0f - lo; /* +0, not -0, when no weight is negative */
            max_scale = fmaxf(max_scale, scale[j]);
            max_min = fmaxf(max_min, mins[j]);
        }
        uint16_t dbits = or_to_f16(max_scale / 63.0f);
        uint16_t mbits = or_to_f16(max_min / 63.0f);
        float d = or_from_f16(dbits), dmin = or_from_f16(mbits);
        uint8_t sc[8], mm[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = d > 0.0f ? (uint8_t)fminf(fmaxf(rintf(scale[j] / d), 0.0f), 63.0f) : 0;
            mm[j] = dmin > 0.0f ? (uint8_t)fminf(fmaxf(rintf(mins[j] / dmin), 0.0f), 63.0f) : 0;
        }
        blk[0] = (uint8_t)(dbits & 0xff);
        blk[1] = (uint8_t)(dbits >> 8);
        blk[2] = (uint8_t)(mbits & 0xff);
        blk[3] = (uint8_t)(mbits >> 8);
        uint8_t *s = blk + 4;
        for (int j = 0; j < 8; j++) {
            if (j < 4) {
                s[j] = sc[j];
                s[j + 4] = mm[j];
            } else {
                s[j + 4] = (uint8_t)((sc[j] & 0xf) | ((mm[j] & 0xf) << 4));
                s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
                s[j] |= (uint8_t)((mm[j] >> 4) << 6);
            }
        }
        for (int j = 0; j < 8; j++) {
            float d1 = d * (float)sc[j], m1 = dmin * (float)mm[j];
            for (int l = 0; l < 32; l++) {
                int q = 0;
                if (d1 > 0.0f) {
                    float r = rintf((xb[32 * j + l] + m1) / d1);
                    q = (int)fminf(fmaxf(r, 0.0f), 15.0f);
                }
                blk[16 + 32 * (j / 2) + l] |= (uint8_t)(q << (4 * (j % 2)));
            }
        }
    }
}
