// Scalar quantization arithmetic shared by the host quantizers and the device
// kernels (cache store, synthetic weights), so that both produce the same bits.
// Every function is a fixed sequence of IEEE f32 operations (no fused
// multiply-add: contraction is switched off below), integer operations and
// rint/round, which gfx950 and x86-64 compute identically.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DQ_HD __host__ __device__ __forceinline__

namespace dq {

DQ_HD uint32_t bits_of(float x) { return __builtin_bit_cast(uint32_t, x); }
DQ_HD float of_bits(uint32_t u) { return __builtin_bit_cast(float, u); }

constexpr float kF16Max = 65504.0f;

// f32 -> nearest IEEE half, ties to even, clamped to ±65504
// (dwim gpu/float.rs:15-29: subnormals as multiples of 2^-24, normals by
// scaling the mantissa to [1024, 2048) and rounding).
DQ_HD uint16_t to_f16(float x) {
#pragma clang fp contract(off)
    uint16_t sign = (uint16_t)((bits_of(x) >> 16) & 0x8000u);
    float a = fminf(fabsf(x), kF16Max);
    if (a < of_bits((uint32_t)(127 - 14) << 23)) return (uint16_t)(sign | (uint16_t)rintf(a * 16777216.0f));
    int e = (int)((bits_of(a) >> 23) & 0xffu) - 127;
    uint32_t m = (uint32_t)rintf(a * of_bits((uint32_t)(127 + 10 - e) << 23));
    if (m == 2048u) { e += 1; m = 1024u; }
    return (uint16_t)(sign | (uint16_t)((e + 15) << 10) | (uint16_t)(m - 1024u));
}

// IEEE half bits -> f32, exact (gpu/float.rs:39-48).
DQ_HD float from_f16(uint16_t h) {
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, s = (uint32_t)(h & 0x8000u) << 16;
    if (e == 0) {
        // subnormal: m * 2^-24, exact in f32
        return of_bits(bits_of((float)m * 5.9604644775390625e-8f) | s);
    }
    return of_bits(s | ((e + 112u) << 23) | (m << 13));
}

DQ_HD float bf16_to_f32(uint16_t b) { return of_bits((uint32_t)b << 16); }

// The cache quantizer for 32 activations (gpu/quant.rs:161-180): scale =
// f16(amax/127); each value the nearest multiple of it, ties away from zero,
// the multiple settled by comparing with midpoints (exact products of a
// 9-bit and an 11-bit number), so an inexact quotient cannot change it.
DQ_HD int8_t quantize_one(float x, float d) {
#pragma clang fp contract(off)
    float a = fabsf(x);
    float n = fminf(roundf(a / d), 128.0f);
    if (a >= (n + 0.5f) * d) n += 1.0f;
    else if (n > 0.0f && a < (n - 0.5f) * d) n -= 1.0f;
    int v = (int)fminf(n, 127.0f);
    return (int8_t)(x < 0.0f ? -v : v);
}

DQ_HD uint16_t block_scale(float amax) {
#pragma clang fp contract(off)
    return to_f16(amax * (1.0f / 127.0f));
}

// ggml get_scale_min_k4: the 6-bit scale and min of sub-block j of a Q4_K
// block from its 12 packed bytes.
DQ_HD void q4k_scale_min(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Q4_K quantizer for one block of 256 (the product's own, format of ggml's
// block_q4_K): each sub-block of 32 maps [min(0, lo), hi] onto 0..15; d and
// dmin are the largest sub-block scale and min over 63, in f16; each
// sub-block's 6-bit multiples of them the nearest; each weight
// q = nearest((x + m1)/d1) in 0..15.  Writes 144 bytes: d, dmin, scales[12], qs[128].
DQ_HD void quantize_q4_k_block(const float *x, uint8_t *blk) {
#pragma clang fp contract(off)
    float scale[8], mins[8], max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = 0.0f, hi = x[32 * j];
        for (int l = 0; l < 32; l++) {
            lo = fminf(lo, x[32 * j + l]);
            hi = fmaxf(hi, x[32 * j + l]);
        }
        scale[j] = (hi - lo) / 15.0f;
        mins[j] = 0.0f - lo;
        max_scale = fmaxf(max_scale, scale[j]);
        max_min = fmaxf(max_min, mins[j]);
    }
    uint16_t dbits = to_f16(max_scale / 63.0f), mbits = to_f16(max_min / 63.0f);
    float d = from_f16(dbits), dmin = from_f16(mbits);
    int sc[8], mm[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0.0f ? (int)fminf(fmaxf(rintf(scale[j] / d), 0.0f), 63.0f) : 0;
        mm[j] = dmin > 0.0f ? (int)fminf(fmaxf(rintf(mins[j] / dmin), 0.0f), 63.0f) : 0;
    }
    blk[0] = (uint8_t)(dbits & 0xff);
    blk[1] = (uint8_t)(dbits >> 8);
    blk[2] = (uint8_t)(mbits & 0xff);
    blk[3] = (uint8_t)(mbits >> 8);
    uint8_t s[12] = {0};
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            s[j] |= (uint8_t)sc[j];
            s[j + 4] |= (uint8_t)mm[j];
        } else {
            s[j + 4] = (uint8_t)((sc[j] & 0xf) | ((mm[j] & 0xf) << 4));
            s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s[j] |= (uint8_t)((mm[j] >> 4) << 6);
        }
    }
    for (int i = 0; i < 12; i++) blk[4 + i] = s[i];
    for (int g = 0; g < 4; g++) {
        float d1 = d * (float)sc[2 * g], m1 = dmin * (float)mm[2 * g];
        float d2 = d * (float)sc[2 * g + 1], m2 = dmin * (float)mm[2 * g + 1];
        for (int l = 0; l < 32; l++) {
            int q1 = 0, q2 = 0;
            if (d1 > 0.0f) q1 = (int)fminf(fmaxf(rintf((x[64 * g + l] + m1) / d1), 0.0f), 15.0f);
            if (d2 > 0.0f) q2 = (int)fminf(fmaxf(rintf((x[64 * g + 32 + l] + m2) / d2), 0.0f), 15.0f);
            blk[16 + 32 * g + l] = (uint8_t)(q1 | (q2 << 4));
        }
    }
}

// Q6_K quantizer for one block of 256 (format of ggml's block_q6_K, as dwim
// inference/quants.rs:79-104 reads it): group s of 16 consecutive weights
// takes its weight of largest magnitude, sign and all, to -32 of its scale;
// d = f16 of the largest group scale over 127, nudged up one half-ulp step
// until 127·d covers it; each group's int8 scale the multiple of d next away
// from zero; each weight the nearest multiple of d·scale in [-32, 31].
// Writes 210 bytes: ql[128], qh[64], scales[16], d.
DQ_HD void quantize_q6_k_block(const float *x, uint8_t *blk) {
#pragma clang fp contract(off)
    for (int i = 0; i < 210; i++) blk[i] = 0;
    float gs[16], amax = 0.0f;
    for (int s = 0; s < 16; s++) {
        float max = 0.0f;
        for (int i = 0; i < 16; i++)
            if (fabsf(x[16 * s + i]) > fabsf(max)) max = x[16 * s + i];
        gs[s] = max / -32.0f;
        amax = fmaxf(amax, fabsf(gs[s]));
    }
    uint16_t dbits = to_f16(amax / 127.0f);
    if (from_f16(dbits) * 127.0f < amax) dbits++;
    float d = from_f16(dbits);
    blk[208] = (uint8_t)(dbits & 0xff);
    blk[209] = (uint8_t)(dbits >> 8);
    for (int s = 0; s < 16; s++) {
        int sc = 0;
        if (d > 0.0f) {
            float r = ceilf(fabsf(gs[s]) / d);
            sc = (int)fminf(r, 127.0f) * (gs[s] < 0.0f ? -1 : 1);
        }
        blk[192 + s] = (uint8_t)(int8_t)sc;
        float ds = d * (float)sc;
        for (int i = 0; i < 16; i++) {
            int w = 16 * s + i, q = 0;
            if (ds != 0.0f) q = (int)fminf(fmaxf(rintf(x[w] / ds), -32.0f), 31.0f);
            int u = q + 32;
            int half = w / 128, rr = w % 128, k = rr / 32, l = rr % 32;
            blk[64 * half + l + 32 * (k % 2)] |= (uint8_t)((u & 0xf) << (4 * (k / 2)));
            blk[128 + 32 * half + l] |= (uint8_t)(((u >> 4) & 3) << (2 * k));
        }
    }
}

// SplitMix64 at position i of stream `seed`: a counter-based hash.
DQ_HD uint64_t splitmix(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// An approximately normal value: the centred sum of the hash's four 16-bit
// fields (mean 131070, standard deviation 65536/sqrt(3)) times `c`, which the
// caller sets to sigma·sqrt(3)/65536.  Integer steps and one f32 multiply.
DQ_HD float synthetic(uint64_t seed, uint64_t i, float c) {
    uint64_t h = splitmix(seed, i);
    int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
                (int32_t)(h >> 48);
    return (float)(s - 131070) * c;
}

}  // namespace dq
