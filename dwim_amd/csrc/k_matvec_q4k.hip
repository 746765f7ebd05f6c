// Q4_K matrix-vector products for decode and small batches (T ≤ 4 tokens per
// pass): out[t][r] (+)= w[r] · x[t] (dwim gpu/cpu.rs:110-149), f32
// activations, f32 arithmetic, the dequantized weights used exactly.
//
// The weights are in the tiled layout of layout.h.  A workgroup of S waves
// owns a tile of 16 rows: lane 16g + r of a wave takes 32-byte quant group g
// (sub-blocks 2g and 2g+1, 64 weights) of row r, and wave w takes the tile's
// blocks (256 columns) b ∈ [w·nb/S, (w+1)·nb/S), about five of them, so that a
// launch has thousands of waves.  Per block a lane makes three 16-byte weight
// loads (a quarter-wave's load is 256 contiguous bytes) and reads its 64
// activations through L1 (a wave touches four 256-byte runs of x).  The
// sub-block sums of x (for the folded-out mins) come from one float4 per lane
// and a reduction over 8 lanes.  The four lanes of a row meet by shuffles and
// the S waves in LDS, in a fixed order: results are deterministic.
//
// Per weight: one v_cvt_f32_ubyte (low nibbles from w & 0x0f0f0f0f, high ones
// from w & 0xf0f0f0f0 as 16·q, their scale divided by 16) and one v_fmac.
// Per sub-block of 32: out += d1·Σq·x − m1·Σx (the weight is d1·q − m1).
#include "device_util.h"
#include "layout.h"
#include "quant_math.h"
#include "runtime.h"

namespace {

constexpr int kMaxS = 16;
constexpr int kBlocksPerWave = 5;

DEV float ub0(uint32_t v) { return (float)(v & 0xffu); }
DEV float ub1(uint32_t v) { return (float)((v >> 8) & 0xffu); }
DEV float ub2(uint32_t v) { return (float)((v >> 16) & 0xffu); }
DEV float ub3(uint32_t v) { return (float)(v >> 24); }

// the 6-bit scale and min of sub-block j from the header's scale words
// (ggml get_scale_min_k4); y, z, w hold scale bytes 0-3, 4-7, 8-11
DEV void scale_min(const uint4 &m, int j, float &sc, float &mn) {
    const int sh = 8 * (j & 3);
    const uint32_t a = (m.y >> sh) & 0xffu, bz = (m.z >> sh) & 0xffu, c = (m.w >> sh) & 0xffu;
    if (j < 4) {
        sc = (float)(a & 63u);
        mn = (float)(bz & 63u);
    } else {
        sc = (float)((c & 0xfu) | ((a >> 6) << 4));
        mn = (float)((c >> 4) | ((bz >> 6) << 4));
    }
}

// Σ nibble·x over one 16-byte quant chunk (4 words): low nibbles against
// xl[0..15], high nibbles (as 16·q) against xh[0..15]
DEV void chunk_dot(const uint4 &q, const float *xl, const float *xh, uint32_t lo_mask, uint32_t hi_mask, float &sl,
                   float &sh) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t lo = w[k] & lo_mask, hi = w[k] & hi_mask;
        sl += ub0(lo) * xl[4 * k];
        sl += ub1(lo) * xl[4 * k + 1];
        sl += ub2(lo) * xl[4 * k + 2];
        sl += ub3(lo) * xl[4 * k + 3];
        sh += ub0(hi) * xh[4 * k];
        sh += ub1(hi) * xh[4 * k + 1];
        sh += ub2(hi) * xh[4 * k + 2];
        sh += ub3(hi) * xh[4 * k + 3];
    }
}

DEV void load16f(const float *p, float *dst) {
#pragma unroll
    for (int k = 0; k < 16; k += 4) *(float4 *)(dst + k) = *(const float4 *)(p + k);
}

// LDS image of the activations: position p at p + 4·(p / 64) (the four
// 64-float runs a wave reads at once start on different banks), per token,
// then the tokens' sub-block sums.
__host__ __device__ inline size_t xpad(size_t p) { return p + 4 * (p >> 6); }
__host__ __device__ inline size_t xlds_floats(size_t cols) { return xpad(cols); }

template <int T>
__global__ void __launch_bounds__(kMaxS * 64) k_mv_q4kt(const uint8_t *__restrict__ wq, size_t rows, size_t nb,
                                                        const float *__restrict__ xg, float *out, int add,
                                                        uint32_t lo_mask, uint32_t hi_mask) {
    extern __shared__ float xl_s[];
    __shared__ float red[kMaxS][T][16];
    const int S = (int)(blockDim.x >> 6);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const size_t tile = blockIdx.x;
    const size_t cols = nb * 256, per_tok = xlds_floats(cols), sbs = cols / 32;
    const size_t b0 = (size_t)wave * nb / S, b1 = (size_t)(wave + 1) * nb / S;
    float *xsum_s = xl_s + T * per_tok;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.0f;
    // every weight load of the wave goes out before any arithmetic: one
    // memory round trip per wave, not one per block
    uint4 mm[kBlocksPerWave], qq0[kBlocksPerWave], qq1[kBlocksPerWave];
#pragma unroll
    for (int i = 0; i < kBlocksPerWave; i++) {
        const size_t b = b0 + i < b1 ? b0 + i : b0;
        const uint8_t *u = wq + q4kt::unit(tile, b, nb);
        mm[i] = *(const uint4 *)(u + q4kt::meta_off(r));
        qq0[i] = *(const uint4 *)(u + q4kt::qs_off(g, 0, r));
        qq1[i] = *(const uint4 *)(u + q4kt::qs_off(g, 1, r));
    }
    // the activations into LDS while the weights are on their way, then each
    // sub-block's sum
    const int nthreads = (int)blockDim.x;
    for (size_t i = threadIdx.x * 4; i < T * cols; i += (size_t)nthreads * 4) {
        const size_t t = i / cols, p = i % cols;
        *(float4 *)(xl_s + t * per_tok + xpad(p)) = *(const float4 *)(xg + i);
    }
    __syncthreads();
    for (size_t i = threadIdx.x; i < T * sbs; i += nthreads) {
        const size_t t = i / sbs, sb = i % sbs;
        const float *p = xl_s + t * per_tok + xpad(sb * 32);
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 32; k += 4) {
            const float4 v = *(const float4 *)(p + k);
            s += (v.x + v.y) + (v.z + v.w);
        }
        xsum_s[i] = s;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kBlocksPerWave; i++) {
        const size_t b = b0 + i;
        if (b >= b1) break;
        const uint4 m = mm[i], q0 = qq0[i], q1 = qq1[i];
        const float d = dq::from_f16((uint16_t)(m.x & 0xffffu)), dmin = dq::from_f16((uint16_t)(m.x >> 16));
        float sc1, mn1, sc2, mn2;
        scale_min(m, 2 * g, sc1, mn1);
        scale_min(m, 2 * g + 1, sc2, mn2);
        const float d1 = d * sc1, m1 = dmin * mn1;
        const float d2 = (d * sc2) * 0.0625f, m2 = dmin * mn2;  // high nibbles arrive as 16·q
#pragma unroll
        for (int t = 0; t < T; t++) {
            // the group's 64 activations are one padded run of the LDS image
            const float *xb = xl_s + t * per_tok + xpad(b * 256 + 64 * g);
            const float xs_lo = xsum_s[t * sbs + b * 8 + 2 * g], xs_hi = xsum_s[t * sbs + b * 8 + 2 * g + 1];
            float sl = 0.0f, sh = 0.0f;
            float xl[16], xh[16];
            load16f(xb, xl);
            load16f(xb + 32, xh);
            chunk_dot(q0, xl, xh, lo_mask, hi_mask, sl, sh);
            load16f(xb + 16, xl);
            load16f(xb + 48, xh);
            chunk_dot(q1, xl, xh, lo_mask, hi_mask, sl, sh);
            acc[t] += d1 * sl - m1 * xs_lo + d2 * sh - m2 * xs_hi;
        }
    }
    // the row's four groups, then the waves
#pragma unroll
    for (int t = 0; t < T; t++) {
        float v = acc[t];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        if (g == 0) red[wave][t][r] = v;
    }
    __syncthreads();
    const size_t row = tile * 16 + r;
    if (wave == 0 && g == 0 && row < rows) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            float v = 0.0f;
            for (int w = 0; w < S; w++) v += red[w][t][r];
            float *o = out + t * rows + row;
            *o = add ? *o + v : v;
        }
    }
}

}  // namespace

hipError_t launch_matvec_q4k(hipStream_t s, const dwim_weight *w, float *out, const float *x, size_t n, int add) {
    const size_t nb = w->cols / 256, tiles = q4kt::tiles(w->rows);
    // waves per tile: about kBlocksPerWave blocks each, at most kMaxS
    size_t waves = (nb + kBlocksPerWave - 1) / kBlocksPerWave;
    if (waves > (size_t)kMaxS) return hipErrorInvalidValue;  // rows of at most 80 blocks (checked at upload)
    const unsigned threads = (unsigned)(waves * 64);
    const uint8_t *wq = (const uint8_t *)w->q;
    const uint32_t lo = 0x0f0f0f0fu, hi = 0xf0f0f0f0u;
    const size_t sbs = w->cols / 32;
    auto lds_of = [&](size_t tt) { return (tt * xlds_floats(w->cols) + tt * sbs) * sizeof(float); };
    constexpr size_t kLdsMax = 144 * 1024;  // of gfx950's 160 KB, beside the 4 KB reduction
    static bool raised[3] = {false, false, false};
    size_t t = 0;
    while (t < n) {
        const size_t left = n - t;
        size_t tt = left >= 4 && lds_of(4) <= kLdsMax ? 4 : left >= 2 && lds_of(2) <= kLdsMax ? 2 : 1;
        const size_t lds = lds_of(tt);
        const int idx = tt == 4 ? 2 : tt == 2 ? 1 : 0;
        const void *fn = tt == 4 ? (const void *)k_mv_q4kt<4> : tt == 2 ? (const void *)k_mv_q4kt<2>
                                                                          : (const void *)k_mv_q4kt<1>;
        if (lds > 64 * 1024 && !raised[idx]) {
            hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
            if (e != hipSuccess) return e;
            raised[idx] = true;
        }
        const float *xt = x + t * w->cols;
        float *ot = out + t * w->rows;
        if (tt == 4)
            k_mv_q4kt<4><<<(unsigned)tiles, threads, lds, s>>>(wq, w->rows, nb, xt, ot, add, lo, hi);
        else if (tt == 2)
            k_mv_q4kt<2><<<(unsigned)tiles, threads, lds, s>>>(wq, w->rows, nb, xt, ot, add, lo, hi);
        else
            k_mv_q4kt<1><<<(unsigned)tiles, threads, lds, s>>>(wq, w->rows, nb, xt, ot, add, lo, hi);
        t += tt;
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
