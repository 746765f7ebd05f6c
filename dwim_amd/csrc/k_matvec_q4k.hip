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

template <int T>
__global__ void __launch_bounds__(kMaxS * 64) k_mv_q4kt(const uint8_t *__restrict__ wq, size_t rows, size_t nb,
                                                        const float *__restrict__ x, float *out, int add,
                                                        uint32_t lo_mask, uint32_t hi_mask) {
    __shared__ float red[kMaxS][T][16];
    const int S = (int)(blockDim.x >> 6);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const size_t tile = blockIdx.x;
    const size_t cols = nb * 256;
    const size_t b0 = (size_t)wave * nb / S, b1 = (size_t)(wave + 1) * nb / S;
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
            const float *xb = x + t * cols + b * 256 + 64 * g;
            // sub-block sums: lane r adds x[4r..4r+3] of the group's 64;
            // lanes 0-7 make sub-block 2g, lanes 8-15 sub-block 2g+1
            const float4 x4 = *(const float4 *)(xb + 4 * r);
            const float own = group_sum<8>((x4.x + x4.y) + (x4.z + x4.w));
            const float other = __shfl_xor(own, 8, 64);
            const float xs_lo = r < 8 ? own : other, xs_hi = r < 8 ? other : own;
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
    size_t t = 0;
    while (t < n) {
        const size_t left = n - t;
        const float *xt = x + t * w->cols;
        float *ot = out + t * w->rows;
        if (left >= 4) {
            k_mv_q4kt<4><<<(unsigned)tiles, threads, 0, s>>>(wq, w->rows, nb, xt, ot, add, lo, hi);
            t += 4;
        } else if (left >= 2) {
            k_mv_q4kt<2><<<(unsigned)tiles, threads, 0, s>>>(wq, w->rows, nb, xt, ot, add, lo, hi);
            t += 2;
        } else {
            k_mv_q4kt<1><<<(unsigned)tiles, threads, 0, s>>>(wq, w->rows, nb, xt, ot, add, lo, hi);
            t += 1;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
