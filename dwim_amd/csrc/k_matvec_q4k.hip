// Q4_K matrix-vector products for decode and small batches (T ≤ 4 tokens per
// pass): out[t][r] (+)= w[r] · x[t] (dwim gpu/cpu.rs:110-149), f32
// activations, f32 arithmetic, the dequantized weights used exactly.
//
// The weights are in the tiled layout of layout.h.  A workgroup of S waves
// owns a tile of 16 rows: lane 16g + r of a wave takes 32-byte quant group g
// (sub-blocks 2g and 2g+1, 64 weights) of row r, and wave w takes the tile's
// blocks (256 columns) b ∈ [w·nb/S, (w+1)·nb/S), at most five, so that a
// launch has thousands of waves.  A wave issues all its weight loads (three
// 16-byte loads per block; a quarter-wave's load is 256 contiguous bytes)
// before anything else; meanwhile the workgroup stages the activations in
// LDS (padded so that the four 64-float runs a wave reads start on different
// banks) with each sub-block's sum, for the folded-out mins.  The four lanes of
// a row meet by shuffles and the S waves in LDS, in a fixed order: results are
// deterministic.
//
// Per weight: one v_cvt_f32_ubyte (low nibbles from w & 0x0f0f0f0f, high ones
// from w & 0xf0f0f0f0 as 16·q, their scale divided by 16) and one v_fmac.
// Per sub-block of 32: out += d1·Σq·x − m1·Σx (the weight is d1·q − m1).
//
// One launch may serve several matrices that read the same activations (the
// projections of a layer's input), each workgroup finding its matrix from its
// index; it may first RMS-normalize the activations (x · (1/rms(x) · w), as
// the reference's `normalize` does before those projections); and it may pair
// two matrices row for row, gate and up, writing silu(gate·x) · (up·x) (the
// reference's `swiglu`, gpu/mod.rs:274-285).
#include "device_util.h"
#include "layout.h"
#include "quant_math.h"
#include "runtime.h"

namespace {

constexpr int kMaxS = 16;
constexpr int kBlocksPerWave = 5;
constexpr size_t kLdsMax = 144 * 1024;  // of gfx950's 160 KB

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

// LDS image of the activations: position p at p + 4·(p / 64), per token,
// then the tokens' sub-block sums.
__host__ __device__ inline size_t xpad(size_t p) { return p + 4 * (p >> 6); }

struct Job {
    const uint8_t *w;
    size_t rows;
    float *out;
    int add;
};

struct Args {
    Job job[4];
    unsigned first_tile[5];  // workgroup index where each job's tiles start
    int njobs;
    int swiglu;              // jobs 0 and 1 paired: job 0's out = silu(gate·x)·(up·x)
    size_t nb;               // blocks per row (all jobs share the row length)
    const float *x;
    const float *norm;       // RMS-normalize x by this weight first, if set
    float *xn_out;           // and have workgroup 0 write the normalized x here, if set
    float eps;
    int waves;               // waves per matrix (a swiglu workgroup has twice as many)
    uint32_t lo_mask, hi_mask;
};

template <int T>
__global__ void __launch_bounds__(1024) k_mv_q4kt(const Args a) {
    extern __shared__ float xl_s[];
    __shared__ float red[2 * kMaxS][T][16];
    __shared__ float norm_red[16][T];
    const int lane = threadIdx.x & 63, wave_all = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int S = a.waves;
    // which matrix and tile
    int j = 0;
    while (j + 1 < a.njobs && blockIdx.x >= a.first_tile[j + 1]) j++;
    const size_t tile = blockIdx.x - a.first_tile[j];
    const int pairj = (a.swiglu && wave_all >= S) ? 1 : 0;  // the up half of a swiglu workgroup
    const int wave = wave_all - pairj * S;
    const Job job = a.job[j + pairj];
    const size_t nb = a.nb, cols = nb * 256, per_tok = xpad(cols), sbs = cols / 32;
    const size_t b0 = (size_t)wave * nb / S, b1 = (size_t)(wave + 1) * nb / S;
    float *xsum_s = xl_s + T * per_tok;

    // every weight load of the wave goes out first: one memory round trip per
    // wave, not one per block
    uint4 mm[kBlocksPerWave], qq0[kBlocksPerWave], qq1[kBlocksPerWave];
#pragma unroll
    for (int i = 0; i < kBlocksPerWave; i++) {
        const size_t b = b0 + i < b1 ? b0 + i : b0;
        const uint8_t *u = job.w + q4kt::unit(tile, b, nb);
        mm[i] = *(const uint4 *)(u + q4kt::meta_off(r));
        qq0[i] = *(const uint4 *)(u + q4kt::qs_off(g, r));
        qq1[i] = *(const uint4 *)(u + q4kt::qs_off(g, r) + 16);
    }
    // the stored high nibbles are XOR 8: back to ggml's bytes
#pragma unroll
    for (int i = 0; i < kBlocksPerWave; i++) {
        qq0[i] = make_uint4(qq0[i].x ^ 0x80808080u, qq0[i].y ^ 0x80808080u, qq0[i].z ^ 0x80808080u, qq0[i].w ^ 0x80808080u);
        qq1[i] = make_uint4(qq1[i].x ^ 0x80808080u, qq1[i].y ^ 0x80808080u, qq1[i].z ^ 0x80808080u, qq1[i].w ^ 0x80808080u);
    }
    // the activations into LDS (and their squares' sums when normalizing)
    const int nthreads = (int)blockDim.x;
    float ss[T];
#pragma unroll
    for (int t = 0; t < T; t++) ss[t] = 0.0f;
    for (size_t i = threadIdx.x * 4; i < T * cols; i += (size_t)nthreads * 4) {
        const size_t t = i / cols, p = i % cols;
        const float4 v = *(const float4 *)(a.x + i);
        *(float4 *)(xl_s + t * per_tok + xpad(p)) = v;
#pragma unroll
        for (int tt = 0; tt < T; tt++)
            if (tt == (int)t) ss[tt] += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
    if (a.norm) {
        // x · (1/sqrt(mean(x²) + eps) · w), the reference's rmsnorm (gpu/cpu.rs:157-166)
#pragma unroll
        for (int t = 0; t < T; t++) {
            const float s = group_sum<64>(ss[t]);
            if (lane == 0) norm_red[wave_all][t] = s;
        }
        __syncthreads();
        for (size_t i = threadIdx.x * 4; i < T * cols; i += (size_t)nthreads * 4) {
            const size_t t = i / cols, p = i % cols;
            float tot = 0.0f;
            for (int w = 0; w < nthreads / 64; w++) tot += norm_red[w][t];
            const float scale = 1.0f / sqrtf(tot / (float)cols + a.eps);
            float4 *dst = (float4 *)(xl_s + t * per_tok + xpad(p));
            const float4 nw = *(const float4 *)(a.norm + p);
            float4 v = *dst;
            v.x *= scale * nw.x;
            v.y *= scale * nw.y;
            v.z *= scale * nw.z;
            v.w *= scale * nw.w;
            *dst = v;
            if (a.xn_out && blockIdx.x == 0) *(float4 *)(a.xn_out + i) = v;
        }
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

    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.0f;
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
            chunk_dot(q0, xl, xh, a.lo_mask, a.hi_mask, sl, sh);
            load16f(xb + 16, xl);
            load16f(xb + 48, xh);
            chunk_dot(q1, xl, xh, a.lo_mask, a.hi_mask, sl, sh);
            acc[t] += d1 * sl - m1 * xs_lo + d2 * sh - m2 * xs_hi;
        }
    }
    // the row's four groups, then the waves
#pragma unroll
    for (int t = 0; t < T; t++) {
        float v = acc[t];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        if (g == 0) red[wave_all][t][r] = v;
    }
    __syncthreads();
    const Job out_job = a.job[j];
    const size_t row = tile * 16 + r;
    if (wave_all == 0 && g == 0 && row < out_job.rows) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            float v = 0.0f;
            for (int w = 0; w < S; w++) v += red[w][t][r];
            if (a.swiglu) {
                float u = 0.0f;
                for (int w = S; w < 2 * S; w++) u += red[w][t][r];
                v = v * sigmoidf_(v) * u;  // silu(gate) · up (gpu/cpu.rs:238-242)
            }
            float *o = out_job.out + t * out_job.rows + row;
            *o = out_job.add ? *o + v : v;
        }
    }
}

// Launches T-token passes of `a` over n tokens (a.x and the outs advance by a
// row per token).
hipError_t run(hipStream_t s, Args a, size_t n) {
    const size_t nb = a.nb, cols = nb * 256, sbs = cols / 32;
    size_t waves = (nb + kBlocksPerWave - 1) / kBlocksPerWave;
    if (waves > (size_t)kMaxS) return hipErrorInvalidValue;  // rows of at most 80 blocks (checked at upload)
    a.waves = (int)waves;
    const unsigned threads = (unsigned)(waves * 64 * (a.swiglu ? 2 : 1));
    if (threads > 1024) return hipErrorInvalidValue;
    unsigned total = 0;
    const int jobs = a.swiglu ? 1 : a.njobs;  // a swiglu launch walks the gate's tiles
    for (int j = 0; j < jobs; j++) {
        a.first_tile[j] = total;
        total += (unsigned)q4kt::tiles(a.job[j].rows);
    }
    a.first_tile[jobs] = total;
    if (a.swiglu) a.njobs = 1;  // workgroups index tiles of job 0; job 1 is read beside it
    auto lds_of = [&](size_t tt) { return (tt * xpad(cols) + tt * sbs) * sizeof(float); };
    static bool raised[3] = {false, false, false};
    size_t t = 0;
    Args b = a;
    while (t < n) {
        const size_t left = n - t;
        const size_t tt = left >= 4 && lds_of(4) <= kLdsMax ? 4 : left >= 2 && lds_of(2) <= kLdsMax ? 2 : 1;
        const size_t lds = lds_of(tt);
        const int idx = tt == 4 ? 2 : tt == 2 ? 1 : 0;
        const void *fn = tt == 4 ? (const void *)k_mv_q4kt<4> : tt == 2 ? (const void *)k_mv_q4kt<2>
                                                                          : (const void *)k_mv_q4kt<1>;
        if (lds > 64 * 1024 && !raised[idx]) {
            hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
            if (e != hipSuccess) return e;
            raised[idx] = true;
        }
        b.x = a.x + t * cols;
        if (a.xn_out) b.xn_out = a.xn_out + t * cols;
        for (int j = 0; j < 4; j++)
            if (a.job[j].out) b.job[j].out = a.job[j].out + t * a.job[j].rows;
        if (tt == 4) k_mv_q4kt<4><<<total, threads, lds, s>>>(b);
        else if (tt == 2) k_mv_q4kt<2><<<total, threads, lds, s>>>(b);
        else k_mv_q4kt<1><<<total, threads, lds, s>>>(b);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        t += tt;
    }
    return hipSuccess;
}

Args base_args(size_t cols) {
    Args a{};
    a.nb = cols / 256;
    a.lo_mask = 0x0f0f0f0fu;
    a.hi_mask = 0xf0f0f0f0u;
    return a;
}

}  // namespace

// Batches of at least kGemmTokens go through the f16 matrix-core GEMM.
constexpr size_t kGemmTokens = 16;

hipError_t launch_matvec_q4k(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n, int add) {
    if (n >= kGemmTokens) return launch_gemm_q4k(dev, w, out, x, n, add);
    if (n == 1) {
        hipError_t e = launch_planes(dev, x, w->cols, nullptr, 0.0f, nullptr, 0);
        if (e != hipSuccess) return e;
        return launch_mv_q4k_mfma(dev, &w, &out, &add, 1, 0, 0);
    }
    Args a = base_args(w->cols);
    a.job[0] = Job{(const uint8_t *)w->q, w->rows, out, add};
    a.njobs = 1;
    a.x = x;
    return run(dev->stream, a, n);
}

hipError_t launch_matvec_q4k_multi(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, int count,
                                   const float *x, size_t n, const float *norm, float eps, float *xn_out) {
    if (count < 1 || count > 4) return hipErrorInvalidValue;
    for (int j = 0; j < count; j++)
        if (ws[j]->cols != ws[0]->cols || ws[j]->fmt != DWIM_Q4_K) return hipErrorInvalidValue;
    if (n == 1) {
        hipError_t e = launch_planes(dev, x, ws[0]->cols, norm, eps, norm ? xn_out : nullptr, 0);
        if (e != hipSuccess) return e;
        return launch_mv_q4k_mfma(dev, ws, outs, nullptr, count, 0, 0);
    }
    if (n >= kGemmTokens) {
        const float *in = x;
        if (norm) {
            float *xn = xn_out ? xn_out : dev_work(dev, n * ws[0]->cols);
            if (!xn) return hipErrorOutOfMemory;
            hipError_t e = launch_rmsnorm(dev->stream, xn, x, norm, n, ws[0]->cols, eps);
            if (e != hipSuccess) return e;
            in = xn;
        }
        for (int j = 0; j < count; j++) {
            hipError_t e = launch_gemm_q4k(dev, ws[j], outs[j], in, n, 0);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    Args a = base_args(ws[0]->cols);
    for (int j = 0; j < count; j++) a.job[j] = Job{(const uint8_t *)ws[j]->q, ws[j]->rows, outs[j], 0};
    a.njobs = count;
    a.x = x;
    a.norm = norm;
    a.xn_out = norm ? xn_out : nullptr;
    a.eps = eps;
    return run(dev->stream, a, n);
}

hipError_t launch_swiglu_q4k(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, float *out, const float *x,
                             size_t n, const float *norm, float eps) {
    if (gate->rows != up->rows || gate->cols != up->cols) return hipErrorInvalidValue;
    if (n == 1) {
        hipError_t e = launch_planes(dev, x, gate->cols, norm, eps, nullptr, 0);
        if (e != hipSuccess) return e;
        const dwim_weight *ws[2] = {gate, up};
        float *outs[2] = {out, nullptr};
        return launch_mv_q4k_mfma(dev, ws, outs, nullptr, 2, 1, 0);
    }
    if (n >= kGemmTokens) {
        // x normalized, gate·x into out, up·x into the work scratch, then silu(out)·up
        const size_t cols = gate->cols, rows = gate->rows;
        float *work = dev_work(dev, n * rows + (norm ? n * cols : 0));
        if (!work) return hipErrorOutOfMemory;
        const float *in = x;
        if (norm) {
            float *xn = work + n * rows;
            hipError_t e = launch_rmsnorm(dev->stream, xn, x, norm, n, cols, eps);
            if (e != hipSuccess) return e;
            in = xn;
        }
        hipError_t e = launch_gemm_q4k(dev, gate, out, in, n, 0);
        if (e == hipSuccess) e = launch_gemm_q4k(dev, up, work, in, n, 0);
        if (e == hipSuccess) e = launch_silu_mul(dev->stream, out, work, n * rows);
        return e;
    }
    Args a = base_args(gate->cols);
    a.job[0] = Job{(const uint8_t *)gate->q, gate->rows, out, 0};
    a.job[1] = Job{(const uint8_t *)up->q, up->rows, nullptr, 0};
    a.njobs = 2;
    a.swiglu = 1;
    a.x = x;
    a.norm = norm;
    a.eps = eps;
    return run(dev->stream, a, n);
}
