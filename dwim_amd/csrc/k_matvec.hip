// Dequantizing matrix-vector products for decode and small batches:
// out[t][r] = w[r] · x[t] (dwim gpu/cpu.rs:110-149, Device::matmul), for every
// weight format, with f32 activations and f32 accumulation (no MFMA: at a
// few tokens the product is bound by HBM, not arithmetic).
//
// Work split (gfx950, wave64): a wave's 64 lanes form 64/LPR groups of LPR
// lanes; each group owns R consecutive rows and walks their columns in
// 16-byte chunks of weights, lane l of the group taking chunks l, l+LPR, ...
// All lanes of a wave load consecutive 16-byte chunks of one row per
// instruction (coalesced, 16 B per lane), and every activation chunk a lane
// loads serves its R rows.  The group's partial sums meet by xor shuffles
// and one lane writes each result.  LPR is picked per shape so that the
// row's chunks divide evenly among the group's lanes.
//
// Chunk semantics of the generic kernel per format (weights per 16-byte chunk
// of the row's main stream):
//   Q6_K  64 weights (one chunk = 16 B of ql for k = 0/2, 16 B for k = 1/3 and
//         16 B of qh): positions l0..l0+15 of the four 32-weight runs of one
//         half of a block; out += (d·sc)·Σq·x per run of 16.
//   Q4_0  one block of 32: out += d·Σ(q−8)·x.
//   Q8_0  half a block (16 weights): out += d·Σq·x.
//   BF16  8 weights: out += Σw·x.
// Q4_K, the format of the model's body, has a kernel of its own below.
#include "device_util.h"
#include "planes.h"
#include "quant_math.h"
#include "runtime.h"

#include <stdlib.h>

namespace {

constexpr int kThreads = 256;  // 4 waves per block

DEV float lo_nib(uint32_t v, int byte) { return (float)((v >> (8 * byte)) & 0xfu); }
DEV float hi_nib(uint32_t v, int byte) { return (float)((v >> (8 * byte + 4)) & 0xfu); }

DEV void load16f(const float *p, float *dst) {
    const float4 *p4 = (const float4 *)p;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 v = p4[i];
        dst[4 * i] = v.x;
        dst[4 * i + 1] = v.y;
        dst[4 * i + 2] = v.z;
        dst[4 * i + 3] = v.w;
    }
}

DEV uint32_t word_of(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

struct Weights {
    const void *q, *s, *s2, *s3;
    size_t rows, cols;
};

// ---- per-format chunk counts and dot products ----

template <int FMT>
struct Fmt;

template <>
struct Fmt<DWIM_Q6_K> {
    __host__ __device__ static size_t chunks(size_t cols) { return cols / 256 * 4; }
    DEV static float dot(const Weights &w, size_t r, size_t c, const float *x) {
        size_t nb = w.cols / 256;
        size_t b = c >> 2;
        int hh = (int)((c >> 1) & 1), l0 = (int)(c & 1) * 16;
        size_t blk = r * nb + b;
        const uint8_t *ql = (const uint8_t *)w.q + blk * 128 + 64 * hh;
        const uint4 a = *(const uint4 *)(ql + l0);       // k = 0 (low), k = 2 (high)
        const uint4 bq = *(const uint4 *)(ql + 32 + l0); // k = 1 (low), k = 3 (high)
        const uint4 hq = *(const uint4 *)((const uint8_t *)w.s + blk * 64 + 32 * hh + l0);
        const int8_t *sc = (const int8_t *)w.s2 + blk * 16 + 8 * hh + (l0 >> 4);
        float d = dq::from_f16(((const uint16_t *)w.s3)[blk]);
        const float *xb = x + b * 256 + 128 * hh + l0;
        float total = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float xv[16];
            load16f(xb + 32 * k, xv);
            const uint4 &lowsrc = (k & 1) ? bq : a;
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                uint32_t lw = word_of(lowsrc, i >> 2), hw = word_of(hq, i >> 2);
                int low = (int)((lw >> (8 * (i & 3) + 4 * (k >> 1))) & 0xfu);
                int high = (int)((hw >> (8 * (i & 3) + 2 * k)) & 3u);
                s += (float)((low | (high << 4)) - 32) * xv[i];
            }
            total += (d * (float)sc[2 * k]) * s;
        }
        return total;
    }
};

template <>
struct Fmt<DWIM_Q4_0> {
    __host__ __device__ static size_t chunks(size_t cols) { return cols / 32; }
    DEV static float dot(const Weights &w, size_t r, size_t c, const float *x) {
        size_t nb = w.cols / 32;
        const uint4 q = ((const uint4 *)w.q)[r * nb + c];
        float d = dq::from_f16(((const uint16_t *)w.s)[r * nb + c]);
        float xl[16], xh[16];
        load16f(x + c * 32, xl);
        load16f(x + c * 32 + 16, xh);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            uint32_t v = word_of(q, i >> 2);
            s += (lo_nib(v, i & 3) - 8.0f) * xl[i] + (hi_nib(v, i & 3) - 8.0f) * xh[i];
        }
        return d * s;
    }
};

template <>
struct Fmt<DWIM_Q8_0> {
    __host__ __device__ static size_t chunks(size_t cols) { return cols / 16; }
    DEV static float dot(const Weights &w, size_t r, size_t c, const float *x) {
        const uint4 q = ((const uint4 *)w.q)[r * (w.cols / 16) + c];
        float d = dq::from_f16(((const uint16_t *)w.s)[r * (w.cols / 32) + (c >> 1)]);
        float xv[16];
        load16f(x + c * 16, xv);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int v = (int)(int8_t)((word_of(q, i >> 2) >> (8 * (i & 3))) & 0xffu);
            s += (float)v * xv[i];
        }
        return d * s;
    }
};

template <>
struct Fmt<DWIM_BF16> {
    __host__ __device__ static size_t chunks(size_t cols) { return cols / 8; }
    DEV static float dot(const Weights &w, size_t r, size_t c, const float *x) {
        const uint4 q = ((const uint4 *)w.q)[r * (w.cols / 8) + c];
        const float4 x0 = ((const float4 *)(x + c * 8))[0];
        const float4 x1 = ((const float4 *)(x + c * 8))[1];
        float s = 0.0f;
        s += dq::bf16_to_f32((uint16_t)(q.x & 0xffff)) * x0.x;
        s += dq::bf16_to_f32((uint16_t)(q.x >> 16)) * x0.y;
        s += dq::bf16_to_f32((uint16_t)(q.y & 0xffff)) * x0.z;
        s += dq::bf16_to_f32((uint16_t)(q.y >> 16)) * x0.w;
        s += dq::bf16_to_f32((uint16_t)(q.z & 0xffff)) * x1.x;
        s += dq::bf16_to_f32((uint16_t)(q.z >> 16)) * x1.y;
        s += dq::bf16_to_f32((uint16_t)(q.w & 0xffff)) * x1.z;
        s += dq::bf16_to_f32((uint16_t)(q.w >> 16)) * x1.w;
        return s;
    }
};

// out[t][r] (+)= w[r]·x[t] for T tokens from `x`, rows in groups of R per LPR lanes.
template <int FMT, int R, int T, int LPR>
__global__ void __launch_bounds__(kThreads) k_matvec(Weights w, const float *__restrict__ x, float *out, size_t n_out_stride,
                                                     int add) {
    const int lane = threadIdx.x & 63;
    const size_t group = ((size_t)blockIdx.x * kThreads + threadIdx.x) / LPR;
    const int sl = lane & (LPR - 1);
    const size_t row0 = group * R;
    if (row0 >= w.rows) return;  // whole groups only: shuffles stay within a group
    const size_t cpr = Fmt<FMT>::chunks(w.cols);
    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < T; t++) acc[r][t] = 0.0f;
    for (size_t c = sl; c < cpr; c += LPR) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            size_t row = row0 + r < w.rows ? row0 + r : w.rows - 1;
#pragma unroll
            for (int t = 0; t < T; t++) acc[r][t] += Fmt<FMT>::dot(w, row, c, x + t * w.cols);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < T; t++) {
            float v = group_sum<LPR>(acc[r][t]);
            if (sl == 0 && row0 + r < w.rows) {
                float *o = out + t * n_out_stride + row0 + r;
                *o = add ? *o + v : v;
            }
        }
}

template <int FMT, int R, int T>
hipError_t launch_lpr(hipStream_t s, const Weights &w, const float *x, float *out, int add, int lpr) {
    size_t groups = (w.rows + R - 1) / R;
    unsigned blocks = (unsigned)((groups * lpr + kThreads - 1) / kThreads);
    switch (lpr) {
    case 64: k_matvec<FMT, R, T, 64><<<blocks, kThreads, 0, s>>>(w, x, out, w.rows, add); break;
    case 32: k_matvec<FMT, R, T, 32><<<blocks, kThreads, 0, s>>>(w, x, out, w.rows, add); break;
    case 16: k_matvec<FMT, R, T, 16><<<blocks, kThreads, 0, s>>>(w, x, out, w.rows, add); break;
    case 8: k_matvec<FMT, R, T, 8><<<blocks, kThreads, 0, s>>>(w, x, out, w.rows, add); break;
    default: k_matvec<FMT, R, T, 4><<<blocks, kThreads, 0, s>>>(w, x, out, w.rows, add); break;
    }
    return hipGetLastError();
}

// Lanes per row group: the largest of 64..4 that splits the row's chunks
// evenly, else the one that wastes the fewest lane-iterations.
int pick_lpr(size_t cpr) {
    int best = 4;
    double best_eff = 0.0;
    for (int l = 64; l >= 4; l >>= 1) {
        size_t iters = (cpr + l - 1) / l;
        double eff = (double)cpr / (double)(iters * l);
        if (eff > best_eff + 1e-9) {
            best_eff = eff;
            best = l;
        }
    }
    return best;
}

template <int FMT>
hipError_t launch_fmt(hipStream_t s, const Weights &w, const float *x, float *out, size_t n, int add) {
    int lpr = pick_lpr(Fmt<FMT>::chunks(w.cols));
    // Few rows: one row per group so that the launch still fills the GPU.
    bool many_rows = w.rows * 64 / lpr >= 4096 * 4;
    size_t t = 0;
    hipError_t e = hipSuccess;
    while (t < n && e == hipSuccess) {
        size_t left = n - t;
        const float *xt = x + t * w.cols;
        float *ot = out + t * w.rows;
        if (left >= 4) {
            e = launch_lpr<FMT, 2, 4>(s, w, xt, ot, add, lpr);
            t += 4;
        } else if (left == 3) {
            e = launch_lpr<FMT, 2, 3>(s, w, xt, ot, add, lpr);
            t += 3;
        } else if (left == 2) {
            e = launch_lpr<FMT, 2, 2>(s, w, xt, ot, add, lpr);
            t += 2;
        } else {
            e = many_rows ? launch_lpr<FMT, 4, 1>(s, w, xt, ot, add, lpr)
                          : launch_lpr<FMT, 1, 1>(s, w, xt, ot, add, lpr);
            t += 1;
        }
    }
    return e;
}

}  // namespace

// Batches through a bf16 matrix of few rows (at most 96, as DeltaNet's gate
// projection has): a block of 256 threads per 8 tokens, thread (token t =
// tid / 32, rows rg, rg + 32, rg + 64) summing in f32 over k (the
// reference's dot product, gpu/cpu.rs:370-384, sums 8 lanes; the tolerance
// covers the order).  The k-chunks of 64 are staged in LDS as f32, W [row][k]
// and x [token][k], each read as float4 along k; the next chunk's global
// loads are issued before the current chunk is summed.
constexpr int kSkTok = 8, kSkK = 64, kSkRows = 96;

__global__ void __launch_bounds__(256) k_skinny_bf16(const uint16_t *__restrict__ w, const float *__restrict__ x,
                                                     float *__restrict__ out, size_t rows, size_t cols, size_t n,
                                                     int add) {
    __shared__ float4 ws[kSkRows][kSkK / 4 + 1];  // [row][k/4], padded
    __shared__ float4 xs[kSkTok][kSkK / 4];
    const int tid = threadIdx.x, tt = tid >> 5, rg = tid & 31;
    const size_t t0 = (size_t)blockIdx.x * kSkTok;
    // a chunk: 96 rows × 64 k of bf16 = 768 16-byte loads (3 a thread), and
    // 8 tokens × 64 k of f32 = 128 16-byte loads (threads < 128)
    uint4 wr[3];
    float4 xr = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto load = [&](size_t k0) {
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int e = tid + 256 * i, r = e >> 3, kk = (e & 7) * 8;
            wr[i] = r < (int)rows ? *(const uint4 *)(w + (size_t)r * cols + k0 + kk) : make_uint4(0, 0, 0, 0);
        }
        if (tid < kSkTok * kSkK / 4) {
            const int t = tid >> 4, kk = (tid & 15) * 4;
            xr = t0 + t < n ? *(const float4 *)(x + (t0 + t) * cols + k0 + kk) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    load(0);
    float acc[3] = {0.0f, 0.0f, 0.0f};
    for (size_t k0 = 0; k0 < cols; k0 += kSkK) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int e = tid + 256 * i, r = e >> 3, q = (e & 7) * 2;
            const uint32_t v[4] = {wr[i].x, wr[i].y, wr[i].z, wr[i].w};
            ws[r][q] = make_float4(dq::bf16_to_f32((uint16_t)(v[0] & 0xffffu)), dq::bf16_to_f32((uint16_t)(v[0] >> 16)),
                                   dq::bf16_to_f32((uint16_t)(v[1] & 0xffffu)), dq::bf16_to_f32((uint16_t)(v[1] >> 16)));
            ws[r][q + 1] = make_float4(dq::bf16_to_f32((uint16_t)(v[2] & 0xffffu)), dq::bf16_to_f32((uint16_t)(v[2] >> 16)),
                                       dq::bf16_to_f32((uint16_t)(v[3] & 0xffffu)), dq::bf16_to_f32((uint16_t)(v[3] >> 16)));
        }
        if (tid < kSkTok * kSkK / 4) xs[tid >> 4][tid & 15] = xr;
        __syncthreads();
        if (k0 + kSkK < cols) load(k0 + kSkK);
#pragma unroll 4
        for (int q = 0; q < kSkK / 4; q++) {
            const float4 xv = xs[tt][q];
#pragma unroll
            for (int i = 0; i < 3; i++) {
                const float4 wv = ws[rg + 32 * i][q];
                acc[i] += wv.x * xv.x;
                acc[i] += wv.y * xv.y;
                acc[i] += wv.z * xv.z;
                acc[i] += wv.w * xv.w;
            }
        }
    }
    if (t0 + tt >= n) return;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const size_t r = rg + 32 * i;
        if (r < rows) {
            float *o = out + (t0 + tt) * rows + r;
            *o = add ? *o + acc[i] : acc[i];
        }
    }
}

// A few tokens (a verify batch) through a bf16 matrix of few rows: a block of
// 256 threads per row and run of up to 4 tokens, thread i summing columns
// 8i.. in steps of 2048 for each token (16-byte weight loads, read once for
// the run), then the block's sums meet per token.  Enough blocks to spread the
// rows' bytes over the chip: 96 × 5120 is 96 blocks of 40 KB.
constexpr int kRowTok = 4;

__global__ void __launch_bounds__(256) k_rows_bf16(const uint16_t *__restrict__ w, const float *__restrict__ x,
                                                   float *__restrict__ out, size_t rows, size_t cols, size_t n,
                                                   int add) {
    __shared__ float part[kRowTok][4];
    const size_t row = blockIdx.x, t0 = (size_t)blockIdx.y * kRowTok;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = (int)(n - t0 < (size_t)kRowTok ? n - t0 : (size_t)kRowTok);
    float acc[kRowTok] = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t *wr = w + row * cols;
    for (size_t c = 8 * (size_t)tid; c < cols; c += 8 * 256) {
        const uint4 q = *(const uint4 *)(wr + c);
        const uint32_t v[4] = {q.x, q.y, q.z, q.w};
        float wf[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            wf[2 * i] = dq::bf16_to_f32((uint16_t)(v[i] & 0xffffu));
            wf[2 * i + 1] = dq::bf16_to_f32((uint16_t)(v[i] >> 16));
        }
#pragma unroll
        for (int t = 0; t < kRowTok; t++) {
            if (t >= nt) break;
            const float4 a = *(const float4 *)(x + (t0 + t) * cols + c), b = *(const float4 *)(x + (t0 + t) * cols + c + 4);
            acc[t] += ((wf[0] * a.x + wf[1] * a.y) + (wf[2] * a.z + wf[3] * a.w)) +
                      ((wf[4] * b.x + wf[5] * b.y) + (wf[6] * b.z + wf[7] * b.w));
        }
    }
#pragma unroll
    for (int t = 0; t < kRowTok; t++) {
        const float v = group_sum<64>(acc[t]);
        if (lane == 0) part[t][wave] = v;
    }
    __syncthreads();
    if (tid < nt) {
        const float v = (part[tid][0] + part[tid][1]) + (part[tid][2] + part[tid][3]);
        float *o = out + (t0 + tid) * rows + row;
        *o = add ? *o + v : v;
    }
}

hipError_t launch_matvec(dwim_dev *dev, const dwim_weight *wt, float *out, const float *x, size_t n, int add) {
    hipStream_t s = dev->stream;
    Weights w{wt->q, wt->s, wt->s2, wt->s3, wt->rows, wt->cols};
    switch (wt->fmt) {
    case DWIM_Q4_K: return launch_matvec_q4k(dev, wt, out, x, n, add);
    case DWIM_Q6_K:
        if (n == 1 && !add && wt->cols <= 10240) {  // (a workgroup's 8 waves take 5 blocks each)
            // one token (the output head): the int8 matrix cores over x's planes
            hipError_t e = launch_planes(dev, x, wt->cols, nullptr, 0.0f, nullptr, 0);
            return e != hipSuccess ? e : launch_mv_q6k_mfma(dev, wt, out, 0);
        }
        // a few tokens (a verify batch): the weights read once a run of four
        if (n > 1 && n < 16 && !add && wt->cols % 256 == 0 && wt->cols <= 10240)
            return launch_mv_q6k_tokens(dev, wt, out, x, n);
        return launch_fmt<DWIM_Q6_K>(s, w, x, out, n, add);
    case DWIM_Q4_0: return launch_fmt<DWIM_Q4_0>(s, w, x, out, n, add);
    case DWIM_Q8_0: return launch_fmt<DWIM_Q8_0>(s, w, x, out, n, add);
    default:
        if (n < 16 && wt->rows <= kSkRows && wt->cols % 8 == 0) {
            k_rows_bf16<<<dim3((unsigned)wt->rows, (unsigned)((n + kRowTok - 1) / kRowTok)), 256, 0, s>>>(
                (const uint16_t *)wt->q, x, out, wt->rows, wt->cols, n, add);
            return hipGetLastError();
        }
        if (n >= 16 && wt->rows <= kSkRows && wt->cols % kSkK == 0) {
            k_skinny_bf16<<<(unsigned)((n + kSkTok - 1) / kSkTok), 256, 0, s>>>((const uint16_t *)wt->q, x, out,
                                                                               wt->rows, wt->cols, n, add);
            return hipGetLastError();
        }
        return launch_fmt<DWIM_BF16>(s, w, x, out, n, add);
    }
}

hipError_t launch_swiglu(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, float *out, float *scratch,
                         const float *x, size_t n) {
    if (gate->fmt == DWIM_Q4_K && up->fmt == DWIM_Q4_K && gate->cols <= 16 * 5 * 256 / 2)
        return launch_swiglu_q4k(dev, gate, up, out, x, n, nullptr, 0.0f);
    hipError_t e = launch_matvec(dev, gate, out, x, n, 0);
    if (e == hipSuccess) e = launch_matvec(dev, up, scratch, x, n, 0);
    if (e == hipSuccess) e = launch_silu_mul(dev->stream, out, scratch, n * gate->rows);
    return e;
}
