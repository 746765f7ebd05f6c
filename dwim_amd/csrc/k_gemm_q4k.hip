// Q4_K matrix products for batches of tokens (prefill and verify): out[t][r]
// (+)= w[r] · x[t] (dwim gpu/cpu.rs:110-149) on the f16 matrix cores, at
// close to f32 accuracy.
//
// Each weight w (the exact Q4_K value d·sc·q − dmin·m) and each activation x
// is split in two f16 parts, hi = f16(w), lo = f16(w − hi), and the products
// hi·hi + hi·lo + lo·hi are summed in f32 by v_mfma_f32_16x16x32_f16: 22 of
// each operand's bits, the dropped lo·lo term below 2^-21 of the product.
// k_split writes the activations' parts once per product; the weights are
// dequantized into LDS by the workgroup that uses them.
//
// A workgroup of 4 waves computes a 128-row × 128-token tile, each wave a
// 64 × 64 quarter as 4 × 4 MFMA tiles.  It walks the row in steps of one
// quant group (64 weights): the 128 rows' 64 weights into LDS as hi and lo
// f16 (two threads a row, each 16 quant bytes: 32 weights), the 128 tokens'
// 64 activations likewise, then 2 × 16 × 3 MFMAs a wave.  LDS rows are padded
// to 72 halves so that the 16 lanes reading one k-slice of 16 rows hit
// different banks.
#include "device_util.h"
#include "layout.h"
#include "quant_math.h"
#include "runtime.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

namespace {

constexpr int kRows = 128, kToks = 128, kStep = 64, kPad = 72;  // halves a padded LDS row
constexpr int kThreads = 256;

// x [n][cols] f32 -> xh, xl [n][cols] f16 (hi and lo parts)
__global__ void k_split(const float *__restrict__ x, _Float16 *__restrict__ xh, _Float16 *__restrict__ xl, size_t total) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const float v = x[i];
    const _Float16 h = (_Float16)v;
    xh[i] = h;
    xl[i] = (_Float16)(v - (float)h);
}

DEV void scale_min(const uint8_t *s, int j, float &sc, float &mn) {
    if (j < 4) {
        sc = (float)(s[j] & 63);
        mn = (float)(s[j + 4] & 63);
    } else {
        sc = (float)((s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4));
        mn = (float)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

struct GemmArgs {
    const uint8_t *w;
    size_t rows, cols, n;
    const _Float16 *xh, *xl;
    float *out;
    int add;
};

// The global loads of one step (a quant group of a block): this thread's 16
// quant bytes of its row and, at a block's first group, the row's header; and
// 32 halves of each part of its token's activations.
struct StepLoad {
    uint4 q, hdr, xh[4], xl[4];
};

__global__ void __launch_bounds__(kThreads) k_gemm_q4k(const GemmArgs a) {
    extern __shared__ _Float16 lds[];
    _Float16 *ah = lds, *al = ah + kRows * kPad, *bh = al + kRows * kPad, *bl = bh + kToks * kPad;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;  // the wave's 64-row, 64-token quarter
    const size_t row0 = (size_t)blockIdx.x * kRows, tok0 = (size_t)blockIdx.y * kToks;
    const size_t nb = a.cols / 256, tiles = q4kt::tiles(a.rows), steps = 4 * nb;

    // the weights this thread dequantizes: row lr of the tile, quant bytes 16·lh..16·lh+15
    const int lr = tid >> 1, lh = tid & 1;
    const size_t wtile = (row0 + lr) / 16;
    const bool wlive = wtile < tiles;
    // the activations this thread stages: token lt, 32 of the step's 64
    const int lt = tid >> 1, lx = tid & 1;
    const bool xlive = tok0 + lt < a.n;

    auto fetch = [&](size_t s, StepLoad &L) {
        const size_t b = s / 4, g = s % 4;
        if (wlive) {
            const uint8_t *u = a.w + q4kt::unit(wtile, b, nb);
            L.q = *(const uint4 *)(u + q4kt::qs_off(g, (row0 + lr) % 16) + 16 * lh);
            if (g == 0) L.hdr = *(const uint4 *)(u + q4kt::meta_off((row0 + lr) % 16));
        } else {
            L.q = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);  // (stored 0 weights)
            L.hdr = make_uint4(0, 0, 0, 0);
        }
        const size_t off = (tok0 + (xlive ? lt : 0)) * a.cols + b * 256 + g * kStep + 32 * lx;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            L.xh[k] = ((const uint4 *)(a.xh + off))[k];
            L.xl[k] = ((const uint4 *)(a.xl + off))[k];
        }
        if (!xlive)
#pragma unroll
            for (int k = 0; k < 4; k++) L.xh[k] = L.xl[k] = make_uint4(0, 0, 0, 0);
    };

    float4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    StepLoad cur, nxt;
    fetch(0, cur);
    uint8_t hdr[16];
    float d = 0.0f, dmin = 0.0f;
    for (size_t s = 0; s < steps; s++) {
        const int g = (int)(s % 4);
        if (g == 0) {
            // this row's block header: d, dmin and the 6-bit scales and mins
            __builtin_memcpy(hdr, &cur.hdr, 16);
            d = dq::from_f16((uint16_t)(hdr[0] | hdr[1] << 8));
            dmin = dq::from_f16((uint16_t)(hdr[2] | hdr[3] << 8));
        }
        // stage the weights: sub-blocks 2g (low nibbles) and 2g+1 (high nibbles)
        {
            float sc0, mn0, sc1, mn1;
            scale_min(hdr + 4, 2 * g, sc0, mn0);
            scale_min(hdr + 4, 2 * g + 1, sc1, mn1);
            const float d0 = d * sc0, m0 = dmin * mn0, d1 = d * sc1, m1 = dmin * mn1;
            const uint32_t words[4] = {cur.q.x, cur.q.y, cur.q.z, cur.q.w};
            // 16 low-nibble weights (sub-block 2g), 16 high (2g+1): hi and lo
            // halves packed in pairs, written 8 halves at a time
            uint32_t hh0[8], hl0[8], hh1[8], hl1[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo = words[k] & 0x0f0f0f0fu, hi = ((words[k] ^ 0x80808080u) >> 4) & 0x0f0f0f0fu;
                float w0[4], w1[4];
                w0[0] = d0 * (float)(lo & 0xffu) - m0;
                w0[1] = d0 * (float)((lo >> 8) & 0xffu) - m0;
                w0[2] = d0 * (float)((lo >> 16) & 0xffu) - m0;
                w0[3] = d0 * (float)(lo >> 24) - m0;
                w1[0] = d1 * (float)(hi & 0xffu) - m1;
                w1[1] = d1 * (float)((hi >> 8) & 0xffu) - m1;
                w1[2] = d1 * (float)((hi >> 16) & 0xffu) - m1;
                w1[3] = d1 * (float)(hi >> 24) - m1;
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const half2v h0 = half2v{(_Float16)w0[2 * e], (_Float16)w0[2 * e + 1]};
                    const half2v h1 = half2v{(_Float16)w1[2 * e], (_Float16)w1[2 * e + 1]};
                    const half2v l0 = half2v{(_Float16)(w0[2 * e] - (float)h0[0]), (_Float16)(w0[2 * e + 1] - (float)h0[1])};
                    const half2v l1 = half2v{(_Float16)(w1[2 * e] - (float)h1[0]), (_Float16)(w1[2 * e + 1] - (float)h1[1])};
                    hh0[2 * k + e] = __builtin_bit_cast(uint32_t, h0);
                    hl0[2 * k + e] = __builtin_bit_cast(uint32_t, l0);
                    hh1[2 * k + e] = __builtin_bit_cast(uint32_t, h1);
                    hl1[2 * k + e] = __builtin_bit_cast(uint32_t, l1);
                }
            }
            uint32_t *dh = (uint32_t *)(ah + lr * kPad + 16 * lh), *dl = (uint32_t *)(al + lr * kPad + 16 * lh);
            *(uint4 *)dh = make_uint4(hh0[0], hh0[1], hh0[2], hh0[3]);
            *(uint4 *)(dh + 4) = make_uint4(hh0[4], hh0[5], hh0[6], hh0[7]);
            *(uint4 *)(dh + 16) = make_uint4(hh1[0], hh1[1], hh1[2], hh1[3]);
            *(uint4 *)(dh + 20) = make_uint4(hh1[4], hh1[5], hh1[6], hh1[7]);
            *(uint4 *)dl = make_uint4(hl0[0], hl0[1], hl0[2], hl0[3]);
            *(uint4 *)(dl + 4) = make_uint4(hl0[4], hl0[5], hl0[6], hl0[7]);
            *(uint4 *)(dl + 16) = make_uint4(hl1[0], hl1[1], hl1[2], hl1[3]);
            *(uint4 *)(dl + 20) = make_uint4(hl1[4], hl1[5], hl1[6], hl1[7]);
        }
        // stage the activations: 32 halves of each part
#pragma unroll
        for (int k = 0; k < 4; k++) {
            *(uint4 *)(bh + lt * kPad + 32 * lx + 8 * k) = cur.xh[k];
            *(uint4 *)(bl + lt * kPad + 32 * lx + 8 * k) = cur.xl[k];
        }
        __syncthreads();
        // the next step's loads fly while this step's products run
        if (s + 1 < steps) {
            fetch(s + 1, nxt);
            if ((s + 1) % 4 != 0) nxt.hdr = cur.hdr;
        }
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const int ko = kk * 32 + 8 * (lane >> 4);
            half8 fah[4], fal[4], fbh[4], fbl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = wr * 64 + i * 16 + (lane & 15);
                fah[i] = *(const half8 *)(ah + r * kPad + ko);
                fal[i] = *(const half8 *)(al + r * kPad + ko);
                const int t = wc * 64 + i * 16 + (lane & 15);
                fbh[i] = *(const half8 *)(bh + t * kPad + ko);
                fbl[i] = *(const half8 *)(bl + t * kPad + ko);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fah[i], fbh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fah[i], fbl[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fal[i], fbh[j], acc[i][j], 0, 0, 0);
                }
        }
        __syncthreads();
        cur = nxt;
    }
    // C tile (i, j): lane holds rows 16i + 4(lane/16) + e of token 16j + lane%16
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const size_t t = tok0 + wc * 64 + j * 16 + (lane & 15);
        if (t >= a.n) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const size_t r = row0 + wr * 64 + i * 16 + 4 * (lane >> 4);
            float *o = a.out + t * a.rows + r;
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (r + e < a.rows) o[e] = a.add ? o[e] + acc[i][j][e] : acc[i][j][e];
        }
    }
}

}  // namespace

size_t gemm_split_bytes(size_t n, size_t cols) { return 2 * n * cols * sizeof(_Float16); }

hipError_t launch_gemm_q4k(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n, int add) {
    if (w->fmt != DWIM_Q4_K || w->cols % 256) return hipErrorInvalidValue;
    const size_t need = gemm_split_bytes(n, w->cols);
    if (dev->split_cap < need) {
        if (dev->split) hipFree(dev->split);
        dev->split = nullptr;
        dev->split_cap = 0;
        hipError_t e = hipMalloc(&dev->split, need);
        if (e != hipSuccess) return e;
        dev->split_cap = need;
    }
    _Float16 *xh = (_Float16 *)dev->split, *xl = xh + n * w->cols;
    const size_t total = n * w->cols;
    k_split<<<(unsigned)((total + 255) / 256), 256, 0, dev->stream>>>(x, xh, xl, total);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    static bool raised = false;
    const size_t lds = (size_t)2 * (kRows + kToks) * kPad * sizeof(_Float16);
    if (!raised) {
        e = hipFuncSetAttribute((const void *)k_gemm_q4k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        raised = true;
    }
    GemmArgs a{(const uint8_t *)w->q, w->rows, w->cols, n, xh, xl, out, add};
    dim3 grid((unsigned)((w->rows + kRows - 1) / kRows), (unsigned)((n + kToks - 1) / kToks));
    k_gemm_q4k<<<grid, kThreads, lds, dev->stream>>>(a);
    return hipGetLastError();
}
