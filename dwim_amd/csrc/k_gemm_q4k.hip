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

__global__ void __launch_bounds__(kThreads) k_gemm_q4k(const GemmArgs a) {
    extern __shared__ _Float16 lds[];
    _Float16 *ah = lds, *al = ah + kRows * kPad, *bh = al + kRows * kPad, *bl = bh + kToks * kPad;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;  // the wave's 64-row, 64-token quarter
    const size_t row0 = (size_t)blockIdx.x * kRows, tok0 = (size_t)blockIdx.y * kToks;
    const size_t nb = a.cols / 256, tiles = q4kt::tiles(a.rows);

    // the weights this thread dequantizes: row lr of the tile, quant bytes 16·lh..16·lh+15
    const int lr = tid >> 1, lh = tid & 1;
    const size_t wtile = (row0 + lr) / 16;
    const bool wlive = wtile < tiles;
    // the activations this thread stages: token lt, 32 of the step's 64
    const int lt = tid >> 1, lx = tid & 1;
    const bool xlive = tok0 + lt < a.n;

    float4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    for (size_t b = 0; b < nb; b++) {
        // this row's block header: d, dmin and the 6-bit scales and mins
        uint8_t hdr[16];
        if (wlive) {
            const uint4 h = *(const uint4 *)(a.w + q4kt::unit(wtile, b, nb) + q4kt::meta_off((row0 + lr) % 16));
            __builtin_memcpy(hdr, &h, 16);
        } else {
            for (int i = 0; i < 16; i++) hdr[i] = 0;
        }
        const float d = dq::from_f16((uint16_t)(hdr[0] | hdr[1] << 8)), dmin = dq::from_f16((uint16_t)(hdr[2] | hdr[3] << 8));
        for (int g = 0; g < 4; g++) {
            // stage the weights: sub-blocks 2g (low nibbles) and 2g+1 (high nibbles)
            {
                float sc0, mn0, sc1, mn1;
                scale_min(hdr + 4, 2 * g, sc0, mn0);
                scale_min(hdr + 4, 2 * g + 1, sc1, mn1);
                const float d0 = d * sc0, m0 = dmin * mn0, d1 = d * sc1, m1 = dmin * mn1;
                uint4 q = make_uint4(0, 0, 0, 0);
                if (wlive) q = *(const uint4 *)(a.w + q4kt::unit(wtile, b, nb) + q4kt::qs_off(g, (row0 + lr) % 16) + 16 * lh);
                const uint32_t words[4] = {q.x, q.y, q.z, q.w};
                _Float16 *dh = ah + lr * kPad + 16 * lh, *dl = al + lr * kPad + 16 * lh;
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const uint32_t byte = q4kt::stored((uint8_t)(words[k / 4] >> (8 * (k % 4))));
                    const float w0 = d0 * (float)(byte & 0xf) - m0, w1 = d1 * (float)(byte >> 4) - m1;
                    const _Float16 h0 = (_Float16)w0, h1 = (_Float16)w1;
                    dh[k] = h0;
                    dl[k] = (_Float16)(w0 - (float)h0);
                    dh[32 + k] = h1;
                    dl[32 + k] = (_Float16)(w1 - (float)h1);
                }
            }
            // stage the activations: 32 halves of each part
            {
                const size_t off = (tok0 + lt) * a.cols + b * 256 + g * kStep + 32 * lx;
                uint4 xh4[4], xl4[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    xh4[k] = xlive ? ((const uint4 *)(a.xh + off))[k] : make_uint4(0, 0, 0, 0);
                    xl4[k] = xlive ? ((const uint4 *)(a.xl + off))[k] : make_uint4(0, 0, 0, 0);
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    *(uint4 *)(bh + lt * kPad + 32 * lx + 8 * k) = xh4[k];
                    *(uint4 *)(bl + lt * kPad + 32 * lx + 8 * k) = xl4[k];
                }
            }
            __syncthreads();
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
        }
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
