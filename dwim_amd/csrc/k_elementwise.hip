// Memory-bound small operations: elementwise, RMS and L2 norms, rotary
// embeddings, the Q8 cache store, the causal convolution, argmax and the
// synthetic-weight generators.  Each reads and writes its operands once.
#include "device_util.h"
#include "layout.h"
#include "quant_math.h"
#include "runtime.h"

static inline unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

// ---------------------------------------------------------------- elementwise

__global__ void k_fill_zero(float *x, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = 0.0f;
}

// x += y (dwim gpu/cpu.rs:151-155)
__global__ void k_add(float *__restrict__ x, const float *__restrict__ y, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += y[i];
}

// g = g * sigmoid(g) * u (gpu/cpu.rs:238-242)
__global__ void k_silu_mul(float *__restrict__ g, const float *__restrict__ u, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = g[i];
        g[i] = v * sigmoidf_(v) * u[i];
    }
}

// x *= sigmoid(g) (gpu/cpu.rs:244-248)
__global__ void k_sigmoid_mul(float *__restrict__ x, const float *__restrict__ g, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] *= sigmoidf_(g[i]);
}

hipError_t launch_fill_zero(hipStream_t s, float *x, size_t n) {
    k_fill_zero<<<blocks_for(n, 256), 256, 0, s>>>(x, n);
    return hipGetLastError();
}
hipError_t launch_add(hipStream_t s, float *x, const float *y, size_t n) {
    k_add<<<blocks_for(n, 256), 256, 0, s>>>(x, y, n);
    return hipGetLastError();
}
hipError_t launch_silu_mul(hipStream_t s, float *g, const float *u, size_t n) {
    k_silu_mul<<<blocks_for(n, 256), 256, 0, s>>>(g, u, n);
    return hipGetLastError();
}
hipError_t launch_sigmoid_mul(hipStream_t s, float *x, const float *g, size_t n) {
    k_sigmoid_mul<<<blocks_for(n, 256), 256, 0, s>>>(x, g, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------- norms

// out[row] = x[row] * (1/sqrt(mean(x^2) + eps) * w), one block per row
// (gpu/cpu.rs:157-166; out may be x).
__global__ void __launch_bounds__(256) k_rmsnorm(float *out, const float *x, const float *__restrict__ w,
                                                 size_t dim, float eps) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * dim;
    float *orow = out + (size_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (size_t i = threadIdx.x; i < dim; i += 256) ss += xr[i] * xr[i];
    ss = block_sum<256>(ss, red);
    float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    for (size_t i = threadIdx.x; i < dim; i += 256) orow[i] = xr[i] * (scale * w[i]);
}

// Rows of up to 256: a wave per row.
__global__ void __launch_bounds__(256) k_rmsnorm_small(float *out, const float *x, const float *__restrict__ w,
                                                       size_t rows, size_t dim, float eps) {
    size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *xr = x + row * dim;
    float *orow = out + row * dim;
    float v[4];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        size_t i = lane + 64 * k;
        v[k] = i < dim ? xr[i] : 0.0f;
        ss += v[k] * v[k];
    }
    ss = group_sum<64>(ss);
    float scale = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        size_t i = lane + 64 * k;
        if (i < dim) orow[i] = v[k] * (scale * w[i]);
    }
}

// Rows of 1024·U floats (U <= 8, the 27B model's 5120 among them): U float4s
// a thread, all loaded before the sum, so that their latencies overlap (a
// loop whose every step waits for its own load took 14.5 µs for one row of
// 5120).  The values are k_rmsnorm's: x·(scale·w).
template <int U>
__global__ void __launch_bounds__(256) k_rmsnorm_wide(float *out, const float *x, const float *__restrict__ w,
                                                      size_t dim, float eps) {
    __shared__ float red[4];
    const float4 *xr = (const float4 *)(x + (size_t)blockIdx.x * dim);
    float4 *orow = (float4 *)(out + (size_t)blockIdx.x * dim);
    float4 v[U], wv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        v[u] = xr[threadIdx.x + 256 * u];
        wv[u] = ((const float4 *)w)[threadIdx.x + 256 * u];
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++) ss += (v[u].x * v[u].x + v[u].y * v[u].y) + (v[u].z * v[u].z + v[u].w * v[u].w);
    ss = block_sum<256>(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
    for (int u = 0; u < U; u++)
        orow[threadIdx.x + 256 * u] = make_float4(v[u].x * (scale * wv[u].x), v[u].y * (scale * wv[u].y),
                                                  v[u].z * (scale * wv[u].z), v[u].w * (scale * wv[u].w));
}

hipError_t launch_rmsnorm(hipStream_t s, float *out, const float *x, const float *w, size_t rows, size_t dim,
                          float eps) {
    if (dim % 1024 == 0 && dim / 1024 >= 1 && dim / 1024 <= 8) {
        const unsigned r = (unsigned)rows;
        switch (dim / 1024) {
            case 1: k_rmsnorm_wide<1><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
            case 2: k_rmsnorm_wide<2><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
            case 3: k_rmsnorm_wide<3><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
            case 4: k_rmsnorm_wide<4><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
            case 5: k_rmsnorm_wide<5><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
            case 6: k_rmsnorm_wide<6><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
            case 7: k_rmsnorm_wide<7><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
            default: k_rmsnorm_wide<8><<<r, 256, 0, s>>>(out, x, w, dim, eps); break;
        }
        return hipGetLastError();
    }
    if (dim <= 256)
        k_rmsnorm_small<<<blocks_for(rows, 4), 256, 0, s>>>(out, x, w, rows, dim, eps);
    else
        k_rmsnorm<<<(unsigned)rows, 256, 0, s>>>(out, x, w, dim, eps);
    return hipGetLastError();
}

// x[row] *= 1/sqrt(sum(x^2) + eps) (gpu/cpu.rs:168-175), a wave per row of up
// to 256, a block per longer row.
__global__ void __launch_bounds__(256) k_l2norm_small(float *x, size_t rows, size_t dim, float eps) {
    size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (row >= rows) return;
    float *xr = x + row * dim;
    float v[4];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        size_t i = lane + 64 * k;
        v[k] = i < dim ? xr[i] : 0.0f;
        ss += v[k] * v[k];
    }
    ss = group_sum<64>(ss);
    float scale = 1.0f / sqrtf(ss + eps);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        size_t i = lane + 64 * k;
        if (i < dim) xr[i] = v[k] * scale;
    }
}

__global__ void __launch_bounds__(256) k_l2norm(float *x, size_t dim, float eps) {
    __shared__ float red[4];
    float *xr = x + (size_t)blockIdx.x * dim;
    float ss = 0.0f;
    for (size_t i = threadIdx.x; i < dim; i += 256) ss += xr[i] * xr[i];
    ss = block_sum<256>(ss, red);
    float scale = 1.0f / sqrtf(ss + eps);
    for (size_t i = threadIdx.x; i < dim; i += 256) xr[i] *= scale;
}

hipError_t launch_l2norm(hipStream_t s, float *x, size_t rows, size_t dim, float eps) {
    if (dim <= 256)
        k_l2norm_small<<<blocks_for(rows, 4), 256, 0, s>>>(x, rows, dim, eps);
    else
        k_l2norm<<<(unsigned)rows, 256, 0, s>>>(x, dim, eps);
    return hipGetLastError();
}

// ---------------------------------------------------------------- rope

// One thread per rotated pair (gpu/cpu.rs:177-200).
__global__ void k_rope(float *x, const float *__restrict__ table, size_t n, size_t pos, size_t n_heads,
                       size_t head_dim, size_t rot_dim) {
    size_t half = rot_dim / 2;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * n_heads * half) return;
    size_t p = i % half, head = (i / half) % n_heads, t = i / (half * n_heads);
    const float *ang = table + (pos + t) * rot_dim + 2 * p;
    float c = ang[0], sn = ang[1];
    float *h = x + (t * n_heads + head) * head_dim;
    float a = h[p], b = h[p + half];
    h[p] = a * c - b * sn;
    h[p + half] = b * c + a * sn;
}

hipError_t launch_rope(hipStream_t s, float *x, const float *table, size_t n, size_t pos, size_t n_heads,
                       size_t head_dim, size_t rot_dim) {
    size_t pairs = n * n_heads * (rot_dim / 2);
    k_rope<<<blocks_for(pairs, 256), 256, 0, s>>>(x, table, n, pos, n_heads, head_dim, rot_dim);
    return hipGetLastError();
}

// ---------------------------------------------------------------- cache store

// Half a wave per block of 32: the block's largest magnitude by shuffles,
// then each lane its own value (gpu/quant.rs:161-180, bit for bit).
__global__ void __launch_bounds__(256) k_store(int8_t *__restrict__ cq, uint16_t *__restrict__ cs,
                                               const float *__restrict__ src, size_t blocks) {
    size_t b = ((size_t)blockIdx.x * 256 + threadIdx.x) >> 5;
    int l = threadIdx.x & 31;
    bool live = b < blocks;
    float x = live ? src[b * 32 + l] : 0.0f;
    float amax = fabsf(x);
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    if (!live) return;
    uint16_t bits = dq::block_scale(amax);
    float d = dq::from_f16(bits);
    cq[b * 32 + l] = d > 0.0f ? dq::quantize_one(x, d) : (int8_t)0;
    if (l == 0) cs[b] = bits;
}

// An f16 cache: each value rounded to the nearest f16 (ties to even, as the
// host's to_f16), a thread a value.
__global__ void __launch_bounds__(256) k_store_f16(uint16_t *__restrict__ c, const float *__restrict__ src, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) c[i] = dq::to_f16(src[i]);
}

hipError_t launch_store_f16(hipStream_t s, uint16_t *c, const float *src, size_t n) {
    k_store_f16<<<blocks_for(n, 256), 256, 0, s>>>(c, src, n);
    return hipGetLastError();
}

hipError_t launch_store(hipStream_t s, int8_t *cq, uint16_t *cs, const float *src, size_t blocks) {
    k_store<<<blocks_for(blocks * 32, 256), 256, 0, s>>>(cq, cs, src, blocks);
    return hipGetLastError();
}

// ---------------------------------------------------------------- conv

// One thread per channel, the 4-tap window carried in registers over the
// batch's tokens (gpu/cpu.rs:250-296).
__global__ void k_conv(float *__restrict__ q, float *__restrict__ k, float *__restrict__ v,
                       float *__restrict__ state_out, const float *__restrict__ x,
                       const float *__restrict__ state, const float *__restrict__ w, size_t n, size_t qd,
                       size_t kd, size_t vd) {
    size_t ch = qd + kd + vd;
    size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= ch) return;
    float w0 = w[c * 4], w1 = w[c * 4 + 1], w2 = w[c * 4 + 2], w3 = w[c * 4 + 3];
    float s0 = state[c], s1 = state[ch + c], s2 = state[2 * ch + c];
    float *dst;
    size_t stride, col;
    if (c < qd) { dst = q; stride = qd; col = c; }
    else if (c < qd + kd) { dst = k; stride = kd; col = c - qd; }
    else { dst = v; stride = vd; col = c - qd - kd; }
    for (size_t t = 0; t < n; t++) {
        float xin = x[t * ch + c];
        float acc = 0.0f;
        acc += w0 * s0;
        acc += w1 * s1;
        acc += w2 * s2;
        acc += w3 * xin;
        dst[t * stride + col] = acc * sigmoidf_(acc);
        s0 = s1;
        s1 = s2;
        s2 = xin;
    }
    state_out[c] = s0;
    state_out[ch + c] = s1;
    state_out[2 * ch + c] = s2;
}

hipError_t launch_conv(hipStream_t s, float *q, float *k, float *v, float *state_out, const float *x,
                       const float *state, const float *w, size_t n, size_t qd, size_t kd, size_t vd) {
    size_t ch = qd + kd + vd;
    k_conv<<<blocks_for(ch, 256), 256, 0, s>>>(q, k, v, state_out, x, state, w, n, qd, kd, vd);
    return hipGetLastError();
}

// ---------------------------------------------------------------- argmax

// (best, index) pairs: the larger value wins, the smaller index on a tie; an
// index of 0xffffffff is "none yet" (qwen35::argmax's strict `>` keeps the
// first maximum).
DEV void argmax_merge(float &best, uint32_t &idx, float ov, uint32_t oi) {
    if (oi != 0xffffffffu && (idx == 0xffffffffu || ov > best || (ov == best && oi < idx))) {
        best = ov;
        idx = oi;
    }
}

constexpr size_t kArgParts = 256;

// Pass 1: block (part, row) scans its contiguous share of the row (a
// multiple of 4 long when the row is), each thread four values at a time in
// increasing order, every load of the block issued before the comparisons,
// and leaves the part's first maximum.
__global__ void __launch_bounds__(256) k_argmax_part(const float *__restrict__ logits, size_t cols, size_t per,
                                                     float *__restrict__ pv, uint32_t *__restrict__ pi) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const size_t row = blockIdx.y, part = blockIdx.x, parts = gridDim.x;
    const float *r = logits + row * cols;
    const size_t lo = part * per, hi = lo + per < cols ? lo + per : cols;
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    if (cols % 4 == 0 && per % 4 == 0) {
        constexpr int kU = 4;  // float4 loads a thread
        for (size_t b = lo + 4 * threadIdx.x; b < hi; b += 4 * 256 * kU) {
            float4 v[kU];
#pragma unroll
            for (int u = 0; u < kU; u++) {
                const size_t i = b + (size_t)u * 4 * 256;
                v[u] = i < hi ? *(const float4 *)(r + i) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            }
#pragma unroll
            for (int u = 0; u < kU; u++) {
                const size_t i = b + (size_t)u * 4 * 256;
                if (i >= hi) continue;
                argmax_merge(best, idx, v[u].x, (uint32_t)i);
                argmax_merge(best, idx, v[u].y, (uint32_t)i + 1);
                argmax_merge(best, idx, v[u].z, (uint32_t)i + 2);
                argmax_merge(best, idx, v[u].w, (uint32_t)i + 3);
            }
        }
    } else {
        for (size_t i = lo + threadIdx.x; i < hi; i += 256) argmax_merge(best, idx, r[i], (uint32_t)i);
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) argmax_merge(best, idx, __shfl_xor(best, m, 64), __shfl_xor(idx, m, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) argmax_merge(best, idx, bv[w], bi[w]);
        pv[row * parts + part] = best;
        pi[row * parts + part] = idx;
    }
}

// Pass 2: a block per row merges its parts (at most kArgParts).
__global__ void __launch_bounds__(256) k_argmax_merge(const float *__restrict__ pv, const uint32_t *__restrict__ pi,
                                                      size_t parts, uint32_t *__restrict__ out) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const size_t row = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float best = threadIdx.x < parts ? pv[row * parts + threadIdx.x] : -INFINITY;
    uint32_t idx = threadIdx.x < parts ? pi[row * parts + threadIdx.x] : 0xffffffffu;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) argmax_merge(best, idx, __shfl_xor(best, m, 64), __shfl_xor(idx, m, 64));
    if (lane == 0) {
        bv[wave] = best;
        bi[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) argmax_merge(best, idx, bv[w], bi[w]);
        out[row] = idx == 0xffffffffu ? 0u : idx;
    }
}

size_t argmax_scratch_words(size_t rows) { return rows * (1 + 2 * kArgParts); }

// scratch: argmax_scratch_words(rows) words; the indices land in its first `rows`
hipError_t launch_argmax(hipStream_t s, const float *logits, size_t rows, size_t cols, uint32_t *scratch) {
    // parts of at least 1024 values, a multiple of 4 long
    const size_t parts = cols >= kArgParts * 1024 ? kArgParts : (cols + 1023) / 1024;
    const size_t per = ((cols + parts - 1) / parts + 3) / 4 * 4;
    float *pv = (float *)(scratch + rows);
    uint32_t *pi = scratch + rows + rows * kArgParts;
    k_argmax_part<<<dim3((unsigned)parts, (unsigned)rows), 256, 0, s>>>(logits, cols, per, pv, pi);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_argmax_merge<<<(unsigned)rows, 256, 0, s>>>(pv, pi, parts, scratch);
    return hipGetLastError();
}

// ---------------------------------------------------------------- embedding rows

// Weight (row, col) dequantized exactly as the host dequantizers do (the same
// operations, unfused), for any device layout.
__device__ float weight_at(const dwim_weight w, size_t row, size_t col) {
#pragma clang fp contract(off)
    switch (w.fmt) {
    case DWIM_BF16: return dq::bf16_to_f32(((const uint16_t *)w.q)[row * w.cols + col]);
    case DWIM_Q4_0: {
        const uint8_t q = ((const uint8_t *)w.q)[row * w.cols / 2 + (col / 32) * 16 + (col % 16)];
        const float d = dq::from_f16(((const uint16_t *)w.s)[row * (w.cols / 32) + col / 32]);
        const int nib = (col % 32) < 16 ? (q & 0xf) : (q >> 4);
        return ((float)nib - 8.0f) * d;
    }
    case DWIM_Q8_0: {
        const int8_t q = ((const int8_t *)w.q)[row * w.cols + col];
        return (float)q * dq::from_f16(((const uint16_t *)w.s)[row * (w.cols / 32) + col / 32]);
    }
    case DWIM_Q4_K: {
        const size_t nb = w.cols / 256, b = col / 256, pos = col % 256;
        const uint8_t *u = (const uint8_t *)w.q + q4kt::unit(row / q4kt::kTile, b, nb);
        const size_t r = row % q4kt::kTile;
        const int g = (int)(pos / 64), within = (int)(pos % 64), hi = within >= 32, l = within % 32;
        const uint8_t byte = q4kt::stored(u[q4kt::qs_off(g, r) + l]);
        const int q = hi ? (byte >> 4) : (byte & 0xf);
        const uint8_t *m = u + q4kt::meta_off(r);
        int sc, mn;
        dq::q4k_scale_min(2 * g + hi, m + 4, sc, mn);
        const float d = dq::from_f16((uint16_t)(m[0] | m[1] << 8)), dmin = dq::from_f16((uint16_t)(m[2] | m[3] << 8));
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        return d1 * (float)q - m1;
    }
    default: {  // Q6_K
        const size_t nb = w.cols / 256, blk = row * nb + col / 256;
        const int i = (int)(col % 256), half = i / 128, rr = i % 128, k = rr / 32, l = rr % 32;
        const uint8_t *ql = (const uint8_t *)w.q + blk * 128, *qh = (const uint8_t *)w.s + blk * 64;
        const int low = (ql[64 * half + l + 32 * (k % 2)] >> (4 * (k / 2))) & 0xf;
        const int high = (qh[32 * half + l] >> (2 * k)) & 3;
        const int q = (low | high << 4) - 32;
        const int8_t sc = ((const int8_t *)w.s2)[blk * 16 + 8 * half + 2 * k + l / 16];
        const float d = dq::from_f16(((const uint16_t *)w.s3)[blk]);
        return d * (float)sc * (float)q;
    }
    }
}

__global__ void k_embed(float *__restrict__ out, const dwim_weight w, const uint32_t *__restrict__ tokens, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * w.cols) return;
    const size_t t = i / w.cols, c = i % w.cols;
    out[i] = weight_at(w, tokens[t], c);
}

hipError_t launch_embed(hipStream_t s, float *out, const dwim_weight *w, const uint32_t *tokens, size_t n) {
    k_embed<<<blocks_for(n * w->cols, 256), 256, 0, s>>>(out, *w, tokens, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------- synthetic weights

// One thread per block of 256 weights: the stream's values for the block,
// quantized as the host quantizers do (quant_math.h).
__global__ void k_synthetic_q4_k(uint8_t *__restrict__ tiled, size_t blocks, size_t nb, uint64_t seed, float c) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    float x[256];
    for (int i = 0; i < 256; i++) x[i] = dq::synthetic(seed, b * 256 + i, c);
    uint8_t blk[144];
    dq::quantize_q4_k_block(x, blk);
    q4kt::place(tiled, nb, b / nb, b % nb, blk);
}

__global__ void k_synthetic_q6_k(uint8_t *__restrict__ ql, uint8_t *__restrict__ qh, int8_t *__restrict__ sc,
                                 uint16_t *__restrict__ d, size_t blocks, uint64_t seed, float c) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= blocks) return;
    float x[256];
    for (int i = 0; i < 256; i++) x[i] = dq::synthetic(seed, b * 256 + i, c);
    uint8_t blk[210];
    dq::quantize_q6_k_block(x, blk);
    for (int i = 0; i < 128; i++) ql[b * 128 + i] = blk[i];
    for (int i = 0; i < 64; i++) qh[b * 64 + i] = blk[128 + i];
    for (int i = 0; i < 16; i++) sc[b * 16 + i] = (int8_t)blk[192 + i];
    d[b] = (uint16_t)(blk[208] | (blk[209] << 8));
}

// bf16 by rounding to nearest, ties to even (gpu/float.rs:32-36).
__global__ void k_synthetic_bf16(uint16_t *__restrict__ q, size_t n, uint64_t seed, float c) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t b = dq::bits_of(dq::synthetic(seed, i, c));
    q[i] = (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

hipError_t launch_synthetic_q4_k(hipStream_t s, uint8_t *tiled, size_t rows, size_t cols, uint64_t seed, float c) {
    size_t blocks = rows * (cols / 256);
    k_synthetic_q4_k<<<blocks_for(blocks, 128), 128, 0, s>>>(tiled, blocks, cols / 256, seed, c);
    return hipGetLastError();
}

hipError_t launch_synthetic_q6_k(hipStream_t s, uint8_t *ql, uint8_t *qh, int8_t *sc, uint16_t *d, size_t rows,
                                 size_t cols, uint64_t seed, float c) {
    size_t blocks = rows * (cols / 256);
    k_synthetic_q6_k<<<blocks_for(blocks, 128), 128, 0, s>>>(ql, qh, sc, d, blocks, seed, c);
    return hipGetLastError();
}

hipError_t launch_synthetic_bf16(hipStream_t s, uint16_t *q, size_t rows, size_t cols, uint64_t seed, float c) {
    size_t n = rows * cols;
    k_synthetic_bf16<<<blocks_for(n, 256), 256, 0, s>>>(q, n, seed, c);
    return hipGetLastError();
}

// ---------------------------------------------------------------- measurement
// The streaming floor the decode products are measured against: a read of
// `bytes` (a multiple of 16) and nothing else, 16 bytes a lane, eight loads
// in flight a lane, grid-strided over a fixed grid.  The words are folded
// into one value that is stored only if it equals `never`, so that no load
// is dropped.  No counterpart in the reference; measurement only.
__global__ void __launch_bounds__(256) k_stream_read(const uint4 *__restrict__ p, size_t n, unsigned never,
                                                     unsigned *sink) {
    unsigned x = 0;
    const size_t step = (size_t)gridDim.x * 256 * 8;
    for (size_t i0 = (size_t)blockIdx.x * 256 * 8 + threadIdx.x; i0 < n; i0 += step) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t i = i0 + (size_t)u * 256;
            v[u] = p[i < n ? i : i0];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) x ^= (v[u].x ^ v[u].y) ^ (v[u].z ^ v[u].w);
    }
    if (x == never) sink[0] = x;
}

extern "C" int dwim_measure_stream(dwim_dev *dev, const void *p, size_t bytes, unsigned *sink, unsigned blocks) {
    if (!dev || !p || !sink || bytes % 16 || blocks == 0) return dwim_fail("measure_stream: bad arguments");
    k_stream_read<<<blocks, 256, 0, dev->stream>>>((const uint4 *)p, bytes / 16, 0x9e3779b9u, sink);
    DWIM_HIP(hipGetLastError());
    return 0;
}
