// Kernels that do in one launch what the reference's token loop does in
// several `Device` calls (inference/qwen35/mod.rs:541-655), for the model
// host of model_qwen35.hip.  Each does the same arithmetic as the separate
// operations, on the values they would have passed each other.
#include "device_util.h"
#include "planes.h"
#include "quant_math.h"
#include "runtime.h"

namespace {

// A sum over the block's `blockDim.x` (a multiple of 64, at most 1024) threads.
DEV float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < waves; i++) s += red[i];
    return s;
}

// conv (gpu/cpu.rs:250-296), then l2norm (gpu/cpu.rs:168-175) of each
// `dim`-row of q and k.  A block of `dim` threads per `dim` channels, a
// channel per thread with its 4-tap window in registers, a token at a time.
__global__ void __launch_bounds__(256) k_conv_l2(float *__restrict__ q, float *__restrict__ k, float *__restrict__ v,
                                                 float *__restrict__ state_out, const float *__restrict__ x,
                                                 const float *__restrict__ state, const float *__restrict__ w,
                                                 size_t n, size_t qd, size_t kd, size_t vd, float eps) {
    __shared__ float red[4];
    const size_t ch = qd + kd + vd;
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const float w0 = w[c * 4], w1 = w[c * 4 + 1], w2 = w[c * 4 + 2], w3 = w[c * 4 + 3];
    float s0 = state[c], s1 = state[ch + c], s2 = state[2 * ch + c];
    float *dst;
    size_t stride, col;
    bool norm = true;
    if (c < qd) { dst = q; stride = qd; col = c; }
    else if (c < qd + kd) { dst = k; stride = kd; col = c - qd; }
    else { dst = v; stride = vd; col = c - qd - kd; norm = false; }
    for (size_t t = 0; t < n; t++) {
        const float xin = x[t * ch + c];
        float acc = 0.0f;
        acc += w0 * s0;
        acc += w1 * s1;
        acc += w2 * s2;
        acc += w3 * xin;
        float y = acc * sigmoidf_(acc);
        if (norm) {  // uniform over the block: its channels are one row of q or k
            const float ss = block_sum(y * y, red);
            y = y * (1.0f / sqrtf(ss + eps));
        }
        dst[t * stride + col] = y;
        s0 = s1;
        s1 = s2;
        s2 = xin;
    }
    state_out[c] = s0;
    state_out[ch + c] = s1;
    state_out[2 * ch + c] = s2;
}

// The same for a batch: a block of `dim` threads per (`dim` channels, token),
// every token at once (the window reads the previous tokens' inputs, or the
// carried state before the first).
__global__ void __launch_bounds__(256) k_conv_l2_batch(float *__restrict__ q, float *__restrict__ k,
                                                       float *__restrict__ v, float *__restrict__ state_out,
                                                       const float *__restrict__ x, const float *__restrict__ state,
                                                       const float *__restrict__ w, size_t n, size_t qd, size_t kd,
                                                       size_t vd, float eps) {
    __shared__ float red[4];
    const size_t ch = qd + kd + vd;
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    // input t' of the window: x[t'] for t' >= 0, else the state's row 3 + t'
    float in[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const long tp = (long)t + j - 3;
        in[j] = tp >= 0 ? x[(size_t)tp * ch + c] : state[(size_t)(3 + tp) * ch + c];
    }
    float acc = 0.0f;
    acc += w[c * 4] * in[0];
    acc += w[c * 4 + 1] * in[1];
    acc += w[c * 4 + 2] * in[2];
    acc += w[c * 4 + 3] * in[3];
    float y = acc * sigmoidf_(acc);
    float *dst;
    size_t stride, col;
    bool norm = true;
    if (c < qd) { dst = q; stride = qd; col = c; }
    else if (c < qd + kd) { dst = k; stride = kd; col = c - qd; }
    else { dst = v; stride = vd; col = c - qd - kd; norm = false; }
    if (norm) {  // uniform over the block
        const float ss = block_sum(y * y, red);
        y = y * (1.0f / sqrtf(ss + eps));
    }
    dst[t * stride + col] = y;
    if (t == n - 1) {
        // the last three inputs carry over
#pragma unroll
        for (int j = 0; j < 3; j++) state_out[(size_t)j * ch + c] = in[j + 1];
    }
}

// The same for kConvT tokens a block: the block's `dim` channels read each
// input row once (the window of 4 slides in registers), the weights once as
// a float4, and each token's l2 sum is a wave sum plus one exchange of the
// waves' partials.
constexpr int kConvT = 16;

__global__ void __launch_bounds__(256) k_conv_l2_tokens(float *__restrict__ q, float *__restrict__ k,
                                                        float *__restrict__ v, float *__restrict__ state_out,
                                                        const float *__restrict__ x, const float *__restrict__ state,
                                                        const float *__restrict__ w, size_t n, size_t qd, size_t kd,
                                                        size_t vd, float eps) {
    __shared__ float red[kConvT][4];
    const size_t ch = qd + kd + vd;
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x, t0 = (size_t)blockIdx.y * kConvT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const float4 wc = *(const float4 *)(w + c * 4);
    // inputs t0 − 3 .. t0 − 1: x rows, or the state's rows before the batch
    float win[3];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const long tp = (long)t0 + j - 3;
        win[j] = tp >= 0 ? x[(size_t)tp * ch + c] : state[(size_t)(3 + tp) * ch + c];
    }
    float y[kConvT];
#pragma unroll
    for (int i = 0; i < kConvT; i++) {
        const size_t t = t0 + i;
        const float xi = t < n ? x[t * ch + c] : 0.0f;
        float acc = 0.0f;
        acc += wc.x * win[0];
        acc += wc.y * win[1];
        acc += wc.z * win[2];
        acc += wc.w * xi;
        y[i] = acc * sigmoidf_(acc);
        if (t == n - 1) {
            // the last three inputs carry over
            state_out[c] = win[1];
            state_out[ch + c] = win[2];
            state_out[2 * ch + c] = xi;
        }
        win[0] = win[1];
        win[1] = win[2];
        win[2] = xi;
    }
    float *dst;
    size_t stride, col;
    bool norm = true;
    if (c < qd) { dst = q; stride = qd; col = c; }
    else if (c < qd + kd) { dst = k; stride = kd; col = c - qd; }
    else { dst = v; stride = vd; col = c - qd - kd; norm = false; }
    if (norm) {  // uniform over the block
#pragma unroll
        for (int i = 0; i < kConvT; i++) {
            const float ss = group_sum<64>(y[i] * y[i]);
            if (lane == 0) red[i][wave] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kConvT; i++) {
            float ss = 0.0f;
            for (int u = 0; u < waves; u++) ss += red[i][u];
            y[i] *= 1.0f / sqrtf(ss + eps);
        }
    }
#pragma unroll
    for (int i = 0; i < kConvT; i++)
        if (t0 + i < n) dst[(t0 + i) * stride + col] = y[i];
}

// z = silu(z) · (att · (1/rms(att) · w)) per `dim`-row (rmsnorm, gpu/cpu.rs:
// 157-166, then silu_mul, :238-242), four values a thread; with one token,
// the result's planes too.
template <int LANES>  // dim / 4: the lanes of a row
__global__ void __launch_bounds__(256) k_gated_norm(float *__restrict__ z, const float *__restrict__ att,
                                                    const float *__restrict__ w, size_t total, size_t dim, float eps,
                                                    planes::View out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // a float4 of the [n][total] rows
    if (i * 4 >= total) return;  // total is whole waves of float4s
    const float4 a = ((const float4 *)att)[i];
    const float ss = group_sum<LANES>((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w));
    const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    const float4 nw = ((const float4 *)w)[(i * 4 % dim) / 4];
    float4 g = ((const float4 *)z)[i];
    g.x = g.x * sigmoidf_(g.x) * (a.x * (scale * nw.x));
    g.y = g.y * sigmoidf_(g.y) * (a.y * (scale * nw.y));
    g.z = g.z * sigmoidf_(g.z) * (a.z * (scale * nw.z));
    g.w = g.w * sigmoidf_(g.w) * (a.w * (scale * nw.w));
    ((float4 *)z)[i] = g;
    if (out.q) planes::write4x4(out, i, g);
}

// The attention projections' epilogue for token t, one block of head_dim
// threads per head: q heads are RMS-normalized by q_norm and rotated
// (gpu/cpu.rs:157-166, 177-200); k heads too, then stored to the key cache;
// v heads stored to the value cache (gpu/cpu.rs:78-87, quantized as
// gpu/quant.rs:161-180 does, bit for bit).
__global__ void __launch_bounds__(256) k_qk_prep(float *__restrict__ q, float *__restrict__ k,
                                                 const float *__restrict__ v, const float *__restrict__ q_norm,
                                                 const float *__restrict__ k_norm, const float *__restrict__ table,
                                                 size_t pos, size_t heads, size_t kv_heads, size_t rot, float eps,
                                                 int8_t *__restrict__ kq, uint16_t *__restrict__ ks,
                                                 int8_t *__restrict__ vq, uint16_t *__restrict__ vs) {
    __shared__ float red[4];
    __shared__ float row[256];
    const size_t slot = blockIdx.x, t = blockIdx.y, D = blockDim.x, d = threadIdx.x;
    const size_t kv_dim = kv_heads * D;
    float *x;
    const float *nw = nullptr;
    int8_t *cq = nullptr;
    uint16_t *cs = nullptr;
    if (slot < heads) {
        x = q + (t * heads + slot) * D;
        nw = q_norm;
    } else if (slot < heads + kv_heads) {
        x = k + t * kv_dim + (slot - heads) * D;
        nw = k_norm;
        cq = kq + (pos + t) * kv_dim + (slot - heads) * D;
        cs = ks + ((pos + t) * kv_dim + (slot - heads) * D) / 32;
    } else {
        x = (float *)v + t * kv_dim + (slot - heads - kv_heads) * D;
        cq = vq + (pos + t) * kv_dim + (slot - heads - kv_heads) * D;
        cs = vs + ((pos + t) * kv_dim + (slot - heads - kv_heads) * D) / 32;
    }
    float y = x[d];
    if (nw) {  // uniform over the block
        const float ss = block_sum(y * y, red);
        const float scale = 1.0f / sqrtf(ss / (float)D + eps);
        y = y * (scale * nw[d]);
        row[d] = y;
        __syncthreads();
        const size_t half = rot / 2;
        if (d < half) {
            const float *ang = table + (pos + t) * rot + 2 * d;
            const float c = ang[0], sn = ang[1], a = row[d], b = row[d + half];
            y = a * c - b * sn;
        } else if (d < rot) {
            const float *ang = table + (pos + t) * rot + 2 * (d - half);
            const float c = ang[0], sn = ang[1], a = row[d - half], b = row[d];
            y = b * c + a * sn;
        }
        x[d] = y;
    }
    if (cq) {
        float amax = fabsf(y);
#pragma unroll
        for (int m = 16; m > 0; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
        const uint16_t bits = dq::block_scale(amax);
        const float dd = dq::from_f16(bits);
        cq[d] = dd > 0.0f ? dq::quantize_one(y, dd) : (int8_t)0;
        if ((d & 31) == 0) cs[d / 32] = bits;
    }
}

}  // namespace

hipError_t launch_conv_l2(hipStream_t s, float *q, float *k, float *v, float *state_out, const float *x,
                          const float *state, const float *w, size_t n, size_t qd, size_t kd, size_t vd, size_t dim,
                          float eps) {
    if (dim % 64 || dim > 256 || qd % dim || kd % dim || vd % dim) return hipErrorInvalidValue;
    if (n == 1)
        k_conv_l2<<<(unsigned)((qd + kd + vd) / dim), (unsigned)dim, 0, s>>>(q, k, v, state_out, x, state, w, n, qd,
                                                                             kd, vd, eps);
    else if (n < (size_t)kConvT)
        k_conv_l2_batch<<<dim3((unsigned)((qd + kd + vd) / dim), (unsigned)n), (unsigned)dim, 0, s>>>(
            q, k, v, state_out, x, state, w, n, qd, kd, vd, eps);
    else
        k_conv_l2_tokens<<<dim3((unsigned)((qd + kd + vd) / dim), (unsigned)((n + kConvT - 1) / kConvT)),
                           (unsigned)dim, 0, s>>>(q, k, v, state_out, x, state, w, n, qd, kd, vd, eps);
    return hipGetLastError();
}

hipError_t launch_gated_norm(dwim_dev *dev, float *z, const float *att, const float *w, size_t n, size_t total,
                             size_t dim, float eps, int area) {
    if (total % 256 || dim % 4 || (dim != 128 && dim != 256)) return hipErrorInvalidValue;
    planes::View out{};
    if (area >= 0) {
        if (n != 1 || total > planes::kMaxCols) return hipErrorInvalidValue;
        out = planes_area(dev, area, total);
        dev->prepared = 0;
    }
    const size_t f4 = n * total / 4;
    const unsigned blocks = (unsigned)((f4 + 255) / 256);
    if (dim == 128) k_gated_norm<32><<<blocks, 256, 0, dev->stream>>>(z, att, w, n * total, dim, eps, out);
    else k_gated_norm<64><<<blocks, 256, 0, dev->stream>>>(z, att, w, n * total, dim, eps, out);
    return hipGetLastError();
}

hipError_t launch_qk_prep(hipStream_t s, float *q, float *k, const float *v, const float *q_norm,
                          const float *k_norm, const float *table, size_t n, size_t pos, size_t heads,
                          size_t kv_heads, size_t head_dim, size_t rot, float eps, dwim_cache *kc, dwim_cache *vc) {
    if (head_dim % 64 || head_dim > 256 || rot > head_dim || rot % 2 || kc->f16 || vc->f16)
        return hipErrorInvalidValue;
    dim3 grid((unsigned)(heads + 2 * kv_heads), (unsigned)n);
    k_qk_prep<<<grid, (unsigned)head_dim, 0, s>>>(q, k, v, q_norm, k_norm, table, pos, heads, kv_heads, rot, eps,
                                                  kc->q, kc->s, vc->q, vc->s);
    return hipGetLastError();
}
