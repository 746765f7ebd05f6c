// The gated delta rule of linear attention, token after token
// (dwim gpu/cpu.rs:298-363).  For value head h (key head h / (n_v/n_k)) and
// each token: g = exp(a·softplus(alpha + dt_bias)), beta = sigmoid(beta_logit);
// S *= g; kv = Sᵀk; S += k ⊗ (v − kv)·beta; o = Sᵀq / sqrt(d); with the state
// S stored s[key][value].
//
// Every value column j of S evolves on its own: kv[j], the update of column j
// and o[j] read only column j.  So a block owns 32 columns of one head (grid =
// 4 × n_v_heads) and keeps its 128×32 slice of the fp32 state in registers
// across all the batch's tokens: thread (column c, part p) holds keys
// 16p..16p+15 of column c, and the 8 parts of a column are 8 adjacent lanes
// whose partial sums meet by shuffles.  The slice is read from HBM once and
// written once per call, through LDS so that both are coalesced.
#include "device_util.h"
#include "runtime.h"

namespace {

constexpr int kD = 128;      // head_dim (the reference asserts 128, gpu/cuda/mod.rs:1437)
constexpr int kCols = 32;    // value columns per block
constexpr int kParts = 8;    // key parts per column
constexpr int kKeys = kD / kParts;
constexpr int kThreads = kCols * kParts;

__global__ void __launch_bounds__(kThreads) k_delta_net(float *__restrict__ out, const float *__restrict__ q,
                                                        const float *__restrict__ k, const float *__restrict__ v,
                                                        const float *__restrict__ gates,
                                                        const float *__restrict__ decay, float *__restrict__ state,
                                                        size_t n, int n_k_heads, int n_v_heads, Rms rms) {
    __shared__ float tile[kD][kCols + 1];
    __shared__ float red[kThreads / 64];
    // the gates' RMS scale, when the gate projection took x·w unscaled
    float gs = 1.0f;
    if (rms.ss) {
        float t = 0.0f;
        for (unsigned g = threadIdx.x; g < rms.groups; g += kThreads) t += rms.ss[g];
        t = block_sum<kThreads>(t, red);
        gs = 1.0f / sqrtf(t / rms.cols + rms.eps);
    }
    const int h = blockIdx.y, c0 = blockIdx.x * kCols;
    const int kh = h / (n_v_heads / n_k_heads);
    const int c = threadIdx.x / kParts, p = threadIdx.x % kParts;
    float *S = state + (size_t)h * kD * kD;

    // state slice in: rows of 32 columns, coalesced
    for (int e = threadIdx.x; e < kD * kCols; e += kThreads) tile[e / kCols][e % kCols] = S[(e / kCols) * kD + c0 + e % kCols];
    __syncthreads();
    float s[kKeys];
#pragma unroll
    for (int i = 0; i < kKeys; i++) s[i] = tile[p * kKeys + i][c];

    const float scale = 1.0f / sqrtf((float)kD);
    const float a = decay[h], dt = decay[n_v_heads + h];
    // token t + 1's inputs are loaded while token t is computed
    struct In {
        float4 k4[kKeys / 4], q4[kKeys / 4];
        float v, alpha, beta;
    };
    auto fetch = [&](size_t t, In &in) {
        const float4 *kt = (const float4 *)(k + (t * n_k_heads + kh) * kD + p * kKeys);
        const float4 *qt = (const float4 *)(q + (t * n_k_heads + kh) * kD + p * kKeys);
#pragma unroll
        for (int i = 0; i < kKeys / 4; i++) {
            in.k4[i] = kt[i];
            in.q4[i] = qt[i];
        }
        in.v = v[(t * n_v_heads + h) * kD + c0 + c];
        in.alpha = gates[t * 2 * n_v_heads + h];
        in.beta = gates[t * 2 * n_v_heads + n_v_heads + h];
    };
    In cur, nxt;
    if (n > 0) fetch(0, nxt);
    for (size_t t = 0; t < n; t++) {
        cur = nxt;
        if (t + 1 < n) fetch(t + 1, nxt);
        float kk[kKeys], qq[kKeys];
#pragma unroll
        for (int i = 0; i < kKeys / 4; i++) {
            kk[4 * i] = cur.k4[i].x; kk[4 * i + 1] = cur.k4[i].y; kk[4 * i + 2] = cur.k4[i].z; kk[4 * i + 3] = cur.k4[i].w;
            qq[4 * i] = cur.q4[i].x; qq[4 * i + 1] = cur.q4[i].y; qq[4 * i + 2] = cur.q4[i].z; qq[4 * i + 3] = cur.q4[i].w;
        }
        const float vj = cur.v;
        const float alpha = gs * cur.alpha;
        const float beta = sigmoidf_(gs * cur.beta);
        const float g = expf(a * softplusf_(alpha + dt));
        float kv = 0.0f;
#pragma unroll
        for (int i = 0; i < kKeys; i++) {
            s[i] *= g;
            kv += s[i] * kk[i];
        }
        kv = group_sum<kParts>(kv);
        const float u = vj - kv;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < kKeys; i++) {
            s[i] += kk[i] * u * beta;
            o += s[i] * qq[i] * scale;
        }
        o = group_sum<kParts>(o);
        if (p == 0) out[(t * n_v_heads + h) * kD + c0 + c] = o;
    }

    // state slice out, through LDS
#pragma unroll
    for (int i = 0; i < kKeys; i++) tile[p * kKeys + i][c] = s[i];
    __syncthreads();
    for (int e = threadIdx.x; e < kD * kCols; e += kThreads) S[(e / kCols) * kD + c0 + e % kCols] = tile[e / kCols][e % kCols];
}

}  // namespace

hipError_t launch_delta_net(hipStream_t s, float *out, const float *q, const float *k, const float *v,
                            const float *gates, const float *decay, float *state, size_t n, size_t n_k_heads,
                            size_t n_v_heads, size_t head_dim, const Rms *rms) {
    dim3 grid(kD / kCols, (unsigned)n_v_heads);
    k_delta_net<<<grid, kThreads, 0, s>>>(out, q, k, v, gates, decay, state, n, (int)n_k_heads, (int)n_v_heads,
                                          rms ? *rms : Rms{});
    return hipGetLastError();
}
