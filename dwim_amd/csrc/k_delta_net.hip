// The gated delta rule of linear attention, token after token
// (dwim gpu/cpu.rs:298-363).  For value head h (key head h / (n_v/n_k)) and
// each token: g = exp(a·softplus(alpha + dt_bias)), beta = sigmoid(beta_logit);
// S *= g; kv = Sᵀk; S += k ⊗ (v − kv)·beta; o = Sᵀq / sqrt(d); with the state
// S stored s[key][value].
//
// Every value column j of S evolves on its own: kv[j], the update of column j
// and o[j] read only column j.  So a block owns 16 columns of one head (grid
// = 8 × n_v_heads) and keeps its 128×16 slice of the fp32 state in registers
// across all the batch's tokens: thread (column c, part p) holds keys
// 8p..8p+7 of column c, and the 16 parts of a column are 16 adjacent lanes
// whose partial sums meet by DPP moves.  The token loop is a chain of
// dependent steps, so it is kept short and free of global loads: the inputs
// of a run of 64 tokens (keys, queries, the block's values, the gates g and
// beta) are staged in LDS at once, the next run's loaded into registers while
// this run's tokens are computed, and each sum runs in two accumulators.  The
// slice is read from HBM once and written once per call, through LDS so that
// both are coalesced.
#include "device_util.h"
#include "runtime.h"

typedef float v4f __attribute__((ext_vector_type(4)));

namespace {

constexpr int kD = 128;      // head_dim (the reference asserts 128, gpu/cuda/mod.rs:1437)
constexpr int kCols = 16;    // value columns per block
constexpr int kParts = 16;   // key parts per column
constexpr int kKeys = kD / kParts;
constexpr int kThreads = kCols * kParts;
constexpr int kRun = 64;  // tokens whose inputs a block stages in LDS at once

// sum over 16 aligned adjacent lanes, every lane getting it: quad xor 1 and
// 2, then the half-row mirror (lane i and 7 − i) and the row mirror (i and
// 15 − i)
DEV float sum16(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xf, 0xf, false));
    return v;
}

__global__ void __launch_bounds__(kThreads) k_delta_net(float *__restrict__ out, const float *__restrict__ q,
                                                        const float *__restrict__ k, const float *__restrict__ v,
                                                        const float *__restrict__ gates,
                                                        const float *__restrict__ decay, float *__restrict__ state,
                                                        size_t n, int n_k_heads, int n_v_heads, Rms rms) {
    // a run's keys and queries [token][key] (also the state slice's staging
    // at the start and the end), values [token][column] and gates
    __shared__ v4f kq[2][kRun][kD / 4];
    __shared__ float vs[kRun][kCols];
    __shared__ float2 gb[kRun];  // per token: g, beta
    __shared__ float red[kThreads / 64];
    float(*tile)[kCols + 1] = (float(*)[kCols + 1]) & kq[0][0][0];  // [kD][kCols + 1]
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

    // state slice in: rows of 16 columns, coalesced
    for (int e = threadIdx.x; e < kD * kCols; e += kThreads) tile[e / kCols][e % kCols] = S[(e / kCols) * kD + c0 + e % kCols];
    __syncthreads();
    float s[kKeys];
#pragma unroll
    for (int i = 0; i < kKeys; i++) s[i] = tile[p * kKeys + i][c];

    const float scale = 1.0f / sqrtf((float)kD);
    const float a = decay[h], dt = decay[n_v_heads + h];
    // a run's inputs, loaded into registers while the run before it is
    // computed: thread i takes float4s i, i + 256, ... of the run's keys and
    // queries ([2][kRun][32] float4s), and value (token i / 16, column i % 16)
    // for i < kRun·16 (four a thread), and the gate logits of token i < kRun
    constexpr int kKQ = 2 * kRun * kD / 4 / kThreads, kV = kRun * kCols / kThreads;
    v4f rkq[kKQ];  // (vector types: an array of float4 structs stays in private memory)
    float rv[kV], ra = 0.0f, rb = 0.0f;
    auto fetch = [&](size_t r0) {
        const size_t rn = n - r0 < (size_t)kRun ? n - r0 : (size_t)kRun;
#pragma unroll
        for (int u = 0; u < kKQ; u++) {
            const int f = threadIdx.x + kThreads * u, which = f / (kRun * kD / 4), tok = (f / (kD / 4)) % kRun;
            const size_t t = r0 + ((size_t)tok < rn ? tok : 0);
            rkq[u] = ((const v4f *)((which ? q : k) + (t * n_k_heads + kh) * kD))[f % (kD / 4)];
        }
#pragma unroll
        for (int u = 0; u < kV; u++) {
            const int f = threadIdx.x + kThreads * u, tok = f / kCols;
            const size_t t = r0 + ((size_t)tok < rn ? tok : 0);
            rv[u] = v[(t * n_v_heads + h) * kD + c0 + f % kCols];
        }
        if (threadIdx.x < kRun) {
            const size_t t = r0 + (threadIdx.x < rn ? threadIdx.x : 0);
            ra = gates[t * 2 * n_v_heads + h];
            rb = gates[t * 2 * n_v_heads + n_v_heads + h];
        }
    };
    if (n > 0) fetch(0);
    for (size_t r0 = 0; r0 < n; r0 += kRun) {
        const size_t rn = n - r0 < (size_t)kRun ? n - r0 : (size_t)kRun;
        __syncthreads();  // the run before has been read
#pragma unroll
        for (int u = 0; u < kKQ; u++) {
            const int f = threadIdx.x + kThreads * u;
            (&kq[0][0][0])[f] = rkq[u];
        }
#pragma unroll
        for (int u = 0; u < kV; u++) (&vs[0][0])[threadIdx.x + kThreads * u] = rv[u];
        // g = exp(a·softplus(alpha + dt_bias)), beta = sigmoid(beta_logit)
        if (threadIdx.x < kRun) gb[threadIdx.x] = make_float2(expf(a * softplusf_(gs * ra + dt)), sigmoidf_(gs * rb));
        __syncthreads();
        if (r0 + kRun < n) fetch(r0 + kRun);
        for (size_t tt = 0; tt < rn; tt++) {
            const size_t t = r0 + tt;
            float kk[kKeys], qq[kKeys];
#pragma unroll
            for (int i = 0; i < kKeys / 4; i++) {
                const v4f k4 = kq[0][tt][p * (kKeys / 4) + i], q4 = kq[1][tt][p * (kKeys / 4) + i];
                kk[4 * i] = k4.x; kk[4 * i + 1] = k4.y; kk[4 * i + 2] = k4.z; kk[4 * i + 3] = k4.w;
                qq[4 * i] = q4.x; qq[4 * i + 1] = q4.y; qq[4 * i + 2] = q4.z; qq[4 * i + 3] = q4.w;
            }
            const float2 g2 = gb[tt];
            const float g = g2.x, beta = g2.y;
            float kv0 = 0.0f, kv1 = 0.0f;
#pragma unroll
            for (int i = 0; i < kKeys; i += 2) {
                s[i] *= g;
                s[i + 1] *= g;
                kv0 += s[i] * kk[i];
                kv1 += s[i + 1] * kk[i + 1];
            }
            const float kv = sum16(kv0 + kv1);
            const float ub = (vs[tt][c] - kv) * beta;
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
            for (int i = 0; i < kKeys; i += 2) {
                s[i] += kk[i] * ub;
                s[i + 1] += kk[i + 1] * ub;
                o0 += s[i] * qq[i];
                o1 += s[i + 1] * qq[i + 1];
            }
            const float o = sum16(o0 + o1) * scale;
            if (p == 0) out[(t * n_v_heads + h) * kD + c0 + c] = o;
        }
    }

    // state slice out, through LDS
    __syncthreads();
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
