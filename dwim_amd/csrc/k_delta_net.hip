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
#include "planes.h"
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
                                                        const float *__restrict__ decay, float *state,
                                                        const float *state_in, size_t n, int n_k_heads, int n_v_heads,
                                                        Rms rms) {
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
    const float *Sin = state_in + (size_t)h * kD * kD;

    // state slice in (from state_in, out to state): rows of 16 columns, coalesced
    for (int e = threadIdx.x; e < kD * kCols; e += kThreads) tile[e / kCols][e % kCols] = Sin[(e / kCols) * kD + c0 + e % kCols];
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


// ---- A small batch's whole mixer step --------------------------------------
//
// For batches of up to kSmallT tokens (speculative-decoding verify batches,
// the rewind's re-run, small prompt pieces): the conv of 4 taps + SiLU over
// the batch with its carried state (gpu/cpu.rs:250-296), the l2 norms of q
// and k (:157-166 without weights) and the delta rule (:298-363), in one
// launch of k_delta_net's blocks (16 value columns of one head a block, the
// state slice in registers).  Each block makes its key head's q and k itself
// (a channel a thread, the window sliding in registers, each token's norm a
// block sum) and its own 16 value channels, straight into the LDS the token
// loop reads; the conv state carried to the next batch is written by the key
// head's first block (q and k channels) and by each block (its value
// channels).  The same arithmetic as the three calls it replaces.
constexpr int kSmallT = 16;

__global__ void __launch_bounds__(kThreads) k_gdn_tokens(float *__restrict__ out, const float *__restrict__ qkv,
                                                         const float *__restrict__ conv_state,
                                                         float *__restrict__ conv_state_out,
                                                         const float *__restrict__ conv_w,
                                                         const float *__restrict__ gates,
                                                         const float *__restrict__ decay, float *state,
                                                         const float *state_in, int n, int n_k_heads, int n_v_heads,
                                                         float eps, GdnSteps steps, GdnGate gg) {
    __shared__ float kqs[2][kSmallT][kD];          // normalized k, q of each token
    __shared__ float tile[kD][kCols + 1];          // the state slice's staging
    __shared__ float vs[kSmallT][kCols];
    __shared__ float2 gb[kSmallT];
    __shared__ float red[kSmallT][kThreads / 64];
    __shared__ float o_s[4][kCols];  // (with gg.planes: the first 4 tokens' o)
    const int h = blockIdx.y, c0 = blockIdx.x * kCols, tid = threadIdx.x;
    const int ratio = n_v_heads / n_k_heads, kh = h / ratio;
    const int c = tid / kParts, p = tid % kParts;
    const size_t ch = (size_t)(2 * n_k_heads + n_v_heads) * kD;
    float *S = state + (size_t)h * kD * kD;
    const float *Sin = state_in + (size_t)h * kD * kD;

    // ---- loads: the state slice, this thread's q or k channel over the
    // batch (with its window and weights), the block's value channels, the
    // gate logits
    // (every load of the block issues before any is waited for: the slice
    // into registers here, into LDS once the others are issued)
    constexpr int kTileLoads = kD * kCols / kThreads;
    float tl[kTileLoads];
#pragma unroll
    for (int u = 0; u < kTileLoads; u++) {
        const int e = tid + u * kThreads;
        tl[u] = Sin[(e / kCols) * kD + c0 + e % kCols];
    }
    const size_t qk = tid < kD ? (size_t)kh * kD + tid : (size_t)(n_k_heads + kh) * kD + (tid - kD);
    float win[kSmallT + 3];
#pragma unroll
    for (int j = 0; j < 3; j++) win[j] = conv_state[(size_t)j * ch + qk];
#pragma unroll
    for (int t = 0; t < kSmallT; t++) win[3 + t] = t < n ? qkv[(size_t)t * ch + qk] : 0.0f;
    const float4 w = ((const float4 *)conv_w)[qk];
    const size_t vc = (size_t)(2 * n_k_heads + h) * kD + c0 + (tid % kCols);
    const bool vlane = tid < kCols;
    const float a = decay[h], dt = decay[n_v_heads + h];
    // the value lanes' channels (loaded by all of wave 0, so that the loads
    // issue here, unconditionally within the wave) and the gate logits
    float vw[kSmallT + 3];
    float4 vwt = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (tid < 64) {
#pragma unroll
        for (int j = 0; j < 3; j++) vw[j] = conv_state[(size_t)j * ch + vc];
#pragma unroll
        for (int t = 0; t < kSmallT; t++) vw[3 + t] = t < n ? qkv[(size_t)t * ch + vc] : 0.0f;
        vwt = ((const float4 *)conv_w)[vc];
    }
    // (with gg.planes: wave 0, lane 16t + c, takes token t's column c at the end)
    float zv = 0.0f, nwv = 0.0f;
    if (gg.planes && tid < 64 && (tid >> 4) < n) {
        zv = gg.z[(size_t)(tid >> 4) * n_v_heads * kD + (size_t)h * kD + c0 + (tid & 15)];
        nwv = gg.norm_w[c0 + (tid & 15)];
    }
    float g_alpha = 0.0f, g_beta = 0.0f;
    if (tid < n) {
        g_alpha = gates[(size_t)tid * 2 * n_v_heads + h];
        g_beta = gates[(size_t)tid * 2 * n_v_heads + n_v_heads + h];
    }

    // ---- q and k: conv + SiLU, each token's sum of squares a block sum
    // over its half (q: waves 0-1, k: waves 2-3)
    float y[kSmallT];
#pragma unroll
    for (int t = 0; t < kSmallT; t++) {
        y[t] = 0.0f;
        if (t < n) {  // (uniform: the batch's tokens only)
            float acc = 0.0f;
            acc += w.x * win[t];
            acc += w.y * win[t + 1];
            acc += w.z * win[t + 2];
            acc += w.w * win[t + 3];
            y[t] = acc * sigmoidf_(acc);
            const float sq = group_sum<64>(y[t] * y[t]);
            if ((tid & 63) == 0) red[t][tid >> 6] = sq;
        }
    }
    // the last three inputs carry over: after the batch, window entries
    // n..n+2 (the state's rows when the batch is shorter); with steps, also
    // after each earlier token t, entries t+1..t+3 (the conv state of t + 1
    // kept).  Stored from the window's registers, every index a constant (a
    // branch per batch size), so that no store waits for a load of its own.
    // (a macro rather than a lambda over the array, which would put the
    // window in scratch memory)
#define DWIM_GDN_CARRY(WV, IDX)                                                                   \
    {                                                                                            \
        float c0 = 0.0f, c1 = 0.0f, c2 = 0.0f;                                                   \
        _Pragma("unroll") for (int m = 1; m <= kSmallT; m++) if (m == n) {                       \
            c0 = WV[m];                                                                          \
            c1 = WV[m + 1];                                                                      \
            c2 = WV[m + 2];                                                                      \
        }                                                                                        \
        conv_state_out[(IDX)] = c0;                                                              \
        conv_state_out[ch + (IDX)] = c1;                                                         \
        conv_state_out[2 * ch + (IDX)] = c2;                                                     \
        _Pragma("unroll") for (int t = 0; t < kMaxSteps && t + 1 < kSmallT; t++) {               \
            if (t + 1 < n && steps.conv[t]) {                                                    \
                steps.conv[t][(IDX)] = WV[t + 1];                                                \
                steps.conv[t][ch + (IDX)] = WV[t + 2];                                           \
                steps.conv[t][2 * ch + (IDX)] = WV[t + 3];                                       \
            }                                                                                    \
        }                                                                                        \
    }
    if (blockIdx.x == 0 && h % ratio == 0) DWIM_GDN_CARRY(win, qk)
    if (vlane) {
#pragma unroll
        for (int t = 0; t < kSmallT; t++) {
            if (t < n) {
                float acc = 0.0f;
                acc += vwt.x * vw[t];
                acc += vwt.y * vw[t + 1];
                acc += vwt.z * vw[t + 2];
                acc += vwt.w * vw[t + 3];
                vs[t][tid] = acc * sigmoidf_(acc);
            }
        }
        DWIM_GDN_CARRY(vw, vc)
    }
    // g = exp(a·softplus(alpha + dt_bias)), beta = sigmoid(beta_logit)
    if (tid < n) gb[tid] = make_float2(expf(a * softplusf_(g_alpha + dt)), sigmoidf_(g_beta));
#pragma unroll
    for (int u = 0; u < kTileLoads; u++) {
        const int e = tid + u * kThreads;
        tile[e / kCols][e % kCols] = tl[u];
    }
    __syncthreads();
    {
        const int half = tid >> 7;  // 0: q, 1: k
#pragma unroll
        for (int t = 0; t < kSmallT; t++) {
            if (t < n) {
                const float ss = red[t][2 * half] + red[t][2 * half + 1];
                kqs[half ? 0 : 1][t][tid & (kD - 1)] = y[t] * (1.0f / sqrtf(ss + eps));
            }
        }
    }
    float s[kKeys];
#pragma unroll
    for (int i = 0; i < kKeys; i++) s[i] = tile[p * kKeys + i][c];
    __syncthreads();

    // ---- the token loop (k_delta_net's)
    const float scale = 1.0f / sqrtf((float)kD);
    for (int t = 0; t < n; t++) {
        float kk[kKeys], qq[kKeys];
#pragma unroll
        for (int i = 0; i < kKeys; i++) {
            kk[i] = kqs[0][t][p * kKeys + i];
            qq[i] = kqs[1][t][p * kKeys + i];
        }
        const float2 g2 = gb[t];
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
        const float ub = (vs[t][c] - kv) * beta;
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int i = 0; i < kKeys; i += 2) {
            s[i] += kk[i] * ub;
            s[i + 1] += kk[i + 1] * ub;
            o0 += s[i] * qq[i];
            o1 += s[i + 1] * qq[i + 1];
        }
        const float o = sum16(o0 + o1) * scale;
        if (p == 0 && out) out[((size_t)t * n_v_heads + h) * kD + c0 + c] = o;
        if (p == 0 && gg.planes && t < 4) o_s[t][c] = o;
        if (t + 1 < n && t < kMaxSteps && steps.state[t]) {
            // the state after token t, for a rewind that keeps t + 1 tokens
            // (through LDS, a row's 16 columns in one run, as at the end)
            float *St = steps.state[t] + (size_t)h * kD * kD;
            __syncthreads();  // (the previous step's copy is done with the tile)
#pragma unroll
            for (int i = 0; i < kKeys; i++) tile[p * kKeys + i][c] = s[i];
            __syncthreads();
            for (int e = tid; e < kD * kCols; e += kThreads) St[(e / kCols) * kD + c0 + e % kCols] = tile[e / kCols][e % kCols];
        }
    }

    // ---- the state slice out, through LDS
    __syncthreads();  // (a step's copy may still read the tile; o_s is written)
    if (gg.planes && tid < 64 && (tid >> 4) < n) {
        // token t's gated output of the block's 16 columns as one planes group
        // (whole groups of 16 lanes), unnormalized, and their Σo²
        const int t = tid >> 4, cc = tid & 15;
        const float ov = o_s[t][cc];
        const float ss = group_sum<16>(ov * ov);
        if (cc == 0) gg.head_ss[((size_t)t * n_v_heads + h) * (kD / kCols) + blockIdx.x] = ss;
        const float r = zv * sigmoidf_(zv) * (ov * nwv);
        planes::write16(planes::view(gg.planes + (size_t)t * planes::kAreaBytes, (size_t)n_v_heads * kD),
                        (size_t)h * kD + c0 + cc, r);
    }
#pragma unroll
    for (int i = 0; i < kKeys; i++) tile[p * kKeys + i][c] = s[i];
    __syncthreads();
    for (int e = tid; e < kD * kCols; e += kThreads) S[(e / kCols) * kD + c0 + e % kCols] = tile[e / kCols][e % kCols];
}
#undef DWIM_GDN_CARRY

// ---- The chunked form, for batches of at least kC tokens -------------------
//
// Over a chunk of kC tokens with log decays lg_t and cumulative sums L_t (from
// the chunk's start, so γ_t = exp(L_t) ≤ 1), the token loop above unrolls to
// (the WY form of the delta rule):
//   R = V − diag(γ)·K·S                  (kC × 128, per value column)
//   U = X·R,   X = (I + A)⁻¹·diag(β),   A_ti = β_t·exp(L_t − L_i)·k_t·k_i (i < t)
//   O = (diag(γ)·Q·S + M·U) / sqrt(d),  M_ti = exp(L_t − L_i)·q_t·k_i (i ≤ t)
//   S ← γ_C·S + Kᵀ·diag(exp(L_C − L_t))·U
// where S is the state at the chunk's start.  Padding tokens past the batch
// have lg = 0, β = 0 and zero k, q, v, and change nothing.  Two kernels:
// k_dn_prep builds X, M and the decays of every (value head, chunk) in
// parallel (K·Kᵀ and Q·Kᵀ once per key head, on the fp32 matrix cores; X by
// forward substitution, a column a lane), and k_dn_chunks walks the chunks of
// a head in order with 16 of the state's value columns in registers, every
// product on the fp32 matrix cores (v_mfma_f32_16x16x4_f32).  The algebra is
// exact; the keys are unit vectors (the conv's l2 norm), so A's entries are
// at most 1 in size and the substitution is well conditioned.
constexpr int kC = 64;
// k_dn_prep's LDS for `ratio` value heads a key head
constexpr size_t kPrepMaxLds = 160 * 1024;  // a workgroup's LDS on gfx950

size_t prep_lds_bytes(int ratio) {
    return (size_t)ratio * kC * sizeof(double) + ((size_t)ratio * kC + (1 + (ratio < 4 ? ratio : 4)) * kC * kC) * sizeof(float);
}

DEV v4f mfma4(float a, float b, v4f c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// grid (chunks, key heads), 256 threads.  X, M: [n_v][chunks][kC][kC];
// dec: [n_v][chunks][2][kC] (γ_t = exp(L_t), then exp(L_C − L_t))
__global__ void __launch_bounds__(256) k_dn_prep(const float *__restrict__ q, const float *__restrict__ k,
                                                 const float *__restrict__ gates, const float *__restrict__ decay,
                                                 float *__restrict__ X, float *__restrict__ M, float *__restrict__ dec,
                                                 size_t n, int n_k, int n_v) {
    // LDS: each value head's cumulative log decays (double) and betas, K·Kᵀ,
    // and an A matrix for each of up to 4 heads solved at once
    extern __shared__ double prep_lds[];
    const int ratio = n_v / n_k;
    double(*Ls)[kC] = (double(*)[kC])prep_lds;
    float(*bs)[kC] = (float(*)[kC])(prep_lds + ratio * kC);
    float(*kk)[kC] = (float(*)[kC])(bs + ratio);
    float(*A)[kC][kC] = (float(*)[kC][kC])(kk + kC);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r = lane & 15, kq = lane >> 4;
    const size_t ch = blockIdx.x, nch = gridDim.x, t0 = ch * kC;
    const int kh = blockIdx.y;
    const size_t stride = (size_t)n_k * kD;
    // K·Kᵀ (all sixteen 16×16 tiles: it is read by columns below) and Q·Kᵀ
    // (the ten on and below the diagonal); lane (kq, r) feeds A[r][kq] and
    // B[kq][r] with keys 4kq + j of each 16
    // every value head's decays: g_t = exp(lg_t), lg_t = a·softplus(alpha +
    // dt_bias), beta_t = sigmoid(beta logit); L_t = Σ lg up to t, in double:
    // differences of sums of up to 64 terms are taken below
    for (int rr = w; rr < ratio; rr += 4) {
        const int h = kh * ratio + rr;
        const size_t t = t0 + lane;
        float lg = 0.0f, beta = 0.0f;
        if (t < n) {
            lg = decay[h] * softplusf_(gates[t * 2 * n_v + h] + decay[n_v + h]);
            beta = sigmoidf_(gates[t * 2 * n_v + n_v + h]);
        }
        double L = lg;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const double u = __shfl_up(L, o, 64);
            if (lane >= o) L += u;
        }
        const double LC = __shfl(L, 63, 64);
        const size_t base = (size_t)h * nch + ch;
        dec[base * 2 * kC + lane] = expf((float)L);
        dec[base * 2 * kC + kC + lane] = expf((float)(LC - L));
        Ls[rr][lane] = L;
        bs[rr][lane] = beta;
    }
    __syncthreads();
    // K·Kᵀ (all sixteen 16×16 tiles: it is read by columns below) and Q·Kᵀ
    // (the ten on and below the diagonal); lane (kq, r) feeds A[r][kq] and
    // B[kq][r] with keys 4kq + j of each 16
    for (int job = w; job < 26; job += 4) {
        const int which = job >= 16;
        int ti, tj;
        if (!which) {
            ti = job / 4;
            tj = job % 4;
        } else {
            int jj = job - 16;
            ti = 0;
            while (jj > ti) jj -= ++ti;
            tj = jj;
        }
        const size_t ta = t0 + 16 * ti + r, tb = t0 + 16 * tj + r;
        const float za = ta < n ? 1.0f : 0.0f, zb = tb < n ? 1.0f : 0.0f;
        const float *pa = (which ? q : k) + (ta < n ? ta : 0) * stride + kh * kD + 4 * kq;
        const float *pb = k + (tb < n ? tb : 0) * stride + kh * kD + 4 * kq;
        v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < kD / 16; m++) {
            const v4f a = *(const v4f *)(pa + 16 * m) * za, b = *(const v4f *)(pb + 16 * m) * zb;
            acc = mfma4(a.x, b.x, acc);
            acc = mfma4(a.y, b.y, acc);
            acc = mfma4(a.z, b.z, acc);
            acc = mfma4(a.w, b.w, acc);
        }
        if (!which) {
#pragma unroll
            for (int i = 0; i < 4; i++) kk[16 * ti + 4 * kq + i][16 * tj + r] = acc[i];
        } else {
            // M_tc = exp(L_t − L_c)·q_t·k_c for c ≤ t, of every value head
            // (the tiles above the diagonal are never read)
            const int c = 16 * tj + r;
            for (int rr = 0; rr < ratio; rr++) {
                float *Mg = M + ((size_t)(kh * ratio + rr) * nch + ch) * kC * kC;
                const double Lc = Ls[rr][c];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 16 * ti + 4 * kq + i;
                    const float e = expf((float)(t >= c ? Ls[rr][t] - Lc : 0.0));
                    Mg[t * kC + c] = t >= c ? e * acc[i] : 0.0f;
                }
            }
        }
    }
    __syncthreads();
    // each value head: A, then X by forward substitution (A[w]: wave w)
    for (int rr = w; rr < ratio; rr += 4) {
        const int h = kh * ratio + rr;
        const size_t base = (size_t)h * nch + ch;
        const double L = Ls[rr][lane];
        const float beta = bs[rr][lane];
        // A by columns (At[i][t] = A_ti, lane t); L falls with t, so each
        // decay below is exp of a value ≤ 0
#pragma unroll 2
        for (int i = 0; i < kC; i++) {
            const double Li = Ls[rr][i];
            const float e = expf((float)(lane > i ? L - Li : 0.0));
            A[w][i][lane] = lane > i ? beta * e * kk[i][lane] : 0.0f;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // (I + A)·X = diag(β), right-looking: once row i of X is known, its
        // terms join every later row's sum; lane j holds column j (its rows
        // go out through LDS: 64 stores from registers would hold 64 addresses)
        float *Xg = X + base * kC * kC;
        float acc[kC];
#pragma unroll
        for (int t = 0; t < kC; t++) acc[t] = 0.0f;
#pragma unroll
        for (int i = 0; i < kC; i++) {
            const float xi = (i == lane ? bs[rr][i] : 0.0f) - acc[i];
#pragma unroll
            for (int t = (i + 4) & ~3; t < kC; t += 4) {
                const v4f a = *(const v4f *)&A[w][i][t];
                acc[t] += a.x * xi;
                acc[t + 1] += a.y * xi;
                acc[t + 2] += a.z * xi;
                acc[t + 3] += a.w * xi;
            }
#pragma unroll
            for (int t = i + 1; t < ((i + 4) & ~3); t++) acc[t] += A[w][i][t] * xi;
            A[w][i][lane] = xi;  // column i of A is spent: row i of X takes its place
            // the sums are brought up to date row by row (left to itself the
            // compiler defers them and keeps all of A in registers)
#pragma unroll
            for (int t = i + 1; t < kC; t++) asm volatile("" : "+v"(acc[t]));
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll 4
        for (int i = 0; i < kC; i++) Xg[i * kC + lane] = A[w][i][lane];
    }
}

// grid: 8 column blocks × n_v heads (all the blocks of a key head on one XCD
// when n_k is a multiple of 8), 256 threads.  Wave w holds keys 32w..32w+31
// of the block's 16 columns, as two 16×16 accumulator tiles.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) k_dn_chunks(float *__restrict__ out, const float *__restrict__ q,
                                                   const float *__restrict__ k, const float *__restrict__ v,
                                                   const float *__restrict__ X, const float *__restrict__ M,
                                                   const float *__restrict__ dec, float *__restrict__ state,
                                                   size_t n, int n_k, int n_v) {
    __shared__ float part[4][2][kC][kCols];
    __shared__ float Rs[kC][kCols], Us[kC][kCols], Ud[kC][kCols];
    // each wave's keys of the chunk, transposed ([key][token], rows padded
    // to stay 16-byte aligned without bank conflicts)
    __shared__ float KT[4][32][kC + 4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r = lane & 15, kq = lane >> 4;
    const int ratio = n_v / n_k;
    const unsigned b = blockIdx.x;
    int h, cb;
    if (n_k % 8 == 0) {
        const unsigned idx = b / 8, per = (unsigned)(ratio * 8);
        const int kh = (int)(b % 8) * (n_k / 8) + (int)(idx / per);
        h = kh * ratio + (int)((idx % per) / 8);
        cb = (int)(idx % 8);
    } else {
        h = (int)(b / 8);
        cb = (int)(b % 8);
    }
    const int kh = h / ratio, c0 = cb * kCols;
    const size_t stride = (size_t)n_k * kD, vstride = (size_t)n_v * kD;
    float *S = state + (size_t)h * kD * kD;
    v4f s[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int i = 0; i < 4; i++) s[kt][i] = S[(32 * w + 16 * kt + 4 * kq + i) * kD + c0 + r];
    const size_t nch = (n + kC - 1) / kC;
    const float scale = 1.0f / sqrtf((float)kD);
    // every global load is issued a step or more before its use: the keys
    // and queries of K·S and Q·S a chunk ahead (right after the last use),
    // the rest at the start of the chunk that uses it
    v4f kf[4][2], qf[4][2];
    auto fetch_kq = [&](size_t t0) {
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            const size_t t = t0 + 16 * tt + r;
            const float z = t < n ? 1.0f : 0.0f;
            const size_t off = (t < n ? t : 0) * stride + kh * kD + 32 * w + 4 * kq;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                kf[tt][kt] = *(const v4f *)(k + off + 16 * kt) * z;
                qf[tt][kt] = *(const v4f *)(q + off + 16 * kt) * z;
            }
        }
    };
    // X's and M's rows of token tile w, the values and decays of its tokens,
    // loaded a chunk ahead too (right after their last use)
    v4f xr[4], mr[4];
    float vv[4], gg[4], ee[4], gC;
    auto fetch_rows = [&](size_t ch) {
        const size_t t0 = ch * kC, base = (size_t)h * nch + ch;
        const float *Lc = dec + base * 2 * kC;
        const float *Xc = X + base * kC * kC + (16 * w + r) * kC + 4 * kq;
        const float *Mc = M + base * kC * kC + (16 * w + r) * kC + 4 * kq;
#pragma unroll
        for (int ut = 0; ut < 4; ut++) {
            xr[ut] = *(const v4f *)(Xc + 16 * ut);
            mr[ut] = *(const v4f *)(Mc + 16 * ut);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * w + 4 * kq + i;
            const size_t tg = t0 + t;
            vv[i] = v[(tg < n ? tg : 0) * vstride + h * kD + c0 + r] * (tg < n ? 1.0f : 0.0f);
            gg[i] = Lc[t];
            ee[i] = Lc[kC + t];
        }
        gC = Lc[kC - 1];
    };
    if (nch) {
        fetch_kq(0);
        fetch_rows(0);
    }
    for (size_t ch = 0; ch < nch; ch++) {
        const size_t t0 = ch * kC;
        // K·S and Q·S over this wave's keys, every token
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            v4f pk = {0.0f, 0.0f, 0.0f, 0.0f}, pq = pk;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const v4f a = kf[tt][kt], aq = qf[tt][kt];
                pk = mfma4(a.x, s[kt].x, pk);
                pk = mfma4(a.y, s[kt].y, pk);
                pk = mfma4(a.z, s[kt].z, pk);
                pk = mfma4(a.w, s[kt].w, pk);
                pq = mfma4(aq.x, s[kt].x, pq);
                pq = mfma4(aq.y, s[kt].y, pq);
                pq = mfma4(aq.z, s[kt].z, pq);
                pq = mfma4(aq.w, s[kt].w, pq);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                part[w][0][16 * tt + 4 * kq + i][r] = pk[i];
                part[w][1][16 * tt + 4 * kq + i][r] = pq[i];
            }
        }
#pragma unroll
        for (int tt = 0; tt < 4; tt++)
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int j = 0; j < 4; j++) KT[w][16 * kt + 4 * kq + j][16 * tt + r] = kf[tt][kt][j];
        if (ch + 1 < nch) fetch_kq(t0 + kC);
        __syncthreads();
        // token tile w: R = V − γ·K·S, and O starts as γ·Q·S
        v4f o;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * w + 4 * kq + i;
            const float ks = part[0][0][t][r] + part[1][0][t][r] + part[2][0][t][r] + part[3][0][t][r];
            const float qs = part[0][1][t][r] + part[1][1][t][r] + part[2][1][t][r] + part[3][1][t][r];
            Rs[t][r] = vv[i] - gg[i] * ks;
            o[i] = gg[i] * qs;
        }
        __syncthreads();
        // U = X·R, X lower triangular (two accumulator chains: the longest
        // chain, wave 3's, holds every wave at the next barrier)
        v4f u = {0.0f, 0.0f, 0.0f, 0.0f}, u2 = u;
#pragma unroll
        for (int ut = 0; ut < 4; ut++) {
            if (ut > w) break;
            const v4f a = xr[ut];
            u = mfma4(a.x, Rs[16 * ut + 4 * kq][r], u);
            u2 = mfma4(a.y, Rs[16 * ut + 4 * kq + 1][r], u2);
            u = mfma4(a.z, Rs[16 * ut + 4 * kq + 2][r], u);
            u2 = mfma4(a.w, Rs[16 * ut + 4 * kq + 3][r], u2);
        }
        u += u2;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * w + 4 * kq + i;
            Us[t][r] = u[i];
            Ud[t][r] = u[i] * ee[i];
        }
        __syncthreads();
        // O += M·U, M lower triangular
        v4f o2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ut = 0; ut < 4; ut++) {
            if (ut > w) break;
            const v4f a = mr[ut];
            o = mfma4(a.x, Us[16 * ut + 4 * kq][r], o);
            o2 = mfma4(a.y, Us[16 * ut + 4 * kq + 1][r], o2);
            o = mfma4(a.z, Us[16 * ut + 4 * kq + 2][r], o);
            o2 = mfma4(a.w, Us[16 * ut + 4 * kq + 3][r], o2);
        }
        o += o2;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const size_t tg = t0 + 16 * w + 4 * kq + i;
            if (tg < n) out[tg * vstride + h * kD + c0 + r] = o[i] * scale;
        }
        const float gCc = gC;
        if (ch + 1 < nch) fetch_rows(ch + 1);
        // S = γ_C·S + Kᵀ·diag(exp(L_C − L_t))·U
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            v4f d = {0.0f, 0.0f, 0.0f, 0.0f};
            s[kt] *= gCc;
#pragma unroll
            for (int ut = 0; ut < 4; ut++) {
                const v4f a = *(const v4f *)&KT[w][16 * kt + r][16 * ut + 4 * kq];
                s[kt] = mfma4(a.x, Ud[16 * ut + 4 * kq][r], s[kt]);
                d = mfma4(a.y, Ud[16 * ut + 4 * kq + 1][r], d);
                s[kt] = mfma4(a.z, Ud[16 * ut + 4 * kq + 2][r], s[kt]);
                d = mfma4(a.w, Ud[16 * ut + 4 * kq + 3][r], d);
            }
            s[kt] += d;
        }
    }
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int i = 0; i < 4; i++) S[(32 * w + 16 * kt + 4 * kq + i) * kD + c0 + r] = s[kt][i];
}

}  // namespace

// The chunked form's per-chunk matrices (X, M and the decays) for n tokens.
size_t delta_net_work_floats(size_t n, size_t n_v_heads) {
    if (n < (size_t)kC) return 0;
    const size_t nch = (n + kC - 1) / kC;
    return n_v_heads * nch * (2 * kC * kC + 2 * kC);
}

hipError_t delta_net_reserve(dwim_dev *dev, size_t n, size_t n_v_heads) {
    return dev_grow(dev, (void **)&dev->dn_work, &dev->dn_work_cap, delta_net_work_floats(n, n_v_heads),
                    sizeof(float));
}

hipError_t launch_gdn_tokens(dwim_dev *dev, float *out, const float *qkv, const float *conv_state,
                             float *conv_state_out, const float *conv_w, const float *gates, const float *decay,
                             float *state, const float *state_in, size_t n, size_t n_k_heads, size_t n_v_heads,
                             size_t head_dim, float eps, const GdnSteps *steps, const GdnGate *gate) {
    if (head_dim != kD || n < 1 || n > (size_t)kSmallT || n_k_heads == 0 || n_v_heads % n_k_heads)
        return hipErrorInvalidValue;
    if (gate && (n > 4 || !gate->z || !gate->norm_w || !gate->planes || !gate->head_ss ||
                 n_v_heads * kD > planes::kMaxCols || (n_v_heads * kD) % 256))
        return hipErrorInvalidValue;
    dim3 grid(kD / kCols, (unsigned)n_v_heads);
    k_gdn_tokens<<<grid, kThreads, 0, dev->stream>>>(out, qkv, conv_state, conv_state_out, conv_w, gates, decay, state,
                                                     state_in ? state_in : state, (int)n, (int)n_k_heads,
                                                     (int)n_v_heads, eps, steps ? *steps : GdnSteps{},
                                                     gate ? *gate : GdnGate{});
    return hipGetLastError();
}

hipError_t launch_delta_net(dwim_dev *dev, float *out, const float *q, const float *k, const float *v,
                            const float *gates, const float *decay, float *state, size_t n, size_t n_k_heads,
                            size_t n_v_heads, size_t head_dim, const Rms *rms, bool unit_keys, const float *state_in) {
    if (head_dim != (size_t)kD || n_k_heads == 0 || n_v_heads % n_k_heads) return hipErrorInvalidValue;
    if (unit_keys && n >= (size_t)kC && !(rms && rms->ss)) {
        if (state_in && state_in != state) return hipErrorInvalidValue;  // (the token loop reads one state, writes another)
        const size_t nch = (n + kC - 1) / kC;
        hipError_t e = delta_net_reserve(dev, n, n_v_heads);
        if (e != hipSuccess) return e;
        float *X = dev->dn_work, *M = X + n_v_heads * nch * kC * kC, *dec = M + n_v_heads * nch * kC * kC;
        const size_t lds = prep_lds_bytes((int)(n_v_heads / n_k_heads));
        // raised to the largest the kernel can take, once a process (a
        // function-local static is initialized once even when host threads
        // reach it together); a larger request is refused below
        static const hipError_t raised = hipFuncSetAttribute(
            (const void *)k_dn_prep, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPrepMaxLds);
        if (raised != hipSuccess) return raised;
        if (lds > kPrepMaxLds) return hipErrorInvalidValue;
        k_dn_prep<<<dim3((unsigned)nch, (unsigned)n_k_heads), 256, lds, dev->stream>>>(q, k, gates, decay, X, M, dec, n,
                                                                                   (int)n_k_heads, (int)n_v_heads);
        k_dn_chunks<<<(unsigned)(8 * n_v_heads), 256, 0, dev->stream>>>(out, q, k, v, X, M, dec, state, n,
                                                                         (int)n_k_heads, (int)n_v_heads);
        return hipGetLastError();
    }
    dim3 grid(kD / kCols, (unsigned)n_v_heads);
    k_delta_net<<<grid, kThreads, 0, dev->stream>>>(out, q, k, v, gates, decay, state, state_in ? state_in : state, n,
                                                    (int)n_k_heads,
                                                    (int)n_v_heads, rms ? *rms : Rms{});
    return hipGetLastError();
}
