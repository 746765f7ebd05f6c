// One token through a gated-DeltaNet mixer in one launch: what the
// reference's token loop does in the calls conv, l2norm(q), l2norm(k),
// delta_net, rmsnorm(att), silu_mul(z, att) (inference/qwen35/mod.rs:606-640;
// gpu/cpu.rs:250-363, 157-166, 238-242), with the same arithmetic on the
// same values.  The gate logits W_ab · x·attn_norm come from the qkv
// product's launch and are RMS-scaled here.
#include "device_util.h"
#include "planes.h"
#include "runtime.h"

namespace {

constexpr int kD = 128;

// The step runs over 4 workgroups a head, 32 value columns each: the delta
// rule's columns are independent of each other (a column's k·S, its update
// and its share of o = Sᵀq read no other column), so a head splits without
// any exchange but the RMS norm of o.  That norm is left to the consumer:
// each workgroup writes silu(z)·o·norm_w of its columns, unnormalized, with
// their planes, and its Σo² to head_ss[h][quarter]; the product that reads
// the planes multiplies each group's scale and sum by the head's
// 1/sqrt(Σ head_ss / 128 + eps), which is the same product.  The gate
// logits come from the qkv product's launch (W_ab · x·attn_norm) and are
// RMS-scaled here; every workgroup recomputes the conv and l2 norms of its
// key head's q and k (the v channels: only its own 32).
constexpr int kQuarters = 4;
constexpr int kCols = kD / kQuarters;     // value columns a workgroup
constexpr int kST = 256;                  // threads: (column, key part) pairs
constexpr int kSParts = kST / kCols;      // 8 key parts of 16 keys
constexpr int kSKeys = kD / kSParts;

struct GdnSplitArgs {
    const float *qkv;
    const float *conv_state;
    float *conv_state_out;
    const float *conv_w;
    const float *ab;           // [2·nv]: W_ab · x·attn_norm, not yet RMS-scaled
    Rms rms;
    const float *decay;
    float *state;
    const float *z;            // [nv·D] the gate z
    const float *norm_w;       // [D]
    float *head_ss;            // [nv][4]: each quarter's Σo²
    float eps;
    unsigned nk, nv;
    planes::View out;
};

__global__ void __launch_bounds__(kST) k_gdn_split(const GdnSplitArgs a) {
    __shared__ float part[2][kSParts][kCols];
    __shared__ float qs[kD], ks[kD], vs[kCols];
    __shared__ float red[4][kST / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const unsigned h = blockIdx.x / kQuarters, qd = blockIdx.x % kQuarters, c0 = qd * kCols;
    const unsigned kh = h / (a.nv / a.nk);
    const unsigned ch = (2 * a.nk + a.nv) * kD;
    float *S = a.state + (size_t)h * kD * kD + c0;

    // ---- every load first: conv inputs (q and k of the key head: thread
    // tid; v of this quarter: threads < 32 a second channel), the gate rows
    // and x·w, the RMS partials, z and the norm weights, then the state
    const unsigned chan = tid < kD ? kh * kD + tid : (a.nk + kh) * kD + (tid - kD);
    const float cx = a.qkv[chan];
    const float c0s = a.conv_state[chan], c1s = a.conv_state[ch + chan], c2s = a.conv_state[2 * ch + chan];
    const float4 cw = ((const float4 *)a.conv_w)[chan];
    const unsigned vchan = (2 * a.nk + h) * kD + c0 + (unsigned)(tid % kCols);
    const float vx = a.qkv[vchan];
    const float v0s = a.conv_state[vchan], v1s = a.conv_state[ch + vchan], v2s = a.conv_state[2 * ch + vchan];
    const float4 vcw = ((const float4 *)a.conv_w)[vchan];
    const float la = a.ab[h], lb = a.ab[a.nv + h];
    // (two loads a thread, unrolled: a load in a loop waits for itself, and
    // the state loads behind it would wait for that too)
    const unsigned g1 = (unsigned)tid + kST;
    const float ss0 = (unsigned)tid < a.rms.groups ? a.rms.ss[tid] : 0.0f;
    const float ss1 = g1 < a.rms.groups ? a.rms.ss[g1] : 0.0f;
    const int c = tid % kCols, p = tid / kCols;
    const float zc = a.z[h * kD + c0 + c], nwc = a.norm_w[c0 + c];
    const float dec_a = a.decay[h], dec_dt = a.decay[a.nv + h];
    float s[kSKeys];
#pragma unroll
    for (int i = 0; i < kSKeys; i++) s[i] = S[(p * kSKeys + i) * kD + c];

    // ---- conv + SiLU: q and k channels, and this quarter's v channels
    float y;
    {
        const float acc = cw.x * c0s + cw.y * c1s + cw.z * c2s + cw.w * cx;
        y = acc * sigmoidf_(acc);
        if (h % (a.nv / a.nk) == 0 && qd == 0) {
            a.conv_state_out[chan] = c1s;
            a.conv_state_out[ch + chan] = c2s;
            a.conv_state_out[2 * ch + chan] = cx;
        }
    }
    if (tid < kCols) {
        const float acc = vcw.x * v0s + vcw.y * v1s + vcw.z * v2s + vcw.w * vx;
        vs[tid] = acc * sigmoidf_(acc);
        a.conv_state_out[vchan] = v1s;
        a.conv_state_out[ch + vchan] = v2s;
        a.conv_state_out[2 * ch + vchan] = vx;
    }

    // ---- one block reduction: the RMS sum, |q|² (waves 0-1), |k|² (2-3)
    {
        const float v[2] = {ss0 + ss1, y * y};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float t = group_sum<64>(v[i]);
            if (lane == 0) red[2 + i][wave] = t;
        }
    }
    __syncthreads();
    const float ss = (red[2][0] + red[2][1]) + (red[2][2] + red[2][3]);
    const float gs = 1.0f / sqrtf(ss / a.rms.cols + a.rms.eps);
    const float alpha = gs * la, beta = sigmoidf_(gs * lb);
    const float g = expf(dec_a * softplusf_(alpha + dec_dt));
    if (tid < kD) qs[tid] = y * (1.0f / sqrtf((red[3][0] + red[3][1]) + a.eps));
    else ks[tid - kD] = y * (1.0f / sqrtf((red[3][2] + red[3][3]) + a.eps));
    __syncthreads();

    // ---- the delta rule: thread (column c, part p), keys 16p..16p+15
    float kv = 0.0f;
#pragma unroll
    for (int i = 0; i < kSKeys; i++) {
        s[i] *= g;
        kv += s[i] * ks[p * kSKeys + i];
    }
    part[0][p][c] = kv;
    __syncthreads();
    kv = 0.0f;
#pragma unroll
    for (int q = 0; q < kSParts; q++) kv += part[0][q][c];
    const float ub = (vs[c] - kv) * beta;
    const float scale = 1.0f / sqrtf((float)kD);
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < kSKeys; i++) {
        s[i] += ks[p * kSKeys + i] * ub;
        o += s[i] * qs[p * kSKeys + i];
    }
#pragma unroll
    for (int i = 0; i < kSKeys; i++) S[(p * kSKeys + i) * kD + c] = s[i];
    part[1][p][c] = o * scale;
    __syncthreads();

    // ---- the unnormalized gated output of the quarter's columns (wave 0,
    // lanes < 32) and its Σo²
    if (tid < kCols) {
        float ov = 0.0f;
#pragma unroll
        for (int q = 0; q < kSParts; q++) ov += part[1][q][tid];
        const float ss = group_sum<kCols>(ov * ov);
        if (tid == 0) a.head_ss[h * kQuarters + qd] = ss;
        const float r = zc * sigmoidf_(zc) * (ov * nwc);
        planes::write16(a.out, h * kD + c0 + tid, r);
    }
}

}  // namespace

hipError_t launch_gdn_split(dwim_dev *dev, const float *qkv, const float *conv_state, float *conv_state_out,
                            const float *conv_w, const float *ab, const Rms &rms, const float *decay, float *state,
                            const float *z, const float *norm_w, float eps, size_t nk, size_t nv, size_t head_dim,
                            float *head_ss, int area) {
    if (head_dim != kD || nk == 0 || nv % nk || !rms.ss || rms.groups > 2 * kST || area < 0 || !head_ss || !ab)
        return hipErrorInvalidValue;
    if (nv * kD > planes::kMaxCols || (nv * kD) % 256) return hipErrorInvalidValue;
    GdnSplitArgs a{};
    a.qkv = qkv;
    a.conv_state = conv_state;
    a.conv_state_out = conv_state_out;
    a.conv_w = conv_w;
    a.ab = ab;
    a.rms = rms;
    a.decay = decay;
    a.state = state;
    a.z = z;
    a.norm_w = norm_w;
    a.head_ss = head_ss;
    a.eps = eps;
    a.nk = (unsigned)nk;
    a.nv = (unsigned)nv;
    a.out = planes_area(dev, area, nv * kD);
    dev->prepared = 0;
    k_gdn_split<<<(unsigned)(nv * kQuarters), kST, 0, dev->stream>>>(a);
    return hipGetLastError();
}
