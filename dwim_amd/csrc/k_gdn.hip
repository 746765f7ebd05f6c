// One token through a gated-DeltaNet mixer in one launch: what the
// reference's token loop does in the calls matmul(ab), conv, l2norm(q),
// l2norm(k), delta_net, rmsnorm(att), silu_mul(z, att) (inference/qwen35/
// mod.rs:606-640; gpu/cpu.rs:168-175, 250-363, 157-166, 238-242), with the
// same arithmetic on the same values.
//
// A workgroup of 1024 threads owns one value head h (key head h / (n_v/n_k)):
//   * the gate logits alpha_h, beta_h: two bf16 rows of W_ab against the
//     layer input x·attn_norm (f32, unscaled), times its RMS scale
//     1/sqrt(Σ ss / cols + eps) from the per-group sums of squares;
//   * the causal conv + SiLU of the 384 channels it reads (the key head's q
//     and k, its own v), then the l2 norms of q and k;
//   * the delta rule over its 128×128 fp32 state, read from HBM once and
//     written once, straight from registers: thread (value c, part p) holds
//     keys 16p..16p+15 of value column c, so that the 64 lanes of a wave read
//     and write 64 consecutive values of a key row; the sums over keys meet
//     across the eight parts in LDS;
//   * o = Sᵀq/√128, RMS-normalized by the head's norm weights and gated by
//     silu(z): z_h ← silu(z_h)·rmsnorm(o), with its planes for the out
//     product when asked.
// The conv state of q/k channels is written by the key head's first value
// head, that of v channels by its own.
#include "device_util.h"
#include "planes.h"
#include "runtime.h"

namespace {

constexpr int kD = 128;
constexpr int kT = 1024;
constexpr int kParts = kT / kD;  // key parts: thread tid takes value tid % kD, keys of part tid / kD
constexpr int kKeys = kD / kParts;

struct GdnArgs {
    const float *qkv;          // [q: nk·D | k: nk·D | v: nv·D]
    const float *conv_state;   // [3][ch]
    float *conv_state_out;     // [3][ch]
    const float *conv_w;       // [ch][4]
    const uint16_t *w_ab;      // bf16 [2·nv][cols]: alpha rows, then beta rows
    const float *xw;           // [cols]: x·attn_norm, unscaled
    Rms rms;
    const float *decay;        // [a ×nv, dt_bias ×nv]
    float *state;              // [nv][D][D], s[key][value]
    float *z;                  // [nv·D], in: the gate z, out: silu(z)·rmsnorm(o)
    const float *norm_w;       // [D]
    float eps;
    unsigned nk, nv, cols;
    planes::View out;          // planes of the result (q = null: none)
};

DEV float bf16f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__global__ void __launch_bounds__(kT) k_gdn(const GdnArgs a) {
    __shared__ float part[2][kParts][kD];  // per-part sums over keys, per value column: k·S, then q·S
    __shared__ float qs[kD], ks[kD], vs[kD];
    __shared__ float red[4][kT / 64];   // wave sums: gate logits, RMS partials, q and k squares
    __shared__ float ored[2];          // the o norm's wave sums
    const int tid = threadIdx.x;
    const unsigned h = blockIdx.x, kh = h / (a.nv / a.nk);
    const unsigned ch = (2 * a.nk + a.nv) * kD;
    float *S = a.state + (size_t)h * kD * kD;

    // ---- every load first: the conv inputs of 384 channels, the gate rows
    // and x·w, the RMS partials, then the state (16 floats a thread, a wave's
    // loads 256 contiguous bytes), which is needed last
    // conv channel of thread tid < 384: q of kh, k of kh, v of h
    const int which = tid / kD, cc = tid % kD;
    const unsigned chan = which == 0 ? kh * kD + cc : which == 1 ? (a.nk + kh) * kD + cc : (2 * a.nk + h) * kD + cc;
    const unsigned chan_c = tid < 3 * kD ? chan : 0u;
    const float cx = a.qkv[chan_c];
    const float c0 = a.conv_state[chan_c], c1 = a.conv_state[ch + chan_c], c2 = a.conv_state[2 * ch + chan_c];
    const float4 cw = ((const float4 *)a.conv_w)[chan_c];
    // gate rows: thread tid < cols/8 takes 8 columns of both rows
    const unsigned n8 = a.cols / 8, e8 = (unsigned)tid < n8 ? (unsigned)tid : 0u;
    const uint4 wa = ((const uint4 *)(a.w_ab + (size_t)h * a.cols))[e8];
    const uint4 wb = ((const uint4 *)(a.w_ab + (size_t)(a.nv + h) * a.cols))[e8];
    const float4 x0 = ((const float4 *)a.xw)[2 * e8], x1 = ((const float4 *)a.xw)[2 * e8 + 1];
    const unsigned g0 = (unsigned)tid < a.rms.groups ? (unsigned)tid : 0u;
    const float ssp = a.rms.ss[g0];
    const float zc = a.z[h * kD + (tid % kD)], nwc = a.norm_w[tid % kD];
    const float dec_a = a.decay[h], dec_dt = a.decay[a.nv + h];
    const int c = tid % kD, p = tid / kD;
    float s[kKeys];
#pragma unroll
    for (int i = 0; i < kKeys; i++) s[i] = S[(p * kKeys + i) * kD + c];

    // ---- conv + SiLU of the 384 channels, their state carried over
    float y = 0.0f;
    if (tid < 3 * kD) {
        float acc = 0.0f;
        acc += cw.x * c0;
        acc += cw.y * c1;
        acc += cw.z * c2;
        acc += cw.w * cx;
        y = acc * sigmoidf_(acc);
        const bool writer = which == 2 || h % (a.nv / a.nk) == 0;
        if (writer) {
            a.conv_state_out[chan] = c1;
            a.conv_state_out[ch + chan] = c2;
            a.conv_state_out[2 * ch + chan] = cx;
        }
    }

    // ---- one block reduction: the gate logits, the RMS scale and the l2
    // norms of q (waves 0-1) and k (waves 2-3)
    float da = 0.0f, db = 0.0f;
    if ((unsigned)tid < n8) {
        const uint32_t pa[4] = {wa.x, wa.y, wa.z, wa.w}, pb[4] = {wb.x, wb.y, wb.z, wb.w};
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            da += bf16f((uint16_t)(pa[i] & 0xffffu)) * xs[2 * i] + bf16f((uint16_t)(pa[i] >> 16)) * xs[2 * i + 1];
            db += bf16f((uint16_t)(pb[i] & 0xffffu)) * xs[2 * i] + bf16f((uint16_t)(pb[i] >> 16)) * xs[2 * i + 1];
        }
    }
    {
        const float v[4] = {da, db, (unsigned)tid < a.rms.groups ? ssp : 0.0f, tid < 2 * kD ? y * y : 0.0f};
        const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float t = group_sum<64>(v[i]);
            if (lane == 0) red[i][wave] = t;
        }
    }
    __syncthreads();
    float sums[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
        float t = 0.0f;
        for (int w = 0; w < kT / 64; w++) t += red[i][w];
        sums[i] = t;
    }
    const float gs = 1.0f / sqrtf(sums[2] / a.rms.cols + a.rms.eps);
    const float alpha = gs * sums[0], beta = sigmoidf_(gs * sums[1]);
    const float g = expf(dec_a * softplusf_(alpha + dec_dt));
    if (tid < kD) qs[tid] = y * (1.0f / sqrtf((red[3][0] + red[3][1]) + a.eps));
    else if (tid < 2 * kD) ks[tid - kD] = y * (1.0f / sqrtf((red[3][2] + red[3][3]) + a.eps));
    else if (tid < 3 * kD) vs[tid - 2 * kD] = y;
    __syncthreads();

    // ---- the delta rule: thread (value c, part p), keys 16p..16p+15
    float kv = 0.0f;
#pragma unroll
    for (int i = 0; i < kKeys; i++) {
        s[i] *= g;
        kv += s[i] * ks[p * kKeys + i];
    }
    part[0][p][c] = kv;
    __syncthreads();
    kv = 0.0f;
#pragma unroll
    for (int q = 0; q < kParts; q++) kv += part[0][q][c];
    const float ub = (vs[c] - kv) * beta;
    const float scale = 1.0f / sqrtf((float)kD);
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < kKeys; i++) {
        s[i] += ks[p * kKeys + i] * ub;
        o += s[i] * qs[p * kKeys + i];
    }
#pragma unroll
    for (int i = 0; i < kKeys; i++) S[(p * kKeys + i) * kD + c] = s[i];
    part[1][p][c] = o * scale;
    __syncthreads();

    // ---- the gated norm of o (threads < 128)
    float ov = 0.0f;
    if (tid < kD) {
#pragma unroll
        for (int q = 0; q < kParts; q++) ov += part[1][q][tid];
        const float ss = group_sum<64>(ov * ov);
        if ((tid & 63) == 0) ored[tid >> 6] = ss;
    }
    __syncthreads();
    if (tid < kD) {
        const float sc = 1.0f / sqrtf((ored[0] + ored[1]) / (float)kD + a.eps);
        const float r = zc * sigmoidf_(zc) * (ov * (sc * nwc));
        a.z[h * kD + tid] = r;
        if (a.out.q) planes::write16(a.out, h * kD + tid, r);
    }
}

// The same step over 4 workgroups a head, 32 value columns each: the delta
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

hipError_t launch_gdn(dwim_dev *dev, const float *qkv, const float *conv_state, float *conv_state_out,
                      const float *conv_w, const dwim_weight *w_ab, const float *xw, const Rms &rms,
                      const float *decay, float *state, float *z, const float *norm_w, float eps, size_t nk,
                      size_t nv, size_t head_dim, int area) {
    if (head_dim != kD || nk == 0 || nv % nk || w_ab->fmt != DWIM_BF16 || w_ab->rows != 2 * nv ||
        w_ab->cols % 8 || w_ab->cols / 8 > kT || rms.groups > kT || !rms.ss)
        return hipErrorInvalidValue;
    GdnArgs a{};
    a.qkv = qkv;
    a.conv_state = conv_state;
    a.conv_state_out = conv_state_out;
    a.conv_w = conv_w;
    a.w_ab = (const uint16_t *)w_ab->q;
    a.xw = xw;
    a.rms = rms;
    a.decay = decay;
    a.state = state;
    a.z = z;
    a.norm_w = norm_w;
    a.eps = eps;
    a.nk = (unsigned)nk;
    a.nv = (unsigned)nv;
    a.cols = (unsigned)w_ab->cols;
    if (area >= 0) {
        if (nv * kD > planes::kMaxCols || (nv * kD) % 256) return hipErrorInvalidValue;
        a.out = planes_area(dev, area, nv * kD);
        dev->prepared = 0;
    }
    k_gdn<<<(unsigned)nv, kT, 0, dev->stream>>>(a);
    return hipGetLastError();
}

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
