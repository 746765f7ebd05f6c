// Causal grouped-query attention over the key/value caches (dwim
// gpu/cpu.rs:202-236), split over chunks of 64 positions so that a single
// decode token still spreads its cache reads over the whole GPU.  A cache is
// the reference's Q8 (int8 with an f16 scale per block of 32) or f16 (each
// kernel a template on the format, F16; an f16 key or value is read as is).
//
// Pass 1, one block per (chunk, key/value head, token): the G query heads
// sharing the key/value head score the chunk's positions (a Q8 block of 32 per
// lane, its f16 scale applied to the block's sum, the 8 lanes of a position
// summed by shuffles), take the chunk's softmax numerator and weight the
// chunk's values.  Every cache load of the block is issued before any
// arithmetic.  It writes, per query head, the chunk's max, sum of
// exponentials and weighted values.  Pass 2, one block per (query head,
// token), merges the chunks.  Each cache byte is read once per token.
#include "device_util.h"
#include "planes.h"
#include "quant_math.h"
#include "runtime.h"

namespace {

constexpr int kMaxG = 8;
constexpr int kMaxD = 256;
constexpr int kPos = 64;        // positions a partial block scores
constexpr int kPThreads = 512;  // 8 lanes a position
constexpr int kQPer = kMaxG * kMaxD / kPThreads;


struct Shape {
    size_t n, pos, n_heads, head_dim, n_kv_heads, ch, chunks;
};

// partials: [token][head][chunk][head_dim + 2]  (o[...], max, sum)
//
// One pass over the chunk's kPos positions, every load issued up front.
// Scores: 8 lanes per position, lane b takes Q8 block b (32 elements) of the
// head for all G query heads.  Values: wave w takes elements 32w..32w+31 (one
// Q8 block: one scale per position), lane l elements 32w + 4(l % 8)..+3 of
// positions l/8 + 8i; the 8 position groups meet by shuffles.
DEV float half_of(uint32_t word, int hi) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? word >> 16 : word & 0xffffu));
}
DEV uint32_t word_of(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

template <int G, bool F16>
__global__ void __launch_bounds__(kPThreads) k_attn_partial(float *__restrict__ partials, const float *__restrict__ q,
                                                            const int8_t *__restrict__ kq,
                                                            const uint16_t *__restrict__ ks,
                                                            const int8_t *__restrict__ vq,
                                                            const uint16_t *__restrict__ vs, Shape sh) {
    // queries, each Q8 block of 32 padded to 36 floats: the 8 lanes of a
    // position, reading blocks 0..7 at once, then hit 8 different banks
    __shared__ float q_s[kMaxG * kMaxD / 32 * 36];
    __shared__ float p_s[kMaxG * kPos];
    __shared__ float stat_s[kMaxG * 2];
    const size_t chunk = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const int D = (int)sh.head_dim;
    const size_t kv_dim = sh.n_kv_heads * sh.head_dim;
    const size_t len = sh.pos + t + 1;  // the token attends up to its own position
    const size_t p0 = chunk * kPos;
    const size_t head0 = kvh * G;
    float *part = partials + ((t * sh.n_heads + head0) * sh.chunks + chunk) * (size_t)(D + 2);
    const size_t part_stride = sh.chunks * (size_t)(D + 2);  // next head
    if (p0 >= len) {
        // a chunk past this token's last position: empty
        if (threadIdx.x < (unsigned)G) {
            part[threadIdx.x * part_stride + D] = -INFINITY;
            part[threadIdx.x * part_stride + D + 1] = 0.0f;
        }
        return;
    }
    const int cnt = (int)min((size_t)kPos, len - p0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // the queries first: in-order completion then lets the scores wait for
    // the queries and keys alone, and the values arrive meanwhile
    float qr[kQPer];
#pragma unroll
    for (int k = 0; k < kQPer; k++) {
        const size_t i = threadIdx.x + k * kPThreads;
        qr[k] = i < (size_t)(G * D) ? q[(t * sh.n_heads + head0) * D + i] : 0.0f;
    }
    // key and value loads, unconditional (positions past the chunk's end read
    // its last position, masked later) and unconverted, so that every load is
    // in flight before the first wait
    const int kp = threadIdx.x >> 3, b = threadIdx.x & 7, nblk = D / 32;
    const bool klive = kp < cnt && b < nblk;
    uint4 kr[F16 ? 4 : 2];
    uint16_t kbits = 0;
    {
        const size_t off = (p0 + min(kp, cnt - 1)) * kv_dim + kvh * D + 32 * min(b, nblk - 1);
        if constexpr (F16) {
            const uint4 *src = (const uint4 *)((const uint16_t *)kq + off);
#pragma unroll
            for (int i = 0; i < 4; i++) kr[i] = src[i];
        } else {
            kr[0] = ((const uint4 *)(kq + off))[0];
            kr[1] = ((const uint4 *)(kq + off))[1];
            kbits = ks[off / 32];
        }
    }
    // values: wave w < nblk takes block w of the head (4 values a lane)
    const bool vlive = wave < nblk;
    uint32_t vw[kPos / 8][F16 ? 2 : 1];
    uint16_t vbits[kPos / 8];
#pragma unroll
    for (int i = 0; i < kPos / 8; i++) {
        const int vp = min((lane >> 3) + 8 * i, cnt - 1);
        const size_t off = (p0 + vp) * kv_dim + kvh * D + 32 * min(wave, nblk - 1) + 4 * (lane & 7);
        if constexpr (F16) {
            const uint2 x = *(const uint2 *)((const uint16_t *)vq + off);
            vw[i][0] = x.x;
            vw[i][F16 ? 1 : 0] = x.y;
            vbits[i] = 0;
        } else {
            vw[i][0] = *(const uint32_t *)(vq + off);
            vbits[i] = vs[off / 32];
        }
    }
    // (the query loads were issued first, so this waits for them alone)
    for (int k = 0; k < kQPer; k++) {
        const unsigned i = threadIdx.x + k * kPThreads;
        if (i < (unsigned)(G * D)) q_s[(i / 32) * 36 + i % 32] = qr[k];
    }
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)D);
    {
        const float ksc = F16 ? 1.0f : dq::from_f16(kbits);
        float kv[32];
#pragma unroll
        for (int i = 0; i < 32; i++) {
            if constexpr (F16) {
                kv[i] = half_of(word_of(kr[i / 8], (i % 8) / 2), i % 2);
            } else {
                const uint32_t w = word_of(kr[i / 16], (i % 16) / 4);
                kv[i] = (float)(int8_t)((w >> (8 * (i & 3))) & 0xff);
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float sc = 0.0f;
            if (klive) {
                const float *qg = q_s + (g * nblk + b) * 36;
#pragma unroll
                for (int i = 0; i < 32; i++) sc += qg[i] * kv[i];
            }
            sc = group_sum<8>(sc * ksc);
            if (b == 0 && kp < cnt) p_s[g * kPos + kp] = scale * sc;
        }
    }
    __syncthreads();
    // softmax numerators: wave g takes head g, a lane per position
    for (int g = wave; g < G; g += kPThreads / 64) {
        const float sc = lane < cnt ? p_s[g * kPos + lane] : -INFINITY;
        const float m = group_max<64>(sc);
        const float e = lane < cnt ? expf(sc - m) : 0.0f;
        const float l = group_sum<64>(e);
        if (lane < cnt) p_s[g * kPos + lane] = e;
        if (lane == 0) {
            stat_s[2 * g] = m;
            stat_s[2 * g + 1] = l;
        }
    }
    __syncthreads();
    if (vlive) {
        float acc[G][4];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[g][e] = 0.0f;
#pragma unroll
        for (int i = 0; i < kPos / 8; i++) {
            const int vp = (lane >> 3) + 8 * i;
            float v0, v1, v2, v3;
            if constexpr (F16) {
                v0 = half_of(vw[i][0], 0);
                v1 = half_of(vw[i][0], 1);
                v2 = half_of(vw[i][F16 ? 1 : 0], 0);
                v3 = half_of(vw[i][F16 ? 1 : 0], 1);
            } else {
                const uint32_t w = vw[i][0];
                const float vsc = dq::from_f16(vbits[i]);
                v0 = (float)(int8_t)(w & 0xff) * vsc;
                v1 = (float)(int8_t)((w >> 8) & 0xff) * vsc;
                v2 = (float)(int8_t)((w >> 16) & 0xff) * vsc;
                v3 = (float)(int8_t)(w >> 24) * vsc;
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float pr = vp < cnt ? p_s[g * kPos + vp] : 0.0f;
                acc[g][0] += pr * v0;
                acc[g][1] += pr * v1;
                acc[g][2] += pr * v2;
                acc[g][3] += pr * v3;
            }
        }
        // the 8 position groups (lanes 8 apart) meet: lanes l, l ^ 8 by a
        // row rotation, l ^ 16 and l ^ 32 by permlane swaps
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float v = acc[g][e];
                v += xlane::mov<0x128>(v);
                float x, y;
                xlane::swap16(v, x, y);
                v = x + y;
                xlane::swap32(v, x, y);
                acc[g][e] = x + y;
            }
        // position group pg stores head pg's four values (a partial row is
        // (D + 2) floats: 8-byte alignment only)
        const int pg = lane >> 3;
        float o[4] = {acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
#pragma unroll
        for (int g = 1; g < G; g++)
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = pg == g ? acc[g][e] : o[e];
        if (pg < G) {
            float2 *dst = (float2 *)(part + pg * part_stride + 32 * wave + 4 * (lane & 7));
            dst[0] = make_float2(o[0], o[1]);
            dst[1] = make_float2(o[2], o[3]);
        }
    }
    if (threadIdx.x < (unsigned)G) {
        part[threadIdx.x * part_stride + D] = stat_s[2 * threadIdx.x];
        part[threadIdx.x * part_stride + D + 1] = stat_s[2 * threadIdx.x + 1];
    }
}

// out[t][h] = Σ_c e^(m_c − M) o_c / Σ_c e^(m_c − M) l_c, times sigmoid(gate)
// when a gate is given (gpu/cpu.rs:244-248); with one token, its planes too.
// A head's elements split over DS = head_dim / 64 blocks (blockIdx.x = head ·
// DS + slice; one block for a head_dim not a multiple of 64) of 16 threads a
// chunk row, four elements a thread, and 16 groups of them (more for a
// smaller row): group cg takes every 16th chunk, all its loads issued at
// once (up to kU chunks, so that a 4k context needs one round trip), merging
// them as it goes (the batch's max first, then one rescale); the groups meet
// in LDS.
constexpr int kCThreads = 256;
constexpr int kU = 8;

DEV int combine_slices(int D) { return D % 64 == 0 ? D / 64 : 1; }

__global__ void __launch_bounds__(kCThreads) k_attn_combine(float *__restrict__ out, const float *__restrict__ partials,
                                                            Shape sh, const float *__restrict__ gate,
                                                            planes::View pv) {
    __shared__ float gm[kCThreads / 8], gl[kCThreads / 8];  // (head_dim >= 32: 8 threads a row at least)
    __shared__ float4 part_s[kCThreads];
    const int D = (int)sh.head_dim, DS = combine_slices(D), TPR = D / (4 * DS);
    const size_t h = blockIdx.x / DS, t = blockIdx.y;
    const int slice = (int)(blockIdx.x % DS);
    const int dg = (int)threadIdx.x % TPR, cg = (int)threadIdx.x / TPR, CG = kCThreads / TPR;
    const int e0 = slice * (D / DS) + 4 * dg;  // the thread's first element
    const size_t stride = (size_t)(D + 2);
    const float *part = partials + (t * sh.n_heads + h) * sh.chunks * stride;
    float M = -INFINITY, L = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // (threads past the last whole group take no chunks)
    for (size_t c0 = cg; cg < CG && c0 < sh.chunks; c0 += (size_t)kU * CG) {
        float m[kU], l[kU];
        float2 oa[kU], ob[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const size_t c = c0 + (size_t)u * CG;
            const size_t cc = c < sh.chunks ? c : c0;  // past the end: a chunk already counted, dropped below
            const float *row = part + cc * stride;
            m[u] = c < sh.chunks ? row[D] : -INFINITY;
            l[u] = row[D + 1];
            oa[u] = *(const float2 *)(row + e0);  // (D + 2)·4 bytes apart: 8-byte aligned only
            ob[u] = *(const float2 *)(row + e0 + 2);
        }
        float Mb = M;
#pragma unroll
        for (int u = 0; u < kU; u++) Mb = fmaxf(Mb, m[u]);
        if (Mb == -INFINITY) continue;  // nothing yet
        const float ra = expf(M - Mb);  // (M = −∞: 0)
        L *= ra;
        acc.x *= ra;
        acc.y *= ra;
        acc.z *= ra;
        acc.w *= ra;
#pragma unroll
        for (int u = 0; u < kU; u++) {
            // an empty chunk, or none: no term (its row holds only m and l)
            const bool live = m[u] != -INFINITY;
            const float rb = expf(m[u] - Mb);
            if (!live) oa[u] = ob[u] = make_float2(0.0f, 0.0f);
            L += live ? l[u] * rb : 0.0f;
            acc.x += oa[u].x * rb;
            acc.y += oa[u].y * rb;
            acc.z += ob[u].x * rb;
            acc.w += ob[u].y * rb;
        }
        M = Mb;
    }
    // the groups meet: every thread of a group holds the same M and L
    if (dg == 0) {
        gm[cg] = M;
        gl[cg] = L;
    }
    part_s[threadIdx.x] = acc;
    __syncthreads();
    if (cg != 0) return;
    float Mt = -INFINITY;
    for (int k = 0; k < CG; k++) Mt = fmaxf(Mt, gm[k]);
    float Lt = 0.0f;
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int k = 0; k < CG; k++) {
        if (gm[k] == -INFINITY) continue;
        const float r = expf(gm[k] - Mt);
        const float4 o = part_s[k * TPR + dg];
        Lt += gl[k] * r;
        sum.x += o.x * r;
        sum.y += o.y * r;
        sum.z += o.z * r;
        sum.w += o.w * r;
    }
    const size_t i = (t * sh.n_heads + h) * D + e0;
    float4 o = make_float4(sum.x / Lt, sum.y / Lt, sum.z / Lt, sum.w / Lt);
    if (gate) {
        const float4 gv = *(const float4 *)(gate + i);
        o.x *= sigmoidf_(gv.x);
        o.y *= sigmoidf_(gv.y);
        o.z *= sigmoidf_(gv.z);
        o.w *= sigmoidf_(gv.w);
    }
    *(float4 *)(out + i) = o;
    if (pv.q) planes::write4x4(pv, i / 4, o);  // a group of 16 is 4 lanes
}

// ---------------------------------------------------------------- prefill
//
// Causal GQA for a batch of tokens on the f16 matrix cores (flash attention
// with an online softmax), head_dim 256.  A block of 8 waves takes one query
// head and 128 tokens, a wave 16 of them (the keys' and values' conversion
// serves 128 queries); the queries stay in registers as f16 hi + lo parts
// (times 1/16 = 1/sqrt(256), exact).  The block walks the positions in
// blocks of 32, the next block's loads in flight meanwhile:
//   * the keys, int8 (exact in f16), give per 32-dimension group g the sums
//     Σ q·k8 (two MFMAs, hi and lo), which the group's f16 cache scale then
//     weights: S = Σ_g s_k[p][g] · Σ_{d∈g} q_d k8_d;
//   * the online softmax (gpu/cpu.rs:388-423 takes the max first, then
//     exp(s − max) / Σ): each row's running max and sum, the output rescaled
//     when the max grows;
//   * the values, dequantized exactly (v8·s as f32) into f16 hi + lo,
//     transposed in LDS so that the MFMA operands read 8 positions as one
//     16-byte chunk, and P as hi + lo: O += P_hi·V_hi + P_hi·V_lo + P_lo·V_hi.
typedef _Float16 ahalf8 __attribute__((ext_vector_type(8)));
typedef float afloat4 __attribute__((ext_vector_type(4)));

constexpr int kFD = 256, kFQ = 128, kFP = 32, kFThreads = 512;

struct PrefillArgs {
    float *out;
    const float *q, *gate;
    const int8_t *kq, *vq;
    const uint16_t *ks, *vs;
    unsigned n, pos, heads, kv_heads;
};

DEV ahalf8 hi8(const float *v) {
    ahalf8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16)v[i];
    return h;
}
DEV ahalf8 lo8(const float *v, const ahalf8 &h) {
    ahalf8 l;
#pragma unroll
    for (int i = 0; i < 8; i++) l[i] = (_Float16)(v[i] - (float)h[i]);
    return l;
}

template <bool F16>
__global__ void __launch_bounds__(kFThreads) k_attn_prefill(const PrefillArgs a) {
    __shared__ uint4 kf[kFP * kFD / 8];          // keys as f16, [pos][256], 16-byte chunks swizzled by pos
    __shared__ float ksc[kFP][kFD / 32];         // key scales
    __shared__ uint32_t v8[kFP][F16 ? kFD / 2 : kFD / 4];  // values as stored (int8 or f16), [pos][256]
    __shared__ float vsc[kFP][kFD / 32];         // value scales
    __shared__ uint4 vt[2][kFD][kFP / 8];        // values hi / lo, [dim][pos]
    __shared__ uint4 pw[kFThreads / 64][2][16][kFP / 8];  // per wave: P hi / lo, [row][pos]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, kg = lane >> 4;
    const unsigned h = blockIdx.y, kvh = h / (a.heads / a.kv_heads);
    const unsigned t0 = blockIdx.x * kFQ;
    const unsigned kv_dim = a.kv_heads * kFD;
    const unsigned last = min(t0 + kFQ, a.n) - 1;   // the block's last token
    const unsigned len = a.pos + last + 1;         // positions it attends to

    // the wave's 16 queries as A fragments: row r16, dims 32g + 8kg..+7
    ahalf8 qh[8], ql[8];
    {
        const unsigned t = t0 + 16 * w + r16;
        const bool live = t < a.n;
        const float *qr = a.q + ((size_t)(live ? t : 0) * a.heads + h) * kFD;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            float v[8];
            const float4 x0 = *(const float4 *)(qr + 32 * g + 8 * kg), x1 = *(const float4 *)(qr + 32 * g + 8 * kg + 4);
            v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = live ? v[i] * 0.0625f : 0.0f;
            qh[g] = hi8(v);
            ql[g] = lo8(v, qh[g]);
        }
    }
    // this lane's rows (C layout): 4kg + e of the wave's 16; their tokens
    unsigned tr[4];
#pragma unroll
    for (int e = 0; e < 4; e++) tr[e] = t0 + 16 * w + 4 * kg + e;
    float m[4], l[4];
    afloat4 o[16];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        m[e] = -INFINITY;
        l[e] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) o[i] = afloat4{0.0f, 0.0f, 0.0f, 0.0f};

    // staging: threads 0-255 take the keys, 256-511 the values, of position
    // pp = (tid % 256) / 8, 32-byte piece c; the next step's are loaded while
    // this step is computed
    const int sp = (tid & 255) >> 3, sc8 = tid & 7;
    const bool skeys = tid < 256;
    const int8_t *const ssrc = skeys ? a.kq : a.vq;
    const uint16_t *const sscl = skeys ? a.ks : a.vs;
    uint4 nx[F16 ? 4 : 2];
    uint16_t nxs;
    auto fetch = [&](unsigned p0) {
        const unsigned p = p0 + sp;
        const bool live = p < len;
        const size_t row = (size_t)(live ? p : 0) * kv_dim + (size_t)kvh * kFD;
        const uint4 z = make_uint4(0, 0, 0, 0);
        if constexpr (F16) {
            const uint4 *src = (const uint4 *)((const uint16_t *)ssrc + row + 32 * sc8);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 v = src[i];
                nx[i] = live ? v : z;
            }
            nxs = 0;
        } else {
            const uint4 v0 = *(const uint4 *)(ssrc + row + 32 * sc8), v1 = *(const uint4 *)(ssrc + row + 32 * sc8 + 16);
            const uint16_t sv = sscl[row / 32 + sc8];
            nx[0] = live ? v0 : z;
            nx[F16 ? 1 : 1] = live ? v1 : z;
            nxs = live ? sv : 0;
        }
    };
    fetch(0);
    for (unsigned p0 = 0; p0 < len; p0 += kFP) {
        // ---- stage the 32 positions: keys to f16, values raw, scales
        __syncthreads();
        {
            uint4 x[F16 ? 4 : 2];
#pragma unroll
            for (int i = 0; i < (F16 ? 4 : 2); i++) x[i] = nx[i];
            const uint16_t xs = nxs;
            if (p0 + kFP < len) fetch(p0 + kFP);
            if constexpr (F16) {
                // keys: as stored; values: raw words of two dims
                if (skeys) {
                    ksc[sp][sc8] = 1.0f;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int chunk = 4 * sc8 + q;
                        kf[sp * 32 + (chunk ^ (sp & 15))] = x[q];
                    }
                } else {
                    vsc[sp][sc8] = 1.0f;
#pragma unroll
                    for (int q = 0; q < 16; q++) v8[sp][16 * sc8 + q] = word_of(x[q / 4], q % 4);
                }
            } else if (skeys) {
                ksc[sp][sc8] = dq::from_f16(xs);
                const uint32_t kw[8] = {x[0].x, x[0].y, x[0].z, x[0].w, x[1].x, x[1].y, x[1].z, x[1].w};
#pragma unroll
                for (int q = 0; q < 4; q++) {  // 8 keys a 16-byte chunk of f16
                    uint32_t hw[4];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t word = kw[2 * q + e];
                        const _Float16 b0 = (_Float16)(float)(int8_t)(word & 0xffu), b1 = (_Float16)(float)(int8_t)((word >> 8) & 0xffu);
                        const _Float16 b2 = (_Float16)(float)(int8_t)((word >> 16) & 0xffu), b3 = (_Float16)(float)(int8_t)(word >> 24);
                        hw[2 * e] = (uint32_t)__builtin_bit_cast(uint16_t, b0) | (uint32_t)__builtin_bit_cast(uint16_t, b1) << 16;
                        hw[2 * e + 1] = (uint32_t)__builtin_bit_cast(uint16_t, b2) | (uint32_t)__builtin_bit_cast(uint16_t, b3) << 16;
                    }
                    const int chunk = 4 * sc8 + q;  // of 32 per row
                    kf[sp * 32 + (chunk ^ (sp & 15))] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                }
            } else {
                vsc[sp][sc8] = dq::from_f16(xs);
                const uint32_t vw[8] = {x[0].x, x[0].y, x[0].z, x[0].w, x[1].x, x[1].y, x[1].z, x[1].w};
#pragma unroll
                for (int q = 0; q < 8; q++) v8[sp][8 * sc8 + q] = vw[q];
            }
        }
        __syncthreads();
        // ---- the values transposed: thread (dims 4dq + 2hf, + 1; positions 8j..8j+7)
        {
            const int dq4 = tid & 63, j = (tid >> 6) & 3, hf = tid >> 8;
            float vv[2][8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int p = 8 * j + i;
                if constexpr (F16) {
                    const uint32_t word = v8[p][2 * dq4 + hf];  // dims 4dq4 + 2hf, + 1
#pragma unroll
                    for (int d = 0; d < 2; d++) vv[d][i] = half_of(word, d);
                } else {
                    const uint32_t word = v8[p][dq4];
                    const float sc = vsc[p][dq4 / 8];
#pragma unroll
                    for (int d = 0; d < 2; d++) vv[d][i] = (float)(int8_t)((word >> (8 * (2 * hf + d))) & 0xffu) * sc;
                }
            }
#pragma unroll
            for (int d = 0; d < 2; d++) {
                const ahalf8 hh = hi8(vv[d]), ll = lo8(vv[d], hh);
                vt[0][4 * dq4 + 2 * hf + d][j] = __builtin_bit_cast(uint4, hh);
                vt[1][4 * dq4 + 2 * hf + d][j] = __builtin_bit_cast(uint4, ll);
            }
        }
        __syncthreads();
        // ---- scores of the wave's 16 rows against the 32 positions (2 tiles)
        afloat4 sacc[2];
#pragma unroll
        for (int tcol = 0; tcol < 2; tcol++) {
            sacc[tcol] = afloat4{0.0f, 0.0f, 0.0f, 0.0f};
            const int pp = 16 * tcol + r16;  // B column: position
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const ahalf8 kb = __builtin_bit_cast(ahalf8, kf[pp * 32 + ((4 * g + kg) ^ (pp & 15))]);
                afloat4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[g], kb, afloat4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[g], kb, c, 0, 0, 0);
                const float sc = ksc[pp][g];  // C column r16 is this position
#pragma unroll
                for (int e = 0; e < 4; e++) sacc[tcol][e] += sc * c[e];
            }
        }
        // ---- mask, online softmax (rows 4kg + e; the 16 lanes of a row group hold its columns)
        float pv[2][4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float mx = -INFINITY;
#pragma unroll
            for (int tcol = 0; tcol < 2; tcol++) {
                const unsigned p = p0 + 16 * tcol + r16;
                const bool ok = p <= a.pos + tr[e] && p < len;
                pv[tcol][e] = ok ? sacc[tcol][e] : -INFINITY;
                mx = fmaxf(mx, pv[tcol][e]);
            }
            mx = group_max<16>(mx);
            const float mn = fmaxf(m[e], mx);
            const float alpha = mn == -INFINITY ? 1.0f : expf(m[e] - mn);
            float sum = 0.0f;
#pragma unroll
            for (int tcol = 0; tcol < 2; tcol++) {
                const float pe = pv[tcol][e] == -INFINITY ? 0.0f : expf(pv[tcol][e] - mn);
                pv[tcol][e] = pe;
                sum += pe;
            }
            sum = group_sum<16>(sum);
            l[e] = l[e] * alpha + sum;
            m[e] = mn;
#pragma unroll
            for (int i = 0; i < 16; i++) o[i][e] *= alpha;
        }
        // ---- P to the A layout through the wave's LDS tile (hi, lo)
        {
            _Float16 *ph = (_Float16 *)&pw[w][0][0][0], *pl = (_Float16 *)&pw[w][1][0][0];
#pragma unroll
            for (int tcol = 0; tcol < 2; tcol++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int row = 4 * kg + e, col = 16 * tcol + r16;
                    const _Float16 hv = (_Float16)pv[tcol][e];
                    ph[row * kFP + col] = hv;
                    pl[row * kFP + col] = (_Float16)(pv[tcol][e] - (float)hv);
                }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const ahalf8 pa_h = __builtin_bit_cast(ahalf8, pw[w][0][r16][kg]);
        const ahalf8 pa_l = __builtin_bit_cast(ahalf8, pw[w][1][r16][kg]);
        // ---- O += P·V over the 16 dimension tiles
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int d = 16 * i + r16;  // B column: dimension
            const ahalf8 vh = __builtin_bit_cast(ahalf8, vt[0][d][kg]);
            const ahalf8 vl = __builtin_bit_cast(ahalf8, vt[1][d][kg]);
            o[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_h, vh, o[i], 0, 0, 0);
            o[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_h, vl, o[i], 0, 0, 0);
            o[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa_l, vh, o[i], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
    }
    // ---- out = O / l, gated
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const unsigned t = tr[e];
        if (t >= a.n) continue;
        const float inv = 1.0f / l[e];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const size_t idx = ((size_t)t * a.heads + h) * kFD + 16 * i + r16;
            float r = o[i][e] * inv;
            if (a.gate) r *= sigmoidf_(a.gate[idx]);
            a.out[idx] = r;
        }
    }
}

}  // namespace

// The decode path's partial results: [token][head][chunk][head_dim + 2] floats.
size_t attention_partials_floats(size_t n, size_t pos, size_t n_heads, size_t head_dim) {
    const size_t chunks = (pos + n + kPos - 1) / kPos;
    return n * n_heads * chunks * (head_dim + 2);
}

// Grows the device's partials buffer to `floats` (a model reserves its
// largest once, when it is built, so that no forward pass allocates).
hipError_t attention_reserve(dwim_dev *dev, size_t floats) {
    return dev_grow(dev, (void **)&dev->partials, &dev->partials_cap, floats, sizeof(float));
}

namespace {

// Both entry points' launches: the batch path on the matrix cores (no
// scratch), or the chunked decode path with its partial results in
// `partials` (at least attention_partials_floats).
hipError_t attention_run(dwim_dev *dev, float *partials, float *out, const float *q, const dwim_cache *k,
                         const dwim_cache *v, size_t n, size_t pos, size_t n_heads, size_t head_dim,
                         size_t n_kv_heads, const float *gate, planes::View pv) {
    if (n >= 16 && !pv.q && head_dim == (size_t)kFD && n_heads % n_kv_heads == 0) {
        // a batch of tokens: flash attention on the matrix cores
        PrefillArgs pa{out, q, gate, k->q, v->q, k->s, v->s, (unsigned)n, (unsigned)pos, (unsigned)n_heads,
                       (unsigned)n_kv_heads};
        dim3 grid((unsigned)((n + kFQ - 1) / kFQ), (unsigned)n_heads);
        if (k->f16) k_attn_prefill<true><<<grid, kFThreads, 0, dev->stream>>>(pa);
        else k_attn_prefill<false><<<grid, kFThreads, 0, dev->stream>>>(pa);
        return hipGetLastError();
    }
    const size_t len = pos + n, ch = kPos, chunks = (len + ch - 1) / ch;
    Shape sh{n, pos, n_heads, head_dim, n_kv_heads, ch, chunks};
    dim3 g1((unsigned)chunks, (unsigned)n_kv_heads, (unsigned)n);
    switch (n_heads / n_kv_heads) {
#define DWIM_PARTIAL(G)                                                                                        \
    case G:                                                                                                    \
        if (k->f16) k_attn_partial<G, true><<<g1, kPThreads, 0, dev->stream>>>(partials, q, k->q, k->s, v->q, v->s, sh); \
        else k_attn_partial<G, false><<<g1, kPThreads, 0, dev->stream>>>(partials, q, k->q, k->s, v->q, v->s, sh);      \
        break;
        DWIM_PARTIAL(1) DWIM_PARTIAL(2) DWIM_PARTIAL(3) DWIM_PARTIAL(4) DWIM_PARTIAL(5) DWIM_PARTIAL(6)
        DWIM_PARTIAL(7) DWIM_PARTIAL(8)
#undef DWIM_PARTIAL
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned ds = head_dim % 64 == 0 ? (unsigned)(head_dim / 64) : 1u;
    dim3 g2((unsigned)n_heads * ds, (unsigned)n);
    k_attn_combine<<<g2, kCThreads, 0, dev->stream>>>(out, partials, sh, gate, pv);
    return hipGetLastError();
}

bool attention_shape_ok(size_t n_heads, size_t head_dim, size_t n_kv_heads) {
    return !(head_dim % 32 || head_dim > kMaxD || n_kv_heads == 0 || n_heads % n_kv_heads ||
             n_heads / n_kv_heads > kMaxG);
}

}  // namespace

hipError_t launch_attention(dwim_dev *dev, float *out, const float *q, const dwim_cache *k, const dwim_cache *v,
                            size_t n, size_t pos, size_t n_heads, size_t head_dim, size_t n_kv_heads) {
    return launch_attention_gated(dev, out, q, k, v, n, pos, n_heads, head_dim, n_kv_heads, nullptr, -1);
}

hipError_t launch_attention_gated(dwim_dev *dev, float *out, const float *q, const dwim_cache *k,
                                  const dwim_cache *v, size_t n, size_t pos, size_t n_heads, size_t head_dim,
                                  size_t n_kv_heads, const float *gate, int area) {
    if (!attention_shape_ok(n_heads, head_dim, n_kv_heads)) return hipErrorInvalidValue;
    planes::View pv{};
    if (area >= 0) {
        if (n != 1 || head_dim % 32 || n_heads * head_dim > planes::kMaxCols || (n_heads * head_dim) % 256)
            return hipErrorInvalidValue;
        pv = planes_area(dev, area, n_heads * head_dim);
        dev->prepared = 0;
    }
    const bool batch = n >= 16 && area < 0 && head_dim == (size_t)kFD;
    if (!batch) {
        hipError_t e = attention_reserve(dev, attention_partials_floats(n, pos, n_heads, head_dim));
        if (e != hipSuccess) return e;
    }
    return attention_run(dev, dev->partials, out, q, k, v, n, pos, n_heads, head_dim, n_kv_heads, gate, pv);
}

// ---------------------------------------------------------------- without allocating
//
// dwim_attention_noalloc keeps the decode path's partial results in this
// file-scope array instead of the device's grown buffer.  Every GPU holds its
// own copy of it (64 MiB) until the process ends; its address on a device is
// taken once, when the device is opened (attention_scratch_init), and used
// wherever host code needs the array.  Calls on one GPU share it, so calls
// that overlap on one device race.  Nothing in it needs to start at zero:
// each chunk's partial row is written before the combine reads it.
namespace {
constexpr size_t kScratchFloats = (size_t)16 << 20;
__device__ __align__(256) float scratch[kScratchFloats];
}  // namespace

hipError_t attention_scratch_init(dwim_dev *dev) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    dev->attn_scratch = (float *)ptr;
    return hipSuccess;
}

extern "C" int dwim_attention_noalloc(dwim_dev *dev, dwim_buf *out, const dwim_buf *q, const dwim_cache *k_cache,
                                      const dwim_cache *v_cache, size_t pos, size_t n_heads, size_t head_dim,
                                      size_t n_kv_heads) {
    DWIM_CHECK(head_dim % 32 == 0 && head_dim <= 256 && head_dim > 0,
               "attention: heads are whole blocks of 32, at most 256");
    DWIM_CHECK(n_kv_heads > 0 && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= 8,
               "attention: at most 8 query heads to a key/value head");
    const size_t width = n_heads * head_dim;
    DWIM_CHECK(q->len % width == 0 && out->len == q->len, "attention: q and out are whole tokens");
    const size_t n = q->len / width, kv_dim = n_kv_heads * head_dim;
    DWIM_CHECK((pos + n) * kv_dim <= k_cache->len && (pos + n) * kv_dim <= v_cache->len,
               "attention: the caches do not hold the tokens' positions");
    DWIM_CHECK(k_cache->f16 == v_cache->f16, "attention: the key and value caches are of different formats");
    DWIM_CHECK(dev->attn_scratch != nullptr, "attention_noalloc: the device's scratch array has no address");
    if (n == 0) return 0;
    const bool batch = n >= 16 && head_dim == (size_t)kFD;
    if (!batch) {
        const size_t need = attention_partials_floats(n, pos, n_heads, head_dim);
        DWIM_CHECK(need <= kScratchFloats,
                   "attention_noalloc: " + std::to_string(n) + " tokens at position " + std::to_string(pos) +
                       " need " + std::to_string(need * 4) + " bytes of partial results, more than the " +
                       std::to_string(kScratchFloats * 4) + " bytes of its scratch array");
    }
    DWIM_HIP(attention_run(dev, dev->attn_scratch, out->data, q->data, k_cache, v_cache, n, pos, n_heads, head_dim,
                           n_kv_heads, nullptr, planes::View{}));
    return 0;
}
