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
//
// A batch of 16 tokens or more (head_dim 256) runs flash attention on the
// f16 matrix cores over a copy of the cache expanded to f16 hi + lo parts in
// the layout the kernel holds in LDS (k_kv_expand, k_attn_flash below).
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

typedef _Float16 ahalf8 __attribute__((ext_vector_type(8)));
typedef float afloat4 __attribute__((ext_vector_type(4)));

constexpr int kFD = 256, kFQ = 128, kFP = 32, kFThreads = 512;

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

// ---------------------------------------------------------------- prefill, expanded cache
//
// The batch path in two launches.  k_kv_expand writes, per key/value head
// and step of 32 positions, 64 KB exactly as k_attn_flash holds a step in
// LDS, so that the attention kernel copies each step straight from global
// memory into LDS (global_load_lds, no registers, no conversion):
//   * keys [position r][64 chunks]: logical chunk c < 32 holds the f16 hi
//     parts of dimensions 8c..8c+7, chunk 32 + c their lo parts; chunk c of
//     row r is stored at c ^ (r % 16), so that the 16 lanes reading one
//     chunk column of 16 rows hit 16 different bank groups;
//   * values transposed, [part][dimension d][4 chunks of 8 positions], chunk
//     j of row d stored at j ^ ((d / 4) % 4), likewise.
// A Q8 value k8·s (an int8 times an f16 scale, 19 significant bits) is hi +
// lo exactly; an f16 cache's value is its hi part, lo 0.  Positions past
// the last are zeros.
constexpr unsigned kXStep = 32;                  // positions a step
constexpr size_t kXStepBytes = 65536;            // a step of one key/value head
constexpr int kXThreads = 256;

template <bool F16>
__global__ void __launch_bounds__(kXThreads) k_kv_expand(uint4 *__restrict__ xs, const int8_t *__restrict__ kq,
                                                          const uint16_t *__restrict__ ks,
                                                          const int8_t *__restrict__ vq,
                                                          const uint16_t *__restrict__ vs, unsigned len,
                                                          unsigned steps, unsigned kv_heads) {
    __shared__ float vt[kXStep][kFD + 1];
    const unsigned s = blockIdx.x, kvh = blockIdx.y, t = threadIdx.x;
    const unsigned r = t >> 3, c8 = t & 7;  // position r of the step, 32 dimensions 32·c8..
    const unsigned p = s * kXStep + r;
    const bool live = p < len;
    const size_t off = (size_t)(live ? p : 0) * kv_heads * kFD + (size_t)kvh * kFD + 32 * c8;
    uint4 *step = xs + ((size_t)kvh * steps + s) * (kXStepBytes / 16);
    float kv[32], vv[32];
    if constexpr (F16) {
        const uint4 *k16 = (const uint4 *)((const uint16_t *)kq + off), *v16 = (const uint4 *)((const uint16_t *)vq + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 a = k16[i], b = v16[i];
            const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kv[8 * i + e] = half_of(aw[e / 2], e % 2);
                vv[8 * i + e] = half_of(bw[e / 2], e % 2);
            }
        }
    } else {
        const float ksc = dq::from_f16(ks[off / 32]), vsc = dq::from_f16(vs[off / 32]);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint4 a = ((const uint4 *)(kq + off))[i], b = ((const uint4 *)(vq + off))[i];
            const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 16; e++) {
                kv[16 * i + e] = (float)(int8_t)((aw[e / 4] >> (8 * (e % 4))) & 0xffu) * ksc;
                vv[16 * i + e] = (float)(int8_t)((bw[e / 4] >> (8 * (e % 4))) & 0xffu) * vsc;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 32; i++) {
        kv[i] = live ? kv[i] : 0.0f;
        vt[r][32 * c8 + i] = live ? vv[i] : 0.0f;
    }
    // keys: chunks 4·c8 + j (hi) and 32 + 4·c8 + j (lo) of row r
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const ahalf8 h = hi8(kv + 8 * j), l = lo8(kv + 8 * j, h);
        const unsigned c = 4 * c8 + j;
        step[r * 64 + (c ^ (r & 15))] = __builtin_bit_cast(uint4, h);
        step[r * 64 + ((32 + c) ^ (r & 15))] = __builtin_bit_cast(uint4, l);
    }
    __syncthreads();
    // values: thread t takes dimension t, 8 positions a chunk
    uint4 *vdst = step + 2048;
    const unsigned d = t, sw = (d >> 2) & 3;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; i++) x[i] = vt[8 * j + i][d];
        const ahalf8 h = hi8(x), l = lo8(x, h);
        vdst[d * 4 + (j ^ sw)] = __builtin_bit_cast(uint4, h);
        vdst[(kFD + d) * 4 + (j ^ sw)] = __builtin_bit_cast(uint4, l);
    }
}

// Causal GQA for a batch of tokens over the expanded cache, on the f16
// matrix cores.  A block of 8 waves takes one query head and 128 tokens, a
// wave 16 of them; the longest tiles are dispatched first.  Per step of 32
// positions, one barrier: every wave waits for its own copies of the step
// (issued a step earlier into the other LDS buffer), the barrier makes the
// whole step visible and frees the buffer of the step before, into which the
// next step's copies are then issued.  Scores S = q·k take three MFMA chains
// (q hi·k hi, q lo·k hi, q hi·k lo; the queries times 1/16 = 1/sqrt(256),
// exact), the online softmax is the one above, and O += P·V three more
// (P hi·V hi, P hi·V lo, P lo·V hi).
constexpr int kFlashLds = 2 * (int)kXStepBytes + 8 * 2 * 16 * 4 * 16;

struct FlashArgs {
    float *out;
    const float *q, *gate;
    const uint8_t *xs;  // the expanded cache, [kv head][step][64 KB]
    unsigned n, pos, heads, kv_heads, steps, tiles;
};

__global__ void __launch_bounds__(kFThreads) k_attn_flash(const FlashArgs a) {
    extern __shared__ uint4 smem[];
    uint4 *pwa = smem + 2 * (kXStepBytes / 16);  // per wave: P hi / lo, [row][4 chunks]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, kg = lane >> 4;
    const unsigned tile = a.tiles - 1 - blockIdx.x / a.heads, h = blockIdx.x % a.heads;
    const unsigned kvh = h / (a.heads / a.kv_heads);
    const unsigned t0 = tile * kFQ;
    const unsigned last = min(t0 + kFQ, a.n) - 1;
    const unsigned len = a.pos + last + 1;
    const unsigned steps = (len + kXStep - 1) / kXStep;
    const uint8_t *src = a.xs + (size_t)kvh * a.steps * kXStepBytes + 8192 * w + 16 * lane;
    auto copy = [&](unsigned s) {
        const uint8_t *g = src + (size_t)s * kXStepBytes;
        uint8_t *d = (uint8_t *)(smem + (s & 1) * (kXStepBytes / 16)) + 8192 * w;
#pragma unroll
        for (int k = 0; k < 8; k++) lds_copy16(g + 1024 * k, d + 1024 * k);
    };
    copy(0);

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
    const int vsw = (r16 >> 2) & 3;  // the value chunks' swizzle of this lane's dimensions

    for (unsigned s = 0; s < steps; s++) {
        __builtin_amdgcn_s_waitcnt(0x0f70);  // this wave's copies of step s
        __syncthreads();
        if (s + 1 < steps) copy(s + 1);
        const uint4 *K = smem + (s & 1) * (kXStepBytes / 16), *V = K + 2048;
        const unsigned p0 = s * kXStep;
        // ---- scores of the wave's 16 rows against the 32 positions (2 tiles)
        afloat4 sacc[2] = {afloat4{0.0f, 0.0f, 0.0f, 0.0f}, afloat4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int g = 0; g < 8; g++)
#pragma unroll
            for (int tcol = 0; tcol < 2; tcol++) {
                const int row = 16 * tcol + r16;
                const ahalf8 kh = __builtin_bit_cast(ahalf8, K[row * 64 + ((4 * g + kg) ^ r16)]);
                const ahalf8 kl = __builtin_bit_cast(ahalf8, K[row * 64 + ((32 + 4 * g + kg) ^ r16)]);
                sacc[tcol] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[g], kh, sacc[tcol], 0, 0, 0);
                sacc[tcol] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[g], kh, sacc[tcol], 0, 0, 0);
                sacc[tcol] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[g], kl, sacc[tcol], 0, 0, 0);
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
            _Float16 *ph = (_Float16 *)(pwa + w * 128), *pl = (_Float16 *)(pwa + w * 128 + 64);
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
        const ahalf8 pa_h = __builtin_bit_cast(ahalf8, pwa[w * 128 + r16 * 4 + kg]);
        const ahalf8 pa_l = __builtin_bit_cast(ahalf8, pwa[w * 128 + 64 + r16 * 4 + kg]);
        // ---- O += P·V over the 16 dimension tiles
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int d = 16 * i + r16;
            const ahalf8 vh = __builtin_bit_cast(ahalf8, V[d * 4 + (kg ^ vsw)]);
            const ahalf8 vl = __builtin_bit_cast(ahalf8, V[(kFD + d) * 4 + (kg ^ vsw)]);
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
                         size_t n_kv_heads, const float *gate, planes::View pv, uint8_t *kvx) {
    if (n >= 16 && !pv.q && head_dim == (size_t)kFD && n_heads % n_kv_heads == 0) {
        // a batch of tokens over the expanded cache (kvx: attention_kvx_bytes)
        const size_t len = pos + n, steps = (len + kXStep - 1) / kXStep;
        dim3 gx((unsigned)steps, (unsigned)n_kv_heads);
        if (k->f16)
            k_kv_expand<true><<<gx, kXThreads, 0, dev->stream>>>((uint4 *)kvx, k->q, k->s, v->q, v->s, (unsigned)len,
                                                               (unsigned)steps, (unsigned)n_kv_heads);
        else
            k_kv_expand<false><<<gx, kXThreads, 0, dev->stream>>>((uint4 *)kvx, k->q, k->s, v->q, v->s, (unsigned)len,
                                                                (unsigned)steps, (unsigned)n_kv_heads);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        // once a process; a function-local static is initialized once even
        // when host threads reach it together
        static const hipError_t raised =
            hipFuncSetAttribute((const void *)k_attn_flash, hipFuncAttributeMaxDynamicSharedMemorySize, kFlashLds);
        if (raised != hipSuccess) return raised;
        const unsigned tiles = (unsigned)((n + kFQ - 1) / kFQ);
        FlashArgs fa{out, q, gate, kvx, (unsigned)n, (unsigned)pos, (unsigned)n_heads, (unsigned)n_kv_heads,
                     (unsigned)steps, tiles};
        k_attn_flash<<<tiles * (unsigned)n_heads, kFThreads, kFlashLds, dev->stream>>>(fa);
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
        return attention_run(dev, dev->partials, out, q, k, v, n, pos, n_heads, head_dim, n_kv_heads, gate, pv,
                             nullptr);
    }
    hipError_t e = attention_kvx_reserve(dev, attention_kvx_bytes(pos + n, n_kv_heads));
    if (e != hipSuccess) return e;
    return attention_run(dev, dev->partials, out, q, k, v, n, pos, n_heads, head_dim, n_kv_heads, gate, pv,
                         (uint8_t *)dev->kvx);
}

// The expanded cache of a batch over `len` positions (head_dim 256).
size_t attention_kvx_bytes(size_t len, size_t n_kv_heads) {
    return (len + kXStep - 1) / kXStep * kXStepBytes * n_kv_heads;
}

hipError_t attention_kvx_reserve(dwim_dev *dev, size_t bytes) {
    return dev_grow(dev, &dev->kvx, &dev->kvx_cap, bytes, 1);
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
    // the decode path's partial results, or a batch's expanded cache
    const size_t need = batch ? attention_kvx_bytes(pos + n, n_kv_heads)
                              : attention_partials_floats(n, pos, n_heads, head_dim) * sizeof(float);
    DWIM_CHECK(need <= kScratchFloats * sizeof(float),
               "attention_noalloc: " + std::to_string(n) + " tokens at position " + std::to_string(pos) + " need " +
                   std::to_string(need) + " bytes of " + (batch ? "expanded cache" : "partial results") +
                   ", more than the " + std::to_string(kScratchFloats * 4) + " bytes of its scratch array");
    DWIM_HIP(attention_run(dev, dev->attn_scratch, out->data, q->data, k_cache, v_cache, n, pos, n_heads, head_dim,
                           n_kv_heads, nullptr, planes::View{}, (uint8_t *)dev->attn_scratch));
    return 0;
}
