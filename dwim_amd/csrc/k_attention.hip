// Causal grouped-query attention over the key/value caches (dwim
// gpu/cpu.rs:202-236), split over chunks of 64 positions so that a single
// decode token still spreads its cache reads over the whole GPU.  A cache is
// the reference's Q8 (int8 with an f16 scale per block of 32) or f16 (each
// kernel a template on the format, F16; an f16 key or value is read as is).
//
// Pass 1, one block per (chunk, key/value head, token; or group of up to 4
// tokens of a small batch, such as a speculative verify step): the G query
// heads sharing the key/value head score the chunk's positions (a Q8 block of
// 32 per lane, its f16 scale applied to the block's sum, the 8 lanes of a
// position summed by shuffles), take the chunk's softmax numerator and weight
// the chunk's values, for each of the block's tokens in turn over the keys
// and values read once.  Every cache load of the block is issued before any
// arithmetic.  It writes, per token and query head, the chunk's max, sum of
// exponentials and weighted values.  Pass 2, one block per (query head,
// token), merges the chunks.  Each cache byte is read once per token (once
// per 4 tokens of a small batch).
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
constexpr int kTok = 4;         // tokens a block of a several-token batch

typedef _Float16 ahalf8 __attribute__((ext_vector_type(8)));
typedef float afloat4 __attribute__((ext_vector_type(4)));

constexpr int kFD = 256, kFQ = 128, kFP = 32, kFThreads = 512;


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

template <int G, bool F16, int T>
__global__ void __launch_bounds__(kPThreads) k_attn_partial(float *__restrict__ partials, const float *__restrict__ q,
                                                            const int8_t *__restrict__ kq,
                                                            const uint16_t *__restrict__ ks,
                                                            const int8_t *__restrict__ vq,
                                                            const uint16_t *__restrict__ vs, Shape sh) {
    // queries, each Q8 block of 32 padded to 36 floats: the 8 lanes of a
    // position, reading blocks 0..7 at once, then hit 8 different banks
    __shared__ float q_s[T * G * kMaxD / 32 * 36];
    __shared__ float p_s[T * G * kPos];
    __shared__ float stat_s[T * G * 2];
    const size_t chunk = blockIdx.x, kvh = blockIdx.y, t0 = blockIdx.z * (size_t)T;
    const int nt = (int)min((size_t)T, sh.n - t0);  // the block's tokens: t0 .. t0 + nt - 1
    const int D = (int)sh.head_dim;
    const size_t kv_dim = sh.n_kv_heads * sh.head_dim;
    const size_t p0 = chunk * kPos;
    const size_t head0 = kvh * G;
    const size_t part_stride = sh.chunks * (size_t)(D + 2);  // next head
    // token t0 + tt attends up to its own position: cnt_of(tt) of the
    // chunk's positions (0 past its last)
    auto cnt_of = [&](int tt) -> int {
        const size_t len = sh.pos + t0 + tt + 1;
        return p0 >= len ? 0 : (int)min((size_t)kPos, len - p0);
    };
    auto part_of = [&](int tt) -> float * {
        return partials + (((t0 + tt) * sh.n_heads + head0) * sh.chunks + chunk) * (size_t)(D + 2);
    };
    const int cnt = cnt_of(nt - 1);  // the last token's: the most
    if (cnt == 0) {
        // a chunk past every token's last position: empty
        if (threadIdx.x < (unsigned)(nt * G)) {
            float *part = part_of((int)threadIdx.x / G) + (threadIdx.x % G) * part_stride;
            part[D] = -INFINITY;
            part[D + 1] = 0.0f;
        }
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // the queries first: in-order completion then lets the scores wait for
    // the queries and keys alone, and the values arrive meanwhile
    float qr[T][kQPer];
#pragma unroll
    for (int tt = 0; tt < T; tt++)
#pragma unroll
        for (int k = 0; k < kQPer; k++) {
            const size_t i = threadIdx.x + k * kPThreads;
            qr[tt][k] = tt < nt && i < (size_t)(G * D) ? q[((t0 + tt) * sh.n_heads + head0) * D + i] : 0.0f;
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
#pragma unroll
    for (int tt = 0; tt < T; tt++)
        for (int k = 0; k < kQPer; k++) {
            const unsigned i = threadIdx.x + k * kPThreads;
            if (i < (unsigned)(G * D)) q_s[(tt * G * nblk + i / 32) * 36 + i % 32] = qr[tt][k];
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
        // every token's G heads against the keys read once
#pragma unroll
        for (int r = 0; r < T * G; r++) {
            if (T > 1 && r >= nt * G) continue;  // (uniform)
            float sc = 0.0f;
            if (klive) {
                const float *qg = q_s + (r * nblk + b) * 36;
#pragma unroll
                for (int i = 0; i < 32; i++) sc += qg[i] * kv[i];
            }
            sc = group_sum<8>(sc * ksc);
            if (b == 0 && kp < cnt) p_s[r * kPos + kp] = scale * sc;
        }
    }
    __syncthreads();
    // softmax numerators: wave w takes rows (token, head) w, w + 8, ..., a
    // lane per position
    for (int r = wave; r < nt * G; r += kPThreads / 64) {
        const int c = cnt_of(r / G);
        const float sc = lane < c ? p_s[r * kPos + lane] : -INFINITY;
        const float m = group_max<64>(sc);
        const float e = lane < c ? expf(sc - m) : 0.0f;
        const float l = group_sum<64>(e);
        if (lane < cnt) p_s[r * kPos + lane] = e;  // (0 past the token's last position)
        if (lane == 0) {
            stat_s[2 * r] = c ? m : -INFINITY;
            stat_s[2 * r + 1] = l;
        }
    }
    __syncthreads();
    if (vlive) {
        float vv[kPos / 8][4];
#pragma unroll
        for (int i = 0; i < kPos / 8; i++) {
            if constexpr (F16) {
                vv[i][0] = half_of(vw[i][0], 0);
                vv[i][1] = half_of(vw[i][0], 1);
                vv[i][2] = half_of(vw[i][F16 ? 1 : 0], 0);
                vv[i][3] = half_of(vw[i][F16 ? 1 : 0], 1);
            } else {
                const uint32_t w = vw[i][0];
                const float vsc = dq::from_f16(vbits[i]);
                vv[i][0] = (float)(int8_t)(w & 0xff) * vsc;
                vv[i][1] = (float)(int8_t)((w >> 8) & 0xff) * vsc;
                vv[i][2] = (float)(int8_t)((w >> 16) & 0xff) * vsc;
                vv[i][3] = (float)(int8_t)(w >> 24) * vsc;
            }
        }
        for (int tt = 0; tt < nt; tt++) {
            float acc[G][4];
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[g][e] = 0.0f;
#pragma unroll
            for (int i = 0; i < kPos / 8; i++) {
                const int vp = (lane >> 3) + 8 * i;
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float pr = vp < cnt ? p_s[(tt * G + g) * kPos + vp] : 0.0f;
                    acc[g][0] += pr * vv[i][0];
                    acc[g][1] += pr * vv[i][1];
                    acc[g][2] += pr * vv[i][2];
                    acc[g][3] += pr * vv[i][3];
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
            // position group pg stores head pg's four values (a partial row
            // is (D + 2) floats: 8-byte alignment only)
            const int pg = lane >> 3;
            float o[4] = {acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
#pragma unroll
            for (int g = 1; g < G; g++)
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = pg == g ? acc[g][e] : o[e];
            if (pg < G) {
                float2 *dst = (float2 *)(part_of(tt) + pg * part_stride + 32 * wave + 4 * (lane & 7));
                dst[0] = make_float2(o[0], o[1]);
                dst[1] = make_float2(o[2], o[3]);
            }
        }
    }
    if (threadIdx.x < (unsigned)(nt * G)) {
        float *part = part_of((int)threadIdx.x / G) + (threadIdx.x % G) * part_stride;
        part[D] = stat_s[2 * threadIdx.x];
        part[D + 1] = stat_s[2 * threadIdx.x + 1];
    }
}

// ---------------------------------------------------------------- decode, matrix cores
//
// The same partial rows for head_dim 256 with the scores and the weighted
// values on the f16 matrix cores (v_mfma_f32_16x16x32_f16).  A block of 4
// waves takes a run of sh.ch positions (64 a step) of one key/value head and
// its query rows, a row a (token, head) pair: the G heads of one token, or
// of up to kTok tokens of a small batch, in RT tiles of 16 rows.
//   * Scores, wave w the step's positions 16w..16w+15: for each Q8 block of
//     32 dimensions, the queries' f16 hi and lo parts (staged in LDS once) as
//     A against the keys as B, exact in f16 (int8, or the f16 cache as is),
//     then times the block's per-position scale, in f32.
//   * Softmax over the step, a running max and sum per row (flash style).
//   * Values, wave w the dimensions 64w..64w+63: the probabilities times the
//     values' per-position scale of the dimension's Q8 block, split into f16
//     hi and lo parts, as A against the values as B (transposed into LDS,
//     8 positions of one dimension a lane).
// Every product is exact up to the hi/lo split (2^-22 relative) and summed
// in f32.
constexpr int kMStep = 64;       // positions a step
constexpr int kMThreads = 256;
constexpr int kQStride = 256 + 8;  // halfs a staged query row (bank spread)
constexpr int kPStride = kMStep + 4;
constexpr int kVRow = kFD + 16;           // Q8: bytes of a value row as the cache holds it (bank spread)
constexpr int kVRow16 = 2 * kFD + 32;     // f16: bytes of such a row

// Eight int8 values (two little-endian words) as f16, exactly: each byte
// biased to u = b + 128 and placed under the f16 exponent of 1024
// (0x64uu = 1024 + u), then 1152 subtracted, two values a packed op.
DEV ahalf8 i8x8_to_f16(uint32_t w0, uint32_t w1) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 bias = h2{(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
    const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) - bias;
    const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) - bias;
    const h2 c = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) - bias;
    const h2 d = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) - bias;
    return ahalf8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// LDS of k_attn_mfma: queries hi and lo, probabilities, value scales, the
// rows' max / sum / rescale, the transposed values
constexpr size_t mfma_lds(int rt, bool f16) {
    return (size_t)16 * rt * kQStride * 2 * 2 + (size_t)16 * rt * kPStride * 4 + (size_t)(kFD / 32) * kMStep * 4 +
           (size_t)16 * rt * 3 * 4 + (size_t)kMStep * (f16 ? kVRow16 : kVRow);
}

template <int RT, bool F16>
__global__ void __launch_bounds__(kMThreads, 2) k_attn_mfma(float *__restrict__ partials, const float *__restrict__ q,
                                                         const int8_t *__restrict__ kq,
                                                         const uint16_t *__restrict__ ks,
                                                         const int8_t *__restrict__ vq,
                                                         const uint16_t *__restrict__ vs, Shape sh, int G, int T) {
    constexpr int NR = 16 * RT;  // rows, padded
    constexpr int D = kFD;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    _Float16 *q_hi = (_Float16 *)lds_raw, *q_lo = q_hi + NR * kQStride;
    float *p_s = (float *)(q_lo + NR * kQStride);
    float(*vsc_s)[kMStep] = (float(*)[kMStep])(p_s + NR * kPStride);
    float *m_s = (float *)(vsc_s + D / 32), *l_s = m_s + NR, *a_s = l_s + NR;
    uint8_t *vt_raw = (uint8_t *)(a_s + NR);
    const size_t chunk = blockIdx.x, kvh = blockIdx.y, t0 = blockIdx.z * (size_t)T;
    const int nt = (int)min((size_t)T, sh.n - t0), R = nt * G;
    const size_t kv_dim = sh.n_kv_heads * D, head0 = kvh * G;
    const size_t c0 = chunk * sh.ch;
    const size_t len_last = sh.pos + t0 + nt;  // positions the group's last token sees
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r16 = lane & 15, kq4 = lane >> 4;
    auto part_of = [&](int r) -> float * {
        return partials + (((t0 + r / G) * sh.n_heads + head0 + r % G) * sh.chunks + chunk) * (size_t)(D + 2);
    };
    if (c0 >= len_last) {
        if (threadIdx.x < (unsigned)R) {
            float *part = part_of((int)threadIdx.x);
            part[D] = -INFINITY;
            part[D + 1] = 0.0f;
        }
        return;
    }
    // the queries, hi and lo parts (rows past R zero)
    for (int r = wave; r < NR; r += kMThreads / 64) {
        float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (r < R) x = *(const float4 *)(q + ((t0 + r / G) * sh.n_heads + head0 + r % G) * D + 4 * lane);
        const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const _Float16 h = (_Float16)xs[e];
            q_hi[r * kQStride + 4 * lane + e] = h;
            q_lo[r * kQStride + 4 * lane + e] = (_Float16)(xs[e] - (float)h);
        }
    }
    if (threadIdx.x < (unsigned)NR) {
        m_s[threadIdx.x] = -INFINITY;
        l_s[threadIdx.x] = 0.0f;
    }
    afloat4 o[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int j = 0; j < 4; j++) o[rt][j] = afloat4{0.0f, 0.0f, 0.0f, 0.0f};
    const float scale = 1.0f / 16.0f;  // 1 / sqrt(256)
    const int steps = (int)(sh.ch / kMStep);
    // ---- loads: this wave's keys (position 16w + r16, 8 dimensions of each
    // Q8 block) and their scales; a 4-dimension x 16-position patch of the
    // values and (wave 0) the value scales.  A step's loads are issued while
    // the previous step computes: the values' once they are in LDS, the
    // keys' once the scores are taken.
    // the value patch: Q8, dimensions 16·(t % 16).. of positions 4·(t / 16)..;
    // f16, dimensions 8·(t % 32).. of positions 8·(t / 32)..
    constexpr int VP = F16 ? 8 : 4;                                   // positions a thread
    const int vd = F16 ? 8 * (threadIdx.x & 31) : 16 * (threadIdx.x & 15);
    const int vp0 = F16 ? 8 * (threadIdx.x >> 5) : 4 * (threadIdx.x >> 4);
    uint4 kf[F16 ? 8 : 4];  // Q8: two blocks a uint4
    uint4 kscale = make_uint4(0, 0, 0, 0);
    uint4 vw[VP];
    uint4 vscale = make_uint4(0, 0, 0, 0);
    auto load_keys = [&](size_t ps, int cnt) __attribute__((always_inline)) {
        const size_t kpos = ps + min(16 * wave + r16, cnt - 1);
        const size_t kbase = kpos * kv_dim + kvh * D + 8 * kq4;
        if constexpr (F16) {
#pragma unroll
            for (int b = 0; b < 8; b++) kf[b] = *(const uint4 *)((const uint16_t *)kq + kbase + 32 * b);
        } else {
#pragma unroll
            for (int b = 0; b < 8; b += 2) {
                const uint2 x = *(const uint2 *)(kq + kbase + 32 * b), y = *(const uint2 *)(kq + kbase + 32 * (b + 1));
                kf[b / 2] = make_uint4(x.x, x.y, y.x, y.y);
            }
            kscale = *(const uint4 *)(ks + kpos * (kv_dim / 32) + kvh * 8);
        }
    };
    auto load_values = [&](size_t ps, int cnt) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < VP; j++) {
            const size_t off = (ps + min(vp0 + j, cnt - 1)) * kv_dim + kvh * D + vd;
            vw[j] = F16 ? *(const uint4 *)((const uint16_t *)vq + off) : *(const uint4 *)(vq + off);
        }
        if (!F16 && threadIdx.x < kMStep)
            vscale = *(const uint4 *)(vs + (ps + min((int)threadIdx.x, cnt - 1)) * (kv_dim / 32) + kvh * 8);
    };
    auto count = [&](size_t ps) { return (int)min((size_t)kMStep, len_last - ps); };
    load_keys(c0, count(c0));
    load_values(c0, count(c0));
    for (int s = 0; s < steps; s++) {
        const size_t ps = c0 + (size_t)s * kMStep;
        if (ps >= len_last) break;
        const size_t pn = ps + kMStep;  // the next step
        const bool next = s + 1 < steps && pn < len_last;
        __syncthreads();  // (the previous step is done with vt, p_s and vsc_s; the queries are staged)
        // ---- the values, in LDS as the cache holds them (read transposed below)
        if constexpr (F16) {
            typedef unsigned u4n __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int j = 0; j < VP; j++)
                *(u4n *)(vt_raw + (vp0 + j) * kVRow16 + 2 * vd) = u4n{vw[j].x, vw[j].y, vw[j].z, vw[j].w};
        } else {
            // Q8: the rows as the cache holds them (read transposed below)
            // (as a native vector: a uint4 struct copy would keep vw in memory)
            typedef unsigned u4n __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int j = 0; j < VP; j++)
                *(u4n *)(vt_raw + (vp0 + j) * kVRow + vd) = u4n{vw[j].x, vw[j].y, vw[j].z, vw[j].w};
            if (threadIdx.x < kMStep) {
                const uint32_t w4[4] = {vscale.x, vscale.y, vscale.z, vscale.w};
#pragma unroll
                for (int b = 0; b < 8; b++) vsc_s[b][threadIdx.x] = dq::from_f16((uint16_t)(w4[b / 2] >> (16 * (b % 2))));
            }
        }
        if (next) load_values(pn, count(pn));
        // ---- scores: rows 4·kq4 + e of each tile, position 16w + r16
        {
            afloat4 sc[RT];
#pragma unroll
            for (int rt = 0; rt < RT; rt++) sc[rt] = afloat4{0.0f, 0.0f, 0.0f, 0.0f};
            const uint32_t ksw[4] = {kscale.x, kscale.y, kscale.z, kscale.w};
#pragma unroll
            for (int b = 0; b < 8; b++) {
                ahalf8 kb;
                if constexpr (F16) {
                    kb = __builtin_bit_cast(ahalf8, kf[b]);
                } else {
                    const uint4 &x = kf[b / 2];
                    kb = (b % 2) ? i8x8_to_f16(x.z, x.w) : i8x8_to_f16(x.x, x.y);
                }
                const float kscl = F16 ? 1.0f : dq::from_f16((uint16_t)(ksw[b / 2] >> (16 * (b % 2))));
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const int qo = (rt * 16 + r16) * kQStride + 32 * b + 8 * kq4;
                    const ahalf8 ah = *(const ahalf8 *)(q_hi + qo), al = *(const ahalf8 *)(q_lo + qo);
                    afloat4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, kb, afloat4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, kb, c, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; e++) sc[rt][e] += c[e] * kscl;
                }
                // (a block at a time: the scheduler would otherwise hoist every
                // block's query reads, and their registers cost a block a CU)
                __builtin_amdgcn_sched_barrier(0);
            }
            const int p = 16 * wave + r16;
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int r = rt * 16 + 4 * kq4 + e;
                    // row r's token sees positions up to sh.pos + t0 + r / G
                    const bool live = r < R && ps + p <= sh.pos + t0 + r / G;
                    p_s[r * kPStride + p] = live ? sc[rt][e] * scale : -INFINITY;
                }
        }
        if (next) load_keys(pn, count(pn));
        __syncthreads();
        // ---- softmax numerators with a running max and sum: wave w takes
        // rows w, w + 4, ..., a lane per position (the padding rows past R
        // are never written out, and their products stay in their own rows)
        for (int r = wave; r < R; r += kMThreads / 64) {
            const float x = p_s[r * kPStride + lane];
            const float mo = m_s[r];
            const float mn = fmaxf(mo, group_max<64>(x));
            const float e = mn == -INFINITY ? 0.0f : expf(x - mn);
            const float l = group_sum<64>(e);
            p_s[r * kPStride + lane] = e;
            if (lane == 0) {
                const float a = mn == -INFINITY ? 1.0f : expf(mo - mn);
                a_s[r] = a;
                m_s[r] = mn;
                l_s[r] = l_s[r] * a + l;
            }
        }
        __syncthreads();
        // ---- values: dimensions 64w + 16j + r16 (j < 4: Q8 blocks 2w, 2w + 1)
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            float a[4];
#pragma unroll
            for (int e = 0; e < 4; e++) a[e] = a_s[rt * 16 + 4 * kq4 + e];
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) o[rt][j][e] *= a[e];
        }
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) {
            const int pp = 32 * k2 + 8 * kq4;  // this lane's 8 positions
            ahalf8 vb[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if constexpr (F16) {
                    // ds_read_b64_tr_b16, twice (positions pp.., pp + 4..):
                    // lane 16g + m + 4b names the row of position b at
                    // dimensions d0 + 4m..+3; lane 16g + 4m + i receives
                    // element i of its m's 4 rows, i.e. dimension d0 + r16
                    const int tb = (lane & 15) >> 2, tm = lane & 3;
                    typedef short v4s_ __attribute__((ext_vector_type(4)));
                    const uint8_t *row = vt_raw + 2 * (64 * wave + 16 * j + 4 * tm);
                    const v4s_ x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s_ *)(row + (pp + tb) * kVRow16));
                    const v4s_ x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s_ *)(row + (pp + 4 + tb) * kVRow16));
                    // (whole words: assembled element by element, the
                    // compiler took x0[2..3] for copies of x0[0..1])
                    typedef unsigned u2n_ __attribute__((ext_vector_type(2)));
                    typedef unsigned u4n_ __attribute__((ext_vector_type(4)));
                    const u2n_ a0 = __builtin_bit_cast(u2n_, x0), a1 = __builtin_bit_cast(u2n_, x1);
                    vb[j] = __builtin_bit_cast(ahalf8, u4n_{a0.x, a0.y, a1.x, a1.y});
                } else {
                    // ds_read_b64_tr_b8: lane 16g + 2b + h names the row of
                    // position pp_g + b at dimensions d0 + 8h..+7; lane 16g +
                    // 8h + i receives byte i of the 8 rows of its h, i.e.
                    // dimension d0 + r16 of positions pp_g..pp_g + 7
                    const int tb = (lane & 15) >> 1, th = lane & 1;
                    typedef int v2i_ __attribute__((ext_vector_type(2)));
                    const v2i_ x = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                        (__attribute__((address_space(3))) v2i_ *)(vt_raw + (pp + tb) * kVRow + 64 * wave + 16 * j +
                                                                     8 * th));
                    vb[j] = i8x8_to_f16((uint32_t)x[0], (uint32_t)x[1]);
                }
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const float4 pa = *(const float4 *)(p_s + (rt * 16 + r16) * kPStride + pp);
                const float4 pb = *(const float4 *)(p_s + (rt * 16 + r16) * kPStride + pp + 4);
                const float pr[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
                for (int h = 0; h < 2; h++) {  // Q8 block 2w + h: tiles j = 2h, 2h + 1
                    ahalf8 ph, pl;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const float x = F16 ? pr[i] : pr[i] * vsc_s[2 * wave + h][pp + i];
                        const _Float16 hh = (_Float16)x;
                        ph[i] = hh;
                        pl[i] = (_Float16)(x - (float)hh);
                    }
#pragma unroll
                    for (int jj = 0; jj < 2; jj++) {
                        const int j = 2 * h + jj;
                        o[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vb[j], o[rt][j], 0, 0, 0);
                        o[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb[j], o[rt][j], 0, 0, 0);
                    }
                }
            }
        }
    }
    // ---- the partial rows: row 4·kq4 + e of tile rt, dimension 64w + 16j + r16
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int r = rt * 16 + 4 * kq4 + e;
            if (r >= R) continue;
            float *part = part_of(r);
#pragma unroll
            for (int j = 0; j < 4; j++) part[64 * wave + 16 * j + r16] = o[rt][j][e];
        }
    if (threadIdx.x < (unsigned)R) {
        float *part = part_of((int)threadIdx.x);
        part[D] = m_s[threadIdx.x];
        part[D + 1] = l_s[threadIdx.x];
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
    if (pv.q) {
        // token t's planes in the t-th area from pv's (a group of 16 is 4 lanes)
        const planes::View pt = t ? planes::view(pv.q + t * planes::kAreaBytes, pv.cols) : pv;
        planes::write4x4(pt, (h * D + e0) / 4, o);
    }
}

// ---------------------------------------------------------------- prefill


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

// the matrix-core pass's blocks resident at once on a CU (its launch bounds)
constexpr size_t kMPerCU = 2;
// one token over at most this many positions: the one-chunk VALU pass, a
// single round of blocks (4k positions: 14.1 against 14.2 us with the merge;
// 32k: 47.8 against 31.2)
constexpr size_t kValuLen = 6144;

template <int RT, bool F16>
hipError_t mfma_pass(dwim_dev *dev, dim3 grid, float *partials, const float *q, const dwim_cache *k,
                     const dwim_cache *v, const Shape &sh, int G, int T) {
    constexpr size_t lds = mfma_lds(RT, F16);
    // once a process (thread-safe: a function-local static)
    static const hipError_t raised =
        hipFuncSetAttribute((const void *)k_attn_mfma<RT, F16>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (raised != hipSuccess) return raised;
    k_attn_mfma<RT, F16><<<grid, kMThreads, lds, dev->stream>>>(partials, q, k->q, k->s, v->q, v->s, sh, G, T);
    return hipGetLastError();
}

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
    const size_t len = pos + n;
    if (head_dim == (size_t)kFD && (n > 1 || len > kValuLen)) {
        // the matrix-core pass: a run of 64-position steps a block, as few as
        // keep every block resident at once (two a CU): a second round of a
        // few blocks costs a whole block's time (32k + 1 positions: 412 blocks
        // of 5 steps, not 516 of 4; in the model 43.3 against 47.5 us a
        // 4-token pass, 9.4 against 10.9 us its merge)
        const int G = (int)(n_heads / n_kv_heads), T = n > 1 ? kTok : 1;
        const size_t groups = (n + T - 1) / T, base = (len + kMStep - 1) / kMStep * n_kv_heads * groups;
        const size_t slots = kMPerCU * (size_t)dev->cus;
        const size_t ch = kMStep * std::max<size_t>(1, (base + slots - 1) / slots), chunks = (len + ch - 1) / ch;
        Shape sh{n, pos, n_heads, head_dim, n_kv_heads, ch, chunks};
        dim3 g1((unsigned)chunks, (unsigned)n_kv_heads, (unsigned)groups);
        hipError_t e = T * G <= 16 ? (k->f16 ? mfma_pass<1, true>(dev, g1, partials, q, k, v, sh, G, T)
                                             : mfma_pass<1, false>(dev, g1, partials, q, k, v, sh, G, T))
                                   : (k->f16 ? mfma_pass<2, true>(dev, g1, partials, q, k, v, sh, G, T)
                                             : mfma_pass<2, false>(dev, g1, partials, q, k, v, sh, G, T));
        if (e != hipSuccess) return e;
        dim3 g2((unsigned)n_heads * (unsigned)(head_dim / 64), (unsigned)n);
        k_attn_combine<<<g2, kCThreads, 0, dev->stream>>>(out, partials, sh, gate, pv);
        return hipGetLastError();
    }
    const size_t ch = kPos, chunks = (len + ch - 1) / ch;
    Shape sh{n, pos, n_heads, head_dim, n_kv_heads, ch, chunks};
    // one token a block, or a few tokens' queries against the chunk read once
    const bool grouped = n > 1;
    dim3 g1((unsigned)chunks, (unsigned)n_kv_heads, (unsigned)(grouped ? (n + kTok - 1) / kTok : n));
    switch (n_heads / n_kv_heads) {
#define DWIM_PARTIAL_T(G, T)                                                                                    \
    if (k->f16) k_attn_partial<G, true, T><<<g1, kPThreads, 0, dev->stream>>>(partials, q, k->q, k->s, v->q, v->s, sh); \
    else k_attn_partial<G, false, T><<<g1, kPThreads, 0, dev->stream>>>(partials, q, k->q, k->s, v->q, v->s, sh);
#define DWIM_PARTIAL(G)                                                                                        \
    case G:                                                                                                    \
        if (grouped) {                                                                                         \
            DWIM_PARTIAL_T(G, kTok)                                                                            \
        } else {                                                                                               \
            DWIM_PARTIAL_T(G, 1)                                                                               \
        }                                                                                                      \
        break;
        DWIM_PARTIAL(1) DWIM_PARTIAL(2) DWIM_PARTIAL(3) DWIM_PARTIAL(4) DWIM_PARTIAL(5) DWIM_PARTIAL(6)
        DWIM_PARTIAL(7) DWIM_PARTIAL(8)
#undef DWIM_PARTIAL
#undef DWIM_PARTIAL_T
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
        // one token's planes, or 2..4 tokens' in a set of batch areas
        const bool areas_ok = n == 1 || (n <= 4 && (area == kBatchArea || area == kBatchArea2));
        if (!areas_ok || head_dim % 32 || n_heads * head_dim > planes::kMaxCols || (n_heads * head_dim) % 256)
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
