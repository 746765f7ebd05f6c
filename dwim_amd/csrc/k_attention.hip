// Causal grouped-query attention over the Q8 key/value caches
// (dwim gpu/cpu.rs:202-236), split over chunks of 64 positions so that a
// single decode token still spreads its cache reads over the whole GPU.
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

constexpr int kThreads = 1024;  // a combine block: 16 groups of chunks
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
    const int D = (int)sh.head_dim, G = (int)(sh.n_heads / sh.n_kv_heads);
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
    uint4 ka, kc;
    uint16_t kbits;
    {
        const size_t off = (p0 + min(kp, cnt - 1)) * kv_dim + kvh * D + 32 * min(b, nblk - 1);
        ka = ((const uint4 *)(kq + off))[0];
        kc = ((const uint4 *)(kq + off))[1];
        kbits = ks[off / 32];
    }
    // values: wave w < nblk takes Q8 block w of the head
    const bool vlive = wave < nblk;
    uint32_t vw[kPos / 8];
    uint16_t vbits[kPos / 8];
#pragma unroll
    for (int i = 0; i < kPos / 8; i++) {
        const int vp = min((lane >> 3) + 8 * i, cnt - 1);
        const size_t off = (p0 + vp) * kv_dim + kvh * D + 32 * min(wave, nblk - 1) + 4 * (lane & 7);
        vw[i] = *(const uint32_t *)(vq + off);
        vbits[i] = vs[off / 32];
    }
    // (the query loads were issued first, so this waits for them alone)
    for (int k = 0; k < kQPer; k++) {
        const unsigned i = threadIdx.x + k * kPThreads;
        if (i < (unsigned)(G * D)) q_s[(i / 32) * 36 + i % 32] = qr[k];
    }
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)D);
    {
        const float ksc = dq::from_f16(kbits);
        float kv[32];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t wa = i < 4 ? ka.x : i < 8 ? ka.y : i < 12 ? ka.z : ka.w;
            const uint32_t wc = i < 4 ? kc.x : i < 8 ? kc.y : i < 12 ? kc.z : kc.w;
            kv[i] = (float)(int8_t)((wa >> (8 * (i & 3))) & 0xff);
            kv[16 + i] = (float)(int8_t)((wc >> (8 * (i & 3))) & 0xff);
        }
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
        float acc[kMaxG][4];
#pragma unroll
        for (int g = 0; g < kMaxG; g++)
            for (int e = 0; e < 4; e++) acc[g][e] = 0.0f;
#pragma unroll
        for (int i = 0; i < kPos / 8; i++) {
            const int vp = (lane >> 3) + 8 * i;
            const uint32_t w = vw[i];
            const float vsc = dq::from_f16(vbits[i]);
            const float v0 = (float)(int8_t)(w & 0xff) * vsc, v1 = (float)(int8_t)((w >> 8) & 0xff) * vsc,
                        v2 = (float)(int8_t)((w >> 16) & 0xff) * vsc, v3 = (float)(int8_t)(w >> 24) * vsc;
#pragma unroll
            for (int g = 0; g < kMaxG; g++)
                if (g < G) {
                    const float pr = vp < cnt ? p_s[g * kPos + vp] : 0.0f;
                    acc[g][0] += pr * v0;
                    acc[g][1] += pr * v1;
                    acc[g][2] += pr * v2;
                    acc[g][3] += pr * v3;
                }
        }
#pragma unroll
        for (int g = 0; g < kMaxG; g++)
            if (g < G)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float v = acc[g][e];
                    v += __shfl_xor(v, 8, 64);
                    v += __shfl_xor(v, 16, 64);
                    v += __shfl_xor(v, 32, 64);
                    acc[g][e] = v;
                }
        if (lane < 8)  // (a partial row is (D + 2) floats: 8-byte alignment only)
            for (int g = 0; g < G; g++)
                for (int e = 0; e < 4; e++) part[g * part_stride + 32 * wave + 4 * lane + e] = acc[g][e];
    }
    if (threadIdx.x < (unsigned)G) {
        part[threadIdx.x * part_stride + D] = stat_s[2 * threadIdx.x];
        part[threadIdx.x * part_stride + D + 1] = stat_s[2 * threadIdx.x + 1];
    }
}

// out[t][h] = Σ_c e^(m_c − M) o_c / Σ_c e^(m_c − M) l_c, times sigmoid(gate)
// when a gate is given (gpu/cpu.rs:244-248); with one token, its planes too.
// Thread group cg = thread / (D/4) takes every CG-th chunk, four elements a
// thread; the groups meet in LDS.
__global__ void __launch_bounds__(kThreads) k_attn_combine(float *__restrict__ out, const float *__restrict__ partials,
                                                           Shape sh, const float *__restrict__ gate, planes::View pv) {
    __shared__ float red[16];
    __shared__ float4 part_s[kThreads];
    const size_t h = blockIdx.x, t = blockIdx.y;
    const int D = (int)sh.head_dim, TPR = D / 4, CG = kThreads / TPR;
    const int dg = threadIdx.x % TPR, cg = threadIdx.x / TPR;
    const size_t stride = (size_t)(D + 2);
    const float *part = partials + (t * sh.n_heads + h) * sh.chunks * stride;
    float M = -INFINITY;
    for (size_t c = threadIdx.x; c < sh.chunks; c += kThreads) M = fmaxf(M, part[c * stride + D]);
    M = group_max<64>(M);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = red[0];
    for (int w = 1; w < kThreads / 64; w++) M = fmaxf(M, red[w]);
    float L = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
    for (size_t c = cg; c < sh.chunks; c += CG) {
        const float m = part[c * stride + D];
        if (m == -INFINITY) continue;
        const float e = expf(m - M);
        L += e * part[c * stride + D + 1];
        const float *o = part + c * stride + 4 * dg;  // (D + 2)·4 bytes apart: 8-byte aligned only
        acc.x += e * o[0];
        acc.y += e * o[1];
        acc.z += e * o[2];
        acc.w += e * o[3];
    }
    // L: every thread of a chunk group added the same terms; take group 0's
    __syncthreads();
    if (dg == 0) red[cg] = L;
    part_s[threadIdx.x] = acc;
    __syncthreads();
    L = 0.0f;
    for (int k = 0; k < CG; k++) L += red[k];
    if (cg == 0) {
        float4 sum = acc;
        for (int k = 1; k < CG; k++) {
            const float4 o = part_s[k * TPR + dg];
            sum.x += o.x;
            sum.y += o.y;
            sum.z += o.z;
            sum.w += o.w;
        }
        part_s[dg] = sum;
    }
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += kThreads) {
        const float4 sum = part_s[d / 4];
        const float a = (d & 3) == 0 ? sum.x : (d & 3) == 1 ? sum.y : (d & 3) == 2 ? sum.z : sum.w;
        const size_t i = (t * sh.n_heads + h) * D + d;
        float o = a / L;
        if (gate) o *= sigmoidf_(gate[i]);
        out[i] = o;
        if (pv.q) planes::write16(pv, i, o);  // D is whole groups of 16 lanes
    }
}

}  // namespace

hipError_t launch_attention(dwim_dev *dev, float *out, const float *q, const dwim_cache *k, const dwim_cache *v,
                            size_t n, size_t pos, size_t n_heads, size_t head_dim, size_t n_kv_heads) {
    return launch_attention_gated(dev, out, q, k, v, n, pos, n_heads, head_dim, n_kv_heads, nullptr, -1);
}

hipError_t launch_attention_gated(dwim_dev *dev, float *out, const float *q, const dwim_cache *k,
                                  const dwim_cache *v, size_t n, size_t pos, size_t n_heads, size_t head_dim,
                                  size_t n_kv_heads, const float *gate, int area) {
    if (head_dim % 32 || head_dim > kMaxD || n_kv_heads == 0 || n_heads % n_kv_heads ||
        n_heads / n_kv_heads > kMaxG)
        return hipErrorInvalidValue;
    planes::View pv{};
    if (area >= 0) {
        if (n != 1 || head_dim % 32 || n_heads * head_dim > planes::kMaxCols || (n_heads * head_dim) % 256)
            return hipErrorInvalidValue;
        pv = planes_area(dev, area, n_heads * head_dim);
        dev->prepared = 0;
    }
    size_t len = pos + n;
    const size_t ch = kPos;
    size_t chunks = (len + ch - 1) / ch;
    size_t need = n * n_heads * chunks * (head_dim + 2);
    if (dev->partials_cap < need) {
        if (dev->partials) hipFree(dev->partials);
        dev->partials = nullptr;
        dev->partials_cap = 0;
        hipError_t e = hipMalloc(&dev->partials, need * sizeof(float));
        if (e != hipSuccess) return e;
        dev->partials_cap = need;
    }
    Shape sh{n, pos, n_heads, head_dim, n_kv_heads, ch, chunks};
    dim3 g1((unsigned)chunks, (unsigned)n_kv_heads, (unsigned)n);
    k_attn_partial<<<g1, kPThreads, 0, dev->stream>>>(dev->partials, q, k->q, k->s, v->q, v->s, sh);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    dim3 g2((unsigned)n_heads, (unsigned)n);
    k_attn_combine<<<g2, kThreads, 0, dev->stream>>>(out, dev->partials, sh, gate, pv);
    return hipGetLastError();
}
