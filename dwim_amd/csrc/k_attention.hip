// Causal grouped-query attention over the Q8 key/value caches
// (dwim gpu/cpu.rs:202-236), split over chunks of positions so that a
// single decode token still spreads its cache reads over the whole GPU.
//
// Pass 1, one block per (chunk of CH positions, key/value head, token): the
// G query heads sharing the key/value head score every position of the chunk
// (a Q8 block of 32 per lane, its f16 scale applied to the block's sum, the 8
// lanes of a head summed by shuffles), take the chunk's softmax numerator and
// weight the chunk's values.  It writes, per query head, the chunk's max,
// sum of exponentials and weighted values.  Pass 2, one block per (query
// head, token), merges the chunks.  Each cache byte is read once per token.
#include "device_util.h"
#include "planes.h"
#include "quant_math.h"
#include "runtime.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxG = 8;
constexpr int kMaxD = 256;
constexpr int kMaxCH = 256;

struct Shape {
    size_t n, pos, n_heads, head_dim, n_kv_heads, ch, chunks;
};

// partials: [token][head][chunk][head_dim + 2]  (o[...], max, sum)
__global__ void __launch_bounds__(kThreads) k_attn_partial(float *__restrict__ partials, const float *__restrict__ q,
                                                           const int8_t *__restrict__ kq, const uint16_t *__restrict__ ks,
                                                           const int8_t *__restrict__ vq, const uint16_t *__restrict__ vs,
                                                           Shape sh) {
    __shared__ float q_s[kMaxG * kMaxD];
    __shared__ float p_s[kMaxG * kMaxCH];
    __shared__ float stat_s[kMaxG * 2];
    const size_t chunk = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const int D = (int)sh.head_dim, G = (int)(sh.n_heads / sh.n_kv_heads);
    const size_t kv_dim = sh.n_kv_heads * sh.head_dim;
    const size_t len = sh.pos + t + 1;  // the token attends up to its own position
    const size_t p0 = chunk * sh.ch;
    const size_t head0 = kvh * G;
    float *part = partials + ((t * sh.n_heads + head0) * sh.chunks + chunk) * (size_t)(D + 2);
    const size_t part_stride = sh.chunks * (size_t)(D + 2);  // next head
    if (p0 >= len) {
        // a chunk past this token's last position: empty
        for (int g = 0; g < G; g++)
            if (threadIdx.x == 0) {
                part[g * part_stride + D] = -INFINITY;
                part[g * part_stride + D + 1] = 0.0f;
            }
        return;
    }
    const int cnt = (int)min((size_t)sh.ch, len - p0);
    const float scale = 1.0f / sqrtf((float)D);
    for (int i = threadIdx.x; i < G * D; i += kThreads)
        q_s[i] = q[(t * sh.n_heads + head0) * D + i];
    __syncthreads();

    // scores: 8 lanes per position, lane b takes block b of the head
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane & 7, nblk = D / 32;
    // (the 8 lanes of a position leave the loop together, so their shuffles
    // stay within the group)
    for (int pl = wave * 8 + (lane >> 3); pl < cnt; pl += 32) {
        const bool live = b < nblk;
        const size_t p = p0 + pl;
        float kv[32];
        float ksc = 0.0f;
        if (live) {
            const int8_t *kr = kq + p * kv_dim + kvh * D + 32 * b;
            const uint4 a = ((const uint4 *)kr)[0], c = ((const uint4 *)kr)[1];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                uint32_t wa = i < 4 ? a.x : i < 8 ? a.y : i < 12 ? a.z : a.w;
                uint32_t wc = i < 4 ? c.x : i < 8 ? c.y : i < 12 ? c.z : c.w;
                kv[i] = (float)(int8_t)((wa >> (8 * (i & 3))) & 0xff);
                kv[16 + i] = (float)(int8_t)((wc >> (8 * (i & 3))) & 0xff);
            }
            ksc = dq::from_f16(ks[(p * kv_dim + kvh * D) / 32 + b]);
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) kv[i] = 0.0f;
        }
        for (int g = 0; g < G; g++) {
            float s = 0.0f;
            const float *qg = q_s + g * D + 32 * b;
            if (live) {
#pragma unroll
                for (int i = 0; i < 32; i++) s += qg[i] * kv[i];
            }
            s = group_sum<8>(s * ksc);
            if (b == 0) p_s[g * kMaxCH + pl] = scale * s;
        }
    }
    __syncthreads();

    // softmax numerators per head: wave w takes heads w, w+4
    for (int g = wave; g < G; g += 4) {
        float m = -INFINITY;
        for (int i = lane; i < cnt; i += 64) m = fmaxf(m, p_s[g * kMaxCH + i]);
        m = group_max<64>(m);
        float l = 0.0f;
        for (int i = lane; i < cnt; i += 64) {
            float e = expf(p_s[g * kMaxCH + i] - m);
            p_s[g * kMaxCH + i] = e;
            l += e;
        }
        l = group_sum<64>(l);
        if (lane == 0) {
            stat_s[2 * g] = m;
            stat_s[2 * g + 1] = l;
        }
    }
    __syncthreads();

    // weighted values: thread d accumulates element d for every head
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float acc[kMaxG];
#pragma unroll
        for (int g = 0; g < kMaxG; g++) acc[g] = 0.0f;
        for (int i = 0; i < cnt; i++) {
            size_t p = p0 + i;
            float v = (float)vq[p * kv_dim + kvh * D + d] * dq::from_f16(vs[(p * kv_dim + kvh * D + d) / 32]);
#pragma unroll
            for (int g = 0; g < kMaxG; g++)
                if (g < G) acc[g] += p_s[g * kMaxCH + i] * v;
        }
        for (int g = 0; g < G; g++) part[g * part_stride + d] = acc[g];
    }
    if (threadIdx.x < G) {
        part[threadIdx.x * part_stride + D] = stat_s[2 * threadIdx.x];
        part[threadIdx.x * part_stride + D + 1] = stat_s[2 * threadIdx.x + 1];
    }
}

// out[t][h] = Σ_c e^(m_c − M) o_c / Σ_c e^(m_c − M) l_c, times sigmoid(gate)
// when a gate is given (gpu/cpu.rs:244-248); with one token, its planes too.
__global__ void __launch_bounds__(kThreads) k_attn_combine(float *__restrict__ out, const float *__restrict__ partials,
                                                           Shape sh, const float *__restrict__ gate, planes::View pv) {
    const size_t h = blockIdx.x, t = blockIdx.y;
    const int D = (int)sh.head_dim;
    const float *part = partials + (t * sh.n_heads + h) * sh.chunks * (size_t)(D + 2);
    float M = -INFINITY;
    for (size_t c = 0; c < sh.chunks; c++) M = fmaxf(M, part[c * (D + 2) + D]);
    float L = 0.0f;
    for (size_t c = 0; c < sh.chunks; c++) {
        float m = part[c * (D + 2) + D];
        if (m != -INFINITY) L += expf(m - M) * part[c * (D + 2) + D + 1];
    }
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float acc = 0.0f;
        for (size_t c = 0; c < sh.chunks; c++) {
            float m = part[c * (D + 2) + D];
            if (m != -INFINITY) acc += expf(m - M) * part[c * (D + 2) + d];
        }
        const size_t i = (t * sh.n_heads + h) * D + d;
        float o = acc / L;
        if (gate) o *= sigmoidf_(gate[i]);
        out[i] = o;
        if (pv.q) planes::write32(pv, i, o);  // D is whole groups of 32 lanes
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
    planes::View pv{};
    if (area >= 0) {
        if (n != 1 || head_dim % 32 || n_heads * head_dim > planes::kMaxCols || (n_heads * head_dim) % 256)
            return hipErrorInvalidValue;
        pv = planes_area(dev, area, n_heads * head_dim);
        dev->prepared = 0;
    }
    size_t len = pos + n;
    // Chunks small enough that a lone token spreads over the GPU, at least 32
    // positions (a wave-step of the scoring loop), at most 256.
    size_t want_blocks = 2 * (size_t)dev->cus;
    size_t per = n * n_kv_heads;
    size_t ch = 32;
    while (ch < kMaxCH && (len + ch - 1) / ch * per > want_blocks * 2) ch *= 2;
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
    k_attn_partial<<<g1, kThreads, 0, dev->stream>>>(dev->partials, q, k->q, k->s, v->q, v->s, sh);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    dim3 g2((unsigned)n_heads, (unsigned)n);
    k_attn_combine<<<g2, kThreads, 0, dev->stream>>>(out, dev->partials, sh, gate, pv);
    return hipGetLastError();
}
