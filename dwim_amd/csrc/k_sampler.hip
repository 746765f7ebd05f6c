// The token sampler (dwim inference/sampler.rs:7-146) on the device, so that
// a sampled token, like a greedy one, costs a few bytes read back instead of
// a row of logits: the top k of a row (the larger logit first, the lower
// index among equal ones, as the reference's ordered insertion keeps them),
// then, in one thread and in the reference's order of f32 operations, their
// softmax at the temperature, the top_p and min_p cut, and the draw with the
// sampler's xorshift64* generator, whose state stays in device memory.
//
// The top k (k <= kSelMax): each block of k_topk_part takes 4096 logits, 16
// a thread in registers as 64-bit keys that order them as the sampler does,
// and picks its k largest in k rounds, each round the largest below the last
// one picked (so nothing is marked); k_finish picks the k largest of the
// blocks' picks the same way, then runs the tail.
// A larger k sorts the whole row (a stable radix sort, descending, of the
// logits with their indices: equal logits keep index order) and the tail
// reads the first k.
//
// exp: the reference's f32::exp is the C library's expf; here the f32
// argument goes through the f64 exp and is rounded to f32 once, the
// correctly rounded value in all but the rarest cases.
#include <hipcub/hipcub.hpp>

#include <algorithm>

#include "device_util.h"
#include "runtime.h"

struct SamplerState {
    uint64_t rng;
    uint32_t token;
    int32_t accepted;
};

struct dwim_sampler {
    dwim_dev *dev;
    float temperature, top_p, min_p;
    size_t top_k;
    SamplerState *state;  // device memory
    // scratch: the blocks' picks; for a large k the row's keys, their sorted
    // copies, indices (in, sorted), the sort's temporary storage and the
    // probabilities
    void *parts = nullptr;
    size_t parts_cap = 0;
    void *sort = nullptr;
    size_t sort_cap = 0;
};

namespace {

constexpr int kSelMax = 64;
constexpr int kSelThreads = 256, kSelPer = 16, kPartSpan = kSelThreads * kSelPer;  // 4096 logits a block
constexpr uint32_t kNone = 0xffffffffu;

// An entry as one 64-bit key, larger in the sampler's order (the larger
// logit, the lower index among equal logits; -0 taken as 0): the logit's
// bits mapped to an order-preserving unsigned (negatives flipped, positives
// with the sign bit set), then the index complemented.  Key 0 is no entry.
DEV uint64_t key_of(float v, uint32_t i) {
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (uint64_t)(~i);
}
DEV uint32_t index_of(uint64_t k) { return ~(uint32_t)k; }
DEV float value_of(uint64_t k) {
    const uint32_t h = (uint32_t)(k >> 32);
    return __uint_as_float((h & 0x80000000u) ? (h & 0x7fffffffu) : ~h);
}

template <int CTRL>
DEV uint64_t mov64(uint64_t k) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)k, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(k >> 32), CTRL, 0xf, 0xf, false);
    return ((uint64_t)hi << 32) | lo;
}
DEV uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// the wave's largest key, in every lane (group_max's pattern on 64 bits)
DEV uint64_t wave_max64(uint64_t k) {
    k = max64(k, mov64<0xb1>(k));
    k = max64(k, mov64<0x4e>(k));
    k = max64(k, mov64<0x141>(k));
    k = max64(k, mov64<0x140>(k));
    {
        const auto h = __builtin_amdgcn_permlane16_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
        const auto l = __builtin_amdgcn_permlane16_swap((uint32_t)k, (uint32_t)k, false, false);
        k = max64(((uint64_t)h[0] << 32) | l[0], ((uint64_t)h[1] << 32) | l[1]);
    }
    {
        const auto h = __builtin_amdgcn_permlane32_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
        const auto l = __builtin_amdgcn_permlane32_swap((uint32_t)k, (uint32_t)k, false, false);
        k = max64(((uint64_t)h[0] << 32) | l[0], ((uint64_t)h[1] << 32) | l[1]);
    }
    return k;
}

// k rounds over the block's keys (kSelPer a thread): round r writes the r-th
// largest (0 once they run out) to out[r] (thread 0).  Each round takes the
// largest key below the last one taken, so nothing is marked; the waves'
// maxima meet in one of two LDS rows by round parity, one barrier a round.
DEV void select_rounds(const uint64_t (&key)[kSelPer], int k, uint64_t *out) {
    __shared__ uint64_t red[2][kSelThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t last = ~0ull;
    for (int r = 0; r < k; r++) {
        uint64_t best = 0;
#pragma unroll
        for (int e = 0; e < kSelPer; e++)
            if (key[e] < last) best = max64(best, key[e]);
        best = wave_max64(best);
        if (lane == 0) red[r & 1][wave] = best;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kSelThreads / 64; w++) best = max64(best, red[r & 1][w]);
        if (threadIdx.x == 0) out[r] = best;
        last = best ? best : 0;  // (none left: every later round finds none)
    }
}

// each block's k largest keys of its 4096 logits, to parts [block][k]
__global__ void __launch_bounds__(kSelThreads) k_topk_part(const float *__restrict__ logits, unsigned vocab, int k,
                                                           uint64_t *parts) {
    uint64_t key[kSelPer];
    const unsigned base = blockIdx.x * (unsigned)kPartSpan;
#pragma unroll
    for (int e = 0; e < kSelPer; e++) {
        const unsigned i = base + (unsigned)e * kSelThreads + threadIdx.x;
        key[e] = i < vocab ? key_of(logits[i], i) : 0ull;
    }
    select_rounds(key, k, parts + (size_t)blockIdx.x * k);
}

DEV float rng_next(uint64_t &s) {
    // sampler.rs:136-146
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    const uint64_t bits = s * 0x2545F4914F6CDD1DULL;
    return (float)(bits >> 40) / (float)(1ULL << 24);
}

struct TailArgs {
    float temperature, top_p, min_p;
    int k;
    int verify;  // 0: Sampler::sample, 1: Sampler::verify of `draft`
    uint32_t draft;
    SamplerState *state;
};

// Sampler::candidates from the top list (cv, ci: k entries in order) and
// then sample or verify (sampler.rs:40-133), by one thread
DEV void tail(const TailArgs &t, const float *cv, const uint32_t *ci, float *probs) {
    uint64_t rng = t.state->rng;
    int n;
    float total;
    if (t.temperature == 0.0f) {
        probs[0] = 1.0f;
        total = 1.0f;
        n = 1;
    } else {
        const float max = cv[0];
        float sum = 0.0f;
        for (int i = 0; i < t.k; i++) {
            const float p = (float)exp((double)((cv[i] - max) / t.temperature));
            probs[i] = p;
            sum += p;
        }
        for (int i = 0; i < t.k; i++) probs[i] /= sum;
        const float floor_ = t.min_p * probs[0];
        float kept = 0.0f;
        n = 0;
        while (n < t.k && kept < t.top_p && probs[n] >= floor_) {
            kept += probs[n];
            n++;
        }
        total = kept;
        if (n < 1) n = 1;  // (the settings the sampler opens with keep one at least)
    }
    uint32_t pick;
    int accepted = 0;
    if (!t.verify) {
        const float r = rng_next(rng) * total;
        float acc = 0.0f;
        pick = ci[n - 1];
        for (int i = 0; i < n; i++) {
            acc += probs[i];
            if (r < acc) {
                pick = ci[i];
                break;
            }
        }
    } else {
        float p = 0.0f;
        for (int i = 0; i < n; i++)
            if (ci[i] == t.draft) {
                p = probs[i];
                break;
            }
        pick = t.draft;
        if (p >= total || rng_next(rng) * total < p) {
            accepted = 1;
        } else {
            const float r = rng_next(rng) * (total - p);
            float acc = 0.0f;
            uint32_t last = t.draft;
            bool found = false;
            for (int i = 0; i < n && !found; i++) {
                if (ci[i] == t.draft) continue;
                acc += probs[i];
                if (r < acc) {
                    pick = ci[i];
                    found = true;
                }
                last = ci[i];
            }
            if (!found) pick = last;
        }
    }
    t.state->rng = rng;
    t.state->token = pick;
    t.state->accepted = accepted;
}

// the k largest of the blocks' picks (ncand <= kPartSpan of them), then the tail
__global__ void __launch_bounds__(kSelThreads) k_finish(const uint64_t *__restrict__ parts, unsigned ncand,
                                                        TailArgs t) {
    __shared__ uint64_t top[kSelMax];
    __shared__ float top_v[kSelMax], probs[kSelMax];
    __shared__ uint32_t top_i[kSelMax];
    uint64_t key[kSelPer];
#pragma unroll
    for (int e = 0; e < kSelPer; e++) {
        const unsigned c = (unsigned)e * kSelThreads + threadIdx.x;
        key[e] = c < ncand ? parts[c] : 0ull;
    }
    select_rounds(key, t.k, top);
    __syncthreads();
    if (threadIdx.x < (unsigned)t.k) {
        top_v[threadIdx.x] = value_of(top[threadIdx.x]);
        top_i[threadIdx.x] = index_of(top[threadIdx.x]);
    }
    __syncthreads();
    if (threadIdx.x == 0) tail(t, top_v, top_i, probs);
}

// a large k: the tail over the sorted row, its first k entries staged in
// LDS by the block when they fit (else read where they lie)
constexpr int kSortedLds = 4096;
__global__ void __launch_bounds__(kSelThreads) k_finish_sorted(const float *__restrict__ sv,
                                                               const uint32_t *__restrict__ si, float *probs,
                                                               TailArgs t) {
    __shared__ float lv[kSortedLds], lp[kSortedLds];
    __shared__ uint32_t li[kSortedLds];
    if (t.k <= kSortedLds) {
        for (int i = threadIdx.x; i < t.k; i += kSelThreads) {
            lv[i] = sv[i];
            li[i] = si[i];
        }
        __syncthreads();
        if (threadIdx.x == 0) tail(t, lv, li, lp);
    } else if (threadIdx.x == 0) {
        tail(t, sv, si, probs);
    }
}

// the row's keys for the sort (-0 as 0, which the sampler takes as equal)
// and their indices
__global__ void k_sort_keys(const float *__restrict__ logits, unsigned vocab, float *keys, uint32_t *idx) {
    const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= vocab) return;
    const float x = logits[i];
    keys[i] = x == 0.0f ? 0.0f : x;
    idx[i] = i;
}

hipError_t grow(void **p, size_t *cap, size_t bytes) {
    if (*cap >= bytes) return hipSuccess;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) *cap = bytes;
    return e;
}

int run(dwim_sampler *s, const dwim_buf *logits, size_t row, size_t vocab, int verify, uint32_t draft,
        uint32_t *token, int *accepted) {
    dwim_dev *dev = s->dev;
    DWIM_CHECK(vocab > 0 && vocab < kNone && (row + 1) * vocab <= logits->len, "sample: the row is not in the logits");
    DWIM_HIP(hipSetDevice(dev->index));
    // (at temperature zero only the first of the top k counts, so one is taken)
    const size_t k = s->temperature == 0.0f ? 1 : std::min(std::max<size_t>(s->top_k, 1), vocab);
    TailArgs t{s->temperature, s->top_p, s->min_p, (int)k, verify, draft, s->state};
    const float *x = logits->data + row * vocab;
    const size_t nparts = (vocab + kPartSpan - 1) / kPartSpan;
    if (k <= (size_t)kSelMax && nparts * k <= (size_t)kPartSpan) {
        DWIM_HIP(grow(&s->parts, &s->parts_cap, nparts * k * 8));
        uint64_t *parts = (uint64_t *)s->parts;
        k_topk_part<<<(unsigned)nparts, kSelThreads, 0, dev->stream>>>(x, (unsigned)vocab, (int)k, parts);
        DWIM_HIP(hipGetLastError());
        k_finish<<<1, kSelThreads, 0, dev->stream>>>(parts, (unsigned)(nparts * k), t);
        DWIM_HIP(hipGetLastError());
    } else {
        // keys and indices, sorted copies, probabilities, then the sort's storage
        size_t temp = 0;
        DWIM_HIP(hipcub::DeviceRadixSort::SortPairsDescending(nullptr, temp, (const float *)nullptr, (float *)nullptr,
                                                               (const uint32_t *)nullptr, (uint32_t *)nullptr,
                                                               (int)vocab, 0, 32, dev->stream));
        const size_t arrays = 5 * vocab * 4, bytes = arrays + temp;
        DWIM_HIP(grow(&s->sort, &s->sort_cap, bytes));
        float *keys = (float *)s->sort, *skeys = keys + vocab, *probs = skeys + vocab;
        uint32_t *idx = (uint32_t *)(probs + vocab), *sidx = idx + vocab;
        void *tmp = (uint8_t *)s->sort + arrays;
        k_sort_keys<<<(unsigned)((vocab + 255) / 256), 256, 0, dev->stream>>>(x, (unsigned)vocab, keys, idx);
        DWIM_HIP(hipGetLastError());
        DWIM_HIP(hipcub::DeviceRadixSort::SortPairsDescending(tmp, temp, keys, skeys, idx, sidx, (int)vocab, 0, 32,
                                                               dev->stream));
        k_finish_sorted<<<1, kSelThreads, 0, dev->stream>>>(skeys, sidx, probs, t);
        DWIM_HIP(hipGetLastError());
    }
    SamplerState out;
    DWIM_HIP(hipMemcpyAsync(&out, s->state, sizeof(out), hipMemcpyDeviceToHost, dev->stream));
    DWIM_HIP(hipStreamSynchronize(dev->stream));
    *token = out.token;
    if (accepted) *accepted = out.accepted;
    return 0;
}

}  // namespace

extern "C" int dwim_sampler_open(dwim_dev *dev, float temperature, size_t top_k, float top_p, float min_p,
                                 uint64_t seed, dwim_sampler **out) {
    *out = nullptr;
    // (with top_p > 0 and min_p <= 1 the most likely token is always kept;
    // otherwise the reference's sampler would keep none, and fail)
    DWIM_CHECK(temperature >= 0.0f && top_p > 0.0f && min_p <= 1.0f,
               "sampler: a negative temperature, or a top_p or min_p that keeps no token");
    DWIM_HIP(hipSetDevice(dev->index));
    SamplerState *st = nullptr;
    DWIM_HIP(hipMalloc((void **)&st, sizeof(SamplerState)));
    const SamplerState init{seed > 1 ? seed : 1, 0, 0};  // Rng(seed.max(1)) (sampler.rs:36)
    if (hipMemcpy(st, &init, sizeof(init), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(st);
        return dwim_fail("sampler: writing its state failed");
    }
    dev->refs++;
    *out = new dwim_sampler{dev, temperature, top_p, min_p, top_k, st};
    return 0;
}

extern "C" void dwim_sampler_free(dwim_sampler *s) {
    if (!s) return;
    dwim_dev *dev = s->dev;
    (void)hipSetDevice(dev->index);
    (void)hipStreamSynchronize(dev->stream);
    (void)hipFree(s->state);
    if (s->parts) (void)hipFree(s->parts);
    if (s->sort) (void)hipFree(s->sort);
    delete s;
    dwim_dev_release(dev);
}

extern "C" int dwim_sampler_rng(dwim_sampler *s, uint64_t *rng) {
    SamplerState st;
    DWIM_HIP(hipSetDevice(s->dev->index));
    DWIM_HIP(hipMemcpyAsync(&st, s->state, sizeof(st), hipMemcpyDeviceToHost, s->dev->stream));
    DWIM_HIP(hipStreamSynchronize(s->dev->stream));
    *rng = st.rng;
    return 0;
}

extern "C" int dwim_sample(dwim_sampler *s, const dwim_buf *logits, size_t row, size_t vocab, uint32_t *token) {
    return run(s, logits, row, vocab, 0, 0, token, nullptr);
}

extern "C" int dwim_sample_verify(dwim_sampler *s, const dwim_buf *logits, size_t row, size_t vocab, uint32_t draft,
                                  uint32_t *token, int *accepted) {
    return run(s, logits, row, vocab, 1, draft, token, accepted);
}
