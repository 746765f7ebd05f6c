// A chain of one-token Q4_K products in one persistent launch.
//
// The decode step runs its matrix products back to back, each consuming the
// previous one's output (dwim inference/qwen35/mod.rs:541-655: o or out, the
// SwiGLU pair, down, then the next layer's input products).  As separate
// launches every product pays a ramp (the chip fills), a tail (the last
// round of workgroups) and the launch itself, about 5 µs against 3-18 µs of
// weight streaming.  Here one workgroup per CU walks the chain's work items,
// streaming weights into LDS ahead of the arithmetic, and waits at a product
// boundary only for the data it reads:
//   * an item is one 16-row tile of a product over a range of its 256-blocks
//     (a "part": at most kUnits tile-block units of 2304 bytes, the matrices
//     of a SwiGLU pair counted apart);
//   * workgroup g of G takes items g, g + G, g + 2G, ... in chain order (all
//     of a product's before any of the next one's); after each item it
//     publishes its progress (the launch's sequence number and the item) in
//     a word of its own, so nothing contends for one address;
//   * the next item's weights are copied from HBM straight into LDS
//     (global_load_lds, 16 bytes a lane) by waves 0..14 while the current
//     item is computed from the other of two LDS slots; wave 15, which has
//     no copies in flight, finishes each item (its stores do not wait for
//     them);
//   * before an item of a product that reads another's output, the threads
//     poll the progress words of the workgroups holding that product's
//     items, one word a thread, until each has passed its last item of it;
//   * the input of the item's part (the int8 planes of the activations,
//     planes.h) is staged into LDS, read device-coherently, and kept while
//     the workgroup's items read the same part of the same input;
//   * outputs another product of the chain reads (the residual x, the planes
//     and their statistics) are written and read device-coherently (they
//     cross XCDs; a device-scope fence would write back the whole L2).
// The arithmetic per item is k_mv_q4k_mfma's: v_mfma_i32_16x16x64_i8 on the
// tiled Q4_K layout with the activations' three digit planes, each group of
// 16 scaled in f32, the min term from the sub-block sums.  A tile split into
// parts meets in the last part to finish, which sums them in part order.
//
// Every wait is bounded: a workgroup that spins past `spin_limit` polls sets
// the error word and goes on (its results are then wrong, and the host
// reports the error), so that a kernel always drains, even if a workgroup
// were not resident.
#include "device_util.h"
#include "layout.h"
#include "mv_common.h"
#include "planes.h"
#include "runtime.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

using namespace mvq;

constexpr int kWaves = 16;
constexpr int kThreads = kWaves * 64;
constexpr int kCopyWaves = kWaves - 1;       // waves that copy weights; the last one finishes items
constexpr int kEpiWave = kWaves - 1;
constexpr int kUnits = 20;                   // tile-block units an item, at most
constexpr unsigned kUnitBytes = (unsigned)q4kt::kUnit;  // 2304
constexpr unsigned kSlotBytes = kUnits * kUnitBytes;
constexpr unsigned kChunk = 1024;            // bytes a wave copies per instruction
constexpr int kMaxCopies = (int)((kSlotBytes / kChunk + 2 + kCopyWaves - 1) / kCopyWaves);  // per wave and item
constexpr unsigned kPartCols = 20 * 256;     // columns of a part, at most
constexpr unsigned kMaxCols = (unsigned)planes::kMaxCols;
// LDS: two weight slots, the staged part (planes [3][kPartCols] bytes, statistics
// [kPartCols/64][8] floats), the whole input's Σx² [kMaxCols/16], zeros, per-wave scales
constexpr unsigned kStagePlanes = 2 * kSlotBytes;
constexpr unsigned kStageStat = kStagePlanes + 3 * kPartCols;
constexpr unsigned kStageSs = kStageStat + 4 * 8 * (kPartCols / 64);
constexpr unsigned kZeroOff = kStageSs + 4 * (kMaxCols / 16);
constexpr unsigned kHdrOff = kZeroOff + 64;
constexpr unsigned kLdsBytes = kHdrOff + kWaves * 256 * 4;
// staging loads a lane makes, at most
constexpr int kPlaneLoads = (int)((3 * kPartCols / 4 + kThreads - 1) / kThreads);
constexpr int kStatLoads = (int)((kPartCols / 64 * 8 + kThreads - 1) / kThreads);
constexpr int kSsLoads = (int)((kMaxCols / 16 + kThreads - 1) / kThreads);

struct Product {
    const uint8_t *w0, *w1;  // w1: the SwiGLU pair's up matrix, or null
    float *out;              // [rows]
    unsigned rows, nb;       // rows of each matrix; 256-blocks a row
    unsigned tiles, parts, first_item, gtile0;
    int dep;                 // the product whose output this one reads (-1: an earlier launch's)
    int add, rms, coherent_out;
    planes::View in;
    planes::View emit;       // q null: no planes out
    const float *emit_norm;
    float *emit_xw;
};

struct ChainArgs {
#ifdef DWIM_CHAIN_PROFILE
    unsigned long long *prof;      // [workgroup][8] time spent per phase, in 100 MHz ticks
#endif
    Product p[kMaxChain];
    unsigned np, items;
    float eps;
    unsigned spin_limit;
    unsigned *error;               // set when a wait gave up
    unsigned long long *progress;  // [workgroup]: seq << 32 | (last finished item + 1)
    unsigned long long seq;        // this launch's sequence number (nonzero, increasing)
    float *partials;               // [gtile][kMaxChainParts][2][16]
    unsigned *counters;            // [gtile], zero between launches
};

DEV unsigned load_agent(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV float load_agent(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void store_agent(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV void store_agent(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DEV unsigned long long load_agent(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DEV void store_agent(unsigned long long *p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The planes of a group of 16 activations that lanes 0..15 hold one each,
// with device-coherent stores: four lanes' digits packed into a word.
DEV void write16_coherent(const planes::View &v, unsigned i, float x, int lane) {
    const float m = group_max<16>(fabsf(x)), s = group_sum<16>(x);
    const float inv = m > 0.0f ? planes::kScale / m : 0.0f;
    int d[3];
    planes::digits(x, inv, d[0], d[1], d[2]);
#pragma unroll
    for (int p = 0; p < 3; p++) {
        const uint32_t b = (uint32_t)(d[p] & 255);
        const uint32_t w = b | (uint32_t)__shfl_down((int)b, 1, 64) << 8 | (uint32_t)__shfl_down((int)b, 2, 64) << 16 |
                           (uint32_t)__shfl_down((int)b, 3, 64) << 24;
        if ((lane & 3) == 0 && lane < 16)
            store_agent((unsigned *)(v.q + (size_t)p * v.cols + i + lane), (unsigned)w);
    }
    if (lane == 0) {
        const size_t g = i / 16;
        store_agent(v.stat + (g / 4) * 8 + g % 4, m / planes::kScale);
        store_agent(v.stat + (g / 4) * 8 + 4 + g % 4, s);
    }
}

// An item's place: its product, tile and part (column blocks [cb0, cb1)).
struct Where {
    int p;
    unsigned tile, part, cb0, cb1;
};

DEV Where locate(const Product *prods, unsigned np, unsigned item) {
    Where w;
    w.p = 0;
    while (w.p + 1 < (int)np && item >= prods[w.p + 1].first_item) w.p++;
    const Product &P = prods[w.p];
    const unsigned local = item - P.first_item;
    w.tile = local / P.parts;
    w.part = local - w.tile * P.parts;
    w.cb0 = w.part * P.nb / P.parts;
    w.cb1 = (w.part + 1) * P.nb / P.parts;
    return w;
}


// Copies an item's weight units into an LDS slot: 1 KB pieces, piece k by
// wave k % kCopyWaves.  Returns how many copies this wave issued.
DEV int copy_item(const Product *prods, const Where &w, uint8_t *slot, int wave, int lane) {
    if (wave >= kCopyWaves) return 0;
    const Product &P = prods[w.p];
    const unsigned ncb = w.cb1 - w.cb0, len = ncb * kUnitBytes;
    const unsigned per = (len + kChunk - 1) / kChunk;  // pieces a matrix
    const unsigned pieces = per * (P.w1 ? 2u : 1u);
    int n = 0;
#pragma unroll
    for (int i = 0; i < kMaxCopies; i++) {
        const unsigned k = (unsigned)wave + (unsigned)i * kCopyWaves;
        if (k >= pieces) break;
        const unsigned j = k >= per ? 1u : 0u, kk = k - j * per;
        const uint8_t *src = (j ? P.w1 : P.w0) + ((size_t)w.tile * P.nb + w.cb0) * kUnitBytes + kk * kChunk;
        uint8_t *dst = slot + j * len + kk * kChunk;
        const unsigned off = kk * kChunk + 16u * (unsigned)lane;
        if (off < len) lds_copy16(src + 16u * (unsigned)lane, dst);
        n++;
    }
    return n;
}

// Waits until at most n vector memory operations of this wave are outstanding.
DEV void wait_vm(int n) {
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(0x0f70); break;
        case 1: __builtin_amdgcn_s_waitcnt(0x0f71); break;
        case 2: __builtin_amdgcn_s_waitcnt(0x0f72); break;
        case 3: __builtin_amdgcn_s_waitcnt(0x0f73); break;
        case 4: __builtin_amdgcn_s_waitcnt(0x0f74); break;
        default: __builtin_amdgcn_s_waitcnt(0x0f75); break;
    }
}

__global__ void __launch_bounds__(kThreads) k_mv_chain(const ChainArgs a) {
    extern __shared__ uint4 lds_all[];
    uint8_t *lds = (uint8_t *)lds_all;
    __shared__ float red[2][kWaves][2][16];
    // the product table in LDS: its reads are counted apart from the vector
    // memory operations (the weight copies in flight), so they never wait for them
    __shared__ Product prods[kMaxChain];
    __shared__ float rms_s[2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kq = lane >> 4, c = lane & 15;
    float *hdr = (float *)(lds + kHdrOff) + wave * 256;
    const uint4 *zero = (const uint4 *)(lds + kZeroOff);
    if (threadIdx.x < 4) ((uint4 *)(lds + kZeroOff))[threadIdx.x] = make_uint4(0, 0, 0, 0);
    if (threadIdx.x < a.np) prods[threadIdx.x] = a.p[threadIdx.x];
    __syncthreads();
    const unsigned G = gridDim.x;
    // the staged part: its product's dependency and input, its columns, Σx² present
    int st_dep = -2;
    const int8_t *st_in = nullptr;
    unsigned st_cb0 = 0, st_cb1 = 0;
    bool st_ss = false;
    unsigned waited = 0;  // bit d: product d is known to be done

#ifdef DWIM_CHAIN_PROFILE
    unsigned long long tp[8] = {0, 0, 0, 0, 0, 0, 0, 0}, tl = __builtin_amdgcn_s_memrealtime();
#define PROF(i) do { const unsigned long long tn = __builtin_amdgcn_s_memrealtime(); tp[i] += tn - tl; tl = tn; } while (0)
#else
#define PROF(i) do { } while (0)
#endif
    unsigned item = blockIdx.x;
    int k = 0;  // the workgroup's item count: item k sits in slot k % 2
    Where cur{};
    if (item < a.items) {
        cur = locate(prods, a.np, item);
        copy_item(prods, cur, lds, wave, lane);
    }
    while (item < a.items) {
        const Product &P = prods[cur.p];
        uint8_t *slot = lds + (k & 1) * kSlotBytes;
        // ---- the next item's weights into the other slot (its last reader,
        // two items back, finished before the barrier that ended its compute)
        const unsigned nitem = item + G;
        Where nxt{};
        int copies = 0;
        if (nitem < a.items) {
            nxt = locate(prods, a.np, nitem);
            copies = copy_item(prods, nxt, lds + ((k + 1) & 1) * kSlotBytes, wave, lane);
        }
        PROF(0);
        // ---- the input: wait for its product, stage the part
        if (P.dep >= 0 && !(waited >> P.dep & 1u)) {
            waited |= 1u << P.dep;
            const Product &D = prods[P.dep];
            const unsigned end = D.first_item + D.tiles * D.parts;
            for (unsigned t = threadIdx.x; t < G && t < end; t += kThreads) {
                // the last item of the product that workgroup t holds
                const unsigned last = t + (end - 1 - t) / G * G;
                if (last < D.first_item) continue;
                const unsigned long long want = a.seq << 32 | (unsigned long long)(last + 1);
                unsigned spins = 0;
                while (load_agent(&a.progress[t]) < want) {
                    if (++spins > a.spin_limit) {
                        store_agent(a.error, 1u);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        }
        PROF(1);
        const unsigned ncb = cur.cb1 - cur.cb0, cols = P.nb * 256u;
        const bool restage = st_dep != P.dep || st_in != P.in.q || st_cb0 != cur.cb0 || st_cb1 != cur.cb1 ||
                             (P.rms && !st_ss);
        __syncthreads();  // the waits are over; the previous staging is no longer read
        PROF(2);
        if (restage) {
            // the part's planes and statistics and the whole Σx², device-
            // coherently, every load of a lane issued before its first store
            const unsigned qw = ncb * 64, words = 3 * qw;  // words of one plane's part, of all three
            const unsigned nst = ncb * 32, nss = P.rms ? cols / 16 : 0u;
            unsigned pv[kPlaneLoads];
            float sv[kStatLoads], qv[kSsLoads];
#pragma unroll
            for (int i = 0; i < kPlaneLoads; i++) {
                const unsigned t = threadIdx.x + i * kThreads, tc = t < words ? t : 0u;
                const unsigned pl = tc / qw, off = tc - pl * qw;
                pv[i] = load_agent((const unsigned *)(P.in.q + (size_t)pl * cols + cur.cb0 * 256u) + off);
            }
#pragma unroll
            for (int i = 0; i < kStatLoads; i++) {
                const unsigned t = threadIdx.x + i * kThreads;
                sv[i] = load_agent(P.in.stat + cur.cb0 * 32u + (t < nst ? t : 0u));
            }
#pragma unroll
            for (int i = 0; i < kSsLoads; i++) {
                const unsigned t = threadIdx.x + i * kThreads;
                qv[i] = nss ? load_agent(P.in.ss + (t < nss ? t : 0u)) : 0.0f;
            }
            unsigned *sp = (unsigned *)(lds + kStagePlanes);
            float *sst = (float *)(lds + kStageStat), *sss = (float *)(lds + kStageSs);
#pragma unroll
            for (int i = 0; i < kPlaneLoads; i++) {
                const unsigned t = threadIdx.x + i * kThreads;
                if (t < words) {
                    const unsigned pl = t / qw, off = t - pl * qw;
                    sp[pl * (kPartCols / 4) + off] = pv[i];
                }
            }
#pragma unroll
            for (int i = 0; i < kStatLoads; i++) {
                const unsigned t = threadIdx.x + i * kThreads;
                if (t < nst) sst[t] = sv[i];
            }
#pragma unroll
            for (int i = 0; i < kSsLoads; i++) {
                const unsigned t = threadIdx.x + i * kThreads;
                if (t < nss) sss[t] = qv[i];
            }
            st_dep = P.dep;
            st_in = P.in.q;
            st_cb0 = cur.cb0;
            st_cb1 = cur.cb1;
            st_ss = P.rms != 0;
        }
        PROF(3);
        // ---- this item's weights have landed (all but the next item's copies)
        wait_vm(copies);
        __syncthreads();
        PROF(4);

        // ---- the products of the wave's units (k_mv_q4k_mfma's arithmetic)
        const unsigned J = P.w1 ? 2u : 1u, U = J * ncb;
        const unsigned u0 = (unsigned)wave * U / kWaves, u1 = (unsigned)(wave + 1) * U / kWaves;
        const uint8_t *xq = lds + kStagePlanes;
        const float *xstat = (const float *)(lds + kStageStat);
        const bool active = c < 12 && c / 3 == kq;
        const int gcol = 4 * (c < 12 ? c / 3 : 0);
        const int k4 = lane & 3, R4 = lane >> 2;
        float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
        float macc[2] = {0.0f, 0.0f};
        for (unsigned u = u0; u < u1; u++) {
            const unsigned jj = u >= ncb ? 1u : 0u, bl = u - jj * ncb;  // block of the part
            const uint8_t *unit = slot + u * kUnitBytes;
            const uint4 wq0 = *(const uint4 *)(unit + q4kt::qs_off(kq, c));
            const uint4 wq1 = *(const uint4 *)(unit + q4kt::qs_off(kq, c) + 16);
            const uint32_t hwv = *(const uint32_t *)(unit + 4 * lane);
            float ma;
            {
                const uint32_t w0 = quad_bcast<0>(hwv), w1 = quad_bcast<1>(hwv), w2 = quad_bcast<2>(hwv),
                               w3 = quad_bcast<3>(hwv);
                const float d = f16_bits(w0 & 0xffffu), dmin = f16_bits(w0 >> 16);
                float sc0, sc1, mn0, mn1;
                scales_pair(w1, w2, w3, k4, sc0, sc1, mn0, mn1);
                const float4 xs = *(const float4 *)(xstat + (bl * 4 + k4) * 8);
                const float4 xm = *(const float4 *)(xstat + (bl * 4 + k4) * 8 + 4);
                const float D0 = d * sc0, D1 = d * sc1;
                ma = (dmin * mn0) * (xm.x + xm.y) + (dmin * mn1 - 8.0f * D1) * (xm.z + xm.w);
                const float D1h = D1 * 0.0625f;
                hdr[(4 * k4) * 16 + R4] = D0 * xs.x;
                hdr[(4 * k4 + 1) * 16 + R4] = D0 * xs.y;
                hdr[(4 * k4 + 2) * 16 + R4] = D1h * xs.z;
                hdr[(4 * k4 + 3) * 16 + R4] = D1h * xs.w;
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            float ac[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t mask = h ? 0xf0f0f0f0u : 0x0f0f0f0fu;
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    const uint4 q = m ? wq1 : wq0;
                    const uint4 xv = active ? *(const uint4 *)(xq + (unsigned)(c % 3) * kPartCols + bl * 256u +
                                                                64u * kq + 32u * h + 16u * m)
                                            : zero[m];
                    const v4i av = {(int)(q.x & mask), (int)(q.y & mask), (int)(q.z & mask), (int)(q.w & mask)};
                    const v4i bv = {(int)xv.x, (int)xv.y, (int)xv.z, (int)xv.w};
                    const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, v4i{0, 0, 0, 0}, 0, 0, 0);
                    const float4 D = *(const float4 *)&hdr[(gcol + 2 * h + m) * 16 + 4 * kq];
                    ac[0] += D.x * (float)C[0];
                    ac[1] += D.y * (float)C[1];
                    ac[2] += D.z * (float)C[2];
                    ac[3] += D.w * (float)C[3];
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) acc[jj][e] += ac[e];
            macc[jj] += ma;
            __builtin_amdgcn_wave_barrier();
        }
        const float f = c < 12 ? (c % 3 == 0 ? 1.0f : c % 3 == 1 ? 256.0f : 65536.0f) : 0.0f;
        float(*rd)[2][16] = red[k & 1];
#pragma unroll
        for (unsigned jj = 0; jj < 2; jj++) {
#pragma unroll
            for (int e = 0; e < 4; e++) acc[jj][e] = group_sum<16>(acc[jj][e] * f);
            const float mm = group_sum<4>(macc[jj]);
            const float mrow = __shfl(mm, 16 * kq + 4 * (c & 3), 64);
            if (c < 4)
                rd[wave][jj][4 * kq + c] =
                    (c == 0 ? acc[jj][0] : c == 1 ? acc[jj][1] : c == 2 ? acc[jj][2] : acc[jj][3]) - mrow;
        }
        if (wave == kEpiWave && P.rms) {
            // the RMS norm of the producer's x from its per-group Σx², in group order
            const float *sss = (const float *)(lds + kStageSs);
            float t = 0.0f;
            for (unsigned g = (unsigned)lane; g < cols / 16; g += 64) t += sss[g];
            t = group_sum<64>(t);
            if (lane == 0) rms_s[k & 1] = 1.0f / sqrtf(t / (float)cols + a.eps);
        }
        __syncthreads();  // the slot, the staging and red of this item are read; the next may start
        PROF(5);

        if (wave == kEpiWave) {
            // ---- wave 15 finishes the item; lanes 0..15 hold its rows
            const int rl = lane & 15;
            const unsigned tile = cur.tile;
            float v = 0.0f, u = 0.0f;
            for (int w = 0; w < kWaves; w++) {
                v += rd[w][0][rl];
                u += rd[w][1][rl];
            }
            bool finish = true;
#ifdef DWIM_CHAIN_ABLATE
            if (false) {
#else
            if (P.parts > 1) {
#endif
                // the parts meet in the last to finish, summed in part order
                const unsigned gt = P.gtile0 + tile;
                float *pp = a.partials + ((size_t)gt * kMaxChainParts + cur.part) * 32;
                if (lane < 16) {
                    store_agent(pp + lane, v);
                    store_agent(pp + 16 + lane, u);
                }
                __builtin_amdgcn_s_waitcnt(kWaitVm0);
                unsigned old = 0;
                if (lane == 0) old = atomicAdd(&a.counters[gt], 1u);
                old = __shfl(old, 0, 64);
                finish = old == P.parts - 1;
                if (finish) {
                    v = 0.0f;
                    u = 0.0f;
                    const float *tp = a.partials + (size_t)gt * kMaxChainParts * 32;
                    for (unsigned q = 0; q < P.parts; q++) {
                        v += load_agent(tp + q * 32 + rl);
                        u += load_agent(tp + q * 32 + 16 + rl);
                    }
                    if (lane == 0) store_agent(&a.counters[gt], 0u);
                }
            }
            if (finish) {
                if (P.rms) {
                    const float sc = rms_s[k & 1];
                    v *= sc;
                    u *= sc;
                }
                if (J == 2) v = v * sigmoidf_(v) * u;  // silu(gate) · up (gpu/cpu.rs:238-242)
                const unsigned orow = tile * 16 + (unsigned)rl;
                const bool valid = orow < P.rows;
                if (valid && lane < 16) {
                    if (P.add) v += P.coherent_out ? load_agent(P.out + orow) : P.out[orow];
                    if (P.coherent_out) store_agent(P.out + orow, v);
                    else P.out[orow] = v;
                }
                if (P.emit.q) {
                    float e = valid ? v : 0.0f;
                    if (P.emit_norm) {
                        const float sq = group_sum<16>(e * e);
                        if (lane == 0) store_agent(P.emit.ss + tile, sq);
                        e = valid ? e * P.emit_norm[orow] : 0.0f;
                        if (P.emit_xw && valid && lane < 16) P.emit_xw[orow] = e;
                    }
                    write16_coherent(P.emit, tile * 16u, e, lane);
                }
            }
            // the item is done once its stores are: the progress word moves
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            if (lane == 0) store_agent(&a.progress[blockIdx.x], a.seq << 32 | (unsigned long long)(item + 1));
            PROF(6);
        }
        item = nitem;
        cur = nxt;
        k++;
    }
#ifdef DWIM_CHAIN_PROFILE
    tp[7] = (unsigned long long)k;
    if (threadIdx.x == 0 || threadIdx.x == kEpiWave * 64)
        for (int i = 0; i < 8; i++)
            if (threadIdx.x == 0 ? i != 6 : i == 6) a.prof[blockIdx.x * 8 + i] = tp[i];
#endif
}

}  // namespace

size_t chain_lds_bytes() { return kLdsBytes; }
#ifdef DWIM_CHAIN_PROFILE
unsigned long long *chain_prof = nullptr;
#endif

hipError_t launch_mv_chain(dwim_dev *dev, const ChainStep *steps, int n) {
    if (n < 1 || n > kMaxChain || !dev->chain_ctl || (size_t)dev->cus > kChainMaxGroups) return hipErrorInvalidValue;
    ChainArgs a{};
    a.np = (unsigned)n;
    a.eps = steps[0].eps;
    a.spin_limit = 1u << 22;
    a.error = dev->chain_ctl;
    a.progress = dev->chain_progress;
    a.seq = ++dev->chain_seq;
    a.partials = dev->chain_partials;
    a.counters = dev->chain_counters;
#ifdef DWIM_CHAIN_PROFILE
    a.prof = chain_prof;
#endif
    unsigned items = 0, gtiles = 0;
    for (int i = 0; i < n; i++) {
        const ChainStep &s = steps[i];
        Product &P = a.p[i];
        const dwim_weight *w0 = s.w[0], *w1 = s.w[1];
        const size_t cols = w0->cols;
        if (w0->fmt != DWIM_Q4_K || cols % 256 || cols > kMaxCols || w0->rows >= (1u << 31)) return hipErrorInvalidValue;
        if (w1 && (w1->fmt != DWIM_Q4_K || w1->rows != w0->rows || w1->cols != cols)) return hipErrorInvalidValue;
        if (s.dep >= i || s.dep < -1 || s.in_area < 0) return hipErrorInvalidValue;
        P.w0 = (const uint8_t *)w0->q;
        P.w1 = w1 ? (const uint8_t *)w1->q : nullptr;
        P.out = s.out;
        P.rows = (unsigned)w0->rows;
        P.nb = (unsigned)(cols / 256);
        P.tiles = (unsigned)q4kt::tiles(w0->rows);
        // parts: the fewest (a power of two, so that a workgroup keeps its
        // part along a product) whose units and columns fit the LDS slots
        const unsigned J = w1 ? 2u : 1u;
        P.parts = 1;
        while (J * ((P.nb + P.parts - 1) / P.parts) > (unsigned)kUnits ||
               (P.nb + P.parts - 1) / P.parts * 256 > kPartCols)
            P.parts *= 2;
        if (P.parts > (unsigned)kMaxChainParts) return hipErrorInvalidValue;
        P.first_item = items;
        P.gtile0 = gtiles;
        if (P.parts > 1) gtiles += P.tiles;
        items += P.tiles * P.parts;
        P.dep = s.dep;
        P.add = s.add;
        P.rms = s.rms;
        P.coherent_out = s.coherent_out;
        P.in = planes_area(dev, s.in_area, cols);
        if (s.emit_area >= 0) {
            if (s.emit_area == s.in_area || w0->rows % 256 || w0->rows > planes::kMaxCols) return hipErrorInvalidValue;
            P.emit = planes_area(dev, s.emit_area, w0->rows);
            P.emit_norm = s.emit_norm;
            P.emit_xw = s.emit_xw;
        }
    }
    if (gtiles > dev->chain_tiles_cap) return hipErrorInvalidValue;
    a.items = items;
    dev->prepared = 0;
    static bool raised = false;  // the attribute holds for the process
    if (!raised) {
        hipError_t e = hipFuncSetAttribute((const void *)k_mv_chain, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)chain_lds_bytes());
        if (e != hipSuccess) return e;
        raised = true;
    }
    k_mv_chain<<<(unsigned)dev->cus, kThreads, chain_lds_bytes(), dev->stream>>>(a);
    return hipGetLastError();
}

int chain_error(dwim_dev *dev) {
    unsigned e = 0;
    if (hipMemcpyAsync(&e, dev->chain_ctl, sizeof e, hipMemcpyDeviceToHost, dev->stream) != hipSuccess ||
        hipStreamSynchronize(dev->stream) != hipSuccess)
        return 1;
    return e != 0;
}
