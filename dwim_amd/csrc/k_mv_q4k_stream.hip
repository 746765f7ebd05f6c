// Q4_K products of two to four tokens at once (a speculative-decoding verify
// batch, small batches) on the int8 matrix cores, reading every weight once
// for all of them (dwim gpu/cpu.rs:110-149 computes each token's product in
// f32; the arithmetic here is the one-token kernel's, exact in int32 and
// scaled in f32).
//
// The MFMA layout is k_mv_q4k_mfma.hip's: v_mfma_i32_16x16x64_i8 with the 16
// rows of a weight tile as A and B's columns (digit, sub-block) of one token's
// planes, nonzero only in their sub-block's k-group; the planes are scaled per
// 32 activations (k_planes' pair mode), so a sub-block's two MFMAs chain in
// int32 and take one scale.
//
// The work is split so that every CU streams the same number of weight
// bytes in one round ("stream-K"):
//   * an item is up to K (k_of) consecutive 256-blocks of one tile (of gate's or of
//     up's rows for a SwiGLU pair); the items of a tile are its blocks in
//     order, gate's then up's;
//   * the row's blocks split into P parts only when the planes of NT tokens
//     of a whole row would not fit in LDS; items are numbered part by part,
//     tile by tile;
//   * one workgroup of 16 waves a CU takes a contiguous run of a part's items
//     (the runs as even as integer division makes them), stages the planes of
//     its part once, and its waves take every 16th item of the run, the next
//     item's weights in flight while the current one is computed;
//   * each item's partial sums (per token, its 16 rows) go to LDS; after one
//     barrier a wave per tile sums them in item order.  A tile that lies in
//     one workgroup's run (and P = 1) is finished there; otherwise the
//     workgroups that share it write their sums with device-coherent stores,
//     count in on the tile's counter, and the last to arrive sums them in
//     (part, workgroup) order, so the result has the same bits whichever
//     finishes last, and clears the counter.
#include "device_util.h"
#include "layout.h"
#include "mv_common.h"
#include "planes.h"
#include "runtime.h"

#include <algorithm>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
// global-memory pointers, so that the loads through them are global loads
// (counted in order by vmcnt) rather than flat ones
#define GMEM __attribute__((address_space(1)))

namespace {

using namespace mvq;

constexpr int kW = 16;           // waves a workgroup
// blocks an item: 3, or 2 for four tokens (whose accumulators take the
// registers of a third block in both of the wave's two item buffers)
constexpr int k_of(int nt) { return nt >= 4 ? 2 : 3; }
constexpr int kJobs = 4;
constexpr int kTok = 4;
constexpr int kParts = 4;
// per wave: d·sc of the 8 sub-blocks × 16 rows (floats), rows of kHdrStride
// floats so that the float4 reads of 16 (sub-block, row-quad) pairs and the
// writes of 4 sub-blocks of 16 rows spread over the banks
constexpr int kHdrStride = 24;
constexpr int kHdrChunks = 8 * kHdrStride / 4;
// the planes of a (block, token): 3 digits of 16 chunks, each padded by one,
// so that the 12 lanes reading B operands (chunks 17p + 4k + const) fall in
// distinct banks; staged chunk s of the unpadded layout lands at s + s / 16
constexpr int kPStride = 17;
constexpr int kBT = 3 * kPStride;
// LDS for one part's planes and statistics: at most this many bytes
constexpr size_t kPlaneBudget = 96 * 1024;

struct StreamArgs {
    const uint8_t *w[kJobs];     // SwiGLU: w[0] gate, w[1] up
    float *out[kJobs];           // [NT][rows_j]
    unsigned rows[kJobs];
    unsigned tile0[kJobs + 1];   // first tile of each matrix in the launch's numbering; [njobs] = all tiles
    unsigned add_mask;
    int swiglu;
    unsigned nb;                 // 256-blocks per row
    unsigned P;                  // parts
    unsigned pb0[kParts + 1];    // part p: blocks [pb0[p], pb0[p + 1])
    unsigned ih[kParts];         // items per tile and matrix in part p: ceil(blocks / K)
    unsigned g0[kParts + 1];     // first workgroup of part p; [P] = the grid
    unsigned cmax;               // partial-sum slots per (tile, part)
    unsigned plane_cap;          // LDS layout: blocks of planes reserved (the largest part)
    unsigned items_cap;          // LDS layout: item slots reserved
    const int8_t *xq[kTok];      // each token's planes [3][cols]
    const float *xstat[kTok];    // [cols/64][8]
    float *partials;             // [tile][part][cmax][NT][32]
    unsigned *counters;          // [tile], zero between launches
    // given: the planes are x·w with Σx² per group (rss[t], [cols/16]), and
    // token t's results scale by 1/sqrt(Σ rss[t] / cols + eps)
    const float *rss[kTok];
    float eps;
    // given: the planes hold heads of 128 columns unnormalized, the groups of
    // token t's head k scaled by 1/sqrt(Σ hss[t][k][0..7] / 128 + heps)
    // (hss: [NT][heads][8] partial sums of squares)
    const float *hss;
    float heps;
    unsigned heads;
    // given: bf_out[t][r] = bf_w[r] · bf_x[t] (a small bf16 matrix [bf_rows]
    // [bf_cols] against f32 rows, times token t's RMS scale when the planes
    // are RMS-scaled): (row, token) pairs g + grid·k, g + grid·(k + 4), ... by
    // wave kW − 4 + k of workgroup g, after its tiles
    const uint16_t *bf_w;
    const float *bf_x;
    float *bf_out;
    unsigned bf_rows, bf_cols;
    // given (one matrix or a SwiGLU pair, rows whole 256-blocks): token t's
    // planes of the results, after the add or the SwiGLU, into the plane area
    // at emit + t·kAreaBytes; of results·emit_norm with Σ results² per group
    // when emit_norm is given (and results·emit_norm in f32 to emit_xw,
    // [NT][rows], when that is given)
    int8_t *emit;
    const float *emit_norm;
    float *emit_xw;
};

// Kernel-argument arrays are copied once, with constant indices, each
// element through readfirstlane into scalar registers, and selected from
// there by value: a select among loads of the argument block would otherwise
// become one vector load at a selected address, or a copy to scratch memory,
// and a wait on it.
DEV uint32_t sload(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
DEV T sload(T v) {
    if constexpr (sizeof(T) == 8) {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        return __builtin_bit_cast(T, (uint64_t)sload((uint32_t)u) | (uint64_t)sload((uint32_t)(u >> 32)) << 32);
    } else {
        return __builtin_bit_cast(T, sload(__builtin_bit_cast(uint32_t, v)));
    }
}
// an opaque copy in scalar registers (the empty asm keeps the selects below
// from being folded back into an indexed load)
template <typename T>
DEV T sreg(T v) {
    T r = sload(v);
    asm volatile("" : "+s"(r));
    return r;
}
template <typename T>
DEV T sel(unsigned i, T v0, T v1, T v2, T v3, T v4 = T()) {
    return i == 1 ? v1 : i == 2 ? v2 : i == 3 ? v3 : i == 4 ? v4 : v0;
}

struct Item {
    const GMEM uint8_t *units;  // the item's first unit
    unsigned tile;         // in the launch's numbering
    unsigned bl;           // its first block, counted from the part's first
    int nblk;
    int half;              // SwiGLU: 0 gate, 1 up
};

template <int K>
struct Regs {
    v4u q[K][2];
    uint32_t h[K];
};

template <int NT>
__global__ void __launch_bounds__(1024) k_mv_stream(const StreamArgs a) {
    constexpr int kK = k_of(NT);
    extern __shared__ uint4 lds[];
    // (the wave index through readfirstlane: the compiler then knows it,
    // and all that follows from it, to be the same across the wave)
    const int lane = threadIdx.x & 63, wave = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kq = lane >> 4, c = lane & 15;
    const unsigned P = a.P, nb = a.nb, J = a.swiglu ? 2u : 1u;
    const unsigned g01 = sreg(a.g0[1]), g02 = sreg(a.g0[2]), g03 = sreg(a.g0[3]), g04 = sreg(a.g0[4]);
    const unsigned pb01 = sreg(a.pb0[1]), pb02 = sreg(a.pb0[2]), pb03 = sreg(a.pb0[3]), pb04 = sreg(a.pb0[4]);
    const unsigned ih0 = sreg(a.ih[0]), ih1 = sreg(a.ih[1]), ih2 = sreg(a.ih[2]), ih3 = sreg(a.ih[3]);
    const unsigned t01 = sreg(a.tile0[1]), t02 = sreg(a.tile0[2]), t03 = sreg(a.tile0[3]);
    const GMEM uint8_t *w0 = (const GMEM uint8_t *)sreg(a.w[0]), *w1 = (const GMEM uint8_t *)sreg(a.w[1]),
                       *w2 = (const GMEM uint8_t *)sreg(a.w[2]), *w3 = (const GMEM uint8_t *)sreg(a.w[3]);
    const unsigned g = blockIdx.x;
    const unsigned p = (unsigned)(1u < P && g >= g01) + (unsigned)(2u < P && g >= g02) + (unsigned)(3u < P && g >= g03);
    const unsigned gfirst = sel(p, 0u, g01, g02, g03), G = sel(p + 1, 0u, g01, g02, g03, g04) - gfirst, gp = g - gfirst;
    const unsigned pb = sel(p, 0u, pb01, pb02, pb03), PB = sel(p + 1, 0u, pb01, pb02, pb03, pb04) - pb;
    const unsigned ih = sel(p, ih0, ih1, ih2, ih3), ip = J * ih;
    const unsigned TT = a.tile0[kJobs];
    const unsigned long long Ip = (unsigned long long)TT * ip;
    const unsigned i0 = (unsigned)((unsigned long long)gp * Ip / G);
    const unsigned i1 = (unsigned)((unsigned long long)(gp + 1) * Ip / G);
    const unsigned cols = nb * 256;

    // LDS: planes [block][token][51 chunks], statistics [block][token][8],
    // the zero region, per wave the decoded scales, the tokens' RMS scales
    // (one chunk), the tokens' head norms ([NT][heads] floats), the items' sums
    const unsigned kStat = a.plane_cap * NT * kBT;
    const unsigned kZero = kStat + a.plane_cap * NT * 8;
    const unsigned kHdr = kZero + kK * NT * kBT;
    const unsigned kTsc = kHdr + kW * kHdrChunks;
    const unsigned kTf = kTsc + 1;
    const unsigned kSlots = kTf + (NT * a.heads + 3) / 4;
    v4i *lv = (v4i *)lds;
    const float4 *stl = (const float4 *)(lds + kStat);
    float *hdr = (float *)(lds + kHdr + wave * kHdrChunks);
    float *slots = (float *)(lds + kSlots);  // [item - i0][NT][16]
    float *tsc = (float *)(lds + kTsc);
    float *tf = (float *)(lds + kTf);

    auto item_of = [=](unsigned i) {
        Item it;
        const unsigned T = i / ip, rem = i - T * ip, half = rem / ih, r = rem - half * ih;
        const unsigned j = (unsigned)(T >= t01) + (unsigned)(T >= t02) + (unsigned)(T >= t03);
        const unsigned tl = T - sel(j, 0u, t01, t02, t03);
        const GMEM uint8_t *wbase = sel(a.swiglu ? half : j, w0, w1, w2, w3);
        it.tile = T;
        it.bl = r * kK;
        it.nblk = (int)min((unsigned)kK, PB - r * kK);
        it.half = (int)half;
        it.units = wbase + ((size_t)tl * nb + pb + it.bl) * q4kt::kUnit;
        return it;
    };
    auto load = [=](Regs<kK> &R, const Item &it) {
#pragma unroll
        for (int u = 0; u < kK; u++) {
            const unsigned off = (unsigned)(u < it.nblk ? u : 0) * (unsigned)q4kt::kUnit;
            R.q[u][0] = *(const GMEM v4u *)(it.units + off + q4kt::qs_off(kq, c));
            R.q[u][1] = *(const GMEM v4u *)(it.units + off + q4kt::qs_off(kq, c) + 16);
            R.h[u] = *(const GMEM uint32_t *)(it.units + off + 4 * lane);
        }
    };

    // B: lane (k-group kq, column c) reads digit c % 3 of sub-block 2kq + h
    // when c / 3 == kq, else the zero region
    const bool active = c < 12 && c / 3 == kq;
    const int gcol = c < 12 ? c / 3 : 0;
    const int k4 = lane & 3, R4 = lane >> 2;
    const float f = c < 12 ? (c % 3 == 0 ? 1.0f : c % 3 == 1 ? 256.0f : 65536.0f) : 0.0f;
    // three or four tokens: B's column c is (group c / 4, token c % 4), one
    // MFMA chain a digit, so that a lane's three digits meet in its own
    // registers and every column but a missing token's carries data
    constexpr bool kPack = NT >= 3;
    const int pg = c / 4, pt = c % 4;
    const bool pactive = pg == kq && pt < NT;

    auto compute_packed = [=](const Regs<kK> &R, const Item &it, unsigned slot) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, macc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) macc[t] = 0.0f;
#pragma unroll
        for (int u = 0; u < kK; u++) {
            if (u >= it.nblk) break;
            const unsigned bl = it.bl + (unsigned)u;
            {
                const uint32_t w0 = quad_bcast<0>(R.h[u]), w1 = quad_bcast<1>(R.h[u]), w2 = quad_bcast<2>(R.h[u]),
                               w3 = quad_bcast<3>(R.h[u]);
                const float d = f16_bits(w0 & 0xffffu), dmin = f16_bits(w0 >> 16);
                float sc0, sc1, mn0, mn1;
                scales_pair(w1, w2, w3, k4, sc0, sc1, mn0, mn1);
                const float D0 = d * sc0, D1 = d * sc1;
                const float mA = dmin * mn0, mB = dmin * mn1 - 8.0f * D1;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const float4 xm = stl[(bl * NT + t) * 8 + 2 * k4 + 1];
                    macc[t] += mA * (xm.x + xm.y) + mB * (xm.z + xm.w);
                }
                hdr[(2 * k4) * kHdrStride + R4] = D0;
                hdr[(2 * k4 + 1) * kHdrStride + R4] = D1 * 0.0625f;
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            // lane (kq, c): token pt's planes of sub-blocks 2kq + h, if pg == kq
            const v4i *bbase = lv + (pactive ? (int)((bl * NT + (unsigned)pt) * kBT) + 4 * kq : (int)kZero);
            const float4 *sxp = stl + (bl * NT + (unsigned)(pt < NT ? pt : 0)) * 8 + 2 * pg;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t mask = h ? 0xf0f0f0f0u : 0x0f0f0f0fu;
                const float4 Dsb = *(const float4 *)&hdr[(2 * pg + h) * kHdrStride + 4 * kq];
                const float sx = ((const float *)sxp)[2 * h];
                const v4u q0 = R.q[u][0], q1 = R.q[u][1];
                const v4i a0 = {(int)(q0.x & mask), (int)(q0.y & mask), (int)(q0.z & mask), (int)(q0.w & mask)};
                const v4i a1 = {(int)(q1.x & mask), (int)(q1.y & mask), (int)(q1.z & mask), (int)(q1.w & mask)};
                // the sub-block's two groups of 16 (its two MFMAs, m = 0, 1)
                // each with its own activation scale
                v4i C[3], E[3];
#pragma unroll
                for (int r = 0; r < 3; r++) {
                    const v4i *bp = bbase + r * kPStride + 2 * h;
                    C[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bp[0], v4i{0, 0, 0, 0}, 0, 0, 0);
                    E[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bp[1], v4i{0, 0, 0, 0}, 0, 0, 0);
                }
                const float sx1 = ((const float *)sxp)[2 * h + 1];
                // the digits meet (weights 1, 256, 65536; the first two in
                // int32: a column sums 16 products of at most 128·128, so
                // |C0| + 256·|C1| < 2^27), then the scales
                const float Ds[4] = {Dsb.x * sx, Dsb.y * sx, Dsb.z * sx, Dsb.w * sx};
                const float Es[4] = {Dsb.x * sx1, Dsb.y * sx1, Dsb.z * sx1, Dsb.w * sx1};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v = (float)(C[0][e] + C[1][e] * 256) + 65536.0f * (float)C[2][e];
                    const float w = (float)(E[0][e] + E[1][e] * 256) + 65536.0f * (float)E[2][e];
                    acc[e] += Ds[e] * v + Es[e] * w;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_wave_barrier();
        }
        // the groups meet: lanes c, c + 4, c + 8, c + 12 of a row of 16 hold
        // token c % 4 (row rotations by 4 and 8); lanes 16kq..16kq+15 hold
        // rows 4kq..4kq+3.  The min terms of row R sit in lanes 4R..4R+3:
        // summed, parked per wave in the (now free) scale rows, read back by
        // the lanes that write the slots
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float v = acc[e];
            v += xlane::mov<0x124>(v);
            v += xlane::mov<0x128>(v);
            acc[e] = v;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float mt = group_sum<4>(macc[t]);
            if (k4 == 0) hdr[t * 16 + R4] = mt;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (c < NT) {
#pragma unroll
            for (int e = 0; e < 4; e++)
                slots[(slot * NT + (unsigned)c) * 16 + 4 * kq + e] = acc[e] - hdr[c * 16 + 4 * kq + e];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    };
    auto compute = [=](const Regs<kK> &R, const Item &it, unsigned slot) {
        if constexpr (kPack) {
            compute_packed(R, it, slot);
            return;
        }
        float acc[NT][4], macc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            acc[t][0] = acc[t][1] = acc[t][2] = acc[t][3] = 0.0f;
            macc[t] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kK; u++) {
            if (u >= it.nblk) break;
            const unsigned bl = it.bl + (unsigned)u;
            {
                const uint32_t w0 = quad_bcast<0>(R.h[u]), w1 = quad_bcast<1>(R.h[u]), w2 = quad_bcast<2>(R.h[u]),
                               w3 = quad_bcast<3>(R.h[u]);
                const float d = f16_bits(w0 & 0xffffu), dmin = f16_bits(w0 >> 16);
                float sc0, sc1, mn0, mn1;
                scales_pair(w1, w2, w3, k4, sc0, sc1, mn0, mn1);
                const float D0 = d * sc0, D1 = d * sc1;
                // the high nibble arrives as 16·(q − 8): scale d·sc/16, and
                // 8·d·sc joins the min term
                const float mA = dmin * mn0, mB = dmin * mn1 - 8.0f * D1;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const float4 xm = stl[(bl * NT + t) * 8 + 2 * k4 + 1];
                    macc[t] += mA * (xm.x + xm.y) + mB * (xm.z + xm.w);
                }
                hdr[(2 * k4) * kHdrStride + R4] = D0;
                hdr[(2 * k4 + 1) * kHdrStride + R4] = D1 * 0.0625f;
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            const v4i *bbase =
                lv + (active ? (int)(bl * NT * kBT) + kPStride * (c % 3) + 4 * kq : (int)kZero + u * NT * kBT);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t mask = h ? 0xf0f0f0f0u : 0x0f0f0f0fu;
                const float4 Dsb = *(const float4 *)&hdr[(2 * gcol + h) * kHdrStride + 4 * kq];
                const v4u q0 = R.q[u][0], q1 = R.q[u][1];
                const v4i a0 = {(int)(q0.x & mask), (int)(q0.y & mask), (int)(q0.z & mask), (int)(q0.w & mask)};
                const v4i a1 = {(int)(q1.x & mask), (int)(q1.y & mask), (int)(q1.z & mask), (int)(q1.w & mask)};
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const v4i *bp = bbase + t * kBT + 2 * h;
                    const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bp[0], v4i{0, 0, 0, 0}, 0, 0, 0);
                    const v4i E = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bp[1], v4i{0, 0, 0, 0}, 0, 0, 0);
                    // token t's scales of sub-block 2·gcol + h (its two groups of 16)
                    const float *sxt = (const float *)&stl[(bl * NT + t) * 8 + 2 * gcol];
                    const float sx = sxt[2 * h], sx1 = sxt[2 * h + 1];
                    acc[t][0] += (Dsb.x * sx) * (float)C[0] + (Dsb.x * sx1) * (float)E[0];
                    acc[t][1] += (Dsb.y * sx) * (float)C[1] + (Dsb.y * sx1) * (float)E[1];
                    acc[t][2] += (Dsb.z * sx) * (float)C[2] + (Dsb.z * sx1) * (float)E[2];
                    acc[t][3] += (Dsb.w * sx) * (float)C[3] + (Dsb.w * sx1) * (float)E[3];
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        // the columns meet, weighted by their digit: lanes 16kq..16kq+15 hold
        // rows 4kq..4kq+3; the min terms of row R sit in lanes 4R..4R+3
#pragma unroll
        for (int t = 0; t < NT; t++) {
#pragma unroll
            for (int e = 0; e < 4; e++) acc[t][e] = group_sum<16>(acc[t][e] * f);
            const float mt = group_sum<4>(macc[t]);
            const float mrow = __shfl(mt, 16 * kq + 4 * (c & 3), 64);
            if (c < 4)
                slots[(slot * NT + t) * 16 + 4 * kq + c] =
                    (c == 0 ? acc[t][0] : c == 1 ? acc[t][1] : c == 2 ? acc[t][2] : acc[t][3]) - mrow;
        }
    };

    // ---- the part's planes and statistics (from L2, every workgroup reads
    // them), then the first item's weights, then the planes' stores: the
    // barrier waits for the planes alone
    const unsigned n_w = i1 - i0 > (unsigned)wave ? (i1 - i0 - (unsigned)wave + kW - 1) / kW : 0u;
    Regs<kK> A, B;
    Item ia{}, ib{};
    // the finishing pass's first tile for this wave (a run holds fewer than
    // kW tiles, as a rule): its old outputs (x of x += W·in) and the emitted
    // planes' norm weights, loaded with the planes rather than in the run's
    // tail; lane (token pair ts, row) as in the finishing pass
    const int hf = lane >> 5, ts = (lane >> 4) & 1, row = lane & 15;
    const unsigned Tfirst = i0 / ip, Tlast = i1 > i0 ? (i1 - 1) / ip : Tfirst - 1;
    const unsigned Tw = Tfirst + (unsigned)wave;
    float pre0 = 0.0f, pre1 = 0.0f, pre_nw = 1.0f;
    // the RMS scales (given): wave t < NT sums token t's Σx² per group, the
    // first kRssLoads · 64 groups loaded with the planes, the rest (if any)
    // after; in group order, so that every workgroup scales by the same bits
    // (the loads are issued below)
    constexpr int kRssLoads = 6;
    const unsigned ngr = cols / 16u;
    const GMEM float *rs0 = (const GMEM float *)sload(a.rss[0]);
    const bool rms = rs0 != nullptr;
    const GMEM float *rsw = rs0;
#pragma unroll
    for (int q = 1; q < NT; q++) {
        const GMEM float *rq = (const GMEM float *)sload(a.rss[q]);
        rsw = wave == q ? rq : rsw;
    }
    float rsv[kRssLoads];
    // the head norms (given): thread (token, head) of the first NT·heads
    const bool hnorm = a.hss != nullptr;
    const unsigned nth = NT * a.heads;
    float4 hs0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), hs1 = hs0;
    {
        // a run of global memory a wave: token t's digit p (PB·16 chunks at
        // xq[t] + p·cols + pb·256) for run 4t + p, its statistics (PB·8 chunks
        // at xstat[t] + pb·32 floats) for run 4t + 3; with two tokens each run
        // is split over two waves.  Loads past a run's end reload its first
        // chunk and are stored nowhere.
        constexpr int kRuns = 4 * NT, kWpr = kW / kRuns > 0 ? kW / kRuns : 1;
        constexpr int kSL = (int)((kPlaneBudget / 16 / NT / 3 + 64 * kWpr - 1) / (64 * kWpr));
        const int run = wave % kRuns, sub = wave / kRuns;
        const bool staging = wave < kRuns * kWpr;
        const unsigned st_t = (unsigned)(run / 4), st_p = (unsigned)(run % 4);
        const bool st_stat = st_p == 3;
        const unsigned len = st_stat ? PB * 8u : PB * 16u;
        const GMEM int8_t *qrun = (const GMEM int8_t *)sload(a.xq[0]);
        const GMEM int8_t *srun = (const GMEM int8_t *)sload(a.xstat[0]);
#pragma unroll
        for (int q = 1; q < NT; q++) {
            const GMEM int8_t *xq_q = (const GMEM int8_t *)sload(a.xq[q]);
            const GMEM int8_t *xs_q = (const GMEM int8_t *)sload(a.xstat[q]);
            qrun = st_t == (unsigned)q ? xq_q : qrun;
            srun = st_t == (unsigned)q ? xs_q : srun;
        }
        const GMEM v4i *src = (const GMEM v4i *)(st_stat ? srun + (size_t)pb * 32u * 4u
                                                         : qrun + (size_t)(st_p < 3 ? st_p : 0u) * cols + pb * 256u);
        v4i v[kSL];
#pragma unroll
        for (int u = 0; u < kSL; u++) {
            const unsigned j = (unsigned)lane + 64u * (unsigned)(sub + kWpr * u);
            v[u] = src[j < len ? j : 0u];
        }
        // (unconditional, so that the waits count it: a wave without items
        // reloads the run's first, which every run has)
        ia = item_of(i0 + (n_w > 0 ? (unsigned)wave : 0u));
        load(A, ia);
        // (behind the planes and the first weights: the first tile's old
        // outputs and norm weights, and the RMS partial sums)
        if (Tw <= Tlast && i1 > i0) {
            const unsigned j = (unsigned)(Tw >= t01) + (unsigned)(Tw >= t02) + (unsigned)(Tw >= t03);
            const unsigned rj = sel(j, sreg(a.rows[0]), sreg(a.rows[1]), sreg(a.rows[2]), sreg(a.rows[3]));
            const unsigned grow = (Tw - sel(j, 0u, t01, t02, t03)) * 16 + (unsigned)row;
            const unsigned gr = grow < rj ? grow : 0u;
            const float *oj = sel(j, sreg(a.out[0]), sreg(a.out[1]), sreg(a.out[2]), sreg(a.out[3]));
            if ((a.add_mask >> j) & 1u) {
                pre0 = oj[(size_t)ts * rj + gr];
                if (ts + 2 < NT) pre1 = oj[(size_t)(ts + 2) * rj + gr];
            }
            if (a.emit_norm) pre_nw = a.emit_norm[gr];
        }
        if (rms && wave < NT) {
#pragma unroll
            for (int u = 0; u < kRssLoads; u++) {
                const unsigned gi = (unsigned)lane + 64u * (unsigned)u;
                rsv[u] = rsw[gi < ngr ? gi : 0u];
            }
        }
        if (hnorm && threadIdx.x < nth) {
            hs0 = ((const float4 *)a.hss)[2 * threadIdx.x];
            hs1 = ((const float4 *)a.hss)[2 * threadIdx.x + 1];
        }
        if (staging) {
#pragma unroll
            for (int u = 0; u < kSL; u++) {
                const unsigned j = (unsigned)lane + 64u * (unsigned)(sub + kWpr * u);
                if (j >= len) continue;
                // plane chunk j: block j / 16, chunk j % 16 of the digit;
                // statistics chunk j: block j / 8, chunk j % 8
                const unsigned dst = st_stat ? kStat + ((j / 8u) * NT + st_t) * 8u + j % 8u
                                             : ((j / 16u) * NT + st_t) * kBT + st_p * kPStride + j % 16u;
                lv[dst] = v[u];
            }
        }
        if (threadIdx.x < (unsigned)(kK * NT * kBT)) lv[kZero + threadIdx.x] = v4i{0, 0, 0, 0};
    }
    if (hnorm && threadIdx.x < nth)
        tf[threadIdx.x] = 1.0f / sqrtf((((hs0.x + hs0.y) + (hs0.z + hs0.w)) + ((hs1.x + hs1.y) + (hs1.z + hs1.w))) / 128.0f +
                                       a.heps);
    if (rms && wave < NT) {
        float t = 0.0f;
#pragma unroll
        for (int u = 0; u < kRssLoads; u++)
            if ((unsigned)lane + 64u * (unsigned)u < ngr) t += rsv[u];
        for (unsigned gi = (unsigned)lane + 64u * kRssLoads; gi < ngr; gi += 64u) t += rsw[gi];
        t = group_sum<64>(t);
        const float sc = 1.0f / sqrtf(t / (float)cols + a.eps);
        if (lane == 0) tsc[wave] = sc;
    }
    __syncthreads();
    if (hnorm) {
        // each statistics chunk (the scales or the sums of a 64-column run)
        // times its token's head norm
        for (unsigned e = threadIdx.x; e < PB * NT * 8u; e += kW * 64u) {
            const unsigned blk = e / (NT * 8u), t = (e / 8u) % NT, k = e % 8u;
            const unsigned head = ((pb + blk) * 4u + k / 2u) / 2u;
            const float f = tf[t * a.heads + head];
            float4 *ch = (float4 *)(lds + kStat) + e;
            float4 v = *ch;
            v.x *= f;
            v.y *= f;
            v.z *= f;
            v.w *= f;
            *ch = v;
        }
        __syncthreads();
    }

    // ---- the wave's items, the next one's weights in flight
    // (the loads are unconditional, past the last item a reload of it, so
    // that the waits before each item's arithmetic count only its own loads)
    for (unsigned k = 0; k < n_w; k += 2) {
        ib = item_of(i0 + wave + min(k + 1, n_w - 1) * kW);
        load(B, ib);
        compute(A, ia, wave + k * kW);
        ia = item_of(i0 + wave + min(k + 2, n_w - 1) * kW);
        load(A, ia);
        if (k + 1 < n_w) compute(B, ib, wave + (k + 1) * kW);
    }
    __syncthreads();

    // ---- each tile of the run: its items' sums in order, by one wave
    // lane (half hf, token pair ts, row): tokens ts and ts + 2
    for (unsigned T = Tw; T <= Tlast && i1 > i0; T += kW) {
        // the lane's half's items of the tile in this run, in order (a few
        // LDS reads in flight at once)
        const unsigned lo = max(max(i0, T * ip), T * ip + (unsigned)hf * ih);
        const unsigned hi = min(min(i1, (T + 1) * ip), T * ip + ((unsigned)hf + 1) * ih);
        float v0 = 0.0f, v1 = 0.0f;
#pragma unroll 4
        for (unsigned i = lo; i < hi; i++) {
            const float *sl = slots + (size_t)(i - i0) * NT * 16;
            v0 += sl[ts * 16 + row];
            if (ts + 2 < NT) v1 += sl[(ts + 2) * 16 + row];
        }
        const bool whole = P == 1 && T * ip >= i0 && (T + 1) * ip <= i1;
        if (!whole) {
            // the workgroups sharing the tile meet: this one's slot is its
            // index among the part's workgroups that hold a piece of the tile
            auto wg_of = [=](unsigned long long item, unsigned long long I, unsigned Gq) {
                return (unsigned)(((item + 1) * Gq - 1) / I);
            };
            const unsigned cl = gp - wg_of((unsigned long long)T * ip, Ip, G);
            float *pp = a.partials + (((size_t)T * P + p) * a.cmax + cl) * NT * 32;
            __hip_atomic_store(pp + ts * 32 + hf * 16 + row, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (ts + 2 < NT)
                __hip_atomic_store(pp + (ts + 2) * 32 + hf * 16 + row, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // the same ordering as the one-token kernel's meeting
            // (k_mv_q4k_mfma.hip): sc1 stores acknowledged before the
            // counter's add, sc1 loads only under a branch on its result
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            unsigned n_c = 0;
            for (unsigned q = 0; q < P; q++) {
                const unsigned ihq = sel(q, ih0, ih1, ih2, ih3), ipq = J * ihq;
                const unsigned Gq = sel(q + 1, 0u, g01, g02, g03, g04) - sel(q, 0u, g01, g02, g03);
                const unsigned long long Iq = (unsigned long long)TT * ipq;
                n_c += wg_of((unsigned long long)(T + 1) * ipq - 1, Iq, Gq) - wg_of((unsigned long long)T * ipq, Iq, Gq) + 1;
            }
            unsigned old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(&a.counters[T], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __shfl(old, 0, 64);
            if (old != n_c - 1) continue;
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            v0 = v1 = 0.0f;
            for (unsigned q = 0; q < P; q++) {
                const unsigned ihq = sel(q, ih0, ih1, ih2, ih3), ipq = J * ihq;
                const unsigned Gq = sel(q + 1, 0u, g01, g02, g03, g04) - sel(q, 0u, g01, g02, g03);
                const unsigned long long Iq = (unsigned long long)TT * ipq;
                const unsigned nq = wg_of((unsigned long long)(T + 1) * ipq - 1, Iq, Gq) -
                                    wg_of((unsigned long long)T * ipq, Iq, Gq) + 1;
                const float *tp = a.partials + ((size_t)T * P + q) * a.cmax * NT * 32;
                for (unsigned s = 0; s < nq; s++) {
                    v0 += __hip_atomic_load(tp + s * NT * 32 + ts * 32 + hf * 16 + row, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
                    if (ts + 2 < NT)
                        v1 += __hip_atomic_load(tp + s * NT * 32 + (ts + 2) * 32 + hf * 16 + row, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            if (lane == 0) __hip_atomic_store(&a.counters[T], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // the tile's results: lanes of half 0 hold gate (or the product),
        // lanes of half 1 up
        // (v_permlane32_swap of a value with itself: lanes < 32 get their
        // own value first, then lane + 32's)
        const auto s0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v0), false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v1), __float_as_uint(v1), false, false);
        float x0 = __uint_as_float(s0[0]), y0 = __uint_as_float(s0[1]);
        float x1 = __uint_as_float(s1[0]), y1 = __uint_as_float(s1[1]);
        if (rms) {
            const float f0 = tsc[ts], f1 = tsc[ts + 2 < NT ? ts + 2 : ts];
            x0 *= f0;
            y0 *= f0;
            x1 *= f1;
            y1 *= f1;
        }
        const unsigned j = (unsigned)(T >= t01) + (unsigned)(T >= t02) + (unsigned)(T >= t03);
        const unsigned rj = sel(j, sreg(a.rows[0]), sreg(a.rows[1]), sreg(a.rows[2]), sreg(a.rows[3]));
        const unsigned grow = (T - sel(j, 0u, t01, t02, t03)) * 16 + (unsigned)row;
        float *oj = sel(j, sreg(a.out[0]), sreg(a.out[1]), sreg(a.out[2]), sreg(a.out[3]));
        if (hf != 0 || grow >= rj) continue;
        const bool adds = (a.add_mask >> j) & 1u;
        float r0 = x0, r1 = x1;
        if (a.swiglu) {
            r0 = x0 * sigmoidf_(x0) * y0;  // silu(gate) · up (gpu/cpu.rs:238-242)
            r1 = x1 * sigmoidf_(x1) * y1;
        }
        const bool first = T == Tw;  // (its old outputs and weights loaded up front)
        float *o0 = oj + (size_t)ts * rj + grow;
        const float e0 = adds ? (first ? pre0 : *o0) + r0 : r0;
        *o0 = e0;
        float e1 = 0.0f;
        if (ts + 2 < NT) {
            float *o1 = oj + (size_t)(ts + 2) * rj + grow;
            e1 = adds ? (first ? pre1 : *o1) + r1 : r1;
            *o1 = e1;
        }
        if (a.emit) {
            // lanes 16ts..16ts+15 (one group of 16, the tile's rows): tokens
            // ts and ts + 2
            const float nw = first ? pre_nw : a.emit_norm ? a.emit_norm[grow] : 1.0f;
            auto emit_one = [&](unsigned tok, float f) {
                const planes::View v = planes::view(a.emit + tok * planes::kAreaBytes, rj);
                const float xv = f * nw;
                if (a.emit_norm) {
                    const float sq = group_sum<16>(f * f);
                    if (row == 0) v.ss[grow / 16] = sq;
                }
                if (a.emit_xw) a.emit_xw[(size_t)tok * rj + grow] = xv;
                planes::write16(v, grow, xv);
            };
            emit_one((unsigned)ts, e0);
            if (ts + 2 < NT) emit_one((unsigned)ts + 2, e1);
        }
    }
    // ---- the small bf16 matrix's (row, token) pairs, a wave each: 8 columns
    // a lane a load, the loads of 5 such steps issued together
    if (a.bf_w && wave >= kW - 4) {
        for (unsigned q = g + gridDim.x * (unsigned)(wave - (kW - 4)); q < a.bf_rows * (unsigned)NT; q += 4u * gridDim.x) {
            const unsigned r = q / (unsigned)NT, t = q % (unsigned)NT;
            const uint4 *wr = (const uint4 *)(a.bf_w + (size_t)r * a.bf_cols);
            const float4 *xr = (const float4 *)(a.bf_x + (size_t)t * a.bf_cols);
            const unsigned n8 = a.bf_cols / 8;
            float acc = 0.0f;
            for (unsigned c0 = (unsigned)lane; c0 < n8; c0 += 5 * 64) {
                uint4 wv[5];
                float4 x0[5], x1[5];
#pragma unroll
                for (int u = 0; u < 5; u++) {
                    const unsigned cu = c0 + 64u * u < n8 ? c0 + 64u * u : c0;
                    wv[u] = wr[cu];
                    x0[u] = xr[2 * cu];
                    x1[u] = xr[2 * cu + 1];
                }
#pragma unroll
                for (int u = 0; u < 5; u++) {
                    if (c0 + 64u * u >= n8) continue;
                    const uint32_t pw[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                    const float xs[8] = {x0[u].x, x0[u].y, x0[u].z, x0[u].w, x1[u].x, x1[u].y, x1[u].z, x1[u].w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc += __uint_as_float(pw[i] << 16) * xs[2 * i] + __uint_as_float(pw[i] & 0xffff0000u) * xs[2 * i + 1];
                }
            }
            acc = group_sum<64>(acc);
            if (lane == 0) a.bf_out[(size_t)t * a.bf_rows + r] = acc * (rms ? tsc[t] : 1.0f);
        }
    }
}

}  // namespace

hipError_t run_mv_stream(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, const int *adds, int count,
                         int swiglu, size_t nt, const int8_t *const *xq, const float *const *xstat,
                         const StreamExtra *se) {
    if (nt < 2 || nt > (size_t)kTok || count < 1 || count > kJobs || (swiglu && count != 2)) return hipErrorInvalidValue;
    const unsigned NT = (unsigned)nt, J = swiglu ? 2u : 1u, njobs = swiglu ? 1u : (unsigned)count;
    const unsigned K = (unsigned)k_of((int)nt);
    StreamArgs a{};
    a.nb = (unsigned)(ws[0]->cols / 256);
    a.swiglu = swiglu;
    unsigned TT = 0;
    for (unsigned j = 0; j < (unsigned)kJobs; j++) {
        a.tile0[j] = j < njobs ? TT : 0xffffffffu;
        if (j < njobs) TT += (unsigned)q4kt::tiles(ws[j]->rows);
    }
    a.tile0[0] = 0;
    a.tile0[kJobs] = TT;
    for (int j = 0; j < count; j++) {
        a.w[j] = (const uint8_t *)ws[j]->q;
        a.out[j] = outs[j];
        a.rows[j] = (unsigned)ws[j]->rows;
        if (adds && adds[j] && (unsigned)j < njobs) a.add_mask |= 1u << j;
    }
    if (TT > dev->mv_tiles_cap) return hipErrorInvalidValue;
    // parts: as few as keep a part's planes within the LDS budget
    const size_t per_block = (size_t)NT * (kBT + 8) * 16;
    const unsigned pb_max = (unsigned)(kPlaneBudget / per_block);
    a.P = (a.nb + pb_max - 1) / pb_max;
    if (a.P > (unsigned)kParts) return hipErrorInvalidValue;
    unsigned long long I = 0, Ipart[kParts];
    unsigned plane_cap = 0;
    for (unsigned p = 0; p <= a.P; p++) a.pb0[p] = p * a.nb / a.P;
    for (unsigned p = 0; p < a.P; p++) {
        const unsigned PB = a.pb0[p + 1] - a.pb0[p];
        plane_cap = std::max(plane_cap, PB);
        a.ih[p] = (PB + K - 1) / K;
        Ipart[p] = (unsigned long long)TT * J * a.ih[p];
        I += Ipart[p];
    }
    // one workgroup a CU, shared out among the parts by their items
    const unsigned G = (unsigned)std::min<unsigned long long>((unsigned long long)dev->cus, I);
    unsigned given = 0;
    unsigned Gp[kParts];
    for (unsigned p = 0; p < a.P; p++) {
        Gp[p] = (unsigned)std::max<unsigned long long>(1, std::min<unsigned long long>(Ipart[p], Ipart[p] * G / I));
        given += Gp[p];
    }
    // the rounding's leftover to the part with the most items a workgroup
    while (given < G) {
        unsigned best = 0;
        for (unsigned p = 1; p < a.P; p++)
            if (Ipart[p] * Gp[best] > Ipart[best] * Gp[p]) best = p;
        if (Gp[best] >= Ipart[best]) break;
        Gp[best]++, given++;
    }
    unsigned items_cap = 0, cmax = 0;
    a.g0[0] = 0;
    for (unsigned p = 0; p < a.P; p++) {
        a.g0[p + 1] = a.g0[p] + Gp[p];
        items_cap = std::max(items_cap, (unsigned)((Ipart[p] + Gp[p] - 1) / Gp[p]));
        const unsigned long long ip = (unsigned long long)J * a.ih[p];
        auto wg_of = [=](unsigned long long item) { return (unsigned)(((item + 1) * Gp[p] - 1) / Ipart[p]); };
        for (unsigned T = 0; T < TT; T++) cmax = std::max(cmax, wg_of((T + 1) * ip - 1) - wg_of(T * ip) + 1);
    }
    for (unsigned p = a.P + 1; p <= (unsigned)kParts; p++) a.g0[p] = a.g0[a.P];
    a.cmax = cmax;
    a.plane_cap = plane_cap;
    a.items_cap = items_cap;
    if ((size_t)TT * a.P * cmax * NT * 32 > dev->mv_stream_cap) return hipErrorInvalidValue;
    a.partials = dev->mv_stream;
    a.counters = dev->mv_counters;
    for (unsigned t = 0; t < NT; t++) {
        a.xq[t] = xq[t];
        a.xstat[t] = xstat[t];
    }
    if (se && se->rms) {
        // (each token's planes are the start of its plane area)
        for (unsigned t = 0; t < NT; t++) a.rss[t] = (const float *)(xq[t] + planes::kSsOff);
        a.eps = se->eps;
    }
    if (se && se->head_ss) {
        if (ws[0]->cols % 128) return hipErrorInvalidValue;
        a.hss = se->head_ss;
        a.heps = se->head_eps;
        a.heads = (unsigned)(ws[0]->cols / 128);
        if (NT * a.heads > (unsigned)(kW * 64)) return hipErrorInvalidValue;
    }
    if (se && se->bf16) {
        const dwim_weight *b = se->bf16;
        if (b->fmt != DWIM_BF16 || b->cols % 8 || !se->bf16_x || !se->bf16_out) return hipErrorInvalidValue;
        a.bf_w = (const uint16_t *)b->q;
        a.bf_x = se->bf16_x;
        a.bf_out = se->bf16_out;
        a.bf_rows = (unsigned)b->rows;
        a.bf_cols = (unsigned)b->cols;
    }
    if (se && se->emit_area >= 0) {
        const size_t rows = ws[0]->rows;
        if ((njobs != 1 && !swiglu) || rows % 256 || rows > planes::kMaxCols || se->emit_area < 0 ||
            (size_t)se->emit_area + NT > (size_t)kBatchArea2 + kTok)
            return hipErrorInvalidValue;
        a.emit = planes_area(dev, se->emit_area, rows).q;
        a.emit_norm = se->emit_norm;
        a.emit_xw = se->emit_xw;
    }
    const size_t lds = ((size_t)plane_cap * NT * (kBT + 8) + (size_t)K * NT * kBT + (size_t)kW * kHdrChunks + 1 +
                        (NT * a.heads + 3) / 4) * 16 +
                       (size_t)items_cap * NT * 16 * 4;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    // raised once a process for each kernel (a function-local static is
    // initialized once even when host threads reach it together)
    static const hipError_t raised[3] = {
        hipFuncSetAttribute((const void *)k_mv_stream<2>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024),
        hipFuncSetAttribute((const void *)k_mv_stream<3>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024),
        hipFuncSetAttribute((const void *)k_mv_stream<4>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024)};
    if (raised[NT - 2] != hipSuccess) return raised[NT - 2];
    if (NT == 2) k_mv_stream<2><<<G, kW * 64, lds, dev->stream>>>(a);
    else if (NT == 3) k_mv_stream<3><<<G, kW * 64, lds, dev->stream>>>(a);
    else k_mv_stream<4><<<G, kW * 64, lds, dev->stream>>>(a);
    return hipGetLastError();
}
