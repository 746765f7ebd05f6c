// Q4_K matrix-vector products for one token on the int8 matrix cores, with
// results at f32 accuracy (dwim gpu/cpu.rs:110-149 computes them in f32).
//
// The activations come as int8 planes (planes.h): per group of 16, 24-bit
// fixed point of the group's largest value, as three digits.  k_planes
// writes them from f32 activations, RMS-normalizing first when asked (the
// reference's `normalize`, gpu/cpu.rs:157-166); the fused kernels of
// k_fused.hip write them from what they produce.
//
// The product runs v_mfma_i32_16x16x64_i8 with the 16 rows of a weight tile as
// A and the planes as B.  For one tile and one 256-block, half h ∈ {0, 1} of
// the block is sub-blocks 2g + h (g = 0..3, the quant group): the lanes of
// k-group g hold row r's 16 quants of sub-block 2g + h at positions
// 16m..16m+15 (m = 0, 1: two MFMAs per half), and B's column 3g' + p holds
// digit p of sub-block 2g' + h, nonzero only in k-group g'.  The two MFMAs of a
// half accumulate, per row, Σ q·X_p of each of the 4 sub-blocks into its own
// column, exactly, in int32.  Each is scaled in f32 by its row's d·sc times
// the group's activation scale (the low nibble is q; the high one arrives as
// 16·(q − 8), so its scale is d·sc/16 and 8·d·sc joins the min term), and the
// columns meet at the end weighted 2^(8p).  The min term −dmin·m·Σx is added
// per row and sub-block by the lanes that decode the headers.
//
// Per weight that is a quarter of a VALU op to unpack, and the MFMA; the f32
// path costs over two.  A wave takes up to K blocks of a tile and issues
// every load before any compute: the planes of its blocks (parked in LDS,
// where the B operands are read from), then the weights.
//
// Modes: several matrices sharing x in one launch (workgroups find their
// matrix from their index), x += W·in (gpu/mod.rs:259), and gate and up paired
// into silu(gate·x)·(up·x) (gpu/mod.rs:274-285): the waves of a workgroup
// take gate's rows of its tile, then up's.
#include "device_util.h"
#include "layout.h"
#include "mv_common.h"
#include "planes.h"
#include "quant_math.h"
#include "runtime.h"

#include <stdlib.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

namespace {

using namespace mvq;

// One token's planes from f32 activations.  A workgroup of 256 writes 1024
// activations (four lanes a group of 16, four each).  With a norm, either
// (handover = 0) x is RMS-normalized first, every workgroup summing the
// squares of the whole vector itself in the same order so that all of them
// scale by the same bits; or (handover = 1) the planes are of x·norm with
// each group's Σx², for a product that applies the RMS scale itself.
// xn_out, when given, receives what the planes hold, in f32.  pair: the
// scales are per 32 activations (planes.h), for the several-token product;
// blockIdx.y numbers the tokens of such a batch.
constexpr int kPlanesThreads = 256;

__global__ void __launch_bounds__(kPlanesThreads) k_planes(const float *__restrict__ x, const float *norm, float eps,
                                                           int handover, float *xn_out, planes::View out,
                                                           int pair = 0) {
    __shared__ float red[kPlanesThreads / 64];
    const unsigned n4 = (unsigned)(out.cols / 4);
    // token blockIdx.y of a batch: its row of x, its area (the next one on)
    x += (size_t)blockIdx.y * out.cols;
    if (xn_out) xn_out += (size_t)blockIdx.y * out.cols;
    if (blockIdx.y) out = planes::view(out.q + blockIdx.y * planes::kAreaBytes, out.cols);
    float scale = 1.0f;
    if (norm && !handover) {
        float ss = 0.0f;
        for (unsigned i = threadIdx.x; i < n4; i += kPlanesThreads) {
            const float4 v = ((const float4 *)x)[i];
            ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        }
        ss = block_sum<kPlanesThreads>(ss, red);
        scale = 1.0f / sqrtf(ss / (float)out.cols + eps);
    }
    // cols / 4 is a whole number of waves, so every group of 4 lanes is whole
    const unsigned i = blockIdx.x * kPlanesThreads + threadIdx.x;
    if (i >= n4) return;
    float4 v = ((const float4 *)x)[i];
    if (norm) {
        if (handover) {
            float sq = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
            sq += __shfl_xor(sq, 1, 64);
            sq += __shfl_xor(sq, 2, 64);
            if ((i & 3) == 0) out.ss[i / 4] = sq;
        }
        const float4 w = ((const float4 *)norm)[i];
        v.x = v.x * (scale * w.x);
        v.y = v.y * (scale * w.y);
        v.z = v.z * (scale * w.z);
        v.w = v.w * (scale * w.w);
        if (xn_out) ((float4 *)xn_out)[i] = v;
    }
    planes::write4x4(out, i, v, pair != 0);
}

// The planes of the DeltaNet layer's output gate, silu(z)·rmsnorm(att)·w per
// head of 128 (gpu/cpu.rs:157-166, 238-242, as k_gated_norm computes it), in
// pair mode, for the tokens of a batch (blockIdx.y): the gated norm made
// where the output product's planes are made, one launch instead of two.  A
// head is 32 lanes of float4s.
__global__ void __launch_bounds__(kPlanesThreads) k_planes_gated(const float *__restrict__ z,
                                                                 const float *__restrict__ att,
                                                                 const float *__restrict__ w, float eps,
                                                                 planes::View out) {
    const unsigned n4 = (unsigned)(out.cols / 4);
    z += (size_t)blockIdx.y * out.cols;
    att += (size_t)blockIdx.y * out.cols;
    if (blockIdx.y) out = planes::view(out.q + blockIdx.y * planes::kAreaBytes, out.cols);
    const unsigned i = blockIdx.x * kPlanesThreads + threadIdx.x;
    if (i >= n4) return;  // (cols / 4 is whole waves)
    const float4 a = ((const float4 *)att)[i];
    const float ss = group_sum<32>((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w));
    const float scale = 1.0f / sqrtf(ss / 128.0f + eps);
    const float4 nw = ((const float4 *)w)[i % 32];
    float4 g = ((const float4 *)z)[i];
    g.x = g.x * sigmoidf_(g.x) * (a.x * (scale * nw.x));
    g.y = g.y * sigmoidf_(g.y) * (a.y * (scale * nw.y));
    g.z = g.z * sigmoidf_(g.z) * (a.z * (scale * nw.z));
    g.w = g.w * sigmoidf_(g.w) * (a.w * (scale * nw.w));
    planes::write4x4(out, i, g, true);
}

constexpr int kMaxJobs = 4;
constexpr int kMaxParts = 4;
constexpr int kMaxTok = 4;     // tokens of a several-token launch (a verify batch: 1 + 3 drafts)
static_assert(kBatchArea2 == kBatchArea + kMaxTok, "the two sets of batch areas lie one after the other");
// RMS partial sums a lane loads up front: 6 · 64 groups of 16 cover 6144
// columns (the rest, if any, are loaded at the end)
constexpr int kRmsLoads = 6;

struct Args {
    const uint8_t *w[kMaxJobs];
    float *out[kMaxJobs];
    unsigned rows[kMaxJobs];
    unsigned first[kMaxJobs];      // first workgroup of each matrix; all ones past the last
    unsigned tile0[kMaxJobs];      // the matrix's first tile in the launch's tile numbering
    unsigned add_mask;             // bit j: out[j] += W_j·x, else out[j] = W_j·x
    unsigned nb;                   // 256-blocks per row
    unsigned S;                    // waves per matrix in a workgroup
    unsigned P;                    // workgroups (parts) per tile
    int swiglu;                    // out[0] = silu(W_0·x) · (W_1·x), waves S..2S-1 taking W_1
    const int8_t *xq;              // the planes, [3][cols]
    const float4 *xstat;           // [cols/64][2]: four groups' scales, then their sums
    const float *rms_ss;           // given: the planes are x·w, results scale by 1/sqrt(Σ ss / cols + eps)
    float eps;
    // given (matrix 0 only): the planes of out[0] (after the add or the
    // SwiGLU) into `emit`; with emit_norm, of out[0]·emit_norm with each
    // group's Σ out[0]² (and out[0]·emit_norm in f32 into emit_xw if given)
    planes::View emit;
    const float *emit_norm;
    float *emit_xw;
    float *partials;               // P > 1: [tile][part][token][2][16]
    unsigned *counters;            // P > 1: [tile], zero between launches
    // given: the planes hold each head of head_dim columns unnormalized;
    // its groups' scales and sums are multiplied by 1/sqrt(Σ head_ss[head]
    // / head_dim + head_eps) (head_ss: [heads][4] partial sums of squares)
    const float4 *head_ss;
    unsigned head_dim;
    float head_eps;
    // given: the first bf_groups workgroups (dispatched first, so that they
    // are done long before the matrices' last) compute out = W·x for a small
    // bf16 matrix [bf_rows][bf_cols] and f32 x, a wave a row
    const uint16_t *bf_w;
    const float *bf_x;
    float *bf_out;
    unsigned bf_rows, bf_cols, bf_groups;
};

// A wave's row of a small bf16 matrix against f32 x (cols a multiple of 8):
// 8 columns a lane a load, the loads of 5 such steps issued together.
DEV void bf16_row(const Args &a, unsigned row, int lane) {
    const uint4 *w = (const uint4 *)(a.bf_w + (size_t)row * a.bf_cols);
    const float4 *x = (const float4 *)a.bf_x;
    const unsigned n8 = a.bf_cols / 8;
    float acc = 0.0f;
    for (unsigned c0 = (unsigned)lane; c0 < n8; c0 += 5 * 64) {
        uint4 wv[5];
        float4 x0[5], x1[5];
#pragma unroll
        for (int u = 0; u < 5; u++) {
            const unsigned c = c0 + 64u * u < n8 ? c0 + 64u * u : c0;
            wv[u] = w[c];
            x0[u] = x[2 * c];
            x1[u] = x[2 * c + 1];
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
    if (lane == 0) a.bf_out[row] = acc;
}

// Per wave LDS, in 16-byte chunks: the planes of its K blocks (chunk
// 51i + 17p + c holds activations 16c..16c+15 of digit p of block i: each
// digit's 16 chunks padded by one, so that the 12 lanes reading B operands,
// chunks 17p + 4k + const, fall in distinct banks), the group statistics
// (chunks 8i + 2k and 8i + 2k + 1: scales and sums of groups 4k..4k+3 of
// block i), two zero chunks and the decoded scales ([group][row] floats,
// rows of 20 floats: the float4 reads of 16 (group, row-quad) pairs and the
// writes of 4 groups of 16 rows then spread over the banks).
// The plane loads come in whole waves of 64 chunks; the spare ones past
// K·48 are stored into the statistics area, which is written after them.
template <int K>
struct Lds {
    static constexpr int kPStride = 17;
    static constexpr int kBlk = 3 * kPStride;
    static constexpr int kPlaneLoads = (K * 48 + 63) / 64;
    static constexpr int kStat = K * kBlk;
    static constexpr int kZero = kStat + 64;
    static constexpr int kHdr = kZero + 2;
    static constexpr int kHdrStride = 20;
    static constexpr int kChunks = kHdr + 16 * kHdrStride / 4;
    // chunk ci of the loads (48 a block, 16 a digit) lands at ci + ci / 16
    static constexpr int kLastSpare = kPlaneLoads * 64 - 1 + (kPlaneLoads * 64 - 1) / 16;
    static_assert(kLastSpare < kZero, "spare plane chunks must land in the statistics area");
};

template <int K>
__global__ void __launch_bounds__(1024) k_mv_q4k_mfma(const Args a) {
    using L = Lds<K>;
    extern __shared__ uint4 lds_all[];
    __shared__ float red[16][16];
    const int lane = threadIdx.x & 63, wave_all = threadIdx.x >> 6, kq = lane >> 4, c = lane & 15;
    if (blockIdx.x < a.bf_groups) {
        // the small bf16 matrix's rows, a wave each
        const unsigned row = blockIdx.x * (blockDim.x / 64) + (unsigned)wave_all;
        if (row < a.bf_rows) bf16_row(a, row, lane);
        return;
    }
    // every argument is read up front and selected without branches, so that
    // the scalar loads of the kernel arguments issue together; a launch's
    // unused first[] entries are all ones
    const unsigned S = a.S, P = a.P, nb = a.nb, bx = blockIdx.x - a.bf_groups;
    const unsigned f1 = a.first[1], f2 = a.first[2], f3 = a.first[3];
    const int j = (int)(bx >= f1) + (int)(bx >= f2) + (int)(bx >= f3);
    const unsigned wg = bx - (j == 0 ? 0u : j == 1 ? f1 : j == 2 ? f2 : f3);
    const unsigned tile = wg / P, part = wg - tile * P;
    const int pairj = a.swiglu != 0 && (unsigned)wave_all >= S;  // a swiglu workgroup's W_1 waves
    const unsigned wave = (unsigned)wave_all - (pairj ? S : 0u);
    const int jw = j + pairj;
    const uint8_t *wbase = jw == 0 ? a.w[0] : jw == 1 ? a.w[1] : jw == 2 ? a.w[2] : a.w[3];
    // this wave's blocks [b0, b1) of the tile: range part·S + wave of P·S
    const unsigned R = P * S, r = part * S + wave;
    const unsigned b0 = r * nb / R, b1 = (r + 1) * nb / R;
    const int nblk = (int)(b1 - b0);
    const uint8_t *wt = wbase + ((size_t)tile * nb + b0) * q4kt::kUnit;
    uint4 *my = lds_all + wave_all * L::kChunks;
    float *hdr = (float *)(my + L::kHdr);

    // every load of the wave is issued before any compute: the planes and
    // statistics of its blocks first, then the weights
    constexpr int kPlaneLoads = L::kPlaneLoads;
    v4u xc[kPlaneLoads];  // (a vector type: uint4 copies went through private memory)
    const unsigned cols = nb * 256;
#pragma unroll
    for (int u = 0; u < kPlaneLoads; u++) {
        // chunks past the wave's blocks reload chunk 0 (no branch around a load)
        const int ci0 = lane + 64 * u;
        const int ci = ci0 < nblk * 48 ? ci0 : 0;
        const unsigned i = (unsigned)ci / 48u, p = ((unsigned)ci % 48u) / 16u, part16 = (unsigned)ci % 16u;
        xc[u] = *(const v4u *)(a.xq + p * cols + (b0 + i) * 256u + 16u * part16);
    }
    const unsigned sti = b0 * 8u + (lane < nblk * 8 ? (unsigned)lane : 0u);
    float4 st = a.xstat[sti];
    // (a 64-column run of the statistics: float4 sti / 2)
    const float4 hss = a.head_ss ? a.head_ss[(sti / 2u) * 64u / a.head_dim] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    // the RMS partial sums (up to kRmsLoads per lane) are loaded here too,
    // by every wave and without a branch, and added up at the end
    const unsigned ng = cols / (unsigned)planes::kGroup;
    const float *ssrc = a.rms_ss ? a.rms_ss : (const float *)a.xstat;
    float ssv[kRmsLoads];
#pragma unroll
    for (int t = 0; t < kRmsLoads; t++) {
        const unsigned g = (unsigned)lane + 64u * t;
        ssv[t] = ssrc[g < ng ? g : 0u];
    }
    // and the tile's old outputs (x of x += W·in) and next norm weights
    const unsigned orow = tile * 16 + (unsigned)(lane & 15);
    const unsigned orows = j == 0 ? a.rows[0] : j == 1 ? a.rows[1] : j == 2 ? a.rows[2] : a.rows[3];
    float *const obase = j == 0 ? a.out[0] : j == 1 ? a.out[1] : j == 2 ? a.out[2] : a.out[3];
    const unsigned orow_c = orow < orows ? orow : 0u;
    const float old_out = (a.add_mask >> j) & 1u ? obase[orow_c] : 0.0f;
    const float next_w = a.emit_norm ? a.emit_norm[orow_c] : 0.0f;
    // (no memory access or instruction crosses this point: the compiler
    // would otherwise move plane loads behind the weights, so that the first
    // block's wait for the planes waits for most of the weights too, or the
    // planes' LDS stores, and their wait, ahead of the other loads)
    asm volatile("");
    uint4 wq[K][2];
    uint32_t hw[K];
#pragma unroll
    for (int i = 0; i < K; i++) {
        const unsigned off = (unsigned)(i < nblk ? i : 0) * (unsigned)q4kt::kUnit;
        wq[i][0] = *(const uint4 *)(wt + off + q4kt::qs_off(kq, c));
        wq[i][1] = *(const uint4 *)(wt + off + q4kt::qs_off(kq, c) + 16);
        hw[i] = *(const uint32_t *)(wt + off + 4 * lane);
    }
    // every chunk is stored, the spare ones too (a store under a branch would
    // let the compiler sink its load behind the weights); the statistics
    // then overwrite the spares
#pragma unroll
    for (int u = 0; u < kPlaneLoads; u++) ((v4u *)my)[lane + 64 * u + ((lane + 64 * u) >> 4)] = xc[u];
    if (a.head_ss) {
        const float f = 1.0f / sqrtf(((hss.x + hss.y) + (hss.z + hss.w)) / (float)a.head_dim + a.head_eps);
        st.x *= f;
        st.y *= f;
        st.z *= f;
        st.w *= f;
    }
    ((float4 *)(my + L::kStat))[lane] = st;
    if (lane < 2) my[L::kZero + lane] = make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

    // B: lane (k-group kq, column c) carries digit c % 3 of sub-block 2·kq + h
    // when c / 3 == kq, else the zero chunks
    const bool active = c < 12 && c / 3 == kq;
    const int bsel = active ? L::kPStride * (c % 3) + 4 * kq : 0;
    const int gcol = 4 * (c < 12 ? c / 3 : 0);  // the column's first group of 16
    const int k4 = lane & 3, R4 = lane >> 2;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float macc = 0.0f;
#pragma unroll
    for (int i = 0; i < K; i++) {
        if (i >= nblk) break;
        {
            // lane l decodes row l/4's sub-blocks 2(l%4), 2(l%4)+1 (groups
            // 4(l%4)..4(l%4)+3) from the header words its quad holds
            const uint32_t w0 = quad_bcast<0>(hw[i]), w1 = quad_bcast<1>(hw[i]), w2 = quad_bcast<2>(hw[i]),
                           w3 = quad_bcast<3>(hw[i]);
            const float d = f16_bits(w0 & 0xffffu), dmin = f16_bits(w0 >> 16);
            float sc0, sc1, mn0, mn1;
            scales_pair(w1, w2, w3, k4, sc0, sc1, mn0, mn1);
            const float4 xs = ((const float4 *)(my + L::kStat))[8 * i + 2 * k4];
            const float4 xm = ((const float4 *)(my + L::kStat))[8 * i + 2 * k4 + 1];
            const float D0 = d * sc0, D1 = d * sc1;
            // the low nibble is q; the high one arrives as 16·(q − 8), so its
            // scale is d·sc/16 and 8·d·sc joins the min term
            macc += (dmin * mn0) * (xm.x + xm.y) + (dmin * mn1 - 8.0f * D1) * (xm.z + xm.w);
            const float D1h = D1 * 0.0625f;
            hdr[(4 * k4) * L::kHdrStride + R4] = D0 * xs.x;
            hdr[(4 * k4 + 1) * L::kHdrStride + R4] = D0 * xs.y;
            hdr[(4 * k4 + 2) * L::kHdrStride + R4] = D1h * xs.z;
            hdr[(4 * k4 + 3) * L::kHdrStride + R4] = D1h * xs.w;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
        for (int h = 0; h < 2; h++) {
            // the two MFMAs of a half cover its two groups of 16, each summed
            // apart to take its own activation scale
            const uint4 *xv = my + (active ? L::kBlk * i + 2 * h + bsel : L::kZero);
            const uint32_t mask = h ? 0xf0f0f0f0u : 0x0f0f0f0fu;
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const uint4 q = wq[i][m], xq = xv[m];
                const v4i av = {(int)(q.x & mask), (int)(q.y & mask), (int)(q.z & mask), (int)(q.w & mask)};
                const v4i bv = {(int)xq.x, (int)xq.y, (int)xq.z, (int)xq.w};
                const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, v4i{0, 0, 0, 0}, 0, 0, 0);
                const float4 D = *(const float4 *)&hdr[(gcol + 2 * h + m) * L::kHdrStride + 4 * kq];
                acc[0] += D.x * (float)C[0];
                acc[1] += D.y * (float)C[1];
                acc[2] += D.z * (float)C[2];
                acc[3] += D.w * (float)C[3];
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    // the columns meet, weighted by their digit: lanes 16kq..16kq+15 hold
    // rows 4kq..4kq+3; the min terms of row R sit in lanes 4R..4R+3
    const float f = c < 12 ? (c % 3 == 0 ? 1.0f : c % 3 == 1 ? 256.0f : 65536.0f) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = group_sum<16>(acc[i] * f);
    macc = group_sum<4>(macc);
    const float mrow = __shfl(macc, 16 * kq + 4 * (c & 3), 64);
    if (c < 4) red[wave_all][4 * kq + c] = (c == 0 ? acc[0] : c == 1 ? acc[1] : c == 2 ? acc[2] : acc[3]) - mrow;
    __syncthreads();
    if (wave_all != 0) return;

    // wave 0 finishes the tile; lanes 0..15 hold its rows
    const bool mine = lane < 16;
    const int rl = lane & 15;
    float v = 0.0f, u = 0.0f;
    for (unsigned w = 0; w < S; w++) v += red[w][rl];
    if (a.swiglu)
        for (unsigned w = S; w < 2 * S; w++) u += red[w][rl];
    const unsigned gtile = (j == 0 ? a.tile0[0] : j == 1 ? a.tile0[1] : j == 2 ? a.tile0[2] : a.tile0[3]) + tile;
    if (P > 1) {
        // the parts of a tile meet in the last workgroup to finish, which sums
        // them in part order (the same bits whichever finishes last) and
        // clears the tile's counter for the next launch.  The ordering is the
        // one a release/acquire pair at agent scope would give, without its
        // cache maintenance, which only non-atomic data needs:
        //  * the partial sums are agent-scope atomic stores, which gfx950
        //    issues with sc1 set: written through every XCD's L2 to the point
        //    of device coherence;
        //  * s_waitcnt vmcnt(0) waits until those stores are acknowledged
        //    there (stores count in vmcnt on gfx9) before the counter's atomic
        //    add issues; the compiler fences on both sides keep the compiler
        //    from moving a store or the add across the wait;
        //  * the partial loads issue only once the add has returned: they are
        //    under a branch on its result (waited for with vmcnt(0) and read
        //    with v_readfirstlane/readlane), the compiler does not speculate
        //    atomic loads above a branch, and the GPU does not speculate;
        //  * they are agent-scope atomic loads (sc1), which read the point of
        //    coherence, not a stale L1 or L2 line, so no cache invalidate is
        //    needed before them.
        // A release fence would add buffer_wbl2 (write back the XCD's whole
        // L2) and an acquire fence buffer_inv sc1 (drop the planes every
        // workgroup of the XCD reads from it): measured at 87 against 14.6 µs
        // a launch.  The emitted order (global_store ... sc1, s_waitcnt
        // vmcnt(0), global_atomic_add ... sc0, s_waitcnt vmcnt(0), the branch,
        // global_load ... sc1) is checked in this file's gfx950 assembly by
        // tests/test_merge_order.py.
        float *pp = a.partials + ((size_t)gtile * kMaxParts + part) * 32;
        if (mine) {
            __hip_atomic_store(pp + lane, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + 16 + lane, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(&a.counters[gtile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0, 64);
        if (old != P - 1) return;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        v = 0.0f;
        u = 0.0f;
        const float *tp = a.partials + (size_t)gtile * kMaxParts * 32;
        for (unsigned q = 0; q < P; q++) {
            v += __hip_atomic_load(tp + q * 32 + rl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            u += __hip_atomic_load(tp + q * 32 + 16 + rl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lane == 0) __hip_atomic_store(&a.counters[gtile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (a.rms_ss) {
        // the RMS norm of the producer's x, from its per-group sums of squares
        // (in group order, so every workgroup scales by the same bits)
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < kRmsLoads; k++)
            if ((unsigned)lane + 64u * k < ng) t += ssv[k];
        for (unsigned g = (unsigned)lane + 64u * kRmsLoads; g < ng; g += 64) t += a.rms_ss[g];
        t = group_sum<64>(t);
        const float sc = 1.0f / sqrtf(t / (float)cols + a.eps);
        v *= sc;
        u *= sc;
    }
    if (!mine) return;
    if (a.swiglu) v = v * sigmoidf_(v) * u;  // silu(gate) · up (gpu/cpu.rs:238-242)
    const unsigned row = orow;
    const bool valid = row < orows;
    if (valid) {
        v += old_out;
        obase[row] = v;
    }
    if (a.emit.q && j == 0) {
        // this tile's rows are one group of 16 of the next product's input
        float e = valid ? v : 0.0f;
        if (a.emit_norm) {
            const float sq = group_sum<16>(e * e);
            if (lane == 0) a.emit.ss[tile] = sq;
            e = valid ? e * next_w : 0.0f;
            if (a.emit_xw && valid) a.emit_xw[row] = e;
        }
        planes::write16(a.emit, row, e);
    }
}

// Blocks per wave, waves per matrix in a workgroup and workgroups per tile
// (measured on MI355X): 5 blocks a wave when the launch has 512 tiles or
// more, else 3 (more, lighter waves for the smaller matrices); a tile's waves
// split over P workgroups only as far as keeps a workgroup to 8 waves per
// matrix, since the meeting of the parts costs about a microsecond.
struct Plan {
    int K;
    unsigned S, P;
};

Plan plan(unsigned nb, unsigned tiles, bool swiglu) {
    Plan p{tiles >= 512 ? 5 : 3, 0, 1};
    if ((unsigned)p.K > nb) p.K = (int)nb;
    const unsigned ranges = (nb + p.K - 1) / p.K;
    while ((ranges + p.P - 1) / p.P > 8 && p.P < (unsigned)kMaxParts) p.P++;
    // a large SwiGLU pair: its 8-wave workgroups (2 a CU resident) would
    // run in 2.1 rounds; halves of tiles in 4-wave workgroups (5 a CU) make
    // 1.7 and lose less to the last round than the meeting costs
    // (17408x5120: 27.8 -> 26.4 us alone, 53 us a token in the 27B decode)
    if (swiglu && tiles >= 512 && ranges >= 4 && p.P == 1) p.P = 2;
    p.S = (ranges + p.P - 1) / p.P;
    return p;
}

template <int K>
hipError_t go(dwim_dev *dev, const Args &a, unsigned grid, unsigned waves) {
    const size_t lds = (size_t)waves * Lds<K>::kChunks * 16;
    // past 64 KB (up to 16 waves) the launch needs the attribute, raised once
    // a process (a function-local static is initialized once even when host
    // threads reach it together)
    static const hipError_t raised = hipFuncSetAttribute(
        (const void *)k_mv_q4k_mfma<K>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(16 * Lds<K>::kChunks * 16));
    if (raised != hipSuccess) return raised;
    k_mv_q4k_mfma<K><<<grid, waves * 64, lds, dev->stream>>>(a);
    return hipGetLastError();
}

hipError_t run(dwim_dev *dev, Args a, unsigned njobs, const size_t *rows) {
    unsigned tiles = 0;
    for (unsigned j = 0; j < njobs; j++) tiles += (unsigned)q4kt::tiles(rows[j]);
    const Plan pl = plan(a.nb, tiles, a.swiglu != 0);
    a.S = pl.S;
    a.P = pl.P;
    if (a.P > 1 && tiles > dev->mv_tiles_cap) a.P = 1, a.S = (a.nb + pl.K - 1) / pl.K;
    const unsigned waves = a.S * (a.swiglu ? 2 : 1);
    if (waves > 16) return hipErrorInvalidValue;
    unsigned total = 0, t0 = 0;
    for (unsigned j = 0; j < kMaxJobs; j++) {
        a.first[j] = j < njobs ? total : 0xffffffffu;
        a.tile0[j] = t0;
        if (j < njobs) {
            const unsigned t = (unsigned)q4kt::tiles(rows[j]);
            total += t * a.P;
            t0 += t;
        }
    }
    a.first[0] = 0;
    a.partials = dev->mv_partials;
    a.counters = dev->mv_counters;
    a.bf_groups = a.bf_w ? (a.bf_rows + waves - 1) / waves : 0u;
    total += a.bf_groups;
    switch (pl.K) {
        case 1: return go<1>(dev, a, total, waves);
        case 2: return go<2>(dev, a, total, waves);
        case 3: return go<3>(dev, a, total, waves);
        case 4: return go<4>(dev, a, total, waves);
        case 5: return go<5>(dev, a, total, waves);
        default: return go<6>(dev, a, total, waves);
    }
}

}  // namespace

size_t planes_scratch_bytes() { return (kBatchArea2 + kMaxTok) * planes::kAreaBytes; }

planes::View planes_area(dwim_dev *dev, int area, size_t cols) {
    return planes::view((int8_t *)dev->planes + area * planes::kAreaBytes, cols);
}

hipError_t launch_planes(dwim_dev *dev, const float *x, size_t cols, const float *norm, float eps, float *xn_out,
                         int area, int handover) {
    if (cols > planes::kMaxCols || cols % 256 || area < 0 || area >= kBatchArea) return hipErrorInvalidValue;
    dev->prepared = 0;
    const unsigned blocks = (unsigned)((cols / 4 + kPlanesThreads - 1) / kPlanesThreads);
    k_planes<<<blocks, kPlanesThreads, 0, dev->stream>>>(x, norm, eps, handover, xn_out, planes_area(dev, area, cols));
    return hipGetLastError();
}

hipError_t launch_planes_batch(dwim_dev *dev, const float *x, size_t cols, size_t nt, int pair, planes::View *views) {
    if (cols > planes::kMaxCols || cols % 256 || nt < 1 || nt > (size_t)kMaxTok) return hipErrorInvalidValue;
    dev->prepared = 0;
    const unsigned blocks = (unsigned)((cols / 4 + kPlanesThreads - 1) / kPlanesThreads);
    k_planes<<<dim3(blocks, (unsigned)nt), kPlanesThreads, 0, dev->stream>>>(x, nullptr, 0.0f, 0, nullptr,
                                                                             planes_area(dev, kBatchArea, cols), pair);
    for (size_t t = 0; t < nt; t++) views[t] = planes_area(dev, kBatchArea + (int)t, cols);
    return hipGetLastError();
}

hipError_t launch_mv_q4k_mfma(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, const int *adds,
                              int count, int swiglu, int area, const MvExtra *extra) {
    if (count < 1 || count > kMaxJobs || (swiglu && count != 2)) return hipErrorInvalidValue;
    const size_t cols = ws[0]->cols;
    if (cols > planes::kMaxCols || cols % 256) return hipErrorInvalidValue;
    Args a{};
    a.nb = (unsigned)(cols / 256);
    const planes::View in = planes_area(dev, area, cols);
    a.xq = in.q;
    a.xstat = (const float4 *)in.stat;
    size_t rows[kMaxJobs];
    for (int j = 0; j < count; j++) {
        if (ws[j]->cols != cols || ws[j]->fmt != DWIM_Q4_K || ws[j]->rows >= (1u << 31)) return hipErrorInvalidValue;
        a.w[j] = (const uint8_t *)ws[j]->q;
        a.out[j] = outs[j];
        a.rows[j] = (unsigned)ws[j]->rows;
        rows[j] = ws[j]->rows;
        if (adds && adds[j]) a.add_mask |= 1u << j;
    }
    if (swiglu && ws[0]->rows != ws[1]->rows) return hipErrorInvalidValue;
    a.swiglu = swiglu;
    if (extra) {
        if (extra->bf16) {
            const dwim_weight *b = extra->bf16;
            if (b->fmt != DWIM_BF16 || b->cols % 8 || !extra->bf16_x || !extra->bf16_out) return hipErrorInvalidValue;
            a.bf_w = (const uint16_t *)b->q;
            a.bf_x = extra->bf16_x;
            a.bf_out = extra->bf16_out;
            a.bf_rows = (unsigned)b->rows;
            a.bf_cols = (unsigned)b->cols;
        }
        if (extra->head_ss) {
            if (extra->head_dim % 64 || cols % extra->head_dim) return hipErrorInvalidValue;
            a.head_ss = (const float4 *)extra->head_ss;
            a.head_dim = (unsigned)extra->head_dim;
            a.head_eps = extra->head_eps;
        }
        if (extra->rms) {
            a.rms_ss = in.ss;
            a.eps = extra->eps;
        }
        if (extra->emit_area >= 0) {
            // the next product's input: whole 256-blocks, in the other area
            if (extra->emit_area == area || ws[0]->rows % 256 || ws[0]->rows > planes::kMaxCols) return hipErrorInvalidValue;
            if (!swiglu && count != 1) return hipErrorInvalidValue;
            a.emit = planes_area(dev, extra->emit_area, ws[0]->rows);
            a.emit_norm = extra->emit_norm;
            a.emit_xw = extra->emit_xw;
            if (extra->emit_area == 0) dev->prepared = 0;  // (dwim_prepare's planes are area 0's)
        }
    }
    // a swiglu workgroup takes gate's tile and reads up's beside it
    return run(dev, a, swiglu ? 1 : (unsigned)count, rows);
}

hipError_t launch_mv_q4k_mfma_tokens(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, const int *adds,
                                     int count, int swiglu, const float *x, size_t n, const float *norm, float eps,
                                     float *xn_out, const float *gate_z, const StreamExtra *se) {
    if (count < 1 || count > kMaxJobs || (swiglu && count != 2) || n < 1) return hipErrorInvalidValue;
    if (se) {
        // one launch of 2..4 tokens, its planes handed over (in_area) or made
        // here into the first batch set, its results' planes handed on
        const int in = se->in_area >= 0 ? se->in_area : kBatchArea;
        if (n < 2 || n > (size_t)kMaxTok || (in != kBatchArea && in != kBatchArea2) || (se->rms && se->in_area < 0) ||
            (se->emit_area >= 0 && se->emit_area != kBatchArea && se->emit_area != kBatchArea2) ||
            se->emit_area == in)
            return hipErrorInvalidValue;
        const size_t cols = ws[0]->cols;
        if (cols > planes::kMaxCols || cols % 256) return hipErrorInvalidValue;
        for (int j = 0; j < count; j++)
            if (ws[j]->cols != cols || ws[j]->fmt != DWIM_Q4_K || ws[j]->rows >= (1u << 31)) return hipErrorInvalidValue;
        if (swiglu && ws[0]->rows != ws[1]->rows) return hipErrorInvalidValue;
        dev->prepared = 0;
        if (se->in_area < 0) {
            if (!x || (gate_z && (!norm || cols % 128))) return hipErrorInvalidValue;
            const unsigned blocks = (unsigned)((cols / 4 + kPlanesThreads - 1) / kPlanesThreads);
            if (gate_z)
                k_planes_gated<<<dim3(blocks, (unsigned)n), kPlanesThreads, 0, dev->stream>>>(
                    gate_z, x, norm, eps, planes_area(dev, kBatchArea, cols));
            else
                k_planes<<<dim3(blocks, (unsigned)n), kPlanesThreads, 0, dev->stream>>>(
                    x, norm, eps, 0, norm ? xn_out : nullptr, planes_area(dev, kBatchArea, cols), 1);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        const int8_t *xq[kMaxTok];
        const float *xs[kMaxTok];
        for (size_t t = 0; t < n; t++) {
            const planes::View v = planes_area(dev, in + (int)t, cols);
            xq[t] = v.q;
            xs[t] = v.stat;
        }
        return run_mv_stream(dev, ws, outs, adds, count, swiglu, n, xq, xs, se);
    }
    const size_t cols = ws[0]->cols;
    if (cols > planes::kMaxCols || cols % 256) return hipErrorInvalidValue;
    size_t rows[kMaxJobs];
    for (int j = 0; j < count; j++) {
        if (ws[j]->cols != cols || ws[j]->fmt != DWIM_Q4_K || ws[j]->rows >= (1u << 31)) return hipErrorInvalidValue;
        rows[j] = ws[j]->rows;
    }
    if (swiglu && ws[0]->rows != ws[1]->rows) return hipErrorInvalidValue;
    if (gate_z && (!norm || cols % 128)) return hipErrorInvalidValue;
    dev->prepared = 0;
    const unsigned njobs = swiglu ? 1 : (unsigned)count;
    const unsigned blocks = (unsigned)((cols / 4 + kPlanesThreads - 1) / kPlanesThreads);
    // runs of up to kMaxTok tokens, as even as they come (7 = 4 + 3)
    const size_t runs = (n + kMaxTok - 1) / kMaxTok;
    for (size_t r = 0, t0 = 0; r < runs; r++) {
        const size_t nt = (n - t0) / (runs - r);
        if (gate_z)
            k_planes_gated<<<dim3(blocks, (unsigned)nt), kPlanesThreads, 0, dev->stream>>>(
                gate_z + t0 * cols, x + t0 * cols, norm, eps, planes_area(dev, kBatchArea, cols));
        else
            k_planes<<<dim3(blocks, (unsigned)nt), kPlanesThreads, 0, dev->stream>>>(
                x + t0 * cols, norm, eps, 0, norm && xn_out ? xn_out + t0 * cols : nullptr,
                planes_area(dev, kBatchArea, cols), 1);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (nt == 1) {
            Args a{};
            a.nb = (unsigned)(cols / 256);
            const planes::View in = planes_area(dev, kBatchArea, cols);
            a.xq = in.q;
            a.xstat = (const float4 *)in.stat;
            for (int j = 0; j < count; j++) {
                a.w[j] = (const uint8_t *)ws[j]->q;
                a.out[j] = outs[j] ? outs[j] + t0 * rows[j] : nullptr;
                a.rows[j] = (unsigned)rows[j];
                if (adds && adds[j]) a.add_mask |= 1u << j;
            }
            a.swiglu = swiglu;
            e = run(dev, a, njobs, rows);
        } else {
            const int8_t *xq[kMaxTok];
            const float *xs[kMaxTok];
            float *o[kMaxJobs];
            for (size_t t = 0; t < nt; t++) {
                const planes::View v = planes_area(dev, kBatchArea + (int)t, cols);
                xq[t] = v.q;
                xs[t] = v.stat;
            }
            for (int j = 0; j < count; j++) o[j] = outs[j] ? outs[j] + t0 * rows[j] : nullptr;
            e = run_mv_stream(dev, ws, o, adds, count, swiglu, nt, xq, xs);
        }
        if (e != hipSuccess) return e;
        t0 += nt;
    }
    return hipSuccess;
}
