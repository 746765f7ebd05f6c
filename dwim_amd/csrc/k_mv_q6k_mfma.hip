// Q6_K matrix-vector products for one token on the int8 matrix cores (the
// output head of the 27B shape: 248320 × 5120), at f32 accuracy (dwim
// gpu/cpu.rs:110-149; the Q6_K bits are ggml's block_q6_K as
// inference/quants.rs:235-275 unpacks them).
//
// A Q6_K weight is d·sc_g·(q − 32): per 256-block an f16 d, per 16 weights an
// int8 scale sc_g, per weight 6 bits q (the low 4 in ql, the high 2 in qh).
// The activations come as int8 planes (planes.h, groups of 16), so a group of
// 16 weights meets one activation group: v_mfma_i32_16x16x64_i8 takes 16 rows
// × 64 weights as A (the 6-bit q, 0..63, exact in int8), and B's column
// 3g' + p holds digit p of activation group g', nonzero only in k-group g' —
// the layout of the Q4_K kernel (k_mv_q4k_mfma.hip), with groups of 16 in place
// of sub-block halves.  Each column's int32 sum is scaled in f32 by
// d·sc·s_x; the −32 is folded into the activations' group sums:
// Σ(q − 32)x = Σqx − 32·Σx.
//
// The weights stay in the planes the upload writes (ql, qh, sc, d row-major
// per block; runtime.h).  In half n of a block, qh byte l holds the high bits
// of weights l, l + 32, l + 64 and l + 96 (of the half), whose low bits are
// the low and high nibbles of ql bytes l and l + 32.  So lane (k-group kq, row
// c) takes l = 16·(kq % 2)..+15 of half kq / 2: 16 bytes of qh and two 16-byte
// runs of ql give it four groups of 16 weights, groups 8n + kq % 2 + 2u for
// u = 0..3 (the lanes' bytes are disjoint: 48 bytes each, the block's 768
// once).  A wave takes up to K blocks of a 16-row tile and issues every load
// before any compute; the planes are staged in LDS as in the Q4_K kernel.
#include "device_util.h"
#include "planes.h"
#include "quant_math.h"
#include "runtime.h"

typedef int v4i6 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kK = 5;  // blocks a wave (at most)

struct Q6Args {
    const uint8_t *ql, *qh;
    const int8_t *sc;
    const uint16_t *d;
    float *out;
    unsigned rows, nb, S;
    const int8_t *xq;       // planes [3][cols]
    const float4 *xstat;    // [cols/64][2]: four groups' scales, then their sums
};

// Per wave LDS, in 16-byte chunks: the planes of its K blocks (chunk
// 48i + 16p + c: activations 16c..16c+15 of digit p of block i), the group
// statistics (chunks 8i + 2k, + 1: scales and sums of groups 4k..4k+3), eight
// zero chunks (the B operands of the lanes outside B's blocks, at the same
// offsets 2u as the others) and the decoded scales ([group][row] floats).
struct Lds6 {
    static constexpr int kPlaneLoads = (kK * 48 + 63) / 64;
    static constexpr int kStat = kK * 48;
    static constexpr int kZero = kStat + 64;
    static constexpr int kHdr = kZero + 8;
    static constexpr int kChunks = kHdr + 16 * 16 / 4;
    static_assert(kPlaneLoads * 64 <= kZero, "spare plane chunks must land in the statistics area");
};

__global__ void __launch_bounds__(512) k_mv_q6k_mfma(const Q6Args a) {
    using L = Lds6;
    extern __shared__ uint4 lds_all[];
    __shared__ float red[8][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kq = lane >> 4, c = lane & 15;
    const unsigned S = a.S, nb = a.nb, tile = blockIdx.x;
    const unsigned b0 = wave * nb / S, b1 = (wave + 1) * nb / S;
    const int nblk = (int)(b1 - b0);
    uint4 *my = lds_all + wave * L::kChunks;
    float *hdr = (float *)(my + L::kHdr);
    const unsigned cols = nb * 256;

    // the planes and statistics of the wave's blocks, then the weights
    uint4 xc[L::kPlaneLoads];
#pragma unroll
    for (int u = 0; u < L::kPlaneLoads; u++) {
        const int ci = lane + 64 * u < nblk * 48 ? lane + 64 * u : 0;
        const unsigned i = (unsigned)ci / 48u, p = ((unsigned)ci % 48u) / 16u, part16 = (unsigned)ci % 16u;
        xc[u] = *(const uint4 *)(a.xq + p * cols + (b0 + i) * 256u + 16u * part16);
    }
    const float4 st = a.xstat[b0 * 8u + (lane < nblk * 8 ? (unsigned)lane : 0u)];
    // lane (kq, c): row c of the tile, bytes l = 16·(kq % 2).. of half kq / 2
    const unsigned row = tile * 16 + (unsigned)c, row_c = row < a.rows ? row : a.rows - 1;
    const unsigned n = (unsigned)kq >> 1, lb = 16u * ((unsigned)kq & 1u);
    uint4 ql[kK][2], qh[kK];
    // header lane (k4, R4): row R4, groups 4k4..4k4+3: their scales, and d
    const int k4 = lane & 3, R4 = lane >> 2;
    const unsigned hrow = tile * 16 + (unsigned)R4, hrow_c = hrow < a.rows ? hrow : a.rows - 1;
    uint32_t scw[kK];
    uint16_t dw[kK];
#pragma unroll
    for (int i = 0; i < kK; i++) {
        const unsigned b = b0 + (unsigned)(i < nblk ? i : 0);
        const size_t blk = (size_t)row_c * nb + b;
        ql[i][0] = *(const uint4 *)(a.ql + blk * 128 + 64 * n + lb);
        ql[i][1] = *(const uint4 *)(a.ql + blk * 128 + 64 * n + 32 + lb);
        qh[i] = *(const uint4 *)(a.qh + blk * 64 + 32 * n + lb);
        const size_t hblk = (size_t)hrow_c * nb + b;
        scw[i] = *(const uint32_t *)(a.sc + hblk * 16 + 4 * k4);
        dw[i] = a.d[hblk];
    }
#pragma unroll
    for (int u = 0; u < L::kPlaneLoads; u++) my[lane + 64 * u] = xc[u];
    if (lane < 64) ((float4 *)(my + L::kStat))[lane] = st;
    if (lane < 8) my[L::kZero + lane] = make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");

    // B: lane (kq, c) carries digit c % 3 of group 8(kq / 2) + kq % 2 + 2u
    // when c / 3 == kq
    const bool active = c < 12 && c / 3 == kq;
    const int bsel = active ? 16 * (c % 3) + 8 * (kq >> 1) + (kq & 1) : 0;
    const int gcol = c < 12 ? c / 3 : 0;  // the column's k-group
    const int gbase = 8 * (gcol >> 1) + (gcol & 1);  // its groups: gbase + 2u
    const float4 *stl = (const float4 *)(my + L::kStat);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, macc = 0.0f;
#pragma unroll
    for (int i = 0; i < kK; i++) {
        if (i >= nblk) break;
        {
            // lane (k4, R4) decodes row R4's groups 4k4..4k4+3: d·sc times the
            // group's activation scale, and the −32 term −32·d·sc·Σx
            const float d = dq::from_f16(dw[i]);
            const float4 xs = stl[8 * i + 2 * k4], xm = stl[8 * i + 2 * k4 + 1];
            const float s0 = d * (float)(int8_t)(scw[i] & 0xffu), s1 = d * (float)(int8_t)((scw[i] >> 8) & 0xffu);
            const float s2 = d * (float)(int8_t)((scw[i] >> 16) & 0xffu), s3 = d * (float)(int8_t)(scw[i] >> 24);
            macc -= 32.0f * ((s0 * xm.x + s1 * xm.y) + (s2 * xm.z + s3 * xm.w));
            hdr[(4 * k4) * 16 + R4] = s0 * xs.x;
            hdr[(4 * k4 + 1) * 16 + R4] = s1 * xs.y;
            hdr[(4 * k4 + 2) * 16 + R4] = s2 * xs.z;
            hdr[(4 * k4 + 3) * 16 + R4] = s3 * xs.w;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const uint4 *xv = my + (active ? 48 * i + bsel : L::kZero);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            // weights l.. of run u (l, l + 32, l + 64, l + 96 of the half):
            // the low (u < 2) or high nibble of ql bytes l or l + 32, the bit
            // pair 2u of qh byte l
            const uint4 lo = ql[i][u & 1], hi = qh[i];
            const unsigned nsh = 4u * (unsigned)(u >> 1), hsh = 2u * (unsigned)u;
            const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w}, hw[4] = {hi.x, hi.y, hi.z, hi.w};
            v4i6 av;
#pragma unroll
            for (int w = 0; w < 4; w++)
                av[w] = (int)(((lw[w] >> nsh) & 0x0f0f0f0fu) | (((hw[w] >> hsh) & 0x03030303u) << 4));
            const uint4 xq = xv[2 * u];
            const v4i6 bv = {(int)xq.x, (int)xq.y, (int)xq.z, (int)xq.w};
            const v4i6 C = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, v4i6{0, 0, 0, 0}, 0, 0, 0);
            const float4 D = *(const float4 *)&hdr[(gbase + 2 * u) * 16 + 4 * kq];
            acc[0] += D.x * (float)C[0];
            acc[1] += D.y * (float)C[1];
            acc[2] += D.z * (float)C[2];
            acc[3] += D.w * (float)C[3];
        }
        __builtin_amdgcn_wave_barrier();
    }
    // the columns meet, weighted by their digit: lanes 16kq..16kq+15 hold
    // rows 4kq..4kq+3; the −32 terms of row R sit in lanes 4R..4R+3
    const float f = c < 12 ? (c % 3 == 0 ? 1.0f : c % 3 == 1 ? 256.0f : 65536.0f) : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = group_sum<16>(acc[e] * f);
    macc = group_sum<4>(macc);
    const float mrow = __shfl(macc, 16 * kq + 4 * (c & 3), 64);
    if (c < 4) red[wave][4 * kq + c] = (c == 0 ? acc[0] : c == 1 ? acc[1] : c == 2 ? acc[2] : acc[3]) + mrow;
    __syncthreads();
    if (wave != 0 || lane >= 16) return;
    float v = 0.0f;
    for (unsigned w = 0; w < S; w++) v += red[w][lane];
    const unsigned r = tile * 16 + (unsigned)lane;
    if (r < a.rows) a.out[r] = v;
}

// ---------------------------------------------------------------- tokens
// Two to four tokens at once (a verify batch through the head), the weights
// read once for all of them.  B's columns are (k-group g, token t), column
// 4g + t, nonzero only in k-group g, so every column is used, and each digit
// of the planes takes one MFMA: B lane (kq, c) carries digit p of token c % 4's
// activations of group G(kq, u) = 8(kq / 2) + kq % 2 + 2u when c / 4 == kq.
// A column's three int32 sums combine in f32 (C0 + 256·C1 + 65536·C2), are
// scaled by the token's activation scale of the column's group and by the
// row's d·sc, and the four k-groups of a token meet by row rotations.  The
// weight loads are the one-token kernel's, every one issued before any
// compute, after the copies of the planes (below).
constexpr int kMaxTok6 = 4;

struct Q6TArgs {
    const uint8_t *ql, *qh;
    const int8_t *sc;
    const uint16_t *d;
    float *out;              // [NT][rows]
    unsigned rows, nb, S;
    unsigned tw;                    // tiles a workgroup
    const int8_t *xq[kMaxTok6];     // each token's planes [3][cols] (groups of 16)
    const float4 *xstat[kMaxTok6];  // [cols/64][2]
};

// A workgroup takes tw tiles (2 when S ≤ 4) of S waves each; wave w takes
// range w % S of the blocks of tile w / S, and the tw waves of a range share
// its planes, copied straight from global memory into LDS (global_load_lds,
// no registers).  That halves the LDS and drops the staging registers of a
// wave, so that twice as many waves stream weights at once (2 workgroups of
// 8 waves a CU at the 27B head's 20 blocks a row, against 8 waves of 4).
//
// LDS, in 16-byte chunks: per range, its planes [block][digit][group][token]
// (so that the 16 B lanes of an MFMA read 16 distinct chunks), then its
// statistics [block][token][8] (chunks 2k, 2k + 1: scales and sums of groups
// 4k..4k+3); per wave, the decoded d·sc ([group][row] floats), then a zero
// chunk.
template <int NT>
struct Lds6T {
    static constexpr int kPlaneChunks = kK * 48 * NT;
    static constexpr int kStatChunks = kK * 8 * NT;
    static constexpr int kRange = kPlaneChunks + kStatChunks;
    static constexpr int kHdrFloats = 16 * 16;
    static constexpr int kWave = kHdrFloats / 4 + 1;
    static_assert(kHdrFloats >= 2 * NT * 16, "the sums of a wave fit its header area");
    static constexpr size_t bytes(unsigned S, unsigned tw) { return ((size_t)S * kRange + (size_t)tw * S * kWave) * 16; }
};

// the group of 16 a k-group x of an MFMA takes in run u (the lanes' layout above)
DEV int q6_group(int x, int u) { return 8 * (x >> 1) + (x & 1) + 2 * u; }

template <int NT>
__global__ void __launch_bounds__(512) k_mv_q6k_tokens(const Q6TArgs a) {
    using L = Lds6T<NT>;
    extern __shared__ uint4 lds_all[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kq = lane >> 4, c = lane & 15;
    const unsigned S = a.S, nb = a.nb, tw = a.tw;
    const unsigned rg = (unsigned)wave % S, sub = (unsigned)wave / S, tile = blockIdx.x * tw + sub;
    const unsigned b0 = rg * nb / S, b1 = (rg + 1) * nb / S;
    const int nblk = (int)(b1 - b0);
    uint4 *range = lds_all + rg * L::kRange;
    uint4 *mine = lds_all + S * L::kRange + wave * L::kWave;
    float *hdr = (float *)mine;
    const uint4 *zero = mine + L::kHdrFloats / 4;
    const unsigned cols = nb * 256;

    // the range's planes and statistics, its copies split over the tw waves
    // that share them (lane l of copy u writes chunk 64u + l)
    {
        const int np = nblk * 48 * NT, ns = nblk * 8 * NT;
        for (int u = (int)sub; 64 * u < np; u += (int)tw) {
            const int d = 64 * u + lane;
            if (d < np) {
                const int t = d % NT, g = (d / NT) % 16, p = (d / (NT * 16)) % 3, i = d / (NT * 48);
                const int8_t *src = t == 0 ? a.xq[0] : t == 1 ? a.xq[1] : t == 2 ? a.xq[2] : a.xq[3];
                lds_copy16((const uint8_t *)(src + p * cols + (b0 + i) * 256u + 16u * g), (uint8_t *)(range + 64 * u));
            }
        }
        for (int u = (int)sub; 64 * u < ns; u += (int)tw) {
            const int d = 64 * u + lane;
            if (d < ns) {
                const int j = d % 8, t = (d / 8) % NT, i = d / (8 * NT);
                const float4 *src = t == 0 ? a.xstat[0] : t == 1 ? a.xstat[1] : t == 2 ? a.xstat[2] : a.xstat[3];
                lds_copy16((const uint8_t *)&src[(b0 + i) * 8u + j], (uint8_t *)(range + L::kPlaneChunks + 64 * u));
            }
        }
    }
    const unsigned row = tile * 16 + (unsigned)c, row_c = row < a.rows ? row : a.rows - 1;
    const unsigned n = (unsigned)kq >> 1, lb = 16u * ((unsigned)kq & 1u);
    const int k4 = lane & 3, R4 = lane >> 2;
    const unsigned hrow = tile * 16 + (unsigned)R4, hrow_c = hrow < a.rows ? hrow : a.rows - 1;
    uint4 ql[kK][2], qh[kK];
    uint32_t scw[kK];
    uint16_t dw[kK];
#pragma unroll
    for (int i = 0; i < kK; i++) {
        const unsigned b = b0 + (unsigned)(i < nblk ? i : 0);
        const size_t blk = (size_t)row_c * nb + b;
        ql[i][0] = *(const uint4 *)(a.ql + blk * 128 + 64 * n + lb);
        ql[i][1] = *(const uint4 *)(a.ql + blk * 128 + 64 * n + 32 + lb);
        qh[i] = *(const uint4 *)(a.qh + blk * 64 + 32 * n + lb);
        const size_t hblk = (size_t)hrow_c * nb + b;
        scw[i] = *(const uint32_t *)(a.sc + hblk * 16 + 4 * k4);
        dw[i] = a.d[hblk];
    }
    if (lane == 0) mine[L::kHdrFloats / 4] = make_uint4(0, 0, 0, 0);
    // the copies land in LDS when the wave's loads are done; then every
    // wave's are
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // B lane (kq, c): token c % 4 of k-group kq when c / 4 == kq; output
    // lane (kq, c): rows 4kq.., column group gq = c / 4, token tc = c % 4
    const int tb = c & 3, gq = c >> 2;
    const bool active = gq == kq && tb < NT;
    const float *stf = (const float *)(range + L::kPlaneChunks);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, macc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) macc[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < kK; i++) {
        if (i >= nblk) break;
        {
            // lane (k4, R4): d·sc of row R4's groups 4k4..4k4+3, and each
            // token's −32 term −32·Σ d·sc·Σx
            const float d = dq::from_f16(dw[i]);
            const float s0 = d * (float)(int8_t)(scw[i] & 0xffu), s1 = d * (float)(int8_t)((scw[i] >> 8) & 0xffu);
            const float s2 = d * (float)(int8_t)((scw[i] >> 16) & 0xffu), s3 = d * (float)(int8_t)(scw[i] >> 24);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float4 xm = *(const float4 *)&stf[((i * NT + t) * 8 + 2 * k4 + 1) * 4];
                macc[t] -= 32.0f * ((s0 * xm.x + s1 * xm.y) + (s2 * xm.z + s3 * xm.w));
            }
            hdr[(4 * k4) * 16 + R4] = s0;
            hdr[(4 * k4 + 1) * 16 + R4] = s1;
            hdr[(4 * k4 + 2) * 16 + R4] = s2;
            hdr[(4 * k4 + 3) * 16 + R4] = s3;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint4 lo = ql[i][u & 1], hi = qh[i];
            const unsigned nsh = 4u * (unsigned)(u >> 1), hsh = 2u * (unsigned)u;
            const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w}, hw[4] = {hi.x, hi.y, hi.z, hi.w};
            v4i6 av;
#pragma unroll
            for (int w = 0; w < 4; w++)
                av[w] = (int)(((lw[w] >> nsh) & 0x0f0f0f0fu) | (((hw[w] >> hsh) & 0x03030303u) << 4));
            const int gb = q6_group(kq, u), go = q6_group(gq, u);
            v4i6 C[3];
#pragma unroll
            for (int p = 0; p < 3; p++) {
                const uint4 xq = *(active ? range + ((i * 3 + p) * 16 + gb) * NT + tb : zero);
                const v4i6 bv = {(int)xq.x, (int)xq.y, (int)xq.z, (int)xq.w};
                C[p] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, v4i6{0, 0, 0, 0}, 0, 0, 0);
            }
            // the column's activation scale (zero for the columns past NT)
            const float sx = tb < NT ? stf[((i * NT + tb) * 8 + 2 * (go >> 2)) * 4 + (go & 3)] : 0.0f;
            const float4 D = *(const float4 *)&hdr[go * 16 + 4 * kq];
            const float Dv[4] = {D.x, D.y, D.z, D.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                acc[e] += Dv[e] * (sx * (((float)C[0][e] + 256.0f * (float)C[1][e]) + 65536.0f * (float)C[2][e]));
        }
        __builtin_amdgcn_wave_barrier();
    }
    // a token's four column groups meet (lanes c, c ± 4, c ± 8 of a row);
    // then lane (kq, t < NT) holds token t's rows 4kq..4kq+3
#pragma unroll
    for (int e = 0; e < 4; e++) {
        acc[e] += xlane::mov<0x124>(acc[e]);
        acc[e] += xlane::mov<0x128>(acc[e]);
    }
    // each wave's sums go to its header area ([token][row], then the −32
    // terms [token][row]), done with
    float *red = hdr;
    if (c < NT)
#pragma unroll
        for (int e = 0; e < 4; e++) red[c * 16 + 4 * kq + e] = acc[e];
#pragma unroll
    for (int t = 0; t < NT; t++) macc[t] = group_sum<4>(macc[t]);
    if (k4 == 0)
#pragma unroll
        for (int t = 0; t < NT; t++) red[(NT + t) * 16 + R4] = macc[t];
    __syncthreads();
    if (rg != 0 || lane >= 16 * NT) return;
    const int t = lane >> 4, rl = lane & 15;
    float v = 0.0f;
    for (unsigned w = 0; w < S; w++) {
        const float *rw = (const float *)(lds_all + S * L::kRange + (sub * S + w) * L::kWave);
        v += rw[t * 16 + rl] + rw[(NT + t) * 16 + rl];
    }
    const unsigned r = tile * 16 + (unsigned)rl;
    if (r < a.rows) a.out[(size_t)t * a.rows + r] = v;
}

template <int NT>
hipError_t go_tokens(dwim_dev *dev, Q6TArgs a, unsigned tiles) {
    using L = Lds6T<NT>;
    a.tw = a.S <= 4 ? 2 : 1;
    // the attribute holds for the process, raised once to the most a launch
    // takes (a function-local static is initialized once even when host
    // threads reach it together)
    static const hipError_t raised =
        hipFuncSetAttribute((const void *)k_mv_q6k_tokens<NT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)std::max(L::bytes(8, 1), L::bytes(4, 2)));
    if (raised != hipSuccess) return raised;
    k_mv_q6k_tokens<NT><<<(tiles + a.tw - 1) / a.tw, a.tw * a.S * 64, L::bytes(a.S, a.tw), dev->stream>>>(a);
    return hipGetLastError();
}

Q6Args one_token_args(const dwim_weight *w, float *out, const planes::View &in) {
    Q6Args a{};
    a.ql = (const uint8_t *)w->q;
    a.qh = (const uint8_t *)w->s;
    a.sc = (const int8_t *)w->s2;
    a.d = (const uint16_t *)w->s3;
    a.out = out;
    a.rows = (unsigned)w->rows;
    a.nb = (unsigned)(w->cols / 256);
    a.S = (a.nb + kK - 1) / kK;
    a.xq = in.q;
    a.xstat = (const float4 *)in.stat;
    return a;
}

bool q6_shape_ok(const dwim_weight *w) {
    return w->fmt == DWIM_Q6_K && w->cols % 256 == 0 && w->cols <= planes::kMaxCols && w->rows < (1u << 31) &&
           (w->cols / 256 + kK - 1) / kK <= 8;
}

}  // namespace

hipError_t launch_mv_q6k_tokens(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n) {
    if (!q6_shape_ok(w) || n < 1) return hipErrorInvalidValue;
    const size_t cols = w->cols, rows = w->rows;
    const unsigned tiles = (unsigned)((rows + 15) / 16);
    // runs of up to four tokens, as even as they come (7 = 4 + 3)
    const size_t runs = (n + kMaxTok6 - 1) / kMaxTok6;
    for (size_t r = 0, t0 = 0; r < runs; r++) {
        const size_t nt = (n - t0) / (runs - r);
        planes::View v[kMaxTok6];
        hipError_t e = launch_planes_batch(dev, x + t0 * cols, cols, nt, 0, v);
        if (e != hipSuccess) return e;
        if (nt == 1) {
            const Q6Args a = one_token_args(w, out + t0 * rows, v[0]);
            k_mv_q6k_mfma<<<tiles, a.S * 64, (size_t)a.S * Lds6::kChunks * 16, dev->stream>>>(a);
            e = hipGetLastError();
        } else {
            Q6TArgs a{};
            a.ql = (const uint8_t *)w->q;
            a.qh = (const uint8_t *)w->s;
            a.sc = (const int8_t *)w->s2;
            a.d = (const uint16_t *)w->s3;
            a.out = out + t0 * rows;
            a.rows = (unsigned)rows;
            a.nb = (unsigned)(cols / 256);
            a.S = (a.nb + kK - 1) / kK;
            for (size_t t = 0; t < (size_t)kMaxTok6; t++) {
                const planes::View &vt = v[t < nt ? t : 0];
                a.xq[t] = vt.q;
                a.xstat[t] = (const float4 *)vt.stat;
            }
            e = nt == 2 ? go_tokens<2>(dev, a, tiles) : nt == 3 ? go_tokens<3>(dev, a, tiles) : go_tokens<4>(dev, a, tiles);
        }
        if (e != hipSuccess) return e;
        t0 += nt;
    }
    return hipSuccess;
}

hipError_t launch_mv_q6k_mfma(dwim_dev *dev, const dwim_weight *w, float *out, int area) {
    if (w->fmt != DWIM_Q6_K || w->cols % 256 || w->cols > planes::kMaxCols || w->rows >= (1u << 31))
        return hipErrorInvalidValue;
    Q6Args a{};
    a.ql = (const uint8_t *)w->q;
    a.qh = (const uint8_t *)w->s;
    a.sc = (const int8_t *)w->s2;
    a.d = (const uint16_t *)w->s3;
    a.out = out;
    a.rows = (unsigned)w->rows;
    a.nb = (unsigned)(w->cols / 256);
    a.S = (a.nb + kK - 1) / kK;
    if (a.S > 8) return hipErrorInvalidValue;
    const planes::View in = planes_area(dev, area, w->cols);
    a.xq = in.q;
    a.xstat = (const float4 *)in.stat;
    const unsigned tiles = (unsigned)((w->rows + 15) / 16);
    k_mv_q6k_mfma<<<tiles, a.S * 64, (size_t)a.S * Lds6::kChunks * 16, dev->stream>>>(a);
    return hipGetLastError();
}
