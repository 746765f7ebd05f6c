// Q4_K matrix products for batches of tokens (prefill and verify): out[t][r]
// (+)= w[r] · x[t] (dwim gpu/cpu.rs:110-149) on the f16 matrix cores, at
// close to f32 accuracy.
//
// A Q4_K weight is d·sc·q − dmin·m (per 256-block f16 d and dmin, per
// 32-sub-block 6-bit sc and m, 4-bit q).  So, per block and row,
//     w · x = d · Σ_k (sc·q)_k x_k − Σ_sb (dmin·m_sb) X_sb,   X_sb = Σ_{k∈sb} x_k,
// and sc·q (an integer up to 945) is exact in f16.  The activations are split
// in two f16 parts x = hi + lo (22 bits), so the first sum is two MFMA chains
// on exact products, summed in f32 over the whole block and then scaled by
// d.  The second is one more MFMA per block: its 32 k-slots hold the 8
// sub-blocks' dmin·m (as f16 hi and lo parts) against X_sb (hi and lo):
//     [hi, hi, lo, 0] · [X_hi, X_lo, X_hi, 0].
// 17 MFMAs per block and 16×16 tile, where splitting the weights too would
// take 24.  k_split writes the activations' parts and sums once per product.
//
// A workgroup of 8 waves computes a 256-row × 128-token tile, in steps of
// one quant group (64 weights), double-buffered in LDS, one barrier a step.
// Its waves have two roles, one of each on every SIMD, so that the matrix
// cores and the vector ALUs work at once: four matrix waves (a 128 × 64 part
// each, 8 × 4 MFMA tiles) multiply step s out of one buffer while four loader
// waves dequantize step s + 1's weights (loaded from global memory during step
// s − 1) into the other and issue the loads of step s + 2.  The activations
// of step s + 1 are copied into the other buffer by the matrix waves
// themselves, straight from global memory into LDS.  LDS rows are 128 bytes whose 16-byte chunks are XOR-swizzled by row,
// so that the 16 lanes reading one k-slice of 16 rows hit different banks.  Workgroups are numbered XCD-major: those on
// one XCD share its L2 and mostly one token tile.
#include "device_util.h"
#include "layout.h"
#include "quant_math.h"
#include "runtime.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef unsigned u4v __attribute__((ext_vector_type(4)));

namespace {

constexpr int kRows = 256, kToks = 128, kStep = 64;
constexpr int kThreads = 768;  // 8 matrix waves, 4 loader waves

// x [n][cols] f32 -> xh, xl [n][cols] f16 (hi and lo parts), and per
// (token, block) xm [n][nb][16] f16: the 8 sub-block sums' hi parts, then
// their lo parts.  A thread per float4, eight lanes per 32-value sub-block,
// so that a wave's loads and stores are contiguous; the sub-block's sum is
// an 8-lane DPP sum.
__global__ void k_split(const float *__restrict__ x, _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                        _Float16 *__restrict__ xm, size_t n, size_t cols) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index over [n][cols/4]
    if (i >= n * (cols / 4)) return;  // whole sub-blocks: cols is a multiple of 32
    const float4 v = ((const float4 *)x)[i];
    const _Float16 h0 = (_Float16)v.x, h1 = (_Float16)v.y, h2 = (_Float16)v.z, h3 = (_Float16)v.w;
    const _Float16 l0 = (_Float16)(v.x - (float)h0), l1 = (_Float16)(v.y - (float)h1);
    const _Float16 l2 = (_Float16)(v.z - (float)h2), l3 = (_Float16)(v.w - (float)h3);
    auto pk = [](_Float16 a, _Float16 b) {
        return (uint32_t)__builtin_bit_cast(uint16_t, a) | (uint32_t)__builtin_bit_cast(uint16_t, b) << 16;
    };
    ((uint2 *)xh)[i] = make_uint2(pk(h0, h1), pk(h2, h3));
    ((uint2 *)xl)[i] = make_uint2(pk(l0, l1), pk(l2, l3));
    const float s = group_sum<8>((v.x + v.y) + (v.z + v.w));
    if ((i & 7) == 0) {
        const size_t sbi = i / 8, t = sbi / (cols / 32), sb = sbi % (cols / 32), b = sb / 8, j = sb % 8;
        _Float16 *m = xm + (t * (cols / 256) + b) * 16;
        const _Float16 sh = (_Float16)s;
        m[j] = sh;
        m[8 + j] = (_Float16)(s - (float)sh);
    }
}

// k_split of silu(g)·u (gpu/cpu.rs:238-242, the SwiGLU's product computed
// here instead of in the up product's epilogue), the same bits as k_split of
// the product written out.
__global__ void k_split_swiglu(const float *__restrict__ g, const float *__restrict__ u, _Float16 *__restrict__ xh,
                               _Float16 *__restrict__ xl, _Float16 *__restrict__ xm, size_t n, size_t cols) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * (cols / 4)) return;
    const float4 a = ((const float4 *)g)[i], b = ((const float4 *)u)[i];
    const float4 v = make_float4(a.x * sigmoidf_(a.x) * b.x, a.y * sigmoidf_(a.y) * b.y, a.z * sigmoidf_(a.z) * b.z,
                                 a.w * sigmoidf_(a.w) * b.w);
    const _Float16 h0 = (_Float16)v.x, h1 = (_Float16)v.y, h2 = (_Float16)v.z, h3 = (_Float16)v.w;
    const _Float16 l0 = (_Float16)(v.x - (float)h0), l1 = (_Float16)(v.y - (float)h1);
    const _Float16 l2 = (_Float16)(v.z - (float)h2), l3 = (_Float16)(v.w - (float)h3);
    auto pk = [](_Float16 p, _Float16 q) {
        return (uint32_t)__builtin_bit_cast(uint16_t, p) | (uint32_t)__builtin_bit_cast(uint16_t, q) << 16;
    };
    ((uint2 *)xh)[i] = make_uint2(pk(h0, h1), pk(h2, h3));
    ((uint2 *)xl)[i] = make_uint2(pk(l0, l1), pk(l2, l3));
    const float sum = group_sum<8>((v.x + v.y) + (v.z + v.w));
    if ((i & 7) == 0) {
        const size_t sbi = i / 8, t = sbi / (cols / 32), sb = sbi % (cols / 32), bk = sb / 8, j = sb % 8;
        _Float16 *m = xm + (t * (cols / 256) + bk) * 16;
        const _Float16 sh = (_Float16)sum;
        m[j] = sh;
        m[8 + j] = (_Float16)(sum - (float)sh);
    }
}

// One float4 v of a row of the activations (float4 index i over [n][cols/4])
// into the split: its f16 hi and lo parts, and (eight consecutive lanes
// holding a 32-value sub-block) the sub-block's sum; every lane of the wave
// active.
DEV void split_put(float4 v, size_t i, size_t cols, _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                   _Float16 *__restrict__ xm) {
    const _Float16 h0 = (_Float16)v.x, h1 = (_Float16)v.y, h2 = (_Float16)v.z, h3 = (_Float16)v.w;
    const _Float16 l0 = (_Float16)(v.x - (float)h0), l1 = (_Float16)(v.y - (float)h1);
    const _Float16 l2 = (_Float16)(v.z - (float)h2), l3 = (_Float16)(v.w - (float)h3);
    auto pk = [](_Float16 a, _Float16 b) {
        return (uint32_t)__builtin_bit_cast(uint16_t, a) | (uint32_t)__builtin_bit_cast(uint16_t, b) << 16;
    };
    ((uint2 *)xh)[i] = make_uint2(pk(h0, h1), pk(h2, h3));
    ((uint2 *)xl)[i] = make_uint2(pk(l0, l1), pk(l2, l3));
    const float s = group_sum<8>((v.x + v.y) + (v.z + v.w));
    if ((i & 7) == 0) {
        const size_t sbi = i / 8, t = sbi / (cols / 32), sb = sbi % (cols / 32), b = sb / 8, j = sb % 8;
        _Float16 *m = xm + (t * (cols / 256) + b) * 16;
        const _Float16 sh = (_Float16)s;
        m[j] = sh;
        m[8 + j] = (_Float16)(s - (float)sh);
    }
}

// k_split of rmsnorm(x)·w (gpu/cpu.rs:157-166) for rows of up to
// kRmsMaxCols: a block a token, a float4 a lane in turn (the split's layout:
// eight consecutive lanes hold a sub-block), its sum of squares reduced over
// the block, y = x·(scale·w) as k_rmsnorm makes it; with xn_out, the
// normalized row written there in f32 too.
constexpr int kRmsMaxCols = 8192;

__global__ void __launch_bounds__(256) k_split_rms(const float *__restrict__ x, const float *__restrict__ w, float eps,
                                                   _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                                                   _Float16 *__restrict__ xm, float *__restrict__ xn_out,
                                                   size_t cols) {
    __shared__ float red[4];
    constexpr int kPer = kRmsMaxCols / 4 / 256;
    const size_t t = blockIdx.x, n4 = cols / 4;
    const float4 *xr = (const float4 *)(x + t * cols);
    const int tid = threadIdx.x;
    float4 v[kPer];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const size_t j = tid + 256 * k;
        v[k] = j < n4 ? xr[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        ss += (v[k].x * v[k].x + v[k].y * v[k].y) + (v[k].z * v[k].z + v[k].w * v[k].w);
    }
    ss = block_sum<256>(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)cols + eps);
#pragma unroll
    for (int k = 0; k < kPer; k++) {
        const size_t j = tid + 256 * k;
        if (j >= n4) break;  // (cols a multiple of 256: whole waves)
        const float4 nw = ((const float4 *)w)[j];
        const float4 y = make_float4(v[k].x * (scale * nw.x), v[k].y * (scale * nw.y), v[k].z * (scale * nw.z),
                                     v[k].w * (scale * nw.w));
        if (xn_out) ((float4 *)(xn_out + t * cols))[j] = y;
        split_put(y, t * n4 + j, cols, xh, xl, xm);
    }
}

// k_split of the DeltaNet output gate, silu(z)·rmsnorm(att)·w per head of
// dim (gpu/cpu.rs:157-166, 238-242): k_gated_norm's values, bit for bit,
// split as they are made (the gated z is not written).
template <int LANES>  // dim / 4: the lanes of a head
__global__ void __launch_bounds__(256) k_split_gated(const float *__restrict__ z, const float *__restrict__ att,
                                                     const float *__restrict__ w, size_t total, size_t dim, float eps,
                                                     _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                                                     _Float16 *__restrict__ xm, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // a float4 of the [n][total] rows
    if (i * 4 >= n * total) return;  // whole waves of float4s
    const float4 a = ((const float4 *)att)[i];
    const float ss = group_sum<LANES>((a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w));
    const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    const float4 nw = ((const float4 *)w)[(i * 4 % dim) / 4];
    float4 g = ((const float4 *)z)[i];
    g.x = g.x * sigmoidf_(g.x) * (a.x * (scale * nw.x));
    g.y = g.y * sigmoidf_(g.y) * (a.y * (scale * nw.y));
    g.z = g.z * sigmoidf_(g.z) * (a.z * (scale * nw.z));
    g.w = g.w * sigmoidf_(g.w) * (a.w * (scale * nw.w));
    split_put(g, i, total, xh, xl, xm);
}

// A small bf16 matrix (up to kBfRows rows: the DeltaNet gate projection's
// 96) against a batch's prepared split, on the f16 matrix cores: every bf16
// weight of f16 range is an f16 exactly (8 significant bits of 11; weights
// under 2^-14 keep f16's subnormal spacing, 2^-24, far below the products'
// rounding), so w·x = w·hi + w·lo as two MFMA chains in f32, the same
// accuracy as the split's other products.  A workgroup of 4 waves takes 16
// tokens and every row (v_mfma_f32_16x16x32_f16: 6 row tiles), its waves
// splitting the columns in 4 runs (the next step's loads issued while the
// current one is multiplied) and meeting in LDS, in wave order; out = or +=
// the sums.
constexpr int kBfRows = 96, kBfWaves = 4, kBfTiles = kBfRows / 16;

__global__ void __launch_bounds__(64 * kBfWaves) k_bf16_split(const uint16_t *__restrict__ w, float *__restrict__ out,
                                                              const _Float16 *__restrict__ xh,
                                                              const _Float16 *__restrict__ xl, unsigned rows,
                                                              unsigned cols, unsigned n, int add) {
    __shared__ float part[kBfWaves][16][kBfRows + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r16 = lane & 15, kq = lane >> 4;
    const unsigned tok0 = blockIdx.x * 16, t = tok0 + r16;
    const bool tlive = t < n;
    const unsigned steps = cols / 32, s0 = wave * steps / kBfWaves, s1 = (wave + 1) * steps / kBfWaves;
    // lane: A row r16 of each 16-row tile, B token r16, k = 32·step + 8·kq..+7
    const uint4 *wr[kBfTiles];
#pragma unroll
    for (int i = 0; i < kBfTiles; i++) {
        const unsigned r = (unsigned)(16 * i + r16) < rows ? (unsigned)(16 * i + r16) : 0u;
        wr[i] = (const uint4 *)(w + (size_t)r * cols + 8 * kq);
    }
    const size_t xo = (size_t)(tlive ? t : 0) * cols + 8 * kq;
    const uint4 *ph = (const uint4 *)(xh + xo), *pl = (const uint4 *)(xl + xo);
    float4v acc[kBfTiles];
#pragma unroll
    for (int i = 0; i < kBfTiles; i++) acc[i] = float4v{};
    uint4 wa[kBfTiles], ha, la;
    auto load = [&](unsigned s) {
#pragma unroll
        for (int i = 0; i < kBfTiles; i++) wa[i] = wr[i][4 * s];
        ha = ph[4 * s];
        la = pl[4 * s];
    };
    if (s0 < s1) load(s0);
    for (unsigned s = s0; s < s1; s++) {
        half8 a[kBfTiles];
#pragma unroll
        for (int i = 0; i < kBfTiles; i++) {
            const uint32_t v[4] = {wa[i].x, wa[i].y, wa[i].z, wa[i].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                a[i][2 * e] = (_Float16)__uint_as_float(v[e] << 16);
                a[i][2 * e + 1] = (_Float16)__uint_as_float(v[e] & 0xffff0000u);
            }
        }
        const half8 bh = __builtin_bit_cast(half8, ha), bl = __builtin_bit_cast(half8, la);
        if (s + 1 < s1) load(s + 1);
#pragma unroll
        for (int i = 0; i < kBfTiles; i++) {
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], bh, acc[i], 0, 0, 0);
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], bl, acc[i], 0, 0, 0);
        }
    }
    // C tile i: lane holds rows 16i + 4kq + e of token r16
#pragma unroll
    for (int i = 0; i < kBfTiles; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) part[wave][r16][16 * i + 4 * kq + e] = acc[i][e];
    __syncthreads();
    for (unsigned idx = threadIdx.x; idx < 16u * kBfRows; idx += 64 * kBfWaves) {
        const unsigned tt = idx / kBfRows, r = idx % kBfRows;
        if (r >= rows || tok0 + tt >= n) continue;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < kBfWaves; q++) v += part[q][tt][r];
        float *o = out + (size_t)(tok0 + tt) * rows + r;
        *o = add ? *o + v : v;
    }
}

// what a product does with its result r and the output's old value o
// (gpu/mod.rs:259 the add, gpu/cpu.rs:238-242 the SwiGLU's silu(gate)·up)
DEV float gemm_out(int mode, float o, float r) {
    return mode == kGemmAdd ? o + r : mode == kGemmSiluGate ? o * sigmoidf_(o) * r : r;
}

struct GemmArgs {
    const uint8_t *w;
    unsigned rows, cols, n;
    unsigned rtiles, ttiles, grid;  // row tiles, token tiles, workgroups launched (a multiple of 8)
    unsigned parts;                 // workgroups a tile (k split): > 1, partial results to part_out
    const _Float16 *xh, *xl, *xm;
    float *out;
    float *part_out;                // [parts][n][rows]
    int mode;                       // GemmMode
    // jobs = 2: a second matrix of the same shape over the same activations
    // (w2 into out2), its tiles after the first's in one launch
    const uint8_t *w2;
    float *out2;
    unsigned jobs;
};

// the physical 16-byte chunk of logical chunk c (0..7) in LDS row r
DEV int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// byte k of a 16-byte block header held in registers
DEV int hbyte(const uint4 &h, int k) {
    const uint32_t w = k < 4 ? h.x : k < 8 ? h.y : k < 12 ? h.z : h.w;
    return (int)((w >> (8 * (k & 3))) & 0xffu);
}

// sub-block j's 6-bit scale and min from the header's 12 packed bytes at
// offset 4 (ggml get_scale_min_k4)
DEV void scale_min(const uint4 &h, int j, int &sc, int &mn) {
    if (j < 4) {
        sc = hbyte(h, 4 + j) & 63;
        mn = hbyte(h, 8 + j) & 63;
    } else {
        sc = (hbyte(h, 8 + j) & 0xf) | ((hbyte(h, j) >> 6) << 4);
        mn = (hbyte(h, 8 + j) >> 4) | ((hbyte(h, 4 + j) >> 6) << 4);
    }
}

DEV uint32_t pack2(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | (uint32_t)__builtin_bit_cast(uint16_t, b) << 16;
}

// A loader thread's global loads of one step: its row's 32 quant bytes of
// the group and 16-byte header, and 16 bytes of its token's sub-block sums
// (the header and sums are reloaded every step; they only change per block).
struct StepLoad {
    uint4 q[2], hdr, m;
};

__global__ void __launch_bounds__(kThreads) k_gemm_q4k(const GemmArgs a) {
    extern __shared__ uint4 lds[];
    // [2][256 rows][8 chunks] weights, [2][128][8] activation hi, lo,
    // [2][256][2] min operands, [2][128][2] sub-block sums, [2][256] d and 1/d
    uint4 *A = lds, *Bh = A + 2 * kRows * 8, *Bl = Bh + 2 * kToks * 8, *Am = Bl + 2 * kToks * 8,
          *Xm = Am + 2 * kRows * 2;
    float *Dd = (float *)(Xm + 2 * kToks * 2), *Dr = Dd + 2 * kRows;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // XCD-major numbering: workgroup bx runs on XCD bx % 8
    const unsigned per = a.grid / 8, lin = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const unsigned tiles = a.rtiles * a.ttiles, jt = tiles * a.parts;
    if (lin >= jt * a.jobs) return;
    const unsigned job = lin / jt, lr = lin - job * jt;
    const unsigned part = lr / tiles, tile = lr % tiles;
    const uint8_t *const wmat = job ? a.w2 : a.w;
    float *const omat = job ? a.out2 : a.out;
    const unsigned tt = tile / a.rtiles, rt = tile % a.rtiles;
    const unsigned row0 = rt * kRows, tok0 = tt * kToks;
    // this part's blocks [b0, b0 + nb) of the row's nbt
    const unsigned nbt = a.cols / 256, b0 = part * nbt / a.parts, nb = (part + 1) * nbt / a.parts - b0;
    const unsigned steps = 4 * nb, wtiles = (a.rows + 15) / 16;

    if (wave >= 8) {
        // ---------------- loader waves: 256 threads
        const int lt = tid - 512;
        // weights: row ar, the group's 32 quant bytes
        const int ar = lt;
        const unsigned wtile = (row0 + ar) / 16;
        const bool wlive = wtile < wtiles;
        typedef const __attribute__((address_space(1))) u4v *gq;
        // sub-block sums: token bt, 16 bytes bq
        const int bt = lt >> 1, bq = lt & 1;
        const bool xlive = tok0 + bt < a.n;
        const uint8_t *wsrc = wmat + ((size_t)(wlive ? wtile : 0) * nbt + b0) * q4kt::kUnit;
        const gq qsrc = (gq)(wsrc + q4kt::qs_off(0, (row0 + ar) % 16));
        const gq hsrc = (gq)(wsrc + q4kt::meta_off((row0 + ar) % 16));
        const gq ms0 = (gq)(a.xm + ((size_t)(tok0 + (xlive ? bt : 0)) * nbt + b0) * 16 + 8 * bq);
        const uint4 z4 = make_uint4(0, 0, 0, 0);
        // step s: block s / 4 (unit b·2304), group s % 4 (512 bytes); x at
        // s·64 halves; sums at b·16 halves
        auto fetch = [&](unsigned s, StepLoad &L) {
            const unsigned b = s / 4, g = s % 4;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const uint4 q = __builtin_bit_cast(uint4, qsrc[(b * q4kt::kUnit + g * 512) / 16 + k]);
                L.q[k] = wlive ? q : z4;
            }
            const uint4 h = __builtin_bit_cast(uint4, hsrc[b * q4kt::kUnit / 16]);
            L.hdr = wlive ? h : z4;  // zero: d = dmin = 0
            const uint4 m = __builtin_bit_cast(uint4, ms0[b * 2]);
            L.m = xlive ? m : z4;
        };
        // the current block's unit and quant factor, the previous block's unit
        float unit = 1.0f, qscale = 1.0f, prev_unit = 1.0f;
        // dequantize step s into buffer s % 2 (and at a block's first group
        // the block's data into its buffer)
        auto stage = [&](unsigned s, const StepLoad &L) {
            const unsigned g = s % 4, buf = s % 2, bb = (s / 4) % 2;
            const uint4 &hdr = L.hdr;
            int sc0, mn0, sc1, mn1;
            scale_min(hdr, 2 * g, sc0, mn0);
            scale_min(hdr, 2 * g + 1, sc1, mn1);
            if ((hdr.x & 0x7fffu) == 0) sc0 = sc1 = 0;  // d = 0: the block's products are zero
            const float d0 = dq::from_f16((uint16_t)(hdr.x & 0xffffu));
            const float dmin = dq::from_f16((uint16_t)(hdr.x >> 16));
            if (g == 0) {
                // the block's unit: d, or (d = 0, or dmin·63/d past f16 range for
                // the min operands) a larger one, the quants scaled by d/unit
                unit = fmaxf(d0 != 0.0f ? fabsf(d0) : 1.0f, fabsf(dmin) * (63.0f / 30000.0f));
                qscale = d0 / unit;  // 1 but for such blocks
            }
            // sc·q exactly in f16: a nibble q ORed into the mantissa of 1024
            // gives 1024 + q (the high nibble, masked in place, 1024 + 16q),
            // minus 1024 exactly, times sc (sc/16), exactly; two weights a
            // packed op
            const float f0 = (float)sc0 * qscale, f1 = (float)sc1 * qscale * 0.0625f;  // (exact when qscale = 1)
            const half2v s0 = half2v{(_Float16)f0, (_Float16)f0};
            const half2v s1 = half2v{(_Float16)f1, (_Float16)f1};
            const half2v k1024 = half2v{(_Float16)1024.0f, (_Float16)1024.0f};
            uint4 *row = A + (buf * kRows + ar) * 8;
#pragma unroll
            for (int hq = 0; hq < 2; hq++) {  // quant bytes 16·hq..16·hq+15: k = 16·hq.. and 32 + 16·hq..
                const uint32_t words[4] = {L.q[hq].x, L.q[hq].y, L.q[hq].z, L.q[hq].w};
                uint32_t lo[8], hi[8];
#pragma unroll
                for (int k = 0; k < 4; k++) {
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t p = __builtin_amdgcn_perm(0u, words[k], e ? 0x0c030c02u : 0x0c010c00u);
                        const half2v ql = __builtin_bit_cast(half2v, (p & 0x000f000fu) | 0x64006400u);
                        // the high nibble is stored XOR 8
                        const half2v qh = __builtin_bit_cast(half2v, ((p ^ 0x00800080u) & 0x00f000f0u) | 0x64006400u);
                        lo[2 * k + e] = __builtin_bit_cast(uint32_t, (half2v)((ql - k1024) * s0));
                        hi[2 * k + e] = __builtin_bit_cast(uint32_t, (half2v)((qh - k1024) * s1));
                    }
                }
                row[swz(ar, 2 * hq)] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                row[swz(ar, 2 * hq + 1)] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
                row[swz(ar, 4 + 2 * hq)] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                row[swz(ar, 5 + 2 * hq)] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
            }
            if (g == 0) {
                // the block's min operands −dmin·m_sb/unit (hi, lo), the unit
                // (for the end) and the previous block's unit over this one
                // (the accumulators' change of units), and the tokens'
                // sub-block sums
                const float nm = -dmin / unit;  // the min term is subtracted
                uint32_t mh[4], ml[4];
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    int sa, ma, sb_, mb;
                    scale_min(hdr, j, sa, ma);
                    scale_min(hdr, j + 1, sb_, mb);
                    const float va = nm * (float)ma, vb = nm * (float)mb;
                    const _Float16 ha = (_Float16)va, hb = (_Float16)vb;
                    mh[j / 2] = pack2(ha, hb);
                    ml[j / 2] = pack2((_Float16)(va - (float)ha), (_Float16)(vb - (float)hb));
                }
                Am[(bb * kRows + ar) * 2] = make_uint4(mh[0], mh[1], mh[2], mh[3]);
                Am[(bb * kRows + ar) * 2 + 1] = make_uint4(ml[0], ml[1], ml[2], ml[3]);
                Dd[bb * kRows + ar] = unit;
                Dr[bb * kRows + ar] = prev_unit / unit;
                prev_unit = unit;
                Xm[(bb * kToks + bt) * 2 + bq] = L.m;
            }
        };
        // two steps' loads in flight: step s + 1 is staged from registers
        // loaded two steps earlier (past the last step, copies of it that
        // nothing reads); one barrier a step, as the matrix waves
        StepLoad L0, L1;
        auto cl = [&](unsigned s) { return s < steps ? s : steps - 1; };
        fetch(0, L0);
        fetch(cl(1), L1);
        stage(0, L0);
        fetch(cl(2), L0);
        __syncthreads();
        for (unsigned s = 0; s < steps; s += 2) {
            stage(s + 1, L1);
            fetch(cl(s + 3), L1);
            __syncthreads();
            if (s + 1 < steps) {
                stage(s + 2, L0);
                fetch(cl(s + 4), L0);
                __syncthreads();
            }
        }
        return;
    }

    // ---------------- matrix waves: wave (wr, wc) computes rows 64·wr..,
    // tokens 64·wc.., as 2 × 2 tiles of 32 × 32 (v_mfma_f32_32x32x16_f16:
    // lane l holds A's row l % 32, B's column l % 32, at k 8(l / 32)..+7 of
    // a 16-wide k slice; C's column l % 32, rows 8g + 4(l / 32) + e).  A
    // step's four k slices are software-pipelined: slice k + 1's fragments are
    // read while slice k's MFMAs run.  acc holds the sums in units of the
    // current block's d (its "unit"): the block's products of exact f16
    // integers and its min term (its operands pre-divided by the unit)
    // accumulate, and at the next block's start acc is multiplied by
    // unit_b / unit_{b+1}, once, at the end by the last unit.
    const int wr = wave >> 1, wc = wave & 1;
    const int r32 = lane & 31, kh = lane >> 5;
    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = float16v{};
    // The activations of step s (hi and lo parts, 32 KB) go into buffer
    // s % 2 straight from global memory (global_load_lds, no registers), 32
    // copies of 8 token rows, wave `wave` taking 4 of them: lane l lands in
    // row 8·(k % 16) + l / 8 at physical chunk l % 8, so it reads the logical
    // chunk that the row's swizzle puts there.  A step's copies are issued
    // when the barrier before it has freed the buffer, and waited for before
    // the barrier that publishes it.
    // Wave w copies part w / 4 (hi, lo) of token rows 32·(w % 4) + 8j + l / 8
    // (j = 0..3); the logical chunk of physical chunk l % 8 in row r is
    // (l % 8) ^ ((r / 2) % 8), which for these rows depends on j's parity.
    const _Float16 *xpart = wave >= 4 ? a.xl : a.xh;
    const unsigned trow0 = 32u * (wave & 3) + (unsigned)(lane >> 3);
    const unsigned cj0 = (unsigned)(lane & 7) ^ ((trow0 >> 1) & 7);
    const unsigned rowoff0 = (tok0 + trow0) * a.cols + 256u * b0;  // halves
    auto dma = [&](unsigned s) {
        const unsigned buf = s % 2;
        // (opaque copies, so that the offsets are formed here each step
        // rather than kept in registers across the step)
        unsigned r0 = rowoff0, t0r = tok0 + trow0, c0 = cj0;
        asm volatile("" : "+v"(r0), "+v"(t0r), "+v"(c0));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool live = t0r + 8u * j < a.n;
            const unsigned ro = live ? r0 + 8u * j * a.cols : tok0 * a.cols + 256u * b0;
            const unsigned off = 2u * (ro + s * kStep + 8u * ((j & 1) ? c0 ^ 4u : c0));
            uint4 *dst = (wave >= 4 ? Bl : Bh) + (buf * kToks + 32 * (wave & 3) + 8 * j) * 8;
            lds_copy16_off(xpart, off, (uint8_t *)dst);
        }
    };
    dma(0);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
    struct Frags {
        half8 a[2], bh[2], bl[2];
    };
    // a lane's LDS rows (A: rows 128wr + 32i + l % 32; B: tokens 64wc + 32j
    // + l % 32) share the swizzle (l % 32 / 2) % 8, so per k slice one
    // pointer each, the tiles, buffers and hi/lo at constant offsets
    const int sw = (r32 >> 1) & 7;
    const uint4 *pa[4], *pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const int c = (2 * ks + kh) ^ sw;
        pa[ks] = A + (wr * 64 + r32) * 8 + c;
        pb[ks] = Bh + (wc * 64 + r32) * 8 + c;
    }
    auto read = [&](unsigned buf, int ks, Frags &f) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            f.bh[j] = __builtin_bit_cast(half8, pb[ks][(buf * kToks + j * 32) * 8]);
            f.bl[j] = __builtin_bit_cast(half8, pb[ks][(buf * kToks + j * 32) * 8 + 2 * kToks * 8]);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) f.a[i] = __builtin_bit_cast(half8, pa[ks][(buf * kRows + i * 32) * 8]);
    };
    // (the hi products of the 8 tiles, then the lo ones: an accumulator's two
    // MFMAs are 8 apart, not back to back)
    auto mma = [&](const Frags &f) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.bl[j], acc[i][j], 0, 0, 0);
    };
    // per-row factors of this lane's rows: tile i, rows 8g + 4kh + e
    auto scale_rows = [&](const float *v) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 d = *(const float4 *)&v[wr * 64 + i * 32 + 8 * g + 4 * kh];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    acc[i][j][4 * g] *= d.x;
                    acc[i][j][4 * g + 1] *= d.y;
                    acc[i][j][4 * g + 2] *= d.z;
                    acc[i][j][4 * g + 3] *= d.w;
                }
            }
    };
    Frags f0, f1;
    auto step = [&](unsigned s, int g) {
        const unsigned buf = s % 2, bb = (s / 4) % 2;
        if (s + 1 < steps) dma(s + 1);
        read(buf, 0, f0);
        if (g == 0 && s > 0) scale_rows(Dr + bb * kRows);
        read(buf, 1, f1);
        mma(f0);
        read(buf, 2, f0);
        mma(f1);
        read(buf, 3, f1);
        mma(f0);
        mma(f1);
        // the order the scheduler keeps: slice 0's 6 fragment reads, then the
        // 8 MFMAs of slices 0-2 each with the next slice's reads between
        // them (a read after each of the first six), then slice 3's MFMAs;
        // left to itself it reuses one set of fragment registers and waits
        // for each read
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
        for (int k = 0; k < 3; k++) {
#pragma unroll
            for (int r = 0; r < 6; r++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        if (g == 3) {
            // the block's min term, in its unit: [−hi, −hi]·[X_hi, X_lo] and
            // [−lo, 0]·[X_hi, 0] over the 8 sub-blocks of each k half
            const half8 zero = half8{0, 0, 0, 0, 0, 0, 0, 0};
            half8 x1[2], x2[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int t = wc * 64 + j * 32 + r32;
                const half8 xh = __builtin_bit_cast(half8, Xm[(bb * kToks + t) * 2]);
                const half8 xl = __builtin_bit_cast(half8, Xm[(bb * kToks + t) * 2 + 1]);
                x1[j] = kh == 0 ? xh : xl;
                x2[j] = kh == 0 ? xh : zero;
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int r = wr * 64 + i * 32 + r32;
                const half8 mh = __builtin_bit_cast(half8, Am[(bb * kRows + r) * 2]);
                const half8 ml = kh == 0 ? __builtin_bit_cast(half8, Am[(bb * kRows + r) * 2 + 1]) : zero;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(mh, x1[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ml, x2[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);  // this wave's copies of step s + 1
        __syncthreads();
    };
    for (unsigned b = 0; b < nb; b++) {
        step(4 * b, 0);
        step(4 * b + 1, 1);
        step(4 * b + 2, 2);
        step(4 * b + 3, 3);
    }
    scale_rows(Dd + ((nb - 1) % 2) * kRows);  // out of the last block's unit
    // C tile (i, j): lane holds rows 32i + 8g + 4kh + e of token 32j + l % 32
    // (a part of a k-split product: its own slice of part_out, plainly)
    float *const dst = a.parts > 1 ? a.part_out + (size_t)part * a.n * a.rows : omat;
    const int mode = a.parts > 1 ? kGemmStore : a.mode;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const unsigned t = tok0 + wc * 64 + j * 32 + r32;
        if (t >= a.n) continue;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const unsigned r = row0 + wr * 64 + i * 32 + 8 * g + 4 * kh;
                float *o = dst + (size_t)t * a.rows + r;
                if (a.rows % 4 == 0 && r + 3 < a.rows) {
                    // four rows of the token: one 16-byte access
                    float4 v = mode == kGemmStore ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : *(const float4 *)o;
                    v.x = gemm_out(mode, v.x, acc[i][j][4 * g]);
                    v.y = gemm_out(mode, v.y, acc[i][j][4 * g + 1]);
                    v.z = gemm_out(mode, v.z, acc[i][j][4 * g + 2]);
                    v.w = gemm_out(mode, v.w, acc[i][j][4 * g + 3]);
                    *(float4 *)o = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (r + e < a.rows) o[e] = gemm_out(mode, o[e], acc[i][j][4 * g + e]);
                }
            }
    }
}

// out = Σ_p parts[p] by the mode, the parts in order (the same bits every run)
__global__ void k_gemm_reduce(float *__restrict__ out, const float *__restrict__ parts, size_t count, unsigned np,
                              int mode) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float v = parts[i];
    for (unsigned p = 1; p < np; p++) v += parts[p * count + i];
    out[i] = gemm_out(mode, mode == kGemmStore ? 0.0f : out[i], v);
}

// Parts a tile: a workgroup fills a CU (its LDS), so a product of W tiles
// runs in about W / 256 rounds.  Measured on MI355X at 2048 tokens, splitting
// the blocks of a row pays when under half the CUs would work (W ≤ 128), and
// when a second round would be short but its tiles long (256 < W ≤ 384, at
// least 48 blocks a row: the 17408-column down product, 10% faster); the
// partial results cost P·n·rows floats of traffic more.
unsigned gemm_parts(unsigned tiles, unsigned nb) {
    unsigned p = 1;
    if (tiles <= 128) p = 256 / tiles < 4 ? 256 / tiles : 4;
    else if (tiles > 256 && tiles <= 384 && nb >= 48) p = 4;
    while (p > 1 && nb / p < 4) p--;
    return p;
}

constexpr size_t kLds = (size_t)16 * (2 * kRows * 8 + 4 * kToks * 8 + 2 * kRows * 2 + 2 * kToks * 2) + 2 * 4 * 2 * kRows;

// The kernel's dynamic-LDS limit, raised once a process (a function-local
// static is initialized once even when host threads reach it together).
hipError_t raise_lds_limit() {
    static const hipError_t raised =
        hipFuncSetAttribute((const void *)k_gemm_q4k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds);
    return raised;
}

}  // namespace

size_t gemm_split_bytes(size_t n, size_t cols) { return 2 * n * cols * sizeof(_Float16) + n * (cols / 256) * 32; }

// The partial results a k-split product of n tokens over a rows × cols
// matrix keeps (0 when it does not split).
size_t gemm_parts_floats(size_t n, size_t rows, size_t cols) {
    const unsigned rtiles = (unsigned)((rows + kRows - 1) / kRows), ttiles = (unsigned)((n + kToks - 1) / kToks);
    const unsigned p = gemm_parts(rtiles * ttiles, (unsigned)(cols / 256));
    return p > 1 ? (size_t)p * n * rows : 0;
}

hipError_t gemm_reserve(dwim_dev *dev, size_t split_bytes, size_t parts_floats) {
    hipError_t e = dev_grow(dev, &dev->split, &dev->split_cap, split_bytes, 1);
    if (e != hipSuccess) return e;
    return dev_grow(dev, (void **)&dev->gemm_parts, &dev->gemm_parts_cap, parts_floats, sizeof(float));
}

hipError_t gemm_prepare(dwim_dev *dev, const float *x, size_t n, size_t cols) {
    if (cols % 256 || n >= (1u << 31)) return hipErrorInvalidValue;
    hipError_t e0 = dev_grow(dev, &dev->split, &dev->split_cap, gemm_split_bytes(n, cols), 1);
    if (e0 != hipSuccess) return e0;
    _Float16 *xh = (_Float16 *)dev->split, *xl = xh + n * cols, *xm = xl + n * cols;
    const size_t subs = n * (cols / 32);
    k_split<<<(unsigned)((subs * 8 + 255) / 256), 256, 0, dev->stream>>>(x, xh, xl, xm, n, cols);
    dev->split_n = n;
    dev->split_cols = cols;
    return hipGetLastError();
}

hipError_t gemm_run(dwim_dev *dev, const dwim_weight *w, float *out, size_t n, int mode) {
    if (w->fmt != DWIM_Q4_K || w->rows >= (1u << 31) || dev->split_n != n || dev->split_cols != w->cols)
        return hipErrorInvalidValue;
    hipError_t e;
    if ((e = raise_lds_limit()) != hipSuccess) return e;
    _Float16 *xh = (_Float16 *)dev->split, *xl = xh + n * w->cols, *xm = xl + n * w->cols;
    GemmArgs a{};
    a.w = (const uint8_t *)w->q;
    a.rows = (unsigned)w->rows;
    a.cols = (unsigned)w->cols;
    a.n = (unsigned)n;
    a.rtiles = (unsigned)((w->rows + kRows - 1) / kRows);
    a.ttiles = (unsigned)((n + kToks - 1) / kToks);
    a.parts = gemm_parts(a.rtiles * a.ttiles, (unsigned)(w->cols / 256));
    if (a.parts > 1) {
        e = dev_grow(dev, (void **)&dev->gemm_parts, &dev->gemm_parts_cap, (size_t)a.parts * n * w->rows,
                     sizeof(float));
        if (e != hipSuccess) return e;
        a.part_out = dev->gemm_parts;
    }
    a.jobs = 1;
    a.grid = (a.rtiles * a.ttiles * a.parts + 7) / 8 * 8;
    a.xh = xh;
    a.xl = xl;
    a.xm = xm;
    a.out = out;
    a.mode = mode;
    k_gemm_q4k<<<a.grid, kThreads, kLds, dev->stream>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess || a.parts == 1) return e;
    const size_t count = n * w->rows;
    k_gemm_reduce<<<(unsigned)((count + 255) / 256), 256, 0, dev->stream>>>(out, a.part_out, count, a.parts, mode);
    return hipGetLastError();
}

// gate and up over the prepared split in one launch (their tiles make
// whole rounds of workgroups together where each alone ends in a part-empty
// one), plain results into g and u; then the split of silu(g)·u for the down
// product.  Falls back to two launches when a k split would be needed.
hipError_t gemm_run_swiglu_pair(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, float *g, float *u,
                                size_t n) {
    if (gate->fmt != DWIM_Q4_K || up->fmt != DWIM_Q4_K || gate->rows != up->rows || gate->cols != up->cols ||
        gate->rows >= (1u << 30) || dev->split_n != n || dev->split_cols != gate->cols)
        return hipErrorInvalidValue;
    const unsigned rtiles = (unsigned)((gate->rows + kRows - 1) / kRows), ttiles = (unsigned)((n + kToks - 1) / kToks);
    hipError_t e;
    if (gemm_parts(rtiles * ttiles, (unsigned)(gate->cols / 256)) > 1) {
        e = gemm_run(dev, gate, g, n, kGemmStore);
        if (e == hipSuccess) e = gemm_run(dev, up, u, n, kGemmStore);
        if (e != hipSuccess) return e;
    } else {
        if ((e = raise_lds_limit()) != hipSuccess) return e;
        _Float16 *xh = (_Float16 *)dev->split, *xl = xh + n * gate->cols, *xm = xl + n * gate->cols;
        GemmArgs a{};
        a.w = (const uint8_t *)gate->q;
        a.w2 = (const uint8_t *)up->q;
        a.rows = (unsigned)gate->rows;
        a.cols = (unsigned)gate->cols;
        a.n = (unsigned)n;
        a.rtiles = rtiles;
        a.ttiles = ttiles;
        a.parts = 1;
        a.jobs = 2;
        a.grid = (2 * rtiles * ttiles + 7) / 8 * 8;
        a.xh = xh;
        a.xl = xl;
        a.xm = xm;
        a.out = g;
        a.out2 = u;
        a.mode = kGemmStore;
        k_gemm_q4k<<<a.grid, kThreads, kLds, dev->stream>>>(a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    // the down product's split, of silu(g)·u
    const size_t cols = gate->rows;
    e = dev_grow(dev, &dev->split, &dev->split_cap, gemm_split_bytes(n, cols), 1);
    if (e != hipSuccess) return e;
    _Float16 *xh = (_Float16 *)dev->split, *xl = xh + n * cols, *xm = xl + n * cols;
    const size_t subs = n * (cols / 32);
    k_split_swiglu<<<(unsigned)((subs * 8 + 255) / 256), 256, 0, dev->stream>>>(g, u, xh, xl, xm, n, cols);
    dev->split_n = n;
    dev->split_cols = cols;
    return hipGetLastError();
}

hipError_t gemm_prepare_rms(dwim_dev *dev, const float *x, const float *norm, float eps, size_t n, size_t cols,
                            float *xn_out) {
    if (cols % 256 || n >= (1u << 31)) return hipErrorInvalidValue;
    if (cols > (size_t)kRmsMaxCols) {
        float *xn = xn_out ? xn_out : dev_work(dev, n * cols);
        if (!xn) return hipErrorOutOfMemory;
        hipError_t e = launch_rmsnorm(dev->stream, xn, x, norm, n, cols, eps);
        return e != hipSuccess ? e : gemm_prepare(dev, xn, n, cols);
    }
    hipError_t e = dev_grow(dev, &dev->split, &dev->split_cap, gemm_split_bytes(n, cols), 1);
    if (e != hipSuccess) return e;
    _Float16 *xh = (_Float16 *)dev->split, *xl = xh + n * cols, *xm = xl + n * cols;
    k_split_rms<<<(unsigned)n, 256, 0, dev->stream>>>(x, norm, eps, xh, xl, xm, xn_out, cols);
    dev->split_n = n;
    dev->split_cols = cols;
    return hipGetLastError();
}

hipError_t gemm_prepare_gated(dwim_dev *dev, const float *z, const float *att, const float *norm, float eps, size_t n,
                              size_t total, size_t dim) {
    if (total % 256 || (dim != 128 && dim != 256) || total % dim || n >= (1u << 31)) return hipErrorInvalidValue;
    hipError_t e = dev_grow(dev, &dev->split, &dev->split_cap, gemm_split_bytes(n, total), 1);
    if (e != hipSuccess) return e;
    _Float16 *xh = (_Float16 *)dev->split, *xl = xh + n * total, *xm = xl + n * total;
    const unsigned blocks = (unsigned)((n * total / 4 + 255) / 256);
    if (dim == 128) k_split_gated<32><<<blocks, 256, 0, dev->stream>>>(z, att, norm, total, dim, eps, xh, xl, xm, n);
    else k_split_gated<64><<<blocks, 256, 0, dev->stream>>>(z, att, norm, total, dim, eps, xh, xl, xm, n);
    dev->split_n = n;
    dev->split_cols = total;
    return hipGetLastError();
}

hipError_t gemm_run_bf16(dwim_dev *dev, const dwim_weight *w, float *out, size_t n, int add) {
    if (w->fmt != DWIM_BF16 || w->rows > (size_t)kBfRows || w->cols % 32 || dev->split_n != n ||
        dev->split_cols != w->cols || n >= (1u << 31))
        return hipErrorInvalidValue;
    const _Float16 *xh = (const _Float16 *)dev->split, *xl = xh + n * w->cols;
    k_bf16_split<<<(unsigned)((n + 15) / 16), 64 * kBfWaves, 0, dev->stream>>>(
        (const uint16_t *)w->q, out, xh, xl, (unsigned)w->rows, (unsigned)w->cols, (unsigned)n, add);
    return hipGetLastError();
}

hipError_t launch_gemm_q4k(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n, int add) {
    hipError_t e = gemm_prepare(dev, x, n, w->cols);
    return e != hipSuccess ? e : gemm_run(dev, w, out, n, add ? kGemmAdd : kGemmStore);
}
