// Q4_K matrix-vector products for one token on the int8 matrix cores, with
// results at f32 accuracy (dwim gpu/cpu.rs:110-149 computes them in f32).
//
// The activations come as int8 planes (planes.h): per group of 32, 24-bit
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
// path costs over two.  A wave takes up to K blocks of a tile, every weight
// load issued first; its plane loads are issued per half-block, as it goes.
//
// Modes: several matrices sharing x in one launch (workgroups find their
// matrix from their index), x += W·in (gpu/mod.rs:259), and gate and up paired
// into silu(gate·x)·(up·x) (gpu/mod.rs:274-285): the waves of a workgroup
// take gate's rows of its tile, then up's.
#include "device_util.h"
#include "layout.h"
#include "planes.h"
#include "quant_math.h"
#include "runtime.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int kMaxWaves = 16;

DEV float block_sum1024(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < waves; i++) s += red[i];
    return s;
}

// One token's planes from f32 activations, in one workgroup; eight lanes take
// a group of 32, four activations each.
__global__ void __launch_bounds__(1024) k_planes(const float *__restrict__ x, const float *norm, float eps,
                                                 float *xn_out, planes::View out) {
    __shared__ float red[16];
    const size_t n4 = out.cols / 4;
    float scale = 1.0f;
    if (norm) {
        float ss = 0.0f;
        for (size_t i = threadIdx.x; i < n4; i += blockDim.x) {
            const float4 v = ((const float4 *)x)[i];
            ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        }
        ss = block_sum1024(ss, red);
        scale = 1.0f / sqrtf(ss / (float)out.cols + eps);
    }
    // cols / 4 is a whole number of waves, so every group of 8 lanes is whole
    for (size_t i = threadIdx.x; i < n4; i += blockDim.x) {
        float4 v = ((const float4 *)x)[i];
        if (norm) {
            const float4 w = ((const float4 *)norm)[i];
            v.x = v.x * (scale * w.x);
            v.y = v.y * (scale * w.y);
            v.z = v.z * (scale * w.z);
            v.w = v.w * (scale * w.w);
            if (xn_out) ((float4 *)xn_out)[i] = v;
        }
        planes::write8x4(out, i, v);
    }
}

DEV void scale_min(uint32_t y, uint32_t z, uint32_t w, int j, float &sc, float &mn) {
    // the 6-bit scale and min of sub-block j (ggml get_scale_min_k4); y, z, w
    // hold scale bytes 0-3, 4-7, 8-11
    const int sh = 8 * (j & 3);
    const uint32_t a = (y >> sh) & 0xffu, bz = (z >> sh) & 0xffu, c = (w >> sh) & 0xffu;
    if (j < 4) {
        sc = (float)(a & 63u);
        mn = (float)(bz & 63u);
    } else {
        sc = (float)((c & 0xfu) | ((a >> 6) << 4));
        mn = (float)((c >> 4) | ((bz >> 6) << 4));
    }
}

struct Job {
    const uint8_t *w;
    size_t rows;
    float *out;
    int add;
};

struct Args {
    Job job[4];
    unsigned first_tile[5];
    int njobs;
    int swiglu;  // job 0's out = silu(job 0 · x) · (job 1 · x)
    size_t nb;
    int waves;   // per matrix and tile
    planes::View in;
    const int8_t *zeros;  // 64 zero bytes: the B operand of lanes with no column
};

template <int K>
__global__ void __launch_bounds__(1024) k_mv_q4k_mfma(const Args a) {
    __shared__ float hdr[kMaxWaves][8][16];  // [wave][sub-block][row]: d·sc·s (high nibbles /16)
    __shared__ float red[kMaxWaves][16];
    const int lane = threadIdx.x & 63, wave_all = threadIdx.x >> 6, kq = lane >> 4, c = lane & 15;
    const int S = a.waves;
    int j = 0;
    while (j + 1 < a.njobs && blockIdx.x >= a.first_tile[j + 1]) j++;
    const size_t tile = blockIdx.x - a.first_tile[j];
    const int pairj = a.swiglu && wave_all >= S ? 1 : 0;  // a swiglu workgroup's up half
    const int wave = wave_all - pairj * S;
    const Job job = a.job[j + pairj];
    const size_t nb = a.nb, cols = nb * 256;
    const int b0 = (int)((size_t)wave * nb / S), b1 = (int)((size_t)(wave + 1) * nb / S);
    // B: lane (k-group kq, column c) carries digit c % 3 of sub-block 2·kq + h when c / 3 == kq
    const bool active = c < 12 && c / 3 == kq;
    const int8_t *xp = active ? a.in.q + (size_t)(c % 3) * cols + 64 * kq : a.zeros;
    const size_t xstride = active ? 256 : 0;
    const float4 *xstat = (const float4 *)a.in.stat;

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float macc = 0.0f;
    {
        uint4 wq[K][2];
        uint32_t hw[K];
        float4 xs[K];
#pragma unroll
        for (int i = 0; i < K; i++) {
            const int b = b0 + i < b1 ? b0 + i : b0;
            const uint8_t *u = job.w + q4kt::unit(tile, b, nb);
            wq[i][0] = *(const uint4 *)(u + q4kt::qs_off(kq, c));
            wq[i][1] = *(const uint4 *)(u + q4kt::qs_off(kq, c) + 16);
            hw[i] = *(const uint32_t *)(u + 4 * lane);
            xs[i] = xstat[(size_t)b * 4 + (lane & 3)];
        }
#pragma unroll
        for (int i = 0; i < K; i++) {
            if (b0 + i >= b1) break;
            {
                // lane l decodes row l/4's sub-blocks 2(l%4) and 2(l%4)+1 from
                // the header words its quad holds
                const int base = lane & ~3, k = lane & 3, R = lane >> 2;
                const uint32_t w0 = __shfl(hw[i], base, 64), w1 = __shfl(hw[i], base + 1, 64),
                               w2 = __shfl(hw[i], base + 2, 64), w3 = __shfl(hw[i], base + 3, 64);
                const float d = dq::from_f16((uint16_t)(w0 & 0xffffu)), dmin = dq::from_f16((uint16_t)(w0 >> 16));
                float sc0, mn0, sc1, mn1;
                scale_min(w1, w2, w3, 2 * k, sc0, mn0);
                scale_min(w1, w2, w3, 2 * k + 1, sc1, mn1);
                const float D0 = d * sc0, D1 = d * sc1;
                macc += (dmin * mn0) * xs[i].x + (dmin * mn1 - 8.0f * D1) * xs[i].y;
                // the two sub-blocks' activation scales join d·sc
                hdr[wave_all][2 * k][R] = D0 * xs[i].z;
                hdr[wave_all][2 * k + 1][R] = (D1 * 0.0625f) * xs[i].w;
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint4 *xv = (const uint4 *)(xp + (size_t)(b0 + i) * xstride) + 2 * h;
                const uint4 xq[2] = {xv[0], xv[1]};
                const uint32_t mask = h ? 0xf0f0f0f0u : 0x0f0f0f0fu;
                v4i C = {0, 0, 0, 0};
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    const uint4 q = wq[i][m];
                    v4i av, bv;
                    av[0] = (int)(q.x & mask);
                    av[1] = (int)(q.y & mask);
                    av[2] = (int)(q.z & mask);
                    av[3] = (int)(q.w & mask);
                    bv[0] = (int)xq[m].x;
                    bv[1] = (int)xq[m].y;
                    bv[2] = (int)xq[m].z;
                    bv[3] = (int)xq[m].w;
                    C = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, C, 0, 0, 0);
                }
                const int sb = 2 * (c < 12 ? c / 3 : 0) + h;
                const float4 D = *(const float4 *)&hdr[wave_all][sb][4 * kq];
                acc[0] += D.x * (float)C[0];
                acc[1] += D.y * (float)C[1];
                acc[2] += D.z * (float)C[2];
                acc[3] += D.w * (float)C[3];
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    // the columns meet, weighted by their digit: lanes 16kq..16kq+15 hold
    // rows 4kq..4kq+3; the min terms of row R sit in lanes 4R..4R+3
    const float f = c < 12 ? (c % 3 == 0 ? 1.0f : c % 3 == 1 ? 256.0f : 65536.0f) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float v = acc[i] * f;
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        v += __shfl_xor(v, 8, 64);
        acc[i] = v;
    }
    macc += __shfl_xor(macc, 1, 64);
    macc += __shfl_xor(macc, 2, 64);
    if (c == 0)
        for (int i = 0; i < 4; i++) red[wave_all][4 * kq + i] = acc[i];
    __syncthreads();
    if ((lane & 3) == 0) red[wave_all][lane >> 2] -= macc;
    __syncthreads();
    const Job out_job = a.job[j];
    const size_t row = tile * 16 + lane;
    if (wave_all == 0 && lane < 16 && row < out_job.rows) {
        float v = 0.0f;
        for (int w = 0; w < S; w++) v += red[w][lane];
        if (a.swiglu) {
            float u = 0.0f;
            for (int w = S; w < 2 * S; w++) u += red[w][lane];
            v = v * sigmoidf_(v) * u;  // silu(gate) · up (gpu/cpu.rs:238-242)
        }
        float *o = out_job.out + row;
        *o = out_job.add ? *o + v : v;
    }
}

hipError_t run(dwim_dev *dev, Args a) {
    const size_t nb = a.nb;
    // blocks per wave (measured on MI355X: 5 for rows of 20 blocks, 3 for 24,
    // 5-6 for 68), enough waves to cover the row, at most 16 a workgroup
    const int per = a.swiglu ? 8 : 16;
    int K = (nb <= 24 && nb % 3 == 0) ? 3 : 5;
    while ((int)((nb + K - 1) / K) > per) K++;
    if (K > 6) return hipErrorInvalidValue;
    a.waves = (int)((nb + K - 1) / K);
    unsigned total = 0;
    const unsigned threads = (unsigned)(64 * a.waves * (a.swiglu ? 2 : 1));
    if (a.swiglu) a.njobs = 1;  // workgroups index gate's tiles; up's are read beside them
    for (int j = 0; j < a.njobs; j++) {
        a.first_tile[j] = total;
        total += (unsigned)q4kt::tiles(a.job[j].rows);
    }
    a.first_tile[a.njobs] = total;
    hipStream_t s = dev->stream;
    if (K == 3) k_mv_q4k_mfma<3><<<total, threads, 0, s>>>(a);
    else if (K == 4) k_mv_q4k_mfma<4><<<total, threads, 0, s>>>(a);
    else if (K == 5) k_mv_q4k_mfma<5><<<total, threads, 0, s>>>(a);
    else k_mv_q4k_mfma<6><<<total, threads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

size_t planes_scratch_bytes() { return 2 * planes::kAreaBytes; }

planes::View planes_area(dwim_dev *dev, int area, size_t cols) {
    return planes::view((int8_t *)dev->planes + area * planes::kAreaBytes, cols);
}

hipError_t launch_planes(dwim_dev *dev, const float *x, size_t cols, const float *norm, float eps, float *xn_out,
                         int area) {
    if (cols > planes::kMaxCols || cols % 256) return hipErrorInvalidValue;
    dev->prepared = 0;
    k_planes<<<1, 1024, 0, dev->stream>>>(x, norm, eps, xn_out, planes_area(dev, area, cols));
    return hipGetLastError();
}

hipError_t launch_mv_q4k_mfma(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, const int *adds,
                              int count, int swiglu, int area) {
    if (count < 1 || count > 4 || (swiglu && count != 2)) return hipErrorInvalidValue;
    const size_t cols = ws[0]->cols;
    if (cols > planes::kMaxCols || cols % 256) return hipErrorInvalidValue;
    Args a{};
    a.nb = cols / 256;
    a.in = planes_area(dev, area, cols);
    a.zeros = (const int8_t *)dev->planes + area * planes::kAreaBytes + planes::kZerosOff;
    for (int j = 0; j < count; j++) {
        if (ws[j]->cols != cols || ws[j]->fmt != DWIM_Q4_K) return hipErrorInvalidValue;
        a.job[j] = Job{(const uint8_t *)ws[j]->q, ws[j]->rows, outs[j], adds ? adds[j] : 0};
    }
    if (swiglu && ws[0]->rows != ws[1]->rows) return hipErrorInvalidValue;
    a.njobs = count;
    a.swiglu = swiglu;
    return run(dev, a);
}
