// One token's activations as the int8 matrix cores take them (the
// "planes"): per group of 16 activations, s = max|x| / 8355000 and
// X = rint(x / s) split into balanced base-256 digits X = 65536·X2 + 256·X1 +
// X0 (each in [-128, 127]), written as three int8 rows [3][cols]; beside them,
// per 64 activations, the four groups' scales and then their four f32 sums
// ([cols/64][8] floats).  A device holds two such areas, so that a kernel can
// read one and write the other, and four more for the tokens of a batch.
//
// A group of 16 is the 16 rows of one tile of a Q4_K matrix-vector product,
// so the product that computes those rows writes their planes itself.  When
// the consumer of a residual sum x normalizes it first (rmsnorm, dwim
// gpu/cpu.rs:157-166), the producer writes the planes of x·w (the norm
// weights) and, per group, Σx² ("ss", [cols/16] floats); the consumer scales
// its results by 1/sqrt(Σ ss / cols + eps), which is the same product.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_util.h"

namespace planes {

constexpr size_t kGroup = 16;
constexpr size_t kMaxCols = 80 * 256;
constexpr int kMax = 8355711;          // 127·(65536 + 256 + 1): every digit within int8
constexpr float kScale = 8355000.0f;   // max|x| maps here, rounding well inside kMax
constexpr size_t kStatOff = 3 * kMaxCols;                          // bytes
constexpr size_t kSsOff = kStatOff + 4 * 8 * (kMaxCols / 64);      // bytes
constexpr size_t kAreaBytes = kSsOff + 4 * (kMaxCols / kGroup);

struct View {
    int8_t *q;      // [3][cols]
    float *stat;    // [cols/64][8]: scales of groups 4k..4k+3, then their sums
    float *ss;      // [cols/16]: Σx² per group (written only for an RMS-scaled handover)
    size_t cols;
};

__host__ __device__ inline View view(void *area, size_t cols) {
    int8_t *p = (int8_t *)area;
    return View{p, (float *)(p + kStatOff), (float *)(p + kSsOff), cols};
}

__device__ __forceinline__ void digits(float x, float inv, int &d0, int &d1, int &d2) {
    const int X = min(max((int)rintf(x * inv), -kMax), kMax);
    d0 = ((X + 128) & 255) - 128;
    const int X1 = (X - d0) >> 8;
    d1 = ((X1 + 128) & 255) - 128;
    d2 = (X1 - d1) >> 8;
}

__device__ __forceinline__ void put_stat(const View &v, size_t group, float sum, float m) {
    v.stat[(group / 4) * 8 + group % 4] = m / kScale;
    v.stat[(group / 4) * 8 + 4 + group % 4] = sum;
}

// Activation i = 16·group + lane of a group that 16 consecutive lanes (a
// 16-aligned run of the wave, all active) hold one each.
__device__ __forceinline__ void write16(const View &v, size_t i, float x) {
    const float m = group_max<16>(fabsf(x)), s = group_sum<16>(x);
    const float inv = m > 0.0f ? kScale / m : 0.0f;
    int d0, d1, d2;
    digits(x, inv, d0, d1, d2);
    v.q[i] = (int8_t)d0;
    v.q[v.cols + i] = (int8_t)d1;
    v.q[2 * v.cols + i] = (int8_t)d2;
    if ((i & 15) == 0) put_stat(v, i / 16, s, m);
}

// Activations 4j..4j+3 of a group that 4 consecutive (4-aligned) lanes hold
// four each.  pair (the same for the whole wave): the two groups of each 32
// take the scale of the pair, their larger max|x| (a product that sees equal
// scales may then sum the pair in int32 before scaling).
__device__ __forceinline__ void write4x4(const View &v, size_t j, float4 x, bool pair = false) {
    float m = group_max<4>(fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
    const float s = group_sum<4>((x.x + x.y) + (x.z + x.w));
    if (pair) m = group_max<8>(m);
    const float inv = m > 0.0f ? kScale / m : 0.0f;
    const float e[4] = {x.x, x.y, x.z, x.w};
    uint32_t p0 = 0, p1 = 0, p2 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int d0, d1, d2;
        digits(e[k], inv, d0, d1, d2);
        p0 |= (uint32_t)(d0 & 255) << (8 * k);
        p1 |= (uint32_t)(d1 & 255) << (8 * k);
        p2 |= (uint32_t)(d2 & 255) << (8 * k);
    }
    ((uint32_t *)v.q)[j] = p0;
    ((uint32_t *)(v.q + v.cols))[j] = p1;
    ((uint32_t *)(v.q + 2 * v.cols))[j] = p2;
    if ((j & 3) == 0) put_stat(v, j / 4, s, m);
}

}  // namespace planes
