// Device helpers for gfx950: wave64 reductions and small math.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DEV __device__ __forceinline__

// Lane exchanges without LDS: DPP within rows of 16 lanes, and gfx950's
// permlane swaps across them.  After a step every lane of the grown group
// holds the same value, so each step may pair any two halves of it.
namespace xlane {
template <int CTRL>
DEV float mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
// {v[l], v[l ^ 16]} and {v[l], v[l ^ 32]}, in some order: their sum or max
// is the pair's
DEV void swap16(float v, float &a, float &b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}
DEV void swap32(float v, float &a, float &b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}
}  // namespace xlane

// Sum over groups of `width` consecutive lanes (width a power of two <= 64;
// all lanes of a group active), every lane of a group getting the group's
// total: lane pairs xor 1 and xor 2 (quad permutes), then the two quads of 8
// (half-row mirror), the two halves of a row of 16 (row mirror), rows
// 16 apart and 32 apart (permlane swaps).
template <int WIDTH>
DEV float group_sum(float v) {
    if (WIDTH >= 2) v += xlane::mov<0xb1>(v);
    if (WIDTH >= 4) v += xlane::mov<0x4e>(v);
    if (WIDTH >= 8) v += xlane::mov<0x141>(v);
    if (WIDTH >= 16) v += xlane::mov<0x140>(v);
    if (WIDTH >= 32) {
        float a, b;
        xlane::swap16(v, a, b);
        v = a + b;
    }
    if (WIDTH >= 64) {
        float a, b;
        xlane::swap32(v, a, b);
        v = a + b;
    }
    return v;
}

template <int WIDTH>
DEV float group_max(float v) {
    if (WIDTH >= 2) v = fmaxf(v, xlane::mov<0xb1>(v));
    if (WIDTH >= 4) v = fmaxf(v, xlane::mov<0x4e>(v));
    if (WIDTH >= 8) v = fmaxf(v, xlane::mov<0x141>(v));
    if (WIDTH >= 16) v = fmaxf(v, xlane::mov<0x140>(v));
    if (WIDTH >= 32) {
        float a, b;
        xlane::swap16(v, a, b);
        v = fmaxf(a, b);
    }
    if (WIDTH >= 64) {
        float a, b;
        xlane::swap32(v, a, b);
        v = fmaxf(a, b);
    }
    return v;
}

// Block-wide sum for blocks of NT threads (a multiple of 64); `red` holds
// NT/64 floats of LDS.  Every thread gets the total.
template <int NT>
DEV float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (NT > 64) {
        __syncthreads();
        if (lane == 0) red[wave] = v;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < NT / 64; i++) t += red[i];
        v = t;
    }
    return v;
}

DEV float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
DEV float softplusf_(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

// One wave's copy of 64 × 16 bytes from global memory (lane l's address) into
// LDS at dst + 16·l (dst the same for every lane): global_load_lds_dwordx4
// with the LDS base in M0.  Issued as inline assembly so that the compiler
// does not wait for every earlier vector memory operation before it (it
// cannot tell which LDS bytes the copy writes); a kernel waits for its copies
// itself (s_waitcnt vmcnt) before a barrier, then reads them.
DEV void lds_copy16(const uint8_t *src, uint8_t *dst) {
    const unsigned base = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(__attribute__((address_space(3))) uint8_t *)dst);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(base), "v"(src) : "memory", "m0");
}

// The same copy with the source as a 64-bit base held in SGPRs (the same for
// every lane) plus a 32-bit byte offset per lane: one VGPR an address.
DEV void lds_copy16_off(const void *base, uint32_t off, uint8_t *dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(__attribute__((address_space(3))) uint8_t *)dst);
    const uint64_t b = (uint64_t)base;
    // (readfirstlane returns an int: through unsigned, so that the low word
    // is not sign-extended into the high one)
    const uint64_t sb = (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)b) |
                        (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)(b >> 32)) << 32;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" : : "s"(m0), "v"(off), "s"(sb)
                 : "memory", "m0");
}
