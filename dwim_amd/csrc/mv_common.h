// Helpers shared by the one-token Q4_K kernels on the int8 matrix cores
// (k_mv_q4k_mfma.hip): the block header decode and lane
// broadcasts.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_util.h"

namespace mvq {

// The d·sc and dmin·m of sub-blocks 2k and 2k + 1 (k = 0..3) from the
// block header words w1, w2, w3 (scale bytes 0-3, 4-7, 8-11), both at once
// in the two bytes of a 16-bit lane, as ggml's get_scale_min_k4 defines them:
// sub-block j < 4 keeps 6 bits of scale byte j and of byte j + 4; j >= 4 takes
// the low / high nibble of byte j + 4 and the top two bits of byte j - 4 / j.
DEV void scales_pair(uint32_t w1, uint32_t w2, uint32_t w3, int k, float &sc0, float &sc1, float &mn0, float &mn1) {
    const int sh = 16 * (k & 1);
    const uint32_t A = (w1 >> sh) & 0xffffu, B = (w2 >> sh) & 0xffffu, C = (w3 >> sh) & 0xffffu;
    const uint32_t sc = k < 2 ? A & 0x3f3fu : (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
    const uint32_t mn = k < 2 ? B & 0x3f3fu : ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u);
    sc0 = (float)(sc & 0xffu);
    sc1 = (float)(sc >> 8);
    mn0 = (float)(mn & 0xffu);
    mn1 = (float)(mn >> 8);
}

DEV float f16_bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// lane j of each quad of lanes, to all four
template <int J>
DEV uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, J * 0x55, 0xf, 0xf, false);
}

// s_waitcnt immediate (gfx9 encoding) waiting for every vector memory
// operation: vmcnt 0, expcnt and lgkmcnt at their maxima (no wait)
constexpr int kWaitVm0 = 0x0f70;

}  // namespace mvq
