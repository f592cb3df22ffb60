// q4k.h -- device helpers for slate's Q4_K super-block (src/util/quant.c:135-166):
// exact f16 decode of d / dmin and the packed 6-bit (scale, min) codes.
#pragma once
#include "common.h"

namespace slate_hip {

// IEEE half -> float by integer arithmetic (precision.c:10-29 semantics,
// exact for every input incl. subnormals, independent of FP mode bits).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int sh = __builtin_clz(m) - 21;          // shifts to expose bit 10
            m = (m << sh) & 0x3ffu;
            bits = sign | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    return __uint_as_float(bits);
}

// Packed 6-bit codes of one block as four bytes per dword (quant.c:157-166):
// sc_lo holds sub-blocks 0..3, sc_hi 4..7; likewise for mins.
struct ScaleBytes { uint32_t sc_lo, sc_hi, mn_lo, mn_hi; };
__device__ __forceinline__ ScaleBytes unpack_scales(uint32_t s0, uint32_t s1, uint32_t s2) {
    ScaleBytes r;
    r.sc_lo = s0 & 0x3f3f3f3fu;
    r.mn_lo = s1 & 0x3f3f3f3fu;
    r.sc_hi = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    r.mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    return r;
}

}  // namespace slate_hip
