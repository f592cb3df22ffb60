// mfma.h -- vector types and load helpers shared by the MFMA matmul kernels
// (Q4_K and Q8_0).
#pragma once
#include "common.h"

namespace slate_hip {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt
// 7 << 4 | lgkmcnt 15 << 8 | vmcnt[5:4] << 14).
#define SH_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14))

// Direct global -> LDS copy of 16 bytes per lane: lane i's bytes come from
// sbase + voff (sbase wave-uniform, held in SGPRs; voff the lane's byte
// offset) and land at LDS byte address lds + 16 i (lds wave-uniform).
// Issued from inline assembly so the compiler does not treat every later
// LDS read as waiting on it (its LDS-DMA tracking would stall the weight
// prefetch too); callers wait with SH_WAIT_VMCNT and a barrier before
// reading the copied units.
__device__ __forceinline__ void lds_copy16(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1 offset:0" : : "v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

// Hardware half -> float (v_cvt_f32_f16; exact, subnormals included).
__device__ __forceinline__ float f16_to_f32_hw(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

}  // namespace slate_hip
