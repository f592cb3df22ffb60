// act16.h -- device-side writer of the Q4_K activation operand, shared by the
// producers that emit it directly (activation split, fused RMSNorm, SwiGLU and
// attention merge).
//
// Layout: 16-row tiles; tile rt's block kb occupies ACT_FRAG_UNITS 16-byte
// units at frag + (rt * K/256 + kb) * ACT_FRAG_UNITS, ordered exactly as the
// MFMA lanes read them (lane = 16 * g + j: row j of the tile, lane group g):
//   unit (2t + h) * 64 + lane : x*s hi (h = 0) / lo (h = 1), elements
//                               64g + 8t + {0, 2, 1, 3, 4, 6, 5, 7} of the
//                               block (the order of the weight operand,
//                               k_q4k.hip q4k_bop)
//   unit 1024 + lane          : bytes 0..7, four halves: for g < 2 the hi
//                               parts of the sums of sub-blocks 4g .. 4g+3,
//                               for g >= 2 the lo parts of sub-blocks
//                               4(g-2) .. +3 (the A operand of the one
//                               16x16x16 MFMA of the min term); bytes 8..15
//                               unused
//   units 1088 .. 1091        : 1/s of rows 0..15 (f32); 1092.. padding
// Each 256-element block of a row has its own exact power-of-two scale s with
// max|x| * s in [2^14, 2^15); x*s = hi + lo; sub-block sums of x*s are stored
// times 2^-6 as hi + lo.
#pragma once
#include "common.h"
#include "lanes.h"

namespace slate_hip {

typedef _Float16 act_half4_t __attribute__((ext_vector_type(4)));

// One wave writes row rr (0..15) of the 16-row tile block whose units start
// at fb (global memory, or an LDS copy of the same layout); lane holds
// elements 4*lane .. 4*lane+3 (zeros for padding rows).  Every lane of the
// wave must call it.
__device__ __forceinline__ void act16_store_tile_row(uint8_t* fb, int rr, int lane, float4 v) {
    const float mx = wave_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    int ex = 0;
    if (mx > 0.f && isfinite(mx)) {
        frexpf(mx, &ex);                          // mx = m * 2^ex, m in [0.5, 1)
        ex = 15 - ex;
        ex = ex > 100 ? 100 : (ex < -100 ? -100 : ex);
    }
    const float sc = ldexpf(1.0f, ex);
    const float vv[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
    act_half4_t h, l;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = (_Float16)vv[i];
        l[i] = (_Float16)(vv[i] - (float)h[i]);
        sum += vv[i];
    }
    sum = group8_sum(sum);                        // 8 lanes = one 32-element sub-block
    const float ss = sum * (1.0f / 64.0f);
    const _Float16 sh = (_Float16)ss;
    const _Float16 sl = (_Float16)(ss - (float)sh);
    const int sub = lane >> 3;
    const int g = lane >> 4, t = (lane >> 1) & 7, half_off = 8 * (lane & 1);
    const act_half4_t hp = {h[0], h[2], h[1], h[3]}, lp = {l[0], l[2], l[1], l[3]};
    *(act_half4_t*)(fb + ((2 * t) * 64 + 16 * g + rr) * 16 + half_off) = hp;
    *(act_half4_t*)(fb + ((2 * t + 1) * 64 + 16 * g + rr) * 16 + half_off) = lp;
    if ((lane & 7) == 0) {
        // sub-block s: hi half in lane group s>>2, lo half in lane group
        // (s>>2) + 2, both as element s&3 of the unit
        const int g0 = sub >> 2;
        *(_Float16*)(fb + (1024 + 16 * g0 + rr) * 16 + 2 * (sub & 3)) = sh;
        *(_Float16*)(fb + (1024 + 16 * (g0 + 2) + rr) * 16 + 2 * (sub & 3)) = sl;
    }
    if (lane == 0) *(float*)(fb + 1088 * 16 + 4 * rr) = ldexpf(1.0f, -ex);
}

// One wave writes block kb of row r of the operand a.
__device__ __forceinline__ void act16_store_block(const Act16& a, int r, int kb, int lane, float4 v) {
    uint8_t* fb = (uint8_t*)a.frag + ((size_t)(r >> 4) * (a.K / QK) + kb) * ACT_FRAG_UNITS * 16;
    act16_store_tile_row(fb, r & 15, lane, v);
}

// Block kb of ROWS rows (16, or the half `part` of 8) of 16-row tile `tile`
// written by a workgroup of 64 * ROWS threads, wave w holding row
// 16 * tile + ROWS * part + w (four elements per lane, as above): the rows'
// units are assembled in LDS (s, ACT_FRAG_UNITS units) and then written out
// contiguously, only the bytes act16_store_tile_row writes (of each group of
// 16 row units, the ROWS of these rows: whole for the hi/lo units, bytes
// 0-7 of the sum units; the rows' 1/s floats).  Eight rows' units of a group
// are one whole 128-byte line.  Rows written piece by piece from different
// workgroups fill each line in 16-byte parts at different times; lines
// written whole convert 304 x 14336 rows in 6.8 us (8-row halves) or 8.5 us
// (16-row tiles) instead of 17.4 us, with the same bytes.  Every thread of
// the workgroup calls it (it holds a barrier).
template <int ROWS>
__device__ __forceinline__ void act16_store_tile(const Act16& a, int tile, int part, int kb, uint4* s, float4 v) {
    static_assert(ROWS == 8 || ROWS == 16, "whole or half tiles");
    const int tid = threadIdx.x, r0 = ROWS * part;
    act16_store_tile_row((uint8_t*)s, r0 + (tid >> 6), tid & 63, v);
    __syncthreads();
    uint4* dst = (uint4*)a.frag + ((size_t)tile * (a.K / QK) + kb) * ACT_FRAG_UNITS;
    {
        // hi/lo units: 64 groups of 16 rows, ROWS of them each: one a thread
        const int u = (tid / ROWS) * 16 + r0 + tid % ROWS;
        dst[u] = s[u];
    }
    if (tid < 4 * ROWS) {                               // sum units: 4 groups
        const int u = 1024 + (tid / ROWS) * 16 + r0 + tid % ROWS;
        *(uint2*)(dst + u) = *(const uint2*)(s + u);
    } else if (tid < 4 * ROWS + ROWS / 4) {             // 1/s: four rows a unit
        const int u = 1088 + r0 / 4 + (tid - 4 * ROWS);
        dst[u] = s[u];
    }
}

}  // namespace slate_hip
