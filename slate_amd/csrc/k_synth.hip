// k_synth.hip -- seeded synthetic weights generated directly in HBM.
//
// Values are std * N(0,1) from a counter-based generator (SplitMix64 hash of
// (seed, index) -> two uniforms -> Box-Muller), so any element can be
// recomputed independently.  Q4_K tensors are quantised per super-block by
// one thread with the same scale/min search as slate_amd/synth.py
// (per sub-block min/max, 6-bit codes against the block maxima); Q8_0
// tensors per 32-element block with d = max|w| / 127 (as synth.py).
#include "launch.h"

namespace slate_hip {

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t key, uint64_t i) {
    uint64_t h = splitmix64(key ^ (i * 0xD1B54A32D192ED03ull));
    float u1 = ((float)(uint32_t)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);   // (0, 1]
    float u2 = (float)(uint32_t)((h >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__global__ void synth_f32_kernel(float* __restrict__ dst, int64_t n, uint64_t key, float std, float fill) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = std == 0.f ? fill : std * normal_at(key, (uint64_t)i);
}

int launch_synth_f32(float* dst, int64_t n, uint64_t seed, float std, float fill, hipStream_t s) {
    if (n <= 0) return 0;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(synth_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, n,
                       splitmix64(seed), std, fill);
    SH_CHECK_LAUNCH();
    return 0;
}

__global__ void synth_q4k_kernel(uint8_t* __restrict__ dst, int64_t nblocks_total, int64_t cols,
                                 uint64_t key, float std) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks_total) return;
    const int64_t nb = cols / QK;
    const int64_t row = b / nb, kb = b - row * nb;
    const uint64_t i0 = (uint64_t)(row * cols + kb * QK);
    float sc[8], mn[8];
    float scmax = 0.f, mnmax = 0.f;
    for (int s = 0; s < 8; ++s) {
        float lo = INFINITY, hi = -INFINITY;
        for (int e = 0; e < 32; ++e) {
            float v = std * normal_at(key, i0 + 32 * s + e);
            lo = fminf(lo, v);
            hi = fmaxf(hi, v);
        }
        mn[s] = fmaxf(-lo, 0.f);
        sc[s] = (hi + mn[s]) / 15.0f;
        scmax = fmaxf(scmax, sc[s]);
        mnmax = fmaxf(mnmax, mn[s]);
    }
    _Float16 d16 = (_Float16)(scmax / 63.0f);
    _Float16 m16 = (_Float16)(mnmax / 63.0f);
    float d = (float)d16, dm = (float)m16;
    uint8_t qsc[8], qmn[8];
    for (int s = 0; s < 8; ++s) {
        qsc[s] = d > 0.f ? (uint8_t)fminf(fmaxf(rintf(sc[s] / d), 0.f), 63.f) : 0;
        qmn[s] = dm > 0.f ? (uint8_t)fminf(fmaxf(rintf(mn[s] / dm), 0.f), 63.f) : 0;
    }
    uint8_t* o = dst + b * QBLOCK;
    uint16_t db = __builtin_bit_cast(uint16_t, d16), mb = __builtin_bit_cast(uint16_t, m16);
    uint8_t hdr[16];
    hdr[0] = db & 0xff; hdr[1] = db >> 8; hdr[2] = mb & 0xff; hdr[3] = mb >> 8;
    for (int j = 0; j < 4; ++j) {
        hdr[4 + j] = (qsc[j] & 63) | ((qsc[j + 4] >> 4) << 6);
        hdr[8 + j] = (qmn[j] & 63) | ((qmn[j + 4] >> 4) << 6);
        hdr[12 + j] = (qsc[j + 4] & 15) | ((qmn[j + 4] & 15) << 4);
    }
    for (int i = 0; i < 16; ++i) o[i] = hdr[i];
    for (int s = 0; s < 8; ++s) {
        float step = d * (float)qsc[s], off = dm * (float)qmn[s];
        uint8_t q[32];
        for (int e = 0; e < 32; ++e) {
            float v = std * normal_at(key, i0 + 32 * s + e);
            float qq = step > 0.f ? rintf((v + off) / step) : 0.f;
            q[e] = (uint8_t)fminf(fmaxf(qq, 0.f), 15.f);
        }
        for (int i = 0; i < 16; ++i) o[16 + 16 * s + i] = (uint8_t)(q[i] | (q[i + 16] << 4));
    }
}

int launch_synth_q4k(void* dst, int64_t rows, int64_t cols, uint64_t seed, float std, hipStream_t s) {
    if (rows <= 0) return 0;
    if (cols % QK) {
        set_error(-1, "synth_q4k: cols %lld not a multiple of 256", (long long)cols);
        return -1;
    }
    int64_t nblk = rows * (cols / QK);
    hipLaunchKernelGGL(synth_q4k_kernel, dim3((unsigned)((nblk + 127) / 128)), dim3(128), 0, s,
                       (uint8_t*)dst, nblk, cols, splitmix64(seed), std);
    SH_CHECK_LAUNCH();
    return 0;
}

__global__ void synth_q8_kernel(uint8_t* __restrict__ dst, int64_t nblocks_total, uint64_t key, float std) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks_total) return;
    const uint64_t i0 = (uint64_t)b * Q8_ELEMS;    // row-major: block b covers elements 32b..32b+31
    float v[Q8_ELEMS], amax = 0.f;
    for (int e = 0; e < Q8_ELEMS; ++e) {
        v[e] = std * normal_at(key, i0 + e);
        amax = fmaxf(amax, fabsf(v[e]));
    }
    const _Float16 d16 = (_Float16)(amax / 127.0f);
    const float d = (float)d16;
    uint8_t* o = dst + b * Q8_BYTES;
    const uint16_t db = __builtin_bit_cast(uint16_t, d16);
    o[0] = db & 0xff;
    o[1] = db >> 8;
    for (int e = 0; e < Q8_ELEMS; ++e) {
        const float q = d > 0.f ? fminf(fmaxf(rintf(v[e] / d), -127.f), 127.f) : 0.f;
        o[2 + e] = (uint8_t)(int8_t)q;
    }
}

int launch_synth_q8(void* dst, int64_t rows, int64_t cols, uint64_t seed, float std, hipStream_t s) {
    if (rows <= 0) return 0;
    if (cols % Q8_ELEMS) {
        set_error(-1, "synth_q8_0: cols %lld not a multiple of 32", (long long)cols);
        return -1;
    }
    const int64_t nblk = rows * (cols / Q8_ELEMS);
    hipLaunchKernelGGL(synth_q8_kernel, dim3((unsigned)((nblk + 127) / 128)), dim3(128), 0, s, (uint8_t*)dst,
                       nblk, splitmix64(seed), std);
    SH_CHECK_LAUNCH();
    return 0;
}

}  // namespace slate_hip
