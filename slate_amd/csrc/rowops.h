// rowops.h -- device helpers of the row kernels: ordered split-K sums and
// the deferred RMSNorm row factor.
#pragma once
#include "launch.h"

namespace slate_hip {

// sum_{k < n} p[k * stride] in split order (n >= 1), loads issued eight at a
// time (clamped, so every address is a valid partial) and added under a
// predicate, so the latency of the partials is paid once per eight splits.
__device__ __forceinline__ float4 split_sum4(const float* p, int n, int64_t stride) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < n; k += 8) {
        float4 t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = *(const float4*)(p + (int64_t)min(k + i, n - 1) * stride);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (k + i < n) { s.x += t[i].x; s.y += t[i].y; s.z += t[i].z; s.w += t[i].w; }
    }
    return s;
}

__device__ __forceinline__ float split_sum1(const float* p, int n, int64_t stride) {
    float s = 0.f;
    for (int k = 0; k < n; k += 8) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = p[(int64_t)min(k + i, n - 1) * stride];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (k + i < n) s += t[i];
    }
    return s;
}

// The first eight partials of split_sum4 / split_sum1, loaded up front so a
// kernel can issue them together with its other independent loads;
// split_fin4 / split_fin1 then add them (and any further splits) in the same
// order and with the same result as split_sum4 / split_sum1.
template <int N = 8> struct Split4N { float4 t[N]; };
using Split4 = Split4N<8>;
struct Split1 { float t[8]; };
template <int N = 8>
__device__ __forceinline__ Split4N<N> split_load4(const float* p, int n, int64_t stride) {
    Split4N<N> r;
#pragma unroll
    for (int i = 0; i < N; ++i) r.t[i] = *(const float4*)(p + (int64_t)min(i, max(n - 1, 0)) * stride);
    return r;
}
__device__ __forceinline__ Split1 split_load1(const float* p, int n, int64_t stride) {
    Split1 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r.t[i] = p[(int64_t)min(i, max(n - 1, 0)) * stride];
    return r;
}
// (N = 16 loads sixteen partials up front: one round trip up to 16 splits)
template <int N = 8>
__device__ __forceinline__ float4 split_fin4(const Split4N<N>& r, const float* p, int n, int64_t stride) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (i < n) { s.x += r.t[i].x; s.y += r.t[i].y; s.z += r.t[i].z; s.w += r.t[i].w; }
    for (int k = N; k < n; k += 8) {
        float4 t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = *(const float4*)(p + (int64_t)min(k + i, n - 1) * stride);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (k + i < n) { s.x += t[i].x; s.y += t[i].y; s.z += t[i].z; s.w += t[i].w; }
    }
    return s;
}
__device__ __forceinline__ float split_fin1(const Split1& r, const float* p, int n, int64_t stride) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (i < n) s += r.t[i];
    for (int k = 8; k < n; k += 8) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = p[(int64_t)min(k + i, n - 1) * stride];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (k + i < n) s += t[i];
    }
    return s;
}

// RMSNorm factor of row r from the per-256-block sums of squares that
// residual_act_kernel leaves: inv = 1/sqrtf((float)(sum x^2 / D) + eps)
// (backend_cpu.c:48-76; block sums added in double, in block order).
__device__ __forceinline__ float row_inv_rms(const float* ssq, int r, int nblk, int D, float eps) {
    double sq = 0.0;
    for (int kb = 0; kb < nblk; ++kb) sq += (double)ssq[(size_t)r * nblk + kb];
    return 1.0f / sqrtf((float)(sq / (double)D) + eps);
}


// row_inv_rms with the block sums loaded up front (up to 32 blocks in one
// batch; the same additions in the same order).
struct RmsPre { float v[32]; };
__device__ __forceinline__ RmsPre row_rms_load(const float* ssq, int r, int nblk) {
    RmsPre p;
#pragma unroll
    for (int kb = 0; kb < 32; ++kb) p.v[kb] = ssq[(size_t)r * nblk + min(kb, nblk - 1)];
    return p;
}
__device__ __forceinline__ float row_rms_fin(const RmsPre& p, const float* ssq, int r, int nblk, int D, float eps) {
    double sq = 0.0;
#pragma unroll
    for (int kb = 0; kb < 32; ++kb)
        if (kb < nblk) sq += (double)p.v[kb];
    for (int kb = 32; kb < nblk; ++kb) sq += (double)ssq[(size_t)r * nblk + kb];
    return 1.0f / sqrtf((float)(sq / (double)D) + eps);
}

}  // namespace slate_hip
