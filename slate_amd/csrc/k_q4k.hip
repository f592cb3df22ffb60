// k_q4k.hip -- Q4_K kernels for gfx950: bit-exact dequant, activation split,
// and the dequant-fused MFMA matmul used for decode and small-batch steps.
//
// Q4_K super-block (src/util/quant.c:135-166): 144 bytes = f16 d, f16 dmin,
// 12 bytes of packed 6-bit (scale, min) for 8 sub-blocks, 128 bytes of
// nibbles.  Slate's nibble order: sub-block s owns qs[16s..16s+15]; the low
// nibble of byte i is element i, the high nibble element i+16.
#include "launch.h"

namespace slate_hip {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

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

// ---------------------------------------------------------------------------
// Bit-exact dequant: one thread produces 8 outputs.  Two roundings exactly as
// the reference: sd = d*sc, sm = dmin*mn, w = sd*q - sm (no fused multiply-add).
__global__ __launch_bounds__(256) void dequant_q4k_kernel(const uint8_t* __restrict__ src,
                                                          float* __restrict__ dst,
                                                          int64_t n_blocks) {
#pragma clang fp contract(off)
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t b = gid >> 5;
    if (b >= n_blocks) return;
    int piece = (int)(gid & 31);
    int s = piece >> 2, quarter = piece & 3;
    const uint8_t* blk = src + b * QBLOCK;
    const uint32_t* hw = (const uint32_t*)blk;
    uint32_t h0 = hw[0];
    float d = f16_bits_to_f32(h0 & 0xffffu), dmin = f16_bits_to_f32(h0 >> 16);
    ScaleBytes sb = unpack_scales(hw[1], hw[2], hw[3]);
    uint32_t scw = s < 4 ? sb.sc_lo : sb.sc_hi, mnw = s < 4 ? sb.mn_lo : sb.mn_hi;
    float sc = (float)((scw >> (8 * (s & 3))) & 0xffu);
    float mn = (float)((mnw >> (8 * (s & 3))) & 0xffu);
    float sd = d * sc;
    float sm = dmin * mn;
    const uint32_t* q = (const uint32_t*)(blk + 16 + 16 * s + 8 * (quarter & 1));
    uint32_t w0 = q[0], w1 = q[1];
    int shift = (quarter >> 1) * 4;
    float out[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        out[e] = sd * (float)((w0 >> (8 * e + shift)) & 15u) - sm;
        out[4 + e] = sd * (float)((w1 >> (8 * e + shift)) & 15u) - sm;
    }
    // elements: quarter 0 -> 0..7, 1 -> 8..15, 2 -> 16..23, 3 -> 24..31
    int e0 = 32 * s + 8 * quarter;
    float4* o = (float4*)(dst + b * QK + e0);
    o[0] = make_float4(out[0], out[1], out[2], out[3]);
    o[1] = make_float4(out[4], out[5], out[6], out[7]);
}

int launch_dequant_q4k(float* dst, const void* src, int64_t n_blocks, hipStream_t s) {
    if (n_blocks <= 0) return 0;
    int64_t threads = n_blocks * 32;
    dim3 grid((unsigned)((threads + 255) / 256));
    hipLaunchKernelGGL(dequant_q4k_kernel, grid, dim3(256), 0, s, (const uint8_t*)src, dst, n_blocks);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Activation split.  Row r of X is scaled by an exact power of two so that
// max|x| lands in [2^14, 2^15), then split x*s = hi + lo (two f16).  The
// per-sub-block sums of x*s (<= 2^20) are stored times 2^-6 as hi + lo.
// Padding rows (r >= rows) are written as zeros.  One workgroup per row.
__global__ __launch_bounds__(256) void act16_kernel(Act16 a, const float* __restrict__ X) {
    const int r = blockIdx.x;
    const int K = a.K;
    __shared__ float red[256];
    const float* x = X + (size_t)r * K;
    bool valid = r < a.rows;
    float mx = 0.f;
    if (valid)
        for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(x[k]));
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    mx = red[0];
    int ex = 0;
    if (mx > 0.f && isfinite(mx)) {
        frexpf(mx, &ex);                 // mx = m * 2^ex, m in [0.5, 1)
        ex = 15 - ex;
        ex = ex > 100 ? 100 : (ex < -100 ? -100 : ex);
    }
    float sc = ldexpf(1.0f, ex);
    if (threadIdx.x == 0) a.rinv[r] = ldexpf(1.0f, -ex);
    _Float16* xh = a.xh + (size_t)r * K;
    _Float16* xl = a.xl + (size_t)r * K;
    const int nsub = K / 32;
    // each thread handles whole 32-element sub-blocks
    for (int sb = threadIdx.x; sb < nsub; sb += 256) {
        float sum = 0.f;
#pragma unroll 4
        for (int e = 0; e < 32; e += 4) {
            float4 v = valid ? *(const float4*)(x + sb * 32 + e) : make_float4(0.f, 0.f, 0.f, 0.f);
            float vv[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
            _Float16 h[4], l[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[i] = (_Float16)vv[i];
                l[i] = (_Float16)(vv[i] - (float)h[i]);
                sum += vv[i];
            }
            *(half4_t*)(xh + sb * 32 + e) = half4_t{h[0], h[1], h[2], h[3]};
            *(half4_t*)(xl + sb * 32 + e) = half4_t{l[0], l[1], l[2], l[3]};
        }
        float ss = sum * (1.0f / 64.0f);
        _Float16 sh = (_Float16)ss;
        _Float16 sl = (_Float16)(ss - (float)sh);
        a.ys[((size_t)r * nsub + sb) * 2 + 0] = sh;
        a.ys[((size_t)r * nsub + sb) * 2 + 1] = sl;
    }
}

int launch_act16_from_f32(const Act16& a, const float* X, hipStream_t s) {
    hipLaunchKernelGGL(act16_kernel, dim3(a.rows_pad), dim3(256), 0, s, a, X);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Dequant-fused Q4_K matmul on MFMA.
//
// Y[b, m] = sum_k X[b, k] * W[m, k].  One wave owns a 16-row weight tile and
// a range of super-blocks; NT tiles of 16 activation rows share each
// dequantised weight operand.  Per super-block and 32-element K step:
//   A (16 act rows x 32 k)   = x*s split into f16 hi and lo (two MFMAs)
//   B (32 k x 16 weight rows) = q * sc, exact in f16 (q <= 15, sc <= 63)
// so sum_s sc_s * sum q*x accumulates in f32 inside the MFMA, and is scaled
// by d once per super-block.  The min term dmin * sum_s mn_s * sum_{i in s} x
// runs as a 16x16x16 MFMA of the per-sub-block sums against mn (exact).
//
// Lane l: j = l & 15 (weight row of B / activation row of A), g = l >> 4.
// In step t (0..7) lane group g covers block-local k = 64g + 8t + e, e < 8,
// i.e. sub-block 2g + t/4, elements 8(t%4)..8(t%4)+7: the low nibbles of
// bytes 0..7 / 8..15 for t%4 = 0 / 1, the high nibbles for t%4 = 2 / 3.
// D[i][j] (16x16 f32) sits in lane (j, g) as rows 4g..4g+3.
template <int NT>
__global__ __launch_bounds__(256) void q4k_mm_kernel(const uint8_t* __restrict__ W, Act16 a,
                                                     float* __restrict__ out, int64_t ldo,
                                                     int64_t split_stride, int M, int nblk,
                                                     int blk_per_split, int rbase) {
    const int lane = threadIdx.x & 63;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int row0 = tile * 16;
    if (row0 >= M) return;
    const int kb0 = blockIdx.y * blk_per_split;
    const int kb1 = min(kb0 + blk_per_split, nblk);
    const int wrow = min(row0 + j, M - 1);
    const int K = a.K;
    const int r0 = rbase + blockIdx.z * NT * 16;      // first activation row of this wave
    const uint8_t* wbase = W + (size_t)wrow * nblk * QBLOCK;

    floatx4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};

    const half2_t k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    for (int kb = kb0; kb < kb1; ++kb) {
        const uint8_t* blk = wbase + (size_t)kb * QBLOCK;
        uint4 hdr = *(const uint4*)blk;
        uint4 qa = *(const uint4*)(blk + 16 + 32 * g);
        uint4 qb = *(const uint4*)(blk + 32 + 32 * g);
        ScaleBytes sb = unpack_scales(hdr.y, hdr.z, hdr.w);
        uint32_t scw = g < 2 ? sb.sc_lo : sb.sc_hi;
        int sh = 16 * (g & 1);
        float sc0 = (float)((scw >> sh) & 0xffu);
        float sc1 = (float)((scw >> (sh + 8)) & 0xffu);
        // q*sc from 1024+q (low nibble) or 1024+16q (high nibble) in one fma
        half2_t lo_m0 = {(_Float16)sc0, (_Float16)sc0};
        half2_t lo_a0 = {(_Float16)(-1024.f * sc0), (_Float16)(-1024.f * sc0)};
        half2_t hi_m0 = {(_Float16)(sc0 * 0.0625f), (_Float16)(sc0 * 0.0625f)};
        half2_t hi_a0 = {(_Float16)(-64.f * sc0), (_Float16)(-64.f * sc0)};
        half2_t lo_m1 = {(_Float16)sc1, (_Float16)sc1};
        half2_t lo_a1 = {(_Float16)(-1024.f * sc1), (_Float16)(-1024.f * sc1)};
        half2_t hi_m1 = {(_Float16)(sc1 * 0.0625f), (_Float16)(sc1 * 0.0625f)};
        half2_t hi_a1 = {(_Float16)(-64.f * sc1), (_Float16)(-64.f * sc1)};

        floatx4 am[NT], an[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) { am[n] = floatx4{0.f, 0.f, 0.f, 0.f}; an[n] = am[n]; }

#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint4 Q = t < 4 ? qa : qb;
            const int tq = t & 3;
            uint32_t w0 = (tq & 1) ? Q.z : Q.x;
            uint32_t w1 = (tq & 1) ? Q.w : Q.y;
            uint32_t mask = (tq & 2) ? 0xf0f0f0f0u : 0x0f0f0f0fu;
            w0 &= mask;
            w1 &= mask;
            half2_t mul = (tq & 2) ? (t < 4 ? hi_m0 : hi_m1) : (t < 4 ? lo_m0 : lo_m1);
            half2_t add = (tq & 2) ? (t < 4 ? hi_a0 : hi_a1) : (t < 4 ? lo_a0 : lo_a1);
            half2_t p0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u));
            half2_t p1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u));
            half2_t p2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u));
            half2_t p3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u));
            p0 = __builtin_elementwise_fma(p0, mul, add);
            p1 = __builtin_elementwise_fma(p1, mul, add);
            p2 = __builtin_elementwise_fma(p2, mul, add);
            p3 = __builtin_elementwise_fma(p3, mul, add);
            half8_t bop = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                size_t off = (size_t)(r0 + n * 16 + j) * K + (size_t)kb * QK + 64 * g + 8 * t;
                half8_t ah = *(const half8_t*)(a.xh + off);
                half8_t al = *(const half8_t*)(a.xl + off);
                am[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bop, am[n], 0, 0, 0);
                am[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bop, am[n], 0, 0, 0);
            }
        }
        // min term: K = 16, lane group g holds sub-blocks 4g..4g+3 (g < 2)
        half4_t bmin = {(_Float16)0.f, (_Float16)0.f, (_Float16)0.f, (_Float16)0.f};
        if (g < 2) {
            uint32_t mw = g == 0 ? sb.mn_lo : sb.mn_hi;
            half2_t m01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, mw, 0x04010400u));
            half2_t m23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, mw, 0x04030402u));
            m01 = m01 + k1024;
            m23 = m23 + k1024;
            bmin = half4_t{m01.x, m01.y, m23.x, m23.y};
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            half4_t ysh = {(_Float16)0.f, (_Float16)0.f, (_Float16)0.f, (_Float16)0.f};
            half4_t ysl = ysh;
            if (g < 2) {
                const _Float16* yp = a.ys + (((size_t)(r0 + n * 16 + j) * (K / 32)) + kb * 8 + 4 * g) * 2;
                half8_t v = *(const half8_t*)yp;     // (hi,lo) x 4 sub-blocks
                ysh = half4_t{v[0], v[2], v[4], v[6]};
                ysl = half4_t{v[1], v[3], v[5], v[7]};
            }
            an[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ysh, bmin, an[n], 0, 0, 0);
            an[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ysl, bmin, an[n], 0, 0, 0);
        }
        float d = f16_bits_to_f32(hdr.x & 0xffffu);
        float dmin64 = f16_bits_to_f32(hdr.x >> 16) * 64.0f;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[n][r] += d * am[n][r] - dmin64 * an[n][r];
        }
    }
    if (row0 + j >= M) return;
    float* o = out + (int64_t)blockIdx.y * split_stride;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            int b = r0 + n * 16 + 4 * g + r;
            o[(int64_t)b * ldo + row0 + j] = acc[n][r] * a.rinv[b];
        }
    }
}

int q4k_pick_splits(int M, int K, int rows_pad) {
    int tiles = (M + 15) / 16;
    int nblk = K / QK;
    int groups = (rows_pad + 63) / 64;
    int waves = tiles * groups;
    int want = (2048 + waves - 1) / waves;     // aim for >= 2048 waves
    if (want > 16) want = 16;
    if (want > nblk) want = nblk;
    if (want < 1) want = 1;
    return want;
}

template <int NT>
static void launch_nt(const uint8_t* w, const Act16& a, float* out, int64_t ldo, int64_t ss, int M, int nblk,
                      int bps, int nsplit, int zgroups, int rbase, hipStream_t s) {
    int tiles = (M + 15) / 16;
    dim3 grid((tiles + 3) / 4, nsplit, zgroups);
    hipLaunchKernelGGL(q4k_mm_kernel<NT>, grid, dim3(256), 0, s, w, a, out, ldo, ss, M, nblk, bps, rbase);
}

int launch_q4k_mm(const void* W, const Act16& a, float* out, int64_t ldo, int64_t split_stride, int M,
                  int nsplit, hipStream_t s) {
    const int nblk = a.K / QK;
    const int bps = (nblk + nsplit - 1) / nsplit;
    const uint8_t* w = (const uint8_t*)W;
    const int ntiles = a.rows_pad / 16;
    const int full = ntiles / 4, rem = ntiles % 4;
    if (full) launch_nt<4>(w, a, out, ldo, split_stride, M, nblk, bps, nsplit, full, 0, s);
    if (rem == 1) launch_nt<1>(w, a, out, ldo, split_stride, M, nblk, bps, nsplit, 1, full * 64, s);
    if (rem == 2) launch_nt<2>(w, a, out, ldo, split_stride, M, nblk, bps, nsplit, 1, full * 64, s);
    if (rem == 3) launch_nt<3>(w, a, out, ldo, split_stride, M, nblk, bps, nsplit, 1, full * 64, s);
    SH_CHECK_LAUNCH();
    return 0;
}

// Y[r, m] = sum over splits of part[split][r][m] (fixed order -> deterministic).
__global__ void sum_splits_kernel(float* __restrict__ Y, const float* __restrict__ part, int nsplit,
                                  int rows, int rows_pad, int M) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t n = (int64_t)rows * M;
    if (i >= n) return;
    float s = part[i];
    for (int k = 1; k < nsplit; ++k) s += part[(int64_t)k * rows_pad * M + i];
    Y[i] = s;
}

int launch_sum_splits(float* Y, const float* part, int nsplit, int rows, int rows_pad, int M,
                      hipStream_t s) {
    int64_t n = (int64_t)rows * M;
    if (n == 0) return 0;
    hipLaunchKernelGGL(sum_splits_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, Y,
                       part, nsplit, rows, rows_pad, M);
    SH_CHECK_LAUNCH();
    return 0;
}

}  // namespace slate_hip
