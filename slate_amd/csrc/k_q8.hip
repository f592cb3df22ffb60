// k_q8.hip -- Q8_0 kernels for gfx950: bit-exact dequant, the tiled weight
// layout, the activation operand and the MFMA matmul.
//
// Q8_0 block (src/util/quant.c:12-25): 34 bytes = f16 d, 32 int8 q, and the
// weight is d * q (one f32 product, exact: 11 x 8 significant bits).
#include <algorithm>

#include "launch.h"
#include "lanes.h"
#include "mfma.h"

namespace slate_hip {

// ---------------------------------------------------------------------------
// Dequant: one thread per block.  d * (float)q is exact, so any order of
// evaluation gives quant.c:12-25's bits.
__global__ __launch_bounds__(256) void dequant_q8_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                         int64_t n_blocks) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= n_blocks) return;
    const uint8_t* blk = src + b * Q8_BYTES;          // 2-byte aligned
    const uint16_t* h = (const uint16_t*)blk;
    const float d = f16_to_f32_hw(h[0]);
    float4* o = (float4*)(dst + b * Q8_ELEMS);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = h[1 + 2 * i], hi = h[2 + 2 * i];
        const uint32_t w = lo | (hi << 16);
        o[i] = make_float4(d * (float)(int8_t)(w & 0xff), d * (float)(int8_t)((w >> 8) & 0xff),
                           d * (float)(int8_t)((w >> 16) & 0xff), d * (float)(int8_t)(w >> 24));
    }
}

int launch_dequant_q8(float* dst, const void* src, int64_t n_blocks, hipStream_t s) {
    if (n_blocks <= 0) return 0;
    if ((uintptr_t)dst % 16) { set_error(-1, "dequant_q8_0: dst must be 16-byte aligned"); return -1; }
    if ((uintptr_t)src % 2) { set_error(-1, "dequant_q8_0: src must be 2-byte aligned"); return -1; }
    hipLaunchKernelGGL(dequant_q8_kernel, dim3((unsigned)((n_blocks + 255) / 256)), dim3(256), 0, s,
                       (const uint8_t*)src, dst, n_blocks);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// TILED layout.  16-row tiles (rows past M zero) by 256-element groups
// (blocks past K/32 zero); tile t's group kb is 4352 contiguous bytes at
// (t * q8_groups(K) + kb) * 4352:
//   bytes 0..255             row j's eight d (f16) of the group at 16 j
//   bytes 256 + 1024 c + 16 l lane l = 16 g + j: q[j][32 (2c) + 8 g + e] for
//                            e < 8, then q[j][32 (2c + 1) + 8 g + e]
// so MFMA K step t (block t of the group) takes from lane group g the 8
// weights 8g..8g+7 of the block, and each load of a wave is one contiguous
// 256- or 1024-byte run.  The bytes are the row layout's, regrouped.
__global__ __launch_bounds__(256) void q8_tile_kernel(uint4* __restrict__ dst, const uint8_t* __restrict__ src,
                                                      int M, int K, int ngrp, int64_t units) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    const int64_t tb = u / (Q8_TB / 16);
    const int w = (int)(u - tb * (Q8_TB / 16));
    const int64_t tile = tb / ngrp;
    const int kb = (int)(tb - tile * ngrp);
    const int nb32 = K / Q8_ELEMS;
    union { uint4 v; uint8_t b[16]; } o;
    if (w < 16) {
        const int64_t row = tile * 16 + w;
        for (int t = 0; t < 8; ++t) {
            const int blk = kb * 8 + t;
            const bool in = row < M && blk < nb32;
            const uint8_t* p = src + (row * nb32 + blk) * Q8_BYTES;
            o.b[2 * t] = in ? p[0] : 0;
            o.b[2 * t + 1] = in ? p[1] : 0;
        }
    } else {
        const int c = (w - 16) >> 6, l = (w - 16) & 63;
        const int j = l & 15, g = l >> 4;
        const int64_t row = tile * 16 + j;
        for (int h = 0; h < 2; ++h) {
            const int blk = kb * 8 + 2 * c + h;
            const bool in = row < M && blk < nb32;
            const uint8_t* p = src + (row * nb32 + blk) * Q8_BYTES + 2 + 8 * g;
            for (int e = 0; e < 8; ++e) o.b[8 * h + e] = in ? p[e] : 0;
        }
    }
    dst[u] = o.v;
}

size_t q8_tiled_bytes(int M, int K) { return (size_t)((M + 15) / 16) * q8_groups(K) * Q8_TB; }

int launch_q8_tile(void* dst, const void* src, int M, int K, hipStream_t s) {
    const int ngrp = q8_groups(K);
    const int64_t units = (int64_t)((M + 15) / 16) * ngrp * (Q8_TB / 16);
    if (units == 0) return 0;
    hipLaunchKernelGGL(q8_tile_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, s, (uint4*)dst,
                       (const uint8_t*)src, M, K, ngrp, units);
    SH_CHECK_LAUNCH();
    return 0;
}

void q8_untile_host(uint8_t* dst, const uint8_t* src, int M, int K) {
    const int ngrp = q8_groups(K), nb32 = K / Q8_ELEMS;
    for (int64_t row = 0; row < M; ++row) {
        const int64_t tile = row / 16;
        const int j = (int)(row % 16);
        for (int blk = 0; blk < nb32; ++blk) {
            const int kb = blk / 8, t = blk % 8, c = t / 2, h = t % 2;
            const uint8_t* tb = src + (tile * ngrp + kb) * Q8_TB;
            uint8_t* b = dst + (row * nb32 + blk) * Q8_BYTES;
            b[0] = tb[16 * j + 2 * t];
            b[1] = tb[16 * j + 2 * t + 1];
            for (int g = 0; g < 4; ++g)
                for (int e = 0; e < 8; ++e) b[2 + 8 * g + e] = tb[256 + 1024 * c + 16 * (16 * g + j) + 8 * h + e];
        }
    }
}

// ---------------------------------------------------------------------------
// Activation operand.  Tile rt's group kb occupies ACT8_UNITS 16-byte units
// at frag + (rt * q8_groups(K) + kb) * ACT8_UNITS, in MFMA lane order
// (lane = 16 g + j: row j of the tile, lane group g):
//   unit (2t + h) * 64 + lane : x*s hi (h = 0) / lo (h = 1), elements
//                               32t + 8g .. +7 of the group
//   units 1024 .. 1027        : 1/s of rows 0..15 (f32); 1028.. padding
// Each 256-element group of a row has its own exact power-of-two scale s
// with max|x| * s in [2^14, 2^15); x*s = hi + lo.  Elements past K are 0.
typedef _Float16 act8_half4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void act8_kernel(Act8 a, const float* __restrict__ X, int64_t ldx) {
    const int lane = threadIdx.x & 63;
    const int kb = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ngrp = q8_groups(a.K);
    if (kb >= ngrp) return;                       // whole wave; no barriers below
    const int r = blockIdx.y;
    const int e = kb * Q8_GROUP + 4 * lane;       // K % 32 == 0: all four in or all out
    const float4 v = (r < a.rows && e < a.K) ? *(const float4*)(X + (size_t)r * ldx + e)
                                             : make_float4(0.f, 0.f, 0.f, 0.f);
    const float mx = wave_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    int ex = 0;
    if (mx > 0.f && isfinite(mx)) {
        frexpf(mx, &ex);                          // mx = m * 2^ex, m in [0.5, 1)
        ex = 15 - ex;
        ex = ex > 100 ? 100 : (ex < -100 ? -100 : ex);
    }
    const float sc = ldexpf(1.0f, ex);
    const float vv[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
    act8_half4_t h, l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = (_Float16)vv[i];
        l[i] = (_Float16)(vv[i] - (float)h[i]);
    }
    const int rr = r & 15;
    uint8_t* fb = (uint8_t*)a.frag + ((size_t)(r >> 4) * ngrp + kb) * ACT8_UNITS * 16;
    // elements 4 lane .. +3: block t = lane / 8, lane group (lane / 2) % 4,
    // first or second half of the unit by lane parity
    const int t = lane >> 3, g = (lane >> 1) & 3, half_off = 8 * (lane & 1);
    *(act8_half4_t*)(fb + ((2 * t) * 64 + 16 * g + rr) * 16 + half_off) = h;
    *(act8_half4_t*)(fb + ((2 * t + 1) * 64 + 16 * g + rr) * 16 + half_off) = l;
    if (lane == 0) *(float*)(fb + 1024 * 16 + 4 * rr) = ldexpf(1.0f, -ex);
}

int launch_act8_from_f32(const Act8& a, const float* X, int64_t ldx, hipStream_t s) {
    const int ngrp = q8_groups(a.K);
    if (ngrp <= 0 || a.rows_pad <= 0) return 0;
    if (!a.frag || a.rows_pad % 16 || a.K % Q8_ELEMS) { set_error(-1, "act8: bad operand buffer"); return -1; }
    if ((uintptr_t)X % 16 || ldx % 4) { set_error(-1, "act8: rows must be 16-byte aligned"); return -1; }
    hipLaunchKernelGGL(act8_kernel, dim3((ngrp + 3) / 4, a.rows_pad), dim3(256), 0, s, a, X, ldx);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Q8_0 matmul on MFMA.
//
// Y[b, m] = sum_k X[b, k] * W[m, k].  Per 32-element K step t (one Q8_0
// block of every weight row):
//   A (16 act rows x 32 k)    = x*s as f16 hi and lo (two MFMAs)
//   B (32 k x 16 weight rows) = q, exact in f16 (from 1152 + q by v_perm and
//                               one exact subtraction)
// and the step's f32 result is scaled by the row's d and accumulated; each
// 256-element group's sum is scaled by the activation rows' 1/s.  D[i][j]
// (16x16 f32) sits in lane (j, g) as activation rows 4g..4g+3 of weight row j.
//
// A workgroup of WAVES waves owns WAVES*R weight tiles (of up to three fused
// tensors), NT activation tiles and one split of groups.  Per group, the NT
// activation tiles are copied into one of two LDS buffers by direct
// global->LDS loads a group ahead, issued before the next group's weight
// loads; each wave holds its R weight tiles in registers, loaded a group
// ahead into the second of two register sets; each step ends with one wait
// for all loads and one barrier.  W and act are not __restrict__: loads
// through restrict pointers count as invariant and may be moved across the
// barriers that order them here.
struct Q8W { uint4 d, q[4]; };

__device__ __forceinline__ void load_q8w(Q8W& w, const uint8_t* tb, int lane) {
    w.d = *(const uint4*)(tb + 16 * (lane & 15));
#pragma unroll
    for (int c = 0; c < 4; ++c) w.q[c] = *(const uint4*)(tb + 256 + 1024 * c + 16 * lane);
}

// B operand of step t: the 8 int8 weights as f16 (1024 + (q + 128) - 1152).
__device__ __forceinline__ half8_t q8_bop(const Q8W& w, int t) {
    const uint4 Q = w.q[t >> 1];
    const uint32_t w0 = ((t & 1) ? Q.z : Q.x) ^ 0x80808080u;
    const uint32_t w1 = ((t & 1) ? Q.w : Q.y) ^ 0x80808080u;
    const half2_t k = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const half2_t p0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u)) + k;
    const half2_t p1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u)) + k;
    const half2_t p2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u)) + k;
    const half2_t p3 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u)) + k;
    return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

__device__ __forceinline__ float q8_d(const Q8W& w, int t) {
    const uint4 D = w.d;
    const uint32_t v = (t >> 1) == 0 ? D.x : ((t >> 1) == 1 ? D.y : ((t >> 1) == 2 ? D.z : D.w));
    return f16_to_f32_hw((t & 1) ? (v >> 16) : (v & 0xffffu));
}

template <int R, int NT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void q8_mm_kernel(Q4kTargets tg, const uint4* act, int act_tiles,
                                                          float* __restrict__ out, int64_t ldo,
                                                          int64_t split_stride, int ngrp, int bps) {
    __shared__ uint4 s_act[2 * NT * ACT8_UNITS];
    constexpr int TCH = ACT8_UNITS / 64;              // 1 KiB wave copies per tile and group
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // SGPR: scalar tensor and address math
    const int grp = blockIdx.x * WAVES + wv;
    const int ti = (tg.n > 2 && grp >= tg.grp0[2]) ? 2 : ((tg.n > 1 && grp >= tg.grp0[1]) ? 1 : 0);
    const uint8_t* W = ti == 2 ? tg.w[2] : (ti == 1 ? tg.w[1] : tg.w[0]);
    const int M = ti == 2 ? tg.M[2] : (ti == 1 ? tg.M[1] : tg.M[0]);
    const int col = ti == 2 ? tg.col[2] : (ti == 1 ? tg.col[1] : tg.col[0]);
    const int g0 = ti == 2 ? tg.grp0[2] : (ti == 1 ? tg.grp0[1] : tg.grp0[0]);
    const int tiles = (M + 15) / 16;
    const int tile0 = (grp - g0) * R;
    // waves past the last tile still stage activations and meet the barriers
    const bool active = grp < tg.grp_end && tile0 < tiles;
    const int at0 = blockIdx.z * NT;
    const int nt = min(NT, act_tiles - at0);          // >= 1: the launcher sizes the grid
    const int kb0 = blockIdx.y * bps;
    const int nb = min(kb0 + bps, ngrp) - kb0;
    float* o = out + (int64_t)blockIdx.y * split_stride + col;
    if (nb <= 0) {
        // a forced split count can leave trailing splits without groups:
        // their partials are zero (the whole workgroup leaves here)
        if (active) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = (tile0 + r) * 16 + j;
                if (tile0 + r < tiles && row < M)
                    for (int n = 0; n < nt; ++n)
#pragma unroll
                        for (int i = 0; i < 4; ++i) o[(int64_t)((at0 + n) * 16 + 4 * g + i) * ldo + row] = 0.f;
            }
        }
        return;
    }
    const uint8_t* wp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wp[r] = W + (size_t)min(tile0 + r, tiles - 1) * ngrp * Q8_TB;
    auto ldw = [&](Q8W& w, int r, int kb) { load_q8w(w, wp[r] + (size_t)kb * Q8_TB, lane); };
    // copy group kb's units of the nt tiles (kb < ngrp: inside the buffer)
    const uint32_t o_act = 16 * lane;
    auto stage = [&](uint4* dst, int kb) {
        for (int c = wv; c < nt * TCH; c += WAVES) {
            const int n = c / TCH, u = (c - n * TCH) * 64;
            lds_copy16(act + ((size_t)(at0 + n) * ngrp + kb) * ACT8_UNITS + u, o_act, lds_addr(dst + n * ACT8_UNITS + u));
        }
    };
    Q8W w0[R], w1[R];
    floatx4 acc[R][NT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};

    stage(s_act, kb0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < R; ++r) ldw(w0[r], r, kb0);
    __builtin_amdgcn_sched_barrier(0);
    SH_WAIT_VMCNT(0);
    __syncthreads();
    // group b from wc (landed) while wn receives group b+1; the two register
    // sets swap roles each step (the loop is unrolled by two)
    auto step = [&](const Q8W (&wc)[R], Q8W (&wn)[R], int b) {
        const uint4* cur = s_act + (b & 1) * NT * ACT8_UNITS;
        const int kn = kb0 + min(b + 1, nb - 1);
        if (b + 1 < nb) stage(s_act + ((b + 1) & 1) * NT * ACT8_UNITS, kn);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < R; ++r) ldw(wn[r], r, kn);   // unconditional (clamped) prefetch
        __builtin_amdgcn_sched_barrier(0);
        if (active) {
            floatx4 blk[R][NT];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int n = 0; n < NT; ++n) blk[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                half8_t B[R];
                float d[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    B[r] = q8_bop(wc[r], t);
                    d[r] = q8_d(wc[r], t);
                }
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    if (n < nt) {
                        const half8_t h = __builtin_bit_cast(half8_t, cur[n * ACT8_UNITS + (2 * t) * 64 + lane]);
                        const half8_t l = __builtin_bit_cast(half8_t, cur[n * ACT8_UNITS + (2 * t + 1) * 64 + lane]);
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            floatx4 am = {0.f, 0.f, 0.f, 0.f};
                            am = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, B[r], am, 0, 0, 0);
                            am = __builtin_amdgcn_mfma_f32_16x16x32_f16(l, B[r], am, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 4; ++i) blk[r][n][i] = fmaf(d[r], am[i], blk[r][n][i]);
                        }
                    }
                }
            }
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                if (n < nt) {
                    const float4 rv = __builtin_bit_cast(float4, cur[n * ACT8_UNITS + 1024 + g]);
                    const floatx4 rs = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[r][n][i] = fmaf(blk[r][n][i], rs[i], acc[r][n][i]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        SH_WAIT_VMCNT(0);                              // next group's units and weights have landed
        __syncthreads();
    };
    int b = 0;
    for (; b + 2 <= nb; b += 2) {
        step(w0, w1, b);
        step(w1, w0, b + 1);
    }
    if (b < nb) step(w0, w1, b);
    if (!active) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = (tile0 + r) * 16 + j;
        if (tile0 + r < tiles && row < M) {
#pragma unroll
            for (int n = 0; n < NT; ++n)
                if (n < nt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[(int64_t)((at0 + n) * 16 + 4 * g + i) * ldo + row] = acc[r][n][i];
        }
    }
}

static int cu_count() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

template <int R, int NT, int WAVES>
static void launch_mm(const Q4kTargets& tg, const Act8& a, float* out, int64_t ldo, int64_t ss, int ngrp,
                      int bps, int nsplit, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    const int act_tiles = a.rows_pad / 16;
    dim3 grid((tg.grp_end + WAVES - 1) / WAVES, nsplit, (act_tiles + NT - 1) / NT);
    SH_LAUNCH(e0, e1, (q8_mm_kernel<R, NT, WAVES>), grid, dim3(64 * WAVES), 0, s, tg, (const uint4*)a.frag,
              act_tiles, out, ldo, ss, ngrp, bps);
}

// Wave groups of R tiles per tensor, as kernel arguments.
static Q4kTargets q8_targets(const Q4kTarget* t, int n, int R) {
    Q4kTargets tg{};
    int grp = 0;
    for (int i = 0; i < n; ++i) {
        tg.w[i] = (const uint8_t*)t[i].w;
        tg.M[i] = t[i].M;
        tg.col[i] = (int)t[i].col;
        tg.grp0[i] = grp;
        grp += ((t[i].M + 15) / 16 + R - 1) / R;
    }
    tg.n = n;
    tg.grp_end = grp;
    return tg;
}

// Plan: one activation tile -> four-wave workgroups and the largest R in
// {2, 1} (R = 4 only when forced), then the fewest splits, reaching `target`
// workgroups (about two per CU); more tiles -> eight-wave workgroups of R = 2 over NT = 4 (or 2)
// activation tiles, splits as long as they fill the chip.  Splits keep >= 2
// groups each unless forced.
int launch_q8(const Q4kTarget* t, int n, const Act8& a, float* out, int64_t ldo, int64_t split_stride,
              int max_splits, int fixed_splits, int* S_out, hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop) {
    if (n < 1 || n > 3) { set_error(-1, "q8_0: 1..3 fused tensors"); return -1; }
    const int ngrp = q8_groups(a.K);
    if (ngrp < 1 || a.K % Q8_ELEMS) { set_error(-1, "q8_0: K=%d", a.K); return -1; }
    if (!a.frag || a.rows_pad < 16 || a.rows_pad % 16) { set_error(-1, "q8_0: bad operand buffer"); return -1; }
    if (max_splits < 1) max_splits = 1;
    const int act_tiles = a.rows_pad / 16;
    const int target = knobs().q8_wgs;
    const int R_env = knobs().q8_r;
    const int S_env = knobs().q8_s;
    int s_cap = std::min(max_splits, std::max(1, ngrp / 2));
    int R = 2, S = 1;
    if (act_tiles == 1) {
        // R = 2 before R = 1: measured ahead of R = 4 (more groups per split
        // beat more tiles per wave at these sizes)
        bool done = false;
        for (int r = R_env == 4 ? 4 : 2; r >= 1 && !done; r >>= 1) {
            if ((R_env == 1 || R_env == 2 || R_env == 4) && r != R_env) continue;
            int groups = 0;
            for (int i = 0; i < n; ++i) groups += ((t[i].M + 15) / 16 + r - 1) / r;
            R = r;
            for (int c = 1; c <= s_cap; c *= 2) {
                S = c;
                if ((groups + 3) / 4 * c >= target) { done = true; break; }
            }
        }
    } else {
        // the split count that minimises rounds of workgroups x (groups per
        // workgroup + a fixed cost of about four groups per workgroup), a
        // last, partly filled round costing a whole one (the Q4_K prompt
        // planner's model)
        const int NT = act_tiles >= 4 ? 4 : 2;
        const int tasks = (q8_targets(t, n, 2).grp_end + 7) / 8 * ((act_tiles + NT - 1) / NT);
        const int per_cu = (160 * 1024) / (2 * NT * ACT8_UNITS * 16);
        const int slots = cu_count() * std::max(1, per_cu);
        double best = 1e30;
        for (int c = 1; c <= 16 && c <= s_cap; c *= 2) {
            const double cost = (double)((tasks * c + slots - 1) / slots) * ((double)(ngrp + c - 1) / c + 4.0);
            if (cost < best - 1e-9) { best = cost; S = c; }
        }
    }
    if (S_env > 0) S = std::min(S_env, s_cap);
    int bps = (ngrp + S - 1) / S;
    S = (ngrp + bps - 1) / bps;
    if (fixed_splits > 0) {
        S = fixed_splits;
        bps = std::max(1, (ngrp + S - 1) / S);
    }
    const Q4kTargets tg = q8_targets(t, n, act_tiles == 1 ? R : 2);
    if (act_tiles == 1) {
        if (R == 4) launch_mm<4, 1, 4>(tg, a, out, ldo, split_stride, ngrp, bps, S, s, ev_start, ev_stop);
        else if (R == 2) launch_mm<2, 1, 4>(tg, a, out, ldo, split_stride, ngrp, bps, S, s, ev_start, ev_stop);
        else launch_mm<1, 1, 4>(tg, a, out, ldo, split_stride, ngrp, bps, S, s, ev_start, ev_stop);
    } else if (act_tiles >= 4) {
        launch_mm<2, 4, 8>(tg, a, out, ldo, split_stride, ngrp, bps, S, s, ev_start, ev_stop);
    } else {
        launch_mm<2, 2, 8>(tg, a, out, ldo, split_stride, ngrp, bps, S, s, ev_start, ev_stop);
    }
    SH_CHECK_LAUNCH();
    *S_out = S;
    return 0;
}

}  // namespace slate_hip
