// k_q4k.hip -- Q4_K kernels for gfx950: bit-exact dequant, activation split,
// and the dequant-fused MFMA matmul used for decode and small-batch steps.
//
// Q4_K super-block (src/util/quant.c:135-166): 144 bytes = f16 d, f16 dmin,
// 12 bytes of packed 6-bit (scale, min) for 8 sub-blocks, 128 bytes of
// nibbles.  Slate's nibble order: sub-block s owns qs[16s..16s+15]; the low
// nibble of byte i is element i, the high nibble element i+16.
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "launch.h"
#include "lanes.h"
#include "act16.h"
#include "mfma.h"
#include "q4k.h"

namespace slate_hip {

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
// Activation operand from f32 rows (layout and scaling in act16.h): one wave
// per 256-element block of a row.
__global__ __launch_bounds__(256) void act16_kernel(Act16 a, const float* __restrict__ X, int64_t ldx) {
    const int lane = threadIdx.x & 63;
    const int kb = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nblk = a.K / QK;
    if (kb >= nblk) return;                       // whole wave; no barriers below
    const int r = blockIdx.y;
    const float4 v = r < a.rows ? *(const float4*)(X + (size_t)r * ldx + (size_t)kb * QK + 4 * lane)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
    act16_store_block(a, r, kb, lane, v);
}

// The same conversion by 8-row half tiles (act16_store_tile): a workgroup
// per (block, half tile), wave w = row w of the half.
__global__ __launch_bounds__(512) void act16_tile_kernel(Act16 a, const float* __restrict__ X, int64_t ldx) {
    __shared__ uint4 s_t[ACT_FRAG_UNITS];
    const int kb = blockIdx.x;
    const int r = blockIdx.y * 8 + (threadIdx.x >> 6);
    const float4 v = r < a.rows ? *(const float4*)(X + (size_t)r * ldx + (size_t)kb * QK + 4 * (threadIdx.x & 63))
                                : make_float4(0.f, 0.f, 0.f, 0.f);
    act16_store_tile<8>(a, blockIdx.y >> 1, blockIdx.y & 1, kb, s_t, v);
}

int launch_act16_from_f32(const Act16& a, const float* X, int64_t ldx, hipStream_t s) {
    const int nblk = a.K / QK;
    if (nblk <= 0 || a.rows_pad <= 0) return 0;
    if (!a.frag || a.rows_pad % 16) { set_error(-1, "act16: bad operand buffer"); return -1; }
    if (a.rows_pad > 16)
        hipLaunchKernelGGL(act16_tile_kernel, dim3(nblk, a.rows_pad / 8), dim3(512), 0, s, a, X, ldx);
    else
        hipLaunchKernelGGL(act16_kernel, dim3((nblk + 3) / 4, a.rows_pad), dim3(256), 0, s, a, X, ldx);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Dequant-fused Q4_K matmul on MFMA.
//
// Y[b, m] = sum_k X[b, k] * W[m, k].  One wave owns 16-row weight tiles and
// a range of super-blocks.  Per super-block and 32-element K step:
//   A (16 act rows x 32 k)   = x*s split into f16 hi and lo (two MFMAs)
//   B (32 k x 16 weight rows) = q * sc, exact in f16 (q <= 15, sc <= 63)
// so sum_s sc_s * sum q*x accumulates in f32 inside the MFMA, and is scaled
// by d (and the block's 1/s) once per super-block.  The min term
// dmin * sum_s mn_s * sum_{i in s} x runs as a 16x16x16 MFMA of the
// per-sub-block sums against mn (exact).
//
// Lane l: j = l & 15 (weight row of B / activation row of A), g = l >> 4.
// In step t (0..7) lane group g covers block-local k = 64g + 8t + e, e < 8,
// i.e. sub-block 2g + t/4, elements 8(t%4)..8(t%4)+7: the low nibbles of
// bytes 0..7 / 8..15 for t%4 = 0 / 1, the high nibbles for t%4 = 2 / 3.
// D[i][j] (16x16 f32) sits in lane (j, g) as rows 4g..4g+3.
//
// Weight layouts:
//   ROW    slate's own: row m is K/256 consecutive 144-byte blocks.
//   TILED  16-row tiles (rows past M zero), tile t's block kb is 2304
//          contiguous bytes at (t * K/256 + kb) * 2304: the 16 rows' 16-byte
//          headers (d, dmin, scales), then for each lane l the 16 bytes
//          qs[32g .. 32g+15] of row j, then qs[32g+16 .. 32g+31].  Every load
//          of a wave is one contiguous 256- or 1024-byte run.
struct WTile { uint4 hdr, qa, qb; };

__device__ __forceinline__ void load_wtile(WTile& w, const uint8_t* blk, int g) {
    w.hdr = *(const uint4*)blk;
    w.qa = *(const uint4*)(blk + 16 + 32 * g);
    w.qb = *(const uint4*)(blk + 32 + 32 * g);
}

__device__ __forceinline__ void load_wtile_tiled(WTile& w, const uint8_t* tb, int lane) {
    w.hdr = *(const uint4*)(tb + 16 * (lane & 15));
    w.qa = *(const uint4*)(tb + 256 + 16 * lane);
    w.qb = *(const uint4*)(tb + 1280 + 16 * lane);
}

// Per-block constants of one weight tile for lane group g: the f16 fma
// terms that turn nibbles into q * sc (low nibble: 1024+q -> (1024+q)*sc -
// 1024*sc; high nibble: 1024+16q -> (1024+16q)*(sc/16) - 64*sc), the
// sub-block mins as the min-term operand, d and 64 * dmin.  Each half2 holds
// sub-block 2g in .x and 2g+1 in .y; the B-operand fma broadcasts one half.
struct WScale { half2_t sc, lo_add, hi_mul, hi_add; half4_t bmin; float d, dmin64; };

__device__ __forceinline__ WScale q4k_wscale(const WTile& w, int g) {
    WScale c;
    ScaleBytes sb = unpack_scales(w.hdr.y, w.hdr.z, w.hdr.w);
    const uint32_t scw = g < 2 ? sb.sc_lo : sb.sc_hi;
    // bytes 2(g&1), 2(g&1)+1 as 1024 + sc in f16, minus 1024 (exact)
    const uint32_t sel = (g & 1) ? 0x04030402u : 0x04010400u;
    const half2_t k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    c.sc = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, scw, sel)) + k1024;
    c.lo_add = c.sc * (_Float16)-1024.0f;
    c.hi_mul = c.sc * (_Float16)0.0625f;
    c.hi_add = c.sc * (_Float16)-64.0f;
    // mins of sub-blocks 4(g&1) .. +3: lane groups 0, 1 meet the hi halves of
    // the activation sub-block sums, groups 2, 3 the lo halves (act16.h)
    const uint32_t mw = (g & 1) ? sb.mn_hi : sb.mn_lo;
    const half2_t m01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, mw, 0x04010400u)) + k1024;
    const half2_t m23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, mw, 0x04030402u)) + k1024;
    c.bmin = half4_t{m01.x, m01.y, m23.x, m23.y};
    c.d = f16_to_f32_hw(w.hdr.x & 0xffffu);
    c.dmin64 = f16_to_f32_hw(w.hdr.x >> 16) * 64.0f;
    return c;
}

// B operand of K step t: q * sc exact in f16 (q <= 15, sc <= 63), built
// from 1024+q (low nibble) or 1024+16q (high nibble) by one v_and_or per
// two values (the nibbles of bytes 0 and 2 of a dword, then of bytes 1 and
// 3 after an 8-bit shift that the low- and high-nibble steps share) and one
// exact fma.  Element order within the lane's 8 values: 0, 2, 1, 3, 4, 6,
// 5, 7 -- the activation operand is stored in the same order (act16.h).
// (x & m) | k in one v_and_or_b32 (the compiler splits it when m and k are
// both literals: one VOP3 instruction takes one literal); m in an SGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t k) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(k));
    return r;
}

__device__ __forceinline__ half8_t q4k_bop(const WTile& w, const WScale& c, int t) {
    const uint4 Q = t < 4 ? w.qa : w.qb;
    const int tq = t & 3;
    const uint32_t q0 = (tq & 1) ? Q.z : Q.x;
    const uint32_t q1 = (tq & 1) ? Q.w : Q.y;
    const uint32_t mask = (tq & 2) ? 0x00f000f0u : 0x000f000fu;
    const uint32_t k1024 = 0x64006400u;
    const half2_t mv = (tq & 2) ? c.hi_mul : c.sc;
    const half2_t av = (tq & 2) ? c.hi_add : c.lo_add;
    const _Float16 m = t < 4 ? mv.x : mv.y, a = t < 4 ? av.x : av.y;
    const half2_t mul = {m, m}, add = {a, a};
    half2_t p0 = __builtin_bit_cast(half2_t, and_or(q0, mask, k1024));
    half2_t p1 = __builtin_bit_cast(half2_t, and_or(q0 >> 8, mask, k1024));
    half2_t p2 = __builtin_bit_cast(half2_t, and_or(q1, mask, k1024));
    half2_t p3 = __builtin_bit_cast(half2_t, and_or(q1 >> 8, mask, k1024));
    p0 = __builtin_elementwise_fma(p0, mul, add);
    p1 = __builtin_elementwise_fma(p1, mul, add);
    p2 = __builtin_elementwise_fma(p2, mul, add);
    p3 = __builtin_elementwise_fma(p3, mul, add);
    return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// Decode kernel (NT = 1 or 2 16-row activation tiles: up to 32 rows).  A
// workgroup of WAVES waves owns WAVES*R weight tiles (possibly spread over
// up to three fused tensors) and one split of super-blocks.  The NT tiles'
// activation units of a block are copied into a double-buffered LDS area by
// direct global->LDS loads, one block ahead and issued after the next
// block's weight loads; each wave holds its R weight tiles in registers,
// loaded one block ahead, and builds each tile's B operand once per K step
// for all NT activation tiles; every step ends with one wait for all loads
// and one barrier.  W and frag are not __restrict__: loads through restrict
// pointers count as invariant and may be moved across the barriers that
// order them here.
//
// CONV (one activation tile; the C ABI's matmuls of 2-16 rows): the operand
// is not read from a buffer but made in the kernel from the f32 rows X (ldx
// floats apart, rows >= xrows zero): each wave loads two rows of the next
// block into registers before computing the current one, and after it
// writes them into the other LDS buffer in the operand layout (act16.h), the
// same values the operand kernel would write.
template <int R, bool TILED, int WAVES = 4, int NT = 1, bool CONV = false>
__global__ __launch_bounds__(64 * WAVES) void q4k_dec_kernel(Q4kTargets tg, const uint4* frag,
                                                             float* __restrict__ out, int64_t ldo,
                                                             int64_t split_stride, int nblk, int bps, int early,
                                                             const float* X = nullptr, int64_t ldx = 0,
                                                             int xrows = 0) {
    static_assert(!CONV || (NT == 1 && WAVES == 8), "CONV: one activation tile, two rows per wave");
    __shared__ uint4 s_act[2 * NT * ACT_FRAG_UNITS];
    constexpr int TCH = ACT_FRAG_UNITS / 64;          // 1 KiB wave copies per tile and block
    constexpr int CHUNKS = NT * TCH;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int j = lane & 15;
    const int g = lane >> 4;
    // wave-uniform (SGPR): the tensor selection and every weight and operand
    // base address below are scalar; loads add the lane's offset
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
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
    const int kb0 = blockIdx.y * bps;
    const int nb = min(kb0 + bps, nblk) - kb0;        // >= 1: the launcher sizes the grid
    const uint8_t* wp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int t = min(tile0 + r, tiles - 1);
        wp[r] = TILED ? W + (size_t)t * nblk * (16 * QBLOCK) : W + (size_t)min(t * 16 + j, M - 1) * nblk * QBLOCK;
    }
    auto ldw = [&](WTile& w, int r, int kb) {
        if (TILED) load_wtile_tiled(w, wp[r] + (size_t)kb * (16 * QBLOCK), lane);
        else load_wtile(w, wp[r] + (size_t)kb * QBLOCK, g);
    };
    // copy block kb's units of the NT tiles (kb < nblk: inside the operand
    // buffer, tile n's block at (n * nblk + kb) units) into dst
    const uint32_t o_act = 16 * lane;
    auto stage = [&](uint4* dst, int kb) {
#pragma unroll
        for (int i = 0; i < (CHUNKS + WAVES - 1) / WAVES; ++i) {
            const int c = wv + WAVES * i;
            if (c < CHUNKS) {
                const int n = c / TCH, u = (c - n * TCH) * 64;
                lds_copy16(frag + ((size_t)n * nblk + kb) * ACT_FRAG_UNITS + u, o_act,
                           lds_addr(dst + n * ACT_FRAG_UNITS + u));
            }
        }
    };
    WTile w0[R], w1[R];
    floatx4 acc[R][NT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};

    // a block's products from the landed weights wc and operand buffer slot
    auto compute = [&](const WTile (&wc)[R], int slot) {
        const uint4* cur = s_act + slot * NT * ACT_FRAG_UNITS;
        if (active) {
            // one K step at a time: each tile's B operand is built once and
            // run against the NT activation fragments of the step
            WScale cs[R];
            floatx4 am[R][NT];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                cs[r] = q4k_wscale(wc[r], g);
#pragma unroll
                for (int n = 0; n < NT; ++n) am[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                half8_t bop[R];
#pragma unroll
                for (int r = 0; r < R; ++r) bop[r] = q4k_bop(wc[r], cs[r], t);
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const uint4* sa = cur + n * ACT_FRAG_UNITS;
                    const half8_t h = __builtin_bit_cast(half8_t, sa[(2 * t) * 64 + lane]);
                    const half8_t l = __builtin_bit_cast(half8_t, sa[(2 * t + 1) * 64 + lane]);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        am[r][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, bop[r], am[r][n], 0, 0, 0);
                        am[r][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(l, bop[r], am[r][n], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const uint4* sa = cur + n * ACT_FRAG_UNITS;
                const half4_t ys = *(const half4_t*)(sa + 1024 + lane);
                const float4 rv = __builtin_bit_cast(float4, sa[1088 + g]);
                const floatx4 rs = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    floatx4 an = {0.f, 0.f, 0.f, 0.f};
                    an = __builtin_amdgcn_mfma_f32_16x16x16f16(ys, cs[r].bmin, an, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[r][n][i] += (cs[r].d * am[r][n][i] - cs[r].dmin64 * an[i]) * rs[i];
                }
            }
        }
    };
    // block b (< nb): weights into w, operand units into buffer b & 1
    auto issue = [&](WTile (&w)[R], int b) {
#pragma unroll
        for (int r = 0; r < R; ++r) ldw(w[r], r, kb0 + b);
        __builtin_amdgcn_sched_barrier(0);
        stage(s_act + (b & 1) * NT * ACT_FRAG_UNITS, kb0 + b);
        __builtin_amdgcn_sched_barrier(0);
    };
    // block b from wc (landed) while wn receives block b+1; the two register
    // sets swap roles each step (the loop is unrolled by two).  Every step
    // ends with one wait for all loads and one barrier.
    auto step = [&](const WTile (&wc)[R], WTile (&wn)[R], int b) {
        if (b + 1 < nb) issue(wn, b + 1);            // the last block prefetches nothing
        compute(wc, b & 1);
        __builtin_amdgcn_sched_barrier(0);
        SH_WAIT_VMCNT(0);                              // block b+1's units and weights have landed
        __syncthreads();
    };

    // Block 0 is peeled off the loop, so that the loop starts with no load
    // in flight on every path into it: the compiler then places no wait of
    // its own inside the loop (a path into the loop with loads in flight
    // makes it wait, in every step, for loads issued in that same step).
    // With `early` block 1 goes out together with block 0 (its index
    // clamped to the last block, so the loads are unconditional and the
    // first wait has one count): both blocks' operand units, block 0's
    // weights, then block 1's; the first wait leaves block 1's weight loads
    // in flight (loads complete in order) while block 0 is computed.
    if constexpr (CONV) {
        // rows 2*wv, 2*wv + 1 of block kb into registers, then into buffer dst
        float4 xr[2];
        auto xload = [&](int kb) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = 2 * wv + i;
                xr[i] = r < xrows ? *(const float4*)(X + (int64_t)r * ldx + (int64_t)kb * QK + 4 * lane)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        };
        auto xstore = [&](uint4* dst) {
#pragma unroll
            for (int i = 0; i < 2; ++i) act16_store_tile_row((uint8_t*)dst, 2 * wv + i, lane, xr[i]);
        };
        xload(kb0);
#pragma unroll
        for (int r = 0; r < R; ++r) ldw(w0[r], r, kb0);
        xstore(s_act);
        SH_WAIT_VMCNT(0);
        __syncthreads();
        for (int b = 0; b < nb; ++b) {
            const bool more = b + 1 < nb;
            if (more) {
                xload(kb0 + b + 1);
#pragma unroll
                for (int r = 0; r < R; ++r) ldw(w1[r], r, kb0 + b + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(w0, b & 1);
            __builtin_amdgcn_sched_barrier(0);
            if (more) xstore(s_act + ((b + 1) & 1) * ACT_FRAG_UNITS);
            SH_WAIT_VMCNT(0);
            __syncthreads();
#pragma unroll
            for (int r = 0; r < R; ++r) w0[r] = w1[r];
        }
    } else if (early) {
        const int b1 = nb > 1 ? 1 : 0;
        stage(s_act, kb0);
        stage(s_act + NT * ACT_FRAG_UNITS, kb0 + b1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < R; ++r) ldw(w0[r], r, kb0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < R; ++r) ldw(w1[r], r, kb0 + b1);
        __builtin_amdgcn_sched_barrier(0);
        SH_WAIT_VMCNT(3 * R);
        __syncthreads();
        compute(w0, 0);
        __builtin_amdgcn_sched_barrier(0);
        SH_WAIT_VMCNT(0);
        __syncthreads();
    } else {
        issue(w0, 0);
        SH_WAIT_VMCNT(0);
        __syncthreads();
        step(w0, w1, 0);
    }
    if constexpr (!CONV) {
        int b = 1;
        for (; b + 2 <= nb; b += 2) {
            step(w1, w0, b);
            step(w0, w1, b + 1);
        }
        if (b < nb) step(w1, w0, b);
    }
    if (!active) return;
    float* o = out + (int64_t)blockIdx.y * split_stride + col;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = (tile0 + r) * 16 + j;
        if (tile0 + r < tiles && row < M) {
#pragma unroll
            for (int n = 0; n < NT; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[(int64_t)(16 * n + 4 * g + i) * ldo + row] = acc[r][n][i];
        }
    }
}

// One-row matvec on MFMA over TILED weights (slate_q4_k_matvec,
// quant.c:306-313, for a single activation row; K up to GV1_MAXB blocks).
// A workgroup owns one 16-row weight tile and all of K; wave w takes blocks
// w, w + 8, ... and issues every one of its weight loads before anything
// else.  Meanwhile it turns
// the same blocks of x into the activation operand in LDS (per 256-element
// block a power-of-two scale s, x*s = hi + lo in f16, the order act16.h
// gives a lane group's eight values of a K step) and the f32 sub-block sums
// of x.  The A operand of every MFMA is x in all 16 rows (each lane group
// reads the same 16 bytes: an LDS broadcast), so each output row of the
// 16x16 result holds the same dot product and a lane's first element is its
// weight row's partial.  The block's min term dmin * sum_s mn_s * sum x_s
// runs on the vector ALUs from the row's header.  The eight waves' partials
// are added through LDS in a fixed order, so results are deterministic, and
// one kernel writes the final row: no operand buffer, no split-K partials,
// and ~0.6 VALU operations per weight against ~2.8 for the vector-ALU GEMV
// (measured per call at B = 1 on the tiled layout: 5.6 / 10.9 / 14.4 us at
// 4096x4096 / 14336x4096 / 4096x14336 against 7.7 / 15.9 / 19.4 us).  On
// slate's row layout the lanes' 16-byte pieces of 16 rows scatter over 32
// cache lines per load and the vector-ALU GEMV, which reads whole rows,
// stays faster (11.7 vs 12.2 us at 14336x4096, also with the row pieces
// regrouped through LDS).
constexpr int GV1_WAVES = 8;
constexpr int GV1_MAXB = 64;                          // K <= 16384 (eight blocks per wave)

// LDS of a workgroup for up to GV1_WAVES * BPW blocks: per block the 32 hi
// and 32 lo units (16 bytes each), eight sub-block sums and 1/s; then the
// waves' partials.
__host__ __device__ constexpr size_t gemv1_lds_bytes(int bpw) {
    return (size_t)GV1_WAVES * bpw * (32 * 16 * 2 + 8 * 4 + 4) + GV1_WAVES * 16 * 4;
}

template <int BPW>
__global__ __launch_bounds__(64 * GV1_WAVES) void q4k_gemv1_kernel(const uint8_t* W, int M,
                                                                    const float* __restrict__ x,
                                                                    float* __restrict__ y, int nblk) {
    __shared__ uint4 s_dyn[gemv1_lds_bytes(BPW) / 16];
    uint4* s_hi = s_dyn;                                       // [nblk][32]: step * 4 + lane group
    uint4* s_lo = s_hi + (size_t)nblk * 32;
    float* s_xs = (float*)(s_lo + (size_t)nblk * 32);          // [nblk][8] sub-block sums of x
    float* s_rs = s_xs + (size_t)nblk * 8;                     // [nblk] 1/s
    float* s_red = s_rs + nblk;                                // [waves][16]
    const int lane = threadIdx.x & 63;
    const int j = lane & 15, g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.x;
    // every load of the wave first: its blocks' weights, then its blocks of x
    WTile w[BPW];
    float4 xv[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int kb = wv + GV1_WAVES * i;
        if (kb < nblk) load_wtile_tiled(w[i], W + ((size_t)tile * nblk + kb) * (16 * QBLOCK), lane);
    }
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int kb = wv + GV1_WAVES * i;
        if (kb < nblk) xv[i] = *(const float4*)(x + (size_t)kb * QK + 4 * lane);
    }
    // the activation operand of this wave's blocks (the act16.h layout of one
    // row: lane l holds elements 4l .. 4l+3 of the block)
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int kb = wv + GV1_WAVES * i;
        if (kb < nblk) {
            const float4 v = xv[i];
            const float mx = wave_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            int ex = 0;
            if (mx > 0.f && isfinite(mx)) {
                frexpf(mx, &ex);
                ex = 15 - ex;
                ex = ex > 100 ? 100 : (ex < -100 ? -100 : ex);
            }
            const float sc = ldexpf(1.0f, ex);
            const float vv[4] = {v.x * sc, v.y * sc, v.z * sc, v.w * sc};
            half4_t h, l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h[e] = (_Float16)vv[e];
                l[e] = (_Float16)(vv[e] - (float)h[e]);
            }
            const int unit = kb * 32 + ((lane >> 1) & 7) * 4 + g, off = 8 * (lane & 1);
            *(half4_t*)((uint8_t*)&s_hi[unit] + off) = half4_t{h[0], h[2], h[1], h[3]};
            *(half4_t*)((uint8_t*)&s_lo[unit] + off) = half4_t{l[0], l[2], l[1], l[3]};
            const float sum = group8_sum((v.x + v.y) + (v.z + v.w));
            if ((lane & 7) == 0) s_xs[kb * 8 + (lane >> 3)] = sum;
            if (lane == 0) s_rs[kb] = ldexpf(1.0f, -ex);
        }
    }
    // this wave's blocks only read what this wave wrote: no barrier
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int kb = wv + GV1_WAVES * i;
        if (kb < nblk) {
            const WScale cs = q4k_wscale(w[i], g);
            floatx4 am = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const half8_t b = q4k_bop(w[i], cs, t);
                const half8_t ah = __builtin_bit_cast(half8_t, s_hi[kb * 32 + t * 4 + g]);
                const half8_t al = __builtin_bit_cast(half8_t, s_lo[kb * 32 + t * 4 + g]);
                am = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, am, 0, 0, 0);
                am = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, am, 0, 0, 0);
            }
            // min term of weight row j from its header: dmin * sum_s mn_s * sum x_s
            const ScaleBytes sb = unpack_scales(w[i].hdr.y, w[i].hdr.z, w[i].hdr.w);
            const float4 xa = *(const float4*)&s_xs[kb * 8], xb = *(const float4*)&s_xs[kb * 8 + 4];
            const float mn = (float)(sb.mn_lo & 255u) * xa.x + (float)((sb.mn_lo >> 8) & 255u) * xa.y +
                             (float)((sb.mn_lo >> 16) & 255u) * xa.z + (float)(sb.mn_lo >> 24) * xa.w +
                             (float)(sb.mn_hi & 255u) * xb.x + (float)((sb.mn_hi >> 8) & 255u) * xb.y +
                             (float)((sb.mn_hi >> 16) & 255u) * xb.z + (float)(sb.mn_hi >> 24) * xb.w;
            acc += cs.d * am[0] * s_rs[kb] - cs.dmin64 * (1.0f / 64.0f) * mn;
        }
    }
    if (g == 0) s_red[wv * 16 + j] = acc;
    __syncthreads();
    if (threadIdx.x < 16) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < GV1_WAVES; ++k) v += s_red[k * 16 + threadIdx.x];
        const int row = tile * 16 + (int)threadIdx.x;
        if (row < M) y[row] = v;
    }
}

template <int BPW>
static void launch_gemv1_t(dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const uint8_t* W, int M,
                           const float* x, float* y, int nblk) {
    SH_LAUNCH(e0, e1, (q4k_gemv1_kernel<BPW>), grid, dim3(64 * GV1_WAVES), 0, s, W, M, x, y, nblk);
}

int launch_q4k_gemv1(const void* W, int M, int K, const float* x, float* y, hipStream_t s, hipEvent_t ev_start,
                     hipEvent_t ev_stop) {
    const int nblk = K / QK;
    if (M < 1 || K < QK || K % QK || nblk > GV1_MAXB) {
        set_error(-1, "q4k_gemv1: M=%d, K=%d (K up to %d)", M, K, GV1_MAXB * QK);
        return -1;
    }
    if ((uintptr_t)x & 15) { set_error(-1, "q4k_gemv1: the activation row must be 16-byte aligned"); return -1; }
    const dim3 grid((M + 15) / 16);
    const uint8_t* w = (const uint8_t*)W;
    const int bpw = (nblk + GV1_WAVES - 1) / GV1_WAVES;
    if (bpw <= 2) launch_gemv1_t<2>(grid, s, ev_start, ev_stop, w, M, x, y, nblk);
    else if (bpw <= 4) launch_gemv1_t<4>(grid, s, ev_start, ev_stop, w, M, x, y, nblk);
    else launch_gemv1_t<8>(grid, s, ev_start, ev_stop, w, M, x, y, nblk);
    SH_CHECK_LAUNCH();
    return 0;
}

// Prefill kernel (several 16-row activation tiles).  A workgroup of WAVES
// waves owns WAVES*R weight tiles of one tensor, NT activation tiles and one split
// of super-blocks.  Per block, the NT tiles' activation units are copied into
// one of two LDS buffers by direct global->LDS loads (issued a block ahead,
// before the weight prefetch, so waiting for them leaves the weights in
// flight); each wave dequantises its R weight tiles once and runs them
// against all NT activation tiles.  W and frag are not __restrict__: loads
// through restrict pointers count as invariant and may be moved across the
// barriers that order them here.
template <int R, int NT, bool TILED, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void q4k_pf_kernel(Q4kTargets tg, const uint4* frag, int act_tiles,
                                                     float* __restrict__ out, int64_t ldo,
                                                     int64_t split_stride, int nblk, int bps) {
    __shared__ uint4 s_act[2 * NT * ACT_FRAG_UNITS];
    constexpr int CHUNKS = NT * ACT_FRAG_UNITS / 64;  // 1 KiB wave copies per block
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // SGPR: scalar staging addresses
    __builtin_assume(wv >= 0 && wv < WAVES);
    // workgroup x -> tensor (tensors start on workgroup boundaries)
    const int wg = blockIdx.x;
    const int ti = (tg.n > 2 && wg >= tg.grp0[2]) ? 2 : ((tg.n > 1 && wg >= tg.grp0[1]) ? 1 : 0);
    const uint8_t* W = ti == 2 ? tg.w[2] : (ti == 1 ? tg.w[1] : tg.w[0]);
    const int M = ti == 2 ? tg.M[2] : (ti == 1 ? tg.M[1] : tg.M[0]);
    const int col = ti == 2 ? tg.col[2] : (ti == 1 ? tg.col[1] : tg.col[0]);
    const int wg0 = ti == 2 ? tg.grp0[2] : (ti == 1 ? tg.grp0[1] : tg.grp0[0]);
    const int tiles = (M + 15) / 16;
    const int tile0 = ((wg - wg0) * WAVES + wv) * R;
    const bool active = tile0 < tiles;
    const int at0 = blockIdx.z * NT;
    const int nt = min(NT, act_tiles - at0);          // >= 1; the last group may hold fewer tiles
    const int kb0 = blockIdx.y * bps;
    const int nb = min(kb0 + bps, nblk) - kb0;        // >= 1: the launcher sizes the grid
    const uint8_t* wp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int t = min(tile0 + r, tiles - 1);
        wp[r] = TILED ? W + (size_t)t * nblk * (16 * QBLOCK) : W + (size_t)min(t * 16 + j, M - 1) * nblk * QBLOCK;
    }
    auto ldw = [&](WTile& w, int r, int kb) {
        if (TILED) load_wtile_tiled(w, wp[r] + (size_t)kb * (16 * QBLOCK), lane);
        else load_wtile(w, wp[r] + (size_t)kb * QBLOCK, g);
    };
    // chunks of block kb of activation tiles at0 .. at0+NT-1 (clamped; the
    // last group copies only the tiles it holds): every address stays inside
    // the operand buffer (at < act_tiles, kb < nblk).
    // The wave's chunks sit at fixed byte offsets from block kb's base (the
    // operand buffer of a prompt chunk is far below 4 GiB) and at fixed LDS
    // offsets, computed once: a copy costs one 64-bit scalar add and an m0 add.
    constexpr int NCH = (CHUNKS + WAVES - 1) / WAVES;
    const uint32_t o_act = 16 * lane;
    uint32_t csrc[NCH], clds[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = min(wv + WAVES * i, CHUNKS - 1);
        const int n = c / (ACT_FRAG_UNITS / 64);
        const int u = (c - n * (ACT_FRAG_UNITS / 64)) * 64;
        const int at = min(at0 + n, act_tiles - 1);
        csrc[i] = (uint32_t)(((uint32_t)at * (uint32_t)nblk * ACT_FRAG_UNITS + u) * 16u);
        clds[i] = (uint32_t)((n * ACT_FRAG_UNITS + u) * 16);
    }
    // The block loop, specialised on the number NTA of activation tiles the
    // workgroup holds (NT, or fewer in the last group along z): every loop
    // over the tiles is unrolled with no branch inside the K steps, so the
    // compiler issues the LDS reads of several tiles ahead of their MFMAs and
    // interleaves the next step's B operands with them.  (A per-tile
    // workgroup-uniform branch there splits each K step into one basic block
    // per tile, and each tile's MFMAs then wait behind their own LDS reads.)
    auto run = [&](auto ntag) {
        constexpr int NTA = decltype(ntag)::value;
        constexpr int CH_A = NTA * (ACT_FRAG_UNITS / 64);   // chunks of the NTA tiles
        auto stage_a = [&](uint4* dst, int kb) {
            const char* sb = (const char*)(frag + (size_t)kb * ACT_FRAG_UNITS);
            const uint32_t lb = lds_addr(dst);
#pragma unroll
            for (int i = 0; i < NCH; ++i)
                if (wv + WAVES * i < CH_A) lds_copy16(sb + csrc[i], o_act, lb + clds[i]);
        };
        WTile wc[R], wn[R];
        floatx4 acc[R][NTA];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int n = 0; n < NTA; ++n) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};

        stage_a(s_act, kb0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < R; ++r) ldw(wc[r], r, kb0);
        __builtin_amdgcn_sched_barrier(0);
        SH_WAIT_VMCNT(0);
        __syncthreads();
        // (swapping two register sets instead of copying, as the decode kernel
        // does, costs this kernel 30 more VGPRs and 8 % at T = 320)
        for (int b = 0; b < nb; ++b) {
            // compute block b from one buffer while the other receives block b+1
            const uint4* cur = s_act + (b & 1) * NT * ACT_FRAG_UNITS;
            const int kn = kb0 + min(b + 1, nb - 1);
            if (b + 1 < nb) stage_a(s_act + ((b + 1) & 1) * NT * ACT_FRAG_UNITS, kn);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < R; ++r) ldw(wn[r], r, kn);
            __builtin_amdgcn_sched_barrier(0);
            if (active) {
                // one K step at a time: each tile's B operand is built once and
                // used against every activation tile, so consecutive MFMAs
                // belong to independent accumulators
                WScale cs[R];
                floatx4 am[R][NTA];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    cs[r] = q4k_wscale(wc[r], g);
#pragma unroll
                    for (int n = 0; n < NTA; ++n) am[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
                }
                // the B operands of K step t + 1 are built while step t's MFMAs run
                half8_t bcur[R];
#pragma unroll
                for (int r = 0; r < R; ++r) bcur[r] = q4k_bop(wc[r], cs[r], 0);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    half8_t bnx[R];
                    if (t < 7) {
#pragma unroll
                        for (int r = 0; r < R; ++r) bnx[r] = q4k_bop(wc[r], cs[r], t + 1);
                    }
#pragma unroll
                    for (int n = 0; n < NTA; ++n) {
                        const uint4* sa = cur + n * ACT_FRAG_UNITS;
                        const half8_t h = __builtin_bit_cast(half8_t, sa[(2 * t) * 64 + lane]);
                        const half8_t l = __builtin_bit_cast(half8_t, sa[(2 * t + 1) * 64 + lane]);
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            am[r][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, bcur[r], am[r][n], 0, 0, 0);
                            am[r][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(l, bcur[r], am[r][n], 0, 0, 0);
                        }
                    }
                    if (t < 7) {
#pragma unroll
                        for (int r = 0; r < R; ++r) bcur[r] = bnx[r];
                    }
                }
#pragma unroll
                for (int n = 0; n < NTA; ++n) {
                    const uint4* sa = cur + n * ACT_FRAG_UNITS;
                    const half4_t ys = *(const half4_t*)(sa + 1024 + lane);
                    const float4 rv = __builtin_bit_cast(float4, sa[1088 + g]);
                    const floatx4 rs = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        floatx4 an = {0.f, 0.f, 0.f, 0.f};
                        an = __builtin_amdgcn_mfma_f32_16x16x16f16(ys, cs[r].bmin, an, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            acc[r][n][i] += (cs[r].d * am[r][n][i] - cs[r].dmin64 * an[i]) * rs[i];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // the next block's units and weights have landed: waiting for the
            // weights here (not at their first use) keeps the compiler's in-order
            // load counting from also waiting on the next step's LDS copies
            SH_WAIT_VMCNT(0);
            __syncthreads();
#pragma unroll
            for (int r = 0; r < R; ++r) wc[r] = wn[r];
        }
        if (!active) return;
        float* o = out + (int64_t)blockIdx.y * split_stride + col;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = (tile0 + r) * 16 + j;
            if (tile0 + r >= tiles || row >= M) continue;
#pragma unroll
            for (int n = 0; n < NTA; ++n)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[(int64_t)((at0 + n) * 16 + 4 * g + i) * ldo + row] = acc[r][n][i];
        }
    };
    // nt is the same for the whole workgroup (blockIdx.z); the barriers
    // inside run() are reached by every wave of it
    if (nt >= NT) run(std::integral_constant<int, NT>{});
    else if (nt == 1) run(std::integral_constant<int, 1>{});
    else if (nt == 2) run(std::integral_constant<int, (NT > 2 ? 2 : 1)>{});
    else run(std::integral_constant<int, (NT > 3 ? 3 : 1)>{});
}

// Decode plan: the fewest splits, then the larger R of {2, 1}, that give at
// least `target` workgroups while a split holds at most bps_max blocks (a
// wave's chain of blocks is latency-bound), or that give twice the target,
// where the workgroups per CU hide a longer chain.  Fewer splits mean fewer
// split-K partials for the consumers to read.  Matmuls whose partials feed
// the engine's consumers (attention prologue, residual and SwiGLU
// epilogues) allow 8 blocks per split: at the 8B shapes and 16 rows QKV
// R 1 / S 4, O R 1 / S 8, gate+up R 2 / S 2, down R 1 / S 8 and the LM head
// R 2 / S 1, each the fastest decode step of the per-shape choices measured
// (decode step -1.5 to -1.8 % against a largest-R-first rule at the same
// target).  The C ABI's matmul of 2-16 rows, whose partials only a split
// sum reads, allows 4 (14336x4096 at 16 rows: 16.9 vs 21.3 us with 8).
// Splits keep >= 2 blocks each: a one-block split never overlaps its weight
// prefetch with compute.  Waves per decode workgroup: 8 by default
// (measured 2 % faster per decode step than 4, since each staged activation
// block feeds twice the weight tiles, and 16 was 8 % slower);
// SLATE_HIP_Q4K_W=4 selects four.
constexpr int DEC_BPS_STEP = 8, DEC_BPS_OP = 4;

static int dec_waves() {
    return knobs().q4k_w;
}

static void dec_plan(const int* tiles, int n, int nblk, int s_max, int bps_max, int* R_out, int* S_out) {
    const int R_env = knobs().q4k_r;
    const int S_env = knobs().q4k_s;
    const int W = dec_waves();
    // SLATE_HIP_Q4K_WGS counts four-wave workgroups: 192 of eight waves by default
    const int target = std::max(1, knobs().q4k_wgs * 4 / W);
    if (s_max > nblk / 2) s_max = nblk / 2;
    if (s_max < 1) s_max = 1;
    // R = 4 only when asked for: at the same target, two tiles per wave with
    // half the splits (twice the blocks per wave) measured faster (gate+up
    // 2x14336x4096 at 16 rows: 18.0 vs 19.8 us; LM head equal)
    const bool r_fixed = R_env == 1 || R_env == 2 || R_env == 4;
    int R_out_v = r_fixed ? R_env : 1, S_out_v = s_max;
    bool done = false;
    for (int S = 1; S <= s_max && !done; S *= 2) {
        const int bps = (nblk + S - 1) / S;
        for (int R = r_fixed ? R_env : 2; R >= 1 && !done; R >>= 1) {
            if (r_fixed && R != R_env) continue;
            int groups = 0;
            for (int i = 0; i < n; ++i) groups += (tiles[i] + R - 1) / R;
            const int wgs = (groups + W - 1) / W * S;
            if (wgs >= target && (bps <= bps_max || wgs >= 2 * target)) {
                R_out_v = R;
                S_out_v = S;
                done = true;
            }
        }
    }
    if (S_env > 0) S_out_v = S_env < s_max ? S_env : s_max;
    *R_out = R_out_v;
    *S_out = S_out_v;
}

template <int R, bool TILED>
static void launch_dec(const Q4kTargets& tg, const Act16& a, float* out, int64_t ldo, int64_t ss, int nblk,
                       int bps, int nsplit, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    const int W = dec_waves();
    const int early = knobs().q4k_early;
    const dim3 grid((tg.grp_end + W - 1) / W, nsplit);
    const uint4* fr = (const uint4*)a.frag;
    if (a.rows_pad == 32) {
        if (W == 8) SH_LAUNCH(e0, e1, (q4k_dec_kernel<R, TILED, 8, 2>), grid, dim3(512), 0, s, tg, fr, out, ldo, ss, nblk, bps,
                  early, (const float*)nullptr, (int64_t)0, 0);
        else SH_LAUNCH(e0, e1, (q4k_dec_kernel<R, TILED, 4, 2>), grid, dim3(256), 0, s, tg, fr, out, ldo, ss, nblk, bps,
                  early, (const float*)nullptr, (int64_t)0, 0);
        return;
    }
    if (W == 8) SH_LAUNCH(e0, e1, (q4k_dec_kernel<R, TILED, 8, 1>), grid, dim3(512), 0, s, tg, fr, out, ldo, ss, nblk, bps,
                  early, (const float*)nullptr, (int64_t)0, 0);
    else SH_LAUNCH(e0, e1, (q4k_dec_kernel<R, TILED, 4, 1>), grid, dim3(256), 0, s, tg, fr, out, ldo, ss, nblk, bps,
                  early, (const float*)nullptr, (int64_t)0, 0);
}

constexpr int PF_R = 2, PF_WAVES = 8;

template <int NT, bool TILED, int R = PF_R, int WAVES = PF_WAVES>
static void launch_pf(const Q4kTargets& tg, const Act16& a, float* out, int64_t ldo, int64_t ss, int nblk, int bps,
                      int nsplit, hipStream_t s, hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr) {
    const int act_tiles = a.rows_pad / 16;
    dim3 grid(tg.grp_end, nsplit, (act_tiles + NT - 1) / NT);
    SH_LAUNCH(e0, e1, (q4k_pf_kernel<R, NT, TILED, WAVES>), grid, dim3(64 * WAVES), 0, s, tg, (const uint4*)a.frag,
              act_tiles, out, ldo, ss, nblk, bps);
}

// Workgroup slots per CU of the prefill kernel (its LDS: NT tiles x 2 buffers).
static int pf_slots(int NT) {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    const int per_cu = (160 * 1024) / (2 * NT * ACT_FRAG_UNITS * 16);
    return cus * (per_cu > 0 ? per_cu : 1);
}

int launch_q4k(const Q4kTarget* t, int n, bool tiled, const Act16& a, float* out, int64_t ldo, int64_t split_stride,
               int max_splits, int* S_out, hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop) {
    if (n < 1 || n > 3) { set_error(-1, "q4k: 1..3 fused tensors"); return -1; }
    const int nblk = a.K / QK;
    if (nblk < 1) { set_error(-1, "q4k: K=%d", a.K); return -1; }
    if (!a.frag || a.rows_pad < 16 || a.rows_pad % 16) { set_error(-1, "q4k: bad operand buffer"); return -1; }
    if (max_splits < 1) max_splits = 1;
    const int act_tiles = a.rows_pad / 16;
    // up to 32 rows: the decode kernel with one or two activation tiles
    // (SLATE_HIP_Q4K_DEC32=0 sends 17..32 rows to the prompt kernel)
    if (act_tiles > 2 || (act_tiles == 2 && !knobs().q4k_dec32)) {
        // the prompt kernel addresses the operand with 32-bit byte offsets
        if ((double)act_tiles * nblk * ACT_FRAG_UNITS * 16.0 >= 4294967296.0) {
            set_error(-1, "q4k: activation operand of %d rows x K=%d exceeds 4 GiB", a.rows_pad, a.K);
            return -1;
        }
        // prefill: all tensors in one launch, NT activation tiles per
        // workgroup; the split count minimises rounds of workgroups x (blocks
        // per workgroup + a fixed cost of about four blocks for the
        // workgroup's set-up, staging prologue and partial stores), a last,
        // partly filled round costing a whole one (measured at T = 320: two
        // splits beat 8 and 14 on the 4096-row shapes by 8-14 %)
        Q4kTargets tg{};
        int wgs = 0;
        for (int i = 0; i < n; ++i) {
            tg.w[i] = (const uint8_t*)t[i].w;
            tg.M[i] = t[i].M;
            tg.col[i] = (int)t[i].col;
            tg.grp0[i] = wgs;
            wgs += ((t[i].M + 15) / 16 + PF_WAVES * PF_R - 1) / (PF_WAVES * PF_R);
        }
        tg.n = n;
        tg.grp_end = wgs;
        // split count for NT activation tiles per workgroup; *fill: how full
        // the last round of workgroups is (1 when the rounds come out even),
        // *nrounds: rounds of workgroups
        auto plan = [&](int NT, double* fill, int* nrounds) {
            const int tasks = wgs * ((act_tiles + NT - 1) / NT);
            const int slots = pf_slots(NT);
            int Sb = 1;
            double best = 1e30;
            // every split count the block ranges can give (c splits of
            // ceil(nblk / c) blocks, the last one shorter), not only powers
            // of two: at about 300 rows the 4096-row shapes fill one round
            // with three splits, where two leave 96 CUs idle and four take
            // two rounds
            const int cmax = std::min(std::min(16, max_splits), nblk > 1 ? nblk / 2 : 1);
            for (int c = 1; c <= cmax; ++c) {
                const int bps_c = (nblk + c - 1) / c;
                if ((nblk + bps_c - 1) / bps_c != c) continue;   // the same ranges as a smaller c
                const int rounds = (tasks * c + slots - 1) / slots;
                const double cost = (double)rounds * ((double)bps_c + 4.0);
                if (cost <= best + 1e-9) { best = cost; Sb = c; }   // ties: more splits (measured faster)
            }
            const int rem = tasks * Sb % slots;
            *fill = rem ? (double)rem / slots : 1.0;
            *nrounds = (tasks * Sb + slots - 1) / slots;
            return Sb;
        };
        // four activation tiles per workgroup (one workgroup per CU: its two
        // operand buffers take 147 KiB of LDS), or two (two per CU) when the
        // four-tile plan runs two or more rounds of workgroups and leaves the
        // last one partly filled: half-size workgroups fill that round better
        // (gate+up 2x14336x4096 at 320 rows 184 vs 202 us, 512 rows 269 vs
        // 280 us; 70B gate+up at 384 rows 799 vs 810 us), and over a whole
        // bench window this threshold beat 60 / 75 / 85 % fill (mixed steps
        // -1.5 % against 60 %, the 70B serving steps unchanged); where the
        // rounds come out even or one round holds everything, four tiles
        double fill = 1.0;
        int rounds = 1;
        int NT = act_tiles >= 4 ? 4 : 2;
        int S = plan(NT, &fill, &rounds);
        if (NT == 4 && rounds >= 2 && fill < 1.0) {
            NT = 2;
            S = plan(2, &fill, &rounds);
        }
        if ((knobs().q4k_pf_nt == 2 || knobs().q4k_pf_nt == 4) && knobs().q4k_pf_nt != NT) {
            NT = knobs().q4k_pf_nt;
            S = plan(NT, &fill, &rounds);
        }
        const int S_env = knobs().q4k_pf_s;
        if (S_env > 0) S = std::min(S_env, std::max(1, std::min(max_splits, nblk)));
        const int bps = (nblk + S - 1) / S;
        S = (nblk + bps - 1) / bps;
        if (NT == 4) {
            if (tiled) launch_pf<4, true>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
            else launch_pf<4, false>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
        } else {
            if (tiled) launch_pf<2, true>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
            else launch_pf<2, false>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
        }
        SH_CHECK_LAUNCH();
        *S_out = S;
        return 0;
    }
    int tiles[3];
    for (int i = 0; i < n; ++i) tiles[i] = (t[i].M + 15) / 16;
    int R, S;
    dec_plan(tiles, n, nblk, max_splits, DEC_BPS_STEP, &R, &S);
    const int bps = (nblk + S - 1) / S;
    S = (nblk + bps - 1) / bps;                       // every split gets >= 1 block
    Q4kTargets tg{};
    int grp = 0;
    for (int i = 0; i < n; ++i) {
        tg.w[i] = (const uint8_t*)t[i].w;
        tg.M[i] = t[i].M;
        tg.col[i] = (int)t[i].col;
        tg.grp0[i] = grp;
        grp += (tiles[i] + R - 1) / R;
    }
    tg.n = n;
    tg.grp_end = grp;
    if (tiled) {
        if (R == 4) launch_dec<4, true>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
        else if (R == 2) launch_dec<2, true>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
        else launch_dec<1, true>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
    } else {
        if (R == 4) launch_dec<4, false>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
        else if (R == 2) launch_dec<2, false>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
        else launch_dec<1, false>(tg, a, out, ldo, split_stride, nblk, bps, S, s, ev_start, ev_stop);
    }
    SH_CHECK_LAUNCH();
    *S_out = S;
    return 0;
}

// The C ABI's Q4_K matmul of 1 < rows <= 16 f32 rows in one launch (plus the
// split sum): the decode kernel in its CONV form, on the decode plan.
template <int R, bool TILED>
static void launch_dec_conv(const Q4kTargets& tg, const float* X, int64_t ldx, int rows, float* out, int64_t ldo,
                            int64_t ss, int nblk, int bps, int nsplit, hipStream_t s) {
    const dim3 grid((tg.grp_end + 7) / 8, nsplit);
    hipLaunchKernelGGL((q4k_dec_kernel<R, TILED, 8, 1, true>), grid, dim3(512), 0, s, tg, (const uint4*)nullptr,
                       out, ldo, ss, nblk, bps, 0, X, ldx, rows);
}

int launch_q4k_conv(const Q4kTarget& t, bool tiled, const float* X, int64_t ldx, int rows, int K, float* out,
                    int64_t ldo, int64_t split_stride, int max_splits, int* S_out, hipStream_t s) {
    const int nblk = K / QK;
    if (rows < 1 || rows > 16 || nblk < 1 || K % QK || t.M < 1) {
        set_error(-1, "q4k: %d rows of K=%d for the one-tile kernel", rows, K);
        return -1;
    }
    if (dec_waves() != 8) return 1;                   // the caller stages the operand instead
    int tiles = (t.M + 15) / 16;
    int R, S;
    dec_plan(&tiles, 1, nblk, max_splits, DEC_BPS_OP, &R, &S);
    const int bps = (nblk + S - 1) / S;
    S = (nblk + bps - 1) / bps;
    Q4kTargets tg{};
    tg.w[0] = (const uint8_t*)t.w;
    tg.M[0] = t.M;
    tg.col[0] = (int)t.col;
    tg.grp0[0] = 0;
    tg.n = 1;
    tg.grp_end = (tiles + R - 1) / R;
    if (tiled) {
        if (R == 4) launch_dec_conv<4, true>(tg, X, ldx, rows, out, ldo, split_stride, nblk, bps, S, s);
        else if (R == 2) launch_dec_conv<2, true>(tg, X, ldx, rows, out, ldo, split_stride, nblk, bps, S, s);
        else launch_dec_conv<1, true>(tg, X, ldx, rows, out, ldo, split_stride, nblk, bps, S, s);
    } else {
        if (R == 4) launch_dec_conv<4, false>(tg, X, ldx, rows, out, ldo, split_stride, nblk, bps, S, s);
        else if (R == 2) launch_dec_conv<2, false>(tg, X, ldx, rows, out, ldo, split_stride, nblk, bps, S, s);
        else launch_dec_conv<1, false>(tg, X, ldx, rows, out, ldo, split_stride, nblk, bps, S, s);
    }
    SH_CHECK_LAUNCH();
    *S_out = S;
    return 0;
}

// ---------------------------------------------------------------------------
// ROW -> TILED repack: one thread per 16-byte unit of the tiled tensor.
__global__ __launch_bounds__(256) void q4k_tile_kernel(uint4* __restrict__ dst, const uint8_t* __restrict__ src,
                                                       int M, int nblk, int64_t units) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    const int64_t tb = u / 144;
    const int w = (int)(u - tb * 144);
    const int64_t tile = tb / nblk;
    const int kb = (int)(tb - tile * nblk);
    int j, off;
    if (w < 16) { j = w; off = 0; }
    else if (w < 80) { const int l = w - 16; j = l & 15; off = 16 + 32 * (l >> 4); }
    else { const int l = w - 80; j = l & 15; off = 32 + 32 * (l >> 4); }
    const int64_t row = tile * 16 + j;
    dst[u] = row < M ? *(const uint4*)(src + (row * nblk + kb) * QBLOCK + off) : make_uint4(0u, 0u, 0u, 0u);
}

size_t q4k_tiled_bytes(int M, int K) { return (size_t)((M + 15) / 16) * 16 * (size_t)(K / QK) * QBLOCK; }

int launch_q4k_tile(void* dst, const void* src, int M, int K, hipStream_t s) {
    const int nblk = K / QK;
    const int64_t units = (int64_t)((M + 15) / 16) * nblk * 144;
    if (units == 0) return 0;
    hipLaunchKernelGGL(q4k_tile_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, s, (uint4*)dst,
                       (const uint8_t*)src, M, nblk, units);
    SH_CHECK_LAUNCH();
    return 0;
}

void q4k_untile_host(uint8_t* dst, const uint8_t* src, int M, int K) {
    const int nblk = K / QK;
    for (int64_t row = 0; row < M; ++row) {
        const int64_t tile = row / 16;
        const int j = (int)(row % 16);
        for (int kb = 0; kb < nblk; ++kb) {
            const uint8_t* tb = src + (tile * nblk + kb) * (16 * QBLOCK);
            uint8_t* b = dst + (row * nblk + kb) * QBLOCK;
            memcpy(b, tb + 16 * j, 16);
            for (int g = 0; g < 4; ++g) {
                memcpy(b + 16 + 32 * g, tb + 256 + 16 * (16 * g + j), 16);
                memcpy(b + 32 + 32 * g, tb + 1280 + 16 * (16 * g + j), 16);
            }
        }
    }
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
