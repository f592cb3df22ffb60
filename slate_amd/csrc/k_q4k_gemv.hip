// k_q4k_gemv.hip -- Q4_K matrix-vector products for 1..4 activation rows on
// the vector ALUs: slate_q4_k_matvec (src/util/quant.c:306-313) for a small
// batch, with no activation operand conversion, no LDS staging of
// activations and no split-K partials (one kernel writes the final rows).
//
// Work split.  A workgroup owns R weight rows and all of K.  Thread t owns
// sub-block s = t & 7 of super-block kb = t >> 3 (32 elements of K): its
// activations (B rows x 32 f32) are loaded once into registers and reused
// for every one of the R rows.  Per row a thread issues two 128-bit loads,
// the block's 16-byte header (d, dmin, packed scales; the 8 threads of a
// block read the same one) and its sub-block's 16 bytes of nibbles, all R
// rows' loads before any arithmetic.  K above 64 super-blocks is covered
// in passes of 64 (one pass per 512 threads).
//
// Arithmetic (quant.c:210-304's formula in f32): per sub-block j of a
// block, d*sc_j * sum_i q_i x_i - dmin*mn_j * sum_i x_i.  Nibbles become
// floats with one AND per four values and one byte conversion each
// (v_cvt_f32_ubyte0..3): the low nibbles (elements 0..15 of the sub-block,
// slate's order) as q, the high nibbles (elements 16..31) as 16*q, whose
// dot product is scaled by 1/16 (exact).  Each thread's partial sums are
// reduced over its 16-lane row with DPP, then over the rows and waves of
// the workgroup through LDS in a fixed order, so results are deterministic.
#include <algorithm>

#include "launch.h"
#include "lanes.h"
#include "mfma.h"
#include "q4k.h"

namespace slate_hip {

constexpr int GEMV_WAVES = 8;                  // 512 threads

// x & m in inline assembly: the compiler cannot fold the mask into the byte
// extractions that follow, so each masked byte becomes a float with one
// v_cvt_f32_ubyte0..3 (folded, every nibble costs a field extract and a
// conversion).
__device__ __forceinline__ uint32_t and_opaque(uint32_t x, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(m), "v"(x));
    return r;
}

// tg: up to three tensors sharing X; tensor i owns workgroups
// [grp0[i], grp0[i+1]) of R rows each and writes Y columns [col, col + M).
// X: nb rows (nb <= B) of K f32, ldx apart; Y: nb rows, ldy apart.
template <int B, int R, bool TILED>
__global__ __launch_bounds__(64 * GEMV_WAVES) void q4k_gemv_kernel(Q4kTargets tg, const float* __restrict__ X,
                                                                   int64_t ldx, int nb, float* __restrict__ Y,
                                                                   int64_t ldy, int nblk) {
    __shared__ float red[GEMV_WAVES * 4 * R * B];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wv = t >> 6;
    const int nw = blockDim.x >> 6;
    const int s = t & 7;
    const int grp = blockIdx.x;
    const int ti = (tg.n > 2 && grp >= tg.grp0[2]) ? 2 : ((tg.n > 1 && grp >= tg.grp0[1]) ? 1 : 0);
    const uint8_t* W = tg.w[ti];
    const int M = tg.M[ti];
    const int m0 = (grp - tg.grp0[ti]) * R;
    // packed-scale selection for sub-block s (quant.c:157-166): byte s & 3
    // of (scales[0..3], scales[4..7]) for s < 4; for s >= 4 the low (high)
    // nibble of scales[8 + (s & 3)] with the top two bits of scales[s & 3]
    // (scales[4 + (s & 3)])
    const int sh = 8 * (s & 3);
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.f;

    for (int kc = 0; kc < nblk; kc += nw * 8) {
        // lanes past the last block read block nblk - 1 and weigh it by x = 0
        const int kb = kc + (t >> 3);
        const bool live = kb < nblk;
        const int kbc = live ? kb : nblk - 1;
        float x[B][32], xs[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float4* xp = (const float4*)(X + (int64_t)min(b, nb - 1) * ldx + (int64_t)kbc * QK + 32 * s);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 v = (b < nb && live) ? xp[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                x[b][4 * i] = v.x;
                x[b][4 * i + 1] = v.y;
                x[b][4 * i + 2] = v.z;
                x[b][4 * i + 3] = v.w;
            }
        }
        uint4 hd[R], qv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int m = min(m0 + r, M - 1);
            const uint8_t* hp;
            const uint8_t* qp;
            if (TILED) {
                const uint8_t* tb = W + ((size_t)(m >> 4) * nblk + kbc) * (16 * QBLOCK);
                hp = tb + 16 * (m & 15);
                qp = tb + ((s & 1) ? 1280 : 256) + 16 * (16 * (s >> 1) + (m & 15));
            } else {
                hp = W + ((size_t)m * nblk + kbc) * QBLOCK;
                qp = hp + 16 + 16 * s;
            }
            hd[r] = *(const uint4*)hp;
            qv[r] = *(const uint4*)qp;
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            xs[b] = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) xs[b] += x[b][i];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint4 h = hd[r];
            const uint32_t sc = s < 4 ? (h.y >> sh) & 63u : ((h.w >> sh) & 15u) | ((h.y >> (sh + 2)) & 0x30u);
            const uint32_t mn = s < 4 ? (h.z >> sh) & 63u : ((h.w >> (sh + 4)) & 15u) | ((h.z >> (sh + 2)) & 0x30u);
            const float dsc = f16_to_f32_hw(h.x & 0xffffu) * (float)sc;
            const float dmn = f16_to_f32_hw(h.x >> 16) * (float)mn;
            const uint32_t q[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
            float lo[B], hi[B];
#pragma unroll
            for (int b = 0; b < B; ++b) lo[b] = hi[b] = 0.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t ql = and_opaque(q[w], 0x0f0f0f0fu), qh = and_opaque(q[w], 0xf0f0f0f0u);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float fl = (float)((ql >> (8 * k)) & 0xffu);
                    const float fh = (float)((qh >> (8 * k)) & 0xffu);
#pragma unroll
                    for (int b = 0; b < B; ++b) {
                        lo[b] = __builtin_fmaf(fl, x[b][4 * w + k], lo[b]);
                        hi[b] = __builtin_fmaf(fh, x[b][16 + 4 * w + k], hi[b]);
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < B; ++b) acc[r][b] += dsc * (lo[b] + hi[b] * 0.0625f) - dmn * xs[b];
        }
    }
    // 16-lane rows by DPP; lane 0 of each row keeps the row's sums
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float v = row16_sum(acc[r][b]);
            if ((lane & 15) == 0) red[((wv * 4 + (lane >> 4)) * R + r) * B + b] = v;
        }
    __syncthreads();
    if (t < R * B) {
        const int r = t / B, b = t - r * B;
        float v = 0.f;
        for (int i = 0; i < nw * 4; ++i) v += red[i * R * B + t];
        const int m = m0 + r;
        if (m < M && b < nb) Y[(int64_t)b * ldy + tg.col[ti] + m] = v;
    }
}

template <int B, int R>
static void launch_gemv(const Q4kTargets& tg, bool tiled, const float* X, int64_t ldx, int nb, float* Y,
                        int64_t ldy, int nblk, int nw, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    if (tiled)
        SH_LAUNCH(e0, e1, (q4k_gemv_kernel<B, R, true>), dim3(tg.grp_end), dim3(64 * nw), 0, s, tg, X, ldx, nb, Y,
                  ldy, nblk);
    else
        SH_LAUNCH(e0, e1, (q4k_gemv_kernel<B, R, false>), dim3(tg.grp_end), dim3(64 * nw), 0, s, tg, X, ldx, nb, Y,
                  ldy, nblk);
}

int launch_q4k_gemv(const Q4kTarget* t, int n, bool tiled, const float* X, int64_t ldx, int B, int K, float* Y,
                    int64_t ldy, hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop) {
    if (n < 1 || n > 3) { set_error(-1, "q4k_gemv: 1..3 fused tensors"); return -1; }
    if (B < 1 || B > GEMV_MAX_ROWS) { set_error(-1, "q4k_gemv: %d rows (1..%d)", B, GEMV_MAX_ROWS); return -1; }
    if (K < QK || K % QK) { set_error(-1, "q4k_gemv: K=%d", K); return -1; }
    if (((uintptr_t)X & 15) || ldx % 4) { set_error(-1, "q4k_gemv: activation rows must be 16-byte aligned"); return -1; }
    const int nblk = K / QK;
    // one row of one tiled tensor: the MFMA matvec (SLATE_HIP_GEMV1=0 keeps
    // this kernel; slate's row layout always stays here, where whole rows
    // load contiguously)
    if (B == 1 && n == 1 && tiled && t[0].col == 0 && nblk <= GEMV1_MAX_BLOCKS && knobs().gemv1)
        return launch_q4k_gemv1(t[0].w, t[0].M, K, X, Y, s, ev_start, ev_stop);
    // rows per workgroup: 8 for one or two activation rows, 4 for three or
    // four (keeps the activations, 32 x B floats per thread, and the loads
    // of all R rows under 256 VGPRs: two waves per SIMD); one row of slate's
    // layout over more than 32 blocks takes 16, since every workgroup reads
    // all of X (at 4096 x 14336: 13.2 vs 15.6 us per call, 12.1 vs 11.5 at
    // 14336 x 4096)
    const bool r16 = B == 1 && nblk > 32 && !tiled;
    const int R = r16 ? 16 : (B <= 2 ? 8 : 4);
    Q4kTargets tg{};
    int grp = 0;
    for (int i = 0; i < n; ++i) {
        if (t[i].M < 1) { set_error(-1, "q4k_gemv: M=%d", t[i].M); return -1; }
        tg.w[i] = (const uint8_t*)t[i].w;
        tg.M[i] = t[i].M;
        tg.col[i] = (int)t[i].col;
        tg.grp0[i] = grp;
        grp += (t[i].M + R - 1) / R;
    }
    tg.n = n;
    tg.grp_end = grp;
    const int nw = std::min(GEMV_WAVES, (nblk + 7) / 8);
    if (r16)
        SH_LAUNCH(ev_start, ev_stop, (q4k_gemv_kernel<1, 16, false>), dim3(tg.grp_end), dim3(64 * nw), 0, s, tg, X,
                  ldx, B, Y, ldy, nblk);
    else if (B == 1) launch_gemv<1, 8>(tg, tiled, X, ldx, B, Y, ldy, nblk, nw, s, ev_start, ev_stop);
    else if (B == 2) launch_gemv<2, 8>(tg, tiled, X, ldx, B, Y, ldy, nblk, nw, s, ev_start, ev_stop);
    else launch_gemv<4, 4>(tg, tiled, X, ldx, B, Y, ldy, nblk, nw, s, ev_start, ev_stop);
    SH_CHECK_LAUNCH();
    return 0;
}

}  // namespace slate_hip
