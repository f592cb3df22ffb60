// k_rows.hip -- row-wise kernels: RMSNorm (+residual), SiLU*mul, RoPE with
// KV append, embedding gather, greedy argmax, ragged-batch packing and the
// small f32 matmuls behind the vtable's matvec / linear_batch.
#include "launch.h"
#include "act16.h"
#include "rowops.h"

namespace slate_hip {

// Block-wide sum over 256 threads (wave64 shuffles, then LDS across waves).
__device__ __forceinline__ double block_sum_256(double v, double* sh) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    double r = 0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r += sh[i];
    return r;
}

// ---------------------------------------------------------------------------
// RMSNorm of B rows (backend_cpu.c:48-76): inv = 1/sqrtf((float)(sum x^2 / D) + eps),
// y = (x * w) * inv.  If delta != nullptr, x += sum_{s<nsplit} delta[s] first
// (residual add of a split-K matmul result) and x is written back.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(float* __restrict__ y, float* __restrict__ x,
                                                           const float* __restrict__ delta, int nsplit,
                                                           int64_t split_stride, const float* __restrict__ w,
                                                           int D, float eps) {
#pragma clang fp contract(off)
    __shared__ double sh[4];
    const int r = blockIdx.x;
    float* xr = x + (size_t)r * D;
    float acc = 0.f;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float v = xr[d];
        if (delta) {
            const float* dr = delta + (size_t)r * D + d;
            float s = dr[0];
            for (int k = 1; k < nsplit; ++k) s += dr[(int64_t)k * split_stride];
            v += s;
            xr[d] = v;
        }
        acc = __builtin_fmaf(v, v, acc);
    }
    double sq = block_sum_256((double)acc, sh);
    float inv = 1.0f / sqrtf((float)(sq / (double)D) + eps);
    float* yr = y + (size_t)r * D;
    for (int d = threadIdx.x; d < D; d += blockDim.x) yr[d] = (xr[d] * w[d]) * inv;
}

int launch_rmsnorm_rows(float* y, float* x, const float* delta, int nsplit, int64_t split_stride,
                        const float* w, int B, int D, float eps, hipStream_t s) {
    if (B <= 0) return 0;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(B), dim3(256), 0, s, y, x, delta, nsplit,
                       split_stride, w, D, eps);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// y = silu(g) * u (backend_cpu.c:78-97).  gate/up may be split-K partials:
// g = sum_s gate[s], u = sum_s up[s].
__global__ void silu_mul_kernel(float* __restrict__ y, const float* __restrict__ gate,
                                const float* __restrict__ up, int64_t n, int nsplit,
                                int64_t split_stride, int H, int64_t gate_ld, int64_t up_ld) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t r = i / H, c = i - r * H;
    const float* gp = gate + r * gate_ld + c;
    const float* upp = up + r * up_ld + c;
    float g = gp[0], u = upp[0];
    for (int k = 1; k < nsplit; ++k) {
        g += gp[(int64_t)k * split_stride];
        u += upp[(int64_t)k * split_stride];
    }
    y[i] = (g / (1.0f + expf(-g))) * u;
}

int launch_silu_mul(float* y, const float* gate, const float* up, int rows, int H, int nsplit,
                    int64_t split_stride, int64_t gate_ld, int64_t up_ld, hipStream_t s) {
    int64_t n = (int64_t)rows * H;
    if (n <= 0) return 0;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, gate, up,
                       n, nsplit, split_stride, H, gate_ld, up_ld);
    SH_CHECK_LAUNCH();
    return 0;
}

__global__ void add_kernel(float* __restrict__ y, const float* __restrict__ x, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] += x[i];
}

int launch_add(float* y, const float* x, int64_t n, hipStream_t s) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, x, n);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Embedding gather: y[t, :] = W[tok[t], :].  Tokens are validated on the
// host; out-of-range ids are clamped here only to keep every access in bounds.
__global__ void embed_rows_kernel(float* __restrict__ y, const float* __restrict__ W,
                                  const int32_t* __restrict__ tok, int V, int D) {
    int t = blockIdx.y;
    int id = tok[t];
    id = id < 0 ? 0 : (id >= V ? V - 1 : id);
    for (int d = blockIdx.x * blockDim.x + threadIdx.x; d < D; d += gridDim.x * blockDim.x)
        y[(size_t)t * D + d] = W[(size_t)id * D + d];
}

int launch_embed_rows(float* y, const float* W, const int32_t* tok, int T, int V, int D, hipStream_t s) {
    if (T <= 0) return 0;
    dim3 grid((D + 255) / 256, T);
    hipLaunchKernelGGL(embed_rows_kernel, grid, dim3(256), 0, s, y, W, tok, V, D);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// RoPE (llama_infer.c:77-92) from a host-built table: cs[(|p|*half + i)*2] =
// {cosf(angle), sinf(angle)} with the reference's exact float expressions, so
// rotation of identical inputs is bit-identical.  Negative positions use
// cos(-a) = cos(a), sin(-a) = -sin(a).  Rows whose |pos| >= max_pos are left
// unchanged and counted in *bad.
__device__ __forceinline__ void rope_apply(float* x, int n_heads, int hd, int pos,
                                           const float* __restrict__ cs, int lane, int nlanes) {
#pragma clang fp contract(off)
    int half = hd / 2;
    int ap = pos < 0 ? -pos : pos;
    float sg = pos < 0 ? -1.0f : 1.0f;
    for (int idx = lane; idx < n_heads * half; idx += nlanes) {
        int h = idx / half, i = idx - h * half;
        float c = cs[((size_t)ap * half + i) * 2 + 0];
        float s = sg * cs[((size_t)ap * half + i) * 2 + 1];
        float* hh = x + h * hd;
        float a = hh[i], b = hh[i + half];
        hh[i] = a * c - b * s;
        hh[i + half] = a * s + b * c;
    }
}

__global__ void rope_rows_kernel(float* __restrict__ x, const int32_t* __restrict__ pos, int n_heads,
                                 int hd, const float* __restrict__ cs, int max_pos, int* bad) {
    int r = blockIdx.x;
    int p = pos[r];
    int ap = p < 0 ? -p : p;
    if (ap >= max_pos) {
        if (threadIdx.x == 0) atomicAdd(bad, 1);
        return;
    }
    rope_apply(x + (size_t)r * n_heads * hd, n_heads, hd, p, cs, threadIdx.x, blockDim.x);
}

int launch_rope_rows(float* x, const int32_t* pos, int n_rows, int n_heads, int hd, const float* cs,
                     int max_pos, int* bad, hipStream_t s) {
    if (n_rows <= 0) return 0;
    hipLaunchKernelGGL(rope_rows_kernel, dim3(n_rows), dim3(256), 0, s, x, pos, n_heads, hd, cs, max_pos,
                       bad);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Engine epilogues that also emit the next Q4_K matmul's activation operand
// (act16.h), so a split-K sum, the row operation and the operand conversion
// are one pass over the row.

// Residual + RMSNorm split across the whole chip (all-Q4_K consumers): one
// wave per 256-element block of a row does x += sum_s delta[s] (fixed split
// order, written back), stores the block's sum of squares in
// ssq[r * D/256 + kb] and emits x * w (without the row factor) as the Q4_K
// operand.  The consumer of the matmul that follows multiplies each row by
// row_inv_rms() (the matmul is linear in each row), so no kernel has to wait
// for a whole row.  Rows >= rows write zero operand rows.
// TILE: a 512-thread workgroup per (block, 8-row half tile), wave w = row w
// of the half, the operand written by act16_store_tile (rows of prompt
// steps).
template <bool DELTA, int NPRE, bool TILE>
__device__ __forceinline__ void residual_act_body(float* __restrict__ x, const float* __restrict__ delta,
                                                  int nsplit, int64_t split_stride, const float* __restrict__ w,
                                                  int rows, int D, const Act16& a, float* __restrict__ ssq,
                                                  uint4* s_t) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int kb = TILE ? blockIdx.x : blockIdx.x * (int)(blockDim.x >> 6) + (threadIdx.x >> 6);
    const int nblk = D / QK;
    if (!TILE && kb >= nblk) return;              // whole wave
    const int r = TILE ? blockIdx.y * 8 + (threadIdx.x >> 6) : blockIdx.y;
    const int e = kb * QK + 4 * lane;
    float4 yv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < rows) {
        // x, w and the first NPRE partials are issued together: one memory
        // round trip before any arithmetic (up to NPRE splits)
        float* xr = x + (size_t)r * D + e;
        const float* dp = DELTA ? delta + (size_t)r * D + e : nullptr;
        float4 xv = *(const float4*)xr;
        const float4 wv = *(const float4*)(w + e);
        Split4N<NPRE> pre;
        if constexpr (DELTA) pre = split_load4<NPRE>(dp, nsplit, split_stride);
        if constexpr (DELTA) {
            const float4 sm = split_fin4(pre, dp, nsplit, split_stride);
            xv.x += sm.x; xv.y += sm.y; xv.z += sm.z; xv.w += sm.w;
        }
        float sq = 0.f;
        sq = __builtin_fmaf(xv.x, xv.x, sq);
        sq = __builtin_fmaf(xv.y, xv.y, sq);
        sq = __builtin_fmaf(xv.z, xv.z, sq);
        sq = __builtin_fmaf(xv.w, xv.w, sq);
        sq = wave_sum(sq);
        yv = make_float4(xv.x * wv.x, xv.y * wv.y, xv.z * wv.z, xv.w * wv.w);
        if constexpr (DELTA) *(float4*)xr = xv;
        if (lane == 0) ssq[(size_t)r * nblk + kb] = sq;
    }
    if constexpr (TILE) act16_store_tile<8>(a, blockIdx.y >> 1, blockIdx.y & 1, kb, s_t, yv);
    else act16_store_block(a, r, kb, lane, yv);
}
template <bool DELTA, int NPRE = 8>
__global__ __launch_bounds__(256) void residual_act_kernel(float* __restrict__ x, const float* __restrict__ delta,
                                                           int nsplit, int64_t split_stride,
                                                           const float* __restrict__ w, int rows, int D, Act16 a,
                                                           float* __restrict__ ssq) {
    residual_act_body<DELTA, NPRE, false>(x, delta, nsplit, split_stride, w, rows, D, a, ssq, nullptr);
}
template <bool DELTA, int NPRE = 8>
__global__ __launch_bounds__(512) void residual_act_tile_kernel(float* __restrict__ x,
                                                                 const float* __restrict__ delta, int nsplit,
                                                                 int64_t split_stride, const float* __restrict__ w,
                                                                 int rows, int D, Act16 a, float* __restrict__ ssq) {
    __shared__ uint4 s_t[ACT_FRAG_UNITS];
    residual_act_body<DELTA, NPRE, true>(x, delta, nsplit, split_stride, w, rows, D, a, ssq, s_t);
}

int launch_residual_act(float* x, const float* delta, int nsplit, int64_t split_stride, const float* w, int rows,
                        int D, const Act16& a, float* ssq, hipStream_t s) {
    if (rows <= 0) return 0;
    if (D % QK || a.K != D) {
        set_error(-1, "residual_act: width %d is not a multiple of 256", D);
        return -1;
    }
    const int nblk = D / QK;
    // row-wise (decode rows): a workgroup per (block, row), so the few rows
    // of a decode step spread over every CU (at 16 rows four-wave
    // workgroups used a quarter of them: decode step -0.9 %)
    const dim3 grid(nblk, a.rows_pad);
    if (a.rows_pad > 16) {   // prompt steps: the operand by 8-row half tiles
        const dim3 tg(nblk, a.rows_pad / 8);
        if (delta && nsplit > 8)
            hipLaunchKernelGGL((residual_act_tile_kernel<true, 16>), tg, dim3(512), 0, s, x, delta, nsplit,
                               split_stride, w, rows, D, a, ssq);
        else if (delta && nsplit > 0)
            hipLaunchKernelGGL((residual_act_tile_kernel<true>), tg, dim3(512), 0, s, x, delta, nsplit, split_stride,
                               w, rows, D, a, ssq);
        else
            hipLaunchKernelGGL((residual_act_tile_kernel<false>), tg, dim3(512), 0, s, x, delta, nsplit,
                               split_stride, w, rows, D, a, ssq);
    } else if (delta && nsplit > 8)   // more than eight splits (forced plans): all in one round trip
        hipLaunchKernelGGL((residual_act_kernel<true, 16>), grid, dim3(64), 0, s, x, delta, nsplit, split_stride, w,
                           rows, D, a, ssq);
    else if (delta && nsplit > 0)
        hipLaunchKernelGGL(residual_act_kernel<true>, grid, dim3(64), 0, s, x, delta, nsplit, split_stride, w, rows,
                           D, a, ssq);
    else
        hipLaunchKernelGGL(residual_act_kernel<false>, grid, dim3(64), 0, s, x, delta, nsplit, split_stride, w,
                           rows, D, a, ssq);
    SH_CHECK_LAUNCH();
    return 0;
}

// Residual + RMSNorm: x += sum_s delta[s] (fixed split order, written back),
// y = (x * w) * inv with inv = 1/sqrtf((float)(sum x^2 / D) + eps)
// (backend_cpu.c:48-76), stored as f32 (y != nullptr) and/or as the operand
// (act != 0, D % 256 == 0).  One workgroup per row keeps the row in
// registers: thread i owns elements 4(i + nt*c) .. +3 of chunk c, so each
// wave owns whole 256-element blocks.  Rows >= rows write zero operand rows.
constexpr int RMS_MAX_CHUNKS = 4;
__global__ __launch_bounds__(1024) void rmsnorm_act_kernel(float* __restrict__ y, float* __restrict__ x,
                                                           const float* __restrict__ delta, int nsplit,
                                                           int64_t split_stride, const float* __restrict__ w,
                                                           int rows, int D, float eps, Act16 a, int act) {
#pragma clang fp contract(off)
    __shared__ double sh[16];
    const int r = blockIdx.x;
    const int nt = blockDim.x, tid = threadIdx.x, lane = tid & 63;
    const bool valid = r < rows;
    // every load (x, w, the first eight partials of each chunk) is issued
    // before any arithmetic; x is written back after the row reduction
    float4 v[RMS_MAX_CHUNKS], wv[RMS_MAX_CHUNKS];
    Split4 pre[RMS_MAX_CHUNKS];
#pragma unroll
    for (int c = 0; c < RMS_MAX_CHUNKS; ++c) {
        v[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        wv[c] = v[c];
        const int e = 4 * (tid + nt * c);
        if (valid && e < D) {
            v[c] = *(const float4*)(x + (size_t)r * D + e);
            wv[c] = *(const float4*)(w + e);
            if (delta) pre[c] = split_load4(delta + (size_t)r * D + e, nsplit, split_stride);
        }
    }
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < RMS_MAX_CHUNKS; ++c) {
        const int e = 4 * (tid + nt * c);
        if (valid && e < D) {
            float4 xv = v[c];
            if (delta) {
                const float4 sm = split_fin4(pre[c], delta + (size_t)r * D + e, nsplit, split_stride);
                xv.x += sm.x; xv.y += sm.y; xv.z += sm.z; xv.w += sm.w;
            }
            v[c] = xv;
            acc = __builtin_fmaf(xv.x, xv.x, acc);
            acc = __builtin_fmaf(xv.y, xv.y, acc);
            acc = __builtin_fmaf(xv.z, xv.z, acc);
            acc = __builtin_fmaf(xv.w, xv.w, acc);
        }
    }
    double sq = (double)acc;
    for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
    if (lane == 0) sh[tid >> 6] = sq;
    __syncthreads();
    sq = 0.0;
    for (int i = 0; i < (nt >> 6); ++i) sq += sh[i];
    const float inv = 1.0f / sqrtf((float)(sq / (double)D) + eps);
#pragma unroll
    for (int c = 0; c < RMS_MAX_CHUNKS; ++c) {
        const int e = 4 * (tid + nt * c);
        if (e >= D) break;                        // uniform per wave when D % 256 == 0
        float4 yv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (valid) {
            if (delta) *(float4*)(x + (size_t)r * D + e) = v[c];
            yv = make_float4((v[c].x * wv[c].x) * inv, (v[c].y * wv[c].y) * inv, (v[c].z * wv[c].z) * inv,
                             (v[c].w * wv[c].w) * inv);
            if (y) *(float4*)(y + (size_t)r * D + e) = yv;
        }
        if (act) act16_store_block(a, r, e / QK, lane, yv);
    }
}

int launch_rmsnorm_act(float* y, float* x, const float* delta, int nsplit, int64_t split_stride, const float* w,
                       int rows, int D, float eps, const Act16* a, hipStream_t s) {
    if (rows <= 0) return 0;
    if (D % 4 || D > 4 * 1024 * RMS_MAX_CHUNKS || (a && (D % QK || a->K != D))) {
        set_error(-1, "rmsnorm_act: unsupported width %d", D);
        return -1;
    }
    int nt = (D / 4 + RMS_MAX_CHUNKS - 1) / RMS_MAX_CHUNKS;
    nt = (nt + 63) / 64 * 64;
    if (nt > 1024) nt = 1024;
    if (nt < 64) nt = 64;
    const int grid = a ? a->rows_pad : rows;
    hipLaunchKernelGGL(rmsnorm_act_kernel, dim3(grid), dim3(nt), 0, s, y, x, delta, nsplit, split_stride, w, rows,
                       D, eps, a ? *a : Act16{}, a ? 1 : 0);
    SH_CHECK_LAUNCH();
    return 0;
}

// SwiGLU of split-K gate/up partials, h = silu(g) * u with g = sum_s gate[s],
// u = sum_s up[s] (backend_cpu.c:78-97 semantics, expf form), stored as f32
// (y != nullptr, [rows][H]) and/or as the operand of the down projection.
// One wave per 256-element block of a row (H % 256 == 0).
// TILE (with the operand): a 512-thread workgroup per (block, 8-row half
// tile), wave w = row w of the half, the operand written by
// act16_store_tile (half tiles: at 114 VGPRs two such workgroups share a
// CU, where one 16-row workgroup would hold it alone).
template <int NPRE, bool TILE>
__device__ __forceinline__ void silu_act_body(float* __restrict__ y, const float* __restrict__ gate,
                                              const float* __restrict__ up, int rows, int H, int nsplit,
                                              int64_t split_stride, int64_t ld, const Act16& a, int act,
                                              const RowNorm& rn, uint4* s_t) {
    const int lane = threadIdx.x & 63;
    const int kb = TILE ? blockIdx.x : blockIdx.x * (int)(blockDim.x >> 6) + (threadIdx.x >> 6);
    if (!TILE && kb * QK >= H) return;            // whole wave
    const int r = TILE ? blockIdx.y * 8 + (threadIdx.x >> 6) : blockIdx.y;
    const int e = kb * QK + 4 * lane;
    float4 h = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r < rows) {
        const float* gp = gate + (size_t)r * ld + e;
        const float* upp = up + (size_t)r * ld + e;
        // gate, up and the row's block sums of squares in one round trip
        const Split4N<NPRE> pg = split_load4<NPRE>(gp, nsplit, split_stride);
        const Split4N<NPRE> pu = split_load4<NPRE>(upp, nsplit, split_stride);
        RmsPre rp;
        if (rn.ssq) rp = row_rms_load(rn.ssq, r, rn.nblk);
        float4 g = split_fin4(pg, gp, nsplit, split_stride), u = split_fin4(pu, upp, nsplit, split_stride);
        if (rn.ssq) {   // gate and up are linear in the normalised row
            const float inv = row_rms_fin(rp, rn.ssq, r, rn.nblk, rn.D, rn.eps);
            g = make_float4(g.x * inv, g.y * inv, g.z * inv, g.w * inv);
            u = make_float4(u.x * inv, u.y * inv, u.z * inv, u.w * inv);
        }
        h = make_float4((g.x / (1.0f + expf(-g.x))) * u.x, (g.y / (1.0f + expf(-g.y))) * u.y,
                        (g.z / (1.0f + expf(-g.z))) * u.z, (g.w / (1.0f + expf(-g.w))) * u.w);
        if (y) *(float4*)(y + (size_t)r * H + e) = h;
    }
    if constexpr (TILE) act16_store_tile<8>(a, blockIdx.y >> 1, blockIdx.y & 1, kb, s_t, h);
    else if (act) act16_store_block(a, r, kb, lane, h);
}
template <int NPRE>
__global__ __launch_bounds__(256) void silu_act_kernel(float* __restrict__ y, const float* __restrict__ gate,
                                                       const float* __restrict__ up, int rows, int H, int nsplit,
                                                       int64_t split_stride, int64_t ld, Act16 a, int act,
                                                       RowNorm rn) {
    silu_act_body<NPRE, false>(y, gate, up, rows, H, nsplit, split_stride, ld, a, act, rn, nullptr);
}
__global__ __launch_bounds__(512) void silu_act_tile_kernel(float* __restrict__ y, const float* __restrict__ gate,
                                                             const float* __restrict__ up, int rows, int H,
                                                             int nsplit, int64_t split_stride, int64_t ld, Act16 a,
                                                             RowNorm rn) {
    __shared__ uint4 s_t[ACT_FRAG_UNITS];
    silu_act_body<1, true>(y, gate, up, rows, H, nsplit, split_stride, ld, a, 1, rn, s_t);
}

int launch_silu_act(float* y, const float* gate, const float* up, int rows, int H, int nsplit,
                    int64_t split_stride, int64_t ld, const Act16* a, const RowNorm& rn, hipStream_t s) {
    if (rows <= 0) return 0;
    if (H % QK || (a && a->K != H)) {
        set_error(-1, "silu_act: width %d is not a multiple of 256", H);
        return -1;
    }
    const int nblk = H / QK;
    // row-wise: a workgroup per (block, row), as the residual epilogue
    // (decode step -0.6 % against four-wave workgroups)
    const dim3 grid(nblk, a ? a->rows_pad : rows);
    // unsplit gate+up (prompt steps): registers for one partial each, so
    // more waves per SIMD on the prompt rows' large grids; with the operand,
    // written by 8-row half tiles
    if (nsplit <= 1 && a && a->rows_pad > 16)
        hipLaunchKernelGGL(silu_act_tile_kernel, dim3(nblk, a->rows_pad / 8), dim3(512), 0, s, y, gate, up, rows,
                           H, nsplit, split_stride, ld, *a, rn);
    else if (nsplit <= 1)
        hipLaunchKernelGGL(silu_act_kernel<1>, grid, dim3(64), 0, s, y, gate, up, rows, H, nsplit, split_stride,
                           ld, a ? *a : Act16{}, a ? 1 : 0, rn);
    else
        hipLaunchKernelGGL(silu_act_kernel<8>, grid, dim3(64), 0, s, y, gate, up, rows, H, nsplit, split_stride,
                           ld, a ? *a : Act16{}, a ? 1 : 0, rn);
    SH_CHECK_LAUNCH();
    return 0;
}

// QKV epilogue, one wave per (token, head), four heads of a token per
// workgroup: sums the split-K partials of the head's columns, rotates q / k
// at the token's position (same table and expressions as rope_apply) and
// writes q to qout, k and v into the KV pool.
template <typename KVT>
__global__ __launch_bounds__(256) void rope_kv_kernel(float* __restrict__ qout, KVT* __restrict__ Kpool,
                                                     KVT* __restrict__ Vpool, const float* __restrict__ part,
                                                     int nsplit, int64_t split_stride, int qkv_ld,
                                                     const int32_t* __restrict__ tok2seq,
                                                     const int32_t* __restrict__ tok_pos,
                                                     const int64_t* __restrict__ kv_base, int n_heads,
                                                     int n_kv_heads, int hd, int64_t head_stride,
                                                     const float* __restrict__ cs, RowNorm rn) {
#pragma clang fp contract(off)
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y, lane = threadIdx.x & 63;
    if (u >= n_heads + n_kv_heads) return;        // whole wave; no barriers below
    const int D = n_heads * hd, kvd = n_kv_heads * hd, half = hd / 2;
    const int p = tok_pos[t];
    const int ap = p < 0 ? -p : p;
    const float sg = p < 0 ? -1.0f : 1.0f;
    const float* pr = part + (size_t)t * qkv_ld;
    // q, k, v are linear in the normalised row: its RMSNorm factor is
    // applied here.  Every load that does not depend on the position (the
    // partials of the lane's columns, the row's block sums) is issued before
    // the position-dependent ones (rotation table, KV row).
    RmsPre rp;
    if (rn.ssq) rp = row_rms_load(rn.ssq, t, rn.nblk);
    float inv = 1.0f;
    auto scale = [&](float v) { return rn.ssq ? v * inv : v; };
    if (u < n_heads) {
        for (int i = lane; i < half; i += 64) {
            const int c0 = u * hd + i;
            const Split1 pa = split_load1(pr + c0, nsplit, split_stride);
            const Split1 pb = split_load1(pr + c0 + half, nsplit, split_stride);
            const float c = cs[((size_t)ap * half + i) * 2 + 0];
            const float sn = sg * cs[((size_t)ap * half + i) * 2 + 1];
            if (rn.ssq) inv = row_rms_fin(rp, rn.ssq, t, rn.nblk, rn.D, rn.eps);
            const float a = scale(split_fin1(pa, pr + c0, nsplit, split_stride));
            const float b = scale(split_fin1(pb, pr + c0 + half, nsplit, split_stride));
            qout[(size_t)t * D + c0] = a * c - b * sn;
            qout[(size_t)t * D + c0 + half] = a * sn + b * c;
        }
    } else {
        const int kh = u - n_heads;
        const int seq = tok2seq[t];
        for (int i = lane; i < half; i += 64) {
            const int ck = D + kh * hd + i, cv = D + kvd + kh * hd + i;
            const Split1 pa = split_load1(pr + ck, nsplit, split_stride);
            const Split1 pb = split_load1(pr + ck + half, nsplit, split_stride);
            const Split1 pv0 = split_load1(pr + cv, nsplit, split_stride);
            const Split1 pv1 = split_load1(pr + cv + half, nsplit, split_stride);
            const float c = cs[((size_t)ap * half + i) * 2 + 0];
            const float sn = sg * cs[((size_t)ap * half + i) * 2 + 1];
            const int64_t base = kv_base[seq] + (int64_t)kh * head_stride + (int64_t)p * hd;
            if (rn.ssq) inv = row_rms_fin(rp, rn.ssq, t, rn.nblk, rn.D, rn.eps);
            const float a = scale(split_fin1(pa, pr + ck, nsplit, split_stride));
            const float b = scale(split_fin1(pb, pr + ck + half, nsplit, split_stride));
            Kpool[base + i] = (KVT)(a * c - b * sn);
            Kpool[base + i + half] = (KVT)(a * sn + b * c);
            Vpool[base + i] = (KVT)scale(split_fin1(pv0, pr + cv, nsplit, split_stride));
            Vpool[base + i + half] = (KVT)scale(split_fin1(pv1, pr + cv + half, nsplit, split_stride));
        }
    }
}

int launch_rope_kv(float* qout, void* Kpool, void* Vpool, const float* part, int nsplit, int64_t split_stride,
                   int qkv_ld, const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int T,
                   int n_heads, int n_kv_heads, int hd, int64_t head_stride, const float* cs, const RowNorm& rn,
                   bool kv_f16, hipStream_t s) {
    if (T <= 0) return 0;
    if (kv_f16)
        hipLaunchKernelGGL(rope_kv_kernel<_Float16>, dim3((n_heads + n_kv_heads + 3) / 4, T), dim3(256), 0, s, qout,
                           (_Float16*)Kpool, (_Float16*)Vpool, part, nsplit, split_stride, qkv_ld, tok2seq, tok_pos,
                           kv_base, n_heads, n_kv_heads, hd, head_stride, cs, rn);
    else
        hipLaunchKernelGGL(rope_kv_kernel<float>, dim3((n_heads + n_kv_heads + 3) / 4, T), dim3(256), 0, s, qout,
                           (float*)Kpool, (float*)Vpool, part, nsplit, split_stride, qkv_ld, tok2seq, tok_pos,
                           kv_base, n_heads, n_kv_heads, hd, head_stride, cs, rn);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Greedy argmax per row with sampling.c:14-18 semantics: the first maximal
// element wins (strict '>'), NaN is never selected unless element 0 is NaN,
// in which case nothing compares greater and index 0 is returned.
// Two passes: chunks of ARGMAX_CHUNK elements of every row in parallel (a
// thread scans its elements in index order, then a tree keeps the larger
// value, or the lower index on ties; NaN never enters), then one wave per
// row combines its chunks the same way.  ws holds (value, index) per
// (row, chunk).
constexpr int ARGMAX_CHUNK = 4096;
struct AmBest { float v; int i; };
__device__ __forceinline__ void am_take(AmBest& b, float v, int i) {
    if (v > b.v || (b.i < 0 && !(v != v))) { b.v = v; b.i = i; }
}
__device__ __forceinline__ AmBest am_pick(AmBest a, AmBest b) {   // a before b in index order
    const bool tk = b.i >= 0 && (a.i < 0 || b.v > a.v || (b.v == a.v && b.i < a.i));
    return tk ? b : a;
}

// With rn.ssq, the logits are those of a row whose RMSNorm factor was left
// to the consumer (deferred norm): each is multiplied by the row's factor,
// written back, and compared scaled.
__global__ __launch_bounds__(256) void argmax_part_kernel(float2* __restrict__ ws, float* __restrict__ logits,
                                                          int V, int nch, RowNorm rn) {
    __shared__ AmBest sb[256];
    const int c = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
    float* p = logits + (size_t)r * V;
    const int e0 = c * ARGMAX_CHUNK, e1 = min(e0 + ARGMAX_CHUNK, V);
    float inv = 1.0f;
    if (rn.ssq) {
        const RmsPre rp = row_rms_load(rn.ssq, r, rn.nblk);
        inv = row_rms_fin(rp, rn.ssq, r, rn.nblk, rn.D, rn.eps);
    }
    AmBest bst{-INFINITY, -1};
    if (((uintptr_t)(p + e0) & 15) == 0 && e1 - e0 == ARGMAX_CHUNK) {
        float4 v[ARGMAX_CHUNK / 1024];
#pragma unroll
        for (int k = 0; k < ARGMAX_CHUNK / 1024; ++k) v[k] = *(const float4*)(p + e0 + 4 * (tid + 256 * k));
#pragma unroll
        for (int k = 0; k < ARGMAX_CHUNK / 1024; ++k) {
            const int i = e0 + 4 * (tid + 256 * k);
            if (rn.ssq) {
                v[k] = make_float4(v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv);
                *(float4*)(p + i) = v[k];
            }
            am_take(bst, v[k].x, i);
            am_take(bst, v[k].y, i + 1);
            am_take(bst, v[k].z, i + 2);
            am_take(bst, v[k].w, i + 3);
        }
    } else {
        for (int i = e0 + tid; i < e1; i += 256) {
            float v = p[i];
            if (rn.ssq) {
                v *= inv;
                p[i] = v;
            }
            am_take(bst, v, i);
        }
    }
    sb[tid] = bst;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) sb[tid] = am_pick(sb[tid], sb[tid + o]);
        __syncthreads();
    }
    if (tid == 0) ws[(size_t)r * nch + c] = make_float2(sb[0].v, __int_as_float(sb[0].i));
}

__global__ __launch_bounds__(64) void argmax_fin_kernel(int32_t* __restrict__ out, const float2* __restrict__ ws,
                                                        const float* __restrict__ logits, int V, int nch) {
    const int r = blockIdx.x, lane = threadIdx.x;
    AmBest bst{-INFINITY, -1};
    for (int c = lane; c < nch; c += 64) {            // chunks in index order per lane
        const float2 w = ws[(size_t)r * nch + c];
        bst = am_pick(bst, AmBest{w.x, __float_as_int(w.y)});
    }
    for (int o = 1; o < 64; o <<= 1) {                // lane-order tree: the lower lane is earlier
        const float ov = __shfl_down(bst.v, o, 64);
        const int oi = __shfl_down(bst.i, o, 64);
        if ((lane & (2 * o - 1)) == 0 && lane + o < 64) bst = am_pick(bst, AmBest{ov, oi});
    }
    if (lane == 0) {
        const float p0 = logits[(size_t)r * V];
        out[r] = (p0 != p0 || bst.i < 0) ? 0 : bst.i;
    }
}

size_t argmax_workspace_bytes(int B, int V) {
    return (size_t)B * ((V + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK) * sizeof(float2);
}

int launch_argmax_rows(int32_t* out, float* logits, int B, int V, void* ws, hipStream_t s, const RowNorm* rn) {
    if (B <= 0) return 0;
    if (!ws || V <= 0) { set_error(-1, "argmax: bad arguments"); return -1; }
    const int nch = (V + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    hipLaunchKernelGGL(argmax_part_kernel, dim3(nch, B), dim3(256), 0, s, (float2*)ws, logits, V, nch,
                       rn ? *rn : RowNorm{});
    hipLaunchKernelGGL(argmax_fin_kernel, dim3(B), dim3(64), 0, s, out, (const float2*)ws, logits, V, nch);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// Ragged-batch packing: one workgroup scans n_new (B <= 1024) and writes the
// per-token indices.  status[0] = 0 ok, -1 bad descriptor, -2 over capacity.
__global__ __launch_bounds__(1024) void pack_batch_kernel(
    const int32_t* __restrict__ slot, const int32_t* __restrict__ pos0, const int32_t* __restrict__ n_new,
    int B, int max_seq, int64_t slot_stride, int T_cap, int32_t* __restrict__ tok_off,
    int32_t* __restrict__ tok2seq, int32_t* __restrict__ tok_pos, int64_t* __restrict__ kv_base,
    int32_t* __restrict__ last_tok, int32_t* __restrict__ status) {
    __shared__ int32_t scan[1024];
    __shared__ int32_t err;
    const int b = threadIdx.x;
    if (b == 0) err = 0;
    __syncthreads();
    int n = 0;
    if (b < B) {
        n = n_new[b];
        int p0 = pos0[b];
        if (n < 1 || p0 < 0 || slot[b] < 0) atomicMin(&err, -1);
        else if ((int64_t)p0 + n > max_seq) atomicMin(&err, -2);
    }
    scan[b] = b < B ? n : 0;
    __syncthreads();
    // Hillis-Steele inclusive scan
    for (int o = 1; o < 1024; o <<= 1) {
        int32_t v = b >= o ? scan[b - o] : 0;
        __syncthreads();
        scan[b] += v;
        __syncthreads();
    }
    int32_t total = scan[1023];
    if (b == 0 && err == 0 && total > T_cap) err = -2;
    __syncthreads();
    if (b == 0) status[0] = err;
    if (err != 0) return;
    if (b < B) {
        int32_t end = scan[b], start = end - n;
        tok_off[b] = start;
        if (b == B - 1) tok_off[B] = end;
        kv_base[b] = (int64_t)slot[b] * slot_stride;
        last_tok[b] = end - 1;
        int p0 = pos0[b];
        for (int i = 0; i < n; ++i) {
            tok2seq[start + i] = b;
            tok_pos[start + i] = p0 + i;
        }
    }
}

int launch_pack_batch(const int32_t* slot, const int32_t* pos0, const int32_t* n_new, int B, int max_seq,
                      int64_t slot_stride, int T_cap, int32_t* tok_off, int32_t* tok2seq,
                      int32_t* tok_pos, int64_t* kv_base, int32_t* last_tok, int32_t* status,
                      hipStream_t s) {
    if (B < 1 || B > 1024) return -1;
    hipLaunchKernelGGL(pack_batch_kernel, dim3(1), dim3(1024), 0, s, slot, pos0, n_new, B, max_seq,
                       slot_stride, T_cap, tok_off, tok2seq, tok_pos, kv_base, last_tok, status);
    SH_CHECK_LAUNCH();
    return 0;
}

// ---------------------------------------------------------------------------
// f32 weights.  Y[b, m] = sum_k X[b, k] * W[m, k]: one wave per output row m,
// lanes stride K, wave reduction; up to 16 batch rows per pass reuse each
// loaded W element (one pass over W for B <= 16).
template <int BT>
__global__ __launch_bounds__(256) void mm_f32_kernel(float* __restrict__ Y, const float* __restrict__ X,
                                                     const float* __restrict__ W, int B, int M, int K,
                                                     int ldy) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (m >= M) return;
    const float* w = W + (size_t)m * K;
    for (int b0 = 0; b0 < B; b0 += BT) {
        const int nb = min(BT, B - b0);
        float acc[BT];
#pragma unroll
        for (int i = 0; i < BT; ++i) acc[i] = 0.f;
        for (int k = lane; k < K; k += 64) {
            const float wv = w[k];
#pragma unroll
            for (int i = 0; i < BT; ++i)
                if (i < nb) acc[i] = __builtin_fmaf(wv, X[(size_t)(b0 + i) * K + k], acc[i]);
        }
#pragma unroll
        for (int i = 0; i < BT; ++i) {
            float v = acc[i];
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == 0 && i < nb) Y[(size_t)(b0 + i) * ldy + m] = v;
        }
    }
}

int launch_mm_f32(float* Y, const float* X, const float* W, int B, int M, int K, int ldy, hipStream_t s) {
    if (B <= 0 || M <= 0) return 0;
    if (B <= 4)
        hipLaunchKernelGGL(mm_f32_kernel<4>, dim3((M + 3) / 4), dim3(256), 0, s, Y, X, W, B, M, K, ldy);
    else
        hipLaunchKernelGGL(mm_f32_kernel<16>, dim3((M + 3) / 4), dim3(256), 0, s, Y, X, W, B, M, K, ldy);
    SH_CHECK_LAUNCH();
    return 0;
}

// C[b, n] = sum_k X[b, k] * W[k, n] (W is [K, N] for linear_batch, backend.h:58-61).
// A workgroup owns 64 columns and LB_ROWS batch rows: lanes over n
// (coalesced W rows), the four waves over k (k = wave mod 4), each W element
// loaded once for all the rows, the waves' sums combined in LDS in a fixed
// order.
constexpr int LB_ROWS = 8;
__global__ __launch_bounds__(256) void linear_batch_kernel(float* __restrict__ C, const float* __restrict__ X,
                                                           const float* __restrict__ W, int B, int K, int N) {
    __shared__ float red[4][LB_ROWS][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n = blockIdx.x * 64 + lane;
    const int b0 = blockIdx.y * LB_ROWS;
    const int nb = min(LB_ROWS, B - b0);
    float acc[LB_ROWS];
#pragma unroll
    for (int i = 0; i < LB_ROWS; ++i) acc[i] = 0.f;
    if (n < N) {
        for (int k = wv; k < K; k += 4) {
            const float w = W[(size_t)k * N + n];
#pragma unroll
            for (int i = 0; i < LB_ROWS; ++i)
                if (i < nb) acc[i] = __builtin_fmaf(X[(size_t)(b0 + i) * K + k], w, acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < LB_ROWS; ++i) red[wv][i][lane] = acc[i];
    __syncthreads();
    if (wv == 0 && n < N) {
        for (int i = 0; i < nb; ++i)
            C[(size_t)(b0 + i) * N + n] = (red[0][i][lane] + red[1][i][lane]) + (red[2][i][lane] + red[3][i][lane]);
    }
}

int launch_linear_batch(float* C, const float* X, const float* W, int B, int K, int N, hipStream_t s) {
    if (B <= 0 || N <= 0) return 0;
    hipLaunchKernelGGL(linear_batch_kernel, dim3((N + 63) / 64, (B + LB_ROWS - 1) / LB_ROWS), dim3(256), 0, s, C,
                       X, W, B, K, N);
    SH_CHECK_LAUNCH();
    return 0;
}

}  // namespace slate_hip
