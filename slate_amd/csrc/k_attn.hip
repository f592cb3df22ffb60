// k_attn.hip -- ragged GQA attention over per-sequence KV caches.
//
// Semantics (llama_infer.c:97-129, applied per packed token): q head hq of
// token t reads kv head hq / (Hq/Hkv) of the token's own sequence over key
// positions 0..tok_pos[t]; score = (q . k) * (1/sqrtf(hd)); softmax; sum p*V.
//
// Work unit = (key chunk, query block, kv head).  A query block is QB
// consecutive tokens of one sequence (QB = 1 for decode tokens; prompt
// chunks use QB = 32/G), so each K/V chunk is streamed from HBM once for all
// G = Hq/Hkv query heads of the group and all tokens of the block, with the
// causal limit applied per token.  Each unit leaves a partial (running max,
// running sum, unnormalised output) per (token, q head, chunk); a merge kernel
// combines the chunks with log-sum-exp rescaling.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "launch.h"
#include "act16.h"
#include "lanes.h"
#include "rowops.h"
#include "mfma.h"

namespace slate_hip {

constexpr int ATT_THREADS = 256;
constexpr int ATT_CHUNK = 256;       // keys per work unit (one per thread in the score phase)

// Partial layout: po[((t * Hq + hq) * nch_max + c) * HD + d], pml[(...) * 2 + {m, l}]
template <int HD, int G, int QB>
__global__ __launch_bounds__(ATT_THREADS) void attn_block_kernel(
    const float* __restrict__ q, const float* __restrict__ Kp, const float* __restrict__ Vp,
    const int32_t* __restrict__ qblk_t0, const int32_t* __restrict__ qblk_n,
    const int32_t* __restrict__ tok2seq, const int32_t* __restrict__ tok_pos,
    const int64_t* __restrict__ kv_base, int Hq, int64_t head_stride, int nch_max,
    float* __restrict__ po, float* __restrict__ pml) {
    constexpr int R = QB * G;                      // query rows of the block
    constexpr int KPT = ATT_THREADS / HD;          // key lanes in the PV phase
    __shared__ float sq[R * HD];
    __shared__ float sp[R * ATT_THREADS];
    __shared__ float salpha[R];
    __shared__ float so[(KPT > 1 ? KPT - 1 : 1) * R * HD];

    const int c = blockIdx.x, h = blockIdx.z;
    const int t0 = qblk_t0 ? qblk_t0[blockIdx.y] : blockIdx.y;
    const int n = qblk_n ? qblk_n[blockIdx.y] : 1;
    const int p0 = tok_pos[t0];
    const int L = p0 + n;                          // keys 0..p0+n-1 over the block
    const int k0 = c * ATT_CHUNK;
    if (k0 >= L) return;                           // merge never reads chunks past a token's end
    const int k1 = min(L, k0 + ATT_CHUNK);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t base = kv_base[tok2seq[t0]] + (int64_t)h * head_stride;
    const float* Kh = Kp + base;
    const float* Vh = Vp + base;
    for (int idx = tid; idx < R * HD; idx += ATT_THREADS) {
        int r = idx / HD, d = idx - r * HD;
        int i = r / G, gi = r - i * G;
        sq[idx] = i < n ? q[(size_t)(t0 + i) * Hq * HD + (size_t)(h * G + gi) * HD + d] : 0.f;
    }
    __syncthreads();

    // running max / sum per row live in lanes of wave (r % 4): row r is owned by
    // wave r & 3 in the softmax phase; all lanes of that wave keep a copy.
    float m_run[(R + 3) / 4], l_run[(R + 3) / 4];
#pragma unroll
    for (int j = 0; j < (R + 3) / 4; ++j) { m_run[j] = -INFINITY; l_run[j] = 0.f; }
    float o_acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) o_acc[r] = 0.f;
    const int dd = tid % HD, kq = tid / HD;

    for (int kt = k0; kt < k1; kt += ATT_THREADS) {
        const int nk = min(ATT_THREADS, k1 - kt);
        // ---- scores: one key per thread, all rows of the block
        {
            float a[R];
#pragma unroll
            for (int r = 0; r < R; ++r) a[r] = 0.f;
            if (tid < nk) {
                const float4* kr = (const float4*)(Kh + (int64_t)(kt + tid) * HD);
#pragma unroll 4
                for (int d4 = 0; d4 < HD / 4; ++d4) {
                    const float4 kv = kr[d4];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        if (r / G < n) {
                            const float4 qv = *(const float4*)(sq + r * HD + 4 * d4);
                            a[r] = __builtin_fmaf(qv.x, kv.x, a[r]);
                            a[r] = __builtin_fmaf(qv.y, kv.y, a[r]);
                            a[r] = __builtin_fmaf(qv.z, kv.z, a[r]);
                            a[r] = __builtin_fmaf(qv.w, kv.w, a[r]);
                        }
                    }
                }
            }
            const int key = kt + tid;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int i = r / G;
                bool ok = tid < nk && i < n && key <= p0 + i;     // causal limit of token i
                sp[r * ATT_THREADS + tid] = ok ? a[r] * scale : -INFINITY;
            }
        }
        __syncthreads();
        // ---- online softmax: wave w owns rows w, w+4, ...
#pragma unroll
        for (int j = 0; j < (R + 3) / 4; ++j) {
            const int r = wv + 4 * j;
            if (r < R) {
                float v0 = sp[r * ATT_THREADS + lane], v1 = sp[r * ATT_THREADS + lane + 64];
                float v2 = sp[r * ATT_THREADS + lane + 128], v3 = sp[r * ATT_THREADS + lane + 192];
                const float mx = wave_max(fmaxf(fmaxf(v0, v1), fmaxf(v2, v3)));
                const float mnew = fmaxf(m_run[j], mx);
                const float alpha = m_run[j] == -INFINITY ? 0.f : expf(m_run[j] - mnew);
                float e0 = v0 == -INFINITY ? 0.f : expf(v0 - mnew);
                float e1 = v1 == -INFINITY ? 0.f : expf(v1 - mnew);
                float e2 = v2 == -INFINITY ? 0.f : expf(v2 - mnew);
                float e3 = v3 == -INFINITY ? 0.f : expf(v3 - mnew);
                sp[r * ATT_THREADS + lane] = e0;
                sp[r * ATT_THREADS + lane + 64] = e1;
                sp[r * ATT_THREADS + lane + 128] = e2;
                sp[r * ATT_THREADS + lane + 192] = e3;
                const float s = wave_sum((e0 + e1) + (e2 + e3));
                l_run[j] = l_run[j] * alpha + s;
                m_run[j] = mnew;
                if (lane == 0) salpha[r] = alpha;
            }
        }
        __syncthreads();
        // ---- PV: thread (dd, kq) sums keys kq, kq+KPT, ... for every row
#pragma unroll
        for (int r = 0; r < R; ++r) o_acc[r] *= salpha[r];
        for (int k = kq; k < nk; k += KPT) {
            const float v = Vh[(int64_t)(kt + k) * HD + dd];
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (r / G < n) o_acc[r] = __builtin_fmaf(sp[r * ATT_THREADS + k], v, o_acc[r]);
        }
        __syncthreads();
    }
    // reduce o over the KPT key lanes
    if (KPT > 1) {
        if (kq > 0)
#pragma unroll
            for (int r = 0; r < R; ++r) so[((kq - 1) * R + r) * HD + dd] = o_acc[r];
        __syncthreads();
        if (kq == 0)
            for (int j = 1; j < KPT; ++j)
#pragma unroll
                for (int r = 0; r < R; ++r) o_acc[r] += so[((j - 1) * R + r) * HD + dd];
    }
    if (kq == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = r / G;
            if (i < n && k0 <= p0 + i) {              // chunk holds at least one key of token i
                size_t pidx = ((size_t)(t0 + i) * Hq + h * G + (r - i * G)) * nch_max + c;
                po[pidx * HD + dd] = o_acc[r];
            }
        }
    }
    // m, l of the rows owned by this wave
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < (R + 3) / 4; ++j) {
            const int r = wv + 4 * j;
            if (r < R) {
                const int i = r / G;
                if (i < n && k0 <= p0 + i) {
                    size_t pidx = ((size_t)(t0 + i) * Hq + h * G + (r - i * G)) * nch_max + c;
                    pml[pidx * 2 + 0] = m_run[j];
                    pml[pidx * 2 + 1] = l_run[j];
                }
            }
        }
    }
}

// The (decode token, key chunk) work units that hold keys, in token order:
// Decode work-unit list, built once per step: pairs[0] = count, then from
// pairs + 4 (16-byte aligned) one int4 per unit {t * 65536 + c, pos,
// kv_base low, kv_base high} for token list entry i (token t = dec_t0[i], or
// i) and key chunk c < ceil((pos + 1) / ATT_CHUNK).  A unit's kernel thus
// reads everything it needs before its first K load in one round trip.  One
// workgroup; a block-wide scan per 1024 tokens.  Decode kernels launch
// n_dec * nch_max units along x and take unit u from this list, so every
// unit that streams keys is dispatched before the empty ones.
__global__ __launch_bounds__(1024) void attn_pairs_kernel(const int32_t* __restrict__ dec_t0, int n_dec,
                                                          const int32_t* __restrict__ tok_pos,
                                                          const int32_t* __restrict__ tok2seq,
                                                          const int64_t* __restrict__ kv_base, int nch_max,
                                                          int32_t* __restrict__ pairs, AttnXcd xq, int Hkv) {
    __shared__ int s_scan[1024];
    __shared__ int s_base;
    const int tid = threadIdx.x;
    int4* units = (int4*)(pairs + 4);
    if (tid == 0) s_base = 0;
    __syncthreads();
    for (int i0 = 0; i0 < n_dec; i0 += 1024) {
        const int i = i0 + tid;
        int n = 0, t = 0, p = 0;
        int64_t kvb = 0;
        if (i < n_dec) {
            t = dec_t0 ? dec_t0[i] : i;
            p = tok_pos[t];
            kvb = kv_base[tok2seq[t]];
            n = min((p + ATT_CHUNK) / ATT_CHUNK, nch_max);
        }
        s_scan[tid] = n;
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            const int v = tid >= o ? s_scan[tid - o] : 0;
            __syncthreads();
            s_scan[tid] += v;
            __syncthreads();
        }
        const int base = s_base + s_scan[tid] - n;
        for (int c = 0; c < n; ++c)
            units[base + c] = make_int4(t * 65536 + c, p, (int)(uint32_t)((uint64_t)kvb & 0xffffffffu),
                                        (int)(uint32_t)((uint64_t)kvb >> 32));
        if (xq.len && i < n_dec) {
            // the per-XCD queues when Hkv % 8 == 0: pair (t, h) goes to queue
            // h % 8, after Hkv / 8 pairs of every earlier token and the
            // token's own heads h - 8, h - 16, ...
            for (int h = 0; h < Hkv; ++h) {
                int4* q = xq.units + (size_t)(h & 7) * xq.cap + (Hkv >> 3) * base + (h >> 3) * n;
                for (int c = 0; c < n; ++c)
                    q[c] = make_int4(t * 65536 + c, p, (int)(uint32_t)((uint64_t)kvb & 0xffffffffu),
                                     (int)((uint32_t)((uint64_t)kvb >> 32) | ((uint32_t)h << 24)));
                xq.arrive[t * Hkv + h] = 0;
            }
        }
        __syncthreads();
        if (tid == 1023) s_base += s_scan[1023];
        __syncthreads();
    }
    if (tid == 0) pairs[0] = s_base;
    if (xq.len && tid < 8) xq.len[tid] = (Hkv >> 3) * s_base;
    if (xq.len && tid == 0) xq.stepc[0] = xq.stepc[0] + 1;   // a new sequence of launch tags
}

// Unit u of the list (both loads issued before either is used; u may lie
// past the count, inside the list's storage, for the grid's empty tail).
struct AttnUnit { int n, t, c, p; int64_t kvb; };
__device__ __forceinline__ AttnUnit attn_unit(const int32_t* pairs, int u) {
    const int n = pairs[0];
    const int4 d = ((const int4*)(pairs + 4))[u];
    AttnUnit r;
    r.n = n;
    r.t = d.x >> 16;
    r.c = d.x & 0xffff;
    r.p = d.y;
    r.kvb = (int64_t)(((uint64_t)(uint32_t)d.w << 32) | (uint64_t)(uint32_t)d.z);
    return r;
}

// Work-unit list storage inside the pml buffer (16-byte aligned).
__host__ __device__ inline int32_t* attn_unit_list(float* pml, int T, int Hq, int nch_max) {
    const uintptr_t a = (uintptr_t)(pml + (size_t)T * Hq * nch_max * 2);
    return (int32_t*)((a + 15) & ~(uintptr_t)15);
}

// Four consecutive K/V elements as floats: f32 caches load 16 bytes, f16
// caches 8 bytes converted exactly.
__device__ __forceinline__ float4 ld_kv4(const float* p) { return *(const float4*)p; }
typedef _Float16 kv_half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ld_kv4(const _Float16* p) {
    const uint2 r = *(const uint2*)p;
    const kv_half2_t a = __builtin_bit_cast(kv_half2_t, r.x), b = __builtin_bit_cast(kv_half2_t, r.y);
    return make_float4((float)a.x, (float)a.y, (float)b.x, (float)b.y);
}
// Eight f16 K/V values (16 bytes) as two float4: elements 0-3 and 4-7.
__device__ __forceinline__ void ld_kv8(const _Float16* p, float4& lo, float4& hi) {
    const uint4 r = *(const uint4*)p;
    const kv_half2_t a = __builtin_bit_cast(kv_half2_t, r.x), b = __builtin_bit_cast(kv_half2_t, r.y);
    const kv_half2_t c = __builtin_bit_cast(kv_half2_t, r.z), d = __builtin_bit_cast(kv_half2_t, r.w);
    lo = make_float4((float)a.x, (float)a.y, (float)b.x, (float)b.y);
    hi = make_float4((float)c.x, (float)c.y, (float)d.x, (float)d.y);
}

// Decode steps in which every sequence adds one token: the attention unit
// also does what rope_kv_kernel does for its token and kv head, from the
// QKV split partials (same expressions, same results).  part / nsplit /
// split_stride / qkv_ld: the partials; cs: the rotation table; rn: the
// deferred RMSNorm factor (rn.ssq null: none); Kw / Vw: the caches written.
struct AttnRope {
    const float* part;
    int nsplit;
    int64_t split_stride;
    int qkv_ld;
    const float* cs;
    RowNorm rn;
    void *Kw, *Vw;
};

// The G query heads of kv head h for token t, rotated, into sq[G][HD]; when
// `append`, the token's K and V rows of kv head h are written at position p
// (kvb: the sequence's rows of kv head h).  Threads of one workgroup; the caller orders the
// results with a barrier (and a fence for the rows).
template <int HD, int G, typename KVT>
__device__ __forceinline__ void attn_rope_prologue(const AttnRope& fr, int t, int h, int p, int64_t kvb, int Hq,
                                                   int Hkv, bool append, float (*sq)[HD]) {
#pragma clang fp contract(off)
    constexpr int half = HD / 2;
    const int tid = threadIdx.x;
    const int ap = p < 0 ? -p : p;
    const float sg = p < 0 ? -1.0f : 1.0f;
    const float* pr = fr.part + (size_t)t * fr.qkv_ld;
    const RowNorm& rn = fr.rn;
    RmsPre rp;
    if (rn.ssq) rp = row_rms_load(rn.ssq, t, rn.nblk);
    float inv = 1.0f;
    auto scale = [&](float v) { return rn.ssq ? v * inv : v; };
    for (int idx = tid; idx < G * half; idx += ATT_THREADS) {
        const int gi = idx / half, i = idx - gi * half;
        const int c0 = (h * G + gi) * HD + i;
        const Split1 pa = split_load1(pr + c0, fr.nsplit, fr.split_stride);
        const Split1 pb = split_load1(pr + c0 + half, fr.nsplit, fr.split_stride);
        const float c = fr.cs[((size_t)ap * half + i) * 2 + 0];
        const float sn = sg * fr.cs[((size_t)ap * half + i) * 2 + 1];
        if (rn.ssq) inv = row_rms_fin(rp, rn.ssq, t, rn.nblk, rn.D, rn.eps);
        const float a = scale(split_fin1(pa, pr + c0, fr.nsplit, fr.split_stride));
        const float b = scale(split_fin1(pb, pr + c0 + half, fr.nsplit, fr.split_stride));
        sq[gi][i] = a * c - b * sn;
        sq[gi][i + half] = a * sn + b * c;
    }
    if (!append) return;
    KVT* Kw = (KVT*)fr.Kw;
    KVT* Vw = (KVT*)fr.Vw;
    const int D = Hq * HD, kvd = Hkv * HD;
    for (int i = tid; i < half; i += ATT_THREADS) {
        const int ck = D + h * HD + i, cv = D + kvd + h * HD + i;
        const Split1 pa = split_load1(pr + ck, fr.nsplit, fr.split_stride);
        const Split1 pb = split_load1(pr + ck + half, fr.nsplit, fr.split_stride);
        const Split1 pv0 = split_load1(pr + cv, fr.nsplit, fr.split_stride);
        const Split1 pv1 = split_load1(pr + cv + half, fr.nsplit, fr.split_stride);
        const float c = fr.cs[((size_t)ap * half + i) * 2 + 0];
        const float sn = sg * fr.cs[((size_t)ap * half + i) * 2 + 1];
        const int64_t base = kvb + (int64_t)p * HD;
        if (rn.ssq) inv = row_rms_fin(rp, rn.ssq, t, rn.nblk, rn.D, rn.eps);
        const float a = scale(split_fin1(pa, pr + ck, fr.nsplit, fr.split_stride));
        const float b = scale(split_fin1(pb, pr + ck + half, fr.nsplit, fr.split_stride));
        Kw[base + i] = (KVT)(a * c - b * sn);
        Kw[base + i + half] = (KVT)(a * sn + b * c);
        Vw[base + i] = (KVT)scale(split_fin1(pv0, pr + cv, fr.nsplit, fr.split_stride));
        Vw[base + i + half] = (KVT)scale(split_fin1(pv1, pr + cv + half, fr.nsplit, fr.split_stride));
    }
}

// Decode work unit (one query token per sequence): (key chunk, token, kv
// head), G query heads.  Every K and V row of the chunk is read once, whole
// and coalesced:
//   scores  8 lanes per key row, lane ls holds dims 32i + 4ls .. +3 of the
//           row and of the G query slices (each load instruction of a wave
//           covers 8 rows x 128 contiguous bytes); dot products reduce over
//           the 8 lanes;
//   softmax over the chunk (max, exp, sum) per query head in LDS;
//   PV      HD/4 lanes per V row (64/(HD/4) rows per wave instruction), the
//           probabilities broadcast from LDS, reduced over lanes and waves.
// Partials (chunk max m, sum l, unnormalised output) as attn_block_kernel.
// With ROPE the unit first runs attn_rope_prologue (q from LDS afterwards).
template <int HD, int G, typename KVT, bool ROPE>
__device__ __forceinline__ void attn_dec_body(const float* q, const KVT* Kp, const KVT* Vp, const int32_t* pairs,
                                              int Hq, int64_t head_stride, int nch_max, float* po, float* pml,
                                              const AttnRope& fr, int Hkv) {
    constexpr int NV = HD / 32;
    constexpr int LPR = HD / 4;
    constexpr int KPI = 64 / LPR;
    __shared__ float sp[G][ATT_CHUNK];
    __shared__ float4 sred[4][G][LPR];
    __shared__ float s_q[ROPE ? G : 1][ROPE ? HD : 1];
    // work unit blockIdx.x of the (token, chunk) list that attn_pairs_kernel
    // wrote; the units past its count are the grid's empty tail
    const AttnUnit un = attn_unit(pairs, blockIdx.x);
    if ((int)blockIdx.x >= un.n) return;
    const int c = un.c, h = blockIdx.z, t = un.t, p = un.p;
    const int k0 = c * ATT_CHUNK;
    if (k0 > p) return;                            // merge never reads chunks past a token's end
    const int nk = min(p + 1 - k0, ATT_CHUNK);
    const int nkp = (nk + 31) & ~31;               // rounds of 32 keys (multiple of 4 * KPI)
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int lg = lane >> 3, ls = lane & 7;
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t base = un.kvb + (int64_t)h * head_stride + (int64_t)k0 * HD;
    if constexpr (ROPE) {
        // the unit of the chunk holding key p appends the token's K and V
        // rows; the fence and barrier make them visible to the key loads
        const bool append = p - k0 < ATT_CHUNK;
        attn_rope_prologue<HD, G, KVT>(fr, t, h, p, un.kvb + (int64_t)h * head_stride, Hq, Hkv, append, s_q);
        if (append) __threadfence_block();
        __syncthreads();
    }
    const KVT* Kh = Kp + base;
    const KVT* Vh = Vp + base;
    const float* qt = q + (size_t)t * Hq * HD + (size_t)h * G * HD;
    float4 qv[G][NV];
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
        for (int i = 0; i < NV; ++i)
            qv[gi][i] = ROPE ? *(const float4*)(&s_q[gi][32 * i + 4 * ls])
                             : *(const float4*)(qt + gi * HD + 32 * i + 4 * ls);

    // ---- scores
#pragma unroll 2
    for (int j0 = 0; j0 < nkp; j0 += 32) {
        const int j = j0 + 8 * wv + lg;
        const KVT* kr = Kh + (int64_t)min(j, nk - 1) * HD;   // clamped: stays inside the token's keys
        float4 kv[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) kv[i] = ld_kv4(kr + 32 * i + 4 * ls);
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                a = __builtin_fmaf(qv[gi][i].x, kv[i].x, a);
                a = __builtin_fmaf(qv[gi][i].y, kv[i].y, a);
                a = __builtin_fmaf(qv[gi][i].z, kv[i].z, a);
                a = __builtin_fmaf(qv[gi][i].w, kv[i].w, a);
            }
            a = group8_sum(a);
            if (ls == 0) sp[gi][j] = j < nk ? a * scale : -INFINITY;
        }
    }
    __syncthreads();
    // ---- softmax over the chunk, one wave per query head
    for (int gi = wv; gi < G; gi += 4) {
        float mx = -INFINITY;
        for (int j = lane; j < nkp; j += 64) mx = fmaxf(mx, sp[gi][j]);
        mx = wave_max(mx);
        float sum = 0.f;
        for (int j = lane; j < nkp; j += 64) {
            const float sc = sp[gi][j];
            const float e = sc == -INFINITY ? 0.f : expf(sc - mx);
            sp[gi][j] = e;
            sum += e;
        }
        sum = wave_sum(sum);
        if (lane == 0) {
            const size_t pidx = ((size_t)t * Hq + h * G + gi) * nch_max + c;
            pml[pidx * 2 + 0] = mx;
            pml[pidx * 2 + 1] = sum;
        }
    }
    __syncthreads();
    // ---- PV
    const int kof = lane / LPR, d4 = lane % LPR;
    float4 acc[G];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) acc[gi] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int j = wv * KPI + kof; j < nkp; j += 4 * KPI) {
        const float4 vv = ld_kv4(Vh + (int64_t)min(j, nk - 1) * HD + 4 * d4);
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const float pj = sp[gi][j];
            acc[gi].x = __builtin_fmaf(pj, vv.x, acc[gi].x);
            acc[gi].y = __builtin_fmaf(pj, vv.y, acc[gi].y);
            acc[gi].z = __builtin_fmaf(pj, vv.z, acc[gi].z);
            acc[gi].w = __builtin_fmaf(pj, vv.w, acc[gi].w);
        }
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
        for (int o = LPR; o < 64; o <<= 1) {
            acc[gi].x += __shfl_xor(acc[gi].x, o, 64);
            acc[gi].y += __shfl_xor(acc[gi].y, o, 64);
            acc[gi].z += __shfl_xor(acc[gi].z, o, 64);
            acc[gi].w += __shfl_xor(acc[gi].w, o, 64);
        }
    if (kof == 0)
#pragma unroll
        for (int gi = 0; gi < G; ++gi) sred[wv][gi][d4] = acc[gi];
    __syncthreads();
    for (int idx = tid; idx < G * LPR; idx += ATT_THREADS) {
        const int gi = idx / LPR, dd = idx - gi * LPR;
        float4 o = sred[0][gi][dd];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const float4 o2 = sred[w][gi][dd];
            o.x += o2.x; o.y += o2.y; o.z += o2.z; o.w += o2.w;
        }
        const size_t pidx = ((size_t)t * Hq + h * G + gi) * nch_max + c;
        *(float4*)(po + pidx * HD + 4 * dd) = o;
    }
}

template <int HD, int G, typename KVT>
__global__ __launch_bounds__(ATT_THREADS) void attn_dec_kernel(
    const float* __restrict__ q, const KVT* __restrict__ Kp, const KVT* __restrict__ Vp,
    const int32_t* __restrict__ dec_t0, const int32_t* __restrict__ tok2seq, const int32_t* __restrict__ tok_pos,
    const int64_t* __restrict__ kv_base, int Hq, int64_t head_stride, int nch_max, float* __restrict__ po,
    float* __restrict__ pml, const int32_t* __restrict__ pairs) {
    attn_dec_body<HD, G, KVT, false>(q, Kp, Vp, pairs, Hq, head_stride, nch_max, po, pml, AttnRope{}, 0);
}

// The phased unit with the rotation and KV append of the step's tokens (one
// token per sequence); Kp / Vp are not __restrict__ (rows written through
// fr.Kw / fr.Vw are read back).
template <int HD, int G, typename KVT>
__global__ __launch_bounds__(ATT_THREADS) void attn_dec_phased_rope_kernel(
    const KVT* Kp, const KVT* Vp, int Hq, int Hkv, int64_t head_stride, int nch_max, float* __restrict__ po,
    float* __restrict__ pml, const int32_t* __restrict__ pairs, AttnRope fr) {
    attn_dec_body<HD, G, KVT, true>(nullptr, Kp, Vp, pairs, Hq, head_stride, nch_max, po, pml, fr, Hkv);
}

// Decode work unit (one query token per sequence): (key chunk, token, kv
// head), G query heads.  Each wave owns 64 keys of the 256-key chunk and
// works through them without barriers:
//   scores  8 lanes per key row (lane ls holds dims 32i + 4ls .. +3 of the
//           row and of the G query slices; one load instruction of a wave
//           covers 8 rows x 128 contiguous bytes), reduced over the 8 lanes
//           by DPP; the wave's 8 x 8 scores per head stay in registers;
//   softmax max and sum over the wave's keys;
//   PV      the same lane owns the same key's V row slice, weighted by its
//           own probability.
// The waves then combine through LDS (log-sum-exp over the four wave
// maxima) into the chunk partial (max m, sum l, unnormalised output), as
// attn_block_kernel writes it.
// With ROPE the unit first runs attn_rope_prologue (q from LDS afterwards).
template <int HD, int G, typename KVT, bool ROPE>
__device__ __forceinline__ void attn_dec_wave_unit(
    const float* q, const KVT* Kp, const KVT* Vp, const AttnUnit& un, int h, int Hq, int64_t head_stride,
    int nch_max, float* po, float* pml, const AttnRope& fr, int Hkv) {
    constexpr int NV = HD / 32;                    // float4 per lane per row
    constexpr int KW = ATT_CHUNK / 4;              // keys per wave
    constexpr int IT = KW / 8;                     // rounds of 8 keys
    __shared__ float4 s_o[4][4][G][HD / 4];        // [wave][16-lane row][head][dims]
    __shared__ float s_m[4][G], s_l[4][G];
    __shared__ float s_q[ROPE ? G : 1][ROPE ? HD : 1];
    const int c = un.c, t = un.t, p = un.p;
    const int k0 = c * ATT_CHUNK;
    if (k0 > p) return;                            // merge never reads chunks past a token's end
    const int nk = min(p + 1 - k0, ATT_CHUNK);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int lg = lane >> 3, ls = lane & 7;
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t base = un.kvb + (int64_t)h * head_stride + (int64_t)k0 * HD;
    const KVT* Kh = Kp + base;
    const KVT* Vh = Vp + base;
    const int kw0 = wv * KW;
    // dims of a row that lane ls holds, as NV float4: f32 rows 32i + 4ls ..
    // +3 (one 16-byte load each); f16 rows (head_dim 64 / 128) in pairs,
    // 64(i/2) + 8ls + 4(i%2) .. +3, so that one 16-byte load brings two
    constexpr bool W16 = sizeof(KVT) == 2 && NV % 2 == 0;
    auto dof = [&](int i) { return W16 ? 64 * (i >> 1) + 8 * ls + 4 * (i & 1) : 32 * i + 4 * ls; };
    auto ld_row = [&](const KVT* row, float4 (&dst)[NV]) {
        if constexpr (W16) {
#pragma unroll
            for (int i = 0; i < NV; i += 2) ld_kv8((const _Float16*)row + dof(i), dst[i], dst[i + 1]);
        } else {
#pragma unroll
            for (int i = 0; i < NV; ++i) dst[i] = ld_kv4(row + dof(i));
        }
    };
    // with ROPE, the first KP rounds of key rows are loaded before the
    // prologue where the chunk does not hold key p (its rows are final), so
    // that their latency overlaps the prologue's
    constexpr int KP = ROPE ? 2 : 0;
    float4 kpre[KP > 0 ? KP : 1][NV];
    auto load_kpre = [&]() {
        if (kw0 < nk) {
#pragma unroll
            for (int it = 0; it < KP; ++it) {
                const KVT* kr = Kh + (int64_t)min(kw0 + 8 * it + lg, nk - 1) * HD;
                ld_row(kr, kpre[it]);
            }
        }
    };
    if constexpr (ROPE) {
        // the unit of the chunk holding key p appends the token's K and V
        // rows; the fence and barrier make them visible to the key loads
        const bool append = p - k0 < ATT_CHUNK;
        if (!append) load_kpre();
        attn_rope_prologue<HD, G, KVT>(fr, t, h, p, un.kvb + (int64_t)h * head_stride, Hq, Hkv, append, s_q);
        if (append) __threadfence_block();
        __syncthreads();
        if (append) load_kpre();
    }
    if (kw0 < nk) {
        const float* qt = q + (size_t)t * Hq * HD + (size_t)h * G * HD;
        float4 qv[G][NV];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int i = 0; i < NV; ++i)
                qv[gi][i] = ROPE ? *(const float4*)(&s_q[gi][dof(i)]) : *(const float4*)(qt + gi * HD + dof(i));
        float sc[G][IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int j = kw0 + 8 * it + lg;
            const KVT* kr = Kh + (int64_t)min(j, nk - 1) * HD;   // clamped: stays inside the token's keys
            float4 kv[NV];
            if (it < KP) {
#pragma unroll
                for (int i = 0; i < NV; ++i) kv[i] = kpre[it < KP ? it : 0][i];
            } else {
                ld_row(kr, kv);
            }
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < NV; ++i) {
                    a = __builtin_fmaf(qv[gi][i].x, kv[i].x, a);
                    a = __builtin_fmaf(qv[gi][i].y, kv[i].y, a);
                    a = __builtin_fmaf(qv[gi][i].z, kv[i].z, a);
                    a = __builtin_fmaf(qv[gi][i].w, kv[i].w, a);
                }
                a = group8_sum(a);
                sc[gi][it] = j < nk ? a * scale : -INFINITY;
            }
        }
        // the first V rows go out before the softmax (which needs no memory),
        // into the registers the K rows no longer use
        constexpr int VP = IT / 4;
        float4 vpre[VP][NV];
#pragma unroll
        for (int it = 0; it < VP; ++it) {
            const KVT* vr = Vh + (int64_t)min(kw0 + 8 * it + lg, nk - 1) * HD;
            ld_row(vr, vpre[it]);
        }
        __builtin_amdgcn_sched_barrier(0);
        float mx[G], sum[G];
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float m = sc[gi][0];
#pragma unroll
            for (int it = 1; it < IT; ++it) m = fmaxf(m, sc[gi][it]);
            mx[gi] = wave_groups_max(m);           // finite: key kw0 is always inside the chunk
            float l = 0.f;
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                const float e = sc[gi][it] == -INFINITY ? 0.f : expf(sc[gi][it] - mx[gi]);
                sc[gi][it] = e;
                l += e;
            }
            sum[gi] = wave_groups_sum(l);
        }
        float4 acc[G][NV];
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int i = 0; i < NV; ++i) acc[gi][i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int j = kw0 + 8 * it + lg;
            const KVT* vr = Vh + (int64_t)min(j, nk - 1) * HD;
            float4 vv[NV];
            if (it < VP) {
#pragma unroll
                for (int i = 0; i < NV; ++i) vv[i] = vpre[it < VP ? it : 0][i];
            } else {
                ld_row(vr, vv);
            }
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                const float pj = sc[gi][it];
#pragma unroll
                for (int i = 0; i < NV; ++i) {
                    acc[gi][i].x = __builtin_fmaf(pj, vv[i].x, acc[gi][i].x);
                    acc[gi][i].y = __builtin_fmaf(pj, vv[i].y, acc[gi][i].y);
                    acc[gi][i].z = __builtin_fmaf(pj, vv[i].z, acc[gi][i].z);
                    acc[gi][i].w = __builtin_fmaf(pj, vv[i].w, acc[gi][i].w);
                }
            }
        }
        // the two lane groups of each 16-lane row; rows are summed below
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                acc[gi][i].x += dpp_mov<DPP_ROW_ROR8>(acc[gi][i].x);
                acc[gi][i].y += dpp_mov<DPP_ROW_ROR8>(acc[gi][i].y);
                acc[gi][i].z += dpp_mov<DPP_ROW_ROR8>(acc[gi][i].z);
                acc[gi][i].w += dpp_mov<DPP_ROW_ROR8>(acc[gi][i].w);
            }
        if ((lane & 8) == 0)
#pragma unroll
            for (int gi = 0; gi < G; ++gi)
#pragma unroll
                for (int i = 0; i < NV; ++i) s_o[wv][lane >> 4][gi][dof(i) >> 2] = acc[gi][i];
        if (lane == 0)
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                s_m[wv][gi] = mx[gi];
                s_l[wv][gi] = sum[gi];
            }
    }
    __syncthreads();
    const int nw = (nk + KW - 1) / KW;             // waves that had keys
    for (int idx = tid; idx < G * (HD / 4); idx += ATT_THREADS) {
        const int gi = idx / (HD / 4), d4 = idx - gi * (HD / 4);
        float M = s_m[0][gi];
        for (int w = 1; w < nw; ++w) M = fmaxf(M, s_m[w][gi]);
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.f;
        for (int w = 0; w < nw; ++w) {
            const float f = expf(s_m[w][gi] - M);
            L += f * s_l[w][gi];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float4 v = s_o[w][r][gi][d4];
                o.x += f * v.x; o.y += f * v.y; o.z += f * v.z; o.w += f * v.w;
            }
        }
        const size_t pidx = ((size_t)t * Hq + h * G + gi) * nch_max + c;
        *(float4*)(po + pidx * HD + 4 * d4) = o;
        if (d4 == 0) {
            pml[pidx * 2 + 0] = M;
            pml[pidx * 2 + 1] = L;
        }
    }
}

// Work unit blockIdx.x of the (token, chunk) list that attn_pairs_kernel
// wrote (kv head blockIdx.z); the units past its count are the grid's
// empty tail.
template <int HD, int G, typename KVT, bool ROPE>
__device__ __forceinline__ void attn_dec_wave_body(
    const float* q, const KVT* Kp, const KVT* Vp, const int32_t* pairs, int Hq, int64_t head_stride, int nch_max,
    float* po, float* pml, const AttnRope& fr, int Hkv) {
    const AttnUnit un = attn_unit(pairs, blockIdx.x);
    if ((int)blockIdx.x >= un.n) return;
    attn_dec_wave_unit<HD, G, KVT, ROPE>(q, Kp, Vp, un, blockIdx.z, Hq, head_stride, nch_max, po, pml, fr, Hkv);
}

template <int HD, int G, typename KVT>
__global__ __launch_bounds__(ATT_THREADS) void attn_dec_wave_kernel(
    const float* __restrict__ q, const KVT* __restrict__ Kp, const KVT* __restrict__ Vp,
    const int32_t* __restrict__ dec_t0, const int32_t* __restrict__ tok2seq, const int32_t* __restrict__ tok_pos,
    const int64_t* __restrict__ kv_base, int Hq, int64_t head_stride, int nch_max, float* __restrict__ po,
    float* __restrict__ pml, const int32_t* __restrict__ pairs) {
    attn_dec_wave_body<HD, G, KVT, false>(q, Kp, Vp, pairs, Hq, head_stride, nch_max, po, pml, AttnRope{}, 0);
}

// The same with the rotation and KV append of the step's tokens (one token
// per sequence).  Kp / Vp are not __restrict__: this kernel writes rows
// through fr.Kw / fr.Vw that its own key loads then read.
template <int HD, int G, typename KVT>
__global__ __launch_bounds__(ATT_THREADS) void attn_dec_rope_kernel(
    const KVT* Kp, const KVT* Vp, int Hq, int Hkv, int64_t head_stride, int nch_max, float* __restrict__ po,
    float* __restrict__ pml, const int32_t* __restrict__ pairs, AttnRope fr) {
    attn_dec_wave_body<HD, G, KVT, true>(nullptr, Kp, Vp, pairs, Hq, head_stride, nch_max, po, pml, fr, Hkv);
}

// Chunk partials of the merge: plain loads (the merge kernel runs after the
// launch that wrote them), or loads that miss in L1 and read L2 (the merge
// inside the decode kernel reads lines other units of the same launch wrote
// to L2 from other CUs of its XCD; buffer loads with sc0, offsets in bytes
// from po and pml, outside them zero).
struct PartPlain {
    const float* po;
    const float* pml;
    __device__ __forceinline__ float2 ml(size_t pc) const { return *(const float2*)(pml + pc * 2); }
    __device__ __forceinline__ float4 o(size_t pc, int HD, int d) const {
        return *(const float4*)(po + pc * HD + d);
    }
};
struct PartL2 {
    __amdgpu_buffer_rsrc_t po, pml;
    __device__ __forceinline__ float2 ml(size_t pc) const {
        return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(pml, (int)(pc * 8), 0, 1));
    }
    __device__ __forceinline__ float4 o(size_t pc, int HD, int d) const {
        return __builtin_bit_cast(float4,
                                  __builtin_amdgcn_raw_buffer_load_b128(po, (int)((pc * HD + d) * 4), 0, 1));
    }
};

// out = sum_c e^{m_c - M} o_c / sum_c e^{m_c - M} l_c over the nch chunks of
// (token, q head) p0 / nch_max, for dims d .. d+3.  The first MB chunks'
// (max, sum) and outputs are loaded in one batch (clamped to the last
// chunk, used under a predicate): one round trip for contexts up to MB
// chunks; the max over every chunk is taken before any chunk is
// accumulated, in chunk order.
template <class P, int MB = 8>
__device__ __forceinline__ float4 merge_chunks(const P& pp, size_t p0, int nch, int HD, int d) {
    float2 ml[MB];
    float4 ov[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const size_t pc = p0 + min(i, max(nch - 1, 0));
        ml[i] = pp.ml(pc);
        ov[i] = pp.o(pc, HD, d);
    }
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < MB; ++i)
        if (i < nch) M = fmaxf(M, ml[i].x);
    for (int c0 = MB; c0 < nch; c0 += MB) {
        float mv[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) mv[i] = pp.ml(p0 + min(c0 + i, nch - 1)).x;
#pragma unroll
        for (int i = 0; i < MB; ++i)
            if (c0 + i < nch) M = fmaxf(M, mv[i]);
    }
    float den = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < MB; ++i)
        if (i < nch) {
            const float f = expf(ml[i].x - M);
            den += f * ml[i].y;
            acc.x += f * ov[i].x; acc.y += f * ov[i].y; acc.z += f * ov[i].z; acc.w += f * ov[i].w;
        }
    for (int c0 = MB; c0 < nch; c0 += MB) {
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const size_t pc = p0 + min(c0 + i, nch - 1);
            ml[i] = pp.ml(pc);
            ov[i] = pp.o(pc, HD, d);
        }
#pragma unroll
        for (int i = 0; i < MB; ++i)
            if (c0 + i < nch) {
                const float f = expf(ml[i].x - M);
                den += f * ml[i].y;
                acc.x += f * ov[i].x; acc.y += f * ov[i].y; acc.z += f * ov[i].z; acc.w += f * ov[i].w;
            }
    }
    const float inv = 1.0f / den;
    return make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

// One wave per 256 output elements of a token row (lane: 4 consecutive
// elements of one head); with `act` the row also goes out as the Q4_K
// activation operand (padding rows t >= T as zeros).
// TILE (with the operand): a 512-thread workgroup per (block, 8-row half
// tile), wave w = row w of the half, the operand written by
// act16_store_tile.
template <bool TILE>
__device__ __forceinline__ void attn_merge_body(float* __restrict__ out, const float* __restrict__ po,
                                                const float* __restrict__ pml, const int32_t* __restrict__ tok_pos,
                                                int T, int Hq, int HD, int nch_max, const Act16& a, int act,
                                                uint4* s_t) {
    const int lane = threadIdx.x & 63;
    const int kb = TILE ? blockIdx.x : blockIdx.x * 4 + (threadIdx.x >> 6);
    const int D = Hq * HD;
    if (!TILE && kb * 256 >= D) return;           // whole wave
    const int t = TILE ? blockIdx.y * 8 + (threadIdx.x >> 6) : blockIdx.y;
    const int e = kb * 256 + 4 * lane;
    float4 res = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < T && e < D) {
        const int hq = e / HD, d = e - hq * HD;
        const int L = tok_pos[t] + 1;
        const int nch = min((L + ATT_CHUNK - 1) / ATT_CHUNK, nch_max);
        res = merge_chunks(PartPlain{po, pml}, ((size_t)t * Hq + hq) * nch_max, nch, HD, d);
        *(float4*)(out + (size_t)t * D + e) = res;
    }
    if constexpr (TILE) act16_store_tile<8>(a, blockIdx.y >> 1, blockIdx.y & 1, kb, s_t, res);
    else if (act) act16_store_block(a, t, kb, lane, res);
}
__global__ __launch_bounds__(256) void attn_merge_kernel(float* __restrict__ out, const float* __restrict__ po,
                                                         const float* __restrict__ pml,
                                                         const int32_t* __restrict__ tok_pos, int T, int Hq,
                                                         int HD, int nch_max, Act16 a, int act) {
    attn_merge_body<false>(out, po, pml, tok_pos, T, Hq, HD, nch_max, a, act, nullptr);
}
__global__ __launch_bounds__(512) void attn_merge_tile_kernel(float* __restrict__ out, const float* __restrict__ po,
                                                               const float* __restrict__ pml,
                                                               const int32_t* __restrict__ tok_pos, int T, int Hq,
                                                               int HD, int nch_max, Act16 a) {
    __shared__ uint4 s_t[ACT_FRAG_UNITS];
    attn_merge_body<true>(out, po, pml, tok_pos, T, Hq, HD, nch_max, a, 1, s_t);
}

// The chunk merge of T query rows into out (and the operand: by 8-row half
// tiles when there is more than one tile).
static void launch_merge(float* out, const float* po, const float* pml, const int32_t* tok_pos, int T, int Hq,
                         int HD, int nch_max, const Act16* act, hipStream_t s, hipEvent_t ev_stop) {
    const int nb = (Hq * HD + 255) / 256;
    if (act && act->rows_pad > 16 && (Hq * HD) % 256 == 0) {
        SH_LAUNCH(nullptr, ev_stop, attn_merge_tile_kernel, dim3(nb, act->rows_pad / 8), dim3(512), 0, s, out, po,
                  pml, tok_pos, T, Hq, HD, nch_max, *act);
        return;
    }
    dim3 mgrid((nb + 3) / 4, act ? act->rows_pad : T);
    SH_LAUNCH(nullptr, ev_stop, attn_merge_kernel, mgrid, dim3(256), 0, s, out, po, pml, tok_pos, T, Hq, HD, nch_max,
              act ? *act : Act16{}, act ? 1 : 0);
}

// ---------------------------------------------------------------------------
// Decode attention with the chunk merge inside (steps in which every
// sequence adds one token).  Workgroups are dealt to the eight XCDs in turn
// and each XCD has its own L2; workgroup i takes its unit from queue i % 8,
// which holds every chunk of the (token, kv head) pairs assigned to it, so
// all of a pair's units run on one XCD as long as the workgroups i with the
// same i % 8 do (a launch whose first workgroup goes to XCD s, with the
// rest following in turn, keeps that).  The unit that finishes a pair's last
// chunk (an atomic count per pair) merges the pair's G heads: its partials
// were written by units of the same XCD, whose stores completed in that L2
// before they counted (a wait for the stores, a barrier, then the count),
// and it reads them with loads that miss in L1.  No writeback of L2 to
// memory is needed, as it would be across XCDs.
//
// Each launch checks that assumption itself: every unit writes a tag beside
// its partial -- the launch's sequence number (the step count the queue
// builder keeps, and the layer) and the XCD it ran on -- and the merging
// unit compares every tag of its pair with its own.  A partial written on
// another XCD cannot show this launch's tag with the merger's XCD (its tag
// is either not visible from this L2 or names the other XCD), so any merge
// that read across XCDs is reported to the host, which runs the step again
// on the separate merge kernel.

__global__ void xcc_probe_kernel(int32_t* out) {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)x;
}

static int device_cus();

// Whether consecutive workgroups of a launch run on consecutive XCDs of an
// eight-XCD device (workgroup i on XCD (i + s) % 8 for the launch's first
// XCD s; measured on MI355X: s = 0 on the null stream, s = 7 on the backend
// stream, the same for every launch), read from the hardware register by 64
// workgroups, once per device and process; -1: not probed yet.
constexpr int XCD_MAX_DEVICES = 64;
static std::atomic<int> g_xcd_rr[XCD_MAX_DEVICES];
static std::once_flag g_xcd_init;
static std::atomic<int>* xcd_flag() {
    std::call_once(g_xcd_init, [] {
        for (auto& f : g_xcd_rr) f.store(-1);
    });
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= XCD_MAX_DEVICES) return nullptr;
    return &g_xcd_rr[dev];
}
bool attention_xcd_probe() {
    std::atomic<int>* f = xcd_flag();
    if (!f) return false;
    int v = f->load();
    if (v >= 0) return v == 1;
    bool ok = device_cus() == 256;
    int32_t* d = nullptr;
    int32_t h[64];
    if (ok) ok = hipMalloc(&d, sizeof h) == hipSuccess;
    if (ok) {
        hipLaunchKernelGGL(xcc_probe_kernel, dim3(64), dim3(64), 0, nullptr, d);
        ok = hipGetLastError() == hipSuccess && hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost) == hipSuccess;
        (void)hipFree(d);
    }
    for (int i = 0; ok && i < 64; ++i) ok = (h[i] & 8) == 0 && ((h[i] - h[0]) & 7) == i % 8;
    f->store(ok ? 1 : 0);
    return ok;
}

static size_t xcd_fixed_ints(int max_tok, int Hkv, size_t nch) {
    return (12 + (size_t)max_tok * Hkv * (1 + nch) + 3) / 4 * 4;
}

size_t attention_xcd_ints(int max_tok, int Hkv, int max_pos) {
    const size_t nch = (size_t)(max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    const size_t cap = ((size_t)max_tok * Hkv + 7) / 8 * nch;
    return xcd_fixed_ints(max_tok, Hkv, nch) + 8 * cap * 4;
}

// Layout of attention_xcd_ints(max_tok, Hkv, max_pos) int32s from a
// 16-byte aligned base: len [8], the step count [1] (+3 padding), arrive,
// tags, then the eight queues.
AttnXcd attention_xcd_view(int32_t* base, int max_tok, int Hkv, int max_pos) {
    const size_t nch = (size_t)(max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    AttnXcd x{};
    x.len = base;
    x.stepc = base + 8;
    x.arrive = base + 12;
    x.tag = x.arrive + (size_t)max_tok * Hkv;
    x.units = (int4*)(base + xcd_fixed_ints(max_tok, Hkv, nch));
    x.max_tok = max_tok;
    x.nch = (int)nch;
    x.cap = (int)(((size_t)max_tok * Hkv + 7) / 8 * nch);
    return x;
}

// The per-XCD queues of the step's decode tokens, one workgroup: per round
// of 1024 tokens, eight block-wide scans of the tokens' unit counts per
// queue; every pair's arrival count reset.
__global__ __launch_bounds__(1024) void attn_xcd_queues_kernel(const int32_t* __restrict__ dec_t0, int n_dec,
                                                               const int32_t* __restrict__ tok_pos,
                                                               const int32_t* __restrict__ tok2seq,
                                                               const int64_t* __restrict__ kv_base, int nch_max,
                                                               int Hkv, AttnXcd xq) {
    __shared__ int s_scan[8][1024];
    __shared__ int s_base[8];
    const int tid = threadIdx.x;
    if (tid < 8) s_base[tid] = 0;
    __syncthreads();
    for (int i0 = 0; i0 < n_dec; i0 += 1024) {
        const int i = i0 + tid;
        int n = 0, t = 0, p = 0;
        int64_t kvb = 0;
        if (i < n_dec) {
            t = dec_t0 ? dec_t0[i] : i;
            p = tok_pos[t];
            kvb = kv_base[tok2seq[t]];
            n = min((p + ATT_CHUNK) / ATT_CHUNK, nch_max);
        }
        int cnt[8];
#pragma unroll
        for (int x = 0; x < 8; ++x) cnt[x] = 0;
        for (int h = 0; h < Hkv && i < n_dec; ++h) {
            const int x = (t * Hkv + h) & 7;
#pragma unroll
            for (int y = 0; y < 8; ++y) cnt[y] += y == x ? n : 0;
            xq.arrive[t * Hkv + h] = 0;
        }
#pragma unroll
        for (int x = 0; x < 8; ++x) s_scan[x][tid] = cnt[x];
        __syncthreads();
        for (int o = 1; o < 1024; o <<= 1) {
            int v[8];
#pragma unroll
            for (int x = 0; x < 8; ++x) v[x] = tid >= o ? s_scan[x][tid - o] : 0;
            __syncthreads();
#pragma unroll
            for (int x = 0; x < 8; ++x) s_scan[x][tid] += v[x];
            __syncthreads();
        }
        int run[8];
#pragma unroll
        for (int x = 0; x < 8; ++x) run[x] = s_base[x] + s_scan[x][tid] - cnt[x];
        for (int h = 0; h < Hkv && i < n_dec; ++h) {
            const int x = (t * Hkv + h) & 7;
            int r = 0;
#pragma unroll
            for (int y = 0; y < 8; ++y) r = y == x ? run[y] : r;
            int4* q = xq.units + (size_t)x * xq.cap + r;
            for (int c = 0; c < n; ++c)
                q[c] = make_int4(t * 65536 + c, p, (int)(uint32_t)((uint64_t)kvb & 0xffffffffu),
                                 (int)((uint32_t)((uint64_t)kvb >> 32) | ((uint32_t)h << 24)));
#pragma unroll
            for (int y = 0; y < 8; ++y) run[y] += y == x ? n : 0;
        }
        __syncthreads();
        if (tid == 1023)
#pragma unroll
            for (int x = 0; x < 8; ++x) s_base[x] += s_scan[x][1023];
        __syncthreads();
    }
    if (tid < 8) xq.len[tid] = s_base[tid];
    if (tid == 0) xq.stepc[0] = xq.stepc[0] + 1;   // a new sequence of launch tags
}

// One unit per workgroup: workgroup i takes unit i / 8 of queue i % 8 (the
// workgroups of one queue share an XCD, as the dispatch order gives and the
// tags check); the grid covers the longest queue and the surplus workgroups
// exit.
template <int HD, int G, typename KVT>
__global__ __launch_bounds__(ATT_THREADS) void attn_dec_rope_xcd_kernel(
    const KVT* Kp, const KVT* Vp, int Hq, int Hkv, int64_t head_stride, int nch_max, float* __restrict__ po,
    float* __restrict__ pml, uint32_t po_bytes, uint32_t pml_bytes, AttnRope fr, AttnXcd xq,
    float* __restrict__ out, Act16 a, int act) {
    constexpr int NB = G * HD / 256;                   // operand blocks of a kv head's G heads
    __shared__ int s_last;
    const int xcc = blockIdx.x & 7, u = blockIdx.x >> 3;
    // the queue length and the unit are read together (one round trip);
    // u < cap for every workgroup of the grid, so the unit read is in bounds
    const int len = xq.len[xcc];
    const int4 d = xq.units[(size_t)xcc * xq.cap + u];
    if (u >= len) return;                              // workgroup-uniform
    AttnUnit un;
    un.n = 0;
    un.t = d.x >> 16;
    un.c = d.x & 0xffff;
    un.p = d.y;
    un.kvb = (int64_t)(((uint64_t)((uint32_t)d.w & 0xffffffu) << 32) | (uint64_t)(uint32_t)d.z);
    const int h = (int)((uint32_t)d.w >> 24);
    attn_dec_wave_unit<HD, G, KVT, true>(nullptr, Kp, Vp, un, h, Hq, head_stride, nch_max, po, pml, fr, Hkv);
    uint32_t hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(hw));
    const uint32_t mytag = ((uint32_t)xq.stepc[0] * 4096u + (uint32_t)xq.layer) * 16u + (hw & 15u);
    const int pair = un.t * Hkv + h;
    if (threadIdx.x == 0) xq.tag[(size_t)pair * xq.nch + un.c] = (int32_t)mytag;
    SH_WAIT_VMCNT(0);                                  // this thread's partial (and tag) stores are in L2
    __syncthreads();
    const int nch = min((un.p + ATT_CHUNK) / ATT_CHUNK, nch_max);
    if (threadIdx.x == 0) {
        s_last = atomicAdd(&xq.arrive[pair], 1) == nch - 1;
        if (s_last) atomicExch(&xq.arrive[pair], 0);   // every chunk has counted: ready for the next layer
    }
    __syncthreads();
    if (!s_last) return;
    if (xq.misplaced) {
        // every chunk of the pair written in this launch on this XCD?
        const __amdgpu_buffer_rsrc_t tr = __builtin_amdgcn_make_buffer_rsrc(
            xq.tag, 0, (int)((size_t)xq.max_tok * Hkv * xq.nch * 4), 0x00020000);
        const uint32_t want = mytag ^ ((uint32_t)xq.rot << 28);
        for (int c = threadIdx.x; c < nch; c += ATT_THREADS) {
            const uint32_t got = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                tr, (int)(((size_t)pair * xq.nch + c) * 4), 0, 1);
            if (got != want) *(volatile int32_t*)xq.misplaced = 1;
        }
    }
    const PartL2 pp{__builtin_amdgcn_make_buffer_rsrc(po, 0, (int)po_bytes, 0x00020000),
                    __builtin_amdgcn_make_buffer_rsrc(pml, 0, (int)pml_bytes, 0x00020000)};
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int w = wv; w < NB; w += ATT_THREADS / 64) {
        const int e = h * G * HD + w * 256 + 4 * lane;
        const int hq = e / HD, dd = e - hq * HD;
        const float4 res = merge_chunks(pp, ((size_t)un.t * Hq + hq) * nch_max, nch, HD, dd);
        *(float4*)(out + (size_t)un.t * Hq * HD + e) = res;
        if (act) act16_store_block(a, un.t, h * NB + w, lane, res);
    }
}

struct AttnArgs {
    const float* q;
    const void *Kp, *Vp;      // f32 or f16 (kv_f16) caches
    const int32_t *qt0, *qn, *tok2seq, *tok_pos;
    const int64_t* kv_base;
    int Hq;
    int64_t head_stride;
    int nch_max;
    float *po, *pml;
    hipEvent_t ev0;    // recorded at the start of the first attention kernel (optional)
    const int32_t* pairs;   // decode work-unit list (attn_pairs_kernel)
    int n_dec;
    bool kv_f16;
};

template <int HD, int G, int QB>
static void launch_blk(dim3 grid, hipStream_t s, const AttnArgs& a) {
    SH_LAUNCH(a.ev0, nullptr, (attn_block_kernel<HD, G, QB>), grid, dim3(ATT_THREADS), 0, s, a.q,
              (const float*)a.Kp, (const float*)a.Vp, a.qt0,
                       a.qn, a.tok2seq, a.tok_pos, a.kv_base, a.Hq, a.head_stride, a.nch_max, a.po, a.pml);
}

template <int HD, int G>
static void launch_g(bool prefill, dim3 grid, hipStream_t s, const AttnArgs& a) {
    if (prefill) launch_blk<HD, G, 32 / G>(grid, s, a);
    else launch_blk<HD, G, 1>(grid, s, a);
}

template <int HD>
static int launch_hd(int G, bool prefill, dim3 grid, hipStream_t s, const AttnArgs& a) {
    switch (G) {
        case 1: launch_g<HD, 1>(prefill, grid, s, a); break;
        case 2: launch_g<HD, 2>(prefill, grid, s, a); break;
        case 4: launch_g<HD, 4>(prefill, grid, s, a); break;
        case 8: launch_g<HD, 8>(prefill, grid, s, a); break;
        default: return -5;
    }
    return 0;
}

int attn_chunk_size() { return ATT_CHUNK; }
int attn_prefill_block(int G) { return G > 0 && G <= 32 ? 32 / G : 1; }

// Partials po [T][Hq][nch][HD], pml [T][Hq][nch][2], then the decode
// work-unit list (1 + T * nch int32).
size_t attention_partial_floats(int T, int Hq, int HD, int max_pos) {
    int nch = (max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    return (size_t)T * Hq * nch * (HD + 2) + 4 * (size_t)T * nch + 12;   // + list header, units, alignment
}

// SLATE_HIP_ATTN_WAVE=0 selects the workgroup-phased decode kernel for every shape.
static bool wave_kernel() { return knobs().attn_wave != 0; }

// The wave kernel where its query slices and accumulators fit the registers
// and the launch is a decode batch (a few query tokens, K/V streamed from
// HBM); prompt tokens, whose K/V re-reads hit L2, run the phased kernel at
// its higher occupancy.
constexpr int ATT_WAVE_MAX_TOKENS = 64;

template <int HD, int G, typename KVT>
static void launch_dec_t(dim3 grid, hipStream_t s, const AttnArgs& a) {
    const KVT* Kp = (const KVT*)a.Kp;
    const KVT* Vp = (const KVT*)a.Vp;
    if constexpr (G * HD <= 512) {
        if (wave_kernel() && a.n_dec <= ATT_WAVE_MAX_TOKENS) {
            SH_LAUNCH(a.ev0, nullptr, (attn_dec_wave_kernel<HD, G, KVT>), grid, dim3(ATT_THREADS), 0, s, a.q, Kp, Vp,
                      a.qt0, a.tok2seq, a.tok_pos, a.kv_base, a.Hq, a.head_stride, a.nch_max, a.po, a.pml,
                      a.pairs);
            return;
        }
    }
    SH_LAUNCH(a.ev0, nullptr, (attn_dec_kernel<HD, G, KVT>), grid, dim3(ATT_THREADS), 0, s, a.q, Kp, Vp, a.qt0,
              a.tok2seq, a.tok_pos, a.kv_base, a.Hq, a.head_stride, a.nch_max, a.po, a.pml, a.pairs);
}

template <int HD, int G>
static void launch_dec_g(dim3 grid, hipStream_t s, const AttnArgs& a) {
    if (a.kv_f16) launch_dec_t<HD, G, _Float16>(grid, s, a);
    else launch_dec_t<HD, G, float>(grid, s, a);
}

template <int HD>
static int launch_dec_hd(int G, dim3 grid, hipStream_t s, const AttnArgs& a) {
    switch (G) {
        case 1: launch_dec_g<HD, 1>(grid, s, a); return 0;
        case 2: launch_dec_g<HD, 2>(grid, s, a); return 0;
        case 4: launch_dec_g<HD, 4>(grid, s, a); return 0;
        case 8: launch_dec_g<HD, 8>(grid, s, a); return 0;
        default: return -5;
    }
}

int launch_attention_blocks(float* out, const float* q, const void* Kp, const void* Vp, const int32_t* tok2seq,
                            const int32_t* tok_pos, const int64_t* kv_base, int T, const int32_t* dec_t0,
                            int n_dec, const int32_t* pre_t0, const int32_t* pre_n, int n_pre, int Hq, int Hkv,
                            int HD, int64_t head_stride, int max_pos, float* po, float* pml, const Act16* act,
                            hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop, bool pairs_ready,
                            bool kv_f16, bool prompt_mfma) {
    if (T <= 0) return 0;
    if (kv_f16 && (n_pre > 0 || !(HD == 32 || HD == 64 || HD == 128))) {
        set_error(-5, "attention: f16 K/V caches need head_dim 32, 64 or 128 and one work unit per token");
        return -5;
    }
    if (Hkv <= 0 || Hq % Hkv != 0) {
        set_error(-1, "attention: n_q_heads %d not a multiple of n_kv_heads %d", Hq, Hkv);
        return -1;
    }
    if (act && ((Hq * HD) % 256 || act->K != Hq * HD)) {
        set_error(-1, "attention: operand output needs a row width that is a multiple of 256");
        return -1;
    }
    const int G = Hq / Hkv;
    const int nch_max = (max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    if (n_dec >= 32768 || nch_max > 65536) {
        set_error(-5, "attention: %d query tokens / %d key chunks exceed the work-unit encoding", n_dec, nch_max);
        return -5;
    }
    int32_t* pairs = attn_unit_list(pml, T, Hq, nch_max);
    AttnArgs a{q, Kp, Vp, nullptr, nullptr, tok2seq, tok_pos, kv_base, Hq, head_stride, nch_max, po, pml, ev_start,
               pairs, n_dec, kv_f16};
    for (int pass = 0; pass < 2; ++pass) {
        const bool prefill = pass == 1;
        const int nblk = prefill ? n_pre : n_dec;
        if (nblk <= 0) continue;
        a.qt0 = prefill ? pre_t0 : dec_t0;
        a.qn = prefill ? pre_n : nullptr;
        dim3 grid(nch_max, nblk, Hkv);
        int rc;
        if (prefill && prompt_mfma) {
            rc = launch_attention_prompt(q, (const float*)Kp, (const float*)Vp, tok2seq, tok_pos, kv_base, pre_t0,
                                         pre_n, n_pre, Hq, Hkv, HD, head_stride, nch_max, po, pml, s, a.ev0);
            if (rc) return rc;
        } else if (!prefill && (HD == 32 || HD == 64 || HD == 128)) {
            if (!pairs_ready) {
                SH_LAUNCH(a.ev0, nullptr, attn_pairs_kernel, dim3(1), dim3(1024), 0, s, dec_t0, n_dec, tok_pos,
                          tok2seq, kv_base, nch_max, pairs, AttnXcd{}, 0);
                SH_CHECK_LAUNCH();
                a.ev0 = nullptr;
            }
            grid = dim3(nch_max * n_dec, 1, Hkv);
            rc = HD == 128 ? launch_dec_hd<128>(G, grid, s, a)
                           : (HD == 64 ? launch_dec_hd<64>(G, grid, s, a) : launch_dec_hd<32>(G, grid, s, a));
        } else {
            switch (HD) {
                case 16: rc = launch_hd<16>(G, prefill, grid, s, a); break;
                case 32: rc = launch_hd<32>(G, prefill, grid, s, a); break;
                case 64: rc = launch_hd<64>(G, prefill, grid, s, a); break;
                case 128: rc = launch_hd<128>(G, prefill, grid, s, a); break;
                default: rc = -5;
            }
        }
        if (rc) {
            set_error(rc, "attention: unsupported head_dim %d / group %d", HD, G);
            return rc;
        }
        SH_CHECK_LAUNCH();
        a.ev0 = nullptr;                           // only the first kernel records the start
    }
    launch_merge(out, po, pml, tok_pos, T, Hq, HD, nch_max, act, s, ev_stop);
    SH_CHECK_LAUNCH();
    return 0;
}

// SLATE_HIP_ATTN_ROPE: 0 keeps rope_kv_kernel separate in decode steps;
// 1 (default) fuses it into the wave kernel where that kernel runs the
// shape (G * HD <= 512, <= 64 tokens) and into the phased kernel elsewhere;
// 2 always into the phased kernel.  The two fused kernels measured equal
// on the 8B bench (3781 tok/s each).
static int rope_fused() { return knobs().attn_rope; }

template <int HD, int G, typename KVT>
static void launch_rope_t(bool wave, dim3 grid, hipStream_t s, hipEvent_t ev0, const void* Kp, const void* Vp,
                          int Hq, int Hkv, int64_t head_stride, int nch_max, float* po, float* pml,
                          const int32_t* pairs, const AttnRope& fr) {
    if constexpr (G * HD <= 512) {
        if (wave) {
            SH_LAUNCH(ev0, nullptr, (attn_dec_rope_kernel<HD, G, KVT>), grid, dim3(ATT_THREADS), 0, s, (const KVT*)Kp,
                      (const KVT*)Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
            return;
        }
    }
    SH_LAUNCH(ev0, nullptr, (attn_dec_phased_rope_kernel<HD, G, KVT>), grid, dim3(ATT_THREADS), 0, s,
              (const KVT*)Kp, (const KVT*)Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
}

template <int HD, int G>
static int launch_rope_g(bool f16, dim3 grid, hipStream_t s, hipEvent_t ev0, const void* Kp, const void* Vp, int Hq,
                         int Hkv, int64_t head_stride, int nch_max, float* po, float* pml, const int32_t* pairs,
                         const AttnRope& fr) {
    const bool wave = rope_fused() == 1 && wave_kernel() && G * HD <= 512 && (int)grid.x / nch_max <= ATT_WAVE_MAX_TOKENS;
    if (f16) launch_rope_t<HD, G, _Float16>(wave, grid, s, ev0, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
    else launch_rope_t<HD, G, float>(wave, grid, s, ev0, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
    return 0;
}

template <int HD>
static int launch_rope_hd(int G, bool f16, dim3 grid, hipStream_t s, hipEvent_t ev0, const void* Kp, const void* Vp,
                          int Hq, int Hkv, int64_t head_stride, int nch_max, float* po, float* pml,
                          const int32_t* pairs, const AttnRope& fr) {
    switch (G) {
        case 1: return launch_rope_g<HD, 1>(f16, grid, s, ev0, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
        case 2: return launch_rope_g<HD, 2>(f16, grid, s, ev0, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
        case 4: return launch_rope_g<HD, 4>(f16, grid, s, ev0, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
        case 8: return launch_rope_g<HD, 8>(f16, grid, s, ev0, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, pairs, fr);
        default: return 1;
    }
}

// Compute units of the current device (256 if the query fails).
static int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus;
}

bool attention_xcd_merge(int T, int Hq, int Hkv, int HD, int max_pos, bool has_act) {
    (void)has_act;
    // consecutive workgroups on consecutive XCDs, as probed (attention_xcd_probe) for this device
    if (!knobs().attn_xcd || rope_fused() != 1 || !wave_kernel() || T <= 0 || T > ATT_WAVE_MAX_TOKENS ||
        Hkv <= 0 || Hq % Hkv != 0)
        return false;
    const std::atomic<int>* f = xcd_flag();
    if (!f || f->load() != 1)
        return false;
    const int G = Hq / Hkv;
    if (!(HD == 32 || HD == 64 || HD == 128) || G * HD > 512 || (G * HD) % 256 != 0) return false;
    const double nch = (double)((max_pos + ATT_CHUNK - 1) / ATT_CHUNK);
    return (double)T * Hq * nch * HD * 4.0 < 2147483648.0;   // buffer offsets of the partials
}

template <int HD, int G, typename KVT>
static void launch_xcd_t(hipStream_t s, hipEvent_t ev0, hipEvent_t ev1, const void* Kp, const void* Vp, int Hq,
                         int Hkv, int64_t head_stride, int nch_max, float* po, float* pml, uint32_t po_bytes,
                         uint32_t pml_bytes, const AttnRope& fr, const AttnXcd& xq, float* out, const Act16* act) {
    if constexpr (G * HD <= 512 && (G * HD) % 256 == 0) {
        // a queue holds at most ceil(T * Hkv / 8) pairs of at most nch_max units
        const int grid = 8 * ((xq.max_tok_step * Hkv + 7) / 8) * nch_max;
        SH_LAUNCH(ev0, ev1, (attn_dec_rope_xcd_kernel<HD, G, KVT>), dim3(grid), dim3(ATT_THREADS), 0, s,
                  (const KVT*)Kp, (const KVT*)Vp, Hq, Hkv, head_stride, nch_max, po, pml, po_bytes, pml_bytes, fr,
                  xq, out, act ? *act : Act16{}, act ? 1 : 0);
    }
}

template <int HD, int G>
static void launch_xcd_g(bool f16, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1, const void* Kp, const void* Vp,
                         int Hq, int Hkv, int64_t head_stride, int nch_max, float* po, float* pml, uint32_t po_bytes,
                         uint32_t pml_bytes, const AttnRope& fr, const AttnXcd& xq, float* out, const Act16* act) {
    if (f16)
        launch_xcd_t<HD, G, _Float16>(s, ev0, ev1, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, po_bytes,
                                      pml_bytes, fr, xq, out, act);
    else
        launch_xcd_t<HD, G, float>(s, ev0, ev1, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml, po_bytes, pml_bytes,
                                   fr, xq, out, act);
}

int launch_attention_rope(float* out, void* Kp, void* Vp, const float* part, int nsplit, int64_t split_stride,
                          int qkv_ld, const float* cs, const RowNorm& rn, const int32_t* tok_pos, int T, int Hq,
                          int Hkv, int HD, int64_t head_stride, int max_pos, float* po, float* pml, const Act16* act,
                          hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop, bool kv_f16, const AttnXcd* xq) {
    if (T <= 0) return 0;
    if (xq && T <= xq->max_tok && (!act || ((Hq * HD) % 256 == 0 && act->K == Hq * HD)) &&
        attention_xcd_merge(T, Hq, Hkv, HD, max_pos, act != nullptr)) {
        const int G = Hq / Hkv;
        const int nch_max = (max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
        const AttnRope fr{part, nsplit, split_stride, qkv_ld, cs, rn, Kp, Vp};
        const uint32_t po_bytes = (uint32_t)((size_t)T * Hq * nch_max * HD * 4);
        const uint32_t pml_bytes = (uint32_t)((size_t)T * Hq * nch_max * 2 * 4);
        AttnXcd x = *xq;
        x.max_tok_step = T;
        if (HD == 128 && G == 2)
            launch_xcd_g<128, 2>(kv_f16, s, ev_start, ev_stop, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml,
                                 po_bytes, pml_bytes, fr, x, out, act);
        else if (HD == 128 && G == 4)
            launch_xcd_g<128, 4>(kv_f16, s, ev_start, ev_stop, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml,
                                 po_bytes, pml_bytes, fr, x, out, act);
        else if (HD == 64 && G == 4)
            launch_xcd_g<64, 4>(kv_f16, s, ev_start, ev_stop, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml,
                                po_bytes, pml_bytes, fr, x, out, act);
        else if (HD == 64 && G == 8)
            launch_xcd_g<64, 8>(kv_f16, s, ev_start, ev_stop, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml,
                                po_bytes, pml_bytes, fr, x, out, act);
        else if (HD == 32 && G == 8)
            launch_xcd_g<32, 8>(kv_f16, s, ev_start, ev_stop, Kp, Vp, Hq, Hkv, head_stride, nch_max, po, pml,
                                po_bytes, pml_bytes, fr, x, out, act);
        else
            return 1;
        SH_CHECK_LAUNCH();
        return 0;
    }
    if (rope_fused() == 0 || Hkv <= 0 || Hq % Hkv != 0 ||
        !(HD == 32 || HD == 64 || HD == 128))
        return 1;
    if (act && ((Hq * HD) % 256 || act->K != Hq * HD)) return 1;
    const int G = Hq / Hkv;
    const int nch_max = (max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    if (T >= 32768 || nch_max > 65536) return 1;
    const int32_t* pairs = attn_unit_list(pml, T, Hq, nch_max);
    const AttnRope fr{part, nsplit, split_stride, qkv_ld, cs, rn, Kp, Vp};
    const dim3 grid(nch_max * T, 1, Hkv);
    const int rc = HD == 128 ? launch_rope_hd<128>(G, kv_f16, grid, s, ev_start, Kp, Vp, Hq, Hkv, head_stride, nch_max,
                                                   po, pml, pairs, fr)
                   : HD == 64 ? launch_rope_hd<64>(G, kv_f16, grid, s, ev_start, Kp, Vp, Hq, Hkv, head_stride,
                                                   nch_max, po, pml, pairs, fr)
                              : launch_rope_hd<32>(G, kv_f16, grid, s, ev_start, Kp, Vp, Hq, Hkv, head_stride,
                                                   nch_max, po, pml, pairs, fr);
    if (rc) return rc;
    SH_CHECK_LAUNCH();
    launch_merge(out, po, pml, tok_pos, T, Hq, HD, nch_max, act, s, ev_stop);
    SH_CHECK_LAUNCH();
    return 0;
}

// Every token its own block (per-token semantics, no grouping).
int launch_attention_ragged(float* out, const float* q, const float* Kp, const float* Vp,
                            const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int T,
                            int Hq, int Hkv, int HD, int64_t head_stride, int max_pos, float* po,
                            float* pml, hipStream_t s) {
    return launch_attention_blocks(out, q, Kp, Vp, tok2seq, tok_pos, kv_base, T, nullptr, T, nullptr, nullptr, 0,
                                   Hq, Hkv, HD, head_stride, max_pos, po, pml, nullptr, s, nullptr, nullptr, false,
                                   false);
}

int launch_attention_pairs(const int32_t* dec_t0, int n_dec, const int32_t* tok_pos, const int32_t* tok2seq,
                           const int64_t* kv_base, int T, int Hq, int max_pos, float* pml, hipStream_t s,
                           const AttnXcd* xq, int Hkv) {
    const int nch_max = (max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    if (n_dec <= 0) return 0;
    if (n_dec >= 32768 || nch_max > 65536) {
        set_error(-5, "attention: %d query tokens / %d key chunks exceed the work-unit encoding", n_dec, nch_max);
        return -5;
    }
    // every decode token's pairs must fit the queues and the arrival counts
    if (xq && (Hkv <= 0 || Hkv > 127 || T > xq->max_tok)) {
        set_error(-1, "attention: %d tokens x %d kv heads exceed the per-XCD queues", T, Hkv);
        return -1;
    }
    // Hkv % 8 == 0: the pair list's own scan places every queue entry
    const bool inline_q = xq && Hkv % 8 == 0;
    hipLaunchKernelGGL(attn_pairs_kernel, dim3(1), dim3(1024), 0, s, dec_t0, n_dec, tok_pos, tok2seq, kv_base,
                       nch_max, attn_unit_list(pml, T, Hq, nch_max), inline_q ? *xq : AttnXcd{}, Hkv);
    SH_CHECK_LAUNCH();
    if (xq && !inline_q) {
        hipLaunchKernelGGL(attn_xcd_queues_kernel, dim3(1), dim3(1024), 0, s, dec_t0, n_dec, tok_pos, tok2seq,
                           kv_base, nch_max, Hkv, *xq);
        SH_CHECK_LAUNCH();
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Single-head step of the vtable (backend_cpu.c:117-166), any D and L: one
// workgroup of 16 waves.  Scores: one wave per key (lanes over d, coalesced
// K rows, DPP sum); softmax with the reference's double sum, leaving the
// probabilities in the caller's scratch `scores` [L] as there; then
// out[d] = sum_t p_t V[t, d] with lanes over d and the waves' t-slices
// combined in LDS in a fixed order (deterministic).  L <= 0 writes zeros.
constexpr int ATT_STEP_THREADS = 1024;
__global__ __launch_bounds__(ATT_STEP_THREADS) void attention_step_kernel(float* __restrict__ out,
                                                                          const float* __restrict__ q,
                                                                          const float* __restrict__ K,
                                                                          const float* __restrict__ V,
                                                                          float* __restrict__ scores, int L, int D) {
    constexpr int NW = ATT_STEP_THREADS / 64;
    __shared__ float red[ATT_STEP_THREADS];
    __shared__ double redd[NW];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float scale = 1.0f / sqrtf((float)D);
    float mx = -INFINITY;
    for (int t = wv; t < L; t += NW) {
        const float* k = K + (size_t)t * D;
        float a = 0.f;
        for (int d = lane; d < D; d += 64) a = __builtin_fmaf(q[d], k[d], a);
        const float sc = wave_sum(a) * scale;
        if (lane == 0) scores[t] = sc;
        mx = fmaxf(mx, sc);
    }
    if (lane == 0) red[wv] = mx;
    __syncthreads();                               // also orders the scores stores
    mx = red[0];
    for (int i = 1; i < NW; ++i) mx = fmaxf(mx, red[i]);
    double S = 0;
    for (int t = tid; t < L; t += ATT_STEP_THREADS) {
        const float e = expf(scores[t] - mx);
        scores[t] = e;
        S += (double)e;
    }
    for (int o = 32; o > 0; o >>= 1) S += __shfl_xor(S, o, 64);
    if (lane == 0) redd[wv] = S;
    __syncthreads();
    S = 0;
    for (int i = 0; i < NW; ++i) S += redd[i];
    const float invS = (float)(1.0 / S);
    for (int t = tid; t < L; t += ATT_STEP_THREADS) scores[t] *= invS;
    __syncthreads();
    // lanes over d (DL of them, whole waves), TS = threads / DL slices of t
    for (int d0 = 0; d0 < D; d0 += ATT_STEP_THREADS) {
        const int Dc = min(D - d0, ATT_STEP_THREADS);
        const int DL = (Dc + 63) & ~63, TS = ATT_STEP_THREADS / DL;
        const int dl = tid % DL, ts = tid / DL, d = d0 + dl;
        float acc = 0.f;
        if (ts < TS && dl < Dc)
            for (int t = ts; t < L; t += TS) acc = __builtin_fmaf(scores[t], V[(size_t)t * D + d], acc);
        red[tid] = acc;
        __syncthreads();
        if (tid < Dc) {
            float v = 0.f;
            for (int i = 0; i < TS; ++i) v += red[i * DL + tid];
            out[d0 + tid] = L > 0 ? v : 0.f;
        }
        __syncthreads();
    }
}

int launch_attention_step(float* out, const float* q, const float* K, const float* V, float* scores, int L,
                          int D, hipStream_t s) {
    hipLaunchKernelGGL(attention_step_kernel, dim3(1), dim3(ATT_STEP_THREADS), 0, s, out, q, K, V, scores, L, D);
    SH_CHECK_LAUNCH();
    return 0;
}

}  // namespace slate_hip
