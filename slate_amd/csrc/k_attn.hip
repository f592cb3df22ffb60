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
#include "launch.h"

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
                float mx = fmaxf(fmaxf(v0, v1), fmaxf(v2, v3));
                for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
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
                float s = (e0 + e1) + (e2 + e3);
                for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
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

// out[t, hq, :] = sum_c e^{m_c - M} o_c / sum_c e^{m_c - M} l_c
__global__ void attn_merge_kernel(float* __restrict__ out, const float* __restrict__ po,
                                  const float* __restrict__ pml, const int32_t* __restrict__ tok_pos,
                                  int Hq, int HD, int nch_max) {
    const int t = blockIdx.x, hq = blockIdx.y;
    const int L = tok_pos[t] + 1;
    const int nch = min((L + ATT_CHUNK - 1) / ATT_CHUNK, nch_max);
    const size_t p0 = ((size_t)t * Hq + hq) * nch_max;
    float M = -INFINITY;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, pml[(p0 + c) * 2]);
    float den = 0.f;
    for (int c = 0; c < nch; ++c) den += expf(pml[(p0 + c) * 2] - M) * pml[(p0 + c) * 2 + 1];
    float inv = 1.0f / den;
    for (int d = threadIdx.x; d < HD; d += blockDim.x) {
        float acc = 0.f;
        for (int c = 0; c < nch; ++c) acc += expf(pml[(p0 + c) * 2] - M) * po[(p0 + c) * HD + d];
        out[((size_t)t * Hq + hq) * HD + d] = acc * inv;
    }
}

struct AttnArgs {
    const float *q, *Kp, *Vp;
    const int32_t *qt0, *qn, *tok2seq, *tok_pos;
    const int64_t* kv_base;
    int Hq;
    int64_t head_stride;
    int nch_max;
    float *po, *pml;
};

template <int HD, int G, int QB>
static void launch_blk(dim3 grid, hipStream_t s, const AttnArgs& a) {
    hipLaunchKernelGGL((attn_block_kernel<HD, G, QB>), grid, dim3(ATT_THREADS), 0, s, a.q, a.Kp, a.Vp, a.qt0,
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

size_t attention_partial_floats(int T, int Hq, int HD, int max_pos) {
    int nch = (max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    return (size_t)T * Hq * nch * (HD + 2);
}

int launch_attention_blocks(float* out, const float* q, const float* Kp, const float* Vp, const int32_t* tok2seq,
                            const int32_t* tok_pos, const int64_t* kv_base, int T, const int32_t* dec_t0,
                            int n_dec, const int32_t* pre_t0, const int32_t* pre_n, int n_pre, int Hq, int Hkv,
                            int HD, int64_t head_stride, int max_pos, float* po, float* pml, hipStream_t s) {
    if (T <= 0) return 0;
    if (Hkv <= 0 || Hq % Hkv != 0) {
        set_error(-1, "attention: n_q_heads %d not a multiple of n_kv_heads %d", Hq, Hkv);
        return -1;
    }
    const int G = Hq / Hkv;
    const int nch_max = (max_pos + ATT_CHUNK - 1) / ATT_CHUNK;
    AttnArgs a{q, Kp, Vp, nullptr, nullptr, tok2seq, tok_pos, kv_base, Hq, head_stride, nch_max, po, pml};
    for (int pass = 0; pass < 2; ++pass) {
        const bool prefill = pass == 1;
        const int nblk = prefill ? n_pre : n_dec;
        if (nblk <= 0) continue;
        a.qt0 = prefill ? pre_t0 : dec_t0;
        a.qn = prefill ? pre_n : nullptr;
        dim3 grid(nch_max, nblk, Hkv);
        int rc;
        switch (HD) {
            case 16: rc = launch_hd<16>(G, prefill, grid, s, a); break;
            case 32: rc = launch_hd<32>(G, prefill, grid, s, a); break;
            case 64: rc = launch_hd<64>(G, prefill, grid, s, a); break;
            case 128: rc = launch_hd<128>(G, prefill, grid, s, a); break;
            default: rc = -5;
        }
        if (rc) {
            set_error(rc, "attention: unsupported head_dim %d / group %d", HD, G);
            return rc;
        }
        SH_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(attn_merge_kernel, dim3(T, Hq), dim3(HD < 256 ? HD : 256), 0, s, out, po, pml, tok_pos,
                       Hq, HD, nch_max);
    SH_CHECK_LAUNCH();
    return 0;
}

// Every token its own block (per-token semantics, no grouping).
int launch_attention_ragged(float* out, const float* q, const float* Kp, const float* Vp,
                            const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int T,
                            int Hq, int Hkv, int HD, int64_t head_stride, int max_pos, float* po,
                            float* pml, hipStream_t s) {
    return launch_attention_blocks(out, q, Kp, Vp, tok2seq, tok_pos, kv_base, T, nullptr, T, nullptr, nullptr, 0,
                                   Hq, Hkv, HD, head_stride, max_pos, po, pml, s);
}

// ---------------------------------------------------------------------------
// Single-head step of the vtable (backend_cpu.c:117-166), any D and L: one
// workgroup; scores land in the caller's scratch `scores` [L] as there.
__global__ __launch_bounds__(256) void attention_step_kernel(float* __restrict__ out,
                                                             const float* __restrict__ q,
                                                             const float* __restrict__ K,
                                                             const float* __restrict__ V,
                                                             float* __restrict__ scores, int L, int D) {
    __shared__ float red[256];
    __shared__ double redd[256];
    const int tid = threadIdx.x;
    const float scale = 1.0f / sqrtf((float)D);
    float mx = -INFINITY;
    for (int t = tid; t < L; t += 256) {
        const float* k = K + (size_t)t * D;
        float a = 0.f;
        for (int d = 0; d < D; ++d) a = __builtin_fmaf(q[d], k[d], a);
        float sc = a * scale;
        scores[t] = sc;
        mx = fmaxf(mx, sc);
    }
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    mx = red[0];
    double S = 0;
    for (int t = tid; t < L; t += 256) {
        float e = expf(scores[t] - mx);
        scores[t] = e;
        S += (double)e;
    }
    redd[tid] = S;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) redd[tid] += redd[tid + o];
        __syncthreads();
    }
    float invS = (float)(1.0 / redd[0]);
    for (int t = tid; t < L; t += 256) scores[t] *= invS;
    __syncthreads();
    for (int d = tid; d < D; d += 256) {
        float acc = 0.f;
        for (int t = 0; t < L; ++t) acc = __builtin_fmaf(scores[t], V[(size_t)t * D + d], acc);
        out[d] = acc;
    }
}

int launch_attention_step(float* out, const float* q, const float* K, const float* V, float* scores, int L,
                          int D, hipStream_t s) {
    hipLaunchKernelGGL(attention_step_kernel, dim3(1), dim3(256), 0, s, out, q, K, V, scores, L, D);
    SH_CHECK_LAUNCH();
    return 0;
}

}  // namespace slate_hip
