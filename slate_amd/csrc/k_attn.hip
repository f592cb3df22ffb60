// k_attn.hip -- ragged GQA attention over per-sequence KV caches.
//
// Semantics (llama_infer.c:97-129, applied per packed token): q head hq of
// token t reads kv head hq / (Hq/Hkv) of the token's own sequence over key
// positions 0..tok_pos[t]; score = (q . k) * (1/sqrtf(hd)); softmax; sum p*V.
//
// Work is split into (key chunk, token, kv head) workgroups: each streams its
// chunk of K and V exactly once for all G = Hq/Hkv query heads of the group,
// producing a partial (max, sum, unnormalised output) per query head; a merge
// kernel combines the chunks with the usual log-sum-exp rescaling.
#include "launch.h"

namespace slate_hip {

constexpr int ATT_THREADS = 256;

// Partial layout: po[((t * Hq + hq) * nch_max + c) * HD + d], pml[(.. c) * 2 + {m, l}]
template <int HD, int G>
__global__ __launch_bounds__(ATT_THREADS) void attn_chunk_kernel(
    const float* __restrict__ q, const float* __restrict__ Kp, const float* __restrict__ Vp,
    const int32_t* __restrict__ tok2seq, const int32_t* __restrict__ tok_pos,
    const int64_t* __restrict__ kv_base, int Hq, int64_t head_stride, int chunk, int nch_max,
    float* __restrict__ po, float* __restrict__ pml) {
    constexpr int KPT = ATT_THREADS / HD;           // key lanes in the PV phase
    __shared__ float sq[G * HD];
    __shared__ float sp[G * ATT_THREADS];
    __shared__ float sred[G * 4];
    __shared__ float so[(KPT > 1 ? KPT - 1 : 1) * G * HD];

    const int c = blockIdx.x, t = blockIdx.y, h = blockIdx.z;
    const int L = tok_pos[t] + 1;
    const int k0 = c * chunk;
    if (k0 >= L) return;                             // merge ignores chunks past the end
    const int k1 = min(L, k0 + chunk);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t base = kv_base[tok2seq[t]] + (int64_t)h * head_stride;
    const float* Kh = Kp + base;
    const float* Vh = Vp + base;
    const float* qt = q + (size_t)t * Hq * HD + (size_t)h * G * HD;
    for (int i = tid; i < G * HD; i += ATT_THREADS) sq[i] = qt[i];
    __syncthreads();

    float m_run[G], l_run[G], o_acc[G];
#pragma unroll
    for (int i = 0; i < G; ++i) { m_run[i] = -INFINITY; l_run[i] = 0.f; o_acc[i] = 0.f; }
    const int dd = tid % HD, kq = tid / HD;

    for (int kt = k0; kt < k1; kt += ATT_THREADS) {
        const int nk = min(ATT_THREADS, k1 - kt);
        // scores: one key per thread, all G heads
        float s[G];
#pragma unroll
        for (int i = 0; i < G; ++i) s[i] = -INFINITY;
        if (tid < nk) {
            const float4* kr = (const float4*)(Kh + (int64_t)(kt + tid) * HD);
            float a[G];
#pragma unroll
            for (int i = 0; i < G; ++i) a[i] = 0.f;
#pragma unroll 8
            for (int d4 = 0; d4 < HD / 4; ++d4) {
                float4 kv = kr[d4];
#pragma unroll
                for (int i = 0; i < G; ++i) {
                    const float4 qv = *(const float4*)(sq + i * HD + 4 * d4);
                    a[i] = __builtin_fmaf(qv.x, kv.x, a[i]);
                    a[i] = __builtin_fmaf(qv.y, kv.y, a[i]);
                    a[i] = __builtin_fmaf(qv.z, kv.z, a[i]);
                    a[i] = __builtin_fmaf(qv.w, kv.w, a[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < G; ++i) s[i] = a[i] * scale;
        }
        // tile max per head
        float mt[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            float v = s[i];
            for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
            mt[i] = v;
        }
        if (lane == 0)
#pragma unroll
            for (int i = 0; i < G; ++i) sred[i * 4 + wv] = mt[i];
        __syncthreads();
        float mnew[G], alpha[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            float v = fmaxf(fmaxf(sred[i * 4 + 0], sred[i * 4 + 1]), fmaxf(sred[i * 4 + 2], sred[i * 4 + 3]));
            mnew[i] = fmaxf(m_run[i], v);
            alpha[i] = m_run[i] == -INFINITY ? 0.f : expf(m_run[i] - mnew[i]);
        }
        __syncthreads();
        float ps[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            float p = tid < nk ? expf(s[i] - mnew[i]) : 0.f;
            sp[i * ATT_THREADS + tid] = p;
            float v = p;
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
            ps[i] = v;
        }
        if (lane == 0)
#pragma unroll
            for (int i = 0; i < G; ++i) sred[i * 4 + wv] = ps[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < G; ++i) {
            float lt = (sred[i * 4 + 0] + sred[i * 4 + 1]) + (sred[i * 4 + 2] + sred[i * 4 + 3]);
            l_run[i] = l_run[i] * alpha[i] + lt;
            m_run[i] = mnew[i];
            o_acc[i] *= alpha[i];
        }
        // PV: thread (dd, kq) sums keys kq, kq+KPT, ...
        for (int k = kq; k < nk; k += KPT) {
            float v = Vh[(int64_t)(kt + k) * HD + dd];
#pragma unroll
            for (int i = 0; i < G; ++i) o_acc[i] = __builtin_fmaf(sp[i * ATT_THREADS + k], v, o_acc[i]);
        }
        __syncthreads();
    }
    // reduce o over the KPT key lanes
    if (KPT > 1) {
        if (kq > 0)
#pragma unroll
            for (int i = 0; i < G; ++i) so[((kq - 1) * G + i) * HD + dd] = o_acc[i];
        __syncthreads();
        if (kq == 0)
            for (int j = 1; j < KPT; ++j)
#pragma unroll
                for (int i = 0; i < G; ++i) o_acc[i] += so[((j - 1) * G + i) * HD + dd];
    }
    if (kq == 0) {
#pragma unroll
        for (int i = 0; i < G; ++i) {
            int hq = h * G + i;
            size_t pidx = ((size_t)t * Hq + hq) * nch_max + c;
            po[pidx * HD + dd] = o_acc[i];
            if (dd == 0) {
                pml[pidx * 2 + 0] = m_run[i];
                pml[pidx * 2 + 1] = l_run[i];
            }
        }
    }
}

// out[t, hq, :] = sum_c e^{m_c - M} o_c / sum_c e^{m_c - M} l_c
__global__ void attn_merge_kernel(float* __restrict__ out, const float* __restrict__ po,
                                  const float* __restrict__ pml, const int32_t* __restrict__ tok_pos,
                                  int Hq, int HD, int chunk, int nch_max) {
    const int t = blockIdx.x, hq = blockIdx.y;
    const int L = tok_pos[t] + 1;
    const int nch = min((L + chunk - 1) / chunk, nch_max);
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

template <int HD, int G>
static void launch_chunk(dim3 grid, hipStream_t s, const float* q, const float* Kp, const float* Vp,
                         const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int Hq,
                         int64_t head_stride, int chunk, int nch_max, float* po, float* pml) {
    hipLaunchKernelGGL((attn_chunk_kernel<HD, G>), grid, dim3(ATT_THREADS), 0, s, q, Kp, Vp, tok2seq,
                       tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml);
}

template <int HD>
static int dispatch_g(int G, dim3 grid, hipStream_t s, const float* q, const float* Kp, const float* Vp,
                      const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int Hq,
                      int64_t head_stride, int chunk, int nch_max, float* po, float* pml) {
    switch (G) {
        case 1: launch_chunk<HD, 1>(grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        case 2: launch_chunk<HD, 2>(grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        case 4: launch_chunk<HD, 4>(grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        case 8: launch_chunk<HD, 8>(grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        default: return -5;
    }
    return 0;
}

int attn_chunk_size() { return 256; }

int launch_attention_ragged(float* out, const float* q, const float* Kp, const float* Vp,
                            const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int T,
                            int Hq, int Hkv, int HD, int64_t head_stride, int max_pos, float* po,
                            float* pml, hipStream_t s) {
    if (T <= 0) return 0;
    if (Hkv <= 0 || Hq % Hkv != 0) {
        set_error(-1, "attention: n_q_heads %d not a multiple of n_kv_heads %d", Hq, Hkv);
        return -1;
    }
    const int G = Hq / Hkv;
    const int chunk = attn_chunk_size();
    const int nch_max = (max_pos + chunk - 1) / chunk;
    dim3 grid(nch_max, T, Hkv);
    int rc;
    switch (HD) {
        case 16: rc = dispatch_g<16>(G, grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        case 32: rc = dispatch_g<32>(G, grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        case 64: rc = dispatch_g<64>(G, grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        case 128: rc = dispatch_g<128>(G, grid, s, q, Kp, Vp, tok2seq, tok_pos, kv_base, Hq, head_stride, chunk, nch_max, po, pml); break;
        default: rc = -5;
    }
    if (rc != 0) {
        set_error(rc, "attention: unsupported head_dim %d / group %d", HD, G);
        return rc;
    }
    SH_CHECK_LAUNCH();
    hipLaunchKernelGGL(attn_merge_kernel, dim3(T, Hq), dim3(HD < 256 ? HD : 256), 0, s, out, po, pml,
                       tok_pos, Hq, HD, chunk, nch_max);
    SH_CHECK_LAUNCH();
    return 0;
}

size_t attention_partial_floats(int T, int Hq, int HD, int max_pos) {
    int nch = (max_pos + attn_chunk_size() - 1) / attn_chunk_size();
    return (size_t)T * Hq * nch * (HD + 2);
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
