// k_attn_mfma.hip -- causal GQA attention of prompt tokens on MFMA.
//
// The per-head attention of llama_infer.c:97-129 (scores q.k * 1/sqrt(hd)
// over keys 0..p, softmax, weighted sum of V) for runs of consecutive
// prompt tokens of one sequence, whose keys are shared.  Work unit = (key
// chunk of 256 positions, query block, kv head), as for the other attention
// kernels, leaving per-(token, q head, chunk) partials (running max m, sum
// l, unnormalised output) that the merge kernel combines.  A unit's W waves
// each own one q head of the group and 16 consecutive tokens of the block
// (W = max(G, 4): with fewer than 4 heads per group the block spans 4/G
// tiles of 16 tokens).  Keys are processed in blocks of 32: each block's K
// and V rows are read once per unit, kept in LDS as f16 halves hi + lo
// (hi = f16(x), lo = f16(x - hi), ~22 bits of x together), V transposed,
// while the next block's rows are already loading into registers.
// Products use three f16 MFMAs, hi*hi + hi*lo + lo*hi (the lo*lo term is
// below f32 rounding), accumulated in f32, in transposed form so that each
// lane owns one token (column) throughout:
//   S^T [32 keys x 16 tokens] = K Q^T     (two 16-key tiles; Q in registers)
//   O^T [hd x 16 tokens]     += V^T P^T   (P^T = exp(S^T - m) straight from
//                                          the S^T registers: the MFMA's
//                                          reduction slots are mapped to the
//                                          keys a lane holds, and V^T is laid
//                                          out in LDS in that slot order)
// with an online softmax in f32 between them, in base 2 (exp(x) computed as
// 2^(x log2 e), one hardware exp per score; the chunk maximum goes out in
// natural-log units for the merge).  Values must lie in the f16 range
// (|x| < 65504), as the K/V caches and queries of a LLaMA model do.
#include "launch.h"
#include "lanes.h"
#include "mfma.h"

namespace slate_hip {

constexpr int APF_TILE = 16;    // query tokens per wave (MFMA columns)
constexpr int APF_KB = 32;      // keys per block (MFMA K of P.V)
constexpr int APF_MIN_WAVES = 4;

__device__ __forceinline__ _Float16 hi_h(float x) { return (_Float16)x; }
__device__ __forceinline__ _Float16 lo_h(float x) { return (_Float16)(x - (float)(_Float16)x); }

// Combine v over the four lanes j, j+16, j+32, j+48 (the four 16-lane rows).
// (v_permlane16/32_swap would do it in VALU, but this compiler folds the
// two results of a swap whose operands are the same value into one.)
__device__ __forceinline__ float cols_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float cols_sum(float v) {
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

// MFMA reduction slot of key k (0..31) of a block: lane group g = (k % 16) / 4
// holds keys 4g + i of S^T tile k / 16 (i = k % 4) and feeds them to slots
// 8g + 4 (k / 16) + i.
__device__ __forceinline__ int key_slot(int k) { return 8 * ((k & 15) >> 2) + 4 * (k >> 4) + (k & 3); }

// Chunk size of the partials: must equal the merge kernel's.
int attn_chunk_size();

template <int HD, int G>
struct PromptGeom {
    static constexpr int W = G > APF_MIN_WAVES ? G : APF_MIN_WAVES;   // waves per unit
    static constexpr int NTH = 64 * W;
    static constexpr int ROWS = APF_TILE * (W / G);                    // query tokens per block
    static constexpr int KTOT = APF_KB * HD / 4;                        // K float4 jobs per key block
    static constexpr int VTOT = (APF_KB / 2) * (HD / 4);               // V (key pair, float4) jobs
    static constexpr int KJOBS = (KTOT + NTH - 1) / NTH;               // per thread
    static constexpr int VJOBS = (VTOT + NTH - 1) / NTH;
};

template <int HD, int G, int CHUNK>
__global__ __launch_bounds__((PromptGeom<HD, G>::NTH)) void attn_prompt_kernel(
    const float* __restrict__ q, const float* __restrict__ Kp, const float* __restrict__ Vp,
    const int32_t* __restrict__ blk_t0, const int32_t* __restrict__ blk_n, const int32_t* __restrict__ tok2seq,
    const int32_t* __restrict__ tok_pos, const int64_t* __restrict__ kv_base, int Hq, int64_t head_stride,
    int nch_max, float* __restrict__ po, float* __restrict__ pml) {
    using Geo = PromptGeom<HD, G>;
    constexpr int NTH = Geo::NTH;
    constexpr int KS = HD + 8;        // K row stride (halves): 16 key rows of a read hit distinct banks
    constexpr int VS = APF_KB + 8;    // V^T row stride (halves)
    constexpr int NT = HD / 32;       // MFMA K steps of K.Q^T
    constexpr int ND = HD / 16;       // 16-row tiles of O^T
    __shared__ _Float16 sKh[APF_KB * KS], sKl[APF_KB * KS];
    __shared__ _Float16 sVh[HD * VS], sVl[HD * VS];
    // kv head fastest: workgroups are dealt round-robin to the 8 XCDs, so
    // with 8 kv heads each XCD's L2 holds one head's K/V rows (re-read by
    // every query block of the head)
    const int h = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
    const int t0 = blk_t0[b], n = blk_n[b];
    const int p0 = tok_pos[t0];
    const int p_last = p0 + n - 1;
    const int k_begin = c * CHUNK;
    if (k_begin > p_last) return;                  // whole unit: no key of the block in this chunk
    const int k_end = min(k_begin + CHUNK, p_last + 1);
    const int nkb = (k_end - k_begin + APF_KB - 1) / APF_KB;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, j = lane & 15;
    const int gi = w % G, rt = w / G;              // q head in the group, token tile
    const int hq = h * G + gi;
    const int r = APF_TILE * rt + j;               // the lane's token in the block
    const int pr = p0 + r;                         // its last visible key
    const bool active = APF_TILE * rt < n;         // the wave has a token of the block
    const int64_t kvb = kv_base[tok2seq[t0]] + (int64_t)h * head_stride;
    const float* Kh = Kp + kvb;
    const float* Vh = Vp + kvb;
    const int D = Hq * HD;
    // scores in the log2 domain: exp(s * scale - m) = 2^(s * scale * log2(e) - m2), one v_exp_f32
    const float scale2 = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;   // llama_infer.c:104

    // Q^T as the B operand: lane (g, j) holds token r, elements 32t + 8g .. +7
    half8_t qh[NT], ql[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (r < n) {
            const float4* qp = (const float4*)(q + (size_t)(t0 + r) * D + hq * HD + 32 * t + 8 * g);
            const float4 a = qp[0], e = qp[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = e.x; v[5] = e.y; v[6] = e.z; v[7] = e.w;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            qh[t][e] = hi_h(v[e]);
            ql[t][e] = lo_h(v[e]);
        }
    }
    floatx4 o[ND];                                 // O^T: lane (g, j) rows 16d + 4g + i, token r
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;                  // the lane's token (same in its four lane groups)

    // Staging jobs: K job u -> key u / (HD/4), elements 4 (u % (HD/4)) ..;
    // V job u -> keys 2 (u % 16), +1, elements 4 (u / 16) ...  Rows past the
    // block's last key load as zeros (their P is 0, and 0 times a stale cache
    // value must not make a NaN).
    float4 kr[Geo::KJOBS], va[Geo::VJOBS], vc[Geo::VJOBS];
    auto load_block = [&](int k0) {
#pragma unroll
        for (int i = 0; i < Geo::KJOBS; ++i) {
            const int u = tid + i * NTH;
            const int key = u / (HD / 4), d4 = u - key * (HD / 4);
            kr[i] = (Geo::KTOT % NTH == 0 || u < Geo::KTOT) && k0 + key <= p_last
                        ? *(const float4*)(Kh + (int64_t)(k0 + key) * HD + 4 * d4)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < Geo::VJOBS; ++i) {
            const int u = tid + i * NTH;
            const int kp = u % (APF_KB / 2), d4 = u / (APF_KB / 2);
            const int ka = (Geo::VTOT % NTH == 0 || u < Geo::VTOT) ? k0 + 2 * kp : p_last + 1;
            va[i] = ka <= p_last ? *(const float4*)(Vh + (int64_t)ka * HD + 4 * d4) : make_float4(0.f, 0.f, 0.f, 0.f);
            vc[i] = ka + 1 <= p_last ? *(const float4*)(Vh + (int64_t)(ka + 1) * HD + 4 * d4)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    load_block(k_begin);
    for (int kb = 0; kb < nkb; ++kb) {
        const int k0 = k_begin + kb * APF_KB;
        __syncthreads();                               // the previous block's LDS reads are done
#pragma unroll
        for (int i = 0; i < Geo::KJOBS; ++i) {
            const int u = tid + i * NTH;
            if (Geo::KTOT % NTH != 0 && u >= Geo::KTOT) break;
            const int key = u / (HD / 4), d4 = u - key * (HD / 4);
            const float4 v = kr[i];
            *(half4_t*)&sKh[key * KS + 4 * d4] = half4_t{hi_h(v.x), hi_h(v.y), hi_h(v.z), hi_h(v.w)};
            *(half4_t*)&sKl[key * KS + 4 * d4] = half4_t{lo_h(v.x), lo_h(v.y), lo_h(v.z), lo_h(v.w)};
        }
        // V^T rows in key-slot order; keys 2kp and 2kp + 1 take adjacent slots
#pragma unroll
        for (int i = 0; i < Geo::VJOBS; ++i) {
            const int u = tid + i * NTH;
            if (Geo::VTOT % NTH != 0 && u >= Geo::VTOT) break;
            const int kp = u % (APF_KB / 2), d4 = u / (APF_KB / 2);
            const int sl = key_slot(2 * kp);
            const float fa[4] = {va[i].x, va[i].y, va[i].z, va[i].w}, fc[4] = {vc[i].x, vc[i].y, vc[i].z, vc[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                *(half2_t*)&sVh[(4 * d4 + e) * VS + sl] = half2_t{hi_h(fa[e]), hi_h(fc[e])};
                *(half2_t*)&sVl[(4 * d4 + e) * VS + sl] = half2_t{lo_h(fa[e]), lo_h(fc[e])};
            }
        }
        __syncthreads();
        if (kb + 1 < nkb) load_block(k0 + APF_KB);     // in flight during this block's products
        if (!active) continue;
        // S^T for two 16-key tiles: lane (g, j) holds keys 16hf + 4g + i of token r
        floatx4 s[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            s[hf] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const half8_t kh = *(const half8_t*)&sKh[(16 * hf + j) * KS + 32 * t + 8 * g];
                const half8_t kl = *(const half8_t*)&sKl[(16 * hf + j) * KS + 32 * t + 8 * g];
                s[hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[t], s[hf], 0, 0, 0);
                s[hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[t], s[hf], 0, 0, 0);
                s[hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[t], s[hf], 0, 0, 0);
            }
        }
        // online softmax of the lane's token over its 8 keys and the other
        // three lane groups' 24
        float v[8];
        float mx = -INFINITY;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = k0 + 16 * hf + 4 * g + i;
                const float x = (r < n && key <= pr) ? s[hf][i] * scale2 : -INFINITY;
                v[4 * hf + i] = x;
                mx = fmaxf(mx, x);
            }
        mx = cols_max(mx);
        const float mn = fmaxf(m, mx);
        const bool live = mn != -INFINITY;
        const float alpha = live ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
        float sum = 0.f;
        half8_t ph, pl;                                // P^T as the B operand, slots 8g + e
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float p = live ? __builtin_amdgcn_exp2f(v[e] - mn) : 0.f;
            sum += p;
            ph[e] = hi_h(p);
            pl[e] = lo_h(p);
        }
        l = l * alpha + cols_sum(sum);
        m = mn;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {   // a running max moved: rescale
#pragma unroll
            for (int d = 0; d < ND; ++d) o[d] *= alpha;
        }
#pragma unroll
        for (int d = 0; d < ND; ++d) {
            const half8_t vh = *(const half8_t*)&sVh[(16 * d + j) * VS + 8 * g];
            const half8_t vl = *(const half8_t*)&sVl[(16 * d + j) * VS + 8 * g];
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, o[d], 0, 0, 0);
        }
    }
    // partials of the tokens that have a key in this chunk (the merge reads
    // chunk c of token t exactly when c * CHUNK <= pos(t))
    if (active && r < n && k_begin <= pr) {
        const size_t pidx = ((size_t)(t0 + r) * Hq + hq) * nch_max + c;
        float* op = po + pidx * HD + 4 * g;
#pragma unroll
        for (int d = 0; d < ND; ++d) *(floatx4*)(op + 16 * d) = o[d];
        if (g == 0) *(float2*)(pml + pidx * 2) = make_float2(m * 0.6931471805599453f, l);   // m in ln units
    }
}

constexpr int APF_CHUNK = 256;  // key positions per unit: the merge kernel's chunk

struct PromptArgs {
    const float *q, *Kp, *Vp;
    const int32_t *blk_t0, *blk_n, *tok2seq, *tok_pos;
    const int64_t* kv_base;
    int Hq;
    int64_t head_stride;
    int nch_max;
    float *po, *pml;
};

template <int HD, int G>
static void launch_pf(int n_blk, int Hkv, hipStream_t s, hipEvent_t ev0, const PromptArgs& a) {
    SH_LAUNCH(ev0, nullptr, (attn_prompt_kernel<HD, G, APF_CHUNK>), dim3(Hkv, a.nch_max, n_blk),
              dim3(PromptGeom<HD, G>::NTH), 0, s, a.q, a.Kp, a.Vp, a.blk_t0, a.blk_n, a.tok2seq, a.tok_pos,
              a.kv_base, a.Hq, a.head_stride, a.nch_max, a.po, a.pml);
}

template <int HD>
static int launch_pf_g(int G, int n_blk, int Hkv, hipStream_t s, hipEvent_t ev0, const PromptArgs& a) {
    switch (G) {
        case 1: launch_pf<HD, 1>(n_blk, Hkv, s, ev0, a); return 0;
        case 2: launch_pf<HD, 2>(n_blk, Hkv, s, ev0, a); return 0;
        case 4: launch_pf<HD, 4>(n_blk, Hkv, s, ev0, a); return 0;
        case 8: launch_pf<HD, 8>(n_blk, Hkv, s, ev0, a); return 0;
        default: return -5;
    }
}

static bool shape_ok(int Hq, int Hkv, int HD) {
    if (Hkv <= 0 || Hq % Hkv) return false;
    const int G = Hq / Hkv;
    return (HD == 64 || HD == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
}

bool attention_prompt_mfma(int Hq, int Hkv, int HD, bool kv_f16) {
    return !kv_f16 && knobs().attn_mfma && shape_ok(Hq, Hkv, HD);
}

int attention_prompt_block(int G) { return G >= APF_MIN_WAVES ? APF_TILE : APF_TILE * (APF_MIN_WAVES / G); }

int launch_attention_prompt(const float* q, const float* Kp, const float* Vp, const int32_t* tok2seq,
                            const int32_t* tok_pos, const int64_t* kv_base, const int32_t* blk_t0,
                            const int32_t* blk_n, int n_blk, int Hq, int Hkv, int HD, int64_t head_stride,
                            int nch_max, float* po, float* pml, hipStream_t s, hipEvent_t ev0) {
    if (n_blk <= 0) return 0;
    if (!shape_ok(Hq, Hkv, HD) || attn_chunk_size() != APF_CHUNK) {
        set_error(-5, "prompt attention: head_dim %d with %d/%d heads is not supported", HD, Hq, Hkv);
        return -5;
    }
    if (n_blk > 65535 || nch_max > 65535) {
        set_error(-5, "prompt attention: %d blocks / %d key chunks exceed the grid", n_blk, nch_max);
        return -5;
    }
    const PromptArgs a{q, Kp, Vp, blk_t0, blk_n, tok2seq, tok_pos, kv_base, Hq, head_stride, nch_max, po, pml};
    const int G = Hq / Hkv;
    const int rc = HD == 128 ? launch_pf_g<128>(G, n_blk, Hkv, s, ev0, a) : launch_pf_g<64>(G, n_blk, Hkv, s, ev0, a);
    if (rc) return rc;
    SH_CHECK_LAUNCH();
    return 0;
}

}  // namespace slate_hip
