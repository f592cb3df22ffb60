/*
 * oracle.c -- CPU restatement of slate's decode hot path (test infrastructure).
 *
 * This file is the checker for the HIP backend, never the product: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * Each function cites the slate source it restates; the AVX2 paths the
 * reference actually runs (it is built with -mavx2 -mfma) are emulated lane
 * by lane so that results match the reference bit-for-bit where the
 * reference itself is deterministic.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* precision.c:10-29 -- IEEE binary16 -> binary32, exact, incl. subnormals. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            /* normalise: shift until the hidden bit (0x400) appears */
            int shift = 0;
            while ((m & 0x400u) == 0) { m <<= 1; ++shift; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)(113 - shift) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* precision.c:53-55 -- element-wise; keeps signalling-NaN payloads intact
 * (a scalar return through a host language would quiet them). */
void orc_f16_to_f32_n(float* dst, const uint16_t* src, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

/* quant.c:157-166 -- 6-bit (scale, min) of sub-block j from the 12-byte table. */
void orc_q4k_scale_min(const uint8_t* s, int j, uint8_t* sc, uint8_t* mn) {
    if (j < 4) {
        *sc = (uint8_t)(s[j] & 63);
        *mn = (uint8_t)(s[j + 4] & 63);
    } else {
        *sc = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

static void q4k_header(const uint8_t* blk, float* d, float* dmin) {
    uint16_t a, b;
    memcpy(&a, blk, 2);
    memcpy(&b, blk + 2, 2);
    *d = orc_f16_to_f32(a);
    *dmin = orc_f16_to_f32(b);
}

/* quant.c:168-202 -- w = (d*sc)*q - dmin*mn.  Slate's nibble order: sub-block
 * j reads qs[16j..16j+15]; the low nibble of byte i is element i and the high
 * nibble is element i+16 (this is NOT upstream ggml's 64-element grouping). */
void orc_dequant_q4k(float* dst, const void* src, int64_t n) {
    const uint8_t* p = (const uint8_t*)src;
    for (int64_t b = 0; b < n / ORC_Q4K_BLOCK_ELEMS; ++b) {
        const uint8_t* blk = p + b * ORC_Q4K_BLOCK_BYTES;
        float d, dmin;
        q4k_header(blk, &d, &dmin);
        float* o = dst + b * ORC_Q4K_BLOCK_ELEMS;
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, mn;
            orc_q4k_scale_min(blk + 4, j, &sc, &mn);
            float sd = d * (float)sc;
            float sm = dmin * (float)mn;
            const uint8_t* q = blk + 16 + 16 * j;
            for (int i = 0; i < 16; ++i) {
                o[32 * j + i]      = sd * (float)(q[i] & 15) - sm;
                o[32 * j + i + 16] = sd * (float)(q[i] >> 4) - sm;
            }
        }
    }
}

/* Horizontal sum in the order of simd_helpers.h:14-21 (lo+hi, then two hadds). */
static float hsum8(const float v[8]) {
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s1) + (s2 + s3);
}

/* quant.c:210-304, AVX2 branch (the one the reference build runs):
 * per sub-block, eight lanes accumulate sc*Sum(q*y) and mn*Sum(y); one
 * horizontal sum per super-block; super-blocks accumulate in double. */
float orc_dot_q4k_f32(const void* blocks, const float* y, int64_t n) {
    const uint8_t* p = (const uint8_t*)blocks;
    double total = 0;
    for (int64_t b = 0; b < n / ORC_Q4K_BLOCK_ELEMS; ++b) {
        const uint8_t* blk = p + b * ORC_Q4K_BLOCK_BYTES;
        float d, dmin;
        q4k_header(blk, &d, &dmin);
        const float* yb = y + b * ORC_Q4K_BLOCK_ELEMS;
        float dacc[8] = {0}, macc[8] = {0};
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, mn;
            orc_q4k_scale_min(blk + 4, j, &sc, &mn);
            const uint8_t* q = blk + 16 + 16 * j;
            const float* yj = yb + 32 * j;
            for (int l = 0; l < 8; ++l) {
                float q0 = (float)(q[l] & 15), q1 = (float)(q[8 + l] & 15);
                float q2 = (float)(q[l] >> 4), q3 = (float)(q[8 + l] >> 4);
                float qy01 = fmaf(q0, yj[l], q1 * yj[8 + l]);
                float qy23 = fmaf(q2, yj[16 + l], q3 * yj[24 + l]);
                float qy = qy01 + qy23;
                float sy = (yj[l] + yj[8 + l]) + (yj[16 + l] + yj[24 + l]);
                dacc[l] = fmaf((float)sc, qy, dacc[l]);
                macc[l] = fmaf((float)mn, sy, macc[l]);
            }
        }
        float sd = hsum8(dacc), sm = hsum8(macc);
        total += (double)d * (double)sd - (double)dmin * (double)sm;
    }
    return (float)total;
}

/* quant.c:306-313 */
void orc_q4k_matvec(float* y, const void* A, const float* x, int M, int K) {
    size_t row_bytes = (size_t)(K / ORC_Q4K_BLOCK_ELEMS) * ORC_Q4K_BLOCK_BYTES;
    for (int m = 0; m < M; ++m)
        y[m] = orc_dot_q4k_f32((const uint8_t*)A + (size_t)m * row_bytes, x, K);
}

void orc_q4k_matmul(float* Y, const void* A, const float* X, int B, int M, int K) {
    for (int b = 0; b < B; ++b)
        orc_q4k_matvec(Y + (size_t)b * M, A, X + (size_t)b * K, M, K);
}

/* ------------------------------------------------------------------------ */
/* quant.c:12-25 -- Q8_0 block: [f16 d][32 x int8 q]; w = d * (float)q. */
void orc_dequant_q8_0(float* dst, const void* src, int64_t n) {
    const uint8_t* p = (const uint8_t*)src;
    for (int64_t b = 0; b < n / ORC_Q8_0_BLOCK_ELEMS; ++b) {
        const uint8_t* blk = p + b * ORC_Q8_0_BLOCK_BYTES;
        uint16_t h;
        memcpy(&h, blk, 2);
        const float d = orc_f16_to_f32(h);
        const int8_t* q = (const int8_t*)(blk + 2);
        for (int i = 0; i < ORC_Q8_0_BLOCK_ELEMS; ++i) dst[b * ORC_Q8_0_BLOCK_ELEMS + i] = d * (float)q[i];
    }
}

/* quant.c:64-109, AVX2 branch (the one the reference build runs): lane l of
 * one 8-wide accumulator takes, per block in order, fma(d*q[i], x[i], acc)
 * for i = l, 8+l, 16+l, 24+l; the eight lanes are then added left to right
 * into a float that starts at 0. */
float orc_dot_q8_0_f32(const void* blocks, const float* x, int64_t n) {
    const uint8_t* p = (const uint8_t*)blocks;
    float acc[8] = {0};
    for (int64_t b = 0; b < n / ORC_Q8_0_BLOCK_ELEMS; ++b) {
        const uint8_t* blk = p + b * ORC_Q8_0_BLOCK_BYTES;
        uint16_t h;
        memcpy(&h, blk, 2);
        const float d = orc_f16_to_f32(h);
        const int8_t* q = (const int8_t*)(blk + 2);
        const float* xb = x + b * ORC_Q8_0_BLOCK_ELEMS;
        for (int r = 0; r < 4; ++r)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(d * (float)q[8 * r + l], xb[8 * r + l], acc[l]);
    }
    float total = 0.0f;
    for (int l = 0; l < 8; ++l) total += acc[l];
    return total;
}

/* quant.c:126-133 -- row stride K/32 * 34 bytes. */
void orc_q8_0_matvec(float* y, const void* A, const float* x, int M, int K) {
    size_t row_bytes = (size_t)(K / ORC_Q8_0_BLOCK_ELEMS) * ORC_Q8_0_BLOCK_BYTES;
    for (int m = 0; m < M; ++m)
        y[m] = orc_dot_q8_0_f32((const uint8_t*)A + (size_t)m * row_bytes, x, K);
}

void orc_q8_0_matmul(float* Y, const void* A, const float* X, int B, int M, int K) {
    for (int b = 0; b < B; ++b)
        orc_q8_0_matvec(Y + (size_t)b * M, A, X + (size_t)b * K, M, K);
}

/* ------------------------------------------------------------------------ */
/* matmul.c:158-199 with the 8x16 microkernel (:85-134): every C element is a
 * sum over KC=128 slices; inside a slice a zero-started fma chain, and each
 * slice's chain is then added to C in ascending slice order.  Blocking over
 * M and N does not change any single element's arithmetic. */
void orc_gemm_accumulate(float* C, int64_t ldc, const float* A, int64_t lda,
                         const float* B, int64_t ldb, int M, int K, int N) {
    enum { KC = 128 };
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            float c = C[i * ldc + j];
            for (int k0 = 0; k0 < K; k0 += KC) {
                int k1 = k0 + KC < K ? k0 + KC : K;
                float acc = 0.0f;
                for (int k = k0; k < k1; ++k) acc = fmaf(A[i * lda + k], B[k * ldb + j], acc);
                c += acc;
            }
            C[i * ldc + j] = c;
        }
    }
}

/* backend_cpu.c:33-36 */
void orc_matvec(float* y, const float* A, const float* x, int M, int K) {
    memset(y, 0, (size_t)M * sizeof(float));
    orc_gemm_accumulate(y, 1, A, K, x, 1, M, K, 1);
}

/* backend_cpu.c:38-42 -- W is [K, N] here (not [out, in]). */
void orc_linear_batch(float* C, const float* X, const float* W, int B, int K, int N) {
    memset(C, 0, (size_t)B * (size_t)N * sizeof(float));
    orc_gemm_accumulate(C, N, X, K, W, N, B, K, N);
}

/* backend_cpu.c:48-76 */
void orc_rmsnorm_row(float* y, const float* x, const float* w, int D, float eps) {
    float acc[8] = {0};
    int d = 0;
    for (; d + 8 <= D; d += 8)
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[d + l], x[d + l], acc[l]);
    double sq = (double)hsum8(acc);
    for (; d < D; ++d) sq += (double)x[d] * (double)x[d];
    float inv = 1.0f / sqrtf((float)(sq / (double)D) + eps);
    for (d = 0; d < D; ++d) y[d] = (x[d] * w[d]) * inv;
}

/* simd_helpers.h:36-69, one lane: clamp to +-88.376, n = floor(x*log2e+1/2),
 * two-constant Cody-Waite reduction, degree-6 polynomial (Cephes expf
 * coefficients, as the reference uses them) evaluated with fused steps,
 * then scaling by 2^n through the exponent bits. */
static float exp_lane(float x) {
    x = fminf(x, 88.3762626647949f);
    x = fmaxf(x, -88.3762626647949f);
    float fx = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
    float r = fmaf(-fx, 0.693359375f, x);
    r = fmaf(-fx, -2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    p = fmaf(p, r * r, r);
    p = p + 1.0f;
    uint32_t bits = (uint32_t)((int32_t)fx + 127) << 23;
    float scale;
    memcpy(&scale, &bits, 4);
    return p * scale;
}

/* backend_cpu.c:78-97: 8-wide groups use sigmoid = 1/(1+exp_poly(-g)) and
 * y = (g*s)*u; the tail uses (g/(1+expf(-g)))*u. */
void orc_silu_mul(float* y, const float* gate, const float* up, int H) {
    int H8 = H & ~7, d;
    for (d = 0; d < H8; ++d) {
        float g = gate[d];
        float s = 1.0f / (1.0f + exp_lane(0.0f - g));
        y[d] = (g * s) * up[d];
    }
    for (; d < H; ++d) {
        float g = gate[d];
        y[d] = (g / (1.0f + expf(-g))) * up[d];
    }
}

/* backend_cpu.c:99-111 */
void orc_add_inplace(float* y, const float* x, int D) {
    for (int d = 0; d < D; ++d) y[d] += x[d];
}

/* backend_cpu.c:113-115 */
void orc_embed_lookup(float* y, const float* W, int token, int D) {
    memcpy(y, W + (int64_t)token * D, (size_t)D * sizeof(float));
}

/* backend_cpu.c:117-166 (AVX2 branch): 8-lane fma dot + hsum, scalar tail;
 * softmax with max subtraction, expf, double sum, multiply by (float)(1/S);
 * output accumulated with fma over 8-lane groups, plain mul+add on the tail. */
void orc_attention_step(float* out, const float* q, const float* K,
                        const float* V, float* scores, int L, int D) {
    float scale = 1.0f / sqrtf((float)D);
    int D8 = D & ~7;
    for (int t = 0; t < L; ++t) {
        const float* k = K + (int64_t)t * D;
        float acc[8] = {0};
        for (int d = 0; d < D8; d += 8)
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(q[d + l], k[d + l], acc[l]);
        float s = hsum8(acc);
        for (int d = D8; d < D; ++d) s += q[d] * k[d];
        scores[t] = s * scale;
    }
    float m = scores[0];
    for (int t = 1; t < L; ++t) if (scores[t] > m) m = scores[t];
    double S = 0;
    for (int t = 0; t < L; ++t) { scores[t] = expf(scores[t] - m); S += scores[t]; }
    float invS = (float)(1.0 / S);
    for (int t = 0; t < L; ++t) scores[t] *= invS;
    memset(out, 0, (size_t)D * sizeof(float));
    for (int t = 0; t < L; ++t) {
        const float* v = V + (int64_t)t * D;
        float w = scores[t];
        for (int d = 0; d < D8; ++d) out[d] = fmaf(w, v[d], out[d]);
        for (int d = D8; d < D; ++d) out[d] += w * v[d];
    }
}

/* ------------------------------------------------------------------------ */
/* llama_infer.c:77-92 -- half-split rotation of (x[i], x[i+hd/2]) per head,
 * angle = pos * theta^(-2i/hd) computed in float with libm powf/cosf/sinf. */
void orc_rope_row(float* row, int n_heads, int head_dim, int pos, float theta) {
    int half = head_dim / 2;
    for (int h = 0; h < n_heads; ++h) {
        float* x = row + h * head_dim;
        for (int i = 0; i < half; ++i) {
            float inv_freq = powf(theta, -2.0f * (float)i / (float)head_dim);
            float ang = (float)pos * inv_freq;
            float c = cosf(ang), s = sinf(ang);
            float a = x[i], b = x[i + half];
            x[i] = a * c - b * s;
            x[i + half] = a * s + b * c;
        }
    }
}

/* llama_infer.c:97-129 -- scalar GQA attention, q head hq reads kv head
 * hq / (Hq/Hkv); scores scaled by 1/sqrtf(hd); double softmax sum. */
void orc_attention_multihead(float* out, const float* q, const float* K,
                             const float* V, float* scores, int L,
                             int n_q_heads, int n_kv_heads, int head_dim) {
    int kv_dim = n_kv_heads * head_dim;
    int group = n_q_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)head_dim);
    for (int hq = 0; hq < n_q_heads; ++hq) {
        int hkv = hq / group;
        const float* qh = q + hq * head_dim;
        float* oh = out + hq * head_dim;
        for (int t = 0; t < L; ++t) {
            const float* k = K + (int64_t)t * kv_dim + hkv * head_dim;
            float s = 0;
            for (int d = 0; d < head_dim; ++d) s += qh[d] * k[d];
            scores[t] = s * scale;
        }
        float m = scores[0];
        for (int t = 1; t < L; ++t) if (scores[t] > m) m = scores[t];
        double S = 0;
        for (int t = 0; t < L; ++t) { scores[t] = expf(scores[t] - m); S += scores[t]; }
        float invS = (float)(1.0 / S);
        for (int t = 0; t < L; ++t) scores[t] *= invS;
        for (int d = 0; d < head_dim; ++d) oh[d] = 0;
        for (int t = 0; t < L; ++t) {
            const float* v = V + (int64_t)t * kv_dim + hkv * head_dim;
            float w = scores[t];
            for (int d = 0; d < head_dim; ++d) oh[d] += w * v[d];
        }
    }
}

/* sampling.c:14-18 -- strict '>' keeps the lowest index on ties. */
int orc_argmax(const float* p, int n) {
    int best = 0;
    float bv = p[0];
    for (int i = 1; i < n; ++i) if (p[i] > bv) { bv = p[i]; best = i; }
    return best;
}

/* ------------------------------------------------------------------------ */
/* Ragged-batch packing.  Sequence b owns KV slot slot[b], already holds
 * pos0[b] positions and contributes n_new[b] >= 1 tokens this step (1 for
 * decode, a prompt chunk for prefill).  Tokens are packed sequence-major. */
int orc_pack_batch(const int32_t* slot, const int32_t* pos0, const int32_t* n_new,
                   int B, int max_seq, int64_t slot_stride, orc_pack_out* out) {
    if (B < 1) return -1;
    int32_t t = 0;
    for (int b = 0; b < B; ++b) {
        if (n_new[b] < 1 || pos0[b] < 0 || slot[b] < 0) return -1;
        if (pos0[b] + n_new[b] > max_seq) return -2;
        out->tok_off[b] = t;
        for (int i = 0; i < n_new[b]; ++i) {
            out->tok2seq[t + i] = b;
            out->tok_pos[t + i] = pos0[b] + i;
        }
        t += n_new[b];
        out->kv_base[b] = (int64_t)slot[b] * slot_stride;
        out->last_tok[b] = t - 1;
    }
    out->tok_off[B] = t;
    return t;
}

/* ------------------------------------------------------------------------ */
/* llama_infer.c:53-71, :212-244 */
struct orc_session {
    const orc_llama_model* m;
    int pos;
    float *K, *V;                               /* [n_layers, max_seq, kv_dim] */
    float *x, *xn, *q, *k, *v, *att, *g, *u, *tmp, *scores;
};

orc_session* orc_session_new(const orc_llama_model* m) {
    if (!m) return NULL;
    const orc_llama_cfg* c = &m->cfg;
    orc_session* s = (orc_session*)calloc(1, sizeof(*s));
    if (!s) return NULL;
    int kv_dim = c->n_kv_heads * c->head_dim;
    size_t kv = (size_t)c->n_layers * c->max_seq * kv_dim;
    int big = c->d_model > c->vocab ? c->d_model : c->vocab;
    s->m = m;
    s->K = (float*)calloc(kv, sizeof(float));
    s->V = (float*)calloc(kv, sizeof(float));
    s->x = (float*)calloc((size_t)c->d_model, 4);
    s->xn = (float*)calloc((size_t)c->d_model, 4);
    s->q = (float*)calloc((size_t)c->d_model, 4);
    s->k = (float*)calloc((size_t)kv_dim, 4);
    s->v = (float*)calloc((size_t)kv_dim, 4);
    s->att = (float*)calloc((size_t)c->d_model, 4);
    s->g = (float*)calloc((size_t)c->ffn_hidden, 4);
    s->u = (float*)calloc((size_t)c->ffn_hidden, 4);
    s->tmp = (float*)calloc((size_t)big, 4);
    s->scores = (float*)calloc((size_t)c->max_seq, 4);
    if (!s->K || !s->V || !s->x || !s->xn || !s->q || !s->k || !s->v || !s->att ||
        !s->g || !s->u || !s->tmp || !s->scores) {
        orc_session_free(s);
        return NULL;
    }
    return s;
}

void orc_session_free(orc_session* s) {
    if (!s) return;
    free(s->K); free(s->V); free(s->x); free(s->xn); free(s->q); free(s->k);
    free(s->v); free(s->att); free(s->g); free(s->u); free(s->tmp); free(s->scores);
    free(s);
}

int orc_session_position(const orc_session* s) { return s ? s->pos : -1; }

void orc_session_kv(const orc_session* s, float* K_out, float* V_out) {
    const orc_llama_cfg* c = &s->m->cfg;
    size_t n = (size_t)c->n_layers * c->max_seq * c->n_kv_heads * c->head_dim;
    memcpy(K_out, s->K, n * sizeof(float));
    memcpy(V_out, s->V, n * sizeof(float));
}

/* Load a KV state (K/V [n_layers, max_seq, kv_dim], the layout
 * orc_session_kv returns) and a position, so that decode steps can be
 * checked from a context that another implementation built.  Test
 * infrastructure, like ref_session_set_state for the compiled reference. */
int orc_session_set_state(orc_session* s, const float* K, const float* V, int pos) {
    if (!s || !K || !V) return -1;
    const orc_llama_cfg* c = &s->m->cfg;
    if (pos < 0 || pos > c->max_seq) return -1;
    size_t n = (size_t)c->n_layers * c->max_seq * c->n_kv_heads * c->head_dim;
    memcpy(s->K, K, n * sizeof(float));
    memcpy(s->V, V, n * sizeof(float));
    s->pos = pos;
    return 0;
}

/* llama_infer.c:43-51 -- dtype 18 (Q4_K) takes the Q4_K matvec and f32 the
 * f32 one.  Dtype 16 (Q8_0) is where this restatement departs on purpose:
 * the reference reads a Q8_0 tensor's bytes as f32 (its dispatch knows only
 * 18), which is a bug, so here it takes quant.c:126-133 -- the corrected
 * dispatch that the HIP engine implements. */
static void mv(float* y, const void* W, int dtype, const float* x, int M, int K) {
    if (dtype == 18) orc_q4k_matvec(y, W, x, M, K);
    else if (dtype == 16) orc_q8_0_matvec(y, W, x, M, K);
    else orc_matvec(y, (const float*)W, x, M, K);
}

/* llama_infer.c:134-206 */
int orc_decode_step(orc_session* s, int32_t token, float* logits) {
    if (!s || !logits) return -1;
    const orc_llama_model* m = s->m;
    const orc_llama_cfg* c = &m->cfg;
    int D = c->d_model, H = c->ffn_hidden, hd = c->head_dim;
    int kv_dim = c->n_kv_heads * hd;
    int p = s->pos;
    if (p >= c->max_seq) return -2;
    if (token < 0 || token >= c->vocab) return -3;
    memcpy(s->x, m->token_embd + (int64_t)token * D, (size_t)D * 4);
    for (int li = 0; li < c->n_layers; ++li) {
        const orc_llama_layer* L = &m->layers[li];
        orc_rmsnorm_row(s->xn, s->x, (const float*)L->attn_norm, D, c->rms_eps);
        mv(s->q, L->attn_q, L->attn_q_dtype, s->xn, D, D);
        mv(s->k, L->attn_k, L->attn_k_dtype, s->xn, kv_dim, D);
        mv(s->v, L->attn_v, L->attn_v_dtype, s->xn, kv_dim, D);
        orc_rope_row(s->q, c->n_heads, hd, p, c->theta_base);
        orc_rope_row(s->k, c->n_kv_heads, hd, p, c->theta_base);
        float* Kl = s->K + (int64_t)li * c->max_seq * kv_dim;
        float* Vl = s->V + (int64_t)li * c->max_seq * kv_dim;
        memcpy(Kl + (int64_t)p * kv_dim, s->k, (size_t)kv_dim * 4);
        memcpy(Vl + (int64_t)p * kv_dim, s->v, (size_t)kv_dim * 4);
        orc_attention_multihead(s->att, s->q, Kl, Vl, s->scores, p + 1,
                                c->n_heads, c->n_kv_heads, hd);
        mv(s->tmp, L->attn_output, L->attn_output_dtype, s->att, D, D);
        orc_add_inplace(s->x, s->tmp, D);
        orc_rmsnorm_row(s->xn, s->x, (const float*)L->ffn_norm, D, c->rms_eps);
        mv(s->g, L->ffn_gate, L->ffn_gate_dtype, s->xn, H, D);
        mv(s->u, L->ffn_up, L->ffn_up_dtype, s->xn, H, D);
        orc_silu_mul(s->g, s->g, s->u, H);
        mv(s->tmp, L->ffn_down, L->ffn_down_dtype, s->g, D, H);
        orc_add_inplace(s->x, s->tmp, D);
    }
    orc_rmsnorm_row(s->xn, s->x, m->output_norm, D, c->rms_eps);
    mv(logits, m->output, m->output_dtype, s->xn, c->vocab, D);
    s->pos = p + 1;
    return 0;
}

/* llama_infer.c:262-272 -- prefill is n sequential decode steps; the logits
 * of the last prompt token are returned. */
int orc_prefill(orc_session* s, const int32_t* toks, int n, float* logits) {
    if (!s || !toks || !logits || n <= 0) return -1;
    for (int i = 0; i < n; ++i) {
        int rc = orc_decode_step(s, toks[i], logits);
        if (rc != 0) return rc;
    }
    return 0;
}
