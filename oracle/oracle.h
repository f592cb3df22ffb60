/*
 * oracle.h -- CPU restatement of slate's decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker.  Every function states
 * the reference file:line it restates (paths relative to the slate tree).
 *
 * Floating-point order follows the reference as built with its own flags
 * (-std=c11 -O3 -mavx2 -mfma, so no implicit FMA contraction in scalar code):
 * where the reference runs an AVX2 path, the eight lanes are emulated in
 * scalar C with fmaf() so the oracle reproduces the reference bit-for-bit.
 */
#ifndef SLATE_ORACLE_H
#define SLATE_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_Q4K_BLOCK_BYTES 144
#define ORC_Q4K_BLOCK_ELEMS 256

/* ---- number formats ---------------------------------------------------- */
float    orc_f16_to_f32(uint16_t h);                               /* precision.c:10-29 */
void     orc_f16_to_f32_n(float* dst, const uint16_t* src, int64_t n);   /* precision.c:53-55 */
void     orc_q4k_scale_min(const uint8_t* s, int j,
                           uint8_t* sc, uint8_t* mn);              /* quant.c:157-166 */
void     orc_dequant_q4k(float* dst, const void* src, int64_t n);  /* quant.c:168-202 */
float    orc_dot_q4k_f32(const void* blocks, const float* y,
                         int64_t n);                               /* quant.c:210-304 */
void     orc_q4k_matvec(float* y, const void* A, const float* x,
                        int M, int K);                             /* quant.c:306-313 */
/* Y[b,:] = A @ X[b,:] for b < B: the reference has no batched Q4_K entry,
 * so batched semantics are B independent calls of quant.c:306-313. */
void     orc_q4k_matmul(float* Y, const void* A, const float* X,
                        int B, int M, int K);

/* ---- Q8_0 (include/slate/quant.h:16-31) --------------------------------- */
#define ORC_Q8_0_BLOCK_BYTES 34
#define ORC_Q8_0_BLOCK_ELEMS 32
void     orc_dequant_q8_0(float* dst, const void* src, int64_t n); /* quant.c:12-25 */
float    orc_dot_q8_0_f32(const void* blocks, const float* x,
                          int64_t n);                              /* quant.c:64-109 */
void     orc_q8_0_matvec(float* y, const void* A, const float* x,
                         int M, int K);                            /* quant.c:126-133 */
/* B independent calls of quant.c:126-133. */
void     orc_q8_0_matmul(float* Y, const void* A, const float* X,
                         int B, int M, int K);

/* ---- f32 GEMM behind the vtable ---------------------------------------- */
/* C[M,N] += A[M,K] @ B[K,N]; KC=128 blocked fma chains, matmul.c:36-199 */
void     orc_gemm_accumulate(float* C, int64_t ldc, const float* A, int64_t lda,
                             const float* B, int64_t ldb, int M, int K, int N);
void     orc_matvec(float* y, const float* A, const float* x, int M, int K);   /* backend_cpu.c:33-36 */
void     orc_linear_batch(float* C, const float* X, const float* W,
                          int B, int K, int N);                                /* backend_cpu.c:38-42 */

/* ---- row primitives (vtable) ------------------------------------------- */
void     orc_rmsnorm_row(float* y, const float* x, const float* w, int D, float eps); /* backend_cpu.c:48-76 */
void     orc_silu_mul(float* y, const float* gate, const float* up, int H);           /* backend_cpu.c:78-97 */
void     orc_add_inplace(float* y, const float* x, int D);                            /* backend_cpu.c:99-111 */
void     orc_embed_lookup(float* y, const float* W, int token, int D);                /* backend_cpu.c:113-115 */
void     orc_attention_step(float* out, const float* q, const float* K,
                            const float* V, float* scores, int L, int D);             /* backend_cpu.c:117-166 */

/* ---- LLaMA pieces -------------------------------------------------------- */
void     orc_rope_row(float* row, int n_heads, int head_dim, int pos, float theta);   /* llama_infer.c:77-92 */
void     orc_attention_multihead(float* out, const float* q, const float* K,
                                 const float* V, float* scores, int L,
                                 int n_q_heads, int n_kv_heads, int head_dim);        /* llama_infer.c:97-129 */
int      orc_argmax(const float* p, int n);                                           /* sampling.c:14-18 */

/* ---- ragged batch packing (no reference function: the reference packs
 * implicitly in its per-session loops, engine.c:556-563 and :582-596) ---- */
typedef struct orc_pack_out {
    int32_t* tok_off;   /* [B+1] exclusive prefix sum of n_new          */
    int32_t* tok2seq;   /* [T]   sequence index of each packed token     */
    int32_t* tok_pos;   /* [T]   absolute position of each packed token  */
    int64_t* kv_base;   /* [B]   float offset of the slot's KV region    */
    int32_t* last_tok;  /* [B]   packed index of each sequence's last token */
} orc_pack_out;
/* Returns T (total packed tokens) or a negative error. */
int      orc_pack_batch(const int32_t* slot, const int32_t* pos0, const int32_t* n_new,
                        int B, int max_seq, int64_t slot_stride, orc_pack_out* out);

/* ---- LLaMA model view + decode (llama_infer.c:134-278) ------------------ */
typedef struct orc_llama_cfg {          /* field order of llama.h:53-65 */
    int   n_layers, d_model, ffn_hidden, n_heads, n_kv_heads, head_dim;
    int   max_seq, vocab;
    float theta_base, rms_eps;
    int   tied_output;
} orc_llama_cfg;

typedef struct orc_llama_layer {        /* field order of llama.h:69-86 */
    const void *attn_norm, *attn_q, *attn_k, *attn_v, *attn_output;
    const void *ffn_norm, *ffn_gate, *ffn_up, *ffn_down;
    int attn_q_dtype, attn_k_dtype, attn_v_dtype, attn_output_dtype;
    int ffn_gate_dtype, ffn_up_dtype, ffn_down_dtype;
} orc_llama_layer;

typedef struct orc_llama_model {
    orc_llama_cfg cfg;
    const float* token_embd;            /* f32 [vocab, d_model] */
    const float* output_norm;           /* f32 [d_model] */
    const void*  output;                /* [vocab, d_model] */
    int          output_dtype;          /* 0 = f32, 18 = Q4_K */
    const orc_llama_layer* layers;      /* [n_layers] */
} orc_llama_model;

typedef struct orc_session orc_session;
orc_session* orc_session_new(const orc_llama_model* m);                   /* llama_infer.c:212-244 */
void         orc_session_free(orc_session* s);
int          orc_session_position(const orc_session* s);
/* Returns 0, -1 bad args, -2 cache full, -3 bad token (llama_infer.c:144-145). */
int          orc_decode_step(orc_session* s, int32_t token, float* logits);        /* llama_infer.c:134-206 */
int          orc_prefill(orc_session* s, const int32_t* toks, int n, float* logits); /* llama_infer.c:262-272 */
/* Copy a session's KV cache out ([n_layers, max_seq, kv_dim] each). */
void         orc_session_kv(const orc_session* s, float* K_out, float* V_out);
int          orc_session_set_state(orc_session* s, const float* K, const float* V, int pos);

#ifdef __cplusplus
}
#endif
#endif
