/*
 * slate_hip.h -- C ABI of the MI355X (gfx950) HIP compute backend for slate.
 *
 * Everything here is plain C: pointers, sizes and ints, no C++ types, no
 * exceptions.  Pointers documented as "device" come from the backend's
 * alloc() (or slate_hip_alloc); "host" pointers are ordinary memory.
 *
 * 1. slate_backend_hip() returns the drop-in vtable.  Its first 14 members
 *    are slate_backend_t exactly as include/slate/backend.h:41-99 declares
 *    it (same order, same signatures, same meaning), so slate's engines call
 *    it unchanged; the extension entries follow `sync`.
 * 2. slate_hip_* functions are the same entry points under stable names for
 *    FFI binders, plus the extensions the vtable appends.
 * 3. slate_hip_llama_* is a device-resident LLaMA engine with the session API
 *    of include/slate/llama.h:124-139 and a ragged continuous-batching step
 *    generalising slate_infer_batch_step (include/slate/infer.h:170-187).
 *
 * Errors: vtable compute entries return void (backend.h:58-98), so failures
 * are recorded in a sticky per-process error that slate_hip_last_error()
 * reports and slate_hip_clear_error() resets; int-returning entries return
 * 0 on success and a negative code: -1 bad argument, -2 cache full /
 * capacity exceeded, -3 bad token (llama_infer.c:144-145), -5 not
 * supported, -7 device/runtime failure.
 *
 * Threading: all work is enqueued on one backend stream created at first
 * use (default priority); entries may be called from several host threads;
 * sync() waits for everything enqueued so far.
 */
#ifndef SLATE_HIP_H
#define SLATE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- slate_backend_t (include/slate/backend.h:41-99) ----------------------
 * When slate's own header is visible -- already included, or reachable as
 * "slate/backend.h" on the include path -- it is used as is, factories
 * (backend.h:104-110) included.  Otherwise the same struct is declared here,
 * member for member, under this header's own guard; slate's guard
 * SLATE_BACKEND_H is never defined here, so a translation unit that later
 * includes slate/backend.h by another path gets a loud redefinition error
 * rather than a silently skipped header.  In a TU that uses both headers,
 * put slate's include/ directory on the include path (or include
 * slate/backend.h first). */
#if !defined(SLATE_BACKEND_H) && defined(__has_include)
#if __has_include("slate/backend.h")
#include "slate/backend.h"
#endif
#endif
#if !defined(SLATE_BACKEND_H) && !defined(SLATE_HIP_BACKEND_T_DECLARED)
#define SLATE_HIP_BACKEND_T_DECLARED 1
typedef struct slate_backend {
    const char* name;
    void* (*alloc)(size_t bytes);
    void  (*release)(void* dev_ptr);
    void  (*copy_h2d)(void* dst_dev, const void* src_host, size_t bytes);
    void  (*copy_d2h)(void* dst_host, const void* src_dev, size_t bytes);
    void  (*matvec)(float* y, const float* A, const float* x, int M, int K);
    void  (*linear_batch)(float* C, const float* X, const float* W, int B, int K, int N);
    void  (*matvec_q4k)(float* y, const void* A_q4k, const float* x, int M, int K);
    void  (*rmsnorm_row)(float* y, const float* x, const float* w, int D, float eps);
    void  (*silu_mul)(float* y, const float* gate, const float* up, int H);
    void  (*add_inplace)(float* y, const float* x, int D);
    void  (*embed_lookup)(float* y, const float* W, int token_id, int D);
    void  (*attention_step)(float* out, const float* q, const float* K_cache,
                            const float* V_cache, float* scores, int L, int D);
    void  (*sync)(void);
} slate_backend_t;
#endif

/* Vtable extended past `sync`.  slate_backend_hip() returns &ext.base. */
typedef struct slate_hip_backend {
    slate_backend_t base;
    /* Y[B,M] = X[B,K] @ dequant(A)[M,K]^T; A is M rows of K/256 Q4_K blocks. */
    int  (*matmul_q4k)(float* Y, const void* A_q4k, const float* X, int B, int M, int K);
    /* Bit-exact dequantisation (quant.c:168-202), n % 256 == 0. */
    int  (*dequant_q4k)(float* dst, const void* A_q4k, int64_t n);
    /* y[b,:] = rmsnorm(x[b,:]) * w for B rows. */
    int  (*rmsnorm_rows)(float* y, const float* x, const float* w, int B, int D, float eps);
    /* Row-wise RoPE (llama_infer.c:77-92) with per-row positions (device
     * int32[n_rows]); |pos| must be < max_pos. */
    int  (*rope_rows)(float* x, const int32_t* pos, int n_rows, int n_heads, int head_dim,
                      float theta_base, int max_pos);
    /* Greedy argmax per row, lowest index on ties (sampling.c:14-18). */
    int  (*argmax_rows)(int32_t* out, const float* logits, int B, int V);
    const char* (*last_error)(void);
} slate_hip_backend_t;

/* NULL when no gfx950 device can be opened (like the reference's stubs). */
const slate_backend_t* slate_backend_hip(void);                 /* replaces backend_cuda_stub.c:33 */
/* The same kernels behind host-visible memory, for callers that treat the
 * backend's memory as host memory (slate's toy engine memcpy's into its KV
 * cache and passes module weights from host memory, src/infer/engine.c:
 * 276-277, 411-412, 586-591): alloc returns pinned host memory the device
 * reads directly, compute entries copy pageable arguments through device
 * buffers and return after their kernel has finished.  Correct, slow; for
 * running slate_infer_engine_new_ex (infer.h:90-96) unchanged.  NULL
 * without a gfx950 device. */
const slate_backend_t* slate_backend_hip_compat(void);

/* ---- errors -------------------------------------------------------------- */
const char* slate_hip_last_error(void);  /* NULL when no error is pending */
void        slate_hip_clear_error(void);

/* ---- the vtable entries under stable names (backend.h:41-99) -------------- */
void* slate_hip_alloc(size_t bytes);                                          /* backend.h:45 */
void  slate_hip_release(void* dev);                                           /* backend.h:46 */
void  slate_hip_copy_h2d(void* dst_dev, const void* src_host, size_t bytes);  /* backend.h:49 */
void  slate_hip_copy_d2h(void* dst_host, const void* src_dev, size_t bytes);  /* backend.h:50 */
void  slate_hip_matvec(float* y, const float* A, const float* x, int M, int K);           /* backend.h:56 */
void  slate_hip_linear_batch(float* C, const float* X, const float* W, int B, int K, int N); /* backend.h:60-61 */
void  slate_hip_matvec_q4k(float* y, const void* A_q4k, const float* x, int M, int K);     /* backend.h:68 */
void  slate_hip_rmsnorm_row(float* y, const float* x, const float* w, int D, float eps);   /* backend.h:71-72 */
void  slate_hip_silu_mul(float* y, const float* gate, const float* up, int H);            /* backend.h:76 */
void  slate_hip_add_inplace(float* y, const float* x, int D);                             /* backend.h:79 */
void  slate_hip_embed_lookup(float* y, const float* W, int token_id, int D);              /* backend.h:82 */
void  slate_hip_attention_step(float* out, const float* q, const float* K_cache,
                               const float* V_cache, float* scores, int L, int D);        /* backend.h:91-93 */
void  slate_hip_sync(void);                                                               /* backend.h:96 */

/* ---- extensions (device pointers, enqueued on the backend stream) -------- */
int   slate_hip_matmul_q4k(float* Y, const void* A_q4k, const float* X, int B, int M, int K);
int   slate_hip_dequant_q4k(float* dst, const void* A_q4k, int64_t n);
/* Tiled Q4_K: the same blocks regrouped into 16-row tiles so that each
 * tile's block kb is 2304 contiguous bytes (16 headers, then the nibbles in
 * the order the matmul lanes read them); rows past M are zero.  It replaces
 * the row layout of quant.c:135-166 only in device memory owned by the
 * caller; the values and results are identical.  q4k_tile converts M rows
 * of K/256 blocks (device src, row layout) into dst of q4k_tiled_bytes. */
int64_t slate_hip_q4k_tiled_bytes(int M, int K);
int   slate_hip_q4k_tile(void* dst_tiled, const void* src_q4k, int M, int K);
int   slate_hip_matmul_q4k_tiled(float* Y, const void* A_tiled, const float* X, int B, int M, int K);
/* slate_hip_matmul_q4k that allocates nothing, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid it); no counterpart in slate.  Same inputs,
 * outputs and results; the activation operand and split-K partials live in
 * a fixed 32 MiB device array of the library, so calls whose operand plus
 * one split of partials ((16-row-padded B) * M * 4 bytes) exceed it return
 * -1 with an error naming the limit.  Calls are serialised on the backend
 * stream; work on that array from another stream (a replay of a captured
 * call next to new calls, say) would race with it. */
int   slate_hip_matmul_q4k_noalloc(float* Y, const void* A_q4k, const float* X, int B, int M, int K);
/* Q8_0 (34-byte blocks [f16 d][32 x int8], quant.h:16-31), device pointers.
 * q8_0_matvec has slate_q8_0_matvec's signature and meaning (quant.c:126-133,
 * y[m] = sum_k d*q[m,k] * x[k], K % 32 == 0); matmul_q8_0 is B such calls in
 * one launch (Y[B,M] = X[B,K] @ dequant(A)[M,K]^T); dequant_q8_0 is
 * slate_dequant_q8_0 (quant.c:12-25), bit-exact, n % 32 == 0.  Sums are in
 * another order than the reference's eight AVX2 lanes (float tolerance). */
void  slate_hip_q8_0_matvec(float* y, const void* A_q8, const float* x, int M, int K);  /* quant.h:31 */
int   slate_hip_matmul_q8_0(float* Y, const void* A_q8, const float* X, int B, int M, int K);
int   slate_hip_dequant_q8_0(float* dst, const void* A_q8, int64_t n);                   /* quant.h:24 */
/* Tiled Q8_0: the same bytes regrouped into 16-row x 256-element tiles of
 * 4352 bytes (the eight d of each row, then the int8 weights in the order
 * the matmul lanes read them); rows past M and blocks past K/32 are zero.
 * matmul_q8_0 regroups into backend scratch on every call; callers that
 * keep weights resident tile them once with q8_0_tile (device src, row
 * layout, into dst of q8_0_tiled_bytes) and call matmul_q8_0_tiled. */
int64_t slate_hip_q8_0_tiled_bytes(int M, int K);
int   slate_hip_q8_0_tile(void* dst_tiled, const void* src_q8, int M, int K);
int   slate_hip_matmul_q8_0_tiled(float* Y, const void* A_tiled, const float* X, int B, int M, int K);
int   slate_hip_rmsnorm_rows(float* y, const float* x, const float* w, int B, int D, float eps);
/* RoPE with the angles of llama_infer.c:83-86 (host powf/cosf/sinf table,
 * so identical inputs rotate bit-identically); rows with |pos| >= max_pos
 * are left unchanged and make the call return -1. */
int   slate_hip_rope_rows(float* x, const int32_t* pos, int n_rows, int n_heads, int head_dim,
                          float theta_base, int max_pos);
/* The host table behind rope_rows: cs[(p*hd/2 + i)*2 + {0,1}] = {cos, sin}. */
void  slate_hip_rope_table(float* cs, int max_pos, int head_dim, float theta_base);
int   slate_hip_argmax_rows(int32_t* out, const float* logits, int B, int V);

/* Ragged-batch packing on the device.  Inputs (device int32[B]): slot,
 * pos0 (positions already cached), n_new (>= 1 tokens this step).  Outputs
 * (device): tok_off[B+1] (exclusive prefix sum of n_new), tok2seq[T],
 * tok_pos[T], kv_base[B] (int64 float offset slot*slot_stride), last_tok[B].
 * Invalid descriptors (n_new < 1, pos0 + n_new > max_seq) are reported in
 * status[0] (0 ok, -1, -2) and produce no index writes. */
int   slate_hip_pack_batch(const int32_t* slot, const int32_t* pos0, const int32_t* n_new,
                           int B, int max_seq, int64_t slot_stride, int T_cap,
                           int32_t* tok_off, int32_t* tok2seq, int32_t* tok_pos,
                           int64_t* kv_base, int32_t* last_tok, int32_t* status);

/* Ragged GQA attention over per-sequence KV caches, split over key chunks.
 * q      : [T, n_q_heads*hd] post-RoPE queries, packed token-major
 * kv     : K and V pools; the cache of kv head h of the sequence that owns
 *          token t starts at kv_base[tok2seq[t]] + h*head_stride and holds
 *          [max_seq, hd] rows (key position-major)
 * token t attends to key positions 0..tok_pos[t] of its own sequence.
 * out    : [T, n_q_heads*hd].  scale = 1/sqrtf(hd) as llama_infer.c:104. */
int   slate_hip_attention_ragged(float* out, const float* q, const float* Kpool,
                                 const float* Vpool, const int32_t* tok2seq,
                                 const int32_t* tok_pos, const int64_t* kv_base,
                                 int T, int n_q_heads, int n_kv_heads, int head_dim,
                                 int64_t head_stride, int max_pos);

/* Synthetic weights generated on the device (seeded, ~N(0, std)):
 * f32 values, or rows x cols quantised to Q4_K. */
int   slate_hip_synth_f32(float* dst, int64_t n, uint64_t seed, float std);
int   slate_hip_synth_q4k(void* dst, int64_t rows, int64_t cols, uint64_t seed, float std);

/* ---- device-resident LLaMA engine ---------------------------------------- */
/* Mirrors slate_llama_config_t (llama.h:53-65). */
typedef struct slate_hip_llama_config {
    int   n_layers, d_model, ffn_hidden, n_heads, n_kv_heads, head_dim;
    int   max_seq, vocab;
    float theta_base, rms_eps;
    int   tied_output;
} slate_hip_llama_config_t;

/* Mirrors slate_llama_layer_t (llama.h:69-86): host pointers, dtypes are
 * slate_dtype_t values (0 = F32, 16 = Q8_0, 18 = Q4_K).  Unlike the
 * reference's mv_dispatch (llama_infer.c:43-51), which reads a Q8_0 tensor
 * as f32, Q8_0 linears run the Q8_0 matmul. */
typedef struct slate_hip_llama_layer {
    const void *attn_norm, *attn_q, *attn_k, *attn_v, *attn_output;
    const void *ffn_norm, *ffn_gate, *ffn_up, *ffn_down;
    int attn_q_dtype, attn_k_dtype, attn_v_dtype, attn_output_dtype;
    int ffn_gate_dtype, ffn_up_dtype, ffn_down_dtype;
} slate_hip_llama_layer_t;

typedef struct slate_hip_llama slate_hip_llama_t;
typedef struct slate_hip_llama_session slate_hip_llama_session_t;

/* Upload a model from host pointers (e.g. the mmap views slate_llama_open
 * resolves).  max_slots = concurrent sessions (KV slots); max_tokens = the
 * largest number of packed tokens one step may carry. */
slate_hip_llama_t* slate_hip_llama_new(const slate_hip_llama_config_t* cfg,
                                       const float* token_embd, const float* output_norm,
                                       const void* output, int output_dtype,
                                       const slate_hip_llama_layer_t* layers,
                                       int max_slots, int max_tokens);
/* Same engine with seeded synthetic weights generated on the device:
 * linears Q4_K (quant = 18), Q8_0 (quant = 16) or F32 (quant = 0),
 * embeddings f32, norms 1. */
slate_hip_llama_t* slate_hip_llama_new_synthetic(const slate_hip_llama_config_t* cfg,
                                                 uint64_t seed, int quant,
                                                 int max_slots, int max_tokens);
void  slate_hip_llama_free(slate_hip_llama_t* m);
/* The model's config (llama.h:98 slate_llama_config); NULL for NULL. */
const slate_hip_llama_config_t* slate_hip_llama_config(const slate_hip_llama_t* m);
/* Copy a weight tensor back to host ("token_embd", "output", "output_norm",
 * or "blk.N.<name>"); returns bytes written or a negative code. */
int64_t slate_hip_llama_get_tensor(const slate_hip_llama_t* m, const char* name,
                                   void* host_dst, int64_t cap, int* dtype);

/* llama.h:124-139 semantics, device-resident.  A session belongs to its
 * engine: free every session before slate_hip_llama_free (as a slate
 * session must not outlive its model). */
slate_hip_llama_session_t* slate_hip_llama_session_new(slate_hip_llama_t* m);
void  slate_hip_llama_session_free(slate_hip_llama_session_t* s);
int   slate_hip_llama_session_position(const slate_hip_llama_session_t* s);
/* Back to position 0 for a new conversation, keeping the KV slot
 * (slate_infer_session_reset, infer.h:116, engine.c:429-431). */
void  slate_hip_llama_session_reset(slate_hip_llama_session_t* s);
int   slate_hip_llama_prefill(slate_hip_llama_session_t* s, const int32_t* tokens,
                              int n_tokens, float* out_logits);
int   slate_hip_llama_decode_step(slate_hip_llama_session_t* s, int32_t token,
                                  float* out_logits);

/* One ragged continuous-batching step: sessions[i] contributes n_new[i]
 * tokens (tokens packed session-major in `tokens`).  For each session the
 * logits of its last new token go to out_logits[i*V..] (host, may be NULL)
 * and the greedy next token to out_next[i] (host, may be NULL).  Positions
 * advance by n_new[i].  Returns 0 or a negative code; on error no session
 * advances. */
int   slate_hip_llama_step(slate_hip_llama_t* m, slate_hip_llama_session_t** sessions,
                           int n, const int32_t* n_new, const int32_t* tokens,
                           float* out_logits, int32_t* out_next);
/* slate_infer_batch_step (engine.c:543-642) semantics: one token each. */
int   slate_hip_llama_batch_step(slate_hip_llama_t* m, slate_hip_llama_session_t** sessions,
                                 int n, const int32_t* tokens, float* out_logits);

/* KV cache of a session copied to host as [n_layers, max_seq, kv_dim] (the
 * reference session layout, llama_infer.c:57-58) for checking. */
int   slate_hip_llama_session_kv(const slate_hip_llama_session_t* s, float* K, float* V);

/* Kernel-class timing with HIP events recorded on the backend stream around
 * each launch: class 0 = Q4_K matmuls of decode shape (<= 16 rows),
 * 1 = attention in decode-only steps, 2 = decode-only steps, 3 = Q4_K
 * matmuls over more rows, 4 = attention in steps carrying prompt chunks,
 * 5 = steps carrying prompt chunks.
 * profile(m, 1) resets the totals and starts recording, profile(m, 2)
 * resumes recording without a reset, profile(m, 0) stops.  Kernel classes
 * are timed by events the dispatches record themselves (kernel start and
 * end).  Steps run while recording are launched one kernel at a time, not
 * from a graph.  profile_read returns the summed device milliseconds, the
 * summed algorithmic bytes (weights once, K/V once per kv head and sequence,
 * activations in and out) and the launch count of a class. */
int   slate_hip_llama_profile(slate_hip_llama_t* m, int enable);
/* graphs(m, 1) (or SLATE_HIP_GRAPHS=1): decode-only steps (one token per
 * session) are captured once per batch size into a HIP graph and replayed.
 * Default off: every kernel is launched separately.  Same results either
 * way.  Refused (-5, graphs stay off) while a rocprofiler tool is attached
 * (ROCPROF* / ROCP_* in the environment): a graph launch under
 * rocprofv3 --kernel-trace has ended in a crash inside the HIP runtime.
 * No slate counterpart (slate has no device graphs). */
int   slate_hip_llama_graphs(slate_hip_llama_t* m, int enable);
/* 1 when the engine keeps its K/V cache in f16 (opt-in at creation with
 * SLATE_HIP_KV_F16=1, head_dim 32/64/128), 0 for f32 as the reference
 * (llama_infer.c:57-58).  f16 halves the attention bytes; it rounds every
 * cached element to 11 bits, a numerics change measured against the parity
 * tolerance.  slate_hip_llama_session_kv returns f32 either way. */
int   slate_hip_llama_kv_f16(const slate_hip_llama_t* m);
/* 1 while the engine's decode steps merge the attention chunks inside the
 * decode attention kernel (workgroup i takes its work from queue i % 8, the
 * workgroups of a queue share one XCD, and the merging unit reads the
 * partials from that XCD's L2), 0 when they use the separate merge kernel:
 * shapes the in-kernel merge does not take, SLATE_HIP_ATTN_XCD=0, a device
 * where the placement probe failed, or after a merge found a partial
 * written on another XCD (the engine then runs that step again on the merge
 * kernel and keeps to it).  No slate counterpart. */
int   slate_hip_llama_attn_xcd_merge(const slate_hip_llama_t* m);
int   slate_hip_llama_profile_read(slate_hip_llama_t* m, int cls, double* ms, double* bytes,
                                   int64_t* launches);

/* The backend stream as a hipStream_t (for timing with events). */
void* slate_hip_stream(void);

#ifdef __cplusplus
}
#endif
#endif
