/*
 * ref_harness.c -- test infrastructure: compiles slate's own
 * src/loader/llama_infer.c into this translation unit (from the slate tree,
 * via the include path the Makefile passes) so that its file-static helpers
 * and the session struct can be reached from the checker.  The output lands
 * in oracle/_ref/ and is never shipped or linked by the product.
 */
#include "src/loader/llama_infer.c"
#include "slate/runtime.h"

/* llama_infer.c:77-92 */
void ref_rope_inplace_row(float* row, int n_heads, int head_dim, int position,
                          float theta_base) {
    rope_inplace_row(row, n_heads, head_dim, position, theta_base);
}

/* llama_infer.c:97-129 */
void ref_attention_multihead(float* out, const float* q, const float* K,
                             const float* V, float* scores, int L, int n_q_heads,
                             int n_kv_heads, int head_dim) {
    attention_multihead(out, q, K, V, scores, L, n_q_heads, n_kv_heads, head_dim);
}

/* Load a KV state into a session (struct at llama_infer.c:53-71) so that a
 * decode window can be timed from a given context without replaying the
 * token-serial prefill.  K/V are [n_layers, max_seq, kv_dim]. */
int ref_session_set_state(slate_llama_session_t* s, const float* K, const float* V,
                          int position) {
    if (!s) return -1;
    const slate_llama_config_t* c = slate_llama_config(s->model);
    size_t n = (size_t)c->n_layers * c->max_seq * c->n_kv_heads * c->head_dim;
    if (position < 0 || position > c->max_seq) return -1;
    if (K) memcpy(s->K_cache, K, n * sizeof(float));
    if (V) memcpy(s->V_cache, V, n * sizeof(float));
    s->position = position;
    return 0;
}

/* Read back a session's KV cache. */
int ref_session_get_kv(const slate_llama_session_t* s, float* K, float* V) {
    if (!s) return -1;
    const slate_llama_config_t* c = slate_llama_config(s->model);
    size_t n = (size_t)c->n_layers * c->max_seq * c->n_kv_heads * c->head_dim;
    memcpy(K, s->K_cache, n * sizeof(float));
    memcpy(V, s->V_cache, n * sizeof(float));
    return 0;
}

/* Harness-level parallelism, not wired in slate's LLaMA path (which decodes
 * one session at a time on one thread): one decode step for each of n
 * sessions, the sessions spread over slate's own global threadpool
 * (slate_threadpool_parallel_for, threadpool.c:122-142; its size comes from
 * SLATE_NUM_THREADS or the online CPU count, pool_global.c:18-25).  Logits
 * of session i go to logits[i * vocab ..]; rc[i] is its return code. */
typedef struct {
    slate_llama_session_t** s;
    const int32_t* tok;
    float* logits;
    int vocab;
    int* rc;
} ref_par_job;

static void ref_par_task(int i, int n, void* u) {
    (void)n;
    ref_par_job* j = (ref_par_job*)u;
    j->rc[i] = slate_llama_decode_step(j->s[i], j->tok[i], j->logits + (size_t)i * j->vocab);
}

void ref_decode_sessions_parallel(slate_llama_session_t** s, const int32_t* tok, int n, float* logits,
                                  int* rc) {
    if (!s || n <= 0) return;
    ref_par_job j = {s, tok, logits, slate_llama_config(s[0]->model)->vocab, rc};
    slate_threadpool_parallel_for(slate_global_pool(), n, ref_par_task, &j);
}

int ref_pool_threads(void) { return slate_threadpool_num_threads(slate_global_pool()); }
