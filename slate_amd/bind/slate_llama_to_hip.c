/* slate_llama_to_hip.c -- the binding a slate maintainer adds next to
 * slate_llama_open (src/loader/llama.c:42-140): a LLaMA model opened by
 * slate's GGUF loader is uploaded into slate_amd's device engine.  The
 * engine's config and layer structs mirror llama.h:53-86 field for field;
 * the asserts below make the compiler check that before the memcpys. */
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#include "slate/llama.h"
#include "slate_hip.h"

#define SLATE_HIP_SAME(T1, T2, f) _Static_assert(offsetof(T1, f) == offsetof(T2, f), #T1 "." #f)
_Static_assert(sizeof(slate_hip_llama_config_t) == sizeof(slate_llama_config_t), "config size");
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, n_layers);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, d_model);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, ffn_hidden);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, n_heads);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, n_kv_heads);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, head_dim);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, max_seq);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, vocab);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, theta_base);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, rms_eps);
SLATE_HIP_SAME(slate_hip_llama_config_t, slate_llama_config_t, tied_output);
_Static_assert(sizeof(slate_hip_llama_layer_t) == sizeof(slate_llama_layer_t), "layer size");
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_norm);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_q);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_k);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_v);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_output);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, ffn_norm);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, ffn_gate);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, ffn_up);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, ffn_down);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_q_dtype);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_k_dtype);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_v_dtype);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, attn_output_dtype);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, ffn_gate_dtype);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, ffn_up_dtype);
SLATE_HIP_SAME(slate_hip_llama_layer_t, slate_llama_layer_t, ffn_down_dtype);

slate_hip_llama_t* slate_llama_to_hip(const slate_llama_t* m, int max_slots, int max_tokens) {
    const slate_llama_config_t* c = slate_llama_config(m);                      /* llama.h:98 */
    /* the engine reads f32 token embeddings, as llama_infer.c:149-150 does
     * (a tied LM head is then f32 too: llama.c:94-101) */
    if (!c || slate_llama_token_embd_dtype(m) != SLATE_DTYPE_F32) return NULL;
    slate_hip_llama_config_t hc;
    memcpy(&hc, c, sizeof hc);
    slate_hip_llama_layer_t* L = (slate_hip_llama_layer_t*)malloc(sizeof *L * (size_t)c->n_layers);
    if (!L) return NULL;
    for (int i = 0; i < c->n_layers; ++i)
        memcpy(&L[i], slate_llama_layer(m, i), sizeof L[i]);                    /* llama.h:104 */
    slate_hip_llama_t* h = slate_hip_llama_new(&hc, (const float*)slate_llama_token_embd(m),   /* llama.h:99 */
                                               (const float*)slate_llama_output_norm(m),       /* llama.h:101 */
                                               slate_llama_output(m), slate_llama_output_dtype(m),
                                               L, max_slots, max_tokens);
    free(L);
    return h;   /* weights copied to HBM: the gguf may be closed afterwards */
}
