// infer_shim.cpp -- slate's inference-engine API (include/slate/infer.h:57-187)
// over the device-resident LLaMA engine, so that callers written against
// slate_infer_* -- the scheduler's decoder thread (src/server/scheduler.c:
// 45-99) and the HTTP workers' prefill (src/server/http.c) -- run a LLaMA
// model on the GPU unchanged.  Built as its own library
// (libslate_hip_infer.so) that a maintainer links in place of
// src/infer/engine.c; the only new entry is the constructor
// slate_hip_infer_engine_new (include/slate_hip_infer.h), since slate's own
// constructors take a slate_module_t (infer.h:74-96).
//
// Semantics kept from src/infer/engine.c: sessions are per conversation
// and not shareable (infer.h:42-45); prefill returns the last prompt
// token's logits (infer.h:124-129); batch_step advances each of
// n in [1, max_batch] sessions by one token and writes logits[i * vocab]
// (engine.c:543-642), returning -1 on bad arguments, -2 when a session is
// full and -3 on a bad token, as engine.c:549-559 does.  The engine is
// shareable across threads: calls are serialised inside the HIP engine.
#include <stdlib.h>

#include <new>
#include <vector>

#include "../../include/slate_hip.h"
#include "../../include/slate_hip_infer.h"

struct slate_infer_engine {
    slate_hip_llama_t* m;
    int vocab, max_seq;
};

struct slate_infer_session {
    slate_infer_engine* eng;
    slate_hip_llama_session_t* s;
};

struct slate_infer_batch {
    slate_infer_engine* eng;
    int max_batch;
    std::vector<slate_hip_llama_session_t*> hs;   // per-step translation of the session handles
};

extern "C" {

slate_infer_engine_t* slate_hip_infer_engine_new(slate_hip_llama_t* model) {
    const slate_hip_llama_config_t* c = slate_hip_llama_config(model);
    if (!c) return nullptr;
    return new (std::nothrow) slate_infer_engine{model, c->vocab, c->max_seq};
}

void slate_infer_engine_free(slate_infer_engine_t* eng) { delete eng; }                     // infer.h:98

int slate_infer_engine_vocab(const slate_infer_engine_t* eng) { return eng ? eng->vocab : 0; }       // infer.h:102
int slate_infer_engine_max_seq(const slate_infer_engine_t* eng) { return eng ? eng->max_seq : 0; }   // infer.h:105

slate_infer_session_t* slate_infer_session_new(slate_infer_engine_t* eng) {                 // infer.h:110
    if (!eng) return nullptr;
    slate_hip_llama_session_t* s = slate_hip_llama_session_new(eng->m);
    if (!s) return nullptr;
    auto* r = new (std::nothrow) slate_infer_session{eng, s};
    if (!r) slate_hip_llama_session_free(s);
    return r;
}

void slate_infer_session_free(slate_infer_session_t* sess) {                                // infer.h:112
    if (!sess) return;
    slate_hip_llama_session_free(sess->s);
    delete sess;
}

void slate_infer_session_reset(slate_infer_session_t* sess) {                               // infer.h:116
    if (sess) slate_hip_llama_session_reset(sess->s);
}

int slate_infer_session_position(const slate_infer_session_t* sess) {                      // infer.h:119
    return sess ? slate_hip_llama_session_position(sess->s) : -1;
}

int slate_infer_prefill(slate_infer_session_t* sess, const int32_t* tokens, int n_tokens,   // infer.h:130-132
                        float* out_logits) {
    if (!sess || !tokens || !out_logits || n_tokens <= 0) return -1;
    return slate_hip_llama_prefill(sess->s, tokens, n_tokens, out_logits);
}

int slate_infer_decode_step(slate_infer_session_t* sess, int32_t token, float* out_logits) {  // infer.h:137-139
    if (!sess || !out_logits) return -1;
    return slate_hip_llama_decode_step(sess->s, token, out_logits);
}

slate_infer_batch_t* slate_infer_batch_new(slate_infer_engine_t* eng, int max_batch) {     // infer.h:170-171
    if (!eng || max_batch <= 0) return nullptr;
    auto* b = new (std::nothrow) slate_infer_batch{eng, max_batch, {}};
    if (!b) return nullptr;
    b->hs.resize((size_t)max_batch);
    return b;
}

void slate_infer_batch_free(slate_infer_batch_t* batch) { delete batch; }                   // infer.h:173

int slate_infer_batch_step(slate_infer_batch_t* batch, slate_infer_session_t** sessions,   // infer.h:183-187
                           int n_sessions, const int32_t* tokens, float* out_logits) {
    if (!batch || !sessions || !tokens || !out_logits) return -1;
    if (n_sessions < 1 || n_sessions > batch->max_batch) return -1;
    for (int i = 0; i < n_sessions; ++i) {
        if (!sessions[i] || sessions[i]->eng != batch->eng) return -1;
        batch->hs[(size_t)i] = sessions[i]->s;
    }
    return slate_hip_llama_batch_step(batch->eng->m, batch->hs.data(), n_sessions, tokens, out_logits);
}

}  // extern "C"
