/*
 * slate_hip_infer.h -- constructor of libslate_hip_infer.so, the library
 * that implements slate's inference-engine API (include/slate/infer.h:
 * 57-187: slate_infer_engine_vocab / _max_seq / _free, slate_infer_session_new
 * / _free / _reset / _position, slate_infer_prefill, slate_infer_decode_step,
 * slate_infer_batch_new / _free / _step) over the device LLaMA engine of
 * slate_hip.h.  Callers written against infer.h -- slate's scheduler
 * (src/server/scheduler.c) and HTTP server -- link this library in place of
 * src/infer/engine.c and run unchanged; only the engine's construction
 * differs, because slate's constructors take a slate_module_t
 * (infer.h:74-96) and this engine runs a LLaMA model.
 *
 * Limits: a batch step takes at most the HIP engine's max_slots sessions
 * (more returns -1, like n > max_batch in engine.c:549); sessions are KV
 * slots of the HIP engine, so slate_infer_session_new returns NULL once
 * max_slots are open.
 */
#ifndef SLATE_HIP_INFER_H
#define SLATE_HIP_INFER_H

#include "slate_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The same opaque types as include/slate/infer.h:57-58, 168. */
typedef struct slate_infer_engine slate_infer_engine_t;
typedef struct slate_infer_session slate_infer_session_t;
typedef struct slate_infer_batch slate_infer_batch_t;

/* An engine over a device LLaMA model (borrowed: free the infer engine,
 * its sessions and batches before slate_hip_llama_free); vocab and max_seq
 * come from the model's config.  Replaces slate_infer_engine_new / _new_ex
 * (infer.h:74-96).  NULL for a NULL model. */
slate_infer_engine_t* slate_hip_infer_engine_new(slate_hip_llama_t* model);

#ifdef __cplusplus
}
#endif
#endif
