/* backend_default_hip.c -- slate's default backend chooser with the HIP
 * backend first: it replaces slate_backend_default in
 * src/backend/backend_cpu.c:189-194.  slate_backend_hip_compat() takes the
 * host pointers slate's callers of the default hand over (llama_infer.c:218
 * passes mmap'd weights and calloc'd buffers; the toy engine, engine.c:318,
 * memcpy's into what alloc returns); it is NULL without a gfx950 GPU, and
 * the chooser then falls through to slate's own order. */
#include "slate/backend.h"
#include "slate_hip.h"

const slate_backend_t* slate_backend_default(void) {
    const slate_backend_t* b;
    if ((b = slate_backend_hip_compat()) != NULL) return b;
    if ((b = slate_backend_cuda())  != NULL) return b;
    if ((b = slate_backend_metal()) != NULL) return b;
    return slate_backend_cpu();
}
