// engine.cpp -- device-resident LLaMA engine with a ragged continuous-batching
// step.  Per-token semantics are those of decode_one (llama_infer.c:134-206);
// the batched step generalises slate_infer_batch_step (engine.c:543-642) to
// LLaMA and to sequences contributing several tokens in one step (prefill
// chunks mixed with decode rows).
//
// HBM layout:
//   weights       Q4_K in the TILED layout (16-row tiles, each tile's
//                 super-block 2304 contiguous bytes; repacked once at load),
//                 Q8_0 in its TILED layout (16-row tiles x 256-element
//                 groups of 4352 bytes), f32 as given [out, in]
//   K/V pools     [slot][layer][kv_head][max_seq][head_dim] f32
//   RoPE table    [max_seq][head_dim/2][2] f32 (host-computed angles)
//   activations   [T][...] f32, packed token-major; split-K partials
//                 [split][T_pad][width]
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "launch.h"

namespace slate_hip {
extern std::mutex g_enqueue_mu;
}
using namespace slate_hip;

namespace {

constexpr int DT_F32 = 0;
constexpr int DT_Q8_0 = 16;
constexpr int DT_Q4K = 18;

struct Lin {
    void* w = nullptr;       // Q4_K, Q8_0: TILED layouts
    int dtype = DT_F32;
    int M = 0, K = 0;
    // bytes of the tensor in slate's own layout (the algorithmic weight bytes)
    size_t bytes() const {
        if (dtype == DT_Q4K) return (size_t)M * (K / QK) * QBLOCK;
        if (dtype == DT_Q8_0) return (size_t)M * (K / Q8_ELEMS) * Q8_BYTES;
        return (size_t)M * K * sizeof(float);
    }
    size_t dev_bytes() const {
        if (dtype == DT_Q4K) return q4k_tiled_bytes(M, K);
        if (dtype == DT_Q8_0) return q8_tiled_bytes(M, K);
        return bytes();
    }
};

struct LayerDev {
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    Lin q, k, v, o, gate, up, down;
};

}  // namespace

struct slate_hip_llama {
    slate_hip_llama_config_t cfg{};
    int max_slots = 0, max_tokens = 0, tpad_cap = 0;
    float* tok_embd = nullptr;
    float* out_norm = nullptr;
    Lin out;
    std::vector<LayerDev> L;
    void *Kpool = nullptr, *Vpool = nullptr;   // f32, or f16 when kv_f16
    bool kv_f16 = false;
    int kv_bytes = 4;
    int64_t slot_stride = 0, layer_stride = 0, head_stride = 0;
    float* rope_cs = nullptr;
    float *x = nullptr, *xn = nullptr, *q = nullptr, *att = nullptr, *h = nullptr;
    float *xlast = nullptr, *logits = nullptr;
    float* part = nullptr;
    size_t part_floats = 0;
    float* ssq = nullptr;          // [T_pad][D/256] block sums of squares (deferred RMSNorm)
    bool defer_norm = true;
    bool tokenwise_attn = false;   // prompt-chunk tokens through the decode attention kernel
    bool prompt_mfma = false;      // prompt-chunk blocks may go to the MFMA prompt attention kernel
    bool step_prompt_mfma = false; // ... and do in the step being enqueued
    float *att_po = nullptr, *att_pml = nullptr;
    int32_t* att_xcd = nullptr;     // per-XCD decode attention queues (attention_xcd_view)
    Act16 act{};
    Act8 act8{};                   // allocated with the first Q8_0 linear
    int32_t *d_desc = nullptr, *d_tok = nullptr, *tok_off = nullptr, *tok2seq = nullptr, *tok_pos = nullptr,
            *last_tok = nullptr, *status = nullptr, *next = nullptr;
    int64_t* kv_base = nullptr;
    void* argmax_ws = nullptr;     // (value, index) per row and chunk of the greedy argmax
    // Per-step host input, uploaded in one copy: [slot|pos0|n_new (max_slots
    // each)] [tokens (T)] [decode query blocks (n_dec)] [prefill block first
    // tokens (n_pre)] [prefill block sizes (n_pre)]; d_desc mirrors it.
    int32_t *h_desc = nullptr, *h_tok = nullptr, *h_next = nullptr, *h_status = nullptr;
    int n_dec = 0, n_pre = 0;
    bool step_mixed = false;       // the step carries a prompt chunk (profiling classes)
    bool step_one_each = false;    // every sequence of the step adds exactly one token
    Knobs knobs;                   // kernel-path switches, read at creation (every step runs under them)
    // The decode attention's in-kernel merge is turned off for this engine
    // once a merge found a partial written on another XCD.
    std::atomic<bool> xcd_off{false};
    float* h_logits = nullptr;
    std::vector<int> free_slots;
    std::vector<void*> allocs;
    std::mutex mu;
    // Optional event timing of kernel classes (slate_hip_llama_profile).
    struct ProfRec { int cls; double bytes; size_t e0, e1; };
    bool prof_on = false;
    std::vector<hipEvent_t> prof_ev;
    size_t prof_used = 0;
    std::vector<ProfRec> prof_recs;
    static constexpr int NPROF = 6;
    double prof_ms[NPROF] = {}, prof_bytes[NPROF] = {};
    int64_t prof_n[NPROF] = {};
    double step_kv_rows = 0;     // sum over sequences of positions attended this step
    // Graphs of decode-only steps, one per (batch size, logits wanted).
    struct StepGraph { int n; bool want; hipGraphExec_t exec; };
    bool graphs_on = false;
    std::vector<StepGraph> graphs;
};

struct slate_hip_llama_session {
    slate_hip_llama* m;
    int slot;
    int pos;
};

namespace {

template <class T>
int dalloc(slate_hip_llama* m, T** p, size_t count) {
    *p = nullptr;
    if (count == 0) count = 1;
    void* v = nullptr;
    if (hipMalloc(&v, count * sizeof(T)) != hipSuccess) {
        set_error(-2, "engine: device allocation of %zu bytes failed", count * sizeof(T));
        return -2;
    }
    m->allocs.push_back(v);
    *p = (T*)v;
    return 0;
}

void free_model(slate_hip_llama* m) {
    if (!m) return;
    (void)hipStreamSynchronize(stream());
    for (void* p : m->allocs) (void)hipFree(p);
    if (m->h_desc) (void)hipHostFree(m->h_desc);
    if (m->h_next) (void)hipHostFree(m->h_next);
    if (m->h_status) (void)hipHostFree(m->h_status);
    if (m->h_logits) (void)hipHostFree(m->h_logits);
    delete m;
}

bool valid_cfg(const slate_hip_llama_config_t* c) {
    return c && c->n_layers > 0 && c->d_model > 0 && c->ffn_hidden > 0 && c->n_heads > 0 && c->n_kv_heads > 0 &&
           c->n_heads % c->n_kv_heads == 0 && c->head_dim > 0 && c->head_dim % 2 == 0 &&
           c->n_heads * c->head_dim == c->d_model && c->max_seq > 0 && c->vocab > 0;
}

// Whether a rocprofiler tool is attached to the process (rocprofv3 passes
// its options as ROCPROF* / ROCP_* variables).  Graph replay stays off then:
// a graph launch under rocprofv3 --kernel-trace has ended in a crash inside
// the HIP runtime, with no cause found in this library.
bool tracer_attached() {
    for (char** e = environ; e && *e; ++e)
        if (strncmp(*e, "ROCPROF", 7) == 0 || strncmp(*e, "ROCP_", 5) == 0) return true;
    return false;
}

// Allocate everything but the weights.
int alloc_runtime(slate_hip_llama* m) {
    const auto& c = m->cfg;
    const int D = c.d_model, H = c.ffn_hidden, kvd = c.n_kv_heads * c.head_dim;
    m->tpad_cap = row_pad(m->max_tokens);
    m->head_stride = (int64_t)c.max_seq * c.head_dim;
    m->layer_stride = (int64_t)c.n_kv_heads * m->head_stride;
    m->slot_stride = (int64_t)c.n_layers * m->layer_stride;
    size_t kv = (size_t)m->max_slots * m->slot_stride;
    // f16 K/V (opt-in, SLATE_HIP_KV_F16=1): half the attention bytes; the
    // reference caches f32 (llama_infer.c:57-58)
    m->kv_f16 = (c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128) && getenv("SLATE_HIP_KV_F16") != nullptr &&
                atoi(getenv("SLATE_HIP_KV_F16")) != 0;
    m->kv_bytes = m->kv_f16 ? 2 : 4;
    {
        char *kp = nullptr, *vp = nullptr;
        if (dalloc(m, &kp, kv * m->kv_bytes) || dalloc(m, &vp, kv * m->kv_bytes)) return -2;
        m->Kpool = kp;
        m->Vpool = vp;
    }
    // RoPE table with the reference's float angle expressions.
    {
        std::vector<float> cs((size_t)c.max_seq * c.head_dim);
        build_rope_table(cs.data(), c.max_seq, c.head_dim, c.theta_base);
        if (dalloc(m, &m->rope_cs, cs.size())) return -2;
        if (hipMemcpy(m->rope_cs, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
            set_error(-7, "engine: rope table upload failed");
            return -7;
        }
    }
    const size_t T = m->tpad_cap;
    if (dalloc(m, &m->x, T * D) || dalloc(m, &m->xn, T * D) || dalloc(m, &m->q, T * D) ||
        dalloc(m, &m->att, T * D) || dalloc(m, &m->h, T * H) || dalloc(m, &m->xlast, (size_t)m->max_slots * D) ||
        // the LM-head matmul writes whole 16-row tiles
        dalloc(m, &m->logits, (size_t)row_pad(m->max_slots) * c.vocab) ||
        dalloc(m, (char**)&m->argmax_ws, argmax_workspace_bytes(m->max_slots, c.vocab)))
        return -2;
    const int W = std::max({D + 2 * kvd, 2 * H, D});
    m->part_floats = (size_t)std::max<size_t>(16 * 64, T) * W;
    if (dalloc(m, &m->part, m->part_floats)) return -2;
    size_t np = attention_partial_floats((int)T, c.n_heads, c.head_dim, c.max_seq);
    if (dalloc(m, &m->att_po, np)) return -2;
    m->att_pml = m->att_po + (size_t)T * c.n_heads * ((c.max_seq + attn_chunk_size() - 1) / attn_chunk_size()) *
                                 c.head_dim;
    // decode steps (one token per sequence, at most max_slots rows) merge
    // the attention chunks inside the attention kernel from per-XCD queues
    if (dalloc(m, &m->att_xcd, attention_xcd_ints(m->max_slots, c.n_kv_heads, c.max_seq))) return -2;
    if (hipMemset(m->att_xcd, 0, attention_xcd_ints(m->max_slots, c.n_kv_heads, c.max_seq) * 4) != hipSuccess) {
        set_error(-7, "engine: attention queue clear failed");
        return -7;
    }
    attention_xcd_probe();
    // Q4_K activation operand for the widest matmul input (max(D, H)), T_pad rows
    const int Kmax = std::max(D, H);
    char* fr = nullptr;
    if (dalloc(m, &fr, act_frag_bytes((int)T, Kmax))) return -2;
    m->act = Act16{fr, 0, (int)T, Kmax};
    if (dalloc(m, &m->ssq, T * (D / QK + 1))) return -2;
    m->defer_norm = getenv("SLATE_HIP_FUSED_NORM") == nullptr || atoi(getenv("SLATE_HIP_FUSED_NORM")) != 0;
    // opt-in: at 8B shapes a decode step is not launch-bound (graph replay
    // measured 3.37 ms per B=16 step against 3.35 ms launched eagerly)
    m->graphs_on = getenv("SLATE_HIP_GRAPHS") != nullptr && atoi(getenv("SLATE_HIP_GRAPHS")) != 0 &&
                   !tracer_attached();
    // prompt-chunk tokens attend through the decode kernel (one query token
    // per work unit, whole coalesced K/V rows; the shared prefix re-reads
    // hit L2), which beats the query-block kernel for these head sizes; the
    // MFMA prompt kernel, where it covers the shape, takes them in steps where
    // it pays (prompt_mfma_pays)
    m->prompt_mfma = attention_prompt_mfma(c.n_heads, c.n_kv_heads, c.head_dim, m->kv_f16);
    m->tokenwise_attn = (c.head_dim == 32 || c.head_dim == 64 || c.head_dim == 128) &&
                        (m->kv_f16 || getenv("SLATE_HIP_ATTN_TOKENWISE") == nullptr ||
                         atoi(getenv("SLATE_HIP_ATTN_TOKENWISE")) != 0);
    const int S = m->max_slots;
    const size_t in_ints = 3 * (size_t)S + 4 * T;
    if (dalloc(m, &m->d_desc, in_ints) || dalloc(m, &m->tok_off, S + 1) ||
        dalloc(m, &m->tok2seq, T) || dalloc(m, &m->tok_pos, T) || dalloc(m, &m->last_tok, S) ||
        dalloc(m, &m->kv_base, S))
        return -2;
    m->d_tok = m->d_desc + 3 * S;
    // index buffers start as valid (all-zero) indices
    if (hipMemset(m->tok2seq, 0, T * 4) != hipSuccess || hipMemset(m->tok_pos, 0, T * 4) != hipSuccess ||
        hipMemset(m->kv_base, 0, S * 8) != hipSuccess || hipMemset(m->last_tok, 0, S * 4) != hipSuccess) {
        set_error(-7, "engine: index clear failed");
        return -7;
    }
    if (hipHostMalloc((void**)&m->h_desc, sizeof(int32_t) * in_ints) != hipSuccess ||
        hipHostMalloc((void**)&m->h_next, sizeof(int32_t) * S) != hipSuccess ||
        hipHostMalloc((void**)&m->h_status, sizeof(int32_t) * 4) != hipSuccess ||
        hipHostMalloc((void**)&m->h_logits, sizeof(float) * (size_t)S * c.vocab) != hipSuccess) {
        set_error(-2, "engine: pinned host allocation failed");
        return -2;
    }
    m->h_tok = m->h_desc + 3 * S;
    // the packing status and the next-token ids are written by the kernels
    // straight into pinned host memory: no device-to-host copies per step
    if (hipHostGetDevicePointer((void**)&m->status, m->h_status, 0) != hipSuccess ||
        hipHostGetDevicePointer((void**)&m->next, m->h_next, 0) != hipSuccess) {
        set_error(-7, "engine: pinned host buffers are not device-accessible");
        return -7;
    }
    // KV pools start zeroed, like calloc in llama_infer.c:225-226
    if (hipMemset(m->Kpool, 0, kv * m->kv_bytes) != hipSuccess ||
        hipMemset(m->Vpool, 0, kv * m->kv_bytes) != hipSuccess) {
        set_error(-7, "engine: KV clear failed");
        return -7;
    }
    // the clears and uploads above run outside the backend stream: finish them
    if (hipDeviceSynchronize() != hipSuccess) {
        set_error(-7, "engine: device synchronisation failed");
        return -7;
    }
    for (int i = S - 1; i >= 0; --i) m->free_slots.push_back(i);
    return 0;
}

int upload(slate_hip_llama* m, void** dst, const void* src, size_t bytes) {
    if (!src) {
        set_error(-1, "engine: missing weight pointer");
        return -1;
    }
    char* p;
    if (dalloc(m, &p, bytes)) return -2;
    if (hipMemcpy(p, src, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        set_error(-7, "engine: weight upload failed");
        return -7;
    }
    *dst = p;
    return 0;
}

// Staging buffer for weights in slate's row layout on their way to the
// TILED layout (grown on demand, released after loading).
struct RowStage {
    void* p = nullptr;
    size_t n = 0;
    void* get(size_t bytes) {
        if (bytes <= n) return p;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            set_error(-2, "engine: staging allocation of %zu bytes failed", bytes);
            return nullptr;
        }
        n = bytes;
        return p;
    }
    ~RowStage() {
        if (p) {
            (void)hipStreamSynchronize(stream());
            (void)hipFree(p);
        }
    }
};

// The Q8_0 activation operand for the widest matmul input, T_pad rows.
int ensure_act8(slate_hip_llama* m) {
    if (m->act8.frag) return 0;
    const int Kmax = std::max(m->cfg.d_model, m->cfg.ffn_hidden);
    char* fr = nullptr;
    if (dalloc(m, &fr, act8_bytes(m->tpad_cap, Kmax))) return -2;
    m->act8 = Act8{fr, 0, m->tpad_cap, Kmax};
    return 0;
}

// Repack a Q4_K or Q8_0 tensor staged in row layout into l.w (TILED).
int tile_lin(slate_hip_llama* m, Lin& l, const void* row_dev) {
    char* p;
    if (l.dtype == DT_Q8_0 && ensure_act8(m)) return -2;
    if (dalloc(m, &p, l.dev_bytes())) return -2;
    l.w = p;
    if (l.dtype == DT_Q8_0) return launch_q8_tile(p, row_dev, l.M, l.K, stream());
    return launch_q4k_tile(p, row_dev, l.M, l.K, stream());
}

int set_lin(slate_hip_llama* m, Lin& l, const void* host, int dtype, int M, int K, RowStage& st) {
    l.M = M;
    l.K = K;
    l.dtype = dtype;
    // the dispatch of llama_infer.c:43-51, with Q8_0 routed to its own
    // matmul (the reference reads a dtype-16 tensor as f32)
    if (dtype != DT_F32 && dtype != DT_Q4K && dtype != DT_Q8_0) {
        set_error(-5, "engine: weight dtype %d not supported (f32=0, q8_0=16, q4_k=18)", dtype);
        return -5;
    }
    if (dtype == DT_Q4K && K % QK) {
        set_error(-1, "engine: Q4_K weight with K=%d (not a multiple of 256)", K);
        return -1;
    }
    if (dtype == DT_Q8_0 && K % Q8_ELEMS) {
        set_error(-1, "engine: Q8_0 weight with K=%d (not a multiple of 32)", K);
        return -1;
    }
    if (dtype == DT_F32) return upload(m, &l.w, host, l.bytes());
    if (!host) {
        set_error(-1, "engine: missing weight pointer");
        return -1;
    }
    // the stream may still be repacking the previous tensor out of the stage
    if (hipStreamSynchronize(stream()) != hipSuccess) {
        set_error(-7, "engine: weight repack failed");
        return -7;
    }
    void* row = st.get(l.bytes());
    if (!row) return -2;
    if (hipMemcpy(row, host, l.bytes(), hipMemcpyHostToDevice) != hipSuccess) {
        set_error(-7, "engine: weight upload failed");
        return -7;
    }
    return tile_lin(m, l, row);
}

// Profiling: event pairs around launches of a kernel class (see the header)
// with the launch's algorithmic bytes; folded into the totals after the
// step's sync.  Kernel classes get events recorded by the dispatches
// themselves (prof_event + SH_LAUNCH), steps get stream events (prof_mark).
size_t prof_event(slate_hip_llama* m) {
    if (m->prof_used == m->prof_ev.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return (size_t)-1;
        m->prof_ev.push_back(e);
    }
    return m->prof_used++;
}

hipEvent_t prof_ev(slate_hip_llama* m, size_t i) { return i == (size_t)-1 ? nullptr : m->prof_ev[i]; }

size_t prof_mark(slate_hip_llama* m, hipStream_t s) {
    size_t i = prof_event(m);
    if (i == (size_t)-1) return i;
    if (hipEventRecord(m->prof_ev[i], s) != hipSuccess) return (size_t)-1;
    return i;
}

void prof_collect(slate_hip_llama* m) {
    for (const auto& r : m->prof_recs) {
        float ms = 0.f;
        if (r.e0 == (size_t)-1 || r.e1 == (size_t)-1) continue;
        if (hipEventElapsedTime(&ms, m->prof_ev[r.e0], m->prof_ev[r.e1]) != hipSuccess) continue;
        m->prof_ms[r.cls] += ms;
        m->prof_bytes[r.cls] += r.bytes;
        m->prof_n[r.cls] += 1;
    }
    m->prof_recs.clear();
    m->prof_used = 0;
}

// What a matmul group reads: the Q4_K activation operand and/or f32 rows
// (f32 linears read them directly, Q8_0 linears through their own operand
// built from them).
struct GroupIn {
    bool q4 = false, q8 = false, f32 = false;
    bool rows() const { return q8 || f32; }
};
GroupIn group_in(const Lin* const* lins, int nl) {
    GroupIn g;
    for (int i = 0; i < nl; ++i) (lins[i]->dtype == DT_Q4K ? g.q4 : (lins[i]->dtype == DT_Q8_0 ? g.q8 : g.f32)) = true;
    return g;
}

// The engine's operand buffer viewed for T rows of width K.
Act16 act_for(slate_hip_llama* m, int T, int K) {
    Act16 a = m->act;
    a.rows = T;
    a.rows_pad = row_pad(T);
    a.K = K;
    return a;
}

// RMSNorm whose row factor is applied by the consumer of the group's matmul
// (residual_act + RowNorm): only for all-Q4_K groups of width % 256 == 0.
bool defer_norm(const slate_hip_llama* m, const GroupIn& gi, int D) {
    return m->defer_norm && gi.q4 && !gi.rows() && D % QK == 0;
}

// One matmul group: the linears in `lins` read the same input (operand `a`
// for Q4_K, rows X [T, K] for f32 and Q8_0) and write column ranges of one
// partial buffer [S][T_pad][ldo]; *S_out = S.  Q8_0 linears write the split
// count the Q4_K ones chose, f32 linears force one split.
int mm_group(slate_hip_llama* m, const Act16* a, const float* X, int T, int K, const Lin* const* lins,
             const int64_t* col, int nl, int64_t ldo, int* S_out, hipStream_t s) {
    const GroupIn gi = group_in(lins, nl);
    const int tpad = row_pad(T);
    const int64_t ss = (int64_t)tpad * ldo;
    // an f32 linear writes one partial, so a group with one stays unsplit
    int max_splits = gi.f32 ? 1 : (int)std::min<size_t>(64, m->part_floats / ((size_t)tpad * ldo));
    int S = 1;
    if (gi.q4) {
        Q4kTarget t[3];
        int nq = 0;
        double bytes = 4.0 * T * K;
        for (int i = 0; i < nl; ++i)
            if (lins[i]->dtype == DT_Q4K) {
                t[nq++] = Q4kTarget{lins[i]->w, lins[i]->M, col[i]};
                bytes += (double)lins[i]->bytes() + 4.0 * T * lins[i]->M;
            }
        const size_t e0 = m->prof_on ? prof_event(m) : (size_t)-1, e1 = m->prof_on ? prof_event(m) : (size_t)-1;
        int rc = launch_q4k(t, nq, true, *a, m->part, ldo, ss, max_splits, &S, s, prof_ev(m, e0), prof_ev(m, e1));
        if (rc) return rc;
        if (m->prof_on) m->prof_recs.push_back({tpad == 16 ? 0 : 3, bytes, e0, e1});
    }
    if (gi.q8) {
        Act8 a8 = m->act8;
        a8.rows = T;
        a8.rows_pad = tpad;
        a8.K = K;
        int rc = launch_act8_from_f32(a8, X, K, s);
        if (rc) return rc;
        Q4kTarget t[3];
        int nq = 0;
        for (int i = 0; i < nl; ++i)
            if (lins[i]->dtype == DT_Q8_0) t[nq++] = Q4kTarget{lins[i]->w, lins[i]->M, col[i]};
        int S8 = 1;
        rc = launch_q8(t, nq, a8, m->part, ldo, ss, max_splits, gi.q4 ? S : 0, &S8, s);
        if (rc) return rc;
        S = S8;
    }
    for (int i = 0; i < nl; ++i) {
        const Lin& l = *lins[i];
        if (l.dtype != DT_F32) continue;
        int rc = launch_mm_f32(m->part + col[i], X, (const float*)l.w, T, l.M, K, (int)ldo, s);
        if (rc) return rc;
    }
    *S_out = S;
    return 0;
}

// Final projection for n rows into m->logits [n][V] (single split).
// Q4_K LM head on a filled operand of its a.rows input rows -> m->logits.
int lm_head_q4k(slate_hip_llama* m, const Act16& a, hipStream_t s) {
    const auto& c = m->cfg;
    const Lin& l = m->out;
    const size_t e0 = m->prof_on ? prof_event(m) : (size_t)-1, e1 = m->prof_on ? prof_event(m) : (size_t)-1;
    Q4kTarget t{l.w, c.vocab, 0};
    int S = 1;
    const int rc = launch_q4k(&t, 1, true, a, m->logits, c.vocab, 0, 1, &S, s, prof_ev(m, e0), prof_ev(m, e1));
    if (m->prof_on)
        m->prof_recs.push_back({a.rows_pad == 16 ? 0 : 3, (double)l.bytes() + 4.0 * a.rows * (c.d_model + c.vocab),
                                e0, e1});
    return rc;
}

int lm_head(slate_hip_llama* m, int n, hipStream_t s) {
    const auto& c = m->cfg;
    const Lin& l = m->out;
    if (l.dtype == DT_Q4K) {
        Act16 a = m->act;
        a.rows = n;
        a.rows_pad = row_pad(n);
        a.K = c.d_model;
        int rc = launch_act16_from_f32(a, m->xlast, c.d_model, s);
        if (rc) return rc;
        return lm_head_q4k(m, a, s);
    }
    if (l.dtype == DT_Q8_0) {
        Act8 a8 = m->act8;
        a8.rows = n;
        a8.rows_pad = row_pad(n);
        a8.K = c.d_model;
        int rc = launch_act8_from_f32(a8, m->xlast, c.d_model, s);
        if (rc) return rc;
        Q4kTarget t{l.w, c.vocab, 0};
        int S = 1;
        return launch_q8(&t, 1, a8, m->logits, c.vocab, 0, 1, 0, &S, s);
    }
    return launch_mm_f32(m->logits, m->xlast, (const float*)l.w, n, c.vocab, c.d_model, c.vocab, s);
}

// Enqueue the whole step (descriptors already in pinned staging).
int enqueue_step(slate_hip_llama* m, int n, int T, bool want_logits, hipStream_t s) {
    const auto& c = m->cfg;
    const int D = c.d_model, H = c.ffn_hidden, hd = c.head_dim, kvd = c.n_kv_heads * hd;
    size_t estep = m->prof_on ? prof_mark(m, s) : 0;
    const size_t in_ints = 3 * (size_t)m->max_slots + T + m->n_dec + 2 * (size_t)m->n_pre;
    SH_CHECK_HIP(hipMemcpyAsync(m->d_desc, m->h_desc, sizeof(int32_t) * in_ints, hipMemcpyHostToDevice, s));
    const int32_t* d_blk = m->d_tok + T;
    int rc = launch_pack_batch(m->d_desc, m->d_desc + m->max_slots, m->d_desc + 2 * m->max_slots, n, c.max_seq,
                               m->slot_stride, m->max_tokens, m->tok_off, m->tok2seq, m->tok_pos, m->kv_base,
                               m->last_tok, m->status, s);
    if (rc) return rc;
    if ((rc = launch_embed_rows(m->x, m->tok_embd, m->d_tok, T, c.vocab, D, s))) return rc;
    // the decode attention work units depend only on positions: once per step
    AttnXcd xq{};
    const bool xcd = !m->xcd_off && m->step_one_each && T <= m->max_slots &&
                     attention_xcd_merge(T, c.n_heads, c.n_kv_heads, hd, c.max_seq, true);
    if (xcd) {
        xq = attention_xcd_view(m->att_xcd, m->max_slots, c.n_kv_heads, c.max_seq);
        xq.misplaced = m->status + 1;   // pinned host word, cleared before the step
        xq.layer = 0;
        xq.rot = knobs().attn_xcd_tamper ? 7 : 0;
    }
    if ((rc = launch_attention_pairs(d_blk, m->n_dec, m->tok_pos, m->tok2seq, m->kv_base, T, c.n_heads, c.max_seq,
                                      m->att_pml, s, xcd ? &xq : nullptr, c.n_kv_heads))) return rc;
    const int tpad = row_pad(T);
    int S_prev = 0;
    RowNorm rn{};
    for (int li = 0; li < c.n_layers; ++li) {
        const LayerDev& Ld = m->L[li];
        int S;
        // x (+= down partials of the previous layer) -> attention norm -> QKV
        {
            const Lin* g[3] = {&Ld.q, &Ld.k, &Ld.v};
            int64_t col[3] = {0, D, D + kvd};
            const GroupIn gi = group_in(g, 3);
            Act16 a = act_for(m, T, D);
            rn = RowNorm{nullptr, 0, D, c.rms_eps};
            if (defer_norm(m, gi, D)) {   // all-Q4_K group: norm factor applied by rope_kv
                rn.ssq = m->ssq;
                rn.nblk = D / QK;
                rc = launch_residual_act(m->x, li ? m->part : nullptr, S_prev, (int64_t)tpad * D, Ld.attn_norm, T, D,
                                         a, m->ssq, s);
            } else {
                rc = launch_rmsnorm_act(gi.rows() ? m->xn : nullptr, m->x, li ? m->part : nullptr, S_prev,
                                        (int64_t)tpad * D, Ld.attn_norm, T, D, c.rms_eps, gi.q4 ? &a : nullptr, s);
            }
            if (rc) return rc;
            if ((rc = mm_group(m, &a, m->xn, T, D, g, col, 3, D + 2 * kvd, &S, s))) return rc;
        }
        char* Kl = (char*)m->Kpool + (int64_t)li * m->layer_stride * m->kv_bytes;
        char* Vl = (char*)m->Vpool + (int64_t)li * m->layer_stride * m->kv_bytes;
        {
            const Lin* g[1] = {&Ld.o};
            int64_t col[1] = {0};
            const GroupIn gi = group_in(g, 1);
            Act16 a = act_for(m, T, D);
            const size_t ea = m->prof_on ? prof_event(m) : (size_t)-1, eb = m->prof_on ? prof_event(m) : (size_t)-1;
            // one token per sequence: RoPE and the K/V append run inside the
            // attention kernel; otherwise (prompt chunks) before it
            rc = 1;
            AttnXcd xl = xq;
            xl.layer = li;
            if (m->step_one_each)
                rc = launch_attention_rope(m->att, Kl, Vl, m->part, S, (int64_t)tpad * (D + 2 * kvd), D + 2 * kvd,
                                           m->rope_cs, rn, m->tok_pos, T, c.n_heads, c.n_kv_heads, hd,
                                           m->head_stride, c.max_seq, m->att_po, m->att_pml, gi.q4 ? &a : nullptr, s,
                                           prof_ev(m, ea), prof_ev(m, eb), m->kv_f16, xcd ? &xl : nullptr);
            if (rc < 0) return rc;
            if (rc > 0) {
                if ((rc = launch_rope_kv(m->q, Kl, Vl, m->part, S, (int64_t)tpad * (D + 2 * kvd), D + 2 * kvd,
                                         m->tok2seq, m->tok_pos, m->kv_base, T, c.n_heads, c.n_kv_heads, hd,
                                         m->head_stride, m->rope_cs, rn, m->kv_f16, s)))
                    return rc;
                if ((rc = launch_attention_blocks(m->att, m->q, Kl, Vl, m->tok2seq, m->tok_pos, m->kv_base, T, d_blk,
                                                  m->n_dec, d_blk + m->n_dec, d_blk + m->n_dec + m->n_pre, m->n_pre,
                                                  c.n_heads, c.n_kv_heads, hd, m->head_stride, c.max_seq, m->att_po,
                                                  m->att_pml, gi.q4 ? &a : nullptr, s, prof_ev(m, ea),
                                                  prof_ev(m, eb), true, m->kv_f16, m->step_prompt_mfma)))
                    return rc;
            }
            if (m->prof_on)   // K and V once per kv head per sequence, q in and out once
                m->prof_recs.push_back({m->step_mixed ? 4 : 1, m->step_kv_rows * 2.0 * kvd * 4 + 2.0 * T * D * 4, ea, eb});
            if ((rc = mm_group(m, &a, m->att, T, D, g, col, 1, D, &S, s))) return rc;
        }
        {
            const Lin* g[2] = {&Ld.gate, &Ld.up};
            int64_t col[2] = {0, H};
            const GroupIn gi = group_in(g, 2);
            Act16 a = act_for(m, T, D);
            rn = RowNorm{nullptr, 0, D, c.rms_eps};
            // all-Q4_K group: the norm factor is applied by silu_act, which
            // exists only for widths H % 256 == 0 (the f32 silu_mul
            // fallback takes no row factor, so other widths normalise here)
            if (defer_norm(m, gi, D) && H % QK == 0) {
                rn.ssq = m->ssq;
                rn.nblk = D / QK;
                rc = launch_residual_act(m->x, m->part, S, (int64_t)tpad * D, Ld.ffn_norm, T, D, a, m->ssq, s);
            } else {
                rc = launch_rmsnorm_act(gi.rows() ? m->xn : nullptr, m->x, m->part, S, (int64_t)tpad * D, Ld.ffn_norm,
                                        T, D, c.rms_eps, gi.q4 ? &a : nullptr, s);
            }
            if (rc) return rc;
            if ((rc = mm_group(m, &a, m->xn, T, D, g, col, 2, 2 * H, &S, s))) return rc;
        }
        {
            const Lin* g[1] = {&Ld.down};
            int64_t col[1] = {0};
            const GroupIn gi = group_in(g, 1);
            Act16 a = act_for(m, T, H);
            if (H % QK == 0)
                rc = launch_silu_act(gi.rows() ? m->h : nullptr, m->part, m->part + H, T, H, S, (int64_t)tpad * 2 * H,
                                     2 * H, gi.q4 ? &a : nullptr, rn, s);
            else   // no Q4_K operand exists for this width (and no deferred norm, above)
                rc = launch_silu_mul(m->h, m->part, m->part + H, T, H, S, (int64_t)tpad * 2 * H, 2 * H, 2 * H, s);
            if (rc) return rc;
            if ((rc = mm_group(m, &a, m->h, T, H, g, col, 1, D, &S, s))) return rc;
        }
        S_prev = S;
    }
    if (m->step_one_each && m->defer_norm && m->out.dtype == DT_Q4K && D % QK == 0) {
        // every token is its sequence's last: the residual kernel writes the
        // LM head operand of x*w directly and the argmax applies the final
        // RMSNorm factor to the logits (as the deferred norms of the layers)
        Act16 a = act_for(m, T, D);
        if ((rc = launch_residual_act(m->x, m->part, S_prev, (int64_t)tpad * D, m->out_norm, T, D, a, m->ssq, s)))
            return rc;
        if ((rc = lm_head_q4k(m, a, s))) return rc;
        const RowNorm rl{m->ssq, D / QK, D, c.rms_eps};
        if ((rc = launch_argmax_rows(m->next, m->logits, n, c.vocab, m->argmax_ws, s, &rl))) return rc;
    } else {
        if ((rc = launch_rmsnorm_act(m->xn, m->x, m->part, S_prev, (int64_t)tpad * D, m->out_norm, T, D,
                                     c.rms_eps, nullptr, s)))
            return rc;
        // rows of each sequence's last token -> xlast (gather by last_tok)
        if ((rc = launch_embed_rows(m->xlast, m->xn, m->last_tok, n, T, D, s))) return rc;
        if ((rc = lm_head(m, n, s))) return rc;
        if ((rc = launch_argmax_rows(m->next, m->logits, n, c.vocab, m->argmax_ws, s))) return rc;
    }
    if (m->prof_on) m->prof_recs.push_back({m->step_mixed ? 5 : 2, 0.0, estep, prof_mark(m, s)});
    if (want_logits)
        SH_CHECK_HIP(hipMemcpyAsync(m->h_logits, m->logits, sizeof(float) * (size_t)n * c.vocab,
                                    hipMemcpyDeviceToHost, s));
    return 0;
}

// Capture one step's launches into an instantiated graph (no memset nodes:
// the step has none).
int capture_step(slate_hip_llama* m, int n, int T, bool want, hipStream_t s, hipGraphExec_t* out) {
    *out = nullptr;
    SH_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_step(m, n, T, want, s);
    hipGraph_t g = nullptr;
    const hipError_t ec = hipStreamEndCapture(s, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (ec != hipSuccess || !g) {
        set_error(-7, "llama_step: graph capture failed: %s", hipGetErrorString(ec));
        return -7;
    }
    const hipError_t ei = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) {
        set_error(-7, "llama_step: graph instantiation failed: %s", hipGetErrorString(ei));
        *out = nullptr;
        return -7;
    }
    return 0;
}

// Whether a step's prompt chunks should attend on the MFMA prompt kernel
// rather than with its decode tokens in the tokenwise decode kernel.  The
// tokenwise launch overlaps prompt work with the decode tokens' K/V streaming
// (HBM-bound), the MFMA kernel runs after them: it pays when the prompt
// attention flops (4 per q head, key and element) reach about 6 per decode
// K/V byte (measured on MI355X at the 8B shape: a 200-token chunk at
// position 300 beside 15 decode tokens at ~1200 context, ratio 7.8, takes
// 61 us on the MFMA kernel and 68 us tokenwise; a 100-token chunk at 0,
// ratio 0.5, 45 and 37 us).  Steps without decode tokens always take it.
bool prompt_mfma_pays(const slate_hip_llama* m, slate_hip_llama_session_t* const* sessions, int n,
                      const int32_t* n_new) {
    if (knobs().attn_mfma == 2) return true;
    const auto& c = m->cfg;
    double prompt_keys = 0, decode_keys = 0;   // (query token, key) pairs
    for (int i = 0; i < n; ++i) {
        const double p0 = sessions[i]->pos, k = n_new[i];
        if (k > 1) prompt_keys += k * p0 + k * (k + 1) / 2;
        else decode_keys += p0 + 1;
    }
    const double flops = prompt_keys * c.n_heads * c.head_dim * 4.0;
    const double bytes = decode_keys * c.n_kv_heads * c.head_dim * 8.0;
    return flops >= 6.0 * bytes;
}

// Enqueue one step (replaying the batch size's graph for decode-only
// steps when graphs are on), wait for it and fold in its profile.
int run_step(slate_hip_llama* m, int n, int T, bool want, hipStream_t s) {
    m->h_status[1] = 0;   // set by a decode attention merge that found a partial from another XCD
    int rc;
    // decode-only steps repeat the same launch sequence for a given batch
    // size: replay it as a HIP graph (the descriptor copy in the graph reads
    // the pinned staging, so the step's inputs are current)
    if (m->graphs_on && !m->prof_on && T == n) {
        hipGraphExec_t ge = nullptr;
        for (const auto& g : m->graphs)
            if (g.n == n && g.want == want) ge = g.exec;
        if (!ge) {
            rc = capture_step(m, n, T, want, s, &ge);
            if (rc) return rc;
            m->graphs.push_back({n, want, ge});
        }
        if (hipGraphLaunch(ge, s) != hipSuccess) {
            set_error(-7, "llama_step: graph launch failed");
            return -7;
        }
    } else {
        rc = enqueue_step(m, n, T, want, s);
        if (rc) {
            m->prof_recs.clear();
            m->prof_used = 0;
            return rc;
        }
    }
    if (hipStreamSynchronize(s) != hipSuccess) {
        set_error(-7, "llama_step: device execution failed");
        return -7;
    }
    if (m->prof_on) {
        if (m->h_status[1] != 0) {   // the step runs again: its timings are dropped
            m->prof_recs.clear();
            m->prof_used = 0;
        } else {
            prof_collect(m);
        }
    }
    return 0;
}

int new_common(slate_hip_llama* m, const slate_hip_llama_config_t* cfg, int max_slots, int max_tokens) {
    if (!valid_cfg(cfg)) {
        set_error(-1, "engine: invalid config");
        return -1;
    }
    if (max_slots < 1 || max_slots > 1024 || max_tokens < max_slots) {
        set_error(-1, "engine: need 1 <= max_slots <= 1024 and max_tokens >= max_slots");
        return -1;
    }
    m->cfg = *cfg;
    m->max_slots = max_slots;
    m->max_tokens = max_tokens;
    m->knobs = read_knobs();   // the switches in force for this engine's steps
    KnobScope ks(&m->knobs);
    return alloc_runtime(m);
}

uint64_t mix(uint64_t a, uint64_t b) {
    uint64_t z = a * 0x9E3779B97F4A7C15ull + b;
    z = (z ^ (z >> 31)) * 0xBF58476D1CE4E5B9ull;
    return z ^ (z >> 29);
}

}  // namespace

extern "C" {

slate_hip_llama_t* slate_hip_llama_new(const slate_hip_llama_config_t* cfg, const float* token_embd,
                                       const float* output_norm, const void* output, int output_dtype,
                                       const slate_hip_llama_layer_t* layers, int max_slots, int max_tokens) {
    if (!device_ok()) return nullptr;
    if (!token_embd || !output_norm || !layers) {
        set_error(-1, "llama_new: NULL weights");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    slate_hip_llama* m = new slate_hip_llama();
    if (new_common(m, cfg, max_slots, max_tokens)) { free_model(m); return nullptr; }
    const auto& c = m->cfg;
    const int D = c.d_model, H = c.ffn_hidden, kvd = c.n_kv_heads * c.head_dim;
    RowStage st;
    void* p;
    if (upload(m, &p, token_embd, (size_t)c.vocab * D * 4)) { free_model(m); return nullptr; }
    m->tok_embd = (float*)p;
    if (upload(m, &p, output_norm, (size_t)D * 4)) { free_model(m); return nullptr; }
    m->out_norm = (float*)p;
    if (!output || c.tied_output) {   // tied LM head (llama.c:94-101)
        m->out.w = m->tok_embd;
        m->out.dtype = DT_F32;
        m->out.M = c.vocab;
        m->out.K = D;
    } else if (set_lin(m, m->out, output, output_dtype, c.vocab, D, st)) {
        free_model(m);
        return nullptr;
    }
    m->L.resize(c.n_layers);
    for (int i = 0; i < c.n_layers; ++i) {
        const slate_hip_llama_layer_t& s = layers[i];
        LayerDev& d = m->L[i];
        if (upload(m, &p, s.attn_norm, (size_t)D * 4)) { free_model(m); return nullptr; }
        d.attn_norm = (float*)p;
        if (upload(m, &p, s.ffn_norm, (size_t)D * 4)) { free_model(m); return nullptr; }
        d.ffn_norm = (float*)p;
        if (set_lin(m, d.q, s.attn_q, s.attn_q_dtype, D, D, st) ||
            set_lin(m, d.k, s.attn_k, s.attn_k_dtype, kvd, D, st) ||
            set_lin(m, d.v, s.attn_v, s.attn_v_dtype, kvd, D, st) ||
            set_lin(m, d.o, s.attn_output, s.attn_output_dtype, D, D, st) ||
            set_lin(m, d.gate, s.ffn_gate, s.ffn_gate_dtype, H, D, st) ||
            set_lin(m, d.up, s.ffn_up, s.ffn_up_dtype, H, D, st) ||
            set_lin(m, d.down, s.ffn_down, s.ffn_down_dtype, D, H, st)) {
            free_model(m);
            return nullptr;
        }
    }
    if (hipStreamSynchronize(stream()) != hipSuccess) {
        set_error(-7, "llama_new: weight repack failed");
        free_model(m);
        return nullptr;
    }
    return m;
}

slate_hip_llama_t* slate_hip_llama_new_synthetic(const slate_hip_llama_config_t* cfg, uint64_t seed, int quant,
                                                 int max_slots, int max_tokens) {
    if (!device_ok()) return nullptr;
    if (quant != DT_F32 && quant != DT_Q4K && quant != DT_Q8_0) {
        set_error(-1, "llama_new_synthetic: quant must be 0 (f32), 16 (q8_0) or 18 (q4_k)");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    slate_hip_llama* m = new slate_hip_llama();
    if (new_common(m, cfg, max_slots, max_tokens)) { free_model(m); return nullptr; }
    const auto& c = m->cfg;
    const int D = c.d_model, H = c.ffn_hidden, kvd = c.n_kv_heads * c.head_dim;
    hipStream_t s = stream();
    uint64_t tid = 0;
    const float std = 0.02f;
    RowStage st;
    auto gen_lin = [&](Lin& l, int M, int K) -> int {
        l.M = M;
        l.K = K;
        l.dtype = quant;
        if ((quant == DT_Q4K && K % QK) || (quant == DT_Q8_0 && K % Q8_ELEMS)) {
            set_error(-1, "llama_new_synthetic: K=%d not a multiple of the block size", K);
            return -1;
        }
        uint64_t sd = mix(seed, ++tid);
        if (quant == DT_F32) {
            char* p;
            if (dalloc(m, &p, l.bytes())) return -2;
            l.w = p;
            return launch_synth_f32((float*)p, (int64_t)M * K, sd, std, 0.f, s);
        }
        // generate in row layout (stream-ordered after the previous repack)
        if (hipStreamSynchronize(s) != hipSuccess) {
            set_error(-7, "llama_new_synthetic: generation failed");
            return -7;
        }
        void* row = st.get(l.bytes());
        if (!row) return -2;
        int rc = quant == DT_Q8_0 ? launch_synth_q8(row, M, K, sd, std, s) : launch_synth_q4k(row, M, K, sd, std, s);
        return rc ? rc : tile_lin(m, l, row);
    };
    auto gen_f32 = [&](float** dst, int64_t n, float sd_std, float fill) -> int {
        if (dalloc(m, dst, (size_t)n)) return -2;
        return launch_synth_f32(*dst, n, mix(seed, ++tid), sd_std, fill, s);
    };
    int rc = gen_f32(&m->tok_embd, (int64_t)c.vocab * D, std, 0.f);
    rc = rc ? rc : gen_f32(&m->out_norm, D, 0.f, 1.0f);
    rc = rc ? rc : gen_lin(m->out, c.vocab, D);
    m->L.resize(c.n_layers);
    for (int i = 0; i < c.n_layers && !rc; ++i) {
        LayerDev& d = m->L[i];
        rc = gen_f32(&d.attn_norm, D, 0.f, 1.0f);
        rc = rc ? rc : gen_f32(&d.ffn_norm, D, 0.f, 1.0f);
        rc = rc ? rc : gen_lin(d.q, D, D);
        rc = rc ? rc : gen_lin(d.k, kvd, D);
        rc = rc ? rc : gen_lin(d.v, kvd, D);
        rc = rc ? rc : gen_lin(d.o, D, D);
        rc = rc ? rc : gen_lin(d.gate, H, D);
        rc = rc ? rc : gen_lin(d.up, H, D);
        rc = rc ? rc : gen_lin(d.down, D, H);
    }
    if (!rc && hipStreamSynchronize(s) != hipSuccess) {
        set_error(-7, "llama_new_synthetic: generation failed");
        rc = -7;
    }
    if (rc) { free_model(m); return nullptr; }
    return m;
}

void slate_hip_llama_free(slate_hip_llama_t* m) {
    if (!m) return;
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    for (hipEvent_t e : m->prof_ev) (void)hipEventDestroy(e);
    (void)hipStreamSynchronize(stream());
    for (const auto& g : m->graphs) (void)hipGraphExecDestroy(g.exec);
    free_model(m);
}

int64_t slate_hip_llama_get_tensor(const slate_hip_llama_t* m, const char* name, void* host_dst, int64_t cap,
                                   int* dtype) {
    if (!m || !name) return -1;
    const void* src = nullptr;
    size_t bytes = 0;
    int dt = DT_F32;
    const Lin* tiled = nullptr;
    const auto& c = m->cfg;
    std::string n(name);
    if (n == "token_embd") { src = m->tok_embd; bytes = (size_t)c.vocab * c.d_model * 4; }
    else if (n == "output_norm") { src = m->out_norm; bytes = (size_t)c.d_model * 4; }
    else if (n == "output") {
        src = m->out.w;
        bytes = m->out.bytes();
        dt = m->out.dtype;
        if (dt == DT_Q4K || dt == DT_Q8_0) tiled = &m->out;
    }
    else if (n.rfind("blk.", 0) == 0) {
        int li = atoi(n.c_str() + 4);
        size_t dot = n.find('.', 4);
        if (li < 0 || li >= c.n_layers || dot == std::string::npos) return -1;
        std::string f = n.substr(dot + 1);
        const LayerDev& d = m->L[li];
        const Lin* l = nullptr;
        if (f == "attn_norm") { src = d.attn_norm; bytes = (size_t)c.d_model * 4; }
        else if (f == "ffn_norm") { src = d.ffn_norm; bytes = (size_t)c.d_model * 4; }
        else if (f == "attn_q") l = &d.q;
        else if (f == "attn_k") l = &d.k;
        else if (f == "attn_v") l = &d.v;
        else if (f == "attn_output") l = &d.o;
        else if (f == "ffn_gate") l = &d.gate;
        else if (f == "ffn_up") l = &d.up;
        else if (f == "ffn_down") l = &d.down;
        else return -1;
        if (l) {
            src = l->w;
            bytes = l->bytes();
            dt = l->dtype;
            if (dt == DT_Q4K || dt == DT_Q8_0) tiled = l;
        }
    } else {
        return -1;
    }
    if (dtype) *dtype = dt;
    if (!host_dst) return (int64_t)bytes;
    if ((int64_t)bytes > cap) return -2;
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    if (hipStreamSynchronize(stream()) != hipSuccess) {
        set_error(-7, "get_tensor: stream failed");
        return -7;
    }
    if (tiled) {   // back to slate's row layout
        std::vector<uint8_t> t(tiled->dev_bytes());
        if (hipMemcpy(t.data(), src, t.size(), hipMemcpyDeviceToHost) != hipSuccess) {
            set_error(-7, "get_tensor copy failed");
            return -7;
        }
        if (tiled->dtype == DT_Q8_0) q8_untile_host((uint8_t*)host_dst, t.data(), tiled->M, tiled->K);
        else q4k_untile_host((uint8_t*)host_dst, t.data(), tiled->M, tiled->K);
        return (int64_t)bytes;
    }
    if (hipMemcpy(host_dst, src, bytes, hipMemcpyDeviceToHost) != hipSuccess) {
        set_error(-7, "get_tensor copy failed");
        return -7;
    }
    return (int64_t)bytes;
}

slate_hip_llama_session_t* slate_hip_llama_session_new(slate_hip_llama_t* m) {
    if (!m) return nullptr;
    std::lock_guard<std::mutex> lk(m->mu);
    if (m->free_slots.empty()) {
        set_error(-2, "session_new: all %d KV slots in use", m->max_slots);
        return nullptr;
    }
    auto* s = new slate_hip_llama_session{m, m->free_slots.back(), 0};
    m->free_slots.pop_back();
    return s;
}

void slate_hip_llama_session_free(slate_hip_llama_session_t* s) {
    if (!s) return;
    {
        std::lock_guard<std::mutex> lk(s->m->mu);
        s->m->free_slots.push_back(s->slot);
    }
    delete s;
}

int slate_hip_llama_session_position(const slate_hip_llama_session_t* s) { return s ? s->pos : -1; }

void slate_hip_llama_session_reset(slate_hip_llama_session_t* s) {
    if (!s) return;
    std::lock_guard<std::mutex> lk(s->m->mu);
    s->pos = 0;   // attention reads positions < pos only: stale K/V rows are never read
}

const slate_hip_llama_config_t* slate_hip_llama_config(const slate_hip_llama_t* m) { return m ? &m->cfg : nullptr; }

int slate_hip_llama_step(slate_hip_llama_t* m, slate_hip_llama_session_t** sessions, int n, const int32_t* n_new,
                         const int32_t* tokens, float* out_logits, int32_t* out_next) {
    if (!m || !sessions || !n_new || !tokens || n < 1 || n > m->max_slots) return -1;
    const auto& c = m->cfg;
    std::lock_guard<std::mutex> lk(m->mu);
    KnobScope ks(&m->knobs);
    int T = 0;
    for (int i = 0; i < n; ++i) {
        slate_hip_llama_session_t* s = sessions[i];
        if (!s || s->m != m || n_new[i] < 1) return -1;
        for (int j = 0; j < i; ++j)
            if (sessions[j] == s) return -1;
        if ((int64_t)s->pos + n_new[i] > c.max_seq) return -2;
        T += n_new[i];
        if (T > m->max_tokens) return -2;
    }
    for (int t = 0; t < T; ++t)
        if (tokens[t] < 0 || tokens[t] >= c.vocab) return -3;
    for (int i = 0; i < m->max_slots; ++i) {
        bool act = i < n;
        m->h_desc[i] = act ? sessions[i]->slot : 0;
        m->h_desc[m->max_slots + i] = act ? sessions[i]->pos : 0;
        m->h_desc[2 * m->max_slots + i] = act ? n_new[i] : 0;
    }
    memcpy(m->h_tok, tokens, sizeof(int32_t) * T);
    // attention work: decode tokens one per block, prompt chunks in blocks of
    // consecutive tokens of one sequence (or one block per token, tokenwise)
    {
        const bool mfma = m->prompt_mfma && prompt_mfma_pays(m, sessions, n, n_new);
        const bool tokenwise = !mfma && m->tokenwise_attn;
        const int G = c.n_heads / c.n_kv_heads;
        const int QB = mfma ? attention_prompt_block(G) : attn_prefill_block(G);
        int32_t* blk = m->h_tok + T;
        int nd = 0, np = 0, t = 0;
        for (int i = 0; i < n; ++i) {
            if (n_new[i] == 1 || tokenwise) nd += n_new[i];
            else np += (n_new[i] + QB - 1) / QB;
        }
        m->step_prompt_mfma = mfma && np > 0;
        int id = 0, ip = 0;
        for (int i = 0; i < n; ++i) {
            if (n_new[i] == 1 || tokenwise) {
                for (int k = 0; k < n_new[i]; ++k) blk[id++] = t + k;
            } else {
                for (int k = 0; k < n_new[i]; k += QB) {
                    blk[nd + ip] = t + k;
                    blk[nd + np + ip] = std::min(QB, n_new[i] - k);
                    ++ip;
                }
            }
            t += n_new[i];
        }
        m->n_dec = nd;
        m->n_pre = np;
        m->step_mixed = T > n;
        m->step_one_each = np == 0 && nd == T && T == n;
        for (int i = 0; i < n; ++i) m->step_one_each = m->step_one_each && n_new[i] == 1;
    }
    m->step_kv_rows = 0;
    for (int i = 0; i < n; ++i) m->step_kv_rows += (double)sessions[i]->pos + n_new[i];
    hipStream_t s = stream();
    {
        std::lock_guard<std::mutex> lk2(g_enqueue_mu);
        const bool want = out_logits != nullptr;
        int rc = run_step(m, n, T, want, s);
        if (rc) return rc;
        if (m->h_status[1] != 0) {
            // A merge inside the decode attention found a partial of its pair
            // written on another XCD, so it may have read what that XCD's L2
            // still held: the step's results are not trusted.  Turn the
            // in-kernel merge off for this engine and run the step again on
            // the merge kernel.  Running it again is exact: a step recomputes
            // everything from its tokens and the K/V rows before its
            // positions, and rewrites the rows at its positions with the same
            // values.
            m->xcd_off = true;
            for (const auto& g : m->graphs) (void)hipGraphExecDestroy(g.exec);
            m->graphs.clear();
            if ((rc = run_step(m, n, T, want, s))) return rc;
        }
    }
    if (m->h_status[0] != 0) {
        set_error(m->h_status[0], "llama_step: device packing rejected the descriptor (%d)", m->h_status[0]);
        return m->h_status[0];
    }
    if (out_logits) memcpy(out_logits, m->h_logits, sizeof(float) * (size_t)n * c.vocab);
    if (out_next) memcpy(out_next, m->h_next, sizeof(int32_t) * n);
    for (int i = 0; i < n; ++i) sessions[i]->pos += n_new[i];
    return 0;
}

int slate_hip_llama_profile(slate_hip_llama_t* m, int enable) {
    if (!m || enable < 0 || enable > 2) return -1;
    std::lock_guard<std::mutex> lk(m->mu);
    m->prof_on = enable != 0;
    if (enable == 1) {
        for (int i = 0; i < slate_hip_llama::NPROF; ++i) m->prof_ms[i] = m->prof_bytes[i] = 0, m->prof_n[i] = 0;
        m->prof_recs.clear();
        m->prof_used = 0;
    }
    return 0;
}

int slate_hip_llama_kv_f16(const slate_hip_llama_t* m) { return m ? (m->kv_f16 ? 1 : 0) : -1; }

int slate_hip_llama_attn_xcd_merge(const slate_hip_llama_t* m) {
    if (!m) return -1;
    const auto& c = m->cfg;
    KnobScope ks(&m->knobs);
    return !m->xcd_off && attention_xcd_merge(1, c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq, true) ? 1 : 0;
}

int slate_hip_llama_graphs(slate_hip_llama_t* m, int enable) {
    if (!m) return -1;
    std::lock_guard<std::mutex> lk(m->mu);
    if (enable && tracer_attached()) {
        m->graphs_on = false;
        set_error(-5, "llama_graphs: refused while a rocprofiler tool is attached; steps launch eagerly");
        return -5;
    }
    m->graphs_on = enable != 0;
    return 0;
}

int slate_hip_llama_profile_read(slate_hip_llama_t* m, int cls, double* ms, double* bytes, int64_t* launches) {
    if (!m || cls < 0 || cls >= slate_hip_llama::NPROF) return -1;
    std::lock_guard<std::mutex> lk(m->mu);
    if (ms) *ms = m->prof_ms[cls];
    if (bytes) *bytes = m->prof_bytes[cls];
    if (launches) *launches = m->prof_n[cls];
    return 0;
}

int slate_hip_llama_batch_step(slate_hip_llama_t* m, slate_hip_llama_session_t** sessions, int n,
                               const int32_t* tokens, float* out_logits) {
    if (!m || n < 1 || n > m->max_slots) return -1;
    std::vector<int32_t> ones(n, 1);
    return slate_hip_llama_step(m, sessions, n, ones.data(), tokens, out_logits, nullptr);
}

int slate_hip_llama_prefill(slate_hip_llama_session_t* s, const int32_t* tokens, int n_tokens, float* out_logits) {
    if (!s || !tokens || !out_logits || n_tokens <= 0) return -1;
    slate_hip_llama* m = s->m;
    if ((int64_t)s->pos + n_tokens > m->cfg.max_seq) return -2;
    for (int i = 0; i < n_tokens; ++i)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab) return -3;
    int done = 0;
    while (done < n_tokens) {
        int chunk = std::min(n_tokens - done, m->max_tokens);
        bool last = done + chunk == n_tokens;
        int rc = slate_hip_llama_step(m, &s, 1, &chunk, tokens + done, last ? out_logits : nullptr, nullptr);
        if (rc) return rc;
        done += chunk;
    }
    return 0;
}

int slate_hip_llama_decode_step(slate_hip_llama_session_t* s, int32_t token, float* out_logits) {
    if (!s || !out_logits) return -1;
    int one = 1;
    return slate_hip_llama_step(s->m, &s, 1, &one, &token, out_logits, nullptr);
}

int slate_hip_llama_session_kv(const slate_hip_llama_session_t* s, float* K, float* V) {
    if (!s || !K || !V) return -1;
    slate_hip_llama* m = s->m;
    const auto& c = m->cfg;
    const int kvd = c.n_kv_heads * c.head_dim;
    std::vector<float> buf((size_t)m->slot_stride);
    std::vector<_Float16> hbuf(m->kv_f16 ? (size_t)m->slot_stride : 0);
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    if (hipStreamSynchronize(stream()) != hipSuccess) return -7;
    for (int which = 0; which < 2; ++which) {
        const char* src = (const char*)(which ? m->Vpool : m->Kpool) + (int64_t)s->slot * m->slot_stride * m->kv_bytes;
        if (m->kv_f16) {
            if (hipMemcpy(hbuf.data(), src, hbuf.size() * 2, hipMemcpyDeviceToHost) != hipSuccess) return -7;
            for (size_t i = 0; i < buf.size(); ++i) buf[i] = (float)hbuf[i];
        } else if (hipMemcpy(buf.data(), src, buf.size() * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
            return -7;
        }
        float* dst = which ? V : K;
        for (int li = 0; li < c.n_layers; ++li)
            for (int h = 0; h < c.n_kv_heads; ++h)
                for (int p = 0; p < c.max_seq; ++p)
                    memcpy(dst + ((size_t)li * c.max_seq + p) * kvd + h * c.head_dim,
                           buf.data() + li * m->layer_stride + h * m->head_stride + (int64_t)p * c.head_dim,
                           sizeof(float) * c.head_dim);
    }
    return 0;
}

}  // extern "C"
