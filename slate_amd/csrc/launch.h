// launch.h -- kernel launchers shared between the kernel files, the vtable
// and the engine.  Every launcher enqueues on the given stream and returns 0
// or a negative code (having recorded the sticky error).
#pragma once

#include "common.h"

namespace slate_hip {

// k_rows.hip
int launch_rmsnorm_rows(float* y, float* x, const float* delta, int nsplit, int64_t split_stride,
                        const float* w, int B, int D, float eps, hipStream_t s);
int launch_silu_mul(float* y, const float* gate, const float* up, int rows, int H, int nsplit,
                    int64_t split_stride, int64_t gate_ld, int64_t up_ld, hipStream_t s);
int launch_add(float* y, const float* x, int64_t n, hipStream_t s);
int launch_embed_rows(float* y, const float* W, const int32_t* tok, int T, int V, int D, hipStream_t s);
int launch_rope_rows(float* x, const int32_t* pos, int n_rows, int n_heads, int hd, const float* cs,
                     int max_pos, int* bad, hipStream_t s);
// Fused engine epilogues; `a` (nullable) receives the Q4_K activation operand
// of rows_pad rows (rows past `rows` zero), y (nullable) the f32 rows.
int launch_rmsnorm_act(float* y, float* x, const float* delta, int nsplit, int64_t split_stride, const float* w,
                       int rows, int D, float eps, const Act16* a, hipStream_t s);
int launch_silu_act(float* y, const float* gate, const float* up, int rows, int H, int nsplit,
                    int64_t split_stride, int64_t ld, const Act16* a, const RowNorm& rn, hipStream_t s);
// K/V rows are written as f32, or rounded to f16 when kv_f16.
int launch_rope_kv(float* qout, void* Kpool, void* Vpool, const float* part, int nsplit, int64_t split_stride,
                   int qkv_ld, const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int T,
                   int n_heads, int n_kv_heads, int hd, int64_t head_stride, const float* cs, const RowNorm& rn,
                   bool kv_f16, hipStream_t s);
// x += sum of split partials, per-block sums of squares into ssq, x * w as
// the Q4_K operand (the row factor is left to the consumer, RowNorm).
int launch_residual_act(float* x, const float* delta, int nsplit, int64_t split_stride, const float* w, int rows,
                        int D, const Act16& a, float* ssq, hipStream_t s);
// ws: argmax_workspace_bytes(B, V) of device scratch ((value, index) per row and chunk).
// rn (deferred RMSNorm of the rows the logits came from): each logit is
// multiplied by its row's factor in place before the comparison.
size_t argmax_workspace_bytes(int B, int V);
int launch_argmax_rows(int32_t* out, float* logits, int B, int V, void* ws, hipStream_t s,
                       const RowNorm* rn = nullptr);
int launch_pack_batch(const int32_t* slot, const int32_t* pos0, const int32_t* n_new, int B, int max_seq,
                      int64_t slot_stride, int T_cap, int32_t* tok_off, int32_t* tok2seq,
                      int32_t* tok_pos, int64_t* kv_base, int32_t* last_tok, int32_t* status,
                      hipStream_t s);
int launch_mm_f32(float* Y, const float* X, const float* W, int B, int M, int K, int ldy, hipStream_t s);
int launch_linear_batch(float* C, const float* X, const float* W, int B, int K, int N, hipStream_t s);

// k_attn.hip
int attn_chunk_size();
int attn_prefill_block(int group);   // query tokens per block for prompt chunks
// Blocks: dec_t0[n_dec] decode tokens (one each); pre_t0/pre_n[n_pre] runs of
// consecutive tokens of one sequence, at most attn_prefill_block(G) tokens
// each, or attention_prompt_block(G) with prompt_mfma (the MFMA prompt kernel,
// for shapes where attention_prompt_mfma holds).  Every token must be covered
// once.
// `act` (nullable) also receives the output rows as the Q4_K activation
// operand (Hq * HD % 256 == 0).
int launch_attention_blocks(float* out, const float* q, const void* Kp, const void* Vp, const int32_t* tok2seq,
                            const int32_t* tok_pos, const int64_t* kv_base, int T, const int32_t* dec_t0,
                            int n_dec, const int32_t* pre_t0, const int32_t* pre_n, int n_pre, int Hq, int Hkv,
                            int HD, int64_t head_stride, int max_pos, float* po, float* pml, const Act16* act,
                            hipStream_t s, hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr,
                            bool pairs_ready = false, bool kv_f16 = false, bool prompt_mfma = false);
// The decode work-unit list that launch_attention_blocks builds (in the tail
// of the pml buffer) when pairs_ready is false: build it once when several
// launches share the same tokens and positions (the layers of one step).
// Decode steps with one token per sequence: RoPE of q and k, the K/V append
// (what launch_rope_kv does) and the attention of launch_attention_blocks in
// one kernel plus the merge.  Returns 1, launching nothing, when the shape
// is not one the fused kernel covers (the caller then runs the two paths).
// Decode attention work queues, one per XCD (attention_xcd_* below): the
// chunk units of (token t, kv head h) all go to queue (t * Hkv + h) % 8, so
// the unit that finishes a pair's last chunk can merge the pair's partials
// from its own XCD's L2 inside the attention kernel.
struct AttnXcd {
    int32_t* len;       // [8] units per queue
    int32_t* stepc;     // [1] steps counted by the queue builders (the launch tags' sequence)
    int32_t* arrive;    // [max_tok * Hkv] finished chunks per (token, kv head)
    int32_t* tag;       // [max_tok * Hkv][nch] the launch and XCD that wrote each chunk's partial
    int4* units;        // [8][cap] {t * 65536 + c, p, kv base low, kv base high | h << 24}
    int cap;
    int max_tok;
    int nch;            // key chunks per pair the tags are laid out for
    int max_tok_step;   // tokens of the step being launched (<= max_tok)
    int layer;          // the launch's layer (part of its tags)
    int32_t* misplaced; // set to 1 when a merge found a partial written on another XCD (nullptr: unchecked)
    int rot;            // nonzero (tests only): the merge expects tags no unit writes, so every merge reports
};
size_t attention_xcd_ints(int max_tok, int Hkv, int max_pos);
AttnXcd attention_xcd_view(int32_t* base, int max_tok, int Hkv, int max_pos);
// Checks once per process (a 64-workgroup launch and a copy) that
// consecutive workgroups run on consecutive XCDs; attention_xcd_merge is
// false until it has returned true.  Each launch also checks itself (the
// tags), so the probe only keeps the kernel off a device where the placement
// is not what it assumes at all.
bool attention_xcd_probe();
int launch_attention_rope(float* out, void* Kp, void* Vp, const float* part, int nsplit, int64_t split_stride,
                          int qkv_ld, const float* cs, const RowNorm& rn, const int32_t* tok_pos, int T, int Hq,
                          int Hkv, int HD, int64_t head_stride, int max_pos, float* po, float* pml, const Act16* act,
                          hipStream_t s, hipEvent_t ev_start, hipEvent_t ev_stop, bool kv_f16,
                          const AttnXcd* xq = nullptr);
// xq (optional): also fill the per-XCD queues (and reset their arrival
// counts) for the decode tokens.
int launch_attention_pairs(const int32_t* dec_t0, int n_dec, const int32_t* tok_pos, const int32_t* tok2seq,
                           const int64_t* kv_base, int T, int Hq, int max_pos, float* pml, hipStream_t s,
                           const AttnXcd* xq = nullptr, int Hkv = 0);
// Whether launch_attention_rope merges inside the attention kernel for this
// shape (the per-XCD queues are needed then).
bool attention_xcd_merge(int T, int Hq, int Hkv, int HD, int max_pos, bool has_act);
size_t attention_partial_floats(int T, int Hq, int HD, int max_pos);
int launch_attention_ragged(float* out, const float* q, const float* Kp, const float* Vp,
                            const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int T,
                            int Hq, int Hkv, int HD, int64_t head_stride, int max_pos, float* po,
                            float* pml, hipStream_t s);
int launch_attention_step(float* out, const float* q, const float* K, const float* V, float* scores, int L,
                          int D, hipStream_t s);

// k_attn_mfma.hip: prompt blocks (<= attention_prompt_block(G) consecutive
// tokens of one sequence, G = Hq / Hkv) on MFMA, leaving partials in the
// layout the merge kernel reads.  attention_prompt_mfma: the shape is one
// the kernel covers (f32 K/V, head_dim 64 or 128, 1, 2, 4 or 8 q heads per
// kv head) and SLATE_HIP_ATTN_MFMA is not 0.
bool attention_prompt_mfma(int Hq, int Hkv, int HD, bool kv_f16);
int attention_prompt_block(int G);
int launch_attention_prompt(const float* q, const float* Kp, const float* Vp, const int32_t* tok2seq,
                            const int32_t* tok_pos, const int64_t* kv_base, const int32_t* blk_t0,
                            const int32_t* blk_n, int n_blk, int Hq, int Hkv, int HD, int64_t head_stride,
                            int nch_max, float* po, float* pml, hipStream_t s, hipEvent_t ev0);

// k_synth.hip
int launch_synth_f32(float* dst, int64_t n, uint64_t seed, float std, float fill, hipStream_t s);
int launch_synth_q4k(void* dst, int64_t rows, int64_t cols, uint64_t seed, float std, hipStream_t s);
int launch_synth_q8(void* dst, int64_t rows, int64_t cols, uint64_t seed, float std, hipStream_t s);

// Host-side RoPE table exactly as llama_infer.c:77-92 computes the angles:
// cs[(p*half + i)*2 + {0,1}] = {cosf, sinf}(p * powf(theta, -2i/hd)).
void build_rope_table(float* cs, int max_pos, int hd, float theta);

}  // namespace slate_hip
