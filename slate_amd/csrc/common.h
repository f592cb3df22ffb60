// common.h -- shared host/device definitions for the gfx950 backend.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stddef.h>
#include <stdlib.h>

#include "../../include/slate_hip.h"

namespace slate_hip {

// ---------------------------------------------------------------------------
// Errors: a sticky process-wide message (compute entries return void at the
// vtable boundary, so failures must be observable afterwards).
void set_error(int code, const char* fmt, ...);
int  error_code();
hipStream_t stream();        // the backend stream (created on first use)
bool device_ok();            // a gfx950 device was opened

#define SH_CHECK_HIP(expr)                                                        \
    do {                                                                          \
        hipError_t _e = (expr);                                                   \
        if (_e != hipSuccess) {                                                   \
            ::slate_hip::set_error(-7, "%s failed: %s (%s:%d)", #expr,            \
                                   hipGetErrorString(_e), __FILE__, __LINE__);    \
            return -7;                                                            \
        }                                                                         \
    } while (0)

#define SH_CHECK_LAUNCH() SH_CHECK_HIP(hipGetLastError())

#define SH_REQUIRE(cond, ...)                                                     \
    do {                                                                          \
        if (!(cond)) { ::slate_hip::set_error(-1, __VA_ARGS__); return -1; }      \
    } while (0)

// Kernel launch that, when timing events are given, has the dispatch itself
// record them at kernel start / end (hipExtLaunchKernelGGL), so the elapsed
// time is the kernel's own duration without the gaps around it.
#define SH_LAUNCH(ev0, ev1, kernel, grid, block, shmem, stream, ...)                                \
    do {                                                                                          \
        if ((ev0) != nullptr || (ev1) != nullptr)                                                 \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ev0, ev1, 0, __VA_ARGS__);   \
        else                                                                                      \
            hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                  \
    } while (0)

// Plan and path switches (SLATE_HIP_* environment variables).  The C ABI's
// entries use the process defaults, read once when the library initialises;
// an engine reads its own copy when it is created (read_knobs) and every
// step it enqueues uses that copy (KnobScope on the enqueuing thread), so
// engines built under different settings keep their own kernel paths and a
// new engine never changes an existing one's.  The defaults are the measured
// fastest at the reference's numerics; every setting gives results within
// the parity tolerances.
struct Knobs {
    int attn_wave = 1;     // SLATE_HIP_ATTN_WAVE=0: phased decode attention for every shape
    int attn_rope = 1;     // SLATE_HIP_ATTN_ROPE: 0 RoPE/append in their own kernel, 2 fused into the phased kernel
    int attn_xcd = 1;      // SLATE_HIP_ATTN_XCD=0: decode attention partials merged by their own kernel
    int attn_xcd_tamper = 0;  // SLATE_HIP_ATTN_XCD_TAMPER=1 (tests): the in-kernel merge's placement check
                              // expects tags no unit writes, so every merge reports a partial from another
                              // XCD and the engine's fallback runs
    int attn_mfma = 1;     // SLATE_HIP_ATTN_MFMA: prompt blocks on the MFMA kernel 0 never, 1 when the
                           // step's prompt work outweighs its decode work, 2 whenever a step has prompt chunks
    int q4k_w = 8;         // SLATE_HIP_Q4K_W: waves per decode workgroup (4 or 8)
    int q4k_r = 0;         // SLATE_HIP_Q4K_R: weight tiles per wave (1, 2, 4; 0 = plan)
    int q4k_s = 0;         // SLATE_HIP_Q4K_S: decode split count (0 = plan)
    int q4k_wgs = 384;     // SLATE_HIP_Q4K_WGS: decode workgroup target of the plan
    int q4k_pf_s = 0;      // SLATE_HIP_Q4K_PF_S: prompt-kernel split count (0 = plan)
    int q4k_pf_nt = 0;     // SLATE_HIP_Q4K_PF_NT: 2 or 4 activation tiles per prompt workgroup (0 = plan)
    int q4k_dec32 = 1;     // SLATE_HIP_Q4K_DEC32=0: 17..32 rows on the prompt kernel, not the decode one
    int q4k_early = 0;     // SLATE_HIP_Q4K_EARLY=1: the decode kernel issues block 1 together with block 0
    int gemv1 = 1;         // SLATE_HIP_GEMV1=0: one-row C-ABI matvecs of tiled weights on the vector-ALU GEMV
    int row_pad64 = 0;     // SLATE_HIP_ROW_PAD64=1: rows beyond 64 padded to multiples of 64, not 16
    int q8_r = 0;          // SLATE_HIP_Q8_R, _S, _WGS: the same for the Q8_0 matmul
    int q8_s = 0;
    int q8_wgs = 448;
};
// The switches in force on this thread: the enclosing KnobScope's, else the
// process defaults.
const Knobs& knobs();
// The switches as the environment sets them now.
Knobs read_knobs();
class KnobScope {
  public:
    explicit KnobScope(const Knobs* k);
    ~KnobScope();
    KnobScope(const KnobScope&) = delete;
    KnobScope& operator=(const KnobScope&) = delete;

  private:
    const Knobs* prev_;
};

// Scratch owned by the backend: grown on demand, reused across calls.  Every
// use happens on the single backend stream, so reuse is ordered.
void* scratch(int slot, size_t bytes);

// ---------------------------------------------------------------------------
// Q4_K super-block geometry (include/slate/quant.h:34-36).
constexpr int QK = 256;
constexpr int QBLOCK = 144;

// Activation operand for the Q4_K MFMA kernels: X split into f16 hi + lo with
// a power-of-two scale per 256-element block, plus per-32-element sums for
// the min term, laid out in the order the matmul lanes read them (act16.h):
// frag [rows_pad/16][K/256][ACT_FRAG_UNITS] 16-byte units.
constexpr int ACT_FRAG_UNITS = 1152;       // 1092 used, padded to 18 x 64
struct Act16 {
    void* frag;
    int rows;       // valid rows
    int rows_pad;   // multiple of 16
    int K;
};
inline size_t act_frag_bytes(int rows_pad, int K) {
    return (size_t)(rows_pad / 16) * (K / QK) * ACT_FRAG_UNITS * 16;
}

// Launchers (all enqueue on the given stream; return 0 or negative code).
int launch_dequant_q4k(float* dst, const void* src, int64_t n_blocks, hipStream_t s);
// Rows of X are ldx floats apart.
int launch_act16_from_f32(const Act16& a, const float* X, int64_t ldx, hipStream_t s);
int launch_sum_splits(float* Y, const float* part, int nsplit, int rows, int rows_pad, int M,
                      hipStream_t s);

// Per-row RMSNorm factor deferred to the consumer of a matmul: ssq holds
// the sums of squares per 256-element block [rows][D/256] (nullptr = none).
struct RowNorm {
    const float* ssq;
    int nblk, D;
    float eps;
};

// Up to three Q4_K tensors sharing one input, fused into one launch; tensor i
// writes output columns [col, col + M).  Split-K partials: element (split,
// row b, col m) goes to out[split * split_stride + b * ldo + m] for
// b < rows_pad; the split count (<= max_splits) is returned in *S_out.
struct Q4kTarget { const void* w; int M; int64_t col; };
struct Q4kTargets {                 // kernel-argument form
    const uint8_t* w[3];
    int M[3];
    int col[3];
    int grp0[3];                    // first wave group of each tensor
    int n, grp_end;
};
// ev_start / ev_stop (optional) are recorded at the start of the first and
// the end of the last kernel of the matmul.
int launch_q4k(const Q4kTarget* t, int n, bool tiled, const Act16& a, float* out, int64_t ldo,
               int64_t split_stride, int max_splits, int* S_out, hipStream_t s,
               hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);
// One tensor, 1 < rows <= 16 f32 rows of X (ldx floats apart): the split-K
// partials of Y = X W^T in one launch that makes the activation operand
// itself (rows padded to 16).  Returns 1 without launching when the decode
// plan is not the 8-wave one (the caller then stages the operand).
int launch_q4k_conv(const Q4kTarget& t, bool tiled, const float* X, int64_t ldx, int rows, int K, float* out,
                    int64_t ldo, int64_t split_stride, int max_splits, int* S_out, hipStream_t s);
// Small-batch Q4_K GEMV (k_q4k_gemv.hip): 1..GEMV_MAX_ROWS activation rows
// X [B, K] f32 (16-byte aligned rows, ldx floats apart) against up to three
// tensors (ROW or TILED layout); writes final rows Y[b * ldy + col + m] in
// one kernel (no operand conversion, no split-K partials).
constexpr int GEMV_MAX_ROWS = 4;
// The C ABI's Q4_K matmuls take the GEMV for a single activation row: the
// VALU dot products cost ~2.9 wave-lane operations per weight element
// (a wave64 f32 operation takes 4 cycles of a SIMD) against ~1 for building
// the MFMA operand, so from two rows on the one-kernel GEMV no longer beats
// the three-kernel MFMA path (operand conversion, matmul, split sum).
constexpr int GEMV_ROUTE_ROWS = 1;
// One activation row on MFMA over TILED weights (k_q4k.hip): one kernel, K
// up to 64 blocks.
constexpr int GEMV1_MAX_BLOCKS = 64;
int launch_q4k_gemv1(const void* W, int M, int K, const float* x, float* y, hipStream_t s,
                     hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);
int launch_q4k_gemv(const Q4kTarget* t, int n, bool tiled, const float* X, int64_t ldx, int B, int K, float* Y,
                    int64_t ldy, hipStream_t s, hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);
// TILED weight layout (16-row tiles, see k_q4k.hip).
size_t q4k_tiled_bytes(int M, int K);
int launch_q4k_tile(void* dst, const void* src, int M, int K, hipStream_t s);
void q4k_untile_host(uint8_t* dst, const uint8_t* src, int M, int K);
// Activation rows are padded to whole 16-row MFMA tiles (the prompt kernels
// take a last group of fewer tiles than the others and skip the missing
// ones); SLATE_HIP_ROW_PAD64=1 pads rows beyond 64 to whole groups of four
// tiles instead.
inline int row_pad(int rows) {
    return knobs().row_pad64 && rows > 64 ? (rows + 63) / 64 * 64 : (rows + 15) / 16 * 16;
}
// Carve an Act16 for B rows x K out of backend scratch slot `slot`.
int make_act16(Act16& a, int B, int K, int slot);

// ---------------------------------------------------------------------------
// Q8_0 (include/slate/quant.h:16-31): 34-byte blocks of [f16 d][32 x int8].
constexpr int Q8_ELEMS = 32;
constexpr int Q8_BYTES = 34;
// TILED Q8_0 layout (k_q8.hip): 16-row tiles x 256-element groups of 4352
// bytes; K is padded to whole groups with zero blocks.
constexpr int Q8_GROUP = 256;
constexpr int Q8_TB = 4352;
__host__ __device__ inline int q8_groups(int K) { return (K + Q8_GROUP - 1) / Q8_GROUP; }
size_t q8_tiled_bytes(int M, int K);
int launch_q8_tile(void* dst, const void* src, int M, int K, hipStream_t s);
void q8_untile_host(uint8_t* dst, const uint8_t* src, int M, int K);
int launch_dequant_q8(float* dst, const void* src, int64_t n_blocks, hipStream_t s);

// Activation operand of the Q8_0 matmul: like Act16 (f16 hi + lo with a
// power-of-two scale per 256-element group and row) but with the elements of
// each MFMA K step inside one 32-element Q8_0 block, and no sums:
// frag [rows_pad/16][q8_groups(K)][ACT8_UNITS] 16-byte units.
constexpr int ACT8_UNITS = 1088;           // 1028 used, padded to 17 x 64
struct Act8 {
    void* frag;
    int rows;       // valid rows
    int rows_pad;   // multiple of 16
    int K;          // multiple of 32
};
inline size_t act8_bytes(int rows_pad, int K) {
    return (size_t)(rows_pad / 16) * q8_groups(K) * ACT8_UNITS * 16;
}
int launch_act8_from_f32(const Act8& a, const float* X, int64_t ldx, hipStream_t s);
int make_act8(Act8& a, int B, int K, int slot);
// Up to three TILED Q8_0 tensors sharing one input (targets and partial
// layout as launch_q4k).  fixed_splits > 0 forces that split count (a group
// that also holds Q4_K tensors must write the same partials); otherwise the
// count is chosen (<= max_splits) and returned in *S_out.
int launch_q8(const Q4kTarget* t, int n, const Act8& a, float* out, int64_t ldo, int64_t split_stride,
              int max_splits, int fixed_splits, int* S_out, hipStream_t s, hipEvent_t ev_start = nullptr,
              hipEvent_t ev_stop = nullptr);

}  // namespace slate_hip
