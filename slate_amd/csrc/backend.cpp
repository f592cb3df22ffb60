// backend.cpp -- the slate_backend_t vtable for gfx950 and the extension
// entries (include/slate_hip.h).  Host code only; kernels live in k_*.hip.
//
// The vtable keeps the contract of include/slate/backend.h:41-99: pointers
// passed to compute entries are device pointers from alloc(); copies are
// synchronous with respect to the host buffers; sync() waits for all work.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "launch.h"

namespace slate_hip {

// ---------------------------------------------------------------------------
static std::mutex g_err_mu;
static std::string g_err;
static int g_err_code = 0;

void set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    std::lock_guard<std::mutex> lk(g_err_mu);
    if (g_err_code == 0) {           // keep the first error until cleared
        g_err_code = code ? code : -7;
        g_err = buf;
    }
    if (getenv("SLATE_HIP_VERBOSE")) fprintf(stderr, "slate_hip: %s\n", buf);
}

int error_code() {
    std::lock_guard<std::mutex> lk(g_err_mu);
    return g_err_code;
}

// ---------------------------------------------------------------------------
static std::once_flag g_init_once;
static int g_device = -1;
static hipStream_t g_stream = nullptr;
static bool g_ok = false;

// Device scratch of slate_hip_matmul_q4k_noalloc: the activation operand and
// the split-K partials of one call live here instead of in allocations.  In
// host code the array's name is only a stand-in for its device copy: every
// use goes through g_noalloc_scratch, the device address that
// hipGetSymbolAddress returns at initialisation (one device per process).
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(32) << 20;
static __device__ __align__(256) unsigned char noalloc_scratch[NOALLOC_SCRATCH_BYTES];
static void* g_noalloc_scratch = nullptr;

static void init_device() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        set_error(-7, "no HIP device available");
        return;
    }
    for (int d = 0; d < n; ++d) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, d) != hipSuccess) continue;
        if (strncmp(prop.gcnArchName, "gfx950", 6) == 0) { g_device = d; break; }
    }
    if (g_device < 0) {
        set_error(-5, "no gfx950 (MI355X) device found");
        return;
    }
    if (hipSetDevice(g_device) != hipSuccess ||
        hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) {
        set_error(-7, "cannot open device %d", g_device);
        return;
    }
    // with the backend device current: its copy of the no-allocation scratch
    const hipError_t es = hipGetSymbolAddress(&g_noalloc_scratch, HIP_SYMBOL(noalloc_scratch));
    if (es != hipSuccess) {
        g_noalloc_scratch = nullptr;
        set_error(-7, "no-allocation scratch unavailable: %s", hipGetErrorString(es));
        return;
    }
    g_ok = true;
}

// Make the backend device current on the calling thread.
static bool ensure() {
    std::call_once(g_init_once, init_device);
    if (!g_ok) return false;
    static thread_local bool bound = false;
    if (!bound) {
        if (hipSetDevice(g_device) != hipSuccess) return false;
        bound = true;
    }
    return true;
}

bool device_ok() { return ensure(); }
hipStream_t stream() { return ensure() ? g_stream : nullptr; }

static Knobs g_knobs;
static std::once_flag g_knobs_once;
static thread_local const Knobs* t_knobs = nullptr;

static int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v ? atoi(v) : dflt;
}

Knobs read_knobs() {
    Knobs k;
    k.attn_wave = env_int("SLATE_HIP_ATTN_WAVE", 1) != 0;
    k.attn_rope = env_int("SLATE_HIP_ATTN_ROPE", 1);
    if (k.attn_rope != 0 && k.attn_rope != 2) k.attn_rope = 1;
    k.attn_xcd = env_int("SLATE_HIP_ATTN_XCD", 1) != 0;
    k.attn_xcd_tamper = env_int("SLATE_HIP_ATTN_XCD_TAMPER", 0) != 0;
    k.attn_mfma = std::min(2, std::max(0, env_int("SLATE_HIP_ATTN_MFMA", 1)));
    k.q4k_w = env_int("SLATE_HIP_Q4K_W", 8) == 4 ? 4 : 8;
    k.q4k_r = env_int("SLATE_HIP_Q4K_R", 0);
    if (k.q4k_r != 1 && k.q4k_r != 2 && k.q4k_r != 4) k.q4k_r = 0;
    k.q4k_s = std::max(0, env_int("SLATE_HIP_Q4K_S", 0));
    k.q4k_wgs = std::max(1, env_int("SLATE_HIP_Q4K_WGS", 384));
    k.q4k_pf_s = std::max(0, env_int("SLATE_HIP_Q4K_PF_S", 0));
    k.q4k_pf_nt = env_int("SLATE_HIP_Q4K_PF_NT", 0);
    k.q4k_dec32 = env_int("SLATE_HIP_Q4K_DEC32", 1) != 0;
    k.q4k_early = env_int("SLATE_HIP_Q4K_EARLY", 0) != 0;
    k.gemv1 = env_int("SLATE_HIP_GEMV1", 1) != 0;
    k.row_pad64 = env_int("SLATE_HIP_ROW_PAD64", 0) != 0;
    k.q8_r = env_int("SLATE_HIP_Q8_R", 0);
    if (k.q8_r != 1 && k.q8_r != 2 && k.q8_r != 4) k.q8_r = 0;
    k.q8_s = std::max(0, env_int("SLATE_HIP_Q8_S", 0));
    k.q8_wgs = std::max(1, env_int("SLATE_HIP_Q8_WGS", 448));
    return k;
}

const Knobs& knobs() {
    if (t_knobs) return *t_knobs;
    std::call_once(g_knobs_once, [] { g_knobs = read_knobs(); });
    return g_knobs;
}

KnobScope::KnobScope(const Knobs* k) : prev_(t_knobs) { t_knobs = k; }
KnobScope::~KnobScope() { t_knobs = prev_; }

// Serialises multi-kernel entry sequences that share scratch buffers.
std::mutex g_enqueue_mu;

struct ScratchBuf { void* p = nullptr; size_t n = 0; };
static ScratchBuf g_scratch[8];

void* scratch(int slot, size_t bytes) {
    ScratchBuf& b = g_scratch[slot];
    if (b.n >= bytes) return b.p;
    (void)hipStreamSynchronize(g_stream);
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.n = 0;
    size_t want = bytes + bytes / 4 + 256;
    if (hipMalloc(&b.p, want) != hipSuccess) {
        set_error(-2, "scratch allocation of %zu bytes failed", want);
        return nullptr;
    }
    b.n = want;
    return b.p;
}

void build_rope_table(float* cs, int max_pos, int hd, float theta) {
    // Same float expressions as llama_infer.c:83-86 (glibc powf/cosf/sinf).
    const int half = hd / 2;
    for (int i = 0; i < half; ++i) {
        float inv_freq = powf(theta, -2.0f * (float)i / (float)hd);
        for (int p = 0; p < max_pos; ++p) {
            float ang = (float)p * inv_freq;
            cs[((size_t)p * half + i) * 2 + 0] = cosf(ang);
            cs[((size_t)p * half + i) * 2 + 1] = sinf(ang);
        }
    }
}

// Activation operand buffer for one Q4_K matmul input of B rows x K.
int make_act16(Act16& a, int B, int K, int slot) {
    a.rows = B;
    a.rows_pad = row_pad(B);
    a.K = K;
    a.frag = scratch(slot, act_frag_bytes(a.rows_pad, K));
    return a.frag ? 0 : -2;
}

// Activation operand buffer for one Q8_0 matmul input of B rows x K.
int make_act8(Act8& a, int B, int K, int slot) {
    a.rows = B;
    a.rows_pad = row_pad(B);
    a.K = K;
    a.frag = scratch(slot, act8_bytes(a.rows_pad, K));
    return a.frag ? 0 : -2;
}

}  // namespace slate_hip

using namespace slate_hip;

// ===========================================================================
// C ABI
extern "C" {

const char* slate_hip_last_error(void) {
    std::lock_guard<std::mutex> lk(g_err_mu);
    return g_err_code ? g_err.c_str() : nullptr;
}

void slate_hip_clear_error(void) {
    std::lock_guard<std::mutex> lk(g_err_mu);
    g_err_code = 0;
    g_err.clear();
}

void* slate_hip_stream(void) { return (void*)stream(); }

void* slate_hip_alloc(size_t bytes) {
    if (bytes == 0 || !ensure()) return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        set_error(-2, "alloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

void slate_hip_release(void* p) {
    if (!p || !ensure()) return;
    (void)hipStreamSynchronize(g_stream);
    if (hipFree(p) != hipSuccess) set_error(-7, "release(%p) failed", p);
}

void slate_hip_copy_h2d(void* dst, const void* src, size_t bytes) {
    if (!bytes || !ensure()) return;
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream) != hipSuccess ||
        hipStreamSynchronize(g_stream) != hipSuccess)
        set_error(-7, "copy_h2d(%zu) failed", bytes);
}

void slate_hip_copy_d2h(void* dst, const void* src, size_t bytes) {
    if (!bytes || !ensure()) return;
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream) != hipSuccess ||
        hipStreamSynchronize(g_stream) != hipSuccess)
        set_error(-7, "copy_d2h(%zu) failed", bytes);
}

void slate_hip_sync(void) {
    if (!ensure()) return;
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e != hipSuccess) set_error(-7, "sync failed: %s", hipGetErrorString(e));
}

void slate_hip_matvec(float* y, const float* A, const float* x, int M, int K) {
    if (!ensure()) return;
    if (!y || !A || !x || M <= 0 || K <= 0) { set_error(-1, "matvec: bad arguments"); return; }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    launch_mm_f32(y, x, A, 1, M, K, M, g_stream);
}

void slate_hip_linear_batch(float* C, const float* X, const float* W, int B, int K, int N) {
    if (!ensure()) return;
    if (!C || !X || !W || B <= 0 || K <= 0 || N <= 0) { set_error(-1, "linear_batch: bad arguments"); return; }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    launch_linear_batch(C, X, W, B, K, N, g_stream);
}

static int matmul_q4k_common(float* Y, const void* A, const float* X, int B, int M, int K, bool tiled) {
    if (!ensure()) return -7;
    SH_REQUIRE(Y && A && X && B > 0 && M > 0 && K > 0, "matmul_q4k: bad arguments");
    SH_REQUIRE(K % QK == 0, "matmul_q4k: K=%d is not a multiple of 256", K);
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    Q4kTarget t{A, M, 0};
    // one row: one GEMV kernel straight into Y (no operand, no partials)
    if (B <= GEMV_ROUTE_ROWS && ((uintptr_t)X & 15) == 0)
        return launch_q4k_gemv(&t, 1, tiled, X, K, B, K, Y, M, g_stream);
    if (B <= 16) {
        // one activation tile: the matmul makes its operand from X itself,
        // then the split sum (two kernels per call)
        const int max_splits = 32;
        float* part = (float*)scratch(1, (size_t)max_splits * 16 * M * sizeof(float));
        if (!part) return -2;
        int S = 1;
        const int rc = launch_q4k_conv(t, tiled, X, K, B, K, part, (int64_t)M, (int64_t)16 * M, max_splits, &S,
                                       g_stream);
        if (rc < 0) return rc;
        if (rc == 0) return launch_sum_splits(Y, part, S, B, 16, M, g_stream);
    }
    Act16 a;
    if (make_act16(a, B, K, 0)) return -2;
    int rc = launch_act16_from_f32(a, X, K, g_stream);
    if (rc) return rc;
    const int max_splits = 32;
    float* part = (float*)scratch(1, (size_t)max_splits * a.rows_pad * M * sizeof(float));
    if (!part) return -2;
    int S = 1;
    rc = launch_q4k(&t, 1, tiled, a, part, (int64_t)M, (int64_t)a.rows_pad * M, max_splits, &S, g_stream);
    if (rc) return rc;
    return launch_sum_splits(Y, part, S, B, a.rows_pad, M, g_stream);
}

int slate_hip_matmul_q4k(float* Y, const void* A, const float* X, int B, int M, int K) {
    return matmul_q4k_common(Y, A, X, B, M, K, false);
}

int slate_hip_matmul_q4k_tiled(float* Y, const void* A, const float* X, int B, int M, int K) {
    return matmul_q4k_common(Y, A, X, B, M, K, true);
}

int slate_hip_matmul_q4k_noalloc(float* Y, const void* A, const float* X, int B, int M, int K) {
    if (!ensure()) return -7;
    SH_REQUIRE(Y && A && X && B > 0 && M > 0 && K > 0, "matmul_q4k_noalloc: bad arguments");
    SH_REQUIRE(K % QK == 0, "matmul_q4k_noalloc: K=%d is not a multiple of 256", K);
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    Q4kTarget t{A, M, 0};
    if (B <= GEMV_ROUTE_ROWS && ((uintptr_t)X & 15) == 0)   // needs no scratch
        return launch_q4k_gemv(&t, 1, false, X, K, B, K, Y, M, g_stream);
    Act16 a;
    a.rows = B;
    a.rows_pad = row_pad(B);
    a.K = K;
    const size_t act_bytes = (act_frag_bytes(a.rows_pad, K) + 255) & ~size_t(255);
    const size_t split_bytes = (size_t)a.rows_pad * M * sizeof(float);
    if (act_bytes + split_bytes > NOALLOC_SCRATCH_BYTES) {
        set_error(-1, "matmul_q4k_noalloc: B=%d, M=%d, K=%d needs %zu bytes of scratch, above the %zu-byte limit",
                  B, M, K, act_bytes + split_bytes, NOALLOC_SCRATCH_BYTES);
        return -1;
    }
    // every split writes all of its partials and the operand covers every
    // padded row, so nothing left by an earlier call is read
    a.frag = g_noalloc_scratch;
    float* part = (float*)((char*)g_noalloc_scratch + act_bytes);
    const int max_splits = (int)std::min<size_t>(32, (NOALLOC_SCRATCH_BYTES - act_bytes) / split_bytes);
    int rc = launch_act16_from_f32(a, X, K, g_stream);
    if (rc) return rc;
    int S = 1;
    rc = launch_q4k(&t, 1, false, a, part, (int64_t)M, (int64_t)a.rows_pad * M, max_splits, &S, g_stream);
    if (rc) return rc;
    return launch_sum_splits(Y, part, S, B, a.rows_pad, M, g_stream);
}

int64_t slate_hip_q4k_tiled_bytes(int M, int K) {
    if (M <= 0 || K <= 0 || K % QK) return -1;
    return (int64_t)q4k_tiled_bytes(M, K);
}

int slate_hip_q4k_tile(void* dst, const void* src, int M, int K) {
    if (!ensure()) return -7;
    SH_REQUIRE(dst && src && M > 0 && K > 0 && K % QK == 0, "q4k_tile: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_q4k_tile(dst, src, M, K, g_stream);
}

void slate_hip_matvec_q4k(float* y, const void* A, const float* x, int M, int K) {
    slate_hip_matmul_q4k(y, A, x, 1, M, K);
}

int slate_hip_dequant_q4k(float* dst, const void* A, int64_t n) {
    if (!ensure()) return -7;
    SH_REQUIRE(dst && A && n >= 0 && n % QK == 0, "dequant_q4k: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_dequant_q4k(dst, A, n / QK, g_stream);
}

static int matmul_q8_common(float* Y, const void* A, const float* X, int B, int M, int K, bool tiled) {
    if (!ensure()) return -7;
    SH_REQUIRE(Y && A && X && B > 0 && M > 0 && K > 0, "matmul_q8_0: bad arguments");
    SH_REQUIRE(K % Q8_ELEMS == 0, "matmul_q8_0: K=%d is not a multiple of 32", K);
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    const void* W = A;
    int rc;
    if (!tiled) {   // regroup the row layout into the matmul's tiles first
        void* t = scratch(5, q8_tiled_bytes(M, K));
        if (!t) return -2;
        if ((rc = launch_q8_tile(t, A, M, K, g_stream))) return rc;
        W = t;
    }
    Act8 a;
    if (make_act8(a, B, K, 4)) return -2;
    if ((rc = launch_act8_from_f32(a, X, K, g_stream))) return rc;
    const int max_splits = 32;
    float* part = (float*)scratch(1, (size_t)max_splits * a.rows_pad * M * sizeof(float));
    if (!part) return -2;
    Q4kTarget t{W, M, 0};
    int S = 1;
    rc = launch_q8(&t, 1, a, part, (int64_t)M, (int64_t)a.rows_pad * M, max_splits, 0, &S, g_stream);
    if (rc) return rc;
    return launch_sum_splits(Y, part, S, B, a.rows_pad, M, g_stream);
}

int slate_hip_matmul_q8_0(float* Y, const void* A, const float* X, int B, int M, int K) {
    return matmul_q8_common(Y, A, X, B, M, K, false);
}

int slate_hip_matmul_q8_0_tiled(float* Y, const void* A, const float* X, int B, int M, int K) {
    return matmul_q8_common(Y, A, X, B, M, K, true);
}

void slate_hip_q8_0_matvec(float* y, const void* A, const float* x, int M, int K) {
    slate_hip_matmul_q8_0(y, A, x, 1, M, K);
}

int64_t slate_hip_q8_0_tiled_bytes(int M, int K) {
    if (M <= 0 || K <= 0 || K % Q8_ELEMS) return -1;
    return (int64_t)q8_tiled_bytes(M, K);
}

int slate_hip_q8_0_tile(void* dst, const void* src, int M, int K) {
    if (!ensure()) return -7;
    SH_REQUIRE(dst && src && M > 0 && K > 0 && K % Q8_ELEMS == 0, "q8_0_tile: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_q8_tile(dst, src, M, K, g_stream);
}

int slate_hip_dequant_q8_0(float* dst, const void* A, int64_t n) {
    if (!ensure()) return -7;
    SH_REQUIRE(dst && A && n >= 0 && n % Q8_ELEMS == 0, "dequant_q8_0: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_dequant_q8(dst, A, n / Q8_ELEMS, g_stream);
}

int slate_hip_rmsnorm_rows(float* y, const float* x, const float* w, int B, int D, float eps) {
    if (!ensure()) return -7;
    SH_REQUIRE(y && x && w && B > 0 && D > 0, "rmsnorm_rows: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_rmsnorm_rows(y, (float*)x, nullptr, 1, 0, w, B, D, eps, g_stream);
}

void slate_hip_rmsnorm_row(float* y, const float* x, const float* w, int D, float eps) {
    slate_hip_rmsnorm_rows(y, x, w, 1, D, eps);
}

void slate_hip_silu_mul(float* y, const float* gate, const float* up, int H) {
    if (!ensure()) return;
    if (!y || !gate || !up || H <= 0) { set_error(-1, "silu_mul: bad arguments"); return; }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    launch_silu_mul(y, gate, up, 1, H, 1, 0, H, H, g_stream);
}

void slate_hip_add_inplace(float* y, const float* x, int D) {
    if (!ensure()) return;
    if (!y || !x || D < 0) { set_error(-1, "add_inplace: bad arguments"); return; }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    launch_add(y, x, D, g_stream);
}

void slate_hip_embed_lookup(float* y, const float* W, int token_id, int D) {
    if (!ensure()) return;
    if (!y || !W || token_id < 0 || D <= 0) { set_error(-1, "embed_lookup: bad arguments"); return; }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    if (hipMemcpyAsync(y, W + (int64_t)token_id * D, (size_t)D * sizeof(float), hipMemcpyDeviceToDevice,
                       g_stream) != hipSuccess)
        set_error(-7, "embed_lookup copy failed");
}

void slate_hip_attention_step(float* out, const float* q, const float* K, const float* V, float* scores,
                              int L, int D) {
    if (!ensure()) return;
    if (!out || !q || !K || !V || !scores || L <= 0 || D <= 0) {
        set_error(-1, "attention_step: bad arguments");
        return;
    }
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    launch_attention_step(out, q, K, V, scores, L, D, g_stream);
}

int slate_hip_argmax_rows(int32_t* out, const float* logits, int B, int V) {
    if (!ensure()) return -7;
    SH_REQUIRE(out && logits && B > 0 && V > 0, "argmax_rows: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    void* ws = scratch(6, argmax_workspace_bytes(B, V));
    if (!ws) return -2;
    // without a row factor the kernels only read the logits
    return launch_argmax_rows(out, const_cast<float*>(logits), B, V, ws, g_stream);
}

struct RopeTable { float* dev = nullptr; int max_pos = 0; };
static std::map<std::pair<int, uint32_t>, RopeTable> g_rope;

int slate_hip_rope_rows(float* x, const int32_t* pos, int n_rows, int n_heads, int head_dim,
                        float theta_base, int max_pos) {
    if (!ensure()) return -7;
    SH_REQUIRE(x && pos && n_rows > 0 && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && max_pos > 0,
               "rope_rows: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    uint32_t tb;
    memcpy(&tb, &theta_base, 4);
    RopeTable& t = g_rope[{head_dim, tb}];
    if (t.max_pos < max_pos) {
        std::vector<float> host((size_t)max_pos * head_dim);
        build_rope_table(host.data(), max_pos, head_dim, theta_base);
        (void)hipStreamSynchronize(g_stream);
        if (t.dev) (void)hipFree(t.dev);
        t.dev = nullptr;
        t.max_pos = 0;
        SH_CHECK_HIP(hipMalloc(&t.dev, host.size() * sizeof(float)));
        SH_CHECK_HIP(hipMemcpy(t.dev, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice));
        t.max_pos = max_pos;
    }
    int* bad = (int*)scratch(2, 256);
    if (!bad) return -2;
    SH_CHECK_HIP(hipMemsetAsync(bad, 0, sizeof(int), g_stream));
    int rc = launch_rope_rows(x, pos, n_rows, n_heads, head_dim, t.dev, max_pos, bad, g_stream);
    if (rc) return rc;
    int hbad = 0;
    SH_CHECK_HIP(hipMemcpyAsync(&hbad, bad, sizeof(int), hipMemcpyDeviceToHost, g_stream));
    SH_CHECK_HIP(hipStreamSynchronize(g_stream));
    SH_REQUIRE(hbad == 0, "rope_rows: %d rows with |pos| >= max_pos=%d left unrotated", hbad, max_pos);
    return 0;
}

void slate_hip_rope_table(float* cs, int max_pos, int head_dim, float theta_base) {
    build_rope_table(cs, max_pos, head_dim, theta_base);
}

int slate_hip_pack_batch(const int32_t* slot, const int32_t* pos0, const int32_t* n_new, int B, int max_seq,
                         int64_t slot_stride, int T_cap, int32_t* tok_off, int32_t* tok2seq, int32_t* tok_pos,
                         int64_t* kv_base, int32_t* last_tok, int32_t* status) {
    if (!ensure()) return -7;
    SH_REQUIRE(slot && pos0 && n_new && B >= 1 && B <= 1024 && tok_off && tok2seq && tok_pos && kv_base &&
                   last_tok && status && T_cap >= 1,
               "pack_batch: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_pack_batch(slot, pos0, n_new, B, max_seq, slot_stride, T_cap, tok_off, tok2seq, tok_pos,
                             kv_base, last_tok, status, g_stream);
}

int slate_hip_attention_ragged(float* out, const float* q, const float* Kpool, const float* Vpool,
                               const int32_t* tok2seq, const int32_t* tok_pos, const int64_t* kv_base, int T,
                               int n_q_heads, int n_kv_heads, int head_dim, int64_t head_stride, int max_pos) {
    if (!ensure()) return -7;
    SH_REQUIRE(out && q && Kpool && Vpool && tok2seq && tok_pos && kv_base && T > 0 && max_pos > 0,
               "attention_ragged: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    size_t nf = attention_partial_floats(T, n_q_heads, head_dim, max_pos);
    float* po = (float*)scratch(3, nf * sizeof(float));
    if (!po) return -2;
    float* pml = po + (size_t)T * n_q_heads * ((max_pos + attn_chunk_size() - 1) / attn_chunk_size()) * head_dim;
    return launch_attention_ragged(out, q, Kpool, Vpool, tok2seq, tok_pos, kv_base, T, n_q_heads, n_kv_heads,
                                   head_dim, head_stride, max_pos, po, pml, g_stream);
}

int slate_hip_synth_f32(float* dst, int64_t n, uint64_t seed, float std) {
    if (!ensure()) return -7;
    SH_REQUIRE(dst && n >= 0, "synth_f32: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_synth_f32(dst, n, seed, std, 0.f, g_stream);
}

int slate_hip_synth_q4k(void* dst, int64_t rows, int64_t cols, uint64_t seed, float std) {
    if (!ensure()) return -7;
    SH_REQUIRE(dst && rows >= 0 && cols > 0, "synth_q4k: bad arguments");
    std::lock_guard<std::mutex> lk(g_enqueue_mu);
    return launch_synth_q4k(dst, rows, cols, seed, std, g_stream);
}

static const char* hip_last_error_entry(void) { return slate_hip_last_error(); }

static slate_hip_backend_t g_vtable = {
    {
        "hip",
        slate_hip_alloc,
        slate_hip_release,
        slate_hip_copy_h2d,
        slate_hip_copy_d2h,
        slate_hip_matvec,
        slate_hip_linear_batch,
        slate_hip_matvec_q4k,
        slate_hip_rmsnorm_row,
        slate_hip_silu_mul,
        slate_hip_add_inplace,
        slate_hip_embed_lookup,
        slate_hip_attention_step,
        slate_hip_sync,
    },
    slate_hip_matmul_q4k,
    slate_hip_dequant_q4k,
    slate_hip_rmsnorm_rows,
    slate_hip_rope_rows,
    slate_hip_argmax_rows,
    hip_last_error_entry,
};

const slate_backend_t* slate_backend_hip(void) {
    if (!ensure()) return nullptr;
    return &g_vtable.base;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Compatibility vtable (slate_backend_hip_compat): the same kernels for
// callers that treat backend memory as host memory, like slate's toy engine
// (src/infer/engine.c memcpy's and memset's its KV cache, engine.c:411-412,
// 586-591, and hands module weights, which live in ordinary host memory,
// straight to the compute entries).  alloc returns pinned host memory that
// the device addresses directly; a compute entry runs its kernel on device
// views of its arguments -- device and pinned memory as they are, any
// other (pageable) host range copied into a temporary device buffer and,
// for outputs, back -- and waits for the kernel before returning, since
// such callers read the results at once.  Correct and slow.

namespace {

struct CompatArg { const void* host; void* dev; size_t bytes; bool out; bool own; };

class CompatCall {
  public:
    ~CompatCall() { finish(); }
    // A device view of [p, p + bytes) for a kernel argument read (in)
    // and/or written (out); the same pointer passed twice gets one view.
    template <class T>
    T* arg(T* p, size_t bytes, bool in, bool out) {
        if (!p || !ok_) return p;
        for (auto& a : args_)
            if (a.host == (const void*)p) {
                a.out = a.out || out;
                return (T*)a.dev;
            }
        hipPointerAttribute_t at{};
        if (hipPointerGetAttributes(&at, (const void*)p) == hipSuccess &&
            (at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeHost) && at.devicePointer) {
            args_.push_back({(const void*)p, at.devicePointer, bytes, false, false});
            return (T*)at.devicePointer;
        }
        (void)hipGetLastError();   // an unregistered pointer is not an error here
        void* d = nullptr;
        if (hipMalloc(&d, bytes ? bytes : 1) != hipSuccess ||
            (in && bytes && hipMemcpy(d, (const void*)p, bytes, hipMemcpyHostToDevice) != hipSuccess)) {
            if (d) (void)hipFree(d);
            set_error(-7, "compat backend: staging %zu bytes failed", bytes);
            ok_ = false;
            return nullptr;
        }
        args_.push_back({(const void*)p, d, bytes, out, true});
        return (T*)d;
    }
    bool ok() const { return ok_; }
    // wait for the kernels, copy staged outputs back, free the staging
    void finish() {
        if (done_) return;
        done_ = true;
        if (hipStreamSynchronize(stream()) != hipSuccess) set_error(-7, "compat backend: kernel failed");
        for (auto& a : args_) {
            if (!a.own) continue;
            if (ok_ && a.out && a.bytes &&
                hipMemcpy((void*)a.host, a.dev, a.bytes, hipMemcpyDeviceToHost) != hipSuccess)
                set_error(-7, "compat backend: copy back of %zu bytes failed", a.bytes);
            (void)hipFree(a.dev);
        }
    }

  private:
    std::vector<CompatArg> args_;
    bool ok_ = true, done_ = false;
};

void* compat_alloc(size_t bytes) {
    if (!bytes || !ensure()) return nullptr;
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
        set_error(-2, "compat alloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

void compat_release(void* p) {
    if (!p || !ensure()) return;
    (void)hipStreamSynchronize(stream());
    if (hipHostFree(p) != hipSuccess) set_error(-7, "compat release(%p) failed", p);
}

void compat_copy(void* dst, const void* src, size_t bytes) {
    if (!bytes || !ensure()) return;
    (void)hipStreamSynchronize(stream());
    if (hipMemcpy(dst, src, bytes, hipMemcpyDefault) != hipSuccess) set_error(-7, "compat copy(%zu) failed", bytes);
}

void compat_matvec(float* y, const float* A, const float* x, int M, int K) {
    if (!ensure() || M <= 0 || K <= 0) { slate_hip_matvec(y, A, x, M, K); return; }
    CompatCall c;
    float* dy = c.arg(y, (size_t)M * 4, false, true);
    const float* dA = c.arg(A, (size_t)M * K * 4, true, false);
    const float* dx = c.arg(x, (size_t)K * 4, true, false);
    if (c.ok()) slate_hip_matvec(dy, dA, dx, M, K);
}

void compat_linear_batch(float* C, const float* X, const float* W, int B, int K, int N) {
    if (!ensure() || B <= 0 || K <= 0 || N <= 0) { slate_hip_linear_batch(C, X, W, B, K, N); return; }
    CompatCall c;
    float* dC = c.arg(C, (size_t)B * N * 4, false, true);
    const float* dX = c.arg(X, (size_t)B * K * 4, true, false);
    const float* dW = c.arg(W, (size_t)K * N * 4, true, false);
    if (c.ok()) slate_hip_linear_batch(dC, dX, dW, B, K, N);
}

void compat_matvec_q4k(float* y, const void* A, const float* x, int M, int K) {
    if (!ensure() || M <= 0 || K <= 0 || K % QK) { slate_hip_matvec_q4k(y, A, x, M, K); return; }
    CompatCall c;
    float* dy = c.arg(y, (size_t)M * 4, false, true);
    const void* dA = c.arg(A, (size_t)M * (K / QK) * QBLOCK, true, false);
    const float* dx = c.arg(x, (size_t)K * 4, true, false);
    if (c.ok()) slate_hip_matvec_q4k(dy, dA, dx, M, K);
}

void compat_rmsnorm_row(float* y, const float* x, const float* w, int D, float eps) {
    if (!ensure() || D <= 0) { slate_hip_rmsnorm_row(y, x, w, D, eps); return; }
    CompatCall c;
    float* dy = c.arg(y, (size_t)D * 4, false, true);
    const float* dx = c.arg(x, (size_t)D * 4, true, false);
    const float* dw = c.arg(w, (size_t)D * 4, true, false);
    if (c.ok()) slate_hip_rmsnorm_row(dy, dx, dw, D, eps);
}

void compat_silu_mul(float* y, const float* gate, const float* up, int H) {
    if (!ensure() || H <= 0) { slate_hip_silu_mul(y, gate, up, H); return; }
    CompatCall c;   // y == gate (in place, llama_infer.c:192) shares one view
    const float* dg = c.arg(gate, (size_t)H * 4, true, false);
    const float* du = c.arg(up, (size_t)H * 4, true, false);
    float* dy = c.arg(y, (size_t)H * 4, false, true);
    if (c.ok()) slate_hip_silu_mul(dy, dg, du, H);
}

void compat_add_inplace(float* y, const float* x, int D) {
    if (!ensure() || D <= 0) { slate_hip_add_inplace(y, x, D); return; }
    CompatCall c;
    float* dy = c.arg(y, (size_t)D * 4, true, true);
    const float* dx = c.arg(x, (size_t)D * 4, true, false);
    if (c.ok()) slate_hip_add_inplace(dy, dx, D);
}

void compat_embed_lookup(float* y, const float* W, int token_id, int D) {
    if (!ensure() || !W || token_id < 0 || D <= 0) { slate_hip_embed_lookup(y, W, token_id, D); return; }
    CompatCall c;   // only the looked-up row of the table is staged
    float* dy = c.arg(y, (size_t)D * 4, false, true);
    const float* dW = c.arg(W + (int64_t)token_id * D, (size_t)D * 4, true, false);
    if (c.ok()) slate_hip_embed_lookup(dy, dW, 0, D);
}

void compat_attention_step(float* out, const float* q, const float* K, const float* V, float* scores, int L,
                           int D) {
    if (!ensure() || L <= 0 || D <= 0) { slate_hip_attention_step(out, q, K, V, scores, L, D); return; }
    CompatCall c;
    float* dout = c.arg(out, (size_t)D * 4, false, true);
    const float* dq = c.arg(q, (size_t)D * 4, true, false);
    const float* dK = c.arg(K, (size_t)L * D * 4, true, false);
    const float* dV = c.arg(V, (size_t)L * D * 4, true, false);
    float* ds = c.arg(scores, (size_t)L * 4, false, true);
    if (c.ok()) slate_hip_attention_step(dout, dq, dK, dV, ds, L, D);
}

const slate_backend_t g_compat = {
    "hip-compat",      compat_alloc,       compat_release,      compat_copy,
    compat_copy,       compat_matvec,      compat_linear_batch, compat_matvec_q4k,
    compat_rmsnorm_row, compat_silu_mul,   compat_add_inplace,  compat_embed_lookup,
    compat_attention_step, slate_hip_sync,
};

}  // namespace

extern "C" {

const slate_backend_t* slate_backend_hip_compat(void) {
    if (!ensure()) return nullptr;
    return &g_compat;
}

}  // extern "C"
