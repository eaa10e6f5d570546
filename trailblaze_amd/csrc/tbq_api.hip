// tbq_api.hip -- the extern "C" device API of libtbq (include/tbq.h): input
// validation on the host, then the gfx950 launchers.  Nothing here falls back
// to the CPU: an input the kernels do not cover returns 0 with a reason.
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "../../include/tbq.h"
#include "tbq_device.hpp"
#include "tbq_kernels.h"

using namespace tbq;

namespace {

thread_local char g_err[512] = "";
std::once_flag g_init_once;
int g_ready = 0;
int g_cu = 0;
char g_name[256] = "";

std::mutex g_ws_mu;
void *g_ws = nullptr;
size_t g_ws_bytes = 0;
void *g_route = nullptr;
size_t g_route_bytes = 0;
void *g_part = nullptr;   // partial sums of matvecs with rows longer than TBQ_MAX_K
size_t g_part_bytes = 0;

int fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return 0;
}

int hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return 1;
    return fail("%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Plain ids are the reference's layouts; QT_GGML | id is ggml's layout of
// the same format (TBQ_GGML in tbq.h).
bool known_qtype(int qt) {
    switch (canon_qt(qt)) {
    case QT_F32: case QT_F16: case QT_BF16: case QT_Q4_0: case QT_Q8_0: case QT_Q2_K:
    case QT_Q3_K: case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: case QT_Q8_K:
    case QT_GF16: case QT_GQ4_0: case QT_GQ8_0: case QT_GQ2_K: case QT_GQ3_K:
    case QT_GQ4_K: case QT_GQ5_K: case QT_GQ6_K:
        return true;
    default:
        return false;
    }
}

hipStream_t S(void *s) { return reinterpret_cast<hipStream_t>(s); }

// TBQ_FORCE_NO_DEVICE=1 in the environment (read at the first call) makes
// libtbq behave as on a host without a GPU: tbq_init and every call that
// needs the device return 0, so tb_cuda_init returns 0, uploads return NULL
// and tb_cuda_matvec_device returns 0 -- the caller's CPU fallback
// (layer4/tb_gguf.c:444-451) -- without any HIP call.
bool forced_no_device() {
    const char *v = getenv("TBQ_FORCE_NO_DEVICE");
    return v && *v && strcmp(v, "0") != 0;
}

int ensure_init() {
    static const bool forced = forced_no_device();
    if (forced) return fail("no HIP device available (TBQ_FORCE_NO_DEVICE is set)");
    std::call_once(g_init_once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return;
        if (hipSetDevice(0) != hipSuccess) return;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, 0) != hipSuccess) return;
        g_cu = p.multiProcessorCount;
        snprintf(g_name, sizeof g_name, "%s (%s)", p.name, p.gcnArchName);
        g_ready = 1;
    });
    if (!g_ready) return fail("no HIP device available");
    return 1;
}

}  // namespace

extern "C" {

int tbq_init(void) { return ensure_init(); }
const char *tbq_last_error(void) { return g_err; }

// Error setter for libtbq's C11 host files (hidden: not part of the ABI).
__attribute__((visibility("hidden"))) int tbq_host_fail(const char *msg) { return fail("%s", msg); }
// Synchronous zero fill for the C11 host files (hidden).
__attribute__((visibility("hidden"))) int tbq_host_zero(void *dev, size_t bytes) {
    if (!dev) return fail("tbq_host_zero: null pointer");
    return hip_ok(hipMemset(dev, 0, bytes), "hipMemset");
}
const char *tbq_device_name(void) { return g_name; }
int tbq_cu_count(void) { return g_cu; }

void *tbq_malloc(size_t bytes) {
    if (!ensure_init()) return nullptr;
    void *p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
    return p;
}
int tbq_free(void *p) { return p ? hip_ok(hipFree(p), "hipFree") : 1; }
int tbq_memcpy_h2d(void *d, const void *h, size_t n, void *s) {
    return hip_ok(hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, S(s)), "hipMemcpyAsync H2D");
}
int tbq_memcpy_d2h(void *h, const void *d, size_t n, void *s) {
    return hip_ok(hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, S(s)), "hipMemcpyAsync D2H");
}
int tbq_stream_sync(void *s) { return hip_ok(hipStreamSynchronize(S(s)), "hipStreamSynchronize"); }
int tbq_device_sync(void) { return hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

size_t tbq_row_bytes(int qt, int K) {
    if (!known_qtype(qt) || K < 0) return 0;
    int bw = block_weights(qt), bb = block_bytes(qt);
    return (size_t)((K + bw - 1) / bw) * (size_t)bb;
}

int tbq_qtype_supported(int qt) { return known_qtype(qt) ? 1 : 0; }

int tbq_dequant(const void *W, int qt, int nrows, int K, float *out, void *s) {
    if (!ensure_init()) return 0;
    qt = canon_qt(qt);
    if (!known_qtype(qt)) return fail("tbq_dequant: unsupported qtype %d", qt);
    if (nrows < 0 || K <= 0 || K % block_weights(qt) || K % 8) return fail("tbq_dequant: K=%d not a multiple of the block size", K);
    if (!W || !out || !aligned16(out)) return fail("tbq_dequant: null or misaligned pointer");
    if (nrows == 0) return 1;
    return hip_ok(launch_dequant(qt, W, (long long)nrows * K, out, S(s)), "dequant launch");
}

static int check_matvec(const void *W, int qt, int M, int K, const float *x, const float *y) {
    if (!known_qtype(qt)) return fail("unsupported qtype %d", qt);
    int chunk = block_weights(qt) == 256 ? 256 : 32;
    if (M < 0 || K <= 0 || K % chunk) return fail("K=%d must be a positive multiple of %d for qtype %d", K, chunk, qt);
    if (!W || !x || !y) return fail("null pointer");
    if (!aligned16(x)) return fail("x must be 16-byte aligned");
    if (((qt & 0xFF) == QT_Q4_K || (qt & 0xFF) == QT_Q5_K || qt == QT_F32) && !aligned16(W))
        return fail("W must be 16-byte aligned for qtype %d", qt);
    if (((uintptr_t)W & 1u)) return fail("W must be 2-byte aligned");
    return 1;
}

// Rows longer than TBQ_MAX_K (x is staged in LDS): column slices of
// TBQ_MAX_K weights through the K-quant kernel with the full row stride,
// the first into y, the others into a library-owned partial buffer (grown
// on demand, so such calls must be ordered on one stream), then y plus the
// partials in slice order.
static int matvec_long_rows(const void *W, int qt, int M, int K, const float *x, float *y, hipStream_t st) {
    const int S = (K + TBQ_MAX_K - 1) / TBQ_MAX_K;
    const long long rb = (long long)tbq_row_bytes(qt, K);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    const size_t need = (size_t)(S - 1) * M * 4;
    if (g_part_bytes < need) {
        if (g_part && !hip_ok(hipFree(g_part), "hipFree")) return 0;
        g_part = nullptr;
        g_part_bytes = 0;
        if (!hip_ok(hipMalloc(&g_part, need), "hipMalloc matvec partials")) return 0;
        g_part_bytes = need;
    }
    for (int sl = 0; sl < S; sl++) {
        const int k0 = sl * TBQ_MAX_K, ks = K - k0 < TBQ_MAX_K ? K - k0 : TBQ_MAX_K;
        MvPro pro{};
        pro.rb = rb;
        const uint8_t *Ws = (const uint8_t *)W + tbq_row_bytes(qt, k0);
        float *ys = sl == 0 ? y : (float *)g_part + (size_t)(sl - 1) * M;
        hipError_t e = launch_matvec_kq_pro(PRO_NONE, pro, qt, Ws, M, ks, x + k0, ys, st, g_cu);
        if (e == hipErrorNotSupported)
            return fail("tbq_matvec: no kernel for qtype %d with rows of K=%d (slices of %d)", qt, K, TBQ_MAX_K);
        if (!hip_ok(e, "matvec launch (long rows)")) return 0;
    }
    return hip_ok(launch_add_rows(y, (const float *)g_part, S - 1, M, st), "matvec slice sum");
}

int tbq_matvec_variant(const void *W, int qt, int M, int K, const float *x, float *y, int variant, void *s) {
    if (!ensure_init()) return 0;
    qt = canon_qt(qt);
    if (!check_matvec(W, qt, M, K, x, y)) return 0;
    if (variant < TBQ_MV_AUTO || variant > TBQ_MV_KQ) return fail("tbq_matvec_variant: unknown variant %d", variant);
    if (M == 0) return 1;
    if (K > TBQ_MAX_K) {
        if (variant != TBQ_MV_AUTO && variant != TBQ_MV_KQ)
            return fail("tbq_matvec_variant: rows of K=%d above %d take the K-quant kernel only", K, TBQ_MAX_K);
        return matvec_long_rows(W, qt, M, K, x, y, S(s));
    }
    // The specialised Q4_K kernels keep x's digits in registers for rows of
    // up to 64 units: one pass of two rows per wave up to 8192 rows,
    // persistent waves walking the rows of taller matrices; longer rows
    // stream through the shared K-quant kernel, and so do taller matrices of
    // 17..63 units per row that are not a power of two, whose segmented
    // mapping keeps every lane busy (151936x2560: 41.6 against 50.2 us,
    // 151936x1536: 28.6 against 30.0-30.7), and
    // matrices of 64-unit rows above 32768 rows (151936x4096: 65.6-66.3
    // against 67.8 us).
    const int U = K / 64;
    const bool seg_rows = (U > 16 && U < 64 && (U & (U - 1)) != 0 && M > 8192) || (U == 64 && M > 32768);
    const bool q4k_special = (qt == QT_Q4_K || qt == QT_GQ4_K) &&
                             (variant == TBQ_MV_INTDOT || (variant == TBQ_MV_AUTO && K <= 4096 && !seg_rows));
    if (q4k_special) {
        hipError_t e = launch_matvec_q4k(W, M, K, x, y, S(s), g_cu, qt == QT_GQ4_K);
        if (e != hipErrorNotSupported) return hip_ok(e, "matvec launch (Q4_K int-dot)");
    }
    if (variant == TBQ_MV_AUTO || variant == TBQ_MV_KQ) {
        hipError_t e = launch_matvec_kq(qt, W, M, K, x, y, S(s), g_cu);
        if (e != hipErrorNotSupported) return hip_ok(e, "matvec launch (int-dot)");
    }
    if (variant == TBQ_MV_INTDOT || variant == TBQ_MV_KQ)
        return fail("tbq_matvec_variant: no int-dot kernel for qtype %d K=%d", qt, K);
    if ((size_t)K * 4 + (size_t)(K / 16) * 4 > 64 * 1024)
        return fail("K=%d exceeds the LDS-resident x limit of the fma kernel", K);
    return hip_ok(launch_matvec_generic(qt, W, M, K, x, y, S(s), g_cu), "matvec launch");
}

int tbq_matvec(const void *W, int qt, int M, int K, const float *x, float *y, void *s) {
    return tbq_matvec_variant(W, qt, M, K, x, y, TBQ_MV_AUTO, s);
}

// Router arrival counters live at the start of every workspace, sized for
// the largest T, so their position does not depend on T.  They are zero on
// entry to every call and left zero on exit.
constexpr int MAX_TOKENS = 65536;
constexpr size_t COUNTER_BYTES = (size_t)MAX_TOKENS * 4;

// For the C11 host files (hidden): the counter area of a MoE workspace.
__attribute__((visibility("hidden"))) size_t tbq_moe_counter_bytes(void) { return COUNTER_BYTES; }

int tbq_route(const float *xn, const float *router, const float *bias, int T, int H, int E, int top_k,
              int *sel_idx, float *sel_w, void *s) {
    if (!ensure_init()) return 0;
    if (T < 0 || H <= 0 || H % 8 || E <= 0 || E > 256 || top_k <= 0)
        return fail("tbq_route: bad shape T=%d H=%d E=%d k=%d", T, H, E, top_k);
    if ((size_t)H * 4 + 1024 > 60 * 1024) return fail("tbq_route: H=%d too large", H);
    if (!xn || !router || !sel_idx || !sel_w || !aligned16(xn) || !aligned16(router))
        return fail("tbq_route: null or misaligned pointer");
    if (T == 0) return 1;
    if (T > MAX_TOKENS) return fail("tbq_route: T=%d above %d", T, MAX_TOKENS);
    std::lock_guard<std::mutex> lk(g_ws_mu);
    const size_t need = COUNTER_BYTES + (size_t)T * E * 4;
    if (g_route_bytes < need) {
        if (g_route && !hip_ok(hipFree(g_route), "hipFree")) return 0;
        g_route = nullptr;
        g_route_bytes = 0;
        if (!hip_ok(hipMalloc(&g_route, need), "hipMalloc router logits")) return 0;
        if (!hip_ok(hipMemset(g_route, 0, COUNTER_BYTES), "hipMemset router counters")) return 0;
        g_route_bytes = need;
    }
    unsigned *counters = (unsigned *)g_route;
    float *logits = (float *)((char *)g_route + COUNTER_BYTES);
    hipError_t e = launch_router(xn, router, bias, T, H, E, top_k, logits, counters, sel_idx, sel_w, S(s));
    if (e == hipErrorNotSupported) e = launch_route(xn, router, bias, T, H, E, top_k, sel_idx, sel_w, S(s));
    return hip_ok(e, "route launch");
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }


// The qtypes of a layer's gate, up and down tensors (a zero field means
// L->qtype, as in layer4/tb_infer.c:807-816 each tensor carries its own).
struct MoeQts {
    int g, u, d;
};
static MoeQts moe_qts(const tbq_moe_layer *L) {
    return {L->qt_gate ? L->qt_gate : L->qtype, L->qt_up ? L->qt_up : L->qtype,
            L->qt_down ? L->qt_down : L->qtype};
}

size_t tbq_moe_workspace_size(const tbq_moe_layer *L, int T, int mode) {
    if (!L || T <= 0) return 0;
    int k = L->top_k > 8 ? 8 : L->top_k;
    const MoeQts q = moe_qts(L);
    size_t n = COUNTER_BYTES;
    n += align256((size_t)T * 8 * 4) * 2;                   // sel idx / w
    n += align256((size_t)T * L->E * 4);                     // router logits
    n += align256((size_t)T * k * L->F * 4);                 // act
    n += align256((size_t)T * k * L->H * 4);                 // y
    n += align256((size_t)(2 + 3 * L->E + T * k) * 4);       // decode order by expert
    if (q.g != q.u) n += align256((size_t)T * k * L->F * 4); // up products (gate and up run apart)
    if (mode == TBQ_MOE_BF16) n += align256(prefill_workspace_bytes(T, k, L->E, L->H, L->F));
    if (mode == TBQ_MOE_I8) n += align256(prefill_i8_workspace_bytes(T, k, L->E, L->H, L->F));
    return n;
}

static bool moe_expert_qtype(int qt) {
    switch (qt) {
    case QT_Q2_K: case QT_Q3_K: case QT_Q4_K: case QT_Q5_K: case QT_Q6_K: case QT_Q8_0:
    case QT_GQ2_K: case QT_GQ3_K: case QT_GQ4_K: case QT_GQ5_K: case QT_GQ6_K: case QT_GQ8_0: return true;
    default: return false;
    }
}

static int check_moe(const tbq_moe_layer *L, int T) {
    if (!L) return fail("tbq_moe_forward: null layer");
    if (T < 0 || T > MAX_TOKENS || L->E <= 0 || L->E > 256 || L->top_k <= 0) return fail("tbq_moe_forward: bad T/E/top_k");
    if (L->H <= 0 || L->F <= 0 || L->H % 256 || L->F % 256) return fail("tbq_moe_forward: H and F must be multiples of 256");
    const MoeQts q = moe_qts(L);
    if (!moe_expert_qtype(q.g) || !moe_expert_qtype(q.u) || !moe_expert_qtype(q.d))
        return fail("tbq_moe_forward: expert qtypes gate %d, up %d, down %d: each must be Q2_K, Q3_K, Q4_K, Q5_K, "
                    "Q6_K or Q8_0 (either layout)", q.g, q.u, q.d);
    if (!L->router || !L->gate || !L->up || !L->down) return fail("tbq_moe_forward: null weight");
    if (!aligned16(L->router) || !aligned16(L->gate) || !aligned16(L->up) || !aligned16(L->down))
        return fail("tbq_moe_forward: weights must be 16-byte aligned");
    if ((size_t)L->H * 4 + (size_t)L->H / 4 > 60 * 1024) return fail("tbq_moe_forward: H too large");
    return 1;
}

// The prefill MFMA modes take layers whose three expert tensors are Q4_K in
// the reference's layout, and the fp16 one also all three in ggml's.
static bool moe_mode_ok(const tbq_moe_layer *L, int mode) {
    if (mode == TBQ_MOE_FP32) return true;
    if (mode != TBQ_MOE_BF16 && mode != TBQ_MOE_I8) return false;
    const MoeQts q = moe_qts(L);
    const bool ref = q.g == QT_Q4_K && q.u == QT_Q4_K && q.d == QT_Q4_K;
    const bool gg = mode == TBQ_MOE_BF16 && q.g == QT_GQ4_K && q.u == QT_GQ4_K && q.d == QT_GQ4_K;
    return (ref || gg) && gemm_k_supported(L->H) && gemm_k_supported(L->F);
}

int tbq_moe_mode_supported(const tbq_moe_layer *L, int mode) {
    if (!L) return 0;
    g_err[0] = 0;
    if (!check_moe(L, 1)) return 0;
    return moe_mode_ok(L, mode) ? 1 : 0;
}

int tbq_moe_forward(const tbq_moe_layer *L, int T, const float *xn, const float *resid, float *out, int *sel_idx,
                    float *sel_w, void *workspace, size_t ws_bytes, int mode, void *s) {
    if (!ensure_init()) return 0;
    if (!check_moe(L, T)) return 0;
    if (mode != TBQ_MOE_FP32 && mode != TBQ_MOE_BF16 && mode != TBQ_MOE_I8)
        return fail("tbq_moe_forward: unknown mode %d", mode);
    if (!moe_mode_ok(L, mode))
        return fail("tbq_moe_forward: the prefill MFMA modes take layers whose gate, up and down are all Q4_K "
                    "(the reference's layout; TBQ_MOE_BF16 also ggml's) with H and F in {256, 512, 768, 1024, "
                    "1536, 2048, 3072, 4096}; use TBQ_MOE_FP32 for this layer");
    if (!xn || !resid || !out || !aligned16(xn) || !aligned16(resid) || !aligned16(out))
        return fail("tbq_moe_forward: null or misaligned activation pointer");
    if (T == 0) return 1;
    size_t need = tbq_moe_workspace_size(L, T, mode);
    std::unique_lock<std::mutex> lk(g_ws_mu, std::defer_lock);
    char *ws = (char *)workspace;
    if (!ws) {
        lk.lock();
        if (g_ws_bytes < need) {
            if (g_ws && !hip_ok(hipFree(g_ws), "hipFree")) return 0;
            g_ws = nullptr;
            g_ws_bytes = 0;
            if (!hip_ok(hipMalloc(&g_ws, need), "hipMalloc workspace")) return 0;
            if (!hip_ok(hipMemset(g_ws, 0, COUNTER_BYTES), "hipMemset workspace")) return 0;
            g_ws_bytes = need;
        }
        ws = (char *)g_ws;
    } else if (ws_bytes < need) {
        return fail("tbq_moe_forward: workspace %zu < %zu bytes", ws_bytes, need);
    }
    const MoeQts q = moe_qts(L);
    MoeArgs a;
    a.T = T; a.H = L->H; a.F = L->F; a.E = L->E; a.top_k = L->top_k;
    a.k = L->top_k > 8 ? 8 : L->top_k;
    a.qg = q.g; a.qu = q.u; a.qd = q.d;
    a.xn = xn; a.resid = resid; a.router = L->router; a.bias = L->bias;
    a.gate = L->gate; a.up = L->up; a.down = L->down; a.out = out;
    size_t off = 0;
    a.counters = (unsigned *)(ws + off); off += COUNTER_BYTES;
    int *ws_idx = (int *)(ws + off); off += align256((size_t)T * 8 * 4);
    float *ws_w = (float *)(ws + off); off += align256((size_t)T * 8 * 4);
    a.logits = (float *)(ws + off); off += align256((size_t)T * a.E * 4);
    a.act = (float *)(ws + off); off += align256((size_t)T * a.k * a.F * 4);
    a.y = (float *)(ws + off); off += align256((size_t)T * a.k * a.H * 4);
    a.grp = (int *)(ws + off); off += align256((size_t)(2 + 3 * a.E + T * a.k) * 4);
    a.u = nullptr;
    if (q.g != q.u) { a.u = (float *)(ws + off); off += align256((size_t)T * a.k * a.F * 4); }
    a.sel_idx = sel_idx ? sel_idx : ws_idx;
    a.sel_w = sel_w ? sel_w : ws_w;
    if (mode == TBQ_MOE_BF16) return hip_ok(launch_moe_bf16(a, ws + off, S(s)), "moe launch (prefill MFMA)");
    if (mode == TBQ_MOE_I8) return hip_ok(launch_moe_i8(a, ws + off, S(s)), "moe launch (prefill int8 MFMA)");
    return hip_ok(launch_moe_fp32(a, S(s)), "moe launch");
}

static int check_dense(const tbq_dense_model *m) {
    if (!m || !m->layers) return fail("tbq_dense: null model");
    if (m->n_layers <= 0 || m->hidden <= 0 || m->n_heads <= 0 || m->n_kv_heads <= 0 || m->ffn <= 0 || m->vocab <= 0 ||
        m->max_ctx <= 0)
        return fail("tbq_dense: non-positive size");
    if (m->head_dim != 64 && m->head_dim != 128) return fail("tbq_dense: head_dim must be 64 or 128");
    const int G = m->n_heads / m->n_kv_heads;
    if (m->n_heads % m->n_kv_heads || (G != 1 && G != 2 && G != 4 && G != 8))
        return fail("tbq_dense: n_heads / n_kv_heads must be 1, 2, 4 or 8");
    if (m->max_ctx > 131072) return fail("tbq_dense: max_ctx above 131072");
    if (m->hidden % 256 || m->ffn % 256 || (m->n_heads * m->head_dim) % 256)
        return fail("tbq_dense: hidden, ffn and n_heads*head_dim must be multiples of 256");
    if (m->hidden > TBQ_MAX_K || m->ffn > TBQ_MAX_K || m->n_heads * m->head_dim > TBQ_MAX_K)
        return fail("tbq_dense: hidden, ffn and n_heads*head_dim must be at most %d (the matvec row limit)",
                    TBQ_MAX_K);
    if (!tbq_qtype_supported(m->qtype_layers) || !tbq_qtype_supported(m->qtype_embd))
        return fail("tbq_dense: unsupported qtype");
    if (!m->tok_embd || !m->lm_head || !m->output_norm || !m->k_cache || !m->v_cache)
        return fail("tbq_dense: null tensor");
    auto qt_ok = [m](int q) { return tbq_qtype_supported(q ? q : m->qtype_layers); };
    auto w_ok = [](const void *p) { return p && aligned16(p); };
    for (int l = 0; l < m->n_layers; l++) {
        const tbq_dense_layer &L = m->layers[l];
        if (!L.attn_norm || !L.q_norm || !L.k_norm || !L.ffn_norm)
            return fail("tbq_dense: null norm weights in layer %d", l);
        const bool qkv = L.wqkv ? w_ok(L.wqkv) && qt_ok(L.qt_qkv)
                                : w_ok(L.wq) && w_ok(L.wk) && w_ok(L.wv) && qt_ok(L.qt_q) && qt_ok(L.qt_k) && qt_ok(L.qt_v);
        const bool gu = L.wgu ? w_ok(L.wgu) && qt_ok(L.qt_gu)
                              : w_ok(L.wgate) && w_ok(L.wup) && qt_ok(L.qt_gate) && qt_ok(L.qt_up);
        if (!qkv || !gu || !w_ok(L.wo) || !w_ok(L.wdown) || !qt_ok(L.qt_o) || !qt_ok(L.qt_down))
            return fail("tbq_dense: layer %d: a weight matrix is null, not 16-byte aligned or of an unsupported qtype", l);
    }
    return 1;
}

size_t tbq_dense_workspace_size(const tbq_dense_model *m) {
    if (!check_dense(m)) return 0;
    return dense_workspace_bytes(m);
}

int tbq_dense_decode(const tbq_dense_model *m, int token, int pos, float *logits, void *workspace,
                     size_t ws_bytes, void *s) {
    if (!ensure_init()) return 0;
    if (!check_dense(m)) return 0;
    if (token < 0 || token >= m->vocab) return fail("tbq_dense_decode: token %d out of range", token);
    if (pos < 0 || pos >= m->max_ctx) return fail("tbq_dense_decode: pos %d out of range", pos);
    if (!logits || !workspace) return fail("tbq_dense_decode: null logits or workspace");
    if (ws_bytes < dense_workspace_bytes(m)) return fail("tbq_dense_decode: workspace too small");
    return hip_ok(launch_dense_decode(m, token, pos, logits, workspace, S(s)), "dense decode launch");
}

size_t tbq_dense_prefill_workspace_size(const tbq_dense_model *m, int T) {
    if (!check_dense(m) || T <= 0 || T > 65536) return 0;
    return dense_prefill_workspace_bytes(m, T);
}

int tbq_dense_prefill_batched(const tbq_dense_model *m) { return check_dense(m) && dense_prefill_batched(m) ? 1 : 0; }

int tbq_dense_prefill(const tbq_dense_model *m, const int *tokens_host, int T, int pos0, float *logits,
                      void *workspace, size_t ws_bytes, void *s) {
    if (!ensure_init()) return 0;
    if (!check_dense(m)) return 0;
    if (T <= 0 || T > 65536) return fail("tbq_dense_prefill: T=%d outside 1..65536", T);
    if (pos0 < 0 || pos0 > m->max_ctx - T) return fail("tbq_dense_prefill: positions %d..%d outside the cache", pos0, pos0 + T - 1);
    if (!tokens_host || !logits || !workspace) return fail("tbq_dense_prefill: null tokens, logits or workspace");
    for (int t = 0; t < T; t++)
        if (tokens_host[t] < 0 || tokens_host[t] >= m->vocab)
            return fail("tbq_dense_prefill: token %d at %d out of range", tokens_host[t], t);
    if (ws_bytes < dense_prefill_workspace_bytes(m, T)) return fail("tbq_dense_prefill: workspace too small");
    return hip_ok(launch_dense_prefill(m, tokens_host, T, pos0, logits, workspace, S(s)), "dense prefill launch");
}

int tbq_quantize_q8k(const float *x, long long n, void *blocks, void *s) {
    if (!ensure_init()) return 0;
    if (n < 0 || n % 256) return fail("tbq_quantize_q8k: n=%lld must be a multiple of 256", n);
    if (!x || !blocks || !aligned16(x) || ((uintptr_t)blocks & 3u))
        return fail("tbq_quantize_q8k: null or misaligned pointer");
    if (n == 0) return 1;
    return hip_ok(launch_quantize_q8k(x, n, blocks, S(s)), "quantize_q8k launch");
}

size_t tbq_gemm_workspace_size(int T, int N, int K) {
    if (T <= 0 || N <= 0 || K <= 0) return 0;
    return hgemm_partial_bytes(T, N, K, hgemm_cus());
}

int tbq_gemm(int wqt, const void *W, const void *X16, int T, int N, int K, float *C, int ldc, void *ws,
             size_t ws_bytes, void *s) {
    if (!ensure_init()) return 0;
    if (wqt != QT_F16 && wqt != QT_Q4_K) return fail("tbq_gemm: weight format %d (F16 or Q4_K only)", wqt);
    if (T <= 0 || N <= 0 || K <= 0 || !hgemm_supported(wqt, N, K) || ldc < N || ldc % 4)
        return fail("tbq_gemm: bad shape T=%d N=%d K=%d ldc=%d (N a multiple of 4, K of 256, ldc >= N)", T, N, K,
                    ldc);
    if ((long long)T * K * 2 >= (1ll << 31)) return fail("tbq_gemm: X above 2 GiB");
    if (!W || !X16 || !C || !aligned16(W) || !aligned16(X16) || !aligned16(C))
        return fail("tbq_gemm: null or misaligned pointer");
    const size_t need = tbq_gemm_workspace_size(T, N, K);
    if (need && (!ws || ws_bytes < need)) return fail("tbq_gemm: workspace %zu < %zu bytes", ws_bytes, need);
    return hip_ok(launch_hgemm(wqt, W, (const _Float16 *)X16, T, N, K, C, ldc, (float *)ws, hgemm_cus(), S(s)),
                  "gemm launch");
}

int tbq_expf_device(const float *in, float *out, size_t n, void *s) {
    if (!ensure_init()) return 0;
    if (!in || !out) return fail("tbq_expf_device: null pointer");
    if (n == 0) return 1;
    return hip_ok(launch_expf(in, out, (long long)n, S(s)), "expf launch");
}

float tbq_expf_host(float x) { return expf_glibc(x); }

}  // extern "C"
