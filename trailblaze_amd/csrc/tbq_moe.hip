// tbq_moe.hip -- gfx950 kernels for the MoE block of the reference's forward
// pass (layer4/tb_infer.c:753-833,876) on the fp32 path:
//
//   k_route          router logits + softmax + top-k + renormalise, one
//                    workgroup per token.  Logits are summed in the
//                    reference's sequential order (acc = acc + w*x, no fma)
//                    so the selected experts and their slot order are
//                    bit-identical to tb_route_experts (tb_infer.c:351-374).
//   k_gate_up        g = W_gate[e] x, u = W_up[e] x, a = swiglu(g, u) for
//                    every (token, slot) pair.
//   k_rows           y[t][s] = W_down[e] a[t][s] (and gate, up one at a
//                    time when their qtypes differ, with k_swiglu_pairs).
//   k_combine        out = resid + sum over slots, in slot order, of w*y.
#include <stdlib.h>

#include "tbq_kquant.hpp"
#include "tbq_kernels.h"

namespace tbq {

// ---------------------------------------------------------------------------
// Router.  blockDim = 256; lane e < E owns expert e.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_route(const float *__restrict__ xn, const float *__restrict__ Wr,
                                               const float *__restrict__ bias, int H, int E, int top_k,
                                               int *__restrict__ sel_idx, float *__restrict__ sel_w) {
    extern __shared__ float lds[];
    float *xl = lds;             // H
    float *p = lds + H;          // 256 scores
    __shared__ int s_cnt[256];
    __shared__ float s_sum;
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *x = xn + (long long)t * H;
    for (int i = tid * 4; i < H; i += 1024) *reinterpret_cast<float4 *>(xl + i) = *reinterpret_cast<const float4 *>(x + i);
    __syncthreads();

    // logits in sequential order: acc = fl(acc + fl(w*x))
    float lg = -__builtin_huge_valf();
    if (tid < E) {
        const float *w = Wr + (long long)tid * H;
        float acc = 0.f;
        for (int k = 0; k < H; k += 8) {
            float4 wa = *reinterpret_cast<const float4 *>(w + k);
            float4 wb = *reinterpret_cast<const float4 *>(w + k + 4);
            float4 xa = *reinterpret_cast<const float4 *>(xl + k);
            float4 xb = *reinterpret_cast<const float4 *>(xl + k + 4);
            acc = acc + wa.x * xa.x; acc = acc + wa.y * xa.y;
            acc = acc + wa.z * xa.z; acc = acc + wa.w * xa.w;
            acc = acc + wb.x * xb.x; acc = acc + wb.y * xb.y;
            acc = acc + wb.z * xb.z; acc = acc + wb.w * xb.w;
        }
        if (bias) acc = acc + bias[tid];
        lg = acc;
    }
    p[tid] = lg;
    __syncthreads();
    // max (order-independent)
    float mx = p[0];
    for (int e = 1; e < E; e++) mx = p[e] > mx ? p[e] : mx;
    float ex = 0.f;
    if (tid < E) ex = expf_glibc(lg - mx);
    __syncthreads();
    p[tid] = ex;
    __syncthreads();
    if (tid == 0) {  // sequential sum, as the reference
        float s = 0.f;
        for (int e = 0; e < E; e++) s = s + p[e];
        s_sum = s;
    }
    __syncthreads();
    float pr = tid < E ? ex / s_sum : 0.f;
    __syncthreads();
    p[tid] = pr;
    __syncthreads();
    // Element e enters the slot array iff fewer than k earlier elements have
    // a score >= its own (the slots always hold the k largest seen so far).
    const int k = top_k > 8 ? 8 : top_k;
    int cnt = 0;
    if (tid < E)
        for (int e2 = 0; e2 < tid; e2++) cnt += p[e2] >= pr ? 1 : 0;
    s_cnt[tid] = (tid < E && cnt < k) ? 1 : 0;
    __syncthreads();
    if (tid == 0) {
        // Replay the slot updates of the entering elements in index order:
        // replace the first slot holding the minimum when strictly larger.
        int idx[8];
        float w[8];
        for (int i = 0; i < 8; i++) { idx[i] = 0; w[i] = -1e30f; }
        for (int e = 0; e < E; e++) {
            if (!s_cnt[e]) continue;
            int lo = 0;
            for (int i = 1; i < k; i++) if (w[i] < w[lo]) lo = i;
            float v = p[e];
            if (v > w[lo]) { w[lo] = v; idx[lo] = e; }
        }
        float ws = 0.f;
        for (int i = 0; i < k; i++) ws = ws + w[i];
        if (ws > 0.f) for (int i = 0; i < k; i++) w[i] = w[i] / ws;
        for (int i = 0; i < 8; i++) {
            sel_idx[t * 8 + i] = i < k ? idx[i] : -1;
            sel_w[t * 8 + i] = i < k ? w[i] : 0.f;
        }
    }
}

// ---------------------------------------------------------------------------
// Expert gate/up + SwiGLU.  grid = (F / RPB, T*k); 256 threads; LPR lanes per
// dot product; each iteration computes RPW = 256/LPR/2 outputs (gate row and
// up row of the same index go to adjacent lane groups).
// ---------------------------------------------------------------------------
template <int QT, int LPR>
__global__ __launch_bounds__(256) void k_gate_up(const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up,
                                                 const float *__restrict__ xn, const int *__restrict__ sel_idx,
                                                 int H, int F, int E, int k, int rows_per_block,
                                                 float *__restrict__ act) {
    extern __shared__ float lds[];
    float *xl = lds, *xs = lds + H;
    const int pair = blockIdx.y, t = pair / k, s = pair % k;
    // an index outside [0, E) (never produced by the router) reads expert 0
    // and contributes 0
    const int e_sel = sel_idx[t * 8 + s];
    const bool ev = (unsigned)e_sel < (unsigned)E;
    const int e = ev ? e_sel : 0;
    stage_x_swizzled<256>(xn + (long long)t * H, H, xl, xs);
    __syncthreads();
    constexpr int GROUPS = 256 / LPR;   // dot products per iteration
    const long long rb = (long long)(H / block_weights(QT)) * block_bytes(QT);
    const int C = H / 32, lane = threadIdx.x % LPR, grp = threadIdx.x / LPR;
    const int which = grp & 1, sub = grp >> 1;   // 0 = gate, 1 = up
    const uint8_t *Wb = (which ? up : gate) + (long long)e * F * rb;
    __shared__ float res[GROUPS];
    const int r_begin = blockIdx.x * rows_per_block;
    for (int r0 = r_begin; r0 < r_begin + rows_per_block; r0 += GROUPS / 2) {
        int r = r0 + sub;
        float acc = 0.f;
        if (r < F) {
            const uint8_t *row = Wb + (long long)r * rb;
            for (int c = lane; c < C; c += LPR) {
                float xv[32];
                load_chunk_x(xl, c, xv);
                acc += chunk_dot<QT>(row, c, xv, xs + 2 * c);
            }
        }
        acc = group_sum<LPR>(acc);
        if (lane == 0) res[grp] = acc;
        __syncthreads();
        if (threadIdx.x < GROUPS / 2) {
            int rr = r0 + threadIdx.x;
            if (rr < F) {
                float g = res[2 * threadIdx.x], u = res[2 * threadIdx.x + 1];
                float den = 1.0f + expf_glibc(-g);
                float sg = g / den;
                act[(long long)pair * F + rr] = ev ? sg * u : 0.f;
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// One expert matrix per (token, slot) pair: out[pair][r] = W[e][r] . x_pair
// over R rows of K weights, x_pair = x + (pair / xdiv) * K (xdiv = k: the
// token's input row; 1: the pair's own row).  The down projection
// (W_down, act, R = H, K = F), and gate and up one at a time when their
// qtypes differ (R = F, K = H).
// ---------------------------------------------------------------------------
template <int QT, int LPR>
__global__ __launch_bounds__(256) void k_rows(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                              const int *__restrict__ sel_idx, int R, int K, int E, int k, int xdiv,
                                              int rows_per_block, float *__restrict__ yout) {
    extern __shared__ float lds[];
    float *xl = lds, *xs = lds + K;
    const int pair = blockIdx.y, t = pair / k, s = pair % k;
    const int e_sel = sel_idx[t * 8 + s];
    const bool ev = (unsigned)e_sel < (unsigned)E;
    const int e = ev ? e_sel : 0;   // out of range: y = 0
    stage_x_swizzled<256>(x + (long long)(pair / xdiv) * K, K, xl, xs);
    __syncthreads();
    constexpr int GROUPS = 256 / LPR;
    const long long rb = (long long)(K / block_weights(QT)) * block_bytes(QT);
    const int C = K / 32, lane = threadIdx.x % LPR, grp = threadIdx.x / LPR;
    const uint8_t *Wb = W + (long long)e * R * rb;
    const int r_begin = blockIdx.x * rows_per_block;
    for (int r0 = r_begin; r0 < r_begin + rows_per_block; r0 += GROUPS) {
        int r = r0 + grp;
        float acc = 0.f;
        if (r < R) {
            const uint8_t *row = Wb + (long long)r * rb;
            for (int c = lane; c < C; c += LPR) {
                float xv[32];
                load_chunk_x(xl, c, xv);
                acc += chunk_dot<QT>(row, c, xv, xs + 2 * c);
            }
        }
        acc = group_sum<LPR>(acc);
        if (lane == 0 && r < R) yout[(long long)pair * R + r] = ev ? acc : 0.f;
    }
}

// act[i] = silu(act[i]) * u[i] (tb_swiglu, layer4/tb_infer.c:130-135, with
// the router's expf), after gate and up ran separately.
__global__ __launch_bounds__(256) void k_swiglu_pairs(float *__restrict__ act, const float *__restrict__ u,
                                                      long long n) {
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
        const float g = act[i];
        const float den = 1.0f + expf_glibc(-g);
        const float sg = g / den;
        act[i] = sg * u[i];
    }
}

// out[t][i] = resid[t][i] + (((0 + w0*y0) + w1*y1) + ...) in slot order;
// a slot whose expert index is outside [0, E) (never produced by the
// router; its y may be unwritten) is skipped.
// Four consecutive outputs per thread (H is a multiple of 4), each summed
// exactly as the scalar form.  A thread's k slot loads are all issued before
// its adds (unwritten y of a skipped slot is read and not used).
template <int NT>
__global__ __launch_bounds__(NT) void k_combine(const float *__restrict__ y, const int *__restrict__ sel_idx,
                                                const float *__restrict__ sel_w, const float *__restrict__ resid,
                                                int T, int H, int E, int k, float *__restrict__ out) {
    const long long n4 = (long long)T * H / 4;
    const int H4 = H / 4;
    for (long long i = blockIdx.x * (long long)NT + threadIdx.x; i < n4; i += (long long)gridDim.x * NT) {
        const int t = (int)(i / H4), h4 = (int)(i - (long long)t * H4);
        float4 v[8];
        float w[8];
        bool ok[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            ok[s] = false;
            if (s < k) {
                ok[s] = (unsigned)sel_idx[t * 8 + s] < (unsigned)E;
                w[s] = sel_w[t * 8 + s];
                v[s] = reinterpret_cast<const float4 *>(y + ((long long)t * k + s) * H)[h4];
            }
        }
        const float4 r = reinterpret_cast<const float4 *>(resid)[i];
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int s = 0; s < 8; s++) {
            if (!ok[s]) continue;
            const float px = w[s] * v[s].x, py = w[s] * v[s].y, pz = w[s] * v[s].z, pw = w[s] * v[s].w;
            acc.x = acc.x + px;
            acc.y = acc.y + py;
            acc.z = acc.z + pz;
            acc.w = acc.w + pw;
        }
        reinterpret_cast<float4 *>(out)[i] = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
}

static int pick_lpr(int K) {
    int C = K / 32, lpr = 64;
    while (lpr > 1 && (lpr > C || C % lpr)) lpr >>= 1;
    if (lpr < 4 && C >= 4) lpr = 4;
    return lpr;
}

template <int QT, int LPR>
static hipError_t launch_gate_up_t(const MoeArgs &a, hipStream_t st) {
    const int pairs = a.T * a.k;
    constexpr int OUT_PER_IT = 256 / LPR / 2;
    int rpb = OUT_PER_IT * 4;
    dim3 grid((a.F + rpb - 1) / rpb, pairs);
    size_t lds = (size_t)a.H * 4 + (size_t)(a.H / 16) * 4;
    hipLaunchKernelGGL((k_gate_up<QT, LPR>), grid, dim3(256), lds, st, (const uint8_t *)a.gate,
                       (const uint8_t *)a.up, a.xn, a.sel_idx, a.H, a.F, a.E, a.k, rpb, a.act);
    return hipGetLastError();
}

template <int QT, int LPR>
static hipError_t launch_rows_t(const void *W, const float *x, int R, int K, int xdiv, float *out, const MoeArgs &a,
                                hipStream_t st) {
    const int pairs = a.T * a.k;
    constexpr int OUT_PER_IT = 256 / LPR;
    int rpb = OUT_PER_IT * 2;
    dim3 grid((R + rpb - 1) / rpb, pairs);
    size_t lds = (size_t)K * 4 + (size_t)(K / 16) * 4;
    hipLaunchKernelGGL((k_rows<QT, LPR>), grid, dim3(256), lds, st, (const uint8_t *)W, x, a.sel_idx, R, K, a.E, a.k,
                       xdiv, rpb, out);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_gate_up_q(const MoeArgs &a, hipStream_t st) {
    switch (pick_lpr(a.H)) {
    case 64: return launch_gate_up_t<QT, 64>(a, st);
    case 32: return launch_gate_up_t<QT, 32>(a, st);
    case 16: return launch_gate_up_t<QT, 16>(a, st);
    case 8: return launch_gate_up_t<QT, 8>(a, st);
    default: return launch_gate_up_t<QT, 4>(a, st);
    }
}

template <int QT>
static hipError_t launch_rows_q(const void *W, const float *x, int R, int K, int xdiv, float *out, const MoeArgs &a,
                                hipStream_t st) {
    switch (pick_lpr(K)) {
    case 64: return launch_rows_t<QT, 64>(W, x, R, K, xdiv, out, a, st);
    case 32: return launch_rows_t<QT, 32>(W, x, R, K, xdiv, out, a, st);
    case 16: return launch_rows_t<QT, 16>(W, x, R, K, xdiv, out, a, st);
    case 8: return launch_rows_t<QT, 8>(W, x, R, K, xdiv, out, a, st);
    default: return launch_rows_t<QT, 4>(W, x, R, K, xdiv, out, a, st);
    }
}

// Dispatch on an expert qtype: CALL(Q) with Q the format's constant, so the
// per-format kernel families above are instantiated for every expert qtype.
#define TBQ_MOE_QT_SWITCH(qt, CALL)                         \
    switch (qt) {                                           \
    case QT_Q2_K: return CALL(QT_Q2_K);                     \
    case QT_Q3_K: return CALL(QT_Q3_K);                     \
    case QT_Q4_K: return CALL(QT_Q4_K);                     \
    case QT_Q5_K: return CALL(QT_Q5_K);                     \
    case QT_Q6_K: return CALL(QT_Q6_K);                     \
    case QT_Q8_0: return CALL(QT_Q8_0);                     \
    case QT_GQ2_K: return CALL(QT_GQ2_K);                   \
    case QT_GQ3_K: return CALL(QT_GQ3_K);                   \
    case QT_GQ4_K: return CALL(QT_GQ4_K);                   \
    case QT_GQ5_K: return CALL(QT_GQ5_K);                   \
    case QT_GQ6_K: return CALL(QT_GQ6_K);                   \
    case QT_GQ8_0: return CALL(QT_GQ8_0);                   \
    default: return hipErrorInvalidValue;                   \
    }

// act = swiglu(W_gate x, W_up x) for one qtype shared by gate and up.
static hipError_t launch_gate_up_generic(const MoeArgs &a, hipStream_t st) {
#define TBQ_CALL(Q) launch_gate_up_q<Q>(a, st)
    TBQ_MOE_QT_SWITCH(a.qg, TBQ_CALL)
#undef TBQ_CALL
}

// y[pair] = W[e] x_pair for the expert tensor W of qtype qt.
static hipError_t launch_rows_generic(int qt, const void *W, const float *x, int R, int K, int xdiv, float *out,
                                      const MoeArgs &a, hipStream_t st) {
#define TBQ_CALL(Q) launch_rows_q<Q>(W, x, R, K, xdiv, out, a, st)
    TBQ_MOE_QT_SWITCH(qt, TBQ_CALL)
#undef TBQ_CALL
}

static bool is_q4k(int qt) { return qt == QT_Q4_K || qt == QT_GQ4_K; }

// The experts of a routed batch (routing already in a.sel_idx / a.sel_w):
// gate/up + SwiGLU into a.act, then down + the slot-ordered combine into
// a.out.  Each phase takes the Q4_K int-dot kernels where its tensors are
// Q4_K (and the shape fits them), else the K-quant int-dot kernels
// (tbq_mv_kq.hip), else the byte->fp32 kernels above; gate and up of
// different qtypes run one at a time.
// grouped_done: the router has already written a.grp.
static hipError_t launch_experts(const MoeArgs &a, hipStream_t st, bool grouped_done) {
    const bool q4_gu = a.qg == a.qu && is_q4k(a.qg), q4_dn = is_q4k(a.qd);
    const bool grouped = moe_decode_grouped(a);
    hipError_t err;
    if (grouped && !grouped_done && (err = launch_group(a, st)) != hipSuccess) return err;
    err = hipErrorNotSupported;
    if (q4_gu) err = launch_moe_q4k_gate_up(a, grouped, st);
    if (err == hipErrorNotSupported && a.qg == a.qu) err = launch_moe_gate_up_kq(a, grouped, st);
    if (err == hipErrorNotSupported) {
        if (a.qg == a.qu) {
            err = launch_gate_up_generic(a, st);
        } else {
            if (!a.u) return hipErrorInvalidValue;
            err = launch_rows_generic(a.qg, a.gate, a.xn, a.F, a.H, a.k, a.act, a, st);
            if (err == hipSuccess) err = launch_rows_generic(a.qu, a.up, a.xn, a.F, a.H, a.k, a.u, a, st);
            if (err == hipSuccess) {
                const long long n = (long long)a.T * a.k * a.F;
                const int grid = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
                hipLaunchKernelGGL(k_swiglu_pairs, dim3(grid), dim3(256), 0, st, a.act, a.u, n);
                err = hipGetLastError();
            }
        }
    }
    if (err != hipSuccess) return err;
    err = hipErrorNotSupported;
    if (q4_dn) err = launch_moe_q4k_down(a, grouped, st);
    if (err == hipErrorNotSupported) err = launch_moe_down_kq(a, grouped, st);
    if (err != hipErrorNotSupported) return err;
    err = launch_rows_generic(a.qd, a.down, a.act, a.H, a.F, 1, a.y, a, st);
    if (err != hipSuccess) return err;
    return launch_combine(a, st);
}

hipError_t launch_route(const float *xn, const float *router, const float *bias, int T, int H, int E, int top_k,
                        int *sel_idx, float *sel_w, hipStream_t st) {
    size_t lds = (size_t)H * 4 + 256 * 4;
    hipLaunchKernelGGL(k_route, dim3(T), dim3(256), lds, st, xn, router, bias, H, E, top_k, sel_idx, sel_w);
    return hipGetLastError();
}

// Tokens are independent in the MoE block (each is routed and combined on
// its own), so a batch may run as consecutive token chunks on one stream,
// each reusing the start of the workspace's per-token buffers.  The limit is
// `cap` tokens, lowered by TBQ_MOE_CHUNK_TOKENS when that is set (the test
// hook for the chunked path).
static int chunk_tokens(int T, long long cap) {
    if (const char *e = getenv("TBQ_MOE_CHUNK_TOKENS")) {
        const long long v = atoll(e);
        if (v > 0 && v < cap) cap = v;
    }
    return (int)(cap < T ? cap : T);
}

template <class Fn>
static hipError_t by_token_chunks(const MoeArgs &a, long long cap, Fn fn) {
    const int Tc = chunk_tokens(a.T, cap < 1 ? 1 : cap);
    for (int t0 = 0; t0 < a.T; t0 += Tc) {
        MoeArgs c = a;
        c.T = a.T - t0 < Tc ? a.T - t0 : Tc;
        c.xn = a.xn + (long long)t0 * a.H;
        c.resid = a.resid + (long long)t0 * a.H;
        c.out = a.out + (long long)t0 * a.H;
        c.sel_idx = a.sel_idx + (long long)t0 * 8;
        c.sel_w = a.sel_w + (long long)t0 * 8;
        const hipError_t err = fn(c);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

hipError_t launch_moe_fp32(const MoeArgs &a, hipStream_t st) {
    bool grouped = false;
    hipError_t err = launch_router(a.xn, a.router, a.bias, a.T, a.H, a.E, a.top_k, a.logits, a.counters, a.sel_idx,
                                   a.sel_w, st, nullptr, nullptr, nullptr, &a, &grouped);
    if (err == hipErrorNotSupported)
        err = launch_route(a.xn, a.router, a.bias, a.T, a.H, a.E, a.top_k, a.sel_idx, a.sel_w, st);
    if (err != hipSuccess) return err;
    // the per-pair kernels take a grid column per (token, slot) pair; the
    // router's grouping covers the whole batch, so a chunk uses it only when
    // it is the whole batch
    return by_token_chunks(a, 65535 / a.k,
                           [&](const MoeArgs &c) { return launch_experts(c, st, grouped && c.T == a.T); });
}

hipError_t launch_combine(const MoeArgs &a, hipStream_t st) {
    const long long n = (long long)a.T * a.H / 4;
    if (n <= 65536) {   // decode batches: small workgroups, one float4 per thread
        hipLaunchKernelGGL(k_combine<64>, dim3((int)((n + 63) / 64)), dim3(64), 0, st, a.y, a.sel_idx, a.sel_w,
                           a.resid, a.T, a.H, a.E, a.k, a.out);
    } else {
        const int grid = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
        hipLaunchKernelGGL(k_combine<256>, dim3(grid), dim3(256), 0, st, a.y, a.sel_idx, a.sel_w, a.resid, a.T, a.H,
                           a.E, a.k, a.out);
    }
    return hipGetLastError();
}

// The prefill kernels address a call's activation rows (fp16, or two int8
// levels) through one buffer resource, whose byte offsets are 32-bit: T
// tokens need T * max(H, k * F) * 2 bytes below 2^31, and larger batches run
// in token chunks.
static long long prefill_chunk_cap(const MoeArgs &a) {
    const long long per_tok = a.H > (long long)a.k * a.F ? a.H : (long long)a.k * a.F;
    return ((1LL << 30) - 1) / per_tok;
}

// Prefill: exact routing, then grouped fp16-MFMA experts and the
// slot-ordered combine.
static hipError_t launch_moe_bf16_chunk(const MoeArgs &a, void *scratch, hipStream_t st) {
    // the batch router also writes the tokens' fp16 rows for the expert GEMMs
    _Float16 *x16 = nullptr;
    float *xinv = nullptr;
    bool x16_done = false;
    prefill_x16(a, scratch, &x16, &xinv);
    hipError_t err = launch_router(a.xn, a.router, a.bias, a.T, a.H, a.E, a.top_k, a.logits,
                                   a.T >= 32 ? nullptr : a.counters, a.sel_idx, a.sel_w, st, x16, xinv, &x16_done);
    if (err == hipErrorNotSupported)
        err = launch_route(a.xn, a.router, a.bias, a.T, a.H, a.E, a.top_k, a.sel_idx, a.sel_w, st);
    if (err != hipSuccess) return err;
    err = launch_moe_prefill_q4k(a, scratch, st, x16_done);
    if (err != hipSuccess) return err;
    return launch_combine(a, st);
}

hipError_t launch_moe_bf16(const MoeArgs &a, void *scratch, hipStream_t st) {
    return by_token_chunks(a, prefill_chunk_cap(a), [&](const MoeArgs &c) { return launch_moe_bf16_chunk(c, scratch, st); });
}

// Prefill on int8 MFMA: exact routing, Q8_K activations, grouped int8
// expert GEMMs, the slot-ordered combine.
static hipError_t launch_moe_i8_chunk(const MoeArgs &a, void *scratch, hipStream_t st) {
    hipError_t err = launch_router(a.xn, a.router, a.bias, a.T, a.H, a.E, a.top_k, a.logits,
                                   a.T >= 32 ? nullptr : a.counters, a.sel_idx, a.sel_w, st);
    if (err == hipErrorNotSupported)
        err = launch_route(a.xn, a.router, a.bias, a.T, a.H, a.E, a.top_k, a.sel_idx, a.sel_w, st);
    if (err != hipSuccess) return err;
    err = launch_moe_prefill_q4k_i8(a, scratch, st);
    if (err != hipSuccess) return err;
    return launch_combine(a, st);
}

hipError_t launch_moe_i8(const MoeArgs &a, void *scratch, hipStream_t st) {
    return by_token_chunks(a, prefill_chunk_cap(a), [&](const MoeArgs &c) { return launch_moe_i8_chunk(c, scratch, st); });
}

}  // namespace tbq
