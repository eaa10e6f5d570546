// tbq_dense.hip -- one-token decode step of a dense Qwen3-style transformer
// on gfx950, built on libtbq's K-quant matvecs.
//
// Per layer (x: fp32 residual stream, h: normed activations):
//   h = rmsnorm(x += y_prev) * attn_norm           } one matvec launch: the
//   qkv = Wqkv h   (q | k | v rows, Q4_K)           } norm is its x staging
//   per head: rmsnorm(q_h) * q_norm, rmsnorm(k_h) * k_norm, RoPE (rotate-half
//   pairs i, i + D/2, angle pos * theta^(-2i/D)); k, v appended to the cache;
//   attn = softmax(q K^T / sqrt(D)) V over positions 0..pos, GQA
//                                                    k_attn_partial + k_attn_combine
//   y = Wo attn                                      tbq_matvec
//   h = rmsnorm(x += y) * ffn_norm                   } one matvec launch: the
//   gu = Wgu h     (gate | up rows)                  } norm is its x staging,
//   a = silu(g) * u                                  } silu(g) * u its epilogue
//   y = Wdown a                                      tbq_matvec
// then h = rmsnorm(x += y) * output_norm and logits = Wlm h.  The token's
// embedding is row `token` of tok_embd, dequantised exactly.
//
// The layer math is the model's (Qwen3): QK-norm before RoPE, rotate-half
// RoPE, head_dim from the model (not hidden / n_heads), and every K head
// rotated once.  The reference's forward (layer4/tb_infer.c:553-883)
// differs in each of these; its rmsnorm (layer1/tb_tensor.c:194-199) and
// online-softmax attention (layer1/tb_tensor.c:300-405) compute the same
// functions as the matvecs' PRO_NORM staging prologue and the attention
// kernels here.
//
// Attention: the cache is [layer][kv head][max_ctx][D] fp32.  A workgroup
// owns one kv head and a chunk of ATT_CH positions and serves all G query
// heads of that kv head, so K and V are read from HBM once per step; it
// writes the chunk's running max, denominator and weighted V sum per query
// head, and k_attn_combine merges the chunks.
#include "tbq_kernels.h"
#include "tbq_device.hpp"
#include "../../include/tbq.h"

namespace tbq {

#ifndef TBQ_ATT_CH
#define TBQ_ATT_CH 128
#endif
constexpr int ATT_CH = TBQ_ATT_CH;   // positions per attention workgroup
#ifndef TBQ_ATT_THREADS
#define TBQ_ATT_THREADS 512
#endif
constexpr int ATT_THREADS = TBQ_ATT_THREADS;
constexpr int ATT_PARTS = ATT_THREADS / ATT_CH;   // threads per position in the score phase

// Block-wide sum of one float per thread (blockDim.x a multiple of 64,
// <= 1024); every thread gets the result.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < nw; i++) s += red[i];
    return s;
}

// v = x + y (y may be null), h = v * rsqrt(mean(v^2) + eps) * w, and v
// stored to vo when vo is not null.  One workgroup.  Used where the matvec
// that follows has no fused staging prologue for the shape.
__global__ __launch_bounds__(1024) void k_add_rmsnorm(const float *__restrict__ x, const float *__restrict__ y,
                                                      const float *__restrict__ w, int n, float eps,
                                                      float *__restrict__ h, float *__restrict__ vo) {
    __shared__ float red[16];
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = y ? x[i] + y[i] : x[i];
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = y ? x[i] + y[i] : x[i];
        if (vo) vo[i] = v;
        h[i] = v * r * w[i];
    }
}

// RoPE table of one step: rc[j] = cos, rc[D/2 + j] = sin of pos *
// theta^(-2j/D), formed and reduced in fp64 so the error does not grow with
// the position.  One workgroup of D/2 threads.
__global__ __launch_bounds__(64) void k_rope_table(int pos, float theta, int D, float *__restrict__ rc) {
    const int j = threadIdx.x;
    if (j < D / 2) {
        double sd, cd;
        sincos((double)pos * pow((double)theta, -2.0 * j / D), &sd, &cd);
        rc[j] = (float)cd;
        rc[D / 2 + j] = (float)sd;
    }
}

// RMSNorm with the head's norm weights then rotate-half RoPE (table rc) of
// one head vector held by one wave: lane l has elements l and l + 64
// (D = 128) or l (D = 64).
template <int D>
__device__ __forceinline__ void head_norm_rope(float (&x)[D / 64], const float *__restrict__ w,
                                               const float *__restrict__ rc, float eps) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < D / 64; i++) ss += x[i] * x[i];
    ss = group_sum<64>(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int i = 0; i < D / 64; i++) x[i] = x[i] * r * w[lane + 64 * i];
    const int j = lane % (D / 2);   // pair (j, j + D/2)
    const float cs = rc[j], sn = rc[D / 2 + j];
    if constexpr (D == 128) {
        const float a = x[0], b = x[1];   // elements j and j + 64
        x[0] = a * cs - b * sn;
        x[1] = a * sn + b * cs;
    } else {
        const float other = __shfl_xor(x[0], 32);   // partner j +- 32
        x[0] = lane < 32 ? x[0] * cs - other * sn : other * sn + x[0] * cs;
    }
}

// Attention for one kv head x one chunk of ATT_CH positions, all G query
// heads of the head, with the head's QK-norm, RoPE and cache append folded
// in.  The chunk's K and V rows are loaded first (coalesced, all in flight
// at once) and staged in LDS; meanwhile each wave normalises and rotates its
// query heads from qkv.  The chunk that holds `pos` also forms the new K row
// (norm + RoPE) and V row, uses them in place of the cache's and writes them
// to the cache.  Writes part[(qh * nsplit + chunk) * (D + 2) + {0..D-1, D:
// max, D+1: denominator}].  grid = (NKV, nsplit), 256 threads.
template <int D, int G>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_partial(const float *__restrict__ qkv, const float *__restrict__ qn,
                                                              const float *__restrict__ kn, int NQ, int pos,
                                                              const float *__restrict__ rc, float eps, float *__restrict__ kc,
                                                              float *__restrict__ vc, int max_ctx, int nsplit,
                                                              float *__restrict__ part) {
    static_assert(D == 64 || D == 128, "head_dim");
    constexpr int KLD = D + 4;                        // K row stride in LDS (conflict-free row reads)
    constexpr int NL = ATT_CH * D / 4 / ATT_THREADS;  // float4 of K (and of V) per thread
    extern __shared__ __attribute__((aligned(16))) float at_lds[];
    float *Ks = at_lds;                      // [ATT_CH][KLD]
    float *Vs = Ks + ATT_CH * KLD;           // [ATT_CH][D]
    float *qs = Vs + ATT_CH * D;             // [G][D]
    float *sc = qs + G * D;                  // [G][ATT_CH]
    float *pd = sc + G * ATT_CH;             // [ATT_PARTS][G][ATT_CH]
    const int kvh = blockIdx.x, ch = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n_pos = pos + 1, p0 = ch * ATT_CH;
    const long long hbase = (long long)kvh * max_ctx * D;
    // K and V rows of the chunk; rows past n_pos read row n_pos - 1 (weighed 0)
    float4 kr[NL], vr[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int f = tid + ATT_THREADS * i, row = f / (D / 4), c4 = f % (D / 4);
        const int pp = p0 + row < n_pos ? p0 + row : n_pos - 1;
        kr[i] = *reinterpret_cast<const float4 *>(kc + hbase + (long long)pp * D + 4 * c4);
        vr[i] = *reinterpret_cast<const float4 *>(vc + hbase + (long long)pp * D + 4 * c4);
    }
    // query heads (scaled by 1/sqrt(D)); wave w takes heads w, w + 4, ...
    const float scale = 1.0f / sqrtf((float)D);
    for (int g = wave; g < G; g += ATT_THREADS / 64) {
        float x[D / 64];
#pragma unroll
        for (int i = 0; i < D / 64; i++) x[i] = qkv[(kvh * G + g) * D + lane + 64 * i];
        head_norm_rope<D>(x, qn, rc, eps);
#pragma unroll
        for (int i = 0; i < D / 64; i++) qs[g * D + lane + 64 * i] = x[i] * scale;
    }
    const bool own = pos >= p0 && pos < p0 + ATT_CH;   // this chunk holds the new row
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int f = tid + ATT_THREADS * i, row = f / (D / 4), c4 = f % (D / 4);
        *reinterpret_cast<float4 *>(Ks + row * KLD + 4 * c4) = kr[i];
        *reinterpret_cast<float4 *>(Vs + row * D + 4 * c4) = vr[i];
    }
    __syncthreads();
    if (own && wave == 0) {
        float x[D / 64], v[D / 64];
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            x[i] = qkv[(NQ + kvh) * D + lane + 64 * i];
            v[i] = qkv[(NQ + (int)gridDim.x + kvh) * D + lane + 64 * i];
        }
        head_norm_rope<D>(x, kn, rc, eps);
        const int row = pos - p0;
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            Ks[row * KLD + lane + 64 * i] = x[i];
            Vs[row * D + lane + 64 * i] = v[i];
            kc[hbase + (long long)pos * D + lane + 64 * i] = x[i];
            vc[hbase + (long long)pos * D + lane + 64 * i] = v[i];
        }
    }
    __syncthreads();
    // scores: thread = (position p, part of the dims), K row from LDS
    {
        constexpr int DP = D / ATT_PARTS;
        const int p = tid % ATT_CH, half = tid / ATT_CH;
        const float *krow = Ks + p * KLD + half * DP;
        float acc[G];
#pragma unroll
        for (int g = 0; g < G; g++) acc[g] = 0.f;
#pragma unroll
        for (int c = 0; c < DP / 4; c++) {
            const float4 k4 = *reinterpret_cast<const float4 *>(krow + 4 * c);
            const int d = half * DP + 4 * c;
#pragma unroll
            for (int g = 0; g < G; g++)
                acc[g] += qs[g * D + d] * k4.x + qs[g * D + d + 1] * k4.y + qs[g * D + d + 2] * k4.z +
                          qs[g * D + d + 3] * k4.w;
        }
#pragma unroll
        for (int g = 0; g < G; g++) pd[(half * G + g) * ATT_CH + p] = acc[g];
    }
    __syncthreads();
    for (int i = tid; i < G * ATT_CH; i += ATT_THREADS) {
        const int g = i / ATT_CH, p = i % ATT_CH;
        float t = pd[g * ATT_CH + p];
#pragma unroll
        for (int q = 1; q < ATT_PARTS; q++) t += pd[(q * G + g) * ATT_CH + p];
        sc[i] = p0 + p < n_pos ? t : -__builtin_huge_valf();
    }
    __syncthreads();
    // per-head max and exp; wave w takes heads w, w + 4, ...
    for (int g = wave; g < G; g += ATT_THREADS / 64) {
        float m = -__builtin_huge_valf();
        for (int p = lane; p < ATT_CH; p += 64) m = fmaxf(m, sc[g * ATT_CH + p]);
        m = wave_max(m);
        float l = 0.f;
        for (int p = lane; p < ATT_CH; p += 64) {
            const float e = expf(sc[g * ATT_CH + p] - m);   // exp(-inf) = 0 past n_pos
            sc[g * ATT_CH + p] = e;
            l += e;
        }
        l = group_sum<64>(l);
        if (lane == 0) {
            part[((long long)(kvh * G + g) * nsplit + ch) * (D + 2) + D] = m;
            part[((long long)(kvh * G + g) * nsplit + ch) * (D + 2) + D + 1] = l;
        }
    }
    __syncthreads();
    // weighted V from LDS: thread = (dim d, head group), 16 positions per
    // step with independent reads; rows past n_pos hold stale cache data and
    // are selected to 0 (a zero weight would not cancel a NaN)
    constexpr int HG = ATT_THREADS / D;
    constexpr int GJ = (G + HG - 1) / HG;
    const int d = tid % D, hg = tid / D;
    const int np = n_pos - p0 < ATT_CH ? n_pos - p0 : ATT_CH;
    float o[GJ];
#pragma unroll
    for (int j = 0; j < GJ; j++) o[j] = 0.f;
#pragma unroll
    for (int pb = 0; pb < ATT_CH; pb += 16) {
        if (pb < np) {   // uniform
            float vv[16];
#pragma unroll
            for (int i = 0; i < 16; i++) vv[i] = pb + i < np ? Vs[(pb + i) * D + d] : 0.f;
#pragma unroll
            for (int j = 0; j < GJ; j++) {
                const int g = hg + HG * j < G ? hg + HG * j : G - 1;
                const float4 *s4 = reinterpret_cast<const float4 *>(sc + g * ATT_CH + pb);
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const float4 w = s4[q4];
                    o[j] += w.x * vv[4 * q4] + w.y * vv[4 * q4 + 1] + w.z * vv[4 * q4 + 2] + w.w * vv[4 * q4 + 3];
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < GJ; j++) {
        const int g = hg + HG * j;
        if (g < G) part[((long long)(kvh * G + g) * nsplit + ch) * (D + 2) + d] = o[j];
    }
}

template <int D, int G>
constexpr size_t attn_lds_bytes() {
    return (size_t)4 * (ATT_CH * (D + 4) + ATT_CH * D + G * D + G * ATT_CH + ATT_PARTS * G * ATT_CH);
}

// out[h][d] = sum_c e^(m_c - M) o_c[d] / sum_c e^(m_c - M) l_c.  grid = NQ,
// D threads; the chunks' maxima and weights go through LDS (2 nsplit
// floats), and the weighted sum's loads are independent (unrolled).
template <int D>
__global__ __launch_bounds__(D) void k_attn_combine(const float *__restrict__ part, int nsplit, float *__restrict__ out) {
    extern __shared__ float cb_lds[];   // f[nsplit] | f * l[nsplit]
    const int h = blockIdx.x, d = threadIdx.x;
    const float *ph = part + (long long)h * nsplit * (D + 2);
    for (int c = d; c < nsplit; c += D) cb_lds[c] = ph[c * (D + 2) + D];
    __syncthreads();
    float M = -__builtin_huge_valf();
    for (int c = 0; c < nsplit; c++) M = fmaxf(M, cb_lds[c]);
    __syncthreads();
    for (int c = d; c < nsplit; c += D) {
        const float f = expf(cb_lds[c] - M);
        cb_lds[c] = f;
        cb_lds[nsplit + c] = f * ph[c * (D + 2) + D + 1];
    }
    __syncthreads();
    float num = 0.f, den = 0.f;
#pragma unroll 8
    for (int c = 0; c < nsplit; c++) {
        num += cb_lds[c] * ph[c * (D + 2) + d];
        den += cb_lds[nsplit + c];
    }
    out[h * D + d] = num / den;
}

// a = silu(g) * u with gu = [g (n) | u (n)] (unfused fallback).
__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ gu, int n, float *__restrict__ a) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) a[i] = pro_swiglu(gu[i], gu[n + i]);
}

struct DenseWs {
    float *x, *x2, *h, *qkv, *att, *y, *gu, *a, *part, *rope;
};

static size_t up256(size_t n) { return (n + 255) & ~(size_t)255; }

static DenseWs dense_ws(const tbq_dense_model *m, void *ws, size_t *total) {
    const size_t H = m->hidden, QD = (size_t)m->n_heads * m->head_dim, KD = (size_t)m->n_kv_heads * m->head_dim;
    const size_t nsplit = (m->max_ctx + ATT_CH - 1) / ATT_CH;
    char *p = (char *)ws;
    size_t off = 0;
    auto take = [&](size_t floats) {
        float *r = (float *)(p + off);
        off += up256(floats * 4);
        return r;
    };
    DenseWs w;
    w.x = take(H);
    w.x2 = take(H);
    w.h = take(H);
    w.qkv = take(QD + 2 * KD);
    w.att = take(QD);
    w.y = take(H > QD ? H : QD);
    w.gu = take(2 * (size_t)m->ffn);
    w.a = take(m->ffn);
    w.part = take((size_t)m->n_heads * nsplit * (m->head_dim + 2));
    w.rope = take(m->head_dim);
    if (total) *total = off;
    return w;
}

size_t dense_workspace_bytes(const tbq_dense_model *m) {
    size_t t = 0;
    dense_ws(m, nullptr, &t);
    return t;
}

template <int D, int G>
static hipError_t launch_attn(const float *qkv, const float *qn, const float *kn, int NQ, int NKV, int pos,
                              const float *rc, float eps, float *kc, float *vc, int max_ctx, float *part, float *out,
                              hipStream_t st) {
    const int nsplit = (pos + 1 + ATT_CH - 1) / ATT_CH;
    constexpr size_t lds = attn_lds_bytes<D, G>();
    static const hipError_t attr = hipFuncSetAttribute((const void *)k_attn_partial<D, G>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((k_attn_partial<D, G>), dim3(NKV, nsplit), dim3(ATT_THREADS), lds, st, qkv, qn, kn, NQ, pos,
                       rc, eps, kc, vc, max_ctx, nsplit, part);
    hipLaunchKernelGGL((k_attn_combine<D>), dim3(NQ), dim3(D), (size_t)2 * nsplit * 4, st, part, nsplit, out);
    return hipGetLastError();
}

template <int D>
static hipError_t launch_attn_d(int G, const float *qkv, const float *qn, const float *kn, int NQ, int NKV, int pos,
                                const float *rc, float eps, float *kc, float *vc, int max_ctx, float *part, float *out,
                                hipStream_t st) {
    switch (G) {
    case 1: return launch_attn<D, 1>(qkv, qn, kn, NQ, NKV, pos, rc, eps, kc, vc, max_ctx, part, out, st);
    case 2: return launch_attn<D, 2>(qkv, qn, kn, NQ, NKV, pos, rc, eps, kc, vc, max_ctx, part, out, st);
    case 4: return launch_attn<D, 4>(qkv, qn, kn, NQ, NKV, pos, rc, eps, kc, vc, max_ctx, part, out, st);
    case 8: return launch_attn<D, 8>(qkv, qn, kn, NQ, NKV, pos, rc, eps, kc, vc, max_ctx, part, out, st);
    default: return hipErrorNotSupported;
    }
}

// out = W prologue(x) for one matvec of the step (mode = PRO_* | MV_GLU):
// the kernels with the fused staging prologue / GLU epilogue where they
// cover the shape (the same choice of kernel as tbq_matvec otherwise), else
// the elementwise steps as launches of their own around tbq_matvec, through
// tmp_x (K floats) and tmp_y (2M floats, MV_GLU only).
static hipError_t dense_mv(int qt, const void *W, int M, int K, const float *x, float *out, int mode, const MvPro &pro,
                           float *tmp_x, float *tmp_y, hipStream_t st) {
    // the register-x Q4_K kernel for plain matvecs; with the norm prologue
    // the K-quant kernel, measured 1.3 us per layer faster at the Qwen3-4B
    // shapes
    hipError_t e = hipErrorNotSupported;
    if ((qt == QT_Q4_K || qt == QT_GQ4_K) && K <= 4096 && M <= 8192 && mode == PRO_NONE)
        e = launch_matvec_q4k_pro(mode, pro, W, M, K, x, out, st, qt == QT_GQ4_K);
    if (e == hipErrorNotSupported) e = launch_matvec_kq_pro(mode, pro, qt, W, M, K, x, out, st, tbq_cu_count());
    if (e != hipErrorNotSupported) return e;
    const float *xin = x;
    if (mode & PRO_NORM) {
        hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(1024), 0, st, x, pro.y, pro.w, K, pro.eps, tmp_x, pro.vo);
        xin = tmp_x;
    }
    if (!(mode & MV_GLU)) return tbq_matvec(W, qt, M, K, xin, out, st) ? hipSuccess : hipErrorUnknown;
    if (!tbq_matvec(W, qt, 2 * M, K, xin, tmp_y, st)) return hipErrorUnknown;
    hipLaunchKernelGGL(k_swiglu, dim3((M + 255) / 256), dim3(256), 0, st, tmp_y, M, out);
    return hipGetLastError();
}

// Validation happens in the C-ABI wrapper.  The residual stream alternates
// between w.x and w.x2: the add + RMSNorm before a matvec is that matvec's
// staging prologue, whose workgroup 0 stores x + y into the other buffer
// (the others are still reading x).
hipError_t launch_dense_decode(const tbq_dense_model *m, int token, int pos, float *logits, void *ws,
                               hipStream_t st) {
    const int H = m->hidden, D = m->head_dim, NQ = m->n_heads, NKV = m->n_kv_heads, G = NQ / NKV, F = m->ffn;
    const int QKVR = (NQ + 2 * NKV) * D;
    auto qt_of = [m](int q) { return canon_qt(q ? q : m->qtype_layers); };
    const DenseWs w = dense_ws(m, ws, nullptr);
    const size_t erb = tbq_row_bytes(m->qtype_embd, H);
    float *xa = w.x, *xb = w.x2;
    hipError_t err = launch_dequant(canon_qt(m->qtype_embd), (const uint8_t *)m->tok_embd + (size_t)token * erb, H, xa, st);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_rope_table, dim3(1), dim3(64), 0, st, pos, m->rope_theta, D, w.rope);
    const float *yprev = nullptr;
    for (int l = 0; l < m->n_layers; l++) {
        const tbq_dense_layer &L = m->layers[l];
        const size_t kvoff = (size_t)l * NKV * m->max_ctx * D;
        // qkv = Wqkv rmsnorm(xa + yprev); xb = xa + yprev (stored by the first
        // launch only when q, k and v are separate matrices)
        const MvPro pa{yprev, L.attn_norm, xb, m->norm_eps}, pa2{yprev, L.attn_norm, nullptr, m->norm_eps};
        if (L.wqkv) {
            err = dense_mv(qt_of(L.qt_qkv), L.wqkv, QKVR, H, xa, w.qkv, PRO_NORM, pa, w.h, nullptr, st);
        } else {
            err = dense_mv(qt_of(L.qt_q), L.wq, NQ * D, H, xa, w.qkv, PRO_NORM, pa, w.h, nullptr, st);
            if (err == hipSuccess)
                err = dense_mv(qt_of(L.qt_k), L.wk, NKV * D, H, xa, w.qkv + NQ * D, PRO_NORM, pa2, w.h, nullptr, st);
            if (err == hipSuccess)
                err = dense_mv(qt_of(L.qt_v), L.wv, NKV * D, H, xa, w.qkv + (NQ + NKV) * D, PRO_NORM, pa2, w.h,
                               nullptr, st);
        }
        if (err != hipSuccess) return err;
        err = D == 128 ? launch_attn_d<128>(G, w.qkv, L.q_norm, L.k_norm, NQ, NKV, pos, w.rope, m->norm_eps,
                                            m->k_cache + kvoff, m->v_cache + kvoff, m->max_ctx, w.part, w.att, st)
                       : launch_attn_d<64>(G, w.qkv, L.q_norm, L.k_norm, NQ, NKV, pos, w.rope, m->norm_eps,
                                           m->k_cache + kvoff, m->v_cache + kvoff, m->max_ctx, w.part, w.att, st);
        if (err != hipSuccess) return err;
        if ((err = dense_mv(qt_of(L.qt_o), L.wo, H, NQ * D, w.att, w.y, PRO_NONE, MvPro{}, nullptr, nullptr, st)) !=
            hipSuccess)
            return err;
        // a = silu(Wg h) * (Wu h) with h = rmsnorm(xb + y); xa = xb + y
        const MvPro pf{w.y, L.ffn_norm, xa, m->norm_eps}, pf2{w.y, L.ffn_norm, nullptr, m->norm_eps};
        if (L.wgu) {
            err = dense_mv(qt_of(L.qt_gu), L.wgu, F, H, xb, w.a, PRO_NORM | MV_GLU, pf, w.h, w.gu, st);
        } else {
            err = dense_mv(qt_of(L.qt_gate), L.wgate, F, H, xb, w.gu, PRO_NORM, pf, w.h, nullptr, st);
            if (err == hipSuccess)
                err = dense_mv(qt_of(L.qt_up), L.wup, F, H, xb, w.gu + F, PRO_NORM, pf2, w.h, nullptr, st);
            if (err == hipSuccess) {
                hipLaunchKernelGGL(k_swiglu, dim3((F + 255) / 256), dim3(256), 0, st, w.gu, F, w.a);
                err = hipGetLastError();
            }
        }
        if (err != hipSuccess) return err;
        // y = Wdown a
        if ((err = dense_mv(qt_of(L.qt_down), L.wdown, H, F, w.a, w.y, PRO_NONE, MvPro{}, nullptr, nullptr, st)) !=
            hipSuccess)
            return err;
        yprev = w.y;
    }
    const MvPro po{yprev, m->output_norm, nullptr, m->norm_eps};
    if ((err = dense_mv(canon_qt(m->qtype_embd), m->lm_head, m->vocab, H, xa, logits, PRO_NORM, po, w.h, nullptr, st)) !=
        hipSuccess)
        return err;
    return hipGetLastError();
}

// logits = Wlm rmsnorm(x + y) * output_norm for one residual row x and the
// last sublayer's output y (the prefill's last token); ws is a decode
// workspace.
hipError_t dense_final_logits(const tbq_dense_model *m, const float *x, const float *y, float *logits, void *ws,
                              hipStream_t st) {
    const DenseWs w = dense_ws(m, ws, nullptr);
    const MvPro po{y, m->output_norm, nullptr, m->norm_eps};
    const hipError_t err =
        dense_mv(canon_qt(m->qtype_embd), m->lm_head, m->vocab, m->hidden, x, logits, PRO_NORM, po, w.h, nullptr, st);
    return err != hipSuccess ? err : hipGetLastError();
}

}  // namespace tbq
