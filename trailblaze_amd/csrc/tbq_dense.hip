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

// res[i] += v[i] (PRO_RES's epilogue as a launch of its own).
__global__ __launch_bounds__(256) void k_res_add(float *__restrict__ res, const float *__restrict__ v, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) res[i] = res[i] + v[i];
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

// Inputs of head_norm_rope for one head vector held by one wave: lane l
// has elements l and l + 64 (D = 128) or l (D = 64), their norm weights and
// the cos / sin of its rotation pair.  Loading them apart from the
// arithmetic lets a kernel issue these loads ahead of larger ones.
template <int D>
struct HeadIn {
    float x[D / 64], w[D / 64], cs, sn;
};

template <int D>
__device__ __forceinline__ void head_load(HeadIn<D> &h, const float *__restrict__ x, const float *__restrict__ w,
                                          const float *__restrict__ rc) {
    const int lane = threadIdx.x & 63, j = lane % (D / 2);
#pragma unroll
    for (int i = 0; i < D / 64; i++) {
        h.x[i] = x[lane + 64 * i];
        h.w[i] = w[lane + 64 * i];
    }
    h.cs = rc[j];
    h.sn = rc[D / 2 + j];
}

// RMSNorm with the head's norm weights then rotate-half RoPE (table rc),
// in place on h.x.
template <int D>
__device__ __forceinline__ void head_norm_rope(HeadIn<D> &h, float eps) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < D / 64; i++) ss += h.x[i] * h.x[i];
    ss = group_sum<64>(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int i = 0; i < D / 64; i++) h.x[i] = h.x[i] * r * h.w[i];
    if constexpr (D == 128) {
        const float a = h.x[0], b = h.x[1];   // elements j and j + 64
        h.x[0] = a * h.cs - b * h.sn;
        h.x[1] = a * h.sn + b * h.cs;
    } else {
        const float other = __shfl_xor(h.x[0], 32);   // partner j +- 32
        h.x[0] = lane < 32 ? h.x[0] * h.cs - other * h.sn : other * h.sn + h.x[0] * h.cs;
    }
}

constexpr int ilog2c(int n) { return n <= 1 ? 0 : 1 + ilog2c(n / 2); }

constexpr int DPP_ROR4 = 0x124, DPP_ROR8 = 0x128;   // row_ror:4 / row_ror:8 (xor 8)

// The DPP exchange that pairs lanes differing in lane bit B (B <= 3) within
// a row of 16: xor 8 (row_ror:8), i <-> 7-i (half mirror), xor 2, xor 1.
template <int B>
__device__ __forceinline__ float xrow_dpp(float v) {
    if constexpr (B == 3) return dpp_f32<DPP_ROR8>(v);
    else if constexpr (B == 2) return dpp_f32<DPP_HALF_MIRROR>(v);
    else if constexpr (B == 1) return dpp_f32<DPP_QXOR2>(v);
    else return dpp_f32<DPP_QXOR1>(v);
}

// Transposing sum over the lanes of an aligned group of 2^(B+1) lanes, lane
// bits B..0 in turn.  With C > 1 values left a step pairs the lanes that
// differ in bit B: the lane with the bit clear keeps the sums of values
// 0..C/2-1, its partner those of C/2..C-1, so one exchange serves two
// values.  With one value left a step is a plain sum over the pair.  At the
// end lane l of the group holds in a[0..] the sums of values
// (l >> S) * C' + j, j < C' = max(1, N / 2^(B+1)), where S = log2 of the
// number of lanes that share each value.
template <int B, int C, int N>
__device__ __forceinline__ void group_xsum(float (&a)[N], int lane) {
    if constexpr (C >= 2) {
        const bool hi = (lane >> B) & 1;
#pragma unroll
        for (int j = 0; j < C / 2; j++) {
            const float x = a[j], y = a[j + C / 2];
            if constexpr (B == 4) {   // rows of 16 lanes 0 <-> 1, 2 <-> 3
                const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                                __builtin_bit_cast(uint32_t, y), false, false);
                const uint32_t r0 = r[0], r1 = r[1];
                a[j] = __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
            } else {
                a[j] = (hi ? y : x) + xrow_dpp<B>(hi ? x : y);
            }
        }
    } else {
        if constexpr (B == 4) a[0] = swap16_sum(a[0]);
        else a[0] += xrow_dpp<B>(a[0]);
    }
    if constexpr (B > 0) group_xsum<B - 1, (C >= 2 ? C / 2 : 1), N>(a, lane);
}

// Max / sum over the 16 lanes of the wave that agree in lane bits 0 and 1;
// every lane gets it.
__device__ __forceinline__ float wave_max_hi4(float v) {
    v = fmaxf(v, dpp_f32<DPP_ROR4>(v));
    v = fmaxf(v, dpp_f32<DPP_ROR8>(v));
    v = swap16_max(v);
    return swap32_max(v);
}
__device__ __forceinline__ float wave_sum_hi4(float v) {
    v += dpp_f32<DPP_ROR4>(v);
    v += dpp_f32<DPP_ROR8>(v);
    v = swap16_sum(v);
    return swap32_sum(v);
}

// Attention for one kv head x one chunk of ATT_CH positions, all G query
// heads of the head, with the head's QK-norm, RoPE and cache append folded
// in.  The chunk's K and V rows stay in registers: thread (row group
// R = tid / (D/4), column c = tid % (D/4)) loads dims 4c..4c+3 of rows
// R + RS*i, i < NL (RS = ATT_THREADS / (D/4)).  The query rows, norm weights
// and RoPE pairs are loaded before the chunk, so they land first; the waves
// normalise and rotate the query heads into LDS while K and V are in flight,
// and the scores start as the K rows land.
//   scores   each thread forms the NL x G partial dot products of its
//            columns; a transposing sum over the D/4 lanes of the row group
//            leaves every lane with whole scores;
//   softmax  max and sum per wave and head over the 16 lanes that hold the
//            head (lane bits 2..5); the weights go through a wave-private
//            LDS slot to every lane of the row group;
//   V        each thread sums weight x V over its rows and columns;
//   merge    after one barrier, thread (head, dim) rescales the waves'
//            partial sums to the chunk's max.
// The chunk that holds `pos` also forms the new K row (norm + RoPE) and V
// row, uses them in place of the cache's and writes them to the cache.
// Rows past pos are loaded from row pos, then take the new row (the cache
// row may hold anything, and a zero weight would not cancel a NaN) and are
// scored -inf.  Writes
// part[(qh * nsplit + chunk) * (D + 2) + {0..D-1, D: max, D+1: denominator}].
// grid = (NKV, nsplit), ATT_THREADS threads.
template <int D, int G>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_partial(const float *__restrict__ qkv, const float *__restrict__ qn,
                                                              const float *__restrict__ kn, int NQ, int pos,
                                                              const float *__restrict__ rc, float eps, float *__restrict__ kc,
                                                              float *__restrict__ vc, int max_ctx, int nsplit,
                                                              float *__restrict__ part) {
    static_assert(D == 64 || D == 128, "head_dim");
    constexpr int LR = D / 4, LB = ilog2c(LR), RS = ATT_THREADS / LR, NL = ATT_CH / RS;
    constexpr int NW = ATT_THREADS / 64, RPW = 64 / LR, NV = NL * G, LG = ilog2c(G);
    constexpr int CV = NV > LR ? NV / LR : 1;           // whole scores per lane
    constexpr int SH = NV < LR ? LB - ilog2c(NV) : 0;   // low lane bits that share a score
    static_assert(G <= NW && (1 << LG) == G, "one query head per wave, G a power of two");
    static_assert(ATT_CH % RS == 0 && NV % 4 == 0, "chunk layout");
    static_assert(LB - ilog2c(NL) == 2 && SH <= 2, "score positions sit in lane bits 2..5");
    __shared__ __attribute__((aligned(16))) float qs[G * D];                 // scaled query heads
    __shared__ __attribute__((aligned(16))) float nrow[2 * D];               // new K | V row
    __shared__ __attribute__((aligned(16))) float pw[NW * RPW * NV];         // weights per row group
    __shared__ __attribute__((aligned(16))) float os[NW * RPW * G * D];      // weighted V per row group
    __shared__ float mw[NW * G], lw[NW * G];                                 // per wave max, sum
    const int kvh = blockIdx.x, ch = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n_pos = pos + 1, p0 = ch * ATT_CH;
    const long long hbase = (long long)kvh * max_ctx * D;
    const bool own = pos >= p0 && pos < p0 + ATT_CH;   // this chunk holds the new row
    const bool newrow = own && wave == NW - 1;
    HeadIn<D> hq, hk;
    float nv[D / 64];
    if (wave < G) head_load<D>(hq, qkv + (kvh * G + wave) * D, qn, rc);
    if (newrow) {
        head_load<D>(hk, qkv + (NQ + kvh) * D, kn, rc);
#pragma unroll
        for (int i = 0; i < D / 64; i++) nv[i] = qkv[(NQ + (int)gridDim.x + kvh) * D + lane + 64 * i];
    }
    asm volatile("" ::: "memory");   // the small rows are issued first
    const int R = tid >> LB, c4 = tid & (LR - 1);
    float4 kr[NL], vr[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int pp = p0 + R + RS * i < n_pos ? p0 + R + RS * i : n_pos - 1;
        kr[i] = *reinterpret_cast<const float4 *>(kc + hbase + (long long)pp * D + 4 * c4);
    }
    asm volatile("" ::: "memory");   // K ahead of V
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int pp = p0 + R + RS * i < n_pos ? p0 + R + RS * i : n_pos - 1;
        vr[i] = *reinterpret_cast<const float4 *>(vc + hbase + (long long)pp * D + 4 * c4);
    }
    const float scale = 1.0f / sqrtf((float)D);
    if (wave < G) {
        head_norm_rope<D>(hq, eps);
#pragma unroll
        for (int i = 0; i < D / 64; i++) qs[wave * D + lane + 64 * i] = hq.x[i] * scale;
    }
    if (newrow) {
        head_norm_rope<D>(hk, eps);
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            nrow[lane + 64 * i] = hk.x[i];
            nrow[D + lane + 64 * i] = nv[i];
            kc[hbase + (long long)pos * D + lane + 64 * i] = hk.x[i];
            vc[hbase + (long long)pos * D + lane + 64 * i] = nv[i];
        }
    }
    // LDS-only barrier: the chunk's loads stay in flight across it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    float4 qv[G];
#pragma unroll
    for (int g = 0; g < G; g++) qv[g] = *reinterpret_cast<const float4 *>(qs + g * D + 4 * c4);
    // rows pos.. of the chunk that holds pos take the new row (rows past pos
    // are weighed 0, and the new row is finite where the stale cache may not be)
    if (own) {
        const float4 k4 = *reinterpret_cast<const float4 *>(nrow + 4 * c4);
#pragma unroll
        for (int i = 0; i < NL; i++)
            if (p0 + R + RS * i >= pos) kr[i] = k4;
    }
    // scores of (row R + RS*i, head g) at value index i*G + g
    float a[NV];
#pragma unroll
    for (int i = 0; i < NL; i++)
#pragma unroll
        for (int g = 0; g < G; g++)
            a[i * G + g] = fmaf(qv[g].w, kr[i].w, fmaf(qv[g].z, kr[i].z, fmaf(qv[g].y, kr[i].y, qv[g].x * kr[i].x)));
    group_xsum<LB - 1, NV, NV>(a, lane);
    const int li = lane & (LR - 1), rg = lane >> LB;
    float *pr = pw + (wave * RPW + rg) * NV;
#pragma unroll
    for (int j = 0; j < CV; j++) {
        const int v = (li >> SH) * CV + j, i = v >> LG, g = v & (G - 1);
        const bool valid = p0 + R + RS * i < n_pos;
        const float s = valid ? a[j] : -__builtin_huge_valf();
        const float m = wave_max_hi4(s);
        const float e = valid ? expf(s - m) : 0.f;
        pr[v] = e;
        const float l = wave_sum_hi4(e);
        if ((lane & 60) == 0) {
            mw[wave * G + g] = m;
            lw[wave * G + g] = l;
        }
    }
    if (own) {
        const float4 v4 = *reinterpret_cast<const float4 *>(nrow + D + 4 * c4);
#pragma unroll
        for (int i = 0; i < NL; i++)
            if (p0 + R + RS * i >= pos) vr[i] = v4;
    }
    // weighted V; the weights were written by lanes of this wave (LDS keeps
    // a wave's accesses in order)
    float4 o[G];
#pragma unroll
    for (int i = 0; i < NL; i++) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float w = pr[i * G + g];
            if (i == 0) {
                o[g] = make_float4(w * vr[0].x, w * vr[0].y, w * vr[0].z, w * vr[0].w);
            } else {
                o[g].x = fmaf(w, vr[i].x, o[g].x);
                o[g].y = fmaf(w, vr[i].y, o[g].y);
                o[g].z = fmaf(w, vr[i].z, o[g].z);
                o[g].w = fmaf(w, vr[i].w, o[g].w);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) *reinterpret_cast<float4 *>(os + ((wave * RPW + rg) * G + g) * D + 4 * c4) = o[g];
    __syncthreads();
    for (int idx = tid; idx < G * D; idx += ATT_THREADS) {
        const int g = idx / D, d = idx % D;
        float M = -__builtin_huge_valf();
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, mw[w * G + g]);
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = expf(mw[w * G + g] - M);   // 0 for a wave with no row below n_pos
            float t = 0.f;
#pragma unroll
            for (int r = 0; r < RPW; r++) t += os[((w * RPW + r) * G + g) * D + d];
            num += f * t;
            den += f * lw[w * G + g];
        }
        float *dst = part + ((long long)(kvh * G + g) * nsplit + ch) * (D + 2);
        dst[d] = num;
        if (d == 0) {
            dst[D] = M;
            dst[D + 1] = den;
        }
    }
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
    hipLaunchKernelGGL((k_attn_partial<D, G>), dim3(NKV, nsplit), dim3(ATT_THREADS), 0, st, qkv, qn, kn, NQ, pos, rc,
                       eps, kc, vc, max_ctx, nsplit, part);
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
    // the register-x Q4_K kernel for plain matvecs, the residual epilogue
    // and the deferred RMSNorm (q|k|v at the Qwen3-4B shapes: 1584 -> 1568
    // us/token against the K-quant kernel, with the norm's sum of squares
    // then read from partials the producer wrote); with the block-sum
    // prologue (PRO_NORM) the K-quant kernel, measured 1.3 us per layer
    // faster there
    hipError_t e = hipErrorNotSupported;
    if ((qt == QT_Q4_K || qt == QT_GQ4_K) && K <= 4096 && M <= 8192 &&
        (mode == PRO_NONE || mode == PRO_RES || mode == PRO_NORMD))
        e = launch_matvec_q4k_pro(mode, pro, W, M, K, x, out, st, qt == QT_GQ4_K);
    if (e == hipErrorNotSupported) e = launch_matvec_kq_pro(mode, pro, qt, W, M, K, x, out, st, tbq_cu_count());
    if (e != hipErrorNotSupported) return e;
    if (mode == PRO_RES) {
        if (!tbq_matvec(W, qt, M, K, x, tmp_y, st)) return hipErrorUnknown;
        hipLaunchKernelGGL(k_res_add, dim3((M + 255) / 256), dim3(256), 0, st, out, tmp_y, M);
        return hipGetLastError();
    }
    const float *xin = x;
    if (mode & PRO_NORM) {
        hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(1024), 0, st, x, pro.y, pro.w, K, pro.eps, tmp_x, pro.vo);
        xin = tmp_x;
    } else if (mode & PRO_NORMD) {
        hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(1024), 0, st, x, nullptr, pro.w, K, pro.eps, tmp_x, nullptr);
        xin = tmp_x;
    }
    if (!(mode & MV_GLU)) return tbq_matvec(W, qt, M, K, xin, out, st) ? hipSuccess : hipErrorUnknown;
    if (!tbq_matvec(W, qt, 2 * M, K, xin, tmp_y, st)) return hipErrorUnknown;
    hipLaunchKernelGGL(k_swiglu, dim3((M + 255) / 256), dim3(256), 0, st, tmp_y, M, out);
    return hipGetLastError();
}

// Validation happens in the C-ABI wrapper.  The residual stream lives in
// w.x: the o and down matvecs add their rows to it in place (PRO_RES), and
// each RMSNorm is the next matvec's PRO_NORMD (x * w staged, the scale
// applied to the dot products, the sum of squares taken over the staged x
// at the staging barrier), so no launch waits on a reduction of its own.
hipError_t launch_dense_decode(const tbq_dense_model *m, int token, int pos, float *logits, void *ws,
                               hipStream_t st) {
    const int H = m->hidden, D = m->head_dim, NQ = m->n_heads, NKV = m->n_kv_heads, G = NQ / NKV, F = m->ffn;
    const int QKVR = (NQ + 2 * NKV) * D;
    auto qt_of = [m](int q) { return canon_qt(q ? q : m->qtype_layers); };
    const DenseWs w = dense_ws(m, ws, nullptr);
    const size_t erb = tbq_row_bytes(m->qtype_embd, H);
    float *res = w.x;
    hipError_t err = launch_dequant(canon_qt(m->qtype_embd), (const uint8_t *)m->tok_embd + (size_t)token * erb, H, res, st);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_rope_table, dim3(1), dim3(64), 0, st, pos, m->rope_theta, D, w.rope);
    // rmsnorm(res) * wn as the next matvec's prologue
    auto norm_pro = [&](const float *wn, int *mode) {
        *mode = PRO_NORMD;
        return MvPro{nullptr, wn, nullptr, m->norm_eps};
    };
    const MvPro pres{};
    for (int l = 0; l < m->n_layers; l++) {
        const tbq_dense_layer &L = m->layers[l];
        const size_t kvoff = (size_t)l * NKV * m->max_ctx * D;
        // qkv = Wqkv rmsnorm(res)
        int pm;
        const MvPro pa = norm_pro(L.attn_norm, &pm);
        if (L.wqkv) {
            err = dense_mv(qt_of(L.qt_qkv), L.wqkv, QKVR, H, res, w.qkv, pm, pa, w.h, nullptr, st);
        } else {
            err = dense_mv(qt_of(L.qt_q), L.wq, NQ * D, H, res, w.qkv, pm, pa, w.h, nullptr, st);
            if (err == hipSuccess)
                err = dense_mv(qt_of(L.qt_k), L.wk, NKV * D, H, res, w.qkv + NQ * D, pm, pa, w.h, nullptr, st);
            if (err == hipSuccess)
                err = dense_mv(qt_of(L.qt_v), L.wv, NKV * D, H, res, w.qkv + (NQ + NKV) * D, pm, pa, w.h, nullptr,
                               st);
        }
        if (err != hipSuccess) return err;
        err = D == 128 ? launch_attn_d<128>(G, w.qkv, L.q_norm, L.k_norm, NQ, NKV, pos, w.rope, m->norm_eps,
                                            m->k_cache + kvoff, m->v_cache + kvoff, m->max_ctx, w.part, w.att, st)
                       : launch_attn_d<64>(G, w.qkv, L.q_norm, L.k_norm, NQ, NKV, pos, w.rope, m->norm_eps,
                                           m->k_cache + kvoff, m->v_cache + kvoff, m->max_ctx, w.part, w.att, st);
        if (err != hipSuccess) return err;
        // res += Wo att
        if ((err = dense_mv(qt_of(L.qt_o), L.wo, H, NQ * D, w.att, res, PRO_RES, pres, nullptr, w.y, st)) !=
            hipSuccess)
            return err;
        // a = silu(Wg h) * (Wu h) with h = rmsnorm(res)
        const MvPro pf = norm_pro(L.ffn_norm, &pm);
        if (L.wgu) {
            err = dense_mv(qt_of(L.qt_gu), L.wgu, F, H, res, w.a, pm | MV_GLU, pf, w.h, w.gu, st);
        } else {
            err = dense_mv(qt_of(L.qt_gate), L.wgate, F, H, res, w.gu, pm, pf, w.h, nullptr, st);
            if (err == hipSuccess) err = dense_mv(qt_of(L.qt_up), L.wup, F, H, res, w.gu + F, pm, pf, w.h, nullptr, st);
            if (err == hipSuccess) {
                hipLaunchKernelGGL(k_swiglu, dim3((F + 255) / 256), dim3(256), 0, st, w.gu, F, w.a);
                err = hipGetLastError();
            }
        }
        if (err != hipSuccess) return err;
        // res += Wdown a
        if ((err = dense_mv(qt_of(L.qt_down), L.wdown, H, F, w.a, res, PRO_RES, pres, nullptr, w.y, st)) !=
            hipSuccess)
            return err;
    }
    int pm;
    const MvPro po = norm_pro(m->output_norm, &pm);
    if ((err = dense_mv(canon_qt(m->qtype_embd), m->lm_head, m->vocab, H, res, logits, pm, po, w.h, nullptr, st)) !=
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
