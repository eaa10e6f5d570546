// tbq_dense_prefill.hip -- batched prefill of a dense Qwen3-style model on
// gfx950: the T prompt tokens at positions pos0 .. pos0 + T - 1 go through
// each layer together, where the reference prefills token by token
// (layer4/tb_infer.c:1068-1075: one tb_infer_decode step per prompt token).
//
// Per layer (x: fp32 residual rows [T][H]; h16: fp16 rows with per-row
// power-of-two scales, the GEMMs' activation operand; each weight matrix
// is dequantised to fp16 (k_dequant_f16, any format or layout) just before
// its GEMM, into one reused buffer):
//   k_pf_norm        x += y (the previous sublayer's output, unscaled by
//                    its row scales), h16 = rmsnorm(x) * attn_norm
//   GEMM             qkv = h16 Wqkv^T             rocBLAS fp16, fp32 acc
//   k_pf_qk          per (token, head): QK-norm + RoPE of q (to qb) and k;
//                    k and v rows written to the cache at pos0 + t
//   k_pf_attn        causal GQA attention over cache positions 0 .. pos,
//                    online softmax, key ranges split over workgroups
//                    (k_pf_attn_combine merges them)
//   rows to fp16, GEMM            y = att Wo^T
//   k_pf_norm        x += y, h16 = rmsnorm(x) * ffn_norm
//   GEMM             gu = h16 [Wg | Wu]^T
//   k_pf_swiglu_f16  a16 = silu(g) * u (fp16, row scales)
//   GEMM             y = a16 Wdown^T
// then the last token's logits = Wlm rmsnorm(x + y) (the decode step's
// lm_head matvec with its norm prologue).
//
// Accuracy: fp16 weights and activations (11-bit mantissa) with fp32
// accumulation, fp32 norms, RoPE and attention; the logits land within
// 1e-2 relative L2 of the float64 sequential decode.
#include <rocblas/rocblas.h>

#include <algorithm>
#include <mutex>

#include "tbq_kernels.h"
#include "tbq_device.hpp"
#include "../../include/tbq.h"

namespace tbq {

constexpr int PN_THREADS = 256;
constexpr int PA_THREADS = 256;
constexpr int PA_KC = 8;      // cache positions per attention step
constexpr int PA_KF = 32;     // cache positions per LDS fill (PA_KF / PA_KC steps)

__device__ __forceinline__ float pf_block_sum(float v, float *red) {
    v = group_sum<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < PN_THREADS / 64; i++) r += red[i];
    return r;
}

__device__ __forceinline__ float pf_block_max(float v, float *red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < PN_THREADS / 64; i++) r = fmaxf(r, red[i]);
    return r;
}

// Row t: v = x[t] + y[t] * ys[t] (y may be null; x[t] = v is stored back
// when y is not; ys, the row scales of a GEMM's fp16 operand, may be null
// for 1), h = v * rsqrt(mean(v^2) + eps) * w, then h16[t] = h * 2^s in fp16
// with s putting max |h| in [2^14, 2^15) and hinv[t] = 2^-s.  grid = T.
// A thread holds up to PN_V float4 of the row (H <= 8192), all loaded
// before any is used.
constexpr int PN_V = 8;
__global__ __launch_bounds__(PN_THREADS) void k_pf_norm(float *__restrict__ x, const float *__restrict__ y,
                                                        const float *__restrict__ ys, const float *__restrict__ w,
                                                        int H, float eps, _Float16 *__restrict__ h16,
                                                        float *__restrict__ hinv) {
    __shared__ float red[PN_THREADS / 64];
    const int t = blockIdx.x, tid = threadIdx.x, n4 = H / 4;
    float4 *xr = reinterpret_cast<float4 *>(x + (long long)t * H);
    const float4 *yr = reinterpret_cast<const float4 *>(y ? y + (long long)t * H : x + (long long)t * H);
    const float4 *wr = reinterpret_cast<const float4 *>(w);
    float4 v[PN_V], b[PN_V], g[PN_V];
#pragma unroll
    for (int i = 0; i < PN_V; i++) {
        const int j = min(tid + PN_THREADS * i, n4 - 1);   // clamped: loads stay unconditional
        v[i] = xr[j];
        b[i] = yr[j];
        g[i] = wr[j];
    }
    float ss = 0.f;
    const float yscale = ys ? ys[t] : 1.f;
#pragma unroll
    for (int i = 0; i < PN_V; i++) {
        if (y) {
            v[i].x += b[i].x * yscale; v[i].y += b[i].y * yscale;
            v[i].z += b[i].z * yscale; v[i].w += b[i].w * yscale;
        }
        if (tid + PN_THREADS * i < n4) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    }
    if (y) {
#pragma unroll
        for (int i = 0; i < PN_V; i++)
            if (tid + PN_THREADS * i < n4) xr[tid + PN_THREADS * i] = v[i];
    }
    ss = pf_block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)H + eps);
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < PN_V; i++) {
        v[i].x = v[i].x * r * g[i].x; v[i].y = v[i].y * r * g[i].y;
        v[i].z = v[i].z * r * g[i].z; v[i].w = v[i].w * r * g[i].w;
        if (tid + PN_THREADS * i < n4)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    mx = pf_block_max(mx, red);
    int e = 0;
    frexpf(mx, &e);
    int sh = mx > 0.f ? 15 - e : 0;
    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
    const float s = ldexpf(1.f, sh);
    uint2 *hr = reinterpret_cast<uint2 *>(h16 + (long long)t * H);
#pragma unroll
    for (int i = 0; i < PN_V; i++) {
        const int j = tid + PN_THREADS * i;
        if (j < n4) {
            const _Float16 a0 = (_Float16)(v[i].x * s), a1 = (_Float16)(v[i].y * s);
            const _Float16 a2 = (_Float16)(v[i].z * s), a3 = (_Float16)(v[i].w * s);
            hr[j] = make_uint2((uint32_t)__builtin_bit_cast(uint16_t, a0) | ((uint32_t)__builtin_bit_cast(uint16_t, a1) << 16),
                               (uint32_t)__builtin_bit_cast(uint16_t, a2) | ((uint32_t)__builtin_bit_cast(uint16_t, a3) << 16));
        }
    }
    if (tid == 0) hinv[t] = ldexpf(1.f, -sh);
}

// Head vector (one wave; lane l holds elements l and l + 64, or l for
// D = 64): RMSNorm with the head's weights, then rotate-half RoPE at
// position pos, the angle formed as the decode step's table forms it.
template <int D>
__device__ __forceinline__ void pf_norm_rope(float (&x)[D / 64], const float *__restrict__ w, int pos, float theta,
                                             float eps) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < D / 64; i++) ss += x[i] * x[i];
    ss = group_sum<64>(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int i = 0; i < D / 64; i++) x[i] = x[i] * r * w[lane + 64 * i];
    const int j = lane % (D / 2);
    double sd, cd;
    sincos((double)pos * pow((double)theta, -2.0 * j / D), &sd, &cd);
    const float cs = (float)cd, sn = (float)sd;
    if constexpr (D == 128) {
        const float a = x[0], b = x[1];
        x[0] = a * cs - b * sn;
        x[1] = a * sn + b * cs;
    } else {
        const float other = __shfl_xor(x[0], 32);
        x[0] = lane < 32 ? x[0] * cs - other * sn : other * sn + x[0] * cs;
    }
}

// grid = (T, NQ + NKV), one wave; qkv row t times rs[t] is the true row.
// Head hh < NQ: q head hh of token t,
// normed, rotated and scaled by 1/sqrt(D) into qb[t][hh]; else k head
// hh - NQ, normed and rotated, and the matching v head, written to the
// layer's cache rows pos0 + t.
template <int D>
__global__ __launch_bounds__(64) void k_pf_qk(const float *__restrict__ qkv, const float *__restrict__ rs,
                                              const float *__restrict__ qn, const float *__restrict__ kn, int NQ,
                                              int NKV, int pos0, float theta, float eps, float *__restrict__ kc,
                                              float *__restrict__ vc, int max_ctx, float *__restrict__ qb) {
    const int t = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
    const int QKVR = (NQ + 2 * NKV) * D, pos = pos0 + t;
    const float sc = rs[t];   // row t of qkv is scaled by 1 / rs[t]
    const float *src = qkv + (long long)t * QKVR + hh * D;
    float x[D / 64];
#pragma unroll
    for (int i = 0; i < D / 64; i++) x[i] = src[lane + 64 * i] * sc;
    pf_norm_rope<D>(x, hh < NQ ? qn : kn, pos, theta, eps);
    if (hh < NQ) {
        const float scale = 1.0f / sqrtf((float)D);
#pragma unroll
        for (int i = 0; i < D / 64; i++) qb[((long long)t * NQ + hh) * D + lane + 64 * i] = x[i] * scale;
    } else {
        const int kvh = hh - NQ;
        const long long row = ((long long)kvh * max_ctx + pos) * D;
        const float *vsrc = qkv + (long long)t * QKVR + (NQ + NKV + kvh) * D;
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            kc[row + lane + 64 * i] = x[i];
            vc[row + lane + 64 * i] = vsrc[lane + 64 * i] * sc;
        }
    }
}

// Row t: a = silu(g * s) * (u * s) with gu[t] = [g (F) | u (F)] and s =
// gs[t], then a16[t] = a * 2^e in fp16 (max |a| in [2^14, 2^15)) and
// ainv[t] = 2^-e.  grid = T, two passes over the row.
__global__ __launch_bounds__(PN_THREADS) void k_pf_swiglu_f16(const float *__restrict__ gu, const float *__restrict__ gs,
                                                              int F, _Float16 *__restrict__ a16,
                                                              float *__restrict__ ainv) {
    __shared__ float red[PN_THREADS / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float *g = gu + (long long)t * 2 * F, *u = g + F;
    const float s = gs[t];
    float mx = 0.f;
    for (int j = tid; j < F; j += PN_THREADS) mx = fmaxf(mx, fabsf(pro_swiglu(g[j] * s, u[j] * s)));
    mx = pf_block_max(mx, red);
    int e = 0;
    frexpf(mx, &e);
    int sh = mx > 0.f ? 15 - e : 0;
    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
    const float sc = ldexpf(1.f, sh);
    _Float16 *ar = a16 + (long long)t * F;
    for (int j = tid; j < F; j += PN_THREADS) ar[j] = (_Float16)(pro_swiglu(g[j] * s, u[j] * s) * sc);
    if (tid == 0) ainv[t] = ldexpf(1.f, -sh);
}

// y[j] *= ys[0] for one row of n floats (the last token's down output
// before the lm_head).
__global__ __launch_bounds__(256) void k_pf_scale_row(float *__restrict__ y, const float *__restrict__ ys, int n) {
    for (int j = threadIdx.x; j < n; j += 256) y[j] *= ys[0];
}

// Causal attention.  grid = (NKV, ceil(T / QB)), 256 threads: the
// workgroup owns QB = 64 / G tokens x the G query heads of kv head kvh = 64
// query rows.  PA_TPR = 16 lanes share PA_R = 4 rows, each lane holding a
// sixteenth of the head dimension of all four (dims 4qq + 4 PA_TPR i + c,
// so a row group's lanes read one contiguous LDS run), so every K and V
// value read from LDS serves four rows.  Cache positions 0 .. the block's
// last position pass through LDS PA_KF at a time, the next fill's rows
// loaded into registers while the current one is used; per PA_KC step each row
// forms its scores (partial dots summed over the 16 lanes), masks
// positions past its own, and updates its running max, denominator and
// output (online softmax).  Position 0 is in every row's range, so the
// running maxima are finite after the first chunk.
constexpr int PA_TPR = 16, PA_R = 4;
constexpr int PA_ROWS = PA_THREADS / PA_TPR * PA_R;

//
// Key splits: grid.z = nsplit workgroups per block, split z taking cache
// positions [z ks, (z + 1) ks) (ks a multiple of PA_KF), so the heavy
// blocks of a causal prompt (whose rows see every earlier position) are
// spread over several workgroups.  With nsplit > 1 each writes its rows'
// unnormalised output, running max and denominator to part[(row * nsplit
// + z) * (D + 2)], and k_pf_attn_combine merges the splits a row reaches.
template <int D, int G>
__global__ __launch_bounds__(PA_THREADS) void k_pf_attn(const float *__restrict__ qb, const float *__restrict__ kc,
                                                        const float *__restrict__ vc, int T, int pos0, int NQ,
                                                        int max_ctx, int ks, int nsplit, float *__restrict__ part,
                                                        float *__restrict__ out) {
    constexpr int QB = PA_ROWS / G, DQ = D / PA_TPR, NI = DQ / 4;
    constexpr int NF = PA_KF * D / 4;                  // float4 of K (and of V) per fill
    constexpr int NL = (NF + PA_THREADS - 1) / PA_THREADS;
    static_assert(NI >= 1, "shape");
    __shared__ __attribute__((aligned(16))) float Ks[PA_KF][D];
    __shared__ __attribute__((aligned(16))) float Vs[PA_KF][D];
    const int kvh = blockIdx.x, tid = threadIdx.x, rg = tid / PA_TPR, qq = tid % PA_TPR;
    const int tend = min(T, (int)(blockIdx.y + 1) * QB);
    const int k0 = blockIdx.z * ks;                  // this split's positions k0 .. kend - 1
    const int kend = min(pos0 + tend, k0 + ks);
    if (k0 >= kend) return;   // no position of the split is seen by the block (uniform)
    const float *kb = kc + (long long)kvh * max_ctx * D;
    const float *vb = vc + (long long)kvh * max_ctx * D;
    // native vectors: arrays of HIP's float4 struct carried across loop
    // iterations are kept in scratch memory
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 kn[NL], vn[NL];
    auto fetch = [&](int c0) {
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int f = tid + PA_THREADS * i, row = f / (D / 4), c4 = f % (D / 4);
            const long long p = min(c0 + row, kend - 1);
            kn[i] = *reinterpret_cast<const f32x4 *>(kb + p * D + 4 * c4);
            vn[i] = *reinterpret_cast<const f32x4 *>(vb + p * D + 4 * c4);
        }
    };
    fetch(k0);
    int qpos[PA_R];
    float q[PA_R][DQ], o[PA_R][DQ], m[PA_R], l[PA_R];
#pragma unroll
    for (int k = 0; k < PA_R; k++) {
        const int rr = rg * PA_R + k, g = rr % G, t = min((int)blockIdx.y * QB + rr / G, T - 1);
        qpos[k] = pos0 + t;
        const float *qsrc = qb + ((long long)t * NQ + kvh * G + g) * D + 4 * qq;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                q[k][4 * i + c] = qsrc[4 * PA_TPR * i + c];
                o[k][4 * i + c] = 0.f;
            }
        m[k] = -__builtin_huge_valf();
        l[k] = 0.f;
    }
    for (int f0 = k0; f0 < kend; f0 += PA_KF) {
        __syncthreads();   // the previous fill is no longer read
#pragma unroll
        for (int i = 0; i < NL; i++) {
            const int f = tid + PA_THREADS * i, row = f / (D / 4), c4 = f % (D / 4);
            if (NF % PA_THREADS == 0 || f < NF) {
                *reinterpret_cast<f32x4 *>(&Ks[row][4 * c4]) = kn[i];
                *reinterpret_cast<f32x4 *>(&Vs[row][4 * c4]) = vn[i];
            }
        }
        __syncthreads();
        fetch(f0 + PA_KF < kend ? f0 + PA_KF : f0);   // the next fill (the last one again at the end)
#pragma unroll
        for (int sub = 0; sub < PA_KF / PA_KC; sub++) {
        const int c0 = f0 + sub * PA_KC;
        if (c0 >= kend) break;   // uniform
        float s[PA_R][PA_KC];
#pragma unroll
        for (int k = 0; k < PA_R; k++)
#pragma unroll
            for (int j = 0; j < PA_KC; j++) s[k][j] = 0.f;
#pragma unroll
        for (int i = 0; i < NI; i++) {
#pragma unroll
            for (int j = 0; j < PA_KC; j++) {
                const float4 k4 = *reinterpret_cast<const float4 *>(&Ks[sub * PA_KC + j][4 * qq + 4 * PA_TPR * i]);
#pragma unroll
                for (int k = 0; k < PA_R; k++) {
                    s[k][j] = fmaf(q[k][4 * i], k4.x, s[k][j]);
                    s[k][j] = fmaf(q[k][4 * i + 1], k4.y, s[k][j]);
                    s[k][j] = fmaf(q[k][4 * i + 2], k4.z, s[k][j]);
                    s[k][j] = fmaf(q[k][4 * i + 3], k4.w, s[k][j]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < PA_R; k++) {
            float cm = -__builtin_huge_valf();
#pragma unroll
            for (int j = 0; j < PA_KC; j++) {
                const float a = group_sum<PA_TPR>(s[k][j]);
                s[k][j] = c0 + j <= qpos[k] ? a : -__builtin_huge_valf();
                cm = fmaxf(cm, s[k][j]);
            }
            // a row that has seen no position yet keeps m = -inf, l = 0, o = 0
            const float mn = fmaxf(m[k], cm);
            const float corr = m[k] == -__builtin_huge_valf() ? 0.f : __expf(m[k] - mn);
            l[k] *= corr;
#pragma unroll
            for (int i = 0; i < DQ; i++) o[k][i] *= corr;
#pragma unroll
            for (int j = 0; j < PA_KC; j++) {
                s[k][j] = s[k][j] == -__builtin_huge_valf() ? 0.f : __expf(s[k][j] - mn);   // 0 where masked
                l[k] += s[k][j];
            }
            m[k] = mn;
        }
#pragma unroll
        for (int j = 0; j < PA_KC; j++) {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const float4 v4 = *reinterpret_cast<const float4 *>(&Vs[sub * PA_KC + j][4 * qq + 4 * PA_TPR * i]);
#pragma unroll
                for (int k = 0; k < PA_R; k++) {
                    o[k][4 * i] = fmaf(s[k][j], v4.x, o[k][4 * i]);
                    o[k][4 * i + 1] = fmaf(s[k][j], v4.y, o[k][4 * i + 1]);
                    o[k][4 * i + 2] = fmaf(s[k][j], v4.z, o[k][4 * i + 2]);
                    o[k][4 * i + 3] = fmaf(s[k][j], v4.w, o[k][4 * i + 3]);
                }
            }
        }
        }
    }
#pragma unroll
    for (int k = 0; k < PA_R; k++) {
        const int rr = rg * PA_R + k, g = rr % G, t = blockIdx.y * QB + rr / G;
        if (t >= T) continue;
        const long long row = (long long)t * NQ + kvh * G + g;
        if (nsplit == 1) {
            const float inv = 1.0f / l[k];
            float *dst = out + row * D + 4 * qq;
#pragma unroll
            for (int i = 0; i < NI; i++)
                *reinterpret_cast<float4 *>(dst + 4 * PA_TPR * i) =
                    make_float4(o[k][4 * i] * inv, o[k][4 * i + 1] * inv, o[k][4 * i + 2] * inv, o[k][4 * i + 3] * inv);
        } else {
            float *dst = part + (row * nsplit + blockIdx.z) * (D + 2);
#pragma unroll
            for (int i = 0; i < NI; i++)
                *reinterpret_cast<float4 *>(dst + 4 * qq + 4 * PA_TPR * i) =
                    make_float4(o[k][4 * i], o[k][4 * i + 1], o[k][4 * i + 2], o[k][4 * i + 3]);
            if (qq == 0) {
                dst[D] = m[k];
                dst[D + 1] = l[k];
            }
        }
    }
}

// out[row] = sum_z e^(m_z - M) o_z / sum_z e^(m_z - M) l_z over the splits
// z <= qpos / ks that row (t, h) reaches.  grid = T * NQ, D threads.
template <int D>
__global__ __launch_bounds__(D) void k_pf_attn_combine(const float *__restrict__ part, int NQ, int pos0, int ks,
                                                       int nsplit, float *__restrict__ out) {
    const long long row = blockIdx.x;
    const int t = (int)(row / NQ), d = threadIdx.x;
    const int nz = (pos0 + t) / ks + 1;
    const float *p = part + row * nsplit * (D + 2);
    float M = -__builtin_huge_valf();
    for (int z = 0; z < nz; z++) M = fmaxf(M, p[z * (D + 2) + D]);
    float num = 0.f, den = 0.f;
    for (int z = 0; z < nz; z++) {
        const float f = __expf(p[z * (D + 2) + D] - M);
        num = fmaf(f, p[z * (D + 2) + d], num);
        den = fmaf(f, p[z * (D + 2) + D + 1], den);
    }
    out[row * D + d] = num / den;
}

// Split size: PA_PREF_KS positions, larger for long contexts so that at
// most PA_MAX_SPLIT splits exist (a multiple of PA_KF either way).
constexpr int PA_PREF_KS = 128, PA_MAX_SPLIT = 8;
static int pf_split_size(int kmax) {
    int ks = PA_PREF_KS;
    if ((kmax + ks - 1) / ks > PA_MAX_SPLIT) ks = ((kmax + PA_MAX_SPLIT - 1) / PA_MAX_SPLIT + PA_KF - 1) / PA_KF * PA_KF;
    return ks;
}

template <int D>
static hipError_t launch_pf_attn(int G, const float *qb, const float *kc, const float *vc, int T, int pos0, int NQ,
                                 int NKV, int max_ctx, float *part, float *out, hipStream_t st) {
    const int ks = pf_split_size(pos0 + T), nsplit = (pos0 + T + ks - 1) / ks;
#define TBQ_PFA(GG)                                                                                                \
    case GG:                                                                                                       \
        hipLaunchKernelGGL((k_pf_attn<D, GG>), dim3(NKV, (T + PA_ROWS / GG - 1) / (PA_ROWS / GG), nsplit),         \
                           dim3(PA_THREADS), 0, st, qb, kc, vc, T, pos0, NQ, max_ctx, ks, nsplit, part, out);      \
        break;
    switch (G) {
        TBQ_PFA(1) TBQ_PFA(2) TBQ_PFA(4) TBQ_PFA(8)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_PFA
    if (nsplit > 1)
        hipLaunchKernelGGL(k_pf_attn_combine<D>, dim3(T * NQ), dim3(D), 0, st, part, NQ, pos0, ks, nsplit, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static size_t pf_up(size_t n) { return (n + 255) & ~(size_t)255; }

// Every model with hidden <= 8192 (the norm kernel's row) takes the batched
// path for T >= 2; its matrices, of any format and layout, are dequantised
// to fp16 one at a time and multiplied by rocBLAS.
bool dense_prefill_batched(const tbq_dense_model *m) { return m->hidden <= PN_THREADS * PN_V * 4; }

struct PfWs {
    float *x, *y, *qkv, *qb, *att, *gu, *sa, *sb, *part;
    _Float16 *h16, *wh;
    int *tok;
    void *dec;
};

static PfWs pf_ws(const tbq_dense_model *m, int T, void *ws, size_t *total) {
    const size_t H = m->hidden, QD = (size_t)m->n_heads * m->head_dim, F = m->ffn;
    const size_t QKVR = (size_t)(m->n_heads + 2 * m->n_kv_heads) * m->head_dim;
    const size_t wide = std::max(std::max(H, QD), F);
    const size_t wmax = std::max(std::max(QKVR * H, H * QD), std::max(2 * F * H, H * F));
    char *p = (char *)ws;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        void *r = p + off;
        off += pf_up(bytes);
        return r;
    };
    PfWs w{};
    w.dec = take(dense_workspace_bytes(m));
    w.tok = (int *)take((size_t)T * 4);
    if (dense_prefill_batched(m) && T >= 2) {
        w.x = (float *)take((size_t)T * H * 4);
        w.y = (float *)take((size_t)T * H * 4);
        w.qkv = (float *)take((size_t)T * QKVR * 4);
        w.qb = (float *)take((size_t)T * QD * 4);
        w.att = (float *)take((size_t)T * QD * 4);
        w.gu = (float *)take((size_t)T * 2 * F * 4);
        w.h16 = (_Float16 *)take((size_t)T * wide * 2);
        w.sa = (float *)take((size_t)T * 4);
        w.sb = (float *)take((size_t)T * 4);
        w.wh = (_Float16 *)take(wmax * 2);
        // attention split partials: a prefill reaching position kmax - 1 uses
        // min(PA_MAX_SPLIT, ceil(kmax / PA_PREF_KS)) splits, and kmax <= max_ctx
        const int ns = std::min(PA_MAX_SPLIT, (m->max_ctx + PA_PREF_KS - 1) / PA_PREF_KS);
        w.part = ns > 1 ? (float *)take((size_t)T * m->n_heads * ns * (m->head_dim + 2) * 4) : nullptr;
    }
    if (total) *total = off;
    return w;
}

size_t dense_prefill_workspace_bytes(const tbq_dense_model *m, int T) {
    size_t t = 0;
    pf_ws(m, T, nullptr, &t);
    return t;
}

// rocBLAS for the prefill's fp16 GEMMs: one handle per process, used under
// a mutex (its stream is set per call).
static std::mutex g_rb_mu;
static rocblas_handle g_rb = nullptr;

// C[T][M] = X[T][K] . W[M][K]^T, row-major, fp16 operands, fp32 accumulate
// and output (column-major: C'[M x T] = W'^T[M x K] X'[K x T]).
static hipError_t pf_gemm(const _Float16 *W, const _Float16 *X, int T, int M, int K, float *C) {
    const float alpha = 1.f, beta = 0.f;
    const rocblas_status r =
        rocblas_gemm_ex(g_rb, rocblas_operation_transpose, rocblas_operation_none, M, T, K, &alpha, W,
                        rocblas_datatype_f16_r, K, X, rocblas_datatype_f16_r, K, &beta, C, rocblas_datatype_f32_r, M, C,
                        rocblas_datatype_f32_r, M, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    return r == rocblas_status_success ? hipSuccess : hipErrorUnknown;
}

// tokens: T device ints (in range); T >= 2.
static hipError_t pf_batched(const tbq_dense_model *m, const PfWs &w, int T, int pos0, float *logits,
                             hipStream_t st) {
    const int H = m->hidden, D = m->head_dim, NQ = m->n_heads, NKV = m->n_kv_heads, G = NQ / NKV, F = m->ffn;
    const int QD = NQ * D, KD = NKV * D, QKVR = QD + 2 * KD;
    auto qt_of = [m](int q) { return canon_qt(q ? q : m->qtype_layers); };
    auto dq = [&](int qt, const void *W, long long rows, int K, _Float16 *dst) {
        return launch_dequant_f16(qt, W, rows * K, dst, st);
    };
    std::lock_guard<std::mutex> lk(g_rb_mu);
    if (!g_rb && rocblas_create_handle(&g_rb) != rocblas_status_success) return hipErrorUnknown;
    if (rocblas_set_stream(g_rb, st) != rocblas_status_success) return hipErrorUnknown;
    hipError_t err = launch_dequant_rows(canon_qt(m->qtype_embd), m->tok_embd, w.tok, T, H, w.x, st);
    for (int l = 0; l < m->n_layers && err == hipSuccess; l++) {
        const tbq_dense_layer &L = m->layers[l];
        const size_t kvoff = (size_t)l * NKV * m->max_ctx * D;
        float *kc = m->k_cache + kvoff, *vc = m->v_cache + kvoff;
        hipLaunchKernelGGL(k_pf_norm, dim3(T), dim3(PN_THREADS), 0, st, w.x, l ? w.y : nullptr, l ? w.sb : nullptr,
                           L.attn_norm, H, m->norm_eps, w.h16, w.sa);
        if (L.wqkv) {
            err = dq(qt_of(L.qt_qkv), L.wqkv, QKVR, H, w.wh);
        } else {
            err = dq(qt_of(L.qt_q), L.wq, QD, H, w.wh);
            if (err == hipSuccess) err = dq(qt_of(L.qt_k), L.wk, KD, H, w.wh + (size_t)QD * H);
            if (err == hipSuccess) err = dq(qt_of(L.qt_v), L.wv, KD, H, w.wh + (size_t)(QD + KD) * H);
        }
        if (err != hipSuccess || (err = pf_gemm(w.wh, w.h16, T, QKVR, H, w.qkv)) != hipSuccess) break;
        if (D == 128) {
            hipLaunchKernelGGL(k_pf_qk<128>, dim3(T, NQ + NKV), dim3(64), 0, st, w.qkv, w.sa, L.q_norm, L.k_norm, NQ,
                               NKV, pos0, m->rope_theta, m->norm_eps, kc, vc, m->max_ctx, w.qb);
            err = launch_pf_attn<128>(G, w.qb, kc, vc, T, pos0, NQ, NKV, m->max_ctx, w.part, w.att, st);
        } else {
            hipLaunchKernelGGL(k_pf_qk<64>, dim3(T, NQ + NKV), dim3(64), 0, st, w.qkv, w.sa, L.q_norm, L.k_norm, NQ,
                               NKV, pos0, m->rope_theta, m->norm_eps, kc, vc, m->max_ctx, w.qb);
            err = launch_pf_attn<64>(G, w.qb, kc, vc, T, pos0, NQ, NKV, m->max_ctx, w.part, w.att, st);
        }
        if (err != hipSuccess || (err = launch_rows_f16(w.att, T, QD, w.h16, w.sb, st)) != hipSuccess) break;
        if ((err = dq(qt_of(L.qt_o), L.wo, H, QD, w.wh)) != hipSuccess) break;
        if ((err = pf_gemm(w.wh, w.h16, T, H, QD, w.y)) != hipSuccess) break;
        hipLaunchKernelGGL(k_pf_norm, dim3(T), dim3(PN_THREADS), 0, st, w.x, w.y, w.sb, L.ffn_norm, H, m->norm_eps,
                           w.h16, w.sa);
        if (L.wgu) {
            err = dq(qt_of(L.qt_gu), L.wgu, 2 * F, H, w.wh);
        } else {
            err = dq(qt_of(L.qt_gate), L.wgate, F, H, w.wh);
            if (err == hipSuccess) err = dq(qt_of(L.qt_up), L.wup, F, H, w.wh + (size_t)F * H);
        }
        if (err != hipSuccess || (err = pf_gemm(w.wh, w.h16, T, 2 * F, H, w.gu)) != hipSuccess) break;
        hipLaunchKernelGGL(k_pf_swiglu_f16, dim3(T), dim3(PN_THREADS), 0, st, w.gu, w.sa, F, w.h16, w.sb);
        if ((err = dq(qt_of(L.qt_down), L.wdown, H, F, w.wh)) != hipSuccess) break;
        err = pf_gemm(w.wh, w.h16, T, H, F, w.y);
    }
    if (err != hipSuccess) return err;
    float *ylast = w.y + (size_t)(T - 1) * H;
    hipLaunchKernelGGL(k_pf_scale_row, dim3(1), dim3(256), 0, st, ylast, w.sb + (T - 1), H);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    return dense_final_logits(m, w.x + (size_t)(T - 1) * H, ylast, logits, w.dec, st);
}

hipError_t launch_dense_prefill(const tbq_dense_model *m, const int *tokens_host, int T, int pos0, float *logits,
                                void *ws, hipStream_t st) {
    const PfWs w = pf_ws(m, T, ws, nullptr);
    if (!dense_prefill_batched(m) || T < 2) {
        // one token, or a row wider than the norm kernel: the decode step per token
        for (int t = 0; t < T; t++) {
            const hipError_t err = launch_dense_decode(m, tokens_host[t], pos0 + t, logits, w.dec, st);
            if (err != hipSuccess) return err;
        }
        return hipSuccess;
    }
    const hipError_t err = hipMemcpyAsync(w.tok, tokens_host, (size_t)T * 4, hipMemcpyHostToDevice, st);
    if (err != hipSuccess) return err;
    return pf_batched(m, w, T, pos0, logits, st);
}

}  // namespace tbq
