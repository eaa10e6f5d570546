// tbq_dense_prefill.hip -- batched prefill of a dense Qwen3-style model on
// gfx950: the T prompt tokens at positions pos0 .. pos0 + T - 1 go through
// each layer together, where the reference prefills token by token
// (layer4/tb_infer.c:1068-1075: one tb_infer_decode step per prompt token).
//
// Per layer (x: fp32 residual rows [T][H]; h16: fp16 rows with per-row
// power-of-two scales, the GEMMs' activation operand; the GEMMs are
// k_hgemm (tbq_gemm.hip): Q4_K weights are dequantised inside it, any other
// format to fp16 first (k_dequant_f16, one reused buffer)):
//   k_pf_norm        x += y (the previous sublayer's output, unscaled by
//                    its row scales), h16 = rmsnorm(x) * attn_norm
//   GEMM             qkv = h16 Wqkv^T             fp16 MFMA, fp32 acc
//   k_pf_qk          per (token, head): QK-norm + RoPE of q (to qb) and k;
//                    k and v rows written to the cache at pos0 + t
//   k_pf_attn        causal GQA attention over cache positions 0 .. pos on
//                    fp16 MFMA, online softmax, key ranges split over
//                    workgroups
//   k_pf_attn_rows   merges the splits of each token's row and writes it
//                    as fp16 rows with row scales (the o GEMM's operand)
//   GEMM             y = att Wo^T
//   k_pf_norm        x += y, h16 = rmsnorm(x) * ffn_norm
//   GEMM             a = silu(h16 Wg^T) * (h16 Wu^T) (SwiGLU in the GEMM's
//                    epilogue for a fused gate|up matrix; else the two
//                    products and k_pf_swiglu_f16), then a16 = fp16 rows
//                    with row scales
//   GEMM             y = a16 Wdown^T
// then the last token's logits = Wlm rmsnorm(x + y) (the decode step's
// lm_head matvec with its norm prologue).
//
// Accuracy: fp16 weights, activations, attention scores' operands and
// probabilities (11-bit mantissa) with fp32 accumulation, fp32 norms, RoPE
// and softmax; the logits land within
// 1e-2 relative L2 of the float64 sequential decode.

#include <algorithm>

#include "tbq_kernels.h"
#include "tbq_device.hpp"
#include "../../include/tbq.h"

namespace tbq {

constexpr int PN_THREADS = 256;
constexpr int PA_KF = 32;     // split sizes are multiples of this many positions

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
// y may be a GEMM's ny split-K slices (slice z at y + z * ystride), added
// here in slice order.  A thread holds up to PN_V float4 of the row (H <=
// 8192), all loaded before any is used.
constexpr int PN_V = 8, PN_MAXY = 8;   // float4 per thread (H <= 8192), slices of y
template <int PV>   // float4 of the row per thread: ceil(H / 4 / PN_THREADS) <= PV
__global__ __launch_bounds__(PN_THREADS) void k_pf_norm(float *__restrict__ x, const float *__restrict__ y, int ny,
                                                        long long ystride, const float *__restrict__ ys,
                                                        const float *__restrict__ w, int H, float eps,
                                                        _Float16 *__restrict__ h16, float *__restrict__ hinv) {
    __shared__ float red[PN_THREADS / 64];
    const int t = blockIdx.x, tid = threadIdx.x, n4 = H / 4;
    float4 *xr = reinterpret_cast<float4 *>(x + (long long)t * H);
    const float4 *yr = reinterpret_cast<const float4 *>(y ? y + (long long)t * H : x + (long long)t * H);
    const float4 *wr = reinterpret_cast<const float4 *>(w);
    float4 v[PV], b[PV], g[PV];
#pragma unroll
    for (int i = 0; i < PV; i++) {
        const int j = min(tid + PN_THREADS * i, n4 - 1);   // clamped: loads stay unconditional
        v[i] = xr[j];
        b[i] = yr[j];
        g[i] = wr[j];
    }
    if (y && ny > 1) {
        // every slice's loads issued at once (slices past ny re-read the
        // last and are not added), then added in slice order
        float4 c[PN_MAXY - 1][PV];
#pragma unroll
        for (int z = 1; z < PN_MAXY; z++) {
            const float4 *yz = yr + min(z, ny - 1) * (ystride / 4);
#pragma unroll
            for (int i = 0; i < PV; i++) c[z - 1][i] = yz[min(tid + PN_THREADS * i, n4 - 1)];
        }
#pragma unroll
        for (int z = 1; z < PN_MAXY; z++) {
            if (z < ny) {
#pragma unroll
                for (int i = 0; i < PV; i++) {
                    b[i].x = b[i].x + c[z - 1][i].x; b[i].y = b[i].y + c[z - 1][i].y;
                    b[i].z = b[i].z + c[z - 1][i].z; b[i].w = b[i].w + c[z - 1][i].w;
                }
            }
        }
    }
    float ss = 0.f;
    const float yscale = ys ? ys[t] : 1.f;
#pragma unroll
    for (int i = 0; i < PV; i++) {
        if (y) {
            v[i].x += b[i].x * yscale; v[i].y += b[i].y * yscale;
            v[i].z += b[i].z * yscale; v[i].w += b[i].w * yscale;
        }
        if (tid + PN_THREADS * i < n4) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    }
    if (y) {
#pragma unroll
        for (int i = 0; i < PV; i++)
            if (tid + PN_THREADS * i < n4) xr[tid + PN_THREADS * i] = v[i];
    }
    ss = pf_block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)H + eps);
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < PV; i++) {
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
    for (int i = 0; i < PV; i++) {
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

static hipError_t launch_pf_norm(int T, float *x, const float *y, int ny, long long ystride, const float *ys,
                                 const float *w, int H, float eps, _Float16 *h16, float *hinv, hipStream_t st) {
    if (ny > PN_MAXY) return hipErrorNotSupported;
    const int pv = (H / 4 + PN_THREADS - 1) / PN_THREADS;
#define TBQ_PN(V)                                                                                                  \
    case V:                                                                                                        \
        hipLaunchKernelGGL(k_pf_norm<V>, dim3(T), dim3(PN_THREADS), 0, st, x, y, ny, ystride, ys, w, H, eps, h16,  \
                           hinv);                                                                                  \
        break;
    switch (pv) {
        TBQ_PN(1) TBQ_PN(2) TBQ_PN(3) TBQ_PN(4) TBQ_PN(5) TBQ_PN(6) TBQ_PN(7) TBQ_PN(8)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_PN
    return hipGetLastError();
}

// RoPE tables of the prompt's positions, shared by every layer: rc[t][j] =
// cos, rc[t][D/2 + j] = sin of (pos0 + t) * theta^(-2j/D), formed and
// reduced in fp64 exactly as the decode step's k_rope_table.  grid = T.
__global__ __launch_bounds__(64) void k_pf_rope(int pos0, float theta, int D, float *__restrict__ rc) {
    const int t = blockIdx.x, j = threadIdx.x;
    if (j < D / 2) {
        double sd, cd;
        sincos((double)(pos0 + t) * pow((double)theta, -2.0 * j / D), &sd, &cd);
        rc[(long long)t * D + j] = (float)cd;
        rc[(long long)t * D + D / 2 + j] = (float)sd;
    }
}

// Head vector (one wave; lane l holds elements l and l + 64, or l for
// D = 64): RMSNorm with the head's weights, then rotate-half RoPE with the
// position's table row rc (cos | sin).
template <int D>
__device__ __forceinline__ void pf_norm_rope(float (&x)[D / 64], const float *__restrict__ w,
                                             const float *__restrict__ rc, float eps) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < D / 64; i++) ss += x[i] * x[i];
    ss = group_sum<64>(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int i = 0; i < D / 64; i++) x[i] = x[i] * r * w[lane + 64 * i];
    const int j = lane % (D / 2);
    const float cs = rc[j], sn = rc[D / 2 + j];
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
__global__ __launch_bounds__(64) void k_pf_qk(const float *__restrict__ qkv, int nq, long long qstride,
                                              const float *__restrict__ rs, const float *__restrict__ qn,
                                              const float *__restrict__ kn, int NQ, int NKV, int pos0,
                                              const float *__restrict__ rope, float eps, float *__restrict__ kc,
                                              float *__restrict__ vc, int max_ctx, float *__restrict__ qb) {
    const int t = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
    const int QKVR = (NQ + 2 * NKV) * D, pos = pos0 + t;
    const float sc = rs[t];   // row t of qkv is scaled by 1 / rs[t]
    // qkv may be a GEMM's nq split-K slices (slice z at qkv + z * qstride),
    // added in slice order
    auto elem = [&](long long off) {
        float a = qkv[off];
        for (int z = 1; z < nq; z++) a = a + qkv[off + z * qstride];
        return a;
    };
    const long long src = (long long)t * QKVR + hh * D;
    float x[D / 64];
#pragma unroll
    for (int i = 0; i < D / 64; i++) x[i] = elem(src + lane + 64 * i) * sc;
    pf_norm_rope<D>(x, hh < NQ ? qn : kn, rope + (long long)t * D, eps);
    if (hh < NQ) {
        const float scale = 1.0f / sqrtf((float)D);
#pragma unroll
        for (int i = 0; i < D / 64; i++) qb[((long long)t * NQ + hh) * D + lane + 64 * i] = x[i] * scale;
    } else {
        const int kvh = hh - NQ;
        const long long row = ((long long)kvh * max_ctx + pos) * D;
        const long long vsrc = (long long)t * QKVR + (NQ + NKV + kvh) * D;
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            kc[row + lane + 64 * i] = x[i];
            vc[row + lane + 64 * i] = elem(vsrc + lane + 64 * i) * sc;
        }
    }
}

// Row t: a = silu(g * s) * (u * s) with gu[t] = [g (F) | u (F)] and s =
// gs[t], then a16[t] = a * 2^e in fp16 (max |a| in [2^14, 2^15)) and
// ainv[t] = 2^-e.  grid = T, 1024 threads, the row read once (up to PS_V
// float4 of g and of u per thread: F <= 16384).
constexpr int PS_THREADS = 1024, PS_V = 4;
__global__ __launch_bounds__(PS_THREADS) void k_pf_swiglu_f16(const float *__restrict__ gu, const float *__restrict__ gs,
                                                              int F, _Float16 *__restrict__ a16,
                                                              float *__restrict__ ainv) {
    __shared__ float red[PS_THREADS / 64];
    const int t = blockIdx.x, tid = threadIdx.x, n4 = F / 4;
    const float4 *g = reinterpret_cast<const float4 *>(gu + (long long)t * 2 * F), *u = g + n4;
    const float s = gs[t];
    float4 a[PS_V];
#pragma unroll
    for (int i = 0; i < PS_V; i++) {
        const int j = min(tid + PS_THREADS * i, n4 - 1);   // clamped: loads stay unconditional
        const float4 gv = g[j], uv = u[j];
        a[i] = make_float4(pro_swiglu(gv.x * s, uv.x * s), pro_swiglu(gv.y * s, uv.y * s),
                           pro_swiglu(gv.z * s, uv.z * s), pro_swiglu(gv.w * s, uv.w * s));
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < PS_V; i++)
        if (tid + PS_THREADS * i < n4)
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a[i].x), fabsf(a[i].y)), fmaxf(fabsf(a[i].z), fabsf(a[i].w))));
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = 0.f;
#pragma unroll
    for (int i = 0; i < PS_THREADS / 64; i++) mx = fmaxf(mx, red[i]);
    int e = 0;
    frexpf(mx, &e);
    int sh = mx > 0.f ? 15 - e : 0;
    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
    const float sc = ldexpf(1.f, sh);
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 *ar = reinterpret_cast<h4 *>(a16 + (long long)t * F);
#pragma unroll
    for (int i = 0; i < PS_V; i++) {
        const int j = tid + PS_THREADS * i;
        if (j < n4)
            ar[j] = h4{(_Float16)(a[i].x * sc), (_Float16)(a[i].y * sc), (_Float16)(a[i].z * sc),
                       (_Float16)(a[i].w * sc)};
    }
    if (tid == 0) ainv[t] = ldexpf(1.f, -sh);
}

// out[j] = (sum over the ny slices, in slice order, of y[z * ystride + j])
// * ys[0] for one row of n floats (the last token's down output before the
// lm_head).
__global__ __launch_bounds__(256) void k_pf_scale_row(const float *__restrict__ y, int ny, long long ystride,
                                                      const float *__restrict__ ys, int n, float *__restrict__ out) {
    for (int j = threadIdx.x; j < n; j += 256) {
        float a = y[j];
        for (int z = 1; z < ny; z++) a = a + y[z * ystride + j];
        out[j] = a * ys[0];
    }
}

// Causal attention on MFMA (v_mfma_f32_32x32x16_f16, fp16 operands, fp32
// accumulate).  grid = (NKV, ceil(T / QB), nsplit), 4 waves: the workgroup
// owns QB = 128 / G tokens x the G query heads of kv head kvh = 128 query
// columns, 32 per wave (query c of a wave: token c / G, head c % G).  Cache
// positions pass through LDS 32 at a time in fp16: K as [position][dim],
// V transposed as [dim][position].  Per chunk a wave forms S^T = K Q^T (32
// positions x its 32 queries), so a lane holds 16 scores of one query:
// lane l, register r: query l % 32, position 8(r/4) + 4(l/32) + r%4.  The
// query's max and denominator need one exchange with lane l ^ 32.  The
// probabilities, rounded to fp16, are already the B operand of
// O^T += V^T P^T when the 16 positions of a step are taken in the order
// k-slot 8h + i <-> position 8(i/4) + 4h + i%4 (h = l / 32), which V^T's A
// operand follows; O^T's accumulators hold dims 32j + 8(r/4) + 4h + r%4
// of the lane's query.  Online softmax over chunks; positions past a
// query's own are masked.
//
// Key splits: split z takes positions [z ks, (z + 1) ks) (ks a multiple of
// PA_KF), so the heavy blocks of a causal prompt (whose queries see every
// earlier position) spread over several workgroups.  With nsplit > 1 each
// writes its queries' unnormalised output, running max and denominator to
// the record part[(row * nsplit + z) * pf_rec(D)] (D outputs, max,
// denominator, two floats of padding so that every record starts 16-byte
// aligned for the float4 stores), and k_pf_attn_rows merges the splits a
// row reaches.
constexpr int PM_THREADS = 256, PM_Q = 128, PM_KC = 32;
__host__ __device__ constexpr int pf_rec(int D) { return D + 4; }
typedef _Float16 pm_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 pm_h4 __attribute__((ext_vector_type(4)));
typedef float pm_f16 __attribute__((ext_vector_type(16)));

template <int D, int G>
__global__ __launch_bounds__(PM_THREADS) void k_pf_attn(const float *__restrict__ qb, const float *__restrict__ kc,
                                                        const float *__restrict__ vc, int T, int pos0, int NQ,
                                                        int max_ctx, int ks, int nsplit, float *__restrict__ part,
                                                        float *__restrict__ out) {
    constexpr int QB = PM_Q / G, KLD = D + 8, VLD = PM_KC + 8, NT = D / 32, NS = D / 16;
    __shared__ __attribute__((aligned(16))) _Float16 Ks[PM_KC * KLD];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D * VLD];
    const int kvh = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, h = lane >> 5;
    const int qc = wave * 32 + li, g = qc % G;
    const int t = blockIdx.y * QB + qc / G;
    const int tt = t < T ? t : T - 1;
    const int qpos = pos0 + tt;
    const int tend = min(T, (int)(blockIdx.y + 1) * QB);
    const int k0 = blockIdx.z * ks;                  // this split's positions k0 .. kend - 1
    const int kend = min(pos0 + tend, k0 + ks);
    if (k0 >= kend) return;   // no position of the split is seen by the block (uniform)
    // Q^T's B fragments: dim step s, lane half h supplies dims 16s + 8h .. + 8
    pm_h8 qf[NS];
    const float *qsrc = qb + ((long long)tt * NQ + kvh * G + g) * D;
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int c = 0; c < 8; c++) qf[s][c] = (_Float16)qsrc[16 * s + 8 * h + c];
    pm_f16 o[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) o[j] = pm_f16{};
    float m = -__builtin_huge_valf(), l = 0.f;
    const float *kb = kc + (long long)kvh * max_ctx * D;
    const float *vb = vc + (long long)kvh * max_ctx * D;
    for (int c0 = k0; c0 < kend; c0 += PM_KC) {
        __syncthreads();   // the previous chunk is no longer read
        for (int f = tid; f < PM_KC * D / 4; f += PM_THREADS) {
            const int key = f / (D / 4), c4 = f % (D / 4);
            const long long p = min(c0 + key, kend - 1);
            const float4 kv = *reinterpret_cast<const float4 *>(kb + p * D + 4 * c4);
            const float4 vv = *reinterpret_cast<const float4 *>(vb + p * D + 4 * c4);
            *reinterpret_cast<pm_h4 *>(&Ks[key * KLD + 4 * c4]) =
                pm_h4{(_Float16)kv.x, (_Float16)kv.y, (_Float16)kv.z, (_Float16)kv.w};
            Vt[(4 * c4) * VLD + key] = (_Float16)vv.x;
            Vt[(4 * c4 + 1) * VLD + key] = (_Float16)vv.y;
            Vt[(4 * c4 + 2) * VLD + key] = (_Float16)vv.z;
            Vt[(4 * c4 + 3) * VLD + key] = (_Float16)vv.w;
        }
        __syncthreads();
        pm_f16 sc = pm_f16{};
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const pm_h8 a = *reinterpret_cast<const pm_h8 *>(&Ks[li * KLD + 16 * s + 8 * h]);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[s], sc, 0, 0, 0);
        }
        float mx = -__builtin_huge_valf();
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = c0 + 8 * (r / 4) + 4 * h + r % 4;
            const float v = key <= qpos ? sc[r] : -__builtin_huge_valf();
            sc[r] = v;
            mx = fmaxf(mx, v);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // a query that has seen no position yet keeps m = -inf, l = 0, o = 0
        const float mn = fmaxf(m, mx);
        const float corr = m == -__builtin_huge_valf() ? 0.f : __expf(m - mn);
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float p = sc[r] == -__builtin_huge_valf() ? 0.f : __expf(sc[r] - mn);
            sc[r] = p;
            ls += p;
        }
        ls += __shfl_xor(ls, 32);
        l = l * corr + ls;
        m = mn;
        pm_h8 pb[2];
#pragma unroll
        for (int r = 0; r < 16; r++) pb[r / 8][r % 8] = (_Float16)sc[r];
#pragma unroll
        for (int j = 0; j < NT; j++) {
            o[j] *= corr;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const _Float16 *vr = &Vt[(32 * j + li) * VLD + 16 * k + 4 * h];
                const pm_h4 lo = *reinterpret_cast<const pm_h4 *>(vr);
                const pm_h4 hi = *reinterpret_cast<const pm_h4 *>(vr + 8);
                const pm_h8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[k], o[j], 0, 0, 0);
            }
        }
    }
    if (t >= T) return;
    const long long row = (long long)t * NQ + kvh * G + g;
    const float inv = nsplit == 1 ? 1.0f / l : 1.f;
    float *dst = nsplit == 1 ? out + row * D : part + (row * nsplit + blockIdx.z) * pf_rec(D);
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++)
            *reinterpret_cast<float4 *>(dst + 32 * j + 8 * r4 + 4 * h) =
                make_float4(o[j][4 * r4] * inv, o[j][4 * r4 + 1] * inv, o[j][4 * r4 + 2] * inv, o[j][4 * r4 + 3] * inv);
    if (nsplit > 1 && h == 0) {
        dst[D] = m;
        dst[D + 1] = l;
    }
}

// Attention rows to the o GEMM's operand in one pass: row t (all NQ heads,
// QD = NQ * D floats) is the attention output -- att[t] itself when the
// keys were not split, else the merge of the splits z <= (pos0 + t) / ks
// with e^(m_z - M) weights and fmaf sums in z order -- and is written as fp16 scaled by
// the power of two that puts its max |value| in [2^14, 2^15), with
// hinv[t] = the inverse scale (k_rows_f16's arithmetic).  grid = T,
// PN_THREADS threads, up to PR_V float4 of the row per thread (QD <= 8192).
constexpr int PR_V = 8;
constexpr int PA_PREF_KS = 128, PA_MAX_SPLIT = 8;   // preferred split size, most splits
template <int D>
__global__ __launch_bounds__(PN_THREADS) void k_pf_attn_rows(const float *__restrict__ part,
                                                             const float *__restrict__ att, int NQ, int pos0, int ks,
                                                             int nsplit, _Float16 *__restrict__ h16,
                                                             float *__restrict__ hinv) {
    __shared__ float red[PN_THREADS / 64];
    constexpr int RS = pf_rec(D);
    const int t = blockIdx.x, tid = threadIdx.x, n4 = NQ * D / 4;
    const int nz = (pos0 + t) / ks + 1;
    float4 v[PR_V];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < PR_V; i++) {
        const int j = tid + PN_THREADS * i;
        if (j >= n4) continue;
        const int hh = 4 * j / D, d = 4 * j % D;
        const long long row = (long long)t * NQ + hh;
        if (nsplit == 1) {
            v[i] = *reinterpret_cast<const float4 *>(att + row * D + d);
        } else {
            // every split's record loaded at once (splits past nz re-read the
            // last one and are skipped), then merged in z order
            const float *p = part + row * nsplit * RS;
            float ml[PA_MAX_SPLIT], ll[PA_MAX_SPLIT];
            float4 o[PA_MAX_SPLIT];
#pragma unroll
            for (int z = 0; z < PA_MAX_SPLIT; z++) {
                const float *r = p + min(z, nz - 1) * RS;
                ml[z] = r[D];
                ll[z] = r[D + 1];
                o[z] = *reinterpret_cast<const float4 *>(r + d);
            }
            float M = -__builtin_huge_valf();
#pragma unroll
            for (int z = 0; z < PA_MAX_SPLIT; z++)
                if (z < nz) M = fmaxf(M, ml[z]);
            float n0 = 0.f, n1 = 0.f, n2 = 0.f, n3 = 0.f, den = 0.f;
#pragma unroll
            for (int z = 0; z < PA_MAX_SPLIT; z++) {
                if (z < nz) {
                    const float f = __expf(ml[z] - M);
                    n0 = fmaf(f, o[z].x, n0);
                    n1 = fmaf(f, o[z].y, n1);
                    n2 = fmaf(f, o[z].z, n2);
                    n3 = fmaf(f, o[z].w, n3);
                    den = fmaf(f, ll[z], den);
                }
            }
            v[i] = make_float4(n0 / den, n1 / den, n2 / den, n3 / den);
        }
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    mx = pf_block_max(mx, red);
    int e = 0;
    frexpf(mx, &e);
    int sh = mx > 0.f ? 15 - e : 0;
    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
    const float sc = ldexpf(1.f, sh);
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 *hr = reinterpret_cast<h4 *>(h16 + (long long)t * NQ * D);
#pragma unroll
    for (int i = 0; i < PR_V; i++) {
        const int j = tid + PN_THREADS * i;
        if (j < n4)
            hr[j] = h4{(_Float16)(v[i].x * sc), (_Float16)(v[i].y * sc), (_Float16)(v[i].z * sc),
                       (_Float16)(v[i].w * sc)};
    }
    if (tid == 0) hinv[t] = ldexpf(1.f, -sh);
}

// Split size: PA_PREF_KS positions, larger for long contexts so that at
// most PA_MAX_SPLIT splits exist (a multiple of PA_KF either way).
static int pf_split_size(int kmax) {
    int ks = PA_PREF_KS;
    if ((kmax + ks - 1) / ks > PA_MAX_SPLIT) ks = ((kmax + PA_MAX_SPLIT - 1) / PA_MAX_SPLIT + PA_KF - 1) / PA_KF * PA_KF;
    return ks;
}

template <int D>
static hipError_t launch_pf_attn(int G, const float *qb, const float *kc, const float *vc, int T, int pos0, int NQ,
                                 int NKV, int max_ctx, float *part, float *out, _Float16 *h16, float *hinv,
                                 hipStream_t st) {
    const int ks = pf_split_size(pos0 + T), nsplit = (pos0 + T + ks - 1) / ks;
#define TBQ_PFA(GG)                                                                                                \
    case GG:                                                                                                       \
        hipLaunchKernelGGL((k_pf_attn<D, GG>), dim3(NKV, (T + PM_Q / GG - 1) / (PM_Q / GG), nsplit),               \
                           dim3(PM_THREADS), 0, st, qb, kc, vc, T, pos0, NQ, max_ctx, ks, nsplit, part, out);      \
        break;
    switch (G) {
        TBQ_PFA(1) TBQ_PFA(2) TBQ_PFA(4) TBQ_PFA(8)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_PFA
    hipLaunchKernelGGL(k_pf_attn_rows<D>, dim3(T), dim3(PN_THREADS), 0, st, part, out, NQ, pos0, ks, nsplit, h16,
                       hinv);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static size_t pf_up(size_t n) { return (n + 255) & ~(size_t)255; }

// Every model with hidden <= 8192, n_heads * head_dim <= 8192 and ffn <=
// 16384 (the rows the norm, attention-row and SwiGLU kernels hold) takes the batched path for T >= 2.  Q4_K matrices go
// straight into the GEMM (dequantised on the way into LDS); every other
// format and layout is dequantised to fp16 first (one matrix at a time) and
// multiplied by the same GEMM.
bool dense_prefill_batched(const tbq_dense_model *m) {
    return m->hidden <= PN_THREADS * PN_V * 4 && m->ffn <= PS_THREADS * PS_V * 4 &&
           m->n_heads * m->head_dim <= PN_THREADS * PR_V * 4;
}

struct PfWs {
    float *x, *y, *qkv, *qb, *att, *gu, *sa, *sb, *part, *rope, *gpart;
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
        // split-K partials of the largest product that splits
        const int cu = hgemm_cus(), Ti = T;
        const size_t gp = std::max(
            std::max(std::max(hgemm_partial_bytes(Ti, (int)QKVR, (int)H, cu), hgemm_partial_bytes(Ti, (int)QD, (int)H, cu)),
                     std::max(hgemm_partial_bytes(Ti, m->n_kv_heads * m->head_dim, (int)H, cu),
                              hgemm_partial_bytes(Ti, (int)H, (int)QD, cu))),
            std::max(std::max(hgemm_partial_bytes(Ti, (int)(2 * F), (int)H, cu), hgemm_partial_bytes(Ti, (int)F, (int)H, cu)),
                     hgemm_partial_bytes(Ti, (int)H, (int)F, cu)));
        w.gpart = gp ? (float *)take(gp) : nullptr;
        w.rope = (float *)take((size_t)T * m->head_dim * 4);
        // attention split partials: a prefill reaching position kmax - 1 uses
        // min(PA_MAX_SPLIT, ceil(kmax / PA_PREF_KS)) splits, and kmax <= max_ctx
        const int ns = std::min(PA_MAX_SPLIT, (m->max_ctx + PA_PREF_KS - 1) / PA_PREF_KS);
        w.part = ns > 1 ? (float *)take((size_t)T * m->n_heads * ns * pf_rec(m->head_dim) * 4) : nullptr;
    }
    if (total) *total = off;
    return w;
}

size_t dense_prefill_workspace_bytes(const tbq_dense_model *m, int T) {
    size_t t = 0;
    pf_ws(m, T, nullptr, &t);
    return t;
}

// tokens: T device ints (in range); T >= 2.
static hipError_t pf_batched(const tbq_dense_model *m, const PfWs &w, int T, int pos0, float *logits,
                             hipStream_t st) {
    const int H = m->hidden, D = m->head_dim, NQ = m->n_heads, NKV = m->n_kv_heads, G = NQ / NKV, F = m->ffn;
    const int QD = NQ * D, KD = NKV * D, QKVR = QD + 2 * KD;
    auto qt_of = [m](int q) { return canon_qt(q ? q : m->qtype_layers); };
    const int cu = hgemm_cus();
    // C[T][rows] (row stride ldc) = h16 . W^T: Q4_K rows directly, any other
    // format through its fp16 form in wh
    // (with ns set, the K slices' partial sums stay in w.gpart for the
    // consumer to add: k_pf_qk, k_pf_norm and k_pf_scale_row take them)
    auto gemm = [&](int qt, const void *W, int rows, int K, float *C, int ldc, int *ns = nullptr) {
        if (qt == QT_Q4_K) return launch_hgemm(QT_Q4_K, W, w.h16, T, rows, K, C, ldc, w.gpart, cu, st, ns);
        const hipError_t e = launch_dequant_f16(qt, W, (long long)rows * K, w.wh, st);
        if (e != hipSuccess) return e;
        return launch_hgemm(QT_F16, w.wh, w.h16, T, rows, K, C, ldc, w.gpart, cu, st, ns);
    };
    const float *ysrc = w.y;   // the previous sublayer's output, as yns slices
    int yns = 1;
    hipLaunchKernelGGL(k_pf_rope, dim3(T), dim3(64), 0, st, pos0, m->rope_theta, D, w.rope);
    hipError_t err = launch_dequant_rows(canon_qt(m->qtype_embd), m->tok_embd, w.tok, T, H, w.x, st);
    for (int l = 0; l < m->n_layers && err == hipSuccess; l++) {
        const tbq_dense_layer &L = m->layers[l];
        const size_t kvoff = (size_t)l * NKV * m->max_ctx * D;
        float *kc = m->k_cache + kvoff, *vc = m->v_cache + kvoff;
        err = launch_pf_norm(T, w.x, l ? ysrc : nullptr, yns, (long long)T * H, l ? w.sb : nullptr, L.attn_norm, H,
                             m->norm_eps, w.h16, w.sa, st);
        if (err != hipSuccess) break;
        int qns = 1;
        if (L.wqkv) {
            err = gemm(qt_of(L.qt_qkv), L.wqkv, QKVR, H, w.qkv, QKVR, &qns);
        } else {
            err = gemm(qt_of(L.qt_q), L.wq, QD, H, w.qkv, QKVR);
            if (err == hipSuccess) err = gemm(qt_of(L.qt_k), L.wk, KD, H, w.qkv + QD, QKVR);
            if (err == hipSuccess) err = gemm(qt_of(L.qt_v), L.wv, KD, H, w.qkv + QD + KD, QKVR);
        }
        if (err != hipSuccess) break;
        const float *qsrc = qns > 1 ? w.gpart : w.qkv;
        if (D == 128) {
            hipLaunchKernelGGL(k_pf_qk<128>, dim3(T, NQ + NKV), dim3(64), 0, st, qsrc, qns, (long long)T * QKVR, w.sa,
                               L.q_norm, L.k_norm, NQ, NKV, pos0, w.rope, m->norm_eps, kc, vc, m->max_ctx, w.qb);
            err = launch_pf_attn<128>(G, w.qb, kc, vc, T, pos0, NQ, NKV, m->max_ctx, w.part, w.att, w.h16, w.sb, st);
        } else {
            hipLaunchKernelGGL(k_pf_qk<64>, dim3(T, NQ + NKV), dim3(64), 0, st, qsrc, qns, (long long)T * QKVR, w.sa,
                               L.q_norm, L.k_norm, NQ, NKV, pos0, w.rope, m->norm_eps, kc, vc, m->max_ctx, w.qb);
            err = launch_pf_attn<64>(G, w.qb, kc, vc, T, pos0, NQ, NKV, m->max_ctx, w.part, w.att, w.h16, w.sb, st);
        }
        if (err != hipSuccess) break;
        if ((err = gemm(qt_of(L.qt_o), L.wo, H, QD, w.y, H, &yns)) != hipSuccess) break;
        ysrc = yns > 1 ? w.gpart : w.y;
        if ((err = launch_pf_norm(T, w.x, ysrc, yns, (long long)T * H, w.sb, L.ffn_norm, H, m->norm_eps, w.h16,
                                  w.sa, st)) != hipSuccess)
            break;
        // a fused gate|up matrix: SwiGLU in the GEMM's epilogue, then the
        // activation rows to fp16; otherwise the gate and up products and
        // k_pf_swiglu_f16
        bool glu = false;
        if (L.wgu) {
            const int qt = qt_of(L.qt_gu);
            const void *Wg = L.wgu;
            if (qt != QT_Q4_K && (err = launch_dequant_f16(qt, L.wgu, (long long)2 * F * H, w.wh, st)) != hipSuccess)
                break;
            if (qt != QT_Q4_K) Wg = w.wh;
            err = launch_hgemm_glu(qt == QT_Q4_K ? QT_Q4_K : QT_F16, Wg, w.h16, w.sa, T, F, H, w.gu, F, cu, st);
            if (err == hipSuccess) glu = true;
            else if (err == hipErrorNotSupported) err = gemm(qt, L.wgu, 2 * F, H, w.gu, 2 * F);
        } else {
            err = gemm(qt_of(L.qt_gate), L.wgate, F, H, w.gu, 2 * F);
            if (err == hipSuccess) err = gemm(qt_of(L.qt_up), L.wup, F, H, w.gu + F, 2 * F);
        }
        if (err != hipSuccess) break;
        if (glu)
            err = launch_rows_f16(w.gu, T, F, w.h16, w.sb, st);
        else
            hipLaunchKernelGGL(k_pf_swiglu_f16, dim3(T), dim3(PS_THREADS), 0, st, w.gu, w.sa, F, w.h16, w.sb);
        if (err != hipSuccess) break;
        err = gemm(qt_of(L.qt_down), L.wdown, H, F, w.y, H, &yns);
        ysrc = yns > 1 ? w.gpart : w.y;
    }
    if (err != hipSuccess) return err;
    float *ylast = w.y + (size_t)(T - 1) * H;
    hipLaunchKernelGGL(k_pf_scale_row, dim3(1), dim3(256), 0, st, ysrc + (size_t)(T - 1) * H, yns, (long long)T * H,
                       w.sb + (T - 1), H, ylast);
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
