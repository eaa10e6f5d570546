// tbq_moe_prefill.hip -- batched (prefill) MoE experts on gfx950 bf16 MFMA.
//
// After routing (exact, as in decode), the (token, slot) pairs are grouped by
// expert and every expert's products run as dense tiles:
//
//   k_dispatch        per-expert histogram, prefix sum and permutation of the
//                     pairs in LDS (one workgroup), plus a tile list of
//                     (expert, first pair, pairs in tile) entries of <= 64
//                     pairs; order inside an expert does not affect results.
//   k_gate_up_mfma    act[p] = swiglu(x_t . W_gate[e], x_t . W_up[e]) for a
//                     64-pair x 64-column tile: Q4_K rows are dequantised to
//                     bf16 into LDS 128 columns of K at a time, x rows are
//                     gathered and rounded to bf16, v_mfma_f32_16x16x32_bf16
//                     accumulates in fp32; act is stored as bf16.
//   k_down_mfma       y[p] = act[p] . W_down[e] for 64 pairs x 128 rows.
//   (k_combine)       out = resid + sum over slots in slot order (tbq_moe.hip).
//
// Accuracy: weights and activations rounded to bf16 (8-bit mantissa), fp32
// accumulation; outputs land within 1e-2 relative L2 of the fp32 reference.
#include "tbq_kernels.h"
#include "tbq_kquant.hpp"

namespace tbq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int PF_MT = 64;          // pairs per tile
constexpr int PF_KC = 128;         // K columns staged per step (half a Q4_K super-block)
constexpr int PF_LD = PF_KC + 8;   // LDS row stride in bf16 (padding breaks bank aliasing)
constexpr int PF_THREADS = 256;

struct PfTile {
    int e, start, n;
};

// ---------------------------------------------------------------------------
// Dispatch: one workgroup of 1024 threads.  pairs p = t*k + s.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_dispatch(const int *__restrict__ sel_idx, int T, int k, int E,
                                                   int *__restrict__ perm, PfTile *__restrict__ tiles,
                                                   int *__restrict__ ntiles) {
    __shared__ int hist[256], off[257], toff[257], cur[256];
    const int tid = threadIdx.x, P = T * k;
    for (int e = tid; e < 256; e += 1024) { hist[e] = 0; cur[e] = 0; }
    __syncthreads();
    for (int p = tid; p < P; p += 1024) atomicAdd(&hist[sel_idx[(p / k) * 8 + p % k]], 1);
    __syncthreads();
    if (tid == 0) {
        int o = 0, to = 0;
        for (int e = 0; e < E; e++) {
            off[e] = o;
            toff[e] = to;
            o += hist[e];
            to += (hist[e] + PF_MT - 1) / PF_MT;
        }
        off[E] = o;
        toff[E] = to;
        *ntiles = to;
    }
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = sel_idx[(p / k) * 8 + p % k];
        perm[off[e] + atomicAdd(&cur[e], 1)] = p;
    }
    for (int e = tid; e < E; e += 1024) {
        const int n = hist[e];
        for (int i = 0; i * PF_MT < n; i++) {
            PfTile tl;
            tl.e = e;
            tl.start = off[e] + i * PF_MT;
            tl.n = n - i * PF_MT < PF_MT ? n - i * PF_MT : PF_MT;
            tiles[toff[e] + i] = tl;
        }
    }
}

// ---------------------------------------------------------------------------
// Staging helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    // round to nearest even, as v_cvt_pk_bf16_f32 does
    const __bf16 ha = (__bf16)a, hb = (__bf16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// Raw bytes of one 32-weight Q4_K sub-block j of a super-block: scale/min
// inputs and the 16 quant bytes.
struct Q4Sub {
    uint4 hdr, q;
    uint32_t mind;
};

__device__ __forceinline__ void q4sub_load(const uint8_t *sb, int j, Q4Sub &r) {
    r.hdr = *reinterpret_cast<const uint4 *>(sb);
    r.q = *reinterpret_cast<const uint4 *>(sb + 16 + 16 * j);
    r.mind = *reinterpret_cast<const uint32_t *>(sb + 16);
}

// Dequantise (reference scale/min selection, layer4/tb_gguf.c:163-168) and
// write 32 bf16 weights to dst (16-byte aligned).
__device__ __forceinline__ void q4sub_store_bf16(const Q4Sub &r, int j, __bf16 *dst) {
    const float d = f16_ref(r.hdr.x & 0xFFFFu), dmin = f16_ref(r.hdr.x >> 16);
    const uint32_t sw = j < 4 ? r.hdr.y : r.hdr.w;
    const uint32_t mw = j < 4 ? r.hdr.z : r.mind;
    const int sh = 8 * (j & 3);
    const float S = d * (float)((sw >> sh) & 63), Mn = dmin * (float)((mw >> sh) & 63);
    const uint32_t qv[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    uint32_t o[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t byte = (qv[i] >> (8 * b)) & 0xFF;
            o[4 * i + b] = pack_bf16x2(fmaf(S, (float)(byte & 15), -Mn), fmaf(S, (float)(byte >> 4), -Mn));
        }
    }
    uint4 *d4 = reinterpret_cast<uint4 *>(dst);
#pragma unroll
    for (int i = 0; i < 4; i++) d4[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

// ---------------------------------------------------------------------------
// Expert tile GEMM.  MODE 0 (gate/up): grid = (max tiles, F/64); W rows
// 0..63 are gate rows n0.., 64..127 up rows n0..; X = x in bf16 by token;
// epilogue act = swiglu(g, u) in bf16.  MODE 1 (down): grid = (max tiles,
// H/128); W rows r0..r0+127 of W_down[e]; X = act by pair; epilogue y fp32.
// K = NS * 128.  Wave w owns pairs 16w..16w+15 and 8 16-column MFMA tiles.
// Global loads for step s+2 are issued before the MFMAs of step s (three
// register slots); each step dequantises its Q4_K half-super-blocks to bf16
// in LDS.
// ---------------------------------------------------------------------------
constexpr int PF_RING = 3;

template <int NS, int MODE>
__global__ __launch_bounds__(PF_THREADS) void k_expert_mfma(const uint8_t *__restrict__ W0, const uint8_t *__restrict__ W1,
                                                            const __bf16 *__restrict__ X, const int *__restrict__ perm,
                                                            const PfTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                                            int H, int F, int k, __bf16 *__restrict__ act,
                                                            float *__restrict__ y) {
    constexpr int K = NS * PF_KC;
    __shared__ __attribute__((aligned(16))) __bf16 Xs[PF_MT * PF_LD];
    __shared__ __attribute__((aligned(16))) __bf16 Ws[128 * PF_LD];
    if ((int)blockIdx.x >= *ntiles) return;
    const PfTile tl = tiles[blockIdx.x];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const long long rb = (long long)(K / 256) * 144;
    const int xi = tid >> 2, xq = tid & 3;
    const bool xv = xi < tl.n;
    const int pair = xv ? perm[tl.start + xi] : 0;
    const __bf16 *xrow = X + (long long)(MODE == 0 ? pair / k : pair) * K;
    const uint8_t *wrow[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int r = xi + 64 * u;
        if (MODE == 0)
            wrow[u] = (u == 0 ? W0 : W1) + ((long long)tl.e * F + blockIdx.y * 64 + xi) * rb;
        else
            wrow[u] = W0 + ((long long)tl.e * H + blockIdx.y * 128 + r) * rb;
    }
    uint4 xr[PF_RING][4];
    Q4Sub wr[PF_RING][2];
    auto load = [&](int slot, int step) {
        const int kc = step * PF_KC;
        if (xv) {
            const uint4 *src = reinterpret_cast<const uint4 *>(xrow + kc + 32 * xq);
#pragma unroll
            for (int i = 0; i < 4; i++) xr[slot][i] = src[i];
        }
        const int sbi = kc / 256, j = ((kc % 256) / 32) + xq;
#pragma unroll
        for (int u = 0; u < 2; u++) q4sub_load(wrow[u] + (long long)sbi * 144, j, wr[slot][u]);
    };
    f32x4 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s0 = 0; s0 < PF_RING - 1 && s0 < NS; s0++) load(s0, s0);
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int slot = s % PF_RING;
        if (s + PF_RING - 1 < NS) load((s + PF_RING - 1) % PF_RING, s + PF_RING - 1);
        __syncthreads();   // the previous step's MFMA reads are done
        {
            uint4 *xd = reinterpret_cast<uint4 *>(Xs + xi * PF_LD + 32 * xq);
#pragma unroll
            for (int i = 0; i < 4; i++) xd[i] = xv ? xr[slot][i] : make_uint4(0, 0, 0, 0);
            const int j = (((s * PF_KC) % 256) / 32) + xq;
#pragma unroll
            for (int u = 0; u < 2; u++) q4sub_store_bf16(wr[slot][u], j, Ws + (xi + 64 * u) * PF_LD + 32 * xq);
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < PF_KC; ks += 32) {
            const int kk = ks + 8 * (lane >> 4);
            const bf16x8 av = *reinterpret_cast<const bf16x8 *>(Xs + (16 * wave + (lane & 15)) * PF_LD + kk);
#pragma unroll
            for (int nt = 0; nt < 8; nt++) {
                const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(Ws + (16 * nt + (lane & 15)) * PF_LD + kk);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[nt], 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // lane holds pairs 16w + 4(l/16) + i of the tile, column 16nt + l%16
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int pi = 16 * wave + 4 * (lane >> 4) + i;
        if (pi < tl.n) {
            const int p = perm[tl.start + pi];
            if (MODE == 0) {
#pragma unroll
                for (int nt = 0; nt < 4; nt++) {
                    const float g = acc[nt][i], u = acc[nt + 4][i];
                    const float a = g / (1.0f + expf_glibc(-g)) * u;
                    act[(long long)p * F + blockIdx.y * 64 + 16 * nt + (lane & 15)] = (__bf16)a;
                }
            } else {
#pragma unroll
                for (int nt = 0; nt < 8; nt++)
                    y[(long long)p * H + blockIdx.y * 128 + 16 * nt + (lane & 15)] = acc[nt][i];
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_to_bf16(const float *__restrict__ x, __bf16 *__restrict__ o, long long n4) {
    for (long long i = blockIdx.x * 256ll + threadIdx.x; i < n4; i += (long long)gridDim.x * 256) {
        const float4 v = reinterpret_cast<const float4 *>(x)[i];
        reinterpret_cast<uint2 *>(o)[i] = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    }
}

size_t prefill_workspace_bytes(int T, int k, int E, int H, int F) {
    const size_t P = (size_t)T * k;
    const size_t max_tiles = (P + PF_MT - 1) / PF_MT + E;
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    return up(P * 4) + up(max_tiles * sizeof(PfTile)) + 256 + up(P * F * 2) + up((size_t)T * H * 2);
}

template <int MODE>
static hipError_t launch_expert_mfma(int ns, dim3 grid, hipStream_t st, const uint8_t *W0, const uint8_t *W1,
                                     const __bf16 *X, const int *perm, const PfTile *tiles, const int *ntiles, int H,
                                     int F, int k, __bf16 *act, float *y) {
#define TBQ_NS(N)                                                                                              \
    case N:                                                                                                    \
        hipLaunchKernelGGL((k_expert_mfma<N, MODE>), grid, dim3(PF_THREADS), 0, st, W0, W1, X, perm, tiles, ntiles, H, F, \
                           k, act, y);                                                                         \
        break;
    switch (ns) {
        TBQ_NS(2) TBQ_NS(4) TBQ_NS(6) TBQ_NS(8) TBQ_NS(12) TBQ_NS(16) TBQ_NS(24) TBQ_NS(32)
    default:
        return hipErrorNotSupported;
    }
#undef TBQ_NS
    return hipGetLastError();
}

// Experts on MFMA for Q4_K weights; routing already in a.sel_idx/a.sel_w.
// Uses a.y (pairs x H fp32) and `scratch` (prefill_workspace_bytes).
// K = H (gate/up) and F (down) must be 256, 512, 768, 1024, 1536, 2048,
// 3072 or 4096.
hipError_t launch_moe_prefill_q4k(const MoeArgs &a, void *scratch, hipStream_t st) {
    auto ok_k = [](int K) {
        const int n = K / PF_KC;
        return K % 256 == 0 && (n == 2 || n == 4 || n == 6 || n == 8 || n == 12 || n == 16 || n == 24 || n == 32);
    };
    if (a.qtype != QT_Q4_K || !ok_k(a.H) || !ok_k(a.F) || a.F % 64 || a.H % 128) return hipErrorNotSupported;
    const size_t P = (size_t)a.T * a.k;
    const int max_tiles = (int)((P + PF_MT - 1) / PF_MT + a.E);
    auto up = [](size_t n) { return (n + 255) & ~(size_t)255; };
    char *w = (char *)scratch;
    int *perm = (int *)w; w += up(P * 4);
    PfTile *tiles = (PfTile *)w; w += up((size_t)max_tiles * sizeof(PfTile));
    int *ntiles = (int *)w; w += 256;
    __bf16 *act = (__bf16 *)w; w += up(P * a.F * 2);
    __bf16 *xb = (__bf16 *)w;
    {
        const long long n4 = (long long)a.T * a.H / 4;
        const int grid = (int)((n4 + 255) / 256 < 2048 ? (n4 + 255) / 256 : 2048);
        hipLaunchKernelGGL(k_to_bf16, dim3(grid), dim3(256), 0, st, a.xn, xb, n4);
    }
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, a.sel_idx, a.T, a.k, a.E, perm, tiles, ntiles);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    err = launch_expert_mfma<0>(a.H / PF_KC, dim3(max_tiles, a.F / 64), st, (const uint8_t *)a.gate,
                                (const uint8_t *)a.up, xb, perm, tiles, ntiles, a.H, a.F, a.k, act, nullptr);
    if (err != hipSuccess) return err;
    return launch_expert_mfma<1>(a.F / PF_KC, dim3(max_tiles, a.H / 128), st, (const uint8_t *)a.down, nullptr, act,
                                 perm, tiles, ntiles, a.H, a.F, a.k, nullptr, a.y);
}

}  // namespace tbq
