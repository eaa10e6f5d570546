// tbq_moe_q4k.hip -- the MoE block's decode path on gfx950:
//
//   k_router_logits<EPB>  logits[t][e] = sum_k fl(W[e][k] * x[k]) summed in the
//                         reference's order (acc = acc + p, k ascending).  The
//                         sum is a dependent chain, so one lane owns one
//                         expert; four loader waves form the products of the
//                         next 32 KB tile in LDS while the chain wave adds
//                         the current one (double-buffered).
//   k_topk                softmax + top-k + renormalise per token, bit-exact
//                         to tb_route_experts (layer4/tb_infer.c:351-374).
//   k_gate_up_q4k         act[t][s] = swiglu(W_gate[e] x, W_up[e] x) with the
//                         Q4_K int-dot units; a wave's two half-waves take
//                         gate row r and up row r.
//   k_down_combine_q4k    out[t][r] = resid[t][r] + sum_s w_s * (W_down[e_s] a_s)[r]
//                         with the sum over slots in slot order, exactly as
//                         the reference's weighted accumulate (tb_infer.c:
//                         829-831) and residual add (:876).
#include "tbq_kernels.h"
#include "tbq_q4k.hpp"
#include "tbq_topk.hpp"

namespace tbq {

// ---------------------------------------------------------------------------
// Router logits.  grid = (T, ceil(E/EPB)); block = 64 (chain) + 256 (loaders).
// ---------------------------------------------------------------------------
constexpr int RT_LOADERS = 256;
constexpr int RT_THREADS = 64 + RT_LOADERS;
constexpr int RT_TILE_FLOATS = 4096;   // 16 KB of products per tile

template <int EPB>
__global__ __launch_bounds__(RT_THREADS) void k_router_logits(const float *__restrict__ xn, const float *__restrict__ Wr,
                                                              const float *__restrict__ bias, int H, int E,
                                                              float *__restrict__ logits) {
    constexpr int KT = RT_TILE_FLOATS / EPB;        // k per tile (256 for EPB=16, 64 for EPB=64)
    constexpr int F4 = KT / 4;                       // float4 per expert row of a tile
    constexpr int SEGS = KT / 16;                    // 16-k segments per expert row
    static_assert(EPB * SEGS == RT_LOADERS, "one 16-k segment per loader thread");
    static_assert(F4 % 8 == 0, "swizzle needs 8 float4 per row");
    extern __shared__ float lds[];
    float *xl = lds;                                 // H floats
    float *buf = lds + H;                            // 2 tiles of EPB x KT products
    const int t = blockIdx.x, e0 = blockIdx.y * EPB, tid = threadIdx.x;
    const float *x = xn + (long long)t * H;
    const int ntiles = H / KT;

    // loader role: expert ei, 16 consecutive k of each tile; W of tile i is
    // held in register set i&1, two tiles ahead of the chain
    const int lt = tid - 64, ei = lt / SEGS, seg = lt % SEGS;
    const bool loader = tid >= 64, lvalid = loader && e0 + ei < E;
    float4 wa[4], wb[4];
    auto issue = [&](float4 *w, int tile) {
        if (lvalid && tile < ntiles) {
            const float4 *src = reinterpret_cast<const float4 *>(Wr + (long long)(e0 + ei) * H + tile * KT + 16 * seg);
#pragma unroll
            for (int i = 0; i < 4; i++) w[i] = src[i];
        }
    };
    auto produce = [&](const float4 *w, int tile) {
        // float4 j of row ei goes to j ^ (ei & 7): chain lanes read distinct banks
        float *dst = buf + (tile & 1) * RT_TILE_FLOATS + ei * KT;
        const float *xk = xl + tile * KT + 16 * seg;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = 4 * seg + i;
            float4 p;
            p.x = lvalid ? w[i].x * xk[4 * i] : 0.f;
            p.y = lvalid ? w[i].y * xk[4 * i + 1] : 0.f;
            p.z = lvalid ? w[i].z * xk[4 * i + 2] : 0.f;
            p.w = lvalid ? w[i].w * xk[4 * i + 3] : 0.f;
            *reinterpret_cast<float4 *>(dst + 4 * (j ^ (ei & 7))) = p;
        }
    };
    float acc = 0.f;
    auto chain = [&](int tile) {
        if (!loader && tid < EPB) {
            // the next 8 float4 are read from LDS while the current 8 are added
            const float *src = buf + (tile & 1) * RT_TILE_FLOATS + tid * KT;
            float4 cur[8], nxt[8];
#pragma unroll
            for (int i = 0; i < 8; i++) cur[i] = *reinterpret_cast<const float4 *>(src + 4 * (i ^ (tid & 7)));
#pragma unroll
            for (int jb = 0; jb < F4; jb += 8) {
                if (jb + 8 < F4) {
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        nxt[i] = *reinterpret_cast<const float4 *>(src + 4 * ((jb + 8 + i) ^ (tid & 7)));
                }
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    acc = acc + cur[i].x;
                    acc = acc + cur[i].y;
                    acc = acc + cur[i].z;
                    acc = acc + cur[i].w;
                }
#pragma unroll
                for (int i = 0; i < 8; i++) cur[i] = nxt[i];
            }
        }
    };
    issue(wa, 0);
    issue(wb, 1);
    for (int i = tid * 4; i < H; i += RT_THREADS * 4) *reinterpret_cast<float4 *>(xl + i) = *reinterpret_cast<const float4 *>(x + i);
    __syncthreads();
    // step it: loaders form tile it, chain adds tile it-1; unrolled by two so
    // the register sets are addressed statically
    for (int it = 0; it <= ntiles; it += 2) {
        if (loader && it < ntiles) { produce(wa, it); issue(wa, it + 2); }
        if (it > 0) chain(it - 1);
        __syncthreads();
        if (it + 1 > ntiles) break;
        if (loader && it + 1 < ntiles) { produce(wb, it + 1); issue(wb, it + 3); }
        chain(it);
        __syncthreads();
    }
    if (tid < EPB && e0 + tid < E) {
        float lg = acc;
        if (bias) lg = lg + bias[e0 + tid];
        logits[(long long)t * E + e0 + tid] = lg;
    }
}

// ---------------------------------------------------------------------------
// Decode-size router: EPB_S experts per workgroup, the whole W slice loaded
// at once (one load latency), products for all of H formed in LDS, then one
// lane per expert runs the sequential chain.  grid = (T, ceil(E/EPB_S)).
// ---------------------------------------------------------------------------
constexpr int EPB_S = 4;
constexpr int RS_THREADS = 256;

template <int KPT>   // floats of W per thread: EPB_S * H / RS_THREADS
__global__ __launch_bounds__(RS_THREADS) void k_router_logits_small(const float *__restrict__ xn,
                                                                    const float *__restrict__ Wr,
                                                                    const float *__restrict__ bias, int H, int E,
                                                                    float *__restrict__ logits) {
    extern __shared__ float prod[];                  // EPB_S rows of H products (float4-swizzled)
    const int t = blockIdx.x, e0 = blockIdx.y * EPB_S, tid = threadIdx.x;
    // thread -> expert ei, KPT consecutive k
    const int tpe = RS_THREADS / EPB_S, ei = tid / tpe, k0 = (tid % tpe) * KPT;
    const bool valid = e0 + ei < E;
    float4 w[KPT / 4], xv[KPT / 4];
    if (valid) {
        const float4 *src = reinterpret_cast<const float4 *>(Wr + (long long)(e0 + ei) * H + k0);
#pragma unroll
        for (int i = 0; i < KPT / 4; i++) w[i] = src[i];
    }
    const float4 *xs = reinterpret_cast<const float4 *>(xn + (long long)t * H + k0);
#pragma unroll
    for (int i = 0; i < KPT / 4; i++) xv[i] = xs[i];
    float *row = prod + ei * H;
#pragma unroll
    for (int i = 0; i < KPT / 4; i++) {
        float4 p;
        p.x = valid ? w[i].x * xv[i].x : 0.f;
        p.y = valid ? w[i].y * xv[i].y : 0.f;
        p.z = valid ? w[i].z * xv[i].z : 0.f;
        p.w = valid ? w[i].w * xv[i].w : 0.f;
        const int j = k0 / 4 + i;                    // float4 index within the row
        *reinterpret_cast<float4 *>(row + 4 * (j ^ (ei & 3))) = p;
    }
    __syncthreads();
    if (tid < EPB_S && valid) {
        const float *src = prod + tid * H;
        const int F4 = H / 4;
        float acc = 0.f;
        float4 cur[8], nxt[8];
#pragma unroll
        for (int i = 0; i < 8; i++) cur[i] = *reinterpret_cast<const float4 *>(src + 4 * (i ^ (tid & 3)));
        for (int jb = 0; jb < F4; jb += 8) {
            if (jb + 8 < F4) {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    nxt[i] = *reinterpret_cast<const float4 *>(src + 4 * ((jb + 8 + i) ^ (tid & 3)));
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                acc = acc + cur[i].x;
                acc = acc + cur[i].y;
                acc = acc + cur[i].z;
                acc = acc + cur[i].w;
            }
#pragma unroll
            for (int i = 0; i < 8; i++) cur[i] = nxt[i];
        }
        if (bias) acc = acc + bias[e0 + tid];
        logits[(long long)t * E + e0 + tid] = acc;
    }
}

template <int NJ>
__global__ __launch_bounds__(64) void k_topk(const float *__restrict__ logits, int E, int top_k,
                                             int *__restrict__ sel_idx, float *__restrict__ sel_w) {
    __shared__ float P[64 * NJ + 16];
    topk_wave<NJ, false>(logits + (long long)blockIdx.x * E, E, top_k, blockIdx.x, P, sel_idx, sel_w);
}

// ---------------------------------------------------------------------------
// DPP router for H = 64*M.  A wave owns 4 experts, one per 16-lane row; lane
// j of a row holds the products of k = 64m + 4j + c (m < M, c < 4) in
// registers, and the row's last lane adds them in k order with
// v_add_f32_dpp row_shr (one instruction per element, no LDS).  The last
// workgroup of a token (per-token arrival counter, reset by that workgroup)
// runs the softmax/top-k.  grid = (ceil(E/4), T), 64 threads.
// ---------------------------------------------------------------------------
// One 64-element block of the chain: lane j of each 16-lane row holds w and
// x for k = 4j..4j+3 of the block; the products are formed in place, then
// the row's last lane (j = 15) adds the 64 products in k order, reading lane
// j's registers with row_shr:(15-j).  s_nop 1 covers the VALU-write ->
// DPP-read hazard.  IEEE fp32 add (commutative, round to nearest), no fma:
// acc = fl(acc + fl(w*x)) exactly as the reference's sequential dot.
#define TBQ_DPP_ADD(SH, R) "v_add_f32_dpp %0, %" #R ", %0 row_shr:" #SH " row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
#define TBQ_DPP_ADD4(SH) TBQ_DPP_ADD(SH, 1) TBQ_DPP_ADD(SH, 2) TBQ_DPP_ADD(SH, 3) TBQ_DPP_ADD(SH, 4)
__device__ __forceinline__ float chain_block64(float acc, float4 w, float4 x) {
    asm volatile(
        "v_mul_f32 %1, %1, %5\n"
        "v_mul_f32 %2, %2, %6\n"
        "v_mul_f32 %3, %3, %7\n"
        "v_mul_f32 %4, %4, %8\n"
        "s_nop 1\n"
        TBQ_DPP_ADD4(15) TBQ_DPP_ADD4(14) TBQ_DPP_ADD4(13) TBQ_DPP_ADD4(12) TBQ_DPP_ADD4(11)
        TBQ_DPP_ADD4(10) TBQ_DPP_ADD4(9) TBQ_DPP_ADD4(8) TBQ_DPP_ADD4(7) TBQ_DPP_ADD4(6)
        TBQ_DPP_ADD4(5) TBQ_DPP_ADD4(4) TBQ_DPP_ADD4(3) TBQ_DPP_ADD4(2) TBQ_DPP_ADD4(1)
        "v_add_f32 %0, %1, %0\n"
        "v_add_f32 %0, %2, %0\n"
        "v_add_f32 %0, %3, %0\n"
        "v_add_f32 %0, %4, %0\n"
        : "+v"(acc), "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w)
        : "v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w));
    return acc;
}
#undef TBQ_DPP_ADD4
#undef TBQ_DPP_ADD

// Chunks of 8 blocks (512 k) stream through two register slots: the loads
// of chunk c+1 are issued before the chain of chunk c; sched_barrier keeps
// the compiler from hoisting further.
constexpr int RD_CH = 8;

template <int C, int NC>
__device__ __forceinline__ void router_dpp_chunks(const float4 *w4, const float4 *x4, int j, float4 (&wb)[2][RD_CH],
                                                  float4 (&xb)[2][RD_CH], float &acc) {
    if constexpr (C < NC) {
        if constexpr (C + 1 < NC) {
#pragma unroll
            for (int i = 0; i < RD_CH; i++) {
                wb[(C + 1) & 1][i] = w4[16 * (RD_CH * (C + 1) + i) + j];
                xb[(C + 1) & 1][i] = x4[16 * (RD_CH * (C + 1) + i) + j];
            }
        }
#pragma unroll
        for (int i = 0; i < RD_CH; i++) acc = chain_block64(acc, wb[C & 1][i], xb[C & 1][i]);
        __builtin_amdgcn_sched_barrier(0);
        router_dpp_chunks<C + 1, NC>(w4, x4, j, wb, xb, acc);
    }
}

// H <= 64 * RD_CH * RD_ALL_NC: every load of the workgroup's slice is
// issued up front (256 VGPRs at H = 2048), so only the first load's latency
// is exposed and the chain consumes the chunks as they arrive.
#ifndef TBQ_RD_ALL_NC
#define TBQ_RD_ALL_NC 4
#endif
constexpr int RD_ALL_NC = TBQ_RD_ALL_NC;

template <int NC>
__device__ __forceinline__ float router_dpp_all(const float4 *w4, const float4 *x4, int j) {
    float4 wb[NC * RD_CH], xb[NC * RD_CH];
#pragma unroll
    for (int i = 0; i < NC * RD_CH; i++) {
        wb[i] = w4[16 * i + j];
        xb[i] = x4[16 * i + j];
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NC * RD_CH; i++) acc = chain_block64(acc, wb[i], xb[i]);
    return acc;
}

// ---------------------------------------------------------------------------
// Decode batches (2 <= T <= 32) in expert order.  group_pairs sorts the
// batch's T*k selections by expert:
//   grp[0]                U, the number of distinct experts
//   grp[1 + u]            expert of group u (ascending)
//   grp[1 + E + u]        first position of group u in the pair list
//   grp[1 + 2E + u]       number of pairs in group u
//   grp[1 + 3E + i]       pair list (t*k + s), by expert (the pairs of one
//                         expert in no particular order)
//   grp[1 + 3E + T*k]     number of valid pairs in the list
// T*k <= 256, T <= 32, E <= 256.  The per-pair expert kernels then take their
// grid's pair column from the list, so the workgroups of the pairs that
// share an expert run back to back on the same XCDs (a workgroup's XCD
// follows its row block) and the later ones read the expert's rows from L2
// instead of HBM.  Each pair's result is computed on its own and the combine
// adds the slots in slot order, so the order within a group does not change
// any result.
// ---------------------------------------------------------------------------

// By the NT threads of a workgroup (a multiple of 64 dividing 256).  cnt:
// 256 ints of LDS; wsum: 2 * NT / 64 ints of LDS.  The selections are read
// with device-scope loads (they may have been stored by another workgroup of
// the same kernel).
template <int NT>
__device__ __forceinline__ void group_pairs(const int *sel_idx, int T, int E, int k, int *__restrict__ grp, int *cnt,
                                            int *wsum) {
    constexpr int PER = 256 / NT, NWV = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, n = T * k;
#pragma unroll
    for (int j = 0; j < PER; j++) cnt[tid + NT * j] = 0;
    __syncthreads();
    int ev[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = tid + NT * j;
        int e = -1;
        if (i < n) {
            const int t = i / k, s = i - t * k;
            e = __hip_atomic_load(sel_idx + t * 8 + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((unsigned)e >= (unsigned)E) e = -1;   // never produced by the router: left out
        }
        ev[j] = e;
        if (e >= 0) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // thread tid owns experts PER*tid .. PER*tid + PER-1: exclusive scans of
    // the pair counts (list offsets) and of the non-empty flags (group ranks)
    int c[PER], sc = 0, sg = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int x = PER * tid + j;
        c[j] = x < E ? cnt[x] : 0;
        sc += c[j];
        sg += c[j] > 0;
    }
    int ic = sc, ig = sg;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int a = __shfl_up(ic, d), b = __shfl_up(ig, d);
        if (lane >= d) {
            ic += a;
            ig += b;
        }
    }
    if constexpr (NWV > 1) {
        if (lane == 63) {
            wsum[tid >> 6] = ic;
            wsum[NWV + (tid >> 6)] = ig;
        }
        __syncthreads();
        for (int w = 0; w < (tid >> 6); w++) {
            ic += wsum[w];
            ig += wsum[NWV + w];
        }
    }
    int off = ic - sc, rank = ig - sg;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int x = PER * tid + j;
        if (c[j] > 0) {
            grp[1 + rank] = x;
            grp[1 + E + rank] = off;
            grp[1 + 2 * E + rank] = c[j];
            rank++;
        }
        if (x < E) cnt[x] = off;   // the expert's list cursor
        off += c[j];
    }
    if (tid == NT - 1) {
        grp[0] = ig;
        grp[1 + 3 * E + n] = ic;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; j++)
        if (ev[j] >= 0) grp[1 + 3 * E + atomicAdd(&cnt[ev[j]], 1)] = tid + NT * j;
}

// With grp, the batch is also sorted by expert (group_pairs) by the
// workgroup that finishes the last token's top-k, which saves a launch of
// k_group: each token's top-k workgroup takes a ticket on the batch counter
// counters[RD_GRP_CTR] after its selection stores have completed.
constexpr int RD_GRP_CTR = 32;   // counters[0, T) are the tokens' (T < 32)

template <int M, int NJ>
__global__ __launch_bounds__(64) void k_router_dpp(const float *__restrict__ xn, const float *__restrict__ Wr,
                                                   const float *__restrict__ bias, int E, int top_k,
                                                   float *__restrict__ logits, unsigned *__restrict__ counters,
                                                   int *__restrict__ sel_idx, float *__restrict__ sel_w, int k,
                                                   int *__restrict__ grp) {
    constexpr int H = 64 * M, NC = M / RD_CH;
    static_assert(M % RD_CH == 0, "H must be a multiple of 512");
    __shared__ float P[64 * NJ + 16];
    __shared__ int gcnt[256];
    const int t = blockIdx.y, lane = threadIdx.x, r = lane >> 4, j = lane & 15;
    const int e = blockIdx.x * 4 + r;
    const bool ev = e < E;
    const float4 *w4 = reinterpret_cast<const float4 *>(Wr + (long long)(ev ? e : 0) * H);
    const float4 *x4 = reinterpret_cast<const float4 *>(xn + (long long)t * H);
    float acc = 0.f;
    if constexpr (NC <= RD_ALL_NC) {
        acc = router_dpp_all<NC>(w4, x4, j);
    } else {
        float4 wb[2][RD_CH], xb[2][RD_CH];
#pragma unroll
        for (int i = 0; i < RD_CH; i++) {
            wb[0][i] = w4[16 * i + j];
            xb[0][i] = x4[16 * i + j];
        }
        router_dpp_chunks<0, NC>(w4, x4, j, wb, xb, acc);
    }
    if (j == 15 && ev) {
        if (bias) acc = acc + bias[e];
        __hip_atomic_store(logits + (long long)t * E + e, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The last arriving workgroup of this token does the top-k.  The logits
    // cross workgroups as device-scope atomic stores and loads (coherent
    // across the XCDs' L2s without a cache write-back or invalidate, which a
    // device-scope fence would cost in every workgroup): each workgroup
    // waits until its stores have completed before it takes its ticket, and
    // the last one reads the logits with device-scope atomic loads.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned ticket = 0;
    if (lane == 0) ticket = __hip_atomic_fetch_add(counters + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ticket = (unsigned)__builtin_amdgcn_readfirstlane((int)ticket);
    if (ticket != gridDim.x - 1) return;
    asm volatile("" ::: "memory");
    topk_wave<NJ>(logits + (long long)t * E, E, top_k, t, P, sel_idx, sel_w);
    if (lane == 0) counters[t] = 0u;
    if (!grp) return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the selection stores have completed
    unsigned bt = 0;
    if (lane == 0)
        bt = __hip_atomic_fetch_add(counters + RD_GRP_CTR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bt = (unsigned)__builtin_amdgcn_readfirstlane((int)bt);
    if (bt != gridDim.y - 1) return;
    asm volatile("" ::: "memory");
    group_pairs<64>(sel_idx, (int)gridDim.y, E, k, grp, gcnt, nullptr);
    if (lane == 0) counters[RD_GRP_CTR] = 0u;
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU, Q4_K experts.  grid = (ceil(F / OUT_PER_WG), T*k); each
// wave owns one output row per pass: lanes [0, 32) dot the gate row, lanes
// [32, 64) the up row (LPR = 32 lanes hold one 64-weight unit each when
// H = 2048; larger H loops units).
// ---------------------------------------------------------------------------
#ifndef TBQ_GU_WAVES
#define TBQ_GU_WAVES 8
#endif
#ifndef TBQ_GU_ROWS
#define TBQ_GU_ROWS 1
#endif
// expert-ordered batches: 4-wave workgroups (b=16 93.0 -> 92.6 us, with a
// Q6_K down 106.7 -> 106.2; at b=1 8 waves stay faster, 22.7 against 23.4)
#ifndef TBQ_GU_WAVES_B
#define TBQ_GU_WAVES_B 4
#endif
constexpr int GU_THREADS = 64 * TBQ_GU_WAVES;
constexpr int GU_ROWS = TBQ_GU_ROWS;   // output rows per wave

template <int UPL, bool GG, int ROWS = GU_ROWS, int NWV = TBQ_GU_WAVES>
__global__ __launch_bounds__(64 * NWV) void k_gate_up_q4k(const uint8_t *__restrict__ gate, const uint8_t *__restrict__ up,
                                                            const float *__restrict__ xn, const int *__restrict__ sel_idx,
                                                            const int *__restrict__ order, const int *__restrict__ nvalid,
                                                            int H, int F, int E, int k, float *__restrict__ act) {
    extern __shared__ uint32_t xd[];
    constexpr int LPR = 32;
    // with an order list (expert-ordered valid pairs), column y runs pair order[y]
    if (order && (int)blockIdx.y >= *nvalid) return;   // workgroup-uniform
    const int pair = order ? order[blockIdx.y] : blockIdx.y, t = pair / k, s = pair % k;
    // an index outside [0, E) (never produced by the router) reads expert 0
    // and contributes 0: no weight read leaves the expert tensors
    const int e_sel = sel_idx[t * 8 + s];
    const bool ev = (unsigned)e_sel < (unsigned)E;
    const int e = ev ? e_sel : 0;
    const long long rb = (long long)(H / 256) * 144;
    const int U = H / 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane & 31, half = lane >> 5;
    const uint8_t *Wb = (half ? up : gate) + (long long)e * F * rb;
    const int r0 = (blockIdx.x * NWV + wave) * ROWS;

    XStager<64 * NWV, (1024 + 64 * NWV - 1) / (64 * NWV)> xs;   // H <= 8192
    xs.load(xn + (long long)t * H, H);
    __builtin_amdgcn_sched_barrier(0);   // x's loads stay ahead of the weights'
    // Unconditional loads (rows past F re-read row F-1, units past U unit 0;
    // their results are never used): under a branch the compiler waits for
    // every weight load before staging x.
    Q4KUnit raw[ROWS][UPL];
#pragma unroll
    for (int rr = 0; rr < ROWS; rr++) {
        const int r = min(r0 + rr, F - 1);
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const int u = lr + LPR * i;
            q4k_load<GG>(Wb + (long long)r * rb, u < U ? u : 0, raw[rr][i]);
        }
    }
    xs.store(xd, H);
    __syncthreads();
    // A lane's unit is the same for all its rows: with one unit per lane
    // its digits are read from LDS once, a quarter of the LDS reads at 4
    // rows (measured no faster or slower); with two, per row (both in
    // registers for 4 rows would cost a wave per SIMD).
    constexpr bool XREG = UPL == 1 && ROWS > 1;
    XUnit xu;
    if constexpr (XREG) xunit_load(xd, lr < U ? lr : 0, xu);
#pragma unroll
    for (int rr = 0; rr < ROWS; rr++) {
        const int r = r0 + rr;
        if (r >= F) break;   // wave-uniform
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const int u = lr + LPR * i;
            if (u < U) {
                if constexpr (XREG)
                    acc = q4k_unit_dot<GG>(raw[rr][i], u, xu, acc);
                else
                    acc = q4k_unit_dot<GG>(raw[rr][i], u, xd, acc);
            }
        }
        acc = group_sum<32>(acc);
        const float u_val = __shfl(acc, 32);
        if (lane == 0) {
            const float g = acc;
            const float den = 1.0f + expf_glibc(-g);
            const float sg = g / den;
            act[(long long)pair * F + r] = ev ? sg * u_val : 0.f;
        }
    }
}

__global__ __launch_bounds__(256) void k_group(const int *__restrict__ sel_idx, int T, int E, int k,
                                               int *__restrict__ grp) {
    __shared__ int cnt[256], wsum[8];
    group_pairs<256>(sel_idx, T, E, k, grp, cnt, wsum);
}

// down for one pair: y[p][r] = W_down[e] act[p] over DG_ROWS rows, p taken
// from the expert-ordered pair list (k_combine then adds the slots in slot
// order).  grid = (H / DG_ROWS, T*k).  4-wave workgroups of 64 rows (b=16
// 92.4 -> 90.6 us against 8 waves of 128 rows; 4 waves of 128: 91.0; 2
// waves of 32 or 64 rows: +1.0 / +1.5 us).
#ifndef TBQ_DG_THREADS
#define TBQ_DG_THREADS 256
#endif
#ifndef TBQ_DG_ROWS
#define TBQ_DG_ROWS 64
#endif
constexpr int DG_THREADS = TBQ_DG_THREADS;
constexpr int DG_ROWS = TBQ_DG_ROWS;   // rows per workgroup: passes of DG_THREADS / 16 (16 lanes per row)
static_assert(DG_ROWS % (DG_THREADS / 16) == 0, "whole passes");

template <int UPL, bool GG>
__global__ __launch_bounds__(DG_THREADS) void k_down_pair_q4k(const uint8_t *__restrict__ down,
                                                              const float *__restrict__ act,
                                                              const int *__restrict__ sel_idx,
                                                              const int *__restrict__ order,
                                                              const int *__restrict__ nvalid, int H, int F, int E,
                                                              int k, float *__restrict__ y) {
    extern __shared__ uint32_t xd[];   // the pair's act digits
    constexpr int LPR = 16, PASSES = DG_ROWS / (DG_THREADS / LPR);
    if ((int)blockIdx.y >= *nvalid) return;   // workgroup-uniform
    const int pair = order[blockIdx.y];
    const int e = sel_idx[(pair / k) * 8 + pair % k];
    if ((unsigned)e >= (unsigned)E) return;   // the list holds valid pairs only
    const long long rb = (long long)(F / 256) * 144;
    const int U = F / 64;
    const int lr = threadIdx.x & 15, rl = threadIdx.x >> 4;   // row of the pass
    const int r0 = blockIdx.x * DG_ROWS;
    XStager<DG_THREADS, (512 + DG_THREADS - 1) / DG_THREADS> xs;   // F <= 4096
    xs.load(act + (long long)pair * F, F);
    __builtin_amdgcn_sched_barrier(0);   // x's loads stay ahead of the weights'
    // unconditional loads (units past U read unit 0, unused), so the
    // staging of act does not wait for the weights
    Q4KUnit raw[PASSES][UPL];
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const uint8_t *row = down + ((long long)e * H + r0 + (DG_THREADS / LPR) * p + rl) * rb;
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const int u = lr + LPR * i;
            q4k_load<GG>(row, u < U ? u : 0, raw[p][i]);
        }
    }
    xs.store(xd, F);
    __syncthreads();
    // with one unit per lane its digits are read from LDS once for all
    // passes (a quarter of the LDS reads; measured no faster or slower)
    constexpr bool XREG = UPL == 1;
    XUnit xu;
    if constexpr (XREG) xunit_load(xd, lr < U ? lr : 0, xu);
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int r = r0 + (DG_THREADS / LPR) * p + rl;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const int u = lr + LPR * i;
            if (u < U) {
                if constexpr (XREG)
                    acc = q4k_unit_dot<GG>(raw[p][i], u, xu, acc);
                else
                    acc = q4k_unit_dot<GG>(raw[p][i], u, xd, acc);
            }
        }
        acc = group_sum<16>(acc);
        if (lr == 0) y[(long long)pair * H + r] = acc;
    }
}

// ---------------------------------------------------------------------------
// down + weighted combine + residual, Q4_K experts.  grid = (H / RB, T);
// the workgroup owns RB output rows of one token for all k slots.  Each
// (row, slot) dot uses LPR = 16 lanes (K = F = 768 gives 12 units; larger F
// loops units).  Results meet in LDS and one lane per row adds them in slot
// order.
// ---------------------------------------------------------------------------
#ifndef TBQ_DC_ROWS
#define TBQ_DC_ROWS 4
#endif
constexpr int DC_THREADS = 512;
constexpr int DC_ROWS = TBQ_DC_ROWS;   // rows per workgroup

template <int UPL, bool GG>
__global__ __launch_bounds__(DC_THREADS) void k_down_combine_q4k(const uint8_t *__restrict__ down, const float *__restrict__ act,
                                                                 const int *__restrict__ sel_idx, const float *__restrict__ sel_w,
                                                                 const float *__restrict__ resid, int H, int F, int E,
                                                                 int k, float *__restrict__ out) {
    extern __shared__ uint32_t xd[];                  // k act vectors' digits
    __shared__ float yv[8][DC_ROWS];
    constexpr int LPR = 16, RPP = 4;
    const int t = blockIdx.y, r0 = blockIdx.x * DC_ROWS;
    const long long rb = (long long)(F / 256) * 144;
    const int U = F / 64, G = F / 32;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lr = lane & 15, rsub = lane >> 4;
    // dot d = (row rd, slot sd), d < DC_ROWS * k; wave w pass p takes dots 4*(w + 8p) + rsub
    constexpr int PASSES = (DC_ROWS * 8 + (DC_THREADS / 64) * RPP - 1) / ((DC_THREADS / 64) * RPP);
    // the experts of the lane's dots first: the weight addresses wait for
    // them, and loaded after x's rows that wait would take x's loads too
    int esel[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int d = min(RPP * (wave + (DC_THREADS / 64) * p) + rsub, DC_ROWS * k - 1);
        esel[p] = sel_idx[t * 8 + d % k];
    }
    XStager<DC_THREADS, 2 * UPL> xs;   // k <= 8 vectors of F <= 1024 * UPL
    xs.load(act + (long long)t * k * F, F, k);
    __builtin_amdgcn_sched_barrier(0);   // x's loads stay ahead of the weights'
    // unconditional loads (dots past DC_ROWS*k redo the last one, units past
    // U read unit 0; unused), so the staging does not wait for the weights
    Q4KUnit raw[PASSES][UPL];
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int d = min(RPP * (wave + (DC_THREADS / 64) * p) + rsub, DC_ROWS * k - 1);
        const int rd = d / k;
        const int e_sel = esel[p];
        const int e = (unsigned)e_sel < (unsigned)E ? e_sel : 0;   // out of range: contributes 0 below
        const uint8_t *row = down + ((long long)e * H + r0 + rd) * rb;
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const int u = lr + LPR * i;
            q4k_load<GG>(row, u < U ? u : 0, raw[p][i]);
        }
    }
    xs.store(xd, F, k);
    __syncthreads();
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int d = RPP * (wave + (DC_THREADS / 64) * p) + rsub;
        const bool dv = d < DC_ROWS * k;
        const int rd = dv ? d / k : 0, sd = dv ? d % k : 0;
        float acc = 0.f;
        if (dv) {
#pragma unroll
            for (int i = 0; i < UPL; i++) {
                const int u = lr + LPR * i;
                if (u < U) acc = q4k_unit_dot<GG>(raw[p][i], u, xd + sd * G * XD_PER_SB, acc);
            }
        }
        acc = group_sum<16>(acc);
        if (dv && lr == 0) yv[sd][rd] = (unsigned)sel_idx[t * 8 + sd] < (unsigned)E ? acc : 0.f;
    }
    __syncthreads();
    if (threadIdx.x < DC_ROWS) {
        const int rd = threadIdx.x, r = r0 + rd;
        float a = 0.f;
        for (int s = 0; s < k; s++) {
            if ((unsigned)sel_idx[t * 8 + s] >= (unsigned)E) continue;   // never produced by the router
            const float pr = sel_w[t * 8 + s] * yv[s][rd];
            a = a + pr;
        }
        out[(long long)t * H + r] = resid[(long long)t * H + r] + a;
    }
}

// ---------------------------------------------------------------------------
// Batch router (T >= 32): a workgroup of 4 waves owns 4 tokens x 64 experts;
// lane e of wave w runs token w's chain for expert e, acc = fl(acc +
// fl(w*x)) over k ascending.  Each 64-k chunk of the 64 experts' W (16 KB)
// and of the 4 tokens' x is loaded once per workgroup with coalesced 16-byte
// loads and stored to LDS transposed ([k/4][expert] float4), so lane e's
// ds_read_b128 is conflict-free and x is a broadcast read.  A chunk's global
// loads are issued while the previous chunk is summed.  Requires H % 256 == 0.
// grid = (ceil(T/4), ceil(E/64)), 256 threads.
// ---------------------------------------------------------------------------
constexpr int RB_TOK = 4, RB_KC = 256, RB_THREADS = 64 * RB_TOK;
constexpr int RB_Q = RB_KC / 4;                      // float4 per row per chunk
constexpr int RB_WPT = 64 * RB_Q / RB_THREADS;       // W float4 per thread per chunk

// Native 4-float vectors: HIP's float4 struct is copied with memcpy between
// address spaces, which keeps a register array in scratch memory.
typedef float rb_f4 __attribute__((ext_vector_type(4)));

// wb[b][q][e ^ (q & 7)] holds W[e][4q..4q+3]: for a fixed q the 64 experts
// are a permutation of one 1 KB row (lane e's ds_read_b128 is conflict-free),
// and the loaders -- lane l stores q = l -- spread every 8-lane store phase
// over 8 distinct bank groups.  xb holds the 4 tokens' x (broadcast reads).
struct RbShared {
    rb_f4 wb[2][RB_Q][64];        // [buffer][k/4][expert, swizzled]
    rb_f4 xb[2][RB_TOK][RB_Q];    // [buffer][token][k/4]
};

// Sum one chunk from LDS, 16 k (4 float4) at a time, with the next group's
// LDS reads issued before the current group's arithmetic (two register
// slots, static indices); the empty asm statements (tied to acc) keep the
// compiler from hoisting more of the chunk's reads, which would push the
// in-flight global loads to scratch.
__device__ __forceinline__ float rb_chunk(const RbShared &sh, int b, int lane, int wave, float acc) {
    constexpr int NG = RB_Q / 4;
    rb_f4 w[2][4], xv[2][4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        w[0][q] = sh.wb[b][q][lane ^ (q & 7)];
        xv[0][q] = sh.xb[b][wave][q];
    }
#pragma unroll
    for (int g = 0; g < NG; g++) {
        if (g + 1 < NG) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int qq = 4 * (g + 1) + q;
                w[(g + 1) & 1][q] = sh.wb[b][qq][lane ^ (qq & 7)];
                xv[(g + 1) & 1][q] = sh.xb[b][wave][qq];
            }
        }
        // the 16 products first (independent), then the dependent adds back
        // to back: interleaved, every add would wait for the multiply just
        // issued as well as for the previous add
        float p[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const rb_f4 ww = w[g & 1][q], xx = xv[g & 1][q];
            p[4 * q] = ww.x * xx.x;
            p[4 * q + 1] = ww.y * xx.y;
            p[4 * q + 2] = ww.z * xx.z;
            p[4 * q + 3] = ww.w * xx.w;
        }
        asm volatile("" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]), "+v"(p[4]), "+v"(p[5]), "+v"(p[6]),
                     "+v"(p[7]), "+v"(p[8]), "+v"(p[9]), "+v"(p[10]), "+v"(p[11]), "+v"(p[12]), "+v"(p[13]),
                     "+v"(p[14]), "+v"(p[15]));
#pragma unroll
        for (int i = 0; i < 16; i++) acc = acc + p[i];
        asm volatile("" : "+v"(acc));
    }
    return acc;
}

// This thread's share of chunk c: W float4 q of rows r0 + RPP*i (row
// stride wstride float4) and x float4 q of token row r0.
__device__ __forceinline__ void rb_load(rb_f4 (&wr)[RB_WPT], rb_f4 &xr, const rb_f4 *wsrc, long long wstride,
                                        const rb_f4 *xsrc, int c) {
#pragma unroll
    for (int i = 0; i < RB_WPT; i++) wr[i] = wsrc[i * wstride + c * RB_Q];
    xr = xsrc[c * RB_Q];
}

__device__ __forceinline__ void rb_store(const rb_f4 (&wr)[RB_WPT], const rb_f4 &xr, RbShared &sh, int b, int q,
                                         int r0) {
    constexpr int RPP = RB_THREADS / RB_Q;
#pragma unroll
    for (int i = 0; i < RB_WPT; i++) sh.wb[b][q][(r0 + RPP * i) ^ (q & 7)] = wr[i];
    sh.xb[b][r0][q] = xr;
}

// One row of x to fp16 by one wave, scaled by the power of two that puts
// its max |value| in [2^14, 2^15); xinv = the inverse scale.  The same
// arithmetic as the prefill's k_rows_f16.  H a multiple of 256, <= 8192.
__device__ __forceinline__ void rb_row_f16(const float *__restrict__ x, int H, _Float16 *__restrict__ o,
                                           float *__restrict__ inv) {
    const int lane = threadIdx.x & 63;
    const rb_f4 *r = reinterpret_cast<const rb_f4 *>(x);
    rb_f4 v[32];   // H / 256 float4 per lane
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        if (256 * i < H) {   // uniform
            v[i] = r[lane + 64 * i];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        }
    }
    mx = wave_max(mx);
    int e = 0;
    frexpf(mx, &e);
    int sh = mx > 0.f ? 15 - e : 0;
    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
    const float sc = ldexpf(1.f, sh);
    uint2 *out = reinterpret_cast<uint2 *>(o);
#pragma unroll
    for (int i = 0; i < 32; i++) {
        if (256 * i < H) {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            const h2 a = {(_Float16)(v[i].x * sc), (_Float16)(v[i].y * sc)};
            const h2 b = {(_Float16)(v[i].z * sc), (_Float16)(v[i].w * sc)};
            out[lane + 64 * i] = make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
        }
    }
    if (lane == 0) *inv = ldexpf(1.f, -sh);
}

// With x16 set, the grid has one more row of workgroups (blockIdx.y ==
// gridDim.y - 1) that write the tokens' fp16 rows for the prefill GEMMs
// (one wave per token) instead of logits.
__global__ __launch_bounds__(RB_THREADS) void k_router_batch(const float *__restrict__ xn, const float *__restrict__ Wr,
                                                             const float *__restrict__ bias, int T, int H, int E,
                                                             float *__restrict__ logits, _Float16 *__restrict__ x16,
                                                             float *__restrict__ xinv) {
    if (x16 && blockIdx.y == gridDim.y - 1) {   // uniform
        const int t = blockIdx.x * RB_TOK + (int)(threadIdx.x >> 6);
        if (t < T) rb_row_f16(xn + (long long)t * H, H, x16 + (long long)t * H, xinv + t);
        return;
    }
    extern __shared__ rb_f4 rb_lds[];
    RbShared &sh = *reinterpret_cast<RbShared *>(rb_lds);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int e0 = blockIdx.y * 64, t0 = blockIdx.x * RB_TOK;
    // thread tid loads float4 q = tid % RB_Q of W rows e0 + tid / RB_Q + RPP*i
    // (E is a multiple of 64, so all exist) and of x row t0 + tid / RB_Q
    // (tokens >= T read the last token instead; their results are never
    // stored), so every load is unconditional and addresses are one base plus
    // uniform strides
    constexpr int RPP = RB_THREADS / RB_Q;   // rows per pass (= RB_TOK)
    const int q = tid % RB_Q, r0 = tid / RB_Q;
    const rb_f4 *wsrc = reinterpret_cast<const rb_f4 *>(Wr + (long long)(e0 + r0) * H) + q;
    const long long wstride = (long long)RPP * H / 4;   // float4 between this thread's rows
    const rb_f4 *xsrc = reinterpret_cast<const rb_f4 *>(xn + (long long)(t0 + r0 < T ? t0 + r0 : T - 1) * H) + q;
    rb_f4 wr[RB_WPT], xr;
    const int NC = H / RB_KC;
    rb_load(wr, xr, wsrc, wstride, xsrc, 0);
    rb_store(wr, xr, sh, 0, q, r0);
    __syncthreads();
    float acc = 0.f;
    for (int c = 0; c < NC; c++) {
        const int b = c & 1;
        if (c + 1 < NC) rb_load(wr, xr, wsrc, wstride, xsrc, c + 1);
        acc = rb_chunk(sh, b, lane, wave, acc);
        if (c + 1 < NC) rb_store(wr, xr, sh, b ^ 1, q, r0);
        __syncthreads();
    }
    const int t = t0 + wave, e = e0 + lane;
    if (t < T && e < E) {
        if (bias) acc = acc + bias[e];
        logits[(long long)t * E + e] = acc;
    }
}

// ---------------------------------------------------------------------------
// Batch router, tiled (T >= 32): a workgroup of 4 waves owns 16 tokens x 16
// experts; wave w takes tokens 8*(w&1).. and experts 8*(w>>1).., and each
// quad of lanes (quad 4a + b of the wave) the 2 x 2 block of tokens 2a, 2a+1
// and experts 2b, 2b+1: acc = fl(acc + fl(w*x)) over k ascending, one chain
// per lane (one wave per SIMD at T = 512, E = 128).  Each lane reads ONE
// operand from LDS, 4 k at a time (ds_read_b128): lanes 0, 1 of the quad the
// x rows of tokens 2a, 2a+1, lanes 2, 3 the W rows of experts 2b, 2b+1; the
// chains are (t0,e0), (t1,e1), (t1,e0), (t0,e1), so each lane's other
// operand is one quad partner's value (DPP quad_perm [2,3,1,0], free as an
// operand modifier).  Half the LDS reads of two operands per lane, which is
// what bounded the kernel (the product is fl(x*w) = fl(w*x)).  Each chunk of
// 256 k of the 16 token and
// 16 expert rows (32 KB) is loaded with coalesced 16-byte loads while the
// previous chunk is summed.  Requires H % 256 == 0, E % 16 == 0.
// grid = (ceil(T/16), E/16 (+1 row of fp16-conversion workgroups)).
// ---------------------------------------------------------------------------
constexpr int RTL_T = 16, RTL_E = 16, RTL_KC = 256;
constexpr int RTL_ROW = RTL_KC + 4;   // floats per LDS row: consecutive rows 4 banks apart
constexpr int RTL_THREADS = 256;
constexpr int RTL_LPT = RTL_KC / 4 / 16;   // float4 of each tile row a loader thread moves per chunk
constexpr int RTL_PARTNER = 2 | 3 << 2 | 1 << 4 | 0 << 6;   // DPP quad_perm [2,3,1,0]
struct RtlShared {
    rb_f4 x[2][RTL_T][RTL_ROW / 4];
    rb_f4 w[2][RTL_E][RTL_ROW / 4];
};

__global__ __launch_bounds__(RTL_THREADS) void k_router_tile(const float *__restrict__ xn, const float *__restrict__ Wr,
                                                             const float *__restrict__ bias, int T, int H, int E,
                                                             float *__restrict__ logits, _Float16 *__restrict__ x16,
                                                             float *__restrict__ xinv) {
    if (x16 && blockIdx.y == gridDim.y - 1) {   // uniform: the fp16 rows of this workgroup's 16 tokens
        for (int i = (int)(threadIdx.x >> 6); i < RTL_T; i += RTL_THREADS / 64) {
            const int t = blockIdx.x * RTL_T + i;
            if (t < T) rb_row_f16(xn + (long long)t * H, H, x16 + (long long)t * H, xinv + t);
        }
        return;
    }
    extern __shared__ rb_f4 rtl_lds[];
    RtlShared &sh = *reinterpret_cast<RtlShared *>(rtl_lds);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * RTL_T, e0 = blockIdx.y * RTL_E;
    // loader role: row r = tid / 16 of the x tile and of the W tile, float4
    // q = tid % 16 + 16 i of the chunk (tokens >= T read the last token; never
    // stored).  A chunk (256 k, 32 rows, 32 KB) is loaded two chunks ahead
    // of its use (below).
    const int lr = tid >> 4, lq = tid & 15;
    const rb_f4 *xsrc = reinterpret_cast<const rb_f4 *>(xn + (long long)(t0 + lr < T ? t0 + lr : T - 1) * H) + lq;
    const rb_f4 *wsrc = reinterpret_cast<const rb_f4 *>(Wr + (long long)(e0 + lr) * H) + lq;
    // chain role: quad qd = 4a + b, lane i of the quad (see above)
    const int qd = lane >> 2, qi = lane & 3;
    const int qt0 = 8 * (wave & 1) + 2 * (qd >> 2), qe0 = 8 * (wave >> 1) + 2 * (qd & 3);
    const int tl = qt0 + ((qi == 1 || qi == 2) ? 1 : 0), el = qe0 + (qi & 1);
    const int NC = H / RTL_KC;
    // chunk j's global loads go to register set j % 2, two chunks ahead of
    // its use: chunk c + 2 is loaded while chunk c is summed, and stored to
    // LDS after chunk c + 1 is (its latency covers two chunks' chains)
    struct Regs {
        rb_f4 x[RTL_LPT], w[RTL_LPT];
    };
    auto gload = [&](Regs &r, int c) {   // unconditional: chunks past the end reload the last
        c = c < NC ? c : NC - 1;
#pragma unroll
        for (int i = 0; i < RTL_LPT; i++) {
            r.x[i] = xsrc[c * (RTL_KC / 4) + 16 * i];
            r.w[i] = wsrc[c * (RTL_KC / 4) + 16 * i];
        }
    };
    auto lstore = [&](const Regs &r, int buf) {
#pragma unroll
        for (int i = 0; i < RTL_LPT; i++) {
            sh.x[buf][lr][lq + 16 * i] = r.x[i];
            sh.w[buf][lr][lq + 16 * i] = r.w[i];
        }
    };
    float acc = 0.f;
    // the chain over chunk c from LDS buffer c % 2: 16 k per group, the next
    // group's LDS reads issued before the current group's arithmetic (two
    // register slots); the empty asm statements (tied to acc) keep the
    // compiler from hoisting more of the chunk's reads, which would need
    // more registers than one wave has.  This lane's operand row: x of token
    // qt0 + qi (qi < 2) or W of expert qe0 + qi - 2.
    auto chain = [&](int c) {
        const int b = c & 1;
        const rb_f4 *own = qi < 2 ? &sh.x[b][qt0 + qi][0] : &sh.w[b][qe0 + qi - 2][0];
        rb_f4 va[4], vb[4];
        auto ld = [&](int g, rb_f4 (&v)[4]) {
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = own[4 * g + q];
        };
        auto sum = [&](const rb_f4 (&v)[4]) {
            float p[16];
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int j = 0; j < 4; j++) p[4 * q + j] = dpp_f32<RTL_PARTNER>(v[q][j]) * v[q][j];
#pragma unroll
            for (int i = 0; i < 16; i++) acc = acc + p[i];
            asm volatile("" : "+v"(acc));
        };
        ld(0, va);
#pragma unroll 1
        for (int g = 0; g < RTL_KC / 16; g += 2) {
            ld(g + 1, vb);
            sum(va);
            if (g + 2 < RTL_KC / 16) ld(g + 2, va);
            sum(vb);
        }
    };
    Regs ra, rb;
    gload(ra, 0);
    gload(rb, 1);
    lstore(ra, 0);
    __syncthreads();
    for (int c = 0; c < NC; c += 2) {
        gload(ra, c + 2);
        chain(c);
        if (c + 1 < NC) lstore(rb, (c + 1) & 1);
        __syncthreads();
        if (c + 1 < NC) {   // uniform
            gload(rb, c + 3);
            chain(c + 1);
            if (c + 2 < NC) lstore(ra, c & 1);
            __syncthreads();
        }
    }
    const int t = t0 + tl, e = e0 + el;
    if (t < T) {
        if (bias) acc = acc + bias[e];
        logits[(long long)t * E + e] = acc;
    }
}

template <int NJ>
static hipError_t launch_topk_t(const float *logits, int T, int E, int top_k, int *sel_idx, float *sel_w, hipStream_t st) {
    hipLaunchKernelGGL((k_topk<NJ>), dim3(T), dim3(64), 0, st, logits, E, top_k, sel_idx, sel_w);
    return hipGetLastError();
}

static hipError_t launch_topk(const float *logits, int T, int E, int top_k, int *sel_idx, float *sel_w, hipStream_t st) {
    if (E <= 64) return launch_topk_t<1>(logits, T, E, top_k, sel_idx, sel_w, st);
    if (E <= 128) return launch_topk_t<2>(logits, T, E, top_k, sel_idx, sel_w, st);
    return launch_topk_t<4>(logits, T, E, top_k, sel_idx, sel_w, st);
}

template <int M, int NJ>
static hipError_t launch_router_dpp_t(const float *xn, const float *router, const float *bias, int T, int E, int top_k,
                                      float *logits, unsigned *counters, int *sel_idx, float *sel_w, hipStream_t st,
                                      int k, int *grp) {
    // expert groups along x: workgroup i runs on XCD i % 8, so each XCD's L2
    // holds one eighth of the router rows for every token of the batch
    // (tokens along x would make every XCD read all of them)
    dim3 grid((E + 3) / 4, T);
    hipLaunchKernelGGL((k_router_dpp<M, NJ>), grid, dim3(64), 0, st, xn, router, bias, E, top_k, logits, counters,
                       sel_idx, sel_w, k, grp);
    return hipGetLastError();
}

template <int M>
static hipError_t launch_router_dpp(const float *xn, const float *router, const float *bias, int T, int E, int top_k,
                                    float *logits, unsigned *counters, int *sel_idx, float *sel_w, hipStream_t st,
                                    int k, int *grp) {
    if (E <= 64)
        return launch_router_dpp_t<M, 1>(xn, router, bias, T, E, top_k, logits, counters, sel_idx, sel_w, st, k, grp);
    if (E <= 128)
        return launch_router_dpp_t<M, 2>(xn, router, bias, T, E, top_k, logits, counters, sel_idx, sel_w, st, k, grp);
    return launch_router_dpp_t<M, 4>(xn, router, bias, T, E, top_k, logits, counters, sel_idx, sel_w, st, k, grp);
}

// Router: logits then softmax/top-k.  With a counter buffer (T unsigned,
// zero on entry, left zero on exit) and H in {512, 1024, 2048} the DPP
// kernel does both in one launch; otherwise an LDS-tiled logits kernel and
// a top-k kernel.  hipErrorNotSupported when H does not fit either tiling.
hipError_t launch_router(const float *xn, const float *router, const float *bias, int T, int H, int E, int top_k,
                         float *logits, unsigned *counters, int *sel_idx, float *sel_w, hipStream_t st,
                         _Float16 *x16, float *xinv, bool *x16_done, const MoeArgs *group, bool *grouped) {
    if (x16_done) *x16_done = false;
    if (grouped) *grouped = false;
    if (counters && T < 32 && (H == 2048 || H == 1024 || H == 512)) {
        // the batch grouping in the same launch, when the batch runs in expert order
        const bool g = group && moe_decode_grouped(*group);
        int *grp = g ? group->grp : nullptr;
        const int k = g ? group->k : 0;
        hipError_t err;
        if (H == 2048)
            err = launch_router_dpp<32>(xn, router, bias, T, E, top_k, logits, counters, sel_idx, sel_w, st, k, grp);
        else if (H == 1024)
            err = launch_router_dpp<16>(xn, router, bias, T, E, top_k, logits, counters, sel_idx, sel_w, st, k, grp);
        else
            err = launch_router_dpp<8>(xn, router, bias, T, E, top_k, logits, counters, sel_idx, sel_w, st, k, grp);
        if (err == hipSuccess && grouped) *grouped = g;
        return err;
    }
    const size_t lds = (size_t)H * 4 + 2 * RT_TILE_FLOATS * 4;
    if (T >= 32 && H % RTL_KC == 0 && E % RTL_E == 0) {
        const bool rows = x16 && xinv && H <= 8192;
        hipLaunchKernelGGL(k_router_tile, dim3((T + RTL_T - 1) / RTL_T, E / RTL_E + (rows ? 1 : 0)),
                           dim3(RTL_THREADS), sizeof(RtlShared), st, xn, router, bias, T, H, E, logits,
                           rows ? x16 : nullptr, xinv);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        if (x16_done) *x16_done = rows;
        return launch_topk(logits, T, E, top_k, sel_idx, sel_w, st);
    }
    if (T >= 32 && H % RB_KC == 0 && E % 64 == 0) {
        const bool rows = x16 && xinv && H <= 8192;
        hipLaunchKernelGGL(k_router_batch, dim3((T + RB_TOK - 1) / RB_TOK, (E + 63) / 64 + (rows ? 1 : 0)),
                           dim3(RB_THREADS), sizeof(RbShared), st, xn, router, bias, T, H, E, logits,
                           rows ? x16 : nullptr, xinv);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        if (x16_done) *x16_done = rows;
        return launch_topk(logits, T, E, top_k, sel_idx, sel_w, st);
    }
    if (H > 8192) return hipErrorNotSupported;
    if (T < 8 && (H == 1024 || H == 2048 || H == 4096)) {
        dim3 grid(T, (E + EPB_S - 1) / EPB_S);
        const size_t plds = (size_t)EPB_S * H * 4;
        if (H == 1024)
            hipLaunchKernelGGL((k_router_logits_small<16>), grid, dim3(RS_THREADS), plds, st, xn, router, bias, H, E, logits);
        else if (H == 2048)
            hipLaunchKernelGGL((k_router_logits_small<32>), grid, dim3(RS_THREADS), plds, st, xn, router, bias, H, E, logits);
        else
            hipLaunchKernelGGL((k_router_logits_small<64>), grid, dim3(RS_THREADS), plds, st, xn, router, bias, H, E, logits);
    } else if (T < 8 && H % 256 == 0) {
        constexpr int EPB = 16;
        dim3 grid(T, (E + EPB - 1) / EPB);
        hipLaunchKernelGGL((k_router_logits<EPB>), grid, dim3(RT_THREADS), lds, st, xn, router, bias, H, E, logits);
    } else if (H % 64 == 0) {
        constexpr int EPB = 64;
        dim3 grid(T, (E + EPB - 1) / EPB);
        hipLaunchKernelGGL((k_router_logits<EPB>), grid, dim3(RT_THREADS), lds, st, xn, router, bias, H, E, logits);
    } else {
        return hipErrorNotSupported;
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_topk(logits, T, E, top_k, sel_idx, sel_w, st);
}

// Batches of at least this many tokens run in expert order.
#ifndef TBQ_GRP_MIN_T
#define TBQ_GRP_MIN_T 8
#endif
#ifndef TBQ_GU_ROWS_B
#define TBQ_GU_ROWS_B 4
#endif

// Whether a decode batch runs in expert order (k_group's pair list).
bool moe_decode_grouped(const MoeArgs &a) {
    const int pairs = a.T * a.k;
    return a.T >= TBQ_GRP_MIN_T && pairs <= 256 && a.T <= 32 && a.E <= 256 && a.H % DG_ROWS == 0 && a.grp;
}

hipError_t launch_group(const MoeArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(k_group, dim3(1), dim3(256), 0, st, a.sel_idx, a.T, a.E, a.k, a.grp);
    return hipGetLastError();
}

template <int UPL, bool GG>
static hipError_t launch_gate_up_q4k_t(const MoeArgs &a, bool grouped, hipStream_t st) {
    const int pairs = a.T * a.k;
    const int *order = grouped ? a.grp + 1 + 3 * a.E : nullptr, *nvalid = grouped ? order + pairs : nullptr;
    // batches: more rows per workgroup, fewer workgroups
    const int rows = grouped ? TBQ_GU_ROWS_B : GU_ROWS;
    const int nwv = rows == GU_ROWS ? TBQ_GU_WAVES : TBQ_GU_WAVES_B;
    const int out_per_wg = nwv * rows;
    dim3 grid((a.F + out_per_wg - 1) / out_per_wg, pairs);
    size_t lds = (size_t)(a.H / 32) * XD_PER_SB * 4;
    if (rows == GU_ROWS)
        hipLaunchKernelGGL((k_gate_up_q4k<UPL, GG>), grid, dim3(GU_THREADS), lds, st, (const uint8_t *)a.gate,
                           (const uint8_t *)a.up, a.xn, a.sel_idx, order, nvalid, a.H, a.F, a.E, a.k, a.act);
    else
        hipLaunchKernelGGL((k_gate_up_q4k<UPL, GG, TBQ_GU_ROWS_B, TBQ_GU_WAVES_B>), grid, dim3(64 * TBQ_GU_WAVES_B), lds, st,
                           (const uint8_t *)a.gate, (const uint8_t *)a.up, a.xn, a.sel_idx, order, nvalid, a.H,
                           a.F, a.E, a.k, a.act);
    return hipGetLastError();
}

template <int UPL, bool GG>
static hipError_t launch_down_q4k_t(const MoeArgs &a, bool grouped, hipStream_t st) {
    const int pairs = a.T * a.k;
    if (grouped) {
        const int *order = a.grp + 1 + 3 * a.E, *nvalid = order + pairs;
        // one pair's rows per workgroup, pairs in expert order; k_combine
        // then adds each token's slots in slot order
        hipLaunchKernelGGL((k_down_pair_q4k<UPL, GG>), dim3(a.H / DG_ROWS, pairs), dim3(DG_THREADS),
                           (size_t)(a.F / 32) * XD_PER_SB * 4, st, (const uint8_t *)a.down, a.act, a.sel_idx, order,
                           nvalid, a.H, a.F, a.E, a.k, a.y);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        return launch_combine(a, st);
    }
    dim3 grid(a.H / DC_ROWS, a.T);
    size_t lds = (size_t)a.k * (a.F / 32) * XD_PER_SB * 4;
    hipLaunchKernelGGL((k_down_combine_q4k<UPL, GG>), grid, dim3(DC_THREADS), lds, st, (const uint8_t *)a.down, a.act,
                       a.sel_idx, a.sel_w, a.resid, a.H, a.F, a.E, a.k, a.out);
    return hipGetLastError();
}

// gate/up + SwiGLU with Q4_K gate and up (a.qg == a.qu, the reference's
// layout or ggml's); hipErrorNotSupported for H > 4096.
hipError_t launch_moe_q4k_gate_up(const MoeArgs &a, bool grouped, hipStream_t st) {
    const int ugu = (a.H / 64 + 31) / 32;
    if (ugu > 2) return hipErrorNotSupported;
    const bool gg = a.qg == QT_GQ4_K;
    if (ugu == 1) return gg ? launch_gate_up_q4k_t<1, true>(a, grouped, st) : launch_gate_up_q4k_t<1, false>(a, grouped, st);
    return gg ? launch_gate_up_q4k_t<2, true>(a, grouped, st) : launch_gate_up_q4k_t<2, false>(a, grouped, st);
}

// down + slot-ordered combine + residual with a Q4_K down tensor;
// hipErrorNotSupported for F > 2048.
hipError_t launch_moe_q4k_down(const MoeArgs &a, bool grouped, hipStream_t st) {
    const int udc = (a.F / 64 + 15) / 16;
    if (udc > 2) return hipErrorNotSupported;
    const bool gg = a.qd == QT_GQ4_K;
    if (udc == 1) return gg ? launch_down_q4k_t<1, true>(a, grouped, st) : launch_down_q4k_t<1, false>(a, grouped, st);
    return gg ? launch_down_q4k_t<2, true>(a, grouped, st) : launch_down_q4k_t<2, false>(a, grouped, st);
}

}  // namespace tbq
