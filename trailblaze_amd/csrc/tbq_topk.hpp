// tbq_topk.hpp -- softmax + top-k + renormalise of the MoE router for one
// token, by one wave, bit-exact to tb_route_experts (layer4/tb_infer.c:
// 351-374) given the reference's logits.
#pragma once

#include "tbq_device.hpp"

namespace tbq {

// ---------------------------------------------------------------------------
// Softmax + top-k + renormalise for one token, by one wave (lane l holds
// experts l + 64j, j < NJ).  lg points at the token's E logits.
// Bit-exact to tb_route_experts (layer4/tb_infer.c:351-374): max, expf of
// (s - max), sequential sum, division, then the slot scan that replaces the
// first slot holding the minimum when a score is strictly larger, and the
// sequential renormalisation over the k slots.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float rdlane(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Ordered integer key of a float: key(a) < key(b) iff a < b for non-NaN a, b
// (with -0 just below +0, which never matters here: probabilities are +0 or
// positive); NaN maps to the lowest key.  topk_unkey inverts it.
__device__ __forceinline__ int topk_key(float f) {
    const int b = __builtin_bit_cast(int, f);
    return f != f ? (int)0x80000000 : b ^ ((b >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float topk_unkey(int k) { return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7FFFFFFF)); }
// DEV: the logits may have been stored by other workgroups of the same
// kernel, and the selection may be read by them: device-scope loads and
// stores; otherwise (logits from an earlier kernel) plain ones.
template <int NJ, bool DEV = true>
__device__ __forceinline__ void topk_wave(const float *lg, int E, int top_k, int t, float *P,
                                          int *__restrict__ sel_idx, float *__restrict__ sel_w) {
    const int lane = threadIdx.x & 63;
    const float NEG = -__builtin_huge_valf();
    float v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? (DEV ? __hip_atomic_load(lg + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : lg[e]) : NEG;
    }
    float m = v[0];
#pragma unroll
    for (int j = 1; j < NJ; j++) m = fmaxf(m, v[j]);
    const float mx = wave_max(m);   // same value the reference's strict '>' scan keeps
    float ex[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int e = lane + 64 * j;
        ex[j] = e < E ? expf_glibc(v[j] - mx) : 0.f;
        P[e] = ex[j];
    }
    if (lane < 16) P[64 * NJ + lane] = 0.f;
    __syncthreads();
    // sequential sum in expert order, by every lane from broadcast LDS reads;
    // P is zero beyond E and adding +0 to the (non-negative) running sum is
    // exact, so whole 32-blocks are added
    float ssum = 0.f;
    {
        const float4 *P4 = reinterpret_cast<const float4 *>(P);
        float4 q[2][8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[0][i] = P4[i];
#pragma unroll
        for (int b = 0; b < 2 * NJ; b++) {
            if (32 * b >= E) break;
            if (b + 1 < 2 * NJ && 32 * (b + 1) < E) {
#pragma unroll
                for (int i = 0; i < 8; i++) q[(b + 1) & 1][i] = P4[8 * (b + 1) + i];
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 c = q[b & 1][i];
                ssum = ssum + c.x;
                ssum = ssum + c.y;
                ssum = ssum + c.z;
                ssum = ssum + c.w;
            }
        }
    }
    float pr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) pr[j] = lane + 64 * j < E ? ex[j] / ssum : 0.f;
    // Slot scan.  Values compare as ordered integer keys (topk_key: a
    // float's order for all non-NaN values; a NaN gets the lowest key, so it
    // never enters, as the reference's float compare never lets it).  The
    // eight slots live in lanes 0..7 of vk (key) and vi (expert); slots k..7
    // and lanes past 7 hold the largest key and never count.  wl is the
    // current minimum over the slots (a DPP min over the 8 lanes), which never
    // decreases, and ms the first slot holding it (lowest set bit of a
    // ballot).  Expert e enters iff key(pr[e]) > wl at its turn: candidates
    // are taken in expert order from a ballot that is re-filtered against the
    // new minimum after every entry, so only entries cost a sequential step,
    // and an entry is a handful of instructions.
    const int k = top_k > 8 ? 8 : top_k;
    constexpr int KMIN = (int)0x80000000, KMAX = 0x7FFFFFFF;
    int kx[NJ];   // lanes past E get the lowest key: never a candidate
#pragma unroll
    for (int j = 0; j < NJ; j++) kx[j] = lane + 64 * j < E ? topk_key(pr[j]) : KMIN;
    int vk = lane < k ? topk_key(-1e30f) : KMAX, vi = 0;
    int wl = topk_key(-1e30f), ms = 0;
    auto slot_min = [&]() {
        int m = vk;
        m = min(m, __builtin_amdgcn_mov_dpp(m, DPP_QXOR1, 0xF, 0xF, false));
        m = min(m, __builtin_amdgcn_mov_dpp(m, DPP_QXOR2, 0xF, 0xF, false));
        m = min(m, __builtin_amdgcn_mov_dpp(m, DPP_HALF_MIRROR, 0xF, 0xF, false));
        wl = __builtin_amdgcn_readfirstlane(m);
        ms = __builtin_ctzll(__ballot(vk == wl));
    };
    // While slots are empty every probability (>= +0) beats the -1e30 they
    // hold, so experts 0..k-1 fill slots 0..k-1 unless one of them is NaN
    // (which never enters); then the scan starts at expert k.
    unsigned long long skip = 0;
    if (E >= k && !__ballot(lane < k && kx[0] == KMIN)) {
        vk = lane < k ? kx[0] : KMAX;
        vi = lane;
        slot_min();
        skip = (1ull << k) - 1;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        unsigned long long cand = __ballot(kx[j] > wl) & ~(j == 0 ? skip : 0ull);
        while (cand) {
            const int l = __builtin_ctzll(cand);
            const int val = __builtin_amdgcn_readlane(kx[j], l);
            vk = lane == ms ? val : vk;
            vi = lane == ms ? 64 * j + l : vi;
            slot_min();
            cand &= cand - 1;
            cand &= __ballot(kx[j] > wl);
        }
    }
    int sk[8], si[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        sk[s] = __builtin_amdgcn_readlane(vk, s);
        si[s] = __builtin_amdgcn_readlane(vi, s);
    }
    // renormalise over the k slots in slot order (sequential fp32 sum)
    float wsum = 0.f;
#pragma unroll
    for (int s = 0; s < 8; s++)
        if (s < k) wsum = wsum + topk_unkey(sk[s]);
    if (lane < 8) {
        int io = -1, ks = 0;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            io = lane == s ? si[s] : io;
            ks = lane == s ? sk[s] : ks;
        }
        float wo = 0.f;
        if (lane < k) {
            const float ws = topk_unkey(ks);
            wo = wsum > 0.f ? ws / wsum : ws;
        } else {
            io = -1;
        }
        // device-scope stores with DEV: a workgroup on another XCD may read
        // the selection within the same kernel (the batch grouping of the
        // DPP router)
        if (DEV) {
            __hip_atomic_store(sel_idx + t * 8 + lane, io, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(sel_w + t * 8 + lane, wo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            sel_idx[t * 8 + lane] = io;
            sel_w[t * 8 + lane] = wo;
        }
    }
}

}  // namespace tbq
