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

template <int NJ>
__device__ __forceinline__ void topk_wave(const float *lg, int E, int top_k, int t, float *P,
                                          int *__restrict__ sel_idx, float *__restrict__ sel_w) {
    const int lane = threadIdx.x & 63;
    const float NEG = -__builtin_huge_valf();
    float v[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? __builtin_nontemporal_load(lg + e) : NEG;
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
    // Slot scan: lane i < k holds slot i (value ws, expert wi); lanes k..7
    // hold +inf so they never count as the minimum.  wl is the current
    // minimum over the k slots, which never decreases, and ms the first slot
    // holding it.  Expert e enters iff pr[e] > wl at its turn (a float
    // compare, so a NaN never enters): candidates are taken in expert order
    // from a ballot that is re-filtered against the new minimum after every
    // entry, so only entries cost a sequential step.
    const int k = top_k > 8 ? 8 : top_k;
    float ws = lane < k ? -1e30f : __builtin_huge_valf();
    int wi = 0;
    float wl = -1e30f;
    int ms = 0;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const bool valid = lane + 64 * j < E;
        unsigned long long cand = __ballot(valid && pr[j] > wl);
        while (cand) {
            const int l = __builtin_ctzll(cand);
            const float val = rdlane(pr[j], l);
            if (lane == ms) {
                ws = val;
                wi = 64 * j + l;
            }
            wl = rdlane(group8_min(ws), 0);
            ms = __builtin_ctzll(__ballot(lane < 8 && ws == wl));
            cand &= cand - 1;
            cand &= __ballot(valid && pr[j] > wl);
        }
    }
    float wsum = 0.f;
    for (int i = 0; i < k; i++) wsum = wsum + rdlane(ws, i);
    if (lane < 8) {
        float wo = 0.f;
        int io = -1;
        if (lane < k) {
            wo = wsum > 0.f ? ws / wsum : ws;
            io = wi;
        }
        sel_idx[t * 8 + lane] = io;
        sel_w[t * 8 + lane] = wo;
    }
}

}  // namespace tbq
