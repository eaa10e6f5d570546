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
// min of two wave-uniform ints as one scalar instruction (left to itself the
// compiler moves such mins to the vector unit and back, a round trip of
// latency on every step of the slot scan)
__device__ __forceinline__ int topk_smin(int a, int b) {
    int r;
    asm("s_min_i32 %0, %1, %2" : "=s"(r) : "s"(a), "s"(b) : "scc");
    return r;
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
    // Slot scan.  Values compare as ordered integer keys (key() below: a
    // float's order for all non-NaN values; a NaN gets the lowest key, so it
    // never enters, as the reference's float compare never lets it), so the
    // eight slots live in scalar registers and an entry costs scalar
    // instructions only.  wl is the current minimum over the k slots (slots
    // k..7 hold the largest key and never count), which never decreases, and
    // ms the first slot holding it.  Expert e enters iff key(pr[e]) > wl at
    // its turn: candidates are taken in expert order from a ballot that is
    // re-filtered against the new minimum after every entry, so only entries
    // cost a sequential step.
    const int k = top_k > 8 ? 8 : top_k;
    constexpr int KMIN = (int)0x80000000;
    int kx[NJ];   // lanes past E get the lowest key: never a candidate
#pragma unroll
    for (int j = 0; j < NJ; j++) kx[j] = lane + 64 * j < E ? topk_key(pr[j]) : KMIN;
    int sk[8], si[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        sk[s] = s < k ? topk_key(-1e30f) : 0x7FFFFFFF;
        si[s] = 0;
    }
    int wl = topk_key(-1e30f), ms = 0;
    // min over the slots and the first slot holding it, in scalar registers
    auto slot_min = [&]() {
        int m = sk[0];
#pragma unroll
        for (int s = 1; s < 8; s++) m = topk_smin(m, sk[s]);
        wl = m;
        int f = 7;
#pragma unroll
        for (int s = 6; s >= 0; s--) f = sk[s] == m ? s : f;
        ms = f;
    };
    // While slots are empty every probability (>= +0) beats the -1e30 they
    // hold, so experts 0..k-1 fill slots 0..k-1 unless one of them is NaN
    // (which never enters); then the scan starts at expert k.
    unsigned long long skip = 0;
    if (E >= k && !__ballot(lane < k && kx[0] == KMIN)) {
#pragma unroll
        for (int s = 0; s < 8; s++) {
            if (s < k) {
                sk[s] = __builtin_amdgcn_readlane(kx[0], s);
                si[s] = s;
            }
        }
        slot_min();
        skip = (1ull << k) - 1;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        unsigned long long cand = __ballot(kx[j] > wl) & ~(j == 0 ? skip : 0ull);
        while (cand) {
            const int l = __builtin_ctzll(cand);
            const int val = __builtin_amdgcn_readlane(kx[j], l);
#pragma unroll
            for (int s = 0; s < 8; s++) {
                sk[s] = s == ms ? val : sk[s];
                si[s] = s == ms ? 64 * j + l : si[s];
            }
            slot_min();
            cand &= cand - 1;
            cand &= __ballot(kx[j] > wl);
        }
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
        sel_idx[t * 8 + lane] = io;
        sel_w[t * 8 + lane] = wo;
    }
}

}  // namespace tbq
