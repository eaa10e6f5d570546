// tbq_q4k.hpp -- Q4_K building blocks shared by the decode matvec and the
// MoE expert kernels: x staged as 24-bit integer digits in LDS, and the
// v_dot4 evaluation of one 64-weight unit (two sub-blocks) of a Q4_K row.
//
// x is re-expressed per 32-element sub-block g as X_i = rint(x_i * 2^s_g)
// with |X_i| <= 2^22, whose bytes are three digits X = 65536*h + 256*m + l
// (h signed, m and l unsigned).  A Q4_K sub-block's dot product is then
//     sum_i q_i x_i  ~=  2^-s_g * (65536*sum q h + 256*sum q m + sum q l)
// where every inner sum is an exact v_dot4 chain (4 nibbles x 4 digits per
// instruction), so a weight costs ~1.7 VALU ops instead of ~3 for
// byte->float conversion + fma.  The per-group scale and min are applied
// afterwards in fp32: S_g * (sum q x) - M_g * (sum x).  Rounding differs from
// the reference's sequential fp32 sum by ~1e-7 relative (x quantised to 22+
// significant bits per sub-block), far inside the 1e-5 parity bound.
#pragma once

#include "tbq_kquant.hpp"

namespace tbq {

constexpr int XD_STRIDE = 28;   // dwords of LDS per 32-element sub-block

// Stage the digits of x (K elements) into LDS; all NT threads of the
// workgroup participate.
// Thread t handles 8 elements (group o = t%4 of sub-block g = t/4).  With
// s_g from the sub-block's max |x|, X = rint(x * 2^s_g) fits 24 bits and its
// little-endian bytes are the digits: l = byte0 and m = byte1 unsigned,
// h = byte2 signed, X = 65536*h + 256*m + l.  Per 8-element group six dwords
// are stored: {h, m, l} x {even elements (low nibbles), odd (high nibbles)}.
// nvec > 1 stages nvec consecutive vectors of K elements (vector v's
// sub-block g lands at sub-block v*K/32 + g), all threads sharing the work.
template <int NT>
__device__ __forceinline__ void stage_x_digits_nibble(const float *__restrict__ x, int K, uint32_t *xd,
                                                      int nvec = 1) {
    const int G = K / 32;
    for (int t = threadIdx.x; t < 4 * G * nvec; t += NT) {
        const int g = t >> 2, o = t & 3;   // g indexes sub-blocks across all vectors
        const float4 *xp = reinterpret_cast<const float4 *>(x + 32 * g + 8 * o);
        const float4 a = xp[0], b = xp[1];
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float mx = 0.f, sm = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            mx = fmaxf(mx, fabsf(v[i]));
            sm += v[i];
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        sm += __shfl_xor(sm, 1);
        sm += __shfl_xor(sm, 2);
        int e = 0;
        frexpf(mx, &e);
        int s = mx > 0.f ? 22 - e : 0;
        s = s > 126 ? 126 : (s < -126 ? -126 : s);
        const float sc = ldexpf(1.f, s);
        uint32_t X[8];
#pragma unroll
        for (int i = 0; i < 8; i++) X[i] = (uint32_t)(int)rintf(v[i] * sc);
        uint32_t dig[6];
#pragma unroll
        for (int par = 0; par < 2; par++) {
            // bytes 0,1 of X[par], X[par+2] and of X[par+4], X[par+6]
            const uint32_t p01 = __builtin_amdgcn_perm(X[par + 2], X[par], 0x05010400u);
            const uint32_t q01 = __builtin_amdgcn_perm(X[par + 6], X[par + 4], 0x05010400u);
            const uint32_t p2 = __builtin_amdgcn_perm(X[par + 2], X[par], 0x07030602u);
            const uint32_t q2 = __builtin_amdgcn_perm(X[par + 6], X[par + 4], 0x07030602u);
            dig[4 + par] = __builtin_amdgcn_perm(q01, p01, 0x05040100u);   // l
            dig[2 + par] = __builtin_amdgcn_perm(q01, p01, 0x07060302u);   // m
            dig[0 + par] = __builtin_amdgcn_perm(q2, p2, 0x05040100u);     // h
        }
        uint32_t *dst = xd + g * XD_STRIDE + o * 6;
        *reinterpret_cast<uint2 *>(dst) = make_uint2(dig[0], dig[1]);
        *reinterpret_cast<uint2 *>(dst + 2) = make_uint2(dig[2], dig[3]);
        *reinterpret_cast<uint2 *>(dst + 4) = make_uint2(dig[4], dig[5]);
        if (o == 0)
            *reinterpret_cast<float2 *>(xd + g * XD_STRIDE + 24) = make_float2(sm, ldexpf(1.f, -s));
    }
}

// sum q*x over one Q4_K sub-block whose 32 nibbles are packed in q (byte i =
// weights 2i, 2i+1), times the sub-block scale S, minus M*sum(x), added to acc.
__device__ __forceinline__ float q4_subblock(uint4 q, const uint32_t *xs, float S, float Mn, float acc) {
    const uint4 *d4 = reinterpret_cast<const uint4 *>(xs);
    uint4 D[6];
#pragma unroll
    for (int i = 0; i < 6; i++) D[i] = d4[i];
    const uint32_t *D32 = reinterpret_cast<const uint32_t *>(D);
    const float2 meta = *reinterpret_cast<const float2 *>(xs + 24);
    const uint32_t qv[4] = {q.x, q.y, q.z, q.w};
    int ah = 0;
    uint32_t am = 0, al = 0;
#pragma unroll
    for (int o = 0; o < 4; o++) {
        const uint32_t lo = qv[o] & 0x0F0F0F0Fu;
        const uint32_t hi = (qv[o] >> 4) & 0x0F0F0F0Fu;
        ah = __builtin_amdgcn_sdot4((int)lo, (int)D32[o * 6 + 0], ah, false);
        ah = __builtin_amdgcn_sdot4((int)hi, (int)D32[o * 6 + 1], ah, false);
        am = __builtin_amdgcn_udot4(lo, D32[o * 6 + 2], am, false);
        am = __builtin_amdgcn_udot4(hi, D32[o * 6 + 3], am, false);
        al = __builtin_amdgcn_udot4(lo, D32[o * 6 + 4], al, false);
        al = __builtin_amdgcn_udot4(hi, D32[o * 6 + 5], al, false);
    }
    const float f = fmaf((float)ah, 65536.f, fmaf((float)am, 256.f, (float)al));
    acc = fmaf(S * meta.y, f, acc);
    return fmaf(-Mn, meta.x, acc);
}

struct Q4KUnit {
    uint4 hdr, q0, q1;
    uint32_t mind;
};

// Unit u of a row: super-block u/4, sub-blocks 2*(u%4) and 2*(u%4)+1.
__device__ __forceinline__ void q4k_load(const uint8_t *row, int u, Q4KUnit &r) {
    const uint8_t *b = row + (size_t)(u >> 2) * 144;
    const int p = u & 3;
    r.hdr = *reinterpret_cast<const uint4 *>(b);
    r.q0 = *reinterpret_cast<const uint4 *>(b + 16 + 32 * p);
    r.q1 = *reinterpret_cast<const uint4 *>(b + 32 + 32 * p);
    r.mind = *reinterpret_cast<const uint32_t *>(b + 16);
}

// Reference scale/min selection (layer4/tb_gguf.c:163-168): sub-block j<4
// takes scale byte 4+j and min byte 8+j; j>=4 takes scale byte 8+j and min
// byte 12+j, i.e. the first four quant bytes.
__device__ __forceinline__ float q4k_unit_dot(const Q4KUnit &r, int u, const uint32_t *xd, float acc) {
    const int p = u & 3;
    const float d = f16_ref(r.hdr.x & 0xFFFFu), dmin = f16_ref(r.hdr.x >> 16);
    const uint32_t sw = p < 2 ? r.hdr.y : r.hdr.w;
    const uint32_t mw = p < 2 ? r.hdr.z : r.mind;
    const int sh = 16 * (p & 1);
    const float S0 = d * (float)((sw >> sh) & 63), S1 = d * (float)((sw >> (sh + 8)) & 63);
    const float M0 = dmin * (float)((mw >> sh) & 63), M1 = dmin * (float)((mw >> (sh + 8)) & 63);
    const uint32_t *xs = xd + (size_t)(2 * u) * XD_STRIDE;
    acc = q4_subblock(r.q0, xs, S0, M0, acc);
    return q4_subblock(r.q1, xs + XD_STRIDE, S1, M1, acc);
}

}  // namespace tbq
