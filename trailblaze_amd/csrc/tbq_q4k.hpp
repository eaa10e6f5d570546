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

#include "tbq_kernels.h"
#include "tbq_kquant.hpp"

namespace tbq {

// LDS layout of the digits, per unit of two sub-blocks (64 elements, 52
// dwords): digits of the even sub-block (24 dwords), digits of the odd one
// (24), then {sum x_even, sum x_odd, 2^-s_even, 2^-s_odd}.  Lanes that own
// consecutive units read at a 52-dword stride, which maps any 8 consecutive
// lanes of a ds_read_b128 onto 8 disjoint 4-bank groups (52 = 20 mod 32).
constexpr int XD_UNIT = 52;
constexpr int XD_PER_SB = XD_UNIT / 2;   // LDS dwords per sub-block on average

// Staging of x into digits, in two phases so that the loads of x can be
// issued before a kernel's weight loads (x then does not queue behind them):
// load() issues the global loads into registers, store() computes and writes
// the digits.  All NT threads of the workgroup take part; each handles
// ceil(4 * G * nvec / NT) <= MAXT tasks of 8 elements (task t: sub-block
// g = t / 4, elements 8 * (t % 4) ..).  nvec > 1 stages nvec consecutive
// vectors of K elements; vector v's sub-block g is staged as sub-block
// v * K / 32 + g, so vector v's digits start at v * (K / 32) * XD_PER_SB.
//
// Per task: s_g from the sub-block's max |x|, X = rint(x * 2^s_g) fits 24
// bits and its little-endian bytes are the digits: l = byte0 and m = byte1
// unsigned, h = byte2 signed, X = 65536*h + 256*m + l.  Six dwords are
// stored: {h, m, l} x {even elements (low nibbles), odd (high nibbles)}.
template <int NT, int MAXT, int PRO = PRO_NONE>
struct XStager {
    float4 v[MAXT][2];
    float4 p1[MAXT][2], p2[MAXT][2];   // PRO_NORM inputs: y, w (PRO_NORMD: w)
    float ss;                          // PRO_NORMD: this thread's sum of x^2

    // Unconditional loads (tasks past the end re-read the last task and are
    // never stored), so no branch makes the compiler wait for every load
    // in flight where it rejoins.
    __device__ __forceinline__ void load(const float *__restrict__ x, int K, int nvec = 1,
                                         const MvPro &pro = MvPro{}) {
        const int ntask = 4 * (K / 32) * nvec;
        const float *yp = (PRO == PRO_NORM && pro.y) ? pro.y : x;   // no y: loads x, adds 0
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const int t = min((int)threadIdx.x + i * NT, ntask - 1);
            const float4 *xp = reinterpret_cast<const float4 *>(x + 8 * t);
            v[i][0] = xp[0];
            v[i][1] = xp[1];
            if constexpr (PRO == PRO_NORM) {
                const float4 *q = reinterpret_cast<const float4 *>(yp + 8 * t);
                const float4 *w = reinterpret_cast<const float4 *>(pro.w + 8 * t);
                p1[i][0] = q[0];
                p1[i][1] = q[1];
                p2[i][0] = w[0];
                p2[i][1] = w[1];
            }
            if constexpr (PRO == PRO_NORMD) {
                const float4 *w = reinterpret_cast<const float4 *>(pro.w + 8 * t);
                p2[i][0] = w[0];
                p2[i][1] = w[1];
            }
        }
    }

    // The prologue, in registers, between load() and store() (one vector,
    // nvec = 1), called after the kernel has issued its weight loads.  Every
    // thread of the workgroup calls it.  The prologue's inputs first pass
    // through empty asm statements that clobber memory: otherwise the
    // compiler computes the prologue as soon as x arrives, ahead of the
    // weight loads, and their latency then adds to x's.
    __device__ __forceinline__ void apply(int K, const MvPro &pro = MvPro{}) {
        if constexpr (PRO == PRO_NORMD) {
            // x^2 over this thread's tasks (a clamped re-read of the last
            // task is not counted), then x' = x * w; r comes after the dots
            const int ntask = 4 * (K / 32);
            ss = 0.f;
#pragma unroll
            for (int i = 0; i < MAXT; i++) {
                const bool ok = (int)threadIdx.x + i * NT < ntask;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    pro_pin(v[i][h]);
                    pro_pin(p2[i][h]);
                    float *a = reinterpret_cast<float *>(&v[i][h]);
                    const float *w = reinterpret_cast<const float *>(&p2[i][h]);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        if (ok) ss += a[c] * a[c];
                        a[c] = a[c] * w[c];
                    }
                }
            }
        }
        if constexpr (PRO == PRO_NORM) {
#pragma unroll
            for (int i = 0; i < MAXT; i++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    pro_pin(v[i][h]);
                    pro_pin(p1[i][h]);
                    pro_pin(p2[i][h]);
                }
        }
        if constexpr (PRO == PRO_NORM) {
            const int ntask = 4 * (K / 32);
            const bool hy = pro.y != nullptr;
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < MAXT; i++) {
                const int t = (int)threadIdx.x + i * NT;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float *a = reinterpret_cast<float *>(&v[i][h]);
                    const float *y = reinterpret_cast<const float *>(&p1[i][h]);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        a[c] = a[c] + (hy ? y[c] : 0.f);
                        if (t < ntask) ss += a[c] * a[c];
                    }
                }
                if (blockIdx.x == 0 && pro.vo && t < ntask) {
                    float4 *o = reinterpret_cast<float4 *>(pro.vo + 8 * t);
                    o[0] = v[i][0];
                    o[1] = v[i][1];
                }
            }
            const float r = 1.0f / sqrtf(pro_block_sum(ss) / (float)K + pro.eps);
#pragma unroll
            for (int i = 0; i < MAXT; i++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float *a = reinterpret_cast<float *>(&v[i][h]);
                    const float *w = reinterpret_cast<const float *>(&p2[i][h]);
#pragma unroll
                    for (int c = 0; c < 4; c++) a[c] = a[c] * r * w[c];
                }
        }
    }

    __device__ __forceinline__ void store(uint32_t *xd, int K, int nvec = 1) const {
        const int ntask = 4 * (K / 32) * nvec;
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            // every round runs on every lane (no early exit: that would let the
            // compiler sink x's loads below the weights'); only tasks < ntask store
            const int t = threadIdx.x + i * NT;
            const int g = t >> 2, o = t & 3;
            const float4 a = v[i][0], b = v[i][1];
            const float e8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float mx = 0.f, sm = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                mx = fmaxf(mx, fabsf(e8[j]));
                sm += e8[j];
            }
            // the task's 4 lanes form one DPP quad (active together)
            mx = fmaxf(mx, dpp_f32<DPP_QXOR1>(mx));
            mx = fmaxf(mx, dpp_f32<DPP_QXOR2>(mx));
            sm += dpp_f32<DPP_QXOR1>(sm);
            sm += dpp_f32<DPP_QXOR2>(sm);
            int e = 0;
            frexpf(mx, &e);
            int s = mx > 0.f ? 22 - e : 0;
            s = s > 126 ? 126 : (s < -126 ? -126 : s);
            const float sc = ldexpf(1.f, s);
            uint32_t X[8];
#pragma unroll
            // rint(x * 2^s) as the low bits of fl(x * 2^s + 1.5 * 2^23): the
            // sum lies in [2^23, 2^24) (|x * 2^s| < 2^22), where one ulp is 1,
            // so the single rounding of the fma is round-to-nearest-even
            for (int j = 0; j < 8; j++) X[j] = __builtin_bit_cast(uint32_t, fmaf(e8[j], sc, 12582912.f)) - 0x4B400000u;
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
            if (t < ntask) {
                uint32_t *unit = xd + (g >> 1) * XD_UNIT;
                uint32_t *dst = unit + (g & 1) * 24 + o * 6;
                *reinterpret_cast<uint2 *>(dst) = make_uint2(dig[0], dig[1]);
                *reinterpret_cast<uint2 *>(dst + 2) = make_uint2(dig[2], dig[3]);
                *reinterpret_cast<uint2 *>(dst + 4) = make_uint2(dig[4], dig[5]);
                if (o == 0) {
                    unit[48 + (g & 1)] = __builtin_bit_cast(uint32_t, sm);
                    unit[50 + (g & 1)] = __builtin_bit_cast(uint32_t, ldexpf(1.f, -s));
                }
            }
        }
    }
};

// sum q*x over one Q4_K sub-block whose 32 nibbles are packed in q (byte i =
// weights 2i, 2i+1), times the sub-block scale S, minus M*sum(x), added to
// acc.  D holds the sub-block's 24 digit dwords, sx = sum of its x, isc =
// 2^-s of its digits.
__device__ __forceinline__ float q4_subblock(uint4 q, const uint4 *D, float sx, float isc, float S, float Mn,
                                             float acc) {
    const uint32_t *D32 = reinterpret_cast<const uint32_t *>(D);
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
    // 256*am + al < 2^31 (|q| <= 15, 32 elements): one integer add, then
    // the same single rounding to fp32 as fmaf(am, 256, al)
    const float f = fmaf((float)ah, 65536.f, (float)(am * 256u + al));
    acc = fmaf(S * isc, f, acc);
    return fmaf(-Mn, sx, acc);
}

// One unit's digits (two sub-blocks) and {sum x_even, sum x_odd, 2^-s_even,
// 2^-s_odd}, as laid out in LDS.
struct XUnit {
    uint4 d[12];
    float4 meta;
};

__device__ __forceinline__ void xunit_load(const uint32_t *xd, int u, XUnit &x) {
    const uint4 *p = reinterpret_cast<const uint4 *>(xd + (size_t)u * XD_UNIT);
#pragma unroll
    for (int i = 0; i < 12; i++) x.d[i] = p[i];
    x.meta = *reinterpret_cast<const float4 *>(p + 12);
}

struct Q4KUnit {
    uint4 hdr, q0, q1;
    uint32_t mind;
};

// Unit u of a row: super-block u/4, sub-blocks 2*(u%4) and 2*(u%4)+1.  In
// both layouts the unit's quants are bytes 32p..32p+31 of qs; the
// reference's layout also needs the first quant dword (its min bytes of
// sub-blocks 4-7).  GG = ggml's layout (QT_GQ4_K).
template <bool GG = false>
__device__ __forceinline__ void q4k_load(const uint8_t *row, int u, Q4KUnit &r) {
    const uint8_t *b = row + (size_t)(u >> 2) * 144;
    const int p = u & 3;
    r.hdr = *reinterpret_cast<const uint4 *>(b);
    r.q0 = *reinterpret_cast<const uint4 *>(b + 16 + 32 * p);
    r.q1 = *reinterpret_cast<const uint4 *>(b + 32 + 32 * p);
    if constexpr (!GG) r.mind = *reinterpret_cast<const uint32_t *>(b + 16);
}

// ggml's layout: quant byte l of the unit holds element l of sub-block 2p
// (low nibble) and of sub-block 2p+1 (high nibble).  The digits are staged
// in even / odd element order per 8-element run, so one v_perm per run and
// parity gathers bytes 8o + {0,2,4,6} (8o + {1,3,5,7}); their low nibbles
// feed sub-block 2p, their high nibbles sub-block 2p+1.
__device__ __forceinline__ float gq4_subblock(const uint32_t *ev, const uint32_t *od, int sh, const uint4 *D, float sx,
                                              float isc, float S, float Mn, float acc) {
    const uint32_t *D32 = reinterpret_cast<const uint32_t *>(D);
    int ah = 0;
    uint32_t am = 0, al = 0;
#pragma unroll
    for (int o = 0; o < 4; o++) {
        const uint32_t lo = (ev[o] >> sh) & 0x0F0F0F0Fu;
        const uint32_t hi = (od[o] >> sh) & 0x0F0F0F0Fu;
        ah = __builtin_amdgcn_sdot4((int)lo, (int)D32[o * 6 + 0], ah, false);
        ah = __builtin_amdgcn_sdot4((int)hi, (int)D32[o * 6 + 1], ah, false);
        am = __builtin_amdgcn_udot4(lo, D32[o * 6 + 2], am, false);
        am = __builtin_amdgcn_udot4(hi, D32[o * 6 + 3], am, false);
        al = __builtin_amdgcn_udot4(lo, D32[o * 6 + 4], al, false);
        al = __builtin_amdgcn_udot4(hi, D32[o * 6 + 5], al, false);
    }
    // 256*am + al < 2^31 (|q| <= 15, 32 elements): one integer add, then
    // the same single rounding to fp32 as fmaf(am, 256, al)
    const float f = fmaf((float)ah, 65536.f, (float)(am * 256u + al));
    acc = fmaf(S * isc, f, acc);
    return fmaf(-Mn, sx, acc);
}

// Reference scale/min selection (layer4/tb_gguf.c:163-168): sub-block j<4
// takes scale byte 4+j and min byte 8+j; j>=4 takes scale byte 8+j and min
// byte 12+j, i.e. the first four quant bytes.  GG: ggml's get_scale_min_k4,
// IEEE fp16 d and dmin, and ggml's quant order.
template <bool GG = false>
__device__ __forceinline__ float q4k_unit_dot(const Q4KUnit &r, int u, const XUnit &x, float acc) {
    const int p = u & 3;
    if constexpr (GG) {
        float d, dmin;
        f16x2_dec<true>(r.hdr.x, d, dmin);
        int s0, m0, s1, m1;
        gq4k_sm(r.hdr, p, 0, s0, m0);
        gq4k_sm(r.hdr, p, 1, s1, m1);
        const uint32_t g[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        uint32_t ev[4], od[4];
#pragma unroll
        for (int o = 0; o < 4; o++) {
            ev[o] = __builtin_amdgcn_perm(g[2 * o + 1], g[2 * o], 0x06040200u);
            od[o] = __builtin_amdgcn_perm(g[2 * o + 1], g[2 * o], 0x07050301u);
        }
        acc = gq4_subblock(ev, od, 0, x.d, x.meta.x, x.meta.z, d * (float)s0, dmin * (float)m0, acc);
        return gq4_subblock(ev, od, 4, x.d + 6, x.meta.y, x.meta.w, d * (float)s1, dmin * (float)m1, acc);
    }
    float d, dmin;
    f16x2_dec<false>(r.hdr.x, d, dmin);
    const uint32_t sw = p < 2 ? r.hdr.y : r.hdr.w;
    const uint32_t mw = p < 2 ? r.hdr.z : r.mind;
    const int sh = 16 * (p & 1);
    const float S0 = d * (float)((sw >> sh) & 63), S1 = d * (float)((sw >> (sh + 8)) & 63);
    const float M0 = dmin * (float)((mw >> sh) & 63), M1 = dmin * (float)((mw >> (sh + 8)) & 63);
    acc = q4_subblock(r.q0, x.d, x.meta.x, x.meta.z, S0, M0, acc);
    return q4_subblock(r.q1, x.d + 6, x.meta.y, x.meta.w, S1, M1, acc);
}

// Same, with the unit's digits read from LDS.
template <bool GG = false>
__device__ __forceinline__ float q4k_unit_dot(const Q4KUnit &r, int u, const uint32_t *xd, float acc) {
    XUnit x;
    xunit_load(xd, u, x);
    return q4k_unit_dot<GG>(r, u, x, acc);
}

}  // namespace tbq
