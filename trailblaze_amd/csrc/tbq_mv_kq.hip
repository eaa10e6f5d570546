// tbq_mv_kq.hip -- decode matvec y = W x on integer dot products for the
// block formats Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 and Q8_K
// (tb_gguf_dequant_matvec, layer4/tb_gguf.c:376-419; block layouts
// layer4/tb_gguf.c:110-288), and for ggml's layouts of the same formats.
//
// x representation.  x is cut into units of 64 elements.  Each unit gets one
// power-of-two scale 2^s (max |x| of the unit maps just below 2^22) and
// X_i = rint(x_i * 2^s) is written in balanced base 256,
//     X = 65536*h + 256*m + l,   h, m, l signed bytes,
// so sum_i q_i x_i over any run of a unit is 2^-s * (65536*sum q h +
// 256*sum q m + sum q l), where every inner sum is an exact v_dot4_i32_i8
// chain over weight bytes.  x is represented to 2^-23 of the unit's max |x|,
// which keeps the matvec within ~1e-7 relative of the reference's fp32 sum
// (the parity bound is 1e-5).
//
// Weights.  A lane unpacks its unit's quants into bytes (4 per dword) in one
// of two element orders, and the digits of x are staged in the same order:
//   PAIR     dword 2k holds elements 8k+{0,2,4,6}, dword 2k+1 holds 8k+{1,3,5,7}
//            (nibble-packed and 2-bit-packed formats: low/high nibbles, and
//            v_perm of a dword with itself shifted by 4 for 2-bit fields);
//   QUAD     dword 4g+k holds elements 16g+k+{0,4,8,12} (Q2_K: the 2-bit
//            fields at bits 2k of a quant dword, one shift and one and);
//   NATURAL  dword t holds elements 4t..4t+3 (int8 formats).
// Dwords 4g..4g+3 always hold the unit's 16-element group g.  Per-group
// integer scales multiply the digit sums in integer arithmetic
// (v_mad_i32_i24), so each unit converts to fp32 once; offsets and mins are
// applied with the fp32 group sums of x.
//
// Work split.  Lane = one unit of a row, LPR lanes per row (a row slice of
// <= 64 units); rows longer than 64 units are split over S waves of the
// workgroup whose partial sums meet in LDS.  A lane keeps its unit's digits
// in VGPRs for every row it visits; rows are grid-strided, and the weights
// of the next pass are loaded before the current pass is reduced.  Rows of
// 17..63 units that are not a power of two, and tall matrices of 64-unit
// rows, use a segmented mapping instead (k_mv_kq_seg): workgroup lane L
// takes unit L % U of row slot L / U, so a row slice wastes no lanes.
#include "tbq_kernels.h"
#include "tbq_kquant.hpp"


namespace tbq {

constexpr int KQ_UNIT = 52;   // LDS dwords per unit: 3 digit planes x 16 + 2^-s + pad

// Launch shape: KQ_NW waves per workgroup (split into slices for K > 4096;
// KQ_G3 row groups of 3 slices for K <= 12288), at most KQ_WG_PER_CU
// workgroups per CU, KQ_R rows per wave and pass, KQ_D passes prefetched.
#ifndef KQ_NW
#define KQ_NW 16
#endif
#ifndef KQ_R
#define KQ_R 1
#endif
#ifndef KQ_D
#define KQ_D 1
#endif
#ifndef KQ_G3
#define KQ_G3 4
#endif
#ifndef KQ_WG_PER_CU
#define KQ_WG_PER_CU 1
#endif

// The unit's digits in registers.
struct KqX {
    uint32_t h[16], m[16], l[16];
    float isc;       // 2^-s
    float gs[4];     // fp32 sums of x over the unit's 16-element groups
};

__device__ __forceinline__ uint32_t bfe(uint32_t v, int off, int w) { return __builtin_amdgcn_ubfe(v, off, w); }
__device__ __forceinline__ int sbfe(uint32_t v, int off, int w) { return __builtin_amdgcn_sbfe((int)v, off, w); }
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }
__device__ __forceinline__ uint32_t mulu24(uint32_t a, uint32_t b) { return (uint32_t)__umul24(a, b); }

// N little-endian dwords starting at a 2-byte-aligned address p, read with
// 4-byte-aligned loads and realigned in registers (v_alignbyte_b32 with a
// per-lane shift of 0 or 2 bytes): a load that is not 4-byte aligned costs
// about 1.5x the HBM time of an aligned one on this part, whatever its
// width.  The reads cover [p - 2, p + 4N + 2) when p is 2 mod 4 and exactly
// [p, p + 4N) otherwise, so a run that ends where its block ends (always
// 4-byte aligned in the layouts below when p is) never reads past it.
// The aligned base is formed by pointer arithmetic on p (not through an
// integer), so the compiler keeps the global address space and emits
// global loads: flat loads would share the LDS wait counter, and every LDS
// wait would then also wait for the prefetched weights.
template <int N>
__device__ __forceinline__ void ld_dw(const uint8_t *p, uint32_t *out) {
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p - sh);
    uint32_t w[N + 1];
    int i = 0;
    for (; i + 4 <= N; i += 4) {
        const uint4 v = *reinterpret_cast<const uint4 *>(q + i);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
    for (; i + 2 <= N; i += 2) {
        const uint2 v = *reinterpret_cast<const uint2 *>(q + i);
        w[i] = v.x; w[i + 1] = v.y;
    }
    for (; i < N; i++) w[i] = q[i];
    w[N] = q[(sh + 4 * N - 1) >> 2];
#pragma unroll
    for (int j = 0; j < N; j++) out[j] = __builtin_amdgcn_alignbyte(w[j + 1], w[j], sh);
}

// Loads of the per-format unit loaders: wide loads at 4-byte-aligned
// addresses, ld_dw for runs that are only 2-byte aligned.
#ifdef TBQ_NT
typedef unsigned tbq_v4u __attribute__((ext_vector_type(4)));
typedef unsigned tbq_v2u __attribute__((ext_vector_type(2)));
struct GMem {
    static __device__ __forceinline__ uint4 ld128(const uint8_t *p) {
        const tbq_v4u v = __builtin_nontemporal_load(reinterpret_cast<const tbq_v4u *>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    }
    static __device__ __forceinline__ uint2 ld64(const uint8_t *p) {
        const tbq_v2u v = __builtin_nontemporal_load(reinterpret_cast<const tbq_v2u *>(p));
        return make_uint2(v.x, v.y);
    }
    static __device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p)); }
#else
struct GMem {
    static __device__ __forceinline__ uint4 ld128(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
    static __device__ __forceinline__ uint2 ld64(const uint8_t *p) { return *reinterpret_cast<const uint2 *>(p); }
    static __device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
#endif
    static __device__ __forceinline__ uint32_t ld16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }
    // 12 bytes at a 4-byte-aligned address, one dwordx3 load
    static __device__ __forceinline__ void ld96(const uint8_t *p, uint32_t *out) {
        __builtin_memcpy(out, __builtin_assume_aligned(p, 4), 12);
    }
    template <int N>
    static __device__ __forceinline__ void ldw(const uint8_t *p, uint32_t *out) { ld_dw<N>(p, out); }
};
// ---------------------------------------------------------------------------
// Staging: NT threads write the digits of all U units into LDS, in two
// phases so that x's loads can be issued before a kernel's weight loads
// (the memory counter is in order: data loaded first can be waited for
// alone).  Task (unit u, dword t) handles the 4 elements of dword t; the 16
// tasks of a unit are 16 consecutive lanes (max |x| over the unit by DPP),
// the 4 tasks of a group are a DPP quad (group sum).  Each thread handles at
// most MAXT tasks (MAXT * NT >= 16 * U).
// ---------------------------------------------------------------------------
template <int NT, int ORD, int MAXT, int PRO = PRO_NONE>   // ORD: 0 NATURAL, 1 PAIR, 2 QUAD
struct KqStager {
    float e[MAXT][4];
    float p1[MAXT][4], p2[MAXT][4];   // PRO_NORM inputs: y, w (PRO_NORMD: w)
    float ss;                         // PRO_NORMD: this thread's sum of x^2

    // PAIR dword t = 2k + par holds elements 8k + par + {0, 2, 4, 6}, QUAD
    // dword t = 4g + k elements 16g + k + {0, 4, 8, 12}: four
    // loads at a per-lane base, no selection after the data arrives.
    // Loads are unconditional (tasks past the end re-read the last one and
    // are never stored), so no branch hides them from the wait counter.
    template <typename F4>
    __device__ __forceinline__ void ld4(const float *__restrict__ src, int task, F4 &o) const {
        const int u = task >> 4, t = task & 15;
        if constexpr (ORD == 1) {
            const float *p = src + 64 * u + 8 * (t >> 1) + (t & 1);
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = p[2 * j];
        } else if constexpr (ORD == 2) {
            const float *p = src + 64 * u + 16 * (t >> 2) + (t & 3);
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = p[4 * j];
        } else {
            const float4 a = *reinterpret_cast<const float4 *>(src + 64 * u + 4 * t);
            o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        }
    }

    __device__ __forceinline__ void load(const float *__restrict__ x, int U, const MvPro &pro = MvPro{}) {
        const float *yp = (PRO == PRO_NORM && pro.y) ? pro.y : x;   // no y: loads x, adds 0
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const int task = min(i * NT + (int)threadIdx.x, U * 16 - 1);
            ld4(x, task, e[i]);
            if constexpr (PRO == PRO_NORM) {
                ld4(yp, task, p1[i]);
                ld4(pro.w, task, p2[i]);
            }
            if constexpr (PRO == PRO_NORMD) ld4(pro.w, task, p2[i]);
        }
    }

    // The prologue, in registers, between load() and store(), called after
    // the kernel has issued its weight loads.  Every thread of the workgroup
    // calls it.  Its inputs pass through pro_pin first, so the compiler
    // cannot start it (and wait for x) ahead of the weight loads.
    __device__ __forceinline__ void apply(int U, const MvPro &pro = MvPro{}) {
        if constexpr (PRO == PRO_NORM) {
#pragma unroll
            for (int i = 0; i < MAXT; i++)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    pro_pin(e[i][c]);
                    pro_pin(p1[i][c]);
                    pro_pin(p2[i][c]);
                }
        }
        if constexpr (PRO == PRO_NORMD) {
            // x^2 over this thread's tasks (a clamped re-read of the last
            // task is not counted), then x' = x * w; r comes after the dots
            ss = 0.f;
#pragma unroll
            for (int i = 0; i < MAXT; i++) {
                const bool ok = i * NT + (int)threadIdx.x < U * 16;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    pro_pin(e[i][c]);
                    pro_pin(p2[i][c]);
                    if (ok) ss += e[i][c] * e[i][c];
                    e[i][c] = e[i][c] * p2[i][c];
                }
            }
        }
        if constexpr (PRO == PRO_NORM) {
            const bool hy = pro.y != nullptr;
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < MAXT; i++) {
                const int task = i * NT + (int)threadIdx.x;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    e[i][c] = e[i][c] + (hy ? p1[i][c] : 0.f);
                    if (task < U * 16) ss += e[i][c] * e[i][c];
                }
                if (blockIdx.x == 0 && pro.vo && task < U * 16) {
                    const int u = task >> 4, t = task & 15;
                    if constexpr (ORD == 1) {
                        float *p = pro.vo + 64 * u + 8 * (t >> 1) + (t & 1);
#pragma unroll
                        for (int j = 0; j < 4; j++) p[2 * j] = e[i][j];
                    } else if constexpr (ORD == 2) {
                        float *p = pro.vo + 64 * u + 16 * (t >> 2) + (t & 3);
#pragma unroll
                        for (int j = 0; j < 4; j++) p[4 * j] = e[i][j];
                    } else {
                        *reinterpret_cast<float4 *>(pro.vo + 64 * u + 4 * t) =
                            make_float4(e[i][0], e[i][1], e[i][2], e[i][3]);
                    }
                }
            }
            const float r = 1.0f / sqrtf(pro_block_sum(ss) / (float)(64 * U) + pro.eps);
#pragma unroll
            for (int i = 0; i < MAXT; i++)
#pragma unroll
                for (int c = 0; c < 4; c++) e[i][c] = e[i][c] * r * p2[i][c];
        }
    }

    __device__ __forceinline__ void store(int U, uint32_t *xd, float *gs) const {
#pragma unroll
        for (int i = 0; i < MAXT; i++) {
            const int task = i * NT + (int)threadIdx.x;
            const bool ok = task < U * 16;        // uniform over each 16-lane row
            const int u = task >> 4, t = task & 15;
            const float *e = this->e[i];
            float mx = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
            float sm = (e[0] + e[1]) + (e[2] + e[3]);
            mx = fmaxf(mx, dpp_f32<DPP_QXOR1>(mx));
            mx = fmaxf(mx, dpp_f32<DPP_QXOR2>(mx));
            mx = fmaxf(mx, dpp_f32<DPP_HALF_MIRROR>(mx));
            mx = fmaxf(mx, dpp_f32<DPP_MIRROR>(mx));
            sm += dpp_f32<DPP_QXOR1>(sm);
            sm += dpp_f32<DPP_QXOR2>(sm);
            int ex = 0;
            frexpf(mx, &ex);
            int s = mx > 0.f ? 22 - ex : 0;
            s = s > 126 ? 126 : (s < -126 ? -126 : s);
            const float sc = ldexpf(1.f, s);
            uint32_t dh = 0, dm = 0, dl = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                // rint(x * 2^s): low bits of fl(x * 2^s + 1.5 * 2^23), |x * 2^s| < 2^22
                const int X = (int)(__builtin_bit_cast(uint32_t, fmaf(e[b], sc, 12582912.f)) - 0x4B400000u);
                const int l = (int)(int8_t)(X & 0xFF);
                const int X1 = (X - l) >> 8;
                const int m = (int)(int8_t)(X1 & 0xFF);
                const int h = (X1 - m) >> 8;
                dh |= (uint32_t)(h & 0xFF) << (8 * b);
                dm |= (uint32_t)(m & 0xFF) << (8 * b);
                dl |= (uint32_t)(l & 0xFF) << (8 * b);
            }
            if (ok) {
                uint32_t *unit = xd + u * KQ_UNIT;
                unit[t] = dh;
                unit[16 + t] = dm;
                unit[32 + t] = dl;
                if (t == 0) unit[48] = __builtin_bit_cast(uint32_t, ldexpf(1.f, -s));
                if ((t & 3) == 0) gs[4 * u + (t >> 2)] = sm;
            }
        }
    }
};

__device__ __forceinline__ void kq_xload(const uint32_t *xd, const float *gs, int u, KqX &x) {
    const uint4 *p = reinterpret_cast<const uint4 *>(xd + u * KQ_UNIT);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 a = p[i], b = p[4 + i], c = p[8 + i];
        x.h[4 * i] = a.x; x.h[4 * i + 1] = a.y; x.h[4 * i + 2] = a.z; x.h[4 * i + 3] = a.w;
        x.m[4 * i] = b.x; x.m[4 * i + 1] = b.y; x.m[4 * i + 2] = b.z; x.m[4 * i + 3] = b.w;
        x.l[4 * i] = c.x; x.l[4 * i + 1] = c.y; x.l[4 * i + 2] = c.z; x.l[4 * i + 3] = c.w;
    }
    x.isc = __builtin_bit_cast(float, xd[u * KQ_UNIT + 48]);
    const float4 g = *reinterpret_cast<const float4 *>(gs + 4 * u);
    x.gs[0] = g.x; x.gs[1] = g.y; x.gs[2] = g.z; x.gs[3] = g.w;
}

// Digit sums of weight dwords q[0..N) against digit dwords T0..T0+N.
template <int N>
__device__ __forceinline__ void kq_dots(const uint32_t *q, const KqX &x, int T0, int &ah, int &am, int &al) {
#pragma unroll
    for (int j = 0; j < N; j++) {
        ah = __builtin_amdgcn_sdot4((int)q[j], (int)x.h[T0 + j], ah, false);
        am = __builtin_amdgcn_sdot4((int)q[j], (int)x.m[T0 + j], am, false);
        al = __builtin_amdgcn_sdot4((int)q[j], (int)x.l[T0 + j], al, false);
    }
}

// Integer-scaled digit accumulators -> fp32: 65536*H + 256*Mm + L.
__device__ __forceinline__ float kq_combine(int H, int Mm, int L) {
    return fmaf((float)H, 65536.f, fmaf((float)Mm, 256.f, (float)L));
}

// 2-bit fields of one dword (16 elements, 4 per byte at bits 0-1, 2-3, 4-5,
// 6-7) as PAIR-ordered bytes: q[0] = [e0,e2,e4,e6], q[1] = [e1,e3,e5,e7],
// q[2] = [e8,e10,e12,e14], q[3] = [e9,e11,e13,e15].  v_perm of Q with Q>>4
// puts the fields of elements 4j and 4j+2 (4j+1 and 4j+3) at bits 0-1
// (2-3) of consecutive bytes.
__device__ __forceinline__ void unpack2(uint32_t Q, uint32_t *q) {
    const uint32_t S = Q >> 4;
    const uint32_t R0 = __builtin_amdgcn_perm(S, Q, 0x05010400u);
    const uint32_t R1 = __builtin_amdgcn_perm(S, Q, 0x07030602u);
    q[0] = R0 & 0x03030303u;
    q[1] = (R0 >> 2) & 0x03030303u;
    q[2] = R1 & 0x03030303u;
    q[3] = (R1 >> 2) & 0x03030303u;
}

// Bits 0,2,4,6 (even) or 1,3,5,7 (odd) of byte b moved to bit SH of bytes
// 0..3.  One multiply spreads the four bits; its cross terms only collide at
// positions whose carries land on bits the mask clears.
template <int SH>
__device__ __forceinline__ uint32_t spread_even(uint32_t b) {
    return mulu24(b & 0x55u, (1u << SH) | (1u << (SH + 6)) | (1u << (SH + 12)) | (1u << (SH + 18)));
}
template <int SH>
__device__ __forceinline__ uint32_t spread_odd(uint32_t b) {
    return mulu24(b & 0xAAu, (1u << (SH - 1)) | (1u << (SH + 5)) | (1u << (SH + 11)) | (1u << (SH + 17)));
}

// ---------------------------------------------------------------------------
// Per-format unit loads and dots.  Unit u of a row: super-block u/4, weights
// 64*(u%4)..+63 (256-weight formats); blocks 2u, 2u+1 (32-weight formats).
// ---------------------------------------------------------------------------
// A Q4_0 unit (two 18-byte blocks, 36 bytes, 4-byte aligned in rows of K %
// 64 == 0 elements) in three loads: block 0's d (bytes 0-1) and quants
// (bytes 2-17, realigned by two bytes), block 1's d (bytes 18-19) and quants
// (bytes 20-35, aligned).
__device__ __forceinline__ void q40_unit_load(const uint8_t *row, int u, uint4 &a, uint4 &b, uint32_t &d0,
                                              uint32_t &d1) {
    const uint32_t *q = reinterpret_cast<const uint32_t *>(row + (size_t)u * 36);
    const uint4 A = *reinterpret_cast<const uint4 *>(q), B = *reinterpret_cast<const uint4 *>(q + 4);
    const uint32_t C = q[8];
    d0 = A.x & 0xFFFFu;
    a = make_uint4(__builtin_amdgcn_alignbyte(A.y, A.x, 2), __builtin_amdgcn_alignbyte(A.z, A.y, 2),
                   __builtin_amdgcn_alignbyte(A.w, A.z, 2), __builtin_amdgcn_alignbyte(B.x, A.w, 2));
    d1 = B.x >> 16;
    b = make_uint4(B.y, B.z, B.w, C);
}

template <int QT> struct KqFmt;

// Q2_K (layer4/tb_gguf.c:210-225): sc[16]@0 (scale lo nibble, min hi
// nibble per 16 weights), qs[64]@16 (weight i at bits 2(i&3) of qs[i>>2]),
// d@80, dmin@82.  w = fl(fl(d*sc)*q) - fl(dmin*m).
template <> struct KqFmt<QT_Q2_K> {
    static constexpr bool PAIR = false;   // digits in QUAD order (kq_order)
    struct Unit { uint4 qs; uint32_t sc, dd; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 84;
        const int p = u & 3;
        w.qs = GMem::ld128(b + 16 + 16 * p);
        w.sc = GMem::ld32(b + 4 * p);
        w.dd = GMem::ld32(b + 80);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x) {
        const uint32_t qv[4] = {w.qs.x, w.qs.y, w.qs.z, w.qs.w};
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            // QUAD order: q[k] byte b = element 16g + 4b + k, at bits 2k of
            // quant byte 4g + b
            uint32_t q[4];
#pragma unroll
            for (int k = 0; k < 4; k++) q[k] = (qv[g] >> (2 * k)) & 0x03030303u;
            int ah = 0, am = 0, al = 0;
            kq_dots<4>(q, x, 4 * g, ah, am, al);
            const int s = (int)bfe(w.sc, 8 * g, 4), m = (int)bfe(w.sc, 8 * g + 4, 4);
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)m, x.gs[g], mn);
        }
        float d, dmin;
        f16x2_dec<false>(w.dd, d, dmin);
        return fmaf(d * x.isc, kq_combine(H, Mm, L), -dmin * mn);
    }
};

// Q3_K (layer4/tb_gguf.c:230-257): hmask[32]@0 (weight i: bit i&7 of
// hmask[i>>3]), qs[64]@32 (2-bit, as Q2_K), sc[12]@96, d@108.  Group j of
// 16 uses scale slot j&7: lo4 from sc[slot>>1] nibble slot&1, hi2 from
// sc[8+(slot>>2)] bits 2(slot&3); S = d*((lo4|hi2<<4)-32); w = S*(q3-4).
template <> struct KqFmt<QT_Q3_K> {
    static constexpr bool PAIR = true;
    struct Unit { uint4 qs; uint2 hm; uint32_t lo; uint2 hi; };
    // 110-byte blocks: every other block starts 2 mod 4 (sh = 2).  Five
    // loads per unit, none past the block: the 16 quant bytes through ld_dw
    // (two); the 8 hmask bytes as one dwordx3 from the aligned-down address;
    // bytes 92 + sh .. 108 + sh (a 16-byte window, aligned, ending at or
    // before the block's end) for sc[0..3] and sc[8..11], plus d as a 16-bit
    // load (for sh = 2 the window holds d as well; the load is issued either
    // way, so every lane issues the same loads).
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 110;
        const int p = u & 3;
        const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(b) & 3u);
        uint32_t t[4];
        GMem::template ldw<4>(b + 32 + 16 * p, t);
        w.qs = make_uint4(t[0], t[1], t[2], t[3]);
        uint32_t h[3];
        GMem::ld96(b + 8 * p - sh, h);
        w.hm = make_uint2(__builtin_amdgcn_alignbyte(h[1], h[0], sh), __builtin_amdgcn_alignbyte(h[2], h[1], sh));
        const uint4 v = GMem::ld128(b + 92 + sh);
        const uint32_t d16 = GMem::ld16(b + 108);
        w.lo = sh ? __builtin_amdgcn_alignbyte(v.y, v.x, 2) : v.y;    // sc[0..3]
        w.hi.x = sh ? __builtin_amdgcn_alignbyte(v.w, v.z, 2) : v.w;  // sc[8..11]
        w.hi.y = (sh ? v.w >> 16 : d16) << 16;                         // d in the high half
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int p1 = u & 1;   // groups 4p..4p+3 use slots 4*(p&1)..+3
        const uint32_t qv[4] = {w.qs.x, w.qs.y, w.qs.z, w.qs.w};
        const uint32_t hi2b = bfe(w.hi.x, 8 * p1, 8);        // sc[8 + (p&1)]
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t q[4];
            unpack2(qv[g], q);
            const uint32_t hv = ((g < 2) ? w.hm.x : w.hm.y) >> (16 * (g & 1));   // bytes 2g, 2g+1
            const uint32_t h1 = hv >> 8;
            q[0] = (spread_even<2>(hv) & 0x04040404u) | q[0];
            q[1] = (spread_odd<2>(hv) & 0x04040404u) | q[1];
            q[2] = (spread_even<2>(h1) & 0x04040404u) | q[2];
            q[3] = (spread_odd<2>(h1) & 0x04040404u) | q[3];
            int ah = 0, am = 0, al = 0;
            kq_dots<4>(q, x, 4 * g, ah, am, al);
            const int lo4 = (int)bfe(w.lo, 16 * p1 + 4 * g, 4);
            const int hi2 = (int)bfe(hi2b, 2 * g, 2);
            const int s = (lo4 | (hi2 << 4)) - 32;
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)s, x.gs[g], mn);
        }
        const float d = f16_dec<false>(w.hi.y >> 16);
        return d * fmaf(x.isc, kq_combine(H, Mm, L), -4.f * mn);
    }
};

// Q4_K (layer4/tb_gguf.c:148-180): d@0, dmin@2, sc[12]@4, qs[128]@16.
// Sub-block j<4: scale sc[j]&63, min sc[j+4]&63; j>=4: scale sc[j+4]&63,
// min byte 12+j of the block (qs[j-4]).
template <> struct KqFmt<QT_Q4_K> {
    static constexpr bool PAIR = true;
    struct Unit { uint4 hdr, q0, q1; uint32_t mind; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 144;
        const int p = u & 3;
        w.hdr = GMem::ld128(b);
        w.q0 = GMem::ld128(b + 16 + 32 * p);
        w.q1 = GMem::ld128(b + 32 + 32 * p);
        w.mind = GMem::ld32(b + 16);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int p = u & 3;
        const uint32_t sw = p < 2 ? w.hdr.y : w.hdr.w;
        const uint32_t mw = p < 2 ? w.hdr.z : w.mind;
        const int sh = 16 * (p & 1);
        const uint32_t qv[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                q[2 * k] = qv[4 * j + k] & 0x0F0F0F0Fu;
                q[2 * k + 1] = (qv[4 * j + k] >> 4) & 0x0F0F0F0Fu;
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<8>(q, x, 8 * j, ah, am, al);
            const int s = (int)bfe(sw, sh + 8 * j, 6), m = (int)bfe(mw, sh + 8 * j, 6);
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)m, x.gs[2 * j] + x.gs[2 * j + 1], mn);
        }
        float d, dmin;
        f16x2_dec<false>(w.hdr.x, d, dmin);
        return fmaf(d * x.isc, kq_combine(H, Mm, L), -dmin * mn);
    }
};

// Q5_K (layer4/tb_gguf.c:262-279 with q4_k_unpack_scales :122-145): d@0,
// dmin@2, sc[12]@4, qh[32]@16 (weight i: bit i&7 of qh[i>>3]), qs[128]@48.
// j<4: scale sc[j]&63, min sc[j+4]&63; j>=4, k=j-4: scale
// (sc[k]>>6)|((sc[k+8]&15)<<2), min (sc[k+4]>>6)|((sc[k+12]&15)<<2) where
// sc[12..15] are qh[0..3].
template <> struct KqFmt<QT_Q5_K> {
    static constexpr bool PAIR = true;
    struct Unit { uint4 hdr, q0, q1; uint32_t qh0; uint2 qh; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 176;
        const int p = u & 3;
        w.hdr = GMem::ld128(b);
        w.qh0 = GMem::ld32(b + 16);
        w.qh = GMem::ld64(b + 16 + 8 * p);
        w.q0 = GMem::ld128(b + 48 + 32 * p);
        w.q1 = GMem::ld128(b + 64 + 32 * p);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int p = u & 3;
        const uint32_t qv[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int kk = 4 * j + k;                    // qs dword of the unit, qh byte kk
                const uint32_t hb = bfe(kk < 4 ? w.qh.x : w.qh.y, 8 * (kk & 3), 8);
                q[2 * k] = (spread_even<4>(hb) & 0x10101010u) | (qv[kk] & 0x0F0F0F0Fu);
                q[2 * k + 1] = (spread_odd<4>(hb) & 0x10101010u) | ((qv[kk] >> 4) & 0x0F0F0F0Fu);
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<8>(q, x, 8 * j, ah, am, al);
            int s, m;
            const int jj = 2 * p + j;   // sub-block within the super-block
            if (jj < 4) {
                s = (int)bfe(w.hdr.y, 8 * jj, 6);
                m = (int)bfe(w.hdr.z, 8 * jj, 6);
            } else {
                const int k = jj - 4;   // 0..3
                s = (int)(bfe(w.hdr.y, 8 * k + 6, 2) | (bfe(w.hdr.w, 8 * k, 4) << 2));
                m = (int)(bfe(w.hdr.z, 8 * k + 6, 2) | (bfe(w.qh0, 8 * k, 4) << 2));
            }
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)m, x.gs[2 * j] + x.gs[2 * j + 1], mn);
        }
        float d, dmin;
        f16x2_dec<false>(w.hdr.x, d, dmin);
        return fmaf(d * x.isc, kq_combine(H, Mm, L), -dmin * mn);
    }
};

// Q6_K (layer4/tb_gguf.c:190-204): ql[128]@0 (weight i: nibble i&1 of
// ql[i>>1]), qh[64]@128 (bits 2(i&3) of qh[i>>2]), int8 sc[16]@192, d@208.
// w = fl(d*sc[i>>4]) * (q - 32).
template <> struct KqFmt<QT_Q6_K> {
    static constexpr bool PAIR = true;
    struct Unit { uint4 ql0, ql1, qh; uint32_t sc, d; };
    // 210-byte blocks: every other block starts 2 mod 4 (ld_dw)
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 210;
        const int p = u & 3;
        uint32_t t[8];
        GMem::template ldw<8>(b + 32 * p, t);
        w.ql0 = make_uint4(t[0], t[1], t[2], t[3]);
        w.ql1 = make_uint4(t[4], t[5], t[6], t[7]);
        GMem::template ldw<4>(b + 128 + 16 * p, t);
        w.qh = make_uint4(t[0], t[1], t[2], t[3]);
        GMem::template ldw<1>(b + 192 + 4 * p, &w.sc);
        w.d = GMem::ld16(b + 208);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int) {
        const uint32_t qv[8] = {w.ql0.x, w.ql0.y, w.ql0.z, w.ql0.w, w.ql1.x, w.ql1.y, w.ql1.z, w.ql1.w};
        const uint32_t hv[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t q[4];
            const uint32_t QH = hv[g], S = QH >> 4;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int k = 2 * g + c;   // ql dword k: weights 8k..8k+7; qh bytes 2k, 2k+1
                const uint32_t R = __builtin_amdgcn_perm(S, QH, c ? 0x07030602u : 0x05010400u);
                q[2 * c] = ((R << 4) & 0x30303030u) | (qv[k] & 0x0F0F0F0Fu);
                q[2 * c + 1] = ((R << 2) & 0x30303030u) | ((qv[k] >> 4) & 0x0F0F0F0Fu);
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<4>(q, x, 4 * g, ah, am, al);
            const int s = sbfe(w.sc, 8 * g, 8);
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)s, x.gs[g], mn);
        }
        const float d = f16_dec<false>(w.d);
        return d * fmaf(x.isc, kq_combine(H, Mm, L), -32.f * mn);
    }
};

// Q8_0 (layer4/tb_gguf.c:183-187): d@0, int8 qs[32]@2; w = d*q.  The ggml
// layout is the same but for its IEEE fp16 d.
template <int QT> struct KqQ80 {
    static constexpr bool PAIR = false;
    struct Unit { uint4 a0, a1, b0, b1; uint32_t d0, d1; };
    // unit = 68 bytes, 4-byte aligned (rows of K % 64 == 0 elements are):
    // its 17 dwords in five loads, then block 0's d (bytes 0-1) and quants
    // (bytes 2-33, realigned by two bytes), block 1's d (bytes 34-35) and
    // quants (bytes 36-67, aligned)
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint32_t *q = reinterpret_cast<const uint32_t *>(row + (size_t)u * 68);
        const uint4 A = *reinterpret_cast<const uint4 *>(q), B = *reinterpret_cast<const uint4 *>(q + 4);
        const uint4 C = *reinterpret_cast<const uint4 *>(q + 8), D = *reinterpret_cast<const uint4 *>(q + 12);
        const uint32_t E = q[16];
        const uint32_t t[9] = {A.x, A.y, A.z, A.w, B.x, B.y, B.z, B.w, C.x};
        uint32_t r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) r[j] = __builtin_amdgcn_alignbyte(t[j + 1], t[j], 2);
        w.d0 = A.x & 0xFFFFu;
        w.a0 = make_uint4(r[0], r[1], r[2], r[3]);
        w.a1 = make_uint4(r[4], r[5], r[6], r[7]);
        w.d1 = C.x >> 16;
        w.b0 = make_uint4(C.y, C.z, C.w, D.x);
        w.b1 = make_uint4(D.y, D.z, D.w, E);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int) {
        const uint32_t q0[8] = {w.a0.x, w.a0.y, w.a0.z, w.a0.w, w.a1.x, w.a1.y, w.a1.z, w.a1.w};
        const uint32_t q1[8] = {w.b0.x, w.b0.y, w.b0.z, w.b0.w, w.b1.x, w.b1.y, w.b1.z, w.b1.w};
        int h0 = 0, m0 = 0, l0 = 0, h1 = 0, m1 = 0, l1 = 0;
        kq_dots<8>(q0, x, 0, h0, m0, l0);
        kq_dots<8>(q1, x, 8, h1, m1, l1);
        const float f0 = f16_dec<(QT & QT_GGML) != 0>(w.d0) * kq_combine(h0, m0, l0);
        return fmaf(f16_dec<(QT & QT_GGML) != 0>(w.d1), kq_combine(h1, m1, l1), f0) * x.isc;
    }
};

template <> struct KqFmt<QT_Q8_0> : KqQ80<QT_Q8_0> {};
template <> struct KqFmt<QT_GQ8_0> : KqQ80<QT_GQ8_0> {};

// Q4_0 (layer4/tb_gguf.c:110-118): d@0, qs[16]@2; weight 2i = low nibble of
// qs[i], 2i+1 = high nibble; w = d*(q-8).
template <> struct KqFmt<QT_Q4_0> {
    static constexpr bool PAIR = true;
    struct Unit { uint4 a, b; uint32_t d0, d1; };
    // unit = 36 bytes: block 0's quants start 2 mod 4 when the unit is
    // aligned (ld_dw)
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        q40_unit_load(row, u, w.a, w.b, w.d0, w.d1);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int) {
        const float d0 = f16_dec<false>(w.d0), d1 = f16_dec<false>(w.d1);
        float r = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint4 v = j ? w.b : w.a;
            const uint32_t qv[4] = {v.x, v.y, v.z, v.w};
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                q[2 * k] = qv[k] & 0x0F0F0F0Fu;
                q[2 * k + 1] = (qv[k] >> 4) & 0x0F0F0F0Fu;
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<8>(q, x, 8 * j, ah, am, al);
            const float sx = x.gs[2 * j] + x.gs[2 * j + 1];
            r = fmaf(j ? d1 : d0, fmaf(x.isc, kq_combine(ah, am, al), -8.f * sx), r);
        }
        return r;
    }
};

// Q8_K (layer4/tb_gguf.c:283-288): f32 d@0, int8 qs[256]@4; w = d*q.
template <> struct KqFmt<QT_Q8_K> {
    static constexpr bool PAIR = false;
    struct Unit { uint4 q[4]; uint32_t d; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 292;
        const int p = u & 3;
        w.d = GMem::ld32(b);
#pragma unroll
        for (int i = 0; i < 4; i++) w.q[i] = GMem::ld128(b + 4 + 64 * p + 16 * i);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int) {
        uint32_t q[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            q[4 * i] = w.q[i].x; q[4 * i + 1] = w.q[i].y; q[4 * i + 2] = w.q[i].z; q[4 * i + 3] = w.q[i].w;
        }
        int ah = 0, am = 0, al = 0;
        kq_dots<16>(q, x, 0, ah, am, al);
        return __builtin_bit_cast(float, w.d) * x.isc * kq_combine(ah, am, al);
    }
};

// ---------------------------------------------------------------------------
// ggml's layouts (QT_GGML ids; ggml-quants.c dequantize_row_*), NATURAL
// element order: in every K format a unit (64 consecutive weights) reads 32
// quant bytes whose byte l holds elements l and 32 + l, so dword t of the
// unit's quants is elements 4t..4t+3 after one shift and mask.  fp16 fields
// decode as IEEE.
// ---------------------------------------------------------------------------

// Q4_K: d@0, dmin@2, sc[12]@4, qs[128]@16; unit p: nibble j of qs[32p+l] is
// element 32j + l of sub-block 2p + j; its 6-bit scale and min as ggml's
// get_scale_min_k4 (gq4k_sm).
template <> struct KqFmt<QT_GQ4_K> {
    static constexpr bool PAIR = false;
    struct Unit { uint4 hdr, q0, q1; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 144;
        const int p = u & 3;
        w.hdr = GMem::ld128(b);
        w.q0 = GMem::ld128(b + 16 + 32 * p);
        w.q1 = GMem::ld128(b + 32 + 32 * p);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int p = u & 3;
        const uint32_t qv[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < 8; k++) q[k] = (qv[k] >> (4 * j)) & 0x0F0F0F0Fu;
            int ah = 0, am = 0, al = 0;
            kq_dots<8>(q, x, 8 * j, ah, am, al);
            int s, m;
            gq4k_sm(w.hdr, p, j, s, m);
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)m, x.gs[2 * j] + x.gs[2 * j + 1], mn);
        }
        float d, dmin;
        f16x2_dec<true>(w.hdr.x, d, dmin);
        return fmaf(d * x.isc, kq_combine(H, Mm, L), -dmin * mn);
    }
};

// Q5_K: d@0, dmin@2, sc[12]@4, qh[32]@16, qs[128]@48; Q4_K's reading plus
// bit 2p + j of qh[l] as 16.
template <> struct KqFmt<QT_GQ5_K> {
    static constexpr bool PAIR = false;
    struct Unit { uint4 hdr, h0, h1, q0, q1; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 176;
        const int p = u & 3;
        w.hdr = GMem::ld128(b);
        w.h0 = GMem::ld128(b + 16);
        w.h1 = GMem::ld128(b + 32);
        w.q0 = GMem::ld128(b + 48 + 32 * p);
        w.q1 = GMem::ld128(b + 64 + 32 * p);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int p = u & 3;
        const uint32_t qv[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        const uint32_t hv[8] = {w.h0.x, w.h0.y, w.h0.z, w.h0.w, w.h1.x, w.h1.y, w.h1.z, w.h1.w};
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int bit = 2 * p + j;
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                q[k] = ((qv[k] >> (4 * j)) & 0x0F0F0F0Fu) | (((hv[k] >> bit) & 0x01010101u) << 4);
            int ah = 0, am = 0, al = 0;
            kq_dots<8>(q, x, 8 * j, ah, am, al);
            int s, m;
            gq4k_sm(w.hdr, p, j, s, m);
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)m, x.gs[2 * j] + x.gs[2 * j + 1], mn);
        }
        float d, dmin;
        f16x2_dec<true>(w.hdr.x, d, dmin);
        return fmaf(d * x.isc, kq_combine(H, Mm, L), -dmin * mn);
    }
};

// Q6_K: ql[128]@0, qh[64]@128, int8 sc[16]@192, d@208; unit p (half
// n = p/2): element e of the unit is nibble p&1 of ql[64n + e] with bits
// 4(p&1) + 2(e/32) of qh[32n + e%32] above it; scale sc[4p + e/16]; q - 32.
// Units 2n and 2n+1 read the same 96 bytes, so the two lanes of a pair
// (adjacent lanes: the unit's parity is the lane's) split them: lane h
// loads ql[64n + 32h ..+31] and qh[32n ..+31], forms the 6-bit quants of
// elements 32h..32h+31 of both units, keeps its own unit's and swaps the
// other unit's with its partner (DPP quad_perm [1,0,3,2]).  Every lane of
// the wave runs dot(): lanes past the row's units pair among themselves.
template <> struct KqFmt<QT_GQ6_K> {
    static constexpr bool PAIR = false;
    struct Unit { uint32_t ql[8], qh[8], sc, d; };
    // 210-byte blocks: every other block starts 2 mod 4 (ld_dw)
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 210;
        const int p = u & 3, n = p >> 1;
        GMem::template ldw<8>(b + 64 * n + 32 * (p & 1), w.ql);
        GMem::template ldw<8>(b + 128 + 32 * n, w.qh);
        GMem::template ldw<1>(b + 192 + 4 * p, &w.sc);
        w.d = GMem::ld16(b + 208);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int h = u & 1;
        // own unit: nibble h, qh bits 2h + 4h; the partner's: nibble 1-h,
        // qh bits 4(1-h) + 2h
        const int so = 4 * h, sho = 6 * h, ss = 4 - 4 * h, shs = 4 - 2 * h;
        uint32_t mine[8], recv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            mine[k] = ((w.ql[k] >> so) & 0x0F0F0F0Fu) | (((w.qh[k] >> sho) & 0x03030303u) << 4);
            const uint32_t send = ((w.ql[k] >> ss) & 0x0F0F0F0Fu) | (((w.qh[k] >> shs) & 0x03030303u) << 4);
            recv[k] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send, DPP_QXOR1, 0xF, 0xF, false);
        }
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t q[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int t = 4 * (g & 1) + c;   // dword within the 32-element half
                q[c] = ((g >> 1) == h) ? mine[t] : recv[t];
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<4>(q, x, 4 * g, ah, am, al);
            const int s = sbfe(w.sc, 8 * g, 8);
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)s, x.gs[g], mn);
        }
        return f16_dec<true>(w.d) * fmaf(x.isc, kq_combine(H, Mm, L), -32.f * mn);
    }
};

// Q3_K: hmask[32]@0, qs[64]@32, sc[12]@96, d@108; unit p (n = p/2,
// k0 = 2(p&1)): element e has bits 2(k0 + e/32) of qs[32n + e%32] and bit
// 4n + k0 + e/32 of hmask[e%32] (set: +4); scale 4p + g of ggml's unpack:
// lo4 = nibble p/2 of sc[4(p&1) + g], hi2 = bits 2p of sc[8 + g]; value
// (q3 - 4) * ((lo4 | hi2 << 4) - 32).
template <> struct KqFmt<QT_GQ3_K> {
    static constexpr bool PAIR = false;
    struct Unit { uint32_t qs[8], hm[8], lo, hi, d; };
    // 110-byte blocks: every other block starts 2 mod 4 (ld_dw)
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 110;
        const int p = u & 3, n = p >> 1;
        GMem::template ldw<8>(b + 32 + 32 * n, w.qs);
        GMem::template ldw<8>(b, w.hm);
        GMem::template ldw<1>(b + 96 + 4 * (p & 1), &w.lo);
        GMem::template ldw<1>(b + 104, &w.hi);
        w.d = GMem::ld16(b + 108);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int p = u & 3, n = p >> 1, k0 = 2 * (p & 1);
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t q[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int t = 4 * g + c, h = t >> 3;
                q[c] = ((w.qs[t & 7] >> (2 * (k0 + h))) & 0x03030303u) |
                       (((w.hm[t & 7] >> (4 * n + k0 + h)) & 0x01010101u) << 2);
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<4>(q, x, 4 * g, ah, am, al);
            const int lo4 = (int)bfe(w.lo, 8 * g + 4 * n, 4);
            const int hi2 = (int)bfe(w.hi, 8 * g + 2 * p, 2);
            const int s = (lo4 | (hi2 << 4)) - 32;
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)s, x.gs[g], mn);
        }
        return f16_dec<true>(w.d) * fmaf(x.isc, kq_combine(H, Mm, L), -4.f * mn);
    }
};

// Q2_K: sc[16]@0, qs[64]@16, d@80, dmin@82; unit p: element e has bits
// 2(k0 + e/32) of qs[32n + e%32]; scale/min byte sc[4p + g].
template <> struct KqFmt<QT_GQ2_K> {
    static constexpr bool PAIR = false;
    struct Unit { uint4 q0, q1; uint32_t sc, dd; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        const uint8_t *b = row + (size_t)(u >> 2) * 84;
        const int p = u & 3, n = p >> 1;
        w.q0 = GMem::ld128(b + 16 + 32 * n);
        w.q1 = GMem::ld128(b + 32 + 32 * n);
        w.sc = GMem::ld32(b + 4 * p);
        w.dd = GMem::ld32(b + 80);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int u) {
        const int k0 = 2 * (u & 1);
        const uint32_t qv[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
        int H = 0, Mm = 0, L = 0;
        float mn = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t q[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int t = 4 * g + c;
                q[c] = (qv[t & 7] >> (2 * (k0 + (t >> 3)))) & 0x03030303u;
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<4>(q, x, 4 * g, ah, am, al);
            const int s = (int)bfe(w.sc, 8 * g, 4), m = (int)bfe(w.sc, 8 * g + 4, 4);
            H = mad24(s, ah, H);
            Mm = mad24(s, am, Mm);
            L = mad24(s, al, L);
            mn = fmaf((float)m, x.gs[g], mn);
        }
        float d, dmin;
        f16x2_dec<true>(w.dd, d, dmin);
        return fmaf(d * x.isc, kq_combine(H, Mm, L), -dmin * mn);
    }
};

// Q4_0: d@0, qs[16]@2; element l < 16 is the low nibble of qs[l], 16 + l
// the high nibble; w = (q - 8) * d.
template <> struct KqFmt<QT_GQ4_0> {
    static constexpr bool PAIR = false;
    struct Unit { uint4 a, b; uint32_t d0, d1; };
    static __device__ __forceinline__ void load(const uint8_t *row, int u, Unit &w) {
        q40_unit_load(row, u, w.a, w.b, w.d0, w.d1);
    }
    static __device__ __forceinline__ float dot(const Unit &w, const KqX &x, int) {
        const float d0 = f16_dec<true>(w.d0), d1 = f16_dec<true>(w.d1);
        float r = 0.f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint4 v = j ? w.b : w.a;
            const uint32_t qv[4] = {v.x, v.y, v.z, v.w};
            uint32_t q[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                q[k] = qv[k] & 0x0F0F0F0Fu;
                q[4 + k] = (qv[k] >> 4) & 0x0F0F0F0Fu;
            }
            int ah = 0, am = 0, al = 0;
            kq_dots<8>(q, x, 8 * j, ah, am, al);
            const float sx = x.gs[2 * j] + x.gs[2 * j + 1];
            r = fmaf(j ? d1 : d0, fmaf(x.isc, kq_combine(ah, am, al), -8.f * sx), r);
        }
        return r;
    }
};

// Uniform entry for formats whose dot does not need the unit index.
// Element order of a format's staged digits (see the header): QUAD for
// Q2_K's reference layout, PAIR or NATURAL as the format declares.
template <int QT>
constexpr int kq_order() {
    return QT == QT_Q2_K ? 2 : (KqFmt<QT>::PAIR ? 1 : 0);
}

template <int QT>
__device__ __forceinline__ float kq_dot(const typename KqFmt<QT>::Unit &w, const KqX &x, int u) {
    if constexpr (QT == QT_Q2_K) return KqFmt<QT>::dot(w, x);
    else return KqFmt<QT>::dot(w, x, u);
}

// ---------------------------------------------------------------------------
// The kernel.  Wave w of the workgroup: row slice s = w % S (units
// s*LPR .. s*LPR+LPR-1), row group g = w / S.  Workgroup b owns rows
// [b*rpw, min((b+1)*rpw, M)); one pass covers RWG = G*R*RPP of them (RPP =
// 64/LPR rows per wave per step p < R), so a wave has R rows' weights in
// flight per pass, and the weights of the next D passes are loaded before
// the current pass is reduced.
// ---------------------------------------------------------------------------
//
// GLU: M counts output rows; output row r is a pair of weight rows, r (gate)
// and M + r (up), taken by the same lanes in one pass (RP = 2 rows in
// flight), and y[r] = silu(gate) * up.
template <int QT, int LPR, int S, int G, int R, int D, int PRO, bool GLU>
__global__ __launch_bounds__(S * G * 64) void k_mv_kq(const uint8_t *__restrict__ W, int M, int K, long long rb,
                                                      const float *__restrict__ x, float *__restrict__ y, int rpw,
                                                      MvPro pro) {
    using F = KqFmt<QT>;
    constexpr int RL = GLU ? 1 : R;   // output rows per lane group and pass
    constexpr int RP = GLU ? 2 : R;   // weight rows per lane group and pass
    constexpr int NT = S * G * 64, RPP = 64 / LPR, RW = RL * RPP, RWG = G * RW, RWP = RP * RPP;
    constexpr int MAXT = (16 * 64 * S + NT - 1) / NT;   // U <= 64 * S
    extern __shared__ uint32_t smem[];
    const int U = K / 64;
    uint32_t *xd = smem;
    float *gs = reinterpret_cast<float *>(smem + U * KQ_UNIT);
    float *red = gs + 4 * U;   // [2][G][S][RWP], S > 1 only
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int s = wave % S, g = wave / S;
    const int lr = lane % LPR, rsub = lane / LPR;
    const int u = s * LPR + lr;
    const bool lv = u < U;
    const int row0 = blockIdx.x * rpw + g * RW + rsub;   // row of pass 0, step 0
    const int rend = min((blockIdx.x + 1) * rpw, M);
    const int npass = (rpw + RWG - 1) / RWG;

    // Every load below is unconditional: rows past the workgroup's last
    // re-read its last row and lanes past the row's last unit re-read unit
    // 0; their results are discarded.  A load under a branch would make the
    // compiler wait for all outstanding loads where the branch rejoins,
    // which serialises the prefetch with this pass's arithmetic.
    const int ul = lv ? u : 0;
    typename F::Unit buf[D + 1][RP];   // buf[0] = this pass, buf[i] = pass + i
    // output row of step p of a pass, and the weight row it reads
    auto orow = [&](int pass, int p) { return row0 + pass * RWG + (GLU ? 0 : p * RPP); };
    auto load = [&](typename F::Unit *dst, int pass) {
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const int r = min(orow(pass, p), rend - 1) + (GLU ? p * M : 0);
            F::load(W + (long long)r * rb, ul, dst[p]);
        }
    };
    KqStager<NT, kq_order<QT>(), MAXT, (PRO & 3)> xs;
    xs.load(x, U, pro);
    __builtin_amdgcn_sched_barrier(0);   // x's loads stay ahead of the weights'
#pragma unroll
    for (int i = 0; i < D; i++) load(buf[i], i);
    // PRO_RES: y[r] += the row's dot.  A pass's residual rows are loaded one
    // pass ahead and before the weights issued with them, so waiting for
    // them never waits for weights.
    float *ssred = red + (S > 1 ? 2 * G * S * RWP : 0);   // PRO_NORMD: S * G floats
    float rn = 1.f;                                       // PRO_NORMD: r
    auto res_load = [&](int pass, float *rv) {
        if constexpr ((PRO & PRO_RES) != 0) {
#pragma unroll
            for (int p = 0; p < RP; p++) rv[p] = y[min(orow(pass, p), rend - 1)];
        }
    };
    auto put = [&](int r, float v, float rv) {
        if constexpr ((PRO & PRO_RES) != 0) y[r] = rv + v;
        else if constexpr ((PRO & 3) == PRO_NORMD) y[r] = v * rn;
        else y[r] = v;
    };
    xs.apply(U, pro);
    xs.store(U, xd, gs);
    if constexpr ((PRO & 3) == PRO_NORMD) pro_ss_put(xs.ss, ssred);
    __syncthreads();
    KqX xr;
    kq_xload(xd, gs, ul, xr);
    if constexpr ((PRO & 3) == PRO_NORMD) rn = pro_ss_scale<S * G>(ssred, K, pro.eps);

    // Q2_K and Q8_0 rows in one slice: two passes per iteration with the
    // two buffers in alternating roles, so the ring needs no register moves
    // (12288x4096: Q2_K 8.1 -> 7.8 us, Q8_0 12.3 -> 11.9 us; Q3_K and Q5_K
    // measured 2-4% slower in this form, the three-slice shapes no faster)
    if constexpr (D == 1 && S == 1 &&
                  (QT == QT_Q2_K || QT == QT_GQ2_K || QT == QT_Q8_0 || QT == QT_GQ8_0)) {
        // reduce and store the rows of `cur` (pass `pass`)
        auto pass_rows = [&](const typename F::Unit *cur, int pass, const float *rv) {
            float acc[RP];
#pragma unroll
            for (int p = 0; p < RP; p++) {
                const int r = orow(pass, p);
                const float v = kq_dot<QT>(cur[p], xr, ul);
                acc[p] = group_sum<LPR>((r < rend && lv) ? v : 0.f);
            }
            if constexpr (GLU) {
                const int r = orow(pass, 0);
                if (lr == 0 && r < rend) y[r] = pro_swiglu(acc[0] * rn, acc[1] * rn);
            } else {
#pragma unroll
                for (int p = 0; p < RP; p++) {
                    const int r = orow(pass, p);
                    if (lr == 0 && r < rend) put(r, acc[p], rv[p]);
                }
            }
        };
        // npass is uniform in the workgroup, so the second pass's guard is too
        float rv0[RP], rv1[RP];
        res_load(0, rv0);   // behind pass 0's weights, which the first store waits for anyway
        for (int pass = 0; pass < npass; pass += 2) {
            res_load(pass + 1, rv1);
            load(buf[1], pass + 1);
            pass_rows(buf[0], pass, rv0);
            if (pass + 1 < npass) {
                res_load(pass + 2, rv0);
                load(buf[0], pass + 2);
                pass_rows(buf[1], pass + 1, rv1);
            }
        }
        return;
    }
    float rv[RP], rvn[RP];
    res_load(0, rv);   // behind pass 0's weights, which the first store waits for anyway
    for (int pass = 0; pass < npass; ++pass) {
        res_load(pass + 1, rvn);
        load(buf[D], pass + D);
        float acc[RP];
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const int r = orow(pass, p);
            const float v = kq_dot<QT>(buf[0][p], xr, ul);
            acc[p] = group_sum<LPR>((r < rend && lv) ? v : 0.f);
        }
        if constexpr (S > 1) {
            // the slices' partial sums meet in LDS; every slice adds them in
            // slice order (slice 0 stores)
            float *rbuf = red + (pass & 1) * (G * S * RWP);
#pragma unroll
            for (int p = 0; p < RP; p++)
                if (lr == 0) rbuf[(g * S + s) * RWP + p * RPP + rsub] = acc[p];
            __syncthreads();
#pragma unroll
            for (int p = 0; p < RP; p++) {
                float t = rbuf[(g * S) * RWP + p * RPP + rsub];
#pragma unroll
                for (int ss = 1; ss < S; ss++) t += rbuf[(g * S + ss) * RWP + p * RPP + rsub];
                acc[p] = t;
            }
        }
        if (s == 0) {
            if constexpr (GLU) {
                const int r = orow(pass, 0);
                if (lr == 0 && r < rend) y[r] = pro_swiglu(acc[0] * rn, acc[1] * rn);
            } else {
#pragma unroll
                for (int p = 0; p < RP; p++) {
                    const int r = orow(pass, p);
                    if (lr == 0 && r < rend) put(r, acc[p], rv[p]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < D; i++)
#pragma unroll
            for (int p = 0; p < RP; p++) buf[i][p] = buf[i + 1][p];
#pragma unroll
        for (int p = 0; p < RP; p++) rv[p] = rvn[p];
    }
}

// Rows of U units with 16 < U < 64, U not a power of two (K = 2560:
// U = 40), where a row slice of the next power of two would leave lanes
// idle, and tall matrices of 64-unit rows.  Segmented mapping: workgroup lane L takes
// unit L % U of row slot
// L / U, RB = NT / U rows per pass, so only NT % U lanes idle; a lane's unit
// is fixed, so its digits stay in registers as in k_mv_kq.  Row blocks of RB
// rows are dealt to the workgroups round-robin, the next block's weights in
// flight while the current one is reduced.  The partial sums meet in LDS
// (double-buffered by pass parity, one barrier per pass): 8 threads per
// row slot add every 8th partial, then a DPP sum over the 8.
template <int QT, int NW, int PRO, bool GLU>
__global__ __launch_bounds__(NW * 64) void k_mv_kq_seg(const uint8_t *__restrict__ W, int M, int K, long long rb,
                                                       const float *__restrict__ x, float *__restrict__ y,
                                                       MvPro pro) {
    using F = KqFmt<QT>;
    constexpr int NT = NW * 64, RP = GLU ? 2 : 1;   // RP: weight rows per lane and pass
    constexpr int MAXT = (16 * 64 + NT - 1) / NT;   // U <= 64
    extern __shared__ uint32_t smem[];
    const int U = K / 64, RB = NT / U;
    uint32_t *xd = smem;
    float *gs = reinterpret_cast<float *>(smem + U * KQ_UNIT);
    float *red = gs + 4 * U;   // [2][RP][NT]
    const int L = threadIdx.x, slot = L / U, u = L % U;   // slot >= RB: idle lane
    const int nblk = (M + RB - 1) / RB;
    const int npass = (nblk - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;   // >= 1: grid <= nblk
    auto block_row = [&](int pass) { return ((int)blockIdx.x + pass * (int)gridDim.x) * RB; };
    // loads are unconditional and their results for rows past M or idle
    // lanes never read: rows past M re-read row M - 1, idle lanes the
    // block's last row (whose lines the same instruction fetches anyway; a
    // row of the next block would be fetched twice)
    const int lslot = min(slot, RB - 1);
    typename F::Unit buf[2][RP];
    auto load = [&](typename F::Unit *dst, int pass) {
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const int r = min(block_row(pass) + lslot, M - 1) + (GLU ? p * M : 0);
            F::load(W + (long long)r * rb, u, dst[p]);
        }
    };
    KqStager<NT, kq_order<QT>(), MAXT, (PRO & 3)> xs;
    xs.load(x, U, pro);
    __builtin_amdgcn_sched_barrier(0);   // x's loads stay ahead of the weights'
    load(buf[0], 0);
    xs.apply(U, pro);
    xs.store(U, xd, gs);
    float *ssred = red + 2 * RP * NT;   // PRO_NORMD: NW floats
    if constexpr ((PRO & 3) == PRO_NORMD) pro_ss_put(xs.ss, ssred);
    __syncthreads();
    KqX xr;
    kq_xload(xd, gs, u, xr);
    float rn = 1.f;
    if constexpr ((PRO & 3) == PRO_NORMD) rn = pro_ss_scale<NW>(ssred, K, pro.eps);
    const int rs = L >> 3, part = L & 7;   // reduction: 8 threads per row slot
    for (int pass = 0; pass < npass; ++pass) {
        load(buf[1], pass + 1);
        float *rbuf = red + (pass & 1) * (RP * NT);
#pragma unroll
        for (int p = 0; p < RP; p++) rbuf[p * NT + L] = kq_dot<QT>(buf[0][p], xr, u);
        __syncthreads();
        float acc[RP];
#pragma unroll
        for (int p = 0; p < RP; p++) {
            float t = 0.f;
            if (rs < RB) {
#pragma unroll
                for (int j = 0; j < 8; j++)
                    if (part + 8 * j < U) t += rbuf[p * NT + rs * U + part + 8 * j];
            }
            acc[p] = group_sum<8>(t);
        }
        const int r = block_row(pass) + rs;
        if (part == 0 && rs < RB && r < M) {
            if constexpr (GLU) y[r] = pro_swiglu(acc[0] * rn, acc[1] * rn);
            else if constexpr ((PRO & 3) == PRO_NORMD) y[r] = acc[0] * rn;
            else y[r] = acc[0];
        }
#pragma unroll
        for (int p = 0; p < RP; p++) buf[0][p] = buf[1][p];
    }
}

template <int QT, int LPR, int S, int G, int R, int D, int PRO, bool GLU>
static hipError_t launch_kq(const void *W, int M, int K, const float *x, float *y, hipStream_t st, int grid,
                            int rpw, const MvPro &pro) {
    constexpr int RPP = 64 / LPR;
    const int U = K / 64;
    const long long rb = pro.rb ? pro.rb : (long long)(K / block_weights(QT)) * block_bytes(QT);
    constexpr int RP = GLU ? 2 : R;
    const size_t lds = (size_t)U * KQ_UNIT * 4 + (size_t)U * 16 + (S > 1 ? (size_t)2 * G * S * RP * RPP * 4 : 0) +
                       ((PRO & 3) == PRO_NORMD ? 32 * 4 : 0);
    if constexpr (S > 4) {
        // rows of more than 256 units stage more than 64 KiB of x: opted
        // into once per instantiation (gfx950 has 160 KiB of LDS per CU)
        static const hipError_t attr = hipFuncSetAttribute(
            (const void *)k_mv_kq<QT, LPR, S, G, R, D, PRO, GLU>, hipFuncAttributeMaxDynamicSharedMemorySize,
            (int)((size_t)S * 64 * (KQ_UNIT * 4 + 16) + 2 * G * S * RP * RPP * 4 + ((PRO & 3) == PRO_NORMD ? 32 * 4 : 0)));
        if (attr != hipSuccess) return attr;
    }
    hipLaunchKernelGGL((k_mv_kq<QT, LPR, S, G, R, D, PRO, GLU>), dim3(grid), dim3(S * G * 64), lds, st,
                       (const uint8_t *)W, M, K, rb, x, y, rpw, pro);
    return hipGetLastError();
}

#ifndef KQ_SEG_NW
#define KQ_SEG_NW 16
#endif
#ifndef KQ_SEG_WPC
#define KQ_SEG_WPC 1
#endif
template <int QT, int NW, int PRO, bool GLU>
static hipError_t launch_kq_seg(const void *W, int M, int K, const float *x, float *y, hipStream_t st, int n_cu,
                                const MvPro &pro) {
    if constexpr ((PRO & PRO_RES) != 0) {
        return hipErrorNotSupported;   // no residual epilogue in the segmented kernel
    } else {
    constexpr int NT = NW * 64, RP = GLU ? 2 : 1;
    const int U = K / 64, RB = NT / U;
    const long long nblk = ((long long)M + RB - 1) / RB, cap = (long long)n_cu * KQ_SEG_WPC;
    const int grid = (int)(nblk < cap ? nblk : cap);
    const long long rb = pro.rb ? pro.rb : (long long)(K / block_weights(QT)) * block_bytes(QT);
    const size_t lds = (size_t)U * KQ_UNIT * 4 + (size_t)U * 16 + (size_t)2 * RP * NT * 4 +
                       ((PRO & 3) == PRO_NORMD ? NW * 4 : 0);
    hipLaunchKernelGGL((k_mv_kq_seg<QT, NW, PRO, GLU>), dim3(grid), dim3(NT), lds, st, (const uint8_t *)W, M, K, rb,
                       x, y, pro);
    return hipGetLastError();
    }
}

// Launch shape for one row slice width: G row groups of S waves, at most
// KQ_WG_PER_CU workgroups per CU (each stages x once), rows split evenly over
// the workgroups; each wave streams R = KQ_R rows per pass with the next
// KQ_D passes' weights in flight.
template <int QT, int LPR, int S, int G, int PRO, bool GLU, int WPC = KQ_WG_PER_CU>
static hipError_t launch_kq_shape(const void *W, int M, int K, const float *x, float *y, hipStream_t st, int n_cu,
                                  const MvPro &pro) {
    constexpr int RPP = 64 / LPR, R = KQ_R, D = KQ_D, RL = GLU ? 1 : R;
    const long long cap = (long long)n_cu * WPC;
    const long long need = ((long long)M + G * RL * RPP - 1) / (G * RL * RPP);
    const int grid = (int)(need < cap ? need : cap);
    const int rpw = (M + grid - 1) / grid;
    return launch_kq<QT, LPR, S, G, R, D, PRO, GLU>(W, M, K, x, y, st, grid, rpw, pro);
}

template <int QT, int PRO, bool GLU>
static hipError_t launch_kq_q(const void *W, int M, int K, const float *x, float *y, hipStream_t st, int n_cu,
                              const MvPro &pro) {
    const int U = K / 64;
    constexpr int NW = KQ_NW, G3 = KQ_G3;
    // 16 < U < 32, not a power of two (K = 1536: U = 24): the segmented
    // row mapping, as for 32 < U < 64 below (8960x1536: Q3_K 6.7 -> 5.5 us,
    // Q5_K 6.8 -> 5.8, Q2_K 5.4 -> 4.7; at U = 12 the 16-lane row slices
    // stay faster: Q5_K 4096x768 4.4 against 5.1 us)
    if constexpr (QT != QT_Q8_0 && QT != QT_GQ8_0)
        if (U > 16 && U < 32 && (U & (U - 1)) != 0)
            return launch_kq_seg<QT, KQ_SEG_NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    if (U <= 4) return launch_kq_shape<QT, 4, 1, NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    if (U <= 8) return launch_kq_shape<QT, 8, 1, NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    if (U <= 16) return launch_kq_shape<QT, 16, 1, NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    if (U <= 32) return launch_kq_shape<QT, 32, 1, NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    // Tall matrices of 64-unit rows: the segmented mapping, 16 rows per
    // workgroup pass (151936x4096: Q5_K 82.0 -> 79.5 us, Q2_K 59.4 -> 56.1,
    // Q8_0 65536x4096 52.5 -> 51.0; up to 24576 rows the row slices are as
    // fast or faster, except Q3_K in the reference layout: 12288x4096
    // 10.1 -> 9.5-9.8 us, ggml's 10.7 -> 11.1); Q6_K keeps
    // the 8-wave shape below (99.3 against 104 us segmented)
    if constexpr (QT != QT_Q6_K && QT != QT_GQ6_K)
        if (U == 64 && M > (QT == QT_Q3_K ? 8192 : 32768))
            return launch_kq_seg<QT, KQ_SEG_NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    // Q6_K's tall matrices (the lm_head): 8-wave workgroups, up to 4 per CU
    // (151936x4096: 99.5 against 106 us with one 16-wave workgroup per CU)
    if constexpr (QT == QT_Q6_K || QT == QT_GQ6_K)
        if (U == 64 && M > 65536) return launch_kq_shape<QT, 64, 1, 8, PRO, GLU, 4>(W, M, K, x, y, st, n_cu, pro);
    // 32 < U < 64, not a power of two: the segmented row mapping (Q8_0
    // keeps the row slice with two passes per iteration, 7.97 against
    // 8.47 us at 9728x2560)
    if constexpr (QT != QT_Q8_0 && QT != QT_GQ8_0)
        if (U < 64 && (U & (U - 1)) != 0) return launch_kq_seg<QT, KQ_SEG_NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    if (U <= 64) return launch_kq_shape<QT, 64, 1, NW, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    if (U <= 128) return launch_kq_shape<QT, 64, 2, NW / 2, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    if (U <= 192) {
        // three slices: 5 row groups when that takes fewer passes than G3
        // over a workgroup's rows (2560 rows on 256 CUs: 10 rows, 2 passes
        // instead of 3; 2560x9728 Q5_K 8.9 -> 8.5 us), else G3 (4096 rows:
        // 4 passes either way, and 5 groups were 7-16% slower)
        const long long rpw = ((long long)M + n_cu - 1) / n_cu;
        if ((rpw + 4) / 5 < (rpw + G3 - 1) / G3)
            return launch_kq_shape<QT, 64, 3, 5, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
        return launch_kq_shape<QT, 64, 3, G3, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    }
    if (U <= 256) return launch_kq_shape<QT, 64, 4, NW / 4, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    // K up to 32768 for plain matvecs (the fused prologue's registers do not
    // fit 8 slices): 6 or 8 slices of 64 units, two row groups
    if constexpr ((PRO & 3) == PRO_NONE && !GLU) {
        if (U <= 384) return launch_kq_shape<QT, 64, 6, 2, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
        if (U <= 512) return launch_kq_shape<QT, 64, 8, 2, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    }
    return hipErrorNotSupported;
}

// Returns hipErrorNotSupported for formats or shapes this kernel does not
// cover (K must be a multiple of 64 and at most 32768; at most 16384 with a
// prologue or the GLU epilogue).
template <int PRO, bool GLU>
static hipError_t launch_matvec_kq_p(int qt, const void *W, int M, int K, const float *x, float *y, hipStream_t st,
                                     int n_cu, const MvPro &pro) {
    if (K % 64 || K > TBQ_MAX_K || K <= 0) return hipErrorNotSupported;
    const bool sb256 = block_weights(qt) == 256;
    if (sb256 && K % 256) return hipErrorNotSupported;
    switch (qt) {
    case QT_Q2_K: return launch_kq_q<QT_Q2_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_Q3_K: return launch_kq_q<QT_Q3_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_Q4_K: return launch_kq_q<QT_Q4_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_Q5_K: return launch_kq_q<QT_Q5_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_Q6_K: return launch_kq_q<QT_Q6_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_Q8_0: return launch_kq_q<QT_Q8_0, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_Q4_0: return launch_kq_q<QT_Q4_0, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_Q8_K: return launch_kq_q<QT_Q8_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_GQ2_K: return launch_kq_q<QT_GQ2_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_GQ3_K: return launch_kq_q<QT_GQ3_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_GQ4_K: return launch_kq_q<QT_GQ4_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_GQ5_K: return launch_kq_q<QT_GQ5_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_GQ6_K: return launch_kq_q<QT_GQ6_K, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_GQ8_0: return launch_kq_q<QT_GQ8_0, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    case QT_GQ4_0: return launch_kq_q<QT_GQ4_0, PRO, GLU>(W, M, K, x, y, st, n_cu, pro);
    default: return hipErrorNotSupported;
    }
}

// ---------------------------------------------------------------------------
// MoE decode experts on the same int-dot units, for the K-quant formats
// other than Q4_K (tbq_moe_q4k.hip has the Q4_K kernels).  One kernel per
// phase, as the Q4_K ones: a layer whose tensors differ in format (llama.cpp
// mixes give down a wider format than gate/up) runs each phase in its own.
//
// k_moe_gate_up_kq: act[pair][r] = silu(W_gate[e] x_t)[r] * (W_up[e] x_t)[r]
// (layer4/tb_infer.c:810-812, tb_swiglu :130-135) for gate and up in one
// format.  grid = (F / 8, T*k); wave w takes output row 8*bx + w, lanes
// 0..31 its gate row and 32..63 its up row, UPL units per lane.
// k_moe_down_kq: out[t][r] = resid[t][r] + sum over slots in slot order of
// w_s * (W_down[e_s] act[t*k + s])[r] (:815-831, :876).  grid = (H / 4, T);
// the token's k activation vectors (k*F contiguous floats) are staged as one
// vector of k*F/64 units, each 16-lane row of a wave takes one (row, slot)
// dot, and one lane per row adds the slots in slot order.
// An expert index outside [0, E) (never produced by the router) reads expert
// 0 and contributes 0.
// ---------------------------------------------------------------------------
constexpr int ME_THREADS = 512;
constexpr int MD_ROWS = 4, MD_LPR = 16;
constexpr int MD_MAX_UNITS = 256;   // staged units of the down kernel (k * F / 64)

template <int QT, int UPL, int MAXT>
__global__ __launch_bounds__(ME_THREADS) void k_moe_gate_up_kq(const uint8_t *__restrict__ gate,
                                                               const uint8_t *__restrict__ up, long long rb,
                                                               const float *__restrict__ xn,
                                                               const int *__restrict__ sel_idx,
                                                               const int *__restrict__ order,
                                                               const int *__restrict__ nvalid, int H, int F, int E,
                                                               int k, float *__restrict__ act) {
    using Fm = KqFmt<QT>;
    extern __shared__ uint32_t smem[];
    const int U = H / 64;
    uint32_t *xd = smem;
    float *gs = reinterpret_cast<float *>(smem + U * KQ_UNIT);
    // with an order list (expert-ordered valid pairs), column y runs pair order[y]
    if (order && (int)blockIdx.y >= *nvalid) return;   // workgroup-uniform
    const int pair = order ? order[blockIdx.y] : blockIdx.y, t = pair / k, s = pair % k;
    const int e_sel = sel_idx[t * 8 + s];
    const bool ev = (unsigned)e_sel < (unsigned)E;
    const int e = ev ? e_sel : 0;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lr = lane & 31, half = lane >> 5;
    const int r = blockIdx.x * (ME_THREADS / 64) + wave;   // output row (F % 8 == 0)
    const uint8_t *row = (half ? up : gate) + ((long long)e * F + r) * rb;
    KqStager<ME_THREADS, kq_order<QT>(), MAXT> xs;
    xs.load(xn + (long long)t * H, U);
    __builtin_amdgcn_sched_barrier(0);   // x's loads stay ahead of the weights'
    typename Fm::Unit w[UPL];
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        const int u = lr + 32 * i;
        Fm::load(row, u < U ? u : 0, w[i]);
    }
    xs.store(U, xd, gs);
    __syncthreads();
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        const int u = lr + 32 * i;
        if (u < U) {
            KqX x;
            kq_xload(xd, gs, u, x);
            acc += kq_dot<QT>(w[i], x, u);
        }
    }
    acc = group_sum<32>(acc);
    const float uv = __shfl(acc, 32);
    if (lane == 0) {
        const float g = acc;
        const float den = 1.0f + expf_glibc(-g);
        const float sg = g / den;
        act[(long long)pair * F + r] = ev ? sg * uv : 0.f;
    }
}

template <int QT, int UPL, int MAXT>
__global__ __launch_bounds__(ME_THREADS) void k_moe_down_kq(const uint8_t *__restrict__ down, long long rb,
                                                            const float *__restrict__ act,
                                                            const int *__restrict__ sel_idx,
                                                            const float *__restrict__ sel_w,
                                                            const float *__restrict__ resid, int H, int F, int E,
                                                            int k, float *__restrict__ out) {
    using Fm = KqFmt<QT>;
    extern __shared__ uint32_t smem[];
    const int U = F / 64, NU = k * U;
    uint32_t *xd = smem;
    float *gs = reinterpret_cast<float *>(smem + NU * KQ_UNIT);
    float *yv = gs + 4 * NU;   // [slot][MD_ROWS]
    const int t = blockIdx.y, r0 = blockIdx.x * MD_ROWS;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lr = lane & 15;
    const int d = wave * (64 / MD_LPR) + (lane >> 4);   // dot (row r0 + d / k, slot d % k), d < 32
    const bool dv = d < MD_ROWS * k;
    const int rd = dv ? d / k : 0, sd = dv ? d % k : 0;
    const int e_sel = sel_idx[t * 8 + sd];
    const bool ev = dv && (unsigned)e_sel < (unsigned)E;
    const int e = ev ? e_sel : 0;
    const uint8_t *row = down + ((long long)e * H + r0 + rd) * rb;
    KqStager<ME_THREADS, kq_order<QT>(), MAXT> xs;
    xs.load(act + (long long)t * k * F, NU);
    __builtin_amdgcn_sched_barrier(0);
    typename Fm::Unit w[UPL];
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        const int u = lr + MD_LPR * i;
        Fm::load(row, u < U ? u : 0, w[i]);
    }
    xs.store(NU, xd, gs);
    __syncthreads();
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        const int u = lr + MD_LPR * i;
        if (u < U) {
            KqX x;
            kq_xload(xd, gs, sd * U + u, x);
            acc += kq_dot<QT>(w[i], x, u);
        }
    }
    acc = group_sum<MD_LPR>(acc);
    if (lr == 0 && dv) yv[sd * MD_ROWS + rd] = ev ? acc : 0.f;
    __syncthreads();
    if (threadIdx.x < MD_ROWS) {
        const int rr = threadIdx.x, r = r0 + rr;
        float a = 0.f;
        for (int sl = 0; sl < k; sl++) {
            if ((unsigned)sel_idx[t * 8 + sl] >= (unsigned)E) continue;   // never produced by the router
            const float pr = sel_w[t * 8 + sl] * yv[sl * MD_ROWS + rr];
            a = a + pr;
        }
        out[(long long)t * H + r] = resid[(long long)t * H + r] + a;
    }
}

// Batches in expert order (k_group's pair list): y[pair][r] = W_down[e] .
// act[pair] over MDP_ROWS rows per workgroup, so the workgroups of the pairs
// that share an expert run back to back and find its rows in L2; k_combine
// then adds the slots in slot order.  grid = (H / MDP_ROWS, T*k).
#ifndef TBQ_MDP_THREADS
#define TBQ_MDP_THREADS 256
#endif
#ifndef TBQ_MDP_ROWS
#define TBQ_MDP_ROWS 128
#endif
constexpr int MDP_THREADS = TBQ_MDP_THREADS, MDP_ROWS = TBQ_MDP_ROWS;
constexpr int MDP_PASSES = MDP_ROWS / (MDP_THREADS / MD_LPR);
static_assert(MDP_ROWS % (MDP_THREADS / MD_LPR) == 0, "whole passes");

template <int QT, int UPL, int MAXT>
__global__ __launch_bounds__(MDP_THREADS) void k_moe_down_pair_kq(const uint8_t *__restrict__ down, long long rb,
                                                                 const float *__restrict__ act,
                                                                 const int *__restrict__ sel_idx,
                                                                 const int *__restrict__ order,
                                                                 const int *__restrict__ nvalid, int H, int F,
                                                                 int E, int k, float *__restrict__ y) {
    using Fm = KqFmt<QT>;
    extern __shared__ uint32_t smem[];
    const int U = F / 64;
    uint32_t *xd = smem;
    float *gs = reinterpret_cast<float *>(smem + U * KQ_UNIT);
    if ((int)blockIdx.y >= *nvalid) return;   // workgroup-uniform
    const int pair = order[blockIdx.y];
    const int e = sel_idx[(pair / k) * 8 + pair % k];
    if ((unsigned)e >= (unsigned)E) return;   // the list holds valid pairs only
    const int lr = threadIdx.x & 15, rl = threadIdx.x >> 4;   // row of the pass
    const int r0 = blockIdx.x * MDP_ROWS;
    KqStager<MDP_THREADS, kq_order<QT>(), MAXT> xs;
    xs.load(act + (long long)pair * F, U);
    __builtin_amdgcn_sched_barrier(0);
    // PB passes' weights in registers at a time: all four at one unit per
    // lane, fewer at more (four passes of four Q6_K units would spill)
#ifndef MDP_PB_BIG
#define MDP_PB_BIG 2
#endif
    constexpr int PB = UPL >= 4 ? 1 : (UPL >= 2 ? 2 : (sizeof(typename Fm::Unit) > 48 ? MDP_PB_BIG : MDP_PASSES));
    typename Fm::Unit w[PB][UPL];
    auto wload = [&](int p0) {
#pragma unroll
        for (int p = 0; p < PB; p++) {
            const uint8_t *row = down + ((long long)e * H + r0 + (MDP_THREADS / MD_LPR) * (p0 + p) + rl) * rb;
#pragma unroll
            for (int i = 0; i < UPL; i++) {
                const int u = lr + MD_LPR * i;
                Fm::load(row, u < U ? u : 0, w[p][i]);
            }
        }
    };
    wload(0);
    xs.store(U, xd, gs);
    __syncthreads();
#pragma unroll
    for (int p0 = 0; p0 < MDP_PASSES; p0 += PB) {
        if (p0 > 0) wload(p0);
#pragma unroll
        for (int p = 0; p < PB; p++) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < UPL; i++) {
                const int u = lr + MD_LPR * i;
                if (u < U) {
                    KqX x;
                    kq_xload(xd, gs, u, x);
                    acc += kq_dot<QT>(w[p][i], x, u);
                }
            }
            acc = group_sum<MD_LPR>(acc);
            if (lr == 0) y[(long long)pair * H + r0 + (MDP_THREADS / MD_LPR) * (p0 + p) + rl] = acc;
        }
    }
}

template <int QT, int UPL, int MAXT>
static hipError_t launch_moe_gate_up_kq_t(const MoeArgs &a, bool grouped, hipStream_t st) {
    const long long rb = (long long)(a.H / block_weights(QT)) * block_bytes(QT);
    const int U = a.H / 64;
    const size_t lds = (size_t)U * KQ_UNIT * 4 + (size_t)U * 16;
    const int *order = grouped ? a.grp + 1 + 3 * a.E : nullptr, *nvalid = grouped ? order + a.T * a.k : nullptr;
    hipLaunchKernelGGL((k_moe_gate_up_kq<QT, UPL, MAXT>), dim3(a.F / (ME_THREADS / 64), a.T * a.k), dim3(ME_THREADS),
                       lds, st, (const uint8_t *)a.gate, (const uint8_t *)a.up, rb, a.xn, a.sel_idx, order, nvalid,
                       a.H, a.F, a.E, a.k, a.act);
    return hipGetLastError();
}

template <int QT, int UPL, int MAXT>
static hipError_t launch_moe_down_pair_kq_t(const MoeArgs &a, hipStream_t st) {
    const long long rb = (long long)(a.F / block_weights(QT)) * block_bytes(QT);
    const int U = a.F / 64;
    const int *order = a.grp + 1 + 3 * a.E, *nvalid = order + a.T * a.k;
    const size_t lds = (size_t)U * KQ_UNIT * 4 + (size_t)U * 16;
    hipLaunchKernelGGL((k_moe_down_pair_kq<QT, UPL, MAXT>), dim3(a.H / MDP_ROWS, a.T * a.k), dim3(MDP_THREADS), lds, st,
                       (const uint8_t *)a.down, rb, a.act, a.sel_idx, order, nvalid, a.H, a.F, a.E, a.k, a.y);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_combine(a, st);
}

template <int QT, int UPL, int MAXT>
static hipError_t launch_moe_down_kq_t(const MoeArgs &a, hipStream_t st) {
    const long long rb = (long long)(a.F / block_weights(QT)) * block_bytes(QT);
    const int NU = a.k * (a.F / 64);
    const size_t lds = (size_t)NU * KQ_UNIT * 4 + (size_t)NU * 16 + 8 * MD_ROWS * 4;
    hipLaunchKernelGGL((k_moe_down_kq<QT, UPL, MAXT>), dim3(a.H / MD_ROWS, a.T), dim3(ME_THREADS), lds, st,
                       (const uint8_t *)a.down, rb, a.act, a.sel_idx, a.sel_w, a.resid, a.H, a.F, a.E, a.k, a.out);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_moe_gate_up_kq_q(const MoeArgs &a, bool grouped, hipStream_t st) {
    const int U = a.H / 64;   // x staged in LDS: U * 16 tasks over 512 threads
    if (U <= 32) return launch_moe_gate_up_kq_t<QT, 1, 1>(a, grouped, st);
    if (U <= 64) return launch_moe_gate_up_kq_t<QT, 2, 2>(a, grouped, st);
    if (U <= 128) return launch_moe_gate_up_kq_t<QT, 4, 4>(a, grouped, st);
    return hipErrorNotSupported;
}

template <int QT>
static hipError_t launch_moe_down_kq_q(const MoeArgs &a, bool grouped, hipStream_t st) {
    const int U = a.F / 64, NU = a.k * U;
    if (grouped) {   // per pair in expert order: one activation vector staged
        if (a.H % MDP_ROWS) return hipErrorNotSupported;
        constexpr int T = MDP_THREADS;   // x staged in LDS: U * 16 tasks
        if (U <= 16) return launch_moe_down_pair_kq_t<QT, 1, (256 + T - 1) / T>(a, st);
        if (U <= 32) return launch_moe_down_pair_kq_t<QT, 2, (512 + T - 1) / T>(a, st);
        if (U <= 64) return launch_moe_down_pair_kq_t<QT, 4, (1024 + T - 1) / T>(a, st);
        return hipErrorNotSupported;
    }
    if (NU > MD_MAX_UNITS) return hipErrorNotSupported;
    const int maxt = (16 * NU + ME_THREADS - 1) / ME_THREADS;
    if (U <= 16) {
        if (maxt <= 2) return launch_moe_down_kq_t<QT, 1, 2>(a, st);
        if (maxt <= 4) return launch_moe_down_kq_t<QT, 1, 4>(a, st);
        return launch_moe_down_kq_t<QT, 1, 8>(a, st);
    }
    if (U <= 32) {
        if (maxt <= 4) return launch_moe_down_kq_t<QT, 2, 4>(a, st);
        return launch_moe_down_kq_t<QT, 2, 8>(a, st);
    }
    return hipErrorNotSupported;
}

#define TBQ_MOE_KQ_SWITCH(qt, FN)                                             \
    switch (qt) {                                                            \
    case QT_Q2_K: return FN<QT_Q2_K>(a, grouped, st);                        \
    case QT_Q3_K: return FN<QT_Q3_K>(a, grouped, st);                        \
    case QT_Q4_K: return FN<QT_Q4_K>(a, grouped, st);                        \
    case QT_Q5_K: return FN<QT_Q5_K>(a, grouped, st);                        \
    case QT_Q6_K: return FN<QT_Q6_K>(a, grouped, st);                        \
    case QT_Q8_0: return FN<QT_Q8_0>(a, grouped, st);                        \
    case QT_GQ2_K: return FN<QT_GQ2_K>(a, grouped, st);                      \
    case QT_GQ3_K: return FN<QT_GQ3_K>(a, grouped, st);                      \
    case QT_GQ4_K: return FN<QT_GQ4_K>(a, grouped, st);                      \
    case QT_GQ5_K: return FN<QT_GQ5_K>(a, grouped, st);                      \
    case QT_GQ6_K: return FN<QT_GQ6_K>(a, grouped, st);                      \
    case QT_GQ8_0: return FN<QT_GQ8_0>(a, grouped, st);                      \
    default: return hipErrorNotSupported;                                    \
    }

hipError_t launch_moe_gate_up_kq(const MoeArgs &a, bool grouped, hipStream_t st) {
    if (a.qg != a.qu || a.F % (ME_THREADS / 64)) return hipErrorNotSupported;
    TBQ_MOE_KQ_SWITCH(a.qg, launch_moe_gate_up_kq_q)
}

hipError_t launch_moe_down_kq(const MoeArgs &a, bool grouped, hipStream_t st) {
    if (a.H % MD_ROWS || a.k > 8) return hipErrorNotSupported;
    TBQ_MOE_KQ_SWITCH(a.qd, launch_moe_down_kq_q)
}
#undef TBQ_MOE_KQ_SWITCH

hipError_t launch_matvec_kq(int qt, const void *W, int M, int K, const float *x, float *y, hipStream_t st, int n_cu) {
    return launch_matvec_kq_p<PRO_NONE, false>(qt, W, M, K, x, y, st, n_cu, MvPro{});
}

// With a staging prologue and epilogue (mode = PRO_* | MV_GLU; with MV_GLU,
// W holds 2M rows).
hipError_t launch_matvec_kq_pro(int mode, const MvPro &pro, int qt, const void *W, int M, int K, const float *x,
                                float *y, hipStream_t st, int n_cu) {
    switch (mode) {
    case PRO_NONE: return launch_matvec_kq_p<PRO_NONE, false>(qt, W, M, K, x, y, st, n_cu, pro);
    case PRO_NORM: return launch_matvec_kq_p<PRO_NORM, false>(qt, W, M, K, x, y, st, n_cu, pro);
    case PRO_NORM | MV_GLU: return launch_matvec_kq_p<PRO_NORM, true>(qt, W, M, K, x, y, st, n_cu, pro);
    case PRO_NORMD: return launch_matvec_kq_p<PRO_NORMD, false>(qt, W, M, K, x, y, st, n_cu, pro);
    case PRO_NORMD | MV_GLU: return launch_matvec_kq_p<PRO_NORMD, true>(qt, W, M, K, x, y, st, n_cu, pro);
    case PRO_RES: return launch_matvec_kq_p<PRO_RES, false>(qt, W, M, K, x, y, st, n_cu, pro);
    default: return hipErrorNotSupported;
    }
}

}  // namespace tbq
