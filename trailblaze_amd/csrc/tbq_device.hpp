// tbq_device.hpp -- shared device code for the gfx950 K-quant / MoE kernels.
//
// Everything here is compiled with -ffp-contract=off: an expression a*b+c is
// a multiply and an add, each rounded, unless the code calls fmaf()
// explicitly.  The dequant path relies on that to reproduce the reference's
// roundings bit for bit (layer4/tb_gguf.c is built with -std=c11, which does
// not contract either).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tbq {

// ggml type ids used by the reference (layer4/tb_gguf.h:24).
enum QType : int {
    QT_F32 = 0, QT_F16 = 1, QT_Q4_0 = 2, QT_Q8_0 = 8, QT_Q2_K = 10, QT_Q3_K = 11,
    QT_Q4_K = 12, QT_Q5_K = 13, QT_Q6_K = 14, QT_Q8_K = 15, QT_BF16 = 30,
    // ggml's own on-disk layouts (QT_GGML | ggml id): the block fields sit at
    // the same byte offsets as in the reference's layouts, but quants, scales
    // and fp16 fields are read as ggml reads them.  F32, BF16 and Q8_K read
    // the same in both and are canonicalised to their plain ids by the host.
    QT_GGML = 0x100,
    QT_GF16 = QT_GGML | QT_F16, QT_GQ4_0 = QT_GGML | QT_Q4_0, QT_GQ8_0 = QT_GGML | QT_Q8_0,
    QT_GQ2_K = QT_GGML | QT_Q2_K, QT_GQ3_K = QT_GGML | QT_Q3_K, QT_GQ4_K = QT_GGML | QT_Q4_K,
    QT_GQ5_K = QT_GGML | QT_Q5_K, QT_GQ6_K = QT_GGML | QT_Q6_K
};

// weights / bytes per block, layer4/tb_gguf.c:380-394 (the same for both
// layouts of a format).
__host__ __device__ constexpr int block_weights(int qt) {
    return ((qt & 0xFF) == QT_F32 || (qt & 0xFF) == QT_F16 || (qt & 0xFF) == QT_BF16) ? 1
         : ((qt & 0xFF) == QT_Q4_0 || (qt & 0xFF) == QT_Q8_0) ? 32 : 256;
}
__host__ __device__ constexpr int block_bytes(int qt) {
    return (qt & 0xFF) == QT_F32 ? 4 : ((qt & 0xFF) == QT_F16 || (qt & 0xFF) == QT_BF16) ? 2
         : (qt & 0xFF) == QT_Q4_0 ? 18 : (qt & 0xFF) == QT_Q8_0 ? 34 : (qt & 0xFF) == QT_Q2_K ? 84
         : (qt & 0xFF) == QT_Q3_K ? 110 : (qt & 0xFF) == QT_Q4_K ? 144 : (qt & 0xFF) == QT_Q5_K ? 176
         : (qt & 0xFF) == QT_Q6_K ? 210 : (qt & 0xFF) == QT_Q8_K ? 292 : 0;
}

// A ggml-layout id of a format whose reading is the same in both layouts
// (F32, BF16, Q8_K) becomes the plain id; every other id is returned as is.
__host__ __device__ constexpr int canon_qt(int qt) {
    return ((qt & QT_GGML) && ((qt & 0xFF) == QT_F32 || (qt & 0xFF) == QT_BF16 || (qt & 0xFF) == QT_Q8_K))
               ? (qt & 0xFF) : qt;
}

// fp16 -> fp32 exactly as layer4/tb_gguf.c:92-101 decodes it.  A zero
// exponent keeps the mantissa in place under a zero f32 exponent (subnormal
// halves become m*2^-136); exponent 31 becomes the f32 inf/nan exponent.
// Integer bit work only -- v_cvt_f32_f16 would decode subnormals correctly
// and so differ from the reference.
__host__ __device__ __forceinline__ float f16_ref(uint32_t h) {
    uint32_t s = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits = e == 0 ? (s | (m << 13))
                  : e == 31 ? (s | 0x7F800000u | (m << 13))
                  : (s | ((e + 112u) << 23) | (m << 13));
    return __builtin_bit_cast(float, bits);
}

// fp16 -> fp32 as IEEE 754 defines it (ggml's layouts): subnormal halves
// are m*2^-24 (exact in fp32: m < 2^10), the rest as f16_ref.  Integer and
// exact fp32 work only, independent of the FP16 denormal mode.
__host__ __device__ __forceinline__ float f16_ieee(uint32_t h) {
    const uint32_t e = (h >> 10) & 0x1Fu;
    if (e == 0) {
        const float v = (float)(h & 0x3FFu) * 0x1p-24f;
        return (h & 0x8000u) ? -v : v;
    }
    return f16_ref(h);
}

// The fp16 decoder of a format: IEEE for the ggml layouts.
template <int QT>
__host__ __device__ __forceinline__ float f16_of(uint32_t h) {
    if constexpr ((QT & QT_GGML) != 0) return f16_ieee(h);
    else return f16_ref(h);
}

// The same decoders for arithmetic kernels, on both halves of a dword (lo =
// bits 0-15).  The hardware conversion (v_cvt_f32_f16) gives exactly the
// decoders' bits for zero and normal halves, the fields real scales hold;
// when any active lane of the wave holds a subnormal, inf or nan half
// (exponent 0 with a nonzero mantissa, or exponent 31) the whole wave takes
// the integer decoders instead.  The branch is wave-uniform.
template <bool IEEE = false>
__device__ __forceinline__ void f16x2_dec(uint32_t h, float &lo, float &hi) {
    const uint32_t a = h & 0x7FFFu, b = (h >> 16) & 0x7FFFu;
    const bool odd = (a - 1u < 0x3FFu) | (a >= 0x7C00u) | (b - 1u < 0x3FFu) | (b >= 0x7C00u);
    if (__builtin_amdgcn_ballot_w64(odd) != 0) {
        lo = IEEE ? f16_ieee(h & 0xFFFFu) : f16_ref(h & 0xFFFFu);
        hi = IEEE ? f16_ieee(h >> 16) : f16_ref(h >> 16);
    } else {
        lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
        hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(h >> 16));
    }
}
template <bool IEEE = false>
__device__ __forceinline__ float f16_dec(uint32_t h) {
    const uint32_t a = h & 0x7FFFu;
    const bool odd = (a - 1u < 0x3FFu) | (a >= 0x7C00u);
    if (__builtin_amdgcn_ballot_w64(odd) != 0) return IEEE ? f16_ieee(h & 0xFFFFu) : f16_ref(h & 0xFFFFu);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

__host__ __device__ __forceinline__ float bf16_ref(uint32_t b) {
    return __builtin_bit_cast(float, b << 16);
}

// ---------------------------------------------------------------------------
// expf, bit-identical to glibc 2.35's expf on every float input.
//
// Method: the table-driven expf of ARM's optimized-routines (Szabolcs Nagy,
// 2017; adopted by glibc 2.27): x*N/ln2 = k + r with N = 32 and |r| <= 1/2;
// exp(x) = 2^(k/N) * 2^(r/N), where 2^(k/N) is a table value with k/N's
// integer part added into the exponent bits, and 2^(r/N) is a cubic
// polynomial in r, all evaluated in double (three explicit fmas, as the
// FMA-enabled x86-64 build evaluates it) and rounded once to float.  The
// table and coefficients are reproduced from that published method; one
// table entry (index 31) carries an offset of 24 ulp so the results match
// glibc's on all 2^32 inputs, which tests/ verify exhaustively on the host
// and on a large sample on the GPU.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float expf_glibc(float x) {
    constexpr int TB = 5, N = 1 << TB;
    const uint64_t T[N] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4558ull};
    const double C0 = 0x1.c6af84b912394p-5 / N / N / N;
    const double C1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double C2 = 0x1.62e42ff0c52d6p-1 / N;
    const double InvLn2N = 0x1.71547652b82fep+0 * N;
    const double Shift = 0x1.8p+52;

    uint32_t ux = __builtin_bit_cast(uint32_t, x);
    uint32_t abstop = (ux >> 20) & 0x7FFu;
    if (abstop >= 0x42Bu) {               // |x| >= 88, inf or nan
        if (ux == 0xFF800000u) return 0.0f;                 // -inf
        if (abstop >= 0x7F8u) return x + x;                 // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_huge_valf(); // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                 // underflow
    }
    double xd = (double)x;
    double z = InvLn2N * xd;
    double kd = z + Shift;
    uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= Shift;
    double r = z - kd;
    uint64_t t = T[ki % N];
    t += ki << (52 - TB);
    double s = __builtin_bit_cast(double, t);
    double p = __builtin_fma(C0, r, C1);
    double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}

// ---------------------------------------------------------------------------
// Wave-level helpers (wave64).
// ---------------------------------------------------------------------------
// Cross-lane moves that stay in the VALU (no LDS crossbar round trip):
// DPP quad_perm xor 1 / xor 2, row_half_mirror (lane i <-> 7-i within 8),
// row_mirror (i <-> 15-i within 16); gfx950's permlane16/32 swaps pair
// 16-lane rows 0<->1, 2<->3 and the two 32-lane halves.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QXOR1 = 0xB1, DPP_QXOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

// The swap builtins return both exchanged operands as a 2-vector.  Its
// elements are copied into scalars before any bit cast: this clang lowers
// __builtin_bit_cast of a vector element r[1] as a load from the vector's
// first element.
__device__ __forceinline__ float swap16_sum(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float swap32_sum(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float swap16_max(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float swap32_max(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}

// Max over the whole wave (all 64 lanes active); every lane gets it.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<DPP_QXOR1>(v));
    v = fmaxf(v, dpp_f32<DPP_QXOR2>(v));
    v = fmaxf(v, dpp_f32<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f32<DPP_MIRROR>(v));
    v = swap16_max(v);
    return swap32_max(v);
}

// Min over aligned groups of 8 lanes; every lane of a group gets it.
__device__ __forceinline__ float group8_min(float v) {
    v = fminf(v, dpp_f32<DPP_QXOR1>(v));
    v = fminf(v, dpp_f32<DPP_QXOR2>(v));
    return fminf(v, dpp_f32<DPP_HALF_MIRROR>(v));
}

// Sum over aligned groups of WIDTH lanes (a power of two <= 64); every lane
// of a group gets the same value.  The whole wave must be active.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (WIDTH >= 2) v += dpp_f32<DPP_QXOR1>(v);
    if constexpr (WIDTH >= 4) v += dpp_f32<DPP_QXOR2>(v);
    if constexpr (WIDTH >= 8) v += dpp_f32<DPP_HALF_MIRROR>(v);
    if constexpr (WIDTH >= 16) v += dpp_f32<DPP_MIRROR>(v);
    if constexpr (WIDTH >= 32) v = swap16_sum(v);
    if constexpr (WIDTH >= 64) v = swap32_sum(v);
    return v;
}

// Sum of one float per thread over the workgroup (blockDim.x a multiple of
// 64, at most 2048), in a fixed order; every thread gets it.
__device__ __forceinline__ float pro_block_sum(float v) {
    __shared__ float red[32];
    v = group_sum<64>(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) s += red[i];
    return s;
}

// PRO_NORMD: this thread's sum of squares of its staged x, summed over the
// wave (fixed order), to red[wave]; every thread of the workgroup calls it
// before the staging barrier.  red: NW floats of the kernel's dynamic LDS
// that nothing else uses (a static __shared__ array beside a kernel's
// dynamic LDS has made kernels here several times slower).
__device__ __forceinline__ void pro_ss_put(float ss, float *red) {
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
}
// after the barrier: r = 1 / sqrt(sum / K + eps), the waves' sums added in
// wave order, so every thread of every workgroup gets the same value
template <int NW>
__device__ __forceinline__ float pro_ss_scale(const float *red, int K, float eps) {
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NW; i++) s += red[i];
    return 1.0f / sqrtf(s / (float)K + eps);
}

// An empty asm statement that takes v and gives it back and clobbers
// memory: code that uses v stays after it, loads issued before it stay
// before it.
__device__ __forceinline__ void pro_pin(float &v) { asm volatile("" : "+v"(v) : : "memory"); }
__device__ __forceinline__ void pro_pin(float4 &v) {
    pro_pin(v.x);
    pro_pin(v.y);
    pro_pin(v.z);
    pro_pin(v.w);
}

// silu(g) * u, as the unfused k_swiglu computes it.
__device__ __forceinline__ float pro_swiglu(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) {
    return *reinterpret_cast<const uint32_t *>(p);
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    return *reinterpret_cast<const uint16_t *>(p);
}
__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) {
    return *reinterpret_cast<const uint4 *>(p);
}

}  // namespace tbq
