// tbq_kquant.hpp -- per-format block decoders for the reference's K-quant
// layouts (layer4/tb_gguf.c:110-288) and ggml's (QT_GGML ids, below), in two
// flavours:
//
//   decode8<QT>(blk, o, out)   eight consecutive weights o..o+7 of one block,
//                              rounded exactly as the reference rounds them
//                              (bit-exact dequant path);
//   chunk_dot<QT>(row, c, ..)  the dot product of one 32-weight chunk with x,
//                              with per-group scales factored out of the sum
//                              (matvec path; fp32 accumulate, fmaf).
//
// Block layouts (byte offsets within one block):
//   Q4_K 144: d f16@0, dmin f16@2, sc[12]@4, qs[128]@16
//   Q5_K 176: d@0, dmin@2, sc[12]@4, qh[32]@16, qs[128]@48
//   Q6_K 210: ql[128]@0, qh[64]@128, int8 sc[16]@192, d@208
//   Q3_K 110: hmask[32]@0, qs[64]@32, sc[12]@96, d@108
//   Q2_K  84: sc[16]@0 (lo nibble scale, hi nibble min), qs[64]@16, d@80, dmin@82
//   Q8_0  34: d@0, int8 qs[32]@2          Q4_0 18: d@0, qs[16]@2
//   Q8_K 292: f32 d@0, int8 qs[256]@4, bsums@260 (unused)
#pragma once

#include "tbq_device.hpp"

namespace tbq {

__device__ __forceinline__ uint32_t ldb(const uint8_t *p) { return *p; }
// Unaligned little-endian loads; gfx9 global memory accepts any alignment.
__device__ __forceinline__ uint32_t ldu16(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}
__device__ __forceinline__ uint32_t ldu32(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}

// ---- Q4_K / Q5_K 6-bit scale and min for sub-block j --------------------
// Q4_K (layer4/tb_gguf.c:163-168): j<4 scale sc[j], min sc[j+4]; j>=4 scale
// sc[j+4] and min sc[j+8] (bytes 12..15 of sc, i.e. qs[0..3]); low 6 bits.
__device__ __forceinline__ void q4k_scale_min(const uint8_t *b, int j, int &s, int &m) {
    if (j < 4) {
        s = ldb(b + 4 + j) & 63;
        m = ldb(b + 8 + j) & 63;
    } else {
        s = ldb(b + 8 + j) & 63;
        m = ldb(b + 12 + j) & 63;
    }
}
// Q5_K via q4_k_unpack_scales (layer4/tb_gguf.c:122-145): j>=4, k=j-4:
// scale (sc[k]>>6)|((sc[k+8]&15)<<2), min (sc[k+4]>>6)|((sc[k+12]&15)<<2).
__device__ __forceinline__ void q5k_scale_min(const uint8_t *b, int j, int &s, int &m) {
    const uint8_t *sc = b + 4;
    if (j < 4) {
        s = ldb(sc + j) & 63;
        m = ldb(sc + j + 4) & 63;
    } else {
        int k = j - 4;
        s = (ldb(sc + k) >> 6) | ((ldb(sc + k + 8) & 15) << 2);
        m = (ldb(sc + k + 4) >> 6) | ((ldb(sc + k + 12) & 15) << 2);
    }
}
// Q3_K scale slot j (layer4/tb_gguf.c:243-248): is = j mod 8.
__device__ __forceinline__ int q3k_scale(const uint8_t *b, int j) {
    const uint8_t *sc = b + 96;
    int is = j & 7;
    int lo4 = (ldb(sc + (is >> 1)) >> ((is & 1) * 4)) & 15;
    int hi2 = (ldb(sc + 8 + (is >> 2)) >> ((is & 3) * 2)) & 3;
    return (lo4 | (hi2 << 4)) - 32;
}

// ===========================================================================
// Bit-exact decode of weights o..o+7 of one block (o a multiple of 8).
// ===========================================================================
template <int QT>
__device__ __forceinline__ void decode8(const uint8_t *b, int o, float *w);

template <>
__device__ __forceinline__ void decode8<QT_Q4_K>(const uint8_t *b, int o, float *w) {
    float d = f16_ref(ldu16(b)), dmin = f16_ref(ldu16(b + 2));
    int j = o >> 5, si, mi;
    q4k_scale_min(b, j, si, mi);
    float S = d * (float)si, Mn = dmin * (float)mi;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t q = ldb(b + 16 + (o >> 1) + i);
        float t0 = S * (float)(q & 15), t1 = S * (float)(q >> 4);
        w[2 * i] = t0 - Mn;
        w[2 * i + 1] = t1 - Mn;
    }
}
template <>
__device__ __forceinline__ void decode8<QT_Q5_K>(const uint8_t *b, int o, float *w) {
    float d = f16_ref(ldu16(b)), dmin = f16_ref(ldu16(b + 2));
    int j = o >> 5, si, mi;
    q5k_scale_min(b, j, si, mi);
    float S = d * (float)si, Mn = dmin * (float)mi;
    uint32_t qh = ldb(b + 16 + (o >> 3));
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int e = o + i;
        int lo = (ldb(b + 48 + (e >> 1)) >> ((e & 1) * 4)) & 15;
        int q = lo | (((qh >> i) & 1) << 4);
        float t = S * (float)q;
        w[i] = t - Mn;
    }
}
template <>
__device__ __forceinline__ void decode8<QT_Q6_K>(const uint8_t *b, int o, float *w) {
    float d = f16_ref(ldu16(b + 208));
    float ds = d * (float)(int8_t)ldb(b + 192 + (o >> 4));
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int e = o + i;
        int lo = (ldb(b + (e >> 1)) >> ((e & 1) * 4)) & 15;
        int hi = (ldb(b + 128 + (e >> 2)) >> ((e & 3) * 2)) & 3;
        w[i] = ds * (float)((lo | (hi << 4)) - 32);
    }
}
template <>
__device__ __forceinline__ void decode8<QT_Q3_K>(const uint8_t *b, int o, float *w) {
    float d = f16_ref(ldu16(b + 108));
    float S = d * (float)q3k_scale(b, o >> 4);
    uint32_t hm = ldb(b + (o >> 3));
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int e = o + i;
        int lo2 = (ldb(b + 32 + (e >> 2)) >> ((e & 3) * 2)) & 3;
        int q3 = lo2 | (((hm >> i) & 1) << 2);
        w[i] = S * (float)(q3 - 4);
    }
}
template <>
__device__ __forceinline__ void decode8<QT_Q2_K>(const uint8_t *b, int o, float *w) {
    float d = f16_ref(ldu16(b + 80)), dmin = f16_ref(ldu16(b + 82));
    uint32_t sm = ldb(b + (o >> 4));
    float S = d * (float)(sm & 15), Mn = dmin * (float)(sm >> 4);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int e = o + i;
        int q = (ldb(b + 16 + (e >> 2)) >> ((e & 3) * 2)) & 3;
        float t = S * (float)q;
        w[i] = t - Mn;
    }
}
template <>
__device__ __forceinline__ void decode8<QT_Q8_0>(const uint8_t *b, int o, float *w) {
    float d = f16_ref(ldu16(b));
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = d * (float)(int8_t)ldb(b + 2 + o + i);
}
template <>
__device__ __forceinline__ void decode8<QT_Q4_0>(const uint8_t *b, int o, float *w) {
    float d = f16_ref(ldu16(b));
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t q = ldb(b + 2 + (o >> 1) + i);
        w[2 * i] = d * (float)((int)(q & 15) - 8);
        w[2 * i + 1] = d * (float)((int)(q >> 4) - 8);
    }
}
template <>
__device__ __forceinline__ void decode8<QT_Q8_K>(const uint8_t *b, int o, float *w) {
    float d = __builtin_bit_cast(float, ldu32(b));
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = d * (float)(int8_t)ldb(b + 4 + o + i);
}

// ===========================================================================
// ggml's on-disk layouts (QT_GGML | id; ggml-quants.c, dequantize_row_*).
// The fields sit at the reference's byte offsets; what differs is which
// quant bits, scale and fp16 decoding belong to weight e of a block:
//   Q4_K/Q5_K  chunk c = e/64, l = e%32: nibble (e/32)&1 of qs[32c+l]; Q5_K
//              adds bit e/32 of qh[l] as 16.  Sub-block e/32 takes its
//              6-bit scale and min from get_scale_min_k4 (gq4k_scale_min).
//   Q6_K       half n = e/128, r = e%128, k = r/32, l = r%32: nibble k>>1 of
//              ql[64n + 32(k&1) + l], bits 2k of qh[32n + l]; int8 sc[e/16];
//              q - 32.
//   Q3_K       n, k, l as Q6_K: bits 2k of qs[32n+l]; bit 4n+k of hmask[l]
//              (clear: q - 4); scale e/16 of the ggml 6-bit unpack, - 32.
//   Q2_K       quants as Q3_K's 2-bit part; scale/min byte sc[e/16].
//   Q4_0       weight l < 16: low nibble of qs[l]; 16 + l: high nibble.
// fp16 fields decode as IEEE (f16_ieee).  Roundings: w = fl(fl(d*s)*q) -
// fl(dmin*m) (K formats with mins), fl(fl(d*s)*q) otherwise, fl(q*d) for
// Q4_0/Q8_0, one rounding per operation.
// ===========================================================================
__device__ __forceinline__ void gq4k_scale_min(const uint8_t *b, int j, int &s, int &m) {
    const uint8_t *q = b + 4;
    if (j < 4) {
        s = ldb(q + j) & 63;
        m = ldb(q + j + 4) & 63;
    } else {
        s = (ldb(q + j + 4) & 15) | ((ldb(q + j - 4) >> 6) << 4);
        m = (ldb(q + j + 4) >> 4) | ((ldb(q + j) >> 6) << 4);
    }
}
// The same for unit p's sub-block 2p + j (j = 0, 1) of a super-block whose
// first 16 bytes are hdr (hdr.y, .z, .w = scale bytes 0-3, 4-7, 8-11):
// j' < 4: sc[j'] & 63, sc[j'+4] & 63; else (sc[j'+4] & 15) | (sc[j'-4] >> 6) << 4,
// (sc[j'+4] >> 4) | (sc[j'] >> 6) << 4.  Selects, no branch on p.
__device__ __forceinline__ void gq4k_sm(const uint4 &hdr, int p, int j, int &s, int &m) {
    const int k = (2 * p + j) & 3;
    const bool hi = p >= 2;
    const uint32_t y = hdr.y >> (8 * k), z = hdr.z >> (8 * k), w = hdr.w >> (8 * k);
    s = hi ? (int)((w & 15) | (((y >> 6) & 3) << 4)) : (int)(y & 63);
    m = hi ? (int)(((w >> 4) & 15) | (((z >> 6) & 3) << 4)) : (int)(z & 63);
}
__device__ __forceinline__ int gq3k_scale(const uint8_t *b, int i) {
    const uint8_t *sc = b + 96;
    const int lo4 = (ldb(sc + (i & 7)) >> (4 * (i >> 3))) & 15;
    const int hi2 = (ldb(sc + 8 + (i & 3)) >> (2 * (i >> 2))) & 3;
    return (lo4 | (hi2 << 4)) - 32;
}

template <>
__device__ __forceinline__ void decode8<QT_GQ4_K>(const uint8_t *b, int o, float *w) {
    const float d = f16_ieee(ldu16(b)), dmin = f16_ieee(ldu16(b + 2));
    int si, mi;
    gq4k_scale_min(b, o >> 5, si, mi);
    const float S = d * (float)si, Mn = dmin * (float)mi;
    const uint8_t *q = b + 16 + 32 * (o >> 6) + (o & 31);
    const int sh = 4 * ((o >> 5) & 1);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float t = S * (float)((ldb(q + i) >> sh) & 15);
        w[i] = t - Mn;
    }
}
template <>
__device__ __forceinline__ void decode8<QT_GQ5_K>(const uint8_t *b, int o, float *w) {
    const float d = f16_ieee(ldu16(b)), dmin = f16_ieee(ldu16(b + 2));
    const int j = o >> 5;
    int si, mi;
    gq4k_scale_min(b, j, si, mi);
    const float S = d * (float)si, Mn = dmin * (float)mi;
    const uint8_t *q = b + 48 + 32 * (o >> 6) + (o & 31);
    const uint8_t *h = b + 16 + (o & 31);
    const int sh = 4 * (j & 1);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int v = ((ldb(q + i) >> sh) & 15) | (((ldb(h + i) >> j) & 1) << 4);
        const float t = S * (float)v;
        w[i] = t - Mn;
    }
}
template <>
__device__ __forceinline__ void decode8<QT_GQ6_K>(const uint8_t *b, int o, float *w) {
    const float d = f16_ieee(ldu16(b + 208));
    const float ds = d * (float)(int8_t)ldb(b + 192 + (o >> 4));
    const int n = o >> 7, k = (o >> 5) & 3, l0 = o & 31;
    const uint8_t *ql = b + 64 * n + 32 * (k & 1) + l0;
    const uint8_t *qh = b + 128 + 32 * n + l0;
    const int shl = 4 * (k >> 1), shh = 2 * k;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int v = ((ldb(ql + i) >> shl) & 15) | (((ldb(qh + i) >> shh) & 3) << 4);
        w[i] = ds * (float)(v - 32);
    }
}
template <>
__device__ __forceinline__ void decode8<QT_GQ3_K>(const uint8_t *b, int o, float *w) {
    const float d = f16_ieee(ldu16(b + 108));
    const float S = d * (float)gq3k_scale(b, o >> 4);
    const int n = o >> 7, k = (o >> 5) & 3, l0 = o & 31;
    const uint8_t *q = b + 32 + 32 * n + l0;
    const uint8_t *hm = b + l0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int v = (int)((ldb(q + i) >> (2 * k)) & 3) - (((ldb(hm + i) >> (4 * n + k)) & 1) ? 0 : 4);
        w[i] = S * (float)v;
    }
}
template <>
__device__ __forceinline__ void decode8<QT_GQ2_K>(const uint8_t *b, int o, float *w) {
    const float d = f16_ieee(ldu16(b + 80)), dmin = f16_ieee(ldu16(b + 82));
    const uint32_t sm = ldb(b + (o >> 4));
    const float S = d * (float)(sm & 15), Mn = dmin * (float)(sm >> 4);
    const int n = o >> 7, k = (o >> 5) & 3, l0 = o & 31;
    const uint8_t *q = b + 16 + 32 * n + l0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float t = S * (float)((ldb(q + i) >> (2 * k)) & 3);
        w[i] = t - Mn;
    }
}
template <>
__device__ __forceinline__ void decode8<QT_GQ8_0>(const uint8_t *b, int o, float *w) {
    const float d = f16_ieee(ldu16(b));
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = d * (float)(int8_t)ldb(b + 2 + o + i);
}
template <>
__device__ __forceinline__ void decode8<QT_GQ4_0>(const uint8_t *b, int o, float *w) {
    const float d = f16_ieee(ldu16(b));
    const uint8_t *q = b + 2 + (o & 15);
    const int sh = 4 * (o >> 4);
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = (float)((int)((ldb(q + i) >> sh) & 15) - 8) * d;
}

// ===========================================================================
// Matvec chunk dots.  A chunk is 32 consecutive weights of one row: one
// 32-weight block for Q8_0/Q4_0, sub-block c%8 of super-block c/8 otherwise.
// xl points at x[32c] in LDS; xs16 at the sums of x over the chunk's two
// 16-element groups (xs16[0], xs16[1]).
// Per group g the exact value is sum_i (S_g q_i - M_g) x_i; it is evaluated
// as S_g*sum(q_i x_i) - M_g*sum(x_i), accumulating in fp32 with fmaf.
// ===========================================================================
template <int QT>
__device__ __forceinline__ float chunk_dot(const uint8_t *row, int c, const float *xl, const float *xs16);

// Sum over 16 bytes of nibble pairs: byte i holds weights 2i (low) and 2i+1
// (high).  Returns sum q*x.
__device__ __forceinline__ float nib_pairs_dot16(uint4 q, const float *xl) {
    float a0 = 0.f, a1 = 0.f;
    const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t v = wv[k];
        float4 xa = *reinterpret_cast<const float4 *>(xl + 8 * k);
        float4 xb = *reinterpret_cast<const float4 *>(xl + 8 * k + 4);
        a0 = fmaf((float)(v & 15), xa.x, a0);
        a1 = fmaf((float)((v >> 4) & 15), xa.y, a1);
        a0 = fmaf((float)((v >> 8) & 15), xa.z, a0);
        a1 = fmaf((float)((v >> 12) & 15), xa.w, a1);
        a0 = fmaf((float)((v >> 16) & 15), xb.x, a0);
        a1 = fmaf((float)((v >> 20) & 15), xb.y, a1);
        a0 = fmaf((float)((v >> 24) & 15), xb.z, a0);
        a1 = fmaf((float)(v >> 28), xb.w, a1);
    }
    return a0 + a1;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q4_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 144;
    int j = c & 7, si, mi;
    float d = f16_ref(ldu16(b)), dmin = f16_ref(ldu16(b + 2));
    q4k_scale_min(b, j, si, mi);
    uint4 q = *reinterpret_cast<const uint4 *>(b + 16 + 16 * j);
    float sq = nib_pairs_dot16(q, xl);
    return fmaf(d * (float)si, sq, -(dmin * (float)mi) * (xs16[0] + xs16[1]));
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q5_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 176;
    int j = c & 7, si, mi;
    float d = f16_ref(ldu16(b)), dmin = f16_ref(ldu16(b + 2));
    q5k_scale_min(b, j, si, mi);
    uint4 q = *reinterpret_cast<const uint4 *>(b + 48 + 16 * j);
    uint32_t h = ldu32(b + 16 + 4 * j);  // bit i -> weight 32j+i
    float sq = nib_pairs_dot16(q, xl);
    float sh = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) sh = fmaf((float)((h >> i) & 1), xl[i], sh);
    sq = fmaf(16.f, sh, sq);
    return fmaf(d * (float)si, sq, -(dmin * (float)mi) * (xs16[0] + xs16[1]));
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q6_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 210;
    int j = c & 7;
    float d = f16_ref(ldu16(b + 208));
    uint32_t sc2 = ldu16(b + 192 + 2 * j);
    float s0 = d * (float)(int8_t)(sc2 & 0xFF), s1 = d * (float)(int8_t)(sc2 >> 8);
    uint32_t ql[4], qh[2];
#pragma unroll
    for (int k = 0; k < 4; k++) ql[k] = ldu32(b + 16 * j + 4 * k);
    qh[0] = ldu32(b + 128 + 8 * j);
    qh[1] = ldu32(b + 128 + 8 * j + 4);
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        int lo = (ql[i >> 3] >> ((i & 7) * 4)) & 15;
        int hi = (qh[i >> 4] >> ((i & 15) * 2)) & 3;
        acc[i >> 4] = fmaf((float)(lo | (hi << 4)), xl[i], acc[i >> 4]);
    }
    // q = u - 32
    float g0 = fmaf(-32.f, xs16[0], acc[0]);
    float g1 = fmaf(-32.f, xs16[1], acc[1]);
    return fmaf(s0, g0, s1 * g1);
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q3_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 110;
    int j = c & 7;
    float d = f16_ref(ldu16(b + 108));
    float s0 = d * (float)q3k_scale(b, 2 * j), s1 = d * (float)q3k_scale(b, 2 * j + 1);
    uint32_t qs0 = ldu32(b + 32 + 8 * j), qs1 = ldu32(b + 32 + 8 * j + 4);
    uint32_t hm = ldu32(b + 4 * j);
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        uint32_t qs = i < 16 ? qs0 : qs1;
        int lo2 = (qs >> ((i & 15) * 2)) & 3;
        int q3 = lo2 | (((hm >> i) & 1) << 2);
        acc[i >> 4] = fmaf((float)q3, xl[i], acc[i >> 4]);
    }
    float g0 = fmaf(-4.f, xs16[0], acc[0]);
    float g1 = fmaf(-4.f, xs16[1], acc[1]);
    return fmaf(s0, g0, s1 * g1);
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q2_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 84;
    int j = c & 7;
    float d = f16_ref(ldu16(b + 80)), dmin = f16_ref(ldu16(b + 82));
    uint32_t sm = ldu16(b + 2 * j);
    uint32_t qs0 = ldu32(b + 16 + 8 * j), qs1 = ldu32(b + 16 + 8 * j + 4);
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        uint32_t qs = i < 16 ? qs0 : qs1;
        acc[i >> 4] = fmaf((float)((qs >> ((i & 15) * 2)) & 3), xl[i], acc[i >> 4]);
    }
    float r = 0.f;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        uint32_t v = (sm >> (8 * g)) & 0xFF;
        float S = d * (float)(v & 15), Mn = dmin * (float)(v >> 4);
        r = fmaf(S, acc[g], r);
        r = fmaf(-Mn, xs16[g], r);
    }
    return r;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q8_0>(const uint8_t *row, int c, const float *xl, const float *) {
    const uint8_t *b = row + (size_t)c * 34;
    float d = f16_ref(ldu16(b));
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t v = ldu32(b + 2 + 4 * k);
#pragma unroll
        for (int t = 0; t < 4; t++) a = fmaf((float)(int8_t)(v >> (8 * t)), xl[4 * k + t], a);
    }
    return d * a;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q4_0>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)c * 18;
    float d = f16_ref(ldu16(b));
    uint4 q;
    q.x = ldu32(b + 2); q.y = ldu32(b + 6); q.z = ldu32(b + 10); q.w = ldu32(b + 14);
    float sq = nib_pairs_dot16(q, xl);
    return d * fmaf(-8.f, xs16[0] + xs16[1], sq);
}

template <>
__device__ __forceinline__ float chunk_dot<QT_Q8_K>(const uint8_t *row, int c, const float *xl, const float *) {
    const uint8_t *b = row + (size_t)(c >> 3) * 292;
    int j = c & 7;
    float d = __builtin_bit_cast(float, ldu32(b));
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t v = ldu32(b + 4 + 32 * j + 4 * k);
#pragma unroll
        for (int t = 0; t < 4; t++) a = fmaf((float)(int8_t)(v >> (8 * t)), xl[4 * k + t], a);
    }
    return d * a;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_F32>(const uint8_t *row, int c, const float *xl, const float *) {
    const float *w = reinterpret_cast<const float *>(row) + 32 * c;
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        float4 v = *reinterpret_cast<const float4 *>(w + i);
        a = fmaf(v.x, xl[i], a); a = fmaf(v.y, xl[i + 1], a);
        a = fmaf(v.z, xl[i + 2], a); a = fmaf(v.w, xl[i + 3], a);
    }
    return a;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_F16>(const uint8_t *row, int c, const float *xl, const float *) {
    const uint8_t *w = row + 64 * c;
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        uint32_t v = ldu32(w + 2 * i);
        a = fmaf(f16_ref(v & 0xFFFF), xl[i], a);
        a = fmaf(f16_ref(v >> 16), xl[i + 1], a);
    }
    return a;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_BF16>(const uint8_t *row, int c, const float *xl, const float *) {
    const uint8_t *w = row + 64 * c;
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        uint32_t v = ldu32(w + 2 * i);
        a = fmaf(bf16_ref(v & 0xFFFF), xl[i], a);
        a = fmaf(bf16_ref(v >> 16), xl[i + 1], a);
    }
    return a;
}

// ---- ggml layouts (the chunk is sub-block c%8 / block c, weights in order).
// Sum over 32 consecutive bytes q[0..31] of ((q[i] >> sh) & mask) * x[i].
__device__ __forceinline__ float bits_run_dot32(const uint8_t *q, int sh, uint32_t mask, const float *xl) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t v = ldu32(q + 4 * k) >> sh;
        a0 = fmaf((float)(v & mask), xl[4 * k], a0);
        a1 = fmaf((float)((v >> 8) & mask), xl[4 * k + 1], a1);
        a0 = fmaf((float)((v >> 16) & mask), xl[4 * k + 2], a0);
        a1 = fmaf((float)((v >> 24) & mask), xl[4 * k + 3], a1);
    }
    return a0 + a1;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GQ4_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 144;
    const int j = c & 7;
    int si, mi;
    gq4k_scale_min(b, j, si, mi);
    const float d = f16_ieee(ldu16(b)), dmin = f16_ieee(ldu16(b + 2));
    const float sq = bits_run_dot32(b + 16 + 32 * (j >> 1), 4 * (j & 1), 15u, xl);
    return fmaf(d * (float)si, sq, -(dmin * (float)mi) * (xs16[0] + xs16[1]));
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GQ5_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 176;
    const int j = c & 7;
    int si, mi;
    gq4k_scale_min(b, j, si, mi);
    const float d = f16_ieee(ldu16(b)), dmin = f16_ieee(ldu16(b + 2));
    float sq = bits_run_dot32(b + 48 + 32 * (j >> 1), 4 * (j & 1), 15u, xl);
    sq = fmaf(16.f, bits_run_dot32(b + 16, j, 1u, xl), sq);
    return fmaf(d * (float)si, sq, -(dmin * (float)mi) * (xs16[0] + xs16[1]));
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GQ6_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 210;
    const int j = c & 7, n = j >> 2, k = j & 3;
    const float d = f16_ieee(ldu16(b + 208));
    const float s0 = d * (float)(int8_t)ldb(b + 192 + 2 * j), s1 = d * (float)(int8_t)ldb(b + 193 + 2 * j);
    const uint8_t *ql = b + 64 * n + 32 * (k & 1), *qh = b + 128 + 32 * n;
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int v = ((ldb(ql + i) >> (4 * (k >> 1))) & 15) | (((ldb(qh + i) >> (2 * k)) & 3) << 4);
        acc[i >> 4] = fmaf((float)v, xl[i], acc[i >> 4]);
    }
    const float g0 = fmaf(-32.f, xs16[0], acc[0]);
    const float g1 = fmaf(-32.f, xs16[1], acc[1]);
    return fmaf(s0, g0, s1 * g1);
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GQ3_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 110;
    const int j = c & 7, n = j >> 2, k = j & 3;
    const float d = f16_ieee(ldu16(b + 108));
    const float s0 = d * (float)gq3k_scale(b, 2 * j), s1 = d * (float)gq3k_scale(b, 2 * j + 1);
    const uint8_t *q = b + 32 + 32 * n;
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int v = ((ldb(q + i) >> (2 * k)) & 3) | (((ldb(b + i) >> (4 * n + k)) & 1) << 2);
        acc[i >> 4] = fmaf((float)v, xl[i], acc[i >> 4]);
    }
    const float g0 = fmaf(-4.f, xs16[0], acc[0]);
    const float g1 = fmaf(-4.f, xs16[1], acc[1]);
    return fmaf(s0, g0, s1 * g1);
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GQ2_K>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)(c >> 3) * 84;
    const int j = c & 7, n = j >> 2, k = j & 3;
    const float d = f16_ieee(ldu16(b + 80)), dmin = f16_ieee(ldu16(b + 82));
    const uint32_t sm = ldu16(b + 2 * j);
    const uint8_t *q = b + 16 + 32 * n;
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 32; i++) acc[i >> 4] = fmaf((float)((ldb(q + i) >> (2 * k)) & 3), xl[i], acc[i >> 4]);
    float r = 0.f;
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const uint32_t v = (sm >> (8 * g)) & 0xFF;
        const float S = d * (float)(v & 15), Mn = dmin * (float)(v >> 4);
        r = fmaf(S, acc[g], r);
        r = fmaf(-Mn, xs16[g], r);
    }
    return r;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GQ8_0>(const uint8_t *row, int c, const float *xl, const float *) {
    const uint8_t *b = row + (size_t)c * 34;
    const float d = f16_ieee(ldu16(b));
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t v = ldu32(b + 2 + 4 * k);
#pragma unroll
        for (int t = 0; t < 4; t++) a = fmaf((float)(int8_t)(v >> (8 * t)), xl[4 * k + t], a);
    }
    return d * a;
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GQ4_0>(const uint8_t *row, int c, const float *xl, const float *xs16) {
    const uint8_t *b = row + (size_t)c * 18;
    const float d = f16_ieee(ldu16(b));
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t v = ldu32(b + 2 + 4 * k);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            a0 = fmaf((float)((v >> (8 * t)) & 15), xl[4 * k + t], a0);
            a1 = fmaf((float)((v >> (8 * t + 4)) & 15), xl[16 + 4 * k + t], a1);
        }
    }
    return d * fmaf(-8.f, xs16[0] + xs16[1], a0 + a1);
}

template <>
__device__ __forceinline__ float chunk_dot<QT_GF16>(const uint8_t *row, int c, const float *xl, const float *) {
    const uint8_t *w = row + 64 * c;
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        const uint32_t v = ldu32(w + 2 * i);
        a = fmaf(f16_ieee(v & 0xFFFF), xl[i], a);
        a = fmaf(f16_ieee(v >> 16), xl[i + 1], a);
    }
    return a;
}

// ---------------------------------------------------------------------------
// x staging for the fp32 chunk kernels.  x lives in LDS with float4 t of
// chunk c (32 floats) at slot 8c + (t ^ (c & 7)): lanes that own
// consecutive chunks then read distinct banks.  xs holds the fp32 sums of
// x over 16-element groups.  NT = threads of the workgroup.
// ---------------------------------------------------------------------------
template <int NT>
__device__ __forceinline__ void stage_x_swizzled(const float *__restrict__ x, int K, float *xl, float *xs) {
    for (int i = threadIdx.x; i < K / 4; i += NT) {
        const int c = i >> 3, t = i & 7;
        *reinterpret_cast<float4 *>(xl + 4 * (8 * c + (t ^ (c & 7)))) = *reinterpret_cast<const float4 *>(x + 4 * i);
    }
    for (int g = threadIdx.x; g < K / 16; g += NT) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) a += x[16 * g + i];
        xs[g] = a;
    }
}

__device__ __forceinline__ void load_chunk_x(const float *xl, int c, float *xv) {
#pragma unroll
    for (int t = 0; t < 8; t++)
        *reinterpret_cast<float4 *>(xv + 4 * t) = *reinterpret_cast<const float4 *>(xl + 4 * (8 * c + (t ^ (c & 7))));
}

}  // namespace tbq
