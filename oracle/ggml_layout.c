/*
 * ggml_layout.c -- CPU restatement of ggml's own block decoders (the layouts
 * llama.cpp writes into GGUF files), for the TBQ_GGML qtype ids.
 * TEST INFRASTRUCTURE ONLY: the parity checker of libtbq's ggml-layout
 * kernels.  Nothing in the product library links or calls this code.
 *
 * Source of the algorithm: ggml (llama.cpp), ggml/src/ggml-quants.c,
 * dequantize_row_q4_0 / _q8_0 / _q2_K / _q3_K / _q4_K / _q5_K / _q6_K and
 * get_scale_min_k4, with the block structs of ggml/src/ggml-common.h.  ggml
 * is a dependency the reference names (layer4/tb_gguf.c:63-85 cites
 * ggml-common.h) but neither vendors nor matches; it is absent from this
 * image.  The K-quant block layouts have been stable since their
 * introduction (llama.cpp, June 2023; GGUF v2/v3 files).  The loops below
 * follow the published nested-loop structure: per 128-weight half for
 * Q2_K / Q3_K / Q6_K, per 64-weight chunk for Q4_K / Q5_K.
 *
 * Floating point: one IEEE rounding per source operation, no contraction
 * (built with -ffp-contract=off), in ggml's operation order:
 *   Q4_K, Q5_K, Q2_K   y = (d*sc) * q - (dmin*m)
 *   Q3_K               y = (d*(sc-32)) * q
 *   Q6_K               y = (d*sc) * q
 *   Q4_0, Q8_0         y = q * d
 * fp16 fields decode as IEEE 754 binary16 (GGML_FP16_TO_FP32), subnormals
 * included.
 *
 * Pinning (tests/test_ggml_layout.py): tbo_f16_ieee against numpy's
 * float16 on all 65536 inputs; every decoder against a block packer written
 * from the struct field descriptions (tests/ggml_pack.py) on random
 * integers, with the closed-form value of each weight; F32 / BF16 / Q8_K
 * against the reference layouts (identical formats).  ggml itself cannot be
 * run here, so these decoders are parity unpinned against ggml's own
 * output.
 */
#include "tbq_oracle.h"

#include <string.h>

static inline uint16_t g16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

float tbo_f16_ieee(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        /* subnormal or zero: m * 2^-24, exact in binary32 */
        const float v = (float)m * 0x1p-24f;
        return (h & 0x8000u) ? -v : v;
    }
    uint32_t bits = ((uint32_t)(h & 0x8000u) << 16) | (e == 31 ? 0x7F800000u : (e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* block_q4_0 { ggml_half d; uint8_t qs[16]; } */
static void g_q4_0(const uint8_t *b, float *y) {
    const float d = tbo_f16_ieee(g16(b));
    const uint8_t *qs = b + 2;
    for (int j = 0; j < 16; j++) {
        const int x0 = (qs[j] & 0x0F) - 8;
        const int x1 = (qs[j] >> 4) - 8;
        y[j] = (float)x0 * d;
        y[j + 16] = (float)x1 * d;
    }
}

/* block_q8_0 { ggml_half d; int8_t qs[32]; } */
static void g_q8_0(const uint8_t *b, float *y) {
    const float d = tbo_f16_ieee(g16(b));
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}

/* get_scale_min_k4: the 6-bit scale and min of sub-block j from the 12
 * packed bytes q. */
static void scale_min_k4(int j, const uint8_t *q, int *d, int *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* block_q4_K { ggml_half d, dmin; uint8_t scales[12]; uint8_t qs[128]; } */
static void g_q4_k(const uint8_t *b, float *y) {
    const float d = tbo_f16_ieee(g16(b)), min = tbo_f16_ieee(g16(b + 2));
    const uint8_t *scales = b + 4, *q = b + 16;
    int is = 0;
    for (int j = 0; j < 256; j += 64) {
        int sc, m;
        scale_min_k4(is + 0, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = min * (float)m;
        scale_min_k4(is + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; l++) {
            const float t = d1 * (float)(q[l] & 0xF);
            *y++ = t - m1;
        }
        for (int l = 0; l < 32; l++) {
            const float t = d2 * (float)(q[l] >> 4);
            *y++ = t - m2;
        }
        q += 32;
        is += 2;
    }
}

/* block_q5_K { ggml_half d, dmin; uint8_t scales[12]; uint8_t qh[32];
 * uint8_t qs[128]; } */
static void g_q5_k(const uint8_t *b, float *y) {
    const float d = tbo_f16_ieee(g16(b)), min = tbo_f16_ieee(g16(b + 2));
    const uint8_t *scales = b + 4, *qh = b + 16, *ql = b + 48;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < 256; j += 64) {
        int sc, m;
        scale_min_k4(is + 0, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = min * (float)m;
        scale_min_k4(is + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; l++) {
            const float t = d1 * (float)((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0));
            *y++ = t - m1;
        }
        for (int l = 0; l < 32; l++) {
            const float t = d2 * (float)((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0));
            *y++ = t - m2;
        }
        ql += 32;
        is += 2;
        u1 <<= 2;
        u2 <<= 2;
    }
}

/* block_q6_K { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16];
 * ggml_half d; } */
static void g_q6_k(const uint8_t *b, float *y) {
    const float d = tbo_f16_ieee(g16(b + 208));
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    for (int n = 0; n < 256; n += 128) {
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 0] = (d * (float)sc[is + 0]) * (float)q1;
            y[l + 32] = (d * (float)sc[is + 2]) * (float)q2;
            y[l + 64] = (d * (float)sc[is + 4]) * (float)q3;
            y[l + 96] = (d * (float)sc[is + 6]) * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

/* block_q3_K { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12];
 * ggml_half d; }.  The 16 6-bit scales: low nibbles of bytes 0..7 (then
 * their high nibbles) under 2-bit pairs of bytes 8..11. */
static void g_q3_k(const uint8_t *b, float *y) {
    const float d_all = tbo_f16_ieee(g16(b + 108));
    const uint8_t *hm = b, *q = b + 32, *s = b + 96;
    int8_t scales[16];
    for (int i = 0; i < 16; i++) {
        const int lo = (i < 8 ? s[i] : s[i - 8] >> 4) & 0xF;
        const int hi = (s[8 + (i % 4)] >> (2 * (i / 4))) & 3;
        scales[i] = (int8_t)(lo | (hi << 4));
    }
    int is = 0;
    uint8_t m = 1;
    for (int n = 0; n < 256; n += 128) {
        int shift = 0;
        for (int j = 0; j < 4; j++) {
            float dl = d_all * (float)(scales[is++] - 32);
            for (int l = 0; l < 16; l++)
                *y++ = dl * (float)((int)((q[l + 0] >> shift) & 3) - ((hm[l + 0] & m) ? 0 : 4));
            dl = d_all * (float)(scales[is++] - 32);
            for (int l = 0; l < 16; l++)
                *y++ = dl * (float)((int)((q[l + 16] >> shift) & 3) - ((hm[l + 16] & m) ? 0 : 4));
            shift += 2;
            m <<= 1;
        }
        q += 32;
    }
}

/* block_q2_K { uint8_t scales[16]; uint8_t qs[64]; ggml_half d, dmin; } */
static void g_q2_k(const uint8_t *b, float *y) {
    const float d = tbo_f16_ieee(g16(b + 80)), min = tbo_f16_ieee(g16(b + 82));
    const uint8_t *sc = b, *q = b + 16;
    int is = 0;
    for (int n = 0; n < 256; n += 128) {
        int shift = 0;
        for (int j = 0; j < 4; j++) {
            int s = sc[is++];
            float dl = d * (float)(s & 0xF), ml = min * (float)(s >> 4);
            for (int l = 0; l < 16; l++) {
                const float t = dl * (float)((q[l] >> shift) & 3);
                *y++ = t - ml;
            }
            s = sc[is++];
            dl = d * (float)(s & 0xF);
            ml = min * (float)(s >> 4);
            for (int l = 0; l < 16; l++) {
                const float t = dl * (float)((q[l + 16] >> shift) & 3);
                *y++ = t - ml;
            }
            shift += 2;
        }
        q += 32;
    }
}

int tbo_ggml_dequant_row(const void *data, int qtype, int n, float *out) {
    const uint8_t *p = (const uint8_t *)data;
    void (*blk)(const uint8_t *, float *) = 0;
    int bw = 0, bb = 0;
    switch (qtype & 0xFF) {
    case 1:
        for (int i = 0; i < n; i++) out[i] = tbo_f16_ieee(g16(p + 2 * i));
        return 1;
    case 0: case 30: case 15:   /* the same in both layouts */
        tbo_dequant_row(data, qtype & 0xFF, n, out);
        return 1;
    case 2: blk = g_q4_0; bw = 32; bb = 18; break;
    case 8: blk = g_q8_0; bw = 32; bb = 34; break;
    case 10: blk = g_q2_k; bw = 256; bb = 84; break;
    case 11: blk = g_q3_k; bw = 256; bb = 110; break;
    case 12: blk = g_q4_k; bw = 256; bb = 144; break;
    case 13: blk = g_q5_k; bw = 256; bb = 176; break;
    case 14: blk = g_q6_k; bw = 256; bb = 210; break;
    default:
        memset(out, 0, (size_t)n * 4);
        return 0;
    }
    for (int done = 0; done < n; done += bw, p += bb) blk(p, out + done);
    return 1;
}
