/*
 * tbq_oracle.c -- CPU restatement of the reference's K-quant decoders,
 * sequential dequant-matvec, softmax top-k router, SwiGLU and MoE assembly.
 * TEST INFRASTRUCTURE ONLY: parity checker and timed CPU baseline.
 *
 * Reference files restated (Trailblaze v0.7):
 *   layer4/tb_gguf.c:92-419     decoders, tb_gguf_dequant_row, _matvec
 *   layer4/tb_infer.c:130-135   tb_swiglu
 *   layer4/tb_infer.c:351-374   softmax / top-k / renormalise (use_hdgl=0)
 *   layer4/tb_infer.c:753-833   MoE expert loop and weighted accumulate
 *   layer4/tb_infer.c:876       residual add
 *   src/tb_analog_dispatch.c:486-524  structure of tb_dot_q4k_avx512 (timing)
 *
 * Build: -std=c11 -ffp-contract=off (no FMA contraction, as the reference's
 * -std=c11 build).  Each statement below keeps one IEEE rounding per source
 * operation in the same order as the reference.
 */
#define _POSIX_C_SOURCE 200809L
#include "tbq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__AVX512F__)
#include <immintrin.h>
#endif

static inline uint16_t rd16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* layer4/tb_gguf.c:92-101.  Exponent 0 keeps the mantissa bits in place with
 * a zero biased exponent (so subnormal halves decode to m*2^-136, not
 * m*2^-24); exponent 31 maps to the f32 inf/nan exponent; otherwise rebias
 * by 112. */
float tbo_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (e == 0)
        bits = s | (m << 13);
    else if (e == 31)
        bits = s | 0x7F800000u | (m << 13);
    else
        bits = s | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* layer4/tb_gguf.c:104-107 */
float tbo_bf16_to_f32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Block geometry as tabulated in layer4/tb_gguf.c:380-394. */
int tbo_block_geometry(int qtype, int *bw, int *bb) {
    int w, b;
    if (qtype & 0x100) {   /* ggml's layout of a format: the same geometry */
        if (qtype == (0x100 | 21)) return 0;
        qtype &= 0xFF;
    }
    switch (qtype) {
    case 0: w = 1; b = 4; break;
    case 1: w = 1; b = 2; break;
    case 30: w = 1; b = 2; break;
    case 8: w = 32; b = 34; break;
    case 2: w = 32; b = 18; break;
    case 12: w = 256; b = 144; break;
    case 10: w = 256; b = 84; break;
    case 11: w = 256; b = 110; break;
    case 21: w = 256; b = 110; break;
    case 13: w = 256; b = 176; break;
    case 15: w = 256; b = 292; break;
    case 14: w = 256; b = 210; break;
    default: return 0;
    }
    if (bw) *bw = w;
    if (bb) *bb = b;
    return 1;
}

/* layer4/tb_gguf.c:397-398 */
size_t tbo_row_bytes(int qtype, int K) {
    int bw, bb;
    if (!tbo_block_geometry(qtype, &bw, &bb)) return 0;
    return (size_t)((K + bw - 1) / bw) * (size_t)bb;
}

/* Q4_0, layer4/tb_gguf.c:110-118: w[2i]=d*(lo-8), w[2i+1]=d*(hi-8). */
static void blk_q4_0(const uint8_t *b, float *out) {
    float d = tbo_f16_to_f32(rd16(b));
    for (int i = 0; i < 16; i++) {
        int v = b[2 + i];
        out[2 * i] = d * (float)((v & 15) - 8);
        out[2 * i + 1] = d * (float)((v >> 4) - 8);
    }
}

/* Q4_K, layer4/tb_gguf.c:148-180.  Sub-block j<4 takes its 6-bit scale from
 * byte 4+j and its min from byte 8+j of the super-block; j>=4 takes the scale
 * from byte 8+j (scale array bytes 8..11) and the min from byte 12+j, which
 * is past the 12-byte scale array: the first four quant bytes. */
static void blk_q4_k(const uint8_t *b, float *out) {
    float d = tbo_f16_to_f32(rd16(b));
    float dmin = tbo_f16_to_f32(rd16(b + 2));
    float S[8], Mn[8];
    for (int j = 0; j < 8; j++) {
        int sbyte = j < 4 ? b[4 + j] : b[4 + j + 4];
        int mbyte = j < 4 ? b[4 + j + 4] : b[4 + j + 8];
        S[j] = d * (float)(sbyte & 63);
        Mn[j] = dmin * (float)(mbyte & 63);
    }
    const uint8_t *qs = b + 16;
    for (int i = 0; i < 128; i++) {
        int g = i >> 4; /* (2i)/32 == (2i+1)/32 */
        float lo = (float)(qs[i] & 15);
        float hi = (float)(qs[i] >> 4);
        float t0 = S[g] * lo;
        float t1 = S[g] * hi;
        out[2 * i] = t0 - Mn[g];
        out[2 * i + 1] = t1 - Mn[g];
    }
}

/* Q8_0, layer4/tb_gguf.c:183-187 */
static void blk_q8_0(const uint8_t *b, float *out) {
    float d = tbo_f16_to_f32(rd16(b));
    const int8_t *q = (const int8_t *)(b + 2);
    for (int i = 0; i < 32; i++) out[i] = d * (float)q[i];
}

/* Q6_K, layer4/tb_gguf.c:190-204: ql[128]@0, qh[64]@128, int8 sc[16]@192,
 * d@208.  w = (d*sc[i/16]) * q, q in [-32,31]. */
static void blk_q6_k(const uint8_t *b, float *out) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = tbo_f16_to_f32(rd16(b + 208));
    for (int i = 0; i < 256; i++) {
        int lo = (ql[i >> 1] >> ((i & 1) * 4)) & 15;
        int hi = (qh[i >> 2] >> ((i & 3) * 2)) & 3;
        int q = (lo | (hi << 4)) - 32;
        float ds = d * (float)sc[i >> 4];
        out[i] = ds * (float)q;
    }
}

/* Q2_K, layer4/tb_gguf.c:210-225: scales[16]@0 (lo nibble scale, hi nibble
 * min), qs[64]@16, d@80, dmin@82. */
static void blk_q2_k(const uint8_t *b, float *out) {
    const uint8_t *qs = b + 16;
    float d = tbo_f16_to_f32(rd16(b + 80));
    float dmin = tbo_f16_to_f32(rd16(b + 82));
    for (int g = 0; g < 16; g++) {
        float S = d * (float)(b[g] & 15);
        float Mn = dmin * (float)(b[g] >> 4);
        for (int t = 0; t < 16; t++) {
            int i = g * 16 + t;
            int q = (qs[i >> 2] >> ((i & 3) * 2)) & 3;
            float p = S * (float)q;
            out[i] = p - Mn;
        }
    }
}

/* Q3_K, layer4/tb_gguf.c:230-257: hmask[32]@0, qs[64]@32, sc[12]@96, d@108.
 * Scale slot j uses packed index is=j mod 8 (slots 8..15 repeat 0..7). */
static void blk_q3_k(const uint8_t *b, float *out) {
    const uint8_t *hm = b, *qs = b + 32, *sc = b + 96;
    float d = tbo_f16_to_f32(rd16(b + 108));
    float S[16];
    for (int j = 0; j < 16; j++) {
        int is = j & 7;
        int lo4 = (sc[is >> 1] >> ((is & 1) * 4)) & 15;
        int hi2 = (sc[8 + (is >> 2)] >> ((is & 3) * 2)) & 3;
        S[j] = d * (float)((lo4 | (hi2 << 4)) - 32);
    }
    for (int i = 0; i < 256; i++) {
        int lo2 = (qs[i >> 2] >> ((i & 3) * 2)) & 3;
        int h = (hm[i >> 3] >> (i & 7)) & 1;
        out[i] = S[i >> 4] * (float)((lo2 | (h << 2)) - 4);
    }
}

/* Q5_K, layer4/tb_gguf.c:262-279 with q4_k_unpack_scales :122-145:
 * d@0, dmin@2, sc[12]@4, qh[32]@16, qs[128]@48.  For j>=4 (k=j-4) the scale is
 * (sc[k]>>6)|((sc[k+8]&15)<<2) and the min (sc[k+4]>>6)|((sc[k+12]&15)<<2),
 * where sc[12..15] are qh[0..3]. */
static void blk_q5_k(const uint8_t *b, float *out) {
    float d = tbo_f16_to_f32(rd16(b));
    float dmin = tbo_f16_to_f32(rd16(b + 2));
    const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
    float S[8], Mn[8];
    for (int j = 0; j < 8; j++) {
        int sr, mr;
        if (j < 4) {
            sr = sc[j] & 63;
            mr = sc[j + 4] & 63;
        } else {
            int k = j - 4;
            sr = (sc[k] >> 6) | ((sc[k + 8] & 15) << 2);
            mr = (sc[k + 4] >> 6) | ((sc[k + 12] & 15) << 2);
        }
        S[j] = d * (float)sr;
        Mn[j] = dmin * (float)mr;
    }
    for (int i = 0; i < 256; i++) {
        int g = i >> 5;
        int hb = (qh[i >> 3] >> (i & 7)) & 1;
        int lo = (qs[i >> 1] >> ((i & 1) * 4)) & 15;
        float p = S[g] * (float)(lo | (hb << 4));
        out[i] = p - Mn[g];
    }
}

/* Q8_K, layer4/tb_gguf.c:283-288: f32 d@0, int8 qs[256]@4 (bsums unused). */
static void blk_q8_k(const uint8_t *b, float *out) {
    float d;
    memcpy(&d, b, 4);
    const int8_t *q = (const int8_t *)(b + 4);
    for (int i = 0; i < 256; i++) out[i] = d * (float)q[i];
}

/* layer4/tb_gguf.c:293-371.  Whole blocks are decoded while fewer than
 * n_weights outputs exist; callers pass multiples of the block size.
 * Unknown qtype (including 21, which only the matvec table knows) zeroes. */
void tbo_dequant_row(const void *data, int qtype, int n, float *out) {
    if (qtype & 0x100) {   /* ggml's layouts: ggml_layout.c */
        tbo_ggml_dequant_row(data, qtype, n, out);
        return;
    }
    const uint8_t *p = (const uint8_t *)data;
    int done = 0;
    void (*blk)(const uint8_t *, float *) = 0;
    int bw = 0, bb = 0;
    switch (qtype) {
    case 0:
        memcpy(out, data, (size_t)n * 4);
        return;
    case 1:
        for (int i = 0; i < n; i++) out[i] = tbo_f16_to_f32(rd16(p + 2 * i));
        return;
    case 30:
        for (int i = 0; i < n; i++) out[i] = tbo_bf16_to_f32(rd16(p + 2 * i));
        return;
    case 8: blk = blk_q8_0; bw = 32; bb = 34; break;
    case 2: blk = blk_q4_0; bw = 32; bb = 18; break;
    case 12: blk = blk_q4_k; bw = 256; bb = 144; break;
    case 10: blk = blk_q2_k; bw = 256; bb = 84; break;
    case 11: blk = blk_q3_k; bw = 256; bb = 110; break;
    case 13: blk = blk_q5_k; bw = 256; bb = 176; break;
    case 15: blk = blk_q8_k; bw = 256; bb = 292; break;
    case 14: blk = blk_q6_k; bw = 256; bb = 210; break;
    default:
        memset(out, 0, (size_t)n * 4);
        return;
    }
    while (done < n) {
        blk(p, out + done);
        p += bb;
        done += bw;
    }
}

void tbo_dequant_rows(const void *W, int qtype, int M, int K, float *out) {
    size_t rb = tbo_row_bytes(qtype, K);
    const uint8_t *p = (const uint8_t *)W;
    for (int m = 0; m < M; m++) tbo_dequant_row(p + (size_t)m * rb, qtype, K, out + (size_t)m * K);
}

/* layer4/tb_gguf.c:376-419.  Row stride ceil(K/bw)*bb; per row: dequantise
 * the whole row, then acc = acc + w[k]*x[k] sequentially from k=0.  qtype 21
 * has a geometry entry but no decoder, so its rows decode to zeros. */
void tbo_dequant_matvec(const void *W, int qtype, int M, int K,
                        const float *x, float *out) {
    size_t rb = tbo_row_bytes(qtype, K);
    if (!rb) {
        memset(out, 0, (size_t)M * 4);
        return;
    }
    float *row = (float *)malloc((size_t)K * 4 + 1024 * 4);
    const uint8_t *p = (const uint8_t *)W;
    for (int m = 0; m < M; m++) {
        tbo_dequant_row(p, qtype, K, row);
        float acc = 0.0f;
        for (int k = 0; k < K; k++) {
            float prod = row[k] * x[k];
            acc = acc + prod;
        }
        out[m] = acc;
        p += rb;
    }
    free(row);
}

/* layer4/tb_infer.c:130-135: out = (g / (1 + expf(-g))) * up. */
void tbo_swiglu(const float *gate, const float *up, float *out, int dim) {
    for (int i = 0; i < dim; i++) {
        float g = gate[i];
        float den = 1.0f + expf(-g);
        float s = g / den;
        out[i] = s * up[i];
    }
}

/* layer4/tb_infer.c:239-377 with ctx->use_hdgl == 0: at most 256 experts are
 * read; softmax with max subtraction and a sequential sum; top-k by a single
 * pass that replaces the first minimal slot when a score is strictly larger
 * (slots start at index 0 / -1e30); weights renormalised by their
 * sequential sum when that sum is positive. */
int tbo_route_experts(const float *logits, int n, int top_k, int idx[8], float w[8]) {
    int k = top_k > 8 ? 8 : top_k;
    float sc[256];
    if (n > 256) n = 256;
    memcpy(sc, logits, (size_t)n * 4);
    float mx = sc[0];
    for (int e = 1; e < n; e++)
        if (sc[e] > mx) mx = sc[e];
    float sum = 0.0f;
    for (int e = 0; e < n; e++) {
        sc[e] = expf(sc[e] - mx);
        sum = sum + sc[e];
    }
    for (int e = 0; e < n; e++) sc[e] = sc[e] / sum;
    for (int i = 0; i < k; i++) {
        idx[i] = 0;
        w[i] = -1e30f;
    }
    for (int e = 0; e < n; e++) {
        int lo = 0;
        for (int i = 1; i < k; i++)
            if (w[i] < w[lo]) lo = i;
        if (sc[e] > w[lo]) {
            w[lo] = sc[e];
            idx[lo] = e;
        }
    }
    float ws = 0.0f;
    for (int i = 0; i < k; i++) ws = ws + w[i];
    if (ws > 0.0f)
        for (int i = 0; i < k; i++) w[i] = w[i] / ws;
    return k;
}

/* Router logits: the reference feeds ffn_gate_inp through a 4-bit "compat"
 * decoder (layer4/tb_infer.c:755-763) that cannot read an F32 GGUF router;
 * the oracle uses the public dequant-matvec with qtype 0 (F32) instead, i.e.
 * a sequential fp32 dot per expert.  The optional bias is added afterwards. */
void tbo_router_logits(int T, int H, int E, const float *xn, const float *router,
                       const float *bias, float *logits) {
    for (int t = 0; t < T; t++) {
        float *lg = logits + (size_t)t * E;
        tbo_dequant_matvec(router, 0, E, H, xn + (size_t)t * H, lg);
        if (bias)
            for (int e = 0; e < E; e++) lg[e] = lg[e] + bias[e];
    }
}

/* layer4/tb_infer.c:753-833 and :876, one token at a time.  Expert e uses
 * gate/up rows [e*F, (e+1)*F) (row bytes for K=H in the gate's and the up
 * tensor's own qtype, :807-812) and down rows [e*H, (e+1)*H) (row bytes for
 * K=F in the down tensor's qtype, :815-816).  The weighted accumulate runs
 * in slot order into a zeroed buffer; the residual is added last. */
void tbo_moe_forward(int T, int H, int F, int E, int top_k, int qg, int qu, int qd,
                     const float *xn, const float *resid, const float *router,
                     const float *bias, const void *gate, const void *up,
                     const void *down, float *out, int *sel_idx, float *sel_w) {
    size_t rbG = tbo_row_bytes(qg, H), rbU = tbo_row_bytes(qu, H), rbF = tbo_row_bytes(qd, F);
    float *lg = (float *)malloc((size_t)E * 4);
    float *g = (float *)malloc((size_t)F * 4);
    float *u = (float *)malloc((size_t)F * 4);
    float *a = (float *)malloc((size_t)F * 4);
    float *y = (float *)malloc((size_t)H * 4);
    float *acc = (float *)malloc((size_t)H * 4);
    for (int t = 0; t < T; t++) {
        const float *x = xn + (size_t)t * H;
        tbo_router_logits(1, H, E, x, router, bias, lg);
        int idx[8];
        float w[8];
        int k = tbo_route_experts(lg, E, top_k, idx, w);
        memset(acc, 0, (size_t)H * 4);
        for (int s = 0; s < k; s++) {
            int e = idx[s];
            const uint8_t *gb = (const uint8_t *)gate + (size_t)e * F * rbG;
            const uint8_t *ub = (const uint8_t *)up + (size_t)e * F * rbU;
            const uint8_t *db = (const uint8_t *)down + (size_t)e * H * rbF;
            tbo_dequant_matvec(gb, qg, F, H, x, g);
            tbo_dequant_matvec(ub, qu, F, H, x, u);
            tbo_swiglu(g, u, a, F);
            tbo_dequant_matvec(db, qd, H, F, a, y);
            for (int i = 0; i < H; i++) {
                float p = w[s] * y[i];
                acc[i] = acc[i] + p;
            }
        }
        const float *r = resid + (size_t)t * H;
        float *o = out + (size_t)t * H;
        for (int i = 0; i < H; i++) o[i] = r[i] + acc[i];
        if (sel_idx)
            for (int s = 0; s < 8; s++) sel_idx[(size_t)t * 8 + s] = s < k ? idx[s] : -1;
        if (sel_w)
            for (int s = 0; s < 8; s++) sel_w[(size_t)t * 8 + s] = s < k ? w[s] : 0.0f;
    }
    free(lg); free(g); free(u); free(a); free(y); free(acc);
}

/* This build's Q8_K activation quantiser (the reference defines only the
 * block layout, layer4/tb_gguf.c:281-288). */
void tbo_quantize_q8k(const float *x, int K, void *blocks) {
    uint8_t *p = (uint8_t *)blocks;
    for (int b = 0; b < K / 256; b++, p += 292) {
        const float *xb = x + (size_t)b * 256;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) {
            float v = fabsf(xb[i]);
            if (v > amax) amax = v;
        }
        float d = amax / 127.0f;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        memcpy(p, &d, 4);
        int8_t *q = (int8_t *)(p + 4);
        for (int i = 0; i < 256; i++) {
            float v = nearbyintf(xb[i] * id);
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            q[i] = (int8_t)v;
        }
        int16_t bs[16];
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += q[j * 16 + i];
            bs[j] = (int16_t)s;
        }
        memcpy(p + 260, bs, 32);
    }
}

void tbo_expf_batch(const float *in, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = expf(in[i]);
}

struct expf_job {
    float (*f)(float);
    uint32_t t, nt;
    long long bad;
};

static void *expf_worker(void *arg) {
    struct expf_job *j = (struct expf_job *)arg;
    long long bad = 0;
    for (uint64_t b = j->t; b < (1ull << 32); b += j->nt) {
        uint32_t u = (uint32_t)b;
        float x;
        memcpy(&x, &u, 4);
        float r = expf(x), m = j->f(x);
        uint32_t ur, um;
        memcpy(&ur, &r, 4);
        memcpy(&um, &m, 4);
        if (ur != um && !(isnan(r) && isnan(m))) bad++;
    }
    j->bad = bad;
    return 0;
}

long long tbo_expf_exhaustive_mismatches(float (*f)(float), int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64];
    struct expf_job jobs[64];
    for (int i = 0; i < nthreads; i++) {
        jobs[i].f = f;
        jobs[i].t = (uint32_t)i;
        jobs[i].nt = (uint32_t)nthreads;
        jobs[i].bad = 0;
        pthread_create(&th[i], 0, expf_worker, &jobs[i]);
    }
    long long bad = 0;
    for (int i = 0; i < nthreads; i++) {
        pthread_join(th[i], 0);
        bad += jobs[i].bad;
    }
    return bad;
}

/* Timing baseline following the structure of tb_dot_q4k_avx512
 * (src/tb_analog_dispatch.c:486-524): per super-block, decode 256 weights
 * into a stack buffer, then a 16-wide FMA dot and one horizontal sum added
 * to the running total.  Decoding uses the oracle's Q4_K semantics. */
float tbo_dot_q4k_avx512s(const uint8_t *row, int K, const float *x) {
    float total = 0.0f;
    float wbuf[256];
    for (int b = 0; b < K / 256; b++) {
        blk_q4_k(row + (size_t)b * 144, wbuf);
        const float *xb = x + (size_t)b * 256;
#if defined(__AVX512F__)
        __m512 acc = _mm512_setzero_ps();
        for (int i = 0; i < 256; i += 16)
            acc = _mm512_fmadd_ps(_mm512_loadu_ps(wbuf + i), _mm512_loadu_ps(xb + i), acc);
        total += _mm512_reduce_add_ps(acc);
#else
        float acc = 0.0f;
        for (int i = 0; i < 256; i++) acc = acc + wbuf[i] * xb[i];
        total += acc;
#endif
    }
    return total;
}

void tbo_matvec_q4k_avx512s(const void *W, int M, int K, const float *x, float *out) {
    size_t rb = (size_t)(K / 256) * 144;
    for (int m = 0; m < M; m++)
        out[m] = tbo_dot_q4k_avx512s((const uint8_t *)W + (size_t)m * rb, K, x);
}

int tbo_have_avx512(void) {
#if defined(__AVX512F__)
    return 1;
#else
    return 0;
#endif
}
