/*
 * ref_harness.c -- thin driver linked with the reference's own C sources
 * (compiled from /root/reference by oracle/Makefile into oracle/_ref/).  It
 * lets the tests and the CPU baseline call the reference functions that
 * need a context struct.  Only tests/, tests/golden/make_golden.py and
 * bench.py's cpu_baseline leg load the resulting library.
 *
 * Wrapped reference entry points:
 *   tb_route_experts   layer4/tb_infer.h:120-122 (use_hdgl=0 context)
 *   tb_swiglu          layer4/tb_infer.c:130-135 (no prototype in a header)
 *   tb_dispatch_matvec src/tb_analog_dispatch.h:102-105 (AVX-512 class)
 *   the MoE branch of tb_layer_forward (layer4/tb_infer.c:753-833), composed
 *   of tb_gguf_dequant_matvec, tb_route_experts and tb_swiglu
 * tb_gguf_dequant_row / tb_gguf_dequant_matvec (layer4/tb_gguf.h:90,95) are
 * exported by the reference objects themselves and called directly.
 */
#include <stdlib.h>
#include <string.h>

#include "tb_infer.h"

void tb_swiglu(const float *gate, const float *up, float *out, int dim);

/* Row bytes of the packed expert tensors, as the _RB macro of
 * layer4/tb_infer.c:806 computes them. */
static long tb_gguf_row_bytes_ref(int qt, int K) {
    return qt == 12 ? (long)(K / 256) * 144 : qt == 11 ? (long)(K / 256) * 110 : qt == 13 ? (long)(K / 256) * 176
         : qt == 14 ? (long)(K / 256) * 210 : qt == 15 ? (long)(K / 256) * 292 : qt == 8 ? (long)(K / 32) * 34
         : qt == 2 ? (long)(K / 32) * 18 : (long)K * 4;
}

int tbref_route(const float *logits, int n_experts, int top_k, int idx[8], float w[8]) {
    TB_GGUFModel *m = (TB_GGUFModel *)calloc(1, sizeof(TB_GGUFModel));
    TB_InferCtx *ctx = (TB_InferCtx *)calloc(1, sizeof(TB_InferCtx));
    m->n_experts_per_tok = top_k;
    ctx->model = m;
    ctx->use_hdgl = 0;
    ctx->hdgl_alpha = 0.0f;
    TB_ExpertSelection sel = tb_route_experts(ctx, 0, 0, logits, n_experts);
    for (int i = 0; i < 8; i++) {
        idx[i] = i < sel.k ? sel.expert_indices[i] : -1;
        w[i] = i < sel.k ? sel.expert_weights[i] : 0.0f;
    }
    free(ctx);
    free(m);
    return sel.k;
}

void tbref_swiglu(const float *gate, const float *up, float *out, int dim) {
    tb_swiglu(gate, up, out, dim);
}

/* The reference's CPU matvec as the forward pass runs it once the dispatch
 * context is set: a warmed-up oscillator in phase 0 on an AVX-512 host
 * selects the AVX-512 kernels (src/tb_analog_dispatch.c:111-145). */
void tbref_dispatch_matvec_avx512(const void *W, int qtype, int M, int K,
                                  const float *x, float *out) {
    TBOscSnapshot snap;
    memset(&snap, 0, sizeof(snap));
    snap.steps = 100;
    snap.s_u = 1.0;
    snap.aphase = 0;
    TBCpuCaps caps;
    memset(&caps, 0, sizeof(caps));
    caps.have_avx2 = 1;
    caps.have_avx512f = 1;
    caps.have_fma = 1;
    tb_dispatch_matvec(W, qtype, M, K, x, out, &snap, &caps);
}

int tbref_sizeof_selection(void) { return (int)sizeof(TB_ExpertSelection); }

/* The MoE branch of tb_layer_forward (layer4/tb_infer.c:753-833, residual
 * :876) for T tokens, composed of the reference's own functions as that
 * branch calls them: router logits by tb_gguf_dequant_matvec on the fp32
 * router (the 4-bit-compat router call at :759-763 cannot read an fp32
 * ffn_gate_inp), tb_route_experts, two tb_gguf_dequant_matvec + tb_swiglu +
 * one tb_gguf_dequant_matvec per slot on the packed expert rows (:794-820,
 * with the three mallocs per slot), each tensor read in its own qtype qg, qu
 * and qd with row bytes from its own format (:807-816), the weighted
 * accumulate (:829-831) and the residual add.  The CPU baseline of the MoE
 * block (one thread). */
void tbref_moe_block(int T, int H, int F, int E, int top_k, int qg, int qu, int qd, const float *xn,
                     const float *resid, const float *router, const void *gate, const void *up, const void *down,
                     float *out) {
    TB_GGUFModel *m = (TB_GGUFModel *)calloc(1, sizeof(TB_GGUFModel));
    TB_InferCtx *ctx = (TB_InferCtx *)calloc(1, sizeof(TB_InferCtx));
    m->n_experts_per_tok = top_k;
    ctx->model = m;
    const size_t rb_g = (size_t)tb_gguf_row_bytes_ref(qg, H), rb_u = (size_t)tb_gguf_row_bytes_ref(qu, H),
                 rb_f = (size_t)tb_gguf_row_bytes_ref(qd, F);
    for (int t = 0; t < T; t++) {
        const float *x = xn + (size_t)t * H;
        float *lg = (float *)calloc(E, sizeof(float));
        tb_gguf_dequant_matvec(router, 0, E, H, x, lg);
        TB_ExpertSelection sel = tb_route_experts(ctx, 0, 0, lg, E);
        free(lg);
        float *ffn = (float *)calloc(H, sizeof(float));
        float *eo = (float *)calloc(H, sizeof(float));
        for (int ei = 0; ei < sel.k; ei++) {
            const int e = sel.expert_indices[ei];
            float *g = (float *)malloc(F * sizeof(float));
            float *u = (float *)malloc(F * sizeof(float));
            float *a = (float *)malloc(F * sizeof(float));
            tb_gguf_dequant_matvec((const char *)gate + (size_t)e * F * rb_g, qg, F, H, x, g);
            tb_gguf_dequant_matvec((const char *)up + (size_t)e * F * rb_u, qu, F, H, x, u);
            tb_swiglu(g, u, a, F);
            tb_gguf_dequant_matvec((const char *)down + (size_t)e * H * rb_f, qd, H, F, a, eo);
            free(g); free(u); free(a);
            const float w = sel.expert_weights[ei];
            for (int i = 0; i < H; i++) ffn[i] += w * eo[i];
        }
        for (int i = 0; i < H; i++) out[(size_t)t * H + i] = resid[(size_t)t * H + i] + ffn[i];
        free(ffn);
        free(eo);
    }
    free(ctx);
    free(m);
}
