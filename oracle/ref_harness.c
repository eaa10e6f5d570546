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
 * tb_gguf_dequant_row / tb_gguf_dequant_matvec (layer4/tb_gguf.h:90,95) are
 * exported by the reference objects themselves and called directly.
 */
#include <stdlib.h>
#include <string.h>

#include "tb_infer.h"

void tb_swiglu(const float *gate, const float *up, float *out, int dim);

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
