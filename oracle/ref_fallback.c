/*
 * ref_fallback.c -- checks the reference's GPU drop-in contract end to end
 * on a host where libtbq has no device (run with TBQ_FORCE_NO_DEVICE=1).
 * Linked by `make -C oracle ref-tbcuda` with the reference's own
 * layer4/tb_gguf.c compiled with -DTB_CUDA (so its guarded calls into
 * tb_cuda_* are live) and with libtbq.so; output only into oracle/_ref/.
 * Test infrastructure: run by tests/test_host_cpu.py only.
 *
 * The three cases the reference handles by recomputing on the CPU
 * (layer4/tb_gguf.c:444-451 for the matvec, :505-514 for the upload):
 *   1. no device: tb_cuda_init() returns 0, tb_cuda_upload_tensor() NULL,
 *      and tb_gguf_tensor_matvec() on a tensor that still carries a
 *      device pointer falls through to the CPU;
 *   2. an unsupported qtype (IQ3_S, 21): tb_cuda_matvec_device returns 0
 *      before touching the device pointer;
 *   3. a NULL device pointer: the CPU path directly.
 * Each matvec must equal tb_gguf_dequant_matvec bit for bit.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tb_gguf.h"
#include "tb_gguf_dequant.h"

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (uint32_t)(rng_state >> 16);
}

static int check(const char *what, const TB_GGUFLoaded *g, TB_GGUFTensorInfo *t, int M, int K, const float *x,
                 const void *W) {
    float *a = malloc((size_t)M * 4), *b = malloc((size_t)M * 4);
    memset(a, 0xFF, (size_t)M * 4);
    tb_gguf_tensor_matvec(g, t, M, K, x, a);
    tb_gguf_dequant_matvec(W, t->qtype, M, K, x, b);
    int same = memcmp(a, b, (size_t)M * 4) == 0;
    printf("%s: %s\n", what, same ? "cpu result bit-identical" : "MISMATCH");
    free(a);
    free(b);
    return same;
}

int main(void) {
    int ok = 1;
    const int init = tb_cuda_init();
    printf("tb_cuda_init: %d\n", init);
    ok &= init == 0;

    /* a Q4_K matrix: d, dmin small fp16, the other bytes random */
    const int M = 64, K = 512, nb = K / 256;
    const size_t bytes = (size_t)M * nb * 144;
    uint8_t *W = malloc(bytes);
    for (size_t i = 0; i < bytes; i++) W[i] = (uint8_t)rnd();
    for (int r = 0; r < M * nb; r++) {
        W[r * 144 + 1] = 0x1C; /* d, dmin ~ 2^-8 */
        W[r * 144 + 3] = 0x1C;
    }
    float *x = malloc((size_t)K * 4);
    for (int i = 0; i < K; i++) x[i] = (float)((int)(rnd() % 2001) - 1000) / 250.0f;

    void *d = tb_cuda_upload_tensor(W, bytes);
    printf("tb_cuda_upload_tensor: %s\n", d ? "device pointer" : "NULL");
    ok &= d == NULL;

    TB_GGUFLoaded g;
    memset(&g, 0, sizeof g);
    g.weights_data = W;
    TB_GGUFTensorInfo t;
    memset(&t, 0, sizeof t);
    strcpy(t.name, "blk.0.ffn_down.weight");
    t.n_dims = 2;
    t.shape[0] = K;
    t.shape[1] = M;
    t.qtype = 12;
    t.offset = 0;

    /* 1: a stale device pointer with no device behind it */
    t.d_data = (void *)(uintptr_t)0x1000;
    ok &= check("no device", &g, &t, M, K, x, W);
    /* 2: an unsupported qtype with a device pointer (IQ3_S decodes as zeros
     * on the CPU, so the bytes' meaning does not matter here) */
    t.qtype = 21;
    ok &= check("unsupported qtype 21", &g, &t, M, K, x, W);
    t.qtype = 12;
    /* 3: no device pointer */
    t.d_data = NULL;
    ok &= check("NULL device pointer", &g, &t, M, K, x, W);

    /* the synchronous ABI calls themselves */
    float y[4];
    ok &= tb_cuda_matvec_device((void *)(uintptr_t)0x1000, 12, 4, 256, x, y) == 0;
    ok &= tb_cuda_upload_x(x, K) == 0;
    tb_cuda_sync_all();
    tb_cuda_cleanup();
    printf("%s\n", ok ? "PASS" : "FAIL");
    free(W);
    free(x);
    return ok ? 0 : 1;
}
