/*
 * tb_cuda_abi.c -- the reference's GPU matvec ABI (layer4/tb_gguf_dequant.h,
 * declared again in include/tb_gguf_dequant.h) implemented in C11 over the
 * device API of include/tbq.h.  Replaces the host half of
 * layer4/tb_gguf_dequant.cu:337-486: one synchronous matvec per call, the
 * same persistent-buffer scheme, the same 1/0 + CPU-fallback contract
 * (layer4/tb_gguf.c:444-451).  The kernels behind tbq_matvec are gfx950 HIP.
 */
#define _POSIX_C_SOURCE 200809L
#include <pthread.h>
#include <stdio.h>
#include <string.h>

#include "../../include/tb_gguf_dequant.h"
#include "../../include/tbq.h"

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static float *g_d_x = NULL;   /* device x, capacity g_cap_x floats */
static int g_cap_x = 0;
static float *g_d_y = NULL;   /* device y, capacity g_cap_y floats */
static int g_cap_y = 0;
static const TBOscSnapshot *g_snap = NULL;

/* layer4/tb_gguf_dequant.cu:388-400 prints the device and returns 1. */
int tb_cuda_init(void) {
    if (!tbq_init()) {
        fprintf(stderr, "[tbq] no device: %s\n", tbq_last_error());
        return 0;
    }
    printf("[tbq] %s  %d CUs  gfx950 K-quant matvec + MoE\n", tbq_device_name(), tbq_cu_count());
    return 1;
}

/* layer4/tb_gguf_dequant.cu:411-416: allocate + synchronous copy, NULL on
 * failure (the caller then keeps the tensor on the CPU). */
void *tb_cuda_upload_tensor(const void *host_data, size_t byte_count) {
    void *d = tbq_malloc(byte_count);
    if (!d) return NULL;
    if (!tbq_memcpy_h2d(d, host_data, byte_count, NULL) || !tbq_stream_sync(NULL)) {
        tbq_free(d);
        return NULL;
    }
    return d;
}

void tb_cuda_free_tensor(void *d_ptr) {
    if (d_ptr) tbq_free(d_ptr);
}

static int ensure_x(int K) {
    if (K <= g_cap_x) return 1;
    tbq_free(g_d_x);
    g_d_x = (float *)tbq_malloc((size_t)K * sizeof(float));
    g_cap_x = g_d_x ? K : 0;
    return g_d_x != NULL;
}

static int ensure_y(int M) {
    if (M <= g_cap_y) return 1;
    tbq_free(g_d_y);
    g_d_y = (float *)tbq_malloc((size_t)M * sizeof(float));
    g_cap_y = g_d_y ? M : 0;
    return g_d_y != NULL;
}

/* layer4/tb_gguf_dequant.cu:403-409 */
int tb_cuda_upload_x(const float *x_host, int K) {
    pthread_mutex_lock(&g_mu);
    int ok = K > 0 && ensure_x(K) && tbq_memcpy_h2d(g_d_x, x_host, (size_t)K * 4, NULL) && tbq_stream_sync(NULL);
    pthread_mutex_unlock(&g_mu);
    return ok;
}

void tb_cuda_set_snap(const TBOscSnapshot *snap) { g_snap = snap; }

/* layer4/tb_gguf_dequant.cu:422-472.  qtype 21 (IQ3_S) is refused: the
 * reference's CPU path, which is the parity target, decodes it as zeros. */
int tb_cuda_matvec_device(const void *W_device, int qtype, int M, int K, const float *x_host, float *out_host) {
    if (!W_device || !x_host || !out_host || M <= 0 || K <= 0) return 0;
    if (!tbq_qtype_supported(qtype)) return 0;
    pthread_mutex_lock(&g_mu);
    int ok = ensure_x(K) && ensure_y(M) &&
             tbq_memcpy_h2d(g_d_x, x_host, (size_t)K * 4, NULL) &&
             tbq_matvec(W_device, qtype, M, K, g_d_x, g_d_y, NULL) &&
             tbq_memcpy_d2h(out_host, g_d_y, (size_t)M * 4, NULL) &&
             tbq_stream_sync(NULL);
    pthread_mutex_unlock(&g_mu);
    return ok;
}

void tb_cuda_sync_all(void) {
    if (tbq_init()) tbq_device_sync();
}

void tb_cuda_cleanup(void) {
    pthread_mutex_lock(&g_mu);
    tbq_free(g_d_x);
    tbq_free(g_d_y);
    g_d_x = g_d_y = NULL;
    g_cap_x = g_cap_y = 0;
    g_snap = NULL;
    pthread_mutex_unlock(&g_mu);
}
