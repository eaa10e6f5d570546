/*
 * tbq_moe_host.c -- the MoE branch of the reference's tb_layer_forward
 * (layer4/tb_infer.c:753-833, residual :876) as one call for a C11 forward
 * pass that holds its activations in host memory: copy xn and the residual
 * to the device, run the gfx950 MoE layer, copy the output (and the routing)
 * back.  Device buffers are cached between calls and guarded by a mutex.
 */
#define _POSIX_C_SOURCE 200809L
#include <pthread.h>
#include <stddef.h>

#include "../../include/tbq.h"

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static void *g_buf = NULL;
static size_t g_cap = 0;

static size_t up256(size_t n) { return (n + 255) & ~(size_t)255; }

int tbq_moe_block_host(const tbq_moe_layer *L, int T, const float *xn_host, const float *resid_host,
                       float *out_host, int *sel_idx_host, float *sel_w_host, int mode) {
    if (!L || T <= 0 || !xn_host || !resid_host || !out_host) return 0;
    size_t act = up256((size_t)T * L->H * sizeof(float));
    size_t sel = up256((size_t)T * 8 * sizeof(float));
    size_t ws = tbq_moe_workspace_size(L, T, mode);
    size_t need = 3 * act + 2 * sel + ws;
    pthread_mutex_lock(&g_mu);
    int ok = 1;
    if (g_cap < need) {
        tbq_free(g_buf);
        g_buf = tbq_malloc(need);
        g_cap = g_buf ? need : 0;
        ok = g_buf != NULL;
    }
    if (ok) {
        char *b = (char *)g_buf;
        float *d_xn = (float *)b;
        float *d_res = (float *)(b + act);
        float *d_out = (float *)(b + 2 * act);
        int *d_idx = (int *)(b + 3 * act);
        float *d_w = (float *)(b + 3 * act + sel);
        void *d_ws = b + 3 * act + 2 * sel;
        ok = tbq_memcpy_h2d(d_xn, xn_host, (size_t)T * L->H * 4, NULL) &&
             tbq_memcpy_h2d(d_res, resid_host, (size_t)T * L->H * 4, NULL) &&
             tbq_moe_forward(L, T, d_xn, d_res, d_out, d_idx, d_w, d_ws, ws, mode, NULL) &&
             tbq_memcpy_d2h(out_host, d_out, (size_t)T * L->H * 4, NULL) &&
             (!sel_idx_host || tbq_memcpy_d2h(sel_idx_host, d_idx, (size_t)T * 8 * 4, NULL)) &&
             (!sel_w_host || tbq_memcpy_d2h(sel_w_host, d_w, (size_t)T * 8 * 4, NULL)) &&
             tbq_stream_sync(NULL);
    }
    pthread_mutex_unlock(&g_mu);
    return ok;
}
