/*
 * tbq_moe_host.c -- the MoE branch of the reference's tb_layer_forward
 * (layer4/tb_infer.c:753-833, residual :876) as one call for a C11 forward
 * pass that holds its activations in host memory: copy xn and the residual
 * to the device, run the gfx950 MoE layer, copy the output (and the routing)
 * back.  Device buffers are cached between calls and guarded by a mutex.
 * A prefill mode that does not take the layer (its experts are not all
 * reference-layout Q4_K) runs the layer on the fp32 decode kernels instead.
 *
 * Buffer layout: the tbq_moe_forward workspace first, at offset 0, so its
 * router arrival counters (the first 256 KiB, which must be zero before a
 * call and are left zero by it) sit at the same address whatever T and the
 * mode are; then xn, resid, out, sel_idx and sel_w.  The counter area is
 * zeroed whenever the buffer is (re)allocated.
 */
#define _POSIX_C_SOURCE 200809L
#include <pthread.h>
#include <stddef.h>

#include "../../include/tbq.h"

/* tbq_api.hip (hidden): synchronous zero fill of device memory */
int tbq_host_zero(void *dev, size_t bytes);
/* tbq_api.hip (hidden): bytes at the start of a MoE workspace that hold the
 * router arrival counters */
size_t tbq_moe_counter_bytes(void);

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static void *g_buf = NULL;
static size_t g_cap = 0;

static size_t up256(size_t n) { return (n + 255) & ~(size_t)255; }

int tbq_moe_block_host(const tbq_moe_layer *L, int T, const float *xn_host, const float *resid_host,
                       float *out_host, int *sel_idx_host, float *sel_w_host, int mode) {
    if (!L || T <= 0 || !xn_host || !resid_host || !out_host) return 0;
    if (mode != TBQ_MOE_FP32 && !tbq_moe_mode_supported(L, mode)) mode = TBQ_MOE_FP32;
    size_t ws = up256(tbq_moe_workspace_size(L, T, mode));
    if (ws == 0) return 0;
    size_t act = up256((size_t)T * L->H * sizeof(float));
    size_t sel = up256((size_t)T * 8 * sizeof(float));
    size_t need = ws + 3 * act + 2 * sel;
    pthread_mutex_lock(&g_mu);
    int ok = 1;
    if (g_cap < need) {
        tbq_free(g_buf);
        g_buf = tbq_malloc(need);
        g_cap = 0;
        ok = g_buf != NULL && tbq_host_zero(g_buf, tbq_moe_counter_bytes());
        if (ok) g_cap = need;
    }
    if (ok) {
        char *b = (char *)g_buf;
        void *d_ws = b;
        float *d_xn = (float *)(b + ws);
        float *d_res = (float *)(b + ws + act);
        float *d_out = (float *)(b + ws + 2 * act);
        int *d_idx = (int *)(b + ws + 3 * act);
        float *d_w = (float *)(b + ws + 3 * act + sel);
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
