/*
 * host_mock.c -- a host-memory stand-in for the device half of libtbq,
 * linked with trailblaze_amd/host/tbq_moe_host.c by tests/test_host_cpu.py
 * so the C11 MoE host block can be checked without a GPU.
 *
 * "Device" allocations are plain malloc'd buffers filled with 0xA5 (memory a
 * fresh hipMalloc hands out is not zeroed).  tbq_moe_forward records the
 * workspace pointer of every call, checks that the counter area is zero on
 * entry (the contract of tbq.h), dirties the rest of the workspace and
 * leaves the counters zero, as the real router does; it writes
 * out = resid + 2 * xn so the copies can be checked.  tbq_moe_mode_supported
 * takes the prefill modes for all-Q4_K layers only, as the real one, and the
 * mode of the last call is recorded.
 */
#include <stdlib.h>
#include <string.h>

#include "../include/tbq.h"

#define MOCK_COUNTER_BYTES (256u * 1024u)

static void *g_last_alloc = NULL;
static void *g_last_ws = NULL;
static int g_calls = 0;
static int g_bad_counters = 0;   /* calls that found non-zero counters */
static int g_allocs = 0;
static int g_last_mode = -1;

void *tbq_malloc(size_t bytes) {
    void *p = malloc(bytes ? bytes : 1);
    if (p) memset(p, 0xA5, bytes);
    g_last_alloc = p;
    g_allocs++;
    return p;
}
int tbq_free(void *p) {
    free(p);
    return 1;
}
int tbq_host_zero(void *dev, size_t bytes) {
    memset(dev, 0, bytes);
    return 1;
}
size_t tbq_moe_counter_bytes(void) { return MOCK_COUNTER_BYTES; }
int tbq_memcpy_h2d(void *d, const void *h, size_t n, void *s) {
    (void)s;
    memcpy(d, h, n);
    return 1;
}
int tbq_memcpy_d2h(void *h, const void *d, size_t n, void *s) {
    (void)s;
    memcpy(h, d, n);
    return 1;
}
int tbq_stream_sync(void *s) {
    (void)s;
    return 1;
}

int tbq_moe_mode_supported(const tbq_moe_layer *L, int mode) {
    if (mode == TBQ_MOE_FP32) return 1;
    const int g = L->qt_gate ? L->qt_gate : L->qtype, u = L->qt_up ? L->qt_up : L->qtype,
              d = L->qt_down ? L->qt_down : L->qtype;
    return g == 12 && u == 12 && d == 12;
}

/* grows with T and with the prefill mode, like the real size */
size_t tbq_moe_workspace_size(const tbq_moe_layer *L, int T, int mode) {
    size_t n = MOCK_COUNTER_BYTES + (size_t)T * (L->E + 16) * 4 + (size_t)T * 8 * (L->F + L->H) * 4;
    if (mode == TBQ_MOE_BF16) n += (size_t)T * 8 * 4096;
    return n;
}

int tbq_moe_forward(const tbq_moe_layer *L, int T, const float *xn, const float *resid, float *out, int *sel_idx,
                    float *sel_w, void *workspace, size_t ws_bytes, int mode, void *stream) {
    (void)stream;
    g_calls++;
    g_last_ws = workspace;
    g_last_mode = mode;
    if (ws_bytes < tbq_moe_workspace_size(L, T, mode)) return 0;
    const unsigned char *c = (const unsigned char *)workspace;
    for (size_t i = 0; i < MOCK_COUNTER_BYTES; i++)
        if (c[i]) {
            g_bad_counters++;
            break;
        }
    memset((char *)workspace + MOCK_COUNTER_BYTES, 0x5A, ws_bytes - MOCK_COUNTER_BYTES);
    for (long i = 0; i < (long)T * L->H; i++) out[i] = resid[i] + 2.0f * xn[i];
    for (int i = 0; i < T * 8; i++) {
        sel_idx[i] = i % 8 < L->top_k ? i % L->E : -1;
        sel_w[i] = 0.125f;
    }
    return 1;
}

/* test hooks */
void *mock_last_alloc(void) { return g_last_alloc; }
void *mock_last_ws(void) { return g_last_ws; }
int mock_calls(void) { return g_calls; }
int mock_bad_counters(void) { return g_bad_counters; }
int mock_allocs(void) { return g_allocs; }
int mock_last_mode(void) { return g_last_mode; }
