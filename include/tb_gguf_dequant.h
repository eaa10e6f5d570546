/*
 * tb_gguf_dequant.h -- the reference's GPU dequant-matvec ABI, served by
 * libtbq on MI355X (gfx950).  Same names, signatures and 1/0 return
 * contract as the reference header layer4/tb_gguf_dequant.h:19-43, so the
 * reference's callers (layer4/tb_gguf.c:446,505,837,842 and
 * layer4/tb_infer.c:198) link against libtbq unchanged.  The names keep the
 * reference's tb_cuda_ prefix for ABI compatibility; the implementation is
 * HIP for gfx950 (the C11 layer trailblaze_amd/host/tb_cuda_abi.c over the
 * device API in tbq.h).
 *
 * Threading: the legacy global-context calls are serialised by an internal
 * mutex (the reference relies on its generate_lock instead).
 */
#ifndef TB_GGUF_DEQUANT_H
#define TB_GGUF_DEQUANT_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef TB_ANALOG_DISPATCH_SNAPSHOT_DEFINED
#define TB_ANALOG_DISPATCH_SNAPSHOT_DEFINED
/* Layout-identical to TBOscSnapshot in src/tb_analog_dispatch.h:51-58.  When
 * building inside the reference tree, include the reference header first and
 * define TB_ANALOG_DISPATCH_SNAPSHOT_DEFINED. */
typedef struct {
    double phase_var;
    double s_u;
    double lambda_u;
    double omega_u;
    int aphase;
    int steps;
} TBOscSnapshot;
#endif

/* layer4/tb_gguf_dequant.h:19.  1 = device ready (prints its name), 0 = none. */
int tb_cuda_init(void);

/* layer4/tb_gguf_dequant.h:22-23.  Device copy of a host blob / free it. */
void *tb_cuda_upload_tensor(const void *host_data, size_t byte_count);
void tb_cuda_free_tensor(void *d_ptr);

/* layer4/tb_gguf_dequant.h:27.  Stage x on the device (kept for ABI; the
 * matvec below copies its own x, as the reference's does). */
int tb_cuda_upload_x(const float *x_host, int K);

/* layer4/tb_gguf_dequant.h:31.  Accepted and stored; launch shapes on
 * gfx950 do not depend on the oscillator state. */
void tb_cuda_set_snap(const TBOscSnapshot *snap);

/* layer4/tb_gguf_dequant.h:36-37.  out_host[M] = dequant(W_device) . x_host,
 * synchronous.  1 = done; 0 = unsupported qtype or error, and the caller
 * recomputes on the CPU (layer4/tb_gguf.c:444-451).  Supported: 0 1 2 8 10
 * 11 12 13 14 15 30 (the reference's kernel set plus Q2_K; qtype 21, which
 * the reference's CPU path decodes as zeros, returns 0). */
int tb_cuda_matvec_device(const void *W_device, int qtype, int M, int K, const float *x_host,
                          float *out_host);

/* layer4/tb_gguf_dequant.h:40,43. */
void tb_cuda_sync_all(void);
void tb_cuda_cleanup(void);

#ifdef __cplusplus
}
#endif

#endif
