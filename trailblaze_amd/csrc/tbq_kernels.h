// tbq_kernels.h -- launchers shared between the kernel files and the C-ABI
// shim (tbq_api.hip).  Internal to libtbq; the public surface is include/.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/tbq.h"

namespace tbq {

struct MoeArgs {
    int T, H, F, E, top_k, k, qtype;
    const float *xn, *resid, *router, *bias;
    const void *gate, *up, *down;
    float *out;
    float *logits;     // [T][E]
    unsigned *counters; // [T], zero between calls (router arrival counters)
    int *sel_idx;      // [T][8]
    float *sel_w;      // [T][8]
    float *act;        // [T*k][F]
    float *y;          // [T*k][H]
};

hipError_t launch_dequant(int qt, const void *W, long long nweights, float *out, hipStream_t s);
hipError_t launch_matvec_generic(int qt, const void *W, int M, int K, const float *x, float *y,
                                 hipStream_t s, int n_cu);
hipError_t launch_matvec_q4k(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu);
hipError_t launch_matvec_kq(int qt, const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu);
hipError_t launch_expf(const float *in, float *out, long long n, hipStream_t s);
hipError_t launch_route(const float *xn, const float *router, const float *bias, int T, int H, int E,
                        int top_k, int *sel_idx, float *sel_w, hipStream_t st);
hipError_t launch_moe_fp32(const MoeArgs &a, hipStream_t st);
hipError_t launch_router(const float *xn, const float *router, const float *bias, int T, int H, int E, int top_k,
                         float *logits, unsigned *counters, int *sel_idx, float *sel_w, hipStream_t st);
hipError_t launch_moe_q4k_experts(const MoeArgs &a, hipStream_t st);
size_t prefill_workspace_bytes(int T, int k, int E, int H, int F);
hipError_t launch_moe_prefill_q4k(const MoeArgs &a, void *scratch, hipStream_t st);
hipError_t launch_moe_bf16(const MoeArgs &a, void *scratch, hipStream_t st);
size_t dense_workspace_bytes(const tbq_dense_model *m);
hipError_t launch_dense_decode(const tbq_dense_model *m, int token, int pos, float *logits, void *ws,
                               hipStream_t st);

}  // namespace tbq
