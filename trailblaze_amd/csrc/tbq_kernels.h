// tbq_kernels.h -- launchers shared between the kernel files and the C-ABI
// shim (tbq_api.hip).  Internal to libtbq; the public surface is include/.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/tbq.h"

namespace tbq {

// Longest row (K) tbq_matvec takes: the int-dot kernel stages all of x in
// LDS (224 bytes per 64 elements).
constexpr int TBQ_MAX_K = 32768;

// Fusions of the dense decode's elementwise steps into a matvec, so they
// need no launch of their own.  Staging prologue (how x is formed):
//   PRO_NONE    x
//   PRO_NORM    v = x[i] + y[i] (y may be null),
//               x'[i] = v * (1 / sqrt(mean(v^2) + eps)) * w[i] over the K
//               elements; workgroup 0 also stores v to vo (if not null)
//   PRO_NORMD   x'[i] = x[i] * w[i], and every output row (both rows of a
//               GLU pair) multiplied by r = 1 / sqrt(sum(x^2) / K + eps)
//               after its dot product: the same function as PRO_NORM with
//               y = null, the scalar r applied after the sum instead of to
//               every element.  The sum of squares is taken over the x the
//               workgroup stages anyway (each wave's share to LDS before the
//               staging barrier, then summed in wave order), so it costs
//               neither loads nor a barrier of its own.
// Every workgroup forms the whole normalised vector (or r) itself, so no
// workgroup waits for another.  Epilogue flag MV_GLU (K-quant kernel): W
// holds 2M rows, gate rows then up rows, and y[r] = silu(W[r] x') *
// (W[M + r] x'); one wave computes both rows.  Epilogue PRO_RES (no
// prologue): y is the residual stream, y[r] += W[r] x.
enum : int { PRO_NONE = 0, PRO_NORMD = 1, PRO_NORM = 2, MV_GLU = 4, PRO_RES = 8 };
struct MvPro {
    const float *y;   // PRO_NORM: added to x (null: nothing added)
    const float *w;   // PRO_NORM, PRO_NORMD: weights [K]
    float *vo;        // PRO_NORM: x + y for the caller (null: not stored)
    float eps;
    long long rb;     // K-quant kernel: bytes between rows (0: K's own row bytes), for
                      // a column slice of a matrix with longer rows
};

struct MoeArgs {
    int T, H, F, E, top_k, k;
    int qg, qu, qd;    // qtypes of the gate, up and down expert tensors
    const float *xn, *resid, *router, *bias;
    const void *gate, *up, *down;
    float *out;
    float *logits;     // [T][E]
    unsigned *counters; // [T], zero between calls (router arrival counters)
    int *sel_idx;      // [T][8]
    float *sel_w;      // [T][8]
    float *act;        // [T*k][F]
    float *y;          // [T*k][H]
    int *grp;          // decode order by expert: 2 + 3E + T*k ints (null: the per-pair order)
    float *u;          // [T*k][F] up products when a.qg != a.qu (null otherwise)
};

hipError_t launch_dequant(int qt, const void *W, long long nweights, float *out, hipStream_t s);
hipError_t launch_dequant_rows(int qt, const void *W, const int *idx, int nrows, int K, float *out, hipStream_t s);
hipError_t launch_dequant_f16(int qt, const void *W, long long nweights, _Float16 *out, hipStream_t s);
hipError_t launch_matvec_generic(int qt, const void *W, int M, int K, const float *x, float *y,
                                 hipStream_t s, int n_cu);
// The Q4_K kernels read the reference's layout, or ggml's (QT_GQ4_K) when ggml.
hipError_t launch_matvec_q4k(const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu,
                             bool ggml = false);
hipError_t launch_matvec_kq(int qt, const void *W, int M, int K, const float *x, float *y, hipStream_t s, int n_cu);
// The same kernels with a staging prologue or epilogue (mode = PRO_* |
// MV_GLU); hipErrorNotSupported where they do not cover the shape or mode
// (the q4k one: K <= 4096, no MV_GLU).
hipError_t launch_matvec_q4k_pro(int mode, const MvPro &pro, const void *W, int M, int K, const float *x, float *y,
                                 hipStream_t s, bool ggml = false);
hipError_t launch_matvec_kq_pro(int mode, const MvPro &pro, int qt, const void *W, int M, int K, const float *x,
                                float *y, hipStream_t s, int n_cu);
hipError_t launch_expf(const float *in, float *out, long long n, hipStream_t s);
// y[i] = (((y[i] + part[0][i]) + part[1][i]) + ...) over nparts rows of M
// floats: the column slices of a matvec with rows longer than TBQ_MAX_K.
hipError_t launch_add_rows(float *y, const float *part, int nparts, int M, hipStream_t s);
hipError_t launch_route(const float *xn, const float *router, const float *bias, int T, int H, int E,
                        int top_k, int *sel_idx, float *sel_w, hipStream_t st);
hipError_t launch_moe_fp32(const MoeArgs &a, hipStream_t st);
// out = resid + sum over slots, in slot order, of sel_w * y[t*k + s]
hipError_t launch_combine(const MoeArgs &a, hipStream_t st);
// group: the layer call whose batch the router may also sort by expert (its
// grp list, when moe_decode_grouped); *grouped tells whether it did.
hipError_t launch_router(const float *xn, const float *router, const float *bias, int T, int H, int E, int top_k,
                         float *logits, unsigned *counters, int *sel_idx, float *sel_w, hipStream_t st,
                         _Float16 *x16 = nullptr, float *xinv = nullptr, bool *x16_done = nullptr,
                         const MoeArgs *group = nullptr, bool *grouped = nullptr);
// Decode expert kernels for Q4_K tensors (tbq_moe_q4k.hip).  A batch runs in
// expert order when moe_decode_grouped(a): launch_group writes a.grp first.
bool moe_decode_grouped(const MoeArgs &a);
hipError_t launch_group(const MoeArgs &a, hipStream_t st);
// act = swiglu(gate x, up x); a.qg == a.qu, QT_Q4_K or QT_GQ4_K
hipError_t launch_moe_q4k_gate_up(const MoeArgs &a, bool grouped, hipStream_t st);
// out = resid + combine(down act); a.qd QT_Q4_K or QT_GQ4_K
hipError_t launch_moe_q4k_down(const MoeArgs &a, bool grouped, hipStream_t st);
// The same two phases on the K-quant int-dot units for the other expert
// formats (tbq_mv_kq.hip; gate and up in one format); hipErrorNotSupported
// for shapes and formats they do not cover.
// grouped: the batch runs in expert order (a.grp written by launch_group);
// the grouped down writes a.y and adds launch_combine.
hipError_t launch_moe_gate_up_kq(const MoeArgs &a, bool grouped, hipStream_t st);
hipError_t launch_moe_down_kq(const MoeArgs &a, bool grouped, hipStream_t st);
size_t prefill_workspace_bytes(int T, int k, int E, int H, int F);
bool gemm_k_supported(int K);
// rows of n floats to fp16 with per-row power-of-two scales (inv = 1 / scale)
hipError_t launch_rows_f16(const float *in, int rows, int n, _Float16 *out, float *inv, hipStream_t st);
hipError_t launch_moe_prefill_q4k(const MoeArgs &a, void *scratch, hipStream_t st, bool x16_done = false);
// Where the prefill scratch keeps the tokens' fp16 rows and their inverse
// scales (so the router can write them).
void prefill_x16(const MoeArgs &a, void *scratch, _Float16 **x16, float **xinv);
hipError_t launch_moe_bf16(const MoeArgs &a, void *scratch, hipStream_t st);
// int8 MFMA prefill (TBQ_MOE_I8): Q8_K activations against the Q4_K nibbles
size_t prefill_i8_workspace_bytes(int T, int k, int E, int H, int F);
hipError_t launch_rows_q8(const float *in, long long rows, int n, int8_t *q8, float *dq, _Float16 *bs16,
                          hipStream_t st);
hipError_t launch_moe_prefill_q4k_i8(const MoeArgs &a, void *scratch, hipStream_t st);
hipError_t launch_quantize_q8k(const float *in, long long n, void *blocks, hipStream_t st);
hipError_t launch_moe_i8(const MoeArgs &a, void *scratch, hipStream_t st);
// Prefill weight products (tbq_gemm.hip): C[T][N] (row stride ldc) =
// X[T][K] . W[N][K]^T, X fp16, W fp16 (QT_F16) or Q4_K rows; N % 4 == 0,
// K % 256 == 0; part = hgemm_partial_bytes() of scratch.
int hgemm_cus();
bool hgemm_supported(int wqt, int N, int K);
size_t hgemm_partial_bytes(int T, int N, int K, int n_cu);
// With nslices set, the K slices' partial sums are left for the consumer to
// add (in slice order): *nslices = S, and slice z is part + z * T * N (row
// stride N) when S > 1; with S = 1 the product is in C as usual.
hipError_t launch_hgemm(int wqt, const void *W, const _Float16 *X, int T, int N, int K, float *C, int ldc,
                        float *part, int n_cu, hipStream_t st, int *nslices = nullptr);
// The gate|up product (W: 2F rows, gate then up) with SwiGLU in the
// epilogue: A[T][F] (row stride lda) = silu(g xs) (u xs), xs = X's row
// scales; hipErrorNotSupported where it would need split K or F % 64 != 0.
hipError_t launch_hgemm_glu(int wqt, const void *W, const _Float16 *X, const float *xs, int T, int F, int K,
                            float *A, int lda, int n_cu, hipStream_t st);
int hgemm_slices(int T, int N, int K, int n_cu);
size_t dense_workspace_bytes(const tbq_dense_model *m);
hipError_t launch_dense_decode(const tbq_dense_model *m, int token, int pos, float *logits, void *ws,
                               hipStream_t st);
hipError_t dense_final_logits(const tbq_dense_model *m, const float *x, const float *y, float *logits, void *ws,
                              hipStream_t st);
// Batched prefill (tbq_dense_prefill.hip): whether the model takes the
// batched path, its workspace, and the T-token prefill (the decode step per
// token where the batched path does not apply).
bool dense_prefill_batched(const tbq_dense_model *m);
size_t dense_prefill_workspace_bytes(const tbq_dense_model *m, int T);
hipError_t launch_dense_prefill(const tbq_dense_model *m, const int *tokens_host, int T, int pos0, float *logits,
                                void *ws, hipStream_t st);

}  // namespace tbq
