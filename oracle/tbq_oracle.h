/*
 * tbq_oracle.h -- CPU restatement of Trailblaze's K-quant dequant-matvec and
 * MoE block, used ONLY as the parity checker (tests/, __graft_entry__.smoke())
 * and as the timed CPU baseline (bench.py cpu_baseline leg).  Nothing in the
 * product library links or calls this code.
 *
 * Every function states the reference file:line it restates.  Floating-point
 * semantics follow the reference's Linux build (scripts/build.sh:27,
 * -std=c11): no FMA contraction, every multiply and add rounds separately,
 * every reduction is strictly sequential.  This file is compiled with
 * -std=c11 -ffp-contract=off for the same reason.
 *
 * Pinning status of each function (what checks it, see tests/):
 *   tbo_f16_to_f32         all 65536 inputs vs the bit formula + KATs
 *                          (layer4/tb_gguf.c:998-1007) + compiled reference
 *   tbo_bf16_to_f32        KAT (layer4/tb_gguf.c:1009-1014)
 *   tbo_dequant_row        KATs (Q8_0 :1016-1033, Q4_0 :1035-1052, Q4_K
 *                          smoke :1054-1070), one-hot bit-layout probes,
 *                          golden vectors from the compiled reference
 *   tbo_dequant_matvec     F32/BF16 identity KATs (:1072-1092), exact
 *                          one-hot matrices, float64 error bound, golden
 *                          vectors from the compiled reference (bit-exact)
 *   tbo_route_experts      brute force over k-subsets on small E, golden
 *                          vectors from the compiled reference (bit-exact)
 *   tbo_swiglu             closed form + golden vectors
 *   tbo_moe_forward        golden vectors from the compiled reference
 *   tbo_quantize_q8k       the reference has no Q8_K activation quantiser
 *                          (it fixes the block layout, layer4/tb_gguf.c:
 *                          281-288); pinned by what a max-abs quantiser
 *                          must satisfy: d bit-equal to fl(max|x|/127),
 *                          |x - d q| <= d/2, the extremal element at +-127
 *                          with its sign, the zero block, bsums, round half
 *                          to even; and its blocks decode through the
 *                          reference-pinned Q8_K decoder to d q
 *   tbo_dot_q4k_avx512s    the CPU timing baseline's restatement: exact on
 *                          integer-valued matrices (bit-equal to the exact
 *                          sum) and within 1e-5 of tbo_dequant_matvec at
 *                          configs[0] (same decode, another sum order)
 *   tbo_f16_ieee,          ggml's layouts (qtype | 0x100, ggml_layout.c):
 *   tbo_ggml_dequant_row   f16 against numpy on all 65536 inputs; decoders
 *                          against an independent block packer and closed
 *                          forms.  ggml is absent here: parity unpinned
 *                          against ggml's own output.
 */
#ifndef TBQ_ORACLE_H
#define TBQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float tbo_f16_to_f32(uint16_t h);
float tbo_bf16_to_f32(uint16_t b);

/* Block geometry for a ggml qtype id: weights per block, bytes per block.
 * Returns 0 for an unknown qtype. */
int tbo_block_geometry(int qtype, int *block_weights, int *block_bytes);
size_t tbo_row_bytes(int qtype, int K);

/* qtype | 0x100 selects ggml's layout of the format (ggml_layout.c). */
void tbo_dequant_row(const void *data, int qtype, int n_weights, float *out);
/* ggml's dequantize_row_* for qtype | 0x100 (or the plain id); 0 = unknown
 * format (out zeroed). */
int tbo_ggml_dequant_row(const void *data, int qtype, int n_weights, float *out);
/* IEEE binary16 -> binary32 (ggml's GGML_FP16_TO_FP32). */
float tbo_f16_ieee(uint16_t h);
void tbo_dequant_matvec(const void *W, int qtype, int M, int K,
                        const float *x, float *out);
/* Dequantise M rows of K weights into out[M*K] (row stride tbo_row_bytes). */
void tbo_dequant_rows(const void *W, int qtype, int M, int K, float *out);

void tbo_swiglu(const float *gate, const float *up, float *out, int dim);

/* Routing with use_hdgl=0.  Writes k=min(top_k,8) indices and weights in the
 * reference's slot order.  Returns k. */
int tbo_route_experts(const float *gate_logits, int n_experts, int top_k,
                      int idx[8], float w[8]);

/* One MoE block for T tokens (each token independent, as the reference's
 * token-by-token decode/prefill does).
 *   xn      [T][H]  post-norm activations (router + expert input)
 *   resid   [T][H]  residual stream x2
 *   router  [E][H]  fp32 router weights (ffn_gate_inp, F32)
 *   bias    [E]     optional per-expert logit bias (NULL = none), added
 *                   to the logits before routing
 *   gate/up packed [E*F rows][H] in qtypes qg/qu, down packed [E*H rows][F]
 *           in qtype qd (each tensor's own format)
 *   out     [T][H]  resid + weighted sum of expert outputs
 *   sel_idx/sel_w [T][8] optional (may be NULL) */
void tbo_moe_forward(int T, int H, int F, int E, int top_k, int qg, int qu, int qd,
                     const float *xn, const float *resid,
                     const float *router, const float *bias,
                     const void *gate, const void *up, const void *down,
                     float *out, int *sel_idx, float *sel_w);

/* Router logits only (F32 sequential matvec + optional bias), [T][E]. */
void tbo_router_logits(int T, int H, int E, const float *xn,
                       const float *router, const float *bias, float *logits);

/* Q8_K activation quantiser (this build's definition): per 256-element block
 * d = max|x|/127 (f32), q = nearbyint(x/d) clamped to [-127,127], bsums[16]
 * = sums of 16 consecutive q.  292-byte blocks in the reference Q8_K layout
 * (layer4/tb_gguf.c:281-288). */
void tbo_quantize_q8k(const float *x, int K, void *blocks);

/* glibc expf over a buffer (the reference's expf). */
void tbo_expf_batch(const float *in, float *out, size_t n);
/* Exhaustive comparison of f against glibc expf over all 2^32 inputs using
 * nthreads threads.  Returns the number of bit mismatches (NaN outputs
 * compare equal when both are NaN). */
long long tbo_expf_exhaustive_mismatches(float (*f)(float), int nthreads);

/* Timing baseline: the structure of the reference's AVX-512 Q4_K row dot
 * (dequantise one super-block to a stack buffer, 16-wide FMA, one horizontal
 * reduction per super-block) with the oracle's decoding. */
float tbo_dot_q4k_avx512s(const uint8_t *row, int K, const float *x);
void tbo_matvec_q4k_avx512s(const void *W, int M, int K, const float *x,
                            float *out);
int tbo_have_avx512(void);

#ifdef __cplusplus
}
#endif
#endif
