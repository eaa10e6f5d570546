/*
 * tbq.h -- explicit, device-resident C API of libtbq, the gfx950 K-quant
 * dequant-matvec and MoE engine.  All tensor pointers are device pointers
 * (HBM) unless a name says _host; `stream` is a hipStream_t (NULL = the
 * default stream).  Every call enqueues work and returns without waiting.
 * Return convention follows the reference's tb_cuda_* ABI: 1 = done,
 * 0 = unsupported input or HIP error (tbq_last_error() says which).
 *
 * Weight tensors use the reference's block layouts and row-major packing
 * (ceil(K / block_weights) blocks per row, rows contiguous;
 * layer4/tb_gguf.c:376-419).  qtype ids are ggml's (layer4/tb_gguf.h:24):
 * 0 F32, 1 F16, 2 Q4_0, 8 Q8_0, 10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K,
 * 15 Q8_K, 30 BF16.
 *
 * TBQ_GGML | id selects ggml's own on-disk layout of the same format (what
 * llama.cpp writes; ggml-quants.c dequantize_row_*), which the reference's
 * decoders do not read (their comment at layer4/tb_gguf.c:63-85 cites ggml,
 * their code differs): the block fields sit at the same byte offsets, but
 * ggml assigns quant bits to weights in 32-byte runs, unpacks the 6-bit
 * K-quant scales differently and decodes fp16 subnormals as IEEE.  Every
 * call that takes a qtype accepts these ids (for F32, BF16 and Q8_K the two
 * layouts are one); the prefill MFMA modes of tbq_moe_forward take only
 * Q4_K (TBQ_MOE_I8 only the reference's layout of it).
 */
#ifndef TBQ_H
#define TBQ_H

#include <stddef.h>

#define TBQ_GGML 0x100

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime ----------------------------------------------------------- */
/* Select device 0 and cache its properties.  Idempotent.  1 = ready. */
int tbq_init(void);
/* Human-readable reason for the last 0 returned on this thread. */
const char *tbq_last_error(void);
/* Device name and compute-unit count of the selected device (after init). */
const char *tbq_device_name(void);
int tbq_cu_count(void);

void *tbq_malloc(size_t bytes);                 /* NULL on failure */
int tbq_free(void *dev);                        /* NULL-safe */
int tbq_memcpy_h2d(void *dev, const void *host, size_t bytes, void *stream);
int tbq_memcpy_d2h(void *host, const void *dev, size_t bytes, void *stream);
int tbq_stream_sync(void *stream);
int tbq_device_sync(void);

/* ---- formats ----------------------------------------------------------- */
/* Bytes of one row of K weights (0 for an unknown qtype);
 * replaces the geometry table of layer4/tb_gguf.c:380-398. */
size_t tbq_row_bytes(int qtype, int K);
/* 1 if tbq_matvec / tbq_dequant accept qtype. */
int tbq_qtype_supported(int qtype);

/* ---- dequantise (bit-exact hook) --------------------------------------- */
/* out[nrows*K] = the reference's dequantised weights, bit for bit
 * (tb_gguf_dequant_row, layer4/tb_gguf.h:90); for a TBQ_GGML id, ggml's
 * dequantize_row_* values.  K must be a multiple of the block size (and of
 * 8). */
int tbq_dequant(const void *W, int qtype, int nrows, int K, float *out, void *stream);

/* ---- decode matvec ----------------------------------------------------- */
/* y[M] = dequant(W[M][K]) . x[K], fp32 accumulate (tb_gguf_dequant_matvec,
 * layer4/tb_gguf.h:95-96; device-resident form of tb_cuda_matvec_device,
 * layer4/tb_gguf_dequant.h:36-37).  K a multiple of 256 for super-block
 * formats, of 32 otherwise (F32, F16 and BF16 rows at most 15360); W and x
 * 16-byte aligned.  x is staged in LDS, so rows longer than 32768 weights
 * (K-quant formats, Q8_0, Q4_0) run as column slices of 32768 whose partial
 * products are added in slice order; their partial sums live in a
 * library-owned buffer, so such calls must be ordered on one stream. */
int tbq_matvec(const void *W, int qtype, int M, int K, const float *x, float *y, void *stream);

/* Kernel choice for tbq_matvec (no counterpart in the reference: it has one
 * CUDA kernel per format).  AUTO picks the fastest kernel for the shape;
 * FMA is the byte->fp32 fma kernel every format has; INTDOT is the Q4_K
 * v_dot4 kernel specialised for K <= 16384; KQ is the v_dot4 kernel shared
 * by Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, Q4_0 and Q8_K (K a multiple of 64,
 * at most 32768).  INTDOT and KQ fail for shapes they do not cover. */
#define TBQ_MV_AUTO 0
#define TBQ_MV_FMA 1
#define TBQ_MV_INTDOT 2
#define TBQ_MV_KQ 3
int tbq_matvec_variant(const void *W, int qtype, int M, int K, const float *x, float *y, int variant,
                       void *stream);

/* ---- MoE block --------------------------------------------------------- */
/* Router: logits[e] = router[e] . xn (summed in the reference's sequential
 * order) + bias[e]; softmax; top-k in the reference's slot order;
 * renormalised weights (tb_route_experts with use_hdgl=0,
 * layer4/tb_infer.h:120-122).  sel_idx/sel_w are [T][8]; slots >= k hold
 * -1 / 0.  E <= 256, top_k clamped to 8. */
int tbq_route(const float *xn, const float *router, const float *bias, int T, int H, int E,
              int top_k, int *sel_idx, float *sel_w, void *stream);
/* (tbq_route keeps its logits and arrival counters in a library-owned
 * buffer: calls must be ordered on one stream.) */

/* One MoE layer in the reference's packed expert layout
 * (layer4/tb_infer.c:780-806): gate/up are [E*F rows][H], down [E*H rows][F];
 * router is fp32 [E][H].  Each expert tensor has its own qtype, as the
 * reference reads eg_t->qtype, the up tensor's and ed_t->qtype
 * (layer4/tb_infer.c:807-816): qt_gate, qt_up and qt_down, where 0 means
 * `qtype` (so a layer whose three tensors share one format sets only
 * `qtype`).  Row strides follow each tensor's own format.  Expert qtypes:
 * Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, or TBQ_GGML | one of them. */
typedef struct {
    int H, F, E, top_k, qtype;
    const float *router;
    const float *bias;   /* [E] logit bias added before routing, or NULL */
    const void *gate;
    const void *up;
    const void *down;
    int qt_gate, qt_up, qt_down;   /* 0 = qtype */
} tbq_moe_layer;

#define TBQ_MOE_FP32 0      /* fp32 decode kernels; outputs within 1e-5 rel-L2 */
#define TBQ_MOE_BF16 1      /* prefill: grouped 16-bit MFMA (fp16 operands with
                               power-of-two row scaling, fp32 accumulate);
                               within 1e-2 rel-L2 */
#define TBQ_MOE_I8 2        /* prefill: grouped int8 MFMA, activations quantised to
                               Q8_K blocks (d = max|x|/127 per 256), the Q4_K
                               nibbles with their 6-bit scales folded in; fp32
                               accumulate; within 1e-2 rel-L2 */

/* 1 if tbq_moe_forward takes layer L in `mode`.  TBQ_MOE_FP32 takes every
 * valid layer; the two prefill modes take layers whose gate, up and down
 * are all Q4_K in the reference's layout (TBQ_MOE_BF16 also all three in
 * ggml's, TBQ_GGML | 12), with H and F in {256, 512, 768, 1024, 1536, 2048,
 * 3072, 4096}.  0 with tbq_last_error() for an invalid layer. */
int tbq_moe_mode_supported(const tbq_moe_layer *L, int mode);

/* Workspace bytes tbq_moe_forward needs for T tokens in `mode` (T <= 65536). */
size_t tbq_moe_workspace_size(const tbq_moe_layer *L, int T, int mode);
/* out[T][H] = resid + sum_slots w_slot * expert_slot(xn) for every token
 * (layer4/tb_infer.c:753-833,876).  sel_idx/sel_w ([T][8]) may be NULL.
 * workspace: device buffer of tbq_moe_workspace_size() bytes whose first
 * 256 KiB (router arrival counters, at the same offset whatever T and mode
 * are) are zero before its first use; every call leaves them at zero.  Or
 * NULL: one library-owned buffer, shared by every NULL-workspace call in the
 * process and grown (freed and reallocated) on demand -- such calls must all
 * be ordered on one stream, as a grow can free memory that a call still
 * queued on another stream uses.  Calls that share a workspace must not
 * overlap. */
int tbq_moe_forward(const tbq_moe_layer *L, int T, const float *xn, const float *resid, float *out,
                    int *sel_idx, float *sel_w, void *workspace, size_t workspace_bytes, int mode,
                    void *stream);

/* tbq_moe_forward with no workspace argument and no allocation of any kind
 * (no hipMalloc/hipFree, no allocating library call): the workspace is a
 * static device array of TBQ_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends.  No counterpart in the reference; for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc).  Returns 0 with a message when T and mode need a larger
 * workspace than the array (tbq_moe_workspace_size > the limit: at the
 * Qwen3-30B-A3B shape, T <= 182 in TBQ_MOE_FP32).  Every call on a GPU
 * shares that GPU's array, so calls that overlap on one GPU (other streams
 * or threads) race; calls ordered on one stream do not. */
#define TBQ_NOALLOC_SCRATCH_BYTES (16u << 20)
int tbq_moe_forward_noalloc(const tbq_moe_layer *L, int T, const float *xn, const float *resid, float *out,
                            int *sel_idx, float *sel_w, int mode, void *stream);

/* Host-memory MoE block: the substitution for the MoE branch of
 * tb_layer_forward (layer4/tb_infer.c:753-833,876).  Weights in L are device
 * pointers (e.g. from tb_cuda_upload_tensor); xn, resid, out, sel_idx and
 * sel_w are host arrays.  Synchronous.  A prefill mode that does not take
 * the layer (tbq_moe_mode_supported) runs it in TBQ_MOE_FP32.  Implemented
 * in C11 over this API. */
int tbq_moe_block_host(const tbq_moe_layer *L, int T, const float *xn_host, const float *resid_host,
                       float *out_host, int *sel_idx_host, float *sel_w_host, int mode);

/* ---- dense decode (Qwen3-style transformer, one token) ------------------ */
/* The step of tb_infer_decode (layer4/tb_infer.c:889-1050: embedding row,
 * layers, output_norm, lm_head falling back to token_embd) for a dense
 * model.  The reference's layer is the static tb_layer_forward
 * (layer4/tb_infer.c:553-883), whose attention path differs from the
 * model's (head_dim, RoPE pairing, QK-norm order).  This is the model's
 * forward on libtbq's matvecs, for decode benchmarks and serving; all
 * pointers in the structs are device pointers.
 * Weights use the reference's row-major block layout; the fused tensors are
 * the separate GGUF tensors' rows concatenated in the order given. */
typedef struct {
    const float *attn_norm;   /* [hidden] */
    const float *q_norm;      /* [head_dim] */
    const float *k_norm;      /* [head_dim] */
    const float *ffn_norm;    /* [hidden] */
    const void *wqkv;         /* [(n_heads + 2 n_kv_heads) head_dim][hidden]: q | k | v rows,
                                 or NULL: wq, wk, wv below */
    const void *wo;           /* [hidden][n_heads head_dim] */
    const void *wgu;          /* [2 ffn][hidden]: gate | up rows, or NULL: wgate, wup below */
    const void *wdown;        /* [hidden][ffn] */
    /* separate matrices of a layer whose q, k, v (gate, up) differ in qtype */
    const void *wq, *wk, *wv; /* [n_heads head_dim], [n_kv_heads head_dim] x2 rows of [hidden] */
    const void *wgate, *wup;  /* [ffn][hidden] each */
    /* qtype of each matrix; 0 = the model's qtype_layers */
    int qt_qkv, qt_o, qt_gu, qt_down, qt_q, qt_k, qt_v, qt_gate, qt_up;
} tbq_dense_layer;

typedef struct {
    int n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_ctx;
    float norm_eps, rope_theta;
    int qtype_layers;         /* qtype of the layer matrices whose qt_* field is 0 (any tbq_matvec qtype) */
    int qtype_embd;           /* qtype of tok_embd and lm_head */
    const void *tok_embd;     /* [vocab][hidden] (may alias lm_head: tied embeddings) */
    const void *lm_head;      /* [vocab][hidden] */
    const float *output_norm; /* [hidden] */
    const tbq_dense_layer *layers;   /* host array of n_layers */
    float *k_cache;           /* [n_layers][n_kv_heads][max_ctx][head_dim] fp32 */
    float *v_cache;           /* same */
} tbq_dense_model;

/* Workspace bytes tbq_dense_decode needs (no zero-fill required). */
size_t tbq_dense_workspace_size(const tbq_dense_model *m);
/* logits[vocab] for `token` at position `pos` (0 <= pos < max_ctx); appends
 * the token's K and V at `pos` of every layer's cache and attends over
 * positions 0..pos.  head_dim 64 or 128; n_heads / n_kv_heads in {1, 2, 4,
 * 8}; hidden, ffn and n_heads*head_dim multiples of 256 and at most 32768
 * (the matvec row limit); max_ctx <= 131072.
 * Calls that share a workspace must not overlap. */
int tbq_dense_decode(const tbq_dense_model *m, int token, int pos, float *logits, void *workspace,
                     size_t workspace_bytes, void *stream);

/* Prefill: the T prompt tokens tokens_host[0..T) at positions pos0 ..
 * pos0 + T - 1 in one batched pass per layer, replacing the reference's
 * token-by-token prefill (layer4/tb_infer.c:1068-1075, one tb_infer_decode
 * step per prompt token).  Writes the K/V rows of every position and the
 * logits of the last token.  Models with hidden <= 8192, n_heads *
 * head_dim <= 8192 and ffn <= 16384 take the batched path for T >= 2, whatever their formats or layouts: the
 * weight products on tbq_gemm's kernel (Q4_K dequantised inside it, other
 * formats to fp16 first), attention on fp16 MFMA,
 * fp32 accumulation (logits within 1e-2 relative L2 of the sequential
 * decode); otherwise, and for T = 1, the decode step runs once per token
 * (identical to T tbq_dense_decode calls).  tokens_host is read by an
 * asynchronous copy on `stream`: keep it valid until the stream has run
 * the call.  1 <= T <= 65536, pos0 + T <= max_ctx. */
size_t tbq_dense_prefill_workspace_size(const tbq_dense_model *m, int T);
int tbq_dense_prefill(const tbq_dense_model *m, const int *tokens_host, int T, int pos0, float *logits,
                      void *workspace, size_t ws_bytes, void *stream);
/* 1 if tbq_dense_prefill takes the batched path for this model. */
int tbq_dense_prefill_batched(const tbq_dense_model *m);

/* ---- activations to Q8_K ----------------------------------------------- */
/* blocks[n / 256] = x quantised to Q8_K blocks of 292 bytes in the
 * reference's layout (layer4/tb_gguf.c:281-288: f32 d, int8 qs[256], int16
 * bsums[16]); the reference defines the layout and its decoder but no
 * quantiser.  Per block d = max|x| / 127, q = rint(x * (1 / d)) clamped to
 * +-127 (0 for an all-zero block), bsums = sums of q over 16 elements: the
 * activation form of the TBQ_MOE_I8 prefill.  n a multiple of 256; x 16-byte
 * and blocks 4-byte aligned. */
int tbq_quantize_q8k(const float *x, long long n, void *blocks, void *stream);

/* ---- prefill GEMM --------------------------------------------------------- */
/* C[T][N] (row stride ldc >= N floats, ldc a multiple of 4) = X[T][K] .
 * W[N][K]^T with the batched prefill's GEMM (hand-written fp16 MFMA, fp32
 * accumulate): X fp16 rows (IEEE halves); W rows of IEEE fp16 halves (wqt =
 * 1, TBQ's F16 id, taken as IEEE halves here) or Q4_K in the reference's
 * layout (wqt = 12), dequantised inside the GEMM to fp16: per sub-block, with
 * S = d*scale and M = dmin*min (fp32), each nibble q becomes the fp16 number
 * 1 + q/16 and one packed fp16 fma with the fp16 roundings of 16*S and of
 * C = -16*S - M gives 16*S*(1 + q/16) + C = S*q - M before the result's own
 * rounding.  A weight can therefore differ from fl16(S*q - M) by up to about
 * ulp(16*S)/2 + ulp(16*S + M)/2 (at d, dmin ~ 1e-2 that is ~4e-4 relative to
 * the sub-block's largest weight); the products stay within 1e-3 relative L2
 * of the fp32 dequantised weights (tests/test_gpu_gemm.py).  Weights must
 * keep 16*d*63 + dmin*63 below 65504 (the fp16 range).  N a multiple of 4,
 * K of 256, T >= 1, X below 2 GiB.  workspace: tbq_gemm_workspace_size()
 * bytes (split-K partial sums; may be 0).  No counterpart in the reference
 * (it prefills token by token, layer4/tb_infer.c:1068-1075). */
size_t tbq_gemm_workspace_size(int T, int N, int K);
int tbq_gemm(int wqt, const void *W, const void *X16, int T, int N, int K, float *C, int ldc, void *workspace,
             size_t workspace_bytes, void *stream);

/* ---- test hooks -------------------------------------------------------- */
/* out[i] = expf(in[i]) evaluated by the device code the router uses. */
int tbq_expf_device(const float *in, float *out, size_t n, void *stream);
/* The same function compiled for the host. */
float tbq_expf_host(float x);

#ifdef __cplusplus
}
#endif
#endif
