/*
 * tbq_gguf.h -- GGUF file to HBM: the loader side of libtbq.
 *
 * Replaces the reference's tb_gguf_load (layer4/tb_gguf.c:563-828: header,
 * metadata and tensor table, data section mapped from the file) and
 * tb_gguf_cuda_upload_all (layer4/tb_gguf.c:469-520), which uploads only the
 * qtypes its CUDA kernels handle; here every tensor whose qtype libtbq knows
 * (F32, F16, BF16, Q4_0, Q8_0, Q2_K..Q8_K, so routers and norms too) goes to
 * HBM, and a dense model or a MoE layer can be assembled from the file for
 * tbq_dense_decode / tbq_moe_forward with every operand device-resident.
 *
 * Format: GGUF v2/v3 (little endian): magic "GGUF", version, tensor and
 * metadata counts, metadata key/value pairs, tensor infos (name, dims,
 * ggml type, offset), then the data section at the next multiple of
 * general.alignment (32 when absent).  Every read is bounds-checked against
 * the file size; a malformed file is rejected with a message in
 * tbq_last_error().
 *
 * Calls that return int: 1 = done, 0 = failure (tbq_last_error() says why).
 * A handle may be read from several threads; the calls that upload or
 * assemble (tbq_gguf_upload_all, tbq_gguf_dense_model, tbq_gguf_moe_layer)
 * must not run concurrently on one handle.
 */
#ifndef TBQ_GGUF_H
#define TBQ_GGUF_H

#include <stddef.h>

#include "tbq.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tbq_gguf tbq_gguf;

/* Parse the file and map its data section read-only.  No device work.
 * NULL on failure. */
tbq_gguf *tbq_gguf_open(const char *path);
/* Unmap the file and free every device buffer the handle owns (uploaded
 * tensors, fused matrices and KV caches of assembled models). */
void tbq_gguf_close(tbq_gguf *g);

int tbq_gguf_n_tensors(const tbq_gguf *g);
/* Index of the tensor called `name`, or -1. */
int tbq_gguf_find(const tbq_gguf *g, const char *name);
const char *tbq_gguf_tensor_name(const tbq_gguf *g, int i);
/* ggml qtype, dimension count and dims (ggml order: dims[0] is the row
 * length), and the tensor's size in bytes (0 for a qtype libtbq does not
 * know). */
int tbq_gguf_tensor_info(const tbq_gguf *g, int i, int *qtype, int *n_dims, long long dims[4], size_t *bytes);
/* The tensor's bytes in the mapped file. */
const void *tbq_gguf_tensor_host(const tbq_gguf *g, int i);

/* Metadata lookups by full key (e.g. "qwen3.block_count").  Integers of any
 * GGUF integer or bool type; floats of either float type (or an integer);
 * strings copied with a terminating NUL (truncated to n - 1 bytes). */
int tbq_gguf_get_int(const tbq_gguf *g, const char *key, long long *out);
int tbq_gguf_get_float(const tbq_gguf *g, const char *key, double *out);
int tbq_gguf_get_str(const tbq_gguf *g, const char *key, char *buf, size_t n);

/* Copy every tensor of known size to HBM (synchronously).  Returns the
 * number of tensors resident afterwards, or -1 on failure. */
int tbq_gguf_upload_all(tbq_gguf *g);
/* Device copy of tensor i (NULL before upload or for an unknown qtype). */
const void *tbq_gguf_tensor_device(const tbq_gguf *g, int i);

/* Block layout the assembled models and layers below read the file's
 * quantised tensors in: 0 (the default) = the reference's layouts, as its
 * decoders read every file (layer4/tb_gguf.c:110-288); TBQ_GGML = ggml's,
 * as llama.cpp writes them.  The qtype fields of tbq_gguf_dense_model and
 * tbq_gguf_moe_layer then carry TBQ_GGML.  Tensor bytes are uploaded
 * unchanged either way; tbq_gguf_tensor_info keeps reporting the file's
 * ids.  No counterpart in the reference, which has no layout choice. */
int tbq_gguf_set_layout(tbq_gguf *g, int layout);

/* A dense (llama / qwen3-style) model from the file: architecture from
 * general.architecture, sizes from its metadata (block_count,
 * embedding_length, attention.head_count[_kv], attention.key_length,
 * feed_forward_length, attention.layer_norm_rms_epsilon, rope.freq_base),
 * tensors blk.N.{attn_norm, attn_q, attn_k, attn_v, attn_q_norm,
 * attn_k_norm, attn_output, ffn_norm, ffn_gate, ffn_up, ffn_down},
 * token_embd, output_norm and output (tied to token_embd when absent).
 * Uploads what is not resident yet, fuses each layer's q|k|v and gate|up
 * rows into one device matrix where they share a qtype (mixed-quant files,
 * e.g. a Q6_K attn_v among Q4_K matrices, keep them separate, each with its
 * own qtype) and allocates fp32 KV caches of max_ctx positions, all owned
 * by g.  `layers` is a caller array of n_layers entries
 * (tbq_gguf_get_int(g, "<arch>.block_count", ...)). */
int tbq_gguf_dense_model(tbq_gguf *g, int max_ctx, tbq_dense_model *m, tbq_dense_layer *layers, int n_layers);

/* MoE layer `layer` of the file (tensors blk.N.ffn_gate_inp (router, F32),
 * ffn_gate_exps, ffn_up_exps, ffn_down_exps; expert count (at most 256) and
 * top-k from <arch>.expert_count / expert_used_count), uploaded if needed,
 * as the reference's packed expert layout (layer4/tb_infer.c:780-806).
 * Each expert tensor keeps its file qtype (qt_gate, qt_up, qt_down: K-quant
 * mixes often give down a wider format than gate and up).  A file without
 * the packed tensors may hold one tensor per expert,
 * blk.N.ffn_{gate,up,down}.<e>.weight (the reference's fallback,
 * layer4/tb_infer.c:783-791); those are copied into packed device matrices
 * owned by g (the experts of one kind must share a qtype). */
int tbq_gguf_moe_layer(tbq_gguf *g, int layer, tbq_moe_layer *L);

#ifdef __cplusplus
}
#endif

#endif /* TBQ_GGUF_H */
