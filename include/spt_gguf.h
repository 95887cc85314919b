/*
 * spt_gguf.h -- GGUF residency loader of libspt_moe.so: the model's tensor
 * directory read from its GGUF file(s) as ggufindex.Open reads it, and the
 * path's tensors copied from their files into HBM unchanged, replacing the
 * reference's streaming of weight windows (ggufmap WithTensorChunks,
 * mmap_linux.go:239-291, and WithExpertRanges, :391-555) by residency.
 *
 * Conventions are those of spt_moe.h (SPT_OK / SPT_ERR_* returns,
 * spt_last_error() for the message).  Index functions need no context and
 * no GPU; the upload functions use the context's device and stream.
 */
#ifndef SPT_GGUF_H
#define SPT_GGUF_H

#include "spt_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct spt_gguf spt_gguf;

/* ggufindex.Tensor (ggufindex/index.go:21-26) as read from the directory:
 * [start, end) is the absolute byte range in file `file` (an index into the
 * paths given to spt_gguf_open); `layer` is N of a "blk.N." name, -1 for
 * the tensors outside the layers.  `name` stays valid until
 * spt_gguf_close(). */
typedef struct spt_gguf_tensor {
    const char *name;
    uint32_t type;
    uint32_t n_dims;
    uint64_t shape[8];
    int32_t file;
    int64_t layer;
    uint64_t start;
    uint64_t end;
} spt_gguf_tensor;

/* ggufindex.Open (ggufindex/index.go:60-234): headers, metadata value
 * ranges and tensor directories of a model in one or more split files (any
 * order), with the reference's checks and messages.  No tensor bytes are
 * read.  SPT_ERR_INVALID for a malformed or inconsistent model, SPT_ERR_IO
 * when a file cannot be opened. */
int spt_gguf_open(const char *const *paths, int32_t n_paths, spt_gguf **out);
int spt_gguf_close(spt_gguf *g);

/* Model.LayerCount, the number of tensors, Model.Alignment. */
int spt_gguf_info(const spt_gguf *g, int64_t *layer_count, int64_t *n_tensors, uint64_t *alignment);

/* Tensor i in the order of Model.Layers (layer 0's tensors sorted by name,
 * then layer 1's, ...) followed by Model.Shared (sorted by name). */
int spt_gguf_tensor_at(const spt_gguf *g, int64_t i, spt_gguf_tensor *out);

/* Model.TensorByName (ggufindex/index.go:577-591); SPT_ERR_NOT_FOUND when
 * absent. */
int spt_gguf_find(const spt_gguf *g, const char *name, spt_gguf_tensor *out);

/* Span i of layer `layer` (Layer.Spans, index.go:202-221: per file, the
 * range enclosing the layer's tensors, sorted by path); SPT_ERR_NOT_FOUND
 * past the last span. */
int spt_gguf_layer_span(const spt_gguf *g, int64_t layer, int32_t i, int32_t *file, uint64_t *start,
                        uint64_t *end);

/* Model.Metadata[key] (ggufindex/metadata.go:13-17): the GGUF value type
 * and the range of its encoded value; SPT_ERR_NOT_FOUND when absent. */
int spt_gguf_metadata(const spt_gguf *g, const char *key, uint32_t *type, int32_t *file, uint64_t *start,
                      uint64_t *end);

/* The bytes of tensor `name` copied from its file to a new device
 * allocation unchanged (read in chunks through the context's pinned
 * staging), and its descriptor: name (valid until spt_gguf_close), type,
 * shape, nbytes = end - start, data.  Tensors of more than four dimensions
 * are refused (spt_tensor holds four).  Free with
 * spt_free(ctx, (void *)out->data). */
int spt_gguf_upload(struct spt_ctx *ctx, const spt_gguf *g, const char *name, spt_tensor *out);

/* The MoE tensors of layer `layer` picked by name suffix as NewLayerWeights
 * does (forward/layer.go:40-85: ffn_gate_inp.weight / .bias,
 * ffn_{gate,up,down}_exps.weight / .bias), each present one uploaded with
 * spt_gguf_upload and the absent ones left unnamed (nbytes 0).  On failure
 * nothing stays allocated.  Free each field's data with spt_free. */
int spt_gguf_upload_moe_layer(struct spt_ctx *ctx, const spt_gguf *g, int64_t layer, spt_moe_layer *out);

#ifdef __cplusplus
}
#endif

#endif /* SPT_GGUF_H */
