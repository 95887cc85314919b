/*
 * spt_moe.h -- C ABI of libspt_moe.so, the MI355X (gfx950) quantized-MoE
 * hot path of Stream-PT.
 *
 * The entry points are what the reference's forward package would bind over
 * cgo in place of its Go operators.  Quantized weights live in HBM with the
 * ggufindex tensor layout unchanged (one spt_tensor per ggufindex.Tensor,
 * data = device address of the bytes [Range.Start, Range.End)).  Activations
 * are quantized to GGML Q8_0 on the device and every dot product uses exact
 * int32 per-block sums with fp32 cross-block accumulation.
 *
 * Conventions
 *   - Every function returns SPT_OK or an SPT_ERR_* code; spt_last_error()
 *     returns the calling thread's message for the last failure.
 *   - Arguments are validated before any device work, with the reference's
 *     rules (shape, type, byte range, overflow, overlap); nothing is launched
 *     on a validation error.
 *   - Pointers named *_dev are device pointers; *_host are host pointers.
 *     Work is enqueued on the context's stream; *_host entry points
 *     synchronise before returning, the others do not.
 *   - A context is not safe for concurrent calls (forward/prefill.go:15);
 *     contexts on different threads are independent.
 *   - Kernels are not interruptible.  A cancellation flag registered with
 *     spt_ctx_set_cancel_flag() is checked before each launch of a
 *     multi-launch entry point (the reference's ctx.Err() checks,
 *     forward/moe_batch.go:84,146,167); outputs may then be partial, as in the
 *     reference (forward/q40.go:34,45).
 */
#ifndef SPT_MOE_H
#define SPT_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SPT_OK = 0,
    SPT_ERR_INVALID = 1,  /* validation failed; nothing was launched       */
    SPT_ERR_DEVICE = 2,   /* HIP runtime error, or a context without device */
    SPT_ERR_NOMEM = 3,    /* device allocation failed                       */
    SPT_ERR_CANCELED = 4, /* cancellation flag was set                      */
    SPT_ERR_IO = 5        /* a model file could not be opened or read       */
};

/* GGML type ids used on this path (ggufindex/index.go:540-551). */
enum {
    SPT_TYPE_F32 = 0,
    SPT_TYPE_F16 = 1,
    SPT_TYPE_Q4_0 = 2,
    SPT_TYPE_Q8_0 = 8,
    SPT_TYPE_BF16 = 30,
    SPT_TYPE_MXFP4 = 39
};

/* ggufindex.Tensor (ggufindex/index.go:15-26) with the file byte range
 * replaced by its HBM-resident copy.  shape[0] is the contiguous (input)
 * dimension, as in GGUF.  An absent optional tensor (bias) has name NULL or
 * "" and nbytes 0, like the reference's unnamed ggufindex.Tensor{}. */
typedef struct spt_tensor {
    const char *name;
    uint32_t type;
    uint32_t n_dims;
    uint64_t shape[4];
    uint64_t nbytes;
    const void *data;
} spt_tensor;

/* The MoE fields of forward.Config (forward/config.go:14-35). */
typedef struct spt_moe_config {
    int32_t hidden_dim;
    int32_t expert_hidden_dim;
    int32_t num_experts;
    int32_t num_experts_used;
} spt_moe_config;

/* The MoE fields of forward.LayerWeights (forward/layer.go:17-37). */
typedef struct spt_moe_layer {
    spt_tensor ffn_gate_inp;      /* F32 router [hidden, experts]          */
    spt_tensor ffn_gate_inp_bias; /* optional [experts]                    */
    spt_tensor ffn_gate_exps;     /* MXFP4 [hidden, expert_dim, experts]   */
    spt_tensor ffn_gate_exps_bias;/* optional [expert_dim, experts]        */
    spt_tensor ffn_up_exps;
    spt_tensor ffn_up_exps_bias;
    spt_tensor ffn_down_exps;     /* MXFP4 [expert_dim, hidden, experts]   */
    spt_tensor ffn_down_exps_bias;/* optional [hidden, experts]            */
} spt_moe_layer;

/* Optional device buffers a forward call fills with its intermediate stages
 * (parity taps), and optional injected router logits.  Any pointer may be
 * NULL.  B = batch, k = experts used, E = experts, H = hidden,
 * D = expert hidden dim. */
typedef struct spt_moe_taps {
    const float *logits_in; /* [B][E]: if set, skip the router and select
                               from these logits                            */
    float *logits;          /* [B][E]                                        */
    int32_t *ids;           /* [B][k]  expert of each selection              */
    float *weights;         /* [B][k]  softmax weight of each selection      */
    int32_t *counts;        /* [E]     selections per expert                 */
    int32_t *offsets;       /* [E+1]   exclusive scan of counts              */
    int32_t *list;          /* [B*k]   idx = token*k+rank, grouped by expert
                                       ascending, descending idx inside     */
    int32_t *active;        /* [E]     experts with a non-empty list         */
    int32_t *n_active;      /* [1]                                           */
    void *xq;               /* [B][H/32] Q8_0 blocks (34 B) of x             */
    float *gate;            /* [B*k][D] gate projection + bias               */
    float *up;              /* [B*k][D] up projection + bias                 */
    float *act;             /* [B*k][D] clamped SwiGLU                       */
    void *actq;             /* [B*k][D/32] Q8_0 blocks of act                */
    float *results;         /* [B*k][H] down projection + bias               */
} spt_moe_taps;

/* ---- context ----------------------------------------------------------- */

/* Thread-local message of the last failed call on this thread. */
const char *spt_last_error(void);

/* Create a context on HIP device `device`, enqueueing on `hip_stream`
 * (a hipStream_t; NULL is the device's default stream).  device = -1
 * creates a validation-only context: every entry point validates its
 * arguments and then fails with SPT_ERR_DEVICE. */
int spt_ctx_create(int device, void *hip_stream, struct spt_ctx **out);
int spt_ctx_destroy(struct spt_ctx *ctx);
int spt_ctx_synchronize(struct spt_ctx *ctx);
/* Register a host flag polled before each launch; NULL clears it. */
int spt_ctx_set_cancel_flag(struct spt_ctx *ctx, const volatile int32_t *flag);

/* Expert groups of at least min_group selections run through the grouped
 * GEMM (bf16 MFMA, up to 64 selections per pass over the expert's weights);
 * smaller groups through the grouped GEMV (4 per pass).  0 restores the
 * default policy: groups of 9 or more when the batch holds at least 384
 * selections and those groups' GEMM work fills half the device.  Results are the
 * same either way within the fp32 tolerance (the per-block sums are exact on
 * both).  No reference counterpart: the reference picks its CPU loop by tile
 * size (forward/mxfp4_batch.go:55-95). */
int spt_ctx_set_gemm_min_group(struct spt_ctx *ctx, int32_t min_group);

/* Batches of up to max_selections selections (batch * experts used; experts
 * used <= 4, and no group on the grouped GEMM) take the decode path: the
 * top-k inside the gate/up launch (a workgroup per selection) and the
 * weighted combine inside the down launch, two launches after the router.
 * 0 restores the default (8 selections: the measured crossover with the
 * grouped GEMV is between 2 and 3 tokens at top-4); a negative value turns the path
 * off (every batch through select, the grouped GEMV and combine).  Results
 * are the same within the fp32 tolerance either way; ids, weights, lists
 * and the Q8_0 stages are identical.  No reference counterpart (a launch
 * policy). */
int spt_ctx_set_decode_max_selections(struct spt_ctx *ctx, int32_t max_selections);

/* Per-kernel timing with HIP events recorded on the context's stream around
 * each launch (measurement instrumentation, off by default).  Kernel kinds: */
enum {
    SPT_KERNEL_QUANTIZE = 0, /* activation -> Q8_0                           */
    SPT_KERNEL_ROUTE = 1,    /* router logits (+ Q8_0 of the input)          */
    SPT_KERNEL_GATE_UP = 2,  /* grouped gate/up GEMV + bias + SwiGLU        */
    SPT_KERNEL_DOWN = 3,     /* grouped down GEMV + bias                      */
    SPT_KERNEL_COMBINE = 4,  /* weighted combine                              */
    SPT_KERNEL_Q40 = 5,      /* Q4_0 GEMV / small GEMM                        */
    SPT_KERNEL_SELECT = 6,   /* top-k + softmax + per-expert packing          */
    SPT_KERNEL_GATE_UP_GEMM = 7, /* grouped gate/up GEMM (large groups)       */
    SPT_KERNEL_DOWN_GEMM = 8,    /* grouped down GEMM (large groups)          */
    SPT_KERNEL_Q80 = 9,      /* Q8_0 LM head (GEMV or argmax)                 */
    SPT_KERNEL_RMSNORM = 10, /* RMSNorm (+ Q8_0 of its output)                */
    SPT_KERNEL_KINDS = 11
};
int spt_ctx_enable_timing(struct spt_ctx *ctx, int enable);
/* Synchronise, then write the summed milliseconds and launch counts of each
 * kind since the last read (arrays of SPT_KERNEL_KINDS) and reset them. */
int spt_ctx_read_timing(struct spt_ctx *ctx, double *total_ms, int64_t *launches);

/* Bytes the context holds in its grow-only device scratch arena and in its
 * pinned host staging (both grow on demand and are kept until
 * spt_ctx_destroy).  No reference counterpart: memory accounting for a
 * serving loop, and how a caller checks that a call allocated nothing. */
int spt_ctx_memory(struct spt_ctx *ctx, uint64_t *arena_bytes, uint64_t *staging_bytes);

/* ---- device memory and weight residency -------------------------------- */

int spt_alloc(struct spt_ctx *ctx, uint64_t nbytes, void **out_dev);
int spt_free(struct spt_ctx *ctx, void *dev);
int spt_copy_h2d(struct spt_ctx *ctx, void *dst_dev, const void *src_host, uint64_t nbytes);
int spt_copy_d2h(struct spt_ctx *ctx, void *dst_host, const void *src_dev, uint64_t nbytes);

/* Copy a tensor's bytes to HBM unchanged and set t->data; replaces the
 * ggufmap mmap windows (ggufmap/mmap_linux.go:210-291,391-555).  Free with
 * spt_free(ctx, (void *)t->data). */
int spt_tensor_upload(struct spt_ctx *ctx, spt_tensor *t, const void *src_host);

/* Residency from the model files: the bytes [start, end) of the file at
 * `path` -- a ggufindex.Tensor's Range (ggufindex/index.go:15-26), as
 * ggufindex.Open recorded it for the tensor -- copied to a new device
 * allocation unchanged, read in 8 MiB chunks through the context's pinned
 * staging (no mmap window is held).  Replaces the per-call streaming of
 * ggufmap's WithTensorChunks / WithExpertRanges
 * (ggufmap/mmap_linux.go:239-291,391-555) with residency.  The caller fills
 * t->name, t->type, t->n_dims (1..4) and t->shape from the ggufindex.Tensor;
 * for the path's types (F32, F16, BF16, Q4_0, Q8_0, MXFP4) the range must
 * hold exactly the bytes that type and shape take.  Sets t->nbytes =
 * end - start and t->data.  SPT_ERR_IO when the file cannot be opened or
 * ends before `end`; nothing stays allocated on failure.  Free with
 * spt_free(ctx, (void *)t->data). */
int spt_upload_range(struct spt_ctx *ctx, const char *path, uint64_t start, uint64_t end, spt_tensor *t);

/* ---- operators ----------------------------------------------------------- */

/* x[n] f32 -> n/32 GGML Q8_0 blocks (fp16 d, 32 int8), n % 32 == 0.
 * No reference counterpart: the activation quantizer of this path. */
int spt_quantize_q8_0(struct spt_ctx *ctx, const float *x_dev, int64_t n, void *out_dev);

/* forward.MulQ40Into (forward/q40.go:33-38): y = W x for a Q4_0 [in, out]
 * matrix.  x_len/y_len are element counts (len(x), len(y)).  in <= 131072
 * (the device GEMV stages a token's Q8_0 input in LDS); the matrix is below
 * 4 GiB.  These limits hold for every Q4_0 entry point. */
int spt_mul_q40_into(struct spt_ctx *ctx, const spt_tensor *w, const float *x_dev,
                     int64_t x_len, float *y_dev, int64_t y_len);

/* forward.MulQ40BatchInto (forward/q40.go:40-103): batch consecutive
 * vectors, y[b*out + row]. */
int spt_mul_q40_batch_into(struct spt_ctx *ctx, const spt_tensor *w, const float *x_dev,
                           int64_t x_len, float *y_dev, int64_t y_len, int64_t batch);

/* The projection step of forward.ForwardLayer / forwardLayerBatch
 * (forward/layer.go:117-165, layer_batch.go:62-100) on the device:
 * MulQ40BatchInto, then addBias / biasBatch of the optional [out] bias
 * (F32, F16 or BF16; absent = NULL or unnamed and empty; layer.go:225-277,
 * layer_batch.go:124-137) -- y = W x + bias with one f32 add -- and, with
 * resid_dev set, the residual addVector (layer.go:305-330): resid += y,
 * resid being the [batch][out] hidden state.  resid must not overlap x or y. */
int spt_mul_q40_batch_bias_into(struct spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias,
                                const float *x_dev, int64_t x_len, float *y_dev, int64_t y_len,
                                int64_t batch, float *resid_dev);

/* MulQ40BatchInto + biasBatch (+ residual addVector) of
 * spt_mul_q40_batch_bias_into with the input given as its GGML Q8_0 blocks:
 * xq_dev holds batch x in/32 blocks of 34 bytes (fp16 d, 32 int8 codes;
 * 2-byte aligned), as spt_rmsnorm[_batch]_into and spt_quantize_q8_0 write
 * them, so an input already quantized on the device (the normed hidden
 * state, the attention context) is not quantized again.  y is the same as
 * spt_mul_q40_batch_bias_into's on the fp32 input those blocks come from.
 * No reference counterpart (the reference multiplies fp32 activations;
 * forward/q40.go:46, layer.go:152-165). */
int spt_mul_q40_batch_q8_into(struct spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias,
                              const void *xq_dev, int64_t batch, float *y_dev, int64_t y_len,
                              float *resid_dev);

/* The Q, K, V projection step of forwardLayerBatch / ForwardLayer
 * (forward/layer_batch.go:62-74, layer.go:117-136): three MulQ40BatchInto
 * + biasBatch over the same normed input, w[i] with optional bias[i] into
 * y_dev[i] (y_len[i] elements), in one pass: the input is quantized once
 * (x_dev, fp32) or given as GGML Q8_0 blocks (xq_dev; exactly one of the
 * two), and the three matrices' rows share one GEMV launch below the GEMM
 * batch sizes.  x_len = batch * in.  Each y equals what
 * spt_mul_q40_batch_bias_into gives for that projection.  bias may be NULL
 * (no biases); outputs must not overlap each other or the input. */
int spt_mul_q40_qkv_batch_into(struct spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias,
                               const float *x_dev, const void *xq_dev, int64_t x_len, int64_t batch,
                               float *const *y_dev, const int64_t *y_len);

/* Host-slice form of MulQ40BatchInto for a cgo caller holding Go slices.
 * The slices are staged through the context's pinned host buffer and its
 * device arena, which grow on demand and are reused: once they have grown,
 * a call allocates nothing. */
int spt_mul_q40_batch_into_host(struct spt_ctx *ctx, const spt_tensor *w, const float *x_host,
                                int64_t x_len, float *y_host, int64_t y_len, int64_t batch);

/* forward.MulQ80Into (forward/q80.go:107-148): y = W x for a Q8_0 [in, out]
 * matrix (the LM head) with fp32 activations, as the reference computes it
 * (no Q8_0 of x): every row in quantQ80AVX2's order (forward/
 * quant_amd64.go:92-116), so y matches the reference's bits.  in <= 4096;
 * x and y must not overlap (the reference does not check; on the device an
 * overlap is a race). */
int spt_mul_q80_into(struct spt_ctx *ctx, const spt_tensor *w, const float *x_dev, int64_t x_len,
                     float *y_dev, int64_t y_len);

/* forward.MulQ80Argmax (forward/q80.go:20-105): the largest logit of W x and
 * the lowest row holding it, without storing the logits.  NaN logits never
 * win, -0 equals +0, and when no logit exceeds -Inf the result is row 0 with
 * -Inf, as in the reference.  Synchronises; the outputs are host values. */
int spt_mul_q80_argmax(struct spt_ctx *ctx, const spt_tensor *w, const float *x_dev, int64_t x_len,
                       int64_t *best_token, float *best_logit);

/* Host-slice forms of MulQ80Into / MulQ80Argmax for a cgo caller holding Go
 * slices (forward/engine.go:223,228 pass the final hidden state), staged
 * like spt_mul_q40_batch_into_host (no allocation once grown). */
int spt_mul_q80_into_host(struct spt_ctx *ctx, const spt_tensor *w, const float *x_host, int64_t x_len,
                          float *y_host, int64_t y_len);
int spt_mul_q80_argmax_host(struct spt_ctx *ctx, const spt_tensor *w, const float *x_host,
                            int64_t x_len, int64_t *best_token, float *best_logit);

/* forward.RMSNormInto (forward/rmsnorm.go:19-167): y = x * w * factor,
 * factor = 1 / sqrt(mean(x^2) + epsilon), with the reference's sum order (an
 * 8-float simd width), so y matches its bits.  weight: F32 (0), F16 (1) or
 * BF16 (28) [len(x)].  y may be x itself but may not partially overlap it.
 * q8_dev: NULL, or len(x)/32 GGML Q8_0 blocks (34 bytes) that receive the
 * Q8_0 of y -- the input format of the MoE and Q4_0 operators (the rule of
 * spt_quantize_q8_0); no reference counterpart (the fused quantization). */
int spt_rmsnorm_into(struct spt_ctx *ctx, const spt_tensor *weight, const float *x_dev, int64_t x_len,
                     float *y_dev, int64_t y_len, float epsilon, void *q8_dev);

/* normBatch (forward/layer_batch.go:139-195): batch rows of len(x)/batch
 * in normBatch's order (one 8-lane accumulator per row, so the bits can
 * differ from spt_rmsnorm_into's by rounding, as in the reference), with
 * the same optional Q8_0 output. */
int spt_rmsnorm_batch_into(struct spt_ctx *ctx, const spt_tensor *weight, const float *x_dev,
                           int64_t x_len, float *y_dev, int64_t y_len, int64_t batch, float epsilon,
                           void *q8_dev);

/* forward.mulMoEBatchExpert (forward/mxfp4_batch.go:29-53) for one expert of
 * an MXFP4 [in, out, experts] tensor with consecutive (not gathered) rows:
 * y[t*out + row] = dot(W_e[row], x[t*in:]) + bias_e[row], t < batch.
 * bias is an optional [out, experts] tensor. */
int spt_mul_mxfp4_expert(struct spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias,
                         int32_t expert, const float *x_dev, int64_t x_len, float *y_dev,
                         int64_t y_len, int64_t batch);

/* forward.routeMoEBatch (forward/moe_batch.go:221-303, vector_amd64.go:11-56):
 * logits[t*E + e] = router_e . x_t + bias[e], in the reference's fp32
 * accumulation order.  The router's F32 data must be 4-byte aligned (as
 * in spt_forward_moe_batch); SPT_ERR_INVALID otherwise. */
int spt_route_moe_batch(struct spt_ctx *ctx, const spt_tensor *router, const spt_tensor *bias,
                        const float *x_dev, int64_t batch, float *logits_dev);

/* forward.forwardMoE (forward/moe.go:28-64): one token. */
int spt_forward_moe(struct spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                    const float *x_dev, int64_t x_len, float *out_dev, int64_t out_len);

/* forward.forwardMoEBatch (forward/moe_batch.go:76-194): router, top-k
 * softmax, per-expert grouping, gate/up, clamped SwiGLU, down and the
 * weighted combine for batch tokens of x [batch][hidden] into out.
 * x and out must not overlap.  Any batch is accepted, as the reference
 * accepts any (moe_batch.go:29-38,84-90): a batch of more than 4096
 * selections (batch * experts used) runs as consecutive slices of
 * 4096 / experts-used whole tokens (1,024 at top-4), each token's output
 * computed from its own row of x as in one call of that slice.  Limits:
 * experts used <= 16 and experts <= 256 (SPT_ERR_INVALID beyond). */
int spt_forward_moe_batch(struct spt_ctx *ctx, const spt_moe_config *cfg,
                          const spt_moe_layer *lw, const float *x_dev, int64_t x_len,
                          float *out_dev, int64_t out_len, int64_t batch);

/* forwardMoEBatch with parity taps / injected logits (taps may be NULL).
 * With taps the batch holds at most 4096 selections (the taps describe one
 * launch sequence's lists); without, it is spt_forward_moe_batch. */
int spt_forward_moe_batch_ex(struct spt_ctx *ctx, const spt_moe_config *cfg,
                             const spt_moe_layer *lw, const float *x_dev, int64_t x_len,
                             float *out_dev, int64_t out_len, int64_t batch,
                             const spt_moe_taps *taps);

/* forwardMoEBatch with the Q8_0 of x supplied: xq_dev holds the GGML Q8_0
 * blocks of x (batch x hidden/32 blocks of 34 bytes, 2-byte aligned), as the
 * fused RMSNorm (spt_rmsnorm[_batch]_into's q8_dev) writes them beside the
 * normed x.  The router still reads the fp32 x (forward/moe_batch.go:137-139
 * routes fp32 activations); the expert projections use the given codes and
 * scales instead of quantizing x again.  With xq_dev = Q8_0(x) the results
 * are those of spt_forward_moe_batch bit for bit.  No reference counterpart
 * (the fused quantization of this path). */
int spt_forward_moe_batch_q8(struct spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                             const float *x_dev, const void *xq_dev, int64_t x_len, float *out_dev,
                             int64_t out_len, int64_t batch);

/* forwardMoEBatch (spt_forward_moe_batch, same results bit for bit) for
 * callers that cannot allocate: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  No reference counterpart.  It
 * calls no hipMalloc / hipFree and records no timing events: its scratch is
 * a fixed 32 MiB device array, one per GPU, held until the process ends
 * (about 91 KB per token at GPT-OSS-120B shape below 256 tokens, 120 KB from
 * there: batches up to about 270 tokens); larger batches fail with
 * SPT_ERR_INVALID.  Every call on a GPU uses that GPU's one array, so calls
 * that overlap on one GPU (several contexts, streams or threads) race; a
 * call may start after the previous one on the same stream without any
 * clearing, since the path needs no zeroed scratch. */
int spt_forward_moe_batch_noalloc(struct spt_ctx *ctx, const spt_moe_config *cfg,
                                  const spt_moe_layer *lw, const float *x_dev, int64_t x_len,
                                  float *out_dev, int64_t out_len, int64_t batch);

/* Host-slice form of forwardMoEBatch for a cgo caller holding Go slices,
 * staged like spt_mul_q40_batch_into_host (no allocation once grown). */
int spt_forward_moe_batch_host(struct spt_ctx *ctx, const spt_moe_config *cfg,
                               const spt_moe_layer *lw, const float *x_host, int64_t x_len,
                               float *out_host, int64_t out_len, int64_t batch);

/* Parity tap: exact int32 per-block sums of rows [0, rows) of one weight
 * matrix against one Q8_0 activation vector, computed by the same device
 * decode as the GEMV kernels.  w is MXFP4 [in, out, experts] (expert used) or
 * Q4_0 [in, out] (expert must be 0); xq_dev holds in/32 Q8_0 blocks;
 * sums_dev is [rows][in/32] int32. */
int spt_block_sums(struct spt_ctx *ctx, const spt_tensor *w, int32_t expert,
                   const void *xq_dev, int64_t rows, int32_t *sums_dev);

/* Synthetic MXFP4 bytes for blocks [first_block, first_block + nblocks) of a
 * tensor, written at dst_dev (block g at dst + (g - first_block)*17): E8M0 =
 * scale_lo + h(3g) mod (scale_hi - scale_lo + 1), nibbles = bytes of h(3g+1),
 * h(3g+2), h = SplitMix64 finaliser over key + i*0x9E3779B97F4A7C15.  Used to
 * fill HBM with benchmark weights without a host round trip. */
int spt_synth_mxfp4(struct spt_ctx *ctx, void *dst_dev, uint64_t key, uint64_t first_block,
                    uint64_t nblocks, int32_t scale_lo, int32_t scale_hi);

#ifdef __cplusplus
}
#endif
#endif
