/*
 * spt_oracle.h -- CPU oracle for the quantized MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, on the CPU, the
 * algorithms of Stream-PT's forward package (pure Go, GOEXPERIMENT=simd) and
 * the Q8_0-activation variant that the HIP kernels implement (activations
 * quantized to Q8_0 before the integer block dots).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the results to compare against or as the timed CPU baseline; the
 * product library never links or calls it.
 *
 * Two families of functions:
 *   so_*_f32 : fp32-activation reference restatement.  Each one follows the
 *              AVX2/FMA kernel of the reference lane-for-lane (same FMA chains,
 *              same horizontal reduction), cited per function.
 *   so_*_q8  : Q8_0-activation path (activations quantized to GGML Q8_0,
 *              integer per-block sums, fp32 cross-block accumulation).  There
 *              is no reference function for it; the rule is defined here and
 *              the GPU must match it (codes/scales/ids/packing/int32 sums
 *              bit-exact, fp32 within the stated tolerance).
 *
 * Every function is pinned by tests/test_oracle_*.py against the reference's
 * own known-answer tests, its deterministic fixture formulas evaluated in
 * float64, closed forms, and library routines (numpy float16, math.ldexp).
 *
 * Parity unpinned (bit level only): the reference is Go with the
 * experimental simd package and no Go toolchain is present, so the exact
 * fp32 bit patterns of its AVX2 reductions (so_dot_mxfp4_f32, so_dot_q40_f32,
 * so_dot_q80_f32, so_dot_q40_batch_f32, so_dot_f32 / so_route) and of Go's
 * math.Exp inside so_select / so_swiglu cannot be observed.  These functions
 * follow the documented lane order and are pinned to the reference tests'
 * tolerances (3e-5 / 1e-4 relative) and, lane by lane, to scalar
 * restatements; their bits against Go itself stay unpinned.  The codecs, the
 * Q8_0 quantizer, the integer block sums and the grouping are pinned exactly.
 */
#ifndef SPT_ORACLE_H
#define SPT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- block codecs ----------------------------------------------------- */
float    so_fp16_to_f32(uint16_t h);
uint16_t so_f32_to_fp16(float f);
float    so_e8m0(uint8_t e);
void     so_mxfp4_decode_row(const uint8_t *row, int nblocks, float *out);
void     so_mxfp4_decode_row_scalar(const uint8_t *row, int nblocks, float *out);

/* ---- fp32-activation reference kernels ---------------------------------- */
float so_dot_mxfp4_f32(const uint8_t *row, const float *x, int nblocks);
float so_dot_mxfp4_f32_scalar(const uint8_t *row, const float *x, int nblocks);
float so_dot_q40_f32(const uint8_t *row, const float *x, int nblocks);
float so_dot_q80_f32(const uint8_t *row, const float *x, int nblocks);
void  so_dot_q40_batch_f32(const uint8_t *row, const float *x, float *y,
                           int input, int output, int row_index, int batch);
float so_dot_f32(const float *w, const float *x, int n);
float so_dot_f32_scalar(const float *w, const float *x, int n);

/* MulQ40BatchInto numerics (batch 1 -> quantQ40AVX2, batch > 1 -> tiled). */
void so_mul_q40_f32(const uint8_t *w, const float *x, float *y,
                    int input, int output, int batch, int threads);

/* MulQ80Into / MulQ80Argmax (the LM head): rows by quantQ80AVX2. */
void so_mul_q80_f32(const uint8_t *w, const float *x, float *y, int input, int output, int threads);
void so_mul_q80_argmax(const uint8_t *w, const float *x, int input, int output, int workers,
                       int window_rows, int64_t *token, float *logit);

/* RMSNormInto / normBatch (AVX2 lane order); w = decoded weights. */
void so_rmsnorm_f32(const float *x, const float *w, int n, float eps, float *y);
void so_rmsnorm_batch_f32(const float *x, const float *w, int dim, int batch, float eps, float *y);

void  so_route(const float *router, const float *bias, const float *x,
               int batch, int hidden, int experts, float *logits);
void  so_select(const float *logits, int experts, int k,
                int32_t *ids, float *weights);
float so_swiglu(float gate, float up);
void  so_combine(const float *results, const float *weights, int batch, int k, int h,
                 float *out);
void  so_group(const int32_t *ids, const float *weights, int batch, int k,
               int experts, int32_t *counts, int32_t *offsets, int32_t *list,
               int32_t *active, int32_t *n_active);

/* ---- Q8_0 activation path ------------------------------------------------ */
void    so_quantize_q8_0(const float *x, int64_t n, uint8_t *out);
int32_t so_isum_mxfp4_q8(const uint8_t *wblk, const int8_t *q);
int32_t so_isum_q40_q8(const uint8_t *wblk, const int8_t *q);
float   so_dot_mxfp4_q8(const uint8_t *row, const uint8_t *xq, int nblocks);
float   so_dot_q40_q8(const uint8_t *row, const uint8_t *xq, int nblocks);
void    so_mul_q40_q8(const uint8_t *w, const float *x, float *y,
                      int input, int output, int batch);
void    so_mul_mxfp4_q8(const uint8_t *w, const uint8_t *xq, const float *bias,
                        float *y, int input, int output);

/* ---- full MoE layer ------------------------------------------------------- */
typedef struct so_moe_weights {
    int hidden, expert_dim, experts, topk;
    const float   *router;          /* [experts][hidden] f32                */
    const void    *router_bias;     /* [experts] or NULL                    */
    int            router_bias_type;/* 0 f32, 1 f16, 30 bf16                */
    const uint8_t *gate, *up, *down;/* MXFP4 [experts][out][in/32*17]       */
    const void    *gate_bias, *up_bias, *down_bias; /* [experts][dim] or NULL */
    int            gate_bias_type, up_bias_type, down_bias_type;
} so_moe_weights;

typedef struct so_moe_debug {       /* every pointer optional               */
    float   *logits;   /* [B][E]            */
    int32_t *ids;      /* [B][k]            */
    float   *weights;  /* [B][k]            */
    int32_t *counts;   /* [E]               */
    int32_t *offsets;  /* [E+1]             */
    int32_t *list;     /* [B*k]             */
    int32_t *active;   /* [E]               */
    int32_t *n_active; /* [1]               */
    uint8_t *xq;       /* [B][H/32][34]     (q8 path only) */
    float   *gate;     /* [B*k][D]          */
    float   *up;       /* [B*k][D]          */
    float   *act;      /* [B*k][D]          */
    uint8_t *actq;     /* [B*k][D/32][34]   (q8 path only) */
    float   *results;  /* [B*k][H]          */
} so_moe_debug;

int so_forward_moe_batch_f32(const so_moe_weights *w, const float *x,
                             float *out, int batch, int threads,
                             so_moe_debug *dbg);
int so_forward_moe_batch_q8(const so_moe_weights *w, const float *x,
                            float *out, int batch, int threads,
                            so_moe_debug *dbg);

#ifdef __cplusplus
}
#endif
#endif
