// spt_kernels.h -- host-side launchers of the gfx950 kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "spt_device.h"

namespace spt {

constexpr int kMaxTopK = 16;
constexpr int kMaxExperts = 256;
constexpr int kMaxSelections = 4096;
// Tokens of an expert's list per pass of the grouped GEMV over its weights.
constexpr int kGemvTokens = 4;
// List entries per work item of the grouped GEMM (spt_mx_gemm.hip).
constexpr int kGemmTokens = 64;
// Largest MXFP4 input dimension of the grouped GEMV: a workgroup stages four
// 16-row tiles of whole rows in LDS (GPT-OSS uses 2880 for both projections).
constexpr int kMxMaxInput = 2880;

struct SelectOut {
    int32_t *ids;
    float *weights;
    int32_t *counts;
    int32_t *offsets;
    int32_t *list;
    int32_t *active;
    int32_t *n_active;
    // Experts with count >= gemm_min go to the grouped GEMM, the others to
    // the grouped GEMV, each with its own packed expert list:
    int32_t gemm_min;
    // ...provided their GEMM work items (token tiles x gemm_units row units)
    // number at least gemm_min_items (enough to fill the device); otherwise
    // every expert goes to the GEMV.
    int32_t gemm_units;
    int32_t gemm_min_items;
    int32_t *gv_active;    // [E] GEMV experts, ascending
    int32_t *gv_n;
    int32_t *gv_pass_off;  // [E+1] prefix over GEMV experts of ceil(count / kGemvTokens)
    int32_t *gm_active;    // [E] GEMM experts, by descending count (equal counts ascending)
    int32_t *gm_n;
    int32_t *gm_tile_off;  // [E+1] prefix over GEMM experts of ceil(count / kGemmTokens)
    int32_t *gm_claim;     // [2] work-item counters of the two GEMM launches (zeroed)
    // Optional start table of the two grouped GEMV launches (gate/up, down):
    // for workgroup b of launch l, kGvStartWords ints at
    // gv_start[(l * kGvStartMax + b) * kGvStartWords]: its item range
    // [w0, w1), the slot, expert and pass of w0 (gv_grid[l] workgroups,
    // gv_tiles[l] row units per pass).
    int32_t *gv_start;
    int32_t gv_grid[2];
    int32_t gv_tiles[2];
};
constexpr int kGvStartMax = 1024;
constexpr int kGvStartWords = 8;

// Optional Q8_0 outputs of a quantized activation (see write_q8_block);
// with src34 set, the router's launch unpacks these GGML Q8_0 blocks of the
// input instead of quantizing it.
struct QuantOut {
    int8_t *codes;
    float *scales;
    uint8_t *mxtab;
    uint8_t *blocks34;
    uint32_t *btab;
    const uint8_t *src34;
};

enum GemvMode { kGateUp = 0, kDown = 1, kRows = 2 };

// Grouped MXFP4 x Q8_0 GEMV on the block-scaled MFMA (spt_mx_mfma.hip).
//   kGateUp: per active expert, gate and up rows for the tokens of the
//            expert's list, bias, clamped SwiGLU -> out = act[idx][row]; each
//            32-row tile also writes the Q8_0 block of act it completes.
//   kDown:   per active expert, down rows for every selection in the list,
//            bias -> out = results[idx][row].
//   kRows:   one expert, consecutive tokens -> out = y[t][row] (+ bias).
struct MxMfmaArgs {
    const uint8_t *w[2];     // MXFP4 expert tensors (gate, up) or (down) or (w)
    uint64_t expert_bytes;   // bytes of one expert matrix
    int rows;                // output rows per expert (= bias dim)
    int nb;                  // input blocks of 32 per row
    const void *bias[2];     // optional [rows][experts] biases
    uint64_t bias_bytes[2];
    int bias_type[2];
    const uint8_t *mxtab;    // activation E4M3 digit table [*][nb][64]
    const float *scales;     // activation Q8_0 scales [*][nb]
    const int8_t *codes;     // activation Q8_0 codes [*][nb*32]
    const int32_t *active;   // grouped modes: packed expert lists
    const int32_t *n_active;
    const int32_t *pass_off;
    const int32_t *offsets;
    const int32_t *list;
    int topk;
    int expert;              // kRows: the expert
    int ntok;                // kRows: tokens 0..ntok-1
    float *out;
    float *tap[2];           // kGateUp: gate / up + bias
    int8_t *act_codes;       // kGateUp: Q8_0 of act, all layouts (optional)
    float *act_scales;
    uint8_t *act_mxtab;
    uint8_t *act_blocks34;
    // grouped modes, optional: this launch's rows of SelectOut::gv_start
    // (the launch's grid must be the one they were computed for)
    const int32_t *start;
};

// The decode path (spt_mx_decode.hip) for batches of a few tokens with
// topk <= kDecMaxTopK: gate/up with the top-k inside, then down with the
// combine inside.
constexpr int kDecMaxTopK = 4;
struct DecGateUpArgs {
    MxMfmaArgs g;          // the kGateUp fields; g.out the optional fp32 act tap
    const float *logits;   // [batch][experts] router logits
    int experts;
    int tab_rows;          // rows of the x tables (batch)
    int32_t *ids;          // [batch][topk] selections written by the launch
    float *weights;
};
struct DecDownArgs {
    MxMfmaArgs g;          // the kDown fields over the act tables
    int tab_rows;          // rows of the act tables (batch * topk)
    const int32_t *ids;    // [batch][topk]
    const float *weights;
    float *out;            // [batch][rows] combined output
    float *results;        // optional [batch*topk][rows] per-selection tap
};
// n_sel = batch * topk selections (a workgroup per selection and 32 rows).
hipError_t launch_dec_gate_up(hipStream_t s, const DecGateUpArgs &a, int n_sel);
hipError_t launch_dec_down(hipStream_t s, const DecDownArgs &a, int batch);

// Grouped MXFP4 x Q8_0 GEMM on the bf16 MFMA (spt_mx_gemm.hip) for the
// experts of the GEMM list (SelectOut.gm_*): the kGateUp and kDown
// semantics of MxMfmaArgs, with the activations read as bf16 code tables
// (write_q8_block's btab layout) and the gate/up epilogue also writing the
// btab table of act.
struct MxGemmArgs {
    const uint8_t *w[2];
    uint64_t expert_bytes;
    int rows;
    int nb;
    const void *bias[2];
    int bias_type[2];
    const uint32_t *btab;    // activation bf16 code tables [tab_rows][nb][16 dwords]
    int64_t tab_rows;        // rows of btab, scales and codes
    const float *scales;     // activation Q8_0 scales [*][nb]
    const int8_t *codes;     // activation Q8_0 codes [*][nb*32] (special-scale rows)
    const int32_t *gm_active;
    const int32_t *gm_n;
    const int32_t *gm_tile_off;
    int32_t *claim;          // work-item counter, zero at launch (items past the first G are claimed)
    const int32_t *offsets;
    const int32_t *list;
    int topk;
    float *out;
    float *tap[2];
    int8_t *act_codes;
    float *act_scales;
    uint8_t *act_mxtab;
    uint8_t *act_blocks34;
    uint32_t *act_btab;
};

// One more Q4_0 matrix of a GEMV launch over several projections of the
// same input (the fields of Q40Args with the same names).
struct Q40Mat {
    const uint8_t *w;
    uint64_t nbytes;
    int rows;
    float *y;
    const void *bias;
    int bias_type;
    float *resid;
};

struct Q40Args {
    const uint8_t *w;
    uint64_t nbytes;
    int rows;
    int nb;
    const int8_t *codes;
    const float *scales;
    const int32_t *sumq;
    int ntok;
    float *y;
    // optional epilogue: y = dot + bias[row] (F32 0, F16 1, BF16 30), then
    // resid += y
    const void *bias;
    int bias_type;
    float *resid;
    // optional scratch of kQ40SplitK * ntok * rows floats (rows summed over
    // the matrices of the launch): narrow projections of large batches then
    // run on the GEMM with K split kQ40SplitK ways
    float *part;
    // GEMV only: the activations as GGML Q8_0 blocks ([ntok][nb] x 34 bytes,
    // 2-byte aligned) in place of codes / scales / sumq
    const uint8_t *xq34;
    // up to two more matrices with the same input; their row tiles follow
    // this matrix's in the grid (the GEMV, and the GEMM, whose partial sums
    // of matrix i then start after the previous matrices' in part)
    int nmore;
    Q40Mat more[2];
    // few-token form only (q40_dec_form): the fp32 activations, quantized to
    // Q8_0 inside the launch, in place of codes / scales / sumq and xq34
    const float *xf;
};

// The matrix of row tile `tile` (of `per_tile` rows) of a launch over
// several matrices with the same input (Q40Args::more): its fields in place
// of the first's, and the tile rebased to it; *rows_before (when given) is
// the number of rows of the matrices before it.
__device__ inline Q40Args q40_matrix(const Q40Args &args, int *tile, int per_tile, int *rows_before = nullptr) {
    Q40Args a = args;
    int before = 0;
    for (int i = 0; i < args.nmore; i++) {
        const int tiles = (a.rows + per_tile - 1) / per_tile;
        if (*tile < tiles) break;
        *tile -= tiles;
        before += a.rows;
        const Q40Mat &m = args.more[i];
        a.w = m.w;
        a.nbytes = m.nbytes;
        a.rows = m.rows;
        a.y = m.y;
        a.bias = m.bias;
        a.bias_type = m.bias_type;
        a.resid = m.resid;
    }
    if (rows_before) *rows_before = before;
    return a;
}

// The projection epilogue of forward/layer.go:120-165 and
// layer_batch.go:68-100: addBias (one f32 add of the decoded bias element),
// the store of y[o], and the residual addVector (x += y, one f32 add).
__device__ inline void q40_store(const Q40Args &a, size_t o, int row, float v) {
    if (a.bias) v = v + bias_at(a.bias, a.bias_type, (uint64_t)row);
    a.y[o] = v;
    if (a.resid) a.resid[o] = a.resid[o] + v;
}

// Q8_0 [in, out] x fp32 x (the LM head, spt_q80_head.hip): y = W x, or with
// part_v set the argmax of W x -- per-wave (logit, row) into part_v / part_i
// (q80_grid_waves entries), merged into *out_v / *out_i.
constexpr int kQ80MaxBlocks = 128;  // input <= 4096
struct Q80Args {
    const uint8_t *w;
    uint64_t nbytes;
    int rows;
    int nb;
    const float *x;
    float *y;
    float *part_v;
    int32_t *part_i;
    float *out_v;
    int32_t *out_i;
};

hipError_t launch_quantize(hipStream_t s, const float *x, int64_t nblocks, int8_t *codes,
                           float *scales, int32_t *sumq, uint8_t *mxtab, uint8_t *blocks34,
                           uint32_t *btab);
// Router logits [batch][experts]; Q8_0 of x into q when q.codes or q.blocks34 is set.
hipError_t launch_route(hipStream_t s, const float *router, const void *bias, int bias_type,
                        const float *x, int batch, int hidden, int experts, float *logits,
                        const QuantOut &q);
// The per-expert lists of SelectOut from the ids and weights already in it
// (one workgroup).
hipError_t launch_pack(hipStream_t s, int batch, int experts, int topk, const SelectOut &o);
// Top-k + softmax per token, then the per-expert lists (one workgroup).
hipError_t launch_select(hipStream_t s, const float *logits, int batch, int experts, int topk,
                         const SelectOut &o);
// Compute units of the current device (queried once per device; 256 if the
// query fails): the persistent launches size their grids by it.
int device_cus();
// slots: upper bound of the active experts (1 for kRows).
hipError_t launch_mx_mfma(hipStream_t s, GemvMode mode, const MxMfmaArgs &a, int slots);
// The grid launch_mx_mfma uses for these arguments (0: nothing to launch).
int mx_mfma_grid(GemvMode mode, const MxMfmaArgs &a, int slots);
// max_items: upper bound of the GEMM work items (0: nothing to launch).
hipError_t launch_mx_gemm(hipStream_t s, GemvMode mode, const MxGemmArgs &a, int max_items);
// Q4_0 x Q8_0 for a batch: the int8-MFMA GEMM (spt_q40_gemm.hip, tiles of
// kQ40TileRows rows x kQ40TileTokens tokens) from kQ40GemmMinTokens tokens
// on kQ40GemmMinRows output rows and more, and from kQ40SplitMinTokens
// tokens on narrower projections; else the GEMV.  The GEMM splits K
// kQ40SplitK ways (partial sums in Q40Args::part, then summed in order,
// when the caller provides the scratch) for narrow projections and for wide
// ones of fewer than kQ40SplitMaxTiles tiles (too few to fill the device).
// Unsplit, its sums are the GEMV's bit for bit; split, the partial sums of
// the K ranges are added in range order (within rounding of the GEMV).
constexpr int kQ40TileRows = 64;
constexpr int kQ40TileTokens = 64;
constexpr int kQ40GemmMinTokens = 32;
constexpr int kQ40GemmMinRows = 1024;
constexpr int kQ40SplitK = 4;
constexpr int kQ40SplitMinTokens = 32;
constexpr int kQ40SplitMaxTiles = 256;
inline bool q40_gemm_form(int64_t rows, int64_t ntok) {
    return (ntok >= kQ40GemmMinTokens && rows >= kQ40GemmMinRows) ||
           (ntok >= kQ40SplitMinTokens && rows < kQ40GemmMinRows);
}
inline bool q40_gemm_split(int64_t rows, int64_t ntok) {
    return rows < kQ40GemmMinRows ||
           ((rows + kQ40TileRows - 1) / kQ40TileRows) * ((ntok + kQ40TileTokens - 1) / kQ40TileTokens) <
               kQ40SplitMaxTiles;
}
// The GEMV stages its tokens' activations (40 bytes per block) in at most
// kQ40GemvLds bytes of LDS, at least one token per pass: inputs up to
// kQ40MaxInput elements.
constexpr int kQ40GemvLds = 160 * 1024;
constexpr int kQ40MaxInput = kQ40GemvLds / 40 * 32;
hipError_t launch_q40_gemv(hipStream_t s, const Q40Args &a);
// Few tokens (spt_q40_dec.hip): up to kQ40DecTokens tokens of inputs up to
// kQ40DecMaxNb blocks, matrices under 2 GiB, in one launch per call from
// the fp32 input (Q40Args::xf) or its GGML Q8_0 blocks (xq34); the activation
// views are not used.
constexpr int kQ40DecTokens = 4;
constexpr int kQ40DecMaxNb = 128;
constexpr uint64_t kQ40DecMaxBytes = 0x80000000ull;
inline bool q40_dec_form(int64_t batch, int64_t nb) { return batch <= kQ40DecTokens && nb <= kQ40DecMaxNb; }
hipError_t launch_q40_dec(hipStream_t s, const Q40Args &a);
// GGML Q8_0 blocks -> codes, widened scales and per-block code sums (the
// views launch_quantize writes), for nblocks blocks.
hipError_t launch_q8_unpack(hipStream_t s, const uint8_t *blocks34, int64_t nblocks, int8_t *codes,
                            float *scales, int32_t *sumq, uint8_t *mxtab);
hipError_t launch_q40_gemm(hipStream_t s, const Q40Args &a);
// 5 to 64 tokens of inputs up to 128 blocks (spt_q40_tile.hip): a
// workgroup per 16 output rows (when those workgroups all fit on the n_cu
// compute units at once) or 32, and 32 tokens (16 when the input is too long
// for 32 tokens' blocks in LDS), the K blocks split over its waves and their
// sums added in wave order; the activations as GGML Q8_0 blocks
// (Q40Args::xq34), all the matrices of the call in one launch.  Used while a
// tile needs at most two token groups (beyond, the GEMM reads each weight
// byte fewer times).
constexpr int kQ40TileMinTokens = kQ40DecTokens + 1;
constexpr int kQ40TileMaxTokens = 64;
constexpr int kQ40TileMaxNb = 128;
bool q40_tile_form(int64_t batch, int64_t nb);
hipError_t launch_q40_tile(hipStream_t s, const Q40Args &a, int n_cu);
int q80_grid_waves(int rows, int nb, int n_cu);
// RMSNorm of `batch` rows of n (spt_rmsnorm.hip): y = x * w * factor in the
// lane order of RMSNormInto, or of normBatch with batch_order; with q8 set,
// also the GGML Q8_0 blocks of y (n % 32 == 0).  y may equal x.
struct RmsArgs {
    const float *x;
    const void *w;
    int wtype;  // 0 F32, 1 F16, 2 BF16
    int n;
    int batch;
    float eps;
    float *y;
    uint8_t *q8;
};
hipError_t launch_rmsnorm(hipStream_t s, const RmsArgs &a, bool batch_order);
hipError_t launch_q80_rows(hipStream_t s, const Q80Args &a, int n_cu);
hipError_t launch_combine(hipStream_t s, const float *results, const float *weights, int batch,
                          int topk, int hidden, float *out);
hipError_t launch_block_sums_mx(hipStream_t s, const uint8_t *w, uint64_t nbytes, int rows, int nb,
                                const uint8_t *xq34, int32_t *sums);
hipError_t launch_block_sums_q40(hipStream_t s, const uint8_t *w, uint64_t nbytes, int rows,
                                 int nb, const uint8_t *xq34, int32_t *sums);
hipError_t launch_synth_mxfp4(hipStream_t s, uint8_t *dst, uint64_t key, uint64_t first_block,
                              uint64_t nblocks, int scale_lo, int scale_hi);

}  // namespace spt
