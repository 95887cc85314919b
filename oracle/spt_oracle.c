/*
 * spt_oracle.c -- CPU oracle for the quantized MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see spt_oracle.h).  Build with
 * -mavx2 -mfma -ffp-contract=off so that the only fused multiply-adds are the
 * explicit ones that restate the reference's simd MulAdd calls.
 *
 * Reference files followed (paths relative to the Stream-PT repository):
 *   forward/mxfp4.go, forward/mxfp4_amd64.go, forward/mxfp4_batch.go,
 *   forward/moe.go, forward/moe_batch.go, forward/moe_schedule.go,
 *   forward/vector_amd64.go, forward/q40.go, forward/quant_amd64.go,
 *   forward/quant_portable.go, forward/q80.go, forward/workers_quant.go.
 */
#include "spt_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define MX_BLOCK 17
#define Q40_BLOCK 18
#define Q80_BLOCK 34
#define MOE_TILE 16 /* moeBatchTile, forward/mxfp4_batch.go:15 */

/* ------------------------------------------------------------------------- */
/* Tables: forward/mxfp4.go:10-28                                             */
/* ------------------------------------------------------------------------- */
static const float FP4_E2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,
                                   4.0f,  6.0f,  -0.0f, -0.5f, -1.0f, -1.5f,
                                   -2.0f, -3.0f, -4.0f, -6.0f};
static float E8M0[256];
static float SCALED_FP4[256][16];
static pthread_once_t tables_once = PTHREAD_ONCE_INIT;

static void init_tables(void) {
    for (int i = 0; i < 256; i++) {
        /* float32(math.Ldexp(1.0, i-127)): i=255 overflows to +Inf. */
        E8M0[i] = (float)ldexp(1.0, i - 127);
        for (int j = 0; j < 16; j++) SCALED_FP4[i][j] = E8M0[i] * FP4_E2M1[j];
    }
}
static inline void tables(void) { pthread_once(&tables_once, init_tables); }

float so_e8m0(uint8_t e) {
    tables();
    return E8M0[e];
}

/* ------------------------------------------------------------------------- */
/* fp16 <-> fp32                                                              */
/* ------------------------------------------------------------------------- */
static inline float f32_from_bits(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

/* forward/quant_portable.go:20-35 (quantFloat16Bits) == forward/q40.go:149. */
float so_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exponent = (h >> 10) & 31;
    uint32_t fraction = h & 1023;
    if (exponent == 31) return f32_from_bits(sign | 0x7f800000u | fraction << 13);
    if (exponent != 0) return f32_from_bits(sign | (exponent + 112) << 23 | fraction << 13);
    if (fraction == 0) return f32_from_bits(sign);
    uint32_t shift = (uint32_t)__builtin_clz(fraction) - 21;
    return f32_from_bits(sign | (113 - shift) << 23 | ((fraction << shift) & 1023) << 13);
}

/* Round-to-nearest-even fp32 -> fp16 (the F16C/_cvtss_sh default used by
 * GGML's quantize_row_q8_0 on x86).  NaN is canonicalised to 0x7e00|sign. */
uint16_t so_f32_to_fp16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00;
    if (ax >= 0x477ff000u) return sign | 0x7c00; /* >= 65520 rounds to Inf */
    if (ax < 0x38800000u) {                       /* below 2^-14: subnormal */
        double v = (double)f32_from_bits(ax) * 16777216.0; /* exact */
        double r = nearbyint(v);                          /* ties to even */
        return sign | (uint16_t)r;                        /* 1024 -> min normal */
    }
    uint32_t e16 = (ax >> 23) - 112;
    uint32_t m23 = ax & 0x7fffff;
    uint32_t m10 = m23 >> 13, rem = m23 & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (m10 & 1))) m10++;
    if (m10 == 0x400) {
        m10 = 0;
        e16++;
    }
    if (e16 >= 31) return sign | 0x7c00;
    return sign | (uint16_t)(e16 << 10 | m10);
}

/* ------------------------------------------------------------------------- */
/* MXFP4 block decode                                                         */
/* ------------------------------------------------------------------------- */

/* forward/mxfp4_amd64.go:43-56 (mxfp4BlockAVX2): vpermps over the 8 positive
 * pre-scaled levels, sign bit XORed from nibble bit 3.  w0 = elements 0..7
 * (low nibbles of bytes 0..7), w1 = 8..15, w2 = 16..23 (high nibbles of bytes
 * 0..7), w3 = 24..31. */
static inline void mxfp4_block_avx2(const uint8_t *blk, __m256 *w0, __m256 *w1,
                                    __m256 *w2, __m256 *w3) {
    __m256 levels = _mm256_loadu_ps(SCALED_FP4[blk[0]]);
    __m128i packed = _mm_loadu_si128((const __m128i *)(blk + 1));
    __m256i a = _mm256_cvtepu8_epi32(packed);
    __m256i b = _mm256_cvtepu8_epi32(_mm_srli_si128(packed, 8));
    __m256i ha = _mm256_srli_epi32(a, 4), hb = _mm256_srli_epi32(b, 4);
    __m256i sign = _mm256_set1_epi32(8);
#define SO_DEC(idx)                                                            \
    _mm256_castsi256_ps(_mm256_xor_si256(                                      \
        _mm256_castps_si256(_mm256_permutevar8x32_ps(levels, idx)),            \
        _mm256_slli_epi32(_mm256_and_si256(idx, sign), 28)))
    *w0 = SO_DEC(a);
    *w1 = SO_DEC(b);
    *w2 = SO_DEC(ha);
    *w3 = SO_DEC(hb);
#undef SO_DEC
}

/* forward/mxfp4_amd64.go:58-72 (decodeMXFP4Fast). */
void so_mxfp4_decode_row(const uint8_t *row, int nblocks, float *out) {
    tables();
    for (int b = 0; b < nblocks; b++) {
        __m256 w0, w1, w2, w3;
        mxfp4_block_avx2(row + (size_t)b * MX_BLOCK, &w0, &w1, &w2, &w3);
        _mm256_storeu_ps(out + 32 * b, w0);
        _mm256_storeu_ps(out + 32 * b + 8, w1);
        _mm256_storeu_ps(out + 32 * b + 16, w2);
        _mm256_storeu_ps(out + 32 * b + 24, w3);
    }
}

/* forward/mxfp4.go:52-59 / mxfp4_batch.go:84-88: table[e][nibble]. */
void so_mxfp4_decode_row_scalar(const uint8_t *row, int nblocks, float *out) {
    tables();
    for (int b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + (size_t)b * MX_BLOCK;
        const float *table = SCALED_FP4[blk[0]];
        for (int i = 0; i < 16; i++) {
            out[32 * b + i] = table[blk[1 + i] & 15];
            out[32 * b + i + 16] = table[blk[1 + i] >> 4];
        }
    }
}

/* forward/quant_amd64.go:112-116 (quantSumAVX2): fold halves, two HADDPS. */
static inline float quant_sum(__m256 v) {
    __m128 p = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    p = _mm_hadd_ps(p, p);
    p = _mm_hadd_ps(p, p);
    return _mm_cvtss_f32(p);
}
static inline float quant_sum_scalar(const float v[8]) {
    float p0 = v[0] + v[4], p1 = v[1] + v[5], p2 = v[2] + v[6], p3 = v[3] + v[7];
    return (p0 + p1) + (p2 + p3);
}

/* ------------------------------------------------------------------------- */
/* fp32-activation reference dots                                             */
/* ------------------------------------------------------------------------- */

/* forward/mxfp4_amd64.go:11-26 (dotMXFP4Fast).  Accumulator q (0..3) lane s
 * takes element 32b+8q+s by FMA over blocks in ascending order; the result is
 * quantSumAVX2(((a0+a1)+a2)+a3).  dotMXFP4PairAVX2 (:101-117) and
 * decodeMXFP4Fast + dotMoEBatchDecodedFast (:28-41, :58-72) run the same
 * chains, so one function covers every tile size. */
float so_dot_mxfp4_f32(const uint8_t *row, const float *x, int nblocks) {
    tables();
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int b = 0; b < nblocks; b++) {
        __m256 w0, w1, w2, w3;
        mxfp4_block_avx2(row + (size_t)b * MX_BLOCK, &w0, &w1, &w2, &w3);
        const float *in = x + 32 * b;
        a0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(in), a0);
        a1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(in + 8), a1);
        a2 = _mm256_fmadd_ps(w2, _mm256_loadu_ps(in + 16), a2);
        a3 = _mm256_fmadd_ps(w3, _mm256_loadu_ps(in + 24), a3);
    }
    return quant_sum(_mm256_add_ps(_mm256_add_ps(_mm256_add_ps(a0, a1), a2), a3));
}

/* Lane-by-lane scalar statement of so_dot_mxfp4_f32 (same bits). */
float so_dot_mxfp4_f32_scalar(const uint8_t *row, const float *x, int nblocks) {
    tables();
    float acc[4][8] = {{0}};
    float w[32];
    for (int b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + (size_t)b * MX_BLOCK;
        for (int i = 0; i < 16; i++) {
            uint8_t lo = blk[1 + i] & 15, hi = blk[1 + i] >> 4;
            uint32_t l = f32_bits(SCALED_FP4[blk[0]][lo & 7]) ^ ((uint32_t)(lo & 8) << 28);
            uint32_t h = f32_bits(SCALED_FP4[blk[0]][hi & 7]) ^ ((uint32_t)(hi & 8) << 28);
            w[i] = f32_from_bits(l);
            w[i + 16] = f32_from_bits(h);
        }
        for (int q = 0; q < 4; q++)
            for (int s = 0; s < 8; s++)
                acc[q][s] = fmaf(w[8 * q + s], x[32 * b + 8 * q + s], acc[q][s]);
    }
    float v[8];
    for (int s = 0; s < 8; s++) v[s] = ((acc[0][s] + acc[1][s]) + acc[2][s]) + acc[3][s];
    return quant_sum_scalar(v);
}

/* forward/quant_amd64.go:65-73 (quantQ40WeightsAVX2): (nibble-8)*scale. */
static inline void q40_block_avx2(const uint8_t *blk, __m256 *w0, __m256 *w1,
                                  __m256 *w2, __m256 *w3) {
    uint16_t hbits;
    memcpy(&hbits, blk, 2);
    __m256 scale = _mm256_set1_ps(so_fp16_to_f32(hbits));
    __m128i packed = _mm_loadu_si128((const __m128i *)(blk + 2));
    __m256i a = _mm256_cvtepu8_epi32(packed);
    __m256i b = _mm256_cvtepu8_epi32(_mm_srli_si128(packed, 8));
    __m256i mask = _mm256_set1_epi32(15), bias = _mm256_set1_epi32(8);
    *w0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_and_si256(a, mask), bias)), scale);
    *w1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_and_si256(b, mask), bias)), scale);
    *w2 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_srli_epi32(a, 4), bias)), scale);
    *w3 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_sub_epi32(_mm256_srli_epi32(b, 4), bias)), scale);
}

/* forward/quant_amd64.go:75-90 (quantQ40AVX2), the batch==1 path. */
float so_dot_q40_f32(const uint8_t *row, const float *x, int nblocks) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int b = 0; b < nblocks; b++) {
        __m256 w0, w1, w2, w3;
        q40_block_avx2(row + (size_t)b * Q40_BLOCK, &w0, &w1, &w2, &w3);
        const float *in = x + 32 * b;
        a0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(in), a0);
        a1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(in + 8), a1);
        a2 = _mm256_fmadd_ps(w2, _mm256_loadu_ps(in + 16), a2);
        a3 = _mm256_fmadd_ps(w3, _mm256_loadu_ps(in + 24), a3);
    }
    return quant_sum(_mm256_add_ps(_mm256_add_ps(_mm256_add_ps(a0, a1), a2), a3));
}

/* forward/quant_amd64.go:118-148 (quantDotQ40Batch): tiles of 8 items, one
 * 8-lane accumulator per item, four FMAs per block in sequence. */
void so_dot_q40_batch_f32(const uint8_t *row, const float *x, float *y, int input,
                          int output, int row_index, int batch) {
    const int tile = 8;
    int nblocks = input / 32;
    for (int first = 0; first < batch; first += tile) {
        int count = batch - first < tile ? batch - first : tile;
        __m256 acc[8];
        for (int i = 0; i < 8; i++) acc[i] = _mm256_setzero_ps();
        for (int b = 0; b < nblocks; b++) {
            __m256 w0, w1, w2, w3;
            q40_block_avx2(row + (size_t)b * Q40_BLOCK, &w0, &w1, &w2, &w3);
            for (int item = 0; item < count; item++) {
                const float *v = x + (size_t)(first + item) * input + 32 * b;
                __m256 a = acc[item];
                a = _mm256_fmadd_ps(w0, _mm256_loadu_ps(v), a);
                a = _mm256_fmadd_ps(w1, _mm256_loadu_ps(v + 8), a);
                a = _mm256_fmadd_ps(w2, _mm256_loadu_ps(v + 16), a);
                a = _mm256_fmadd_ps(w3, _mm256_loadu_ps(v + 24), a);
                acc[item] = a;
            }
        }
        for (int item = 0; item < count; item++)
            y[(size_t)(first + item) * output + row_index] = quant_sum(acc[item]);
    }
}

/* forward/quant_amd64.go:92-110 (quantQ80AVX2). */
float so_dot_q80_f32(const uint8_t *row, const float *x, int nblocks) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int b = 0; b < nblocks; b++) {
        const uint8_t *blk = row + (size_t)b * Q80_BLOCK;
        uint16_t hbits;
        memcpy(&hbits, blk, 2);
        __m256 scale = _mm256_set1_ps(so_fp16_to_f32(hbits));
        __m128i p0 = _mm_loadu_si128((const __m128i *)(blk + 2));
        __m128i p1 = _mm_loadu_si128((const __m128i *)(blk + 18));
        __m256 w0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(p0)), scale);
        __m256 w1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(p0, 8))), scale);
        __m256 w2 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(p1)), scale);
        __m256 w3 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(p1, 8))), scale);
        const float *in = x + 32 * b;
        a0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(in), a0);
        a1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(in + 8), a1);
        a2 = _mm256_fmadd_ps(w2, _mm256_loadu_ps(in + 16), a2);
        a3 = _mm256_fmadd_ps(w3, _mm256_loadu_ps(in + 24), a3);
    }
    return quant_sum(_mm256_add_ps(_mm256_add_ps(_mm256_add_ps(a0, a1), a2), a3));
}

/* forward/vector_amd64.go:28-56 (dotF32AVX2): 8 accumulators over 64-element
 * chunks, a 32-element tail into a0..a3, then
 * quantSumAVX2((((a0+a1)+a2)+a3) + (((a4+a5)+a6)+a7)).  n % 32 == 0. */
float so_dot_f32(const float *w, const float *x, int n) {
    __m256 a[8];
    for (int i = 0; i < 8; i++) a[i] = _mm256_setzero_ps();
    int offset = 0;
    for (; offset + 64 <= n; offset += 64)
        for (int j = 0; j < 8; j++)
            a[j] = _mm256_fmadd_ps(_mm256_loadu_ps(w + offset + 8 * j),
                                   _mm256_loadu_ps(x + offset + 8 * j), a[j]);
    for (; offset < n; offset += 32)
        for (int j = 0; j < 4; j++)
            a[j] = _mm256_fmadd_ps(_mm256_loadu_ps(w + offset + 8 * j),
                                   _mm256_loadu_ps(x + offset + 8 * j), a[j]);
    __m256 s0 = _mm256_add_ps(_mm256_add_ps(_mm256_add_ps(a[0], a[1]), a[2]), a[3]);
    __m256 s1 = _mm256_add_ps(_mm256_add_ps(_mm256_add_ps(a[4], a[5]), a[6]), a[7]);
    return quant_sum(_mm256_add_ps(s0, s1));
}

float so_dot_f32_scalar(const float *w, const float *x, int n) {
    float a[8][8] = {{0}};
    int offset = 0;
    for (; offset + 64 <= n; offset += 64)
        for (int j = 0; j < 8; j++)
            for (int s = 0; s < 8; s++)
                a[j][s] = fmaf(w[offset + 8 * j + s], x[offset + 8 * j + s], a[j][s]);
    for (; offset < n; offset += 32)
        for (int j = 0; j < 4; j++)
            for (int s = 0; s < 8; s++)
                a[j][s] = fmaf(w[offset + 8 * j + s], x[offset + 8 * j + s], a[j][s]);
    float v[8];
    for (int s = 0; s < 8; s++) {
        float s0 = ((a[0][s] + a[1][s]) + a[2][s]) + a[3][s];
        float s1 = ((a[4][s] + a[5][s]) + a[6][s]) + a[7][s];
        v[s] = s0 + s1;
    }
    return quant_sum_scalar(v);
}

/* forward/q40.go:141-198 (MulQ40BatchInto numerics; rows split over workers
 * as in workers_quant.go:42-55 -- partitioning does not change the bits). */
void so_mul_q40_f32(const uint8_t *w, const float *x, float *y, int input, int output,
                    int batch, int threads) {
    int nb = input / 32;
    size_t row_bytes = (size_t)nb * Q40_BLOCK;
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int row = 0; row < output; row++) {
        const uint8_t *enc = w + (size_t)row * row_bytes;
        if (batch == 1)
            y[row] = so_dot_q40_f32(enc, x, nb);
        else
            so_dot_q40_batch_f32(enc, x, y, input, output, row, batch);
    }
}

/* forward/q80.go:107-148 (MulQ80Into numerics): every row by quantQ80AVX2;
 * the pair form the reference runs (quantQ80PairAVX2, quant_amd64.go:19-47)
 * keeps each row's four chains and reduction, so the bits are the same.
 * Rows are split over threads; partitioning does not change the bits. */
void so_mul_q80_f32(const uint8_t *w, const float *x, float *y, int input, int output, int threads) {
    int nb = input / 32;
    size_t row_bytes = (size_t)nb * Q80_BLOCK;
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int row = 0; row < output; row++) y[row] = so_dot_q80_f32(w + (size_t)row * row_bytes, x, nb);
}

/* forward/q80.go:20-105 (MulQ80Argmax): rows in windows of window_rows rows
 * (WithTensorChunks), each window split over min(workers, rows) workers as
 * in workers_quant.go:42-55.  A worker scans its rows in order from (its
 * first row, -Inf) and keeps strict maxima (q80.go:64-82); after each window
 * the workers' results merge into the running best, which starts at
 * (0, -Inf), by a larger logit or an equal logit with a lower token
 * (q80.go:93-99).  Workers run one after another here; the result does not
 * depend on their timing. */
void so_mul_q80_argmax(const uint8_t *w, const float *x, int input, int output, int workers,
                       int window_rows, int64_t *token, float *logit) {
    int nb = input / 32;
    size_t row_bytes = (size_t)nb * Q80_BLOCK;
    if (window_rows < 1 || window_rows > output) window_rows = output;
    if (workers < 1) workers = 1;
    if (workers > window_rows) workers = window_rows;
    int64_t best_t = 0;
    float best_l = -INFINITY;
    for (int first = 0; first < output; first += window_rows) {
        int rows = output - first < window_rows ? output - first : window_rows;
        int active = workers < rows ? workers : rows;
        for (int wk = 0; wk < active; wk++) {
            int begin = (int)((int64_t)wk * rows / active), end = (int)((int64_t)(wk + 1) * rows / active);
            int64_t lt = first + begin;
            float ll = -INFINITY;
            for (int r = begin; r < end; r++) {
                float v = so_dot_q80_f32(w + (size_t)(first + r) * row_bytes, x, nb);
                if (v > ll) {
                    ll = v;
                    lt = first + r;
                }
            }
            if (ll > best_l || (ll == best_l && lt < best_t)) {
                best_l = ll;
                best_t = lt;
            }
        }
    }
    *token = best_t;
    *logit = best_l;
}

/* forward/rmsnorm.go:59-97,152-164 (RMSNormInto) with the simd width of the
 * AVX2 build (8 float lanes): four accumulators over 32-element chunks
 * (MulAdd = FMA), combined ((a0+a1)+a2)+a3, then 8-element chunks into the
 * combined vector (a partial last chunk zero-filled), the eight lanes summed
 * in order into a float from 0, factor = 1 / float32(sqrt(float64(sum / n +
 * eps))), y = (x * w) * factor.  w is the decoded weight vector. */
void so_rmsnorm_f32(const float *x, const float *w, int n, float eps, float *y) {
    float sq[4][8] = {{0}};
    int off = 0;
    for (; off + 32 <= n; off += 32)
        for (int a = 0; a < 4; a++)
            for (int s = 0; s < 8; s++) {
                float v = x[off + 8 * a + s];
                sq[a][s] = fmaf(v, v, sq[a][s]);
            }
    float lanes[8];
    for (int s = 0; s < 8; s++) lanes[s] = ((sq[0][s] + sq[1][s]) + sq[2][s]) + sq[3][s];
    for (; off < n; off += 8)
        for (int s = 0; s < 8; s++) {
            float v = off + s < n ? x[off + s] : 0.0f;
            lanes[s] = fmaf(v, v, lanes[s]);
        }
    float sum = 0.0f;
    for (int s = 0; s < 8; s++) sum += lanes[s];
    float factor = 1.0f / (float)sqrt((double)(sum / (float)n + eps));
    for (int i = 0; i < n; i++) y[i] = (x[i] * w[i]) * factor;
}

/* forward/layer_batch.go:139-195 (normBatch): per item one accumulator over
 * 8-element chunks (a partial last chunk zero-filled), then the same sum,
 * factor and products as so_rmsnorm_f32. */
void so_rmsnorm_batch_f32(const float *x, const float *w, int dim, int batch, float eps, float *y) {
    for (int t = 0; t < batch; t++) {
        const float *in = x + (size_t)t * dim;
        float *out = y + (size_t)t * dim;
        float lanes[8] = {0};
        for (int off = 0; off < dim; off += 8)
            for (int s = 0; s < 8; s++) {
                float v = off + s < dim ? in[off + s] : 0.0f;
                lanes[s] = fmaf(v, v, lanes[s]);
            }
        float sum = 0.0f;
        for (int s = 0; s < 8; s++) sum += lanes[s];
        float factor = 1.0f / (float)sqrt((double)(sum / (float)dim + eps));
        for (int i = 0; i < dim; i++) out[i] = (in[i] * w[i]) * factor;
    }
}

/* ------------------------------------------------------------------------- */
/* Router, selection, SwiGLU, grouping                                        */
/* ------------------------------------------------------------------------- */

/* forward/vector_amd64.go:11-25 (routeMoEBatchFast). */
void so_route(const float *router, const float *bias, const float *x, int batch, int hidden,
              int experts, float *logits) {
    for (int e = 0; e < experts; e++)
        for (int t = 0; t < batch; t++)
            logits[(size_t)t * experts + e] =
                so_dot_f32(router + (size_t)e * hidden, x + (size_t)t * hidden, hidden) +
                (bias ? bias[e] : 0.0f);
}

/* forward/moe_batch.go:305-342 (selectMoEBatch). */
void so_select(const float *logits, int experts, int k, int32_t *ids, float *weights) {
    for (int r = 0; r < k; r++) {
        int best = -1;
        float value = -INFINITY;
        for (int e = 0; e < experts; e++) {
            int already = 0;
            for (int prev = 0; prev < r; prev++)
                if (ids[prev] == e) {
                    already = 1;
                    break;
                }
            if (!already && logits[e] > value) {
                best = e;
                value = logits[e];
            }
        }
        if (best < 0) {
            best = r;
            value = 0.0f;
        }
        ids[r] = best;
        weights[r] = value;
    }
    float max_logit = -INFINITY;
    for (int r = 0; r < k; r++)
        if (weights[r] > max_logit) max_logit = weights[r];
    float sum = 0.0f;
    for (int r = 0; r < k; r++) {
        weights[r] = (float)exp((double)(weights[r] - max_logit));
        sum += weights[r];
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int r = 0; r < k; r++) weights[r] *= inv;
    }
}

/* Go's built-in min/max on floats: NaN if either operand is NaN, and
 * -0 < +0. */
static inline float go_min(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a < b) return a;
    if (b < a) return b;
    return signbit(a) ? a : b;
}
static inline float go_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a > b) return a;
    if (b > a) return b;
    return signbit(a) ? b : a;
}

/* forward/moe.go:66-70 (gptOSSSwiGLU). */
float so_swiglu(float gate, float up) {
    float g = go_min(gate, 7.0f);
    float u = go_max(-7.0f, go_min(up, 7.0f));
    float e = (float)exp((double)(-1.702f * g));
    return g / (1.0f + e) * (u + 1.0f);
}

/* forward/moe_batch.go:142-159: heads[e]/next[idx] linked lists pushed at the
 * head, so each expert's list is in descending idx = token*k + rank;
 * selections with Weight <= 0 are skipped (NaN weights are kept).  The lists
 * are flattened in ascending expert order (offsets = exclusive scan of
 * counts), each list in traversal (descending idx) order. */
void so_group(const int32_t *ids, const float *weights, int batch, int k, int experts,
              int32_t *counts, int32_t *offsets, int32_t *list, int32_t *active,
              int32_t *n_active) {
    int n = batch * k;
    int32_t *heads = malloc(sizeof(int32_t) * (size_t)experts);
    int32_t *next = malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
    for (int e = 0; e < experts; e++) heads[e] = -1;
    for (int t = 0; t < batch; t++)
        for (int r = 0; r < k; r++) {
            int idx = t * k + r;
            if (weights[idx] <= 0.0f) continue;
            next[idx] = heads[ids[idx]];
            heads[ids[idx]] = idx;
        }
    int pos = 0, na = 0;
    for (int e = 0; e < experts; e++) {
        offsets[e] = pos;
        int c = 0;
        for (int h = heads[e]; h >= 0; h = next[h]) list[pos + c++] = h;
        counts[e] = c;
        pos += c;
        if (heads[e] >= 0 && active) active[na++] = e;
    }
    offsets[experts] = pos;
    if (n_active) *n_active = na;
    free(heads);
    free(next);
}

/* ------------------------------------------------------------------------- */
/* Q8_0 activation path                                                       */
/* ------------------------------------------------------------------------- */

/* GGML's reference rule (quantize_row_q8_0_ref, llama.cpp, MIT): per block of
 * 32, amax = max|x|, d = amax/127, id = d ? 1/d : 0, q = roundf(x*id)
 * (half away from zero), scale stored as fp16(d) rounded to nearest even.
 * Build-defined edge cases: a NaN element makes d NaN; a NaN product gives
 * code 0; codes are clamped to [-127, 127]. */
void so_quantize_q8_0(const float *x, int64_t n, uint8_t *out) {
    for (int64_t blk = 0; blk < n / 32; blk++) {
        const float *v = x + blk * 32;
        uint8_t *o = out + blk * Q80_BLOCK;
        float amax = 0.0f;
        int nan = 0;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(v[i]);
            if (a != a)
                nan = 1;
            else if (a > amax)
                amax = a;
        }
        float d = nan ? NAN : amax / 127.0f;
        float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint16_t dh = so_f32_to_fp16(d);
        memcpy(o, &dh, 2);
        for (int i = 0; i < 32; i++) {
            float r = roundf(v[i] * id);
            int q = (r != r) ? 0 : (r > 127.0f ? 127 : (r < -127.0f ? -127 : (int)r));
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* 2 x E2M1: exact small integers, so per-block sums are exact in int32. */
static const int8_t LUT2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

int32_t so_isum_mxfp4_q8(const uint8_t *wblk, const int8_t *q) {
    int32_t s = 0;
    for (int i = 0; i < 16; i++) {
        s += LUT2[wblk[1 + i] & 15] * q[i];
        s += LUT2[wblk[1 + i] >> 4] * q[i + 16];
    }
    return s;
}

int32_t so_isum_q40_q8(const uint8_t *wblk, const int8_t *q) {
    int32_t s = 0;
    for (int i = 0; i < 16; i++) {
        s += ((wblk[2 + i] & 15) - 8) * q[i];
        s += ((wblk[2 + i] >> 4) - 8) * q[i + 16];
    }
    return s;
}

/* Weight block scale of the integer form: E8M0/2 (LUT2 holds 2*E2M1), with
 * the reference's e=255 -> +Inf kept. */
static inline float mx_half_scale(uint8_t e) {
    return e == 255 ? INFINITY : ldexpf(1.0f, (int)e - 128);
}

/* Canonical MXFP4 x Q8_0 row dot: acc = fma(float(isum_b), d_x*s_w, acc)
 * over blocks in ascending order. */
float so_dot_mxfp4_q8(const uint8_t *row, const uint8_t *xq, int nblocks) {
    float acc = 0.0f;
    for (int b = 0; b < nblocks; b++) {
        const uint8_t *w = row + (size_t)b * MX_BLOCK;
        const uint8_t *a = xq + (size_t)b * Q80_BLOCK;
        uint16_t dh;
        memcpy(&dh, a, 2);
        float ds = so_fp16_to_f32(dh) * mx_half_scale(w[0]);
        int32_t s = so_isum_mxfp4_q8(w, (const int8_t *)(a + 2));
        acc = fmaf((float)s, ds, acc);
    }
    return acc;
}

/* Canonical Q4_0 x Q8_0 row dot: d_w*d_x is exact in fp32 (two 11-bit
 * significands), acc = fma(float(isum_b), d_w*d_x, acc). */
float so_dot_q40_q8(const uint8_t *row, const uint8_t *xq, int nblocks) {
    float acc = 0.0f;
    for (int b = 0; b < nblocks; b++) {
        const uint8_t *w = row + (size_t)b * Q40_BLOCK;
        const uint8_t *a = xq + (size_t)b * Q80_BLOCK;
        uint16_t dw, dx;
        memcpy(&dw, w, 2);
        memcpy(&dx, a, 2);
        float ds = so_fp16_to_f32(dw) * so_fp16_to_f32(dx);
        int32_t s = so_isum_q40_q8(w, (const int8_t *)(a + 2));
        acc = fmaf((float)s, ds, acc);
    }
    return acc;
}

void so_mul_q40_q8(const uint8_t *w, const float *x, float *y, int input, int output,
                   int batch) {
    int nb = input / 32;
    uint8_t *xq = malloc((size_t)batch * nb * Q80_BLOCK);
    so_quantize_q8_0(x, (int64_t)batch * input, xq);
#pragma omp parallel for schedule(static)
    for (int row = 0; row < output; row++)
        for (int t = 0; t < batch; t++)
            y[(size_t)t * output + row] =
                so_dot_q40_q8(w + (size_t)row * nb * Q40_BLOCK, xq + (size_t)t * nb * Q80_BLOCK, nb);
    free(xq);
}

void so_mul_mxfp4_q8(const uint8_t *w, const uint8_t *xq, const float *bias, float *y,
                     int input, int output) {
    int nb = input / 32;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < output; row++)
        y[row] = so_dot_mxfp4_q8(w + (size_t)row * nb * MX_BLOCK, xq, nb) +
                 (bias ? bias[row] : 0.0f);
}

/* ------------------------------------------------------------------------- */
/* Full MoE layer                                                             */
/* ------------------------------------------------------------------------- */

/* forward/layer.go:279-303 (readFloatVector) element decode for biases. */
static inline float bias_at(const void *p, int type, size_t i) {
    if (!p) return 0.0f;
    if (type == 1) {
        uint16_t h;
        memcpy(&h, (const uint8_t *)p + 2 * i, 2);
        return so_fp16_to_f32(h);
    }
    if (type == 30) {
        uint16_t h;
        memcpy(&h, (const uint8_t *)p + 2 * i, 2);
        return f32_from_bits((uint32_t)h << 16);
    }
    float f;
    memcpy(&f, (const uint8_t *)p + 4 * i, 4);
    return f;
}

static void fill_bias(const void *p, int type, int expert, int dim, float *dst) {
    for (int i = 0; i < dim; i++) dst[i] = bias_at(p, type, (size_t)expert * dim + i);
}

/* forward/moe_batch.go:163-192: clear(out), then for each token and rank
 * with Weight > 0 (NaN kept), out = fma(results[idx], weight, out). */
void so_combine(const float *results, const float *weights, int batch, int k, int h, float *out) {
    memset(out, 0, sizeof(float) * (size_t)batch * h);
    for (int t = 0; t < batch; t++)
        for (int r = 0; r < k; r++) {
            int idx = t * k + r;
            float wt = weights[idx];
            if (wt <= 0.0f) continue;
            for (int i = 0; i < h; i++)
                out[(size_t)t * h + i] = fmaf(results[(size_t)idx * h + i], wt, out[(size_t)t * h + i]);
        }
}

/* forward/mxfp4_batch.go:31-95 (mulMoEBatchExpert / computeMoEBatchExpertRows)
 * for one tile of <= 16 gathered tokens: count 1 -> dotMXFP4, 2..4 -> pair
 * kernel, 5..16 -> decoded row.  All three give the same bits per token. */
static void mxfp4_tile_f32(const uint8_t *data, int input, int output, const float *x,
                           const int *xoff, int count, const float *bias, float *y,
                           const int *yoff, int threads) {
    int nb = input / 32;
    size_t row_bytes = (size_t)nb * MX_BLOCK;
#pragma omp parallel num_threads(threads)
    {
        float *decoded = count >= 5 ? malloc(sizeof(float) * (size_t)input) : NULL;
#pragma omp for schedule(static)
        for (int row = 0; row < output; row++) {
            const uint8_t *enc = data + (size_t)row * row_bytes;
            if (count >= 5) {
                so_mxfp4_decode_row(enc, nb, decoded);
                for (int t = 0; t < count; t++) {
                    const float *v = x + xoff[t];
                    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
                    for (int o = 0; o < input; o += 32) {
                        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(decoded + o), _mm256_loadu_ps(v + o), a0);
                        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(decoded + o + 8), _mm256_loadu_ps(v + o + 8), a1);
                        a2 = _mm256_fmadd_ps(_mm256_loadu_ps(decoded + o + 16), _mm256_loadu_ps(v + o + 16), a2);
                        a3 = _mm256_fmadd_ps(_mm256_loadu_ps(decoded + o + 24), _mm256_loadu_ps(v + o + 24), a3);
                    }
                    y[yoff[t] + row] =
                        quant_sum(_mm256_add_ps(_mm256_add_ps(_mm256_add_ps(a0, a1), a2), a3)) + bias[row];
                }
            } else {
                for (int t = 0; t < count; t++)
                    y[yoff[t] + row] = so_dot_mxfp4_f32(enc, x + xoff[t], nb) + bias[row];
            }
        }
        free(decoded);
    }
}

/* forward/moe_schedule.go:103-127 (projectSelectedMoE): walk one expert's
 * list in tiles of 16. */
static void project_f32(const uint8_t *data, const float *x, const float *bias, float *dst,
                        int head, const int32_t *next, int hidden, int expert_dim, int k,
                        int down, int threads) {
    int inputs[MOE_TILE], outputs[MOE_TILE];
    int input = down ? expert_dim : hidden, output = down ? hidden : expert_dim;
    while (head >= 0) {
        int count = 0;
        while (head >= 0 && count < MOE_TILE) {
            if (down) {
                inputs[count] = head * expert_dim;
                outputs[count] = head * hidden;
            } else {
                inputs[count] = head / k * hidden;
                outputs[count] = head * expert_dim;
            }
            head = next[head];
            count++;
        }
        mxfp4_tile_f32(data, input, output, x, inputs, count, bias, dst, outputs, threads);
    }
}

static size_t expert_bytes(int input, int output) { return (size_t)input / 32 * MX_BLOCK * output; }

/* forward/moe_batch.go:78-194 (forwardMoEBatch) + moe_schedule.go:25-101
 * (evaluateSelectedMoE), fp32 activations. */
int so_forward_moe_batch_f32(const so_moe_weights *w, const float *x, float *out, int batch,
                             int threads, so_moe_debug *dbg) {
    int h = w->hidden, d = w->expert_dim, E = w->experts, k = w->topk;
    int n = batch * k;
    if (threads < 1) threads = 1;
    float *logits = malloc(sizeof(float) * (size_t)batch * E);
    int32_t *ids = malloc(sizeof(int32_t) * n);
    float *wts = malloc(sizeof(float) * n);
    int32_t *heads = malloc(sizeof(int32_t) * E), *next = malloc(sizeof(int32_t) * n);
    float *gate = calloc((size_t)n * d, sizeof(float)), *up = calloc((size_t)n * d, sizeof(float));
    float *act = calloc((size_t)n * d, sizeof(float));
    float *results = calloc((size_t)n * h, sizeof(float));
    float *gb = malloc(sizeof(float) * d), *ub = malloc(sizeof(float) * d), *db = malloc(sizeof(float) * h);
    float *rbias = calloc((size_t)(E > 0 ? E : 1), sizeof(float));
    for (int e = 0; e < E; e++) rbias[e] = bias_at(w->router_bias, w->router_bias_type, e);
    so_route(w->router, rbias, x, batch, h, E, logits);
    for (int e = 0; e < E; e++) heads[e] = -1;
    for (int t = 0; t < batch; t++) {
        so_select(logits + (size_t)t * E, E, k, ids + t * k, wts + t * k);
        for (int r = 0; r < k; r++) {
            int idx = t * k + r;
            if (wts[idx] <= 0.0f) continue;
            next[idx] = heads[ids[idx]];
            heads[ids[idx]] = idx;
        }
    }
    for (int e = 0; e < E; e++) {
        if (heads[e] < 0) continue;
        fill_bias(w->gate_bias, w->gate_bias_type, e, d, gb);
        project_f32(w->gate + (size_t)e * expert_bytes(h, d), x, gb, gate, heads[e], next, h, d, k, 0,
                    threads);
        fill_bias(w->up_bias, w->up_bias_type, e, d, ub);
        project_f32(w->up + (size_t)e * expert_bytes(h, d), x, ub, up, heads[e], next, h, d, k, 0,
                    threads);
    }
    for (int idx = 0; idx < n; idx++) {
        if (wts[idx] <= 0.0f) continue;
        for (int i = idx * d; i < (idx + 1) * d; i++) act[i] = so_swiglu(gate[i], up[i]);
    }
    for (int e = 0; e < E; e++) {
        if (heads[e] < 0) continue;
        fill_bias(w->down_bias, w->down_bias_type, e, h, db);
        project_f32(w->down + (size_t)e * expert_bytes(d, h), act, db, results, heads[e], next, h, d,
                    k, 1, threads);
    }
    so_combine(results, wts, batch, k, h, out);
    if (dbg) {
        if (dbg->logits) memcpy(dbg->logits, logits, sizeof(float) * (size_t)batch * E);
        if (dbg->ids) memcpy(dbg->ids, ids, sizeof(int32_t) * n);
        if (dbg->weights) memcpy(dbg->weights, wts, sizeof(float) * n);
        if (dbg->counts || dbg->offsets || dbg->list) {
            int32_t *c = malloc(sizeof(int32_t) * E), *o = malloc(sizeof(int32_t) * (E + 1));
            int32_t *l = malloc(sizeof(int32_t) * (n > 0 ? n : 1)), *a = malloc(sizeof(int32_t) * E);
            int32_t na;
            so_group(ids, wts, batch, k, E, c, o, l, a, &na);
            if (dbg->counts) memcpy(dbg->counts, c, sizeof(int32_t) * E);
            if (dbg->offsets) memcpy(dbg->offsets, o, sizeof(int32_t) * (E + 1));
            if (dbg->list) memcpy(dbg->list, l, sizeof(int32_t) * o[E]);
            if (dbg->active) memcpy(dbg->active, a, sizeof(int32_t) * na);
            if (dbg->n_active) *dbg->n_active = na;
            free(c), free(o), free(l), free(a);
        }
        if (dbg->gate) memcpy(dbg->gate, gate, sizeof(float) * (size_t)n * d);
        if (dbg->up) memcpy(dbg->up, up, sizeof(float) * (size_t)n * d);
        if (dbg->act) memcpy(dbg->act, act, sizeof(float) * (size_t)n * d);
        if (dbg->results) memcpy(dbg->results, results, sizeof(float) * (size_t)n * h);
    }
    free(logits), free(ids), free(wts), free(heads), free(next), free(gate), free(up), free(act);
    free(results), free(gb), free(ub), free(db), free(rbias);
    return 0;
}

/* The same layer with Q8_0 activations: router, selection, grouping, SwiGLU
 * and combine exactly as above; each token row is quantized to Q8_0 before
 * gate/up, and each SwiGLU row is quantized to Q8_0 before down. */
int so_forward_moe_batch_q8(const so_moe_weights *w, const float *x, float *out, int batch,
                            int threads, so_moe_debug *dbg) {
    int h = w->hidden, d = w->expert_dim, E = w->experts, k = w->topk;
    int n = batch * k, nbh = h / 32, nbd = d / 32;
    if (threads < 1) threads = 1;
    float *logits = malloc(sizeof(float) * (size_t)batch * E);
    int32_t *ids = malloc(sizeof(int32_t) * n);
    float *wts = malloc(sizeof(float) * n);
    int32_t *counts = malloc(sizeof(int32_t) * E), *offsets = malloc(sizeof(int32_t) * (E + 1));
    int32_t *list = malloc(sizeof(int32_t) * (n > 0 ? n : 1)), *active = malloc(sizeof(int32_t) * E);
    int32_t n_active = 0;
    uint8_t *xq = malloc((size_t)batch * nbh * Q80_BLOCK);
    uint8_t *actq = calloc((size_t)n * nbd, Q80_BLOCK);
    float *gate = calloc((size_t)n * d, sizeof(float)), *up = calloc((size_t)n * d, sizeof(float));
    float *act = calloc((size_t)n * d, sizeof(float));
    float *results = calloc((size_t)n * h, sizeof(float));
    float *rbias = calloc((size_t)(E > 0 ? E : 1), sizeof(float));
    for (int e = 0; e < E; e++) rbias[e] = bias_at(w->router_bias, w->router_bias_type, e);
    so_route(w->router, rbias, x, batch, h, E, logits);
    for (int t = 0; t < batch; t++) so_select(logits + (size_t)t * E, E, k, ids + t * k, wts + t * k);
    so_group(ids, wts, batch, k, E, counts, offsets, list, active, &n_active);
    so_quantize_q8_0(x, (int64_t)batch * h, xq);
    for (int a = 0; a < n_active; a++) {
        int e = active[a];
        const uint8_t *G = w->gate + (size_t)e * expert_bytes(h, d);
        const uint8_t *U = w->up + (size_t)e * expert_bytes(h, d);
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int row = 0; row < d; row++) {
            float gbv = bias_at(w->gate_bias, w->gate_bias_type, (size_t)e * d + row);
            float ubv = bias_at(w->up_bias, w->up_bias_type, (size_t)e * d + row);
            for (int j = offsets[e]; j < offsets[e + 1]; j++) {
                int idx = list[j], t = idx / k;
                const uint8_t *xt = xq + (size_t)t * nbh * Q80_BLOCK;
                float g = so_dot_mxfp4_q8(G + (size_t)row * nbh * MX_BLOCK, xt, nbh) + gbv;
                float u = so_dot_mxfp4_q8(U + (size_t)row * nbh * MX_BLOCK, xt, nbh) + ubv;
                gate[(size_t)idx * d + row] = g;
                up[(size_t)idx * d + row] = u;
                act[(size_t)idx * d + row] = so_swiglu(g, u);
            }
        }
    }
    for (int idx = 0; idx < n; idx++)
        if (!(wts[idx] <= 0.0f))
            so_quantize_q8_0(act + (size_t)idx * d, d, actq + (size_t)idx * nbd * Q80_BLOCK);
    for (int a = 0; a < n_active; a++) {
        int e = active[a];
        const uint8_t *D = w->down + (size_t)e * expert_bytes(d, h);
#pragma omp parallel for schedule(static) num_threads(threads)
        for (int row = 0; row < h; row++) {
            float dbv = bias_at(w->down_bias, w->down_bias_type, (size_t)e * h + row);
            for (int j = offsets[e]; j < offsets[e + 1]; j++) {
                int idx = list[j];
                results[(size_t)idx * h + row] =
                    so_dot_mxfp4_q8(D + (size_t)row * nbd * MX_BLOCK,
                                    actq + (size_t)idx * nbd * Q80_BLOCK, nbd) + dbv;
            }
        }
    }
    so_combine(results, wts, batch, k, h, out);
    if (dbg) {
        if (dbg->logits) memcpy(dbg->logits, logits, sizeof(float) * (size_t)batch * E);
        if (dbg->ids) memcpy(dbg->ids, ids, sizeof(int32_t) * n);
        if (dbg->weights) memcpy(dbg->weights, wts, sizeof(float) * n);
        if (dbg->counts) memcpy(dbg->counts, counts, sizeof(int32_t) * E);
        if (dbg->offsets) memcpy(dbg->offsets, offsets, sizeof(int32_t) * (E + 1));
        if (dbg->list) memcpy(dbg->list, list, sizeof(int32_t) * offsets[E]);
        if (dbg->active) memcpy(dbg->active, active, sizeof(int32_t) * n_active);
        if (dbg->n_active) *dbg->n_active = n_active;
        if (dbg->xq) memcpy(dbg->xq, xq, (size_t)batch * nbh * Q80_BLOCK);
        if (dbg->gate) memcpy(dbg->gate, gate, sizeof(float) * (size_t)n * d);
        if (dbg->up) memcpy(dbg->up, up, sizeof(float) * (size_t)n * d);
        if (dbg->act) memcpy(dbg->act, act, sizeof(float) * (size_t)n * d);
        if (dbg->actq) memcpy(dbg->actq, actq, (size_t)n * nbd * Q80_BLOCK);
        if (dbg->results) memcpy(dbg->results, results, sizeof(float) * (size_t)n * h);
    }
    free(logits), free(ids), free(wts), free(counts), free(offsets), free(list), free(active);
    free(xq), free(actq), free(gate), free(up), free(act), free(results), free(rbias);
    return 0;
}
