// spt_kernels.hip -- gfx950 kernels of the quantized MoE hot path.
//
// The Q4_0 GEMV uses 16 lanes per weight row (one DPP row of a 64-wide
// wavefront), 16 rows per 256-thread workgroup: lane j of a row owns blocks
// j, j+16, j+32, ... so each group of 16 lanes reads 16 consecutive 18-byte
// blocks (288 contiguous bytes) per load.  Activations (Q8_0 codes + scales
// of the workgroup's tokens) are staged in LDS once and shared by the rows.
// The MXFP4 GEMV lives in spt_mx_mfma.hip.
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

constexpr int kWG = 256;
constexpr int kRowsPerWG = 16;

// ---------------------------------------------------------------------------
// Q8_0 quantization: one thread per block of 32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kWG) void k_quantize(const float *__restrict__ x, int64_t nblocks,
                                                  int8_t *__restrict__ codes,
                                                  float *__restrict__ scales,
                                                  int32_t *__restrict__ sumq,
                                                  uint8_t *__restrict__ mxtab,
                                                  uint8_t *__restrict__ blocks34) {
    int64_t b = (int64_t)blockIdx.x * kWG + threadIdx.x;
    if (b >= nblocks) return;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = x[b * 32 + i];
    uint32_t w[8];
    uint16_t dh;
    q8_quantize32(v, w, &dh);
    write_q8_block(w, dh, (size_t)b, codes, scales, mxtab, blocks34);
    if (sumq) {
        int32_t s = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) s = __builtin_amdgcn_sdot4((int)w[k], 0x01010101, s, false);
        sumq[b] = s;
    }
}

hipError_t launch_quantize(hipStream_t s, const float *x, int64_t nblocks, int8_t *codes,
                           float *scales, int32_t *sumq, uint8_t *mxtab, uint8_t *blocks34) {
    if (nblocks <= 0) return hipSuccess;
    dim3 grid((unsigned)((nblocks + kWG - 1) / kWG));
    hipLaunchKernelGGL(k_quantize, grid, dim3(kWG), 0, s, x, nblocks, codes, scales, sumq, mxtab, blocks34);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Router (forward/vector_amd64.go:11-56) and selection/packing
// (forward/moe_batch.go:142-159,305-342).
// ---------------------------------------------------------------------------

// One wavefront per (expert, token).  Lane L = 8a + s owns AVX2 accumulator
// a, SIMD lane s of dotF32AVX2: it takes element 64c + L by FMA over chunks c
// in order (lanes 0..31 also take a trailing 32-element chunk).  The
// cross-lane reduction repeats the reference's tree:
//   t_s = (((A0+A1)+A2)+A3) + (((A4+A5)+A6)+A7),  p_s = t_s + t_{s+4},
//   result = (p0+p1) + (p2+p3)   (quantSumAVX2, forward/quant_amd64.go:112).
__device__ inline float router_reduce(float a, int lane) {
    float a1 = __shfl(a, lane + 8), a2 = __shfl(a, lane + 16), a3 = __shfl(a, lane + 24);
    float t = ((a + a1) + a2) + a3;
    float u = __shfl(t, lane + 32);
    float v = t + u;
    float w = __shfl(v, lane + 4);
    float p = v + w;
    float p1 = __shfl(p, lane + 1), p2 = __shfl(p, lane + 2), p3 = __shfl(p, lane + 3);
    return (p + p1) + (p2 + p3);
}

// Top-k + softmax for every token, then the per-expert lists.  Runs on one
// workgroup.  s_ids/s_w: [batch*k], s_cnt/s_off: [experts(+1)] in LDS.
// Lane L owns experts L, L+64, ...; a per-lane bit mask marks the ones already
// selected for the current token, so exclusion costs one bit test.
__device__ void select_pack(const float *logits, int batch, int E, int k, const SelectOut &o,
                            int32_t *s_ids, float *s_w, int32_t *s_cnt, int32_t *s_off) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int n = batch * k;
    for (int t = wave; t < batch; t += nw) {
        const float *lg = logits + (size_t)t * E;
        uint32_t taken = 0;
#pragma unroll 1
        for (int r = 0; r < k; r++) {
            // selectMoEBatch round r: strict '>' scan, lowest index wins
            // ties, NaN and -Inf never win, picked experts are excluded.
            float bv = -__builtin_inff();
            int bi = -1;
#pragma unroll 1
            for (int ex = lane, i = 0; ex < E; ex += 64, i++) {
                float v = lg[ex];
                if (!((taken >> i) & 1u) && v > bv) {
                    bv = v;
                    bi = ex;
                }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                float ov = __shfl_xor(bv, off);
                int oi = __shfl_xor(bi, off);
                bool take = oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi));
                if (take) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (bi < 0) {  // nothing selectable: fallback Index=k, logit 0
                bi = r;
                bv = 0.0f;
            }
            if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
            if (lane == 0) {
                s_ids[t * k + r] = bi;
                s_w[t * k + r] = bv;
            }
        }
        if (lane == 0) {
            float mx = -__builtin_inff();
#pragma unroll 1
            for (int r = 0; r < k; r++)
                if (s_w[t * k + r] > mx) mx = s_w[t * k + r];
            float sum = 0.0f;
#pragma unroll 1
            for (int r = 0; r < k; r++) {
                float w = static_cast<float>(exp(static_cast<double>(s_w[t * k + r] - mx)));
                s_w[t * k + r] = w;
                sum += w;
            }
            float inv = sum > 0.0f ? 1.0f / sum : 1.0f;
#pragma unroll 1
            for (int r = 0; r < k; r++) {
                float w = s_w[t * k + r];
                if (sum > 0.0f) w *= inv;
                s_w[t * k + r] = w;
                o.ids[t * k + r] = s_ids[t * k + r];
                o.weights[t * k + r] = w;
            }
        }
    }
    for (int i = threadIdx.x; i < E; i += blockDim.x) s_cnt[i] = 0;
    __syncthreads();
    // Selections with Weight <= 0 are skipped (NaN weights are kept).
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        if (!(s_w[i] <= 0.0f)) atomicAdd(&s_cnt[s_ids[i]], 1);
    __syncthreads();
    if (threadIdx.x == 0) {
        int pos = 0, na = 0;
        for (int e = 0; e < E; e++) {
            s_off[e] = pos;
            pos += s_cnt[e];
            if (s_cnt[e] > 0) o.active[na++] = e;
        }
        s_off[E] = pos;
        *o.n_active = na;
    }
    __syncthreads();
    for (int i = threadIdx.x; i <= E; i += blockDim.x) {
        o.offsets[i] = s_off[i];
        if (i < E) o.counts[i] = s_cnt[i];
    }
    // Linked-list order: each expert's entries in descending idx.
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        if (s_w[i] <= 0.0f) continue;
        int e = s_ids[i], rank = 0;
        for (int q = i + 1; q < n; q++) rank += (s_ids[q] == e && !(s_w[q] <= 0.0f)) ? 1 : 0;
        o.list[s_off[e] + rank] = i;
    }
}

constexpr int kRouteTokens = 8;

__global__ __launch_bounds__(kWG) void k_route(const float *__restrict__ router,
                                               const void *bias, int bias_type,
                                               const float *__restrict__ x, int batch, int H,
                                               int E, float *logits, int topk, int do_select,
                                               SelectOut o, uint32_t *counter) {
    extern __shared__ int32_t smem_i[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = blockIdx.x * 4 + wave;
    const int t0 = blockIdx.y * kRouteTokens;
    if (e < E) {
        const float *w = router + (size_t)e * H;
        const float be = bias_at(bias, bias_type, e);
        for (int t = t0; t < batch && t < t0 + kRouteTokens; t++) {
            const float *xt = x + (size_t)t * H;
            float acc = 0.0f;
            int off = 0;
            for (; off + 64 <= H; off += 64) acc = __builtin_fmaf(w[off + lane], xt[off + lane], acc);
            if (off < H && lane < 32) acc = __builtin_fmaf(w[off + lane], xt[off + lane], acc);
            float r = router_reduce(acc, lane);
            if (lane == 0) {
                logits[(size_t)t * E + e] = r + be;
                __threadfence();
            }
        }
    }
    if (!do_select) return;
    __shared__ int s_last;
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence();
        uint32_t total = gridDim.x * gridDim.y;
        s_last = atomicAdd(counter, 1u) == total - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const int n = batch * topk;
    int32_t *s_ids = smem_i;
    float *s_w = reinterpret_cast<float *>(smem_i + n);
    int32_t *s_cnt = smem_i + 2 * n;
    int32_t *s_off = s_cnt + E;
    select_pack(logits, batch, E, topk, o, s_ids, s_w, s_cnt, s_off);
    if (threadIdx.x == 0) atomicExch(counter, 0u);
}

__global__ __launch_bounds__(kWG) void k_select(const float *logits, int batch, int E, int topk,
                                                SelectOut o) {
    extern __shared__ int32_t smem_i[];
    const int n = batch * topk;
    int32_t *s_ids = smem_i;
    float *s_w = reinterpret_cast<float *>(smem_i + n);
    int32_t *s_cnt = smem_i + 2 * n;
    int32_t *s_off = s_cnt + E;
    select_pack(logits, batch, E, topk, o, s_ids, s_w, s_cnt, s_off);
}

static size_t select_lds(int batch, int E, int topk) {
    return sizeof(int32_t) * (2 * (size_t)batch * topk + 2 * (size_t)E + 1);
}

hipError_t launch_route(hipStream_t s, const float *router, const void *bias, int bias_type,
                        const float *x, int batch, int hidden, int experts, float *logits,
                        int topk, bool select, const SelectOut &o, uint32_t *counter) {
    dim3 grid((experts + 3) / 4, (batch + kRouteTokens - 1) / kRouteTokens);
    size_t lds = select ? select_lds(batch, experts, topk) : 0;
    hipLaunchKernelGGL(k_route, grid, dim3(kWG), lds, s, router, bias, bias_type, x, batch,
                       hidden, experts, logits, topk, select ? 1 : 0, o, counter);
    return hipGetLastError();
}

hipError_t launch_select(hipStream_t s, const float *logits, int batch, int experts, int topk,
                         const SelectOut &o) {
    hipLaunchKernelGGL(k_select, dim3(1), dim3(kWG), select_lds(batch, experts, topk), s, logits,
                       batch, experts, topk, o);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Q4_0 x Q8_0 GEMV / small GEMM: y[t][row] for consecutive tokens.
// ---------------------------------------------------------------------------
template <int MAXP, int NT>
__global__ __launch_bounds__(kWG) void k_q40_gemv(Q40Args a) {
    extern __shared__ uint32_t smem_u[];
    const int nb = a.nb, words = nb * 8;
    uint32_t *s_codes = smem_u;
    float *s_scales = reinterpret_cast<float *>(smem_u + NT * words);
    int32_t *s_sumq = reinterpret_cast<int32_t *>(s_scales + NT * nb);
    const int tid = threadIdx.x, j = tid & 15, g = tid >> 4;
    const int r = blockIdx.x * kRowsPerWG + g;
    const bool row_ok = r < a.rows;
    const uint32_t row_pos = (uint32_t)(row_ok ? r : 0) * (uint32_t)(nb * kQ40Block);
    const ByteView view = make_view(a.w, a.nbytes);

    for (int c0 = 0; c0 < a.ntok; c0 += NT) {
        const int nt = min(NT, a.ntok - c0);
        for (int t = 0; t < nt; t++) {
            const uint32_t *src = reinterpret_cast<const uint32_t *>(a.codes + (size_t)(c0 + t) * nb * 32);
            for (int i = tid; i < words; i += kWG) s_codes[t * words + i] = src[i];
            for (int i = tid; i < nb; i += kWG) {
                s_scales[t * nb + i] = a.scales[(size_t)(c0 + t) * nb + i];
                s_sumq[t * nb + i] = a.sumq[(size_t)(c0 + t) * nb + i];
            }
        }
        __syncthreads();
        float acc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = 0.0f;
        for (int seg = 0; seg < nb; seg += 16 * MAXP) {
            uint32_t raw[MAXP][5];
            uint32_t off[MAXP];
#pragma unroll
            for (int p = 0; p < MAXP; p++) {
                const int b = seg + j + 16 * p;
                if (row_ok && b < nb) load_block5(view, row_pos + (uint32_t)b * kQ40Block, raw[p], &off[p]);
            }
#pragma unroll
            for (int p = 0; p < MAXP; p++) {
                const int b = seg + j + 16 * p;
                if (row_ok && b < nb) {
                    Q40Decoded dec;
                    q40_decode(raw[p], off[p], dec);
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        if (t < nt) {
                            const uint4 *q4 = reinterpret_cast<const uint4 *>(s_codes + t * words + b * 8);
                            uint4 qa = q4[0], qb = q4[1];
                            uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                            int32_t s = q40_isum(dec, q, s_sumq[t * nb + b]);
                            float ds = dec.d * s_scales[t * nb + b];
                            acc[t] = __builtin_fmaf((float)s, ds, acc[t]);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float v = acc[t];
            v += __shfl_xor(v, 8, 16);
            v += __shfl_xor(v, 4, 16);
            v += __shfl_xor(v, 2, 16);
            v += __shfl_xor(v, 1, 16);
            acc[t] = v;
        }
        if (j == 0 && row_ok) {
#pragma unroll
            for (int t = 0; t < NT; t++)
                if (t < nt) a.y[(size_t)(c0 + t) * a.rows + r] = acc[t];
        }
        __syncthreads();
    }
}

template <int MAXP>
static hipError_t launch_q40_maxp(hipStream_t s, const Q40Args &a) {
    constexpr int NT = 8;
    size_t lds = (size_t)NT * a.nb * (32 + 4 + 4);
    hipLaunchKernelGGL((k_q40_gemv<MAXP, NT>), dim3((a.rows + kRowsPerWG - 1) / kRowsPerWG), dim3(kWG),
                       lds, s, a);
    return hipGetLastError();
}

hipError_t launch_q40_gemv(hipStream_t s, const Q40Args &a) {
    if (a.rows <= 0 || a.ntok <= 0) return hipSuccess;
    const int per_lane = (a.nb + 15) / 16;
    if (per_lane <= 1) return launch_q40_maxp<1>(s, a);
    if (per_lane <= 2) return launch_q40_maxp<2>(s, a);
    if (per_lane <= 4) return launch_q40_maxp<4>(s, a);
    if (per_lane <= 6) return launch_q40_maxp<6>(s, a);
    return launch_q40_maxp<8>(s, a);
}

// ---------------------------------------------------------------------------
// Weighted combine (forward/moe_batch.go:163-192): out = 0, then for ranks
// 0..k-1 with weight > 0, out = fma(result, weight, out).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kWG) void k_combine(const float *__restrict__ results,
                                                 const float *__restrict__ weights, int topk,
                                                 int H, float *__restrict__ out) {
    const int i = blockIdx.x * kWG + threadIdx.x, t = blockIdx.y;
    if (i >= H) return;
    float o = 0.0f;
    for (int r = 0; r < topk; r++) {
        float w = weights[t * topk + r];
        if (w <= 0.0f) continue;
        o = __builtin_fmaf(results[(size_t)(t * topk + r) * H + i], w, o);
    }
    out[(size_t)t * H + i] = o;
}

hipError_t launch_combine(hipStream_t s, const float *results, const float *weights, int batch,
                          int topk, int hidden, float *out) {
    dim3 grid((hidden + kWG - 1) / kWG, batch);
    hipLaunchKernelGGL(k_combine, grid, dim3(kWG), 0, s, results, weights, topk, hidden, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Parity taps: exact per-block int32 sums with the GEMV decode functions.
// ---------------------------------------------------------------------------
__device__ inline void load_q8_block(const uint8_t *xq34, int b, uint32_t q[8], int32_t *sumq) {
    const uint8_t *c = xq34 + (size_t)b * kQ80Block + 2;
    int32_t s = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w |= (uint32_t)c[4 * k + i] << (8 * i);
            s += (int8_t)c[4 * k + i];
        }
        q[k] = w;
    }
    *sumq = s;
}

__global__ void k_block_sums_mx(const uint8_t *w, uint64_t nbytes, int rows, int nb,
                                const uint8_t *xq34, int32_t *sums) {
    const int64_t i = (int64_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= (int64_t)rows * nb) return;
    const int row = (int)(i / nb), b = (int)(i % nb);
    const ByteView v = make_view(w, nbytes);
    uint32_t d[5], o;
    load_block5(v, (uint32_t)row * nb * kMxBlock + (uint32_t)b * kMxBlock, d, &o);
    MxDecoded dec;
    mx_decode(d, o, dec);
    uint32_t q[8];
    int32_t sq;
    load_q8_block(xq34, b, q, &sq);
    sums[i] = mx_isum(dec, q);
}

__global__ void k_block_sums_q40(const uint8_t *w, uint64_t nbytes, int rows, int nb,
                                 const uint8_t *xq34, int32_t *sums) {
    const int64_t i = (int64_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= (int64_t)rows * nb) return;
    const int row = (int)(i / nb), b = (int)(i % nb);
    const ByteView v = make_view(w, nbytes);
    uint32_t d[5], o;
    load_block5(v, (uint32_t)row * nb * kQ40Block + (uint32_t)b * kQ40Block, d, &o);
    Q40Decoded dec;
    q40_decode(d, o, dec);
    uint32_t q[8];
    int32_t sq;
    load_q8_block(xq34, b, q, &sq);
    sums[i] = q40_isum(dec, q, sq);
}

hipError_t launch_block_sums_mx(hipStream_t s, const uint8_t *w, uint64_t nbytes, int rows, int nb,
                                const uint8_t *xq34, int32_t *sums) {
    int64_t n = (int64_t)rows * nb;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_block_sums_mx, dim3((unsigned)((n + kWG - 1) / kWG)), dim3(kWG), 0, s, w,
                       nbytes, rows, nb, xq34, sums);
    return hipGetLastError();
}

hipError_t launch_block_sums_q40(hipStream_t s, const uint8_t *w, uint64_t nbytes, int rows,
                                 int nb, const uint8_t *xq34, int32_t *sums) {
    int64_t n = (int64_t)rows * nb;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_block_sums_q40, dim3((unsigned)((n + kWG - 1) / kWG)), dim3(kWG), 0, s, w,
                       nbytes, rows, nb, xq34, sums);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic MXFP4 weights (same bytes as the host generator).
// ---------------------------------------------------------------------------
__device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void k_synth_mxfp4(uint8_t *dst, uint64_t key, uint64_t first, uint64_t n, int lo,
                              int span) {
    const uint64_t i = (uint64_t)blockIdx.x * kWG + threadIdx.x;
    if (i >= n) return;
    const uint64_t g = first + i;
    const uint64_t h0 = mix64(key + (3 * g) * 0x9E3779B97F4A7C15ull);
    const uint64_t h1 = mix64(key + (3 * g + 1) * 0x9E3779B97F4A7C15ull);
    const uint64_t h2 = mix64(key + (3 * g + 2) * 0x9E3779B97F4A7C15ull);
    uint8_t *o = dst + i * kMxBlock;
    o[0] = (uint8_t)(lo + (int)(h0 % (uint64_t)span));
#pragma unroll
    for (int k = 0; k < 8; k++) {
        o[1 + k] = (uint8_t)(h1 >> (8 * k));
        o[9 + k] = (uint8_t)(h2 >> (8 * k));
    }
}

hipError_t launch_synth_mxfp4(hipStream_t s, uint8_t *dst, uint64_t key, uint64_t first_block,
                              uint64_t nblocks, int scale_lo, int scale_hi) {
    if (nblocks == 0) return hipSuccess;
    const uint64_t per_launch = (uint64_t)kWG * 1048576;
    for (uint64_t done = 0; done < nblocks; done += per_launch) {
        uint64_t n = nblocks - done < per_launch ? nblocks - done : per_launch;
        hipLaunchKernelGGL(k_synth_mxfp4, dim3((unsigned)((n + kWG - 1) / kWG)), dim3(kWG), 0, s,
                           dst + done * kMxBlock, key, first_block + done, n, scale_lo,
                           scale_hi - scale_lo + 1);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

}  // namespace spt
