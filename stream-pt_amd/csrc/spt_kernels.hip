// spt_kernels.hip -- gfx950 kernels of the quantized MoE hot path.
//
// The Q4_0 GEMV uses 16 lanes per weight row (one DPP row of a 64-wide
// wavefront), 16 rows per 256-thread workgroup: lane j of a row owns blocks
// j, j+16, j+32, ... so each group of 16 lanes reads 16 consecutive 18-byte
// blocks (288 contiguous bytes) per load.  Activations (Q8_0 codes + scales
// of the workgroup's tokens) are staged in LDS once and shared by the rows.
// The MXFP4 GEMV lives in spt_mx_mfma.hip.
#include <atomic>

#include "spt_device.h"
#include "spt_kernels.h"
#include "spt_select.h"

namespace spt {

constexpr int kWG = 256;
constexpr int kRowsPerWG = 16;

// ---------------------------------------------------------------------------
// Q8_0 quantization: one half-wave per block of 32, one element per lane
// (coalesced loads; the block's amax by DPP and a swizzle).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kWG) void k_quantize(const float *__restrict__ x, int64_t nblocks,
                                                  int8_t *__restrict__ codes,
                                                  float *__restrict__ scales,
                                                  int32_t *__restrict__ sumq,
                                                  uint8_t *__restrict__ mxtab,
                                                  uint8_t *__restrict__ blocks34,
                                                  uint32_t *__restrict__ btab) {
    const int tid = threadIdx.x, lane = tid & 63, i = tid & 31;
    const int64_t b = (int64_t)blockIdx.x * (kWG / 32) + (tid >> 5);
    const bool ok = b < nblocks;
    const float v = ok ? x[b * 32 + i] : 0.0f;
    uint16_t dh;
    const int q = q8_quantize_half(v, lane, &dh);  // every lane takes part (cross-lane steps)
    if (ok) write_q8_lane(q, dh, i, (size_t)b, codes, scales, mxtab, blocks34, btab);
    if (sumq) {
        int s = q;
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) s += __shfl_xor(s, off, 32);
        if (ok && i == 0) sumq[b] = s;
    }
}

hipError_t launch_quantize(hipStream_t s, const float *x, int64_t nblocks, int8_t *codes,
                           float *scales, int32_t *sumq, uint8_t *mxtab, uint8_t *blocks34,
                           uint32_t *btab) {
    if (nblocks <= 0) return hipSuccess;
    dim3 grid((unsigned)((nblocks + kWG / 32 - 1) / (kWG / 32)));
    hipLaunchKernelGGL(k_quantize, grid, dim3(kWG), 0, s, x, nblocks, codes, scales, sumq, mxtab, blocks34, btab);
    return hipGetLastError();
}

// GGML Q8_0 blocks -> the quantizer's views: one half-wave per block, lane i
// holding code i (the layouts of write_q8_lane) and its code sum by shuffles.
__global__ __launch_bounds__(kWG) void k_q8_unpack(const uint8_t *__restrict__ blocks34, int64_t nblocks,
                                                   int8_t *__restrict__ codes, float *__restrict__ scales,
                                                   int32_t *__restrict__ sumq, uint8_t *__restrict__ mxtab) {
    const int tid = threadIdx.x, lane = tid & 63, i = tid & 31;
    const int64_t b = (int64_t)blockIdx.x * (kWG / 32) + (tid >> 5);
    if (b >= nblocks) return;  // whole half-waves
    const uint8_t *blk = blocks34 + b * kQ80Block;
    const int q = (int)(int8_t)blk[2 + i];
    const uint16_t dh = (uint16_t)(blk[0] | (blk[1] << 8));
    write_q8_lane(q, dh, lane & 31, (size_t)b, codes, scales, mxtab, nullptr, nullptr);
    if (sumq) {
        int s = q;
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) s += __shfl_xor(s, off, 32);
        if (i == 0) sumq[b] = s;
    }
}

hipError_t launch_q8_unpack(hipStream_t s, const uint8_t *blocks34, int64_t nblocks, int8_t *codes,
                            float *scales, int32_t *sumq, uint8_t *mxtab) {
    if (nblocks <= 0) return hipSuccess;
    dim3 grid((unsigned)((nblocks + kWG / 32 - 1) / (kWG / 32)));
    hipLaunchKernelGGL(k_q8_unpack, grid, dim3(kWG), 0, s, blocks34, nblocks, codes, scales, sumq, mxtab);
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

// Inclusive prefix sum over the 64 lanes of a wavefront: Hillis-Steele by
// DPP row shifts within rows of 16, then the row totals carried by the row
// broadcasts (lane 15 to the next row, lane 31 to rows 2-3).
__device__ __attribute__((always_inline)) inline int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false); // row_bcast:15 -> rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false); // row_bcast:31 -> rows 2, 3
    return x;
}

__device__ __attribute__((always_inline)) inline int lane63(int x) { return __builtin_amdgcn_readlane(x, 63); }

// Per-expert lists (forward/moe_batch.go:142-159) for n = batch*k selections
// held in LDS (s_ids/s_w), by one workgroup of kSelWG threads.  Selections
// with Weight <= 0 are skipped (NaN weights are kept); experts ascending;
// inside a list descending idx, as the reference's push-at-head linked list
// yields.  Counts by LDS atomics, offsets and the active-expert list by one
// wavefront's prefix scan; ranks from kSelChunk-entry chunks taken in
// descending idx order: a per-expert bit row marks the chunk's members, so an
// entry's rank is its expert's running count plus the bits below it.
constexpr int kSelWG = 1024;
static_assert(kSelWG >= 4 * kMaxExperts, "four threads per expert rank the GEMM experts");
constexpr int kSelChunk = 512;
constexpr int kSelWords = kSelChunk / 32;

__device__ void pack_lists(int n, int E, const SelectOut &o, const int32_t *s_ids, const float *s_w,
                           int32_t *s_cnt, int32_t *s_off, int32_t *s_run, uint32_t *s_bits) {
    __shared__ int s_gemm_on, s_nv;
    // the GEMV experts and their pass prefix, for the start table
    int32_t *s_poff = reinterpret_cast<int32_t *>(s_bits + kSelWords * E);
    int32_t *s_gva = s_poff + E + 1;
    const int tid = threadIdx.x;
    for (int i = tid; i < E; i += blockDim.x) {
        s_cnt[i] = 0;
        s_run[i] = 0;
    }
    __syncthreads();
    for (int i = tid; i < n; i += blockDim.x)
        if (!(s_w[i] <= 0.0f)) atomicAdd(&s_cnt[s_ids[i]], 1);
    __syncthreads();
    if (tid < 64) {
        // offsets (scan of counts), the active list, and the GEMV expert
        // list with its prefix (passes of kGemvTokens) in ascending expert
        // order; the GEMM experts' count and tiles (ordered below)
        int pos = 0, na = 0, nv = 0, nm = 0, npass = 0, ntile = 0;
        const uint64_t below = (1ull << tid) - 1ull;
        // GEMM work items the threshold would give
        int tiles = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int c = e0 + tid < E ? s_cnt[e0 + tid] : 0;
            tiles += lane63(wave_incl_scan((c > 0 && c >= o.gemm_min) ? (c + kGemmTokens - 1) / kGemmTokens : 0));
        }
        const bool gemm_on = (int64_t)tiles * o.gemm_units >= (int64_t)o.gemm_min_items;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + tid;
            const int c = e < E ? s_cnt[e] : 0;
            const bool big = gemm_on && c > 0 && c >= o.gemm_min;
            const int np = big ? 0 : (c + kGemvTokens - 1) / kGemvTokens;
            const int ntl = big ? (c + kGemmTokens - 1) / kGemmTokens : 0;
            const int incl = wave_incl_scan(c), pincl = wave_incl_scan(np), tincl = wave_incl_scan(ntl);
            const uint64_t act = __ballot(c > 0), actv = __ballot(c > 0 && !big), actm = __ballot(big);
            if (e < E) {
                s_off[e] = pos + incl - c;
                o.offsets[e] = pos + incl - c;
                o.counts[e] = c;
                if (c > 0) o.active[na + __builtin_popcountll(act & below)] = e;
                if (c > 0 && !big) {
                    const int r = nv + __builtin_popcountll(actv & below);
                    o.gv_active[r] = e;
                    o.gv_pass_off[r] = npass + pincl - np;
                    s_gva[r] = e;
                    s_poff[r] = npass + pincl - np;
                }
            }
            pos += lane63(incl);
            npass += lane63(pincl);
            ntile += lane63(tincl);
            na += __builtin_popcountll(act);
            nv += __builtin_popcountll(actv);
            nm += __builtin_popcountll(actm);
        }
        if (tid == 0) {
            s_off[E] = pos;
            o.offsets[E] = pos;
            *o.n_active = na;
            *o.gv_n = nv;
            o.gv_pass_off[nv] = npass;
            s_poff[nv] = npass;
            s_nv = nv;
            *o.gm_n = nm;
            o.gm_tile_off[nm] = ntile;
            if (o.gm_claim) {
                o.gm_claim[0] = 0;
                o.gm_claim[1] = 0;
            }
            s_gemm_on = gemm_on;
        }
    }
    // The GEMM experts by descending count (equal counts by ascending id), so
    // the GEMM's work items, claimed in order by workgroups as they free up,
    // end with the smallest: an expert's rank and tile prefix count the GEMM
    // experts ordered before it.
    // Four threads per expert, each counting over a quarter of the experts
    // (kSelWG >= 4 * kMaxExperts), summed across the four lanes.
    __syncthreads();
    if (s_gemm_on && tid < 4 * E) {
        const int e = tid >> 2, part = tid & 3, q = (E + 3) / 4;
        const int c = s_cnt[e];
        int rank = 0, pre = 0;
        for (int f = part * q; f < min(E, part * q + q); f++) {
            const int cf = s_cnt[f];
            if (cf > 0 && cf >= o.gemm_min && (cf > c || (cf == c && f < e))) {
                rank++;
                pre += (cf + kGemmTokens - 1) / kGemmTokens;
            }
        }
        rank += __shfl_xor(rank, 1);
        pre += __shfl_xor(pre, 1);
        rank += __shfl_xor(rank, 2);
        pre += __shfl_xor(pre, 2);
        if (part == 0 && c > 0 && c >= o.gemm_min) {
            o.gm_active[rank] = e;
            o.gm_tile_off[rank] = pre;
        }
    }
    // Start table of the two GEMV launches (threads [0, G0) the first,
    // [G0, G0 + G1) the second): workgroup b of G takes items
    // [b W / G, (b + 1) W / G) of the W = passes x row units, from the slot
    // holding the pass of its first item (the last slot whose pass prefix is
    // at most that pass).  Written before the lists, so the stores' latency
    // overlaps them.
    if (o.gv_start) {
        const int nv = s_nv, P = s_poff[nv];
        for (int i = tid; i < o.gv_grid[0] + o.gv_grid[1]; i += blockDim.x) {
            const int l = i < o.gv_grid[0] ? 0 : 1, b = i - (l ? o.gv_grid[0] : 0);
            const int G = o.gv_grid[l], tiles = o.gv_tiles[l];
            const int W = P * tiles;
            const int w0 = (int)((int64_t)b * W / G), w1 = (int)((int64_t)(b + 1) * W / G);
            const int q0 = tiles > 0 ? w0 / tiles : 0;
            int lo = 0, hi = nv - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_poff[mid] <= q0) lo = mid;
                else hi = mid - 1;
            }
            int32_t *d = o.gv_start + ((size_t)l * kGvStartMax + b) * kGvStartWords;
            *reinterpret_cast<int4 *>(d) = make_int4(w0, w1, lo, nv > 0 ? s_gva[lo] : 0);
            d[4] = nv > 0 ? q0 - s_poff[lo] : 0;
        }
    }
    for (int p0 = 0; p0 < n; p0 += kSelChunk) {
        for (int i = tid; i < E * kSelWords; i += blockDim.x) s_bits[i] = 0u;
        __syncthreads();
        const int p = p0 + tid;
        const int idx = n - 1 - p;
        const bool valid = tid < kSelChunk && p < n && !(s_w[idx] <= 0.0f);
        const int e = valid ? s_ids[idx] : 0;
        if (valid) atomicOr(&s_bits[e * kSelWords + (tid >> 5)], 1u << (tid & 31));
        __syncthreads();
        if (valid) {
            int rank = s_run[e];
            const int wi = tid >> 5;
            for (int w = 0; w < wi; w++) rank += __builtin_popcount(s_bits[e * kSelWords + w]);
            rank += __builtin_popcount(s_bits[e * kSelWords + wi] & ((1u << (tid & 31)) - 1u));
            o.list[s_off[e] + rank] = idx;
        }
        __syncthreads();
        for (int i = tid; i < E; i += blockDim.x) {
            int add = 0;
            for (int w = 0; w < kSelWords; w++) add += __builtin_popcount(s_bits[i * kSelWords + w]);
            s_run[i] += add;
        }
        __syncthreads();
    }
}

static size_t select_lds(int n, int E) {
    return sizeof(int32_t) * (2 * (size_t)n + 3 * (size_t)E + 1) + sizeof(uint32_t) * kSelWords * (size_t)E +
           sizeof(int32_t) * (2 * (size_t)E + 1);
}

// Router logits for batches of more than kRouteLdsMaxBatch tokens: a
// workgroup per (4 experts, EW * TT tokens), its four wavefronts in a
// (4 / EW) x EW arrangement of (EW experts, TT tokens) each.  Lane L keeps one
// accumulator per (expert, token) of its wavefront, each the FMA chain of
// k_route below (element 64c + L over chunks c in order, the same bits), and
// loads a chunk's element of each of its router rows and token rows once for
// all of those chains, the loads of U chunks of every row in flight at once
// (one pass over a 2880-wide row at U = 45).  With q set,
// the workgroups of a token group also quantize its rows of x to Q8_0 (a
// half-wave per block).
template <int EW, int TT, int U>
__global__ __launch_bounds__(kWG) void k_route_tile(const float *__restrict__ router, const void *bias,
                                                    int bias_type, const float *__restrict__ x, int B, int H, int E,
                                                    float *__restrict__ logits, QuantOut q) {
    static_assert(EW == 1 || EW == 2 || EW == 4, "wavefronts of one, two or four experts");
    constexpr int TW = EW * TT;  // tokens per workgroup (U: chunks per pass of loads)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tg0 = blockIdx.y * TW;
    if (q.codes || q.blocks34) {
        const int nbh = H / 32, nq = min(TW, B - tg0) * nbh;
        for (int f0 = blockIdx.x * (kWG / 32); f0 < nq; f0 += gridDim.x * (kWG / 32)) {
            const int f = f0 + (tid >> 5), i = tid & 31;
            const int fi = f < nq ? f : 0;
            const int t = tg0 + fi / nbh, b = fi % nbh;
            uint16_t dh;
            int qv;
            if (q.src34) {
                const uint8_t *blk = q.src34 + ((size_t)t * nbh + b) * kQ80Block;
                qv = (int)(int8_t)blk[2 + i];
                dh = (uint16_t)(blk[0] | (blk[1] << 8));
            } else {
                const float v = f < nq ? x[(size_t)t * H + b * 32 + i] : 0.0f;
                qv = q8_quantize_half(v, lane, &dh);  // every lane takes part
            }
            if (f < nq) write_q8_lane(qv, dh, i, (size_t)t * nbh + b, q.codes, q.scales, q.mxtab, q.blocks34, q.btab);
        }
    }
    const int e0 = blockIdx.x * 4 + EW * (wave % (4 / EW)), t0 = tg0 + TT * (wave / (4 / EW));
    if (e0 >= E || t0 >= B) return;  // whole wavefronts
    const float *wr[EW], *xr[TT];
#pragma unroll
    for (int i = 0; i < EW; i++) wr[i] = router + (size_t)min(e0 + i, E - 1) * H + lane;
#pragma unroll
    for (int j = 0; j < TT; j++) xr[j] = x + (size_t)min(t0 + j, B - 1) * H + lane;
    float acc[EW][TT];
#pragma unroll
    for (int i = 0; i < EW; i++)
#pragma unroll
        for (int j = 0; j < TT; j++) acc[i][j] = 0.0f;
    // passes of U chunks with every load of a pass in flight at once;
    // chunks past the row load its last chunk and are not multiplied
    const int nfull = H / 64;
    for (int c0 = 0; c0 < nfull; c0 += U) {
        float wv[U][EW], xv[U][TT];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = min(c0 + u, nfull - 1) * 64;
#pragma unroll
            for (int i = 0; i < EW; i++) wv[u][i] = wr[i][c];
#pragma unroll
            for (int j = 0; j < TT; j++) xv[u][j] = xr[j][c];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (c0 + u < nfull) {
#pragma unroll
                for (int i = 0; i < EW; i++)
#pragma unroll
                    for (int j = 0; j < TT; j++) acc[i][j] = __builtin_fmaf(wv[u][i], xv[u][j], acc[i][j]);
            }
        }
    }
    if (nfull * 64 < H && lane < 32) {
#pragma unroll
        for (int i = 0; i < EW; i++)
#pragma unroll
            for (int j = 0; j < TT; j++)
                acc[i][j] = __builtin_fmaf(wr[i][nfull * 64], xr[j][nfull * 64], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < EW; i++)
#pragma unroll
        for (int j = 0; j < TT; j++) {
            const float r = router_reduce(acc[i][j], lane);
            if (lane == 0 && e0 + i < E && t0 + j < B)
                logits[(size_t)(t0 + j) * E + e0 + i] = r + bias_at(bias, bias_type, e0 + i);
        }
}

// Router logits: one wavefront per (expert, token), a workgroup each, so a
// decode step's 128 logits spread over 128 CUs.  The router row and x arrive
// in LDS through 16-byte loads (segments of kRouteSeg floats, every load of a
// segment in flight at once; loads past a row read zeros), then lane L runs
// dotF32AVX2's chain for its accumulator from LDS.  While the loads fly, the
// wavefronts e < H/64 quantize two blocks of x each (a half-wave per block).
constexpr int kRouteSeg = 4096;
// Up to this many tokens the router spreads over one workgroup per (expert,
// token) with LDS staging (latency); beyond, k_route_tile (throughput).
// Measured on the 36-layer step (ms, this form against the tiled one): 2
// tokens 1.401 / 1.433, 4: 2.176 / 2.212, 6: 2.764 / 2.780, 8: 3.230 /
// 3.235, 12: 4.167 / 4.082, 16: 4.873 / 4.780.
constexpr int kRouteLdsMaxBatch = 8;
template <bool MULTI>  // MULTI: H > kRouteSeg, segments in a loop; else one segment, straight-line
__global__ __launch_bounds__(64) void k_route(const float *__restrict__ router, const void *bias, int bias_type,
                                              const float *__restrict__ x, int H, int E,
                                              float *__restrict__ logits, QuantOut q) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) float s_w[kRouteSeg], s_x[kRouteSeg];
    const int lane = threadIdx.x;
    const int e = blockIdx.x, t = blockIdx.y;
    const float *xt = x + (size_t)t * H;
    // wavefronts past the experts only quantize (their router range is empty)
    const rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(router + (size_t)(e < E ? e : 0) * H), (short)0,
                                                        e < E ? H * 4 : 0, kRsrcWord3);
    const rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(xt), (short)0, H * 4, kRsrcWord3);
    const int nfull = H / 64, nbh = H / 32;
    // this wavefront's share of the Q8_0 of x, read before the segment loads
    const bool qon = (q.codes || q.blocks34) && 2 * e < nbh;
    const int qb = 2 * e + (lane >> 5), qi = lane & 31;
    float qin = 0.0f;
    int qcode = 0;
    uint16_t qdh = 0;
    if (qon && qb < nbh) {
        if (q.src34) {
            const uint8_t *blk = q.src34 + ((size_t)t * nbh + qb) * kQ80Block;
            qcode = (int)(int8_t)blk[2 + qi];
            qdh = (uint16_t)(blk[0] | (blk[1] << 8));
        } else {
            qin = xt[qb * 32 + qi];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr int kLoads = kRouteSeg / 256;  // 16-byte loads per lane per segment and row
    float acc = 0.0f;
    for (int s0 = 0; s0 == 0 || (MULTI && s0 < nfull * 64); s0 += kRouteSeg) {
        u32x4 wv[kLoads], xv[kLoads];
#pragma unroll
        for (int j = 0; j < kLoads; j++) {
            const uint32_t off = (uint32_t)(s0 + 4 * (lane + 64 * j)) * 4u;
            wv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0));
            xv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
        }
        if (s0 == 0 && qon) {
            uint16_t dh = qdh;
            const int qv = q.src34 ? qcode : q8_quantize_half(qin, lane, &dh);  // every lane takes part
            if (qb < nbh) write_q8_lane(qv, dh, qi, (size_t)t * nbh + qb, q.codes, q.scales, q.mxtab, q.blocks34, q.btab);
        }
        __syncthreads();  // the previous segment's LDS reads are done
#pragma unroll
        for (int j = 0; j < kLoads; j++) {
            reinterpret_cast<u32x4 *>(s_w)[lane + 64 * j] = wv[j];
            reinterpret_cast<u32x4 *>(s_x)[lane + 64 * j] = xv[j];
        }
        __syncthreads();
        // chunks of 64 of this segment, in order (dotF32AVX2's FMA chains)
        const int c1 = min(nfull, (s0 + kRouteSeg) / 64);
        for (int c = s0 / 64; c < c1; c++) acc = __builtin_fmaf(s_w[c * 64 - s0 + lane], s_x[c * 64 - s0 + lane], acc);
    }
    if (e >= E) return;
    if (nfull * 64 < H && lane < 32) acc = __builtin_fmaf(router[(size_t)e * H + nfull * 64 + lane], xt[nfull * 64 + lane], acc);
    const float r = router_reduce(acc, lane);
    if (lane == 0) logits[(size_t)t * E + e] = r + bias_at(bias, bias_type, e);
}

// Selection and packing from the logits of a whole batch: one workgroup;
// its wavefronts take tokens in turn, then the lists are packed.
__global__ __launch_bounds__(kSelWG) void k_select(const float *__restrict__ logits, int batch, int E,
                                                   int topk, SelectOut o) {
    extern __shared__ int32_t smem_i[];
    const int n = batch * topk;
    int32_t *s_ids = smem_i;
    float *s_w = reinterpret_cast<float *>(smem_i + n);
    int32_t *s_cnt = smem_i + 2 * n;
    int32_t *s_off = s_cnt + E;
    int32_t *s_run = s_off + E + 1;
    uint32_t *s_bits = reinterpret_cast<uint32_t *>(s_run + E);
    const int wave = threadIdx.x >> 6;
    // each wave takes tokens wave, wave + 16, ...; the next token's logits
    // are loaded while the current one is selected
    constexpr int kStride = kSelWG / 64;
    TokenLogits next{};
    if (wave < batch) next = load_token_logits(logits + (size_t)wave * E, E);
    for (int t = wave; t < batch; t += kStride) {
        const TokenLogits cur = next;
        if (t + kStride < batch) next = load_token_logits(logits + (size_t)(t + kStride) * E, E);
        select_token(cur, E, topk, o.ids + t * topk, o.weights + t * topk, s_ids + t * topk, s_w + t * topk);
    }
    __syncthreads();
    pack_lists(n, E, o, s_ids, s_w, s_cnt, s_off, s_run, s_bits);
}

// Large batches: the selections first, a wavefront per token over the whole
// grid (kTopkWG / 64 tokens per workgroup) ...
constexpr int kTopkWG = 256;
__global__ __launch_bounds__(kTopkWG) void k_topk(const float *__restrict__ logits, int batch, int E, int topk,
                                                  int32_t *ids, float *weights) {
    const int t = blockIdx.x * (kTopkWG / 64) + (int)(threadIdx.x >> 6);
    if (t >= batch) return;  // whole wavefronts
    select_token(load_token_logits(logits + (size_t)t * E, E), E, topk, ids + t * topk, weights + t * topk,
                 nullptr, nullptr);
}

// ... then the packing of all of them by one workgroup, from the ids and
// weights just written.
__global__ __launch_bounds__(kSelWG) void k_pack(int batch, int E, int topk, SelectOut o) {
    extern __shared__ int32_t smem_i[];
    const int n = batch * topk;
    int32_t *s_ids = smem_i;
    float *s_w = reinterpret_cast<float *>(smem_i + n);
    int32_t *s_cnt = smem_i + 2 * n;
    int32_t *s_off = s_cnt + E;
    int32_t *s_run = s_off + E + 1;
    uint32_t *s_bits = reinterpret_cast<uint32_t *>(s_run + E);
    for (int i = threadIdx.x; i < n; i += kSelWG) {
        s_ids[i] = o.ids[i];
        s_w[i] = o.weights[i];
    }
    __syncthreads();
    pack_lists(n, E, o, s_ids, s_w, s_cnt, s_off, s_run, s_bits);
}

int device_cus() {
    constexpr int kMaxCuDevices = 64;
    static std::atomic<int> cus[kMaxCuDevices];  // 0: not queried yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxCuDevices) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

hipError_t launch_route(hipStream_t s, const float *router, const void *bias, int bias_type,
                        const float *x, int batch, int hidden, int experts, float *logits,
                        const QuantOut &q) {
    if (batch > kRouteLdsMaxBatch) {
        // Every wavefront loads its router rows and token rows whole, so a
        // wider (experts x tokens) tile reads fewer bytes per logit from the
        // caches (rows per logit: 1 at 2 x 2, 0.75 at 2 x 4, 0.5 at 4 x 4)
        // but makes fewer workgroups.  Measured per router launch at 128
        // experts (us, 2 x 2 / 2 x 4 / 4 x 4): 64 tokens 11.2 / 13.2 / 18.6,
        // 96: 16.4 / 15.0 / 19.2, 192: 24.9 / 18.5 / 22.6, 256: 33.3 / 27.0
        // / 24.9, 512: 58.8 / 42.0 / 42.1, 1024: 108 / 74 / 68.  So from 256
        // tokens 4 x 4 in passes of 15 chunks, from 80 tokens 2 x 4 in passes
        // of 23, from 32 tokens 2 x 2 (512 workgroups at 64 tokens, one
        // round); below, (1 expert, 1 token), so few tokens still fill the
        // CUs, in passes of 23 chunks (76 VGPRs; measured while this form
        // also took 8 tokens: 7.1-7.5 against 7.9 us there, and 9.6-9.9
        // against 10.7-12.6 at 31, with one pass of 45).
        if (batch >= 256) {
            dim3 grid((experts + 3) / 4, (batch + 15) / 16);
            hipLaunchKernelGGL((k_route_tile<4, 4, 15>), grid, dim3(kWG), 0, s, router, bias, bias_type, x, batch,
                               hidden, experts, logits, q);
        } else if (batch >= 80) {
            dim3 grid((experts + 3) / 4, (batch + 7) / 8);
            hipLaunchKernelGGL((k_route_tile<2, 4, 23>), grid, dim3(kWG), 0, s, router, bias, bias_type, x, batch,
                               hidden, experts, logits, q);
        } else if (batch >= 32) {
            dim3 grid((experts + 3) / 4, (batch + 3) / 4);
            hipLaunchKernelGGL((k_route_tile<2, 2, 45>), grid, dim3(kWG), 0, s, router, bias, bias_type, x, batch,
                               hidden, experts, logits, q);
        } else {
            dim3 grid((experts + 3) / 4, batch);
            hipLaunchKernelGGL((k_route_tile<1, 1, 23>), grid, dim3(kWG), 0, s, router, bias, bias_type, x, batch,
                               hidden, experts, logits, q);
        }
        return hipGetLastError();
    }
    // a wavefront per (expert, token); the Q8_0 of x needs H/64 of them per token
    const int ex = experts > (hidden / 32 + 1) / 2 ? experts : (hidden / 32 + 1) / 2;
    dim3 grid(ex, batch);
    if (hidden > kRouteSeg)
        hipLaunchKernelGGL(k_route<true>, grid, dim3(64), 0, s, router, bias, bias_type, x, hidden, experts, logits, q);
    else
        hipLaunchKernelGGL(k_route<false>, grid, dim3(64), 0, s, router, bias, bias_type, x, hidden, experts, logits, q);
    return hipGetLastError();
}

hipError_t launch_pack(hipStream_t s, int batch, int experts, int topk, const SelectOut &o) {
    hipLaunchKernelGGL(k_pack, dim3(1), dim3(kSelWG), select_lds(batch * topk, experts), s, batch, experts, topk, o);
    return hipGetLastError();
}

hipError_t launch_select(hipStream_t s, const float *logits, int batch, int experts, int topk,
                         const SelectOut &o) {
    // Up to one token per wavefront of the packing workgroup: one kernel;
    // beyond, the selections spread over the grid first.
    if (batch <= kSelWG / 64) {
        hipLaunchKernelGGL(k_select, dim3(1), dim3(kSelWG), select_lds(batch * topk, experts), s, logits,
                           batch, experts, topk, o);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_topk, dim3((batch + kTopkWG / 64 - 1) / (kTopkWG / 64)), dim3(kTopkWG), 0, s, logits, batch,
                       experts, topk, o.ids, o.weights);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_pack, dim3(1), dim3(kSelWG), select_lds(batch * topk, experts), s, batch, experts, topk, o);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Q4_0 x Q8_0 GEMV / small GEMM: y[t][row] for consecutive tokens.
// ---------------------------------------------------------------------------
template <int MAXP, int NT>
__global__ __launch_bounds__(kWG) void k_q40_gemv(Q40Args args) {
    extern __shared__ uint32_t smem_u[];
    int tile = blockIdx.x;
    const Q40Args a = q40_matrix(args, &tile, kRowsPerWG);
    const int nb = a.nb, words = nb * 8;
    uint32_t *s_codes = smem_u;
    float *s_scales = reinterpret_cast<float *>(smem_u + NT * words);
    int32_t *s_sumq = reinterpret_cast<int32_t *>(s_scales + NT * nb);
    const int tid = threadIdx.x, j = tid & 15, g = tid >> 4;
    const int r = tile * kRowsPerWG + g;
    const bool row_ok = r < a.rows;
    const uint32_t row_pos = (uint32_t)(row_ok ? r : 0) * (uint32_t)(nb * kQ40Block);
    const ByteView view = make_view(a.w, a.nbytes);

    // token passes of NT tokens: workgroup (x, y) takes passes y, y + G, ...
    for (int c0 = blockIdx.y * NT; c0 < a.ntok; c0 += gridDim.y * NT) {
        const int nt = min(NT, a.ntok - c0);
        if (a.xq34) {
            // GGML Q8_0 blocks (34 bytes, 2-byte aligned): one thread per
            // block unpacks codes, the widened scale and the code sum
            for (int i = tid; i < nt * nb; i += kWG) {
                const uint16_t *blk = reinterpret_cast<const uint16_t *>(a.xq34 + ((size_t)c0 * nb + i) * kQ80Block);
                uint16_t h[17];
#pragma unroll
                for (int k = 0; k < 17; k++) h[k] = blk[k];
                int32_t sq = 0;
                const int t = i / nb, b = i - t * nb;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t w = (uint32_t)h[1 + 2 * k] | ((uint32_t)h[2 + 2 * k] << 16);
                    s_codes[t * words + b * 8 + k] = w;
                    sq += __builtin_amdgcn_sdot4((int)w, 0x01010101, 0, false);
                }
                s_scales[i] = f16_bits_to_f32(h[0]);
                s_sumq[i] = sq;
            }
        } else {
            // the pass's codes (consecutive tokens: one contiguous run),
            // scales and code sums; every load issued before the stores
            typedef uint32_t u4 __attribute__((ext_vector_type(4)));
            const u4 *src = reinterpret_cast<const u4 *>(a.codes + (size_t)c0 * nb * 32);
            const int n16 = nt * words / 4;
            constexpr int kU = 8;
            for (int i0 = 0; i0 < n16; i0 += kU * kWG) {
                u4 v[kU];
#pragma unroll
                for (int u = 0; u < kU; u++) {
                    const int i = i0 + u * kWG + tid;
                    if (i < n16) v[u] = src[i];
                }
#pragma unroll
                for (int u = 0; u < kU; u++) {
                    const int i = i0 + u * kWG + tid;
                    if (i < n16) reinterpret_cast<u4 *>(s_codes)[i] = v[u];
                }
            }
            for (int i = tid; i < nt * nb; i += kWG) {
                s_scales[i] = a.scales[(size_t)c0 * nb + i];
                s_sumq[i] = a.sumq[(size_t)c0 * nb + i];
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
                if (t < nt) q40_store(a, (size_t)(c0 + t) * a.rows + r, r, acc[t]);
        }
        __syncthreads();
    }
}

template <int MAXP, int NT>
static hipError_t launch_q40_nt(hipStream_t s, const Q40Args &a) {
    const size_t lds = (size_t)NT * a.nb * (32 + 4 + 4);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_q40_gemv<MAXP, NT>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    // row tiles (of every matrix) x token passes, up to about four
    // workgroups per CU
    int tiles = (a.rows + kRowsPerWG - 1) / kRowsPerWG;
    for (int i = 0; i < a.nmore; i++) tiles += (a.more[i].rows + kRowsPerWG - 1) / kRowsPerWG;
    const int passes = (a.ntok + NT - 1) / NT;
    int gy = (1024 + tiles - 1) / tiles;
    gy = gy < 1 ? 1 : (gy > passes ? passes : gy);
    hipLaunchKernelGGL((k_q40_gemv<MAXP, NT>), dim3(tiles, gy), dim3(kWG), lds, s, a);
    return hipGetLastError();
}

// Eight tokens per pass while their activations fit the LDS, fewer for wider
// inputs (kQ40MaxInput: one token of 40 bytes per block).
template <int MAXP>
static hipError_t launch_q40_maxp(hipStream_t s, const Q40Args &a) {
    const size_t per_tok = (size_t)a.nb * (32 + 4 + 4);
    if (8 * per_tok <= kQ40GemvLds) return launch_q40_nt<MAXP, 8>(s, a);
    if (4 * per_tok <= kQ40GemvLds) return launch_q40_nt<MAXP, 4>(s, a);
    if (2 * per_tok <= kQ40GemvLds) return launch_q40_nt<MAXP, 2>(s, a);
    if (per_tok <= kQ40GemvLds) return launch_q40_nt<MAXP, 1>(s, a);
    return hipErrorInvalidValue;  // beyond kQ40MaxInput, rejected by the ABI
}

hipError_t launch_q40_gemv(hipStream_t s, const Q40Args &a) {
    if (a.rows <= 0 || a.ntok <= 0) return hipSuccess;
    if (a.nmore > 0 || a.xq34) {
        // several matrices, or Q8_0 blocks in: the GEMV (the caller runs the
        // GEMM forms one matrix at a time on unpacked activations)
        const int per_lane = (a.nb + 15) / 16;
        if (per_lane <= 1) return launch_q40_maxp<1>(s, a);
        if (per_lane <= 2) return launch_q40_maxp<2>(s, a);
        if (per_lane <= 4) return launch_q40_maxp<4>(s, a);
        if (per_lane <= 6) return launch_q40_maxp<6>(s, a);
        return launch_q40_maxp<8>(s, a);
    }
    if (q40_gemm_form(a.rows, a.ntok)) {
        // split K with the caller's scratch where the form asks for it;
        // without scratch, wide projections take the GEMM unsplit and
        // narrow ones the GEMV
        Q40Args g = a;
        if (!q40_gemm_split(a.rows, a.ntok)) g.part = nullptr;
        if (g.part || a.rows >= kQ40GemmMinRows) return launch_q40_gemm(s, g);
    }
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
// Four outputs per thread; each group of four ranks' weights and results is
// loaded at once (a skipped rank's results are read and not used), then
// applied in rank order.  OUT16: the output is 16-byte aligned (else four
// dword stores).
template <bool OUT16>
__global__ __launch_bounds__(kWG) void k_combine(const float *__restrict__ results,
                                                 const float *__restrict__ weights, int topk,
                                                 int H, float *__restrict__ out) {
    const int i = 4 * (blockIdx.x * kWG + threadIdx.x), t = blockIdx.y;
    if (i >= H) return;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int r0 = 0; r0 < topk; r0 += 4) {
        float w[4];
        float4 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = min(r0 + j, topk - 1);
            w[j] = weights[t * topk + r];
            v[j] = *reinterpret_cast<const float4 *>(results + (size_t)(t * topk + r) * H + i);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (r0 + j >= topk || w[j] <= 0.0f) continue;
            o.x = __builtin_fmaf(v[j].x, w[j], o.x);
            o.y = __builtin_fmaf(v[j].y, w[j], o.y);
            o.z = __builtin_fmaf(v[j].z, w[j], o.z);
            o.w = __builtin_fmaf(v[j].w, w[j], o.w);
        }
    }
    float *d = out + (size_t)t * H + i;
    if constexpr (OUT16) {
        *reinterpret_cast<float4 *>(d) = o;
    } else {
        d[0] = o.x;
        d[1] = o.y;
        d[2] = o.z;
        d[3] = o.w;
    }
}

hipError_t launch_combine(hipStream_t s, const float *results, const float *weights, int batch,
                          int topk, int hidden, float *out) {
    if (hidden % 4 != 0) return hipErrorInvalidValue;  // hidden is a multiple of the 32-element block
    dim3 grid((hidden / 4 + kWG - 1) / kWG, batch);
    if ((reinterpret_cast<uintptr_t>(out) & 15u) == 0)
        hipLaunchKernelGGL(k_combine<true>, grid, dim3(kWG), 0, s, results, weights, topk, hidden, out);
    else
        hipLaunchKernelGGL(k_combine<false>, grid, dim3(kWG), 0, s, results, weights, topk, hidden, out);
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
