// spt_q80_head.hip -- Q8_0 weights x fp32 activations for the LM head:
// forward.MulQ80Into and forward.MulQ80Argmax (forward/q80.go:20-148).
//
// The reference multiplies the fp32 activations directly (no Q8_0 of x).  Per
// row it keeps 32 accumulation chains -- chain e takes element e of every
// block, c_e = fma(float(q_e) * d, x[32b + e], c_e) over the blocks in order
// -- and ends with t_s = ((c_s + c_{8+s}) + c_{16+s}) + c_{24+s},
// p_i = t_i + t_{i+4}, y = (p_0 + p_1) + (p_2 + p_3) (quantQ80AVX2 and
// quantSumAVX2, forward/quant_amd64.go:92-116).  Here 8 lanes take a row,
// lane j owning chains 4j .. 4j+3 (per block: two code pairs, one fp16 scale
// and one float4 of x), so every row's bits equal the reference's.
// float(q) * d is exact (at most 8 x 11 significant bits, never subnormal);
// v_fma_mix_f32(q, d, -0.0) forms it from the fp16 bits in one instruction
// (adding -0.0 leaves every product, -0.0 included, unchanged).
//
// Memory: the matrix is read once.  A wave takes tiles of 16 consecutive
// rows (tiles w, w + W, ... of the grid's W waves) and walks each tile's K
// in segments of kSeg blocks; a segment's 16 row windows are loaded into the
// wave's own LDS stage by LDS DMA, kBufs - 1 segments in flight while one is
// multiplied.  x is staged once per workgroup in LDS.  The argmax form keeps
// each wave's best (logit, row) and a one-workgroup pass merges them.
//
// Ten waves per workgroup, one segment in flight each: a compute unit's
// memory queue holds about 48 KB of loads, and a wave whose load finds it
// full stalls at the issue instead of multiplying, so 10 x 6 KB in flight
// keeps the queue full with few stalls (eight waves with two segments in
// flight each: 126.9 us for the 201,088 x 2,880 head; one each: 124.5 us).
// Ten waves also split that head's 12,568 tiles almost evenly (at most 5
// per wave against 4.91 on average; with 8, 9, 11 or 12 waves the slowest
// waves take 7, 6, 5 or 5 against 6.14, 5.45, 4.46 or 4.09): 121.5 us, and
// 133.6, 128.3 and 132.3 us with 9, 11 and 12 waves.
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

constexpr int kWaves = 10;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerLane = 2;                                       // rows rg and rg + 8 share x reads
constexpr int kTileRows = 8 * kRowsPerLane;                           // 8 lanes per row
constexpr int kSeg = 9;                                               // blocks per K segment (90 = 10 x 9)
constexpr int kPieces = (15 + kSeg * kQ80Block + 15) / 16;            // 16-byte loads per row window
constexpr int kSlot = 16 * kPieces;                                   // LDS bytes per row in a stage
constexpr int kSegInstr = (kTileRows * kPieces + 63) / 64;            // LDS DMA loads per segment
constexpr int kStageBytes = 1024 * kSegInstr;
constexpr int kBufs = 2;
constexpr int kGroup = 3;                                             // blocks per LDS read group
constexpr uint32_t kOOR = 0xFFFFFFF0u;                                // past every descriptor's range
static_assert(kSeg % kGroup == 0, "segment of whole groups");
static_assert(kBufs - 1 <= 3, "the store count of the wait covers three units");

// float(q) * fp16(dbits) exactly.
__device__ __attribute__((always_inline)) inline float q80_weight(int q, uint32_t dbits, float neg_zero) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"((float)q), "v"(dbits), "v"(neg_zero));
    return r;
}

// (v, i) replaces (bv, bi) when it is larger, or equal with a lower row: the
// merge rule of forward/q80.go:70-78,93-99 (NaN never replaces anything).
__device__ __attribute__((always_inline)) inline void argmax_take(float v, int i, float &bv, int &bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// One block of a lane's four chains: codes 4j, 4j+1 in qa, 4j+2, 4j+3 in qb.
__device__ __attribute__((always_inline)) inline void q80_block(uint32_t qa, uint32_t qb, uint32_t d, float4 x,
                                                                float nz, float (&c)[4]) {
    c[0] = __builtin_fmaf(q80_weight((int)(int8_t)(qa & 0xFFu), d, nz), x.x, c[0]);
    c[1] = __builtin_fmaf(q80_weight((int)(int8_t)(qa >> 8), d, nz), x.y, c[1]);
    c[2] = __builtin_fmaf(q80_weight((int)(int8_t)(qb & 0xFFu), d, nz), x.z, c[2]);
    c[3] = __builtin_fmaf(q80_weight((int)(int8_t)(qb >> 8), d, nz), x.w, c[3]);
}

struct Q80Grp {
    uint32_t qa[kRowsPerLane][kGroup], qb[kRowsPerLane][kGroup], d[kRowsPerLane][kGroup];
    float4 x[kGroup];
};

// A full segment for the lane's rows: kSeg / kGroup groups, each group's LDS
// reads issued while the previous group is multiplied (two register sets,
// no copies); one read of x serves every row.
__device__ __attribute__((always_inline)) inline void q80_segment(const uint16_t *const (&qp)[kRowsPerLane],
                                                                  const uint16_t *const (&dp)[kRowsPerLane],
                                                                  const float4 *xp, float nz,
                                                                  float (&c)[kRowsPerLane][4]) {
    constexpr int kNG = kSeg / kGroup;
    Q80Grp g[2];
    auto fetch = [&](int gi, Q80Grp &t) {
#pragma unroll
        for (int k = 0; k < kGroup; k++) {
            const int b = kGroup * gi + k;
#pragma unroll
            for (int r = 0; r < kRowsPerLane; r++) {
                t.qa[r][k] = qp[r][(kQ80Block / 2) * b];
                t.qb[r][k] = qp[r][(kQ80Block / 2) * b + 1];
                t.d[r][k] = dp[r][(kQ80Block / 2) * b];
            }
            t.x[k] = xp[8 * b];
        }
    };
    fetch(0, g[0]);
#pragma unroll
    for (int gi = 0; gi < kNG; gi++) {
        if (gi + 1 < kNG) fetch(gi + 1, g[(gi + 1) & 1]);
#pragma unroll
        for (int k = 0; k < kGroup; k++)
#pragma unroll
            for (int r = 0; r < kRowsPerLane; r++)
                q80_block(g[gi & 1].qa[r][k], g[gi & 1].qb[r][k], g[gi & 1].d[r][k], g[gi & 1].x[k], nz, c[r]);
    }
}

}  // namespace

template <bool ARGMAX>
__global__ __launch_bounds__(kThreads) void k_q80_rows(Q80Args a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wl = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = blockIdx.x * kWaves + wl, nw = gridDim.x * kWaves;
    const int rg = lane >> 3, j = lane & 7;  // rows rg + 8r of the tile, chain quad
    const int nb = a.nb, rows = a.rows;
    const uint32_t rb = (uint32_t)nb * kQ80Block;
    const int nseg = (nb + kSeg - 1) / kSeg;
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    const int units = gw < tiles ? ((tiles - gw + nw - 1) / nw) * nseg : 0;

    // x for the workgroup: x[32b + e] at 128b + 4e
    float *xs = reinterpret_cast<float *>(lds);
    for (int i = tid; i < 32 * nb; i += kThreads) xs[i] = a.x[i];
    uint8_t *stages = lds + 128 * nb + wl * (kBufs * kStageBytes);

    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t st0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)stages);
    const uintptr_t wb = reinterpret_cast<uintptr_t>(a.w);
    const uint32_t le = (uint32_t)(wb & 15u);
    const u32x4v rs = rsrc_words(reinterpret_cast<const void *>(wb - le), (uint32_t)((a.nbytes + le + 15u) & ~15ull));

    // this lane's pieces: load i covers piece (64i + lane) % kPieces of row
    // (64i + lane) / kPieces of the tile
    int prow[kSegInstr], pk[kSegInstr];
#pragma unroll
    for (int i = 0; i < kSegInstr; i++) {
        const int p = 64 * i + lane;
        prow[i] = p / kPieces;
        pk[i] = p - prow[i] * kPieces;
    }
    // Units are (tile, segment) pairs in order: segment sg of tile t, the
    // tiles gw, gw + nw, ...  A row's window starts at the 16-byte boundary
    // at or below its segment's first byte; pieces past the segment's end
    // are not read.  The issue position runs kBufs - 1 units ahead.
    int it = gw, isg = 0, iu = 0;
    auto issue = [&]() {
        const int t = it, sg = isg;
        const uint32_t seg0 = (uint32_t)(kSeg * kQ80Block) * (uint32_t)sg;
        const uint32_t seg1 = min(seg0 + (uint32_t)(kSeg * kQ80Block), rb);
        const uint32_t st = st0 + (uint32_t)(iu % kBufs) * kStageBytes;
        if (++isg == nseg) {
            isg = 0;
            it += nw;
        }
        iu++;
#pragma unroll
        for (int i = 0; i < kSegInstr; i++) {
            const int row = kTileRows * t + prow[i];
            const uint32_t rpos = le + (uint32_t)row * rb;
            const uint32_t off = ((rpos + seg0) & ~15u) + 16u * (uint32_t)pk[i];
            const bool ok = prow[i] < kTileRows && row < rows && off < rpos + seg1;
            dma16(rs, st + 1024u * (uint32_t)i, ok ? off : kOOR, 0u);
        }
    };
    for (int u = 0; u < kBufs - 1 && u < units; u++) issue();
    __syncthreads();  // x staged

    const float nz = -0.0f;
    float best_v = -__builtin_inff();
    int best_i = 0;
    float c[kRowsPerLane][4];  // chains 4j .. 4j+3 of rows rg + 8r
#pragma unroll
    for (int r = 0; r < kRowsPerLane; r++)
#pragma unroll
        for (int k = 0; k < 4; k++) c[r][k] = 0.0f;
    // y of MulQ80Into: lane kTileRows * k + i collects row i of the wave's
    // tile k of each group of kTilesPerStore; one store per group
    constexpr int kTilesPerStore = 64 / kTileRows;
    float yv = 0.0f;
    int yrow = -1;
    int t = gw, sg = 0, ti = 0;
    for (int u = 0; u < units; u++) {
        // Wait for unit u: with the kBufs - 1 later units' loads issued, at
        // most that many loads may stay outstanding.  Loads complete in
        // issue order, so this holds whether or not stores issued in between
        // have completed.
        if (u + kBufs - 1 < units) {
            issue();
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kBufs - 1) * kSegInstr) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const int b0 = kSeg * sg, jn = min(kSeg, nb - b0);
        const uint16_t *qp[kRowsPerLane];
        const uint16_t *dp[kRowsPerLane];
#pragma unroll
        for (int r = 0; r < kRowsPerLane; r++) {
            const int rl = rg + 8 * r;  // row within the tile
            const uint8_t *rowp = stages + (u % kBufs) * kStageBytes + kSlot * rl +
                                  ((le + (uint32_t)(kTileRows * t + rl) * rb + (uint32_t)(b0 * kQ80Block)) & 15u);
            qp[r] = reinterpret_cast<const uint16_t *>(rowp + 2 + 4 * j);
            dp[r] = reinterpret_cast<const uint16_t *>(rowp);
        }
        const float4 *xp = reinterpret_cast<const float4 *>(xs + 32 * b0) + j;
        if (jn == kSeg) {
            q80_segment(qp, dp, xp, nz, c);
        } else {
            for (int b = 0; b < jn; b++)
#pragma unroll
                for (int r = 0; r < kRowsPerLane; r++)
                    q80_block(qp[r][(kQ80Block / 2) * b], qp[r][(kQ80Block / 2) * b + 1], dp[r][(kQ80Block / 2) * b],
                              xp[8 * b], nz, c[r]);
        }
        if (sg == nseg - 1) {
#pragma unroll
            for (int r = 0; r < kRowsPerLane; r++) {
                // t_{4m+k} at lane m < 2 of the row: chains 4m+k + 8, 16, 24
                // sit in lanes m + 2, 4, 6; p_k = t_k + t_{k+4} (lanes 0 and 1)
                float pk4[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float tk =
                        ((c[r][k] + __shfl_down(c[r][k], 2, 8)) + __shfl_down(c[r][k], 4, 8)) + __shfl_down(c[r][k], 6, 8);
                    pk4[k] = tk + __shfl_down(tk, 1, 8);
                    c[r][k] = 0.0f;
                }
                const float y = (pk4[0] + pk4[1]) + (pk4[2] + pk4[3]);
                const int row = kTileRows * t + rg + 8 * r;
                if constexpr (ARGMAX) {
                    // lane 8i keeps the best of its rows across the wave's tiles
                    if (j == 0 && row < rows) argmax_take(y, row, best_v, best_i);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const float yr =
                            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, y), 8 * i));
                        const bool mine_r = lane == kTileRows * (ti % kTilesPerStore) + i + 8 * r;
                        yv = mine_r ? yr : yv;
                        yrow = mine_r ? kTileRows * t + i + 8 * r : yrow;
                    }
                }
            }
            if constexpr (!ARGMAX) {
                if (ti % kTilesPerStore == kTilesPerStore - 1 || u + 1 == units) {
                    if (yrow >= 0 && yrow < rows) a.y[yrow] = yv;
                    yrow = -1;
                }
            }
            ti++;
            t += nw;
        }
        if (++sg == nseg) sg = 0;
    }
    if constexpr (ARGMAX) {
        float bv = -__builtin_inff();
        int bi = 0;
#pragma unroll
        for (int r = 0; r < kTileRows; r++)
            argmax_take(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, best_v), 8 * r)),
                        __builtin_amdgcn_readlane(best_i, 8 * r), bv, bi);
        if (lane == 0) {
            a.part_v[gw] = bv;
            a.part_i[gw] = bi;
        }
    }
}

// One workgroup merges the per-wave results in the same rule.
__global__ __launch_bounds__(1024) void k_q80_argmax_merge(const float *part_v, const int32_t *part_i, int n,
                                                          float *out_v, int32_t *out_i) {
    __shared__ float sv[1024];
    __shared__ int si[1024];
    float bv = -__builtin_inff();
    int bi = 0;
    for (int k = threadIdx.x; k < n; k += 1024) argmax_take(part_v[k], part_i[k], bv, bi);
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 512; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            float v = sv[threadIdx.x];
            int i = si[threadIdx.x];
            argmax_take(sv[threadIdx.x + s], si[threadIdx.x + s], v, i);
            sv[threadIdx.x] = v;
            si[threadIdx.x] = i;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        *out_v = sv[0];
        *out_i = si[0];
    }
}

int q80_grid_waves(int rows, int nb, int n_cu) {
    (void)nb;
    const int tiles = (rows + kTileRows - 1) / kTileRows;
    const int wgs = min((tiles + kWaves - 1) / kWaves, max(n_cu, 1));
    return wgs * kWaves;
}

hipError_t launch_q80_rows(hipStream_t s, const Q80Args &a, int n_cu) {
    if (a.nb < 1 || a.nb > kQ80MaxBlocks || a.rows < 1) return hipErrorInvalidValue;
    constexpr size_t kMaxLds = (size_t)128 * kQ80MaxBlocks + (size_t)kWaves * kBufs * kStageBytes;
    static_assert(kMaxLds <= 160 * 1024, "LDS");
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_q80_rows<false>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_q80_rows<true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
        return e;
    }();
    if (attr != hipSuccess) return attr;
    const int waves = q80_grid_waves(a.rows, a.nb, n_cu);
    const size_t lds = (size_t)128 * a.nb + (size_t)kWaves * kBufs * kStageBytes;
    if (a.part_v) {
        hipLaunchKernelGGL(k_q80_rows<true>, dim3(waves / kWaves), dim3(kThreads), lds, s, a);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        hipLaunchKernelGGL(k_q80_argmax_merge, dim3(1), dim3(1024), 0, s, a.part_v, a.part_i, waves, a.out_v,
                           a.out_i);
    } else {
        hipLaunchKernelGGL(k_q80_rows<false>, dim3(waves / kWaves), dim3(kThreads), lds, s, a);
    }
    return hipGetLastError();
}

}  // namespace spt
