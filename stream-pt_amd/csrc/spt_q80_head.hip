// spt_q80_head.hip -- Q8_0 weights x fp32 activations for the LM head:
// forward.MulQ80Into and forward.MulQ80Argmax (forward/q80.go:20-148).
//
// The reference multiplies the fp32 activations directly (no Q8_0 of x).  Per
// row it keeps 32 accumulation chains -- chain e takes element e of every
// block, c_e = fma(float(q_e) * d, x[32b + e], c_e) over the blocks in order
// -- and ends with t_s = ((c_s + c_{8+s}) + c_{16+s}) + c_{24+s},
// p_i = t_i + t_{i+4}, y = (p_0 + p_1) + (p_2 + p_3) (quantQ80AVX2 and
// quantSumAVX2, forward/quant_amd64.go:92-116).  Here a half-wave takes a
// row, lane e owning chain e, so every row's bits equal the reference's.
// float(q) * d is exact (at most 8 x 11 significant bits, never subnormal);
// v_fma_mix_f32(q, d, -0.0) forms it from the fp16 bits in one instruction
// (adding -0.0 leaves every product, -0.0 included, unchanged).
//
// Memory: the matrix is read once, in chunks of whole consecutive rows (as
// many as fit in kChunkBytes) that a wave loads into its own LDS buffers by
// LDS DMA, kBufs - 1 chunks in flight while one is multiplied; x is staged
// once per workgroup in LDS.  Waves take chunks w, w + W, w + 2W, ... of the
// grid's W waves.  The argmax form keeps each wave's best (logit, row) and a
// one-workgroup pass merges them.
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunkInstr = 6;                    // 1 KiB LDS DMA loads per chunk
constexpr int kChunkBytes = 1024 * kChunkInstr;   // two rows of 2880 inputs (2 x 3060 + 15)
constexpr int kBufs = 3;
constexpr uint32_t kOOR = 0xFFFFFFF0u;            // an offset past every descriptor's range
constexpr int kUnroll = 8;
constexpr int kMaxChunkRows = 64;                 // a chunk's y values fit one store (one per lane)

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

}  // namespace

template <bool ARGMAX>
__global__ __launch_bounds__(kThreads) void k_q80_rows(Q80Args a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wl = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = blockIdx.x * kWaves + wl, nw = gridDim.x * kWaves;
    const int half = lane >> 5, e = lane & 31;
    const int nb = a.nb;
    const uint32_t rb = (uint32_t)nb * kQ80Block;
    const int R = a.rows_per_chunk;

    // x for the workgroup: x[32b + e] at 128b + 4e
    float *xs = reinterpret_cast<float *>(lds);
    for (int i = tid; i < 32 * nb; i += kThreads) xs[i] = a.x[i];
    uint8_t *bufs = lds + 128 * nb + wl * (kBufs * kChunkBytes);

    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t buf0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)bufs);
    const uintptr_t wb = reinterpret_cast<uintptr_t>(a.w);
    const uint32_t le = (uint32_t)(wb & 15u);
    const u32x4v rs = rsrc_words(reinterpret_cast<const void *>(wb - le), (uint32_t)((a.nbytes + le + 15u) & ~15ull));
    const int mine = gw < a.chunks ? (a.chunks - gw + nw - 1) / nw : 0;

    // chunk c's rows [c*R, c*R + R) as 16-byte pieces from the boundary at
    // or below their first byte; pieces at or past the rows' end are not read
    auto issue = [&](int i) {
        const int c = gw + i * nw;
        const uint32_t start = le + (uint32_t)c * (uint32_t)R * rb;
        const uint32_t end = le + (uint32_t)min((uint64_t)(c + 1) * (uint64_t)R * rb, a.nbytes);
        const uint32_t base = start & ~15u;
        const uint32_t buf = buf0 + (uint32_t)(i % kBufs) * kChunkBytes;
#pragma unroll
        for (int k = 0; k < kChunkInstr; k++) {
            const uint32_t off = base + 16u * (uint32_t)(64 * k + lane);
            dma16(rs, buf + 1024u * (uint32_t)k, off < end ? off : kOOR, 0u);
        }
    };
    for (int i = 0; i < kBufs - 1 && i < mine; i++) issue(i);
    __syncthreads();  // x staged

    const float nz = -0.0f;
    float best_v = -__builtin_inff();
    int best_i = 0;
    for (int i = 0; i < mine; i++) {
        // Wait for chunk i.  Memory operations complete in issue order for
        // the counter, so the wait names how many may stay outstanding:
        // the later chunks' loads and, for y, the one store of each earlier
        // chunk that was issued after chunk i's loads (chunks i-2 and i-1).
        if (i + kBufs - 1 < mine) {
            issue(i + kBufs - 1);
            constexpr int kLater = (kBufs - 1) * kChunkInstr;
            static_assert(kBufs == 3, "the store counts below assume two chunks in flight");
            if (ARGMAX || i == 0)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLater) : "memory");
            else if (i == 1)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLater + 1) : "memory");
            else
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLater + 2) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const int c = gw + i * nw;
        const int r0 = c * R, nr = min(R, a.rows - r0);
        const uint8_t *cb = bufs + (i % kBufs) * kChunkBytes + ((le + (uint32_t)r0 * rb) & 15u);
        float yv = 0.0f;  // lane j: row r0 + j
        for (int p = 0; p < nr; p += 2) {
            const int rr = p + half;
            const uint8_t *rowp = cb + (rr < nr ? rr : p) * rb;
            const int8_t *qp = reinterpret_cast<const int8_t *>(rowp + 2 + e);
            const uint16_t *dp = reinterpret_cast<const uint16_t *>(rowp);
            const float *xp = xs + e;
            float acc = 0.0f;
            int b = 0;
            for (; b + kUnroll <= nb; b += kUnroll) {
#pragma unroll
                for (int j = 0; j < kUnroll; j++) {
                    const float w = q80_weight(qp[kQ80Block * (b + j)], dp[(kQ80Block / 2) * (b + j)], nz);
                    acc = __builtin_fmaf(w, xp[32 * (b + j)], acc);
                }
            }
            for (; b < nb; b++) {
                const float w = q80_weight(qp[kQ80Block * b], dp[(kQ80Block / 2) * b], nz);
                acc = __builtin_fmaf(w, xp[32 * b], acc);
            }
            // chains e, e+8, e+16, e+24 -> t_e (e < 8); then the pairwise sum
            const float c8 = __shfl_down(acc, 8, 32), c16 = __shfl_down(acc, 16, 32), c24 = __shfl_down(acc, 24, 32);
            const float t = ((acc + c8) + c16) + c24;
            const float pr = t + __shfl_down(t, 4, 32);
            const float qd = pr + __shfl_down(pr, 1, 32);
            const float y = qd + __shfl_down(qd, 2, 32);
            const float y0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, y), 0));
            const float y1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, y), 32));
            if constexpr (ARGMAX) {
                argmax_take(y0, r0 + p, best_v, best_i);
                if (p + 1 < nr) argmax_take(y1, r0 + p + 1, best_v, best_i);
            } else {
                yv = lane == p ? y0 : yv;
                yv = lane == p + 1 ? y1 : yv;
            }
        }
        if constexpr (!ARGMAX) {
            if (lane < nr) a.y[r0 + lane] = yv;
        }
    }
    if constexpr (ARGMAX) {
        if (lane == 0) {
            a.part_v[gw] = best_v;
            a.part_i[gw] = best_i;
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

static int q80_rows_per_chunk(int nb) {
    const int rb = nb * kQ80Block;
    return min(kMaxChunkRows, (kChunkBytes - 15) / rb);
}

int q80_grid_waves(int rows, int nb, int n_cu) {
    const int chunks = (rows + q80_rows_per_chunk(nb) - 1) / q80_rows_per_chunk(nb);
    const int wgs = min((chunks + kWaves - 1) / kWaves, max(n_cu, 1));
    return wgs * kWaves;
}

hipError_t launch_q80_rows(hipStream_t s, const Q80Args &a0, int n_cu) {
    if (a0.nb < 1 || a0.nb > kQ80MaxBlocks || a0.rows < 1) return hipErrorInvalidValue;
    Q80Args a = a0;
    a.rows_per_chunk = q80_rows_per_chunk(a.nb);
    a.chunks = (a.rows + a.rows_per_chunk - 1) / a.rows_per_chunk;
    const int waves = q80_grid_waves(a.rows, a.nb, n_cu);
    constexpr size_t kMaxLds = (size_t)128 * kQ80MaxBlocks + (size_t)kWaves * kBufs * kChunkBytes;
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
    const size_t lds = (size_t)128 * a.nb + (size_t)kWaves * kBufs * kChunkBytes;
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
