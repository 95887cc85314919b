// spt_rmsnorm.hip -- RMSNorm of activation rows, fused with the Q8_0 of its
// output: forward.RMSNormInto (forward/rmsnorm.go:19-167) and normBatch
// (forward/layer_batch.go:139-195), the step upstream of the MoE and Q4_0
// operators.
//
// The sum of squares follows the reference's lane order for an 8-float simd
// width (the AVX2 build): RMSNormInto keeps four accumulators over 32-element
// chunks -- 32 FMA chains, chain c taking elements 32k + c -- combined
// ((a0 + a1) + a2) + a3, then 8-element chunks (the last zero-filled);
// normBatch keeps one 8-lane accumulator over 8-element chunks.  The eight
// lanes are summed in order, factor = 1 / float32(sqrt(float64(sum / n +
// eps))) and y = (x * w) * factor, so y matches the reference's bits.  The
// Q8_0 of y (GGML blocks, the quantizer of spt_quantize_q8_0) is formed from
// the same registers.  One workgroup per row (16 waves while the rows fit
// one per compute unit, else 8): where the row fits
// (kStageMax elements) the whole workgroup stages it and the norm weights in
// LDS (as fp32, kStageBatch loads per thread in flight), else the chains and
// the output read global memory; the chains run in one wave with the next
// kChainBatch chunks in flight ahead of their FMAs; the waves then share
// the y / Q8_0 blocks, so each takes few of them once the factor is known.
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

constexpr int kWide = 1024;   // threads of a row's workgroup up to one row per compute unit
constexpr int kNarrow = 512;  // and above
constexpr int kStageMax = 8192;  // elements of a row staged in LDS (row and weights: 64 KB)
constexpr int kStageBatch = 8;   // staged elements a thread loads ahead at once
constexpr int kChainBatch = 32;  // chunks of a chain loaded at once

__device__ __attribute__((always_inline)) inline float norm_weight(const void *w, int type, int i) {
    if (type == 0) return reinterpret_cast<const float *>(w)[i];
    const uint32_t h = reinterpret_cast<const uint16_t *>(w)[i];
    return type == 1 ? f16_bits_to_f32(h) : __uint_as_float(h << 16);
}

__device__ __attribute__((always_inline)) inline float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// acc = fma(v, v, acc) over xr[stride * k + c] for k = 0 .. full - 1 in
// order (one lane's chain), the loads of the next kChainBatch chunks in
// flight while the current kChainBatch are accumulated.
__device__ __attribute__((always_inline)) inline float sumsq_chain(const float *xr, int stride, int c, int full) {
    constexpr int U = kChainBatch;
    float acc = 0.0f;
    int k = 0;
    if (full >= U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = xr[stride * u + c];
#pragma unroll 2
        for (; k + 2 * U <= full; k += U) {
            float nx[U];
#pragma unroll
            for (int u = 0; u < U; u++) nx[u] = xr[stride * (k + U + u) + c];
#pragma unroll
            for (int u = 0; u < U; u++) acc = __builtin_fmaf(v[u], v[u], acc);
#pragma unroll
            for (int u = 0; u < U; u++) v[u] = nx[u];
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc = __builtin_fmaf(v[u], v[u], acc);
        k += U;
    }
    for (; k < full; k++) {
        const float v = xr[stride * k + c];
        acc = __builtin_fmaf(v, v, acc);
    }
    return acc;
}

}  // namespace

template <bool BATCH_ORDER, bool STAGED, int T>
__global__ __launch_bounds__(T) void k_rmsnorm(RmsArgs a) {
    __shared__ float s_factor;
    extern __shared__ float s_row[];  // staged: the row, then the weights as fp32
    const int tid = threadIdx.x, lane = tid & 63;
    const int n = a.n;
    const float *x = a.x + (size_t)blockIdx.x * n;
    const float *xr = x;  // where the chains read the row
    float *sw = nullptr;  // the staged weights
    if constexpr (STAGED) {
        sw = s_row + n;
        for (int i0 = tid; i0 < n; i0 += kStageBatch * T) {
            float xv[kStageBatch], wv[kStageBatch];
#pragma unroll
            for (int u = 0; u < kStageBatch; u++) {
                const int i = min(i0 + u * T, n - 1);
                xv[u] = x[i];
                wv[u] = norm_weight(a.w, a.wtype, i);
            }
#pragma unroll
            for (int u = 0; u < kStageBatch; u++) {
                const int i = i0 + u * T;
                if (i < n) {
                    s_row[i] = xv[u];
                    sw[i] = wv[u];
                }
            }
        }
        __syncthreads();
        xr = s_row;
    }
    auto weight = [&](int i) { return STAGED ? sw[i] : norm_weight(a.w, a.wtype, i); };
    if (tid < 64) {
        float lanes8;  // lane s < 8: the simd lane s of the reference's accumulator
        if constexpr (!BATCH_ORDER) {
            const int c = lane & 31;
            const int full = n / 32;
            const float acc = sumsq_chain(xr, 32, c, full);
            lanes8 = ((acc + __shfl_down(acc, 8, 32)) + __shfl_down(acc, 16, 32)) + __shfl_down(acc, 24, 32);
            for (int off = 32 * full; off < n; off += 8) {
                const float v = (lane < 8 && off + lane < n) ? xr[off + lane] : 0.0f;
                lanes8 = __builtin_fmaf(v, v, lanes8);
            }
        } else {
            const int full = n / 8;
            float acc = sumsq_chain(xr, 8, lane & 7, full);
            if (8 * full < n) {
                const float v = (lane < 8 && 8 * full + lane < n) ? xr[8 * full + lane] : 0.0f;
                acc = __builtin_fmaf(v, v, acc);
            }
            lanes8 = acc;
        }
        float sum = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; s++) sum += lane_f(lanes8, s);
        if (tid == 0) s_factor = 1.0f / (float)__builtin_sqrt((double)(sum / (float)n + a.eps));
    }
    __syncthreads();  // factor known; every read of x for the sum is done (y may alias x)
    const float factor = s_factor;
    float *y = a.y ? a.y + (size_t)blockIdx.x * n : nullptr;
    if (a.q8) {
        // wave w takes block pairs 2w, 2w + 8, ...; half-wave h the block
        // 2w + h of the pair, element lane & 31 (whole waves iterate
        // together: the quantizer reduces across each half-wave)
        const int wv = tid >> 6, h = lane >> 5, e = lane & 31;
        const int nblk = n / 32;
        for (int b0 = 2 * wv; b0 < nblk; b0 += 2 * (T / 64)) {
            const int b = b0 + h;
            const bool ok = b < nblk;
            const int i = 32 * b + e;
            const float v = ok ? (xr[i] * weight(i)) * factor : 0.0f;
            if (ok && y) y[i] = v;
            uint16_t dh;
            const int q = q8_quantize_half(v, lane, &dh);
            if (ok) write_q8_lane(q, dh, e, (size_t)blockIdx.x * nblk + b, nullptr, nullptr, nullptr, a.q8);
        }
    } else {
        for (int i = tid; i < n; i += T) y[i] = (xr[i] * weight(i)) * factor;
    }
}

hipError_t launch_rmsnorm(hipStream_t s, const RmsArgs &a, bool batch_order) {
    if (a.n <= 0 || a.batch <= 0) return hipSuccess;
    if (a.q8 && a.n % 32 != 0) return hipErrorInvalidValue;
    if (!a.q8 && !a.y) return hipErrorInvalidValue;
    const bool staged = a.n <= kStageMax;
    const size_t lds = staged ? (size_t)a.n * 8 : 0;
    // a workgroup of 16 waves per row while the rows fit one per compute
    // unit; 8 waves above that, so that two rows share a compute unit
    const bool wide = a.batch <= device_cus();
    auto go = [&](auto kern, int threads) { hipLaunchKernelGGL(kern, dim3(a.batch), dim3(threads), lds, s, a); };
    if (batch_order) {
        if (staged)
            wide ? go(k_rmsnorm<true, true, kWide>, kWide) : go(k_rmsnorm<true, true, kNarrow>, kNarrow);
        else
            wide ? go(k_rmsnorm<true, false, kWide>, kWide) : go(k_rmsnorm<true, false, kNarrow>, kNarrow);
    } else {
        if (staged)
            wide ? go(k_rmsnorm<false, true, kWide>, kWide) : go(k_rmsnorm<false, true, kNarrow>, kNarrow);
        else
            wide ? go(k_rmsnorm<false, false, kWide>, kWide) : go(k_rmsnorm<false, false, kNarrow>, kNarrow);
    }
    return hipGetLastError();
}

}  // namespace spt
