// Q4_0 x Q8_0 projections of a few tokens in one launch: MulQ40Into
// (forward/layer.go:120-165) and MulQ40BatchInto (forward/layer_batch.go:
// 68-100) for batches of up to kQ40DecTokens, including the fused Q/K/V
// call.  At these sizes a projection is a few megabytes of weights and the
// time goes to latency, so the kernel issues every load it will need at
// its start, the activations' first and then the weight blocks, and
// quantizes the activations (from fp32, by the rule of k_quantize) or
// unpacks their GGML Q8_0 blocks while the weights are in flight; one
// LDS-only barrier separates that staging from the dot products.
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {
namespace {

// A wavefront per output row, WG / 64 rows per workgroup: 1024 threads when
// the workgroup quantizes fp32 activations (one staging pass over up to 128
// blocks), 256 on GGML Q8_0 input (whose staging is a copy), so that the
// rows spread over four or five workgroups per CU.
constexpr int kDecWGQuant = 1024;
constexpr int kDecWGBlocks = 256;
constexpr uint32_t kNoLoad = 0x80000000u;  // past every view here: the load reads zeros

// Largest value over each group of 8 lanes of non-negative non-NaN floats
// given as bit patterns (which order like the values): DPP half-row mirror
// (lane ^ 7), then lane ^ 1 and lane ^ 2.
__device__ __attribute__((always_inline)) inline uint32_t max8_bits(uint32_t m) {
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));
    return m;
}

// Q8_0 of a block of 32 held four consecutive elements per lane by an
// aligned group of 8 lanes: the element arithmetic of q8_quantize_half
// (d = amax of the non-NaN |x| / 127, NaN when any element is NaN, codes
// roundf(x * (1/d)) clamped to [-127, 127], a NaN product giving 0), so the
// codes and the fp16 scale are the same bits.  Returns the four codes
// packed in element order.
__device__ __attribute__((always_inline)) inline uint32_t q8_quantize_quad(const float v[4], int lane,
                                                                           uint16_t *dbits) {
    uint32_t m = 0;
    bool nan = false;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float a = __builtin_fabsf(v[k]);
        nan |= (a != a);
        m = max(m, a == a ? __float_as_uint(a) : 0u);
    }
    const uint64_t nm = __ballot(nan);
    const bool nan_any = ((nm >> (lane & 56)) & 0xFFull) != 0;
    const float amax = __uint_as_float(max8_bits(m));
    const float d = nan_any ? __builtin_nanf("") : amax / 127.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    *dbits = f32_to_f16_bits(d);
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float r = __builtin_roundf(v[k] * id);
        const int q = (r != r) ? 0 : (r > 127.0f ? 127 : (r < -127.0f ? -127 : (int)r));
        w |= (uint32_t)(q & 0xff) << (8 * k);
    }
    return w;
}

// Sum over the 64 lanes, the same in every lane: within rows of 16 by DPP
// (lane ^ 1, ^ 2, then the half-row and row mirrors), then the four rows in
// order.
__device__ __attribute__((always_inline)) inline float wave_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return ((r0 + r1) + r2) + r3;
}

// The matrix of row tile `tile` of a call over up to three matrices
// (Q40Args::more), chosen by selects over fields all read up front, so that
// the kernel arguments arrive in one round trip.
__device__ __attribute__((always_inline)) inline Q40Args dec_matrix(const Q40Args &args, int *tile, int per_tile) {
    const Q40Mat m0 = args.more[0], m1 = args.more[1];
    const int t0 = (args.rows + per_tile - 1) / per_tile;
    const int t1 = args.nmore > 0 ? (m0.rows + per_tile - 1) / per_tile : 0;
    const bool s1 = *tile >= t0 && *tile < t0 + t1, s2 = *tile >= t0 + t1;
    Q40Args a = args;
    a.w = s2 ? m1.w : (s1 ? m0.w : args.w);
    a.nbytes = s2 ? m1.nbytes : (s1 ? m0.nbytes : args.nbytes);
    a.rows = s2 ? m1.rows : (s1 ? m0.rows : args.rows);
    a.y = s2 ? m1.y : (s1 ? m0.y : args.y);
    a.bias = s2 ? m1.bias : (s1 ? m0.bias : args.bias);
    a.bias_type = s2 ? m1.bias_type : (s1 ? m0.bias_type : args.bias_type);
    a.resid = s2 ? m1.resid : (s1 ? m0.resid : args.resid);
    *tile -= s2 ? t0 + t1 : (s1 ? t0 : 0);
    return a;
}

// Row tile blockIdx.x (of every matrix of the call) of kRows rows,
// wavefront g taking row kRows x + g, lane j its blocks j, j + 64 (MAXP of
// them at most), for NT token slots (ntok <= NT).  The activations' blocks
// are staged by the whole workgroup, kStagePass per pass: block
// i = tid / 8 + kStagePass p, part tid % 8 (four fp32 elements, or code word
// c of a GGML block).
template <int MAXP, int NT, bool F32>
__global__ __launch_bounds__(F32 ? kDecWGQuant : kDecWGBlocks) void k_q40_dec(Q40Args args) {
    constexpr int kWG = F32 ? kDecWGQuant : kDecWGBlocks;
    constexpr int kRows = kWG / 64, kStagePass = kWG / 8;
    constexpr int kBlocks = NT * 64 * MAXP;  // >= ntok * nb, and every index t * nb + b below
    constexpr int kPasses = (kBlocks + kStagePass - 1) / kStagePass;
    __shared__ __attribute__((aligned(16))) uint32_t s_codes[kBlocks * 8];
    __shared__ float s_scales[kBlocks];
    int tile = blockIdx.x;
    const Q40Args a = dec_matrix(args, &tile, kRows);
    const int nb = a.nb, tid = threadIdx.x, lane = tid & 63, c = tid & 7;
    const int nx = a.ntok * nb;

    // 1. the activations
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const ByteView xv = F32 ? make_view(a.xf, (uint64_t)nx * 128) : make_view(a.xq34, (uint64_t)nx * kQ80Block);
    u32x4 xf[F32 ? kPasses : 1];
    u32x2 xq[F32 ? 1 : kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; p++) {
        const int i = (tid >> 3) + kStagePass * p;
        if constexpr (F32) {
            const uint32_t off = i < nx ? (uint32_t)i * 128u + 16u * c : kNoLoad;
            xf[p] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xv.r, off, 0, 0));
        } else {
            const uint32_t off = i < nx ? ((uint32_t)i * kQ80Block + xv.lead + 4u * c) & ~3u : kNoLoad;
            xq[p] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(xv.r, off, 0, 0));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the weight blocks
    const int j = lane, g = tid >> 6;
    const int r = tile * kRows + g;
    const bool row_ok = r < a.rows;  // uniform over the wavefront
    const ByteView wv = make_view(a.w, a.nbytes);
    const uint32_t row_pos = (uint32_t)(row_ok ? r : 0) * (uint32_t)(nb * kQ40Block);
    uint32_t raw[MAXP][5], off[MAXP];
#pragma unroll
    for (int p = 0; p < MAXP; p++) {
        const int b = j + 64 * p;
        const bool ok = row_ok && b < nb;
        load_block5(wv, ok ? row_pos + (uint32_t)b * kQ40Block : kNoLoad, raw[p], &off[p]);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. activations -> LDS: code words [block][8], widened fp16 scales
#pragma unroll
    for (int p = 0; p < kPasses; p++) {
        const int i = (tid >> 3) + kStagePass * p;
        uint32_t w;
        uint16_t dh;
        if constexpr (F32) {
            float v[4] = {__uint_as_float(xf[p].x), __uint_as_float(xf[p].y), __uint_as_float(xf[p].z),
                          __uint_as_float(xf[p].w)};
            w = q8_quantize_quad(v, lane, &dh);  // every lane takes part (cross-lane steps)
        } else {
            const uint32_t o = ((uint32_t)i * kQ80Block + xv.lead) & 3u;  // 0 or 2
            w = __builtin_amdgcn_perm(xq[p].y, xq[p].x, 0x05040302u + o * 0x01010101u);
            dh = (uint16_t)__builtin_amdgcn_ubfe(xq[p].x, o * 8u, 16u);
        }
        if (i < nx) {
            s_codes[i * 8 + c] = w;
            if (c == 0) s_scales[i] = f16_bits_to_f32(dh);
        }
    }
    lds_barrier();

    // 4. dot products: per block sum over (n - 8) * q by sdot4 (q40_isum),
    // times d_w * d_x, accumulated by fmaf over the lane's blocks in order
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = 0.0f;
#pragma unroll
    for (int p = 0; p < MAXP; p++) {
        const int b = j + 64 * p;
        const bool ok = row_ok && b < nb;
        Q40Decoded dec;
        q40_decode(raw[p], off[p], dec);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int i = t * nb + b;  // < kBlocks; slots past ntok or b read unused LDS words
            const uint4 *q4 = reinterpret_cast<const uint4 *>(s_codes + i * 8);
            const uint4 qa = q4[0], qb = q4[1];
            const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
            int32_t sq = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) sq = __builtin_amdgcn_sdot4((int)q[k], 0x01010101, sq, false);
            const int32_t s = q40_isum(dec, q, sq);
            const float nv = __builtin_fmaf((float)s, dec.d * s_scales[i], acc[t]);
            acc[t] = ok ? nv : acc[t];
        }
    }
    if (!row_ok) return;  // whole wavefronts; no barrier follows
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float v = wave_sum(acc[t]);
        if (lane == 0 && t < a.ntok) q40_store(a, (size_t)t * a.rows + r, r, v);
    }
}

int row_tiles(const Q40Args &a, int per_tile) {
    int tiles = (a.rows + per_tile - 1) / per_tile;
    for (int i = 0; i < a.nmore; i++) tiles += (a.more[i].rows + per_tile - 1) / per_tile;
    return tiles;
}

template <int MAXP, int NT>
hipError_t launch_nt(hipStream_t s, const Q40Args &a) {
    if (a.xf)
        hipLaunchKernelGGL((k_q40_dec<MAXP, NT, true>), dim3(row_tiles(a, kDecWGQuant / 64)), dim3(kDecWGQuant), 0,
                           s, a);
    else
        hipLaunchKernelGGL((k_q40_dec<MAXP, NT, false>), dim3(row_tiles(a, kDecWGBlocks / 64)), dim3(kDecWGBlocks),
                           0, s, a);
    return hipGetLastError();
}

template <int MAXP>
hipError_t launch_maxp(hipStream_t s, const Q40Args &a) {
    if (a.ntok == 1) return launch_nt<MAXP, 1>(s, a);
    if (a.ntok == 2) return launch_nt<MAXP, 2>(s, a);
    return launch_nt<MAXP, 4>(s, a);
}

}  // namespace

hipError_t launch_q40_dec(hipStream_t s, const Q40Args &a) {
    if (a.rows <= 0 || a.ntok <= 0) return hipSuccess;
    if (!q40_dec_form(a.ntok, a.nb) || a.nb < 1 || (a.xf == nullptr) == (a.xq34 == nullptr) || a.nmore < 0 ||
        a.nmore > 2 || a.nbytes >= kQ40DecMaxBytes)
        return hipErrorInvalidValue;
    for (int i = 0; i < a.nmore; i++)
        if (a.more[i].nbytes >= kQ40DecMaxBytes || a.more[i].rows <= 0) return hipErrorInvalidValue;
    return a.nb <= 64 ? launch_maxp<1>(s, a) : launch_maxp<2>(s, a);
}

}  // namespace spt
