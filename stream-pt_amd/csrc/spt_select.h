// spt_select.h -- top-k selection of one token by one wavefront
// (selectMoEBatch, forward/moe_batch.go:305-342), shared by the selection
// kernels (spt_kernels.hip) and the decode gate/up kernel (spt_mx_decode.hip).
#pragma once

#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

// Largest of the wave's 64 values (every lane gets it); NaN operands lose
// (v_max_f32 returns the other operand), so the result is NaN only when all
// are.  DPP within rows of 16 (lane ^ 1, ^ 2, half-row and row mirrors), then
// the four row results through readlane.
__device__ __attribute__((always_inline)) inline float wave_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// selectMoEBatch (forward/moe_batch.go:305-342) for one token by one
// wavefront: k rounds of a strict '>' scan where the lowest index wins ties,
// NaN and -Inf never win and picked experts are excluded.  Lane L owns
// experts L, L+64, ...; excluded experts (picked, or past E) hold NaN.  A
// round takes the largest value m (NaN candidates lose), and if m > -Inf the
// lowest expert holding a value equal to m (ballots by slot; -0 and +0 tie,
// as under '>'); otherwise nothing is selectable and the round falls back to
// Index = round, logit 0.  Then the softmax
// over the k logits: w = f32(exp(f64(l - max))) (lane r computes rank r's),
// summed in f32 in rank order, scaled by 1/sum when sum > 0.  Results go to
// LDS (s_ids/s_w, the token's k slots) and to global ids/weights.
struct TokenLogits {
    float v[kMaxExperts / 64];
};

// Lane L's logits of a token (experts L, L+64, ...; NaN past E).
__device__ inline TokenLogits load_token_logits(const float *lg, int E) {
    const int lane = threadIdx.x & 63;
    TokenLogits tl;
#pragma unroll
    for (int i = 0; i < kMaxExperts / 64; i++) {
        const int ex = lane + 64 * i;
        tl.v[i] = ex < E ? lg[ex] : __builtin_nanf("");
    }
    return tl;
}

__device__ void select_token(TokenLogits tl, int E, int k, int32_t *ids, float *weights,
                             int32_t *s_ids, float *s_w) {
    const int lane = threadIdx.x & 63;
    const float qnan = __builtin_nanf("");
    float *v = tl.v;
    const int nslot = (E + 63) / 64;
    int my_id = 0;
    float my_val = 0.0f;
    for (int r = 0; r < k; r++) {
        float lm = qnan;
#pragma unroll
        for (int i = 0; i < kMaxExperts / 64; i++) lm = fmaxf(lm, v[i]);
        const float m = wave_max(lm);
        int bi = r;
        float bv = 0.0f;
        if (m > -__builtin_inff()) {
            bv = m;
#pragma unroll
            for (int i = 0; i < kMaxExperts / 64; i++) {
                if (i >= nslot) break;
                const uint64_t hit = __ballot(v[i] == m);
                if (hit) {
                    bi = 64 * i + __builtin_ctzll(hit);
                    break;
                }
            }
        }
        // exclude the pick (in the fallback, expert `round`)
#pragma unroll
        for (int i = 0; i < kMaxExperts / 64; i++)
            if (bi == lane + 64 * i) v[i] = qnan;
        if (lane == r) {
            my_id = bi;
            my_val = bv;
        }
    }
    // max over ranks in order (NaN never replaces: strict '>')
    float mx = -__builtin_inff();
    for (int r = 0; r < k; r++) {
        const float l = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_val), r));
        if (l > mx) mx = l;
    }
    const float e = lane < k ? static_cast<float>(exp(static_cast<double>(my_val - mx))) : 0.0f;
    float sum = 0.0f;
    for (int r = 0; r < k; r++) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), r));
    if (lane < k) {
        const float w = sum > 0.0f ? e * (1.0f / sum) : e;
        if (s_ids) {
            s_ids[lane] = my_id;
            s_w[lane] = w;
        }
        ids[lane] = my_id;
        weights[lane] = w;
    }
}

}  // namespace spt
