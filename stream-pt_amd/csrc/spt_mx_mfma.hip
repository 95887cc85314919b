// spt_mx_mfma.hip -- grouped MXFP4 x Q8_0 GEMV on the gfx950 block-scaled MFMA.
//
// v_mfma_scale_f32_16x16x128_f8f6f4 with A = E2M1 (the MXFP4 weights, fed as
// stored) and B = FP8 E4M3.  Lane layout (measured on the hardware):
//   A: lane 16*g + r holds row r, K-block g: the 16 nibble bytes of one GGUF
//      MXFP4 block in file order; its scale operand is that block's E8M0 byte.
//   B: lane 16*g + c holds column c; byte j (0..31) pairs with A K-block
//      (g>>1) + 2*(j>=16), nibble p = (j&15) + 16*(g&1); the B scale of
//      (column c, K-block g) is taken from lane 16*g + c.
//   D: lane 16*g + c holds D[4g+i][c], i = 0..3.
// A Q8_0 code q (int8) is split exactly into two E4M3 digits q = 16*h + l,
// h in [-8,7], l in [0,15].  Each MFMA covers 4 consecutive MXFP4 blocks of
// 16 rows; its 16 B columns are block-diagonal: column c = 8*slot + 4*part + g
// carries digit `part` (h with B scale 2^4, l with 2^0) of token `slot`'s
// block g, zero elsewhere.  So D[r][c] = 2^(e-127) * 2^(4 or 0) * sum(E2M1*digit)
// exactly, and D[r][g] + D[r][g+4] = 2^(e-127) * sum(E2M1*q) exactly: the same
// value as the integer form isum * 2^(e-128) (isum = sum of 2*E2M1*q).  The
// activation scale d_x is applied per block with one FMA:
//   acc = fma(D_h + D_l, d_x, acc)  ==  fma(float(isum), d_x * 2^(e-128), acc).
// Rows of a 16-row tile that contain an E8M0 outside [4, 254] (the +Inf
// scale 255, or scales whose products could leave the normal fp32 range) are
// computed with the integer LUT decode instead, so the results keep the
// reference's special-value semantics.
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWG = 256;
constexpr int kTokPerPass = 4;   // two MFMA token slots x two MFMAs per chunk
constexpr int kSeg = 4;          // chunks (of 4 blocks) per register buffer; two buffers
constexpr int kEMin = 4, kEMax = 254;

__device__ inline float dpp_down4(float v) {
    // lane c (within a row of 16) receives lane c+4 (row_shl:4)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x104, 0xF, 0xF, false));
}

// Integer-decode dot of one row (16 lanes of 64 cooperate: 4 lanes per row,
// used for the rare tiles with special E8M0 scales).
__device__ float lut_row_dot(const ByteView &v, uint32_t row_pos, int nb, const uint32_t *codes,
                             const float *s_dx, int sub) {
    float acc = 0.0f;
    for (int b = sub; b < nb; b += 4) {
        uint32_t d[5], o;
        load_block5(v, row_pos + (uint32_t)b * kMxBlock, d, &o);
        MxDecoded dec;
        mx_decode(d, o, dec);
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = codes[b * 8 + k];
        int32_t s = mx_isum(dec, q);
        acc = __builtin_fmaf((float)s, mx_block_scale(s_dx[b], dec.e), acc);
    }
    acc += __shfl_xor(acc, 1, 4);
    acc += __shfl_xor(acc, 2, 4);
    return acc;
}

}  // namespace

// One chunk: 16 rows x 4 blocks of A (this lane: row rowA, block 4*chunk+gb),
// against up to two token pairs; acc[tp][i] += (D_h + D_l) * d_x.
struct LaneRole {
    uint32_t sel;    // perm selector extracting the 16 nibble bytes
    uint32_t esh;    // bit offset of the E8M0 byte in dword 0
    int gb, gc, slot, boff, sb;
    bool lo_on, hi_on, row_ok;
};

__device__ inline void mx_chunk(const uint32_t raw[5], int chunk, int nb, int nt, const LaneRole &L,
                                const uint8_t *s_mx, const float *s_dx, const uint8_t *s_zero,
                                float acc[2][4], bool &special) {
    const int blk = 4 * chunk + L.gb;
    v8i A = {0, 0, 0, 0, 0, 0, 0, 0};
    int sa = 127;
    if (L.row_ok && blk < nb) {
        const int e = (int)__builtin_amdgcn_ubfe(raw[0], L.esh, 8u);
        if (e >= kEMin && e <= kEMax) {
            A[0] = (int)__builtin_amdgcn_perm(raw[1], raw[0], L.sel);
            A[1] = (int)__builtin_amdgcn_perm(raw[2], raw[1], L.sel);
            A[2] = (int)__builtin_amdgcn_perm(raw[3], raw[2], L.sel);
            A[3] = (int)__builtin_amdgcn_perm(raw[4], raw[3], L.sel);
            sa = e;
        } else {
            special = true;
        }
    }
    const int bB = 4 * chunk + L.gc;  // block of this lane's B column
    const bool bok = bB < nb;
#pragma unroll
    for (int tp = 0; tp < 2; tp++) {
        if (2 * tp >= nt) break;
        const int t = 2 * tp + L.slot;
        const bool live = bok && t < nt;
        const uint8_t *base = s_mx + ((size_t)t * nb + (live ? bB : 0)) * 64 + L.boff;
        const uint4 lo = *reinterpret_cast<const uint4 *>((L.lo_on && live) ? base : s_zero);
        const uint4 hi = *reinterpret_cast<const uint4 *>((L.hi_on && live) ? base : s_zero);
        v8i B = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        v4f d = {0.0f, 0.0f, 0.0f, 0.0f};
        d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, d, 4, 0, 0, sa, 0, L.sb);
        const float dx = live ? s_dx[t * nb + bB] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float sum = d[i] + dpp_down4(d[i]);
            acc[tp][i] = __builtin_fmaf(sum, dx, acc[tp][i]);
        }
    }
}

__device__ inline void mx_load_seg(const ByteView &view, uint32_t rowA_pos, int seg, int nch, int nb,
                                   const LaneRole &L, uint32_t raw[kSeg][5]) {
#pragma unroll
    for (int ch = 0; ch < kSeg; ch++) {
        const int chunk = seg * kSeg + ch;
        const int blk = 4 * chunk + L.gb;
        if (chunk < nch && L.row_ok && blk < nb)
            load_block5_raw(view, rowA_pos + (uint32_t)blk * kMxBlock, raw[ch]);
    }
}

__device__ inline void mx_compute_seg(const uint32_t raw[kSeg][5], int seg, int nch, int nb, int nt,
                                      const LaneRole &L, const uint8_t *s_mx, const float *s_dx,
                                      const uint8_t *s_zero, float acc[2][4], bool &special) {
#pragma unroll
    for (int ch = 0; ch < kSeg; ch++) {
        const int chunk = seg * kSeg + ch;
        if (chunk >= nch) break;
        mx_chunk(raw[ch], chunk, nb, nt, L, s_mx, s_dx, s_zero, acc, special);
    }
}

template <int MODE>
__global__ __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(3))) void k_mx_mfma(MxMfmaArgs a) {
    extern __shared__ __align__(16) uint8_t smem_b[];
    __shared__ int s_entry[kTokPerPass];
    __shared__ int s_arow[kTokPerPass];
    __shared__ float s_res[4][16][kTokPerPass];
    __shared__ float s_act[kTokPerPass][32];
    __shared__ __align__(16) uint8_t s_zero[16];

    const int nb = a.nb;
    const int nch = (nb + 3) >> 2;
    const int nseg = (nch + kSeg - 1) / kSeg;
    // LDS: [tok][nb][64] digit table, then [tok][nb] d_x
    uint8_t *s_mx = smem_b;
    float *s_dx = reinterpret_cast<float *>(s_mx + (size_t)kTokPerPass * nb * 64);

    const int tile_rows = MODE == kGateUp ? 32 : 64;
    const int tiles = (a.rows + tile_rows - 1) / tile_rows;
    const int slot_i = blockIdx.x / tiles, tile = blockIdx.x - slot_i * tiles;
    int e, begin, count;
    if (MODE == kRows) {
        e = a.expert;
        begin = 0;
        count = a.ntok;
    } else {
        if (slot_i >= *a.n_active) return;
        e = a.active[slot_i];
        begin = a.offsets[e];
        count = a.offsets[e + 1] - begin;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = MODE == kGateUp ? (wave >> 1) : 0;
    const int r0 = MODE == kGateUp ? tile * 32 + (wave & 1) * 16 : tile * 64 + wave * 16;
    LaneRole L;
    L.gb = lane >> 4;
    const int c = lane & 15;
    const int rowA = r0 + c;  // A operand row of this lane
    L.row_ok = rowA < a.rows;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const ByteView view = make_view(a.w[m] + (uint64_t)e * a.expert_bytes, a.expert_bytes);
    const uint32_t rowA_pos = (uint32_t)(L.row_ok ? rowA : 0) * row_bytes;
    // Blocks 4 apart are 68 bytes apart, so a lane's byte offset inside the
    // first dword of its block is the same for every chunk.
    const uint32_t o_lane = (rowA_pos + (uint32_t)L.gb * kMxBlock + view.lead) & 3u;
    L.sel = 0x04030201u + o_lane * 0x01010101u;
    L.esh = o_lane * 8u;
    // Static B-lane roles.
    L.slot = c >> 3;
    const int part = (c >> 2) & 1;
    L.gc = c & 3;
    L.lo_on = L.gc == (L.gb >> 1);
    L.hi_on = L.gc == (L.gb >> 1) + 2;
    L.boff = part * 32 + 16 * (L.gb & 1);
    L.sb = (L.gb == L.gc) ? (part == 0 ? 131 : 127) : 127;

    if (tid < 4) reinterpret_cast<uint32_t *>(s_zero)[tid] = 0u;

    uint32_t bufA[kSeg][5], bufB[kSeg][5];
    // The first segment's weights do not depend on the tokens: start them now.
    mx_load_seg(view, rowA_pos, 0, nch, nb, L, bufA);

    for (int c0 = 0; c0 < count; c0 += kTokPerPass) {
        const int nt = min(kTokPerPass, count - c0);
        if (tid < kTokPerPass) {
            int ent = 0, arow = 0;
            if (tid < nt) {
                ent = MODE == kRows ? c0 + tid : a.list[begin + c0 + tid];
                arow = MODE == kGateUp ? ent / a.topk : ent;
            }
            s_entry[tid] = ent;
            s_arow[tid] = arow;
        }
        __syncthreads();
        {
            const int mxw = nb * 16;  // dwords of digit table per token
            for (int t = 0; t < nt; t++) {
                uint32_t *dst = reinterpret_cast<uint32_t *>(s_mx + (size_t)t * nb * 64);
                const uint32_t *src = reinterpret_cast<const uint32_t *>(a.mxtab + (size_t)s_arow[t] * nb * 64);
                for (int i = tid; i < mxw; i += kWG) dst[i] = src[i];
                const float *sx = a.scales + (size_t)s_arow[t] * nb;
                for (int i = tid; i < nb; i += kWG) s_dx[t * nb + i] = sx[i];
            }
        }
        __syncthreads();
        if (c0 > 0) mx_load_seg(view, rowA_pos, 0, nch, nb, L, bufA);

        float acc[2][4];
#pragma unroll
        for (int p = 0; p < 2; p++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[p][i] = 0.0f;
        bool special = false;

        for (int seg = 0; seg < nseg; seg += 2) {
            if (seg + 1 < nseg) mx_load_seg(view, rowA_pos, seg + 1, nch, nb, L, bufB);
            mx_compute_seg(bufA, seg, nch, nb, nt, L, s_mx, s_dx, s_zero, acc, special);
            if (seg + 1 >= nseg) break;
            if (seg + 2 < nseg) mx_load_seg(view, rowA_pos, seg + 2, nch, nb, L, bufA);
            mx_compute_seg(bufB, seg + 1, nch, nb, nt, L, s_mx, s_dx, s_zero, acc, special);
        }
        // sum the four block positions g of each token slot (lanes c&3)
#pragma unroll
        for (int tp = 0; tp < 2; tp++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = acc[tp][i];
                v += __shfl_xor(v, 1, 4);
                v += __shfl_xor(v, 2, 4);
                acc[tp][i] = v;
            }
        if ((c & 7) == 0) {
#pragma unroll
            for (int tp = 0; tp < 2; tp++) {
                const int t = 2 * tp + L.slot;
                if (t < nt) {
#pragma unroll
                    for (int i = 0; i < 4; i++) s_res[wave][4 * L.gb + i][t] = acc[tp][i];
                }
            }
        }
        // Tiles with special scales: recompute with the integer decode.
        if (__any(special)) {
            const int row_l = lane >> 2, sub = lane & 3;
            const int row = r0 + row_l;
            const uint32_t pos = (uint32_t)(row < a.rows ? row : 0) * row_bytes;
            for (int t = 0; t < nt; t++) {
                const uint32_t *codes = reinterpret_cast<const uint32_t *>(a.codes + (size_t)s_arow[t] * nb * 32);
                float v = lut_row_dot(view, pos, nb, codes, s_dx + t * nb, sub);
                if (sub == 0) s_res[wave][row_l][t] = v;
            }
        }
        __syncthreads();

        // Epilogue.
        if (MODE == kGateUp) {
            // 32 rows x nt tokens: bias, clamped SwiGLU, taps.
            if (tid < 32 * kTokPerPass) {
                const int row = tid & 31, t = tid >> 5;
                const int r = tile * 32 + row;
                if (t < nt && r < a.rows) {
                    const uint64_t brow = (uint64_t)e * a.rows + r;
                    const float gv = s_res[row >> 4][row & 15][t] + bias_at(a.bias[0], a.bias_type[0], brow);
                    const float uv = s_res[2 + (row >> 4)][row & 15][t] + bias_at(a.bias[1], a.bias_type[1], brow);
                    const float act = swiglu(gv, uv);
                    const size_t o = (size_t)s_entry[t] * a.rows + r;
                    a.out[o] = act;
                    if (a.tap[0]) a.tap[0][o] = gv;
                    if (a.tap[1]) a.tap[1][o] = uv;
                    s_act[t][row] = act;
                }
            }
            __syncthreads();
            // The tile is one Q8_0 block of every token's act row: wave t
            // quantizes token t's block, one element per lane.
            if (wave < nt && a.act_codes && tile * 32 + 32 <= a.rows) {
                const float v = lane < 32 ? s_act[wave][lane] : 0.0f;
                uint16_t dh;
                const int q = q8_quantize_lane(v, lane, &dh);
                const size_t blk = (size_t)s_entry[wave] * (a.rows / 32) + tile;
                write_q8_lane(q, dh, lane, blk, a.act_codes, a.act_scales, a.act_mxtab, a.act_blocks34);
            }
        } else {
            for (int idx = tid; idx < 64 * kTokPerPass; idx += kWG) {
                const int row = idx & 63, t = idx >> 6;
                const int r = tile * 64 + row;
                if (t < nt && r < a.rows) {
                    const float v = s_res[row >> 4][row & 15][t] +
                                    bias_at(a.bias[0], a.bias_type[0], (uint64_t)e * a.rows + r);
                    a.out[(size_t)s_entry[t] * a.rows + r] = v;
                }
            }
        }
        __syncthreads();
    }
}

hipError_t launch_mx_mfma(hipStream_t s, GemvMode mode, const MxMfmaArgs &a, int slots) {
    if (slots <= 0 || a.rows <= 0) return hipSuccess;
    const size_t lds = (size_t)kTokPerPass * a.nb * (64 + 4);
    if (mode == kGateUp) {
        const int tiles = (a.rows + 31) / 32;
        hipLaunchKernelGGL(k_mx_mfma<kGateUp>, dim3(slots * tiles), dim3(kWG), lds, s, a);
    } else if (mode == kDown) {
        const int tiles = (a.rows + 63) / 64;
        hipLaunchKernelGGL(k_mx_mfma<kDown>, dim3(slots * tiles), dim3(kWG), lds, s, a);
    } else {
        const int tiles = (a.rows + 63) / 64;
        hipLaunchKernelGGL(k_mx_mfma<kRows>, dim3(slots * tiles), dim3(kWG), lds, s, a);
    }
    return hipGetLastError();
}

}  // namespace spt
