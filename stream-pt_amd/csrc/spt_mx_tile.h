// spt_mx_tile.h -- MFMA tile helpers shared by the MXFP4 x Q8_0 GEMV kernels
// (spt_mx_mfma.hip, spt_mx_decode.hip): lane roles and operands of
// v_mfma_scale_f32_16x16x128_f8f6f4 over an LDS image of 16-row tiles, with
// the K range split over eight waves, and the integer-decode row dot used
// for tiles with special E8M0 scales.  The lane layouts are described at
// the top of spt_mx_mfma.hip.
#pragma once

#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kWG = 64 * kWaves;
constexpr int kTokPerPass = kGemvTokens;  // two MFMA token slots x two MFMAs per chunk
constexpr int kEMin = 4, kEMax = 240;

// Integer-decode dot of one row (16 lanes of 64 cooperate: 4 lanes per row,
// used for the rare tiles with special E8M0 scales).
__device__ inline float lut_row_dot(const ByteView &v, uint32_t row_pos, int nb, const uint32_t *codes,
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

// Weights reach the MFMA through an LDS image of each 16-row tile.  The rows
// of an expert matrix are contiguous, so a tile's 16 rows are one run of
// 16 * nb * 17 bytes: two waves stream it with fully coalesced 16-byte loads
// (64 lanes x 16 B = 1 KB per instruction) starting at the 16-byte boundary
// at or below the run's first byte, store the image to LDS unchanged, and
// the MFMA lanes read their blocks back at any byte alignment (five dwords,
// realigned by byte permutes).  While the workgroup multiplies one unit (four
// tiles) the loads of its next unit are in flight, in registers.
constexpr int kMaxNb = kMxMaxInput / 32;
// 1 KB loads of a tile image: 16 rows plus up to 15 bytes before them.
__host__ __device__ constexpr int tile_loads(int nb) { return (16 * nb * kMxBlock + 15 + 1023) / 1024; }
// LDS bytes of a tile image: whole groups of four loads, and room for the
// reads of the blocks past nb in the last chunk (up to nb + 2, 20 bytes each
// from a dword boundary; the bound below allows nb + 6).
__host__ __device__ constexpr int tile_region(int nb) {
    return (4 * ((tile_loads(nb) + 3) / 4) > (16 * nb * kMxBlock + 137 + 1023) / 1024
                ? 4 * ((tile_loads(nb) + 3) / 4)
                : (16 * nb * kMxBlock + 137 + 1023) / 1024) *
           1024;
}

// Static lane roles.  MFMA A: row i = lane & 15, block gb = lane >> 4 of each
// chunk.  MFMA B: column c = 8*slot + 4*part + gc holds digit `part` of token
// `slot`'s block gc; its non-zero half is lo (A blocks gb>>1) or hi (A
// blocks (gb>>1)+2) of this lane, or neither.
struct LaneRole {
    int i, gb, gc, slot, boff, sb;
    bool lo_on, hi_on;
};

// A wave's B operands and d_x for one token pass: chunk c_j = wave + 8j
// (j < kChunksPerWave), token pair tp.  They are the same for every row of
// the expert, so they stay in registers for all the units of the pass.
constexpr int kChunksPerWave = (kMaxNb + 3) / 4 / kWaves + ((kMaxNb + 3) / 4 % kWaves != 0);
struct PassB {
    v8i b[kChunksPerWave][2];
    float dx[kChunksPerWave][2];
};

// Loads a pass's B operands from the digit tables (zero past nb, for the
// unused token slots and for the lane's empty half) and d_x from the scales.
// Every lane loads (the table's first block where it has nothing to load,
// then zeroes it), so the twelve loads go out back to back and are waited
// for once, instead of one round trip each behind a branch.
__device__ inline void load_pass_b(PassB &pb, int nb, const uint8_t *mxtab, const float *scales,
                                   const int (&arow)[kTokPerPass], int nt, const LaneRole &L, int wave) {
    u32x4v v[kChunksPerWave][2];
    float d[kChunksPerWave][2];
    bool okb[kChunksPerWave][2], okd[kChunksPerWave][2];
#pragma unroll
    for (int j = 0; j < kChunksPerWave; j++) {
        const int b = 4 * (wave + kWaves * j) + L.gc;
#pragma unroll
        for (int tp = 0; tp < 2; tp++) {
            const int t = 2 * tp + L.slot;
            const bool ok = t < nt && b < nb;
            const int ar = t == 0 ? arow[0] : t == 1 ? arow[1] : t == 2 ? arow[2] : arow[3];
            const size_t blk = ok ? (size_t)ar * nb + b : 0;
            okd[j][tp] = ok;
            okb[j][tp] = ok && (L.lo_on || L.hi_on);
            v[j][tp] = *reinterpret_cast<const u32x4v *>(mxtab + blk * 64 + (okb[j][tp] ? L.boff : 0));
            d[j][tp] = scales[blk];
        }
    }
#pragma unroll
    for (int j = 0; j < kChunksPerWave; j++)
#pragma unroll
        for (int tp = 0; tp < 2; tp++) {
            const u32x4v z = {0u, 0u, 0u, 0u};
            const u32x4v w = okb[j][tp] ? v[j][tp] : z;
            pb.b[j][tp] = L.lo_on ? __builtin_bit_cast(v8i, __builtin_shufflevector(w, z, 0, 1, 2, 3, 4, 5, 6, 7))
                                  : __builtin_bit_cast(v8i, __builtin_shufflevector(z, w, 0, 1, 2, 3, 4, 5, 6, 7));
            pb.dx[j][tp] = okd[j][tp] ? d[j][tp] : 0.0f;
        }
}

// Per-lane view of a tile image.  Chunk c covers blocks 4c..4c+3 of the 16
// rows: A lane (gb, i) takes row i, block 4c + gb, at byte rpos + 17 *
// (4c + gb) of the image; a chunk advances 68 bytes (17 dwords), so the
// lane's byte offset within a dword, and with it the realigning permute, is
// fixed for the tile.
struct TileView {
    const uint32_t *pa;
    uint32_t sel, esh;
    uint32_t emin, emax;
};

__device__ __attribute__((always_inline)) inline TileView tile_view(const uint8_t *img, uint32_t rpos, const LaneRole &L) {
    const uint32_t pos0 = rpos + (uint32_t)L.gb * kMxBlock;
    const uint32_t o = pos0 & 3u;
    TileView v;
    v.pa = reinterpret_cast<const uint32_t *>(img + (pos0 & ~3u));
    v.sel = 0x04030201u + o * 0x01010101u;  // bytes o+1 .. o+4
    v.esh = o * 8u;
    v.emin = 255u;
    v.emax = 0u;
    return v;
}

// A special E8M0 (outside [4, 240]) in the blocks this wave multiplied of a
// tile's valid rows: the tile's rows are then recomputed with the integer
// decode, so the MFMA results of such a tile are unused.
__device__ inline bool tile_special(const TileView &v, bool row_ok) {
    return row_ok && (v.emin < (uint32_t)kEMin || v.emax > (uint32_t)kEMax);
}

// The wave's chunks j < NC (chunk c_j = wave + 8j) of two row tiles r0,
// r0 + 1: all their LDS reads, then the A operands, then the MFMAs back to
// back, then the FMAs that apply d_x (in chunk order per accumulator), so
// the LDS and MFMA latencies are met once per call.  MASKLAST: the last
// chunk holds blocks past nb, which get scale 2^0 (their B operands and d_x
// are zero, so they add 0) and stay out of the special-scale check.  A tile
// past the matrix's rows is multiplied too (whatever its LDS region holds;
// E2M1 codes are finite): its results are never stored and its rows are not
// checked for special scales.
template <int NP, int NC, bool MASKLAST>
__device__ __attribute__((always_inline)) inline void tile_pair_run(TileView (&tv)[4], int r0, int wave, int nb,
                                                                    const LaneRole &L, const PassB &pb,
                                                                    float (&acc)[2][2][4]) {
    uint32_t d[NC][2][5];
#pragma unroll
    for (int j = 0; j < NC; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int i = 0; i < 5; i++) d[j][h][i] = tv[r0 + h].pa[17 * (wave + kWaves * j) + i];
    v8i A[NC][2];
    int sa[NC][2];
#pragma unroll
    for (int j = 0; j < NC; j++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            TileView &v = tv[r0 + h];
            const uint32_t ev = __builtin_amdgcn_ubfe(d[j][h][0], v.esh, 8u);
            sa[j][h] = (int)ev;
            if (MASKLAST && j == NC - 1) {
                const bool in = 4 * (wave + kWaves * j) + L.gb < nb;
                sa[j][h] = in ? sa[j][h] : 127;
                v.emin = in ? min(v.emin, ev) : v.emin;
                v.emax = in ? max(v.emax, ev) : v.emax;
            } else {
                v.emin = min(v.emin, ev);
                v.emax = max(v.emax, ev);
            }
            A[j][h] = v8i{(int)__builtin_amdgcn_perm(d[j][h][1], d[j][h][0], v.sel),
                          (int)__builtin_amdgcn_perm(d[j][h][2], d[j][h][1], v.sel),
                          (int)__builtin_amdgcn_perm(d[j][h][3], d[j][h][2], v.sel),
                          (int)__builtin_amdgcn_perm(d[j][h][4], d[j][h][3], v.sel), 0, 0, 0, 0};
        }
    v4f dd[NC][2][NP];
#pragma unroll
    for (int j = 0; j < NC; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int tp = 0; tp < NP; tp++) {
                const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
                dd[j][h][tp] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[j][h], pb.b[j][tp], z, 4, 0, 0,
                                                                                sa[j][h], 0, L.sb);
            }
#pragma unroll
    for (int j = 0; j < NC; j++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int tp = 0; tp < NP; tp++)
#pragma unroll
                for (int k = 0; k < 4; k++)
                    acc[h][tp][k] = __builtin_fmaf(dd[j][h][tp][k], pb.dx[j][tp], acc[h][tp][k]);
}

// The wave's chunks of row tiles r0, r0 + 1: nc (0..kChunksPerWave) of
// them, the last masked when it holds blocks past nb.
template <int NP>
__device__ __attribute__((always_inline)) inline void tile_pair(TileView (&tv)[4], int r0, int wave, int nc, bool mask_last,
                                                                int nb, const LaneRole &L, const PassB &pb,
                                                                float (&acc)[2][2][4]) {
    static_assert(kChunksPerWave == 3, "cases below");
    if (nc == 3) {
        if (mask_last)
            tile_pair_run<NP, 3, true>(tv, r0, wave, nb, L, pb, acc);
        else
            tile_pair_run<NP, 3, false>(tv, r0, wave, nb, L, pb, acc);
    } else if (nc == 2) {
        if (mask_last)
            tile_pair_run<NP, 2, true>(tv, r0, wave, nb, L, pb, acc);
        else
            tile_pair_run<NP, 2, false>(tv, r0, wave, nb, L, pb, acc);
    } else if (nc == 1) {
        if (mask_last)
            tile_pair_run<NP, 1, true>(tv, r0, wave, nb, L, pb, acc);
        else
            tile_pair_run<NP, 1, false>(tv, r0, wave, nb, L, pb, acc);
    }
}

// Sum over each group of eight lanes (every lane of the group gets it),
// pairing lanes by DPP: lane ^ 7, then ^ 1, then ^ 2.
__device__ __attribute__((always_inline)) inline float sum8(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    return v;
}

}  // namespace spt
