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
// Rows of a 16-row tile that contain an E8M0 outside [4, 240] are computed
// with the integer LUT decode instead, so the results keep the reference's
// special-value semantics: 255 is the +Inf scale, and above 240 a D value
// (up to 2^(e-127) * 16 * 32 * 6 * 8 = 2^(e-112.4)) can overflow fp32 where
// the oracle's d_x * 2^(e-128) * isum stays finite; below 4 the smallest
// products (2^(e-128)) leave the normal range.
#include <type_traits>

#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kWG = 64 * kWaves;
constexpr int kTokPerPass = kGemvTokens;  // two MFMA token slots x two MFMAs per chunk
constexpr int kEMin = 4, kEMax = 240;

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

// Weights reach the MFMA through a wave-private LDS image of the wave's 16
// rows.  The rows of an expert matrix are contiguous, so a wave's 16 rows are
// one run of 16 * nb * 17 bytes: the wave streams it with fully coalesced
// 16-byte loads (64 lanes x 16 B = 1 KB per instruction) starting at the
// 16-byte boundary at or below the run's first byte, stores the image to LDS
// unchanged, and the MFMA lanes read their blocks back at any byte alignment
// (five dwords, realigned by byte permutes).  While a wave multiplies one
// tile the loads of its next tile are in flight.  The image of one tile (nb
// up to kMaxNb) plus the token tables must fit the LDS of a CU, which holds
// one workgroup of four waves.
constexpr int kMaxNb = kMxMaxInput / 32;
constexpr int kMaxNbp = (kMaxNb + 7) / 8 * 8;
// 1 KB loads of a tile image: 16 rows plus up to 15 bytes before them.
__host__ __device__ constexpr int tile_loads(int nb) { return (16 * nb * kMxBlock + 15 + 1023) / 1024; }
// LDS bytes of a wave's image: whole groups of four loads, and room for the
// reads of the blocks past nb in the last chunk pair (up to nb + 6, 20 bytes
// each from a dword boundary).
__host__ __device__ constexpr int tile_region(int nb) {
    return (4 * ((tile_loads(nb) + 3) / 4) > (16 * nb * kMxBlock + 137 + 1023) / 1024
                ? 4 * ((tile_loads(nb) + 3) / 4)
                : (16 * nb * kMxBlock + 137 + 1023) / 1024) *
           1024;
}
constexpr int kTileGroups = (tile_loads(kMaxNb) + 3) / 4;  // groups of four 1 KB loads per tile
constexpr int kWaveGroups = (kTileGroups + 1) / 2;            // of them, loaded by one wave
constexpr int kTabLoads = (16 * kMaxNbp + kWG - 1) / kWG;  // 16-byte digit-table pieces per thread
constexpr int kDxLoads = (kTokPerPass * kMaxNbp + kWG - 1) / kWG;  // d_x entries per thread
constexpr size_t kMaxMxLds = 146 * 1024;  // dynamic LDS; with the static part (< 14 KB) within 160 KB

template <int MODE> struct MxTraits {
    // Unit outputs staged in LDS before a flush, and the values staged per
    // row and token (gate/up: act, gate, up; down: the result).
    static constexpr int kStageUnits = MODE == kGateUp ? 4 : 6;
    static constexpr int kStageVals = MODE == kGateUp ? 3 : 1;
    static constexpr int kUnitRows = MODE == kGateUp ? 32 : 64;
};

// Orders a wave's accesses to its own LDS tile for the compiler (the hardware
// executes one wave's LDS instructions in order).
__device__ inline void wave_lds_fence() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
}

// Workgroup barrier ordering LDS only.  All communication between the
// waves of k_mx_mfma goes through LDS, and __syncthreads() would also wait
// for every outstanding global load, draining the next tile in flight.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// A wave's part of a tile image in flight: four loads of 1 KB per group.
// The loads are issued and waited for with inline assembly, out of sight of
// the compiler's wait-count analysis, which turns conservative (a full
// drain) at the loop's control-flow joins: tile_issue writes the registers
// asynchronously, tile_wait (s_waitcnt vmcnt(0)) names every one of them,
// and only tile_store reads them, after the wait.  Each issue block opens
// with five wait states: its descriptor and offset SGPRs may have just been
// written by a VALU instruction, which a following VMEM read must not see
// early, and the compiler cannot pad inside inline assembly.  Offsets past
// the descriptor's range read zeros.
struct TileRegs {
    u32x4v q[4 * kWaveGroups];
};

template <int G>
__device__ inline void tile_issue(TileRegs &t, uint32_t vo, const u32x4v &rs, uint32_t so) {
    asm volatile(
        "s_nop 4\n\t"
        "buffer_load_dwordx4 %0, %4, %5, %6 offen\n\t"
        "buffer_load_dwordx4 %1, %4, %5, %6 offen offset:1024\n\t"
        "buffer_load_dwordx4 %2, %4, %5, %6 offen offset:2048\n\t"
        "buffer_load_dwordx4 %3, %4, %5, %6 offen offset:3072"
        : "=&v"(t.q[4 * G]), "=&v"(t.q[4 * G + 1]), "=&v"(t.q[4 * G + 2]), "=&v"(t.q[4 * G + 3])
        : "v"(vo), "s"(rs), "s"(so));
}

__device__ inline void tile_wait(TileRegs &t) {
    static_assert(kWaveGroups == 3, "operand list below");
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(t.q[0]), "+v"(t.q[1]), "+v"(t.q[2]), "+v"(t.q[3]), "+v"(t.q[4]), "+v"(t.q[5]),
                   "+v"(t.q[6]), "+v"(t.q[7]), "+v"(t.q[8]), "+v"(t.q[9]), "+v"(t.q[10]), "+v"(t.q[11]));
}

template <int G>
__device__ inline void tile_store(uint32_t lds, const TileRegs &t) {
    asm volatile(
        "ds_write_b128 %0, %1\n\t"
        "ds_write_b128 %0, %2 offset:1024\n\t"
        "ds_write_b128 %0, %3 offset:2048\n\t"
        "ds_write_b128 %0, %4 offset:3072"
        :
        : "v"(lds), "v"(t.q[4 * G]), "v"(t.q[4 * G + 1]), "v"(t.q[4 * G + 2]), "v"(t.q[4 * G + 3])
        : "memory");
}

// Static lane roles.  MFMA A: row i = lane & 15, block gb = lane >> 4 of each
// chunk.  MFMA B: column c = 8*slot + 4*part + gc holds digit `part` of token
// `slot`'s block gc; its non-zero half is lo (A blocks gb>>1) or hi (A
// blocks (gb>>1)+2) of this lane, or neither.
struct LaneRole {
    int i, gb, gc, slot, boff, sb;
    bool lo_on, hi_on;
};

// Per token pass and token pair: where this lane's B operand halves and d_x
// are read at chunk 0 (add 256 bytes and 4 floats per chunk).  A half that
// carries no data reads the zero area, which is as long as the tables.
struct PassRole {
    const uint8_t *bl[2], *bh[2];
    const float *dx[2];
};

// The LDS words of one chunk: the five dwords holding this lane's A block,
// and per token pair the two halves of the B operand and d_x.
template <int NP>
struct ChunkRaw {
    uint32_t d[5];
    u32x4v blo[NP], bhi[NP];
    float x[NP];
};

template <int NP>
__device__ __attribute__((always_inline)) inline void chunk_fetch(ChunkRaw<NP> &r, const uint32_t *pa, const PassRole &P, int c) {
#pragma unroll
    for (int i = 0; i < 5; i++) r.d[i] = pa[17 * c + i];
#pragma unroll
    for (int tp = 0; tp < NP; tp++) {
        r.blo[tp] = *reinterpret_cast<const u32x4v *>(P.bl[tp] + 256 * c);
        r.bhi[tp] = *reinterpret_cast<const u32x4v *>(P.bh[tp] + 256 * c);
        r.x[tp] = P.dx[tp][4 * c];
    }
}

// MFMAs of a fetched chunk.  MASK: the chunk may hold blocks past nb, which
// get scale 2^0 (their tables and d_x are zero, so they add 0) and stay out
// of the special-scale check.
template <int NP, bool MASK>
__device__ __attribute__((always_inline)) inline void chunk_mfma(const ChunkRaw<NP> &r, int c, int nb, uint32_t sel, uint32_t esh, const LaneRole &L,
                                  float acc[2][4], uint32_t &emin, uint32_t &emax) {
    const uint32_t ev = __builtin_amdgcn_ubfe(r.d[0], esh, 8u);
    int sa = (int)ev;
    if (MASK) {
        const bool in = 4 * c + L.gb < nb;
        sa = in ? sa : 127;
        emin = in ? min(emin, ev) : emin;
        emax = in ? max(emax, ev) : emax;
    } else {
        emin = min(emin, ev);
        emax = max(emax, ev);
    }
    const v8i A = {(int)__builtin_amdgcn_perm(r.d[1], r.d[0], sel), (int)__builtin_amdgcn_perm(r.d[2], r.d[1], sel),
                   (int)__builtin_amdgcn_perm(r.d[3], r.d[2], sel), (int)__builtin_amdgcn_perm(r.d[4], r.d[3], sel),
                   0, 0, 0, 0};
#pragma unroll
    for (int tp = 0; tp < NP; tp++) {
        const v8i B = __builtin_bit_cast(v8i, __builtin_shufflevector(r.blo[tp], r.bhi[tp], 0, 1, 2, 3, 4, 5, 6, 7));
        v4f dd = {0.0f, 0.0f, 0.0f, 0.0f};
        dd = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, dd, 4, 0, 0, sa, 0, L.sb);
#pragma unroll
        for (int k = 0; k < 4; k++) acc[tp][k] = __builtin_fmaf(dd[k], r.x[tp], acc[tp][k]);
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

// A special E8M0 (outside [4, 240]) in the tile's valid blocks: the tile's
// rows are then recomputed with the integer decode, so the MFMA results of
// such a tile are unused.
__device__ inline bool tile_special(const TileView &v, bool row_ok) {
    return row_ok && (v.emin < (uint32_t)kEMin || v.emax > (uint32_t)kEMax);
}

// NC consecutive chunks from c0: all their LDS reads, then their A operands,
// then all their MFMAs back to back, then the FMAs that apply d_x (in chunk
// order per accumulator), so no FMA waits on the MFMA issued just before it.
template <int NP, bool MASK, int NC>
__device__ __attribute__((always_inline)) inline void chunk_run(TileView &v, int c0, int nb, const LaneRole &L,
                                                                const PassRole &P, float acc[2][4]) {
    ChunkRaw<NP> r[NC];
#pragma unroll
    for (int h = 0; h < NC; h++) chunk_fetch<NP>(r[h], v.pa, P, c0 + h);
    // d_x is first needed after the MFMAs; naming it here keeps its reads
    // with the others, behind one wait, rather than late behind a second.
#pragma unroll
    for (int h = 0; h < NC; h++)
#pragma unroll
        for (int tp = 0; tp < NP; tp++) asm volatile("" : "+v"(r[h].x[tp]));
    v8i A[NC];
    int sa[NC];
#pragma unroll
    for (int h = 0; h < NC; h++) {
        const uint32_t ev = __builtin_amdgcn_ubfe(r[h].d[0], v.esh, 8u);
        sa[h] = (int)ev;
        if (MASK) {
            const bool in = 4 * (c0 + h) + L.gb < nb;
            sa[h] = in ? sa[h] : 127;
            v.emin = in ? min(v.emin, ev) : v.emin;
            v.emax = in ? max(v.emax, ev) : v.emax;
        } else {
            v.emin = min(v.emin, ev);
            v.emax = max(v.emax, ev);
        }
        A[h] = v8i{(int)__builtin_amdgcn_perm(r[h].d[1], r[h].d[0], v.sel), (int)__builtin_amdgcn_perm(r[h].d[2], r[h].d[1], v.sel),
                   (int)__builtin_amdgcn_perm(r[h].d[3], r[h].d[2], v.sel), (int)__builtin_amdgcn_perm(r[h].d[4], r[h].d[3], v.sel),
                   0, 0, 0, 0};
    }
    v4f dd[NC][NP];
#pragma unroll
    for (int h = 0; h < NC; h++)
#pragma unroll
        for (int tp = 0; tp < NP; tp++) {
            const v8i B = __builtin_bit_cast(v8i, __builtin_shufflevector(r[h].blo[tp], r[h].bhi[tp], 0, 1, 2, 3, 4, 5, 6, 7));
            const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
            dd[h][tp] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A[h], B, z, 4, 0, 0, sa[h], 0, L.sb);
        }
#pragma unroll
    for (int h = 0; h < NC; h++)
#pragma unroll
        for (int tp = 0; tp < NP; tp++)
#pragma unroll
            for (int k = 0; k < 4; k++) acc[tp][k] = __builtin_fmaf(dd[h][tp][k], r[h].x[tp], acc[tp][k]);
}

template <int NP, bool MASK>
__device__ __attribute__((always_inline)) inline void chunk_quad(TileView &v, int c0, int nb, const LaneRole &L, const PassRole &P, float acc[2][4]) {
    chunk_run<NP, MASK, 4>(v, c0, nb, L, P, acc);
}

template <int NP, bool MASK>
__device__ __attribute__((always_inline)) inline void chunk_pair(TileView &v, int c0, int nb, const LaneRole &L, const PassRole &P, float acc[2][4]) {
    chunk_run<NP, MASK, 2>(v, c0, nb, L, P, acc);
}

// Part `part` (0..2) of the chunks of wave half h (the waves of a row tile
// split its chunks in halves, each in three parts; before each part a wave
// issues one group of the next tile's loads).  24 chunks (nb in [89, 96]:
// the GPT-OSS dimension 2880 has nb = 90): half h takes chunks 12h..12h+11
// as three straight-line quads, chunks 22-23 (possibly past nb) masked; any
// other even chunk count: half h takes half of the chunk pairs, split over
// the three parts, the pairs holding blocks past nb masked.
template <int NP>
__device__ __attribute__((always_inline)) inline void tile_part(int part, int h, TileView &v, int nb, int nch,
                                                                const LaneRole &L, const PassRole &P, float acc[2][4]) {
    if (nch == 24) {
        const int c0 = 12 * h + 4 * part;
        if (c0 < 20) {
            chunk_quad<NP, false>(v, c0, nb, L, P, acc);
        } else {
            chunk_pair<NP, false>(v, 20, nb, L, P, acc);
            chunk_pair<NP, true>(v, 22, nb, L, P, acc);
        }
        return;
    }
    const int npairs = nch / 2, nfull = nb / 8;  // pairs, and pairs whose 8 blocks are all < nb
    const int p0 = h ? npairs / 2 : 0, np = h ? npairs - npairs / 2 : npairs / 2;
    for (int p = p0 + part * np / 3; p < p0 + (part + 1) * np / 3; p++) {
        if (p < nfull)
            chunk_pair<NP, false>(v, 2 * p, nb, L, P, acc);
        else
            chunk_pair<NP, true>(v, 2 * p, nb, L, P, acc);
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

// Position in a workgroup's range of work items (slot, pass, tile), in that
// order: w = (pass_off[slot] + pass) * tiles + tile.  slot = an active
// expert, pass = kTokPerPass tokens of its list, tile = a row tile.
struct Cursor {
    int w, slot, p, tile, e, begin, count, npass;
};

// Routing arrays of the select kernel, read-only here.
struct Route {
    const int32_t *__restrict__ active;
    const int32_t *__restrict__ offsets;
    const int32_t *__restrict__ pass_off;
    const int32_t *__restrict__ list;
};

template <int MODE>
__device__ inline void slot_info(const MxMfmaArgs &a, const Route &rt, Cursor &c) {
    if (MODE == kRows) {
        c.e = a.expert;
        c.begin = 0;
        c.count = a.ntok;
    } else {
        c.e = rt.active[c.slot];
        c.begin = rt.offsets[c.e];
        c.count = rt.offsets[c.e + 1] - c.begin;
    }
    c.npass = (c.count + kTokPerPass - 1) / kTokPerPass;
}

template <int MODE>
__device__ inline void cursor_advance(const MxMfmaArgs &a, const Route &rt, Cursor &c, int tiles) {
    ++c.w;
    if (++c.tile < tiles) return;
    c.tile = 0;
    if (++c.p < c.npass) return;
    c.p = 0;
    ++c.slot;
    slot_info<MODE>(a, rt, c);
}

// The tokens of a cursor's pass: list entries (idx = token * topk + rank for
// the grouped modes, the token for kRows) and the rows of the activation
// tables they read (gate/up: the token; down: the entry).
struct PassTokens {
    int nt;
    int ent[kTokPerPass], arow[kTokPerPass];
};

template <int MODE>
__device__ inline PassTokens pass_tokens(const MxMfmaArgs &a, const Route &rt, const Cursor &c) {
    PassTokens pt;
    pt.nt = min(kTokPerPass, c.count - c.p * kTokPerPass);
#pragma unroll
    for (int t = 0; t < kTokPerPass; t++) {
        int ent = 0;
        if (t < pt.nt) ent = MODE == kRows ? c.p * kTokPerPass + t : rt.list[c.begin + c.p * kTokPerPass + t];
        pt.ent[t] = ent;
        pt.arow[t] = MODE == kGateUp ? ent / a.topk : ent;
    }
    return pt;
}

__device__ inline int pick4(const int (&v)[kTokPerPass], int t) {
    return t == 0 ? v[0] : t == 1 ? v[1] : t == 2 ? v[2] : v[3];
}

// Persistent workgroups, one per CU, of eight waves: workgroup b takes work
// items [b*W/G, (b+1)*W/G) of the W = total passes x row tiles, in order, so
// consecutive items share an expert's token pass and its staged token
// tables, and every workgroup streams the same number of weight bytes.
// Gate/up units are 32 output rows (row tiles 0-1 gate, 2-3 up, so SwiGLU
// and the Q8_0 of the 32-element act block stay in the workgroup); down and
// single-expert units are 64 rows; a row tile is 16 rows.  Waves r and r + 4
// (the same SIMD) share row tile r's image: each loads half of its load
// groups and multiplies half of its chunks, and their partial row sums are
// added in the epilogue, so every SIMD runs two waves that hide each
// other's latencies.
//
// Each step: wait for the prefetched tile and write it (and, at a new pass,
// the token tables) to LDS; flush staged outputs if the stage is full;
// multiply, issuing the next unit's load groups between parts of the
// multiply; reduce and stage the unit's outputs.  The only wait for global
// loads is at the top of a step, for loads issued during the step before.
template <int MODE>
__global__ __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(2))) void k_mx_mfma(MxMfmaArgs a, const int32_t *__restrict__ r_active,
                                                                      const int32_t *__restrict__ r_offsets,
                                                                      const int32_t *__restrict__ r_pass_off,
                                                                      const int32_t *__restrict__ r_list,
                                                                      const int32_t *__restrict__ r_n_active) {
    extern __shared__ __align__(16) uint8_t smem_b[];
    // Output pointers of the epilogue, kept in LDS rather than in scalar
    // registers across the loop.
    struct EpiPtrs {
        float *out, *tap0, *tap1, *act_scales;
        int8_t *act_codes;
        uint8_t *act_mxtab, *act_blocks34;
    };
    __shared__ EpiPtrs s_epi;
    // Partial row sums of a unit per wave half and row tile, and the waves'
    // special-scale flags (double-buffered by step parity, so a step's
    // staging and the next step's sums need no barrier apart).
    __shared__ float s_res[2][2][4][16][kTokPerPass];
    __shared__ int s_special[2][kWaves];
    // Outputs of finished units, written to global memory kStageUnits units
    // at a time, at the top of a step.  Gate/up also stages each act block's
    // Q8_0 codes, digit-table bytes and fp16 scale bits.
    constexpr int kStage = MxTraits<MODE>::kStageUnits;
    constexpr int kUnitRows = MxTraits<MODE>::kUnitRows;
    constexpr int kQStage = MODE == kGateUp ? kStage : 1;
    __shared__ float s_stage[kStage][MxTraits<MODE>::kStageVals][kTokPerPass][kUnitRows];
    __shared__ int8_t s_sq[kQStage][kTokPerPass][32];
    __shared__ uint8_t s_smx[kQStage][kTokPerPass][64];
    __shared__ uint16_t s_sdh[kQStage][kTokPerPass];
    __shared__ int s_stage_ent[kStage][kTokPerPass];
    __shared__ int s_stage_tile[kStage];
    __shared__ int s_stage_nt[kStage];

    const int nb = a.nb;
    const int nbp = (nb + 7) & ~7;  // token tables padded with zero blocks to whole chunk pairs
    const int nch = nbp / 4;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const int ngroups = (tile_loads(nb) + 3) / 4;
    const int region = tile_region(nb);
    // wave-uniform: keeps per-wave descriptors and offsets in scalar registers
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rt4 = wave & 3, half = wave >> 2;  // row tile, and which half of it this wave takes
    // load groups of this wave: [g0, g0 + gmine)
    const int g0 = half ? (ngroups + 1) / 2 : 0;
    const int gmine = half ? ngroups / 2 : (ngroups + 1) / 2;
    // LDS: row tiles' images, then [tok][nbp][64] digit tables, [tok][nbp] d_x, zeros
    uint8_t *img = smem_b + (size_t)rt4 * region;
    uint8_t *s_mx = smem_b + (size_t)4 * region;
    // LDS address of this lane's 16 bytes of the image's first group of this wave
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t img_lds =
        (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)img) + 4096u * (uint32_t)g0 + 16u * (uint32_t)lane;
    float *s_dx = reinterpret_cast<float *>(s_mx + (size_t)kTokPerPass * nbp * 64);
    uint8_t *s_zero = reinterpret_cast<uint8_t *>(s_dx + kTokPerPass * nbp);  // nbp * 64 bytes of zeros

    const int tile_rows = MODE == kGateUp ? 32 : 64;
    const int tiles = (a.rows + tile_rows - 1) / tile_rows;
    const Route rt{r_active, r_offsets, r_pass_off, r_list};
    const int n_slots = MODE == kRows ? 1 : *r_n_active;
    const int P = MODE == kRows ? (a.ntok + kTokPerPass - 1) / kTokPerPass : rt.pass_off[n_slots];
    const int W = P * tiles;
    const int w0 = (int)((int64_t)blockIdx.x * W / gridDim.x);
    const int w1 = (int)((int64_t)(blockIdx.x + 1) * W / gridDim.x);
    if (w0 >= w1) return;
    // slot of the first item: the number of pass_off[s] <= w0 / tiles, minus 1
    const int q0 = w0 / tiles;
    int slot0 = 0;
    if (MODE != kRows) {
        int ones = 0;
        for (int s0 = 0; s0 <= n_slots; s0 += kWG) {
            const int sidx = s0 + tid;
            ones += __syncthreads_count(sidx <= n_slots && rt.pass_off[sidx] <= q0);
        }
        slot0 = ones - 1;
    }

    const int m = MODE == kGateUp ? (rt4 >> 1) : 0;
    const int roff = MODE == kGateUp ? (rt4 & 1) * 16 : rt4 * 16;
    LaneRole L;
    L.i = lane & 15;
    L.gb = lane >> 4;
    const int c16 = lane & 15;
    L.slot = c16 >> 3;
    const int part = (c16 >> 2) & 1;
    L.gc = c16 & 3;
    L.lo_on = L.gc == (L.gb >> 1);
    L.hi_on = L.gc == (L.gb >> 1) + 2;
    L.boff = part * 32 + 16 * (L.gb & 1);
    L.sb = (L.gb == L.gc) ? (part == 0 ? 131 : 127) : 127;
    if (tid == 0) s_epi = EpiPtrs{a.out, a.tap[0], a.tap[1], a.act_scales, a.act_codes, a.act_mxtab, a.act_blocks34};
    for (int i = tid; i < nbp * 4; i += kWG) reinterpret_cast<u32x4v *>(s_zero)[i] = u32x4v{0u, 0u, 0u, 0u};

    // Epilogue element of this thread: gate/up: row tid&31 of the unit,
    // token tid>>5 (waves 0-1); down/rows: row tid&63, token tid>>6 (waves 0-3).
    const int erow = MODE == kGateUp ? (tid & 31) : (tid & 63);
    const BiasView bv0 = make_bias_view(a.bias[0], a.bias_bytes[0], a.bias_type[0]);
    const BiasView bv1 = make_bias_view(a.bias[1], a.bias_bytes[1], a.bias_type[1]);
    const uint8_t *wbase = a.w[m];

    Cursor cur;
    cur.w = w0;
    cur.slot = slot0;
    cur.p = MODE == kRows ? q0 : q0 - rt.pass_off[slot0];
    cur.tile = w0 - q0 * tiles;
    slot_info<MODE>(a, rt, cur);

    // Registers of the next unit: this wave's groups of its tile image, and
    // the epilogue element's raw bias words.
    TileRegs tr;
    // the next unit's tile: descriptor, aligned start of this wave's groups,
    // and whether this wave loads it
    u32x4v nrs = {0u, 0u, 0u, 0u};
    uint32_t na0 = 0u;
    bool nxt_ok = false;
    const uint32_t vo = 16u * (uint32_t)lane;
    // local group G of the next tile's loads (G a compile-time constant, so
    // every issue block writes fixed registers)
    auto issue = [&](auto gc) {
        constexpr int G = decltype(gc)::value;
        static_assert(G < kWaveGroups, "group");
        if (nxt_ok && G < gmine) tile_issue<G>(tr, vo, nrs, na0 + 4096u * G);
    };
    uint32_t b0r = 0u, b1r = 0u;
    auto prefetch = [&](const Cursor &c) {
        const uint32_t brow = (uint32_t)c.e * (uint32_t)a.rows + (uint32_t)(c.tile * tile_rows + erow);
        b0r = bias_raw(bv0, brow);
        if (MODE == kGateUp) b1r = bias_raw(bv1, brow);
        const int row0 = c.tile * tile_rows + roff;
        nxt_ok = false;
        if (row0 < a.rows) {
            // The expert matrix from the 16-byte boundary at or below its
            // first byte to the one at or above its end (a 16-byte load
            // that crosses the range's end reads zeros, and the bytes up to
            // that boundary share the last byte's page); loads past it read
            // zeros.  Bytes past the matrix only reach rows past a.rows.
            const uintptr_t mb = reinterpret_cast<uintptr_t>(wbase + (uint64_t)c.e * a.expert_bytes);
            const uint32_t le = (uint32_t)(mb & 15u);
            const uint64_t base = mb - le;
            // descriptor words: base, base_hi (stride 0), num_records, format
            const u32x4v rs = {(uint32_t)base, (uint32_t)(base >> 32) & 0xFFFFu,
                               (uint32_t)((a.expert_bytes + le + 15u) & ~15ull), (uint32_t)kRsrcWord3};
            nrs = rs;
            na0 = ((le + (uint32_t)row0 * row_bytes) & ~15u) + 4096u * (uint32_t)g0;
            nxt_ok = true;
        }
    };

    int staged_slot = -1, staged_p = -1, npair = 0;
    PassRole PR;
    float acc[2][4];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[p][i] = 0.0f;

    // Write out the staged units (all waves, after a barrier).  Gate/up:
    // thread-per-element act (for the tap), the gate/up taps and the act
    // blocks' Q8_0 in every layout (the unit is one Q8_0 block of each
    // token's act row); down: thread-per-element results.
    int n_staged = 0;
    auto flush = [&](int count) {
        const EpiPtrs ep = s_epi;
        if constexpr (MODE == kGateUp) {
            for (int i = tid; i < count * kTokPerPass * 32; i += kWG) {
                const int k = i >> 7, t = (i >> 5) & 3, e = i & 31;
                if (t >= s_stage_nt[k]) continue;
                const int tile = s_stage_tile[k], ent = s_stage_ent[k][t];
                const int r = tile * 32 + e;
                if (r < a.rows) {
                    const size_t o = (size_t)ent * a.rows + r;
                    if (ep.out) ep.out[o] = s_stage[k][0][t][e];
                    if (ep.tap0) ep.tap0[o] = s_stage[k][1][t][e];
                    if (ep.tap1) ep.tap1[o] = s_stage[k][2][t][e];
                }
                if (ep.act_codes && tile * 32 + 32 <= a.rows) {
                    const size_t blk = (size_t)ent * (a.rows / 32) + tile;
                    const int8_t qv = s_sq[k][t][e];
                    const uint16_t dh = s_sdh[k][t];
                    ep.act_codes[blk * 32 + e] = qv;
                    if (ep.act_mxtab) {
                        ep.act_mxtab[blk * 64 + e] = s_smx[k][t][e];
                        ep.act_mxtab[blk * 64 + 32 + e] = s_smx[k][t][32 + e];
                    }
                    if (ep.act_scales && e == 0) ep.act_scales[blk] = f16_bits_to_f32(dh);
                    if (ep.act_blocks34) {
                        if (e == 0) {
                            ep.act_blocks34[blk * kQ80Block] = (uint8_t)(dh & 0xff);
                            ep.act_blocks34[blk * kQ80Block + 1] = (uint8_t)(dh >> 8);
                        }
                        ep.act_blocks34[blk * kQ80Block + 2 + e] = (uint8_t)qv;
                    }
                }
            }
        } else {
            for (int i = tid; i < count * kTokPerPass * kUnitRows; i += kWG) {
                const int k = i / (kTokPerPass * kUnitRows), t = (i / kUnitRows) % kTokPerPass, r = i % kUnitRows;
                const int row = s_stage_tile[k] * kUnitRows + r;
                if (t < s_stage_nt[k] && row < a.rows)
                    ep.out[(size_t)s_stage_ent[k][t] * a.rows + row] = s_stage[k][0][t][r];
            }
        }
    };

    PassTokens npt = pass_tokens<MODE>(a, rt, cur);  // tokens of the unit in the registers
    prefetch(cur);
    static_assert(kWaveGroups == 3, "issue list below");
    issue(std::integral_constant<int, 0>{});
    issue(std::integral_constant<int, 1>{});
    issue(std::integral_constant<int, 2>{});

    for (int w = w0; w < w1; w++) {
        const Cursor u = cur;
        const PassTokens pt = npt;
        const bool new_tab = u.slot != staged_slot || u.p != staged_p;
        if (new_tab) {
            // Every wave is past the previous unit's first epilogue barrier,
            // after its last table read, so the tables are free.  Digit
            // tables [tok][nbp][64] and d_x [tok][nbp] of the pass's tokens,
            // zero past nb and for the unused token slots.  A pass change is
            // rare (each workgroup walks a contiguous range of work items),
            // so these loads are not prefetched.
            u32x4v tq[kTabLoads];
            float tdx[kDxLoads];
#pragma unroll
            for (int k = 0; k < kTabLoads; k++) {
                const int j = tid + kWG * k;  // 16-byte piece of [tok][nbp][64]
                const int t = j / (4 * nbp), rem = j - t * 4 * nbp, b = rem >> 2;
                u32x4v v = {0u, 0u, 0u, 0u};
                if (t < pt.nt && b < nb)
                    v = *reinterpret_cast<const u32x4v *>(a.mxtab + ((size_t)pick4(pt.arow, t) * nb + b) * 64 +
                                                          (rem & 3) * 16);
                tq[k] = v;
            }
#pragma unroll
            for (int k = 0; k < kDxLoads; k++) {
                const int i = tid + kWG * k;
                const int t = i / nbp, b = i - t * nbp;
                float v = 0.0f;
                if (t < pt.nt && b < nb) v = a.scales[(size_t)pick4(pt.arow, t) * nb + b];
                tdx[k] = v;
            }
#pragma unroll
            for (int k = 0; k < kTabLoads; k++) {
                const int j = tid + kWG * k;
                if (j < 16 * nbp) *reinterpret_cast<u32x4v *>(s_mx + (size_t)j * 16) = tq[k];
            }
#pragma unroll
            for (int k = 0; k < kDxLoads; k++) {
                const int i = tid + kWG * k;
                if (i < kTokPerPass * nbp) s_dx[i] = tdx[k];
            }
#pragma unroll
            for (int tp = 0; tp < 2; tp++) {
                const int t = 2 * tp + L.slot;
                const uint8_t *tb = s_mx + (t * nbp + L.gc) * 64 + L.boff;
                PR.bl[tp] = (L.lo_on && t < pt.nt) ? tb : s_zero;
                PR.bh[tp] = (L.hi_on && t < pt.nt) ? tb : s_zero;
                PR.dx[tp] = s_dx + t * nbp + L.gc;
            }
            npair = (pt.nt + 1) >> 1;
            staged_slot = u.slot;
            staged_p = u.p;
        }
        const int row0 = u.tile * tile_rows + roff;
        const bool wave_ok = row0 < a.rows;
        tile_wait(tr);
        // Both waves of a row tile have passed the previous unit's first
        // epilogue barrier, after their last read of the image.
        if (wave_ok) {
            static_assert(kWaveGroups == 3, "stores below");
            if (gmine > 0) tile_store<0>(img_lds, tr);
            if (gmine > 1) tile_store<1>(img_lds + 4096u, tr);
            if (gmine > 2) tile_store<2>(img_lds + 8192u, tr);
        }
        // The bias words arrived with the tile; take them now so no later
        // use waits on the next unit's loads.
        uint32_t bw0 = b0r, bw1 = b1r;
        asm volatile("" : "+v"(bw0), "+v"(bw1));
        nxt_ok = false;
        if (w + 1 < w1) {
            cursor_advance<MODE>(a, rt, cur, tiles);
            const bool ntab = cur.slot != u.slot || cur.p != u.p;
            if (ntab) npt = pass_tokens<MODE>(a, rt, cur);
            prefetch(cur);
        }
        // the other wave's half of the image, and new tables, are in place
        lds_barrier();
        if (n_staged == kStage) {
            flush(n_staged);
            n_staged = 0;
        }

        const uint8_t *view_base = wbase + (uint64_t)u.e * a.expert_bytes;
        bool special = false;
        {
            const uint32_t lead = (uint32_t)((reinterpret_cast<uintptr_t>(view_base) & 15u) + (uint32_t)row0 * row_bytes) & 15u;
            TileView tv = tile_view(img, lead + (uint32_t)L.i * row_bytes, L);
            auto segment = [&](auto gc) {
                constexpr int G = decltype(gc)::value;
                issue(gc);
                if (wave_ok) {
                    if (npair == 2)
                        tile_part<2>(G, half, tv, nb, nch, L, PR, acc);
                    else
                        tile_part<1>(G, half, tv, nb, nch, L, PR, acc);
                }
            };
            static_assert(kWaveGroups == 3, "segments below");
            segment(std::integral_constant<int, 0>{});
            segment(std::integral_constant<int, 1>{});
            segment(std::integral_constant<int, 2>{});
            special = wave_ok && tile_special(tv, row0 + L.i < a.rows);
        }

        // Sum the eight columns of each token slot (parts h/l x blocks).
#pragma unroll
        for (int tp = 0; tp < 2; tp++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[tp][i] = sum8(acc[tp][i]);
        const int par = w & 1;
        if ((c16 & 7) == 0) {
#pragma unroll
            for (int tp = 0; tp < 2; tp++) {
                const int t = 2 * tp + L.slot;
                if (t < pt.nt) {
#pragma unroll
                    for (int i = 0; i < 4; i++) s_res[par][half][rt4][4 * L.gb + i][t] = acc[tp][i];
                }
            }
        }
        const bool wsp = __any(special);
        if (lane == 0) s_special[par][wave] = wsp ? 1 : 0;
        lds_barrier();
        // Row tiles with special scales: the half-0 wave recomputes all 16
        // rows with the integer decode (workgroup-uniform test, so the
        // barrier after it is reached by every wave).
        bool any_special = false;
#pragma unroll
        for (int i = 0; i < kWaves; i++) any_special |= s_special[par][i] != 0;
        if (any_special) {
            if (half == 0 && (s_special[par][rt4] | s_special[par][rt4 + 4])) {
                const ByteView cview = make_view(view_base, a.expert_bytes);
                const int row_l = lane >> 2, sub = lane & 3;
                const int row = row0 + row_l;
                const uint32_t pos = (uint32_t)(row < a.rows ? row : 0) * row_bytes;
                for (int t = 0; t < pt.nt; t++) {
                    const uint32_t *codes = reinterpret_cast<const uint32_t *>(a.codes + (size_t)pick4(pt.arow, t) * nb * 32);
                    const float v = lut_row_dot(cview, pos, nb, codes, s_dx + t * nbp, sub);
                    if (sub == 0) {
                        s_res[par][0][rt4][row_l][t] = v;
                        s_res[par][1][rt4][row_l][t] = 0.0f;
                    }
                }
            }
            lds_barrier();
        }
        float(*res0)[16][kTokPerPass] = s_res[par][0];
        float(*res1)[16][kTokPerPass] = s_res[par][1];
        const uint32_t brow = (uint32_t)u.e * (uint32_t)a.rows + (uint32_t)(u.tile * tile_rows + erow);
        const int k = n_staged;
        if (tid == 0) {
            s_stage_tile[k] = u.tile;
            s_stage_nt[k] = pt.nt;
        }
        if (tid < kTokPerPass) s_stage_ent[k][tid] = pick4(pt.ent, tid);
        if constexpr (MODE == kGateUp) {
            // 32 rows x nt tokens (waves 0-1, a half-wave per token): bias,
            // clamped SwiGLU, and the Q8_0 block of the act row.
            if (wave < 2) {
                const int t = tid >> 5;
                const float b0 = bias_value(bv0, bw0, brow), b1 = bias_value(bv1, bw1, brow);
                const int rg = erow >> 4, ri = erow & 15;
                const float gv = (res0[rg][ri][t] + res1[rg][ri][t]) + b0;
                const float uv = (res0[2 + rg][ri][t] + res1[2 + rg][ri][t]) + b1;
                const float v = swiglu(gv, uv);
                uint16_t dh;
                const int qv = q8_quantize_half(v, lane, &dh);
                if (t < pt.nt) {
                    s_stage[k][0][t][erow] = v;
                    s_stage[k][1][t][erow] = gv;
                    s_stage[k][2][t][erow] = uv;
                    s_sq[k][t][erow] = (int8_t)qv;
                    const int pn = 2 * (erow & 15) + (erow >> 4);  // nibble position of element erow
                    s_smx[k][t][pn] = (uint8_t)e4m3_small(qv >> 4);
                    s_smx[k][t][32 + pn] = (uint8_t)e4m3_small(qv & 15);
                    if (erow == 0) s_sdh[k][t] = dh;
                }
            }
        } else {
            if (wave < 4) {
                const int t = tid >> 6;
                const float b0 = bias_value(bv0, bw0, brow);
                const int rg = erow >> 4, ri = erow & 15;
                if (t < pt.nt) s_stage[k][0][t][erow] = (res0[rg][ri][t] + res1[rg][ri][t]) + b0;
            }
        }
        ++n_staged;
#pragma unroll
        for (int p = 0; p < 2; p++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[p][i] = 0.0f;
        // the stage is complete before the next step's flush
        if (n_staged == kStage || w + 1 == w1) lds_barrier();
    }
    if (n_staged > 0) flush(n_staged);
}

hipError_t launch_mx_mfma(hipStream_t s, GemvMode mode, const MxMfmaArgs &a, int slots) {
    if (slots <= 0 || a.rows <= 0) return hipSuccess;
    if (a.nb <= 0 || a.nb > kMaxNb) return hipErrorInvalidConfiguration;
    const size_t nbp = (size_t)(a.nb + 7) / 8 * 8;
    const size_t lds = 4 * (size_t)tile_region(a.nb) + (size_t)kTokPerPass * nbp * (64 + 4) + nbp * 64;
    if (lds > kMaxMxLds) return hipErrorInvalidConfiguration;
    // one-time opt-in to more than 64 KB of dynamic LDS
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_mfma<kGateUp>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxMxLds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_mfma<kDown>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxMxLds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_mfma<kRows>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxMxLds);
        return e;
    }();
    if (attr != hipSuccess) return attr;
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    // Upper bound of the work items: every selection its own pass.
    const int tile_rows = mode == kGateUp ? 32 : 64;
    const int max_passes = mode == kRows ? (a.ntok + kTokPerPass - 1) / kTokPerPass : slots;
    const int64_t items = (int64_t)max_passes * ((a.rows + tile_rows - 1) / tile_rows);
    // one workgroup of eight waves per CU (its LDS holds four tile images)
    const int grid = items < n_cu ? (int)items : n_cu;
    if (mode == kGateUp) {
        hipLaunchKernelGGL(k_mx_mfma<kGateUp>, dim3(grid), dim3(kWG), lds, s, a, a.active, a.offsets, a.pass_off,
                           a.list, a.n_active);
    } else if (mode == kDown) {
        hipLaunchKernelGGL(k_mx_mfma<kDown>, dim3(grid), dim3(kWG), lds, s, a, a.active, a.offsets, a.pass_off,
                           a.list, a.n_active);
    } else {
        hipLaunchKernelGGL(k_mx_mfma<kRows>, dim3(grid), dim3(kWG), lds, s, a, a.active, a.offsets, a.pass_off,
                           a.list, a.n_active);
    }
    return hipGetLastError();
}

}  // namespace spt
