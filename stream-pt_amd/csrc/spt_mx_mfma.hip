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
// value as the integer form isum * 2^(e-128) (isum = sum of 2*E2M1*q).  Each
// lane applies the activation scale to its own digit column,
//   acc = fma(D_part, d_x, acc),
// and the product is exact (D_part has at most 13 significant bits, the fp16
// d_x at most 11), so what rounds is only the fp32 adding of the two digit
// halves and of the blocks, in the lanes' and waves' order: with one block
// the result is the single rounding of isum * d_x * 2^(e-128).
// Rows of a 16-row tile that contain an E8M0 outside [4, 240] are computed
// with the integer LUT decode instead, so the results keep the reference's
// special-value semantics: 255 is the +Inf scale, and above 240 a D value
// (up to 2^(e-127) * 16 * 32 * 6 * 8 = 2^(e-112.4)) can overflow fp32 where
// the oracle's d_x * 2^(e-128) * isum stays finite; below 4 the smallest
// products (2^(e-128)) leave the normal range.
#include <type_traits>

#include "spt_device.h"
#include "spt_kernels.h"
#include "spt_mx_tile.h"

namespace spt {

constexpr int kTileGroups = (tile_loads(kMaxNb) + 3) / 4;  // groups of four 1 KB loads per tile
constexpr int kWaveGroups = (kTileGroups + 1) / 2;         // of them, loaded by one wave
constexpr size_t kMaxMxLds = 120 * 1024;  // dynamic LDS; with the static part (< 36 KB) within 160 KB
constexpr int kStageUnits = 2;             // units per stage set (two sets: one fills while the other is flushed)


// A wave's part of a tile image in flight: four loads of 1 KB per group,
// ordinary buffer loads whose waits the compiler places (before the LDS
// stores that read the registers).  Every step of the loop issues every
// group, at an offset past the descriptor's range (read as zeros, no
// memory traffic) when there is no next unit or the group is not the
// wave's, so that all paths into the loop's joins carry the same loads in
// the same order and the compiler's wait counts stay exact there (with the
// issue conditional it drained every load at the joins).  The loads are
// nontemporal (cache policy bit 1, `nt`): each weight byte is read once per
// pass and the stream is far larger than the caches, and a plain streaming
// read reaches about 7.0 TB/s with the bit against 6.1 TB/s without it on
// MI355X.
constexpr uint32_t kPastRange = 0x80000000u;
struct TileRegs {
    u32x4v q[4 * kWaveGroups];
};

template <int G, int K0, int K1>
__device__ inline void tile_issue(TileRegs &t, uint32_t vo, rsrc_t r, uint32_t so) {
#pragma unroll
    for (int k = K0; k < K1; k++)
        t.q[4 * G + k] = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(r, vo + 1024u * k, so, 2));
}

// After the stores of a step: the LDS writes are complete, so their data
// registers have been read before the next loads overwrite them.
__device__ inline void tile_stored(TileRegs &t) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(t.q[0]), "+v"(t.q[1]), "+v"(t.q[2]), "+v"(t.q[3]), "+v"(t.q[4]), "+v"(t.q[5]),
                   "+v"(t.q[6]), "+v"(t.q[7]), "+v"(t.q[8]), "+v"(t.q[9]), "+v"(t.q[10]), "+v"(t.q[11])::"memory");
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
// items [b*W/G, (b+1)*W/G) of the W = total passes x units, in order, so
// consecutive items share an expert's token pass.  Gate/up units are 32
// output rows (row tiles 0-1 gate, 2-3 up, so SwiGLU and the Q8_0 of the
// 32-element act block stay in the workgroup); down and single-expert units
// are 64 rows; a row tile is 16 rows.
//
// The waves split the unit's K range, not its rows: wave w multiplies chunks
// w, w + 8, w + 16 of all four row tiles, so its B operands (the pass's
// tokens, block-diagonal) are loaded into registers once per pass and each
// tile image in LDS is read once, as A.  Wave w streams half of tile
// (w & 3)'s image: the image's load groups are split between waves w and
// w ^ 4.  Each wave's partial row sums go to LDS, in two stage sets of
// kStage units; when a set is full, the workgroup adds the eight partials
// of each of its outputs in wave order during the next unit's multiply (and
// the rest at the end) and applies the epilogue: bias, and for gate/up the
// clamped SwiGLU and the Q8_0 of the act block.
//
// Each step: wait for this wave's prefetched groups; advance the cursor to
// the next unit; barrier (every wave is past the previous unit's multiply);
// write the groups to LDS, issuing the next unit's first load group after
// the first; barrier; multiply (tiles 0-1, then 2-3), issuing half of the
// second group before tiles 0-1 and half after them, the third likewise
// around tiles 2-3, and flushing a full stage set after the second group's
// first half; write the partial sums.  Measured alternatives, all
// slower for gate/up at 64 tokens: one wave role loading and another
// multiplying (208 us against 190 us at the time: one multiplying wave per
// SIMD leaves the LDS and MFMA latencies exposed), tile pairs streamed by
// LDS DMA into a two-deep ring (370 us: in-flight bytes drop to zero at
// every pair), and tile pairs as the step with two pair images in LDS and
// two pairs of loads in these registers (181 us against 168.5 us: with two
// pairs in flight every issue finds the CU's memory queue full, and the
// issuing wave stalls before its multiply).
template <int MODE>
__global__ __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(2))) void k_mx_mfma(MxMfmaArgs a, const int32_t *__restrict__ r_active,
                                                                      const int32_t *__restrict__ r_offsets,
                                                                      const int32_t *__restrict__ r_pass_off,
                                                                      const int32_t *__restrict__ r_list,
                                                                      const int32_t *__restrict__ r_n_active) {
    extern __shared__ __align__(16) uint8_t smem_b[];
    constexpr int kStage = kStageUnits;
    constexpr int kUnitRows = MODE == kGateUp ? 32 : 64;
    constexpr int kNBias = MODE == kGateUp ? 2 : 1;
    // Output pointers of the epilogue, kept in LDS rather than in scalar
    // registers across the loop.
    typedef __attribute__((address_space(1))) float gf32;
    typedef __attribute__((address_space(1))) int8_t gi8;
    typedef __attribute__((address_space(1))) uint8_t gu8;
    struct EpiPtrs {
        gf32 *out, *tap0, *tap1, *act_scales;
        gi8 *act_codes;
        gu8 *act_mxtab, *act_blocks34;
    };
    __shared__ EpiPtrs s_epi;
    // Per staged unit: partial row sums [wave][tile][row][token], the
    // waves' special-scale tile masks, biases, and where the unit's outputs go.
    __shared__ float s_part[2 * kStage][kWaves][4][16][kTokPerPass];
    __shared__ int s_special[2 * kStage][kWaves];
    __shared__ float s_bias[2 * kStage][kNBias][kUnitRows];
    __shared__ int s_stage_ent[2 * kStage][kTokPerPass];
    __shared__ int s_stage_tile[2 * kStage], s_stage_nt[2 * kStage], s_stage_e[2 * kStage];

    const int nb = a.nb;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const int ngroups = (tile_loads(nb) + 3) / 4;
    const int region = tile_region(nb);
    // wave-uniform: keeps per-wave descriptors and offsets in scalar registers
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rt4 = wave & 3, half = wave >> 2;  // the row tile this wave loads, and which half of its groups
    // load groups of this wave: [g0, g0 + gmine)
    const int g0 = half ? (ngroups + 1) / 2 : 0;
    const int gmine = half ? ngroups / 2 : (ngroups + 1) / 2;
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    // LDS address of this lane's 16 bytes of the first group this wave loads
    const uint32_t img_lds = (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)(smem_b + (size_t)rt4 * region)) +
                             4096u * (uint32_t)g0 + 16u * (uint32_t)lane;

    const int tile_rows = kUnitRows;
    const int tiles = (a.rows + tile_rows - 1) / tile_rows;
    const Route rt{r_active, r_offsets, r_pass_off, r_list};
    // The workgroup's item range and its first item's slot, expert and
    // pass: one load from the start table the packing wrote when there is
    // one, else found here (the expert count, the pass total and the slot
    // scan: three dependent round trips before the first weight load).
    // Workgroup b runs on XCD b % 8 (round-robin dispatch), each XCD with its
    // own L2: the item ranges are dealt XCD-major, so neighbouring ranges
    // (the passes of one expert, which read the same tiles at about the same
    // time) run on one XCD (measured: the 36-layer step at 64 tokens 9.99 ->
    // 9.91 ms, the 32-token Zipf layer 168.7 -> 166.3 us).
    const int G = gridDim.x;
    const int vb = (G % 8 == 0) ? ((int)blockIdx.x % 8) * (G / 8) + (int)blockIdx.x / 8 : (int)blockIdx.x;
    const bool table = MODE != kRows && a.start != nullptr;
    int w0, w1, slot0 = 0, e0 = a.expert, p0 = 0;
    if (table) {
        const int32_t *st = a.start + (size_t)vb * kGvStartWords;
        w0 = st[0];
        w1 = st[1];
        slot0 = st[2];
        e0 = st[3];
        p0 = st[4];
        if (w0 >= w1) return;
    } else {
        const int n_slots = MODE == kRows ? 1 : *r_n_active;
        const int P = MODE == kRows ? (a.ntok + kTokPerPass - 1) / kTokPerPass : rt.pass_off[n_slots];
        const int W = P * tiles;
        w0 = (int)((int64_t)vb * W / G);
        w1 = (int)((int64_t)(vb + 1) * W / G);
        if (w0 >= w1) return;
        // slot of the first item: the number of pass_off[s] <= w0 / tiles, minus 1
        if (MODE != kRows) {
            const int q = w0 / tiles;
            int ones = 0;
            for (int s0 = 0; s0 <= n_slots; s0 += kWG) {
                const int sidx = s0 + tid;
                ones += __syncthreads_count(sidx <= n_slots && rt.pass_off[sidx] <= q);
            }
            slot0 = ones - 1;
            e0 = rt.active[slot0];
        }
    }
    const int q0 = w0 / tiles;

    // matrix and first row (within the unit) of each row tile
    auto tile_m = [](int r) { return MODE == kGateUp ? (r >> 1) : 0; };
    auto tile_roff = [](int r) { return MODE == kGateUp ? (r & 1) * 16 : r * 16; };
    const int m_load = tile_m(rt4), roff_load = tile_roff(rt4);
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
    if (tid == 0)
        s_epi = EpiPtrs{(gf32 *)a.out,        (gf32 *)a.tap[0],    (gf32 *)a.tap[1],      (gf32 *)a.act_scales,
                        (gi8 *)a.act_codes, (gu8 *)a.act_mxtab, (gu8 *)a.act_blocks34};

    // Bias element of this thread (rows of a unit): threads tid < kUnitRows
    // stage row tid of each unit's biases.
    const int brow_l = tid & (kUnitRows - 1);
    const BiasView bv0 = make_bias_view(a.bias[0], a.bias_bytes[0], a.bias_type[0]);
    const BiasView bv1 = make_bias_view(a.bias[1], a.bias_bytes[1], a.bias_type[1]);
    const uint8_t *wload = a.w[m_load];

    Cursor cur;
    cur.w = w0;
    cur.slot = slot0;
    cur.tile = w0 - q0 * tiles;
    // The first unit's expert is all its tile loads need: they are issued
    // before its pass and token list are read (two dependent round trips
    // fewer before the first weights are in flight).
    cur.e = e0;

    // Registers of the next unit: this wave's groups of its tile image, and
    // the bias words of this thread's row.
    TileRegs tr;
    rsrc_t nrs = __builtin_amdgcn_make_buffer_rsrc(nullptr, (short)0, 0, kRsrcWord3);
    uint32_t na0 = 0u;
    bool nxt_ok = false;
    const uint32_t vo = 16u * (uint32_t)lane;
    // loads K0 .. K1-1 of local group G of the next tile's loads (compile-
    // time constants, so every issue block writes fixed registers).  The
    // wave issues them at the highest wave priority, so they go out ahead of
    // the other waves' MFMA and LDS work (gate/up at 64 tokens, four runs
    // each, alternating builds: 167.6-168.0 against 168.3-168.6 us; priority
    // 2: 168.0-168.5; priority 3 also over the image stores: 167.3-168.7).
    auto issue = [&](auto gc, auto k0, auto k1) {
        constexpr int G = decltype(gc)::value, K0 = decltype(k0)::value, K1 = decltype(k1)::value;
        static_assert(G < kWaveGroups && 0 <= K0 && K0 < K1 && K1 <= 4, "group");
        __builtin_amdgcn_s_setprio(3);
        tile_issue<G, K0, K1>(tr, vo, nrs, nxt_ok && G < gmine ? na0 + 4096u * G : kPastRange);
        __builtin_amdgcn_s_setprio(0);
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    using C4 = std::integral_constant<int, 4>;
    uint32_t b0r = 0u, b1r = 0u;
    auto prefetch = [&](const Cursor &c) {
        const uint32_t brow = (uint32_t)c.e * (uint32_t)a.rows + (uint32_t)(c.tile * tile_rows + brow_l);
        b0r = bias_raw(bv0, brow);
        if (MODE == kGateUp) b1r = bias_raw(bv1, brow);
        const int row0 = c.tile * tile_rows + roff_load;
        nxt_ok = false;
        if (row0 < a.rows) {
            // The expert matrix from the 16-byte boundary at or below its
            // first byte to the one at or above its end (a 16-byte load
            // that crosses the range's end reads zeros, and the bytes up to
            // that boundary share the last byte's page); loads past it read
            // zeros.  Bytes past the matrix only reach rows past a.rows.
            const uintptr_t mb = reinterpret_cast<uintptr_t>(wload + (uint64_t)c.e * a.expert_bytes);
            const uint32_t le = (uint32_t)(mb & 15u);
            const uint64_t base = mb - le;
            // descriptor words: base, base_hi (stride 0), num_records, format
            nrs = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(base), (short)0,
                                                    (int)(uint32_t)((a.expert_bytes + le + 15u) & ~15ull), kRsrcWord3);
            na0 = ((le + (uint32_t)row0 * row_bytes) & ~15u) + 4096u * (uint32_t)g0;
            nxt_ok = true;
        }
    };

    // Adds each output's eight partials in wave order and writes the staged
    // units out.  Row tiles with special scales are first recomputed with
    // the integer decode (their sums replace wave 0's partials, the others
    // zeroed).  Called by every thread after a barrier; the caller's next
    // barrier separates it from the stage's reuse.
    auto flush = [&](int base, int count) {
        int spec = 0;
        for (int k = 0; k < count; k++)
#pragma unroll
            for (int v = 0; v < kWaves; v++) spec |= s_special[base + k][v];
        if (spec) {
            for (int ci = wave; ci < 4 * count; ci += kWaves) {
                const int k = ci >> 2, r = ci & 3;
                int mask = 0;
#pragma unroll
                for (int v = 0; v < kWaves; v++) mask |= s_special[base + k][v];
                if (!((mask >> r) & 1)) continue;
                const int e = s_stage_e[base + k], nt = s_stage_nt[base + k];
                const int row0 = s_stage_tile[base + k] * tile_rows + tile_roff(r);
                const ByteView cview = make_view(a.w[tile_m(r)] + (uint64_t)e * a.expert_bytes, a.expert_bytes);
                const int row_l = lane >> 2, sub = lane & 3;
                const int row = row0 + row_l;
                const uint32_t pos = (uint32_t)(row < a.rows ? row : 0) * row_bytes;
                for (int t = 0; t < nt; t++) {
                    const int ent = s_stage_ent[base + k][t];
                    const int ar = MODE == kGateUp ? ent / a.topk : ent;
                    const uint32_t *codes = reinterpret_cast<const uint32_t *>(a.codes + (size_t)ar * nb * 32);
                    const float v = lut_row_dot(cview, pos, nb, codes, a.scales + (size_t)ar * nb, sub);
                    if (sub == 0) {
                        s_part[base + k][0][r][row_l][t] = v;
#pragma unroll
                        for (int q = 1; q < kWaves; q++) s_part[base + k][q][r][row_l][t] = 0.0f;
                    }
                }
            }
            lds_barrier();
        }
        const EpiPtrs ep = s_epi;
        if constexpr (MODE == kGateUp) {
            // thread: unit k, token t, act row e (a half-wave per token)
            const int k = tid >> 7, t = (tid >> 5) & 3, e = tid & 31;
            if (k < count) {
                const int rg = e >> 4, ri = e & 15;
                float gv = s_part[base + k][0][rg][ri][t], uv = s_part[base + k][0][2 + rg][ri][t];
#pragma unroll
                for (int v = 1; v < kWaves; v++) {
                    gv += s_part[base + k][v][rg][ri][t];
                    uv += s_part[base + k][v][2 + rg][ri][t];
                }
                gv += s_bias[base + k][0][e];
                uv += s_bias[base + k][kNBias - 1][e];
                const float act = swiglu(gv, uv);
                uint16_t dh;
                const int qv = q8_quantize_half(act, lane, &dh);
                const int tile = s_stage_tile[base + k];
                if (t < s_stage_nt[base + k]) {
                    const int ent = s_stage_ent[base + k][t];
                    const int r = tile * 32 + e;
                    if (r < a.rows) {
                        const size_t o = (size_t)ent * a.rows + r;
                        if (ep.out) ep.out[o] = act;
                        if (ep.tap0) ep.tap0[o] = gv;
                        if (ep.tap1) ep.tap1[o] = uv;
                    }
                    if (ep.act_codes && tile * 32 + 32 <= a.rows) {
                        const size_t blk = (size_t)ent * (a.rows / 32) + tile;
                        ep.act_codes[blk * 32 + e] = (int8_t)qv;
                        if (ep.act_mxtab) {
                            const int pn = 2 * (e & 15) + (e >> 4);  // nibble position of element e
                            ep.act_mxtab[blk * 64 + pn] = (uint8_t)e4m3_small(qv >> 4);
                            ep.act_mxtab[blk * 64 + 32 + pn] = (uint8_t)e4m3_small(qv & 15);
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
            }
        } else {
            for (int i = tid; i < count * kTokPerPass * kUnitRows; i += kWG) {
                const int k = i / (kTokPerPass * kUnitRows), t = (i / kUnitRows) % kTokPerPass, r = i % kUnitRows;
                const int row = s_stage_tile[base + k] * kUnitRows + r;
                if (t < s_stage_nt[base + k] && row < a.rows) {
                    const int rg = r >> 4, ri = r & 15;
                    float v = s_part[base + k][0][rg][ri][t];
#pragma unroll
                    for (int q = 1; q < kWaves; q++) v += s_part[base + k][q][rg][ri][t];
                    ep.out[(size_t)s_stage_ent[base + k][t] * a.rows + row] = v + s_bias[base + k][0][r];
                }
            }
        }
    };

    int staged_slot = -1, staged_p = -1, npair = 0;
    PassB pb;

    // stage slots kStage * set + i; a full set is flushed during the next
    // unit's multiply, after its first loads are issued
    int n_staged = 0, cur_set = 0, pending = -1;
    prefetch(cur);
    static_assert(kWaveGroups == 3, "issue list below");
    issue(C0{}, C0{}, C4{});
    issue(C1{}, C0{}, C4{});
    issue(C2{}, C0{}, C4{});
    cur.p = MODE == kRows ? q0 : table ? p0 : q0 - rt.pass_off[slot0];
    slot_info<MODE>(a, rt, cur);
    PassTokens npt = pass_tokens<MODE>(a, rt, cur);  // tokens of the unit in the registers

    for (int w = w0; w < w1; w++) {
        const Cursor u = cur;
        const PassTokens pt = npt;
        if (u.slot != staged_slot || u.p != staged_p) {
            // A new token pass: its B operands and d_x (pass changes are
            // rare: each workgroup walks a contiguous range of work items).
            load_pass_b(pb, a.nb, a.mxtab, a.scales, pt.arow, pt.nt, L, wave);
            npair = (pt.nt + 1) >> 1;
            staged_slot = u.slot;
            staged_p = u.p;
        }
        // The pass's B operands and the bias words are taken here, before
        // the next unit's loads are issued, so that no later use of them
        // waits on those loads (a wait covers every older load); a new
        // pass's B operands, loaded after this unit's tile loads, wait for
        // those too, as the image stores below would.
#pragma unroll
        for (int j = 0; j < kChunksPerWave; j++)
#pragma unroll
            for (int tp = 0; tp < 2; tp++) asm volatile("" : "+v"(pb.b[j][tp]), "+v"(pb.dx[j][tp]));
        uint32_t bw0 = b0r, bw1 = b1r;
        asm volatile("" : "+v"(bw0), "+v"(bw1));
        // the next unit's cursor and load addresses, before the barrier
        nxt_ok = false;
        if (w + 1 < w1) {
            cursor_advance<MODE>(a, rt, cur, tiles);
            if (cur.slot != u.slot || cur.p != u.p) npt = pass_tokens<MODE>(a, rt, cur);
            prefetch(cur);
        }
        // every wave is past the previous unit's multiply (its image reads)
        // and has written that unit's partial sums
        lds_barrier();
        const int row0_load = u.tile * tile_rows + roff_load;
        if (row0_load < a.rows) {
            static_assert(kWaveGroups == 3, "stores below");
            if (gmine > 0) tile_store<0>(img_lds, tr);
        }
        // the first group's registers are free once its stores are done
        tile_stored(tr);
        issue(C0{}, C0{}, C4{});
        if (row0_load < a.rows) {
            if (gmine > 1) tile_store<1>(img_lds + 4096u, tr);
            if (gmine > 2) tile_store<2>(img_lds + 8192u, tr);
        }
        // The next unit's first load group went out between the stores
        // (measured for gate/up at 64 tokens: 172 us; after all the stores
        // 176 us; a second group there too 189 us; none before the barrier
        // 188 us); after the barrier the images are in place.
        lds_barrier();
        const int k = kStage * cur_set + n_staged;
        if (tid < kUnitRows) {
            const uint32_t brow = (uint32_t)u.e * (uint32_t)a.rows + (uint32_t)(u.tile * tile_rows + tid);
            s_bias[k][0][tid] = bias_value(bv0, bw0, brow);
            if (MODE == kGateUp) s_bias[k][kNBias - 1][tid] = bias_value(bv1, bw1, brow);
        }
        if (tid == 0) {
            s_stage_tile[k] = u.tile;
            s_stage_nt[k] = pt.nt;
            s_stage_e[k] = u.e;
        }
        if (tid < kTokPerPass) s_stage_ent[k][tid] = pick4(pt.ent, tid);

        TileView tv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint8_t *vb = a.w[tile_m(r)] + (uint64_t)u.e * a.expert_bytes;
            const int row0 = u.tile * tile_rows + tile_roff(r);
            const uint32_t lead = (uint32_t)((reinterpret_cast<uintptr_t>(vb) & 15u) + (uint32_t)row0 * row_bytes) & 15u;
            tv[r] = tile_view(smem_b + (size_t)r * region, lead + (uint32_t)L.i * row_bytes, L);
        }
        // Two row tiles at a time: the wave's chunks of both, then their
        // partial sums (add the eight columns of each token slot, parts h/l
        // x blocks; lane j of each group of eight then holds token pair
        // j >> 2, row 4 * gb + (j & 3) of the slot: one store per tile).
        const int nchunks = (nb + 3) >> 2;
        // this wave's chunks wave + 8j < nchunks; only the last chunk of the
        // matrix can hold blocks past nb
        const int nc = nchunks > wave ? min(kChunksPerWave, (nchunks - 1 - wave) / kWaves + 1) : 0;
        const bool mask_last = nc > 0 && 4 * (wave + kWaves * (nc - 1)) + 3 >= nb;
        const int j8 = c16 & 7;
        int smask = 0;
#pragma unroll
        for (int r0 = 0; r0 < 4; r0 += 2) {
            float acc[2][2][4];
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int p = 0; p < 2; p++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[h][p][i] = 0.0f;
            // the next unit's second load group around the first tile
            // pair's multiplies, the third around the second's: half of the
            // group before, half after (a wave stalls at a load's issue
            // while its CU's memory queue is full, so each stall holds up
            // half as much of the multiply; measured for gate/up at 64
            // tokens: 168.6 against 169.8 us with whole groups before, 169.7
            // with whole groups after, 180 with the first group and half the
            // second before the first pair; both whole groups before the
            // first pair: 184 against 172 us)
            if (r0 == 0) {
                issue(C1{}, C0{}, C2{});
                if (pending >= 0) {
                    flush(kStage * pending, kStage);
                    pending = -1;
                }
            } else {
                issue(C2{}, C0{}, C2{});
            }
            if (npair == 2)
                tile_pair<2>(tv, r0, wave, nc, mask_last, nb, L, pb, acc);
            else
                tile_pair<1>(tv, r0, wave, nc, mask_last, nb, L, pb, acc);
            if (r0 == 0)
                issue(C1{}, C2{}, C4{});
            else
                issue(C2{}, C2{}, C4{});
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int r = r0 + h;
                float sm[2][4];
#pragma unroll
                for (int tp = 0; tp < 2; tp++)
#pragma unroll
                    for (int i = 0; i < 4; i++) sm[tp][i] = sum8(acc[h][tp][i]);
                float v = sm[0][0];
#pragma unroll
                for (int q = 1; q < 8; q++) v = j8 == q ? sm[q >> 2][q & 3] : v;
                s_part[k][wave][r][4 * L.gb + (j8 & 3)][2 * (j8 >> 2) + L.slot] = v;
                const int row0 = u.tile * tile_rows + tile_roff(r);
                if (__any(tile_special(tv[r], row0 + L.i < a.rows))) smask |= 1 << r;
            }
        }
        if (lane == 0) s_special[k][wave] = smask;
        if (++n_staged == kStage) {
            pending = cur_set;
            cur_set ^= 1;
            n_staged = 0;
        }
    }
    lds_barrier();
    if (pending >= 0) flush(kStage * pending, kStage);
    if (n_staged > 0) flush(kStage * cur_set, n_staged);
}

int mx_mfma_grid(GemvMode mode, const MxMfmaArgs &a, int slots) {
    if (slots <= 0 || a.rows <= 0) return 0;
    const int n_cu = device_cus();
    // Upper bound of the work items: every selection its own pass.
    const int tile_rows = mode == kGateUp ? 32 : 64;
    const int max_passes = mode == kRows ? (a.ntok + kTokPerPass - 1) / kTokPerPass : slots;
    const int64_t items = (int64_t)max_passes * ((a.rows + tile_rows - 1) / tile_rows);
    // one workgroup of eight waves per CU (its LDS holds four tile images)
    return items < n_cu ? (int)items : n_cu;
}

hipError_t launch_mx_mfma(hipStream_t s, GemvMode mode, const MxMfmaArgs &a, int slots) {
    if (slots <= 0 || a.rows <= 0) return hipSuccess;
    if (a.nb <= 0 || a.nb > kMaxNb) return hipErrorInvalidConfiguration;
    const size_t lds = 4 * (size_t)tile_region(a.nb);
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
    const int grid = mx_mfma_grid(mode, a, slots);
    if (a.start && grid > kGvStartMax) return hipErrorInvalidConfiguration;
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
