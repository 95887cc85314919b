// spt_mx_decode.hip -- the MoE layer at decode batch sizes (a few tokens,
// k <= 4): after the router, two launches instead of select, gate/up, down
// and combine.
//
//   k_dec_gate_up: a workgroup per (selection idx = token * k + rank, 32
//     act rows).  Its first wavefront takes the token's top-k from the
//     router logits (selectMoEBatch, forward/moe_batch.go:305-342; every
//     workgroup of the token computes the same bits), so the expert is known
//     one logits read after the launch and the unit's weight loads go out at
//     once.  Then gate and up rows of that expert for that token, bias,
//     clamped SwiGLU and the Q8_0 of the 32-element act block.  Selections
//     with Weight <= 0 are skipped, as the reference's grouping skips them
//     (moe_batch.go:150-157).
//   k_dec_down: a workgroup per (token, 16 output rows): the down rows of
//     the token's k selected experts, each against its own act row, bias,
//     then the weighted combine in rank order (moe_batch.go:163-192), so the
//     per-selection results never go through memory (they are written only
//     for the parity tap).
//
// A unit is four 16-row tiles in two pairs, on W waves (8 for gate/up, 16
// for down).  Waves W/2 p .. W/2 p + W/2 - 1 hold pair p's loads in
// registers (all issued at the start: about 98 KB per unit in flight); pair
// 0 is written to an LDS image of two tiles and multiplied by all W waves
// (K split: wave w takes chunks w, w+W, ... of four MXFP4 blocks), then
// pair 1 replaces it.  A workgroup needs two tile images (50 KB at 2880
// inputs): two gate/up workgroups run per CU, so a batch-1 layer's 360
// gate/up units are resident at once; its 180 down units take one CU each,
// with twice the waves, which halves each wave's share of the multiply
// (8.0 against 8.5 us per batch-1 launch, measured).  The MFMA arithmetic
// is that of the grouped
// GEMV (spt_mx_mfma.hip, spt_mx_tile.h): E2M1 weights as stored with their
// E8M0 as the A scale, the Q8_0 codes split into two exact E4M3 digits, and
// rows holding an E8M0 outside [4, 240] recomputed with the integer decode.
#include "spt_device.h"
#include "spt_kernels.h"
#include "spt_mx_tile.h"
#include "spt_select.h"

namespace spt {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A decode workgroup of W waves: W / 2 per pair of tiles, W / 4 per tile,
// each taking every (W / 4)-th 1 KB load of its tile's image; the K chunks of
// a multiply split over all W waves.
template <int W>
constexpr int pair_loads() { return (tile_loads(kMaxNb) + W / 4 - 1) / (W / 4); }
template <int W>
constexpr int dec_chunks() { return ((kMaxNb + 3) / 4 + W - 1) / W; }
constexpr int kGateUpWaves = 8, kDownWaves = 16;

// Where a tile's bytes come from: a descriptor over its expert matrix from
// the 16-byte boundary at or below the matrix's first byte (loads past the
// matrix read zeros), the offset of the tile's first 16-byte load in it, and
// the tile's first byte within that load.
struct TileSrc {
    rsrc_t rs;
    uint32_t start, lead;
};

__device__ inline TileSrc tile_src(const uint8_t *matrix, uint64_t matrix_bytes, int row0, uint32_t row_bytes) {
    const uintptr_t mb = reinterpret_cast<uintptr_t>(matrix);
    const uint32_t le = (uint32_t)(mb & 15u);
    TileSrc s;
    s.rs = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(mb - le), (short)0,
                                             (int)(uint32_t)((matrix_bytes + le + 15u) & ~15ull), kRsrcWord3);
    const uint32_t first = le + (uint32_t)row0 * row_bytes;
    s.start = first & ~15u;
    s.lead = first & 15u;
    return s;
}

// This wave's loads of its tile (loads h0, h0 + 2, ... of nl), nontemporal:
// each weight byte is read once.
template <int W>
struct PairRegs {
    u32x4 v[pair_loads<W>()];
};

// Issued unconditionally (a load this wave does not need reads past the
// descriptor's range, which returns zeros), so the compiler's wait counts
// stay exact: a wait for one of these loads never drains a later one.
template <int W>
__device__ inline void pair_issue(PairRegs<W> &pr, const TileSrc &s, int h0, int nl, bool on, int lane) {
#pragma unroll
    for (int j = 0; j < pair_loads<W>(); j++) {
        const int i = h0 + (W / 4) * j;
        const uint32_t off = (on && i < nl) ? s.start + 1024u * (uint32_t)i + 16u * (uint32_t)lane : 0xFFFFFFF0u;
        pr.v[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(s.rs, off, 0, 2 /* nt */));
    }
}

template <int W>
__device__ inline void pair_store(uint8_t *region, const PairRegs<W> &pr, int h0, int nl, int lane) {
#pragma unroll
    for (int j = 0; j < pair_loads<W>(); j++) {
        const int i = h0 + (W / 4) * j;
        if (i < nl) *reinterpret_cast<u32x4 *>(region + 1024 * i + 16 * lane) = pr.v[j];
    }
}

// The B operand of one chunk for the two token slots of an MFMA: lane (slot,
// part, gc) carries digit `part` of slot `slot`'s block 4c + gc, in the half
// of its 32 bytes that meets A's blocks (lo: gb >> 1, hi: (gb >> 1) + 2).
// Branch-free loads through descriptors over the activation tables (rows of
// nb blocks): the lanes and chunks without a block read past the range and
// get zeros.
struct ActTables {
    rsrc_t mx, sc;
};

__device__ inline ActTables act_tables(const uint8_t *mxtab, const float *scales, int rows, int nb) {
    const uint64_t nblk = (uint64_t)rows * (uint64_t)nb;
    ActTables t;
    t.mx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(mxtab), (short)0, (int)(uint32_t)(nblk * 64u), kRsrcWord3);
    t.sc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(scales), (short)0, (int)(uint32_t)(nblk * 4u), kRsrcWord3);
    return t;
}

struct ChunkB {
    u32x4v v;   // this lane's 16 digit bytes (zeros if none)
    float dx;   // the block's d_x (0 if none)
};

__device__ inline ChunkB chunk_b(const ActTables &t, int nb, int c, int arow, bool slot_on, const LaneRole &L) {
    const int blkc = 4 * c + L.gc;
    const bool ok = slot_on && blkc < nb;
    const uint32_t blk = (uint32_t)arow * (uint32_t)nb + (uint32_t)blkc;
    const uint32_t vo = (ok && (L.lo_on || L.hi_on)) ? blk * 64u + (uint32_t)L.boff : 0xFFFFFFF0u;
    const uint32_t so = ok ? blk * 4u : 0xFFFFFFF0u;
    ChunkB r;
    r.v = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(t.mx, vo, 0, 0));
    r.dx = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(t.sc, so, 0, 0));
    return r;
}

// The B operand of an MFMA from a lane's digit bytes: in the half of its 32
// bytes that meets A's blocks (lo: gb >> 1, hi: (gb >> 1) + 2).
__device__ inline v8i b_operand(const u32x4v &v, const LaneRole &L) {
    const u32x4v z = {0u, 0u, 0u, 0u};
    return L.lo_on ? __builtin_bit_cast(v8i, __builtin_shufflevector(v, z, 0, 1, 2, 3, 4, 5, 6, 7))
                   : __builtin_bit_cast(v8i, __builtin_shufflevector(z, v, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Chunk c (blocks 4c..4c+3) of the pair's two tiles: A operands from the
// image (E8M0 as the A scale; blocks past nb get scale 2^0 and add 0, their
// B and d_x being zero), one MFMA per tile, then the FMA of d_x.
__device__ __attribute__((always_inline)) inline void pair_chunk(TileView (&tv)[2], int c, bool last, int nb,
                                                                const LaneRole &L, const v8i &b, float dx,
                                                                float (&acc)[2][4]) {
    uint32_t d[2][5];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < 5; i++) d[h][i] = tv[h].pa[17 * c + i];
    v4f dd[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        TileView &v = tv[h];
        const uint32_t ev = __builtin_amdgcn_ubfe(d[h][0], v.esh, 8u);
        int sa = (int)ev;
        const bool in = !last || 4 * c + L.gb < nb;
        sa = in ? sa : 127;
        v.emin = in ? min(v.emin, ev) : v.emin;
        v.emax = in ? max(v.emax, ev) : v.emax;
        const v8i A = v8i{(int)__builtin_amdgcn_perm(d[h][1], d[h][0], v.sel), (int)__builtin_amdgcn_perm(d[h][2], d[h][1], v.sel),
                          (int)__builtin_amdgcn_perm(d[h][3], d[h][2], v.sel), (int)__builtin_amdgcn_perm(d[h][4], d[h][3], v.sel),
                          0, 0, 0, 0};
        const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
        dd[h] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, b, z, 4, 0, 0, sa, 0, L.sb);
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int k = 0; k < 4; k++) acc[h][k] = __builtin_fmaf(dd[h][k], dx, acc[h][k]);
}

// The unit's per-tile partial row sums: [wave][tile][row], for the token
// slot each tile is multiplied against.
template <int W>
struct DecShared {
    float part[W][4][16];
    int special[W];
};

// Multiplies the pair in the image (tiles 2p, 2p+1 with views tv) over this
// wave's chunks and stores its partial sums for token slot slot_of(h);
// returns the pair's special-scale tile bits (tile 2p + h) for rows in range.
template <int W, class SlotOf>
__device__ __attribute__((always_inline)) inline int pair_multiply(TileView (&tv)[2], int p, int nb, int wave,
                                                                  const LaneRole &L, const ChunkB (&cb)[dec_chunks<W>()],
                                                                  DecShared<W> &sh, SlotOf slot_of, const bool (&row_ok)[2]) {
    float acc[2][4];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int k = 0; k < 4; k++) acc[h][k] = 0.0f;
    const int nchunks = (nb + 3) >> 2;
#pragma unroll
    for (int j = 0; j < dec_chunks<W>(); j++) {
        const int c = wave + W * j;
        if (c < nchunks) pair_chunk(tv, c, 4 * c + 3 >= nb, nb, L, b_operand(cb[j].v, L), cb[j].dx, acc);
    }
    const int lane = threadIdx.x & 63, j8 = lane & 7;
    int smask = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        // add the eight columns of each token slot (digits h/l x blocks):
        // lane j8 < 4 of a slot's group then stores row 4 * gb + j8
        float sm[4];
#pragma unroll
        for (int k = 0; k < 4; k++) sm[k] = sum8(acc[h][k]);
        const float v = j8 == 0 ? sm[0] : j8 == 1 ? sm[1] : j8 == 2 ? sm[2] : sm[3];
        if (L.slot == slot_of(h) && j8 < 4) sh.part[wave][2 * p + h][4 * L.gb + j8] = v;
        if (__any(tile_special(tv[h], row_ok[h]))) smask |= 1 << (2 * p + h);
    }
    return smask;
}

}  // namespace

// ---------------------------------------------------------------------------
// gate/up
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64 * kGateUpWaves) __attribute__((amdgpu_waves_per_eu(4))) void k_dec_gate_up(DecGateUpArgs da) {
    const MxMfmaArgs &a = da.g;
    extern __shared__ __align__(16) uint8_t smem_b[];
    constexpr int W = kGateUpWaves;
    __shared__ DecShared<W> sh;
    __shared__ int32_t s_ids[kMaxTopK];
    __shared__ float s_w[kMaxTopK];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int units = a.rows >> 5;
    const int idx = blockIdx.x / units, u = blockIdx.x - idx * units;
    const int k = a.topk, t = idx / k, r = idx - t * k;
    // the token's top-k into LDS (only LDS pointers, so no flat accesses: a
    // pending flat access would make every later LDS access wait for every
    // load in flight); one workgroup per token writes the selections out
    if (wave == 0)
        select_token(load_token_logits(da.logits + (size_t)t * da.experts, da.experts), da.experts, k, s_ids, s_w,
                     nullptr, nullptr);
    lds_barrier();
    if (u == 0 && r == 0 && tid < k) {
        typedef __attribute__((address_space(1))) int32_t gi32;
        typedef __attribute__((address_space(1))) float gf32;
        reinterpret_cast<gi32 *>(reinterpret_cast<uintptr_t>(da.ids))[(size_t)t * k + tid] = s_ids[tid];
        reinterpret_cast<gf32 *>(reinterpret_cast<uintptr_t>(da.weights))[(size_t)t * k + tid] = s_w[tid];
    }
    const int e = s_ids[r];
    if (s_w[r] <= 0.0f) return;  // not grouped (a NaN weight is kept)

    // tiles: 0 gate rows 32u..32u+15, 1 up rows 32u.., 2 gate rows 32u+16.., 3 up rows 32u+16..
    const int nb = a.nb;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const int nl = tile_loads(nb), region = tile_region(nb);
    const int pair = wave / (W / 2), q = wave % (W / 2), my_tile = 2 * pair + (q & 1), h0 = q >> 1;
    auto tile_row0 = [&](int T) { return 32 * u + 16 * (T >> 1); };
    auto tile_matrix = [&](int T) { return a.w[T & 1] + (uint64_t)e * a.expert_bytes; };
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
    // Loads in this order: the token's B operands (slot 0) for this wave's
    // chunks and the biases (small, from L2), then the unit's weights, so
    // that waiting for the former never drains the latter.
    const ActTables xt = act_tables(a.mxtab, a.scales, da.tab_rows, nb);
    ChunkB cb[dec_chunks<W>()];
#pragma unroll
    for (int j = 0; j < dec_chunks<W>(); j++) cb[j] = chunk_b(xt, nb, wave + W * j, t, L.slot == 0, L);
    // the gate and up bias words of act row 32u + (lane & 31), kept in
    // registers until the epilogue (wave 0 adds them)
    const BiasView bv0 = make_bias_view(a.bias[0], a.bias_bytes[0], a.bias_type[0]);
    const BiasView bv1 = make_bias_view(a.bias[1], a.bias_bytes[1], a.bias_type[1]);
    const uint32_t bidx = (uint32_t)e * (uint32_t)a.rows + (uint32_t)(32 * u + (lane & 31));
    const uint32_t braw0 = bias_raw(bv0, bidx), braw1 = bias_raw(bv1, bidx);
    __builtin_amdgcn_sched_barrier(0);  // keep the small loads ahead of the weights
    PairRegs<W> pr;
    {
        const TileSrc src = tile_src(tile_matrix(my_tile), a.expert_bytes, tile_row0(my_tile), row_bytes);
        pair_issue(pr, src, h0, nl, tile_row0(my_tile) < a.rows, lane);
    }
    auto slot0 = [](int) { return 0; };
    int smask = 0;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        if (pair == p) pair_store(smem_b + (size_t)(my_tile & 1) * region, pr, h0, nl, lane);
        lds_barrier();
        TileView tv[2];
        bool row_ok[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int T = 2 * p + h;
            const uint32_t lead = tile_src(tile_matrix(T), a.expert_bytes, tile_row0(T), row_bytes).lead;
            tv[h] = tile_view(smem_b + (size_t)h * region, lead + (uint32_t)L.i * row_bytes, L);
            row_ok[h] = tile_row0(T) + L.i < a.rows;
        }
        smask |= pair_multiply<W>(tv, p, nb, wave, L, cb, sh, slot0, row_ok);
        lds_barrier();  // the image is free for the next pair; partial sums in place
    }
    if (lane == 0) sh.special[wave] = smask;
    lds_barrier();
    int spec = 0;
#pragma unroll
    for (int v = 0; v < W; v++) spec |= sh.special[v];
    if (spec) {
        // tiles with an E8M0 outside [kEMin, kEMax]: wave T recomputes tile
        // T's rows with the integer decode (four lanes per row)
        if (wave < 4 && ((spec >> wave) & 1)) {
            const int T = wave, row_l = lane >> 2, sub = lane & 3, row = tile_row0(T) + row_l;
            const ByteView cv = make_view(tile_matrix(T), a.expert_bytes);
            const uint32_t pos = (uint32_t)(row < a.rows ? row : 0) * row_bytes;
            const uint32_t *codes = reinterpret_cast<const uint32_t *>(a.codes + (size_t)t * nb * 32);
            const float v = lut_row_dot(cv, pos, nb, codes, a.scales + (size_t)t * nb, sub);
            if (sub == 0) {
                sh.part[0][T][row_l] = v;
#pragma unroll
                for (int w = 1; w < W; w++) sh.part[w][T][row_l] = 0.0f;
            }
        }
        lds_barrier();
    }
    if (wave == 0) {
        // act row 32u + el: the eight partials of gate and up in wave order,
        // bias, SwiGLU, then the block's Q8_0 (the two half-waves compute
        // the same block; the first stores it)
        const int el = lane & 31, Tg = el < 16 ? 0 : 2, ri = el & 15;
        float gv = sh.part[0][Tg][ri], uv = sh.part[0][Tg + 1][ri];
#pragma unroll
        for (int v = 1; v < W; v++) {
            gv += sh.part[v][Tg][ri];
            uv += sh.part[v][Tg + 1][ri];
        }
        gv += bias_value(bv0, braw0, bidx);
        uv += bias_value(bv1, braw1, bidx);
        const float act = swiglu(gv, uv);
        uint16_t dh;
        const int qv = q8_quantize_half(act, lane, &dh);
        if (lane < 32) {
            const size_t o = (size_t)idx * a.rows + 32 * u + el;
            if (a.out) a.out[o] = act;
            if (a.tap[0]) a.tap[0][o] = gv;
            if (a.tap[1]) a.tap[1][o] = uv;
            write_q8_lane(qv, dh, el, (size_t)idx * (a.rows >> 5) + u, a.act_codes, a.act_scales, a.act_mxtab,
                          a.act_blocks34, nullptr);
        }
    }
}

// ---------------------------------------------------------------------------
// down + combine
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64 * kDownWaves) __attribute__((amdgpu_waves_per_eu(4))) void k_dec_down(DecDownArgs da) {
    const MxMfmaArgs &a = da.g;
    extern __shared__ __align__(16) uint8_t smem_b[];
    constexpr int W = kDownWaves;
    __shared__ DecShared<W> sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int units = a.rows >> 4;
    const int t = blockIdx.x / units, u = blockIdx.x - t * units;
    const int k = a.topk;
    // tile T: rank T's expert, rows 16u..16u+15, against act row t*k + T
    int ex[4];
    float wt[4];
    bool on[4];
#pragma unroll
    for (int T = 0; T < 4; T++) {
        ex[T] = T < k ? da.ids[(size_t)t * k + T] : 0;
        wt[T] = T < k ? da.weights[(size_t)t * k + T] : 0.0f;
        on[T] = T < k && !(wt[T] <= 0.0f);
    }
    const int nb = a.nb;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const int nl = tile_loads(nb), region = tile_region(nb);
    const int pair = wave / (W / 2), q = wave % (W / 2), my_tile = 2 * pair + (q & 1), h0 = q >> 1;
    const int row0 = 16 * u;
    auto pick = [](const int (&v)[4], int T) { return T == 0 ? v[0] : T == 1 ? v[1] : T == 2 ? v[2] : v[3]; };
    auto pickb = [](const bool (&v)[4], int T) { return T == 0 ? v[0] : T == 1 ? v[1] : T == 2 ? v[2] : v[3]; };
    auto tile_matrix = [&](int T) { return a.w[0] + (uint64_t)pick(ex, T) * a.expert_bytes; };
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
    // pair p: tiles 2p (slot 0), 2p + 1 (slot 1); this lane's slot reads act
    // row t*k + 2p + slot.  Loads in this order: pair 0's B operands and the
    // biases, the unit's weights, then pair 1's B operands (needed only
    // after pair 1's weights), so no wait drains a load issued after it.
    const ActTables at = act_tables(a.mxtab, a.scales, da.tab_rows, nb);
    ChunkB cb[2][dec_chunks<W>()];
#pragma unroll
    for (int j = 0; j < dec_chunks<W>(); j++) cb[0][j] = chunk_b(at, nb, wave + W * j, t * k + L.slot, pickb(on, L.slot), L);
    // each rank's bias word of row row0 + (tid & 15), kept in registers until
    // the epilogue (threads tid < 16 add them)
    const BiasView bv = make_bias_view(a.bias[0], a.bias_bytes[0], a.bias_type[0]);
    auto bias_index = [&](int T) { return (uint32_t)pick(ex, T) * (uint32_t)a.rows + (uint32_t)(row0 + (tid & 15)); };
    uint32_t braw[4];
#pragma unroll
    for (int T = 0; T < 4; T++) braw[T] = bias_raw(bv, bias_index(T));
    __builtin_amdgcn_sched_barrier(0);  // keep the small loads ahead of the weights
    PairRegs<W> pr;
    {
        const TileSrc src = tile_src(tile_matrix(my_tile), a.expert_bytes, row0, row_bytes);
        pair_issue(pr, src, h0, nl, pickb(on, my_tile), lane);
    }
#pragma unroll
    for (int j = 0; j < dec_chunks<W>(); j++)
        cb[1][j] = chunk_b(at, nb, wave + W * j, t * k + 2 + L.slot, pickb(on, 2 + L.slot), L);
    auto slot_h = [](int h) { return h; };
    int smask = 0;
#pragma unroll
    for (int p = 0; p < 2; p++) {
        if (pair == p) pair_store(smem_b + (size_t)(my_tile & 1) * region, pr, h0, nl, lane);
        lds_barrier();
        TileView tv[2];
        bool row_ok[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int T = 2 * p + h;
            const uint32_t lead = tile_src(tile_matrix(T), a.expert_bytes, row0, row_bytes).lead;
            tv[h] = tile_view(smem_b + (size_t)h * region, lead + (uint32_t)L.i * row_bytes, L);
            row_ok[h] = pickb(on, T) && row0 + L.i < a.rows;
        }
        if (on[2 * p] || on[2 * p + 1]) smask |= pair_multiply<W>(tv, p, nb, wave, L, cb[p], sh, slot_h, row_ok);
        lds_barrier();
    }
    if (lane == 0) sh.special[wave] = smask;
    lds_barrier();
    int spec = 0;
#pragma unroll
    for (int v = 0; v < W; v++) spec |= sh.special[v];
    if (spec) {
        if (wave < 4 && ((spec >> wave) & 1)) {
            const int T = wave, row_l = lane >> 2, sub = lane & 3, row = row0 + row_l;
            const ByteView cv = make_view(tile_matrix(T), a.expert_bytes);
            const uint32_t pos = (uint32_t)(row < a.rows ? row : 0) * row_bytes;
            const size_t ar = (size_t)t * k + T;
            const uint32_t *codes = reinterpret_cast<const uint32_t *>(a.codes + ar * nb * 32);
            const float v = lut_row_dot(cv, pos, nb, codes, a.scales + ar * nb, sub);
            if (sub == 0) {
                sh.part[0][T][row_l] = v;
#pragma unroll
                for (int w = 1; w < W; w++) sh.part[w][T][row_l] = 0.0f;
            }
        }
        lds_barrier();
    }
    if (tid < 16) {
        // per rank: the eight partials in wave order + bias (the result of
        // selection t*k + T), then out = fma(result, weight, out) in rank
        // order from 0, skipping Weight <= 0
        const int row = row0 + tid;
        float o = 0.0f;
#pragma unroll
        for (int T = 0; T < 4; T++) {
            if (!on[T]) continue;
            float v = sh.part[0][T][tid];
#pragma unroll
            for (int w = 1; w < W; w++) v += sh.part[w][T][tid];
            v += bias_value(bv, braw[T], bias_index(T));
            if (da.results) da.results[((size_t)t * k + T) * a.rows + row] = v;
            o = __builtin_fmaf(v, wt[T], o);
        }
        if (row < a.rows) da.out[(size_t)t * a.rows + row] = o;
    }
}

size_t dec_lds(int nb) { return 2 * (size_t)tile_region(nb); }

hipError_t launch_dec_gate_up(hipStream_t s, const DecGateUpArgs &a, int n_sel) {
    if (n_sel <= 0 || a.g.rows <= 0) return hipSuccess;
    if (a.g.nb <= 0 || a.g.nb > kMaxNb || a.g.topk > kDecMaxTopK || (a.g.rows & 31)) return hipErrorInvalidConfiguration;
    const int units = a.g.rows >> 5;
    hipLaunchKernelGGL(k_dec_gate_up, dim3(n_sel * units), dim3(64 * kGateUpWaves), dec_lds(a.g.nb), s, a);
    return hipGetLastError();
}

hipError_t launch_dec_down(hipStream_t s, const DecDownArgs &a, int batch) {
    if (batch <= 0 || a.g.rows <= 0) return hipSuccess;
    if (a.g.nb <= 0 || a.g.nb > kMaxNb || a.g.topk > kDecMaxTopK || (a.g.rows & 15)) return hipErrorInvalidConfiguration;
    const int units = a.g.rows >> 4;
    hipLaunchKernelGGL(k_dec_down, dim3(batch * units), dim3(64 * kDownWaves), dec_lds(a.g.nb), s, a);
    return hipGetLastError();
}

}  // namespace spt
