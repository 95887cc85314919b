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
constexpr int kTokPerPass = kGemvTokens;  // two MFMA token slots x two MFMAs per chunk
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

// Weights reach the MFMA through a wave-private LDS tile.  A wave owns 16
// weight rows and walks K in segments of kKSeg = 32 blocks.  Each load
// instruction covers two rows x 32 consecutive blocks (two 544-byte runs),
// lane j taking row 2q + (j >> 5), block j & 31, as 20 aligned bytes; the
// 16 nibble bytes are realigned in registers and stored with the E8M0 byte
// into the tile, where the MFMA's lane (g, i) reads row i, block 4c + g.
// Tile slots are XOR-swizzled (slot = block ^ row) so both the stores (32
// consecutive blocks of one row) and the MFMA reads (16 rows of one block)
// are free of bank conflicts.
constexpr int kKSeg = 32;
constexpr int kChunks = kKSeg / 4;
constexpr int kSegLoads = 8;
constexpr int kATile = 16 * kKSeg * 16;  // bytes of nibble data per wave
constexpr int kETile = 16 * kKSeg;       // bytes of E8M0 per wave
constexpr int kWaveLds = kATile + kETile;
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr size_t kMaxMxLds = 128 * 1024;  // dynamic LDS of two workgroups per CU stays within 160 KB  // byte offset past any expert matrix (< 4 GiB)

// Orders a wave's accesses to its own LDS tile for the compiler (the hardware
// executes one wave's LDS instructions in order).
__device__ inline void wave_lds_fence() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
}

// Static lane roles.  Loads: row lr = lane >> 5 of each row pair, block
// bl = lane & 31 of the segment.  MFMA A: row i = lane & 15, block gb =
// lane >> 4 of each chunk.  MFMA B: column c = 8*slot + 4*part + gc holds
// digit `part` of token `slot`'s block gc; its non-zero half is lo (A blocks
// gb>>1) or hi (A blocks (gb>>1)+2) of this lane, or neither.
struct LaneRole {
    int lr, bl, i, gb, gc, slot, boff, sb;
    bool lo_on, hi_on;
};

// Per token pass: LDS byte offsets of this lane's B rows and d_x entries for
// each token pair, at block 0 (add 64 * block / 4 * block).  A half that is
// off reads 16 zero bytes instead.
struct PassRole {
    uint32_t tb[2], db[2];
    bool lo[2], hi[2];
};

__device__ inline void seg_load(const ByteView &view, uint32_t p0, bool bin, uint32_t pair_step,
                                uint32_t d[kSegLoads][5]) {
    // Unconditional loads (a slot outside the matrix reads past the buffer's
    // range, which returns zeros) keep the load count static, so the
    // compiler's wait counts let the next segment stay in flight.
#pragma unroll
    for (int q = 0; q < kSegLoads; q++) {
        const uint32_t base = bin ? ((p0 + (uint32_t)q * pair_step) & ~3u) : kOutOfRange;
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(view.r, base, 0, 0));
        d[q][0] = v.x;
        d[q][1] = v.y;
        d[q][2] = v.z;
        d[q][3] = v.w;
        d[q][4] = __builtin_amdgcn_raw_buffer_load_b32(view.r, base + 16u, 0, 0);
    }
}

// Realign the loaded blocks and store them into the wave's tile.  Blocks
// outside the matrix load as zeros and get scale 2^0, contributing 0; a
// block with a special E8M0 gets scale 2^0 and flags its rows, which are
// then recomputed with the integer decode.
__device__ inline void seg_store(const uint32_t d[kSegLoads][5], uint32_t p0, bool bin, uint32_t pair_step,
                                 int row0, int rows, const LaneRole &L, uint4 *sA, uint8_t *sE, bool &special) {
#pragma unroll
    for (int q = 0; q < kSegLoads; q++) {
        const int rl = 2 * q + L.lr;
        const bool in = bin && row0 + rl < rows;
        const uint32_t o = (p0 + (uint32_t)q * pair_step) & 3u;
        const uint32_t sel = 0x04030201u + o * 0x01010101u;
        const uint32_t ev = __builtin_amdgcn_ubfe(d[q][0], o * 8u, 8u);
        const bool normal = ev - (uint32_t)kEMin <= (uint32_t)(kEMax - kEMin);
        special |= in && !normal;
        uint4 nib;
        nib.x = __builtin_amdgcn_perm(d[q][1], d[q][0], sel);
        nib.y = __builtin_amdgcn_perm(d[q][2], d[q][1], sel);
        nib.z = __builtin_amdgcn_perm(d[q][3], d[q][2], sel);
        nib.w = __builtin_amdgcn_perm(d[q][4], d[q][3], sel);
        sA[rl * kKSeg + (L.bl ^ rl)] = nib;
        sE[rl * kKSeg + L.bl] = (uint8_t)(in && normal ? ev : 127u);
    }
}

// MFMAs of one segment: for each chunk c of 4 blocks, A from the tile and
// up to two token pairs of B from the staged digit tables (padded to whole
// segments with zeros); each lane accumulates its own column,
// acc[tp][k] += D[k] * d_x (the h and l columns are summed per unit).
__device__ inline void seg_mfma(int ks, int npair, const LaneRole &L, const PassRole &P, const uint8_t *s_zero,
                                const uint4 *sA, const uint8_t *sE, const uint8_t *s_mx, const uint8_t *s_dxb,
                                float acc[2][4]) {
#pragma unroll 2
    for (int c = 0; c < kChunks; c++) {
        const uint4 a4 = sA[L.i * kKSeg + ((4 * c + L.gb) ^ L.i)];
        const int sa = sE[L.i * kKSeg + 4 * c + L.gb];
        const v8i A = {(int)a4.x, (int)a4.y, (int)a4.z, (int)a4.w, 0, 0, 0, 0};
        const uint32_t blk0 = (uint32_t)(ks * kKSeg + 4 * c);  // uniform
#pragma unroll
        for (int tp = 0; tp < 2; tp++) {
            if (tp >= npair) break;
            const uint32_t at = P.tb[tp] + blk0 * 64u;
            const uint4 lo = *reinterpret_cast<const uint4 *>(P.lo[tp] ? s_mx + at : s_zero);
            const uint4 hi = *reinterpret_cast<const uint4 *>(P.hi[tp] ? s_mx + at : s_zero);
            const v8i B = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
            const float dx = *reinterpret_cast<const float *>(s_dxb + P.db[tp] + blk0 * 4u);
            v4f dd = {0.0f, 0.0f, 0.0f, 0.0f};
            dd = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, dd, 4, 0, 0, sa, 0, L.sb);
#pragma unroll
            for (int k = 0; k < 4; k++) acc[tp][k] = __builtin_fmaf(dd[k], dx, acc[tp][k]);
        }
    }
}

// Position in a workgroup's stream of weight segments.  Work items are
// (slot, pass, tile) in that order, w = (pass_off[slot] + pass) * tiles +
// tile: slot = an active expert, pass = kTokPerPass tokens of its list,
// tile = a row tile; each item is nseg K segments.
struct Cursor {
    int w, slot, p, tile, ks, e, begin, count, npass;
    bool done;
};

template <int MODE>
__device__ inline void slot_info(const MxMfmaArgs &a, Cursor &c) {
    if (MODE == kRows) {
        c.e = a.expert;
        c.begin = 0;
        c.count = a.ntok;
    } else {
        c.e = a.active[c.slot];
        c.begin = a.offsets[c.e];
        c.count = a.offsets[c.e + 1] - c.begin;
    }
    c.npass = (c.count + kTokPerPass - 1) / kTokPerPass;
}

template <int MODE>
__device__ inline void cursor_advance(const MxMfmaArgs &a, Cursor &c, int nseg, int tiles, int w1) {
    if (c.done) return;
    if (++c.ks < nseg) return;
    c.ks = 0;
    if (++c.w >= w1) {
        c.done = true;
        return;
    }
    if (++c.tile < tiles) return;
    c.tile = 0;
    if (++c.p < c.npass) return;
    c.p = 0;
    ++c.slot;
    slot_info<MODE>(a, c);
}

// Persistent workgroups: workgroup b takes work items [b*W/G, (b+1)*W/G)
// of the W = total passes x row tiles, in order, so consecutive items share
// an expert's token pass and its staged token tables, and every workgroup
// streams the same number of weight bytes.  Each wave streams its 16 rows
// segment after segment with the next segment always in flight, across
// tile, pass and expert boundaries.  Gate/up units are 32 output rows (waves
// 0-1 gate, 2-3 up, so SwiGLU and the Q8_0 of the 32-element act block stay
// in the workgroup); down and single-expert units are 64 rows.
template <int MODE>
__global__ __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(2))) void k_mx_mfma(MxMfmaArgs a) {
    extern __shared__ __align__(16) uint8_t smem_b[];
    __shared__ int s_entry[kTokPerPass];
    __shared__ int s_arow[kTokPerPass];
    __shared__ float s_res[4][16][kTokPerPass];
    __shared__ float s_act[kTokPerPass][32];
    __shared__ __align__(16) uint8_t s_zero[16];

    const int nb = a.nb;
    const int nseg = (nb + kKSeg - 1) / kKSeg;
    const int nbp = nseg * kKSeg;  // token tables padded with zero blocks
    // wave-uniform: keeps the per-wave buffer descriptors in scalar registers
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // LDS: per-wave weight tiles, then [tok][nbp][64] digit tables, [tok][nbp] d_x
    uint4 *sA = reinterpret_cast<uint4 *>(smem_b + (size_t)wave * kATile);
    uint8_t *sE = smem_b + 4 * kATile + wave * kETile;
    uint8_t *s_mx = smem_b + 4 * kWaveLds;
    float *s_dx = reinterpret_cast<float *>(s_mx + (size_t)kTokPerPass * nbp * 64);

    const int tile_rows = MODE == kGateUp ? 32 : 64;
    const int tiles = (a.rows + tile_rows - 1) / tile_rows;
    const int n_slots = MODE == kRows ? 1 : *a.n_active;
    const int P = MODE == kRows ? (a.ntok + kTokPerPass - 1) / kTokPerPass : a.pass_off[n_slots];
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
            ones += __syncthreads_count(sidx <= n_slots && a.pass_off[sidx] <= q0);
        }
        slot0 = ones - 1;
    }

    const int m = MODE == kGateUp ? (wave >> 1) : 0;
    const int roff = MODE == kGateUp ? (wave & 1) * 16 : wave * 16;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const uint32_t pair_step = 2u * row_bytes;
    LaneRole L;
    L.lr = lane >> 5;
    L.bl = lane & 31;
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
    if (tid < 4) reinterpret_cast<uint32_t *>(s_zero)[tid] = 0u;

    // Epilogue element of this thread: gate/up: row tid&31 of the unit,
    // token tid>>5; down/rows: row tid&63, token tid>>6.
    const int erow = MODE == kGateUp ? (tid & 31) : (tid & 63);
    const BiasView bv0 = make_bias_view(a.bias[0], a.bias_bytes[0], a.bias_type[0]);
    const BiasView bv1 = make_bias_view(a.bias[1], a.bias_bytes[1], a.bias_type[1]);

    Cursor c;
    c.w = w0;
    c.slot = slot0;
    c.p = MODE == kRows ? q0 : q0 - a.pass_off[slot0];
    c.tile = w0 - q0 * tiles;
    c.ks = 0;
    c.done = false;
    slot_info<MODE>(a, c);
    Cursor l = c;
    cursor_advance<MODE>(a, l, nseg, tiles, w1);

    // Per-lane byte position (relative to the view's aligned base) of this
    // lane's first block of a segment, and whether that block exists.
    auto seg_pos = [&](const Cursor &k, const ByteView &v, uint32_t &p0, bool &bin) {
        const int blk = (k.done ? nseg : k.ks) * kKSeg + L.bl;
        bin = blk < nb;
        p0 = (uint32_t)(k.tile * tile_rows + roff + L.lr) * row_bytes + (uint32_t)blk * kMxBlock + v.lead;
    };
    // A buffer holds a segment's weights and the raw bias words of its
    // unit's epilogue element, loaded together before the segment so that
    // the epilogue's wait for them never drains the segment in flight.
    struct SegBuf {
        uint32_t d[kSegLoads][5];
        uint32_t b0, b1;
    };
    auto fetch = [&](const Cursor &k, const ByteView &v, SegBuf &buf) {
        const uint32_t brow = (uint32_t)k.e * (uint32_t)a.rows + (uint32_t)(k.tile * tile_rows + erow);
        buf.b0 = bias_raw(bv0, brow);
        buf.b1 = MODE == kGateUp ? bias_raw(bv1, brow) : 0u;
        uint32_t p0;
        bool bin;
        seg_pos(k, v, p0, bin);
        seg_load(v, p0, bin, pair_step, buf.d);
    };

    ByteView cview = make_view(a.w[m] + (uint64_t)c.e * a.expert_bytes, a.expert_bytes);
    SegBuf buf0, buf1;
    fetch(c, cview, buf0);

    int staged_slot = -1, staged_p = -1, nt = 0, npair = 0;
    PassRole PR;
    float acc[2][4];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[p][i] = 0.0f;
    bool special = false;

    // One segment of the stream: cur holds segment c, nxt receives segment l.
    auto step = [&](SegBuf &cur, SegBuf &nxt) -> bool {
        if (c.ks == 0 && (c.slot != staged_slot || c.p != staged_p)) {
            // New token set.  Every wave is past the previous epilogue's
            // final barrier, so the tables are free.
            nt = min(kTokPerPass, c.count - c.p * kTokPerPass);
            npair = (nt + 1) >> 1;
            if (tid < kTokPerPass) {
                int ent = 0, arow = 0;
                if (tid < nt) {
                    ent = MODE == kRows ? c.p * kTokPerPass + tid : a.list[c.begin + c.p * kTokPerPass + tid];
                    arow = MODE == kGateUp ? ent / a.topk : ent;
                }
                s_entry[tid] = ent;
                s_arow[tid] = arow;
            }
            __syncthreads();
            // Tables of the nt tokens, zero past block nb; d_x zero past nb
            // and for the unused token slots.
            const int mxw = nbp * 16;  // dwords of digit table per token
            for (int t = 0; t < nt; t++) {
                uint32_t *dst = reinterpret_cast<uint32_t *>(s_mx + (size_t)t * nbp * 64);
                const uint32_t *src = reinterpret_cast<const uint32_t *>(a.mxtab + (size_t)s_arow[t] * nb * 64);
                for (int i = tid; i < mxw; i += kWG) dst[i] = i < nb * 16 ? src[i] : 0u;
            }
            for (int i = tid; i < kTokPerPass * nbp; i += kWG) {
                const int t = i / nbp, b = i - t * nbp;
                s_dx[i] = (t < nt && b < nb) ? a.scales[(size_t)s_arow[t] * nb + b] : 0.0f;
            }
#pragma unroll
            for (int tp = 0; tp < 2; tp++) {
                const int t = 2 * tp + L.slot;
                PR.tb[tp] = (uint32_t)((t * nbp + L.gc) * 64 + L.boff);
                PR.db[tp] = (uint32_t)((t * nbp + L.gc) * 4);
                PR.lo[tp] = L.lo_on && t < nt;
                PR.hi[tp] = L.hi_on && t < nt;
            }
            __syncthreads();
            staged_slot = c.slot;
            staged_p = c.p;
        }
        const ByteView lview = l.done ? cview : make_view(a.w[m] + (uint64_t)l.e * a.expert_bytes, a.expert_bytes);
        fetch(l, lview, nxt);
        const uint32_t brow = (uint32_t)c.e * (uint32_t)a.rows + (uint32_t)(c.tile * tile_rows + erow);

        const int r0 = c.tile * tile_rows + roff;
        {
            uint32_t p0;
            bool bin;
            seg_pos(c, cview, p0, bin);
            seg_store(cur.d, p0, bin, pair_step, r0, a.rows, L, sA, sE, special);
        }
        wave_lds_fence();
        seg_mfma(c.ks, npair, L, PR, s_zero, sA, sE, s_mx, reinterpret_cast<const uint8_t *>(s_dx), acc);
        wave_lds_fence();

        if (c.ks == nseg - 1) {
            // Sum the eight columns of each token slot (parts h/l x blocks).
#pragma unroll
            for (int tp = 0; tp < 2; tp++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float v = acc[tp][i];
                    v += __shfl_xor(v, 4, 8);
                    v += __shfl_xor(v, 1, 4);
                    v += __shfl_xor(v, 2, 4);
                    acc[tp][i] = v;
                }
            if ((c16 & 7) == 0) {
#pragma unroll
                for (int tp = 0; tp < 2; tp++) {
                    const int t = 2 * tp + L.slot;
                    if (t < nt) {
#pragma unroll
                        for (int i = 0; i < 4; i++) s_res[wave][4 * L.gb + i][t] = acc[tp][i];
                    }
                }
            }
            // Rows with special scales: recompute with the integer decode.
            if (__any(special)) {
                const int row_l = lane >> 2, sub = lane & 3;
                const int row = r0 + row_l;
                const uint32_t pos = (uint32_t)(row < a.rows ? row : 0) * row_bytes;
                for (int t = 0; t < nt; t++) {
                    const uint32_t *codes = reinterpret_cast<const uint32_t *>(a.codes + (size_t)s_arow[t] * nb * 32);
                    float v = lut_row_dot(cview, pos, nb, codes, s_dx + t * nbp, sub);
                    if (sub == 0) s_res[wave][row_l][t] = v;
                }
            }
            __syncthreads();
            const int tile = c.tile;
            if (MODE == kGateUp) {
                // 32 rows x nt tokens: bias, clamped SwiGLU, taps.
                const int t = tid >> 5;
                const int r = tile * 32 + erow;
                const float b0 = bias_value(bv0, cur.b0, brow), b1 = bias_value(bv1, cur.b1, brow);
                if (t < nt && r < a.rows) {
                    const float gv = s_res[erow >> 4][erow & 15][t] + b0;
                    const float uv = s_res[2 + (erow >> 4)][erow & 15][t] + b1;
                    const float act = swiglu(gv, uv);
                    const size_t o = (size_t)s_entry[t] * a.rows + r;
                    a.out[o] = act;
                    if (a.tap[0]) a.tap[0][o] = gv;
                    if (a.tap[1]) a.tap[1][o] = uv;
                    s_act[t][erow] = act;
                }
                __syncthreads();
                // The unit is one Q8_0 block of every token's act row: wave t
                // quantizes token t's block, one element per lane.
                if (wave < nt && a.act_codes && tile * 32 + 32 <= a.rows) {
                    const float v = lane < 32 ? s_act[wave][lane] : 0.0f;
                    uint16_t dh;
                    const int q = q8_quantize_lane(v, lane, &dh);
                    const size_t blk = (size_t)s_entry[wave] * (a.rows / 32) + tile;
                    write_q8_lane(q, dh, lane, blk, a.act_codes, a.act_scales, a.act_mxtab, a.act_blocks34);
                }
            } else {
                const int t = tid >> 6;
                const int r = tile * 64 + erow;
                const float b0 = bias_value(bv0, cur.b0, brow);
                if (t < nt && r < a.rows) a.out[(size_t)s_entry[t] * a.rows + r] = s_res[erow >> 4][erow & 15][t] + b0;
            }
            __syncthreads();
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[p][i] = 0.0f;
            special = false;
        }
        c = l;
        cview = lview;
        if (c.done) return true;
        cursor_advance<MODE>(a, l, nseg, tiles, w1);
        return false;
    };

    for (;;) {
        if (step(buf0, buf1)) break;
        if (step(buf1, buf0)) break;
    }
}

hipError_t launch_mx_mfma(hipStream_t s, GemvMode mode, const MxMfmaArgs &a, int slots) {
    if (slots <= 0 || a.rows <= 0) return hipSuccess;
    const int nbp = (a.nb + kKSeg - 1) / kKSeg * kKSeg;
    const size_t lds = 4 * (size_t)kWaveLds + (size_t)kTokPerPass * nbp * (64 + 4);
    if (lds > kMaxMxLds) return hipErrorInvalidConfiguration;
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
    const int grid = items < 2 * n_cu ? (int)items : 2 * n_cu;  // two workgroups per CU fit the LDS
    if (mode == kGateUp) {
        hipLaunchKernelGGL(k_mx_mfma<kGateUp>, dim3(grid), dim3(kWG), lds, s, a);
    } else if (mode == kDown) {
        hipLaunchKernelGGL(k_mx_mfma<kDown>, dim3(grid), dim3(kWG), lds, s, a);
    } else {
        hipLaunchKernelGGL(k_mx_mfma<kRows>, dim3(grid), dim3(kWG), lds, s, a);
    }
    return hipGetLastError();
}

}  // namespace spt
