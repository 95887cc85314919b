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
// weight rows and walks K in segments of kKSeg = 16 blocks.  Each load
// instruction covers four rows x 16 consecutive blocks (four 272-byte
// runs), lane j taking row 4q + (j >> 4), block j & 15, as 20 aligned bytes;
// the 16 nibble bytes are realigned in registers and stored with the E8M0
// byte into the tile, where the MFMA's lane (g, i) reads row i, block 4c + g.
// Tile slots are XOR-swizzled (slot = block ^ row) so both the stores (16
// consecutive blocks of one row) and the MFMA reads (16 rows of one block)
// are free of bank conflicts.  Segments stream through a ring of NBUF
// register buffers, NBUF - 1 of them in flight while one is stored.
constexpr int kKSeg = 16;
constexpr int kRowsPerLoad = 64 / kKSeg;
constexpr int kSegLoads = 16 / kRowsPerLoad;
constexpr int kChunks = kKSeg / 4;
constexpr int kATile = 16 * kKSeg * 16;   // bytes of nibble data per wave
constexpr int kETile = 16 * kKSeg;        // bytes of E8M0 per wave
constexpr int kWaveLds = kATile + kETile;
constexpr uint32_t kOutOfRange = 0x80000000u;  // byte offset past any expert matrix (< 4 GiB)
constexpr size_t kMaxMxLds = 48 * 1024;        // dynamic LDS of three workgroups per CU within 160 KB

// Ring depth and occupancy per mode.  Gate/up carries the SwiGLU and the
// Q8_0 of act in its epilogue and runs two waves per SIMD with four
// segments in flight per wave; down and single-expert run three waves per
// SIMD with two in flight.
template <int MODE> struct MxTraits {
    static constexpr int kNBuf = MODE == kGateUp ? 5 : 3;
    static constexpr int kWavesPerEU = MODE == kGateUp ? 2 : 3;
    // Unit outputs staged in LDS before a flush, and the values staged per
    // row and token (gate/up: act, gate, up; down: the result).
    static constexpr int kStageUnits = MODE == kGateUp ? 8 : 6;
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
// for every outstanding global load, draining the weight segments in flight.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Static lane roles.  Loads: row lr = lane / kKSeg of each row group, block
// bl = lane % kKSeg of the segment.  MFMA A: row i = lane & 15, block gb =
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

// The weight stream is issued with inline assembly, out of sight of the
// compiler's wait-count analysis, and waited for explicitly (stream_wait):
// the compiler's analysis turns conservative (a full drain) at control-flow
// joins around stores and around the loop, which would empty the ring of
// segments in flight every step.  Loads complete in order, so waiting until
// at most N loads are outstanding, with N the number of stream loads issued
// after a segment, is exact whatever else was issued in between.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Buffer descriptor words, the layout __builtin_amdgcn_make_buffer_rsrc
// builds: base, base_hi | stride << 16 (stride 0), num_records, flags.
__device__ inline u32x4v rsrc_words(const void *base, uint32_t nrec) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4v{(uint32_t)a, (uint32_t)(a >> 32) & 0xFFFFu, nrec, (uint32_t)kRsrcWord3};
}

// A segment in registers: per load instruction q, the 16-byte word at the
// block's aligned start and the next dword; plus the raw bias words of the
// segment's unit (loaded first).
struct SegRegs {
    u32x4v q4[kSegLoads];
    uint32_t q1[kSegLoads];
    uint32_t b0, b1;
};

// One segment's stream loads in one block: the bias word(s), then per load
// instruction q the 16 bytes at off[q] and the dword after them.  The block
// opens with five wait states: descriptor SGPRs may have just been written
// by a VALU instruction (a spill reload), which a following VMEM read must
// not see early, and the compiler cannot pad inside inline assembly.
// Offsets past a descriptor's range read as zeros.
template <bool TWO_BIAS>
__device__ inline void stream_fetch(SegRegs &d, uint32_t bo0, uint32_t bo1, const u32x4v &brs0,
                                    const u32x4v &brs1, const uint32_t off[kSegLoads], const u32x4v &rs) {
    static_assert(kSegLoads == 4, "operand list below");
    if constexpr (TWO_BIAS) {
        asm volatile(
            "s_nop 4\n\t"
            "buffer_load_dword %0, %10, %12, 0 offen\n\t"
            "buffer_load_dword %1, %11, %13, 0 offen\n\t"
            "buffer_load_dwordx4 %2, %14, %18, 0 offen\n\t"
            "buffer_load_dword %6, %14, %18, 0 offen offset:16\n\t"
            "buffer_load_dwordx4 %3, %15, %18, 0 offen\n\t"
            "buffer_load_dword %7, %15, %18, 0 offen offset:16\n\t"
            "buffer_load_dwordx4 %4, %16, %18, 0 offen\n\t"
            "buffer_load_dword %8, %16, %18, 0 offen offset:16\n\t"
            "buffer_load_dwordx4 %5, %17, %18, 0 offen\n\t"
            "buffer_load_dword %9, %17, %18, 0 offen offset:16"
            : "=&v"(d.b0), "=&v"(d.b1), "=&v"(d.q4[0]), "=&v"(d.q4[1]), "=&v"(d.q4[2]), "=&v"(d.q4[3]),
              "=&v"(d.q1[0]), "=&v"(d.q1[1]), "=&v"(d.q1[2]), "=&v"(d.q1[3])
            : "v"(bo0), "v"(bo1), "s"(brs0), "s"(brs1), "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]),
              "s"(rs));
    } else {
        asm volatile(
            "s_nop 4\n\t"
            "buffer_load_dword %0, %9, %10, 0 offen\n\t"
            "buffer_load_dwordx4 %1, %11, %15, 0 offen\n\t"
            "buffer_load_dword %5, %11, %15, 0 offen offset:16\n\t"
            "buffer_load_dwordx4 %2, %12, %15, 0 offen\n\t"
            "buffer_load_dword %6, %12, %15, 0 offen offset:16\n\t"
            "buffer_load_dwordx4 %3, %13, %15, 0 offen\n\t"
            "buffer_load_dword %7, %13, %15, 0 offen offset:16\n\t"
            "buffer_load_dwordx4 %4, %14, %15, 0 offen\n\t"
            "buffer_load_dword %8, %14, %15, 0 offen offset:16"
            : "=&v"(d.b0), "=&v"(d.q4[0]), "=&v"(d.q4[1]), "=&v"(d.q4[2]), "=&v"(d.q4[3]), "=&v"(d.q1[0]),
              "=&v"(d.q1[1]), "=&v"(d.q1[2]), "=&v"(d.q1[3])
            : "v"(bo0), "s"(brs0), "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(rs));
        d.b1 = 0u;
    }
}

// Per-lane offsets of a segment's load instructions; a slot outside the
// matrix reads past the buffer's range, which returns zeros, so the number
// of stream loads per segment is fixed.
__device__ inline void seg_offsets(uint32_t p0, bool bin, uint32_t grp_step, uint32_t off[kSegLoads]) {
#pragma unroll
    for (int q = 0; q < kSegLoads; q++) off[q] = bin ? ((p0 + (uint32_t)q * grp_step) & ~3u) : kOutOfRange;
}

// Wait until at most N stream loads are outstanding; the segment's registers
// are operands, so nothing reads them before the wait.
template <int N>
__device__ inline void stream_wait(SegRegs &d) {
    static_assert(kSegLoads == 4, "operand list below");
    asm volatile("s_waitcnt vmcnt(%10)"
                 : "+v"(d.q4[0]), "+v"(d.q4[1]), "+v"(d.q4[2]), "+v"(d.q4[3]), "+v"(d.q1[0]), "+v"(d.q1[1]),
                   "+v"(d.q1[2]), "+v"(d.q1[3]), "+v"(d.b0), "+v"(d.b1)
                 : "n"(N));
}

// Realign the loaded blocks and store them into the wave's tile.  Blocks
// outside the matrix load as zeros and get scale 2^0, contributing 0; a
// block with a special E8M0 gets scale 2^0 and flags its rows, which are
// then recomputed with the integer decode.
__device__ inline void seg_store(const SegRegs &sr, uint32_t p0, bool bin, uint32_t grp_step,
                                 int row0, int rows, const LaneRole &L, uint4 *sA, uint8_t *sE, bool &special) {
#pragma unroll
    for (int q = 0; q < kSegLoads; q++) {
        const uint32_t d[5] = {sr.q4[q].x, sr.q4[q].y, sr.q4[q].z, sr.q4[q].w, sr.q1[q]};
        const int rl = kRowsPerLoad * q + L.lr;
        const bool in = bin && row0 + rl < rows;
        const uint32_t o = (p0 + (uint32_t)q * grp_step) & 3u;
        const uint32_t sel = 0x04030201u + o * 0x01010101u;
        const uint32_t ev = __builtin_amdgcn_ubfe(d[0], o * 8u, 8u);
        const bool normal = ev - (uint32_t)kEMin <= (uint32_t)(kEMax - kEMin);
        special |= in && !normal;
        uint4 nib;
        nib.x = __builtin_amdgcn_perm(d[1], d[0], sel);
        nib.y = __builtin_amdgcn_perm(d[2], d[1], sel);
        nib.z = __builtin_amdgcn_perm(d[3], d[2], sel);
        nib.w = __builtin_amdgcn_perm(d[4], d[3], sel);
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
#pragma unroll 1
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

// Position of the lead cursor in a workgroup's stream of weight segments.
// Work items are (slot, pass, tile) in that order, w = (pass_off[slot] +
// pass) * tiles + tile: slot = an active expert, pass = kTokPerPass tokens
// of its list, tile = a row tile; each item is nseg K segments.
struct Cursor {
    int w, slot, p, tile, ks, e, begin, count, npass;
    bool done;
};

// What a buffer holds, packed into three scalars: m0 = expert | ks << 16,
// m1 = tile | pass << 16, m2 = slot | done << 31.
struct Meta {
    uint32_t m0, m1, m2;
    __device__ int e() const { return (int)(m0 & 0xFFFFu); }
    __device__ int ks() const { return (int)(m0 >> 16); }
    __device__ int tile() const { return (int)(m1 & 0xFFFFu); }
    __device__ int p() const { return (int)(m1 >> 16); }
    __device__ int slot() const { return (int)(m2 & 0x7FFFFFFFu); }
    __device__ bool done() const { return (m2 >> 31) != 0; }
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
__device__ inline void cursor_advance(const MxMfmaArgs &a, const Route &rt, Cursor &c, int nseg, int tiles, int w1) {
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
    slot_info<MODE>(a, rt, c);
}

// Persistent workgroups: workgroup b takes work items [b*W/G, (b+1)*W/G)
// of the W = total passes x row tiles, in order, so consecutive items share
// an expert's token pass and its staged token tables, and every workgroup
// streams the same number of weight bytes.  Each wave streams its 16 rows
// segment after segment with the next NBUF - 1 segments in flight, across
// tile, pass and expert boundaries.  Gate/up units are 32 output rows
// (waves 0-1 gate, 2-3 up, so SwiGLU and the Q8_0 of the 32-element act
// block stay in the workgroup); down and single-expert units are 64 rows.
template <int MODE>
__global__ __launch_bounds__(kWG) __attribute__((amdgpu_waves_per_eu(MxTraits<MODE>::kWavesPerEU))) void k_mx_mfma(MxMfmaArgs a, const int32_t *__restrict__ r_active,
                                                                                  const int32_t *__restrict__ r_offsets,
                                                                                  const int32_t *__restrict__ r_pass_off,
                                                                                  const int32_t *__restrict__ r_list,
                                                                                  const int32_t *__restrict__ r_n_active) {
    extern __shared__ __align__(16) uint8_t smem_b[];
    // Output pointers of the epilogue, kept in LDS rather than in scalar
    // registers across the stream.
    struct EpiPtrs {
        float *out, *tap0, *tap1, *act_scales;
        int8_t *act_codes;
        uint8_t *act_mxtab, *act_blocks34;
    };
    __shared__ EpiPtrs s_epi;
    __shared__ int s_entry[kTokPerPass];
    __shared__ int s_arow[kTokPerPass];
    __shared__ float s_res[4][16][kTokPerPass];
    __shared__ __align__(16) uint8_t s_zero[16];
    // Outputs of finished units, written to global memory kStageUnits units
    // at a time.  Vector-memory stores and loads share one counter and may
    // complete out of order, so while a store is outstanding a wave can only
    // wait for all of its loads; flushing in batches keeps the weight
    // segments in flight across most unit boundaries.
    constexpr int kStage = MxTraits<MODE>::kStageUnits;
    constexpr int kUnitRows = MxTraits<MODE>::kUnitRows;
    __shared__ float s_stage[kStage][MxTraits<MODE>::kStageVals][kTokPerPass][kUnitRows];
    __shared__ int s_stage_ent[kStage][kTokPerPass];
    __shared__ int s_stage_tile[kStage];
    __shared__ int s_stage_nt[kStage];

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

    const int m = MODE == kGateUp ? (wave >> 1) : 0;
    const int roff = MODE == kGateUp ? (wave & 1) * 16 : wave * 16;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const uint32_t grp_step = (uint32_t)kRowsPerLoad * row_bytes;
    LaneRole L;
    L.lr = lane / kKSeg;
    L.bl = lane % kKSeg;
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
    if (tid == 0) s_epi = EpiPtrs{a.out, a.tap[0], a.tap[1], a.act_scales, a.act_codes, a.act_mxtab, a.act_blocks34};

    // Epilogue element of this thread: gate/up: row tid&31 of the unit,
    // token tid>>5; down/rows: row tid&63, token tid>>6.
    const int erow = MODE == kGateUp ? (tid & 31) : (tid & 63);
    const BiasView bv0 = make_bias_view(a.bias[0], a.bias_bytes[0], a.bias_type[0]);
    const BiasView bv1 = make_bias_view(a.bias[1], a.bias_bytes[1], a.bias_type[1]);
    auto bias_words = [](const void *p, uint64_t nbytes) {
        return rsrc_words(p, p ? (uint32_t)(nbytes < 0xFFFFFFF0ull ? nbytes : 0xFFFFFFF0ull) : 0u);
    };
    const u32x4v brs0 = bias_words(a.bias[0], a.bias_bytes[0]);
    const u32x4v brs1 = bias_words(a.bias[1], a.bias_bytes[1]);
    // expert matrices: 4-byte aligned base below the expert's first byte,
    // `lead` bytes before it (the same for every expert when expert_bytes is
    // a multiple of 4, else recomputed per expert)
    const uint8_t *wbase = a.w[m];

    Cursor lead;
    lead.w = w0;
    lead.slot = slot0;
    lead.p = MODE == kRows ? q0 : q0 - rt.pass_off[slot0];
    lead.tile = w0 - q0 * tiles;
    lead.ks = 0;
    lead.done = false;
    slot_info<MODE>(a, rt, lead);

    // Per-lane byte position (relative to the view's aligned base) of this
    // lane's first block of a segment, and whether that block exists.
    auto seg_pos = [&](int tile, int ks, bool done, uint32_t lead, uint32_t &p0, bool &bin) {
        const int blk = (done ? nseg : ks) * kKSeg + L.bl;
        bin = blk < nb;
        p0 = (uint32_t)(tile * tile_rows + roff + L.lr) * row_bytes + (uint32_t)blk * kMxBlock + lead;
    };
    // Stream descriptor of expert e's matrix and its lead.
    auto expert_words = [&](int e, uint32_t &lead) {
        const uintptr_t p = reinterpret_cast<uintptr_t>(wbase + (uint64_t)e * a.expert_bytes);
        lead = (uint32_t)(p & 3u);
        return rsrc_words(reinterpret_cast<const void *>(p - lead),
                          (uint32_t)((a.expert_bytes + lead + 3u) & ~uint64_t(3)));
    };
    // A buffer holds a segment's weights, its place, and the raw bias words
    // of its unit's epilogue element, loaded before the segment so that the
    // epilogue's wait for them never drains the segments in flight.
    struct SegBuf {
        SegRegs r;
        Meta m;
    };
    constexpr int kStreamPerSeg = 2 * kSegLoads + (MODE == kGateUp ? 2 : 1);
    auto fetch = [&](SegBuf &buf) {
        buf.m = Meta{(uint32_t)lead.e | ((uint32_t)lead.ks << 16), (uint32_t)lead.tile | ((uint32_t)lead.p << 16),
                     (uint32_t)lead.slot | (lead.done ? 0x80000000u : 0u)};
        const uint32_t brow = (uint32_t)lead.e * (uint32_t)a.rows + (uint32_t)(lead.tile * tile_rows + erow);
        // bias dword offsets as bias_raw computes them
        const uint32_t bo0 = bv0.type == 0 ? brow * 4u : (brow * 2u) & ~3u;
        const uint32_t bo1 = bv1.type == 0 ? brow * 4u : (brow * 2u) & ~3u;
        uint32_t ld;
        const u32x4v rs = expert_words(lead.e, ld);
        uint32_t p0, off[kSegLoads];
        bool bin;
        seg_pos(lead.tile, lead.ks, lead.done, ld, p0, bin);
        seg_offsets(p0, bin, grp_step, off);
        stream_fetch<MODE == kGateUp>(buf.r, bo0, bo1, brs0, brs1, off, rs);
        cursor_advance<MODE>(a, rt, lead, nseg, tiles, w1);
    };

    constexpr int NBUF = MxTraits<MODE>::kNBuf;
    SegBuf bufs[NBUF];
#pragma unroll
    for (int k = 0; k < NBUF - 1; k++) fetch(bufs[k]);

    int staged_slot = -1, staged_p = -1, nt = 0, npair = 0;
    PassRole PR;
    float acc[2][4];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[p][i] = 0.0f;
    bool special = false;

    // Write out the staged units (all waves).  Gate/up: wave-per-token act
    // rows, their Q8_0 block in every layout, and the gate/up taps; down:
    // thread-per-element results.
    int n_staged = 0;
    auto flush = [&](int count) {
        const EpiPtrs ep = s_epi;
        if constexpr (MODE == kGateUp) {
            for (int pi = wave; pi < count * kTokPerPass; pi += 4) {
                const int k = pi / kTokPerPass, t = pi % kTokPerPass;
                if (t >= s_stage_nt[k]) continue;
                const int tile = s_stage_tile[k], ent = s_stage_ent[k][t];
                const int r = tile * 32 + (lane & 31);
                const float v = lane < 32 ? s_stage[k][0][t][lane] : 0.0f;
                if (lane < 32 && r < a.rows) {
                    const size_t o = (size_t)ent * a.rows + r;
                    ep.out[o] = v;
                    if (ep.tap0) ep.tap0[o] = s_stage[k][1][t][lane];
                    if (ep.tap1) ep.tap1[o] = s_stage[k][2][t][lane];
                }
                // the unit is one Q8_0 block of the token's act row
                if (ep.act_codes && tile * 32 + 32 <= a.rows) {
                    uint16_t dh;
                    const int q = q8_quantize_lane(v, lane, &dh);
                    const size_t blk = (size_t)ent * (a.rows / 32) + tile;
                    write_q8_lane(q, dh, lane, blk, ep.act_codes, ep.act_scales, ep.act_mxtab, ep.act_blocks34);
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
        // Leave with the stores complete so the compiler's wait counts on
        // the streaming path stay exact.
        __builtin_amdgcn_s_waitcnt(0);
    };

    // One segment of the stream: cur is stored and multiplied, nxt is
    // refilled with the lead cursor's segment.
    auto step = [&](SegBuf &cur, SegBuf &nxt) -> bool {
        const Meta cm = cur.m;
        if (cm.done()) return true;
        const int ce = cm.e(), cks = cm.ks(), ctile = cm.tile(), cp = cm.p(), cslot = cm.slot();
        if (cks == 0 && (cslot != staged_slot || cp != staged_p)) {
            // New token set.  Every wave is past the previous epilogue's
            // final barrier, so the tables are free.
            const int begin = MODE == kRows ? 0 : rt.offsets[ce];
            const int count = MODE == kRows ? a.ntok : rt.offsets[ce + 1] - begin;
            nt = min(kTokPerPass, count - cp * kTokPerPass);
            npair = (nt + 1) >> 1;
            if (tid < kTokPerPass) {
                int ent = 0, arow = 0;
                if (tid < nt) {
                    ent = MODE == kRows ? cp * kTokPerPass + tid : rt.list[begin + cp * kTokPerPass + tid];
                    arow = MODE == kGateUp ? ent / a.topk : ent;
                }
                s_entry[tid] = ent;
                s_arow[tid] = arow;
            }
            lds_barrier();
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
            lds_barrier();
            staged_slot = cslot;
            staged_p = cp;
            // This rare path loads in loops; ending it with nothing
            // outstanding keeps the compiler's wait counts on the common
            // path exact.
            __builtin_amdgcn_s_waitcnt(0);
        }
        fetch(nxt);

        const int r0 = ctile * tile_rows + roff;
        const ByteView cview = make_view(wbase + (uint64_t)ce * a.expert_bytes, a.expert_bytes);
        // cur's loads are complete once no more than the later segments'
        // stream loads are outstanding
        stream_wait<(NBUF - 1) * kStreamPerSeg>(cur.r);
        {
            uint32_t p0;
            bool bin;
            seg_pos(ctile, cks, false, cview.lead, p0, bin);
            seg_store(cur.r, p0, bin, grp_step, r0, a.rows, L, sA, sE, special);
        }
        wave_lds_fence();
        seg_mfma(cks, npair, L, PR, s_zero, sA, sE, s_mx, reinterpret_cast<const uint8_t *>(s_dx), acc);
        wave_lds_fence();

        if (cks == nseg - 1) {
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
                __builtin_amdgcn_s_waitcnt(0);
            }
            lds_barrier();
            const int tile = ctile;
            const uint32_t brow = (uint32_t)ce * (uint32_t)a.rows + (uint32_t)(tile * tile_rows + erow);
            const int k = n_staged;
            if (tid == 0) {
                s_stage_tile[k] = tile;
                s_stage_nt[k] = nt;
            }
            if (tid < kTokPerPass) s_stage_ent[k][tid] = s_entry[tid];
            if constexpr (MODE == kGateUp) {
                // 32 rows x nt tokens: bias, clamped SwiGLU.
                const int t = tid >> 5;
                const float b0 = bias_value(bv0, cur.r.b0, brow), b1 = bias_value(bv1, cur.r.b1, brow);
                if (t < nt) {
                    const float gv = s_res[erow >> 4][erow & 15][t] + b0;
                    const float uv = s_res[2 + (erow >> 4)][erow & 15][t] + b1;
                    s_stage[k][0][t][erow] = swiglu(gv, uv);
                    s_stage[k][MxTraits<MODE>::kStageVals - 2][t][erow] = gv;
                    s_stage[k][MxTraits<MODE>::kStageVals - 1][t][erow] = uv;
                }
            } else {
                const int t = tid >> 6;
                const float b0 = bias_value(bv0, cur.r.b0, brow);
                if (t < nt) s_stage[k][0][t][erow] = s_res[erow >> 4][erow & 15][t] + b0;
            }
            if (++n_staged == kStage) {
                lds_barrier();
                flush(n_staged);
                n_staged = 0;
            }
            lds_barrier();
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[p][i] = 0.0f;
            special = false;
        }
        return false;
    };

    // The ring, unrolled so every buffer keeps fixed registers; leaving by
    // jump keeps the load count at the loop's back edge the same on every
    // path, so the compiler's wait counts stay exact.
    for (;;) {
#pragma unroll
        for (int k = 0; k < NBUF; k++) {
            if (step(bufs[k], bufs[(k + NBUF - 1) % NBUF])) goto ring_done;
        }
    }
ring_done:
    // The last NBUF - 1 fetches (past the end, reading zeros) are still in
    // flight and will write their registers; keep those registers reserved
    // until the loads have landed, so the code below cannot be handed a
    // register that a late load overwrites.
#pragma unroll
    for (int k = 0; k < NBUF; k++) stream_wait<0>(bufs[k].r);
    if (n_staged > 0) {
        lds_barrier();
        flush(n_staged);
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
    // workgroups of four waves: as many per CU as waves per SIMD
    const int per_cu = mode == kGateUp ? MxTraits<kGateUp>::kWavesPerEU : MxTraits<kDown>::kWavesPerEU;
    const int grid = items < per_cu * n_cu ? (int)items : per_cu * n_cu;
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
