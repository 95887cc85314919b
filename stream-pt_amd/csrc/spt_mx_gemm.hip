// spt_mx_gemm.hip -- grouped MXFP4 x Q8_0 GEMM for large expert groups on the
// gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// An expert whose list holds many selections (batched prefill) is a real
// contraction: its weight rows are multiplied with up to 64 list entries per
// pass instead of kGemvTokens.  The per-block arithmetic stays exact:
//   A (16 rows x 32 K): the weights of one MXFP4 block, decoded to bf16 by
//     v_cvt_scalef32_pk_bf16_fp4 with the block scale 2^(e-127); every value
//     E2M1 * 2^(e-127) has at most two significant bits, so it is exact for
//     e in [2, 252];
//   B (32 K x 16 tokens): the entries' Q8_0 codes as bf16 (|q| <= 127, exact);
//   D = sum over the block of A*B: every product is a multiple of 2^(e-128)
//     and |isum| <= 48,768 < 2^24, so D = isum * 2^(e-128) exactly (every
//     partial sum is representable), for e in [4, 240] (above 240 D can
//     overflow fp32 where the oracle's isum * (d_x * 2^(e-128)) does not);
//   acc = fma(D, d_x, acc) per block -- the value of the integer form
//     fma(float(isum), d_x * 2^(e-128), acc).
// K order inside a block: lane group g of the MFMA (k = 8g .. 8g+7) takes
// nibble bytes 1+4g .. 4+4g of the block; byte p gives the bf16 pair
// (element 4g+p, element 4g+p+16) -- the low and high nibble -- so the B
// table of a token holds, per block, the dwords
//   j = 0..15: bf16(q[j]) | bf16(q[j+16]) << 16.
// Rows with an E8M0 outside [4, 240] anywhere in K are recomputed with the
// integer LUT decode (rare; keeps the reference's Inf/NaN semantics).
//
// MFMA lane layout (measured on the hardware): lane l holds A row l%16 and B
// column l%16 at k = 8*(l/16) + 0..7; D lane l, register r is row
// 4*(l/16) + r, column l%16.
#include <type_traits>

#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 256;               // weight rows per work item (gate/up: 128 gate + 128 up)
constexpr int kBN = kGemmTokens;       // list entries per work item
constexpr int kSeg = 8;                // 32-element blocks per K segment (136 bytes of a row)
constexpr int kStages = 2;             // LDS stages; the next segment is in flight while one is multiplied
// A stage: row r's window (the segment's bytes from the 16-byte boundary at
// or below its first byte) in 10 slots of 16 bytes (16-byte aligned loads:
// a load crossing the end of the descriptor's range would read zeros for all
// its bytes).  The 64 lanes of a DMA load fill 64 consecutive slots, so a
// stage's 256 x 10 slots take 40 loads per workgroup, five per wave; loads
// 0-19 hold rows 0-127.
constexpr int kAPieces = 10;
constexpr int kASlots = kAPieces;
constexpr int kARow = 16 * kASlots;
constexpr int kAInstr = kBM * kASlots / 64;
// B stage: per entry 32 slots of 16 bytes (8 blocks x 4 quarters of the bf16
// code table); quarter piece p of entry t sits in slot p ^ (t & 15), so the
// 16 entries of an MFMA fragment read 16 different bank groups.
constexpr int kOffB = kBM * kARow;
constexpr int kOffD = kOffB + kBN * kSeg * 64;  // d_x [entry][kSeg]
constexpr int kStageBytes = kOffD + kBN * kSeg * 4;
constexpr int kEMin = 4, kEMax = 240;
constexpr int kXcds = 8;  // accelerator complex dies of an MI355X
constexpr uint32_t kOOR = 0x80000000u;  // buffer offset past every range: reads zero
static_assert(kSeg * kMxBlock + 15 <= 16 * kAPieces, "A window");
static_assert(kAInstr % kWaves == 0 && kBN * kSeg * 4 % kThreads == 0, "stage loads");
static_assert(kBM / 2 * kASlots % 64 == 0, "gate rows fill whole A loads");
static_assert(kBN * kSeg == 64 * kWaves, "one d_x load per wave");
constexpr int kALoads = kAInstr / kWaves;           // 5
constexpr int kBLoads = kBN * kSeg * 4 / kThreads;  // 4


// Integer-decode dot of one weight row with one entry's Q8_0 row (the
// special-scale fallback).
__device__ float lut_dot(const ByteView &v, uint32_t row_pos, int nb, const int8_t *codes, const float *scales) {
    float acc = 0.0f;
    const uint32_t *cw = reinterpret_cast<const uint32_t *>(codes);
    for (int b = 0; b < nb; b++) {
        uint32_t d[5], o;
        load_block5(v, row_pos + (uint32_t)b * kMxBlock, d, &o);
        MxDecoded dec;
        mx_decode(d, o, dec);
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = cw[b * 8 + k];
        const int32_t s = mx_isum(dec, q);
        acc = __builtin_fmaf((float)s, mx_block_scale(scales[b], dec.e), acc);
    }
    return acc;
}


// Descriptor of expert e's matrix from the 16-byte boundary at or below its
// first byte to the one at or above its end (a 16-byte load crossing the
// range's end reads zeros; the bytes up to that boundary share the last
// byte's page); *le = the matrix's offset in its first 16 bytes.
__device__ inline u32x4v expert_rsrc(const uint8_t *w, uint64_t expert_bytes, int e, uint32_t *le) {
    const uintptr_t mb = reinterpret_cast<uintptr_t>(w + (uint64_t)e * expert_bytes);
    *le = (uint32_t)(mb & 15u);
    const uint64_t b = mb - *le;
    return u32x4v{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, (uint32_t)((expert_bytes + *le + 15u) & ~15ull),
                  (uint32_t)kRsrcWord3};
}

// Workgroup barrier that leaves the LDS DMA loads in flight: the caller has
// already waited for what it needs (s_waitcnt in inline assembly, out of
// sight of the compiler's own wait insertion).
__device__ inline void stage_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Four bytes of the stage at byte offset o (any alignment): two aligned
// dwords and a byte shift (an unaligned LDS dword read returns the same
// bytes but is far slower).
__device__ __attribute__((always_inline)) inline uint32_t nibble_word(const uint8_t *st, uint32_t o) {
    const uint32_t *pw = reinterpret_cast<const uint32_t *>(st + (o & ~3u));
    return __builtin_amdgcn_alignbyte(pw[1], pw[0], o & 3u);
}

// One full segment (kSeg blocks) with NTF token fragments, straight-line:
// the A bytes of all blocks first, the B fragments and d_x one block ahead,
// then per block its A decode, MFMAs and the FMAs that apply d_x (the two
// waves of a SIMD overlap one's FMAs with the other's MFMAs).
template <int NTF>
__device__ __attribute__((always_inline)) inline void seg_full(const uint8_t *st, const uint32_t (&a_img)[2],
                                                               const uint32_t (&b_lane)[kSeg], int g, int i16,
                                                               float (&acc)[2][4][4], uint32_t (&emin)[2],
                                                               uint32_t (&emax)[2]) {
    uint32_t eb[kSeg][2], w4[kSeg][2];
#pragma unroll
    for (int j = 0; j < kSeg; j++)
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            eb[j][rf] = st[a_img[rf] + 17 * j];
            w4[j][rf] = nibble_word(st, a_img[rf] + 17u * (uint32_t)j + 1u + 4u * (uint32_t)g);
        }
    bf16x8 Bv[2][NTF];
    float dx[2][NTF];
    auto load_b = [&](int j) {
#pragma unroll
        for (int tf = 0; tf < NTF; tf++) {
            Bv[j & 1][tf] = *reinterpret_cast<const bf16x8 *>(st + kOffB + tf * (16 * kSeg * 64) + b_lane[j]);
            dx[j & 1][tf] = *reinterpret_cast<const float *>(st + kOffD + ((16 * tf + i16) * kSeg + j) * 4);
        }
    };
    load_b(0);
#pragma unroll
    for (int j = 0; j < kSeg; j++) {
        if (j + 1 < kSeg) load_b(j + 1);
        v4f D[2][NTF];
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const float sc = __uint_as_float(eb[j][rf] << 23);
            u32x4 av;
            av.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4[j][rf], sc, 0));
            av.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4[j][rf], sc, 1));
            av.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4[j][rf], sc, 2));
            av.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4[j][rf], sc, 3));
            const bf16x8 A = __builtin_bit_cast(bf16x8, av);
#pragma unroll
            for (int tf = 0; tf < NTF; tf++)
                D[rf][tf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, Bv[j & 1][tf], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        }
#pragma unroll
        for (int rf = 0; rf < 2; rf++)
#pragma unroll
            for (int tf = 0; tf < NTF; tf++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rf][tf][r] = __builtin_fmaf(D[rf][tf][r], dx[j & 1][tf], acc[rf][tf][r]);
    }
#pragma unroll
    for (int rf = 0; rf < 2; rf++)
#pragma unroll
        for (int j = 0; j < kSeg; j += 2) {
            emin[rf] = min(emin[rf], min(eb[j][rf], eb[j + 1][rf]));
            emax[rf] = max(emax[rf], max(eb[j][rf], eb[j + 1][rf]));
        }
}
static_assert(kSeg % 2 == 0, "seg_full's exponent reduction");

// The last segment when it holds jn < kSeg blocks.
template <int NTF>
__device__ __attribute__((always_inline)) inline void seg_part(const uint8_t *st, const uint32_t (&a_img)[2],
                                                               const uint32_t (&b_lane)[kSeg], int g, int i16, int jn,
                                                               float (&acc)[2][4][4], uint32_t (&emin)[2],
                                                               uint32_t (&emax)[2]) {
    for (int j = 0; j < jn; j++) {
        bf16x8 A[2];
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const uint32_t eb = st[a_img[rf] + 17 * j];
            const uint32_t w4 = nibble_word(st, a_img[rf] + 17u * (uint32_t)j + 1u + 4u * (uint32_t)g);
            emin[rf] = min(emin[rf], eb);
            emax[rf] = max(emax[rf], eb);
            const float sc = __uint_as_float(eb << 23);
            u32x4 av;
            av.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 0));
            av.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 1));
            av.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 2));
            av.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 3));
            A[rf] = __builtin_bit_cast(bf16x8, av);
        }
#pragma unroll
        for (int tf = 0; tf < NTF; tf++) {
            const uint32_t bl = (uint32_t)i16 * (kSeg * 64) + 16u * (uint32_t)((4 * j + g) ^ i16);
            const bf16x8 B = *reinterpret_cast<const bf16x8 *>(st + kOffB + tf * (16 * kSeg * 64) + bl);
            const float dx = *reinterpret_cast<const float *>(st + kOffD + ((16 * tf + i16) * kSeg + j) * 4);
#pragma unroll
            for (int rf = 0; rf < 2; rf++) {
                const v4f D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[rf], B, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rf][tf][r] = __builtin_fmaf(D[r], dx, acc[rf][tf][r]);
            }
        }
    }
}

}  // namespace

// Persistent workgroups of eight waves.  Work items are (GEMM expert, unit of
// output rows, tile of 64 list entries), ordered so the token tiles of one
// unit are consecutive (they share the unit's weight rows through the
// caches); workgroup b takes items b, b + G, b + 2G, ...  Gate/up units are
// 128 output rows: weight rows 0-127 of the item are gate rows, 128-255 the
// up rows of the same outputs, and wave w multiplies gate and up rows
// 16w .. 16w+15, so the SwiGLU is local to the wave; the Q8_0 block of act
// (32 rows) spans waves 2b and 2b+1.  Down units are 256 rows, wave w rows
// 32w .. 32w+31.  Every wave takes all 64 entries: 2 x 4 MFMA tiles per block.
//
// The K loop runs over segments of kSeg blocks through kStages LDS stages
// filled by LDS DMA loads (global/buffer -> LDS, no registers): segment s+1
// is loaded while segment s is multiplied.
template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_mx_gemm(MxGemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float s_amax[kWaves][kBN];  // gate/up: per wave and entry, |act| max of its 16 rows (-1: NaN)

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = a.nb;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const int unit_rows = MODE == kGateUp ? kBM / 2 : kBM;
    const int units = (a.rows + unit_rows - 1) / unit_rows;
    const int n_slots = *a.gm_n;
    const int total = n_slots > 0 ? a.gm_tile_off[n_slots] * units : 0;
    // Workgroup b runs on XCD b % 8 (round-robin dispatch), each XCD with its
    // own L2: number the workgroups XCD-major so consecutive items (the token
    // tiles of one unit, which read the same weight rows) run on one XCD.
    const int G = gridDim.x;
    const int vb = (G % kXcds == 0) ? ((int)blockIdx.x % kXcds) * (G / kXcds) + (int)blockIdx.x / kXcds : (int)blockIdx.x;
    if (vb >= total) return;

    const int i16 = lane & 15, g = lane >> 4;
    const int nseg = (nb + kSeg - 1) / kSeg;
    // activation tables through buffer descriptors (the per-stage advance is
    // a scalar offset)
    const u32x4v rs_b = rsrc_words(a.btab, (uint32_t)(a.tab_rows * (uint64_t)nb * 64u));
    const u32x4v rs_d = rsrc_words(a.scales, (uint32_t)(a.tab_rows * (uint64_t)nb * 4u));
    // per lane: B slot offsets of quarter g of block j for this lane's entry
    uint32_t b_lane[kSeg];
#pragma unroll
    for (int j = 0; j < kSeg; j++) b_lane[j] = (uint32_t)i16 * (kSeg * 64) + 16u * (uint32_t)((4 * j + g) ^ i16);

    for (int it = vb; it < total; it += G) {
        // item -> (slot, unit, token tile)
        int lo = 0, hi = n_slots - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (a.gm_tile_off[mid] * units <= it)
                lo = mid;
            else
                hi = mid - 1;
        }
        const int slot = lo;
        const int tile0 = a.gm_tile_off[slot], ntile = a.gm_tile_off[slot + 1] - tile0;
        const int rel = it - tile0 * units;
        const int u = rel / ntile, tt = rel - u * ntile;
        const int e = a.gm_active[slot];
        const int begin = a.offsets[e] + tt * kBN;
        const int nt = min(kBN, a.offsets[e + 1] - begin);
        const int ntf = (nt + 15) >> 4;  // token fragments holding entries

        uint32_t le0 = 0, le1 = 0;
        const u32x4v rs0 = expert_rsrc(a.w[0], a.expert_bytes, e, &le0);
        const u32x4v rs1 = MODE == kGateUp ? expert_rsrc(a.w[1], a.expert_bytes, e, &le1) : rs0;
        if (MODE != kGateUp) le1 = le0;
        // LDS row r -> matrix row
        auto mrow = [&](int r) { return MODE == kGateUp ? u * (kBM / 2) + (r & (kBM / 2 - 1)) : u * kBM + r; };

        // this thread's DMA loads: A load i = wave + 8k fills slots 64i..64i+63
        // (slot q: row q / 10, piece q % 10), B slots (entry (tid + 512k)/32),
        // d_x (entry (64*wave + lane)/8)
        uint32_t a_pos[kALoads];
        bool a_ok[kALoads];
#pragma unroll
        for (int k = 0; k < kALoads; k++) {
            const int q = 64 * (wave + kWaves * k) + lane, r = q / kASlots, pc = q - r * kASlots;
            const int row = mrow(r);
            a_ok[k] = row < a.rows;
            a_pos[k] = ((MODE == kGateUp && r >= kBM / 2) ? le1 : le0) + (uint32_t)(a_ok[k] ? row : 0) * row_bytes +
                       16u * (uint32_t)pc;
        }
        uint32_t b_off[kBLoads];
#pragma unroll
        for (int k = 0; k < kBLoads; k++) {
            const int q = tid + kThreads * k, t = q >> 5, piece = (q & 31) ^ (t & 15);
            int ar = 0;  // entries past nt load row 0 (unused)
            if (t < nt) {
                const int ent = a.list[begin + t];
                ar = MODE == kGateUp ? ent / a.topk : ent;
            }
            b_off[k] = ((uint32_t)ar * (uint32_t)nb + (uint32_t)(piece >> 2)) * 64u + 16u * (uint32_t)(piece & 3);
        }
        uint32_t d_off = 0;
        {
            const int idx = 64 * wave + lane, t = idx / kSeg, j = idx % kSeg;
            int ar = 0;
            if (t < nt) {
                const int ent = a.list[begin + t];
                ar = MODE == kGateUp ? ent / a.topk : ent;
            }
            d_off = ((uint32_t)ar * (uint32_t)nb + (uint32_t)j) * 4u;
        }
        typedef __attribute__((address_space(3))) uint8_t lds_u8;
        const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)lds);
        // ten DMA loads per wave and stage (A x5, B x4, d_x x1).  The A
        // window of segment s starts at the 16-byte boundary at or below
        // the row's byte pos + 136s (a_pos holds pos + 16 * piece).
        auto issue = [&](int s) {
            const uint32_t st = lds0 + (uint32_t)(s % kStages) * kStageBytes;
#pragma unroll
            for (int k = 0; k < kALoads; k++) {
                const int i = wave + kWaves * k;
                const uint32_t pos = a_pos[k] + (uint32_t)(kSeg * kMxBlock) * (uint32_t)s;
                // (pos - 16*piece) rounded down to 16, plus 16*piece
                dma16((MODE == kGateUp && i >= kAInstr / 2) ? rs1 : rs0, st + 16u * 64u * (uint32_t)i,
                      a_ok[k] ? (pos & ~15u) : kOOR, 0u);
            }
#pragma unroll
            for (int k = 0; k < kBLoads; k++)
                dma16(rs_b, st + kOffB + 16u * (64 * wave + kThreads * k), b_off[k], (uint32_t)(kSeg * 64) * (uint32_t)s);
            dma4(rs_d, st + kOffD + 256u * wave, d_off, (uint32_t)(kSeg * 4) * (uint32_t)s);
        };

        // this lane's A rows: LDS row and matrix byte position (the window of
        // segment s starts (pos + 68s) & 15 bytes into the row's LDS slots)
        uint32_t l_row[2], l_pos[2];
        bool row_ok[2];
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const int r = MODE == kGateUp ? 16 * wave + (kBM / 2) * rf + i16 : 32 * wave + 16 * rf + i16;
            const int row = mrow(r);
            row_ok[rf] = row < a.rows;
            l_row[rf] = (uint32_t)r * kARow;
            l_pos[rf] = ((MODE == kGateUp && rf == 1) ? le1 : le0) + (uint32_t)(row_ok[rf] ? row : 0) * row_bytes;
        }

        float acc[2][4][4];
#pragma unroll
        for (int rf = 0; rf < 2; rf++)
#pragma unroll
            for (int tf = 0; tf < 4; tf++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rf][tf][r] = 0.0f;
        uint32_t emin[2] = {255u, 255u}, emax[2] = {0u, 0u};

        // The K loop, instantiated per number of token fragments (so the
        // accumulators stay in place through it).
        auto kloop = [&](auto ntf_c) {
            constexpr int NTF = decltype(ntf_c)::value;
            issue(0);
            for (int s = 0; s < nseg; s++) {
                // this wave's loads of segment s have landed; after the
                // barrier every wave's have, and every wave is done with
                // segment s-1, whose stage segment s+1 reuses
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
                stage_barrier();
                if (s + 1 < nseg) issue(s + 1);
                const uint8_t *st = lds + (size_t)(s % kStages) * kStageBytes;
                const int jn = min(kSeg, nb - kSeg * s);
                uint32_t a_img[2];
#pragma unroll
                for (int rf = 0; rf < 2; rf++)
                    a_img[rf] = l_row[rf] + ((l_pos[rf] + (uint32_t)(kSeg * kMxBlock) * (uint32_t)s) & 15u);
                if (jn == kSeg)
                    seg_full<NTF>(st, a_img, b_lane, g, i16, acc, emin, emax);
                else
                    seg_part<NTF>(st, a_img, b_lane, g, i16, jn, acc, emin, emax);
            }
        };
        if (ntf == 4)
            kloop(std::integral_constant<int, 4>{});
        else if (ntf == 3)
            kloop(std::integral_constant<int, 3>{});
        else if (ntf == 2)
            kloop(std::integral_constant<int, 2>{});
        else
            kloop(std::integral_constant<int, 1>{});

        // entries of this lane's token columns
        int ent[4];
#pragma unroll
        for (int tf = 0; tf < 4; tf++) {
            const int t = 16 * tf + i16;
            ent[tf] = t < nt ? a.list[begin + t] : -1;
        }

        // rows with an E8M0 outside [kEMin, kEMax]: the integer decode, one
        // entry per lane, moved into the accumulators by lane shuffles
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const bool sp = row_ok[rf] && (emin[rf] < (uint32_t)kEMin || emax[rf] > (uint32_t)kEMax);
            const uint32_t rows16 = (uint32_t)__ballot(sp) & 0xFFFFu;  // lanes 0..15 hold rows 0..15
            if (rows16) {
                int ar = -1;
                if (lane < nt) {
                    const int en = a.list[begin + lane];
                    ar = MODE == kGateUp ? en / a.topk : en;
                }
                const int rbase = MODE == kGateUp ? 16 * wave + (kBM / 2) * rf : 32 * wave + 16 * rf;
                const ByteView cv = make_view(((MODE == kGateUp && rf == 1) ? a.w[1] : a.w[0]) + (uint64_t)e * a.expert_bytes,
                                              a.expert_bytes);
                for (int i = 0; i < 16; i++) {
                    if (!((rows16 >> i) & 1u)) continue;
                    float v = 0.0f;
                    if (ar >= 0)
                        v = lut_dot(cv, (uint32_t)mrow(rbase + i) * row_bytes, nb, a.codes + (size_t)ar * nb * 32,
                                    a.scales + (size_t)ar * nb);
#pragma unroll
                    for (int tf = 0; tf < 4; tf++) {
                        const float fv = __shfl(v, 16 * tf + i16);
                        if (g == (i >> 2)) acc[rf][tf][i & 3] = fv;
                    }
                }
            }
        }

        if constexpr (MODE == kDown) {
#pragma unroll
            for (int rf = 0; rf < 2; rf++) {
                const int row = u * kBM + 32 * wave + 16 * rf + 4 * g;
                if (row >= a.rows) continue;
                float bsum[4];
#pragma unroll
                for (int r = 0; r < 4; r++) bsum[r] = bias_at(a.bias[0], a.bias_type[0], (uint64_t)e * a.rows + row + r);
#pragma unroll
                for (int tf = 0; tf < 4; tf++) {
                    if (ent[tf] < 0) continue;
                    v4f o;
#pragma unroll
                    for (int r = 0; r < 4; r++) o[r] = acc[rf][tf][r] + bsum[r];
                    *reinterpret_cast<v4f *>(a.out + (size_t)ent[tf] * a.rows + row) = o;
                }
            }
            // every wave is done with the stages before the next item's loads
            stage_barrier();
        } else {
            // output rows u*128 + 16*wave + 4g + r: gate (rf 0), up (rf 1)
            const int row = u * (kBM / 2) + 16 * wave + 4 * g;
            const bool rok = row < a.rows;
            float bg[4], bu[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                bg[r] = rok ? bias_at(a.bias[0], a.bias_type[0], (uint64_t)e * a.rows + row + r) : 0.0f;
                bu[r] = rok ? bias_at(a.bias[1], a.bias_type[1], (uint64_t)e * a.rows + row + r) : 0.0f;
            }
            float act[4][4];
#pragma unroll
            for (int tf = 0; tf < 4; tf++) {
                float amax = 0.0f;
                bool nan = false;
                v4f gv, uv, av;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    gv[r] = acc[0][tf][r] + bg[r];
                    uv[r] = acc[1][tf][r] + bu[r];
                    av[r] = swiglu(gv[r], uv[r]);
                    act[tf][r] = av[r];
                    const float m = __builtin_fabsf(av[r]);
                    nan |= m != m;
                    amax = m > amax ? m : amax;
                }
                if (ent[tf] >= 0 && rok) {
                    const size_t o = (size_t)ent[tf] * a.rows + row;
                    if (a.tap[0]) *reinterpret_cast<v4f *>(a.tap[0] + o) = gv;
                    if (a.tap[1]) *reinterpret_cast<v4f *>(a.tap[1] + o) = uv;
                    if (a.out) *reinterpret_cast<v4f *>(a.out + o) = av;
                }
                // the wave's 16 rows of the entry: lanes i16 + 16g
                amax = fmaxf(amax, __shfl_xor(amax, 16));
                amax = fmaxf(amax, __shfl_xor(amax, 32));
                const bool nan_any = ((__ballot(nan) >> i16) & 0x0001000100010001ull) != 0;
                if (g == 0) s_amax[wave][16 * tf + i16] = nan_any ? -1.0f : amax;
            }
            // every wave is also done with the stages before the next item's loads
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            stage_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            const int blk_row = u * (kBM / 2) + 32 * (wave >> 1);  // first row of this wave pair's Q8_0 block
            const int half = wave & 1;                             // elements 16*half .. 16*half+15 of it
            const int nbo = a.rows / 32;
#pragma unroll
            for (int tf = 0; tf < 4; tf++) {
                if (ent[tf] < 0 || blk_row >= a.rows) continue;
                const float m0 = s_amax[wave][16 * tf + i16], m1 = s_amax[wave ^ 1][16 * tf + i16];
                const bool nan_any = m0 < 0.0f || m1 < 0.0f;
                const float d = nan_any ? __builtin_nanf("") : fmaxf(m0, m1) / 127.0f;
                const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
                const uint16_t dh = f32_to_f16_bits(d);
                int q[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float rq = __builtin_roundf(act[tf][r] * id);
                    q[r] = (rq != rq) ? 0 : (rq > 127.0f ? 127 : (rq < -127.0f ? -127 : (int)rq));
                }
                const size_t blk = (size_t)ent[tf] * nbo + blk_row / 32;
                const int el = 16 * half + 4 * g;  // element of q[0]
                if (a.act_codes)
                    *reinterpret_cast<uint32_t *>(a.act_codes + blk * 32 + el) =
                        (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
                        ((uint32_t)(q[3] & 0xff) << 24);
                if (half == 0 && g == 0) {
                    if (a.act_scales) a.act_scales[blk] = f16_bits_to_f32(dh);
                    if (a.act_blocks34) {
                        a.act_blocks34[blk * kQ80Block] = (uint8_t)(dh & 0xff);
                        a.act_blocks34[blk * kQ80Block + 1] = (uint8_t)(dh >> 8);
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    // element 16*half + 4g + r: nibble position 2*(4g + r) + half
                    const int p = 2 * (4 * g + r) + half;
                    if (a.act_mxtab) {
                        a.act_mxtab[blk * 64 + p] = (uint8_t)e4m3_small(q[r] >> 4);
                        a.act_mxtab[blk * 64 + 32 + p] = (uint8_t)e4m3_small(q[r] & 15);
                    }
                    if (a.act_btab)
                        reinterpret_cast<uint16_t *>(a.act_btab + blk * 16)[2 * (4 * g + r) + half] =
                            (uint16_t)(__float_as_uint((float)q[r]) >> 16);
                    if (a.act_blocks34) a.act_blocks34[blk * kQ80Block + 2 + el + r] = (uint8_t)q[r];
                }
            }
            // the partner wave has read this wave's s_amax before the next item writes it
            stage_barrier();
        }
    }
}

hipError_t launch_mx_gemm(hipStream_t s, GemvMode mode, const MxGemmArgs &a, int max_items) {
    if (max_items <= 0 || a.rows <= 0 || a.nb <= 0) return hipSuccess;
    constexpr size_t lds = (size_t)kStages * kStageBytes;
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_gemm<kGateUp>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_gemm<kDown>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
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
    const int grid = max_items < n_cu ? max_items : n_cu;
    if (mode == kGateUp)
        hipLaunchKernelGGL(k_mx_gemm<kGateUp>, dim3(grid), dim3(kThreads), lds, s, a);
    else if (mode == kDown)
        hipLaunchKernelGGL(k_mx_gemm<kDown>, dim3(grid), dim3(kThreads), lds, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace spt
