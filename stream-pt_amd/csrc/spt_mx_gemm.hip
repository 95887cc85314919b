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
constexpr int kSeg = 4;                // 32-element blocks per K segment (68 bytes of a row)
// A stage: row r's window (the segment's bytes from the 16-byte boundary at
// or below its first byte) in 6 slots of 16 bytes (16-byte aligned loads:
// a load crossing the end of the descriptor's range would read zeros for all
// its bytes).  The 64 lanes of a DMA load fill 64 consecutive slots, so a
// stage's 256 x 6 slots take 24 loads per workgroup, three per wave; loads
// 0-11 hold rows 0-127.
constexpr int kAPieces = (kSeg * kMxBlock + 15 + 15) / 16;
constexpr int kASlots = kAPieces;
constexpr int kARow = 16 * kASlots;
constexpr int kAInstr = kBM * kASlots / 64;
// B: per entry 4 * kSeg slots of 16 bytes (kSeg blocks x 4 quarters of the
// bf16 code table); quarter piece p of entry t sits in slot p ^ (t & 15), so
// the 16 entries of an MFMA fragment read 16 different bank groups.  A stage
// holds the B slots of the item's token fragments only, then d_x
// [entry][kSeg] and the slots of the d_x loads without entries, so items
// with fewer fragments have smaller stages.  At most three stages (two
// segments in flight) whatever the stage size: a compute unit's memory
// queue holds about 48 KB of loads, and a wave whose DMA load finds it full
// stalls at the issue instead of multiplying (512-token layer with 25 %
// hot tokens: 583.8 us with at most three stages, 585.5 with four, 589.3
// with five).
constexpr int kOffB = kBM * kARow;
constexpr int kBFrag = 16 * kSeg * 64;            // B bytes of one token fragment
constexpr int kDBytes = 64 * 8 * 4;               // d_x region: one 256-byte load per wave
constexpr int kLdsDynamic = 155648;               // dynamic LDS of a workgroup (stages)
constexpr int kMaxStages = 3;
constexpr int kEMin = 4, kEMax = 240;
constexpr int kXcds = 8;  // accelerator complex dies of an MI355X
constexpr uint32_t kOOR = 0x80000000u;  // buffer offset past every range: reads zero
static_assert(kSeg * kMxBlock + 15 <= 16 * kAPieces, "A window");
static_assert(kAInstr % kWaves == 0, "stage loads");
static_assert(kBM / 2 * kASlots % 64 == 0, "gate rows fill whole A loads");
static_assert(kBN * kSeg <= 64 * kWaves && 4 * kSeg <= 16 && 64 * kWaves * 4 == kDBytes,
              "one d_x load per wave; B swizzle within 16 slots");
constexpr int kALoads = kAInstr / kWaves;  // 3

// Stage geometry of an item with NTF token fragments: the d_x offset, the
// stage size, the number of stages and the DMA loads per wave and segment
// (A x3, B x NTF/2 -- a wave with an odd NTF's extra load has one more -- and
// d_x x1).
template <int NTF>
struct Geo {
    static constexpr int kOffD = kOffB + NTF * kBFrag;
    static constexpr int kBytes = kOffD + kDBytes;
    static constexpr int kStages = kLdsDynamic / kBytes < kMaxStages ? kLdsDynamic / kBytes : kMaxStages;
    static constexpr int kAhead = kStages - 1;  // segments in flight while one is multiplied
    static constexpr int kLoadsMin = kALoads + NTF / 2 + 1;
    static_assert(kStages >= 3 && kStages * kBytes <= kLdsDynamic, "stages");
};


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

typedef __attribute__((address_space(3))) const uint8_t lds_cu8;
typedef __attribute__((address_space(3))) const uint32_t lds_cu32;

// A segment's operands in one stage, as LDS pointers computed once per
// segment (every block's read is then a constant offset from them):
// a[rf] = this lane's row window of fragment rf (the E8M0 byte of block j at
// a[rf][17j]); n[rf] = a[rf] + 1 + 4g (the nibble bytes of block j for lane
// group g at n[rf] + 17j); b[j] = quarter g of block j of this lane's entry
// in token fragment 0 (fragment tf at + tf * 16 * kSeg * 64); d = d_x of this
// lane's entry, block 0 (fragment tf, block j at + tf * 16 * kSeg + j).
struct SegView {
    lds_cu8 *a[2];
    lds_cu8 *n[2];
    lds_cu8 *b[kSeg];
    __attribute__((address_space(3))) const float *d;
};

// Four bytes at LDS address p (any alignment): two aligned dwords and a byte
// shift (an unaligned LDS dword read returns the same bytes but is far
// slower; the shift operand's low two bits are the address's).
__device__ __attribute__((always_inline)) inline uint32_t nibble_word(lds_cu8 *p) {
    const uint32_t o = (uint32_t)reinterpret_cast<uintptr_t>(p);
    lds_cu32 *pw = reinterpret_cast<lds_cu32 *>((uintptr_t)(o & ~3u));
    return __builtin_amdgcn_alignbyte(pw[1], pw[0], o);
}

// A fragment of 16 weight rows x 32 K of block j as bf16 (the E2M1 nibbles
// scaled by 2^(e-127)), and the block's E8M0.
__device__ __attribute__((always_inline)) inline bf16x8 decode_a(uint32_t w4, uint32_t eb) {
    const float sc = __uint_as_float(eb << 23);
    u32x4 av;
    av.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 0));
    av.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 1));
    av.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 2));
    av.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 3));
    return __builtin_bit_cast(bf16x8, av);
}

// Blocks [J0, J1) of a full segment with NTF token fragments, straight-line:
// the A bytes of those blocks first, the B fragments and d_x one block
// ahead, then per block its A decode, MFMAs and the FMAs that apply d_x (the
// two waves of a SIMD overlap one's FMAs with the other's MFMAs).  A full
// segment is two such halves, so the rest of the next segment's loads can
// go out between them without stretching the live ranges of either.
template <int NTF, int J0, int J1>
__device__ __attribute__((always_inline)) inline void seg_blocks(const SegView &v, float (&acc)[2][4][4],
                                                                 uint32_t (&emin)[2], uint32_t (&emax)[2]) {
    constexpr int NJ = J1 - J0;
    uint32_t eb[NJ][2], w4[NJ][2];
#pragma unroll
    for (int jj = 0; jj < NJ; jj++)
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const int j = J0 + jj;
            eb[jj][rf] = v.a[rf][17 * j];
            w4[jj][rf] = nibble_word(v.n[rf] + 17 * j);
        }
    bf16x8 Bv[2][NTF];
    float dx[2][NTF];
    auto load_b = [&](int jj) {
        const int j = J0 + jj;
#pragma unroll
        for (int tf = 0; tf < NTF; tf++) {
            Bv[jj & 1][tf] = *reinterpret_cast<__attribute__((address_space(3))) const bf16x8 *>(
                v.b[j] + tf * (16 * kSeg * 64));
            dx[jj & 1][tf] = v.d[tf * 16 * kSeg + j];
        }
    };
    load_b(0);
#pragma unroll
    for (int jj = 0; jj < NJ; jj++) {
        if (jj + 1 < NJ) load_b(jj + 1);
        v4f D[2][NTF];
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const bf16x8 A = decode_a(w4[jj][rf], eb[jj][rf]);
#pragma unroll
            for (int tf = 0; tf < NTF; tf++)
                D[rf][tf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, Bv[jj & 1][tf], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        }
#pragma unroll
        for (int rf = 0; rf < 2; rf++)
#pragma unroll
            for (int tf = 0; tf < NTF; tf++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rf][tf][r] = __builtin_fmaf(D[rf][tf][r], dx[jj & 1][tf], acc[rf][tf][r]);
    }
#pragma unroll
    for (int rf = 0; rf < 2; rf++)
#pragma unroll
        for (int jj = 0; jj < NJ; jj += 2) {
            emin[rf] = min(emin[rf], min(eb[jj][rf], eb[jj + 1][rf]));
            emax[rf] = max(emax[rf], max(eb[jj][rf], eb[jj + 1][rf]));
        }
}
static_assert(kSeg % 4 == 0, "seg_blocks' halves and exponent reduction");

// The last segment when it holds jn < kSeg blocks (unrolled with a guard:
// a loop bound by jn would index the view's pointer array at run time,
// which puts it in scratch memory).
template <int NTF>
__device__ __attribute__((always_inline)) inline void seg_part(const SegView &v, int jn, float (&acc)[2][4][4],
                                                               uint32_t (&emin)[2], uint32_t (&emax)[2]) {
#pragma unroll
    for (int j = 0; j < kSeg - 1; j++) {
        if (j >= jn) break;
        bf16x8 A[2];
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const uint32_t eb = v.a[rf][17 * j];
            const uint32_t w4 = nibble_word(v.n[rf] + 17 * j);
            emin[rf] = min(emin[rf], eb);
            emax[rf] = max(emax[rf], eb);
            A[rf] = decode_a(w4, eb);
        }
#pragma unroll
        for (int tf = 0; tf < NTF; tf++) {
            const bf16x8 B =
                *reinterpret_cast<__attribute__((address_space(3))) const bf16x8 *>(v.b[j] + tf * (16 * kSeg * 64));
            const float dx = v.d[tf * 16 * kSeg + j];
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
// up rows of the same outputs, and wave w multiplies the gate and up rows of
// the same 16 outputs, so the SwiGLU is local to the wave.  Those 16 outputs
// are half of the Q8_0 block 32 * (w / 2) .. +31 of the unit: elements
// 8 * (w % 2) + 0..7 and 16 + 8 * (w % 2) + 0..7 (the unit's local row with
// bits 3 and 4 exchanged), so every dword j of the block's bf16 code table
// (elements j and j + 16) is made by one wave.  Down units are 256 rows,
// wave w rows 32w .. 32w+31.  Every wave takes all 64 entries: 2 x 4 MFMA
// tiles per block.
//
// The K loop runs over segments of kSeg blocks through LDS stages filled by
// LDS DMA loads (global/buffer -> LDS, no registers): kAhead segments are
// in flight while one is multiplied.  A stage holds the B codes of the
// item's token fragments only, so an item with one fragment has five stages
// (four segments in flight), with two or three fragments four, with four
// three: the bytes in flight per CU, which set the rate at which its loads
// arrive, stay near the LDS size.
template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_mx_gemm(MxGemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float s_amax[kWaves][kBN];  // gate/up: per wave and entry, |act| max of its 16 rows (-1: NaN)
    // per item parity: the bias of the item's rows (matrix order; gate/up:
    // gate rows then up rows) and the item's list entries (-1 past its end)
    __shared__ __align__(16) float s_bias[2][kBM];
    __shared__ int s_ent[2][kBN];
    __shared__ int s_next[2];  // per item parity: the workgroup's next item

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

    const int nseg = (nb + kSeg - 1) / kSeg;
    // activation tables through buffer descriptors (the per-stage advance is
    // a scalar offset)
    const u32x4v rs_b = rsrc_words(a.btab, (uint32_t)(a.tab_rows * (uint64_t)nb * 64u));
    const u32x4v rs_d = rsrc_words(a.scales, (uint32_t)(a.tab_rows * (uint64_t)nb * 4u));
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)lds);

    // The first item of workgroup b is vb; later ones are claimed from the
    // launch's counter (items G, G+1, ... in order, largest experts first),
    // so the workgroups finish together.
    int parity = 0;  // item parity (s_bias / s_ent / s_next buffer)
    for (int it = vb; it < total; parity ^= 1) {
        // The lane's roles, from the lane index made opaque per item: the
        // addresses derived from it are recomputed per item (a few VALU
        // operations) rather than held across the item loop, where the K
        // loop's registers leave no room for them.
        int lane_it = lane;
        asm volatile("" : "+v"(lane_it));
        const int i16 = lane_it & 15, g = lane_it >> 4, tid_it = 64 * wave + lane_it;
        // stage offsets of the B slot of quarter g of block j for this lane's entry
        uint32_t b_lane[kSeg];
#pragma unroll
        for (int j = 0; j < kSeg; j++)
            b_lane[j] = kOffB + (uint32_t)i16 * (kSeg * 64) + 16u * (uint32_t)((4 * j + g) ^ i16);
        // item -> slot: the number of slots i >= 1 whose first item is at or
        // below it (gm_tile_off is increasing), 64 slots per ballot
        int slot = 0;
        for (int c = 1; c < n_slots; c += 64) {
            const int i = c + lane_it;
            const bool le = i < n_slots && a.gm_tile_off[i] * units <= it;
            slot += __popcll(__ballot(le));
        }
        slot = __builtin_amdgcn_readfirstlane(slot);
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
        // LDS row r -> matrix row (gate/up: bits 3 and 4 of the unit's local
        // row exchanged, so a wave's 16 rows hold whole code-table dwords)
        auto mrow = [&](int r) {
            if (MODE == kGateUp) {
                const int x = r & (kBM / 2 - 1);
                return u * (kBM / 2) + ((x & ~0x18) | ((x & 8) << 1) | ((x >> 1) & 8));
            }
            return u * kBM + r;
        };

        // this thread's DMA loads: A load i = wave + 8k fills slots 64i..64i+63
        // (slot q: row q / kASlots, piece q % kASlots), B slots (entry
        // (tid + 512k) / (4 kSeg)), d_x (entry (64*wave + lane) / kSeg);
        // entries past nt read nothing
        uint32_t a_pos[kALoads];
        bool a_ok[kALoads];
#pragma unroll
        for (int k = 0; k < kALoads; k++) {
            const int q = 64 * (wave + kWaves * k) + lane_it, r = q / kASlots, pc = q - r * kASlots;
            const int row = mrow(r);
            a_ok[k] = row < a.rows;
            a_pos[k] = ((MODE == kGateUp && r >= kBM / 2) ? le1 : le0) + (uint32_t)(a_ok[k] ? row : 0) * row_bytes +
                       16u * (uint32_t)pc;
        }
        uint32_t b_off[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int q = tid_it + kThreads * k, t = q / (4 * kSeg), piece = (q % (4 * kSeg)) ^ (t & 15);
            b_off[k] = kOOR;
            if (t < nt) {
                const int ent = a.list[begin + t];
                const int ar = MODE == kGateUp ? ent / a.topk : ent;
                b_off[k] = ((uint32_t)ar * (uint32_t)nb + (uint32_t)(piece >> 2)) * 64u + 16u * (uint32_t)(piece & 3);
            }
        }
        uint32_t d_off = kOOR;
        {
            const int idx = 64 * wave + lane_it, t = idx / kSeg, j = idx % kSeg;
            if (t < nt) {
                const int ent = a.list[begin + t];
                const int ar = MODE == kGateUp ? ent / a.topk : ent;
                d_off = ((uint32_t)ar * (uint32_t)nb + (uint32_t)j) * 4u;
            }
        }
        // this thread's share of the item's bias and entries, and the next
        // item (staged in LDS once segment 0's loads have landed)
        float bias_v = 0.0f;
        int ent_v = -1, next_v = 0;
        if (tid_it == 0) next_v = G + atomicAdd(a.claim, 1);
        if (tid_it < kBM) {
            const int m = MODE == kGateUp ? tid_it / (kBM / 2) : 0;
            const int row = MODE == kGateUp ? u * (kBM / 2) + (tid_it & (kBM / 2 - 1)) : u * kBM + tid_it;
            if (row < a.rows) bias_v = bias_at(a.bias[m], a.bias_type[m], (uint64_t)e * a.rows + row);
        } else if (tid_it < kBM + kBN) {
            if (tid_it - kBM < nt) ent_v = a.list[begin + tid_it - kBM];
        }
        // The DMA loads of segment s into the stage at LDS byte address st, in
        // two parts: the weights and d_x, then the B codes (a wave stalls at
        // a load's issue while its CU's memory queue is full; the second part
        // goes out half a segment later, when the first has drained).  The
        // A window of segment s starts at the 16-byte boundary at or below
        // the row's byte pos + 68s (a_pos holds pos + 16 * piece).  Lanes
        // whose entries are past nt read nothing (zeros); the d_x loads of
        // the waves past the item's entries fill the stage's spare d_x slots.
        auto issue_a = [&](int s, uint32_t st, uint32_t off_d) {
#pragma unroll
            for (int k = 0; k < kALoads; k++) {
                const int i = wave + kWaves * k;
                const uint32_t pos = a_pos[k] + (uint32_t)(kSeg * kMxBlock) * (uint32_t)s;
                // (pos - 16*piece) rounded down to 16, plus 16*piece
                dma16((MODE == kGateUp && i >= kAInstr / 2) ? rs1 : rs0, st + 16u * 64u * (uint32_t)i,
                      a_ok[k] ? (pos & ~15u) : kOOR, 0u);
            }
            dma4(rs_d, st + off_d + 256u * wave, d_off, (uint32_t)(kSeg * 4) * (uint32_t)s);
        };
        // B load k of wave w covers entries 32k + 4w .. 32k + 4w + 3: the item's
        // NTF fragments take loads k < NTF / 2 of every wave, and with an odd
        // NTF load NTF / 2 of waves 0-3
        auto issue_b = [&](auto ntf_c, int s, uint32_t st) {
            constexpr int NTF = decltype(ntf_c)::value;
#pragma unroll
            for (int k = 0; k < NTF / 2; k++)
                dma16_other_stage(rs_b, st + kOffB + 16u * (64 * wave + kThreads * k), b_off[k],
                                  (uint32_t)(kSeg * 64) * (uint32_t)s);
            if constexpr (NTF % 2 == 1) {
                if (wave < 4)
                    dma16_other_stage(rs_b, st + kOffB + 16u * (64 * wave + kThreads * (NTF / 2)), b_off[NTF / 2],
                                      (uint32_t)(kSeg * 64) * (uint32_t)s);
            }
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
        // accumulators stay in place through it, and the stages have that
        // many fragments' B slots): segment s in stage s % kStages of the
        // item's geometry; the loads of segments 0 .. kAhead-1 first, then
        // the segments whose loads issue a later segment's in a loop of
        // their own (one straight-line body, so the accumulators keep their
        // registers across iterations), then the last kAhead segments.
        auto kloop = [&](auto ntf_c) {
            constexpr int NTF = decltype(ntf_c)::value;
            typedef Geo<NTF> G;
            auto st_of = [&](int stage) { return lds0 + (uint32_t)stage * (uint32_t)G::kBytes; };
            // segment 0's loads, the bias and entries into LDS (waiting for
            // their loads waits for segment 0's too, which the K loop would),
            // then the loads of the other segments issued ahead
            issue_a(0, st_of(0), G::kOffD);
            issue_b(ntf_c, 0, st_of(0));
            asm volatile("" ::: "memory");
            if (tid_it < kBM)
                s_bias[parity][tid_it] = bias_v;
            else if (tid_it < kBM + kBN)
                s_ent[parity][tid_it - kBM] = ent_v;
            if (tid_it == 0) s_next[parity] = next_v;
            asm volatile("" ::: "memory");
            for (int q = 1; q < G::kAhead && q < nseg; q++) {
                issue_a(q, st_of(q), G::kOffD);
                issue_b(ntf_c, q, st_of(q));
            }
            auto view_of = [&](int s, int stage) {
                SegView v;
                lds_cu8 *st = reinterpret_cast<lds_cu8 *>((uintptr_t)st_of(stage));
#pragma unroll
                for (int rf = 0; rf < 2; rf++) {
                    v.a[rf] = st + l_row[rf] + ((l_pos[rf] + (uint32_t)(kSeg * kMxBlock) * (uint32_t)s) & 15u);
                    v.n[rf] = v.a[rf] + 1 + 4 * g;
                }
#pragma unroll
                for (int j = 0; j < kSeg; j++) v.b[j] = st + b_lane[j];
                v.d = reinterpret_cast<__attribute__((address_space(3))) const float *>(st + G::kOffD) + i16 * kSeg;
                return v;
            };
            int s = 0, cur = 0;  // segment, its stage
            for (; s + G::kAhead < nseg; s++) {
                // this wave's loads of segment s have landed (those of the
                // kAhead-1 segments issued after them may not have: every
                // wave issues at least kLoadsMin loads per segment); after
                // the barrier every wave's have, and every wave is done with
                // segment s-1, whose stage segment s + kAhead reuses
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((G::kAhead - 1) * G::kLoadsMin) : "memory");
                stage_barrier();
                const int nxt = cur == 0 ? G::kStages - 1 : cur - 1;
                issue_a(s + G::kAhead, st_of(nxt), G::kOffD);
                const SegView v = view_of(s, cur);
                seg_blocks<NTF, 0, kSeg / 2>(v, acc, emin, emax);
                issue_b(ntf_c, s + G::kAhead, st_of(nxt));
                seg_blocks<NTF, kSeg / 2, kSeg>(v, acc, emin, emax);
                cur = cur + 1 == G::kStages ? 0 : cur + 1;
            }
            // the last kAhead segments (or fewer): every load is issued, and
            // only the last segment can be partial
            for (; s < nseg; s++) {
                const int later = nseg - 1 - s;  // segments in flight after s
                if (later >= 3)
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(3 * G::kLoadsMin) : "memory");
                else if (later == 2)
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(2 * G::kLoadsMin) : "memory");
                else if (later == 1)
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(G::kLoadsMin) : "memory");
                else
                    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
                stage_barrier();
                const SegView v = view_of(s, cur);
                const int jn = nb - kSeg * s;
                if (jn >= kSeg) {
                    seg_blocks<NTF, 0, kSeg / 2>(v, acc, emin, emax);
                    seg_blocks<NTF, kSeg / 2, kSeg>(v, acc, emin, emax);
                } else {
                    seg_part<NTF>(v, jn, acc, emin, emax);
                }
                cur = cur + 1 == G::kStages ? 0 : cur + 1;
            }
            static_assert(G::kAhead <= 4, "the tail's waits cover three later segments");
        };
        if (ntf == 4)
            kloop(std::integral_constant<int, 4>{});
        else if (ntf == 3)
            kloop(std::integral_constant<int, 3>{});
        else if (ntf == 2)
            kloop(std::integral_constant<int, 2>{});
        else
            kloop(std::integral_constant<int, 1>{});
        // down: every wave is done with the stages before the next item's
        // loads (gate/up waits at its epilogue's barrier)
        if constexpr (MODE == kDown) stage_barrier();

        // entries of this lane's token columns
        int ent[4];
#pragma unroll
        for (int tf = 0; tf < 4; tf++) ent[tf] = s_ent[parity][16 * tf + i16];

        // rows with an E8M0 outside [kEMin, kEMax]: the integer decode, one
        // entry per lane, moved into the accumulators by lane shuffles
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const bool sp = row_ok[rf] && (emin[rf] < (uint32_t)kEMin || emax[rf] > (uint32_t)kEMax);
            const uint32_t rows16 = (uint32_t)__ballot(sp) & 0xFFFFu;  // lanes 0..15 hold rows 0..15
            if (rows16) {
                int ar = -1;
                if (lane_it < nt) {
                    const int en = a.list[begin + lane_it];
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
                const int lrow = 32 * wave + 16 * rf + 4 * g, row = u * kBM + lrow;
                if (row >= a.rows) continue;
                const v4f bsum = *reinterpret_cast<const v4f *>(&s_bias[parity][lrow]);
#pragma unroll
                for (int tf = 0; tf < 4; tf++) {
                    if (ent[tf] < 0) continue;
                    v4f o;
#pragma unroll
                    for (int r = 0; r < 4; r++) o[r] = acc[rf][tf][r] + bsum[r];
                    *reinterpret_cast<v4f *>(a.out + (size_t)ent[tf] * a.rows + row) = o;
                }
            }
        } else {
            // output rows row + r (r = 0..3): element el0 + r of the unit's
            // Q8_0 block 32 * (wave / 2) .. +31; gate (rf 0), up (rf 1)
            const int half = wave & 1;
            const int el0 = 16 * (g >> 1) + 8 * half + 4 * (g & 1);
            const int lrow = 32 * (wave >> 1) + el0, row = u * (kBM / 2) + lrow;
            const bool rok = row < a.rows;
            const v4f bg = *reinterpret_cast<const v4f *>(&s_bias[parity][lrow]);
            const v4f bu = *reinterpret_cast<const v4f *>(&s_bias[parity][kBM / 2 + lrow]);
            // (token fragments past ntf hold no entries: their SwiGLU, the
            // epilogue's main cost, is skipped)
            float act[4][4];
#pragma unroll
            for (int tf = 0; tf < 4; tf++) {
                if (tf >= ntf) continue;
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
            // both halves of each block's |act| max are in LDS (the next
            // item writes s_amax only after a barrier of its K loop, which
            // every wave reaches after reading this item's)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            stage_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            const int blk_row = u * (kBM / 2) + 32 * (wave >> 1);  // first row of this wave pair's Q8_0 block
            const int nbo = a.rows / 32;
#pragma unroll
            for (int tf = 0; tf < 4; tf++) {
                if (tf >= ntf) continue;
                const float m0 = s_amax[wave][16 * tf + i16], m1 = s_amax[wave ^ 1][16 * tf + i16];
                const bool nan_any = m0 < 0.0f || m1 < 0.0f;
                const float d = nan_any ? __builtin_nanf("") : fmaxf(m0, m1) / 127.0f;
                const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
                const uint16_t dh = f32_to_f16_bits(d);
                uint32_t qw = 0;  // the four codes, element el0 + r in byte r
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float rq = __builtin_roundf(act[tf][r] * id);
                    const int q = (rq != rq) ? 0 : (rq > 127.0f ? 127 : (rq < -127.0f ? -127 : (int)rq));
                    qw |= (uint32_t)(q & 0xff) << (8 * r);
                }
                // the codes of elements el0 ^ 16 + r (lane ^ 32), for the
                // code-table dwords: this lane writes r = 2 * (g >> 1) + 0..1
                const uint32_t qp = (uint32_t)__shfl_xor((int)qw, 32);
                if (ent[tf] < 0 || blk_row >= a.rows) continue;
                const size_t blk = (size_t)ent[tf] * nbo + blk_row / 32;
                if (a.act_codes) *reinterpret_cast<uint32_t *>(a.act_codes + blk * 32 + el0) = qw;
                if (a.act_btab) {
                    const uint32_t lo = (g >> 1) ? qp : qw, hi = (g >> 1) ? qw : qp;  // elements j and j + 16
                    const int r0 = 2 * (g >> 1);
                    uint32_t dw[2];
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const int ql = (int8_t)(lo >> (8 * (r0 + k))), qh = (int8_t)(hi >> (8 * (r0 + k)));
                        dw[k] = (__float_as_uint((float)ql) >> 16) | (__float_as_uint((float)qh) & 0xFFFF0000u);
                    }
                    *reinterpret_cast<uint2 *>(a.act_btab + blk * 16 + (el0 & 15) + r0) = make_uint2(dw[0], dw[1]);
                }
                if (half == 0 && g == 0) {
                    if (a.act_scales) a.act_scales[blk] = f16_bits_to_f32(dh);
                    if (a.act_blocks34) {
                        a.act_blocks34[blk * kQ80Block] = (uint8_t)(dh & 0xff);
                        a.act_blocks34[blk * kQ80Block + 1] = (uint8_t)(dh >> 8);
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int q = (int8_t)(qw >> (8 * r));
                    // element el: nibble position 2 * (el & 15) + (el >> 4)
                    const int p = 2 * ((el0 + r) & 15) + (el0 >> 4);
                    if (a.act_mxtab) {
                        a.act_mxtab[blk * 64 + p] = (uint8_t)e4m3_small(q >> 4);
                        a.act_mxtab[blk * 64 + 32 + p] = (uint8_t)e4m3_small(q & 15);
                    }
                    if (a.act_blocks34) a.act_blocks34[blk * kQ80Block + 2 + el0 + r] = (uint8_t)q;
                }
            }
        }
        it = s_next[parity];
    }
}

hipError_t launch_mx_gemm(hipStream_t s, GemvMode mode, const MxGemmArgs &a, int max_items) {
    if (max_items <= 0 || a.rows <= 0 || a.nb <= 0) return hipSuccess;
    constexpr size_t lds = (size_t)kLdsDynamic;
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_gemm<kGateUp>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_mx_gemm<kDown>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        return e;
    }();
    if (attr != hipSuccess) return attr;
    const int n_cu = device_cus();
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
