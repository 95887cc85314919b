// spt_q40_gemm.hip -- Q4_0 x Q8_0 GEMM for batches of 32 tokens and more on
// the gfx950 int8 MFMA (v_mfma_i32_16x16x32_i8).
//
// forward.MulQ40BatchInto (forward/q40.go:40-103) for batches large enough
// that the projection is a contraction: y[t][row] = sum_b float(isum) *
// (d_w * d_x), with isum = sum (n - 8) * q the exact int32 block sum.  One
// MFMA per 16 rows x 16 tokens x one block of 32: A = the weight values
// n - 8 (-8..7 as int8: (n | 0x80) - 8, then ^ 0x80, per byte), B = the Q8_0
// codes, D = isum exactly; then acc = fma(float(isum), d_w * d_x, acc), the
// GEMV's arithmetic per block.
// K order inside a block: lane group g of the MFMA (k = 8g .. 8g+7) takes
// nibble bytes 2+4g .. 5+4g of the block: low nibbles are elements 4g..4g+3,
// high nibbles 16+4g..16+4g+3, matched by code dwords g and 4+g.
// MFMA lane layout (measured on the hardware): lane l holds A row l%16 and
// B column l%16 at k = 8*(l/16) + 0..7 (byte i of the 64-bit operand is
// k offset i); D lane l, register r is row 4*(l/16) + r, column l%16.
#include <type_traits>

#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTR = 16 * kWaves;  // rows per workgroup (16 per wave)
constexpr int kTN = 64;           // tokens per workgroup (4 fragments)
static_assert(kTR == kQ40TileRows && kTN == kQ40TileTokens, "the tiles the split rule counts");
constexpr int kSeg = 8;           // blocks per K segment (144 bytes of a row)
constexpr int kAPieces = 10;      // 16-byte loads per row window (144 + 15 <= 160)
constexpr int kASlots = 11;       // LDS slots of 16 B per staged row (44 dwords: rows over distinct banks)
constexpr int kARow = 16 * kASlots;
constexpr int kAInstr = kTR * kASlots / 64;  // LDS DMA loads of a stage's A (64 slots each): 11
constexpr int kBSlots = 2 * kSeg + 1;        // LDS slots of 16 B per staged token (the last is padding)
constexpr int kBTok = 16 * kBSlots;          // 68 dwords: a fragment's tokens over distinct banks
constexpr int kBInstr = kTN * kBSlots / 64;  // LDS DMA loads of a stage's B: 17
constexpr int kOffB = kTR * kARow;
constexpr int kOffD = kOffB + kTN * kBTok;  // d_x [kSeg][token] (a fragment's 16 tokens in consecutive banks)
constexpr int kStageBytes = kOffD + kTN * kSeg * 4;
constexpr uint32_t kOOR = 0x80000000u;      // buffer offset past every range: reads zero
static_assert(kSeg * kQ40Block + 15 <= 16 * kAPieces && kAPieces < kASlots, "A window");
static_assert(kTR * kASlots % 64 == 0, "whole A loads");
constexpr int kALoadsMax = (kAInstr + kWaves - 1) / kWaves;  // 3 (wave w: loads w, w + 4, w + 8 below 11)
constexpr int kBLoadsMax = (kBInstr + kWaves - 1) / kWaves;  // 5 (wave w: loads w, w + 4, ... below 17)
constexpr int kDLoads = kSeg / kWaves;                       // 2 (one block of the 64 tokens' d_x each)
static_assert(kTN * kBSlots % 64 == 0 && kSeg % kWaves == 0 && kTN == 64, "stage loads");

// Four bytes of the stage at byte offset o (o even: Q4_0 rows are 2-byte
// aligned): two aligned dwords and a byte shift.
__device__ __attribute__((always_inline)) inline uint32_t word_at(const uint8_t *st, uint32_t o) {
    const uint32_t *pw = reinterpret_cast<const uint32_t *>(st + (o & ~3u));
    return __builtin_amdgcn_alignbyte(pw[1], pw[0], o & 3u);
}

// Blocks [j0, j1) of a stage (JN = j1 - j0 known when the segment is full)
// for NTF token fragments: each block's LDS reads are issued one block ahead
// of its MFMAs.
struct Q40Lane {
    uint32_t alead;     // LDS offset of this lane's nibble word of block 0
    uint32_t dlead[4];  // LDS offsets of the D rows' fp16 scales of block 0
    int i16, g;
};

template <int NTF, int JN>
__device__ __attribute__((always_inline)) inline void q40_blocks(const uint8_t *st, const Q40Lane &L, int jn,
                                                                 float (&acc)[4][4]) {
    struct Blk {
        uint32_t w4;
        uint32_t dwb[4];
        uint32_t bq[NTF][2];
        float dx[NTF];
    };
    auto fetch = [&](int j, Blk &b) {
        b.w4 = word_at(st, L.alead + (uint32_t)j * kQ40Block);
#pragma unroll
        for (int r = 0; r < 4; r++) b.dwb[r] = *reinterpret_cast<const uint16_t *>(st + L.dlead[r] + (uint32_t)j * kQ40Block);
#pragma unroll
        for (int tf = 0; tf < NTF; tf++) {
            const int t = 16 * tf + L.i16;
            const uint32_t *bq = reinterpret_cast<const uint32_t *>(st + kOffB + t * kBTok + 32 * j);
            b.bq[tf][0] = bq[L.g];
            b.bq[tf][1] = bq[4 + L.g];
            b.dx[tf] = *reinterpret_cast<const float *>(st + kOffD + 4 * (j * kTN + t));
        }
    };
    auto run = [&](const Blk &b) {
        // per byte: nibble n -> n - 8 as int8
        const uint32_t lo = (((b.w4 & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        const uint32_t hi = ((((b.w4 >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        const long A = (long)lo | ((long)hi << 32);
        float dw[4];
#pragma unroll
        for (int r = 0; r < 4; r++) dw[r] = f16_bits_to_f32(b.dwb[r]);
        v4i D[NTF];
#pragma unroll
        for (int tf = 0; tf < NTF; tf++)
            D[tf] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, (long)b.bq[tf][0] | ((long)b.bq[tf][1] << 32), v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int tf = 0; tf < NTF; tf++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[tf][r] = __builtin_fmaf((float)D[tf][r], dw[r] * b.dx[tf], acc[tf][r]);
    };
    if constexpr (JN > 0) {
        Blk cur, nxt;
        fetch(0, cur);
#pragma unroll
        for (int j = 0; j < JN; j++) {
            if (j + 1 < JN) fetch(j + 1, nxt);
            run(cur);
            cur = nxt;
            // keep the schedule one block deep (measured: Q at 512 tokens
            // 45.6 us, 46.7 us when later blocks' reads may be hoisted)
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        for (int j = 0; j < jn; j++) {
            Blk b;
            fetch(j, b);
            run(b);
        }
    }
}

}  // namespace

// Workgroup (x, y): rows 64x .. 64x+63, tokens 64y .. 64y+63.  Wave w takes
// rows 16w .. 16w+15 with all 64 tokens (four MFMA fragments per block).
// The K loop runs over segments of kSeg blocks with two LDS stages filled by
// LDS DMA loads (global/buffer -> LDS, no registers): while a segment is
// multiplied, the next one's loads are in flight.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_q40_gemm(Q40Args args) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g = lane >> 4;
    int tile = blockIdx.x, rows_before = 0;
    const Q40Args a = q40_matrix(args, &tile, kTR, &rows_before);
    const int nb = a.nb;
    const uint32_t row_bytes = (uint32_t)nb * kQ40Block;
    const int r0 = tile * kTR, t0 = blockIdx.y * kTN;
    const int nt = min(kTN, a.ntok - t0);
    const int ntf = (nt + 15) >> 4;
    // K range of this workgroup: blocks [kb0, kb1) (split over grid z when
    // the partial sums go to a.part)
    const int ks = gridDim.z, kz = blockIdx.z;
    const int kb0 = kz * nb / ks, kb1 = (kz + 1) * nb / ks;
    const int nseg = (kb1 - kb0 + kSeg - 1) / kSeg;

    // the matrix from the 16-byte boundary at or below its first byte
    const uintptr_t wb = reinterpret_cast<uintptr_t>(a.w);
    const uint32_t le = (uint32_t)(wb & 15u);

    // this thread's LDS DMA loads of a stage: A load i = wave + 4k fills slots
    // 64i..64i+63 (slot q: row q / 11, piece q % 11; piece 10 is padding),
    // B load i = wave + 4k likewise (slot q: token q / 17, piece q % 17;
    // piece 16 is padding), d_x load k: block wave + 4k of token lane; past
    // the rows, tokens or K range the loads read zeros
    const u32x4v rsa = rsrc_words(reinterpret_cast<const void *>(wb - le), (uint32_t)((a.nbytes + le + 15u) & ~15ull));
    const u32x4v rsb = rsrc_words(a.codes, (uint32_t)((size_t)a.ntok * nb * 32));
    const u32x4v rsd = rsrc_words(a.scales, (uint32_t)((size_t)a.ntok * nb * 4));
    uint32_t a_pos[kALoadsMax];
    bool a_ok[kALoadsMax];
#pragma unroll
    for (int k = 0; k < kALoadsMax; k++) {
        const int q = 64 * (wave + kWaves * k) + lane, r = q / kASlots, pc = q - r * kASlots;
        const int row = r0 + r;
        a_ok[k] = wave + kWaves * k < kAInstr && pc < kAPieces && row < a.rows;
        a_pos[k] = le + (uint32_t)(a_ok[k] ? row : 0) * row_bytes + 16u * (uint32_t)pc;
    }
    uint32_t b_tok[kBLoadsMax], b_pc[kBLoadsMax];
    bool b_ok[kBLoadsMax];
#pragma unroll
    for (int k = 0; k < kBLoadsMax; k++) {
        const int q = 64 * (wave + kWaves * k) + lane, t = q / kBSlots, p = q - t * kBSlots;
        b_ok[k] = wave + kWaves * k < kBInstr && t < nt && p < 2 * kSeg;
        b_tok[k] = (uint32_t)(t0 + (t < nt ? t : 0));
        b_pc[k] = (uint32_t)p;
    }
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)lds);
    auto issue = [&](int s) {
        const uint32_t st = lds0 + (uint32_t)(s & 1) * kStageBytes;
        const int b0 = kb0 + s * kSeg;
#pragma unroll
        for (int k = 0; k < kALoadsMax; k++) {
            if (wave + kWaves * k >= kAInstr) continue;  // wave-uniform
            // (pos - 16*piece) rounded down to 16, plus 16*piece
            const uint32_t pos = a_pos[k] + (uint32_t)b0 * kQ40Block;
            dma16(rsa, st + 1024u * (uint32_t)(wave + kWaves * k), a_ok[k] ? (pos & ~15u) : kOOR, 0u);
        }
#pragma unroll
        for (int k = 0; k < kBLoadsMax; k++) {
            if (wave + kWaves * k >= kBInstr) continue;  // wave-uniform
            const int b = b0 + (int)(b_pc[k] >> 1);
            const uint32_t off = (b_ok[k] && b < kb1) ? (b_tok[k] * (uint32_t)nb + (uint32_t)b) * 32u + 16u * (b_pc[k] & 1u) : kOOR;
            dma16(rsb, st + kOffB + 1024u * (uint32_t)(wave + kWaves * k), off, 0u);
        }
#pragma unroll
        for (int k = 0; k < kDLoads; k++) {
            const int b = b0 + wave + kWaves * k;
            const uint32_t off = (lane < nt && b < kb1) ? ((uint32_t)(t0 + lane) * (uint32_t)nb + (uint32_t)b) * 4u : kOOR;
            dma4(rsd, st + kOffD + 256u * (uint32_t)(wave + kWaves * k), off, 0u);
        }
    };

    // this lane's A row (MFMA layout: row i16) and D rows (4g .. 4g+3)
    const int arow = 16 * wave + i16;
    const uint32_t apos = le + (uint32_t)(r0 + arow < a.rows ? r0 + arow : 0) * row_bytes;
    uint32_t dpos[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int row = r0 + 16 * wave + 4 * g + r;
        dpos[r] = le + (uint32_t)(row < a.rows ? row : 0) * row_bytes;
    }
    float acc[4][4];
#pragma unroll
    for (int tf = 0; tf < 4; tf++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[tf][r] = 0.0f;

    // The K loop, instantiated per number of token fragments: the full
    // segments in a loop of their own (one straight-line body, so the
    // accumulators keep their registers), then a last partial segment.
    auto kloop = [&](auto ntf_c) {
        constexpr int NTF = decltype(ntf_c)::value;
        auto lane_of = [&](int s) {
            // window offsets of segment s: A row (nibble bytes 2+4g..5+4g of
            // block j at lead + 18j + 2 + 4g), and the D rows' scales
            const int b0 = kb0 + s * kSeg;
            Q40Lane L;
            L.alead = (uint32_t)arow * kARow + ((apos + (uint32_t)b0 * kQ40Block) & 15u) + 2u + 4u * (uint32_t)g;
#pragma unroll
            for (int r = 0; r < 4; r++)
                L.dlead[r] = (uint32_t)(16 * wave + 4 * g + r) * kARow + ((dpos[r] + (uint32_t)b0 * kQ40Block) & 15u);
            L.i16 = i16;
            L.g = g;
            return L;
        };
        // this wave's loads of segment s have landed; after the barrier
        // every wave's have, and every wave is done with segment s-1, whose
        // stage segment s+1 reuses
        auto wait_stage = [] {
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        };
        const int nfull = (kb1 - kb0) / kSeg;
        issue(0);
        int s = 0;
        for (; s < nfull; s++) {
            wait_stage();
            if (s + 1 < nseg) issue(s + 1);
            q40_blocks<NTF, kSeg>(lds + (size_t)(s & 1) * kStageBytes, lane_of(s), kSeg, acc);
        }
        if (s < nseg) {
            wait_stage();
            q40_blocks<NTF, 0>(lds + (size_t)(s & 1) * kStageBytes, lane_of(s), kb1 - kb0 - kSeg * s, acc);
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

    // y[t][row]: rows 4g .. 4g+3 of the wave's 16 for token 16tf + i16
    const int row = r0 + 16 * wave + 4 * g;
    if (a.part) {
        // partial sums of K range kz, summed in order by k_q40_reduce
#pragma unroll
        for (int tf = 0; tf < 4; tf++) {
            const int t = 16 * tf + i16;
            if (t >= nt) continue;
            float *pp = a.part + (size_t)ks * a.ntok * rows_before + ((size_t)kz * a.ntok + t0 + t) * a.rows + row;
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (row + r < a.rows) pp[r] = acc[tf][r];
        }
        return;
    }
#pragma unroll
    for (int tf = 0; tf < 4; tf++) {
        const int t = 16 * tf + i16;
        if (t >= nt) continue;
        const size_t o = (size_t)(t0 + t) * a.rows + row;
        float *yp = a.y + o;
        if (!a.bias && !a.resid && row + 3 < a.rows && ((reinterpret_cast<uintptr_t>(yp) & 15u) == 0)) {
            *reinterpret_cast<v4f *>(yp) = v4f{acc[tf][0], acc[tf][1], acc[tf][2], acc[tf][3]};
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (row + r < a.rows) q40_store(a, o + r, row + r, acc[tf][r]);
        }
    }
}

// y[t][row] = the K ranges' partial sums added in range order, then the
// projection epilogue; element o of the launch's matrices in order (matrix i
// holds ntok * rows_i of them; its ks partial sums start after the previous
// matrices').
__global__ __launch_bounds__(256) void k_q40_reduce(Q40Args args, int ks, size_t total) {
    size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= total) return;
    int tile = 0, rows_before = 0;
    Q40Args a = args;
    for (int i = 0; i <= args.nmore; i++) {
        int t = tile;
        a = q40_matrix(args, &t, 1, &rows_before);
        const size_t n = (size_t)a.ntok * a.rows;
        if (o < n) break;
        o -= n;
        tile += a.rows;
    }
    const size_t n = (size_t)a.ntok * a.rows;
    const float *pp = a.part + (size_t)ks * a.ntok * rows_before + o;
    float v = pp[0];
    for (int z = 1; z < ks; z++) v = v + pp[(size_t)z * n];
    q40_store(a, o, (int)(o % (size_t)a.rows), v);
}

hipError_t launch_q40_gemm(hipStream_t s, const Q40Args &a) {
    if (a.rows <= 0 || a.ntok <= 0 || a.nb <= 0) return hipSuccess;
    if (a.nmore < 0 || a.nmore > 2) return hipErrorInvalidValue;
    int tiles = (a.rows + kTR - 1) / kTR, rows = a.rows;
    for (int i = 0; i < a.nmore; i++) {
        if (a.more[i].rows <= 0) return hipErrorInvalidValue;
        tiles += (a.more[i].rows + kTR - 1) / kTR;
        rows += a.more[i].rows;
    }
    const int ks = a.part ? (a.nb < kQ40SplitK ? a.nb : kQ40SplitK) : 1;
    dim3 grid(tiles, (a.ntok + kTN - 1) / kTN, ks);
    hipLaunchKernelGGL(k_q40_gemm, grid, dim3(kThreads), 2 * (size_t)kStageBytes, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.part) return e;
    const size_t n = (size_t)a.ntok * rows;
    hipLaunchKernelGGL(k_q40_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a, ks, n);
    return hipGetLastError();
}

}  // namespace spt
