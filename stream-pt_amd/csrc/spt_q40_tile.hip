// spt_q40_tile.hip -- Q4_0 x Q8_0 projections of 5 to 64 tokens, a
// workgroup per 16 or 32 output rows and 16 or 32 tokens, on the gfx950 int8
// MFMA.
//
// forward.MulQ40BatchInto (forward/q40.go:40-103) at the batch sizes of
// continuous-batching decode and short prefill chunks: y[t][row] =
// sum_b float(isum) * (d_w * d_x) with isum = sum (n - 8) * q the exact int32
// block sum.  At these sizes a projection is a few megabytes of weights;
// every workgroup needs its rows' weights (18 bytes per block) and all of
// its tokens' Q8_0 blocks (34 bytes per block), and once they are in LDS its
// multiply is bound by the compute unit's VALU: three ops per output and
// block (the int32 sum to fp32, d_w * d_x, the fma) against one MFMA per
// 256 outputs (32 rows x 32 tokens over 90 blocks: 3.7 us of a 9 us
// workgroup, the loads 2 us).  So the launch takes 16-row tiles when their
// workgroups all run at once, and 32-row tiles (half the workgroups, each
// loading the tokens' blocks once for twice the rows) when they would not;
// 32 tokens per workgroup when both images fit in LDS (inputs up to 91
// blocks).
// Everything is loaded at the start by LDS DMA, 1 KB per wave instruction:
//   * the rows of the tile (GGUF rows are contiguous) and the tokens'
//     GGML Q8_0 blocks ([ntok][nb] x 34 bytes: the caller's, or written by
//     the quantizer just before -- no unpacking launch), each as one run of
//     bytes; when the rows (tokens) start on 16-byte boundaries they are
//     copied row by row to a pitch 16 bytes longer, so that the 16 rows an
//     MFMA operand reads do not meet in one LDS bank (a row of a multiple of
//     128 bytes would put them all in the same bank);
//   * the rows' fp16 d_w are then widened into a [block][row] table (one
//     16-byte read gives the four rows of an MFMA lane's results).
// The K blocks are split over the eight waves (wave w takes blocks w, w + 8,
// ...), each multiplying its blocks for every 16-row half and token
// fragment, the next
// block's LDS reads issued before the current block's MFMAs; the waves'
// partial sums are added in wave order through LDS, so there is no split-K
// scratch and no reduce launch.  The workgroups of one tile's token groups
// are numbered to run on the same XCD, where all but the first find the
// tile's bytes in that XCD's L2.
// MFMA v_mfma_i32_16x16x32_i8: lane l holds A row l%16 and B column l%16 at
// k = 8*(l/16) + 0..7; D lane l, register r is row 4*(l/16) + r, column l%16.
// K order inside a block: lane group g takes elements 8g .. 8g+7, which are
// the low nibbles (g < 2) or high nibbles (g >= 2) of nibble bytes
// 8(g&1) .. 8(g&1)+7, and code bytes 8g .. 8g+7 of the Q8_0 block.
// Per block and output: acc = fma(float(isum), d_w * d_x, acc) (d_w * d_x is
// exact in fp32), blocks in ascending order within a wave, then the waves
// in order.
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr size_t kMaxLds = 160 * 1024;
// The waves' partial sums, [wave][register][lane] with registers kPartPitch
// floats apart: the 32 outputs a half-wave adds (16 or 32 rows of one token)
// then fall in distinct banks.
constexpr int kPartPitch = 66;
__host__ __device__ constexpr uint32_t part_bytes(int rt, int ntf) {
    return (uint32_t)kWaves * rt * ntf * 4 * kPartPitch * 4;
}

// How `n` runs of `len` bytes, `len` apart from byte `first` of a buffer,
// are copied to LDS: pitched (row by row, each run at pitch * i, when every
// run starts on a 16-byte boundary) or as one contiguous copy from the
// 16-byte boundary at or below `first` (run i at lead + len * i).
struct Runs {
    uint32_t pitch, lead, bytes;  // LDS pitch, offset of run 0, LDS bytes used
    bool pitched;
};
__host__ __device__ inline Runs plan_runs(uint32_t first, uint32_t len, int n) {
    Runs r;
    r.pitched = (first & 15u) == 0 && (len & 15u) == 0;
    r.pitch = r.pitched ? len + 16u : len;
    r.lead = r.pitched ? 0u : (first & 15u);
    r.bytes = r.pitched ? r.pitch * (uint32_t)n
                        : (((uint32_t)n * len + r.lead + 1023u) / 1024u) * 1024u;
    r.bytes += 64u;  // the 12-byte reads past a run's last block
    return r;
}

struct TileLayout {
    Runs w, x;
    uint32_t xo, dwo, total;  // LDS offsets of the tokens' image and of the d_w table
};
__host__ __device__ inline TileLayout tile_layout(uint32_t wfirst, uint32_t xfirst, int nb, int rt, int ntf) {
    TileLayout L;
    L.w = plan_runs(wfirst, (uint32_t)nb * kQ40Block, 16 * rt);
    L.x = plan_runs(xfirst, (uint32_t)nb * kQ80Block, 16 * ntf);
    const uint32_t w = L.w.bytes > part_bytes(rt, ntf) ? L.w.bytes : part_bytes(rt, ntf);  // partial sums reuse it
    L.xo = (w + 15u) & ~15u;
    L.dwo = (L.xo + L.x.bytes + 15u) & ~15u;
    L.total = L.dwo + (uint32_t)nb * 16u * (uint32_t)rt * 4u;
    return L;
}

// n -> n - 8 as int8 in each byte of four nibbles (one per byte, low 4 bits)
__device__ __attribute__((always_inline)) inline uint32_t nib_to_s8(uint32_t n) {
    return ((n | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

// The eight LDS bytes at byte o (o even): the three dwords at or after the
// 4-byte boundary below it, read as they are (so that a prefetch does not
// wait for them), then realigned by bytes8().
struct Raw3 {
    uint32_t v0, v1, v2, s;
};
__device__ __attribute__((always_inline)) inline Raw3 lds_raw3(const uint8_t *base, uint32_t o) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(base + (o & ~3u));
    return Raw3{p[0], p[1], p[2], o & 3u};
}
__device__ __attribute__((always_inline)) inline uint2 bytes8(const Raw3 &r) {
    return uint2{__builtin_amdgcn_alignbyte(r.v1, r.v0, r.s), __builtin_amdgcn_alignbyte(r.v2, r.v1, r.s)};
}

// Copies the n runs of `len` bytes at `first` of the view rs into LDS at
// lds as planned, wave w issuing loads w, w + 8, ...; bytes past the view
// read zero.
__device__ __attribute__((always_inline)) inline void stage_runs(const u32x4v &rs, uint32_t lds, uint32_t first,
                                                                 uint32_t len, int n, const Runs &p, bool nt, int wave,
                                                                 int lane) {
    if (p.pitched) {
        const int per = (int)((len / 16u + 63u) / 64u);  // loads per run
        const int chunks = (int)(len / 16u);
        for (int run = wave; run < n; run += kWaves)  // wave-uniform
            for (int part = 0; part < per; part++) {
                const int c = 64 * part + lane;
                if (c < chunks) {
                    const uint32_t m0 = lds + (uint32_t)run * p.pitch + 1024u * (uint32_t)part;
                    const uint32_t off = first + (uint32_t)run * len + 16u * (uint32_t)c;
                    if (nt)
                        dma16_nt(rs, m0, off, 0u);
                    else
                        dma16(rs, m0, off, 0u);
                }
            }
    } else {
        const uint32_t start = first & ~15u;
        const int nl = (int)(((uint32_t)n * len + p.lead + 1023u) / 1024u);
        for (int i = wave; i < nl; i += kWaves) {  // wave-uniform
            const uint32_t off = start + 1024u * (uint32_t)i + 16u * (uint32_t)lane;
            if (nt)
                dma16_nt(rs, lds + 1024u * (uint32_t)i, off, 0u);
            else
                dma16(rs, lds + 1024u * (uint32_t)i, off, 0u);
        }
    }
}

// Workgroup id -> (tile, token group): the groups of a tile on one XCD
// (workgroups go to XCD id % 8 in turn).
struct TileJob {
    int tile, group;
};
__device__ inline TileJob tile_job(int id, int groups) {
    const int rest = id >> 3;
    return TileJob{(rest / groups) * 8 + (id & 7), rest % groups};
}

template <int RT, int NTF>
__global__ __launch_bounds__(kThreads) void k_q40_tile(Q40Args args, int tiles, int groups) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int kRT = RT;             // 16-row halves per tile
    constexpr int kTileRows = 16 * RT;  // rows per workgroup
    constexpr int kTokens = 16 * NTF;   // tokens per workgroup
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15, g = lane >> 4;
    const TileJob job = tile_job(blockIdx.x, groups);
    if (job.tile >= tiles) return;  // the last octet's missing tiles
    int tile = job.tile;
    const Q40Args a = q40_matrix(args, &tile, kTileRows);
    const int nb = a.nb, ntok = a.ntok;
    const uint32_t rb = (uint32_t)nb * kQ40Block, xb = (uint32_t)nb * kQ80Block;
    const int r0 = tile * kTileRows, t0 = job.group * kTokens;

    // 1. the tile's rows and the group's tokens into LDS
    const uintptr_t wa = reinterpret_cast<uintptr_t>(a.w);
    const uint32_t wle = (uint32_t)(wa & 15u);
    const u32x4v rsw = rsrc_words(reinterpret_cast<const void *>(wa - wle), (uint32_t)((a.nbytes + wle + 15u) & ~15ull));
    const uintptr_t xa = reinterpret_cast<uintptr_t>(a.xq34);
    const uint32_t xle = (uint32_t)(xa & 15u);
    const u32x4v rsx =
        rsrc_words(reinterpret_cast<const void *>(xa - xle), (uint32_t)(((uint64_t)ntok * xb + xle + 15u) & ~15ull));
    const uint32_t wfirst = wle + (uint32_t)r0 * rb, xfirst = xle + (uint32_t)t0 * xb;
    const TileLayout L = tile_layout(wfirst, xfirst, nb, RT, NTF);
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_u8 *)lds);
    stage_runs(rsw, lds0, wfirst, rb, kTileRows, L.w, groups == 1, wave, lane);
    stage_runs(rsx, lds0 + L.xo, xfirst, xb, kTokens, L.x, false, wave, lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();

    // 2. the d_w table [block][row], widened: thread k takes row k % 32,
    // blocks k / 32, k / 32 + 16, ... (a wave writes 64 consecutive floats)
    {
        const int row = tid & (kTileRows - 1);
        const uint8_t *rp = lds + L.w.lead + (uint32_t)row * L.w.pitch;
        float *tab = reinterpret_cast<float *>(lds + L.dwo);
        for (int b = tid / kTileRows; b < nb; b += kThreads / kTileRows)
            tab[b * kTileRows + row] = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(rp + (uint32_t)b * kQ40Block));
    }
    lds_barrier();

    // 3. the wave's blocks for both row halves and every token fragment
    float acc[kRT][NTF][4];
#pragma unroll
    for (int h = 0; h < kRT; h++)
#pragma unroll
        for (int tf = 0; tf < NTF; tf++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[h][tf][r] = 0.0f;
    const uint32_t nsh = 4u * (uint32_t)(g >> 1);
    const uint32_t arow = L.w.lead + (uint32_t)i16 * L.w.pitch + 2u + 8u * (uint32_t)(g & 1);
    const uint32_t xrow = L.xo + L.x.lead + (uint32_t)i16 * L.x.pitch;
    const float *dwt = reinterpret_cast<const float *>(lds + L.dwo);
    struct Frag {
        Raw3 a[kRT], bq[NTF];
        v4f_t dw[kRT];
        uint32_t dx[NTF];
    };
    auto fetch = [&](int b, Frag &f) {
#pragma unroll
        for (int h = 0; h < kRT; h++) {
            f.a[h] = lds_raw3(lds, arow + (uint32_t)(16 * h) * L.w.pitch + (uint32_t)b * kQ40Block);
            f.dw[h] = *reinterpret_cast<const v4f_t *>(dwt + b * kTileRows + 16 * h + 4 * g);
        }
#pragma unroll
        for (int tf = 0; tf < NTF; tf++) {
            const uint32_t xo = xrow + (uint32_t)(16 * tf) * L.x.pitch + (uint32_t)b * kQ80Block;
            f.bq[tf] = lds_raw3(lds, xo + 2u + 8u * (uint32_t)g);
            f.dx[tf] = *reinterpret_cast<const uint16_t *>(lds + xo);
        }
    };
    auto run = [&](const Frag &f) {
        long B[NTF];
        float dx[NTF];
#pragma unroll
        for (int tf = 0; tf < NTF; tf++) {
            const uint2 bq = bytes8(f.bq[tf]);
            B[tf] = (long)bq.x | ((long)bq.y << 32);
            dx[tf] = f16_bits_to_f32(f.dx[tf]);
        }
#pragma unroll
        for (int h = 0; h < kRT; h++) {
            const uint2 aw = bytes8(f.a[h]);
            const long A = (long)nib_to_s8((aw.x >> nsh) & 0x0F0F0F0Fu) |
                           ((long)nib_to_s8((aw.y >> nsh) & 0x0F0F0F0Fu) << 32);
#pragma unroll
            for (int tf = 0; tf < NTF; tf++) {
                const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B[tf], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[h][tf][r] = __builtin_fmaf((float)D[r], f.dw[h][r] * dx[tf], acc[h][tf][r]);
            }
        }
    };
    // blocks wave + 8j, j < nw, in two register sets that alternate (no
    // copies between iterations, which would wait for a whole prefetch);
    // a fetch past the wave's last block reads its last block again, unused
    const int nw = wave < nb ? (nb - wave + kWaves - 1) / kWaves : 0;
    const int last = wave + kWaves * (nw - 1);
    auto blk = [&](int j) { return min(wave + kWaves * j, last); };
    if (nw > 0) {
        Frag f0, f1;
        fetch(blk(0), f0);
        int j = 0;
        // the barriers keep each fetch's reads issued before the multiply
        // that overlaps them
        for (; j + 2 <= nw; j += 2) {
            fetch(blk(j + 1), f1);
            __builtin_amdgcn_sched_barrier(0);
            run(f0);
            __builtin_amdgcn_sched_barrier(0);
            fetch(blk(j + 2), f0);
            __builtin_amdgcn_sched_barrier(0);
            run(f1);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (j < nw) run(f0);
    }

    // 4. the waves' partial sums (over the weights image, every wave done
    // with it) added in wave order; thread k takes row k % tile rows of
    // token k / tile rows
    constexpr int kRegs = kRT * NTF * 4;
    lds_barrier();
    float *part = reinterpret_cast<float *>(lds);  // [wave][h][tf][r] x kPartPitch + lane
#pragma unroll
    for (int h = 0; h < kRT; h++)
#pragma unroll
        for (int tf = 0; tf < NTF; tf++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                part[(wave * kRegs + (h * NTF + tf) * 4 + r) * kPartPitch + lane] = acc[h][tf][r];
    lds_barrier();
#pragma unroll
    for (int k = tid; k < kTileRows * kTokens; k += kThreads) {
        const int rho = k & (kTileRows - 1), tl = k / kTileRows;
        const int h = rho >> 4, rr = rho & 15, tf = tl >> 4;
        const int reg = ((h * NTF + tf) * 4 + (rr & 3)) * kPartPitch + 16 * (rr >> 2) + (tl & 15);
        float v = part[reg];
#pragma unroll
        for (int w = 1; w < kWaves; w++) v = v + part[w * kRegs * kPartPitch + reg];
        const int row = r0 + rho, t = t0 + tl;
        if (row < a.rows && t < ntok) q40_store(a, (size_t)t * a.rows + row, row, v);
    }
}

// The LDS the tile launch needs for an input of nb blocks, 16 * rt rows and
// 16 * ntf tokens per workgroup: the largest of the plans for
// 16-byte-aligned runs (pitched) and for runs at the largest even lead
// (14 bytes) of a contiguous copy.
size_t q40_tile_lds(int nb, int rt, int ntf) {
    size_t worst = 0;
    for (uint32_t wle : {0u, 14u})
        for (uint32_t xle : {0u, 14u}) {
            const size_t t = tile_layout(wle, xle, nb, rt, ntf).total;
            worst = t > worst ? t : worst;
        }
    return worst;
}

// Tokens per workgroup: 32 when they and a 32-row tile fit in LDS, else 16.
int tile_tokens(int nb) { return q40_tile_lds(nb, 2, 2) <= kMaxLds ? 32 : 16; }

// Workgroups of a launch over rt x 16-row tiles and 16 * ntf tokens.
int tile_grid(const Q40Args &a, int rt, int ntf) {
    const int tr = 16 * rt;
    int tiles = (a.rows + tr - 1) / tr;
    for (int i = 0; i < a.nmore; i++) tiles += (a.more[i].rows + tr - 1) / tr;
    const int groups = (a.ntok + 16 * ntf - 1) / (16 * ntf);
    return (tiles + 7) / 8 * 8 * groups;
}

template <int RT, int NTF>
hipError_t launch_shape(hipStream_t s, const Q40Args &a) {
    constexpr int kTileRows = 16 * RT;
    const size_t lds = q40_tile_lds(a.nb, RT, NTF);
    if (lds > kMaxLds) return hipErrorInvalidConfiguration;
    // one-time opt-in to more than 64 KB of dynamic LDS
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&k_q40_tile<RT, NTF>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
    if (attr != hipSuccess) return attr;
    int nt = (a.rows + kTileRows - 1) / kTileRows;
    for (int i = 0; i < a.nmore; i++) nt += (a.more[i].rows + kTileRows - 1) / kTileRows;
    const int groups = (a.ntok + 16 * NTF - 1) / (16 * NTF);
    hipLaunchKernelGGL((k_q40_tile<RT, NTF>), dim3(tile_grid(a, RT, NTF)), dim3(kThreads), lds, s, a, nt, groups);
    return hipGetLastError();
}

}  // namespace

bool q40_tile_form(int64_t batch, int64_t nb) {
    if (batch < kQ40TileMinTokens || batch > kQ40TileMaxTokens || nb < 1 || nb > kQ40TileMaxNb) return false;
    return batch <= 2 * tile_tokens((int)nb);
}

hipError_t launch_q40_tile(hipStream_t s, const Q40Args &a, int n_cu) {
    if (a.rows <= 0 || a.ntok <= 0 || a.nb <= 0) return hipSuccess;
    if (a.nmore < 0 || a.nmore > 2 || !a.xq34 || a.nb > kQ40TileMaxNb || a.ntok > kQ40TileMaxTokens || n_cu <= 0)
        return hipErrorInvalidValue;
    for (int i = 0; i < a.nmore; i++)
        if (a.more[i].rows <= 0) return hipErrorInvalidValue;
    const int ntf = a.ntok > 16 && tile_tokens(a.nb) == 32 ? 2 : 1;
    // 16-row tiles when their workgroups all run at once (as many as the LDS
    // lets each compute unit hold), else 32-row tiles: the multiply is bound
    // by the compute unit's VALU (three ops per output and block), so twice
    // the workgroups on idle compute units halve it, while a second round
    // of workgroups costs a whole workgroup's time again.
    const int per_cu = (int)(kMaxLds / q40_tile_lds(a.nb, 1, ntf));
    const bool rows16 = tile_grid(a, 1, ntf) <= n_cu * per_cu;
    if (rows16) return ntf == 2 ? launch_shape<1, 2>(s, a) : launch_shape<1, 1>(s, a);
    return ntf == 2 ? launch_shape<2, 2>(s, a) : launch_shape<2, 1>(s, a);
}

}  // namespace spt
