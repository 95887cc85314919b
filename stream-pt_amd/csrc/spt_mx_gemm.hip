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
#include "spt_device.h"
#include "spt_kernels.h"

namespace spt {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 256;               // weight rows per work item (gate/up: 128 gate + 128 up)
constexpr int kBN = kGemmTokens;       // list entries per work item
constexpr int kSeg = 6;                // 32-element blocks per K segment
constexpr int kAPieces = 8;            // 16-byte loads per row and segment
constexpr int kARow = 144;             // LDS bytes per staged row (36 dwords: rows spread over banks)
constexpr int kBTok = kSeg * 64 + 16;  // LDS bytes per staged token (100 dwords)
constexpr int kOffE = kBM * kARow;      // E8M0 bytes [row][8]
constexpr int kOffB = kOffE + kBM * 8;  // bf16 code tables [token][block][64 B]
constexpr int kOffD = kOffB + kBN * kBTok;  // d_x [token][8]
constexpr int kStageBytes = kOffD + kBN * 8 * 4;
constexpr int kEMin = 4, kEMax = 240;
// After the K loop the stage buffers hold the special-row values (per wave
// 2 x 16 rows x 64 tokens) and the gate/up exchange ([token][128 rows]).
constexpr int kFixBytes = kWaves * 2 * 16 * kBN * 4;
constexpr int kXTok = 128 * 4 + 16;
static_assert(kSeg * kMxBlock + 15 <= 16 * kAPieces, "a row's segment fits its loads");
static_assert(16 * kAPieces <= kARow, "row stride");
static_assert(kFixBytes + kBN * kXTok <= 2 * kStageBytes, "epilogue areas");
static_assert(kBM * kAPieces % kThreads == 0 && kBN * kSeg * 4 % kThreads == 0, "stage loads");
constexpr int kALoads = kBM * kAPieces / kThreads;  // 4
constexpr int kBLoads = kBN * kSeg * 4 / kThreads;  // 3

__device__ inline rsrc_t expert_rsrc(const uint8_t *w, uint64_t expert_bytes, int e, uint32_t *le) {
    // from the 16-byte boundary at or below the matrix's first byte to the
    // one at or above its end (a 16-byte load crossing the range's end reads
    // zeros; the bytes up to that boundary share the last byte's page)
    const uintptr_t mb = reinterpret_cast<uintptr_t>(w + (uint64_t)e * expert_bytes);
    *le = (uint32_t)(mb & 15u);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(mb - *le), (short)0,
                                             (int)(uint32_t)((expert_bytes + *le + 15u) & ~15ull), kRsrcWord3);
}

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

}  // namespace

// Persistent workgroups of eight waves.  Work items are (GEMM expert, unit of
// output rows, tile of 64 list entries), ordered so the token tiles of one
// unit are consecutive (they share the unit's weight rows through the
// caches); workgroup b takes items b, b + G, b + 2G, ...  Gate/up units are
// 128 output rows (weight rows 0-127 of the item gate, 128-255 up, so the
// SwiGLU and the Q8_0 of act stay in the workgroup); down units are 256 rows.
// Wave w multiplies weight rows 32w .. 32w+31 of the item with all 64
// entries: 2 x 4 MFMA tiles per block.
//
// The K loop runs over segments of kSeg blocks with two LDS stages: while a
// segment is multiplied, the next one's loads are in flight in registers;
// they are written to the other stage after the multiply, then one barrier.
template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_mx_gemm(MxGemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int s_spec[kBM];  // item tag where the row has a special E8M0

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = a.nb;
    const uint32_t row_bytes = (uint32_t)nb * kMxBlock;
    const int unit_rows = MODE == kGateUp ? kBM / 2 : kBM;
    const int units = (a.rows + unit_rows - 1) / unit_rows;
    const int n_slots = *a.gm_n;
    const int total = n_slots > 0 ? a.gm_tile_off[n_slots] * units : 0;
    if ((int)blockIdx.x >= total) return;
    for (int i = tid; i < kBM; i += kThreads) s_spec[i] = 0;
    __syncthreads();

    const int i16 = lane & 15, g = lane >> 4;
    const int nseg = (nb + kSeg - 1) / kSeg;
    int tag = 0;
    for (int it = blockIdx.x; it < total; it += gridDim.x) {
        ++tag;
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

        // weight rows of this item: LDS row r (0..255) -> matrix m, row
        uint32_t le0 = 0, le1 = 0;
        const rsrc_t rs0 = expert_rsrc(a.w[0], a.expert_bytes, e, &le0);
        const rsrc_t rs1 = MODE == kGateUp ? expert_rsrc(a.w[1], a.expert_bytes, e, &le1) : rs0;
        if (MODE != kGateUp) le1 = le0;
        auto mrow = [&](int r) { return MODE == kGateUp ? u * (kBM / 2) + (r & (kBM / 2 - 1)) : u * kBM + r; };

        // this thread's stage loads: A pieces k (rows tid/8 + 64k), B pieces,
        // d_x entry; entries past nt read nothing
        uint32_t a_pos[kALoads];
        bool a_ok[kALoads];
#pragma unroll
        for (int k = 0; k < kALoads; k++) {
            const int p = tid + kThreads * k, r = p >> 3;
            const int row = mrow(r);
            a_ok[k] = row < a.rows;
            a_pos[k] = ((k < kALoads / 2 || MODE != kGateUp) ? le0 : le1) + (uint32_t)(a_ok[k] ? row : 0) * row_bytes;
        }
        int64_t b_row[kBLoads];
#pragma unroll
        for (int k = 0; k < kBLoads; k++) {
            const int t = (tid + kThreads * k) / (kSeg * 4);
            int ar = -1;
            if (t < nt) {
                const int ent = a.list[begin + t];
                ar = MODE == kGateUp ? ent / a.topk : ent;
            }
            b_row[k] = ar < 0 ? -1 : (int64_t)ar * nb;
        }
        int64_t d_row = -1;
        if (tid < kBN * kSeg) {
            const int t = tid / kSeg;
            if (t < nt) {
                const int ent = a.list[begin + t];
                d_row = (int64_t)(MODE == kGateUp ? ent / a.topk : ent) * nb;
            }
        }

        u32x4 ra[kALoads], rb[kBLoads];
        float rd = 0.0f;
        auto stage_load = [&](int s) {
            const int b0 = s * kSeg;
#pragma unroll
            for (int k = 0; k < kALoads; k++) {
                const int pc = tid & 7;
                const uint32_t off = ((a_pos[k] + (uint32_t)b0 * kMxBlock) & ~15u) + 16u * pc;
                const rsrc_t rs = (k < kALoads / 2 || MODE != kGateUp) ? rs0 : rs1;
                ra[k] = a_ok[k] ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0))
                                : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int k = 0; k < kBLoads; k++) {
                const int q = (tid + kThreads * k) % (kSeg * 4), j = q >> 2, sub = q & 3;
                u32x4 v = {0u, 0u, 0u, 0u};
                if (b_row[k] >= 0 && b0 + j < nb)
                    v = *reinterpret_cast<const u32x4 *>(a.btab + ((size_t)(b_row[k] + b0 + j) * 16 + 4 * sub));
                rb[k] = v;
            }
            rd = 0.0f;
            if (d_row >= 0) {
                const int j = tid % kSeg;
                if (b0 + j < nb) rd = a.scales[d_row + b0 + j];
            }
        };
        auto stage_store = [&](int s) {
            uint8_t *st = lds + (size_t)(s & 1) * kStageBytes;
            const int b0 = s * kSeg;
            const int jn = min(kSeg, nb - b0);
#pragma unroll
            for (int k = 0; k < kALoads; k++) {
                const int p = tid + kThreads * k, r = p >> 3, pc = p & 7;
                *reinterpret_cast<u32x4 *>(st + r * kARow + 16 * pc) = ra[k];
                // the E8M0 byte of block j sits at lead + 17j of the row's
                // window; at most one falls in each 16-byte piece
                const int lead = (int)((a_pos[k] + (uint32_t)b0 * kMxBlock) & 15u);
                const int num = 16 * pc - lead;
                const int j = num <= 0 ? 0 : (num + 16) / 17;
                const int pos = lead + 17 * j - 16 * pc;
                if (pos < 16 && j < jn) {
                    const uint32_t w = pos < 4 ? ra[k].x : pos < 8 ? ra[k].y : pos < 12 ? ra[k].z : ra[k].w;
                    const uint32_t ev = (w >> (8 * (pos & 3))) & 0xFFu;
                    st[kOffE + r * 8 + j] = (uint8_t)ev;
                    if (a_ok[k] && (ev < (uint32_t)kEMin || ev > (uint32_t)kEMax)) s_spec[r] = tag;
                }
            }
#pragma unroll
            for (int k = 0; k < kBLoads; k++) {
                const int p = tid + kThreads * k, t = p / (kSeg * 4), q = p % (kSeg * 4);
                *reinterpret_cast<u32x4 *>(st + kOffB + t * kBTok + 64 * (q >> 2) + 16 * (q & 3)) = rb[k];
            }
            if (tid < kBN * kSeg) {
                const int t = tid / kSeg, j = tid % kSeg;
                *reinterpret_cast<float *>(st + kOffD + (t * 8 + j) * 4) = rd;
            }
        };

        // this lane's A rows (LDS rows 32*wave + 16*rf + i16) and their
        // window offsets
        uint32_t l_pos[2];
#pragma unroll
        for (int rf = 0; rf < 2; rf++) {
            const int r = 32 * wave + 16 * rf + i16;
            const int row = mrow(r);
            l_pos[rf] = ((MODE == kGateUp && r >= kBM / 2) ? le1 : le0) + (uint32_t)(row < a.rows ? row : 0) * row_bytes;
        }
        float acc[2][4][4];
#pragma unroll
        for (int rf = 0; rf < 2; rf++)
#pragma unroll
            for (int tf = 0; tf < 4; tf++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[rf][tf][r] = 0.0f;

        stage_load(0);
        stage_store(0);
        __syncthreads();
        for (int s = 0; s < nseg; s++) {
            if (s + 1 < nseg) stage_load(s + 1);
            const uint8_t *st = lds + (size_t)(s & 1) * kStageBytes;
            const int b0 = s * kSeg;
            const int jn = min(kSeg, nb - b0);
            // per row fragment: E8M0 bytes of the segment, and for blocks
            // j = jj + 4m the dword offset (jj) + 68m and byte shift of this
            // lane's four nibble bytes (1 + 4g .. 4 + 4g of the block)
            u32x2 ev[2];
            uint32_t aoff[2][4], ash[2][4];
#pragma unroll
            for (int rf = 0; rf < 2; rf++) {
                const int r = 32 * wave + 16 * rf + i16;
                ev[rf] = *reinterpret_cast<const u32x2 *>(st + kOffE + r * 8);
                const uint32_t lead = (l_pos[rf] + (uint32_t)b0 * kMxBlock) & 15u;
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const uint32_t o = lead + 1u + 4u * (uint32_t)g + 17u * (uint32_t)jj;
                    aoff[rf][jj] = (uint32_t)r * kARow + (o & ~3u);
                    ash[rf][jj] = o & 3u;
                }
            }
#pragma unroll
            for (int j = 0; j < kSeg; j++) {
                if (j >= jn) break;
                const int jj = j & 3, m = j >> 2;
                bf16x8 A[2];
#pragma unroll
                for (int rf = 0; rf < 2; rf++) {
                    const uint32_t *pw = reinterpret_cast<const uint32_t *>(st + aoff[rf][jj] + 68 * m);
                    const uint32_t w4 = __builtin_amdgcn_alignbyte(pw[1], pw[0], ash[rf][jj]);
                    const uint32_t eb = ((j < 4 ? ev[rf].x : ev[rf].y) >> (8 * (j & 3))) & 0xFFu;
                    const float sc = __uint_as_float(eb << 23);
                    u32x4 av;
                    av.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 0));
                    av.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 1));
                    av.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 2));
                    av.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w4, sc, 3));
                    A[rf] = __builtin_bit_cast(bf16x8, av);
                }
                bf16x8 B[4];
                float dx[4];
#pragma unroll
                for (int tf = 0; tf < 4; tf++) {
                    const int t = 16 * tf + i16;
                    B[tf] = *reinterpret_cast<const bf16x8 *>(st + kOffB + t * kBTok + 64 * j + 16 * g);
                    dx[tf] = *reinterpret_cast<const float *>(st + kOffD + (t * 8 + j) * 4);
                }
                v4f D[2][4];
#pragma unroll
                for (int rf = 0; rf < 2; rf++)
#pragma unroll
                    for (int tf = 0; tf < 4; tf++)
                        D[rf][tf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[rf], B[tf], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                for (int rf = 0; rf < 2; rf++)
#pragma unroll
                    for (int tf = 0; tf < 4; tf++)
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[rf][tf][r] = __builtin_fmaf(D[rf][tf][r], dx[tf], acc[rf][tf][r]);
            }
            if (s + 1 < nseg) stage_store(s + 1);
            __syncthreads();
        }

        // entries of this lane's token columns
        int ent[4];
#pragma unroll
        for (int tf = 0; tf < 4; tf++) {
            const int t = 16 * tf + i16;
            ent[tf] = t < nt ? a.list[begin + t] : -1;
        }

        // rows with special E8M0 bytes: the integer decode, one token per
        // lane, through LDS into the accumulators
        {
            const bool mine = lane < 32 && s_spec[32 * wave + lane] == tag;
            const uint64_t sm = __ballot(mine);
            if (sm) {
                float *fix = reinterpret_cast<float *>(lds) + wave * 2 * 16 * kBN;
                int ar = -1;
                if (lane < nt) {
                    const int en = a.list[begin + lane];
                    ar = MODE == kGateUp ? en / a.topk : en;
                }
                for (int rr = 0; rr < 32; rr++) {
                    if (!((sm >> rr) & 1ull)) continue;
                    const int r = 32 * wave + rr;
                    const bool up = MODE == kGateUp && r >= kBM / 2;
                    const ByteView cv = make_view((up ? a.w[1] : a.w[0]) + (uint64_t)e * a.expert_bytes, a.expert_bytes);
                    float v = 0.0f;
                    if (ar >= 0)
                        v = lut_dot(cv, (uint32_t)mrow(r) * row_bytes, nb, a.codes + (size_t)ar * nb * 32,
                                    a.scales + (size_t)ar * nb);
                    fix[rr * kBN + lane] = v;
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
                for (int rf = 0; rf < 2; rf++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int rr = 16 * rf + 4 * g + r;
                        if ((sm >> rr) & 1ull) {
#pragma unroll
                            for (int tf = 0; tf < 4; tf++) acc[rf][tf][r] = fix[rr * kBN + 16 * tf + i16];
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
        } else {
            // gate (waves 0-3) and up (waves 4-7) rows of output rows
            // u*128 + 32*(wave&3) + 16*rf + 4g + r; up values go to the gate
            // waves through LDS
            const int w4 = wave & 3;
            const bool is_up = wave >= 4;
            float *xch = reinterpret_cast<float *>(lds + kFixBytes);
            float val[2][4][4];
#pragma unroll
            for (int rf = 0; rf < 2; rf++) {
                const int row = u * (kBM / 2) + 32 * w4 + 16 * rf + 4 * g;
                float bsum[4];
#pragma unroll
                for (int r = 0; r < 4; r++)
                    bsum[r] = row < a.rows ? bias_at(a.bias[is_up ? 1 : 0], a.bias_type[is_up ? 1 : 0], (uint64_t)e * a.rows + row + r) : 0.0f;
#pragma unroll
                for (int tf = 0; tf < 4; tf++)
#pragma unroll
                    for (int r = 0; r < 4; r++) val[rf][tf][r] = acc[rf][tf][r] + bsum[r];
            }
            if (is_up) {
#pragma unroll
                for (int rf = 0; rf < 2; rf++)
#pragma unroll
                    for (int tf = 0; tf < 4; tf++) {
                        const int t = 16 * tf + i16;
                        const int lr = 32 * w4 + 16 * rf + 4 * g;
                        *reinterpret_cast<v4f *>(reinterpret_cast<uint8_t *>(xch) + t * kXTok + lr * 4) =
                            v4f{val[rf][tf][0], val[rf][tf][1], val[rf][tf][2], val[rf][tf][3]};
                    }
            }
            __syncthreads();
            if (!is_up) {
                const int blk_row = u * (kBM / 2) + 32 * w4;  // first output row of this wave's Q8_0 block
                const bool blk_ok = blk_row < a.rows;
                const int nbo = a.rows / 32;
#pragma unroll
                for (int tf = 0; tf < 4; tf++) {
                    const int t = 16 * tf + i16;
                    float act[2][4];
                    float amax = 0.0f;
                    bool nan = false;
#pragma unroll
                    for (int rf = 0; rf < 2; rf++) {
                        const int lr = 32 * w4 + 16 * rf + 4 * g;
                        const v4f uv = *reinterpret_cast<const v4f *>(reinterpret_cast<const uint8_t *>(xch) + t * kXTok + lr * 4);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const float v = swiglu(val[rf][tf][r], uv[r]);
                            act[rf][r] = v;
                            const float av = __builtin_fabsf(v);
                            nan |= av != av;
                            amax = av > amax ? av : amax;
                        }
                        const int row = blk_row + 16 * rf + 4 * g;
                        if (ent[tf] >= 0 && row < a.rows) {
                            const size_t o = (size_t)ent[tf] * a.rows + row;
                            if (a.tap[0]) *reinterpret_cast<v4f *>(a.tap[0] + o) = v4f{val[rf][tf][0], val[rf][tf][1], val[rf][tf][2], val[rf][tf][3]};
                            if (a.tap[1]) *reinterpret_cast<v4f *>(a.tap[1] + o) = uv;
                            if (a.out) *reinterpret_cast<v4f *>(a.out + o) = v4f{act[rf][0], act[rf][1], act[rf][2], act[rf][3]};
                        }
                    }
                    // Q8_0 of the 32-element block (rows 4g+r and 16+4g+r of
                    // the four lanes i16, i16+16, i16+32, i16+48)
                    amax = fmaxf(amax, __shfl_xor(amax, 16));
                    amax = fmaxf(amax, __shfl_xor(amax, 32));
                    const uint64_t nm = __ballot(nan);
                    const bool nan_any = ((nm >> i16) & 0x0001000100010001ull) != 0;
                    const float d = nan_any ? __builtin_nanf("") : amax / 127.0f;
                    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
                    const uint16_t dh = f32_to_f16_bits(d);
                    int q[2][4];
#pragma unroll
                    for (int rf = 0; rf < 2; rf++)
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const float rq = __builtin_roundf(act[rf][r] * id);
                            q[rf][r] = (rq != rq) ? 0 : (rq > 127.0f ? 127 : (rq < -127.0f ? -127 : (int)rq));
                        }
                    if (ent[tf] >= 0 && blk_ok) {
                        const size_t blk = (size_t)ent[tf] * nbo + blk_row / 32;
#pragma unroll
                        for (int rf = 0; rf < 2; rf++) {
                            const uint32_t cw = (uint32_t)(q[rf][0] & 0xff) | ((uint32_t)(q[rf][1] & 0xff) << 8) |
                                                ((uint32_t)(q[rf][2] & 0xff) << 16) | ((uint32_t)(q[rf][3] & 0xff) << 24);
                            if (a.act_codes) *reinterpret_cast<uint32_t *>(a.act_codes + blk * 32 + 16 * rf + 4 * g) = cw;
                            if (a.act_blocks34) {
#pragma unroll
                                for (int r = 0; r < 4; r++) a.act_blocks34[blk * kQ80Block + 2 + 16 * rf + 4 * g + r] = (uint8_t)q[rf][r];
                            }
                        }
                        if (g == 0) {
                            if (a.act_scales) a.act_scales[blk] = f16_bits_to_f32(dh);
                            if (a.act_blocks34) {
                                a.act_blocks34[blk * kQ80Block] = (uint8_t)(dh & 0xff);
                                a.act_blocks34[blk * kQ80Block + 1] = (uint8_t)(dh >> 8);
                            }
                        }
                        if (a.act_mxtab) {
                            // nibble position 2*el' + h of elements (4g+r, 16+4g+r): 8g + 2r + {0,1}
                            u32x2 hw, lw;
                            hw.x = e4m3_small(q[0][0] >> 4) | (e4m3_small(q[1][0] >> 4) << 8) | (e4m3_small(q[0][1] >> 4) << 16) | (e4m3_small(q[1][1] >> 4) << 24);
                            hw.y = e4m3_small(q[0][2] >> 4) | (e4m3_small(q[1][2] >> 4) << 8) | (e4m3_small(q[0][3] >> 4) << 16) | (e4m3_small(q[1][3] >> 4) << 24);
                            lw.x = e4m3_small(q[0][0] & 15) | (e4m3_small(q[1][0] & 15) << 8) | (e4m3_small(q[0][1] & 15) << 16) | (e4m3_small(q[1][1] & 15) << 24);
                            lw.y = e4m3_small(q[0][2] & 15) | (e4m3_small(q[1][2] & 15) << 8) | (e4m3_small(q[0][3] & 15) << 16) | (e4m3_small(q[1][3] & 15) << 24);
                            *reinterpret_cast<u32x2 *>(a.act_mxtab + blk * 64 + 8 * g) = hw;
                            *reinterpret_cast<u32x2 *>(a.act_mxtab + blk * 64 + 32 + 8 * g) = lw;
                        }
                        if (a.act_btab) {
                            const u32x4 bw = {bf16_code_pair(q[0][0], q[1][0]), bf16_code_pair(q[0][1], q[1][1]),
                                              bf16_code_pair(q[0][2], q[1][2]), bf16_code_pair(q[0][3], q[1][3])};
                            *reinterpret_cast<u32x4 *>(a.act_btab + blk * 16 + 4 * g) = bw;
                        }
                    }
                }
            }
        }
        // every wave is done with the epilogue areas before the next item's
        // first stage is written over them
        __syncthreads();
    }
}

hipError_t launch_mx_gemm(hipStream_t s, GemvMode mode, const MxGemmArgs &a, int max_items) {
    if (max_items <= 0 || a.rows <= 0 || a.nb <= 0) return hipSuccess;
    constexpr size_t lds = 2 * (size_t)kStageBytes;
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
