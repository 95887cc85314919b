// spt_device.h -- gfx950 device helpers shared by the quantized-MoE kernels.
//
// Block formats (GGUF layout, unchanged in HBM):
//   MXFP4 (type 39, 17 B): byte 0 = E8M0 exponent e, bytes 1..16 = 32 E2M1
//     codes; element i = low nibble of byte 1+i, element i+16 = high nibble
//     (forward/mxfp4.go:52-59).
//   Q4_0 (type 2, 18 B): fp16 d, then 16 bytes of nibbles n, w = (n-8)*d,
//     same element order (forward/quant_portable.go:66-72).
//   Q8_0 (type 8, 34 B): fp16 d, then 32 int8 (forward/q80.go:15-18).
//
// Activations are held on device as split Q8_0: int8 codes [rows][K] and
// fp32 scales [rows][K/32] (the fp16 d widened exactly), so the 32 codes of a
// block are 8 aligned dwords that feed v_dot4_i32_i8 directly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spt {

constexpr int kMxBlock = 17;
constexpr int kQ40Block = 18;
constexpr int kQ80Block = 34;

// gfx9 raw buffer descriptor word 3 (DATA_FORMAT=32, no swizzle).
constexpr int kRsrcWord3 = 0x00020000;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer descriptor as four dwords (for inline assembly).
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// LDS DMA load (buffer -> LDS, no registers): lane l's `bytes` land at LDS
// address lds + bytes * l.  Issued with inline assembly so that the
// compiler, which cannot tell which stage an LDS read touches, does not
// wait for every load in flight before each LDS read; the kernel waits for
// them itself (s_waitcnt vmcnt in stage order).  Five wait
// states open each load: M0, the descriptor and the offset may have just
// been written (by SALU, or by VALU for SGPRs), which an LDS DMA must not see
// early, and the compiler cannot pad inside inline assembly.
__device__ inline void dma16(const u32x4v &rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds)
                 : "memory");
}
// The same for a stream read once (weights): nontemporal, which lets a
// streaming read reach about 7.0 TB/s on MI355X against 6.1 TB/s without.
__device__ inline void dma16_nt(const u32x4v &rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds" ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds)
                 : "memory");
}
// dma16 without the memory clobber, for a load issued in the middle of the
// reads of another stage: it writes only LDS that nothing reads before the
// next full wait and barrier (which are memory clobbers themselves), so the
// compiler may keep scheduling the surrounding LDS reads across it.
__device__ inline void dma16_other_stage(const u32x4v &rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds));
}
__device__ inline void dma4(const u32x4v &rs, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds)
                 : "memory");
}

__device__ inline u32x4v rsrc_words(const void *base, uint32_t nbytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    return u32x4v{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, nbytes, (uint32_t)kRsrcWord3};
}

// A bounds-checked view of `nbytes` bytes at `p`: the descriptor base is p
// rounded down to 4 bytes and `lead` (0..3) is p's offset inside it, so every
// dword load stays aligned; dwords wholly past the end read as zero.
struct ByteView {
    rsrc_t r;
    uint32_t lead;
};

__device__ inline ByteView make_view(const void *p, uint64_t nbytes) {
    uintptr_t a = reinterpret_cast<uintptr_t>(p);
    uint32_t lead = static_cast<uint32_t>(a & 3u);
    uint64_t nrec = (nbytes + lead + 3u) & ~uint64_t(3);
    ByteView v;
    v.r = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(a - lead), (short)0,
                                            (int)(uint32_t)nrec, kRsrcWord3);
    v.lead = lead;
    return v;
}

// Five consecutive aligned dwords covering bytes [pos, pos+17) of the view;
// *o = pos & 3 is the offset of byte `pos` inside the first dword.
__device__ inline void load_block5(const ByteView &v, uint32_t pos, uint32_t d[5], uint32_t *o) {
    uint32_t p = pos + v.lead;
    uint32_t base = p & ~3u;
    *o = p & 3u;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(v.r, base, 0, 0));
    d[0] = q.x;
    d[1] = q.y;
    d[2] = q.z;
    d[3] = q.w;
    d[4] = __builtin_amdgcn_raw_buffer_load_b32(v.r, base + 16, 0, 0);
}

// The same five dwords when the caller already knows pos & 3.
__device__ inline void load_block5_raw(const ByteView &v, uint32_t pos, uint32_t d[5]) {
    uint32_t base = (pos + v.lead) & ~3u;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(v.r, base, 0, 0));
    d[0] = q.x;
    d[1] = q.y;
    d[2] = q.z;
    d[3] = q.w;
    d[4] = __builtin_amdgcn_raw_buffer_load_b32(v.r, base + 16, 0, 0);
}

// Workgroup barrier ordering LDS only: kernels whose waves communicate
// through LDS alone use it in place of __syncthreads(), which would also wait
// for every outstanding global load (draining the loads kept in flight).
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- fp16 -----------------------------------------------------------------
__device__ inline float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// Round-to-nearest-even fp32 -> fp16 bits; NaN becomes 0x7e00 | sign.
__device__ inline uint16_t f32_to_f16_bits(float f) {
    if (f != f) return static_cast<uint16_t>(((__float_as_uint(f) >> 16) & 0x8000u) | 0x7e00u);
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// forward/layer.go:279-303 (readFloatVector) element decode: F32, F16, BF16.
__device__ inline float bias_at(const void *p, int type, uint64_t i) {
    if (!p) return 0.0f;
    if (type == 1) return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
    if (type == 30) return __uint_as_float(uint32_t(reinterpret_cast<const uint16_t *>(p)[i]) << 16);
    return reinterpret_cast<const float *>(p)[i];
}

// The same decode through a buffer descriptor: an absent bias is a zero-length
// range, so the load is issued unconditionally and reads 0.
struct BiasView {
    rsrc_t r;
    int type;
};

__device__ inline BiasView make_bias_view(const void *p, uint64_t nbytes, int type) {
    BiasView v;
    // whole dwords: the last 2-byte element of an odd count sits in a dword
    // that crosses the end, and a load crossing the range's end reads zero
    const uint64_t nw = (nbytes + 3u) & ~uint64_t(3);
    const uint32_t n = p ? (uint32_t)(nw < 0xFFFFFFF0ull ? nw : 0xFFFFFFF0ull) : 0u;
    v.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)n, kRsrcWord3);
    v.type = p ? type : 0;
    return v;
}

// Raw dword holding element i (one load for every type, no branch), then the
// conversion where the value is used.
__device__ inline uint32_t bias_raw(const BiasView &v, uint32_t i) {
    const uint32_t off = v.type == 0 ? i * 4u : (i * 2u) & ~3u;
    return __builtin_amdgcn_raw_buffer_load_b32(v.r, off, 0, 0);
}

__device__ inline float bias_value(const BiasView &v, uint32_t raw, uint32_t i) {
    const uint32_t h = (i & 1u) ? raw >> 16 : raw & 0xFFFFu;
    if (v.type == 1) return f16_bits_to_f32(h);
    if (v.type == 30) return __uint_as_float(h << 16);
    return __uint_as_float(raw);
}

// ---- MXFP4 block decode ------------------------------------------------------
// LUT2 = 2*E2M1 = {0,1,2,3,4,6,8,12} and their negatives: exact int8 values,
// so sdot4 against Q8_0 codes gives the exact block sum; the block scale of
// the integer form is 2^(e-128) (half the reference's 2^(e-127)).
constexpr uint32_t kPosLo = 0x03020100u, kPosHi = 0x0C080604u;
constexpr uint32_t kNegLo = 0xFDFEFF00u, kNegHi = 0xF4F8FAFCu;

struct MxDecoded {
    uint32_t lo[4];  // int8x4: elements 4k..4k+3
    uint32_t hi[4];  // int8x4: elements 16+4k..16+4k+3
    uint32_t e;      // E8M0 byte
};

// Eight nibbles of one dword -> two int8x4 words through v_perm_b32 lookups:
// magnitude from the positive and negative tables by (nibble & 7), then a
// byte select by the sign bit (bit 3 of the nibble).
__device__ inline void mx_lut(uint32_t w, uint32_t *lo, uint32_t *hi) {
    uint32_t il = w & 0x07070707u;
    uint32_t ih = (w >> 4) & 0x07070707u;
    uint32_t pl = __builtin_amdgcn_perm(kPosHi, kPosLo, il);
    uint32_t nl = __builtin_amdgcn_perm(kNegHi, kNegLo, il);
    uint32_t ph = __builtin_amdgcn_perm(kPosHi, kPosLo, ih);
    uint32_t nh = __builtin_amdgcn_perm(kNegHi, kNegLo, ih);
    uint32_t sl = ((w >> 1) & 0x04040404u) | 0x03020100u;
    uint32_t sh = ((w >> 5) & 0x04040404u) | 0x03020100u;
    *lo = __builtin_amdgcn_perm(nl, pl, sl);
    *hi = __builtin_amdgcn_perm(nh, ph, sh);
}

// d[0..4] from load_block5 at the block's first byte, o = its offset.
__device__ inline void mx_decode(const uint32_t d[5], uint32_t o, MxDecoded &m) {
    uint32_t sel = 0x04030201u + o * 0x01010101u;  // bytes o+1..o+4
    m.e = __builtin_amdgcn_ubfe(d[0], o * 8u, 8u);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t w = __builtin_amdgcn_perm(d[k + 1], d[k], sel);
        mx_lut(w, &m.lo[k], &m.hi[k]);
    }
}

// Exact int32 block sum of a decoded MXFP4 block against 8 code dwords.
__device__ inline int32_t mx_isum(const MxDecoded &m, const uint32_t q[8]) {
    int32_t s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        s = __builtin_amdgcn_sdot4((int)m.lo[k], (int)q[k], s, false);
        s = __builtin_amdgcn_sdot4((int)m.hi[k], (int)q[k + 4], s, false);
    }
    return s;
}

// d_x * 2^(e-128); e = 255 keeps the reference's +Inf block scale
// (forward/mxfp4.go:23: float32(math.Ldexp(1, 128)) = +Inf).
__device__ inline float mx_block_scale(float dx, uint32_t e) {
    return e == 255u ? dx * __builtin_inff() : __builtin_ldexpf(dx, (int)e - 128);
}

// ---- Q4_0 block decode ---------------------------------------------------------
struct Q40Decoded {
    uint32_t lo[4];  // nibbles 0..15 (unsigned) of elements 4k..4k+3
    uint32_t hi[4];  // nibbles of elements 16+4k..
    float d;         // fp16 scale widened
};

// o is 0 or 2 (Q4_0 rows are 2-byte aligned).
__device__ inline void q40_decode(const uint32_t d[5], uint32_t o, Q40Decoded &m) {
    uint32_t sel = 0x05040302u + o * 0x01010101u;  // bytes o+2..o+5
    m.d = f16_bits_to_f32(__builtin_amdgcn_ubfe(d[0], o * 8u, 16u));
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t w = __builtin_amdgcn_perm(d[k + 1], d[k], sel);
        m.lo[k] = w & 0x0F0F0F0Fu;
        m.hi[k] = (w >> 4) & 0x0F0F0F0Fu;
    }
}

// sum (n-8)*q = sum n*q - 8*sum q (n in 0..15 is a non-negative int8).
__device__ inline int32_t q40_isum(const Q40Decoded &m, const uint32_t q[8], int32_t sumq) {
    int32_t s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        s = __builtin_amdgcn_sdot4((int)m.lo[k], (int)q[k], s, false);
        s = __builtin_amdgcn_sdot4((int)m.hi[k], (int)q[k + 4], s, false);
    }
    return s - 8 * sumq;
}

// ---- Q8_0 quantization of one block of 32 ---------------------------------------
// GGML quantize_row_q8_0 reference rule: d = amax/127 (IEEE division),
// id = d ? 1/d : 0, q = roundf(x*id) half away from zero; a NaN element makes
// d NaN; a NaN product gives code 0; codes clamp to [-127, 127].
__device__ inline void q8_quantize32(const float v[32], uint32_t codes[8], uint16_t *dbits) {
    float amax = 0.0f;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        float a = __builtin_fabsf(v[i]);
        nan |= (a != a);
        amax = a > amax ? a : amax;
    }
    float d = nan ? __builtin_nanf("") : amax / 127.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    *dbits = f32_to_f16_bits(d);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float r = __builtin_roundf(v[4 * k + i] * id);
            int q = (r != r) ? 0 : (r > 127.0f ? 127 : (r < -127.0f ? -127 : (int)r));
            word |= (uint32_t)(q & 0xff) << (8 * i);
        }
        codes[k] = word;
    }
}

// ---- Q8_0 digit table for the block-scaled MFMA -------------------------------
// FP8 E4M3 encoding of a small integer, exact for |v| <= 15.
__device__ inline uint32_t e4m3_small(int v) {
    const uint32_t a = (uint32_t)(v < 0 ? -v : v);
    if (a == 0) return 0u;
    const uint32_t e = 31u - __builtin_clz(a);               // floor(log2 a), 0..3
    const uint32_t code = ((e + 7u) << 3) | ((a << (3u - e)) & 7u);
    return v < 0 ? (code | 0x80u) : code;
}

// Store one quantized block of 32 (codes w[8], fp16 scale bits dh) as block
// `blk` of every requested layout:
//   codes  : int8 [blk][32]
//   scales : f32  [blk]          (fp16 d widened exactly)
//   mxtab  : u8   [blk][64]      E4M3 digits of q = 16*h + l in MXFP4 nibble
//                                 order (position p <-> element (p>>1) +
//                                 16*(p&1)): h digits at [0,32), l at [32,64)
//   blocks34: u8  [blk][34]      GGML Q8_0 block
//   btab   : u32 [blk][16]       bf16 codes for the bf16 MFMA, dword j =
//                                 bf16(q[j]) | bf16(q[j+16]) << 16 (the
//                                 MXFP4 nibble order of bytes 1+j)
__device__ inline uint32_t bf16_code_pair(int lo, int hi) {
    return (__float_as_uint((float)lo) >> 16) | (__float_as_uint((float)hi) & 0xFFFF0000u);
}

__device__ inline void write_q8_block(const uint32_t w[8], uint16_t dh, size_t blk, int8_t *codes,
                                      float *scales, uint8_t *mxtab, uint8_t *blocks34,
                                      uint32_t *btab = nullptr) {
    if (codes) {
        uint32_t *c = reinterpret_cast<uint32_t *>(codes + blk * 32);
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = w[k];
    }
    if (scales) scales[blk] = f16_bits_to_f32(dh);
    if (mxtab) {
        uint32_t hw[8], lw[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            hw[k] = 0;
            lw[k] = 0;
        }
#pragma unroll
        for (int p = 0; p < 32; p++) {
            const int el = (p >> 1) + 16 * (p & 1);
            const int q = (int)(int8_t)(w[el >> 2] >> (8 * (el & 3)));
            const int h = q >> 4, l = q & 15;
            hw[p >> 2] |= e4m3_small(h) << (8 * (p & 3));
            lw[p >> 2] |= e4m3_small(l) << (8 * (p & 3));
        }
        uint32_t *o = reinterpret_cast<uint32_t *>(mxtab + blk * 64);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            o[k] = hw[k];
            o[8 + k] = lw[k];
        }
    }
    if (blocks34) {
        uint8_t *o = blocks34 + blk * kQ80Block;
        o[0] = (uint8_t)(dh & 0xff);
        o[1] = (uint8_t)(dh >> 8);
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) o[2 + 4 * k + i] = (uint8_t)(w[k] >> (8 * i));
    }
    if (btab) {
        uint32_t *o = btab + blk * 16;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int lo = (int)(int8_t)(w[j >> 2] >> (8 * (j & 3)));
            const int hi = (int)(int8_t)(w[4 + (j >> 2)] >> (8 * (j & 3)));
            o[j] = bf16_code_pair(lo, hi);
        }
    }
}

// The same rule with one element per lane (lanes 0..31 of a wavefront hold
// the block; lanes 32..63 pass v = 0 and their results are unused).  amax
// skips NaN elements exactly as the sequential form does, so codes and scale
// are identical to q8_quantize32.
__device__ inline int q8_quantize_lane(float v, int lane, uint16_t *dbits) {
    const float a = __builtin_fabsf(v);
    const bool in_block = lane < 32;
    const bool nan_any = __any(in_block && (a != a));
    float m = (in_block && a == a) ? a : 0.0f;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off, 32);
        m = o > m ? o : m;
    }
    const float d = nan_any ? __builtin_nanf("") : m / 127.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    *dbits = f32_to_f16_bits(d);
    const float r = __builtin_roundf(v * id);
    return (r != r) ? 0 : (r > 127.0f ? 127 : (r < -127.0f ? -127 : (int)r));
}

// Largest value over each half-wave (32 lanes) of non-negative non-NaN
// floats given as bit patterns (which order like the values): DPP lane ^ 15,
// ^ 7, ^ 1, ^ 2 within rows of 16, then a swizzle for lane ^ 16.
__device__ __attribute__((always_inline)) inline uint32_t max32_bits(uint32_t m) {
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x140, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));
    m = max(m, (uint32_t)__builtin_amdgcn_ds_swizzle((int)m, 0x401F));
    return m;
}

// Q8_0 of a 32-element block held one element per lane by each half-wave:
// the arithmetic of q8_quantize_lane (scale amax / 127, a NaN anywhere in
// the block makes the scale NaN), with the reductions done per half-wave.
__device__ __attribute__((always_inline)) inline int q8_quantize_half(float v, int lane, uint16_t *dbits) {
    const float a = __builtin_fabsf(v);
    const uint64_t nanm = __ballot(a != a);
    const bool nan_any = ((lane < 32 ? nanm : nanm >> 32) & 0xFFFFFFFFull) != 0;
    const float m = __uint_as_float(max32_bits(a == a ? __float_as_uint(a) : 0u));
    const float d = nan_any ? __builtin_nanf("") : m / 127.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    *dbits = f32_to_f16_bits(d);
    const float r = __builtin_roundf(v * id);
    return (r != r) ? 0 : (r > 127.0f ? 127 : (r < -127.0f ? -127 : (int)r));
}

// Lane i (< 32) of a wavefront stores element i of Q8_0 block `blk` (code q)
// into every requested layout of write_q8_block; lane 0 also stores the scale.
__device__ inline void write_q8_lane(int q, uint16_t dh, int lane, size_t blk, int8_t *codes,
                                     float *scales, uint8_t *mxtab, uint8_t *blocks34,
                                     uint32_t *btab = nullptr) {
    if (lane >= 32) return;
    if (btab)
        reinterpret_cast<uint16_t *>(btab + blk * 16)[2 * (lane & 15) + (lane >> 4)] =
            (uint16_t)(__float_as_uint((float)q) >> 16);
    if (codes) codes[blk * 32 + lane] = (int8_t)q;
    if (scales && lane == 0) scales[blk] = f16_bits_to_f32(dh);
    if (mxtab) {
        const int p = 2 * (lane & 15) + (lane >> 4);  // nibble position of element `lane`
        mxtab[blk * 64 + p] = (uint8_t)e4m3_small(q >> 4);
        mxtab[blk * 64 + 32 + p] = (uint8_t)e4m3_small(q & 15);
    }
    if (blocks34) {
        if (lane == 0) {
            blocks34[blk * kQ80Block] = (uint8_t)(dh & 0xff);
            blocks34[blk * kQ80Block + 1] = (uint8_t)(dh >> 8);
        }
        blocks34[blk * kQ80Block + 2 + lane] = (uint8_t)q;
    }
}

// ---- clamped SwiGLU (forward/moe.go:66-70) ------------------------------------
// Go's min/max return NaN when either operand is NaN; the comparisons below
// keep that (a NaN gate or up propagates).
// exp in double by Cody-Waite reduction (x = k*ln2 + r, ln2 split into the
// fdlibm hi/lo pair) and a degree-14 Taylor polynomial for |r| <= ln2/2
// (truncation < 1e-17), scaled by 2^k.  Relative error <= 2^-52 against
// libm exp; rounded to float it equals float(exp(x)) for every float input
// of the SwiGLU below (checked exhaustively for gate in [-60, 7]; beyond,
// both overflow to +Inf).  Far fewer registers than the library routine,
// which matters inside the streaming GEMV.
// A double constant written into registers where it is used: the volatile
// moves cannot be hoisted out of a loop, so a routine called once per
// several iterations does not hold its constants in registers across the
// whole loop (where a register-bound loop would spill them).  KREG picks the
// registers: kConstVgpr, two vector moves per use; kConstSgpr, two scalar
// moves per use (issued beside the vector instructions, and the double FMA
// takes the scalar pair as an operand).
enum KConst { kConstVgpr = 0, kConstSgpr = 1 };
template <int KREG, uint64_t BITS>
__device__ __attribute__((always_inline)) inline double kdouble() {
    uint32_t lo, hi;
    if constexpr (KREG == kConstSgpr)
        asm volatile("s_mov_b32 %0, %2\n\ts_mov_b32 %1, %3"
                     : "=s"(lo), "=s"(hi)
                     : "i"((uint32_t)(BITS & 0xFFFFFFFFu)), "i"((uint32_t)(BITS >> 32)));
    else
        asm volatile("v_mov_b32 %0, %2\n\tv_mov_b32 %1, %3"
                     : "=v"(lo), "=v"(hi)
                     : "i"((uint32_t)(BITS & 0xFFFFFFFFu)), "i"((uint32_t)(BITS >> 32)));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
#define SPT_KD(c) kdouble<KREG, __builtin_bit_cast(uint64_t, (double)(c))>()

template <int KREG = kConstVgpr>
__device__ inline double exp_f64(double x) {
    if (!(x <= 709.78)) return x != x ? x : __builtin_inf();
    if (x < -745.2) return 0.0;
    const double k = __builtin_rint(x * SPT_KD(1.4426950408889634));
    const double r = __builtin_fma(-k, SPT_KD(1.90821492927058770002e-10), __builtin_fma(-k, SPT_KD(6.93147180369123816490e-01), x));
    double p = SPT_KD(1.0 / 87178291200.0);  // 1/14!
    p = __builtin_fma(p, r, SPT_KD(1.0 / 6227020800.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 479001600.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 39916800.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 3628800.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 362880.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 40320.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 5040.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 720.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 120.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 24.0));
    p = __builtin_fma(p, r, SPT_KD(1.0 / 6.0));
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return __builtin_ldexp(p, (int)k);
}

template <int KREG = kConstVgpr>
__device__ inline float swiglu(float gate, float up) {
    float g = (gate > 7.0f) ? 7.0f : gate;
    float u = (up > 7.0f) ? 7.0f : up;
    u = (u < -7.0f) ? -7.0f : u;
    float e = static_cast<float>(exp_f64<KREG>(static_cast<double>(-1.702f * g)));
    return g / (1.0f + e) * (u + 1.0f);
}

}  // namespace spt
