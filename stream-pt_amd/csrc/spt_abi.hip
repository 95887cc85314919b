// spt_abi.hip -- C ABI of libspt_moe.so (include/spt_moe.h).
//
// Host side of the drop-in boundary: argument validation with the rules and
// messages of Stream-PT's forward package, a per-context device scratch
// arena, and the launch sequences of the operators.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "spt_kernels.h"
#include "spt_moe.h"

struct spt_ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    const volatile int32_t *cancel = nullptr;
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    void *pinned = nullptr;  // host staging of the *_host entry points
    size_t pinned_bytes = 0;
    void *noalloc = nullptr;          // this device's copy of `scratch` (below)
    hipError_t noalloc_err = hipSuccess;
    bool timing = false;
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
    std::vector<hipEvent_t> free_events;
    double total_ms[SPT_KERNEL_KINDS] = {};
    int64_t launches[SPT_KERNEL_KINDS] = {};
    int32_t gemm_min_group = 0;  // 0: the default policy (kGemmMinGroup)
    int32_t decode_max_selections = 0;  // 0: kDecodeMaxSelections; < 0: decode path off
    int n_cu = 0;                // compute units of the device
    // A second stream of the device and two events: a layer's grouped GEMM
    // launches run there beside its GEMV launches (fork after the
    // selection, join before the combine).  Null: everything on `stream`.
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

// Scratch of spt_forward_moe_batch_noalloc: a fixed device array, one copy
// per GPU the library runs on, held until the process ends.  Host code
// never passes this name to a kernel (on the host it is only a stand-in for
// the symbol): the context looks up the device address of the current
// device's copy once per device (noalloc_scratch_of) and uses that address.
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

// Device address of `scratch` on each device, looked up once per device
// with that device current.
constexpr int kMaxDevices = 64;
struct NoAllocSlot {
    std::once_flag once;
    void *ptr = nullptr;
    hipError_t err = hipSuccess;
};
NoAllocSlot g_noalloc[kMaxDevices];

void noalloc_scratch_of(int device, void **ptr, hipError_t *err) {
    if (device < 0 || device >= kMaxDevices) {
        *ptr = nullptr;
        *err = hipErrorInvalidDevice;
        return;
    }
    NoAllocSlot &slot = g_noalloc[device];
    std::call_once(slot.once, [&] {
        void *p = nullptr;
        slot.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        slot.ptr = slot.err == hipSuccess ? p : nullptr;
    });
    *ptr = slot.ptr;
    *err = slot.err;
}

// The calling thread's last error message (a fixed buffer: reporting an
// error allocates nothing).
thread_local char g_error[512];

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t err, const char *what) {
    return fail(SPT_ERR_DEVICE, "%s: %s", what, hipGetErrorString(err));
}

#define SPT_HIP(call)                                                   \
    do {                                                                \
        hipError_t err_ = (call);                                       \
        if (err_ != hipSuccess) return hip_fail(err_, #call);           \
    } while (0)

const char *tname(const spt_tensor *t) { return (t && t->name) ? t->name : ""; }
bool named(const spt_tensor &t) { return t.name && t.name[0]; }

// moeBatchProduct (forward/moe_batch.go:29-38): product of positive factors
// without overflowing int64.
bool product(int64_t *out, std::initializer_list<int64_t> values) {
    int64_t n = 1;
    for (int64_t v : values) {
        if (v <= 0 || n > INT64_MAX / v) return false;
        n *= v;
    }
    *out = n;
    return true;
}

bool ranges_overlap(const void *a, uint64_t an, const void *b, uint64_t bn) {
    uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return an && bn && x < y + bn && y < x + an;
}

int check_ctx(spt_ctx *ctx) {
    if (!ctx) return fail(SPT_ERR_INVALID, "nil context");
    return SPT_OK;
}

int check_device(spt_ctx *ctx) {
    if (ctx->device < 0) return fail(SPT_ERR_DEVICE, "validation-only context has no device");
    hipError_t err = hipSetDevice(ctx->device);
    if (err != hipSuccess) return hip_fail(err, "hipSetDevice");
    return SPT_OK;
}

int check_cancel(spt_ctx *ctx) {
    if (ctx->cancel && *ctx->cancel) return fail(SPT_ERR_CANCELED, "context canceled");
    return SPT_OK;
}

hipEvent_t take_event(spt_ctx *ctx) {
    if (!ctx->free_events.empty()) {
        hipEvent_t e = ctx->free_events.back();
        ctx->free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Runs `launch` (returning hipError_t); with timing on, brackets it with a
// pair of events on the context's stream.
template <class F>
hipError_t timed(spt_ctx *ctx, int kind, F &&launch) {
    if (!ctx->timing) return launch();
    hipEvent_t a = take_event(ctx), b = take_event(ctx);
    if (!a || !b) return hipErrorOutOfMemory;
    hipError_t err = hipEventRecord(a, ctx->stream);
    if (err == hipSuccess) err = launch();
    if (err == hipSuccess) err = hipEventRecord(b, ctx->stream);
    if (err != hipSuccess) return err;
    ctx->pending.push_back({kind, {a, b}});
    return hipSuccess;
}

// Grow-only device scratch arena; returns a pointer to at least `bytes` bytes.
int arena(spt_ctx *ctx, size_t bytes, char **out) {
    if (bytes > ctx->scratch_bytes) {
        if (ctx->scratch) {
            hipError_t e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
            (void)hipFree(ctx->scratch);
            ctx->scratch = nullptr;
            ctx->scratch_bytes = 0;
        }
        size_t want = bytes + bytes / 4 + 4096;
        if (hipMalloc(&ctx->scratch, want) != hipSuccess) {
            ctx->scratch = nullptr;
            return fail(SPT_ERR_NOMEM, "cannot allocate %zu bytes of device scratch", want);
        }
        ctx->scratch_bytes = want;
    }
    *out = static_cast<char *>(ctx->scratch);
    return SPT_OK;
}

// Bump allocator over the scratch arena, 256-byte aligned slices.
struct Carve {
    size_t off = 0;
    size_t take(size_t n) {
        size_t o = off;
        off += (n + 255) & ~size_t(255);
        return o;
    }
};

// q40Shape (forward/q40.go:105-130).
int q40_shape(const spt_tensor *t, int64_t *in, int64_t *out, int64_t *row_bytes) {
    if (t->type != SPT_TYPE_Q4_0)
        return fail(SPT_ERR_INVALID, "\"%s\": GGML type %u instead of Q4_0 (2)", tname(t), t->type);
    if (t->n_dims != 2) return fail(SPT_ERR_INVALID, "\"%s\": expected a two-dimensional matrix", tname(t));
    uint64_t i = t->shape[0], o = t->shape[1];
    if (i == 0 || o == 0 || i % 32 != 0)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid Q4_0 matrix shape [%llu %llu]", tname(t),
                    (unsigned long long)i, (unsigned long long)o);
    if (i > (uint64_t)INT64_MAX || o > (uint64_t)INT64_MAX || i / 32 > (uint64_t)INT64_MAX / 18)
        return fail(SPT_ERR_INVALID, "\"%s\": matrix dimensions exceed platform limits", tname(t));
    uint64_t bytes = i / 32 * 18;
    if (o > UINT64_MAX / bytes || t->nbytes == 0 || t->nbytes != o * bytes)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid tensor byte range for shape [%llu %llu]", tname(t),
                    (unsigned long long)i, (unsigned long long)o);
    if (!t->data) return fail(SPT_ERR_INVALID, "\"%s\": tensor is not resident (nil data)", tname(t));
    if ((uintptr_t)t->data & 1)
        return fail(SPT_ERR_INVALID, "\"%s\": Q4_0 data must be 2-byte aligned", tname(t));
    if (t->nbytes > 0xFFFFFFFCull)
        return fail(SPT_ERR_INVALID, "\"%s\": tensor larger than 4 GiB is not supported", tname(t));
    *in = (int64_t)i;
    *out = (int64_t)o;
    *row_bytes = (int64_t)bytes;
    return SPT_OK;
}

// q80Shape (forward/q80.go:150-171), plus this library's limits: the
// input fits the kernel's x staging (kQ80MaxBlocks blocks), the rows are
// 2-byte aligned and the matrix below 4 GiB.
int q80_shape(const spt_tensor *t, int64_t *in, int64_t *out) {
    if (t->type != SPT_TYPE_Q8_0)
        return fail(SPT_ERR_INVALID, "\"%s\": GGML type %u instead of Q8_0 (8)", tname(t), t->type);
    if (t->n_dims != 2) return fail(SPT_ERR_INVALID, "\"%s\": expected 2D matrix", tname(t));
    uint64_t i = t->shape[0], o = t->shape[1];
    if (i == 0 || o == 0 || i % 32 != 0)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid Q8_0 shape [%llu %llu]", tname(t), (unsigned long long)i,
                    (unsigned long long)o);
    if (i > (uint64_t)INT64_MAX || o > (uint64_t)INT64_MAX || i / 32 > (uint64_t)INT64_MAX / 34)
        return fail(SPT_ERR_INVALID, "\"%s\": matrix dimensions exceed platform limits", tname(t));
    uint64_t bytes = i / 32 * 34;
    if (o > UINT64_MAX / bytes || t->nbytes == 0 || t->nbytes != o * bytes)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid byte range", tname(t));
    if (!t->data) return fail(SPT_ERR_INVALID, "\"%s\": tensor is not resident (nil data)", tname(t));
    if (i > (uint64_t)spt::kQ80MaxBlocks * 32)
        return fail(SPT_ERR_INVALID, "\"%s\": Q8_0 input dimension %llu exceeds the supported %d", tname(t),
                    (unsigned long long)i, spt::kQ80MaxBlocks * 32);
    if ((uintptr_t)t->data & 1)
        return fail(SPT_ERR_INVALID, "\"%s\": Q8_0 data must be 2-byte aligned", tname(t));
    if (t->nbytes > 0xFFFFFF00ull || o > (uint64_t)INT_MAX)
        return fail(SPT_ERR_INVALID, "\"%s\": tensor larger than 4 GiB is not supported", tname(t));
    *in = (int64_t)i;
    *out = (int64_t)o;
    return SPT_OK;
}

// The normalization weight of RMSNormInto (forward/rmsnorm.go:42-58) and
// normBatch (forward/layer_batch.go:145-155): F32 (0), F16 (1) or BF16 (28),
// one element per input; *wtype is the kernel's encoding (0, 1, 2).
int norm_weight_check(const spt_tensor *w, int64_t dim, bool batch_form, int *wtype) {
    uint64_t width;
    switch (w->type) {
        case SPT_TYPE_F32: width = 4; *wtype = 0; break;
        case SPT_TYPE_F16: width = 2; *wtype = 1; break;
        case 28: width = 2; *wtype = 2; break;
        default:
            return fail(SPT_ERR_INVALID, "\"%s\": unsupported normalization weight type %u", tname(w), w->type);
    }
    if (batch_form) {
        if (w->n_dims != 1 || w->shape[0] != (uint64_t)dim || w->nbytes != width * (uint64_t)dim)
            return fail(SPT_ERR_INVALID, "\"%s\": invalid float vector shape or range", tname(w));
    } else {
        if ((uint64_t)dim > (uint64_t)INT64_MAX / width)
            return fail(SPT_ERR_INVALID, "\"%s\": normalization weight exceeds platform limits", tname(w));
        if (w->nbytes == 0 || w->nbytes != (uint64_t)dim * width)
            return fail(SPT_ERR_INVALID, "\"%s\": invalid weight data length", tname(w));
    }
    if (!w->data) return fail(SPT_ERR_INVALID, "\"%s\": tensor is not resident (nil data)", tname(w));
    if ((uintptr_t)w->data & (width - 1))
        return fail(SPT_ERR_INVALID, "\"%s\": weight data must be %llu-byte aligned", tname(w),
                    (unsigned long long)width);
    return SPT_OK;
}

bool bad_epsilon(float e) { return e < 0.0f || e != e || e == __builtin_inff(); }

// The Q8_0 output of the fused normalization: whole blocks, apart from x and y.
int norm_q8_check(const void *q8, int64_t total, const float *x, const float *y) {
    if (!q8) return SPT_OK;
    if (total % 32 != 0)
        return fail(SPT_ERR_INVALID, "Q8_0 output needs a dimension that is a multiple of 32, got %lld",
                    (long long)total);
    const uint64_t qb = (uint64_t)total / 32 * 34;
    if (ranges_overlap(q8, qb, x, (uint64_t)total * 4) || (y && ranges_overlap(q8, qb, y, (uint64_t)total * 4)))
        return fail(SPT_ERR_INVALID, "Q8_0 output overlaps the input or output");
    return SPT_OK;
}

// validateMoEBatchExpert (forward/mxfp4_batch.go:17-27).
int validate_expert(const spt_tensor *t, int64_t input, int64_t output, int64_t experts) {
    if (t->type != SPT_TYPE_MXFP4 || t->n_dims != 3 || t->shape[0] != (uint64_t)input ||
        t->shape[1] != (uint64_t)output || t->shape[2] != (uint64_t)experts || input % 32 != 0)
        return fail(SPT_ERR_INVALID, "\"%s\": expected MXFP4 expert tensor [%lld %lld %lld]", tname(t),
                    (long long)input, (long long)output, (long long)experts);
    int64_t n;
    if (!product(&n, {input / 32, 17, output, experts}) || t->nbytes != (uint64_t)n)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid expert range or overflow", tname(t));
    if (!t->data) return fail(SPT_ERR_INVALID, "\"%s\": tensor is not resident (nil data)", tname(t));
    if ((uint64_t)(input / 32 * 17) * (uint64_t)output > 0xFFFFFFF0ull)
        return fail(SPT_ERR_INVALID, "\"%s\": expert matrix larger than 4 GiB is not supported", tname(t));
    return SPT_OK;
}

// The grouped GEMV stages whole weight rows in LDS (no counterpart in the
// reference, whose CPU loops take any width).
int validate_gemv_input(const spt_tensor *t, int64_t input) {
    if (input > spt::kMxMaxInput)
        return fail(SPT_ERR_INVALID, "\"%s\": MXFP4 input dimension %lld exceeds the supported %d", tname(t),
                    (long long)input, spt::kMxMaxInput);
    return SPT_OK;
}

// validateMoEBatchBias (forward/moe_batch.go:196-219).
int validate_bias(const spt_tensor *t, int64_t dim, int64_t count) {
    if (!named(*t)) {
        if (t->nbytes != 0) return fail(SPT_ERR_INVALID, "unnamed MoE bias has nonempty range");
        return SPT_OK;
    }
    int64_t width = 4;
    if (t->type == SPT_TYPE_F16 || t->type == SPT_TYPE_BF16)
        width = 2;
    else if (t->type != SPT_TYPE_F32)
        return fail(SPT_ERR_INVALID, "\"%s\": unsupported bias type", tname(t));
    int64_t n;
    bool ok = product(&n, {dim, count, width});
    uint32_t want_dims = (count == 1 && t->n_dims == 1) ? 1 : 2;
    if (!ok || t->n_dims != want_dims || t->shape[0] != (uint64_t)dim ||
        (want_dims == 2 && t->shape[1] != (uint64_t)count) || t->nbytes != (uint64_t)n)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid bias shape or range", tname(t));
    if (!t->data) return fail(SPT_ERR_INVALID, "\"%s\": tensor is not resident (nil data)", tname(t));
    return SPT_OK;
}

const void *bias_ptr(const spt_tensor &t) { return named(t) ? t.data : nullptr; }
int bias_type(const spt_tensor &t) { return named(t) ? (int)t.type : 0; }
uint64_t bias_bytes(const spt_tensor &t) { return named(t) ? t.nbytes : 0; }

struct MoEDims {
    int64_t h, d, E, k, batch;
};

// forwardMoEBatch validation (forward/moe_batch.go:81-130).  With `sliced`
// the batch may hold more selections than one launch sequence takes
// (spt::kMaxSelections): the caller runs it as slices of whole tokens.
int validate_moe(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                 const float *x, int64_t x_len, const float *out, int64_t out_len, int64_t batch,
                 MoEDims *dims, bool sliced = false) {
    if (!ctx || !cfg || !lw) return fail(SPT_ERR_INVALID, "nil MoE context, reader, configuration or weights");
    int64_t h = cfg->hidden_dim, d = cfg->expert_hidden_dim, E = cfg->num_experts, k = cfg->num_experts_used;
    int64_t n;
    if (!product(&n, {batch, h, 4}) || x_len != n / 4 || out_len != n / 4 || k <= 0 || k > E || d <= 0)
        return fail(SPT_ERR_INVALID, "invalid MoE batch dimensions");
    if (!x || !out) return fail(SPT_ERR_INVALID, "invalid MoE batch dimensions");
    if (ranges_overlap(x, (uint64_t)n, out, (uint64_t)n)) return fail(SPT_ERR_INVALID, "MoE input and output overlap");
    const spt_tensor &router = lw->ffn_gate_inp;
    int64_t rb;
    if (!product(&rb, {h, E, 4}) || router.type != SPT_TYPE_F32 || router.n_dims != 2 ||
        router.shape[0] != (uint64_t)h || router.shape[1] != (uint64_t)E || router.nbytes != (uint64_t)rb)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid F32 router shape or range", tname(&router));
    if (!router.data) return fail(SPT_ERR_INVALID, "\"%s\": tensor is not resident (nil data)", tname(&router));
    if ((uintptr_t)router.data & 3u)
        return fail(SPT_ERR_INVALID, "\"%s\": router data must be 4-byte aligned", tname(&router));
    int rc;
    if ((rc = validate_expert(&lw->ffn_gate_exps, h, d, E))) return rc;
    if ((rc = validate_expert(&lw->ffn_up_exps, h, d, E))) return rc;
    if ((rc = validate_expert(&lw->ffn_down_exps, d, h, E))) return rc;
    if ((rc = validate_gemv_input(&lw->ffn_gate_exps, h))) return rc;
    if ((rc = validate_gemv_input(&lw->ffn_down_exps, d))) return rc;
    if ((rc = validate_bias(&lw->ffn_gate_inp_bias, E, 1))) return rc;
    if ((rc = validate_bias(&lw->ffn_gate_exps_bias, d, E))) return rc;
    if ((rc = validate_bias(&lw->ffn_up_exps_bias, d, E))) return rc;
    if ((rc = validate_bias(&lw->ffn_down_exps_bias, h, E))) return rc;
    // readFloatVector (forward/layer.go:279-287) reads the router bias as a vector.
    if (named(lw->ffn_gate_inp_bias) && lw->ffn_gate_inp_bias.n_dims != 1)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid float vector shape or range", tname(&lw->ffn_gate_inp_bias));
    if (h % 32 != 0) return fail(SPT_ERR_INVALID, "hidden dimension %lld is not a multiple of 32", (long long)h);
    if (k > spt::kMaxTopK || E > spt::kMaxExperts || (!sliced && batch * k > spt::kMaxSelections))
        return fail(SPT_ERR_INVALID,
                    "MoE shape beyond this device path's limits (experts used <= %d, experts <= %d, "
                    "batch*experts used <= %d per call with taps or without allocation)",
                    spt::kMaxTopK, spt::kMaxExperts, spt::kMaxSelections);
    *dims = MoEDims{h, d, E, k, batch};
    return SPT_OK;
}

int copy_tap(spt_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!dst || bytes == 0) return SPT_OK;
    SPT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return SPT_OK;
}

// Default policy for the grouped GEMM (measured on MI355X with GPT-OSS
// shapes): groups of at least kGemmMinGroup selections (three or more GEMV
// passes over the expert's weights) go to the GEMM when the batch holds at
// least kGemmMinSelections selections and their work items fill at least
// half the device; below that the GEMV's passes are faster (a GEMM item
// walks the whole input dimension serially, and the persistent GEMV holds
// every CU until it ends, so a few GEMM items run after it as a tail).
// Measured per layer, Zipf(1.1) routing, default against GEMV only: 96
// tokens 299 / 322 us, 128: 338 / 373, 160: 379 / 483, 192: 392 / 545;
// uniform routing at 96 and 128 tokens (one or two groups of 9 or 10) stays
// on the GEMV (328, 400 us; 386, 457 with those groups on the GEMM).
constexpr int kGemmMinGroup = 9;
constexpr int kGemmMinSelections = 384;
// Batches of up to this many selections (topk <= 4, no GEMM group) take the
// decode path: top-k inside the gate/up launch, combine inside the down
// launch, a workgroup per selection (spt_mx_decode.hip).  Measured on the
// 36-layer step at GPT-OSS-120B shape (top-4, HIP graph replay, decode path
// against the grouped GEMV): 1 token 0.925 / 1.317 ms, 2 tokens 1.403 /
// 1.619, 3 tokens 2.000 / 1.975, 4 tokens 2.245 / 2.179, 6 tokens 3.220 /
// 2.771.
constexpr int kDecodeMaxSelections = 8;

// Scratch layout of one forwardMoEBatch call (offsets into the arena).
struct MoELayout {
    bool use_gemm;
    bool decode;  // the two-launch decode path (spt_mx_decode.hip)
    int gemm_min;
    bool forced;
    size_t o_xc, o_xs, o_xm, o_xb, o_logits, o_ids, o_w, o_cnt, o_off, o_list, o_act_list, o_na;
    size_t o_gv, o_gvn, o_gvp, o_gvs, o_gm, o_gmn, o_gmt, o_act, o_ac, o_as, o_am, o_ab, o_res;
    size_t total;
};

// An expert's group holds at most n selections: with fewer than the
// threshold no expert can reach the GEMM, which is then not launched.  An
// explicit threshold (spt_ctx_set_gemm_min_group) applies as given; the
// default also needs kGemmMinSelections and half a device of items.  The
// fp32 act buffer exists only for the act tap.
MoELayout moe_layout(const spt_ctx *ctx, const MoEDims &m, bool act_tap, size_t base) {
    const int64_t h = m.h, d = m.d, E = m.E, B = m.batch, n = m.batch * m.k;
    const int64_t nbh = h / 32, nbd = d / 32;
    MoELayout L{};
    L.forced = ctx->gemm_min_group > 0;
    L.gemm_min = L.forced ? ctx->gemm_min_group : kGemmMinGroup;
    L.use_gemm = n >= L.gemm_min && (L.forced || n >= kGemmMinSelections);
    const int dec_max = ctx->decode_max_selections == 0 ? kDecodeMaxSelections : ctx->decode_max_selections;
    L.decode = !L.use_gemm && m.k <= spt::kDecMaxTopK && n <= dec_max;
    Carve c;
    c.off = base;
    L.o_xc = c.take(B * h), L.o_xs = c.take(B * nbh * 4), L.o_xm = c.take(B * nbh * 64);
    L.o_xb = c.take(L.use_gemm ? B * nbh * 64 : 0);
    L.o_logits = c.take(B * E * 4);
    L.o_ids = c.take(n * 4), L.o_w = c.take(n * 4), L.o_cnt = c.take(E * 4), L.o_off = c.take((E + 1) * 4);
    L.o_list = c.take(n * 4), L.o_act_list = c.take(E * 4), L.o_na = c.take(4);
    L.o_gv = c.take(E * 4), L.o_gvn = c.take(4), L.o_gvp = c.take((E + 1) * 4);
    L.o_gvs = c.take(L.decode ? 0 : sizeof(int32_t) * 2 * spt::kGvStartMax * spt::kGvStartWords);
    L.o_gm = c.take(E * 4), L.o_gmn = c.take(12), L.o_gmt = c.take((E + 1) * 4);  // gm_n, then the two claim counters
    L.o_act = c.take(act_tap ? n * d * 4 : 0), L.o_ac = c.take(n * d), L.o_as = c.take(n * nbd * 4);
    L.o_am = c.take(n * nbd * 64);
    L.o_ab = c.take(L.use_gemm ? n * nbd * 64 : 0);
    L.o_res = c.take(L.decode ? 0 : n * h * 4);  // the decode path combines in its down launch
    L.total = c.off;
    return L;
}

// The launch sequence of forwardMoEBatch over a scratch arena S laid out by L
// (S holds at least L.total bytes).
int run_moe_at(spt_ctx *ctx, const spt_moe_layer *lw, const float *x, float *out, const MoEDims &m,
               const spt_moe_taps *taps, char *S, const MoELayout &L, const uint8_t *xq34 = nullptr) {
    const int64_t h = m.h, d = m.d, E = m.E, k = m.k, B = m.batch, n = B * k;
    const int64_t nbh = h / 32, nbd = d / 32;
    const bool use_gemm = L.use_gemm, forced = L.forced;
    const int gemm_min = L.gemm_min;
    int rc;
    int8_t *xc = (int8_t *)(S + L.o_xc), *ac = (int8_t *)(S + L.o_ac);
    float *xs = (float *)(S + L.o_xs), *logits = (float *)(S + L.o_logits);
    float *act = taps && taps->act ? (float *)(S + L.o_act) : nullptr;
    uint8_t *xm = (uint8_t *)(S + L.o_xm), *am = (uint8_t *)(S + L.o_am);
    uint32_t *xb = use_gemm ? (uint32_t *)(S + L.o_xb) : nullptr, *ab = use_gemm ? (uint32_t *)(S + L.o_ab) : nullptr;
    float *as = (float *)(S + L.o_as), *res = (float *)(S + L.o_res);
    spt::SelectOut so{};
    so.ids = (int32_t *)(S + L.o_ids);
    so.weights = (float *)(S + L.o_w);
    so.counts = (int32_t *)(S + L.o_cnt);
    so.offsets = (int32_t *)(S + L.o_off);
    so.list = (int32_t *)(S + L.o_list);
    so.active = (int32_t *)(S + L.o_act_list);
    so.n_active = (int32_t *)(S + L.o_na);
    so.gemm_min = use_gemm ? gemm_min : INT_MAX;
    so.gemm_units = (int32_t)((d + 127) / 128);
    so.gemm_min_items = forced ? 0 : ctx->n_cu / 2;
    so.gv_active = (int32_t *)(S + L.o_gv);
    so.gv_n = (int32_t *)(S + L.o_gvn);
    so.gv_pass_off = (int32_t *)(S + L.o_gvp);
    so.gm_active = (int32_t *)(S + L.o_gm);
    so.gm_n = (int32_t *)(S + L.o_gmn);
    so.gm_claim = (int32_t *)(S + L.o_gmn) + 1;
    so.gm_tile_off = (int32_t *)(S + L.o_gmt);
    // the two grouped GEMV launches' start table, for their grids
    const int slots = (int)(n < E ? n : E);
    if (!L.decode) {
        spt::MxMfmaArgs g{};
        g.rows = (int)d;
        so.gv_grid[0] = spt::mx_mfma_grid(spt::kGateUp, g, slots);
        g.rows = (int)h;
        so.gv_grid[1] = spt::mx_mfma_grid(spt::kDown, g, slots);
        so.gv_tiles[0] = (int32_t)((d + 31) / 32);
        so.gv_tiles[1] = (int32_t)((h + 63) / 64);
        if (so.gv_grid[0] <= spt::kGvStartMax && so.gv_grid[1] <= spt::kGvStartMax)
            so.gv_start = (int32_t *)(S + L.o_gvs);
    }
    hipStream_t s = ctx->stream;

    // the Q8_0 of x: quantized by the router's launch, or unpacked there from
    // the caller's GGML blocks (the fused RMSNorm's output)
    const spt::QuantOut xq{xc, xs, xm, taps ? (uint8_t *)taps->xq : nullptr, xb, xq34};
    if ((rc = check_cancel(ctx))) return rc;
    if (taps && taps->logits_in) {
        SPT_HIP(timed(ctx, SPT_KERNEL_QUANTIZE, [&] {
            return spt::launch_quantize(s, x, B * nbh, xq.codes, xq.scales, nullptr, xq.mxtab, xq.blocks34, xq.btab);
        }));
        if (!L.decode)
            SPT_HIP(timed(ctx, SPT_KERNEL_SELECT, [&] { return spt::launch_select(s, taps->logits_in, (int)B, (int)E, (int)k, so); }));
        if ((rc = copy_tap(ctx, taps->logits, taps->logits_in, B * E * 4))) return rc;
    } else {
        // router logits + Q8_0 of x in one launch, then top-k + lists
        SPT_HIP(timed(ctx, SPT_KERNEL_ROUTE, [&] {
            return spt::launch_route(s, (const float *)lw->ffn_gate_inp.data, bias_ptr(lw->ffn_gate_inp_bias),
                                     bias_type(lw->ffn_gate_inp_bias), x, (int)B, (int)h, (int)E, logits, xq);
        }));
        if ((rc = check_cancel(ctx))) return rc;
        if (!L.decode)
            SPT_HIP(timed(ctx, SPT_KERNEL_SELECT, [&] { return spt::launch_select(s, logits, (int)B, (int)E, (int)k, so); }));
        if (taps && (rc = copy_tap(ctx, taps->logits, logits, B * E * 4))) return rc;
    }
    if (L.decode) {
        // gate/up with the top-k of each workgroup's token inside, then down
        // with the combine inside
        spt::DecGateUpArgs gu{};
        gu.g.w[0] = (const uint8_t *)lw->ffn_gate_exps.data;
        gu.g.w[1] = (const uint8_t *)lw->ffn_up_exps.data;
        gu.g.expert_bytes = (uint64_t)nbh * 17 * d;
        gu.g.rows = (int)d;
        gu.g.nb = (int)nbh;
        gu.g.bias[0] = bias_ptr(lw->ffn_gate_exps_bias);
        gu.g.bias_type[0] = bias_type(lw->ffn_gate_exps_bias);
        gu.g.bias_bytes[0] = bias_bytes(lw->ffn_gate_exps_bias);
        gu.g.bias[1] = bias_ptr(lw->ffn_up_exps_bias);
        gu.g.bias_type[1] = bias_type(lw->ffn_up_exps_bias);
        gu.g.bias_bytes[1] = bias_bytes(lw->ffn_up_exps_bias);
        gu.g.mxtab = xm;
        gu.g.scales = xs;
        gu.g.codes = xc;
        gu.g.topk = (int)k;
        gu.g.out = act;
        gu.g.tap[0] = taps ? taps->gate : nullptr;
        gu.g.tap[1] = taps ? taps->up : nullptr;
        gu.g.act_codes = ac;
        gu.g.act_scales = as;
        gu.g.act_mxtab = am;
        gu.g.act_blocks34 = taps ? (uint8_t *)taps->actq : nullptr;
        gu.logits = taps && taps->logits_in ? taps->logits_in : logits;
        gu.experts = (int)E;
        gu.tab_rows = (int)B;
        gu.ids = so.ids;
        gu.weights = so.weights;
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_GATE_UP, [&] { return spt::launch_dec_gate_up(s, gu, (int)n); }));
        const bool lists = taps && (taps->counts || taps->offsets || taps->list || taps->active || taps->n_active);
        if (lists) SPT_HIP(timed(ctx, SPT_KERNEL_SELECT, [&] { return spt::launch_pack(s, (int)B, (int)E, (int)k, so); }));
        spt::DecDownArgs dn{};
        dn.g.w[0] = (const uint8_t *)lw->ffn_down_exps.data;
        dn.g.expert_bytes = (uint64_t)nbd * 17 * h;
        dn.g.rows = (int)h;
        dn.g.nb = (int)nbd;
        dn.g.bias[0] = bias_ptr(lw->ffn_down_exps_bias);
        dn.g.bias_type[0] = bias_type(lw->ffn_down_exps_bias);
        dn.g.bias_bytes[0] = bias_bytes(lw->ffn_down_exps_bias);
        dn.g.mxtab = am;
        dn.g.scales = as;
        dn.g.codes = ac;
        dn.g.topk = (int)k;
        dn.tab_rows = (int)n;
        dn.ids = so.ids;
        dn.weights = so.weights;
        dn.out = out;
        dn.results = taps ? taps->results : nullptr;
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_DOWN, [&] { return spt::launch_dec_down(s, dn, (int)B); }));
        if (taps) {
            if ((rc = copy_tap(ctx, taps->ids, so.ids, n * 4))) return rc;
            if ((rc = copy_tap(ctx, taps->weights, so.weights, n * 4))) return rc;
            if (lists) {
                if ((rc = copy_tap(ctx, taps->counts, so.counts, E * 4))) return rc;
                if ((rc = copy_tap(ctx, taps->offsets, so.offsets, (E + 1) * 4))) return rc;
                if ((rc = copy_tap(ctx, taps->list, so.list, n * 4))) return rc;
                if ((rc = copy_tap(ctx, taps->active, so.active, E * 4))) return rc;
                if ((rc = copy_tap(ctx, taps->n_active, so.n_active, 4))) return rc;
            }
            if ((rc = copy_tap(ctx, taps->act, act, n * d * 4))) return rc;
        }
        return SPT_OK;
    }
    spt::MxMfmaArgs ga{};
    ga.w[0] = (const uint8_t *)lw->ffn_gate_exps.data;
    ga.w[1] = (const uint8_t *)lw->ffn_up_exps.data;
    ga.expert_bytes = (uint64_t)nbh * 17 * d;
    ga.rows = (int)d;
    ga.nb = (int)nbh;
    ga.bias[0] = bias_ptr(lw->ffn_gate_exps_bias);
    ga.bias_type[0] = bias_type(lw->ffn_gate_exps_bias);
    ga.bias_bytes[0] = bias_bytes(lw->ffn_gate_exps_bias);
    ga.bias[1] = bias_ptr(lw->ffn_up_exps_bias);
    ga.bias_type[1] = bias_type(lw->ffn_up_exps_bias);
    ga.bias_bytes[1] = bias_bytes(lw->ffn_up_exps_bias);
    ga.mxtab = xm;
    ga.scales = xs;
    ga.codes = xc;
    ga.active = so.gv_active;
    ga.n_active = so.gv_n;
    ga.pass_off = so.gv_pass_off;
    ga.offsets = so.offsets;
    ga.list = so.list;
    ga.topk = (int)k;
    ga.out = act;  // fp32 act only for the tap
    ga.tap[0] = taps ? taps->gate : nullptr;
    ga.tap[1] = taps ? taps->up : nullptr;
    ga.act_codes = ac;
    ga.act_scales = as;
    ga.act_mxtab = am;
    ga.act_blocks34 = taps ? (uint8_t *)taps->actq : nullptr;
    ga.start = so.gv_start;
    if ((rc = check_cancel(ctx))) return rc;
    // The grouped GEMM (its own experts, act rows and results) on the side
    // stream from here to the combine, so its launches fill the CUs the
    // GEMV launches leave idle and the reverse; with timing on, in line.
    // The join is recorded however the call ends.
    struct Join {
        spt_ctx *ctx;
        hipStream_t s;
        bool on = false;
        ~Join() {
            if (on && hipEventRecord(ctx->ev_join, ctx->side) == hipSuccess)
                (void)hipStreamWaitEvent(s, ctx->ev_join, 0);
        }
    } join{ctx, s};
    hipStream_t sg = s;
    if (use_gemm && ctx->side && !ctx->timing) {
        SPT_HIP(hipEventRecord(ctx->ev_fork, s));
        SPT_HIP(hipStreamWaitEvent(ctx->side, ctx->ev_fork, 0));
        sg = ctx->side;
        join.on = true;
    }
    SPT_HIP(timed(ctx, SPT_KERNEL_GATE_UP, [&] { return spt::launch_mx_mfma(s, spt::kGateUp, ga, slots); }));
    // Upper bound of the GEMM work items (token tiles x row units): every
    // GEMM expert holds at least gemm_min selections.
    const int64_t gm_experts = use_gemm ? std::min<int64_t>(E, n / gemm_min) : 0;
    const int64_t gm_tiles = gm_experts + (n + spt::kGemmTokens - 1) / spt::kGemmTokens;
    spt::MxGemmArgs gg{};
    if (use_gemm) {
        gg.w[0] = ga.w[0];
        gg.w[1] = ga.w[1];
        gg.expert_bytes = ga.expert_bytes;
        gg.rows = ga.rows;
        gg.nb = ga.nb;
        gg.bias[0] = ga.bias[0];
        gg.bias[1] = ga.bias[1];
        gg.bias_type[0] = ga.bias_type[0];
        gg.bias_type[1] = ga.bias_type[1];
        gg.btab = xb;
        gg.tab_rows = B;
        gg.scales = xs;
        gg.codes = xc;
        gg.gm_active = so.gm_active;
        gg.gm_n = so.gm_n;
        gg.claim = so.gm_claim;
        gg.gm_tile_off = so.gm_tile_off;
        gg.offsets = so.offsets;
        gg.list = so.list;
        gg.topk = (int)k;
        gg.out = ga.out;
        gg.tap[0] = ga.tap[0];
        gg.tap[1] = ga.tap[1];
        gg.act_codes = ac;
        gg.act_scales = as;
        gg.act_mxtab = nullptr;  // read only by the GEMV's down pass
        gg.act_blocks34 = ga.act_blocks34;
        gg.act_btab = ab;
        const int64_t items = gm_tiles * ((d + 127) / 128);
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_GATE_UP_GEMM, [&] {
            return spt::launch_mx_gemm(sg, spt::kGateUp, gg, (int)std::min<int64_t>(items, INT_MAX));
        }));
    }
    spt::MxMfmaArgs da{};
    da.w[0] = (const uint8_t *)lw->ffn_down_exps.data;
    da.expert_bytes = (uint64_t)nbd * 17 * h;
    da.rows = (int)h;
    da.nb = (int)nbd;
    da.bias[0] = bias_ptr(lw->ffn_down_exps_bias);
    da.bias_type[0] = bias_type(lw->ffn_down_exps_bias);
    da.bias_bytes[0] = bias_bytes(lw->ffn_down_exps_bias);
    da.mxtab = am;
    da.scales = as;
    da.codes = ac;
    da.active = so.gv_active;
    da.n_active = so.gv_n;
    da.pass_off = so.gv_pass_off;
    da.offsets = so.offsets;
    da.list = so.list;
    da.topk = (int)k;
    da.out = res;
    da.start = so.gv_start ? so.gv_start + spt::kGvStartMax * spt::kGvStartWords : nullptr;
    if ((rc = check_cancel(ctx))) return rc;
    SPT_HIP(timed(ctx, SPT_KERNEL_DOWN, [&] { return spt::launch_mx_mfma(s, spt::kDown, da, slots); }));
    if (use_gemm) {
        spt::MxGemmArgs gd{};
        gd.w[0] = da.w[0];
        gd.expert_bytes = da.expert_bytes;
        gd.rows = da.rows;
        gd.nb = da.nb;
        gd.bias[0] = da.bias[0];
        gd.bias_type[0] = da.bias_type[0];
        gd.btab = ab;
        gd.tab_rows = n;
        gd.scales = as;
        gd.codes = ac;
        gd.gm_active = so.gm_active;
        gd.gm_n = so.gm_n;
        gd.claim = so.gm_claim + 1;
        gd.gm_tile_off = so.gm_tile_off;
        gd.offsets = so.offsets;
        gd.list = so.list;
        gd.topk = (int)k;
        gd.out = res;
        const int64_t items = gm_tiles * ((h + 255) / 256);
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_DOWN_GEMM, [&] {
            return spt::launch_mx_gemm(sg, spt::kDown, gd, (int)std::min<int64_t>(items, INT_MAX));
        }));
    }
    if (join.on) {
        join.on = false;
        SPT_HIP(hipEventRecord(ctx->ev_join, sg));
        SPT_HIP(hipStreamWaitEvent(s, ctx->ev_join, 0));
    }
    if ((rc = check_cancel(ctx))) return rc;
    SPT_HIP(timed(ctx, SPT_KERNEL_COMBINE, [&] { return spt::launch_combine(s, res, so.weights, (int)B, (int)k, (int)h, out); }));
    if (taps) {
        if ((rc = copy_tap(ctx, taps->ids, so.ids, n * 4))) return rc;
        if ((rc = copy_tap(ctx, taps->weights, so.weights, n * 4))) return rc;
        if ((rc = copy_tap(ctx, taps->counts, so.counts, E * 4))) return rc;
        if ((rc = copy_tap(ctx, taps->offsets, so.offsets, (E + 1) * 4))) return rc;
        if ((rc = copy_tap(ctx, taps->list, so.list, n * 4))) return rc;
        if ((rc = copy_tap(ctx, taps->active, so.active, E * 4))) return rc;
        if ((rc = copy_tap(ctx, taps->n_active, so.n_active, 4))) return rc;
        if ((rc = copy_tap(ctx, taps->act, act, n * d * 4))) return rc;
        if ((rc = copy_tap(ctx, taps->results, res, n * h * 4))) return rc;
    }
    return SPT_OK;
}

// Tokens per launch sequence: a batch of more selections than
// spt::kMaxSelections runs as consecutive slices of this many whole tokens.
// The reference accepts any batch (forward/moe_batch.go:29-38,84-90), and a
// token's output depends only on its own row of x, so slicing changes no
// routing; the slices' own expert groups decide which of the grouped GEMV
// and GEMM each group takes, as for separate calls of those tokens.
int64_t moe_slice_tokens(const MoEDims &m) { return spt::kMaxSelections / m.k; }

int run_moe(spt_ctx *ctx, const spt_moe_layer *lw, const float *x, float *out, const MoEDims &m,
            const spt_moe_taps *taps) {
    const MoELayout L = moe_layout(ctx, m, taps && taps->act, 0);
    char *S;
    int rc;
    if ((rc = arena(ctx, L.total, &S))) return rc;
    return run_moe_at(ctx, lw, x, out, m, taps, S, L);
}

// Quantize `rows` activation rows of nb blocks into the scratch arena: Q8_0
// codes, scales, per-block code sums (Q4_0) and the E4M3 digit table (MXFP4).
int quantize_into_scratch(spt_ctx *ctx, const float *x, int64_t rows, int64_t nb, Carve &c, char **S,
                          int8_t **codes, float **scales, int32_t **sumq, uint8_t **mxtab) {
    size_t o_c = c.take(rows * nb * 32), o_s = c.take(rows * nb * 4), o_q = c.take(rows * nb * 4);
    size_t o_m = c.take(mxtab ? rows * nb * 64 : 0);
    int rc;
    if ((rc = arena(ctx, c.off, S))) return rc;
    *codes = (int8_t *)(*S + o_c);
    *scales = (float *)(*S + o_s);
    *sumq = (int32_t *)(*S + o_q);
    if (mxtab) *mxtab = (uint8_t *)(*S + o_m);
    SPT_HIP(timed(ctx, SPT_KERNEL_QUANTIZE, [&] {
        return spt::launch_quantize(ctx->stream, x, rows * nb, *codes, *scales, *sumq, mxtab ? *mxtab : nullptr, nullptr,
                                    nullptr);
    }));
    return SPT_OK;
}

int validate_q40_call(spt_ctx *ctx, const spt_tensor *w, const float *x, int64_t x_len, const float *y,
                      int64_t y_len, int64_t batch, int64_t *in, int64_t *out) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil GGUF reader");
    if ((rc = check_cancel(ctx))) return rc;
    int64_t row_bytes;
    if ((rc = q40_shape(w, in, out, &row_bytes))) return rc;
    // no reference counterpart: the device GEMV stages a token's Q8_0 input in LDS
    if (*in > spt::kQ40MaxInput)
        return fail(SPT_ERR_INVALID, "\"%s\": Q4_0 input dimension %lld exceeds the supported %d", tname(w),
                    (long long)*in, spt::kQ40MaxInput);
    if (batch < 1 || batch > INT64_MAX / *in || batch > INT64_MAX / *out)
        return fail(SPT_ERR_INVALID, "invalid or oversized batch: %lld", (long long)batch);
    if (x_len != batch * *in || y_len != batch * *out)
        return fail(SPT_ERR_INVALID, "\"%s\": expected %lld input and %lld output elements, got %lld and %lld",
                    tname(w), (long long)(batch * *in), (long long)(batch * *out), (long long)x_len,
                    (long long)y_len);
    if (!x || !y) return fail(SPT_ERR_INVALID, "nil input or output");
    if (ranges_overlap(x, (uint64_t)x_len * 4, y, (uint64_t)y_len * 4))
        return fail(SPT_ERR_INVALID, "input and output must not overlap");
    if (batch > INT_MAX || *out > INT_MAX) return fail(SPT_ERR_INVALID, "invalid or oversized batch: %lld", (long long)batch);
    return SPT_OK;
}

// The projection bias: addBias (forward/layer.go:225-242) for one vector,
// biasBatch / readFloatVector (layer_batch.go:124-128, layer.go:279-289)
// for a batch.  *present = false for an absent bias.
int projection_bias_check(const spt_tensor *b, int64_t out, int64_t batch, bool *present, int *btype) {
    *present = false;
    if (!b) return SPT_OK;
    const bool empty = b->nbytes == 0;
    if (empty && !named(*b)) return SPT_OK;
    if (empty && batch == 1) return fail(SPT_ERR_INVALID, "\"%s\": invalid bias range", tname(b));
    uint64_t width = 4;
    if (b->type == SPT_TYPE_F16 || b->type == SPT_TYPE_BF16)
        width = 2;
    else if (b->type != SPT_TYPE_F32)
        return fail(SPT_ERR_INVALID, "\"%s\": unsupported float tensor type %u", tname(b), b->type);
    if (b->n_dims != 1 || b->shape[0] != (uint64_t)out || b->nbytes != width * (uint64_t)out)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid float vector shape or range", tname(b));
    if (!b->data) return fail(SPT_ERR_INVALID, "\"%s\": tensor is not resident (nil data)", tname(b));
    if ((uintptr_t)b->data & (width - 1))
        return fail(SPT_ERR_INVALID, "\"%s\": bias data must be %llu-byte aligned", tname(b),
                    (unsigned long long)width);
    *present = true;
    *btype = (int)b->type;
    return SPT_OK;
}

int check_resid(const float *resid, int64_t y_len, const void *in, uint64_t in_bytes, const float *y) {
    if (resid && (ranges_overlap(resid, (uint64_t)y_len * 4, in, in_bytes) ||
                  ranges_overlap(resid, (uint64_t)y_len * 4, y, (uint64_t)y_len * 4)))
        return fail(SPT_ERR_INVALID, "residual overlaps the input or output");
    return SPT_OK;
}

// MulQ40BatchInto's checks (forward/q40.go:46-71) with the input given as
// batch x in/32 GGML Q8_0 blocks (34 bytes each, 2-byte aligned).
int validate_q40_q8_call(spt_ctx *ctx, const spt_tensor *w, const void *xq, int64_t batch, const float *y,
                         int64_t y_len, int64_t *in, int64_t *out) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil GGUF reader");
    if ((rc = check_cancel(ctx))) return rc;
    int64_t row_bytes;
    if ((rc = q40_shape(w, in, out, &row_bytes))) return rc;
    if (*in > spt::kQ40MaxInput)
        return fail(SPT_ERR_INVALID, "\"%s\": Q4_0 input dimension %lld exceeds the supported %d", tname(w),
                    (long long)*in, spt::kQ40MaxInput);
    if (batch < 1 || batch > INT_MAX || batch > INT64_MAX / (*in / 32 * 34) || batch > INT64_MAX / *out)
        return fail(SPT_ERR_INVALID, "invalid or oversized batch: %lld", (long long)batch);
    if (y_len != batch * *out)
        return fail(SPT_ERR_INVALID, "\"%s\": expected %lld output elements, got %lld", tname(w),
                    (long long)(batch * *out), (long long)y_len);
    if (!xq || !y) return fail(SPT_ERR_INVALID, "nil input or output");
    if ((uintptr_t)xq & 1) return fail(SPT_ERR_INVALID, "Q8_0 input must be 2-byte aligned");
    if (ranges_overlap(xq, (uint64_t)(batch * (*in / 32)) * 34, y, (uint64_t)y_len * 4))
        return fail(SPT_ERR_INVALID, "input and output must not overlap");
    if (*out > INT_MAX) return fail(SPT_ERR_INVALID, "invalid or oversized batch: %lld", (long long)batch);
    return SPT_OK;
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Grow-only pinned host buffer of the context: the host-slice entry points
// stage their inputs and outputs there (a pageable copy, then DMA).
int staging(spt_ctx *ctx, size_t bytes, char **out) {
    if (bytes > ctx->pinned_bytes) {
        if (ctx->pinned) {
            hipError_t e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
            (void)hipHostFree(ctx->pinned);
            ctx->pinned = nullptr;
            ctx->pinned_bytes = 0;
        }
        const size_t want = bytes + bytes / 4 + 4096;
        if (hipHostMalloc(&ctx->pinned, want, hipHostMallocDefault) != hipSuccess) {
            ctx->pinned = nullptr;
            return fail(SPT_ERR_NOMEM, "cannot allocate %zu bytes of pinned host staging", want);
        }
        ctx->pinned_bytes = want;
    }
    *out = static_cast<char *>(ctx->pinned);
    return SPT_OK;
}

// One Q4_0 projection of a call (validated).
struct Q40Proj {
    const spt_tensor *w;
    int64_t out;
    bool has_bias;
    int btype;
    const void *bias;
    float *y;
    float *resid;
};

// The int8-MFMA GEMM forms and their split-K subset: spt::q40_gemm_form
// and spt::q40_gemm_split (launch_q40_gemv's choice).
bool q40_gemm_form(int64_t out, int64_t batch) { return spt::q40_gemm_form(out, batch); }
bool q40_split(int64_t out, int64_t batch) { return spt::q40_gemm_split(out, batch); }

// The launch of each of the np <= 3 projections of a call over one input:
// 0 the GEMV, 1 the GEMM, 2 the split-K GEMM.
void q40_launches(const Q40Proj *p, int np, int64_t batch, int *k) {
    for (int i = 0; i < np; i++) k[i] = !q40_gemm_form(p[i].out, batch) ? 0 : !q40_split(p[i].out, batch) ? 1 : 2;
}

// Arena layout of a Q4_0 call over np projections sharing one input.  The
// activation views (codes, widened scales, code sums) exist unless the input
// is GGML Q8_0 blocks that every projection's GEMV reads directly.
// A call of a few tokens (spt::q40_dec_form) runs as one launch that
// quantizes or unpacks its input itself: no views.
// A call of 5 to 64 tokens on inputs up to 128 blocks (spt::q40_tile_form)
// runs as one launch over every projection reading GGML Q8_0 blocks: the
// caller's, or those the quantizer writes into the arena (o_q34) first.
struct Q40Plan {
    bool views, dec, tile;
    int64_t nb, batch;
    size_t o_c, o_s, o_q, o_part, o_q34, total;
};

Q40Plan q40_plan(const Q40Proj *p, int np, int64_t nb, int64_t batch, bool q8_in, size_t base) {
    Q40Plan L{};
    bool gemm = false;
    size_t part = 0;
    L.dec = spt::q40_dec_form(batch, nb);
    for (int i = 0; i < np; i++)
        if (p[i].w->nbytes >= spt::kQ40DecMaxBytes) L.dec = false;
    L.tile = !L.dec && spt::q40_tile_form(batch, nb);
    int k[3];
    q40_launches(p, np, batch, k);
    for (int i = 0; i < np && !L.tile; i++) {
        if (k[i] == 0) continue;
        gemm = true;
        if (k[i] == 2) part += (size_t)spt::kQ40SplitK * batch * p[i].out * 4;
    }
    L.views = !L.dec && !L.tile && (!q8_in || gemm);
    L.nb = nb;
    L.batch = batch;
    Carve c;
    c.off = base;
    L.o_c = c.take(L.views ? batch * nb * 32 : 0);
    L.o_s = c.take(L.views ? batch * nb * 4 : 0);
    L.o_q = c.take(L.views ? batch * nb * 4 : 0);
    L.o_part = c.take(part);
    L.o_q34 = c.take(L.tile && !q8_in ? batch * nb * spt::kQ80Block : 0);
    L.total = c.off;
    return L;
}

// Quantize (x) or unpack (xq34) the input into the plan's views when it has
// them, then one GEMV launch over every projection not on a GEMM form, one
// GEMM launch over those on the wide GEMM form and one over those on the
// split form (launches over several matrices of the same input fill the GPU
// where one narrow matrix alone would not).
int run_q40_at(spt_ctx *ctx, const Q40Proj *p, int np, const Q40Plan &L, char *S, const float *x,
               const uint8_t *xq34) {
    const int64_t nb = L.nb, batch = L.batch;
    int rc;
    if (L.tile) {
        if (x) {
            uint8_t *q = (uint8_t *)(S + L.o_q34);
            SPT_HIP(timed(ctx, SPT_KERNEL_QUANTIZE, [&] {
                return spt::launch_quantize(ctx->stream, x, batch * nb, nullptr, nullptr, nullptr, nullptr, q, nullptr);
            }));
            xq34 = q;
        }
        spt::Q40Args g{};
        for (int i = 0; i < np; i++) {
            const spt_tensor *w = p[i].w;
            if (i == 0) {
                g = spt::Q40Args{(const uint8_t *)w->data, w->nbytes, (int)p[i].out, (int)nb, nullptr, nullptr, nullptr,
                                 (int)batch, p[i].y, p[i].bias, p[i].btype, p[i].resid, nullptr};
            } else {
                g.more[i - 1] = spt::Q40Mat{(const uint8_t *)w->data, w->nbytes, (int)p[i].out, p[i].y, p[i].bias,
                                            p[i].btype, p[i].resid};
            }
        }
        g.nmore = np - 1;
        g.xq34 = xq34;
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_Q40, [&] { return spt::launch_q40_tile(ctx->stream, g, ctx->n_cu); }));
        return SPT_OK;
    }
    int8_t *codes = L.views ? (int8_t *)(S + L.o_c) : nullptr;
    float *scales = L.views ? (float *)(S + L.o_s) : nullptr;
    int32_t *sumq = L.views ? (int32_t *)(S + L.o_q) : nullptr;
    if (L.views) {
        SPT_HIP(timed(ctx, SPT_KERNEL_QUANTIZE, [&] {
            return x ? spt::launch_quantize(ctx->stream, x, batch * nb, codes, scales, sumq, nullptr, nullptr, nullptr)
                     : spt::launch_q8_unpack(ctx->stream, xq34, batch * nb, codes, scales, sumq, nullptr);
        }));
    }
    // the three launches' arguments: 0 GEMV, 1 wide GEMM, 2 split GEMM
    spt::Q40Args g[3]{};
    int ng[3] = {0, 0, 0}, kl[3];
    q40_launches(p, np, batch, kl);
    for (int i = 0; i < np; i++) {
        const spt_tensor *w = p[i].w;
        const int k = kl[i];
        if (ng[k] == 0) {
            g[k] = spt::Q40Args{(const uint8_t *)w->data, w->nbytes, (int)p[i].out, (int)nb, codes, scales, sumq,
                                (int)batch, p[i].y, p[i].bias, p[i].btype, p[i].resid,
                                k == 2 ? (float *)(S + L.o_part) : nullptr};
        } else {
            g[k].more[ng[k] - 1] = spt::Q40Mat{(const uint8_t *)w->data, w->nbytes, (int)p[i].out, p[i].y, p[i].bias,
                                               p[i].btype, p[i].resid};
        }
        g[k].nmore = ng[k]++;
    }
    for (int k = 1; k < 3; k++) {
        if (!ng[k]) continue;
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_Q40, [&] { return spt::launch_q40_gemm(ctx->stream, g[k]); }));
    }
    if (ng[0]) {
        g[0].xq34 = L.views ? nullptr : xq34;
        if ((rc = check_cancel(ctx))) return rc;
        if (L.dec) {
            g[0].xf = x;
            SPT_HIP(timed(ctx, SPT_KERNEL_Q40, [&] { return spt::launch_q40_dec(ctx->stream, g[0]); }));
        } else {
            SPT_HIP(timed(ctx, SPT_KERNEL_Q40, [&] { return spt::launch_q40_gemv(ctx->stream, g[0]); }));
        }
    }
    return SPT_OK;
}

// MulQ80Argmax's checks (forward/q80.go:20-45).
int validate_q80_argmax(spt_ctx *ctx, const spt_tensor *w, const float *x, int64_t x_len, int64_t *best_token,
                        float *best_logit, int64_t *in, int64_t *out) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil reader");
    if ((rc = check_cancel(ctx))) return rc;
    if ((rc = q80_shape(w, in, out))) return rc;
    if (x_len != *in)
        return fail(SPT_ERR_INVALID, "\"%s\": expected %lld input elements, got %lld", tname(w), (long long)*in,
                    (long long)x_len);
    if (!x || !best_token || !best_logit) return fail(SPT_ERR_INVALID, "nil input or output");
    return SPT_OK;
}

// Arena layout of the argmax: per-wave partial (logit, row) pairs and the
// merged pair (8 bytes at o_out).
struct Q80ArgmaxPlan {
    int waves;
    size_t o_v, o_i, o_out;
};

Q80ArgmaxPlan q80_argmax_plan(const spt_ctx *ctx, int64_t in, int64_t out, size_t base, size_t *total) {
    Q80ArgmaxPlan L{};
    L.waves = spt::q80_grid_waves((int)out, (int)(in / 32), ctx->n_cu);
    Carve c;
    c.off = base;
    L.o_v = c.take((size_t)L.waves * 4);
    L.o_i = c.take((size_t)L.waves * 4);
    L.o_out = c.take(8);
    *total = c.off;
    return L;
}

int q80_argmax_at(spt_ctx *ctx, const spt_tensor *w, int64_t in, int64_t out, const float *x, char *S,
                  const Q80ArgmaxPlan &L) {
    spt::Q80Args a{};
    a.w = (const uint8_t *)w->data;
    a.nbytes = w->nbytes;
    a.rows = (int)out;
    a.nb = (int)(in / 32);
    a.x = x;
    a.part_v = (float *)(S + L.o_v);
    a.part_i = (int32_t *)(S + L.o_i);
    a.out_v = (float *)(S + L.o_out);
    a.out_i = (int32_t *)(S + L.o_out + 4);
    SPT_HIP(timed(ctx, SPT_KERNEL_Q80, [&] { return spt::launch_q80_rows(ctx->stream, a, ctx->n_cu); }));
    return SPT_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Residency from the model files
// ---------------------------------------------------------------------------
namespace {

// Byte size of a tensor of one of the path's GGML types from its shape (the
// per-type sizes of ggufindex's tensorSize, ggufindex/index.go:535-574):
// false for another type or a shape that is not a whole number of blocks.
bool path_tensor_bytes(const spt_tensor &t, uint64_t *out) {
    if (t.n_dims < 1 || t.n_dims > 4) return false;
    uint64_t e = 1;
    for (uint32_t i = 0; i < t.n_dims; i++) {
        if (t.shape[i] != 0 && e > UINT64_MAX / t.shape[i]) return false;
        e *= t.shape[i];
    }
    uint64_t block = 1, bytes;
    switch (t.type) {
    case SPT_TYPE_F32: bytes = 4; break;
    case SPT_TYPE_F16:
    case SPT_TYPE_BF16: bytes = 2; break;
    case SPT_TYPE_Q4_0: block = 32, bytes = 18; break;
    case SPT_TYPE_Q8_0: block = 32, bytes = 34; break;
    case SPT_TYPE_MXFP4: block = 32, bytes = 17; break;
    default: return false;
    }
    if (t.shape[0] % block != 0 || e / block > UINT64_MAX / bytes) return false;
    *out = e / block * bytes;
    return true;
}

// Bytes [start, start + n) of a file into device memory at dst: chunks read
// into the two halves of the pinned staging in turn, each half refilled only
// after the copy out of it has completed.
constexpr size_t kLoadChunk = size_t(8) << 20;

int load_range(spt_ctx *ctx, const std::string &path, uint64_t start, uint64_t n, char *dst) {
    char *buf;
    int rc;
    if ((rc = staging(ctx, 2 * kLoadChunk, &buf))) return rc;
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return fail(SPT_ERR_IO, "open %s: %s", path.c_str(), strerror(errno));
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    rc = SPT_OK;
    if (fseeko(f, (off_t)start, SEEK_SET) != 0) rc = fail(SPT_ERR_IO, "seek %s: %s", path.c_str(), strerror(errno));
    for (int h = 0; h < 2 && rc == SPT_OK; h++)
        if (hipEventCreateWithFlags(&ev[h], hipEventDisableTiming) != hipSuccess)
            rc = fail(SPT_ERR_DEVICE, "cannot create an event");
    for (uint64_t off = 0, i = 0; rc == SPT_OK && off < n; off += kLoadChunk, i++) {
        const int h = (int)(i & 1);
        if (used[h] && hipEventSynchronize(ev[h]) != hipSuccess) {
            rc = fail(SPT_ERR_DEVICE, "copy to the device failed");
            break;
        }
        const size_t c = (size_t)std::min<uint64_t>(kLoadChunk, n - off);
        char *half = buf + (size_t)h * kLoadChunk;
        if (fread(half, 1, c, f) != c) {
            rc = fail(SPT_ERR_IO, "read %s: unexpected end of file", path.c_str());
            break;
        }
        hipError_t e = hipMemcpyAsync(dst + off, half, c, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipEventRecord(ev[h], ctx->stream);
        if (e != hipSuccess) {
            rc = hip_fail(e, "hipMemcpyAsync");
            break;
        }
        used[h] = true;
    }
    const hipError_t se = hipStreamSynchronize(ctx->stream);  // the staging is free again
    if (rc == SPT_OK && se != hipSuccess) rc = hip_fail(se, "hipStreamSynchronize");
    for (int h = 0; h < 2; h++)
        if (ev[h]) (void)hipEventDestroy(ev[h]);
    fclose(f);
    return rc;
}

}  // namespace

extern "C" {

const char *spt_last_error(void) { return g_error; }

int spt_ctx_create(int device, void *hip_stream, spt_ctx **out) {
    if (!out) return fail(SPT_ERR_INVALID, "nil output pointer");
    *out = nullptr;
    spt_ctx *ctx = new spt_ctx();
    ctx->device = device;
    if (device >= 0) {
        hipError_t err = hipSetDevice(device);
        if (err != hipSuccess) {
            delete ctx;
            return hip_fail(err, "hipSetDevice");
        }
        ctx->stream = (hipStream_t)hip_stream;  // NULL: the device's default stream
        if (hipDeviceGetAttribute(&ctx->n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
            ctx->n_cu <= 0)
            ctx->n_cu = 256;
        // with the device current: its copy of the no-allocation scratch
        noalloc_scratch_of(device, &ctx->noalloc, &ctx->noalloc_err);
        // the side stream (default priority) and its fork / join events; if
        // any of them cannot be made, layers run on the one stream
        if (hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&ctx->ev_fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&ctx->ev_join, hipEventDisableTiming) != hipSuccess) {
            if (ctx->side) (void)hipStreamDestroy(ctx->side);
            if (ctx->ev_fork) (void)hipEventDestroy(ctx->ev_fork);
            if (ctx->ev_join) (void)hipEventDestroy(ctx->ev_join);
            ctx->side = nullptr;
            ctx->ev_fork = ctx->ev_join = nullptr;
        }
    }
    *out = ctx;
    return SPT_OK;
}

int spt_ctx_destroy(spt_ctx *ctx) {
    if (!ctx) return SPT_OK;
    if (ctx->device >= 0) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->scratch) (void)hipFree(ctx->scratch);
        if (ctx->pinned) (void)hipHostFree(ctx->pinned);
        for (auto &p : ctx->pending) {
            (void)hipEventDestroy(p.second.first);
            (void)hipEventDestroy(p.second.second);
        }
        for (hipEvent_t e : ctx->free_events) (void)hipEventDestroy(e);
        if (ctx->side) {
            (void)hipStreamSynchronize(ctx->side);
            (void)hipStreamDestroy(ctx->side);
            (void)hipEventDestroy(ctx->ev_fork);
            (void)hipEventDestroy(ctx->ev_join);
        }
        if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    }
    delete ctx;
    return SPT_OK;
}

int spt_ctx_enable_timing(spt_ctx *ctx, int enable) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    ctx->timing = enable != 0;
    return SPT_OK;
}

int spt_ctx_read_timing(spt_ctx *ctx, double *total_ms, int64_t *launches) {
    int rc;
    if ((rc = check_ctx(ctx)) || (rc = check_device(ctx))) return rc;
    if (!total_ms || !launches) return fail(SPT_ERR_INVALID, "nil output pointer");
    SPT_HIP(hipStreamSynchronize(ctx->stream));
    for (auto &p : ctx->pending) {
        float ms = 0.0f;
        SPT_HIP(hipEventElapsedTime(&ms, p.second.first, p.second.second));
        ctx->total_ms[p.first] += ms;
        ctx->launches[p.first] += 1;
        ctx->free_events.push_back(p.second.first);
        ctx->free_events.push_back(p.second.second);
    }
    ctx->pending.clear();
    for (int k = 0; k < SPT_KERNEL_KINDS; k++) {
        total_ms[k] = ctx->total_ms[k];
        launches[k] = ctx->launches[k];
        ctx->total_ms[k] = 0.0;
        ctx->launches[k] = 0;
    }
    return SPT_OK;
}

int spt_ctx_synchronize(spt_ctx *ctx) {
    int rc;
    if ((rc = check_ctx(ctx)) || (rc = check_device(ctx))) return rc;
    SPT_HIP(hipStreamSynchronize(ctx->stream));
    return SPT_OK;
}

int spt_ctx_set_gemm_min_group(spt_ctx *ctx, int32_t min_group) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (min_group < 0) return fail(SPT_ERR_INVALID, "negative GEMM group threshold %d", (int)min_group);
    ctx->gemm_min_group = min_group;
    return SPT_OK;
}

int spt_ctx_set_decode_max_selections(spt_ctx *ctx, int32_t max_selections) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    ctx->decode_max_selections = max_selections;
    return SPT_OK;
}

int spt_ctx_set_cancel_flag(spt_ctx *ctx, const volatile int32_t *flag) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    ctx->cancel = flag;
    return SPT_OK;
}

int spt_alloc(spt_ctx *ctx, uint64_t nbytes, void **out_dev) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!out_dev) return fail(SPT_ERR_INVALID, "nil output pointer");
    if ((rc = check_device(ctx))) return rc;
    // 64 spare bytes: no kernel reads past a tensor, the slack only keeps
    // rounding-up arithmetic inside the allocation.
    if (hipMalloc(out_dev, nbytes + 64) != hipSuccess) {
        *out_dev = nullptr;
        return fail(SPT_ERR_NOMEM, "cannot allocate %llu bytes", (unsigned long long)nbytes);
    }
    return SPT_OK;
}

int spt_free(spt_ctx *ctx, void *dev) {
    int rc;
    if ((rc = check_ctx(ctx)) || (rc = check_device(ctx))) return rc;
    if (dev) SPT_HIP(hipFree(dev));
    return SPT_OK;
}

int spt_copy_h2d(spt_ctx *ctx, void *dst_dev, const void *src_host, uint64_t nbytes) {
    int rc;
    if ((rc = check_ctx(ctx)) || (rc = check_device(ctx))) return rc;
    if (nbytes == 0) return SPT_OK;
    if (!dst_dev || !src_host) return fail(SPT_ERR_INVALID, "nil copy pointer");
    SPT_HIP(hipMemcpyAsync(dst_dev, src_host, nbytes, hipMemcpyHostToDevice, ctx->stream));
    SPT_HIP(hipStreamSynchronize(ctx->stream));
    return SPT_OK;
}

int spt_copy_d2h(spt_ctx *ctx, void *dst_host, const void *src_dev, uint64_t nbytes) {
    int rc;
    if ((rc = check_ctx(ctx)) || (rc = check_device(ctx))) return rc;
    if (nbytes == 0) return SPT_OK;
    if (!dst_host || !src_dev) return fail(SPT_ERR_INVALID, "nil copy pointer");
    SPT_HIP(hipMemcpyAsync(dst_host, src_dev, nbytes, hipMemcpyDeviceToHost, ctx->stream));
    SPT_HIP(hipStreamSynchronize(ctx->stream));
    return SPT_OK;
}

int spt_tensor_upload(spt_ctx *ctx, spt_tensor *t, const void *src_host) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!t || (!src_host && t->nbytes)) return fail(SPT_ERR_INVALID, "nil tensor or source");
    if ((rc = check_device(ctx))) return rc;
    void *d = nullptr;
    if ((rc = spt_alloc(ctx, t->nbytes, &d))) return rc;
    if ((rc = spt_copy_h2d(ctx, d, src_host, t->nbytes))) {
        (void)hipFree(d);
        return rc;
    }
    t->data = d;
    return SPT_OK;
}

int spt_quantize_q8_0(spt_ctx *ctx, const float *x_dev, int64_t n, void *out_dev) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (n < 0 || n % 32 != 0) return fail(SPT_ERR_INVALID, "length %lld is not a multiple of 32", (long long)n);
    if (n && (!x_dev || !out_dev)) return fail(SPT_ERR_INVALID, "nil input or output");
    if (ranges_overlap(x_dev, (uint64_t)n * 4, out_dev, (uint64_t)n / 32 * 34))
        return fail(SPT_ERR_INVALID, "input and output must not overlap");
    if ((rc = check_device(ctx)) || (rc = check_cancel(ctx))) return rc;
    SPT_HIP(spt::launch_quantize(ctx->stream, x_dev, n / 32, nullptr, nullptr, nullptr, nullptr, (uint8_t *)out_dev,
                                 nullptr));
    return SPT_OK;
}

int spt_mul_q40_batch_into(spt_ctx *ctx, const spt_tensor *w, const float *x_dev, int64_t x_len,
                           float *y_dev, int64_t y_len, int64_t batch) {
    return spt_mul_q40_batch_bias_into(ctx, w, nullptr, x_dev, x_len, y_dev, y_len, batch, nullptr);
}

int spt_mul_q40_into(spt_ctx *ctx, const spt_tensor *w, const float *x_dev, int64_t x_len, float *y_dev,
                     int64_t y_len) {
    return spt_mul_q40_batch_bias_into(ctx, w, nullptr, x_dev, x_len, y_dev, y_len, 1, nullptr);
}

int spt_mul_q40_batch_bias_into(spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias, const float *x_dev,
                                int64_t x_len, float *y_dev, int64_t y_len, int64_t batch, float *resid_dev) {
    Q40Proj p;
    int64_t in;
    int rc;
    if ((rc = validate_q40_call(ctx, w, x_dev, x_len, y_dev, y_len, batch, &in, &p.out))) return rc;
    if ((rc = projection_bias_check(bias, p.out, batch, &p.has_bias, &p.btype))) return rc;
    if ((rc = check_resid(resid_dev, y_len, x_dev, (uint64_t)x_len * 4, y_dev))) return rc;
    if ((rc = check_device(ctx))) return rc;
    p.w = w;
    p.bias = p.has_bias ? bias->data : nullptr;
    p.y = y_dev;
    p.resid = resid_dev;
    const Q40Plan plan = q40_plan(&p, 1, in / 32, batch, false, 0);
    char *S;
    if ((rc = arena(ctx, plan.total, &S))) return rc;
    return run_q40_at(ctx, &p, 1, plan, S, x_dev, nullptr);
}

int spt_mul_q40_batch_q8_into(spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias, const void *xq_dev,
                              int64_t batch, float *y_dev, int64_t y_len, float *resid_dev) {
    Q40Proj p;
    int64_t in;
    int rc;
    if ((rc = validate_q40_q8_call(ctx, w, xq_dev, batch, y_dev, y_len, &in, &p.out))) return rc;
    if ((rc = projection_bias_check(bias, p.out, batch, &p.has_bias, &p.btype))) return rc;
    if ((rc = check_resid(resid_dev, y_len, xq_dev, (uint64_t)(batch * (in / 32)) * 34, y_dev))) return rc;
    if ((rc = check_device(ctx))) return rc;
    p.w = w;
    p.bias = p.has_bias ? bias->data : nullptr;
    p.y = y_dev;
    p.resid = resid_dev;
    const Q40Plan plan = q40_plan(&p, 1, in / 32, batch, true, 0);
    char *S;
    if ((rc = arena(ctx, plan.total, &S))) return rc;
    return run_q40_at(ctx, &p, 1, plan, S, nullptr, (const uint8_t *)xq_dev);
}

int spt_mul_q40_qkv_batch_into(spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias, const float *x_dev,
                               const void *xq_dev, int64_t x_len, int64_t batch, float *const *y_dev,
                               const int64_t *y_len) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w || !y_dev || !y_len) return fail(SPT_ERR_INVALID, "nil GGUF reader");
    if (!x_dev == !xq_dev) return fail(SPT_ERR_INVALID, "exactly one of the fp32 and the Q8_0 input must be given");
    Q40Proj p[3];
    int64_t in = 0;
    for (int i = 0; i < 3; i++) {
        int64_t in_i;
        if (x_dev) {
            rc = validate_q40_call(ctx, &w[i], x_dev, x_len, y_dev[i], y_len[i], batch, &in_i, &p[i].out);
        } else {
            rc = validate_q40_q8_call(ctx, &w[i], xq_dev, batch, y_dev[i], y_len[i], &in_i, &p[i].out);
            if (!rc && x_len != batch * in_i)
                rc = fail(SPT_ERR_INVALID, "\"%s\": expected %lld input elements, got %lld", tname(&w[i]),
                          (long long)(batch * in_i), (long long)x_len);
        }
        if (rc) return rc;
        if (i > 0 && in_i != in)
            return fail(SPT_ERR_INVALID, "\"%s\": input dimension %lld differs from %lld", tname(&w[i]),
                        (long long)in_i, (long long)in);
        in = in_i;
        if ((rc = projection_bias_check(bias ? &bias[i] : nullptr, p[i].out, batch, &p[i].has_bias, &p[i].btype)))
            return rc;
        for (int j = 0; j < i; j++)
            if (ranges_overlap(y_dev[i], (uint64_t)y_len[i] * 4, y_dev[j], (uint64_t)y_len[j] * 4))
                return fail(SPT_ERR_INVALID, "projection outputs overlap");
        p[i].w = &w[i];
        p[i].bias = p[i].has_bias ? bias[i].data : nullptr;
        p[i].y = y_dev[i];
        p[i].resid = nullptr;
    }
    if ((rc = check_device(ctx))) return rc;
    const Q40Plan plan = q40_plan(p, 3, in / 32, batch, xq_dev != nullptr, 0);
    char *S;
    if ((rc = arena(ctx, plan.total, &S))) return rc;
    return run_q40_at(ctx, p, 3, plan, S, x_dev, (const uint8_t *)xq_dev);
}

int spt_mul_q40_batch_into_host(spt_ctx *ctx, const spt_tensor *w, const float *x_host, int64_t x_len,
                                float *y_host, int64_t y_len, int64_t batch) {
    Q40Proj p;
    int64_t in;
    int rc;
    if ((rc = validate_q40_call(ctx, w, x_host, x_len, y_host, y_len, batch, &in, &p.out))) return rc;
    if ((rc = check_device(ctx))) return rc;
    // x and y travel through the context's pinned staging buffer and the
    // head of its device arena; nothing is allocated once both have grown
    const size_t xb = align256((size_t)x_len * 4), yb = align256((size_t)y_len * 4);
    p.w = w;
    p.has_bias = false;
    p.btype = 0;
    p.bias = nullptr;
    p.resid = nullptr;
    const Q40Plan plan = q40_plan(&p, 1, in / 32, batch, false, xb + yb);
    char *S, *P;
    if ((rc = arena(ctx, plan.total, &S)) || (rc = staging(ctx, xb + yb, &P))) return rc;
    p.y = (float *)(S + xb);
    memcpy(P, x_host, (size_t)x_len * 4);
    SPT_HIP(hipMemcpyAsync(S, P, (size_t)x_len * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = run_q40_at(ctx, &p, 1, plan, S, (const float *)S, nullptr);
    if (!rc) {
        SPT_HIP(hipMemcpyAsync(P + xb, S + xb, (size_t)y_len * 4, hipMemcpyDeviceToHost, ctx->stream));
    }
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (rc) return rc;
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    memcpy(y_host, P + xb, (size_t)y_len * 4);
    return SPT_OK;
}

int spt_mul_q80_into(spt_ctx *ctx, const spt_tensor *w, const float *x_dev, int64_t x_len, float *y_dev,
                     int64_t y_len) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil context or reader");
    if ((rc = check_cancel(ctx))) return rc;
    int64_t in, out;
    if ((rc = q80_shape(w, &in, &out))) return rc;
    if (x_len != in || y_len != out)
        return fail(SPT_ERR_INVALID, "\"%s\": expected input/output lengths %lld/%lld, got %lld/%lld", tname(w),
                    (long long)in, (long long)out, (long long)x_len, (long long)y_len);
    if (!x_dev || !y_dev) return fail(SPT_ERR_INVALID, "nil input or output");
    if (ranges_overlap(x_dev, (uint64_t)x_len * 4, y_dev, (uint64_t)y_len * 4))
        return fail(SPT_ERR_INVALID, "input and output must not overlap");
    if ((rc = check_device(ctx))) return rc;
    spt::Q80Args a{};
    a.w = (const uint8_t *)w->data;
    a.nbytes = w->nbytes;
    a.rows = (int)out;
    a.nb = (int)(in / 32);
    a.x = x_dev;
    a.y = y_dev;
    SPT_HIP(timed(ctx, SPT_KERNEL_Q80, [&] { return spt::launch_q80_rows(ctx->stream, a, ctx->n_cu); }));
    return SPT_OK;
}

int spt_mul_q80_argmax(spt_ctx *ctx, const spt_tensor *w, const float *x_dev, int64_t x_len, int64_t *best_token,
                       float *best_logit) {
    int rc;
    int64_t in, out;
    if ((rc = validate_q80_argmax(ctx, w, x_dev, x_len, best_token, best_logit, &in, &out))) return rc;
    if ((rc = check_device(ctx))) return rc;
    size_t total;
    const Q80ArgmaxPlan L = q80_argmax_plan(ctx, in, out, 0, &total);
    char *S;
    if ((rc = arena(ctx, total, &S))) return rc;
    if ((rc = q80_argmax_at(ctx, w, in, out, x_dev, S, L))) return rc;
    struct {
        float v;
        int32_t i;
    } res;
    SPT_HIP(hipMemcpyAsync(&res, S + L.o_out, sizeof res, hipMemcpyDeviceToHost, ctx->stream));
    SPT_HIP(hipStreamSynchronize(ctx->stream));
    *best_token = res.i;
    *best_logit = res.v;
    return SPT_OK;
}

int spt_mul_q80_into_host(spt_ctx *ctx, const spt_tensor *w, const float *x_host, int64_t x_len, float *y_host,
                          int64_t y_len) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil context or reader");
    int64_t in, out;
    if ((rc = q80_shape(w, &in, &out))) return rc;
    if (x_len != in || y_len != out)
        return fail(SPT_ERR_INVALID, "\"%s\": expected input/output lengths %lld/%lld, got %lld/%lld", tname(w),
                    (long long)in, (long long)out, (long long)x_len, (long long)y_len);
    if (!x_host || !y_host) return fail(SPT_ERR_INVALID, "nil input or output");
    if ((rc = check_device(ctx))) return rc;
    // x and the logits travel through the context's pinned staging buffer and
    // the head of its device arena
    const size_t xb = align256((size_t)x_len * 4), yb = align256((size_t)y_len * 4);
    char *S, *P;
    if ((rc = arena(ctx, xb + yb, &S)) || (rc = staging(ctx, xb + yb, &P))) return rc;
    memcpy(P, x_host, (size_t)x_len * 4);
    SPT_HIP(hipMemcpyAsync(S, P, (size_t)x_len * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = spt_mul_q80_into(ctx, w, (const float *)S, x_len, (float *)(S + xb), y_len);
    if (!rc) {
        SPT_HIP(hipMemcpyAsync(P + xb, S + xb, (size_t)y_len * 4, hipMemcpyDeviceToHost, ctx->stream));
    }
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (rc) return rc;
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    memcpy(y_host, P + xb, (size_t)y_len * 4);
    return SPT_OK;
}

int spt_mul_q80_argmax_host(spt_ctx *ctx, const spt_tensor *w, const float *x_host, int64_t x_len,
                            int64_t *best_token, float *best_logit) {
    int rc;
    int64_t in, out;
    if ((rc = validate_q80_argmax(ctx, w, x_host, x_len, best_token, best_logit, &in, &out))) return rc;
    if ((rc = check_device(ctx))) return rc;
    const size_t xb = align256((size_t)x_len * 4);
    size_t total;
    const Q80ArgmaxPlan L = q80_argmax_plan(ctx, in, out, xb, &total);
    char *S, *P;
    if ((rc = arena(ctx, total, &S)) || (rc = staging(ctx, xb + 256, &P))) return rc;
    memcpy(P, x_host, (size_t)x_len * 4);
    SPT_HIP(hipMemcpyAsync(S, P, (size_t)x_len * 4, hipMemcpyHostToDevice, ctx->stream));
    rc = q80_argmax_at(ctx, w, in, out, (const float *)S, S, L);
    if (!rc) {
        SPT_HIP(hipMemcpyAsync(P + xb, S + L.o_out, 8, hipMemcpyDeviceToHost, ctx->stream));
    }
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (rc) return rc;
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    float v;
    int32_t i;
    memcpy(&v, P + xb, 4);
    memcpy(&i, P + xb + 4, 4);
    *best_token = i;
    *best_logit = v;
    return SPT_OK;
}

int spt_rmsnorm_into(spt_ctx *ctx, const spt_tensor *weight, const float *x_dev, int64_t x_len, float *y_dev,
                     int64_t y_len, float epsilon, void *q8_dev) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!weight) return fail(SPT_ERR_INVALID, "nil GGUF reader");
    if ((rc = check_cancel(ctx))) return rc;
    if (x_len <= 0 || y_len != x_len || weight->n_dims != 1 || weight->shape[0] != (uint64_t)x_len)
        return fail(SPT_ERR_INVALID, "\"%s\": normalization weight, input, and output dimensions differ",
                    tname(weight));
    if (!x_dev || !y_dev) return fail(SPT_ERR_INVALID, "nil input or output");
    if (x_dev != y_dev && ranges_overlap(x_dev, (uint64_t)x_len * 4, y_dev, (uint64_t)y_len * 4))
        return fail(SPT_ERR_INVALID, "input and output partially overlap");
    if (bad_epsilon(epsilon)) return fail(SPT_ERR_INVALID, "invalid epsilon: %g", (double)epsilon);
    int wtype;
    if ((rc = norm_weight_check(weight, x_len, false, &wtype))) return rc;
    if ((rc = norm_q8_check(q8_dev, x_len, x_dev, y_dev))) return rc;
    if (x_len > INT_MAX) return fail(SPT_ERR_INVALID, "input of %lld elements is too long", (long long)x_len);
    if ((rc = check_device(ctx))) return rc;
    spt::RmsArgs a{x_dev, weight->data, wtype, (int)x_len, 1, epsilon, y_dev, (uint8_t *)q8_dev};
    SPT_HIP(timed(ctx, SPT_KERNEL_RMSNORM, [&] { return spt::launch_rmsnorm(ctx->stream, a, false); }));
    return SPT_OK;
}

int spt_rmsnorm_batch_into(spt_ctx *ctx, const spt_tensor *weight, const float *x_dev, int64_t x_len, float *y_dev,
                           int64_t y_len, int64_t batch, float epsilon, void *q8_dev) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!weight) return fail(SPT_ERR_INVALID, "nil GGUF reader");
    if ((rc = check_cancel(ctx))) return rc;
    if (bad_epsilon(epsilon)) return fail(SPT_ERR_INVALID, "invalid epsilon: %g", (double)epsilon);
    if (batch < 1 || x_len <= 0 || x_len % batch != 0 || y_len != x_len)
        return fail(SPT_ERR_INVALID, "invalid batch %lld for %lld input and %lld output elements", (long long)batch,
                    (long long)x_len, (long long)y_len);
    const int64_t dim = x_len / batch;
    int wtype;
    if ((rc = norm_weight_check(weight, dim, true, &wtype))) return rc;
    if (!x_dev || !y_dev) return fail(SPT_ERR_INVALID, "nil input or output");
    if (x_dev != y_dev && ranges_overlap(x_dev, (uint64_t)x_len * 4, y_dev, (uint64_t)y_len * 4))
        return fail(SPT_ERR_INVALID, "input and output partially overlap");
    if ((rc = norm_q8_check(q8_dev, x_len, x_dev, y_dev))) return rc;
    if (dim > INT_MAX || batch > INT_MAX)
        return fail(SPT_ERR_INVALID, "invalid batch %lld for %lld input and %lld output elements", (long long)batch,
                    (long long)x_len, (long long)y_len);
    if ((rc = check_device(ctx))) return rc;
    spt::RmsArgs a{x_dev, weight->data, wtype, (int)dim, (int)batch, epsilon, y_dev, (uint8_t *)q8_dev};
    SPT_HIP(timed(ctx, SPT_KERNEL_RMSNORM, [&] { return spt::launch_rmsnorm(ctx->stream, a, true); }));
    return SPT_OK;
}

int spt_mul_mxfp4_expert(spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias, int32_t expert,
                         const float *x_dev, int64_t x_len, float *y_dev, int64_t y_len, int64_t batch) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil tensor");
    if (w->n_dims != 3) return fail(SPT_ERR_INVALID, "\"%s\": expected MXFP4 expert tensor", tname(w));
    const int64_t in = (int64_t)w->shape[0], out = (int64_t)w->shape[1], E = (int64_t)w->shape[2];
    if ((rc = validate_expert(w, in, out, E))) return rc;
    if ((rc = validate_gemv_input(w, in))) return rc;
    spt_tensor none{};
    if ((rc = validate_bias(bias ? bias : &none, out, E))) return rc;
    if (expert < 0 || expert >= E) return fail(SPT_ERR_INVALID, "expert %d out of range", expert);
    if (batch < 1 || batch > INT_MAX || x_len != batch * in || y_len != batch * out)
        return fail(SPT_ERR_INVALID, "\"%s\": expected %lld input and %lld output elements, got %lld and %lld",
                    tname(w), (long long)(batch * in), (long long)(batch * out), (long long)x_len,
                    (long long)y_len);
    if (!x_dev || !y_dev) return fail(SPT_ERR_INVALID, "nil input or output");
    if (ranges_overlap(x_dev, (uint64_t)x_len * 4, y_dev, (uint64_t)y_len * 4))
        return fail(SPT_ERR_INVALID, "input and output must not overlap");
    if ((rc = check_device(ctx)) || (rc = check_cancel(ctx))) return rc;
    const int64_t nb = in / 32;
    Carve c;
    char *S;
    int8_t *codes;
    float *scales;
    int32_t *sumq;
    uint8_t *mxtab;
    if ((rc = quantize_into_scratch(ctx, x_dev, batch, nb, c, &S, &codes, &scales, &sumq, &mxtab))) return rc;
    spt::MxMfmaArgs a{};
    a.w[0] = (const uint8_t *)w->data;
    a.expert_bytes = (uint64_t)nb * 17 * out;
    a.rows = (int)out;
    a.nb = (int)nb;
    a.bias[0] = bias ? bias_ptr(*bias) : nullptr;
    a.bias_type[0] = bias ? bias_type(*bias) : 0;
    a.bias_bytes[0] = bias ? bias_bytes(*bias) : 0;
    a.mxtab = mxtab;
    a.codes = codes;
    a.scales = scales;
    a.expert = expert;
    a.ntok = (int)batch;
    a.out = y_dev;
    SPT_HIP(timed(ctx, SPT_KERNEL_DOWN, [&] { return spt::launch_mx_mfma(ctx->stream, spt::kRows, a, 1); }));
    return SPT_OK;
}

int spt_route_moe_batch(spt_ctx *ctx, const spt_tensor *router, const spt_tensor *bias, const float *x_dev,
                        int64_t batch, float *logits_dev) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!router) return fail(SPT_ERR_INVALID, "nil router");
    const int64_t h = (int64_t)router->shape[0], E = (int64_t)router->shape[1];
    int64_t rb;
    if (router->type != SPT_TYPE_F32 || router->n_dims != 2 || !product(&rb, {h, E, 4}) ||
        router->nbytes != (uint64_t)rb || !router->data)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid F32 router shape or range", tname(router));
    if ((uintptr_t)router->data & 3u)
        return fail(SPT_ERR_INVALID, "\"%s\": router data must be 4-byte aligned", tname(router));
    spt_tensor none{};
    if ((rc = validate_bias(bias ? bias : &none, E, 1))) return rc;
    if (h % 32 != 0) return fail(SPT_ERR_INVALID, "hidden dimension %lld is not a multiple of 32", (long long)h);
    if (E > 65535) return fail(SPT_ERR_INVALID, "too many experts: %lld", (long long)E);
    if (batch < 1 || batch > 65535 || batch > INT_MAX / E) return fail(SPT_ERR_INVALID, "invalid or oversized batch: %lld", (long long)batch);
    if (!x_dev || !logits_dev) return fail(SPT_ERR_INVALID, "nil input or output");
    if ((rc = check_device(ctx)) || (rc = check_cancel(ctx))) return rc;
    spt::QuantOut no_q{};
    SPT_HIP(spt::launch_route(ctx->stream, (const float *)router->data, bias ? bias_ptr(*bias) : nullptr,
                              bias ? bias_type(*bias) : 0, x_dev, (int)batch, (int)h, (int)E, logits_dev, no_q));
    return SPT_OK;
}

int spt_forward_moe_batch_ex(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                             const float *x_dev, int64_t x_len, float *out_dev, int64_t out_len, int64_t batch,
                             const spt_moe_taps *taps) {
    MoEDims m;
    int rc;
    if ((rc = validate_moe(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, batch, &m, !taps))) return rc;
    if ((rc = check_cancel(ctx))) return rc;
    if ((rc = check_device(ctx))) return rc;
    const int64_t st = moe_slice_tokens(m);
    for (int64_t t0 = 0; t0 < batch; t0 += st) {
        MoEDims ms = m;
        ms.batch = std::min(st, batch - t0);
        if ((rc = check_cancel(ctx))) return rc;
        if ((rc = run_moe(ctx, lw, x_dev + t0 * m.h, out_dev + t0 * m.h, ms, taps))) return rc;
    }
    return SPT_OK;
}

int spt_forward_moe_batch(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw, const float *x_dev,
                          int64_t x_len, float *out_dev, int64_t out_len, int64_t batch) {
    return spt_forward_moe_batch_ex(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, batch, nullptr);
}

int spt_forward_moe(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw, const float *x_dev,
                    int64_t x_len, float *out_dev, int64_t out_len) {
    if (!cfg) return fail(SPT_ERR_INVALID, "nil MoE configuration");
    if (!lw) return spt_forward_moe_batch_ex(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, 1, nullptr);
    // Decode callers disable an optional expert bias with an empty name: such
    // a descriptor is replaced by the absent tensor whatever its other fields
    // hold (forward/moe.go:57-62).  The router bias is left as given.
    spt_moe_layer w = *lw;
    for (spt_tensor *b : {&w.ffn_gate_exps_bias, &w.ffn_up_exps_bias, &w.ffn_down_exps_bias})
        if (!named(*b)) *b = spt_tensor{};
    return spt_forward_moe_batch_ex(ctx, cfg, &w, x_dev, x_len, out_dev, out_len, 1, nullptr);
}

int spt_forward_moe_batch_host(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                               const float *x_host, int64_t x_len, float *out_host, int64_t out_len,
                               int64_t batch) {
    MoEDims m;
    int rc;
    if ((rc = validate_moe(ctx, cfg, lw, x_host, x_len, out_host, out_len, batch, &m, true))) return rc;
    if ((rc = check_cancel(ctx)) || (rc = check_device(ctx))) return rc;
    // x and out travel through the context's pinned staging buffer and the
    // head of its device arena; nothing is allocated once both have grown
    const int64_t st = moe_slice_tokens(m);
    for (int64_t t0 = 0; t0 < batch; t0 += st) {
        MoEDims ms = m;
        ms.batch = std::min(st, batch - t0);
        const size_t n = (size_t)(ms.batch * m.h);
        const size_t xb = align256(n * 4), ob = align256(n * 4);
        const MoELayout L = moe_layout(ctx, ms, false, xb + ob);
        char *S, *P;
        if ((rc = check_cancel(ctx))) return rc;
        if ((rc = arena(ctx, L.total, &S)) || (rc = staging(ctx, xb + ob, &P))) return rc;
        memcpy(P, x_host + t0 * m.h, n * 4);
        SPT_HIP(hipMemcpyAsync(S, P, n * 4, hipMemcpyHostToDevice, ctx->stream));
        rc = run_moe_at(ctx, lw, (const float *)S, (float *)(S + xb), ms, nullptr, S, L);
        if (!rc) {
            SPT_HIP(hipMemcpyAsync(P + xb, S + xb, n * 4, hipMemcpyDeviceToHost, ctx->stream));
        }
        const hipError_t e = hipStreamSynchronize(ctx->stream);
        if (rc) return rc;
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        memcpy(out_host + t0 * m.h, P + xb, n * 4);
    }
    return SPT_OK;
}

int spt_forward_moe_batch_q8(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw, const float *x_dev,
                             const void *xq_dev, int64_t x_len, float *out_dev, int64_t out_len, int64_t batch) {
    MoEDims m;
    int rc;
    if ((rc = validate_moe(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, batch, &m, true))) return rc;
    if (!xq_dev) return fail(SPT_ERR_INVALID, "nil Q8_0 input");
    if ((uintptr_t)xq_dev & 1) return fail(SPT_ERR_INVALID, "Q8_0 input must be 2-byte aligned");
    if (ranges_overlap(xq_dev, (uint64_t)x_len / 32 * 34, out_dev, (uint64_t)out_len * 4))
        return fail(SPT_ERR_INVALID, "MoE Q8_0 input and output overlap");
    if ((rc = check_cancel(ctx)) || (rc = check_device(ctx))) return rc;
    const int64_t st = moe_slice_tokens(m);
    for (int64_t t0 = 0; t0 < batch; t0 += st) {
        MoEDims ms = m;
        ms.batch = std::min(st, batch - t0);
        const MoELayout L = moe_layout(ctx, ms, false, 0);
        char *S;
        if ((rc = check_cancel(ctx))) return rc;
        if ((rc = arena(ctx, L.total, &S))) return rc;
        if ((rc = run_moe_at(ctx, lw, x_dev + t0 * m.h, out_dev + t0 * m.h, ms, nullptr, S, L,
                             (const uint8_t *)xq_dev + t0 * (m.h / 32) * 34)))
            return rc;
    }
    return SPT_OK;
}

int spt_forward_moe_batch_noalloc(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                                  const float *x_dev, int64_t x_len, float *out_dev, int64_t out_len,
                                  int64_t batch) {
    MoEDims m;
    int rc;
    if ((rc = validate_moe(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, batch, &m))) return rc;
    if ((rc = check_cancel(ctx)) || (rc = check_device(ctx))) return rc;
    const MoELayout L = moe_layout(ctx, m, false, 0);
    if (L.total > kNoAllocScratchBytes)
        return fail(SPT_ERR_INVALID,
                    "MoE batch of %lld tokens needs %zu bytes of scratch; the no-allocation form holds %zu",
                    (long long)batch, L.total, kNoAllocScratchBytes);
    if (!ctx->noalloc)
        return fail(SPT_ERR_DEVICE, "no-allocation scratch unavailable on device %d: %s", ctx->device,
                    hipGetErrorString(ctx->noalloc_err));
    // the same launches as spt_forward_moe_batch over the fixed array; no
    // timing events are recorded (creating them would allocate)
    const bool timing = ctx->timing;
    ctx->timing = false;
    rc = run_moe_at(ctx, lw, x_dev, out_dev, m, nullptr, static_cast<char *>(ctx->noalloc), L);
    ctx->timing = timing;
    return rc;
}

int spt_block_sums(spt_ctx *ctx, const spt_tensor *w, int32_t expert, const void *xq_dev, int64_t rows,
                   int32_t *sums_dev) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w || !xq_dev || !sums_dev) return fail(SPT_ERR_INVALID, "nil argument");
    if (w->type == SPT_TYPE_MXFP4) {
        if (w->n_dims != 3) return fail(SPT_ERR_INVALID, "\"%s\": expected MXFP4 expert tensor", tname(w));
        const int64_t in = (int64_t)w->shape[0], out = (int64_t)w->shape[1], E = (int64_t)w->shape[2];
        if ((rc = validate_expert(w, in, out, E))) return rc;
        if (expert < 0 || expert >= E || rows < 0 || rows > out)
            return fail(SPT_ERR_INVALID, "expert or row count out of range");
        if ((rc = check_device(ctx))) return rc;
        const uint64_t eb = (uint64_t)in / 32 * 17 * out;
        SPT_HIP(spt::launch_block_sums_mx(ctx->stream, (const uint8_t *)w->data + expert * eb, eb, (int)rows,
                                          (int)(in / 32), (const uint8_t *)xq_dev, sums_dev));
        return SPT_OK;
    }
    int64_t in, out, rb;
    if ((rc = q40_shape(w, &in, &out, &rb))) return rc;
    if (expert != 0 || rows < 0 || rows > out) return fail(SPT_ERR_INVALID, "expert or row count out of range");
    if ((rc = check_device(ctx))) return rc;
    SPT_HIP(spt::launch_block_sums_q40(ctx->stream, (const uint8_t *)w->data, w->nbytes, (int)rows,
                                       (int)(in / 32), (const uint8_t *)xq_dev, sums_dev));
    return SPT_OK;
}

int spt_synth_mxfp4(spt_ctx *ctx, void *dst_dev, uint64_t key, uint64_t first_block, uint64_t nblocks,
                    int32_t scale_lo, int32_t scale_hi) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (nblocks && !dst_dev) return fail(SPT_ERR_INVALID, "nil destination");
    if (scale_lo < 0 || scale_hi > 255 || scale_lo > scale_hi)
        return fail(SPT_ERR_INVALID, "invalid E8M0 range [%d, %d]", scale_lo, scale_hi);
    if ((rc = check_device(ctx))) return rc;
    SPT_HIP(spt::launch_synth_mxfp4(ctx->stream, (uint8_t *)dst_dev, key, first_block, nblocks, scale_lo, scale_hi));
    return SPT_OK;
}


// Residency from the model files: a ggufindex.Tensor's Range copied to HBM.
int spt_upload_range(spt_ctx *ctx, const char *path, uint64_t start, uint64_t end, spt_tensor *t) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!path || !t) return fail(SPT_ERR_INVALID, "nil path or tensor");
    if (end < start)
        return fail(SPT_ERR_INVALID, "\"%s\": invalid byte range [%llu, %llu)", tname(t), (unsigned long long)start,
                    (unsigned long long)end);
    if (t->n_dims < 1 || t->n_dims > 4)
        return fail(SPT_ERR_INVALID, "\"%s\": %u dimensions (1 to 4 are supported)", tname(t), t->n_dims);
    const uint64_t n = end - start;
    uint64_t want;
    const bool known = path_tensor_bytes(*t, &want);
    if (t->type == SPT_TYPE_F32 || t->type == SPT_TYPE_F16 || t->type == SPT_TYPE_BF16 || t->type == SPT_TYPE_Q4_0 ||
        t->type == SPT_TYPE_Q8_0 || t->type == SPT_TYPE_MXFP4) {
        if (!known || want != n)
            return fail(SPT_ERR_INVALID, "\"%s\": byte range of %llu bytes does not match its type %u and shape",
                        tname(t), (unsigned long long)n, t->type);
    }
    if ((rc = check_device(ctx))) return rc;
    void *d = nullptr;
    if (n) {
        if ((rc = spt_alloc(ctx, n, &d))) return rc;
        if ((rc = load_range(ctx, path, start, n, (char *)d))) {
            (void)hipFree(d);
            return rc;
        }
    }
    t->nbytes = n;
    t->data = d;
    return SPT_OK;
}

int spt_ctx_memory(spt_ctx *ctx, uint64_t *arena_bytes, uint64_t *staging_bytes) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!arena_bytes || !staging_bytes) return fail(SPT_ERR_INVALID, "nil output pointer");
    *arena_bytes = ctx->scratch_bytes;
    *staging_bytes = ctx->pinned_bytes;
    return SPT_OK;
}

}  // extern "C"
