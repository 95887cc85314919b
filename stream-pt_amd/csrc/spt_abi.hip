// spt_abi.hip -- C ABI of libspt_moe.so (include/spt_moe.h).
//
// Host side of the drop-in boundary: argument validation with the rules and
// messages of Stream-PT's forward package, a per-context device scratch
// arena, and the launch sequences of the operators.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
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
    bool timing = false;
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
    std::vector<hipEvent_t> free_events;
    double total_ms[SPT_KERNEL_KINDS] = {};
    int64_t launches[SPT_KERNEL_KINDS] = {};
    int32_t gemm_min_group = 0;  // 0: the default policy (kGemmMinGroup)
    int n_cu = 0;                // compute units of the device
};

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
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

// Grow-only device scratch; returns a pointer to at least `bytes` bytes.
int scratch(spt_ctx *ctx, size_t bytes, char **out) {
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

// forwardMoEBatch validation (forward/moe_batch.go:81-130).
int validate_moe(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                 const float *x, int64_t x_len, const float *out, int64_t out_len, int64_t batch,
                 MoEDims *dims) {
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
    if (k > spt::kMaxTopK || E > spt::kMaxExperts || batch * k > spt::kMaxSelections)
        return fail(SPT_ERR_INVALID,
                    "MoE shape beyond this device path's limits (experts used <= %d, experts <= %d, "
                    "batch*experts used <= %d)",
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
// least kGemmMinSelections selections and their work items fill the device;
// below that the GEMV's passes are faster (a GEMM item walks the whole input
// dimension serially, so a few large groups leave most CUs idle).
constexpr int kGemmMinGroup = 9;
constexpr int kGemmMinSelections = 1024;

int run_moe(spt_ctx *ctx, const spt_moe_layer *lw, const float *x, float *out, const MoEDims &m,
            const spt_moe_taps *taps) {
    const int64_t h = m.h, d = m.d, E = m.E, k = m.k, B = m.batch, n = B * k;
    const int64_t nbh = h / 32, nbd = d / 32;
    // An expert's group holds at most n selections: with fewer than the
    // threshold no expert can reach the GEMM, which is then not launched.
    // An explicit threshold (spt_ctx_set_gemm_min_group) applies as given;
    // the default also needs kGemmMinSelections and a full device of items.
    const bool forced = ctx->gemm_min_group > 0;
    const int gemm_min = forced ? ctx->gemm_min_group : kGemmMinGroup;
    const bool use_gemm = n >= gemm_min && (forced || n >= kGemmMinSelections);
    Carve c;
    size_t o_xc = c.take(B * h), o_xs = c.take(B * nbh * 4), o_xm = c.take(B * nbh * 64);
    size_t o_xb = c.take(use_gemm ? B * nbh * 64 : 0);
    size_t o_logits = c.take(B * E * 4);
    size_t o_ids = c.take(n * 4), o_w = c.take(n * 4), o_cnt = c.take(E * 4), o_off = c.take((E + 1) * 4);
    size_t o_list = c.take(n * 4), o_act_list = c.take(E * 4), o_na = c.take(4);
    size_t o_gv = c.take(E * 4), o_gvn = c.take(4), o_gvp = c.take((E + 1) * 4);
    size_t o_gm = c.take(E * 4), o_gmn = c.take(4), o_gmt = c.take((E + 1) * 4);
    size_t o_act = c.take(n * d * 4), o_ac = c.take(n * d), o_as = c.take(n * nbd * 4), o_am = c.take(n * nbd * 64);
    size_t o_ab = c.take(use_gemm ? n * nbd * 64 : 0);
    size_t o_res = c.take(n * h * 4);
    char *S;
    int rc;
    if ((rc = scratch(ctx, c.off, &S))) return rc;
    int8_t *xc = (int8_t *)(S + o_xc), *ac = (int8_t *)(S + o_ac);
    float *xs = (float *)(S + o_xs), *logits = (float *)(S + o_logits), *act = (float *)(S + o_act);
    uint8_t *xm = (uint8_t *)(S + o_xm), *am = (uint8_t *)(S + o_am);
    uint32_t *xb = use_gemm ? (uint32_t *)(S + o_xb) : nullptr, *ab = use_gemm ? (uint32_t *)(S + o_ab) : nullptr;
    float *as = (float *)(S + o_as), *res = (float *)(S + o_res);
    spt::SelectOut so{};
    so.ids = (int32_t *)(S + o_ids);
    so.weights = (float *)(S + o_w);
    so.counts = (int32_t *)(S + o_cnt);
    so.offsets = (int32_t *)(S + o_off);
    so.list = (int32_t *)(S + o_list);
    so.active = (int32_t *)(S + o_act_list);
    so.n_active = (int32_t *)(S + o_na);
    so.gemm_min = use_gemm ? gemm_min : INT_MAX;
    so.gemm_units = (int32_t)((d + 127) / 128);
    so.gemm_min_items = forced ? 0 : ctx->n_cu;
    so.gv_active = (int32_t *)(S + o_gv);
    so.gv_n = (int32_t *)(S + o_gvn);
    so.gv_pass_off = (int32_t *)(S + o_gvp);
    so.gm_active = (int32_t *)(S + o_gm);
    so.gm_n = (int32_t *)(S + o_gmn);
    so.gm_tile_off = (int32_t *)(S + o_gmt);
    hipStream_t s = ctx->stream;

    const spt::QuantOut xq{xc, xs, xm, taps ? (uint8_t *)taps->xq : nullptr, xb};
    if ((rc = check_cancel(ctx))) return rc;
    if (taps && taps->logits_in) {
        SPT_HIP(timed(ctx, SPT_KERNEL_QUANTIZE, [&] {
            return spt::launch_quantize(s, x, B * nbh, xq.codes, xq.scales, nullptr, xq.mxtab, xq.blocks34, xq.btab);
        }));
        SPT_HIP(timed(ctx, SPT_KERNEL_SELECT, [&] { return spt::launch_select(s, taps->logits_in, (int)B, (int)E, (int)k, so); }));
        if ((rc = copy_tap(ctx, taps->logits, taps->logits_in, B * E * 4))) return rc;
    } else {
        // router logits + Q8_0 of x in one launch, then top-k + lists
        SPT_HIP(timed(ctx, SPT_KERNEL_ROUTE, [&] {
            return spt::launch_route(s, (const float *)lw->ffn_gate_inp.data, bias_ptr(lw->ffn_gate_inp_bias),
                                     bias_type(lw->ffn_gate_inp_bias), x, (int)B, (int)h, (int)E, logits, xq);
        }));
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_SELECT, [&] { return spt::launch_select(s, logits, (int)B, (int)E, (int)k, so); }));
        if (taps && (rc = copy_tap(ctx, taps->logits, logits, B * E * 4))) return rc;
    }
    const int slots = (int)(n < E ? n : E);
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
    ga.out = taps && taps->act ? act : nullptr;  // fp32 act only for the tap
    ga.tap[0] = taps ? taps->gate : nullptr;
    ga.tap[1] = taps ? taps->up : nullptr;
    ga.act_codes = ac;
    ga.act_scales = as;
    ga.act_mxtab = am;
    ga.act_blocks34 = taps ? (uint8_t *)taps->actq : nullptr;
    if ((rc = check_cancel(ctx))) return rc;
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
            return spt::launch_mx_gemm(s, spt::kGateUp, gg, (int)std::min<int64_t>(items, INT_MAX));
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
        gd.gm_tile_off = so.gm_tile_off;
        gd.offsets = so.offsets;
        gd.list = so.list;
        gd.topk = (int)k;
        gd.out = res;
        const int64_t items = gm_tiles * ((h + 255) / 256);
        if ((rc = check_cancel(ctx))) return rc;
        SPT_HIP(timed(ctx, SPT_KERNEL_DOWN_GEMM, [&] {
            return spt::launch_mx_gemm(s, spt::kDown, gd, (int)std::min<int64_t>(items, INT_MAX));
        }));
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

// Quantize `rows` activation rows of nb blocks into the scratch arena: Q8_0
// codes, scales, per-block code sums (Q4_0) and the E4M3 digit table (MXFP4).
int quantize_into_scratch(spt_ctx *ctx, const float *x, int64_t rows, int64_t nb, Carve &c, char **S,
                          int8_t **codes, float **scales, int32_t **sumq, uint8_t **mxtab) {
    size_t o_c = c.take(rows * nb * 32), o_s = c.take(rows * nb * 4), o_q = c.take(rows * nb * 4);
    size_t o_m = c.take(mxtab ? rows * nb * 64 : 0);
    int rc;
    if ((rc = scratch(ctx, c.off, S))) return rc;
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

}  // namespace

extern "C" {

const char *spt_last_error(void) { return g_error.c_str(); }

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
        for (auto &p : ctx->pending) {
            (void)hipEventDestroy(p.second.first);
            (void)hipEventDestroy(p.second.second);
        }
        for (hipEvent_t e : ctx->free_events) (void)hipEventDestroy(e);
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
    int64_t in, out;
    int rc;
    if ((rc = validate_q40_call(ctx, w, x_dev, x_len, y_dev, y_len, batch, &in, &out))) return rc;
    if ((rc = check_device(ctx))) return rc;
    const int64_t nb = in / 32;
    Carve c;
    // partial sums of the split-K GEMM for narrow projections of large batches
    const bool split = batch >= spt::kQ40SplitMinTokens && out < spt::kQ40GemmMinRows;
    const size_t o_part = c.take(split ? (size_t)spt::kQ40SplitK * batch * out * 4 : 0);
    char *S;
    int8_t *codes;
    float *scales;
    int32_t *sumq;
    if ((rc = quantize_into_scratch(ctx, x_dev, batch, nb, c, &S, &codes, &scales, &sumq, nullptr))) return rc;
    if ((rc = check_cancel(ctx))) return rc;
    spt::Q40Args a{(const uint8_t *)w->data, w->nbytes, (int)out, (int)nb, codes, scales, sumq, (int)batch, y_dev};
    a.part = split ? (float *)(S + o_part) : nullptr;
    SPT_HIP(timed(ctx, SPT_KERNEL_Q40, [&] { return spt::launch_q40_gemv(ctx->stream, a); }));
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

int spt_mul_q40_into(spt_ctx *ctx, const spt_tensor *w, const float *x_dev, int64_t x_len, float *y_dev,
                     int64_t y_len) {
    return spt_mul_q40_batch_into(ctx, w, x_dev, x_len, y_dev, y_len, 1);
}

int spt_mul_q40_batch_bias_into(spt_ctx *ctx, const spt_tensor *w, const spt_tensor *bias, const float *x_dev,
                                int64_t x_len, float *y_dev, int64_t y_len, int64_t batch, float *resid_dev) {
    int64_t in, out;
    int rc;
    if ((rc = validate_q40_call(ctx, w, x_dev, x_len, y_dev, y_len, batch, &in, &out))) return rc;
    bool has_bias;
    int btype = 0;
    if ((rc = projection_bias_check(bias, out, batch, &has_bias, &btype))) return rc;
    if (resid_dev && (ranges_overlap(resid_dev, (uint64_t)y_len * 4, x_dev, (uint64_t)x_len * 4) ||
                      ranges_overlap(resid_dev, (uint64_t)y_len * 4, y_dev, (uint64_t)y_len * 4)))
        return fail(SPT_ERR_INVALID, "residual overlaps the input or output");
    if ((rc = check_device(ctx))) return rc;
    const int64_t nb = in / 32;
    Carve c;
    const bool split = batch >= spt::kQ40SplitMinTokens && out < spt::kQ40GemmMinRows;
    const size_t o_part = c.take(split ? (size_t)spt::kQ40SplitK * batch * out * 4 : 0);
    char *S;
    int8_t *codes;
    float *scales;
    int32_t *sumq;
    if ((rc = quantize_into_scratch(ctx, x_dev, batch, nb, c, &S, &codes, &scales, &sumq, nullptr))) return rc;
    if ((rc = check_cancel(ctx))) return rc;
    spt::Q40Args a{(const uint8_t *)w->data, w->nbytes, (int)out, (int)nb, codes, scales, sumq, (int)batch, y_dev,
                   has_bias ? bias->data : nullptr, btype, resid_dev, split ? (float *)(S + o_part) : nullptr};
    SPT_HIP(timed(ctx, SPT_KERNEL_Q40, [&] { return spt::launch_q40_gemv(ctx->stream, a); }));
    return SPT_OK;
}

int spt_mul_q40_batch_into_host(spt_ctx *ctx, const spt_tensor *w, const float *x_host, int64_t x_len,
                                float *y_host, int64_t y_len, int64_t batch) {
    int64_t in, out;
    int rc;
    if ((rc = validate_q40_call(ctx, w, x_host, x_len, y_host, y_len, batch, &in, &out))) return rc;
    if ((rc = check_device(ctx))) return rc;
    void *xd = nullptr, *yd = nullptr;
    if ((rc = spt_alloc(ctx, (uint64_t)x_len * 4, &xd))) return rc;
    if ((rc = spt_alloc(ctx, (uint64_t)y_len * 4, &yd))) {
        (void)hipFree(xd);
        return rc;
    }
    rc = spt_copy_h2d(ctx, xd, x_host, (uint64_t)x_len * 4);
    if (!rc) rc = spt_mul_q40_batch_into(ctx, w, (const float *)xd, x_len, (float *)yd, y_len, batch);
    if (!rc) rc = spt_copy_d2h(ctx, y_host, yd, (uint64_t)y_len * 4);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(xd);
    (void)hipFree(yd);
    return rc;
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
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil reader");
    if ((rc = check_cancel(ctx))) return rc;
    int64_t in, out;
    if ((rc = q80_shape(w, &in, &out))) return rc;
    if (x_len != in)
        return fail(SPT_ERR_INVALID, "\"%s\": expected %lld input elements, got %lld", tname(w), (long long)in,
                    (long long)x_len);
    if (!x_dev || !best_token || !best_logit) return fail(SPT_ERR_INVALID, "nil input or output");
    if ((rc = check_device(ctx))) return rc;
    const int waves = spt::q80_grid_waves((int)out, (int)(in / 32), ctx->n_cu);
    Carve c;
    const size_t o_v = c.take((size_t)waves * 4), o_i = c.take((size_t)waves * 4), o_out = c.take(8);
    char *S;
    if ((rc = scratch(ctx, c.off, &S))) return rc;
    spt::Q80Args a{};
    a.w = (const uint8_t *)w->data;
    a.nbytes = w->nbytes;
    a.rows = (int)out;
    a.nb = (int)(in / 32);
    a.x = x_dev;
    a.part_v = (float *)(S + o_v);
    a.part_i = (int32_t *)(S + o_i);
    a.out_v = (float *)(S + o_out);
    a.out_i = (int32_t *)(S + o_out + 4);
    SPT_HIP(timed(ctx, SPT_KERNEL_Q80, [&] { return spt::launch_q80_rows(ctx->stream, a, ctx->n_cu); }));
    struct {
        float v;
        int32_t i;
    } res;
    SPT_HIP(hipMemcpyAsync(&res, S + o_out, sizeof res, hipMemcpyDeviceToHost, ctx->stream));
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
    void *xd = nullptr, *yd = nullptr;
    if ((rc = spt_alloc(ctx, (uint64_t)x_len * 4, &xd))) return rc;
    if ((rc = spt_alloc(ctx, (uint64_t)y_len * 4, &yd))) {
        (void)hipFree(xd);
        return rc;
    }
    rc = spt_copy_h2d(ctx, xd, x_host, (uint64_t)x_len * 4);
    if (!rc) rc = spt_mul_q80_into(ctx, w, (const float *)xd, x_len, (float *)yd, y_len);
    if (!rc) rc = spt_copy_d2h(ctx, y_host, yd, (uint64_t)y_len * 4);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(xd);
    (void)hipFree(yd);
    return rc;
}

int spt_mul_q80_argmax_host(spt_ctx *ctx, const spt_tensor *w, const float *x_host, int64_t x_len,
                            int64_t *best_token, float *best_logit) {
    int rc;
    if ((rc = check_ctx(ctx))) return rc;
    if (!w) return fail(SPT_ERR_INVALID, "nil reader");
    int64_t in, out;
    if ((rc = q80_shape(w, &in, &out))) return rc;
    if (x_len != in)
        return fail(SPT_ERR_INVALID, "\"%s\": expected %lld input elements, got %lld", tname(w), (long long)in,
                    (long long)x_len);
    if (!x_host || !best_token || !best_logit) return fail(SPT_ERR_INVALID, "nil input or output");
    if ((rc = check_device(ctx))) return rc;
    void *xd = nullptr;
    if ((rc = spt_alloc(ctx, (uint64_t)x_len * 4, &xd))) return rc;
    rc = spt_copy_h2d(ctx, xd, x_host, (uint64_t)x_len * 4);
    if (!rc) rc = spt_mul_q80_argmax(ctx, w, (const float *)xd, x_len, best_token, best_logit);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(xd);
    return rc;
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
    if ((rc = validate_moe(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, batch, &m))) return rc;
    if ((rc = check_cancel(ctx))) return rc;
    if ((rc = check_device(ctx))) return rc;
    return run_moe(ctx, lw, x_dev, out_dev, m, taps);
}

int spt_forward_moe_batch(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw, const float *x_dev,
                          int64_t x_len, float *out_dev, int64_t out_len, int64_t batch) {
    return spt_forward_moe_batch_ex(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, batch, nullptr);
}

int spt_forward_moe(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw, const float *x_dev,
                    int64_t x_len, float *out_dev, int64_t out_len) {
    if (!cfg) return fail(SPT_ERR_INVALID, "nil MoE configuration");
    return spt_forward_moe_batch_ex(ctx, cfg, lw, x_dev, x_len, out_dev, out_len, 1, nullptr);
}

int spt_forward_moe_batch_host(spt_ctx *ctx, const spt_moe_config *cfg, const spt_moe_layer *lw,
                               const float *x_host, int64_t x_len, float *out_host, int64_t out_len,
                               int64_t batch) {
    MoEDims m;
    int rc;
    if ((rc = validate_moe(ctx, cfg, lw, x_host, x_len, out_host, out_len, batch, &m))) return rc;
    if ((rc = check_cancel(ctx)) || (rc = check_device(ctx))) return rc;
    void *xd = nullptr, *od = nullptr;
    if ((rc = spt_alloc(ctx, (uint64_t)x_len * 4, &xd))) return rc;
    if ((rc = spt_alloc(ctx, (uint64_t)out_len * 4, &od))) {
        (void)hipFree(xd);
        return rc;
    }
    rc = spt_copy_h2d(ctx, xd, x_host, (uint64_t)x_len * 4);
    if (!rc) rc = run_moe(ctx, lw, (const float *)xd, (float *)od, m, nullptr);
    if (!rc) rc = spt_copy_d2h(ctx, out_host, od, (uint64_t)out_len * 4);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(xd);
    (void)hipFree(od);
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

}  // extern "C"
