// C ABI of the MI355X MoE block (include/pbmoe.h).
//
// Host responsibilities: validate every shape, dtype, alignment and route
// before anything is launched (as scheduler/protocol.rs:1564-1676 and
// metal/mod.rs:3264-3319 do), own device copies of bound weights, size the
// scratch buffers, and launch the gfx950 kernels on the context stream.
// Errors are explicit status codes plus a thread-local message; there is no
// fallback implementation behind any entry point.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <thread>

#include "../../include/pbmoe.h"
#include "pbmoe_internal.h"
#include "pbmoe_pack.h"

#define PBMOE_API extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok()
{
    return PBMOE_OK;
}

#define HIP_TRY(expr)                                                                          \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return fail(e_ == hipErrorOutOfMemory ? PBMOE_ERR_OUT_OF_MEMORY : PBMOE_ERR_DEVICE, \
                        "%s: %s", #expr, hipGetErrorString(e_));                               \
    } while (0)

// Limits of the current kernels (explicitly rejected beyond them).
constexpr uint32_t MAX_EXPERTS = 1024;
static_assert(MAX_EXPERTS + 1 <= pbmoe::TILE_TABLE_MAX_ITEMS, "prefill tile table too small");
constexpr uint32_t MAX_K = 16;
constexpr uint32_t MAX_DECODE_TOKENS = 16;
constexpr uint32_t MAX_PREFILL_TOKENS = 32768;
constexpr uint32_t MAX_HIDDEN = 8192;

struct DeviceBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
};

struct LayerBinding {
    pbmoe_layer_desc desc{};
    pbmoe_q4_layout layout{};
    const uint8_t* slots = nullptr;
    size_t slots_bytes = 0;
    DeviceBuf slots_owned;
    const void* router = nullptr; // dense weight, or the codes of router_q4
    uint32_t router_dtype = 0;    // PBMOE_DTYPE_*, or pbmoe::DT_Q4
    pbmoe::Q4Rows router_q4{};
    DeviceBuf router_owned, router_s_owned, router_b_owned;
    const float* sel_bias = nullptr;
    DeviceBuf bias_owned;
    bool has_shared = false;
    pbmoe_q4_layout shared_layout{};
    const uint8_t* shared_slot = nullptr;
    DeviceBuf shared_owned;
    const void* shared_gate = nullptr; // dense row, or the codes of gate_q4
    uint32_t shared_gate_dtype = 0;
    pbmoe::Q4Rows gate_q4{};
    DeviceBuf gate_owned, gate_s_owned, gate_b_owned;
};

// Attention layer: weights referenced, KV cache and rotary table owned.
struct AttnBinding {
    pbmoe_attn_desc desc{};
    pbmoe::AttnArgs base{}; // weights, shapes, cache pointers
    DeviceBuf cache_k, cache_v, inv_freq;
};

} // namespace

struct pbmoe_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::map<uint32_t, LayerBinding> layers;
    std::map<uint32_t, AttnBinding> attn;
    uint32_t* status = nullptr; // device status word
    DeviceBuf logits, act, act_shared, shared_weight, plan;
    DeviceBuf route_ids, route_w;
    DeviceBuf prefill; // prefill scratch (operand splits, activations, y)
    DeviceBuf plan_work; // multi-workgroup plan scratch of pbmoe_dispatch_plan
    DeviceBuf attn_scratch; // q/k/v, chunk partials and attention values of one decode step
    DeviceBuf x_normed;     // [T][H] input RMSNorm rows of pbmoe_moe_layer_norm
    uint32_t cus = 0;            // compute units of the device
    hipEvent_t phase_ev[6] = {};
    bool phase_timing = false;
    hipEvent_t attn_ev[8] = {}; // null unless 14 phase events were set
};

namespace {

void free_buf(DeviceBuf& b)
{
    if (b.ptr)
        (void)hipFree(b.ptr);
    b.ptr = nullptr;
    b.bytes = 0;
}

int ensure(pbmoe_ctx* ctx, DeviceBuf& b, size_t bytes)
{
    if (b.bytes >= bytes && b.ptr)
        return ok();
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    free_buf(b);
    size_t want = bytes < 256 ? 256 : bytes;
    HIP_TRY(hipMalloc(&b.ptr, want));
    b.bytes = want;
    return ok();
}

int set_device(pbmoe_ctx* ctx)
{
    HIP_TRY(hipSetDevice(ctx->device));
    return ok();
}

// Copy or reference a weight source.
int adopt(pbmoe_ctx* ctx, const void* src, size_t bytes, uint32_t flags, DeviceBuf& owned,
          const void** out)
{
    if (flags != PBMOE_MEM_HOST && flags != PBMOE_MEM_DEVICE)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "unknown memory flags %u", flags);
    if (owned.ptr) { // a copy made by an earlier bind: no launch may still read it
        HIP_TRY(hipStreamSynchronize(ctx->stream));
        free_buf(owned);
    }
    if (flags == PBMOE_MEM_DEVICE) {
        *out = src;
        return ok();
    }
    HIP_TRY(hipMalloc(&owned.ptr, bytes));
    owned.bytes = bytes;
    HIP_TRY(hipMemcpyAsync(owned.ptr, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    *out = owned.ptr;
    return ok();
}

bool aligned(const void* p, size_t a)
{
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// Q4 layout checks: QwenMoeQ4ExpertLayout::validate (model_family.rs:1132-1152)
// plus component sizes for the given shape and kernel alignment.
int check_layout(const pbmoe_q4_layout* l, uint32_t hidden, uint32_t intermediate)
{
    if (!l)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "layout is null");
    uint64_t expected = 0;
    for (uint32_t i = 0; i < 9; ++i) {
        const pbmoe_component& c = l->components[i];
        if (c.kind != i)
            return fail(PBMOE_ERR_SHAPE, "expert component %u has kind %u, expected %u", i, c.kind, i);
        if (c.offset != expected)
            return fail(PBMOE_ERR_SHAPE, "expert component %u starts at %llu, expected %llu", i,
                        (unsigned long long)c.offset, (unsigned long long)expected);
        expected += c.bytes;
    }
    if (expected != l->expert_bytes)
        return fail(PBMOE_ERR_SHAPE, "expert layout totals %llu bytes, expected %llu",
                    (unsigned long long)expected, (unsigned long long)l->expert_bytes);
    if (l->scale_bias_dtype == PBMOE_DTYPE_F32)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "F32 scale/bias is the import format only; bind BF16 or F16 slots");
    if (l->scale_bias_dtype != PBMOE_DTYPE_F16 && l->scale_bias_dtype != PBMOE_DTYPE_BF16)
        return fail(PBMOE_ERR_DTYPE, "unknown scale/bias dtype %u", l->scale_bias_dtype);
    if (hidden == 0 && intermediate == 0)
        return ok();
    uint32_t g = l->group_size;
    if (g != 32 && g != 64 && g != 128)
        return fail(PBMOE_ERR_UNSUPPORTED, "group size %u not supported (32, 64, 128)", g);
    if (hidden % g || intermediate % g)
        return fail(PBMOE_ERR_SHAPE, "hidden=%u intermediate=%u must be divisible by group_size=%u",
                    hidden, intermediate, g);
    uint64_t packed = (uint64_t)hidden * intermediate / 2;
    uint64_t sb = (uint64_t)hidden * (intermediate / g) * 2;
    uint64_t sb_gu = (uint64_t)intermediate * (hidden / g) * 2;
    for (int p = 0; p < 3; ++p) {
        uint64_t want_sb = p == 2 ? sb : sb_gu;
        if (l->components[3 * p].bytes != packed || l->components[3 * p + 1].bytes != want_sb ||
            l->components[3 * p + 2].bytes != want_sb)
            return fail(PBMOE_ERR_SHAPE, "projection %d component sizes do not match %ux%u group %u",
                        p, hidden, intermediate, g);
        if (l->components[3 * p].offset % 16)
            return fail(PBMOE_ERR_ALIGNMENT, "projection %d packed weights not 16-byte aligned", p);
        if (l->components[3 * p + 1].offset % 2 || l->components[3 * p + 2].offset % 2)
            return fail(PBMOE_ERR_ALIGNMENT, "projection %d scale/bias not 2-byte aligned", p);
    }
    if (l->expert_bytes % 16)
        return fail(PBMOE_ERR_ALIGNMENT, "expert slot stride %llu not a multiple of 16",
                    (unsigned long long)l->expert_bytes);
    return ok();
}

pbmoe::ExpertSet make_set(const uint8_t* base, const pbmoe_q4_layout& l, uint32_t count,
                          uint32_t hidden, uint32_t intermediate)
{
    pbmoe::ExpertSet s{};
    s.base = base;
    s.stride = l.expert_bytes;
    s.count = count;
    s.group = l.group_size;
    s.group_shift = l.group_size == 32 ? 5u : (l.group_size == 64 ? 6u : 7u);
    s.sb_dtype = l.scale_bias_dtype;
    auto proj = [&](int p) {
        pbmoe::Q4Proj q{};
        q.w_off = l.components[3 * p].offset;
        q.s_off = l.components[3 * p + 1].offset;
        q.b_off = l.components[3 * p + 2].offset;
        q.rows = p == 2 ? hidden : intermediate;
        q.cols = p == 2 ? intermediate : hidden;
        return q;
    };
    s.gate = proj(0);
    s.up = proj(1);
    s.down = proj(2);
    return s;
}

int get_layer(pbmoe_ctx* ctx, uint32_t layer, LayerBinding** out)
{
    auto it = ctx->layers.find(layer);
    if (it == ctx->layers.end())
        return fail(PBMOE_ERR_NOT_BOUND, "layer %u is not bound", layer);
    *out = &it->second;
    return ok();
}

int plan_buffers(pbmoe_ctx* ctx, uint32_t experts, uint32_t routes, pbmoe::Plan* plan)
{
    size_t words = (size_t)experts * 3 + 1 + (size_t)routes * 3;
    const size_t work = pbmoe::plan_work_words(routes, experts);
    int rc = ensure(ctx, ctx->plan, (words + work) * 4);
    if (rc)
        return rc;
    uint32_t* p = static_cast<uint32_t*>(ctx->plan.ptr);
    plan->unique_ids = p;
    plan->unique_count = p + experts;
    plan->groups = p + experts + 1;
    plan->route_slots = p + experts * 3 + 1;
    plan->src_rows = plan->route_slots + routes;
    plan->out_idx = plan->src_rows + routes;
    plan->work = plan->out_idx + routes;
    return ok();
}

} // namespace

// ---------------------------------------------------------------------------
PBMOE_API int pbmoe_abi_version(void)
{
    return PBMOE_ABI_VERSION;
}

PBMOE_API const char* pbmoe_last_error(void)
{
    return g_last_error.c_str();
}

// QwenMoeQ4ExpertLayout::fixed_bf16, model_family.rs:954-1068
PBMOE_API int pbmoe_q4_layout_fixed(uint32_t hidden, uint32_t intermediate, uint32_t group_size,
                                    uint32_t sb_dtype, pbmoe_q4_layout* out)
{
    if (!out)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "out is null");
    if (hidden == 0 || intermediate == 0 || group_size == 0)
        return fail(PBMOE_ERR_SHAPE,
                    "fixed-Q4 expert layout requires non-zero hidden, intermediate, and group dimensions");
    if (hidden % group_size || intermediate % group_size)
        return fail(PBMOE_ERR_SHAPE,
                    "fixed-Q4 expert dimensions hidden=%u intermediate=%u must be divisible by group_size=%u",
                    hidden, intermediate, group_size);
    if (sb_dtype != PBMOE_DTYPE_F16 && sb_dtype != PBMOE_DTYPE_BF16)
        return fail(PBMOE_ERR_DTYPE, "fixed-Q4 scale/bias dtype must be F16 or BF16");
    uint64_t values = (uint64_t)hidden * intermediate;
    if (values % 2)
        return fail(PBMOE_ERR_SHAPE, "fixed-Q4 projection element count %llu must be even",
                    (unsigned long long)values);
    uint64_t packed = values / 2;
    uint64_t sb_gu = (uint64_t)intermediate * (hidden / group_size) * 2;
    uint64_t sb_d = (uint64_t)hidden * (intermediate / group_size) * 2;
    uint64_t sizes[9] = {packed, sb_gu, sb_gu, packed, sb_gu, sb_gu, packed, sb_d, sb_d};
    uint64_t off = 0;
    for (uint32_t i = 0; i < 9; ++i) {
        out->components[i].kind = i;
        out->components[i].reserved = 0;
        out->components[i].offset = off;
        out->components[i].bytes = sizes[i];
        off += sizes[i];
    }
    out->expert_bytes = off;
    out->group_size = group_size;
    out->scale_bias_dtype = sb_dtype;
    return ok();
}

PBMOE_API int pbmoe_q4_layout_validate(const pbmoe_q4_layout* layout)
{
    return check_layout(layout, 0, 0);
}

// validate_preselected, scheduler/protocol.rs:1044-1081
PBMOE_API int pbmoe_validate_routes(const uint32_t* ids, const float* scores, uint32_t count,
                                    uint32_t active_experts, uint32_t experts)
{
    if (active_experts == 0 || active_experts > experts)
        return fail(PBMOE_ERR_INVALID_ARGUMENT,
                    "active expert count %u must be in 1..=%u", active_experts, experts);
    if (count != active_experts)
        return fail(PBMOE_ERR_ROUTE, "received %u preselected experts; expected %u", count,
                    active_experts);
    if (!ids || !scores)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ids/scores are null");
    for (uint32_t i = 0; i < count; ++i) {
        if (ids[i] >= experts)
            return fail(PBMOE_ERR_ROUTE, "selected expert %u outside expert count %u", ids[i],
                        experts);
        if (!std::isfinite(scores[i]))
            return fail(PBMOE_ERR_NONFINITE, "selected expert %u has non-finite score %g", ids[i],
                        (double)scores[i]);
        for (uint32_t j = 0; j < i; ++j)
            if (ids[j] == ids[i])
                return fail(PBMOE_ERR_ROUTE, "selected expert %u more than once", ids[i]);
    }
    return ok();
}

// ScheduledExpertRoutes::from_routes_with_policy, expert_access.rs:80-135
PBMOE_API int pbmoe_renormalize_routes(const float* scores, uint32_t count, uint32_t normalization,
                                       float routed_scale, float* weights)
{
    if (!scores || !weights)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "scores/weights are null");
    if (!(std::isfinite(routed_scale) && routed_scale > 0.0f))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "routed expert scale must be positive and finite");
    for (uint32_t i = 0; i < count; ++i)
        if (!std::isfinite(scores[i]))
            return fail(PBMOE_ERR_NONFINITE, "route score %u is not finite", i);
    float sum = -0.0f;
    for (uint32_t i = 0; i < count; ++i)
        sum = sum + scores[i];
    float inv;
    if (normalization == PBMOE_NORM_RENORMALIZE_SELECTED) {
        if (!(std::isfinite(sum) && sum > 0.0f))
            return fail(PBMOE_ERR_ROUTE, "selected expert probabilities must have a positive finite sum");
        inv = 1.0f / sum;
    } else if (normalization == PBMOE_NORM_DEEPSEEK_FLOOR) {
        if (!(std::isfinite(sum) && sum >= 0.0f))
            return fail(PBMOE_ERR_ROUTE,
                        "DeepSeek selected expert probabilities must have a finite non-negative sum");
        inv = 1.0f / std::fmax(sum, 6.103515625e-5f);
    } else if (normalization == PBMOE_NORM_PRESERVE_FULL_SOFTMAX) {
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "unsupported routing weights: preserving probabilities from the full expert softmax");
    } else {
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "unknown normalization %u", normalization);
    }
    for (uint32_t i = 0; i < count; ++i) {
        if (scores[i] < 0.0f)
            return fail(PBMOE_ERR_ROUTE, "selected expert probabilities must be non-negative");
        weights[i] = scores[i] * inv;
    }
    for (uint32_t i = 0; i < count; ++i)
        weights[i] = weights[i] * routed_scale;
    return ok();
}

PBMOE_API int pbmoe_ctx_create(int device, pbmoe_ctx** out)
{
    if (!out)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n)
        return fail(PBMOE_ERR_DEVICE, "device %d not present (%d devices)", device, n);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(PBMOE_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950",
                    device, prop.gcnArchName);
    pbmoe_ctx* ctx = new pbmoe_ctx();
    ctx->device = device;
    ctx->cus = prop.multiProcessorCount > 0 ? (uint32_t)prop.multiProcessorCount : 0u;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess)
        e = pbmoe::static_scratch_init(device); // device address of the static scratch, once per device
    if (e == hipSuccess)
        e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess)
        e = hipMalloc(reinterpret_cast<void**>(&ctx->status), 256);
    if (e == hipSuccess)
        e = hipMemsetAsync(ctx->status, 0, 256, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        int rc = fail(PBMOE_ERR_DEVICE, "context setup failed: %s", hipGetErrorString(e));
        if (ctx->stream)
            (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return rc;
    }
    *out = ctx;
    return ok();
}

PBMOE_API int pbmoe_ctx_destroy(pbmoe_ctx* ctx)
{
    if (!ctx)
        return ok();
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->layers) {
        free_buf(kv.second.slots_owned);
        free_buf(kv.second.router_owned);
        free_buf(kv.second.bias_owned);
        free_buf(kv.second.shared_owned);
        free_buf(kv.second.gate_owned);
    }
    for (auto& kv : ctx->attn) {
        free_buf(kv.second.cache_k);
        free_buf(kv.second.cache_v);
        free_buf(kv.second.inv_freq);
    }
    for (DeviceBuf* b : {&ctx->logits, &ctx->act, &ctx->act_shared, &ctx->shared_weight,
                         &ctx->plan, &ctx->route_ids, &ctx->route_w, &ctx->prefill,
                         &ctx->plan_work, &ctx->attn_scratch, &ctx->x_normed})
        free_buf(*b);
    (void)hipFree(ctx->status);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return ok();
}

PBMOE_API int pbmoe_ctx_stream(pbmoe_ctx* ctx, void** stream)
{
    if (!ctx || !stream)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    *stream = ctx->stream;
    return ok();
}

// commit_and_wait with the reference's 120 s limit (metal/mod.rs:539-540)
PBMOE_API int pbmoe_sync(pbmoe_ctx* ctx)
{
    if (!ctx)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ctx is null");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    auto t0 = std::chrono::steady_clock::now();
    for (;;) {
        hipError_t q = hipStreamQuery(ctx->stream);
        if (q == hipSuccess)
            break;
        if (q != hipErrorNotReady)
            return fail(PBMOE_ERR_DEVICE, "stream failed: %s", hipGetErrorString(q));
        if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(120))
            return fail(PBMOE_ERR_TIMEOUT, "device work did not complete within 120 s");
        std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
    uint32_t st = 0;
    HIP_TRY(hipMemcpy(&st, ctx->status, 4, hipMemcpyDeviceToHost));
    if (st) {
        HIP_TRY(hipMemset(ctx->status, 0, 4));
        if (st & pbmoe::ST_NONFINITE)
            return fail(PBMOE_ERR_NONFINITE, "router produced a non-finite score");
        if (st & pbmoe::ST_ROUTE_RANGE)
            return fail(PBMOE_ERR_ROUTE, "a route selected an expert outside the expert count");
        if (st & (pbmoe::ST_BAD_SUM | pbmoe::ST_NEGATIVE))
            return fail(PBMOE_ERR_ROUTE,
                        "selected expert probabilities must have a positive finite sum");
        if (st & pbmoe::ST_F16_RANGE)
            return fail(PBMOE_ERR_NONFINITE,
                        "a prefill SwiGLU activation, or a sum of 64 of them, exceeded the f16 "
                        "operand range (|a| > 65504)");
        return fail(PBMOE_ERR_DEVICE, "device status 0x%x", st);
    }
    return ok();
}

// Per-kernel device timing of the decode launches (the counterpart of the
// reference's FlashMoeTimingBuckets / record_detailed_timing, types.rs:600-619,
// runtime/mod.rs:1470): events (hipEvent_t) 2i / 2i+1 are the start / stop
// events of kernel i (router stage, gate/up, down+combine), attached to the
// dispatch packets; 8 more time the attention decode kernels.
PBMOE_API int pbmoe_set_phase_events(pbmoe_ctx* ctx, void* const* events, uint32_t count)
{
    if (!ctx)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ctx is null");
    if (count == 0) {
        ctx->phase_timing = false;
        for (hipEvent_t& e : ctx->attn_ev)
            e = nullptr;
        return ok();
    }
    if ((count != 6 && count != 14) || !events)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "phase timing takes 6 or 14 events (or 0 to disable)");
    for (uint32_t i = 0; i < count; ++i)
        if (!events[i])
            return fail(PBMOE_ERR_INVALID_ARGUMENT, "phase event %u is null", i);
    for (uint32_t i = 0; i < 6; ++i)
        ctx->phase_ev[i] = static_cast<hipEvent_t>(events[i]);
    for (uint32_t i = 0; i < 8; ++i)
        ctx->attn_ev[i] = count == 14 ? static_cast<hipEvent_t>(events[6 + i]) : nullptr;
    ctx->phase_timing = true;
    return ok();
}

// Measurement reference: a read stream of known size (see the header).
PBMOE_API int pbmoe_stream_read(pbmoe_ctx* ctx, const void* src, size_t bytes, uint32_t* xor_out)
{
    if (!ctx || !src || !xor_out)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if (bytes == 0 || bytes % 16 || !aligned(src, 16) || !aligned(xor_out, 4))
        return fail(PBMOE_ERR_ALIGNMENT, "stream read needs a 16-byte aligned source of a multiple of 16 bytes");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    HIP_TRY(pbmoe::launch_stream_read(ctx->stream, src, bytes, xor_out));
    return ok();
}

PBMOE_API int pbmoe_device_alloc(pbmoe_ctx* ctx, size_t bytes, void** dptr)
{
    if (!ctx || !dptr)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    HIP_TRY(hipMalloc(dptr, bytes ? bytes : 1));
    return ok();
}

PBMOE_API int pbmoe_device_free(pbmoe_ctx* ctx, void* dptr)
{
    if (!ctx)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ctx is null");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(dptr));
    return ok();
}

PBMOE_API int pbmoe_upload(pbmoe_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    if (!ctx || (!dst && bytes) || (!src && bytes))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok();
}

PBMOE_API int pbmoe_download(pbmoe_ctx* ctx, void* dst, const void* src, size_t bytes)
{
    if (!ctx || (!dst && bytes) || (!src && bytes))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok();
}

// Sigmoid routing selects on sigmoid(l) + bias and needs the bias; the
// DeepSeek-V4 router's correction bias is optional (deepseek.rs:1361-1374).
static bool needs_selection_bias(uint32_t routing)
{
    return routing == PBMOE_ROUTING_SIGMOID_NOAUX || routing == PBMOE_ROUTING_SIGMOID_GROUPED;
}

// Drop whatever is bound at `layer` (slots, router, selection bias, shared
// expert), after the stream has finished every launch that may read it.  A
// rebind therefore starts from an empty binding: the router and the shared
// expert sized for the old descriptor are never used with the new one.
static int release_layer(pbmoe_ctx* ctx, uint32_t layer)
{
    auto it = ctx->layers.find(layer);
    if (it == ctx->layers.end())
        return PBMOE_OK;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    LayerBinding& b = it->second;
    free_buf(b.slots_owned);
    for (DeviceBuf* o : {&b.router_owned, &b.router_s_owned, &b.router_b_owned, &b.bias_owned,
                         &b.shared_owned, &b.gate_owned, &b.gate_s_owned, &b.gate_b_owned})
        free_buf(*o);
    ctx->layers.erase(it);
    return PBMOE_OK;
}

// Layer descriptor + slot layout checks shared by pbmoe_bind_layer and
// pbmoe_bind_layer_file.
static int check_layer_desc(const pbmoe_layer_desc* d, const pbmoe_q4_layout* layout)
{
    if (d->experts == 0 || d->experts > MAX_EXPERTS)
        return fail(PBMOE_ERR_UNSUPPORTED, "experts=%u outside 1..=%u", d->experts, MAX_EXPERTS);
    if (d->active_experts == 0 || d->active_experts > d->experts)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "active expert count %u must be in 1..=%u",
                    d->active_experts, d->experts);
    if (d->active_experts > MAX_K)
        return fail(PBMOE_ERR_UNSUPPORTED, "active experts %u > %u", d->active_experts, MAX_K);
    if (d->hidden == 0 || d->hidden % 256 || d->hidden > MAX_HIDDEN)
        return fail(PBMOE_ERR_UNSUPPORTED, "hidden=%u must be a multiple of 256 and <= %u",
                    d->hidden, MAX_HIDDEN);
    // the decode down kernel is instantiated for these row lengths only
    switch (d->intermediate) {
    case 256: case 512: case 768: case 1024: case 1536: case 2048: break;
    default:
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "intermediate=%u is not one of 256, 512, 768, 1024, 1536, 2048", d->intermediate);
    }
    if (d->routing > PBMOE_ROUTING_SQRT_SOFTPLUS)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "unknown routing %u", d->routing);
    if (d->normalization == PBMOE_NORM_PRESERVE_FULL_SOFTMAX)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "unsupported routing weights: preserving probabilities from the full expert "
                    "softmax requires a declared scheduler implementation");
    if (d->normalization > PBMOE_NORM_DEEPSEEK_FLOOR)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "unknown normalization %u", d->normalization);
    if (d->route_order > PBMOE_ORDER_REFERENCE_SLOT)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "unknown route order %u", d->route_order);
    if (!(std::isfinite(d->routed_scale) && d->routed_scale > 0.0f))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "routed expert scale must be positive and finite");
    if (d->routing == PBMOE_ROUTING_SQRT_SOFTPLUS && d->route_order == PBMOE_ORDER_REFERENCE_SLOT)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "the DeepSeek-V4 router orders routes by a stable sort; use the canonical order");
    if (d->routing == PBMOE_ROUTING_SIGMOID_GROUPED) {
        if (d->n_group == 0 || d->n_group > 64 || d->experts % d->n_group ||
            d->topk_group == 0 || d->topk_group > d->n_group ||
            (d->n_group > 1 && d->experts / d->n_group < 2))
            return fail(PBMOE_ERR_SHAPE, "group-limited routing needs experts %% n_group == 0, "
                                         "n_group <= 64, 1 <= topk_group <= n_group");
        if (d->route_order == PBMOE_ORDER_REFERENCE_SLOT)
            return fail(PBMOE_ERR_UNSUPPORTED,
                        "group-limited routing has no reference slot order; use canonical");
        if (d->active_experts > d->topk_group * (d->experts / d->n_group))
            return fail(PBMOE_ERR_SHAPE, "K=%u exceeds the %u experts of the kept groups",
                        d->active_experts, d->topk_group * (d->experts / d->n_group));
    }
    if (d->shared_intermediate && d->shared_intermediate != d->intermediate)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "shared intermediate %u must equal routed intermediate %u",
                    d->shared_intermediate, d->intermediate);
    return check_layout(layout, d->hidden, d->intermediate);
}

PBMOE_API int pbmoe_bind_layer(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_layer_desc* d,
                               const pbmoe_q4_layout* layout, const void* slots,
                               size_t slots_bytes, uint32_t flags)
{
    if (!ctx || !d || !layout || !slots)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_layer_desc(d, layout);
    if (rc)
        return rc;
    if (slots_bytes < (size_t)layout->expert_bytes * d->experts)
        return fail(PBMOE_ERR_SHAPE, "slots hold %zu bytes, %u experts need %llu", slots_bytes,
                    d->experts, (unsigned long long)layout->expert_bytes * d->experts);
    if (flags == PBMOE_MEM_DEVICE && !aligned(slots, 16))
        return fail(PBMOE_ERR_ALIGNMENT, "device slot base must be 16-byte aligned");
    rc = set_device(ctx);
    if (rc)
        return rc;
    if ((rc = release_layer(ctx, layer)))
        return rc;
    LayerBinding& b = ctx->layers[layer];
    b.desc = *d;
    b.layout = *layout;
    const void* dev = nullptr;
    rc = adopt(ctx, slots, (size_t)layout->expert_bytes * d->experts, flags, b.slots_owned, &dev);
    if (rc) {
        free_buf(b.slots_owned);
        ctx->layers.erase(layer);
        return rc;
    }
    b.slots = static_cast<const uint8_t*>(dev);
    b.slots_bytes = (size_t)layout->expert_bytes * d->experts;
    return ok();
}

// ---- on-disk expert packs (layer_NN.bin + layer_NN.json) -------------------

static void copy_format(char (&dst)[48], const std::string& src)
{
    const size_t n = std::min(src.size(), sizeof(dst) - 1);
    memcpy(dst, src.data(), n);
    dst[n] = 0;
}

PBMOE_API int pbmoe_pack_inspect(const char* root, uint32_t layer, pbmoe_pack_info* info)
{
    if (!root || !info)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    pbmoe::pack::LayerMeta m;
    std::string err;
    int rc = pbmoe::pack::read_layer_meta(root, layer, &m, &err);
    if (rc)
        return fail(rc, "%s", err.c_str());
    *info = pbmoe_pack_info{};
    copy_format(info->format, m.format);
    info->layer = (uint32_t)m.layer;
    info->experts = (uint32_t)std::min<uint64_t>(m.experts, UINT32_MAX);
    info->expert_size = m.expert_size;
    const int64_t fb = pbmoe::pack::file_size(pbmoe::pack::layer_bin_path(root, layer));
    info->file_bytes = fb < 0 ? 0 : (uint64_t)fb;
    info->packs = (uint32_t)m.packs.size();
    for (const auto& p : m.packs)
        info->records += (uint32_t)p.records.size();
    return ok();
}

// Per-tensor records of a fixed-Q4 pack, when present, must describe the
// bound layout: copy_pbq4_record_to_fixed_q4_component (experts/slots.rs:
// 1056-1113) writes one record per projection with record_offset and
// packed_bytes of its weight component, the projection's shape, the layout's
// group size, groups = scale count, scale_bias_dtype "BF16".  F16 is
// accepted for an F16 layout.
static int check_pack_records(const pbmoe::pack::LayerMeta& m, const pbmoe_q4_layout* l,
                              uint32_t hidden, uint32_t inter, const std::string& path)
{
    static const char* const suffix[3] = {"gate_proj.weight", "up_proj.weight", "down_proj.weight"};
    for (const auto& p : m.packs) {
        for (const auto& r : p.records) {
            int proj = -1;
            for (int q = 0; q < 3; ++q) {
                const size_t n = strlen(suffix[q]);
                if (r.tensor.size() >= n && r.tensor.compare(r.tensor.size() - n, n, suffix[q]) == 0)
                    proj = q;
            }
            if (proj < 0)
                return fail(PBMOE_ERR_FORMAT, "%s expert %llu: record %s is not a gate/up/down projection",
                            path.c_str(), (unsigned long long)p.expert, r.tensor.c_str());
            const pbmoe_component& w = l->components[3 * proj];
            const pbmoe_component& sc = l->components[3 * proj + 1];
            const uint64_t rows = proj == 2 ? hidden : inter, cols = proj == 2 ? inter : hidden;
            if (r.shape.size() != 2 || r.shape[0] != rows || r.shape[1] != cols)
                return fail(PBMOE_ERR_FORMAT, "%s expert %llu: record %s shape does not match %llux%llu",
                            path.c_str(), (unsigned long long)p.expert, r.tensor.c_str(),
                            (unsigned long long)rows, (unsigned long long)cols);
            if (r.record_offset != w.offset || r.packed_bytes != w.bytes)
                return fail(PBMOE_ERR_FORMAT,
                            "%s expert %llu: record %s at offset %llu (%llu bytes), layout has %llu (%llu)",
                            path.c_str(), (unsigned long long)p.expert, r.tensor.c_str(),
                            (unsigned long long)r.record_offset, (unsigned long long)r.packed_bytes,
                            (unsigned long long)w.offset, (unsigned long long)w.bytes);
            if (r.group_size != l->group_size || r.groups != sc.bytes / 2)
                return fail(PBMOE_ERR_FORMAT, "%s expert %llu: record %s has %llu groups of %llu, layout %llu of %u",
                            path.c_str(), (unsigned long long)p.expert, r.tensor.c_str(),
                            (unsigned long long)r.groups, (unsigned long long)r.group_size,
                            (unsigned long long)(sc.bytes / 2), l->group_size);
            const bool bf16 = strcasecmp(r.scale_bias_dtype.c_str(), "BF16") == 0 ||
                              strcasecmp(r.scale_bias_dtype.c_str(), "BFLOAT16") == 0;
            const bool f16 = strcasecmp(r.scale_bias_dtype.c_str(), "F16") == 0 ||
                             strcasecmp(r.scale_bias_dtype.c_str(), "FLOAT16") == 0;
            if ((l->scale_bias_dtype == PBMOE_DTYPE_BF16 && !bf16) || (l->scale_bias_dtype == PBMOE_DTYPE_F16 && !f16))
                return fail(PBMOE_ERR_DTYPE, "%s expert %llu: record %s scale/bias dtype %s does not match the layout",
                            path.c_str(), (unsigned long long)p.expert, r.tensor.c_str(),
                            r.scale_bias_dtype.c_str());
        }
    }
    return ok();
}

// Copy `bytes` of the file at `path` into device memory through two pinned
// staging buffers: while the copy engine moves chunk i, reader threads fill
// chunk i + 1 with positioned reads (the reference reads expert bytes with
// parallel pread, experts/mod.rs:267-281).
static int stream_file_to_device(pbmoe_ctx* ctx, const std::string& path, uint64_t bytes, uint8_t* dev)
{
    constexpr size_t CHUNK = 64u << 20;
    constexpr int READERS = 4;
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0)
        return fail(PBMOE_ERR_IO, "failed to open %s: %s", path.c_str(), strerror(errno));
    void* pin[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = ok();
    hipError_t he = hipSuccess;
    for (int i = 0; i < 2 && he == hipSuccess; ++i) {
        he = hipHostMalloc(&pin[i], CHUNK, hipHostMallocDefault);
        if (he == hipSuccess)
            he = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    }
    if (he != hipSuccess)
        rc = fail(PBMOE_ERR_DEVICE, "staging buffers: %s", hipGetErrorString(he));
    uint64_t off = 0;
    for (uint32_t i = 0; rc == 0 && off < bytes; ++i) {
        const int b = i & 1;
        if (i >= 2 && (he = hipEventSynchronize(done[b])) != hipSuccess) {
            rc = fail(PBMOE_ERR_DEVICE, "staging wait: %s", hipGetErrorString(he));
            break;
        }
        const size_t n = (size_t)std::min<uint64_t>(CHUNK, bytes - off);
        std::atomic<int> read_err{0};
        std::thread readers[READERS];
        for (int k = 0; k < READERS; ++k) {
            readers[k] = std::thread([&, k]() {
                size_t lo = n * k / READERS, hi = n * (k + 1) / READERS;
                uint8_t* dst = static_cast<uint8_t*>(pin[b]);
                while (lo < hi) {
                    const ssize_t got = pread(fd, dst + lo, hi - lo, (off_t)(off + lo));
                    if (got < 0 && errno == EINTR)
                        continue;
                    if (got <= 0) {
                        read_err.store(got < 0 ? errno : EIO);
                        return;
                    }
                    lo += (size_t)got;
                }
            });
        }
        for (auto& t : readers)
            t.join();
        if (read_err.load()) {
            rc = fail(PBMOE_ERR_IO, "failed to read %s at %llu: %s", path.c_str(), (unsigned long long)off,
                      strerror(read_err.load()));
            break;
        }
        if ((he = hipMemcpyAsync(dev + off, pin[b], n, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess ||
            (he = hipEventRecord(done[b], ctx->stream)) != hipSuccess) {
            rc = fail(PBMOE_ERR_DEVICE, "upload: %s", hipGetErrorString(he));
            break;
        }
        off += n;
    }
    // the staging buffers may still be read by queued copies
    he = hipStreamSynchronize(ctx->stream);
    if (he != hipSuccess && rc == 0)
        rc = fail(PBMOE_ERR_DEVICE, "upload: %s", hipGetErrorString(he));
    for (int i = 0; i < 2; ++i) {
        if (done[i])
            (void)hipEventDestroy(done[i]);
        if (pin[i])
            (void)hipHostFree(pin[i]);
    }
    close(fd);
    return rc;
}

// Bind layer `layer` from root/layer_NN.json + layer_NN.bin (NN = file_layer):
// the fixed-Q4 checks of ExpertSlotStore::resolve_execution_descriptor_from
// (experts/store.rs:481-565), then the slots are streamed into HBM, as the
// resident backing of prepare_resident_expert_backing (metal/mod.rs:1382-1402).
PBMOE_API int pbmoe_bind_layer_file(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_layer_desc* d,
                                    const pbmoe_q4_layout* layout, const char* root, uint32_t file_layer)
{
    namespace pk = pbmoe::pack;
    if (!ctx || !d || !layout || !root)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_layer_desc(d, layout);
    if (rc)
        return rc;
    pk::LayerMeta m;
    std::string err;
    if ((rc = pk::read_layer_meta(root, file_layer, &m, &err)))
        return fail(rc, "%s", err.c_str());
    const std::string json = pk::layer_json_path(root, file_layer);
    if (m.format != pk::FORMAT_FIXED_Q4)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "unsupported expert storage at layer %u: format %s; expected %s (PBQ4 formats are "
                    "import compatibility only)", file_layer, m.format.c_str(), pk::FORMAT_FIXED_Q4);
    if (m.expert_size != layout->expert_bytes)
        return fail(PBMOE_ERR_SHAPE, "expert storage layer %u has slot size %llu, expected %llu", file_layer,
                    (unsigned long long)m.expert_size, (unsigned long long)layout->expert_bytes);
    if (m.experts != d->experts || m.packs.size() != d->experts)
        return fail(PBMOE_ERR_SHAPE, "expert storage layer %u declares %llu experts and %zu records, expected %u",
                    file_layer, (unsigned long long)m.experts, m.packs.size(), d->experts);
    for (uint32_t e = 0; e < d->experts; ++e) {
        const pk::Pack* p = m.pack_for(e);
        if (!p)
            return fail(PBMOE_ERR_FORMAT, "expert storage layer %u is missing expert %u", file_layer, e);
        if (p->packed_bytes != m.expert_size)
            return fail(PBMOE_ERR_FORMAT,
                        "expert storage layer %u expert %u has %llu bytes, expected whole-slot payload %llu",
                        file_layer, e, (unsigned long long)p->packed_bytes, (unsigned long long)m.expert_size);
    }
    if ((rc = check_pack_records(m, layout, d->hidden, d->intermediate, json)))
        return rc;
    const std::string bin = pk::layer_bin_path(root, file_layer);
    const int64_t fsize = pk::file_size(bin);
    const uint64_t want = (uint64_t)d->experts * layout->expert_bytes;
    if (fsize < 0)
        return fail(PBMOE_ERR_IO, "failed to stat expert layer %s: %s", bin.c_str(), strerror(errno));
    if ((uint64_t)fsize != want)
        return fail(PBMOE_ERR_SHAPE, "expert storage layer %u has file size %lld, expected %llu", file_layer,
                    (long long)fsize, (unsigned long long)want);
    if ((rc = set_device(ctx)))
        return rc;
    DeviceBuf buf;
    if (hipMalloc(&buf.ptr, want) != hipSuccess)
        return fail(PBMOE_ERR_OUT_OF_MEMORY, "no device memory for %llu slot bytes", (unsigned long long)want);
    buf.bytes = want;
    if ((rc = stream_file_to_device(ctx, bin, want, static_cast<uint8_t*>(buf.ptr)))) {
        free_buf(buf);
        return rc;
    }
    if ((rc = release_layer(ctx, layer))) {
        free_buf(buf);
        return rc;
    }
    LayerBinding& b = ctx->layers[layer];
    b.desc = *d;
    b.layout = *layout;
    b.slots_owned = buf;
    b.slots = static_cast<const uint8_t*>(buf.ptr);
    b.slots_bytes = want;
    return ok();
}

PBMOE_API int pbmoe_layer_slots(pbmoe_ctx* ctx, uint32_t layer, const void** slots, size_t* bytes)
{
    if (!ctx || !slots || !bytes)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    *slots = b->slots;
    *bytes = b->slots_bytes;
    return ok();
}

// After a failed router / gate bind the old pointers may name freed copies:
// leave the layer without a router (gate) rather than with a dangling one.
static void drop_router(pbmoe_ctx* ctx, LayerBinding* b)
{
    (void)hipStreamSynchronize(ctx->stream);
    for (DeviceBuf* o : {&b->router_owned, &b->router_s_owned, &b->router_b_owned})
        free_buf(*o);
    b->router = nullptr;
    b->router_dtype = 0;
    b->router_q4 = pbmoe::Q4Rows{};
    b->sel_bias = nullptr; // its copy may have been replaced by the failed bind
}

static void drop_gate(pbmoe_ctx* ctx, LayerBinding* b)
{
    (void)hipStreamSynchronize(ctx->stream);
    for (DeviceBuf* o : {&b->gate_owned, &b->gate_s_owned, &b->gate_b_owned})
        free_buf(*o);
    b->shared_gate = nullptr;
    b->shared_gate_dtype = 0;
    b->gate_q4 = pbmoe::Q4Rows{};
}

// The selection bias of a router bind, adopted before the router itself so
// that a failed copy leaves no new router without its bias.  No bias: an
// owned copy from an earlier bind is freed.  On failure the layer keeps no
// bias (a sigmoid-routed call then reports it as not bound).
static int adopt_selection_bias(pbmoe_ctx* ctx, LayerBinding* b, const float* selection_bias, uint32_t flags,
                                const float** out)
{
    *out = nullptr;
    if (!selection_bias) {
        if (b->bias_owned.ptr) {
            HIP_TRY(hipStreamSynchronize(ctx->stream));
            free_buf(b->bias_owned);
        }
        return ok();
    }
    const void* dev = nullptr;
    int rc = adopt(ctx, selection_bias, (size_t)b->desc.experts * 4, flags, b->bias_owned, &dev);
    if (rc) {
        b->sel_bias = nullptr;
        return rc;
    }
    *out = static_cast<const float*>(dev);
    return ok();
}

PBMOE_API int pbmoe_bind_router(pbmoe_ctx* ctx, uint32_t layer, const void* weight, uint32_t dtype,
                                const float* selection_bias, uint32_t flags)
{
    if (!ctx || !weight)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    if (dtype > PBMOE_DTYPE_BF16)
        return fail(PBMOE_ERR_DTYPE, "router dtype %u not one of F32/F16/BF16", dtype);
    if (needs_selection_bias(b->desc.routing) && !selection_bias)
        return fail(PBMOE_ERR_INVALID_ARGUMENT,
                    "sigmoid routing requires the per-expert selection bias");
    if (flags == PBMOE_MEM_DEVICE && !aligned(weight, 16))
        return fail(PBMOE_ERR_ALIGNMENT, "device router weight must be 16-byte aligned");
    rc = set_device(ctx);
    if (rc)
        return rc;
    size_t esz = dtype == PBMOE_DTYPE_F32 ? 4 : 2;
    const float* bias = nullptr;
    if ((rc = adopt_selection_bias(ctx, b, selection_bias, flags, &bias)))
        return rc;
    const void* dev = nullptr;
    rc = adopt(ctx, weight, (size_t)b->desc.experts * b->desc.hidden * esz, flags, b->router_owned,
               &dev);
    if (rc) {
        drop_router(ctx, b);
        return rc;
    }
    b->router = dev;
    b->router_dtype = dtype;
    b->router_q4 = pbmoe::Q4Rows{};
    free_buf(b->router_s_owned); // a Q4 router bound before (the stream was synchronised by adopt)
    free_buf(b->router_b_owned);
    b->sel_bias = bias;
    return ok();
}

// Adopt a Q4 matrix [rows][cols] (codes, then 2-byte scales and biases
// [rows][cols / group]) into `out`, copying host memory into the owned buffers.
static int check_q4(const pbmoe_q4_matrix* m, uint32_t cols, uint32_t group, uint32_t flags)
{
    if (!m->codes || !m->scales || !m->biases)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "Q4 matrix needs codes, scales and biases");
    if (group != 32 && group != 64 && group != 128)
        return fail(PBMOE_ERR_UNSUPPORTED, "Q4 group size %u not one of 32/64/128", group);
    if (cols % group)
        return fail(PBMOE_ERR_SHAPE, "Q4 columns %u not divisible by group size %u", cols, group);
    if (flags != PBMOE_MEM_HOST && flags != PBMOE_MEM_DEVICE)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "unknown memory flags %u", flags);
    if (flags == PBMOE_MEM_DEVICE && (!aligned(m->codes, 16) || !aligned(m->scales, 2) || !aligned(m->biases, 2)))
        return fail(PBMOE_ERR_ALIGNMENT, "device Q4 codes must be 16-byte and scales/biases 2-byte aligned");
    return PBMOE_OK;
}

// (arguments checked by check_q4 first)
static int adopt_q4(pbmoe_ctx* ctx, const pbmoe_q4_matrix* m, uint32_t rows, uint32_t cols, uint32_t group,
                    uint32_t flags, DeviceBuf& oc, DeviceBuf& os, DeviceBuf& ob, pbmoe::Q4Rows* out)
{
    const size_t sb = (size_t)rows * (cols / group) * 2;
    const void *c = nullptr, *sc = nullptr, *bi = nullptr;
    int rc = adopt(ctx, m->codes, (size_t)rows * cols / 2, flags, oc, &c);
    if (!rc)
        rc = adopt(ctx, m->scales, sb, flags, os, &sc);
    if (!rc)
        rc = adopt(ctx, m->biases, sb, flags, ob, &bi);
    if (rc)
        return rc;
    out->codes = static_cast<const uint8_t*>(c);
    out->scales = static_cast<const uint8_t*>(sc);
    out->biases = static_cast<const uint8_t*>(bi);
    out->gshift = group == 32 ? 5u : (group == 64 ? 6u : 7u);
    return PBMOE_OK;
}

PBMOE_API int pbmoe_bind_router_q4(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_q4_matrix* weight,
                                   uint32_t group_size, uint32_t scale_bias_dtype,
                                   const float* selection_bias, uint32_t flags)
{
    if (!ctx || !weight)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    if (scale_bias_dtype != b->layout.scale_bias_dtype)
        return fail(PBMOE_ERR_UNSUPPORTED, "Q4 router scale/bias dtype %u must match the experts' (%u)",
                    scale_bias_dtype, b->layout.scale_bias_dtype);
    if (needs_selection_bias(b->desc.routing) && !selection_bias)
        return fail(PBMOE_ERR_INVALID_ARGUMENT,
                    "sigmoid routing requires the per-expert selection bias");
    if ((rc = check_q4(weight, b->desc.hidden, group_size, flags)) || (rc = set_device(ctx)))
        return rc;
    const float* bias = nullptr;
    if ((rc = adopt_selection_bias(ctx, b, selection_bias, flags, &bias)))
        return rc;
    pbmoe::Q4Rows q{};
    if ((rc = adopt_q4(ctx, weight, b->desc.experts, b->desc.hidden, group_size, flags, b->router_owned,
                       b->router_s_owned, b->router_b_owned, &q))) {
        drop_router(ctx, b);
        return rc;
    }
    b->router_q4 = q;
    b->router = q.codes;
    b->router_dtype = pbmoe::DT_Q4;
    b->sel_bias = bias;
    return ok();
}

PBMOE_API int pbmoe_bind_shared_gate_q4(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_q4_matrix* gate,
                                        uint32_t group_size, uint32_t scale_bias_dtype, uint32_t flags)
{
    if (!ctx || !gate)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    if (!b->has_shared)
        return fail(PBMOE_ERR_NOT_BOUND, "layer %u: bind the shared expert before its Q4 gate", layer);
    if (!b->desc.shared_gated)
        return fail(PBMOE_ERR_SHAPE, "layer %u declares an ungated shared expert", layer);
    if (scale_bias_dtype != b->layout.scale_bias_dtype)
        return fail(PBMOE_ERR_UNSUPPORTED, "Q4 gate scale/bias dtype %u must match the experts' (%u)",
                    scale_bias_dtype, b->layout.scale_bias_dtype);
    if ((rc = check_q4(gate, b->desc.hidden, group_size, flags)) || (rc = set_device(ctx)))
        return rc;
    pbmoe::Q4Rows q{};
    if ((rc = adopt_q4(ctx, gate, 1, b->desc.hidden, group_size, flags, b->gate_owned, b->gate_s_owned,
                       b->gate_b_owned, &q))) {
        drop_gate(ctx, b);
        return rc;
    }
    b->gate_q4 = q;
    b->shared_gate = q.codes;
    b->shared_gate_dtype = pbmoe::DT_Q4;
    return ok();
}

PBMOE_API int pbmoe_bind_shared(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_q4_layout* sl,
                                const void* shared_slot, const void* gate_weight,
                                uint32_t gate_dtype, uint32_t flags)
{
    if (!ctx || !sl || !shared_slot)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    if (b->desc.shared_intermediate == 0)
        return fail(PBMOE_ERR_SHAPE, "layer %u declares no shared expert", layer);
    rc = check_layout(sl, b->desc.hidden, b->desc.shared_intermediate);
    if (rc)
        return rc;
    if (sl->scale_bias_dtype != b->layout.scale_bias_dtype)
        return fail(PBMOE_ERR_UNSUPPORTED, "shared and routed scale/bias dtypes must match");
    if (b->desc.shared_gated && !gate_weight)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "layer declares a gated shared expert but no gate weight");
    if (gate_weight && gate_dtype > PBMOE_DTYPE_BF16)
        return fail(PBMOE_ERR_DTYPE, "shared gate dtype %u not one of F32/F16/BF16", gate_dtype);
    if (flags == PBMOE_MEM_DEVICE && !aligned(shared_slot, 16))
        return fail(PBMOE_ERR_ALIGNMENT, "device shared slot must be 16-byte aligned");
    rc = set_device(ctx);
    if (rc)
        return rc;
    // from here on the old shared expert may be freed: until the bind
    // completes the layer has none (a failure leaves it that way)
    b->has_shared = false;
    const void* dev = nullptr;
    rc = adopt(ctx, shared_slot, sl->expert_bytes, flags, b->shared_owned, &dev);
    if (rc) {
        b->shared_slot = nullptr;
        drop_gate(ctx, b);
        return rc;
    }
    b->shared_layout = *sl;
    b->shared_slot = static_cast<const uint8_t*>(dev);
    drop_gate(ctx, b); // a gate bound before, dense or Q4
    if (b->desc.shared_gated && gate_weight) {
        size_t esz = gate_dtype == PBMOE_DTYPE_F32 ? 4 : 2;
        rc = adopt(ctx, gate_weight, (size_t)b->desc.hidden * esz, flags, b->gate_owned, &dev);
        if (rc)
            return rc;
        b->shared_gate = dev;
        b->shared_gate_dtype = gate_dtype;
    }
    b->has_shared = true;
    return ok();
}

PBMOE_API int pbmoe_unbind_layer(pbmoe_ctx* ctx, uint32_t layer)
{
    if (!ctx)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ctx is null");
    if (ctx->layers.find(layer) == ctx->layers.end())
        return fail(PBMOE_ERR_NOT_BOUND, "layer %u is not bound", layer);
    int rc = set_device(ctx);
    if (rc)
        return rc;
    if ((rc = release_layer(ctx, layer)))
        return rc;
    return ok();
}

static pbmoe::RouteParams route_params(const pbmoe_layer_desc& d)
{
    pbmoe::RouteParams p{};
    p.experts = d.experts;
    p.k = d.active_experts;
    p.kind = d.routing;
    p.order = d.route_order;
    p.norm = d.normalization;
    p.n_group = d.routing == PBMOE_ROUTING_SIGMOID_GROUPED ? d.n_group : 1;
    p.topk_group = d.routing == PBMOE_ROUTING_SIGMOID_GROUPED ? d.topk_group : 1;
    p.routed_scale = d.routed_scale;
    return p;
}

static int route_many(pbmoe_ctx* ctx, LayerBinding* b, const float* logits, uint32_t tokens,
                      uint32_t* ids, float* weights)
{
    if (needs_selection_bias(b->desc.routing) && !b->sel_bias)
        return fail(PBMOE_ERR_NOT_BOUND, "sigmoid routing needs the selection bias (bind_router)");
    HIP_TRY(pbmoe::launch_route_topk(ctx->stream, logits, b->sel_bias, tokens, route_params(b->desc),
                                     ids, weights, ctx->status));
    return ok();
}

// Byte offsets of the decode scratch of `tokens` rows inside one region
// (each piece 256-byte aligned): the layout of the static scratch used by
// pbmoe_moe_layer_noalloc.
struct DecodeScratchLayout {
    size_t logits, act, act_shared, shared_weight, plan, route_ids, route_w, total;
};

static DecodeScratchLayout decode_scratch_layout(const pbmoe_layer_desc& d, uint32_t tokens)
{
    const size_t routes = (size_t)tokens * d.active_experts;
    DecodeScratchLayout l{};
    size_t at = 0;
    auto take = [&at](size_t bytes) {
        const size_t off = at;
        at += (bytes + 255) / 256 * 256;
        return off;
    };
    l.logits = take((size_t)tokens * d.experts * 4);
    l.act = take(routes * d.intermediate * 4);
    l.act_shared = take((size_t)tokens * (d.shared_intermediate + 1) * 4);
    l.shared_weight = take((size_t)tokens * 4);
    l.plan = take(((size_t)d.experts * 3 + 1 + routes * 3 + pbmoe::plan_work_words((uint32_t)routes, d.experts)) * 4);
    l.route_ids = take(routes * 4);
    l.route_w = take(routes * 4);
    l.total = at;
    return l;
}

// Fill the decode launch description for a bound layer.  Scratch: grown in
// the context's own buffers, or carved from `fixed` (the static scratch of
// the allocation-free entry point; its size was checked by the caller).
static int decode_args(pbmoe_ctx* ctx, LayerBinding* b, const float* x, const float* residual,
                       uint32_t tokens, uint32_t* ids, float* weights, const float* next_norm_weight,
                       float* hidden_out, float* next_normed_out, pbmoe::ExpertSet* sh,
                       pbmoe::DecodeArgs* a, uint8_t* fixed = nullptr)
{
    const pbmoe_layer_desc& d = b->desc;
    const uint32_t K = d.active_experts, H = d.hidden, I = d.intermediate;
    const uint32_t routes = tokens * K;
    int rc;
    pbmoe::Plan plan{};
    float *logits, *act, *act_shared, *shared_weight;
    if (fixed) {
        const DecodeScratchLayout l = decode_scratch_layout(d, tokens);
        logits = reinterpret_cast<float*>(fixed + l.logits);
        act = reinterpret_cast<float*>(fixed + l.act);
        act_shared = reinterpret_cast<float*>(fixed + l.act_shared);
        shared_weight = reinterpret_cast<float*>(fixed + l.shared_weight);
        uint32_t* p = reinterpret_cast<uint32_t*>(fixed + l.plan);
        plan.unique_ids = p;
        plan.unique_count = p + d.experts;
        plan.groups = p + d.experts + 1;
        plan.route_slots = p + d.experts * 3 + 1;
        plan.src_rows = plan.route_slots + routes;
        plan.out_idx = plan.src_rows + routes;
        plan.work = plan.out_idx + routes;
    } else {
        if ((rc = ensure(ctx, ctx->logits, (size_t)tokens * d.experts * 4)))
            return rc;
        if ((rc = ensure(ctx, ctx->act, (size_t)routes * I * 4)))
            return rc;
        if ((rc = ensure(ctx, ctx->act_shared, (size_t)tokens * (d.shared_intermediate + 1) * 4)))
            return rc;
        if ((rc = ensure(ctx, ctx->shared_weight, (size_t)tokens * 4)))
            return rc;
        if ((rc = plan_buffers(ctx, d.experts, routes, &plan)))
            return rc;
        logits = static_cast<float*>(ctx->logits.ptr);
        act = static_cast<float*>(ctx->act.ptr);
        act_shared = static_cast<float*>(ctx->act_shared.ptr);
        shared_weight = static_cast<float*>(ctx->shared_weight.ptr);
    }
    *a = pbmoe::DecodeArgs{};
    a->router_w = b->router;
    a->router_dtype = b->router_dtype;
    a->sel_bias = b->sel_bias;
    a->rp = route_params(d);
    a->logits = logits;
    a->ids = ids;
    a->weights = weights;
    a->ex = make_set(b->slots, b->layout, d.experts, H, I);
    a->shared = nullptr;
    if (b->has_shared) {
        *sh = make_set(b->shared_slot, b->shared_layout, 1, H, d.shared_intermediate);
        a->shared = sh;
    }
    a->sgate_w = b->shared_gate;
    a->sgate_dtype = b->shared_gate_dtype;
    a->router_q4 = b->router_q4;
    a->sgate_q4 = b->gate_q4;
    a->x = x;
    a->residual = residual;
    a->tokens = tokens;
    a->hidden = H;
    a->act = act;
    a->act_shared = act_shared;
    a->shared_weight = shared_weight;
    a->hidden_out = hidden_out;
    a->next_norm_w = next_norm_weight;
    a->eps = d.norm_epsilon > 0.0f ? d.norm_epsilon : 1e-6f;
    a->next_normed = next_normed_out;
    a->plan = plan;
    a->ticket = ctx->status + 32;
    a->status = ctx->status;
    a->phase_timing = ctx->phase_timing;
    for (int i = 0; i < 6; ++i)
        a->phase_ev[i] = ctx->phase_ev[i];
    return ok();
}

PBMOE_API int pbmoe_route(pbmoe_ctx* ctx, uint32_t layer, const float* x, uint32_t tokens,
                          uint32_t* ids, float* weights, float* logits_out)
{
    if (!ctx || !x || !ids || !weights)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if (tokens == 0)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "routing requires at least one token row");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    if (!b->router)
        return fail(PBMOE_ERR_NOT_BOUND, "layer %u has no bound router projection", layer);
    if (needs_selection_bias(b->desc.routing) && !b->sel_bias)
        return fail(PBMOE_ERR_NOT_BOUND, "sigmoid routing needs the selection bias (bind_router)");
    if (!aligned(x, 16))
        return fail(PBMOE_ERR_ALIGNMENT, "x must be 16-byte aligned");
    rc = set_device(ctx);
    if (rc)
        return rc;
    if (tokens <= MAX_DECODE_TOKENS) {
        pbmoe::DecodeArgs a;
        pbmoe::ExpertSet sh;
        if ((rc = decode_args(ctx, b, x, nullptr, tokens, ids, weights, nullptr, nullptr, nullptr, &sh, &a)))
            return rc;
        if (logits_out)
            a.logits = logits_out;
        HIP_TRY(pbmoe::launch_decode_layer(ctx->stream, a, pbmoe::DECODE_ROUTE_ONLY));
        return ok();
    }
    float* logits = logits_out;
    if (!logits) {
        rc = ensure(ctx, ctx->logits, (size_t)tokens * b->desc.experts * 4);
        if (rc)
            return rc;
        logits = static_cast<float*>(ctx->logits.ptr);
    }
    HIP_TRY(pbmoe::launch_router_logits(ctx->stream, b->router, b->router_dtype, x, tokens,
                                        b->desc.experts, b->desc.hidden, logits, &b->router_q4,
                                        b->layout.scale_bias_dtype));
    return route_many(ctx, b, logits, tokens, ids, weights);
}

PBMOE_API int pbmoe_route_logits(pbmoe_ctx* ctx, uint32_t layer, const float* logits,
                                 uint32_t tokens, uint32_t* ids, float* weights)
{
    if (!ctx || !logits || !ids || !weights)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if (tokens == 0)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "routing requires at least one token row");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    rc = set_device(ctx);
    if (rc)
        return rc;
    return route_many(ctx, b, logits, tokens, ids, weights);
}

static int expert_phase(pbmoe_ctx* ctx, uint32_t layer, const float* x, const float* residual,
                        uint32_t tokens, uint32_t* ids, float* weights,
                        const float* next_norm_weight, float* hidden_out, float* next_normed_out,
                        uint32_t mode, const float* in_norm_weight = nullptr, bool noalloc = false)
{
    if (!ctx || !x || !residual || !hidden_out || (mode == pbmoe::DECODE_EXPERTS && (!ids || !weights)))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if (tokens == 0)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "expert phase requires at least one token row");
    if ((next_norm_weight == nullptr) != (next_normed_out == nullptr))
        return fail(PBMOE_ERR_INVALID_ARGUMENT,
                    "next_norm_weight and next_normed_out must be given together");
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    const pbmoe_layer_desc& d = b->desc;
    if (d.shared_intermediate && !b->has_shared)
        return fail(PBMOE_ERR_NOT_BOUND, "layer %u declares a shared expert that is not bound",
                    layer);
    if (mode == pbmoe::DECODE_FULL_LAYER) {
        if (!b->router)
            return fail(PBMOE_ERR_NOT_BOUND, "layer %u has no bound router projection", layer);
        if (b->shared_gate && b->shared_gate_dtype != b->router_dtype)
            return fail(PBMOE_ERR_UNSUPPORTED,
                        "the fused layer needs the shared gate and router in one dtype");
        if (needs_selection_bias(d.routing) && !b->sel_bias)
            return fail(PBMOE_ERR_NOT_BOUND, "sigmoid routing needs the selection bias (bind_router)");
    }
    if (tokens > MAX_DECODE_TOKENS)
        return fail(PBMOE_ERR_UNSUPPORTED, "decode expert phase supports at most %u tokens, got %u",
                    MAX_DECODE_TOKENS, tokens);
    for (const void* p : {(const void*)x, (const void*)residual, (const void*)hidden_out,
                          (const void*)in_norm_weight})
        if (!aligned(p, 16))
            return fail(PBMOE_ERR_ALIGNMENT, "activation and norm buffers must be 16-byte aligned");
    rc = set_device(ctx);
    if (rc)
        return rc;
    uint8_t* fixed = nullptr;
    if (noalloc) {
        // every scratch byte from the device's static scratch: no allocation
        size_t cap = 0;
        fixed = static_cast<uint8_t*>(pbmoe::static_scratch(ctx->device, &cap));
        if (!fixed)
            return fail(PBMOE_ERR_DEVICE, "static scratch of device %d was not set up", ctx->device);
        const DecodeScratchLayout l = decode_scratch_layout(d, tokens);
        if (l.total > cap)
            return fail(PBMOE_ERR_UNSUPPORTED,
                        "allocation-free layer: %u tokens of this layer need %zu scratch bytes, the static "
                        "scratch holds %zu", tokens, l.total, cap);
        if (mode == pbmoe::DECODE_FULL_LAYER && (!ids || !weights)) {
            ids = reinterpret_cast<uint32_t*>(fixed + l.route_ids);
            weights = reinterpret_cast<float*>(fixed + l.route_w);
        }
    }
    if (in_norm_weight && (rc = ensure(ctx, ctx->x_normed, (size_t)tokens * d.hidden * 4)))
        return rc;
    if (mode == pbmoe::DECODE_FULL_LAYER && (!ids || !weights)) {
        if ((rc = ensure(ctx, ctx->route_ids, (size_t)tokens * d.active_experts * 4)))
            return rc;
        if ((rc = ensure(ctx, ctx->route_w, (size_t)tokens * d.active_experts * 4)))
            return rc;
        ids = static_cast<uint32_t*>(ctx->route_ids.ptr);
        weights = static_cast<float*>(ctx->route_w.ptr);
    }
    pbmoe::DecodeArgs a;
    pbmoe::ExpertSet sh;
    if ((rc = decode_args(ctx, b, x, residual, tokens, ids, weights, next_norm_weight, hidden_out,
                          next_normed_out, &sh, &a, fixed)))
        return rc;
    if (in_norm_weight) {
        a.in_norm_w = in_norm_weight;
        a.x_normed = static_cast<float*>(ctx->x_normed.ptr);
    }
    HIP_TRY(pbmoe::launch_decode_layer(ctx->stream, a, mode));
    return ok();
}

PBMOE_API int pbmoe_moe_decode(pbmoe_ctx* ctx, uint32_t layer, const float* x,
                               const float* residual, uint32_t tokens, const uint32_t* ids,
                               const float* weights, const float* next_norm_weight,
                               float* hidden_out, float* next_normed_out)
{
    return expert_phase(ctx, layer, x, residual, tokens, const_cast<uint32_t*>(ids),
                        const_cast<float*>(weights), next_norm_weight, hidden_out, next_normed_out,
                        pbmoe::DECODE_EXPERTS);
}

// Router + routing + expert phase of one layer in one call (CMD2 routing
// followed by CMD3, metal/mod.rs:2864-3036 then :3252-3332).  ids/weights
// receive the routes when not NULL.
PBMOE_API int pbmoe_moe_layer(pbmoe_ctx* ctx, uint32_t layer, const float* x,
                              const float* residual, uint32_t tokens, uint32_t* ids_out,
                              float* weights_out, const float* next_norm_weight, float* hidden_out,
                              float* next_normed_out)
{
    if ((ids_out == nullptr) != (weights_out == nullptr))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ids_out and weights_out must be given together");
    return expert_phase(ctx, layer, x, residual, tokens, ids_out, weights_out, next_norm_weight,
                        hidden_out, next_normed_out, pbmoe::DECODE_FULL_LAYER);
}

// pbmoe_moe_layer with every scratch buffer in the device's static scratch
// (no allocation; see include/pbmoe.h).
PBMOE_API int pbmoe_moe_layer_noalloc(pbmoe_ctx* ctx, uint32_t layer, const float* x,
                                      const float* residual, uint32_t tokens, uint32_t* ids_out,
                                      float* weights_out, const float* next_norm_weight,
                                      float* hidden_out, float* next_normed_out)
{
    if ((ids_out == nullptr) != (weights_out == nullptr))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ids_out and weights_out must be given together");
    return expert_phase(ctx, layer, x, residual, tokens, ids_out, weights_out, next_norm_weight,
                        hidden_out, next_normed_out, pbmoe::DECODE_FULL_LAYER, nullptr, true);
}

// The same layer taking the un-normalised hidden state: the input RMSNorm
// (the post-attention norm, rms_norm_with_weight_and_epsilon,
// math.rs:151-167, as CMD2 fuses it after out_proj + residual,
// metal/mod.rs:2864-2917) runs inside the router stage, and `hidden` is also
// the residual.  Saves the separate norm launch of a decode step.
PBMOE_API int pbmoe_moe_layer_norm(pbmoe_ctx* ctx, uint32_t layer, const float* hidden,
                                   const float* norm_weight, uint32_t tokens, uint32_t* ids_out,
                                   float* weights_out, const float* next_norm_weight,
                                   float* hidden_out, float* next_normed_out)
{
    if (!norm_weight)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if ((ids_out == nullptr) != (weights_out == nullptr))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ids_out and weights_out must be given together");
    if (hidden && hidden == hidden_out)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "hidden_out must not alias hidden");
    return expert_phase(ctx, layer, hidden, hidden, tokens, ids_out, weights_out, next_norm_weight,
                        hidden_out, next_normed_out, pbmoe::DECODE_FULL_LAYER, norm_weight);
}

static size_t align256(size_t v)
{
    return (v + 255) & ~(size_t)255;
}

// Layer-major prefill (qwen_layer_major_experts, runtime/mod.rs:1151-1161;
// metal/mod.rs:3583-4106).  Up to 16 tokens run through the decode kernels
// (the same arithmetic as pbmoe_moe_decode); larger chunks run the grouped
// GEMM on the matrix cores.
PBMOE_API int pbmoe_moe_prefill(pbmoe_ctx* ctx, uint32_t layer, const float* x,
                                const float* residual, uint32_t tokens, const uint32_t* ids,
                                const float* weights, const float* next_norm_weight,
                                float* hidden_out, float* next_normed_out)
{
    if (tokens <= MAX_DECODE_TOKENS)
        return expert_phase(ctx, layer, x, residual, tokens, const_cast<uint32_t*>(ids),
                            const_cast<float*>(weights), next_norm_weight, hidden_out,
                            next_normed_out, pbmoe::DECODE_EXPERTS);
    if (!ctx || !x || !residual || !hidden_out || !ids || !weights)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if ((next_norm_weight == nullptr) != (next_normed_out == nullptr))
        return fail(PBMOE_ERR_INVALID_ARGUMENT,
                    "next_norm_weight and next_normed_out must be given together");
    if (tokens > MAX_PREFILL_TOKENS)
        return fail(PBMOE_ERR_UNSUPPORTED, "prefill chunk of %u tokens exceeds %u", tokens,
                    MAX_PREFILL_TOKENS);
    LayerBinding* b;
    int rc = get_layer(ctx, layer, &b);
    if (rc)
        return rc;
    const pbmoe_layer_desc& d = b->desc;
    if (d.shared_intermediate && !b->has_shared)
        return fail(PBMOE_ERR_NOT_BOUND, "layer %u declares a shared expert that is not bound",
                    layer);
    if (b->has_shared && b->shared_layout.group_size != b->layout.group_size)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "prefill needs the shared expert in the routed experts' group size");
    if (b->has_shared && b->shared_layout.scale_bias_dtype != b->layout.scale_bias_dtype)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "prefill needs the shared expert in the routed experts' scale/bias dtype");
    for (const void* p : {(const void*)x, (const void*)residual, (const void*)hidden_out,
                          (const void*)next_norm_weight, (const void*)next_normed_out})
        if (p && !aligned(p, 16))
            return fail(PBMOE_ERR_ALIGNMENT, "activation buffers must be 16-byte aligned");
    if ((rc = set_device(ctx)))
        return rc;
    const uint32_t K = d.active_experts, H = d.hidden, I = d.intermediate;
    const size_t T = tokens, routes = T * K, rows = routes + T;
    pbmoe::Plan plan{};
    if ((rc = plan_buffers(ctx, d.experts, (uint32_t)routes, &plan)))
        return rc;
    const uint32_t max_tiles = pbmoe::prefill_max_tiles(tokens, K, d.experts, b->has_shared);
    // scratch layout, each part 256-byte aligned; the tile table holds a
    // multiple of 8 records (the GEMM workgroups read their record before
    // checking it against the tile count, and the grid covers max_tiles
    // rounded up to 8)
    size_t off[14], total = 0;
    const size_t part[14] = {
        (size_t)((max_tiles + 7) / 8 * 8) * 32, 4,     T * H * 2, T * H * 2, T * (H / 32) * 4, rows * 4, T * 4,
        rows * I * 2,          rows * I * 2, rows * (I / 32) * 4, rows * H * 4, rows * 4,
        T * ((H / 64 + 15) / 16 * 16) * 4, rows * ((I / 64 + 15) / 16 * 16) * 4};
    for (int i = 0; i < 14; ++i) {
        off[i] = total;
        total += align256(part[i]);
    }
    if ((rc = ensure(ctx, ctx->prefill, total)))
        return rc;
    uint8_t* base = static_cast<uint8_t*>(ctx->prefill.ptr);
    pbmoe::ExpertSet sh;
    pbmoe::PrefillArgs a{};
    a.ex = make_set(b->slots, b->layout, d.experts, H, I);
    a.shared = nullptr;
    if (b->has_shared) {
        sh = make_set(b->shared_slot, b->shared_layout, 1, H, d.shared_intermediate);
        a.shared = &sh;
    }
    a.sgate_w = b->has_shared ? b->shared_gate : nullptr;
    a.sgate_dtype = b->shared_gate_dtype;
    a.sgate_q4 = b->gate_q4;
    a.ids = ids;
    a.weights = weights;
    a.x = x;
    a.residual = residual;
    a.tokens = tokens;
    a.k = K;
    a.hidden = H;
    a.hidden_out = hidden_out;
    a.next_norm_w = next_norm_weight;
    a.eps = d.norm_epsilon > 0.0f ? d.norm_epsilon : 1e-6f;
    a.next_normed = next_normed_out;
    a.plan = plan;
    a.tiles = reinterpret_cast<uint32_t*>(base + off[0]);
    a.tile_count = reinterpret_cast<uint32_t*>(base + off[1]);
    a.x_hi = reinterpret_cast<uint16_t*>(base + off[2]);
    a.x_lo = reinterpret_cast<uint16_t*>(base + off[3]);
    a.x_sum32 = reinterpret_cast<float*>(base + off[4]);
    a.rowscale = reinterpret_cast<float*>(base + off[5]);
    a.shared_logit = reinterpret_cast<float*>(base + off[6]);
    a.act_hi = reinterpret_cast<uint16_t*>(base + off[7]);
    a.act_lo = reinterpret_cast<uint16_t*>(base + off[8]);
    a.act_sum32 = reinterpret_cast<float*>(base + off[9]);
    a.y = reinterpret_cast<float*>(base + off[10]);
    a.x_lo_any = reinterpret_cast<uint32_t*>(base + off[11]);
    a.x_sumhl = reinterpret_cast<uint16_t*>(base + off[12]);
    a.act_sumhl = reinterpret_cast<uint16_t*>(base + off[13]);
    a.status = ctx->status;
    a.phase_timing = ctx->phase_timing;
    for (int i = 0; i < 6; ++i)
        a.phase_ev[i] = ctx->phase_ev[i];
    HIP_TRY(pbmoe::launch_prefill(ctx->stream, a));
    return ok();
}

PBMOE_API int pbmoe_dispatch_plan(pbmoe_ctx* ctx, uint32_t experts, uint32_t active_experts,
                                  uint32_t tokens, const uint32_t* ids, uint32_t* unique_ids,
                                  uint32_t* unique_count, uint32_t* route_slots,
                                  uint32_t* grouped_source_rows, uint32_t* grouped_output_indices,
                                  uint32_t* groups)
{
    if (!ctx || !ids || !unique_ids || !unique_count || !route_slots || !grouped_source_rows ||
        !grouped_output_indices || !groups)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if (tokens == 0 || experts == 0 || active_experts == 0)
        return fail(PBMOE_ERR_INVALID_ARGUMENT,
                    "layer-major group plan requires non-empty routes and experts");
    if (experts > MAX_EXPERTS)
        return fail(PBMOE_ERR_UNSUPPORTED, "experts=%u > %u", experts, MAX_EXPERTS);
    int rc = set_device(ctx);
    if (rc)
        return rc;
    pbmoe::Plan p;
    p.unique_ids = unique_ids;
    p.unique_count = unique_count;
    p.route_slots = route_slots;
    p.src_rows = grouped_source_rows;
    p.out_idx = grouped_output_indices;
    p.groups = groups;
    const uint32_t routes = tokens * active_experts;
    if ((rc = ensure(ctx, ctx->plan_work, (size_t)pbmoe::plan_work_words(routes, experts) * 4)))
        return rc;
    p.work = static_cast<uint32_t*>(ctx->plan_work.ptr);
    HIP_TRY(pbmoe::launch_dispatch_plan(ctx->stream, ids, routes, experts,
                                        active_experts, p, ctx->status));
    return ok();
}

PBMOE_API int pbmoe_q4_dequantize(pbmoe_ctx* ctx, const void* packed, const void* scales,
                                  const void* biases, uint32_t sb_dtype, uint32_t rows,
                                  uint32_t cols, uint32_t group_size, float* out)
{
    if (!ctx || !packed || !scales || !biases || !out)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if (rows == 0 || cols == 0 || group_size == 0)
        return fail(PBMOE_ERR_SHAPE, "dequantisation needs non-zero rows, cols and group size");
    if (cols % 8 || cols % group_size || group_size % 8)
        return fail(PBMOE_ERR_UNSUPPORTED,
                    "device dequantisation needs cols and group size divisible by 8 and cols by group");
    if (sb_dtype != PBMOE_DTYPE_F16 && sb_dtype != PBMOE_DTYPE_BF16)
        return fail(PBMOE_ERR_DTYPE, "scale/bias dtype must be F16 or BF16");
    if (!aligned(packed, 4) || !aligned(scales, 2) || !aligned(biases, 2))
        return fail(PBMOE_ERR_ALIGNMENT, "packed must be 4-byte, scale/bias 2-byte aligned");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    HIP_TRY(pbmoe::launch_q4_dequantize(ctx->stream, static_cast<const uint8_t*>(packed), scales,
                                        biases, sb_dtype, rows, cols, group_size, out));
    return ok();
}

PBMOE_API int pbmoe_synth_fill_q4(pbmoe_ctx* ctx, void* slots_device,
                                  const pbmoe_q4_layout* layout, uint32_t hidden,
                                  uint32_t intermediate, uint64_t seed, uint32_t tensor,
                                  uint32_t layer, uint32_t first_expert, uint32_t count)
{
    if (!ctx || !slots_device || !layout)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_layout(layout, hidden, intermediate);
    if (rc)
        return rc;
    rc = set_device(ctx);
    if (rc)
        return rc;
    uint64_t off[9];
    for (int i = 0; i < 9; ++i)
        off[i] = layout->components[i].offset;
    HIP_TRY(pbmoe::launch_synth_fill(ctx->stream, static_cast<uint8_t*>(slots_device),
                                     layout->expert_bytes, off, hidden, intermediate,
                                     layout->group_size, layout->scale_bias_dtype, seed, tensor,
                                     layer, first_expert, count));
    return ok();
}

PBMOE_API int pbmoe_synth_center_q4(pbmoe_ctx* ctx, void* slots_device, const pbmoe_q4_layout* layout,
                                    uint32_t hidden, uint32_t intermediate, uint32_t count)
{
    if (!ctx || !slots_device || !layout)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_layout(layout, hidden, intermediate);
    if (rc)
        return rc;
    if ((rc = set_device(ctx)))
        return rc;
    uint64_t off[9];
    for (int i = 0; i < 9; ++i)
        off[i] = layout->components[i].offset;
    HIP_TRY(pbmoe::launch_synth_center(ctx->stream, static_cast<uint8_t*>(slots_device), layout->expert_bytes,
                                       off, hidden, intermediate, layout->group_size,
                                       layout->scale_bias_dtype, count));
    return ok();
}

// ---- GQA decode attention --------------------------------------------------

namespace {

constexpr uint32_t ATTN_HEAD_DIM = 128;

int attn_matrix(const pbmoe_q4_matrix& m, uint32_t rows, uint32_t cols, const char* name,
                pbmoe::Q4Mat* out)
{
    if (!m.codes || !m.scales || !m.biases)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "attention %s projection has a null component", name);
    if (!aligned(m.codes, 16) || !aligned(m.scales, 2) || !aligned(m.biases, 2))
        return fail(PBMOE_ERR_ALIGNMENT,
                    "attention %s projection: codes must be 16-byte and scales/biases 2-byte aligned", name);
    out->codes = static_cast<const uint8_t*>(m.codes);
    out->scales = static_cast<const uint8_t*>(m.scales);
    out->biases = static_cast<const uint8_t*>(m.biases);
    out->rows = rows;
    out->cols = cols;
    return ok();
}

} // namespace

// full_attention_output_values (runtime/mod.rs:2215-2367) state of one
// layer: FullAttentionLayout shape checks (the kernels' limits explicitly
// rejected), the KV cache of the layer (KvCache, state/kv_cache.rs) and the
// rotary table of split_half_rope_rotations (math.rs:303-325).
PBMOE_API int pbmoe_bind_attention(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_attn_desc* desc,
                                   const pbmoe_attn_weights* w)
{
    if (!ctx || !desc || !w)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    const pbmoe_attn_desc d = *desc;
    if (d.head_dim != ATTN_HEAD_DIM || d.rotary_dim != d.head_dim)
        return fail(PBMOE_ERR_UNSUPPORTED, "attention head_dim=%u rotary_dim=%u: head_dim 128 with full "
                    "split-half rotary is implemented", d.head_dim, d.rotary_dim);
    if (d.kv_heads == 0 || d.q_heads == 0 || d.q_heads % d.kv_heads)
        return fail(PBMOE_ERR_SHAPE, "q_heads=%u must be a non-zero multiple of kv_heads=%u", d.q_heads,
                    d.kv_heads);
    const uint32_t nq = d.q_heads / d.kv_heads;
    if (nq != 1 && nq != 2 && nq != 4 && nq != 8)
        return fail(PBMOE_ERR_UNSUPPORTED, "%u q heads per kv head (1, 2, 4 or 8 implemented)", nq);
    const uint32_t qw = d.q_heads * d.head_dim, kvw = d.kv_heads * d.head_dim;
    if (d.hidden == 0 || d.hidden > MAX_HIDDEN || qw > MAX_HIDDEN)
        return fail(PBMOE_ERR_UNSUPPORTED, "attention hidden=%u, q width=%u (at most %u)", d.hidden, qw,
                    MAX_HIDDEN);
    if (d.group_size != 32 && d.group_size != 64 && d.group_size != 128)
        return fail(PBMOE_ERR_UNSUPPORTED, "attention group size %u (32, 64 or 128)", d.group_size);
    if (d.hidden % d.group_size || qw % d.group_size || d.hidden % 2)
        return fail(PBMOE_ERR_SHAPE, "hidden=%u and q width=%u must be multiples of group %u", d.hidden, qw,
                    d.group_size);
    if (d.scale_bias_dtype != PBMOE_DTYPE_F16 && d.scale_bias_dtype != PBMOE_DTYPE_BF16)
        return fail(PBMOE_ERR_DTYPE, "attention scale/bias dtype must be F16 or BF16");
    if (d.max_context == 0 || !(d.rope_theta > 0.0f))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "max_context and rope_theta must be positive");
    if (d.max_context > 65536)
        return fail(PBMOE_ERR_UNSUPPORTED, "max_context %u (at most 65536 positions)", d.max_context);
    if (!w->q_norm || !w->k_norm)
        return fail(PBMOE_ERR_NOT_BOUND, "attention layer %u: self_attn.q_norm / k_norm are required", layer);
    int rc;
    pbmoe::AttnArgs a{};
    if ((rc = attn_matrix(w->q, qw, d.hidden, "q", &a.q)) || (rc = attn_matrix(w->k, kvw, d.hidden, "k", &a.k)) ||
        (rc = attn_matrix(w->v, kvw, d.hidden, "v", &a.v)) || (rc = attn_matrix(w->o, d.hidden, qw, "o", &a.o)))
        return rc;
    if ((rc = set_device(ctx)))
        return rc;
    if (ctx->attn.count(layer))
        if ((rc = pbmoe_unbind_attention(ctx, layer)))
            return rc;
    AttnBinding b;
    b.desc = d;
    const size_t cache_bytes = (size_t)d.max_context * kvw * 2;
    HIP_TRY(hipMalloc(&b.cache_k.ptr, cache_bytes));
    b.cache_k.bytes = cache_bytes;
    hipError_t e = hipMalloc(&b.cache_v.ptr, cache_bytes);
    if (e == hipSuccess)
        b.cache_v.bytes = cache_bytes;
    if (e == hipSuccess)
        e = hipMalloc(&b.inv_freq.ptr, 256 * sizeof(float));
    if (e == hipSuccess) {
        b.inv_freq.bytes = 256 * sizeof(float);
        // theta.powf(-(2 i) / rotary_dim) in f32, as the reference computes it
        float inv[256] = {};
        const uint32_t half = d.rotary_dim / 2;
        for (uint32_t i = 0; i < half; ++i)
            inv[i] = powf(d.rope_theta, -((float)(2 * i)) / (float)d.rotary_dim);
        e = hipMemcpyAsync(b.inv_freq.ptr, inv, sizeof inv, hipMemcpyHostToDevice, ctx->stream);
    }
    if (e == hipSuccess)
        e = hipMemsetAsync(b.cache_k.ptr, 0, cache_bytes, ctx->stream);
    if (e == hipSuccess)
        e = hipMemsetAsync(b.cache_v.ptr, 0, cache_bytes, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        free_buf(b.cache_k);
        free_buf(b.cache_v);
        free_buf(b.inv_freq);
        return fail(e == hipErrorOutOfMemory ? PBMOE_ERR_OUT_OF_MEMORY : PBMOE_ERR_DEVICE,
                    "attention layer %u setup: %s", layer, hipGetErrorString(e));
    }
    a.q_norm = w->q_norm;
    a.k_norm = w->k_norm;
    a.group_shift = 0;
    while ((1u << a.group_shift) < d.group_size)
        ++a.group_shift;
    a.sb_dtype = d.scale_bias_dtype;
    a.hidden = d.hidden;
    a.q_heads = d.q_heads;
    a.kv_heads = d.kv_heads;
    a.head_dim = d.head_dim;
    a.inv_freq = static_cast<const float*>(b.inv_freq.ptr);
    a.cache_k = static_cast<uint16_t*>(b.cache_k.ptr);
    a.cache_v = static_cast<uint16_t*>(b.cache_v.ptr);
    a.post_eps = d.norm_epsilon > 0.0f ? d.norm_epsilon : 1e-6f;
    b.base = a;
    ctx->attn[layer] = b;
    return ok();
}

PBMOE_API int pbmoe_unbind_attention(pbmoe_ctx* ctx, uint32_t layer)
{
    if (!ctx)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "ctx is null");
    auto it = ctx->attn.find(layer);
    if (it == ctx->attn.end())
        return fail(PBMOE_ERR_NOT_BOUND, "attention layer %u is not bound", layer);
    int rc = set_device(ctx);
    if (rc)
        return rc;
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    free_buf(it->second.cache_k);
    free_buf(it->second.cache_v);
    free_buf(it->second.inv_freq);
    ctx->attn.erase(it);
    return ok();
}

PBMOE_API int pbmoe_attention_kv_cache(pbmoe_ctx* ctx, uint32_t layer, void** keys, void** values)
{
    if (!ctx || !keys || !values)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    auto it = ctx->attn.find(layer);
    if (it == ctx->attn.end())
        return fail(PBMOE_ERR_NOT_BOUND, "attention layer %u is not bound", layer);
    *keys = it->second.cache_k.ptr;
    *values = it->second.cache_v.ptr;
    return ok();
}

PBMOE_API int pbmoe_attention_decode(pbmoe_ctx* ctx, uint32_t layer, const float* normed,
                                     const float* input_norm_weight, const float* residual,
                                     uint32_t position, float* hidden_out,
                                     const float* post_norm_weight, float* post_normed_out,
                                     float* attn_out)
{
    if (!ctx || !normed || !residual || !hidden_out)
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "null argument");
    if ((post_norm_weight == nullptr) != (post_normed_out == nullptr))
        return fail(PBMOE_ERR_INVALID_ARGUMENT, "post_norm_weight and post_normed_out go together");
    auto it = ctx->attn.find(layer);
    if (it == ctx->attn.end())
        return fail(PBMOE_ERR_NOT_BOUND, "attention layer %u is not bound", layer);
    const AttnBinding& b = it->second;
    if (position >= b.desc.max_context)
        return fail(PBMOE_ERR_SHAPE, "position %u beyond the KV cache (%u positions)", position,
                    b.desc.max_context);
    for (const void* p : {(const void*)normed, (const void*)input_norm_weight, (const void*)residual,
                          (const void*)hidden_out, (const void*)post_normed_out, (const void*)attn_out})
        if (p && !aligned(p, 16))
            return fail(PBMOE_ERR_ALIGNMENT, "activation buffers must be 16-byte aligned");
    int rc = set_device(ctx);
    if (rc)
        return rc;
    const uint32_t qw = b.desc.q_heads * b.desc.head_dim, kvw = b.desc.kv_heads * b.desc.head_dim;
    // partials sized for the whole cache, so the scratch does not grow with
    // the position (one allocation before a decode loop or graph capture)
    const uint32_t chunks = (b.desc.max_context + pbmoe::ATTN_CHUNK - 1) / pbmoe::ATTN_CHUNK;
    const size_t qkv_bytes = align256((size_t)(qw + 2 * kvw) * 4);
    const size_t part_bytes = align256((size_t)b.desc.q_heads * chunks * (b.desc.head_dim + 2) * 4);
    const size_t out_bytes = align256((size_t)qw * 4);
    if ((rc = ensure(ctx, ctx->attn_scratch, qkv_bytes + part_bytes + out_bytes)))
        return rc;
    uint8_t* base = static_cast<uint8_t*>(ctx->attn_scratch.ptr);
    pbmoe::AttnArgs a = b.base;
    a.position = position;
    a.normed = normed;
    a.in_norm_w = input_norm_weight;
    a.residual = residual;
    a.hidden_out = hidden_out;
    a.post_norm_w = post_norm_weight;
    a.post_normed = post_normed_out;
    a.qkv = reinterpret_cast<float*>(base);
    a.part = reinterpret_cast<float*>(base + qkv_bytes);
    a.attn_out = attn_out ? attn_out : reinterpret_cast<float*>(base + qkv_bytes + part_bytes);
    for (int i = 0; i < 8; ++i)
        a.ev[i] = ctx->phase_timing ? ctx->attn_ev[i] : nullptr;
    HIP_TRY(pbmoe::launch_attention_decode(ctx->stream, a));
    return ok();
}

