// gfx950 (MI355X) kernels for the FlashMoE MoE block.
//
// Wave64 throughout.  Weights are streamed from HBM once per call with
// 16-byte loads (32 nibbles per lane); activations stay in registers, LDS or
// L2.  Every kernel bounds-checks route ids against the expert count and
// reports problems through a device status word instead of reading out of
// range.
//
// Reference kernels these replace (src/inference/flashmoe/metal/qwen/
// shaders.metal of Jc2k/pb): dense_mmap_fma_matvec_* (router, :1059-1111),
// q4_fma_matvec_bf16_scale_bias (:97-199), silu_product (:1699-1708),
// shared_expert_activation (:1710-1721), qwen_layer_major_combine
// (:1756-1786), rms_norm_reduced (:1176-1213); the CPU routing stage
// math.rs:746-819 and scheduler/expert_access.rs:80-135; the group plan
// metal/mod.rs:3197-3233.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "pbmoe_internal.h"
#include "pbmoe_synth.h"

namespace pbmoe {

constexpr int WAVE = 64;

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
template <int SBT>
__device__ __forceinline__ float sb_at(const uint8_t* base, uint64_t i)
{
    uint16_t v = reinterpret_cast<const uint16_t*>(base)[i];
    if constexpr (SBT == 2)
        return __uint_as_float((uint32_t)v << 16);
    else
        return __half2float(__ushort_as_half(v));
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1)
        v += __shfl_xor(v, o);
    return v;
}

template <int W>
__device__ __forceinline__ float group_sum(float v)
{
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1)
        v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v)
{
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) {
        uint32_t lo = __shfl_xor((uint32_t)v, o);
        uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o);
        uint64_t w = ((uint64_t)hi << 32) | lo;
        v = w > v ? w : v;
    }
    return v;
}

// f32 total order (Rust f32::total_cmp) mapped onto unsigned order.
__device__ __forceinline__ uint32_t total_key(float f)
{
    uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float sigmoidf_(float l) { return 1.0f / (1.0f + expf(-l)); }

// Dot of one 16-byte chunk (32 nibbles, columns col0..col0+31) with x.
// Returns sum(q*x); xs receives sum(x).  Factored affine form:
// row = sum_g s_g * sum(q*x) + b_g * sum(x).
__device__ __forceinline__ float q4_chunk_qx(uint4 w, const float* __restrict__ x, float& xs)
{
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float qx = 0.0f, sx = 0.0f;
    uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float4 a = x4[2 * i];
        float4 b = x4[2 * i + 1];
        uint32_t q = words[i];
        qx = fmaf((float)(q & 15u), a.x, qx);
        qx = fmaf((float)((q >> 4) & 15u), a.y, qx);
        qx = fmaf((float)((q >> 8) & 15u), a.z, qx);
        qx = fmaf((float)((q >> 12) & 15u), a.w, qx);
        qx = fmaf((float)((q >> 16) & 15u), b.x, qx);
        qx = fmaf((float)((q >> 20) & 15u), b.y, qx);
        qx = fmaf((float)((q >> 24) & 15u), b.z, qx);
        qx = fmaf((float)(q >> 28), b.w, qx);
        sx += (a.x + a.y) + (a.z + a.w) + ((b.x + b.y) + (b.z + b.w));
    }
    xs = sx;
    return qx;
}

// ---------------------------------------------------------------------------
// router logits: one wave per expert row, all tokens (tokens <= 16)
// l[t][e] = sum_c W[e][c] * x[t][c]
// ---------------------------------------------------------------------------
template <int WDT, int TT>
__global__ __launch_bounds__(256) void router_logits_kernel(const void* __restrict__ w,
                                                            const float* __restrict__ x,
                                                            uint32_t tokens, uint32_t experts,
                                                            uint32_t hidden,
                                                            float* __restrict__ logits)
{
    const int lane = threadIdx.x & 63;
    const uint32_t e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= experts)
        return;
    for (uint32_t t0 = 0; t0 < tokens; t0 += TT) {
        float acc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t)
            acc[t] = 0.0f;
        for (uint32_t c = lane * 8; c < hidden; c += WAVE * 8) {
            float wv[8];
            if constexpr (WDT == 0) {
                const float4* p = reinterpret_cast<const float4*>(
                    reinterpret_cast<const float*>(w) + (uint64_t)e * hidden + c);
                float4 a = p[0], b = p[1];
                wv[0] = a.x, wv[1] = a.y, wv[2] = a.z, wv[3] = a.w;
                wv[4] = b.x, wv[5] = b.y, wv[6] = b.z, wv[7] = b.w;
            } else {
                uint4 raw = *reinterpret_cast<const uint4*>(
                    reinterpret_cast<const uint16_t*>(w) + (uint64_t)e * hidden + c);
                uint32_t r[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (WDT == 2) {
                        wv[2 * i] = __uint_as_float(r[i] << 16);
                        wv[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
                    } else {
                        wv[2 * i] = __half2float(__ushort_as_half((uint16_t)(r[i] & 0xFFFFu)));
                        wv[2 * i + 1] = __half2float(__ushort_as_half((uint16_t)(r[i] >> 16)));
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                if (t0 + t < tokens) {
                    const float4* xp =
                        reinterpret_cast<const float4*>(x + (uint64_t)(t0 + t) * hidden + c);
                    float4 a = xp[0], b = xp[1];
                    float s = acc[t];
                    s = fmaf(wv[0], a.x, s);
                    s = fmaf(wv[1], a.y, s);
                    s = fmaf(wv[2], a.z, s);
                    s = fmaf(wv[3], a.w, s);
                    s = fmaf(wv[4], b.x, s);
                    s = fmaf(wv[5], b.y, s);
                    s = fmaf(wv[6], b.z, s);
                    s = fmaf(wv[7], b.w, s);
                    acc[t] = s;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            float v = wave_sum(acc[t]);
            if (lane == 0 && t0 + t < tokens)
                logits[(uint64_t)(t0 + t) * experts + e] = v;
        }
    }
}

hipError_t launch_router_logits(hipStream_t s, const void* w, uint32_t w_dtype, const float* x,
                                uint32_t tokens, uint32_t experts, uint32_t hidden, float* logits)
{
    dim3 grid((experts + 3) / 4), block(256);
    switch (w_dtype) {
    case 0:
        router_logits_kernel<0, 4><<<grid, block, 0, s>>>(w, x, tokens, experts, hidden, logits);
        break;
    case 2:
        router_logits_kernel<2, 4><<<grid, block, 0, s>>>(w, x, tokens, experts, hidden, logits);
        break;
    default:
        router_logits_kernel<1, 4><<<grid, block, 0, s>>>(w, x, tokens, experts, hidden, logits);
        break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// routing: one wave per token.  Selection (canonical: score desc / index asc,
// or the reference replacement-slot scan), softmax or sigmoid weights, and
// renormalisation — math.rs:746-819, expert_access.rs:80-135.
// ---------------------------------------------------------------------------
constexpr int MAX_K = 16;

template <int EPL>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias,
                                                         uint32_t tokens, RouteParams p,
                                                         uint32_t* __restrict__ ids,
                                                         float* __restrict__ weights,
                                                         uint32_t* __restrict__ status)
{
    __shared__ float group_buf[4][EPL * WAVE];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 4 + wv;
    if (t >= tokens)
        return;
    const uint32_t E = p.experts, K = p.k;
    const float* l = logits + (uint64_t)t * E;

    float raw[EPL], sel[EPL];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        uint32_t e = lane + WAVE * j;
        raw[j] = e < E ? l[e] : 0.0f;
        if (e < E && !isfinite(raw[j]))
            bad = true;
    }
    if (__ballot(bad) != 0ull && lane == 0)
        atomicOr(status, ST_NONFINITE);

    float mx = 0.0f, inv_sum = 0.0f;
    bool have_inv = false;
    if (p.kind == 0) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            if (lane + WAVE * j < E)
                m = fmaxf(m, raw[j]);
        mx = wave_max(m);
        float sm = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            if (lane + WAVE * j < E)
                sm += expf(raw[j] - mx);
        float sum = wave_sum(sm);
        have_inv = sum > 0.0f && isfinite(sum);
        inv_sum = have_inv ? 1.0f / sum : 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            sel[j] = raw[j];
    } else {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            uint32_t e = lane + WAVE * j;
            sel[j] = e < E ? sigmoidf_(raw[j]) + bias[e] : 0.0f;
        }
    }

    // group-limited selection mask (DeepSeek-V3 noaux_tc)
    uint64_t group_keep = ~0ull;
    uint32_t per = E / (p.n_group ? p.n_group : 1);
    if (p.kind == 2 && p.n_group > 1) {
        float* buf = group_buf[wv];
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            if (lane + WAVE * j < E)
                buf[lane + WAVE * j] = sel[j];
        // the buffer is private to this wave: a wave-scope fence orders the
        // LDS stores before the reads below
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        // lane g scores group g: sum of the two largest biased scores
        uint64_t gkey = 0;
        if ((uint32_t)lane < p.n_group) {
            float a = -INFINITY, b = -INFINITY;
            uint32_t ka = 0, kb = 0;
            for (uint32_t i = 0; i < per; ++i) {
                float v = buf[lane * per + i];
                uint32_t kv = total_key(v);
                if (kv > ka) {
                    kb = ka, b = a;
                    ka = kv, a = v;
                } else if (kv > kb) {
                    kb = kv, b = v;
                }
            }
            float gs = per >= 2 ? a + b : a;
            gkey = ((uint64_t)total_key(gs) << 32) | (0xFFFFFFFFu - (uint32_t)lane);
        }
        group_keep = 0ull;
        for (uint32_t r = 0; r < p.topk_group; ++r) {
            uint64_t best = wave_max_u64(gkey);
            uint32_t g = 0xFFFFFFFFu - (uint32_t)best;
            group_keep |= 1ull << g;
            if ((uint32_t)lane == g)
                gkey = 0;
        }
    }

    // per-lane candidate keys
    uint64_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        uint32_t e = lane + WAVE * j;
        bool ok = e < E && ((group_keep >> (e / (per ? per : 1))) & 1ull);
        key[j] = ok ? (((uint64_t)total_key(sel[j]) << 32) | (0xFFFFFFFFu - e)) : 0ull;
    }

    uint32_t out_e[MAX_K];
    float out_v[MAX_K]; // raw logit (softmax) or unbiased sigmoid
    if (p.order == 0) {
        for (uint32_t r = 0; r < K; ++r) {
            uint64_t mine = 0;
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                mine = key[j] > mine ? key[j] : mine;
            uint64_t best = wave_max_u64(mine);
            uint32_t e = 0xFFFFFFFFu - (uint32_t)best;
            out_e[r] = e;
#pragma unroll
            for (int j = 0; j < EPL; ++j)
                if (key[j] == best)
                    key[j] = 0;
        }
    } else {
        // replacement-slot scan (routing_top_k_iter): state is wave-uniform
        float sv[MAX_K];
        uint32_t se[MAX_K];
        for (uint32_t s = 0; s < K; ++s)
            sv[s] = -INFINITY, se[s] = 0;
        uint32_t mi = 0;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            uint32_t e = lane + WAVE * j;
            uint64_t cand = __ballot(e < E && sel[j] > sv[mi]);
            while (cand) {
                int src = __ffsll((unsigned long long)cand) - 1;
                cand &= cand - 1ull;
                float s = __shfl(sel[j], src);
                if (s > sv[mi]) {
                    sv[mi] = s;
                    se[mi] = (uint32_t)src + WAVE * j;
                    mi = 0;
                    for (uint32_t c = 1; c < K; ++c)
                        if (sv[c] < sv[mi])
                            mi = c;
                }
            }
        }
        for (uint32_t s = 0; s < K; ++s)
            out_e[s] = se[s];
    }
    // gather the value behind each selected id
    for (uint32_t r = 0; r < K; ++r) {
        uint32_t e = out_e[r];
        int src = (int)(e & 63u);
        int jj = (int)(e >> 6);
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            if (j == jj)
                v = raw[j];
        v = __shfl(v, src);
        out_v[r] = p.kind == 0 ? v : sigmoidf_(v);
    }
    if (lane == 0) {
        float prob[MAX_K];
        for (uint32_t r = 0; r < K; ++r) {
            if (p.kind == 0) {
                float v = expf(out_v[r] - mx);
                prob[r] = have_inv ? v * inv_sum : v;
            } else {
                prob[r] = out_v[r];
            }
        }
        float sum = -0.0f;
        for (uint32_t r = 0; r < K; ++r)
            sum = sum + prob[r];
        float inv;
        if (p.norm == 1) {
            if (!(isfinite(sum) && sum >= 0.0f))
                atomicOr(status, ST_BAD_SUM);
            inv = 1.0f / fmaxf(sum, 6.103515625e-5f);
        } else {
            if (!(isfinite(sum) && sum > 0.0f))
                atomicOr(status, ST_BAD_SUM);
            inv = 1.0f / sum;
        }
        for (uint32_t r = 0; r < K; ++r) {
            if (prob[r] < 0.0f)
                atomicOr(status, ST_NEGATIVE);
            float wgt = prob[r] * inv;
            ids[(uint64_t)t * K + r] = out_e[r];
            weights[(uint64_t)t * K + r] = wgt * p.routed_scale;
        }
    }
}

hipError_t launch_route_topk(hipStream_t s, const float* logits, const float* bias, uint32_t tokens,
                             const RouteParams& p, uint32_t* ids, float* weights, uint32_t* status)
{
    dim3 grid((tokens + 3) / 4), block(256);
    uint32_t epl = (p.experts + WAVE - 1) / WAVE;
    if (epl <= 2)
        route_topk_kernel<2><<<grid, block, 0, s>>>(logits, bias, tokens, p, ids, weights, status);
    else if (epl <= 4)
        route_topk_kernel<4><<<grid, block, 0, s>>>(logits, bias, tokens, p, ids, weights, status);
    else if (epl <= 8)
        route_topk_kernel<8><<<grid, block, 0, s>>>(logits, bias, tokens, p, ids, weights, status);
    else
        route_topk_kernel<16><<<grid, block, 0, s>>>(logits, bias, tokens, p, ids, weights, status);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// dispatch plan: sorted unique union + stable counting sort of routes by
// expert, deterministic (no order-dependent atomics on result positions).
// One workgroup of 8 waves; each wave owns a contiguous route range.
// ---------------------------------------------------------------------------
constexpr int PLAN_WAVES = 8;
constexpr int PLAN_MAX_E = 1024;

__global__ __launch_bounds__(PLAN_WAVES * 64) void dispatch_plan_kernel(
    const uint32_t* __restrict__ ids, uint32_t routes, uint32_t experts, uint32_t k, Plan plan,
    uint32_t* __restrict__ status)
{
    __shared__ uint32_t wcnt[PLAN_WAVES][PLAN_MAX_E];
    __shared__ uint32_t start[PLAN_MAX_E];
    __shared__ uint32_t slot[PLAN_MAX_E];
    __shared__ uint32_t scan_a[PLAN_MAX_E];
    __shared__ uint32_t scan_b[PLAN_MAX_E];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nthr = PLAN_WAVES * 64;

    for (int i = tid; i < PLAN_WAVES * PLAN_MAX_E; i += nthr)
        (&wcnt[0][0])[i] = 0;
    __syncthreads();

    uint32_t per_wave = (routes + PLAN_WAVES - 1) / PLAN_WAVES;
    per_wave = (per_wave + 63u) & ~63u;
    const uint32_t r_begin = wv * per_wave;
    const uint32_t r_end = min(routes, r_begin + per_wave);

    bool bad = false;
    for (uint32_t r = r_begin + lane; r < r_end; r += 64) {
        uint32_t e = ids[r];
        if (e < experts)
            atomicAdd(&wcnt[wv][e], 1u);
        else
            bad = true;
    }
    if (__ballot(bad) != 0ull && lane == 0)
        atomicOr(status, ST_ROUTE_RANGE);
    __syncthreads();

    // per expert: exclusive prefix over waves, total
    for (uint32_t e = tid; e < PLAN_MAX_E; e += nthr) {
        uint32_t run = 0;
        if (e < experts) {
            for (int w = 0; w < PLAN_WAVES; ++w) {
                uint32_t c = wcnt[w][e];
                wcnt[w][e] = run;
                run += c;
            }
        }
        scan_a[e] = run;                 // total count
        scan_b[e] = run > 0 ? 1u : 0u;   // used flag
    }
    __syncthreads();
    // inclusive Hillis-Steele scans of counts (scan_a) and flags (scan_b)
    for (uint32_t off = 1; off < PLAN_MAX_E; off <<= 1) {
        uint32_t va[2], vb[2];
        for (int i = 0; i < 2; ++i) {
            uint32_t e = tid + i * nthr;
            va[i] = scan_a[e] + (e >= off ? scan_a[e - off] : 0u);
            vb[i] = scan_b[e] + (e >= off ? scan_b[e - off] : 0u);
        }
        __syncthreads();
        for (int i = 0; i < 2; ++i) {
            uint32_t e = tid + i * nthr;
            scan_a[e] = va[i];
            scan_b[e] = vb[i];
        }
        __syncthreads();
    }
    for (uint32_t e = tid; e < PLAN_MAX_E; e += nthr) {
        uint32_t incl = scan_a[e];
        uint32_t prev = e > 0 ? scan_a[e - 1] : 0u;
        uint32_t cnt = incl - prev;
        uint32_t s_incl = scan_b[e];
        start[e] = prev;
        slot[e] = s_incl - (cnt > 0 ? 1u : 0u);
        if (e < experts && cnt > 0) {
            uint32_t sl = s_incl - 1u;
            plan.unique_ids[sl] = e;
            plan.groups[2 * sl] = prev;
            plan.groups[2 * sl + 1] = cnt;
        }
    }
    if (tid == 0)
        plan.unique_count[0] = scan_b[PLAN_MAX_E - 1];
    __syncthreads();

    // stable placement: chunks of 64 routes in order; rank among equal ids
    // inside a chunk comes from a ballot match loop.
    for (uint32_t r0 = r_begin; r0 < r_end; r0 += 64) {
        uint32_t r = r0 + lane;
        bool valid = r < r_end;
        uint32_t e = valid ? ids[r] : 0xFFFFFFFFu;
        bool in_range = valid && e < experts;
        uint64_t remaining = __ballot(in_range);
        uint64_t peers = 0;
        while (remaining) {
            int leader = __ffsll((unsigned long long)remaining) - 1;
            uint32_t le = __shfl(e, leader);
            uint64_t m = __ballot(in_range && e == le);
            if (in_range && e == le)
                peers = m;
            remaining &= ~m;
        }
        if (in_range) {
            uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
            uint32_t rank = __popcll(peers & below);
            uint32_t base = wcnt[wv][e];
            uint32_t pos = start[e] + base + rank;
            plan.src_rows[pos] = r / k;
            plan.out_idx[r] = pos;
            plan.route_slots[r] = slot[e];
        } else if (valid) {
            plan.out_idx[r] = 0xFFFFFFFFu;
            plan.route_slots[r] = 0xFFFFFFFFu;
        }
        // the highest lane of each peer group advances the wave cursor
        if (in_range) {
            int top = 63 - __clzll((long long)peers);
            if (top == lane)
                wcnt[wv][e] += __popcll(peers);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    }
}

hipError_t launch_dispatch_plan(hipStream_t s, const uint32_t* ids, uint32_t routes,
                                uint32_t experts, uint32_t k, const Plan& plan, uint32_t* status)
{
    dispatch_plan_kernel<<<1, PLAN_WAVES * 64, 0, s>>>(ids, routes, experts, k, plan, status);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// decode expert phase 1: gate/up projections + SiLU(g)*u for every work
// item (unique expert with its routed tokens, or the shared expert with all
// tokens).  One wave per intermediate row; the gate and up rows of the same
// index are read together so the activation is formed in registers.
// ---------------------------------------------------------------------------
struct ItemRef {
    const uint8_t* slot;
    uint32_t g0, n;   // grouped route range (or token range for shared)
    bool shared;
};

template <int SBT, int CPL>
__global__ __launch_bounds__(256) void decode_gateup_kernel(
    ExpertSet ex, ExpertSet sh, bool has_shared, const void* __restrict__ sgate_w,
    uint32_t sgate_dtype, const float* __restrict__ x, uint32_t tokens, uint32_t k,
    uint32_t hidden, const uint32_t* __restrict__ ids, Plan plan, bool use_plan,
    float* __restrict__ act, float* __restrict__ act_shared, float* __restrict__ shared_weight,
    uint32_t* __restrict__ status)
{
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const uint32_t item = blockIdx.y;
    const uint32_t routed_items = use_plan ? plan.unique_count[0] : tokens * k;
    const uint32_t max_routed = gridDim.y - (has_shared ? 1u : 0u);

    const uint8_t* slot;
    uint32_t g0, n, I;
    bool shared = false;
    if (has_shared && item == max_routed) {
        shared = true;
        slot = sh.base;
        g0 = 0;
        n = tokens;
        I = sh.gate.rows;
    } else {
        if (item >= routed_items)
            return;
        uint32_t e;
        if (use_plan) {
            e = plan.unique_ids[item];
            g0 = plan.groups[2 * item];
            n = plan.groups[2 * item + 1];
        } else {
            e = ids[item];
            g0 = item;
            n = 1;
        }
        if (e >= ex.count) {
            if (lane == 0 && wv == 0 && blockIdx.x == 0)
                atomicOr(status, ST_ROUTE_RANGE);
            return;
        }
        slot = ex.base + (uint64_t)e * ex.stride;
        I = ex.gate.rows;
    }
    const ExpertSet& set = shared ? sh : ex;
    const uint32_t row = blockIdx.x * 4 + wv;

    // shared-expert sigmoid gate: sigma(W_sg . x_t), or 1 without a gate
    if (shared && blockIdx.x == 0 && wv == 0) {
        for (uint32_t t = 0; t < tokens; ++t) {
            float g = 80.0f;
            if (sgate_w) {
                float a = 0.0f;
                for (uint32_t c = lane; c < hidden; c += WAVE) {
                    float wvv;
                    if (sgate_dtype == 0)
                        wvv = reinterpret_cast<const float*>(sgate_w)[c];
                    else if (sgate_dtype == 2)
                        wvv = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(sgate_w)[c] << 16);
                    else
                        wvv = __half2float(__ushort_as_half(reinterpret_cast<const uint16_t*>(sgate_w)[c]));
                    a = fmaf(wvv, x[(uint64_t)t * hidden + c], a);
                }
                g = wave_sum(a);
            }
            if (lane == 0)
                shared_weight[t] = sigmoidf_(g);
        }
    }
    if (row >= I)
        return;

    const uint32_t chunks = hidden / 32; // 16-byte chunks per row
    const uint32_t gpr = hidden / set.group;
    const uint8_t* gw = slot + set.gate.w_off + (uint64_t)row * (hidden / 2);
    const uint8_t* uw = slot + set.up.w_off + (uint64_t)row * (hidden / 2);
    const uint8_t* gs = slot + set.gate.s_off;
    const uint8_t* gb = slot + set.gate.b_off;
    const uint8_t* us = slot + set.up.s_off;
    const uint8_t* ub = slot + set.up.b_off;

    uint4 wg[CPL], wu[CPL];
    float sg[CPL], bg[CPL], su[CPL], bu[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        uint32_t c = lane + WAVE * j;
        if (c < chunks) {
            wg[j] = reinterpret_cast<const uint4*>(gw)[c];
            wu[j] = reinterpret_cast<const uint4*>(uw)[c];
            uint64_t gi = (uint64_t)row * gpr + (c * 32u) / set.group;
            sg[j] = sb_at<SBT>(gs, gi);
            bg[j] = sb_at<SBT>(gb, gi);
            su[j] = sb_at<SBT>(us, gi);
            bu[j] = sb_at<SBT>(ub, gi);
        }
    }
    for (uint32_t j = 0; j < n; ++j) {
        uint32_t gidx = g0 + j;
        uint32_t tok = shared ? j : (use_plan ? plan.src_rows[gidx] : gidx / k);
        const float* xt = x + (uint64_t)tok * hidden;
        float pg = 0.0f, pu = 0.0f;
#pragma unroll
        for (int jj = 0; jj < CPL; ++jj) {
            uint32_t c = lane + WAVE * jj;
            if (c < chunks) {
                float xs;
                float qg = q4_chunk_qx(wg[jj], xt + c * 32, xs);
                float xs2;
                float qu = q4_chunk_qx(wu[jj], xt + c * 32, xs2);
                pg = fmaf(sg[jj], qg, fmaf(bg[jj], xs, pg));
                pu = fmaf(su[jj], qu, fmaf(bu[jj], xs, pu));
            }
        }
        float g = wave_sum(pg);
        float u = wave_sum(pu);
        if (lane == 0) {
            float a = (g / (1.0f + expf(-g))) * u;
            if (shared)
                act_shared[(uint64_t)j * I + row] = a;
            else
                act[(uint64_t)gidx * I + row] = a;
        }
    }
}

// ---------------------------------------------------------------------------
// decode expert phase 2: down projection fused with the weighted combine and
// the shared-expert add.  A block owns R = 64/LPR output rows; its 4 waves
// split the work items; y values meet in LDS and one thread per (token, row)
// forms  h = (r + sum_k w_k y_k) + sw * S  in route order.
// ---------------------------------------------------------------------------
constexpr int DEC_MAX_T = 16;
constexpr int DEC_MAX_ROUTES = DEC_MAX_T * MAX_K;

template <int SBT, int LPR, int CPL>
__global__ __launch_bounds__(256) void decode_down_combine_kernel(
    ExpertSet ex, ExpertSet sh, bool has_shared, const float* __restrict__ act,
    const float* __restrict__ act_shared, const float* __restrict__ shared_weight,
    uint32_t tokens, uint32_t k, uint32_t hidden, const uint32_t* __restrict__ ids,
    const float* __restrict__ weights, Plan plan, bool use_plan,
    const float* __restrict__ residual, float* __restrict__ hidden_out,
    uint32_t* __restrict__ status)
{
    constexpr int R = 64 / LPR;
    __shared__ float ylds[DEC_MAX_ROUTES][R];
    __shared__ float yshl[DEC_MAX_T][R];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int gl = lane % LPR;      // lane within the row group
    const int rr = lane / LPR;      // row within the block
    const uint32_t row = blockIdx.x * R + rr;
    const uint32_t routed_items = use_plan ? plan.unique_count[0] : tokens * k;
    const uint32_t items = routed_items + (has_shared ? 1u : 0u);

    for (uint32_t item = wv; item < items; item += 4) {
        const bool shared = has_shared && item == routed_items;
        const ExpertSet& set = shared ? sh : ex;
        const uint8_t* slot;
        uint32_t g0, n;
        if (shared) {
            slot = sh.base;
            g0 = 0;
            n = tokens;
        } else {
            uint32_t e;
            if (use_plan) {
                e = plan.unique_ids[item];
                g0 = plan.groups[2 * item];
                n = plan.groups[2 * item + 1];
            } else {
                e = ids[item];
                g0 = item;
                n = 1;
            }
            if (e >= ex.count) {
                for (uint32_t j = 0; j < n; ++j)
                    if (gl == 0)
                        ylds[g0 + j][rr] = 0.0f;
                continue;
            }
            slot = ex.base + (uint64_t)e * ex.stride;
        }
        const uint32_t I = set.down.cols;
        const uint32_t chunks = I / 32;
        const uint32_t gpr = I / set.group;
        const uint8_t* dw = slot + set.down.w_off + (uint64_t)row * (I / 2);
        uint4 w[CPL];
        float s[CPL], b[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            uint32_t c = gl + LPR * j;
            if (c < chunks) {
                w[j] = reinterpret_cast<const uint4*>(dw)[c];
                uint64_t gi = (uint64_t)row * gpr + (c * 32u) / set.group;
                s[j] = sb_at<SBT>(slot + set.down.s_off, gi);
                b[j] = sb_at<SBT>(slot + set.down.b_off, gi);
            }
        }
        for (uint32_t j = 0; j < n; ++j) {
            const float* a = shared ? act_shared + (uint64_t)j * I : act + (uint64_t)(g0 + j) * I;
            float part = 0.0f;
#pragma unroll
            for (int jj = 0; jj < CPL; ++jj) {
                uint32_t c = gl + LPR * jj;
                if (c < chunks) {
                    float xs;
                    float qx = q4_chunk_qx(w[jj], a + c * 32, xs);
                    part = fmaf(s[jj], qx, fmaf(b[jj], xs, part));
                }
            }
            float y = group_sum<LPR>(part);
            if (gl == 0) {
                if (shared)
                    yshl[j][rr] = y;
                else
                    ylds[g0 + j][rr] = y;
            }
        }
    }
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < tokens * R; idx += 256) {
        uint32_t t = idx / R, r = idx % R;
        float moe = 0.0f;
        for (uint32_t kk = 0; kk < k; ++kk) {
            uint32_t route = t * k + kk;
            uint32_t gi = use_plan ? plan.out_idx[route] : route;
            float y = gi < DEC_MAX_ROUTES ? ylds[gi][r] : 0.0f;
            moe = moe + weights[route] * y;
        }
        uint64_t o = (uint64_t)t * hidden + blockIdx.x * R + r;
        float rm = residual[o] + moe;
        float sw = has_shared ? shared_weight[t] : 0.0f;
        float sv = has_shared ? yshl[t][r] : 0.0f;
        hidden_out[o] = rm + sw * sv;
    }
}

// next-layer RMSNorm: one block per token (rms_norm_reduced)
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ h,
                                                       const float* __restrict__ w,
                                                       uint32_t width, float eps,
                                                       float* __restrict__ out)
{
    __shared__ float part[4];
    const float* row = h + (uint64_t)blockIdx.x * width;
    float s = 0.0f;
    for (uint32_t i = threadIdx.x; i < width; i += 256)
        s = fmaf(row[i], row[i], s);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0)
        part[threadIdx.x >> 6] = s;
    __syncthreads();
    float ms = ((part[0] + part[1]) + (part[2] + part[3])) / (float)(width > 1 ? width : 1);
    float scale = 1.0f / sqrtf(ms + eps);
    for (uint32_t i = threadIdx.x; i < width; i += 256)
        out[(uint64_t)blockIdx.x * width + i] = (row[i] * scale) * w[i];
}

template <int SBT>
static hipError_t launch_decode_typed(hipStream_t s, const ExpertSet& ex, const ExpertSet* shared,
                                      const void* sgw, uint32_t sgdt, const float* x,
                                      const float* residual, uint32_t tokens, uint32_t k,
                                      uint32_t hidden, const uint32_t* ids, const float* weights,
                                      const Plan* plan, float* act, float* act_shared,
                                      float* shared_weight, float* hidden_out,
                                      const float* next_norm_w, float eps, float* next_normed,
                                      uint32_t* status)
{
    const bool has_shared = shared != nullptr;
    ExpertSet sh = has_shared ? *shared : ExpertSet{};
    Plan pl = plan ? *plan : Plan{};
    const bool use_plan = plan != nullptr;
    uint32_t routed_items = use_plan ? std::min(ex.count, tokens * k) : tokens * k;
    uint32_t I = ex.gate.rows;
    uint32_t Imax = has_shared && sh.gate.rows > I ? sh.gate.rows : I;
    dim3 g1((Imax + 3) / 4, routed_items + (has_shared ? 1u : 0u));
    uint32_t cpl = (hidden / 32 + WAVE - 1) / WAVE;
#define PBM_GU(C)                                                                              \
    decode_gateup_kernel<SBT, C><<<g1, 256, 0, s>>>(ex, sh, has_shared, sgw, sgdt, x, tokens, k, \
                                                    hidden, ids, pl, use_plan, act, act_shared, \
                                                    shared_weight, status)
    if (cpl <= 1)
        PBM_GU(1);
    else if (cpl <= 2)
        PBM_GU(2);
    else if (cpl <= 4)
        PBM_GU(4);
    else
        return hipErrorInvalidValue;
#undef PBM_GU
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return err;

    // down: LPR = 8 lanes per row, CPL2 = I / 256 chunks per lane
    uint32_t Id = I;
    if (has_shared && sh.down.cols != Id)
        return hipErrorInvalidValue; // shared and routed intermediates must match here
    uint32_t cpl2 = Id / 256;
    dim3 g2(hidden / 8);
#define PBM_DN(C)                                                                              \
    decode_down_combine_kernel<SBT, 8, C><<<g2, 256, 0, s>>>(                                  \
        ex, sh, has_shared, act, act_shared, shared_weight, tokens, k, hidden, ids, weights,    \
        pl, use_plan, residual, hidden_out, status)
    if (cpl2 == 1)
        PBM_DN(1);
    else if (cpl2 == 2)
        PBM_DN(2);
    else if (cpl2 == 3)
        PBM_DN(3);
    else if (cpl2 == 4)
        PBM_DN(4);
    else if (cpl2 <= 8)
        PBM_DN(8);
    else
        return hipErrorInvalidValue;
#undef PBM_DN
    err = hipGetLastError();
    if (err != hipSuccess)
        return err;
    if (next_norm_w && next_normed) {
        rms_norm_kernel<<<tokens, 256, 0, s>>>(hidden_out, next_norm_w, hidden, eps, next_normed);
        err = hipGetLastError();
    }
    return err;
}

hipError_t launch_decode_experts(hipStream_t s, const ExpertSet& ex, const ExpertSet* shared,
                                 const void* shared_gate_w, uint32_t shared_gate_dtype,
                                 const float* x, const float* residual, uint32_t tokens,
                                 uint32_t k, uint32_t hidden, const uint32_t* ids,
                                 const float* weights, const Plan* plan, float* act,
                                 float* act_shared, float* shared_weight, float* hidden_out,
                                 const float* next_norm_w, float eps, float* next_normed,
                                 uint32_t* status)
{
    if (ex.sb_dtype == 2)
        return launch_decode_typed<2>(s, ex, shared, shared_gate_w, shared_gate_dtype, x,
                                      residual, tokens, k, hidden, ids, weights, plan, act,
                                      act_shared, shared_weight, hidden_out, next_norm_w, eps,
                                      next_normed, status);
    return launch_decode_typed<1>(s, ex, shared, shared_gate_w, shared_gate_dtype, x, residual,
                                  tokens, k, hidden, ids, weights, plan, act, act_shared,
                                  shared_weight, hidden_out, next_norm_w, eps, next_normed,
                                  status);
}

// ---------------------------------------------------------------------------
// dequantisation: out = fma(q, s, b)  (math.rs:913-954)
// ---------------------------------------------------------------------------
template <int SBT>
__global__ void q4_dequant_kernel(const uint8_t* __restrict__ packed,
                                  const uint8_t* __restrict__ scales,
                                  const uint8_t* __restrict__ biases, uint32_t rows,
                                  uint32_t cols, uint32_t group, float* __restrict__ out)
{
    uint64_t words = (uint64_t)rows * cols / 8;
    for (uint64_t wi = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; wi < words;
         wi += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t q = reinterpret_cast<const uint32_t*>(packed)[wi];
        uint64_t c0 = wi * 8;
        uint64_t r = c0 / cols;
        uint32_t c = (uint32_t)(c0 % cols);
        uint64_t gi = r * (cols / group) + c / group;
        float s = sb_at<SBT>(scales, gi);
        float b = sb_at<SBT>(biases, gi);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            out[c0 + i] = fmaf((float)((q >> (4 * i)) & 15u), s, b);
    }
}

hipError_t launch_q4_dequantize(hipStream_t s, const uint8_t* packed, const void* scales,
                                const void* biases, uint32_t sb_dtype, uint32_t rows,
                                uint32_t cols, uint32_t group, float* out)
{
    uint64_t words = (uint64_t)rows * cols / 8;
    uint32_t blocks = (uint32_t)std::min<uint64_t>((words + 255) / 256, 65535);
    if (sb_dtype == 2)
        q4_dequant_kernel<2><<<blocks, 256, 0, s>>>(packed, (const uint8_t*)scales,
                                                   (const uint8_t*)biases, rows, cols, group, out);
    else
        q4_dequant_kernel<1><<<blocks, 256, 0, s>>>(packed, (const uint8_t*)scales,
                                                   (const uint8_t*)biases, rows, cols, group, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// seeded synthetic fill (bit-identical to synth_host.c)
// ---------------------------------------------------------------------------
struct SynthArgs {
    uint64_t off[9];
    uint64_t stride, seed;
    uint32_t hidden, intermediate, group, sb_dtype, tensor, layer, first_expert;
};

__global__ void synth_fill_kernel(uint8_t* __restrict__ slots, SynthArgs a)
{
    const uint32_t ei = blockIdx.y;
    const uint32_t expert = a.first_expert + ei;
    uint8_t* slot = slots + (uint64_t)ei * a.stride;
    const uint64_t wpp = (uint64_t)a.hidden * a.intermediate / 8; // words per projection
    const uint64_t gpp = (uint64_t)a.hidden * a.intermediate / a.group;
    const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t tid = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
    for (uint64_t i = tid; i < 3 * wpp; i += nthreads) {
        uint32_t p = (uint32_t)(i / wpp);
        uint64_t w = i % wpp;
        uint32_t v = pbm_q4_word(a.seed, a.tensor, a.layer, expert, p, w);
        reinterpret_cast<uint32_t*>(slot + a.off[3 * p])[w] = v;
    }
    for (uint64_t i = tid; i < 3 * gpp; i += nthreads) {
        uint32_t p = (uint32_t)(i / gpp);
        uint64_t j = i % gpp;
        uint16_t sv = pbm_q4_scale_bias(a.seed, a.tensor, a.layer, expert, p, 1u, j, a.sb_dtype);
        uint16_t bv = pbm_q4_scale_bias(a.seed, a.tensor, a.layer, expert, p, 2u, j, a.sb_dtype);
        reinterpret_cast<uint16_t*>(slot + a.off[3 * p + 1])[j] = sv;
        reinterpret_cast<uint16_t*>(slot + a.off[3 * p + 2])[j] = bv;
    }
}

hipError_t launch_synth_fill(hipStream_t s, uint8_t* slots, uint64_t stride,
                             const uint64_t* offsets9, uint32_t hidden, uint32_t intermediate,
                             uint32_t group, uint32_t sb_dtype, uint64_t seed, uint32_t tensor,
                             uint32_t layer, uint32_t first_expert, uint32_t count)
{
    SynthArgs a;
    for (int i = 0; i < 9; ++i)
        a.off[i] = offsets9[i];
    a.stride = stride;
    a.seed = seed;
    a.hidden = hidden;
    a.intermediate = intermediate;
    a.group = group;
    a.sb_dtype = sb_dtype;
    a.tensor = tensor;
    a.layer = layer;
    a.first_expert = first_expert;
    for (uint32_t done = 0; done < count; done += 65535u) {
        uint32_t n = std::min(count - done, 65535u);
        a.first_expert = first_expert + done;
        dim3 grid(256, n);
        synth_fill_kernel<<<grid, 256, 0, s>>>(slots + (uint64_t)done * stride, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return e;
    }
    return hipSuccess;
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, uint64_t n)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

hipError_t launch_fill_u32(hipStream_t s, uint32_t* p, uint32_t value, uint64_t n)
{
    uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 1024);
    fill_u32_kernel<<<blocks ? blocks : 1, 256, 0, s>>>(p, value, n);
    return hipGetLastError();
}

} // namespace pbmoe
