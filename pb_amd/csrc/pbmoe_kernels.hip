// gfx950 (MI355X) kernels of the MoE block outside the decode path: router
// logits and routing for many tokens (prefill router matrix), the standalone
// deterministic dispatch plan, dequantisation and the seeded weight fill.
//
// Reference counterparts (src/inference/flashmoe/ of Jc2k/pb):
// dense_mmap_fma_matvec_* (metal/qwen/shaders.metal:1059-1111), the CPU
// routing stage (math.rs:746-819, scheduler/expert_access.rs:80-135), the
// group plan (metal/mod.rs:3197-3233), q4_dequantize_rows_with_group_size
// (math.rs:913-954).
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "pbmoe_device.h"
#include "pbmoe_internal.h"
#include "pbmoe_synth.h"

namespace pbmoe {

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

// Q4 router rows: one wave per expert row, lane l takes the 32-column
// chunks l + 64 c; per chunk s . sum(q x) + b . sum(x) (the factored form of
// the dequantised row, q4_mmap_fma_matvec of the reference's shaders).
template <int SBT, int TT>
__global__ __launch_bounds__(256) void router_logits_q4_kernel(Q4Rows m, const float* __restrict__ x,
                                                               uint32_t tokens, uint32_t experts,
                                                               uint32_t hidden, float* __restrict__ logits)
{
    const int lane = threadIdx.x & 63;
    const uint32_t e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= experts)
        return;
    const uint32_t chunks = hidden / 32, gpr = hidden >> m.gshift;
    const uint4* wp = reinterpret_cast<const uint4*>(m.codes + (uint64_t)e * (hidden / 2));
    for (uint32_t t0 = 0; t0 < tokens; t0 += TT) {
        float acc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t)
            acc[t] = 0.0f;
        for (uint32_t ch = lane; ch < chunks; ch += WAVE) {
            const uint4 w = wp[ch];
            const uint64_t gi = (uint64_t)e * gpr + ((ch * 32u) >> m.gshift);
            const float sc = sb_at<SBT>(m.scales, gi), bi = sb_at<SBT>(m.biases, gi);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                if (t0 + t < tokens) {
                    float xs;
                    const float qx = q4_chunk_qx(w, x + (uint64_t)(t0 + t) * hidden + ch * 32u, xs);
                    acc[t] = fmaf(sc, qx, fmaf(bi, xs, acc[t]));
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
                                uint32_t tokens, uint32_t experts, uint32_t hidden, float* logits,
                                const Q4Rows* q4, uint32_t sb_dtype)
{
    dim3 grid((experts + 3) / 4), block(256);
    if (w_dtype == DT_Q4) {
        if (!q4)
            return hipErrorInvalidValue;
        if (sb_dtype == 2)
            router_logits_q4_kernel<2, 4><<<grid, block, 0, s>>>(*q4, x, tokens, experts, hidden, logits);
        else
            router_logits_q4_kernel<1, 4><<<grid, block, 0, s>>>(*q4, x, tokens, experts, hidden, logits);
        return hipGetLastError();
    }
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
// routing for many tokens: one wave per token (see route_token_wave)
// ---------------------------------------------------------------------------
template <int EPL>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias,
                                                         uint32_t tokens, RouteParams p,
                                                         uint32_t* __restrict__ ids,
                                                         float* __restrict__ weights,
                                                         uint32_t* __restrict__ status)
{
    __shared__ __align__(16) float grp[4][2 * EPL * WAVE + 192];
    __shared__ uint32_t sel[4][MAX_K];
    const int wv = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 4 + wv;
    if (t >= tokens)
        return;
    route_token_wave<EPL>(logits + (uint64_t)t * p.experts, bias, p, ids + (uint64_t)t * p.k,
                          weights + (uint64_t)t * p.k, sel[wv], grp[wv], status);
}

// decode token counts (block_routing): one workgroup per token
// (route_token_block), the same routing the fused decode layer performs, so
// both entry points agree bitwise
template <int EPT>
__global__ __launch_bounds__(256) void route_block_kernel(const float* __restrict__ logits,
                                                         const float* __restrict__ bias, RouteParams p,
                                                         uint32_t* __restrict__ ids,
                                                         float* __restrict__ weights,
                                                         uint32_t* __restrict__ status)
{
    __shared__ __align__(16) float scratch[1024 + 8 + 144];
    const uint32_t t = blockIdx.x;
    route_token_block<EPT>(logits + (uint64_t)t * p.experts, bias, p, ids + (uint64_t)t * p.k,
                           weights + (uint64_t)t * p.k, scratch, status);
}

hipError_t launch_route_topk(hipStream_t s, const float* logits, const float* bias, uint32_t tokens,
                             const RouteParams& p, uint32_t* ids, float* weights, uint32_t* status)
{
    if (block_routing(tokens, p)) {
        if (p.experts <= 256)
            route_block_kernel<1><<<tokens, 256, 0, s>>>(logits, bias, p, ids, weights, status);
        else if (p.experts <= 512)
            route_block_kernel<2><<<tokens, 256, 0, s>>>(logits, bias, p, ids, weights, status);
        else
            route_block_kernel<4><<<tokens, 256, 0, s>>>(logits, bias, p, ids, weights, status);
        return hipGetLastError();
    }
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

// ---------------------------------------------------------------------------
// multi-workgroup plan for long route lists (prefill): the same stable order
// as dispatch_plan_kernel.  Routes are cut into blocks of PLAN_CHUNK;
//   count: per block, per expert route counts;
//   scan:  per expert the exclusive prefix over blocks, then the sorted union
//          (unique ids, group starts/counts, slots) over experts;
//   place: per block the single-workgroup placement with absolute bases.
// ---------------------------------------------------------------------------
constexpr uint32_t PLAN_CHUNK = PLAN_WAVES * 64; // one route per lane
constexpr uint32_t PLAN_SINGLE_MAX = 2048;        // routes the one-workgroup kernel takes

__global__ __launch_bounds__(PLAN_WAVES * 64) void plan_count_kernel(
    const uint32_t* __restrict__ ids, uint32_t routes, uint32_t experts, uint32_t* __restrict__ cnt,
    uint32_t* __restrict__ status)
{
    __shared__ uint32_t c[PLAN_MAX_E];
    const int tid = threadIdx.x, lane = tid & 63;
    const int nthr = PLAN_WAVES * 64;
    for (int i = tid; i < PLAN_MAX_E; i += nthr)
        c[i] = 0;
    __syncthreads();
    const uint32_t r0 = blockIdx.x * PLAN_CHUNK;
    const uint32_t r1 = min(routes, r0 + PLAN_CHUNK);
    bool bad = false;
    for (uint32_t r = r0 + tid; r < r1; r += nthr) {
        const uint32_t e = ids[r];
        if (e < experts)
            atomicAdd(&c[e], 1u);
        else
            bad = true;
    }
    if (__ballot(bad) != 0ull && lane == 0)
        atomicOr(status, ST_ROUTE_RANGE);
    __syncthreads();
    for (uint32_t e = tid; e < experts; e += nthr)
        cnt[(uint64_t)blockIdx.x * experts + e] = c[e];
}

// P = 1024 / experts threads per expert (a power of two, at most 64, the
// lanes of one wave): thread (e, p) takes a contiguous range of blocks, so
// every count is loaded once, in one round trip when a range holds at most
// PLAN_SCAN_NB blocks (kept in registers for the bases); the prefix over
// experts is a wave scan plus the sums of the earlier waves.
constexpr uint32_t PLAN_SCAN_NB = 16;
__global__ __launch_bounds__(PLAN_MAX_E) void plan_scan_kernel(const uint32_t* __restrict__ cnt,
                                                              uint32_t nblk, uint32_t experts, Plan plan,
                                                              uint32_t* __restrict__ base,
                                                              uint32_t* __restrict__ slot_of)
{
    __shared__ uint32_t tot[PLAN_MAX_E], start[PLAN_MAX_E], wtot[PLAN_MAX_E / 64][2];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint32_t P = 1;
    while (P < 64 && 2 * P * experts <= PLAN_MAX_E)
        P *= 2;
    const uint32_t e = tid / P, p = tid % P;
    const uint32_t per = (nblk + P - 1) / P;
    const uint32_t b0 = min(nblk, p * per), b1 = min(nblk, b0 + per);
    const bool live = e < experts;
    const bool held = per <= PLAN_SCAN_NB; // the range's counts stay in registers
    uint32_t v[PLAN_SCAN_NB];
    uint32_t part = 0;
    if (held) {
#pragma unroll
        for (uint32_t j = 0; j < PLAN_SCAN_NB; ++j) {
            const uint32_t b = b0 + j;
            v[j] = live && b < b1 ? cnt[(uint64_t)b * experts + e] : 0u;
        }
#pragma unroll
        for (uint32_t j = 0; j < PLAN_SCAN_NB; ++j)
            part += v[j];
    } else if (live) {
        for (uint32_t c0 = b0; c0 < b1; c0 += PLAN_SCAN_NB) {
            uint32_t w[PLAN_SCAN_NB];
#pragma unroll
            for (uint32_t j = 0; j < PLAN_SCAN_NB; ++j)
                w[j] = c0 + j < b1 ? cnt[(uint64_t)(c0 + j) * experts + e] : 0u;
#pragma unroll
            for (uint32_t j = 0; j < PLAN_SCAN_NB; ++j)
                part += w[j];
        }
    }
    // exclusive prefix of the parts within the expert's P lanes, and its total
    uint32_t incl = part;
    for (uint32_t o = 1; o < P; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o);
        if (p >= o)
            incl += y;
    }
    const uint32_t run = __shfl(incl, (int)(lane | (P - 1))); // the group's last lane: the expert's count
    const uint32_t before = incl - part;
    if (p == 0 && live)
        tot[e] = run;
    __syncthreads();
    // per expert (one per thread): start = counts of the experts before,
    // slot = used experts before
    const uint32_t r = tid < experts ? tot[tid] : 0u;
    uint32_t ir = r, iu = r > 0 ? 1u : 0u;
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const uint32_t yr = __shfl_up(ir, o), yu = __shfl_up(iu, o);
        if (lane >= o)
            ir += yr, iu += yu;
    }
    if (lane == 63)
        wtot[wv][0] = ir, wtot[wv][1] = iu;
    __syncthreads();
    uint32_t pr = 0, pu = 0, all_u = 0;
    for (uint32_t w = 0; w < PLAN_MAX_E / 64; ++w) {
        if (w < wv)
            pr += wtot[w][0], pu += wtot[w][1];
        all_u += wtot[w][1];
    }
    if (tid < experts) {
        const uint32_t st = pr + ir - r;
        uint32_t sl = 0xFFFFFFFFu;
        if (r > 0) {
            sl = pu + iu - 1u;
            plan.unique_ids[sl] = tid;
            plan.groups[2 * sl] = st;
            plan.groups[2 * sl + 1] = r;
        }
        slot_of[tid] = sl;
        start[tid] = st;
    }
    if (tid == 0)
        plan.unique_count[0] = all_u;
    __syncthreads();
    // absolute base of every block: the expert's start + the counts of its
    // blocks before
    if (live) {
        uint32_t acc = start[e] + before;
        if (held) {
#pragma unroll
            for (uint32_t j = 0; j < PLAN_SCAN_NB; ++j) {
                const uint32_t b = b0 + j;
                if (b < b1) {
                    base[(uint64_t)b * experts + e] = acc;
                    acc += v[j];
                }
            }
        } else {
            for (uint32_t c0 = b0; c0 < b1; c0 += PLAN_SCAN_NB) {
                uint32_t w[PLAN_SCAN_NB];
#pragma unroll
                for (uint32_t j = 0; j < PLAN_SCAN_NB; ++j)
                    w[j] = c0 + j < b1 ? cnt[(uint64_t)(c0 + j) * experts + e] : 0u;
#pragma unroll
                for (uint32_t j = 0; j < PLAN_SCAN_NB; ++j)
                    if (c0 + j < b1) {
                        base[(uint64_t)(c0 + j) * experts + e] = acc;
                        acc += w[j];
                    }
            }
        }
    }
}

__global__ __launch_bounds__(PLAN_WAVES * 64) void plan_place_kernel(
    const uint32_t* __restrict__ ids, uint32_t routes, uint32_t experts, uint32_t k, Plan plan,
    const uint32_t* __restrict__ base, const uint32_t* __restrict__ slot_of)
{
    static_assert(PLAN_CHUNK == PLAN_WAVES * 64, "one route per lane");
    __shared__ uint32_t wcnt[PLAN_WAVES][PLAN_MAX_E];
    __shared__ uint32_t slt[PLAN_MAX_E];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int nthr = PLAN_WAVES * 64;
    const uint32_t r = blockIdx.x * PLAN_CHUNK + tid; // wave wv owns routes 64 wv .. 64 wv + 63 of the block
    const bool valid = r < routes;
    const uint32_t e = valid ? ids[r] : 0xFFFFFFFFu;
    const bool in_range = valid && e < experts;
    // this block's bases (the scan's output), loaded beside the ids rather
    // than after the two barriers below (experts <= 2 * PLAN_CHUNK)
    uint32_t bpre[PLAN_MAX_E / PLAN_CHUNK];
#pragma unroll
    for (int j = 0; j < (int)(PLAN_MAX_E / PLAN_CHUNK); ++j) {
        const uint32_t x = min(tid + (uint32_t)nthr * j, experts - 1);
        bpre[j] = base[(uint64_t)blockIdx.x * experts + x];
    }
    for (int i = tid; i < PLAN_WAVES * PLAN_MAX_E; i += nthr)
        (&wcnt[0][0])[i] = 0;
    for (uint32_t x = tid; x < experts; x += nthr)
        slt[x] = slot_of[x];
    __syncthreads();
    if (in_range)
        atomicAdd(&wcnt[wv][e], 1u);
    __syncthreads();
    // per expert: the block's absolute base, then the exclusive prefix over waves
#pragma unroll
    for (int j = 0; j < (int)(PLAN_MAX_E / PLAN_CHUNK); ++j) {
        const uint32_t x = tid + (uint32_t)nthr * j;
        if (x >= experts)
            break;
        uint32_t run = bpre[j];
        for (int w = 0; w < PLAN_WAVES; ++w) {
            const uint32_t c = wcnt[w][x];
            wcnt[w][x] = run;
            run += c;
        }
    }
    __syncthreads();
    // rank among this wave's earlier lanes with the same expert (stable order)
    uint64_t remaining = __ballot(in_range);
    uint64_t peers = 0;
    while (remaining) {
        const int leader = __ffsll((unsigned long long)remaining) - 1;
        const uint32_t le = __shfl(e, leader);
        const uint64_t m = __ballot(in_range && e == le);
        if (in_range && e == le)
            peers = m;
        remaining &= ~m;
    }
    if (in_range) {
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        const uint32_t pos = wcnt[wv][e] + __popcll(peers & below);
        plan.src_rows[pos] = r / k;
        plan.out_idx[r] = pos;
        plan.route_slots[r] = slt[e];
    } else if (valid) {
        plan.out_idx[r] = 0xFFFFFFFFu;
        plan.route_slots[r] = 0xFFFFFFFFu;
    }
}

uint32_t plan_work_words(uint32_t routes, uint32_t experts)
{
    const uint32_t nblk = (routes + PLAN_CHUNK - 1) / PLAN_CHUNK;
    return 2 * nblk * experts + experts;
}

hipError_t launch_dispatch_plan(hipStream_t s, const uint32_t* ids, uint32_t routes,
                                uint32_t experts, uint32_t k, const Plan& plan, uint32_t* status)
{
    if (routes <= PLAN_SINGLE_MAX || plan.work == nullptr) {
        dispatch_plan_kernel<<<1, PLAN_WAVES * 64, 0, s>>>(ids, routes, experts, k, plan, status);
        return hipGetLastError();
    }
    const uint32_t nblk = (routes + PLAN_CHUNK - 1) / PLAN_CHUNK;
    uint32_t* cnt = plan.work;
    uint32_t* base = cnt + (uint64_t)nblk * experts;
    uint32_t* slot_of = base + (uint64_t)nblk * experts;
    plan_count_kernel<<<nblk, PLAN_WAVES * 64, 0, s>>>(ids, routes, experts, cnt, status);
    plan_scan_kernel<<<1, PLAN_MAX_E, 0, s>>>(cnt, nblk, experts, plan, base, slot_of);
    plan_place_kernel<<<nblk, PLAN_WAVES * 64, 0, s>>>(ids, routes, experts, k, plan, base, slot_of);
    return hipGetLastError();
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

// zero-mean variant of the seeded weights: bias' = bias - 7.5 scale for every
// group of the three projections (codes are uniform over 0..15), rounded back
// to the scale/bias dtype; 7.5 scale is exact in f32, so one rounding.
__global__ void synth_center_kernel(uint8_t* __restrict__ slots, SynthArgs a)
{
    uint8_t* slot = slots + (uint64_t)blockIdx.y * a.stride;
    const uint64_t gpp = (uint64_t)a.hidden * a.intermediate / a.group;
    const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < 3 * gpp; i += nthreads) {
        const uint32_t p = (uint32_t)(i / gpp);
        const uint64_t j = i % gpp;
        const uint16_t sv = reinterpret_cast<const uint16_t*>(slot + a.off[3 * p + 1])[j];
        uint16_t* bp = reinterpret_cast<uint16_t*>(slot + a.off[3 * p + 2]) + j;
        if (a.sb_dtype == 2)
            *bp = pbm_f32_to_bf16(pbm_bf16_to_f32(*bp) - 7.5f * pbm_bf16_to_f32(sv));
        else
            *bp = pbm_f32_to_f16(pbm_f16_to_f32(*bp) - 7.5f * pbm_f16_to_f32(sv));
    }
}

hipError_t launch_synth_center(hipStream_t s, uint8_t* slots, uint64_t stride, const uint64_t* offsets9,
                               uint32_t hidden, uint32_t intermediate, uint32_t group, uint32_t sb_dtype,
                               uint32_t count)
{
    SynthArgs a{};
    for (int i = 0; i < 9; ++i)
        a.off[i] = offsets9[i];
    a.stride = stride;
    a.hidden = hidden;
    a.intermediate = intermediate;
    a.group = group;
    a.sb_dtype = sb_dtype;
    for (uint32_t done = 0; done < count; done += 65535u) {
        const uint32_t n = std::min(count - done, 65535u);
        synth_center_kernel<<<dim3(64, n), 256, 0, s>>>(slots + (uint64_t)done * stride, a);
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

// A plain read stream with the access shape of the decode weight loads: one
// 16-byte load per lane and step, grid-stride over n16 chunks; the words are
// XOR-folded (so the loads cannot be dropped) into *out with one atomic per
// workgroup.  The reference point for the PMC traffic counters.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ src, uint64_t n16,
                                                          uint32_t* __restrict__ out)
{
    __shared__ uint32_t red[4];
    uint32_t acc = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * 256) {
        const uint4 v = src[i];
        acc ^= (v.x ^ v.y) ^ (v.z ^ v.w);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
        atomicXor(out, (red[0] ^ red[1]) ^ (red[2] ^ red[3]));
}

hipError_t launch_stream_read(hipStream_t s, const void* src, uint64_t bytes, uint32_t* out)
{
    fill_u32_kernel<<<1, 64, 0, s>>>(out, 0u, 1);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    const uint64_t n16 = bytes / 16;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>(std::max<uint64_t>((n16 + 255) / 256, 1), 2048);
    stream_read_kernel<<<blocks, 256, 0, s>>>(static_cast<const uint4*>(src), n16, out);
    return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t s, uint32_t* p, uint32_t value, uint64_t n)
{
    uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 1024);
    fill_u32_kernel<<<blocks ? blocks : 1, 256, 0, s>>>(p, value, n);
    return hipGetLastError();
}

} // namespace pbmoe
