// Device helpers shared by the gfx950 kernels: DPP wave reductions, Q4
// chunk dot products, f32 total-order keys and the wave-level top-k.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pbmoe_internal.h"

namespace pbmoe {

constexpr int WAVE = 64;
constexpr int MAX_K = 16;

// DPP controls (gfx9 encoding)
constexpr int DPP_QUAD_1032 = 0xB1; // quad_perm [1,0,3,2]: lane ^ 1
constexpr int DPP_QUAD_2301 = 0x4E; // quad_perm [2,3,0,1]: lane ^ 2
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float readlane_f(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over aligned groups of W lanes (W in 2,4,8,16); every lane of the
// group receives the group sum.
template <int W>
__device__ __forceinline__ float group_sum(float v)
{
    static_assert(W == 2 || W == 4 || W == 8 || W == 16, "group width");
    v += dpp_f<DPP_QUAD_1032>(v);
    if constexpr (W >= 4)
        v += dpp_f<DPP_QUAD_2301>(v);
    if constexpr (W >= 8)
        v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    if constexpr (W >= 16)
        v += dpp_f<DPP_ROW_MIRROR>(v);
    return v;
}

// Whole-wave sum, uniform result (row sums via DPP, rows via readlane in a
// fixed order, so every call sums in the same order).
__device__ __forceinline__ float wave_sum(float v)
{
    v = group_sum<16>(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_f<DPP_QUAD_1032>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_2301>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, dpp_u<DPP_QUAD_1032>(v));
    v = max(v, dpp_u<DPP_QUAD_2301>(v));
    v = max(v, dpp_u<DPP_ROW_HALF_MIRROR>(v));
    v = max(v, dpp_u<DPP_ROW_MIRROR>(v));
    uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}

// f32 total order (Rust f32::total_cmp) mapped onto unsigned order.
__device__ __forceinline__ uint32_t total_key(float f)
{
    uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float sigmoidf_(float l) { return 1.0f / (1.0f + expf(-l)); }

template <int SBT>
__device__ __forceinline__ float sb_at(const uint8_t* base, uint64_t i)
{
    uint16_t v = reinterpret_cast<const uint16_t*>(base)[i];
    if constexpr (SBT == 2)
        return __uint_as_float((uint32_t)v << 16);
    else
        return __half2float(__ushort_as_half(v));
}

// One 16-byte chunk = 32 nibbles (columns 32c .. 32c+31, all in one quant
// group since the group size is a multiple of 32).  Returns sum(q * x) and
// sum(x): row = sum over chunks of s * sum(q*x) + b * sum(x).
__device__ __forceinline__ float q4_chunk_qx(uint4 w, const float* __restrict__ x, float& xs)
{
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float qx0 = 0.0f, qx1 = 0.0f, sx = 0.0f;
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 a = x4[2 * i];
        const float4 b = x4[2 * i + 1];
        const uint32_t q = words[i];
        qx0 = fmaf((float)(q & 15u), a.x, qx0);
        qx1 = fmaf((float)((q >> 4) & 15u), a.y, qx1);
        qx0 = fmaf((float)((q >> 8) & 15u), a.z, qx0);
        qx1 = fmaf((float)((q >> 12) & 15u), a.w, qx1);
        qx0 = fmaf((float)((q >> 16) & 15u), b.x, qx0);
        qx1 = fmaf((float)((q >> 20) & 15u), b.y, qx1);
        qx0 = fmaf((float)((q >> 24) & 15u), b.z, qx0);
        qx1 = fmaf((float)(q >> 28), b.w, qx1);
        sx += ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
    }
    xs = sx;
    return qx0 + qx1;
}

// Same with the 32 x values already in registers.
__device__ __forceinline__ float q4_chunk_qx_reg(uint4 w, const float (&xv)[32])
{
    float qx0 = 0.0f, qx1 = 0.0f;
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = words[i];
        qx0 = fmaf((float)(q & 15u), xv[8 * i + 0], qx0);
        qx1 = fmaf((float)((q >> 4) & 15u), xv[8 * i + 1], qx1);
        qx0 = fmaf((float)((q >> 8) & 15u), xv[8 * i + 2], qx0);
        qx1 = fmaf((float)((q >> 12) & 15u), xv[8 * i + 3], qx1);
        qx0 = fmaf((float)((q >> 16) & 15u), xv[8 * i + 4], qx0);
        qx1 = fmaf((float)((q >> 20) & 15u), xv[8 * i + 5], qx1);
        qx0 = fmaf((float)((q >> 24) & 15u), xv[8 * i + 6], qx0);
        qx1 = fmaf((float)(q >> 28), xv[8 * i + 7], qx1);
    }
    return qx0 + qx1;
}

// ---------------------------------------------------------------------------
// Wave-level canonical top-k (score desc, then lower index) of E <= 64*EPL
// candidates.  Lane l holds candidates e = l + 64*j in key[j] (total_key of
// the selection score; 0 = excluded).  Each lane sorts its own list, then K
// rounds pick the best head across the wave with a DPP max; an exact tie
// between lane heads resolves to the lowest expert index.  out_e receives
// the K ids (wave-uniform).
// ---------------------------------------------------------------------------
template <int EPL>
__device__ __forceinline__ void wave_topk_canonical(uint32_t (&key)[EPL], uint32_t k, uint32_t* out_e)
{
    const int lane = threadIdx.x & 63;
    uint32_t idx[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j)
        idx[j] = (uint32_t)lane + WAVE * j;
    // insertion-sort network, descending key, ascending index on equal keys
#pragma unroll
    for (int i = 1; i < EPL; ++i) {
#pragma unroll
        for (int j = i; j > 0; --j) {
            bool sw = key[j] > key[j - 1];
            uint32_t ka = key[j - 1], kb = key[j], ia = idx[j - 1], ib = idx[j];
            key[j - 1] = sw ? kb : ka;
            key[j] = sw ? ka : kb;
            idx[j - 1] = sw ? ib : ia;
            idx[j] = sw ? ia : ib;
        }
    }
    uint32_t p = 0; // this lane's cursor into its sorted list
#pragma unroll 1
    for (uint32_t r = 0; r < k; ++r) {
        uint32_t hk = 0, hi = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            hk = (p == (uint32_t)j) ? key[j] : hk;
            hi = (p == (uint32_t)j) ? idx[j] : hi;
        }
        const uint32_t best = wave_max_u32(hk);
        const uint64_t tied = __ballot(hk == best);
        uint32_t win_lane = (uint32_t)(__ffsll((unsigned long long)tied) - 1);
        uint32_t win_e = (uint32_t)__builtin_amdgcn_readlane((int)hi, (int)win_lane);
        if (__popcll(tied) > 1) { // exact tie across lanes: lowest index wins
            uint64_t rest = tied & (tied - 1ull);
            while (rest) {
                uint32_t l2 = (uint32_t)(__ffsll((unsigned long long)rest) - 1);
                rest &= rest - 1ull;
                uint32_t e2 = (uint32_t)__builtin_amdgcn_readlane((int)hi, (int)l2);
                if (e2 < win_e) {
                    win_e = e2;
                    win_lane = l2;
                }
            }
        }
        if ((uint32_t)lane == win_lane)
            ++p;
        out_e[r] = win_e;
    }
}

// ---------------------------------------------------------------------------
// routing of one token by one wave (math.rs:746-819 + expert_access.rs:80-135)
// ---------------------------------------------------------------------------
template <int EPL>
__device__ inline void route_token_wave(const float* __restrict__ l, const float* __restrict__ bias,
                                 const RouteParams& p, uint32_t* ids_out, float* w_out,
                                 uint32_t* lds_e, float* lds_grp, uint32_t* status)
{
    const int lane = threadIdx.x & 63;
    const uint32_t E = p.experts, K = p.k;
    float raw[EPL];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        uint32_t e = lane + WAVE * j;
        raw[j] = e < E ? l[e] : 0.0f;
        bad |= e < E && !isfinite(raw[j]);
    }
    if (__ballot(bad) != 0ull && lane == 0)
        atomicOr(status, ST_NONFINITE);

    float mx = 0.0f, inv_sum = 0.0f;
    bool have_inv = false;
    float sel[EPL];
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

    uint64_t keep = ~0ull;
    const uint32_t per = E / (p.n_group ? p.n_group : 1);
    if (p.kind == 2 && p.n_group > 1) {
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            if (lane + WAVE * j < E)
                lds_grp[lane + WAVE * j] = sel[j];
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        uint32_t gkey = 0;
        if ((uint32_t)lane < p.n_group) {
            uint32_t ka = 0, kb = 0;
            float a = -INFINITY, b = -INFINITY;
            for (uint32_t i = 0; i < per; ++i) {
                float v = lds_grp[lane * per + i];
                uint32_t kv = total_key(v);
                if (kv > ka) {
                    kb = ka, b = a;
                    ka = kv, a = v;
                } else if (kv > kb) {
                    kb = kv, b = v;
                }
            }
            gkey = total_key(per >= 2 ? a + b : a);
        }
        uint32_t gk[1] = {gkey};
        // group ranking: same canonical rule (score desc, lower index)
        wave_topk_canonical<1>(gk, p.topk_group, lds_e);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        keep = 0ull;
        for (uint32_t r = 0; r < p.topk_group; ++r)
            keep |= 1ull << lds_e[r];
    }

    uint32_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        uint32_t e = lane + WAVE * j;
        bool ok = e < E && ((keep >> (e / (per ? per : 1))) & 1ull);
        key[j] = ok ? total_key(sel[j]) : 0u;
    }

    if (p.order == 0) {
        wave_topk_canonical<EPL>(key, K, lds_e);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    } else {
        // replacement-slot scan of routing_top_k_iter; the scan state is
        // wave-uniform and only candidates above the current minimum are
        // visited, in index order
        float sv[MAX_K];
        uint32_t se[MAX_K];
#pragma unroll
        for (int s = 0; s < MAX_K; ++s)
            sv[s] = -INFINITY, se[s] = 0;
        uint32_t mi = 0;
        float mv = -INFINITY;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            uint32_t e = lane + WAVE * j;
            uint64_t cand = __ballot(e < E && sel[j] > mv);
            while (cand) {
                int src = __ffsll((unsigned long long)cand) - 1;
                cand &= cand - 1ull;
                float s = readlane_f(sel[j], src);
                if (s > mv) {
#pragma unroll
                    for (int c = 0; c < MAX_K; ++c)
                        if ((uint32_t)c == mi) {
                            sv[c] = s;
                            se[c] = (uint32_t)src + WAVE * j;
                        }
                    mi = 0;
                    mv = sv[0];
#pragma unroll
                    for (int c = 1; c < MAX_K; ++c)
                        if ((uint32_t)c < K && sv[c] < mv) {
                            mi = c;
                            mv = sv[c];
                        }
                }
            }
        }
#pragma unroll
        for (int s = 0; s < MAX_K; ++s)
            if ((uint32_t)s < K && lane == 0)
                lds_e[s] = se[s];
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }

    // value behind each selected id: lane r fetches route r's logit
    uint32_t myid = (uint32_t)lane < K ? lds_e[lane] : 0u;
    float v = (uint32_t)lane < K && myid < E ? l[myid] : 0.0f;
    float prob;
    if (p.kind == 0) {
        float ev = expf(v - mx);
        prob = have_inv ? ev * inv_sum : ev;
    } else {
        prob = sigmoidf_(v);
    }
    // sequential renormalisation in route order (lane 0 sums like the CPU)
    float sum = -0.0f;
    for (uint32_t r = 0; r < K; ++r)
        sum = sum + readlane_f(prob, (int)r);
    float inv;
    if (p.norm == 1) {
        if (lane == 0 && !(isfinite(sum) && sum >= 0.0f))
            atomicOr(status, ST_BAD_SUM);
        inv = 1.0f / fmaxf(sum, 6.103515625e-5f);
    } else {
        if (lane == 0 && !(isfinite(sum) && sum > 0.0f))
            atomicOr(status, ST_BAD_SUM);
        inv = 1.0f / sum;
    }
    if ((uint32_t)lane < K) {
        if (prob < 0.0f)
            atomicOr(status, ST_NEGATIVE);
        ids_out[lane] = myid;
        w_out[lane] = (prob * inv) * p.routed_scale;
    }
}

} // namespace pbmoe
