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
    static_assert(W == 2 || W == 4 || W == 8 || W == 16 || W == 32, "group width");
    v += dpp_f<DPP_QUAD_1032>(v);
    if constexpr (W >= 4)
        v += dpp_f<DPP_QUAD_2301>(v);
    if constexpr (W >= 8)
        v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    if constexpr (W >= 16)
        v += dpp_f<DPP_ROW_MIRROR>(v);
    if constexpr (W >= 32)
        v += __shfl_xor(v, 16);
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

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
    v = min(v, dpp_u<DPP_QUAD_1032>(v));
    v = min(v, dpp_u<DPP_QUAD_2301>(v));
    v = min(v, dpp_u<DPP_ROW_HALF_MIRROR>(v));
    v = min(v, dpp_u<DPP_ROW_MIRROR>(v));
    uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return min(min(a, b), min(c, d));
}

// f32 total order (Rust f32::total_cmp) mapped onto unsigned order.
__device__ __forceinline__ uint32_t total_key(float f)
{
    uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float sigmoidf_(float l) { return 1.0f / (1.0f + expf(-l)); }

// DeepSeek-V4 router probability sqrt(softplus(l)) in f32, softplus = l above
// 20, exp(l) below -20, log1p(exp(l)) between
// (deepseek_v4_router_probabilities, deepseek.rs:1300-1324)
__device__ __forceinline__ float sqrt_softplusf_(float l)
{
    const float sp = l > 20.0f ? l : (l < -20.0f ? expf(l) : log1pf(expf(l)));
    return sqrtf(sp);
}

// probability of the sigmoid-family routing kinds (1, 2: sigmoid; 3:
// sqrt-softplus); the selection score adds the per-expert bias when given
__device__ __forceinline__ float route_prob(uint32_t kind, float l)
{
    return kind == 3 ? sqrt_softplusf_(l) : sigmoidf_(l);
}
__device__ __forceinline__ float fast_sigmoid(float l) { return 1.0f / (1.0f + __expf(-l)); }

// a 16-bit scale/bias value (SBT 2: bf16, else f16) as f32
template <int SBT>
__device__ __forceinline__ float sb_bits(uint32_t v)
{
    if constexpr (SBT == 2)
        return __uint_as_float(v << 16);
    else
        return __half2float(__ushort_as_half((uint16_t)v));
}

template <int SBT>
__device__ __forceinline__ float sb_at(const uint8_t* base, uint64_t i)
{
    return sb_bits<SBT>(reinterpret_cast<const uint16_t*>(base)[i]);
}

// The 8 nibbles of a code word as floats, nibble j (columns j) in f[j]: the
// even and odd nibbles are masked into bytes, and each byte converts with
// one v_cvt_f32_ubyte{0..3} (2 + 8 instructions per word instead of a
// bit-field extract and a conversion per nibble).
__device__ __forceinline__ void q4_word_to_float(uint32_t q, float (&f)[8])
{
    uint32_t e = q & 0x0F0F0F0Fu, o = (q >> 4) & 0x0F0F0F0Fu;
    // opaque: otherwise the two masks fold into a 4-bit extract per nibble
    asm("" : "+v"(e), "+v"(o));
    f[0] = (float)(e & 0xFFu), f[2] = (float)((e >> 8) & 0xFFu);
    f[4] = (float)((e >> 16) & 0xFFu), f[6] = (float)(e >> 24);
    f[1] = (float)(o & 0xFFu), f[3] = (float)((o >> 8) & 0xFFu);
    f[5] = (float)((o >> 16) & 0xFFu), f[7] = (float)(o >> 24);
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
        float f[8];
        q4_word_to_float(words[i], f);
        qx0 = fmaf(f[0], a.x, qx0);
        qx1 = fmaf(f[1], a.y, qx1);
        qx0 = fmaf(f[2], a.z, qx0);
        qx1 = fmaf(f[3], a.w, qx1);
        qx0 = fmaf(f[4], b.x, qx0);
        qx1 = fmaf(f[5], b.y, qx1);
        qx0 = fmaf(f[6], b.z, qx0);
        qx1 = fmaf(f[7], b.w, qx1);
        sx += ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
    }
    xs = sx;
    return qx0 + qx1;
}

// sum(q * x) only (the sum of x is known).
__device__ __forceinline__ float q4_chunk_q(uint4 w, const float* __restrict__ x)
{
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float qx0 = 0.0f, qx1 = 0.0f;
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 a = x4[2 * i];
        const float4 b = x4[2 * i + 1];
        float f[8];
        q4_word_to_float(words[i], f);
        qx0 = fmaf(f[0], a.x, qx0);
        qx1 = fmaf(f[1], a.y, qx1);
        qx0 = fmaf(f[2], a.z, qx0);
        qx1 = fmaf(f[3], a.w, qx1);
        qx0 = fmaf(f[4], b.x, qx0);
        qx1 = fmaf(f[5], b.y, qx1);
        qx0 = fmaf(f[6], b.z, qx0);
        qx1 = fmaf(f[7], b.w, qx1);
    }
    return qx0 + qx1;
}

// Same with the 32 x values already in registers.  BYTES = false converts
// each nibble with its own bit-field extract: more instructions, fewer live
// registers (kernels holding many chunks of codes per lane keep their
// waves per SIMD).
template <bool BYTES = true>
__device__ __forceinline__ float q4_chunk_qx_reg(uint4 w, const float (&xv)[32])
{
    float qx0 = 0.0f, qx1 = 0.0f;
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (BYTES) {
            float f[8];
            q4_word_to_float(words[i], f);
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                qx0 = fmaf(f[j], xv[8 * i + j], qx0);
                qx1 = fmaf(f[j + 1], xv[8 * i + j + 1], qx1);
            }
        } else {
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
        uint32_t win_e;
        if (__popcll(tied) == 1) {
            win_e = (uint32_t)__builtin_amdgcn_readlane((int)hi, __ffsll((unsigned long long)tied) - 1);
        } else { // exact tie across lanes: lowest index wins (constant time)
            win_e = wave_min_u32(hk == best ? hi : 0xFFFFFFFFu);
        }
        if ((uint32_t)lane == (win_e & 63u))
            ++p;
        out_e[r] = win_e;
    }
}

// ---------------------------------------------------------------------------
// Faster canonical top-k for the common case.  The K-th largest lane maximum
// is a lower bound of the K-th largest element, so every member of the top-k
// has a key >= that bound.  When at most 64 elements pass the bound they are
// compacted one per lane (through LDS scratch of 64 entries) and K rounds of
// a wave max pick them in canonical order; otherwise the sorted-list
// selection above runs.  Both return the same ids.
// ---------------------------------------------------------------------------
template <int EPL>
__device__ __forceinline__ void wave_topk_filtered(uint32_t (&key)[EPL], uint32_t k, uint32_t* out_e,
                                                   uint32_t* scratch128)
{
    const int lane = threadIdx.x & 63;
    uint32_t head = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
        head = max(head, key[j]);
    // K-th largest lane head, by parallel ranking against broadcast LDS
    // reads: lane l holds it when #(heads > h_l) <= K-1 < #(heads >= h_l)
    scratch128[128 + lane] = head;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    uint32_t gt = 0, ge = 0;
    const uint4* hv4 = reinterpret_cast<const uint4*>(scratch128 + 128);
#pragma unroll
    for (int j = 0; j < WAVE / 4; ++j) {
        const uint4 h4 = hv4[j];
        gt += (h4.x > head ? 1u : 0u) + (h4.y > head ? 1u : 0u) + (h4.z > head ? 1u : 0u) + (h4.w > head ? 1u : 0u);
        ge += (h4.x >= head ? 1u : 0u) + (h4.y >= head ? 1u : 0u) + (h4.z >= head ? 1u : 0u) + (h4.w >= head ? 1u : 0u);
    }
    const uint64_t holds = __ballot(gt <= k - 1 && k - 1 < ge);
    const uint32_t bound = (uint32_t)__builtin_amdgcn_readlane((int)head, __ffsll((unsigned long long)holds) - 1);
    uint32_t total = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j)
        total += (uint32_t)__popcll(__ballot(key[j] >= bound && key[j] != 0u));
    if (total > 64u || bound == 0u || holds == 0ull) {
        wave_topk_canonical<EPL>(key, k, out_e);
        return;
    }
    // compact candidates one per lane
    uint32_t base = 0;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const bool c = key[j] >= bound && key[j] != 0u;
        const uint64_t b = __ballot(c);
        if (c) {
            const uint32_t pos = base + (uint32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
            scratch128[pos] = key[j];
            scratch128[64 + pos] = (uint32_t)lane + WAVE * j;
        }
        base += (uint32_t)__popcll(b);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const uint32_t ck = (uint32_t)lane < total ? scratch128[lane] : 0u;
    const uint32_t ci = (uint32_t)lane < total ? scratch128[64 + lane] : 0xFFFFFFFFu;
    // canonical rank among the candidates (score desc, then lower index),
    // candidates read back as broadcast LDS vectors
    uint32_t rank = 0;
    const uint4* k4 = reinterpret_cast<const uint4*>(scratch128);
    const uint4* i4 = reinterpret_cast<const uint4*>(scratch128 + 64);
    const uint32_t n4 = (total + 3) / 4;
    for (uint32_t j = 0; j < n4; ++j) {
        const uint4 kk = k4[j], ii = i4[j];
        const uint32_t kv[4] = {kk.x, kk.y, kk.z, kk.w}, iv[4] = {ii.x, ii.y, ii.z, ii.w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (4 * j + q < total)
                rank += (kv[q] > ck || (kv[q] == ck && iv[q] < ci)) ? 1u : 0u;
    }
    if ((uint32_t)lane < total && rank < k)
        out_e[rank] = ci;
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

    // raw logits of this token, for the value lookup after selection
#pragma unroll
    for (int j = 0; j < EPL; ++j)
        if (lane + WAVE * j < E)
            lds_grp[lane + WAVE * j] = raw[j];
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
                sm += __expf(raw[j] - mx);
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
            sel[j] = e < E ? route_prob(p.kind, raw[j]) + (bias ? bias[e] : 0.0f) : 0.0f;
        }
    }

    uint64_t keep = ~0ull;
    const uint32_t per = E / (p.n_group ? p.n_group : 1);
    float* grp_sel = lds_grp + E; // lds_grp holds 2*E floats
    if (p.kind == 2 && p.n_group > 1) {
#pragma unroll
        for (int j = 0; j < EPL; ++j)
            if (lane + WAVE * j < E)
                grp_sel[lane + WAVE * j] = sel[j];
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        uint32_t gkey = 0;
        if ((uint32_t)lane < p.n_group) {
            uint32_t ka = 0, kb = 0;
            float a = -INFINITY, b = -INFINITY;
            for (uint32_t i = 0; i < per; ++i) {
                float v = grp_sel[lane * per + i];
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
    const bool grouped = p.kind == 2 && p.n_group > 1;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const uint32_t e = lane + WAVE * j;
        bool ok = e < E;
        if (grouped)
            ok = ok && ((keep >> (e / per)) & 1ull);
        key[j] = ok ? total_key(sel[j]) : 0u;
    }

    if (p.order == 0) {
        wave_topk_filtered<EPL>(key, K, lds_e, reinterpret_cast<uint32_t*>(lds_grp) + 2 * E);
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
    float v = (uint32_t)lane < K && myid < E ? lds_grp[myid] : 0.0f;
    float prob;
    if (p.kind == 0) {
        float ev = expf(v - mx);
        prob = have_inv ? ev * inv_sum : ev;
    } else {
        prob = route_prob(p.kind, v);
    }
    // renormalisation over the K selected probabilities (lanes < K)
    const float sum = wave_sum((uint32_t)lane < K ? prob : 0.0f);
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

// ---------------------------------------------------------------------------
// Bitonic sorting across a wave, keys descending.  A key is 64-bit:
// total_key << 32 | ~index, so the order is score descending, then the lower
// index first (the canonical rule), and keys are distinct.
// ---------------------------------------------------------------------------
// the value of lane ^ J: DPP within rows of 16 lanes (row_shl:4 /
// row_shr:4 for 4, row_ror:8 for 8), a swizzle for 16, a permute for 32
template <int J>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v)
{
    if constexpr (J == 1)
        return dpp_u<DPP_QUAD_1032>(v);
    else if constexpr (J == 2)
        return dpp_u<DPP_QUAD_2301>(v);
    else if constexpr (J == 4) {
        // both moves in every lane: a DPP move reads its source lane only
        // where that lane is active, so neither may sit under the select
        const uint32_t up = dpp_u<0x104>(v), dn = dpp_u<0x114>(v);
        return (threadIdx.x & 4) ? dn : up;
    }
    else if constexpr (J == 8)
        return dpp_u<0x128>(v);
    else if constexpr (J == 16)
        return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F); // and 0x1f, xor 0x10
    else
        return (uint32_t)__shfl_xor((int)v, 32);
}

template <int J>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v)
{
    return ((uint64_t)xor_lane<J>((uint32_t)(v >> 32)) << 32) | xor_lane<J>((uint32_t)v);
}

// one merge stage (block size K2) of a 128-key sort, key i = element i & 1
// of lane i >> 1; distances J .. 1
template <int K2, int J>
__device__ __forceinline__ void bsort128_stage(uint64_t& a0, uint64_t& a1)
{
    const int lane = threadIdx.x & 63;
    if constexpr (J == 1) { // the lane's own pair
        const bool desc = ((2 * lane) & K2) == 0;
        const bool gt = a0 > a1;
        const uint64_t mx = gt ? a0 : a1, mn = gt ? a1 : a0;
        a0 = desc ? mx : mn;
        a1 = desc ? mn : mx;
    } else {
        constexpr int JL = J / 2; // lane distance
        const uint64_t o0 = xor_lane64<JL>(a0), o1 = xor_lane64<JL>(a1);
        const bool keep_max = ((lane & JL) == 0) == (((2 * lane) & K2) == 0);
        a0 = keep_max == (a0 > o0) ? a0 : o0;
        a1 = keep_max == (a1 > o1) ? a1 : o1;
        bsort128_stage<K2, J / 2>(a0, a1);
    }
}

// 128 keys of a wave (2 per lane) sorted descending: key i in element i & 1 of lane i >> 1
__device__ __forceinline__ void wave_sort128_desc(uint64_t& a0, uint64_t& a1)
{
    bsort128_stage<2, 1>(a0, a1);
    bsort128_stage<4, 2>(a0, a1);
    bsort128_stage<8, 4>(a0, a1);
    bsort128_stage<16, 8>(a0, a1);
    bsort128_stage<32, 16>(a0, a1);
    bsort128_stage<64, 32>(a0, a1);
    bsort128_stage<128, 64>(a0, a1);
}

template <int K2, int J>
__device__ __forceinline__ void bsort64_stage(uint64_t& a)
{
    const int lane = threadIdx.x & 63;
    const uint64_t o = xor_lane64<J>(a);
    const bool keep_max = ((lane & J) == 0) == ((lane & K2) == 0);
    a = keep_max == (a > o) ? a : o;
    if constexpr (J > 1)
        bsort64_stage<K2, J / 2>(a);
}

// 64 keys of a wave (one per lane) sorted descending across the lanes
__device__ __forceinline__ void wave_sort64_desc(uint64_t& a)
{
    bsort64_stage<2, 1>(a);
    bsort64_stage<4, 2>(a);
    bsort64_stage<8, 4>(a);
    bsort64_stage<16, 8>(a);
    bsort64_stage<32, 16>(a);
    bsort64_stage<64, 32>(a);
}

// ---------------------------------------------------------------------------
// routing of one token by a whole 256-thread workgroup (canonical order,
// softmax or ungrouped sigmoid): each wave takes the canonical top-K of its
// quarter of the experts (K rounds of a wave max over per-thread sorted
// heads), then wave 0 merges the <= 4K candidates, one per lane.  Same
// selection rule (score desc, lower index) and value arithmetic as
// route_token_wave; every thread of the workgroup must call it.  need_w
// false (the same in every thread): the ids only, no softmax sums, weights
// or weight checks (callers that publish no weights).
// lds: >= 1024 + 8 + 144 floats of workgroup scratch, 8-byte aligned (64-bit
// keys are stored at lds + 512 and lds + 1032).
// ---------------------------------------------------------------------------
template <int EPT>
__device__ inline void route_token_block(const float* __restrict__ l, const float* __restrict__ bias,
                                         const RouteParams& p, uint32_t* ids_out, float* w_out, float* lds,
                                         uint32_t* status, bool need_w = true)
{
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t E = p.experts, K = p.k;
    float* raw_l = lds;                                         // [E <= 1024]
    float* red = lds + 1024;                                    // [8]
    uint32_t* cand_k = reinterpret_cast<uint32_t*>(lds + 1032); // [4][16]
    uint32_t* cand_i = cand_k + 64;                             // [4][16]
    float raw[EPT];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const uint32_t e = tid + 256 * j;
        raw[j] = e < E ? l[e] : 0.0f;
        bad |= e < E && !isfinite(raw[j]);
        if (e < E)
            raw_l[e] = raw[j];
    }
    if (__ballot(bad) != 0ull && lane == 0)
        atomicOr(status, ST_NONFINITE);
    float mx = 0.0f;
    float sel[EPT];
    if (p.kind == 0 && need_w) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (tid + 256 * j < E)
                m = fmaxf(m, raw[j]);
        m = wave_max(m);
        if (lane == 0)
            red[wv] = m;
        __syncthreads();
        mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        float sm = 0.0f;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (tid + 256 * j < E)
                sm += __expf(raw[j] - mx);
        sm = wave_sum(sm);
        if (lane == 0)
            red[4 + wv] = sm;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            sel[j] = raw[j];
    } else if (p.kind == 0) { // selection only: softmax is monotonic, select on the logits
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            sel[j] = raw[j];
    } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const uint32_t e = tid + 256 * j;
            sel[j] = e < E ? route_prob(p.kind, raw[j]) + (bias ? bias[e] : 0.0f) : 0.0f;
        }
    }
    uint32_t myid = 0;
    if constexpr (EPT <= 2) {
        // E <= 512: keys above a threshold (below), else each wave sorts its
        // 128 keys (bitonic, across lanes by DPP), writes its top 16, and
        // wave 0 sorts the 64 candidates; lane r < K then holds the r-th
        // selected expert.  Same rule as the rounds below.
        uint64_t c2[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t e = tid + 256 * j;
            const uint32_t kj = j < EPT && e < E ? total_key(sel[j < EPT ? j : 0]) : 0u;
            c2[j] = ((uint64_t)kj << 32) | (uint32_t)~e;
        }
        uint64_t* cand = reinterpret_cast<uint64_t*>(cand_k); // [64]
        bool done = false;
        if (K <= 16) {
            // Threshold first: the 16 groups of 16 threads (32 keys each)
            // publish their maxima; tau, the K-th largest of them, is at most
            // the K-th largest key (K distinct keys are >= tau), so the keys
            // >= tau hold the top K.  They are few for any spread of scores:
            // when they fit one wave (64), wave 0 ranks just them.
            uint64_t* gmax = reinterpret_cast<uint64_t*>(lds + 512);  // [16] (raw_l holds E <= 512)
            uint32_t* ncand = reinterpret_cast<uint32_t*>(lds + 544); // candidate count
            uint64_t gm = c2[0] > c2[1] ? c2[0] : c2[1];
            uint64_t o = xor_lane64<1>(gm);
            gm = o > gm ? o : gm;
            o = xor_lane64<2>(gm);
            gm = o > gm ? o : gm;
            o = xor_lane64<4>(gm);
            gm = o > gm ? o : gm;
            o = xor_lane64<8>(gm);
            gm = o > gm ? o : gm;
            if ((lane & 15) == 0)
                gmax[wv * 4 + (lane >> 4)] = gm;
            if (tid == 0)
                *ncand = 0;
            __syncthreads();
            // the maxima are distinct (distinct keys): one rank K - 1 among them
            const uint64_t v = gmax[lane & 15];
            uint32_t above = 0;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                above += gmax[j] > v ? 1u : 0u;
            const uint64_t hit = __ballot(above == K - 1);
            const int src = __ffsll((unsigned long long)hit) - 1;
            const uint64_t tau = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), src) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, src);
            const bool f0 = c2[0] >= tau, f1 = c2[1] >= tau;
            const uint64_t b0 = __ballot(f0), b1 = __ballot(f1);
            const uint32_t n0 = (uint32_t)__popcll(b0), nw = n0 + (uint32_t)__popcll(b1);
            uint32_t base = 0;
            if (lane == 0)
                base = atomicAdd(ncand, nw);
            base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
            const uint32_t p0 = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(b0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b0, 0u));
            const uint32_t p1 = base + n0 + __builtin_amdgcn_mbcnt_hi((uint32_t)(b1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b1, 0u));
            if (f0 && p0 < 64)
                cand[p0] = c2[0];
            if (f1 && p1 < 64)
                cand[p1] = c2[1];
            __syncthreads();
            const uint32_t n = *ncand;
            if (n <= 64) {
                if (wv != 0)
                    return;
                // the keys are distinct: a candidate's rank is the number of
                // larger keys, counted over the candidates read from LDS as
                // broadcasts (n steps; a bitonic sort of 64 lanes took
                // 1,900 cycles, the largest part of the routing); the K
                // first land in rank order, lane r then holds the r-th
                const uint64_t c = (uint32_t)lane < n ? cand[lane] : 0ull;
                uint32_t rank = 0;
                for (uint32_t j = 0; j < n; ++j)
                    rank += cand[j] > c ? 1u : 0u;
                uint32_t* sel = reinterpret_cast<uint32_t*>(cand); // the candidates are read
                if ((uint32_t)lane < n && rank < K)
                    sel[rank] = ~(uint32_t)c;
                myid = (uint32_t)lane < K ? sel[lane] : 0u;
                done = true;
            }
        }
        if (!done) { // every wave sorts its 128 keys, wave 0 sorts the 4 x 16 heads
            wave_sort128_desc(c2[0], c2[1]);
            if (lane < 8) {
                cand[wv * 16 + 2 * lane] = c2[0];
                cand[wv * 16 + 2 * lane + 1] = c2[1];
            }
            __syncthreads();
            if (wv != 0)
                return;
            uint64_t c = (uint32_t)(lane & 15) < K ? cand[(lane >> 4) * 16 + (lane & 15)] : 0ull;
            wave_sort64_desc(c);
            myid = ~(uint32_t)c;
        }
    } else {
    // per-thread keys sorted descending (ascending index on equal keys)
    uint32_t key[EPT], idx[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const uint32_t e = tid + 256 * j;
        key[j] = e < E ? total_key(sel[j]) : 0u;
        idx[j] = e;
    }
#pragma unroll
    for (int i = 1; i < EPT; ++i)
#pragma unroll
        for (int j = i; j > 0; --j) {
            const bool sw = key[j] > key[j - 1];
            const uint32_t ka = key[j - 1], kb2 = key[j], ia = idx[j - 1], ib = idx[j];
            key[j - 1] = sw ? kb2 : ka, key[j] = sw ? ka : kb2;
            idx[j - 1] = sw ? ib : ia, idx[j] = sw ? ia : ib;
        }
    // K rounds per wave over the heads
    uint32_t ptr = 0;
    for (uint32_t r = 0; r < K; ++r) {
        uint32_t hk = 0, hi = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if ((uint32_t)j == ptr)
                hk = key[j], hi = idx[j];
        const uint32_t best = wave_max_u32(hk);
        const uint64_t tied = __ballot(hk == best);
        uint32_t win;
        if (__popcll(tied) == 1)
            win = (uint32_t)__builtin_amdgcn_readlane((int)hi, __ffsll((unsigned long long)tied) - 1);
        else // exact tie between heads: the lower index first
            win = wave_min_u32(hk == best ? hi : 0xFFFFFFFFu);
        if (hk == best && hi == win)
            ++ptr;
        if (lane == 0) {
            cand_k[wv * 16 + r] = best;
            cand_i[wv * 16 + r] = win;
        }
    }
    __syncthreads();
    if (wv != 0)
        return;
    // merge: candidate (wave w, rank r) on lane w * K + r
    const uint32_t n = 4 * K;
    uint32_t ck = 0, ci = 0xFFFFFFFFu;
    if ((uint32_t)lane < n) {
        const uint32_t w = (uint32_t)lane / K, r = (uint32_t)lane % K;
        ck = cand_k[w * 16 + r];
        ci = cand_i[w * 16 + r];
    }
    for (uint32_t r = 0; r < K; ++r) {
        const uint32_t best = wave_max_u32(ck);
        const uint64_t tied = __ballot(ck == best);
        uint32_t win;
        if (__popcll(tied) == 1)
            win = (uint32_t)__builtin_amdgcn_readlane((int)ci, __ffsll((unsigned long long)tied) - 1);
        else
            win = wave_min_u32(ck == best ? ci : 0xFFFFFFFFu);
        if (ck == best && ci == win)
            ck = 0u;
        if ((uint32_t)lane == r)
            myid = win;
    }
    }
    if (!need_w) { // the ids only (the caller publishes no weights)
        if ((uint32_t)lane < K)
            ids_out[lane] = myid;
        return;
    }
    // value behind each selected id, renormalisation (as route_token_wave)
    const float v = (uint32_t)lane < K && myid < E ? raw_l[myid] : 0.0f;
    float prob;
    if (p.kind == 0) {
        const float sum = (red[4] + red[5]) + (red[6] + red[7]);
        const bool have_inv = sum > 0.0f && isfinite(sum);
        const float ev = expf(v - mx);
        prob = have_inv ? ev * (1.0f / sum) : ev;
    } else {
        prob = route_prob(p.kind, v);
    }
    const float sum = wave_sum((uint32_t)lane < K ? prob : 0.0f);
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
