// Batch-1 decode of the whole MoE layer in ONE persistent launch on gfx950.
//
// Every workgroup of the grid is resident at once (the host sizes the grid
// to at most one workgroup per CU) and the phases hand data to each other
// through tagged 64-bit words instead of kernel boundaries:
//
//   low 32 bits  = the value (f32 bits)
//   high 32 bits = the call's tag (epoch + 1; the epoch lives in device
//                  memory and advances once per call)
//
// Each word is written by one relaxed agent-scope 64-bit atomic store and
// read by agent-scope atomic loads (global_store/load_dwordx2 sc1: coherent
// across the eight XCD L2s), so a reader sees either an older call's word
// (old tag: not ready) or the complete new one.  A producing workgroup
// raises one tagged "done" flag after its words; consumers poll the flags
// (few words, with a growing pause) and then read the data once, so polling
// stays light while other workgroups still stream weights.  Every wait is
// bounded (spin_max rounds): one that runs out sets ST_TIMEOUT and the
// workgroup carries on, so every wave always exits.
//
// Work of workgroup b:
//   1. router rows (one wave per row) and the shared sigmoid gate row, as
//      tagged logits;
//   2. gate/up unit b = (route slot k or the shared expert, 32 intermediate
//      rows): SiLU(g)*u of its rows, as tagged activations.  The shared
//      expert's units start at once; the routed units wait for the logits
//      and route the token (every workgroup routes: the same ids and
//      weights everywhere);
//   3. output rows [b R, b R + R) of every expert's down projection: the
//      weight rows are loaded right after routing (contiguous 16-byte lane
//      loads), the activations of all experts are gathered once, and the
//      combine h = (r + sum_k w_k y_k) + sigma(g) * S runs in route order
//      for those rows.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "pbmoe_device.h"
#include "pbmoe_internal.h"

namespace pbmoe {

namespace {

constexpr int PT = 256;        // threads per workgroup
constexpr int CHUNK = 32;      // intermediate rows per gate/up unit
constexpr int XPAD = 36;       // LDS stride of a 32-float activation chunk (bank spread)
constexpr int MAX_ACT = 8192;  // activations gathered per workgroup (items x I)
constexpr int MAX_ROWS = 64;   // combine rows per workgroup

__device__ __forceinline__ uint64_t tagged(uint32_t tag, float v)
{
    return ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}

__device__ __forceinline__ void publish(uint64_t* p, uint32_t tag, float v)
{
    __hip_atomic_store(p, tagged(tag, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t peek(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Pause between polls, growing with the number of unsuccessful rounds.
__device__ __forceinline__ void backoff(uint32_t round)
{
    const uint32_t n = round < 4 ? 1u : (round < 12 ? 2u : 4u);
    for (uint32_t i = 0; i < n; ++i)
        __builtin_amdgcn_s_sleep(4);
}

// This workgroup's tagged stores are done: every wave waits for its stores
// to complete, then one thread raises `flag`.  (The data words keep their
// own tags, so a word not yet visible when its flag is seen is polled again.)
__device__ __forceinline__ void publish_done(uint64_t* flag, uint32_t tag)
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        publish(flag, tag, 1.0f);
}

// Waits for the tagged words src(i), i in [0, n), this thread's share being
// i = base + tid + PT*j; writes their values to dst(i).  All loads of a
// batch are in flight together; only stale words are loaded again.
template <int NB, typename Src, typename Dst>
__device__ void wait_words(Src src, uint32_t n, uint32_t tag, Dst dst, uint32_t spin_max, uint32_t* status)
{
    const uint32_t tid = threadIdx.x;
    for (uint32_t base = 0; base < n; base += PT * NB) {
        uint64_t w[NB];
        uint32_t pending = 0;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t i = base + tid + PT * j;
            w[j] = 0;
            if (i < n) {
                w[j] = peek(src(i));
                pending |= 1u << j;
            }
        }
        uint32_t spins = 0;
        while (true) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                if (((pending >> j) & 1u) && (uint32_t)(w[j] >> 32) == tag) {
                    dst(base + tid + PT * j) = __uint_as_float((uint32_t)w[j]);
                    pending &= ~(1u << j);
                }
            }
            if (!pending)
                break;
            if (++spins > spin_max) {
                atomicOr(status, ST_TIMEOUT);
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    if ((pending >> j) & 1u)
                        dst(base + tid + PT * j) = 0.0f;
                break;
            }
            backoff(spins);
#pragma unroll
            for (int j = 0; j < NB; ++j)
                if ((pending >> j) & 1u)
                    w[j] = peek(src(base + tid + PT * j));
        }
    }
}

// 32 consecutive 16-bit dense weights of a row -> floats
template <int WDT>
__device__ __forceinline__ void dense32(const void* row, uint32_t col, float (&v)[32])
{
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(row) + col);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 r = p[q];
        const uint32_t r4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (WDT == 2) {
                v[8 * q + 2 * i] = __uint_as_float(r4[i] << 16);
                v[8 * q + 2 * i + 1] = __uint_as_float(r4[i] & 0xFFFF0000u);
            } else {
                v[8 * q + 2 * i] = __half2float(__ushort_as_half((uint16_t)(r4[i] & 0xFFFFu)));
                v[8 * q + 2 * i + 1] = __half2float(__ushort_as_half((uint16_t)(r4[i] >> 16)));
            }
        }
    }
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c)
{
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, a), __builtin_bit_cast(half2v, b), c, false);
}

__device__ __forceinline__ uint32_t h2bits(_Float16 a, _Float16 b)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// x of this lane's 32 columns as f16 hi + lo pairs in the nibble pairing
// order of a packed word: pair j of word q is (x[8q+j], x[8q+j+4]); hi =
// f16(x), lo = f16(x - hi), so hi + lo carries 22 significant bits.  x is
// first scaled by 2^-e (exact) so that every |x| fits the f16 range; sums of
// the hi and lo parts serve the 1024-offset correction below.
struct XF16 {
    uint32_t hi[16], lo[16];
    float shi, slo; // sums of the scaled hi and lo parts
    float scale;    // 2^e: multiply the scaled dot products back
    bool any_lo;    // some lo part is not zero (wave-uniform)
};

__device__ __forceinline__ void split_x(const float (&xv)[32], XF16& o)
{
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
        m = fmaxf(m, fabsf(xv[i]));
    m = wave_max(m);
    // largest |x| below 2^15 after scaling, so hi never overflows f16
    int e = 0;
    if (m >= 32768.0f)
        e = ilogbf(m) - 14;
    const float down = ldexpf(1.0f, -e);
    o.scale = ldexpf(1.0f, e);
    float shi = 0.0f, slo = 0.0f;
    bool lo_any = false;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = xv[8 * q + j] * down, b = xv[8 * q + j + 4] * down;
            const _Float16 ah = (_Float16)a, bh = (_Float16)b;
            const float ar = a - (float)ah, br = b - (float)bh;
            const _Float16 al = (_Float16)ar, bl = (_Float16)br;
            o.hi[4 * q + j] = h2bits(ah, bh);
            o.lo[4 * q + j] = h2bits(al, bl);
            shi += (float)ah + (float)bh;
            slo += (float)al + (float)bl;
            lo_any |= (ar != 0.0f) || (br != 0.0f);
        }
    }
    o.shi = shi;
    o.slo = slo;
    o.any_lo = __ballot(lo_any) != 0ull;
}

// sum over the 32 columns of a 16-byte code chunk of q * xs (xs = scaled x):
// the nibbles become the f16 values 1024 + q (exact), paired like the x
// pairs, dotted by v_dot2_f32_f16 into f32; the 1024 * sum(x) term is
// removed afterwards.  Returns sum(q * x) (unscaled).
__device__ __forceinline__ float q4_dot_f16(uint4 w, const XF16& x)
{
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    float h0 = 0.0f, h1 = 0.0f, l0 = 0.0f, l1 = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t v = wd[q];
        const uint32_t p0 = (v & 0x000F000Fu) | 0x64006400u;
        const uint32_t p1 = ((v >> 4) & 0x000F000Fu) | 0x64006400u;
        const uint32_t p2 = ((v >> 8) & 0x000F000Fu) | 0x64006400u;
        const uint32_t p3 = ((v >> 12) & 0x000F000Fu) | 0x64006400u;
        h0 = dot2(p0, x.hi[4 * q], h0);
        h1 = dot2(p1, x.hi[4 * q + 1], h1);
        h0 = dot2(p2, x.hi[4 * q + 2], h0);
        h1 = dot2(p3, x.hi[4 * q + 3], h1);
        if (x.any_lo) {
            l0 = dot2(p0, x.lo[4 * q], l0);
            l1 = dot2(p1, x.lo[4 * q + 1], l1);
            l0 = dot2(p2, x.lo[4 * q + 2], l0);
            l1 = dot2(p3, x.lo[4 * q + 3], l1);
        }
    }
    const float hs = (h0 + h1) - 1024.0f * x.shi;
    const float ls = x.any_lo ? (l0 + l1) - 1024.0f * x.slo : 0.0f;
    return (hs + ls) * x.scale;
}

// f16 dense row chunk (32 weights, natural order in 4 x 16 bytes) . x
template <int WDT>
__device__ __forceinline__ float dense_dot(const void* row, uint32_t col, const XF16& x, const float (&xv)[32])
{
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(row) + col);
    if constexpr (WDT == 1) {
        float h0 = 0.0f, h1 = 0.0f, l0 = 0.0f, l1 = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 r = p[q]; // (c0,c1) (c2,c3) (c4,c5) (c6,c7)
            const uint32_t w0 = __builtin_amdgcn_perm(r.z, r.x, 0x05040100u); // (c0, c4)
            const uint32_t w1 = __builtin_amdgcn_perm(r.z, r.x, 0x07060302u); // (c1, c5)
            const uint32_t w2 = __builtin_amdgcn_perm(r.w, r.y, 0x05040100u); // (c2, c6)
            const uint32_t w3 = __builtin_amdgcn_perm(r.w, r.y, 0x07060302u); // (c3, c7)
            h0 = dot2(w0, x.hi[4 * q], h0);
            h1 = dot2(w1, x.hi[4 * q + 1], h1);
            h0 = dot2(w2, x.hi[4 * q + 2], h0);
            h1 = dot2(w3, x.hi[4 * q + 3], h1);
            if (x.any_lo) {
                l0 = dot2(w0, x.lo[4 * q], l0);
                l1 = dot2(w1, x.lo[4 * q + 1], l1);
                l0 = dot2(w2, x.lo[4 * q + 2], l0);
                l1 = dot2(w3, x.lo[4 * q + 3], l1);
            }
        }
        return ((h0 + h1) + (l0 + l1)) * x.scale;
    } else {
        float wv32[32];
        dense32<WDT>(row, col, wv32);
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i += 2) {
            acc0 = fmaf(wv32[i], xv[i], acc0);
            acc1 = fmaf(wv32[i + 1], xv[i + 1], acc1);
        }
        return acc0 + acc1;
    }
}

struct Shared {
    float lg[1024 + 8];          // routing: the token's logits
    alignas(16) float rgrp[2048 + 192 + 16]; // routing scratch (route_token_wave / route_token_block)
    alignas(16) uint32_t heads[PT]; // fast top-k: per-thread best key
    alignas(16) uint32_t ck[64]; // fast top-k: candidates (keys, ids)
    alignas(16) uint32_t ci[64];
    uint32_t ncand, bound;
    float red[8];                // block reductions
    uint32_t sel[MAX_K];
    uint32_t ids[MAX_K];
    float w[MAX_K];
    float act_u[CHUNK];          // this unit's activations
    float part[4];
    alignas(16) float actx[MAX_ACT / 32 * XPAD]; // all experts' activations, chunk q at q * XPAD
    float yk[MAX_K + 1][MAX_ROWS];   // per item and combine row: the item's down output
    float misc[4];               // [0] shared gate logit
};

// Canonical top-K (score desc, then lower index) of E <= 1024 selection keys
// held four per thread (expert tid + 256 j), by a threshold: the K-th
// largest per-thread maximum bounds the K-th largest key from below, so the
// top K are among the keys >= that bound; those (at most 64, else false is
// returned and the caller falls back) are ranked by one wave.  Writes sh.sel.
__device__ bool block_topk_threshold(const uint32_t (&key)[4], uint32_t K, Shared& sh)
{
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    uint32_t head = max(max(key[0], key[1]), max(key[2], key[3]));
    sh.heads[tid] = head;
    if (tid == 0) {
        sh.ncand = 0;
        sh.bound = 0;
    }
    __syncthreads();
    uint32_t gt = 0, ge = 0;
    const uint4* h4 = reinterpret_cast<const uint4*>(sh.heads);
#pragma unroll 8
    for (int q = 0; q < PT / 4; ++q) {
        const uint4 v = h4[q];
        gt += (v.x > head ? 1u : 0u) + (v.y > head ? 1u : 0u) + (v.z > head ? 1u : 0u) + (v.w > head ? 1u : 0u);
        ge += (v.x >= head ? 1u : 0u) + (v.y >= head ? 1u : 0u) + (v.z >= head ? 1u : 0u) + (v.w >= head ? 1u : 0u);
    }
    if (gt <= K - 1 && K - 1 < ge) // every holder has the same head: the K-th largest
        sh.bound = head;
    __syncthreads();
    const uint32_t bound = sh.bound;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (bound != 0u && key[j] >= bound) {
            const uint32_t pos = atomicAdd(&sh.ncand, 1u);
            if (pos < 64) {
                sh.ck[pos] = key[j];
                sh.ci[pos] = tid + PT * j;
            }
        }
    }
    __syncthreads();
    const uint32_t n = sh.ncand;
    if (n > 64 || bound == 0u)
        return false;
    if (tid < 64) {
        if (lane >= n) { // pad to a multiple of 4 with entries that rank last
            sh.ck[lane] = 0u;
            sh.ci[lane] = 0xFFFFFFFFu;
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const uint32_t mk = sh.ck[lane], mi = sh.ci[lane];
        uint32_t rank = 0;
        const uint4* k4 = reinterpret_cast<const uint4*>(sh.ck);
        const uint4* i4 = reinterpret_cast<const uint4*>(sh.ci);
#pragma unroll
        for (int q = 0; q < 16; ++q) { // broadcast reads, all issued together
            const uint4 kk = k4[q], ii = i4[q];
            rank += (kk.x > mk || (kk.x == mk && ii.x < mi)) ? 1u : 0u;
            rank += (kk.y > mk || (kk.y == mk && ii.y < mi)) ? 1u : 0u;
            rank += (kk.z > mk || (kk.z == mk && ii.z < mi)) ? 1u : 0u;
            rank += (kk.w > mk || (kk.w == mk && ii.w < mi)) ? 1u : 0u;
        }
        if (lane < n && rank < K)
            sh.sel[rank] = mi;
    }
    __syncthreads();
    return true;
}

// Routing of the token from sh.lg (softmax or ungrouped sigmoid /
// sqrt-softplus kinds, canonical order): ids and renormalised weights into
// sh.ids / sh.w, the arithmetic of route_token_block.  False: the fast
// selection declined (many exact ties); nothing was written.
__device__ bool route_fast(const RouteParams& p, const float* __restrict__ bias, Shared& sh, uint32_t* status)
{
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
    const uint32_t E = p.experts, K = p.k;
    float raw[4], sel[4];
    uint32_t key[4];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = tid + PT * j;
        raw[j] = e < E ? sh.lg[e] : 0.0f;
        bad |= e < E && !isfinite(raw[j]);
    }
    if (__ballot(bad) != 0ull && lane == 0)
        atomicOr(status, ST_NONFINITE);
    float mx = 0.0f;
    if (p.kind == 0) {
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (tid + PT * j < E)
                m = fmaxf(m, raw[j]);
        m = wave_max(m);
        if (lane == 0)
            sh.red[wv] = m;
        __syncthreads();
        mx = fmaxf(fmaxf(sh.red[0], sh.red[1]), fmaxf(sh.red[2], sh.red[3]));
        float sm = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (tid + PT * j < E)
                sm += __expf(raw[j] - mx);
        sm = wave_sum(sm);
        if (lane == 0)
            sh.red[4 + wv] = sm;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            sel[j] = raw[j];
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = tid + PT * j;
            sel[j] = e < E ? route_prob(p.kind, raw[j]) + (bias ? bias[e] : 0.0f) : 0.0f;
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        key[j] = tid + PT * j < E ? total_key(sel[j]) : 0u;
    if (!block_topk_threshold(key, K, sh))
        return false;
    if (wv == 0) {
        const uint32_t myid = lane < K ? sh.sel[lane] : 0u;
        const float v = lane < K && myid < E ? sh.lg[myid] : 0.0f;
        float prob;
        if (p.kind == 0) {
            const float sum = (sh.red[4] + sh.red[5]) + (sh.red[6] + sh.red[7]);
            const bool have_inv = sum > 0.0f && isfinite(sum);
            const float ev = expf(v - mx);
            prob = have_inv ? ev * (1.0f / sum) : ev;
        } else {
            prob = route_prob(p.kind, v);
        }
        const float s = wave_sum(lane < K ? prob : 0.0f);
        float inv;
        if (p.norm == 1) {
            if (lane == 0 && !(isfinite(s) && s >= 0.0f))
                atomicOr(status, ST_BAD_SUM);
            inv = 1.0f / fmaxf(s, 6.103515625e-5f);
        } else {
            if (lane == 0 && !(isfinite(s) && s > 0.0f))
                atomicOr(status, ST_BAD_SUM);
            inv = 1.0f / s;
        }
        if (lane < K) {
            if (prob < 0.0f)
                atomicOr(status, ST_NEGATIVE);
            sh.ids[lane] = myid;
            sh.w[lane] = (prob * inv) * p.routed_scale;
        }
    }
    __syncthreads();
    return true;
}

} // namespace

// Fields of one expert set the kernel reads, by value (no reference to the
// kernel-argument struct, which would force it into scratch memory).
struct SetView {
    const uint8_t* base;
    uint64_t stride;
    uint64_t gw, gs, gb, uw, us, ub, dw, ds, db; // component offsets
    uint32_t count, gshift;
};

__device__ __forceinline__ SetView view_of(const ExpertSet& s)
{
    return SetView{s.base, s.stride, s.gate.w_off, s.gate.s_off, s.gate.b_off, s.up.w_off, s.up.s_off,
                   s.up.b_off, s.down.w_off, s.down.s_off, s.down.b_off, s.count, s.group_shift};
}

// LPR lanes per (item, output row), CPD 32-column chunks per lane
// (I = 32 LPR CPD); NP passes of PT / LPR (item, row) pairs.
template <int SBT, int WDT, int LPR, int CPD, int NP>
__global__ __launch_bounds__(PT) void persist_decode_kernel(PersistArgs a)
{
    __shared__ Shared sh;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
    const uint32_t b = blockIdx.x;
    const uint32_t H = a.hidden, E = a.rp.experts, K = a.rp.k;
    const uint32_t NW = gridDim.x;
    constexpr uint32_t I = 32u * LPR * CPD;
    constexpr uint32_t NCI = I / CHUNK; // units per expert
    const RouteParams rp = a.rp;
    const SetView ex = view_of(a.ex), sx = view_of(a.sh);
    const bool has_shared = a.has_shared != 0u, full = a.full != 0u;
    const float* __restrict__ in_norm_w = a.in_norm_w;
    const uint32_t spin_max = a.spin_max;
    uint32_t* const status = a.status;
    uint64_t* const tl = a.tl;
    uint64_t* const ta = a.ta;
    uint64_t* const tn = a.tn;
    uint64_t* const tfr = a.tfr;
    uint64_t* const tfu = a.tfu;
    uint64_t* const arrive = a.arrive;
    const uint32_t tag = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if (tid == 0)
        publish(arrive + b, tag, 0.0f);

    // x (or x * norm weight) for this lane's columns [32 lane, 32 lane + 32),
    // their sum, and (fused input norm) 1 / rms(x)
    float xv[32];
    float ss = 0.0f;
    {
        const uint32_t col = 32u * lane;
        const float4* xp = reinterpret_cast<const float4*>(a.x + col);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 f = xp[q];
            xv[4 * q] = f.x, xv[4 * q + 1] = f.y, xv[4 * q + 2] = f.z, xv[4 * q + 3] = f.w;
        }
        if (in_norm_w) {
            const float4* wp = reinterpret_cast<const float4*>(in_norm_w + col);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 f = wp[q];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ss = fmaf(xv[4 * q + i], xv[4 * q + i], ss);
                xv[4 * q] *= f.x, xv[4 * q + 1] *= f.y, xv[4 * q + 2] *= f.z, xv[4 * q + 3] *= f.w;
            }
        }
    }
    float xsum = 0.0f;
#pragma unroll
    for (int q = 0; q < 32; q += 4)
        xsum += (xv[q] + xv[q + 1]) + (xv[q + 2] + xv[q + 3]);
    float inv_rms = 1.0f;
    if (in_norm_w) // every wave holds all of x: the same sum in every wave
        inv_rms = 1.0f / sqrtf(wave_sum(ss) / (float)H + a.eps);
    XF16 xf;
    split_x(xv, xf);

    // combine rows of this workgroup and their residuals
    const uint32_t RPW = a.rpw;
    const uint32_t h0 = b * RPW;
    const uint32_t nrows = h0 < H ? min(RPW, H - h0) : 0u;
    float resid = 0.0f;
    if (tid < nrows)
        resid = a.residual[h0 + tid];

    const uint32_t items = K + (has_shared ? 1u : 0u);
    const uint32_t NU = a.nunits;
    const bool has_unit = b < NU;
    const uint32_t item = b / NCI, chunk = b % NCI;
    const bool shared_unit = has_unit && has_shared && item == K;

    // ---- gate/up unit: rows 32 chunk + [0, 32), 8 gate + 8 up rows per wave
    constexpr int RW = 8;
    uint4 wg[RW], wu[RW];
    float sg[RW], bg[RW], su[RW], bu[RW];
#define PBM_UNIT_LOAD(V, SLOT)                                                                \
    do {                                                                                      \
        const uint32_t gpr = H >> (V).gshift;                                                 \
        const uint32_t r0 = chunk * CHUNK + wv * RW;                                          \
        _Pragma("unroll") for (int r = 0; r < RW; ++r) {                                      \
            const uint32_t row = r0 + r;                                                      \
            wg[r] = reinterpret_cast<const uint4*>((SLOT) + (V).gw + (uint64_t)row * (H / 2))[lane]; \
            wu[r] = reinterpret_cast<const uint4*>((SLOT) + (V).uw + (uint64_t)row * (H / 2))[lane]; \
            const uint64_t gi = (uint64_t)row * gpr + ((lane * 32u) >> (V).gshift);           \
            sg[r] = sb_at<SBT>((SLOT) + (V).gs, gi);                                          \
            bg[r] = sb_at<SBT>((SLOT) + (V).gb, gi);                                          \
            su[r] = sb_at<SBT>((SLOT) + (V).us, gi);                                          \
            bu[r] = sb_at<SBT>((SLOT) + (V).ub, gi);                                          \
        }                                                                                     \
    } while (0)
#define PBM_UNIT_FINISH(U)                                                                    \
    do {                                                                                      \
        _Pragma("unroll") for (int r = 0; r < RW; ++r) {                                      \
            const float qg = q4_dot_f16(wg[r], xf);                                           \
            const float qu = q4_dot_f16(wu[r], xf);                                           \
            float g = wave_sum(fmaf(sg[r], qg, bg[r] * xsum));                                \
            float uu = wave_sum(fmaf(su[r], qu, bu[r] * xsum));                               \
            if (in_norm_w)                                                                    \
                g *= inv_rms, uu *= inv_rms;                                                  \
            if (lane == 0)                                                                    \
                sh.act_u[wv * RW + r] = (g / (1.0f + expf(-g))) * uu;                         \
        }                                                                                     \
        __syncthreads();                                                                      \
        if (tid < CHUNK)                                                                      \
            publish(ta + (uint64_t)(U) * CHUNK + tid, tag, sh.act_u[tid]);                    \
        publish_done(tfu + (U), tag);                                                         \
    } while (0)

    // ---- 1. router rows and the shared gate logit (one wave per row)
    if (full || has_shared) {
        const uint32_t nE = full ? E : 0u;
        const uint32_t tasks = nE + (has_shared ? 1u : 0u);
        for (uint32_t t = b * 4u + wv; t < tasks; t += NW * 4u) {
            float v = 80.0f; // no gate projection: sigma(80) = 1 (metal/mod.rs:4666-4669)
            if (t < nE || a.sgate_w) {
                const void* row = t < nE ? (const void*)(reinterpret_cast<const uint16_t*>(a.router_w) + (uint64_t)t * H)
                                         : a.sgate_w;
                v = wave_sum(dense_dot<WDT>(row, 32u * lane, xf, xv)) * inv_rms;
            }
            if (lane == 0)
                publish(tl + (t < nE ? t : E), tag, v);
        }
        if (b * 4u < tasks)
            publish_done(tfr + b, tag);
    }

    // ---- 2a. shared unit: no routing needed
    if (shared_unit) {
        PBM_UNIT_LOAD(sx, sx.base);
        PBM_UNIT_FINISH(b);
    }

    // ---- routes (every workgroup: the routed units need their expert, the
    // combine needs the weights)
    if (full) {
        const uint32_t nrw = min(NW, (E + (has_shared ? 1u : 0u) + 3u) / 4u); // workgroups with router rows
        wait_words<1>([tfr](uint32_t i) { return tfr + i; }, nrw, tag,
                      [](uint32_t i) -> float& { return sh.actx[i]; }, spin_max, status);
        wait_words<4>([tl](uint32_t i) { return tl + i; }, E, tag, [](uint32_t i) -> float& { return sh.lg[i]; },
                      spin_max, status);
        __syncthreads();
        const bool grouped = rp.kind == 2 && rp.n_group > 1;
        bool done = false;
        if (rp.order == 0 && !grouped)
            done = route_fast(rp, a.sel_bias, sh, status);
        if (!done) {
            if (rp.order == 0 && !grouped)
                route_token_block<4>(sh.lg, a.sel_bias, rp, sh.ids, sh.w, sh.rgrp, status);
            else if (wv == 0)
                route_token_wave<16>(sh.lg, a.sel_bias, rp, sh.ids, sh.w, sh.sel, sh.rgrp, status);
            __syncthreads();
        }
        if (b == 0 && tid < K) {
            a.ids[tid] = sh.ids[tid];
            a.weights[tid] = sh.w[tid];
        }
    } else {
        if (tid < K) {
            sh.ids[tid] = a.ids[tid];
            sh.w[tid] = a.weights[tid];
        }
        __syncthreads();
    }

    // ---- 2b. routed unit: issue its gate/up loads
    const bool routed_unit = has_unit && !shared_unit;
    bool routed_ok = false;
    if (routed_unit) {
        const uint32_t e = sh.ids[item];
        routed_ok = e < ex.count;
        if (routed_ok) {
            const uint8_t* slot = ex.base + (uint64_t)e * ex.stride;
            PBM_UNIT_LOAD(ex, slot);
        }
    }

    // ---- 3a. issue the down loads of this workgroup's rows, all items
    constexpr uint32_t PAIRS = PT / LPR; // (item, row) pairs per pass
    const uint32_t gl = tid % LPR, slot_id = tid / LPR;
    uint4 wd[NP][CPD];
    float sd[NP][CPD], bd[NP][CPD];
    const uint32_t npairs = items * nrows;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const uint32_t pr = p * PAIRS + slot_id;
        const uint32_t k = nrows ? pr / nrows : 0u, j = nrows ? pr % nrows : 0u;
        const bool sh_item = has_shared && k == K;
        const uint32_t e = sh_item ? 0u : (k < K ? sh.ids[k] : 0u);
        const bool live = pr < npairs && (sh_item || e < ex.count);
        const uint8_t* slot = sh_item ? sx.base : ex.base + (uint64_t)e * ex.stride;
        const uint64_t dw = sh_item ? sx.dw : ex.dw, dsc = sh_item ? sx.ds : ex.ds, dbi = sh_item ? sx.db : ex.db;
        const uint32_t gsh = sh_item ? sx.gshift : ex.gshift;
        const uint32_t h = h0 + j;
        const uint32_t gpr_d = I >> gsh;
#pragma unroll
        for (int c = 0; c < CPD; ++c) {
            const uint32_t ch = gl + LPR * c;
            if (live) {
                wd[p][c] = reinterpret_cast<const uint4*>(slot + dw + (uint64_t)h * (I / 2))[ch];
                const uint64_t gi = (uint64_t)h * gpr_d + ((ch * 32u) >> gsh);
                sd[p][c] = sb_at<SBT>(slot + dsc, gi);
                bd[p][c] = sb_at<SBT>(slot + dbi, gi);
            } else {
                wd[p][c] = make_uint4(0, 0, 0, 0);
                sd[p][c] = 0.0f;
                bd[p][c] = 0.0f;
            }
        }
    }
    if (routed_unit && !routed_ok && tid == 0)
        atomicOr(status, ST_ROUTE_RANGE); // out-of-range route: its items contribute zero

    // ---- 2c. routed unit: activations
    if (routed_unit) {
        if (routed_ok) {
            PBM_UNIT_FINISH(b);
        } else {
            if (tid < CHUNK)
                publish(ta + (uint64_t)b * CHUNK + tid, tag, 0.0f);
            publish_done(tfu + b, tag);
        }
    }
#undef PBM_UNIT_LOAD
#undef PBM_UNIT_FINISH

    // ---- 3b. gather every item's activations, down rows, combine
    if (nrows) {
        wait_words<2>([tfu](uint32_t i) { return tfu + i; }, NU, tag,
                      [](uint32_t i) -> float& { return sh.actx[i]; }, spin_max, status);
        __syncthreads(); // sh.actx is reused below
        wait_words<MAX_ACT / PT>([ta](uint32_t i) { return ta + i; }, items * I, tag,
                      [](uint32_t i) -> float& { return sh.actx[(i >> 5) * XPAD + (i & 31u)]; }, spin_max,
                      status);
        if (has_shared && tid == 0) {
            float g = 0.0f;
            const uint64_t* gl_word = tl + E;
            wait_words<1>([gl_word](uint32_t) { return gl_word; }, 1u, tag, [&g](uint32_t) -> float& { return g; },
                          spin_max, status);
            sh.misc[0] = g;
        }
    }
    __syncthreads();
    if (nrows) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const uint32_t pr = p * PAIRS + slot_id;
            const uint32_t k = pr / nrows, j = pr % nrows;
            float part = 0.0f;
            if (pr < npairs) {
#pragma unroll
                for (int c = 0; c < CPD; ++c) {
                    const uint32_t ch = gl + LPR * c;
                    float xs;
                    const float qa = q4_chunk_qx(wd[p][c], sh.actx + (k * NCI + ch) * XPAD, xs);
                    part = fmaf(sd[p][c], qa, fmaf(bd[p][c], xs, part));
                }
            }
            const float y = group_sum<LPR>(part);
            if (gl == 0 && pr < npairs)
                sh.yk[k][j] = y;
        }
    }
    __syncthreads();
    float hv = 0.0f;
    if (tid < nrows) {
        float moe = 0.0f;
        for (uint32_t k = 0; k < K; ++k)
            moe = moe + sh.w[k] * sh.yk[k][tid];
        const float rm = resid + moe;
        float sv = 0.0f, sw = 0.0f;
        if (has_shared) {
            sv = sh.yk[K][tid];
            sw = sigmoidf_(sh.misc[0]);
        }
        hv = rm + sw * sv;
        a.hidden_out[h0 + tid] = hv;
    }

    // ---- next-layer RMSNorm of the output rows: per-workgroup sums of
    // squares exchanged, summed in workgroup order by every workgroup
    if (a.next_norm_w) {
        float q = tid < nrows ? hv * hv : 0.0f;
        q = wave_sum(q);
        if (lane == 0)
            sh.part[wv] = q;
        __syncthreads();
        if (tid == 0)
            publish(tn + b, tag, (sh.part[0] + sh.part[1]) + (sh.part[2] + sh.part[3]));
        wait_words<1>([tn](uint32_t i) { return tn + i; }, NW, tag, [](uint32_t i) -> float& { return sh.actx[i]; },
                      spin_max, status);
        __syncthreads();
        if (tid < nrows) {
            float tot = 0.0f;
            for (uint32_t i = 0; i < NW; ++i)
                tot += sh.actx[i];
            const float scale = 1.0f / sqrtf(tot / (float)H + a.eps);
            a.next_normed[h0 + tid] = (hv * scale) * a.next_norm_w[h0 + tid];
        }
    }

    // ---- advance the epoch once every workgroup has read it (each published
    // its arrival after reading); the next call runs after this grid ends
    if (b == 0) {
        __syncthreads(); // sh.actx is free again
        wait_words<1>([arrive](uint32_t i) { return arrive + i; }, NW, tag,
                      [](uint32_t i) -> float& { return sh.actx[i]; }, spin_max, status);
        __syncthreads();
        if (tid == 0)
            __hip_atomic_store(a.epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

namespace {
// (LPR, CPD, NP) of the down rows for an intermediate size
struct DownShape {
    uint32_t lpr, cpd, np;
};
bool down_shape(uint32_t I, DownShape* s)
{
    switch (I) {
    case 256: *s = {8, 1, 8}; return true;
    case 512: *s = {16, 1, 12}; return true;
    case 768: *s = {8, 3, 4}; return true;
    case 1024: *s = {16, 2, 6}; return true;
    case 1536: *s = {16, 3, 4}; return true;
    case 2048: *s = {16, 4, 3}; return true;
    default: return false;
    }
}
} // namespace

// Host: does the one-launch path cover this call, and with how many
// workgroups?  One token, hidden 2048, 16-bit router (and gate row), one
// workgroup per gate/up unit, at most one workgroup per CU.
bool persist_plan(const DecodeArgs& d, uint32_t max_wgs, PersistPlan* p)
{
    if (d.tokens != 1 || d.hidden != 2048 || d.rp.experts > 1024 || d.rp.experts == 0 || d.rp.experts % 4 ||
        d.rp.k > (uint32_t)MAX_K || d.rp.k == 0)
        return false;
    // 16-bit dense router and gate rows only (f32 and Q4 rows take the
    // three-kernel decode)
    if ((d.router_w && (d.router_dtype == 0 || d.router_dtype == DT_Q4)) ||
        (d.sgate_w && (d.sgate_dtype == 0 || d.sgate_dtype == DT_Q4)))
        return false;
    if (d.router_w && d.sgate_w && d.router_dtype != d.sgate_dtype)
        return false;
    const uint32_t I = d.ex.gate.rows;
    DownShape ds;
    if (!down_shape(I, &ds) || (d.shared && d.shared->gate.rows != I) || d.ex.group < 32)
        return false;
    const uint32_t items = d.rp.k + (d.shared ? 1u : 0u);
    const uint32_t nunits = items * (I / CHUNK);
    const uint32_t nw = (nunits + 7) / 8 * 8;
    if (nw > 256 || nw > max_wgs || items * I > (uint32_t)MAX_ACT)
        return false;
    const uint32_t rpw = (d.hidden + nw - 1) / nw;
    if (rpw > (uint32_t)MAX_ROWS || items * rpw > ds.np * (PT / ds.lpr))
        return false;
    p->nw = nw;
    p->ngroups = 0;
    p->nci = I / CHUNK;
    p->nunits = nunits;
    p->rpw = rpw;
    // epoch, arrivals, logits, activations, norm sums, router flags, unit flags
    p->words = 1 + nw + (d.rp.experts + 1) + (size_t)items * I + nw + nw + nunits;
    return true;
}

hipError_t launch_persist_decode(hipStream_t st, const DecodeArgs& d, bool full, const PersistPlan& p,
                                 uint64_t* scratch)
{
    PersistArgs a{};
    a.router_w = d.router_w;
    a.sel_bias = d.sel_bias;
    a.rp = d.rp;
    a.sgate_w = d.sgate_w;
    a.ex = d.ex;
    a.has_shared = d.shared != nullptr;
    if (d.shared)
        a.sh = *d.shared;
    a.x = d.x;
    a.in_norm_w = d.in_norm_w;
    a.eps = d.eps;
    a.residual = d.residual;
    a.hidden_out = d.hidden_out;
    a.next_norm_w = d.next_norm_w && d.next_normed ? d.next_norm_w : nullptr;
    a.next_normed = d.next_normed;
    a.ids = d.ids;
    a.weights = d.weights;
    a.full = full ? 1u : 0u;
    a.hidden = d.hidden;
    a.nunits = p.nunits;
    a.rpw = p.rpw;
    const uint32_t items = d.rp.k + (d.shared ? 1u : 0u);
    const uint32_t I = d.ex.gate.rows;
    a.epoch = reinterpret_cast<uint32_t*>(scratch);
    a.arrive = scratch + 1;
    a.tl = a.arrive + p.nw;
    a.ta = a.tl + d.rp.experts + 1;
    a.tn = a.ta + (size_t)items * I;
    a.tfr = a.tn + p.nw;
    a.tfu = a.tfr + p.nw;
    a.status = d.status;
    a.spin_max = 200000;
    if (full && !d.router_w)
        return hipErrorInvalidValue;
    const uint32_t wdt = full ? d.router_dtype : (d.sgate_w ? d.sgate_dtype : 1u);
    if (wdt != 1 && wdt != 2)
        return hipErrorInvalidValue;
    hipEvent_t e0 = d.phase_timing ? d.phase_ev[0] : nullptr, e1 = d.phase_timing ? d.phase_ev[1] : nullptr;
#define PBM_PK(S, W, L, C, N)                                                                 \
    hipExtLaunchKernelGGL((persist_decode_kernel<S, W, L, C, N>), dim3(p.nw), dim3(PT), 0, st, e0, e1, 0, a)
#define PBM_PK_I(S, W)                                                                        \
    do {                                                                                      \
        switch (I) {                                                                          \
        case 256: PBM_PK(S, W, 8, 1, 8); break;                                               \
        case 512: PBM_PK(S, W, 16, 1, 12); break;                                             \
        case 768: PBM_PK(S, W, 8, 3, 4); break;                                               \
        case 1024: PBM_PK(S, W, 16, 2, 6); break;                                             \
        case 1536: PBM_PK(S, W, 16, 3, 4); break;                                             \
        case 2048: PBM_PK(S, W, 16, 4, 3); break;                                             \
        default: return hipErrorInvalidValue;                                                 \
        }                                                                                     \
    } while (0)
    if (d.ex.sb_dtype == 2) {
        if (wdt == 2) PBM_PK_I(2, 2);
        else PBM_PK_I(2, 1);
    } else {
        if (wdt == 2) PBM_PK_I(1, 2);
        else PBM_PK_I(1, 1);
    }
#undef PBM_PK
#undef PBM_PK_I
    hipError_t err = hipGetLastError();
    if (err == hipSuccess && d.phase_timing) // one kernel: the other phase slots are empty
        for (int i = 2; i < 6 && err == hipSuccess; ++i)
            err = hipEventRecord(d.phase_ev[i], st);
    return err;
}

} // namespace pbmoe
