// Batch-1 decode attention of one layer on gfx950 (GQA, head_dim 128):
// the Qwen full-attention step that precedes every MoE block
// (full_attention_output_values, flashmoe/runtime/mod.rs:2215-2367).
//
//  1. q4_rows_kernel: q, k, v = W . normed (three resident Q4 projections
//     in one launch, one wave per two rows).
//  2. attn_chunk_kernel: one workgroup per (64-position chunk, kv head, up
//     to 4 of its q heads): per-head q RMSNorm + split-half RoPE; the
//     chunk holding this position also normalises/rotates the new k, rounds
//     k and v to f16 and writes them to the cache; scores over the chunk,
//     softmax partial (max, sum), P.V partial.
//  3. attn_merge_kernel: log-sum-exp merge of the chunk partials per head.
//  4. q4_rows_kernel: hidden = residual + W_o . attention.
//  5. rms_norm_kernel: post-attention RMSNorm (optional).
// Arithmetic is f32 throughout; keys and values are stored as f16 (the
// cache format), queries stay f32.
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>

#include "pbmoe_device.h"
#include "pbmoe_internal.h"

namespace pbmoe {

constexpr int HD = 128;        // head_dim the attention kernels are written for
constexpr int HALF = HD / 2;   // split-half RoPE pairs (i, i + 64): lane i holds both
constexpr int KPITCH = HD + 8; // halfs per staged K row: 272 bytes, rows fall on distinct banks
constexpr int CH = (int)ATTN_CHUNK;
static_assert(CH == 64, "one position per lane");

// ---------------------------------------------------------------------------
// Q4 rows . x for up to three matrices with the same column count; output
// rows are concatenated (matrix i starts at first[i]).  The factored form
// sum_g s_g * sum(q x) + b_g * sum(x) of the reference's fma(q, s x, b x)
// (q4_fma_row_bf16_ptrs, shaders.metal:97-199).
// ---------------------------------------------------------------------------
struct RowsArgs {
    Q4Mat m[3];
    uint32_t n_mat;
    uint32_t first[4];
    uint32_t group_shift;
    const float* x;        // [cols]
    const float* norm_w;   // null, or RMSNorm weight [cols]: x is normalised first
    float eps;
    const float* residual; // null or [total rows]
    float* y;              // [total rows]
};

template <int SBT, int CPL, int RPW, bool NORM>
__global__ __launch_bounds__(256) void q4_rows_kernel(RowsArgs a)
{
    // x is staged in LDS once per workgroup with coalesced loads (a lane's
    // own 32-float chunk read straight from memory would touch a different
    // cache line in every lane); chunks sit XP floats apart so that the
    // lanes' 16-byte reads of consecutive chunks fall on distinct banks.
    constexpr int XP = 36;
    __shared__ __align__(16) float xl[WAVE * CPL * XP];
    __shared__ float red[4];
    const int lane = threadIdx.x & 63;
    // The wave index is read as a scalar, so that the matrix choice and the
    // row pointers are scalar too and the weight loads issue at once (a
    // per-lane choice fetches the matrix descriptor per lane first: one more
    // memory round trip).
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r0 = (blockIdx.x * 4 + wv) * RPW;
    const bool active = r0 < a.first[a.n_mat];
    const uint32_t rr = active ? r0 : 0u; // idle waves still reach the barrier
    const uint32_t mi = (a.n_mat > 1 && rr >= a.first[1]) + (a.n_mat > 2 && rr >= a.first[2]);
    const uint8_t* codes = mi == 0 ? a.m[0].codes : mi == 1 ? a.m[1].codes : a.m[2].codes;
    const uint16_t* scales =
        reinterpret_cast<const uint16_t*>(mi == 0 ? a.m[0].scales : mi == 1 ? a.m[1].scales : a.m[2].scales);
    const uint16_t* biases =
        reinterpret_cast<const uint16_t*>(mi == 0 ? a.m[0].biases : mi == 1 ? a.m[1].biases : a.m[2].biases);
    const uint32_t row0 = rr - (mi == 0 ? 0u : mi == 1 ? a.first[1] : a.first[2]);
    const uint32_t cols = a.m[0].cols; // every matrix of one launch has the same columns
    const uint32_t chunks = cols / 32, gpr = cols >> a.group_shift;
    // Every load is issued before any is used: lanes past the last chunk
    // read the last chunk again (clamped, no branch: a load inside a
    // divergent branch is waited for where the branch ends), and the 16-bit
    // scales and biases are converted where they are used.
    uint4 w[RPW][CPL];
    uint32_t sr[RPW][CPL], br[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint32_t row = row0 + r;
        const uint4* wp = reinterpret_cast<const uint4*>(codes + (uint64_t)row * (cols / 2));
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = min(lane + WAVE * c, chunks - 1);
            w[r][c] = wp[ch];
            const uint64_t gi = (uint64_t)row * gpr + ((ch * 32u) >> a.group_shift);
            sr[r][c] = scales[gi];
            br[r][c] = biases[gi];
        }
    }
    // residual of this wave's rows (lane r holds row r's), or y itself as a
    // harmless stand-in that is not used
    const float* rsrc = a.residual ? a.residual : a.y;
    const float resv = rsrc[rr + min(lane, RPW - 1)];
    // Stage x (times the norm weight when the input RMSNorm is fused).  Every
    // row product is linear in the norm's scale, so the sums are multiplied
    // by 1 / sqrt(mean(x^2) + eps) at the end (math.rs:151-167).  The float4
    // slots past cols / 4 hold zeros in chunks no lane reads.
    const uint32_t nf = cols / 4;
    float4 xv4[2 * CPL], nv4[2 * CPL];
#pragma unroll
    for (int j = 0; j < 2 * CPL; ++j) {
        const uint32_t f = min(threadIdx.x + 256u * j, nf - 1);
        xv4[j] = reinterpret_cast<const float4*>(a.x)[f];
        if constexpr (NORM)
            nv4[j] = reinterpret_cast<const float4*>(a.norm_w)[f];
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 2 * CPL; ++j) {
        const uint32_t f = threadIdx.x + 256u * j;
        const bool in = f < nf;
        float4 v = xv4[j];
        v.x = in ? v.x : 0.0f, v.y = in ? v.y : 0.0f, v.z = in ? v.z : 0.0f, v.w = in ? v.w : 0.0f;
        if constexpr (NORM) {
            const float4 nw = nv4[j];
            ss = fmaf(v.x, v.x, ss), ss = fmaf(v.y, v.y, ss), ss = fmaf(v.z, v.z, ss), ss = fmaf(v.w, v.w, ss);
            v.x *= nw.x, v.y *= nw.y, v.z *= nw.z, v.w *= nw.w;
        }
        *reinterpret_cast<float4*>(&xl[(f >> 3) * XP + (f & 7) * 4]) = v;
    }
    if constexpr (NORM) {
        ss = wave_sum(ss);
        if (lane == 0)
            red[threadIdx.x >> 6] = ss;
    }
    __syncthreads();
    if (!active)
        return;
    const float inv_rms =
        NORM ? 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)cols + a.eps) : 1.0f;
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
        acc[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const uint32_t ch = lane + WAVE * c;
        if (ch < chunks) {
            const float4* x4 = reinterpret_cast<const float4*>(&xl[ch * XP]);
            float xv[32];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 v = x4[q];
                xv[4 * q] = v.x, xv[4 * q + 1] = v.y, xv[4 * q + 2] = v.z, xv[4 * q + 3] = v.w;
            }
            float xs = 0.0f;
#pragma unroll
            for (int q = 0; q < 32; q += 4)
                xs += (xv[q] + xv[q + 1]) + (xv[q + 2] + xv[q + 3]);
#pragma unroll
            for (int r = 0; r < RPW; ++r)
                acc[r] = fmaf(sb_bits<SBT>(sr[r][c]), q4_chunk_qx_reg(w[r][c], xv),
                              fmaf(sb_bits<SBT>(br[r][c]), xs, acc[r]));
        }
    }
    const float res = a.residual ? resv : 0.0f;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const float s = wave_sum(acc[r]) * inv_rms;
        if (lane == r)
            a.y[r0 + r] = res + s;
    }
}

// Per-head RMSNorm with weight, then the split-half rotation of pair
// (lane, lane + 64): the order of
// apply_optional_per_head_rms_norm_and_split_half_rope (math.rs:278-300):
// value *= (1 / sqrt(mean(v^2) + 1e-6)) * weight, then x0 cos - x1 sin,
// x0 sin + x1 cos.
// w0, w1: the weights of dims lane and lane + 64.
__device__ __forceinline__ void norm_rope_pair(float& x0, float& x1, float w0, float w1, float sn, float cs)
{
    const float ms = wave_sum(x0 * x0 + x1 * x1) / (float)HD;
    const float scale = 1.0f / sqrtf(ms + 1e-6f);
    const float a0 = x0 * (scale * w0);
    const float a1 = x1 * (scale * w1);
    x0 = a0 * cs - a1 * sn;
    x1 = a0 * sn + a1 * cs;
}

// ---------------------------------------------------------------------------
// attention partials: workgroup (chunk c, kv head j, head group z), NH <= 8
// q heads per workgroup (heads j*NQ + z*NH .. +NH), wave w handles head w.
// Partial record per (q head, chunk): sum_t exp(s_t - m) v_t [HD], m,
// sum_t exp(s_t - m).
// ---------------------------------------------------------------------------
// CHUNK_THREADS: four waves, or one per q head for eight heads (the kv
// head's keys and values are then loaded by one workgroup, not two)
template <int NH>
constexpr int CHUNK_THREADS = NH <= 4 ? 256 : 64 * NH;

template <int NH>
__global__ __launch_bounds__(CHUNK_THREADS<NH>) void attn_chunk_kernel(AttnArgs a)
{
    constexpr int NT = CHUNK_THREADS<NH>;
    __shared__ float qs[NH][HD];
    __shared__ __align__(16) uint16_t kc[CH][KPITCH];
    __shared__ __align__(16) uint16_t vc[CH][HD];
    __shared__ float ps[NH][CH];
    __shared__ __align__(16) uint16_t knew[HD];
    __shared__ __align__(16) uint16_t vnew[HD];
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6); // wave index, scalar
    const uint32_t chunk = blockIdx.x, j = blockIdx.y;
    const uint32_t nq = a.q_heads / a.kv_heads;
    // this wave's q head (waves past NH read head NH - 1 and store nothing)
    const uint32_t qh = j * nq + blockIdx.z * NH + min(wv, (uint32_t)NH - 1);
    const uint32_t n = a.position + 1; // attended positions 0..position
    const uint32_t t0 = chunk * CH;
    const uint32_t cnt = min((uint32_t)CH, n - t0);
    const uint32_t chunks = gridDim.x;
    const bool has_new = a.position >= t0 && a.position < t0 + CH;

    // The small loads (rotation frequency, q row, this position's k and v
    // rows, the q and k norm weights) are issued first and unconditionally: a wave's loads complete in
    // issue order, so the rotation below waits only for these, while the
    // chunk's key/value loads (16 bytes per thread per step) stay in flight.
    const float ifr = a.inv_freq[lane];
    const float* qr = a.qkv + (uint64_t)qh * HD;
    const float* kr = a.qkv + (uint64_t)a.q_heads * HD + (uint64_t)j * HD;
    const float* vr = kr + (uint64_t)a.kv_heads * HD;
    const float q0 = qr[lane], q1 = qr[lane + HALF];
    const float k0 = kr[lane], k1 = kr[lane + HALF];
    const float v0 = vr[lane], v1 = vr[lane + HALF];
    const float qn0 = a.q_norm[lane], qn1 = a.q_norm[lane + HALF];
    const float kn0 = a.k_norm[lane], kn1 = a.k_norm[lane + HALF];
    // Rows past cnt read the chunk's last row (no branch around a load: one
    // inside a divergent branch is waited for where the branch ends) and are
    // zeroed when staged; this position's row is taken from LDS below, not
    // from the cache.
    constexpr int PIECES = CH * (HD / 8) / NT;
    uint4 kk[PIECES], vv[PIECES];
#pragma unroll
    for (int u = 0; u < PIECES; ++u) {
        const uint32_t i = tid + NT * u, t = min(i / (HD / 8), cnt - 1), q = i % (HD / 8);
        const uint64_t o = ((uint64_t)(t0 + t) * a.kv_heads + j) * HD;
        kk[u] = reinterpret_cast<const uint4*>(a.cache_k + o)[q];
        vv[u] = reinterpret_cast<const uint4*>(a.cache_v + o)[q];
    }

    // rotation of the pair (lane, lane + 64) at this position: the f32 angle
    // of split_half_rope_rotations (math.rs:303-325)
    float sn, cs;
    sincosf((float)a.position * ifr, &sn, &cs);
    if (wv < NH) {
        float x0 = q0, x1 = q1;
        norm_rope_pair(x0, x1, qn0, qn1, sn, cs);
        qs[wv][lane] = x0;
        qs[wv][lane + HALF] = x1;
    }
    if (has_new && wv == 0) {
        float x0 = k0, x1 = k1;
        norm_rope_pair(x0, x1, kn0, kn1, sn, cs);
        const uint16_t nk0 = __half_as_ushort(__float2half(x0)), nk1 = __half_as_ushort(__float2half(x1));
        const uint16_t nv0 = __half_as_ushort(__float2half(v0));
        const uint16_t nv1 = __half_as_ushort(__float2half(v1));
        knew[lane] = nk0, knew[lane + HALF] = nk1;
        vnew[lane] = nv0, vnew[lane + HALF] = nv1;
        if (blockIdx.z == 0) { // one writer per kv head
            const uint64_t o = ((uint64_t)a.position * a.kv_heads + j) * HD;
            a.cache_k[o + lane] = nk0, a.cache_k[o + lane + HALF] = nk1;
            a.cache_v[o + lane] = nv0, a.cache_v[o + lane + HALF] = nv1;
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < PIECES; ++u) {
        const uint32_t i = tid + NT * u, t = i / (HD / 8), q = i % (HD / 8);
        const bool live = t < cnt;
        uint4 kx = kk[u], vx = vv[u];
        kx.x = live ? kx.x : 0u, kx.y = live ? kx.y : 0u, kx.z = live ? kx.z : 0u, kx.w = live ? kx.w : 0u;
        vx.x = live ? vx.x : 0u, vx.y = live ? vx.y : 0u, vx.z = live ? vx.z : 0u, vx.w = live ? vx.w : 0u;
        if (t0 + t == a.position) {
            kx = reinterpret_cast<const uint4*>(knew)[q];
            vx = reinterpret_cast<const uint4*>(vnew)[q];
        }
        reinterpret_cast<uint4*>(&kc[t][0])[q] = kx;
        reinterpret_cast<uint4*>(&vc[t][0])[q] = vx;
    }
    __syncthreads();
    if (wv >= NH)
        return;

    // scores: lane = position t of the chunk
    const float scale = 1.0f / sqrtf((float)HD);
    float s = 0.0f;
    const uint16_t* krow = &kc[lane][0];
#pragma unroll
    for (int d8 = 0; d8 < HD / 8; ++d8) {
        const uint4 raw = reinterpret_cast<const uint4*>(krow)[d8];
        const uint32_t r4[4] = {raw.x, raw.y, raw.z, raw.w};
        const float4 qa = reinterpret_cast<const float4*>(&qs[wv][8 * d8])[0];
        const float4 qb = reinterpret_cast<const float4*>(&qs[wv][8 * d8])[1];
        const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s = fmaf(qv[2 * e], __half2float(__ushort_as_half((uint16_t)(r4[e] & 0xFFFFu))), s);
            s = fmaf(qv[2 * e + 1], __half2float(__ushort_as_half((uint16_t)(r4[e] >> 16))), s);
        }
    }
    const bool valid = (uint32_t)lane < cnt;
    const float sv = valid ? s * scale : -INFINITY;
    const float mx = wave_max(sv);
    const float p = valid ? expf(sv - mx) : 0.0f;
    const float sum = wave_sum(p);
    ps[wv][lane] = p; // read back by this wave only (LDS operations of a wave complete in order)
    // P . V: lane holds dims 2 lane, 2 lane + 1.  All CH rows, unrolled so
    // that the LDS reads overlap: rows past cnt hold zeros and have p = 0.
    float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
#pragma unroll
    for (int t = 0; t < CH; t += 2) {
        const uint32_t va = reinterpret_cast<const uint32_t*>(&vc[t][0])[lane];
        const uint32_t vb = reinterpret_cast<const uint32_t*>(&vc[t + 1][0])[lane];
        const float pa = ps[wv][t], pb = ps[wv][t + 1];
        o0 = fmaf(pa, __half2float(__ushort_as_half((uint16_t)(va & 0xFFFFu))), o0);
        o1 = fmaf(pa, __half2float(__ushort_as_half((uint16_t)(va >> 16))), o1);
        o2 = fmaf(pb, __half2float(__ushort_as_half((uint16_t)(vb & 0xFFFFu))), o2);
        o3 = fmaf(pb, __half2float(__ushort_as_half((uint16_t)(vb >> 16))), o3);
    }
    o0 += o2, o1 += o3;
    float* rec = a.part + ((uint64_t)qh * chunks + chunk) * (HD + 2);
    reinterpret_cast<float2*>(rec)[lane] = make_float2(o0, o1);
    if (lane == 0) {
        rec[HD] = mx;
        rec[HD + 1] = sum;
    }
}

// merge the chunk partials of one q head: out = sum_c e^(m_c - M) o_c /
// sum_c e^(m_c - M) l_c, i.e. softmax over every position (softmax_in_place,
// math.rs:728-744) then the weighted sum of values.  Workgroup (head h,
// slice y) takes MERGE_DIMS of the head's dims, MERGE_PARTS threads per dim
// (each over every MERGE_PARTS-th chunk), so that the head's loads spread
// over MERGE_SPLIT CUs.  The partials were just written by other XCDs, so
// every round trip is slow: the values of the first MERGE_BLOCK chunks are
// loaded together with the (m, l) pairs, before any reduction.
constexpr uint32_t MERGE_MAX_CHUNKS = 1024; // max_context / ATTN_CHUNK (65536 positions)
constexpr int MERGE_BLOCK = 64;             // chunks whose values are loaded up front
// workgroups per head (C4 stack, 32 heads at context 4096: 1 / 2 / 4 / 8
// per head 1.943 / 1.884 / 1.848 / 1.838 ms per token)
constexpr int MERGE_SPLIT = 8;
constexpr int MERGE_DIMS = HD / MERGE_SPLIT;            // dims per workgroup
constexpr int MERGE_PARTS = 256 / MERGE_DIMS;           // threads per dim
static_assert(MERGE_DIMS * MERGE_PARTS == 256 && MERGE_BLOCK % MERGE_PARTS == 0, "merge tiling");
__global__ __launch_bounds__(256) void attn_merge_kernel(const float* __restrict__ part, uint32_t chunks,
                                                         float* __restrict__ out)
{
    __shared__ float ec[MERGE_MAX_CHUNKS];
    __shared__ float red[8];
    __shared__ float part_acc[MERGE_PARTS][MERGE_DIMS];
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float* ph = part + (uint64_t)h * chunks * (HD + 2);
    const uint32_t dl = tid % MERGE_DIMS, part_i = tid / MERGE_DIMS;
    const uint32_t d = blockIdx.y * MERGE_DIMS + dl;
    constexpr int PV = MERGE_BLOCK / MERGE_PARTS;
    float val[PV];
#pragma unroll
    for (int u = 0; u < PV; ++u) {
        const uint32_t c = part_i + MERGE_PARTS * u;
        val[u] = c < chunks ? ph[(uint64_t)c * (HD + 2) + d] : 0.0f;
    }
    float m = -INFINITY;
    float ml[MERGE_MAX_CHUNKS / 256][2];
#pragma unroll
    for (int u = 0; u < (int)(MERGE_MAX_CHUNKS / 256); ++u) {
        const uint32_t c = tid + 256 * u;
        ml[u][0] = -INFINITY, ml[u][1] = 0.0f;
        if (c < chunks) {
            const float2 v = *reinterpret_cast<const float2*>(ph + (uint64_t)c * (HD + 2) + HD);
            ml[u][0] = v.x, ml[u][1] = v.y;
            m = fmaxf(m, v.x);
        }
    }
    m = wave_max(m);
    if (lane == 0)
        red[wv] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float l = 0.0f;
#pragma unroll
    for (int u = 0; u < (int)(MERGE_MAX_CHUNKS / 256); ++u) {
        const uint32_t c = tid + 256 * u;
        if (c < chunks) {
            const float e = expf(ml[u][0] - M);
            ec[c] = e;
            l = fmaf(e, ml[u][1], l);
        }
    }
    l = wave_sum(l);
    if (lane == 0)
        red[4 + wv] = l;
    __syncthreads();
    const float L = (red[4] + red[5]) + (red[6] + red[7]);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < PV; ++u) {
        const uint32_t c = part_i + MERGE_PARTS * u;
        if (c < chunks)
            acc[u & 3] = fmaf(ec[c], val[u], acc[u & 3]);
    }
    for (uint32_t c = part_i + MERGE_BLOCK; c < chunks; c += MERGE_PARTS) // long contexts
        acc[0] = fmaf(ec[c], ph[(uint64_t)c * (HD + 2) + d], acc[0]);
    part_acc[part_i][dl] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    __syncthreads();
    if (part_i == 0) {
        float sum = part_acc[0][dl];
#pragma unroll
        for (int q = 1; q < MERGE_PARTS; ++q)
            sum += part_acc[q][dl];
        out[(uint64_t)h * HD + d] = sum / L;
    }
}

// RMSNorm with weight, one workgroup: rms_norm_with_weight_and_epsilon
// (math.rs:151-167): value *= 1 / sqrt(mean(v^2) + eps); value *= weight.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ h, const float* __restrict__ w,
                                                       uint32_t width, float eps, float* __restrict__ out)
{
    __shared__ float red[4];
    float s = 0.0f;
    for (uint32_t i = threadIdx.x; i < width; i += 256)
        s = fmaf(h[i], h[i], s);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float ms = ((red[0] + red[1]) + (red[2] + red[3])) / (float)width;
    const float scale = 1.0f / sqrtf(ms + eps);
    for (uint32_t i = threadIdx.x; i < width; i += 256)
        out[i] = (h[i] * scale) * w[i];
}

// e0, e1: start / stop events of the dispatch, or null
template <int SBT, int RPW, bool NORM>
static hipError_t launch_rows(hipStream_t st, const RowsArgs& r, hipEvent_t e0, hipEvent_t e1)
{
    const uint32_t total = r.first[r.n_mat];
    const uint32_t cols = r.m[0].cols;
    const uint32_t cpl = (cols / 32 + 63) / 64;
    const dim3 grid((total / RPW + 3) / 4);
    if (cpl <= 1)
        hipExtLaunchKernelGGL((q4_rows_kernel<SBT, 1, RPW, NORM>), grid, dim3(256), 0, st, e0, e1, 0, r);
    else if (cpl <= 2)
        hipExtLaunchKernelGGL((q4_rows_kernel<SBT, 2, RPW, NORM>), grid, dim3(256), 0, st, e0, e1, 0, r);
    else if (cpl <= 4)
        hipExtLaunchKernelGGL((q4_rows_kernel<SBT, 4, RPW, NORM>), grid, dim3(256), 0, st, e0, e1, 0, r);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int SBT, int RPW>
static hipError_t launch_rows(hipStream_t st, const RowsArgs& r, hipEvent_t e0, hipEvent_t e1)
{
    return r.norm_w ? launch_rows<SBT, RPW, true>(st, r, e0, e1) : launch_rows<SBT, RPW, false>(st, r, e0, e1);
}

// rows per wave: 2 for q/k/v (640 workgroups at C4), 1 for o_proj (512
// workgroups instead of 256; measured on the C4 stack: 1.134 -> 1.079 ms of
// attention per token; 4 for either was slower, 1 for q/k/v the same)
constexpr int RPW_QKV = 2, RPW_O = 1;

hipError_t launch_attention_decode(hipStream_t st, const AttnArgs& a)
{
    if (a.head_dim != HD || a.kv_heads == 0 || a.q_heads % a.kv_heads)
        return hipErrorInvalidValue;
    const uint32_t nq = a.q_heads / a.kv_heads;
    const uint32_t qw = a.q_heads * HD, kvw = a.kv_heads * HD;
    // 1. q, k, v
    RowsArgs r{};
    r.m[0] = a.q, r.m[1] = a.k, r.m[2] = a.v;
    r.n_mat = 3;
    r.first[0] = 0, r.first[1] = qw, r.first[2] = qw + kvw, r.first[3] = qw + 2 * kvw;
    r.group_shift = a.group_shift;
    r.x = a.normed;
    r.norm_w = a.in_norm_w;
    r.eps = a.post_eps;
    r.residual = nullptr;
    r.y = a.qkv;
    hipError_t e = a.sb_dtype == 2 ? launch_rows<2, RPW_QKV>(st, r, a.ev[0], a.ev[1])
                                  : launch_rows<1, RPW_QKV>(st, r, a.ev[0], a.ev[1]);
    if (e != hipSuccess)
        return e;
    // 2. chunk partials
    const uint32_t chunks = (a.position + 1 + CH - 1) / CH;
    switch (nq) {
    case 1:
        hipExtLaunchKernelGGL((attn_chunk_kernel<1>), dim3(chunks, a.kv_heads, 1), dim3(256), 0, st, a.ev[2], a.ev[3],
                              0, a);
        break;
    case 2:
        hipExtLaunchKernelGGL((attn_chunk_kernel<2>), dim3(chunks, a.kv_heads, 1), dim3(256), 0, st, a.ev[2], a.ev[3],
                              0, a);
        break;
    case 4:
        hipExtLaunchKernelGGL((attn_chunk_kernel<4>), dim3(chunks, a.kv_heads, 1), dim3(256), 0, st, a.ev[2], a.ev[3],
                              0, a);
        break;
    case 8:
        hipExtLaunchKernelGGL((attn_chunk_kernel<8>), dim3(chunks, a.kv_heads, 1), dim3(CHUNK_THREADS<8>), 0, st,
                              a.ev[2], a.ev[3], 0, a);
        break;
    default: return hipErrorInvalidValue;
    }
    if ((e = hipGetLastError()) != hipSuccess)
        return e;
    // 3. merge
    if (chunks > MERGE_MAX_CHUNKS)
        return hipErrorInvalidValue;
    hipExtLaunchKernelGGL(attn_merge_kernel, dim3(a.q_heads, MERGE_SPLIT), dim3(256), 0, st, a.ev[4], a.ev[5], 0,
                          (const float*)a.part, chunks, a.attn_out);
    if ((e = hipGetLastError()) != hipSuccess)
        return e;
    // 4. o_proj + residual
    RowsArgs o{};
    o.m[0] = a.o;
    o.n_mat = 1;
    o.first[0] = 0, o.first[1] = a.hidden;
    o.group_shift = a.group_shift;
    o.x = a.attn_out;
    o.norm_w = nullptr;
    o.residual = a.residual;
    o.y = a.hidden_out;
    e = a.sb_dtype == 2 ? launch_rows<2, RPW_O>(st, o, a.ev[6], a.ev[7])
                          : launch_rows<1, RPW_O>(st, o, a.ev[6], a.ev[7]);
    if (e != hipSuccess)
        return e;
    // 5. post-attention RMSNorm
    if (a.post_norm_w) {
        hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(256), 0, st, (const float*)a.hidden_out, a.post_norm_w,
                           a.hidden, a.post_eps, a.post_normed);
        e = hipGetLastError();
    }
    return e;
}

} // namespace pbmoe
