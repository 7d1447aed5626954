// Decode path of the MoE block on gfx950: three kernels per layer.
//
//  1. stage: router rows (W_r . x), shared-expert gate/up rows and the
//     shared sigmoid gate, spread one task per wave over the whole chip.
//  2. gate/up: every workgroup derives the routes of the batch from the
//     logits in LDS (selection, softmax/sigmoid, renormalisation, dispatch
//     plan), then routed gate/up with SiLU(g)*u formed in registers; extra
//     workgroups touch the down weights of the selected experts so that
//     kernel 3 finds them in cache.
//  3. down + combine: down projection of every routed and shared item for a
//     block of output rows, then h = (r + sum_k w_k y_k) + sw * S per token
//     in route order.
// Every wave issues all of its weight loads before it consumes any of them:
// at batch 1 the layer is latency-bound, so the number of dependent memory
// round trips, not instruction count, sets the time.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "pbmoe.h"
#include "pbmoe_device.h"
#include "pbmoe_internal.h"

namespace pbmoe {

constexpr int DEC_T = 16;                 // max tokens of the decode path
constexpr int DEC_ROUTES = DEC_T * MAX_K; // max routes
constexpr int DOWN_R = 4;                 // output rows per down workgroup

// ---------------------------------------------------------------------------
// kernel 1: router rows (W_r . x), shared gate/up rows and the shared sigmoid
// gate, one task per wave.  No cross-workgroup synchronisation: the kernel
// boundary publishes the logits to kernel 2.
// ---------------------------------------------------------------------------
struct RouterArgs {
    const void* router_w;
    Q4Rows router_q4;     // WDT == DT_Q4
    Q4Rows sgate_q4;      // GDT == DT_Q4
    uint32_t experts;     // 0: no router rows
    ExpertSet sh;
    uint32_t shared_rows; // shared gate/up rows computed here (0: none, or computed by the gate/up kernel)
    uint32_t gate_task;   // 1: a shared expert, whose gate logit (or the 80.0 constant) is a task here
    const void* sgate_w;
    uint32_t sgate_dtype;
    const float* x;
    uint32_t tokens, hidden;
    float* logits;        // [T][E]
    float* act_shared;    // [T][Is]
    float* shared_weight; // [T]
    const float* norm_w;  // null, or the input RMSNorm weight [H]: x is the hidden state
    float eps;
    float* x_out;         // [T][H] normalised rows, written by the last workgroup (norm_w set)
};

// Fused input RMSNorm (rms_norm_with_weight_and_epsilon, math.rs:151-167).
// Every product W . (x * inv_rms * w) is linear in the scale, so a wave
// dots W with x * w and multiplies the wave sum by inv_rms, which it forms
// from sum(x^2) over the same x registers: no extra loads, no barrier.
//
// x [t][col .. col+8) as two float4; with NORM: the squares go to ss and
// the values are multiplied by the weight.  NORM is a template argument, not
// a test of norm_w: a runtime branch around the multiply made the compiler
// wait for every call's loads inside the branch, one round trip per call.
template <bool NORM>
__device__ __forceinline__ void load_x8(const float* __restrict__ x, uint64_t off, const float* norm_w,
                                        uint32_t col, float4& u, float4& v, float& ss)
{
    const float4* xp = reinterpret_cast<const float4*>(x + off);
    u = xp[0], v = xp[1];
    if constexpr (NORM) {
        ss = fmaf(u.x, u.x, ss), ss = fmaf(u.y, u.y, ss), ss = fmaf(u.z, u.z, ss), ss = fmaf(u.w, u.w, ss);
        ss = fmaf(v.x, v.x, ss), ss = fmaf(v.y, v.y, ss), ss = fmaf(v.z, v.z, ss), ss = fmaf(v.w, v.w, ss);
        const float4 w0 = *reinterpret_cast<const float4*>(norm_w + col);
        const float4 w1 = *reinterpret_cast<const float4*>(norm_w + col + 4);
        u.x *= w0.x, u.y *= w0.y, u.z *= w0.z, u.w *= w0.w;
        v.x *= w1.x, v.y *= w1.y, v.z *= w1.z, v.w *= w1.w;
    }
}

// 1 / sqrt(mean(x^2) + eps) from this lane's partial sum of squares
__device__ __forceinline__ float inv_rms_of(float ss, uint32_t H, float eps)
{
    return 1.0f / sqrtf(wave_sum(ss) / (float)H + eps);
}

template <int WDT>
__device__ __forceinline__ void load_dense8(const void* w, uint64_t off, float (&v)[8])
{
    if constexpr (WDT == 0) {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + off);
        float4 a = p[0], b = p[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
        uint4 raw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + off);
        const uint32_t r4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (WDT == 2) {
                v[2 * i] = __uint_as_float(r4[i] << 16);
                v[2 * i + 1] = __uint_as_float(r4[i] & 0xFFFF0000u);
            } else {
                v[2 * i] = __half2float(__ushort_as_half((uint16_t)(r4[i] & 0xFFFFu)));
                v[2 * i + 1] = __half2float(__ushort_as_half((uint16_t)(r4[i] >> 16)));
            }
        }
    }
}

// dense row . x for every token (8 columns per lane per chunk of 512).
// Rows longer than CR chunks (H > 512 CR) are taken in passes of CR chunks
// per token, the weights reloaded per pass (L2 hits after the first token).
template <int WDT>
__device__ __forceinline__ void dense8_to_float(const uint32_t (&wr)[WDT == 0 ? 8 : 4], float (&wv8)[8])
{
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (WDT == 0) {
            wv8[2 * i] = __uint_as_float(wr[2 * i]);
            wv8[2 * i + 1] = __uint_as_float(wr[2 * i + 1]);
        } else if constexpr (WDT == 2) {
            wv8[2 * i] = __uint_as_float(wr[i] << 16);
            wv8[2 * i + 1] = __uint_as_float(wr[i] & 0xFFFF0000u);
        } else {
            wv8[2 * i] = __half2float(__ushort_as_half((uint16_t)(wr[i] & 0xFFFFu)));
            wv8[2 * i + 1] = __half2float(__ushort_as_half((uint16_t)(wr[i] >> 16)));
        }
    }
}

// tscale: null, or the per-token scale 1 / rms of the rows of x (already
// formed; the sums of squares here are then unused)
template <int WDT, int CR, bool NORM>
__device__ __forceinline__ void dense_row_dots(const void* w, uint64_t row_off, const float* x,
                                               uint32_t T, uint32_t H, float* out, uint32_t out_stride,
                                               const float* norm_w, float eps, const float* tscale = nullptr)
{
    const int lane = threadIdx.x & 63;
    // 16-bit weights stay packed in registers until use
    constexpr int WW = WDT == 0 ? 8 : 4; // 32-bit words per 8 weights
    uint32_t wr[CR][WW];
    auto load_pass = [&](uint32_t base) {
#pragma unroll
        for (int c = 0; c < CR; ++c) {
            const uint32_t col = base + (uint32_t)lane * 8 + c * 512;
#pragma unroll
            for (int i = 0; i < WW; ++i)
                wr[c][i] = 0u;
            if (col < H) {
                if constexpr (WDT == 0) {
                    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(w) + row_off + col);
                    const uint4 a = p[0], b = p[1];
                    wr[c][0] = a.x, wr[c][1] = a.y, wr[c][2] = a.z, wr[c][3] = a.w;
                    wr[c][4] = b.x, wr[c][5] = b.y, wr[c][6] = b.z, wr[c][7] = b.w;
                } else {
                    const uint4 raw =
                        *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + row_off + col);
                    wr[c][0] = raw.x, wr[c][1] = raw.y, wr[c][2] = raw.z, wr[c][3] = raw.w;
                }
            }
        }
    };
    auto dot_pass = [&](uint32_t base, uint32_t t, float& acc0, float& acc1, float& ss) {
#pragma unroll
        for (int c = 0; c < CR; ++c) {
            const uint32_t col = base + (uint32_t)lane * 8 + c * 512;
            if (col < H) {
                float wvc[8];
                dense8_to_float<WDT>(wr[c], wvc);
                float4 u, v;
                load_x8<NORM>(x, (uint64_t)t * H + col, norm_w, col, u, v, ss);
                acc0 = fmaf(wvc[0], u.x, acc0);
                acc1 = fmaf(wvc[1], u.y, acc1);
                acc0 = fmaf(wvc[2], u.z, acc0);
                acc1 = fmaf(wvc[3], u.w, acc1);
                acc0 = fmaf(wvc[4], v.x, acc0);
                acc1 = fmaf(wvc[5], v.y, acc1);
                acc0 = fmaf(wvc[6], v.z, acc0);
                acc1 = fmaf(wvc[7], v.w, acc1);
            }
        }
    };
    const bool one_pass = H <= (uint32_t)CR * 512;
    if (one_pass)
        load_pass(0);
    for (uint32_t t = 0; t < T; ++t) {
        float acc0 = 0.0f, acc1 = 0.0f, ss = 0.0f;
        for (uint32_t base = 0; base < H; base += CR * 512) {
            if (!one_pass)
                load_pass(base);
            // conversions stay inside the token loop (hoisted, they would
            // hold 8 floats per chunk)
#pragma unroll
            for (int c = 0; c < CR; ++c)
#pragma unroll
                for (int i = 0; i < WW; ++i)
                    asm volatile("" : "+v"(wr[c][i]));
            dot_pass(base, t, acc0, acc1, ss);
        }
        float s = wave_sum(acc0 + acc1);
        if (tscale)
            s *= tscale[t];
        else if constexpr (NORM)
            s *= inv_rms_of(ss, H, eps);
        if (lane == 0)
            out[(uint64_t)t * out_stride] = s;
    }
}

// Q4 row . x for every token (a Q4 router row or shared gate row): lane l
// takes the 32-column chunks l + 64 c; the row is s . sum(q x) + b . sum(x)
// per group, the factored form of the dequantised row.
template <int SBT, int CS, bool NORM>
__device__ __forceinline__ void q4_row_dots(const Q4Rows& m, uint64_t row, const float* x, uint32_t T, uint32_t H,
                                            float* out, uint32_t out_stride, const float* norm_w, float eps,
                                            const float* tscale = nullptr)
{
    const int lane = threadIdx.x & 63;
    const uint32_t chunks = H / 32, gpr = H >> m.gshift;
    const uint4* wp = reinterpret_cast<const uint4*>(m.codes + row * (H / 2));
    uint4 w[CS];
    float sc[CS], bi[CS];
#pragma unroll
    for (int c = 0; c < CS; ++c) {
        const uint32_t ch = lane + WAVE * c;
        w[c] = make_uint4(0, 0, 0, 0);
        sc[c] = 0.0f, bi[c] = 0.0f;
        if (ch < chunks) {
            w[c] = wp[ch];
            const uint64_t gi = row * gpr + ((ch * 32u) >> m.gshift);
            sc[c] = sb_at<SBT>(m.scales, gi);
            bi[c] = sb_at<SBT>(m.biases, gi);
        }
    }
    for (uint32_t t = 0; t < T; ++t) {
#pragma unroll
        for (int c = 0; c < CS; ++c) // keep the nibble conversions inside the token loop
            asm volatile("" : "+v"(w[c].x), "+v"(w[c].y), "+v"(w[c].z), "+v"(w[c].w));
        float p = 0.0f, ss = 0.0f;
#pragma unroll
        for (int c = 0; c < CS; ++c) {
            const uint32_t ch = lane + WAVE * c;
            if (ch < chunks) {
                float xv[32];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float4 u, v;
                    load_x8<NORM>(x, (uint64_t)t * H + ch * 32 + 8 * q, norm_w, ch * 32 + 8 * q, u, v, ss);
                    xv[8 * q] = u.x, xv[8 * q + 1] = u.y, xv[8 * q + 2] = u.z, xv[8 * q + 3] = u.w;
                    xv[8 * q + 4] = v.x, xv[8 * q + 5] = v.y, xv[8 * q + 6] = v.z, xv[8 * q + 7] = v.w;
                }
                float xs = 0.0f;
#pragma unroll
                for (int q = 0; q < 32; q += 8)
                    xs += ((xv[q] + xv[q + 1]) + (xv[q + 2] + xv[q + 3])) +
                          ((xv[q + 4] + xv[q + 5]) + (xv[q + 6] + xv[q + 7]));
                p = fmaf(sc[c], q4_chunk_qx_reg(w[c], xv), fmaf(bi[c], xs, p));
            }
        }
        float r = wave_sum(p);
        if (tscale)
            r *= tscale[t];
        else if constexpr (NORM)
            r *= inv_rms_of(ss, H, eps);
        if (lane == 0)
            out[(uint64_t)t * out_stride] = r;
    }
}

// Several tokens (XL): grid (task workgroups, token groups of XL_FLOATS / H
// tokens); a workgroup stages its group's rows of x in LDS by coalesced
// loads (times the norm weight when the norm is fused), so that a wave's row
// runs every token of the group from LDS instead of one L2 round trip per
// token, and the groups' workgroups run side by side.
constexpr uint32_t XL_FLOATS = 8192; // staged x floats (32 KB)
constexpr uint32_t XL_MAX_H = 8192;  // widest row of the staged variant
// dynamic LDS of the staged variant: the x rows (32 KB, four workgroups per
// CU with or without a fused norm)
inline size_t xl_lds_bytes(uint32_t, bool) { return XL_FLOATS * sizeof(float); }

template <int WDT, int GDT, int SBT, int CR, int CS, bool XL>
__global__ __launch_bounds__(256) void router_stage_kernel(RouterArgs a)
{
    const int lane = threadIdx.x & 63;
    const uint32_t H = a.hidden, T = a.tokens;
    const uint32_t n_router = a.experts;
    const uint32_t Is = a.shared_rows;
    const uint32_t n_tasks = n_router + Is + (a.gate_task ? 1u : 0u);
    const uint32_t wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t n_waves = gridDim.x * 4;
    // task over tokens t0 .. t0 + nt - 1 with their rows at x (row t at
    // x + t H); norm_w (used when NORM), tscale as for the row helpers
    auto run_task = [&](auto norm_tag, uint32_t task, const float* x, uint32_t t0, uint32_t nt, const float* norm_w,
                        const float* tscale) {
        constexpr bool NORM = decltype(norm_tag)::value;
        if (task < n_router) {
            if constexpr (WDT == (int)DT_Q4)
                q4_row_dots<SBT, CS, NORM>(a.router_q4, task, x, nt, H, a.logits + (uint64_t)t0 * n_router + task,
                                           n_router, norm_w, a.eps, tscale);
            else
                dense_row_dots<WDT, CR, NORM>(a.router_w, (uint64_t)task * H, x, nt, H,
                                              a.logits + (uint64_t)t0 * n_router + task, n_router, norm_w, a.eps,
                                              tscale);
        } else if (task < n_router + Is) {
            const uint32_t i = task - n_router;
            const ExpertSet& s = a.sh;
            const uint32_t chunks = H / 32, gpr = H >> s.group_shift;
            const uint4* gw = reinterpret_cast<const uint4*>(s.base + s.gate.w_off + (uint64_t)i * (H / 2));
            const uint4* uw = reinterpret_cast<const uint4*>(s.base + s.up.w_off + (uint64_t)i * (H / 2));
            // unconditional loads (a lane's chunk past the row reloads the
            // last chunk; its products are masked below): a load inside a
            // per-lane branch is waited for at the end of the branch
            uint4 wg[CS], wu[CS];
            float sg[CS], bg[CS], su[CS], bu[CS];
#pragma unroll
            for (int c = 0; c < CS; ++c) {
                const uint32_t ch = min((uint32_t)(lane + WAVE * c), chunks - 1);
                wg[c] = gw[ch];
                wu[c] = uw[ch];
                const uint64_t gi = (uint64_t)i * gpr + ((ch * 32u) >> s.group_shift);
                sg[c] = sb_at<SBT>(s.base + s.gate.s_off, gi);
                bg[c] = sb_at<SBT>(s.base + s.gate.b_off, gi);
                su[c] = sb_at<SBT>(s.base + s.up.s_off, gi);
                bu[c] = sb_at<SBT>(s.base + s.up.b_off, gi);
            }
            for (uint32_t t = 0; t < nt; ++t) {
                float pg = 0.0f, pu = 0.0f, ss = 0.0f;
                // x of one chunk (times the norm weight), its sum and the
                // two products
                auto chunk = [&](int c, const float(&xc)[32]) __attribute__((always_inline)) {
                    float xs = 0.0f;
#pragma unroll
                    for (int q = 0; q < 32; q += 8)
                        xs += ((xc[q] + xc[q + 1]) + (xc[q + 2] + xc[q + 3])) +
                              ((xc[q + 4] + xc[q + 5]) + (xc[q + 6] + xc[q + 7]));
                    const float qg = q4_chunk_qx_reg(wg[c], xc);
                    const float qu = q4_chunk_qx_reg(wu[c], xc);
                    pg = fmaf(sg[c], qg, fmaf(bg[c], xs, pg));
                    pu = fmaf(su[c], qu, fmaf(bu[c], xs, pu));
                };
                auto load_chunk = [&](int c, float(&xc)[32], float& ssc) __attribute__((always_inline)) {
                    const uint32_t ch = min((uint32_t)(lane + WAVE * c), chunks - 1);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        float4 u4, v4;
                        load_x8<NORM>(x, (uint64_t)t * H + ch * 32 + 8 * q, norm_w, ch * 32 + 8 * q, u4, v4, ssc);
                        xc[8 * q] = u4.x, xc[8 * q + 1] = u4.y, xc[8 * q + 2] = u4.z, xc[8 * q + 3] = u4.w;
                        xc[8 * q + 4] = v4.x, xc[8 * q + 5] = v4.y, xc[8 * q + 6] = v4.z, xc[8 * q + 7] = v4.w;
                    }
                };
                if constexpr (CS <= 2) {
                    // the token's x first, so that its loads are in flight
                    // with the weights' (one round trip), then the opaque
                    // step, which waits for the weights
                    float xv[CS][32];
                    float ssc[CS];
#pragma unroll
                    for (int c = 0; c < CS; ++c) {
                        ssc[c] = 0.0f;
                        load_chunk(c, xv[c], ssc[c]);
                    }
                    asm volatile("" ::: "memory");
                    // the nibble conversions do not depend on the token:
                    // without this opaque step the compiler hoists them out
                    // of the loop
#pragma unroll
                    for (int c = 0; c < CS; ++c) {
                        asm volatile("" : "+v"(wg[c].x), "+v"(wg[c].y), "+v"(wg[c].z), "+v"(wg[c].w));
                        asm volatile("" : "+v"(wu[c].x), "+v"(wu[c].y), "+v"(wu[c].z), "+v"(wu[c].w));
                    }
#pragma unroll
                    for (int c = 0; c < CS; ++c)
                        if (lane + WAVE * c < chunks) {
                            ss += ssc[c];
                            chunk(c, xv[c]);
                        }
                } else {
                    // four chunks per lane: 128 floats of x would cost waves
                    // per SIMD; x one chunk at a time (32 floats per chunk
                    // and matrix in the conversions: one wave per SIMD if
                    // hoisted, hence the opaque step)
#pragma unroll
                    for (int c = 0; c < CS; ++c) {
                        asm volatile("" : "+v"(wg[c].x), "+v"(wg[c].y), "+v"(wg[c].z), "+v"(wg[c].w));
                        asm volatile("" : "+v"(wu[c].x), "+v"(wu[c].y), "+v"(wu[c].z), "+v"(wu[c].w));
                    }
#pragma unroll
                    for (int c = 0; c < CS; ++c) {
                        float xc[32];
                        float ssc = 0.0f;
                        load_chunk(c, xc, ssc);
                        if (lane + WAVE * c < chunks) {
                            ss += ssc;
                            chunk(c, xc);
                        }
                    }
                }
                float g = wave_sum(pg);
                float u = wave_sum(pu);
                if (tscale) {
                    g *= tscale[t], u *= tscale[t];
                } else if constexpr (NORM) {
                    const float inv = inv_rms_of(ss, H, a.eps);
                    g *= inv, u *= inv;
                }
                if (lane == 0)
                    a.act_shared[(uint64_t)(t0 + t) * Is + i] = (g / (1.0f + expf(-g))) * u;
            }
        } else if (a.sgate_w) {
            if constexpr (GDT == (int)DT_Q4)
                q4_row_dots<SBT, CS, NORM>(a.sgate_q4, 0, x, nt, H, a.shared_weight + t0, 1, norm_w, a.eps, tscale);
            else
                dense_row_dots<GDT, CR, NORM>(a.sgate_w, 0, x, nt, H, a.shared_weight + t0, 1, norm_w, a.eps, tscale);
            // sigma applied by the consumer: shared_weight holds the gate logit
        } else if (lane == 0) {
            for (uint32_t t = 0; t < nt; ++t)
                a.shared_weight[t0 + t] = 80.0f; // sigma(80) = 1 (metal/mod.rs:4666-4669)
        }
    };
    if constexpr (!XL) {
        if (a.norm_w) {
            for (uint32_t task = wave_id; task < n_tasks; task += n_waves)
                run_task(std::true_type{}, task, a.x, 0, T, a.norm_w, nullptr);
        } else {
            for (uint32_t task = wave_id; task < n_tasks; task += n_waves)
                run_task(std::false_type{}, task, a.x, 0, T, nullptr, nullptr);
        }
    } else {
        extern __shared__ __align__(16) float xl_dyn[]; // xl_lds_bytes
        float* const xsh = xl_dyn;
        __shared__ float inv_sh[XL_FLOATS / 256];     // per token of the group (H >= 256)
        __shared__ float ss_sh[XL_FLOATS / 256][4];   // per token and wave: partial sums of squares
        const uint32_t TG = XL_FLOATS / H, H4 = H / 4;
        const uint32_t g0 = blockIdx.y * TG, nt = min(TG, T - g0), n4 = nt * H4;
        constexpr int PER = XL_FLOATS / 4 / 256; // float4 per thread
        const float4* src = reinterpret_cast<const float4*>(a.x + (uint64_t)g0 * H);
        if (a.norm_w) {
            // the staged rows are x times the norm weight (one buffer: the
            // workgroup's LDS stays at 32 KB); the sums of squares of x are
            // taken from the loaded values, per slot, then per token
            const float4* nsrc = reinterpret_cast<const float4*>(a.norm_w);
            float4 xv[PER], wv4[PER];
#pragma unroll
            for (int j = 0; j < PER; ++j) { // unconditional loads: slots past the data reload the last float4
                const uint32_t i = min(threadIdx.x + 256u * j, n4 - 1);
                xv[j] = src[i];
                wv4[j] = nsrc[i % H4];
            }
            float ssp[PER];
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const float4 q = xv[j], w = wv4[j];
                reinterpret_cast<float4*>(xsh)[threadIdx.x + 256u * j] =
                    make_float4(q.x * w.x, q.y * w.y, q.z * w.z, q.w * w.w);
                float sq = 0.0f;
                sq = fmaf(q.x, q.x, sq), sq = fmaf(q.y, q.y, sq), sq = fmaf(q.z, q.z, sq), sq = fmaf(q.w, q.w, sq);
                ssp[j] = threadIdx.x + 256u * j < n4 ? sq : 0.0f;
            }
            const int wv = threadIdx.x >> 6;
            for (uint32_t t = 0; t < nt; ++t) {
                float p = 0.0f;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    p += (threadIdx.x + 256u * j) / H4 == t ? ssp[j] : 0.0f;
                p = wave_sum(p);
                if (lane == 0)
                    ss_sh[t][wv] = p;
            }
            __syncthreads();
            if (threadIdx.x < nt) {
                const float ss = (ss_sh[threadIdx.x][0] + ss_sh[threadIdx.x][1]) +
                                 (ss_sh[threadIdx.x][2] + ss_sh[threadIdx.x][3]);
                inv_sh[threadIdx.x] = 1.0f / sqrtf(ss / (float)H + a.eps);
            }
            __syncthreads();
        } else {
#pragma unroll
            for (int j = 0; j < PER; ++j)
                reinterpret_cast<float4*>(xsh)[threadIdx.x + 256u * j] = src[min(threadIdx.x + 256u * j, n4 - 1)];
            __syncthreads();
        }
        // with a norm: x already times its weight, the 1 / rms per token as tscale
        if (wave_id < n_tasks)
            run_task(std::false_type{}, wave_id, xsh, g0, nt, nullptr, a.norm_w ? inv_sh : nullptr);
    }
    // the extra last workgroup (no tasks) writes the normalised rows for the
    // gate/up kernel
    if constexpr (!XL) {
        // all four waves on each token: every thread's x and norm-weight
        // loads (H <= 8192: at most 8 float4 each) issued at once, the sum
        // of squares through LDS, the row written from registers (one round
        // trip; one wave per token paid two dependent passes)
        if (a.norm_w && blockIdx.x == gridDim.x - 1) {
            __shared__ float nrm[4];
            constexpr int NF = 8;
            const uint32_t H4 = H / 4;
            const float4* wr4 = reinterpret_cast<const float4*>(a.norm_w);
            for (uint32_t t = 0; t < T; ++t) {
                const float4* xr = reinterpret_cast<const float4*>(a.x + (uint64_t)t * H);
                float4 v[NF], w[NF];
#pragma unroll
                for (int j = 0; j < NF; ++j) { // unconditional: slots past the row reload its last float4
                    const uint32_t i = min(threadIdx.x + 256u * j, H4 - 1);
                    v[j] = xr[i];
                    w[j] = wr4[i];
                }
                float ss = 0.0f;
#pragma unroll
                for (int j = 0; j < NF; ++j)
                    if (threadIdx.x + 256u * j < H4) {
                        const float4 q = v[j];
                        ss = fmaf(q.x, q.x, ss), ss = fmaf(q.y, q.y, ss), ss = fmaf(q.z, q.z, ss), ss = fmaf(q.w, q.w, ss);
                    }
                ss = wave_sum(ss);
                if (lane == 0)
                    nrm[threadIdx.x >> 6] = ss;
                __syncthreads();
                const float inv = 1.0f / sqrtf(((nrm[0] + nrm[1]) + (nrm[2] + nrm[3])) / (float)H + a.eps);
#pragma unroll
                for (int j = 0; j < NF; ++j) {
                    const uint32_t i = threadIdx.x + 256u * j;
                    if (i < H4) {
                        const float4 q = v[j], ww = w[j];
                        reinterpret_cast<float4*>(a.x_out + (uint64_t)t * H)[i] =
                            make_float4((q.x * inv) * ww.x, (q.y * inv) * ww.y, (q.z * inv) * ww.z, (q.w * inv) * ww.w);
                    }
                }
                __syncthreads(); // nrm is read before the next token writes it
            }
        }
    } else if (a.norm_w && blockIdx.x == gridDim.x - 1) {
        // XL: the tokens of this workgroup's group, wave w the tokens w, w + 4, ...
        const uint32_t tb = XL ? blockIdx.y * (XL_FLOATS / H) : 0u;
        const uint32_t te = XL ? min(tb + XL_FLOATS / H, T) : T;
        for (uint32_t t = tb + (threadIdx.x >> 6); t < te; t += 4) {
            const float* xr = a.x + (uint64_t)t * H;
            float ss = 0.0f;
            for (uint32_t i = (uint32_t)lane * 4; i < H; i += 256) {
                const float4 v = *reinterpret_cast<const float4*>(xr + i);
                ss = fmaf(v.x, v.x, ss), ss = fmaf(v.y, v.y, ss), ss = fmaf(v.z, v.z, ss), ss = fmaf(v.w, v.w, ss);
            }
            const float inv = inv_rms_of(ss, H, a.eps);
            for (uint32_t i = (uint32_t)lane * 4; i < H; i += 256) {
                const float4 v = *reinterpret_cast<const float4*>(xr + i);
                const float4 w = *reinterpret_cast<const float4*>(a.norm_w + i);
                *reinterpret_cast<float4*>(a.x_out + (uint64_t)t * H + i) =
                    make_float4((v.x * inv) * w.x, (v.y * inv) * w.y, (v.z * inv) * w.z, (v.w * inv) * w.w);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Routing + plan in LDS, redone by every workgroup of kernel 2 from the
// published logits (or loaded when the caller gave the routes).
// ---------------------------------------------------------------------------
struct RouteLds {
    uint32_t ids[DEC_ROUTES];
    float w[DEC_ROUTES];
    uint32_t unique_ids[DEC_ROUTES];
    uint32_t groups[2 * DEC_ROUTES];
    uint32_t src_rows[DEC_ROUTES];
    uint32_t out_idx[DEC_ROUTES];
    uint32_t count[1024];
    uint32_t start[1024];
    uint32_t unique_count;
    uint32_t sel[4][MAX_K];
    // 16-byte aligned: the routing code reads and writes 64-bit keys here
    // (an LDS access of 8 bytes at an address that is 4 mod 8 runs far slower)
    alignas(16) float grp[4][2048 + 192];
};

// Stable plan of `routes` routes from s.ids (block-wide, routes <= 256):
// sorted unique union and stable grouping by expert, the definition of the
// standalone plan kernel (metal/mod.rs:3197-3233, scheduler/mod.rs:685-769).
__device__ void lds_plan(RouteLds& s, uint32_t routes, uint32_t experts, uint32_t k, uint32_t* status)
{
    const int tid = threadIdx.x;
    for (uint32_t e = tid; e < 1024; e += blockDim.x)
        s.count[e] = 0;
    __syncthreads();
    for (uint32_t r = tid; r < routes; r += blockDim.x) {
        const uint32_t e = s.ids[r];
        if (e < experts)
            atomicAdd(&s.count[e], 1u);
        else
            atomicOr(status, ST_ROUTE_RANGE);
    }
    __syncthreads();
    if (tid < 64) { // one wave scans the 1024 counters, 16 per lane
        uint32_t c[16], run_c = 0, run_f = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            c[j] = s.count[tid * 16 + j];
            run_c += c[j];
            run_f += c[j] ? 1u : 0u;
        }
        uint32_t inc_c = run_c, inc_f = run_f;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t x = __shfl_up(inc_c, o);
            const uint32_t y = __shfl_up(inc_f, o);
            if (tid >= o) {
                inc_c += x;
                inc_f += y;
            }
        }
        uint32_t base_c = inc_c - run_c, base_f = inc_f - run_f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t e = tid * 16 + j;
            s.start[e] = base_c;
            if (c[j] && e < experts) {
                s.unique_ids[base_f] = e;
                s.groups[2 * base_f] = base_c;
                s.groups[2 * base_f + 1] = c[j];
            }
            base_c += c[j];
            base_f += c[j] ? 1u : 0u;
        }
        if (tid == 63)
            s.unique_count = inc_f;
    }
    __syncthreads();
    for (uint32_t r = tid; r < routes; r += blockDim.x) {
        const uint32_t e = s.ids[r];
        if (e >= experts) {
            s.out_idx[r] = 0xFFFFFFFFu;
            continue;
        }
        uint32_t rank = 0;
        for (uint32_t q = 0; q < r; ++q)
            rank += s.ids[q] == e ? 1u : 0u;
        const uint32_t pos = s.start[e] + rank;
        s.src_rows[pos] = r / k;
        s.out_idx[r] = pos;
    }
    __syncthreads();
}

struct ExpertArgs {
    ExpertSet ex;
    const float* logits;      // route from these when route_here
    const float* sel_bias;
    RouteParams rp;
    bool route_here;          // false: ids/weights given
    uint32_t* ids;            // [T][K]
    float* weights;           // [T][K]
    Plan plan;                // global copy for kernel 3 (tokens > 1)
    const float* x;
    uint32_t tokens, hidden;
    float* act;               // [T*K][I]
    uint32_t* status;
    ExpertSet sh;             // shared expert (has_shared)
    bool has_shared;
    uint32_t pf_base;         // first down-prefetch workgroup (multiple of 8)
    uint32_t pf_wgs;          // down-prefetch workgroups (multiple of 8, 0: none)
    bool pf_paired;           // the down kernel maps row blocks by down_row_block
    uint32_t shared_rows;     // one token: the shared expert's gate/up rows, computed by the
                              // prefetch workgroups before they route (0: by the router stage)
    float* act_shared;        // [Is]
};

constexpr int PF_LINES = 4; // cache lines touched per prefetch lane per round
// workgroups of route_gateup_kernel resident at once on gfx950: 256 CUs x 3
// (the routing scratch in LDS limits a CU to three); prefetch workgroups are
// added only while the whole grid fits in that one round
constexpr uint32_t GATEUP_RESIDENT_WGS = 768;

// Row block of down_rows_kernel workgroup b in a grid of a multiple of 16
// workgroups: the 64-byte scale and bias runs of blocks 2m and 2m + 1 share
// 128-byte lines, so the pair goes to one XCD (workgroup b runs on XCD
// b % 8): workgroups b and b + 8 of XCD x take blocks 16j + 2x and
// 16j + 2x + 1.  Other grids: block b.
__host__ __device__ inline uint32_t down_row_block(uint32_t b, uint32_t grid)
{
    if (grid % 16)
        return b;
    const uint32_t x = b & 7, q = b >> 3;
    return 16 * (q >> 1) + 2 * x + (q & 1);
}

// Down-weight prefetch: touch every 128-byte line of the down codes, scales
// and biases of the selected experts (and the shared expert) while the
// gate/up workgroups run, so that the down kernel finds them in the L2 /
// MALL instead of HBM.  Row block rb (DOWN_R output rows) is read by down
// workgroup rb (down_combine_kernel: XCD rb % 8), or by the workgroup
// down_row_block assigns it (down_rows_kernel, pf_paired: XCD (rb / 2) % 8);
// a prefetch workgroup on XCD x touches only that XCD's blocks.
// lane0/lanes: this lane's index among the lanes of this XCD that share the
// work, and their number.  Returns a value that depends on every load.
__device__ uint32_t touch_down_lines(const ExpertArgs& a, const RouteLds& s, uint32_t n_routed, bool use_plan,
                                     uint32_t lane0, uint32_t lanes)
{
    const uint32_t xcd = blockIdx.x & 7;
    const uint32_t I = a.ex.down.cols;
    const uint32_t gpr = I >> a.ex.group_shift;
    const uint32_t blk_w = DOWN_R * I / 2;   // code bytes of one row block
    const uint32_t blk_sb = DOWN_R * gpr * 2; // scale (bias) bytes of one row block
    const uint32_t w_lines = (blk_w + 127) / 128, s_lines = (blk_sb + 127) / 128;
    const uint32_t per_block = w_lines + 2 * s_lines;
    const uint32_t n_blocks = a.hidden / DOWN_R;
    // this XCD's blocks: xcd + 8i, or (pf_paired) 16 (i / 2) + 2 xcd + i % 2
    const uint32_t per_item = a.pf_paired ? (n_blocks / 16) * 2 : (n_blocks > xcd ? (n_blocks - xcd + 7) / 8 : 0u);
    const uint32_t n_items = n_routed + (a.has_shared ? 1u : 0u);
    const uint32_t total = n_items * per_item * per_block;
    uint32_t acc = 0;
    for (uint32_t base = lane0; base < total; base += lanes * PF_LINES) {
        uint32_t v[PF_LINES];
#pragma unroll
        for (int u = 0; u < PF_LINES; ++u) {
            v[u] = 0;
            const uint32_t L = base + lanes * u;
            if (L >= total)
                continue;
            const uint32_t b = L / per_block, off = L % per_block;
            const uint32_t item = b / per_item;
            const uint32_t i = b % per_item;
            const uint32_t rb = a.pf_paired ? 16 * (i >> 1) + 2 * xcd + (i & 1) : xcd + 8 * i;
            const bool shared = item == n_routed;
            const ExpertSet& set = shared ? a.sh : a.ex;
            const uint8_t* slot = set.base;
            if (!shared) {
                const uint32_t e = use_plan ? s.unique_ids[item] : s.ids[item];
                if (e >= a.ex.count)
                    continue;
                slot += (uint64_t)e * a.ex.stride;
            }
            const uint8_t* p;
            if (off < w_lines)
                p = slot + set.down.w_off + (uint64_t)rb * blk_w + off * 128u;
            else if (off < w_lines + s_lines)
                p = slot + set.down.s_off + (uint64_t)rb * blk_sb + (off - w_lines) * 128u;
            else
                p = slot + set.down.b_off + (uint64_t)rb * blk_sb + (off - w_lines - s_lines) * 128u;
            v[u] = *reinterpret_cast<const uint32_t*>(p);
        }
#pragma unroll
        for (int u = 0; u < PF_LINES; ++u)
            acc ^= v[u];
    }
    return acc;
}

template <int EPL>
__device__ void route_all_tokens(const ExpertArgs& a, RouteLds& s, bool need_w)
{
    const int wv = threadIdx.x >> 6;
    const uint32_t K = a.rp.k;
    if (block_routing(a.tokens, a.rp)) {
        // decode tokens: all four waves route each token in turn
        constexpr int EPT = EPL <= 4 ? 1 : (EPL <= 8 ? 2 : 4); // ceil(E / 256) bucket
        for (uint32_t t = 0; t < a.tokens; ++t) {
            if (t)
                __syncthreads(); // scratch reuse
            route_token_block<EPT>(a.logits + (uint64_t)t * a.rp.experts, a.sel_bias, a.rp, s.ids + t * K,
                                   s.w + t * K, &s.grp[0][0], a.status, need_w);
        }
        return;
    }
    for (uint32_t t = wv; t < a.tokens; t += 4)
        route_token_wave<EPL>(a.logits + (uint64_t)t * a.rp.experts, a.sel_bias, a.rp, s.ids + t * K,
                              s.w + t * K, s.sel[wv], s.grp[wv], a.status);
}

// ---------------------------------------------------------------------------
// kernel 2: routing (every workgroup) + routed gate/up with SiLU(g)*u.
// Task = (work item, RPW consecutive rows) per wave.
// ---------------------------------------------------------------------------
// One shared-expert gate/up row of one token (x already normalised):
// SiLU(g) * u into *out (lane 0).  Lane l takes the 32-column chunks
// l + 64 c; every load is issued before the first wait (chunks past the row
// reload the last one and are masked).
template <int SBT, int CPL>
__device__ __forceinline__ void shared_row_one_token(const ExpertSet& sh, uint32_t i, const float* __restrict__ x,
                                                     uint32_t H, float* out)
{
    const int lane = threadIdx.x & 63;
    const uint32_t chunks = H / 32, gpr = H >> sh.group_shift;
    const uint4* gw = reinterpret_cast<const uint4*>(sh.base + sh.gate.w_off + (uint64_t)i * (H / 2));
    const uint4* uw = reinterpret_cast<const uint4*>(sh.base + sh.up.w_off + (uint64_t)i * (H / 2));
    const uint16_t* gs = reinterpret_cast<const uint16_t*>(sh.base + sh.gate.s_off) + (uint64_t)i * gpr;
    const uint16_t* gb = reinterpret_cast<const uint16_t*>(sh.base + sh.gate.b_off) + (uint64_t)i * gpr;
    const uint16_t* us = reinterpret_cast<const uint16_t*>(sh.base + sh.up.s_off) + (uint64_t)i * gpr;
    const uint16_t* ub = reinterpret_cast<const uint16_t*>(sh.base + sh.up.b_off) + (uint64_t)i * gpr;
    uint4 wg[CPL], wu[CPL];
    uint32_t sg[CPL], bg[CPL], su[CPL], bu[CPL];
    float xv[CPL][32];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const uint32_t ch = min((uint32_t)(lane + WAVE * c), chunks - 1);
        const uint32_t g = (ch * 32u) >> sh.group_shift;
        wg[c] = gw[ch];
        wu[c] = uw[ch];
        sg[c] = gs[g];
        bg[c] = gb[g];
        su[c] = us[g];
        bu[c] = ub[g];
        const float4* x4 = reinterpret_cast<const float4*>(x + ch * 32);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = x4[q];
            xv[c][4 * q] = v.x, xv[c][4 * q + 1] = v.y, xv[c][4 * q + 2] = v.z, xv[c][4 * q + 3] = v.w;
        }
    }
    float pg = 0.0f, pu = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        if (lane + WAVE * c < chunks) {
            float xs = 0.0f;
#pragma unroll
            for (int q = 0; q < 32; q += 4)
                xs += (xv[c][q] + xv[c][q + 1]) + (xv[c][q + 2] + xv[c][q + 3]);
            const float qg = q4_chunk_qx_reg(wg[c], xv[c]);
            const float qu = q4_chunk_qx_reg(wu[c], xv[c]);
            pg = fmaf(sb_bits<SBT>(sg[c]), qg, fmaf(sb_bits<SBT>(bg[c]), xs, pg));
            pu = fmaf(sb_bits<SBT>(su[c]), qu, fmaf(sb_bits<SBT>(bu[c]), xs, pu));
        }
    }
    const float g = wave_sum(pg);
    const float u = wave_sum(pu);
    if (lane == 0)
        *out = (g / (1.0f + expf(-g))) * u;
}

template <int SBT, int CPL, int RPW, int EPL>
__global__ __launch_bounds__(256) void route_gateup_kernel(ExpertArgs a)
{
    __shared__ RouteLds s;
    const int lane = threadIdx.x & 63;
    const uint32_t T = a.tokens, K = a.rp.k, H = a.hidden, I = a.ex.gate.rows;
    const uint32_t routes = T * K;
    const bool use_plan = T > 1;

    if (a.shared_rows && blockIdx.x >= a.pf_base) {
        // the shared expert's rows of the one token need no routes: the
        // prefetch workgroups take them first (in the router stage their
        // weights arrived last and held back this launch), wave w of
        // prefetch workgroup b the rows 4 b + w, + 4 pf_wgs, ...
        const uint32_t w0 = (blockIdx.x - a.pf_base) * 4 + (threadIdx.x >> 6);
        for (uint32_t i = w0; i < a.shared_rows; i += a.pf_wgs * 4)
            shared_row_one_token<SBT, CPL>(a.sh, i, a.x, H, a.act_shared + i);
    }

    if (a.route_here) {
        // only the publishing workgroup needs the route weights (the down
        // kernel reads them); the others select the ids and move on to
        // their weight loads sooner
        route_all_tokens<EPL>(a, s, blockIdx.x == 0);
    } else {
        for (uint32_t r = threadIdx.x; r < routes; r += blockDim.x) {
            s.ids[r] = a.ids[r];
            s.w[r] = a.weights[r];
        }
    }
    __syncthreads();
    if (use_plan)
        lds_plan(s, routes, a.rp.experts, K, a.status);
    if (blockIdx.x == 0) { // publish routes and plan for kernel 3 and the caller
        for (uint32_t r = threadIdx.x; r < routes; r += blockDim.x) {
            if (a.route_here) {
                a.ids[r] = s.ids[r];
                a.weights[r] = s.w[r];
            }
            if (use_plan) {
                a.plan.src_rows[r] = s.src_rows[r];
                a.plan.out_idx[r] = s.out_idx[r];
            }
        }
        if (use_plan) {
            for (uint32_t u = threadIdx.x; u < s.unique_count; u += blockDim.x) {
                a.plan.unique_ids[u] = s.unique_ids[u];
                a.plan.groups[2 * u] = s.groups[2 * u];
                a.plan.groups[2 * u + 1] = s.groups[2 * u + 1];
            }
            if (threadIdx.x == 0)
                a.plan.unique_count[0] = s.unique_count;
        }
    }

    const uint32_t n_items = use_plan ? s.unique_count : routes;
    if (a.pf_wgs && blockIdx.x >= a.pf_base) { // down-prefetch workgroups
        const uint32_t acc = touch_down_lines(a, s, n_items, use_plan,
                                              ((blockIdx.x - a.pf_base) >> 3) * blockDim.x + threadIdx.x,
                                              (a.pf_wgs >> 3) * blockDim.x);
        asm volatile("" ::"v"(acc));
        return;
    }
    const uint32_t row_tasks = I / RPW;
    const uint32_t wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t item = wave_id / row_tasks;
    const uint32_t row0 = (wave_id % row_tasks) * RPW;
    if (item >= n_items)
        return;
    uint32_t e, g0, n;
    if (use_plan) {
        e = s.unique_ids[item];
        g0 = s.groups[2 * item];
        n = s.groups[2 * item + 1];
    } else {
        e = s.ids[item];
        g0 = item;
        n = 1;
    }
    if (e >= a.ex.count) {
        if (lane == 0)
            atomicOr(a.status, ST_ROUTE_RANGE);
        return;
    }
    const ExpertSet& ex = a.ex;
    const uint8_t* slot = ex.base + (uint64_t)e * ex.stride;
    const uint32_t chunks = H / 32, gpr = H >> ex.group_shift;
    // Every weight load is issued before anything waits on them: no load
    // sits in a branch (a load inside a divergent branch is waited on at the
    // branch's end); lanes past the row's last chunk load that chunk again
    // and do not use it.
    uint4 wg[RPW][CPL], wu[RPW][CPL];
    uint32_t sgr[RPW][CPL], bgr[RPW][CPL], sur[RPW][CPL], bur[RPW][CPL]; // raw 16-bit scale / bias
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint32_t row = row0 + r;
        const uint4* gw = reinterpret_cast<const uint4*>(slot + ex.gate.w_off + (uint64_t)row * (H / 2));
        const uint4* uw = reinterpret_cast<const uint4*>(slot + ex.up.w_off + (uint64_t)row * (H / 2));
        const uint16_t* gs = reinterpret_cast<const uint16_t*>(slot + ex.gate.s_off) + (uint64_t)row * gpr;
        const uint16_t* gb = reinterpret_cast<const uint16_t*>(slot + ex.gate.b_off) + (uint64_t)row * gpr;
        const uint16_t* us = reinterpret_cast<const uint16_t*>(slot + ex.up.s_off) + (uint64_t)row * gpr;
        const uint16_t* ub = reinterpret_cast<const uint16_t*>(slot + ex.up.b_off) + (uint64_t)row * gpr;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = min(lane + WAVE * c, chunks - 1);
            const uint32_t g = (ch * 32u) >> ex.group_shift;
            wg[r][c] = gw[ch];
            wu[r][c] = uw[ch];
            sgr[r][c] = gs[g];
            bgr[r][c] = gb[g];
            sur[r][c] = us[g];
            bur[r][c] = ub[g];
        }
    }
    // one chunk per lane and two rows (X0): the first token's activations
    // are loaded with the weights (with more chunks or rows the registers
    // would cost waves per SIMD)
    constexpr bool X0 = CPL == 1 && RPW == 2;
    float x0[X0 ? 32 : 1];
    if constexpr (X0) {
        const uint32_t tok = use_plan ? s.src_rows[g0] : g0 / K;
        const float4* x4 = reinterpret_cast<const float4*>(a.x + (uint64_t)tok * H + min((uint32_t)lane, chunks - 1) * 32);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = x4[q];
            x0[4 * q] = v.x, x0[4 * q + 1] = v.y, x0[4 * q + 2] = v.z, x0[4 * q + 3] = v.w;
        }
    }
    for (uint32_t j = 0; j < n; ++j) {
        const uint32_t gidx = g0 + j;
        const uint32_t tok = use_plan ? s.src_rows[gidx] : gidx / K;
        const float* xt = a.x + (uint64_t)tok * H;
        // the nibble conversions below do not depend on the token; without
        // this opaque step the compiler hoists all of them out of the loop
        // (hundreds of registers, one wave per SIMD)
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                asm volatile("" : "+v"(wg[r][c].x), "+v"(wg[r][c].y), "+v"(wg[r][c].z), "+v"(wg[r][c].w));
                asm volatile("" : "+v"(wu[r][c].x), "+v"(wu[r][c].y), "+v"(wu[r][c].z), "+v"(wu[r][c].w));
            }
        float pg[RPW], pu[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            pg[r] = 0.0f, pu[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = lane + WAVE * c;
            float xv[32];
            if (X0 && j == 0) {
#pragma unroll
                for (int q = 0; q < 32; ++q)
                    xv[q] = x0[X0 ? q : 0];
            } else if (ch < chunks) {
                const float4* x4 = reinterpret_cast<const float4*>(xt + ch * 32);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = x4[q];
                    xv[4 * q] = v.x, xv[4 * q + 1] = v.y, xv[4 * q + 2] = v.z, xv[4 * q + 3] = v.w;
                }
            }
            if (ch < chunks) {
                float xs = 0.0f;
#pragma unroll
                for (int q = 0; q < 32; q += 4)
                    xs += (xv[q] + xv[q + 1]) + (xv[q + 2] + xv[q + 3]);
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float qg = q4_chunk_qx_reg<RPW * CPL <= 2>(wg[r][c], xv);
                    const float qu = q4_chunk_qx_reg<RPW * CPL <= 2>(wu[r][c], xv);
                    pg[r] = fmaf(sb_bits<SBT>(sgr[r][c]), qg, fmaf(sb_bits<SBT>(bgr[r][c]), xs, pg[r]));
                    pu[r] = fmaf(sb_bits<SBT>(sur[r][c]), qu, fmaf(sb_bits<SBT>(bur[r][c]), xs, pu[r]));
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const float g = wave_sum(pg[r]);
            const float u = wave_sum(pu[r]);
            if (lane == r)
                a.act[(uint64_t)gidx * I + row0 + r] = (g / (1.0f + expf(-g))) * u;
        }
    }
}

// ---------------------------------------------------------------------------
// kernel 2, persistent variant (several tokens; one token of a wide layer):
// grid (workgroups per token, tokens); every workgroup first routes its
// token from the logits (route_here; workgroup 0 of the token publishes
// the routes) or loads the given routes; the workgroups of token t stage
// its x row in LDS once and their waves run over the token's units (route k,
// RPW consecutive rows), strided by the waves of the token; activations in
// route order [T*K][I].  A wave holds two units' weights in registers
// (buffers A and B, alternating, so no register copies): the next unit's
// weights load while this unit is computed.  x comes from LDS, so reading
// it never waits for those loads (and the waves do not all read the same
// few L2 lines: every unit would otherwise load the whole 8 KB row).  Each
// route is its own unit (a token pair that shares an expert reads its
// weights twice, mostly from the MALL).
// ---------------------------------------------------------------------------
template <int CPL, int RPW>
struct UnitWeights {
    uint4 wg[RPW][CPL], wu[RPW][CPL];
    uint32_t sg[RPW][CPL], bg[RPW][CPL], su[RPW][CPL], bu[RPW][CPL]; // raw 16-bit scale / bias
};

template <int SBT, int CPL, int RPW, int EPL>
__global__ __launch_bounds__(256) void gateup_multi_kernel(ExpertArgs a)
{
    // staged chunk q (32 floats) at q * XQ floats: the lanes' 16-byte reads
    // of consecutive chunks fall on distinct banks
    constexpr int XQ = 36;
    constexpr int EPT = EPL <= 4 ? 1 : (EPL <= 8 ? 2 : 4); // ceil(E / 256) bucket of the block routing
    constexpr int RSCR = 2 * EPL * WAVE + 192 > 1176 ? 2 * EPL * WAVE + 192 : 1176;
    __shared__ __align__(16) float xl[WAVE * CPL * XQ];
    __shared__ uint32_t sid[MAX_K];
    __shared__ float sw[MAX_K];
    __shared__ __align__(16) float rscr[RSCR]; // routing scratch (64-bit keys: 8-byte aligned)
    const int lane = threadIdx.x & 63;
    const uint32_t K = a.rp.k, H = a.hidden, I = a.ex.gate.rows;
    const uint32_t t = blockIdx.y;
    const uint32_t chunks = H / 32, gsh = a.ex.group_shift, gpr = H >> gsh;
    {
        // the token's x row (coalesced), loaded before the routes are known
        // and stored after; float4 slots past H / 4 hold zeros in chunks no
        // lane reads
        const uint32_t nf = H / 4;
        float4 v[2 * CPL];
#pragma unroll
        for (int j = 0; j < 2 * CPL; ++j)
            v[j] = reinterpret_cast<const float4*>(a.x + (uint64_t)t * H)[min(threadIdx.x + 256u * j, nf - 1)];
        if (a.route_here) {
            // every workgroup routes its token (the routing launch's own
            // device routines, so the ids agree bitwise); workgroup 0 of
            // the token publishes the routes for the down kernel and the
            // caller
            const float* lt = a.logits + (uint64_t)t * a.rp.experts;
            if (block_routing(a.tokens, a.rp)) {
                route_token_block<EPT>(lt, a.sel_bias, a.rp, sid, sw, rscr, a.status, blockIdx.x == 0);
            } else if (threadIdx.x < 64) {
                uint32_t* sel = reinterpret_cast<uint32_t*>(xl); // (x is stored after the routing)
                route_token_wave<EPL>(lt, a.sel_bias, a.rp, sid, sw, sel, rscr, a.status);
            }
            __syncthreads();
            if (blockIdx.x == 0 && threadIdx.x < K) {
                a.ids[t * K + threadIdx.x] = sid[threadIdx.x];
                a.weights[t * K + threadIdx.x] = sw[threadIdx.x];
            }
        } else {
            const uint32_t idv = a.ids[t * K + min((uint32_t)threadIdx.x, K - 1)];
            if (threadIdx.x < K)
                sid[threadIdx.x] = idv;
        }
#pragma unroll
        for (int j = 0; j < 2 * CPL; ++j) {
            const uint32_t f = threadIdx.x + 256u * j;
            const bool in = f < nf;
            float4 w = v[j];
            w.x = in ? w.x : 0.0f, w.y = in ? w.y : 0.0f, w.z = in ? w.z : 0.0f, w.w = in ? w.w : 0.0f;
            *reinterpret_cast<float4*>(&xl[(f >> 3) * XQ + (f & 7) * 4]) = w;
        }
    }
    __syncthreads();
    const uint32_t row_tasks = I / RPW;
    const uint32_t n_units = K * row_tasks; // this token's
    const uint32_t nw = gridDim.x * 4;
    // the expert set's fields as plain values (uniform)
    const uint8_t* const base = a.ex.base;
    const uint64_t stride = a.ex.stride;
    const uint32_t count = a.ex.count;
    const uint64_t gw_off = a.ex.gate.w_off, gs_off = a.ex.gate.s_off, gb_off = a.ex.gate.b_off;
    const uint64_t uw_off = a.ex.up.w_off, us_off = a.ex.up.s_off, ub_off = a.ex.up.b_off;

    // unconditional loads: a unit past the end loads the last unit again
    auto load_w = [&](uint32_t u, UnitWeights<CPL, RPW>& W) {
        const uint32_t uc = min(u, n_units - 1);
        const uint32_t k = uc / row_tasks, row0 = (uc % row_tasks) * RPW;
        uint32_t e = __builtin_amdgcn_readfirstlane(sid[k]);
        e = e < count ? e : 0u;
        const uint8_t* slot = base + (uint64_t)e * stride;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint32_t row = row0 + r;
            const uint4* gw = reinterpret_cast<const uint4*>(slot + gw_off + (uint64_t)row * (H / 2));
            const uint4* uw = reinterpret_cast<const uint4*>(slot + uw_off + (uint64_t)row * (H / 2));
            const uint16_t* gs = reinterpret_cast<const uint16_t*>(slot + gs_off) + (uint64_t)row * gpr;
            const uint16_t* gb = reinterpret_cast<const uint16_t*>(slot + gb_off) + (uint64_t)row * gpr;
            const uint16_t* us = reinterpret_cast<const uint16_t*>(slot + us_off) + (uint64_t)row * gpr;
            const uint16_t* ub = reinterpret_cast<const uint16_t*>(slot + ub_off) + (uint64_t)row * gpr;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const uint32_t ch = min((uint32_t)(lane + WAVE * c), chunks - 1);
                const uint32_t g = (ch * 32u) >> gsh;
                W.wg[r][c] = gw[ch];
                W.wu[r][c] = uw[ch];
                W.sg[r][c] = gs[g];
                W.bg[r][c] = gb[g];
                W.su[r][c] = us[g];
                W.bu[r][c] = ub[g];
            }
        }
    };
    auto compute = [&](uint32_t u, UnitWeights<CPL, RPW>& W) {
        const uint32_t k = u / row_tasks, row0 = (u % row_tasks) * RPW;
        const bool ok = __builtin_amdgcn_readfirstlane(sid[k]) < count;
        float pg[RPW], pu[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            pg[r] = 0.0f, pu[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = lane + WAVE * c;
            if (ch < chunks) {
                const float4* x4 = reinterpret_cast<const float4*>(&xl[ch * XQ]);
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
                for (int r = 0; r < RPW; ++r) {
                    const float qg = q4_chunk_qx_reg<RPW * CPL <= 2>(W.wg[r][c], xv);
                    const float qu = q4_chunk_qx_reg<RPW * CPL <= 2>(W.wu[r][c], xv);
                    pg[r] = fmaf(sb_bits<SBT>(W.sg[r][c]), qg, fmaf(sb_bits<SBT>(W.bg[r][c]), xs, pg[r]));
                    pu[r] = fmaf(sb_bits<SBT>(W.su[r][c]), qu, fmaf(sb_bits<SBT>(W.bu[r][c]), xs, pu[r]));
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const float g = wave_sum(pg[r]);
            const float up = wave_sum(pu[r]);
            if (ok && lane == r)
                a.act[(uint64_t)(t * K + k) * I + row0 + r] = (g / (1.0f + expf(-g))) * up;
        }
        if (!ok && lane == 0)
            atomicOr(a.status, ST_ROUTE_RANGE);
    };
    UnitWeights<CPL, RPW> A, B;
    uint32_t u = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    load_w(u, A);
    while (u < n_units) {
        load_w(u + nw, B);
        compute(u, A);
        u += nw;
        if (u >= n_units)
            break;
        load_w(u + nw, A);
        compute(u, B);
        u += nw;
    }
}

// ---------------------------------------------------------------------------
// kernel 3: down projection + combine for R output rows per workgroup.
// Unit = (item, row) handled by LPR lanes with CPL chunks each.  When every
// route's activations fit STAGE_FLOATS (one token, or two of C2's) they are
// staged in LDS by loads that do not wait for the routes; otherwise they are
// read from L2 per unit.
// ---------------------------------------------------------------------------
constexpr uint32_t STAGE_FLOATS = 12288; // activations staged (54 KB of LDS in XP-padded chunks)
// Several tokens (down_rows_kernel): one token's routed + shared activations
// (27 KB of LDS).
constexpr uint32_t PT_STAGE_FLOATS = 6144;
// Staged chunk q (32 floats) sits at q * XP floats, so that the lanes'
// 16-byte reads of consecutive chunks fall on distinct banks.
constexpr int XP = 36;

struct DownArgs {
    ExpertSet ex, sh;
    bool has_shared;
    const float* act;
    const float* act_shared;
    const float* shared_logit; // sigma applied here
    uint32_t tokens, k, hidden;
    const uint32_t* ids;
    const float* weights;
    Plan plan;
    bool use_plan;
    bool stage; // every route's activations fit STAGE_FLOATS
    const float* residual;
    float* hidden_out;
    uint32_t* status;
};

// STG: the variant with the LDS staging (direct mode); without it the
// workgroup holds no staging buffer, so more workgroups fit a CU (layers
// whose activations never fit STAGE_FLOATS, such as I = 2048 with K = 8).
// ONE: one token without the dispatch plan only (the token-loop path is not
// compiled, which keeps the registers of the straight-line path low).
template <int SBT, int LPR, int CPL, int MAXR, bool STG, bool ONE = false>
__global__ __launch_bounds__(256) void down_combine_kernel(DownArgs a)
{
    constexpr int R = DOWN_R;
    constexpr int SLOTS = 256 / LPR;
    constexpr uint32_t SF = STAGE_FLOATS;
    constexpr int NR = DEC_ROUTES;
    __shared__ float ylds[NR][R];
    __shared__ float yshl[DEC_T][R];
    __shared__ float c_w[NR];    // combine inputs, loaded at the start
    __shared__ uint32_t c_oi[NR];
    __shared__ float c_sw[DEC_T];
    __shared__ __align__(16) float astage[STG ? SF / 32 * XP : 4];
    __shared__ float xsl[STG ? SF / 32 : 4]; // per-chunk sums of the staged activations
    const bool stage = STG && a.stage;
    const int gl = threadIdx.x % LPR;
    const int slot_id = threadIdx.x / LPR;
    const uint32_t row_base = blockIdx.x * R;
    const uint32_t T = a.tokens, K = a.k;
    const uint32_t I = a.ex.down.cols;
    const uint32_t routes = T * K;
    const bool use_plan = a.use_plan;
    const uint32_t* const ids = a.ids;
    const float* const rweights = a.weights;
    const float* const residual = a.residual;
    float* const hidden_out = a.hidden_out;
    const float* const act_shared = a.act_shared;
    const float* const shared_logit = a.has_shared ? a.shared_logit : rweights;

    // Load order.  Every load below is issued before anything waits on it,
    // and none sits in a branch (a load inside a divergent branch is waited
    // on at the branch's end): the residual, the expert id of each unit (the
    // previous kernel's routes), the activations to stage (direct mode),
    // then the weights, whose addresses need the ids; the staged
    // activations are stored to LDS while the weights are in flight.  Loads
    // of units and chunks that do not exist read a fixed valid address.
    const uint32_t ri = min((uint32_t)threadIdx.x, T * R - 1); // lanes >= T * R do not use it
    const uint32_t rq = min((uint32_t)threadIdx.x, routes - 1), tq = min((uint32_t)threadIdx.x, T - 1);
    // residual, and the combine's route weights, output slots and shared gate
    // logits (each thread one route, routes <= 256, and one token): loaded
    // in every pass right after the expert ids, not at the end where they
    // would cost a round trip, and not before the pass loop, whose header
    // would wait for them
    float res_v = 0.0f, cw_v = 0.0f, csl_v = 0.0f;
    uint32_t coi_v = 0;
    const uint32_t n_routed = use_plan ? a.plan.unique_count[0] : routes;
    const uint32_t n_items = n_routed + (a.has_shared ? 1u : 0u);
    const uint32_t n_units = n_items * R;
    const uint32_t* id_src = use_plan ? a.plan.unique_ids : ids;
    const uint32_t gsh_e = a.ex.group_shift, gsh_s = a.has_shared ? a.sh.group_shift : gsh_e;

    // the fields of both sets as plain values (selected per unit below;
    // selecting through the argument struct would load them per lane)
    const uint8_t* const ex_base = a.ex.base;
    const uint64_t ex_stride = a.ex.stride;
    const uint32_t ex_count = a.ex.count;
    const uint64_t ex_w = a.ex.down.w_off, ex_s = a.ex.down.s_off, ex_b = a.ex.down.b_off;
    const uint8_t* const sh_base = a.has_shared ? a.sh.base : ex_base;
    const uint64_t sh_w = a.sh.down.w_off, sh_s = a.sh.down.s_off, sh_b = a.sh.down.b_off;
    for (uint32_t u0 = 0; u0 < n_units; u0 += SLOTS * MAXR) {
        uint4 w[MAXR][CPL];
        uint32_t scr[MAXR][CPL], bir[MAXR][CPL]; // raw 16-bit scale / bias, converted where used
        uint32_t it[MAXR], rw[MAXR], eid[MAXR];
        bool live[MAXR];
#pragma unroll
        for (int m = 0; m < MAXR; ++m) {
            const uint32_t unit = u0 + slot_id + SLOTS * m;
            live[m] = unit < n_units;
            it[m] = unit / R;
            rw[m] = unit % R;
            eid[m] = id_src[min(it[m], routes - 1)]; // n_routed <= routes
        }
        res_v = residual[(uint64_t)(ri / R) * a.hidden + row_base + ri % R];
        cw_v = rweights[rq];
        coi_v = (use_plan ? a.plan.out_idx : ids)[rq];
        csl_v = shared_logit[tq];
        constexpr int NST = STG ? SF / 4 / 256 : 1;
        float4 stv[NST];
        uint32_t n4 = 0, n_st = 0;
        if (stage && u0 == 0) {
            n4 = (routes * I) / 4;
            n_st = n4 + (a.has_shared ? (T * I) / 4 : 0u);
        }
        if constexpr (STG) {
#pragma unroll
            for (int q = 0; q < NST; ++q) {
                // (passes that stage nothing read a.act[0])
                const uint32_t i = min(threadIdx.x + 256u * q, n_st > 0 ? n_st - 1 : 0u);
                // I % 32 == 0: the shared rows start on a chunk
                const float4* src = i < n4 || n_st == 0 ? reinterpret_cast<const float4*>(a.act) + i
                                                        : reinterpret_cast<const float4*>(act_shared) + (i - n4);
                stv[q] = *src;
            }
        }
#pragma unroll
        for (int m = 0; m < MAXR; ++m) {
            const bool shared = a.has_shared && it[m] == n_routed;
            if (!shared && eid[m] >= ex_count)
                live[m] = false;
            const bool ok = live[m];
            const uint8_t* slot = shared ? sh_base : ex_base + (uint64_t)(ok ? eid[m] : 0u) * ex_stride;
            const uint64_t w_off = shared ? sh_w : ex_w;
            const uint64_t s_off = shared ? sh_s : ex_s;
            const uint64_t b_off = shared ? sh_b : ex_b;
            const uint32_t gsh = shared ? gsh_s : gsh_e;
            const uint32_t row = row_base + rw[m];
            const uint8_t* dw = slot + w_off + (uint64_t)row * (I / 2);
            const uint16_t* sp = reinterpret_cast<const uint16_t*>(slot + s_off) + (uint64_t)row * (I >> gsh);
            const uint16_t* bp = reinterpret_cast<const uint16_t*>(slot + b_off) + (uint64_t)row * (I >> gsh);
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const uint32_t ch = gl + LPR * c;
                const uint32_t g = (ch * 32u) >> gsh;
                w[m][c] = *reinterpret_cast<const uint4*>(ok ? dw + ch * 16u : ex_base);
                scr[m][c] = *(ok ? sp + g : reinterpret_cast<const uint16_t*>(ex_base));
                bir[m][c] = *(ok ? bp + g : reinterpret_cast<const uint16_t*>(ex_base));
            }
        }
        if (stage && u0 == 0) {
            if constexpr (STG) {
#pragma unroll
                for (int q = 0; q < NST; ++q) {
                    // no branch: elements past n_st go to the never-read
                    // padding of the last chunk
                    const uint32_t i = threadIdx.x + 256u * q;
                    const uint32_t d = i < n_st ? (i >> 3) * XP + (i & 7) * 4 : (SF / 32 - 1) * XP + 32;
                    *reinterpret_cast<float4*>(&astage[d]) = stv[q];
                }
            }
            __syncthreads(); // staged activations visible
            const uint32_t n_chunks = (routes + (a.has_shared ? T : 0u)) * (I / 32);
            for (uint32_t q = threadIdx.x; q < n_chunks; q += 256) {
                const float4* c4 = reinterpret_cast<const float4*>(astage + q * XP);
                float sum = 0.0f;
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float4 f = c4[v];
                    sum += (f.x + f.y) + (f.z + f.w);
                }
                xsl[q] = sum;
            }
            __syncthreads();
        }
        float sc[MAXR][CPL], bi[MAXR][CPL];
#pragma unroll
        for (int m = 0; m < MAXR; ++m)
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                sc[m][c] = sb_bits<SBT>(scr[m][c]);
                bi[m][c] = sb_bits<SBT>(bir[m][c]);
            }
        if (ONE || (!STG && !use_plan)) {
            // one token, activations read from L2: every unit's loads in one
            // straight-line block (no token loop between them), so that they
            // are in flight together instead of one round trip per unit
            float part[MAXR];
#pragma unroll
            for (int m = 0; m < MAXR; ++m) {
                part[m] = 0.0f;
                const uint32_t unit = u0 + slot_id + SLOTS * m;
                if (unit < n_units && live[m]) {
                    const bool shared = a.has_shared && it[m] == n_routed;
                    const float* av = shared ? act_shared : a.act + (uint64_t)it[m] * I;
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const uint32_t ch = gl + LPR * c;
                        float xs;
                        const float qx = q4_chunk_qx(w[m][c], av + ch * 32, xs);
                        part[m] = fmaf(sc[m][c], qx, fmaf(bi[m][c], xs, part[m]));
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < MAXR; ++m) {
                const uint32_t unit = u0 + slot_id + SLOTS * m;
                if (unit >= n_units)
                    continue;
                const float y = group_sum<LPR>(part[m]);
                if (gl == 0) {
                    if (a.has_shared && it[m] == n_routed)
                        yshl[0][rw[m]] = y;
                    else
                        ylds[it[m]][rw[m]] = y;
                }
            }
            continue;
        }
        if constexpr (!ONE) {
#pragma unroll
        for (int m = 0; m < MAXR; ++m) {
            const uint32_t unit = u0 + slot_id + SLOTS * m;
            if (unit >= n_units)
                continue;
            const bool shared = a.has_shared && it[m] == n_routed;
            uint32_t g0 = 0, n = 0;
            if (shared) {
                n = T;
            } else if (use_plan) {
                g0 = a.plan.groups[2 * it[m]];
                n = a.plan.groups[2 * it[m] + 1];
            } else {
                g0 = it[m];
                n = 1;
            }
            for (uint32_t j = 0; j < n; ++j) {
                float part = 0.0f;
                if (live[m]) {
                    if (stage) {
                        const uint32_t rt = shared ? routes + j : g0 + j;
                        const float* av = astage + rt * (I / 32) * XP;
                        const float* xs = xsl + rt * (I / 32);
#pragma unroll
                        for (int c = 0; c < CPL; ++c) {
                            const uint32_t ch = gl + LPR * c;
                            const float qx = q4_chunk_q(w[m][c], av + ch * XP);
                            part = fmaf(sc[m][c], qx, fmaf(bi[m][c], xs[ch], part));
                        }
                    } else {
                        const float* av = shared ? act_shared + (uint64_t)j * I : a.act + (uint64_t)(g0 + j) * I;
#pragma unroll
                        for (int c = 0; c < CPL; ++c) {
                            const uint32_t ch = gl + LPR * c;
                            float xs;
                            const float qx = q4_chunk_qx(w[m][c], av + ch * 32, xs);
                            part = fmaf(sc[m][c], qx, fmaf(bi[m][c], xs, part));
                        }
                    }
                }
                const float y = group_sum<LPR>(part);
                if (gl == 0) {
                    if (shared)
                        yshl[j][rw[m]] = y;
                    else
                        ylds[g0 + j][rw[m]] = y;
                }
            }
        }
        }
        }
    if (stage && n_units == 0) {
        __syncthreads();
        __syncthreads();
    }
    if (threadIdx.x < routes) {
        c_w[threadIdx.x] = cw_v;
        c_oi[threadIdx.x] = use_plan ? coi_v : threadIdx.x;
    }
    if (threadIdx.x < T)
        c_sw[threadIdx.x] = a.has_shared ? sigmoidf_(csl_v) : 0.0f;
    __syncthreads();
    if (threadIdx.x < T * R) {
        const uint32_t t = threadIdx.x / R, r = threadIdx.x % R;
        float moe = 0.0f;
        for (uint32_t kk = 0; kk < K; ++kk) {
            const uint32_t route = t * K + kk;
            const uint32_t gi = c_oi[route];
            const float y = gi < NR ? ylds[gi][r] : 0.0f;
            moe = moe + c_w[route] * y;
        }
        const float rm = res_v + moe;
        const float sw = c_sw[t];
        const float sv = a.has_shared ? yshl[t][r] : 0.0f;
        hidden_out[(uint64_t)t * a.hidden + row_base + r] = rm + sw * sv;
    }
}

// ---------------------------------------------------------------------------
// kernel 3, several tokens (routes given, activations in route order):
// grid (workgroups per token, tokens).  A workgroup stages its token's K
// routed and shared activation rows in LDS once; each wave then computes
// whole output rows, strided over the token's workgroups.  Lane l takes
// the (item, 32-column chunk) slots l, l + 64, ... of a row and folds the
// item's combine weight (the route weight, or sigma of the shared gate
// logit) into its partial sum, so one wave reduction gives the row:
// h = r + sum over lanes of c_m (s q.x + b sum x).  The next row's weights
// load while this row is computed (buffers A and B, alternating: no
// register copies).
// ---------------------------------------------------------------------------
constexpr uint32_t ROWS_CHUNKS = PT_STAGE_FLOATS / 32; // staged chunks (<= 3 slots per lane)

template <int NCH>
struct RowWeights {
    uint4 w[NCH];
    uint32_t sr[NCH], br[NCH]; // raw 16-bit scale / bias
    float res;                 // residual of the row
};

template <int SBT, int NCH>
__global__ __launch_bounds__(256) void down_rows_kernel(DownArgs a)
{
    __shared__ __align__(16) float astage[ROWS_CHUNKS * XP];
    __shared__ float xsl[ROWS_CHUNKS]; // per-chunk sums of the staged activations
    __shared__ float cwl[MAX_K + 1];   // combine weight per item
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.y, K = a.k, H = a.hidden, I = a.ex.down.cols;
    const uint32_t cpi = I / 32; // chunks per item
    const uint32_t n_items = K + (a.has_shared ? 1u : 0u);
    const uint32_t n_ch = n_items * cpi;
    const uint32_t n4 = n_ch * 8, r4 = K * (I / 4); // staged float4, routed ones
    constexpr int NST = PT_STAGE_FLOATS / 4 / 256;
    // every load issued before any is used, none in a branch: activations,
    // combine inputs, the slots' expert ids
    float4 stv[NST];
#pragma unroll
    for (int q = 0; q < NST; ++q) {
        const uint32_t i = min(threadIdx.x + 256u * q, n4 - 1);
        stv[q] = i < r4 ? reinterpret_cast<const float4*>(a.act + (uint64_t)t * K * I)[i]
                        : reinterpret_cast<const float4*>(a.act_shared + (uint64_t)t * I)[i - r4];
    }
    const uint32_t mi = min((uint32_t)threadIdx.x, n_items - 1);
    const float rw = a.weights[t * K + min(mi, K - 1)];
    const float lg = (a.has_shared ? a.shared_logit : a.weights)[a.has_shared ? t : 0u];
    uint32_t eid[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const uint32_t m = min((uint32_t)(lane + 64 * j) / cpi, n_items - 1);
        eid[j] = a.ids[t * K + min(m, K - 1)];
    }
#pragma unroll
    for (int q = 0; q < NST; ++q) {
        // elements past n4 go to the never-read padding of the last chunk
        const uint32_t i = threadIdx.x + 256u * q;
        const uint32_t d = i < n4 ? (i >> 3) * XP + (i & 7) * 4 : (ROWS_CHUNKS - 1) * XP + 32;
        *reinterpret_cast<float4*>(&astage[d]) = stv[q];
    }
    if (threadIdx.x < n_items)
        cwl[threadIdx.x] = mi < K ? rw : sigmoidf_(lg);
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < n_ch; q += 256) {
        const float4* c4 = reinterpret_cast<const float4*>(astage + q * XP);
        float sum = 0.0f;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 f = c4[v];
            sum += (f.x + f.y) + (f.z + f.w);
        }
        xsl[q] = sum;
    }
    __syncthreads();

    // this lane's slots: item, chunk, expert base and offsets, combine weight
    // (0 for slots past the last chunk and for out-of-range routes, whose
    // weights are read from expert 0 and not used)
    // per slot: its chunk's code bytes in row 0 and its group's scale and
    // bias in row 0 (row r adds r * I / 2 bytes, r * gpr entries)
    const uint8_t* p_w[NCH];
    const uint16_t* p_s[NCH];
    const uint16_t* p_b[NCH];
    uint32_t s_gpr[NCH], s_q[NCH];
    float s_cw[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const uint32_t f = lane + 64 * j;
        const uint32_t m = min(f / cpi, n_items - 1);
        const bool sh = a.has_shared && m == K;
        const bool ok = f < n_ch && (sh || eid[j] < a.ex.count);
        const uint8_t* base = sh ? a.sh.base : a.ex.base + (uint64_t)(ok ? eid[j] : 0u) * a.ex.stride;
        const uint32_t gsh = sh ? a.sh.group_shift : a.ex.group_shift;
        const uint32_t ch = f < n_ch ? f % cpi : 0u;
        p_w[j] = base + (sh ? a.sh.down.w_off : a.ex.down.w_off) + ch * 16u;
        p_s[j] = reinterpret_cast<const uint16_t*>(base + (sh ? a.sh.down.s_off : a.ex.down.s_off)) + ((ch * 32u) >> gsh);
        p_b[j] = reinterpret_cast<const uint16_t*>(base + (sh ? a.sh.down.b_off : a.ex.down.b_off)) + ((ch * 32u) >> gsh);
        s_gpr[j] = I >> gsh;
        s_q[j] = f < n_ch ? f : 0u;
        s_cw[j] = ok ? cwl[m] : 0.0f;
    }
    const float* res_row = a.residual + (uint64_t)t * H;
    auto load_row = [&](uint32_t r, RowWeights<NCH>& W) {
        const uint32_t rc = min(r, H - 1);
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            W.w[j] = *reinterpret_cast<const uint4*>(p_w[j] + (uint64_t)rc * (I / 2));
            W.sr[j] = p_s[j][(uint64_t)rc * s_gpr[j]];
            W.br[j] = p_b[j][(uint64_t)rc * s_gpr[j]];
        }
        W.res = res_row[rc];
    };
    auto compute = [&](uint32_t r, RowWeights<NCH>& W) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            const float qx = q4_chunk_q(W.w[j], astage + s_q[j] * XP);
            acc = fmaf(s_cw[j], fmaf(sb_bits<SBT>(W.sr[j]), qx, sb_bits<SBT>(W.br[j]) * xsl[s_q[j]]), acc);
        }
        const float y = wave_sum(acc);
        if (lane == 0)
            a.hidden_out[(uint64_t)t * H + r] = W.res + y;
    };
    RowWeights<NCH> A, B;
    const uint32_t step = gridDim.x * 4;
    uint32_t r = down_row_block(blockIdx.x, gridDim.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    load_row(r, A);
    while (r < H) {
        load_row(r + step, B);
        compute(r, A);
        r += step;
        if (r >= H)
            break;
        load_row(r + step, A);
        compute(r, B);
        r += step;
    }
}

// ---------------------------------------------------------------------------
// kernel 3, wide variant: tokens whose routed + shared activations are
// too large for the staging buffer of down_combine_kernel (C5: 9 items x
// 2048 columns), one token per grid row (blockIdx.y), activations in route
// order.  WIDE_R = 16 output rows per workgroup, so that one staged
// copy of the activations (72 KB, two workgroups per CU) serves 16 rows of
// every item and the grid (H / 16 workgroups) is one round of residency.
// Wave w owns rows 4w .. 4w + 3 of the block; lane l owns 32-column chunk l
// (I <= 2048), reads that chunk of an item's activations from LDS once and
// applies it to its rows.  Each lane folds the combine weight of the
// item into its partial sums, so a row needs one wave reduction in all:
// h = r + sum over lanes of sum_m c_m (s q.x + b sum x), c_m = w_m for a
// routed item, sigma(shared logit) for the shared one.  Float4 j of staged
// chunk q sits at q * 32 + 4 (j ^ ((q >> 1) & 7)): 16 consecutive chunks
// fall on distinct banks.
// ---------------------------------------------------------------------------
constexpr int WIDE_R = 16;
constexpr int WIDE_THREADS = 256;
constexpr uint32_t WIDE_FLOATS = 18432;
__device__ __forceinline__ uint32_t wide_f4(uint32_t q, uint32_t j) { return q * 32u + 4u * (j ^ ((q >> 1) & 7u)); }

template <int SBT>
__global__ __launch_bounds__(WIDE_THREADS, 2) void down_wide_kernel(DownArgs a)
{
    constexpr int RW = WIDE_R / (WIDE_THREADS / 64); // rows per wave
    constexpr int MAXI = 3;                          // items per pass
    constexpr int NST = WIDE_FLOATS / 4 / WIDE_THREADS; // staged float4 per thread
    __shared__ __align__(16) float xst[WIDE_FLOATS];
    __shared__ float xsum[WIDE_FLOATS / 32];
    __shared__ float c_m[MAX_K + 1];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6); // uniform: row addresses stay scalar
    const uint32_t K = a.k, I = a.ex.down.cols, chunks = I / 32;
    const uint32_t n_items = K + (a.has_shared ? 1u : 0u);
    const uint32_t row0 = blockIdx.x * WIDE_R + wv * RW;
    // token blockIdx.y (grid H / WIDE_R x tokens; activations in route order)
    const uint32_t t = blockIdx.y, H = a.hidden;
    const uint32_t* const ids = a.ids + t * K;
    const float* const rweights = a.weights + t * K;
    const float* const act = a.act + (uint64_t)t * K * I;
    const float* const act_sh = a.act_shared + (uint64_t)t * I;
    const uint32_t ch = min(lane, chunks - 1); // lanes past the row read its last chunk, unused
    const bool lane_on = lane < chunks;
    // loads that need nothing: the routes' expert ids (uniform), the
    // combine weights, the residual, then every staged activation
    uint32_t eid[MAX_K];
#pragma unroll
    for (int m = 0; m < MAX_K; ++m)
        eid[m] = ids[min((uint32_t)m, K - 1)];
    const float cw_v = rweights[min(tid, K - 1)];
    const float csl_v = (a.has_shared ? a.shared_logit + t : rweights)[0];
    const float res_v = a.residual[(uint64_t)t * H + row0 + min(lane, (uint32_t)RW - 1)];
    const uint32_t n4 = K * I / 4, n_st = n_items * I / 4;
    float4 stv[NST];
#pragma unroll
    for (int q = 0; q < NST; ++q) {
        const uint32_t i = min(tid + (uint32_t)WIDE_THREADS * q, n_st - 1);
        stv[q] = i < n4 ? reinterpret_cast<const float4*>(act)[i] : reinterpret_cast<const float4*>(act_sh)[i - n4];
    }
    const uint8_t* const ex_base = a.ex.base;
    const uint64_t ex_stride = a.ex.stride;
    const uint64_t ex_w = a.ex.down.w_off, ex_s = a.ex.down.s_off, ex_b = a.ex.down.b_off;
    const uint8_t* const sh_base = a.has_shared ? a.sh.base : ex_base;
    const uint64_t sh_w = a.sh.down.w_off, sh_s = a.sh.down.s_off, sh_b = a.sh.down.b_off;
    const uint32_t gsh_e = a.ex.group_shift, gsh_s = a.has_shared ? a.sh.group_shift : gsh_e;
    // codes and raw scale/bias of this lane's chunk, four rows, the items of
    // pass p (3p + j): every address is a uniform base plus the lane's
    // chunk offset; items past the last (also whole passes) and experts out
    // of range read the same rows of slot 0 and are not used
    struct PassRegs {
        uint4 w[MAXI][RW];
        uint32_t scr[MAXI][RW], bir[MAXI][RW];
        bool live[MAXI];
    };
    auto load_pass = [&](PassRegs& r, uint32_t p) {
#pragma unroll
        for (int j = 0; j < MAXI; ++j) {
            const uint32_t m = (uint32_t)MAXI * p + j;
            const bool shared = a.has_shared && m == K;
            uint32_t e = 0;
#pragma unroll
            for (int q = 0; q < MAX_K; ++q)
                e = (uint32_t)q == m ? eid[q] : e;
            r.live[j] = m < n_items && (shared || e < a.ex.count);
            const bool use_sh = shared && m < n_items;
            const uint8_t* slot_p = use_sh ? sh_base : ex_base + (uint64_t)(r.live[j] ? e : 0u) * ex_stride;
            const uint64_t w_off = use_sh ? sh_w : ex_w, s_off = use_sh ? sh_s : ex_s, b_off = use_sh ? sh_b : ex_b;
            const uint32_t gsh = use_sh ? gsh_s : gsh_e;
            // unused items read the first row of slot 0 for every row, the
            // same lines in every workgroup (cache hits, not HBM traffic)
            const uint32_t gpr = r.live[j] ? I >> gsh : 0u, g = (ch * 32u) >> gsh;
            const uint32_t wstride = r.live[j] ? I / 2 : 0u, rb = r.live[j] ? row0 : 0u;
            const uint8_t* wrow = slot_p + w_off + (uint64_t)rb * wstride;
            const uint16_t* srow = reinterpret_cast<const uint16_t*>(slot_p + s_off) + (uint64_t)rb * gpr;
            const uint16_t* brow = reinterpret_cast<const uint16_t*>(slot_p + b_off) + (uint64_t)rb * gpr;
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                r.w[j][rr] = *reinterpret_cast<const uint4*>(wrow + (uint64_t)rr * wstride + ch * 16u);
                r.scr[j][rr] = srow[rr * gpr + g];
                r.bir[j][rr] = brow[rr * gpr + g];
            }
        }
    };
    float part[RW];
#pragma unroll
    for (int rr = 0; rr < RW; ++rr)
        part[rr] = 0.0f;
    auto compute_pass = [&](PassRegs& r, uint32_t p) {
#pragma unroll
        for (int j = 0; j < MAXI; ++j) {
            const uint32_t m = (uint32_t)MAXI * p + j;
            // this lane's chunk of item m (passes past the last read item 0)
            const uint32_t q = (m < n_items ? m : 0u) * chunks + ch;
            float xv[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(&xst[wide_f4(q, i)]);
                xv[4 * i] = v.x, xv[4 * i + 1] = v.y, xv[4 * i + 2] = v.z, xv[4 * i + 3] = v.w;
            }
            const float xs = xsum[q];
            const float cm = r.live[j] && lane_on ? c_m[m < n_items ? m : 0u] : 0.0f;
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                // the nibble conversions of one row at a time (scheduled
                // together, those of a pass would need 384 registers)
                asm volatile("" : "+v"(r.w[j][rr].x), "+v"(r.w[j][rr].y), "+v"(r.w[j][rr].z), "+v"(r.w[j][rr].w));
                const float qx = q4_chunk_qx_reg(r.w[j][rr], xv);
                const float y = fmaf(sb_bits<SBT>(r.scr[j][rr]), qx, sb_bits<SBT>(r.bir[j][rr]) * xs);
                part[rr] = fmaf(cm, y, part[rr]);
            }
        }
    };
    PassRegs ra;
    load_pass(ra, 0);
    // stage: elements past n_st go to the last float4 of the buffer, which
    // no read touches unless the buffer is full (then there are none)
#pragma unroll
    for (int q = 0; q < NST; ++q) {
        const uint32_t i = tid + (uint32_t)WIDE_THREADS * q;
        const uint32_t d = i < n_st ? wide_f4(i >> 3, i & 7u) : WIDE_FLOATS - 4;
        *reinterpret_cast<float4*>(&xst[d]) = stv[q];
        // chunk sums: the 8 float4 of chunk i >> 3 sit on 8 consecutive lanes
        float s4 = (stv[q].x + stv[q].y) + (stv[q].z + stv[q].w);
        s4 += __shfl_xor(s4, 1);
        s4 += __shfl_xor(s4, 2);
        s4 += __shfl_xor(s4, 4);
        if ((i & 7u) == 0 && i < n_st)
            xsum[i >> 3] = s4;
    }
    if (tid < K)
        c_m[tid] = cw_v;
    if (tid == K)
        c_m[K] = a.has_shared ? sigmoidf_(csl_v) : 0.0f;
    __syncthreads();
    // passes in turn: a second register set for the next pass's loads
    // (two items per pass to fit) measured slower, 22.6 against 19.9 us on
    // C5; the lanes' VALU work, not the load latency, bounds the passes
    const uint32_t npass = (n_items + MAXI - 1) / MAXI;
    for (uint32_t p = 0; p < npass; ++p) {
        if (p > 0)
            load_pass(ra, p);
        compute_pass(ra, p);
    }
    // one reduction per row; lane rr writes row rr
    float out = 0.0f;
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
        const float t = wave_sum(part[rr]);
        out = lane == (uint32_t)rr ? t : out;
    }
    if (lane < (uint32_t)RW)
        a.hidden_out[(uint64_t)t * H + row0 + lane] = res_v + out;
}

// next-layer RMSNorm: one block per token (rms_norm_reduced)
__global__ __launch_bounds__(256) void next_norm_kernel(const float* __restrict__ h,
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
    const float ms = ((part[0] + part[1]) + (part[2] + part[3])) / (float)(width > 1 ? width : 1);
    const float scale = 1.0f / sqrtf(ms + eps);
    for (uint32_t i = threadIdx.x; i < width; i += 256)
        out[(uint64_t)blockIdx.x * width + i] = (row[i] * scale) * w[i];
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
// start/stop events of kernel phase i/2 when the caller asked for phase
// timing: attached to the dispatch packet itself, so they bracket exactly
// the kernel's execution
static inline hipEvent_t phase_event(const DecodeArgs& d, int i)
{
    return d.phase_timing ? d.phase_ev[i] : nullptr;
}

static hipError_t launch_router_stage(hipStream_t st, const DecodeArgs& d, bool do_router,
                                      bool do_shared, bool shared_rows_here = true)
{
    RouterArgs a{};
    a.router_w = d.router_w;
    a.experts = do_router ? d.rp.experts : 0u;
    if (do_shared && d.shared)
        a.sh = *d.shared;
    a.shared_rows = do_shared && d.shared && shared_rows_here ? d.shared->gate.rows : 0u;
    a.gate_task = do_shared && d.shared ? 1u : 0u;
    a.sgate_w = do_shared ? d.sgate_w : nullptr;
    a.sgate_dtype = d.sgate_dtype;
    a.router_q4 = d.router_q4;
    a.sgate_q4 = d.sgate_q4;
    a.x = d.x;
    a.norm_w = d.in_norm_w;
    a.eps = d.eps;
    a.x_out = d.x_normed;
    a.tokens = d.tokens;
    a.hidden = d.hidden;
    a.logits = d.logits;
    a.act_shared = d.act_shared;
    a.shared_weight = d.shared_weight;
    const uint32_t tasks = a.experts + a.shared_rows + a.gate_task;
    if (tasks == 0) {
        if (d.phase_timing) {
            hipError_t e = hipEventRecord(d.phase_ev[0], st);
            if (e == hipSuccess)
                e = hipEventRecord(d.phase_ev[1], st);
            return e;
        }
        return hipSuccess;
    }
    // with the fused norm, one more workgroup (past every task) writes the
    // normalised rows
    const uint32_t blocks = (tasks + 3) / 4 + (a.norm_w ? 1u : 0u);
    const uint32_t cr = (d.hidden + 511) / 512;
    const uint32_t cs = (d.hidden / 32 + 63) / 64;
    if (cr > 16 || cs > 4)
        return hipErrorInvalidValue;
    // four tokens or more, or rows past 4096 columns: x staged in LDS per
    // group of tokens (with two tokens of C2 the staging round trip before
    // the weight loads costs more than it saves: 6.2 -> 7.0 us; C5's
    // 7168-column rows, whose every task would read 28 KB of x from L2,
    // gain at any token count)
    const bool xl = (d.tokens >= 4 || d.hidden > 4096) && d.hidden <= XL_MAX_H && d.hidden >= 256 &&
                    d.hidden % 4 == 0;
    const uint32_t xl_groups = xl ? (d.tokens + XL_FLOATS / d.hidden - 1) / (XL_FLOATS / d.hidden) : 1u;
    // router/gate dtypes: the benchmark layers use f16 for both; other
    // combinations share the f16 gate path only when the gate is f16
    const uint32_t gdt = a.sgate_w ? d.sgate_dtype : d.router_dtype;
    const uint32_t wdt = a.experts ? d.router_dtype : gdt;
    const uint32_t sbt = a.gate_task ? a.sh.sb_dtype : 1u;
#define PBM_RS(W, G, S, CRV, CSV)                                                              \
    do {                                                                                       \
        if (xl)                                                                                \
            hipExtLaunchKernelGGL((router_stage_kernel<W, G, S, CRV, CSV, true>), dim3(blocks, xl_groups), \
                                  dim3(256), xl_lds_bytes(d.hidden, a.norm_w != nullptr), st,  \
                                  phase_event(d, 0), phase_event(d, 1), 0, a);                 \
        else                                                                                   \
            hipExtLaunchKernelGGL((router_stage_kernel<W, G, S, CRV, CSV, false>), dim3(blocks), dim3(256), 0, \
                                  st, phase_event(d, 0), phase_event(d, 1), 0, a);             \
    } while (0)
#define PBM_RS_CS(W, G, S, CRV)                                                                \
    do {                                                                                       \
        if (cs <= 1) PBM_RS(W, G, S, CRV, 1);                                                  \
        else if (cs <= 2) PBM_RS(W, G, S, CRV, 2);                                             \
        else PBM_RS(W, G, S, CRV, 4);                                                          \
    } while (0)
#define PBM_RS_CR(W, G, S)                                                                     \
    do {                                                                                       \
        if (cr <= 4) PBM_RS_CS(W, G, S, 4);                                                    \
        else PBM_RS_CS(W, G, S, 8); /* longer rows in passes of 8 chunks */                    \
    } while (0)
    if (wdt != gdt)
        return hipErrorInvalidValue; // bind validates matching dtypes
    // a Q4 router or gate row carries the layer's scale/bias dtype
    const uint32_t qsb = wdt == DT_Q4 ? d.ex.sb_dtype : sbt;
    if (wdt == DT_Q4 && a.gate_task && sbt != qsb)
        return hipErrorInvalidValue;
    if (wdt == DT_Q4) {
        if (qsb == 2) PBM_RS_CS(DT_Q4, DT_Q4, 2, 4);
        else PBM_RS_CS(DT_Q4, DT_Q4, 1, 4);
    } else if (sbt == 2) {
        if (wdt == 0) PBM_RS_CR(0, 0, 2);
        else if (wdt == 2) PBM_RS_CR(2, 2, 2);
        else PBM_RS_CR(1, 1, 2);
    } else {
        if (wdt == 0) PBM_RS_CR(0, 0, 1);
        else if (wdt == 2) PBM_RS_CR(2, 2, 1);
        else PBM_RS_CR(1, 1, 1);
    }
#undef PBM_RS
#undef PBM_RS_CS
#undef PBM_RS_CR
    return hipGetLastError();
}

// Rows per wave of the gate/up kernel and its workgroups (without the
// down-prefetch ones): two rows per wave; four where two would need several
// rounds of resident workgroups (large I and H: fewer workgroups, so the
// routing each of them repeats is done fewer times).
static uint32_t gateup_rpw(const DecodeArgs& d, uint32_t* wgs)
{
    const uint32_t T = d.tokens, K = d.rp.k, I = d.ex.gate.rows;
    const uint32_t max_items = T > 1 ? std::min(d.ex.count, T * K) : T * K;
    const uint32_t rpw = (max_items * (I / 2) + 3) / 4 > 2 * GATEUP_RESIDENT_WGS && I % 4 == 0 ? 4 : 2;
    if (wgs)
        *wgs = (max_items * (I / rpw) + 3) / 4;
    return rpw;
}

// Route in a launch of its own (route_topk) when the gate/up grid does not
// fit one round of residency: every gate/up workgroup would repeat the
// routing, once per round.  C5 (1024 workgroups, two rounds): 98.0 ->
// 89.5 us per layer; C2 (640 workgroups, one round): the extra launch
// costs more than the routing it saves (23.7 -> 25.9 us).
// Several tokens whose per-token activations fit down_rows_kernel: the
// persistent gate/up kernel over routes (each workgroup routing its token)
// and the row kernel for down + combine (no dispatch plan).
static bool multi_token_path(const DecodeArgs& d)
{
    const uint32_t T = d.tokens, K = d.rp.k, H = d.hidden, I = d.ex.gate.rows;
    return T > 1 && (uint64_t)(K + (d.shared ? 1u : 0u)) * I <= PT_STAGE_FLOATS && I <= 1536 && I % 4 == 0 &&
           H % 4 == 0 && H <= 64 * 32 * 4;
}

static bool route_separately(const DecodeArgs& d)
{
    if (multi_token_path(d))
        return false; // gateup_multi_kernel routes
    uint32_t wgs = 0;
    gateup_rpw(d, &wgs);
    return wgs > GATEUP_RESIDENT_WGS;
}

// resident workgroups of gateup_multi_kernel per CU, by its registers:
// one chunk per lane (95 VGPRs) 5 waves per SIMD, two or four (140-146) 3
static uint32_t multi_wgs_per_cu(uint32_t cpl) { return cpl <= 1 ? 5u : 3u; }
// workgroups of down_rows_kernel per CU (its registers allow two; more only
// wait)
constexpr uint32_t ROWS_WGS_PER_CU = 2;
// one token whose routed + shared activations (items x I floats) fit the
// row kernel's staging: the down kernel is down_rows_kernel, on this grid
static bool one_token_rows(uint32_t tokens, uint32_t items, uint32_t I)
{
    return tokens == 1 && (uint64_t)items * I <= PT_STAGE_FLOATS && I <= 1536;
}
static uint32_t rows_grid_one_token(uint32_t H) { return std::min(H / 4, 256u * ROWS_WGS_PER_CU); }

// gateup_multi_kernel with the routes in d.ids: two rows per unit (one with
// four chunks per lane, for the registers) and about the resident number of
// workgroups, shared by the tokens (more workgroups than that only wait)
template <int SBT>
static hipError_t launch_gateup_multi(hipStream_t st, const DecodeArgs& d, bool route_here)
{
    const uint32_t T = d.tokens, K = d.rp.k, H = d.hidden, I = d.ex.gate.rows;
    ExpertArgs ea{};
    ea.ex = d.ex;
    ea.rp = d.rp;
    ea.logits = d.logits;
    ea.sel_bias = d.sel_bias;
    ea.route_here = route_here;
    ea.ids = d.ids;
    ea.weights = d.weights;
    ea.x = d.in_norm_w ? d.x_normed : d.x; // normalised by the router stage
    ea.tokens = T;
    ea.hidden = H;
    ea.act = d.act;
    ea.status = d.status;
    const uint32_t cpl = (H / 32 + 63) / 64;
    const uint32_t rpw = cpl <= 2 ? 2u : 1u;
    const uint32_t wgs_cu = multi_wgs_per_cu(cpl);
    const uint32_t units = K * (I / rpw); // per token
    const uint32_t per_token = std::max(1u, std::min((units + 3) / 4, 256u * wgs_cu / T));
    const dim3 g1(per_token, T);
    const uint32_t epl = (d.rp.experts + 63) / 64;
#define PBM_GM(C, R)                                                                           \
    do {                                                                                       \
        if (epl <= 2)                                                                          \
            hipExtLaunchKernelGGL((gateup_multi_kernel<SBT, C, R, 2>), g1, dim3(256), 0, st,   \
                                  phase_event(d, 2), phase_event(d, 3), 0, ea);                \
        else if (epl <= 4)                                                                     \
            hipExtLaunchKernelGGL((gateup_multi_kernel<SBT, C, R, 4>), g1, dim3(256), 0, st,   \
                                  phase_event(d, 2), phase_event(d, 3), 0, ea);                \
        else if (epl <= 8)                                                                     \
            hipExtLaunchKernelGGL((gateup_multi_kernel<SBT, C, R, 8>), g1, dim3(256), 0, st,   \
                                  phase_event(d, 2), phase_event(d, 3), 0, ea);                \
        else                                                                                   \
            hipExtLaunchKernelGGL((gateup_multi_kernel<SBT, C, R, 16>), g1, dim3(256), 0, st,  \
                                  phase_event(d, 2), phase_event(d, 3), 0, ea);                \
    } while (0)
    if (cpl <= 1)
        PBM_GM(1, 2);
    else if (cpl <= 2)
        PBM_GM(2, 2);
    else if (cpl <= 4)
        PBM_GM(4, 1);
    else
        return hipErrorInvalidValue;
#undef PBM_GM
    return hipGetLastError();
}

template <int SBT>
static hipError_t launch_multi_token(hipStream_t st, const DecodeArgs& d, bool route_here)
{
    const uint32_t T = d.tokens, K = d.rp.k, H = d.hidden, I = d.ex.gate.rows;
    hipError_t err = launch_gateup_multi<SBT>(st, d, route_here);
    if (err != hipSuccess)
        return err;
    DownArgs da{};
    da.ex = d.ex;
    da.has_shared = d.shared != nullptr;
    if (da.has_shared)
        da.sh = *d.shared;
    da.act = d.act;
    da.act_shared = d.act_shared;
    da.shared_logit = d.shared_weight;
    da.tokens = T;
    da.k = K;
    da.hidden = H;
    da.ids = d.ids; // activations in route order
    da.weights = d.weights;
    da.residual = d.residual;
    da.hidden_out = d.hidden_out;
    da.status = d.status;
    // rows: workgroups per token, ROWS_WGS_PER_CU per CU in all
    const uint32_t nch = ((K + (da.has_shared ? 1u : 0u)) * (I / 32) + 63) / 64;
    const dim3 gr(std::max(1u, std::min(H / 4, 256u * ROWS_WGS_PER_CU / T)), T);
    if (nch <= 1)
        hipExtLaunchKernelGGL((down_rows_kernel<SBT, 1>), gr, dim3(256), 0, st, phase_event(d, 4), phase_event(d, 5),
                              0, da);
    else if (nch <= 2)
        hipExtLaunchKernelGGL((down_rows_kernel<SBT, 2>), gr, dim3(256), 0, st, phase_event(d, 4), phase_event(d, 5),
                              0, da);
    else
        hipExtLaunchKernelGGL((down_rows_kernel<SBT, 3>), gr, dim3(256), 0, st, phase_event(d, 4), phase_event(d, 5),
                              0, da);
    err = hipGetLastError();
    if (err != hipSuccess)
        return err;
    if (d.next_norm_w && d.next_normed) {
        next_norm_kernel<<<T, 256, 0, st>>>(d.hidden_out, d.next_norm_w, H, d.eps, d.next_normed);
        err = hipGetLastError();
    }
    return err;
}

// Launch shape of route_gateup_kernel outside the several-token path: its
// gate/up workgroups (pf_base, a multiple of 8) and the down-weight prefetch
// workgroups appended after them.  Down-weight prefetch by extra workgroups
// while gate/up runs, when the down bytes of the selected experts fit
// comfortably in the L2s (8 x 4 MB): about two touched lines per prefetch
// lane, at most 16 workgroups per XCD (more than that no longer fit beside
// the gate/up workgroups).  Measured on C2 batch 1: down kernel 10.5 -> 9.2
// us, gate/up +0.4 us.  Returns false when the gate/up phase runs another
// kernel (the persistent one).
static bool gateup_prefetch(const DecodeArgs& d, bool route_here, uint32_t& pf_base, uint32_t& pf_wgs)
{
    const ExpertSet& ex = d.ex;
    const uint32_t T = d.tokens, K = d.rp.k, H = d.hidden, I = ex.gate.rows;
    const bool use_plan = T > 1;
    const bool wide_shape = (uint64_t)(K + (d.shared ? 1u : 0u)) * I > STAGE_FLOATS &&
                            (uint64_t)(K + (d.shared ? 1u : 0u)) * I <= WIDE_FLOATS && I % 512 == 0 &&
                            I >= 1024 && I <= 2048 && H % WIDE_R == 0;
    const uint32_t max_items = use_plan ? std::min(ex.count, T * K) : T * K;
    const uint32_t RPW = gateup_rpw(d, nullptr);
    const uint32_t waves = max_items * (I / RPW);
    pf_base = ((waves + 3) / 4 + 7) / 8 * 8;
    pf_wgs = 0;
    const bool multi_gu = wide_shape && H <= 64 * 32 * 4 && (T > 1 || !route_here);
    const bool wide = wide_shape && (T == 1 || multi_gu); // the wide down kernel takes no prefetch
    const uint32_t items = max_items + (d.shared ? 1u : 0u);
    const uint32_t gpr_d = I >> ex.group_shift;
    const uint64_t down_bytes = (uint64_t)items * H * (I / 2 + 4u * gpr_d);
    if (!wide && down_bytes <= (16u << 20) && pf_base < GATEUP_RESIDENT_WGS) {
        const uint32_t per_block = (DOWN_R * I / 2 + 127) / 128 + 2 * ((DOWN_R * gpr_d * 2 + 127) / 128);
        const uint64_t lines_xcd = (uint64_t)items * ((H / DOWN_R + 7) / 8) * per_block;
        const uint64_t per_xcd = (lines_xcd + 2 * 256 - 1) / (2 * 256);
        pf_wgs = 8u * (uint32_t)std::min<uint64_t>(per_xcd, 16);
        pf_wgs = std::min(pf_wgs, (GATEUP_RESIDENT_WGS - pf_base) / 8 * 8);
    }
    return !multi_gu;
}

// One token through route_gateup_kernel with down-prefetch workgroups and a
// shared expert of the routed experts' scale/bias type: the prefetch
// workgroups compute the shared gate/up rows (no routes needed) instead of
// the router stage, whose launch their weight loads held back (C2: the
// shared rows' workgroups ended 1.3 us after the router rows').
static bool shared_rows_in_gateup(const DecodeArgs& d, bool route_here)
{
    if (!d.shared || d.tokens != 1 || multi_token_path(d) || d.shared->sb_dtype != d.ex.sb_dtype ||
        d.shared->gate.cols != d.hidden || d.shared->up.cols != d.hidden)
        return false;
    const uint32_t K = d.rp.k, I = d.ex.gate.rows, H = d.hidden;
    const bool wide_shape = (uint64_t)(K + 1u) * I > STAGE_FLOATS && (uint64_t)(K + 1u) * I <= WIDE_FLOATS &&
                            I % 512 == 0 && I >= 1024 && I <= 2048 && H % WIDE_R == 0;
    if (wide_shape)
        return false;
    // room in the single round of resident workgroups for one shared row
    // per prefetch wave (with two rows a wave became the launch's tail)
    uint32_t pf_base, pf_wgs;
    return gateup_prefetch(d, route_here, pf_base, pf_wgs) && pf_wgs >= 8 && (H / 32 + 63) / 64 <= 4 &&
           pf_base < GATEUP_RESIDENT_WGS && (GATEUP_RESIDENT_WGS - pf_base) / 8 * 8 * 4 >= d.shared->gate.rows;
}

template <int SBT>
static hipError_t launch_experts_typed(hipStream_t st, const DecodeArgs& d, bool route_here)
{
    if (multi_token_path(d))
        return launch_multi_token<SBT>(st, d, route_here);
    const ExpertSet& ex = d.ex;
    const uint32_t T = d.tokens, K = d.rp.k, H = d.hidden, I = ex.gate.rows;
    const bool use_plan = T > 1;
    // Activations of a token too large for the down kernel's staging buffer
    // but within the wide kernel's (C5: 9 x 2048 floats): the wide down
    // kernel, one token per grid row.  Its gate/up runs in the persistent
    // kernel (activations in route order; C5 one token 44.7 -> 35.0 us)
    // unless one token is routed inside route_gateup_kernel.
    const bool wide_shape = (uint64_t)(K + (d.shared ? 1u : 0u)) * I > STAGE_FLOATS &&
                            (uint64_t)(K + (d.shared ? 1u : 0u)) * I <= WIDE_FLOATS && I % 512 == 0 &&
                            I >= 1024 && I <= 2048 && H % WIDE_R == 0;
    const bool multi_gu = wide_shape && H <= 64 * 32 * 4 && (T > 1 || !route_here);
    const bool wide = wide_shape && (T == 1 || multi_gu);
    ExpertArgs ea{};
    ea.ex = ex;
    ea.logits = d.logits;
    ea.sel_bias = d.sel_bias;
    ea.rp = d.rp;
    ea.route_here = route_here;
    ea.ids = d.ids;
    ea.weights = d.weights;
    ea.plan = d.plan;
    ea.x = d.in_norm_w ? d.x_normed : d.x; // normalised by the router stage
    ea.tokens = T;
    ea.hidden = H;
    ea.act = d.act;
    ea.status = d.status;
    ea.has_shared = d.shared != nullptr;
    if (ea.has_shared)
        ea.sh = *d.shared;
    const int RPW = (int)gateup_rpw(d, nullptr);
    const uint32_t cpl = (H / 32 + 63) / 64;
    const uint32_t epl = (d.rp.experts + 63) / 64;
    gateup_prefetch(d, route_here, ea.pf_base, ea.pf_wgs);
    ea.pf_paired = one_token_rows(T, K + (d.shared ? 1u : 0u), I) && rows_grid_one_token(H) % 16 == 0;
    if (shared_rows_in_gateup(d, route_here)) {
        ea.shared_rows = d.shared->gate.rows;
        ea.act_shared = d.act_shared;
        // one shared row per prefetch wave where the single round of
        // resident workgroups allows (a wave with two paid two round trips
        // before routing and became the launch's tail)
        const uint32_t want = (ea.shared_rows + 31) / 32 * 8;
        ea.pf_wgs = std::max(ea.pf_wgs, std::min(want, (GATEUP_RESIDENT_WGS - ea.pf_base) / 8 * 8));
    }
    dim3 g1(ea.pf_base + ea.pf_wgs);
#define PBM_GU(C, EP)                                                                          \
    do {                                                                                       \
        if (RPW == 4)                                                                          \
            hipExtLaunchKernelGGL((route_gateup_kernel<SBT, C, 4, EP>), g1, dim3(256), 0, st,  \
                                  phase_event(d, 2), phase_event(d, 3), 0, ea);                \
        else                                                                                   \
            hipExtLaunchKernelGGL((route_gateup_kernel<SBT, C, 2, EP>), g1, dim3(256), 0, st,  \
                                  phase_event(d, 2), phase_event(d, 3), 0, ea);                \
    } while (0)
#define PBM_GU_E(C)                                                                            \
    do {                                                                                       \
        if (epl <= 2) PBM_GU(C, 2);                                                            \
        else if (epl <= 4) PBM_GU(C, 4);                                                       \
        else if (epl <= 8) PBM_GU(C, 8);                                                       \
        else PBM_GU(C, 16);                                                                    \
    } while (0)
    hipError_t err;
    if (multi_gu) {
        err = launch_gateup_multi<SBT>(st, d, route_here);
    } else {
        if (cpl <= 1) PBM_GU_E(1);
        else if (cpl <= 2) PBM_GU_E(2);
        else if (cpl <= 4) PBM_GU_E(4);
        else return hipErrorInvalidValue;
        err = hipGetLastError();
    }
#undef PBM_GU
#undef PBM_GU_E
    if (err != hipSuccess)
        return err;

    DownArgs da{};
    da.ex = ex;
    da.has_shared = d.shared != nullptr;
    if (da.has_shared)
        da.sh = *d.shared;
    da.act = d.act;
    da.act_shared = d.act_shared;
    da.shared_logit = d.shared_weight;
    da.tokens = T;
    da.k = K;
    da.hidden = H;
    da.ids = d.ids;
    da.weights = d.weights;
    da.plan = d.plan;
    da.use_plan = use_plan;
    // every route's activations (plan order for several tokens) and the
    // shared expert's, when they fit the staging buffer
    da.stage = (uint64_t)(T * K + (da.has_shared ? T : 0u)) * I <= STAGE_FLOATS;
    da.residual = d.residual;
    da.hidden_out = d.hidden_out;
    da.status = d.status;
    if (wide) {
        dim3 gw(H / WIDE_R, T);
#define PBM_DW()                                                                               \
    hipExtLaunchKernelGGL((down_wide_kernel<SBT>), gw, dim3(WIDE_THREADS), 0, st, phase_event(d, 4), phase_event(d, 5), 0, da)
        PBM_DW();
#undef PBM_DW
        err = hipGetLastError();
        if (err != hipSuccess)
            return err;
        if (d.next_norm_w && d.next_normed) {
            next_norm_kernel<<<T, 256, 0, st>>>(d.hidden_out, d.next_norm_w, H, d.eps, d.next_normed);
            err = hipGetLastError();
        }
        return err;
    }
    // one token whose routed + shared activations fit: the row kernel (no
    // LDS combine and barrier; C2 down 7.8 -> 6.0 us per layer)
    if (one_token_rows(T, K + (da.has_shared ? 1u : 0u), I)) {
        const uint32_t nch = ((K + (da.has_shared ? 1u : 0u)) * (I / 32) + 63) / 64;
        const dim3 gr(rows_grid_one_token(H), 1);
        if (nch <= 1)
            hipExtLaunchKernelGGL((down_rows_kernel<SBT, 1>), gr, dim3(256), 0, st, phase_event(d, 4),
                                  phase_event(d, 5), 0, da);
        else if (nch <= 2)
            hipExtLaunchKernelGGL((down_rows_kernel<SBT, 2>), gr, dim3(256), 0, st, phase_event(d, 4),
                                  phase_event(d, 5), 0, da);
        else
            hipExtLaunchKernelGGL((down_rows_kernel<SBT, 3>), gr, dim3(256), 0, st, phase_event(d, 4),
                                  phase_event(d, 5), 0, da);
        err = hipGetLastError();
        if (err != hipSuccess)
            return err;
        if (d.next_norm_w && d.next_normed) {
            next_norm_kernel<<<T, 256, 0, st>>>(d.hidden_out, d.next_norm_w, H, d.eps, d.next_normed);
            err = hipGetLastError();
        }
        return err;
    }
    dim3 g2(H / DOWN_R);
#define PBM_DN(L, C, M, S)                                                                     \
    hipExtLaunchKernelGGL((down_combine_kernel<SBT, L, C, M, S>), g2, dim3(256), 0, st, phase_event(d, 4), \
                          phase_event(d, 5), 0, da)
    switch (I) {
    case 256: PBM_DN(8, 1, 4, true); break;
    case 512: PBM_DN(8, 2, 4, true); break;
    case 768: PBM_DN(8, 3, 4, true); break;
    case 1024: PBM_DN(16, 2, 4, true); break;
    case 1536: PBM_DN(16, 3, 4, true); break;
    case 2048: // never staged with K >= 6: 32 lanes x 2 chunks per row, no staging buffer
        if (da.stage)
            PBM_DN(16, 4, 4, true);
        else if (!da.use_plan) // one token: 48 units per pass, the 36 of K = 8 + shared in one
            hipExtLaunchKernelGGL((down_combine_kernel<SBT, 16, 4, 3, false, true>), g2, dim3(256), 0, st,
                                  phase_event(d, 4), phase_event(d, 5), 0, da);
        else
            PBM_DN(32, 2, 4, false);
        break;
    default: return hipErrorInvalidValue;
    }
#undef PBM_DN
    err = hipGetLastError();
    if (err != hipSuccess)
        return err;
    if (d.next_norm_w && d.next_normed) {
        next_norm_kernel<<<T, 256, 0, st>>>(d.hidden_out, d.next_norm_w, H, d.eps, d.next_normed);
        err = hipGetLastError();
    }
    return err;
}

static bool set_ok(const ExpertSet& s)
{
    return (1u << s.group_shift) == s.group && s.group >= 32 && s.group <= 128;
}

// ---------------------------------------------------------------------------
// Static scratch of pbmoe_moe_layer_noalloc.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): static_scratch_init looks up the device address once per device
// and every launch uses that pointer.
// ---------------------------------------------------------------------------
constexpr size_t STATIC_SCRATCH_BYTES = PBMOE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};
} // namespace

hipError_t static_scratch_init(int device)
{
    if (device < 0 || device >= MAX_DEVICES)
        return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device])
        return hipSuccess;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
        return e;
    if (!p)
        return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = p;
    return hipSuccess;
}

void* static_scratch(int device, size_t* bytes)
{
    if (bytes)
        *bytes = STATIC_SCRATCH_BYTES;
    if (device < 0 || device >= MAX_DEVICES)
        return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_ptr[device];
}

hipError_t launch_decode_layer(hipStream_t st, const DecodeArgs& d, uint32_t mode)
{
    if (mode != DECODE_ROUTE_ONLY && (!set_ok(d.ex) || (d.shared && !set_ok(*d.shared))))
        return hipErrorInvalidValue; // the kernels index scales with group_shift
    if (d.in_norm_w && (mode != DECODE_FULL_LAYER || !d.x_normed || d.tokens > (uint32_t)DEC_T))
        return hipErrorInvalidValue; // the fused norm runs in the router stage of the full layer
    hipError_t err;
    if (mode == DECODE_ROUTE_ONLY) {
        // router rows, then the routing stage of one wave per token
        err = launch_router_stage(st, d, true, false);
        if (err != hipSuccess)
            return err;
        return launch_route_topk(st, d.logits, d.sel_bias, d.tokens, d.rp, d.ids, d.weights, d.status);
    }
    const bool full = mode == DECODE_FULL_LAYER;
    const bool route_here = full && !route_separately(d);
    err = launch_router_stage(st, d, full, d.shared != nullptr, !shared_rows_in_gateup(d, route_here));
    if (err != hipSuccess)
        return err;
    if (full && !route_here) {
        err = launch_route_topk(st, d.logits, d.sel_bias, d.tokens, d.rp, d.ids, d.weights, d.status);
        if (err != hipSuccess)
            return err;
    }
    if (d.ex.sb_dtype == 2)
        err = launch_experts_typed<2>(st, d, route_here);
    else
        err = launch_experts_typed<1>(st, d, route_here);
    return err;
}

} // namespace pbmoe
