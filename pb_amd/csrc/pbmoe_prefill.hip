// Layer-major prefill of the MoE block on gfx950: a grouped Q4 GEMM on the
// matrix cores (v_mfma_f32_32x32x16_f16).  It replaces the reference's
// per-expert batched matvecs for many-token chunks
// (q4_mmap_fma_matvec_batch_*, metal/qwen/shaders.metal:973-1057, driven by
// qwen_layer_major_experts, metal/mod.rs:3583-4106).
//
// Arithmetic.  The 4-bit codes q in [0, 15] enter the MFMA as exact f16
// values (0x6400 | q is the f16 number 1024 + q; subtracting 1024 is exact),
// and each 16-wide K-step of an MFMA lies inside one quantisation group.  A
// group's partial product P = sum(q * x) is therefore formed in f32 and the
// group scale and bias are applied outside the MFMA:
//     row . x = sum_g  s_g * P_g + b_g * sum_{c in g} x_c
// which is the factored form of fma(q, s, b) . x.  Activations enter as two
// f16 parts, x = hi + lo (about 22 significant bits), so a product keeps
// f32-level accuracy; token rows of x are first scaled by a power of two so
// that hi stays inside the f16 range.  Rounding activations to one f16 (or
// the weights to bf16) would put errors of several 1e-2 on layer outputs
// whose magnitude is in the tens to hundreds.
//
// K order.  Inside every 8-column block the operands are stored in the
// order (c0 c4 c1 c5 c2 c6 c3 c7): the nibble unpack then yields f16 pairs
// without any shuffling.  Activation buffers written here use that order.
//
// Kernels (one layer, T tokens, K routes per token, U used experts):
//   tile_table: per used expert ceil(count / 64) tiles (+ shared expert)
//   split:      x [T][H] f32 -> hi, lo f16 (K order above), sums per 32
//               columns, row scale, whether the row's lo part is nonzero
//   gemm<gate/up>: per (tile, 128-row block of I): gate and up, SiLU(g)*u,
//               act hi/lo f16 (K order) + sums per 32 rows; tiles whose
//               rows all have lo == 0 (f16-valued inputs) skip the lo
//               products, which would add exact zeros
//   gemm<down>: per (tile, 128-row block of H): y [route][H] f32
//   combine:    h = (r + sum_k w_k y_k) + sw * S in route order, optional
//               next-layer RMSNorm
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "pbmoe_device.h"
#include "pbmoe_internal.h"

namespace pbmoe {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int TOK = 64;              // tokens per tile (4 MFMA fragments of 16)
#ifndef PBMOE_GEMM_WAVES
#define PBMOE_GEMM_WAVES 4
#endif
constexpr int GEMM_WAVES = PBMOE_GEMM_WAVES; // waves per GEMM workgroup
constexpr int GEMM_THREADS = 64 * GEMM_WAVES;
constexpr int WG_ROWS = 32 * GEMM_WAVES;      // weight rows per GEMM workgroup (32 per wave)
constexpr float F16_SAFE = 16384.0f; // |hi| bound after the row scale

// position of column c (0..7) inside an 8-column block in the K order
__device__ __forceinline__ uint32_t kpos(uint32_t c) { return c < 4 ? 2 * c : 2 * (c - 4) + 1; }

// (x & mask) | orv in one VALU op; written out because the compiler splits
// it into two instructions with literal operands
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t orv)
{
    uint32_t d;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(x), "s"(mask), "v"(orv));
    return d;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// 8 nibbles of one word as exact f16 codes, in K order; `magic` is
// 0x64006400 (f16 pair 1024, 1024) kept in a vector register.  Nibbles
// 0/4 and 2/6 (after one shift by 8) land in mantissa bits 0-3 (1024 + q,
// minus 1024); nibbles 1/5 and 3/7 are masked in place into bits 4-7
// (1024 + 16q) and recovered as (1024 + 16q) / 16 - 64 = q by one packed
// FMA.  Every step is exact.
__device__ __forceinline__ half8_t unpack8(uint32_t w, uint32_t magic)
{
    const uint32_t w8 = w >> 8;
    const half2_t off = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const half2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2_t off16 = {(_Float16)-64.0f, (_Float16)-64.0f};
    const half2_t v0 = __builtin_bit_cast(half2_t, and_or(w, 0x000F000Fu, magic)) + off;
    const half2_t v1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, and_or(w, 0x00F000F0u, magic)),
                                                 sixteenth, off16);
    const half2_t v2 = __builtin_bit_cast(half2_t, and_or(w8, 0x000F000Fu, magic)) + off;
    const half2_t v3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, and_or(w8, 0x00F000F0u, magic)),
                                                 sixteenth, off16);
    half8_t r;
    r[0] = v0[0], r[1] = v0[1], r[2] = v1[0], r[3] = v1[1];
    r[4] = v2[0], r[5] = v2[1], r[6] = v3[0], r[7] = v3[1];
    return r;
}

// ---------------------------------------------------------------------------
// tile table: for every used expert ceil(count / tok) tiles (records of
// TILE_REC words); the shared expert, when present, is item U with all T
// tokens.  Order:
// the full tiles of all items, then the partial ones (the last tile of an
// item whose count is not a multiple of tok) by their 32-token fragments,
// most first, so that the GEMMs (which deal the list to the XCDs in turn)
// start the longest workgroups first and end on the shortest.  One wave:
// per class, a scan of the per-item tile counts, then each lane writes its
// item's tiles.  Runs in the first workgroup of the split launch (both follow
// the plan and precede the GEMMs).
// ---------------------------------------------------------------------------
struct TileArgs {
    const uint32_t* unique_count;
    const uint32_t* groups;
    const uint32_t* unique_ids;
    uint32_t has_shared;
    uint32_t tokens;
    uint32_t routes; // T*K: the shared expert's rows start here in grouped order
    uint32_t* tiles;
    uint32_t* tile_count;
    uint32_t tok; // tokens per tile (64 or 128)
};
// one tile record: item, first token of the item, the item's first grouped
// row and token count, the expert slot (all ones: the shared expert), 3 unused
constexpr int TILE_REC = 8;

// Tile table, by one 256-thread workgroup: the items' token counts, first
// grouped rows and expert slots are loaded into LDS first (one round trip
// after the item count, every load issued at once), then wave 0 writes the
// records class by class (loaded inside its loop, each class and chunk of
// 64 items waited for its own loads: ~20 dependent round trips).
constexpr uint32_t TT_PER_THREAD = (TILE_TABLE_MAX_ITEMS + 255) / 256;
__device__ void tile_table_block(const TileArgs& a)
{
    __shared__ uint32_t t_cnt[TILE_TABLE_MAX_ITEMS], t_g0[TILE_TABLE_MAX_ITEMS], t_e[TILE_TABLE_MAX_ITEMS];
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t has_shared = a.has_shared, tokens = a.tokens;
    uint32_t* tiles = a.tiles;
    const uint32_t U = a.unique_count[0];
    const uint32_t items = U + has_shared; // <= experts + 1 <= TILE_TABLE_MAX_ITEMS (the ABI's limit)
    {
        // clamped indices, no branch around the loads (a load inside a
        // divergent branch is waited for where the branch ends)
        uint32_t c[TT_PER_THREAD], g[TT_PER_THREAD], e[TT_PER_THREAD];
        const uint32_t last = U > 0 ? U - 1 : 0;
#pragma unroll
        for (int k = 0; k < (int)TT_PER_THREAD; ++k) {
            const uint32_t u = min(threadIdx.x + 256u * k, last);
            g[k] = a.groups[2 * u];
            c[k] = a.groups[2 * u + 1];
            e[k] = a.unique_ids[u];
        }
#pragma unroll
        for (int k = 0; k < (int)TT_PER_THREAD; ++k) {
            const uint32_t u = threadIdx.x + 256u * k;
            if (u < U)
                t_cnt[u] = c[k], t_g0[u] = g[k], t_e[u] = e[k];
            else if (u < items) // the shared expert: every token, rows after the routes
                t_cnt[u] = tokens, t_g0[u] = a.routes, t_e[u] = 0xFFFFFFFFu;
        }
    }
    __syncthreads();
    if (threadIdx.x >= 64)
        return;
    const uint32_t nfrag = a.tok / 32;
    uint32_t base = 0;
    // class 0: full tiles; class c = 1 .. nfrag: the partial tile with
    // nfrag + 1 - c fragments
    for (uint32_t c = 0; c <= nfrag; ++c) {
        for (uint32_t u0 = 0; u0 < items; u0 += 64) {
            const uint32_t u = u0 + lane;
            const uint32_t cnt = u < items ? t_cnt[u] : 0u;
            const uint32_t full = cnt / a.tok, rest = cnt % a.tok;
            uint32_t nt;
            if (c == 0)
                nt = full;
            else
                nt = rest != 0 && (rest + 31) / 32 == nfrag + 1 - c ? 1u : 0u;
            uint32_t inc = nt; // inclusive scan over the wave
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t v = __shfl_up(inc, o);
                if ((int)lane >= o)
                    inc += v;
            }
            const uint32_t first = base + inc - nt;
            if (nt) {
                const uint32_t g0 = t_g0[u], e = t_e[u];
                for (uint32_t j = 0; j < nt; ++j) {
                    uint4* rec = reinterpret_cast<uint4*>(tiles + TILE_REC * (first + j));
                    rec[0] = make_uint4(u, c == 0 ? j * a.tok : full * a.tok, g0, cnt);
                    rec[1] = make_uint4(e, 0u, 0u, 0u);
                }
            }
            base += __shfl(inc, 63);
        }
    }
    if (lane == 0)
        a.tile_count[0] = base;
}

// Work unit of a GEMM workgroup: the tiles are dealt to the 8 XCDs in turn
// (tile t on XCD t % 8: workgroup b runs on XCD b % 8), and the row blocks
// of one tile are consecutive on its XCD, so they share that XCD's L2 for
// the tile's activation rows.  In tile-table order, each XCD meets its
// largest tiles first.  Grid: 8 * RB * ceil(max_tiles / 8) (gemm_units).
__device__ __forceinline__ void gemm_unit_of(uint32_t RB, uint32_t& tile, uint32_t& rb)
{
    const uint32_t j = blockIdx.x >> 3, xcd = blockIdx.x & 7;
    tile = 8 * (j / RB) + xcd;
    rb = j % RB;
}
__device__ __forceinline__ bool gemm_unit(uint32_t ntiles, uint32_t RB, uint32_t& tile, uint32_t& rb)
{
    gemm_unit_of(RB, tile, rb);
    return tile < ntiles;
}

// ---------------------------------------------------------------------------
// split: one workgroup per token row, one 8-column block per thread and
// step (two 16-byte loads, one 16-byte store each for hi and lo).  hi/lo f16
// of x * 2^-e in K order, sums of x * 2^-e per 32 columns (four lanes),
// with sum_hl also the group sums (ks = 2 sums of 32 columns) as f16 hi and
// lo, the operand of the 128-token GEMM's bias term ([T][hi: GP][lo: GP],
// GP = groups rounded up to 16, the padding zero), rowscale = 2^e (e > 0
// only for rows whose elements would leave the f16 range, or whose group
// sums, bounded by ks times the largest sum of 32 columns, would), and
// whether any lo is nonzero (rows of f16-valued inputs have
// lo == 0 throughout; the gate/up GEMM then skips the lo products, which
// would add exact zeros).  The row scale and the lo flag are written in
// grouped order, once per route of the token (out_idx) and for the shared
// expert's row (routes + t), where the GEMMs read them beside the token
// rows.  cols is a multiple of 64.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ x, uint32_t cols,
                                                         uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo,
                                                         float* __restrict__ sum32,
                                                         uint16_t* __restrict__ sum_hl, uint32_t ks,
                                                         float* __restrict__ rowscale,
                                                         uint32_t* __restrict__ lo_any,
                                                         const uint32_t* __restrict__ out_idx, uint32_t k,
                                                         TileArgs ta)
{
    // the tile table in the first workgroup, which starts before the token
    // rows' workgroups and runs beside them (it needs the plan only)
    if (blockIdx.x == 0) {
        tile_table_block(ta);
        return;
    }
    __shared__ float red[8];
    const uint32_t t = blockIdx.x - 1;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const float4* xr = reinterpret_cast<const float4*>(x + (uint64_t)t * cols);
    const uint32_t nb = cols / 8;
    float amax = 0.0f, smax = 0.0f;
    // the thread's first NBR blocks stay in registers for the second pass
    // (cols <= 8192), loaded unconditionally (clamped) so that every load is
    // in flight at once; blocks past them are read again there (L2 hits)
    constexpr int NBR = 4;
    float4 pr[NBR], qr[NBR];
#pragma unroll
    for (int k = 0; k < NBR; ++k) {
        const uint32_t b = min(threadIdx.x + 256u * k, nb - 1);
        pr[k] = xr[2 * b], qr[k] = xr[2 * b + 1];
    }
    auto first = [&](const float4 p, const float4 q) __attribute__((always_inline)) {
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(p.x), fabsf(p.y)), fmaxf(fabsf(p.z), fabsf(p.w))));
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(q.x), fabsf(q.y)), fmaxf(fabsf(q.z), fabsf(q.w))));
        float s = ((p.x + p.y) + (p.z + p.w)) + ((q.x + q.y) + (q.z + q.w));
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        smax = fmaxf(smax, fabsf(s));
    };
#pragma unroll
    for (int k = 0; k < NBR; ++k)
        if (threadIdx.x + 256u * k < nb)
            first(pr[k], qr[k]);
    for (uint32_t b = threadIdx.x + 256u * NBR; b < nb; b += 256)
        first(xr[2 * b], xr[2 * b + 1]);
    amax = wave_max(amax);
    smax = wave_max(smax);
    if (lane == 0)
        red[wv] = amax, red[4 + wv] = smax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    smax = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
    // e: elements within F16_SAFE and group sums (at most ks * smax, up to
    // rounding) within 32768, so that their f16 hi parts stay finite; a
    // power of two scales every element and sum exactly
    const float r = fmaxf(amax / F16_SAFE, smax * (float)ks / 32768.0f);
    int e = 0;
    if (r > 1.0f)
        (void)frexpf(r, &e); // r * 2^-e < 1
    const float f = ldexpf(1.0f, -e);
    const uint32_t G = cols / 64, GP = (G + 15) / 16 * 16;
    uint16_t* const hl = sum_hl != nullptr ? sum_hl + (uint64_t)t * 2 * GP : nullptr;
    int any_lo = 0;
    // nb is a multiple of 4: the four blocks of 32 columns are on four
    // consecutive lanes, all present or all absent
    auto second = [&](uint32_t b, const float4 p, const float4 q) __attribute__((always_inline)) {
        const float v[8] = {p.x * f, p.y * f, p.z * f, p.w * f, q.x * f, q.y * f, q.z * f, q.w * f};
        uint32_t hw[4], lw[4];
        // K order inside the block: c0 c4 c1 c5 c2 c6 c3 c7 (word j = columns j, j + 4)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const _Float16 ha = (_Float16)v[j], hb = (_Float16)v[j + 4];
            const _Float16 la = (_Float16)(v[j] - (float)ha), lb = (_Float16)(v[j + 4] - (float)hb);
            hw[j] = __builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
            lw[j] = __builtin_bit_cast(uint16_t, la) | ((uint32_t)__builtin_bit_cast(uint16_t, lb) << 16);
            any_lo |= la != (_Float16)0.0f || lb != (_Float16)0.0f;
        }
        const uint64_t o = (uint64_t)t * cols + 8 * b;
        *reinterpret_cast<uint4*>(hi + o) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *reinterpret_cast<uint4*>(lo + o) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        if ((lane & 3) == 0)
            sum32[(uint64_t)t * (cols / 32) + b / 4] = s;
        if (hl != nullptr) {
            // the group of 64 columns on 8 lanes (cols is a multiple of 64):
            // its two sums of 32 added as the GEMMs add them, then hi + lo
            const float g = s + __shfl_xor(s, 4);
            if ((lane & 7) == 0) {
                const _Float16 gh = (_Float16)g;
                hl[b / 8] = __builtin_bit_cast(uint16_t, gh);
                hl[GP + b / 8] = __builtin_bit_cast(uint16_t, (_Float16)(g - (float)gh));
            }
        }
    };
#pragma unroll
    for (int k = 0; k < NBR; ++k) {
        const uint32_t b = threadIdx.x + 256u * k;
        if (b < nb)
            second(b, pr[k], qr[k]);
    }
    for (uint32_t b = threadIdx.x + 256u * NBR; b < nb; b += 256)
        second(b, xr[2 * b], xr[2 * b + 1]);
    if (hl != nullptr)
        for (uint32_t gi = G + threadIdx.x; gi < GP; gi += 256)
            hl[gi] = 0, hl[GP + gi] = 0;
    any_lo = __syncthreads_or(any_lo);
    const uint32_t j = threadIdx.x;
    if (j < k + (ta.has_shared ? 1u : 0u)) {
        // a route the plan rejected (expert out of range) has no grouped row:
        // out_idx all ones
        const uint32_t pos = j < k ? out_idx[(uint64_t)t * k + j] : ta.routes + t;
        if (pos < ta.routes + ta.tokens) {
            rowscale[pos] = ldexpf(1.0f, e);
            lo_any[pos] = any_lo ? 1u : 0u;
        }
    }
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
struct GemmArgs {
    ExpertSet ex, sh;
    uint32_t has_shared;
    const uint32_t* unique_ids;
    const uint32_t* unique_count;
    const uint32_t* groups;   // [items][2] (start, count) in grouped order
    const uint32_t* src_rows; // grouped route -> token
    const uint32_t* tiles;    // [n][2] (item, first token of the item)
    const uint32_t* tile_count;
    uint32_t routes;          // T*K: grouped rows of the routed experts
    uint32_t tokens;
    // B operand rows (hi/lo f16 in K order + sums per 32 columns)
    const uint16_t* b_hi;
    const uint16_t* b_lo;
    const float* b_sum32;
    const uint16_t* b_sumhl;  // 128-token GEMMs: group sums as f16 hi, lo [b_rows][hi: GP][lo: GP]
    const float* rowscale;    // gate/up: per grouped row; down: unused
    const uint32_t* b_lo_any; // gate/up: per grouped row, its B row's lo part is not all zero (null: assume it is not)
    uint32_t kdim;            // H (gate/up) or I (down)
    uint32_t b_rows;          // rows of the B operand buffers
    uint32_t lo_delta;        // bytes from b_hi to b_lo (one allocation)
    // outputs
    uint16_t* act_hi;         // [routes + T][I]
    uint16_t* act_lo;
    float* act_sum32;         // [routes + T][I/32] (64-token gate/up)
    uint16_t* act_sumhl;      // [routes + T][2][GP] (128-token gate/up: the down GEMM's b_sumhl)
    float* y;                 // [routes + T][H]
    uint32_t* status;
};

// LDS plan of one GEMM workgroup.  Staging: NBUF buffers, each the
// activation tile of one quantisation group, [TOK tokens][CH 16-byte
// chunks], the group's hi and lo chunks interleaved (chunk 2c = hi chunk c,
// 2c + 1 = lo chunk c) and chunk c of token row r stored at position
// c ^ (r % CH), so that the rows of a fragment read fall on distinct bank
// groups.  The tiles are written by direct global->LDS loads (one wave
// instruction fills 1 KB, lane i bytes 16i .. 16i + 15), which is why the
// layout is swizzled rather than padded.  The epilogue reuses the bytes for
// the f32 output tile [TOK][WG_ROWS + 4].
template <int KS>
struct GemmLds {
    static constexpr int CH = 8 * KS;            // 16-byte chunks per token row
    static constexpr int NBUF = KS >= 4 ? 2 : 4; // groups resident (staged ahead: NBUF - 1)
    static constexpr int TILE_BYTES = TOK * CH * 16;
    static constexpr int STAGE_BYTES = NBUF * TILE_BYTES;
    static constexpr int OPITCH = WG_ROWS + 4;
    static constexpr int OUT_BYTES = TOK * OPITCH * 4;
    static constexpr int BYTES = STAGE_BYTES > OUT_BYTES ? STAGE_BYTES : OUT_BYTES;
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// raw buffer resource over [p, p + bytes): 32-bit offsets, loads past the
// end return zero
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <int N>
__device__ __forceinline__ void load_words(rsrc_t r, uint32_t voff, uint32_t soff, uint32_t (&w)[N])
{
    if constexpr (N == 8) {
        const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
        const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
        w[0] = v0[0], w[1] = v0[1], w[2] = v0[2], w[3] = v0[3];
        w[4] = v1[0], w[5] = v1[1], w[6] = v1[2], w[7] = v1[3];
    } else if constexpr (N == 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
        w[0] = v[0], w[1] = v[1], w[2] = v[2], w[3] = v[3];
    } else if constexpr (N == 2) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
        w[0] = v[0], w[1] = v[1];
    } else {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
}

template <int SBT>
__device__ __forceinline__ float sb_buf(rsrc_t r, uint32_t voff, uint32_t soff)
{
    const uint16_t v = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
    if constexpr (SBT == 2)
        return __uint_as_float((uint32_t)v << 16);
    else
        return __half2float(__ushort_as_half(v));
}

// One workgroup: TOK tokens of one item x WG_ROWS weight rows, GEMM_WAVES
// waves; two workgroups per CU, so that the two waves sharing a SIMD belong
// to different workgroups and their barriers do not lock them into the same
// phase (one wave's VALU work then overlaps the other's MFMAs).
// MFMA 32x32x16 f16: the activation tile is the A operand (32 tokens x 16 K
// per fragment), the weights the B operand (16 K x 32 rows); wave w owns
// rows 32w .. 32w+31 of the block, one row per lane (lane & 31), and both
// 32-token fragments.  Lane half h = lane >> 5 supplies, for quantisation
// group g, the 2KS words (16KS columns) [g*32KS + 16KS*h, +16KS) of its
// row; word s is K-step s, so each K-step stays inside group g and a
// lane's group of weights is one 4KS-byte load.  The accumulator element
// (token 8(j/4) + 4h + (j%4) of the fragment, the lane's row) gets
// s[row][g] * P after each group; the bias term sum_g b[row][g] * xsum_g
// runs on the matrix cores after the loop.
//
// Work mapping (gemm_unit): tile t on XCD t % 8, its row blocks back to
// back there, sharing the activation tile in that XCD's L2; largest tiles
// first.
template <int SBT, bool GATEUP, int KS>
__global__ __launch_bounds__(GEMM_THREADS, 2) void q4_group_gemm_kernel(GemmArgs a)
{
    using L = GemmLds<KS>;
    constexpr int NMAT = GATEUP ? 2 : 1;
    constexpr int NSTEP = 2 * KS; // 16-column K-steps per quantisation group
    __shared__ __align__(16) uint8_t lds[L::BYTES];
    __shared__ uint32_t row_lds[TOK];
    __shared__ float rs_lds[TOK];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    // ---- work item ----
    const uint32_t ntiles = a.tile_count[0];
    const uint32_t rows_total = GATEUP ? a.ex.gate.rows : a.ex.down.rows;
    const uint32_t RB = rows_total / WG_ROWS;
    uint32_t tile, rb;
    if (!gemm_unit(ntiles, RB, tile, rb))
        return;
    // the tile record: item, first token, the item's first grouped row and
    // token count, expert slot (all ones: the shared expert)
    const uint4 rec = *reinterpret_cast<const uint4*>(a.tiles + TILE_REC * tile);
    const uint32_t n0 = rec.y, g0 = rec.z, cnt = rec.w, e = a.tiles[TILE_REC * tile + 4];
    const bool shared = e == 0xFFFFFFFFu;
    if (shared ? a.has_shared == 0u : e >= a.ex.count) {
        if (tid == 0)
            atomicOr(a.status, ST_ROUTE_RANGE);
        return;
    }
    const uint8_t* const slot = shared ? a.sh.base : a.ex.base + (uint64_t)e * a.ex.stride;
    const ExpertSet& set = shared ? a.sh : a.ex;
    const Q4Proj p0 = GATEUP ? set.gate : set.down;
    const Q4Proj p1 = set.up;
    const uint32_t K = a.kdim;
    const uint32_t G = K / (32 * KS), C32 = K / 32, WPR = K / 8;

    // ---- staging: direct global->LDS loads, DW wave instructions per group;
    //      instruction j fills chunk positions 64j .. 64j + 63 of the tile ----
    constexpr int CH = L::CH, NBUF = L::NBUF, PF = NBUF - 1;
    constexpr int DW = TOK * CH / 64 / GEMM_WAVES;
    auto tok_row = [&](uint32_t n) -> uint32_t {
        return GATEUP ? (shared ? n : a.src_rows[g0 + n]) : g0 + n;
    };
    int lo_flag = 0;
    if (tid < TOK) {
        const uint32_t n = n0 + tid;
        const bool v = n < cnt;
        const uint32_t r = v ? tok_row(n) : 0u;
        row_lds[tid] = v ? r : 0xFFFFFFFFu;
        if (GATEUP)
            rs_lds[tid] = v ? a.rowscale[g0 + n] : 1.0f;
        lo_flag = v && (a.b_lo_any == nullptr || a.b_lo_any[g0 + n] != 0u);
    }
    // whether any token row of the tile has a nonzero lo part; if none has,
    // the lo products would all be exact zeros and are skipped
    const bool tile_lo = __syncthreads_or(lo_flag) != 0;
    const uint32_t first_row = tok_row(n0); // n0 < cnt
    const uint16_t* dsrc[DW];               // this lane's chunk of each instruction, group 0
#pragma unroll
    for (int i = 0; i < DW; ++i) {
        const uint32_t pos = 64 * (wv + GEMM_WAVES * i) + lane;
        const uint32_t r = pos / CH, c = (pos % CH) ^ (r % CH);
        const uint32_t n = n0 + r;
        const uint32_t trow = n < cnt ? tok_row(n) : first_row; // rows past the item: any valid row
        dsrc[i] = ((c & 1) ? a.b_lo : a.b_hi) + (uint64_t)trow * K + (c >> 1) * 8;
    }
    auto stage = [&](uint32_t g, int buf) {
#pragma unroll
        for (int i = 0; i < DW; ++i)
            __builtin_amdgcn_global_load_lds(
                (const void*)(dsrc[i] + g * 32 * KS),
                (__attribute__((address_space(3))) void*)(lds + buf * L::TILE_BYTES + 1024 * (wv + GEMM_WAVES * i)),
                16, 0, 0);
    };

    // ---- compute role ----
    const uint32_t n32 = lane & 31, h = lane >> 5;
    const uint32_t row = rb * WG_ROWS + wv * 32 + n32; // this lane's weight row
    const rsrc_t wr = make_rsrc(slot, (uint32_t)set.stride);
    const uint32_t w_voff = (row * WPR + h * 2 * KS) * 4;
    const uint32_t sb_voff = row * G * 2;
    const uint32_t w_soff[2] = {(uint32_t)p0.w_off, (uint32_t)p1.w_off};
    const uint32_t s_soff[2] = {(uint32_t)p0.s_off, (uint32_t)p1.s_off};
    const uint32_t b_soff[2] = {(uint32_t)p0.b_off, (uint32_t)p1.b_off};
    const uint32_t magic = 0x64006400u;
    typedef uint32_t Words[NMAT][2 * KS];
    Words w0, w1; // codes of the even / odd group in flight
    constexpr int WL = 2 * KS == 8 ? 2 : 1; // load instructions per w_load matrix
    auto w_load = [&](uint32_t g, Words& w) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
            load_words<2 * KS>(wr, w_voff, w_soff[m] + g * 16 * KS, w[m]);
    };
    // scales of a pair of groups (g even; G is even) in one 32-bit load
    uint32_t spa[NMAT], spb[NMAT];
    auto s_load = [&](uint32_t g, uint32_t (&sp)[NMAT]) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
            sp[m] = __builtin_amdgcn_raw_buffer_load_b32(wr, sb_voff, s_soff[m] + g * 2, 0);
    };
    auto s_of = [&](uint32_t pair, uint32_t g) -> float {
        const uint16_t v = (uint16_t)(pair >> ((g & 1) * 16));
        if constexpr (SBT == 2)
            return __uint_as_float((uint32_t)v << 16);
        else
            return __half2float(__ushort_as_half(v));
    };
    // fragment reads: row 32tf + n32 of the tile, chunk c = 2(h NSTEP + k) + hl
    // at position c ^ (n32 % CH) (32tf is a multiple of CH)
    uint32_t rd_off[NSTEP][2];
#pragma unroll
    for (int k = 0; k < NSTEP; ++k)
#pragma unroll
        for (int hl = 0; hl < 2; ++hl)
            rd_off[k][hl] = (n32 * CH + ((2 * (h * NSTEP + k) + hl) ^ (n32 % CH))) * 16;

    float16_t acc[2][NMAT];
#pragma unroll
    for (int tf = 0; tf < 2; ++tf)
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                acc[tf][m][j] = 0.0f;

    // Pipeline (the loop is unrolled by NBUF, so buffers and registers have
    // fixed roles).  Step g, buffer g % NBUF: stage group g + PF into buffer
    // (g + PF) % NBUF, which held group g - 1 (read before the last barrier).
    // The MFMAs of group g use codes unpacked during step g - 1 (wf_cur);
    // beside them the step unpacks group g + 1's codes (w, into wf_next; then
    // group g + 3's codes are loaded into w) and applies the group scales to
    // finished fragments: fragment 0 of group g while fragment 1's MFMAs run,
    // fragment 1 of group g - 1 while fragment 0's run.  None of that VALU
    // work depends on the MFMAs beside it, so the wave issues it while the
    // matrix core works.  Then wait until this wave's loads of group g + 1's
    // tile have landed and meet the other waves at the barrier.  The last
    // NBUF steps (TAIL) issue no loads past group G - 1.  Wait counts: the
    // instructions of steps g - 1 and g were all issued after the staging of
    // group g + 1 (the order inside one step is the compiler's).
    constexpr int VMW = (PF - 1) * (DW + NMAT * WL) + (PF >= 2 ? NMAT : 0);
    constexpr bool PIPE = !GATEUP && KS <= 2; // larger groups: the pipeline spills
    typedef half8_t Unpacked[NMAT][NSTEP];
    Unpacked wfA, wfB;              // unpacked codes of even / odd groups
    float16_t pf1[NMAT];             // fragment 1's partial products, scaled one step later
    float sa_prev[NMAT];            // their group scales
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        sa_prev[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            pf1[m][j] = 0.0f;
    }
    auto unpack_m = [&](Words& w, Unpacked& wf, int m) {
#pragma unroll
        for (int k = 0; k < NSTEP; ++k) {
            // keeps each unpack in its step: without it the compiler hoists
            // the unpacks of load-free tail steps and spills
            asm volatile("" : "+v"(w[m][k]));
            wf[m][k] = unpack8(w[m][k], magic);
        }
    };
    auto step = [&](auto lo_tag, auto tf_tag, uint32_t g, auto b_tag, auto tail_tag, Words& w, Unpacked& wf_cur,
                    Unpacked& wf_next) {
        constexpr bool LO = decltype(lo_tag)::value; // lo products of the activations
        constexpr int NTF = decltype(tf_tag)::value; // 32-token fragments holding tokens of the item
        constexpr int NHL = LO ? 2 : 1;
        constexpr int B = decltype(b_tag)::value;    // g % NBUF
        constexpr bool TAIL = decltype(tail_tag)::value;
        constexpr bool ST = !TAIL || B + PF < NBUF;  // stage group g + PF
        constexpr bool UNP = !TAIL || B + 1 < NBUF;  // unpack group g + 1
        constexpr bool WLD = !TAIL || B + 3 < NBUF;  // codes of group g + 3
        constexpr bool SLD = B % 2 == 0 && (!TAIL || B + 2 < NBUF); // scales of groups g + 2, g + 3
        // VMEM instructions of tail step b (b = -1: the steady step before)
        constexpr auto cnt = [](int b) {
            if (b < 0)
                return DW + NMAT * WL;
            return (b + PF < NBUF ? DW : 0) + (b % 2 == 0 && b + 2 < NBUF ? NMAT : 0) +
                   (b + 3 < NBUF ? NMAT * WL : 0);
        };
        constexpr int WAIT = PF < 2 ? 0 : (TAIL ? cnt(B - 1) + cnt(B) : VMW);
        if constexpr (ST)
            stage(g + PF, (B + PF) % NBUF);
        if constexpr (SLD)
            s_load(g + 2, spb);
        float sa[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
            sa[m] = s_of(spa[m], g);
        const uint8_t* xb = lds + B * L::TILE_BYTES;
        auto mfmas = [&](int tf, float16_t (&p)[NMAT]) {
            half8_t ah[NSTEP], al[NSTEP];
#pragma unroll
            for (int k = 0; k < NSTEP; ++k) {
                ah[k] = *reinterpret_cast<const half8_t*>(xb + tf * 32 * CH * 16 + rd_off[k][0]);
                if constexpr (LO)
                    al[k] = *reinterpret_cast<const half8_t*>(xb + tf * 32 * CH * 16 + rd_off[k][1]);
            }
#pragma unroll
            for (int k = 0; k < NSTEP; ++k)
#pragma unroll
                for (int hl = 0; hl < NHL; ++hl)
#pragma unroll
                    for (int m = 0; m < NMAT; ++m) {
                        float16_t c;
                        if (k == 0 && hl == 0) {
#pragma unroll
                            for (int j = 0; j < 16; ++j)
                                c[j] = 0.0f;
                        } else {
                            c = p[m];
                        }
                        p[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(hl ? al[k] : ah[k], wf_cur[m][k], c, 0, 0, 0);
                    }
        };
        auto scale = [&](int tf, const float16_t (&p)[NMAT], const float (&s)[NMAT]) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    acc[tf][m][j] = fmaf(s[m], p[m][j], acc[tf][m][j]);
        };
        // fragment 0 of group g; beside it: group g + 1's unpack (then the
        // codes of group g + 3 are loaded into the freed registers) and
        // fragment 1 of group g - 1
        float16_t p0[NMAT];
        mfmas(0, p0);
        if constexpr (UNP) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                unpack_m(w, wf_next, m);
        }
        if constexpr (WLD)
            w_load(g + 3, w);
        if constexpr (NTF == 2) {
            scale(1, pf1, sa_prev);
            // fragment 1 of group g; beside it: fragment 0 of group g
            mfmas(1, pf1);
        }
        scale(0, p0, sa);
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
            sa_prev[m] = sa[m];
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT) : "memory");
        __syncthreads();
        if constexpr (B % 2 == 1) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                spa[m] = spb[m];
        }
    };
    // The same step without the software pipeline (codes of group g unpacked
    // and scaled within step g), for the gate/up GEMM: the pipeline's extra
    // live registers (next group's codes, a fragment's partial products
    // across steps) do not fit beside its two weight matrices.
    auto step_serial = [&](auto lo_tag, auto tf_tag, uint32_t g, auto b_tag, auto tail_tag, Words& w) {
        constexpr bool LO = decltype(lo_tag)::value; // lo products of the activations
        constexpr int NTF = decltype(tf_tag)::value; // 32-token fragments holding tokens of the item
        constexpr int NHL = LO ? 2 : 1;
        constexpr int B = decltype(b_tag)::value;    // g % NBUF
        constexpr bool TAIL = decltype(tail_tag)::value;
        constexpr bool ST = !TAIL || B + PF < NBUF;  // stage group g + PF
        constexpr bool WLD = !TAIL || B + 2 < NBUF;  // codes of group g + 2
        constexpr bool SLD = B % 2 == 0 && WLD;      // scales of groups g + 2, g + 3
        // VMEM instructions of tail step b (b = -1: the steady step before)
        constexpr auto cnt = [](int b) {
            if (b < 0)
                return DW + NMAT * WL;
            return (b + PF < NBUF ? DW : 0) + (b % 2 == 0 && b + 2 < NBUF ? NMAT : 0) +
                   (b + 2 < NBUF ? NMAT * WL : 0);
        };
        constexpr int WAIT = PF < 2 ? 0 : (TAIL ? cnt(B - 1) + cnt(B) : VMW);
        if constexpr (ST)
            stage(g + PF, (B + PF) % NBUF);
        if constexpr (SLD)
            s_load(g + 2, spb);
        float sa[NMAT];
        half8_t wf[NMAT][NSTEP];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            sa[m] = s_of(spa[m], g);
#pragma unroll
            for (int k = 0; k < NSTEP; ++k) {
                // keeps the unpack inside its step: without it the compiler
                // hoists the unpacks of load-free tail steps and spills
                asm volatile("" : "+v"(w[m][k]));
                wf[m][k] = unpack8(w[m][k], magic);
            }
        }
        if constexpr (WLD)
            w_load(g + 2, w);
        const uint8_t* xb = lds + B * L::TILE_BYTES;
#pragma unroll
        for (int tf = 0; tf < NTF; ++tf) {
            half8_t ah[NSTEP], al[NSTEP];
#pragma unroll
            for (int k = 0; k < NSTEP; ++k) {
                ah[k] = *reinterpret_cast<const half8_t*>(xb + tf * 32 * CH * 16 + rd_off[k][0]);
                if constexpr (LO)
                    al[k] = *reinterpret_cast<const half8_t*>(xb + tf * 32 * CH * 16 + rd_off[k][1]);
            }
            float16_t p[NMAT];
#pragma unroll
            for (int k = 0; k < NSTEP; ++k)
#pragma unroll
                for (int hl = 0; hl < NHL; ++hl)
#pragma unroll
                    for (int m = 0; m < NMAT; ++m) {
                        float16_t c;
                        if (k == 0 && hl == 0) {
#pragma unroll
                            for (int j = 0; j < 16; ++j)
                                c[j] = 0.0f;
                        } else {
                            c = p[m];
                        }
                        p[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(hl ? al[k] : ah[k], wf[m][k], c, 0, 0, 0);
                    }
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    acc[tf][m][j] = fmaf(sa[m], p[m][j], acc[tf][m][j]);
        }
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT) : "memory");
        __syncthreads();
        if constexpr (B % 2 == 1) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                spa[m] = spb[m];
        }
    };
    // prologue: the first PF tiles, group 0's codes unpacked, groups 1 and 2's
    // codes loaded (G >= NBUF > PF)
#pragma unroll
    for (int d = 0; d < PF; ++d)
        stage(d, d);
    w_load(0, w0);
    s_load(0, spa);
    w_load(1, w1);
    if constexpr (PIPE) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
            unpack_m(w0, wfA, m);
        if (G > 2)
            w_load(2, w0);
    }

    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    auto iter = [&](auto lo_tag, auto tf_tag, uint32_t g, auto tail_tag) {
        if constexpr (PIPE) {
            step(lo_tag, tf_tag, g, I0{}, tail_tag, w1, wfA, wfB);
            step(lo_tag, tf_tag, g + 1, I1{}, tail_tag, w0, wfB, wfA);
            if constexpr (NBUF == 4) {
                step(lo_tag, tf_tag, g + 2, I2{}, tail_tag, w1, wfA, wfB);
                step(lo_tag, tf_tag, g + 3, I3{}, tail_tag, w0, wfB, wfA);
            }
        } else {
            step_serial(lo_tag, tf_tag, g, I0{}, tail_tag, w0);
            step_serial(lo_tag, tf_tag, g + 1, I1{}, tail_tag, w1);
            if constexpr (NBUF == 4) {
                step_serial(lo_tag, tf_tag, g + 2, I2{}, tail_tag, w0);
                step_serial(lo_tag, tf_tag, g + 3, I3{}, tail_tag, w1);
            }
        }
    };
    auto run = [&](auto lo_tag, auto tf_tag) {
        uint32_t g = 0;
        for (; g + NBUF < G; g += NBUF) // G is a multiple of NBUF
            iter(lo_tag, tf_tag, g, std::false_type{});
        iter(lo_tag, tf_tag, g, std::true_type{});
        if constexpr (PIPE && decltype(tf_tag)::value == 2) { // fragment 1 of the last group
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    acc[1][m][j] = fmaf(sa_prev[m], pf1[m][j], acc[1][m][j]);
        }
    };
    // the last tile of an item often holds at most 32 tokens: the second
    // fragment's MFMAs, LDS reads and scale FMAs would only produce rows
    // that are never written
    const bool two_frag = cnt - n0 > 32;
    if (tile_lo) {
        if (two_frag)
            run(std::true_type{}, I2{});
        else
            run(std::true_type{}, I1{});
    } else {
        if (two_frag)
            run(std::false_type{}, I2{});
        else
            run(std::false_type{}, I1{});
    }
    // the last step waited for every load and met the other waves: the
    // staging buffers are free for the epilogue

    // ---- bias term on the matrix cores: acc += sum_g b[row][g] * xsum[token][g],
    //      K' = groups in steps of 16 (lane half h: groups k0 + 8h .. +8),
    //      the group sums split into f16 hi + lo.  Vector loads through buffer
    //      resources (reads past a row are masked, past the buffer return 0) ----
    const rsrc_t sum_r = make_rsrc(a.b_sum32, a.b_rows * C32 * 4);
    // the loads of MAXS slices of 16 groups are issued together (one memory
    // round trip instead of MAXS); loads of a slice past G read in-bounds
    // neighbouring data or zeros and are masked below
    constexpr int MAXS = KS >= 4 ? 1 : 2;
    bool sum_range = false; // a group sum outside the f16 range of its hi part
    for (uint32_t k00 = 0; k00 < G; k00 += 16 * MAXS) {
        uint32_t b2[MAXS][NMAT][4]; // 8 consecutive 16-bit biases per slice (4-byte aligned: G is even)
        u32x4 v4[MAXS][2][2 * KS];  // sums per 32 columns of groups gb .. gb + 7
#pragma unroll
        for (int sl = 0; sl < MAXS; ++sl) {
            const uint32_t gb = k00 + 16 * sl + 8 * h; // first group of this lane half
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    b2[sl][m][q] = __builtin_amdgcn_raw_buffer_load_b32(wr, sb_voff, b_soff[m] + gb * 2 + 4 * q, 0);
#pragma unroll
            for (int tf = 0; tf < 2; ++tf) {
                const uint32_t brow = row_lds[32 * tf + n32];
                const uint32_t rrow = brow != 0xFFFFFFFFu ? brow : 0u;
#pragma unroll
                for (int q = 0; q < 2 * KS; ++q)
                    v4[sl][tf][q] = __builtin_amdgcn_raw_buffer_load_b128(sum_r, rrow * C32 * 4, (gb * KS + 4 * q) * 4, 0);
            }
        }
#pragma unroll
        for (int sl = 0; sl < MAXS; ++sl) {
            const uint32_t gb = k00 + 16 * sl + 8 * h;
            if (k00 + 16 * sl >= G)
                break;
            half8_t bw[NMAT];
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint16_t raw = (uint16_t)(b2[sl][m][j / 2] >> (16 * (j & 1)));
                    float bv;
                    if constexpr (SBT == 2)
                        bv = __uint_as_float((uint32_t)raw << 16);
                    else
                        bv = __half2float(__ushort_as_half(raw));
                    bw[m][j] = gb + j < G ? (_Float16)bv : (_Float16)0.0f;
                }
#pragma unroll
            for (int tf = 0; tf < 2; ++tf) {
                const bool bvalid = row_lds[32 * tf + n32] != 0xFFFFFFFFu;
                half8_t xh, xl;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float v = 0.0f;
#pragma unroll
                    for (int c = 0; c < KS; ++c)
                        v += __uint_as_float(v4[sl][tf][(j * KS + c) / 4][(j * KS + c) % 4]);
                    if (!bvalid || gb + j >= G)
                        v = 0.0f;
                    sum_range |= !(fabsf(v) <= 65504.0f);
                    const _Float16 hv = (_Float16)v;
                    xh[j] = hv;
                    xl[j] = (_Float16)(v - (float)hv);
                }
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    float16_t c;
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        c[j] = 0.0f;
                    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, bw[m], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, bw[m], c, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        acc[tf][m][j] += c[j];
                }
            }
        }
    }
    if (sum_range)
        atomicOr(a.status, ST_F16_RANGE);

    // ---- epilogue: accumulator element (token 32tf + 8(j/4) + 4h + (j%4),
    //      row wv*32 + n32 of the block) -> f32 tile in LDS -> each thread
    //      (token, 32-row chunk) writes whole rows ----
    float* ot = reinterpret_cast<float*>(lds);
    const uint32_t col = wv * 32 + n32;
#pragma unroll
    for (int tf = 0; tf < 2; ++tf)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t tk = 32 * tf + 8 * (j / 4) + 4 * h + (j % 4);
            float v;
            if constexpr (GATEUP) {
                const float rs = rs_lds[tk];
                const float gg = acc[tf][0][j] * rs, uu = acc[tf][1][j] * rs;
                // SiLU with the hardware exponential and reciprocal (relative
                // error ~1e-6, far inside the layer tolerance)
                v = gg * __builtin_amdgcn_rcpf(1.0f + __expf(-gg)) * uu;
            } else {
                v = acc[tf][0][j];
            }
            ot[tk * L::OPITCH + col] = v;
        }
    __syncthreads();
    const uint32_t c_tok = tid / GEMM_WAVES, c_chunk = tid % GEMM_WAVES; // rows 32 c_chunk .. +32
    const uint32_t n = n0 + c_tok;
    if (n < cnt) {
        const float* src = ot + c_tok * L::OPITCH + 32 * c_chunk;
        if constexpr (GATEUP) {
            const uint32_t I = rows_total;
            float v[32];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 f = reinterpret_cast<const float4*>(src)[q];
                v[4 * q] = f.x, v[4 * q + 1] = f.y, v[4 * q + 2] = f.z, v[4 * q + 3] = f.w;
            }
            float sum = 0.0f;
            bool overflow = false;
            uint16_t hv[32], lv[32];
#pragma unroll
            for (int q = 0; q < 32; ++q) {
                // K order inside every 8-row block: c0 c4 c1 c5 c2 c6 c3 c7
                const int cb = (q & ~7) + ((q & 1) ? 4 + ((q & 7) >> 1) : ((q & 7) >> 1));
                const float x = v[cb];
                sum += v[q];
                overflow |= !(fabsf(x) <= 65504.0f);
                const _Float16 hh = (_Float16)x;
                hv[q] = __builtin_bit_cast(uint16_t, hh);
                lv[q] = __builtin_bit_cast(uint16_t, (_Float16)(x - (float)hh));
            }
            if (overflow)
                atomicOr(a.status, ST_F16_RANGE);
            const uint64_t o = (uint64_t)(g0 + n) * I + rb * WG_ROWS + 32 * c_chunk;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint4 hq, lq;
                hq.x = hv[8 * q] | ((uint32_t)hv[8 * q + 1] << 16);
                hq.y = hv[8 * q + 2] | ((uint32_t)hv[8 * q + 3] << 16);
                hq.z = hv[8 * q + 4] | ((uint32_t)hv[8 * q + 5] << 16);
                hq.w = hv[8 * q + 6] | ((uint32_t)hv[8 * q + 7] << 16);
                lq.x = lv[8 * q] | ((uint32_t)lv[8 * q + 1] << 16);
                lq.y = lv[8 * q + 2] | ((uint32_t)lv[8 * q + 3] << 16);
                lq.z = lv[8 * q + 4] | ((uint32_t)lv[8 * q + 5] << 16);
                lq.w = lv[8 * q + 6] | ((uint32_t)lv[8 * q + 7] << 16);
                reinterpret_cast<uint4*>(a.act_hi + o)[q] = hq;
                reinterpret_cast<uint4*>(a.act_lo + o)[q] = lq;
            }
            a.act_sum32[(uint64_t)(g0 + n) * (I / 32) + rb * (WG_ROWS / 32) + c_chunk] = sum;
        } else {
            const uint32_t H = rows_total;
            float* dst = a.y + (uint64_t)(g0 + n) * H + rb * WG_ROWS + 32 * c_chunk;
#pragma unroll
            for (int q = 0; q < 8; ++q)
                reinterpret_cast<float4*>(dst)[q] = reinterpret_cast<const float4*>(src)[q];
        }
    }
}

// ---------------------------------------------------------------------------
// grouped GEMM, 128-token tiles
//
// One workgroup: 128 tokens of one item x WGR weight rows, four waves (one
// per SIMD), two workgroups per CU.  Wave w owns two sets of 32 rows (set
// 0/1 = gate/up rows 32w .. 32w+31 of the block, or down rows 64w + 32m ..
// +32) and all four 32-token fragments: every unpacked code fragment feeds
// four MFMAs (one per token fragment), so the unpack costs a quarter of an
// MFMA's issue time instead of half.  Per quantisation group and (fragment,
// set): a chain of 2KS (x2 with lo) MFMAs into a fresh partial P, then
// acc += s * P (the group scale, in f32).  The activation tile of a group is
// staged by buffer loads straight into LDS ([128 tokens][CH chunks], hi
// only when no row of the tile has a lo part, else hi and lo interleaved;
// chunks of a row in an XOR-swizzled order), NBUF groups resident; the
// codes come two groups ahead into registers.  The bias term runs on the
// matrix cores before the loop.
// ---------------------------------------------------------------------------
constexpr int TOK_L = 128;
constexpr int GL_THREADS = 256;

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane,
// written out so that the compiler does not see an LDS write it cannot tell
// apart from the LDS reads of other staging buffers (it would wait for the
// load before each of them).  The caller waits for completion (vmcnt)
// before the barrier that publishes the buffer.  M0 is written here and
// read by the load only; no compiler-generated code of the kernels that
// call it uses M0.
// Address: a scalar base plus a 32-bit per-lane offset; LDS destination: a
// wave-uniform LDS address (M0).
__device__ __forceinline__ void load_lds16(const uint8_t* sbase, uint32_t voff, uint32_t lds_addr)
{
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_addr)
                 : "memory");
}

// f16 bits to f32 through an explicit conversion: left to itself the
// compiler keeps the group scales packed and runs out of registers
__device__ __forceinline__ float cvt_f16_bits(uint16_t v)
{
    float f;
    asm("v_cvt_f32_f16 %0, %1" : "=v"(f) : "v"((uint32_t)v));
    return f;
}

template <int KS, int WPC>
struct GemmLLds {
    static constexpr int CH_HI = 4 * KS; // 16-byte chunks of a token row per group, hi only
    static constexpr int CH_LO = 8 * KS; // hi and lo interleaved
    static constexpr int TILE_HI = TOK_L * CH_HI * 16;
    static constexpr int TILE_LO = TOK_L * CH_LO * 16;
    static constexpr int NBUF_HI = 4, NBUF_LO = 2; // hi tiles: one quarter each; hi + lo tiles: two
    // gate/up epilogue tile: 4 x [32 tokens][OPITCH] f32, the 32-row chunk
    // c of a token at 36c (a row's four chunk reads by four lanes, and the
    // rows of neighbouring lanes, fall on distinct banks)
    static constexpr int OCH = 36, OPITCH = 4 * OCH;
    // LDS as four separate arrays ("quarters"): a hi tile fills one, a
    // hi + lo tile two (token rows 0-63, 64-127), an epilogue block of 32
    // tokens one.  Being distinct objects, the compiler can tell the reads
    // of one staging buffer from the direct loads into another, and does not
    // wait for those loads before every LDS read.
    static constexpr int QBYTES_ = TILE_HI > TILE_LO / 2 ? TILE_HI : TILE_LO / 2;
    static constexpr int QBYTES = QBYTES_ > 32 * OPITCH * 4 ? QBYTES_ : 32 * OPITCH * 4;
    static_assert(WPC == 2 && KS == 2, "the quarter layout is sized for group 64, two workgroups per CU");
};

template <int SBT, bool GATEUP, int KS, int WPC>
__global__ __launch_bounds__(GL_THREADS, WPC) void q4_gemm_t128_kernel(GemmArgs a)
{
    using L = GemmLLds<KS, WPC>;
    constexpr int NSTEP = 2 * KS;          // 16-column K-steps per quantisation group
    constexpr int WGR = GATEUP ? 128 : 256; // output rows per workgroup
    constexpr int WL = 2 * KS == 8 ? 2 : 1; // load instructions per code fragment
    __shared__ __align__(16) uint8_t q0[L::QBYTES];
    __shared__ __align__(16) uint8_t q1[L::QBYTES];
    __shared__ __align__(16) uint8_t q2[L::QBYTES];
    __shared__ __align__(16) uint8_t q3[L::QBYTES];
    __shared__ uint32_t row_lds[TOK_L];
    __shared__ float rs_lds[TOK_L];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t wvs = __builtin_amdgcn_readfirstlane(wv); // the wave index as a scalar
    auto lds_addr = [](const uint8_t* p) __attribute__((always_inline)) -> uint32_t {
        return (uint32_t)(uintptr_t)p;
    };
    // quarter Q (compile-time, so each access names its array)
    auto quarter = [&](auto q_tag) __attribute__((always_inline)) -> uint8_t* {
        constexpr int Q = decltype(q_tag)::value;
        if constexpr (Q == 0)
            return q0;
        else if constexpr (Q == 1)
            return q1;
        else if constexpr (Q == 2)
            return q2;
        else
            return q3;
    };

    // ---- work item (gemm_unit: tile t on XCD t % 8, its row blocks back to
    //      back there) ----
    const uint32_t rows_total = GATEUP ? a.ex.gate.rows : a.ex.down.rows;
    const uint32_t RB = rows_total / WGR;
    uint32_t tile, rb;
    gemm_unit_of(RB, tile, rb);
    // the tile record: item, first token, the item's first grouped row and
    // token count, expert slot (all ones: the shared expert).  Loaded beside
    // the tile count, not after it (the table holds the grid's tiles rounded
    // up to 8 records, so the read is in bounds for every workgroup; a record
    // past the count is never used)
    const uint4 rec = *reinterpret_cast<const uint4*>(a.tiles + TILE_REC * tile);
    const uint32_t e = a.tiles[TILE_REC * tile + 4];
    const uint32_t ntiles = a.tile_count[0];
    // the record's values in registers before the check (the compiler
    // would otherwise load them after it, a second round trip)
    asm volatile("" ::"s"(rec.y), "s"(rec.z), "s"(rec.w), "s"(e), "s"(ntiles));
    if (tile >= ntiles)
        return;
    const uint32_t n0 = rec.y, g0 = rec.z, cnt = rec.w;
    const bool shared = e == 0xFFFFFFFFu;
    if (shared ? a.has_shared == 0u : e >= a.ex.count) {
        if (tid == 0)
            atomicOr(a.status, ST_ROUTE_RANGE);
        return;
    }
    const uint8_t* const slot = shared ? a.sh.base : a.ex.base + (uint64_t)e * a.ex.stride;
    const ExpertSet& set = shared ? a.sh : a.ex;
    const uint32_t K = a.kdim;
    const uint32_t G = K / (32 * KS), WPR = K / 8;
    auto tok_row = [&](uint32_t n) __attribute__((always_inline)) -> uint32_t {
        return GATEUP ? (shared ? n : a.src_rows[g0 + n]) : g0 + n;
    };
    // the tile's token rows, row scales and lo flags: the three loads first,
    // then their LDS writes (one round trip, not one per load)
    int lo_flag = 0;
    {
        const uint32_t n = n0 + tid;
        const bool v = tid < TOK_L && n < cnt;
        uint32_t r = 0xFFFFFFFFu, lo = 1u;
        float rs = 1.0f;
        if (v) {
            r = tok_row(n);
            if (GATEUP)
                rs = a.rowscale[g0 + n];
            if (a.b_lo_any != nullptr)
                lo = a.b_lo_any[g0 + n];
        }
        if (tid < TOK_L) {
            row_lds[tid] = r;
            if (GATEUP)
                rs_lds[tid] = rs;
            lo_flag = v && lo != 0u;
        }
    }
    const bool tile_lo = __syncthreads_or(lo_flag) != 0;
    const uint32_t first_row = row_lds[0];
    const uint32_t nvalid = cnt - n0 < (uint32_t)TOK_L ? cnt - n0 : (uint32_t)TOK_L;

    // ---- this lane's weight rows: set m, row (lane & 31), lane half h takes
    //      the K-steps' upper 8 columns ----
    const uint32_t n32 = lane & 31, h = lane >> 5;
    uint32_t rowm[2];
    if constexpr (GATEUP) {
        rowm[0] = rowm[1] = rb * WGR + wv * 32 + n32;
    } else {
        rowm[0] = rb * WGR + wv * 64 + n32;
        rowm[1] = rowm[0] + 32;
    }
    const Q4Proj pm0 = GATEUP ? set.gate : set.down;
    const Q4Proj pm1 = GATEUP ? set.up : set.down;
    const rsrc_t wr = make_rsrc(slot, (uint32_t)set.stride);
    const uint32_t w_voff[2] = {(rowm[0] * WPR + h * 2 * KS) * 4, (rowm[1] * WPR + h * 2 * KS) * 4};
    const uint32_t sb_voff[2] = {rowm[0] * G * 2, rowm[1] * G * 2};
    const uint32_t w_soff[2] = {(uint32_t)pm0.w_off, (uint32_t)pm1.w_off};
    const uint32_t s_soff[2] = {(uint32_t)pm0.s_off, (uint32_t)pm1.s_off};
    const uint32_t b_soff[2] = {(uint32_t)pm0.b_off, (uint32_t)pm1.b_off};
    const uint32_t magic = 0x64006400u;
    typedef uint32_t Words[2][2 * KS];
    auto w_load = [&](uint32_t g, Words& w) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
            load_words<2 * KS>(wr, w_voff[m], w_soff[m] + g * 16 * KS, w[m]);
    };
    auto s_load = [&](uint32_t g, uint32_t (&sp)[2]) { // scales of groups g, g + 1 (g even)
#pragma unroll
        for (int m = 0; m < 2; ++m)
            sp[m] = __builtin_amdgcn_raw_buffer_load_b32(wr, sb_voff[m], s_soff[m] + g * 2, 0);
    };
    auto s_of = [&](uint32_t pair, uint32_t g) __attribute__((always_inline)) -> float {
        const uint16_t v = (uint16_t)(pair >> ((g & 1) * 16));
        if constexpr (SBT == 2)
            return __uint_as_float((uint32_t)v << 16);
        else
            return cvt_f16_bits(v);
    };


    // accumulators: set by the bias term (fragments holding tokens) and
    // after the group loop (the others, zero)
    float16_t acc[4][2];

    // ---- bias term on the matrix cores: acc = sum_g b[row][g] * xsum[token][g]
    //      (K' = groups in slices of 16, lane half h: groups k0 + 8h .. +8;
    //      sums split into f16 hi + lo).  Run before the group loop, with the
    //      loop's first loads in flight: acc is the only live state then ----
    // the group sums as f16 hi and lo, [row][hi: GP][lo: GP], zero past G
    // (written by split_rows_kernel for gate/up, by the gate/up epilogue for
    // down), so a slice's 8 groups are one 16-byte load each and a slice
    // past G reads zeros
    const uint32_t GP = (G + 15) / 16 * 16;
    const rsrc_t hl_r = make_rsrc(a.b_sumhl, a.b_rows * GP * 4);
    auto bias_term = [&](auto ntf_tag) __attribute__((always_inline)) {
        constexpr int NTF = decltype(ntf_tag)::value;
        uint32_t rrow[NTF];
#pragma unroll
        for (int tf = 0; tf < NTF; ++tf) {
            const uint32_t brow = row_lds[32 * tf + n32];
            rrow[tf] = brow != 0xFFFFFFFFu ? brow : 0u;
        }
        // slice k00 for fragments T0 .. T1 - 1 (FIRST: k00 = 0, which sets acc)
        auto slice = [&](uint32_t k00, auto first_tag, auto t0_tag, auto t1_tag) __attribute__((always_inline)) {
            constexpr bool FIRST = decltype(first_tag)::value;
            constexpr int T0 = decltype(t0_tag)::value, T1 = decltype(t1_tag)::value;
            const uint32_t gb = k00 + 8 * h;
            uint32_t b2[2][4];
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    b2[m][q] = __builtin_amdgcn_raw_buffer_load_b32(wr, sb_voff[m], b_soff[m] + gb * 2 + 4 * q, 0);
            u32x4 v4[T1 - T0][2]; // hi, lo of groups gb .. gb + 7
#pragma unroll
            for (int tf = T0; tf < T1; ++tf)
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    v4[tf - T0][q] = __builtin_amdgcn_raw_buffer_load_b128(hl_r, rrow[tf] * GP * 4,
                                                                           (q * GP + gb) * 2, 0);
            half8_t bw[2];
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint16_t raw = (uint16_t)(b2[m][j / 2] >> (16 * (j & 1)));
                    float bv;
                    if constexpr (SBT == 2)
                        bv = __uint_as_float((uint32_t)raw << 16);
                    else
                        bv = (float)__builtin_bit_cast(_Float16, raw);
                    bw[m][j] = gb + j < G ? (_Float16)bv : (_Float16)0.0f;
                }
#pragma unroll
            for (int tf = T0; tf < T1; ++tf) {
                // rows past the item read row 0: their outputs are never stored
                const half8_t xh = __builtin_bit_cast(half8_t, v4[tf - T0][0]);
                const half8_t xl = __builtin_bit_cast(half8_t, v4[tf - T0][1]);
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    float16_t c;
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        c[j] = 0.0f;
                    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, bw[m], c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, bw[m], c, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        acc[tf][m][j] = FIRST ? 0.0f + c[j] : acc[tf][m][j] + c[j];
                }
            }
        };
        using F0 = std::integral_constant<int, 0>;
        using FH = std::integral_constant<int, NTF < 2 ? NTF : 2>;
        using FN = std::integral_constant<int, NTF>;
        // the first slice: every fragment's loads at once (acc is not live yet);
        // the others two fragments at a time
        slice(0u, std::true_type{}, F0{}, FN{});
        for (uint32_t k00 = 16; k00 < G; k00 += 16) {
            slice(k00, std::false_type{}, F0{}, FH{});
            if constexpr (NTF > 2)
                slice(k00, std::false_type{}, FH{}, FN{});
        }
    };

    // staging source: b_hi, b_lo at b_hi + lo_delta; 32-bit byte offsets.
    // (Direct-to-LDS loads through a buffer resource measured 4-6x slower
    // than these global ones on this part.)
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(a.b_hi);
    auto run = [&](auto lo_tag, auto ntf_tag) __attribute__((always_inline)) {
        constexpr bool LO = decltype(lo_tag)::value;
        constexpr int NTF = decltype(ntf_tag)::value; // token fragments holding tokens of the item
        constexpr int NHL = LO ? 2 : 1;
        constexpr int CH = LO ? L::CH_LO : L::CH_HI;
        constexpr int NBUF = LO ? L::NBUF_LO : L::NBUF_HI;
        constexpr int PF = NBUF - 1;
        constexpr int DW = TOK_L * CH / 64 / 4; // staging instructions per wave and group
        // chunk c of token row r sits at position c ^ swz(r) of the row, so
        // that the 16 rows one cycle of 16-byte LDS reads serves (64 banks)
        // fall on distinct banks, and any 8 consecutive rows (32 banks); with
        // 8 chunks per row (hi only) r % 8 would repeat after 8 rows
        auto swz = [](uint32_t r) __attribute__((always_inline)) -> uint32_t {
            return LO ? r % CH : (r & 7u) ^ ((r >> 3) & 3u); // period 32: a fragment's rows
        };
        // staging: instruction i of wave wv fills positions 64(wv + 4i) .. +63
        uint32_t st_off[DW];
#pragma unroll
        for (int i = 0; i < DW; ++i) {
            const uint32_t pos = 64 * (wv + 4 * i) + lane;
            const uint32_t r = pos / CH, c = (pos % CH) ^ swz(r);
            const uint32_t rr = row_lds[r];
            const uint32_t trow = rr != 0xFFFFFFFFu ? rr : first_row; // rows past the item: any valid row
            if constexpr (LO)
                st_off[i] = (c & 1) * a.lo_delta + trow * K * 2 + (c >> 1) * 16;
            else
                st_off[i] = trow * K * 2 + c * 16;
        }
        // buffer b: quarter b (hi), quarters 2b, 2b + 1 (hi + lo; instructions
        // 0-3 fill token rows 0-63, 4-7 rows 64-127)
        auto stage = [&](uint32_t g, auto buf_tag) __attribute__((always_inline)) {
            constexpr int BUF = decltype(buf_tag)::value;
            const uint8_t* sb = xbase + g * 64 * KS;
#pragma unroll
            for (int i = 0; i < DW; ++i) {
                uint32_t dst;
                if constexpr (LO)
                    dst = i < DW / 2 ? lds_addr(quarter(std::integral_constant<int, 2 * BUF>{})) + 1024 * (wvs + 4 * i)
                                     : lds_addr(quarter(std::integral_constant<int, 2 * BUF + 1>{})) +
                                           1024 * (wvs + 4 * (i - DW / 2));
                else
                    dst = lds_addr(quarter(std::integral_constant<int, BUF>{})) + 1024 * (wvs + 4 * i);
                load_lds16(sb, st_off[i], dst);
            }
        };
        // fragment reads: row 32tf + n32, chunk (NSTEP h + k) (x2 + hl with lo)
        // at position chunk ^ swz(n32)
        uint32_t rd_off[NSTEP][NHL];
#pragma unroll
        for (int k = 0; k < NSTEP; ++k)
#pragma unroll
            for (int hl = 0; hl < NHL; ++hl) {
                const uint32_t c = LO ? 2 * (h * NSTEP + k) + hl : h * NSTEP + k;
                rd_off[k][hl] = (n32 * CH + (c ^ swz(n32))) * 16;
            }
        Words wA, wB;
        half8_t wf[2][NSTEP];
        uint32_t spa[2], spb[2];
        constexpr bool PIPE = GATEUP && !LO; // the pipelined scaling below
        // chain results (PIPE): the MFMA chain (tf, m) of a group
        // accumulates its products in pp[m], and its scaling acc[tf][m] +=
        // s * pp[m] is issued between the MFMAs of the next chain (tf, 1) or
        // (tf + 1, 0), which write the other one, so that the scale FMAs
        // co-execute with the MFMAs instead of waiting for their own chain
        // (the order of the FMAs per element is unchanged).  The group's
        // last chain (NTF - 1, 1) is scaled during the next group's first
        // chain, with scale s_carry; before the first group pp[1] and
        // s_carry are zero (the first group's carried scaling adds 0).
        float16_t pp[2];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            pp[1][j] = 0.0f;
        float s_carry = 0.0f;
        auto unpack_all = [&](Words& w) __attribute__((always_inline)) {
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int k = 0; k < NSTEP; ++k) {
                    asm volatile("" : "+v"(w[m][k]));
                    wf[m][k] = unpack8(w[m][k], magic);
                }
        };
        // one quantisation group: B = g % NBUF; TAIL: among the last NBUF groups
        auto step = [&](uint32_t g, auto b_tag, auto tail_tag) __attribute__((always_inline)) {
            constexpr int B = decltype(b_tag)::value;
            constexpr bool TAIL = decltype(tail_tag)::value;
            constexpr bool ST = !TAIL || B + PF < NBUF;            // stage group g + PF
            constexpr bool WLD = !TAIL || B + 2 < NBUF;            // codes of group g + 2
            constexpr bool SLD = B % 2 == 0 && WLD;                // scales of groups g + 2, g + 3
            constexpr bool NEXT = !TAIL || B + 1 < NBUF;           // a group g + 1 exists
            // vmcnt at the wait: the loads issued in this step after the
            // staging of group g + 1 and the codes of group g + 1 may stay in
            // flight (PF = 1: the staging of g + 1 is this step's own, issued
            // last; else an earlier step's)
            constexpr int WAIT = PF == 1 ? 0 : (WLD ? 2 * WL : 0) + (SLD ? 2 : 0) + (ST ? DW : 0);
            Words& wcur = B % 2 == 0 ? wA : wB; // codes of group g (unpacked in wf)
            Words& wnext = B % 2 == 0 ? wB : wA;
            // register loads first: the compiler counts only those, so its
            // own waits for them never wait for the staging issued after
            if constexpr (WLD)
                w_load(g + 2, wcur);
            if constexpr (SLD)
                s_load(g + 2, spb);
            if constexpr (ST)
                stage(g + PF, std::integral_constant<int, (B + PF) % NBUF>{});
            float sa[2];
#pragma unroll
            for (int m = 0; m < 2; ++m)
                sa[m] = s_of(spa[m], g);
            // token fragment tf of buffer B
            auto frag = [&](int tf) __attribute__((always_inline)) -> const uint8_t* {
                if constexpr (LO)
                    return tf < 2 ? quarter(std::integral_constant<int, 2 * B>{}) + tf * 32 * CH * 16
                                  : quarter(std::integral_constant<int, 2 * B + 1>{}) + (tf - 2) * 32 * CH * 16;
                else
                    return quarter(std::integral_constant<int, B>{}) + tf * 32 * CH * 16;
            };
#pragma unroll
            for (int tf = 0; tf < NTF; ++tf) {
                if (tf == NTF - 1) {
                    // codes of group g + 1 (loaded a step earlier) and its
                    // staged tile: in place before the last fragment, so the
                    // unpack can run beside its MFMAs
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT) : "memory");
                }
                if constexpr (!PIPE) {
                    // hi + lo: twice the MFMAs per scale FMA, and the
                    // pipelined order below would hold all eight activation
                    // fragments of the token fragment (spills); the down
                    // GEMM measured slower with it.  K-step outer, the two
                    // sets' chains alternating, the scaling after them
                    float16_t qq[2];
#pragma unroll
                    for (int k = 0; k < NSTEP; ++k) {
                        half8_t ax[NHL];
#pragma unroll
                        for (int hl = 0; hl < NHL; ++hl)
                            ax[hl] = *reinterpret_cast<const half8_t*>(frag(tf) + rd_off[k][hl]);
#pragma unroll
                        for (int hl = 0; hl < NHL; ++hl)
#pragma unroll
                            for (int m = 0; m < 2; ++m) {
                                float16_t c;
                                if (k == 0 && hl == 0) {
#pragma unroll
                                    for (int j = 0; j < 16; ++j)
                                        c[j] = 0.0f;
                                } else {
                                    c = qq[m];
                                }
                                qq[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[hl], wf[m][k], c, 0, 0, 0);
                            }
                    }
#pragma unroll
                    for (int m = 0; m < 2; ++m)
#pragma unroll
                        for (int j = 0; j < 16; ++j)
                            acc[tf][m][j] = fmaf(sa[m], qq[m][j], acc[tf][m][j]);
                    continue;
                }
                half8_t ax[NSTEP][NHL];
#pragma unroll
                for (int k = 0; k < NSTEP; ++k)
#pragma unroll
                    for (int hl = 0; hl < NHL; ++hl)
                        ax[k][hl] = *reinterpret_cast<const half8_t*>(frag(tf) + rd_off[k][hl]);
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    // the previous chain: (tf, 0) for m = 1, else (tf - 1, 1),
                    // for tf = 0 the previous group's last
                    const int ptf = m == 1 ? tf : (tf == 0 ? NTF - 1 : tf - 1);
                    const float ps = m == 1 ? sa[0] : (tf == 0 ? s_carry : sa[1]);
                    // each MFMA followed by its share of the previous
                    // chain's scale FMAs, in this order (a scheduling
                    // barrier after each pair: left alone, the compiler
                    // issues the FMAs as one block behind the chain)
                    constexpr int F = 16 / (NSTEP * NHL);
                    const float16_t prev = pp[1 - m];
#pragma unroll
                    for (int k = 0; k < NSTEP; ++k)
#pragma unroll
                        for (int hl = 0; hl < NHL; ++hl) {
                            float16_t c;
                            if (k == 0 && hl == 0) {
#pragma unroll
                                for (int j = 0; j < 16; ++j)
                                    c[j] = 0.0f;
                            } else {
                                c = pp[m];
                            }
                            pp[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[k][hl], wf[m][k], c, 0, 0, 0);
                            const int i = k * NHL + hl;
#pragma unroll
                            for (int j = F * i; j < F * (i + 1); ++j)
                                acc[ptf][1 - m][j] = fmaf(ps, prev[j], acc[ptf][1 - m][j]);
                            __builtin_amdgcn_sched_barrier(0x3F4); // memory and scalar instructions may cross
                        }
                }
            }
            s_carry = sa[1];
            if constexpr (NEXT)
                unpack_all(wnext);
            __syncthreads();
            if constexpr (B % 2 == 1) {
#pragma unroll
                for (int m = 0; m < 2; ++m)
                    spa[m] = spb[m];
            }
        };
        // prologue: the first PF tiles, codes of groups 0 and 1, scales of
        // 0 and 1 (loaded here, not before the token rows' round trip: held
        // through the bias term, the codes were spilled)
        stage(0, std::integral_constant<int, 0>{});
        if constexpr (PF >= 2)
            stage(1, std::integral_constant<int, 1>{});
        if constexpr (PF >= 3)
            stage(2, std::integral_constant<int, 2>{});
        w_load(0, wA);
        w_load(1, wB);
        s_load(0, spa);
        bias_term(ntf_tag); // waits for its loads, and so for the prologue's
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        unpack_all(wA);
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        auto iter = [&](uint32_t g, auto tail_tag) __attribute__((always_inline)) {
            step(g, I0{}, tail_tag);
            step(g + 1, I1{}, tail_tag);
            if constexpr (NBUF == 4) {
                step(g + 2, I2{}, tail_tag);
                step(g + 3, I3{}, tail_tag);
            }
        };
        uint32_t g = 0;
        for (; g + NBUF < G; g += NBUF) // G is a multiple of NBUF
            iter(g, std::false_type{});
        iter(g, std::true_type{});
        if constexpr (PIPE) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                acc[NTF - 1][1][j] = fmaf(s_carry, pp[1][j], acc[NTF - 1][1][j]);
        }
#pragma unroll
        for (int tf = NTF; tf < 4; ++tf)
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    acc[tf][m][j] = 0.0f;
    };
    using T1 = std::integral_constant<int, 1>;
    using T2 = std::integral_constant<int, 2>;
    using T3 = std::integral_constant<int, 3>;
    using T4 = std::integral_constant<int, 4>;
    auto run_lo = [&](auto lo_tag) __attribute__((always_inline)) {
        if (nvalid > 96)
            run(lo_tag, T4{});
        else if (nvalid > 64)
            run(lo_tag, T3{});
        else if (nvalid > 32)
            run(lo_tag, T2{});
        else
            run(lo_tag, T1{});
    };
    if (tile_lo)
        run_lo(std::true_type{});
    else
        run_lo(std::false_type{});
    // the last step waited for every load and met the other waves: the
    // staging buffers are free for the epilogue
    // ---- epilogue ----
    if constexpr (GATEUP) {
        // accumulator element (token 32tf + 8(j/4) + 4h + (j%4), row wv*32 + n32)
        // -> SiLU(g) * u in an f32 tile in LDS -> each thread (token, 32-row
        // chunk) writes act hi/lo in K order and the chunk's sum
        // token block b of the tile: quarter b
        auto ot = [&](uint32_t b) __attribute__((always_inline)) -> float* {
            return reinterpret_cast<float*>(b == 0 ? q0 : b == 1 ? q1 : b == 2 ? q2 : q3);
        };
        const uint32_t col = wv * L::OCH + n32;
#pragma unroll
        for (int tf = 0; tf < 4; ++tf)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t tl = 8 * (j / 4) + 4 * h + (j % 4); // token within fragment tf
                const float rs = rs_lds[32 * tf + tl];
                const float gg = acc[tf][0][j] * rs, uu = acc[tf][1][j] * rs;
                // SiLU with the hardware exponential and reciprocal (relative
                // error ~1e-6, far inside the layer tolerance; __fdividef
                // compiles to the full IEEE division sequence here, about ten
                // instructions)
                ot(tf)[tl * L::OPITCH + col] = gg * __builtin_amdgcn_rcpf(1.0f + __expf(-gg)) * uu;
            }
        __syncthreads();
        const uint32_t I = rows_total;
#pragma unroll
        for (int rep = 0; rep < 2; ++rep) {
            const uint32_t task = tid + 256 * rep; // (token, chunk of 32 rows)
            const uint32_t c_tok = task >> 2, c_chunk = task & 3;
            const uint32_t n = n0 + c_tok;
            if (n >= cnt)
                continue;
            const float* src = ot(c_tok / 32) + (c_tok % 32) * L::OPITCH + L::OCH * c_chunk;
            float v[32];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 f = reinterpret_cast<const float4*>(src)[q];
                v[4 * q] = f.x, v[4 * q + 1] = f.y, v[4 * q + 2] = f.z, v[4 * q + 3] = f.w;
            }
            float sum = 0.0f;
            bool overflow = false;
            uint16_t hv[32], lv[32];
#pragma unroll
            for (int q = 0; q < 32; ++q) {
                // K order inside every 8-row block: c0 c4 c1 c5 c2 c6 c3 c7
                const int cb = (q & ~7) + ((q & 1) ? 4 + ((q & 7) >> 1) : ((q & 7) >> 1));
                const float x = v[cb];
                sum += v[q];
                overflow |= !(fabsf(x) <= 65504.0f);
                const _Float16 hh = (_Float16)x;
                hv[q] = __builtin_bit_cast(uint16_t, hh);
                lv[q] = __builtin_bit_cast(uint16_t, (_Float16)(x - (float)hh));
            }
            if (overflow)
                atomicOr(a.status, ST_F16_RANGE);
            const uint64_t o = (uint64_t)(g0 + n) * I + rb * WGR + 32 * c_chunk;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint4 hq, lq;
                hq.x = hv[8 * q] | ((uint32_t)hv[8 * q + 1] << 16);
                hq.y = hv[8 * q + 2] | ((uint32_t)hv[8 * q + 3] << 16);
                hq.z = hv[8 * q + 4] | ((uint32_t)hv[8 * q + 5] << 16);
                hq.w = hv[8 * q + 6] | ((uint32_t)hv[8 * q + 7] << 16);
                lq.x = lv[8 * q] | ((uint32_t)lv[8 * q + 1] << 16);
                lq.y = lv[8 * q + 2] | ((uint32_t)lv[8 * q + 3] << 16);
                lq.z = lv[8 * q + 4] | ((uint32_t)lv[8 * q + 5] << 16);
                lq.w = lv[8 * q + 6] | ((uint32_t)lv[8 * q + 7] << 16);
                reinterpret_cast<uint4*>(a.act_hi + o)[q] = hq;
                reinterpret_cast<uint4*>(a.act_lo + o)[q] = lq;
            }
            // the down GEMM's bias-term operand: the group sum (this chunk
            // and its pair on the neighbouring lane) as f16 hi + lo, in
            // range like the activations; zeros for the groups past I/64
            const float gsum = sum + __shfl_xor(sum, 1);
            if (!(fabsf(gsum) <= 65504.0f))
                atomicOr(a.status, ST_F16_RANGE);
            const uint32_t GI = I / 64, GPI = (GI + 15) / 16 * 16;
            uint16_t* const hl = a.act_sumhl + (uint64_t)(g0 + n) * 2 * GPI;
            if ((c_chunk & 1) == 0) {
                const uint32_t gi = rb * (WGR / 64) + c_chunk / 2;
                const _Float16 gh = (_Float16)gsum;
                hl[gi] = __builtin_bit_cast(uint16_t, gh);
                hl[GPI + gi] = __builtin_bit_cast(uint16_t, (_Float16)(gsum - (float)gh));
            }
            if (rb == RB - 1 && c_chunk == 0)
                for (uint32_t gi = GI; gi < GPI; ++gi)
                    hl[gi] = 0, hl[GPI + gi] = 0;
        }
    } else {
        // y [grouped row][H] f32: each wave turns its 64 rows of one 32-token
        // fragment around in its own staging quarter ([token][YP floats]),
        // then stores 16 bytes per lane, 256 contiguous bytes per token row
        // (4-byte stores straight from the accumulators took four times the
        // store instructions).  A wave reads back only what it wrote, in
        // order, so no barrier is needed.
        constexpr int YP = 72; // 64 rows + 8: the two lane halves' rows land on distinct banks
        const uint32_t H = rows_total;
        float* const tb = reinterpret_cast<float*>(wv == 0 ? q0 : wv == 1 ? q1 : wv == 2 ? q2 : q3);
        float* const yb = a.y + rb * WGR + wv * 64;
#pragma unroll
        for (int tf = 0; tf < 4; ++tf) {
            if (n0 + 32 * tf >= cnt)
                break;
#pragma unroll
            for (int j = 0; j < 16; ++j)
#pragma unroll
                for (int m = 0; m < 2; ++m)
                    tb[(8 * (j / 4) + 4 * h + (j % 4)) * YP + 32 * m + n32] = acc[tf][m][j];
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const uint32_t idx = 64 * it + lane, t = idx >> 4, c = idx & 15;
                const uint32_t tk = n0 + 32 * tf + t;
                if (tk < cnt)
                    *reinterpret_cast<float4*>(yb + (uint64_t)(g0 + tk) * H + 4 * c) =
                        *reinterpret_cast<const float4*>(tb + t * YP + 4 * c);
            }
        }
    }
}

// shared-expert gate logit per token: one wave per token, f32 accumulation
template <int WDT>
__global__ __launch_bounds__(256) void gate_row_kernel(const void* __restrict__ w, const float* __restrict__ x,
                                                      uint32_t tokens, uint32_t hidden, float* __restrict__ out)
{
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= tokens)
        return;
    const float* xr = x + (uint64_t)t * hidden;
    float acc = 0.0f;
    for (uint32_t c = lane; c < hidden; c += 64) {
        float wv;
        if constexpr (WDT == 0)
            wv = reinterpret_cast<const float*>(w)[c];
        else
            wv = sb_at<WDT>(reinterpret_cast<const uint8_t*>(w), c);
        acc = fmaf(wv, xr[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0)
        out[t] = acc;
}

// the same for a Q4 gate row [1][hidden]: lane l takes the 32-column chunks
// l + 64 c, s . sum(q x) + b . sum(x) per chunk
template <int SBT>
__global__ __launch_bounds__(256) void gate_row_q4_kernel(Q4Rows m, const float* __restrict__ x, uint32_t tokens,
                                                         uint32_t hidden, float* __restrict__ out)
{
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= tokens)
        return;
    const float* xr = x + (uint64_t)t * hidden;
    const uint4* wp = reinterpret_cast<const uint4*>(m.codes);
    float acc = 0.0f;
    for (uint32_t ch = lane; ch < hidden / 32; ch += 64) {
        const uint32_t gi = (ch * 32u) >> m.gshift;
        float xs;
        const float qx = q4_chunk_qx(wp[ch], xr + ch * 32u, xs);
        acc = fmaf(sb_at<SBT>(m.scales, gi), qx, fmaf(sb_at<SBT>(m.biases, gi), xs, acc));
    }
    acc = wave_sum(acc);
    if (lane == 0)
        out[t] = acc;
}

// h[t][c] = (r + sum_k w[t,k] y[out_idx[t,k]][c]) + sw_t * S[t][c], then
// the optional next-layer RMSNorm.  One workgroup per token.
__global__ __launch_bounds__(256) void prefill_combine_kernel(
    const float* __restrict__ y, const float* __restrict__ ysh, const float* __restrict__ shared_logit,
    uint32_t has_shared, const uint32_t* __restrict__ out_idx, const float* __restrict__ weights,
    const float* __restrict__ residual, uint32_t k, uint32_t hidden, float* __restrict__ out,
    const float* __restrict__ norm_w, float eps, float* __restrict__ normed)
{
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    float sw = 0.0f;
    if (has_shared)
        sw = sigmoidf_(shared_logit ? shared_logit[t] : 80.0f);
    float ss = 0.0f;
    for (uint32_t c = threadIdx.x * 4; c < hidden; c += 1024) {
        float4 moe = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t kk = 0; kk < k; ++kk) {
            const uint32_t route = t * k + kk;
            const uint32_t gi = out_idx[route];
            if (gi == 0xFFFFFFFFu)
                continue;
            const float w = weights[route];
            const float4 v = *reinterpret_cast<const float4*>(y + (uint64_t)gi * hidden + c);
            moe.x = moe.x + w * v.x;
            moe.y = moe.y + w * v.y;
            moe.z = moe.z + w * v.z;
            moe.w = moe.w + w * v.w;
        }
        const uint64_t o = (uint64_t)t * hidden + c;
        const float4 r = *reinterpret_cast<const float4*>(residual + o);
        float4 h = make_float4(r.x + moe.x, r.y + moe.y, r.z + moe.z, r.w + moe.w);
        if (has_shared) {
            const float4 s = *reinterpret_cast<const float4*>(ysh + o);
            h.x = h.x + sw * s.x;
            h.y = h.y + sw * s.y;
            h.z = h.z + sw * s.z;
            h.w = h.w + sw * s.w;
        }
        *reinterpret_cast<float4*>(out + o) = h;
        ss += h.x * h.x + h.y * h.y + h.z * h.z + h.w * h.w;
    }
    if (!norm_w)
        return;
    ss = wave_sum(ss);
    if (lane == 0)
        red[wv] = ss;
    __syncthreads();
    const float ms = ((red[0] + red[1]) + (red[2] + red[3])) / (float)hidden;
    const float scale = 1.0f / sqrtf(ms + eps);
    for (uint32_t c = threadIdx.x * 4; c < hidden; c += 1024) {
        const uint64_t o = (uint64_t)t * hidden + c;
        const float4 h = *reinterpret_cast<const float4*>(out + o);
        const float4 w = *reinterpret_cast<const float4*>(norm_w + c);
        *reinterpret_cast<float4*>(normed + o) =
            make_float4(h.x * scale * w.x, h.y * scale * w.y, h.z * scale * w.z, h.w * scale * w.w);
    }
}

static uint32_t max_tiles_of(uint32_t tok, uint32_t tokens, uint32_t k, uint32_t experts, bool has_shared)
{
    const uint32_t routes = tokens * k;
    return routes / tok + std::min(experts, routes) + (has_shared ? (tokens + tok - 1) / tok : 0u) + 1;
}

uint32_t prefill_max_tiles(uint32_t tokens, uint32_t k, uint32_t experts, bool has_shared)
{
    return max_tiles_of(TOK, tokens, k, experts, has_shared); // the larger count: 64-token tiles
}

// The 128-token kernels take group 64, rows in blocks of 256 (down) and
// operand buffers addressed with 32-bit offsets; PBMOE_PREFILL_TILE=64 in
// the environment keeps the 64-token kernels (for comparison).
static bool use_t128(const PrefillArgs& p, uint32_t routes)
{
    static const bool forced64 = [] {
        const char* v = std::getenv("PBMOE_PREFILL_TILE");
        return v && std::strcmp(v, "64") == 0;
    }();
    const uint64_t I = p.ex.gate.rows, H = p.hidden, T = p.tokens;
    const uint64_t x_bytes = (uint64_t)((const uint8_t*)p.x_lo - (const uint8_t*)p.x_hi) + T * H * 2;
    const uint64_t a_bytes = (uint64_t)((const uint8_t*)p.act_lo - (const uint8_t*)p.act_hi) + (routes + T) * I * 2;
    return !forced64 && p.ex.group == 64 && H % 256 == 0 && I % 128 == 0 && p.x_lo > p.x_hi &&
           p.act_lo > p.act_hi && x_bytes < (1ull << 32) && a_bytes < (1ull << 32);
}

// start/stop events of kernel i/2 (gate/up GEMM, down GEMM, combine) when
// the caller asked for per-kernel timing; attached to the dispatch packets
static inline hipEvent_t phase_event(const PrefillArgs& p, int i)
{
    return p.phase_timing ? p.phase_ev[i] : nullptr;
}

// 8 x ceil(work / 8) workgroups for the XCD-split work list (see the kernel)
static dim3 grid_of(uint32_t max_tiles, uint32_t row_blocks)
{
    return dim3((uint32_t)(8 * (uint64_t)row_blocks * ((max_tiles + 7) / 8)));
}

static dim3 gemm_grid(uint32_t max_tiles, uint32_t rows)
{
    return grid_of(max_tiles, rows / WG_ROWS);
}

// the 128-token kernels (group 64: KS = 2), two workgroups per CU
template <int SBT, bool GATEUP>
static void launch_gemm_t128(hipStream_t st, dim3 grid, hipEvent_t e0, hipEvent_t e1, const GemmArgs& a)
{
    hipExtLaunchKernelGGL((q4_gemm_t128_kernel<SBT, GATEUP, 2, 2>), grid, dim3(GL_THREADS), 0, st, e0, e1, 0, a);
}

template <int SBT, int KS>
static hipError_t launch_prefill_typed(hipStream_t st, const PrefillArgs& p)
{
    const ExpertSet& ex = p.ex;
    const uint32_t T = p.tokens, K = p.k, H = p.hidden, I = ex.gate.rows;
    const uint32_t routes = T * K;
    const uint32_t has_shared = p.shared ? 1u : 0u;
    hipError_t err = launch_dispatch_plan(st, p.ids, routes, ex.count, K, p.plan, p.status);
    if (err != hipSuccess)
        return err;
    const bool t128 = KS == 2 && use_t128(p, routes);
    const TileArgs ta{p.plan.unique_count, p.plan.groups, p.plan.unique_ids, has_shared, T, routes, p.tiles,
                      p.tile_count, t128 ? (uint32_t)TOK_L : (uint32_t)TOK};
    split_rows_kernel<<<T + 1, 256, 0, st>>>(p.x, H, p.x_hi, p.x_lo, p.x_sum32, t128 ? p.x_sumhl : nullptr,
                                             (uint32_t)KS, p.rowscale, p.x_lo_any, p.plan.out_idx, K, ta);
    if ((err = hipGetLastError()) != hipSuccess)
        return err;
    if (has_shared && p.sgate_w) {
        const dim3 gg((T + 3) / 4);
        if (p.sgate_dtype == DT_Q4 && ex.sb_dtype == 2)
            gate_row_q4_kernel<2><<<gg, 256, 0, st>>>(p.sgate_q4, p.x, T, H, p.shared_logit);
        else if (p.sgate_dtype == DT_Q4)
            gate_row_q4_kernel<1><<<gg, 256, 0, st>>>(p.sgate_q4, p.x, T, H, p.shared_logit);
        else if (p.sgate_dtype == 0)
            gate_row_kernel<0><<<gg, 256, 0, st>>>(p.sgate_w, p.x, T, H, p.shared_logit);
        else if (p.sgate_dtype == 2)
            gate_row_kernel<2><<<gg, 256, 0, st>>>(p.sgate_w, p.x, T, H, p.shared_logit);
        else
            gate_row_kernel<1><<<gg, 256, 0, st>>>(p.sgate_w, p.x, T, H, p.shared_logit);
        if ((err = hipGetLastError()) != hipSuccess)
            return err;
    }
    GemmArgs a{};
    a.ex = ex;
    a.has_shared = has_shared;
    if (has_shared)
        a.sh = *p.shared;
    a.unique_ids = p.plan.unique_ids;
    a.unique_count = p.plan.unique_count;
    a.groups = p.plan.groups;
    a.src_rows = p.plan.src_rows;
    a.tiles = p.tiles;
    a.tile_count = p.tile_count;
    a.routes = routes;
    a.tokens = T;
    a.status = p.status;
    const uint32_t max_tiles = prefill_max_tiles(T, K, ex.count, has_shared != 0);
    a.b_hi = p.x_hi;
    a.b_lo = p.x_lo;
    a.b_sum32 = p.x_sum32;
    a.b_sumhl = p.x_sumhl;
    a.rowscale = p.rowscale;
    a.b_lo_any = p.x_lo_any;
    a.kdim = H;
    a.b_rows = T;
    a.act_hi = p.act_hi;
    a.act_lo = p.act_lo;
    a.act_sum32 = p.act_sum32;
    a.act_sumhl = p.act_sumhl;
    a.lo_delta = (uint32_t)((const uint8_t*)p.x_lo - (const uint8_t*)p.x_hi);
    const uint32_t tiles128 = max_tiles_of(TOK_L, T, K, ex.count, has_shared != 0);
    if (t128)
        launch_gemm_t128<SBT, true>(st, grid_of(tiles128, I / 128), phase_event(p, 0), phase_event(p, 1), a);
    else
        hipExtLaunchKernelGGL((q4_group_gemm_kernel<SBT, true, KS>), gemm_grid(max_tiles, I), dim3(GEMM_THREADS), 0,
                              st, phase_event(p, 0), phase_event(p, 1), 0, a);
    if ((err = hipGetLastError()) != hipSuccess)
        return err;
    a.b_hi = p.act_hi;
    a.b_lo = p.act_lo;
    a.b_sum32 = p.act_sum32;
    a.b_sumhl = p.act_sumhl;
    a.rowscale = nullptr;
    a.b_lo_any = nullptr;
    a.kdim = I;
    a.b_rows = routes + T;
    a.y = p.y;
    a.lo_delta = (uint32_t)((const uint8_t*)p.act_lo - (const uint8_t*)p.act_hi);
    if (t128)
        launch_gemm_t128<SBT, false>(st, grid_of(tiles128, H / 256), phase_event(p, 2), phase_event(p, 3), a);
    else
        hipExtLaunchKernelGGL((q4_group_gemm_kernel<SBT, false, KS>), gemm_grid(max_tiles, H), dim3(GEMM_THREADS), 0,
                              st, phase_event(p, 2), phase_event(p, 3), 0, a);
    if ((err = hipGetLastError()) != hipSuccess)
        return err;
    hipExtLaunchKernelGGL(prefill_combine_kernel, dim3(T), dim3(256), 0, st, phase_event(p, 4), phase_event(p, 5), 0,
                          (const float*)p.y, (const float*)(p.y + (uint64_t)routes * H),
                          (const float*)(p.sgate_w ? p.shared_logit : nullptr), has_shared,
                          (const uint32_t*)p.plan.out_idx, p.weights, p.residual, K, H, p.hidden_out,
                          p.next_norm_w, p.eps, p.next_normed);
    return hipGetLastError();
}

template <int SBT>
static hipError_t launch_prefill_sb(hipStream_t st, const PrefillArgs& p)
{
    switch (p.ex.group) {
    case 32:
        return launch_prefill_typed<SBT, 1>(st, p);
    case 64:
        return launch_prefill_typed<SBT, 2>(st, p);
    case 128:
        return launch_prefill_typed<SBT, 4>(st, p);
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_prefill(hipStream_t st, const PrefillArgs& p)
{
    // shapes the kernels assume: WG_ROWS-row blocks of H and I, a multiple
    // of NBUF quantisation groups along both (the group loop is unrolled by
    // the number of staging buffers; 256 columns in every case), group =
    // 2^shift, a shared expert in the routed experts' format
    const uint32_t kmul = p.ex.group * (p.ex.group >= 128 ? 2u : 4u);
    if ((1u << p.ex.group_shift) != p.ex.group || p.hidden % WG_ROWS || p.ex.gate.rows % WG_ROWS ||
        p.hidden % kmul || p.ex.gate.rows % kmul ||
        p.ex.gate.cols != p.hidden || p.ex.down.rows != p.hidden)
        return hipErrorInvalidValue;
    if (p.shared && (p.shared->group != p.ex.group || p.shared->sb_dtype != p.ex.sb_dtype ||
                     p.shared->gate.rows != p.ex.gate.rows || p.shared->down.rows != p.hidden))
        return hipErrorInvalidValue;
    if (p.ex.sb_dtype == 2)
        return launch_prefill_sb<2>(st, p);
    return launch_prefill_sb<1>(st, p);
}

} // namespace pbmoe
