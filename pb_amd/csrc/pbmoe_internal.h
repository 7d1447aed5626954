// Internal interface between the C ABI (pbmoe_abi.cpp) and the gfx950
// kernels (pbmoe_kernels.hip).  Not part of the public boundary.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pbmoe {

// Device status bits, OR-ed by kernels and mapped to pbmoe_status by
// pbmoe_sync().
enum : uint32_t {
    ST_ROUTE_RANGE = 1u << 0,  // route id >= experts: route skipped
    ST_NONFINITE = 1u << 1,    // non-finite router logit
    ST_BAD_SUM = 1u << 2,      // renormalisation sum not positive/finite
    ST_NEGATIVE = 1u << 3,     // negative selected probability
    ST_PLAN_OVERFLOW = 1u << 4, // more routes than the plan buffers hold
    ST_F16_RANGE = 1u << 5      // prefill activation outside the f16 operand range
};

// One projection inside a fixed expert slot.
struct Q4Proj {
    uint64_t w_off, s_off, b_off; // component byte offsets in the slot
    uint32_t rows, cols;
};

// A set of fixed Q4 slots (a bound layer, or the one shared expert).
struct ExpertSet {
    const uint8_t* base; // slot 0
    uint64_t stride;     // expert_bytes
    uint32_t count;      // number of slots
    uint32_t group;      // quantisation group size (32, 64 or 128)
    uint32_t group_shift; // log2(group)
    uint32_t sb_dtype;   // 1 = f16, 2 = bf16
    Q4Proj gate, up, down;
};

// A resident Q4 projection [rows][cols] given as separate arrays: codes
// rows*cols/2 bytes, 2-byte scale and bias [rows][cols >> gshift] (their
// dtype is the layer's scale/bias dtype).  Used for a Q4 router and a Q4
// shared-expert gate row (dtype code DT_Q4).
struct Q4Rows {
    const uint8_t* codes;
    const uint8_t* scales;
    const uint8_t* biases;
    uint32_t gshift;
};
constexpr uint32_t DT_Q4 = 3; // weight dtype code beside 0 f32, 1 f16, 2 bf16

// Routing parameters for the routing kernel.
struct RouteParams {
    uint32_t experts, k, kind, order, norm, n_group, topk_group;
    float routed_scale;
};

// One token routed by a whole workgroup (route_token_block) rather than one
// wave (route_token_wave): decode token counts, canonical order, no expert
// groups.  Every entry point that routes decode tokens uses this choice, so
// that they agree bitwise on the route weights.
__host__ __device__ inline bool block_routing(uint32_t tokens, const RouteParams& p)
{
    return tokens <= 16 && p.order == 0 && !(p.kind == 2 && p.n_group > 1);
}

// Dispatch plan buffers (device), layout documented in pbmoe.h.
struct Plan {
    uint32_t* unique_ids;  // [experts]
    uint32_t* unique_count;// [1]
    uint32_t* route_slots; // [routes]
    uint32_t* src_rows;    // [routes]
    uint32_t* out_idx;     // [routes]
    uint32_t* groups;      // [experts][2]
    uint32_t* work;        // multi-workgroup scratch (plan_work_words), or null
};

// w_dtype DT_Q4: the router is `q4` (scale/bias dtype sb_dtype), w unused
hipError_t launch_router_logits(hipStream_t s, const void* w, uint32_t w_dtype, const float* x,
                                uint32_t tokens, uint32_t experts, uint32_t hidden, float* logits,
                                const Q4Rows* q4 = nullptr, uint32_t sb_dtype = 1);
hipError_t launch_route_topk(hipStream_t s, const float* logits, const float* bias, uint32_t tokens,
                             const RouteParams& p, uint32_t* ids, float* weights,
                             uint32_t* status);
// words of Plan::work needed for the multi-workgroup plan of `routes`
uint32_t plan_work_words(uint32_t routes, uint32_t experts);
hipError_t launch_dispatch_plan(hipStream_t s, const uint32_t* ids, uint32_t routes,
                                uint32_t experts, uint32_t k, const Plan& plan,
                                uint32_t* status);
// Decode path (tokens <= 16).  Modes: the full layer (router + routing +
// experts), the expert phase for given routes, or routing only.
enum : uint32_t { DECODE_FULL_LAYER = 0, DECODE_EXPERTS = 1, DECODE_ROUTE_ONLY = 2 };

struct DecodeArgs {
    const void* router_w;      // null: route from the given logits
    uint32_t router_dtype;     // 0 f32, 1 f16, 2 bf16, DT_Q4 (router_q4)
    Q4Rows router_q4;
    const float* sel_bias;     // [E] for sigmoid routing
    RouteParams rp;
    float* logits;             // [T][E]
    uint32_t* ids;             // [T][K]
    float* weights;            // [T][K]
    ExpertSet ex;              // routed experts
    const ExpertSet* shared;   // host pointer, null without a shared expert
    const void* sgate_w;       // shared gate row [H], null: sigma = 1
    uint32_t sgate_dtype;      // as router_dtype (DT_Q4: sgate_q4)
    Q4Rows sgate_q4;
    const float* x;            // [T][H] (the hidden state when in_norm_w is set)
    const float* in_norm_w;    // null, or input RMSNorm weight [H] (full layer only)
    float* x_normed;           // [T][H] scratch: RMSNorm(x) * in_norm_w
    const float* residual;     // [T][H]
    uint32_t tokens, hidden;
    float* act;                // [T*K][I]
    float* act_shared;         // [T][Is]
    float* shared_weight;      // [T]
    float* hidden_out;         // [T][H]
    const float* next_norm_w;  // [H] or null
    float eps;
    float* next_normed;        // [T][H] or null
    Plan plan;                 // scratch plan (tokens > 1)
    uint32_t* ticket;          // zeroed counter for last-workgroup election
    hipEvent_t phase_ev[6];    // start/stop per kernel when phase_timing
    bool phase_timing;
    uint32_t* status;
};

hipError_t launch_decode_layer(hipStream_t s, const DecodeArgs& d, uint32_t mode);

// Static scratch of the allocation-free decode entry point: a file-scope
// device array in pbmoe_decode.hip.  static_scratch_init looks up its address
// on `device` (which must be current) once; static_scratch returns it (null
// before init) and its size.
hipError_t static_scratch_init(int device);
void* static_scratch(int device, size_t* bytes);
// Prefill path (grouped GEMM on the matrix cores, any token count).
struct PrefillArgs {
    ExpertSet ex;              // routed experts
    const ExpertSet* shared;   // host pointer, null without a shared expert
    const void* sgate_w;       // shared gate row [H], null: sigma(80) = 1
    uint32_t sgate_dtype;      // 0 f32, 1 f16, 2 bf16, DT_Q4 (sgate_q4)
    Q4Rows sgate_q4;
    const uint32_t* ids;       // [T][K]
    const float* weights;      // [T][K]
    const float* x;            // [T][H]
    const float* residual;     // [T][H]
    uint32_t tokens, k, hidden;
    float* hidden_out;         // [T][H]
    const float* next_norm_w;  // [H] or null
    float eps;
    float* next_normed;        // [T][H] or null
    Plan plan;                 // [routes] plan scratch
    // scratch (sizes from prefill_scratch_bytes)
    uint32_t* tiles;           // [max_tiles][8] tile records
    uint32_t* tile_count;      // [1]
    uint16_t* x_hi;            // [T][H] f16
    uint16_t* x_lo;            // [T][H] f16
    float* x_sum32;            // [T][H/32]
    uint16_t* x_sumhl;         // [T][2][GP] f16 group sums hi, lo (GP = H/64 rounded up to 16)
    float* rowscale;           // [T*K + T] per grouped row: its token's x scale
    uint32_t* x_lo_any;        // [T*K + T] per grouped row: nonzero when its token's lo part is not all zero
    float* shared_logit;       // [T]
    uint16_t* act_hi;          // [T*K + T][I] f16
    uint16_t* act_lo;          // [T*K + T][I] f16
    float* act_sum32;          // [T*K + T][I/32]
    uint16_t* act_sumhl;       // [T*K + T][2][GP] f16 group sums hi, lo (GP = I/64 rounded up to 16)
    float* y;                  // [T*K + T][H]
    uint32_t* status;
    hipEvent_t phase_ev[6];    // start/stop of gate/up, down, combine
    bool phase_timing;
};

uint32_t prefill_max_tiles(uint32_t tokens, uint32_t k, uint32_t experts, bool has_shared);
// items (used experts + the shared expert) the prefill tile table holds
constexpr uint32_t TILE_TABLE_MAX_ITEMS = 1280;
hipError_t launch_prefill(hipStream_t s, const PrefillArgs& p);

hipError_t launch_q4_dequantize(hipStream_t s, const uint8_t* packed, const void* scales,
                                const void* biases, uint32_t sb_dtype, uint32_t rows,
                                uint32_t cols, uint32_t group, float* out);
hipError_t launch_synth_fill(hipStream_t s, uint8_t* slots, uint64_t stride,
                             const uint64_t* offsets9, uint32_t hidden, uint32_t intermediate,
                             uint32_t group, uint32_t sb_dtype, uint64_t seed, uint32_t tensor,
                             uint32_t layer, uint32_t first_expert, uint32_t count);
hipError_t launch_synth_center(hipStream_t s, uint8_t* slots, uint64_t stride, const uint64_t* offsets9,
                               uint32_t hidden, uint32_t intermediate, uint32_t group, uint32_t sb_dtype,
                               uint32_t count);
hipError_t launch_fill_u32(hipStream_t s, uint32_t* p, uint32_t value, uint64_t n);
// XOR of every 32-bit word of src[0, bytes) into *out (bytes a multiple of 16)
hipError_t launch_stream_read(hipStream_t s, const void* src, uint64_t bytes, uint32_t* out);

// One resident Q4 matrix [rows][cols] (codes, 2-byte scale and bias rows).
struct Q4Mat {
    const uint8_t* codes;
    const uint8_t* scales;
    const uint8_t* biases;
    uint32_t rows, cols;
};

// Batch-1 decode attention of one layer (pbmoe_attention_decode).
struct AttnArgs {
    Q4Mat q, k, v, o;
    const float* q_norm; // [head_dim]
    const float* k_norm; // [head_dim]
    uint32_t group_shift, sb_dtype;
    uint32_t hidden, q_heads, kv_heads, head_dim;
    const float* inv_freq; // [head_dim / 2] rotary inverse frequencies (f32, host-computed)
    uint16_t* cache_k;     // [max_context][kv_heads][head_dim] f16
    uint16_t* cache_v;
    uint32_t position;
    const float* normed;   // [H]: the normalised input, or the hidden state when in_norm_w is set
    const float* in_norm_w; // null, or the input RMSNorm weight [H] (normalised inside)
    const float* residual; // [H]
    float* hidden_out;     // [H]
    const float* post_norm_w; // null: no post-attention norm
    float post_eps;
    float* post_normed;    // [H]
    float* attn_out;       // [q_heads * head_dim] (scratch or the caller's buffer)
    // scratch
    float* qkv;            // [(q_heads + 2 kv_heads) * head_dim]
    float* part;           // [q_heads][chunks][head_dim + 2]
    // start/stop events of q/k/v, chunk partials, merge, o_proj (all null:
    // untimed)
    hipEvent_t ev[8];
};

constexpr uint32_t ATTN_CHUNK = 64; // positions per attention workgroup
hipError_t launch_attention_decode(hipStream_t s, const AttnArgs& a);

} // namespace pbmoe
