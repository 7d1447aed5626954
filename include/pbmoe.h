/*
 * pbmoe.h — C ABI of the MI355X (gfx950) MoE block for pb's FlashMoE runtime.
 *
 * This is the drop-in boundary: a Rust `extern "C"` crate (or any FFI) binds
 * exactly these symbols.  Signatures use plain pointers and sizes only.
 * Every entry point returns a pbmoe_status; pbmoe_last_error() returns a
 * thread-local description of the last failure.  Nothing falls back to a
 * different implementation: an unsupported shape or dtype is an explicit
 * PBMOE_ERR_UNSUPPORTED, mirroring the reference's "explicit unsupported
 * capability, never a fallback" rule.
 *
 * Reference interfaces replaced (paths relative to
 * src/inference/flashmoe/ of Jc2k/pb):
 *   MetalExecutionFacade                       runtime/mod.rs:648-1410
 *   router prep + CPU top-k                    metal/mod.rs:2864-3036,
 *                                              math.rs:746-819
 *   route renormalisation                      scheduler/expert_access.rs:80-135
 *   submit_scheduled_expert_command (CMD3)     runtime/mod.rs:922-961,
 *                                              metal/mod.rs:3252-3332
 *   qwen_layer_major_experts (prefill)         runtime/mod.rs:1151-1161,
 *                                              metal/mod.rs:3334-3393
 *   resolve_layer_major_experts + group plan   scheduler/mod.rs:685-769,
 *                                              metal/mod.rs:3197-3233
 *   prepare_resident_expert_backing            metal/mod.rs:1382-1402
 *   QwenMoeQ4ExpertLayout::fixed_bf16          model_family.rs:954-1068
 *
 * Memory: activation, route and output pointers are DEVICE pointers (HBM)
 * unless an argument says otherwise; pbmoe_device_alloc/upload/download
 * give FFI callers without a HIP binding a way to own them.  Weight bind
 * calls accept host or device sources (flags) and keep a device copy or a
 * reference for the lifetime of the binding.
 *
 * Threading: one HIP stream per context; a context is not re-entrant.
 * Launches are asynchronous; pbmoe_sync() waits and reports deferred device
 * errors (for example a route id outside the expert count).
 */
#ifndef PBMOE_H
#define PBMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PBMOE_ABI_VERSION 1

typedef enum pbmoe_status {
    PBMOE_OK = 0,
    PBMOE_ERR_INVALID_ARGUMENT = 1, /* null pointer, zero size, bad enum      */
    PBMOE_ERR_SHAPE = 2,            /* dimensions disagree with the binding   */
    PBMOE_ERR_DTYPE = 3,            /* dtype not accepted for this tensor     */
    PBMOE_ERR_ALIGNMENT = 4,        /* offsets/pointers not 4-byte aligned    */
    PBMOE_ERR_ROUTE = 5,            /* route out of range, duplicate, bad sum */
    PBMOE_ERR_UNSUPPORTED = 6,      /* declared capability not implemented    */
    PBMOE_ERR_DEVICE = 7,           /* HIP runtime failure                    */
    PBMOE_ERR_TIMEOUT = 8,          /* device wait exceeded its limit         */
    PBMOE_ERR_NOT_BOUND = 9,        /* layer / router / shared not bound      */
    PBMOE_ERR_OUT_OF_MEMORY = 10,
    PBMOE_ERR_NONFINITE = 11,       /* non-finite router score or weight      */
    PBMOE_ERR_IO = 12,              /* expert pack file missing or unreadable */
    PBMOE_ERR_FORMAT = 13           /* expert pack metadata malformed         */
} pbmoe_status;

typedef enum pbmoe_dtype {
    PBMOE_DTYPE_F32 = 0,
    PBMOE_DTYPE_F16 = 1,
    PBMOE_DTYPE_BF16 = 2
} pbmoe_dtype;

/* Expert slot components, in slot order (model_family.rs:818-843). */
typedef enum pbmoe_component_kind {
    PBMOE_GATE_WEIGHT = 0,
    PBMOE_GATE_SCALE = 1,
    PBMOE_GATE_BIAS = 2,
    PBMOE_UP_WEIGHT = 3,
    PBMOE_UP_SCALE = 4,
    PBMOE_UP_BIAS = 5,
    PBMOE_DOWN_WEIGHT = 6,
    PBMOE_DOWN_SCALE = 7,
    PBMOE_DOWN_BIAS = 8
} pbmoe_component_kind;

typedef struct pbmoe_component {
    uint32_t kind;     /* pbmoe_component_kind */
    uint32_t reserved; /* zero */
    uint64_t offset;   /* byte offset inside the expert slot */
    uint64_t bytes;
} pbmoe_component;

/* Fixed-slot 4-bit affine expert layout: QwenMoeQ4ExpertLayout
 * (model_family.rs:954-1068) plus the 2-byte scale/bias dtype tag
 * (BF16 in the reference artifacts, F16 for the benchmark shapes).
 * Packed weights: rows x cols/2 bytes, low nibble first, i.e. column 8w+i at
 * bits 4i of little-endian uint32 word w (shaders.metal:37-65).  Gate/up are
 * [intermediate][hidden], down is [hidden][intermediate]; scale and bias are
 * [rows][cols/group_size]. */
typedef struct pbmoe_q4_layout {
    uint64_t expert_bytes;
    uint32_t group_size;
    uint32_t scale_bias_dtype; /* PBMOE_DTYPE_F16 or PBMOE_DTYPE_BF16 */
    pbmoe_component components[9];
} pbmoe_q4_layout;

/* One resident Q4 projection [rows][cols]: codes rows*cols/2 bytes (low
 * nibble = even column), scale and bias [rows][cols/group] 2-byte each
 * (the q4_mmap_fma_matvec_bf16_scale_bias operand, shaders.metal:488-660). */
typedef struct pbmoe_q4_matrix {
    const void* codes;
    const void* scales;
    const void* biases;
} pbmoe_q4_matrix;

typedef enum pbmoe_routing {
    PBMOE_ROUTING_SOFTMAX_TOPK = 0,     /* routing_softmax_top_k, math.rs:771-783      */
    PBMOE_ROUTING_SIGMOID_NOAUX = 1,    /* routing_sigmoid_noaux_top_k, math.rs:788-819 */
    PBMOE_ROUTING_SIGMOID_GROUPED = 2,  /* DeepSeek-V3 group-limited noaux (no reference
                                           counterpart; equals SIGMOID_NOAUX at n_group=1) */
    PBMOE_ROUTING_SQRT_SOFTPLUS = 3     /* DeepSeek-V4: p = sqrt(softplus(l)), select on
                                           p + bias (bias optional; ties -> lower index),
                                           weights p (deepseek_v4_router_probabilities /
                                           deepseek_v4_select_routes, deepseek.rs:1300-1394);
                                           canonical route order only */
} pbmoe_routing;

typedef enum pbmoe_normalization {      /* QwenMoeRoutingWeightNormalization,
                                           model_family.rs:111-115 */
    PBMOE_NORM_RENORMALIZE_SELECTED = 0,
    PBMOE_NORM_DEEPSEEK_FLOOR = 1,      /* max(sum, 6.103515625e-5) denominator */
    PBMOE_NORM_PRESERVE_FULL_SOFTMAX = 2 /* rejected, as in the reference */
} pbmoe_normalization;

typedef enum pbmoe_route_order {
    PBMOE_ORDER_CANONICAL = 0,      /* score desc, then lower expert index (ties)
                                       — compare_scored_tokens, math.rs:709-718 */
    PBMOE_ORDER_REFERENCE_SLOT = 1  /* replacement-slot scan set and slot order of
                                       routing_top_k_iter, math.rs:746-765 */
} pbmoe_route_order;

/* One MoE layer's graph description (QwenMoeModelLayout routing policy,
 * model_family.rs:1181-1244). */
typedef struct pbmoe_layer_desc {
    uint32_t hidden;
    uint32_t intermediate;
    uint32_t experts;
    uint32_t active_experts;      /* K */
    uint32_t routing;             /* pbmoe_routing */
    uint32_t normalization;       /* pbmoe_normalization */
    uint32_t route_order;         /* pbmoe_route_order */
    float routed_scale;           /* routed_expert_scale (1.0 Qwen) */
    uint32_t n_group;             /* SIGMOID_GROUPED only; 1 otherwise */
    uint32_t topk_group;
    uint32_t shared_intermediate; /* 0: no shared expert */
    uint32_t shared_gated;        /* 1: sigmoid(W_sg . x) gate; 0: constant 1 */
    float norm_epsilon;           /* next-layer RMSNorm epsilon (1e-6) */
} pbmoe_layer_desc;

/* Memory-kind flags for bind calls. */
#define PBMOE_MEM_HOST 0u   /* source is host memory: copied into HBM        */
#define PBMOE_MEM_DEVICE 1u /* source is device memory: referenced, not owned */

typedef struct pbmoe_ctx pbmoe_ctx;

/* ---- errors / version --------------------------------------------------- */
int pbmoe_abi_version(void);
const char* pbmoe_last_error(void);

/* ---- layout (model_family.rs:954-1068, :1132-1152) ---------------------- */
/* QwenMoeQ4ExpertLayout::fixed_bf16 generalised to a scale/bias dtype. */
int pbmoe_q4_layout_fixed(uint32_t hidden, uint32_t intermediate, uint32_t group_size,
                          uint32_t scale_bias_dtype, pbmoe_q4_layout* out);
/* QwenMoeQ4ExpertLayout::validate: contiguous components, sum = expert_bytes. */
int pbmoe_q4_layout_validate(const pbmoe_q4_layout* layout);

/* ---- host-side route validation (scheduler/protocol.rs:1044-1081) -------- */
/* ids/scores are HOST arrays of length `count`. */
int pbmoe_validate_routes(const uint32_t* ids, const float* scores, uint32_t count,
                          uint32_t active_experts, uint32_t experts);
/* ScheduledExpertRoutes::from_routes_with_policy (expert_access.rs:80-135)
 * on HOST arrays: renormalise `count` scores into `weights`. */
int pbmoe_renormalize_routes(const float* scores, uint32_t count, uint32_t normalization,
                             float routed_scale, float* weights);

/* ---- context / stream / memory ------------------------------------------ */
/* MetalExecutionContext::compile_resolved counterpart (runtime/mod.rs:648-687). */
int pbmoe_ctx_create(int device, pbmoe_ctx** out);
int pbmoe_ctx_destroy(pbmoe_ctx* ctx);
/* The context's HIP stream (hipStream_t) for event timing by the caller.
 * Work recorded from this stream into a hipGraph references the context's
 * scratch buffers (routes, plans, activations, attention partials) as they
 * are at capture time.  These grow on demand, and growing frees the old
 * allocation after a stream synchronisation, which is an error while the
 * stream is capturing.  Graph users therefore make one call of every shape
 * they will replay before capturing, and make no larger call on the context
 * while the graph may still be replayed. */
int pbmoe_ctx_stream(pbmoe_ctx* ctx, void** stream);
/* Wait for all work on the context stream (commit_and_wait, ffi.rs:613-634,
 * with the 120 s limit of metal/mod.rs:539-540) and report deferred device
 * errors.  Returns PBMOE_ERR_ROUTE if a kernel saw an out-of-range route. */
int pbmoe_sync(pbmoe_ctx* ctx);
/* Per-kernel device timing (FlashMoeTimingBuckets / record_detailed_timing,
 * types.rs:600-619, runtime/mod.rs:1470): with count == 6, the expert-phase
 * calls attach events[2i] / events[2i+1] (hipEvent_t) as the start / stop
 * events of kernel i's dispatch packet.  Decode and whole-layer calls:
 * 0 router stage, 1 gate/up, 2 down + combine.  Grouped prefill (more than
 * 16 tokens): 0 gate/up GEMM, 1 down GEMM, 2 combine.  With count == 14,
 * events[6 + 2i] / events[7 + 2i] also time pbmoe_attention_decode's kernel
 * i: 0 q/k/v projections, 1 chunk partials, 2 merge, 3 o_proj + residual.
 * count == 0 disables.  Timed calls are not for graph capture. */
int pbmoe_set_phase_events(pbmoe_ctx* ctx, void* const* events, uint32_t count);
/* Measurement reference (no counterpart in the reference): read the device
 * buffer src[0, bytes) once with one 16-byte load per lane, the access shape
 * of the decode weight loads, and store the XOR of all its 32-bit words in
 * the device word *xor_out.  Hardware traffic counters of this launch
 * calibrate those of the MoE kernels.  bytes: a multiple of 16. */
int pbmoe_stream_read(pbmoe_ctx* ctx, const void* src, size_t bytes, uint32_t* xor_out);
int pbmoe_device_alloc(pbmoe_ctx* ctx, size_t bytes, void** dptr);
int pbmoe_device_free(pbmoe_ctx* ctx, void* dptr);
int pbmoe_upload(pbmoe_ctx* ctx, void* dst_device, const void* src_host, size_t bytes);
int pbmoe_download(pbmoe_ctx* ctx, void* dst_host, const void* src_device, size_t bytes);

/* ---- residency (prepare_resident_expert_backing, metal/mod.rs:1382-1402;
 *      ScheduledResidentExpertTable, expert_access.rs:705-798) ----------- */
/* Bind layer `layer`: `experts` fixed slots back to back (layer_NN.bin,
 * experts/mod.rs:2478-2484), slot stride = expert_layout->expert_bytes. */
int pbmoe_bind_layer(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_layer_desc* desc,
                     const pbmoe_q4_layout* expert_layout, const void* slots,
                     size_t slots_bytes, uint32_t mem_flags);

/* ---- on-disk expert packs (experts/mod.rs:283-454, 2478-2519;
 *      experts/store.rs:481-565) ---------------------------------------- */
/* root/layer_NN.json describes root/layer_NN.bin: `experts` fixed slots of
 * `expert_size` bytes back to back (expert e at e * expert_size). */
typedef struct pbmoe_pack_info {
    char format[48];      /* metadata format, e.g. "FIXED_Q4_EXPERT_LAYER_V1" */
    uint32_t layer;
    uint32_t experts;
    uint64_t expert_size; /* slot bytes */
    uint64_t file_bytes;  /* size of layer_NN.bin, 0 when absent */
    uint32_t packs;       /* per-expert entries */
    uint32_t records;     /* per-tensor records over all entries */
} pbmoe_pack_info;
/* Read and validate root/layer_NN.json (read_expert_layer_pack_metadata +
 * ExpertLayerPackMetadata::validate, experts/mod.rs:2501-2519, 372-429):
 * known format, layer, non-zero sizes, experts in range and unique, no pack
 * beyond its slot.  PBMOE_ERR_IO: missing or unreadable file;
 * PBMOE_ERR_FORMAT: malformed or inconsistent metadata. */
int pbmoe_pack_inspect(const char* root, uint32_t layer, pbmoe_pack_info* info);
/* Bind layer `layer` from the pack of file layer `file_layer`: the checks of
 * ExpertSlotStore::resolve_execution_descriptor_from for fixed-Q4 storage
 * (experts/store.rs:481-565: format FIXED_Q4_EXPERT_LAYER_V1, slot size ==
 * expert_layout->expert_bytes, experts and entries == desc->experts, every
 * entry a whole slot, file size == experts * slot size), per-tensor records
 * (when present) matching the layout, then the file is streamed into HBM
 * (two pinned staging buffers, parallel positioned reads) and owned by the
 * binding, as the resident backing of prepare_resident_expert_backing
 * (metal/mod.rs:1382-1402).  Same descriptor rules as pbmoe_bind_layer. */
int pbmoe_bind_layer_file(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_layer_desc* desc,
                          const pbmoe_q4_layout* expert_layout, const char* root,
                          uint32_t file_layer);
/* Device address and size of layer `layer`'s bound slots (the resident
 * table of ScheduledResidentExpertTable, expert_access.rs:705-798). */
int pbmoe_layer_slots(pbmoe_ctx* ctx, uint32_t layer, const void** slots, size_t* bytes);
/* Router projection W [experts][hidden] (dense F16/BF16/F32, the declared
 * resident router of metal/projection.rs:184-281) and, for sigmoid routing,
 * the per-expert selection bias [experts] f32 (e_score_correction_bias);
 * optional (NULL) for the DeepSeek-V4 router. */
int pbmoe_bind_router(pbmoe_ctx* ctx, uint32_t layer, const void* weight, uint32_t dtype,
                      const float* selection_bias, uint32_t mem_flags);
/* Shared expert: one Q4 slot with its own layout (intermediate =
 * desc->shared_intermediate) and, when desc->shared_gated, the gate
 * projection W_sg [1][hidden] (mlp.shared_expert_gate.weight,
 * weights/mod.rs:1843-1845).  encode_shared, metal/mod.rs:4609-4716. */
int pbmoe_bind_shared(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_q4_layout* shared_layout,
                      const void* shared_slot, const void* gate_weight, uint32_t gate_dtype,
                      uint32_t mem_flags);
/* Q4 router projection (the ResidentMmapMatvecProjection::Q4 router of
 * metal/projection.rs:232-259, computed as q4_mmap_fma_matvec /
 * q4_mmap_fma_matvec_bf16_scale_bias, shaders.metal:488-660): codes
 * [experts][hidden/2] (low nibble first), scales and biases
 * [experts][hidden/group_size] in scale_bias_dtype, which must be the
 * experts' scale/bias dtype; group_size 32, 64 or 128.  Replaces a router
 * bound before; selection_bias as for pbmoe_bind_router.  Device codes
 * 16-byte aligned. */
int pbmoe_bind_router_q4(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_q4_matrix* weight,
                         uint32_t group_size, uint32_t scale_bias_dtype,
                         const float* selection_bias, uint32_t mem_flags);
/* Q4 shared-expert gate row W_sg [1][hidden] (a Q4 mlp.shared_expert_gate,
 * resident like the router above): replaces the gate given to
 * pbmoe_bind_shared, which must come first (a later pbmoe_bind_shared
 * replaces this gate again).  The fused decode layer needs the router and
 * the shared gate in one dtype, so a Q4 gate goes with a Q4 router there. */
int pbmoe_bind_shared_gate_q4(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_q4_matrix* gate,
                              uint32_t group_size, uint32_t scale_bias_dtype, uint32_t mem_flags);
int pbmoe_unbind_layer(pbmoe_ctx* ctx, uint32_t layer);

/* ---- router (CMD2 router projection + routing stage) -------------------- */
/* x [tokens][hidden] f32 -> ids [tokens][K] u32, weights [tokens][K] f32
 * (selected, renormalised, scaled), logits_out [tokens][experts] f32
 * (optional, may be NULL).  Replaces encode_resident_projection(router)
 * + readback + routing_softmax_top_k / routing_sigmoid_noaux_top_k +
 * from_routes_with_policy (metal/mod.rs:2943-3013, expert_access.rs:80-135). */
int pbmoe_route(pbmoe_ctx* ctx, uint32_t layer, const float* x, uint32_t tokens, uint32_t* ids,
                float* weights, float* logits_out);
/* Same routing stage from given logits [tokens][experts] (the prefill
 * router matrix, runtime/mod.rs:2707-2711). */
int pbmoe_route_logits(pbmoe_ctx* ctx, uint32_t layer, const float* logits, uint32_t tokens,
                       uint32_t* ids, float* weights);

/* ---- expert phase -------------------------------------------------------- */
/* Decode CMD3 (submit_scheduled_expert_command): for each token, K routed
 * Q4 SwiGLU experts + optional shared expert, combined as
 *   hidden = (residual + sum_k w_k y_k) + sigma(g) * shared
 * (qwen_layer_major_combine, shaders.metal:1756-1786, route order), then,
 * when next_norm_weight != NULL, next_normed = RMSNorm(hidden) * weight
 * (rms_norm_reduced, metal/mod.rs:4433-4461).  tokens <= 16.
 * x, residual, hidden_out, next_normed_out: [tokens][hidden] f32;
 * ids, weights: [tokens][K] (route order). */
int pbmoe_moe_decode(pbmoe_ctx* ctx, uint32_t layer, const float* x, const float* residual,
                     uint32_t tokens, const uint32_t* ids, const float* weights,
                     const float* next_norm_weight, float* hidden_out, float* next_normed_out);
/* Whole MoE block for a decode batch (tokens <= 16): router projection,
 * routing stage and expert phase of pbmoe_route + pbmoe_moe_decode in one
 * call (CMD2 routing then CMD3, metal/mod.rs:2864-3036 and :3252-3332).
 * ids_out/weights_out ([tokens][K], device) receive the routes, or are both
 * NULL. */
int pbmoe_moe_layer(pbmoe_ctx* ctx, uint32_t layer, const float* x, const float* residual,
                    uint32_t tokens, uint32_t* ids_out, float* weights_out,
                    const float* next_norm_weight, float* hidden_out, float* next_normed_out);
/* pbmoe_moe_layer without any allocation.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, results and errors as pbmoe_moe_layer; every scratch buffer
 * (logits, activations, plan, and the routes when ids_out/weights_out are
 * NULL) comes from one static device array of PBMOE_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends.  A call whose scratch would exceed
 * it returns PBMOE_ERR_UNSUPPORTED.  All calls on one GPU share that array:
 * calls that overlap on one GPU (two streams, two contexts) race and must
 * be serialised by the caller. */
#define PBMOE_NOALLOC_SCRATCH_BYTES (8u << 20)
int pbmoe_moe_layer_noalloc(pbmoe_ctx* ctx, uint32_t layer, const float* x, const float* residual,
                            uint32_t tokens, uint32_t* ids_out, float* weights_out,
                            const float* next_norm_weight, float* hidden_out, float* next_normed_out);
/* pbmoe_moe_layer on the un-normalised hidden state: x = RMSNorm(hidden) *
 * norm_weight (the post-attention norm, rms_norm_with_weight_and_epsilon,
 * math.rs:151-167, eps = norm_epsilon) is formed inside the router stage,
 * as CMD2 fuses it after out_proj + residual (metal/mod.rs:2864-2917), and
 * hidden is the residual.  hidden_out must not alias hidden; tokens <= 16. */
int pbmoe_moe_layer_norm(pbmoe_ctx* ctx, uint32_t layer, const float* hidden,
                         const float* norm_weight, uint32_t tokens, uint32_t* ids_out,
                         float* weights_out, const float* next_norm_weight, float* hidden_out,
                         float* next_normed_out);
/* Layer-major prefill (qwen_layer_major_experts, runtime/mod.rs:1151-1161,
 * metal/mod.rs:3583-4106): 1 <= tokens <= 32768.  Same arguments and result
 * contract as pbmoe_moe_decode.  Up to 16 tokens run the decode kernels, so
 * tokens == 1 is bitwise equal to pbmoe_moe_decode (one-row parity,
 * metal/mod.rs:4015-4079).  Larger chunks build the dispatch plan on the
 * device and run the grouped expert GEMMs on the matrix cores (exact 4-bit
 * codes, activations as f16 hi + lo pairs), then the combine in route
 * order.  A SwiGLU activation beyond the f16 range (|a| > 65504), or a sum
 * of 64 of them (the down GEMM's bias-term operand), is reported by
 * pbmoe_sync as PBMOE_ERR_NONFINITE; the shared expert must
 * use the routed experts' group size and scale/bias dtype. */
int pbmoe_moe_prefill(pbmoe_ctx* ctx, uint32_t layer, const float* x, const float* residual,
                      uint32_t tokens, const uint32_t* ids, const float* weights,
                      const float* next_norm_weight, float* hidden_out, float* next_normed_out);

/* ---- dispatch plan (exposed for parity) ---------------------------------- */
/* resolve_layer_major_experts union + qwen_layer_major_group_plan on the
 * device.  ids [tokens][K] u32 (device).  Outputs (device):
 *   unique_ids [experts] (first *unique_count valid, ascending),
 *   unique_count [1], route_slots [tokens*K], grouped_source_rows
 *   [tokens*K], grouped_output_indices [tokens*K], groups [experts][2]
 *   = (start, count) per unique slot. */
int pbmoe_dispatch_plan(pbmoe_ctx* ctx, uint32_t experts, uint32_t active_experts,
                        uint32_t tokens, const uint32_t* ids, uint32_t* unique_ids,
                        uint32_t* unique_count, uint32_t* route_slots,
                        uint32_t* grouped_source_rows, uint32_t* grouped_output_indices,
                        uint32_t* groups);

/* ---- dequantisation (q4_dequantize_rows_with_group_size, math.rs:913-954) */
/* out[r][c] = fma(q, scale, bias) in f32 (device buffers). */
int pbmoe_q4_dequantize(pbmoe_ctx* ctx, const void* packed, const void* scales,
                        const void* biases, uint32_t scale_bias_dtype, uint32_t rows,
                        uint32_t cols, uint32_t group_size, float* out);

/* ---- seeded synthetic weights (benchmarks and tests) --------------------- */
/* Fill `count` Q4 expert slots (experts first_expert..) on the device with
 * the seeded generator of pbmoe_synth.h; bit-identical to the host
 * generator.  tensor: 1 routed experts, 3 shared expert. */
int pbmoe_synth_fill_q4(pbmoe_ctx* ctx, void* slots_device, const pbmoe_q4_layout* layout,
                        uint32_t hidden, uint32_t intermediate, uint64_t seed, uint32_t tensor,
                        uint32_t layer, uint32_t first_expert, uint32_t count);
/* Zero-mean variant of the filled slots: bias -= 7.5 * scale for every group
 * of the three projections (rounded to the scale/bias dtype), as an affine
 * quantisation of zero-mean weights gives; the multi-layer decode stack uses
 * it so that its activations stay bounded across layers. */
int pbmoe_synth_center_q4(pbmoe_ctx* ctx, void* slots_device, const pbmoe_q4_layout* layout,
                          uint32_t hidden, uint32_t intermediate, uint32_t count);

/* ---- GQA full attention, batch-1 decode (the layer before each MoE block)
 * Replaces the Qwen full-attention step of the decode loop:
 * full_attention_output_values (flashmoe/runtime/mod.rs:2215-2367): q/k/v
 * resident Q4 projections, per-head q/k RMSNorm + split-half RoPE
 * (apply_optional_per_head_rms_norm_and_split_half_rope, math.rs:252-325),
 * the KV record of this position (KvCache, state/kv_cache.rs:456-480),
 * causal attention over positions 0..position (causal_attention,
 * math.rs:671-707, softmax_in_place math.rs:728-744); then the o_proj
 * projection and residual add, and the post-attention RMSNorm that feeds the
 * MoE block (add_in_place + rms_norm_with_model_weight, runtime/mod.rs
 * :2979-2996; residual_add_rms_norm, metal/qwen/shaders.metal:1239-1283). */
typedef struct pbmoe_attn_desc {
    uint32_t hidden;       /* H */
    uint32_t q_heads;      /* num_attention_heads */
    uint32_t kv_heads;     /* num_key_value_heads (q_heads multiple, <= 8 q per kv) */
    uint32_t head_dim;     /* 128 */
    uint32_t rotary_dim;   /* == head_dim (split-half pairs (i, i + head_dim/2)) */
    float rope_theta;      /* theta.max(1.0) as f32 (1e6 for Qwen3) */
    float norm_epsilon;    /* post-attention RMSNorm epsilon; q/k norms use 1e-6 */
    uint32_t max_context;  /* KV cache positions */
    uint32_t group_size;   /* Q4 group of the four projections */
    uint32_t scale_bias_dtype; /* PBMOE_DTYPE_F16 or PBMOE_DTYPE_BF16 */
} pbmoe_attn_desc;

/* q [q_heads*head_dim][H], k and v [kv_heads*head_dim][H], o [H][q_heads*
 * head_dim]; q_norm / k_norm [head_dim] f32 (self_attn.q_norm / k_norm, both
 * required as in the reference).  All device memory, referenced. */
typedef struct pbmoe_attn_weights {
    pbmoe_q4_matrix q, k, v, o;
    const float* q_norm;
    const float* k_norm;
} pbmoe_attn_weights;

/* Bind attention layer `layer` and allocate its KV cache (f16, keys and
 * values [max_context][kv_heads][head_dim] each, zeroed). */
int pbmoe_bind_attention(pbmoe_ctx* ctx, uint32_t layer, const pbmoe_attn_desc* desc,
                         const pbmoe_attn_weights* weights);
int pbmoe_unbind_attention(pbmoe_ctx* ctx, uint32_t layer);
/* Device pointers of the layer's KV cache (keys, values). */
int pbmoe_attention_kv_cache(pbmoe_ctx* ctx, uint32_t layer, void** keys, void** values);
/* One token at `position`: normed [H] (x after input_layernorm) -> attention
 * over positions 0..position (this position's k/v written to the cache
 * first) -> o_proj; hidden_out [H] = residual + o; when post_norm_weight is
 * not NULL, post_normed_out [H] = RMSNorm(hidden_out) * post_norm_weight.
 * When input_norm_weight is not NULL, `normed` is the hidden state before
 * input_layernorm and the RMSNorm (desc->norm_epsilon) is applied inside the
 * projection kernel (the deferred next-layer norm handoff; callers then pass
 * the same hidden state as `residual`).  attn_out [q_heads*head_dim]
 * (optional, may be NULL) receives the attention values before o_proj.  All
 * pointers are device memory. */
int pbmoe_attention_decode(pbmoe_ctx* ctx, uint32_t layer, const float* normed,
                           const float* input_norm_weight, const float* residual,
                           uint32_t position, float* hidden_out, const float* post_norm_weight,
                           float* post_normed_out, float* attn_out);

#ifdef __cplusplus
}
#endif

#endif /* PBMOE_H */
