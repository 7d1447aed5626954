/*
 * pbmoe oracle — TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C restatement of the reference's CPU arithmetic for the FlashMoE
 * MoE block (Jc2k/pb, src/inference/flashmoe).  It is the parity checker for
 * the HIP path and the CPU baseline timed by bench.py; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Build: oracle/Makefile, with -ffp-contract=off so that every a*b+c stays
 * two roundings unless the reference itself calls mul_add (written here as
 * an explicit fmaf).  Rust's f32 `exp` is the platform expf; `recip` is 1/x;
 * `Iterator::sum::<f32>` is a sequential left fold.
 *
 * Reference citations are relative to src/inference/flashmoe/.
 *
 * Parity pinning (checked by tests/test_oracle_golden.py):
 *   routing_top_k_iter / top_k / softmax / sigmoid-noaux / renormalise /
 *   validate / dequant / q4 matvec / swiglu / rms norm / group plan:
 *     reference golden vectors plus brute-force and closed-form checks.
 *   or_qk_norm_rope / or_causal_attention / or_attention_decode (the GQA
 *     attention layer of the decode stack): the reference's golden attention
 *     vector (tests/scheduler.rs:826-860), f64 brute force, RoPE closed forms
 *     (identity at position 0, norm preservation per pair, the i = 0
 *     frequency equals the position) and the softmax/GQA invariants.
 *   or_routing_sqrt_softplus_top_k (DeepSeek-V4 router): no golden vector in
 *     the reference's tests; pinned by f64 closed forms of the three softplus
 *     branches, a brute-force stable sort and exact ties.
 *   or_routing_sigmoid_grouped_top_k (DeepSeek-V3 group-limited routing):
 *     no reference implementation exists; pinned by its n_group=1 reduction
 *     to routing_sigmoid_noaux_top_k and by an independent brute-force
 *     restatement of DeepSeek-V3's published definition (group score = sum
 *     of the two largest biased scores, keep topk_group groups, top-k among
 *     their experts; ties to the lower index), exact ties included.
 */
#ifdef __FMA__
#include <immintrin.h>
#endif
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../pb_amd/csrc/pbmoe_synth.h"

enum { OR_DT_F32 = 0, OR_DT_F16 = 1, OR_DT_BF16 = 2 };
enum { OR_ORDER_CANONICAL = 0, OR_ORDER_REFERENCE_SLOT = 1 };
enum { OR_NORM_RENORMALIZE = 0, OR_NORM_DEEPSEEK_FLOOR = 1, OR_NORM_PRESERVE_FULL = 2 };
enum {
    OR_OK = 0,
    OR_ERR_ARG = 1,
    OR_ERR_SHAPE = 2,
    OR_ERR_ROUTE = 5,
    OR_ERR_UNSUPPORTED = 6,
    OR_ERR_NONFINITE = 11
};

static float or_load(const void* base, int dtype, size_t i)
{
    switch (dtype) {
    case OR_DT_F16:
        return pbm_f16_to_f32(((const uint16_t*)base)[i]);
    case OR_DT_BF16:
        return pbm_bf16_to_f32(((const uint16_t*)base)[i]);
    default:
        return ((const float*)base)[i];
    }
}

/* f32::max / f32::min (NaN-ignoring, like Rust). */
static float or_fmax(float a, float b) { return isnan(a) ? b : (isnan(b) ? a : (a > b ? a : b)); }

/* ------------------------------------------------------------------------
 * a1  router logits, sequential mul-then-add
 *     weights/store.rs:880-897 (declared_router_projection),
 *     weights/mod.rs:115-130 (non-macOS dense_f32_matvec_rows)
 * ---------------------------------------------------------------------- */
void or_router_logits(const void* w, int w_dtype, const float* x, int experts, int hidden,
                      float* out)
{
    for (int e = 0; e < experts; ++e) {
        float acc = -0.0f;
        for (int c = 0; c < hidden; ++c) {
            float p = or_load(w, w_dtype, (size_t)e * hidden + c) * x[c];
            acc = acc + p;
        }
        out[e] = acc;
    }
}

/* The same rows split over `threads` OpenMP threads (the all-cores CPU
 * baseline): each row is still one sequential sum, so the result is
 * bitwise that of or_router_logits. */
void or_router_logits_mt(const void* w, int w_dtype, const float* x, int experts, int hidden,
                         float* out, int threads)
{
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
    for (int e = 0; e < experts; ++e) {
        const char* row = (const char*)w + (size_t)e * hidden * (w_dtype == OR_DT_F32 ? 4 : 2);
        or_router_logits(row, w_dtype, x, 1, hidden, out + e);
    }
}

/* ------------------------------------------------------------------------
 * a2  routing_top_k_iter — K-slot replacement scan, slot order
 *     math.rs:746-769
 * ---------------------------------------------------------------------- */
static int or_routing_top_k_iter(const float* scores, int n, int k, int32_t* ids, float* vals)
{
    if (k > n)
        k = n;
    for (int s = 0; s < k; ++s) {
        ids[s] = 0;
        vals[s] = -INFINITY;
    }
    for (int e = 0; e < n; ++e) {
        int minimum = 0;
        for (int c = 1; c < k; ++c)
            if (vals[c] < vals[minimum])
                minimum = c;
        if (k > 0 && scores[e] > vals[minimum]) {
            ids[minimum] = e;
            vals[minimum] = scores[e];
        }
    }
    return k;
}

int or_routing_top_k(const float* scores, int n, int k, int32_t* ids, float* vals)
{
    return or_routing_top_k_iter(scores, n, k, ids, vals);
}

/* total_cmp order on f32: positive NaN > +inf > ... > -inf > negative NaN. */
static int32_t or_total_key(float f)
{
    int32_t b = (int32_t)pbm_f32_bits(f);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* ------------------------------------------------------------------------
 * top_k with the stable order of compare_scored_tokens: score descending by
 * total_cmp, then ascending index (math.rs:710-726).  This is the "lower
 * index tie-break" order and the canonical order of the HIP router.
 * ---------------------------------------------------------------------- */
int or_top_k_sorted(const float* scores, int n, int k, int32_t* ids, float* vals)
{
    if (k > n)
        k = n;
    /* selection by repeated best-of-remaining: O(n*k), exact */
    unsigned char* taken = (unsigned char*)calloc((size_t)n, 1);
    if (!taken)
        return -1;
    for (int s = 0; s < k; ++s) {
        int best = -1;
        for (int e = 0; e < n; ++e) {
            if (taken[e])
                continue;
            if (best < 0 || or_total_key(scores[e]) > or_total_key(scores[best]))
                best = e;
        }
        taken[best] = 1;
        ids[s] = best;
        vals[s] = scores[best];
    }
    free(taken);
    return k;
}

static int or_select(const float* scores, int n, int k, int order, int32_t* ids, float* vals)
{
    return order == OR_ORDER_REFERENCE_SLOT ? or_routing_top_k_iter(scores, n, k, ids, vals)
                                            : or_top_k_sorted(scores, n, k, ids, vals);
}

/* softmax_in_place, math.rs:728-744 */
void or_softmax_in_place(float* v, int n)
{
    if (n <= 0)
        return;
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i)
        mx = or_fmax(mx, v[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    if (sum > 0.0f && isfinite(sum)) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n; ++i)
            v[i] *= inv;
    }
}

/* ------------------------------------------------------------------------
 * a3  routing_softmax_top_k, math.rs:771-783: max over all, sum of
 *     exp(l - max) in index order, select on RAW logits, p = exp(l-max)/sum
 * ---------------------------------------------------------------------- */
int or_routing_softmax_top_k(const float* logits, int n, int k, int order, int32_t* ids,
                             float* p)
{
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i)
        mx = or_fmax(mx, logits[i]);
    float sum = -0.0f;
    for (int i = 0; i < n; ++i)
        sum = sum + expf(logits[i] - mx);
    float vals[1024];
    if (k > 1024)
        return -1;
    int kk = or_select(logits, n, k, order, ids, vals);
    int have_inv = sum > 0.0f && isfinite(sum);
    float inv = have_inv ? 1.0f / sum : 0.0f;
    for (int s = 0; s < kk; ++s) {
        float v = expf(vals[s] - mx);
        if (have_inv)
            v = v * inv;
        p[s] = v;
    }
    return kk;
}

static float or_sigmoid(float l) { return 1.0f / (1.0f + expf(-l)); }

/* ------------------------------------------------------------------------
 * a4  routing_sigmoid_noaux_top_k, math.rs:788-819: select on
 *     sigmoid(l)+bias, return the unbiased sigmoid(l)
 * ---------------------------------------------------------------------- */
int or_routing_sigmoid_noaux_top_k(const float* logits, const float* bias, int n, int k,
                                   int order, int32_t* ids, float* w)
{
    float* biased = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    float vals[1024];
    if (!biased || k > 1024) {
        free(biased);
        return -1;
    }
    for (int e = 0; e < n; ++e)
        biased[e] = or_sigmoid(logits[e]) + bias[e];
    int kk = or_select(biased, n, k, order, ids, vals);
    for (int s = 0; s < kk; ++s)
        w[s] = or_sigmoid(logits[ids[s]]);
    free(biased);
    return kk;
}

/* ------------------------------------------------------------------------
 * DeepSeek-V3 group-limited noaux_tc routing (workload C5).
 * No reference implementation (GLM rejects n_group != 1,
 * model_family.rs:613-614).  Textbook definition:
 *   biased_e = sigmoid(l_e) + bias_e
 *   group score = sum of the two largest biased scores in the group
 *   keep the topk_group best groups (ties -> lower group index)
 *   select top-k of biased among kept experts (ties -> lower index)
 *   weights = unbiased sigmoid of the selected logits
 * With n_group == topk_group == 1 this is routing_sigmoid_noaux_top_k.
 * ---------------------------------------------------------------------- */
int or_routing_sigmoid_grouped_top_k(const float* logits, const float* bias, int n, int k,
                                     int n_group, int topk_group, int32_t* ids, float* w)
{
    if (n_group <= 0 || n % n_group != 0 || topk_group <= 0 || topk_group > n_group)
        return -1;
    int per = n / n_group;
    if (per < 2 && n_group > 1)
        return -1;
    float* biased = (float*)malloc(sizeof(float) * (size_t)n);
    float* gscore = (float*)malloc(sizeof(float) * (size_t)n_group);
    float* masked = (float*)malloc(sizeof(float) * (size_t)n);
    int32_t gids[1024];
    float gv[1024], vals[1024];
    if (!biased || !gscore || !masked || n_group > 1024 || k > 1024) {
        free(biased), free(gscore), free(masked);
        return -1;
    }
    for (int e = 0; e < n; ++e)
        biased[e] = or_sigmoid(logits[e]) + bias[e];
    for (int g = 0; g < n_group; ++g) {
        int32_t t2[2];
        float v2[2];
        int m = or_top_k_sorted(biased + (size_t)g * per, per, per >= 2 ? 2 : 1, t2, v2);
        gscore[g] = m == 2 ? v2[0] + v2[1] : v2[0];
    }
    or_top_k_sorted(gscore, n_group, topk_group, gids, gv);
    for (int e = 0; e < n; ++e)
        masked[e] = -INFINITY;
    for (int s = 0; s < topk_group; ++s)
        for (int j = 0; j < per; ++j)
            masked[gids[s] * per + j] = biased[gids[s] * per + j];
    int kk = or_top_k_sorted(masked, n, k, ids, vals);
    for (int s = 0; s < kk; ++s)
        w[s] = or_sigmoid(logits[ids[s]]);
    free(biased), free(gscore), free(masked);
    return kk;
}

/* ------------------------------------------------------------------------
 * a20 DeepSeek-V4 router (deepseek.rs:1300-1394):
 *   deepseek_v4_router_probabilities: p_e = sqrt(softplus(l_e)) in f32 with
 *     softplus = l (l > 20), exp(l) (l < -20), ln_1p(exp(l)) otherwise;
 *   deepseek_v4_select_routes: experts ordered by p + bias with total_cmp,
 *     descending, ties to the lower index (a stable sort), the first k, each
 *     with its unbiased p.  bias may be NULL (no correction bias: p + 0).
 * The reference fixes n = 256 and k = 6; the arithmetic is the same for
 * any n, k.  Returns -1 on a non-finite logit or bias.
 * ---------------------------------------------------------------------- */
float or_sqrt_softplus(float l)
{
    float sp = l > 20.0f ? l : (l < -20.0f ? expf(l) : log1pf(expf(l)));
    return sqrtf(sp);
}

int or_routing_sqrt_softplus_top_k(const float* logits, const float* bias, int n, int k, int32_t* ids,
                                   float* w)
{
    float* biased = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    float vals[1024];
    if (!biased || k > 1024) {
        free(biased);
        return -1;
    }
    for (int e = 0; e < n; ++e) {
        const float pe = or_sqrt_softplus(logits[e]);
        const float be = bias ? bias[e] : 0.0f;
        if (!isfinite(logits[e]) || !isfinite(pe) || pe < 0.0f || !isfinite(be)) {
            free(biased);
            return -1;
        }
        biased[e] = pe + be;
    }
    int kk = or_top_k_sorted(biased, n, k, ids, vals);
    for (int s = 0; s < kk; ++s)
        w[s] = or_sqrt_softplus(logits[ids[s]]);
    free(biased);
    return kk;
}

/* ------------------------------------------------------------------------
 * a5  ScheduledExpertRoutes::from_routes_with_policy,
 *     scheduler/expert_access.rs:80-135
 * ---------------------------------------------------------------------- */
int or_renormalize(const float* p, int k, int policy, float routed_scale, float* w)
{
    if (!(isfinite(routed_scale) && routed_scale > 0.0f))
        return OR_ERR_ARG;
    for (int s = 0; s < k; ++s)
        if (!isfinite(p[s]))
            return OR_ERR_NONFINITE; /* ExpertRoute::validate */
    float sum = -0.0f;
    for (int s = 0; s < k; ++s)
        sum = sum + p[s];
    float inv;
    if (policy == OR_NORM_RENORMALIZE) {
        if (!(isfinite(sum) && sum > 0.0f))
            return OR_ERR_ROUTE;
        inv = 1.0f / sum;
    } else if (policy == OR_NORM_DEEPSEEK_FLOOR) {
        if (!(isfinite(sum) && sum >= 0.0f))
            return OR_ERR_ROUTE;
        inv = 1.0f / or_fmax(sum, 6.103515625e-5f);
    } else {
        return OR_ERR_UNSUPPORTED; /* PreserveFullSoftmax */
    }
    for (int s = 0; s < k; ++s) {
        if (p[s] < 0.0f)
            return OR_ERR_ROUTE;
        w[s] = p[s] * inv;
    }
    for (int s = 0; s < k; ++s)
        w[s] = w[s] * routed_scale;
    return OR_OK;
}

/* ------------------------------------------------------------------------
 * a6  validate_preselected, scheduler/protocol.rs:1044-1081
 * ---------------------------------------------------------------------- */
int or_validate_preselected(const int32_t* ids, const float* scores, int k, int active_experts,
                            int experts)
{
    if (active_experts <= 0 || active_experts > experts)
        return OR_ERR_ARG; /* validate_bounds */
    if (k != active_experts)
        return OR_ERR_ROUTE;
    for (int s = 0; s < k; ++s) {
        if (ids[s] < 0 || ids[s] >= experts)
            return OR_ERR_ROUTE;
        if (!isfinite(scores[s]))
            return OR_ERR_NONFINITE;
        for (int t = 0; t < s; ++t)
            if (ids[t] == ids[s])
                return OR_ERR_ROUTE;
    }
    return OR_OK;
}

/* ------------------------------------------------------------------------
 * a11 q4_dequantize_rows_with_group_size, math.rs:913-954: w = fma(q,s,b)
 *     q = low nibble for even column, high nibble for odd (byte view), which
 *     is bits 4*(c%8) of the little-endian word (shaders.metal:37-65).
 * ---------------------------------------------------------------------- */
static inline float or_nibble(const uint8_t* packed, size_t row_stride, int row, int col)
{
    uint8_t byte = packed[(size_t)row * row_stride + (size_t)(col / 2)];
    return (float)((col & 1) == 0 ? (byte & 0x0F) : (byte >> 4));
}

int or_q4_dequantize_rows(const uint8_t* packed, const void* scales, const void* biases,
                          int sb_dtype, int rows, int cols, int group, float* out)
{
    if (group <= 0)
        return OR_ERR_ARG;
    int gpr = (cols + group - 1) / group;
    size_t stride = (size_t)(cols + 1) / 2;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < gpr; ++g) {
            float s = or_load(scales, sb_dtype, (size_t)r * gpr + g);
            float b = or_load(biases, sb_dtype, (size_t)r * gpr + g);
            int end = (g + 1) * group < cols ? (g + 1) * group : cols;
            for (int c = g * group; c < end; ++c)
                out[(size_t)r * cols + c] = fmaf(or_nibble(packed, stride, r, c), s, b);
        }
    return OR_OK;
}

/* ------------------------------------------------------------------------
 * a12 q4_fma_matvec_with_group_size, math.rs:861-911:
 *     acc += fma(q, s*x, b*x), sequential over columns
 * ---------------------------------------------------------------------- */
int or_q4_fma_matvec(const uint8_t* packed, const float* x, const void* scales,
                     const void* biases, int sb_dtype, int rows, int cols, int group, float* out)
{
    if (group <= 0)
        return OR_ERR_ARG;
    int gpr = (cols + group - 1) / group;
    size_t stride = (size_t)(cols + 1) / 2;
    /* Eight rows side by side: each row's sum is the same sequential chain of
     * operations as one row alone (bitwise equal); the eight chains run in
     * the lanes of one vector, so that their additions overlap.  A group's
     * codes of the eight rows are decoded into q8 first. */
    int r = 0;
    float q8[128 * 8];
    if (group <= 128)
        for (; r + 8 <= rows; r += 8) {
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            for (int g = 0; g < gpr; ++g) {
                float s[8], b[8];
                for (int j = 0; j < 8; ++j) {
                    s[j] = or_load(scales, sb_dtype, (size_t)(r + j) * gpr + g);
                    b[j] = or_load(biases, sb_dtype, (size_t)(r + j) * gpr + g);
                }
                int c0 = g * group, end = (g + 1) * group < cols ? (g + 1) * group : cols;
                if ((c0 & 1) == 0 && ((end - c0) & 1) == 0) {
                    for (int j = 0; j < 8; ++j) {
                        const uint8_t* row = packed + (size_t)(r + j) * stride + c0 / 2;
                        for (int i = 0; i < (end - c0) / 2; ++i) {
                            q8[(2 * i) * 8 + j] = (float)(row[i] & 0x0F);
                            q8[(2 * i + 1) * 8 + j] = (float)(row[i] >> 4);
                        }
                    }
                } else {
                    for (int c = c0; c < end; ++c)
                        for (int j = 0; j < 8; ++j)
                            q8[(c - c0) * 8 + j] = or_nibble(packed, stride, r + j, c);
                }
#ifdef __FMA__
                /* lane j = row r + j: mul, mul, fused multiply-add, add, the
                 * operations (and roundings) of the scalar loop below */
                __m256 va = _mm256_loadu_ps(acc);
                const __m256 vs = _mm256_loadu_ps(s), vb = _mm256_loadu_ps(b);
                for (int c = c0; c < end; ++c) {
                    const __m256 xc = _mm256_set1_ps(x[c]);
                    const __m256 q = _mm256_loadu_ps(q8 + (c - c0) * 8);
                    va = _mm256_add_ps(va, _mm256_fmadd_ps(q, _mm256_mul_ps(vs, xc), _mm256_mul_ps(vb, xc)));
                }
                _mm256_storeu_ps(acc, va);
#else
                for (int c = c0; c < end; ++c) {
                    const float xc = x[c];
                    const float* q = q8 + (c - c0) * 8;
                    for (int j = 0; j < 8; ++j)
                        acc[j] = acc[j] + fmaf(q[j], s[j] * xc, b[j] * xc);
                }
#endif
            }
            for (int j = 0; j < 8; ++j)
                out[r + j] = acc[j];
        }
    for (; r < rows; ++r) {
        float acc = 0.0f;
        for (int g = 0; g < gpr; ++g) {
            float s = or_load(scales, sb_dtype, (size_t)r * gpr + g);
            float b = or_load(biases, sb_dtype, (size_t)r * gpr + g);
            int end = (g + 1) * group < cols ? (g + 1) * group : cols;
            for (int c = g * group; c < end; ++c) {
                float sx = s * x[c];
                float bx = b * x[c];
                acc = acc + fmaf(or_nibble(packed, stride, r, c), sx, bx);
            }
        }
        out[r] = acc;
    }
    return OR_OK;
}

/* Explicit-dequant form of the test helper reference_q4_matvec,
 * tests/scheduler.rs:308-325: sum of (q*s + b) * x. */
int or_q4_explicit_matvec(const uint8_t* packed, const float* x, const void* scales,
                          const void* biases, int sb_dtype, int rows, int cols, int group,
                          float* out)
{
    int gpr = (cols + group - 1) / group;
    size_t stride = (size_t)(cols + 1) / 2;
    for (int r = 0; r < rows; ++r) {
        float acc = -0.0f;
        for (int c = 0; c < cols; ++c) {
            int g = r * gpr + c / group;
            float w = or_nibble(packed, stride, r, c) * or_load(scales, sb_dtype, (size_t)g) +
                      or_load(biases, sb_dtype, (size_t)g);
            acc = acc + w * x[c];
        }
        out[r] = acc;
    }
    return OR_OK;
}

/* a13 SwiGLU: g/(1+exp(-g)) * u  (tests/scheduler.rs:327-336,
 *     shaders.metal:1699-1708) */
void or_swiglu(const float* g, const float* u, int n, float* out)
{
    for (int i = 0; i < n; ++i)
        out[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* a16 rms norm, math.rs:147-167 (eps 1e-6 by default) */
void or_rms_norm(const float* x, const float* w, int n, float eps, float* out)
{
    float ms = -0.0f;
    for (int i = 0; i < n; ++i)
        ms = ms + x[i] * x[i];
    ms = ms / (float)(n > 1 ? n : 1);
    float scale = 1.0f / sqrtf(ms + eps);
    for (int i = 0; i < n; ++i) {
        float v = x[i] * scale;
        out[i] = w ? v * w[i] : v;
    }
}

/* ------------------------------------------------------------------------
 * a7  resolve_layer_major_experts union: sorted unique expert ids and the
 *     per-route slot index into that union, scheduler/mod.rs:685-769
 * ---------------------------------------------------------------------- */
int or_layer_major_union(const int32_t* ids, int rows, int k, int experts, int32_t* unique_ids,
                         int* unique_count, int32_t* route_slots)
{
    if (rows <= 0)
        return OR_ERR_ARG;
    int32_t* slot_of = (int32_t*)malloc(sizeof(int32_t) * (size_t)experts);
    if (!slot_of)
        return OR_ERR_ARG;
    for (int e = 0; e < experts; ++e)
        slot_of[e] = -1;
    for (int i = 0; i < rows * k; ++i) {
        if (ids[i] < 0 || ids[i] >= experts) {
            free(slot_of);
            return OR_ERR_ROUTE;
        }
        slot_of[ids[i]] = 0;
    }
    int u = 0;
    for (int e = 0; e < experts; ++e)
        if (slot_of[e] == 0) {
            slot_of[e] = u;
            unique_ids[u++] = e;
        }
    for (int i = 0; i < rows * k; ++i)
        route_slots[i] = slot_of[ids[i]];
    *unique_count = u;
    free(slot_of);
    return OR_OK;
}

/* ------------------------------------------------------------------------
 * a8  qwen_layer_major_group_plan, metal/mod.rs:3197-3233: stable counting
 *     sort of routes by slot.  groups is [unique][2] = (start, count).
 * ---------------------------------------------------------------------- */
int or_group_plan(const int32_t* route_slots, int n_routes, int unique, int active,
                  uint32_t* src_rows, uint32_t* out_idx, uint32_t* groups)
{
    if (n_routes <= 0 || unique <= 0 || active <= 0)
        return OR_ERR_ARG;
    uint32_t* count = (uint32_t*)calloc((size_t)unique, sizeof(uint32_t));
    if (!count)
        return OR_ERR_ARG;
    for (int r = 0; r < n_routes; ++r) {
        if (route_slots[r] < 0 || route_slots[r] >= unique) {
            free(count);
            return OR_ERR_ROUTE;
        }
        count[route_slots[r]]++;
    }
    uint32_t start = 0;
    for (int s = 0; s < unique; ++s) {
        if (count[s] == 0) {
            free(count);
            return OR_ERR_ROUTE; /* unused slot in the union */
        }
        groups[2 * s] = start;
        groups[2 * s + 1] = count[s];
        start += count[s];
    }
    uint32_t* cursor = (uint32_t*)calloc((size_t)unique, sizeof(uint32_t));
    for (int r = 0; r < n_routes; ++r) {
        int s = route_slots[r];
        uint32_t i = groups[2 * s] + cursor[s]++;
        src_rows[i] = (uint32_t)(r / active);
        out_idx[r] = i;
    }
    free(cursor);
    free(count);
    return OR_OK;
}

/* ------------------------------------------------------------------------
 * Whole MoE block for T rows (decode CMD3 and layer-major prefill compute
 * the same per-row arithmetic, metal/mod.rs:4289-4765 and :3583-4106):
 *   per route k: g = Q4(gate)x, u = Q4(up)x, a = silu(g)*u, y_k = Q4(down)a
 *   shared (optional): S = Q4(down_s)(silu(Q4(gate_s)x)*Q4(up_s)x),
 *     gate weight sigma(W_sg . x), or sigma(80) = 1 without a gate
 *     projection (metal/mod.rs:4666-4669)
 *   h = (r + sum_k w_k y_k) + sw * S   (qwen_layer_major_combine,
 *     shaders.metal:1756-1786, route order)
 *   optional next-layer RMSNorm (metal/mod.rs:4433-4461)
 * ---------------------------------------------------------------------- */
typedef struct {
    uint32_t hidden, intermediate, group_size, sb_dtype;
    uint64_t expert_bytes;
    uint64_t offset[9];
} or_q4_layout;

static void or_projection(const or_q4_layout* l, const uint8_t* slot, int proj, const float* x,
                          float* out)
{
    int rows = proj == 2 ? (int)l->hidden : (int)l->intermediate;
    int cols = proj == 2 ? (int)l->intermediate : (int)l->hidden;
    or_q4_fma_matvec(slot + l->offset[3 * proj], x, slot + l->offset[3 * proj + 1],
                     slot + l->offset[3 * proj + 2], (int)l->sb_dtype, rows, cols,
                     (int)l->group_size, out);
}

static void or_expert_swiglu(const or_q4_layout* l, const uint8_t* slot, const float* x,
                             float* y, float* scratch)
{
    int I = (int)l->intermediate;
    float* g = scratch;
    float* u = scratch + I;
    float* a = scratch + 2 * I;
    or_projection(l, slot, 0, x, g);
    or_projection(l, slot, 1, x, u);
    or_swiglu(g, u, I, a);
    or_projection(l, slot, 2, a, y);
}

/* One expert's SwiGLU MLP on one row (CMD3 per-expert chain,
 * metal/mod.rs:4365-4405; reference_q4_swiglu, tests/scheduler.rs:327-336). */
int or_expert_mlp(const or_q4_layout* l, const uint8_t* slot, const float* x, float* y)
{
    float* scratch = (float*)malloc(sizeof(float) * 3 * (size_t)l->intermediate);
    if (!scratch)
        return OR_ERR_ARG;
    or_expert_swiglu(l, slot, x, y, scratch);
    free(scratch);
    return OR_OK;
}

/* qwen_layer_major_combine for one row (shaders.metal:1756-1786):
 * moe accumulates w_k * y_k in route order; h = (r + moe) + sw * S. */
void or_combine(const float* residual, const float* y, const float* w, int k, const float* shared,
                float sw, int hidden, float* out)
{
    for (int c = 0; c < hidden; ++c) {
        float moe = 0.0f;
        for (int j = 0; j < k; ++j)
            moe = moe + w[j] * y[(size_t)j * hidden + c];
        float rm = residual[c] + moe;
        out[c] = rm + sw * (shared ? shared[c] : 0.0f);
    }
}

/* A resident Q4 row set (a Q4 router or shared-expert gate projection,
 * ResidentMmapMatvecProjection::Q4, metal/projection.rs:232-259), given to
 * or_moe_block as its shared gate when shared_gate_dtype == OR_DT_Q4. */
typedef struct {
    const uint8_t* codes;
    const void* scales;
    const void* biases;
    int group, sb_dtype;
} or_q4_rows;
#define OR_DT_Q4 3

int or_moe_block(const or_q4_layout* lay, const uint8_t* slots, int experts,
                 const or_q4_layout* shared_lay, const uint8_t* shared_slot,
                 const void* shared_gate_w, int shared_gate_dtype, const float* x,
                 const float* residual, int rows, int k, const int32_t* ids,
                 const float* weights, const float* next_norm_w, float eps, float* hidden,
                 float* next_normed, int threads)
{
    int H = (int)lay->hidden;
    int I = (int)lay->intermediate;
    if (shared_lay && (int)shared_lay->hidden != H)
        return OR_ERR_SHAPE;
    for (int i = 0; i < rows * k; ++i)
        if (ids[i] < 0 || ids[i] >= experts)
            return OR_ERR_ROUTE;
    int Is = shared_lay ? (int)shared_lay->intermediate : 0;
    int Imax = I > Is ? I : Is;
    /* y for every route, then S for every row */
    float* y = (float*)malloc(sizeof(float) * (size_t)rows * k * H);
    float* S = (float*)malloc(sizeof(float) * (size_t)rows * H);
    float* sw = (float*)malloc(sizeof(float) * (size_t)rows);
    if (!y || !S || !sw) {
        free(y), free(S), free(sw);
        return OR_ERR_ARG;
    }
    (void)threads;
#ifdef _OPENMP
    if (threads > 0)
        omp_set_num_threads(threads);
#pragma omp parallel if (threads > 1)
#endif
    {
        float* scratch = (float*)malloc(sizeof(float) * 3 * (size_t)Imax);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int job = 0; job < rows * (k + 1); ++job) {
            int t = job / (k + 1), j = job % (k + 1);
            const float* xt = x + (size_t)t * H;
            if (j < k) {
                int r = t * k + j;
                or_expert_swiglu(lay, slots + (size_t)ids[r] * lay->expert_bytes, xt,
                                 y + (size_t)r * H, scratch);
            } else if (shared_lay) {
                or_expert_swiglu(shared_lay, shared_slot, xt, S + (size_t)t * H, scratch);
                float g = 80.0f;
                if (shared_gate_w && shared_gate_dtype == OR_DT_Q4) {
                    const or_q4_rows* q = (const or_q4_rows*)shared_gate_w;
                    or_q4_fma_matvec(q->codes, xt, q->scales, q->biases, q->sb_dtype, 1, H, q->group, &g);
                } else if (shared_gate_w)
                    or_router_logits(shared_gate_w, shared_gate_dtype, xt, 1, H, &g);
                sw[t] = or_sigmoid(g);
            } else {
                memset(S + (size_t)t * H, 0, sizeof(float) * (size_t)H);
                sw[t] = 0.0f;
            }
        }
        free(scratch);
    }
    for (int t = 0; t < rows; ++t) {
        float* h = hidden + (size_t)t * H;
        or_combine(residual + (size_t)t * H, y + (size_t)t * k * H, weights + (size_t)t * k, k,
                   S + (size_t)t * H, sw[t], H, h);
        if (next_norm_w && next_normed)
            or_rms_norm(h, next_norm_w, H, eps, next_normed + (size_t)t * H);
    }
    free(y), free(S), free(sw);
    return OR_OK;
}

/* ------------------------------------------------------------------------
 * Route T rows from router logits: softmax/sigmoid selection, then the
 * scheduler's renormalisation (the CPU routing stage of metal/mod.rs:
 * 3005-3013 followed by expert_access.rs:80-135).
 * kind: 0 softmax top-k, 1 sigmoid noaux, 2 sigmoid grouped, 3 DeepSeek-V4
 * sqrt-softplus (then batch_route_rows' floor renormalisation and scale,
 * metal/deepseek_execution.rs:3547-3583, with policy DEEPSEEK_FLOOR).
 * ---------------------------------------------------------------------- */
int or_route_rows(const float* logits, const float* bias, int rows, int experts, int k, int kind,
                  int order, int n_group, int topk_group, int policy, float routed_scale,
                  int32_t* ids, float* weights)
{
    float p[1024];
    if (k > 1024)
        return OR_ERR_ARG;
    for (int t = 0; t < rows; ++t) {
        const float* l = logits + (size_t)t * experts;
        for (int e = 0; e < experts; ++e)
            if (!isfinite(l[e]))
                return OR_ERR_NONFINITE; /* protocol.rs:999-1007 */
        int kk;
        if (kind == 0)
            kk = or_routing_softmax_top_k(l, experts, k, order, ids + (size_t)t * k, p);
        else if (kind == 1)
            kk = or_routing_sigmoid_noaux_top_k(l, bias, experts, k, order, ids + (size_t)t * k, p);
        else if (kind == 2)
            kk = or_routing_sigmoid_grouped_top_k(l, bias, experts, k, n_group, topk_group,
                                                  ids + (size_t)t * k, p);
        else
            kk = or_routing_sqrt_softplus_top_k(l, bias, experts, k, ids + (size_t)t * k, p);
        if (kk != k)
            return OR_ERR_ROUTE;
        int rc = or_renormalize(p, k, policy, routed_scale, weights + (size_t)t * k);
        if (rc)
            return rc;
    }
    return OR_OK;
}

/* ------------------------------------------------------------------------
 * fp64 evaluation of the same block (not a reference restatement: the exact
 * value the f32 paths approximate).  Used to measure the reference's own
 * f32 rounding error where outputs are large enough that a fixed absolute
 * tolerance falls below f32 resolution.
 * ---------------------------------------------------------------------- */
/* Row r of a Q4 projection [rows][cols] as exact f64 weights q*s + b. */
static void or_q4_row_f64(const uint8_t* packed, const void* sc, const void* bi, int sb_dtype, int cols, int g,
                          int r, double* w)
{
    const int gpr = cols / g;
    const uint8_t* row = packed + (size_t)r * (size_t)(cols / 2);
    for (int k = 0; k < gpr; ++k) {
        const double s = or_load(sc, sb_dtype, (size_t)r * gpr + k);
        const double b = or_load(bi, sb_dtype, (size_t)r * gpr + k);
        for (int i = k * g / 2; i < (k + 1) * g / 2; ++i) {
            w[2 * i] = (double)(row[i] & 0x0F) * s + b;
            w[2 * i + 1] = (double)(row[i] >> 4) * s + b;
        }
    }
}

static double or_dot_f64(const double* a, const double* b, int n)
{
    double acc = 0.0;
#ifdef _OPENMP
#pragma omp simd reduction(+ : acc)
#endif
    for (int i = 0; i < n; ++i)
        acc += a[i] * b[i];
    return acc;
}

/* One expert's SwiGLU MLP in f64 for n input rows x[n][H] -> y[n][H]: every
 * weight row is decoded once and applied to all n rows. */
static void or_expert_f64_rows(const or_q4_layout* l, const uint8_t* slot, const double* x, int n, double* y)
{
    const int H = (int)l->hidden, I = (int)l->intermediate, g = (int)l->group_size, sbt = (int)l->sb_dtype;
    double* w = (double*)malloc(sizeof(double) * (size_t)(H > I ? H : I));
    double* gu = (double*)malloc(sizeof(double) * 2 * (size_t)n * I);
    double* act = (double*)malloc(sizeof(double) * (size_t)n * I);
    for (int m = 0; m < 2; ++m) /* gate, up */
        for (int i = 0; i < I; ++i) {
            or_q4_row_f64(slot + l->offset[3 * m], slot + l->offset[3 * m + 1], slot + l->offset[3 * m + 2], sbt,
                          H, g, i, w);
            for (int t = 0; t < n; ++t)
                gu[((size_t)m * n + t) * I + i] = or_dot_f64(w, x + (size_t)t * H, H);
        }
    for (size_t e = 0; e < (size_t)n * I; ++e) {
        const double gg = gu[e], uu = gu[(size_t)n * I + e];
        act[e] = gg / (1.0 + exp(-gg)) * uu;
    }
    for (int r = 0; r < H; ++r) {
        or_q4_row_f64(slot + l->offset[6], slot + l->offset[7], slot + l->offset[8], sbt, I, g, r, w);
        for (int t = 0; t < n; ++t)
            y[(size_t)t * H + r] = or_dot_f64(w, act + (size_t)t * I, I);
    }
    free(w);
    free(gu);
    free(act);
}

/* Expert-major: the routes of each expert (and the shared expert over all
 * rows) form one job; then the combine in f64. */
int or_moe_block_f64(const or_q4_layout* lay, const uint8_t* slots, int experts,
                     const or_q4_layout* shared_lay, const uint8_t* shared_slot,
                     const void* shared_gate_w, int shared_gate_dtype, const float* x,
                     const float* residual, int rows, int k, const int32_t* ids,
                     const float* weights, double* hidden, int threads)
{
    const int H = (int)lay->hidden;
    const int R = rows * k;
    for (int i = 0; i < R; ++i)
        if (ids[i] < 0 || ids[i] >= experts)
            return OR_ERR_ROUTE;
    if (shared_lay && (int)shared_lay->hidden != H)
        return OR_ERR_SHAPE;
    /* routes grouped by expert (stable) */
    int* start = (int*)calloc((size_t)experts + 1, sizeof(int));
    int* order = (int*)malloc(sizeof(int) * (size_t)(R > 0 ? R : 1));
    double* xd = (double*)malloc(sizeof(double) * (size_t)rows * H);
    double* y = (double*)malloc(sizeof(double) * (size_t)(R > 0 ? R : 1) * H);
    double* S = shared_lay ? (double*)malloc(sizeof(double) * (size_t)rows * H) : NULL;
    for (int i = 0; i < R; ++i)
        start[ids[i] + 1]++;
    for (int e = 0; e < experts; ++e)
        start[e + 1] += start[e];
    {
        int* fill = (int*)malloc(sizeof(int) * (size_t)experts);
        memcpy(fill, start, sizeof(int) * (size_t)experts);
        for (int i = 0; i < R; ++i)
            order[fill[ids[i]]++] = i;
        free(fill);
    }
    for (size_t i = 0; i < (size_t)rows * H; ++i)
        xd[i] = x[i];
    const int jobs = experts + (shared_lay ? 1 : 0);
    (void)threads;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic, 1)
#endif
    for (int j = 0; j < jobs; ++j) {
        if (j == experts) { /* the shared expert over every row */
            or_expert_f64_rows(shared_lay, shared_slot, xd, rows, S);
            continue;
        }
        const int n = start[j + 1] - start[j];
        if (n == 0)
            continue;
        double* xin = (double*)malloc(sizeof(double) * (size_t)n * H);
        double* yo = (double*)malloc(sizeof(double) * (size_t)n * H);
        for (int q = 0; q < n; ++q)
            memcpy(xin + (size_t)q * H, xd + (size_t)(order[start[j] + q] / k) * H, sizeof(double) * (size_t)H);
        or_expert_f64_rows(lay, slots + (size_t)j * lay->expert_bytes, xin, n, yo);
        for (int q = 0; q < n; ++q)
            memcpy(y + (size_t)order[start[j] + q] * H, yo + (size_t)q * H, sizeof(double) * (size_t)H);
        free(xin);
        free(yo);
    }
    for (int t = 0; t < rows; ++t) {
        double* h = hidden + (size_t)t * H;
        for (int c = 0; c < H; ++c)
            h[c] = residual[(size_t)t * H + c];
        for (int j = 0; j < k; ++j)
            for (int c = 0; c < H; ++c)
                h[c] += (double)weights[t * k + j] * y[((size_t)t * k + j) * H + c];
        if (shared_lay) {
            double g = 80.0;
            const double* xt = xd + (size_t)t * H;
            if (shared_gate_w && shared_gate_dtype == OR_DT_Q4) {
                const or_q4_rows* q = (const or_q4_rows*)shared_gate_w;
                double* w = (double*)malloc(sizeof(double) * (size_t)H);
                or_q4_row_f64(q->codes, q->scales, q->biases, q->sb_dtype, H, q->group, 0, w);
                g = or_dot_f64(w, xt, H);
                free(w);
            } else if (shared_gate_w) {
                g = 0.0;
                for (int c = 0; c < H; ++c)
                    g += (double)or_load(shared_gate_w, shared_gate_dtype, (size_t)c) * xt[c];
            }
            const double sw = 1.0 / (1.0 + exp(-g));
            for (int c = 0; c < H; ++c)
                h[c] += sw * S[(size_t)t * H + c];
        }
    }
    free(start);
    free(order);
    free(xd);
    free(y);
    free(S);
    return OR_OK;
}

/* ---- GQA attention of the decode stack ----------------------------------- */

/* Per-head RMSNorm with weight then split-half RoPE:
 * apply_optional_per_head_rms_norm_and_split_half_rope (math.rs:252-301)
 * with the rotations of split_half_rope_rotations (math.rs:303-325):
 * inv_freq = theta^(-(2i)/rotary_dim) and angle = position * inv_freq in
 * f32, (sin, cos) of that f32 angle; value *= scale * weight[d] with
 * scale = 1 / sqrt(mean(v^2) + 1e-6); pairs (i, i + rotary_dim / 2).
 * weight NULL: no norm. */
void or_qk_norm_rope(float* v, int heads, int head_dim, const float* weight, int position,
                     int rotary_dim, float theta)
{
    if (theta < 1.0f)
        theta = 1.0f;
    if (head_dim < 2)
        head_dim = 2;
    int rot = rotary_dim < head_dim ? rotary_dim : head_dim;
    rot -= rot % 2;
    const int half = rot / 2;
    float* sn = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    float* cs = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
    for (int i = 0; i < half; ++i) {
        const float inv = powf(theta, -((float)(2 * i)) / (float)(rot > 0 ? rot : 1));
        const float ang = (float)position * inv;
        sn[i] = sinf(ang);
        cs[i] = cosf(ang);
    }
    for (int h = 0; h < heads; ++h) {
        float* x = v + (size_t)h * head_dim;
        if (weight) {
            float ms = 0.0f;
            for (int d = 0; d < head_dim; ++d)
                ms = ms + x[d] * x[d];
            ms = ms / (float)head_dim;
            const float scale = 1.0f / sqrtf(ms + 1e-6f);
            for (int d = 0; d < head_dim; ++d)
                x[d] = x[d] * (scale * weight[d]);
        }
        for (int i = 0; i < half; ++i) {
            const float x0 = x[i], x1 = x[i + half];
            x[i] = x0 * cs[i] - x1 * sn[i];
            x[i + half] = x0 * sn[i] + x1 * cs[i];
        }
    }
    free(sn);
    free(cs);
}

/* causal_attention (math.rs:671-707): for every q head, scores over the n
 * rows of keys [n][kv_heads*head_dim] (sum of q*k in order, times
 * 1/sqrt(head_dim)), softmax_in_place (math.rs:728-744), then the weighted
 * sum of the value rows; q head h reads kv head h / (q_heads / kv_heads). */
void or_causal_attention(const float* q, const float* keys, const float* values, int n, int q_heads,
                         int kv_heads, int head_dim, float* out)
{
    const int qw = q_heads * head_dim, kvw = kv_heads * head_dim;
    for (int i = 0; i < qw; ++i)
        out[i] = 0.0f;
    if (n <= 0 || q_heads <= 0 || head_dim <= 0)
        return;
    const int groups = q_heads / (kv_heads > 0 ? kv_heads : 1);
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* sc = (float*)malloc(sizeof(float) * (size_t)n);
    for (int qh = 0; qh < q_heads; ++qh) {
        const int kh = qh / (groups > 0 ? groups : 1);
        const float* qs = q + (size_t)qh * head_dim;
        for (int t = 0; t < n; ++t) {
            const float* ks = keys + (size_t)t * kvw + (size_t)kh * head_dim;
            float s = 0.0f;
            for (int d = 0; d < head_dim; ++d)
                s = s + qs[d] * ks[d];
            sc[t] = s * scale;
        }
        or_softmax_in_place(sc, n);
        float* o = out + (size_t)qh * head_dim;
        for (int t = 0; t < n; ++t) {
            const float* vs = values + (size_t)t * kvw + (size_t)kh * head_dim;
            for (int d = 0; d < head_dim; ++d)
                o[d] = o[d] + sc[t] * vs[d];
        }
    }
    free(sc);
}

static float or_f16_round(float x)
{
    return pbm_f16_to_f32(pbm_f32_to_f16(x));
}

/* One decode token through the attention layer (full_attention_output_values,
 * runtime/mod.rs:2215-2367, then the o_proj projection of the decode loop):
 * q, k, v = Q4 projections of `normed` (q4_fma_matvec form); per-head q/k
 * norm + RoPE at `position`; k and v rounded to f16 (the KV cache format)
 * into cache row `position` (the cache holds the f16 values as f32,
 * [rows][kv_heads*head_dim]); causal attention over rows 0..position;
 * o_out = W_o . attention.  Matrices: q [qh*hd][H], k/v [kvh*hd][H],
 * o [H][qh*hd], codes + 2-byte scale/bias (sb_dtype). */
int or_attention_decode(const uint8_t* const* codes, const void* const* scales, const void* const* biases,
                        int sb_dtype, int group, const float* q_norm, const float* k_norm, int hidden,
                        int q_heads, int kv_heads, int head_dim, int rotary_dim, float theta, int position,
                        const float* normed, float* cache_k, float* cache_v, float* attn_out, float* o_out)
{
    const int qw = q_heads * head_dim, kvw = kv_heads * head_dim;
    float* q = (float*)malloc(sizeof(float) * (size_t)qw);
    float* k = (float*)malloc(sizeof(float) * (size_t)kvw);
    float* v = (float*)malloc(sizeof(float) * (size_t)kvw);
    int rc = or_q4_fma_matvec(codes[0], normed, scales[0], biases[0], sb_dtype, qw, hidden, group, q);
    if (rc == OR_OK)
        rc = or_q4_fma_matvec(codes[1], normed, scales[1], biases[1], sb_dtype, kvw, hidden, group, k);
    if (rc == OR_OK)
        rc = or_q4_fma_matvec(codes[2], normed, scales[2], biases[2], sb_dtype, kvw, hidden, group, v);
    if (rc == OR_OK) {
        or_qk_norm_rope(q, q_heads, head_dim, q_norm, position, rotary_dim, theta);
        or_qk_norm_rope(k, kv_heads, head_dim, k_norm, position, rotary_dim, theta);
        for (int i = 0; i < kvw; ++i) {
            cache_k[(size_t)position * kvw + i] = or_f16_round(k[i]);
            cache_v[(size_t)position * kvw + i] = or_f16_round(v[i]);
        }
        or_causal_attention(q, cache_k, cache_v, position + 1, q_heads, kv_heads, head_dim, attn_out);
        rc = or_q4_fma_matvec(codes[3], attn_out, scales[3], biases[3], sb_dtype, hidden, qw, group, o_out);
    }
    free(q);
    free(k);
    free(v);
    return rc;
}

