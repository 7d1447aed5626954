/*
 * Host-side seeded generator for the MoE block's synthetic inputs
 * (libpbmoe_synth.so).  Uniform Q4 data uses the integer/fmaf formulas of
 * pbmoe_synth.h, so the device fill kernel produces the same bytes; normal
 * draws (router weights, activations, drawn logits) are produced here only.
 *
 * Workloads (synthetic, seeded):
 *   Q4 experts: nibbles uniform 0..15, scale ~U(0.005,0.02), bias
 *     ~U(-0.1,0.1) per group, stored as f16 or bf16.
 *   Router / shared gate weights: f16 N(0, 0.02).
 *   Inputs x and residual: f16 N(0, 1) widened to f32.
 *   Prefill logits: 0.1*N(0,1) + 4*[e in S_t], S_t = K distinct experts
 *     drawn from Zipf(s) over a seeded permutation of the expert ids.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "pbmoe_synth.h"

#define PBM_EXPORT __attribute__((visibility("default")))

static void pbm_fill_projection(uint64_t seed, uint32_t tensor, uint32_t layer, uint32_t expert,
                                uint32_t proj, uint64_t rows, uint64_t cols, uint32_t group,
                                uint32_t sb_dtype, uint8_t* packed, uint8_t* scales,
                                uint8_t* biases)
{
    uint64_t words = rows * cols / 8u;
    uint32_t* pw = (uint32_t*)packed;
    for (uint64_t w = 0; w < words; ++w) {
        uint32_t v = pbm_q4_word(seed, tensor, layer, expert, proj, w);
        memcpy(pw + w, &v, 4);
    }
    uint64_t groups = rows * (cols / group);
    for (uint64_t j = 0; j < groups; ++j) {
        uint16_t s = pbm_q4_scale_bias(seed, tensor, layer, expert, proj, 1u, j, sb_dtype);
        uint16_t b = pbm_q4_scale_bias(seed, tensor, layer, expert, proj, 2u, j, sb_dtype);
        memcpy(scales + 2 * j, &s, 2);
        memcpy(biases + 2 * j, &b, 2);
    }
}

/* Fill `count` fixed-slot Q4 experts (experts first_expert..) laid out
 * back to back with stride expert_bytes.  offsets: the 9 component offsets
 * GateW, GateS, GateB, UpW, UpS, UpB, DownW, DownS, DownB. */
PBM_EXPORT void pbm_fill_q4_experts(uint64_t seed, uint32_t tensor, uint32_t layer,
                                    uint32_t first_expert, uint32_t count, uint32_t hidden,
                                    uint32_t intermediate, uint32_t group, uint32_t sb_dtype,
                                    const uint64_t* offsets, uint64_t expert_bytes,
                                    uint8_t* slots, int threads)
{
    (void)threads;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic, 1)
#endif
    for (uint32_t i = 0; i < count; ++i) {
        uint8_t* slot = slots + (uint64_t)i * expert_bytes;
        memset(slot, 0, expert_bytes);
        for (uint32_t p = 0; p < 3; ++p) {
            uint64_t rows = p == 2 ? hidden : intermediate;
            uint64_t cols = p == 2 ? intermediate : hidden;
            pbm_fill_projection(seed, tensor, layer, first_expert + i, p, rows, cols, group,
                                sb_dtype, slot + offsets[3 * p], slot + offsets[3 * p + 1],
                                slot + offsets[3 * p + 2]);
        }
    }
}

static double pbm_unit53_open(uint64_t v) /* (0, 1] */
{
    return ((double)(v >> 11) + 1.0) * 1.1102230246251565e-16;
}

static double pbm_unit53(uint64_t v) /* [0, 1) */
{
    return (double)(v >> 11) * 1.1102230246251565e-16;
}

/* Standard normal number n of a stream: Box-Muller on two draws. */
static double pbm_normal(uint64_t key, uint64_t n)
{
    double u1 = pbm_unit53_open(pbm_draw(key, 2 * n));
    double u2 = pbm_unit53(pbm_draw(key, 2 * n + 1));
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

/* n binary16 values ~ N(0, sigma^2) (round to nearest even). */
PBM_EXPORT void pbm_fill_normal_f16(uint64_t seed, uint32_t tensor, uint32_t layer,
                                    uint32_t expert, uint32_t part, uint64_t n, double sigma,
                                    uint16_t* out, int threads)
{
    uint64_t key = pbm_stream_key(seed, tensor, layer, expert, part);
    (void)threads;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
    for (uint64_t i = 0; i < n; ++i)
        out[i] = pbm_f32_to_f16((float)(sigma * pbm_normal(key, i)));
}

PBM_EXPORT void pbm_f16_to_f32_array(const uint16_t* in, uint64_t n, float* out)
{
    for (uint64_t i = 0; i < n; ++i)
        out[i] = pbm_f16_to_f32(in[i]);
}

PBM_EXPORT void pbm_f32_to_f16_array(const float* in, uint64_t n, uint16_t* out)
{
    for (uint64_t i = 0; i < n; ++i)
        out[i] = pbm_f32_to_f16(in[i]);
}

PBM_EXPORT void pbm_f32_to_bf16_array(const float* in, uint64_t n, uint16_t* out)
{
    for (uint64_t i = 0; i < n; ++i)
        out[i] = pbm_f32_to_bf16(in[i]);
}

/* n f32 values ~ U(lo, lo+width) with 24 random bits each. */
PBM_EXPORT void pbm_fill_uniform_f32(uint64_t seed, uint32_t tensor, uint32_t layer,
                                     uint32_t expert, uint32_t part, uint64_t n, float lo,
                                     float width, float* out)
{
    uint64_t key = pbm_stream_key(seed, tensor, layer, expert, part);
    for (uint64_t i = 0; i < n; ++i)
        out[i] = pbm_uniform(pbm_draw(key, i), lo, width);
}

/* Drawn router logits with a Zipf(s) expert load (the C3 prefill workload):
 * logits[t][e] = 0.1*N(0,1) + 4*[e in S_t], where S_t holds k distinct
 * experts drawn with P(rank r) ~ r^-s over a seeded permutation of ids.
 * The continuous noise keeps exact ties away.  hist (optional) receives the
 * per-expert selection counts. */
PBM_EXPORT int pbm_drawn_logits_zipf(uint64_t seed, uint32_t layer, uint32_t tokens,
                                     uint32_t experts, uint32_t k, double s, float* logits,
                                     uint32_t* hist)
{
    if (k > experts || experts == 0)
        return -1;
    uint32_t* perm = (uint32_t*)malloc(sizeof(uint32_t) * experts);
    double* cdf = (double*)malloc(sizeof(double) * experts);
    unsigned char* chosen = (unsigned char*)malloc(experts);
    if (!perm || !cdf || !chosen) {
        free(perm), free(cdf), free(chosen);
        return -1;
    }
    uint64_t pkey = pbm_stream_key(seed, PBM_T_LOGITS, layer, 0xFFFFFFFFu, 0);
    for (uint32_t e = 0; e < experts; ++e)
        perm[e] = e;
    for (uint32_t e = experts - 1; e > 0; --e) { /* Fisher-Yates */
        uint32_t j = (uint32_t)(pbm_draw(pkey, e) % (uint64_t)(e + 1));
        uint32_t t = perm[e];
        perm[e] = perm[j];
        perm[j] = t;
    }
    double total = 0.0;
    for (uint32_t r = 0; r < experts; ++r) {
        total += pow((double)(r + 1), -s);
        cdf[r] = total;
    }
    if (hist)
        memset(hist, 0, sizeof(uint32_t) * experts);
    for (uint32_t t = 0; t < tokens; ++t) {
        uint64_t nkey = pbm_stream_key(seed, PBM_T_LOGITS, layer, t, 1);
        uint64_t zkey = pbm_stream_key(seed, PBM_T_LOGITS, layer, t, 2);
        memset(chosen, 0, experts);
        uint64_t draw = 0;
        for (uint32_t got = 0; got < k;) {
            double u = pbm_unit53(pbm_draw(zkey, draw++)) * total;
            uint32_t lo = 0, hi = experts - 1;
            while (lo < hi) {
                uint32_t mid = (lo + hi) / 2;
                if (cdf[mid] > u)
                    hi = mid;
                else
                    lo = mid + 1;
            }
            uint32_t e = perm[lo];
            if (!chosen[e]) {
                chosen[e] = 1;
                ++got;
            }
        }
        for (uint32_t e = 0; e < experts; ++e) {
            double v = 0.1 * pbm_normal(nkey, e) + (chosen[e] ? 4.0 : 0.0);
            logits[(uint64_t)t * experts + e] = (float)v;
            if (hist && chosen[e])
                hist[e]++;
        }
    }
    free(perm), free(cdf), free(chosen);
    return 0;
}
