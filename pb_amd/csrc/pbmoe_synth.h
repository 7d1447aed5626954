/*
 * Seeded synthetic inputs for the MoE block, shared bit-for-bit by the host
 * generator (synth_host.c), the device fill kernel (pbmoe_kernels.hip) and
 * every test and benchmark.
 *
 * The generator is counter-based: element n of a stream is
 *     mix64(key + (n + 1) * GAMMA)
 * i.e. SplitMix64 evaluated at an arbitrary position, with the stream key
 * derived from (seed, tensor kind, layer, expert, part).  Any element can be
 * produced independently, so a GPU kernel and a CPU loop produce identical
 * bytes without sharing state.
 *
 * Only integer arithmetic and explicitly fused fmaf() are used for uniform
 * values, so the device and host results are bit-identical (fmaf is
 * correctly rounded on both).  Normal draws (router weights, activations)
 * use Box-Muller in double precision and are generated on the host only.
 */
#ifndef PBMOE_SYNTH_H
#define PBMOE_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define PBM_HD __host__ __device__ static inline
#else
#define PBM_HD static inline
#endif

#define PBM_GAMMA 0x9E3779B97F4A7C15ull

/* Tensor kinds used in stream keys. */
enum {
    PBM_T_EXPERT = 1,      /* routed expert slot components          */
    PBM_T_ROUTER = 2,      /* router projection [E][H]               */
    PBM_T_SHARED = 3,      /* shared expert slot components          */
    PBM_T_SHARED_GATE = 4, /* shared expert sigmoid gate [1][H]      */
    PBM_T_INPUT = 5,       /* normed hidden input x [T][H]           */
    PBM_T_RESIDUAL = 6,    /* residual [T][H]                        */
    PBM_T_ROUTER_BIAS = 7, /* per-expert selection bias [E]          */
    PBM_T_LOGITS = 8       /* drawn router logits (prefill config)   */
};

/* Parts within an expert slot: projection p (0 gate, 1 up, 2 down) times
 * component c (0 packed nibbles, 1 scale, 2 bias): part = 3p + c. */

PBM_HD uint64_t pbm_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

PBM_HD uint64_t pbm_stream_key(uint64_t seed, uint32_t tensor, uint32_t layer,
                               uint32_t expert, uint32_t part)
{
    uint64_t k = pbm_mix64(seed + PBM_GAMMA);
    k = pbm_mix64(k ^ (((uint64_t)tensor << 32) | layer));
    k = pbm_mix64(k ^ (((uint64_t)expert << 32) | part));
    return k;
}

PBM_HD uint64_t pbm_draw(uint64_t key, uint64_t n)
{
    return pbm_mix64(key + (n + 1ull) * PBM_GAMMA);
}

/* Uniform in [0, 1) with 24 random bits: exact in binary32. */
PBM_HD float pbm_unit24(uint64_t v)
{
    return (float)(uint32_t)(v >> 40) * 5.9604644775390625e-08f;
}

/* lo + u * width, one correctly rounded fused operation. */
PBM_HD float pbm_uniform(uint64_t v, float lo, float width)
{
    return __builtin_fmaf(pbm_unit24(v), width, lo);
}

PBM_HD uint32_t pbm_f32_bits(float f)
{
    union { float f; uint32_t u; } c;
    c.f = f;
    return c.u;
}

PBM_HD float pbm_bits_f32(uint32_t u)
{
    union { float f; uint32_t u; } c;
    c.u = u;
    return c.f;
}

/* binary32 -> binary16, round to nearest even, integer-only. */
PBM_HD uint16_t pbm_f32_to_f16(float f)
{
    uint32_t x = pbm_f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf or nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) /* rounds to >= 65520: overflow to inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x33000001u) /* below half the smallest subnormal: zero */
        return (uint16_t)sign;
    uint32_t exp = ax >> 23;
    uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    if (exp < 113) { /* subnormal half */
        uint32_t shift = 126 - exp; /* 14..24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u)))
            q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((exp - 112) << 10) | ((mant >> 13) & 0x3FFu);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))
        q += 1u;
    return (uint16_t)(sign | q);
}

/* binary16 -> binary32 (exact). */
PBM_HD float pbm_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    if (exp == 0x1Fu)
        return pbm_bits_f32(sign | 0x7F800000u | (mant << 13));
    if (exp == 0) {
        if (mant == 0)
            return pbm_bits_f32(sign);
        /* subnormal: mant * 2^-24 is exact in binary32 */
        float v = (float)mant * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return pbm_bits_f32(sign | ((exp + 112u) << 23) | (mant << 13));
}

/* binary32 -> bfloat16, round to nearest even (nan kept quiet). */
PBM_HD uint16_t pbm_f32_to_bf16(float f)
{
    uint32_t x = pbm_f32_bits(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u)
        return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7FFFu + lsb) >> 16);
}

PBM_HD float pbm_bf16_to_f32(uint16_t b)
{
    return pbm_bits_f32((uint32_t)b << 16);
}

/* Scale/bias ranges of the seeded Q4 experts. */
#define PBM_SCALE_LO 0.005f
#define PBM_SCALE_WIDTH 0.015f
#define PBM_BIAS_LO (-0.1f)
#define PBM_BIAS_WIDTH 0.2f

/* Scale or bias element j of projection p, as a 2-byte value of the given
 * dtype (1 = f16, 2 = bf16). */
PBM_HD uint16_t pbm_q4_scale_bias(uint64_t seed, uint32_t tensor, uint32_t layer,
                                  uint32_t expert, uint32_t proj, uint32_t comp,
                                  uint64_t j, uint32_t dtype)
{
    uint64_t key = pbm_stream_key(seed, tensor, layer, expert, proj * 3u + comp);
    float v = comp == 1u ? pbm_uniform(pbm_draw(key, j), PBM_SCALE_LO, PBM_SCALE_WIDTH)
                         : pbm_uniform(pbm_draw(key, j), PBM_BIAS_LO, PBM_BIAS_WIDTH);
    return dtype == 2u ? pbm_f32_to_bf16(v) : pbm_f32_to_f16(v);
}

/* Packed nibble word w of projection p (8 nibbles, column 8w+i at bits 4i). */
PBM_HD uint32_t pbm_q4_word(uint64_t seed, uint32_t tensor, uint32_t layer,
                            uint32_t expert, uint32_t proj, uint64_t w)
{
    uint64_t key = pbm_stream_key(seed, tensor, layer, expert, proj * 3u);
    return (uint32_t)pbm_draw(key, w);
}

#endif
