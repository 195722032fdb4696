/*
 * qk_synth.c - seeded synthetic inputs (SplitMix64, Box-Muller, software
 * double->fp16 RNE).  The generator is specified in qk_synth.h.
 */
#include "qk_synth.h"

#include <math.h>
#include <string.h>

void qs_rng_init(qs_rng *rng, uint64_t seed, uint64_t stream) {
    rng->state = seed ^ (stream * 0xD1B54A32D192ED03ULL);
    (void)qs_next_u64(rng);
}

uint64_t qs_next_u64(qs_rng *rng) {
    uint64_t z = (rng->state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

double qs_uniform01(qs_rng *rng) {
    return (double)(qs_next_u64(rng) >> 11) * 0x1.0p-53;
}

double qs_normal(qs_rng *rng) {
    /* u1 in (0, 1] keeps the logarithm finite. */
    double u1 = (double)((qs_next_u64(rng) >> 11) + 1) * 0x1.0p-53;
    double u2 = (double)(qs_next_u64(rng) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

int64_t qs_uniform_int(qs_rng *rng, int64_t lo, int64_t hi) {
    uint64_t span = (uint64_t)(hi - lo) + 1u;
    /* Multiply-shift on the top 32 bits; spans here are far below 2^32. */
    uint64_t r = qs_next_u64(rng) >> 32;
    return lo + (int64_t)((r * span) >> 32);
}

uint16_t qs_f64_to_f16(double value) {
    uint64_t bits;
    memcpy(&bits, &value, sizeof bits);
    uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
    uint64_t mag = bits & 0x7FFFFFFFFFFFFFFFULL;
    if (mag >= 0x7FF0000000000000ULL)               /* inf or nan */
        return (uint16_t)(sign | (mag > 0x7FF0000000000000ULL ? 0x7E00u : 0x7C00u));
    int exp = (int)(mag >> 52) - 1023;
    if (exp < -25) return sign;                     /* below half of the smallest subnormal */
    uint64_t mant = (mag & 0x000FFFFFFFFFFFFFULL) | 0x0010000000000000ULL;
    if (exp >= -14) {                               /* normal half candidate */
        const int shift = 42;                       /* 52 fraction bits -> 10 */
        uint64_t q = mant >> shift;
        uint64_t rem = mant & ((1ULL << shift) - 1);
        uint64_t half = 1ULL << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        if (q == 2048) { q = 1024; ++exp; }
        if (exp > 15) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | ((uint16_t)(exp + 15) << 10) | (uint16_t)(q & 0x3FFu));
    }
    /* Subnormal half: units of 2^-24.  A carry into 1024 encodes the smallest
       normal, which is exactly the right bit pattern. */
    int shift = 28 - exp;                           /* 43..53 */
    uint64_t q = mant >> shift;
    uint64_t rem = mant & ((1ULL << shift) - 1);
    uint64_t half = 1ULL << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return (uint16_t)(sign | (uint16_t)q);
}

void qs_f64_to_f16_array(const double *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = qs_f64_to_f16(src[i]);
}

static void put_u64_le(uint8_t *dst, uint64_t v, int nbytes) {
    for (int i = 0; i < nbytes; ++i) dst[i] = (uint8_t)(v >> (8 * i));
}

static void put_f16(uint8_t *dst, uint16_t h) {
    dst[0] = (uint8_t)(h & 0xFF);
    dst[1] = (uint8_t)(h >> 8);
}

void qs_fill_bytes(uint8_t *dst, int64_t n, uint64_t seed, uint64_t stream) {
    qs_rng rng;
    qs_rng_init(&rng, seed, stream);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) put_u64_le(dst + i, qs_next_u64(&rng), 8);
    if (i < n) put_u64_le(dst + i, qs_next_u64(&rng), (int)(n - i));
}

void qs_fill_q4k(uint8_t *dst, int64_t n_blocks, uint64_t seed, uint64_t stream, double d_sigma) {
    qs_rng rng;
    qs_rng_init(&rng, seed, stream);
    for (int64_t b = 0; b < n_blocks; ++b) {
        uint8_t *blk = dst + b * 144;
        put_f16(blk + 0, qs_f64_to_f16(fabs(qs_normal(&rng)) * d_sigma));   /* d */
        put_f16(blk + 2, qs_f64_to_f16(fabs(qs_normal(&rng)) * d_sigma));   /* dmin */
        put_u64_le(blk + 4, qs_next_u64(&rng), 8);                          /* scales[0..7] */
        put_u64_le(blk + 12, qs_next_u64(&rng), 4);                         /* scales[8..11] */
        for (int i = 0; i < 128; i += 8) put_u64_le(blk + 16 + i, qs_next_u64(&rng), 8);
    }
}

void qs_fill_q6k(uint8_t *dst, int64_t n_blocks, uint64_t seed, uint64_t stream, double d_sigma) {
    qs_rng rng;
    qs_rng_init(&rng, seed, stream);
    for (int64_t b = 0; b < n_blocks; ++b) {
        uint8_t *blk = dst + b * 210;
        for (int i = 0; i < 192; i += 8) put_u64_le(blk + i, qs_next_u64(&rng), 8);  /* ql, qh */
        for (int s = 0; s < 16; ++s)                                                 /* int8 scales */
            blk[192 + s] = (uint8_t)(int8_t)((int)(qs_next_u64(&rng) >> 58) - 32);
        put_f16(blk + 208, qs_f64_to_f16(fabs(qs_normal(&rng)) * d_sigma));         /* d */
    }
}

void qs_fill_normal_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream, double mean, double sigma) {
    qs_rng rng;
    qs_rng_init(&rng, seed, stream);
    for (int64_t i = 0; i < n; ++i) dst[i] = (float)(mean + sigma * qs_normal(&rng));
}

void qs_fill_uniform_i32(int32_t *dst, int64_t n, uint64_t seed, uint64_t stream, int32_t lo, int32_t hi) {
    qs_rng rng;
    qs_rng_init(&rng, seed, stream);
    for (int64_t i = 0; i < n; ++i) dst[i] = (int32_t)qs_uniform_int(&rng, lo, hi);
}
