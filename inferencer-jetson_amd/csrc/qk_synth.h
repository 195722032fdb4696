/*
 * qk_synth.h - seeded synthetic inputs for the Q4_K / Q6_K GEMV workloads.
 *
 * The reference runs real GGUF weights; the workloads here are random-init,
 * so every input (block bytes, activations, token ids, KV contents, context
 * lengths) comes from this one documented generator.  It is host-only C with
 * no GPU dependency, so the CPU tests and the GPU bench build identical
 * inputs from the same (seed, stream) pair.
 *
 * Generator: SplitMix64.  A (seed, stream) pair selects an independent
 * sequence: state0 = seed ^ (stream * 0xD1B54A32D192ED03), and the first
 * output is discarded.  Uniform doubles take the top 53 bits.  Normals use
 * Box-Muller in double (cosine branch only, two draws per normal).  fp16
 * values are produced by a software double->half conversion with
 * round-to-nearest-even (subnormals and overflow to inf handled).
 *
 * Block contents follow the workloads' specification:
 *   Q4_K (144 B): d, dmin = fp16(|N(0, sigma)|); the 12 scale bytes pack sixteen
 *     6-bit scale/min values uniform in 0..63 -- the packing is a bijection
 *     between those 96 bits and the 12 bytes, so the bytes are uniform 0..255;
 *     the 128 quant bytes hold 256 nibbles uniform in 0..15 (uniform bytes).
 *   Q6_K (210 B): ql (128 B) and qh (64 B) uniform random bits; 16 int8
 *     sub-block scales uniform in -32..31; d = fp16(|N(0, sigma)|).
 * Layouts are the GGML super-block layouts the reference decodes
 * (inferencer.cu:453-487).
 */
#ifndef QK_SYNTH_H
#define QK_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qs_rng {
    uint64_t state;
} qs_rng;

void qs_rng_init(qs_rng *rng, uint64_t seed, uint64_t stream);
uint64_t qs_next_u64(qs_rng *rng);
double qs_uniform01(qs_rng *rng);              /* [0, 1) */
double qs_normal(qs_rng *rng);                 /* N(0, 1) */
int64_t qs_uniform_int(qs_rng *rng, int64_t lo, int64_t hi); /* inclusive */
uint16_t qs_f64_to_f16(double value);          /* round to nearest even */

/* Bulk fills.  Each call starts a fresh sequence at (seed, stream). */
void qs_fill_q4k(uint8_t *dst, int64_t n_blocks, uint64_t seed, uint64_t stream, double d_sigma);
void qs_fill_q6k(uint8_t *dst, int64_t n_blocks, uint64_t seed, uint64_t stream, double d_sigma);
void qs_fill_normal_f32(float *dst, int64_t n, uint64_t seed, uint64_t stream, double mean, double sigma);
void qs_fill_uniform_i32(int32_t *dst, int64_t n, uint64_t seed, uint64_t stream, int32_t lo, int32_t hi);
void qs_fill_bytes(uint8_t *dst, int64_t n, uint64_t seed, uint64_t stream);
void qs_f64_to_f16_array(const double *src, uint16_t *dst, int64_t n);

#ifdef __cplusplus
}
#endif

#endif
