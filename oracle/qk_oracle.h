/*
 * qk_oracle.h - CPU restatement of inferencer.cu's Q4_K / Q6_K decode, GEMV,
 * INT8-mode and decode-step semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the test oracle: only tests/, the
 * smoke() entry of __graft_entry__.py and the cpu_baseline leg of bench.py
 * load it.  The product (libqk.so) never links, calls or falls back to it.
 *
 * Every function cites the reference lines it restates (inferencer.cu:N).
 * How each one is pinned (tests/test_oracle_*.py):
 *   oq_f16_to_f32        all 65,536 half patterns against numpy's float16.
 *   oq_q4k_* / oq_q6k_*  hand-built known-answer blocks (closed forms), the
 *                        published GGML dequantize_row_q4_K/q6_K loop
 *                        structure restated independently in numpy, and
 *                        every fp16 d pattern.
 *   oq_gemv_f64          numpy float64 matmul of the dequantized matrix,
 *                        one-hot / all-ones / 2^k-scaling invariants.
 *   oq_gemv_f32_ref      tolerance against oq_gemv_f64 (the fp32 lane order
 *                        and nvcc's FMA contraction cannot be pinned bitwise).
 *   oq_quantize_x32      numpy closed form (IEEE divide, round-half-even,
 *                        clamp), bit-exact.
 *   oq_gemv_i8_f64 /     numpy int64 sub-block dots of the same codes, exact;
 *   oq_subblock_dots_i8  the float combine against a numpy float64 combine.
 *   step ops             torch float64 library routines (softmax, matmul,
 *                        rsqrt) and closed forms (rope at pos 0 is identity,
 *                        rotation preserves pair norms).
 *   oq_llama_*           a vectorised torch float64 restatement of the step
 *                        order on a small configuration.
 */
#ifndef QK_ORACLE_H
#define QK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OQ_F32 = 0, OQ_F16 = 1, OQ_Q4_K = 12, OQ_Q6_K = 14 };

float oq_f16_to_f32(uint16_t h);
int oq_block_bytes(int type);
void oq_q4k_scale_min(const uint8_t *scales, int sub, int *scale, int *minimum);
float oq_q4k_value(const uint8_t *block, int i);
float oq_q6k_value(const uint8_t *block, int i);

int oq_dequant_rows(int type, const uint8_t *w, float *out, int64_t cols, int64_t row0, int64_t nrows);
int oq_embedding(int type, const uint8_t *w, const int32_t *tokens, int64_t n_tokens,
                 float *out, int64_t cols);

/* FP32-mode GEMV.  y[t*ldy + r] = sum_c W[r][c] * x[t*ldx + c], exact fp32
   dequantized weights, accumulated in fp64. */
int oq_gemv_f64(int type, const uint8_t *w, const float *x, int64_t ldx, double *y, int64_t ldy,
                int64_t cols, int64_t rows, int64_t n_tokens);
/* The reference's fp32 kernel order (32 lanes, serial blocks, shuffle tree),
   row-parallel with OpenMP.  This is the CPU baseline. */
int oq_gemv_f32_ref(int type, const uint8_t *w, const float *x, float *y, int64_t cols, int64_t rows);

/* INT8 mode. */
void oq_quantize_x32(const float *x, int8_t *xq, float *xscale, int64_t n);
int oq_subblock_dots_i8(int type, const uint8_t *w, const int8_t *xq, int32_t *dots,
                        int32_t *xsums, int64_t cols, int64_t rows);
int oq_gemv_i8_f64(int type, const uint8_t *w, const int8_t *xq, const float *xscale, double *y,
                   int64_t cols, int64_t rows);

/* Decode-step operations, fp64 activations. */
void oq_rmsnorm(const double *x, const float *weight, double *out, int64_t n, double eps);
void oq_rope_tables(float *cosine, float *sine, int context, int head_dim, float theta);
void oq_rope(double *v, int64_t n, const float *cosine, const float *sine, int pos, int head_dim);
void oq_attention(const double *q, const double *key_cache, const double *value_cache, double *out,
                  int pos, int heads, int kv_heads, int head_dim);
void oq_silu_mul(double *gate, const double *up, int64_t n);
int64_t oq_argmax_f64(const double *v, int64_t n);
int64_t oq_argmax_f32(const float *v, int64_t n);

typedef struct oq_llama_config {
    int dim, layers, heads, kv_heads, hidden, vocab, context;
    float eps, rope_theta;
} oq_llama_config;

typedef struct oq_llama_layer {
    int q_type, k_type, v_type, o_type, gate_type, up_type, down_type;
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *ffn_norm;
} oq_llama_layer;

typedef struct oq_llama_weights {
    int embd_type;               /* Q6_K in the reference (inferencer.cu:1428) */
    const uint8_t *token_embd;
    int output_type;
    const uint8_t *output;       /* NULL: tied to token_embd (inferencer.cu:1521-1522) */
    const float *output_norm;
    const oq_llama_layer *layers;
} oq_llama_weights;

typedef struct oq_llama oq_llama;

oq_llama *oq_llama_create(const oq_llama_config *cfg, const oq_llama_weights *w);
void oq_llama_destroy(oq_llama *m);
/* Copies the first n_positions of each layer from fp32 caches laid out as
   [layer][context][kv_dim] (inferencer.cu:1132-1134, 923). */
int oq_llama_load_cache(oq_llama *m, const float *key_cache, const float *value_cache, int n_positions);
/* One decode step (inferencer.cu:1424-1531).  Writes the fp64 logits when
   logits != NULL and need_logits, and the greedy token. */
/* INT8 GEMV modes of the decode step (use_dp4a for Q4_K, use_q6_dp4a for
   Q6_K; both off after create). */
void oq_llama_set_int8(oq_llama *m, int q4k_int8, int q6k_int8);
int oq_llama_forward(oq_llama *m, int token, int pos, int need_logits, double *logits, int *next_token);

/* omp_get_max_threads() of this library's OpenMP runtime: the threads its
   parallel loops use (the CPU baseline reports it). */
int oq_omp_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif
