/*
 * qk_oracle.c - CPU restatement of inferencer.cu's quantized GEMV path.
 * TEST INFRASTRUCTURE ONLY (see qk_oracle.h for who may load it and how each
 * function is pinned).
 */
#include "qk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 -- */

/* Exact IEEE binary16 -> binary32, the semantics of __half2float used at
   inferencer.cu:455-456, 477. */
float oq_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                          /* subnormal: renormalise */
            int e = -1;
            do { ++e; man <<= 1; } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

static inline float load_f16(const uint8_t *p) {
    return oq_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

int oq_block_bytes(int type) {
    /* Size rule of inferencer.cu:252-259. */
    return type == OQ_Q4_K ? 144 : type == OQ_Q6_K ? 210 : 0;
}

/* ------------------------------------------------------------- decode -- */

/* inferencer.cu:489-497 */
void oq_q4k_scale_min(const uint8_t *scales, int sub, int *scale, int *minimum) {
    if (sub < 4) {
        *scale = scales[sub] & 63;
        *minimum = scales[sub + 4] & 63;
    } else {
        *scale = (scales[sub + 4] & 15) | ((scales[sub - 4] >> 6) << 4);
        *minimum = (scales[sub + 4] >> 4) | ((scales[sub] >> 6) << 4);
    }
}

/* inferencer.cu:454-471: w = d*sc*q - dmin*m.  The products are exact in
   fp32, so the single rounding is the subtraction. */
float oq_q4k_value(const uint8_t *block, int i) {
    float d = load_f16(block);
    float dmin = load_f16(block + 2);
    const uint8_t *qs = block + 16;
    int sub = i / 32;
    int q_index = (i / 64) * 32 + (i % 32);
    int q = (i % 64) < 32 ? (qs[q_index] & 15) : (qs[q_index] >> 4);
    int sc, m;
    oq_q4k_scale_min(block + 4, sub, &sc, &m);
    float dsc = d * (float)sc;
    float dm = dmin * (float)m;
    return dsc * (float)q - dm;
}

/* inferencer.cu:473-487: w = d*scale*(code-32), exact in fp32. */
float oq_q6k_value(const uint8_t *block, int i) {
    const uint8_t *ql = block;
    const uint8_t *qh = block + 128;
    const int8_t *scales = (const int8_t *)(block + 192);
    float d = load_f16(block + 208);
    int group = i / 128, p = i % 128, lane = p % 32, part = p / 32;
    int low = ql[group * 64 + (part % 2) * 32 + lane];
    low = part < 2 ? (low & 15) : (low >> 4);
    int high = (qh[group * 32 + lane] >> (part * 2)) & 3;
    int q = (low | (high << 4)) - 32;
    return d * (float)scales[group * 8 + part * 2 + lane / 16] * (float)q;
}

/* Whole-block forms of oq_q4k_value / oq_q6k_value: the same operations in
   the same order per element (so the same bits), with the block header
   decoded once. */
static void q4k_block(const uint8_t *blk, float *out) {
    float d = load_f16(blk), dmin = load_f16(blk + 2);
    for (int sub = 0; sub < 8; ++sub) {
        int sc, m;
        oq_q4k_scale_min(blk + 4, sub, &sc, &m);
        float dsc = d * (float)sc, dm = dmin * (float)m;
        const uint8_t *q = blk + 16 + (sub / 2) * 32;
        for (int l = 0; l < 32; ++l) {
            int code = (sub & 1) ? (q[l] >> 4) : (q[l] & 15);
            out[sub * 32 + l] = dsc * (float)code - dm;
        }
    }
}

static void q6k_block(const uint8_t *blk, float *out) {
    const int8_t *scales = (const int8_t *)(blk + 192);
    float d = load_f16(blk + 208);
    for (int group = 0; group < 2; ++group)
        for (int part = 0; part < 4; ++part)
            for (int lane = 0; lane < 32; ++lane) {
                int low = blk[group * 64 + (part % 2) * 32 + lane];
                low = part < 2 ? (low & 15) : (low >> 4);
                int high = (blk[128 + group * 32 + lane] >> (part * 2)) & 3;
                int q = (low | (high << 4)) - 32;
                out[group * 128 + part * 32 + lane] = d * (float)scales[group * 8 + part * 2 + lane / 16] * (float)q;
            }
}

static void dequant_row(int type, const uint8_t *row, float *out, int64_t cols) {
    int bpb = oq_block_bytes(type);
    for (int64_t b = 0; b < cols / 256; ++b) {
        if (type == OQ_Q4_K)
            q4k_block(row + b * bpb, out + b * 256);
        else
            q6k_block(row + b * bpb, out + b * 256);
    }
}

static int check_shape(int type, int64_t cols, int64_t rows) {
    if (type != OQ_Q4_K && type != OQ_Q6_K) return -1;
    if (cols <= 0 || cols % 256 || rows < 0) return -1;
    return 0;
}

int oq_dequant_rows(int type, const uint8_t *w, float *out, int64_t cols, int64_t row0, int64_t nrows) {
    if (check_shape(type, cols, nrows) || row0 < 0) return -1;
    int64_t row_bytes = cols / 256 * oq_block_bytes(type);
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nrows; ++r)
        dequant_row(type, w + (row0 + r) * row_bytes, out + r * cols, cols);
    return 0;
}

/* inferencer.cu:806-819: out[t][i] = value(row(tokens[t]), i). */
int oq_embedding(int type, const uint8_t *w, const int32_t *tokens, int64_t n_tokens,
                 float *out, int64_t cols) {
    if (check_shape(type, cols, n_tokens)) return -1;
    int64_t row_bytes = cols / 256 * oq_block_bytes(type);
    for (int64_t t = 0; t < n_tokens; ++t)
        dequant_row(type, w + (int64_t)tokens[t] * row_bytes, out + t * cols, cols);
    return 0;
}

/* --------------------------------------------------------- FP32 GEMV -- */

int oq_gemv_f64(int type, const uint8_t *w, const float *x, int64_t ldx, double *y, int64_t ldy,
                int64_t cols, int64_t rows, int64_t n_tokens) {
    if (check_shape(type, cols, rows) || n_tokens < 0) return -1;
    int64_t row_bytes = cols / 256 * oq_block_bytes(type);
    #pragma omp parallel
    {
        float *wrow = (float *)malloc((size_t)cols * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            dequant_row(type, w + r * row_bytes, wrow, cols);
            for (int64_t t = 0; t < n_tokens; ++t) {
                const float *xt = x + t * ldx;
                double acc = 0.0;
                for (int64_t c = 0; c < cols; ++c) acc += (double)wrow[c] * (double)xt[c];
                y[t * ldy + r] = acc;
            }
        }
        free(wrow);
    }
    return 0;
}

/* dot_q4_block, inferencer.cu:500-516, for one of 32 lanes.  nvcc contracts
   "sum += w * x" into an FMA; fmaf restates that. */
static float ref_dot_q4_lane(const uint8_t *blk, const float *x, int lane) {
    float d = load_f16(blk), dmin = load_f16(blk + 2);
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    float sum = 0.f;
    for (int group = 0; group < 4; ++group) {
        int s0, m0, s1, m1;
        oq_q4k_scale_min(scales, group * 2, &s0, &m0);
        oq_q4k_scale_min(scales, group * 2 + 1, &s1, &m1);
        int quant = qs[group * 32 + lane];
        float w0 = d * (float)s0 * (float)(quant & 15) - dmin * (float)m0;
        sum = fmaf(w0, x[group * 64 + lane], sum);
        float w1 = d * (float)s1 * (float)(quant >> 4) - dmin * (float)m1;
        sum = fmaf(w1, x[group * 64 + 32 + lane], sum);
    }
    return sum;
}

/* dot_q6_block, inferencer.cu:572-595 (integer scale*code, one d per block). */
static float ref_dot_q6_lane_raw(const uint8_t *blk, const float *x, int lane) {
    const uint8_t *low = blk, *high = blk + 128;
    const int8_t *scales = (const int8_t *)(blk + 192);
    float sum = 0.f;
    for (int group = 0; group < 2; ++group) {
        int a = low[group * 64 + lane], b = low[group * 64 + 32 + lane], h = high[group * 32 + lane];
        int q0 = ((a & 15) | ((h & 3) << 4)) - 32;
        int q1 = ((b & 15) | (((h >> 2) & 3) << 4)) - 32;
        int q2 = ((a >> 4) | (((h >> 4) & 3) << 4)) - 32;
        int q3 = ((b >> 4) | (((h >> 6) & 3) << 4)) - 32;
        int offset = group * 128 + lane, s = group * 8 + lane / 16;
        sum = fmaf((float)(scales[s] * q0), x[offset], sum);
        sum = fmaf((float)(scales[s + 2] * q1), x[offset + 32], sum);
        sum = fmaf((float)(scales[s + 4] * q2), x[offset + 64], sum);
        sum = fmaf((float)(scales[s + 6] * q3), x[offset + 96], sum);
    }
    return sum;
}

/* gemv_quant<TYPE>, inferencer.cu:645-661: 32 lanes walk the blocks of one
   row, then a __shfl_down_sync tree 16..1 leaves the total in lane 0. */
static float ref_gemv_row(int type, const uint8_t *row, const float *x, int64_t nb) {
    float lane_sum[32];
    int bpb = oq_block_bytes(type);
    for (int lane = 0; lane < 32; ++lane) {
        float sum = 0.f;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *blk = row + b * bpb;
            if (type == OQ_Q4_K) {
                sum += ref_dot_q4_lane(blk, x + b * 256, lane);
            } else {
                float d = load_f16(blk + 208);
                sum = fmaf(d, ref_dot_q6_lane_raw(blk, x + b * 256, lane), sum);
            }
        }
        lane_sum[lane] = sum;
    }
    for (int delta = 16; delta > 0; delta /= 2)
        for (int lane = 0; lane < delta; ++lane) lane_sum[lane] += lane_sum[lane + delta];
    return lane_sum[0];
}

int oq_gemv_f32_ref(int type, const uint8_t *w, const float *x, float *y, int64_t cols, int64_t rows) {
    if (check_shape(type, cols, rows)) return -1;
    int64_t nb = cols / 256, row_bytes = nb * oq_block_bytes(type);
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) y[r] = ref_gemv_row(type, w + r * row_bytes, x, nb);
    return 0;
}

/* ---------------------------------------------------------- INT8 mode -- */

/* quantize_x32_cuda, inferencer.cu:544-556: per 32 values, scale =
   amax/127 (1 when amax is 0), xq = clamp(rne(x/scale), -127, 127). */
void oq_quantize_x32(const float *x, int8_t *xq, float *xscale, int64_t n) {
    for (int64_t g = 0; g * 32 < n; ++g) {
        float amax = 0.f;
        for (int64_t i = g * 32; i < g * 32 + 32 && i < n; ++i) amax = fmaxf(amax, fabsf(x[i]));
        float scale = amax > 0.f ? amax / 127.f : 1.f;
        xscale[g] = scale;
        for (int64_t i = g * 32; i < g * 32 + 32 && i < n; ++i) {
            float r = rintf(x[i] / scale);        /* round half to even */
            int v = (int)r;
            xq[i] = (int8_t)(v < -127 ? -127 : v > 127 ? 127 : v);
        }
    }
}

static int q4_code(const uint8_t *blk, int i) {
    const uint8_t *qs = blk + 16;
    int q_index = (i / 64) * 32 + (i % 32);
    return (i % 64) < 32 ? (qs[q_index] & 15) : (qs[q_index] >> 4);
}

static int q6_code(const uint8_t *blk, int i) {
    int group = i / 128, p = i % 128, lane = p % 32, part = p / 32;
    int low = blk[group * 64 + (part % 2) * 32 + lane];
    low = part < 2 ? (low & 15) : (low >> 4);
    int high = (blk[128 + group * 32 + lane] >> (part * 2)) & 3;
    return (low | (high << 4)) - 32;
}

/* Exact integer partials of dot_q4_block_dp4a (inferencer.cu:520-542) and
   dot_q6_block_dp4a (inferencer.cu:613-643), summed over each sub-block:
   Q4_K: dots[r][b*8+s] = sum code*xq over the 32-value sub-block s,
         xsums[b*8+s]   = sum xq over it (the min term);
   Q6_K: dots[r][b*16+j] = sum (code-32)*xq over the 16-value sub-block j. */
int oq_subblock_dots_i8(int type, const uint8_t *w, const int8_t *xq, int32_t *dots,
                        int32_t *xsums, int64_t cols, int64_t rows) {
    if (check_shape(type, cols, rows)) return -1;
    int64_t nb = cols / 256, bpb = oq_block_bytes(type), row_bytes = nb * bpb;
    int sub_len = type == OQ_Q4_K ? 32 : 16, nsub = 256 / sub_len;
    if (xsums)
        for (int64_t s = 0; s < nb * nsub; ++s) {
            int32_t acc = 0;
            for (int i = 0; i < sub_len; ++i) acc += xq[s * sub_len + i];
            xsums[s] = acc;
        }
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *blk = w + r * row_bytes + b * bpb;
            for (int s = 0; s < nsub; ++s) {
                int32_t acc = 0;
                for (int i = s * sub_len; i < (s + 1) * sub_len; ++i)
                    acc += (type == OQ_Q4_K ? q4_code(blk, i) : q6_code(blk, i)) * xq[b * 256 + i];
                dots[(r * nb + b) * nsub + s] = acc;
            }
        }
    return 0;
}

/* INT8-mode row result with the float combine done in fp64:
   Q4_K: sum_b sum_s (d*sc*dot - dmin*m*sum_xq) * xscale[b*8+s]
   Q6_K: sum_b sum_j d*scale[j]*dot * xscale[b*8+j/2]. */
int oq_gemv_i8_f64(int type, const uint8_t *w, const int8_t *xq, const float *xscale, double *y,
                   int64_t cols, int64_t rows) {
    if (check_shape(type, cols, rows)) return -1;
    int64_t nb = cols / 256, bpb = oq_block_bytes(type), row_bytes = nb * bpb;
    int nsub = type == OQ_Q4_K ? 8 : 16;
    int32_t *xs = (int32_t *)malloc((size_t)(nb * nsub) * sizeof(int32_t));
    int32_t *dots = (int32_t *)malloc((size_t)(rows * nb * nsub) * sizeof(int32_t));
    oq_subblock_dots_i8(type, w, xq, dots, xs, cols, rows);
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        double acc = 0.0;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *blk = w + r * row_bytes + b * bpb;
            const int32_t *dt = dots + (r * nb + b) * nsub;
            if (type == OQ_Q4_K) {
                double d = load_f16(blk), dmin = load_f16(blk + 2);
                for (int s = 0; s < 8; ++s) {
                    int sc, m;
                    oq_q4k_scale_min(blk + 4, s, &sc, &m);
                    acc += (d * sc * dt[s] - dmin * m * xs[b * 8 + s]) * (double)xscale[b * 8 + s];
                }
            } else {
                double d = load_f16(blk + 208);
                const int8_t *scales = (const int8_t *)(blk + 192);
                for (int j = 0; j < 16; ++j)
                    acc += d * scales[j] * (double)dt[j] * (double)xscale[b * 8 + j / 2];
            }
        }
        y[r] = acc;
    }
    free(dots);
    free(xs);
    return 0;
}

/* ------------------------------------------------------- step kernels -- */

/* rmsnorm_cuda, inferencer.cu:821-834: out = x / sqrt(mean(x^2) + eps) * w. */
void oq_rmsnorm(const double *x, const float *weight, double *out, int64_t n, double eps) {
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) ss += x[i] * x[i];
    double scale = 1.0 / sqrt(ss / (double)n + eps);
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] * scale * (double)weight[i];
}

/* FastRunner constructor tables, inferencer.cu:1218-1226, generalised from
   64 to head_dim/2 frequencies: float powf / cosf / sinf exactly as there. */
void oq_rope_tables(float *cosine, float *sine, int context, int head_dim, float theta) {
    int half = head_dim / 2;
    float *freq = (float *)malloc((size_t)half * sizeof(float));
    for (int i = 0; i < half; ++i) freq[i] = powf(theta, -2.f * (float)i / (float)head_dim);
    for (int pos = 0; pos < context; ++pos)
        for (int i = 0; i < half; ++i) {
            float angle = (float)pos * freq[i];
            cosine[(int64_t)pos * half + i] = cosf(angle);
            sine[(int64_t)pos * half + i] = sinf(angle);
        }
    free(freq);
}

/* rope_cuda, inferencer.cu:906-917: rotate adjacent pairs (2p, 2p+1) with
   frequency p mod head_dim/2. */
void oq_rope(double *v, int64_t n, const float *cosine, const float *sine, int pos, int head_dim) {
    int half = head_dim / 2;
    for (int64_t pair = 0; pair < n / 2; ++pair) {
        int f = (int)(pair % half);
        double c = cosine[(int64_t)pos * half + f], s = sine[(int64_t)pos * half + f];
        double a = v[2 * pair], b = v[2 * pair + 1];
        v[2 * pair] = a * c - b * s;
        v[2 * pair + 1] = a * s + b * c;
    }
}

/* attention_cuda, inferencer.cu:981-1009: per query head, softmax over
   positions 0..pos of q.k/sqrt(head_dim), GQA kv_head = head/group.  Caches
   are one layer, [position][kv_dim]. */
void oq_attention(const double *q, const double *key_cache, const double *value_cache, double *out,
                  int pos, int heads, int kv_heads, int head_dim) {
    int group = heads / kv_heads, kv_dim = kv_heads * head_dim;
    double inv = 1.0 / sqrt((double)head_dim);
    double *score = (double *)malloc((size_t)(pos + 1) * sizeof(double));
    for (int h = 0; h < heads; ++h) {
        int kvh = h / group;
        const double *qh = q + (int64_t)h * head_dim;
        double mx = -INFINITY;
        for (int t = 0; t <= pos; ++t) {
            const double *k = key_cache + (int64_t)t * kv_dim + (int64_t)kvh * head_dim;
            double dot = 0.0;
            for (int i = 0; i < head_dim; ++i) dot += qh[i] * k[i];
            score[t] = dot * inv;
            if (score[t] > mx) mx = score[t];
        }
        double den = 0.0;
        for (int t = 0; t <= pos; ++t) { score[t] = exp(score[t] - mx); den += score[t]; }
        for (int i = 0; i < head_dim; ++i) {
            double acc = 0.0;
            for (int t = 0; t <= pos; ++t)
                acc += score[t] * value_cache[(int64_t)t * kv_dim + (int64_t)kvh * head_dim + i];
            out[(int64_t)h * head_dim + i] = acc / den;
        }
    }
    free(score);
}

/* silu_cuda, inferencer.cu:1053-1056: g = g / (1 + exp(-g)) * u. */
void oq_silu_mul(double *gate, const double *up, int64_t n) {
    for (int64_t i = 0; i < n; ++i) gate[i] = gate[i] / (1.0 + exp(-gate[i])) * up[i];
}

/* argmax_blocks_cuda + argmax_final_cuda, inferencer.cu:1063-1099: the
   strict '>' in both trees keeps the lowest index among equal maxima. */
int64_t oq_argmax_f64(const double *v, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

int64_t oq_argmax_f32(const float *v, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

/* ------------------------------------------------------- decode step -- */

struct oq_llama {
    oq_llama_config cfg;
    oq_llama_weights w;
    oq_llama_layer *layers;
    int head_dim, kv_dim;
    float *cosine, *sine;
    double *key_cache, *value_cache;     /* [layer][context][kv_dim] */
    double *x, *xn, *q, *k, *v, *attn, *tmp, *gate, *up;
    int int8_q4k, int8_q6k;              /* the reference's use_dp4a / use_q6_dp4a */
};

oq_llama *oq_llama_create(const oq_llama_config *cfg, const oq_llama_weights *w) {
    if (cfg->heads <= 0 || cfg->kv_heads <= 0 || cfg->dim % cfg->heads ||
        cfg->heads % cfg->kv_heads || cfg->dim % 256 || cfg->hidden % 256)
        return NULL;
    oq_llama *m = (oq_llama *)calloc(1, sizeof *m);
    m->cfg = *cfg;
    m->w = *w;
    m->layers = (oq_llama_layer *)malloc((size_t)cfg->layers * sizeof(oq_llama_layer));
    memcpy(m->layers, w->layers, (size_t)cfg->layers * sizeof(oq_llama_layer));
    m->w.layers = m->layers;
    m->head_dim = cfg->dim / cfg->heads;
    m->kv_dim = m->head_dim * cfg->kv_heads;
    size_t tab = (size_t)cfg->context * (m->head_dim / 2);
    m->cosine = (float *)malloc(tab * sizeof(float));
    m->sine = (float *)malloc(tab * sizeof(float));
    oq_rope_tables(m->cosine, m->sine, cfg->context, m->head_dim, cfg->rope_theta);
    size_t cache = (size_t)cfg->layers * cfg->context * m->kv_dim;
    m->key_cache = (double *)calloc(cache, sizeof(double));
    m->value_cache = (double *)calloc(cache, sizeof(double));
    m->x = (double *)malloc((size_t)cfg->dim * sizeof(double));
    m->xn = (double *)malloc((size_t)cfg->dim * sizeof(double));
    m->q = (double *)malloc((size_t)cfg->dim * sizeof(double));
    m->k = (double *)malloc((size_t)m->kv_dim * sizeof(double));
    m->v = (double *)malloc((size_t)m->kv_dim * sizeof(double));
    m->attn = (double *)malloc((size_t)cfg->dim * sizeof(double));
    m->tmp = (double *)malloc((size_t)cfg->dim * sizeof(double));
    m->gate = (double *)malloc((size_t)cfg->hidden * sizeof(double));
    m->up = (double *)malloc((size_t)cfg->hidden * sizeof(double));
    return m;
}

void oq_llama_destroy(oq_llama *m) {
    if (!m) return;
    free(m->layers); free(m->cosine); free(m->sine);
    free(m->key_cache); free(m->value_cache);
    free(m->x); free(m->xn); free(m->q); free(m->k); free(m->v);
    free(m->attn); free(m->tmp); free(m->gate); free(m->up);
    free(m);
}

int oq_llama_load_cache(oq_llama *m, const float *key_cache, const float *value_cache, int n_positions) {
    if (n_positions < 0 || n_positions > m->cfg.context) return -1;
    for (int l = 0; l < m->cfg.layers; ++l)
        for (int64_t i = 0; i < (int64_t)n_positions * m->kv_dim; ++i) {
            int64_t o = (int64_t)l * m->cfg.context * m->kv_dim + i;
            m->key_cache[o] = key_cache[o];
            m->value_cache[o] = value_cache[o];
        }
    return 0;
}

/* y = W x with fp64 activations; rows in parallel, dequantizing one row at a
   time. */
static void matvec_f64(int type, const uint8_t *w, const double *x, double *y, int64_t cols, int64_t rows) {
    int64_t row_bytes = cols / 256 * oq_block_bytes(type);
    #pragma omp parallel
    {
        float *wrow = (float *)malloc((size_t)cols * sizeof(float));
        #pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            dequant_row(type, w + r * row_bytes, wrow, cols);
            double acc = 0.0;
            for (int64_t c = 0; c < cols; ++c) acc += (double)wrow[c] * x[c];
            y[r] = acc;
        }
        free(wrow);
    }
}

/* INT8 mode of FastGPU::matvec (inferencer.cu:1159-1166): the activation,
   rounded to fp32 as the device holds it, is quantized per 32 values
   (quantize_x32_cuda, 544-556) and the product is the exact integer
   sub-block dots combined in fp64 (oq_gemv_i8_f64). */
static void matvec_i8(int type, const uint8_t *w, const double *x, double *y, int64_t cols, int64_t rows) {
    float *xf = (float *)malloc((size_t)cols * sizeof(float));
    int8_t *xq = (int8_t *)malloc((size_t)cols);
    float *xs = (float *)malloc((size_t)(cols / 32) * sizeof(float));
    for (int64_t i = 0; i < cols; ++i) xf[i] = (float)x[i];
    oq_quantize_x32(xf, xq, xs, cols);
    oq_gemv_i8_f64(type, w, xq, xs, y, cols, rows);
    free(xf);
    free(xq);
    free(xs);
}

static void matvec_mode(const oq_llama *m, int type, const uint8_t *w, const double *x, double *y, int64_t cols,
                        int64_t rows) {
    if ((type == 12 && m->int8_q4k) || (type == 14 && m->int8_q6k))
        matvec_i8(type, w, x, y, cols, rows);
    else
        matvec_f64(type, w, x, y, cols, rows);
}

void oq_llama_set_int8(oq_llama *m, int q4k_int8, int q6k_int8) {
    m->int8_q4k = q4k_int8 != 0;
    m->int8_q6k = q6k_int8 != 0;
}

/* FastRunner::forward, inferencer.cu:1424-1531, with head_dim, heads and the
   frequency count generalised; the GEMVs follow the INT8 modes set by
   oq_llama_set_int8 (FP32 by default). */
int oq_llama_forward(oq_llama *m, int token, int pos, int need_logits, double *logits, int *next_token) {
    const oq_llama_config *c = &m->cfg;
    if (pos < 0 || pos >= c->context || token < 0 || token >= c->vocab) return -1;
    int dim = c->dim, kv = m->kv_dim, hd = m->head_dim;
    {
        float *row = (float *)malloc((size_t)dim * sizeof(float));
        int32_t t = token;
        oq_embedding(m->w.embd_type, m->w.token_embd, &t, 1, row, dim);
        for (int i = 0; i < dim; ++i) m->x[i] = row[i];
        free(row);
    }
    for (int l = 0; l < c->layers; ++l) {
        const oq_llama_layer *L = &m->layers[l];
        double *kc = m->key_cache + (int64_t)l * c->context * kv;
        double *vc = m->value_cache + (int64_t)l * c->context * kv;
        oq_rmsnorm(m->x, L->attn_norm, m->xn, dim, c->eps);
        matvec_mode(m, L->q_type, L->q, m->xn, m->q, dim, dim);
        matvec_mode(m, L->k_type, L->k, m->xn, m->k, dim, kv);
        matvec_mode(m, L->v_type, L->v, m->xn, m->v, dim, kv);
        oq_rope(m->q, dim, m->cosine, m->sine, pos, hd);
        oq_rope(m->k, kv, m->cosine, m->sine, pos, hd);
        memcpy(kc + (int64_t)pos * kv, m->k, (size_t)kv * sizeof(double));
        memcpy(vc + (int64_t)pos * kv, m->v, (size_t)kv * sizeof(double));
        oq_attention(m->q, kc, vc, m->attn, pos, c->heads, c->kv_heads, hd);
        matvec_mode(m, L->o_type, L->o, m->attn, m->tmp, dim, dim);
        for (int i = 0; i < dim; ++i) m->x[i] += m->tmp[i];
        oq_rmsnorm(m->x, L->ffn_norm, m->xn, dim, c->eps);
        matvec_mode(m, L->gate_type, L->gate, m->xn, m->gate, dim, c->hidden);
        matvec_mode(m, L->up_type, L->up, m->xn, m->up, dim, c->hidden);
        oq_silu_mul(m->gate, m->up, c->hidden);
        matvec_mode(m, L->down_type, L->down, m->gate, m->tmp, c->hidden, dim);
        for (int i = 0; i < dim; ++i) m->x[i] += m->tmp[i];
    }
    if (!need_logits) {
        if (next_token) *next_token = -1;
        return 0;
    }
    oq_rmsnorm(m->x, m->w.output_norm, m->xn, dim, c->eps);
    const uint8_t *out_w = m->w.output ? m->w.output : m->w.token_embd;
    int out_type = m->w.output ? m->w.output_type : m->w.embd_type;
    double *lg = logits ? logits : (double *)malloc((size_t)c->vocab * sizeof(double));
    matvec_mode(m, out_type, out_w, m->xn, lg, dim, c->vocab);
    if (next_token) *next_token = (int)oq_argmax_f64(lg, c->vocab);
    if (!logits) free(lg);
    return 0;
}

int oq_omp_max_threads(void) { return omp_get_max_threads(); }
