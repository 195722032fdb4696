/*
 * qk.h - C ABI of the MI355X (gfx950) Q4_K / Q6_K dequant-GEMV library.
 *
 * Drop-in boundary for inferencer.cu's quantized matrix path.  The reference
 * has no plugin layer: its kernels are launched from FastGPU / FastRunner.
 * Each entry point below names the reference code it replaces.  Conventions
 * shared by every call:
 *
 *  - Weights are GGUF/GGML super-block bytes, rows contiguous, row stride
 *    (cols/256) * 144 B for Q4_K (type 12) and (cols/256) * 210 B for Q6_K
 *    (type 14) (inferencer.cu:252-259, 652).  cols = dims[0] is a multiple
 *    of 256, rows = dims[1] (inferencer.cu:184-185).
 *  - Activations and outputs are fp32.  Outputs are overwritten, never
 *    accumulated (inferencer.cu:660); inputs and outputs must not alias.
 *  - Device pointers only.  Weight bases must be 16-byte aligned (GGUF tensor
 *    data is aligned to general.alignment, default 32: inferencer.cu:270-272);
 *    fp32 activation bases and leading dimensions must keep 16-byte alignment.
 *  - stream is a hipStream_t (NULL selects the null stream).  Calls are
 *    asynchronous, allocate nothing and keep no per-call state: they are
 *    reentrant and may be issued from several host threads.
 *  - Every call validates its arguments on the host before any launch and
 *    returns a qk status (QK_OK = 0).  Nothing throws across the ABI; the
 *    reference's runtime_error texts (inferencer.cu:126-128, 1157-1158) map
 *    to the status plus qk_last_error(), a thread-local message.
 */
#ifndef QK_H
#define QK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage type ids: the GGUF type numbers of storage_name (inferencer.cu:194-202). */
#define QK_TYPE_F32 0
#define QK_TYPE_F16 1
#define QK_TYPE_Q4_K 12
#define QK_TYPE_Q6_K 14
/* A Q6_K matrix in the split layout made by qk_q6k_split (no reference
   counterpart): the same 210 bytes per super-block, each row of nb =
   cols/256 blocks stored as four streams -- ql [nb][128], qh [nb][64],
   scales [nb][16], d [nb] (fp16) -- and padded to a multiple of 16 bytes,
   so every field a kernel reads is 16-byte aligned (in the GGUF layout a
   Q6_K block is only 2-byte aligned at odd block indices).  Accepted
   wherever Q6_K is. */
#define QK_TYPE_Q6_K_SPLIT 114

/* Status codes. */
#define QK_OK 0
#define QK_ERR_INVALID_ARG 1   /* null pointer, negative count, bad leading dimension */
#define QK_ERR_SHAPE 2         /* cols not a positive multiple of 256, rows < 1 */
#define QK_ERR_TYPE 3          /* storage type other than Q4_K / Q6_K / Q6_K split */
#define QK_ERR_ALIGN 4         /* base pointer or leading dimension misaligned */
#define QK_ERR_DEVICE 5        /* HIP runtime error at launch */
#define QK_ERR_LIMIT 6         /* size beyond what the kernels index */
#define QK_ERR_FORMAT 7        /* malformed or unsupported GGUF file */
#define QK_ERR_IO 8            /* file cannot be opened or mapped */

typedef void *qk_stream;

/* ------------------------------------------------------------ utility -- */

/* Status text; replaces the cuda_check / runtime_error messages
   (inferencer.cu:126-128). */
const char *qk_status_string(int status);
/* Detail of the last failing call on this host thread ("" if none). */
const char *qk_last_error(void);
/* Bytes per 256-value super-block (144 / 210; 0 for other types) and bytes of
   a cols x rows tensor: the size rule of inferencer.cu:252-259 (split Q6_K
   rows rounded up to 16 bytes). */
int qk_block_bytes(int type);
int64_t qk_tensor_bytes(int type, int64_t cols, int64_t rows);

/* ------------------------------------------------ FP32 dequant-GEMV -- */

/* Precision of the FP32 entry points (this section, the FP32 step kernels
   that feed them and the FP32 decode drivers): x is carried as 22-bit block
   fixed point per 16 consecutive values, X = rint(x * 2^(21-e)) with e =
   ilogb of the group's largest |x|, so each value is rounded to within
   2^(e-22) -- relative 2^-22 for the group's largest value, coarser for
   values far below it -- and the products and sums that follow are exact
   integer dots plus fp32 combines.  An output therefore differs from the
   reference's fp32 products by at most sum_c |W[r][c]| 2^(e_c - 22) plus
   fp32 rounding (tests/test_gpu_gemv.py pins both terms); on N(0, 1)-like
   activations that is within 1e-6 rel-L2 of an fp64 product.  The
   multi-token forms carry the same 22 bits per 256-column block as fp16
   high / low halves.  The INT8 entry points below follow the reference's
   INT8 arithmetic instead. */

/* y[r] = sum_c W[r][c] * x[c] for r < rows.
   Replaces FastGPU::matvec's FP32 branch (inferencer.cu:1156-1171) and the
   gemv_quant<12|14> kernel (inferencer.cu:645-661) it launches. */
int qk_gemv_f32(int type, const void *w, const float *x, float *y, int cols, int rows,
                qk_stream stream);

/* One matrix of a fused launch. */
typedef struct qk_matrix {
    int type;          /* QK_TYPE_Q4_K or QK_TYPE_Q6_K */
    int rows;
    const void *w;
    float *y;          /* rows outputs */
} qk_matrix;

/* Several matrices that share x and cols, in one launch: y_m = W_m x.
   Replaces qkv_cuda (inferencer.cu:753-784: Q, K and a Q4_K or Q6_K V) and
   gate_up_cuda (inferencer.cu:786-804).  At most QK_MAX_FUSED matrices. */
#define QK_MAX_FUSED 8
int qk_gemv_multi_f32(const qk_matrix *mats, int n_mats, const float *x, int cols,
                      qk_stream stream);

/* Device workspace a multi-token call needs: cols activations, `rows` output
   rows in total (the sum over the matrices of a fused call) and n_tokens
   tokens.  From 8 tokens on it holds the activations packed for the matrix
   cores (4.1 KiB per token and 256 columns, tokens rounded up to 32) and,
   when one row group's blocks are split over several workgroups, their
   partial sums; below 8 tokens it is 0 and the pointer may be NULL.  It
   plays the part of the reference's preallocated batch buffers
   (inferencer.cu:1237-1238) and never needs clearing.  Base alignment 256
   bytes. */
size_t qk_gemv_batched_workspace_bytes(int cols, int rows, int n_tokens);

/* Multi-token variant: y[t*ldy + r] = sum_c W[r][c] * x[t*ldx + c] for
   t < n_tokens (token-major like inferencer.cu:698).  The FP32 arithmetic
   above (22-bit block fixed point per 256-column block) applied to the
   reference's batched path FastRunner::batch_matvec +
   gemv_batch_dp4a (inferencer.cu:1265-1278, 678-699), without its 32-token
   cap; n_tokens = 0 is a no-op.  workspace holds at least
   qk_gemv_batched_workspace_bytes(cols, rows, n_tokens) device bytes and
   must not be shared by calls in flight at the same time. */
int qk_gemv_batched_f32(int type, const void *w, const float *x, int ldx, float *y, int ldy,
                        int cols, int rows, int n_tokens, void *workspace,
                        size_t workspace_bytes, qk_stream stream);

/* Fused multi-token launch over matrices sharing x: y_m[t*rows_m + r].
   Replaces qkv_batch_cuda (inferencer.cu:701-731) and gate_up_batch_cuda
   (inferencer.cu:733-751). */
int qk_gemv_multi_batched_f32(const qk_matrix *mats, int n_mats, const float *x, int ldx,
                              int cols, int n_tokens, void *workspace, size_t workspace_bytes,
                              qk_stream stream);

/* The feed-forward block of n_tokens tokens: y[t*ldy + r] (+)= (W_down
   (SiLU(W_gate x_t) * (W_up x_t)))[r] -- gate and up are hidden x dim (cols
   dim), down dim x hidden; `accumulate` adds into y (the residual; y may be
   x).  Replaces the reference's batched FFN sequence gate_up_batch_cuda +
   silu_cuda + the down projection (inferencer.cu:733-751, 1043-1056,
   1362-1380) with FP32 semantics.  From 8 tokens on it runs as five
   launches on the matrix cores: the gate / up reduction packs SiLU(gate) *
   up straight into the down projection's input records, so neither gate,
   up nor their product is stored as fp32; below 8 tokens, the fused GEMV
   pair of qk_gemv_multi_f32 and a down GEMV staging SiLU * up.  workspace:
   qk_ffn_batched_workspace_bytes(dim, hidden, n_tokens) bytes (256-byte
   aligned; also enough for fewer tokens), not shared by calls in flight at
   the same time.  dim and hidden multiples of 256.  No reference
   counterpart as one call. */
size_t qk_ffn_batched_workspace_bytes(int dim, int hidden, int n_tokens);
int qk_ffn_batched_f32(int gate_type, const void *gate, int up_type, const void *up, int down_type, const void *down,
                       const float *x, int ldx, float *y, int ldy, int dim, int hidden, int n_tokens, int accumulate,
                       void *workspace, size_t workspace_bytes, qk_stream stream);

/* ------------------------------------------------------------ dequant -- */

/* out[r*cols + c] = W[row0 + r][c] as fp32, bit-exact with q4_value /
   q6_value (inferencer.cu:454-487). */
int qk_dequant_rows(int type, const void *w, float *out, int cols, int row0, int nrows,
                    qk_stream stream);

/* Copy a cols x rows Q6_K matrix (GGUF block bytes at src) into the split
   layout of QK_TYPE_Q6_K_SPLIT at dst (qk_tensor_bytes(QK_TYPE_Q6_K_SPLIT,
   cols, rows) bytes, 16-byte aligned, not overlapping src).  A load-time
   step: the block bytes are moved, never decoded. */
int qk_q6k_split(const void *src, void *dst, int cols, int rows, qk_stream stream);

/* out[t*cols + c] = W[tokens[t]][c]; tokens is a device array of n_tokens
   ids in [0, vocab).  Replaces embedding_cuda / embedding_batch_cuda
   (inferencer.cu:806-819); any Q4_K, Q6_K or split Q6_K table. */
int qk_embedding(int type, const void *w, const int32_t *tokens, int n_tokens, float *out,
                 int cols, int vocab, qk_stream stream);

/* y = W x as qk_gemv_f32, and out[0] = the lowest row index among the
   maxima of y (NaN never wins; 0 when no value exceeds -inf): the LM head and
   the greedy pick of argmax_blocks_cuda / argmax_final_cuda
   (inferencer.cu:1414, 1523-1526, 1063-1099) in two launches -- each GEMV
   workgroup keeps the best of the rows it stores, one small kernel reduces
   those partials.  workspace: qk_gemv_argmax_workspace_bytes() bytes, 4-byte
   aligned; calls sharing it must not overlap. */
size_t qk_gemv_argmax_workspace_bytes(void);
int qk_gemv_argmax_f32(int type, const void *w, const float *x, float *y, int cols, int rows, int32_t *out,
                       void *workspace, qk_stream stream);

/* qk_gemv_argmax_f32 without a workspace argument and without any device
   allocation: the partials live in a 128 KiB array compiled into the library
   (one per GPU, held until the process ends).  No reference counterpart: it
   serves callers that cannot allocate or pass a workspace (code under HIP
   graph capture, tight serving loops).  Any rows / cols that
   qk_gemv_argmax_f32 accepts fit the array (the GEMV keeps at most 16384
   partials); the call otherwise fails with QK_ERR_LIMIT before its
   argmax launch.  Every call on one GPU shares the array and leaves its
   partials there: calls that overlap on one GPU (two streams, two host
   threads) race and must be serialised by the caller. */
int qk_gemv_argmax_f32_noalloc(int type, const void *w, const float *x, float *y, int cols, int rows,
                               int32_t *out, qk_stream stream);

/* ---------------------------------------------------------- INT8 mode -- */

/* Per 32 values: scale = amax/127 (1 if amax == 0), xq = clamp(rne(x/scale),
   -127, 127).  Token t reads x + t*ldx and writes xq + t*ldxq, xscale +
   t*ldscale (the reference's fixed strides are 8192 and 256,
   inferencer.cu:687-688).  Replaces quantize_x32_cuda (inferencer.cu:544-556)
   and quantize_batch_cuda (inferencer.cu:891-904). */
int qk_quantize_x32(const float *x, int ldx, int8_t *xq, int ldxq, float *xscale, int ldscale,
                    int cols, int n_tokens, qk_stream stream);

/* RMSNorm and the per-32 quantization in one launch: out = x * 1/sqrt(
   mean(x^2) + eps) * weight exactly as qk_rmsnorm_f32 (out may be NULL to
   skip the fp32 copy), then xq / xscale of those values exactly as
   qk_quantize_x32 -- bit-identical to the two calls in sequence.  Token t
   reads x + t*ldx and writes out + t*ldout, xq + t*ldxq, xscale + t*ldscale.
   cols % 32 == 0 (QK_ERR_SHAPE); x, weight and out 16-byte aligned with ldx,
   ldout multiples of 4, xq 4-byte aligned with ldxq a multiple of 4
   (QK_ERR_ALIGN).  Replaces rmsnorm_quantize_cuda and
   rmsnorm_quantize_batch_cuda (inferencer.cu:839-889; the reference's batch
   strides are 8192 and 256). */
int qk_rmsnorm_quantize_x32(const float *x, int ldx, const float *weight, float *out, int ldout,
                            int8_t *xq, int ldxq, float *xscale, int ldscale, int cols, int n_tokens,
                            float eps, qk_stream stream);

/* INT8-activation GEMV for n_tokens tokens (1 = decode): exact integer
   sub-block dots, fp32 combine.  Replaces gemv_q4_dp4a / gemv_q6_dp4a
   (inferencer.cu:558-569, 663-674) and gemv_batch_dp4a
   (inferencer.cu:678-699). */
int qk_gemv_i8(int type, const void *w, const int8_t *xq, int ldxq, const float *xscale,
               int ldscale, float *y, int ldy, int cols, int rows, int n_tokens,
               qk_stream stream);

/* qk_gemv_i8 for a batch of tokens: y[t*ldy + r] for t < n_tokens, the
   reference's INT8 multi-token semantics (gemv_batch_dp4a, inferencer.cu:
   678-699; its default batched mode, inferencer.cu:1611) without the
   32-token cap and without re-reading the weights per token.  From 8 tokens
   on the exact integer sub-block dots run on the integer matrix cores
   (v_mfma_i32_32x32x32_i8 per Q4_K sub-block of 32 columns,
   v_mfma_i32_32x32x16_i8 per Q6_K sub-block of 16) for 32 tokens x 32 rows
   at a time, and each sub-block is combined in fp32 as the reference does:
   (d*sc*dot - dmin*m*sum(xq)) * xscale (Q4_K, inferencer.cu:520-542) and
   d*scale*dot*xscale (Q6_K, 613-643; two sub-blocks sharing an xscale are
   added in integers first); below 8 tokens it is qk_gemv_i8.  A workgroup
   takes 32 rows x 32 tokens x up to 12 or 16 blocks of the row, one per
   wave.  Each launch's plan, chosen from the kernels' occupancy on the
   device, may split rows over workgroups, whose sums a second launch adds
   in split order (deterministic), and a launch larger than the chip holds
   at once lets resident workgroups walk the row tiles.  The workspace
   holds the split sums of any plan:
   qk_gemv_batched_i8_workspace_bytes(cols, rows, n_tokens) bytes, 16-byte
   aligned (0, and NULL allowed, below 8 tokens or at 256 columns; a plan
   without splits ignores it). */
size_t qk_gemv_batched_i8_workspace_bytes(int cols, int rows, int n_tokens);
int qk_gemv_batched_i8(int type, const void *w, const int8_t *xq, int ldxq, const float *xscale, int ldscale,
                       float *y, int ldy, int cols, int rows, int n_tokens, void *workspace, size_t workspace_bytes,
                       qk_stream stream);

/* Fused INT8 GEMV over 1..QK_MAX_FUSED matrices sharing one token's
   quantized activations (xq: cols int8, xscale: cols/32): the dp4a branch of
   qkv_cuda / gate_up_cuda (inferencer.cu:753-804) for any mix of Q4_K and
   Q6_K (either layout).  Each matrix's rows go to its own y. */
int qk_gemv_multi_i8(const qk_matrix *mats, int n_mats, const int8_t *xq, const float *xscale, int cols,
                     qk_stream stream);

/* The fused form of qk_gemv_batched_i8 (qkv_batch_cuda, gate_up_batch_cuda,
   inferencer.cu:701-751): 1..QK_MAX_FUSED matrices (any mix of Q4_K, Q6_K
   and split Q6_K) of cols columns read the same n_tokens quantized rows (xq
   + t*ldxq, xscale + t*ldscale); mats[m].y receives [n_tokens][rows_m].
   One launch from 8 tokens on (two when the plan splits the rows);
   workspace qk_gemv_batched_i8_workspace_bytes(cols, sum of the rows,
   n_tokens). */
int qk_gemv_multi_batched_i8(const qk_matrix *mats, int n_mats, const int8_t *xq, int ldxq, const float *xscale,
                             int ldscale, int cols, int n_tokens, void *workspace, size_t workspace_bytes,
                             qk_stream stream);

/* The feed-forward block in the reference's INT8 batched arithmetic for
   n_tokens quantized rows of dim values: gate / up (gate_up_batch_cuda,
   inferencer.cu:733-751), SiLU(gate) * up (silu_batch_cuda) quantized per 32
   values (quantize_batch_cuda, 891-904), down (gemv_batch_dp4a), into
   y[t*ldy + c] (overwritten, or added with accumulate: add_batch_cuda).
   From 8 tokens on, the gate / up product forms SiLU * up and its
   quantization in its own epilogue (or its reduction launch when the plan
   splits its rows), then down.  gate and up have one storage type.  The workspace
   holds the quantized hidden rows and the split sums:
   qk_ffn_batched_i8_workspace_bytes(dim, hidden, n_tokens), 256-byte
   aligned (also enough for fewer tokens). */
size_t qk_ffn_batched_i8_workspace_bytes(int dim, int hidden, int n_tokens);
int qk_ffn_batched_i8(int gate_type, const void *gate, int up_type, const void *up, int down_type, const void *down,
                      const int8_t *xq, int ldxq, const float *xscale, int ldscale, float *y, int ldy, int dim,
                      int hidden, int n_tokens, int accumulate, void *workspace, size_t workspace_bytes,
                      qk_stream stream);

/* -------------------------------------------------------- step kernels -- */

/* out = x * 1/sqrt(mean(x^2) + eps) * weight per token of n values.
   Replaces rmsnorm_cuda (inferencer.cu:821-834). */
int qk_rmsnorm_f32(const float *x, const float *weight, float *out, int n, int n_tokens,
                   float eps, qk_stream stream);

/* Rotates q (heads*head_dim) and k (kv_heads*head_dim) in adjacent pairs at
   position pos, writes rotated k and v into the caches at
   [(layer*context + pos)*kv_dim].  Tables are [context][head_dim/2].
   Replaces rope_cache_cuda / rope_cuda + cache_cuda (inferencer.cu:906-951),
   generalised from head_dim 128. */
int qk_rope_kv_write(float *q, const float *k, const float *v, const float *cosine,
                     const float *sine, float *key_cache, float *value_cache, int layer, int pos,
                     int context, int heads, int kv_heads, int head_dim, qk_stream stream);

/* GQA attention of one query token over cache positions 0..pos of a layer
   (caches and out 16-byte aligned).  Replaces attention_cuda
   (inferencer.cu:981-1009), generalised head_dim. */
int qk_attention_f32(const float *q, const float *key_cache, const float *value_cache,
                     float *out, int layer, int pos, int context, int heads, int kv_heads,
                     int head_dim, qk_stream stream);

/* x += y (add_cuda, inferencer.cu:1043-1046). */
int qk_add_f32(float *x, const float *y, int n, qk_stream stream);

/* gate = gate / (1 + exp(-gate)) * up (silu_cuda, inferencer.cu:1053-1056). */
int qk_silu_mul_f32(float *gate, const float *up, int n, qk_stream stream);

/* Index of the maximum of v[0..n), lowest index among equal maxima, into
   *out (device).  workspace holds qk_argmax_workspace_bytes(n) device bytes.
   Replaces argmax_blocks_cuda + argmax_final_cuda (inferencer.cu:1063-1099). */
size_t qk_argmax_workspace_bytes(int n);
int qk_argmax_f32(const float *v, int n, int32_t *out, void *workspace, qk_stream stream);

/* ----------------------------------------------- ragged decode batches -- */

/* One token of a ragged batch: the position of the token in its sequence
   and the first row of that sequence in the packed KV caches
   ([layer][cache_rows][kv_dim]; a sequence owns rows kv_row .. kv_row +
   capacity - 1).  The token's key / value go to row kv_row + pos and it
   attends to rows kv_row .. kv_row + pos.  The nearest reference code serves
   one sequence at contiguous positions (start_pos + token,
   inferencer.cu:956-959, 1012-1016); this descriptor lets the tokens of a
   batch come from any mix of sequences -- one decode token each, or a chunk
   of consecutive positions of one sequence (prefill). */
typedef struct qk_batch_token {
    int32_t pos;
    int32_t seq;       /* sequence id; informational (kv_row identifies the rows) */
    int64_t kv_row;
} qk_batch_token;

/* RoPE of token t's q (heads*head_dim at q + t*heads*head_dim, in place) and
   k at its own position, k and v written to row kv_row + pos of `layer`.
   desc is a device array of n_tokens entries; tokens outside the cache
   (pos >= context or kv_row + pos >= cache_rows) are skipped.  Replaces
   rope_cache_batch_cuda (inferencer.cu:953-979). */
int qk_rope_kv_write_batched(float *q, const float *k, const float *v, const float *cosine, const float *sine,
                             float *key_cache, float *value_cache, int layer, int64_t cache_rows,
                             const qk_batch_token *desc, int n_tokens, int context, int heads, int kv_heads,
                             int head_dim, qk_stream stream);

/* GQA attention of every token of a ragged batch over rows kv_row ..
   kv_row + pos of its sequence; out is [n_tokens][heads*head_dim] (16-byte
   aligned, like the caches).  max_pos bounds every pos; a token beyond it or
   beyond the cache gets NaN outputs.  Replaces attention_batch_cuda
   (inferencer.cu:1011-1041). */
int qk_attention_batched_f32(const float *q, const float *key_cache, const float *value_cache, float *out, int layer,
                             int64_t cache_rows, const qk_batch_token *desc, int n_tokens, int max_pos, int heads,
                             int kv_heads, int head_dim, qk_stream stream);

/* qk_attention_batched_f32 with every token's rows spread over several
   workgroups: rows 0..pos of a token are cut into splits of split_rows rows
   (0: chosen from the batch), each split leaves a partial (max, sum of exp,
   output) in workspace and a second kernel merges them in split order.  A
   token whose rows fit one split is written directly.  workspace holds
   qk_attention_split_workspace_bytes(n_tokens, ..., max_pos) bytes for the
   chosen split; with less (or none) the call takes fewer, longer splits.
   Calls sharing a workspace must not overlap.  No reference counterpart:
   attention_cuda (inferencer.cu:981-1009) runs one block per head over the
   whole context, which one CU reads at a few tens of GB/s. */
size_t qk_attention_split_workspace_bytes(int n_tokens, int heads, int kv_heads, int head_dim, int max_pos,
                                          int split_rows);
int qk_attention_split_f32(const float *q, const float *key_cache, const float *value_cache, float *out, int layer,
                           int64_t cache_rows, const qk_batch_token *desc, int n_tokens, int max_pos, int heads,
                           int kv_heads, int head_dim, int split_rows, void *workspace, size_t workspace_size,
                           qk_stream stream);

/* Greedy token of each of `rows` rows of n values (row r at v + r*ldv), the
   lowest index among equal maxima; out is a device array of rows ints.
   workspace holds qk_argmax_rows_workspace_bytes(n, rows) bytes.  The
   per-token form of argmax_blocks_cuda + argmax_final_cuda. */
size_t qk_argmax_rows_workspace_bytes(int n, int rows);
int qk_argmax_rows_f32(const float *v, int n, int64_t ldv, int rows, int32_t *out, void *workspace,
                       qk_stream stream);

/* ---------------------------------------------------- decode-step driver -- */

/* Llama configuration (the llama.* GGUF keys read at inferencer.cu:1205-1214). */
typedef struct qk_llama_config {
    int dim, layers, heads, kv_heads, hidden, vocab, context;
    float eps, rope_theta;
} qk_llama_config;

/* Device pointers to one layer's tensors (blk.N.* names of inferencer.cu:1434-1502). */
typedef struct qk_llama_layer {
    int q_type, k_type, v_type, o_type, gate_type, up_type, down_type;
    const void *q, *k, *v, *o, *gate, *up, *down;
    const float *attn_norm, *ffn_norm;
} qk_llama_layer;

typedef struct qk_llama_weights {
    int embd_type;
    const void *token_embd;
    int output_type;
    const void *output;            /* NULL: tied to token_embd (inferencer.cu:1521-1522) */
    const float *output_norm;
    const qk_llama_layer *layers;  /* host array of cfg.layers entries */
} qk_llama_weights;

typedef struct qk_llama qk_llama;

/* Allocates the step buffers, KV cache and RoPE tables once (the FastGPU /
   FastRunner constructors, inferencer.cu:1115-1142, 1196-1249).  Every Q6_K
   tensor is copied once into the split layout (QK_TYPE_Q6_K_SPLIT, owned by
   the handle, freed by destroy); create returns after those copies, so the
   caller's Q6_K buffers may be released then.  Q4_K, split Q6_K and norm
   tensors are read in place at every step and stay owned by the caller.
   Like the reference's upload (inferencer.cu:329-333), create first checks
   that everything it allocates (caches, split copies, activation buffers,
   logits, workspaces) fits in free device memory with a 64 MiB margin
   (QK_ERR_DEVICE otherwise). */
int qk_llama_create(const qk_llama_config *cfg, const qk_llama_weights *w, qk_stream stream,
                    qk_llama **out);

/* Device bytes a decode handle holds: the split-layout Q6_K copies, the two
   KV caches, and every other buffer (activations, logits, workspaces, RoPE
   tables).  The copies cost as much as the model's Q6_K tensors (449 MB for
   the Llama-3.2-1B Q4_K_M-style mix). */
typedef struct qk_llama_memory {
    uint64_t weight_copies;
    uint64_t kv_cache;
    uint64_t buffers;
} qk_llama_memory;
int qk_llama_memory_bytes(const qk_llama *m, qk_llama_memory *out);
int qk_llama_destroy(qk_llama *m);
/* The reference's INT8 GEMV modes (FastGPU's use_dp4a for Q4_K and
   use_q6_dp4a for Q6_K, inferencer.cu:1159-1166, 1611; both on by default
   there, both off here): enabled types run their GEMVs on per-32 int8
   activations -- RMSNorm and quantization in one launch before QKV, gate/up
   and the LM head (--fused-norm-quant), the attention output quantized
   before o, SiLU * up and its quantization in one launch before down, and
   the residual adds in the o / down GEMVs' epilogues -- and the other types
   stay FP32.  (With both types enabled the driver folds the quantizations
   into the GEMVs and the attention, with the same codes.)  Takes effect at
   the next qk_llama_forward. */
int qk_llama_set_int8(qk_llama *m, int q4k_int8, int q6k_int8);
/* Device pointers to the fp32 caches, [layer][kv_heads][context][head_dim]:
   the drivers keep each KV head's rows contiguous, so the attention
   workgroup of a (token, KV head) streams one run of memory (the reference's
   FastGPU caches are [layer][context][kv_dim]; the Python load_kv and
   cache-row helpers convert). */
int qk_llama_kv_cache(qk_llama *m, float **key_cache, float **value_cache);
/* Device pointer to the fp32 logits of the last step with need_logits. */
int qk_llama_logits(qk_llama *m, const float **logits);
/* Device pointer to the fp32 residual stream x (dim values) after the last
   step: the state --compare-prefill downloads from FastGPU::x
   (inferencer.cu:1744).  Ask again after each step: a greedy INT8 step fed
   the previous step's token swaps in the embedding row that step's final
   pick wrote into a second buffer, so x moves between two buffers, and the
   other one is overwritten by the next pick. */
int qk_llama_residual(qk_llama *m, const float **x);
/* Quantized matrix products the handle has issued since create: seven per
   layer and step (q, k, v, o, gate, up, down) plus one per LM head, the
   count FastGPU::calls keeps for the --stats line "GPU pipeline ... across
   N quantized matrix calls" (inferencer.cu:1170, 1457, 1500, 1909-1910). */
int qk_llama_matrix_calls(const qk_llama *m, uint64_t *calls);
/* The per-layer state --compare-prefill reads (FastRunner::forward's
   layer_trace and quant_trace, inferencer.cu:1424-1531): while set, every
   step copies the residual stream after each layer to residuals
   [layer][dim] and, for the products that run in an INT8 mode, their
   quantized inputs to quantized [layer][4][max(dim, hidden)] -- QKV,
   attention output (o), gate / up, down; the first dim (down: hidden)
   bytes of each slot.  Both are device buffers the caller owns (either may
   be NULL); the copies run on the handle's stream. */
int qk_llama_set_trace(qk_llama *m, float *residuals, int8_t *quantized);
/* One decode step at position pos (FastRunner::forward, inferencer.cu:1424-1531).
   With need_logits, *next_token receives the greedy token (synchronises the
   stream like the reference's 4-byte copy, inferencer.cu:1529); otherwise
   the step stays asynchronous and *next_token is -1. */
int qk_llama_forward(qk_llama *m, int token, int pos, int need_logits, int *next_token);

/* ------------------------------------------- batched decode-step driver -- */

/* A step for a ragged batch of up to max_tokens tokens -- decode tokens of
   different sequences, prefill chunks of consecutive positions of one
   sequence, or any mix (a continuous batch) -- with packed KV caches of
   cache_rows rows per layer ([layer][kv_heads][cache_rows][head_dim], fp32,
   as qk_llama_kv_cache).  The
   multi-sequence counterpart of FastRunner::prefill's batched path
   (inferencer.cu:1279-1423), which serves one sequence; every projection
   runs through qk_gemv_multi_batched_f32 / qk_gemv_batched_f32 (matrix cores
   from 8 tokens on).  Buffers, caches and workspaces are allocated once at
   create; weights are handled as by qk_llama_create (Q6_K copied into the
   split layout, the rest read in place). */
typedef struct qk_llama_batch qk_llama_batch;

int qk_llama_batch_create(const qk_llama_config *cfg, const qk_llama_weights *w, int max_tokens,
                          int64_t cache_rows, qk_stream stream, qk_llama_batch **out);
int qk_llama_batch_destroy(qk_llama_batch *m);
/* The handle's device bytes, as qk_llama_memory_bytes. */
int qk_llama_batch_memory_bytes(const qk_llama_batch *m, qk_llama_memory *out);
/* Device pointers to the fp32 caches, [layer][kv_heads][cache_rows][head_dim]. */
int qk_llama_batch_kv_cache(qk_llama_batch *m, float **key_cache, float **value_cache);
/* Device pointer to the fp32 logits of the last step with need_logits,
   [n_tokens][vocab]. */
int qk_llama_batch_logits(qk_llama_batch *m, const float **logits);
/* Device pointer to the fp32 residual streams after the last step,
   [n_tokens][dim] in the step's token order (inferencer.cu:1744). */
int qk_llama_batch_residual(qk_llama_batch *m, const float **x);
/* Quantized matrix products issued since create: seven per layer and token,
   one per logit row (FastRunner::prefill's counts, inferencer.cu:1277, 1321,
   1368). */
int qk_llama_batch_matrix_calls(const qk_llama_batch *m, uint64_t *calls);
/* qk_llama_set_trace for the batched driver (FastRunner::prefill's
   all_layer_trace and quant_trace, inferencer.cu:1279-1423): per token of
   the step, residuals [token][layer][dim] and, in the INT8 mode, quantized
   [token][layer][4][max(dim, hidden)]; sized for the step's n_tokens. */
int qk_llama_batch_set_trace(qk_llama_batch *m, float *residuals, int8_t *quantized);
/* The reference's INT8 batched arithmetic for the steps that follow
   (FastRunner::prefill with use_dp4a and use_q6_dp4a, inferencer.cu:
   1279-1423; its batched prefill requires both, 1662-1663): per layer
   RMSNorm and per-32 quantization of x, the fused QKV product, attention,
   the attention output quantized, o added into x, RMSNorm and quantization,
   gate / up with SiLU(gate) * up quantized, down added into x; the LM head
   over the RMSNorm of x quantized.  Products run as qk_gemv_multi_batched_i8
   (exact integer sub-block dots).  q4k_int8 and q6k_int8 must be equal
   (QK_ERR_INVALID_ARG otherwise); the first enable allocates the quantized
   activation buffers (QK_ERR_DEVICE when they do not fit). */
int qk_llama_batch_set_int8(qk_llama_batch *m, int q4k_int8, int q6k_int8);
/* One step for n_tokens tokens: tokens[t] (host) at desc[t] (host).  Every
   token writes its key / value row kv_row + pos before any token's
   attention reads the cache, so a token sees the rows of earlier positions
   of its sequence written in the same step (causal within a prefill chunk,
   rope_cache_batch_cuda before attention_batch_cuda, inferencer.cu:953-1041).
   Two tokens writing the same row is QK_ERR_INVALID_ARG.  With need_logits,
   next_tokens[t] (host) receives each token's greedy successor and the call
   synchronises the stream; otherwise it stays asynchronous. */
int qk_llama_batch_forward(qk_llama_batch *m, const int32_t *tokens, const qk_batch_token *desc, int n_tokens,
                           int need_logits, int32_t *next_tokens);
/* The same step with the LM head run only for the n_rows tokens listed in
   logit_rows (host, token indices in [0, n_tokens), any order): logits are
   [n_rows][vocab] in list order and next_tokens[i] (host) is the greedy
   successor of token logit_rows[i].  The reference's prefill computes the
   logits of a chunk's last token only (inferencer.cu:1410-1414); a
   continuous batch needs them for each chunk end and each decode token.
   n_rows = 0 runs no LM head and stays asynchronous. */
int qk_llama_batch_forward_rows(qk_llama_batch *m, const int32_t *tokens, const qk_batch_token *desc, int n_tokens,
                                const int32_t *logit_rows, int n_rows, int32_t *next_tokens);

/* --------------------------------------------------------------- GGUF -- */

/* A GGUF v3 model file, mapped read-only (the reference's GGUF struct,
   inferencer.cu:204-340).  Scalar metadata is kept as doubles, string values
   as strings, tokenizer.ggml.tokens / merges as string arrays; other arrays
   are skipped.  Tensors may be FP32 (0), FP16 (1), Q4_K (12) or Q6_K (14).
   Stricter than the reference: every tensor's offset + bytes must lie inside
   the data section (the reference checks offset < size, inferencer.cu:282),
   offsets must be multiples of general.alignment, and names must be unique;
   each violation is QK_ERR_FORMAT. */
typedef struct qk_gguf qk_gguf;

typedef struct qk_gguf_tensor {
    const char *name;      /* valid until qk_gguf_close */
    int type;              /* 0 FP32, 1 FP16, 12 Q4_K, 14 Q6_K */
    int n_dims;            /* 1..4 */
    int64_t dims[4];       /* dims[0] is contiguous (cols); unused dims are 1 */
    uint64_t offset;       /* from the start of the data section */
    uint64_t bytes;
    const void *host;      /* inside the mapping */
    const void *device;    /* after qk_gguf_upload, else NULL */
} qk_gguf_tensor;

/* QK_ERR_IO if the file cannot be opened or mapped, QK_ERR_FORMAT with the
   reason in qk_last_error() if it is not a valid GGUF v3 file. */
int qk_gguf_open(const char *path, qk_gguf **out);
/* Unmaps the file and frees the device copy. */
int qk_gguf_close(qk_gguf *g);
/* A scalar metadata value (GGUF::param, inferencer.cu:290-294); missing keys
   are QK_ERR_INVALID_ARG. */
int qk_gguf_param(const qk_gguf *g, const char *key, double *value);
/* A string metadata value, or NULL. */
const char *qk_gguf_string(const qk_gguf *g, const char *key);
int64_t qk_gguf_tensor_count(const qk_gguf *g);
/* Tensors in file order. */
int qk_gguf_tensor_at(const qk_gguf *g, int64_t index, qk_gguf_tensor *out);
/* GGUF::tensor (inferencer.cu:317-321); missing names are QK_ERR_INVALID_ARG. */
int qk_gguf_find_tensor(const qk_gguf *g, const char *name, qk_gguf_tensor *out);
/* which = 0: tokenizer.ggml.tokens, 1: tokenizer.ggml.merges. */
int64_t qk_gguf_token_count(const qk_gguf *g, int which);
/* The bytes of entry i (not NUL-terminated; *length receives the size). */
const char *qk_gguf_token(const qk_gguf *g, int which, int64_t i, int64_t *length);
/* The mapped data section, its size and the alignment in effect. */
int qk_gguf_data(const qk_gguf *g, const void **host, uint64_t *bytes, uint64_t *alignment);
/* Copies the data section into one device buffer owned by the handle
   (GGUF::upload, inferencer.cu:322-339: same free-memory margin) and sets
   every tensor's device pointer.  Synchronises the stream. */
int qk_gguf_upload(qk_gguf *g, qk_stream stream);
/* The llama.* hyper-parameters and every tensor of a Llama model by its GGUF
   name (FastRunner's constructor, inferencer.cu:1196-1214, any shape the
   decode drivers support), ready for qk_llama_create: matrices Q4_K or Q6_K
   with dims {cols, rows}, norms FP32 of dims {dim}; output.weight optional
   (tied to token_embd.weight).  llama.vocab_size when present, else the
   embedding's row count.  Requires qk_gguf_upload; layers receives
   cfg.layers entries (at most max_layers); w->layers points at it. */
int qk_gguf_llama(const qk_gguf *g, int context, qk_llama_config *cfg, qk_llama_weights *w,
                  qk_llama_layer *layers, int max_layers);

#ifdef __cplusplus
}
#endif

#endif
