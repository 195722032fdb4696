// qk_internal.h - shared host plumbing and device helpers of libqk.so.
//
// Super-block layouts (GGML, decoded by inferencer.cu:453-497):
//   Q4_K, 144 B: fp16 d @0, fp16 dmin @2, 12 packed 6-bit scale/min bytes @4,
//                128 bytes of nibbles @16.  w = d*sc*q - dmin*m.
//   Q6_K, 210 B: ql[128] @0, qh[64] @128, int8 scales[16] @192, fp16 d @208.
//                w = d*scale*(code - 32).
//
// The GEMV kernels cut every row into "pieces" of 64 weights, one piece per
// lane.  Piece p of a row covers block b = p/4, g = (p/2)%2, h = p%2 and the
// columns b*256 + g*128 + part*32 + h*16 + k for part 0..3, k 0..15.  The
// same column set serves both formats:
//   Q4_K: 16 B of nibbles at 16 + g*64 + h*16 (parts 0/1 = low/high nibbles)
//         and at 16 + g*64 + 32 + h*16 (parts 2/3), plus the 16 B header.
//   Q6_K: 16 B of ql at g*64 + h*16 (parts 0/2), at g*64 + 32 + h*16
//         (parts 1/3), 16 B of qh at 128 + g*32 + h*16, the four scales
//         scales[g*8 + part*2 + h] and d.
// so a lane's 64 activations are fixed for every row of a matrix and for
// every matrix of a fused launch, whatever their types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/qk.h"

namespace qk {

// ------------------------------------------------------------------ host --

// Records a thread-local message and returns the status (never throws).
int fail(int status, const std::string &message);
// Clears the thread-local message; returns QK_OK.
int ok();
// Maps a HIP error after launches to QK_ERR_DEVICE.
int launch_status(const char *where);

inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int block_bytes(int type);
// Bytes of one row of nb blocks: nb * 144 (Q4_K), nb * 210 (Q6_K), nb * 210
// rounded up to 16 (split Q6_K, so every row starts 16-byte aligned).
int64_t row_bytes(int type, int nb);
// Validates a Q4_K / Q6_K weight operand shape; returns QK_OK or a status.
int check_weights(const char *where, int type, const void *w, int cols, int rows);

// Decode-step fusions of the FP32 GEMV (driver-internal, not in the C ABI):
// the activations are staged as RMSNorm(x) * norm_w (rmsnorm_cuda) or as
// x / (1 + exp(-x)) * up (silu_cuda), and the epilogue adds W x into y (the
// residual add_cuda) instead of overwriting it.
struct GemvFusion {
    const float *norm_w = nullptr;
    float norm_eps = 0.f;
    const float *up = nullptr;
    int accumulate = 0;
    // Matrix-core decode chain (from 8 tokens on; all unset: none).  The
    // input comes as records a previous call's reduction packed
    // (in_records, cols / 256 blocks per 32-token tile), with per (token,
    // block) sums of squares in_ss when its RMSNorm is deferred to the
    // outputs (norm_eps).  out_records: the reduction packs this call's
    // output as the next call's input -- y * out_gain with sums of squares in
    // out_ss (one matrix, y after the residual add), or SiLU(y0) * y1 with
    // pair (two matrices of equal rows, y not stored); rows % 256 == 0.
    const uint8_t *in_records = nullptr;
    const float *in_ss = nullptr;
    uint8_t *out_records = nullptr;
    const float *out_gain = nullptr;
    float *out_ss = nullptr;
    int pair = 0;
    // Greedy-token epilogue (one matrix, one token): every wave writes the
    // best (value, row) of the rows it stored to arg_v / arg_i and the launch
    // reports the number of such partials in *arg_parts (at most
    // kArgPartsMax).
    float *arg_v = nullptr;
    int *arg_i = nullptr;
    int *arg_parts = nullptr;
};
constexpr int kArgPartsMax = 16384;
// The picked token's embedding row, written by the final pick for the next
// step (out NULL: none): table rows of row_bytes, nb blocks of type.
struct NextEmbedding {
    const uint8_t *table = nullptr;
    int type = 0, nb = 0;
    int64_t row_bytes = 0;
    float *out = nullptr;
};
// The argmax partials -> out[0] (the lowest row among maxima; 0 if none),
// also stored to host_out[0] when given (device address of host-coherent
// pinned memory); with next, the token's embedding row into next->out.
int launch_argmax_final(const float *pv, const int *pi, int parts, int32_t *out, hipStream_t stream,
                        int32_t *host_out = nullptr, const NextEmbedding *next = nullptr);

// dst[i][0..cols) = src[idx[i]][0..cols) (row stride ld) for i < n; idx is a
// device array of n row indices.  cols and ld multiples of 4, src and dst
// 16-byte aligned.
int launch_gather_rows(const float *src, int64_t ld, const int32_t *idx, int n, int cols, float *dst,
                       hipStream_t stream);

// The greedy-token order (argmax_blocks_cuda / argmax_final_cuda,
// inferencer.cu:1063-1099): a larger value wins, equal values keep the lower
// index; NaN never wins.
__device__ __forceinline__ void arg_better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}
// FP32 GEMV of n_tokens activation rows (x + t*ldx; y + t*ldy[m], NULL:
// rows), arguments already validated.
int launch_gemv_f32(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                    const int *ldy, hipStream_t stream);
// INT8 GEMV of n_tokens quantized activation rows (xq + t*ldxq, xscale +
// t*ldscale; y + t*ldy[m]), arguments already validated; accumulate != 0
// adds W x into y instead of overwriting it.
// One token's INT8 GEMV over one matrix that also leaves each wave's best
// (value, row) in arg_v / arg_i (*parts of them, at most kArgPartsMax) for
// launch_argmax_final: the greedy token without a pass over the outputs.
int launch_gemv_i8_argmax(const qk_matrix *mat, const int8_t *xq, const float *xscale, int cols, float *arg_v,
                          int *arg_i, int *parts, hipStream_t stream);
// The same over the fp32 row x, RMSNorm'd with norm_w and quantized by every
// workgroup (launch_gemv_i8_staged's staging; 256-thread workgroups, so the
// codes are rmsnorm_quantize_kernel's).
int launch_gemv_i8_staged_argmax(const qk_matrix *mat, const float *x, const float *norm_w, float eps, int cols,
                                 float *arg_v, int *arg_i, int *parts, hipStream_t stream);
int launch_gemv_i8(const qk_matrix *mats, int n_mats, const int8_t *xq, int ldxq, const float *xscale, int ldscale,
                   int cols, int n_tokens, const int *ldy, int accumulate, hipStream_t stream);
// The INT8 GEMV quantizing its own fp32 input per 32 values in LDS, after
// RMSNorm with norm_w (eps) or SiLU(x) * up when given -- bit for bit the
// separate quantization kernels' codes with 256-thread blocks.  Only for
// rows gemv_i8_stageable accepts.
int launch_gemv_i8_staged(const qk_matrix *mats, int n_mats, const float *x, int ldx, const float *norm_w, float eps,
                          const float *up, int cols, int n_tokens, const int *ldy, int accumulate, hipStream_t stream);
bool gemv_i8_stageable(int cols);
// The INT8 gate / up pair (two matrices of one type and equal rows, a
// multiple of 32) over staged inputs (RMSNorm with norm_w when given),
// writing SiLU(gate) * up quantized per 32 into hq [token][ldq] and hs
// [token][ldsc] instead of gate and up.  cols of 1, 2, 4, 8 or 16 blocks.
bool gemv_i8_pair_supported(int cols, int rows);
// The INT8 GEMV (one token, 256-thread workgroups) whose input is the
// one-sequence attention's unmerged wide-form partials (n_parts splits per
// head of head_dim; launch_split_attention with defer_merge): each
// workgroup merges and quantizes the row as the merge kernel and
// quantize_x32_kernel would.  cols of 1, 2, 4 or 8 blocks, at most 8 splits.
bool gemv_i8_mergeable(int cols, int head_dim, int n_parts);
int launch_gemv_i8_merged(const qk_matrix *mats, int n_mats, const float *parts, int n_parts, int head_dim, int cols,
                          int accumulate, hipStream_t stream);
int launch_gemv_i8_pair_quant(const qk_matrix *gu, const float *x, int ldx, const float *norm_w, float eps, int cols,
                              int n_tokens, int8_t *hq, float *hs, int ldq, int ldsc, hipStream_t stream);
// INT8 product of n_tokens per-32 quantized rows with n_mats matrices on
// the integer matrix cores (csrc/qk_skinny.hip), arguments already
// validated: y_m[t*ldy[m] + r] overwritten (or added with accumulate); with
// out_xq, matrices 0 and 1 are a gate / up pair and SiLU(gate) * up is
// quantized per 32 values into out_xq / out_xs (ldy and y unused).  Rows
// longer than 2048 columns are split over workgroups whose sums a second
// launch adds: the workspace holds them (skinny_i8_workspace_bytes of the
// launch's row tiles: sum of ceil(rows / 32), or rows / 32 for a pair).
size_t skinny_i8_workspace_bytes(int cols, int tiles, int n_tokens, bool pair);
// The next RMSNorm + quantization of an accumulating one-matrix launch's
// output rows, folded into its split reduction: x (the launch's y) as
// rmsnorm_quantize_kernel would normalise it with w, into xq [token][ldxq]
// and xs [token][ldxs], bit for bit.  *done is set when the launch did it
// (it split its sums; rows of at most 4096), cleared otherwise.  With
// plan_only the launch is planned as if folding (the same split sums) but
// reduces plainly and leaves the normalisation to the caller.
struct SkNorm {
    const float *w = nullptr;
    float eps = 0.f;
    int8_t *xq = nullptr;
    float *xs = nullptr;
    int ldxq = 0, ldxs = 0;
    int *done = nullptr;
    int plan_only = 0;
};
// A storing launch (not a pair, not accumulating, no SkNorm) whose split
// sums the consumer adds itself: the plan costs no reduction launch, and a
// launch that splits writes no y and reports its partials' layout here
// (splits 0: it wrote y itself).  Partial (row tile, token tile, split) is
// 1024 floats at ((tile * token_tiles + ttile) * splits + split) * 1024, in
// the accumulator's element order.
struct SkDeferred {
    const float *partials = nullptr;
    int splits = 0, token_tiles = 0;
    int tile_begin[QK_MAX_FUSED] = {};
};
int launch_skinny_i8(const qk_matrix *mats, int n_mats, const int *ldy, const int8_t *xq, int ldxq,
                     const float *xscale, int ldscale, int cols, int n_tokens, int accumulate, int8_t *out_xq,
                     float *out_xs, int out_ldxq, int out_ldxs, void *workspace, size_t workspace_size,
                     hipStream_t stream, const char *where, const SkNorm *norm = nullptr,
                     SkDeferred *defer = nullptr);
// SiLU(gate) * up quantized per 32 values straight into xq / xscale (n a
// multiple of 32): bit-identical to qk_silu_mul_f32 then qk_quantize_x32,
// without the fp32 product written.  Arguments already validated.
int launch_silu_mul_quantize(const float *gate, const float *up, int8_t *xq, float *xscale, int n,
                             hipStream_t stream);

// SiLU(g) * u in silu_cuda's expression (inferencer.cu:1053-1057), shared by
// every kernel that forms it so their results agree bit for bit.
__device__ __forceinline__ float silu_mul_value(float g, float u) { return g / (1.f + expf(-g)) * u; }

// Wave-wide sum (xor tree, every lane gets the total) and block-wide sum for
// blockDim.x = 256 (every wave's tree, then (w0 + w1) + (w2 + w3)): the
// order rmsnorm_kernel and rmsnorm_quantize_kernel sum their squares in.
__device__ __forceinline__ float wave_sum(float v) {
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float block_sum256(float v, float *scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    return (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
}

// quantize_x32_cuda (inferencer.cu:544-556) for the value a lane holds: the
// 32 lanes of its half-wave form one group; lanes past the row hold 0.
// scale = amax/127 (1 when amax is 0), q = clamp(rne(value/scale), +-127),
// IEEE divide.  Lane 0 of the group stores the scale.
__device__ __forceinline__ void quantize_group_store(float value, bool in_row, int lane32, int8_t *q_out,
                                                     float *scale_out) {
    float amax = fabsf(value);
    #pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float scale = amax > 0.f ? amax / 127.f : 1.f;
    if (lane32 == 0 && in_row) *scale_out = scale;
    if (in_row) {
        int q = static_cast<int>(rintf(value / scale));
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        *q_out = static_cast<int8_t>(q);
    }
}

// The same for four values a lane holds: eight adjacent lanes form one
// 32-value group (amax in three xor shuffles, so all eight must be active
// together); the first of them stores the scale.  q: the four codes, lowest
// column in the low byte.
__device__ __forceinline__ void quantize_quad_store(const float4 &o, bool first, uint32_t *q, float *scale_out) {
    float amax = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const float gs = amax > 0.f ? amax / 127.f : 1.f;
    if (first) *scale_out = gs;
    auto q8 = [gs](float val) {
        int c = static_cast<int>(rintf(val / gs));
        c = c < -127 ? -127 : (c > 127 ? 127 : c);
        return static_cast<uint32_t>(c) & 0xFFu;
    };
    *q = q8(o.x) | (q8(o.y) << 8) | (q8(o.z) << 16) | (q8(o.w) << 24);
}
// Whether a row of cols columns can stage its activations for the fusions.
bool gemv_fusable(int cols);
// n_tokens tokens (x + t*ldx; y + t*ldy[m], NULL: rows), arguments already
// validated.
int launch_gemv_fused(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                      const int *ldy, const GemvFusion &f, hipStream_t stream);
// The same for a batch of n_tokens tokens, token-major (ldy = rows): the
// matrix-core GEMM from 8 tokens on (staging fused into its pack kernel, the
// residual add into its epilogue), the fused GEMV below.  workspace as for
// qk_gemv_multi_batched_f32.
// Decode chains on the matrix cores (GemvFusion in_records / out_records):
// whether n_tokens takes that path, the workspace a chained call needs
// (partial sums even without a split), and the bytes of one call's packed
// activation records of `cols` columns.
bool batched_chain_supported(int n_tokens);
size_t batched_chain_workspace_bytes(int cols, int rows_total, int n_tokens);
size_t batched_records_bytes(int cols, int n_tokens);
int launch_batched_fused(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                         const GemvFusion &f, void *workspace, size_t workspace_size, hipStream_t stream);
// ------------------------------------------------ activation records --
//
// The FP32 GEMVs read activations as 64-byte records, one per 16 columns:
// the 16 values as X = rint(x * 2^(21-e)) with e = ilogb(max|x|), |X| <=
// 2^22, split into three signed bytes X = L2*65536 + L1*256 + L0 (packed
// four per dword: L0 x16, L1 x16, L2 x16), the scale 2^(e-21) and the fp32
// sum of the 16 values.  A dot of 16 integer codes with a record is then
// three exact v_dot4 sums.  Records are made by the GEMV workgroups
// themselves (staging) or, in the decode driver, by the kernel that
// produces the activations.
struct XGroup {
    int limb[12];   // L0 x16, L1 x16, L2 x16 as int8, four per dword
    float scale;    // 2^(e-21); 0 for an all-zero group, NaN/inf if x is not finite
    float sum;      // fp32 sum of the 16 activations (min / code-offset terms)
    int pad[2];
};
static_assert(sizeof(XGroup) == 64, "XGroup is one 64-byte record");

__device__ __forceinline__ void load16f(const float *x16, float *v) {
    #pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 q = *reinterpret_cast<const float4 *>(x16 + 4 * k);
        v[4 * k] = q.x;
        v[4 * k + 1] = q.y;
        v[4 * k + 2] = q.z;
        v[4 * k + 3] = q.w;
    }
}

__device__ __forceinline__ XGroup make_group_regs(const float *v);

__device__ __forceinline__ XGroup make_group(const float *x16) {
    float v[16];
    load16f(x16, v);
    return make_group_regs(v);
}

// The records of four 16-value groups at once: lanes 16g .. 16g+15 of a
// wave hold group g's values (x) and make its 64-byte record at dst (each
// lane passes its own group's; nothing is stored where store is false) --
// make_group_regs' arithmetic, with the group's sum taken as a tree.  Every
// lane of the wave must call it.
__device__ __forceinline__ void record16_quads(float x, int lane, XGroup *dst, bool store) {
    float m = fabsf(x), sum = x;
    #pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        sum += __shfl_xor(sum, off);
    }
    const bool ok = m > 0.f && isfinite(m);
    const int e = __builtin_amdgcn_frexp_expf(m) - 1;
    const int X = ok ? static_cast<int>(rintf(ldexpf(x, 21 - e))) : 0;
    const int b0 = (X << 24) >> 24;
    const int X1 = (X - b0) >> 8;
    const int b1 = (X1 << 24) >> 24;
    const int b2 = (X1 - b1) >> 8;
    const int sh = 8 * (lane & 3);
    uint32_t u0 = (static_cast<uint32_t>(b0) & 0xFFu) << sh;
    uint32_t u1 = (static_cast<uint32_t>(b1) & 0xFFu) << sh;
    uint32_t u2 = (static_cast<uint32_t>(b2) & 0xFFu) << sh;
    #pragma unroll
    for (int off = 1; off < 4; off <<= 1) {
        u0 |= __shfl_xor(u0, off);
        u1 |= __shfl_xor(u1, off);
        u2 |= __shfl_xor(u2, off);
    }
    // Dword k of limb set j sits in lanes base + 4k .. +3 of u_j.
    const int base = lane & 48, k = lane & 3, li = lane & 15;
    const uint32_t d0 = __shfl(u0, base + 4 * k), d1 = __shfl(u1, base + 4 * k), d2 = __shfl(u2, base + 4 * k);
    const float scale = ok ? ldexpf(1.f, e - 21) : (m == 0.f ? 0.f : __builtin_nanf(""));
    uint32_t word = 0;   // the two pad words stay zero
    if (li < 4) word = d0;
    else if (li < 8) word = d1;
    else if (li < 12) word = d2;
    else if (li == 12) word = __builtin_bit_cast(uint32_t, scale);
    else if (li == 13) word = __builtin_bit_cast(uint32_t, sum);
    if (store) reinterpret_cast<uint32_t *>(dst)[li] = word;
}

// record16_quads' record of 16 values made by one lane: the same maximum,
// the sum in its xor-tree order ((v0+v8) + (v4+v12)) + ((v2+v10) + (v6+v14))
// + ... (every lane of that butterfly ends with these bits: fp32 addition
// commutes), the same exponent, limbs and words.
__device__ __forceinline__ XGroup make_group_tree(const float *v) {
    float a[8], b[4];
    #pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = v[i] + v[i + 8];
    #pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = a[i] + a[i + 4];
    const float sum = (b[0] + b[2]) + (b[1] + b[3]);
    float m = fabsf(v[0]);
    #pragma unroll
    for (int i = 1; i < 16; ++i) m = fmaxf(m, fabsf(v[i]));
    const bool ok = m > 0.f && isfinite(m);
    const int e = __builtin_amdgcn_frexp_expf(m) - 1;
    uint32_t l0[4] = {0, 0, 0, 0}, l1[4] = {0, 0, 0, 0}, l2[4] = {0, 0, 0, 0};
    #pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int X = ok ? static_cast<int>(rintf(ldexpf(v[i], 21 - e))) : 0;
        const int b0 = (X << 24) >> 24;
        const int X1 = (X - b0) >> 8;
        const int b1 = (X1 << 24) >> 24;
        const int b2 = (X1 - b1) >> 8;
        l0[i >> 2] |= (static_cast<uint32_t>(b0) & 0xFFu) << (8 * (i & 3));
        l1[i >> 2] |= (static_cast<uint32_t>(b1) & 0xFFu) << (8 * (i & 3));
        l2[i >> 2] |= (static_cast<uint32_t>(b2) & 0xFFu) << (8 * (i & 3));
    }
    XGroup gr;
    #pragma unroll
    for (int k = 0; k < 4; ++k) {
        gr.limb[k] = static_cast<int>(l0[k]);
        gr.limb[4 + k] = static_cast<int>(l1[k]);
        gr.limb[8 + k] = static_cast<int>(l2[k]);
    }
    gr.scale = ok ? ldexpf(1.f, e - 21) : (m == 0.f ? 0.f : __builtin_nanf(""));
    gr.sum = sum;
    gr.pad[0] = gr.pad[1] = 0;
    return gr;
}

__device__ __forceinline__ XGroup make_group_regs(const float *v) {
    float m = 0.f, s = 0.f;
    #pragma unroll
    for (int i = 0; i < 16; ++i) {
        m = fmaxf(m, fabsf(v[i]));
        s += v[i];
    }
    XGroup gr;
    gr.sum = s;
    gr.pad[0] = gr.pad[1] = 0;
    if (!(m > 0.f) || !isfinite(m)) {
        #pragma unroll
        for (int i = 0; i < 12; ++i) gr.limb[i] = 0;
        gr.scale = m == 0.f ? 0.f : __builtin_nanf("");   // a non-finite input poisons its rows
        return gr;
    }
    // v_frexp_exp gives e+1 for m in [2^e, 2^(e+1)).
    const int e = __builtin_amdgcn_frexp_expf(m) - 1;
    uint32_t l0[4] = {0, 0, 0, 0}, l1[4] = {0, 0, 0, 0}, l2[4] = {0, 0, 0, 0};
    #pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int X = static_cast<int>(rintf(ldexpf(v[i], 21 - e)));
        const int b0 = (X << 24) >> 24;
        const int X1 = (X - b0) >> 8;
        const int b1 = (X1 << 24) >> 24;
        const int b2 = (X1 - b1) >> 8;
        l0[i >> 2] |= (static_cast<uint32_t>(b0) & 0xFFu) << (8 * (i & 3));
        l1[i >> 2] |= (static_cast<uint32_t>(b1) & 0xFFu) << (8 * (i & 3));
        l2[i >> 2] |= (static_cast<uint32_t>(b2) & 0xFFu) << (8 * (i & 3));
    }
    #pragma unroll
    for (int k = 0; k < 4; ++k) {
        gr.limb[k] = static_cast<int>(l0[k]);
        gr.limb[4 + k] = static_cast<int>(l1[k]);
        gr.limb[8 + k] = static_cast<int>(l2[k]);
    }
    gr.scale = ldexpf(1.f, e - 21);
    return gr;
}



// Whether the attention kernel serves `group` query heads per KV head and
// head_dim (group in {1, 2, 3, 4, 6, 8}; head_dim a multiple of 4 dividing 256).
bool attention_supported(int group, int head_dim);

// Split-row attention (GQA, one or many tokens): the rows 0..pos of every
// (token, KV head) are cut into splits of split_rows rows, one 256-thread
// workgroup each, so a token's cache read spreads over many CUs.  With k set
// it also rotates q and k at pos and writes the key / value row (the
// workgroup holding row pos writes it and takes it from LDS, so no other
// workgroup reads it); with k NULL q is already rotated and the caches hold
// row pos.  Every token of one call must own its cache rows.
struct SplitAttention {
    const float *q;                  // [n_tokens][heads * head_dim]
    const float *k, *v;              // [n_tokens][kv_heads * head_dim] or NULL
    const float *cosine, *sine;      // [context][head_dim / 2] (with k)
    float *key_cache, *value_cache;  // [layers][cache_rows][kv_heads * head_dim]
    float *out;                      // [n_tokens][heads * head_dim]
    const qk_batch_token *desc;      // device, n_tokens entries; NULL: one token at pos, kv_row 0
    XGroup *rec_out;                 // the outputs' activation records too (head_dim % 16 == 0), or NULL
    // The outputs as the matrix-core GEMM's records too ([tile][block][...],
    // blocks of heads * head_dim / 256 per tile; needs G * head_dim % 256 ==
    // 0 so each workgroup's heads fill whole blocks), or NULL.
    uint8_t *gemm_rec;
    int64_t cache_rows;
    int64_t rows_hint;               // sum over tokens of pos + 1 (0: n_tokens * (max_pos + 1))
    // The outputs quantized per 32 values as well ([n_tokens][heads *
    // head_dim] codes, [n_tokens][heads * head_dim / 32] scales; head_dim % 32
    // == 0), or NULL: the INT8 o projection's input.
    int8_t *q8_out;
    float *q8_scale;
    // The wide form (one workgroup per query head, few tokens over short
    // rows) takes all of a head's rows in one split unless wide_split_rows
    // > 0 caps its rows per split.
    int wide_split_rows;
    // Leave split partials unmerged (no merge launch): the caller merges.
    int defer_merge;
    // q, k and v as the INT8 QKV product's unreduced split sums (SkDeferred)
    // when qkv_splits > 1, read with k set: element (token b, column c) of
    // matrix m is the sum in split order of the partials of row tile
    // tile0[m] + c / 32, token tile b / 32 (skinny_reduce's additions).
    const float *qkv_parts;
    int qkv_splits, qkv_ttiles, qkv_tile0[3];
    int layer, pos, max_pos, n_tokens, heads, kv_heads, head_dim;
    // Cache layout: 0 the reference's [layers][cache_rows][kv_heads][head_dim],
    // 1 [layers][kv_heads][cache_rows][head_dim] (the decode drivers' own: a
    // (token, KV head) workgroup then reads one contiguous run of memory
    // instead of head_dim floats out of every kv_heads * head_dim).
    int head_major;
};
// Offset in floats of row `row` of KV head `h` in layer `layer` of a cache of
// either layout.
__host__ __device__ __forceinline__ int64_t kv_offset(int head_major, int layer, int64_t cache_rows, int kv_heads,
                                                      int head_dim, int64_t row, int h) {
    return head_major ? ((static_cast<int64_t>(layer) * kv_heads + h) * cache_rows + row) * head_dim
                      : (static_cast<int64_t>(layer) * cache_rows + row) * kv_heads * head_dim +
                            static_cast<int64_t>(h) * head_dim;
}
// RoPE of q and k at each token's position, k and v written to row kv_row +
// pos of the caches in either layout (qk_rope_kv_write_batched's kernel;
// arguments validated by the caller).
int launch_rope_kv_batched(float *q, const float *k, const float *v, const float *cosine, const float *sine,
                           float *key_cache, float *value_cache, int layer, int64_t cache_rows,
                           const qk_batch_token *desc, int n_tokens, int context, int heads, int kv_heads,
                           int head_dim, int head_major, hipStream_t stream);
// Rows per split for head_rows (token, KV head) rows in all, the longest
// token max_rows rows (the split policy).
int split_attention_rows(int64_t head_rows, int max_rows);
// Workspace of launch_split_attention (the split partials) for n_tokens
// tokens of at most max_rows rows (at most 64 MiB; 0 when one split always
// serves).  A call with less workspace takes fewer, longer splits, one with
// none a single split.  Calls sharing a workspace must not overlap.
size_t split_attention_workspace_bytes(int n_tokens, int heads, int kv_heads, int head_dim, int max_rows);
// split_rows <= 0 takes the policy's value.  Arguments validated by the
// caller.  splits_used (optional) receives the splits per token left for
// the caller to merge, or 1 when the outputs are written: with a.defer_merge
// a wide-form launch of several splits leaves its partials in the workspace,
// split_partial_floats(head_dim) per (query head, split), split-minor, and
// writes no outputs.
int launch_split_attention(const SplitAttention &a, int split_rows, void *workspace, size_t workspace_size,
                           hipStream_t stream, int *splits_used = nullptr);
// Floats of one split partial of one query head in the wide form: the
// running max and sum of exp (base-2 units) padded to 4, then the
// unnormalised output row of head_dim.
constexpr int split_partial_floats(int head_dim) { return 4 + head_dim; }
// Whether a launch of a (split_rows <= 0, gemm_rec aside) can write the
// matrix-core GEMM's records of its outputs (a.gemm_rec).
bool attention_gemm_records(const SplitAttention &a);

// Per-device properties, cached once per device (thread-safe).
struct DeviceInfo {
    int device = -1;
    int cus = 0;          // compute units
    int max_threads = 1024;
};
const DeviceInfo &device_info();
// Workgroups of `block` threads and `lds` bytes of dynamic LDS the current
// device holds at once (per CU times CUs), cached.
int resident_blocks(const void *kernel, int block, size_t lds);

// ---------------------------------------------------------------- device --

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16));
    return static_cast<float>(h);
}

// Byte j of v as a float; the backend emits v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ float ubyte0(uint32_t v) { return static_cast<float>(v & 0xFFu); }
__device__ __forceinline__ float ubyte1(uint32_t v) { return static_cast<float>((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ubyte2(uint32_t v) { return static_cast<float>((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ubyte3(uint32_t v) { return static_cast<float>(v >> 24); }

// 16 / 8 / 2 byte loads at any 2-byte alignment.  gfx950 global loads
// tolerate unaligned addresses (Q6_K blocks are 210 B, so odd blocks are
// only 2-byte aligned); memcpy keeps the C++ side free of misaligned
// pointer dereferences.
__device__ __forceinline__ uint4 load16(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
__device__ __forceinline__ uint2 load8(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
__device__ __forceinline__ uint32_t load2(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// Scalar decode of element i of a block: the bit-exact semantics of
// q4_value / q6_value (inferencer.cu:454-487).
__device__ __forceinline__ float q4k_value(const uint8_t *block, int i) {
    float d = f16_bits_to_f32(load2(block));
    float dmin = f16_bits_to_f32(load2(block + 2));
    const uint8_t *s = block + 4;
    const uint8_t *qs = block + 16;
    int sub = i >> 5;
    int qi = (i >> 6) * 32 + (i & 31);
    int q = (i & 63) < 32 ? (qs[qi] & 15) : (qs[qi] >> 4);
    int sc, m;
    if (sub < 4) {
        sc = s[sub] & 63;
        m = s[sub + 4] & 63;
    } else {
        sc = (s[sub + 4] & 15) | ((s[sub - 4] >> 6) << 4);
        m = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4);
    }
    // Products are exact in fp32; the subtraction is the only rounding.
    return d * static_cast<float>(sc) * static_cast<float>(q) - dmin * static_cast<float>(m);
}

// The four fields of a Q6_K block: ql (128 B), qh (64 B), scales (16 B), d.
struct Q6Fields {
    const uint8_t *ql, *qh, *sc, *d;
};

// Block b of a row of nb blocks starting at `row`: contiguous in the GGUF
// layout, or in the split layout (QK_TYPE_Q6_K_SPLIT) the row's ql [nb][128],
// qh [nb][64], scales [nb][16] and d [nb] streams, every field 16-byte
// aligned when the row is.
__device__ __forceinline__ Q6Fields q6_fields(const uint8_t *row, int nb, int b, bool split) {
    if (split) return {row + b * 128, row + nb * 128 + b * 64, row + nb * 192 + b * 16, row + nb * 208 + b * 2};
    const uint8_t *blk = row + b * 210;
    return {blk, blk + 128, blk + 192, blk + 208};
}

__device__ __forceinline__ float q6k_value(const Q6Fields &f, int i) {
    int group = i >> 7, p = i & 127, lane = p & 31, part = p >> 5;
    int low = f.ql[group * 64 + (part & 1) * 32 + lane];
    low = part < 2 ? (low & 15) : (low >> 4);
    int high = (f.qh[group * 32 + lane] >> (part * 2)) & 3;
    int q = (low | (high << 4)) - 32;
    float d = f16_bits_to_f32(load2(f.d));
    int sc = static_cast<int8_t>(f.sc[group * 8 + part * 2 + (lane >> 4)]);
    return d * static_cast<float>(sc) * static_cast<float>(q);
}

__device__ __forceinline__ float q6k_value(const uint8_t *block, int i) {
    return q6k_value(Q6Fields{block, block + 128, block + 192, block + 208}, i);
}

// Lane-group sums within a wave (DPP row operations, then cross-row
// shuffles).
__device__ __forceinline__ float dpp_add(float v, int ctrl_id) {
    int moved;
    const int bits = __builtin_bit_cast(int, v);
    switch (ctrl_id) {
        case 0: moved = __builtin_amdgcn_update_dpp(0, bits, 0xB1, 0xF, 0xF, true); break;   // quad_perm 1,0,3,2
        case 1: moved = __builtin_amdgcn_update_dpp(0, bits, 0x4E, 0xF, 0xF, true); break;   // quad_perm 2,3,0,1
        case 2: moved = __builtin_amdgcn_update_dpp(0, bits, 0x141, 0xF, 0xF, true); break;  // row_half_mirror
        default: moved = __builtin_amdgcn_update_dpp(0, bits, 0x140, 0xF, 0xF, true); break; // row_mirror
    }
    return v + __builtin_bit_cast(float, moved);
}

// Sum over aligned groups of GROUP lanes; every lane of a group receives
// the group's total.  DPP covers groups up to a 16-lane row; wider groups
// finish with cross-row shuffles.
template <int GROUP>
__device__ __forceinline__ float group_sum(float v) {
    if (GROUP >= 2) v = dpp_add(v, 0);
    if (GROUP >= 4) v = dpp_add(v, 1);
    if (GROUP >= 8) v = dpp_add(v, 2);
    if (GROUP >= 16) v = dpp_add(v, 3);
    if (GROUP >= 32) v += __shfl_xor(v, 16);
    if (GROUP >= 64) v += __shfl_xor(v, 32);
    return v;
}

// 6-bit scale / min of Q4_K sub-blocks 4g + part (q4_scale_min,
// inferencer.cu:489-497), one per byte.
__device__ __forceinline__ void q4k_scale_min4(const uint4 &hdr, int g, uint32_t &sc, uint32_t &mn) {
    const uint32_t M = 0x0F0F0F0Fu;
    const uint32_t s03 = hdr.y, s47 = hdr.z, s811 = hdr.w;
    sc = g ? ((s811 & M) | ((s03 >> 2) & 0x30303030u)) : (s03 & 0x3F3F3F3Fu);
    mn = g ? (((s811 >> 4) & M) | ((s47 >> 2) & 0x30303030u)) : (s47 & 0x3F3F3F3Fu);
}

// The decode driver's FP32 GEMV over activation records (no staging): y_m =
// W_m x for the matrices, x given as records (cols/16 of them), optionally
// scaled by an RMSNorm factor reduced from the records' sums of squares
// (the records then hold x * gain), added into y (residual), and leaving the
// next GEMV's records: of y * gain with sums of squares (one matrix of whole
// 16-row blocks), or of SiLU(y_0) * y_1 (pair: gate and up).  With arg_v,
// the greedy pick's per-wave partials (count in *arg_parts).
struct RecGemv {
    const XGroup *rec = nullptr;
    const float *ss = nullptr;
    float norm_eps = 0.f;
    int accumulate = 0;
    int pair = 0;
    XGroup *rec_out = nullptr;
    float *ss_out = nullptr;
    const float *gain = nullptr;
    float *arg_v = nullptr;
    int *arg_i = nullptr;
    int *arg_parts = nullptr;
    // Instead of rec: the one-sequence attention's unmerged wide-form split
    // partials (launch_split_attention with defer_merge), n_parts splits per
    // head of part_hd, merged and made into records by every workgroup.
    // One matrix of 2048 columns with rec_out, no ss, pair or greedy pick.
    const float *parts = nullptr;
    int n_parts = 0;
    int part_hd = 0;
};
// Whether rows of cols columns have a record-GEMV launch plan, and whether
// the matrices' types can share one launch (a pair needs one type).
bool rec_gemv_supported(int cols, bool pair);
// Whether a one-matrix record GEMV of cols columns can take the attention's
// unmerged partials of head_dim (RecGemv::parts).
bool rec_gemv_mergeable(int cols, int head_dim);
bool rec_gemv_types(const qk_matrix *mats, int n_mats, bool pair);
int launch_rec_gemv(const qk_matrix *mats, int n_mats, int cols, const RecGemv &r, hipStream_t stream);
// The embedding of one token (device id) into out (cols fp32) and the
// records of out * gain with their sums of squares: embedding_cuda
// (inferencer.cu:806-819) plus the first QKV's activation records.
int launch_embedding_records(int type, const void *w, const int32_t *token, int cols, int vocab, float *out,
                             const float *gain, XGroup *rec, float *ss, hipStream_t stream);
// A split-layout Q6_K matrix (cols x rows) written back as GGUF blocks at
// dst (rows * cols / 256 * 210 bytes, not overlapping src); arguments
// already validated.
int launch_q6k_join(const void *src, void *dst, int cols, int rows, hipStream_t stream);

}  // namespace qk
