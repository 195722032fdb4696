// qk_dequant.hip - bit-exact Q4_K / Q6_K dequantization and embedding gather.
//
// Replaces embedding_cuda / embedding_batch_cuda (inferencer.cu:806-819),
// generalised to either format, and exposes the q4_value / q6_value decode
// (inferencer.cu:454-487) for whole rows.  One 256-thread block handles one
// super-block: thread i decodes element i, so a block's reads hit one
// 144 / 210-byte span and its 1 KiB of fp32 output is written coalesced.
#include "qk_internal.h"

namespace qk {
namespace {

// Element i of block b of a row (any of the three layouts).
__device__ __forceinline__ float block_value(const uint8_t *row, int type, int nb, int b, int i) {
    if (type == QK_TYPE_Q4_K) return q4k_value(row + b * 144, i);
    return q6k_value(q6_fields(row, nb, b, type == QK_TYPE_Q6_K_SPLIT), i);
}

__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t *w, float *out, int type, int nb,
                                                           int64_t row_bytes, int row0, int nrows) {
    const int i = threadIdx.x;
    const int64_t total = static_cast<int64_t>(nrows) * nb;
    for (int64_t blk = blockIdx.x; blk < total; blk += gridDim.x) {
        const int64_t r = blk / nb, b = blk - r * nb;
        out[blk * 256 + i] = block_value(w + (row0 + r) * row_bytes, type, nb, static_cast<int>(b), i);
    }
}

// Token ids are device data, so the range check of FastRunner::forward
// (inferencer.cu:1426-1427) happens here: an id outside [0, vocab) reads
// nothing and yields a NaN row.
__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t *w, const int32_t *tokens, float *out,
                                                        int type, int nb, int64_t row_bytes, int n_tokens,
                                                        int vocab) {
    const int i = threadIdx.x;
    const int64_t total = static_cast<int64_t>(n_tokens) * nb;
    for (int64_t blk = blockIdx.x; blk < total; blk += gridDim.x) {
        const int64_t t = blk / nb, b = blk - t * nb;
        const int token = tokens[t];
        if (token < 0 || token >= vocab) {
            out[blk * 256 + i] = __builtin_nanf("");
            continue;
        }
        out[blk * 256 + i] = block_value(w + static_cast<int64_t>(token) * row_bytes, type, nb, static_cast<int>(b), i);
    }
}

// One token's embedding row, block b = blockIdx.x (embedding_kernel's
// arithmetic), plus the activation records of out * gain for the first GEMV
// that reads it and their sums of squares of out.
__global__ __launch_bounds__(256) void embedding_records_kernel(const uint8_t *w, const int32_t *token, float *out,
                                                                int type, int nb, int64_t row_bytes, int vocab,
                                                                const float *gain, XGroup *rec, float *ss) {
    __shared__ float v[256];
    const int i = threadIdx.x, b = blockIdx.x;
    const int t = *token;
    const float x = t < 0 || t >= vocab ? __builtin_nanf("")
                                        : block_value(w + static_cast<int64_t>(t) * row_bytes, type, nb, b, i);
    out[b * 256 + i] = x;
    v[i] = x;
    __syncthreads();
    if (i < 16) {
        float g[16], sq = 0.f;
        #pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float xv = v[i * 16 + k];
            sq = fmaf(xv, xv, sq);
            g[k] = gain ? xv * gain[b * 256 + i * 16 + k] : xv;
        }
        rec[b * 16 + i] = make_group_regs(g);
        ss[b * 16 + i] = sq;
    }
}

// GGUF Q6_K rows -> split rows: one 64-thread workgroup per block moves its
// 105 two-byte units (the source block is only 2-byte aligned): units 0..63
// are ql, 64..95 qh, 96..103 scales, 104 d.  The workgroup of a row's last
// block also zeroes the row's padding.
__global__ __launch_bounds__(64) void q6k_split_kernel(const uint8_t *src, uint8_t *dst, int nb, int64_t dst_row_bytes,
                                                       int64_t nblocks) {
    for (int64_t blk = blockIdx.x; blk < nblocks; blk += gridDim.x) {
        const int64_t r = blk / nb;
        const int b = static_cast<int>(blk - r * nb);
        const uint8_t *s = src + blk * 210;
        uint8_t *row = dst + r * dst_row_bytes;
        const Q6Fields f = q6_fields(row, nb, b, true);
        for (int u = threadIdx.x; u < 105; u += 64) {
            const uint16_t v = static_cast<uint16_t>(load2(s + 2 * u));
            const uint8_t *o = u < 64 ? f.ql + 2 * u : u < 96 ? f.qh + 2 * (u - 64) : u < 104 ? f.sc + 2 * (u - 96) : f.d;
            __builtin_memcpy(const_cast<uint8_t *>(o), &v, 2);
        }
        if (b == nb - 1)
            for (int64_t i = static_cast<int64_t>(nb) * 210 + threadIdx.x; i < dst_row_bytes; i += 64) row[i] = 0;
    }
}

// The inverse: split rows back into 210-byte GGUF blocks (one workgroup per
// block, grid-stride).
__global__ __launch_bounds__(64) void q6k_join_kernel(const uint8_t *src, uint8_t *dst, int nb, int64_t src_row_bytes,
                                                      int64_t nblocks) {
    for (int64_t blk = blockIdx.x; blk < nblocks; blk += gridDim.x) {
        const int64_t r = blk / nb;
        const int b = static_cast<int>(blk - r * nb);
        const Q6Fields f = q6_fields(src + r * src_row_bytes, nb, b, true);
        uint8_t *d = dst + blk * 210;
        for (int u = threadIdx.x; u < 105; u += 64) {
            const uint8_t *i = u < 64 ? f.ql + 2 * u : u < 96 ? f.qh + 2 * (u - 64) : u < 104 ? f.sc + 2 * (u - 96) : f.d;
            const uint16_t v = static_cast<uint16_t>(load2(i));
            __builtin_memcpy(d + 2 * u, &v, 2);
        }
    }
}

int grid_for(int64_t blocks) {
    int64_t cap = static_cast<int64_t>(device_info().cus) * 16;
    return static_cast<int>(blocks < cap ? (blocks > 0 ? blocks : 1) : cap);
}

}  // namespace

int launch_q6k_join(const void *src, void *dst, int cols, int rows, hipStream_t stream) {
    const int nb = cols / 256;
    const int64_t nblocks = static_cast<int64_t>(rows) * nb;
    hipLaunchKernelGGL(q6k_join_kernel, dim3(grid_for(nblocks)), dim3(64), 0, stream, static_cast<const uint8_t *>(src),
                       static_cast<uint8_t *>(dst), nb, row_bytes(QK_TYPE_Q6_K_SPLIT, nb), nblocks);
    return launch_status("Q6_K join launch");
}

int launch_embedding_records(int type, const void *w, const int32_t *token, int cols, int vocab, float *out,
                             const float *gain, XGroup *rec, float *ss, hipStream_t stream) {
    const int nb = cols / 256;
    hipLaunchKernelGGL(embedding_records_kernel, dim3(nb), dim3(256), 0, stream, static_cast<const uint8_t *>(w),
                       token, out, type, nb, row_bytes(type, nb), vocab, gain, rec, ss);
    return launch_status("embedding records launch");
}

}  // namespace qk

extern "C" {

int qk_dequant_rows(int type, const void *w, float *out, int cols, int row0, int nrows, qk_stream stream) {
    int st = qk::check_weights("qk_dequant_rows", type, w, cols, 1);
    if (st) return st;
    if (!out || row0 < 0 || nrows < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_dequant_rows: null output or negative row range");
    if (nrows == 0) return qk::ok();
    const int nb = cols / 256;
    hipLaunchKernelGGL(qk::dequant_rows_kernel, dim3(qk::grid_for(static_cast<int64_t>(nrows) * nb)), dim3(256),
                       0, static_cast<hipStream_t>(stream), static_cast<const uint8_t *>(w), out, type, nb,
                       qk::row_bytes(type, nb), row0, nrows);
    return qk::launch_status("qk_dequant_rows launch");
}

int qk_embedding(int type, const void *w, const int32_t *tokens, int n_tokens, float *out, int cols, int vocab,
                 qk_stream stream) {
    int st = qk::check_weights("qk_embedding", type, w, cols, vocab);
    if (st) return st;
    if (!tokens || !out || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_embedding: null pointer or negative token count");
    if (n_tokens == 0) return qk::ok();
    const int nb = cols / 256;
    hipLaunchKernelGGL(qk::embedding_kernel, dim3(qk::grid_for(static_cast<int64_t>(n_tokens) * nb)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t *>(w), tokens, out, type, nb,
                       qk::row_bytes(type, nb), n_tokens, vocab);
    return qk::launch_status("qk_embedding launch");
}

int qk_q6k_split(const void *src, void *dst, int cols, int rows, qk_stream stream) {
    int st = qk::check_weights("qk_q6k_split", QK_TYPE_Q6_K, src, cols, rows);
    if (st) return st;
    if (!dst) return qk::fail(QK_ERR_INVALID_ARG, "qk_q6k_split: null destination");
    if (!qk::aligned(dst, 16)) return qk::fail(QK_ERR_ALIGN, "qk_q6k_split: destination not 16-byte aligned");
    const int nb = cols / 256;
    const int64_t src_bytes = static_cast<int64_t>(rows) * nb * 210;
    const int64_t dst_row = qk::row_bytes(QK_TYPE_Q6_K_SPLIT, nb);
    const uint8_t *s = static_cast<const uint8_t *>(src);
    const uint8_t *d = static_cast<const uint8_t *>(dst);
    if (d < s + src_bytes && s < d + dst_row * rows)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_q6k_split: source and destination overlap");
    const int64_t nblocks = static_cast<int64_t>(rows) * nb;
    hipLaunchKernelGGL(qk::q6k_split_kernel, dim3(qk::grid_for(nblocks)), dim3(64), 0, static_cast<hipStream_t>(stream),
                       s, static_cast<uint8_t *>(dst), nb, dst_row, nblocks);
    return qk::launch_status("qk_q6k_split launch");
}

}  // extern "C"
