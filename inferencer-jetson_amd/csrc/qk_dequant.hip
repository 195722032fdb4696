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

__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t *w, float *out, int type, int nb,
                                                           int row0, int nrows) {
    const int i = threadIdx.x;
    const int bpb = type == QK_TYPE_Q4_K ? 144 : 210;
    const int64_t total = static_cast<int64_t>(nrows) * nb;
    for (int64_t blk = blockIdx.x; blk < total; blk += gridDim.x) {
        const int64_t r = blk / nb, b = blk - r * nb;
        const uint8_t *block = w + ((row0 + r) * nb + b) * bpb;
        float v = type == QK_TYPE_Q4_K ? q4k_value(block, i) : q6k_value(block, i);
        out[blk * 256 + i] = v;
    }
}

// Token ids are device data, so the range check of FastRunner::forward
// (inferencer.cu:1426-1427) happens here: an id outside [0, vocab) reads
// nothing and yields a NaN row.
__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t *w, const int32_t *tokens, float *out,
                                                        int type, int nb, int n_tokens, int vocab) {
    const int i = threadIdx.x;
    const int bpb = type == QK_TYPE_Q4_K ? 144 : 210;
    const int64_t total = static_cast<int64_t>(n_tokens) * nb;
    for (int64_t blk = blockIdx.x; blk < total; blk += gridDim.x) {
        const int64_t t = blk / nb, b = blk - t * nb;
        const int token = tokens[t];
        if (token < 0 || token >= vocab) {
            out[blk * 256 + i] = __builtin_nanf("");
            continue;
        }
        const uint8_t *block = w + (static_cast<int64_t>(token) * nb + b) * bpb;
        out[blk * 256 + i] = type == QK_TYPE_Q4_K ? q4k_value(block, i) : q6k_value(block, i);
    }
}

int grid_for(int64_t blocks) {
    int64_t cap = static_cast<int64_t>(device_info().cus) * 16;
    return static_cast<int>(blocks < cap ? (blocks > 0 ? blocks : 1) : cap);
}

}  // namespace
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
                       0, static_cast<hipStream_t>(stream), static_cast<const uint8_t *>(w), out, type, nb, row0,
                       nrows);
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
                       n_tokens, vocab);
    return qk::launch_status("qk_embedding launch");
}

}  // extern "C"
