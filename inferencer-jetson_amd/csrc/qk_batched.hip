// qk_batched.hip - multi-token FP32 dequant-GEMV entry points.
//
// FP32 semantics for the reference's INT8-only batched path
// (FastRunner::batch_matvec + gemv_batch_dp4a, inferencer.cu:1265-1278,
// 678-699; qkv_batch_cuda / gate_up_batch_cuda, inferencer.cu:701-751).
// Token t reads x + t*ldx and writes y + t*ldy.  Few tokens run the tiled
// GEMV kernel with blockIdx.y = token: blocks of one tile range run side by
// side, so the repeated weight reads of the other tokens hit L2.
#include "qk_internal.h"

namespace qk {
int launch_gemv_f32(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                    const int *ldy, hipStream_t stream);
}

namespace {

int check_batched(const char *where, const float *x, int ldx, int cols, int n_tokens) {
    if (!x || n_tokens < 0) return qk::fail(QK_ERR_INVALID_ARG, std::string(where) + ": null x or negative count");
    if (ldx < cols) return qk::fail(QK_ERR_INVALID_ARG, std::string(where) + ": ldx smaller than cols");
    if (!qk::aligned(x, 16) || ldx % 4)
        return qk::fail(QK_ERR_ALIGN, std::string(where) + ": x and ldx must keep 16-byte alignment");
    return QK_OK;
}

}  // namespace

extern "C" {

size_t qk_gemv_batched_workspace_bytes(int cols, int n_tokens) {
    if (cols <= 0 || n_tokens <= 0) return 0;
    // fp16 high and low halves of every activation, tokens padded to 32.
    const size_t padded = (static_cast<size_t>(n_tokens) + 31) / 32 * 32;
    return padded * static_cast<size_t>(cols) * 4;
}

int qk_gemv_batched_f32(int type, const void *w, const float *x, int ldx, float *y, int ldy, int cols, int rows,
                        int n_tokens, void *workspace, size_t workspace_bytes, qk_stream stream) {
    int st = qk::check_weights("qk_gemv_batched_f32", type, w, cols, rows);
    if (st) return st;
    if ((st = check_batched("qk_gemv_batched_f32", x, ldx, cols, n_tokens))) return st;
    if (!y || ldy < rows) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_batched_f32: null y or ldy smaller than rows");
    if (!qk::aligned(y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_gemv_batched_f32: y must be 4-byte aligned");
    if (n_tokens == 0) return qk::ok();
    (void)workspace;
    (void)workspace_bytes;
    const qk_matrix m{type, rows, w, y};
    return qk::launch_gemv_f32(&m, 1, x, ldx, cols, n_tokens, &ldy, static_cast<hipStream_t>(stream));
}

int qk_gemv_multi_batched_f32(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                              void *workspace, size_t workspace_bytes, qk_stream stream) {
    if (!mats || n_mats < 1 || n_mats > QK_MAX_FUSED)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_batched_f32: need 1.." + std::to_string(QK_MAX_FUSED) +
                                                " matrices");
    int st = check_batched("qk_gemv_multi_batched_f32", x, ldx, cols, n_tokens);
    if (st) return st;
    int ldy[QK_MAX_FUSED];
    for (int m = 0; m < n_mats; ++m) {
        if ((st = qk::check_weights("qk_gemv_multi_batched_f32", mats[m].type, mats[m].w, cols, mats[m].rows)))
            return st;
        if (!mats[m].y) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_batched_f32: null output pointer");
        if (!qk::aligned(mats[m].y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_gemv_multi_batched_f32: misaligned output");
        ldy[m] = mats[m].rows;
    }
    if (n_tokens == 0) return qk::ok();
    (void)workspace;
    (void)workspace_bytes;
    return qk::launch_gemv_f32(mats, n_mats, x, ldx, cols, n_tokens, ldy, static_cast<hipStream_t>(stream));
}

}  // extern "C"
