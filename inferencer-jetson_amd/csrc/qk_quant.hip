// qk_quant.hip - per-32 int8 activation quantization of the INT8 GEMV mode.
//
// Replaces quantize_x32_cuda (inferencer.cu:544-556) and quantize_batch_cuda
// (inferencer.cu:891-904): per group of 32 values, amax over the group,
// scale = amax/127 (1 when amax is 0), xq = clamp(rne(x/scale), -127, 127).
// The divide is IEEE (hipcc's default correctly rounded fp32 division) and
// rintf rounds half to even, so xq and xscale are bit-exact.  A wave holds
// two 32-value groups; the amax reduction stays inside each half-wave.
#include "qk_internal.h"

namespace qk {
namespace {

__global__ __launch_bounds__(256) void quantize_x32_kernel(const float *x, int ldx, int8_t *xq, int ldxq,
                                                           float *xscale, int ldscale, int cols) {
    const int token = blockIdx.y;
    const int index = blockIdx.x * 256 + threadIdx.x;
    const bool in_row = index < cols;
    const float value = in_row ? x[static_cast<int64_t>(token) * ldx + index] : 0.f;
    quantize_group_store(value, in_row, threadIdx.x & 31, xq + static_cast<int64_t>(token) * ldxq + index,
                         xscale + static_cast<int64_t>(token) * ldscale + (index >> 5));
}

// SiLU * up and the per-32 quantization in one pass (the INT8 step's input
// of the down GEMV): one thread per value, n a multiple of 32.
__global__ __launch_bounds__(256) void silu_mul_quantize_kernel(const float *gate, const float *up, int8_t *xq,
                                                                float *xscale, int n) {
    const int index = blockIdx.x * 256 + threadIdx.x;
    const bool in_row = index < n;
    const float value = in_row ? silu_mul_value(gate[index], up[index]) : 0.f;
    quantize_group_store(value, in_row, threadIdx.x & 31, xq + index, xscale + (index >> 5));
}

}  // namespace

int launch_silu_mul_quantize(const float *gate, const float *up, int8_t *xq, float *xscale, int n,
                             hipStream_t stream) {
    hipLaunchKernelGGL(silu_mul_quantize_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, gate, up, xq, xscale,
                       n);
    return launch_status("SiLU * up quantization launch");
}
}  // namespace qk

extern "C" int qk_quantize_x32(const float *x, int ldx, int8_t *xq, int ldxq, float *xscale, int ldscale, int cols,
                               int n_tokens, qk_stream stream) {
    if (!x || !xq || !xscale || cols < 1 || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_quantize_x32: null pointer or bad size");
    if (n_tokens == 0) return qk::ok();
    if (ldx < cols || ldxq < cols || ldscale < (cols + 31) / 32)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_quantize_x32: leading dimension smaller than the row");
    if (n_tokens > 65535) return qk::fail(QK_ERR_LIMIT, "qk_quantize_x32: too many tokens in one launch");
    hipLaunchKernelGGL(qk::quantize_x32_kernel, dim3((cols + 255) / 256, n_tokens), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, ldx, xq, ldxq, xscale, ldscale, cols);
    return qk::launch_status("qk_quantize_x32 launch");
}
