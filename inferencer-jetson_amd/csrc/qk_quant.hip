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
    const float value = index < cols ? x[static_cast<int64_t>(token) * ldx + index] : 0.f;
    float amax = fabsf(value);
    #pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float scale = amax > 0.f ? amax / 127.f : 1.f;
    const int group = index >> 5;
    if ((threadIdx.x & 31) == 0 && index < cols) xscale[static_cast<int64_t>(token) * ldscale + group] = scale;
    if (index < cols) {
        int q = static_cast<int>(rintf(value / scale));
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        xq[static_cast<int64_t>(token) * ldxq + index] = static_cast<int8_t>(q);
    }
}

}  // namespace
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
