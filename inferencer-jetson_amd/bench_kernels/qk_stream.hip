// qk_stream.hip - bandwidth reference kernels for bench.py (libqkbench.so).
//
// Not part of the GEMV library: a plain streaming read (the practical HBM
// ceiling for a read-only kernel such as the GEMV) and a plain copy of known
// size, whose FETCH_SIZE / WRITE_SIZE counters calibrate the per-dispatch
// traffic numbers that rocprofv3 reports for the GEMV kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

// Every thread streams 16-byte words with four loads in flight and folds
// them into one value; one word per block is written so nothing is elided.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4 *src, size_t n16, uint32_t *sink) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off);
    if ((threadIdx.x & 63) == 0) atomicXor(sink + blockIdx.x, acc);
}

__global__ __launch_bounds__(256) void copy_kernel(const uint4 *src, uint4 *dst, size_t n16) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

int device_cus() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        hipDeviceProp_t p{};
        if (hipGetDeviceProperties(&p, dev) == hipSuccess) cus = p.multiProcessorCount;
    }
    return cus;
}

int grid_blocks() { return device_cus() * 8; }

// The streaming read's grid: two workgroups per CU, four 16-byte loads in
// flight per lane, was the fastest of 1-16 workgroups per CU, 4-16 loads in
// flight and grid-stride or contiguous chunks per workgroup on MI355X
// (215 MB from 4 rotating buffers: 34.5 us, 6.25 TB/s; 8 per CU 40.5 us).
int read_blocks() { return device_cus() * 2; }

}  // namespace

extern "C" {

// Number of uint32 sink words stream_read needs.
int qkb_sink_words(void) { return grid_blocks(); }

int qkb_stream_read(const void *src, size_t bytes, uint32_t *sink, void *stream) {
    if (!src || !sink || (reinterpret_cast<uintptr_t>(src) & 15) || (bytes & 15)) return 1;
    hipLaunchKernelGGL(stream_read_kernel, dim3(read_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4 *>(src), bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

int qkb_copy(const void *src, void *dst, size_t bytes, void *stream) {
    if (!src || !dst || ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) || (bytes & 15))
        return 1;
    hipLaunchKernelGGL(copy_kernel, dim3(grid_blocks()), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4 *>(src), static_cast<uint4 *>(dst), bytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // extern "C"
