// qk_step.hip - the decode step's small kernels around the GEMVs.
//
// Replace rmsnorm_cuda, rope_cuda / cache_cuda / rope_cache_cuda,
// attention_cuda, add_cuda, silu_cuda and the two-stage argmax
// (inferencer.cu:821-834, 906-1009, 1043-1099), generalised from the
// reference's hard-coded head_dim 128 / 64 RoPE frequencies to any even
// head_dim, and written for wave64.
#include "qk_internal.h"

#include <cmath>

namespace qk {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Block-wide sum for blockDim.x = 256 (4 waves); every thread gets the total.
__device__ __forceinline__ float block_sum256(float v, float *scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    return (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
}

__device__ __forceinline__ float block_max256(float v, float *scratch) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
}

// rmsnorm_cuda (inferencer.cu:821-834): one 256-thread block per token.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *x, const float *weight, float *out, int n,
                                                      float eps) {
    __shared__ float scratch[4];
    const float *xt = x + static_cast<int64_t>(blockIdx.x) * n;
    float *ot = out + static_cast<int64_t>(blockIdx.x) * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(xt[i], xt[i], ss);
    ss = block_sum256(ss, scratch);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
    for (int i = threadIdx.x; i < n; i += 256) ot[i] = xt[i] * scale * weight[i];
}

// rope_cache_cuda (inferencer.cu:930-951) for any head_dim: rotate adjacent
// pairs of q in place; rotate k into the key cache and copy v.
__global__ void rope_kv_kernel(float *q, const float *k, const float *v, const float *cosine, const float *sine,
                               float *key_cache, float *value_cache, int layer, int pos, int context, int q_pairs,
                               int kv_pairs, int half_head) {
    const int pair = blockIdx.x * blockDim.x + threadIdx.x;
    if (pair >= q_pairs) return;
    const int f = pair % half_head;
    const float c = cosine[static_cast<int64_t>(pos) * half_head + f];
    const float s = sine[static_cast<int64_t>(pos) * half_head + f];
    const int i = pair * 2;
    const float q0 = q[i], q1 = q[i + 1];
    q[i] = q0 * c - q1 * s;
    q[i + 1] = q0 * s + q1 * c;
    if (pair < kv_pairs) {
        const int kv_dim = kv_pairs * 2;
        const int64_t o = (static_cast<int64_t>(layer) * context + pos) * kv_dim + i;
        const float k0 = k[i], k1 = k[i + 1];
        key_cache[o] = k0 * c - k1 * s;
        key_cache[o + 1] = k0 * s + k1 * c;
        value_cache[o] = v[i];
        value_cache[o + 1] = v[i + 1];
    }
}

// attention_cuda (inferencer.cu:981-1009): one 256-thread block per query
// head.  Phase 1: thread t scores positions t, t+256, ... (each reads its
// own contiguous key row), scores staged in LDS.  Phase 2: softmax
// normalisation.  Phase 3: thread (i, grp) accumulates p_t * v_t[i] over
// positions t = grp mod G, coalesced over i; the G partial vectors are
// summed in LDS.
__global__ __launch_bounds__(256) void attention_kernel(const float *q, const float *key_cache,
                                                        const float *value_cache, float *out, int layer, int pos,
                                                        int context, int heads, int kv_heads, int head_dim) {
    extern __shared__ float smem[];
    float *qs = smem;                      // head_dim
    float *score = smem + head_dim;        // pos + 1
    float *part = score + pos + 1;         // 256
    __shared__ float scratch[4];
    const int head = blockIdx.x;
    const int group = heads / kv_heads;
    const int kvh = head / group;
    const int kv_dim = kv_heads * head_dim;
    const float inv = 1.0f / sqrtf(static_cast<float>(head_dim));
    const float *kc = key_cache + static_cast<int64_t>(layer) * context * kv_dim + kvh * head_dim;
    const float *vc = value_cache + static_cast<int64_t>(layer) * context * kv_dim + kvh * head_dim;
    for (int i = threadIdx.x; i < head_dim; i += 256) qs[i] = q[head * head_dim + i];
    __syncthreads();
    float mx = -INFINITY;
    for (int t = threadIdx.x; t <= pos; t += 256) {
        const float *kr = kc + static_cast<int64_t>(t) * kv_dim;
        float dot = 0.f;
        for (int i = 0; i < head_dim; i += 4) {
            float4 kv4 = *reinterpret_cast<const float4 *>(kr + i);
            dot = fmaf(qs[i], kv4.x, dot);
            dot = fmaf(qs[i + 1], kv4.y, dot);
            dot = fmaf(qs[i + 2], kv4.z, dot);
            dot = fmaf(qs[i + 3], kv4.w, dot);
        }
        dot *= inv;
        score[t] = dot;
        mx = fmaxf(mx, dot);
    }
    mx = block_max256(mx, scratch);
    float den = 0.f;
    for (int t = threadIdx.x; t <= pos; t += 256) {
        float e = expf(score[t] - mx);
        score[t] = e;
        den += e;
    }
    den = block_sum256(den, scratch);   // its barriers also publish score[]
    const int groups = 256 / head_dim;  // head_dim divides 256 (checked on the host)
    const int i = threadIdx.x % head_dim, grp = threadIdx.x / head_dim;
    float acc = 0.f;
    if (grp < groups)
        for (int t = grp; t <= pos; t += groups) acc = fmaf(score[t], vc[static_cast<int64_t>(t) * kv_dim + i], acc);
    part[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < head_dim) {
        float s = 0.f;
        for (int g = 0; g < groups; ++g) s += part[g * head_dim + threadIdx.x];
        out[head * head_dim + threadIdx.x] = s / den;
    }
}

__global__ void add_kernel(float *x, const float *y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += y[i];
}

__global__ void silu_mul_kernel(float *gate, const float *up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float g = gate[i];
        gate[i] = g / (1.f + expf(-g)) * up[i];
    }
}

// (value, index) order of argmax_blocks_cuda / argmax_final_cuda
// (inferencer.cu:1063-1099): larger value wins, equal values keep the lower
// index.
__device__ __forceinline__ void arg_better(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

constexpr int kArgmaxBlock = 1024;

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *v, int n, float *pv, int *pi) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    const int base = blockIdx.x * kArgmaxBlock;
    for (int k = threadIdx.x; k < kArgmaxBlock; k += 256) {
        const int i = base + k;
        if (i < n) arg_better(bv, bi, v[i], i);
    }
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float ov = __shfl_xor(bv, off);
        int oi = __shfl_xor(bi, off);
        arg_better(bv, bi, ov, oi);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) arg_better(bv, bi, sv[w], si[w]);
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float *pv, const int *pi, int parts, int32_t *out) {
    __shared__ float sv[4];
    __shared__ int si[4];
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int k = threadIdx.x; k < parts; k += 256) arg_better(bv, bi, pv[k], pi[k]);
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        float ov = __shfl_xor(bv, off);
        int oi = __shfl_xor(bi, off);
        arg_better(bv, bi, ov, oi);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) arg_better(bv, bi, sv[w], si[w]);
        // All -inf (or NaN) input: fall back to index 0 like an empty tree.
        *out = bi == 0x7FFFFFFF ? 0 : bi;
    }
}

inline hipStream_t S(qk_stream s) { return static_cast<hipStream_t>(s); }

}  // namespace

size_t attention_lds_bytes(int pos, int head_dim) {
    return (static_cast<size_t>(head_dim) + pos + 1 + 256) * sizeof(float);
}

}  // namespace qk

extern "C" {

int qk_rmsnorm_f32(const float *x, const float *weight, float *out, int n, int n_tokens, float eps, qk_stream stream) {
    if (!x || !weight || !out || n < 1 || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rmsnorm_f32: null pointer or bad size");
    if (n_tokens == 0) return qk::ok();
    hipLaunchKernelGGL(qk::rmsnorm_kernel, dim3(n_tokens), dim3(256), 0, qk::S(stream), x, weight, out, n, eps);
    return qk::launch_status("qk_rmsnorm_f32 launch");
}

int qk_rope_kv_write(float *q, const float *k, const float *v, const float *cosine, const float *sine,
                     float *key_cache, float *value_cache, int layer, int pos, int context, int heads, int kv_heads,
                     int head_dim, qk_stream stream) {
    if (!q || !k || !v || !cosine || !sine || !key_cache || !value_cache)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rope_kv_write: null pointer");
    if (head_dim < 2 || head_dim % 2 || heads < 1 || kv_heads < 1 || heads % kv_heads || layer < 0 || pos < 0 ||
        pos >= context)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rope_kv_write: bad head layout or position outside context");
    const int q_pairs = heads * head_dim / 2, kv_pairs = kv_heads * head_dim / 2;
    hipLaunchKernelGGL(qk::rope_kv_kernel, dim3((q_pairs + 255) / 256), dim3(256), 0, qk::S(stream), q, k, v, cosine,
                       sine, key_cache, value_cache, layer, pos, context, q_pairs, kv_pairs, head_dim / 2);
    return qk::launch_status("qk_rope_kv_write launch");
}

int qk_attention_f32(const float *q, const float *key_cache, const float *value_cache, float *out, int layer, int pos,
                     int context, int heads, int kv_heads, int head_dim, qk_stream stream) {
    if (!q || !key_cache || !value_cache || !out)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_attention_f32: null pointer");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || layer < 0 || pos < 0 || pos >= context)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_attention_f32: bad head layout or position outside context");
    if (head_dim < 4 || head_dim % 4 || 256 % head_dim)
        return qk::fail(QK_ERR_LIMIT, "qk_attention_f32: head_dim must be a multiple of 4 dividing 256");
    if (!qk::aligned(key_cache, 16) || !qk::aligned(value_cache, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_attention_f32: caches must be 16-byte aligned");
    const size_t lds = qk::attention_lds_bytes(pos, head_dim);
    if (lds > 150 * 1024) return qk::fail(QK_ERR_LIMIT, "qk_attention_f32: position beyond the LDS score buffer");
    hipLaunchKernelGGL(qk::attention_kernel, dim3(heads), dim3(256), lds, qk::S(stream), q, key_cache, value_cache, out,
                       layer, pos, context, heads, kv_heads, head_dim);
    return qk::launch_status("qk_attention_f32 launch");
}

int qk_add_f32(float *x, const float *y, int n, qk_stream stream) {
    if (!x || !y || n < 0) return qk::fail(QK_ERR_INVALID_ARG, "qk_add_f32: null pointer or negative size");
    if (n == 0) return qk::ok();
    hipLaunchKernelGGL(qk::add_kernel, dim3((n + 255) / 256), dim3(256), 0, qk::S(stream), x, y, n);
    return qk::launch_status("qk_add_f32 launch");
}

int qk_silu_mul_f32(float *gate, const float *up, int n, qk_stream stream) {
    if (!gate || !up || n < 0) return qk::fail(QK_ERR_INVALID_ARG, "qk_silu_mul_f32: null pointer or negative size");
    if (n == 0) return qk::ok();
    hipLaunchKernelGGL(qk::silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, qk::S(stream), gate, up, n);
    return qk::launch_status("qk_silu_mul_f32 launch");
}

size_t qk_argmax_workspace_bytes(int n) {
    if (n < 1) return 0;
    const size_t parts = (static_cast<size_t>(n) + qk::kArgmaxBlock - 1) / qk::kArgmaxBlock;
    return parts * (sizeof(float) + sizeof(int));
}

int qk_argmax_f32(const float *v, int n, int32_t *out, void *workspace, qk_stream stream) {
    if (!v || !out || !workspace || n < 1)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_argmax_f32: null pointer or empty input");
    if (!qk::aligned(workspace, 4)) return qk::fail(QK_ERR_ALIGN, "qk_argmax_f32: workspace must be 4-byte aligned");
    const int parts = (n + qk::kArgmaxBlock - 1) / qk::kArgmaxBlock;
    float *pv = static_cast<float *>(workspace);
    int *pi = reinterpret_cast<int *>(pv + parts);
    hipLaunchKernelGGL(qk::argmax_partial_kernel, dim3(parts), dim3(256), 0, qk::S(stream), v, n, pv, pi);
    hipLaunchKernelGGL(qk::argmax_final_kernel, dim3(1), dim3(256), 0, qk::S(stream), pv, pi, parts, out);
    return qk::launch_status("qk_argmax_f32 launch");
}

}  // extern "C"
