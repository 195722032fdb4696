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
// Rows whose length is a multiple of 4 (and 16-byte aligned) read x as
// float4 with every load of a thread in flight at once; the kernel is
// latency-bound at decode sizes, so the loads must not wait on each other.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *x, const float *weight, float *out, int n,
                                                      float eps, int vec4) {
    __shared__ float scratch[4];
    const float *xt = x + static_cast<int64_t>(blockIdx.x) * n;
    float *ot = out + static_cast<int64_t>(blockIdx.x) * n;
    float ss = 0.f;
    if (vec4) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xt);
        const float4 *w4 = reinterpret_cast<const float4 *>(weight);
        float4 *o4 = reinterpret_cast<float4 *>(ot);
        const int n4 = n >> 2;
        #pragma unroll 4
        for (int i = threadIdx.x; i < n4; i += 256) {
            const float4 v = x4[i];
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
        ss = block_sum256(ss, scratch);
        const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
        #pragma unroll 4
        for (int i = threadIdx.x; i < n4; i += 256) {
            const float4 v = x4[i], w = w4[i];
            o4[i] = make_float4(v.x * scale * w.x, v.y * scale * w.y, v.z * scale * w.z, v.w * scale * w.w);
        }
        return;
    }
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

// attention_cuda (inferencer.cu:981-1009), GQA, one query token.  One
// 1024-thread workgroup per KV head serves the G = heads / kv_heads query
// heads that share it, so every key and value row is read from memory once.
// At decode sizes the kernel is latency-bound: each phase issues all of its
// loads before it consumes them.
//   1. scores: thread t takes positions t, t + 1024, ...; it loads the key
//      row (16 float4 at a time) and dots it with the G query rows (LDS
//      broadcast), scaled by 1/sqrt(head_dim); scores go to LDS.
//   2. per-head maximum, exp, per-head sum (block reductions in LDS).
//   3. values: wave w owns a contiguous run of positions, lane = dimension;
//      the 16 partial vectors per head are added in wave order and divided
//      by the sum (deterministic).
constexpr int kAttnThreads = 1024;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kAttnMaxGroup = 8;
constexpr int kAttnMaxDimLanes = 4;   // head_dim <= 256: four dimensions per lane

struct AttnLds {
    float *qs;      // [G][head_dim]
    float *score;   // [G][pos + 1]
    float *part;    // [waves][G][head_dim]
    float *red;     // [waves][G]
};

__device__ __forceinline__ AttnLds attn_lds(float *smem, int G, int head_dim, int pos) {
    AttnLds l;
    l.qs = smem;
    l.score = l.qs + G * head_dim;
    l.part = l.score + G * (pos + 1);
    l.red = l.part + kAttnWaves * G * head_dim;
    return l;
}

// Block-wide reduction of G per-thread values (max or sum); every thread
// receives the G results in v.
template <bool MAX>
__device__ __forceinline__ void attn_block_reduce(float *v, int G, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int g = 0; g < G; ++g) {
        const float r = MAX ? wave_max(v[g]) : wave_sum(v[g]);
        if (lane == 0) red[wave * G + g] = r;
    }
    __syncthreads();
    for (int g = 0; g < G; ++g) {
        float r = red[g];
        for (int w = 1; w < kAttnWaves; ++w) r = MAX ? fmaxf(r, red[w * G + g]) : r + red[w * G + g];
        v[g] = r;
    }
    __syncthreads();
}

// q: the token's query rows of the G heads of KV head kvh (already rotated);
// kc / vc: the layer's caches offset to this KV head; out: the G output rows.
__device__ void attend_kv_head(const float *q, const float *kc, const float *vc, float *out, int pos, int G,
                               int head_dim, int kv_dim, float *smem) {
    const AttnLds L = attn_lds(smem, G, head_dim, pos);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = pos + 1;
    const float inv = 1.0f / sqrtf(static_cast<float>(head_dim));
    for (int i = tid; i < G * head_dim; i += kAttnThreads) L.qs[i] = q[i];
    __syncthreads();

    float m[kAttnMaxGroup];
    for (int g = 0; g < G; ++g) m[g] = -INFINITY;
    for (int t = tid; t < n; t += kAttnThreads) {
        const float4 *kr = reinterpret_cast<const float4 *>(kc + static_cast<int64_t>(t) * kv_dim);
        float dot[kAttnMaxGroup];
        for (int g = 0; g < G; ++g) dot[g] = 0.f;
        for (int c = 0; c < head_dim; c += 64) {
            float4 k4[16];
            const int nc = min(16, (head_dim - c) >> 2);
            #pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < nc) k4[j] = kr[(c >> 2) + j];
            for (int g = 0; g < G; ++g) {
                const float *qg = L.qs + g * head_dim + c;
                float a = dot[g];
                #pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (j < nc) {
                        a = fmaf(qg[4 * j], k4[j].x, a);
                        a = fmaf(qg[4 * j + 1], k4[j].y, a);
                        a = fmaf(qg[4 * j + 2], k4[j].z, a);
                        a = fmaf(qg[4 * j + 3], k4[j].w, a);
                    }
                dot[g] = a;
            }
        }
        for (int g = 0; g < G; ++g) {
            const float sc = dot[g] * inv;
            L.score[g * n + t] = sc;
            m[g] = fmaxf(m[g], sc);
        }
    }
    attn_block_reduce<true>(m, G, L.red);   // its barriers also publish score[]

    float den[kAttnMaxGroup];
    for (int g = 0; g < G; ++g) den[g] = 0.f;
    for (int t = tid; t < n; t += kAttnThreads)
        for (int g = 0; g < G; ++g) {
            const float e = expf(L.score[g * n + t] - m[g]);
            L.score[g * n + t] = e;
            den[g] += e;
        }
    attn_block_reduce<false>(den, G, L.red);

    const int per = (n + kAttnWaves - 1) / kAttnWaves;
    const int t0 = wave * per, t1 = min(n, t0 + per);
    const int dims = (head_dim + 63) >> 6;   // dimensions per lane
    float acc[kAttnMaxGroup][kAttnMaxDimLanes];
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int j = 0; j < kAttnMaxDimLanes; ++j) acc[g][j] = 0.f;
    int t = t0;
    for (; t + 4 <= t1; t += 4) {
        float v[4][kAttnMaxDimLanes];
        #pragma unroll
        for (int u = 0; u < 4; ++u)
            #pragma unroll
            for (int j = 0; j < kAttnMaxDimLanes; ++j) {
                const int d = lane + 64 * j;
                v[u][j] = (j < dims && d < head_dim) ? vc[static_cast<int64_t>(t + u) * kv_dim + d] : 0.f;
            }
        for (int g = 0; g < G; ++g)
            #pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float pr = L.score[g * n + t + u];
                #pragma unroll
                for (int j = 0; j < kAttnMaxDimLanes; ++j) acc[g][j] = fmaf(pr, v[u][j], acc[g][j]);
            }
    }
    for (; t < t1; ++t) {
        float v[kAttnMaxDimLanes];
        #pragma unroll
        for (int j = 0; j < kAttnMaxDimLanes; ++j) {
            const int d = lane + 64 * j;
            v[j] = (j < dims && d < head_dim) ? vc[static_cast<int64_t>(t) * kv_dim + d] : 0.f;
        }
        for (int g = 0; g < G; ++g) {
            const float pr = L.score[g * n + t];
            #pragma unroll
            for (int j = 0; j < kAttnMaxDimLanes; ++j) acc[g][j] = fmaf(pr, v[j], acc[g][j]);
        }
    }
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int j = 0; j < kAttnMaxDimLanes; ++j) {
            const int d = lane + 64 * j;
            if (j < dims && d < head_dim) L.part[(wave * G + g) * head_dim + d] = acc[g][j];
        }
    __syncthreads();
    for (int i = tid; i < G * head_dim; i += kAttnThreads) {
        const int g = i / head_dim;
        float s = 0.f;
        for (int w = 0; w < kAttnWaves; ++w) s += L.part[w * G * head_dim + i];
        out[i] = s / den[g];
    }
}

__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float *q, const float *key_cache,
                                                                 const float *value_cache, float *out, int layer,
                                                                 int pos, int context, int heads, int kv_heads,
                                                                 int head_dim) {
    extern __shared__ float smem[];
    const int kvh = blockIdx.x;
    const int G = heads / kv_heads;
    const int kv_dim = kv_heads * head_dim;
    const int64_t base = static_cast<int64_t>(layer) * context * kv_dim + kvh * head_dim;
    attend_kv_head(q + kvh * G * head_dim, key_cache + base, value_cache + base, out + kvh * G * head_dim, pos, G,
                   head_dim, kv_dim, smem);
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

size_t attention_lds_bytes(int pos, int head_dim, int group) {
    return static_cast<size_t>(group) * (head_dim + (pos + 1) + kAttnWaves * head_dim + kAttnWaves) * sizeof(float);
}

}  // namespace qk

extern "C" {

int qk_rmsnorm_f32(const float *x, const float *weight, float *out, int n, int n_tokens, float eps, qk_stream stream) {
    if (!x || !weight || !out || n < 1 || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rmsnorm_f32: null pointer or bad size");
    if (n_tokens == 0) return qk::ok();
    const int vec4 = n % 4 == 0 && qk::aligned(x, 16) && qk::aligned(weight, 16) && qk::aligned(out, 16);
    hipLaunchKernelGGL(qk::rmsnorm_kernel, dim3(n_tokens), dim3(256), 0, qk::S(stream), x, weight, out, n, eps, vec4);
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
    if (heads / kv_heads > qk::kAttnMaxGroup)
        return qk::fail(QK_ERR_LIMIT, "qk_attention_f32: more than 8 query heads per KV head");
    if (!qk::aligned(key_cache, 16) || !qk::aligned(value_cache, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_attention_f32: caches must be 16-byte aligned");
    const size_t lds = qk::attention_lds_bytes(pos, head_dim, heads / kv_heads);
    if (lds > 150 * 1024) return qk::fail(QK_ERR_LIMIT, "qk_attention_f32: position beyond the LDS score buffer");
    hipLaunchKernelGGL(qk::attention_kernel, dim3(kv_heads), dim3(qk::kAttnThreads), lds, qk::S(stream), q, key_cache,
                       value_cache, out, layer, pos, context, heads, kv_heads, head_dim);
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
