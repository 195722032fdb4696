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

// Query rows, scores of positions 0..pos, the 8 waves' partial outputs and
// their reduction slots, for `group` query heads.
__host__ __device__ size_t attention_lds_bytes(int pos, int head_dim, int group) {
    return static_cast<size_t>(group) * (head_dim + (pos + 1) + 8 * head_dim + 8) * sizeof(float);
}

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
// 512-thread workgroup per KV head serves the G = heads / kv_heads query
// heads that share it, so every key and value row is read from memory once.
//   1. scores: 16 lanes per key row, each row dotted with the G query rows
//      (held in registers), 16-lane DPP sums, scaled by 1/sqrt(head_dim);
//      scores go to LDS.
//   2. per-head maximum, exp, per-head sum (block reductions in LDS).
//   3. values: wave w owns a contiguous run of positions, 16 lanes per row;
//      the 8 partial vectors per head are added in wave order and divided by
//      the sum (deterministic).
// Each phase keeps several steps of loads in flight before it consumes them.
constexpr int kAttnThreads = 512;
constexpr int kAttnWaves = kAttnThreads / 64;
static_assert(kAttnWaves == 8, "attention_lds_bytes sizes 8 waves");

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
template <bool MAX, int G>
__device__ __forceinline__ void attn_block_reduce(float *v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    #pragma unroll
    for (int g = 0; g < G; ++g) {
        const float r = MAX ? wave_max(v[g]) : wave_sum(v[g]);
        if (lane == 0) red[wave * G + g] = r;
    }
    __syncthreads();
    #pragma unroll
    for (int g = 0; g < G; ++g) {
        float r = red[g];
        for (int w = 1; w < kAttnWaves; ++w) r = MAX ? fmaxf(r, red[w * G + g]) : r + red[w * G + g];
        v[g] = r;
    }
    __syncthreads();
}

__device__ __forceinline__ float4 ld_row4(__amdgpu_buffer_rsrc_t r, int lane_off, int row_off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, row_off, 0));
}

__device__ __forceinline__ float dot4(const float4 &a, const float4 &b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    return fmaf(a.w, b.w, acc);
}

// q: the token's query rows of the G heads of KV head kvh (already rotated);
// kc / vc: the layer's caches offset to this KV head's first row; out: the G
// output rows.  G query heads per KV head and DL = ceil(head_dim / 64) are
// compile-time, so every per-head array stays in registers.
//
// Memory access: 16 lanes share a cache row (lane sub reads dimensions
// 64c + 4*sub .. +3 of chunk c as one float4), so one load instruction of a
// wave covers four whole rows.  Rows are read through buffer resources that
// span exactly the rows a phase may read: a row past the range reads as zero.
template <int G, int DL>
__device__ __forceinline__ void attend_kv_head(const float *q, const float *kc, const float *vc, float *out, int pos,
                                               int head_dim, int kv_dim, float *smem) {
    const AttnLds L = attn_lds(smem, G, head_dim, pos);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane & 15, rq = lane >> 4;
    const bool act = 4 * sub < head_dim;         // head_dim < 64 leaves lanes idle
    const int n = pos + 1;
    const int row_bytes = kv_dim * 4;
    const int lane_off = (rq * kv_dim + 4 * min(sub, max(head_dim / 4 - 1, 0))) * 4;
    constexpr int U = (16 / DL) / (G > 4 ? 2 : 1);   // 4-row steps in flight per wave
    const float inv = 1.0f / sqrtf(static_cast<float>(head_dim));
    for (int i = tid; i < G * head_dim; i += kAttnThreads) L.qs[i] = q[i];
    __syncthreads();
    float4 qv[G][DL];
    #pragma unroll
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int c = 0; c < DL; ++c)
            qv[g][c] = act ? *reinterpret_cast<const float4 *>(L.qs + g * head_dim + 64 * c + 4 * sub)
                           : make_float4(0.f, 0.f, 0.f, 0.f);

    // 1. Scores.  Step u of wave w covers rows it0 + (u*waves + w)*4 + rq.
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(kc), 0, n * row_bytes, 0x00020000);
    float m[G];
    #pragma unroll
    for (int g = 0; g < G; ++g) m[g] = -INFINITY;
    for (int it0 = 0; it0 < n; it0 += kAttnWaves * 4 * U) {
        float4 k4[U][DL];
        #pragma unroll
        for (int u = 0; u < U; ++u)
            #pragma unroll
            for (int c = 0; c < DL; ++c)
                k4[u][c] = ld_row4(krs, lane_off + 256 * c, (it0 + (u * kAttnWaves + wave) * 4) * row_bytes);
        #pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = it0 + (u * kAttnWaves + wave) * 4 + rq;
            #pragma unroll
            for (int g = 0; g < G; ++g) {
                float a = 0.f;
                #pragma unroll
                for (int c = 0; c < DL; ++c) a = dot4(qv[g][c], k4[u][c], a);
                const float sc = group_sum<16>(a) * inv;
                if (t < n) {
                    if (sub == 0) L.score[g * n + t] = sc;
                    m[g] = fmaxf(m[g], sc);
                }
            }
        }
    }
    attn_block_reduce<true, G>(m, L.red);   // its barriers also publish score[]

    // 2. exp and the per-head sums.
    float den[G];
    #pragma unroll
    for (int g = 0; g < G; ++g) den[g] = 0.f;
    for (int t = tid; t < n; t += kAttnThreads)
        #pragma unroll
        for (int g = 0; g < G; ++g) {
            const float e = expf(L.score[g * n + t] - m[g]);
            L.score[g * n + t] = e;
            den[g] += e;
        }
    attn_block_reduce<false, G>(den, L.red);

    // 3. Values: wave w owns rows t0 .. t1-1, four per step (row t0 + 4s + rq).
    const int per = (n + kAttnWaves - 1) / kAttnWaves;
    const int t0 = min(n, wave * per), t1 = min(n, t0 + per);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(vc + static_cast<int64_t>(t0) * kv_dim), 0, (t1 - t0) * row_bytes, 0x00020000);
    float4 acc[G][DL];
    #pragma unroll
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int c = 0; c < DL; ++c) acc[g][c] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0; s0 < t1 - t0; s0 += 4 * U) {
        float4 v4[U][DL];
        #pragma unroll
        for (int u = 0; u < U; ++u)
            #pragma unroll
            for (int c = 0; c < DL; ++c) v4[u][c] = ld_row4(vrs, lane_off + 256 * c, (s0 + 4 * u) * row_bytes);
        #pragma unroll
        for (int u = 0; u < U; ++u) {
            const int t = t0 + s0 + 4 * u + rq;
            #pragma unroll
            for (int g = 0; g < G; ++g) {
                const float pr = t < t1 ? L.score[g * n + t] : 0.f;
                #pragma unroll
                for (int c = 0; c < DL; ++c) {
                    acc[g][c].x = fmaf(pr, v4[u][c].x, acc[g][c].x);
                    acc[g][c].y = fmaf(pr, v4[u][c].y, acc[g][c].y);
                    acc[g][c].z = fmaf(pr, v4[u][c].z, acc[g][c].z);
                    acc[g][c].w = fmaf(pr, v4[u][c].w, acc[g][c].w);
                }
            }
        }
    }
    // The four row groups of the wave meet in lanes 0..15.
    #pragma unroll
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int c = 0; c < DL; ++c) {
            float4 &a = acc[g][c];
            a.x += __shfl_xor(a.x, 16);
            a.y += __shfl_xor(a.y, 16);
            a.z += __shfl_xor(a.z, 16);
            a.w += __shfl_xor(a.w, 16);
            a.x += __shfl_xor(a.x, 32);
            a.y += __shfl_xor(a.y, 32);
            a.z += __shfl_xor(a.z, 32);
            a.w += __shfl_xor(a.w, 32);
            if (rq == 0 && act) *reinterpret_cast<float4 *>(L.part + (wave * G + g) * head_dim + 64 * c + 4 * sub) = a;
        }
    __syncthreads();
    for (int i = tid; i < G * head_dim; i += kAttnThreads) {
        const int g = i / head_dim;
        float s = 0.f;
        for (int w = 0; w < kAttnWaves; ++w) s += L.part[w * G * head_dim + i];
        out[i] = s / den[g];
    }
}

template <int G, int DL>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float *q, const float *key_cache,
                                                                 const float *value_cache, float *out, int layer,
                                                                 int pos, int context, int kv_heads, int head_dim) {
    extern __shared__ float smem[];
    const int kvh = blockIdx.x;
    const int kv_dim = kv_heads * head_dim;
    const int64_t base = static_cast<int64_t>(layer) * context * kv_dim + kvh * head_dim;
    attend_kv_head<G, DL>(q + kvh * G * head_dim, key_cache + base, value_cache + base, out + kvh * G * head_dim, pos,
                          head_dim, kv_dim, smem);
}

// Decode-step form: RoPE of the G query rows and of key head kvh at pos,
// the key / value write into the caches at pos (rope_cache_cuda,
// inferencer.cu:930-951), then attend_kv_head.  The rotated query rows live
// in LDS after the attention's own buffers.  The cache row of pos is written
// by this workgroup only (heads occupy disjoint 256-byte runs of a row) and
// read back after a barrier.
template <int G, int DL>
__global__ __launch_bounds__(kAttnThreads) void rope_attention_kernel(
    const float *q, const float *k, const float *v, const float *cosine, const float *sine, float *key_cache,
    float *value_cache, float *out, int layer, int pos, int context, int kv_heads, int head_dim) {
    extern __shared__ float smem[];
    const int kvh = blockIdx.x, tid = threadIdx.x;
    const int kv_dim = kv_heads * head_dim, half = head_dim / 2;
    const int64_t base = static_cast<int64_t>(layer) * context * kv_dim + kvh * head_dim;
    float *qrot = smem + attention_lds_bytes(pos, head_dim, G) / sizeof(float);
    const float *cs = cosine + static_cast<int64_t>(pos) * half;
    const float *sn = sine + static_cast<int64_t>(pos) * half;
    for (int i = tid; i < G * half; i += kAttnThreads) {
        const int f = i % half;
        const int o = kvh * G * head_dim + 2 * i;   // pair i of this KV head's query rows
        const float c = cs[f], si = sn[f];
        const float q0 = q[o], q1 = q[o + 1];
        qrot[2 * i] = q0 * c - q1 * si;
        qrot[2 * i + 1] = q0 * si + q1 * c;
    }
    for (int f = tid; f < half; f += kAttnThreads) {
        const float c = cs[f], si = sn[f];
        const int o = kvh * head_dim + 2 * f;
        const int64_t row = base + static_cast<int64_t>(pos) * kv_dim + 2 * f;
        const float k0 = k[o], k1 = k[o + 1];
        key_cache[row] = k0 * c - k1 * si;
        key_cache[row + 1] = k0 * si + k1 * c;
        value_cache[row] = v[o];
        value_cache[row + 1] = v[o + 1];
    }
    __syncthreads();   // workgroup-scope release / acquire: this workgroup reads the row back
    attend_kv_head<G, DL>(qrot, key_cache + base, value_cache + base, out + kvh * G * head_dim, pos, head_dim, kv_dim,
                          smem);
}

// ------------------------------------------------ chunked decode attention --
//
// The decode driver's attention: RoPE + KV write + GQA attention with the
// positions split into chunks of kChunkPos, one 256-thread workgroup per
// (KV head, chunk), so a step at a few hundred positions spreads over tens
// of CUs instead of one per KV head.  Each workgroup rotates the G query
// rows itself; the workgroup of the last chunk (the one holding pos) also
// rotates the new key and writes key / value row pos of the caches, which
// only it reads.  A chunk leaves (max, sum of exp, unnormalised output) per
// head in the workspace; the last workgroup of a KV head to finish (an
// atomic ticket per head, reset by that workgroup) merges the chunks in
// chunk order -- the online-softmax merge of attention_cuda's running max
// (inferencer.cu:991-1007) done across chunks.
constexpr int kChunkPos = 64;
constexpr int kChunkThreads = 256;

template <int G, int DL>
__global__ __launch_bounds__(kChunkThreads) void rope_attention_chunked_kernel(
    const float *q, const float *k, const float *v, const float *cosine, const float *sine, float *key_cache,
    float *value_cache, float *out, float *partials, int *tickets, int layer, int pos, int context, int kv_heads,
    int head_dim) {
    // head_dim == 64 * DL (checked on the host).
    __shared__ float qs[G * 64 * DL];
    __shared__ float score[G][kChunkPos];
    __shared__ float part[4][G * 64 * DL];
    __shared__ float red[4][G];
    __shared__ int last;
    const int kvh = blockIdx.x, chunk = blockIdx.y, nchunks = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kv_dim = kv_heads * head_dim, half = head_dim / 2;
    const int n = pos + 1;
    const int c0 = chunk * kChunkPos, c1 = min(n, c0 + kChunkPos);
    const int64_t base = static_cast<int64_t>(layer) * context * kv_dim + kvh * head_dim;
    const float *kc = key_cache + base, *vc = value_cache + base;
    const float *cs = cosine + static_cast<int64_t>(pos) * half;
    const float *sn = sine + static_cast<int64_t>(pos) * half;

    for (int i = tid; i < G * half; i += kChunkThreads) {
        const int f = i % half;
        const int o = kvh * G * head_dim + 2 * i;
        const float c = cs[f], si = sn[f];
        const float q0 = q[o], q1 = q[o + 1];
        qs[2 * i] = q0 * c - q1 * si;
        qs[2 * i + 1] = q0 * si + q1 * c;
    }
    if (chunk == nchunks - 1) {
        for (int f = tid; f < half; f += kChunkThreads) {
            const float c = cs[f], si = sn[f];
            const int o = kvh * head_dim + 2 * f;
            const int64_t row = base + static_cast<int64_t>(pos) * kv_dim + 2 * f;
            const float k0 = k[o], k1 = k[o + 1];
            key_cache[row] = k0 * c - k1 * si;
            key_cache[row + 1] = k0 * si + k1 * c;
            value_cache[row] = v[o];
            value_cache[row + 1] = v[o + 1];
        }
    }
    __syncthreads();   // workgroup-scope release / acquire: this workgroup reads the row back

    // 1. Scores: four lanes per position, each a quarter of head_dim.
    const float inv = 1.0f / sqrtf(static_cast<float>(head_dim));
    const int quarter = head_dim / 4;          // 16 * DL columns
    const int pl = wave * 16 + (lane >> 2);    // position within the chunk
    const int qd = lane & 3;
    const int t = c0 + pl;
    float dot[G];
    #pragma unroll
    for (int g = 0; g < G; ++g) dot[g] = 0.f;
    if (t < c1) {
        const float4 *kr = reinterpret_cast<const float4 *>(kc + static_cast<int64_t>(t) * kv_dim + qd * quarter);
        float4 k4[4 * DL];
        #pragma unroll
        for (int j = 0; j < 4 * DL; ++j) k4[j] = kr[j];
        #pragma unroll
        for (int g = 0; g < G; ++g) {
            const float *qg = qs + g * head_dim + qd * quarter;
            float a = 0.f;
            #pragma unroll
            for (int j = 0; j < 4 * DL; ++j) {
                a = fmaf(qg[4 * j], k4[j].x, a);
                a = fmaf(qg[4 * j + 1], k4[j].y, a);
                a = fmaf(qg[4 * j + 2], k4[j].z, a);
                a = fmaf(qg[4 * j + 3], k4[j].w, a);
            }
            dot[g] = a;
        }
    }
    #pragma unroll
    for (int g = 0; g < G; ++g) {
        dot[g] += __shfl_xor(dot[g], 1);
        dot[g] += __shfl_xor(dot[g], 2);
    }
    float m[G];
    #pragma unroll
    for (int g = 0; g < G; ++g) {
        const float sc = dot[g] * inv;
        if (qd == 0) score[g][pl] = t < c1 ? sc : -INFINITY;
        m[g] = t < c1 ? sc : -INFINITY;
        m[g] = wave_max(m[g]);
        if (lane == 0) red[wave][g] = m[g];
    }
    __syncthreads();
    #pragma unroll
    for (int g = 0; g < G; ++g) m[g] = fmaxf(fmaxf(red[0][g], red[1][g]), fmaxf(red[2][g], red[3][g]));
    __syncthreads();

    // 2. exp and the chunk's sum per head.
    float l[G];
    #pragma unroll
    for (int g = 0; g < G; ++g) {
        float e = 0.f;
        if (tid < kChunkPos) {
            e = c0 + tid < c1 ? expf(score[g][tid] - m[g]) : 0.f;
            score[g][tid] = e;
        }
        l[g] = wave_sum(e);   // wave 0 holds every position
    }
    __syncthreads();

    // 3. Values: wave w takes positions w*16 .. +15 of the chunk, lane = dimension.
    float acc[G][DL];
    #pragma unroll
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int j = 0; j < DL; ++j) acc[g][j] = 0.f;
    {
        float vv[16][DL];
        #pragma unroll
        for (int u = 0; u < 16; ++u)
            #pragma unroll
            for (int j = 0; j < DL; ++j) {
                const int tt = c0 + wave * 16 + u, d = lane + 64 * j;
                vv[u][j] = (tt < c1 && d < head_dim) ? vc[static_cast<int64_t>(tt) * kv_dim + d] : 0.f;
            }
        #pragma unroll
        for (int g = 0; g < G; ++g)
            #pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float pr = score[g][wave * 16 + u];
                #pragma unroll
                for (int j = 0; j < DL; ++j) acc[g][j] = fmaf(pr, vv[u][j], acc[g][j]);
            }
    }
    #pragma unroll
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int j = 0; j < DL; ++j) {
            const int d = lane + 64 * j;
            if (d < head_dim) part[wave][g * head_dim + d] = acc[g][j];
        }
    __syncthreads();

    // The chunk's partial: [G] max, [G] sum, [G][head_dim] output.
    const int stride = G * (head_dim + 2);
    float *mine = partials + (static_cast<size_t>(kvh) * nchunks + chunk) * stride;
    #pragma unroll
    for (int g = 0; g < G; ++g)
        if (tid == g) {
            mine[g] = m[g];
            mine[G + g] = l[g];
        }
    for (int i = tid; i < G * head_dim; i += kChunkThreads)
        mine[2 * G + i] = (part[0][i] + part[1][i]) + (part[2][i] + part[3][i]);
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(tickets + kvh, 1) == nchunks - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    const float *all = partials + static_cast<size_t>(kvh) * nchunks * stride;
    for (int i = tid; i < G * head_dim; i += kChunkThreads) {
        const int g = i / head_dim;
        float mx = -INFINITY;
        for (int c = 0; c < nchunks; ++c) mx = fmaxf(mx, all[c * stride + g]);
        float num = 0.f, den = 0.f;
        for (int c = 0; c < nchunks; ++c) {
            const float w = expf(all[c * stride + g] - mx);
            den = fmaf(w, all[c * stride + G + g], den);
            num = fmaf(w, all[c * stride + 2 * G + i], num);
        }
        out[kvh * G * head_dim + i] = num / den;
    }
    if (tid == 0) atomicExch(tickets + kvh, 0);
}

// ------------------------------------------------- ragged decode batches --
//
// Token t of a batch attends to its own sequence: rows kv_row .. kv_row + pos
// of layer `layer` in caches laid out [layer][cache_rows][kv_dim] (each
// sequence owns a contiguous run of rows).  The reference's batched kernels
// (rope_cache_batch_cuda, attention_batch_cuda, inferencer.cu:953-1041) serve
// one sequence at contiguous positions; the descriptor generalises them to
// a ragged batch.  A token whose descriptor falls outside the cache is not
// written and its attention output is NaN.

__device__ __forceinline__ bool token_ok(const qk_batch_token &d, int64_t cache_rows, int max_pos) {
    return d.pos >= 0 && d.pos <= max_pos && d.kv_row >= 0 && d.kv_row + d.pos < cache_rows;
}

__global__ void rope_kv_batched_kernel(float *q, const float *k, const float *v, const float *cosine,
                                       const float *sine, float *key_cache, float *value_cache, int layer,
                                       int64_t cache_rows, const qk_batch_token *desc, int context, int q_pairs,
                                       int kv_pairs, int half_head) {
    const int t = blockIdx.y;
    const int pair = blockIdx.x * blockDim.x + threadIdx.x;
    if (pair >= q_pairs) return;
    const qk_batch_token d = desc[t];
    if (!token_ok(d, cache_rows, context - 1)) return;
    const int f = pair % half_head;
    const float c = cosine[static_cast<int64_t>(d.pos) * half_head + f];
    const float s = sine[static_cast<int64_t>(d.pos) * half_head + f];
    const int i = pair * 2;
    float *qt = q + static_cast<int64_t>(t) * q_pairs * 2;
    const float q0 = qt[i], q1 = qt[i + 1];
    qt[i] = q0 * c - q1 * s;
    qt[i + 1] = q0 * s + q1 * c;
    if (pair < kv_pairs) {
        const int kv_dim = kv_pairs * 2;
        const float *kt = k + static_cast<int64_t>(t) * kv_dim, *vt = v + static_cast<int64_t>(t) * kv_dim;
        const int64_t o = (static_cast<int64_t>(layer) * cache_rows + d.kv_row + d.pos) * kv_dim + i;
        const float k0 = kt[i], k1 = kt[i + 1];
        key_cache[o] = k0 * c - k1 * s;
        key_cache[o + 1] = k0 * s + k1 * c;
        value_cache[o] = vt[i];
        value_cache[o + 1] = vt[i + 1];
    }
}

template <int G, int DL>
__global__ __launch_bounds__(kAttnThreads) void attention_batched_kernel(const float *q, const float *key_cache,
                                                                         const float *value_cache, float *out,
                                                                         int layer, int64_t cache_rows,
                                                                         const qk_batch_token *desc, int max_pos,
                                                                         int kv_heads, int head_dim) {
    extern __shared__ float smem[];
    const int kvh = blockIdx.x, t = blockIdx.y;
    const int kv_dim = kv_heads * head_dim, heads = kv_heads * G;
    const qk_batch_token d = desc[t];
    float *o = out + static_cast<int64_t>(t) * heads * head_dim + kvh * G * head_dim;
    if (!token_ok(d, cache_rows, max_pos)) {
        for (int i = threadIdx.x; i < G * head_dim; i += kAttnThreads) o[i] = __builtin_nanf("");
        return;
    }
    const int64_t base = (static_cast<int64_t>(layer) * cache_rows + d.kv_row) * kv_dim + kvh * head_dim;
    attend_kv_head<G, DL>(q + static_cast<int64_t>(t) * heads * head_dim + kvh * G * head_dim, key_cache + base,
                          value_cache + base, o, d.pos, head_dim, kv_dim, smem);
}

// Decode-driver form for ragged batches: RoPE of token t's G query rows and
// of its key head kvh at its own position, the key / value write into row
// kv_row + pos (written and read back by this workgroup only, ordered by
// the barrier), then attend_kv_head over the token's own rows.
template <int G, int DL>
__global__ __launch_bounds__(kAttnThreads) void rope_attention_batched_kernel(
    const float *q, const float *k, const float *v, const float *cosine, const float *sine, float *key_cache,
    float *value_cache, float *out, int layer, int64_t cache_rows, const qk_batch_token *desc, int max_pos,
    int kv_heads, int head_dim) {
    extern __shared__ float smem[];
    const int kvh = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int kv_dim = kv_heads * head_dim, heads = kv_heads * G, half = head_dim / 2;
    const qk_batch_token d = desc[t];
    float *o = out + static_cast<int64_t>(t) * heads * head_dim + kvh * G * head_dim;
    if (!token_ok(d, cache_rows, max_pos)) {
        for (int i = tid; i < G * head_dim; i += kAttnThreads) o[i] = __builtin_nanf("");
        return;
    }
    const int64_t base = (static_cast<int64_t>(layer) * cache_rows + d.kv_row) * kv_dim + kvh * head_dim;
    float *qrot = smem + attention_lds_bytes(max_pos, head_dim, G) / sizeof(float);
    const float *cs = cosine + static_cast<int64_t>(d.pos) * half;
    const float *sn = sine + static_cast<int64_t>(d.pos) * half;
    const float *qt = q + static_cast<int64_t>(t) * heads * head_dim + kvh * G * head_dim;
    for (int i = tid; i < G * half; i += kAttnThreads) {
        const int f = i % half;
        const float c = cs[f], si = sn[f];
        const float q0 = qt[2 * i], q1 = qt[2 * i + 1];
        qrot[2 * i] = q0 * c - q1 * si;
        qrot[2 * i + 1] = q0 * si + q1 * c;
    }
    const float *kt = k + static_cast<int64_t>(t) * kv_dim + kvh * head_dim;
    const float *vt = v + static_cast<int64_t>(t) * kv_dim + kvh * head_dim;
    for (int f = tid; f < half; f += kAttnThreads) {
        const float c = cs[f], si = sn[f];
        const int64_t row = base + static_cast<int64_t>(d.pos) * kv_dim + 2 * f;
        const float k0 = kt[2 * f], k1 = kt[2 * f + 1];
        key_cache[row] = k0 * c - k1 * si;
        key_cache[row + 1] = k0 * si + k1 * c;
        value_cache[row] = vt[2 * f];
        value_cache[row + 1] = vt[2 * f + 1];
    }
    __syncthreads();   // workgroup-scope release / acquire: this workgroup reads the row back
    attend_kv_head<G, DL>(qrot, key_cache + base, value_cache + base, o, d.pos, head_dim, kv_dim, smem);
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

// Row blockIdx.y of v (stride ldv) -> partials pv / pi + row * gridDim.x.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *v, int n, int64_t ldv, float *pv, int *pi) {
    v += static_cast<int64_t>(blockIdx.y) * ldv;
    pv += static_cast<int64_t>(blockIdx.y) * gridDim.x;
    pi += static_cast<int64_t>(blockIdx.y) * gridDim.x;
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

// One block per row: the row's parts partials -> out[row].
__global__ __launch_bounds__(256) void argmax_final_kernel(const float *pv, const int *pi, int parts, int32_t *out) {
    pv += static_cast<int64_t>(blockIdx.x) * parts;
    pi += static_cast<int64_t>(blockIdx.x) * parts;
    out += blockIdx.x;
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

// Kernel instance for G query heads per KV head and head_dim: G in
// {1, 2, 3, 4, 6, 8}, head_dim <= 256.  NULL when unsupported.
template <template <int, int> class K>
const void *attention_instance(int G, int head_dim) {
    const int dl = (head_dim + 63) / 64;
#define QK_ATTN_CASE(g)                                        \
    case g:                                                    \
        return dl == 1   ? K<g, 1>::fn()                       \
               : dl == 2 ? K<g, 2>::fn()                       \
               : dl <= 4 ? K<g, 4>::fn()                       \
                         : nullptr;
    switch (G) {
        QK_ATTN_CASE(1)
        QK_ATTN_CASE(2)
        QK_ATTN_CASE(3)
        QK_ATTN_CASE(4)
        QK_ATTN_CASE(6)
        QK_ATTN_CASE(8)
        default: return nullptr;
    }
#undef QK_ATTN_CASE
}

template <int G, int DL>
struct PlainAttention {
    static const void *fn() { return reinterpret_cast<const void *>(attention_kernel<G, DL>); }
};
template <int G, int DL>
struct BatchedAttention {
    static const void *fn() { return reinterpret_cast<const void *>(attention_batched_kernel<G, DL>); }
};
template <int G, int DL>
struct RopeBatchedAttention {
    static const void *fn() { return reinterpret_cast<const void *>(rope_attention_batched_kernel<G, DL>); }
};
template <int G, int DL>
struct ChunkedAttention {
    static const void *fn() { return reinterpret_cast<const void *>(rope_attention_chunked_kernel<G, DL>); }
};
template <int G, int DL>
struct RopeAttention {
    static const void *fn() { return reinterpret_cast<const void *>(rope_attention_kernel<G, DL>); }
};

inline hipStream_t S(qk_stream s) { return static_cast<hipStream_t>(s); }

}  // namespace

size_t attention_workspace_bytes(int kv_heads, int group, int head_dim, int context) {
    const size_t chunks = (static_cast<size_t>(context) + kChunkPos - 1) / kChunkPos;
    return (static_cast<size_t>(kv_heads) * chunks * group * (head_dim + 2)) * sizeof(float) +
           static_cast<size_t>(kv_heads) * sizeof(int) + 256;
}

int launch_rope_attention_chunked(const float *q, const float *k, const float *v, const float *cosine,
                                  const float *sine, float *key_cache, float *value_cache, float *out, void *workspace,
                                  int layer, int pos, int context, int heads, int kv_heads, int head_dim,
                                  hipStream_t stream) {
    const int G = heads / kv_heads;
    const void *fn = head_dim % 64 == 0 && kv_heads <= 64 ? attention_instance<ChunkedAttention>(G, head_dim) : nullptr;
    if (!fn) return fail(QK_ERR_LIMIT, "chunked attention: unsupported head layout");
    const int nchunks = (pos + kChunkPos) / kChunkPos;
    int *tickets = static_cast<int *>(workspace);
    float *partials = reinterpret_cast<float *>(static_cast<uint8_t *>(workspace) + 256);
    void *args[] = {&q, &k, &v, &cosine, &sine, &key_cache, &value_cache, &out, &partials, &tickets, &layer, &pos,
                    &context, &kv_heads, &head_dim};
    if (hipLaunchKernel(fn, dim3(kv_heads, nchunks), dim3(kChunkThreads), args, 0, stream) != hipSuccess)
        return launch_status("chunked attention launch");
    return launch_status("chunked attention launch");
}

int launch_rope_attention_batched(const float *q, const float *k, const float *v, const float *cosine,
                                  const float *sine, float *key_cache, float *value_cache, float *out, int layer,
                                  int64_t cache_rows, const qk_batch_token *desc, int n_tokens, int max_pos,
                                  int heads, int kv_heads, int head_dim, hipStream_t stream) {
    const int G = heads / kv_heads;
    const void *fn = attention_instance<RopeBatchedAttention>(G, head_dim);
    if (!fn) return fail(QK_ERR_LIMIT, "batched rope + attention: unsupported head layout");
    if (n_tokens > 65535) return fail(QK_ERR_LIMIT, "batched rope + attention: too many tokens in one launch");
    const size_t lds = attention_lds_bytes(max_pos, head_dim, G) + static_cast<size_t>(G) * head_dim * sizeof(float);
    void *args[] = {&q, &k, &v, &cosine, &sine, &key_cache, &value_cache, &out, &layer, &cache_rows, &desc, &max_pos,
                    &kv_heads, &head_dim};
    if (hipLaunchKernel(fn, dim3(kv_heads, n_tokens), dim3(kAttnThreads), args, lds, stream) != hipSuccess)
        return launch_status("batched rope + attention launch");
    return launch_status("batched rope + attention launch");
}

bool chunked_attention_supported(int kv_heads, int group, int head_dim) {
    return head_dim % 64 == 0 && head_dim <= 256 && kv_heads <= 64 &&
           attention_instance<ChunkedAttention>(group, head_dim) != nullptr;
}

bool attention_supported(int group, int head_dim) {
    return head_dim >= 4 && head_dim % 4 == 0 && 256 % head_dim == 0 &&
           attention_instance<PlainAttention>(group, head_dim) != nullptr;
}

int launch_rope_attention(const float *q, const float *k, const float *v, const float *cosine, const float *sine,
                          float *key_cache, float *value_cache, float *out, int layer, int pos, int context,
                          int heads, int kv_heads, int head_dim, hipStream_t stream) {
    const int G = heads / kv_heads;
    const void *fn = attention_instance<RopeAttention>(G, head_dim);
    if (!fn) return fail(QK_ERR_LIMIT, "rope + attention: unsupported query heads per KV head or head_dim");
    const size_t lds = attention_lds_bytes(pos, head_dim, G) + static_cast<size_t>(G) * head_dim * sizeof(float);
    void *args[] = {&q, &k, &v, &cosine, &sine, &key_cache, &value_cache, &out, &layer, &pos, &context, &kv_heads,
                    &head_dim};
    if (hipLaunchKernel(fn, dim3(kv_heads), dim3(kAttnThreads), args, lds, stream) != hipSuccess)
        return launch_status("rope + attention launch");
    return launch_status("rope + attention launch");
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
    const void *fn = qk::attention_instance<qk::PlainAttention>(heads / kv_heads, head_dim);
    if (!fn) return qk::fail(QK_ERR_LIMIT, "qk_attention_f32: query heads per KV head must be 1, 2, 3, 4, 6 or 8");
    if (!qk::aligned(key_cache, 16) || !qk::aligned(value_cache, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_attention_f32: caches must be 16-byte aligned");
    const size_t lds = qk::attention_lds_bytes(pos, head_dim, heads / kv_heads);
    if (lds > 150 * 1024) return qk::fail(QK_ERR_LIMIT, "qk_attention_f32: position beyond the LDS score buffer");
    void *args[] = {&q, &key_cache, &value_cache, &out, &layer, &pos, &context, &kv_heads, &head_dim};
    if (hipLaunchKernel(fn, dim3(kv_heads), dim3(qk::kAttnThreads), args, lds, qk::S(stream)) != hipSuccess)
        return qk::launch_status("qk_attention_f32 launch");
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

int qk_rope_kv_write_batched(float *q, const float *k, const float *v, const float *cosine, const float *sine,
                             float *key_cache, float *value_cache, int layer, int64_t cache_rows,
                             const qk_batch_token *desc, int n_tokens, int context, int heads, int kv_heads,
                             int head_dim, qk_stream stream) {
    if (!q || !k || !v || !cosine || !sine || !key_cache || !value_cache || (!desc && n_tokens > 0) || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rope_kv_write_batched: null pointer or negative count");
    if (head_dim < 2 || head_dim % 2 || heads < 1 || kv_heads < 1 || heads % kv_heads || layer < 0 ||
        cache_rows < 1 || context < 1)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rope_kv_write_batched: bad head layout or cache shape");
    if (n_tokens == 0) return qk::ok();
    if (n_tokens > 65535) return qk::fail(QK_ERR_LIMIT, "qk_rope_kv_write_batched: too many tokens in one launch");
    const int q_pairs = heads * head_dim / 2, kv_pairs = kv_heads * head_dim / 2;
    hipLaunchKernelGGL(qk::rope_kv_batched_kernel, dim3((q_pairs + 255) / 256, n_tokens), dim3(256), 0, qk::S(stream),
                       q, k, v, cosine, sine, key_cache, value_cache, layer, cache_rows, desc, context, q_pairs,
                       kv_pairs, head_dim / 2);
    return qk::launch_status("qk_rope_kv_write_batched launch");
}

int qk_attention_batched_f32(const float *q, const float *key_cache, const float *value_cache, float *out, int layer,
                             int64_t cache_rows, const qk_batch_token *desc, int n_tokens, int max_pos, int heads,
                             int kv_heads, int head_dim, qk_stream stream) {
    if (!q || !key_cache || !value_cache || !out || (!desc && n_tokens > 0) || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_attention_batched_f32: null pointer or negative count");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || layer < 0 || cache_rows < 1 || max_pos < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_attention_batched_f32: bad head layout or cache shape");
    if (head_dim < 4 || head_dim % 4 || 256 % head_dim)
        return qk::fail(QK_ERR_LIMIT, "qk_attention_batched_f32: head_dim must be a multiple of 4 dividing 256");
    const void *fn = qk::attention_instance<qk::BatchedAttention>(heads / kv_heads, head_dim);
    if (!fn)
        return qk::fail(QK_ERR_LIMIT, "qk_attention_batched_f32: query heads per KV head must be 1, 2, 3, 4, 6 or 8");
    if (!qk::aligned(key_cache, 16) || !qk::aligned(value_cache, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_attention_batched_f32: caches must be 16-byte aligned");
    const size_t lds = qk::attention_lds_bytes(max_pos, head_dim, heads / kv_heads);
    if (lds > 150 * 1024) return qk::fail(QK_ERR_LIMIT, "qk_attention_batched_f32: max_pos beyond the LDS score buffer");
    if (n_tokens == 0) return qk::ok();
    if (n_tokens > 65535) return qk::fail(QK_ERR_LIMIT, "qk_attention_batched_f32: too many tokens in one launch");
    void *args[] = {&q, &key_cache, &value_cache, &out, &layer, &cache_rows, &desc, &max_pos, &kv_heads, &head_dim};
    if (hipLaunchKernel(fn, dim3(kv_heads, n_tokens), dim3(qk::kAttnThreads), args, lds, qk::S(stream)) != hipSuccess)
        return qk::launch_status("qk_attention_batched_f32 launch");
    return qk::launch_status("qk_attention_batched_f32 launch");
}

size_t qk_argmax_workspace_bytes(int n) {
    if (n < 1) return 0;
    const size_t parts = (static_cast<size_t>(n) + qk::kArgmaxBlock - 1) / qk::kArgmaxBlock;
    return parts * (sizeof(float) + sizeof(int));
}

size_t qk_argmax_rows_workspace_bytes(int n, int rows) {
    if (rows < 1) return 0;
    return qk_argmax_workspace_bytes(n) * static_cast<size_t>(rows);
}

int qk_argmax_rows_f32(const float *v, int n, int64_t ldv, int rows, int32_t *out, void *workspace,
                       qk_stream stream) {
    if (!v || !out || !workspace || n < 1 || rows < 0 || ldv < n)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_argmax_rows_f32: null pointer, empty row or bad stride");
    if (!qk::aligned(workspace, 4)) return qk::fail(QK_ERR_ALIGN, "qk_argmax_rows_f32: workspace must be 4-byte aligned");
    if (rows == 0) return qk::ok();
    if (rows > 65535) return qk::fail(QK_ERR_LIMIT, "qk_argmax_rows_f32: too many rows in one launch");
    const int parts = (n + qk::kArgmaxBlock - 1) / qk::kArgmaxBlock;
    float *pv = static_cast<float *>(workspace);
    int *pi = reinterpret_cast<int *>(pv + static_cast<size_t>(parts) * rows);
    hipLaunchKernelGGL(qk::argmax_partial_kernel, dim3(parts, rows), dim3(256), 0, qk::S(stream), v, n, ldv, pv, pi);
    hipLaunchKernelGGL(qk::argmax_final_kernel, dim3(rows), dim3(256), 0, qk::S(stream), pv, pi, parts, out);
    return qk::launch_status("qk_argmax_rows_f32 launch");
}

int qk_argmax_f32(const float *v, int n, int32_t *out, void *workspace, qk_stream stream) {
    if (!v || !out || !workspace || n < 1)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_argmax_f32: null pointer or empty input");
    if (!qk::aligned(workspace, 4)) return qk::fail(QK_ERR_ALIGN, "qk_argmax_f32: workspace must be 4-byte aligned");
    const int parts = (n + qk::kArgmaxBlock - 1) / qk::kArgmaxBlock;
    float *pv = static_cast<float *>(workspace);
    int *pi = reinterpret_cast<int *>(pv + parts);
    hipLaunchKernelGGL(qk::argmax_partial_kernel, dim3(parts), dim3(256), 0, qk::S(stream), v, n, int64_t(n), pv, pi);
    hipLaunchKernelGGL(qk::argmax_final_kernel, dim3(1), dim3(256), 0, qk::S(stream), pv, pi, parts, out);
    return qk::launch_status("qk_argmax_f32 launch");
}

}  // extern "C"
