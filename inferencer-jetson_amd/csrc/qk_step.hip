// qk_step.hip - the decode step's small kernels around the GEMVs.
//
// Replace rmsnorm_cuda, rope_cuda / cache_cuda / rope_cache_cuda,
// attention_cuda, add_cuda, silu_cuda and the two-stage argmax
// (inferencer.cu:821-834, 906-1009, 1043-1099), generalised from the
// reference's hard-coded head_dim 128 / 64 RoPE frequencies to any even
// head_dim, and written for wave64.
#include "qk_internal.h"
#include "qk_records.h"

#include <algorithm>
#include <cmath>

namespace qk {

namespace {

__device__ __forceinline__ float wave_max(float v) {
    #pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
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

// rmsnorm_quantize_cuda / rmsnorm_quantize_batch_cuda (inferencer.cu:839-889):
// one 256-thread block per token normalises the row exactly as rmsnorm_kernel's
// float4 path (same sum-of-squares order, same scale) and quantizes it in the
// same pass: a 32-value group is eight float4 of eight adjacent lanes, whose
// amax meets in three xor shuffles; scale and rounding are those of
// quantize_x32_kernel, so xq / xscale equal the two-launch result bit for bit.
// The reference reduces the row once per 32-value block; here once per token.
__global__ __launch_bounds__(256) void rmsnorm_quantize_kernel(const float *x, int ldx, const float *weight,
                                                               float *out, int ldout, int8_t *xq, int ldxq,
                                                               float *xscale, int ldscale, int n, float eps) {
    __shared__ float scratch[4];
    const int64_t token = blockIdx.x;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + token * ldx);
    const float4 *w4 = reinterpret_cast<const float4 *>(weight);
    const int n4 = n >> 2;
    float ss = 0.f;
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
    float4 *o4 = out ? reinterpret_cast<float4 *>(out + token * ldout) : nullptr;
    uint32_t *q4 = reinterpret_cast<uint32_t *>(xq + token * ldxq);
    float *st = xscale + token * ldscale;
    // n4 is a multiple of 8, so the eight lanes of a group are all in range
    // together and the shuffles never mix groups.
    for (int i = threadIdx.x; i < n4; i += 256) {
        const float4 v = x4[i], w = w4[i];
        const float4 o = make_float4(v.x * scale * w.x, v.y * scale * w.y, v.z * scale * w.z, v.w * scale * w.w);
        if (o4) o4[i] = o;
        float amax = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
        amax = fmaxf(amax, __shfl_xor(amax, 1));
        amax = fmaxf(amax, __shfl_xor(amax, 2));
        amax = fmaxf(amax, __shfl_xor(amax, 4));
        const float gs = amax > 0.f ? amax / 127.f : 1.f;
        if ((i & 7) == 0) st[i >> 3] = gs;
        auto q8 = [gs](float val) {
            int q = static_cast<int>(rintf(val / gs));
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            return static_cast<uint32_t>(q) & 0xFFu;
        };
        q4[i] = q8(o.x) | (q8(o.y) << 8) | (q8(o.z) << 16) | (q8(o.w) << 24);
    }
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
__device__ __forceinline__ float4 ld_row4(__amdgpu_buffer_rsrc_t r, int lane_off, int row_off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, row_off, 0));
}

__device__ __forceinline__ float dot4(const float4 &a, const float4 &b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    return fmaf(a.w, b.w, acc);
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

// Written without kv_row + pos, which a huge kv_row would overflow.
__device__ __forceinline__ bool token_ok(const qk_batch_token &d, int64_t cache_rows, int max_pos) {
    return d.pos >= 0 && d.pos <= max_pos && d.kv_row >= 0 && d.kv_row < cache_rows - d.pos;
}

__global__ void rope_kv_batched_kernel(float *q, const float *k, const float *v, const float *cosine,
                                       const float *sine, float *key_cache, float *value_cache, int layer,
                                       int64_t cache_rows, const qk_batch_token *desc, int context, int q_pairs,
                                       int kv_pairs, int half_head, int head_major) {
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
        const int hd = 2 * half_head;
        const int64_t o = kv_offset(head_major, layer, cache_rows, kv_dim / hd, hd, d.kv_row + d.pos, i / hd) + i % hd;
        const float k0 = kt[i], k1 = kt[i + 1];
        key_cache[o] = k0 * c - k1 * s;
        key_cache[o + 1] = k0 * s + k1 * c;
        value_cache[o] = vt[i];
        value_cache[o + 1] = vt[i + 1];
    }
}

// ------------------------------------------------- split-row attention --
//
// One 256-thread workgroup per (KV head, token, split of split_rows rows).
// A CU on its own reads a few tens of GB/s, so a token's rows are spread
// over many CUs.  L lanes share a cache row (8, or 16 when G * head_dim >
// 512 to bound the registers), lane `sub` holding dimensions 4L*j + 4*sub
// .. +3 for j < NF, so one load instruction of a wave covers 64 / L rows.
// Every K / V load of the first round is issued before the query rows are
// read (the cache latency overlaps the RoPE); later rounds are issued while
// the previous one is consumed.  Lane group rq keeps its own running (max,
// sum of exp, unnormalised output) over the rows it sees -- the online
// softmax of attention_cuda (inferencer.cu:991-1007), in base-2 units -- and
// the groups and the waves meet by the same merge.  A token with one split
// writes its output directly; otherwise each split leaves a partial and a
// second kernel merges them in split order.  (A merge by the last workgroup
// to finish needs a device-scope release per workgroup, an L2 write-back
// that costs about a microsecond each and serialises per XCD.)
constexpr int kSplitThreads = 256;
constexpr int kMaxSplits = 64;        // splits per token at most
constexpr int kMinSplitRows = 64;     // rows per split at least
constexpr int kSplitTarget = 128;     // workgroups a call aims at
constexpr size_t kMaxSplitWorkspace = size_t(64) << 20;
constexpr int kWideMaxPairs = 64;              // (token, KV head) pairs of a wide launch at most
constexpr int64_t kWideMaxBytes = 512 << 10;   // K + V bytes of one pair's rows at most

struct SplitAttnKernelArgs {
    SplitAttention a;
    float *partials;   // [n_tokens * gridDim.x][splits][split_header(G) + G * head_dim]
    int split_rows;
    int splits;        // most splits of any token (the partials' stride)
    int head_split;    // workgroups sharing a KV head, each with heads / kv_heads / head_split query heads
};

// A split partial: max [G], sum of exp [G], padded to 16 bytes, then the
// unnormalised output rows [G][head_dim].
__host__ __device__ constexpr int split_header(int G) { return (2 * G + 3) & ~3; }
static_assert(split_header(1) + 64 == split_partial_floats(64), "one-head partials: max, sum, pad, row");

// Register plan of an instance: NU steps of 64/L rows per wave per round,
// K / V buffers (8 * NU * NF VGPRs) within what the query and output rows
// (8 * G * NF) leave of about 200.
template <int G, int NF>
constexpr int split_steps() {
    constexpr int cap = NF >= 8 ? 1 : 8 / NF;
    constexpr int fit = (200 - 8 * G * NF) / (8 * NF + 4 * G);
    return fit < 1 ? 1 : fit < cap ? fit : cap;
}

__device__ __forceinline__ float4 scale4(const float4 &a, float f) {
    return make_float4(a.x * f, a.y * f, a.z * f, a.w * f);
}

__device__ __forceinline__ void fma4(float p, const float4 &v, float4 &acc) {
    acc.x = fmaf(p, v.x, acc.x);
    acc.y = fmaf(p, v.y, acc.y);
    acc.z = fmaf(p, v.z, acc.z);
    acc.w = fmaf(p, v.w, acc.w);
}

// Scores (base-2 units, -inf outside the split) of NU rows, one per lane
// group, against the G query rows.
template <int G, int NF, int L, int NU>
__device__ __forceinline__ void score_rows(const float4 (&qv)[G][NF], const float4 (&kk)[NU][NF], const bool (&ok)[NU],
                                           float scale, float (&s)[NU][G]) {
    #pragma unroll
    for (int u = 0; u < NU; ++u)
        #pragma unroll
        for (int g = 0; g < G; ++g) {
            float a = 0.f;
            #pragma unroll
            for (int j = 0; j < NF; ++j) a = dot4(qv[g][j], kk[u][j], a);
            const float sc = group_sum<L>(a) * scale;
            s[u][g] = ok[u] ? sc : -INFINITY;
        }
}

// Online-softmax update of a lane group's state with NU scored rows.
template <int G, int NF, int NU>
__device__ __forceinline__ void absorb_rows(const float (&s)[NU][G], const float4 (&vv)[NU][NF], float (&m)[G],
                                            float (&l)[G], float4 (&acc)[G][NF]) {
    #pragma unroll
    for (int g = 0; g < G; ++g) {
        float mb = s[0][g];
        #pragma unroll
        for (int u = 1; u < NU; ++u) mb = fmaxf(mb, s[u][g]);
        const float mn = fmaxf(m[g], mb);
        const float ref = mn == -INFINITY ? 0.f : mn;   // no row yet: the state stays zero
        const float f = __builtin_amdgcn_exp2f(m[g] - ref);
        l[g] *= f;
        #pragma unroll
        for (int j = 0; j < NF; ++j) acc[g][j] = scale4(acc[g][j], f);
        #pragma unroll
        for (int u = 0; u < NU; ++u) {
            const float p = __builtin_amdgcn_exp2f(s[u][g] - ref);
            l[g] += p;
            #pragma unroll
            for (int j = 0; j < NF; ++j) fma4(p, vv[u][j], acc[g][j]);
        }
        m[g] = mn;
    }
}

// Token b's attention outputs of this workgroup's heads (G * hd values at
// `of`, head g's at of + g * stride) as GEMM records, one 256-column block
// at a time by the first wave: lane (q, j) = (lane / 8, lane % 8) stages
// columns q*32 + 4j .. +3 in the record layout of stage_store (the same
// power-of-two block scale, fp16 high / low halves and sub-block sums).
template <int G>
__device__ __forceinline__ void write_gemm_records(const SplitAttention &a, int b, int kvh, const float *of,
                                                   int stride) {
    const int hd = a.head_dim, blocks = G * hd / 256;
    const int lane = threadIdx.x;
    if (lane >= 64) return;
    const int q = lane >> 3, j = lane & 7;
    const int nb = a.heads * hd / 256;
    for (int blk = 0; blk < blocks; ++blk) {
        float v[4];
        const int c0 = blk * 256 + q * 32 + 4 * j;   // column within this workgroup's heads
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + i, g = c / hd;
            v[i] = of[g * stride + (c - g * hd)];
        }
        stage_store_wave(v, lane, b % kTokTile,
                         a.gemm_rec + (static_cast<size_t>(b / kTokTile) * nb + kvh * blocks + blk) * kTileBytes);
    }
}

// Element (token b, column c) of matrix m (q 0, k 1, v 2) of the QKV
// product: from its buffer (row stride ld), or, with the product's split
// sums left unreduced, their sum in split order -- skinny_reduce's
// additions over the partial of row tile qkv_tile0[m] + c / 32 and token
// tile b / 32, at the accumulator's element for (token b % 32, row c % 32).
__device__ __forceinline__ float qkv_elem(const SplitAttention &a, const float *buf, int64_t ld, int m, int b, int c) {
    if (a.qkv_splits <= 1) return buf[b * ld + c];
    const int tl = b & 31;
    const int e = (4 * (tl >> 3) + (tl & 3)) * 64 + 32 * ((tl >> 2) & 1) + (c & 31);
    const float *src =
        a.qkv_parts + (static_cast<int64_t>(a.qkv_tile0[m] + (c >> 5)) * a.qkv_ttiles + (b >> 5)) * a.qkv_splits * 1024 + e;
    float sum = src[0];
    for (int sp = 1; sp < a.qkv_splits; ++sp) sum += src[static_cast<int64_t>(sp) * 1024];
    return sum;
}

// Merge of two (max, sum) states: the scale factors of each side.
__device__ __forceinline__ void merge_scales(float &m, float &l, float mo, float lo, float &f, float &fo) {
    const float mn = fmaxf(m, mo);
    const float ref = mn == -INFINITY ? 0.f : mn;
    f = __builtin_amdgcn_exp2f(m - ref);
    fo = __builtin_amdgcn_exp2f(mo - ref);
    l = l * f + lo * fo;
    m = mn;
}

// The nsplit partials of (token b, workgroup kvh) merged in split order,
// by 256 threads; mo: G * head_dim floats of LDS for the records.
template <int G>
__device__ void merge_splits(const SplitAttnKernelArgs &ka, int b, int kvh, int nsplit, float *mo) {
    const SplitAttention &a = ka.a;
    const int hd = a.head_dim;
    constexpr int kHdr = split_header(G);
    const int pstride = kHdr + G * hd;
    const float *all = ka.partials + (static_cast<int64_t>(b) * gridDim.x + kvh) * ka.splits * pstride;
    float *o = a.out + static_cast<int64_t>(b) * a.heads * hd + kvh * G * hd;
    for (int i = threadIdx.x; i < G * hd; i += 256) {
        const int g = i / hd;
        float mx = -INFINITY;
        #pragma unroll 8
        for (int p = 0; p < nsplit; ++p) mx = fmaxf(mx, all[p * pstride + g]);
        float num = 0.f, den = 0.f;
        #pragma unroll 8
        for (int p = 0; p < nsplit; ++p) {
            const float w = __builtin_amdgcn_exp2f(all[p * pstride + g] - mx);
            den = fmaf(w, all[p * pstride + G + g], den);
            num = fmaf(w, all[p * pstride + kHdr + i], num);
        }
        o[i] = num / den;
        if (a.rec_out || a.gemm_rec) mo[i] = num / den;
        if (a.q8_out) {
            // G * hd % 32 == 0: a half-wave holds one group, active together.
            const int64_t c = static_cast<int64_t>(b) * a.heads * hd + kvh * G * hd + i;
            quantize_group_store(num / den, true, threadIdx.x & 31, a.q8_out + c, a.q8_scale + c / 32);
        }
    }
    if (a.gemm_rec) {
        __syncthreads();
        write_gemm_records<G>(a, b, kvh, mo, hd);
    }
    if (a.rec_out) {
        __syncthreads();
        XGroup *rec = a.rec_out + (static_cast<int64_t>(b) * a.heads * hd + kvh * G * hd) / 16;
        const int groups = G * hd / 16, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        for (int g0 = wave * 4; g0 < groups; g0 += 16) {   // four waves, four groups each
            const int gi = g0 + (lane >> 4), live = gi < groups;
            record16_quads(live ? mo[16 * gi + (lane & 15)] : 0.f, lane, rec + gi, live);
        }
    }
}

template <int G, int NF, int L, int NW>
__global__ __launch_bounds__(NW * 64) void split_attention_kernel(SplitAttnKernelArgs ka) {
    constexpr int kSplitWaves = NW;
    constexpr int kSplitThreads = NW * 64;
    constexpr int NU = split_steps<G, NF>();
    constexpr int R = 64 / L;          // rows per load instruction
    constexpr int HD = 4 * NF * L;     // dimensions a lane group covers (>= head_dim)
    constexpr int kRound = NU * kSplitWaves * R;
    __shared__ float4 qs[G * HD / 4];
    __shared__ float4 knew[HD / 4], vnew[HD / 4];
    __shared__ float4 part[kSplitWaves][G * HD / 4];
    __shared__ float wm[kSplitWaves][G], wl[kSplitWaves][G];
    const SplitAttention &a = ka.a;
    // Workgroup kvh serves query heads kvh*G .. kvh*G + G - 1 of KV head
    // kvh / head_split; the first of a KV head's workgroups writes its row.
    // With head_split > 1 the workgroups sharing a KV head are numbered
    // kv_heads apart: workgroups are dealt to the XCDs round-robin, so they
    // land on one XCD (kv_heads a multiple of 8) and read the rows through
    // one L2 instead of fetching them head_split times.
    const int kvh = ka.head_split > 1 ? static_cast<int>(blockIdx.x % a.kv_heads) * ka.head_split +
                                            static_cast<int>(blockIdx.x / a.kv_heads)
                                      : static_cast<int>(blockIdx.x);
    const int b = blockIdx.y, split = blockIdx.z;
    const int cache_kvh = kvh / ka.head_split;
    const bool writer = kvh % ka.head_split == 0;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane % L, rq = lane / L;
    const int hd = a.head_dim, hv = hd / 4, kv_dim = a.kv_heads * hd, half = hd / 2;
    const qk_batch_token d = a.desc ? a.desc[b] : qk_batch_token{a.pos, 0, 0};
    float *o = a.out + static_cast<int64_t>(b) * a.heads * hd + kvh * G * hd;
    if (!token_ok(d, a.cache_rows, a.max_pos)) {
        if (split == 0)
            for (int i = tid; i < G * hd; i += kSplitThreads) o[i] = __builtin_nanf("");
        return;
    }
    const int n = d.pos + 1;
    const int r0 = split * ka.split_rows;
    if (r0 >= n) return;
    const int r1 = min(n, r0 + ka.split_rows);
    const int nsplit = (n + ka.split_rows - 1) / ka.split_rows;
    const bool fresh = a.k != nullptr && r1 == n;   // this split holds row pos and writes it
    const int rows = (fresh ? r1 - 1 : r1) - r0;    // rows read from the caches
    const int rs = a.head_major ? hd : kv_dim;   // floats from one row of the head to the next
    const int64_t head0 = kv_offset(a.head_major, a.layer, a.cache_rows, a.kv_heads, hd, d.kv_row, cache_kvh);
    const int64_t first = head0 + static_cast<int64_t>(r0) * rs;
    const int row_bytes = rs * 4;
    const bool act = sub < hv;   // head_dim < 4L leaves lanes idle
    const int lane_off = (rq * rs + 4 * min(sub, hv - 1)) * 4;
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc(a.key_cache + first, 0, rows * row_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc(a.value_cache + first, 0, rows * row_bytes, 0x00020000);

    // Step u of wave w in the round at rb covers rows rb + (u * waves + w) * R
    // + rq of the split; rows past `rows` read as zero.
    float4 kk[NU][NF], vv[NU][NF];
    #pragma unroll
    for (int u = 0; u < NU; ++u)
        #pragma unroll
        for (int j = 0; j < NF; ++j)
            kk[u][j] = ld_row4(krs, lane_off + 16 * L * j, (u * kSplitWaves + wave) * R * row_bytes);
    #pragma unroll
    for (int u = 0; u < NU; ++u)
        #pragma unroll
        for (int j = 0; j < NF; ++j)
            vv[u][j] = ld_row4(vrs, lane_off + 16 * L * j, (u * kSplitWaves + wave) * R * row_bytes);

    // Query rows (rotated here when k is given) and the fresh key / value row.
    const float *qt = a.q + static_cast<int64_t>(b) * a.heads * hd + kvh * G * hd;
    float *qsf = reinterpret_cast<float *>(qs);
    if (a.k) {
        const float *cs = a.cosine + static_cast<int64_t>(d.pos) * half;
        const float *sn = a.sine + static_cast<int64_t>(d.pos) * half;
        const int64_t q_ld = static_cast<int64_t>(a.heads) * hd;
        for (int i = tid; i < G * half; i += kSplitThreads) {
            const int g = i / half, f = i - g * half;
            const float c = cs[f], si = sn[f];
            const int qc = (kvh * G + g) * hd + 2 * f;
            const float q0 = qkv_elem(a, a.q, q_ld, 0, b, qc), q1 = qkv_elem(a, a.q, q_ld, 0, b, qc + 1);
            qsf[g * HD + 2 * f] = q0 * c - q1 * si;
            qsf[g * HD + 2 * f + 1] = q0 * si + q1 * c;
        }
        if (fresh) {
            float *kn = reinterpret_cast<float *>(knew), *vn = reinterpret_cast<float *>(vnew);
            const int64_t row = head0 + static_cast<int64_t>(d.pos) * rs;
            for (int f = tid; f < half; f += kSplitThreads) {
                const float c = cs[f], si = sn[f];
                const int kc = cache_kvh * hd + 2 * f;
                const float k0 = qkv_elem(a, a.k, kv_dim, 1, b, kc), k1 = qkv_elem(a, a.k, kv_dim, 1, b, kc + 1);
                const float kr0 = k0 * c - k1 * si, kr1 = k0 * si + k1 * c;
                const float v0 = qkv_elem(a, a.v, kv_dim, 2, b, kc), v1 = qkv_elem(a, a.v, kv_dim, 2, b, kc + 1);
                kn[2 * f] = kr0;
                kn[2 * f + 1] = kr1;
                vn[2 * f] = v0;
                vn[2 * f + 1] = v1;
                if (writer) {
                    a.key_cache[row + 2 * f] = kr0;
                    a.key_cache[row + 2 * f + 1] = kr1;
                    a.value_cache[row + 2 * f] = v0;
                    a.value_cache[row + 2 * f + 1] = v1;
                }
            }
        }
    } else {
        for (int i = tid; i < G * hd; i += kSplitThreads) {
            const int g = i / hd;
            qsf[g * HD + i - g * hd] = qt[i];
        }
    }
    __syncthreads();
    float4 qv[G][NF];
    #pragma unroll
    for (int g = 0; g < G; ++g)
        #pragma unroll
        for (int j = 0; j < NF; ++j)
            qv[g][j] = act ? qs[g * HD / 4 + L * j + sub] : make_float4(0.f, 0.f, 0.f, 0.f);

    // Scores in base-2 units: exp(x) = exp2(x * log2(e)).
    const float scale = 1.4426950408889634f / sqrtf(static_cast<float>(hd));
    float m[G], l[G];
    float4 acc[G][NF];
    #pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
        #pragma unroll
        for (int j = 0; j < NF; ++j) acc[g][j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int rb = 0; rb < rows; rb += kRound) {
        bool ok[NU];
        #pragma unroll
        for (int u = 0; u < NU; ++u) ok[u] = rb + (u * kSplitWaves + wave) * R + rq < rows;
        float s[NU][G];
        score_rows<G, NF, L, NU>(qv, kk, ok, scale, s);
        // The next round's keys load while this round's values are consumed.
        // Unconditional: past the split they read as zero without memory
        // traffic, and a branch here would make the compiler wait for every
        // load in flight before the values.
        #pragma unroll
        for (int u = 0; u < NU; ++u)
            #pragma unroll
            for (int j = 0; j < NF; ++j)
                kk[u][j] = ld_row4(krs, lane_off + 16 * L * j, (rb + kRound + (u * kSplitWaves + wave) * R) * row_bytes);
        __builtin_amdgcn_sched_barrier(0);   // keep the loads ahead of the value work
        absorb_rows<G, NF, NU>(s, vv, m, l, acc);
        #pragma unroll
        for (int u = 0; u < NU; ++u)
            #pragma unroll
            for (int j = 0; j < NF; ++j)
                vv[u][j] = ld_row4(vrs, lane_off + 16 * L * j, (rb + kRound + (u * kSplitWaves + wave) * R) * row_bytes);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (fresh && wave == kSplitWaves - 1) {   // row pos, from LDS, in lane group 0
        float4 k1[1][NF], v1[1][NF];
        #pragma unroll
        for (int j = 0; j < NF; ++j) {
            k1[0][j] = act ? knew[L * j + sub] : make_float4(0.f, 0.f, 0.f, 0.f);
            v1[0][j] = act ? vnew[L * j + sub] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const bool ok1[1] = {rq == 0};
        float s1[1][G];
        score_rows<G, NF, L, 1>(qv, k1, ok1, scale, s1);
        absorb_rows<G, NF, 1>(s1, v1, m, l, acc);
    }

    // The wave's lane groups meet in every lane, then the waves in LDS.
    #pragma unroll
    for (int off = L; off < 64; off *= 2)
        #pragma unroll
        for (int g = 0; g < G; ++g) {
            float f, fo;
            merge_scales(m[g], l[g], __shfl_xor(m[g], off), __shfl_xor(l[g], off), f, fo);
            #pragma unroll
            for (int j = 0; j < NF; ++j) {
                float4 &x = acc[g][j];
                x.x = x.x * f + __shfl_xor(x.x, off) * fo;
                x.y = x.y * f + __shfl_xor(x.y, off) * fo;
                x.z = x.z * f + __shfl_xor(x.z, off) * fo;
                x.w = x.w * f + __shfl_xor(x.w, off) * fo;
            }
        }
    if (rq == 0 && act)
        #pragma unroll
        for (int g = 0; g < G; ++g)
            #pragma unroll
            for (int j = 0; j < NF; ++j) part[wave][g * HD / 4 + L * j + sub] = acc[g][j];
    if (lane == 0)
        #pragma unroll
        for (int g = 0; g < G; ++g) {
            wm[wave][g] = m[g];
            wl[wave][g] = l[g];
        }
    __syncthreads();

    constexpr int kHdr = split_header(G);
    const int pstride = kHdr + G * hd;
    float *mine = ka.partials + ((static_cast<int64_t>(b) * gridDim.x + kvh) * ka.splits + split) * pstride;
    for (int i = tid; i < G * hv; i += kSplitThreads) {
        const int g = i / hv, e = i - g * hv;
        float mw = wm[0][g], lw = wl[0][g];
        float4 x = part[0][g * HD / 4 + e];
        #pragma unroll
        for (int w = 1; w < kSplitWaves; ++w) {
            float f, fo;
            merge_scales(mw, lw, wm[w][g], wl[w][g], f, fo);
            const float4 y = part[w][g * HD / 4 + e];
            x.x = x.x * f + y.x * fo;
            x.y = x.y * f + y.y * fo;
            x.z = x.z * f + y.z * fo;
            x.w = x.w * f + y.w * fo;
        }
        if (nsplit == 1) {
            const float4 r = scale4(x, 1.0f / lw);
            *reinterpret_cast<float4 *>(o + g * hd + 4 * e) = r;
            if (a.rec_out || a.gemm_rec) qs[g * HD / 4 + e] = r;   // the query rows are in registers by now
            if (a.q8_out) {
                // Column kvh * G * hd + 4 * i of the token's row; hv % 8 == 0, so
                // the eight lanes of a group share g and are active together.
                const int64_t c4 = (static_cast<int64_t>(b) * a.heads * hd + kvh * G * hd) / 4 + i;
                quantize_quad_store(r, (i & 7) == 0, reinterpret_cast<uint32_t *>(a.q8_out) + c4,
                                    a.q8_scale + c4 / 8);
            }
        } else {
            if (e == 0) {
                mine[g] = mw;
                mine[G + g] = lw;
            }
            *reinterpret_cast<float4 *>(mine + kHdr + g * hd + 4 * e) = x;
        }
    }
    if (nsplit == 1 && a.gemm_rec) {
        // The o projection's matrix-core records of this token's G heads.
        __syncthreads();
        write_gemm_records<G>(a, b, kvh, reinterpret_cast<const float *>(qs), HD);
    }
    if (nsplit == 1 && a.rec_out) {
        // The o projection's activation records of this token's G heads.
        __syncthreads();
        // Four groups per wave, 16 lanes each.
        const float *of = reinterpret_cast<const float *>(qs);
        XGroup *rec = a.rec_out + (static_cast<int64_t>(b) * a.heads * hd + kvh * G * hd) / 16;
        const int groups = G * hd / 16;
        for (int g0 = wave * 4; g0 < groups; g0 += kSplitWaves * 4) {
            const int gi = g0 + (lane >> 4), live = gi < groups;
            const int g = gi / (hd / 16), c = (gi - g * (hd / 16)) * 16;
            record16_quads(live ? of[g * HD + c + (lane & 15)] : 0.f, lane, rec + gi, live);
        }
    }
}

// The splits of (token, KV head) with more than one, when the attention
// launch did not merge them itself.
template <int G>
__global__ __launch_bounds__(256) void split_merge_kernel(SplitAttnKernelArgs ka) {
    __shared__ float mo[G * 256];   // the merged outputs, for the records (head_dim <= 256)
    const SplitAttention &a = ka.a;
    const int kvh = blockIdx.x, b = blockIdx.y;
    const qk_batch_token d = a.desc ? a.desc[b] : qk_batch_token{a.pos, 0, 0};
    if (!token_ok(d, a.cache_rows, a.max_pos)) return;
    const int nsplit = (d.pos + ka.split_rows) / ka.split_rows;
    if (nsplit == 1) return;
    merge_splits<G>(ka, b, kvh, nsplit, mo);
}

// dst row i = src row idx[i] (cols floats, cols % 4 == 0, 16-byte aligned
// rows): the activations of the tokens whose logits a step computes.
__global__ void gather_rows_kernel(const float *src, int64_t ld, const int32_t *idx, int cols, float *dst) {
    const int i = blockIdx.y;
    const int c = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (c >= cols) return;
    const float4 v = *reinterpret_cast<const float4 *>(src + static_cast<int64_t>(idx[i]) * ld + c);
    *reinterpret_cast<float4 *>(dst + static_cast<int64_t>(i) * cols + c) = v;
}

__global__ void add_kernel(float *x, const float *y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += y[i];
}

__global__ void silu_mul_kernel(float *gate, const float *up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        gate[i] = silu_mul_value(gate[i], up[i]);
    }
}

// (value, index) order of argmax_blocks_cuda / argmax_final_cuda
// (inferencer.cu:1063-1099): larger value wins, equal values keep the lower
// index.

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

// One block per row: the row's parts partials -> out[row] (and host_out[row]
// when given: host-coherent pinned memory, so the host reads the token once
// the stream is done, with no copy launch).  With e.out (one row), the
// block then writes the picked token's embedding row there (embedding_kernel's
// decode, the next step's input).
__global__ __launch_bounds__(256) void argmax_final_kernel(const float *pv, const int *pi, int parts, int32_t *out,
                                                           int32_t *host_out, NextEmbedding e) {
    __shared__ int picked;
    pv += static_cast<int64_t>(blockIdx.x) * parts;
    pi += static_cast<int64_t>(blockIdx.x) * parts;
    __shared__ float sv[4];
    __shared__ int si[4];
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    // Every load of a round is issued before the first comparison (the
    // kernel is one workgroup: its time is the loads' round trips).
    // arg_better keeps the lowest index among maxima whatever the order.
    constexpr int kPer = 16;
    for (int base = 0; base < parts; base += 256 * kPer) {
        float v[kPer];
        int ix[kPer];
        #pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int k = base + j * 256 + static_cast<int>(threadIdx.x);
            v[j] = k < parts ? pv[k] : -INFINITY;
            ix[j] = k < parts ? pi[k] : 0x7FFFFFFF;
        }
        #pragma unroll
        for (int j = 0; j < kPer; ++j) arg_better(bv, bi, v[j], ix[j]);
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
        // All -inf (or NaN) input: fall back to index 0 like an empty tree.
        const int r = bi == 0x7FFFFFFF ? 0 : bi;
        if (blockIdx.y == 0) {
            out[blockIdx.x] = r;
            if (host_out) host_out[blockIdx.x] = r;
        }
        picked = r;
    }
    if (e.out) {   // workgroup (0, b) decodes block b of the picked row
        __syncthreads();
        const int i = threadIdx.x, b = blockIdx.y;
        const uint8_t *row = e.table + static_cast<int64_t>(picked) * e.row_bytes;
        e.out[b * 256 + i] = e.type == QK_TYPE_Q4_K
                                 ? q4k_value(row + b * 144, i)
                                 : q6k_value(q6_fields(row, e.nb, b, e.type == QK_TYPE_Q6_K_SPLIT), i);
    }
}

// Split-attention instance for G and head_dim: 8 lanes per cache row when
// G * head_dim <= 512, else 16; NF float4 per lane.  NULL when unsupported.
// NW: waves per workgroup -- 4 for splits and for the one-split form that
// needs no merge (section below).
template <int G, int NF, int L, int NW>
const void *split_fn() {
    return reinterpret_cast<const void *>(split_attention_kernel<G, NF, L, NW>);
}

template <int G, int NW>
const void *split_for(int head_dim) {
    if (G * head_dim <= 512) {
        if (head_dim <= 32) return split_fn<G, 1, 8, NW>();
        if (head_dim == 64) return split_fn<G, 2, 8, NW>();
        if constexpr (G <= 4)
            if (head_dim == 128) return split_fn<G, 4, 8, NW>();
        if constexpr (G <= 2)
            if (head_dim == 256) return split_fn<G, 8, 8, NW>();
        return nullptr;
    }
    if constexpr (G >= 6)
        if (head_dim == 128) return split_fn<G, 2, 16, NW>();
    if constexpr (G >= 3)
        if (head_dim == 256) return split_fn<G, 4, 16, NW>();
    return nullptr;
}

template <int NW>
const void *split_instance_w(int G, int head_dim) {
    if (head_dim < 4 || head_dim % 4 || 256 % head_dim) return nullptr;
    switch (G) {
        case 1: return split_for<1, NW>(head_dim);
        case 2: return split_for<2, NW>(head_dim);
        case 3: return split_for<3, NW>(head_dim);
        case 4: return split_for<4, NW>(head_dim);
        case 6: return split_for<6, NW>(head_dim);
        case 8: return split_for<8, NW>(head_dim);
        default: return nullptr;
    }
}

// Waves of a one-split workgroup: 4 (1B decode at positions 528..591:
// 0.844 ms/token against 0.857 with 8 waves and 0.886 with 16; the
// cross-wave merge at the end is on every token's critical path).
constexpr int kWideWaves = 4;

const void *split_instance(int G, int head_dim, bool wide = false) {
    return wide ? split_instance_w<kWideWaves>(G, head_dim) : split_instance_w<4>(G, head_dim);
}

const void *split_merge_instance(int G) {
    switch (G) {
        case 1: return reinterpret_cast<const void *>(split_merge_kernel<1>);
        case 2: return reinterpret_cast<const void *>(split_merge_kernel<2>);
        case 3: return reinterpret_cast<const void *>(split_merge_kernel<3>);
        case 4: return reinterpret_cast<const void *>(split_merge_kernel<4>);
        case 6: return reinterpret_cast<const void *>(split_merge_kernel<6>);
        case 8: return reinterpret_cast<const void *>(split_merge_kernel<8>);
        default: return nullptr;
    }
}

inline hipStream_t S(qk_stream s) { return static_cast<hipStream_t>(s); }

}  // namespace

int split_attention_rows(int64_t head_rows, int max_rows) {
    // About kSplitTarget workgroups over the call's (token, KV head) rows, at
    // least kMinSplitRows rows a split, at most kMaxSplits splits a token.
    int64_t rows = (head_rows + kSplitTarget - 1) / kSplitTarget;
    rows = std::max<int64_t>(rows, (static_cast<int64_t>(max_rows) + kMaxSplits - 1) / kMaxSplits);
    rows = std::max<int64_t>(kMinSplitRows, (rows + 15) / 16 * 16);
    return static_cast<int>(std::min<int64_t>(rows, std::max(max_rows, 1)));
}

size_t split_attention_workspace_bytes(int n_tokens, int heads, int kv_heads, int head_dim, int max_rows) {
    if (n_tokens < 1 || kv_heads < 1 || heads < kv_heads || max_rows <= kMinSplitRows) return 0;
    const int G = heads / kv_heads;
    const size_t splits = std::min<size_t>(kMaxSplits, (static_cast<size_t>(max_rows) + kMinSplitRows - 1) / kMinSplitRows);
    const size_t part = static_cast<size_t>(split_header(G) + G * head_dim) * sizeof(float);
    return std::min<size_t>(kMaxSplitWorkspace, static_cast<size_t>(n_tokens) * kv_heads * splits * part);
}

// Whether the policy runs a's tokens in the wide form (one workgroup per
// query head, one split).
bool wide_attention(const SplitAttention &a) {
    return static_cast<int64_t>(a.n_tokens) * a.heads <= kWideMaxPairs &&
           int64_t(2) * (a.max_pos + 1) * a.head_dim * static_cast<int64_t>(sizeof(float)) <= kWideMaxBytes &&
           split_instance(1, a.head_dim, true) != nullptr;
}

bool attention_gemm_records(const SplitAttention &a) {
    const int G = a.heads / a.kv_heads;
    return !wide_attention(a) && G * a.head_dim % 256 == 0 && a.head_dim <= 256 && a.heads * a.head_dim % 256 == 0;
}

int launch_split_attention(const SplitAttention &a, int split_rows, void *workspace, size_t workspace_size,
                           hipStream_t stream, int *splits_used) {
    const int G = a.heads / a.kv_heads;
    const void *fn = split_instance(G, a.head_dim);
    if (!fn) return fail(QK_ERR_LIMIT, "split attention: unsupported head layout");
    if (a.n_tokens > 65535) return fail(QK_ERR_LIMIT, "split attention: too many tokens in one launch");
    if (a.rec_out && a.head_dim % 16) return fail(QK_ERR_LIMIT, "split attention: records need head_dim % 16 == 0");
    if (a.q8_out && (a.head_dim % 32 || !a.q8_scale))
        return fail(QK_ERR_LIMIT, "split attention: quantized outputs need head_dim % 32 == 0 and scales");
    if (a.qkv_splits > 1 && (!a.qkv_parts || !a.k || !a.v || a.qkv_ttiles < (a.n_tokens + 31) / 32))
        return fail(QK_ERR_INVALID_ARG, "split attention: split QKV sums need k, v and their partials");
    const int max_rows = a.max_pos + 1;
    // Few (token, KV head) pairs over short rows: one wide workgroup each
    // reads all of its rows, and no merge kernel runs.  A CU alone streams
    // its 2 x 531 rows of 256 B (one 1B token at position ~530) in about
    // 3.5 us, against 2.9 us for splits of 64 rows plus a 4 us merge.
    // Each wide workgroup serves one query head (its KV head's rows are read
    // by G workgroups, mostly from cache), so the softmax arithmetic spreads
    // over heads CUs instead of kv_heads.
    const bool wide = split_rows <= 0 && wide_attention(a);
    int head_split = 1, Gk = G;
    if (wide) {
        head_split = G;
        Gk = 1;
        fn = split_instance(1, a.head_dim, true);
        split_rows = a.wide_split_rows > 0 ? std::min(a.wide_split_rows, max_rows) : max_rows;
    }
    // GEMM records: each workgroup's heads must fill whole 256-column blocks
    // (never so in the one-head-per-workgroup form).
    if (a.gemm_rec && (Gk * a.head_dim % 256 || a.head_dim > 256))
        return fail(QK_ERR_LIMIT, "split attention: GEMM records need whole 256-column blocks per workgroup");
    const int groups = a.kv_heads * head_split;   // workgroups per token and split
    if (split_rows <= 0) {
        const int64_t rows = a.rows_hint > 0 ? a.rows_hint : static_cast<int64_t>(a.n_tokens) * max_rows;
        split_rows = split_attention_rows(rows * a.kv_heads, max_rows);
    }
    split_rows = std::min(split_rows, max_rows);
    int nsplit = (max_rows + split_rows - 1) / split_rows;
    if (nsplit > 1) {
        // Fewer, longer splits when the workspace is short; one without it.
        const size_t per = static_cast<size_t>(a.n_tokens) * groups *
                           static_cast<size_t>(split_header(Gk) + Gk * a.head_dim) * sizeof(float);
        const int64_t fit = workspace ? static_cast<int64_t>(workspace_size / per) : 0;
        if (fit < 2)
            split_rows = max_rows;
        else if (nsplit > fit)
            split_rows = static_cast<int>((max_rows + fit - 1) / fit);
        nsplit = (max_rows + split_rows - 1) / split_rows;
    }
    // Row offsets of a split (plus one round of prefetch past it) stay below 2 GiB.
    if ((static_cast<int64_t>(split_rows) + 512) * a.kv_heads * a.head_dim * static_cast<int64_t>(sizeof(float)) >=
        (1ll << 31))
        return fail(QK_ERR_LIMIT, "split attention: a split spans 2 GiB of cache rows");
    SplitAttnKernelArgs ka;
    ka.a = a;
    ka.partials = nsplit > 1 ? static_cast<float *>(workspace) : nullptr;
    ka.split_rows = split_rows;
    ka.splits = nsplit;
    ka.head_split = head_split;
    void *args[] = {&ka};
    if (hipLaunchKernel(fn, dim3(groups, a.n_tokens, nsplit), dim3(wide ? kWideWaves * 64 : kSplitThreads), args,
                        0, stream) != hipSuccess)
        return launch_status("split attention launch");
    // Deferred merges only in the wide form (its partials are one query
    // head per workgroup).
    const bool defer = nsplit > 1 && wide && a.defer_merge;
    if (splits_used) *splits_used = defer ? nsplit : 1;
    if (nsplit > 1 && !defer) {
        const void *merge = split_merge_instance(Gk);
        if (hipLaunchKernel(merge, dim3(groups, a.n_tokens), dim3(256), args, 0, stream) != hipSuccess)
            return launch_status("split attention merge launch");
    }
    return launch_status("split attention launch");
}

bool attention_supported(int group, int head_dim) { return split_instance(group, head_dim) != nullptr; }

int launch_argmax_final(const float *pv, const int *pi, int parts, int32_t *out, hipStream_t stream,
                        int32_t *host_out, const NextEmbedding *next) {
    // With a next embedding, one workgroup per 256-value block of the row,
    // each repeating the (small) final pick over the partials.
    const int blocks = next && next->out ? next->nb : 1;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1, blocks), dim3(256), 0, stream, pv, pi, parts, out, host_out,
                       next ? *next : NextEmbedding{});
    return launch_status("argmax final launch");
}

int launch_gather_rows(const float *src, int64_t ld, const int32_t *idx, int n, int cols, float *dst,
                       hipStream_t stream) {
    if (n < 1) return QK_OK;
    if (n > 65535 || cols % 4 || ld % 4 || !aligned(src, 16) || !aligned(dst, 16))
        return fail(QK_ERR_LIMIT, "row gather: unsupported shape");
    hipLaunchKernelGGL(gather_rows_kernel, dim3((cols / 4 + 255) / 256, n), dim3(256), 0, stream, src, ld, idx, cols,
                       dst);
    return launch_status("row gather launch");
}

int launch_rope_kv_batched(float *q, const float *k, const float *v, const float *cosine, const float *sine,
                           float *key_cache, float *value_cache, int layer, int64_t cache_rows,
                           const qk_batch_token *desc, int n_tokens, int context, int heads, int kv_heads,
                           int head_dim, int head_major, hipStream_t stream) {
    const int q_pairs = heads * head_dim / 2, kv_pairs = kv_heads * head_dim / 2;
    hipLaunchKernelGGL(rope_kv_batched_kernel, dim3((q_pairs + 255) / 256, n_tokens), dim3(256), 0, stream, q, k, v,
                       cosine, sine, key_cache, value_cache, layer, cache_rows, desc, context, q_pairs, kv_pairs,
                       head_dim / 2, head_major);
    return launch_status("qk_rope_kv_write_batched launch");
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

int qk_rmsnorm_quantize_x32(const float *x, int ldx, const float *weight, float *out, int ldout, int8_t *xq,
                            int ldxq, float *xscale, int ldscale, int cols, int n_tokens, float eps,
                            qk_stream stream) {
    if (!x || !weight || !xq || !xscale || cols < 1 || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rmsnorm_quantize_x32: null pointer or bad size");
    if (cols % 32) return qk::fail(QK_ERR_SHAPE, "qk_rmsnorm_quantize_x32: cols must be a multiple of 32");
    if (n_tokens == 0) return qk::ok();
    if (ldx < cols || ldxq < cols || ldscale < cols / 32 || (out && ldout < cols))
        return qk::fail(QK_ERR_INVALID_ARG, "qk_rmsnorm_quantize_x32: leading dimension smaller than the row");
    if (!qk::aligned(x, 16) || !qk::aligned(weight, 16) || (out && !qk::aligned(out, 16)) || !qk::aligned(xq, 4) ||
        ldx % 4 || (out && ldout % 4) || ldxq % 4)
        return qk::fail(QK_ERR_ALIGN, "qk_rmsnorm_quantize_x32: x, weight, out need 16-byte rows, xq 4-byte rows");
    hipLaunchKernelGGL(qk::rmsnorm_quantize_kernel, dim3(n_tokens), dim3(256), 0, qk::S(stream), x, ldx, weight, out,
                       ldout, xq, ldxq, xscale, ldscale, cols, eps);
    return qk::launch_status("qk_rmsnorm_quantize_x32 launch");
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
    if (!qk::attention_supported(heads / kv_heads, head_dim))
        return qk::fail(QK_ERR_LIMIT, "qk_attention_f32: query heads per KV head must be 1, 2, 3, 4, 6 or 8");
    if (!qk::aligned(key_cache, 16) || !qk::aligned(value_cache, 16) || !qk::aligned(out, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_attention_f32: caches and out must be 16-byte aligned");
    qk::SplitAttention a{};
    a.q = q;
    a.key_cache = const_cast<float *>(key_cache);
    a.value_cache = const_cast<float *>(value_cache);
    a.out = out;
    a.cache_rows = context;
    a.layer = layer;
    a.pos = a.max_pos = pos;
    a.n_tokens = 1;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    return qk::launch_split_attention(a, 0, nullptr, 0, qk::S(stream));
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
    return qk::launch_rope_kv_batched(q, k, v, cosine, sine, key_cache, value_cache, layer, cache_rows, desc, n_tokens,
                                      context, heads, kv_heads, head_dim, 0, qk::S(stream));
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
    if (!qk::attention_supported(heads / kv_heads, head_dim))
        return qk::fail(QK_ERR_LIMIT, "qk_attention_batched_f32: query heads per KV head must be 1, 2, 3, 4, 6 or 8");
    if (!qk::aligned(key_cache, 16) || !qk::aligned(value_cache, 16) || !qk::aligned(out, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_attention_batched_f32: caches and out must be 16-byte aligned");
    if (n_tokens == 0) return qk::ok();
    qk::SplitAttention a{};
    a.q = q;
    a.key_cache = const_cast<float *>(key_cache);
    a.value_cache = const_cast<float *>(value_cache);
    a.out = out;
    a.desc = desc;
    a.cache_rows = cache_rows;
    a.layer = layer;
    a.max_pos = max_pos;
    a.n_tokens = n_tokens;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    return qk::launch_split_attention(a, 0, nullptr, 0, qk::S(stream));
}

size_t qk_attention_split_workspace_bytes(int n_tokens, int heads, int kv_heads, int head_dim, int max_pos,
                                          int split_rows) {
    if (n_tokens < 1 || heads < 1 || kv_heads < 1 || heads % kv_heads || head_dim < 4 || max_pos < 0) return 0;
    if (split_rows <= 0) return qk::split_attention_workspace_bytes(n_tokens, heads, kv_heads, head_dim, max_pos + 1);
    const size_t splits = (static_cast<size_t>(max_pos) + split_rows) / split_rows;
    if (splits < 2) return 0;
    const int G = heads / kv_heads;
    return static_cast<size_t>(n_tokens) * kv_heads * splits * (qk::split_header(G) + G * head_dim) * sizeof(float);
}

int qk_attention_split_f32(const float *q, const float *key_cache, const float *value_cache, float *out, int layer,
                           int64_t cache_rows, const qk_batch_token *desc, int n_tokens, int max_pos, int heads,
                           int kv_heads, int head_dim, int split_rows, void *workspace, size_t workspace_size,
                           qk_stream stream) {
    if (!q || !key_cache || !value_cache || !out || (!desc && n_tokens > 0) || n_tokens < 0 || split_rows < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_attention_split_f32: null pointer or negative count");
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || layer < 0 || cache_rows < 1 || max_pos < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_attention_split_f32: bad head layout or cache shape");
    if (head_dim < 4 || head_dim % 4 || 256 % head_dim)
        return qk::fail(QK_ERR_LIMIT, "qk_attention_split_f32: head_dim must be a multiple of 4 dividing 256");
    if (!qk::attention_supported(heads / kv_heads, head_dim))
        return qk::fail(QK_ERR_LIMIT, "qk_attention_split_f32: query heads per KV head must be 1, 2, 3, 4, 6 or 8");
    if (!qk::aligned(key_cache, 16) || !qk::aligned(value_cache, 16) || !qk::aligned(out, 16) ||
        !qk::aligned(workspace, 16))
        return qk::fail(QK_ERR_ALIGN, "qk_attention_split_f32: caches, out and workspace must be 16-byte aligned");
    if (n_tokens == 0) return qk::ok();
    qk::SplitAttention a{};
    a.q = q;
    a.key_cache = const_cast<float *>(key_cache);
    a.value_cache = const_cast<float *>(value_cache);
    a.out = out;
    a.desc = desc;
    a.cache_rows = cache_rows;
    a.layer = layer;
    a.max_pos = max_pos;
    a.n_tokens = n_tokens;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    return qk::launch_split_attention(a, split_rows, workspace, workspace_size, qk::S(stream));
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
    hipLaunchKernelGGL(qk::argmax_final_kernel, dim3(rows), dim3(256), 0, qk::S(stream), pv, pi, parts, out, nullptr,
                       qk::NextEmbedding{});
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
    hipLaunchKernelGGL(qk::argmax_final_kernel, dim3(1), dim3(256), 0, qk::S(stream), pv, pi, parts, out, nullptr,
                       qk::NextEmbedding{});
    return qk::launch_status("qk_argmax_f32 launch");
}

}  // extern "C"
