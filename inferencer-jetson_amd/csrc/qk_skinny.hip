// qk_skinny.hip - the INT8 multi-token GEMM on the integer matrix cores.
//
// The reference's INT8 multi-token path -- gemv_batch_dp4a over per-32
// quantized activations (inferencer.cu:678-699; qkv_batch_cuda and
// gate_up_batch_cuda, 701-751; FastRunner::batch_matvec, 1265-1278) --
// takes xq / xscale from quantize_x32_cuda (544-556) and, per row, exact
// integer sub-block dots combined in float:
//   Q4_K sub-block s (32 columns): (d*sc_s*I_s - dmin*m_s*S_s) * xscale_s,
//        I_s = sum xq*q, S_s = sum xq          (dot_q4_block_dp4a, 520-542)
//   Q6_K sub-block j (16 columns): d*scale_j*I_j*xscale_(j/2),
//        I_j = sum xq*(code - 32)              (dot_q6_block_dp4a, 613-643)
// Here the integer dots run on the matrix cores, 32 tokens x 32 weight rows
// at a time: v_mfma_i32_32x32x32_i8 takes one Q4_K sub-block per
// instruction, v_mfma_i32_32x32x16_i8 one Q6_K sub-block (A = the tokens'
// xq, B = the rows' codes; lane l holds token / row l % 32 and half l / 32
// of the sub-block's columns).  The float combine follows each sub-block
// (the two Q6_K sub-blocks sharing an xscale meet first in integers), and
// the Q4_K min term -dmin * sum_s m_s * xscale_s * S_s of a whole block is
// one K = 8 product on v_mfma_f32_32x32x2_f32.
//
// A workgroup owns 32 weight rows (one row tile; a gate / up pair owns the
// same 32 rows of both) x 32 tokens x every block of the row: its waves
// split the row's blocks, each issuing its first block's loads before any
// arithmetic and the next block's before each block's arithmetic, then the
// waves' partial sums meet in LDS in wave order (deterministic) and the
// workgroup applies the epilogue itself -- store, residual add, or SiLU(gate)
// * up quantized per 32 values for the next product (silu_cuda then
// quantize_batch_cuda, inferencer.cu:1053-1057, 891-904) -- so the call
// needs no workspace and no reduction launch.
#include "qk_internal.h"

#include <algorithm>

namespace qk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kRows = 32;      // weight rows per row tile (the MFMA's N)
constexpr int kToks = 32;      // tokens per token tile (the MFMA's M)
// Waves (one block each) a workgroup may spread a row over: 16 where the
// kernel fits 128 VGPRs (Q4_K, one row tile), else 12 (at most 170 VGPRs).
// A 3072-column row (12 blocks) then needs one workgroup.
__host__ __device__ constexpr int waves_max(int type, int rt) { return type == QK_TYPE_Q4_K && rt == 1 ? 16 : 12; }

enum Epilogue { kStore = 0, kAccumulate = 1, kPairQuant = 2 };

struct SkMatrix {
    const uint8_t *w;
    float *y;
    int rows, type, row_bytes, ldy;
    int tile_begin;   // first 32-row tile of this matrix in the launch
};

struct SkParams {
    SkMatrix mat[QK_MAX_FUSED];
    int n_mats;
    const int8_t *xq;
    const float *xs;
    int ldxq, ldxs;
    int n_tokens, nb;
    int tiles;           // row tiles of the launch
    int splits, waves;   // workgroups per row and blocks (= waves) per workgroup
    int epilogue;
    // kPairQuant: SiLU(y0) * y1 of matrices 0 and 1, quantized per 32 values
    // into out_xq [token][out_ldxq] / out_xs [token][out_ldxs].
    int8_t *out_xq;
    float *out_xs;
    int out_ldxq, out_ldxs;
    float *partials;   // splits > 1: [tile][token tile][split][RT * 1024]
};

// One block of one row as the lane loads it.
//   Q4_K: v[0] the 16-byte header, v[1 + g] bytes 16 + 32g + 16kh .. +15 of
//         qs (group g's low nibbles are sub-block 2g, high nibbles 2g + 1).
//   Q6_K: runs of 8 bytes at ql g*64 + h*32 + 16e + 8kh (run n = 4g + 2h + e,
//         v[n / 2], the low half for even n) and qh g*32 + 16e + 8kh (run
//         n = 2g + e, v[4 + n / 2]); v[6] the sixteen int8 scales; d.
struct Raw {
    uint4 v[7];
    uint32_t d;
};

template <int TYPE>
__device__ __forceinline__ bool is_q4(int type) {
    return TYPE == QK_TYPE_Q4_K || (TYPE == 0 && type == QK_TYPE_Q4_K);
}

template <int TYPE>
__device__ __forceinline__ void load_raw(Raw &r, const uint8_t *row, int b, int nb, int type, int kh) {
    if (is_q4<TYPE>(type)) {
        const uint8_t *blk = row + static_cast<size_t>(b) * 144;
        r.v[0] = load16(blk);
        #pragma unroll
        for (int g = 0; g < 4; ++g) r.v[1 + g] = load16(blk + 16 + 32 * g + 16 * kh);
        r.v[5] = r.v[6] = make_uint4(0, 0, 0, 0);
        r.d = 0;
    } else {
        const bool split = TYPE == QK_TYPE_Q6_K_SPLIT || (TYPE == 0 && type == QK_TYPE_Q6_K_SPLIT);
        const Q6Fields f = q6_fields(row, nb, b, split);
        #pragma unroll
        for (int n = 0; n < 8; n += 2) {
            const int g = n >> 2, h = (n >> 1) & 1;
            const uint2 lo = load8(f.ql + g * 64 + h * 32 + 8 * kh);
            const uint2 hi = load8(f.ql + g * 64 + h * 32 + 16 + 8 * kh);
            r.v[n >> 1] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
        #pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint2 lo = load8(f.qh + g * 32 + 8 * kh);
            const uint2 hi = load8(f.qh + g * 32 + 16 + 8 * kh);
            r.v[4 + g] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
        r.v[6] = load16(f.sc);
        r.d = load2(f.d);
    }
}

// The lane's token's quantized activations of block b (A operands) and its
// eight per-32 scales.  Q4_K sub-block s: bytes 32s + 16kh .. +15 (a[s]);
// Q6_K sub-blocks 2c and 2c + 1: bytes 32c + 8kh .. +7 and 32c + 16 + 8kh ..
// +7 (a[c], low and high half).
template <int TYPE>
__device__ __forceinline__ void load_act(uint4 (&a)[8], float (&x)[8], const int8_t *xrow, const float *srow, int b,
                                         int type, int kh) {
    const uint8_t *base = reinterpret_cast<const uint8_t *>(xrow) + static_cast<size_t>(b) * 256;
    #pragma unroll
    for (int s = 0; s < 8; ++s) {
        if (is_q4<TYPE>(type)) {
            a[s] = *reinterpret_cast<const uint4 *>(base + 32 * s + 16 * kh);
        } else {
            const uint2 lo = *reinterpret_cast<const uint2 *>(base + 32 * s + 8 * kh);
            const uint2 hi = *reinterpret_cast<const uint2 *>(base + 32 * s + 16 + 8 * kh);
            a[s] = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
    }
    #pragma unroll
    for (int c = 0; c < 8; ++c) x[c] = srow[b * 8 + c];
}

__device__ __forceinline__ v4i as_v4i(uint4 u) { return v4i{int(u.x), int(u.y), int(u.z), int(u.w)}; }
__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) {
    return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Codes (0..63) of four Q6_K weights as int8 code - 32: the bytes lie in
// 128..191 after | 0x80, so - 0x20 borrows across no byte, and ^ 0x80 maps
// 96..159 to code - 32 in two's complement.
__device__ __forceinline__ uint32_t q6_centre(uint32_t code) {
    return ((code | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

// This block's scales of the lane's 16 output tokens for chunk c (the
// wave's transposed copy in LDS: xst[c][token]); register i of an
// accumulator holds token 8*(i/4) + 4*kh + i%4.
__device__ __forceinline__ void chunk_scales(const float *xst, int c, int kh, float (&xr)[16]) {
    #pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 v = *reinterpret_cast<const float4 *>(xst + c * kToks + 8 * q + 4 * kh);
        xr[4 * q] = v.x;
        xr[4 * q + 1] = v.y;
        xr[4 * q + 2] = v.z;
        xr[4 * q + 3] = v.w;
    }
}

// Q4_K sub-block s (2g + h: the low / high nibbles of qs group g) of the
// lane's row against its token's xq: exact int32 dots, tokens x rows.
__device__ __forceinline__ v16i q4_dot(const Raw &r, const uint4 (&a)[8], int s) {
    const v16i zero = {};
    const uint4 q = r.v[1 + (s >> 1)];
    const uint32_t sh = 4 * (s & 1);
    const uint4 nib = make_uint4((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu, (q.z >> sh) & 0x0F0F0F0Fu,
                                 (q.w >> sh) & 0x0F0F0F0Fu);
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(as_v4i(a[s]), as_v4i(nib), zero, 0, 0, 0);
}

// Q6_K sub-block 2c + e (chunk c = part c % 4 of half c / 4): the lane's
// eight codes, centred, against its token's eight xq.
__device__ __forceinline__ v16i q6_dot(const Raw &r, const uint4 (&a)[8], int c, int e) {
    const v16i zero = {};
    const int g = c >> 2, part = c & 3;
    const uint4 ql = r.v[g * 2 + (part & 1)];
    const uint4 qh = r.v[4 + g];
    const uint32_t lsh = 4 * (part >> 1), hsh = 2 * part;
    const uint32_t l0 = e ? ql.z : ql.x, l1 = e ? ql.w : ql.y;
    const uint32_t h0 = e ? qh.z : qh.x, h1 = e ? qh.w : qh.y;
    const uint32_t c0 = q6_centre(((l0 >> lsh) & 0x0F0F0F0Fu) | (((h0 >> hsh) & 0x03030303u) << 4));
    const uint32_t c1 = q6_centre(((l1 >> lsh) & 0x0F0F0F0Fu) | (((h1 >> hsh) & 0x03030303u) << 4));
    const long av = e ? as_long(a[c].z, a[c].w) : as_long(a[c].x, a[c].y);
    return __builtin_amdgcn_mfma_i32_32x32x16_i8(av, as_long(c0, c1), zero, 0, 0, 0);
}

// Ends one step of a block: the step's combine must be complete here (the
// accumulator passes through an empty asm statement), and the scheduler
// moves nothing across.  Without it the instruction selector orders every
// step's matrix-core dots ahead of every combine, and the dots' results and
// scales no longer fit the registers.
__device__ __forceinline__ void step_fence(v16f &acc) {
    asm volatile("" : "+v"(acc));
    __builtin_amdgcn_sched_barrier(0);
}

// acc += this block's contribution for one row tile.  a: the lane's token's
// xq; xst: the wave's [8][32] transpose of the block's per-32 scales;
// xss[s] = xscale_s * S_s of the lane's token (Q4_K).  The matrix-core dots
// of step k + 1 are issued before step k is combined.
template <int TYPE>
__device__ __forceinline__ void block_i8(const Raw &r, int type, const uint4 (&a)[8], const float *xst,
                                         const float (&xss)[8], int kh, v16f &acc, v16f &accmin) {
    if (is_q4<TYPE>(type)) {
        const float d = f16_bits_to_f32(r.v[0].x & 0xFFFFu), dmin = f16_bits_to_f32(r.v[0].x >> 16);
        uint32_t sc03, mn03, sc47, mn47;
        q4k_scale_min4(r.v[0], 0, sc03, mn03);
        q4k_scale_min4(r.v[0], 1, sc47, mn47);
        v16i cur = q4_dot(r, a, 0);
        #pragma unroll
        for (int s = 0; s < 8; ++s) {
            v16i nxt;
            if (s < 7) nxt = q4_dot(r, a, s + 1);
            const float dsc = d * static_cast<float>(((s < 4 ? sc03 : sc47) >> (8 * (s & 3))) & 0xFFu);
            float xr[16];
            chunk_scales(xst, s, kh, xr);
            #pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = fmaf(static_cast<float>(cur[i]), dsc * xr[i], acc[i]);
            if (s < 7) cur = nxt;
            step_fence(acc);
        }
        // -dmin * sum_s m_s * (xscale_s * S_s): A = the tokens' xss (K index
        // = sub-block 2j + kh, selected rather than indexed by lane), B = the
        // rows' -dmin * m.
        #pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t mb = (j < 2 ? mn03 : mn47) >> (16 * (j & 1));
            const float m = static_cast<float>(kh ? (mb >> 8) & 0xFFu : mb & 0xFFu);
            const float xa = kh ? xss[2 * j + 1] : xss[2 * j];
            accmin = __builtin_amdgcn_mfma_f32_32x32x2f32(xa, -dmin * m, accmin, 0, 0, 0);
        }
    } else {
        const float d = f16_bits_to_f32(r.d);
        v16f blk = {};
        v16i c0 = q6_dot(r, a, 0, 0), c1 = q6_dot(r, a, 0, 1);
        #pragma unroll
        for (int c = 0; c < 8; ++c) {
            v16i n0, n1;
            if (c < 7) {
                n0 = q6_dot(r, a, c + 1, 0);
                n1 = q6_dot(r, a, c + 1, 1);
            }
            // scales[2c], scales[2c + 1] (int8)
            const uint32_t sw = c < 2 ? r.v[6].x : c < 4 ? r.v[6].y : c < 6 ? r.v[6].z : r.v[6].w;
            const int s0 = static_cast<int8_t>((sw >> (16 * (c & 1))) & 0xFFu);
            const int s1 = static_cast<int8_t>((sw >> (16 * (c & 1) + 8)) & 0xFFu);
            float xr[16];
            chunk_scales(xst, c, kh, xr);
            #pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int jsum = __mul24(s0, c0[i]) + __mul24(s1, c1[i]);   // |.| < 2^24: exact
                blk[i] = fmaf(static_cast<float>(jsum), xr[i], blk[i]);
            }
            if (c < 7) {
                c0 = n0;
                c1 = n1;
            }
            step_fence(blk);
        }
        #pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = fmaf(d, blk[i], acc[i]);
    }
}

// Partial sums of one wave in LDS: red[wave][rt][i][lane].
__device__ __forceinline__ float *red_slot(float *red, int wave, int rt, int RT) {
    return red + static_cast<size_t>(wave * RT + rt) * 1024;
}

// Orders one wave's LDS accesses around a lane-to-lane exchange: no
// compiler motion across it (the hardware runs a wave's DS operations in
// order).
__device__ __forceinline__ void wave_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

// The wave's activation block, prepared once for every row tile it meets:
// the block's per-32 scales transposed through the wave's LDS slice (a
// wave's DS operations complete in order) and the Q4_K sums S per
// sub-block of the lane's token (both column halves).
template <int TYPE>
__device__ __forceinline__ void act_prep(const uint4 (&ca)[8], const float (&cx)[8], float *xst, int col, int kh,
                                         float (&xss)[8]) {
    // Both column halves write the same values (no branch for the
    // compiler to sink the scale loads into).
    #pragma unroll
    for (int c = 0; c < 8; ++c) xst[c * kToks + col] = cx[c];
    wave_sync();
    if (is_q4<TYPE>(TYPE)) {
        #pragma unroll
        for (int s = 0; s < 8; ++s) {
            int part = __builtin_amdgcn_sdot4(static_cast<int>(ca[s].x), 0x01010101, 0, false);
            part = __builtin_amdgcn_sdot4(static_cast<int>(ca[s].y), 0x01010101, part, false);
            part = __builtin_amdgcn_sdot4(static_cast<int>(ca[s].z), 0x01010101, part, false);
            part = __builtin_amdgcn_sdot4(static_cast<int>(ca[s].w), 0x01010101, part, false);
            part += __shfl_xor(part, 32);
            xss[s] = static_cast<float>(part) * cx[s];
        }
    } else {
        #pragma unroll
        for (int s = 0; s < 8; ++s) xss[s] = 0.f;
    }
}

// The matrix of row tile `tile` in a launch over one tile column per 32
// rows of each matrix (RT 1).
__device__ __forceinline__ int tile_matrix(const SkParams &p, int tile) {
    int m = 0;
    #pragma unroll
    for (int i = 1; i < QK_MAX_FUSED; ++i) m += (i < p.n_mats && tile >= p.mat[i].tile_begin) ? 1 : 0;
    return __builtin_amdgcn_readfirstlane(m);
}

// The row tiles of workgroup tile `tile`: one of some matrix (RT 1), or the
// same 32 rows of matrices 0 and 1 (a gate / up pair, RT 2).
template <int RT>
__device__ __forceinline__ void tile_rows(const SkParams &p, int tile, int (&mi)[RT], int (&row0)[RT]) {
    if (RT == 1) {
        mi[0] = tile_matrix(p, tile);
        row0[0] = (tile - p.mat[mi[0]].tile_begin) * kRows;
    } else {
        #pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            mi[rt] = rt;
            row0[rt] = tile * kRows;
        }
    }
}

// The epilogue of one (row tile, token tile): sum(e) is the finished value
// of element e = rt*1024 + i*64 + ln -- row row0[rt] + ln % 32, token
// 8*(i/4) + 4*(ln/32) + i%4 of the token tile (the accumulator layout).
// Store, residual add, or for a gate / up pair each half-wave takes one
// token's 32 outputs, forms SiLU(gate) * up and quantizes them as one group
// of 32.
template <int RT, class Sum>
__device__ __forceinline__ void epilogue(const SkParams &p, const int (&mi)[RT], const int (&row0)[RT], int ttile,
                                         int nthreads, Sum sum) {
    if (p.epilogue != kPairQuant) {
        for (int e = threadIdx.x; e < RT * 1024; e += nthreads) {
            float v = sum(e);
            const int rt = e >> 10, i = (e >> 6) & 15, ln = e & 63;
            const SkMatrix &M = p.mat[mi[rt]];
            const int row = row0[rt] + (ln & 31);
            const int t = ttile * kToks + 8 * (i >> 2) + 4 * (ln >> 5) + (i & 3);
            if (row < M.rows && t < p.n_tokens) {
                float *y = M.y + static_cast<int64_t>(t) * M.ldy + row;
                if (p.epilogue == kAccumulate) v += *y;
                *y = v;
            }
        }
        return;
    }
    for (int base = 0; base < kToks; base += nthreads / 32) {
        const int tl = base + static_cast<int>(threadIdx.x >> 5), j = threadIdx.x & 31;
        if (tl >= kToks) break;   // uniform per half-wave
        const int e = (4 * (tl >> 3) + (tl & 3)) * 64 + j + 32 * ((tl >> 2) & 1);
        const int t = ttile * kToks + tl;
        const bool live = t < p.n_tokens;
        const int64_t tq = live ? t : 0;
        quantize_group_store(silu_mul_value(sum(e), sum(1024 + e)), live, j,
                             p.out_xq + tq * p.out_ldxq + row0[0] + j, p.out_xs + tq * p.out_ldxs + row0[0] / 32);
    }
}

// Takes the loaded words through an empty asm statement: the compiler must
// have them in registers here (it waits for their loads here, not at a
// later copy it would sink below other memory operations).
__device__ __forceinline__ void own_regs(Raw &r) {
    #pragma unroll
    for (int k = 0; k < 7; ++k) asm volatile("" : "+v"(r.v[k].x), "+v"(r.v[k].y), "+v"(r.v[k].z), "+v"(r.v[k].w));
    asm volatile("" : "+v"(r.d));
}

// Block b of the raw weight rows of row tile `tile` (every row tile of the
// workgroup: RT matrices' rows), the lane's row clamped into its matrix.
template <int TYPE, int RT>
__device__ __forceinline__ void load_tile(const SkParams &p, int tile, int b, int col, int kh, Raw (&r)[RT]) {
    int mi[RT], row0[RT];
    tile_rows<RT>(p, tile, mi, row0);
    #pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const SkMatrix &M = p.mat[mi[rt]];
        const uint8_t *wrow = M.w + static_cast<size_t>(min(row0[rt] + col, M.rows - 1)) * M.row_bytes;
        load_raw<TYPE>(r[rt], wrow, b, p.nb, TYPE, kh);
    }
}

// One workgroup: the row tiles tile0, tile0 + stride, ... (stride =
// workgroups per split and token tile; one tile unless LOOP) x its token
// tile x the `waves` blocks of its split, one block per wave.  The wave's
// activations are loaded and prepared once; with LOOP the next tile's
// weights load while this one computes (the last tile's reload is
// redundant and in bounds).
template <int TYPE, int RT, bool LOOP>
__device__ __forceinline__ void skinny_body(const SkParams &p, float *lds) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kh = lane >> 5, col = lane & 31;
    const int split = static_cast<int>(blockIdx.x) % p.splits;
    const int stride = static_cast<int>(gridDim.x) / p.splits;
    const int ttile = blockIdx.y;
    const int t_a = min(ttile * kToks + col, p.n_tokens - 1);   // token of the lane's A operand (in bounds)
    float *red = lds;
    float *xst = lds + static_cast<size_t>(p.waves) * RT * 1024 + wave * (8 * kToks);
    const int b = split * p.waves + wave;
    const bool live = b < p.nb;   // wave-uniform
    // Loads are unconditional (a wave past the row's end reloads the last
    // block, in bounds), so every path has the same loads in flight and the
    // waits before the first use of a tile stay partial.
    const int bl = min(b, p.nb - 1);
    int tile = static_cast<int>(blockIdx.x) / p.splits;

    Raw cur[RT];
    uint4 ca[8];
    float cx[8], xss[8];
    load_tile<TYPE, RT>(p, tile, bl, col, kh, cur);
    load_act<TYPE>(ca, cx, p.xq + static_cast<int64_t>(t_a) * p.ldxq, p.xs + static_cast<int64_t>(t_a) * p.ldxs, bl,
                   TYPE, kh);
    act_prep<TYPE>(ca, cx, xst, col, kh, xss);
    const int nthreads = 64 * p.waves;
    auto wave_sum = [&](int e) {   // the waves' partial sums in wave order
        float v = red[e];
        for (int w = 1; w < p.waves; ++w) v += red[static_cast<size_t>(w) * RT * 1024 + e];
        return v;
    };
    for (;;) {
        Raw nxt[RT];
        if constexpr (LOOP) load_tile<TYPE, RT>(p, min(tile + stride, p.tiles - 1), bl, col, kh, nxt);
        v16f acc[RT], accmin[RT];
        #pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            #pragma unroll
            for (int i = 0; i < 16; ++i) acc[rt][i] = accmin[rt][i] = 0.f;
        if (live) {
            #pragma unroll
            for (int rt = 0; rt < RT; ++rt) block_i8<TYPE>(cur[rt], TYPE, ca, xst, xss, kh, acc[rt], accmin[rt]);
        }
        #pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float *mine = red_slot(red, wave, rt, RT) + lane;
            #pragma unroll
            for (int i = 0; i < 16; ++i) mine[i * 64] = acc[rt][i] + accmin[rt][i];
        }
        __syncthreads();
        // The next tile's weights move into place before this tile's stores
        // go out: the wait for them then leaves the stores in flight (vector
        // memory counts complete in order, so a wait placed after the stores
        // would also wait for their write-back).
        if constexpr (LOOP) {
            #pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                own_regs(nxt[rt]);
                cur[rt] = nxt[rt];
            }
        }
        if (p.splits == 1) {
            int mi[RT], row0[RT];
            tile_rows<RT>(p, tile, mi, row0);
            epilogue<RT>(p, mi, row0, ttile, nthreads, wave_sum);
        } else {
            // Several splits of the row: this one's sums to the workspace,
            // [tile][token tile][split][RT * 1024]; skinny_reduce finishes.
            float *dst =
                p.partials + (static_cast<size_t>(tile * gridDim.y + ttile) * p.splits + split) * (RT * 1024);
            for (int e = threadIdx.x; e < RT * 1024; e += nthreads) dst[e] = wave_sum(e);
        }
        if constexpr (!LOOP) return;
        tile += stride;
        if (tile >= p.tiles) return;
        __syncthreads();   // every wave's sums read before the next tile's overwrite them
    }
}

template <int TYPE, int RT>
__global__ __launch_bounds__(64 * waves_max(TYPE, RT)) void skinny_i8(SkParams p) {
    extern __shared__ __align__(16) float lds[];
    if constexpr (TYPE != 0) {
        skinny_body<TYPE, RT, false>(p, lds);
    } else {
        // A launch over matrices of several types (one row tile each): the
        // tile's matrix fixes the type, uniformly for the workgroup.
        const int type = p.mat[tile_matrix(p, static_cast<int>(blockIdx.x) / p.splits)].type;
        if (type == QK_TYPE_Q4_K)
            skinny_body<QK_TYPE_Q4_K, RT, false>(p, lds);
        else if (type == QK_TYPE_Q6_K)
            skinny_body<QK_TYPE_Q6_K, RT, false>(p, lds);
        else
            skinny_body<QK_TYPE_Q6_K_SPLIT, RT, false>(p, lds);
    }
}

// Workgroups of the looping kernel hold at most kLoopWaves waves (room for
// two tiles' weights in registers).
constexpr int kLoopWaves = 8;

// Rows of at most kRowsMaxBlocks blocks, one row tile per wave: the token
// tile's activation codes, their transposed scales and (Q4_K) the S-scale
// products of every block sit in LDS, written once per workgroup; each wave
// then walks its own row tiles block by block, the next block's weights in
// flight, with no cross-wave reduction and no barrier in the loop.
constexpr int kRowsMaxBlocks = 12;
// A token's 256 codes of a block take 272 bytes of LDS: the lanes of a
// half-wave (32 tokens) then start 4 banks apart instead of all in one bank.
constexpr int kCodeStride = 272;

__host__ __device__ constexpr size_t rows_lds(int nb) {
    return static_cast<size_t>(nb) * (kToks * kCodeStride + 2 * 8 * kToks * sizeof(float));
}

template <int TYPE>
__device__ __forceinline__ void rows_body(const SkParams &p, float *lds) {
    const int nb = p.nb;
    uint8_t *codes = reinterpret_cast<uint8_t *>(lds);   // [nb][32 tokens][kCodeStride]
    float *xst = reinterpret_cast<float *>(codes + static_cast<size_t>(nb) * kToks * kCodeStride);   // [nb][8][32]
    float *xsl = xst + nb * 8 * kToks;                                       // [nb][8][32] xscale * S
    const int ttile = blockIdx.y;
    const int nthreads = blockDim.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kh = lane >> 5, col = lane & 31;
    const int waves = nthreads >> 6;
    const int stride = gridDim.x * waves;
    const int first = blockIdx.x * waves + wave;
    const bool has_tiles = first < p.tiles;   // wave-uniform
    const int first_c = min(first, p.tiles - 1);
    const int n_tiles = has_tiles ? (p.tiles - 1 - first) / stride + 1 : 1;
    const int steps = n_tiles * nb;
    auto tile_of = [&](int k) { return first_c + min(k, steps - 1) / nb * stride; };
    auto block_of = [&](int k) { return min(k, steps - 1) % nb; };
    // The first two blocks' weights load while the activations are staged
    // (a wave without tiles loads its clamped tile and discards it).
    Raw w0[1], w1[1];
    load_tile<TYPE, 1>(p, tile_of(0), block_of(0), col, kh, w0);
    load_tile<TYPE, 1>(p, tile_of(1), block_of(1), col, kh, w1);

    for (int i = threadIdx.x; i < nb * kToks * 16; i += nthreads) {   // 16-byte chunks
        const int chunk = i & 15, tok = (i >> 4) & (kToks - 1), b = i >> 9;
        const int t = min(ttile * kToks + tok, p.n_tokens - 1);
        *reinterpret_cast<uint4 *>(codes + (b * kToks + tok) * kCodeStride + chunk * 16) =
            *reinterpret_cast<const uint4 *>(p.xq + static_cast<int64_t>(t) * p.ldxq + b * 256 + chunk * 16);
    }
    for (int i = threadIdx.x; i < nb * 8 * kToks; i += nthreads) {
        const int tok = i & (kToks - 1), sb = i >> 5;   // sb = b * 8 + sub-block
        const int t = min(ttile * kToks + tok, p.n_tokens - 1);
        xst[i] = p.xs[static_cast<int64_t>(t) * p.ldxs + sb];
    }
    __syncthreads();
    if (TYPE == QK_TYPE_Q4_K) {
        for (int i = threadIdx.x; i < nb * 8 * kToks; i += nthreads) {
            const int tok = i & (kToks - 1), sb = i >> 5, b = sb >> 3, sub = sb & 7;
            const uint4 *c = reinterpret_cast<const uint4 *>(codes + (b * kToks + tok) * kCodeStride + sub * 32);
            int sum = 0;
            #pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint4 v = c[h];
                sum = __builtin_amdgcn_sdot4(static_cast<int>(v.x), 0x01010101, sum, false);
                sum = __builtin_amdgcn_sdot4(static_cast<int>(v.y), 0x01010101, sum, false);
                sum = __builtin_amdgcn_sdot4(static_cast<int>(v.z), 0x01010101, sum, false);
                sum = __builtin_amdgcn_sdot4(static_cast<int>(v.w), 0x01010101, sum, false);
            }
            xsl[i] = static_cast<float>(sum) * xst[i];
        }
        __syncthreads();
    }
    if (!has_tiles) return;   // no barrier follows

    v16f acc[1], accmin[1];
    #pragma unroll
    for (int i = 0; i < 16; ++i) acc[0][i] = accmin[0][i] = 0.f;
    // Two blocks ahead: step k computes w0 while w1 (step k + 1) and w2
    // (step k + 2, issued now) are in flight; the last steps reload their
    // own block, in bounds.
    for (int k = 0; k < steps; ++k) {
        const int b = k % nb;
        Raw w2[1];
        load_tile<TYPE, 1>(p, tile_of(k + 2), block_of(k + 2), col, kh, w2);
        uint4 ca[8];
        const uint8_t *cb = codes + (b * kToks + col) * kCodeStride;
        #pragma unroll
        for (int sub = 0; sub < 8; ++sub) {
            if (is_q4<TYPE>(TYPE)) {
                ca[sub] = *reinterpret_cast<const uint4 *>(cb + 32 * sub + 16 * kh);
            } else {
                const uint2 lo = *reinterpret_cast<const uint2 *>(cb + 32 * sub + 8 * kh);
                const uint2 hi = *reinterpret_cast<const uint2 *>(cb + 32 * sub + 16 + 8 * kh);
                ca[sub] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
        }
        float xss[8];
        #pragma unroll
        for (int sub = 0; sub < 8; ++sub) xss[sub] = is_q4<TYPE>(TYPE) ? xsl[(b * 8 + sub) * kToks + col] : 0.f;
        block_i8<TYPE>(w0[0], TYPE, ca, xst + b * 8 * kToks, xss, kh, acc[0], accmin[0]);
        own_regs(w1[0]);
        w0[0] = w1[0];
        w1[0] = w2[0];
        if (b == nb - 1) {   // wave-uniform: the tile is done
            int mi[1], row0[1];
            tile_rows<1>(p, tile_of(k), mi, row0);
            const SkMatrix &M = p.mat[mi[0]];
            const int row = row0[0] + col;
            #pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = ttile * kToks + 8 * (i >> 2) + 4 * kh + (i & 3);
                if (row < M.rows && t < p.n_tokens) {
                    float *y = M.y + static_cast<int64_t>(t) * M.ldy + row;
                    float v = acc[0][i] + accmin[0][i];
                    if (p.epilogue == kAccumulate) v += *y;
                    *y = v;
                }
                acc[0][i] = accmin[0][i] = 0.f;
            }
        }
    }
}

template <int TYPE>
__global__ __launch_bounds__(64 * kLoopWaves) void skinny_i8_rows(SkParams p) {
    extern __shared__ __align__(16) float lds[];
    rows_body<TYPE>(p, lds);
}

// Launches of more (row tile, token tile) units than the chip holds at
// once, over matrices of one type: resident workgroups walk the row tiles.
template <int TYPE, int RT>
__global__ __launch_bounds__(64 * kLoopWaves) void skinny_i8_loop(SkParams p) {
    extern __shared__ __align__(16) float lds[];
    skinny_body<TYPE, RT, true>(p, lds);
}

constexpr int kSplitsMax = 8;

// The splits' sums of one (row tile, token tile), added in split order
// (deterministic) with every split's load issued first, then the epilogue.
template <int RT>
__global__ __launch_bounds__(256) void skinny_reduce(SkParams p) {
    const int tile = blockIdx.x, ttile = blockIdx.y;
    int mi[RT], row0[RT];
    tile_rows<RT>(p, tile, mi, row0);
    const float *src = p.partials + static_cast<size_t>(tile * gridDim.y + ttile) * p.splits * (RT * 1024);
    epilogue<RT>(p, mi, row0, ttile, 256, [&](int e) {
        float v[kSplitsMax];
        #pragma unroll
        for (int s = 0; s < kSplitsMax; ++s) v[s] = s < p.splits ? src[static_cast<size_t>(s) * RT * 1024 + e] : 0.f;
        float sum = v[0];
        #pragma unroll
        for (int s = 1; s < kSplitsMax; ++s)
            if (s < p.splits) sum += v[s];
        return sum;
    });
}

// float4 of a row one thread holds in skinny_reduce_norm: rows of at most
// 4 * 256 * kNormHeld values.
constexpr int kNormHeld = 4;

// One 256-thread workgroup per token of a one-matrix accumulating launch:
// each output of the token's row is skinny_reduce's split sum plus the
// residual (the same additions in the same order), stored to y, and the row
// is then normalised and quantized as rmsnorm_quantize_kernel does (thread
// t holds float4 t, t + 256, ...; the same sum of squares, scale, codes and
// scales), so the next projection's input needs no launch of its own.
__global__ __launch_bounds__(256) void skinny_reduce_norm(SkParams p, int token_tiles, SkNorm nq) {
    __shared__ float scratch[4];
    const SkMatrix &M = p.mat[0];
    const int t = blockIdx.x;
    const int ttile = t / kToks, tl = t - ttile * kToks;
    const int n4 = M.rows >> 2;
    // Element of token tl and row r within its tile's partial sums (the
    // epilogue's index map inverted).
    const int ebase = (4 * (tl >> 3) + (tl & 3)) * 64 + 32 * ((tl >> 2) & 1);
    float *y = M.y + static_cast<int64_t>(t) * M.ldy;
    float4 v[kNormHeld];
    float ss = 0.f;
    #pragma unroll
    for (int k = 0; k < kNormHeld; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i >= n4) continue;
        // Rows 4i .. 4i + 3 lie in one row tile, at consecutive elements.
        const int tile = 4 * i / kRows;
        const float4 *src = reinterpret_cast<const float4 *>(
            p.partials + static_cast<size_t>(tile * token_tiles + ttile) * p.splits * 1024 + ebase + 4 * i -
            tile * kRows);
        float4 sum = src[0];
        #pragma unroll
        for (int sp = 1; sp < kSplitsMax; ++sp) {
            if (sp < p.splits) {
                const float4 t = src[static_cast<size_t>(sp) * 256];
                sum.x += t.x;
                sum.y += t.y;
                sum.z += t.z;
                sum.w += t.w;
            }
        }
        const float4 old = reinterpret_cast<const float4 *>(y)[i];
        v[k] = make_float4(sum.x + old.x, sum.y + old.y, sum.z + old.z, sum.w + old.w);
        reinterpret_cast<float4 *>(y)[i] = v[k];
        ss = fmaf(v[k].x, v[k].x, ss);
        ss = fmaf(v[k].y, v[k].y, ss);
        ss = fmaf(v[k].z, v[k].z, ss);
        ss = fmaf(v[k].w, v[k].w, ss);
    }
    ss = block_sum256(ss, scratch);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(M.rows) + nq.eps);
    const float4 *w4 = reinterpret_cast<const float4 *>(nq.w);
    uint32_t *q4 = reinterpret_cast<uint32_t *>(nq.xq + static_cast<int64_t>(t) * nq.ldxq);
    float *st = nq.xs + static_cast<int64_t>(t) * nq.ldxs;
    #pragma unroll
    for (int k = 0; k < kNormHeld; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i >= n4) continue;   // n4 is a multiple of 8: groups stay whole
        const float4 w = w4[i];
        quantize_quad_store(make_float4(v[k].x * scale * w.x, v[k].y * scale * w.y, v[k].z * scale * w.z,
                                        v[k].w * scale * w.w),
                            (i & 7) == 0, q4 + i, st + (i >> 3));
    }
}

template <int RT, bool LOOP>
const void *kernel_of(int type) {
    if constexpr (LOOP) {
        return type == QK_TYPE_Q4_K   ? reinterpret_cast<const void *>(skinny_i8_loop<QK_TYPE_Q4_K, RT>)
               : type == QK_TYPE_Q6_K ? reinterpret_cast<const void *>(skinny_i8_loop<QK_TYPE_Q6_K, RT>)
                                      : reinterpret_cast<const void *>(skinny_i8_loop<QK_TYPE_Q6_K_SPLIT, RT>);
    } else {
        if (type == 0) {
            if constexpr (RT == 1) return reinterpret_cast<const void *>(skinny_i8<0, 1>);
            return nullptr;
        }
        return type == QK_TYPE_Q4_K   ? reinterpret_cast<const void *>(skinny_i8<QK_TYPE_Q4_K, RT>)
               : type == QK_TYPE_Q6_K ? reinterpret_cast<const void *>(skinny_i8<QK_TYPE_Q6_K, RT>)
                                      : reinterpret_cast<const void *>(skinny_i8<QK_TYPE_Q6_K_SPLIT, RT>);
    }
}

// The kernel of a launch: type 0 (several types) has only the one-pass form.
const void *skinny_kernel(int type, int rt, bool loop) {
    if (rt == 2) return loop ? kernel_of<2, true>(type) : kernel_of<2, false>(type);
    return loop ? kernel_of<1, true>(type) : kernel_of<1, false>(type);
}

// LDS of a workgroup of `waves` waves: the waves' sums, then each wave's
// activation transpose.
size_t skinny_lds(int waves, int rt) {
    return (static_cast<size_t>(waves) * rt * 1024 + static_cast<size_t>(waves) * 8 * kToks) * sizeof(float);
}

// Splits beyond the fewest a row needs are planned only while the split
// sums of a launch stay within this many (row tile, token tile, split)
// units, which bounds the workspace.
constexpr int64_t kPartialUnitsMax = 2048;

// Duration model of a plan, fitted to 3B-shaped launches: each round of
// resident workgroups costs about kRoundUs plus kWaveUs per wave a SIMD
// runs in it (one block of RT row tiles each), and the second launch that
// adds split sums about kReduceUs.
constexpr float kRoundUs = 10.f, kWaveUs = 1.f, kReduceUs = 4.7f;

int fewest_splits(int nb, int wmax) { return (nb + wmax - 1) / wmax; }

struct SkPlan {
    int splits, waves;
    int loop_groups;   // workgroups per (split, token tile) of the looping kernel; 0: one pass
    bool rows;         // the looping kernel is skinny_i8_rows (one row tile per wave, one split)
};

const void *rows_kernel(int type) {
    return type == QK_TYPE_Q4_K   ? reinterpret_cast<const void *>(skinny_i8_rows<QK_TYPE_Q4_K>)
           : type == QK_TYPE_Q6_K ? reinterpret_cast<const void *>(skinny_i8_rows<QK_TYPE_Q6_K>)
                                  : reinterpret_cast<const void *>(skinny_i8_rows<QK_TYPE_Q6_K_SPLIT>);
}

// Splits of a row of nb blocks (one block per wave, the blocks spread
// evenly over a workgroup's waves) for a launch of `units` (row tile, token
// tile) pairs on kernel (type, rt): the plan of least modelled duration,
// from the fewest splits the widest workgroup allows up to kSplitsMax.
// Wider workgroups hold fewer per CU, narrower ones need more splits.  A
// launch of one type whose best plan needs more than one round of
// workgroups instead runs the looping kernel: the fewest splits of
// kLoopWaves-wave workgroups, as many as the chip holds, each walking its
// share of the row tiles.
// fold: the caller folds its next RMSNorm into a split reduction, so a plan
// without splits pays for that separate launch too.
SkPlan split_plan(int nb, int64_t units, int64_t ttiles, int type, int rt, bool fold, bool deferred) {
    const int s0 = fewest_splits(nb, waves_max(type, rt));
    const int cus = std::max(1, device_info().cus);
    const void *kernel = skinny_kernel(type, rt, false);
    int splits = s0, waves = (nb + s0 - 1) / s0;
    int64_t best_rounds = 0;
    float best = 0.f;
    for (int s = s0; s <= std::min(nb, kSplitsMax); ++s) {
        const int w = (nb + s - 1) / s;
        if (s > s0 && w == (nb + s - 2) / (s - 1)) continue;   // as wide as the previous plan: only more waves idle
        const int64_t wgs = units * s;
        if (s > s0 && wgs > kPartialUnitsMax) break;
        const int per_cu = std::max(1, resident_blocks(kernel, 64 * w, skinny_lds(w, rt)) / cus);
        const int64_t rounds = (wgs + static_cast<int64_t>(cus) * per_cu - 1) / (static_cast<int64_t>(cus) * per_cu);
        const int load = static_cast<int>(std::min<int64_t>(per_cu, (wgs + cus - 1) / cus));   // busiest CU
        const float cost = static_cast<float>(rounds) * (kRoundUs + kWaveUs * rt * ((load * w + 3) / 4)) +
                           ((s > 1 && !deferred) || fold ? kReduceUs : 0.f);
        if (s == s0 || cost < best - 1e-3f) {
            best = cost;
            best_rounds = rounds;
            splits = s;
            waves = w;
        }
    }
    if (type == 0 || best_rounds <= 1) return SkPlan{splits, waves, 0, false};
    const int64_t tiles = units / ttiles;
    if (rt == 1 && nb <= kRowsMaxBlocks) {
        // Row tiles per wave: as many 8-wave workgroups per token tile as the
        // chip holds (one per CU with the activations' LDS).
        const int resident = resident_blocks(rows_kernel(type), 64 * kLoopWaves, rows_lds(nb));
        const int64_t per_tt = std::max<int64_t>(1, resident / ttiles);
        const int64_t need = (tiles + kLoopWaves - 1) / kLoopWaves;
        return SkPlan{1, kLoopWaves, static_cast<int>(std::min(per_tt, need)), true};
    }
    SkPlan lp;
    lp.splits = fewest_splits(nb, kLoopWaves);
    lp.waves = (nb + lp.splits - 1) / lp.splits;
    const int resident = resident_blocks(skinny_kernel(type, rt, true), 64 * lp.waves, skinny_lds(lp.waves, rt));
    lp.rows = false;
    lp.loop_groups =
        static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(tiles, resident / (lp.splits * ttiles))));
    return lp;
}

int row_tiles(const qk_matrix *mats, int n_mats, bool pair) {
    if (pair) return mats[0].rows / kRows;
    int t = 0;
    for (int i = 0; i < n_mats; ++i) t += (mats[i].rows + kRows - 1) / kRows;
    return t;
}

}  // namespace

// Workspace bound of a launch, for any storage type: the split sums of
// the fewest splits of the narrowest workgroups (the looping kernel's), or
// of the planner's extra splits (at most kPartialUnitsMax units).
size_t skinny_i8_workspace_bytes(int cols, int tiles, int n_tokens, bool pair) {
    const int nb = cols / 256;
    if (nb <= 1 || n_tokens <= 0 || tiles <= 0) return 0;
    const int64_t units = static_cast<int64_t>(tiles) * ((n_tokens + kToks - 1) / kToks);
    const int s0 = fewest_splits(nb, kLoopWaves);
    const int64_t sums = std::max<int64_t>(s0 > 1 ? units * s0 : 0,
                                           std::min<int64_t>(units * std::min(nb, kSplitsMax), kPartialUnitsMax));
    return static_cast<size_t>(sums) * (pair ? 2 : 1) * 1024 * sizeof(float);
}

// The INT8 product of n_tokens per-32 quantized activation rows with
// n_mats matrices (arguments validated by the caller): y_m[t][r] (overwrite
// or add), or with out_xq the pair's SiLU(y0) * y1 quantized per 32 values
// (y unused; the two matrices of one type, rows equal and a multiple of 32).
// Rows of more blocks than a workgroup's waves are split over workgroups, whose sums
// a second launch adds (workspace: skinny_i8_workspace_bytes).
int launch_skinny_i8(const qk_matrix *mats, int n_mats, const int *ldy, const int8_t *xq, int ldxq,
                     const float *xscale, int ldscale, int cols, int n_tokens, int accumulate, int8_t *out_xq,
                     float *out_xs, int out_ldxq, int out_ldxs, void *workspace, size_t workspace_size,
                     hipStream_t stream, const char *where, const SkNorm *norm, SkDeferred *defer) {
    const int nb = cols / 256;
    if (norm && norm->done) *norm->done = 0;
    if (defer) defer->splits = 0;
    SkParams p{};
    p.n_mats = n_mats;
    p.xq = xq;
    p.xs = xscale;
    p.ldxq = ldxq;
    p.ldxs = ldscale;
    p.n_tokens = n_tokens;
    p.nb = nb;
    if (nb > kSplitsMax * 12)
        return fail(QK_ERR_LIMIT, std::string(where) + ": rows longer than 24576 columns are not supported");
    const bool pair = out_xq != nullptr;
    p.epilogue = pair ? kPairQuant : accumulate ? kAccumulate : kStore;
    p.out_xq = out_xq;
    p.out_xs = out_xs;
    p.out_ldxq = out_ldxq;
    p.out_ldxs = out_ldxs;
    if (pair && (n_mats != 2 || mats[0].rows != mats[1].rows || mats[0].rows % kRows || mats[0].type != mats[1].type))
        return fail(QK_ERR_INVALID_ARG, std::string(where) + ": a gate / up pair needs two matrices of one type "
                                                             "and equal rows, a multiple of 32");
    int tiles = 0, type = mats[0].type;
    for (int i = 0; i < n_mats; ++i) {
        SkMatrix &M = p.mat[i];
        M.w = static_cast<const uint8_t *>(mats[i].w);
        M.y = mats[i].y;
        M.rows = mats[i].rows;
        M.type = mats[i].type;
        M.row_bytes = static_cast<int>(row_bytes(M.type, nb));
        M.ldy = ldy ? ldy[i] : mats[i].rows;
        M.tile_begin = tiles;
        tiles += (M.rows + kRows - 1) / kRows;
        if (M.type != type) type = 0;
    }
    if (pair) tiles = mats[0].rows / kRows;
    const int token_tiles = (n_tokens + kToks - 1) / kToks;
    if (token_tiles > 65535 || static_cast<int64_t>(tiles) * kSplitsMax > (1 << 30))
        return fail(QK_ERR_LIMIT, std::string(where) + ": launch too large");
    const int rt = pair ? 2 : 1;
    const bool fold = norm && !pair && n_mats == 1 && accumulate && mats[0].rows % 32 == 0 &&
                      mats[0].rows <= 4 * 256 * kNormHeld && (ldy ? ldy[0] : mats[0].rows) % 4 == 0 &&
                      aligned(mats[0].y, 16) && norm->w && norm->xq && norm->xs && norm->ldxq % 4 == 0 &&
                      aligned(norm->xq, 4) && aligned(norm->w, 16);
    const bool deferrable = defer && !pair && !accumulate && !norm && n_mats <= QK_MAX_FUSED;
    const SkPlan plan =
        split_plan(nb, static_cast<int64_t>(tiles) * token_tiles, token_tiles, type, rt, fold, deferrable);
    p.splits = plan.splits;
    p.waves = plan.waves;
    p.tiles = tiles;
    // The plan's split sums; callers size the workspace by
    // skinny_i8_workspace_bytes, which bounds every plan.
    const size_t need = p.splits > 1 ? static_cast<size_t>(tiles) * token_tiles * p.splits * rt * 1024 * sizeof(float)
                                     : 0;
    if (need) {
        if (!workspace || workspace_size < need)
            return fail(QK_ERR_INVALID_ARG, std::string(where) + ": workspace smaller than " + std::to_string(need) +
                                                " bytes");
        if (!aligned(workspace, 16)) return fail(QK_ERR_ALIGN, std::string(where) + ": workspace not 16-byte aligned");
        p.partials = static_cast<float *>(workspace);
    }
    const size_t lds = plan.rows ? rows_lds(nb) : skinny_lds(p.waves, rt);
    const int groups = plan.loop_groups ? plan.loop_groups : tiles;   // workgroups per (split, token tile)
    void *args[] = {&p};
    if (hipLaunchKernel(plan.rows ? rows_kernel(type) : skinny_kernel(type, rt, plan.loop_groups > 0),
                        dim3(static_cast<unsigned>(groups * p.splits), static_cast<unsigned>(token_tiles)),
                        dim3(64 * p.waves), args, lds, stream) != hipSuccess)
        return launch_status(where);
    if (p.splits > 1 && deferrable && !plan.rows && !plan.loop_groups) {
        // The consumer adds the split sums (skinny_reduce's order).
        defer->partials = p.partials;
        defer->splits = p.splits;
        defer->token_tiles = token_tiles;
        for (int i = 0; i < n_mats; ++i) defer->tile_begin[i] = p.mat[i].tile_begin;
    } else if (p.splits > 1 && fold && !norm->plan_only) {
        hipLaunchKernelGGL(skinny_reduce_norm, dim3(static_cast<unsigned>(n_tokens)), dim3(256), 0, stream, p,
                           token_tiles, *norm);
        if (norm->done) *norm->done = 1;
    } else if (p.splits > 1) {
        const dim3 rgrid(static_cast<unsigned>(tiles), static_cast<unsigned>(token_tiles));
        if (pair)
            hipLaunchKernelGGL(skinny_reduce<2>, rgrid, dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL(skinny_reduce<1>, rgrid, dim3(256), 0, stream, p);
    }
    return launch_status(where);
}

}  // namespace qk

namespace {

// Shared checks of the INT8 multi-token entry points: quantized rows of
// cols values at xq + t*ldxq (16-byte aligned), scales at xscale + t*ldscale.
int check_i8_input(const char *where, const int8_t *xq, int ldxq, const float *xscale, int ldscale, int cols,
                   int n_tokens) {
    if (!xq || !xscale || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, std::string(where) + ": null activation pointer or negative token count");
    if (ldxq < cols || ldscale < cols / 32)
        return qk::fail(QK_ERR_INVALID_ARG, std::string(where) + ": leading dimension smaller than the row");
    if (!qk::aligned(xq, 16) || ldxq % 16 || !qk::aligned(xscale, 4))
        return qk::fail(QK_ERR_ALIGN, std::string(where) + ": xq and ldxq must keep 16-byte alignment, xscale 4");
    return QK_OK;
}

constexpr int kMatrixCoreTokens = 8;   // from here on the matrix cores take the product

size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// Workspace of the INT8 FFN: SiLU(gate) * up quantized (hidden bytes and
// hidden / 32 scales per token, each array 256-byte aligned), then the
// split sums of the two products (the larger); below kMatrixCoreTokens the
// fp32 gate and up outputs of the GEMV form instead.
size_t ffn_i8_bytes(int dim, int hidden, int n_tokens) {
    const size_t t = static_cast<size_t>(n_tokens);
    const size_t h = al256(t * hidden) + al256(t * (hidden / 32) * sizeof(float));
    if (n_tokens < kMatrixCoreTokens) return h + 2 * al256(t * hidden * sizeof(float));
    return h + std::max(qk::skinny_i8_workspace_bytes(dim, hidden / 32, n_tokens, true),
                        qk::skinny_i8_workspace_bytes(hidden, (dim + 31) / 32, n_tokens, false));
}

}  // namespace

extern "C" {

size_t qk_gemv_batched_i8_workspace_bytes(int cols, int rows, int n_tokens) {
    if (cols <= 0 || cols % 256 || rows <= 0 || n_tokens < kMatrixCoreTokens) return 0;
    // Any split of rows over up to QK_MAX_FUSED matrices has at most
    // rows / 32 + QK_MAX_FUSED row tiles.
    return qk::skinny_i8_workspace_bytes(cols, rows / 32 + QK_MAX_FUSED, n_tokens, false);
}

int qk_gemv_batched_i8(int type, const void *w, const int8_t *xq, int ldxq, const float *xscale, int ldscale,
                       float *y, int ldy, int cols, int rows, int n_tokens, void *workspace, size_t workspace_bytes,
                       qk_stream stream) {
    const char *where = "qk_gemv_batched_i8";
    int st = qk::check_weights(where, type, w, cols, rows);
    if (st || (st = check_i8_input(where, xq, ldxq, xscale, ldscale, cols, n_tokens))) return st;
    if (!y || ldy < rows) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_batched_i8: null y or ldy smaller than rows");
    if (!qk::aligned(y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_gemv_batched_i8: y must be 4-byte aligned");
    if (n_tokens == 0) return qk::ok();
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const qk_matrix m{type, rows, w, y};
    if (n_tokens < kMatrixCoreTokens) return qk::launch_gemv_i8(&m, 1, xq, ldxq, xscale, ldscale, cols, n_tokens, &ldy, 0, s);
    return qk::launch_skinny_i8(&m, 1, &ldy, xq, ldxq, xscale, ldscale, cols, n_tokens, 0, nullptr, nullptr, 0, 0,
                                workspace, workspace_bytes, s, where);
}

int qk_gemv_multi_batched_i8(const qk_matrix *mats, int n_mats, const int8_t *xq, int ldxq, const float *xscale,
                             int ldscale, int cols, int n_tokens, void *workspace, size_t workspace_bytes,
                             qk_stream stream) {
    const char *where = "qk_gemv_multi_batched_i8";
    if (!mats || n_mats < 1 || n_mats > QK_MAX_FUSED)
        return qk::fail(QK_ERR_INVALID_ARG, std::string(where) + ": need 1.." + std::to_string(QK_MAX_FUSED) +
                                                " matrices");
    int st = check_i8_input(where, xq, ldxq, xscale, ldscale, cols, n_tokens);
    if (st) return st;
    int ldy[QK_MAX_FUSED];
    for (int m = 0; m < n_mats; ++m) {
        if ((st = qk::check_weights(where, mats[m].type, mats[m].w, cols, mats[m].rows))) return st;
        if (!mats[m].y) return qk::fail(QK_ERR_INVALID_ARG, std::string(where) + ": null output pointer");
        if (!qk::aligned(mats[m].y, 4)) return qk::fail(QK_ERR_ALIGN, std::string(where) + ": misaligned output");
        ldy[m] = mats[m].rows;
    }
    if (n_tokens == 0) return qk::ok();
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_tokens < kMatrixCoreTokens)
        return qk::launch_gemv_i8(mats, n_mats, xq, ldxq, xscale, ldscale, cols, n_tokens, ldy, 0, s);
    return qk::launch_skinny_i8(mats, n_mats, ldy, xq, ldxq, xscale, ldscale, cols, n_tokens, 0, nullptr, nullptr, 0,
                                0, workspace, workspace_bytes, s, where);
}

size_t qk_ffn_batched_i8_workspace_bytes(int dim, int hidden, int n_tokens) {
    if (dim <= 0 || dim % 256 || hidden <= 0 || hidden % 256 || n_tokens <= 0) return 0;
    // Enough for any token count up to n_tokens: each form's need grows
    // with the count, so the larger of the two forms' needs covers both.
    return std::max(ffn_i8_bytes(dim, hidden, n_tokens),
                    ffn_i8_bytes(dim, hidden, std::min(n_tokens, kMatrixCoreTokens - 1)));
}

int qk_ffn_batched_i8(int gate_type, const void *gate, int up_type, const void *up, int down_type, const void *down,
                      const int8_t *xq, int ldxq, const float *xscale, int ldscale, float *y, int ldy, int dim,
                      int hidden, int n_tokens, int accumulate, void *workspace, size_t workspace_bytes,
                      qk_stream stream) {
    const char *where = "qk_ffn_batched_i8";
    int st;
    if ((st = qk::check_weights(where, gate_type, gate, dim, hidden)) ||
        (st = qk::check_weights(where, up_type, up, dim, hidden)) ||
        (st = qk::check_weights(where, down_type, down, hidden, dim)) ||
        (st = check_i8_input(where, xq, ldxq, xscale, ldscale, dim, n_tokens)))
        return st;
    if (gate_type != up_type)
        return qk::fail(QK_ERR_TYPE, "qk_ffn_batched_i8: gate and up must have one storage type");
    if (!y || ldy < dim) return qk::fail(QK_ERR_INVALID_ARG, "qk_ffn_batched_i8: null y or ldy smaller than dim");
    if (!qk::aligned(y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_ffn_batched_i8: y must be 4-byte aligned");
    if (n_tokens == 0) return qk::ok();
    const size_t need = ffn_i8_bytes(dim, hidden, n_tokens);
    if (!workspace || workspace_bytes < need)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_ffn_batched_i8: workspace smaller than " + std::to_string(need) +
                                                " bytes (qk_ffn_batched_i8_workspace_bytes)");
    if (!qk::aligned(workspace, 256)) return qk::fail(QK_ERR_ALIGN, "qk_ffn_batched_i8: workspace not 256-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t T = static_cast<size_t>(n_tokens);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    int8_t *hq = reinterpret_cast<int8_t *>(ws);
    float *hs = reinterpret_cast<float *>(ws + al256(T * hidden));
    uint8_t *rest = ws + al256(T * hidden) + al256(T * (hidden / 32) * sizeof(float));
    const size_t rest_bytes = workspace_bytes - (rest - ws);
    const qk_matrix dm{down_type, dim, down, y};
    if (n_tokens < kMatrixCoreTokens) {
        // The GEMV form: gate and up in fp32, SiLU * up quantized, down.
        float *g = reinterpret_cast<float *>(rest);
        float *u = g + al256(T * hidden * sizeof(float)) / sizeof(float);
        const qk_matrix gu[2] = {{gate_type, hidden, gate, g}, {up_type, hidden, up, u}};
        const int ldg[2] = {hidden, hidden};
        if ((st = qk::launch_gemv_i8(gu, 2, xq, ldxq, xscale, ldscale, dim, n_tokens, ldg, 0, s)) ||
            (st = qk::launch_silu_mul_quantize(g, u, hq, hs, n_tokens * hidden, s)))
            return st;
        return qk::launch_gemv_i8(&dm, 1, hq, hidden, hs, hidden / 32, hidden, n_tokens, &ldy, accumulate != 0, s);
    }
    const qk_matrix gu[2] = {{gate_type, hidden, gate, nullptr}, {up_type, hidden, up, nullptr}};
    if ((st = qk::launch_skinny_i8(gu, 2, nullptr, xq, ldxq, xscale, ldscale, dim, n_tokens, 0, hq, hs, hidden,
                                   hidden / 32, rest, rest_bytes, s, where)))
        return st;
    return qk::launch_skinny_i8(&dm, 1, &ldy, hq, hidden, hs, hidden / 32, hidden, n_tokens, accumulate != 0, nullptr,
                                nullptr, 0, 0, rest, rest_bytes, s, where);
}

}  // extern "C"
