// qk_gemv.hip - Q4_K / Q6_K dequant-GEMV on gfx950: the FP32 path and the
// INT8-activation path, batch 1 and few-token.
//
// Replaces gemv_quant<12|14> (inferencer.cu:645-661), qkv_cuda
// (inferencer.cu:753-784), gate_up_cuda (inferencer.cu:786-804), and the
// INT8 kernels gemv_q4_dp4a / gemv_q6_dp4a / gemv_batch_dp4a
// (inferencer.cu:558-569, 663-699).
//
// Work decomposition (wave64):
//   A row of nb super-blocks is P = 4*nb pieces of 64 weights (layout in
//   qk_internal.h).  A "tile" is TR = 64/gcd(P,64) consecutive rows, i.e.
//   TR*P (row, piece) pairs, a multiple of 64, split into C = P/gcd(P,64)
//   chunks of 64.  Wave w of a wave-group owns chunk w for every tile, so each
//   lane owns one fixed (row-in-tile, piece) and keeps that piece's 64
//   activations in VGPRs for the whole launch: x is read once per wave, never
//   per row.  Weights stream as 16-byte loads; each lane unpacks nibbles /
//   6-bit codes in registers.
//     FP32: per part (16 columns of one sub-block) S = sum code*x, then
//       Q4_K: d * sum_p sc_p*S_p - dmin * sum_p m_p*X_p
//       Q6_K: d * sum_p sc_p*(S_p - 32*X_p)
//       with X_p the lane's activation sums: the reference's per-weight
//       d*sc*q - dmin*m reassociated (tolerance-graded, rel-L2 1e-5).
//     INT8: the part dots are exact v_dot4_i32_i8 sums; the float combine
//       (d*sc*dot - dmin*m*sum)*xscale (Q4_K) or d*sc*dot*xscale (Q6_K) of
//       inferencer.cu:541, 642 runs per 16-column half of each sub-block.
//   Lanes of one row form aligned groups of gcd(P,64) lanes reduced with xor
//   shuffles.  When C > 1 the group sums of a tile meet in LDS and lane t of
//   the first wave adds row t's C sums in a fixed order (deterministic).
//   The grid (at most two workgroups per CU) walks tiles grid-stride; a tile's loads are issued
//   before the previous tile's arithmetic, and the first two tiles' loads
//   before the activation staging.
//   blockIdx.y selects the token when several tokens share the weights.
#include "qk_internal.h"

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

namespace qk {
namespace {

constexpr int kMaxChunks = 16;
// Workgroups per CU of the grid-stride GEMV kernels.  Each workgroup stages
// the activations once, so a launch with few tiles per wave runs fewer
// workgroups; a long launch over 16-byte aligned weight fields runs more
// waves to keep more loads in flight (measured on MI355X, 1 token):
//   gemv_wave, 128256 x 2048 split Q6_K: 40.0 us at 2 / CU, 39.7 at 3,
//     38.8 at 4, 5 and 6 (the GGUF Q6_K layout, bound by its misaligned
//     field loads, slows to 41.3 us at 4); Q4_K 128256 x 2048: 30.5 us at 3,
//     30.1 at 4, 29.3 at 5 and 6; Q4_K gate/up 2 x 8192 x 2048 (a short
//     launch): 9.6 us at 2, 10.2 at 4.
//   gemv_split, split Q6_K 2048 x 8192: 9.6 us at 2 / CU, 8.6 at 1; Q4_K
//     3072 x 3072: 6.6 / 6.1; Q4_K 8192 x 3072: 8.7 / 10.1; split Q6_K
//     128256 x 3072 (3-wave workgroups, a long launch): 111 at 1, 72.8 at
//     2, 60.8 at 4, 62.4 at 6 and 8 (INT8: 81.9 at 2, 56.2 at 4, 58.2 at
//     6 and 8).
constexpr int kWaveBlocksPerCu = 2;
constexpr int kWaveBlocksPerCuLong = 5;
// The INT8 kernels' lighter arithmetic needs fewer waves per CU: Q4_K
// 128256 x 2048, 26.45 us at 4 / CU against 26.9 at 5 (the FP32 kernel 29.0
// at 4, 28.2 at 5).
constexpr int kWaveBlocksPerCuLongInt8 = 4;
constexpr int kWaveLongTiles = 16;      // tiles per wave at kWaveBlocksPerCu
constexpr int kSplitBlocksPerCu = 2;
constexpr int kSplitBlocksPerCuLong = 4;   // >= kWaveLongTiles tiles per wave-group at 2 / CU
constexpr int kSplitShortTiles = 3;     // tiles per wave-group at kSplitBlocksPerCu
// Activations staged per workgroup plus the split kernels' reduction slots.
constexpr size_t kMaxLds = 64 * 1024;

struct GemvMatrix {
    const uint8_t *w;
    float *y;
    int rows;
    int type;
    int tile_begin;
    int row_bytes;
    int ldy;
};

struct GemvParams {
    GemvMatrix mat[QK_MAX_FUSED];
    int n_mats;
    const void *x;        // fp32 activations, or int8 codes for the INT8 path
    const float *xscale;  // INT8 path: per-32 activation scales
    int ldx;              // elements between tokens
    int ldscale;
    int pieces;           // P
    int tile_rows;        // TR
    int chunks;           // C
    int group_lanes;      // gcd(P, 64)
    int total_tiles;
    // Decode-step fusions of the FP32 path (all off when zero):
    const float *norm_w;  // stage RMSNorm(x) * norm_w instead of x
    float norm_eps;
    const float *up;      // stage x / (1 + exp(-x)) * up instead of x
    int accumulate;       // y += W x instead of y = W x
    float *arg_v;         // greedy-token epilogue: per-workgroup best value / row
    int *arg_i;
    int *grid_out;        // host: receives the launch's workgroup count (not read on the device)
    // I8MergePolicy: the attention's unmerged split partials,
    // [head][n_parts][split_partial_floats(part_hd)], in place of x.
    const float *parts;
    int n_parts;
    int part_hd;
};

struct Raw {
    uint4 a, b, c;
    uint2 s;
    uint32_t d;
};

struct TileRef {
    const uint8_t *blk;   // the lane's block (GGUF layouts) or its row (split Q6_K)
    float *y;
    int row;
    int type;
    int b;                // block index within the row
    bool valid;
};

__device__ __forceinline__ TileRef locate(const GemvParams &p, int tile, int rit, int piece_block, int token) {
    int m = 0;
    #pragma unroll 1
    while (m + 1 < p.n_mats && tile >= p.mat[m + 1].tile_begin) ++m;
    const GemvMatrix &M = p.mat[m];
    TileRef t;
    t.row = (tile - M.tile_begin) * p.tile_rows + rit;
    t.valid = t.row < M.rows;
    const int row = t.valid ? t.row : M.rows - 1;   // keep loads in bounds
    t.type = M.type;
    t.b = piece_block;
    t.y = M.y + static_cast<int64_t>(token) * M.ldy;
    const int bpb = M.type == QK_TYPE_Q4_K ? 144 : M.type == QK_TYPE_Q6_K ? 210 : 0;
    t.blk = M.w + static_cast<size_t>(row) * M.row_bytes + static_cast<size_t>(piece_block) * bpb;
    return t;
}

// Q6_K codes 0..63 of the four parts, one byte each, for dword k.
__device__ __forceinline__ void q6k_codes(uint32_t la, uint32_t lb, uint32_t qh, uint32_t &c0, uint32_t &c1,
                                          uint32_t &c2, uint32_t &c3) {
    const uint32_t M = 0x0F0F0F0Fu, H = 0x30303030u;
    c0 = (la & M) | ((qh << 4) & H);
    c1 = (lb & M) | ((qh << 2) & H);
    c2 = ((la >> 4) & M) | (qh & H);
    c3 = ((lb >> 4) & M) | ((qh >> 2) & H);
}

// scales[g*8 + part*2 + h] as floats, from the 8 loaded scale bytes.
__device__ __forceinline__ void q6k_scales(const uint2 &s, int h, float *sc) {
    const uint32_t s0 = h ? (s.x >> 8) : s.x;
    const uint32_t s1 = h ? (s.y >> 8) : s.y;
    sc[0] = static_cast<float>(static_cast<int8_t>(s0 & 0xFFu));
    sc[1] = static_cast<float>(static_cast<int8_t>((s0 >> 16) & 0xFFu));
    sc[2] = static_cast<float>(static_cast<int8_t>(s1 & 0xFFu));
    sc[3] = static_cast<float>(static_cast<int8_t>((s1 >> 16) & 0xFFu));
}

// ------------------------------------------------------------ FP32 path --
//
// fp32 activations become exact integer work: each 16-column group of x is
// written as X = rint(x * 2^(21-e)) with e = ilogb(max|x| of the group), so
// |X| <= 2^22, then split into three signed bytes X = L2*65536 + L1*256 + L0
// (L0, L1 in [-128, 127], L2 in [-64, 64]).  A part's dot with 16 codes
// (0..63) is three exact v_dot4_i32_i8 sums, recombined in fp32 and scaled
// by 2^(e-21): 22 significant bits of every activation relative to its
// group maximum, i.e. a relative error of at most 2^-22 of the group's
// largest value per activation, far inside the 1e-5 rel-L2 budget, at a
// quarter of the VALU work of a convert + fma per weight.  Each workgroup
// prepares the groups of its token once in LDS (64 B per group); every lane
// then copies the four groups of its piece into registers.

extern __shared__ __align__(16) unsigned char qk_smem[];

// sum_i code_i * x_i of one part: codes are four dwords of byte codes 0..63.
// The L1 and L0 dots share one integer accumulator: for 16 codes below 64
// and limbs of at most 128 in magnitude, |256 * sum(c * L1) + sum(c * L0)|
// < 257 * 16 * 63 * 128 < 2^25, so it is exact, and its conversion rounds
// once, like fma(float(d1), 256, float(d0)).
__device__ __forceinline__ float limb_dot(const uint32_t *codes, const int *limb, float scale) {
    int d01 = 0, d2 = 0;
    #pragma unroll
    for (int k = 0; k < 4; ++k) {
        d01 = __builtin_amdgcn_sdot4(static_cast<int>(codes[k]), limb[4 + k], d01, false);
        d2 = __builtin_amdgcn_sdot4(static_cast<int>(codes[k]), limb[8 + k], d2, false);
    }
    d01 <<= 8;
    #pragma unroll
    for (int k = 0; k < 4; ++k) d01 = __builtin_amdgcn_sdot4(static_cast<int>(codes[k]), limb[k], d01, false);
    return fmaf(static_cast<float>(d2), 65536.f, static_cast<float>(d01)) * scale;
}

struct F32Policy {
    static constexpr bool kPrepLds = true;
    static constexpr bool kInt8 = false;
    static constexpr bool kDirect = true;   // load_direct exists (rows too long to stage)
    // Staging inputs loaded ahead of the weights (prep_early), or none.
    static constexpr bool kEarly = false;
    struct Early {};

    struct Lane {
        int limb[4][12];
        float scale[4];
        float X[4];
    };

    static constexpr bool kAccumulate = false;   // y += W x when p.accumulate
    static constexpr bool kArgmax = false;   // greedy-token epilogue

    // LDS bytes of the prepared activations of one token.
    __host__ __device__ static size_t lds_bytes(int cols) { return static_cast<size_t>(cols / 16) * sizeof(XGroup); }

    // Cooperative: the block writes every 16-column group of its token.
    __device__ static void prep(const GemvParams &p, int token, int cols, XGroup *lds) {
        const float *x = static_cast<const float *>(p.x) + static_cast<int64_t>(token) * p.ldx;
        for (int gi = threadIdx.x; gi < cols / 16; gi += blockDim.x) lds[gi] = make_group(x + gi * 16);
    }

    __device__ static void set_part(Lane &L, int part, const XGroup &gr) {
        #pragma unroll
        for (int i = 0; i < 12; ++i) L.limb[part][i] = gr.limb[i];
        L.scale[part] = gr.scale;
        L.X[part] = gr.sum;
    }

    // Group of part `part` of a piece: column b*256 + g*128 + part*32 + h*16.
    __device__ static int group_of(int piece, int part) {
        return 16 * (piece >> 2) + 8 * ((piece >> 1) & 1) + 2 * part + (piece & 1);
    }

    __device__ static void load(Lane &L, const GemvParams &, int, int piece, const XGroup *lds) {
        #pragma unroll
        for (int part = 0; part < 4; ++part) set_part(L, part, lds[group_of(piece, part)]);
    }

    // Without LDS (rows too long to stage): each lane builds its own groups.
    __device__ static void load_direct(Lane &L, const GemvParams &p, int token, int piece) {
        const float *x = static_cast<const float *>(p.x) + static_cast<int64_t>(token) * p.ldx;
        #pragma unroll
        for (int part = 0; part < 4; ++part) set_part(L, part, make_group(x + 16 * group_of(piece, part)));
    }

    __device__ static float q4k(const Raw &r, const Lane &L, int g) {
        const uint32_t M = 0x0F0F0F0Fu;
        const uint32_t c0[4] = {r.b.x & M, r.b.y & M, r.b.z & M, r.b.w & M};
        const uint32_t c1[4] = {(r.b.x >> 4) & M, (r.b.y >> 4) & M, (r.b.z >> 4) & M, (r.b.w >> 4) & M};
        const uint32_t c2[4] = {r.c.x & M, r.c.y & M, r.c.z & M, r.c.w & M};
        const uint32_t c3[4] = {(r.c.x >> 4) & M, (r.c.y >> 4) & M, (r.c.z >> 4) & M, (r.c.w >> 4) & M};
        const float S0 = limb_dot(c0, L.limb[0], L.scale[0]);
        const float S1 = limb_dot(c1, L.limb[1], L.scale[1]);
        const float S2 = limb_dot(c2, L.limb[2], L.scale[2]);
        const float S3 = limb_dot(c3, L.limb[3], L.scale[3]);
        uint32_t sc, mn;
        q4k_scale_min4(r.a, g, sc, mn);
        const float d = f16_bits_to_f32(r.a.x & 0xFFFFu);
        const float dmin = f16_bits_to_f32(r.a.x >> 16);
        float a = ubyte0(sc) * S0;
        a = fmaf(ubyte1(sc), S1, a);
        a = fmaf(ubyte2(sc), S2, a);
        a = fmaf(ubyte3(sc), S3, a);
        float b = ubyte0(mn) * L.X[0];
        b = fmaf(ubyte1(mn), L.X[1], b);
        b = fmaf(ubyte2(mn), L.X[2], b);
        b = fmaf(ubyte3(mn), L.X[3], b);
        return fmaf(d, a, -dmin * b);
    }

    __device__ static float q6k(const Raw &r, const Lane &L, int h) {
        const uint32_t la[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const uint32_t lb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t qh[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        uint32_t c[4][4];
        #pragma unroll
        for (int k = 0; k < 4; ++k) q6k_codes(la[k], lb[k], qh[k], c[0][k], c[1][k], c[2][k], c[3][k]);
        float sc[4];
        q6k_scales(r.s, h, sc);
        float a = 0.f;
        #pragma unroll
        for (int part = 0; part < 4; ++part)
            a = fmaf(sc[part], fmaf(-32.f, L.X[part], limb_dot(c[part], L.limb[part], L.scale[part])), a);
        return f16_bits_to_f32(r.d) * a;
    }
};

// The decode driver's fused staging: RMSNorm or SiLU * up applied while the
// activations are staged, and the residual add in the epilogue.  A policy
// of its own so the plain kernels carry none of it.
struct F32FusedPolicy : F32Policy {
    static constexpr bool kAccumulate = true;

    // LDS bytes of the prepared activations of one token, plus 64 bytes of
    // reduction scratch for the fused RMSNorm.
    __host__ __device__ static size_t lds_bytes(int cols) {
        return static_cast<size_t>(cols / 16) * sizeof(XGroup) + 64;
    }

    // Cooperative: the block writes every 16-column group of its token.
    // With norm_w the staged values are x * (1/sqrt(mean(x^2) + eps)) * w,
    // the arithmetic of rmsnorm_cuda (inferencer.cu:821-834); with up they
    // are x / (1 + exp(-x)) * up, that of silu_cuda (inferencer.cu:1053-1056).
    __device__ static void prep(const GemvParams &p, int token, int cols, XGroup *lds) {
        const float *x = static_cast<const float *>(p.x) + static_cast<int64_t>(token) * p.ldx;
        float scale = 1.f;
        if (p.norm_w) {
            float *scratch = reinterpret_cast<float *>(lds + cols / 16);
            const float4 *x4 = reinterpret_cast<const float4 *>(x);
            float ss = 0.f;
            #pragma unroll 4
            for (int i = threadIdx.x; i < cols / 4; i += blockDim.x) {
                const float4 v = x4[i];
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
            }
            #pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = ss;
            __syncthreads();
            ss = 0.f;
            for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) ss += scratch[w];
            scale = 1.0f / sqrtf(ss / static_cast<float>(cols) + p.norm_eps);
        }
        for (int gi = threadIdx.x; gi < cols / 16; gi += blockDim.x) {
            float v[16];
            load16f(x + gi * 16, v);
            if (p.norm_w) {
                float w[16];
                load16f(p.norm_w + gi * 16, w);
                #pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = v[i] * scale * w[i];
            }
            if (p.up) {
                float u[16];
                load16f(p.up + static_cast<int64_t>(token) * p.ldx + gi * 16, u);
                #pragma unroll
                for (int i = 0; i < 16; ++i) v[i] = v[i] / (1.f + expf(-v[i])) * u[i];
            }
            lds[gi] = make_group_regs(v);
        }
    }

};

// ------------------------------------------------------------ INT8 path --

// The LM head with the greedy pick: F32FusedPolicy's staging plus every
// wave's best (value, row) written at the end (arg_epilogue).  A policy of
// its own so the other fused GEMVs carry none of the bookkeeping.
struct F32ArgPolicy : F32FusedPolicy {
    static constexpr bool kArgmax = true;
};

struct I8Policy {
    static constexpr bool kPrepLds = false;
    static constexpr bool kInt8 = true;
    static constexpr bool kDirect = true;
    static constexpr bool kAccumulate = true;   // the INT8 step's residual adds
    static constexpr bool kArgmax = false;
    static constexpr bool kEarly = false;
    struct Early {};
    __host__ __device__ static size_t lds_bytes(int) { return 0; }
    __device__ static void prep(const GemvParams &, int, int, XGroup *) {}

    struct Lane {
        int xq[16];       // the piece's 64 int8 activations, 4 per dword
        int xs[4];        // sum of the 16 int8 values of each part
        float scale[4];   // activation scale of each part's 32-value group
    };

    __device__ static void load(Lane &L, const GemvParams &p, int token, int piece, const XGroup *) {
        load_direct(L, p, token, piece);
    }

    __device__ static void load_direct(Lane &L, const GemvParams &p, int token, int piece) {
        const int b = piece >> 2, g = (piece >> 1) & 1, h = piece & 1;
        const int8_t *xq = static_cast<const int8_t *>(p.x) + static_cast<int64_t>(token) * p.ldx + b * 256 + g * 128 +
                           h * 16;
        const float *xsc = p.xscale + static_cast<int64_t>(token) * p.ldscale + b * 8 + g * 4;
        #pragma unroll
        for (int part = 0; part < 4; ++part) {
            uint4 v = *reinterpret_cast<const uint4 *>(xq + part * 32);
            L.xq[part * 4 + 0] = static_cast<int>(v.x);
            L.xq[part * 4 + 1] = static_cast<int>(v.y);
            L.xq[part * 4 + 2] = static_cast<int>(v.z);
            L.xq[part * 4 + 3] = static_cast<int>(v.w);
            int s = 0;
            #pragma unroll
            for (int k = 0; k < 4; ++k) s = __builtin_amdgcn_sdot4(L.xq[part * 4 + k], 0x01010101, s, false);
            L.xs[part] = s;
            L.scale[part] = xsc[part];
        }
    }

    __device__ static float q4k(const Raw &r, const Lane &L, int g) {
        const uint32_t M = 0x0F0F0F0Fu;
        int D[4] = {0, 0, 0, 0};
        const uint32_t qa[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t qb[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        #pragma unroll
        for (int k = 0; k < 4; ++k) {
            D[0] = __builtin_amdgcn_sdot4(static_cast<int>(qa[k] & M), L.xq[0 * 4 + k], D[0], false);
            D[1] = __builtin_amdgcn_sdot4(static_cast<int>((qa[k] >> 4) & M), L.xq[1 * 4 + k], D[1], false);
            D[2] = __builtin_amdgcn_sdot4(static_cast<int>(qb[k] & M), L.xq[2 * 4 + k], D[2], false);
            D[3] = __builtin_amdgcn_sdot4(static_cast<int>((qb[k] >> 4) & M), L.xq[3 * 4 + k], D[3], false);
        }
        uint32_t sc, mn;
        q4k_scale_min4(r.a, g, sc, mn);
        const float d = f16_bits_to_f32(r.a.x & 0xFFFFu);
        const float dmin = f16_bits_to_f32(r.a.x >> 16);
        const float scf[4] = {ubyte0(sc), ubyte1(sc), ubyte2(sc), ubyte3(sc)};
        const float mnf[4] = {ubyte0(mn), ubyte1(mn), ubyte2(mn), ubyte3(mn)};
        float acc = 0.f;
        #pragma unroll
        for (int part = 0; part < 4; ++part)
            acc = fmaf(d * scf[part] * static_cast<float>(D[part]) -
                           dmin * mnf[part] * static_cast<float>(L.xs[part]),
                       L.scale[part], acc);
        return acc;
    }

    __device__ static float q6k(const Raw &r, const Lane &L, int h) {
        int D[4] = {0, 0, 0, 0};
        const uint32_t la[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const uint32_t lb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t qh[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        #pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t c[4];
            q6k_codes(la[k], lb[k], qh[k], c[0], c[1], c[2], c[3]);
            #pragma unroll
            for (int part = 0; part < 4; ++part)
                D[part] = __builtin_amdgcn_sdot4(static_cast<int>(c[part]), L.xq[part * 4 + k], D[part], false);
        }
        float sc[4];
        q6k_scales(r.s, h, sc);
        const float d = f16_bits_to_f32(r.d);
        float acc = 0.f;
        #pragma unroll
        for (int part = 0; part < 4; ++part)
            acc = fmaf(d * sc[part] * static_cast<float>(D[part] - 32 * L.xs[part]), L.scale[part], acc);
        return acc;
    }
};

// The INT8 LM head with the greedy-token epilogue (per-wave best row,
// lowest index among maxima, as F32ArgPolicy).
struct I8ArgPolicy : I8Policy {
    static constexpr bool kArgmax = true;
};

// The INT8 step's activations quantized by the GEMV itself: every block
// quantizes its token's fp32 row into LDS (codes, then per-32 scales, then
// 64 bytes of reduction scratch) and the lanes read their pieces from
// there.  The row is RMSNorm(x) * norm_w (norm_w set), SiLU(x) * up (up
// set) or x, quantized per 32 values -- the arithmetic of
// rmsnorm_quantize_kernel, silu_mul_quantize_kernel and quantize_x32_kernel
// (rmsnorm_quantize_cuda, silu_cuda + quantize_x32_cuda, quantize_x32_cuda;
// inferencer.cu:839-889, 1053-1056, 544-556).  With 256-thread blocks the
// sum of squares runs in rmsnorm_quantize_kernel's order, so the codes and
// scales are those kernels' bit for bit; other block sizes (3072 columns)
// sum in their own order.
struct I8FusedPolicy : I8Policy {
    static constexpr bool kPrepLds = true;
    static constexpr bool kDirect = false;

    __host__ __device__ static size_t lds_bytes(int cols) {
        return static_cast<size_t>(cols) + static_cast<size_t>(cols / 32) * sizeof(float) + 64;
    }

    // A group of 32 values is eight float4 of eight adjacent lanes (n4 is a
    // multiple of 8 and blocks hold whole waves).
    __device__ static void quantize4(const float4 &o, int i, uint32_t *q4, float *st) {
        quantize_quad_store(o, (i & 7) == 0, q4 + i, st + (i >> 3));
    }

    // Rows of up to kHeld float4 per thread are read once, x and the gains
    // together, and held in registers across the sum of squares; longer rows
    // read x twice.
    static constexpr int kHeld = 4;

    // The kernels that take the early form load a thread's kHeld float4 of
    // x and of the gains (or up, or x again) before their weights: the
    // loads return in order, so the staging then waits for these alone and
    // overlaps the weights' arrival.  Indexes are clamped to the row and
    // the loads are unconditional (static wait counts); rows longer than
    // kHeld float4 per thread ignore them.
    static constexpr bool kEarly = true;
    struct Early {
        float4 v[kHeld], w[kHeld];
    };

    __device__ static void early(Early &e, const GemvParams &p, int token, int cols) {
        const float *x = static_cast<const float *>(p.x) + static_cast<int64_t>(token) * p.ldx;
        const float *w = p.norm_w ? p.norm_w : p.up ? p.up + static_cast<int64_t>(token) * p.ldx : x;
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const float4 *w4 = reinterpret_cast<const float4 *>(w);
        const int last = (cols >> 2) - 1;
        #pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int i = min(static_cast<int>(threadIdx.x) + k * stage_threads(), last);
            e.v[k] = x4[i];
            e.w[k] = w4[i];
        }
    }

    // prep over what early loaded: the same values, sums and codes.
    __device__ static void prep_early(const Early &e, const GemvParams &p, int token, int cols, XGroup *lds) {
        const int n4 = cols >> 2;
        const int nt = stage_threads();
        const int tid = threadIdx.x;
        if (n4 > kHeld * nt) {
            prep(p, token, cols, lds);
            return;
        }
        const bool stager = tid < nt;   // whole waves
        uint32_t *q4 = reinterpret_cast<uint32_t *>(lds);
        float *st = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(lds) + cols);
        float *scratch = st + cols / 32;
        float scale = 1.f;
        if (p.norm_w) {
            float ss = 0.f;
            #pragma unroll
            for (int k = 0; k < kHeld; ++k) {
                if (stager && tid + k * nt < n4) {
                    ss = fmaf(e.v[k].x, e.v[k].x, ss);
                    ss = fmaf(e.v[k].y, e.v[k].y, ss);
                    ss = fmaf(e.v[k].z, e.v[k].z, ss);
                    ss = fmaf(e.v[k].w, e.v[k].w, ss);
                }
            }
            scale = 1.0f / sqrtf(block_sum(ss, scratch, nt) / static_cast<float>(cols) + p.norm_eps);
        }
        #pragma unroll
        for (int k = 0; k < kHeld; ++k) {
            const int i = tid + k * nt;
            if (!stager || i >= n4) continue;
            const float4 v = e.v[k], w = e.w[k];
            float4 o = v;
            if (p.norm_w)
                o = make_float4(v.x * scale * w.x, v.y * scale * w.y, v.z * scale * w.z, v.w * scale * w.w);
            else if (p.up)
                o = make_float4(silu_mul_value(v.x, w.x), silu_mul_value(v.y, w.y), silu_mul_value(v.z, w.z),
                                silu_mul_value(v.w, w.w));
            quantize4(o, i, q4, st);
        }
    }

    __device__ static void prep(const GemvParams &p, int token, int cols, XGroup *lds) {
        uint32_t *q4 = reinterpret_cast<uint32_t *>(lds);
        float *st = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(lds) + cols);
        float *scratch = st + cols / 32;
        const float4 *x4 = reinterpret_cast<const float4 *>(static_cast<const float *>(p.x) +
                                                            static_cast<int64_t>(token) * p.ldx);
        const float4 *w4 = reinterpret_cast<const float4 *>(p.norm_w);
        const float4 *u4 = reinterpret_cast<const float4 *>(p.up + (p.up ? static_cast<int64_t>(token) * p.ldx : 0));
        const int n4 = cols >> 2;
        const int nt = blockDim.x;
        const int tid = threadIdx.x;
        if (p.norm_w && n4 <= kHeld * nt) {
            float4 v[kHeld], w[kHeld];
            #pragma unroll
            for (int k = 0; k < kHeld; ++k) {
                const int i = tid + k * nt;
                if (i < n4) {
                    v[k] = x4[i];
                    w[k] = w4[i];
                }
            }
            float ss = 0.f;
            #pragma unroll
            for (int k = 0; k < kHeld; ++k) {
                if (tid + k * nt < n4) {
                    ss = fmaf(v[k].x, v[k].x, ss);
                    ss = fmaf(v[k].y, v[k].y, ss);
                    ss = fmaf(v[k].z, v[k].z, ss);
                    ss = fmaf(v[k].w, v[k].w, ss);
                }
            }
            const float scale = 1.0f / sqrtf(block_sum(ss, scratch, blockDim.x) / static_cast<float>(cols) + p.norm_eps);
            #pragma unroll
            for (int k = 0; k < kHeld; ++k) {
                const int i = tid + k * nt;
                if (i < n4)
                    quantize4(make_float4(v[k].x * scale * w[k].x, v[k].y * scale * w[k].y, v[k].z * scale * w[k].z,
                                          v[k].w * scale * w[k].w),
                              i, q4, st);
            }
            return;
        }
        float scale = 1.f;
        if (p.norm_w) {
            float ss = 0.f;
            #pragma unroll 4
            for (int i = tid; i < n4; i += nt) {
                const float4 v = x4[i];
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
            }
            scale = 1.0f / sqrtf(block_sum(ss, scratch, blockDim.x) / static_cast<float>(cols) + p.norm_eps);
        }
        for (int i = tid; i < n4; i += nt) {
            const float4 v = x4[i];
            float4 o = v;
            if (p.norm_w) {
                const float4 w = w4[i];
                o = make_float4(v.x * scale * w.x, v.y * scale * w.y, v.z * scale * w.z, v.w * scale * w.w);
            } else if (p.up) {
                const float4 u = u4[i];
                o = make_float4(silu_mul_value(v.x, u.x), silu_mul_value(v.y, u.y), silu_mul_value(v.z, u.z),
                                silu_mul_value(v.w, u.w));
            }
            quantize4(o, i, q4, st);
        }
    }

    // Sum over the first nt threads (whole waves; every thread of the block
    // calls it) in rmsnorm_quantize_kernel's order for 256 (every wave's xor
    // tree, then (w0 + w1) + (w2 + w3)); in wave order otherwise.
    __device__ static float block_sum(float ss, float *scratch, int nt) {
        #pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
        if ((threadIdx.x & 63) == 0 && static_cast<int>(threadIdx.x) < nt) scratch[threadIdx.x >> 6] = ss;
        __syncthreads();
        if (nt == 256) return (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
        ss = 0.f;
        for (int w = 0; w < nt >> 6; ++w) ss += scratch[w];
        return ss;
    }

    // Threads that stage the row in the early form: at most 256 (the
    // separate kernel's block, so its sum order holds); the rest of a larger
    // block waits at the barriers.
    __device__ static int stage_threads() { return min(static_cast<int>(blockDim.x), 256); }

    // The lane's piece from LDS: I8Policy::load_direct's layout.
    __device__ static void load(Lane &L, const GemvParams &p, int, int piece, const XGroup *lds) {
        const int cols = p.pieces * 64;
        const int b = piece >> 2, g = (piece >> 1) & 1, h = piece & 1;
        const uint8_t *xq = reinterpret_cast<const uint8_t *>(lds) + b * 256 + g * 128 + h * 16;
        const float *st = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(lds) + cols) + b * 8 + g * 4;
        #pragma unroll
        for (int part = 0; part < 4; ++part) {
            const uint4 v = *reinterpret_cast<const uint4 *>(xq + part * 32);
            L.xq[part * 4 + 0] = static_cast<int>(v.x);
            L.xq[part * 4 + 1] = static_cast<int>(v.y);
            L.xq[part * 4 + 2] = static_cast<int>(v.z);
            L.xq[part * 4 + 3] = static_cast<int>(v.w);
            int sum = 0;
            #pragma unroll
            for (int k = 0; k < 4; ++k) sum = __builtin_amdgcn_sdot4(L.xq[part * 4 + k], 0x01010101, sum, false);
            L.xs[part] = sum;
            L.scale[part] = st[part];
        }
    }

    __device__ static void load_direct(Lane &, const GemvParams &, int, int) {}
};

// The INT8 LM head of the one-sequence step: RMSNorm + quantization staged
// as I8FusedPolicy does, and the greedy-token epilogue.
struct I8FusedArgPolicy : I8FusedPolicy {
    static constexpr bool kArgmax = true;
};

// The one-sequence attention's unmerged split partials, as a GEMV that
// stages them loads them: thread t holds float4 t + k * nt of the row (k <
// kPartsHeld) from each of at most kMaxParts splits, with every load clamped
// (split, column) and unconditional so the wait counts stay static.
constexpr int kMaxParts = 8;
constexpr int kPartsHeld = 2;
struct PartsEarly {
    float4 acc[kPartsHeld][kMaxParts];
    float2 ml[kPartsHeld][kMaxParts];   // running max, sum of exp
};

__device__ __forceinline__ void parts_load(PartsEarly &e, const float *parts, int n_parts, int hd, int cols, int tid,
                                           int nt) {
    const int ps = split_partial_floats(hd);
    const int last = (cols >> 2) - 1;
    #pragma unroll
    for (int k = 0; k < kPartsHeld; ++k) {
        const int i = min(tid + k * nt, last);
        const int h = 4 * i / hd, c = 4 * i - h * hd;
        const float *base = parts + static_cast<int64_t>(h) * n_parts * ps;
        #pragma unroll
        for (int sp = 0; sp < kMaxParts; ++sp) {
            const float *q = base + min(sp, n_parts - 1) * ps;
            e.ml[k][sp] = *reinterpret_cast<const float2 *>(q);
            e.acc[k][sp] = *reinterpret_cast<const float4 *>(q + 4 + c);
        }
    }
}

// Float4 k of the thread's share merged: the attention merge kernel's
// arithmetic (the largest running max, exp2 weights, fma sums in split
// order, one divide per value).
__device__ __forceinline__ float4 parts_merge(const PartsEarly &e, int k, int n_parts) {
    float mx = -INFINITY;
    #pragma unroll
    for (int sp = 0; sp < kMaxParts; ++sp)
        if (sp < n_parts) mx = fmaxf(mx, e.ml[k][sp].x);
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    float den = 0.f;
    #pragma unroll
    for (int sp = 0; sp < kMaxParts; ++sp) {
        if (sp >= n_parts) continue;
        const float w = __builtin_amdgcn_exp2f(e.ml[k][sp].x - mx);
        den = fmaf(w, e.ml[k][sp].y, den);
        num.x = fmaf(w, e.acc[k][sp].x, num.x);
        num.y = fmaf(w, e.acc[k][sp].y, num.y);
        num.z = fmaf(w, e.acc[k][sp].z, num.z);
        num.w = fmaf(w, e.acc[k][sp].w, num.w);
    }
    return make_float4(num.x / den, num.y / den, num.z / den, num.w / den);
}

// The INT8 o projection of the one-sequence step over the attention's
// unmerged split partials: the staging merges each head's splits and
// quantizes the row per 32 as I8FusedPolicy does, so the codes equal those
// of the merge kernel's outputs through quantize_x32_kernel.  One token;
// rows of at most kPartsHeld * 4 * blockDim.x columns.
struct I8MergePolicy : I8FusedPolicy {
    using Early = PartsEarly;

    __device__ static void early(Early &e, const GemvParams &p, int, int cols) {
        parts_load(e, p.parts, p.n_parts, p.part_hd, cols, threadIdx.x, blockDim.x);
    }

    __device__ static void prep_early(const Early &e, const GemvParams &p, int, int cols, XGroup *lds) {
        uint32_t *q4 = reinterpret_cast<uint32_t *>(lds);
        float *st = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(lds) + cols);
        const int n4 = cols >> 2;
        #pragma unroll
        for (int k = 0; k < kPartsHeld; ++k) {
            const int i = static_cast<int>(threadIdx.x) + k * static_cast<int>(blockDim.x);
            if (i < n4) quantize4(parts_merge(e, k, p.n_parts), i, q4, st);
        }
    }

    // Kernels without the early form stage the same way, loads first.
    __device__ static void prep(const GemvParams &p, int token, int cols, XGroup *lds) {
        Early e;
        early(e, p, token, cols);
        prep_early(e, p, token, cols, lds);
    }
};

// Type dispatch of one piece: TYPE is the storage type when every matrix of
// the launch shares it, 0 for fused launches over mixed types (then `type`
// is wave-uniform and the branch is scalar).
template <int TYPE>
__device__ __forceinline__ bool is_q4k(int type) {
    return TYPE == QK_TYPE_Q4_K || (TYPE == 0 && type == QK_TYPE_Q4_K);
}

template <int TYPE>
__device__ __forceinline__ bool is_q6s(int type) {
    return TYPE == QK_TYPE_Q6_K_SPLIT || (TYPE == 0 && type == QK_TYPE_Q6_K_SPLIT);
}

// nb: blocks per row (the split layout's stream offsets).
template <int TYPE>
__device__ __forceinline__ Raw fetch_typed(const TileRef &t, int g, int h, int nb) {
    Raw r;
    if (is_q6s<TYPE>(t.type)) {
        const Q6Fields f = q6_fields(t.blk, nb, t.b, true);   // every field 16-byte aligned
        r.a = load16(f.ql + g * 64 + h * 16);
        r.b = load16(f.ql + 32 + g * 64 + h * 16);
        r.c = load16(f.qh + g * 32 + h * 16);
        r.s = load8(f.sc + g * 8);
        r.d = load2(f.d);
    } else if (is_q4k<TYPE>(t.type)) {
        r.a = load16(t.blk);                              // d, dmin, scales
        r.b = load16(t.blk + 16 + g * 64 + h * 16);      // parts 0 / 1
        r.c = load16(t.blk + 48 + g * 64 + h * 16);      // parts 2 / 3
        r.s = make_uint2(0, 0);
        r.d = 0;
    } else {
        r.a = load16(t.blk + g * 64 + h * 16);           // ql: parts 0 / 2
        r.b = load16(t.blk + 32 + g * 64 + h * 16);      // ql: parts 1 / 3
        r.c = load16(t.blk + 128 + g * 32 + h * 16);     // qh
        r.s = load8(t.blk + 192 + g * 8);                // scales[g*8 .. g*8+7]
        r.d = load2(t.blk + 208);
    }
    return r;
}

template <class Policy, int TYPE>
__device__ __forceinline__ float piece_dot(int type, const Raw &r, const typename Policy::Lane &L, int g, int h) {
    return is_q4k<TYPE>(type) ? Policy::q4k(r, L, g) : Policy::q6k(r, L, h);
}

// Output store: overwrite, or (policies that carry it, with p.accumulate)
// add into y.  Returns the stored value.
template <class Policy>
__device__ __forceinline__ float store_y(const GemvParams &p, float *y, float v) {
    if constexpr (Policy::kAccumulate) {
        if (p.accumulate) v += *y;
    }
    *y = v;
    return v;
}

// A lane's running best row (greedy-token policy only).
template <class Policy>
__device__ __forceinline__ void keep_best(float &bv, int &bi, float v, int row) {
    if constexpr (Policy::kArgmax) arg_better(bv, bi, v, row);
}

// Greedy-token epilogue: the wave's best (value, row) over its lanes'
// running bests, written to arg_v / arg_i[blockIdx.x * waves + wave] -- one
// partial per wave, so no wave waits for another.
template <class Policy>
__device__ __forceinline__ void arg_epilogue(const GemvParams &p, float bv, int bi) {
    if constexpr (Policy::kArgmax) {
        #pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            arg_better(bv, bi, ov, oi);
        }
        if ((threadIdx.x & 63) == 0) {
            const int slot = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
            p.arg_v[slot] = bv;
            p.arg_i[slot] = bi;
        }
    }
}

// One prefetched tile: where its result goes and its raw bytes.
struct Slot {
    TileRef t;
    Raw r;
};

template <int TYPE>
__device__ __forceinline__ Slot prep(const GemvParams &p, int tile, int rit, int piece, int token, int g, int h) {
    Slot s;
    s.t = locate(p, tile, rit, piece >> 2, token);
    s.r = fetch_typed<TYPE>(s.t, g, h, p.pieces >> 2);
    return s;
}

// C == 1 (P divides 64): every tile lives inside one wave; no LDS, no
// barriers.  GROUP == P lanes per row, 64/P rows per tile.  Each wave keeps
// two tiles in flight; the prefetch index is clamped to the last tile so the
// loads are unconditional (a wave's last prefetches re-read a valid tile).
template <class Policy, int TYPE, int GROUP>
__global__ __launch_bounds__(384) void gemv_wave(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_waves = blockDim.x >> 6;
    const int token = blockIdx.y;
    const int rit = lane / GROUP;
    const int piece = lane & (GROUP - 1);
    const int g = (piece >> 1) & 1, h = piece & 1;
    XGroup *xg = reinterpret_cast<XGroup *>(qk_smem);
    const int stride = gridDim.x * n_waves;
    const int first = blockIdx.x * n_waves + wave;
    const int last = p.total_tiles - 1;
    typename Policy::Early e;
    if constexpr (Policy::kEarly) Policy::early(e, p, token, p.pieces * 64);
    // The first two tiles' loads are in flight while the block prepares the
    // activations (a wave without tiles loads the last one and discards it).
    Slot a = prep<TYPE>(p, min(first, last), rit, piece, token, g, h);
    Slot b = prep<TYPE>(p, min(first + stride, last), rit, piece, token, g, h);
    if (Policy::kPrepLds) {
        if constexpr (Policy::kEarly)
            Policy::prep_early(e, p, token, p.pieces * 64, xg);
        else
            Policy::prep(p, token, p.pieces * 64, xg);
        __syncthreads();
    }
    typename Policy::Lane L;
    Policy::load(L, p, token, piece, xg);
    float bv = -INFINITY;   // greedy-token epilogue: this lane's best row so far
    int bi = 0x7FFFFFFF;
    const int n_iter = first < p.total_tiles ? (last - first) / stride + 1 : 0;
    int k = 0;
    while (k < n_iter) {
        float v = group_sum<GROUP>(piece_dot<Policy, TYPE>(a.t.type, a.r, L, g, h));
        if (piece == 0 && a.t.valid) keep_best<Policy>(bv, bi, store_y<Policy>(p, a.t.y + a.t.row, v), a.t.row);
        a = prep<TYPE>(p, min(first + (k + 2) * stride, last), rit, piece, token, g, h);
        if (++k == n_iter) break;
        v = group_sum<GROUP>(piece_dot<Policy, TYPE>(b.t.type, b.r, L, g, h));
        if (piece == 0 && b.t.valid) keep_best<Policy>(bv, bi, store_y<Policy>(p, b.t.y + b.t.row, v), b.t.row);
        b = prep<TYPE>(p, min(first + (k + 2) * stride, last), rit, piece, token, g, h);
        ++k;
    }
    arg_epilogue<Policy>(p, bv, bi);
}

// ------------------------------------- C == 1 over one whole-tile matrix --
//
// gemv_wave's work for a launch over one matrix whose rows fill whole tiles:
// tile t is the span w + t * TR * row_bytes, so its base is wave-uniform
// (scalar registers) and a lane's five field offsets inside a tile never
// change.  The loads take the scalar base plus 32-bit lane offsets computed
// once, so no per-tile vector address arithmetic is left (gemv_wave rebuilds
// five 64-bit addresses per tile: 13 of its 177 VALU instructions).

// Byte offsets of a lane's fields from the first byte of its tile (the
// bytes fetch_typed loads).
struct LaneFields {
    uint32_t a, b, c, s, d;
};

template <int TYPE>
__device__ __forceinline__ LaneFields lane_fields(int rit, int row_bytes, int nb, int b, int g, int h) {
    const uint32_t r = static_cast<uint32_t>(rit * row_bytes);
    LaneFields f;
    if constexpr (TYPE == QK_TYPE_Q6_K_SPLIT) {
        f.a = r + b * 128 + g * 64 + h * 16;
        f.b = f.a + 32;
        f.c = r + nb * 128 + b * 64 + g * 32 + h * 16;
        f.s = r + nb * 192 + b * 16 + g * 8;
        f.d = r + nb * 208 + b * 2;
    } else if constexpr (TYPE == QK_TYPE_Q4_K) {
        const uint32_t blk = r + b * 144;
        f.a = blk;
        f.b = blk + 16 + g * 64 + h * 16;
        f.c = blk + 48 + g * 64 + h * 16;
        f.s = f.d = 0;
    } else {
        const uint32_t blk = r + b * 210;
        f.a = blk + g * 64 + h * 16;
        f.b = blk + 32 + g * 64 + h * 16;
        f.c = blk + 128 + g * 32 + h * 16;
        f.s = blk + 192 + g * 8;
        f.d = blk + 208;
    }
    return f;
}

// The tile as a raw buffer resource (scalar registers: base, no stride,
// `bytes` records; the third descriptor word of gfx9-family chips), so every
// field load is a buffer load at a 32-bit lane offset from a scalar base.
// Offsets past `bytes` would read zero; every lane offset lies inside it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const uint8_t *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, bytes, 0x00020000);
}

template <int TYPE>
__device__ __forceinline__ Raw fetch_whole(const uint8_t *tile, int tile_bytes, const LaneFields &f) {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc(tile, tile_bytes);
    Raw r;
    r.a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, f.a, 0, 0));
    r.b = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, f.b, 0, 0));
    r.c = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, f.c, 0, 0));
    if constexpr (TYPE == QK_TYPE_Q4_K) {
        r.s = make_uint2(0, 0);
        r.d = 0;
    } else {
        r.s = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, f.s, 0, 0));
        r.d = __builtin_amdgcn_raw_buffer_load_b16(rs, f.d, 0, 0);
    }
    return r;
}

template <class Policy, int TYPE, int GROUP>
__global__ __launch_bounds__(256) void gemv_whole(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_waves = blockDim.x >> 6;
    const int token = blockIdx.y;
    const int rit = lane / GROUP;
    const int piece = lane & (GROUP - 1);
    const int g = (piece >> 1) & 1, h = piece & 1;
    const GemvMatrix &M = p.mat[0];
    const int tile_bytes = p.tile_rows * M.row_bytes;
    const LaneFields lf = lane_fields<TYPE>(rit, M.row_bytes, p.pieces >> 2, piece >> 2, g, h);
    XGroup *xg = reinterpret_cast<XGroup *>(qk_smem);
    const int stride = gridDim.x * n_waves;
    const int first = blockIdx.x * n_waves + wave;
    const int last = p.total_tiles - 1;
    // Prefetch indexes clamp to the last tile: unconditional, in-bounds loads.
    auto fetch = [&](int k) {
        return fetch_whole<TYPE>(M.w + static_cast<size_t>(min(first + k * stride, last)) * tile_bytes, tile_bytes, lf);
    };
    typename Policy::Early e;
    if constexpr (Policy::kEarly) Policy::early(e, p, token, p.pieces * 64);
    Raw a = fetch(0);
    Raw b = fetch(1);
    if (Policy::kPrepLds) {
        if constexpr (Policy::kEarly)
            Policy::prep_early(e, p, token, p.pieces * 64, xg);
        else
            Policy::prep(p, token, p.pieces * 64, xg);
        __syncthreads();
    }
    typename Policy::Lane L;
    Policy::load(L, p, token, piece, xg);
    float bv = -INFINITY;   // greedy-token epilogue: this lane's best row so far
    int bi = 0x7FFFFFFF;
    float *y = M.y + static_cast<int64_t>(token) * M.ldy + rit;
    const int n_iter = first < p.total_tiles ? (last - first) / stride + 1 : 0;
    int k = 0;
    while (k < n_iter) {
        int row0 = (first + k * stride) * p.tile_rows;
        float v = group_sum<GROUP>(piece_dot<Policy, TYPE>(TYPE, a, L, g, h));
        if (piece == 0) keep_best<Policy>(bv, bi, store_y<Policy>(p, y + row0, v), row0 + rit);
        a = fetch(k + 2);
        if (++k == n_iter) break;
        row0 = (first + k * stride) * p.tile_rows;
        v = group_sum<GROUP>(piece_dot<Policy, TYPE>(TYPE, b, L, g, h));
        if (piece == 0) keep_best<Policy>(bv, bi, store_y<Policy>(p, y + row0, v), row0 + rit);
        b = fetch(k + 2);
        ++k;
    }
    arg_epilogue<Policy>(p, bv, bi);
}

// ------------------------------------------- LDS-staged C == 1 variant --
//
// The INT8 kernel over the split Q6_K layout, for long launches over one
// matrix of whole tiles.  A C == 1 tile is 16 blocks (TR rows of P/4
// blocks, TR*P = 64): one contiguous span of TR * row_bytes bytes (3360-3584)
// that starts 16-byte aligned.  Each wave copies its tiles into a
// wave-private LDS ring of kLdsDepth slots with global_load_lds_dwordx4
// (lane i of a copy instruction moves 16 bytes to slot + 16*i; the slot
// address goes in M0), kLdsDepth - 1 tiles ahead of the one it computes, and
// lanes read their fields from LDS: the weights never pass through VGPRs.
// Measured on MI355X (128256 x 2048, 4 rotating copies, results bit-identical
// to gemv_wave): INT8 split Q6_K 36.0 us against 37.8; no gain for the FP32
// policies (38.7-40.0 against 38.5-38.7: the 3-limb arithmetic, not the
// loads, sets their pace), the GGUF Q6_K layout (39.6-40.9 against 39.8-40.0)
// or Q4_K (INT8 26.3-31.7 against 26.9), so those keep gemv_wave.
//
// The copies are inline assembly with an explicit s_waitcnt vmcnt: the
// compiler's own tracking of LDS DMA waits for every copy in flight
// (vmcnt(0)) before the first LDS read, which removes the pipelining.
// Vector memory loads complete in issue order, so when at most
// kLdsCopies * (kLdsDepth - 1) vector memory operations remain outstanding,
// every copy of the oldest tile has landed (the copies of the younger tiles
// are that many loads; stores and loads issued in between only make the
// wait stricter).
constexpr int kLdsDepth = 2;
constexpr int kLdsBlocksPerCu = 2;
constexpr int kLdsCopies = 4;                // 16-byte chunks per tile: 210-224, four instructions of 64
constexpr int kLdsMaxTileBytes = 16 * 224;   // one block per row, padded to 224 B

__device__ __forceinline__ uint32_t lds_offset(const void *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void *)p));
}

// 16 bytes from global memory to LDS: this lane's `src` lands at
// m0 + 16 * lane (m0 wave-uniform).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const uint8_t *src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Issue the copies of one tile (`chunks` 16-byte chunks at src, 210..224)
// into the slot at LDS address dst.  Every instruction has at least one
// active lane, so each tile is exactly kLdsCopies vector memory operations.
__device__ __forceinline__ void copy_tile(const uint8_t *src, uint32_t dst, int chunks, int lane) {
    constexpr int kFull = kLdsCopies - 1;
    #pragma unroll
    for (int i = 0; i < kFull; ++i) lds_copy16(src + static_cast<size_t>(i * 64 + lane) * 16, dst + i * 1024);
    if (lane < chunks - kFull * 64) lds_copy16(src + static_cast<size_t>(kFull * 64 + lane) * 16, dst + kFull * 1024);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// A lane's fields from its tile's LDS copy: the bytes fetch_typed loads for
// the split layout (rows padded to 16 bytes, so every field is aligned).
// row_off = the lane's row within the tile times row_bytes.
__device__ __forceinline__ Raw lds_fetch_split(const unsigned char *tb, int row_off, int nb, int b, int g, int h) {
    const Q6Fields f = q6_fields(tb + row_off, nb, b, true);
    Raw r;
    r.a = *reinterpret_cast<const uint4 *>(f.ql + g * 64 + h * 16);
    r.b = *reinterpret_cast<const uint4 *>(f.ql + 32 + g * 64 + h * 16);
    r.c = *reinterpret_cast<const uint4 *>(f.qh + g * 32 + h * 16);
    r.s = *reinterpret_cast<const uint2 *>(f.sc + g * 8);
    r.d = *reinterpret_cast<const uint16_t *>(f.d);
    return r;
}

template <class Policy, int GROUP>
__global__ __launch_bounds__(256) void gemv_lds(GemvParams p) {
    constexpr int TYPE = QK_TYPE_Q6_K_SPLIT;
    constexpr int D = kLdsDepth;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_waves = blockDim.x >> 6;
    const int token = blockIdx.y;
    const int rit = lane / GROUP;
    const int piece = lane & (GROUP - 1);
    const int g = (piece >> 1) & 1, h = piece & 1;
    const int nb = p.pieces >> 2;
    const GemvMatrix &M = p.mat[0];
    const int tile_bytes = p.tile_rows * M.row_bytes;
    const int chunks = tile_bytes >> 4;
    XGroup *xg = reinterpret_cast<XGroup *>(qk_smem);
    const size_t x_lds = (Policy::lds_bytes(p.pieces * 64) + 15) & ~size_t(15);
    unsigned char *ring = qk_smem + x_lds + static_cast<size_t>(wave) * D * kLdsMaxTileBytes;
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_offset(ring));
    const int stride = gridDim.x * n_waves;
    const int first = blockIdx.x * n_waves + wave;
    const int last = p.total_tiles - 1;
    const int n_iter = first < p.total_tiles ? (last - first) / stride + 1 : 0;
    // Copies of the first D - 1 tiles are in flight while the block prepares
    // the activations (indexes clamp to the last tile, so every wave issues
    // the same number of copies and its last prefetches re-read a valid tile).
    // A staging policy's inputs load first (loads return in order: its
    // staging then waits for them alone, not for the tile copies).
    typename Policy::Early e;
    if constexpr (Policy::kEarly) Policy::early(e, p, token, p.pieces * 64);
    #pragma unroll
    for (int k = 0; k < D - 1; ++k)
        copy_tile(M.w + static_cast<size_t>(min(first + k * stride, last)) * tile_bytes,
                  ring_lds + k * kLdsMaxTileBytes, chunks, lane);
    if (Policy::kPrepLds) {
        if constexpr (Policy::kEarly)
            Policy::prep_early(e, p, token, p.pieces * 64, xg);
        else
            Policy::prep(p, token, p.pieces * 64, xg);
        __syncthreads();
    }
    typename Policy::Lane L;
    Policy::load(L, p, token, piece, xg);
    float bv = -INFINITY;   // greedy-token epilogue: this lane's best row so far
    int bi = 0x7FFFFFFF;
    float *y = M.y + static_cast<int64_t>(token) * M.ldy;
    const int row_off = rit * M.row_bytes;
    for (int k = 0; k < n_iter; ++k) {
        // The slot refilled here was read in iteration k - 1, whose values
        // fed that iteration's store; the lgkmcnt wait makes the order explicit.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const int ahead = k + D - 1;
        copy_tile(M.w + static_cast<size_t>(min(first + ahead * stride, last)) * tile_bytes,
                  ring_lds + (ahead % D) * kLdsMaxTileBytes, chunks, lane);
        wait_vm<kLdsCopies * (D - 1)>();
        const Raw r = lds_fetch_split(ring + (k % D) * kLdsMaxTileBytes, row_off, nb, piece >> 2, g, h);
        const float v = group_sum<GROUP>(piece_dot<Policy, TYPE>(TYPE, r, L, g, h));
        const int row = (first + k * stride) * p.tile_rows + rit;   // whole tiles: always < M.rows
        if (piece == 0) keep_best<Policy>(bv, bi, store_y<Policy>(p, y + row, v), row);
    }
    // Nothing may still be writing this workgroup's LDS when it exits.
    wait_vm<0>();
    arg_epilogue<Policy>(p, bv, bi);
}

// C > 1: the C waves of a wave-group share each tile; the group sums of a
// tile meet in LDS (double-buffered, one barrier per tile) and lane t of the
// group's first wave adds row t's C sums in chunk order.
template <class Policy, int TYPE, int GROUP>
__device__ __forceinline__ void split_step(const GemvParams &p, const Slot &s, const typename Policy::Lane &L,
                                           float *red, int k, int tile, int wgroup, int chunk, int lane, int q,
                                           int g, int h, int token, float &bv, int &bi) {
    const int slots = p.tile_rows * p.chunks;
    float v = group_sum<GROUP>(piece_dot<Policy, TYPE>(s.t.type, s.r, L, g, h));
    float *buf = red + (wgroup * 2 + (k & 1)) * slots;
    if ((lane & (GROUP - 1)) == 0) buf[q / GROUP] = v;
    __syncthreads();
    if (tile < p.total_tiles && chunk == 0 && lane < p.tile_rows) {
        const TileRef rowref = locate(p, tile, lane, 0, token);
        if (rowref.valid) {
            float sum = 0.f;
            for (int c = 0; c < p.chunks; ++c) sum += buf[lane * p.chunks + c];
            keep_best<Policy>(bv, bi, store_y<Policy>(p, rowref.y + rowref.row, sum), rowref.row);
        }
    }
}

// WHOLE: one matrix of whole tiles, read like gemv_whole (a raw buffer
// resource per tile in scalar registers, 32-bit lane offsets computed once).
template <class Policy, int TYPE, int GROUP, bool WHOLE = false>
__global__ __launch_bounds__(1024) void gemv_split(GemvParams p) {
    XGroup *xg = reinterpret_cast<XGroup *>(qk_smem);
    float *red = reinterpret_cast<float *>(qk_smem + Policy::lds_bytes(p.pieces * 64));
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int token = blockIdx.y;
    const int chunk = wave % p.chunks;
    const int wgroup = wave / p.chunks;
    const int n_wgroups = (blockDim.x >> 6) / p.chunks;
    const int q = chunk * 64 + lane;
    const int rit = q / p.pieces;
    const int piece = q - rit * p.pieces;
    const int g = (piece >> 1) & 1, h = piece & 1;
    const int per_iter = gridDim.x * n_wgroups;
    const int iters = (p.total_tiles + per_iter - 1) / per_iter;   // same for every wave of the block
    const int first = blockIdx.x * n_wgroups + wgroup;
    const int last = p.total_tiles - 1;
    const GemvMatrix &M = p.mat[0];
    const int tile_bytes = p.tile_rows * M.row_bytes;
    LaneFields lf{};
    if constexpr (WHOLE) lf = lane_fields<TYPE>(rit, M.row_bytes, p.pieces >> 2, piece >> 2, g, h);
    auto fetch = [&](int tile) -> Slot {
        if constexpr (WHOLE) {
            Slot sl;
            sl.t.type = TYPE;
            sl.r = fetch_whole<TYPE>(M.w + static_cast<size_t>(tile) * tile_bytes, tile_bytes, lf);
            return sl;
        } else {
            return prep<TYPE>(p, tile, rit, piece, token, g, h);
        }
    };
    Slot a = fetch(min(first, last));
    Slot b = fetch(min(first + per_iter, last));
    if (Policy::kPrepLds) {
        Policy::prep(p, token, p.pieces * 64, xg);
        __syncthreads();
    }
    typename Policy::Lane L;
    Policy::load(L, p, token, piece, xg);
    float bv = -INFINITY;   // greedy-token epilogue: this lane's best row so far
    int bi = 0x7FFFFFFF;
    int k = 0;
    while (true) {
        split_step<Policy, TYPE, GROUP>(p, a, L, red, k, first + k * per_iter, wgroup, chunk, lane, q, g, h, token,
                                        bv, bi);
        a = fetch(min(first + (k + 2) * per_iter, last));
        if (++k == iters) break;
        split_step<Policy, TYPE, GROUP>(p, b, L, red, k, first + k * per_iter, wgroup, chunk, lane, q, g, h, token,
                                        bv, bi);
        b = fetch(min(first + (k + 2) * per_iter, last));
        if (++k == iters) break;
    }
    arg_epilogue<Policy>(p, bv, bi);
}

// Rows whose chunk count exceeds kMaxChunks: one wave per row, lanes stride
// over the pieces and reload each piece's activations through the cache.
template <class Policy>
__global__ __launch_bounds__(256) void gemv_long(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_waves = blockDim.x >> 6;
    const int token = blockIdx.y;
    for (int tile = blockIdx.x * n_waves + wave; tile < p.total_tiles; tile += gridDim.x * n_waves) {
        float acc = 0.f;
        for (int piece = lane; piece < p.pieces; piece += 64) {
            const int g = (piece >> 1) & 1, h = piece & 1;
            typename Policy::Lane L;
            Policy::load_direct(L, p, token, piece);
            const TileRef t = locate(p, tile, 0, piece >> 2, token);
            const Raw r = fetch_typed<0>(t, g, h, p.pieces >> 2);
            acc += piece_dot<Policy, 0>(t.type, r, L, g, h);
        }
        acc = group_sum<64>(acc);
        const TileRef t = locate(p, tile, 0, 0, token);
        if (lane == 0 && t.valid) store_y<Policy>(p, t.y + t.row, acc);
    }
}

int gcd_int(int a, int b) {
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    return a;
}

// Waves of a gate / up pair workgroup: eight (two per SIMD: the dot
// products of one wave's tiles overlap another's; 1B decode 0.671 -> 0.656
// ms/token against four), fewer when the workgroup has fewer tiles (it has
// GROUP: 2 x 32 rows of 64 / GROUP rows each).
__host__ __device__ constexpr int pair_waves(int group) { return group < 8 ? group : 8; }

// The INT8 step's gate / up pair with SiLU(gate) * up quantized in the
// epilogue (silu_cuda and quantize_x32_cuda's arithmetic): workgroup w owns
// rows 32w .. 32w + 31 of both matrices -- 32 / TR tiles of TR = 64 / GROUP
// rows each -- and its waves take those 64 / TR tiles in turn; the row
// sums meet in LDS and one half-wave forms and quantizes the workgroup's
// 32 values into hq / hs (token-major, ldq / ldsc).  The first 256 threads
// stage the input (the separate kernel's sum order).
template <class Policy, int TYPE, int GROUP>
__global__ __launch_bounds__(pair_waves(GROUP) * 64) void gemv_pair_quant(GemvParams p, int8_t *hq, float *hs, int ldq,
                                                                         int ldsc) {
    constexpr int TR = 64 / GROUP;
    constexpr int kHalf = 32 / TR;         // tiles per matrix
    constexpr int NW = pair_waves(GROUP);
    constexpr int kPerWave = 2 * kHalf / NW;
    static_assert(kPerWave >= 1 && kPerWave * NW == 2 * kHalf, "whole tiles per wave");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int token = blockIdx.y;
    const int rit = lane / GROUP;
    const int piece = lane & (GROUP - 1);
    const int g = (piece >> 1) & 1, h = piece & 1;
    XGroup *xg = reinterpret_cast<XGroup *>(qk_smem);
    float *vals = reinterpret_cast<float *>(qk_smem + ((Policy::lds_bytes(p.pieces * 64) + 15) & ~size_t(15)));
    const int up_begin = p.mat[1].tile_begin;
    auto tile_at = [&](int k) {   // k < 2 * kHalf: gate tiles, then up tiles
        const int j = min(k, 2 * kHalf - 1);
        return (j >= kHalf ? up_begin : 0) + static_cast<int>(blockIdx.x) * kHalf + j % kHalf;
    };
    // The staging inputs, then up to kDepth tiles per wave (one wave per
    // SIMD: the registers are there), are in flight before the staging.
    typename Policy::Early e;
    Policy::early(e, p, token, p.pieces * 64);
    constexpr int kDepth = kPerWave < 8 ? kPerWave : 8;
    Slot sl[kDepth];
    #pragma unroll
    for (int j = 0; j < kDepth; ++j) sl[j] = prep<TYPE>(p, tile_at(wave + NW * j), rit, piece, token, g, h);
    Policy::prep_early(e, p, token, p.pieces * 64, xg);
    __syncthreads();
    typename Policy::Lane L;
    Policy::load(L, p, token, piece, xg);
    #pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        Slot &cur = sl[j % kDepth];
        const float v = group_sum<GROUP>(piece_dot<Policy, TYPE>(cur.t.type, cur.r, L, g, h));
        const int k = wave + NW * j;
        if (piece == 0) vals[(k >= kHalf ? 32 : 0) + (k % kHalf) * TR + rit] = v;
        if (j + kDepth < kPerWave) cur = prep<TYPE>(p, tile_at(wave + NW * (j + kDepth)), rit, piece, token, g, h);
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const int64_t r = static_cast<int64_t>(blockIdx.x) * 32 + threadIdx.x;
        quantize_group_store(silu_mul_value(vals[threadIdx.x], vals[32 + threadIdx.x]), true, threadIdx.x,
                             hq + static_cast<int64_t>(token) * ldq + r,
                             hs + static_cast<int64_t>(token) * ldsc + blockIdx.x);
    }
}

template <class Policy, int TYPE, int GROUP>
void launch_tiled(const GemvParams &p, int n_tokens, hipStream_t stream) {
    const size_t x_lds = Policy::lds_bytes(p.pieces * 64);
    if (p.chunks == 1) {
        // A staged multi-matrix launch (the INT8 step's QKV) runs six waves
        // per workgroup: every workgroup stages the whole row (the first 256
        // threads, so the sum order and codes hold), and one staging then
        // serves six waves' tiles instead of four (1B QKV 7.9 -> 7.4 us,
        // INT8 decode 0.603 -> 0.594 ms/token; eight waves: 8.7 us).
        const bool six = std::is_same_v<Policy, I8FusedPolicy> && p.n_mats > 1;
        const int block = six ? 6 * 64 : 256, waves = block / 64;
        const void *k = reinterpret_cast<const void *>(gemv_wave<Policy, TYPE, GROUP>);
        const int cus = device_info().cus;
        const bool aligned = TYPE == QK_TYPE_Q4_K || TYPE == QK_TYPE_Q6_K_SPLIT;
        const bool long_launch =
            static_cast<int64_t>(p.total_tiles) * n_tokens >= int64_t(kWaveLongTiles) * kWaveBlocksPerCu * waves * cus;
        // The LDS-staged kernel (INT8, split Q6_K): one matrix of whole tiles
        // at a 16-byte aligned address, in a launch long enough for its
        // pipeline to fill.
        if constexpr ((std::is_same_v<Policy, I8Policy> || std::is_same_v<Policy, I8ArgPolicy> ||
                       std::is_same_v<Policy, I8FusedArgPolicy>) &&
                      TYPE == QK_TYPE_Q6_K_SPLIT) {
            if (long_launch && p.n_mats == 1 && p.mat[0].rows % p.tile_rows == 0 &&
                (reinterpret_cast<uintptr_t>(p.mat[0].w) & 15) == 0 &&
                p.tile_rows * p.mat[0].row_bytes <= kLdsMaxTileBytes) {
                const size_t lds = ((x_lds + 15) & ~size_t(15)) + static_cast<size_t>(waves) * kLdsDepth * kLdsMaxTileBytes;
                const void *kl = reinterpret_cast<const void *>(gemv_lds<Policy, GROUP>);
                const int cap = std::max(1, std::min(resident_blocks(kl, block, lds), kLdsBlocksPerCu * cus) / n_tokens);
                const int grid_all = std::max(1, std::min<int>((p.total_tiles + waves - 1) / waves, cap));
                const int grid = std::min(grid_all, p.arg_v ? kArgPartsMax / waves : grid_all);
                if (p.grid_out) *p.grid_out = grid * waves;
                hipLaunchKernelGGL((gemv_lds<Policy, GROUP>), dim3(grid, n_tokens), dim3(block), lds, stream, p);
                return;
            }
        }
        // One matrix of whole tiles: gemv_whole (scalar tile bases), else gemv_wave.
        const bool whole = TYPE != 0 && p.n_mats == 1 && p.mat[0].rows % p.tile_rows == 0;
        const void *fn = whole ? reinterpret_cast<const void *>(gemv_whole<Policy, TYPE, GROUP>) : k;
        const int per_cu = aligned && long_launch ? (Policy::kInt8 ? kWaveBlocksPerCuLongInt8 : kWaveBlocksPerCuLong)
                                                  : kWaveBlocksPerCu;
        const int cap = std::max(1, std::min(resident_blocks(fn, block, x_lds), per_cu * cus) / n_tokens);
        const int grid_all = std::max(1, std::min<int>((p.total_tiles + waves - 1) / waves, cap));
        // Grid-stride tiles: clamping keeps the argmax partials (one per wave)
        // in their buffer.
        const int grid = std::min(grid_all, p.arg_v ? kArgPartsMax / waves : grid_all);
        if (p.grid_out) *p.grid_out = grid * waves;
        if (whole)
            hipLaunchKernelGGL((gemv_whole<Policy, TYPE, GROUP>), dim3(grid, n_tokens), dim3(block), x_lds, stream, p);
        else
            hipLaunchKernelGGL((gemv_wave<Policy, TYPE, GROUP>), dim3(grid, n_tokens), dim3(block), x_lds, stream, p);
    } else {
        // Every block stages the whole activation row: two blocks per CU (one
        // when each wave-group would see fewer than kSplitShortTiles tiles)
        // keep that staging small next to the weights.  A short launch's one
        // block per CU holds eight waves instead of four: two per SIMD, so
        // one wave's dot products and reductions overlap another's (INT8 1B
        // down, 2048 x 8192: 1B decode 0.657 -> 0.639 ms/token).
        const int cus = device_info().cus;
        const int wgroups4 = std::max(1, 4 / p.chunks);
        const bool short_launch = static_cast<int64_t>(p.total_tiles) * n_tokens <
                                  int64_t(kSplitShortTiles) * kSplitBlocksPerCu * wgroups4 * cus;
        const int wgroups = short_launch ? std::max(1, 8 / p.chunks) : wgroups4;
        const int block = wgroups * p.chunks * 64;
        const size_t lds = x_lds + static_cast<size_t>(wgroups) * 2 * p.tile_rows * p.chunks * sizeof(float);
        bool whole = false;
        const void *k = reinterpret_cast<const void *>(gemv_split<Policy, TYPE, GROUP>);
        // Whole-tile reads for the FP32 policies (3B LM head 60.3 against
        // 60.9 us); the INT8 kernel measured slower with them (57.4 / 56.4).
        if constexpr (TYPE != 0 && !Policy::kInt8) {
            whole = p.n_mats == 1 && p.mat[0].rows % p.tile_rows == 0;
            if (whole) k = reinterpret_cast<const void *>(gemv_split<Policy, TYPE, GROUP, true>);
        }
        const bool long_split = static_cast<int64_t>(p.total_tiles) * n_tokens >=
                                int64_t(kWaveLongTiles) * kSplitBlocksPerCu * wgroups * cus;
        const int per_cu = short_launch ? 1 : long_split ? kSplitBlocksPerCuLong : kSplitBlocksPerCu;
        const int cap = std::max(1, std::min(resident_blocks(k, block, lds), per_cu * cus) / n_tokens);
        const int grid_all = std::max(1, std::min<int>((p.total_tiles + wgroups - 1) / wgroups, cap));
        const int grid = std::min(grid_all, p.arg_v ? kArgPartsMax / (block / 64) : grid_all);
        if (p.grid_out) *p.grid_out = grid * (block / 64);
        if constexpr (TYPE != 0 && !Policy::kInt8) {
            if (whole) {
                hipLaunchKernelGGL((gemv_split<Policy, TYPE, GROUP, true>), dim3(grid, n_tokens), dim3(block), lds,
                                   stream, p);
                return;
            }
        }
        hipLaunchKernelGGL((gemv_split<Policy, TYPE, GROUP>), dim3(grid, n_tokens), dim3(block), lds, stream, p);
    }
}

template <class Policy, int TYPE>
void launch_group(const GemvParams &p, int n_tokens, hipStream_t stream) {
    switch (p.group_lanes) {
        case 4: launch_tiled<Policy, TYPE, 4>(p, n_tokens, stream); break;
        case 8: launch_tiled<Policy, TYPE, 8>(p, n_tokens, stream); break;
        case 16: launch_tiled<Policy, TYPE, 16>(p, n_tokens, stream); break;
        case 32: launch_tiled<Policy, TYPE, 32>(p, n_tokens, stream); break;
        default: launch_tiled<Policy, TYPE, 64>(p, n_tokens, stream); break;
    }
}

template <class Policy>
int launch(GemvParams &p, const qk_matrix *mats, int n_mats, int cols, int n_tokens, const int *ldy,
           hipStream_t stream, const char *where) {
    const int nb = cols / 256;
    p.n_mats = n_mats;
    p.pieces = 4 * nb;
    p.group_lanes = gcd_int(p.pieces, 64);
    p.tile_rows = 64 / p.group_lanes;
    p.chunks = p.pieces / p.group_lanes;
    const bool long_rows = p.chunks > kMaxChunks || Policy::lds_bytes(cols) + 4096 > kMaxLds;
    if (long_rows) p.tile_rows = 1;
    int64_t tiles = 0;
    int type = mats[0].type;
    for (int m = 0; m < n_mats; ++m) {
        GemvMatrix &M = p.mat[m];
        M.w = static_cast<const uint8_t *>(mats[m].w);
        M.y = mats[m].y;
        M.rows = mats[m].rows;
        M.type = mats[m].type;
        M.row_bytes = static_cast<int>(row_bytes(M.type, nb));
        M.ldy = ldy ? ldy[m] : M.rows;
        M.tile_begin = static_cast<int>(tiles);
        tiles += (M.rows + p.tile_rows - 1) / p.tile_rows;
        if (static_cast<int64_t>(M.rows) * M.row_bytes > (int64_t(1) << 40))
            return fail(QK_ERR_LIMIT, std::string(where) + ": matrix too large");
        if (M.type != type) type = 0;
    }
    if (tiles > (1 << 30)) return fail(QK_ERR_LIMIT, std::string(where) + ": too many rows");
    if (n_tokens > 65535) return fail(QK_ERR_LIMIT, std::string(where) + ": too many tokens in one launch");
    p.total_tiles = static_cast<int>(tiles);

    if (long_rows) {
        if constexpr (Policy::kDirect) {
            const int block = 256, waves = block / 64;
            const int grid = std::max(1, std::min<int>((p.total_tiles + waves - 1) / waves, device_info().cus * 8));
            hipLaunchKernelGGL(gemv_long<Policy>, dim3(grid, n_tokens), dim3(block), 0, stream, p);
        } else {
            return fail(QK_ERR_LIMIT, std::string(where) + ": rows too long to stage in LDS");
        }
    } else if (type == QK_TYPE_Q4_K) {
        launch_group<Policy, QK_TYPE_Q4_K>(p, n_tokens, stream);
    } else if (type == QK_TYPE_Q6_K) {
        launch_group<Policy, QK_TYPE_Q6_K>(p, n_tokens, stream);
    } else if (type == QK_TYPE_Q6_K_SPLIT) {
        launch_group<Policy, QK_TYPE_Q6_K_SPLIT>(p, n_tokens, stream);
    } else {
        launch_group<Policy, 0>(p, n_tokens, stream);
    }
    return launch_status(where);
}

// ------------------------------------------- decode GEMV over records --
//
// The decode driver's FP32 GEMVs read activation records that the kernel
// producing the activations made (no staging, no barrier before the first
// dot), and can make the next GEMV's records in their epilogue.  A
// workgroup of W waves walks row blocks of kRecRows rows -- of one matrix,
// or of matrices 0 and 1 together (gate and up: `pair`) -- grid-stride.
// Within a block, step s of wave w covers the (row, piece) pairs
// q = s*64W + 64w + lane in row-major order; 64W is a multiple of P, so a
// lane's piece q % P is the same at every step and its four records are
// loaded once.  Aligned groups of G = gcd(P, 64) lanes share a row; their
// sums meet in LDS when a row spans waves (C = P/G > 1) or an epilogue needs
// the block's values together.  With an RMSNorm on the input, the records
// hold x * gain and every output is scaled by 1/sqrt(mean(x^2) + eps) after
// the dot (W (s x * g) = s W (x * g)), the scale reduced from the records'
// sums of squares by each wave on its own.
constexpr int kRecRows = 16;
constexpr int kRecMaxChunks = 16;

struct RecMatrix {
    const uint8_t *w;
    float *y;
    int rows, type, row_bytes, block_begin;
};

constexpr int kRecMaxMats = 4;   // matrices of one record launch (QKV: 3, gate/up: 2)

struct RecParams {
    RecMatrix mat[kRecMaxMats];
    int n_mats;
    int pair;              // blocks cover rows of matrices 0 and 1 (SiLU records)
    int nb, pieces;        // blocks per row, P = 4 nb
    int steps;             // per wave and block: W * steps * 64 = (pair ? 2 : 1) * kRecRows * P
    int steps_log2;        // steps is a power of two
    int waves;             // W (the workgroup's size in waves)
    int n_blocks;
    const XGroup *rec;     // input records, cols / 16
    const float *ss;       // input: sum of squares of the raw activations per record (RMSNorm), or NULL
    float norm_eps;
    int accumulate;        // y += W x
    XGroup *rec_out;       // output records (NULL: none): y * gain, or SiLU(gate) * up with pair
    float *ss_out;         // their sums of squares of y (not with pair)
    const float *gain;     // NULL: 1
    float *arg_v;          // greedy-pick partials, one per wave (NULL: none)
    int *arg_i;
    // MERGE kernels: the input is the attention's unmerged split partials
    // ([head][n_parts][split_partial_floats(part_hd)]), merged and made into
    // records in LDS instead of read from rec.
    const float *parts;
    int n_parts;
    int part_hd;
};

struct RecSlot {
    Raw r;
    int m;         // matrix (wave-uniform)
    int row;       // row of the lane's pair (may be past the matrix: not stored)
    float yold;    // residual input of the row (the lane that stores it)
};

// Matrix m of the launch with every field read at a static offset and
// selected (m wave-uniform): the parameter loads of all matrices go out at
// once instead of one dependent load per field.
__device__ __forceinline__ RecMatrix rec_mat(const RecParams &p, int m) {
    if (p.n_mats == 1) return p.mat[0];
    RecMatrix r;
    r.w = p.mat[0].w;
    r.y = p.mat[0].y;
    r.rows = p.mat[0].rows;
    r.type = p.mat[0].type;
    r.row_bytes = p.mat[0].row_bytes;
    r.block_begin = p.mat[0].block_begin;
    #pragma unroll
    for (int i = 1; i < kRecMaxMats; ++i) {
        const bool s = m == i;
        r.w = s ? p.mat[i].w : r.w;
        r.y = s ? p.mat[i].y : r.y;
        r.rows = s ? p.mat[i].rows : r.rows;
        r.type = s ? p.mat[i].type : r.type;
        r.row_bytes = s ? p.mat[i].row_bytes : r.row_bytes;
        r.block_begin = s ? p.mat[i].block_begin : r.block_begin;
    }
    return r;
}

// Matrix and first row of row block blk (wave-uniform), without a loop over
// the matrices.
__device__ __forceinline__ void rec_block(const RecParams &p, int blk, int m_local, int &m, int &row0) {
    if (p.pair) {
        m = m_local;
        row0 = blk * kRecRows;
        return;
    }
    if (p.n_mats == 1) {
        m = 0;
        row0 = blk * kRecRows;
        return;
    }
    m = 0;
    int begin = 0;
    #pragma unroll
    for (int i = 1; i < kRecMaxMats; ++i) {
        const bool in = i < p.n_mats && blk >= p.mat[i].block_begin;
        m += in ? 1 : 0;
        begin = in ? p.mat[i].block_begin : begin;
    }
    row0 = (blk - begin) * kRecRows;
}

// ri: the lane's row within the block (all matrices) at this step, piece:
// the lane's piece (the same at every step: 64 W is a multiple of P).
template <int TYPE>
__device__ __forceinline__ RecSlot rec_fetch(const RecParams &p, int blk, int ri, int piece, int g, int h,
                                             bool loads_yold) {
    const int m_local = __builtin_amdgcn_readfirstlane(ri / kRecRows);   // one block half per wave step
    int m, row0;
    rec_block(p, blk, m_local, m, row0);
    RecSlot t;
    t.m = __builtin_amdgcn_readfirstlane(m);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    const RecMatrix M = rec_mat(p, t.m);
    t.row = row0 + ri - m_local * kRecRows;
    const bool valid = t.row < M.rows;
    const int row = valid ? t.row : M.rows - 1;   // keep loads in bounds
    TileRef ref;
    ref.type = M.type;
    ref.b = piece >> 2;
    const int bpb = M.type == QK_TYPE_Q4_K ? 144 : M.type == QK_TYPE_Q6_K ? 210 : 0;
    ref.blk = M.w + static_cast<size_t>(row) * M.row_bytes + static_cast<size_t>(piece >> 2) * bpb;
    t.r = fetch_typed<TYPE>(ref, g, h, p.nb);
    t.yold = M.y[row];   // unconditional (any valid row); used only where loads_yold
    if (!loads_yold) t.yold = 0.f;
    return t;
}

// EPI: the block's row sums go through LDS (rows spanning waves, output
// records or the gate/up pair); otherwise each row's group stores it.
// Every wave keeps D tiles' loads in flight (2 when it has at most two).
constexpr int kRecMaxWaves = 8;
constexpr int kRecSsPerLane = 8;    // sums of squares a lane reads: nb <= 32

// The record of the 16 values x held by lanes 0..15 of a wave (the other
// lanes' values are ignored), made by those lanes together: the group's
// maximum, sum and exponent through xor shuffles, each lane's three limb
// bytes packed four lanes to a dword, and lane i storing dword i of the
// 64-byte record -- make_group_regs' arithmetic, with the sum of the 16
// values taken as a tree.  sq: the lanes' squares, summed into *ss when ss
// is given.  Every lane of the wave must call it.
__device__ __forceinline__ void record16(float x, float sq, int lane, XGroup *dst, float *ss) {
    const bool in = lane < 16;
    x = in ? x : 0.f;
    sq = in ? sq : 0.f;
    float m = fabsf(x), sum = x;
    #pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        sum += __shfl_xor(sum, off);
        sq += __shfl_xor(sq, off);
    }
    const bool ok = m > 0.f && isfinite(m);
    const int e = __builtin_amdgcn_frexp_expf(m) - 1;
    const int X = ok ? static_cast<int>(rintf(ldexpf(x, 21 - e))) : 0;
    const int b0 = (X << 24) >> 24;
    const int X1 = (X - b0) >> 8;
    const int b1 = (X1 << 24) >> 24;
    const int b2 = (X1 - b1) >> 8;
    const int sh = 8 * (lane & 3);
    uint32_t u0 = (static_cast<uint32_t>(b0) & 0xFFu) << sh;
    uint32_t u1 = (static_cast<uint32_t>(b1) & 0xFFu) << sh;
    uint32_t u2 = (static_cast<uint32_t>(b2) & 0xFFu) << sh;
    #pragma unroll
    for (int off = 1; off < 4; off <<= 1) {
        u0 |= __shfl_xor(u0, off);
        u1 |= __shfl_xor(u1, off);
        u2 |= __shfl_xor(u2, off);
    }
    // Dword k of limb set j sits in lanes 4k..4k+3 of u_j.
    const int k = lane & 3;
    const uint32_t d0 = __shfl(u0, 4 * k), d1 = __shfl(u1, 4 * k), d2 = __shfl(u2, 4 * k);
    const float scale = ok ? ldexpf(1.f, e - 21) : (m == 0.f ? 0.f : __builtin_nanf(""));
    uint32_t word = 0;
    if (lane < 4) word = d0;
    else if (lane < 8) word = d1;
    else if (lane < 12) word = d2;
    else if (lane == 12) word = __builtin_bit_cast(uint32_t, scale);
    else if (lane == 13) word = __builtin_bit_cast(uint32_t, sum);
    if (in) reinterpret_cast<uint32_t *>(dst)[lane] = word;
    if (ss && lane == 0) *ss = sq;
}

// Columns a MERGE kernel stages (its records live in LDS).
constexpr int kRecMergeCols = 2048;

template <int TYPE, int G, bool EPI, int D, bool MERGE>
__device__ __forceinline__ void rec_body(const RecParams &p) {
    __shared__ float part[2 * kRecRows * kRecMaxChunks];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = p.waves;   // not blockDim.x: that reads the dispatch packet before any other load
    const int P = p.pieces;
    const int C = P / G;
    const int nm = p.pair ? 2 : 1;
    const int q0 = wave * 64 + lane;
    const int piece = q0 % P;
    // Step s of a block puts the lane on row s * step_rows + ri0 of it (64 W
    // is a multiple of P, so the lane's piece never changes).
    const int step_rows = 64 * W / P, ri0 = q0 / P;
    const int sl2 = p.steps_log2, smask = p.steps - 1;
    const int g = (piece >> 1) & 1, h = piece & 1;
    const bool head = (lane & (G - 1)) == 0;   // the lane that holds its group's sum

    // Every load below is unconditional (indices clamped into range), so no
    // branch makes a wave wait for the loads in flight.  The first D tiles'
    // weight loads go out first, then the block's residual inputs and gains,
    // the activation records and the sums of squares.
    // Tile k of this wave: block blockIdx.x + (k / steps) * gridDim.x, step k % steps.
    const int my_blocks = static_cast<int>(blockIdx.x) < p.n_blocks
                              ? (p.n_blocks - 1 - static_cast<int>(blockIdx.x)) / static_cast<int>(gridDim.x) + 1
                              : 0;
    const int n_iter = my_blocks * p.steps;
    auto fetch = [&](int k) {
        const int blk = static_cast<int>(blockIdx.x) + (k >> sl2) * static_cast<int>(gridDim.x);
        return rec_fetch<TYPE>(p, blk, (k & smask) * step_rows + ri0, piece, g, h, !EPI && head && p.accumulate);
    };
    const int last = max(n_iter - 1, 0);
    // MERGE: the partials' loads go out ahead of the weights'.
    PartsEarly pe;
    if constexpr (MERGE) parts_load(pe, p.parts, p.n_parts, p.part_hd, p.nb * 256, threadIdx.x, W * 64);
    RecSlot sl[D];
    #pragma unroll
    for (int i = 0; i < D; ++i) sl[i] = fetch(min(i, last));
    // With EPI, thread t < nm * kRecRows finishes row t of each block: it
    // reads the row's residual input one block ahead (never with pair).  The
    // matrix index stays wave-uniform, so its fields are scalar loads.
    auto load_yold = [&](int blk) -> float {
        if (!EPI || p.pair || !p.accumulate || blk >= p.n_blocks) return 0.f;
        int m, row0;
        rec_block(p, blk, 0, m, row0);
        const RecMatrix M = rec_mat(p, __builtin_amdgcn_readfirstlane(m));
        row0 = __builtin_amdgcn_readfirstlane(row0);
        return M.y[min(row0 + static_cast<int>(threadIdx.x & (kRecRows - 1)), M.rows - 1)];
    };
    float yold_blk = load_yold(blockIdx.x);
    // Output records of y * gain: lane t < 16 of wave 0 holds the gain of
    // row t of its block, read one block ahead.
    auto load_gain = [&](int blk) -> float {
        if (!EPI || !p.gain || blk >= p.n_blocks) return 1.f;
        return p.gain[blk * kRecRows + (threadIdx.x & (kRecRows - 1))];   // one matrix: block_begin 0
    };
    float gain_blk = load_gain(blockIdx.x);
    // Each lane reads its piece's four records straight from memory (they
    // stay in L1 / L2 for the workgroup's other lanes), and the sums of
    // squares, with no LDS copy and no barrier before the first dot.
    F32Policy::Lane L;
    if constexpr (MERGE) {
        // The row merged into LDS, then its records made there (one per
        // thread, make_group_tree: the records the attention's own epilogue
        // would have written), then each lane's four read back.
        __shared__ float xs[kRecMergeCols];
        __shared__ XGroup recs[kRecMergeCols / 16];
        const int cols = p.nb * 256, n4 = cols / 4;
        #pragma unroll
        for (int k = 0; k < kPartsHeld; ++k) {
            const int i = static_cast<int>(threadIdx.x) + k * W * 64;
            if (i < n4) reinterpret_cast<float4 *>(xs)[i] = parts_merge(pe, k, p.n_parts);
        }
        __syncthreads();
        for (int gi = threadIdx.x; gi < cols / 16; gi += W * 64) {
            float v[16];
            load16f(xs + 16 * gi, v);
            recs[gi] = make_group_tree(v);
        }
        __syncthreads();
        #pragma unroll
        for (int part_i = 0; part_i < 4; ++part_i) F32Policy::set_part(L, part_i, recs[F32Policy::group_of(piece, part_i)]);
    } else {
        #pragma unroll
        for (int part_i = 0; part_i < 4; ++part_i)
            F32Policy::set_part(L, part_i, p.rec[F32Policy::group_of(piece, part_i)]);
    }
    const float *ssp = p.ss ? p.ss : reinterpret_cast<const float *>(p.rec);   // any readable address
    float ssv[kRecSsPerLane];
    if constexpr (!MERGE) {   // (MERGE launches take no sums of squares)
        #pragma unroll
        for (int i = 0; i < kRecSsPerLane; ++i) ssv[i] = ssp[min(lane + 64 * i, p.nb * 16 - 1)];
    }
    float nscale = 1.f;
    if (!MERGE && p.ss) {
        float acc = 0.f;
        #pragma unroll
        for (int i = 0; i < kRecSsPerLane; ++i) acc += lane + 64 * i < p.nb * 16 ? ssv[i] : 0.f;
        #pragma unroll
        for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
        nscale = 1.0f / sqrtf(acc / static_cast<float>(p.nb * 256) + p.norm_eps);
    }
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;

    auto block_epilogue = [&](int blk) {
        __syncthreads();
        const int t = threadIdx.x;
        float v = 0.f;
        if (t < nm * kRecRows) {
            // The block's matrix (wave-uniform); with pair, rows t >= 16 go
            // to matrix 1 (selected, not indexed, to keep scalar loads).
            int m, row0;
            rec_block(p, blk, 0, m, row0);
            const RecMatrix M = rec_mat(p, __builtin_amdgcn_readfirstlane(m));
            row0 = __builtin_amdgcn_readfirstlane(row0);
            float *ybase = p.pair && t >= kRecRows ? p.mat[1].y : M.y;
            const int rows = M.rows;
            const int row = row0 + (t & (kRecRows - 1));
            for (int c = 0; c < C; ++c) v += part[t * C + c];
            v *= nscale;
            if (p.accumulate) v += yold_blk;
            yold_blk = load_yold(blk + gridDim.x);
            if (row < rows) {
                ybase[row] = v;
                if (p.arg_v) arg_better(bv, bi, v, row);
            } else {
                v = 0.f;
            }
        }
        if (p.rec_out && wave == 0) {
            // Lanes 0..15 of wave 0 hold the block's 16 values (gate rows;
            // up rows in lanes 16..31 with pair) and make its record together.
            float x;
            if (p.pair) {
                x = silu_mul_value(v, __shfl(v, (lane + kRecRows) & 63));
            } else {
                x = v * gain_blk;
                gain_blk = load_gain(blk + gridDim.x);
            }
            const int rec_index = blk;   // one matrix (block_begin 0) or the pair
            record16(x, v * v, lane, p.rec_out + rec_index, p.pair ? nullptr : p.ss_out + rec_index);
        }
        __syncthreads();   // part is reused by the next block
    };

    auto consume = [&](const RecSlot &t, int k) {
        const RecMatrix M = rec_mat(p, t.m);
        float v = group_sum<G>(piece_dot<F32Policy, TYPE>(M.type, t.r, L, g, h));
        const int s = k & smask;
        if constexpr (EPI) {
            if (head) part[(s * step_rows + ri0) * C + piece / G] = v;
            if (s == smask)
                block_epilogue(static_cast<int>(blockIdx.x) + (k >> sl2) * static_cast<int>(gridDim.x));
        } else {
            if (head && t.row < M.rows) {
                v *= nscale;
                if (p.accumulate) v += t.yold;
                M.y[t.row] = v;
                if (p.arg_v) arg_better(bv, bi, v, t.row);
            }
        }
    };

    // D tiles in flight: tile k + D is fetched as tile k is consumed (past
    // the wave's last tile the last one is fetched again, unconditionally).
    for (int k = 0; k < n_iter; k += D) {
        #pragma unroll
        for (int i = 0; i < D; ++i) {
            if (k + i < n_iter) {
                consume(sl[i], k + i);
                sl[i] = fetch(min(k + i + D, last));
            }
        }
    }
    if (p.arg_v) {
        #pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            arg_better(bv, bi, ov, oi);
        }
        if (lane == 0) {
            p.arg_v[blockIdx.x * W + wave] = bv;
            p.arg_i[blockIdx.x * W + wave] = bi;
        }
    }
}

// TYPE 0 (Q4_K and split Q6_K matrices in one launch): one row block per
// workgroup, run by the body of its matrix's type.
template <int TYPE, int G, bool EPI, int D>
__global__ __launch_bounds__(kRecMaxWaves * 64) void rec_gemv(RecParams p) {
    if constexpr (TYPE != 0) {
        rec_body<TYPE, G, EPI, D, false>(p);
    } else {
        int m, row0;
        rec_block(p, blockIdx.x, 0, m, row0);
        const int type = __builtin_amdgcn_readfirstlane(rec_mat(p, __builtin_amdgcn_readfirstlane(m)).type);
        if (type == QK_TYPE_Q4_K)
            rec_body<QK_TYPE_Q4_K, G, EPI, D, false>(p);
        else
            rec_body<QK_TYPE_Q6_K_SPLIT, G, EPI, D, false>(p);
    }
}

// The one-sequence o projection over the attention's unmerged splits (one
// matrix, one type, output records).
template <int TYPE, int G, int D>
__global__ __launch_bounds__(kRecMaxWaves * 64) void rec_gemv_merge(RecParams p) {
    rec_body<TYPE, G, true, D, true>(p);
}

// Waves per workgroup W and steps S of a launch: W * S = (pair ? 2 : 1) * nb
// with 64 W a multiple of P = 4 nb (S divides 16 * (pair ? 2 : 1)), the
// fewest steps that keep W <= kRecMaxWaves (up to kRecDepth steps, every
// tile's loads go out at once), and at most kRecMaxChunks group sums per
// row.  False when no such plan exists.
bool rec_plan(int nb, bool pair, int &waves, int &steps, int &group) {
    const int units = (pair ? 2 : 1) * nb;
    group = gcd_int(4 * nb, 64);
    if ((4 * nb) / group > kRecMaxChunks) return false;
    if (nb * 16 > 64 * kRecSsPerLane) return false;   // the sums of squares fit kRecSsPerLane per lane
    // A gate/up pair runs four steps per wave (one 32-row block per 4-wave
    // workgroup, 512 of them at 1B shapes: 11.5 us against 12.4 with 8-wave
    // workgroups of two blocks each); the others two (o 5.0 us, 6.3 at four).
    const int pair_order[5] = {4, 2, 1, 8, 16}, order[5] = {2, 1, 4, 8, 16};
    for (int s : (pair ? pair_order : order)) {
        if (units % s || (16 * (pair ? 2 : 1)) % s) continue;
        const int w = units / s;
        if (w < 1 || w > kRecMaxWaves) continue;
        waves = w;
        steps = s;
        return true;
    }
    return false;
}

template <int TYPE, bool EPI, int D>
const void *rec_kernel_g(int group) {
    switch (group) {
        case 4: return reinterpret_cast<const void *>(rec_gemv<TYPE, 4, EPI, D>);
        case 8: return reinterpret_cast<const void *>(rec_gemv<TYPE, 8, EPI, D>);
        case 16: return reinterpret_cast<const void *>(rec_gemv<TYPE, 16, EPI, D>);
        case 32: return reinterpret_cast<const void *>(rec_gemv<TYPE, 32, EPI, D>);
        default: return reinterpret_cast<const void *>(rec_gemv<TYPE, 64, EPI, D>);
    }
}

template <int TYPE>
const void *rec_kernel_t(int group, bool epi, bool deep) {
    if (deep) return epi ? rec_kernel_g<TYPE, true, 4>(group) : rec_kernel_g<TYPE, false, 4>(group);
    return epi ? rec_kernel_g<TYPE, true, 2>(group) : rec_kernel_g<TYPE, false, 2>(group);
}

const void *rec_merge_kernel(int type, int group, bool deep) {
    if (group != 32) return nullptr;   // rows of 2048 columns
    if (type == QK_TYPE_Q4_K)
        return deep ? reinterpret_cast<const void *>(rec_gemv_merge<QK_TYPE_Q4_K, 32, 4>)
                    : reinterpret_cast<const void *>(rec_gemv_merge<QK_TYPE_Q4_K, 32, 2>);
    if (type == QK_TYPE_Q6_K_SPLIT)
        return deep ? reinterpret_cast<const void *>(rec_gemv_merge<QK_TYPE_Q6_K_SPLIT, 32, 4>)
                    : reinterpret_cast<const void *>(rec_gemv_merge<QK_TYPE_Q6_K_SPLIT, 32, 2>);
    return nullptr;
}

const void *rec_kernel(int type, int group, bool epi, bool deep) {
    return type == QK_TYPE_Q4_K         ? rec_kernel_t<QK_TYPE_Q4_K>(group, epi, deep)
           : type == QK_TYPE_Q6_K_SPLIT ? rec_kernel_t<QK_TYPE_Q6_K_SPLIT>(group, epi, deep)
                                        : rec_kernel_t<0>(group, epi, deep);
}

// ------------------------------------------------ no-allocation variant --
//
// Scratch of qk_gemv_argmax_f32_noalloc: the per-wave (value, row) partials
// of the LM head's greedy-pick epilogue, kArgPartsMax of each, in a
// file-scope device array -- one copy per GPU, held until the process ends.
// On the host `scratch` names a host-side stand-in, not device memory: host
// code uses only the address hipGetSymbolAddress returns for the current
// device, looked up once per device and kept.
constexpr size_t kNoAllocScratchBytes = 2 * kArgPartsMax * sizeof(float);
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

int scratch_address(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0)
        return fail(QK_ERR_DEVICE, "qk_gemv_argmax_f32_noalloc: no current device");
    static std::mutex mutex;
    static std::vector<void *> addr;   // by device ordinal
    std::lock_guard<std::mutex> lock(mutex);
    if (static_cast<size_t>(dev) >= addr.size()) addr.resize(dev + 1, nullptr);
    if (!addr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
            return fail(QK_ERR_DEVICE, "qk_gemv_argmax_f32_noalloc: cannot resolve the scratch array on device " +
                                           std::to_string(dev));
        addr[dev] = p;
    }
    *out = addr[dev];
    return QK_OK;
}

}  // namespace

// FP32 path shared by the single, fused and few-token entry points (arguments
// already validated).  ldy: per-matrix token stride of y, or NULL for rows.
int launch_gemv_f32(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                    const int *ldy, hipStream_t stream) {
    GemvParams p{};
    p.x = x;
    p.ldx = ldx;
    return launch<F32Policy>(p, mats, n_mats, cols, n_tokens, ldy, stream, "qk_gemv_f32 launch");
}

// INT8 path shared by qk_gemv_i8 and qk_gemv_multi_i8 (arguments already
// validated): quantized activations xq / xscale of n_tokens tokens.
int launch_gemv_i8(const qk_matrix *mats, int n_mats, const int8_t *xq, int ldxq, const float *xscale, int ldscale,
                   int cols, int n_tokens, const int *ldy, int accumulate, hipStream_t stream) {
    GemvParams p{};
    p.x = xq;
    p.xscale = xscale;
    p.ldx = ldxq;
    p.ldscale = ldscale;
    p.accumulate = accumulate;
    return launch<I8Policy>(p, mats, n_mats, cols, n_tokens, ldy, stream, "INT8 GEMV launch");
}

int launch_gemv_i8_argmax(const qk_matrix *mat, const int8_t *xq, const float *xscale, int cols, float *arg_v,
                          int *arg_i, int *parts, hipStream_t stream) {
    GemvParams p{};
    p.x = xq;
    p.xscale = xscale;
    p.ldx = cols;
    p.ldscale = cols / 32;
    p.arg_v = arg_v;
    p.arg_i = arg_i;
    p.grid_out = parts;
    return launch<I8ArgPolicy>(p, mat, 1, cols, 1, nullptr, stream, "INT8 GEMV + greedy pick launch");
}

int launch_gemv_i8_staged_argmax(const qk_matrix *mat, const float *x, const float *norm_w, float eps, int cols,
                                 float *arg_v, int *arg_i, int *parts, hipStream_t stream) {
    GemvParams p{};
    p.x = x;
    p.ldx = cols;
    p.norm_w = norm_w;
    p.norm_eps = eps;
    p.arg_v = arg_v;
    p.arg_i = arg_i;
    p.grid_out = parts;
    return launch<I8FusedArgPolicy>(p, mat, 1, cols, 1, nullptr, stream, "staged INT8 GEMV + greedy pick launch");
}

// The INT8 GEMV quantizing its own input (I8FusedPolicy): fp32 rows x of
// n_tokens tokens, RMSNorm'd with norm_w (eps) or multiplied by SiLU with up
// (same strides as x) first when either is set.
int launch_gemv_i8_staged(const qk_matrix *mats, int n_mats, const float *x, int ldx, const float *norm_w, float eps,
                          const float *up, int cols, int n_tokens, const int *ldy, int accumulate,
                          hipStream_t stream) {
    GemvParams p{};
    p.x = x;
    p.ldx = ldx;
    p.norm_w = norm_w;
    p.norm_eps = eps;
    p.up = up;
    p.accumulate = accumulate;
    return launch<I8FusedPolicy>(p, mats, n_mats, cols, n_tokens, ldy, stream, "staged INT8 GEMV launch");
}

bool gemv_i8_mergeable(int cols, int head_dim, int n_parts) {
    const int pieces = cols / 256 * 4;
    return cols > 0 && cols % 256 == 0 && cols <= kPartsHeld * 4 * 256 && 64 % pieces == 0 && head_dim > 0 &&
           head_dim % 4 == 0 && cols % head_dim == 0 && n_parts >= 1 && n_parts <= kMaxParts;
}

int launch_gemv_i8_merged(const qk_matrix *mats, int n_mats, const float *parts, int n_parts, int head_dim, int cols,
                          int accumulate, hipStream_t stream) {
    if (!gemv_i8_mergeable(cols, head_dim, n_parts))
        return fail(QK_ERR_LIMIT, "merged INT8 GEMV: unsupported shape");
    GemvParams p{};
    p.x = parts;
    p.parts = parts;
    p.n_parts = n_parts;
    p.part_hd = head_dim;
    p.accumulate = accumulate;
    return launch<I8MergePolicy>(p, mats, n_mats, cols, 1, nullptr, stream, "merged INT8 GEMV launch");
}

template <int TYPE>
int launch_pair_quant_type(const GemvParams &p, int group, int n_tokens, int8_t *hq, float *hs, int ldq, int ldsc,
                           size_t lds, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(p.mat[0].rows / 32), static_cast<unsigned>(n_tokens));
    if (group == 4)
        hipLaunchKernelGGL((gemv_pair_quant<I8FusedPolicy, TYPE, 4>), grid, dim3(pair_waves(4) * 64), lds, stream, p, hq,
                           hs, ldq, ldsc);
    else if (group == 8)
        hipLaunchKernelGGL((gemv_pair_quant<I8FusedPolicy, TYPE, 8>), grid, dim3(pair_waves(8) * 64), lds, stream, p, hq,
                           hs, ldq, ldsc);
    else if (group == 16)
        hipLaunchKernelGGL((gemv_pair_quant<I8FusedPolicy, TYPE, 16>), grid, dim3(pair_waves(16) * 64), lds, stream, p, hq,
                           hs, ldq, ldsc);
    else if (group == 32)
        hipLaunchKernelGGL((gemv_pair_quant<I8FusedPolicy, TYPE, 32>), grid, dim3(pair_waves(32) * 64), lds, stream, p, hq,
                           hs, ldq, ldsc);
    else
        hipLaunchKernelGGL((gemv_pair_quant<I8FusedPolicy, TYPE, 64>), grid, dim3(pair_waves(64) * 64), lds, stream, p, hq,
                           hs, ldq, ldsc);
    return launch_status("INT8 gate / up pair launch");
}

bool gemv_i8_pair_supported(int cols, int rows) {
    const int pieces = cols / 256 * 4;
    return cols > 0 && cols % 256 == 0 && 64 % pieces == 0 && rows > 0 && rows % 32 == 0 &&
           gemv_i8_stageable(cols);
}

int launch_gemv_i8_pair_quant(const qk_matrix *gu, const float *x, int ldx, const float *norm_w, float eps, int cols,
                              int n_tokens, int8_t *hq, float *hs, int ldq, int ldsc, hipStream_t stream) {
    const int rows = gu[0].rows, type = gu[0].type;
    if (!gemv_i8_pair_supported(cols, rows) || gu[1].rows != rows || gu[1].type != type || n_tokens > 65535)
        return fail(QK_ERR_LIMIT, "INT8 gate / up pair: unsupported shape");
    GemvParams p{};
    p.x = x;
    p.ldx = ldx;
    p.norm_w = norm_w;
    p.norm_eps = eps;
    const int nb = cols / 256;
    p.n_mats = 2;
    p.pieces = 4 * nb;
    p.group_lanes = p.pieces;
    p.tile_rows = 64 / p.pieces;
    p.chunks = 1;
    for (int m = 0; m < 2; ++m) {
        GemvMatrix &M = p.mat[m];
        M.w = static_cast<const uint8_t *>(gu[m].w);
        M.y = nullptr;
        M.rows = rows;
        M.type = type;
        M.row_bytes = static_cast<int>(row_bytes(type, nb));
        M.ldy = rows;
        M.tile_begin = m * (rows / p.tile_rows);
    }
    p.total_tiles = 2 * (rows / p.tile_rows);
    const size_t lds = ((I8FusedPolicy::lds_bytes(cols) + 15) & ~size_t(15)) + 64 * sizeof(float);
    if (type == QK_TYPE_Q4_K)
        return launch_pair_quant_type<QK_TYPE_Q4_K>(p, p.pieces, n_tokens, hq, hs, ldq, ldsc, lds, stream);
    if (type == QK_TYPE_Q6_K)
        return launch_pair_quant_type<QK_TYPE_Q6_K>(p, p.pieces, n_tokens, hq, hs, ldq, ldsc, lds, stream);
    return launch_pair_quant_type<QK_TYPE_Q6_K_SPLIT>(p, p.pieces, n_tokens, hq, hs, ldq, ldsc, lds, stream);
}

bool gemv_i8_stageable(int cols) {
    if (cols <= 0 || cols % 256) return false;
    const int pieces = cols / 64;
    return pieces / gcd_int(pieces, 64) <= kMaxChunks && I8FusedPolicy::lds_bytes(cols) + 4096 <= kMaxLds;
}

bool gemv_fusable(int cols) {
    if (cols <= 0 || cols % 256) return false;
    const int pieces = cols / 64;
    const int chunks = pieces / gcd_int(pieces, 64);
    return chunks <= kMaxChunks && F32FusedPolicy::lds_bytes(cols) + 4096 <= kMaxLds;
}

bool rec_gemv_mergeable(int cols, int head_dim) {
    int W, S, G;
    return cols % 256 == 0 && cols <= kRecMergeCols && rec_plan(cols / 256, false, W, S, G) && G == 32 &&
           W * 64 * kPartsHeld * 4 >= cols && head_dim > 0 && head_dim % 4 == 0 && cols % head_dim == 0;
}

bool rec_gemv_supported(int cols, bool pair) {
    int w, s, g;
    return cols > 0 && cols % 256 == 0 && rec_plan(cols / 256, pair, w, s, g);
}

bool rec_gemv_types(const qk_matrix *mats, int n_mats, bool pair) {
    // Q4_K and split Q6_K (the decode drivers repack every GGUF Q6_K tensor).
    if (n_mats < 1 || n_mats > kRecMaxMats) return false;
    bool mixed = false;
    for (int m = 0; m < n_mats; ++m) {
        if (mats[m].type != QK_TYPE_Q4_K && mats[m].type != QK_TYPE_Q6_K_SPLIT) return false;
        mixed |= mats[m].type != mats[0].type;
    }
    return !pair || (n_mats == 2 && !mixed);
}

int launch_rec_gemv(const qk_matrix *mats, int n_mats, int cols, const RecGemv &r, hipStream_t stream) {
    const int nb = cols / 256;
    int W, S, G;
    if (n_mats < 1 || n_mats > kRecMaxMats || !rec_plan(nb, r.pair, W, S, G))
        return fail(QK_ERR_LIMIT, "record GEMV: unsupported launch");
    if (r.pair && (n_mats != 2 || mats[0].rows != mats[1].rows))
        return fail(QK_ERR_INVALID_ARG, "record GEMV: a SiLU pair is two matrices of equal rows");
    if (!rec_gemv_types(mats, n_mats, r.pair))
        return fail(QK_ERR_TYPE, "record GEMV: unsupported matrix types");
    if (r.rec_out && !r.pair && (n_mats != 1 || mats[0].rows % kRecRows))
        return fail(QK_ERR_INVALID_ARG, "record GEMV: output records need one matrix of whole 16-row blocks");
    RecParams p{};
    p.n_mats = n_mats;
    p.pair = r.pair;
    p.nb = nb;
    p.pieces = 4 * nb;
    p.steps = S;
    p.steps_log2 = __builtin_ctz(static_cast<unsigned>(S));
    p.waves = W;
    int64_t blocks = 0;
    int type = mats[0].type;
    for (int m = 0; m < n_mats; ++m) {
        RecMatrix &M = p.mat[m];
        M.w = static_cast<const uint8_t *>(mats[m].w);
        M.y = mats[m].y;
        M.rows = mats[m].rows;
        M.type = mats[m].type;
        M.row_bytes = static_cast<int>(row_bytes(M.type, nb));
        M.block_begin = static_cast<int>(blocks);
        if (!r.pair || m == 0) blocks += (M.rows + kRecRows - 1) / kRecRows;
        if (static_cast<int64_t>(M.rows) * M.row_bytes > (int64_t(1) << 40))
            return fail(QK_ERR_LIMIT, "record GEMV: matrix too large");
        if (M.type != type) type = 0;
    }
    if (blocks > (1 << 30)) return fail(QK_ERR_LIMIT, "record GEMV: too many rows");
    p.n_blocks = static_cast<int>(blocks);
    p.rec = r.rec;
    p.ss = r.ss;
    p.norm_eps = r.norm_eps;
    p.accumulate = r.accumulate;
    p.rec_out = r.rec_out;
    p.ss_out = r.ss_out;
    p.gain = r.gain;
    p.arg_v = r.arg_v;
    p.arg_i = r.arg_i;
    const bool epi = (4 * nb) / G > 1 || r.rec_out || r.pair;
    if (r.parts) {
        // o over the attention's unmerged splits: one matrix of one type,
        // output records, one row block per workgroup, all resident.
        const void *fn2 = type == 0 ? nullptr : rec_merge_kernel(type, G, false);
        if (!fn2 || !r.rec_out || r.pair || r.arg_v || r.ss || cols > kRecMergeCols ||
            W * 64 * kPartsHeld * 4 < cols || r.n_parts < 1 || r.n_parts > kMaxParts || r.part_hd <= 0 ||
            r.part_hd % 4 || cols % r.part_hd)
            return fail(QK_ERR_LIMIT, "record GEMV: unsupported merged launch");
        p.parts = r.parts;
        p.n_parts = r.n_parts;
        p.part_hd = r.part_hd;
        p.rec = reinterpret_cast<const XGroup *>(r.parts);   // any readable address (the unused loads)
        const bool deep = S > 2;
        const void *fn = rec_merge_kernel(type, G, deep);
        const int grid = static_cast<int>(blocks);
        if (resident_blocks(fn, W * 64, 0) < grid)
            return fail(QK_ERR_LIMIT, "record GEMV: merged launch does not fit in one round");
        void *args[] = {&p};
        if (hipLaunchKernel(fn, dim3(grid), dim3(W * 64), args, 0, stream) != hipSuccess)
            return launch_status("merged record GEMV launch");
        return launch_status("merged record GEMV launch");
    }
    // One row block per workgroup when they all fit at once (always for
    // mixed types); grid-stride otherwise (the LM head), within the argmax
    // partials' buffer.  Two tiles in flight per wave when a wave has no
    // more, four otherwise.
    // A grid-stride launch (more blocks than resident workgroups: the LM
    // head) runs the two-deep kernel, whose fewer registers fit one more
    // workgroup per CU: more waves keep more loads in flight than deeper
    // prefetch per wave (LM head 128256 x 2048: 48.9 us with four tiles in
    // flight at 3 workgroups per CU).
    const int deep_resident = type == 0 ? 0 : resident_blocks(rec_kernel(type, G, epi, true), W * 64, 0);
    const bool strided = type != 0 && blocks > deep_resident;
    int grid = type == 0 ? static_cast<int>(blocks)
               : static_cast<int>(std::min<int64_t>(
                     blocks, strided ? resident_blocks(rec_kernel(type, G, epi, false), W * 64, 0) : deep_resident));
    if (r.arg_v) {
        if (type == 0 && grid > kArgPartsMax / W)
            return fail(QK_ERR_LIMIT, "record GEMV: too many argmax partials for mixed types");
        grid = std::min(grid, kArgPartsMax / W);
    }
    grid = std::max(grid, 1);
    const int64_t tiles_per_wave = (blocks + grid - 1) / grid * S;
    const void *fn = rec_kernel(type, G, epi, !strided && tiles_per_wave > 2);
    if (r.arg_parts) *r.arg_parts = grid * W;
    void *args[] = {&p};
    if (hipLaunchKernel(fn, dim3(grid), dim3(W * 64), args, 0, stream) != hipSuccess)
        return launch_status("record GEMV launch");
    return launch_status("record GEMV launch");
}

int launch_gemv_fused(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                      const int *ldy, const GemvFusion &f, hipStream_t stream) {
    if (!gemv_fusable(cols)) return fail(QK_ERR_LIMIT, "fused GEMV: rows too long to stage the activations");
    GemvParams p{};
    p.x = x;
    p.ldx = ldx;
    p.norm_w = f.norm_w;
    p.norm_eps = f.norm_eps;
    p.up = f.up;
    p.accumulate = f.accumulate;
    if (f.arg_v) {
        if (!f.arg_i || !f.arg_parts || n_mats != 1 || n_tokens != 1)
            return fail(QK_ERR_INVALID_ARG, "fused GEMV: the argmax epilogue takes one matrix and one token");
        p.arg_v = f.arg_v;
        p.arg_i = f.arg_i;
        p.grid_out = f.arg_parts;
        *f.arg_parts = 0;
    }
    const int st = f.arg_v ? launch<F32ArgPolicy>(p, mats, n_mats, cols, n_tokens, ldy, stream, "fused GEMV launch")
                           : launch<F32FusedPolicy>(p, mats, n_mats, cols, n_tokens, ldy, stream, "fused GEMV launch");
    if (!st && f.arg_v && (*f.arg_parts < 1 || *f.arg_parts > kArgPartsMax))
        return fail(QK_ERR_LIMIT, "fused GEMV: argmax partials beyond their buffer");
    return st;
}

}  // namespace qk

extern "C" {

int qk_gemv_f32(int type, const void *w, const float *x, float *y, int cols, int rows, qk_stream stream) {
    int st = qk::check_weights("qk_gemv_f32", type, w, cols, rows);
    if (st) return st;
    if (!x || !y) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_f32: null activation or output pointer");
    if (!qk::aligned(x, 16) || !qk::aligned(y, 4))
        return qk::fail(QK_ERR_ALIGN, "qk_gemv_f32: x must be 16-byte and y 4-byte aligned");
    const qk_matrix m{type, rows, w, y};
    return qk::launch_gemv_f32(&m, 1, x, cols, cols, 1, nullptr, static_cast<hipStream_t>(stream));
}

size_t qk_gemv_argmax_workspace_bytes(void) { return 2 * qk::kArgPartsMax * sizeof(float); }

int qk_gemv_argmax_f32(int type, const void *w, const float *x, float *y, int cols, int rows, int32_t *out,
                       void *workspace, qk_stream stream) {
    int st = qk::check_weights("qk_gemv_argmax_f32", type, w, cols, rows);
    if (st) return st;
    if (!x || !y || !out || !workspace)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_argmax_f32: null activation, output or workspace pointer");
    if (!qk::aligned(x, 16) || !qk::aligned(y, 4) || !qk::aligned(workspace, 4))
        return qk::fail(QK_ERR_ALIGN, "qk_gemv_argmax_f32: x must be 16-byte, y and workspace 4-byte aligned");
    if (!qk::gemv_fusable(cols)) return qk::fail(QK_ERR_LIMIT, "qk_gemv_argmax_f32: rows too long to stage");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const qk_matrix m{type, rows, w, y};
    qk::GemvFusion f;
    f.arg_v = static_cast<float *>(workspace);
    f.arg_i = reinterpret_cast<int *>(f.arg_v + qk::kArgPartsMax);
    int parts = 0;
    f.arg_parts = &parts;
    if ((st = qk::launch_gemv_fused(&m, 1, x, cols, cols, 1, nullptr, f, s))) return st;
    return qk::launch_argmax_final(f.arg_v, f.arg_i, parts, out, s);
}

int qk_gemv_argmax_f32_noalloc(int type, const void *w, const float *x, float *y, int cols, int rows, int32_t *out,
                               qk_stream stream) {
    int st = qk::check_weights("qk_gemv_argmax_f32_noalloc", type, w, cols, rows);
    if (st) return st;
    if (!x || !y || !out)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_argmax_f32_noalloc: null activation or output pointer");
    if (!qk::aligned(x, 16) || !qk::aligned(y, 4))
        return qk::fail(QK_ERR_ALIGN, "qk_gemv_argmax_f32_noalloc: x must be 16-byte and y 4-byte aligned");
    if (!qk::gemv_fusable(cols)) return qk::fail(QK_ERR_LIMIT, "qk_gemv_argmax_f32_noalloc: rows too long to stage");
    void *ws = nullptr;
    if ((st = qk::scratch_address(&ws))) return st;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const qk_matrix m{type, rows, w, y};
    qk::GemvFusion f;
    f.arg_v = static_cast<float *>(ws);
    f.arg_i = reinterpret_cast<int *>(f.arg_v + qk::kArgPartsMax);
    int parts = 0;
    f.arg_parts = &parts;
    // The launch keeps its partials within kArgPartsMax (the grid is clamped)
    // and fails with QK_ERR_LIMIT otherwise, so the scratch always suffices.
    static_assert(qk::kNoAllocScratchBytes >= 2 * qk::kArgPartsMax * sizeof(float), "scratch holds every partial");
    if ((st = qk::launch_gemv_fused(&m, 1, x, cols, cols, 1, nullptr, f, s))) return st;
    return qk::launch_argmax_final(f.arg_v, f.arg_i, parts, out, s);
}

int qk_gemv_multi_f32(const qk_matrix *mats, int n_mats, const float *x, int cols, qk_stream stream) {
    if (!mats || n_mats < 1 || n_mats > QK_MAX_FUSED)
        return qk::fail(QK_ERR_INVALID_ARG,
                        "qk_gemv_multi_f32: need 1.." + std::to_string(QK_MAX_FUSED) + " matrices");
    if (!x) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_f32: null activation pointer");
    if (!qk::aligned(x, 16)) return qk::fail(QK_ERR_ALIGN, "qk_gemv_multi_f32: x must be 16-byte aligned");
    for (int m = 0; m < n_mats; ++m) {
        int st = qk::check_weights("qk_gemv_multi_f32", mats[m].type, mats[m].w, cols, mats[m].rows);
        if (st) return st;
        if (!mats[m].y) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_f32: null output pointer");
        if (!qk::aligned(mats[m].y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_gemv_multi_f32: misaligned output");
    }
    return qk::launch_gemv_f32(mats, n_mats, x, cols, cols, 1, nullptr, static_cast<hipStream_t>(stream));
}

int qk_gemv_i8(int type, const void *w, const int8_t *xq, int ldxq, const float *xscale, int ldscale, float *y,
               int ldy, int cols, int rows, int n_tokens, qk_stream stream) {
    int st = qk::check_weights("qk_gemv_i8", type, w, cols, rows);
    if (st) return st;
    if (!xq || !xscale || !y || n_tokens < 0)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_i8: null pointer or negative token count");
    if (n_tokens == 0) return qk::ok();
    if (ldxq < cols || ldscale < cols / 32 || ldy < rows)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_i8: leading dimension smaller than the row");
    if (!qk::aligned(xq, 16) || ldxq % 16 || !qk::aligned(xscale, 4) || !qk::aligned(y, 4))
        return qk::fail(QK_ERR_ALIGN, "qk_gemv_i8: xq and ldxq must keep 16-byte alignment");
    const qk_matrix m{type, rows, w, y};
    return qk::launch_gemv_i8(&m, 1, xq, ldxq, xscale, ldscale, cols, n_tokens, &ldy, 0,
                              static_cast<hipStream_t>(stream));
}

int qk_gemv_multi_i8(const qk_matrix *mats, int n_mats, const int8_t *xq, const float *xscale, int cols,
                     qk_stream stream) {
    if (!mats || n_mats < 1 || n_mats > QK_MAX_FUSED)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_i8: need 1.." + std::to_string(QK_MAX_FUSED) + " matrices");
    if (!xq || !xscale) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_i8: null activation pointer");
    if (!qk::aligned(xq, 16) || !qk::aligned(xscale, 4))
        return qk::fail(QK_ERR_ALIGN, "qk_gemv_multi_i8: xq must be 16-byte and xscale 4-byte aligned");
    int ldy[QK_MAX_FUSED];
    for (int m = 0; m < n_mats; ++m) {
        int st = qk::check_weights("qk_gemv_multi_i8", mats[m].type, mats[m].w, cols, mats[m].rows);
        if (st) return st;
        if (!mats[m].y) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_i8: null output pointer");
        if (!qk::aligned(mats[m].y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_gemv_multi_i8: misaligned output");
        ldy[m] = mats[m].rows;
    }
    return qk::launch_gemv_i8(mats, n_mats, xq, cols, xscale, cols / 32, cols, 1, ldy, 0,
                              static_cast<hipStream_t>(stream));
}

}  // extern "C"
