// qk_batched.hip - multi-token FP32 dequant-GEMV entry points.
//
// FP32 semantics for the reference's INT8-only batched path
// (FastRunner::batch_matvec + gemv_batch_dp4a, inferencer.cu:1265-1278,
// 678-699; qkv_batch_cuda / gate_up_batch_cuda, inferencer.cu:701-751).
// Token t reads x + t*ldx and writes y + t*ldy.
//
// Few tokens (< kMfmaMinTokens) run the batch-1 GEMV kernels with one grid
// column per token.  From kMfmaMinTokens on, the product is a dense
// contraction and runs on the matrix cores:
//
//   Y[t][r] = sum_b d_rb * sum_{c in b} W_int[r][c] * x[t][c]
//             - dmin_rb * sum_j m_rbj * X[t][b][j]          (Q4_K only)
//
// with W_int = sc*q (Q4_K, 0..945) or sc*(code-32) (Q6_K): integers that
// fp16 holds exactly while |sc| <= 62 (|W_int| <= 1984); a block with a
// wider Q6_K scale (real GGUF Q6_K tensors use the whole int8 range) carries
// each weight as an fp16 pair W_a + W_b and adds a third MFMA chain (W_b
// times the high halves; W_b x the low halves is below 2^-22 of the block's
// terms and is left out).  Activations are scaled per (token,
// block) by a power of two so the block maximum lies in [2^14, 2^15) and
// split into fp16 high and low halves (22 significant bits), so each block
// is two v_mfma_f32_32x32x16_f16 chains over exact operands; the block's d
// (and dmin with the sub-block sums X, through v_mfma_f32_32x32x8_f16) and
// the activation scale are applied in fp32 when the block is done.
//
// Three kernels:
//   pack_activations  once per (block, 8 tokens): x -> the record of
//                     MFMA A operands (fp16 hi / lo, sub-block sums, scales)
//                     in the caller's workspace.
//   batch_gemm        a workgroup (4 waves) owns 128 or 256 weight rows (one
//                     or two 32-row tiles per wave, as many as its token
//                     tiles) x one or two token tiles x a run of blocks.  Per block it copies the token tiles' records
//                     into LDS with direct global->LDS loads (double-buffered:
//                     the next block's records and weight bytes load while
//                     this block computes); each wave decodes the raw bytes of
//                     its rows into MFMA B operands in registers (lane l: row
//                     l%32, block half l/32), and every decoded operand feeds
//                     every token tile.  When one row group's blocks are split
//                     over several workgroups (to put enough waves on the
//                     chip), each writes its partial sums to the workspace;
//   reduce_splits     adds them in split order, so results are deterministic,
//                     and applies the call's epilogue (one thread per output).
#include "qk_internal.h"
#include "qk_records.h"

#include <algorithm>

namespace qk {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kMfmaMinTokens = 8;
// 32-row tiles per wave (RT): one for a single 32-token tile, two from two
// token tiles on, so a workgroup (4 waves) owns 128 * RT weight rows and
// writes 4 * RT * 1024 partial sums per token tile when blocks are split.
// Measured: one row tile at 32 tokens (two workgroups per CU share each
// SIMD's VALU and MFMA pipes) took the 32-sequence 1B step 2.15 -> 1.94 ms;
// at 256 tokens two row tiles stay faster (4.60 against 4.74-4.78 ms).
__host__ __device__ constexpr int group_rows(int rt) { return 128 * rt; }
__host__ __device__ constexpr int partial_floats(int rt) { return 4 * rt * 16 * 64; }
constexpr int kMaxSplit = 16;           // workgroups splitting one row group's blocks
static_assert(partial_floats(1) % 256 == 0, "reduce_splits covers whole partial slots with 256-thread workgroups");

// K order of the A / B operands inside a block.  Step s (0..15) and half kh
// (lane / 32) hold eight columns of the 64-column group G = 2*kh + s/8:
//   e 0..3: G*64 +      4*(s%8) + {0, 2, 1, 3}[e]
//   e 4..7: G*64 + 32 + 4*(s%8) + {0, 2, 1, 3}[e-4]
// i.e. the low nibbles (e < 4) and high nibbles (e >= 4) of Q4_K qs bytes
// G*32 + 4*(s%8) .. +3, even bytes first; Q6_K uses the same columns.

struct BatchMatrix {
    const uint8_t *w;
    float *y;
    int rows;
    int type;
    int row_bytes;
    int ldy;
    int group_begin;   // first row group (group_rows(RT) rows) of this matrix in the launch
};

struct BatchParams {
    BatchMatrix mat[QK_MAX_FUSED];
    int n_mats;
    const float *x;
    int ldx;
    int n_tokens;
    int nb;
    int tiles;
    int splits;             // workgroups sharing one row group's blocks
    int blocks_per_split;
    float *partials;        // [group][tile][split][partial_floats(RT)] when splits > 1
    const uint8_t *records; // packed activations, [tile][block][kTileBytes]
    // Decode-driver fusions (zero: plain x, overwrite y):
    const float *norm_w;    // stage RMSNorm(x) * norm_w
    float norm_eps;
    const float *up;        // stage x / (1 + exp(-x)) * up (up has x's layout)
    int accumulate;         // y += W x
    // Decode-driver chain (zero: none).  in_ss: per (token, input block) sums
    // of squares of the unnormalised input, whose RMSNorm is applied as an
    // output scale (W (s x * g) = s W (x * g)) where the outputs are final.
    const float *in_ss;
    // The reduction also packs the next GEMM's input into out_records
    // (out_nb blocks of 256 of this call's output rows per token): x * gain
    // with its sums of squares in out_ss when out_gain is set, SiLU(y0) * y1
    // of a gate / up pair (matrices 0 and 1) when pair is set.
    uint8_t *out_records;
    int out_nb;
    const float *out_gain;
    float *out_ss;
    int pair;
};

// ---------------------------------------------------- activation staging --
//
// One wave per (token, 256-column block): lane (q, j) = (lane / 8, lane % 8)
// stages columns q*32 + 4j .. +3 of the block (stage_store_wave's layout).

// The token's RMSNorm scale 1/sqrt(mean(x^2) + eps) over all cols
// (rmsnorm_cuda's arithmetic, inferencer.cu:821-834): each lane reads every
// 64th float4 of the row, all in flight at once (the kernel is
// latency-bound), and the lanes meet in six xor shuffles.
__device__ __forceinline__ float stage_norm_scale(const BatchParams &p, int t, int lane) {
    const int cols = p.nb * 256;
    float ss = 0.f;
    if (t < p.n_tokens) {
        const float4 *row = reinterpret_cast<const float4 *>(p.x + static_cast<int64_t>(t) * p.ldx);
        #pragma unroll 8
        for (int i = lane; i < cols / 4; i += 64) {
            const float4 v = row[i];
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
    }
    #pragma unroll
    for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
    return 1.0f / sqrtf(ss / static_cast<float>(cols) + p.norm_eps);
}

// The lane's four values of column c = b*256 + q*32 + 4j: x (times the
// token's RMSNorm scale and the gain with norm_w; x / (1 + exp(-x)) * up
// with up, silu_cuda, inferencer.cu:1053-1056); zero past the last token.
__device__ __forceinline__ void stage_load4(const BatchParams &p, int t, int c, float scale, float (&v)[4]) {
    v[0] = v[1] = v[2] = v[3] = 0.f;
    if (t >= p.n_tokens) return;
    const int64_t at = static_cast<int64_t>(t) * p.ldx + c;
    const float4 u = *reinterpret_cast<const float4 *>(p.x + at);
    v[0] = u.x;
    v[1] = u.y;
    v[2] = u.z;
    v[3] = u.w;
    if (p.norm_w) {
        const float4 w = *reinterpret_cast<const float4 *>(p.norm_w + c);
        v[0] = v[0] * scale * w.x;
        v[1] = v[1] * scale * w.y;
        v[2] = v[2] * scale * w.z;
        v[3] = v[3] * scale * w.w;
    }
    if (p.up) {
        const float4 w = *reinterpret_cast<const float4 *>(p.up + at);
        const float up4[4] = {w.x, w.y, w.z, w.w};
        #pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = v[k] / (1.f + expf(-v[k])) * up4[k];
    }
}

// One 256-thread workgroup per (block, four tokens of a 32-token tile), a
// wave per token: the tokens' activations of the block, packed into the
// workspace record the GEMM copies into LDS.
constexpr int kPackTokens = 4;
__global__ __launch_bounds__(256) void pack_activations(BatchParams p, uint8_t *__restrict__ records) {
    const int b = blockIdx.x;
    const int tile = blockIdx.y / (kTokTile / kPackTokens);
    const int tl = (blockIdx.y % (kTokTile / kPackTokens)) * kPackTokens + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t = tile * kTokTile + tl;
    const float scale = p.norm_w ? stage_norm_scale(p, t, lane) : 1.f;
    float v[4];
    stage_load4(p, t, b * 256 + (lane >> 3) * 32 + 4 * (lane & 7), scale, v);
    stage_store_wave(v, lane, tl, records + (static_cast<size_t>(tile) * p.nb + b) * kTileBytes);
}

// ------------------------------------------------------- weight operands --

// Raw bytes of one block of one row that lane half kh needs.
struct RawBlock {
    uint4 q[4];        // Q4_K: qs[kh*64 .. +64); Q6_K: ql[kh*64 .. +64)
    uint4 h[2];        // Q6_K: qh[kh*32 .. +32)
    uint4 hdr;         // Q4_K: d, dmin, scales; Q6_K: x, y = scales[kh*8 .. +8), z = d
};

template <int TYPE>
__device__ __forceinline__ bool is_q4(int type) {
    return TYPE == QK_TYPE_Q4_K || (TYPE == 0 && type == QK_TYPE_Q4_K);
}

// Block b of the row at `row` (nb blocks per row; Q6_K in the GGUF or the
// split layout).
template <int TYPE>
__device__ __forceinline__ RawBlock load_block(const uint8_t *row, int b, int nb, int type, int kh) {
    RawBlock r;
    if (is_q4<TYPE>(type)) {
        const uint8_t *blk = row + b * 144;
        r.hdr = load16(blk);
        #pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = load16(blk + 16 + kh * 64 + 16 * i);
        r.h[0] = r.h[1] = make_uint4(0, 0, 0, 0);
    } else {
        const bool split = TYPE == QK_TYPE_Q6_K_SPLIT || (TYPE == 0 && type == QK_TYPE_Q6_K_SPLIT);
        const Q6Fields f = q6_fields(row, nb, b, split);
        #pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = load16(f.ql + kh * 64 + 16 * i);
        r.h[0] = load16(f.qh + kh * 32);
        r.h[1] = load16(f.qh + kh * 32 + 16);
        const uint2 sc = load8(f.sc + kh * 8);
        r.hdr = make_uint4(sc.x, sc.y, load2(f.d), 0);
    }
    return r;
}

__device__ __forceinline__ uint32_t word(const uint4 *v, int i) {
    const uint4 &u = v[i >> 2];
    return (i & 3) == 0 ? u.x : (i & 3) == 1 ? u.y : (i & 3) == 2 ? u.z : u.w;
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Bytes 0 and 2 (sel 0x04020400) or 1 and 3 (sel 0x04030401) of v as the
// fp16 halves 0x64nn = 1024 + n, then fma(1024 + n, s, bias) with bias =
// -(1024 + offset) * s: the exact product (n - offset) * s, rounded once.
__device__ __forceinline__ uint32_t nib_h2(uint32_t v, uint32_t sel, half2v s, half2v bias) {
    const uint32_t h = __builtin_amdgcn_perm(0x64646464u, v, sel);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2v, h), s, bias));
}

// B operand of step j (0..7) of block half hf: eight exact fp16 integer
// weights in the K order above; (sa, ba) scale columns e < 4 and (sb, bb)
// columns e >= 4.
template <int TYPE>
__device__ __forceinline__ half8 decode_b(const RawBlock &r, int type, int hf, int j, half2v sa, half2v ba,
                                          half2v sb, half2v bb) {
    uint32_t c0, c1;
    if (is_q4<TYPE>(type)) {
        const uint32_t w = word(r.q, hf * 8 + j);
        c0 = w & 0x0F0F0F0Fu;
        c1 = (w >> 4) & 0x0F0F0F0Fu;
    } else {
        const uint32_t la = word(r.q, j), lb = word(r.q, 8 + j), hq = word(r.h, j);
        const int sh = 4 * hf;
        c0 = ((la >> sh) & 0x0F0F0F0Fu) | (((hq >> sh) & 0x03030303u) << 4);
        c1 = ((lb >> sh) & 0x0F0F0F0Fu) | (((hq >> (sh + 2)) & 0x03030303u) << 4);
    }
    uint4 out;
    out.x = nib_h2(c0, 0x04020400u, sa, ba);
    out.y = nib_h2(c0, 0x04030401u, sa, ba);
    out.z = nib_h2(c1, 0x04020400u, sb, bb);
    out.w = nib_h2(c1, 0x04030401u, sb, bb);
    return __builtin_bit_cast(half8, out);
}

// Q6_K with a sub-block scale beyond +-62: the narrow decode's bias
// -1056 * s leaves fp16's range (65504), and s * (code - 32) reaches 4096 in
// magnitude, which fp16 holds only to even integers above 2048.  The weight
// is then written as W_a + W_b with W_a = fp16(s * (code - 32)) and W_b =
// fma(code - 32, s, -W_a), the exact rounding residual of an fp16 product
// (|W_b| <= 1), so B operand pairs (W_a, W_b) carry the integer weight
// exactly; code - 32 itself is exact (1024 + code - 1056).
__device__ __forceinline__ void q6_wide_h2(uint32_t v, uint32_t sel, half2v s, uint32_t &wa, uint32_t &wb) {
    const half2v off = {static_cast<_Float16>(-1056.f), static_cast<_Float16>(-1056.f)};
    const half2v c = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, v, sel)) + off;
    const half2v a = c * s;
    wa = __builtin_bit_cast(uint32_t, a);
    wb = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s, -a));
}

__device__ __forceinline__ void decode_b_wide(const RawBlock &r, int hf, int j, half2v sa, half2v sb, half8 &wa,
                                              half8 &wb) {
    const uint32_t la = word(r.q, j), lb = word(r.q, 8 + j), hq = word(r.h, j);
    const int sh = 4 * hf;
    const uint32_t c0 = ((la >> sh) & 0x0F0F0F0Fu) | (((hq >> sh) & 0x03030303u) << 4);
    const uint32_t c1 = ((lb >> sh) & 0x0F0F0F0Fu) | (((hq >> (sh + 2)) & 0x03030303u) << 4);
    uint4 a, b;
    q6_wide_h2(c0, 0x04020400u, sa, a.x, b.x);
    q6_wide_h2(c0, 0x04030401u, sa, a.y, b.y);
    q6_wide_h2(c1, 0x04020400u, sb, a.z, b.z);
    q6_wide_h2(c1, 0x04030401u, sb, a.w, b.w);
    wa = __builtin_bit_cast(half8, a);
    wb = __builtin_bit_cast(half8, b);
}

// Whether any of the lane's eight Q6_K scales (scales[kh*8 .. +8)) lies
// outside [-62, 62], where the narrow decode is not exact.
__device__ __forceinline__ bool q6_scales_wide(const RawBlock &r) {
    bool w = false;
    #pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int s = static_cast<int8_t>(((k < 4 ? r.hdr.x : r.hdr.y) >> (8 * (k & 3))) & 0xFFu);
        w |= s > 62 || s < -62;
    }
    return w;
}

__device__ __forceinline__ _Float16 u8_to_h(uint32_t v) { return static_cast<_Float16>(static_cast<float>(v & 0xFFu)); }
__device__ __forceinline__ _Float16 s8_to_h(uint32_t v) {
    return static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(v & 0xFFu)));
}

// Scale / bias operands of step j of block half hf for one row tile: the
// Q4_K sub-block scales (code offset 0) or the Q6_K int8 scales (code - 32).
template <int TYPE>
__device__ __forceinline__ void step_scales(const RawBlock &r, int type, uint32_t sc4, int hf, int j, half2v &sa2,
                                            half2v &ba2, half2v &sb2, half2v &bb2) {
    _Float16 sa, sb, off;
    if (is_q4<TYPE>(type)) {
        sa = u8_to_h(sc4 >> (16 * hf));
        sb = u8_to_h(sc4 >> (16 * hf + 8));
        off = static_cast<_Float16>(-1024.f);
    } else {
        // scales[kh*8 + 4*hf + 2*half + j/4]
        const uint32_t sw = hf ? r.hdr.y : r.hdr.x;
        sa = s8_to_h(sw >> (8 * (j >> 2)));
        sb = s8_to_h(sw >> (8 * (j >> 2) + 16));
        off = static_cast<_Float16>(-1056.f);   // code - 32
    }
    sa2 = half2v{sa, sa};
    sb2 = half2v{sb, sb};
    ba2 = half2v{static_cast<_Float16>(off * sa), static_cast<_Float16>(off * sa)};
    bb2 = half2v{static_cast<_Float16>(off * sb), static_cast<_Float16>(off * sb)};
}

// acc[r][t] += this block's contribution: RT row tiles (32 weight rows each,
// lane l -> row l%32, block half l/32) x TT token tiles (32 tokens each).
// Each decoded weight operand feeds TT token tiles; each activation operand
// read from LDS feeds RT row tiles.
template <int TYPE, int RT, int TT, bool WIDE = false>
__device__ __forceinline__ void block_mma(const RawBlock (&r)[RT], int type, const uint8_t *buf_lds, int kh, int col,
                                          float16v (&acc)[RT][TT]) {
    float d[RT], dmin[RT];
    uint32_t sc4[RT], mn4[RT];
    #pragma unroll
    for (int i = 0; i < RT; ++i) {
        dmin[i] = 0.f;
        sc4[i] = mn4[i] = 0;
        if (is_q4<TYPE>(type)) {
            d[i] = f16_bits_to_f32(r[i].hdr.x & 0xFFFFu);
            dmin[i] = f16_bits_to_f32(r[i].hdr.x >> 16);
            q4k_scale_min4(r[i].hdr, kh, sc4[i], mn4[i]);
        } else {
            d[i] = f16_bits_to_f32(r[i].hdr.z);
        }
    }
    float16v t[RT][TT];
    #pragma unroll
    for (int i = 0; i < RT; ++i)
        #pragma unroll
        for (int u = 0; u < TT; ++u)
            #pragma unroll
            for (int k = 0; k < 16; ++k) t[i][u][k] = 0.f;
    // Activation operands are read from LDS one step ahead of their use.
    half8 ah[TT], al[TT];
    #pragma unroll
    for (int u = 0; u < TT; ++u) {
        const uint8_t *tile = buf_lds + u * kTileBytes;
        ah[u] = reinterpret_cast<const half8 *>(tile)[kh * 32 + col];
        al[u] = reinterpret_cast<const half8 *>(tile + kTileA)[kh * 32 + col];
    }
    #pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        #pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int st = hf * 8 + j;
            half8 ahn[TT], aln[TT];
            #pragma unroll
            for (int u = 0; u < TT; ++u) {
                const uint8_t *tile = buf_lds + u * kTileBytes;
                const int sn = st < 15 ? st + 1 : st;
                ahn[u] = reinterpret_cast<const half8 *>(tile)[sn * 64 + kh * 32 + col];
                aln[u] = reinterpret_cast<const half8 *>(tile + kTileA)[sn * 64 + kh * 32 + col];
            }
            #pragma unroll
            for (int i = 0; i < RT; ++i) {
                half2v sa2, ba2, sb2, bb2;
                step_scales<TYPE>(r[i], type, sc4[i], hf, j, sa2, ba2, sb2, bb2);
                if constexpr (WIDE) {
                    // Q6_K with wide scales: W = W_a + W_b exactly.
                    half8 wa, wb;
                    decode_b_wide(r[i], hf, j, sa2, sb2, wa, wb);
                    #pragma unroll
                    for (int u = 0; u < TT; ++u) {
                        t[i][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[u], wa, t[i][u], 0, 0, 0);
                        t[i][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[u], wa, t[i][u], 0, 0, 0);
                        t[i][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[u], wb, t[i][u], 0, 0, 0);
                    }
                } else {
                    const half8 bw = decode_b<TYPE>(r[i], type, hf, j, sa2, ba2, sb2, bb2);
                    #pragma unroll
                    for (int u = 0; u < TT; ++u) {
                        t[i][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[u], bw, t[i][u], 0, 0, 0);
                        t[i][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[u], bw, t[i][u], 0, 0, 0);
                    }
                }
            }
            #pragma unroll
            for (int u = 0; u < TT; ++u) {
                ah[u] = ahn[u];
                al[u] = aln[u];
            }
        }
    }
    #pragma unroll
    for (int u = 0; u < TT; ++u) {
        const uint8_t *tile = buf_lds + u * kTileBytes;
        const float4 *fr = reinterpret_cast<const float4 *>(tile + 2 * kTileA + 2 * kTileM) + kh * 4;
        float f[16];
        #pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = fr[q];
            f[4 * q] = v.x;
            f[4 * q + 1] = v.y;
            f[4 * q + 2] = v.z;
            f[4 * q + 3] = v.w;
        }
        #pragma unroll
        for (int i = 0; i < RT; ++i)
            #pragma unroll
            for (int k = 0; k < 16; ++k) acc[i][u][k] = fmaf(d[i] * f[k], t[i][u][k], acc[i][u][k]);
        if (is_q4<TYPE>(type)) {
            const half4 mh = reinterpret_cast<const half4 *>(tile + 2 * kTileA)[kh * 32 + col];
            const half4 ml = reinterpret_cast<const half4 *>(tile + 2 * kTileA + kTileM)[kh * 32 + col];
            #pragma unroll
            for (int i = 0; i < RT; ++i) {
                half4 bm;
                #pragma unroll
                for (int e = 0; e < 4; ++e) bm[e] = u8_to_h(mn4[i] >> (8 * e));
                float16v tm;
                #pragma unroll
                for (int k = 0; k < 16; ++k) tm[k] = 0.f;
                tm = __builtin_amdgcn_mfma_f32_32x32x8f16(mh, bm, tm, 0, 0, 0);
                tm = __builtin_amdgcn_mfma_f32_32x32x8f16(ml, bm, tm, 0, 0, 0);
                #pragma unroll
                for (int k = 0; k < 16; ++k) acc[i][u][k] = fmaf(-64.f * dmin[i] * f[k], tm[k], acc[i][u][k]);
            }
        }
    }
}

// Output store: overwrite, or add into y (the driver's residual add).
__device__ __forceinline__ void store_out(const BatchParams &p, float *y, float v) {
    if (p.accumulate) v += *y;
    *y = v;
}

// ---------------------------------------------------------------- GEMM --
//
// Workgroup = 4 waves x RT row tiles = 128 RT weight rows, x TT token
// tiles of 32 tokens, x a run of blocks.  Per block the workgroup copies the
// TT activation records into LDS with direct global->LDS loads (no register
// round trip), double-buffered: block b+1's records and weight bytes are in
// flight while block b computes.  Wave w owns rows (i*4 + w)*32 .. +31 of
// the group for row tile i.

constexpr int kChunks = kTileBytes / 16;       // 16-byte chunks per record
static_assert(kChunks > 8 * 256 && kChunks <= 9 * 256, "record copy layout");

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void global_void_t;

// Wave-cooperative copy of one record into LDS: chunk c of the record goes
// to LDS byte 16*c; wave w issues chunks i*256 + w*64 + lane.
__device__ __forceinline__ void record_dma(const uint8_t *rec, uint8_t *tile_lds, int wave, int lane) {
    #pragma unroll
    for (int i = 0; i < 9; ++i) {
        const int c0 = i * 256 + wave * 64;   // wave-uniform
        if (c0 + lane < kChunks)
            __builtin_amdgcn_global_load_lds((global_void_t *)(rec + static_cast<size_t>(c0 + lane) * 16),
                                             (lds_void_t *)(tile_lds + c0 * 16), 16, 0, 0);
    }
}

__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int TYPE, int TT>
__global__ __launch_bounds__(256) void batch_gemm(BatchParams p) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int RT = TT;
    constexpr int kGroupRows = group_rows(RT);
    constexpr int kPartialFloats = partial_floats(RT);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kh = lane >> 5, col = lane & 31;
    const int split = blockIdx.x % p.splits, group = blockIdx.x / p.splits;
    const int tile0 = blockIdx.y * TT;

    int m = 0;
    #pragma unroll
    for (int i = 1; i < QK_MAX_FUSED; ++i) m += (i < p.n_mats && group >= p.mat[i].group_begin) ? 1 : 0;
    m = __builtin_amdgcn_readfirstlane(m);
    const BatchMatrix &M = p.mat[m];
    const int type = TYPE ? TYPE : M.type;
    const uint8_t *wrow[RT];
    int row[RT];
    #pragma unroll
    for (int i = 0; i < RT; ++i) {
        row[i] = (group - M.group_begin) * kGroupRows + (i * 4 + wave) * 32 + col;
        wrow[i] = M.w + static_cast<size_t>(min(row[i], M.rows - 1)) * M.row_bytes;
    }
    // Token tiles past the end read the last tile's records (in bounds) and store nothing.
    const uint8_t *recs[TT];
    #pragma unroll
    for (int u = 0; u < TT; ++u)
        recs[u] = p.records + static_cast<size_t>(min(tile0 + u, p.tiles - 1)) * p.nb * kTileBytes;

    const int b0 = split * p.blocks_per_split;
    const int b1 = min(p.nb, b0 + p.blocks_per_split);
    #pragma unroll
    for (int u = 0; u < TT; ++u) record_dma(recs[u] + static_cast<size_t>(b0) * kTileBytes, lds + u * kTileBytes, wave, lane);
    RawBlock cur[RT];
    #pragma unroll
    for (int i = 0; i < RT; ++i) cur[i] = load_block<TYPE>(wrow[i], b0, p.nb, type, kh);
    wait_loads();
    __syncthreads();

    float16v acc[RT][TT];
    #pragma unroll
    for (int i = 0; i < RT; ++i)
        #pragma unroll
        for (int u = 0; u < TT; ++u)
            #pragma unroll
            for (int k = 0; k < 16; ++k) acc[i][u][k] = 0.f;
    for (int b = b0; b < b1; ++b) {
        const int buf = (b - b0) & 1;
        // The last iteration reloads its own weight bytes (unconditional, in bounds).
        const int bn = min(b + 1, b1 - 1);
        if (b + 1 < b1) {
            #pragma unroll
            for (int u = 0; u < TT; ++u)
                record_dma(recs[u] + static_cast<size_t>(bn) * kTileBytes, lds + ((buf ^ 1) * TT + u) * kTileBytes, wave,
                           lane);
        }
        RawBlock nxt[RT];
        #pragma unroll
        for (int i = 0; i < RT; ++i) nxt[i] = load_block<TYPE>(wrow[i], bn, p.nb, type, kh);
        // A Q6_K block whose scales leave [-62, 62] in any of the wave's rows
        // takes the exact three-chain decode (wave-uniform branch).
        bool wide = false;
        if constexpr (TYPE != QK_TYPE_Q4_K) {
            if (!is_q4<TYPE>(type)) {
                bool lane_wide = false;
                #pragma unroll
                for (int i = 0; i < RT; ++i) lane_wide |= q6_scales_wide(cur[i]);
                wide = __builtin_amdgcn_ballot_w64(lane_wide) != 0;
            }
        }
        if (wide)
            block_mma<TYPE, RT, TT, true>(cur, type, lds + buf * TT * kTileBytes, kh, col, acc);
        else
            block_mma<TYPE, RT, TT>(cur, type, lds + buf * TT * kTileBytes, kh, col, acc);
        #pragma unroll
        for (int i = 0; i < RT; ++i) cur[i] = nxt[i];
        wait_loads();
        __syncthreads();
    }

    // Accumulator register k holds token 8*(k/4) + 4*kh + k%4 of its tile.
    if (!p.partials) {
        #pragma unroll
        for (int u = 0; u < TT; ++u) {
            const int tbase = (tile0 + u) * kTokTile + 4 * kh;
            #pragma unroll
            for (int i = 0; i < RT; ++i) {
                if (row[i] >= M.rows) continue;
                #pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const int t = tbase + 8 * (k >> 2) + (k & 3);
                    if (t < p.n_tokens) store_out(p, M.y + static_cast<int64_t>(t) * M.ldy + row[i], acc[i][u][k]);
                }
            }
        }
        return;
    }
    // Split blocks: partial sums to the workspace in accumulator order,
    // [group][token tile][split][wave][row tile][k][lane]; reduce_splits adds
    // them.  (A last-workgroup reduction inside this kernel would need a
    // device-scope fence per workgroup, measured slower than the extra launch.)
    #pragma unroll
    for (int u = 0; u < TT; ++u) {
        if (tile0 + u >= p.tiles) break;
        const size_t slot = static_cast<size_t>(group) * p.tiles + tile0 + u;
        float *mine = p.partials + (slot * p.splits + split) * kPartialFloats + wave * (RT * 1024) + lane;
        #pragma unroll
        for (int i = 0; i < RT; ++i)
            #pragma unroll
            for (int k = 0; k < 16; ++k) mine[i * 1024 + k * 64] = acc[i][u][k];
    }
}

// y = the sum of a row group's split partials, in split order (deterministic),
// stored with the call's epilogue (overwrite or add).  One thread per output
// value: thread u owns float u % kPartialFloats of slot u / kPartialFloats
// (slot = group * tiles + tile) -- GEMM wave, row tile, accumulator register
// and lane in the partials' own order, so a wave reads 64 consecutive floats
// per split -- and issues every split's load before the first add: the
// kernel is latency-bound, so it spreads over the whole chip.
// The RMSNorm factor 1/sqrt(mean(x^2) + eps) of token t's input, from the
// per-block sums of squares its producer wrote (in block order).
__device__ __forceinline__ float input_norm_scale(const BatchParams &p, int t) {
    const float *ss = p.in_ss + static_cast<int64_t>(t) * p.nb;
    float acc = 0.f;
    for (int b = 0; b < p.nb; ++b) acc += ss[b];
    return 1.0f / sqrtf(acc / static_cast<float>(p.nb * 256) + p.norm_eps);
}

template <int RT>
__global__ __launch_bounds__(256) void reduce_splits(BatchParams p) {
    constexpr int kGroupRows = group_rows(RT);
    constexpr int kPartialFloats = partial_floats(RT);
    const int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t slot = u / kPartialFloats;
    const int rem = static_cast<int>(u - slot * kPartialFloats);
    const int group = static_cast<int>(slot / p.tiles), tile = static_cast<int>(slot - static_cast<int64_t>(group) * p.tiles);
    const int wave = rem / (RT * 1024), i = (rem / 1024) % RT, k = (rem / 64) % 16, lane = rem % 64;
    const int kh = lane >> 5, col = lane & 31;
    int m = 0;
    #pragma unroll
    for (int j = 1; j < QK_MAX_FUSED; ++j) m += (j < p.n_mats && group >= p.mat[j].group_begin) ? 1 : 0;
    const BatchMatrix &M = p.mat[m];
    const float *part = p.partials + slot * p.splits * kPartialFloats + rem;
    float v[kMaxSplit];
    #pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp) v[sp] = sp < p.splits ? part[static_cast<int64_t>(sp) * kPartialFloats] : 0.f;
    float sum = v[0];
    #pragma unroll
    for (int sp = 1; sp < kMaxSplit; ++sp)
        if (sp < p.splits) sum += v[sp];
    // Accumulator register k holds token 8*(k/4) + 4*kh + k%4 of its tile.
    const int row = (group - M.group_begin) * kGroupRows + (i * 4 + wave) * 32 + col;
    const int t = tile * kTokTile + 8 * (k >> 2) + 4 * kh + (k & 3);
    if (row >= M.rows || t >= p.n_tokens) return;
    if (p.in_ss) sum *= input_norm_scale(p, t);
    float *yp = M.y + static_cast<int64_t>(t) * M.ldy + row;
    if (p.accumulate) sum = *yp + sum;
    *yp = sum;
}

// One wave per (output block ob of 256 rows, token): as many workgroups as
// output values / 256, so the latency-bound loads spread over the chip.
// Lane (q, part) = (lane / 8, lane % 8) sums the split
// partials of rows ob*256 + q*32 + part*4 .. +3 in split order, every
// split's load in flight before the first add (the kernel is latency-bound:
// a loop over splits would wait one L2 round trip per split), applies the
// deferred input norm and the residual add and stores y (not for a gate /
// up pair).  Then every lane packs its four values of the next GEMM's input
// block -- x * gain with the block's sum of squares of x, or SiLU(gate) * up
// -- into the record (the pack kernel's layout, stage_store_wave).
template <int RT>
__global__ __launch_bounds__(64) void reduce_pack(BatchParams p) {
    constexpr int kGroupRows = group_rows(RT);
    constexpr int kPartialFloats = partial_floats(RT);
    const int ob = blockIdx.x;
    const int tile = blockIdx.y / kTokTile;
    const int lane = threadIdx.x;
    const int tl = blockIdx.y % kTokTile;   // token within the tile
    const int q = lane >> 3, part = lane & 7;
    const int t = tile * kTokTile + tl;
    const bool live = t < p.n_tokens;
    const int row_q = ob * 256 + q * 32, row = row_q + part * 4;
    // Partial float4 of (matrix m, split sp) for these four rows and the token.
    const int k = 4 * (tl >> 3) + (tl & 3), kh = (tl >> 2) & 1;
    auto partial = [&](int m, int sp) -> const float4 * {
        const BatchMatrix &M = p.mat[m];
        const int g = M.group_begin + row_q / kGroupRows, rr = (row_q % kGroupRows) / 32;
        const int64_t slot = static_cast<int64_t>(g) * p.tiles + tile;
        return reinterpret_cast<const float4 *>(p.partials + (slot * p.splits + sp) * kPartialFloats +
                                                (rr & 3) * (RT * 1024) + (rr >> 2) * 1024 + k * 64 + kh * 32 +
                                                part * 4);
    };
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    float ss = 0.f;
    if (live) {
        const float s_in = p.in_ss ? input_norm_scale(p, t) : 1.f;
        float4 a[kMaxSplit], b[kMaxSplit];
        #pragma unroll
        for (int sp = 0; sp < kMaxSplit; ++sp) {
            a[sp] = sp < p.splits ? *partial(0, sp) : make_float4(0.f, 0.f, 0.f, 0.f);
            b[sp] = sp < p.splits && p.pair ? *partial(1, sp) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float4 sa = a[0], sb = b[0];
        #pragma unroll
        for (int sp = 1; sp < kMaxSplit; ++sp)
            if (sp < p.splits) {
                sa = make_float4(sa.x + a[sp].x, sa.y + a[sp].y, sa.z + a[sp].z, sa.w + a[sp].w);
                sb = make_float4(sb.x + b[sp].x, sb.y + b[sp].y, sb.z + b[sp].z, sb.w + b[sp].w);
            }
        sa = make_float4(sa.x * s_in, sa.y * s_in, sa.z * s_in, sa.w * s_in);
        if (p.pair) {
            sb = make_float4(sb.x * s_in, sb.y * s_in, sb.z * s_in, sb.w * s_in);
            v = make_float4(silu_mul_value(sa.x, sb.x), silu_mul_value(sa.y, sb.y), silu_mul_value(sa.z, sb.z),
                            silu_mul_value(sa.w, sb.w));
        } else {
            float4 *y = reinterpret_cast<float4 *>(p.mat[0].y + static_cast<int64_t>(t) * p.mat[0].ldy + row);
            v = sa;
            if (p.accumulate) {
                const float4 o = *y;
                v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
            }
            *y = v;
            if (p.out_gain) {
                ss = v.x * v.x;
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
                const float4 g = *reinterpret_cast<const float4 *>(p.out_gain + row);
                v = make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w);
            }
        }
    }
    if (p.out_gain) {
        #pragma unroll
        for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
        if (live && lane == 0) p.out_ss[static_cast<int64_t>(t) * p.out_nb + ob] = ss;
    }
    // Lane (q, part) holds values q*32 + 4*part .. +3 of the output block:
    // the whole wave stages the block's record.
    const float vr[4] = {v.x, v.y, v.z, v.w};
    stage_store_wave(vr, lane, tl, p.out_records + (static_cast<size_t>(tile) * p.out_nb + ob) * kTileBytes);
}

int check_batched(const char *where, const float *x, int ldx, int cols, int n_tokens) {
    if (!x || n_tokens < 0) return fail(QK_ERR_INVALID_ARG, std::string(where) + ": null x or negative count");
    if (ldx < cols) return fail(QK_ERR_INVALID_ARG, std::string(where) + ": ldx smaller than cols");
    if (!aligned(x, 16) || ldx % 4)
        return fail(QK_ERR_ALIGN, std::string(where) + ": x and ldx must keep 16-byte alignment");
    return QK_OK;
}

int tile_count(int n_tokens) { return (n_tokens + kTokTile - 1) / kTokTile; }

// Token tiles per workgroup: two once there are two tiles (each decoded
// weight operand then feeds 64 tokens), else one.  The row tiles per wave
// follow it.
int token_tiles_per_group(int tiles) { return tiles >= 2 ? 2 : 1; }
int row_tiles(int tiles) { return token_tiles_per_group(tiles); }

// Workgroups sharing a row group's blocks: enough that about one workgroup
// per CU is in flight (two with one row tile), at most kMaxSplit, at least
// one block each.  Every split writes as many partial-sum bytes per token
// tile as the weight bytes of one block of its rows, so more splits cost
// more than the extra workgroups gain (measured with two row tiles at 32
// tokens: one per CU 2.14 ms per 1B step, two per CU 2.20 ms; with one row
// tile, two per CU 1.94 ms against 1.98 at one).
void split_plan(int64_t groups, int nb, int tiles, int &splits, int &per_split) {
    const int tt = token_tiles_per_group(tiles);
    const int64_t target = static_cast<int64_t>(device_info().cus) * (row_tiles(tiles) == 1 ? 2 : 1);
    const int64_t have = std::max<int64_t>(1, groups * ((tiles + tt - 1) / tt));
    const int64_t want = (target + have - 1) / have;
    int s = static_cast<int>(std::min<int64_t>(std::max<int64_t>(want, 1), std::min(kMaxSplit, nb)));
    per_split = (nb + s - 1) / s;
    splits = (nb + per_split - 1) / per_split;
}

size_t records_bytes(int cols, int n_tokens) {
    return static_cast<size_t>(tile_count(n_tokens)) * (cols / 256) * kTileBytes;
}

int64_t group_count(const int *rows, int n, int rt) {
    int64_t g = 0;
    for (int i = 0; i < n; ++i) g += (rows[i] + group_rows(rt) - 1) / group_rows(rt);
    return g;
}

// Workspace: packed activation records, then (when blocks are split, or
// always with `partials`: a reduction stage that must run) the partial sums
// of every (row group, token tile, split).
size_t workspace_bytes(int cols, const int *rows, int n_mats, int n_tokens, bool partials = false) {
    if (cols <= 0 || cols % 256 || n_mats < 1 || n_tokens < kMfmaMinTokens) return 0;
    const int tiles = tile_count(n_tokens);
    size_t bytes = (records_bytes(cols, n_tokens) + 255) / 256 * 256;
    const int rt = row_tiles(tiles);
    const int64_t groups = group_count(rows, n_mats, rt);
    if (groups < 1) return 0;
    int splits, per_split;
    split_plan(groups, cols / 256, tiles, splits, per_split);
    if (splits == 1 && !partials) return bytes;
    return bytes + static_cast<size_t>(groups) * tiles * splits * partial_floats(rt) * sizeof(float);
}

// Workspace bound for the public query, which knows only the total row
// count: the group count of any split of `rows_total` rows over at most
// QK_MAX_FUSED matrices is at most rows_total/group_rows + QK_MAX_FUSED.
size_t workspace_bound(int cols, int rows_total, int n_tokens, bool partials = false) {
    if (rows_total <= 0) return 0;
    const int tiles = tile_count(n_tokens);
    if (cols <= 0 || cols % 256 || n_tokens < kMfmaMinTokens) return 0;
    size_t bytes = (records_bytes(cols, n_tokens) + 255) / 256 * 256;
    const int rt = row_tiles(tiles);
    const int64_t gmin = (rows_total + group_rows(rt) - 1) / group_rows(rt);
    const int64_t gmax = rows_total / group_rows(rt) + QK_MAX_FUSED;
    const size_t slot = static_cast<size_t>(partial_floats(rt)) * sizeof(float);
    size_t best = 0;
    for (int64_t g : {gmin, gmax}) {
        int splits, per_split;
        split_plan(g, cols / 256, tiles, splits, per_split);
        if (splits > 1 || partials) best = std::max(best, static_cast<size_t>(g) * tiles * splits * slot);
    }
    // Between gmin and gmax the split count only falls as groups grow, and the
    // partial bytes are groups * splits: bounded by gmax * splits(gmin).
    int s_min, ps;
    split_plan(gmin, cols / 256, tiles, s_min, ps);
    if (s_min > 1 || partials) best = std::max(best, static_cast<size_t>(gmax) * tiles * s_min * slot);
    return bytes + best;
}

template <int TT>
void launch_gemm(int type, const dim3 &grid, size_t lds, hipStream_t stream, const BatchParams &p) {
    if (type == QK_TYPE_Q4_K)
        hipLaunchKernelGGL((batch_gemm<QK_TYPE_Q4_K, TT>), grid, dim3(256), lds, stream, p);
    else if (type == QK_TYPE_Q6_K)
        hipLaunchKernelGGL((batch_gemm<QK_TYPE_Q6_K, TT>), grid, dim3(256), lds, stream, p);
    else if (type == QK_TYPE_Q6_K_SPLIT)
        hipLaunchKernelGGL((batch_gemm<QK_TYPE_Q6_K_SPLIT, TT>), grid, dim3(256), lds, stream, p);
    else
        hipLaunchKernelGGL((batch_gemm<0, TT>), grid, dim3(256), lds, stream, p);
}

int launch_mfma(const qk_matrix *mats, int n_mats, const int *ldy, const float *x, int ldx, int cols, int n_tokens,
                void *workspace, size_t workspace_size, hipStream_t stream, const char *where,
                const GemvFusion *fusion = nullptr) {
    const int nb = cols / 256;
    const int tiles = tile_count(n_tokens);
    const int tt = token_tiles_per_group(tiles);
    const int rt = row_tiles(tiles);
    if (tiles > 65535) return fail(QK_ERR_LIMIT, std::string(where) + ": too many tokens in one launch");
    BatchParams p{};
    p.n_mats = n_mats;
    p.x = x;
    p.ldx = ldx;
    p.n_tokens = n_tokens;
    p.nb = nb;
    p.tiles = tiles;
    int64_t groups = 0;
    int type = mats[0].type;
    int rows[QK_MAX_FUSED];
    for (int i = 0; i < n_mats; ++i) {
        BatchMatrix &M = p.mat[i];
        M.w = static_cast<const uint8_t *>(mats[i].w);
        M.y = mats[i].y;
        M.rows = mats[i].rows;
        M.type = mats[i].type;
        M.row_bytes = static_cast<int>(row_bytes(M.type, nb));
        M.ldy = ldy[i];
        M.group_begin = static_cast<int>(groups);
        groups += (M.rows + group_rows(rt) - 1) / group_rows(rt);
        rows[i] = M.rows;
        if (static_cast<int64_t>(M.rows) * M.row_bytes > (int64_t(1) << 40))
            return fail(QK_ERR_LIMIT, std::string(where) + ": matrix too large");
        if (M.type != type) type = 0;
    }
    split_plan(groups, nb, tiles, p.splits, p.blocks_per_split);
    if (groups * p.splits > (1 << 30)) return fail(QK_ERR_LIMIT, std::string(where) + ": too many rows");
    // A decode chain's reduction stage (deferred input norm, or packing the
    // next call's records) runs even without a split.
    const bool chain_out = fusion && fusion->out_records;
    const bool need_partials = p.splits > 1 || (fusion && fusion->in_ss) || chain_out;
    if (chain_out) {
        const bool pair = fusion->pair != 0;
        if ((pair && (n_mats != 2 || rows[0] != rows[1])) || (!pair && n_mats != 1) || rows[0] % 256 ||
            (!pair && !fusion->out_gain) || (fusion->out_gain && !fusion->out_ss))
            return fail(QK_ERR_INVALID_ARG, std::string(where) + ": unsupported chained reduction");
    }
    const size_t need = workspace_bytes(cols, rows, n_mats, n_tokens, need_partials);
    if (!workspace || workspace_size < need)
        return fail(QK_ERR_INVALID_ARG, std::string(where) + ": workspace smaller than " + std::to_string(need) +
                                            " bytes (qk_gemv_batched_workspace_bytes)");
    if (!aligned(workspace, 256)) return fail(QK_ERR_ALIGN, std::string(where) + ": workspace not 256-byte aligned");
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    const int tgroups = (tiles + tt - 1) / tt;
    p.records = ws;
    if (need_partials) p.partials = reinterpret_cast<float *>(ws + (records_bytes(cols, n_tokens) + 255) / 256 * 256);
    if (fusion) {
        p.norm_w = fusion->norm_w;
        p.norm_eps = fusion->norm_eps;
        p.up = fusion->up;
        p.accumulate = fusion->accumulate;
        p.in_ss = fusion->in_ss;
        if (fusion->in_records) p.records = fusion->in_records;
        p.out_records = fusion->out_records;
        p.out_nb = rows[0] / 256;
        p.out_gain = fusion->out_gain;
        p.out_ss = fusion->out_ss;
        p.pair = fusion->pair;
    }
    if (!(fusion && fusion->in_records))
        hipLaunchKernelGGL(pack_activations, dim3(nb, tiles * (kTokTile / kPackTokens)), dim3(256), 0, stream, p, ws);
    const dim3 grid(static_cast<unsigned>(groups * p.splits), tgroups);
    const size_t lds = 2 * static_cast<size_t>(tt) * kTileBytes;
    if (tt == 2)
        launch_gemm<2>(type, grid, lds, stream, p);
    else
        launch_gemm<1>(type, grid, lds, stream, p);
    if (chain_out) {
        const dim3 rgrid(static_cast<unsigned>(p.out_nb), static_cast<unsigned>(tiles * kTokTile));
        if (rt == 2)
            hipLaunchKernelGGL(reduce_pack<2>, rgrid, dim3(64), 0, stream, p);
        else
            hipLaunchKernelGGL(reduce_pack<1>, rgrid, dim3(64), 0, stream, p);
    } else if (need_partials) {
        const dim3 rgrid(static_cast<unsigned>(groups * tiles * (partial_floats(rt) / 256)));
        if (rt == 2)
            hipLaunchKernelGGL(reduce_splits<2>, rgrid, dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL(reduce_splits<1>, rgrid, dim3(256), 0, stream, p);
    }
    return launch_status(where);
}

}  // namespace

size_t batched_chain_workspace_bytes(int cols, int rows_total, int n_tokens) {
    return workspace_bound(cols, rows_total, n_tokens, true);
}

size_t batched_records_bytes(int cols, int n_tokens) {
    return n_tokens < kMfmaMinTokens || cols % 256 ? 0 : records_bytes(cols, n_tokens);
}

bool batched_chain_supported(int n_tokens) { return n_tokens >= kMfmaMinTokens; }

// The FFN's workspace from kMfmaMinTokens tokens on: the GEMM workspace the
// gate / up chain and the down call share (the larger of the two, over
// every token-tile count up to n_tokens, since the split plan -- not the
// token count alone -- fixes the partials' size), then the SiLU * up
// records the chain leaves for down.
size_t ffn_shared_bytes(int dim, int hidden, int n_tokens) {
    size_t ws = 0;
    for (int tq = 1; tq <= tile_count(n_tokens); ++tq) {
        const int n = std::min(n_tokens, std::max(kMfmaMinTokens, tq * kTokTile));
        ws = std::max({ws, workspace_bound(dim, 2 * hidden, n, true), workspace_bound(hidden, dim, n)});
    }
    return (ws + 255) / 256 * 256;
}

// Below kMfmaMinTokens: the gate and up outputs, each 256-byte aligned.
size_t ffn_gemv_slot(int hidden, int n_tokens) {
    return (static_cast<size_t>(n_tokens) * hidden * sizeof(float) + 255) / 256 * 256;
}

int launch_batched_fused(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                         const GemvFusion &f, void *workspace, size_t workspace_size, hipStream_t stream) {
    int ldy[QK_MAX_FUSED];
    for (int m = 0; m < n_mats; ++m) ldy[m] = mats[m].rows;
    if (n_tokens >= kMfmaMinTokens)
        return launch_mfma(mats, n_mats, ldy, x, ldx, cols, n_tokens, workspace, workspace_size, stream,
                           "fused batched GEMM", &f);
    return launch_gemv_fused(mats, n_mats, x, ldx, cols, n_tokens, ldy, f, stream);
}

}  // namespace qk

extern "C" {

size_t qk_gemv_batched_workspace_bytes(int cols, int rows, int n_tokens) {
    return qk::workspace_bound(cols, rows, n_tokens);
}

int qk_gemv_batched_f32(int type, const void *w, const float *x, int ldx, float *y, int ldy, int cols, int rows,
                        int n_tokens, void *workspace, size_t workspace_bytes, qk_stream stream) {
    int st = qk::check_weights("qk_gemv_batched_f32", type, w, cols, rows);
    if (st) return st;
    if ((st = qk::check_batched("qk_gemv_batched_f32", x, ldx, cols, n_tokens))) return st;
    if (!y || ldy < rows) return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_batched_f32: null y or ldy smaller than rows");
    if (!qk::aligned(y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_gemv_batched_f32: y must be 4-byte aligned");
    if (n_tokens == 0) return qk::ok();
    const qk_matrix m{type, rows, w, y};
    if (n_tokens >= qk::kMfmaMinTokens)
        return qk::launch_mfma(&m, 1, &ldy, x, ldx, cols, n_tokens, workspace, workspace_bytes,
                               static_cast<hipStream_t>(stream), "qk_gemv_batched_f32");
    return qk::launch_gemv_f32(&m, 1, x, ldx, cols, n_tokens, &ldy, static_cast<hipStream_t>(stream));
}

size_t qk_ffn_batched_workspace_bytes(int dim, int hidden, int n_tokens) {
    if (dim <= 0 || hidden <= 0 || n_tokens <= 0 || dim % 256 || hidden % 256) return 0;
    if (n_tokens < qk::kMfmaMinTokens) return 2 * qk::ffn_gemv_slot(hidden, n_tokens);
    // Also enough for any smaller call: the GEMV form's gate and up outputs.
    return std::max(qk::ffn_shared_bytes(dim, hidden, n_tokens) + (qk::records_bytes(hidden, n_tokens) + 255) / 256 * 256,
                    2 * qk::ffn_gemv_slot(hidden, qk::kMfmaMinTokens - 1));
}

int qk_ffn_batched_f32(int gate_type, const void *gate, int up_type, const void *up, int down_type, const void *down,
                       const float *x, int ldx, float *y, int ldy, int dim, int hidden, int n_tokens, int accumulate,
                       void *workspace, size_t workspace_bytes, qk_stream stream) {
    const char *where = "qk_ffn_batched_f32";
    int st;
    if ((st = qk::check_weights(where, gate_type, gate, dim, hidden)) ||
        (st = qk::check_weights(where, up_type, up, dim, hidden)) ||
        (st = qk::check_weights(where, down_type, down, hidden, dim)) ||
        (st = qk::check_batched(where, x, ldx, dim, n_tokens)))
        return st;
    if (!y || ldy < dim) return qk::fail(QK_ERR_INVALID_ARG, "qk_ffn_batched_f32: null y or ldy smaller than dim");
    if (!qk::aligned(y, 4)) return qk::fail(QK_ERR_ALIGN, "qk_ffn_batched_f32: y must be 4-byte aligned");
    if (n_tokens == 0) return qk::ok();
    const size_t need = qk_ffn_batched_workspace_bytes(dim, hidden, n_tokens);
    if (!workspace || workspace_bytes < need)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_ffn_batched_f32: workspace smaller than " + std::to_string(need) +
                                                " bytes (qk_ffn_batched_workspace_bytes)");
    if (!qk::aligned(workspace, 256)) return qk::fail(QK_ERR_ALIGN, "qk_ffn_batched_f32: workspace not 256-byte aligned");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    const qk_matrix dm{down_type, dim, down, y};
    qk::GemvFusion df;
    df.accumulate = accumulate != 0;
    if (n_tokens < qk::kMfmaMinTokens) {
        // Gate and up into the workspace, then down with SiLU(gate) * up
        // staged in its own activation load.
        if (!qk::gemv_fusable(hidden)) return qk::fail(QK_ERR_LIMIT, "qk_ffn_batched_f32: hidden too long to stage");
        float *g = reinterpret_cast<float *>(ws);
        float *u = reinterpret_cast<float *>(ws + qk::ffn_gemv_slot(hidden, n_tokens));
        const qk_matrix gu[2] = {{gate_type, hidden, gate, g}, {up_type, hidden, up, u}};
        const int ldg[2] = {hidden, hidden};
        if ((st = qk::launch_gemv_f32(gu, 2, x, ldx, dim, n_tokens, ldg, s))) return st;
        df.up = u;
        return qk::launch_gemv_fused(&dm, 1, g, hidden, hidden, n_tokens, &ldy, df, s);
    }
    // Matrix cores: gate / up's reduction writes the records of SiLU(gate) *
    // up (gate and up themselves are never stored), which down reads.
    const size_t shared = qk::ffn_shared_bytes(dim, hidden, n_tokens);
    uint8_t *rec = ws + shared;
    const qk_matrix gu[2] = {{gate_type, hidden, gate, y}, {up_type, hidden, up, y}};
    const int ldg[2] = {hidden, hidden};
    qk::GemvFusion gf;
    gf.pair = 1;
    gf.out_records = rec;
    if ((st = qk::launch_mfma(gu, 2, ldg, x, ldx, dim, n_tokens, ws, shared, s, where, &gf))) return st;
    df.in_records = rec;
    return qk::launch_mfma(&dm, 1, &ldy, x, ldx, hidden, n_tokens, ws, shared, s, where, &df);
}

int qk_gemv_multi_batched_f32(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                              void *workspace, size_t workspace_bytes, qk_stream stream) {
    if (!mats || n_mats < 1 || n_mats > QK_MAX_FUSED)
        return qk::fail(QK_ERR_INVALID_ARG, "qk_gemv_multi_batched_f32: need 1.." + std::to_string(QK_MAX_FUSED) +
                                                " matrices");
    int st = qk::check_batched("qk_gemv_multi_batched_f32", x, ldx, cols, n_tokens);
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
    if (n_tokens >= qk::kMfmaMinTokens)
        return qk::launch_mfma(mats, n_mats, ldy, x, ldx, cols, n_tokens, workspace, workspace_bytes,
                               static_cast<hipStream_t>(stream), "qk_gemv_multi_batched_f32");
    return qk::launch_gemv_f32(mats, n_mats, x, ldx, cols, n_tokens, ldy, static_cast<hipStream_t>(stream));
}

}  // extern "C"
