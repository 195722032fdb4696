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
// with W_int = sc*q (Q4_K, 0..945) or sc*(code-32) (Q6_K, -1024..1024):
// integers that fp16 holds exactly.  Activations are scaled per (token,
// block) by a power of two so the block maximum lies in [2^14, 2^15) and
// split into fp16 high and low halves (22 significant bits), so each block
// is two v_mfma_f32_32x32x16_f16 chains over exact operands; the block's d
// (and dmin with the sub-block sums X, through v_mfma_f32_32x32x8_f16) and
// the activation scale are applied in fp32 when the block is done.
//
// Two kernels:
//   pack_activations  x -> per (32-token tile, block) records in the caller's
//                     workspace, laid out as MFMA A operands.
//   batch_mfma        one wave = 64 weight rows x 32 tokens over a run of
//                     blocks; the waves of a workgroup split the row's blocks
//                     and meet in LDS (fixed order, deterministic).
// The weights are MFMA B operands decoded in registers from the raw block
// bytes: lane l owns weight row l%32 and block half l/32.
#include "qk_internal.h"

namespace qk {
int launch_gemv_f32(const qk_matrix *mats, int n_mats, const float *x, int ldx, int cols, int n_tokens,
                    const int *ldy, hipStream_t stream);
}

namespace qk {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kMfmaMinTokens = 8;
constexpr int kTokTile = 32;            // tokens per MFMA tile (the A rows)
constexpr int kRowTiles = 2;            // 32-row MFMA column tiles per wave
constexpr int kGroupRows = 32 * kRowTiles;
constexpr int kMaxSplit = 8;            // waves per workgroup splitting the blocks

// One (token tile, block) record of packed activations.
//   hi   [16 steps][2 halves][32 tokens][8]  fp16   16 KiB
//   lo   same                                fp16   16 KiB
//   mhi  [2 halves][32 tokens][4]            fp16   512 B  (sub-block sums / 64)
//   mlo  same                                fp16   512 B
//   f    [2 halves][16]                      fp32   128 B  (2^e per token, lane order)
constexpr size_t kRecA = 16384;
constexpr size_t kRecM = 512;
constexpr size_t kRecF = 128;
constexpr size_t kRecBytes = 2 * kRecA + 2 * kRecM + kRecF;
static_assert(kRecBytes % 16 == 0, "records keep 16-byte alignment");

// K order of the A / B operands inside a block.  Step s (0..15) and half kh
// (lane / 32) hold eight columns of the 64-column group G = 2*kh + s/8:
//   e 0..3: G*64 +      4*(s%8) + {0, 2, 1, 3}[e]
//   e 4..7: G*64 + 32 + 4*(s%8) + {0, 2, 1, 3}[e-4]
// i.e. the low nibbles (e < 4) and high nibbles (e >= 4) of Q4_K qs bytes
// G*32 + 4*(s%8) .. +3, even bytes first; Q6_K uses the same columns.

// ------------------------------------------------------------- packing --

__global__ __launch_bounds__(256) void pack_activations(const float *__restrict__ x, int ldx, int n_tokens, int nb,
                                                        uint8_t *__restrict__ ws) {
    const int b = blockIdx.x, tile = blockIdx.y;
    const int tl = threadIdx.x >> 3;           // token within the tile
    const int q = threadIdx.x & 7;             // 32-column sub-block of the block
    const int t = tile * kTokTile + tl;
    float v[32];
    if (t < n_tokens) {
        const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<int64_t>(t) * ldx + b * 256 + q * 32);
        #pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 u = src[i];
            v[4 * i] = u.x;
            v[4 * i + 1] = u.y;
            v[4 * i + 2] = u.z;
            v[4 * i + 3] = u.w;
        }
    } else {
        #pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = 0.f;
    }
    float m = 0.f;
    #pragma unroll
    for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    m = fmaxf(m, __shfl_xor(m, 4));
    // x' = x * 2^(14-e), e = floor(log2 max): the block maximum in [2^14, 2^15).
    // The shift is capped at 140 so that 2^-shift stays a finite nonzero fp32.
    int shift = 0;
    float f = 0.f;
    bool bad = false;
    #pragma unroll
    for (int i = 0; i < 32; ++i) bad |= !isfinite(v[i]);
    if (m > 0.f && isfinite(m)) {
        shift = min(15 - __builtin_amdgcn_frexp_expf(m), 140);
        f = ldexpf(1.f, -shift);
    }
    bad = __shfl_xor(static_cast<int>(bad), 1) | bad;
    bad = __shfl_xor(static_cast<int>(bad), 2) | bad;
    bad = __shfl_xor(static_cast<int>(bad), 4) | bad;
    if (bad) f = __builtin_nanf("");            // a non-finite input poisons the token's outputs

    uint8_t *rec = ws + (static_cast<size_t>(tile) * nb + b) * kRecBytes;
    _Float16 *hi = reinterpret_cast<_Float16 *>(rec);
    _Float16 *lo = reinterpret_cast<_Float16 *>(rec + kRecA);
    const int G = q >> 1, half = q & 1, kh = G >> 1, hf = G & 1;
    float sum = 0.f;
    #pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int s = hf * 8 + j;
        half4 h4, l4;
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float xs = bad ? 0.f : ldexpf(v[4 * j + i], shift);
            sum += xs;
            const _Float16 h = static_cast<_Float16>(xs);
            const int e = (i == 1) ? 2 : (i == 2) ? 1 : i;   // column order {0, 2, 1, 3}
            h4[e] = h;
            l4[e] = static_cast<_Float16>(xs - static_cast<float>(h));
        }
        const size_t at = (static_cast<size_t>((s * 2 + kh) * 32 + tl)) * 8 + half * 4;
        *reinterpret_cast<half4 *>(hi + at) = h4;
        *reinterpret_cast<half4 *>(lo + at) = l4;
    }
    // Sub-block sums for the Q4_K min term: K index j = q, lane half q/4.
    _Float16 *mhi = reinterpret_cast<_Float16 *>(rec + 2 * kRecA);
    _Float16 *mlo = reinterpret_cast<_Float16 *>(rec + 2 * kRecA + kRecM);
    // |sum| < 32 * 2^15: stored / 64 to stay inside the fp16 range.
    const float s64 = sum * (1.f / 64.f);
    const _Float16 sh = static_cast<_Float16>(s64);
    const int mat = ((q >> 2) * 32 + tl) * 4 + (q & 3);
    mhi[mat] = sh;
    mlo[mat] = static_cast<_Float16>(s64 - static_cast<float>(sh));
    // Token scales in the accumulator lane order: lane half kh' = (tl/4)%2,
    // register k = 4*(tl/8) + tl%4.
    if (q == 0) {
        float *fr = reinterpret_cast<float *>(rec + 2 * kRecA + 2 * kRecM);
        fr[((tl >> 2) & 1) * 16 + 4 * (tl >> 3) + (tl & 3)] = f;
    }
}

// ---------------------------------------------------------------- GEMM --

struct BatchMatrix {
    const uint8_t *w;
    float *y;
    int rows;
    int type;
    int row_bytes;
    int ldy;
    int group_begin;   // first 64-row group of this matrix in the launch
};

struct BatchParams {
    BatchMatrix mat[QK_MAX_FUSED];
    int n_mats;
    const uint8_t *ws;
    int nb;
    int n_tokens;
    int blocks_per_wave;
};

// Raw bytes of one block of one row that lane half kh needs.
struct RawBlock {
    uint4 q[4];        // Q4_K: qs[kh*64 .. +64); Q6_K: ql[kh*64 .. +64)
    uint4 h[2];        // Q6_K: qh[kh*32 .. +32)
    uint4 hdr;         // Q4_K: d, dmin, scales; Q6_K: x = scales[kh*8 .. +4), y = scales[kh*8+4 .. +8), z = d
};

template <int TYPE>
__device__ __forceinline__ bool is_q4(int type) {
    return TYPE == QK_TYPE_Q4_K || (TYPE == 0 && type == QK_TYPE_Q4_K);
}

template <int TYPE>
__device__ __forceinline__ RawBlock load_block(const uint8_t *blk, int type, int kh) {
    RawBlock r;
    if (is_q4<TYPE>(type)) {
        r.hdr = load16(blk);
        #pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = load16(blk + 16 + kh * 64 + 16 * i);
        r.h[0] = r.h[1] = make_uint4(0, 0, 0, 0);
    } else {
        #pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = load16(blk + kh * 64 + 16 * i);
        r.h[0] = load16(blk + 128 + kh * 32);
        r.h[1] = load16(blk + 128 + kh * 32 + 16);
        const uint2 s = load8(blk + 192 + kh * 8);
        r.hdr = make_uint4(s.x, s.y, load2(blk + 208), 0);
    }
    return r;
}

__device__ __forceinline__ uint32_t word(const uint4 *v, int i) {
    const uint4 &u = v[i >> 2];
    return (i & 3) == 0 ? u.x : (i & 3) == 1 ? u.y : (i & 3) == 2 ? u.z : u.w;
}

// Two bytes (0 and 2, or 1 and 3 after a shift) of v as two fp16 integers
// minus `bias`: 0x6400 | n is the fp16 1024 + n.
__device__ __forceinline__ uint32_t bytes_to_h2(uint32_t v, _Float16 bias) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t bits = (v & 0x00FF00FFu) | 0x64006400u;
    h2 r = __builtin_bit_cast(h2, bits);
    const h2 b = {bias, bias};
    r = r - b;
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t mul_h2(uint32_t a, _Float16 s) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 m = {s, s};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) * m);
}

// B operand of step j (0..7) of block half hf: eight exact fp16 integer
// weights in the K order above.
template <int TYPE>
__device__ __forceinline__ half8 decode_b(const RawBlock &r, int type, int hf, int j, _Float16 sa, _Float16 sb) {
    uint32_t c0, c1;
    _Float16 bias;
    if (is_q4<TYPE>(type)) {
        const uint32_t w = word(r.q, hf * 8 + j);
        c0 = w & 0x0F0F0F0Fu;
        c1 = (w >> 4) & 0x0F0F0F0Fu;
        bias = static_cast<_Float16>(1024.f);
    } else {
        const uint32_t la = word(r.q, j), lb = word(r.q, 8 + j), hq = word(r.h, j);
        const int sh = 4 * hf;
        c0 = ((la >> sh) & 0x0F0F0F0Fu) | (((hq >> sh) & 0x03030303u) << 4);
        c1 = ((lb >> sh) & 0x0F0F0F0Fu) | (((hq >> (sh + 2)) & 0x03030303u) << 4);
        bias = static_cast<_Float16>(1056.f);   // 1024 + 32: code - 32
    }
    uint4 out;
    out.x = mul_h2(bytes_to_h2(c0, bias), sa);
    out.y = mul_h2(bytes_to_h2(c0 >> 8, bias), sa);
    out.z = mul_h2(bytes_to_h2(c1, bias), sb);
    out.w = mul_h2(bytes_to_h2(c1 >> 8, bias), sb);
    return __builtin_bit_cast(half8, out);
}

__device__ __forceinline__ float16v mfma16(half8 a, half8 b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <int TYPE>
__global__ __launch_bounds__(64 * kMaxSplit) void batch_mfma(BatchParams p) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_waves = blockDim.x >> 6;
    const int kh = lane >> 5, col = lane & 31;
    const int group = blockIdx.x, tile = blockIdx.y;

    int m = 0;
    #pragma unroll
    for (int i = 1; i < QK_MAX_FUSED; ++i) m += (i < p.n_mats && group >= p.mat[i].group_begin) ? 1 : 0;
    m = __builtin_amdgcn_readfirstlane(m);
    const BatchMatrix &M = p.mat[m];
    const int type = TYPE ? TYPE : M.type;
    const int row0 = (group - M.group_begin) * kGroupRows;
    const uint8_t *wrow[kRowTiles];
    #pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt)
        wrow[rt] = M.w + static_cast<size_t>(min(row0 + rt * 32 + col, M.rows - 1)) * M.row_bytes;
    const int bpb = is_q4<TYPE>(type) ? 144 : 210;

    float16v acc[kRowTiles];
    #pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt)
        #pragma unroll
        for (int k = 0; k < 16; ++k) acc[rt][k] = 0.f;

    const int b_begin = wave * p.blocks_per_wave;
    const int b_end = min(p.nb, b_begin + p.blocks_per_wave);
    for (int b = b_begin; b < b_end; ++b) {
        RawBlock raw[kRowTiles];
        #pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) raw[rt] = load_block<TYPE>(wrow[rt] + b * bpb, type, kh);
        const uint8_t *rec = p.ws + (static_cast<size_t>(tile) * p.nb + b) * kRecBytes;
        const float4 *fr = reinterpret_cast<const float4 *>(rec + 2 * kRecA + 2 * kRecM) + kh * 4;
        float f[16];
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 u = fr[i];
            f[4 * i] = u.x;
            f[4 * i + 1] = u.y;
            f[4 * i + 2] = u.z;
            f[4 * i + 3] = u.w;
        }
        // Per-row block scales.
        float d[kRowTiles], dmin[kRowTiles];
        uint32_t sc4[kRowTiles], mn4[kRowTiles];
        #pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
            if (is_q4<TYPE>(type)) {
                d[rt] = f16_bits_to_f32(raw[rt].hdr.x & 0xFFFFu);
                dmin[rt] = f16_bits_to_f32(raw[rt].hdr.x >> 16);
                q4k_scale_min4(raw[rt].hdr, kh, sc4[rt], mn4[rt]);
            } else {
                d[rt] = f16_bits_to_f32(raw[rt].hdr.z);
                dmin[rt] = 0.f;
                sc4[rt] = mn4[rt] = 0;
            }
        }
        #pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            half8 ah[8], al[8];
            const half8 *ahp = reinterpret_cast<const half8 *>(rec) + (hf * 8 * 2 + kh) * 32 + col;
            const half8 *alp = reinterpret_cast<const half8 *>(rec + kRecA) + (hf * 8 * 2 + kh) * 32 + col;
            #pragma unroll
            for (int j = 0; j < 8; ++j) {
                ah[j] = ahp[j * 64];
                al[j] = alp[j * 64];
            }
            #pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) {
                float16v t;
                #pragma unroll
                for (int k = 0; k < 16; ++k) t[k] = 0.f;
                #pragma unroll
                for (int j = 0; j < 8; ++j) {
                    _Float16 sa, sb;
                    if (is_q4<TYPE>(type)) {
                        sa = static_cast<_Float16>(static_cast<float>((sc4[rt] >> (16 * hf)) & 0xFFu));
                        sb = static_cast<_Float16>(static_cast<float>((sc4[rt] >> (16 * hf + 8)) & 0xFFu));
                    } else {
                        // scales[kh*8 + 4*hf + 2*half + j/4] (int8)
                        const uint32_t sw = hf ? raw[rt].hdr.y : raw[rt].hdr.x;
                        const int sh = 8 * (j >> 2);
                        sa = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((sw >> sh) & 0xFFu)));
                        sb = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>((sw >> (sh + 16)) & 0xFFu)));
                    }
                    const half8 bw = decode_b<TYPE>(raw[rt], type, hf, j, sa, sb);
                    t = mfma16(ah[j], bw, t);
                    t = mfma16(al[j], bw, t);
                }
                #pragma unroll
                for (int k = 0; k < 16; ++k) acc[rt][k] = fmaf(d[rt] * f[k], t[k], acc[rt][k]);
            }
        }
        if (is_q4<TYPE>(type)) {
            const half4 mh = reinterpret_cast<const half4 *>(rec + 2 * kRecA)[kh * 32 + col];
            const half4 ml = reinterpret_cast<const half4 *>(rec + 2 * kRecA + kRecM)[kh * 32 + col];
            #pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) {
                half4 bm;
                #pragma unroll
                for (int e = 0; e < 4; ++e) bm[e] = static_cast<_Float16>(static_cast<float>((mn4[rt] >> (8 * e)) & 0xFFu));
                float16v t;
                #pragma unroll
                for (int k = 0; k < 16; ++k) t[k] = 0.f;
                t = __builtin_amdgcn_mfma_f32_32x32x8f16(mh, bm, t, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_32x32x8f16(ml, bm, t, 0, 0, 0);
                #pragma unroll
                for (int k = 0; k < 16; ++k) acc[rt][k] = fmaf(-64.f * dmin[rt] * f[k], t[k], acc[rt][k]);
            }
        }
    }

    // Token k of the accumulators: 8*(k/4) + 4*kh + k%4 of the tile.
    const int t0 = tile * kTokTile + 4 * kh;
    if (n_waves == 1) {
        #pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
            const int row = row0 + rt * 32 + col;
            if (row >= M.rows) continue;
            #pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int t = t0 + 8 * (k >> 2) + (k & 3);
                if (t < p.n_tokens) M.y[static_cast<int64_t>(t) * M.ldy + row] = acc[rt][k];
            }
        }
        return;
    }
    // Split blocks: partial sums meet in LDS, added in wave order.
    float *red = reinterpret_cast<float *>(lds);
    #pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt)
        #pragma unroll
        for (int k = 0; k < 16; ++k) red[((wave * kRowTiles + rt) * 16 + k) * 64 + lane] = acc[rt][k];
    __syncthreads();
    constexpr int kOut = kRowTiles * 16 * 64;
    for (int o = threadIdx.x; o < kOut; o += blockDim.x) {
        float s = 0.f;
        for (int w = 0; w < n_waves; ++w) s += red[w * kOut + o];
        const int ln = o & 63, k = (o >> 6) & 15, rt = o >> 10;
        const int row = row0 + rt * 32 + (ln & 31);
        const int t = tile * kTokTile + 4 * (ln >> 5) + 8 * (k >> 2) + (k & 3);
        if (row < M.rows && t < p.n_tokens) M.y[static_cast<int64_t>(t) * M.ldy + row] = s;
    }
}

int check_batched(const char *where, const float *x, int ldx, int cols, int n_tokens) {
    if (!x || n_tokens < 0) return fail(QK_ERR_INVALID_ARG, std::string(where) + ": null x or negative count");
    if (ldx < cols) return fail(QK_ERR_INVALID_ARG, std::string(where) + ": ldx smaller than cols");
    if (!aligned(x, 16) || ldx % 4)
        return fail(QK_ERR_ALIGN, std::string(where) + ": x and ldx must keep 16-byte alignment");
    return QK_OK;
}

size_t workspace_bytes(int cols, int n_tokens) {
    if (cols <= 0 || cols % 256 || n_tokens <= 0) return 0;
    const size_t tiles = (static_cast<size_t>(n_tokens) + kTokTile - 1) / kTokTile;
    return tiles * static_cast<size_t>(cols / 256) * kRecBytes;
}

int launch_mfma(const qk_matrix *mats, int n_mats, const int *ldy, const float *x, int ldx, int cols, int n_tokens,
                void *workspace, size_t workspace_size, hipStream_t stream, const char *where) {
    const size_t need = workspace_bytes(cols, n_tokens);
    if (!workspace || workspace_size < need)
        return fail(QK_ERR_INVALID_ARG, std::string(where) + ": workspace smaller than " + std::to_string(need) +
                                            " bytes (qk_gemv_batched_workspace_bytes)");
    if (!aligned(workspace, 16)) return fail(QK_ERR_ALIGN, std::string(where) + ": workspace not 16-byte aligned");
    const int nb = cols / 256;
    const int tiles = (n_tokens + kTokTile - 1) / kTokTile;
    if (tiles > 65535) return fail(QK_ERR_LIMIT, std::string(where) + ": too many tokens in one launch");
    BatchParams p{};
    p.n_mats = n_mats;
    p.ws = static_cast<const uint8_t *>(workspace);
    p.nb = nb;
    p.n_tokens = n_tokens;
    int64_t groups = 0;
    int type = mats[0].type;
    for (int i = 0; i < n_mats; ++i) {
        BatchMatrix &M = p.mat[i];
        M.w = static_cast<const uint8_t *>(mats[i].w);
        M.y = mats[i].y;
        M.rows = mats[i].rows;
        M.type = mats[i].type;
        M.row_bytes = nb * block_bytes(M.type);
        M.ldy = ldy[i];
        M.group_begin = static_cast<int>(groups);
        groups += (M.rows + kGroupRows - 1) / kGroupRows;
        if (static_cast<int64_t>(M.rows) * M.row_bytes > (int64_t(1) << 40))
            return fail(QK_ERR_LIMIT, std::string(where) + ": matrix too large");
        if (M.type != type) type = 0;
    }
    if (groups > (1 << 30)) return fail(QK_ERR_LIMIT, std::string(where) + ": too many rows");
    // Split a row group's blocks over up to kMaxSplit waves until about 2048
    // waves are in flight.
    const int64_t base = groups * tiles;
    int split = static_cast<int>(std::min<int64_t>(kMaxSplit, std::max<int64_t>(1, 2048 / std::max<int64_t>(1, base))));
    split = std::min(split, nb);
    p.blocks_per_wave = (nb + split - 1) / split;
    split = (nb + p.blocks_per_wave - 1) / p.blocks_per_wave;
    const size_t lds = split > 1 ? static_cast<size_t>(split) * kRowTiles * 16 * 64 * sizeof(float) : 0;

    hipLaunchKernelGGL(pack_activations, dim3(nb, tiles), dim3(256), 0, stream, x, ldx, n_tokens, nb,
                       static_cast<uint8_t *>(workspace));
    const dim3 grid(static_cast<unsigned>(groups), tiles), block(64 * split);
    if (type == QK_TYPE_Q4_K)
        hipLaunchKernelGGL(batch_mfma<QK_TYPE_Q4_K>, grid, block, lds, stream, p);
    else if (type == QK_TYPE_Q6_K)
        hipLaunchKernelGGL(batch_mfma<QK_TYPE_Q6_K>, grid, block, lds, stream, p);
    else
        hipLaunchKernelGGL(batch_mfma<0>, grid, block, lds, stream, p);
    return launch_status(where);
}

}  // namespace
}  // namespace qk

extern "C" {

size_t qk_gemv_batched_workspace_bytes(int cols, int n_tokens) {
    return qk::workspace_bytes(cols, n_tokens);
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
