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
// Three kernels:
//   pack_activations  once per (block, 32-token tile): x -> the record of
//                     MFMA A operands (fp16 hi / lo, sub-block sums, scales)
//                     in the caller's workspace.
//   batch_mfma        a workgroup (4 waves) owns 128 weight rows x one token
//                     tile x a run of blocks.  Per block it copies the record
//                     into LDS (double-buffered: the next record and the next
//                     block's weight bytes load while this block computes) and
//                     each wave decodes the raw bytes of its 32 rows into MFMA
//                     B operands in registers (lane l: row l%32, block half
//                     l/32).  When one row group's blocks are split over
//                     several workgroups (to put enough waves on the chip),
//                     each writes its partial sums to the workspace;
//   reduce_splits     adds them in split order, so results are deterministic.
#include "qk_internal.h"

#include <algorithm>

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
constexpr int kGroupRows = 128;         // weight rows per workgroup (4 waves x 32)
constexpr int kMaxSplit = 4;            // workgroups splitting one row group's blocks
constexpr int kTargetGroups = 512;      // two workgroups per CU

// LDS tile of one block's activations for one 32-token tile, in MFMA A
// operand order:
//   hi   [16 steps][2 halves][32 tokens][8]  fp16   16 KiB
//   lo   same                                fp16   16 KiB
//   mhi  [2 halves][32 tokens][4]            fp16   512 B  (sub-block sums / 64)
//   mlo  same                                fp16   512 B
//   f    [2 halves][16]                      fp32   128 B  (2^-shift per token, lane order)
constexpr int kTileA = 16384;
constexpr int kTileM = 512;
constexpr int kTileF = 128;
constexpr int kTileBytes = 2 * kTileA + 2 * kTileM + kTileF;
static_assert(kTileBytes % 16 == 0, "tiles keep 16-byte alignment");

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
    int group_begin;   // first 128-row group of this matrix in the launch
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
    float *partials;        // [group][tile][split][4096] when splits > 1
    const uint8_t *records; // packed activations, [tile][block][kTileBytes]
};

// ---------------------------------------------------- activation staging --
//
// Thread (tl = tid/8, q = tid%8) owns token tl of the tile and the 32
// columns q*32 .. q*32+31 (Q4_K sub-block q) of the block.

struct XStage {
    float v[32];
};

__device__ __forceinline__ void stage_load(const BatchParams &p, int tile, int b, XStage &s) {
    const int tl = threadIdx.x >> 3, q = threadIdx.x & 7;
    const int t = tile * kTokTile + tl;
    if (t < p.n_tokens) {
        const float4 *src = reinterpret_cast<const float4 *>(p.x + static_cast<int64_t>(t) * p.ldx + b * 256 + q * 32);
        #pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 u = src[i];
            s.v[4 * i] = u.x;
            s.v[4 * i + 1] = u.y;
            s.v[4 * i + 2] = u.z;
            s.v[4 * i + 3] = u.w;
        }
    } else {
        #pragma unroll
        for (int i = 0; i < 32; ++i) s.v[i] = 0.f;
    }
}

// x' = x * 2^shift with the block maximum of the token in [2^14, 2^15)
// (shift capped at 140 so 2^-shift stays a nonzero fp32), split into fp16
// hi + lo; a non-finite activation makes the token's scale NaN.
__device__ __forceinline__ void stage_store(const XStage &s, uint8_t *tile) {
    const int tl = threadIdx.x >> 3, q = threadIdx.x & 7;
    float m = 0.f;
    bool bad = false;
    #pragma unroll
    for (int i = 0; i < 32; ++i) {
        m = fmaxf(m, fabsf(s.v[i]));
        bad |= !isfinite(s.v[i]);
    }
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    m = fmaxf(m, __shfl_xor(m, 4));
    int nb_bad = bad ? 1 : 0;
    nb_bad |= __shfl_xor(nb_bad, 1);
    nb_bad |= __shfl_xor(nb_bad, 2);
    nb_bad |= __shfl_xor(nb_bad, 4);
    int shift = 0;
    float f = 0.f;
    if (m > 0.f && isfinite(m)) {
        shift = min(15 - __builtin_amdgcn_frexp_expf(m), 140);
        f = ldexpf(1.f, -shift);
    }
    if (nb_bad) f = __builtin_nanf("");

    _Float16 *hi = reinterpret_cast<_Float16 *>(tile);
    _Float16 *lo = reinterpret_cast<_Float16 *>(tile + kTileA);
    const int G = q >> 1, half = q & 1, kh = G >> 1, hf = G & 1;
    float sum = 0.f;
    #pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int st = hf * 8 + j;
        half4 h4, l4;
        #pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float xs = nb_bad ? 0.f : ldexpf(s.v[4 * j + i], shift);
            sum += xs;
            const _Float16 h = static_cast<_Float16>(xs);
            const int e = (i == 1) ? 2 : (i == 2) ? 1 : i;   // column order {0, 2, 1, 3}
            h4[e] = h;
            l4[e] = static_cast<_Float16>(xs - static_cast<float>(h));
        }
        const int at = ((st * 2 + kh) * 32 + tl) * 8 + half * 4;
        *reinterpret_cast<half4 *>(hi + at) = h4;
        *reinterpret_cast<half4 *>(lo + at) = l4;
    }
    // |sum| < 32 * 2^15: stored / 64 to stay inside the fp16 range.
    const float s64 = sum * (1.f / 64.f);
    const _Float16 sh = static_cast<_Float16>(s64);
    _Float16 *mhi = reinterpret_cast<_Float16 *>(tile + 2 * kTileA);
    _Float16 *mlo = reinterpret_cast<_Float16 *>(tile + 2 * kTileA + kTileM);
    const int mat = ((q >> 2) * 32 + tl) * 4 + (q & 3);
    mhi[mat] = sh;
    mlo[mat] = static_cast<_Float16>(s64 - static_cast<float>(sh));
    // Token scales in accumulator lane order: lane half (tl/4)%2, register 4*(tl/8) + tl%4.
    if (q == 0) {
        float *fr = reinterpret_cast<float *>(tile + 2 * kTileA + 2 * kTileM);
        fr[((tl >> 2) & 1) * 16 + 4 * (tl >> 3) + (tl & 3)] = f;
    }
}

// One workgroup per (block, 32-token tile): the tile's activations of the
// block, packed once into the workspace record the GEMM copies into LDS.
__global__ __launch_bounds__(256) void pack_activations(BatchParams p, uint8_t *__restrict__ records) {
    const int b = blockIdx.x, tile = blockIdx.y;
    XStage xs;
    stage_load(p, tile, b, xs);
    stage_store(xs, records + (static_cast<size_t>(tile) * p.nb + b) * kTileBytes);
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
        const uint2 sc = load8(blk + 192 + kh * 8);
        r.hdr = make_uint4(sc.x, sc.y, load2(blk + 208), 0);
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

__device__ __forceinline__ _Float16 u8_to_h(uint32_t v) { return static_cast<_Float16>(static_cast<float>(v & 0xFFu)); }
__device__ __forceinline__ _Float16 s8_to_h(uint32_t v) {
    return static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(v & 0xFFu)));
}

// acc += this block's contribution (32 tokens x the lane's row).
template <int TYPE>
__device__ __forceinline__ void block_mfma(const RawBlock &r, int type, const uint8_t *tile_lds, int kh, int col,
                                           float16v &acc) {
    const float4 *fr = reinterpret_cast<const float4 *>(tile_lds + 2 * kTileA + 2 * kTileM) + kh * 4;
    float f[16];
    #pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 u = fr[i];
        f[4 * i] = u.x;
        f[4 * i + 1] = u.y;
        f[4 * i + 2] = u.z;
        f[4 * i + 3] = u.w;
    }
    float d, dmin = 0.f;
    uint32_t sc4 = 0, mn4 = 0;
    if (is_q4<TYPE>(type)) {
        d = f16_bits_to_f32(r.hdr.x & 0xFFFFu);
        dmin = f16_bits_to_f32(r.hdr.x >> 16);
        q4k_scale_min4(r.hdr, kh, sc4, mn4);
    } else {
        d = f16_bits_to_f32(r.hdr.z);
    }
    const half8 *ahp = reinterpret_cast<const half8 *>(tile_lds) + kh * 32 + col;
    const half8 *alp = reinterpret_cast<const half8 *>(tile_lds + kTileA) + kh * 32 + col;
    float16v t;
    #pragma unroll
    for (int k = 0; k < 16; ++k) t[k] = 0.f;
    #pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        #pragma unroll
        for (int j = 0; j < 8; ++j) {
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
            const half2v sa2 = {sa, sa}, sb2 = {sb, sb};
            const half2v ba2 = {static_cast<_Float16>(off * sa), static_cast<_Float16>(off * sa)};
            const half2v bb2 = {static_cast<_Float16>(off * sb), static_cast<_Float16>(off * sb)};
            const half8 bw = decode_b<TYPE>(r, type, hf, j, sa2, ba2, sb2, bb2);
            const int st = hf * 8 + j;
            t = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahp[st * 64], bw, t, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_32x32x16_f16(alp[st * 64], bw, t, 0, 0, 0);
        }
    }
    #pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] = fmaf(d * f[k], t[k], acc[k]);
    if (is_q4<TYPE>(type)) {
        const half4 mh = reinterpret_cast<const half4 *>(tile_lds + 2 * kTileA)[kh * 32 + col];
        const half4 ml = reinterpret_cast<const half4 *>(tile_lds + 2 * kTileA + kTileM)[kh * 32 + col];
        half4 bm;
        #pragma unroll
        for (int e = 0; e < 4; ++e) bm[e] = u8_to_h(mn4 >> (8 * e));
        float16v tm;
        #pragma unroll
        for (int k = 0; k < 16; ++k) tm[k] = 0.f;
        tm = __builtin_amdgcn_mfma_f32_32x32x8f16(mh, bm, tm, 0, 0, 0);
        tm = __builtin_amdgcn_mfma_f32_32x32x8f16(ml, bm, tm, 0, 0, 0);
        #pragma unroll
        for (int k = 0; k < 16; ++k) acc[k] = fmaf(-64.f * dmin * f[k], tm[k], acc[k]);
    }
}

// ---------------------------------------------------------------- GEMM --
//
// Workgroup = 4 waves = 128 weight rows (32 per wave, lane l -> row l%32,
// block half l/32) x one 32-token tile x a run of blocks.  Per block the
// workgroup stages the activations once in LDS (double-buffered) and each
// wave decodes its rows' raw block bytes into MFMA B operands; the next
// block's activations and weight bytes are loaded while this one computes.

// Copy of one packed record into LDS in 16-byte chunks: the 2048 chunks of
// the fp16 operands, eight per thread, then the 72 chunks of sums and
// scales (every thread loads one, clamped; the first 72 store theirs).
constexpr int kChunks = kTileBytes / 16;
constexpr int kMainChunks = 2 * kTileA / 16;
constexpr int kTailChunks = kChunks - kMainChunks;
static_assert(kMainChunks == 8 * 256 && kTailChunks <= 256, "record copy layout");

struct RecordStage {
    uint4 v[8];
    uint4 tail;
};

__device__ __forceinline__ void record_load(const uint8_t *rec, RecordStage &s) {
    const uint4 *src = reinterpret_cast<const uint4 *>(rec);
    #pragma unroll
    for (int i = 0; i < 8; ++i) s.v[i] = src[i * 256 + threadIdx.x];
    s.tail = src[kMainChunks + min(static_cast<int>(threadIdx.x), kTailChunks - 1)];
}

__device__ __forceinline__ void record_store(const RecordStage &s, uint8_t *tile_lds) {
    uint4 *dst = reinterpret_cast<uint4 *>(tile_lds);
    #pragma unroll
    for (int i = 0; i < 8; ++i) dst[i * 256 + threadIdx.x] = s.v[i];
    if (threadIdx.x < kTailChunks) dst[kMainChunks + threadIdx.x] = s.tail;
}

template <int TYPE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void batch_mfma(BatchParams p) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kh = lane >> 5, col = lane & 31;
    const int split = blockIdx.x % p.splits, group = blockIdx.x / p.splits, tile = blockIdx.y;

    int m = 0;
    #pragma unroll
    for (int i = 1; i < QK_MAX_FUSED; ++i) m += (i < p.n_mats && group >= p.mat[i].group_begin) ? 1 : 0;
    m = __builtin_amdgcn_readfirstlane(m);
    const BatchMatrix &M = p.mat[m];
    const int type = TYPE ? TYPE : M.type;
    const int bpb = is_q4<TYPE>(type) ? 144 : 210;
    const int row = (group - M.group_begin) * kGroupRows + wave * 32 + col;
    const uint8_t *wrow = M.w + static_cast<size_t>(min(row, M.rows - 1)) * M.row_bytes;
    const uint8_t *recs = p.records + static_cast<size_t>(tile) * p.nb * kTileBytes;

    const int b0 = split * p.blocks_per_split;
    const int b1 = min(p.nb, b0 + p.blocks_per_split);
    RecordStage rs;
    record_load(recs + static_cast<size_t>(b0) * kTileBytes, rs);
    RawBlock cur = load_block<TYPE>(wrow + b0 * bpb, type, kh);
    record_store(rs, lds);
    __syncthreads();

    float16v acc;
    #pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] = 0.f;
    for (int b = b0; b < b1; ++b) {
        const int buf = (b - b0) & 1;
        // The last iteration reloads its own block (unconditional, in bounds).
        const int bn = min(b + 1, b1 - 1);
        record_load(recs + static_cast<size_t>(bn) * kTileBytes, rs);
        const RawBlock nxt = load_block<TYPE>(wrow + bn * bpb, type, kh);
        block_mfma<TYPE>(cur, type, lds + buf * kTileBytes, kh, col, acc);
        record_store(rs, lds + (buf ^ 1) * kTileBytes);
        cur = nxt;
        __syncthreads();
    }

    // Accumulator register k holds token 8*(k/4) + 4*kh + k%4 of the tile.
    const int tbase = tile * kTokTile + 4 * kh;
    if (p.splits == 1) {
        if (row < M.rows) {
            #pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int t = tbase + 8 * (k >> 2) + (k & 3);
                if (t < p.n_tokens) M.y[static_cast<int64_t>(t) * M.ldy + row] = acc[k];
            }
        }
        return;
    }

    // Split blocks: the partial sums go to the workspace in accumulator
    // order; reduce_splits adds them.
    const size_t slot = static_cast<size_t>(group) * p.tiles + tile;
    float *mine = p.partials + (slot * p.splits + split) * 4096 + wave * 1024 + lane;
    #pragma unroll
    for (int k = 0; k < 16; ++k) mine[k * 64] = acc[k];
}

// y = the sum of a row group's split partials, in split order (deterministic).
// One workgroup per (row group, tile); thread (wave, lane) owns the 16
// outputs the same thread of batch_mfma produced.
__global__ __launch_bounds__(256) void reduce_splits(BatchParams p) {
    const int group = blockIdx.x, tile = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kh = lane >> 5, col = lane & 31;
    int m = 0;
    #pragma unroll
    for (int i = 1; i < QK_MAX_FUSED; ++i) m += (i < p.n_mats && group >= p.mat[i].group_begin) ? 1 : 0;
    const BatchMatrix &M = p.mat[m];
    const int row = (group - M.group_begin) * kGroupRows + wave * 32 + col;
    const size_t slot = static_cast<size_t>(group) * p.tiles + tile;
    const float *part = p.partials + slot * p.splits * 4096 + wave * 1024 + lane;
    const int tbase = tile * kTokTile + 4 * kh;
    // Every load is issued before the first add: the kernel is latency-bound.
    float v[kMaxSplit][16];
    #pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp)
        #pragma unroll
        for (int k = 0; k < 16; ++k) v[sp][k] = sp < p.splits ? part[sp * 4096 + k * 64] : 0.f;
    #pragma unroll
    for (int k = 0; k < 16; ++k) {
        float s = v[0][k];
        #pragma unroll
        for (int sp = 1; sp < kMaxSplit; ++sp) s += v[sp][k];
        const int t = tbase + 8 * (k >> 2) + (k & 3);
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

int tile_count(int n_tokens) { return (n_tokens + kTokTile - 1) / kTokTile; }

// Workgroups sharing a row group's blocks: enough that about kTargetGroups
// workgroups run, at most kMaxSplit, at least two blocks each.
void split_plan(int64_t rows_total, int nb, int tiles, int &splits, int &per_split) {
    const int64_t groups = std::max<int64_t>(1, (rows_total + kGroupRows - 1) / kGroupRows);
    const int64_t want = (kTargetGroups + groups * tiles - 1) / (groups * tiles);
    int s = static_cast<int>(std::min<int64_t>(std::max<int64_t>(want, 1), std::min(kMaxSplit, std::max(1, nb / 2))));
    per_split = (nb + s - 1) / s;
    splits = (nb + per_split - 1) / per_split;
}

size_t records_bytes(int cols, int n_tokens) {
    return static_cast<size_t>(tile_count(n_tokens)) * (cols / 256) * kTileBytes;
}

// Workspace: packed activation records, then (when blocks are split) one
// counter per (row group, tile) and the partial sums.
size_t workspace_bytes(int cols, int64_t rows_total, int n_tokens) {
    if (cols <= 0 || cols % 256 || rows_total <= 0 || n_tokens < kMfmaMinTokens) return 0;
    const int tiles = tile_count(n_tokens);
    size_t bytes = (records_bytes(cols, n_tokens) + 255) / 256 * 256;
    int splits, per_split;
    split_plan(rows_total, cols / 256, tiles, splits, per_split);
    if (splits == 1) return bytes;
    const int64_t groups = (rows_total + kGroupRows - 1) / kGroupRows + QK_MAX_FUSED - 1;
    return bytes + static_cast<size_t>(groups) * tiles * splits * 4096 * sizeof(float);
}

int launch_mfma(const qk_matrix *mats, int n_mats, const int *ldy, const float *x, int ldx, int cols, int n_tokens,
                void *workspace, size_t workspace_size, hipStream_t stream, const char *where) {
    const int nb = cols / 256;
    const int tiles = tile_count(n_tokens);
    if (tiles > 65535) return fail(QK_ERR_LIMIT, std::string(where) + ": too many tokens in one launch");
    BatchParams p{};
    p.n_mats = n_mats;
    p.x = x;
    p.ldx = ldx;
    p.n_tokens = n_tokens;
    p.nb = nb;
    p.tiles = tiles;
    int64_t groups = 0, rows_total = 0;
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
        rows_total += M.rows;
        if (static_cast<int64_t>(M.rows) * M.row_bytes > (int64_t(1) << 40))
            return fail(QK_ERR_LIMIT, std::string(where) + ": matrix too large");
        if (M.type != type) type = 0;
    }
    split_plan(rows_total, nb, tiles, p.splits, p.blocks_per_split);
    if (groups * p.splits > (1 << 30)) return fail(QK_ERR_LIMIT, std::string(where) + ": too many rows");
    const size_t need = workspace_bytes(cols, rows_total, n_tokens);
    if (!workspace || workspace_size < need)
        return fail(QK_ERR_INVALID_ARG, std::string(where) + ": workspace smaller than " + std::to_string(need) +
                                            " bytes (qk_gemv_batched_workspace_bytes)");
    if (!aligned(workspace, 256)) return fail(QK_ERR_ALIGN, std::string(where) + ": workspace not 256-byte aligned");
    uint8_t *ws = static_cast<uint8_t *>(workspace);
    p.records = ws;
    if (p.splits > 1) p.partials = reinterpret_cast<float *>(ws + (records_bytes(cols, n_tokens) + 255) / 256 * 256);
    hipLaunchKernelGGL(pack_activations, dim3(nb, tiles), dim3(256), 0, stream, p, ws);
    const dim3 grid(static_cast<unsigned>(groups * p.splits), tiles), block(256);
    const size_t lds = 2 * kTileBytes;
    if (type == QK_TYPE_Q4_K)
        hipLaunchKernelGGL(batch_mfma<QK_TYPE_Q4_K>, grid, block, lds, stream, p);
    else if (type == QK_TYPE_Q6_K)
        hipLaunchKernelGGL(batch_mfma<QK_TYPE_Q6_K>, grid, block, lds, stream, p);
    else
        hipLaunchKernelGGL(batch_mfma<0>, grid, block, lds, stream, p);
    if (p.splits > 1)
        hipLaunchKernelGGL(reduce_splits, dim3(static_cast<unsigned>(groups), tiles), dim3(256), 0, stream, p);
    return launch_status(where);
}

}  // namespace
}  // namespace qk

extern "C" {

size_t qk_gemv_batched_workspace_bytes(int cols, int rows, int n_tokens) {
    return qk::workspace_bytes(cols, rows, n_tokens);
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
