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
//   The grid covers the resident capacity and walks tiles grid-stride; a
//   tile's loads are issued before the previous tile's arithmetic.
//   blockIdx.y selects the token when several tokens share the weights.
#include "qk_internal.h"

#include <algorithm>

namespace qk {
namespace {

constexpr int kMaxChunks = 16;

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
};

struct Raw {
    uint4 a, b, c;
    uint2 s;
    uint32_t d;
};

struct TileRef {
    const uint8_t *blk;
    float *y;
    int row;
    int type;
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
    t.y = M.y + static_cast<int64_t>(token) * M.ldy;
    const int bpb = M.type == QK_TYPE_Q4_K ? 144 : 210;
    t.blk = M.w + static_cast<size_t>(row) * M.row_bytes + static_cast<size_t>(piece_block) * bpb;
    return t;
}

__device__ __forceinline__ Raw fetch(const TileRef &t, int g, int h) {
    Raw r;
    if (t.type == QK_TYPE_Q4_K) {
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

// 6-bit scale / min of Q4_K sub-blocks 4g + part (q4_scale_min,
// inferencer.cu:489-497), one per byte.
__device__ __forceinline__ void q4k_scale_min4(const uint4 &hdr, int g, uint32_t &sc, uint32_t &mn) {
    const uint32_t M = 0x0F0F0F0Fu;
    const uint32_t s03 = hdr.y, s47 = hdr.z, s811 = hdr.w;
    sc = g ? ((s811 & M) | ((s03 >> 2) & 0x30303030u)) : (s03 & 0x3F3F3F3Fu);
    mn = g ? (((s811 >> 4) & M) | ((s47 >> 2) & 0x30303030u)) : (s47 & 0x3F3F3F3Fu);
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

struct F32Policy {
    struct Lane {
        float xr[64];
        float X[4];
    };

    __device__ static void load(Lane &L, const GemvParams &p, int token, int piece) {
        const int b = piece >> 2, g = (piece >> 1) & 1, h = piece & 1;
        const float *xs = static_cast<const float *>(p.x) + static_cast<int64_t>(token) * p.ldx + b * 256 + g * 128 +
                          h * 16;
        #pragma unroll
        for (int part = 0; part < 4; ++part) {
            float s = 0.f;
            #pragma unroll
            for (int k = 0; k < 4; ++k) {
                float4 v = *reinterpret_cast<const float4 *>(xs + part * 32 + k * 4);
                L.xr[part * 16 + 4 * k + 0] = v.x;
                L.xr[part * 16 + 4 * k + 1] = v.y;
                L.xr[part * 16 + 4 * k + 2] = v.z;
                L.xr[part * 16 + 4 * k + 3] = v.w;
                s += (v.x + v.y) + (v.z + v.w);
            }
            L.X[part] = s;
        }
    }

    __device__ static float q4k(const Raw &r, const Lane &L, int g) {
        const uint32_t M = 0x0F0F0F0Fu;
        float S[4] = {0.f, 0.f, 0.f, 0.f};
        const uint32_t qa[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t qb[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        #pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t c[4] = {qa[k] & M, (qa[k] >> 4) & M, qb[k] & M, (qb[k] >> 4) & M};
            #pragma unroll
            for (int part = 0; part < 4; ++part) {
                const float *x = L.xr + part * 16 + 4 * k;
                S[part] = fmaf(ubyte0(c[part]), x[0], S[part]);
                S[part] = fmaf(ubyte1(c[part]), x[1], S[part]);
                S[part] = fmaf(ubyte2(c[part]), x[2], S[part]);
                S[part] = fmaf(ubyte3(c[part]), x[3], S[part]);
            }
        }
        uint32_t sc, mn;
        q4k_scale_min4(r.a, g, sc, mn);
        const float d = f16_bits_to_f32(r.a.x & 0xFFFFu);
        const float dmin = f16_bits_to_f32(r.a.x >> 16);
        float a = ubyte0(sc) * S[0];
        a = fmaf(ubyte1(sc), S[1], a);
        a = fmaf(ubyte2(sc), S[2], a);
        a = fmaf(ubyte3(sc), S[3], a);
        float b = ubyte0(mn) * L.X[0];
        b = fmaf(ubyte1(mn), L.X[1], b);
        b = fmaf(ubyte2(mn), L.X[2], b);
        b = fmaf(ubyte3(mn), L.X[3], b);
        return fmaf(d, a, -dmin * b);
    }

    __device__ static float q6k(const Raw &r, const Lane &L, int h) {
        float S[4] = {0.f, 0.f, 0.f, 0.f};
        const uint32_t la[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
        const uint32_t lb[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
        const uint32_t qh[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
        #pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t c[4];
            q6k_codes(la[k], lb[k], qh[k], c[0], c[1], c[2], c[3]);
            #pragma unroll
            for (int part = 0; part < 4; ++part) {
                const float *x = L.xr + part * 16 + 4 * k;
                S[part] = fmaf(ubyte0(c[part]), x[0], S[part]);
                S[part] = fmaf(ubyte1(c[part]), x[1], S[part]);
                S[part] = fmaf(ubyte2(c[part]), x[2], S[part]);
                S[part] = fmaf(ubyte3(c[part]), x[3], S[part]);
            }
        }
        float sc[4];
        q6k_scales(r.s, h, sc);
        float a = sc[0] * fmaf(-32.f, L.X[0], S[0]);
        a = fmaf(sc[1], fmaf(-32.f, L.X[1], S[1]), a);
        a = fmaf(sc[2], fmaf(-32.f, L.X[2], S[2]), a);
        a = fmaf(sc[3], fmaf(-32.f, L.X[3], S[3]), a);
        return f16_bits_to_f32(r.d) * a;
    }
};

// ------------------------------------------------------------ INT8 path --

struct I8Policy {
    struct Lane {
        int xq[16];       // the piece's 64 int8 activations, 4 per dword
        int xs[4];        // sum of the 16 int8 values of each part
        float scale[4];   // activation scale of each part's 32-value group
    };

    __device__ static void load(Lane &L, const GemvParams &p, int token, int piece) {
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

template <class Policy>
__device__ __forceinline__ float piece_dot(const TileRef &t, const Raw &r, const typename Policy::Lane &L, int g,
                                           int h) {
    return t.type == QK_TYPE_Q4_K ? Policy::q4k(r, L, g) : Policy::q6k(r, L, h);
}

__device__ __forceinline__ float group_sum(float v, int group_lanes) {
    #pragma unroll 1
    for (int off = group_lanes >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// C == 1: every tile lives inside one wave; no LDS, no barriers.
template <class Policy>
__global__ __launch_bounds__(256) void gemv_wave(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n_waves = blockDim.x >> 6;
    const int token = blockIdx.y;
    const int rit = lane / p.pieces;
    const int piece = lane - rit * p.pieces;
    const int g = (piece >> 1) & 1, h = piece & 1;
    typename Policy::Lane L;
    Policy::load(L, p, token, piece);

    const int stride = gridDim.x * n_waves;
    int tile = blockIdx.x * n_waves + wave;
    if (tile >= p.total_tiles) return;
    TileRef cur = locate(p, tile, rit, piece >> 2, token);
    Raw rc = fetch(cur, g, h);
    while (true) {
        const int next = tile + stride;
        const bool more = next < p.total_tiles;
        TileRef nt;
        Raw rn;
        if (more) {
            nt = locate(p, next, rit, piece >> 2, token);
            rn = fetch(nt, g, h);
        }
        const float v = group_sum(piece_dot<Policy>(cur, rc, L, g, h), p.group_lanes);
        if (piece == 0 && cur.valid) cur.y[cur.row] = v;
        if (!more) break;
        tile = next;
        cur = nt;
        rc = rn;
    }
}

// C > 1: the C waves of a wave-group share each tile; group sums meet in LDS.
template <class Policy>
__global__ __launch_bounds__(1024) void gemv_split(GemvParams p) {
    extern __shared__ float red[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int token = blockIdx.y;
    const int chunk = wave % p.chunks;
    const int wgroup = wave / p.chunks;
    const int n_wgroups = (blockDim.x >> 6) / p.chunks;
    const int q = chunk * 64 + lane;
    const int rit = q / p.pieces;
    const int piece = q - rit * p.pieces;
    const int g = (piece >> 1) & 1, h = piece & 1;
    const int slots = p.tile_rows * p.chunks;      // group sums per tile
    typename Policy::Lane L;
    Policy::load(L, p, token, piece);

    const int per_iter = gridDim.x * n_wgroups;
    const int iters = (p.total_tiles + per_iter - 1) / per_iter;
    int tile = blockIdx.x * n_wgroups + wgroup;
    bool have = tile < p.total_tiles;
    TileRef cur{};
    Raw rc{};
    if (have) {
        cur = locate(p, tile, rit, piece >> 2, token);
        rc = fetch(cur, g, h);
    }
    for (int it = 0; it < iters; ++it) {
        const int next = tile + per_iter;
        const bool have_next = next < p.total_tiles;
        TileRef nt{};
        Raw rn{};
        if (have_next) {
            nt = locate(p, next, rit, piece >> 2, token);
            rn = fetch(nt, g, h);
        }
        float v = have ? piece_dot<Policy>(cur, rc, L, g, h) : 0.f;
        v = group_sum(v, p.group_lanes);
        float *buf = red + (wgroup * 2 + (it & 1)) * slots;
        if ((lane & (p.group_lanes - 1)) == 0) buf[q / p.group_lanes] = v;
        __syncthreads();
        if (have && chunk == 0 && lane < p.tile_rows) {
            // Row `lane` of the tile: its C group sums, added in chunk order.
            const TileRef rowref = locate(p, tile, lane, 0, token);
            if (rowref.valid) {
                float s = 0.f;
                for (int c = 0; c < p.chunks; ++c) s += buf[lane * p.chunks + c];
                rowref.y[rowref.row] = s;
            }
        }
        tile = next;
        have = have_next;
        cur = nt;
        rc = rn;
    }
}

// Rows whose chunk count exceeds kMaxChunks: one wave per row, lanes stride
// over the pieces and reload each piece's activations through the cache.
template <class Policy>
__global__ __launch_bounds__(256) void gemv_long(GemvParams p) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n_waves = blockDim.x >> 6;
    const int token = blockIdx.y;
    for (int tile = blockIdx.x * n_waves + wave; tile < p.total_tiles; tile += gridDim.x * n_waves) {
        float acc = 0.f;
        for (int piece = lane; piece < p.pieces; piece += 64) {
            const int g = (piece >> 1) & 1, h = piece & 1;
            typename Policy::Lane L;
            Policy::load(L, p, token, piece);
            const TileRef t = locate(p, tile, 0, piece >> 2, token);
            const Raw r = fetch(t, g, h);
            acc += piece_dot<Policy>(t, r, L, g, h);
        }
        acc = group_sum(acc, 64);
        const TileRef t = locate(p, tile, 0, 0, token);
        if (lane == 0 && t.valid) t.y[t.row] = acc;
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

int resident_blocks(const void *kernel, int block, size_t lds) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    return per_cu * device_info().cus;
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
    const bool long_rows = p.chunks > kMaxChunks;
    if (long_rows) p.tile_rows = 1;
    int64_t tiles = 0;
    for (int m = 0; m < n_mats; ++m) {
        GemvMatrix &M = p.mat[m];
        M.w = static_cast<const uint8_t *>(mats[m].w);
        M.y = mats[m].y;
        M.rows = mats[m].rows;
        M.type = mats[m].type;
        M.row_bytes = nb * block_bytes(M.type);
        M.ldy = ldy ? ldy[m] : M.rows;
        M.tile_begin = static_cast<int>(tiles);
        tiles += (M.rows + p.tile_rows - 1) / p.tile_rows;
        if (static_cast<int64_t>(M.rows) * M.row_bytes > (int64_t(1) << 40))
            return fail(QK_ERR_LIMIT, std::string(where) + ": matrix too large");
    }
    if (tiles > (1 << 30)) return fail(QK_ERR_LIMIT, std::string(where) + ": too many rows");
    if (n_tokens > 65535) return fail(QK_ERR_LIMIT, std::string(where) + ": too many tokens in one launch");
    p.total_tiles = static_cast<int>(tiles);

    if (long_rows) {
        const int block = 256, waves = block / 64;
        const int grid = std::max(1, std::min<int>((p.total_tiles + waves - 1) / waves, device_info().cus * 8));
        hipLaunchKernelGGL(gemv_long<Policy>, dim3(grid, n_tokens), dim3(block), 0, stream, p);
    } else if (p.chunks == 1) {
        const int block = 256, waves = block / 64;
        const int cap = std::max(1, resident_blocks(reinterpret_cast<const void *>(gemv_wave<Policy>), block, 0) /
                                        n_tokens);
        const int grid = std::max(1, std::min<int>((p.total_tiles + waves - 1) / waves, cap));
        hipLaunchKernelGGL(gemv_wave<Policy>, dim3(grid, n_tokens), dim3(block), 0, stream, p);
    } else {
        const int wgroups = std::max(1, 4 / p.chunks);
        const int block = wgroups * p.chunks * 64;
        const size_t lds = static_cast<size_t>(wgroups) * 2 * p.tile_rows * p.chunks * sizeof(float);
        const int cap = std::max(1, resident_blocks(reinterpret_cast<const void *>(gemv_split<Policy>), block, lds) /
                                        n_tokens);
        const int grid = std::max(1, std::min<int>((p.total_tiles + wgroups - 1) / wgroups, cap));
        hipLaunchKernelGGL(gemv_split<Policy>, dim3(grid, n_tokens), dim3(block), lds, stream, p);
    }
    return launch_status(where);
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
    qk::GemvParams p{};
    p.x = xq;
    p.xscale = xscale;
    p.ldx = ldxq;
    p.ldscale = ldscale;
    const qk_matrix m{type, rows, w, y};
    return qk::launch<qk::I8Policy>(p, &m, 1, cols, n_tokens, &ldy, static_cast<hipStream_t>(stream),
                                    "qk_gemv_i8 launch");
}

}  // extern "C"
