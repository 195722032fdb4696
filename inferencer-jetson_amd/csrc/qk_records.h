// qk_records.h - the matrix-core GEMM's activation records (one block of
// 256 columns for one 32-token tile, in MFMA A-operand order) and the device
// routine that writes them.  Shared by the GEMM's pack and reduction
// kernels (csrc/qk_batched.hip) and by attention, which writes the o
// projection's records itself (csrc/qk_step.hip).
#pragma once

#include "qk_internal.h"

namespace qk {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

constexpr int kTokTile = 32;            // tokens per MFMA tile (the A rows)

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

// One token's 256-value block into its record, by a whole wave: lane (q, j)
// = (lane / 8, lane % 8) holds values q*32 + 4j .. +3 (v).  x' = x * 2^shift
// with the block maximum in [2^14, 2^15) (shift capped at 140 so 2^-shift
// stays a nonzero fp32), split into fp16 hi + lo, each lane writing its own
// quads; the 32-value sums (of x') are taken as a tree over their eight
// lanes; a non-finite value makes the token's scale NaN.
__device__ __forceinline__ void stage_store_wave(const float (&v)[4], int lane, int tl, uint8_t *tile) {
    const int q = lane >> 3, j = lane & 7;
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    int bad = isfinite(v[0]) && isfinite(v[1]) && isfinite(v[2]) && isfinite(v[3]) ? 0 : 1;
    #pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        m = fmaxf(m, __shfl_xor(m, off));
        bad |= __shfl_xor(bad, off);
    }
    int shift = 0;
    float f = 0.f;
    if (m > 0.f && isfinite(m)) {
        shift = min(15 - __builtin_amdgcn_frexp_expf(m), 140);
        f = ldexpf(1.f, -shift);
    }
    if (bad) f = __builtin_nanf("");
    _Float16 *hi = reinterpret_cast<_Float16 *>(tile);
    _Float16 *lo = reinterpret_cast<_Float16 *>(tile + kTileA);
    const int G = q >> 1, half = q & 1, kh = G >> 1, hf = G & 1, st = hf * 8 + j;
    half4 h4, l4;
    float sum = 0.f;
    #pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float xs = bad ? 0.f : ldexpf(v[i], shift);
        sum += xs;
        const _Float16 h = static_cast<_Float16>(xs);
        const int e = (i == 1) ? 2 : (i == 2) ? 1 : i;   // column order {0, 2, 1, 3}
        h4[e] = h;
        l4[e] = static_cast<_Float16>(xs - static_cast<float>(h));
    }
    const int at = ((st * 2 + kh) * 32 + tl) * 8 + half * 4;
    *reinterpret_cast<half4 *>(hi + at) = h4;
    *reinterpret_cast<half4 *>(lo + at) = l4;
    #pragma unroll
    for (int off = 1; off < 8; off <<= 1) sum += __shfl_xor(sum, off);
    if (j == 0) {
        // |sum| < 32 * 2^15: stored / 64 to stay inside the fp16 range.
        const float s64 = sum * (1.f / 64.f);
        const _Float16 sh = static_cast<_Float16>(s64);
        _Float16 *mhi = reinterpret_cast<_Float16 *>(tile + 2 * kTileA);
        _Float16 *mlo = reinterpret_cast<_Float16 *>(tile + 2 * kTileA + kTileM);
        const int mat = ((q >> 2) * 32 + tl) * 4 + (q & 3);
        mhi[mat] = sh;
        mlo[mat] = static_cast<_Float16>(s64 - static_cast<float>(sh));
    }
    if (lane == 0) {
        float *fr = reinterpret_cast<float *>(tile + 2 * kTileA + 2 * kTileM);
        fr[((tl >> 2) & 1) * 16 + 4 * (tl >> 3) + (tl & 3)] = f;
    }
}

}  // namespace qk
