// gemm_h16_device.h -- device helpers shared by the fp16-MFMA prefill
// kernels (gemm_h16.hip, gemm_h16q.hip): the code x scale -> fp16 operand
// conversion, the MFMA fragment layout in LDS, the LDS DMA and the tile order.
// See gemm_h16.hip for the numerics.
#pragma once

#include "wush_device.h"

namespace wush {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kH16Tile = 256;                    // output rows and columns per workgroup
constexpr int kH16Slice = kH16Tile * 32;         // bytes of one K16 slice of one operand (256 rows x 16 halves)
constexpr int kH16Op = 2 * kH16Slice;            // one group of one operand
constexpr int kH16Buf = 2 * kH16Op;              // activations + weights of one group
constexpr int kH16Batch = 4;                     // groups per global load batch
constexpr int kH16NonFinite = 1 << 20;           // row/column shift marking a non-finite scale

// Power of two that moves the largest |scale| of a row (bf16 bits mx, sign
// cleared) into [2^12, 2^13): mx < 2^(e-126) for exponent field e.
__device__ __forceinline__ int h16_shift(uint32_t mx) {
    return mx >= 0x7f80u ? kH16NonFinite : 139 - (int)(mx >> 7);
}

// Largest |bf16| of the n scales of an activation row (pa) and of a weight
// column (pb), as bits with the sign cleared.  Loads go out 8 per row per
// round trip: one at a time, the 2 * G / 8 dependent loads of a long row cost
// a memory latency each.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u16x2 abs_bits2(uint32_t w) {
    return __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
}

template <bool VEC>
__device__ __forceinline__ void h16_row_max(const uint16_t* __restrict__ pa, const uint16_t* __restrict__ pb,
                                            int n, uint32_t& mxa, uint32_t& mxb) {
    u16x2 ma = {0, 0}, mb = {0, 0};
    if constexpr (VEC) {
        const uint4* qa = reinterpret_cast<const uint4*>(pa);
        const uint4* qb = reinterpret_cast<const uint4*>(pb);
        const int n8 = n >> 3;
        int i = 0;
        for (; i + 8 <= n8; i += 8) {
            uint4 va[8], vb[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                va[u] = qa[i + u];
                vb[u] = qb[i + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                ma = __builtin_elementwise_max(ma, __builtin_elementwise_max(abs_bits2(va[u].x), abs_bits2(va[u].y)));
                ma = __builtin_elementwise_max(ma, __builtin_elementwise_max(abs_bits2(va[u].z), abs_bits2(va[u].w)));
                mb = __builtin_elementwise_max(mb, __builtin_elementwise_max(abs_bits2(vb[u].x), abs_bits2(vb[u].y)));
                mb = __builtin_elementwise_max(mb, __builtin_elementwise_max(abs_bits2(vb[u].z), abs_bits2(vb[u].w)));
            }
        }
        for (; i < n8; ++i) {
            const uint4 va = qa[i], vb = qb[i];
            ma = __builtin_elementwise_max(ma, __builtin_elementwise_max(abs_bits2(va.x), abs_bits2(va.y)));
            ma = __builtin_elementwise_max(ma, __builtin_elementwise_max(abs_bits2(va.z), abs_bits2(va.w)));
            mb = __builtin_elementwise_max(mb, __builtin_elementwise_max(abs_bits2(vb.x), abs_bits2(vb.y)));
            mb = __builtin_elementwise_max(mb, __builtin_elementwise_max(abs_bits2(vb.z), abs_bits2(vb.w)));
        }
    } else {
        int i = 0;
        for (; i + 16 <= n; i += 16) {
            uint32_t va[16], vb[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                va[u] = pa[i + u];
                vb[u] = pb[i + u];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                ma = __builtin_elementwise_max(ma, abs_bits2(va[u]));
                mb = __builtin_elementwise_max(mb, abs_bits2(vb[u]));
            }
        }
        for (; i < n; ++i) {
            ma = __builtin_elementwise_max(ma, abs_bits2(pa[i]));
            mb = __builtin_elementwise_max(mb, abs_bits2(pb[i]));
        }
    }
    mxa = max((uint32_t)ma.x, (uint32_t)ma.y);
    mxb = max((uint32_t)mb.x, (uint32_t)mb.y);
}

// Scale operand pair (s, s) in fp16 for the fp32 value f of a bf16 scale
// and the row's shift.
__device__ __forceinline__ h2 h16_scale(float f, int shift) {
    const _Float16 a = (_Float16)__builtin_ldexpf(f, shift);
    return (h2){a, a};
}

// 8 s4 codes (element 2k in the low nibble of byte k) -> 8 fp16 code*scale
// values, in the order k = 0,4,1,5,2,6,3,7 (the same for both operands, so
// the dot product only sums in another order).  One v_bitop3_b32 per pair
// (truth table 0x6A: b ? a ^ c : c, for src0 = a, src1 = b, src2 = c) keeps
// a nibble (b = its mask), flips its top bit (c = 1 there: two's complement
// -> code + 8 in [0, 15]) and sets the fp16 exponent bits of the constant
// (b = 0, c = 1).  A low nibble lands in mantissa bits 0-3 of 1024.0
// (0x6400, ulp 1): 1024 + code + 8.  A high nibble (bits 4-7) lands in
// mantissa bits 4-7 of 64.0 (0x5400, ulp 1/16, so bits 4-7 weigh 1..8):
// 64 + code + 8.  Subtracting 1032 or 72 leaves the code exactly, and the
// product with s is one exact fp16 rounding.
__device__ __forceinline__ uint32_t h16_nib(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x6a" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

__device__ __forceinline__ uint4 h16_codes(uint32_t w, h2 s) {
    const uint32_t w8 = w >> 8;
    const h2 b0 = {(_Float16)1032.0f, (_Float16)1032.0f};
    const h2 b1 = {(_Float16)72.0f, (_Float16)72.0f};
    const h2 p0 = __builtin_bit_cast(h2, h16_nib(w, 0x000F000Fu, 0x64086408u));
    const h2 p1 = __builtin_bit_cast(h2, h16_nib(w, 0x00F000F0u, 0x54805480u));
    const h2 p2 = __builtin_bit_cast(h2, h16_nib(w8, 0x000F000Fu, 0x64086408u));
    const h2 p3 = __builtin_bit_cast(h2, h16_nib(w8, 0x00F000F0u, 0x54805480u));
    uint4 r;
    r.x = __builtin_bit_cast(uint32_t, (h2)((p0 - b0) * s));
    r.y = __builtin_bit_cast(uint32_t, (h2)((p1 - b1) * s));
    r.z = __builtin_bit_cast(uint32_t, (h2)((p2 - b0) * s));
    r.w = __builtin_bit_cast(uint32_t, (h2)((p3 - b1) * s));
    return r;
}

// An MFMA operand fragment (one 32-row block and K16 slice) is 1 KiB in LDS
// and in the activation workspace: lane l's 16 bytes at 16 * l, read with one
// ds_read_b128 (on gfx950 the fastest LDS read form for contiguous data:
// ~169 B/clk per CU with 8 wavefronts reading, against ~152 for two
// ds_read_b64 and ~127 for ds_read2st64_b64, measured).
__device__ __forceinline__ h8 frag_read(const uint8_t* frag, int lane) {
    return *reinterpret_cast<const h8*>(frag + 16 * lane);
}
// Store lane L's 16-byte operand v into fragment frag (LDS or global).
__device__ __forceinline__ void frag_write(uint8_t* frag, int L, uint4 v) {
    *reinterpret_cast<uint4*>(frag + 16 * L) = v;
}

// One load batch of a thread: 4 groups of its activation row and weight
// column.  Scales: with VEC, sa[0..1] / sb[0..1] hold the 4 bf16 scales as
// two packed pairs (one 8-byte load per row); otherwise sa[i] / sb[i] hold
// group i's bf16 bits.
// Value of the partner lane's `other` (DPP quad permutation CTRL: 0xB1 =
// [1,0,3,2], lane ^ 1; 0x4E = [2,3,0,1], lane ^ 2) where take_other, else keep.
template <int CTRL>
__device__ __forceinline__ uint32_t h16_xchg(uint32_t keep, uint32_t other, bool take_other) {
    const uint32_t v = (uint32_t)__builtin_amdgcn_mov_dpp((int)other, CTRL, 0xf, 0xf, false);
    return take_other ? v : keep;
}

// fp32 value of scale i of a batch (bits are only re-read here, at the
// conversion, so the load's wait lands there too)
template <bool VEC>
__device__ __forceinline__ float h16_batch_scale(const uint32_t (&v)[kH16Batch], int i) {
    if constexpr (VEC) return __uint_as_float((i & 1) ? (v[i >> 1] & 0xffff0000u) : (v[i >> 1] << 16));
    return __uint_as_float(v[i] << 16);
}


}  // namespace
}  // namespace wush
