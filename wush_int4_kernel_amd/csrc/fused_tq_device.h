// fused_tq_device.h -- one (row, block) pair of the WUSH transform fused with
// the INT4 group quantization, handled by 32 lanes (csrc/fused_tq_int4.cu:27-85;
// tests/test_sw2.py:12-24 fix the arithmetic):
//   x'_j = sum_{i=0..31} x_i * T[c][j][i]   (fp32, i ascending, mul then add)
//   then the quant_int4 chain on the fp32 x' (no bf16 rounding of x').
// Lane j computes x'_j from T[c][j] (64 coalesced bytes) and x broadcast from
// LDS; the group sums are re-run in i-order by every lane from LDS so they
// keep the sequential order, and lane pairs pack the nibbles.  These are the
// steps of the small-M fused_tq kernel.
#pragma once
#include "wush_device.h"

namespace wush {

// Range check for exact bf16 x bf16 products, on packed pairs of bf16 bits.
// A value is "safe" when it is zero or its magnitude bits m = bits & 0x7fff
// lie in [0x1e00, 0x58ff], i.e. |v| in [2^-67, 2^51).  The product of two
// safe values has at most 16 significant bits, its lowest bit is at least
// 2^-148 and it is below 2^102, so it is exact in fp32 (no rounding,
// underflow or overflow), and a sum of 32 of them stays finite.
// BfRange accumulates, two values per 32-bit word, the largest m and the
// smallest m - 1 (16-bit wrap-around sends zeros to 0xffff, out of the way)
// with packed 16-bit integer min / max.
struct BfRange {
    uint32_t mx = 0u, mn = 0xffffffffu;
    __device__ __forceinline__ void add(uint32_t w) {
        typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
        const u16x2 m = __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
        const u16x2 m1 = m - (u16x2){1, 1};
        mx = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, mx), m));
        mn = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, mn), m1));
    }
    // every nonzero magnitude at least the bf16 magnitude bits lo (and below
    // 2^51)
    __device__ __forceinline__ bool safe_from(uint32_t lo) const {
        const uint32_t mx_lo = mx & 0xffffu, mx_hi = mx >> 16;
        const uint32_t mn_lo = mn & 0xffffu, mn_hi = mn >> 16;
        return (mx_lo <= 0x58ffu) & (mx_hi <= 0x58ffu) & (mn_lo >= lo - 1) & (mn_hi >= lo - 1);
    }
    __device__ __forceinline__ bool safe() const { return safe_from(0x1e00u); }
};

__device__ __forceinline__ void load_bf16x32(const uint16_t* p, float (&v)[32]) {
    const uint4* p4 = reinterpret_cast<const uint4*>(p);
    uint4 r[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) r[c] = p4[c];
    const uint32_t* u = reinterpret_cast<const uint32_t*>(r);
#pragma unroll
    for (int d = 0; d < 16; ++d) {
        v[2 * d] = bf16_to_f32(u[d] & 0xffffu);
        v[2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
    }
}

// Step 1: lane j stages x_j of pair (row r, block c) in LDS (xs_l, 32
// floats) and loads row j of T[c] as raw bf16 pairs (element 2d in the low
// half of word d); returns x_j.  A barrier must follow before step 2.
__device__ __forceinline__ float tq_pair_load(const uint16_t* __restrict__ x, const uint16_t* __restrict__ t,
                                              int64_t K, int64_t r, int64_t c, bool active, int j, float* xs_l,
                                              uint4 (&tj)[4]) {
    if (!active) r = c = 0;
    const float xj = active ? bf16_to_f32(x[r * K + c * 32 + j]) : 0.0f;
    xs_l[j] = xj;
    const uint4* row = reinterpret_cast<const uint4*>(t + c * 1024 + j * 32);
#pragma unroll
    for (int k = 0; k < 4; ++k) tj[k] = active ? row[k] : make_uint4(0, 0, 0, 0);
    return xj;
}

// Step 2: x'_j (T converted to fp32 as it is used).  The caller stores it
// to LDS (xps_l[j]) and syncs.  FAST (every x and T value of the wavefront
// in BfRange's safe range, so each product is exact): one fma per MAC, bit
// for bit the reference's acc + x*T; otherwise mul then add.
template <bool FAST>
__device__ __forceinline__ float tq_pair_matvec(const float* xs_l, const uint4 (&tj)[4]) {
    const uint32_t* u = &tj[0].x;
    float acc = 0.0f;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
        const float t0 = bf16_to_f32(u[d] & 0xffffu), t1 = __uint_as_float(u[d] & 0xffff0000u);
        if constexpr (FAST) {
            acc = __builtin_fmaf(xs_l[2 * d], t0, acc);
            acc = __builtin_fmaf(xs_l[2 * d + 1], t1, acc);
        } else {
            acc = acc + xs_l[2 * d] * t0;
            acc = acc + xs_l[2 * d + 1] * t1;
        }
    }
    return acc;
}

// Whether this lane's T row and staged x_j lie in BfRange's safe range.
__device__ __forceinline__ bool tq_pair_safe(const uint4 (&tj)[4], float xj) {
    BfRange rg;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        rg.add(tj[k].x); rg.add(tj[k].y); rg.add(tj[k].z); rg.add(tj[k].w);
    }
    rg.add(__float_as_uint(xj) >> 16);        // bf16 bits in the low half; the zero high half is ignored
    return rg.safe();
}

// Step 3: the group's sums in i-order, its scale, lane j's code; even lanes
// store one byte (element j low nibble, j+1 high), lane 0 the scale.  The 32
// lanes of a pair must be one half of a wavefront.
__device__ __forceinline__ void tq_pair_quant(const float* xps_l, float xj, int j, bool active, int64_t p,
                                              uint8_t* q, uint16_t* s) {
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float v = xps_l[i];
        s1 = s1 + v;
        s2 = s2 + v * v;
    }
    float sf;
    const uint32_t sb = group_scale(s1, s2, &sf);
    const int code = code_of(xj, sf) & 0xF;
    const int partner = __shfl_xor(code, 1, 32);
    if (active) {
        if ((j & 1) == 0) q[p * 16 + (j >> 1)] = (uint8_t)(code | (partner << 4));
        if (j == 0) s[p] = (uint16_t)sb;
    }
}

}  // namespace wush
