// wush_device.h -- device helpers shared by the gfx950 kernels.
//
// Numerics contract: every source file is compiled with -ffp-contract=off,
// fp32 denormals kept and correctly rounded '/' and sqrt, so each float
// expression below is one IEEE operation rounded to nearest even -- the
// arithmetic of the reference (my_int4/rtn_int4.py:22-55,
// csrc/quant_int4.cu:59-100).  Explicit __builtin_fmaf is used only where the
// fused and unfused forms are provably identical.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define WUSH_HOST_DEVICE __host__ __device__ __forceinline__

namespace wush {

constexpr int kGroup = 32;                       // quantization group along K
// my_int4/rtn_int4.py:19: C_CLIP = 0.35337862372398376 -> fp32 0x3EB4EE0B.
constexpr float kClip = 0.35337862372398376f;
// my_int4/rtn_int4.py:44: "+ 1e-8" -> fp32 0x322BCC77.
constexpr float kEps = 1e-8f;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 for non-NaN inputs (the scale is never
// NaN: a NaN variance selects 1.0).  Same result as torch's .to(bfloat16).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// The pointer as a wave-uniform (SGPR) global-memory pointer: p must be the
// same in every lane.  Loads and stores through it plus a 32-bit lane offset
// then use the scalar-base address form with no per-lane 64-bit arithmetic.
template <typename T>
using global_cptr = const __attribute__((address_space(1))) T*;
template <typename T>
using global_ptr = __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ global_cptr<T> uniform_ptr(const T* p) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return reinterpret_cast<global_cptr<T>>(((uint64_t)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ global_ptr<T> uniform_wptr(T* p) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return reinterpret_cast<global_ptr<T>>(((uint64_t)hi << 32) | lo);
}

// Group scale from the two sequential sums (rtn_int4.py:39-48):
// mean = s1/32, var = s2/32 - mean*mean, scale = sqrt(var)*C + 1e-8 if
// var >= 0 else 1.0; returns the bf16 bits, *sf gets the bf16 value.
__device__ __forceinline__ uint32_t group_scale(float s1, float s2, float* sf) {
    float mean = s1 * 0.03125f;                  // exact: power-of-two scaling
    float var = s2 * 0.03125f - mean * mean;
    float scale = 1.0f;
    if (var >= 0.0f) scale = __builtin_sqrtf(var) * kClip + kEps;
    uint32_t b = f32_to_bf16_rne(scale);
    *sf = bf16_to_f32(b);
    return b;
}

// INT4 code of v under bf16 scale sf: clamp(rint(v / sf), -7, 7), NaN -> 0
// (rtn_int4.py:50-51; quant_int4.cu:90-93).
__device__ __forceinline__ int code_of(float v, float sf) {
    float y = v / sf;
    float r = __builtin_rintf(y);
    r = __builtin_fminf(__builtin_fmaxf(r, -7.0f), 7.0f);
    return (y == y) ? (int)r : 0;
}

// RN(v / sf) without a division: r = RN(1/sf) once per group, then two fma
// corrections of q0 = RN(v*r).  q0 is within 1.5 ulps of v/sf and sf has 8
// significant bits, so each remainder v - q*sf is exactly representable and
// fma computes it exactly; q1 is then within an ulp of v/sf, and Markstein's
// theorem (r = RN(1/sf), q1 faithful, exact remainder) makes
// q2 = RN(q1 + e1*r) = RN(v/sf).  Requires finite v with |v| < 1.8e19 and a
// normal sf >= 1e-8 (no overflow); below 2^-100 a remainder may underflow,
// but such quotients are far below 0.5 and give code 0 either way.
// tests/native/quant_codes_fp32.c checks quotients and codes against the
// division at and next to every rounding tie and on random operands.
__device__ __forceinline__ float quotient_fma(float v, float sf, float r) {
    const float q0 = v * r;
    const float e0 = __builtin_fmaf(-q0, sf, v);
    const float q1 = __builtin_fmaf(e0, r, q0);
    const float e1 = __builtin_fmaf(-q1, sf, v);
    return __builtin_fmaf(e1, r, q1);
}

// code + 8 in [1, 15] as a float, from a quotient (rint, +8 exact, clamp).
__device__ __forceinline__ float code8_of_quotient(float q) {
    return __builtin_amdgcn_fmed3f(__builtin_rintf(q) + 8.0f, 1.0f, 15.0f);
}

// Code + 8 of v from t = RN(v*r + 8), one fma, with r = RN(1/sf); *far gets
// the larger of itself and |t - rint(t)|.  For finite |v| < 1.8e19 and a
// normal sf >= 1e-8, let q = v/sf (real).  If |q| <= 16, |t - (q + 8)| <= 2^-19
// (r is within 2^-24 relative of 1/sf and t is rounded once, with an ulp of at
// most 2^-19 below 32), and RN(q) is within 2^-21 of q.  So when
// |t - rint(t)| < 0.5 - 2^-17 -- t more than 2^-17 away from every
// half-integer -- q + 8 and RN(q) + 8 lie strictly inside the same unit
// interval around k = rint(t), and clamp(rint(RN(q)), -7, 7) + 8 ==
// clamp(k, 1, 15).  If |q| > 16 both sides clamp to the same end.  A lane
// whose |t - rint(t)| reaches the band redoes its group with quotient_fma
// (see quant_group32).  tests/native/quant_codes_fp32.c checks these codes
// against the division at and next to every rounding tie.
__device__ __forceinline__ float code8_fast(float v, float r, float* far) {
    const float t = __builtin_fmaf(v, r, 8.0f);
    const float k = __builtin_rintf(t);
    *far = __builtin_fmaxf(*far, __builtin_fabsf(t - k));
    return __builtin_amdgcn_fmed3f(k, 1.0f, 15.0f);
}

// |t - rint(t)| at or above this takes the exact quotient (code8_fast).
constexpr float kTieBand = 0.5f - 0x1p-17f;

// Quantize 32 fp32 values in registers: sequential sums, scale, 16 packed
// bytes as 4 dwords (element 2k low nibble of byte k).
// A group whose sum of squares is finite takes the one-fma codes of
// code8_fast, and a lane with a quotient near a rounding tie redoes its group
// with the correctly rounded division-free quotient; one with an inf or NaN
// element (s2 not finite) keeps code_of's division.
__device__ __forceinline__ uint32_t quant_group32(const float (&v)[32], uint32_t (&w)[4]) {
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        s1 = s1 + v[i];
        s2 = s2 + v[i] * v[i];
    }
    float sf;
    uint32_t sb = group_scale(s1, s2, &sf);
    if (!__builtin_isfinite(s2)) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t acc = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                acc |= (uint32_t)(code_of(v[d * 8 + e], sf) & 0xF) << (4 * e);
            w[d] = acc;
        }
        return sb;
    }
    const float r = 1.0f / sf;
    float far = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        // even elements 8d+2k -> byte k of a, odd ones -> byte k of b; the
        // bytes hold code + 8, an xor with 8 makes them two's complement nibbles
        uint32_t a = 0, b = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a = __builtin_amdgcn_cvt_pk_u8_f32(code8_fast(v[8 * d + 2 * k], r, &far), k, a);
            b = __builtin_amdgcn_cvt_pk_u8_f32(code8_fast(v[8 * d + 2 * k + 1], r, &far), k, b);
        }
        w[d] = (a ^ 0x08080808u) | ((b ^ 0x08080808u) << 4);
    }
    if (far >= kTieBand) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t a = 0, b = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                a = __builtin_amdgcn_cvt_pk_u8_f32(code8_of_quotient(quotient_fma(v[8 * d + 2 * k], sf, r)), k, a);
                b = __builtin_amdgcn_cvt_pk_u8_f32(code8_of_quotient(quotient_fma(v[8 * d + 2 * k + 1], sf, r)),
                                                   k, b);
            }
            w[d] = (a ^ 0x08080808u) | ((b ^ 0x08080808u) << 4);
        }
    }
    return sb;
}

// Sum over the 64 lanes of a wavefront on the VALU (DPP), result returned
// to every lane: quad_perm swaps and row mirrors reduce each 16-lane row,
// row_bcast:15 / row_bcast:31 fold rows 0-2 into row 3, lane 63 holds the
// total.  Lanes whose DPP source is masked add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add<0xB1, 0xf>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xf>(v);    // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);   // row_half_mirror
    v = dpp_add<0x140, 0xf>(v);   // row_mirror: every lane holds its row's sum
    v = dpp_add<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---------------------------------------------------------------------------
// Sum of V values (V a power of two, 1..64) over the 64 lanes of a wavefront
// by recursive halving.  At each step a lane keeps half of its values and adds
// its partner's copies of that half: partners across lane halves and 16-lane
// rows are exchanged with v_permlane32_swap / v_permlane16_swap, within a row
// with DPP (row_mirror, row_half_mirror, quad swaps).  Once one value is left,
// the remaining steps are plain pair sums.  V outputs cost about 2V + 3 log V
// VALU operations instead of ~8 per output with one full reduction each.
// Every lane returns the total of value wave_rs_index<V>(lane); the lanes with
// (lane & (64 / V - 1)) == 0 hold each index exactly once.
// Summation order differs from a sequential sum (fp32, tolerance-checked).
template <int D>
__device__ __forceinline__ float dpp_partner(float v) {
    constexpr int ctrl = D == 8 ? 0x140 : D == 4 ? 0x141 : D == 2 ? 0x4E : 0xB1;
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xf, 0xf, false));
}

// (a, b) -> the pair v_permlane{32,16}_swap leaves: a's lanes in the upper
// half (odd rows) exchanged with b's lanes in the lower half (even rows).
template <int D>
__device__ __forceinline__ float lanes_swap_sum(float a, float b) {
    if constexpr (D == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

template <int D, int H, int V>
__device__ __forceinline__ void rs_step(float (&v)[V], int lane) {
    if constexpr (H == 0) {                       // one value left: pair sum
        if constexpr (D >= 16) v[0] = lanes_swap_sum<D>(v[0], v[0]);
        else v[0] = v[0] + dpp_partner<D>(v[0]);
    } else {
#pragma unroll
        for (int i = 0; i < H; ++i) {
            if constexpr (D >= 16) {
                // lanes with bit D clear keep i, the others i + H
                v[i] = lanes_swap_sum<D>(v[i], v[i + H]);
            } else {
                const bool up = (lane & D) != 0;
                const float keep = up ? v[i + H] : v[i];
                const float send = up ? v[i] : v[i + H];
                v[i] = keep + dpp_partner<D>(send);
            }
        }
    }
}

template <int V>
__device__ __forceinline__ float wave_reduce_scatter(float (&v)[V], int lane) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V: power of two <= 64");
    rs_step<32, V / 2>(v, lane);
    rs_step<16, V / 4>(v, lane);
    rs_step<8, V / 8>(v, lane);
    rs_step<4, V / 16>(v, lane);
    rs_step<2, V / 32>(v, lane);
    rs_step<1, V / 64>(v, lane);
    return v[0];
}

template <int V>
__device__ __forceinline__ int wave_rs_index(int lane) {
    int idx = 0;
#pragma unroll
    for (int j = 0; (1 << (j + 1)) <= V; ++j)
        if (lane & (32 >> j)) idx += V >> (j + 1);
    return idx;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load with the non-temporal hint (weights are read once).
__device__ __forceinline__ uint4 load_nt16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Unpack 8 signed INT4 codes (one dword) into two dwords of int8 that hold
// 16*code: lo gets the even elements, hi the odd ones.  Exact: 16*[-8,7] fits
// int8.  Any fixed permutation of k is fine for a dot product as long as both
// operands use the same one.
__device__ __forceinline__ void unpack_s4x8_x16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    lo = (w << 4) & 0xF0F0F0F0u;
    hi = w & 0xF0F0F0F0u;
}

// LDS address (wave-uniform) of a __shared__ pointer
__device__ __forceinline__ uint32_t lds_addr(const void* l) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)l;
}
// LDS DMA: 16 (4) bytes per lane from g into LDS at lds + 16 (4) * lane.
// The compiler does not count these in its vmcnt waits: a caller waits for
// them itself (WUSH_WAIT_VMCNT) and keeps its own LDS reads of the target in
// order (sched_barrier, or the memory clobber of dma16_ordered).
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds) : "m0");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" : : "v"(g), "s"(lds) : "m0");
}
__device__ __forceinline__ void dma16_ordered(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds) : "m0", "memory");
}

// s_waitcnt vmcnt(n) (n < 64) with the other counters left alone, and a
// workgroup barrier after this wavefront's LDS operations (no wait on vector
// memory).  The LDS wait is a builtin, so that the compiler's own wait
// insertion knows every earlier LDS operation has completed (after an asm
// wait it still counts them outstanding and waits for later operations too).
#define WUSH_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define WUSH_LDS_BARRIER() do { __builtin_amdgcn_s_waitcnt(0xC07F); asm volatile("s_barrier" ::: "memory"); } while (0)

}  // namespace wush

// Common argument check used by the extern "C" entry points.
#define WUSH_REQUIRE(cond)                                   \
    do {                                                     \
        if (!(cond)) return (int)hipErrorInvalidValue;       \
    } while (0)
