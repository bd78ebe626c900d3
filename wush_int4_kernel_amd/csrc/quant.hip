// quant.hip -- group-wise sigma-clip INT4 quantization (bit-exact) and the
// per-tensor INT4 quantization, with their C-ABI entry points.
//
// quant_int4: one lane owns one 32-element group.  The reference defines the
// group's sums as a sequential i = 0..31 chain (my_int4/rtn_int4.py:22-30,
// csrc/quant_int4.cu:66-70), so a group cannot be split across lanes without
// changing bits; lane-per-group keeps that chain in one lane and lets a
// wavefront cover 64 consecutive groups (4 KiB of bf16 input, 1 KiB of codes,
// 128 B of scales) per instruction group.  The op is HBM-bound:
// 2.5625 B per bf16 element moved.
#include "wush_device.h"
#include "../../include/wush_int4.h"

namespace wush {

template <int DT>
struct InputTraits;

template <>
struct InputTraits<WUSH_DTYPE_BF16> {
    static constexpr int kBytes = 64;            // 32 x 2 B
    __device__ static void load(const void* base, int64_t g, float (&v)[32]) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + g * 32);
        uint4 r[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) r[c] = p[c];
        const uint32_t* u = reinterpret_cast<const uint32_t*>(r);
#pragma unroll
        for (int d = 0; d < 16; ++d) {
            v[2 * d] = bf16_to_f32(u[d] & 0xffffu);
            v[2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
        }
    }
};

template <>
struct InputTraits<WUSH_DTYPE_F16> {
    __device__ static void load(const void* base, int64_t g, float (&v)[32]) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + g * 32);
        uint4 r[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) r[c] = p[c];
        const uint32_t* u = reinterpret_cast<const uint32_t*>(r);
#pragma unroll
        for (int d = 0; d < 16; ++d) {
            v[2 * d] = f16_to_f32(u[d] & 0xffffu);
            v[2 * d + 1] = f16_to_f32(u[d] >> 16);
        }
    }
};

template <>
struct InputTraits<WUSH_DTYPE_F32> {
    __device__ static void load(const void* base, int64_t g, float (&v)[32]) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(base) + g * 32);
        uint4 r[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) r[c] = p[c];
        const uint32_t* u = reinterpret_cast<const uint32_t*>(r);
#pragma unroll
        for (int d = 0; d < 32; ++d) v[d] = __uint_as_float(u[d]);
    }
};

// Codes of a finite bf16 or fp16 group without a division per element:
// clamp(rint(RN(v/sf)), -7, 7) from one reciprocal r = RN(1/sf) per group and
// an fma correction per element.
//  * y = RN(v*r) is within 2^-22 |v/sf| of the quotient.  v has at most 11
//    significant bits and sf at most 8, so the remainder e = v - y*sf is a
//    multiple of ulp(y)*ulp(sf) of about 9 bits: exactly representable, and
//    fma computes it exactly.  y1 = RN(y + e*r) is the quotient up to 2^-46
//    relative.
//  * Write sf = ms*2^es (ms < 2^8) and v = mv*2^ev (|mv| < 2^11).  For a
//    half-integer h, v/sf - h = (2v - 2h*sf) / (2sf) with a numerator that is
//    a multiple of 2^min(ev+1, es); if it is not zero and v/sf is near
//    h >= 0.5, |v/sf - h| >= 2^(ev-es)/255 > 2^-13.  So a quotient that is not
//    a half-integer is far from every rounding tie and rint(y1) equals
//    rint(RN(v/sf)); an exact half-integer quotient h comes out as y1 = h
//    exactly (the perturbation is far below half an ulp of h).
//  * Codes are formed as c + 8 in [1, 15]: adding 8 keeps the parity that
//    round-half-even needs, and y1 + 8 cannot cross a half-integer.  They are
//    converted straight into bytes with v_cvt_pk_u8_f32 and turned into two's
//    complement nibbles by an xor with 8.
// About 8 VALU operations per element, against about 15 with a tie band
// around RN(v*r) and more with a division.  Checked against the division for
// every finite bf16 and fp16 v (|v| < 1.8e19, i.e. s2 finite) and every bf16
// sf >= 1e-8 (tests/test_quant_codes_exhaustive.py).  Groups with a non-finite
// element (s2 not finite) take code_of, whose division handles inf and NaN.
__device__ __forceinline__ float code_plus8(float v, float sf, float r) {
    const float y = v * r;
    const float e = __builtin_fmaf(-y, sf, v);
    const float y1 = __builtin_fmaf(e, r, y);
    return __builtin_amdgcn_fmed3f(__builtin_rintf(y1 + 8.0f), 1.0f, 15.0f);
}

__device__ __forceinline__ uint32_t quant_group32_fma(const float (&v)[32], uint32_t (&w)[4]) {
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        s1 = s1 + v[i];
        s2 = s2 + v[i] * v[i];
    }
    float sf;
    const uint32_t sb = group_scale(s1, s2, &sf);
    if (!__builtin_isfinite(s2)) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t acc = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc |= (uint32_t)(code_of(v[d * 8 + e], sf) & 0xF) << (4 * e);
            w[d] = acc;
        }
        return sb;
    }
    const float r = 1.0f / sf;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        // even elements 8d+2k -> byte k of a, odd elements 8d+2k+1 -> byte k of b
        uint32_t a = 0, b = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a = __builtin_amdgcn_cvt_pk_u8_f32(code_plus8(v[8 * d + 2 * k], sf, r), k, a);
            b = __builtin_amdgcn_cvt_pk_u8_f32(code_plus8(v[8 * d + 2 * k + 1], sf, r), k, b);
        }
        w[d] = (a ^ 0x08080808u) | ((b ^ 0x08080808u) << 4);
    }
    return sb;
}

// 2-byte inputs: the wavefront's 64 groups (4 KiB) are read with four
// load instructions of 1 KiB contiguous each, then redistributed so that
// lane l holds group l.  Instruction c gives lane l the 16 bytes at
// c*1024 + 16*sig(l), sig(l) = 4*(l%16) + l/16: quarter l/16 of group
// 16c + l%16.  A 4x4 transpose between register index c and lane bits 5..4
// (v_permlane32_swap on register pairs (c, c+2), then v_permlane16_swap on
// (c, c+1)) leaves quarter p of group l in register p of lane l.  All lanes
// take part; lanes past the last group load zeros and store nothing.
__device__ __forceinline__ void swap_regs32(uint4& a, uint4& b) {
    auto x = __builtin_amdgcn_permlane32_swap(a.x, b.x, false, false);
    auto y = __builtin_amdgcn_permlane32_swap(a.y, b.y, false, false);
    auto z = __builtin_amdgcn_permlane32_swap(a.z, b.z, false, false);
    auto w = __builtin_amdgcn_permlane32_swap(a.w, b.w, false, false);
    a = make_uint4(x[0], y[0], z[0], w[0]);
    b = make_uint4(x[1], y[1], z[1], w[1]);
}
__device__ __forceinline__ void swap_regs16(uint4& a, uint4& b) {
    auto x = __builtin_amdgcn_permlane16_swap(a.x, b.x, false, false);
    auto y = __builtin_amdgcn_permlane16_swap(a.y, b.y, false, false);
    auto z = __builtin_amdgcn_permlane16_swap(a.z, b.z, false, false);
    auto w = __builtin_amdgcn_permlane16_swap(a.w, b.w, false, false);
    a = make_uint4(x[0], y[0], z[0], w[0]);
    b = make_uint4(x[1], y[1], z[1], w[1]);
}

template <int DT>
__device__ __forceinline__ void load_group_coalesced(const void* x, int64_t g, int64_t n_groups, float (&v)[32]) {
    const int lane = threadIdx.x & 63;
    const int64_t g0 = g - lane;                     // first group of the wavefront
    const int sig = 4 * (lane & 15) + (lane >> 4);
    const uint16_t* base = static_cast<const uint16_t*>(x);
    uint4 r[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int64_t gi = g0 + 16 * c + (sig >> 2);
        r[c] = gi < n_groups ? load_nt16(base + gi * 32 + (sig & 3) * 8) : make_uint4(0, 0, 0, 0);
    }
    swap_regs32(r[0], r[2]);
    swap_regs32(r[1], r[3]);
    swap_regs16(r[0], r[1]);
    swap_regs16(r[2], r[3]);
    const uint32_t* u = reinterpret_cast<const uint32_t*>(r);
#pragma unroll
    for (int d = 0; d < 16; ++d) {
        if constexpr (DT == WUSH_DTYPE_BF16) {
            v[2 * d] = bf16_to_f32(u[d] & 0xffffu);
            v[2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
        } else {
            v[2 * d] = f16_to_f32(u[d] & 0xffffu);
            v[2 * d + 1] = f16_to_f32(u[d] >> 16);
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void quant_int4_kernel(const void* __restrict__ x,
                                                         uint8_t* __restrict__ q,
                                                         uint16_t* __restrict__ s,
                                                         int64_t n_groups) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    float v[32];
    if constexpr (DT == WUSH_DTYPE_F32) {
        if (g >= n_groups) return;
        InputTraits<DT>::load(x, g, v);
    } else {
        load_group_coalesced<DT>(x, g, n_groups, v);   // whole wavefront, before any exit
        if (g >= n_groups) return;
    }
    uint32_t w[4];
    const uint32_t sb = DT == WUSH_DTYPE_F32 ? quant_group32(v, w) : quant_group32_fma(v, w);
    reinterpret_cast<uint4*>(q)[g] = make_uint4(w[0], w[1], w[2], w[3]);
    s[g] = (uint16_t)sb;
}

// Per-tensor quantization (csrc/fast_path.cu:17-39): code =
// clamp(rint(x * inv_scale), -7, 7) with one fp32 multiply; NaN -> 0.
__device__ __forceinline__ int code_mul(float v, float inv) {
    float y = v * inv;
    float r = __builtin_rintf(y);
    r = __builtin_fminf(__builtin_fmaxf(r, -7.0f), 7.0f);
    return (y == y) ? (int)r : 0;
}

__global__ __launch_bounds__(256) void quant_tensor_scale_kernel(const uint16_t* __restrict__ x,
                                                                 uint8_t* __restrict__ q,
                                                                 int64_t n32, float inv_host,
                                                                 const float* __restrict__ inv_dev) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n32) return;
    const float inv = inv_dev ? *inv_dev : inv_host;
    const uint4* p = reinterpret_cast<const uint4*>(x + g * 32);
    uint4 r[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) r[c] = p[c];
    const uint32_t* u = reinterpret_cast<const uint32_t*>(r);
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t acc = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t pair = u[d * 4 + e];
            const int c0 = code_mul(bf16_to_f32(pair & 0xffffu), inv);
            const int c1 = code_mul(__uint_as_float(pair & 0xffff0000u), inv);
            acc |= (uint32_t)((c0 & 0xF) | ((c1 & 0xF) << 4)) << (8 * e);
        }
        w[d] = acc;
    }
    reinterpret_cast<uint4*>(q)[g] = make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace wush

extern "C" {

int wush_abi_version(void) { return WUSH_INT4_ABI_VERSION; }

const char* wush_error_string(int status) {
    if (status == (int)hipErrorInvalidValue) return "wush_int4: invalid argument";
    if (status == WUSH_ERROR_SCRATCH_TOO_SMALL)
        return "wush_int4: the shape's split-K plan needs more than WUSH_GEMM_SCRATCH_BYTES of scratch "
               "(call wush_gemm_s4 with a workspace instead)";
    return hipGetErrorString((hipError_t)status);
}

int wush_quant_int4(const void* x, int dtype, uint8_t* q, uint16_t* s, int64_t n_groups,
                    hipStream_t stream) {
    WUSH_REQUIRE(n_groups >= 0);
    if (n_groups == 0) return (int)hipSuccess;
    WUSH_REQUIRE(x && q && s);
    WUSH_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)q & 15u) == 0 && ((uintptr_t)s & 1u) == 0);
    const int threads = 256;
    const int64_t blocks = (n_groups + threads - 1) / threads;
    WUSH_REQUIRE(blocks <= 0x7fffffffLL);
    switch (dtype) {
        case WUSH_DTYPE_BF16:
            wush::quant_int4_kernel<WUSH_DTYPE_BF16><<<(unsigned)blocks, threads, 0, stream>>>(x, q, s, n_groups);
            break;
        case WUSH_DTYPE_F16:
            wush::quant_int4_kernel<WUSH_DTYPE_F16><<<(unsigned)blocks, threads, 0, stream>>>(x, q, s, n_groups);
            break;
        case WUSH_DTYPE_F32:
            wush::quant_int4_kernel<WUSH_DTYPE_F32><<<(unsigned)blocks, threads, 0, stream>>>(x, q, s, n_groups);
            break;
        default:
            return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

int wush_quant_int4_tensor_scale(const uint16_t* x, uint8_t* q, int64_t n, float inv_scale,
                                 const float* inv_scale_dev, hipStream_t stream) {
    WUSH_REQUIRE(n >= 0 && n % 32 == 0);
    if (n == 0) return (int)hipSuccess;
    WUSH_REQUIRE(x && q);
    WUSH_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)q & 15u) == 0);
    const int64_t n32 = n / 32;
    const int threads = 256;
    const int64_t blocks = (n32 + threads - 1) / threads;
    WUSH_REQUIRE(blocks <= 0x7fffffffLL);
    wush::quant_tensor_scale_kernel<<<(unsigned)blocks, threads, 0, stream>>>(x, q, n32, inv_scale,
                                                                             inv_scale_dev);
    return (int)hipGetLastError();
}

}  // extern "C"
