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

// Codes of bf16 or fp16 inputs without a division per element.
// Write sf = ms * 2^es (ms < 256, sf is a normal bf16) and v = mv * 2^ev
// (|mv| < 2^11).  For a half-integer h, v/sf - h = (2v - 2h*sf) / (2 sf) and
// the numerator is a multiple of 2^min(ev+1, es); if it is not zero and
// |v/sf| is near h >= 0.5 (so 2^(ev-es) >= 0.5*128/2047), then
// |v/sf - h| >= 2^(ev-es)/255 > 2^-13.  With r = RN(1/sf) and y = RN(v*r),
// |y - v/sf| < 2^-20 for |v/sf| < 8.  Hence rint(y) == rint(RN(v/sf)) except
// when v/sf is exactly a half-integer, and then |y - h| < 2^-20: such y
// (within kHalfBand of a half-integer) are replaced by floor(y) + 0.5 = h
// and rounded half to even like the reference.  |y| >= 8 clamps like
// |v/sf| > 7.5; NaN and infinities give the codes of code_of.  Bit-identical
// to code_of for bf16 and fp16 inputs; fp32 inputs keep the division.
constexpr float kHalfBand = 0x1p-14f;
__device__ __forceinline__ int code_of_narrow(float v, float r) {
    const float y = v * r;
    const float f = __builtin_floorf(y);
    const float y2 = __builtin_fabsf(y - f - 0.5f) < kHalfBand ? f + 0.5f : y;
    float c = __builtin_rintf(y2);
    c = __builtin_fminf(__builtin_fmaxf(c, -7.0f), 7.0f);
    return (y == y) ? (int)c : 0;
}

__device__ __forceinline__ uint32_t quant_group32_narrow(const float (&v)[32], uint32_t (&w)[4]) {
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        s1 = s1 + v[i];
        s2 = s2 + v[i] * v[i];
    }
    float sf;
    const uint32_t sb = group_scale(s1, s2, &sf);
    const float r = 1.0f / sf;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t acc = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc |= (uint32_t)(code_of_narrow(v[d * 8 + e], r) & 0xF) << (4 * e);
        w[d] = acc;
    }
    return sb;
}

template <int DT>
__global__ __launch_bounds__(256) void quant_int4_kernel(const void* __restrict__ x,
                                                         uint8_t* __restrict__ q,
                                                         uint16_t* __restrict__ s,
                                                         int64_t n_groups) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    float v[32];
    InputTraits<DT>::load(x, g, v);
    uint32_t w[4];
    const uint32_t sb = DT == WUSH_DTYPE_F32 ? quant_group32(v, w) : quant_group32_narrow(v, w);
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
