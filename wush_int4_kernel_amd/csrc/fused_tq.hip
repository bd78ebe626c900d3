// fused_tq.hip -- WUSH block-diagonal transform fused with the INT4 group
// quantization, bit-exact with the reference's sequential form
// (csrc/fused_tq_int4.cu:27-85; tests/test_sw2.py:12-24):
//   x'_j = sum_{i=0..31} x_i * T[c][j][i]   (fp32, i ascending, mul then add)
//   then the quant_int4 chain on the fp32 x' (no bf16 rounding of x').
// Transformed activations never touch HBM.
//
// Two launch shapes, one numerics (the small-M per-pair steps live in
// fused_tq_device.h):
//  * rows kernel (rows >= 384): lane = row, wavefront = 64 rows of one block c.
//    T[c] is wave-uniform, so it is read with scalar loads into SGPRs and
//    every MAC takes an SGPR operand: no LDS and no cross-lane traffic in the
//    inner loop.  A product of two bf16 values is exact in fp32 unless an
//    operand is extreme (tiny, huge, inf or NaN), and then fma(x, T, acc)
//    equals the reference's acc + x*T bit for bit: when the wavefront's x and
//    the block's T are all in range (checked per launch, almost always) the
//    loop is 1024 v_fma_f32 per lane instead of 1024 v_mul + 1024 v_add.
//    4 wavefronts of a workgroup take 4 adjacent blocks of the same 64 rows,
//    so each row's 256 B of bf16 input is consumed by one workgroup.
//  * small-M kernel (rows < 384: decode, small batches): 32 lanes per (row, block), two
//    pairs per one-wavefront workgroup so a decode row spreads over K/64 CUs;
//    lane j
//    computes x'_j with T[c][j] read as 64 coalesced bytes and x broadcast
//    from LDS; the group sums are then re-run in i-order by every lane from
//    LDS (so they keep the sequential order) and lane pairs pack nibbles.
#include "fused_tq_device.h"
#include "../../include/wush_int4.h"

namespace wush {

constexpr int kRowsPerWave = 64;
constexpr int kBlocksPerWg = 4;

__global__ __launch_bounds__(256) void fused_tq_rows_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ t,
                                                            uint8_t* __restrict__ q,
                                                            uint16_t* __restrict__ s,
                                                            int64_t rows, int64_t K) {
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int64_t C = K >> 5;
    const int64_t c = (int64_t)blockIdx.x * kBlocksPerWg + wave;
    if (c >= C) return;
    const int64_t r = (int64_t)blockIdx.y * kRowsPerWave + lane;
    const bool active = r < rows;

    float xv[32];
    BfRange xr;
    if (active) {
        const uint4* p4 = reinterpret_cast<const uint4*>(x + r * K + c * 32);
        uint4 raw[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) raw[k] = p4[k];
        const uint32_t* u = reinterpret_cast<const uint32_t*>(raw);
#pragma unroll
        for (int d = 0; d < 16; ++d) {
            xv[2 * d] = bf16_to_f32(u[d] & 0xffffu);
            xv[2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
            xr.add(u[d]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) xv[i] = 0.0f;
    }

    // T[c][j][i] as bf16 pairs (i even in the low half), wave-uniform.
    const uint32_t* tc = reinterpret_cast<const uint32_t*>(t + c * 1024);
    // Each lane checks 16 of the block's 1024 entries.
    BfRange tr;
    {
        const uint4* t4 = reinterpret_cast<const uint4*>(tc) + lane * 2;
        const uint4 a = t4[0], b = t4[1];
        tr.add(a.x); tr.add(a.y); tr.add(a.z); tr.add(a.w);
        tr.add(b.x); tr.add(b.y); tr.add(b.z); tr.add(b.w);
    }
    // x_i * T[c][j][i] of two bf16 values is exact in fp32 when both lie in
    // the safe range, and then fma(x, T, acc) == acc + x*T bit for bit: one
    // fma per MAC instead of a mul and an add.  Otherwise the sequential
    // mul-then-add form, which also carries inf / NaN / underflow exactly.
    float xp[32];
    if (__all(xr.safe() & tr.safe())) {
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            float acc = 0.0f;
#pragma unroll
            for (int d = 0; d < 16; ++d) {
                const uint32_t pair = tc[j * 16 + d];
                acc = __builtin_fmaf(xv[2 * d], bf16_to_f32(pair & 0xffffu), acc);
                acc = __builtin_fmaf(xv[2 * d + 1], __uint_as_float(pair & 0xffff0000u), acc);
            }
            xp[j] = acc;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            float acc = 0.0f;
#pragma unroll
            for (int d = 0; d < 16; ++d) {
                const uint32_t pair = tc[j * 16 + d];
                acc = acc + xv[2 * d] * bf16_to_f32(pair & 0xffffu);
                acc = acc + xv[2 * d + 1] * __uint_as_float(pair & 0xffff0000u);
            }
            xp[j] = acc;
        }
    }

    uint32_t w[4];
    const uint32_t sb = quant_group32(xp, w);
    if (active) {
        reinterpret_cast<uint4*>(q + (r * C + c) * 16)[0] = make_uint4(w[0], w[1], w[2], w[3]);
        s[r * C + c] = (uint16_t)sb;
    }
}

constexpr int kPairsPerWg = 2;   // (row, block) pairs per one-wavefront workgroup

__global__ __launch_bounds__(64) void fused_tq_smallm_kernel(const uint16_t* __restrict__ x,
                                                              const uint16_t* __restrict__ t,
                                                              uint8_t* __restrict__ q,
                                                              uint16_t* __restrict__ s,
                                                              int64_t rows, int64_t K) {
    __shared__ float xs[kPairsPerWg][32];
    __shared__ float xps[kPairsPerWg][32];
    const int pl = threadIdx.x >> 5;             // pair within the workgroup
    const int j = threadIdx.x & 31;              // output index within the block
    const int64_t C = K >> 5;
    const int64_t p = (int64_t)blockIdx.x * kPairsPerWg + pl;
    const bool active = p < rows * C;

    uint4 tj[4];
    tq_pair_load(x, t, K, p, active, j, xs[pl], tj);
    __syncthreads();
    const float xj = tq_pair_matvec(xs[pl], tj);
    xps[pl][j] = xj;
    __syncthreads();
    tq_pair_quant(xps[pl], xj, j, active, p, q, s);
}

}  // namespace wush

// Rows below this use the small-M kernel (32 lanes per (row, block)); above
// it the rows kernel, whose 64-row wavefronts are latency-bound when few
// (K=8192, T cold: 64 rows 9.1 vs 23.6 us, 256 rows 19.9 vs 24.0 us, 512 rows
// 32.4 vs 25.3 us).
#ifndef WUSH_TQ_SMALLM_ROWS
#define WUSH_TQ_SMALLM_ROWS 384
#endif

extern "C" int wush_fused_tq(const uint16_t* x, const uint16_t* t, uint8_t* q, uint16_t* s,
                             int64_t rows, int64_t K, hipStream_t stream) {
    WUSH_REQUIRE(rows >= 0 && K > 0 && K % 32 == 0);
    if (rows == 0) return (int)hipSuccess;
    WUSH_REQUIRE(x && t && q && s);
    WUSH_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)t & 15u) == 0 &&
                 ((uintptr_t)q & 15u) == 0 && ((uintptr_t)s & 1u) == 0);
    const int64_t C = K / 32;
    if (rows < WUSH_TQ_SMALLM_ROWS) {
        const int64_t blocks = (rows * C + wush::kPairsPerWg - 1) / wush::kPairsPerWg;
        WUSH_REQUIRE(blocks <= 0x7fffffffLL);
        wush::fused_tq_smallm_kernel<<<(unsigned)blocks, 64, 0, stream>>>(x, t, q, s, rows, K);
    } else {
        const int64_t gx = (C + wush::kBlocksPerWg - 1) / wush::kBlocksPerWg;
        const int64_t gy = (rows + wush::kRowsPerWave - 1) / wush::kRowsPerWave;
        WUSH_REQUIRE(gx <= 0x7fffffffLL && gy <= 65535);
        wush::fused_tq_rows_kernel<<<dim3((unsigned)gx, (unsigned)gy), 256, 0, stream>>>(x, t, q, s,
                                                                                         rows, K);
    }
    return (int)hipGetLastError();
}
