// fused_tq.hip -- WUSH block-diagonal transform fused with the INT4 group
// quantization, bit-exact with the reference's sequential form
// (csrc/fused_tq_int4.cu:27-85; tests/test_sw2.py:12-24):
//   x'_j = sum_{i=0..31} x_i * T[c][j][i]   (fp32, i ascending, mul then add)
//   then the quant_int4 chain on the fp32 x' (no bf16 rounding of x').
// Transformed activations never touch HBM.
//
// Three launch shapes, one numerics (the small-M per-pair steps live in
// fused_tq_device.h):
//  * rows kernel: lane = row, wavefront = 64 rows of one block c, 4
//    wavefronts of a workgroup on 4 adjacent blocks of the same 64 rows (each
//    row's 256 B of bf16 input is consumed by one workgroup).  T[c] is
//    wave-uniform.  A product of two bf16 values is exact in fp32 unless an
//    operand is extreme (tiny, huge, inf or NaN), and then fma(x, T, acc)
//    equals the reference's acc + x*T bit for bit: when the wavefront's x and
//    the block's T are all in range (checked per launch, almost always) the
//    transform is 1024 fmas per lane instead of 1024 muls + 1024 adds.  T
//    reaches the MACs in one of two ways:
//     - SGPR form (launches of 1536 wavefronts or more): scalar loads into
//       SGPRs, converted to fp32 on the SALU, every MAC takes an SGPR operand;
//     - DPP form (fewer wavefronts, where the scalar loads' latency is not
//       hidden): vector loads, 16 pairs per VGPR converted on the VALU, every
//       MAC reads its T value from another lane through DPP row_newbcast.
//  * small-M kernel (at most 16384 (row, block) pairs: decode, small batches):
//    32 lanes per (row, block), two adjacent blocks of one row per
//    one-wavefront workgroup (grid: block pairs x rows) so a decode row
//    spreads over K/64 CUs; lane j computes x'_j with T[c][j] read
//    as 64 coalesced bytes and x broadcast from LDS (one fma per MAC when the
//    wavefront's x and T are in range, as above); the group sums are then
//    re-run in i-order by every lane from LDS (so they keep the sequential
//    order) and lane pairs pack nibbles.
#include <type_traits>

#include "fused_tq_device.h"
#include "../../include/wush_int4.h"

namespace wush {

constexpr int kRowsPerWave = 64;
constexpr int kBlocksPerWg = 4;

// T[c] row j (32 bf16 as 16 pairs) -> fp32 in SGPRs.
__device__ __forceinline__ void t_row_f32(const uint32_t (&raw)[16], float (&tf)[32]) {
#pragma unroll
    for (int d = 0; d < 16; ++d) {
        tf[2 * d] = bf16_to_f32(raw[d] & 0xffffu);
        tf[2 * d + 1] = __uint_as_float(raw[d] & 0xffff0000u);
    }
}

__device__ __forceinline__ void t_row_load(const uint32_t* __restrict__ row, uint32_t (&raw)[16]) {
    const uint4* r4 = reinterpret_cast<const uint4*>(row);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 v = r4[k];
        raw[4 * k] = v.x; raw[4 * k + 1] = v.y; raw[4 * k + 2] = v.z; raw[4 * k + 3] = v.w;
    }
}

// x'_j for j = 0..31 from x (fp32, 32 per lane) and the wave-uniform T[c].
// Row j of T is converted to fp32 (SALU) before row j + 1 is requested, so
// the wait for row j never waits for the prefetch (scalar loads return out of
// order, a wait covers every load in flight); row j + 1 then arrives while
// row j's 32 MACs run.  FAST: one fma per MAC (exact products), else the
// reference's mul then add.
template <bool FAST>
__device__ __forceinline__ void transform_block(const float (&xv)[32], const uint32_t* __restrict__ tc,
                                                float (&xp)[32]) {
    uint32_t raw[16];
    t_row_load(tc, raw);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        float tf[32];
        t_row_f32(raw, tf);
        __builtin_amdgcn_sched_barrier(0);
        if (j + 1 < 32) t_row_load(tc + (j + 1) * 16, raw);
        __builtin_amdgcn_sched_barrier(0);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            if constexpr (FAST) acc = __builtin_fmaf(xv[i], tf[i], acc);
            else acc = acc + xv[i] * tf[i];
        }
        xp[j] = acc;
    }
}

template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

// acc = acc + t' * x, where t' is t read from lane 16 * (lane / 16) + M
// (DPP row_newbcast: lane M of each 16-lane row, broadcast to the row).
// FAST: one v_fmac_f32_dpp, valid when t' * x is exact.  Otherwise
// v_mul_f32_dpp then v_add_f32: the product and the sum rounded separately.
template <int M, bool FAST>
__device__ __forceinline__ void mac_bcast(float& acc, float t, float x) {
    if constexpr (FAST) {
        asm volatile("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
                     : "+v"(acc)
                     : "v"(t), "v"(x), "n"(M));
    } else {
        float sum;
        asm volatile("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf\n\t"
                     "v_add_f32_e32 %0, %4, %0"
                     : "=&v"(sum)
                     : "v"(t), "v"(x), "n"(M), "v"(acc));
        acc = sum;
    }
}

// Four bf16 pairs -> their eight fp32 values (low halves, high halves).  The
// trailing s_nop gives the two wait states a DPP read of a VGPR needs after a
// VALU write of it.
__device__ __forceinline__ void pairs_to_f32(const uint4& w, float (&lo)[4], float (&hi)[4]) {
    asm volatile(
        "v_lshlrev_b32_e32 %0, 16, %8\n\t"
        "v_lshlrev_b32_e32 %1, 16, %9\n\t"
        "v_lshlrev_b32_e32 %2, 16, %10\n\t"
        "v_lshlrev_b32_e32 %3, 16, %11\n\t"
        "v_and_b32_e32 %4, 0xffff0000, %8\n\t"
        "v_and_b32_e32 %5, 0xffff0000, %9\n\t"
        "v_and_b32_e32 %6, 0xffff0000, %10\n\t"
        "v_and_b32_e32 %7, 0xffff0000, %11\n\t"
        "s_nop 1"
        : "=&v"(lo[0]), "=&v"(lo[1]), "=&v"(lo[2]), "=&v"(lo[3]),
          "=&v"(hi[0]), "=&v"(hi[1]), "=&v"(hi[2]), "=&v"(hi[3])
        : "v"(w.x), "v"(w.y), "v"(w.z), "v"(w.w));
}

// x'_j = sum_i x_i * T[c][j][i] for j = 0..31, i ascending, lane = row.
// T[c] is read with vector loads in groups of 4 rows: lane m of every 16-lane
// row loads row 4g + m/4, pairs 4(m%4)..4(m%4)+3 (16 bytes), so register k of
// lane 4a + b holds pair 4b + k of row 4g + a, and row_newbcast:(4a + b)
// hands that pair to every lane.  The 4 rows of a group are 4 interleaved
// accumulation chains.  Loads run two groups ahead.
template <bool FAST>
__device__ __forceinline__ void transform_block_dpp(const float (&xv)[32], const uint4* __restrict__ tq4, int lane,
                                                float (&xp)[32]) {
    const uint4* src = tq4 + ((lane & 15) >> 2) * 4 + (lane & 3);
#pragma unroll
    for (int j = 0; j < 32; ++j) xp[j] = 0.0f;
    uint4 raw_next = src[16];
    float lo[2][4], hi[2][4];
    pairs_to_f32(src[0], lo[0], hi[0]);
    static_for<8>([&](auto gc) {
        constexpr int g = decltype(gc)::value;
        uint4 raw_after;
        if constexpr (g + 2 < 8) raw_after = src[(g + 2) * 16];
        if constexpr (g + 1 < 8) pairs_to_f32(raw_next, lo[(g + 1) & 1], hi[(g + 1) & 1]);
        static_for<16>([&](auto pc) {
            constexpr int p = decltype(pc)::value, b = p / 4, k = p % 4;
            static_for<4>([&](auto ac) {
                constexpr int a = decltype(ac)::value;
                mac_bcast<4 * a + b, FAST>(xp[4 * g + a], lo[g & 1][k], xv[2 * p]);
            });
            static_for<4>([&](auto ac) {
                constexpr int a = decltype(ac)::value;
                mac_bcast<4 * a + b, FAST>(xp[4 * g + a], hi[g & 1][k], xv[2 * p + 1]);
            });
        });
        if constexpr (g + 2 < 8) raw_next = raw_after;
    });
}

// One wavefront: 64 rows (r0 + lane) of block c; 4 wavefronts of a workgroup
// take 4 adjacent blocks.  DPP picks transform_block_dpp, else the SGPR form.
template <bool DPP>
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
    const int64_t r0 = (int64_t)blockIdx.y * kRowsPerWave;
    const int64_t r = r0 + lane;
    const bool active = r < rows;

    // T[c][j][i] as bf16 pairs (i even in the low half), wave-uniform.  Each
    // lane range-checks 16 of the block's 1024 entries; these loads go first
    // so that the check waits for them alone.
    const uint32_t* tc = reinterpret_cast<const uint32_t*>(t + c * 1024);
    const uint4* t4 = reinterpret_cast<const uint4*>(tc) + lane * 2;
    const uint4 ta = t4[0], tb = t4[1];
    // Lanes past the last row read row r0 (their results are not stored).
    const uint4* p4 = reinterpret_cast<const uint4*>(x + (active ? r : r0) * K + c * 32);
    uint4 raw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) raw[k] = p4[k];
    BfRange tr;
    tr.add(ta.x); tr.add(ta.y); tr.add(ta.z); tr.add(ta.w);
    tr.add(tb.x); tr.add(tb.y); tr.add(tb.z); tr.add(tb.w);

    float xv[32];
    BfRange xr;
    const uint32_t* u = &raw[0].x;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
        xv[2 * d] = bf16_to_f32(u[d] & 0xffffu);
        xv[2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
        xr.add(u[d]);
    }
    // x_i * T[c][j][i] of two bf16 values is exact in fp32 when both lie in
    // the safe range, and then fma(x, T, acc) == acc + x*T bit for bit: one
    // fma per MAC instead of a mul and an add.  Otherwise the sequential
    // mul-then-add form, which also carries inf / NaN / underflow exactly.
    float xp[32];
    const bool fast = __all(xr.safe() & tr.safe());
    if constexpr (DPP) {
        const uint4* tq4 = reinterpret_cast<const uint4*>(tc);
        if (fast) transform_block_dpp<true>(xv, tq4, lane, xp);
        else transform_block_dpp<false>(xv, tq4, lane, xp);
    } else {
        if (fast) transform_block<true>(xv, tc, xp);
        else transform_block<false>(xv, tc, xp);
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
    __shared__ __align__(16) float xs[kPairsPerWg][32];
    __shared__ __align__(16) float xps[kPairsPerWg][32];
    const int pl = threadIdx.x >> 5;             // pair within the workgroup
    const int j = threadIdx.x & 31;              // output index within the block
    // grid (ceil(C / 2), rows): the two pairs of a workgroup are blocks c,
    // c + 1 of one row (no division for the pair's row and block)
    const int64_t C = K >> 5;
    const int64_t r = blockIdx.y;
    const int64_t c = (int64_t)blockIdx.x * kPairsPerWg + pl;
    const bool active = c < C;
    const int64_t p = r * C + c;

    uint4 tj[4];
    const float x_own = tq_pair_load(x, t, K, r, c, active, j, xs[pl], tj);
    const bool fast = __all(tq_pair_safe(tj, x_own));
    __syncthreads();
    const float xj = fast ? tq_pair_matvec<true>(xs[pl], tj) : tq_pair_matvec<false>(xs[pl], tj);
    xps[pl][j] = xj;
    __syncthreads();
    tq_pair_quant(xps[pl], xj, j, active, p, q, s);
}

}  // namespace wush

// Launches of at most this many (row, block) pairs use the small-M kernel,
// whose time grows with the pairs from a lower floor than the rows kernel's
// (K=4096: 64 rows 4.1 vs 6.0 us, 128 rows 5.7 vs 5.9 us, 256 rows 9.0 vs 6.2 us).
#ifndef WUSH_TQ_SMALLM_PAIRS
#define WUSH_TQ_SMALLM_PAIRS 16384
#endif
// Rows-kernel launches with fewer wavefronts than this take the DPP form
// (K=4096: 512 rows 6.4 vs 8.5 us; 768 rows 9.2 vs 9.1 us; 2048 rows 16.2 vs
// 14.2 us for DPP vs SGPR).
#ifndef WUSH_TQ_DPP_WAVES
#define WUSH_TQ_DPP_WAVES 1536
#endif

extern "C" int wush_fused_tq(const uint16_t* x, const uint16_t* t, uint8_t* q, uint16_t* s,
                             int64_t rows, int64_t K, hipStream_t stream) {
    WUSH_REQUIRE(rows >= 0 && K > 0 && K % 32 == 0);
    if (rows == 0) return (int)hipSuccess;
    WUSH_REQUIRE(x && t && q && s);
    WUSH_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)t & 15u) == 0 &&
                 ((uintptr_t)q & 15u) == 0 && ((uintptr_t)s & 1u) == 0);
    const int64_t C = K / 32;
    if (rows * C <= WUSH_TQ_SMALLM_PAIRS) {
        const int64_t gx = (C + wush::kPairsPerWg - 1) / wush::kPairsPerWg;
        WUSH_REQUIRE(gx <= 0x7fffffffLL && rows <= 65535);
        wush::fused_tq_smallm_kernel<<<dim3((unsigned)gx, (unsigned)rows), 64, 0, stream>>>(x, t, q, s, rows, K);
    } else {
        const int64_t gx = (C + wush::kBlocksPerWg - 1) / wush::kBlocksPerWg;
        const int64_t gy = (rows + wush::kRowsPerWave - 1) / wush::kRowsPerWave;
        WUSH_REQUIRE(gx <= 0x7fffffffLL && gy <= 65535);
        const dim3 grid((unsigned)gx, (unsigned)gy);
        if (gy * C < WUSH_TQ_DPP_WAVES)
            wush::fused_tq_rows_kernel<true><<<grid, 256, 0, stream>>>(x, t, q, s, rows, K);
        else
            wush::fused_tq_rows_kernel<false><<<grid, 256, 0, stream>>>(x, t, q, s, rows, K);
    }
    return (int)hipGetLastError();
}
