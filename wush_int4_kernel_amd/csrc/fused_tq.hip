// fused_tq.hip -- WUSH block-diagonal transform fused with the INT4 group
// quantization, bit-exact with the reference's sequential form
// (csrc/fused_tq_int4.cu:27-85; tests/test_sw2.py:12-24):
//   x'_j = sum_{i=0..31} x_i * T[c][j][i]   (fp32, i ascending, mul then add)
//   then the quant_int4 chain on the fp32 x' (no bf16 rounding of x').
// Transformed activations never touch HBM.
//
// Two launch shapes, one numerics (the small-M per-pair steps live in
// fused_tq_device.h):
//  * rows kernel: lane = row, wavefront = 64 rows of one block c, 4
//    wavefronts of a workgroup on 4 adjacent blocks of the same 64 rows (each
//    row's 256 B of bf16 input is consumed by one workgroup).  A product of
//    two bf16 values is exact in fp32 unless an operand is extreme (tiny,
//    huge, inf or NaN), and then fma(x, T, acc) equals the reference's
//    acc + x*T bit for bit.  When the wavefront's x and T lie in the range
//    that also keeps every partial sum normal (almost always), the transform
//    runs as 32 rank-1 steps of the fp32 matrix cores (MFMA form below);
//    otherwise as 1024 fmas per lane, or the mul-then-add sequence itself,
//    with T in SGPRs (scalar loads converted on the SALU).
//  * small-M kernel (at most 16384 (row, block) pairs: decode, small batches):
//    32 lanes per (row, block), two adjacent blocks of one row per
//    one-wavefront workgroup (grid: block pairs x rows) so a decode row
//    spreads over K/64 CUs; lane j computes x'_j with T[c][j] read
//    as 64 coalesced bytes and x broadcast from LDS (one fma per MAC when the
//    wavefront's x and T are in range, as above); the group sums are then
//    re-run in i-order by every lane from LDS (so they keep the sequential
//    order) and lane pairs pack nibbles.
#include "fused_tq_device.h"
#include "setup.h"
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

// ------------------------------------------------------------- MFMA form
// The transform as 32 rank-1 steps on the fp32 matrix cores.
// v_mfma_f32_32x32x1_2b_f32 adds a[m] * b[n] to acc[m][n] for two
// independent 32 x 32 blocks, one product per output and step, rounded once
// to nearest even as fma rounds (x' itself is compared bit for bit with the
// sequential sums, ties included, by test_fused_transform_stage_bit_exact
// through wush_fused_tq_transform32).  With a[m] =
// T[c][m][i] and b[n] = x[r0 + 32k + n][i] for block k, step i adds x_i *
// T[c][j][i] to x'_j of the wavefront's 64 rows, i ascending: the
// reference's sequence whenever every product is exact and nothing is
// subnormal.  Both hold when every x and T value is zero or has magnitude in
// [2^-56, 2^51): a product then has at most 16 significant bits, the lowest
// at or above 2^-126, so every partial sum is a multiple of 2^-126 (zero or
// normal) below 2^107.  Wavefronts with a value outside that range take the
// fma or mul-then-add loop instead (transform_block).  The matrix cores run
// the fp32 MACs at twice the VALU's rate; on gfx950 they do not overlap the
// quantization's VALU work, so a wavefront costs 32 MFMAs of 64 cycles plus
// about 600 VALU instructions (4096 rows, K = 8192: 43 -> 37 us).
constexpr uint32_t kMfmaSafeLo = 0x2380u;        // bf16 magnitude bits of 2^-56

typedef float v32f __attribute__((ext_vector_type(32)));

// x'_j of the wavefront's 64 rows in xp (lane = row): the 32 MFMA steps on
// tf (the lane's row l % 32 of T[c] in fp32), then the regrouping.  Block k's output is
// in registers 16k .. 16k + 15: lane l, register e holds n = l % 32 and m =
// 8 (e / 4) + 4 (l / 32) + e % 4.  Swapping block 1's registers of lanes 0-31
// with block 0's of lanes 32-63 leaves lane l with all 32 x'_j of row r0 + l:
// j = 8a + b from the first register of the pair, 8a + 4 + b from the second
// (e = 4a + b).
__device__ __forceinline__ void tq_mfma_steps_f32(const float (&tf)[32], const float (&xv)[32], float (&xp)[32]) {
    v32f acc = (v32f){0.0f};
#pragma unroll
    for (int i = 0; i < 32; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x1f32(tf[i], xv[i], acc, 0, 0, 0);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e]), __float_as_uint(acc[16 + e]),
                                                         false, false);
        xp[8 * (e >> 2) + (e & 3)] = __uint_as_float(pr[0]);
        xp[8 * (e >> 2) + 4 + (e & 3)] = __uint_as_float(pr[1]);
    }
}

// The rows kernel's transform stage: x'_j (j = 0..31) of block c from the
// lane's 32 x values (ux: 16 bf16 pairs), lane = row.  The wavefront's range
// vote picks the MFMA steps, the fma loop or the mul-then-add loop (T
// through SGPRs for the last two).
__device__ __forceinline__ void tq_rows_transform(const uint32_t (&ux)[16], const uint16_t* __restrict__ t,
                                                  int64_t c, int lane, float (&xp)[32]) {
    // lane l: row l % 32 of T[c], the MFMA's A operand for both blocks
    const uint32_t* tc = reinterpret_cast<const uint32_t*>(t + c * 1024);
    const uint4* t4 = reinterpret_cast<const uint4*>(tc + (lane & 31) * 16);
    uint32_t ut[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 a = t4[k];
        ut[4 * k] = a.x; ut[4 * k + 1] = a.y; ut[4 * k + 2] = a.z; ut[4 * k + 3] = a.w;
    }
    // range of the wavefront's x and T (each lane checks its T row)
    BfRange rg;
    float xv[32];
#pragma unroll
    for (int d = 0; d < 16; ++d) {
        xv[2 * d] = bf16_to_f32(ux[d] & 0xffffu);
        xv[2 * d + 1] = __uint_as_float(ux[d] & 0xffff0000u);
        rg.add(ux[d]);
        rg.add(ut[d]);
    }
    if (__all(rg.safe_from(kMfmaSafeLo))) {
        float tf[32];
#pragma unroll
        for (int d = 0; d < 16; ++d) {
            tf[2 * d] = bf16_to_f32(ut[d] & 0xffffu);
            tf[2 * d + 1] = __uint_as_float(ut[d] & 0xffff0000u);
        }
        tq_mfma_steps_f32(tf, xv, xp);
    }
    else if (__all(rg.safe())) transform_block<true>(xv, tc, xp);
    else transform_block<false>(xv, tc, xp);
}

__device__ __forceinline__ void load_words16(const uint16_t* __restrict__ p, uint32_t (&u)[16]) {
    const uint4* p4 = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 v = p4[k];
        u[4 * k] = v.x; u[4 * k + 1] = v.y; u[4 * k + 2] = v.z; u[4 * k + 3] = v.w;
    }
}

// Workgroup: 64 rows (r0 ..) x 4 adjacent blocks (cb ..); wavefront w
// computes block cb + w, lane = row.  Each row's 256 input bytes and its 64
// bytes of codes and 8 of scales are contiguous, but a lane-per-row access
// touches one row per lane.  So the workgroup stages both through LDS: 16
// lanes read one row's 256 bytes (4 rows per load instruction), and 4 lanes
// write one row's codes and scales.  Rows past the last row and blocks past
// the last block are read clamped and not stored.
constexpr int kTqXPitch = 272;                   // LDS bytes per staged input row (256 + 16: no bank conflicts)
constexpr int kTqQPitch = 80;                    // ... per staged code row (64 + 16)

__global__ __launch_bounds__(256) void fused_tq_rows_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ t,
                                                            uint8_t* __restrict__ q,
                                                            uint16_t* __restrict__ s,
                                                            int64_t rows, int64_t K) {
    __shared__ __align__(16) uint8_t sx[kRowsPerWave * kTqXPitch];
    __shared__ __align__(16) uint8_t sq[kRowsPerWave * kTqQPitch];
    __shared__ __align__(16) uint16_t ss[kRowsPerWave * kBlocksPerWg];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int64_t C = K >> 5;
    const int64_t cb = (int64_t)blockIdx.x * kBlocksPerWg;
    const int64_t r0 = (int64_t)blockIdx.y * kRowsPerWave;

    // tile inside both tensors (workgroup-uniform): wave-uniform bases plus
    // 32-bit lane offsets (below 8 K + 128 bytes, so K < 2^28 keeps them in
    // range), no clamping
    const bool full = r0 + kRowsPerWave <= rows && cb + kBlocksPerWg <= C && K < ((int64_t)1 << 28);

    // coalesced input: wavefront w loads rows 16w .. 16w + 15 of the tile
    if (full) {
        const global_cptr<uint8_t> xb =
            uniform_ptr(reinterpret_cast<const uint8_t*>(x + (r0 + 16 * wave) * K + cb * 32));
        uint32_t lo = ((uint32_t)(lane >> 4) * (uint32_t)K + (uint32_t)(lane & 15) * 8u) * 2u;
        asm("" : "+v"(lo));                      // keeps the 32-bit lane offset form
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32x4 v = *reinterpret_cast<global_cptr<u32x4>>(xb + (size_t)(8 * k) * (size_t)K + lo);
            *reinterpret_cast<u32x4*>(sx + (16 * wave + 4 * k + (lane >> 4)) * kTqXPitch + (lane & 15) * 16) = v;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int rl = 16 * wave + 4 * k + (lane >> 4);
            const int64_t rr = min(r0 + rl, rows - 1);
            const int64_t cc = min(cb + ((lane & 15) >> 2), C - 1);
            const uint4 v = *reinterpret_cast<const uint4*>(x + rr * K + cc * 32 + (lane & 3) * 8);
            *reinterpret_cast<uint4*>(sx + rl * kTqXPitch + (lane & 15) * 16) = v;
        }
    }
    __syncthreads();
    uint32_t ux[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 v = *reinterpret_cast<const uint4*>(sx + lane * kTqXPitch + wave * 64 + k * 16);
        ux[4 * k] = v.x; ux[4 * k + 1] = v.y; ux[4 * k + 2] = v.z; ux[4 * k + 3] = v.w;
    }

    const int64_t c = min(cb + wave, C - 1);
    float xp[32];
    tq_rows_transform(ux, t, c, lane, xp);
    uint32_t w[4];
    const uint32_t sb = quant_group32(xp, w);
    *reinterpret_cast<uint4*>(sq + lane * kTqQPitch + wave * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    ss[lane * kBlocksPerWg + wave] = (uint16_t)sb;
    __syncthreads();

    // coalesced output: wavefront w stores rows 16w .. 16w + 15, 4 lanes a row
    const int rl = 16 * wave + (lane >> 2);
    const int bl = lane & 3;
    const u32x4 qv = *reinterpret_cast<const u32x4*>(sq + rl * kTqQPitch + bl * 16);
    const uint16_t sv = ss[rl * kBlocksPerWg + bl];
    if (full) {
        const int64_t e0 = (r0 + 16 * wave) * C + cb;           // first (row, block) of the wavefront
        const global_ptr<uint8_t> qb = uniform_wptr(q + e0 * 16);
        const global_ptr<uint16_t> sp = uniform_wptr(s + e0);
        uint32_t eo = (uint32_t)(lane >> 2) * (uint32_t)C + (uint32_t)bl;
        asm("" : "+v"(eo));
        *reinterpret_cast<global_ptr<u32x4>>(qb + eo * 16u) = qv;
        sp[eo] = sv;
    } else {
        const int64_t r = r0 + rl, cs = cb + bl;
        if (r < rows && cs < C) {
            *reinterpret_cast<u32x4*>(q + (r * C + cs) * 16) = qv;
            s[r * C + cs] = sv;
        }
    }
}

// Two 64-row tiles per wavefront (128 rows x 4 blocks per workgroup): the
// rows kernel's steps, with the wavefront's T row requested first, converted
// to fp32 and range-checked once for both tiles, and both tiles' input
// requested before the first tile's transform.  On gfx950 the fp32 MFMA
// steps and the VALU do not run at the same time (not in one wavefront, not
// across the wavefronts of a SIMD), so the tiles simply run one after the
// other; the gain is the shared T work and its hidden latency.  Launched
// where its 128-row workgroups leave no CU with more tiles than the rows
// kernel's 64-row ones would.
constexpr int kRows2 = 2 * kRowsPerWave;

__global__ __launch_bounds__(256) void fused_tq_rows2_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ t,
                                                             uint8_t* __restrict__ q,
                                                             uint16_t* __restrict__ s,
                                                             int64_t rows, int64_t K) {
    __shared__ __align__(16) uint8_t sx[kRows2 * kTqXPitch];
    __shared__ __align__(16) uint8_t sq[kRows2 * kTqQPitch];
    __shared__ __align__(16) uint16_t ss[kRows2 * kBlocksPerWg];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int64_t C = K >> 5;
    const int64_t cb = (int64_t)blockIdx.x * kBlocksPerWg;
    const int64_t r0 = (int64_t)blockIdx.y * kRows2;
    const bool full = r0 + kRows2 <= rows && cb + kBlocksPerWg <= C && K < ((int64_t)1 << 28);

    // row lane % 32 of this wavefront's T[c], the MFMA's A operand for both tiles
    const int64_t c = min(cb + wave, C - 1);
    const uint32_t* tc = reinterpret_cast<const uint32_t*>(t + c * 1024);
    uint32_t ut[16];
    {
        const uint4* t4 = reinterpret_cast<const uint4*>(tc + (lane & 31) * 16);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 a = t4[k];
            ut[4 * k] = a.x; ut[4 * k + 1] = a.y; ut[4 * k + 2] = a.z; ut[4 * k + 3] = a.w;
        }
    }
    // both tiles' input, coalesced: wavefront w loads rows 16w .. 16w + 15 of each
    u32x4 vin[2][4];
    if (full) {
        uint32_t lo = ((uint32_t)(lane >> 4) * (uint32_t)K + (uint32_t)(lane & 15) * 8u) * 2u;
        asm("" : "+v"(lo));                      // keeps the 32-bit lane offset form
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const global_cptr<uint8_t> xb = uniform_ptr(
                reinterpret_cast<const uint8_t*>(x + (r0 + kRowsPerWave * h + 16 * wave) * K + cb * 32));
#pragma unroll
            for (int k = 0; k < 4; ++k)
                vin[h][k] = *reinterpret_cast<global_cptr<u32x4>>(xb + (size_t)(8 * k) * (size_t)K + lo);
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int rl = kRowsPerWave * h + 16 * wave + 4 * k + (lane >> 4);
                const int64_t rr = min(r0 + rl, rows - 1);
                const int64_t cc = min(cb + ((lane & 15) >> 2), C - 1);
                const uint4 v = *reinterpret_cast<const uint4*>(x + rr * K + cc * 32 + (lane & 3) * 8);
                vin[h][k] = (u32x4){v.x, v.y, v.z, v.w};
            }
    }
    float tf[32];
    BfRange rg_t;
#pragma unroll
    for (int d = 0; d < 16; ++d) {
        tf[2 * d] = bf16_to_f32(ut[d] & 0xffffu);
        tf[2 * d + 1] = __uint_as_float(ut[d] & 0xffff0000u);
        rg_t.add(ut[d]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        // tile h through LDS (rows 64h ..; tile 0's rows are not written again)
#pragma unroll
        for (int k = 0; k < 4; ++k)
            *reinterpret_cast<u32x4*>(sx + (kRowsPerWave * h + 16 * wave + 4 * k + (lane >> 4)) * kTqXPitch +
                                      (lane & 15) * 16) = vin[h][k];
        __syncthreads();
        uint32_t ux[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint4 v = *reinterpret_cast<const uint4*>(sx + (kRowsPerWave * h + lane) * kTqXPitch + wave * 64 +
                                                            k * 16);
            ux[4 * k] = v.x; ux[4 * k + 1] = v.y; ux[4 * k + 2] = v.z; ux[4 * k + 3] = v.w;
        }
        float xv[32];
        BfRange rg = rg_t;
#pragma unroll
        for (int d = 0; d < 16; ++d) {
            xv[2 * d] = bf16_to_f32(ux[d] & 0xffffu);
            xv[2 * d + 1] = __uint_as_float(ux[d] & 0xffff0000u);
            rg.add(ux[d]);
        }
        float xp[32];
        if (__all(rg.safe_from(kMfmaSafeLo))) tq_mfma_steps_f32(tf, xv, xp);
        else if (__all(rg.safe())) transform_block<true>(xv, tc, xp);
        else transform_block<false>(xv, tc, xp);
        uint32_t w[4];
        const uint32_t sb = quant_group32(xp, w);
        *reinterpret_cast<uint4*>(sq + (kRowsPerWave * h + lane) * kTqQPitch + wave * 16) =
            make_uint4(w[0], w[1], w[2], w[3]);
        ss[(kRowsPerWave * h + lane) * kBlocksPerWg + wave] = (uint16_t)sb;
    }
    __syncthreads();

    // coalesced output: wavefront w stores rows 32w .. 32w + 31, 16 a pass, 4 lanes a row
    const int bl = lane & 3;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const int rl = 32 * wave + 16 * p + (lane >> 2);
        const u32x4 qv = *reinterpret_cast<const u32x4*>(sq + rl * kTqQPitch + bl * 16);
        const uint16_t sv = ss[rl * kBlocksPerWg + bl];
        if (full) {
            const int64_t e0 = (r0 + 32 * wave + 16 * p) * C + cb;
            const global_ptr<uint8_t> qb = uniform_wptr(q + e0 * 16);
            const global_ptr<uint16_t> sp = uniform_wptr(s + e0);
            uint32_t eo = (uint32_t)(lane >> 2) * (uint32_t)C + (uint32_t)bl;
            asm("" : "+v"(eo));
            *reinterpret_cast<global_ptr<u32x4>>(qb + eo * 16u) = qv;
            sp[eo] = sv;
        } else {
            const int64_t r = r0 + rl, cs = cb + bl;
            if (r < rows && cs < C) {
                *reinterpret_cast<u32x4*>(q + (r * C + cs) * 16) = qv;
                s[r * C + cs] = sv;
            }
        }
    }
}

// The transform stage alone, for one block: x rows x 32, xp rows x 32 fp32.
__global__ __launch_bounds__(64) void fused_tq_transform32_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ t,
                                                                  float* __restrict__ xp, int64_t rows) {
    const int lane = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * kRowsPerWave;
    const int64_t r = r0 + lane;
    const bool active = r < rows;
    uint32_t ux[16];
    load_words16(x + (active ? r : r0) * 32, ux);
    float v[32];
    tq_rows_transform(ux, t, 0, lane, v);
    if (active) {
#pragma unroll
        for (int j = 0; j < 32; j += 4)
            *reinterpret_cast<float4*>(xp + r * 32 + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
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
// Smallest number of two-tile workgroups per CU at which the rows launches
// may take the two-tile kernel (a large value: never).
#ifndef WUSH_TQ_ROWS2_MIN_PER_CU
#define WUSH_TQ_ROWS2_MIN_PER_CU 2
#endif
#ifndef WUSH_TQ_SMALLM_PAIRS
#define WUSH_TQ_SMALLM_PAIRS 16384
#endif
extern "C" int wush_fused_tq(const uint16_t* x, const uint16_t* t, uint8_t* q, uint16_t* s,
                             int64_t rows, int64_t K, hipStream_t stream) {
    WUSH_REQUIRE(rows >= 0 && K > 0 && K % 32 == 0);
    if (rows == 0) return (int)hipSuccess;
    WUSH_REQUIRE(x && t && q && s);
    WUSH_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)t & 15u) == 0 &&
                 ((uintptr_t)q & 15u) == 0 && ((uintptr_t)s & 1u) == 0);
    const int64_t C = K / 32;
    // the small-M grid holds the rows in grid.y (at most 65535), so any
    // value of the tuning macro leaves larger launches to the rows kernel
    if (rows * C <= WUSH_TQ_SMALLM_PAIRS && rows <= 65535) {
        const int64_t gx = (C + wush::kPairsPerWg - 1) / wush::kPairsPerWg;
        WUSH_REQUIRE(gx <= 0x7fffffffLL);
        wush::fused_tq_smallm_kernel<<<dim3((unsigned)gx, (unsigned)rows), 64, 0, stream>>>(x, t, q, s, rows, K);
    } else {
        const int64_t gx = (C + wush::kBlocksPerWg - 1) / wush::kBlocksPerWg;
        const int64_t gy = (rows + wush::kRowsPerWave - 1) / wush::kRowsPerWave;
        const int64_t gy2 = (rows + wush::kRows2 - 1) / wush::kRows2;
        WUSH_REQUIRE(gx <= 0x7fffffffLL && gy <= 65535);
        int dev = 0;
        const int st = wush::device_setup(&dev);
        if (st != 0) return st;
        // the two-tile kernel where no CU gets more tiles than with the rows
        // kernel (workgroups spread evenly over the CUs), at least 2
        // workgroups per CU
        const int64_t cus = wush::device_cus(dev);
        const int64_t per_cu1 = (gx * gy + cus - 1) / cus, per_cu2 = (gx * gy2 + cus - 1) / cus;
        if (gx * gy2 >= WUSH_TQ_ROWS2_MIN_PER_CU * cus && 2 * per_cu2 <= per_cu1) {
            wush::fused_tq_rows2_kernel<<<dim3((unsigned)gx, (unsigned)gy2), 256, 0, stream>>>(x, t, q, s, rows, K);
        } else {
            const dim3 grid((unsigned)gx, (unsigned)gy);
            wush::fused_tq_rows_kernel<<<grid, 256, 0, stream>>>(x, t, q, s, rows, K);
        }
    }
    return (int)hipGetLastError();
}

extern "C" int wush_fused_tq_transform32(const uint16_t* x, const uint16_t* t, float* xp, int64_t rows,
                                         hipStream_t stream) {
    WUSH_REQUIRE(rows >= 0);
    if (rows == 0) return (int)hipSuccess;
    WUSH_REQUIRE(x && t && xp);
    WUSH_REQUIRE(((uintptr_t)x & 15u) == 0 && ((uintptr_t)t & 15u) == 0 && ((uintptr_t)xp & 15u) == 0);
    const int64_t g = (rows + wush::kRowsPerWave - 1) / wush::kRowsPerWave;
    WUSH_REQUIRE(g <= 0x7fffffffLL);
    wush::fused_tq_transform32_kernel<<<(unsigned)g, 64, 0, stream>>>(x, t, xp, rows);
    return (int)hipGetLastError();
}
