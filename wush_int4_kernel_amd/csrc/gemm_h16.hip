// gemm_h16.hip -- group-scaled W4A4 GEMM for prefill-sized M on fp16 MFMA
// (csrc/gemm_s4.cu:85-379 is the reference contract).
//
//   y[m][n] = sum_g sum_{k in g} (qx[m][k] * sx[m][g]) * (qw[n][k] * sw[n][g])
//
// The int8 kernels fold every 32x32 block of exact group dots into fp32 with
// two VALU operations per output and group, which bounds them at a quarter of
// the int8 MFMA rate.  Here the scales go into the operands instead: a code
// (3 bits of magnitude) times a bf16 scale (8-bit significand) is exact in
// fp16 (11-bit significand) once the scale sits in fp16's exponent range, and
// the product of two such operands is exact in fp32 (22 bits).  So
// v_mfma_f32_32x32x16_f16 accumulates exact terms in fp32 over the whole K and
// nothing runs per output in the main loop.
//
// Range: every activation row m gets a power of two 2^ea[m], chosen from the
// row's largest scale so that it lands in [2^12, 2^13) (code * scale <= 7 *
// 2^13 < 65504); likewise 2^eb[n] per weight column.  The epilogue multiplies
// by 2^-(ea[m] + eb[n]) with v_ldexp_f32 (exact).  Every scale down to
// 2^-22 of its row's largest converts exactly; smaller ones land in fp16's
// subnormal range and keep fewer bits (an absolute error below 2^-36 of the
// row's largest scale per term).  A row or column with a non-finite scale
// gives NaN, as the reference's dequantized product does (code 0 * inf).
//
// Workgroup: 8 wavefronts in 2 x 4, a 256 x 256 output tile, each wavefront
// 128 x 64 (8 accumulator blocks), one workgroup per CU.  A stage is one
// group (K = 32): thread t converts row t of the activation tile (t < 256)
// or column t - 256 of the weight tile (16 code bytes each) to fp16 in a
// double-buffered LDS tile laid out fragment-major, [K16 slice][32-row block]
// [k-half][row][8 halves], so that a wavefront's operand read of one 32-row
// block is 1 KiB contiguous (lane l at 16*l) and the conversion writes of
// 64 consecutive rows are contiguous too.  Global loads run in batches of four
// groups (64 bytes of every row, four stages ahead), four lanes per row so an
// instruction reads 16 rows of 64 contiguous bytes, then a 4 x 4 in-quad
// transpose gives every lane its own row; addresses are clamped, so the loop
// has no conditional loads.
#include "wush_device.h"
#include "gemm_h16.h"
#include "setup.h"

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
#ifndef WUSH_H16_XCD
#define WUSH_H16_XCD 1                           // XCD-aware tile order in the 8-wavefront kernel
#endif

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

// Scale operand pair (s, s) and (s/16, s/16) in fp16 for the fp32 value f
// of a bf16 scale and the row's shift.
__device__ __forceinline__ void h16_scale(float f, int shift, h2& s, h2& s16) {
    const _Float16 a = (_Float16)__builtin_ldexpf(f, shift);
    const _Float16 c = (_Float16)__builtin_ldexpf(f, shift - 4);
    s = (h2){a, a};
    s16 = (h2){c, c};
}

// 8 s4 codes (element 2k in the low nibble of byte k) -> 8 fp16 code*scale
// values, in the order k = 0,4,1,5,2,6,3,7 (the same for both operands, so
// the dot product only sums in another order).  After the XOR each nibble is
// code + 8 in [1, 15]; OR-ing it into 0x6400 (1024.0) gives 1024 + code + 8
// (low nibble) or 1024 + 16 * (code + 8) (high nibble of a byte), both exact;
// the subtraction leaves code or 16 * code exactly and the product with s or
// s/16 is one exact fp16 rounding.
// (a & b) | c in one v_bitop3_b32 (truth table 0xEA for src0 = a, src1 = b,
// src2 = c); left to itself the compiler fuses the XOR below into the AND
// instead and spends a v_or_b32 per pair.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0xea" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

__device__ __forceinline__ uint4 h16_codes(uint32_t w, h2 s, h2 s16) {
    const uint32_t t = w ^ 0x88888888u;
    const uint32_t t8 = t >> 8;
    const h2 b0 = {(_Float16)1032.0f, (_Float16)1032.0f};
    const h2 b1 = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2 p0 = __builtin_bit_cast(h2, and_or(t, 0x000F000Fu, 0x64006400u));
    const h2 p1 = __builtin_bit_cast(h2, and_or(t, 0x00F000F0u, 0x64006400u));
    const h2 p2 = __builtin_bit_cast(h2, and_or(t8, 0x000F000Fu, 0x64006400u));
    const h2 p3 = __builtin_bit_cast(h2, and_or(t8, 0x00F000F0u, 0x64006400u));
    uint4 r;
    r.x = __builtin_bit_cast(uint32_t, (h2)((p0 - b0) * s));
    r.y = __builtin_bit_cast(uint32_t, (h2)((p1 - b1) * s16));
    r.z = __builtin_bit_cast(uint32_t, (h2)((p2 - b0) * s));
    r.w = __builtin_bit_cast(uint32_t, (h2)((p3 - b1) * s16));
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

// 8 wavefronts per workgroup (2 per SIMD): the MFMA tiles are 128 x 64 per
// wavefront (2 x 4 wavefronts, 128 fp32 accumulators), and wavefronts 0-3
// convert the activation rows, 4-7 the weight columns.  A second wavefront
// per SIMD lets the conversion VALU of one run beside the MFMAs of the other
// (with 4 wavefronts of 128 x 128, L70 M=4096 took 4.51 ms against 3.75).
template <bool VEC>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_h16w8_kernel(const uint8_t* __restrict__ xq, const uint16_t* __restrict__ xs,
                       const uint8_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                       uint16_t* __restrict__ y, float* __restrict__ partial, int M, int N, int K,
                       int groups_per_split) {
    extern __shared__ __align__(16) uint8_t smem[];
    int* sh_e = reinterpret_cast<int*>(smem + 2 * kH16Buf);   // [0, 256) rows, [256, 512) columns

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
#if WUSH_H16_XCD
    // Workgroup i runs on XCD i % 8.  When the column tiles split evenly
    // over the 8 XCDs, XCD x takes column tiles x, x + 8, ... and walks all
    // row tiles of one before the next, so the workgroups in flight on an XCD
    // share a few weight tiles in its L2.
    int tm = blockIdx.y, tn = blockIdx.x;
    if ((gridDim.x & 7) == 0) {
        const uint64_t id = (uint64_t)blockIdx.y * gridDim.x + blockIdx.x;
        const uint64_t slot = id >> 3;
        tm = (int)(slot % gridDim.y);
        tn = (int)((slot / gridDim.y) * 8 + (id & 7));
    }
    const int m0 = tm * kH16Tile;
    const int n0 = tn * kH16Tile;
#else
    const int m0 = blockIdx.y * kH16Tile;
    const int n0 = blockIdx.x * kH16Tile;
#endif
    const int GR = K >> 5;                       // groups of a row
    const int K2 = K >> 1;
    // K slice of this workgroup (blockIdx.z): groups [gb, gb + G), G % 8 == 0
    const int gb = blockIdx.z * groups_per_split;
    const int G = min(GR - gb, groups_per_split);

    // conversion role (wavefront-uniform): operand, its row r in the tile
    const bool wside = wave >= 4;
    const int r = tid & 255;
    const uint8_t* codes = wside ? wq : xq;
    const int lim = (wside ? N : M) - 1;
    const int base = wside ? n0 : m0;
    const uint16_t* ps = (wside ? ws : xs) + (size_t)min(base + r, lim) * GR + gb;

    uint32_t mx, mx2;
    h16_row_max<VEC>(ps, ps, G, mx, mx2);
    const int e = h16_shift(mx);
    sh_e[tid] = e;

    const int p4 = lane & 3;
    const int wrow = base + (wave & 3) * 64 + (lane & ~3);
    const uint8_t* qc[kH16Batch];
#pragma unroll
    for (int i = 0; i < kH16Batch; ++i) qc[i] = codes + (size_t)min(wrow + i, lim) * K2 + gb * 16 + p4 * 16;

    struct Batch {
        uint4 c[kH16Batch];
        uint32_t s[kH16Batch];
    };
    auto load_batch = [&](int b, Batch& rr) {
        const int g0 = min(b * kH16Batch, G - kH16Batch) * 16;
#pragma unroll
        for (int i = 0; i < kH16Batch; ++i) rr.c[i] = *reinterpret_cast<const uint4*>(qc[i] + g0);
        if constexpr (VEC) {
            const uint2 v = *reinterpret_cast<const uint2*>(ps + min(b * kH16Batch, G - kH16Batch));
            rr.s[0] = v.x; rr.s[1] = v.y;
        } else {
#pragma unroll
            for (int i = 0; i < kH16Batch; ++i) rr.s[i] = ps[min(b * kH16Batch + i, G - 1)];
        }
    };
    const bool odd1 = (lane & 1) != 0;
    const bool odd2 = (lane & 2) != 0;
    auto transpose = [&](uint4 (&x)[kH16Batch]) {
        uint4 z[kH16Batch];
#pragma unroll
        for (int i = 0; i < kH16Batch; ++i) {
            const bool own = ((i & 1) != 0) == odd1;
            const uint4 o = x[i ^ 1];
            z[i].x = h16_xchg<0xB1>(x[i].x, o.x, !own);
            z[i].y = h16_xchg<0xB1>(x[i].y, o.y, !own);
            z[i].z = h16_xchg<0xB1>(x[i].z, o.z, !own);
            z[i].w = h16_xchg<0xB1>(x[i].w, o.w, !own);
        }
#pragma unroll
        for (int i = 0; i < kH16Batch; ++i) {
            const bool own = ((i & 2) != 0) == odd2;
            const uint4 o = z[i ^ 2];
            x[i].x = h16_xchg<0x4E>(z[i].x, o.x, !own);
            x[i].y = h16_xchg<0x4E>(z[i].y, o.y, !own);
            x[i].z = h16_xchg<0x4E>(z[i].z, o.z, !own);
            x[i].w = h16_xchg<0x4E>(z[i].w, o.w, !own);
        }
    };

    Batch R0, R1;
    load_batch(0, R0);
    load_batch(1, R1);

    const int wofs = (wside ? kH16Op : 0) + (r >> 5) * 1024;
    auto convert = [&](int buf, Batch& rr, int i) {
        if (i == 0) transpose(rr.c);
        uint8_t* dst = smem + buf * kH16Buf + wofs;
        h2 sc, sc16;
        h16_scale(h16_batch_scale<VEC>(rr.s, i), e, sc, sc16);
        const uint32_t w4[4] = {rr.c[i].x, rr.c[i].y, rr.c[i].z, rr.c[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            frag_write(dst + (j >> 1) * kH16Slice, (r & 31) + 32 * (j & 1), h16_codes(w4[j], sc, sc16));
    };

    v16f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){0.0f};

    const int rba = (wave >> 2) * 4;             // this wavefront's first 32-row block
    const int rbb = (wave & 3) * 2;              // ... and first 32-column block
    auto compute = [&](int buf) {
        const uint8_t* b0 = smem + buf * kH16Buf;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            h8 af[4], bf[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = frag_read(b0 + kk * kH16Slice + (rba + i) * 1024, lane);
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = frag_read(b0 + kH16Op + kk * kH16Slice + (rbb + j) * 1024, lane);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    convert(0, R0, 0);
    __syncthreads();

    for (int s0 = 0; s0 < G; s0 += 2 * kH16Batch) {
#pragma unroll
        for (int j = 0; j < 2 * kH16Batch; ++j) {
            compute(j & 1);
            if (j < kH16Batch - 1) convert((j + 1) & 1, R0, j + 1);
            else if (j == kH16Batch - 1) convert(0, R1, 0);
            else if (j < 2 * kH16Batch - 1) convert((j + 1) & 1, R1, j + 1 - kH16Batch);
            else convert(0, R0, 0);
            if (j == kH16Batch - 1) load_batch(s0 / kH16Batch + 2, R0);
            if (j == 2 * kH16Batch - 1) load_batch(s0 / kH16Batch + 3, R1);
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    const int half = lane >> 5;
    const int l32 = lane & 31;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int cl = (rbb + j) * 32 + l32;
        const int col = n0 + cl;
        const int e_col = sh_e[256 + cl];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int rl = (rba + i) * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                const int row = m0 + rl;
                const int e_row = sh_e[rl];
                float v = __builtin_ldexpf(acc[i][j][q], -(e_row + e_col));
                if (e_row == kH16NonFinite || e_col == kH16NonFinite) v = __builtin_nanf("");
                if (row < M && col < N) {
                    if (partial != nullptr)
                        partial[((size_t)blockIdx.z * M + row) * N + col] = v;
                    else
                        y[(size_t)row * N + col] = f32_to_f16_bits(v);
                }
            }
        }
    }
}

// ------------------------------------------------ pre-converted activations
// For wide weight matrices every 256-row activation tile above is converted
// again by each of the N/256 column tiles.  gemm_h16a converts the
// activations once (h16_prep_a_kernel, M x K x 2 bytes of workspace), in the
// MFMA fragment layout, and streams them into a 4-slot LDS ring with
// global_load_lds_dwordx4 (no VGPRs, issued 3 stages ahead by wavefronts
// 0-3); wavefronts 4-7 convert the weight columns as above.  Same operands,
// same MFMA order: bit-identical to gemm_h16w8_kernel.

// a16 layout: [32-row block][group][K16 slice][64 lanes][16 B] (one block
// and group: the two 1 KiB operand fragments of v_mfma_f32_32x32x16_f16);
// ea[slice][row] = the row's power-of-two shift over the K slice, as the
// per-tile conversion computes it.  Grid: (Mpad / 32, splits): a workgroup
// converts 32 rows of one slice.
constexpr int kH16aRing = 4;                      // LDS ring slots of the activation operand

__global__ __launch_bounds__(256) void h16_prep_a_kernel(const uint8_t* __restrict__ xq,
                                                         const uint16_t* __restrict__ xs,
                                                         uint8_t* __restrict__ a16, int* __restrict__ ea,
                                                         int M, int K, int groups_per_split) {
    const int G = K >> 5;
    const int mpad = gridDim.x * 32;
    const int rb = blockIdx.x;
    const int slice = blockIdx.y;
    const int sg0 = slice * groups_per_split, sg1 = min(G, sg0 + groups_per_split);
    const int tid = threadIdx.x;
    __shared__ int se[32];
    {
        // largest |scale| of each of the block's 32 rows over the slice: 8
        // threads per row, 8 scales per load (slices are whole multiples of 8
        // groups; scales 16-byte aligned)
        const int r = tid >> 3, part = tid & 7;
        const int row = rb * 32 + r;
        u16x2 m2 = {0, 0};
        if (row < M) {
            const uint4* ps = reinterpret_cast<const uint4*>(xs + (size_t)row * G + sg0);
            const int n8 = (sg1 - sg0) >> 3;
#pragma unroll 4
            for (int i = part; i < n8; i += 8) {
                const uint4 v = ps[i];
                m2 = __builtin_elementwise_max(m2, __builtin_elementwise_max(abs_bits2(v.x), abs_bits2(v.y)));
                m2 = __builtin_elementwise_max(m2, __builtin_elementwise_max(abs_bits2(v.z), abs_bits2(v.w)));
            }
        }
        uint32_t mx = max((uint32_t)m2.x, (uint32_t)m2.y);
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 1));
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 2));
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 4));
        if (part == 0) {
            const int e = h16_shift(mx);
            se[r] = e;
            ea[(size_t)slice * mpad + row] = e;   // rows past M: never stored
        }
    }
    __syncthreads();
    // thread: row tid % 32 of groups sg0 + tid / 32, + 8, ...
    const int rr = tid & 31;
    const int row = rb * 32 + rr;
    const int e = se[rr];
#pragma unroll 4
    for (int g = sg0 + (tid >> 5); g < sg1; g += 8) {
        uint4 w = {0, 0, 0, 0};
        float f = 0.0f;
        if (row < M) {
            w = *reinterpret_cast<const uint4*>(xq + (size_t)row * (K >> 1) + g * 16);
            f = __uint_as_float((uint32_t)xs[(size_t)row * G + g] << 16);
        }
        h2 sc, sc16;
        h16_scale(f, e, sc, sc16);
        uint8_t* dst = a16 + ((size_t)rb * G + g) * 2048;
        frag_write(dst, rr, h16_codes(w.x, sc, sc16));
        frag_write(dst, rr + 32, h16_codes(w.y, sc, sc16));
        frag_write(dst + 1024, rr, h16_codes(w.z, sc, sc16));
        frag_write(dst + 1024, rr + 32, h16_codes(w.w, sc, sc16));
    }
}

// s_waitcnt vmcnt(n) (n < 64) with the other counters left alone, and a
// workgroup barrier after this wavefront's LDS writes (no wait on vector
// memory: the activation DMA has its own explicit vmcnt waits)
#define WUSH_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define WUSH_LDS_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

typedef __attribute__((address_space(3))) void* h16_lds_ptr;
typedef __attribute__((address_space(1))) void* h16_glb_ptr;
// 16 bytes per lane from global memory straight into LDS at dst + 16 * lane
// (dst wave-uniform)
__device__ __forceinline__ void h16_dma16(const void* g, void* l) {
    __builtin_amdgcn_global_load_lds((h16_glb_ptr)(g), (h16_lds_ptr)(l), 16, 0, 0);
}

// Tile order: workgroup id i runs on XCD i % 8; each XCD walks its column
// tiles in groups of 8, row-major within a group, so the workgroups in
// flight on an XCD share 8 weight column tiles and a few activation tiles
// in its L2.
__device__ __forceinline__ void h16a_tile(int& tm, int& tn) {
    tm = blockIdx.y;
    tn = blockIdx.x;
    if ((gridDim.x & 7) != 0) return;
    constexpr uint32_t kGroup = 8;
    const uint32_t id = blockIdx.y * gridDim.x + blockIdx.x;
    const uint32_t q = id >> 3, x = id & 7;
    const uint32_t NR = gridDim.y, NC = gridDim.x >> 3;
    const uint32_t gsize = kGroup * NR;
    const uint32_t g = q / gsize, w = q % gsize;
    const uint32_t width = min(kGroup, NC - g * kGroup);
    tm = (int)(w / width);
    tn = (int)((g * kGroup + w % width) * 8 + x);
}

// Scales 16-byte aligned and K % 256 == 0 (whole batches of 8 groups).
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_h16a_kernel(const uint8_t* __restrict__ a16, const int* __restrict__ ea, const uint8_t* __restrict__ wq,
                      const uint16_t* __restrict__ ws, uint16_t* __restrict__ y, float* __restrict__ partial, int M,
                      int N, int K, int groups_per_split) {
    // one LDS object per ring slot, so that the waitcnt insertion sees that an
    // operand read of one slot does not alias a DMA into another
    __shared__ __align__(16) uint8_t sA0[kH16Op], sA1[kH16Op], sA2[kH16Op], sA3[kH16Op];
    __shared__ __align__(16) uint8_t sB0[kH16Op], sB1[kH16Op];
    auto slotA = [&](int i) -> uint8_t* { return i == 0 ? sA0 : i == 1 ? sA1 : i == 2 ? sA2 : sA3; };
    auto slotB = [&](int i) -> uint8_t* { return i == 0 ? sB0 : sB1; };
    __shared__ int sh_e[512];                    // [0, 256) rows, [256, 512) columns

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    int tm, tn;
    h16a_tile(tm, tn);
    const int m0 = tm * kH16Tile;
    const int n0 = tn * kH16Tile;
    const int GR = K >> 5;
    const int K2 = K >> 1;
    const int gb = blockIdx.z * groups_per_split;
    const int G = min(GR - gb, groups_per_split);

    const bool wside = wave >= 4;
    const int r = tid & 255;
    const int limn = N - 1;
    const uint16_t* ps = ws + (size_t)min(n0 + r, limn) * GR + gb;
    int e = 0;
    if (wside) {
        uint32_t mx, mx2;
        h16_row_max<true>(ps, ps, G, mx, mx2);
        e = h16_shift(mx);
        sh_e[tid] = e;
    } else {
        sh_e[tid] = ea[(size_t)blockIdx.z * (gridDim.y * kH16Tile) + m0 + tid];   // padded rows included
    }

    // activation DMA of this wavefront (0-3): row blocks 2w, 2w + 1
    const uint8_t* asrc = a16 + ((size_t)((m0 >> 5) + 2 * (wave & 3)) * GR + gb) * 2048 + lane * 16;
    const size_t arb = (size_t)GR * 2048;        // next row block
    auto issue_a = [&](int st, int slot) {
        const int sc = min(st, G - 1);           // stages past the slice re-read the last one
        uint8_t* dst = slotA(slot) + 2 * (wave & 3) * 1024;
        const uint8_t* src = asrc + (size_t)sc * 2048;
        h16_dma16(src, dst);
        h16_dma16(src + 1024, dst + kH16Slice);
        h16_dma16(src + arb, dst + 1024);
        h16_dma16(src + arb + 1024, dst + kH16Slice + 1024);
    };

    // weight loads (wavefronts 4-7), as in gemm_h16w8_kernel
    const int p4 = lane & 3;
    const int wrow = n0 + (wave & 3) * 64 + (lane & ~3);
    const uint8_t* qc[kH16Batch];
#pragma unroll
    for (int i = 0; i < kH16Batch; ++i) qc[i] = wq + (size_t)min(wrow + i, limn) * K2 + gb * 16 + p4 * 16;
    struct Batch {
        uint4 c[kH16Batch];
        uint32_t s[kH16Batch];                   // s[0..1]: the 4 bf16 scales as two pairs
    };
    auto load_batch = [&](int b, Batch& rr) {
        const int g0 = min(b * kH16Batch, G - kH16Batch) * 16;
#pragma unroll
        for (int i = 0; i < kH16Batch; ++i) rr.c[i] = *reinterpret_cast<const uint4*>(qc[i] + g0);
        const uint2 v = *reinterpret_cast<const uint2*>(ps + min(b * kH16Batch, G - kH16Batch));
        rr.s[0] = v.x; rr.s[1] = v.y;
    };
    const bool odd1 = (lane & 1) != 0;
    const bool odd2 = (lane & 2) != 0;
    auto transpose = [&](uint4 (&x)[kH16Batch]) {
        uint4 z[kH16Batch];
#pragma unroll
        for (int i = 0; i < kH16Batch; ++i) {
            const bool own = ((i & 1) != 0) == odd1;
            const uint4 o = x[i ^ 1];
            z[i].x = h16_xchg<0xB1>(x[i].x, o.x, !own);
            z[i].y = h16_xchg<0xB1>(x[i].y, o.y, !own);
            z[i].z = h16_xchg<0xB1>(x[i].z, o.z, !own);
            z[i].w = h16_xchg<0xB1>(x[i].w, o.w, !own);
        }
#pragma unroll
        for (int i = 0; i < kH16Batch; ++i) {
            const bool own = ((i & 2) != 0) == odd2;
            const uint4 o = z[i ^ 2];
            x[i].x = h16_xchg<0x4E>(z[i].x, o.x, !own);
            x[i].y = h16_xchg<0x4E>(z[i].y, o.y, !own);
            x[i].z = h16_xchg<0x4E>(z[i].z, o.z, !own);
            x[i].w = h16_xchg<0x4E>(z[i].w, o.w, !own);
        }
    };
    const int wofs = (r >> 5) * 1024;
    auto convert = [&](int buf, Batch& rr, int i) {
        if (i == 0) transpose(rr.c);
        uint8_t* dst = slotB(buf) + wofs;
        h2 sc, sc16;
        h16_scale(h16_batch_scale<true>(rr.s, i), e, sc, sc16);
        const uint32_t w4[4] = {rr.c[i].x, rr.c[i].y, rr.c[i].z, rr.c[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            frag_write(dst + (j >> 1) * kH16Slice, (r & 31) + 32 * (j & 1), h16_codes(w4[j], sc, sc16));
    };

    v16f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){0.0f};

    const int rba = (wave >> 2) * 4;             // this wavefront's first 32-row block
    const int rbb = (wave & 3) * 2;              // ... and first 32-column block
    auto compute = [&](int abuf, int bbuf) {
        const uint8_t* a0 = slotA(abuf);
        const uint8_t* b0 = slotB(bbuf);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            h8 af[4], bf[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = frag_read(a0 + kk * kH16Slice + (rba + i) * 1024, lane);
#pragma unroll
            for (int j = 0; j < 2; ++j) bf[j] = frag_read(b0 + kk * kH16Slice + (rbb + j) * 1024, lane);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    // Both roles run the same number of barriers: one before the first stage
    // and one after each of the G stages (G % 8 == 0).
    if (wside) {
        // weight wavefronts: convert the next stage's weights while multiplying
        Batch R0, R1;
        load_batch(0, R0);
        load_batch(1, R1);
        convert(0, R0, 0);
        WUSH_LDS_BARRIER();
        for (int s0 = 0; s0 < G; s0 += 2 * kH16Batch) {
#pragma unroll
            for (int j = 0; j < 2 * kH16Batch; ++j) {
                compute(j & (kH16aRing - 1), j & 1);
                if (j < kH16Batch - 1) convert((j + 1) & 1, R0, j + 1);
                else if (j == kH16Batch - 1) convert(0, R1, 0);
                else if (j < 2 * kH16Batch - 1) convert((j + 1) & 1, R1, j + 1 - kH16Batch);
                else convert(0, R0, 0);
                if (j == kH16Batch - 1) load_batch(s0 / kH16Batch + 2, R0);
                if (j == 2 * kH16Batch - 1) load_batch(s0 / kH16Batch + 3, R1);
                WUSH_LDS_BARRIER();
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    } else {
        // activation wavefronts: DMA the fragments kH16aRing - 1 stages ahead;
        // 4 DMAs per stage, so vmcnt <= 8 means all but the last two stages landed
        issue_a(0, 0);
        issue_a(1, 1);
        issue_a(2, 2);
        WUSH_WAIT_VMCNT(8);
        WUSH_LDS_BARRIER();
        for (int s0 = 0; s0 < G; s0 += 2 * kH16Batch) {
#pragma unroll
            for (int j = 0; j < 2 * kH16Batch; ++j) {
                issue_a(s0 + j + kH16aRing - 1, (j + kH16aRing - 1) & (kH16aRing - 1));
                compute(j & (kH16aRing - 1), j & 1);
                WUSH_WAIT_VMCNT(8);
                WUSH_LDS_BARRIER();
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        WUSH_WAIT_VMCNT(0);
    }

    const int half = lane >> 5;
    const int l32 = lane & 31;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int cl = (rbb + j) * 32 + l32;
        const int col = n0 + cl;
        const int e_col = sh_e[256 + cl];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int rl = (rba + i) * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                const int row = m0 + rl;
                const int e_row = sh_e[rl];
                float v = __builtin_ldexpf(acc[i][j][q], -(e_row + e_col));
                if (e_row == kH16NonFinite || e_col == kH16NonFinite) v = __builtin_nanf("");
                if (row < M && col < N) {
                    if (partial != nullptr)
                        partial[((size_t)blockIdx.z * M + row) * N + col] = v;
                    else
                        y[(size_t)row * N + col] = f32_to_f16_bits(v);
                }
            }
        }
    }
}

}  // namespace

size_t gemm_h16_smem_bytes() { return 2 * kH16Buf + 2 * kH16Tile * sizeof(int); }

int gemm_h16_init_device() {
    // the workgroup's LDS is above the default 64 KiB limit of dynamic LDS
    const int smem = (int)gemm_h16_smem_bytes();
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_h16w8_kernel<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_h16w8_kernel<false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, smem);
    return (int)e;
}

size_t gemm_h16a_workspace_bytes(int64_t M, int64_t K, int splits) {
    const int64_t mpad = (M + kH16Tile - 1) / kH16Tile * kH16Tile;
    return (size_t)mpad * (size_t)K * 2 + (size_t)splits * (size_t)mpad * sizeof(int);
}

int launch_gemm_h16a(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                     uint16_t* y, float* partial, int M, int N, int K, int splits, int groups_per_split,
                     void* a_ws, hipStream_t stream) {
    const int G = K >> 5;
    if (M <= 0 || N <= 0 || K <= 0 || K % 256 != 0 || splits < 1 || groups_per_split <= 0 ||
        groups_per_split % 8 != 0 || (long long)splits * groups_per_split < G ||
        (long long)(splits - 1) * groups_per_split >= G || (splits > 1 && partial == nullptr) || a_ws == nullptr ||
        ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(ws) | reinterpret_cast<uintptr_t>(a_ws)) &
         15u) != 0)
        return (int)hipErrorInvalidValue;
    const int mpad = (M + kH16Tile - 1) / kH16Tile * kH16Tile;
    uint8_t* a16 = static_cast<uint8_t*>(a_ws);
    int* ea = reinterpret_cast<int*>(a16 + (size_t)mpad * K * 2);
    h16_prep_a_kernel<<<dim3((unsigned)(mpad / 32), (unsigned)splits), 256, 0, stream>>>(xq, xs, a16, ea, M, K,
                                                                                     groups_per_split);
    dim3 grid((unsigned)((N + kH16Tile - 1) / kH16Tile), (unsigned)(mpad / kH16Tile), (unsigned)splits);
    gemm_h16a_kernel<<<grid, 512, 0, stream>>>(a16, ea, wq, ws, y, partial, M, N, K, groups_per_split);
    return (int)hipGetLastError();
}

int launch_gemm_h16(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                    uint16_t* y, float* partial, int M, int N, int K, int splits, int groups_per_split,
                    hipStream_t stream) {
    const int G = K >> 5;
    // every K slice holds a positive multiple of 8 groups
    if (M <= 0 || N <= 0 || K <= 0 || K % 256 != 0 || splits < 1 || groups_per_split <= 0 ||
        groups_per_split % 8 != 0 || (long long)splits * groups_per_split < G ||
        (long long)(splits - 1) * groups_per_split >= G || (splits > 1 && partial == nullptr))
        return (int)hipErrorInvalidValue;
    int dev = 0;
    const int st = device_setup(&dev);
    if (st != 0) return st;
    const bool vec = G % 8 == 0 && ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(ws)) & 15u) == 0;
    dim3 grid((unsigned)((N + kH16Tile - 1) / kH16Tile), (unsigned)((M + kH16Tile - 1) / kH16Tile), (unsigned)splits);
    const size_t smem = gemm_h16_smem_bytes();
    if (vec)
        gemm_h16w8_kernel<true><<<grid, 512, smem, stream>>>(xq, xs, wq, ws, y, partial, M, N, K, groups_per_split);
    else
        gemm_h16w8_kernel<false><<<grid, 512, smem, stream>>>(xq, xs, wq, ws, y, partial, M, N, K, groups_per_split);
    return (int)hipGetLastError();
}

}  // namespace wush
