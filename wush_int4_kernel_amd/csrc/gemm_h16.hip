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
// 2^-29 of its row's largest converts exactly (its lowest significand bit
// stays at or above fp16's 2^-24); smaller ones keep fewer bits (an absolute
// error below 2^-37 of the row's largest scale per scale operand).  A row or column with a non-finite scale
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
#include "gemm_h16_device.h"
#include "gemm_h16.h"
#include "setup.h"

namespace wush {
namespace {

#ifndef WUSH_H16_XCD
#define WUSH_H16_XCD 1                           // XCD-aware tile order in the 8-wavefront kernel
#endif

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
        const h2 sc = h16_scale(h16_batch_scale<VEC>(rr.s, i), e);
        const uint32_t w4[4] = {rr.c[i].x, rr.c[i].y, rr.c[i].z, rr.c[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            frag_write(dst + (j >> 1) * kH16Slice, (r & 31) + 32 * (j & 1), h16_codes(w4[j], sc));
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
// again by each of the N/256 column tiles.  The workspace route converts the
// activations once (h16_prep_a_kernel, M x K x 2 bytes of workspace), in the
// MFMA fragment layout that gemm_h16q_kernel (gemm_h16q.hip) DMAs into LDS.
// Same fp16 operands as gemm_h16w8_kernel; the K order within a block of four
// groups differs (below), so the fp32 sums agree to rounding, not bit for bit.
//
// a16 layout: [32-row block][stage][K16 slice][64 lanes][16 B] (one block
// and stage: the two 1 KiB operand fragments of v_mfma_f32_32x32x16_f16).
// Within each block of 4 groups, stage 2 * (q & 1) + d / 2 of the block takes
// dword d of group q at K16 slice d & 1 in lane half q >> 1 -- every stage
// holds 32 codes of two groups, so that a wavefront converting a weight
// column reads 32 contiguous bytes per half-wavefront for 4 stages.
// ea[slice][row] = the row's power-of-two shift over the K slice, as the
// per-tile conversion computes it.  Workgroups past mpad / 32 compute every
// weight column's shift per slice, eb[slice][column] (npad columns, 0 past
// N), once, instead of every 256 x 256 tile re-reading its columns' scales.
// Grid: (mpad / 32 + npad / 256, splits): a workgroup converts 32 rows, or
// takes 256 columns, of one slice.
__global__ __launch_bounds__(256) void h16_prep_a_kernel(const uint8_t* __restrict__ xq,
                                                         const uint16_t* __restrict__ xs,
                                                         uint8_t* __restrict__ a16, int* __restrict__ ea,
                                                         const uint16_t* __restrict__ ws, int* __restrict__ eb,
                                                         int M, int N, int K, int groups_per_split, int mpad) {
    const int G = K >> 5;
    const int rb = blockIdx.x;
    const int slice = blockIdx.y;
    const int sg0 = slice * groups_per_split, sg1 = min(G, sg0 + groups_per_split);
    const int tid = threadIdx.x;
    if (rb >= mpad / 32) {
        // weight column shifts: thread t, column 256 * (rb - mpad / 32) + t
        const int npad = (N + kH16Tile - 1) / kH16Tile * kH16Tile;
        const int c = (rb - mpad / 32) * 256 + tid;
        int e = 0;
        if (c < N) {
            uint32_t mx, mx2;
            const uint16_t* ps = ws + (size_t)c * G + sg0;
            h16_row_max<true>(ps, ps, sg1 - sg0, mx, mx2);
            e = h16_shift(mx);
        }
        eb[(size_t)slice * npad + c] = e;
        return;
    }
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
        const h2 sc = h16_scale(f, e);
        const int q = g & 3;
        const int st = (g & ~3) + 2 * (q & 1);                // stage of dwords 0, 1 (2, 3: st + 1)
        uint8_t* dst = a16 + ((size_t)rb * G + st) * 2048;
        const int L = rr + 32 * (q >> 1);
        frag_write(dst, L, h16_codes(w.x, sc));
        frag_write(dst + 1024, L, h16_codes(w.y, sc));
        frag_write(dst + 2048, L, h16_codes(w.z, sc));
        frag_write(dst + 3072, L, h16_codes(w.w, sc));
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

size_t gemm_h16a_workspace_bytes(int64_t M, int64_t N, int64_t K, int splits) {
    const int64_t mpad = (M + kH16Tile - 1) / kH16Tile * kH16Tile;
    const int64_t npad = (N + kH16Tile - 1) / kH16Tile * kH16Tile;
    return (size_t)mpad * (size_t)K * 2 + (size_t)splits * (size_t)(mpad + npad) * sizeof(int);
}

int launch_gemm_h16a(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                     uint16_t* y, float* partial, int M, int N, int K, int splits, int groups_per_split,
                     void* a_ws, bool rows128, hipStream_t stream) {
    const int G = K >> 5;
    if (M <= 0 || N <= 0 || K <= 0 || K % 256 != 0 || splits < 1 || groups_per_split <= 0 ||
        groups_per_split % 8 != 0 || (long long)splits * groups_per_split < G ||
        (long long)(splits - 1) * groups_per_split >= G || (splits > 1 && partial == nullptr) || a_ws == nullptr ||
        ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(ws) | reinterpret_cast<uintptr_t>(a_ws)) &
         15u) != 0)
        return (int)hipErrorInvalidValue;
    const int mpad = (M + kH16Tile - 1) / kH16Tile * kH16Tile;
    const int npad = (N + kH16Tile - 1) / kH16Tile * kH16Tile;
    uint8_t* a16 = static_cast<uint8_t*>(a_ws);
    int* ea = reinterpret_cast<int*>(a16 + (size_t)mpad * K * 2);
    int* eb = ea + (size_t)splits * mpad;
    h16_prep_a_kernel<<<dim3((unsigned)(mpad / 32 + npad / 256), (unsigned)splits), 256, 0, stream>>>(
        xq, xs, a16, ea, ws, eb, M, N, K, groups_per_split, mpad);
    const int e = (int)hipGetLastError();
    if (e != 0) return e;
    return launch_gemm_h16q(a16, ea, eb, wq, ws, y, partial, M, N, K, groups_per_split, splits, rows128, stream);
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
