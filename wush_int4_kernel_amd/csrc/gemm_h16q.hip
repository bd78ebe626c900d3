// gemm_h16q.hip -- the pre-converted-activation fp16-MFMA prefill GEMM with
// one wavefront per SIMD (csrc/gemm_s4.cu:85-379 is the reference contract;
// operands and numerics as in gemm_h16.hip).
//
// Workgroup: 4 wavefronts side by side, a 256 x 256 output tile, wavefront w
// owning all 256 rows and weight columns 64w .. 64w + 63 (8 x 2 accumulator
// blocks, 256 fp32 accumulators in AGPRs).  Because no other wavefront needs
// its columns, a wavefront converts its weight codes straight into MFMA
// B-operand registers: no LDS traffic for converted weights, no transpose.
// The activations, converted once beforehand in the matching layout
// (h16_prep_a_kernel<true>), are DMA'd into a 4-slot LDS ring four stages
// ahead and read by all four wavefronts.
//
// With one wavefront per SIMD there is no second wavefront to run the memory
// work beside the MFMAs, so every wavefront runs a software pipeline of its
// own, issued between its 32 MFMAs of stage t: stage t+1's activation
// fragments, the conversion of stage t+1's weights, the DMAs of stage t+4.
// One barrier per stage.  A wavefront's weight codes come in batches of four
// stages, DMA'd into LDS two batches ahead and read into registers once per
// batch (6 LDS reads per 4 stages, not 4 per stage: 4% faster at L70).  The
// codes are DMA'd two batches at a time, each column's whole 128-byte line
// per 8 lanes: with 32 bytes of 32 columns per DMA the kernel took 2-4%
// longer (a load touching 32 lines costs the vector memory path about as much
// as one reading them whole).
//
// Every global load of the kernel is an LDS DMA issued by an asm statement
// (activations, weight codes and scales, shifts), and the kernel orders them
// itself: at the end of stage t a wavefront waits until its DMAs of stage
// t+2 (and so everything it issued before them) have landed, then the barrier
// publishes them.  Left to the compiler, LDS DMA is tracked per LDS object in
// a small table; once the table overflows, every LDS read waits for all DMAs
// in flight, and register loads mixed with such DMAs get waits counted
// without them.
//
// Outputs: fp16 through LDS (the ring is free after the last stage), so that
// the global stores are 16-byte row chunks instead of one 2-byte store per
// accumulator.
//
// Stage layout (h16_prep_a_kernel<true>): in each block of 4 groups a lane of
// half h reads the 32 contiguous code bytes [32h, 32h + 32) of its column
// (groups 2h and 2h + 1); stage s of the block takes dwords 2s and 2s + 1 of
// them (K16 slices 0 and 1).
#include "gemm_h16_device.h"
#include "gemm_h16.h"
#include "setup.h"

namespace wush {
namespace {

#ifndef WUSH_H16Q_SCHED
#define WUSH_H16Q_SCHED 1                        // explicit MFMA / LDS / VALU interleave
#endif

// Tile id -> (row tile, column tile): workgroup i runs on XCD i % 8.  Each
// XCD walks its column tiles in groups of 8, all row tiles of a group before
// the next, so the workgroups in flight on an XCD share 8 weight column
// tiles and a few activation row tiles in its L2.
__device__ __forceinline__ void h16q_tile(uint32_t id, uint32_t NC, uint32_t NR, int& tm, int& tn) {
    if ((NC & 7) != 0) {
        tm = (int)(id / NC);
        tn = (int)(id % NC);
        return;
    }
    constexpr uint32_t kGroup = 8;
    const uint32_t q = id >> 3, x = id & 7;
    const uint32_t gsize = kGroup * NR;
    const uint32_t g = q / gsize, w = q % gsize;
    const uint32_t width = min(kGroup, (NC >> 3) - g * kGroup);
    tm = (int)(w / width);
    tn = (int)((g * kGroup + w % width) * 8 + x);
}

// RB: 32-row blocks per wavefront, 8 (256-row tiles) or 4 (128-row tiles, for
// 64 < M <= 128: half the accumulators, the same weight conversion per stage).
template <int RB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_h16q_kernel(const uint8_t* __restrict__ a16, const int* __restrict__ ea, const int* __restrict__ eb,
                      const uint8_t* __restrict__ wq, const uint16_t* __restrict__ ws, uint16_t* __restrict__ y,
                      float* __restrict__ partial, int M, int N, int K, int groups_per_split, int splits) {
    // activation ring (4 stages) and, per wavefront, two double batches of
    // weight codes [64 columns][128 B, pieces swizzled] and two batches of
    // scales [2 columns][64 lanes][4 B]
    __shared__ __align__(16) uint8_t sA[4][kH16Op];
    __shared__ __align__(16) uint8_t sBc[2][4][8192];
    __shared__ __align__(16) uint32_t sBs[2][4][128];
    __shared__ __align__(16) int sh_e[512];      // [0, 256) rows, [256, 512) columns

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int GR = K >> 5;
    const int K2 = K >> 1;
    const int limn = N - 1;
    constexpr int TR = 32 * RB;                  // rows per tile
    constexpr int NA = RB / 4;                   // activation row blocks DMA'd per wavefront
    constexpr int kSlice = RB * 1024;            // bytes of one K16 slice of a stage's activations
    const int NC = (N + kH16Tile - 1) / kH16Tile;
    const int NR = (M + TR - 1) / TR;
    // shifts and converted activations are laid out over 256-row padding
    const int mpad = (M + kH16Tile - 1) / kH16Tile * kH16Tile, npad = NC * kH16Tile;
    const int per_slice = NC * NR;

    const int id = blockIdx.x;
    const int slice = id / per_slice;
    int tm, tn;
    h16q_tile((uint32_t)(id - slice * per_slice), (uint32_t)NC, (uint32_t)NR, tm, tn);
    const int m0 = tm * TR;
    const int n0 = tn * kH16Tile;
    const int gb = slice * groups_per_split;
    const int G = min(GR - gb, groups_per_split);

    // activation DMA of this wavefront: row blocks NA w .. NA w + NA - 1, both K16 slices
    const uint8_t* asrc = a16 + ((size_t)((m0 >> 5) + NA * wave) * GR + gb) * 2048 + lane * 16;
    const size_t arb = (size_t)GR * 2048;
    auto issue_a = [&](int st, int slot) {
        const uint8_t* src = asrc + (size_t)min(st, G - 1) * 2048;   // past the slice: the last stage
        const uint32_t dst = lds_addr(sA[slot]) + NA * wave * 1024;
#pragma unroll
        for (int b = 0; b < NA; ++b) {
            dma16(src + b * arb, dst + b * 1024);
            dma16(src + b * arb + 1024, dst + kSlice + b * 1024);
        }
    };
    // this lane's two weight columns (blocks 2w and 2w + 1): their scales
    const int colA = min(n0 + wave * 64 + l32, limn);
    const int colB = min(n0 + wave * 64 + 32 + l32, limn);
    const uint16_t* sa = ws + (size_t)colA * GR + gb + 2 * half;
    const uint16_t* sb = ws + (size_t)colB * GR + gb + 2 * half;
    // Weight codes come in double batches (8 groups, each column's whole
    // 128-byte line): DMA k of a double batch reads columns 8k .. 8k+7 of the
    // wavefront's 64, 8 lanes a line.  Lane l fetches piece (l % 8) ^ f(c) of
    // column c = 8k + l / 8, so that piece p of column c sits at
    // 128 c + 16 (p ^ f(c)) with f(c) = (c / 2) % 8: 16 consecutive readers
    // (columns c .. c+15, one piece) hit distinct banks.
    const uint32_t cbase = (uint32_t)(n0 + wave * 64);
    auto issue_db = [&](int d, int buf) {
        const int o = min(d * 2 * kH16Batch, G - 2 * kH16Batch);
        const uint8_t* base = wq + (size_t)(gb + o) * 16;
        const uint32_t c0 = lds_addr(sBc[buf][wave]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int c = 8 * k + (lane >> 3);
            const int p = (lane & 7) ^ ((c >> 1) & 7);
            const uint32_t col = min(cbase + (uint32_t)c, (uint32_t)limn);
            dma16(base + (size_t)col * K2 + p * 16, c0 + 1024 * k);
        }
    };
    auto issue_s = [&](int b, int buf) {
        const int o = min(b * kH16Batch, G - kH16Batch);
        const uint32_t s = lds_addr(sBs[buf][wave]);
        dma4(sa + o, s);
        dma4(sb + o, s + 256);
    };
    v16f acc[RB][2];
    h8 fa[2][2][RB];                             // [register set][K16 slice][row block]
    h8 fb[2][2][2];                              // [register set][K16 slice][column block]
    auto read_frag = [&](int slot, int P, int kk, int i) {
        fa[P][kk][i] = frag_read(sA[slot] + kk * kSlice + i * 1024, lane);
    };
    int eA = 0, eB = 0;
    // A weight batch in registers, read from its LDS buffer once: this
    // lane's 32 code bytes of each of its two columns, and their scales
    // (two bf16 per column: groups 2h and 2h + 1 of the batch's block).
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    struct Batch {
        u32x4 c[2][2];                           // [column block][16-byte half]
        uint32_t s[2];
    };
    // batch b: double batch b / 2 in code buffer (b / 2) & 1, its half b & 1;
    // scales in buffer b & 1
    const int fsw = (l32 >> 1) & 7;                // f(c) of both the lane's columns
    auto read_batch = [&](int b, Batch& r) {
        const uint8_t* cb = sBc[(b >> 1) & 1][wave];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int c = (k >> 1) * 32 + l32;       // column block A, then B
            const int p = 4 * (b & 1) + 2 * half + (k & 1);
            r.c[k >> 1][k & 1] = *reinterpret_cast<const u32x4*>(cb + c * 128 + 16 * (p ^ fsw));
        }
        r.s[0] = sBs[b & 1][wave][lane];
        r.s[1] = sBs[b & 1][wave][64 + lane];
    };
    // stage s (0-3) of a batch, column block jb -> B operands of register set P
    auto convert_b = [&](int P, const Batch& r, int s, int jb) {
        const uint32_t sv = r.s[jb];
        const float f = __uint_as_float((s & 2) ? (sv & 0xffff0000u) : (sv << 16));
        const h2 sc = h16_scale(f, jb ? eB : eA);
        const u32x4& c = r.c[jb][s >> 1];
        fb[P][0][jb] = __builtin_bit_cast(h8, h16_codes((s & 1) ? c[2] : c[0], sc));
        fb[P][1][jb] = __builtin_bit_cast(h8, h16_codes((s & 1) ? c[3] : c[1], sc));
    };
    Batch R0, R1;                                // batches in LDS buffers 0 and 1

    // Prologue: shifts, activation stages 0-3, weight batches 0 and 1.
    if (64 * wave < TR)                          // the tile's rows, padded rows included
        dma4(ea + (size_t)slice * mpad + m0 + wave * 64 + lane, lds_addr(sh_e + wave * 64));
    dma4(eb + (size_t)slice * npad + n0 + wave * 64 + lane, lds_addr(sh_e + 256 + wave * 64));
    issue_a(0, 0);
    issue_a(1, 1);
    issue_a(2, 2);
    issue_a(3, 3);
    issue_db(0, 0);
    issue_s(0, 0);
    issue_s(1, 1);
    WUSH_WAIT_VMCNT(2);                          // all but batch 1's scales
    WUSH_LDS_BARRIER();
    eA = sh_e[256 + wave * 64 + l32];
    eB = sh_e[256 + wave * 64 + 32 + l32];
    read_batch(0, R0);
    convert_b(0, R0, 0, 0);
    convert_b(0, R0, 0, 1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int i = 0; i < RB; ++i) read_frag(0, 0, kk, i);
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){0.0f};
    __builtin_amdgcn_sched_barrier(0);

    for (int s0 = 0; s0 < G; s0 += 2 * kH16Batch) {
        // fully unrolled: the batch registers and register sets are picked by j
#pragma clang loop unroll(full)
        for (int j = 0; j < 2 * kH16Batch; ++j) {
            const int t = s0 + j;
            const int P = j & 1;
            issue_a(t + 4, j & 3);               // into the slot stage t left
            // a batch buffer's next batch once its last stage is converted
            // double batch s0 / 8 + 1 once batch s0 / 4 - 1 (its buffer's
            // last) is in registers; batch scales as before
            if (j == 3) {
                issue_db(s0 / (2 * kH16Batch) + 1, (s0 / (2 * kH16Batch) + 1) & 1);
                issue_s(s0 / kH16Batch + 2, 0);
            }
            if (j == 7) issue_s(s0 / kH16Batch + 3, 1);
            // stage t + 1's weights: batch (t + 1) / 4, in LDS buffer
            // ((t + 1) / 4) & 1, stage (j + 1) % 4 of it.  A batch goes into
            // registers at the stage before its first, ahead of that stage's
            // fragment reads (LDS returns in order: read late, the
            // conversion would wait for all of them).
            if (j == 3) read_batch(s0 / kH16Batch + 1, R1);
            if (j == 7) read_batch(s0 / kH16Batch + 2, R0);
            const Batch& Rc = (j < 3 || j == 7) ? R0 : R1;
            const int sc = (j + 1) & 3;
            // 32 MFMAs of stage t; between them stage t+1's 16 activation
            // fragment reads (past the last stage they read a stale slot,
            // unused) and its weight conversions
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
                for (int i = 0; i < RB; ++i) {
#pragma unroll
                    for (int jb = 0; jb < 2; ++jb) {
                        acc[i][jb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[P][kk][i], fb[P][kk][jb],
                                                                            acc[i][jb], 0, 0, 0);
                        const int m = kk * 2 * RB + i * 2 + jb;   // MFMA index in the stage
                        if (m < 2 * RB) read_frag((j + 1) & 3, P ^ 1, m / RB, m % RB);
                        if (m == 2 * RB) convert_b(P ^ 1, Rc, sc, 0);
                        if (m == 3 * RB) convert_b(P ^ 1, Rc, sc, 1);
                    }
                }
            }
#if WUSH_H16Q_SCHED
            // a batch's reads, then per MFMA one activation fragment read over
            // the first 16; the conversion VALU spread over all
#pragma unroll
            for (int m = 0; m < 4 * RB; ++m) {
                if (m == 0 && (j == 3 || j == 7)) __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);   // DS read: batch
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                if (m < 2 * RB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read: activations
                if (m < 2 * RB) __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
                else __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
#endif
            // activation stage t + 2 landed: the DMAs issued after its 4 are
            // stage t+3's and t+4's (8) plus the batches of stages t-2 .. t
            // (issued after their stage's activations); at the first stages
            // the count also covers the prologue's DMAs
            // (10 weight DMAs at j = 3, 2 at j = 7)
            const int nb = (j >= 3 && j <= 5) ? 10 : (j == 7 || j <= 1) ? 2 : 0;
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (NA == 2) {
                if (nb == 0) WUSH_WAIT_VMCNT(8);
                else if (nb == 2) WUSH_WAIT_VMCNT(10);
                else WUSH_WAIT_VMCNT(18);
            } else {
                static_assert(NA == 1, "activation DMAs per stage: 2 * NA");
                if (nb == 0) WUSH_WAIT_VMCNT(4);
                else if (nb == 2) WUSH_WAIT_VMCNT(6);
                else WUSH_WAIT_VMCNT(14);
            }
            WUSH_LDS_BARRIER();
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // The stages past the slice DMA'd copies of its last stage into the ring
    WUSH_WAIT_VMCNT(0);
    __syncthreads();                             // the ring is free

    const int ecA = sh_e[256 + wave * 64 + l32];
    const int ecB = sh_e[256 + wave * 64 + 32 + l32];
    auto out_value = [&](int i, int jb, int q, int e_row) {
        const int e_col = jb ? ecB : ecA;
        float v = __builtin_ldexpf(acc[i][jb][q], -(e_row + e_col));
        if (e_row == kH16NonFinite || e_col == kH16NonFinite) v = __builtin_nanf("");
        return v;
    };
    if (partial != nullptr) {
        // fp32 partials of a K slice: one store per accumulator
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            const int col = n0 + wave * 64 + jb * 32 + l32;
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int rl = i * 32 + 8 * (q >> 2) + 4 * half + (q & 3);
                    const int row = m0 + rl;
                    const float v = out_value(i, jb, q, sh_e[rl]);
                    if (row < M && col < N) partial[((size_t)slice * M + row) * N + col] = v;
                }
        }
        return;
    }
    // fp16: each wavefront's 256 x 64 outputs through its ring slot (16 KiB),
    // 128 rows at a time: 2-byte LDS writes in the accumulator layout, then
    // 16-byte reads and stores of 8 columns of a row
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    uint8_t* stg = sA[wave];
    uint8_t* wbase = stg + 4 * half * 128 + l32 * 2;                 // row 4 * half, column l32
    const uint8_t* rbase = stg + (lane >> 3) * 128 + (lane & 7) * 16;
    const int* erow = sh_e + 4 * half;
#pragma unroll
    for (int pass = 0; pass < RB / 4; ++pass) {
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const int i = 4 * pass + i4;
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const int4 er4 = *reinterpret_cast<const int4*>(erow + 32 * i + 8 * q4);
                const int e_r[4] = {er4.x, er4.y, er4.z, er4.w};
#pragma unroll
                for (int jb = 0; jb < 2; ++jb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint16_t h = f32_to_f16_bits(out_value(i, jb, 4 * q4 + r, e_r[r]));
                        *reinterpret_cast<uint16_t*>(wbase + (32 * i4 + 8 * q4 + r) * 128 + 64 * jb) = h;
                    }
            }
            __builtin_amdgcn_sched_barrier(0);   // one row block at a time
        }
        const int row0 = m0 + 128 * pass + (lane >> 3);
        const int col = n0 + wave * 64 + (lane & 7) * 8;
        uint16_t* dst0 = y + (size_t)row0 * N + col;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint4 v = *reinterpret_cast<const uint4*>(rbase + k * 1024);
            if (row0 + 8 * k < M) {
                uint16_t* dst = dst0 + (size_t)(8 * k) * N;
                if (vec && col + 8 <= N) {
                    *reinterpret_cast<uint4*>(dst) = v;
                } else {
                    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (col + e < N) dst[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

}  // namespace

int launch_gemm_h16q(const uint8_t* a16, const int* ea, const int* eb, const uint8_t* wq, const uint16_t* ws,
                     uint16_t* y, float* partial, int M, int N, int K, int groups_per_split, int splits,
                     bool rows128, hipStream_t stream) {
    const int tr = rows128 ? 128 : 256;
    const long long tiles = (long long)((N + kH16Tile - 1) / kH16Tile) * ((M + tr - 1) / tr) * splits;
    if (rows128) {
        gemm_h16q_kernel<4><<<dim3((unsigned)tiles), 256, 0, stream>>>(a16, ea, eb, wq, ws, y, partial, M, N, K,
                                                                        groups_per_split, splits);
        return (int)hipGetLastError();
    }
    gemm_h16q_kernel<8><<<dim3((unsigned)tiles), 256, 0, stream>>>(a16, ea, eb, wq, ws, y, partial, M, N, K,
                                                                 groups_per_split, splits);
    return (int)hipGetLastError();
}

}  // namespace wush
