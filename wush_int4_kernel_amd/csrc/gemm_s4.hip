// gemm_s4.hip -- group-scaled W4A4 GEMM on CDNA4 int8 MFMA
// (csrc/gemm_s4.cu:85-379 is the reference contract).
//
//   y[m][n] = sum_g sx[m][g] * sw[n][g] * D[m][n][g],
//   D[m][n][g] = sum_{k in g} qx[m][k] * qw[n][k]   (exact int32)
//
// One 32-wide quantization group is exactly one K step of
// v_mfma_i32_32x32x32_i8, so every MFMA produces D of one group for a 32x32
// block, exact in int32.  The s4 codes are unpacked to int8 in VGPRs as
// 16*code ((w<<4)&0xF0F0F0F0 and w&0xF0F0F0F0, exact for [-8,7]) so the MFMA
// returns 256*D.  D is folded into an fp32 accumulator with the product of the
// two bf16 group scales: acc = fma(float(D), 2*sx*sw, acc).  The scale
// products come from a second MFMA, v_mfma_f32_32x32x16_bf16, whose operands
// hold only the lane's own scale in element 0: both lane halves contribute the
// same exact bf16 x bf16 product (8-bit x 8-bit significands), so the MFMA
// returns 2*sx*sw exactly, already in the accumulator layout of D.  The
// factor 2*256 is removed once at the output (exact power of two), so the
// result equals the per-element fold fma(float(D), sx*sw, acc) / 256.
//
// Workgroup = 4 wavefronts in a WAVES_M x WAVES_N grid, each wavefront owns a
// (32*BM) x (32*BN) output tile.  K advances 4 groups (64 code bytes per row)
// per stage through a double-buffered LDS tile laid out fragment-major,
// [group][k-half][row][8 B], so the MFMA operand reads (lane = row, 8 B) are
// conflict-free.  Skinny M uses split-K: each K slice writes fp32 partials to
// a caller-provided workspace and a second kernel sums the slices in a fixed
// order (deterministic, graph-capturable, no atomics, no memset).
#include "wush_device.h"
#include "gemm_h16.h"
#include "setup.h"
#include "../../include/wush_int4.h"

namespace wush {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Fold factor of every D element, 2*sx[row]*sw[col], for one 32x32 block in
// the 32x32 MFMA accumulator layout.  sx_bits / sw_bits: bf16 bits (upper 16
// bits zero) of the scale of row l%32 / column l%32.  Element 0 of the two
// operands sits at a distinct k in each lane half and every other element is
// zero, so the MFMA sums exactly two equal exact products.
__device__ __forceinline__ v16f scale_products(uint32_t sx_bits, uint32_t sw_bits) {
    const v4i a = {(int)sx_bits, 0, 0, 0};
    const v4i b = {(int)sw_bits, 0, 0, 0};
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   (v16f){0.0f}, 0, 0, 0);
}

// fp32 accumulator -> output: removes the 16*16 of the unpacked codes and the
// 2 of scale_products.
constexpr float kFoldOutScale = 1.0f / 512.0f;

constexpr int kPlanePad = 32;                    // bytes of padding per (group, half) plane

// LDS layout of one pipeline buffer: codes fragment-major
// [group][k-half][row][8 B] (+ padding per plane) so the MFMA operand reads
// (lane = row, 8 B) are conflict-free, then bf16 scales [group][row].
template <int TM, int TN, int SG>
struct GemmSmem {
    static constexpr int kAPlane = TM * 8 + kPlanePad;
    static constexpr int kBPlane = TN * 8 + kPlanePad;
    static constexpr int kACodes = SG * 2 * kAPlane;
    static constexpr int kBCodes = SG * 2 * kBPlane;
    static constexpr int kAScale = SG * TM * 2;
    static constexpr int kBScale = SG * TN * 2;
    static constexpr int kBuf = kACodes + kBCodes + kAScale + kBScale;
    static constexpr int kBytes = 2 * kBuf;
};

// Global -> register prefetch of one stage, spread over the 256 threads.
// Chunk id -> (row = id / SG, group = id % SG): SG consecutive threads read
// one row's SG*16 contiguous code bytes, so with SG = 8 every wavefront load
// instruction reads eight whole 128-byte lines.
template <int TM, int TN, int SG>
struct StageRegs {
    static constexpr int kAChunks = (TM * SG + 255) / 256;
    static constexpr int kBChunks = (TN * SG + 255) / 256;
    uint4 a[kAChunks];
    uint4 b[kBChunks];
    uint16_t sa[kAChunks];
    uint16_t sb[kBChunks];
};

// BM x BN 32x32 blocks per wavefront, WAVES_M x WAVES_N wavefronts, SG groups
// per stage, MR = rows of each 32-row block that can hold output (the fold is
// skipped for accumulator registers of rows >= MR: at decode M <= 8 only a
// quarter of the MFMA rows are real).
template <int BM, int BN, int WAVES_M, int WAVES_N, int SG, int MR, bool PER_TENSOR>
__global__ __launch_bounds__(256) void gemm_s4_kernel(const uint8_t* __restrict__ xq,
                                                      const uint16_t* __restrict__ xs,
                                                      const uint8_t* __restrict__ wq,
                                                      const uint16_t* __restrict__ ws,
                                                      uint16_t* __restrict__ y,
                                                      float* __restrict__ partial,
                                                      int M, int N, int K, int groups_per_split,
                                                      float alpha, const float* __restrict__ alpha_dev) {
    static_assert(WAVES_M * WAVES_N == 4, "4 wavefronts per workgroup");
    static_assert(MR % 8 == 0 && MR <= 32, "fold rows");
    constexpr int TM = 32 * BM * WAVES_M;
    constexpr int TN = 32 * BN * WAVES_N;
    constexpr int NR = MR / 2;
    using S = GemmSmem<TM, TN, SG>;
    using R = StageRegs<TM, TN, SG>;
    extern __shared__ __align__(16) uint8_t smem[];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int half = lane >> 5;                  // k-half of the MFMA operand
    const int l32 = lane & 31;
    const int wm = (wave / WAVES_N) * (32 * BM);
    const int wn = (wave % WAVES_N) * (32 * BN);
    const int m0 = blockIdx.y * TM;
    const int n0 = blockIdx.x * TN;

    const int G = K >> 5;
    const int K2 = K >> 1;
    const int g_begin = blockIdx.z * groups_per_split;
    const int g_end = min(G, g_begin + groups_per_split);
    const int n_stages = (g_end - g_begin + SG - 1) / SG;

    auto load_stage = [&](int st, R& r) {
        const int gs = g_begin + st * SG;
#pragma unroll
        for (int c = 0; c < R::kAChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id / SG, g = id % SG;
            const int gm = m0 + row, gg = gs + g;
            const bool ok = row < TM && gm < M && gg < g_end;
            r.a[c] = ok ? *reinterpret_cast<const uint4*>(xq + (size_t)gm * K2 + (size_t)gg * 16)
                        : make_uint4(0, 0, 0, 0);
            if constexpr (!PER_TENSOR) r.sa[c] = ok ? xs[(size_t)gm * G + gg] : (uint16_t)0;
        }
#pragma unroll
        for (int c = 0; c < R::kBChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id / SG, g = id % SG;
            const int gn = n0 + row, gg = gs + g;
            const bool ok = row < TN && gn < N && gg < g_end;
            r.b[c] = ok ? *reinterpret_cast<const uint4*>(wq + (size_t)gn * K2 + (size_t)gg * 16)
                        : make_uint4(0, 0, 0, 0);
            if constexpr (!PER_TENSOR) r.sb[c] = ok ? ws[(size_t)gn * G + gg] : (uint16_t)0;
        }
    };

    auto store_stage = [&](int buf, const R& r) {
        uint8_t* base = smem + buf * S::kBuf;
        uint8_t* bbase = base + S::kACodes;
        uint16_t* sa = reinterpret_cast<uint16_t*>(base + S::kACodes + S::kBCodes);
        uint16_t* sbp = sa + SG * TM;
#pragma unroll
        for (int c = 0; c < R::kAChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id / SG, g = id % SG;
            if (row < TM) {
                *reinterpret_cast<uint2*>(base + (g * 2 + 0) * S::kAPlane + row * 8) = make_uint2(r.a[c].x, r.a[c].y);
                *reinterpret_cast<uint2*>(base + (g * 2 + 1) * S::kAPlane + row * 8) = make_uint2(r.a[c].z, r.a[c].w);
                if constexpr (!PER_TENSOR) sa[row * SG + g] = r.sa[c];
            }
        }
#pragma unroll
        for (int c = 0; c < R::kBChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id / SG, g = id % SG;
            if (row < TN) {
                *reinterpret_cast<uint2*>(bbase + (g * 2 + 0) * S::kBPlane + row * 8) = make_uint2(r.b[c].x, r.b[c].y);
                *reinterpret_cast<uint2*>(bbase + (g * 2 + 1) * S::kBPlane + row * 8) = make_uint2(r.b[c].z, r.b[c].w);
                if constexpr (!PER_TENSOR) sbp[row * SG + g] = r.sb[c];
            }
        }
    };

    // Accumulators: fp32 (group-scaled) or int32 (per-tensor, whole K).
    float acc[BM][BN][NR];
    v16i iacc[BM][BN];
#pragma unroll
    for (int bm = 0; bm < BM; ++bm)
#pragma unroll
        for (int bn = 0; bn < BN; ++bn) {
#pragma unroll
            for (int j = 0; j < NR; ++j) acc[bm][bn][j] = 0.0f;
            iacc[bm][bn] = (v16i){0};
        }

    // weight-scale operands of the fold factors: quad [bn][p] carries scale
    // dword p (groups 2p, 2p+1), its other dwords stay zero
    v4i fbq[BN][SG / 2 > 0 ? SG / 2 : 1];
#pragma unroll
    for (int bn = 0; bn < BN; ++bn)
#pragma unroll
        for (int p = 0; p < (SG / 2 > 0 ? SG / 2 : 1); ++p) fbq[bn][p] = (v4i){0, 0, 0, 0};

    auto compute_stage = [&](int buf, int st) {
        const uint8_t* base = smem + buf * S::kBuf;
        const uint8_t* bbase = base + S::kACodes;
        const uint16_t* sa = reinterpret_cast<const uint16_t*>(base + S::kACodes + S::kBCodes);
        const uint16_t* sbp = sa + SG * TM;
        const int groups_here = min(SG, g_end - (g_begin + st * SG));
        // per-stage scale operands (group-scaled fold only): the SG bf16
        // scales of this lane's activation row / weight column
        static_assert(PER_TENSOR || SG == 4 || SG == 8, "scale operand layout");
        v4i fa[BM];
        uint32_t swv[BN][SG / 2];
        if constexpr (!PER_TENSOR) {
#pragma unroll
            for (int bm = 0; bm < BM; ++bm) {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(sa + (wm + bm * 32 + l32) * SG);
                if constexpr (SG == 4) fa[bm] = (v4i){(int)p[0], (int)p[1], 0, 0};
                else fa[bm] = (v4i){(int)p[0], (int)p[1], (int)p[2], (int)p[3]};
            }
#pragma unroll
            for (int bn = 0; bn < BN; ++bn) {
                const uint32_t* p = reinterpret_cast<const uint32_t*>(sbp + (wn + bn * 32 + l32) * SG);
#pragma unroll
                for (int e = 0; e < SG / 2; ++e) swv[bn][e] = p[e];
            }
        }
#pragma unroll
        for (int g = 0; g < SG; ++g) {
            if (g >= groups_here) break;
            v4i afr[BM], bfr[BN];
#pragma unroll
            for (int bm = 0; bm < BM; ++bm) {
                const uint2 w = *reinterpret_cast<const uint2*>(base + (g * 2 + half) * S::kAPlane +
                                                                (wm + bm * 32 + l32) * 8);
                uint32_t lo0, hi0, lo1, hi1;
                unpack_s4x8_x16(w.x, lo0, hi0);
                unpack_s4x8_x16(w.y, lo1, hi1);
                afr[bm] = (v4i){(int)lo0, (int)hi0, (int)lo1, (int)hi1};
            }
#pragma unroll
            for (int bn = 0; bn < BN; ++bn) {
                const uint2 w = *reinterpret_cast<const uint2*>(bbase + (g * 2 + half) * S::kBPlane +
                                                                (wn + bn * 32 + l32) * 8);
                uint32_t lo0, hi0, lo1, hi1;
                unpack_s4x8_x16(w.x, lo0, hi0);
                unpack_s4x8_x16(w.y, lo1, hi1);
                bfr[bn] = (v4i){(int)lo0, (int)hi0, (int)lo1, (int)hi1};
            }
            if constexpr (PER_TENSOR) {
#pragma unroll
                for (int bm = 0; bm < BM; ++bm)
#pragma unroll
                    for (int bn = 0; bn < BN; ++bn)
                        iacc[bm][bn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[bm], bfr[bn],
                                                                              iacc[bm][bn], 0, 0, 0);
            } else {
                // fold factors 2*sx*sw: the A operand holds the row's SG
                // activation scales of the stage (read once per stage), the B
                // operand only group g's weight scale, its other elements zero
#pragma unroll
                for (int bn = 0; bn < BN; ++bn) {
                    v4i& q = fbq[bn][g >> 1];
                    q[g >> 1] = (int)(swv[bn][g >> 1] & ((g & 1) ? 0xffff0000u : 0x0000ffffu));
                }
#pragma unroll
                for (int bm = 0; bm < BM; ++bm) {
#pragma unroll
                    for (int bn = 0; bn < BN; ++bn) {
                        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[bm], bfr[bn],
                                                                             (v16i){0}, 0, 0, 0);
                        const v16f sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, fa[bm]), __builtin_bit_cast(bf16x8, fbq[bn][g >> 1]),
                            (v16f){0.0f}, 0, 0, 0);
#pragma unroll
                        for (int j = 0; j < NR; ++j)
                            acc[bm][bn][j] = __builtin_fmaf((float)d[j], sc[j], acc[bm][bn][j]);
                    }
                }
            }
        }
    };

    if (n_stages > 0) {
        R r;
        load_stage(0, r);
        store_stage(0, r);
        __syncthreads();
        for (int st = 0; st < n_stages; ++st) {
            const bool more = st + 1 < n_stages;
            if (more) load_stage(st + 1, r);
            compute_stage(st & 1, st);
            if (more) store_stage((st + 1) & 1, r);
            __syncthreads();
        }
    }

    // Epilogue.  The MFMA ran on 16*code operands (2^-8); the group-scaled
    // fold also carries the 2 of scale_products.
    float out_scale = kFoldOutScale;
    if constexpr (PER_TENSOR) out_scale = (alpha_dev ? *alpha_dev : alpha) * (1.0f / 256.0f);
#pragma unroll
    for (int bm = 0; bm < BM; ++bm)
#pragma unroll
        for (int bn = 0; bn < BN; ++bn) {
            const int col = n0 + wn + bn * 32 + l32;
#pragma unroll
            for (int j = 0; j < (PER_TENSOR ? 16 : NR); ++j) {
                const int row = m0 + wm + bm * 32 + 8 * (j >> 2) + 4 * half + (j & 3);
                if (row < M && col < N) {
                    float v;
                    if constexpr (PER_TENSOR)
                        v = (float)iacc[bm][bn][j] * out_scale;
                    else
                        v = acc[bm][bn][j] * out_scale;
                    if (partial != nullptr)
                        partial[((size_t)blockIdx.z * M + row) * N + col] = v;
                    else
                        y[(size_t)row * N + col] = f32_to_f16_bits(v);
                }
            }
        }
}

// ---------------------------------------------------- streaming kernels
// Decode-sized M: the run time is the weight stream.  A stage is 8 groups
// (one 128-byte line per weight row).  Its weights are read with fully
// coalesced loads (lane i: row 8j + i/8, line chunk i%8) and transposed
// through a wavefront-private LDS slab into the MFMA operand layout
// [group][k-half][row][8 B]; the slab's plane stride (272 B for 32 rows)
// makes both the transposing writes and the fragment reads bank-conflict-free,
// and no workgroup barrier is needed.  Requires K % 256 == 0 and slices of
// whole stages.
constexpr int kStreamSG = 8;                     // groups per stage
constexpr int kStreamPlane = 32 * 8 + 16;        // bytes per (group, half) plane of a 32-row block

// ---------------------------- streaming kernel, 8 < M <= 32, K split in-workgroup
// One workgroup per 32-row weight block (and global K slice); its KW
// wavefronts take contiguous runs of the slice's stages (wavefront w: stages
// [w c, (w+1) c)), so a Llama-70B FFN layer (N = 57344) runs 7168 wavefronts.
// Every global load is whole 128-byte lines or, for scales, whole 64-byte
// runs: a load instruction whose 64 lanes touch 32 different lines costs the
// vector memory path about as much as one that reads them whole (measured:
// with each row's 16- and 32-byte pieces loaded per lane, the L70 M=32 kernel
// took 80 us; without the scale loads alone, 54).  Per stage a wavefront loads
// the block's weights and the activations as 8 rows x 128 bytes per
// instruction, both transposed through its LDS slab, and every fourth stage
// the next four stages' bf16 scales of its activation rows and weight columns
// by LDS DMA (64 contiguous bytes per row).  Addresses are a wave-uniform
// base plus a 32-bit lane offset (no 64-bit address arithmetic per load).
//
// Fold factors: the bf16 MFMA takes the lane's 8 activation scales of the
// stage and a weight-scale operand holding only group g's scale (the other 7
// elements zero), so each factor is 2*sx[g]*sw[g] exactly.  The four weight
// operands (one per scale dword) keep their zero elements in registers across
// the loop: one AND per group builds an operand.  A non-finite activation
// scale meets a zero and gives NaN for its whole row, as the reference's
// dequantized product does (code 0 * inf scale).  Groups are software
// pipelined: group g+1's two MFMAs are issued before group g's fold.  At the
// end the KW partial accumulators go through LDS and are summed in wavefront
// order (deterministic).  Requires K % 256 == 0, 16-byte aligned scales and
// slices of whole stages.
template <int MB>
struct Stream32Stage {
    uint4 w[4];         // weight line chunks: row 8j + lane/8, group lane%8
    uint4 x[MB][4];     // activation line chunks: row 32b + 8j + lane/8, group lane%8
};
// the bf16 scales of one stage: activation row 32b + lane%32, weight column lane%32
template <int MB>
struct Stream32Scales {
    uint4 sx[MB];
    uint4 sw;
};
constexpr int kStreamXRow = 2 * 64 + 16;         // slab bytes per activation row: [k-half][group][8 B] + pad
constexpr int kStreamSC = 4;                     // stages per scale DMA
constexpr int kStreamSBlock = 32 * kStreamSC * 16;   // slab bytes per 32-row scale block
constexpr int stream32_slab(int mb) {
    return kStreamSG * 2 * kStreamPlane + mb * 32 * kStreamXRow + (mb + 1) * kStreamSBlock;
}

// MR: rows folded in the last 32-row activation block (8..32); MB: activation
// blocks per wavefront (1: M <= 32; 2: 32 < M <= 64, the first block full).
// Both blocks multiply the same staged weights, so the weights stream once.
template <int MR, int MB, int KW, int OCC>
__global__ __launch_bounds__(64 * KW) __attribute__((amdgpu_waves_per_eu(OCC)))
void gemm_s4_stream32_kernel(const uint8_t* __restrict__ xq, const uint16_t* __restrict__ xs,
                             const uint8_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                             uint16_t* __restrict__ y, float* __restrict__ partial, int M, int N, int K,
                             int groups_per_split) {
    constexpr int NRL = MR / 2;                  // accumulator registers of the last block
    constexpr int NA = 16 * (MB - 1) + NRL;      // accumulator registers in all
    constexpr int kSlab = stream32_slab(MB);
    static_assert(MR % 8 == 0 && MR <= 32 && (MB == 1 || MB == 2), "fold rows");
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    // wave-uniform (readfirstlane): the stage loop is uniform control flow
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int G = K >> 5;
    const int K2 = K >> 1;
    const int g_begin = blockIdx.y * groups_per_split;
    const int g_end = min(G, g_begin + groups_per_split);
    const int nst = (g_end - g_begin) / kStreamSG;
    const int chunk = (nst + KW - 1) / KW;                     // wavefront w: stages [w chunk, (w+1) chunk)
    const int s0 = wave * chunk;
    const int cnt = max(0, min(nst, s0 + chunk) - s0);           // stages of this wavefront
    const int n0 = blockIdx.x * 32;
    uint8_t* slab = smem + (size_t)wave * kSlab;

    // Uniform bases; rows past N read the block's row 0 and activation rows
    // past M read row 0 (their outputs are never stored), so the loop has no
    // branches.
    const uint8_t* wbase = wq + (size_t)n0 * K2 + (size_t)g_begin * 16;
    const uint16_t* swbase = ws + (size_t)n0 * G + g_begin;
    const uint8_t* xbase = xq + (size_t)g_begin * 16;
    const uint16_t* sxbase = xs + g_begin;
    const int nvalid = N - n0;
    uint32_t woff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 8 * j + (lane >> 3);
        woff[j] = (uint32_t)(r < nvalid ? r : 0) * (uint32_t)K2 + (uint32_t)(lane & 7) * 16u;
    }
    uint32_t xoff[MB][4];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = 32 * b + 8 * j + (lane >> 3);
            xoff[b][j] = (uint32_t)(r < M ? r : 0) * (uint32_t)K2 + (uint32_t)(lane & 7) * 16u;
        }
    uint8_t* xslab = slab + kStreamSG * 2 * kStreamPlane;
    uint8_t* sslab = xslab + MB * 32 * kStreamXRow;
    // Scale DMA lanes (instruction j of a block): row (64 j + lane) / SC and
    // stage (lane % SC) ^ f(row), so that the reader of row r, stage q finds
    // it at 16 (SC r + (q ^ f(r))) with f(r) = (r / (16 / SC)) % SC: 16
    // consecutive rows then read distinct banks.
    constexpr int SC = kStreamSC, NJ = 32 * SC / 64;
    auto swz = [](int r) { return (r / (16 / SC)) % SC; };
    uint32_t dsx[MB][NJ], dsw[NJ];
    int dpc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int rr = (64 * j + lane) / SC;
        dpc[j] = (lane % SC) ^ swz(rr);
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            const int r = 32 * b + rr;
            dsx[b][j] = (uint32_t)(r < M ? r : 0) * (uint32_t)G;
        }
        dsw[j] = (uint32_t)(rr < nvalid ? rr : 0) * (uint32_t)G;
    }
    const int rsw = swz(l32);

    float acc[NA];
#pragma unroll
    for (int j = 0; j < NA; ++j) acc[j] = 0.0f;
    // weight-scale operands: quad p carries scale dword p, the rest stay zero
    v4i fb[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) fb[p] = (v4i){0, 0, 0, 0};

    auto stage_of = [&](int i) { return s0 + i; };
    // scales of stages st .. st + SC - 1 (at most the wavefront's last) into
    // the slab: each row's 16 SC contiguous bytes
    auto dma_sc = [&](int st) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int sp = min(st + dpc[j], s0 + cnt - 1) * kStreamSG;
#pragma unroll
            for (int b = 0; b < MB; ++b)
                dma16_ordered(sxbase + dsx[b][j] + sp, lds_addr(sslab + b * kStreamSBlock + 1024 * j));
            dma16_ordered(swbase + dsw[j] + sp, lds_addr(sslab + MB * kStreamSBlock + 1024 * j));
        }
    };
    auto read_sc = [&](int q, Stream32Scales<MB>& C) {
        const int o = l32 * (16 * SC) + 16 * (q ^ rsw);
#pragma unroll
        for (int b = 0; b < MB; ++b) C.sx[b] = *reinterpret_cast<const uint4*>(sslab + b * kStreamSBlock + o);
        C.sw = *reinterpret_cast<const uint4*>(sslab + MB * kStreamSBlock + o);
    };
    auto load_w = [&](int st, Stream32Stage<MB>& S) {
        const uint8_t* b = wbase + (size_t)st * (kStreamSG * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) S.w[j] = load_nt16(b + woff[j]);
    };
    auto load_x = [&](int st, Stream32Stage<MB>& S) {
        const uint8_t* bx = xbase + (size_t)st * (kStreamSG * 16);
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) S.x[b][j] = *reinterpret_cast<const uint4*>(bx + xoff[b][j]);
    };
    // weights and activations of a stage into the slab
    auto to_slab = [&](const Stream32Stage<MB>& S) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 v = S.w[j];
            const int row = 8 * j + (lane >> 3), g = lane & 7;
            uint8_t* base = slab + row * 8;
            *reinterpret_cast<uint2*>(base + (g * 2 + 0) * kStreamPlane) = make_uint2(v.x, v.y);
            *reinterpret_cast<uint2*>(base + (g * 2 + 1) * kStreamPlane) = make_uint2(v.z, v.w);
        }
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint4 v = S.x[b][j];
                const int row = 8 * j + (lane >> 3), g = lane & 7;
                uint8_t* base = xslab + (b * 32 + row) * kStreamXRow + g * 8;
                *reinterpret_cast<uint2*>(base) = make_uint2(v.x, v.y);
                *reinterpret_cast<uint2*>(base + 64) = make_uint2(v.z, v.w);
            }
    };
    auto compute = [&](const Stream32Scales<MB>& S) {
        // k-half `half` of groups 2t and 2t+1 of row 32b + l32 (rows >= M: not stored)
        uint4 xr[MB][kStreamSG / 2];
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int t = 0; t < kStreamSG / 2; ++t)
                xr[b][t] = *reinterpret_cast<const uint4*>(xslab + (b * 32 + l32) * kStreamXRow + half * 64 + t * 16);
        const uint32_t* sww = &S.sw.x;
        // group g, activation block b: D and the fold factors
        auto issue = [&](int g, int b, v16i& d, v16f& f) {
            const uint4& xv = xr[b][g >> 1];
            uint32_t a0, a1, a2, a3, b0, b1, b2, b3;
            unpack_s4x8_x16((g & 1) ? xv.z : xv.x, a0, a1);
            unpack_s4x8_x16((g & 1) ? xv.w : xv.y, a2, a3);
            const uint2 w = *reinterpret_cast<const uint2*>(slab + (g * 2 + half) * kStreamPlane + l32 * 8);
            unpack_s4x8_x16(w.x, b0, b1);
            unpack_s4x8_x16(w.y, b2, b3);
            const v4i A = {(int)a0, (int)a1, (int)a2, (int)a3};
            const v4i B = {(int)b0, (int)b1, (int)b2, (int)b3};
            const v4i fa = {(int)S.sx[b].x, (int)S.sx[b].y, (int)S.sx[b].z, (int)S.sx[b].w};
            v4i& fbg = fb[g >> 1];
            if (b == 0) fbg[g >> 1] = (int)(sww[g >> 1] & ((g & 1) ? 0xffff0000u : 0x0000ffffu));
            d = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, (v16i){0}, 0, 0, 0);
            f = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa),
                                                        __builtin_bit_cast(bf16x8, fbg), (v16f){0.0f}, 0, 0, 0);
        };
        auto fold = [&](int b, const v16i& d, const v16f& f) {
            constexpr int kLast = NRL;
            const int nr = b == MB - 1 ? kLast : 16;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < nr) acc[16 * b + j] = __builtin_fmaf((float)d[j], f[j], acc[16 * b + j]);
        };
        v16i d0, d1;
        v16f f0, f1;
        if constexpr (MB == 1) {
            // groups pipelined: group g+1's MFMAs are issued before group g's fold
            issue(0, 0, d0, f0);
#pragma unroll
            for (int g = 0; g < kStreamSG; g += 2) {
                issue(g + 1, 0, d1, f1);
                fold(0, d0, f0);
                if (g + 2 < kStreamSG) issue(g + 2, 0, d0, f0);
                fold(0, d1, f1);
            }
        } else {
            // blocks pipelined: block 1's MFMAs are issued before block 0's fold
#pragma unroll
            for (int g = 0; g < kStreamSG; ++g) {
                issue(g, 0, d0, f0);
                issue(g, 1, d1, f1);
                fold(0, d0, f0);
                fold(1, d1, f1);
            }
        }
    };

    // One stage in flight: the next stage's weights and activations are
    // requested as soon as this stage's sit in the slab, before its MFMAs and
    // fold.  The scales of stages 4c .. 4c+3 arrive by DMA, requested after
    // the last read of the previous chunk's (before stage 4c-1's MFMAs) and
    // waited for at stage 4c, where nothing else is in flight.
    Stream32Stage<MB> S;
    if (cnt > 0) {
        load_w(stage_of(0), S);
        load_x(stage_of(0), S);
        dma_sc(stage_of(0));
    }
    for (int i = 0; i < cnt; ++i) {
        Stream32Scales<MB> C;
        to_slab(S);
        if (i % SC == 0) WUSH_WAIT_VMCNT(0);       // this chunk's scales have landed
        const int nx = min(i + 1, cnt - 1);          // past the last stage: the last again (not used)
        load_w(stage_of(nx), S);
        load_x(stage_of(nx), S);
        __builtin_amdgcn_sched_barrier(0);
        read_sc(i % SC, C);
        if (i % SC == SC - 1 && i + 1 < cnt) {
            __builtin_amdgcn_s_waitcnt(0xC07F);      // lgkmcnt(0): the chunk's last scale reads are done
            dma_sc(stage_of(i + 1));
        }
        __builtin_amdgcn_sched_barrier(0);
        compute(C);
        __builtin_amdgcn_sched_barrier(0);
    }

    // Sum the KW partial accumulators in wavefront order; wavefront w stores
    // accumulator registers w, w + KW, ...
    __syncthreads();                                   // every slab is consumed
    float* red = reinterpret_cast<float*>(smem);       // [KW][NA][64]
#pragma unroll
    for (int j = 0; j < NA; ++j) red[(wave * NA + j) * 64 + lane] = acc[j];
    __syncthreads();
    const int col = n0 + l32;
    for (int j = wave; j < NA; j += KW) {
        float v = red[j * 64 + lane];
#pragma unroll
        for (int w = 1; w < KW; ++w) v += red[(w * NA + j) * 64 + lane];
        const int jb = j & 15;
        const int row = 32 * (j >> 4) + 8 * (jb >> 2) + 4 * half + (jb & 3);
        if (row < M && col < N) {
            v *= kFoldOutScale;
            if (partial != nullptr)
                partial[((size_t)blockIdx.y * M + row) * N + col] = v;
            else
                y[(size_t)row * N + col] = f32_to_f16_bits(v);
        }
    }
}

constexpr size_t stream32_smem(int kw, int na) {
    const size_t slab = (size_t)kw * stream32_slab(na > 16 ? 2 : 1);
    return slab > (size_t)kw * na * 64 * 4 ? slab : (size_t)kw * na * 64 * 4;
}

// Sum the split-K partials in slice order and convert to fp16.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial,
                                                            uint16_t* __restrict__ y, int64_t MN,
                                                            int splits) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= MN) return;
    float v = 0.0f;
    for (int z = 0; z < splits; ++z) v += partial[(int64_t)z * MN + i];
    y[i] = f32_to_f16_bits(v);
}

// MFMA operand-layout self-test (one wavefront): c = a(8x32) @ b(32x8) via
// the same fragment assignment the GEMM uses (A: lane -> row l%32, bytes of
// k-half l/32; B: lane -> column l%32, same k-half; D[j] -> row
// 8*(j/4)+4*(l/32)+j%4, column l%32).
__global__ void mfma_selftest_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ b,
                                     int32_t* __restrict__ c) {
    const int lane = threadIdx.x & 63;
    const int half = lane >> 5, l32 = lane & 31;
    uint32_t av[4] = {0, 0, 0, 0}, bv[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int k = half * 16 + e;
        const uint32_t ae = (l32 < 8) ? (uint8_t)a[l32 * 32 + k] : 0u;
        const uint32_t be = (l32 < 8) ? (uint8_t)b[k * 8 + l32] : 0u;
        av[e >> 2] |= ae << (8 * (e & 3));
        bv[e >> 2] |= be << (8 * (e & 3));
    }
    const v4i A = {(int)av[0], (int)av[1], (int)av[2], (int)av[3]};
    const v4i B = {(int)bv[0], (int)bv[1], (int)bv[2], (int)bv[3]};
    const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, (v16i){0}, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int row = 8 * (j >> 2) + 4 * half + (j & 3);
        if (row < 8 && l32 < 8) c[row * 8 + l32] = d[j];
    }
}

// ---------------------------------------------------------------- planning
struct Plan {
    int cfg;        // 0: 32x128 (M <= 32), 1: 64x128, 2: 128x128,
                    // 4: streaming with in-workgroup K split (M <= 64),
                    // 5: 256x256 fp16-MFMA tiles (gemm_h16.hip),
                    // 6: fp16-MFMA streaming, 8 < M <= 64 (gemm_h16s.hip)
    int mr;         // fold rows per 32-row block (cfg 0, 4)
    int splits;
    int groups_per_split;
    int tm, tn, sg;
    bool a16 = false;  // cfg 5: activations pre-converted into the workspace (gemm_h16q.hip)
};

// Workspace layout: fp32 split-K partials [splits][M][N] from offset 0, then
// (a16 plans) the pre-converted activations at the next 256-byte boundary.
static size_t plan_partial_bytes(const Plan& p, int64_t M, int64_t N) {
    return p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
}
static size_t plan_a16_offset(const Plan& p, int64_t M, int64_t N) {
    return (plan_partial_bytes(p, M, N) + 255) / 256 * 256;
}
static size_t plan_bytes(const Plan& p, int64_t M, int64_t N, int64_t K) {
    return p.a16 ? plan_a16_offset(p, M, N) + gemm_h16a_workspace_bytes(M, N, K, p.splits) : plan_partial_bytes(p, M, N);
}

#ifndef WUSH_PF_BM
#define WUSH_PF_BM 2             // prefill tile: 32x32 blocks per wavefront along M
#endif
#ifndef WUSH_PF_MIN_TILES
#define WUSH_PF_MIN_TILES 400    // fewer 128x128 tiles than this take 64x128 tiles (plus split-K):
#endif                           // M=128 K=N=8192 55.4 -> 46.5 us, M=256 K=4096 N=24576 (384 tiles)
                                 // 101.5 -> 96.0 us; L70 M=128 (448 tiles) 216 us with 128x128, 230 without
#ifndef WUSH_PF_BN
#define WUSH_PF_BN 2             // and along N (2 x 2 wavefronts per workgroup)
#endif
// fp16-MFMA 256x256 tiles (gemm_h16.hip) from this M when they make at least
// this many tiles (K % 256 == 0).  Against the int8 tiles on MI355X: L70
// M=256 (224 tiles) 249 vs 392 us, M=2048 K=N=4096 (128) 108 vs 128,
// M=1024 K=N=8192 (128) 195 vs 217; L70 M=160 251 vs 434, M=192 239 vs 410,
// M=224 239 vs 386 (half-empty row tiles); below: L70 M=128 254 vs 238 (the
// 128-row tiles take it), M=256 K=4096 N=24576 (96 tiles) 105 vs 100, M=512
// K=N=8192 (64) 192 vs 138.
#ifndef WUSH_H16_MIN_M
#define WUSH_H16_MIN_M 129
#endif
#ifndef WUSH_H16_MIN_TILES
#define WUSH_H16_MIN_TILES 128       // workgroups, counting K slices
#endif
// K split of the fp16 tiles (fp32 partials in the workspace, summed by
// splitk_reduce_kernel) from this M while fewer than 256 workgroups would run:
// M=1024 K=N=4096 (64 tiles, 4 slices) 80 -> 67 us against the int8 tiles,
// M=512 K=N=8192 135 -> 97, M=1024 K=N=8192 (128 tiles, 2 slices) 206 -> 163;
// at M=256 it lost (K=4096 N=24576: 97 -> 112 us, 384 workgroups).
#ifndef WUSH_H16_MAX_SPLITS
#define WUSH_H16_MAX_SPLITS 8
#endif
// Every K slice of the fp16 tiles keeps at least this many groups: a slice
// of 16 groups spends more on its ring fill, prologue and epilogue and on the
// fp32 partials than on MFMAs (M=2048 N=512 K=4096: 8 slices 41.5 us, 4
// slices 28.7; K=N=2048 M=1024: 40.8 -> 30.6; M=512 N=2048 K=4096 38.4 ->
// 30.2; unchanged at 1024 x 4096 x 4096, 512 x 8192 x 8192, 2048 x 4096 x 4096).
#ifndef WUSH_H16_MIN_SPLIT_GROUPS
#define WUSH_H16_MIN_SPLIT_GROUPS 32
#endif
// With fewer than this many 256x256 tiles and N below WUSH_H16_FEW_TILES_MIN_N
// the int8 tiles win (K=4096: M=4096 N=512 51.2 -> 46.1 us, M=2048 N=1024
// 49.0 -> 46.1; K=8192: M=1024 N=1024 50.0 -> 45.1, M=2048 N=512 50.1 ->
// 46.3); from N = 2048 the fp16 tiles keep them (M=1024 N=2048 K=8192: 64.9
// against 72.3 us with the int8 tiles), and from 64 tiles at any N (M=4096
// N=1024 K=4096: 66.6 against 74.9).
#ifndef WUSH_H16_FEW_TILES
#define WUSH_H16_FEW_TILES 64
#endif
#ifndef WUSH_H16_FEW_TILES_MIN_N
#define WUSH_H16_FEW_TILES_MIN_N 2048
#endif
#ifndef WUSH_H16_SPLIT_MIN_M
#define WUSH_H16_SPLIT_MIN_M 512
#endif
// Pre-converted activations (gemm_h16q.hip) when the weights have at least this
// many columns, the scales are 16-byte aligned and the workspace has room
// for M x K x 2 bytes more.
#ifndef WUSH_H16A_MIN_N
#define WUSH_H16A_MIN_N 8192
#endif
// 64 < M <= this, where the 256-row fp16 tiles do not run: the
// pre-converted-activation fp16 tiles with 128-row tiles (gemm_h16q_kernel<4>)
// on weights of at least WUSH_H16A_MIN_N columns, when they make at least
// WUSH_H16R_MIN_WGS workgroups, in place of the int8 tiles (0: off).
// Measured on MI355X against the int8 tiles: L70 (K=8192, N=57344) M=128 154
// vs 254 us, M=96 156 vs 248, M=72 147 vs 225, K=8192 N=28672 M=128 95 vs 134;
// K=4096 N=24576 M=128 (2 K slices) 59.7 vs 67.9.  With 4 slices it was not
// a steady gain (K=N=8192 M=128: 47.4 vs 49.8 on one box, 56.2 vs 52.3 on
// another), and with slices of 32 groups (K=4096 N=8192) it took 40.2
// against 32.0: hence at most 2 slices of at least 64 groups.  Above M = 128
// (256-row tiles too few): K=4096 N=24576 M=256 74.9 vs 111.4, M=192 73.1 vs
// 102.8, K=4096 N=16384 M=200 (2 slices) 61.6 vs 75.4; with 128 workgroups
// it lost (K=N=8192 M=256 83.7 vs 81.3, M=192 79.5 vs 66.2; K=4096 N=8192
// M=256 54.8 vs 50.2), hence at least 192.
#ifndef WUSH_H16R_MAX_M
#define WUSH_H16R_MAX_M 256
#endif
#ifndef WUSH_H16R_MIN_WGS
#define WUSH_H16R_MIN_WGS 192
#endif
#ifndef WUSH_H16R_MIN_SPLIT_GROUPS
#define WUSH_H16R_MIN_SPLIT_GROUPS 64
#endif
#ifndef WUSH_H16R_MAX_SPLITS
#define WUSH_H16R_MAX_SPLITS 2
#endif
// 8 < M <= 64 streaming kernel (gemm_s4_stream32_kernel).  K ways: 4
// wavefronts per workgroup on wide weights, 8 on narrow ones (measured on
// MI355X, M = 32: L70 (K=8192, N=57344) 66 us with 4, 83 with 8, 67 with 2 (M=24:
// 62 vs 69, M=16: 59 vs 62 with 2); K=N=8192
// 14.7 with 8, 17.8 with 4; K=28672 N=8192 33.4 with 8, 36.2 with 4; K=4096
// N=24576 18.5 with 4, 23.4 with 8).  Three wavefronts per SIMD at M <= 32
// (159-166 VGPRs), two at 32 < M <= 64.
#ifndef WUSH_S32_KW_WIDE
#define WUSH_S32_KW_WIDE 4       // wavefronts per workgroup (= K ways) when N > WUSH_S32_WIDE_N
#endif
#ifndef WUSH_S32_KW_NARROW
#define WUSH_S32_KW_NARROW 8     // ... and otherwise
#endif
#ifndef WUSH_S32_WIDE_N
#define WUSH_S32_WIDE_N 16384
#endif
#ifndef WUSH_S32_OCC
#define WUSH_S32_OCC 3           // wavefronts per SIMD the registers allow, M <= 32
#endif
#ifndef WUSH_S32_OCC64
#define WUSH_S32_OCC64 2         // ... and at 32 < M <= 64
#endif
#ifndef WUSH_S32_MIN_STAGES
#define WUSH_S32_MIN_STAGES 2    // split K across workgroups only while every wavefront keeps this many stages
                                 // (1 was slower at M <= 16 and equal elsewhere: the split-K sum costs more)
#endif
#ifndef WUSH_S32_WAVES
#define WUSH_S32_WAVES 2048      // split K across workgroups below this many wavefronts
#endif
#ifndef WUSH_S32_MAXM
#define WUSH_S32_MAXM 64         // largest M of the streaming kernel (64: two activation blocks)
#endif
constexpr int kStream32MaxM = WUSH_S32_MAXM;
constexpr int stream32_kw(int64_t n) { return n > WUSH_S32_WIDE_N ? WUSH_S32_KW_WIDE : WUSH_S32_KW_NARROW; }
constexpr int kStream32Waves = WUSH_S32_WAVES;

// scales16: both scale tensors (and both code tensors) are 16-byte aligned
// (the streaming kernels read them 16 bytes at a time).
static Plan make_plan(int64_t M, int64_t N, int64_t K, size_t ws_bytes_available, bool allow_split,
                      bool scales16, bool allow_a16 = true) {
    Plan p;
    p.mr = 32;
    const int64_t G0 = K / 32;
    if (allow_split && scales16 && gemm_h16s_shape_ok(M, N, K)) {
        // wide weights at 8 < M <= 64: fp16-MFMA streaming, no workspace
        p.cfg = 6; p.tm = 32; p.tn = 32; p.sg = 16;
        p.splits = 1;
        p.groups_per_split = (int)G0;
        return p;
    }
    if (allow_split && scales16 && M <= kStream32MaxM && K % 256 == 0) {
        // in-workgroup K split: one workgroup of stream32_kw wavefronts per
        // 32-row block; split K across workgroups only while fewer than
        // kStream32Waves wavefronts would stream and every wavefront keeps
        // at least two stages
        p.cfg = 4; p.tm = 32; p.tn = 32; p.sg = kStreamSG;
        p.mr = M > 32 ? 64 : (int)((M + 7) / 8 * 8);
        const int kw = stream32_kw(N);
        const int64_t wgs = (N + 31) / 32;
        int s = 1;
        while (s < 16 && wgs * s * kw < kStream32Waves &&
               G0 / (2 * s) >= (int64_t)kw * WUSH_S32_MIN_STAGES * kStreamSG)
            s *= 2;
        int64_t gps = (G0 + s - 1) / s;
        gps = (gps + kStreamSG - 1) / kStreamSG * kStreamSG;
        s = (int)((G0 + gps - 1) / gps);
        if (s > 1 && (size_t)s * (size_t)M * (size_t)N * sizeof(float) > ws_bytes_available) {
            s = 1;                               // no room for partials: one slice
            gps = G0;
        }
        p.splits = s;
        p.groups_per_split = (int)gps;
        return p;
    }
    if (allow_split && K % 256 == 0 && M >= WUSH_H16_MIN_M &&
        (((M + 255) / 256) * ((N + 255) / 256) >= WUSH_H16_FEW_TILES || N >= WUSH_H16_FEW_TILES_MIN_N)) {
        // fp16-MFMA tiles, with K split across workgroups (slices of a
        // multiple of 8 groups) while fewer than 256 workgroups would run
        const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
        int s = 1;
        while (M >= WUSH_H16_SPLIT_MIN_M && s < WUSH_H16_MAX_SPLITS && tiles * s < 256 && G0 % (16 * s) == 0 &&
               G0 / (2 * s) >= WUSH_H16_MIN_SPLIT_GROUPS &&
               (size_t)(2 * s) * (size_t)M * (size_t)N * sizeof(float) <= ws_bytes_available)
            s *= 2;
        if (tiles * s >= WUSH_H16_MIN_TILES) {
            p.cfg = 5; p.tm = 256; p.tn = 256; p.sg = 1;
            p.splits = s;
            p.groups_per_split = (int)(G0 / s);
            if (allow_a16 && scales16 && N >= WUSH_H16A_MIN_N) {
                Plan q = p;
                q.a16 = true;
                if (plan_bytes(q, M, N, K) <= ws_bytes_available) p.a16 = true;
            }
            return p;
        }
    }
    if (allow_split && allow_a16 && scales16 && K % 256 == 0 && M > 64 && M <= WUSH_H16R_MAX_M &&
        N >= WUSH_H16A_MIN_N) {
        // 128-row fp16 tiles (where the 256-row ones do not run), K split
        // while twice the workgroups still run in one round on 256 CUs (one
        // workgroup per CU fits)
        const int64_t tiles = ((M + 127) / 128) * ((N + 255) / 256);
        int s = 1;
        while (s < WUSH_H16R_MAX_SPLITS && tiles * 2 * s <= 256 && G0 % (16 * s) == 0 &&
               G0 / (2 * s) >= WUSH_H16R_MIN_SPLIT_GROUPS &&
               (size_t)(2 * s) * (size_t)M * (size_t)N * sizeof(float) <= ws_bytes_available)
            s *= 2;
        Plan q = p;
        q.cfg = 5; q.tm = 128; q.tn = 256; q.sg = 1;
        q.splits = s;
        q.groups_per_split = (int)(G0 / s);
        q.a16 = true;
        if (tiles * s >= WUSH_H16R_MIN_WGS && plan_bytes(q, M, N, K) <= ws_bytes_available) return q;
    }
    const int64_t big_tiles = ((M + 32 * WUSH_PF_BM * 2 - 1) / (32 * WUSH_PF_BM * 2)) *
                              ((N + 32 * WUSH_PF_BN * 2 - 1) / (32 * WUSH_PF_BN * 2));
    if (M <= 32) {
        p.cfg = 0; p.tm = 32; p.tn = 128; p.sg = 8;
        p.mr = (int)((M + 7) / 8 * 8);
    } else if (M <= 64 || big_tiles < WUSH_PF_MIN_TILES) {
        p.cfg = 1; p.tm = 64; p.tn = 128; p.sg = 8;
    } else {
        p.cfg = 2; p.tm = 32 * WUSH_PF_BM * 2; p.tn = 32 * WUSH_PF_BN * 2; p.sg = 4;
    }
    const int64_t G = K / 32;
    const int64_t tiles = ((M + p.tm - 1) / p.tm) * ((N + p.tn - 1) / p.tn);
    int s = 1;
    if (allow_split) {
        // Aim for >= 3 workgroups per CU (256 CUs) while each slice keeps
        // at least 4 stages of K.
        while (s < 16 && tiles * s < 768 && G / (2 * s) >= 4 * p.sg) s *= 2;
    }
    int64_t gps = (G + s - 1) / s;
    gps = (gps + p.sg - 1) / p.sg * p.sg;
    s = (int)((G + gps - 1) / gps);
    if (s > 1 && (size_t)s * (size_t)M * (size_t)N * sizeof(float) > ws_bytes_available) {
        s = 1;
        gps = G;
    }
    p.splits = s;
    p.groups_per_split = (int)gps;
    return p;
}

template <int BM, int BN, int WM, int WN, int SG, int MR, bool PT>
static void launch_gemm(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                        uint16_t* y, float* partial, int M, int N, int K, const Plan& p, float alpha,
                        const float* alpha_dev, hipStream_t stream) {
    constexpr int TM = 32 * BM * WM, TN = 32 * BN * WN;
    const size_t smem = GemmSmem<TM, TN, SG>::kBytes;
    static_assert(GemmSmem<TM, TN, SG>::kBytes <= 64 * 1024, "LDS budget");
    dim3 grid((unsigned)((N + TN - 1) / TN), (unsigned)((M + TM - 1) / TM), (unsigned)p.splits);
    gemm_s4_kernel<BM, BN, WM, WN, SG, MR, PT><<<grid, 256, smem, stream>>>(
        xq, xs, wq, ws, y, partial, M, N, K, p.groups_per_split, alpha, alpha_dev);
}

// The streaming kernel for MR rows in the last of MB activation blocks, with
// the K ways of wide or narrow weights (p.groups_per_split groups per
// workgroup along grid.y).
template <int MR, int MB, int OCC>
static void launch_stream32(dim3 grid, bool wide, const uint8_t* xq, const uint16_t* xs, const uint8_t* wq,
                            const uint16_t* ws, uint16_t* y, float* partial, int m, int n, int k, const Plan& p,
                            hipStream_t stream) {
    constexpr int NA = 16 * (MB - 1) + MR / 2;
    if (wide) {
        constexpr int KW = WUSH_S32_KW_WIDE;
        gemm_s4_stream32_kernel<MR, MB, KW, OCC><<<grid, 64 * KW, stream32_smem(KW, NA), stream>>>(
            xq, xs, wq, ws, y, partial, m, n, k, p.groups_per_split);
    } else {
        constexpr int KW = WUSH_S32_KW_NARROW;
        gemm_s4_stream32_kernel<MR, MB, KW, OCC><<<grid, 64 * KW, stream32_smem(KW, NA), stream>>>(
            xq, xs, wq, ws, y, partial, m, n, k, p.groups_per_split);
    }
}

template <bool PT>
static int run_gemm(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                    uint16_t* y, int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes,
                    float alpha, const float* alpha_dev, hipStream_t stream, bool allow_a16 = true) {
    const bool scales16 = ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(ws) |
                            reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq)) & 15u) == 0;
    // the pre-converted activations need a 16-byte aligned workspace
    allow_a16 = allow_a16 && (reinterpret_cast<uintptr_t>(workspace) & 15u) == 0;
    const Plan p = make_plan(M, N, K, workspace ? ws_bytes : 0, !PT, scales16, allow_a16);
    WUSH_REQUIRE((N + p.tn - 1) / p.tn <= 0x7fffffffLL && (M + p.tm - 1) / p.tm <= 65535);
    float* partial = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const int m = (int)M, n = (int)N, k = (int)K;
    if (p.cfg == 6) {
        if constexpr (!PT) return launch_gemm_h16s(xq, xs, wq, ws, y, m, n, k, stream);
    }
    if (p.cfg == 5) {
        if constexpr (!PT) {
            uint8_t* wsp = static_cast<uint8_t*>(workspace);
            const int st = p.a16 ? launch_gemm_h16a(xq, xs, wq, ws, y, partial, m, n, k, p.splits,
                                                    p.groups_per_split, wsp + plan_a16_offset(p, M, N),
                                                    p.tm == 128, stream)
                                 : launch_gemm_h16(xq, xs, wq, ws, y, partial, m, n, k, p.splits,
                                                   p.groups_per_split, stream);
            if (st != 0 || p.splits == 1) return st;
        }
    }
    if (p.cfg == 4) {
        if constexpr (!PT) {
            const dim3 grid((unsigned)((N + 31) / 32), (unsigned)p.splits);
            const bool wide = N > WUSH_S32_WIDE_N;
            switch (p.mr) {
                case 8: launch_stream32<8, 1, WUSH_S32_OCC>(grid, wide, xq, xs, wq, ws, y, partial, m, n, k, p, stream); break;
                case 16: launch_stream32<16, 1, WUSH_S32_OCC>(grid, wide, xq, xs, wq, ws, y, partial, m, n, k, p, stream); break;
                case 24: launch_stream32<24, 1, WUSH_S32_OCC>(grid, wide, xq, xs, wq, ws, y, partial, m, n, k, p, stream); break;
                case 32: launch_stream32<32, 1, WUSH_S32_OCC>(grid, wide, xq, xs, wq, ws, y, partial, m, n, k, p, stream); break;
                default: launch_stream32<32, 2, WUSH_S32_OCC64>(grid, wide, xq, xs, wq, ws, y, partial, m, n, k, p, stream); break;
            }
        }
    } else if (p.cfg == 0) {
        if (PT || p.mr == 32)
            launch_gemm<1, 1, 1, 4, 8, 32, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream);
        else if (p.mr == 8)
            launch_gemm<1, 1, 1, 4, 8, 8, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream);
        else if (p.mr == 16)
            launch_gemm<1, 1, 1, 4, 8, 16, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream);
        else
            launch_gemm<1, 1, 1, 4, 8, 24, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream);
    } else if (p.cfg == 1) {
        launch_gemm<1, 2, 2, 2, 8, 32, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream);
    } else if (p.cfg == 2) {
        launch_gemm<WUSH_PF_BM, WUSH_PF_BN, 2, 2, 4, 32, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream);
    }
    if (p.splits > 1) {
        const int64_t MN = M * N;
        const int64_t blocks = (MN + 255) / 256;
        splitk_reduce_kernel<<<(unsigned)blocks, 256, 0, stream>>>(partial, y, MN, p.splits);
    }
    return (int)hipGetLastError();
}

}  // namespace wush

extern "C" {

size_t wush_gemm_s4_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 32) return 0;
    const wush::Plan p = wush::make_plan(M, N, K, (size_t)-1, true, true);
    return wush::plan_bytes(p, M, N, K);
}

int wush_gemm_s4(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                 uint16_t* y, int64_t M, int64_t N, int64_t K, void* workspace,
                 size_t workspace_bytes, hipStream_t stream) {
    WUSH_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 32 == 0);
    WUSH_REQUIRE(M <= 0x7fffffffLL && N <= 0x7fffffffLL && K <= 0x7fffffffLL);
    if (M == 0 || N == 0) return (int)hipSuccess;
    WUSH_REQUIRE(xq && xs && wq && ws && y);
    WUSH_REQUIRE(((uintptr_t)xq & 15u) == 0 && ((uintptr_t)wq & 15u) == 0);
    WUSH_REQUIRE(((uintptr_t)xs & 1u) == 0 && ((uintptr_t)ws & 1u) == 0 && ((uintptr_t)y & 1u) == 0);
    WUSH_REQUIRE(workspace == nullptr || ((uintptr_t)workspace & 3u) == 0);
    return wush::run_gemm<false>(xq, xs, wq, ws, y, M, N, K, workspace, workspace_bytes, 1.0f, nullptr,
                                 stream);
}

int wush_gemm_s4_noalloc(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                         uint16_t* y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    WUSH_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 32 == 0);
    WUSH_REQUIRE(M <= 0x7fffffffLL && N <= 0x7fffffffLL && K <= 0x7fffffffLL);
    if (M == 0 || N == 0) return (int)hipSuccess;
    WUSH_REQUIRE(xq && xs && wq && ws && y);
    WUSH_REQUIRE(((uintptr_t)xq & 15u) == 0 && ((uintptr_t)wq & 15u) == 0);
    WUSH_REQUIRE(((uintptr_t)xs & 1u) == 0 && ((uintptr_t)ws & 1u) == 0 && ((uintptr_t)y & 1u) == 0);
    // the plan wush_gemm_s4 runs when its workspace is the scratch's size:
    // split-K partials only (no pre-converted activations), with fewer K
    // slices where the shape's full split would need more than the scratch
    // (one slice needs none, so every shape has such a plan)
    const bool scales16 = ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(ws) |
                            reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq)) & 15u) == 0;
    const size_t cap = (size_t)WUSH_GEMM_SCRATCH_BYTES;
    const size_t need = wush::plan_bytes(wush::make_plan(M, N, K, cap, true, scales16, false), M, N, K);
    if (need > cap) return WUSH_ERROR_SCRATCH_TOO_SMALL;
    int dev = 0;
    const int st = wush::device_setup(&dev);
    if (st != 0) return st;
    void* scratch = need ? wush::scratch_address(dev) : nullptr;
    if (need && scratch == nullptr) return (int)hipErrorInvalidSymbol;
    return wush::run_gemm<false>(xq, xs, wq, ws, y, M, N, K, scratch, need ? cap : 0, 1.0f, nullptr, stream,
                                 false);
}

int wush_gemm_s4_tensor_scale(const uint8_t* xq, const uint8_t* wq, uint16_t* y, int64_t M, int64_t N,
                              int64_t K, float alpha, const float* alpha_dev, hipStream_t stream) {
    WUSH_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 32 == 0);
    // the MFMA accumulates products of 16*code operands, 256 * 64 per k at
    // most (codes -8 * -8): the int32 sum over K stays exact up to this K
    WUSH_REQUIRE(M <= 0x7fffffffLL && N <= 0x7fffffffLL && K <= WUSH_TENSOR_SCALE_MAX_K);
    if (M == 0 || N == 0) return (int)hipSuccess;
    WUSH_REQUIRE(xq && wq && y);
    WUSH_REQUIRE(((uintptr_t)xq & 15u) == 0 && ((uintptr_t)wq & 15u) == 0 && ((uintptr_t)y & 1u) == 0);
    return wush::run_gemm<true>(xq, nullptr, wq, nullptr, y, M, N, K, nullptr, 0, alpha, alpha_dev,
                                stream);
}

int wush_mfma_selftest(const int8_t* a, const int8_t* b, int32_t* c, hipStream_t stream) {
    WUSH_REQUIRE(a && b && c);
    wush::mfma_selftest_kernel<<<1, 64, 0, stream>>>(a, b, c);
    return (int)hipGetLastError();
}

}  // extern "C"
