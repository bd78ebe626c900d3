// gemm_h16s.hip -- the group-scaled W4A4 product for 32 < M <= 64 on weight
// matrices about 57344 rows long, on fp16 MFMA (csrc/gemm_s4.cu:85-379 is
// the reference contract; operands and numerics as in gemm_h16.hip: code *
// scale operands, exact in fp16, each row and column shifted by a power of
// two, exact fp32 products summed over the whole K in the MFMA accumulator).
//
// For these M the weights stream from HBM once and the work per weight byte
// is the conversion of its codes to fp16 operands (13 VALU per 8 codes).  The
// int8 kernels instead fold every 32 x 32 block of exact group dots into fp32
// with two VALU per output and group, after an MFMA whose result the fold
// waits for; here the operand conversion is the only VALU per MFMA and no
// result comes back before the epilogue.
//
// Workgroup: 7 column blocks of 32 weight rows (output columns) over all of
// K, one workgroup per CU (N = 57344 fills 256 CUs): 8 wavefronts, two per
// SIMD.  Wavefronts 0-6 own a column block each and convert its codes
// straight from registers into MFMA B operands; wavefront 7 converts the
// activations (MB 32-row blocks) of the next batch into an LDS double buffer
// -- the same VALU as one column block -- which all seven read back as A
// operands.  Every wavefront owns its outputs: no partial sums, one barrier
// per batch.  Loads run four batches ahead in registers; plain loads (the
// nontemporal hint made the stream half as fast).
//
// K order: a batch is 8 groups, 16 K16 MFMA slices; slice j gives lane half h
// dword j % 4 of group 4h + j / 4 of the batch (8 codes).  So a lane reads 64
// contiguous code bytes of its row or column per batch (four 16-byte loads
// issued together, and the two halves make the whole 128-byte line), and
// 8 bytes of scales.  Both operands use the same order.
//
// Shifts: per row and per column over all of K, from a prologue pass over the
// scales that reads whole 128-byte lines (the first batches of codes are
// already in flight).  With each lane reading 16 bytes of its own row or
// column per instruction (32 lines touched per instruction) the prologue took
// 20 us of the 108 at L70 M=64; with whole lines 12.
#include "gemm_h16_device.h"
#include "gemm_h16.h"
#include "setup.h"

namespace wush {
namespace {

constexpr int kSBatch = 8;                       // groups per batch
constexpr int kSSlices = 2 * kSBatch;            // K16 slices per batch
constexpr int kSCols = 7;                        // column blocks (wavefronts) per workgroup
constexpr int kSDepth = 4;                       // batches of loads in flight (even)

// One wavefront's work: NCB (0 or 1) column blocks from column block cb0
// and, with A_ALL, the activation conversion.  Compile-time roles keep the
// loop free of branches (the compiler would wait for every load at a join).
template <int MB, int NCB, bool A_ALL>
__device__ __forceinline__ void h16s_wave(const uint8_t* __restrict__ xq, const uint16_t* __restrict__ xs,
                                          const uint8_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                          uint16_t* __restrict__ y, int M, int N, int K, int cb0, int wave,
                                          uint8_t (*sA)[MB][kSSlices][64 * 16], uint32_t (*sh_mx)[MB * 32],
                                          int* sh_ea) {
    const int lane = threadIdx.x & 63;
    const int half = lane >> 5;
    const int l32 = lane & 31;
    const int G = K >> 5;
    const int K2 = K >> 1;
    const int nbat = G / kSBatch;                // batches (even)

    // lane offsets (bytes, 32-bit): rows past M and columns past N read the
    // last valid one (never stored)
    constexpr int NC1 = NCB > 0 ? NCB : 1;
    uint32_t xo[MB], xso[MB], wo[NC1], wso[NC1];
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        const int r = min(32 * b + l32, M - 1);
        xo[b] = (uint32_t)r * (uint32_t)K2 + (uint32_t)half * 64u;
        xso[b] = ((uint32_t)r * (uint32_t)G + (uint32_t)half * 4u) * 2u;
    }
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const int col = min(32 * (cb0 + c) + l32, N - 1);
        wo[c] = (uint32_t)col * (uint32_t)K2 + (uint32_t)half * 64u;
        wso[c] = ((uint32_t)col * (uint32_t)G + (uint32_t)half * 4u) * 2u;
    }
    const global_cptr<uint8_t> xqb = uniform_ptr(xq);
    const global_cptr<uint8_t> wqb = uniform_ptr(wq);
    const global_cptr<uint8_t> xsb = uniform_ptr(reinterpret_cast<const uint8_t*>(xs));
    const global_cptr<uint8_t> wsb = uniform_ptr(reinterpret_cast<const uint8_t*>(ws));
    auto ld16 = [](global_cptr<uint8_t> base, uint32_t off) {
        const u32x4 v = *reinterpret_cast<global_cptr<u32x4>>(base + off);
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    auto ld8 = [](global_cptr<uint8_t> base, uint32_t off) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = *reinterpret_cast<global_cptr<u32x2>>(base + off);
        return make_uint2(v.x, v.y);
    };
    auto max8 = [](const uint4& v) {
        const u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(abs_bits2(v.x), abs_bits2(v.y)),
                                                  __builtin_elementwise_max(abs_bits2(v.z), abs_bits2(v.w)));
        return max((uint32_t)m.x, (uint32_t)m.y);
    };

    int ea[MB], eb[NC1];                         // shifts (set by the prologue below)

    // codes and scales of one batch (activations: the four groups of the
    // lane half's quarter)
    constexpr int kAG = A_ALL ? 4 : 0;
    struct WBatch {
        uint4 w[NC1][4];
        uint2 wsc[NC1];
    };
    struct ABatch {
        uint4 a[MB][kAG > 0 ? kAG : 1];
        uint2 as[MB];
    };
    // past the last batch: the last again
    auto load_w = [&](int bt, WBatch& B) {
        bt = min(bt, nbat - 1);
        const uint32_t co = (uint32_t)bt * (kSBatch * 16), so = (uint32_t)bt * (kSBatch * 2);
#pragma unroll
        for (int c = 0; c < NCB; ++c) {
#pragma unroll
            for (int k = 0; k < 4; ++k) B.w[c][k] = ld16(wqb, wo[c] + co + 16u * k);
            B.wsc[c] = ld8(wsb, wso[c] + so);
        }
    };
    auto load_a = [&](int bt, ABatch& B) {
        if constexpr (A_ALL) {
            bt = min(bt, nbat - 1);
            const uint32_t co = (uint32_t)bt * (kSBatch * 16), so = (uint32_t)bt * (kSBatch * 2);
#pragma unroll
            for (int b = 0; b < MB; ++b) {
#pragma unroll
                for (int k = 0; k < kAG; ++k) B.a[b][k] = ld16(xqb, xo[b] + co + 16u * k);
                B.as[b] = ld8(xsb, xso[b] + so);
            }
        }
    };
    // fp32 value of scale k (0-3) of a lane's 4
    auto scale_of = [](const uint2& v, int k) {
        const uint32_t d = (k >> 1) ? v.y : v.x;
        return __uint_as_float((k & 1) ? (d & 0xffff0000u) : (d << 16));
    };
    auto dword_of = [](const uint4& v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; };
    // activation operands of a batch into LDS buffer buf (this wavefront's slices)
    auto convert_a = [&](const ABatch& B, int buf) {
        if constexpr (A_ALL) {
#pragma unroll
            for (int b = 0; b < MB; ++b) {
#pragma unroll
                for (int g = 0; g < kAG; ++g) {          // slices 4g .. 4g+3: group 4h + g
                    const h2 s = h16_scale(scale_of(B.as[b], g), ea[b]);
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        frag_write(sA[buf][b][4 * g + d], lane, h16_codes(dword_of(B.a[b][g], d), s));
                }
            }
        }
    };

    v16f acc[MB][NC1];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int c = 0; c < NCB; ++c) acc[b][c] = (v16f){0.0f};

    // Weights of batch b in R[b % D], loaded D batches ahead; activations of
    // batch b in RA[b % D], loaded D + 1 batches ahead and converted into LDS
    // buffer b & 1 at the end of batch b - 1.
    constexpr int D = kSDepth;
    WBatch R[D];
    ABatch RA[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        load_a(d, RA[d]);
        load_w(d, R[d]);
    }
    // (the first batches stream in during the prologue)
    // Prologue: the shifts, from the largest |scale| of every row and column.
    // The scan reads whole 128-byte lines: 8 lanes per row or column, lane
    // l % 8 taking its 16-byte pieces l % 8, l % 8 + 8, ... (P = G / 8 pieces;
    // an index past the last repeats it).  Rows: the 4 MB groups of 8 rows
    // are split over the 8 wavefronts (2 / MB wavefronts per group, each
    // taking every (2 / MB)-th run of 8 pieces); the partial maxima meet in
    // LDS.  Columns: each column wavefront scans its own 4 groups of 8.
    const int P = G >> 3;
    auto max_at = [&](global_cptr<uint8_t> base, uint32_t row_off, int p) {
        return max8(ld16(base, row_off + 16u * (uint32_t)min(p, P - 1)));
    };
    // largest over the 8 lanes of each aligned group
    auto max_over8 = [](uint32_t v) {
        v = max(v, (uint32_t)__shfl_xor((int)v, 1));
        v = max(v, (uint32_t)__shfl_xor((int)v, 2));
        return max(v, (uint32_t)__shfl_xor((int)v, 4));
    };
    {
        constexpr int kWpg = 2 / MB;                 // wavefronts per row group
        const int gi = wave % (4 * MB), part = wave / (4 * MB);
        const int r = min(8 * gi + (lane >> 3), M - 1);
        const uint32_t ro = (uint32_t)r * (uint32_t)G * 2u;
        uint32_t m = 0;
        for (int p0 = 8 * part; p0 < P; p0 += 8 * kWpg * 4) {
            uint32_t v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = max_at(xsb, ro, p0 + 8 * kWpg * u + (lane & 7));
#pragma unroll
            for (int u = 0; u < 4; ++u) m = max(m, v[u]);
        }
        m = max_over8(m);
        if ((lane & 7) == 0) sh_mx[part][8 * gi + (lane >> 3)] = m;
    }
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        uint32_t mg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int col = min(32 * (cb0 + c) + 8 * i + (lane >> 3), N - 1);
            const uint32_t co = (uint32_t)col * (uint32_t)G * 2u;
            uint32_t m = 0;
            for (int p0 = 0; p0 < P; p0 += 32) {
                uint32_t v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = max_at(wsb, co, p0 + 8 * u + (lane & 7));
#pragma unroll
                for (int u = 0; u < 4; ++u) m = max(m, v[u]);
            }
            mg[i] = max_over8(m);
        }
        // column l32 = 8 i + j: group i's maximum, held by lane 8 j
        const int src = 8 * (l32 & 7);
        uint32_t mx = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t v = (uint32_t)__shfl((int)mg[i], src);
            if ((l32 >> 3) == i) mx = v;
        }
        eb[c] = h16_shift(mx);
    }
    __syncthreads();                                 // row maxima
#pragma unroll
    for (int b = 0; b < MB; ++b) {
        uint32_t m = 0;
#pragma unroll
        for (int k = 0; k < 2 / MB; ++k) m = max(m, sh_mx[k][32 * b + l32]);
        ea[b] = h16_shift(m);
        if (wave == 0 && half == 0) sh_ea[32 * b + l32] = ea[b];
    }

    convert_a(RA[0], 0);
    load_a(D, RA[0]);
    __syncthreads();                             // sh_ea, activation batch 0

    // Batch bt + u: its weights against its activations (LDS buffer u & 1);
    // then batch bt + u + 1's activations into the other buffer, which every
    // wavefront finished reading before the last barrier; then the loads of
    // batch bt + u + 1 + D's activations and bt + u + D's weights.
    for (int bt = 0; bt < nbat; bt += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            WBatch& B = R[u];
            // all of the batch's activation operands first (LDS latency
            // behind the weight conversion), then per slice the weight
            // operands and the MFMAs
            if constexpr (NCB > 0) {
            h8 fa[kSSlices][MB];
#pragma unroll
            for (int j = 0; j < kSSlices; ++j)
#pragma unroll
                for (int b = 0; b < MB; ++b) fa[j][b] = frag_read(sA[u & 1][b][j], lane);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                h2 s[NC1];
#pragma unroll
                for (int c = 0; c < NCB; ++c) s[c] = h16_scale(scale_of(B.wsc[c], g), eb[c]);
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int j = 4 * g + d;
#pragma unroll
                    for (int c = 0; c < NCB; ++c) {
                        const h8 fb = __builtin_bit_cast(h8, h16_codes(dword_of(B.w[c][g], d), s[c]));
#pragma unroll
                        for (int b = 0; b < MB; ++b)
                            acc[b][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[j][b], fb, acc[b][c], 0, 0, 0);
                    }
                }
            }
            }
            // (the scheduler keeps each batch's loads and uses in place: a
            // use moved ahead of later loads would wait for all of them)
            __builtin_amdgcn_sched_barrier(0);
            convert_a(RA[(u + 1) % D], (u + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            load_a(bt + u + 1 + D, RA[(u + 1) % D]);
            load_w(bt + u + D, B);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();                     // the next batch's activations written, this one's read
        }
    }

    // Epilogue: this wavefront's outputs without their shifts
#pragma unroll
    for (int c = 0; c < NCB; ++c) {
        const int col = 32 * (cb0 + c) + l32;
#pragma unroll
        for (int b = 0; b < MB; ++b) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int rl = 32 * b + 8 * (q >> 2) + 4 * half + (q & 3);
                const int e_row = sh_ea[rl];
                float v = __builtin_ldexpf(acc[b][c][q], -(e_row + eb[c]));
                if (e_row == kH16NonFinite || eb[c] == kH16NonFinite) v = __builtin_nanf("");
                if (rl < M && col < N) y[(size_t)rl * N + col] = f32_to_f16_bits(v);
            }
        }
    }
}

template <int MB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_h16s_kernel(const uint8_t* __restrict__ xq, const uint16_t* __restrict__ xs,
                      const uint8_t* __restrict__ wq, const uint16_t* __restrict__ ws, uint16_t* __restrict__ y,
                      int M, int N, int K) {
    // activation operands of a batch: [buffer][row block][slice][lane][16 B]
    __shared__ __align__(16) uint8_t sA[2][MB][kSSlices][64 * 16];
    __shared__ uint32_t sh_mx[2][MB * 32];
    __shared__ int sh_ea[MB * 32];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave == kSCols)
        h16s_wave<MB, 0, true>(xq, xs, wq, ws, y, M, N, K, 0, wave, sA, sh_mx, sh_ea);
    else
        h16s_wave<MB, 1, false>(xq, xs, wq, ws, y, M, N, K, blockIdx.x * kSCols + wave, wave, sA, sh_mx, sh_ea);
}

template <int MB>
int launch_h16s(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws, uint16_t* y, int M,
                int N, int K, hipStream_t stream) {
    const unsigned grid = (unsigned)((N + 32 * kSCols - 1) / (32 * kSCols));
    gemm_h16s_kernel<MB><<<grid, 64 * (kSCols + 1), 0, stream>>>(xq, xs, wq, ws, y, M, N, K);
    return (int)hipGetLastError();
}

}  // namespace

// Where it beats the int8 streaming kernel (measured on MI355X): above M =
// 32 (two 32-row activation blocks) and while the grid fills 7/8 to all of
// the 256 CUs in one round.  Llama-70B FFN (K = 8192, N = 57344), layer
// steps cycling three weight copies through HBM: M = 64 110 us against 119,
// M = 32 86 against 81; weights reused (partly cache-resident): M = 32 / 48
// / 64 76 / 95 / 96 us against 81 / 109 / 115, M = 16 73 against 64; N =
// 28672 (128 workgroups) 58 against 45, N = 65536 (293) 141 against 91.
// Lane offsets are 32-bit byte offsets into the code tensors; batches come
// in groups of kSDepth (K % 1024 == 0).
bool gemm_h16s_shape_ok(int64_t M, int64_t N, int64_t K) {
    constexpr int64_t kCUs = 256;
    const int64_t wgs = (N + 32 * kSCols - 1) / (32 * kSCols);
    return M > 32 && M <= 64 && 8 * wgs >= 7 * kCUs && wgs <= kCUs && K > 0 && K % (256 * kSDepth) == 0 &&
           N * (K / 2) <= 0xffffffffLL;
}

bool gemm_h16s_supported(int64_t M, int64_t N, int64_t K, const void* xs, const void* ws) {
    return gemm_h16s_shape_ok(M, N, K) &&
           ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(ws)) & 15u) == 0;
}

int launch_gemm_h16s(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws, uint16_t* y,
                     int M, int N, int K, hipStream_t stream) {
    if (!gemm_h16s_supported(M, N, K, xs, ws) ||
        ((reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq)) & 15u) != 0)
        return (int)hipErrorInvalidValue;
    return M > 32 ? launch_h16s<2>(xq, xs, wq, ws, y, M, N, K, stream)
                  : launch_h16s<1>(xq, xs, wq, ws, y, M, N, K, stream);
}

}  // namespace wush
