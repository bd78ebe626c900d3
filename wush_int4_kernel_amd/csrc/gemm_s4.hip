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
// returns 256*D; the 2^-8 is applied once at the output.  D is folded into an
// fp32 accumulator with the fp32 product of the two bf16 group scales
// (exact: 8-bit x 8-bit significands): acc = fma(float(D), sx*sw, acc).
//
// Workgroup = 4 wavefronts in a WAVES_M x WAVES_N grid, each wavefront owns a
// (32*BM) x (32*BN) output tile.  K advances 4 groups (64 code bytes per row)
// per stage through a double-buffered LDS tile laid out fragment-major,
// [group][k-half][row][8 B], so the MFMA operand reads (lane = row, 8 B) are
// conflict-free.  Skinny M uses split-K: each K slice writes fp32 partials to
// a caller-provided workspace and a second kernel sums the slices in a fixed
// order (deterministic, graph-capturable, no atomics, no memset).
#include "wush_device.h"
#include "../../include/wush_int4.h"

namespace wush {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kStageGroups = 4;                  // groups per LDS stage
constexpr int kPlanePad = 32;                    // bytes of padding per (group, half) plane

template <int TM, int TN>
struct GemmSmem {
    static constexpr int kAPlane = TM * 8 + kPlanePad;
    static constexpr int kBPlane = TN * 8 + kPlanePad;
    static constexpr int kACodes = kStageGroups * 2 * kAPlane;
    static constexpr int kBCodes = kStageGroups * 2 * kBPlane;
    static constexpr int kAScale = kStageGroups * TM * 4;
    static constexpr int kBScale = kStageGroups * TN * 4;
    static constexpr int kBuf = kACodes + kBCodes + kAScale + kBScale;
    static constexpr int kBytes = 2 * kBuf;
};

// Global -> register prefetch of one stage, spread over the 256 threads.
template <int TM, int TN>
struct StageRegs {
    static constexpr int kAChunks = (TM * kStageGroups + 255) / 256;
    static constexpr int kBChunks = (TN * kStageGroups + 255) / 256;
    static constexpr int kAScal = (TM * kStageGroups + 255) / 256;
    static constexpr int kBScal = (TN * kStageGroups + 255) / 256;
    uint4 a[kAChunks];
    uint4 b[kBChunks];
    float sa[kAScal];
    float sb[kBScal];
};

template <int BM, int BN, int WAVES_M, int WAVES_N, bool PER_TENSOR>
__global__ __launch_bounds__(256) void gemm_s4_kernel(const uint8_t* __restrict__ xq,
                                                      const uint16_t* __restrict__ xs,
                                                      const uint8_t* __restrict__ wq,
                                                      const uint16_t* __restrict__ ws,
                                                      uint16_t* __restrict__ y,
                                                      float* __restrict__ partial,
                                                      int M, int N, int K, int groups_per_split,
                                                      float alpha, const float* __restrict__ alpha_dev) {
    static_assert(WAVES_M * WAVES_N == 4, "4 wavefronts per workgroup");
    constexpr int TM = 32 * BM * WAVES_M;
    constexpr int TN = 32 * BN * WAVES_N;
    using S = GemmSmem<TM, TN>;
    using R = StageRegs<TM, TN>;
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
    const int n_stages = (g_end - g_begin + kStageGroups - 1) / kStageGroups;

    auto load_stage = [&](int st, R& r) {
        const int gs = g_begin + st * kStageGroups;
#pragma unroll
        for (int c = 0; c < R::kAChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id >> 2, g = id & 3;
            const int gm = m0 + row, gg = gs + g;
            r.a[c] = (row < TM && gm < M && gg < g_end)
                         ? *reinterpret_cast<const uint4*>(xq + (size_t)gm * K2 + (size_t)gg * 16)
                         : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < R::kBChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id >> 2, g = id & 3;
            const int gn = n0 + row, gg = gs + g;
            r.b[c] = (row < TN && gn < N && gg < g_end)
                         ? load_nt16(wq + (size_t)gn * K2 + (size_t)gg * 16)
                         : make_uint4(0, 0, 0, 0);
        }
        if constexpr (!PER_TENSOR) {
#pragma unroll
            for (int c = 0; c < R::kAScal; ++c) {
                const int id = tid + c * 256;
                const int row = id >> 2, g = id & 3;
                const int gm = m0 + row, gg = gs + g;
                r.sa[c] = (row < TM && gm < M && gg < g_end) ? bf16_to_f32(xs[(size_t)gm * G + gg]) : 0.0f;
            }
#pragma unroll
            for (int c = 0; c < R::kBScal; ++c) {
                const int id = tid + c * 256;
                const int row = id >> 2, g = id & 3;
                const int gn = n0 + row, gg = gs + g;
                r.sb[c] = (row < TN && gn < N && gg < g_end) ? bf16_to_f32(ws[(size_t)gn * G + gg]) : 0.0f;
            }
        }
    };

    auto store_stage = [&](int buf, const R& r) {
        uint8_t* base = smem + buf * S::kBuf;
#pragma unroll
        for (int c = 0; c < R::kAChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id >> 2, g = id & 3;
            if (row < TM) {
                uint2* p0 = reinterpret_cast<uint2*>(base + (g * 2 + 0) * S::kAPlane + row * 8);
                uint2* p1 = reinterpret_cast<uint2*>(base + (g * 2 + 1) * S::kAPlane + row * 8);
                *p0 = make_uint2(r.a[c].x, r.a[c].y);
                *p1 = make_uint2(r.a[c].z, r.a[c].w);
            }
        }
        uint8_t* bbase = base + S::kACodes;
#pragma unroll
        for (int c = 0; c < R::kBChunks; ++c) {
            const int id = tid + c * 256;
            const int row = id >> 2, g = id & 3;
            if (row < TN) {
                uint2* p0 = reinterpret_cast<uint2*>(bbase + (g * 2 + 0) * S::kBPlane + row * 8);
                uint2* p1 = reinterpret_cast<uint2*>(bbase + (g * 2 + 1) * S::kBPlane + row * 8);
                *p0 = make_uint2(r.b[c].x, r.b[c].y);
                *p1 = make_uint2(r.b[c].z, r.b[c].w);
            }
        }
        if constexpr (!PER_TENSOR) {
            float* sa = reinterpret_cast<float*>(base + S::kACodes + S::kBCodes);
            float* sbp = sa + kStageGroups * TM;
#pragma unroll
            for (int c = 0; c < R::kAScal; ++c) {
                const int id = tid + c * 256;
                const int row = id >> 2, g = id & 3;
                if (row < TM) sa[g * TM + row] = r.sa[c];
            }
#pragma unroll
            for (int c = 0; c < R::kBScal; ++c) {
                const int id = tid + c * 256;
                const int row = id >> 2, g = id & 3;
                if (row < TN) sbp[g * TN + row] = r.sb[c];
            }
        }
    };

    // Accumulators: fp32 (group-scaled) or int32 (per-tensor, whole K).
    float acc[BM][BN][16];
    v16i iacc[BM][BN];
#pragma unroll
    for (int bm = 0; bm < BM; ++bm)
#pragma unroll
        for (int bn = 0; bn < BN; ++bn) {
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[bm][bn][j] = 0.0f;
            iacc[bm][bn] = (v16i){0};
        }

    auto compute_stage = [&](int buf, int st) {
        const uint8_t* base = smem + buf * S::kBuf;
        const uint8_t* bbase = base + S::kACodes;
        const float* sa = reinterpret_cast<const float*>(base + S::kACodes + S::kBCodes);
        const float* sbp = sa + kStageGroups * TM;
        const int groups_here = min(kStageGroups, g_end - (g_begin + st * kStageGroups));
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) {
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
                float swv[BN];
#pragma unroll
                for (int bn = 0; bn < BN; ++bn) swv[bn] = sbp[g * TN + wn + bn * 32 + l32];
#pragma unroll
                for (int bm = 0; bm < BM; ++bm) {
                    // rows of this lane: 8*(j/4) + 4*half + (j%4), j = 0..15
                    float sxv[16];
#pragma unroll
                    for (int jb = 0; jb < 4; ++jb) {
                        const float4 v = *reinterpret_cast<const float4*>(
                            sa + g * TM + wm + bm * 32 + jb * 8 + half * 4);
                        sxv[jb * 4 + 0] = v.x;
                        sxv[jb * 4 + 1] = v.y;
                        sxv[jb * 4 + 2] = v.z;
                        sxv[jb * 4 + 3] = v.w;
                    }
#pragma unroll
                    for (int bn = 0; bn < BN; ++bn) {
                        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[bm], bfr[bn],
                                                                             (v16i){0}, 0, 0, 0);
#pragma unroll
                        for (int j = 0; j < 16; ++j)
                            acc[bm][bn][j] = __builtin_fmaf((float)d[j], sxv[j] * swv[bn], acc[bm][bn][j]);
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

    // Epilogue.  The MFMA ran on 16*code operands: scale by 2^-8.
    float out_scale = 1.0f / 256.0f;
    if constexpr (PER_TENSOR) out_scale = (alpha_dev ? *alpha_dev : alpha) * (1.0f / 256.0f);
#pragma unroll
    for (int bm = 0; bm < BM; ++bm)
#pragma unroll
        for (int bn = 0; bn < BN; ++bn) {
            const int col = n0 + wn + bn * 32 + l32;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
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
    int cfg;        // 0: 32x128 (skinny), 1: 64x128, 2: 128x128
    int splits;
    int groups_per_split;
    int tm, tn;
};

static Plan make_plan(int64_t M, int64_t N, int64_t K, size_t ws_bytes_available, bool allow_split) {
    Plan p;
    if (M <= 32) {
        p.cfg = 0; p.tm = 32; p.tn = 128;
    } else if (M <= 64) {
        p.cfg = 1; p.tm = 64; p.tn = 128;
    } else {
        p.cfg = 2; p.tm = 128; p.tn = 128;
    }
    const int64_t G = K / 32;
    const int64_t tiles = ((M + p.tm - 1) / p.tm) * ((N + p.tn - 1) / p.tn);
    int s = 1;
    if (allow_split) {
        // Aim for >= 2 workgroups per CU (256 CUs) while each slice keeps
        // at least 8 stages of K.
        while (s < 16 && tiles * s < 512 && G / (2 * s) >= 8 * kStageGroups) s *= 2;
    }
    int64_t gps = (G + s - 1) / s;
    gps = (gps + kStageGroups - 1) / kStageGroups * kStageGroups;
    s = (int)((G + gps - 1) / gps);
    if (s > 1 && (size_t)s * (size_t)M * (size_t)N * sizeof(float) > ws_bytes_available) {
        s = 1;
        gps = G;
    }
    p.splits = s;
    p.groups_per_split = (int)gps;
    return p;
}

template <int BM, int BN, int WM, int WN, bool PT>
static void launch_gemm(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                        uint16_t* y, float* partial, int M, int N, int K, const Plan& p, float alpha,
                        const float* alpha_dev, hipStream_t stream) {
    constexpr int TM = 32 * BM * WM, TN = 32 * BN * WN;
    const size_t smem = GemmSmem<TM, TN>::kBytes;
    dim3 grid((unsigned)((N + TN - 1) / TN), (unsigned)((M + TM - 1) / TM), (unsigned)p.splits);
    gemm_s4_kernel<BM, BN, WM, WN, PT><<<grid, 256, smem, stream>>>(
        xq, xs, wq, ws, y, partial, M, N, K, p.groups_per_split, alpha, alpha_dev);
}

template <bool PT>
static int run_gemm(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                    uint16_t* y, int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes,
                    float alpha, const float* alpha_dev, hipStream_t stream) {
    const Plan p = make_plan(M, N, K, workspace ? ws_bytes : 0, !PT);
    WUSH_REQUIRE((N + p.tn - 1) / p.tn <= 0x7fffffffLL && (M + p.tm - 1) / p.tm <= 65535);
    float* partial = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const int m = (int)M, n = (int)N, k = (int)K;
    switch (p.cfg) {
        case 0: launch_gemm<1, 1, 1, 4, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream); break;
        case 1: launch_gemm<1, 2, 2, 2, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream); break;
        default: launch_gemm<2, 2, 2, 2, PT>(xq, xs, wq, ws, y, partial, m, n, k, p, alpha, alpha_dev, stream); break;
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
    const wush::Plan p = wush::make_plan(M, N, K, (size_t)-1, true);
    return p.splits > 1 ? (size_t)p.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
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

int wush_gemm_s4_tensor_scale(const uint8_t* xq, const uint8_t* wq, uint16_t* y, int64_t M, int64_t N,
                              int64_t K, float alpha, const float* alpha_dev, hipStream_t stream) {
    WUSH_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 32 == 0);
    WUSH_REQUIRE(M <= 0x7fffffffLL && N <= 0x7fffffffLL && K <= (1LL << 20));
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
