// gemv.hip -- decode W4A4 GEMV for 1 <= M <= 8 (csrc/gemv_int4.cu:23-223).
//
//   y[m][n] = sum_g sx[m][g] * sw[n][g] * D[m][n][g],
//   D[m][n][g] = sum_{k in g} qx[m][k] * qw[n][k]   (exact int32)
//
// A pure HBM-streaming kernel: no MFMA.  The packed activations (M*K/2 bytes)
// and their scales are staged once per workgroup in LDS; every wavefront then
// streams whole weight rows: lane l takes groups l, l+64, ... so each load
// instruction of a wavefront reads 1 KiB of contiguous codes (16 B per lane)
// and 128 B of contiguous scales.  The group dot is 4 v_dot8_i32_i4 on the
// packed nibbles as stored (element 2k low nibble pairs with element 2k low
// nibble).  The fold is one cvt + one mul + one fma in fp32 at M = 1; for
// M >= 2 the dot starts from the bits of 1.5*2^23, so two fmas fold it
// without a conversion (see kMagicBits).  A chunk of R
// weight rows (R = 1 at M = 1, else 2) is reduced over the wavefront at once:
// the R x M partial sums go through a recursive-halving reduction (permlane
// swaps and DPP, VALU only) that costs about two operations per output.  The
// next chunk is requested before the current one is reduced, so each lane
// keeps 2 x R x (K/2048) 16-byte loads outstanding.  At M = 7, 8 on long
// rows (K % 2048 == 0, N > 32768) gemv_ks_kernel takes the product instead:
// the K of a row is split over the wavefronts of a workgroup and every lane
// keeps its group's activations in registers.
#include "wush_device.h"
#include "setup.h"
#include "../../include/wush_int4.h"

namespace wush {

// Tuning knobs (defaults measured at K=8192 N=57344 and K=4096 N=24576).
#ifndef WUSH_GEMV_WAVES
#define WUSH_GEMV_WAVES 4       // wavefronts per workgroup at M = 1 (2 / 8 / 16 no better)
#endif
#ifndef WUSH_GEMV_WAVES_M
#define WUSH_GEMV_WAVES_M 16    // ... for M >= 2: the staged activations (M*K*3/4 bytes of
#endif                          // LDS) are shared by 16 wavefronts (L70 M=8: 51.5 vs 53.5 us)
#ifndef WUSH_GEMV_WAVES_M78
#define WUSH_GEMV_WAVES_M78 WUSH_GEMV_WAVES_M  // ... for M = 7, 8 (8 or 4 were slower with 1 row)
#endif
template <int M>
constexpr int gemv_waves() { return M == 1 ? WUSH_GEMV_WAVES : M >= 7 ? WUSH_GEMV_WAVES_M78 : WUSH_GEMV_WAVES_M; }
#ifndef WUSH_GEMV_TBAR
#define WUSH_GEMV_TBAR 1        // scheduling barrier after each group (fewer live VGPRs)
#endif
#ifndef WUSH_GEMV_R1
#define WUSH_GEMV_R1 1          // weight rows per chunk at M = 1 (measured best)
#endif
#ifndef WUSH_GEMV_R2
#define WUSH_GEMV_R2 2          // ... at M = 2
#endif
#ifndef WUSH_GEMV_R4
#define WUSH_GEMV_R4 2          // ... at M = 3, 4
#endif
#ifndef WUSH_GEMV_R8
#define WUSH_GEMV_R8 2          // ... at M = 5, 6
#endif
#ifndef WUSH_GEMV_R78
#define WUSH_GEMV_R78 1         // ... at M = 7, 8 (L70 M=8: 48.3 us with 1 row, 51.4 with 2)
#endif

// dot32_s4 with the start value in an SGPR: the first v_dot8 reads it as its
// third operand (the compiler would copy it to a VGPR per chain otherwise).
__device__ __forceinline__ int dot32_s4_s(const uint4& a, const uint4& b, int init_s) {
    int d;
    asm("v_dot8_i32_i4 %0, %1, %2, %3" : "=v"(d) : "v"(a.x), "v"(b.x), "s"(init_s));
    d = __builtin_amdgcn_sdot8((int)a.y, (int)b.y, d, false);
    d = __builtin_amdgcn_sdot8((int)a.z, (int)b.z, d, false);
    d = __builtin_amdgcn_sdot8((int)a.w, (int)b.w, d, false);
    return d;
}

__device__ __forceinline__ int dot32_s4(const uint4& a, const uint4& b, int init = 0) {
    int d = __builtin_amdgcn_sdot8((int)a.x, (int)b.x, init, false);
    d = __builtin_amdgcn_sdot8((int)a.y, (int)b.y, d, false);
    d = __builtin_amdgcn_sdot8((int)a.z, (int)b.z, d, false);
    d = __builtin_amdgcn_sdot8((int)a.w, (int)b.w, d, false);
    return d;
}

// One wavefront streams the weight rows [n_begin, n_end), R rows at a time.
// GPL = groups per lane (K/2048): when it is known at compile time all R*GPL
// 16-byte weight loads of a chunk are issued together and the next chunk is
// prefetched while the current one is reduced, so ~2*R*GPL KiB stay in flight
// per wavefront.  The first chunk is requested before the activations are
// staged in LDS (weights do not depend on them).  GPL == 0 is the generic
// any-K loop.
template <int R, int GPL>
struct GemvChunk {
    uint4 w[R][GPL];
    uint32_t s[R][GPL];
};

constexpr int pow2_ceil(int v) { return v <= 1 ? 1 : 2 * pow2_ceil((v + 1) / 2); }

// Reduce the R x M per-lane partial sums over the wavefront and store the
// fp16 outputs of rows n0 .. n0+R-1.  All reductions happen before the one
// store branch (a store branch per output lets the compiler sink later
// outputs' dot products past it and keep every group's activations live).
template <int M, int R>
__device__ __forceinline__ void store_outputs(const float (&acc)[R][M], int lane, int n0, int n_end, int N,
                                              uint16_t* __restrict__ y) {
    constexpr int V = pow2_ceil(R * M);
    if constexpr (V > 1) {
        // recursive-halving reduce-scatter: about 2V VALU operations for V outputs
        float v[V];
#pragma unroll
        for (int i = 0; i < V; ++i) v[i] = i < R * M ? acc[i / M][i % M] : 0.0f;
        const float total = wave_reduce_scatter<V>(v, lane);
        const int idx = wave_rs_index<V>(lane);
        const int r = idx / M, m = idx % M;
        if ((lane & (64 / V - 1)) == 0 && idx < R * M && n0 + r < n_end)
            y[(size_t)m * N + n0 + r] = f32_to_f16_bits(total);
    } else {
        const float total = wave_sum_dpp(acc[0][0]);
        if (lane == 0 && n0 < n_end) y[n0] = f32_to_f16_bits(total);
    }
}

// Fold without an int -> float conversion (M >= 2): the dot products start
// from kMagicBits, the bits of kMagic = 1.5 * 2^23, so the int32 result read
// as a float is kMagic + dot exactly (|dot| <= 1568).
constexpr int kMagicBits = 0x4B400000;
constexpr float kMagic = 12582912.0f;

// Activation scales for which the conversion-free fold is exact: finite and
// |sx| <= 2^60, so -kMagic*sx is exact and finite.
__device__ __forceinline__ bool scale_in_range(float s) { return __builtin_fabsf(s) <= 0x1p60f; }

// Activation scales in LDS: sx at M = 1 (plain fold), (sx, -kMagic*sx) for
// M >= 2.
template <int M> struct XsStageT { using type = float2; };
template <> struct XsStageT<1> { using type = float; };
template <int M> using XsStage = typename XsStageT<M>::type;
__device__ __forceinline__ float xs_at(const float* xs_l, int i) { return xs_l[i]; }
__device__ __forceinline__ float xs_at(const float2* xs_l, int i) { return xs_l[i].x; }

// Stage the activation codes and scales in LDS; for M >= 2 returns whether
// every sx of the block is in range (block-uniform).
template <int M>
__device__ __forceinline__ bool stage_activations(const uint8_t* __restrict__ xq, const uint16_t* __restrict__ xs,
                                                  uint4* xq_l, XsStage<M>* xs_l, int G) {
    const uint4* xq4 = reinterpret_cast<const uint4*>(xq);
    for (int i = threadIdx.x; i < M * G; i += blockDim.x) xq_l[i] = xq4[i];
    if constexpr (M == 1) {
        for (int i = threadIdx.x; i < G; i += blockDim.x) xs_l[i] = bf16_to_f32(xs[i]);
        __syncthreads();
        return false;
    } else {
        int bad = 0;
        for (int i = threadIdx.x; i < M * G; i += blockDim.x) {
            const float sx = bf16_to_f32(xs[i]);
            xs_l[i] = make_float2(sx, -kMagic * sx);
            bad |= !scale_in_range(sx);
        }
        return !__syncthreads_or(bad);
    }
}

template <int M, int R, int GPL>
__global__ __launch_bounds__(64 * gemv_waves<M>()) void gemv_int4_kernel(const uint8_t* __restrict__ xq,
                                                        const uint16_t* __restrict__ xs,
                                                        const uint8_t* __restrict__ wq,
                                                        const uint16_t* __restrict__ ws,
                                                        uint16_t* __restrict__ y, int N, int K,
                                                        int rows_per_wave) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int G = K >> 5;
    const int K2 = K >> 1;
    using XS = XsStage<M>;
    uint4* xq_l = reinterpret_cast<uint4*>(smem);                       // [M][G] x 16 B
    XS* xs_l = reinterpret_cast<XS*>(smem + (size_t)M * K2);            // [M][G]

    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int n_begin = (blockIdx.x * gemv_waves<M>() + wave) * rows_per_wave;
    const int n_step = R;
    const int n_end = min(N, n_begin + rows_per_wave);

    if constexpr (GPL > 0) {
        using Chunk = GemvChunk<R, GPL>;
        auto load = [&](int n0, Chunk& c) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = max(0, min(n0 + r, n_end - 1));   // clamp: duplicate rows are never stored
                // wave-uniform row base plus the lane's 32-bit offset
                const global_cptr<uint8_t> wrow = uniform_ptr(wq + (size_t)n * K2);
                const global_cptr<uint16_t> srow = uniform_ptr(ws + (size_t)n * G);
#pragma unroll
                for (int t = 0; t < GPL; ++t) {
                    uint32_t wo = (uint32_t)(lane + 64 * t) * 16u;
                    asm("" : "+v"(wo));          // keeps the 32-bit lane offset form
                    const u32x4 wv = __builtin_nontemporal_load(reinterpret_cast<global_cptr<u32x4>>(wrow + wo));
                    c.w[r][t] = make_uint4(wv.x, wv.y, wv.z, wv.w);
                    c.s[r][t] = srow[(uint32_t)(lane + 64 * t)];
                }
            }
        };
        Chunk cur, nxt;
        if (n_begin < n_end) load(n_begin, cur);
        int magic;
        asm("s_mov_b32 %0, %1" : "=s"(magic) : "n"(kMagicBits));   // kMagicBits in an SGPR (see dot32_s4_s)

        const bool x_in_range = stage_activations<M>(xq, xs, xq_l, xs_l, G);

        for (int n0 = n_begin; n0 < n_end; n0 += n_step) {
            const bool more = n0 + n_step < n_end;
            if (more) load(n0 + n_step, nxt);
            __builtin_amdgcn_sched_barrier(0);
            float acc[R][M];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
            if (M > 1 && x_in_range) {
                if constexpr (M > 1) {
                // d' = kMagicBits + dot, read as a float, is kMagic + dot
                // exactly, so fma(d', sx, -kMagic*sx) = dot*sx exactly (at most
                // 19 significant bits) without a conversion, and fma(dot*sx, sw,
                // acc) rounds dot*sx*sw + acc once, like fma(dot, sx*sw, acc)
                // with its exact bf16 x bf16 factor: one VALU operation fewer
                // per output.
#pragma unroll
                for (int t = 0; t < GPL; ++t) {
                    const int g = lane + 64 * t;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const uint4 xv = xq_l[m * G + g];
                        const float2 sx2 = xs_l[m * G + g];
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const int d = dot32_s4_s(cur.w[r][t], xv, magic);
                            const float v = __builtin_fmaf(__int_as_float(d), sx2.x, sx2.y);
                            acc[r][m] = __builtin_fmaf(v, bf16_to_f32(cur.s[r][t]), acc[r][m]);
                        }
                    }
#if WUSH_GEMV_TBAR
                    // keep one group's activations live at a time (M x 24 B per lane)
                    __builtin_amdgcn_sched_barrier(0);
#endif
                }
                }
            } else {
#pragma unroll
                for (int t = 0; t < GPL; ++t) {
                    const int g = lane + 64 * t;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const uint4 xv = xq_l[m * G + g];
                        const float sxv = xs_at(xs_l, m * G + g);
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const int d = dot32_s4(cur.w[r][t], xv);
                            acc[r][m] = __builtin_fmaf((float)d, sxv * bf16_to_f32(cur.s[r][t]), acc[r][m]);
                        }
                    }
#if WUSH_GEMV_TBAR
                    if constexpr (M > 1) __builtin_amdgcn_sched_barrier(0);
#endif
                }
            }
            store_outputs<M, R>(acc, lane, n0, n_end, N, y);
            if (more) cur = nxt;
        }
    } else {
        (void)stage_activations<M>(xq, xs, xq_l, xs_l, G);
        for (int n0 = n_begin; n0 < n_end; n0 += n_step) {
            float acc[R][M];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
            for (int g = lane; g < G; g += 64) {
                uint4 wv[R];
                float swv[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int n = min(n0 + r, n_end - 1);
                    wv[r] = load_nt16(wq + (size_t)n * K2 + (size_t)g * 16);
                    swv[r] = bf16_to_f32(ws[(size_t)n * G + g]);
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const uint4 xv = xq_l[m * G + g];
                    const float sxv = xs_at(xs_l, m * G + g);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const int d = dot32_s4(wv[r], xv);
                        acc[r][m] = __builtin_fmaf((float)d, sxv * swv[r], acc[r][m]);
                    }
                }
            }
            store_outputs<M, R>(acc, lane, n0, n_end, N, y);
        }
    }
}

// ------------------------------------------------ K-split GEMV, 5 <= M <= 8
// For K % (2048 * GL) == 0: a workgroup of KS = K/(2048*GL) wavefronts streams
// a range of weight rows; wavefront q takes groups 64(GL*q + t) + lane
// (t < GL), so each row is read in loads of 1 KiB contiguous codes (and 128 B
// of scales), and every lane keeps its GL groups' M activation codes and
// scale terms in registers for the whole kernel -- no LDS activation reads per
// row (which cost ~12 us at L70 M=8 in the staged kernel above).  GL = 1 is
// built (GL = 2 halves the per-row reductions but needs 198 VGPRs at M=8 and
// measured within 2%).  Rows go through a ring of kKsRing 16-byte loads per
// lane, addressed as a wave-uniform row base (SGPRs) plus the lane's 32-bit
// offset, and the first ring is requested before the activations.  Per row,
// the M partial sums (one group per lane, so each is the single rounding of
// dot*sx*sw) are reduced over the wavefront by recursive halving into an LDS
// table [row][wavefront][m]; after the last row one barrier, and the KS
// wavefront partials of each output are added in wavefront order and stored.
// A row costs 71 VALU instructions at M=8 (32 v_dot8, 16 fma, 23 for the
// reduction and the row's scale; no per-chain v_mov of the start value and no
// per-row address arithmetic: L70 M=8 46.9 against 50.2 us before).
#ifndef WUSH_GEMV_KS_RING
#define WUSH_GEMV_KS_RING 8
#endif
constexpr int kKsRing = WUSH_GEMV_KS_RING;        // rows in flight per wavefront
#ifndef WUSH_GEMV_KS_MIN_M
#define WUSH_GEMV_KS_MIN_M 7     // smallest M of the K-split kernel (9: off)
#endif
#ifndef WUSH_GEMV_KS_MIN_WAVES
#define WUSH_GEMV_KS_MIN_WAVES 4 // ... and of K / 2048 (its wavefronts per workgroup)
#endif
#ifndef WUSH_GEMV_KS_GL
#define WUSH_GEMV_KS_GL 1        // groups per lane (K / (2048 * GL) wavefronts per workgroup)
#endif
constexpr int kKsGl = WUSH_GEMV_KS_GL;
#ifndef WUSH_GEMV_KS_MIN_N
#define WUSH_GEMV_KS_MIN_N 32769 // ... and of N (K=8192 N=28672 M=8: 30.2 us against 27.9 staged)
#endif
constexpr int kGemvKsMinM = WUSH_GEMV_KS_MIN_M;
constexpr size_t kGemvKsLds = 32 * 1024;          // bytes of the partial-sum table per workgroup
// K % 2048 == 0 and at most 16 wavefronts per workgroup
__host__ __device__ constexpr bool gemv_ks_shape(int64_t N, int64_t K) {
    return N >= WUSH_GEMV_KS_MIN_N && K % (2048 * kKsGl) == 0 && K / 2048 >= WUSH_GEMV_KS_MIN_WAVES &&
           K / (2048 * kKsGl) <= (kKsGl == 1 ? 16 : 4);
}

template <int M, int GL>
__global__ __launch_bounds__(GL == 1 ? 1024 : 256) void gemv_ks_kernel(const uint8_t* __restrict__ xq,
                                                       const uint16_t* __restrict__ xs,
                                                       const uint8_t* __restrict__ wq,
                                                       const uint16_t* __restrict__ ws,
                                                       uint16_t* __restrict__ y, int N, int K,
                                                       int rows_per_wg) {
    // [rows_per_wg][KS * M + 1]: the pad word puts consecutive rows of one
    // output index in different banks for the summing loop below (without it
    // their stride was KS * M = 32 words, one bank for a whole half-wavefront)
    extern __shared__ __align__(16) float part[];
    const int KS = blockDim.x >> 6;
    const int RP = KS * M + 1;                       // words per row of the partial table
    const int G = K >> 5;
    const int K2 = K >> 1;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int n_begin = blockIdx.x * rows_per_wg;
    const int n_end = min(N, n_begin + rows_per_wg);
    const int cnt = n_end - n_begin;                 // >= 1: the grid covers N exactly

    // Row r of the range: a wave-uniform base (SGPR arithmetic per row) plus
    // the lane's 32-bit offset, so a row costs no VALU address arithmetic.
    const uint8_t* wbase = wq + (size_t)n_begin * K2 + (size_t)(64 * GL * wave) * 16;
    const uint16_t* sbase = ws + (size_t)n_begin * G + 64 * GL * wave;
    const uint32_t woff = (uint32_t)lane * 16u;
    uint4 rw[kKsRing][GL];
    uint32_t rs[kKsRing][GL];
    auto load = [&](int i, int d) {
        const int r = min(i, cnt - 1);           // rows past the range re-read the last one (not stored)
#pragma unroll
        for (int t = 0; t < GL; ++t) {
            uint32_t wo = woff;
            asm("" : "+v"(wo));                  // keeps the 32-bit lane offset form (no hoisted 64-bit add)
            const global_cptr<u32x4> wp =
                reinterpret_cast<global_cptr<u32x4>>(uniform_ptr(wbase + ((size_t)r * K2 + t * 1024)) + wo);
            const u32x4 wv = __builtin_nontemporal_load(wp);
            rw[d][t] = make_uint4(wv.x, wv.y, wv.z, wv.w);
            rs[d][t] = uniform_ptr(sbase + ((size_t)r * G + t * 64))[(uint32_t)lane];
        }
    };
    // the first rows are requested before the activations: weights do not
    // depend on them, and the range check below waits for the scales
#pragma unroll
    for (int d = 0; d < kKsRing; ++d) load(d, d);
    __builtin_amdgcn_sched_barrier(0);

    // this lane's GL groups (64 * (GL * wave + t) + lane) of every activation
    // row; d' = kMagicBits + dot read as a float is kMagic + dot, so
    // fma(d', sx, -kMagic*sx) = dot*sx exactly
    uint4 xa[GL][M];
    float sx[GL][M], nmx[GL][M];
    bool ok = true;
#pragma unroll
    for (int t = 0; t < GL; ++t) {
        const int g = 64 * (GL * wave + t) + lane;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            xa[t][m] = *reinterpret_cast<const uint4*>(xq + (size_t)m * K2 + (size_t)g * 16);
            sx[t][m] = bf16_to_f32(xs[(size_t)m * G + g]);
            nmx[t][m] = -kMagic * sx[t][m];
            ok = ok && scale_in_range(sx[t][m]);
        }
    }
    const bool fast = __builtin_amdgcn_ballot_w64(!ok) == 0;

    constexpr int V = pow2_ceil(M);
    const int idx = wave_rs_index<V>(lane);
    const bool holder = (lane & (64 / V - 1)) == 0 && idx < M;
    // The magic start value as a wave-uniform operand: the first v_dot8 of
    // each chain reads it from an SGPR instead of a per-row v_mov.
    int magic;
    asm("s_mov_b32 %0, %1" : "=s"(magic) : "n"(kMagicBits));   // kMagicBits in an SGPR (see dot32_s4_s)
    if (fast) {
        for (int i0 = 0; i0 < cnt; i0 += kKsRing) {
#pragma unroll
            for (int d = 0; d < kKsRing; ++d) {
                const int i = i0 + d;
                float v[V];
#pragma unroll
                for (int m = 0; m < V; ++m) v[m] = 0.0f;
#pragma unroll
                for (int t = 0; t < GL; ++t) {
                    const float sw = bf16_to_f32(rs[d][t]);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const int dot = dot32_s4_s(rw[d][t], xa[t][m], magic);
                        v[m] = __builtin_fmaf(__builtin_fmaf(__int_as_float(dot), sx[t][m], nmx[t][m]), sw, v[m]);
                    }
                }
                load(i + kKsRing, d);
                const float total = wave_reduce_scatter<V>(v, lane);
                if (holder && i < cnt) part[i * RP + wave * M + idx] = total;
            }
        }
    } else {
        // A scale outside the conversion-free range (rare): fma((float)dot,
        // sx*sw, .), one row at a time with its own loads, so this form adds
        // nothing to the register budget of the one above.  The prefetched
        // ring is only waited for here (which keeps its loads ahead of the
        // activation range check on both paths).
#pragma unroll
        for (int d = 0; d < kKsRing; ++d)
#pragma unroll
            for (int t = 0; t < GL; ++t) asm volatile("" ::"v"(rw[d][t].x), "v"(rs[d][t]));
        for (int i = 0; i < cnt; ++i) {
            float v[V];
#pragma unroll
            for (int m = 0; m < V; ++m) v[m] = 0.0f;
#pragma unroll
            for (int t = 0; t < GL; ++t) {
                const uint4 wv = load_nt16(wbase + ((size_t)i * K2 + t * 1024) + woff);
                const float sw = bf16_to_f32(sbase[((size_t)i * G + t * 64) + (uint32_t)lane]);
#pragma unroll
                for (int m = 0; m < M; ++m)
                    v[m] = __builtin_fmaf((float)dot32_s4(wv, xa[t][m]), sx[t][m] * sw, v[m]);
            }
            const float total = wave_reduce_scatter<V>(v, lane);
            if (holder) part[i * RP + wave * M + idx] = total;
        }
    }
    __syncthreads();
    // outputs of the range: add the KS partials in wavefront order
    for (int o = threadIdx.x; o < M * cnt; o += blockDim.x) {
        const int m = o / cnt, i = o - m * cnt;
        float acc = part[i * RP + m];
        for (int q = 1; q < KS; ++q) acc += part[i * RP + q * M + m];
        y[(size_t)m * N + n_begin + i] = f32_to_f16_bits(acc);
    }
}

// Register-limited workgroups per CU of every kernel instance and the
// device's LDS per CU and CU count, per device, filled by gemv_init_device
// (the library's one-time set-up) before any launch.
constexpr int kGemvGpl[3] = {0, 2, 4};
struct GemvDeviceInfo {
    int blocks_by_regs[8][3];                    // [M - 1][GPL index]
    int ks_waves_per_cu[8];                      // gemv_ks_kernel<M, GL>: register-limited wavefronts per CU
    int lds_per_cu;
    int cus;
};
static GemvDeviceInfo g_gemv_info[kMaxDevices];

template <int M>
constexpr int gemv_rows() {
    return M == 1 ? WUSH_GEMV_R1 : M == 2 ? WUSH_GEMV_R2 : M <= 4 ? WUSH_GEMV_R4 : M <= 6 ? WUSH_GEMV_R8 : WUSH_GEMV_R78;
}

template <int M, int GI>
static int gemv_query(GemvDeviceInfo& info) {
    constexpr int R = gemv_rows<M>();
    constexpr int GPL = kGemvGpl[GI];
    int b = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, gemv_int4_kernel<M, R, GPL>,
                                                                      64 * gemv_waves<M>(), 0);
    if (e != hipSuccess) return (int)e;
    info.blocks_by_regs[M - 1][GI] = b < 1 ? 1 : b;
    if constexpr (GI < 2) return gemv_query<M, GI + 1>(info);
    else if constexpr (M < 8) return gemv_query<M + 1, 0>(info);
    else return 0;
}

template <int M>
static int gemv_ks_query(GemvDeviceInfo& info) {
    if constexpr (M <= 8) {
        int b = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, gemv_ks_kernel<M, kKsGl>, 256, 0);
        if (e != hipSuccess) return (int)e;
        info.ks_waves_per_cu[M - 1] = b < 1 ? 4 : 4 * b;
        return gemv_ks_query<M + 1>(info);
    }
    return 0;
}

int gemv_init_device(int dev) {
    GemvDeviceInfo& info = g_gemv_info[dev];
    if (hipDeviceGetAttribute(&info.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || info.cus < 1)
        info.cus = 256;
    if (hipDeviceGetAttribute(&info.lds_per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) !=
            hipSuccess || info.lds_per_cu < 65536)
        info.lds_per_cu = 65536;
    const int st = gemv_query<1, 0>(info);
    return st != 0 ? st : gemv_ks_query<kGemvKsMinM>(info);
}

template <int M, int GI>
static void launch_gemv_t(const GemvDeviceInfo& info, const uint8_t* xq, const uint16_t* xs, const uint8_t* wq,
                          const uint16_t* ws, uint16_t* y, int N, int K, hipStream_t stream) {
    constexpr int R = gemv_rows<M>();
    constexpr int GPL = kGemvGpl[GI];
    const int G = K / 32;
    const size_t smem = (size_t)M * (K / 2) + (size_t)M * G * sizeof(XsStage<M>);
    // Spread the rows evenly over the wavefronts that are resident at once
    // (workgroups per CU: the register limit and the LDS limit for this
    // smem), so every CU finishes together.
    constexpr int kGemvWaves = gemv_waves<M>();
    const int per_cu = max(1, min(info.blocks_by_regs[M - 1][GI], (int)(info.lds_per_cu / smem)));
    const int resident_waves = per_cu * kGemvWaves * info.cus;
    const int rows_per_wave = max((N + resident_waves - 1) / resident_waves, 1);
    const int blocks = (N + kGemvWaves * rows_per_wave - 1) / (kGemvWaves * rows_per_wave);
    gemv_int4_kernel<M, R, GPL><<<dim3(blocks), dim3(64 * kGemvWaves), smem, stream>>>(xq, xs, wq, ws, y, N, K,
                                                                                        rows_per_wave);
}

// K-split launch: KS = K/(2048*GL) wavefronts per workgroup, rows spread evenly
// over the workgroups resident at once (registers and LDS).
template <int M>
static void launch_gemv_ks(const GemvDeviceInfo& info, const uint8_t* xq, const uint16_t* xs, const uint8_t* wq,
                           const uint16_t* ws, uint16_t* y, int N, int K, hipStream_t stream) {
    const int KS = K / (2048 * kKsGl);
    const int per_cu = max(1, info.ks_waves_per_cu[M - 1] / KS);
    int rows = max(1, (N + per_cu * info.cus - 1) / (per_cu * info.cus));
    while ((size_t)rows * (KS * M + 1) * sizeof(float) > kGemvKsLds) rows = (rows + 1) / 2;
    const int blocks = (N + rows - 1) / rows;
    gemv_ks_kernel<M, kKsGl><<<dim3(blocks), dim3(64 * KS), (size_t)rows * (KS * M + 1) * sizeof(float), stream>>>(
        xq, xs, wq, ws, y, N, K, rows);
}

template <int M>
static void launch_gemv(const GemvDeviceInfo& info, const uint8_t* xq, const uint16_t* xs, const uint8_t* wq,
                        const uint16_t* ws, uint16_t* y, int N, int K, hipStream_t stream) {
    const int G = K / 32;
    if constexpr (M >= kGemvKsMinM) {
        if (gemv_ks_shape(N, K)) return launch_gemv_ks<M>(info, xq, xs, wq, ws, y, N, K, stream);
    }
    if (G == 128)
        launch_gemv_t<M, 1>(info, xq, xs, wq, ws, y, N, K, stream);
    else if (G == 256)
        launch_gemv_t<M, 2>(info, xq, xs, wq, ws, y, N, K, stream);
    else
        launch_gemv_t<M, 0>(info, xq, xs, wq, ws, y, N, K, stream);
}

namespace {
// The shapes wush_gemv_int4 runs: 1 <= M <= 8 and K % 32 == 0, with the
// staged kernel's activations (M*K/2 code bytes + M*K/32 pairs of fp32
// scale terms) in 64 KiB of LDS, or a shape of the K-split kernel (which
// stages nothing) at M >= kGemvKsMinM.  Both depend on the build's tuning
// macros, so callers ask the library (wush_gemv_int4_supported).
bool gemv_shape_supported(int64_t M, int64_t N, int64_t K) {
    if (M < 1 || M > 8 || N < 0 || K <= 0 || K % 32 != 0 || N > 0x7fffffffLL || K > 0x7fffffffLL) return false;
    const bool ksplit = M >= kGemvKsMinM && gemv_ks_shape(N, K);
    return ksplit || (size_t)M * (K / 2) + (size_t)M * (K / 32) * 8 <= 64 * 1024;
}
}  // namespace
}  // namespace wush

extern "C" int wush_gemv_int4_supported(int64_t M, int64_t N, int64_t K) {
    return wush::gemv_shape_supported(M, N, K) ? 1 : 0;
}

extern "C" int wush_gemv_int4(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq,
                              const uint16_t* ws, uint16_t* y, int64_t M, int64_t N, int64_t K,
                              hipStream_t stream) {
    WUSH_REQUIRE(M >= 1 && M <= 8 && N >= 0 && K > 0 && K % 32 == 0);
    WUSH_REQUIRE(N <= 0x7fffffffLL && K <= 0x7fffffffLL);
    if (N == 0) return (int)hipSuccess;
    WUSH_REQUIRE(xq && xs && wq && ws && y);
    WUSH_REQUIRE(((uintptr_t)xq & 15u) == 0 && ((uintptr_t)wq & 15u) == 0);
    WUSH_REQUIRE(((uintptr_t)xs & 1u) == 0 && ((uintptr_t)ws & 1u) == 0 && ((uintptr_t)y & 1u) == 0);
    WUSH_REQUIRE(wush::gemv_shape_supported(M, N, K));
    int dev = 0;
    const int st = wush::device_setup(&dev);
    if (st != 0) return st;
    const wush::GemvDeviceInfo& info = wush::g_gemv_info[dev];
    const int n = (int)N, k = (int)K;
    switch (M) {
        case 1: wush::launch_gemv<1>(info, xq, xs, wq, ws, y, n, k, stream); break;
        case 2: wush::launch_gemv<2>(info, xq, xs, wq, ws, y, n, k, stream); break;
        case 3: wush::launch_gemv<3>(info, xq, xs, wq, ws, y, n, k, stream); break;
        case 4: wush::launch_gemv<4>(info, xq, xs, wq, ws, y, n, k, stream); break;
        case 5: wush::launch_gemv<5>(info, xq, xs, wq, ws, y, n, k, stream); break;
        case 6: wush::launch_gemv<6>(info, xq, xs, wq, ws, y, n, k, stream); break;
        case 7: wush::launch_gemv<7>(info, xq, xs, wq, ws, y, n, k, stream); break;
        default: wush::launch_gemv<8>(info, xq, xs, wq, ws, y, n, k, stream); break;
    }
    return (int)hipGetLastError();
}
