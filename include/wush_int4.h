/*
 * wush_int4.h -- C ABI of the MI355X (gfx950) WUSH INT4 W4A4 library
 * (libwush_int4.so).
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream; it validates its arguments, enqueues its kernels on `stream` and
 * returns a hipError_t value (hipSuccess == 0).  Nothing here allocates:
 * outputs and the optional split-K workspace come from the caller, so every
 * call is safe under HIP graph capture.  Launches are asynchronous.
 *
 * Data formats (identical to the reference's my_int4._C tensors):
 *   codes  uint8, two signed INT4 codes per byte, element 2k in the low
 *          nibble, element 2k+1 in the high nibble (docs/SPEC.md:10-11;
 *          my_int4/rtn_int4.py:53-55); codes are in [-7, 7].
 *   scales bf16 bit patterns (uint16), one per 32-element group along K.
 *   T      bf16 (K/32, 32, 32): T[c][j][i], x'_j = sum_i x_i * T[c][j][i].
 *   y      fp16 bit patterns (uint16), row-major (M, N).
 * Bad arguments return hipErrorInvalidValue and launch nothing.
 *
 * Citations are to files of the reference repository (rib12316/WUSH_int4_kernel).
 */
#ifndef WUSH_INT4_H
#define WUSH_INT4_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WUSH_INT4_ABI_VERSION 1

/* Element type of the activations handed to wush_quant_int4. */
enum wush_dtype {
    WUSH_DTYPE_BF16 = 0,
    WUSH_DTYPE_F16 = 1,
    WUSH_DTYPE_F32 = 2
};

/* ABI version of the loaded library (WUSH_INT4_ABI_VERSION). */
int wush_abi_version(void);

/* One-time set-up of every visible device: the prefill kernel's dynamic LDS
 * limit (a function attribute) and the decode GEMV's occupancy table.  Call
 * it once before capturing any entry point in a HIP graph (the torch module
 * calls it at import).  An entry point called on a device that was not set up
 * runs the set-up there first, which sets a function attribute and so must not
 * happen during a capture.  Thread-safe; returns the first error, or
 * hipSuccess.  Replaces the reference's lazy static-flag attribute set-up
 * (csrc/gemm_cutlass_int4.cu:62-67, :111-119). */
int wush_init(void);

/* Text for a status returned by any entry point. */
const char *wush_error_string(int status);

/* Group-wise sigma-clip INT4 quantization, bit-exact with the reference.
 * x: n_groups*32 contiguous values of type `dtype`; q: n_groups*16 bytes;
 * s: n_groups bf16 scales.
 * Replaces quant_int4() in csrc/quant_int4.cu:109-134 (bf16 input, bound at
 * csrc/bindings.cpp:38) and, for fp16/fp32 input, the torch reference
 * my_int4/rtn_int4.py:33-55. */
int wush_quant_int4(const void *x, int dtype, uint8_t *q, uint16_t *s,
                    int64_t n_groups, hipStream_t stream);

/* WUSH block-diagonal transform fused with the quantization, bit-exact with
 * the reference's sequential form: x'_j = sum_i x_i*T[c][j][i] (fp32, i
 * ascending, every product and sum rounded), then wush_quant_int4's math on
 * x'.  x: rows*K bf16; t: (K/32)*1024 bf16; q: rows*K/2; s: rows*K/32.
 * Replaces fused_transform_quant_int4 (csrc/fused_tq_int4.cu:87-118) and the
 * _smallm / _v3 / _wmma variants (csrc/fused_tq_smallm.cu:89-121,
 * csrc/fused_tq_v3.cu:109-140, csrc/fused_tq_wmma.cu:131-162), which share
 * its contract (csrc/bindings.cpp:60-68). */
int wush_fused_tq(const uint16_t *x, const uint16_t *t, uint8_t *q, uint16_t *s,
                  int64_t rows, int64_t K, hipStream_t stream);

/* The transform stage of wush_fused_tq's rows kernel alone, for one block:
 * x'[r][j] = sum_i x[r][i] * t[j][i] (fp32, i ascending, every sum rounded),
 * x rows*32 bf16, t 32*32 bf16, xp rows*32 fp32.  Runs the same code path as
 * wush_fused_tq for the same values (fp32 MFMA steps, fma loop or mul-then-add
 * loop, chosen per 64 rows).  No counterpart in the reference, whose transform
 * is internal to fused_transform_quant_int4 (csrc/fused_tq_int4.cu:38-84): it
 * lets tests compare x' itself, which the codes and scales see only near a
 * rounding boundary. */
int wush_fused_tq_transform32(const uint16_t *x, const uint16_t *t, float *xp, int64_t rows,
                              hipStream_t stream);

/* Decode GEMV for 1 <= M <= 8: y[m][n] = sum_g sx[m][g]*sw[n][g]*D[m][n][g]
 * with D the exact int32 dot of group g.  xq: M*K/2; xs: M*K/32; wq: N*K/2;
 * ws: N*K/32; y: M*N fp16.  Shapes that wush_gemv_int4_supported rejects
 * return hipErrorInvalidValue (wush_gemm_s4 takes any shape).
 * Replaces w4a4_gemv (csrc/gemv_int4.cu:191-223, M == 1) and w4a4_gemv_multi
 * (csrc/gemv_int4.cu:145-189, M <= 8). */
int wush_gemv_int4(const uint8_t *xq, const uint16_t *xs, const uint8_t *wq, const uint16_t *ws,
                   uint16_t *y, int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* 1 if wush_gemv_int4 runs (M, N, K), else 0.  The rule depends on the
 * library's build (its tuning macros): 1 <= M <= 8, K % 32 == 0, and either
 * the activations fit the staged kernel's 64 KiB of LDS (M*K/2 + M*K/4
 * bytes) or the shape is one of the K-split kernel's (by default M = 7, 8,
 * K a multiple of 2048 in [8192, 32768], N > 32768), which keeps them in
 * registers.  A host that routes products between wush_gemv_int4 and
 * wush_gemm_s4 asks this instead of restating the rule.  The reference has
 * no counterpart: its w4a4_gemv_multi checks M <= 8 and fails at launch when
 * its shared memory does not fit (csrc/gemv_int4.cu:160-169). */
int wush_gemv_int4_supported(int64_t M, int64_t N, int64_t K);

/* Bytes of workspace wush_gemm_s4 uses for (M, N, K); 0 when it needs none:
 * fp32 split-K partials, and for prefill shapes with N >= 8192 the
 * activations converted once to fp16 operands (M*K*2 bytes, padded to 256
 * rows).  A caller may pass a larger buffer; a smaller one makes wush_gemm_s4
 * choose a plan that needs no more than it is given (same results). */
size_t wush_gemm_s4_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* Group-scaled W4A4 GEMM, any M >= 1, K % 32 == 0: the product of
 * wush_gemv_int4, y (M, N) fp16.  On int8 MFMA with exact int32 group dots,
 * except for prefill shapes (K % 256 == 0, M > 128, at least 64 tiles of
 * 256x256 or N >= 2048, and at least 128 workgroups counting the K slices of
 * at least 32 groups each that the workspace holds from M = 512), for
 * 64 < M <= 256 with N >= 8192 when the workspace holds the converted
 * activations (128-row tiles, at least 192 workgroups with at most 2 K slices
 * of at least 64 groups), and for 32 < M <= 64 with 49953 <= N <= 57344 and
 * K % 1024 == 0 (16-byte aligned codes and scales), which run fp16 MFMA on
 * code*scale operands (exact after
 * a power-of-two shift per row and column) accumulated in fp32 over all of K.
 * Both agree with the fp64 product to 2e-3 relative Frobenius (tested); a row
 * or column with a non-finite scale gives NaN there.
 * Replaces w4a4_gemm_s4 (csrc/gemm_s4.cu:320-379) and the superseded
 * w4a4_gemm / _v1 / _v2 (csrc/gemm_int4.cu:89-130, csrc/gemm_wmma.cu:128-172,
 * csrc/gemm_wmma2.cu:141-181) that compute the same product. */
int wush_gemm_s4(const uint8_t *xq, const uint16_t *xs, const uint8_t *wq, const uint16_t *ws,
                 uint16_t *y, int64_t M, int64_t N, int64_t K,
                 void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Bytes of the static split-K scratch that wush_gemm_s4_noalloc uses: one
 * array per device, held from the library's load until the process ends. */
#define WUSH_GEMM_SCRATCH_BYTES (64u << 20)

/* Status of wush_gemm_s4_noalloc if no plan of the shape fits
 * WUSH_GEMM_SCRATCH_BYTES (wush_error_string explains it).  The planner
 * always has one (a single K slice needs no scratch), so this is a guard. */
#define WUSH_ERROR_SCRATCH_TOO_SMALL 0x57550001

/* wush_gemm_s4 that allocates nothing and takes no workspace: its split-K
 * partials (if the plan splits K) go to the library's static scratch of
 * WUSH_GEMM_SCRATCH_BYTES on the current device.  The plan is the one
 * wush_gemm_s4 chooses for a workspace of WUSH_GEMM_SCRATCH_BYTES that holds
 * split-K partials only, and the results are those of such a call, bit for
 * bit: a shape whose full split of K would need more partials than the
 * scratch holds is split into fewer slices.  The scratch never holds
 * converted activations, so where wush_gemm_s4 with a workspace converts them
 * once (N >= 8192 at M > 64, on enough workgroups) this entry point runs the
 * per-tile fp16 tiles or the int8 tiles: equal to the parity tolerance, not
 * bit for bit.  Nothing needs clearing
 * between calls: every partial is written before it is summed.  All calls on
 * one device share its scratch, so calls that overlap on one device (on
 * different streams, or from different host threads without ordering) race.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture that must not call hipMalloc, tight
 * serving loops, harnesses that forbid allocation). */
int wush_gemm_s4_noalloc(const uint8_t *xq, const uint16_t *xs, const uint8_t *wq, const uint16_t *ws,
                         uint16_t *y, int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* Self-test of the int8 MFMA operand layout the GEMM relies on:
 * c (8x8 int32) = a (8x32 int8, row-major) @ b (32x8 int8, row-major).
 * Replaces s4_atom_selftest (csrc/gemm_s4.cu:74-82). */
int wush_mfma_selftest(const int8_t *a, const int8_t *b, int32_t *c, hipStream_t stream);

/* Per-tensor INT4 quantization: code = clamp(rint(x * inv_scale), -7, 7),
 * packed like the group codes, n bf16 values (n % 32 == 0) -> n/2 bytes.
 * inv_scale_dev, when not NULL, is a device pointer to the fp32 inverse
 * scale and overrides inv_scale.
 * Replaces quant_int4_tensor_scale / _dev (csrc/fast_path.cu:42-59, :92-109). */
int wush_quant_int4_tensor_scale(const uint16_t *x, uint8_t *q, int64_t n, float inv_scale,
                                 const float *inv_scale_dev, hipStream_t stream);

/* Largest K of wush_gemm_s4_tensor_scale: the int8 MFMA multiplies 16*code
 * operands, so the int32 accumulator holds 256 * sum(qx*qw), up to
 * 256 * 64 * K with codes of -8; 256 * 64 * 131040 < 2^31. */
#define WUSH_TENSOR_SCALE_MAX_K 131040

/* Per-tensor W4A4 GEMM: y = alpha * (xq @ wq^T) with an exact int32 dot over
 * all of K, y (M, N) fp16, K % 32 == 0, K <= WUSH_TENSOR_SCALE_MAX_K (larger K
 * is rejected with hipErrorInvalidValue).  alpha_dev, when not NULL, is a
 * device pointer to the fp32 alpha and overrides alpha.
 * Replaces w4a4_gemm_cutlass / _dev (csrc/gemm_cutlass_int4.cu:132-188). */
int wush_gemm_s4_tensor_scale(const uint8_t *xq, const uint8_t *wq, uint16_t *y,
                              int64_t M, int64_t N, int64_t K, float alpha,
                              const float *alpha_dev, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* WUSH_INT4_H */
