// gemm_h16.h -- launcher of the fp16-MFMA prefill GEMM (gemm_h16.hip), called
// by the planner in gemm_s4.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace wush {

// LDS bytes of one workgroup (the launcher raises the kernel's dynamic LDS
// limit to this once).
size_t gemm_h16_smem_bytes();

// y = group-scaled product, M x N fp16, for M, N >= 1 and K % 256 == 0 (code
// tensors 16-byte aligned, scales 2-byte aligned).  splits > 1 splits K into
// slices of groups_per_split groups (a multiple of 8) and writes fp32 partials
// [split][M][N] to partial instead of y (the caller sums them).
// hipErrorInvalidValue for arguments outside these limits.
int launch_gemm_h16(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                    uint16_t* y, float* partial, int M, int N, int K, int splits, int groups_per_split,
                    hipStream_t stream);

// The same product with the activations converted once into a workspace of
// gemm_h16a_workspace_bytes(M, N, K, splits) bytes (a_ws, 16-byte aligned) by a
// first kernel (with every weight column's shift), then DMA'd into LDS by
// launch_gemm_h16q.  The same fp16 operands as launch_gemm_h16, summed in
// another K order within blocks of four groups: equal to fp32 rounding.
// Needs 16-byte aligned scale tensors.  rows128: 128-row output tiles
// (for 64 < M <= 128) instead of 256-row ones.
size_t gemm_h16a_workspace_bytes(int64_t M, int64_t N, int64_t K, int splits);
int launch_gemm_h16a(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws,
                     uint16_t* y, float* partial, int M, int N, int K, int splits, int groups_per_split,
                     void* a_ws, bool rows128, hipStream_t stream);

// The GEMM stage of launch_gemm_h16a, one wavefront per SIMD (gemm_h16q.hip):
// a16 / ea / eb as h16_prep_a_kernel leaves them; arguments checked there.
int launch_gemm_h16q(const uint8_t* a16, const int* ea, const int* eb, const uint8_t* wq, const uint16_t* ws,
                     uint16_t* y, float* partial, int M, int N, int K, int groups_per_split, int splits,
                     bool rows128, hipStream_t stream);

// The product for 32 < M <= 64 on weight matrices whose 224-column blocks
// fill the GPU in one round (gemm_h16s.hip; the rule is gemm_h16s_shape_ok):
// fp16 operands as above, the weights streamed once, no workspace.  Needs
// K % 1024 == 0 and 16-byte aligned code and scale tensors.
bool gemm_h16s_shape_ok(int64_t M, int64_t N, int64_t K);
bool gemm_h16s_supported(int64_t M, int64_t N, int64_t K, const void* xs, const void* ws);
int launch_gemm_h16s(const uint8_t* xq, const uint16_t* xs, const uint8_t* wq, const uint16_t* ws, uint16_t* y,
                     int M, int N, int K, hipStream_t stream);

}  // namespace wush
