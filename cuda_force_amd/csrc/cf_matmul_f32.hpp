// Internal interface of the fp32 GEMM on the bf16 MFMA units
// (cf_matmul_f32.hip), used by cf_matmul and cf_matmul_tensor_core.
#pragma once

#include "cf_common.hpp"

namespace cf {

/// True when the kernel takes c[M, N] = a[M, K] @ b[K, N]: K and N multiples
/// of 4, a, b and c 16-byte aligned, 31-bit buffer offsets sufficient.
bool matmul_f32_eligible(const void* a, const void* b, const void* c, int64_t M, int64_t N, int64_t K);

/// Slices of the reduction range for this shape when a workspace is given
/// (1 when the output tiles alone fill the GPU).
int matmul_f32_splits(int64_t M, int64_t N, int64_t K);

/// Workspace for `splits` slices: their fp32 partial outputs (0 for one).
size_t matmul_f32_workspace_bytes(int64_t M, int64_t N, int splits);

/// c = a @ b in fp32, each operand split into bf16 high and low parts on its
/// way into LDS (three MFMA products per term). With splits > 1 the slices'
/// partial outputs go to `workspace` and a second launch sums them in slice
/// order.
cf_status launch_matmul_f32(const float* a, const float* b, float* c, int64_t M, int64_t N, int64_t K,
                            int splits, void* workspace, hipStream_t stream);

}  // namespace cf
