// Internal interface of the fp32 LoRA linear on the bf16 MFMA units
// (cf_lora_f32.hip), used by the C ABI entry points in cf_lora.hip.
#pragma once

#include "cf_common.hpp"

namespace cf {

/// True when the fp32 MFMA kernel takes this problem: rank <= 16, K and N
/// multiples of 4, x, w, b and y 16-byte aligned, a 4-byte aligned, 31-bit
/// buffer offsets sufficient.
bool lora_f32_eligible(const void* x, const void* w, const void* a, const void* b, const void* y,
                       int64_t M, int64_t N, int64_t K, int64_t rank);

/// Slices of the reduction range the kernel uses for this shape when a
/// workspace is available (1 when the output alone fills the GPU).
int lora_f32_splits(int64_t M, int64_t N, int64_t K);

/// Workspace for `splits` slices: fp32 partial outputs and partial x @ a
/// (0 for one slice).
size_t lora_f32_workspace_bytes(int64_t M, int64_t N, int64_t rank, int splits);

/// y = x @ w + scale * (x @ a) @ b in fp32 on the MFMA units; writes the fp32
/// x @ a to xa_out when it is non-null. With splits > 1 the reduction range is
/// cut into slices whose partial results go to `workspace` and are summed in
/// slice order by a second launch.
cf_status launch_lora_f32(const float* x, const float* w, const float* a, const float* b, float* y,
                          float* xa_out, int64_t M, int64_t N, int64_t K, int64_t rank, float scale,
                          int splits, void* workspace, hipStream_t stream);

}  // namespace cf
