// Internal interface of the bf16 MFMA LoRA adapter backward (cf_lora_bwd.hip),
// used by cf_lora_backward in cf_lora.hip.
#pragma once

#include "cf_common.hpp"

namespace cf {

/// True when the MFMA backward takes this bf16 problem: 0 < rank <= 16,
/// K and N multiples of 8, 16-byte aligned x, dy and b, 31-bit offsets.
bool lora_backward_fast_eligible(const void* x, const void* dy, const void* b, int64_t M,
                                 int64_t K, int64_t N, int64_t rank);

/// Workspace bytes of launch_lora_backward_fast (256-byte aligned pieces).
size_t lora_backward_fast_workspace_bytes(int64_t M, int64_t K, int64_t N);

/// grad_a = scale * x^T bf16(dy b^T), grad_b = scale * bf16(xa)^T dy (bf16
/// outputs, fp32 accumulation, fixed-order sums).
cf_status launch_lora_backward_fast(const void* x, const void* dy, const void* b, const float* xa,
                                    void* grad_a, void* grad_b, int64_t M, int64_t K, int64_t N,
                                    int64_t rank, float scale, void* workspace,
                                    hipStream_t stream);

}  // namespace cf
