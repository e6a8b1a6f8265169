// Internal interface of the fused bf16 MFMA LoRA kernel (cf_lora_fused.hip),
// used by the C ABI entry points in cf_lora.hip.
#pragma once

#include "cf_common.hpp"

namespace cf {

/// True when the fused kernel takes this bf16 problem: K a multiple of 64,
/// N a multiple of 8, rank 0 or even and <= 16, 16-byte aligned x, w and b,
/// 4-byte aligned a, 31-bit buffer offsets sufficient.
bool lora_fused_eligible(const void* x, const void* w, const void* a, const void* b, int64_t M,
                         int64_t N, int64_t K, int64_t rank);

/// Bytes of workspace launch_lora_fused can use for an M-row problem of
/// rank `rank` (0 for rank 0): a flag and 8 KiB of bf16 x @ a per 256-row
/// tile, through which the column tiles of a row tile that start late take
/// x @ a from its first column tile instead of forming it again.
size_t lora_fused_workspace_bytes(int64_t M, int64_t rank);

/// y = x @ w + scale * bf16(x @ a) @ b in one launch (rank 0: y = x @ w);
/// writes the fp32 x @ a to xa_out when it is non-null. `workspace`, when
/// non-null, holds lora_fused_workspace_bytes(M, rank) bytes, 16-byte
/// aligned, in any state; the output is the same with or without it.
cf_status launch_lora_fused(const void* x, const void* w, const void* a, const void* b, void* y,
                            float* xa_out, int64_t M, int64_t N, int64_t K, int64_t rank,
                            float scale, void* workspace, hipStream_t stream);

/// y (fp32) = x @ w for bf16 x [M, K] and w [K, N] on the same kernel
/// (rank 0, fp32 stores); same eligibility as lora_fused_eligible with rank 0
/// and a 16-byte aligned y. With splits > 1 (K a multiple of 64 * splits)
/// the K range is cut into `splits` slices and y holds splits consecutive
/// [M, N] partial products, slice s's at y + s * M * N, for the caller to sum.
cf_status launch_matmul_bf16_f32out(const void* x, const void* w, float* y, int64_t M, int64_t N,
                                    int64_t K, int splits, hipStream_t stream);

}  // namespace cf
