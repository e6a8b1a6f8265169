// PyTorch-ROCm dispatcher registration for the cudaforge:: operators.
//
// Same namespace, the same ten schemas, the same Autograd guard list and the
// same CPU (ATen) implementations as the reference's extension
// (cpp/src/bindings.cpp:342-404), so code written against
// torch.ops.cudaforge.* runs unchanged. On ROCm a GPU tensor carries the CUDA
// dispatch key, so the GPU implementations register under CUDA; they call the
// C ABI of libcudaforge_hip.so on PyTorch's current HIP stream and never
// synchronise (bindings.cpp:56-63 does the same with the CUDA stream).
//
// Differences from the reference, all widening:
//   * the GPU implementations accept float32, bfloat16 and float16 where the
//     reference's accept float32 only (bindings.cpp:45-48); lora_linear takes
//     float32 and bfloat16;
//   * a few extra operators the Python layer uses: dequantize_int8_to (half
//     outputs), quantize_dequantize, softmax_as (output dtype),
//     softmax_scaled (scaled, causally masked attention scores), row_sum,
//     lora_linear_fwd / lora_linear_bwd for the adapter autograd path, and
//     attention_scores_causal / attention_pv_causal, the two causal attention
//     products of the transformer block.
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/autograd_not_implemented_fallback.h>
#include <torch/extension.h>

#include <limits>
#include <string>
#include <tuple>
#include <vector>

#include "cudaforge_hip.h"

namespace cudaforge_amd {
namespace {

// ---- shared checks ---------------------------------------------------------

void check_contiguous(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous; call .contiguous() first. ",
                "The kernels index rows as `base + row * cols`, which is only "
                "valid for a contiguous row-major layout.");
}

void check_2d(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.dim() == 2, name, " must be 2-D, got ", t.dim(), " dimensions");
}

cf_dtype to_cf(const torch::Tensor& t, const char* name) {
    switch (t.scalar_type()) {
        case torch::kFloat32:
            return CF_F32;
        case torch::kBFloat16:
            return CF_BF16;
        case torch::kFloat16:
            return CF_F16;
        default:
            TORCH_CHECK(false, name, " has dtype ", t.scalar_type(),
                        ", which has no HIP kernel (float32, bfloat16 or float16)");
    }
}

cf_dtype to_cf(torch::ScalarType type) {
    switch (type) {
        case torch::kFloat32:
            return CF_F32;
        case torch::kBFloat16:
            return CF_BF16;
        case torch::kFloat16:
            return CF_F16;
        default:
            TORCH_CHECK(false, "dtype ", type, " has no HIP kernel (float32, bfloat16 or float16)");
    }
}

void check_same_device(const torch::Tensor& a, const torch::Tensor& b, const char* name) {
    TORCH_CHECK(a.device() == b.device(), name, " is on ", b.device(), " but the input is on ",
                a.device());
}

/// PyTorch's current stream on the tensor's device, as the C ABI's void*.
void* stream_for(const torch::Tensor& t) {
    return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_status(cf_status status) {
    TORCH_CHECK(status == CF_OK, "cudaforge HIP kernel failed: ", cf_last_error());
}

// ---- GPU implementations -----------------------------------------------------

torch::Tensor rmsnorm_hip(const torch::Tensor& input, const torch::Tensor& weight, double eps) {
    check_2d(input, "input");
    check_contiguous(input, "input");
    check_contiguous(weight, "weight");
    check_same_device(input, weight, "weight");
    TORCH_CHECK(weight.dim() == 1, "weight must be 1-D, got ", weight.dim(), " dimensions");
    TORCH_CHECK(weight.size(0) == input.size(1), "weight length ", weight.size(0),
                " does not match the input's last dimension ", input.size(1));
    TORCH_CHECK(weight.scalar_type() == input.scalar_type(), "weight dtype ",
                weight.scalar_type(), " must match the input's ", input.scalar_type());
    const at::DeviceGuard guard(input.device());
    torch::Tensor output = torch::empty_like(input);
    check_status(cf_rmsnorm(input.data_ptr(), weight.data_ptr(), output.data_ptr(),
                            to_cf(input, "input"), input.size(0), input.size(1),
                            static_cast<float>(eps), stream_for(input)));
    return output;
}

torch::Tensor softmax_as_hip(const torch::Tensor& input, torch::ScalarType out_dtype) {
    check_2d(input, "input");
    check_contiguous(input, "input");
    const at::DeviceGuard guard(input.device());
    torch::Tensor output = torch::empty(input.sizes(), input.options().dtype(out_dtype));
    check_status(cf_softmax(input.data_ptr(), to_cf(input, "input"), output.data_ptr(),
                            to_cf(out_dtype), input.size(0), input.size(1), stream_for(input)));
    return output;
}

torch::Tensor softmax_hip(const torch::Tensor& input) {
    return softmax_as_hip(input, input.scalar_type());
}

torch::Tensor softmax_scaled_hip(const torch::Tensor& input, double scale, int64_t causal_period,
                                 torch::ScalarType out_dtype) {
    check_2d(input, "input");
    check_contiguous(input, "input");
    TORCH_CHECK(causal_period >= 0, "causal_period must be >= 0, got ", causal_period);
    const at::DeviceGuard guard(input.device());
    torch::Tensor output = torch::empty(input.sizes(), input.options().dtype(out_dtype));
    check_status(cf_softmax_scaled(input.data_ptr(), to_cf(input, "input"), output.data_ptr(),
                                   to_cf(out_dtype), input.size(0), input.size(1),
                                   static_cast<float>(scale), causal_period, stream_for(input)));
    return output;
}

// Causal attention products: q, k, v [batch, seq, heads * head_dim],
// probs [batch, heads, seq, seq].
void check_attention(const torch::Tensor& rows, int64_t heads, const char* name) {
    TORCH_CHECK(rows.dim() == 3, name, " must be [batch, seq, hidden], got ", rows.dim(), " dims");
    TORCH_CHECK(heads > 0 && rows.size(2) % heads == 0, "hidden ", rows.size(2), " is not divisible by heads ",
                heads);
}

torch::Tensor attention_scores_causal_hip(const torch::Tensor& q, const torch::Tensor& k, int64_t heads) {
    check_attention(q, heads, "q");
    TORCH_CHECK(k.sizes() == q.sizes(), "q and k differ in shape");
    TORCH_CHECK(k.scalar_type() == q.scalar_type(), "q and k differ in dtype");
    check_same_device(q, k, "k");
    check_contiguous(q, "q");
    check_contiguous(k, "k");
    const at::DeviceGuard guard(q.device());
    const int64_t batch = q.size(0), seq = q.size(1);
    torch::Tensor scores = torch::empty({batch, heads, seq, seq}, q.options());
    check_status(cf_attention_scores_causal(q.data_ptr(), k.data_ptr(), scores.data_ptr(), to_cf(q, "q"), batch,
                                            seq, heads, q.size(2) / heads, stream_for(q)));
    return scores;
}

torch::Tensor attention_pv_causal_hip(const torch::Tensor& probs, const torch::Tensor& v, int64_t heads) {
    check_attention(v, heads, "v");
    const int64_t batch = v.size(0), seq = v.size(1);
    TORCH_CHECK(probs.dim() == 4 && probs.size(0) == batch && probs.size(1) == heads && probs.size(2) == seq &&
                    probs.size(3) == seq,
                "probs must be [batch, heads, seq, seq] = [", batch, ", ", heads, ", ", seq, ", ", seq, "]");
    TORCH_CHECK(probs.scalar_type() == v.scalar_type(), "probs and v differ in dtype");
    check_same_device(v, probs, "probs");
    check_contiguous(probs, "probs");
    check_contiguous(v, "v");
    const at::DeviceGuard guard(v.device());
    torch::Tensor out = torch::empty(v.sizes(), v.options());
    check_status(cf_attention_pv_causal(probs.data_ptr(), v.data_ptr(), out.data_ptr(), to_cf(v, "v"), batch, seq,
                                        heads, v.size(2) / heads, stream_for(v)));
    return out;
}

std::tuple<torch::Tensor, torch::Tensor> lora_linear_fwd_hip(const torch::Tensor& x,
                                                             const torch::Tensor& w,
                                                             const torch::Tensor& a,
                                                             const torch::Tensor& b,
                                                             double scale) {
    check_2d(x, "x");
    check_2d(w, "w");
    check_2d(a, "a");
    check_2d(b, "b");
    for (const auto& [tensor, name] : std::vector<std::pair<torch::Tensor, const char*>>{
             {x, "x"}, {w, "w"}, {a, "a"}, {b, "b"}}) {
        check_contiguous(tensor, name);
        check_same_device(x, tensor, name);
        TORCH_CHECK(tensor.scalar_type() == x.scalar_type(), name, " has dtype ",
                    tensor.scalar_type(), " but x has ", x.scalar_type());
    }
    TORCH_CHECK(x.scalar_type() == torch::kFloat32 || x.scalar_type() == torch::kBFloat16,
                "lora_linear has HIP kernels for float32 and bfloat16, got ", x.scalar_type());
    const int64_t batch = x.size(0);
    const int64_t in_features = x.size(1);
    const int64_t out_features = w.size(1);
    const int64_t rank = a.size(1);
    TORCH_CHECK(w.size(0) == in_features, "w must be [in_features, out_features]; got [",
                w.size(0), ", ", w.size(1), "] for in_features=", in_features);
    TORCH_CHECK(a.size(0) == in_features, "a must be [in_features, rank]; got [", a.size(0), ", ",
                a.size(1), "] for in_features=", in_features);
    TORCH_CHECK(b.size(0) == rank && b.size(1) == out_features,
                "b must be [rank, out_features] = [", rank, ", ", out_features, "]; got [",
                b.size(0), ", ", b.size(1), "]");
    const at::DeviceGuard guard(x.device());
    torch::Tensor output = torch::empty({batch, out_features}, x.options());
    torch::Tensor xa = torch::empty({batch, rank}, x.options().dtype(torch::kFloat32));
    // Small fp32 problems split their reduction through a workspace from
    // torch's caching allocator (no synchronising hipMalloc).
    const size_t ws_bytes =
        cf_lora_linear_ws_bytes(to_cf(x, "x"), batch, in_features, out_features, rank);
    torch::Tensor workspace =
        torch::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)}, x.options().dtype(torch::kUInt8));
    check_status(cf_lora_linear_ws(x.data_ptr(), w.data_ptr(), a.data_ptr(), b.data_ptr(),
                                   output.data_ptr(), xa.data_ptr<float>(), to_cf(x, "x"), batch,
                                   in_features, out_features, rank, static_cast<float>(scale),
                                   ws_bytes > 0 ? workspace.data_ptr() : nullptr, ws_bytes,
                                   stream_for(x)));
    return {output, xa};
}

torch::Tensor lora_linear_hip(const torch::Tensor& x, const torch::Tensor& w,
                              const torch::Tensor& a, const torch::Tensor& b, double scale) {
    return std::get<0>(lora_linear_fwd_hip(x, w, a, b, scale));
}

std::tuple<torch::Tensor, torch::Tensor> lora_linear_bwd_hip(const torch::Tensor& x,
                                                             const torch::Tensor& dy,
                                                             const torch::Tensor& b,
                                                             const torch::Tensor& xa,
                                                             double scale) {
    check_2d(x, "x");
    check_2d(dy, "dy");
    check_2d(b, "b");
    check_2d(xa, "xa");
    for (const auto& [tensor, name] : std::vector<std::pair<torch::Tensor, const char*>>{
             {x, "x"}, {dy, "dy"}, {b, "b"}, {xa, "xa"}}) {
        check_contiguous(tensor, name);
        check_same_device(x, tensor, name);
    }
    TORCH_CHECK(dy.scalar_type() == x.scalar_type() && b.scalar_type() == x.scalar_type(),
                "x, dy and b must share a dtype");
    TORCH_CHECK(xa.scalar_type() == torch::kFloat32, "xa must be float32");
    const int64_t batch = x.size(0);
    const int64_t in_features = x.size(1);
    const int64_t rank = b.size(0);
    const int64_t out_features = b.size(1);
    TORCH_CHECK(dy.size(0) == batch && dy.size(1) == out_features, "dy must be [", batch, ", ",
                out_features, "]");
    TORCH_CHECK(xa.size(0) == batch && xa.size(1) == rank, "xa must be [", batch, ", ", rank, "]");
    const at::DeviceGuard guard(x.device());
    torch::Tensor grad_a = torch::empty({in_features, rank}, x.options());
    torch::Tensor grad_b = torch::empty({rank, out_features}, x.options());
    const size_t bytes = cf_lora_backward_workspace_bytes(batch, in_features, out_features, rank);
    torch::Tensor workspace =
        torch::empty({static_cast<int64_t>(bytes > 0 ? bytes : 1)}, x.options().dtype(torch::kUInt8));
    check_status(cf_lora_backward(x.data_ptr(), dy.data_ptr(), b.data_ptr(), xa.data_ptr<float>(),
                                  grad_a.data_ptr(), grad_b.data_ptr(), to_cf(x, "x"), batch,
                                  in_features, out_features, rank, static_cast<float>(scale),
                                  workspace.data_ptr(), bytes, stream_for(x)));
    return {grad_a, grad_b};
}

std::vector<torch::Tensor> fused_residual_rmsnorm_hip(const torch::Tensor& x,
                                                      const torch::Tensor& residual,
                                                      const torch::Tensor& weight, double eps) {
    check_2d(x, "x");
    check_contiguous(x, "x");
    check_contiguous(residual, "residual");
    check_contiguous(weight, "weight");
    check_same_device(x, residual, "residual");
    check_same_device(x, weight, "weight");
    TORCH_CHECK(x.sizes() == residual.sizes(), "x and residual must have the same shape, got ",
                x.sizes(), " and ", residual.sizes());
    TORCH_CHECK(weight.dim() == 1 && weight.size(0) == x.size(1), "weight must be 1-D of length ",
                x.size(1), ", got ", weight.sizes());
    TORCH_CHECK(residual.scalar_type() == x.scalar_type() &&
                    weight.scalar_type() == x.scalar_type(),
                "x, residual and weight must share a dtype");
    const at::DeviceGuard guard(x.device());
    torch::Tensor output = torch::empty_like(x);
    torch::Tensor residual_out = torch::empty_like(x);
    check_status(cf_fused_residual_rmsnorm(x.data_ptr(), residual.data_ptr(), weight.data_ptr(),
                                           output.data_ptr(), residual_out.data_ptr(),
                                           to_cf(x, "x"), x.size(0), x.size(1),
                                           static_cast<float>(eps), stream_for(x)));
    return {output, residual_out};
}

torch::Tensor silu_hip(const torch::Tensor& input) {
    check_contiguous(input, "input");
    const at::DeviceGuard guard(input.device());
    torch::Tensor output = torch::empty_like(input);
    check_status(cf_silu(input.data_ptr(), output.data_ptr(), to_cf(input, "input"),
                         input.numel(), stream_for(input)));
    return output;
}

torch::Tensor gelu_hip(const torch::Tensor& input) {
    check_contiguous(input, "input");
    const at::DeviceGuard guard(input.device());
    torch::Tensor output = torch::empty_like(input);
    check_status(cf_gelu(input.data_ptr(), output.data_ptr(), to_cf(input, "input"),
                         input.numel(), stream_for(input)));
    return output;
}

torch::Tensor swiglu_hip(const torch::Tensor& gate, const torch::Tensor& up) {
    check_contiguous(gate, "gate");
    check_contiguous(up, "up");
    check_same_device(gate, up, "up");
    TORCH_CHECK(gate.sizes() == up.sizes(), "gate and up must have the same shape, got ",
                gate.sizes(), " and ", up.sizes());
    TORCH_CHECK(gate.scalar_type() == up.scalar_type(), "gate and up must have the same dtype");
    const at::DeviceGuard guard(gate.device());
    torch::Tensor output = torch::empty_like(gate);
    check_status(cf_swiglu(gate.data_ptr(), up.data_ptr(), output.data_ptr(),
                           to_cf(gate, "gate"), gate.numel(), stream_for(gate)));
    return output;
}

torch::Tensor sum_hip(const torch::Tensor& input) {
    check_contiguous(input, "input");
    const at::DeviceGuard guard(input.device());
    const cf_dtype dtype = to_cf(input, "input");
    // accumulate = 0: the kernel writes the sum, so no fill is needed (and
    // none is recorded when the op is captured into a graph).
    const int64_t count = input.numel();
    if (count == 0) return torch::zeros({}, input.options());
    torch::Tensor out = torch::empty({1}, input.options().dtype(torch::kFloat32));
    {
        const size_t bytes = cf_reduce_sum_workspace_bytes(count);
        torch::Tensor workspace =
            torch::empty({static_cast<int64_t>(bytes)}, input.options().dtype(torch::kUInt8));
        check_status(cf_reduce_sum(input.data_ptr(), dtype, out.data_ptr<float>(), count,
                                   workspace.data_ptr(), bytes, /*accumulate=*/0,
                                   stream_for(input)));
    }
    return out.squeeze().to(input.scalar_type());
}

torch::Tensor row_sum_hip(const torch::Tensor& input) {
    check_2d(input, "input");
    check_contiguous(input, "input");
    const at::DeviceGuard guard(input.device());
    torch::Tensor out = torch::empty({input.size(0)}, input.options().dtype(torch::kFloat32));
    check_status(cf_row_sum(input.data_ptr(), to_cf(input, "input"), out.data_ptr<float>(),
                            input.size(0), input.size(1), stream_for(input)));
    return out;
}

std::vector<torch::Tensor> quantize_int8_hip(const torch::Tensor& input) {
    check_contiguous(input, "input");
    const at::DeviceGuard guard(input.device());
    const int64_t count = input.numel();
    torch::Tensor quantised = torch::empty({count}, input.options().dtype(torch::kInt8));
    torch::Tensor scales =
        torch::empty({cf_quant_scale_count(count)}, input.options().dtype(torch::kFloat32));
    check_status(cf_quantize_int8(input.data_ptr(), to_cf(input, "input"),
                                  quantised.data_ptr<int8_t>(), scales.data_ptr<float>(), count,
                                  stream_for(input)));
    return {quantised.view(input.sizes()), scales};
}

torch::Tensor dequantize_int8_to_hip(const torch::Tensor& quantised, const torch::Tensor& scales,
                                     torch::ScalarType out_dtype) {
    TORCH_CHECK(quantised.scalar_type() == torch::kInt8, "quantised must be int8");
    TORCH_CHECK(scales.scalar_type() == torch::kFloat32, "scales must be float32, got ",
                scales.scalar_type());
    check_contiguous(quantised, "quantised");
    check_contiguous(scales, "scales");
    check_same_device(quantised, scales, "scales");
    const int64_t count = quantised.numel();
    TORCH_CHECK(scales.numel() == cf_quant_scale_count(count), "expected ",
                cf_quant_scale_count(count), " block scales, got ", scales.numel());
    const at::DeviceGuard guard(quantised.device());
    torch::Tensor output = torch::empty(quantised.sizes(), scales.options().dtype(out_dtype));
    check_status(cf_dequantize_int8(quantised.data_ptr<int8_t>(), scales.data_ptr<float>(),
                                    output.data_ptr(), to_cf(out_dtype), count,
                                    stream_for(quantised)));
    return output;
}

torch::Tensor dequantize_int8_hip(const torch::Tensor& quantised, const torch::Tensor& scales) {
    return dequantize_int8_to_hip(quantised, scales, scales.scalar_type());
}

torch::Tensor quantize_dequantize_hip(const torch::Tensor& input) {
    check_contiguous(input, "input");
    const at::DeviceGuard guard(input.device());
    torch::Tensor output = torch::empty_like(input);
    check_status(cf_quantize_dequantize(input.data_ptr(), output.data_ptr(),
                                        to_cf(input, "input"), input.numel(),
                                        stream_for(input)));
    return output;
}

// ---- CPU implementations (ATen), as the reference's ----------------------------

torch::Tensor rmsnorm_cpu(const torch::Tensor& input, const torch::Tensor& weight, double eps) {
    check_2d(input, "input");
    TORCH_CHECK(weight.size(0) == input.size(1), "weight length ", weight.size(0),
                " does not match the input's last dimension ", input.size(1));
    const torch::Tensor promoted = input.to(torch::kFloat32);
    const torch::Tensor variance = promoted.pow(2).mean(-1, /*keepdim=*/true);
    const torch::Tensor normalised = promoted * torch::rsqrt(variance + eps);
    return (normalised * weight.to(torch::kFloat32)).to(input.scalar_type());
}

torch::Tensor softmax_cpu(const torch::Tensor& input) {
    check_2d(input, "input");
    return torch::softmax(input, /*dim=*/-1);
}

torch::Tensor softmax_as_cpu(const torch::Tensor& input, torch::ScalarType out_dtype) {
    check_2d(input, "input");
    return torch::softmax(input.to(torch::kFloat32), /*dim=*/-1).to(out_dtype);
}

torch::Tensor softmax_scaled_cpu(const torch::Tensor& input, double scale, int64_t causal_period,
                                 torch::ScalarType out_dtype) {
    check_2d(input, "input");
    TORCH_CHECK(causal_period >= 0, "causal_period must be >= 0, got ", causal_period);
    torch::Tensor logits = input.to(torch::kFloat32) * scale;
    if (causal_period > 0) {
        const auto options = torch::TensorOptions().dtype(torch::kLong).device(input.device());
        const torch::Tensor cols = torch::arange(input.size(1), options).unsqueeze(0);
        const torch::Tensor rows =
            torch::remainder(torch::arange(input.size(0), options), causal_period).unsqueeze(1);
        logits = logits.masked_fill(cols > rows, -std::numeric_limits<float>::infinity());
    }
    return torch::softmax(logits, /*dim=*/-1).to(out_dtype);
}

// The same products on the CPU: heads split out, the full q k^T (the
// kernel leaves the entries above the diagonal unspecified; these hold their
// dot products) and the lower triangle of probs times v.
torch::Tensor attention_scores_causal_cpu(const torch::Tensor& q, const torch::Tensor& k, int64_t heads) {
    check_attention(q, heads, "q");
    TORCH_CHECK(k.sizes() == q.sizes(), "q and k differ in shape");
    const int64_t batch = q.size(0), seq = q.size(1), d = q.size(2) / heads;
    const torch::Tensor qh = q.view({batch, seq, heads, d}).transpose(1, 2).to(torch::kFloat32);
    const torch::Tensor kh = k.view({batch, seq, heads, d}).transpose(1, 2).to(torch::kFloat32);
    return torch::matmul(qh, kh.transpose(-2, -1)).to(q.scalar_type());
}

torch::Tensor attention_pv_causal_cpu(const torch::Tensor& probs, const torch::Tensor& v, int64_t heads) {
    check_attention(v, heads, "v");
    const int64_t batch = v.size(0), seq = v.size(1), d = v.size(2) / heads;
    TORCH_CHECK(probs.dim() == 4 && probs.size(0) == batch && probs.size(1) == heads && probs.size(2) == seq &&
                    probs.size(3) == seq,
                "probs must be [batch, heads, seq, seq] = [", batch, ", ", heads, ", ", seq, ", ", seq, "]");
    const torch::Tensor vh = v.view({batch, seq, heads, d}).transpose(1, 2).to(torch::kFloat32);
    const torch::Tensor out = torch::matmul(torch::tril(probs.to(torch::kFloat32)), vh);
    return out.transpose(1, 2).reshape({batch, seq, heads * d}).to(v.scalar_type());
}

torch::Tensor lora_linear_cpu(const torch::Tensor& x, const torch::Tensor& w,
                              const torch::Tensor& a, const torch::Tensor& b, double scale) {
    return torch::matmul(x, w) + scale * torch::matmul(torch::matmul(x, a), b);
}

std::tuple<torch::Tensor, torch::Tensor> lora_linear_fwd_cpu(const torch::Tensor& x,
                                                             const torch::Tensor& w,
                                                             const torch::Tensor& a,
                                                             const torch::Tensor& b,
                                                             double scale) {
    const torch::Tensor xa = torch::matmul(x.to(torch::kFloat32), a.to(torch::kFloat32));
    const torch::Tensor y =
        torch::matmul(x, w) + scale * torch::matmul(xa.to(x.scalar_type()), b);
    return {y, xa};
}

std::tuple<torch::Tensor, torch::Tensor> lora_linear_bwd_cpu(const torch::Tensor& x,
                                                             const torch::Tensor& dy,
                                                             const torch::Tensor& b,
                                                             const torch::Tensor& xa,
                                                             double scale) {
    const auto type = x.scalar_type();
    const torch::Tensor xf = x.to(torch::kFloat32);
    const torch::Tensor dyf = dy.to(torch::kFloat32);
    const torch::Tensor g = torch::matmul(dyf, b.to(torch::kFloat32).t()).to(type).to(torch::kFloat32);
    const torch::Tensor grad_a = (scale * torch::matmul(xf.t(), g)).to(type);
    const torch::Tensor grad_b =
        (scale * torch::matmul(xa.to(type).to(torch::kFloat32).t(), dyf)).to(type);
    return {grad_a, grad_b};
}

torch::Tensor sum_cpu(const torch::Tensor& input) { return input.sum(); }

torch::Tensor row_sum_cpu(const torch::Tensor& input) {
    check_2d(input, "input");
    return input.to(torch::kFloat32).sum(-1);
}

std::vector<torch::Tensor> fused_residual_rmsnorm_cpu(const torch::Tensor& x,
                                                      const torch::Tensor& residual,
                                                      const torch::Tensor& weight, double eps) {
    TORCH_CHECK(x.sizes() == residual.sizes(), "x and residual must have the same shape, got ",
                x.sizes(), " and ", residual.sizes());
    const torch::Tensor summed = x + residual;
    return {rmsnorm_cpu(summed, weight, eps), summed};
}

torch::Tensor silu_cpu(const torch::Tensor& input) { return torch::silu(input); }

torch::Tensor gelu_cpu(const torch::Tensor& input) { return torch::gelu(input, "tanh"); }

torch::Tensor swiglu_cpu(const torch::Tensor& gate, const torch::Tensor& up) {
    TORCH_CHECK(gate.sizes() == up.sizes(), "gate and up must have the same shape, got ",
                gate.sizes(), " and ", up.sizes());
    if (gate.scalar_type() == torch::kHalf || gate.scalar_type() == torch::kBFloat16) {
        return (torch::silu(gate.to(torch::kFloat32)) * up.to(torch::kFloat32))
            .to(gate.scalar_type());
    }
    return torch::silu(gate) * up;
}

std::vector<torch::Tensor> quantize_int8_cpu(const torch::Tensor& input) {
    const int64_t count = input.numel();
    const int64_t block = 64;
    const int64_t blocks = (count + block - 1) / block;
    const torch::Tensor flat = input.reshape({-1}).to(torch::kFloat32);
    const torch::Tensor padded = torch::constant_pad_nd(flat, {0, blocks * block - count}, 0.0);
    const torch::Tensor grouped = padded.reshape({blocks, block});
    torch::Tensor scales = std::get<0>(grouped.abs().max(/*dim=*/1)) / 127.0;
    scales = torch::where(scales > 0, scales, torch::ones_like(scales));
    const torch::Tensor quantised =
        torch::clamp(torch::round(grouped / scales.unsqueeze(1)), -127, 127)
            .reshape({-1})
            .slice(0, 0, count)
            .to(torch::kInt8);
    return {quantised.view_as(input), scales};
}

torch::Tensor dequantize_int8_cpu(const torch::Tensor& quantised, const torch::Tensor& scales) {
    const int64_t count = quantised.numel();
    const int64_t block = 64;
    const int64_t blocks = (count + block - 1) / block;
    const torch::Tensor flat = quantised.reshape({-1}).to(torch::kFloat32);
    const torch::Tensor padded = torch::constant_pad_nd(flat, {0, blocks * block - count}, 0.0);
    const torch::Tensor grouped = padded.reshape({blocks, block});
    return (grouped * scales.unsqueeze(1)).reshape({-1}).slice(0, 0, count).view_as(quantised);
}

torch::Tensor dequantize_int8_to_cpu(const torch::Tensor& quantised, const torch::Tensor& scales,
                                     torch::ScalarType out_dtype) {
    return dequantize_int8_cpu(quantised, scales).to(out_dtype);
}

torch::Tensor quantize_dequantize_cpu(const torch::Tensor& input) {
    const auto parts = quantize_int8_cpu(input);
    return dequantize_int8_cpu(parts[0], parts[1]).to(input.scalar_type());
}

bool cuda_kernels_available() { return true; }

}  // namespace
}  // namespace cudaforge_amd

TORCH_LIBRARY(cudaforge, m) {
    // The reference's ten schemas, verbatim (cpp/src/bindings.cpp:342-355).
    m.def("rmsnorm(Tensor input, Tensor weight, float eps) -> Tensor");
    m.def("softmax(Tensor input) -> Tensor");
    m.def("lora_linear(Tensor x, Tensor w, Tensor a, Tensor b, float scale) -> Tensor");
    m.def("sum(Tensor input) -> Tensor");
    m.def("silu(Tensor input) -> Tensor");
    m.def("gelu(Tensor input) -> Tensor");
    m.def("swiglu(Tensor gate, Tensor up) -> Tensor");
    m.def(
        "fused_residual_rmsnorm(Tensor x, Tensor residual, Tensor weight, float eps) "
        "-> Tensor[]");
    m.def("quantize_int8(Tensor input) -> Tensor[]");
    m.def("dequantize_int8(Tensor quantised, Tensor scales) -> Tensor");
    // Extensions used by the Python layer.
    m.def("dequantize_int8_to(Tensor quantised, Tensor scales, ScalarType dtype) -> Tensor");
    m.def("quantize_dequantize(Tensor input) -> Tensor");
    m.def("softmax_as(Tensor input, ScalarType dtype) -> Tensor");
    m.def("softmax_scaled(Tensor input, float scale, int causal_period, ScalarType dtype) -> Tensor");
    m.def("row_sum(Tensor input) -> Tensor");
    m.def(
        "lora_linear_fwd(Tensor x, Tensor w, Tensor a, Tensor b, float scale) "
        "-> (Tensor, Tensor)");
    m.def(
        "lora_linear_bwd(Tensor x, Tensor dy, Tensor b, Tensor xa, float scale) "
        "-> (Tensor, Tensor)");
    m.def("attention_scores_causal(Tensor q, Tensor k, int heads) -> Tensor");
    m.def("attention_pv_causal(Tensor probs, Tensor v, int heads) -> Tensor");
}

// Inference-only operators raise on differentiation instead of silently
// producing wrong gradients; the same per-operator registration as the
// reference (bindings.cpp:369-377), extended to the extra operators.
// fused_residual_rmsnorm is left out, as it is there.
TORCH_LIBRARY_IMPL(cudaforge, Autograd, m) {
    for (const char* name :
         {"rmsnorm", "softmax", "lora_linear", "sum", "silu", "gelu", "swiglu", "quantize_int8",
          "dequantize_int8", "dequantize_int8_to", "quantize_dequantize", "softmax_as",
          "softmax_scaled", "row_sum", "lora_linear_fwd", "lora_linear_bwd", "attention_scores_causal",
          "attention_pv_causal"}) {
        m.impl(name, torch::autograd::autogradNotImplementedFallback());
    }
}

TORCH_LIBRARY_IMPL(cudaforge, CPU, m) {
    using namespace cudaforge_amd;
    m.impl("rmsnorm", &rmsnorm_cpu);
    m.impl("softmax", &softmax_cpu);
    m.impl("lora_linear", &lora_linear_cpu);
    m.impl("sum", &sum_cpu);
    m.impl("silu", &silu_cpu);
    m.impl("gelu", &gelu_cpu);
    m.impl("swiglu", &swiglu_cpu);
    m.impl("fused_residual_rmsnorm", &fused_residual_rmsnorm_cpu);
    m.impl("quantize_int8", &quantize_int8_cpu);
    m.impl("dequantize_int8", &dequantize_int8_cpu);
    m.impl("dequantize_int8_to", &dequantize_int8_to_cpu);
    m.impl("quantize_dequantize", &quantize_dequantize_cpu);
    m.impl("softmax_as", &softmax_as_cpu);
    m.impl("softmax_scaled", &softmax_scaled_cpu);
    m.impl("row_sum", &row_sum_cpu);
    m.impl("lora_linear_fwd", &lora_linear_fwd_cpu);
    m.impl("lora_linear_bwd", &lora_linear_bwd_cpu);
    m.impl("attention_scores_causal", &attention_scores_causal_cpu);
    m.impl("attention_pv_causal", &attention_pv_causal_cpu);
}

TORCH_LIBRARY_IMPL(cudaforge, CUDA, m) {
    using namespace cudaforge_amd;
    m.impl("rmsnorm", &rmsnorm_hip);
    m.impl("softmax", &softmax_hip);
    m.impl("lora_linear", &lora_linear_hip);
    m.impl("sum", &sum_hip);
    m.impl("silu", &silu_hip);
    m.impl("gelu", &gelu_hip);
    m.impl("swiglu", &swiglu_hip);
    m.impl("fused_residual_rmsnorm", &fused_residual_rmsnorm_hip);
    m.impl("quantize_int8", &quantize_int8_hip);
    m.impl("dequantize_int8", &dequantize_int8_hip);
    m.impl("dequantize_int8_to", &dequantize_int8_to_hip);
    m.impl("quantize_dequantize", &quantize_dequantize_hip);
    m.impl("softmax_as", &softmax_as_hip);
    m.impl("softmax_scaled", &softmax_scaled_hip);
    m.impl("row_sum", &row_sum_hip);
    m.impl("lora_linear_fwd", &lora_linear_fwd_hip);
    m.impl("lora_linear_bwd", &lora_linear_bwd_hip);
    m.impl("attention_scores_causal", &attention_scores_causal_hip);
    m.impl("attention_pv_causal", &attention_pv_causal_hip);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "cudaforge operators on MI355X (gfx950) HIP kernels";
    m.def("cuda_kernels_available", &cudaforge_amd::cuda_kernels_available,
          "True when the extension was compiled with its HIP kernels");
}
