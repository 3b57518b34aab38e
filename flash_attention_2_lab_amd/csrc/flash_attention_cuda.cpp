// PyTorch operator surface of the MI355X FlashAttention-2 library.
//
// Builds the Python module `flash_attention_cuda` with the reference's tensor-core
// attention entry points (reference csrc/bindings.cpp:39-68, 113-140):
//   tensorcore_attention_forward_production_128x128(query, key, value, causal)
//   tensorcore_attention_forward(query, key, value)                     N % 16 == 0
//   tensorcore_attention_forward_bc32(query, key, value)                N % 32 == 0
//   tensorcore_attention_forward_bc32_raw_pv(query, key, value)         N % 32 == 0
//   tensorcore_attention_forward_bc32_raw_qk_raw_pv(query, key, value)  N % 32 == 0
// The four Bc=16/32 entries compute the same noncausal attention; the reference's
// variants differ only in how its kernels issue the MMAs. Validation order and
// message text follow the reference (csrc/tensorcore_attention.cu:2731-2823,
// 2840-2895, 3025-3038) so callers see the same RuntimeError text. The arithmetic
// is done by the C ABI (include/fa2_mi355x.h), launched on the current HIP stream
// of the query's device.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cmath>
#include <cstdint>
#include <limits>

#include "fa2_mi355x.h"

namespace {

constexpr int64_t kHeadDimension = 64;
constexpr int64_t kProductionBlockM = 128;
constexpr int64_t kProductionBlockN = 128;
// Query tile of the reference's Bc=16/32 launcher: 4 warps x 16 rows
// (csrc/tensorcore_attention.cu:28-33, 2834-2839).
constexpr int64_t kTensorcoreBlockM = 64;

// Device checks come first in the reference; `check_device` lets the CPU test
// suite exercise the remaining checks on CPU tensors.
void validate_inputs(const torch::Tensor& query, const torch::Tensor& key,
                     const torch::Tensor& value, int64_t key_tile, bool check_device) {
    if (check_device) {
        TORCH_CHECK(query.is_cuda(), "query must be a CUDA tensor");
        TORCH_CHECK(key.is_cuda(), "key must be a CUDA tensor");
        TORCH_CHECK(value.is_cuda(), "value must be a CUDA tensor");
        TORCH_CHECK(query.device() == key.device() && query.device() == value.device(),
                    "query, key, and value must be on the same device");
    }
    TORCH_CHECK(query.scalar_type() == at::kHalf, "query must have dtype torch.float16");
    TORCH_CHECK(key.scalar_type() == at::kHalf, "key must have dtype torch.float16");
    TORCH_CHECK(value.scalar_type() == at::kHalf, "value must have dtype torch.float16");
    TORCH_CHECK(query.dim() == 4, "query must have shape [B, H, N, D]");
    TORCH_CHECK(key.dim() == 4, "key must have shape [B, H, N, D]");
    TORCH_CHECK(value.dim() == 4, "value must have shape [B, H, N, D]");
    TORCH_CHECK(query.sizes() == key.sizes(), "query and key must have identical shapes");
    TORCH_CHECK(query.sizes() == value.sizes(), "query and value must have identical shapes");
    TORCH_CHECK(query.is_contiguous(), "query must be contiguous");
    TORCH_CHECK(key.is_contiguous(), "key must be contiguous");
    TORCH_CHECK(value.is_contiguous(), "value must be contiguous");
    TORCH_CHECK(query.size(3) == kHeadDimension, "head dimension must equal 64");
    TORCH_CHECK(query.size(2) % key_tile == 0, "sequence length must be divisible by ", key_tile);
}

// Grid limits of the reference launchers (csrc/tensorcore_attention.cu:2876-2895,
// 3014-3038); `block_m` is the launcher's query tile.
void check_reference_grid_limits(int64_t batch, int64_t heads, int64_t seq_len,
                                 int64_t block_m = kProductionBlockM) {
    const int64_t num_query_tiles = (seq_len + block_m - 1) / block_m;
    TORCH_CHECK(num_query_tiles <= static_cast<int64_t>(std::numeric_limits<unsigned int>::max()),
                "too many query tiles for CUDA grid.x");
    TORCH_CHECK(batch * heads <= 65535, "batch * heads exceeds CUDA grid.y limit");
}

}  // namespace

torch::Tensor tensorcore_attention_forward_production_128x128(torch::Tensor query,
                                                               torch::Tensor key,
                                                               torch::Tensor value,
                                                               bool causal) {
    validate_inputs(query, key, value, kProductionBlockN, /*check_device=*/true);
    const c10::DeviceGuard device_guard(query.device());
    torch::Tensor output = torch::empty_like(query);

    const int64_t batch = query.size(0);
    const int64_t heads = query.size(1);
    const int64_t seq_len = query.size(2);
    if (batch == 0 || heads == 0 || seq_len == 0) return output;
    check_reference_grid_limits(batch, heads, seq_len);

    hipStream_t stream =
        c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(query.get_device()).stream();
    const int status = fa2_forward_production_128x128(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(), batch, heads,
        seq_len, query.size(3), causal ? 1 : 0, static_cast<void*>(stream));
    TORCH_CHECK(status == FA2_STATUS_SUCCESS,
                "fa2_forward_production_128x128 failed: ", fa2_status_string(status));
    return output;
}

// Shared body of the Bc=16/32 entries (reference tensorcore_attention_forward_impl,
// csrc/tensorcore_attention.cu:2826-2967).
torch::Tensor tensorcore_forward(const torch::Tensor& query, const torch::Tensor& key,
                                 const torch::Tensor& value, int64_t key_tile) {
    validate_inputs(query, key, value, key_tile, /*check_device=*/true);
    const c10::DeviceGuard device_guard(query.device());
    torch::Tensor output = torch::empty_like(query);

    const int64_t batch = query.size(0);
    const int64_t heads = query.size(1);
    const int64_t seq_len = query.size(2);
    if (batch == 0 || heads == 0 || seq_len == 0) return output;
    check_reference_grid_limits(batch, heads, seq_len, kTensorcoreBlockM);

    hipStream_t stream =
        c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(query.get_device()).stream();
    const int status = fa2_forward_tensorcore(
        query.data_ptr(), key.data_ptr(), value.data_ptr(), output.data_ptr(), batch, heads,
        seq_len, query.size(3), key_tile, static_cast<void*>(stream));
    TORCH_CHECK(status == FA2_STATUS_SUCCESS, "fa2_forward_tensorcore failed: ",
                fa2_status_string(status));
    return output;
}

torch::Tensor tensorcore_attention_forward(torch::Tensor query, torch::Tensor key,
                                           torch::Tensor value) {
    return tensorcore_forward(query, key, value, 16);
}

torch::Tensor tensorcore_attention_forward_bc32(torch::Tensor query, torch::Tensor key,
                                                torch::Tensor value) {
    return tensorcore_forward(query, key, value, 32);
}

torch::Tensor tensorcore_attention_forward_bc32_raw_pv(torch::Tensor query, torch::Tensor key,
                                                       torch::Tensor value) {
    return tensorcore_forward(query, key, value, 32);
}

torch::Tensor tensorcore_attention_forward_bc32_raw_qk_raw_pv(torch::Tensor query,
                                                              torch::Tensor key,
                                                              torch::Tensor value) {
    return tensorcore_forward(query, key, value, 32);
}

// Runs the host-side validation of the production entry without a launch. With
// check_device=false the device checks are skipped so CPU tensors reach the
// dtype/shape/layout checks; used by the CPU test suite.
void check_production_inputs(torch::Tensor query, torch::Tensor key, torch::Tensor value,
                             bool check_device) {
    validate_inputs(query, key, value, kProductionBlockN, check_device);
    if (query.numel() > 0) check_reference_grid_limits(query.size(0), query.size(1), query.size(2));
}

// The same for a Bc=16/32 entry (`key_tile` 16 or 32).
void check_tensorcore_inputs(torch::Tensor query, torch::Tensor key, torch::Tensor value,
                             int64_t key_tile, bool check_device) {
    validate_inputs(query, key, value, key_tile, check_device);
    if (query.numel() > 0)
        check_reference_grid_limits(query.size(0), query.size(1), query.size(2), kTensorcoreBlockM);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, module) {
    module.def("tensorcore_attention_forward", &tensorcore_attention_forward,
               "Fused FP16 Tensor Core attention forward pass");
    module.def("tensorcore_attention_forward_bc32", &tensorcore_attention_forward_bc32,
               "Fused FP16 Tensor core attention forward with Bc=32");
    module.def("tensorcore_attention_forward_bc32_raw_pv", &tensorcore_attention_forward_bc32_raw_pv,
               "Fused FP16 Tensor Core attention with raw MMA PV");
    module.def("tensorcore_attention_forward_bc32_raw_qk_raw_pv",
               &tensorcore_attention_forward_bc32_raw_qk_raw_pv,
               "Fused FP16 Tensor Core attention with raw MMA QK");
    module.def("tensorcore_attention_forward_production_128x128",
               &tensorcore_attention_forward_production_128x128, "Production kernel");
    module.def("_check_production_inputs", &check_production_inputs,
               "Validate inputs of the production entry without launching (testing hook)");
    module.def("_check_tensorcore_inputs", &check_tensorcore_inputs,
               "Validate inputs of a Bc=16/32 entry without launching (testing hook)");
    module.attr("abi_version") = fa2_abi_version();
}
