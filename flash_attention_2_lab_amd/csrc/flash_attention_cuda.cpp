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
//
// The module's other operators (reference csrc/bindings.cpp:71-111) are here too,
// with the reference's checks and messages:
//   copy_cuda(input)                                  csrc/copy_kernel.cu:23-53
//   naive_attention_forward(query, key, value)        csrc/naive_attention.cu:203-328
//   naive_attention_scores(query, key)                csrc/naive_attention.cu:330-418
//   block_attention_forward(query, key, value)        csrc/naive_attention.cu:420-502
//   tiled_attention_forward(query, key, value)        csrc/tiled_attention.cu:220-333
//   tilewise_attention_forward(query, key, value)     csrc/tilewise_attention.cu:285-388
//   wmma_matmul_16x64x16(matrix_a, matrix_b)          csrc/wmma_matmul.cu:195-315
// The four FP32 forwards run one FP32 attention kernel; the reference's differ
// only in their thread mappings.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cmath>
#include <cstdint>
#include <limits>
#include <string>
#include <vector>

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

// ---------------------------------------------------------------------------
// The module's other operators.

namespace {

hipStream_t current_stream(const torch::Tensor& t) {
    return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.get_device()).stream();
}

void check_status(int status, const char* entry) {
    TORCH_CHECK(status == FA2_STATUS_SUCCESS, entry, " failed: ", fa2_status_string(status));
}

// reference csrc/naive_attention.cu:203-245 (naive and block forwards).
void validate_naive_inputs(const torch::Tensor& query, const torch::Tensor& key,
                           const torch::Tensor& value, bool check_device) {
    if (check_device) {
        TORCH_CHECK(query.is_cuda(), "query must be a CUDA tensor");
        TORCH_CHECK(key.is_cuda(), "key must be a CUDA tensor");
        TORCH_CHECK(value.is_cuda(), "value must be a CUDA tensor");
    }
    TORCH_CHECK(query.is_contiguous(), "query must be contiguous");
    TORCH_CHECK(key.is_contiguous(), "key must be contiguous");
    TORCH_CHECK(value.is_contiguous(), "value must be contiguous");
    TORCH_CHECK(query.dim() == 4, "query must be rank 4");
    TORCH_CHECK(key.dim() == 4, "key must be rank 4");
    TORCH_CHECK(value.dim() == 4, "value must be rank 4");
    TORCH_CHECK(query.scalar_type() == at::kFloat, "query must use float32");
    TORCH_CHECK(key.scalar_type() == at::kFloat, "key must use float32");
    TORCH_CHECK(value.scalar_type() == at::kFloat, "value must use float32");
    if (check_device)
        TORCH_CHECK(query.device() == key.device() && query.device() == value.device(),
                    "query, key, and value must be on the same CUDA device");
    TORCH_CHECK(query.sizes() == key.sizes() && query.sizes() == value.sizes(),
                "the initial naive kernel requires query, key, and value to have identical shapes");
}

// reference csrc/naive_attention.cu:334-363.
void validate_score_inputs(const torch::Tensor& query, const torch::Tensor& key, bool check_device) {
    if (check_device) {
        TORCH_CHECK(query.is_cuda(), "query must be a CUDA tensor");
        TORCH_CHECK(key.is_cuda(), "key must be a CUDA tensor");
    }
    TORCH_CHECK(query.is_contiguous(), "query must be contiguous");
    TORCH_CHECK(key.is_contiguous(), "key must be contiguous");
    TORCH_CHECK(query.dim() == 4, "query must be rank 4");
    TORCH_CHECK(key.dim() == 4, "key must be rank 4");
    TORCH_CHECK(query.scalar_type() == at::kFloat, "query must use float32");
    TORCH_CHECK(key.scalar_type() == at::kFloat, "key must use float32");
    if (check_device)
        TORCH_CHECK(query.device() == key.device(), "query and key must be on the same CUDA device");
    TORCH_CHECK(query.sizes() == key.sizes(),
                "the initial score kernel requires query and key to have identical shapes");
}

// Checks of the tiled (csrc/tiled_attention.cu:220-269) and tilewise
// (csrc/tilewise_attention.cu:285-334) forwards: the same order, their own text.
struct TiledMessages {
    const char* dtype;
    const char* shapes;
    const char* head_dim;
    const char* query_tiles;
    const char* batch_heads;
};
constexpr TiledMessages kTiledMessages = {
    "the initial tiled kernel requires float32 inputs",
    "the initial tiled kernel requires identical Q, K, and V shapes",
    "the initial tiled kernel supports head dimension 64",
    "too many query tiles for CUDA grid",
    "batch x heads exceeds CUDA grid.y limit"};
constexpr TiledMessages kTilewiseMessages = {
    "tilewise attention currently requires float32",
    "tilewise attention currently requires identical Q, K, and V shapes",
    "tilewise attention currently supports head dimension 64",
    "too many query tiles for CUDA grid.x",
    "batch * num_heads exceeds CUDA grid.y limit"};

void validate_tiled_inputs(const torch::Tensor& query, const torch::Tensor& key,
                           const torch::Tensor& value, const TiledMessages& text, bool check_device) {
    if (check_device)
        TORCH_CHECK(query.is_cuda() && key.is_cuda() && value.is_cuda(),
                    "query, key, and value must be CUDA tensors");
    TORCH_CHECK(query.is_contiguous() && key.is_contiguous() && value.is_contiguous(),
                "query, key, and value must be contiguous");
    TORCH_CHECK(query.dim() == 4 && key.dim() == 4 && value.dim() == 4,
                "query, key, and value must be rank 4");
    TORCH_CHECK(query.scalar_type() == at::kFloat && key.scalar_type() == at::kFloat &&
                    value.scalar_type() == at::kFloat,
                text.dtype);
    if (check_device)
        TORCH_CHECK(query.device() == key.device() && query.device() == value.device(),
                    "query, key, and value must be on the same CUDA device");
    TORCH_CHECK(query.sizes() == key.sizes() && query.sizes() == value.sizes(), text.shapes);
    TORCH_CHECK(query.size(3) == kHeadDimension, text.head_dim);
}

// Grid checks of the tiled launchers: 16-query tiles in grid.x, batch*heads in
// grid.y (csrc/tiled_attention.cu:295-312, csrc/tilewise_attention.cu:350-365).
void check_tiled_grid(int64_t batch, int64_t heads, int64_t seq_len, const TiledMessages& text) {
    const int64_t query_tiles = (seq_len + 15) / 16;
    TORCH_CHECK(query_tiles <= static_cast<int64_t>(std::numeric_limits<unsigned int>::max()),
                text.query_tiles);
    TORCH_CHECK(batch * heads <= 65535, text.batch_heads);
}

// reference csrc/wmma_matmul.cu:195-245.
void validate_matmul_inputs(const torch::Tensor& a, const torch::Tensor& b, bool check_device) {
    if (check_device) TORCH_CHECK(a.is_cuda() && b.is_cuda(), "A and B must be CUDA tensors");
    TORCH_CHECK(a.is_contiguous() && b.is_contiguous(), "A and B must be contiguous");
    TORCH_CHECK(a.scalar_type() == at::kHalf && b.scalar_type() == at::kHalf, "A and B must use float16");
    if (check_device) TORCH_CHECK(a.device() == b.device(), "A and B must be on the same CUDA device");
    TORCH_CHECK(a.dim() == 3 && b.dim() == 3, "A and B must be rank-3 tensors");
    TORCH_CHECK(a.size(0) == b.size(0), "A and B must have the same batch size");
    TORCH_CHECK(a.size(1) == 16 && a.size(2) == 64, "A must have shape [batch, 16, 64]");
    TORCH_CHECK(b.size(1) == 64 && b.size(2) == 16, "B must have shape [batch, 64, 16]");
}

// Launch of the shared FP32 forward on validated inputs.
void run_f32_attention(const torch::Tensor& query, const torch::Tensor& key, const torch::Tensor& value,
                       torch::Tensor& output) {
    const int64_t batch_heads = query.size(0) * query.size(1);
    check_status(fa2_attention_forward_f32(query.data_ptr<float>(), key.data_ptr<float>(),
                                           value.data_ptr<float>(), output.data_ptr<float>(),
                                           batch_heads, query.size(2), query.size(3),
                                           static_cast<void*>(current_stream(query))),
                 "fa2_attention_forward_f32");
}

// Shared body of the tiled and tilewise forwards (head dimension 64).
torch::Tensor tiled_forward(const torch::Tensor& query, const torch::Tensor& key,
                            const torch::Tensor& value, const TiledMessages& text) {
    validate_tiled_inputs(query, key, value, text, /*check_device=*/true);
    const c10::DeviceGuard device_guard(query.device());
    torch::Tensor output = torch::empty_like(query);
    const int64_t seq_len = query.size(2);
    if (seq_len == 0) return output;
    check_tiled_grid(query.size(0), query.size(1), seq_len, text);
    run_f32_attention(query, key, value, output);
    return output;
}

}  // namespace

torch::Tensor copy_cuda(torch::Tensor input) {
    TORCH_CHECK(input.is_cuda(), "input must be a CUDA tensor");
    TORCH_CHECK(input.is_contiguous(), "input must be contiguous");
    const c10::DeviceGuard device_guard(input.device());
    torch::Tensor output = torch::empty_like(input);
    if (input.numel() == 0) return output;
    // The reference dispatches on float, double, half and bfloat16 and rejects any
    // other dtype the way AT_DISPATCH_FLOATING_TYPES_AND2 does.
    const at::ScalarType type = input.scalar_type();
    TORCH_CHECK_NOT_IMPLEMENTED(type == at::kFloat || type == at::kDouble || type == at::kHalf ||
                                    type == at::kBFloat16,
                                "\"copy_cuda\" not implemented for '", c10::toString(type), "'");
    check_status(fa2_copy(input.data_ptr(), output.data_ptr(), input.numel() * input.element_size(),
                          static_cast<void*>(current_stream(input))),
                 "fa2_copy");
    return output;
}

torch::Tensor naive_attention_forward(torch::Tensor query, torch::Tensor key, torch::Tensor value) {
    validate_naive_inputs(query, key, value, /*check_device=*/true);
    const c10::DeviceGuard device_guard(query.device());
    torch::Tensor output = torch::empty_like(query);
    const int64_t rows = query.size(0) * query.size(1) * query.size(2);
    const int64_t head_dim = query.size(3);
    if (rows == 0 || head_dim == 0) return output;
    TORCH_CHECK(head_dim == 64 || head_dim == 128,
                "naive_attention_forward currently supports head dimensions 64 and 128");
    run_f32_attention(query, key, value, output);
    return output;
}

torch::Tensor naive_attention_scores(torch::Tensor query, torch::Tensor key) {
    validate_score_inputs(query, key, /*check_device=*/true);
    const c10::DeviceGuard device_guard(query.device());
    const int64_t batch = query.size(0), heads = query.size(1), seq_len = query.size(2);
    torch::Tensor scores = torch::empty({batch, heads, seq_len, seq_len}, query.options());
    if (scores.numel() == 0) return scores;
    check_status(fa2_attention_scores_f32(query.data_ptr<float>(), key.data_ptr<float>(),
                                          scores.data_ptr<float>(), batch * heads, seq_len,
                                          query.size(3), static_cast<void*>(current_stream(query))),
                 "fa2_attention_scores_f32");
    return scores;
}

torch::Tensor block_attention_forward(torch::Tensor query, torch::Tensor key, torch::Tensor value) {
    validate_naive_inputs(query, key, value, /*check_device=*/true);
    const c10::DeviceGuard device_guard(query.device());
    torch::Tensor output = torch::empty_like(query);
    const int64_t rows = query.size(0) * query.size(1) * query.size(2);
    if (rows == 0) return output;
    TORCH_CHECK(query.size(3) == 64 || query.size(3) == 128,
                "block_attention_forward currently supports head dimensions 64 and 128");
    run_f32_attention(query, key, value, output);
    return output;
}

torch::Tensor tiled_attention_forward(torch::Tensor query, torch::Tensor key, torch::Tensor value) {
    return tiled_forward(query, key, value, kTiledMessages);
}

torch::Tensor tilewise_attention_forward(torch::Tensor query, torch::Tensor key, torch::Tensor value) {
    return tiled_forward(query, key, value, kTilewiseMessages);
}

torch::Tensor wmma_matmul_16x64x16(torch::Tensor matrix_a, torch::Tensor matrix_b) {
    validate_matmul_inputs(matrix_a, matrix_b, /*check_device=*/true);
    const c10::DeviceGuard device_guard(matrix_a.device());
    const int64_t batch = matrix_a.size(0);
    torch::Tensor matrix_c = torch::empty({batch, 16, 16}, matrix_a.options().dtype(at::kFloat));
    if (batch == 0) return matrix_c;
    TORCH_CHECK(batch <= static_cast<int64_t>(std::numeric_limits<unsigned int>::max()),
                "batch size exceeds CUDA grid.x limit");
    check_status(fa2_matmul_16x64x16_f16(matrix_a.data_ptr(), matrix_b.data_ptr(),
                                         matrix_c.data_ptr<float>(), batch,
                                         static_cast<void*>(current_stream(matrix_a))),
                 "fa2_matmul_16x64x16_f16");
    return matrix_c;
}

// Runs an operator's host-side validation without a launch (testing hook). With
// check_device=false the device checks are skipped so CPU tensors reach the later
// checks. `op` is the operator's name; `tensors` its tensor arguments in order.
void check_op_inputs(const std::string& op, std::vector<torch::Tensor> tensors, bool check_device) {
    auto arg = [&](size_t i) -> const torch::Tensor& {
        TORCH_CHECK(i < tensors.size(), op, " takes more tensor arguments");
        return tensors[i];
    };
    if (op == "naive_attention_forward" || op == "block_attention_forward") {
        validate_naive_inputs(arg(0), arg(1), arg(2), check_device);
        const int64_t rows = arg(0).size(0) * arg(0).size(1) * arg(0).size(2);
        const int64_t head_dim = arg(0).size(3);
        if (rows == 0 || (op == "naive_attention_forward" && head_dim == 0)) return;
        TORCH_CHECK(head_dim == 64 || head_dim == 128, op, " currently supports head dimensions 64 and 128");
    } else if (op == "naive_attention_scores") {
        validate_score_inputs(arg(0), arg(1), check_device);
    } else if (op == "tiled_attention_forward" || op == "tilewise_attention_forward") {
        const TiledMessages& text = op == "tiled_attention_forward" ? kTiledMessages : kTilewiseMessages;
        validate_tiled_inputs(arg(0), arg(1), arg(2), text, check_device);
        if (arg(0).size(2) > 0) check_tiled_grid(arg(0).size(0), arg(0).size(1), arg(0).size(2), text);
    } else if (op == "wmma_matmul_16x64x16") {
        validate_matmul_inputs(arg(0), arg(1), check_device);
    } else {
        TORCH_CHECK(false, "no validation hook for ", op);
    }
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, module) {
    module.def("copy_cuda", &copy_cuda, "Copy a CUDA tensor");
    module.def("naive_attention_forward", &naive_attention_forward, "Naive attention forward pass");
    module.def("naive_attention_scores", &naive_attention_scores, "Compute naive scaled attention scores");
    module.def("block_attention_forward", &block_attention_forward, "Block-cooperative online attention");
    module.def("tiled_attention_forward", &tiled_attention_forward,
               "Tiled SIMT online attention forward pass");
    module.def("tilewise_attention_forward", &tilewise_attention_forward,
               "Tilewise SIMT attention forward pass");
    module.def("wmma_matmul_16x64x16", &wmma_matmul_16x64x16,
               "WMMA FP16 16x64 by 64x16 matrix multiplication with FP32 accumulation");
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
    module.def("_check_op_inputs", &check_op_inputs,
               "Validate inputs of one of the other operators without launching (testing hook)");
    module.attr("abi_version") = fa2_abi_version();
}
