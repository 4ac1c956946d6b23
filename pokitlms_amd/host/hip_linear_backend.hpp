// hip_linear_backend.hpp -- the MI355X (gfx950) HIP backend as a PokitLMs
// linear backend, for the reference's C++20 tree.
//
// HipLinearBackend implements model::TensorLinearBackend
// (include/pokitlms/model/tensor_linear.hpp:11-18), so tensor_linear's
// existing hook (src/tensor_linear.cpp:213) and a runner's
// set_linear_backend (src/qwen35_runner.cpp:939-943) take it exactly as they
// take VulkanLinearBackend (include/pokitlms/gpu/vulkan_linear.hpp:72-88).
// It adds a second hook, try_moe_block, that runs a whole routed MoE block
// (route_experts + gate/up SwiGLU + down + combine,
// src/qwen3_moe_runner.cpp:643-692) over expert tensors held resident in HBM.
//
// Everything below calls the C ABI of include/pokit_hip.h; no HIP or torch
// type appears here.  Error convention (tensor_linear.hpp:14-15 and
// src/vulkan_linear.cpp:612-736): false = unsupported (the caller runs its
// CPU kernel); shape errors throw std::invalid_argument; device failures
// throw std::runtime_error and every later call throws too.
#pragma once

#include "pokitlms/model/tensor_linear.hpp"
#include "pokitlms/model/tensor_reader.hpp"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <span>
#include <string>

namespace pokitlms::gpu {

struct HipLinearOptions {
    // HIP device ordinal; negative selects device 0.
    int device_index = -1;
    // Accumulate per-kernel device time (synchronises after every call).
    bool time_kernels = false;
    // Keep file-backed tensors resident in HBM after their first use (the
    // whole-model cache of the Vulkan backend, src/vulkan_linear.cpp:516-563).
    bool cache_file_tensors = true;
    // In-memory tensors (the expert slices a runner's ExpertStore hands to
    // tensor_linear, src/qwen35_runner.cpp:716-733) are kept in HBM in a
    // least-recently-used set of at most this many bytes, keyed by tensor
    // name, offset, type and shape.  An entry is reused only when the call's
    // bytes equal the bytes it was uploaded from (a host copy is kept for the
    // comparison: the set costs up to this many bytes of host memory as well
    // as of device memory), so a hit never serves stale weights.  0 (the
    // default, as the Vulkan backend, which keeps no copy) uploads every
    // in-memory tensor for its call and releases it; runners that hand over
    // the same expert slices repeatedly opt in.
    std::size_t transient_cache_bytes = 0;
    // Run every matrix and MoE block in the reference's own operation order
    // (pk_hip_matvec_reference_order, pk_hip_moe_decode_reference_order): the
    // CPU kernels' outputs bit for bit, so a runner's greedy tokens equal the
    // CPU runner's.  Types those kernels do not cover return false (the CPU
    // kernel runs), as does a Qwen3.5 block with a shared expert.
    bool reference_order = false;
    // The host libm's expf exceptions the reference-order SwiGLU needs (the
    // libm_expf.bin file the build writes); empty: the file beside
    // libpokit_hip.so.
    std::string libm_expf_table;
};

// Counters in the style of VulkanLinearStats (vulkan_linear.hpp:41-67).
struct HipLinearStats {
    std::uint64_t linear_calls{};        // try_linear calls that ran on the GPU
    std::uint64_t unsupported_calls{};   // try_linear calls that returned false
    std::uint64_t moe_calls{};           // try_moe_block calls that ran on the GPU
    std::uint64_t dispatches{};
    std::uint64_t q4_0_dispatches{};
    std::uint64_t q8_0_dispatches{};
    std::uint64_t q4_k_dispatches{};
    std::uint64_t q5_k_dispatches{};
    std::uint64_t q6_k_dispatches{};
    std::uint64_t other_dispatches{};    // F32 / F16 / BF16 / Q4_1
    std::uint64_t weight_bytes{};        // algorithmic weight bytes streamed
    std::uint64_t gpu_time_ns{};         // with HipLinearOptions::time_kernels
    std::uint64_t resident_bytes{};      // device bytes of resident tensors
    std::uint64_t uploaded_bytes{};      // host->device weight bytes so far
    std::uint64_t resident_tensors{};    // file-backed tensors kept in HBM
    std::uint64_t transient_uploads{};   // in-memory tensors uploaded per call
    std::uint64_t router_fallbacks{};    // tokens routed through exact serial logits
    std::uint64_t transient_hits{};      // in-memory tensors served from the LRU set
    std::uint64_t transient_bytes{};     // device bytes held by the LRU set
    std::uint64_t expert_hits{};         // routed expert accesses of try_moe_block
    std::uint64_t expert_misses{};       // always 0: uploaded experts never leave HBM
    std::uint64_t expert_resident_bytes{};  // expert tensor bytes of live MoE layers
};

// ExpertCacheStats of the runners (include/pokitlms/model/qwen3_moe_runner.hpp:44-52,
// qwen35_runner.hpp:47-55) for the experts of the MoE layers this backend holds:
// every expert is resident from upload on, so capacity and resident bytes are the
// uploaded expert bytes, nothing is read from the file afterwards, and every
// routed access is a hit.
struct HipExpertCacheStats {
    std::size_t capacity_bytes{};
    std::size_t resident_bytes{};
    std::uint64_t bytes_read{};
    std::uint64_t read_operations{};
    std::uint64_t read_time_ns{};
    std::uint64_t hits{};
    std::uint64_t misses{};
};

// A routed MoE layer resident in HBM (router F32 [hidden, experts]; gate/up
// [hidden, ffn, experts]; down [ffn, hidden, experts]).  Holds the backend's
// device context alive; release it to free the device memory.
class HipMoeLayer;

class HipLinearBackend final : public model::TensorLinearBackend {
public:
    explicit HipLinearBackend(const HipLinearOptions& options = {});
    ~HipLinearBackend() override;
    HipLinearBackend(const HipLinearBackend&) = delete;
    HipLinearBackend& operator=(const HipLinearBackend&) = delete;

    bool try_linear(const model::TensorReader& weights, std::span<const float> input,
                    std::span<float> output) override;

    // Uploads one routed MoE layer.  experts_per_token / expert_weights_norm
    // are the runner's config fields (qwen3_moe_runner.cpp:646-647);
    // expert_weights_scale is Qwen3.5's multiplier (qwen35_runner.cpp:738).
    [[nodiscard]] std::shared_ptr<HipMoeLayer> upload_moe_layer(
        const model::TensorReader& router, const model::TensorReader& gate_exps,
        const model::TensorReader& up_exps, const model::TensorReader& down_exps,
        std::size_t experts_per_token, bool expert_weights_norm,
        float expert_weights_scale = 1.0F);

    // Qwen3.5-MoE: attaches the layer's shared expert (ffn_gate_inp_shexp
    // [hidden], ffn_gate_shexp / ffn_up_shexp [hidden, ffn], ffn_down_shexp
    // [ffn, hidden]; qwen35_runner.cpp:670-764).  try_moe_block then returns
    // the block's mixer output: the routed sum with select_experts' weights
    // (times expert_weights_scale) plus sigmoid(shared gate) * shared output.
    // The shared expert must have the routed experts' types and width, or
    // try_moe_block returns false.
    void attach_shared_expert(HipMoeLayer& layer, const model::TensorReader& shared_router,
                              const model::TensorReader& shared_gate,
                              const model::TensorReader& shared_up,
                              const model::TensorReader& shared_down);

    // moe_result = the MoE block of src/qwen3_moe_runner.cpp:644-691 for one
    // normalised hidden state (the residual add stays with the caller).
    // route_ids / route_probabilities (optional, size experts_per_token)
    // receive the routes in order.  false = shape not covered by the
    // kernels: the caller runs its CPU block.  Non-finite router logits
    // throw std::runtime_error, as route_experts does (:270-276).
    bool try_moe_block(const HipMoeLayer& layer, std::span<const float> normalized,
                       std::span<float> moe_result,
                       std::span<std::uint32_t> route_ids = {},
                       std::span<float> route_probabilities = {});

    [[nodiscard]] HipLinearStats stats() const;
    [[nodiscard]] HipExpertCacheStats expert_cache_stats() const;
    [[nodiscard]] std::string device_name() const;

    class Impl;

private:
    std::shared_ptr<Impl> impl_;
};

}  // namespace pokitlms::gpu
