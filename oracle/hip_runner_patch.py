"""Writes the reference's Qwen3MoeRunner and C API with the HIP backend hook --
TEST INFRASTRUCTURE (the recipe a maintainer would apply to the reference
tree, compiled here against the reference in place).

    python oracle/hip_runner_patch.py REF OUT

copies four files of the reference checkout REF into OUT (the git-ignored
oracle/_ref/hip_tree) and inserts, at anchor lines that must each occur once,
the lines below; nothing of the reference is removed or changed, and no
reference file is written into the repository:

* include/pokitlms/model/qwen3_moe_runner.hpp: a public
  ``set_linear_backend(std::shared_ptr<TensorLinearBackend>)``, the same
  setter Qwen35Runner has (include/pokitlms/model/qwen35_runner.hpp:91);
* src/qwen3_moe_runner.cpp: the backend installed in the runner's
  TensorLinearScratch (so every tensor_linear call, src/tensor_linear.cpp:213,
  tries it first), and, when it is a HipLinearBackend, every layer's router and
  expert tensors uploaded once and the MoE block (:643-691) sent through
  HipLinearBackend::try_moe_block, the unchanged CPU code running when that
  returns false;
* include/pokitlms/pokitlms.h and src/c_api.cpp: a backend selector for the C
  API, ``pokitlms_qwen3moe_create_with_backend`` beside
  ``pokitlms_qwen3moe_create_ex`` (pokitlms.h:62-75, c_api.cpp:54-102).
"""
from __future__ import annotations

import os
import sys

RUNNER_HPP_DECL = '''class TensorLinearBackend;

'''

RUNNER_HPP_METHOD = '''    // Sends every tensor_linear call of this runner through `backend` first
    // (false = the CPU kernel), as Qwen35Runner::set_linear_backend does.  A
    // pokitlms::gpu::HipLinearBackend also takes each layer's whole MoE block
    // with every expert resident in its device memory; null restores the CPU.
    void set_linear_backend(std::shared_ptr<TensorLinearBackend> backend);
'''

RUNNER_INCLUDE = '''#include "hip_linear_backend.hpp"
'''

RUNNER_MEMBERS = '''    std::shared_ptr<TensorLinearBackend> linear_backend;
    std::shared_ptr<gpu::HipLinearBackend> hip_backend;
    std::vector<std::shared_ptr<gpu::HipMoeLayer>> hip_moe_layers;  // one per layer
'''

RUNNER_HOOK_OPEN = '''                auto& moe_result = scratch.moe_result;
                if (!(hip_backend &&
                      hip_backend->try_moe_block(*hip_moe_layers[layer], normalized, moe_result))) {
'''

RUNNER_HOOK_CLOSE = '''                }
'''

RUNNER_SETTER = '''
namespace pokitlms::model {

void Qwen3MoeRunner::set_linear_backend(std::shared_ptr<TensorLinearBackend> backend) {
    auto& impl = *impl_;
    std::vector<std::shared_ptr<gpu::HipMoeLayer>> layers;
    auto hip = std::dynamic_pointer_cast<gpu::HipLinearBackend>(backend);
    if (hip) {
        const auto& config = impl.index.config();
        const auto top_k = as_size(config.experts_per_token, "experts_per_token");
        for (const auto& block : impl.index.blocks()) {
            layers.push_back(hip->upload_moe_layer(
                TensorReader(impl.file, block.router), TensorReader(impl.file, block.expert_gate),
                TensorReader(impl.file, block.expert_up), TensorReader(impl.file, block.expert_down),
                top_k, config.expert_weights_norm));
        }
    }
    impl.linear_backend = std::move(backend);
    impl.hip_backend = std::move(hip);
    impl.hip_moe_layers = std::move(layers);
    impl.scratch.tensor_linear.backend = impl.linear_backend.get();
}

}  // namespace pokitlms::model
'''

CAPI_H = '''// Backends the C API can place a Qwen3-MoE model's linear algebra on: the
// CPU kernels, the MI355X HIP backend (bandwidth-optimised kernels), or the
// HIP backend in the CPU kernels' own operation order (the CPU's tokens).
typedef enum pokitlms_backend {
    POKITLMS_BACKEND_CPU = 0,
    POKITLMS_BACKEND_HIP = 1,
    POKITLMS_BACKEND_HIP_REFERENCE_ORDER = 2
} pokitlms_backend;
// create_ex with a backend on HIP device `device_index` (negative: device 0).
pokitlms_status pokitlms_qwen3moe_create_with_backend(
    const char* model_path, size_t expert_cache_budget_bytes, size_t context_capacity,
    pokitlms_kv_cache_precision kv_precision, pokitlms_backend backend, int device_index,
    pokitlms_model** out_model, char* error_buffer, size_t error_capacity);
'''

CAPI_INCLUDE = '''#include "hip_linear_backend.hpp"
'''

CAPI_FN = '''
pokitlms_status pokitlms_qwen3moe_create_with_backend(
    const char* model_path, size_t expert_cache_budget_bytes, size_t context_capacity,
    pokitlms_kv_cache_precision kv_precision, pokitlms_backend backend, int device_index,
    pokitlms_model** out_model, char* error_buffer, size_t error_capacity) {
    if (backend != POKITLMS_BACKEND_CPU && backend != POKITLMS_BACKEND_HIP &&
        backend != POKITLMS_BACKEND_HIP_REFERENCE_ORDER) {
        if (out_model) *out_model = nullptr;
        set_error(error_buffer, error_capacity, "unknown backend");
        return POKITLMS_STATUS_INVALID_ARGUMENT;
    }
    const auto status = pokitlms_qwen3moe_create_ex(model_path, expert_cache_budget_bytes,
                                                    context_capacity, kv_precision, out_model,
                                                    error_buffer, error_capacity);
    if (status != POKITLMS_STATUS_OK || backend == POKITLMS_BACKEND_CPU) return status;
    auto fail = [&](pokitlms_status code, const char* message) {
        delete *out_model;
        *out_model = nullptr;
        set_error(error_buffer, error_capacity, message);
        return code;
    };
    try {
        pokitlms::gpu::HipLinearOptions options;
        options.device_index = device_index;
        options.reference_order = backend == POKITLMS_BACKEND_HIP_REFERENCE_ORDER;
        (*out_model)->runner.set_linear_backend(
            std::make_shared<pokitlms::gpu::HipLinearBackend>(options));
        return POKITLMS_STATUS_OK;
    } catch (const std::invalid_argument& error) {
        return fail(POKITLMS_STATUS_INVALID_ARGUMENT, error.what());
    } catch (const std::exception& error) {
        return fail(POKITLMS_STATUS_RUNTIME_ERROR, error.what());
    } catch (...) {
        return fail(POKITLMS_STATUS_INTERNAL_ERROR, "unknown backend creation failure");
    }
}
'''

# (file, [(anchor line, text, before?)], text appended at the end)
PLAN = {
    "include/pokitlms/model/qwen3_moe_runner.hpp": (
        [("struct GenerationOptions {", RUNNER_HPP_DECL, True),
         ("    [[nodiscard]] ExpertCacheStats expert_cache_stats() const;", RUNNER_HPP_METHOD,
          False)], ""),
    "src/qwen3_moe_runner.cpp": (
        [('#include "simd_kernels.hpp"', RUNNER_INCLUDE, False),
         ("    ExpertLoader expert_loader;", RUNNER_MEMBERS, False),
         ("                auto& router_logits = scratch.router_logits;", RUNNER_HOOK_OPEN, True),
         ("                for (std::size_t i = 0; i < hidden_size; ++i) hidden[i] += moe_result[i];",
          RUNNER_HOOK_CLOSE, True)], RUNNER_SETTER),
    "include/pokitlms/pokitlms.h": (
        [("void pokitlms_model_destroy(pokitlms_model* model);", CAPI_H, True)], ""),
    "src/c_api.cpp": (
        [('#include "pokitlms/model/qwen3_moe_runner.hpp"', CAPI_INCLUDE, False)], CAPI_FN),
}


def patch(ref: str, out: str) -> None:
    for rel, (inserts, tail) in PLAN.items():
        with open(os.path.join(ref, rel)) as f:
            lines = f.read().split("\n")
        for anchor, text, before in inserts:
            hits = [i for i, line in enumerate(lines) if line == anchor]
            if len(hits) != 1:
                raise SystemExit(f"{rel}: anchor {anchor!r} found {len(hits)} times")
            at = hits[0] if before else hits[0] + 1
            lines[at:at] = text.rstrip("\n").split("\n")
        dst = os.path.join(out, rel)
        os.makedirs(os.path.dirname(dst), exist_ok=True)
        with open(dst, "w") as f:
            f.write("\n".join(lines) + tail)


if __name__ == "__main__":
    patch(sys.argv[1], sys.argv[2])
