// ref_shim35.cpp -- C entry points into the compiled reference's Qwen3.5-MoE
// routing and MoE block.
//
// TEST INFRASTRUCTURE ONLY, built like ref_shim.cpp into oracle/_ref/libpkref.so
// from the reference's sources read in place.  select_experts, sigmoid and
// silu live in an anonymous namespace of src/qwen35_runner.cpp, so that
// translation unit is included here to make them reachable; the MoE block
// itself is inlined in Qwen35Runner's forward pass (:690-761), so
// pkref_moe35_forward repeats that loop over the reference's own functions.
#include "qwen35_runner.cpp"  // resolved through -I/root/reference/src

#include "pokitlms/model/tensor_linear.hpp"
#include "pokitlms/model/tensor_reader.hpp"

#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <vector>

namespace {

int status35_of_current_exception() {
    try {
        throw;
    } catch (const std::invalid_argument&) {
        return 1;
    } catch (const std::exception&) {
        return 2;
    } catch (...) {
        return 4;
    }
}

// Payload bytes of `rows` rows of `in` elements (the layouts of
// src/gguf_reader.cpp:21-57); throws for a type these shims do not pass.
std::uint64_t gguf_bytes(std::uint32_t type, std::uint64_t in, std::uint64_t rows) {
    std::uint64_t block = 32, bytes = 0;
    switch (type) {
        case 0: block = 1; bytes = 4; break;
        case 2: bytes = 18; break;
        case 3: bytes = 20; break;
        case 8: bytes = 34; break;
        case 12: block = 256; bytes = 144; break;
        case 13: block = 256; bytes = 176; break;
        case 14: block = 256; bytes = 210; break;
        default: throw std::invalid_argument("tensor type outside the shim's list");
    }
    return rows * (in / block) * bytes;
}

pokitlms::model::TensorReader reader35(std::uint32_t type, std::uint64_t in, std::uint64_t rows,
                                       const void* bytes) {
    pokitlms::model::TensorInfo tensor;
    tensor.name = "pkref35";
    tensor.dimensions = {in, rows};
    tensor.type = type;
    const auto nbytes = gguf_bytes(type, in, rows);
    tensor.payload_size = nbytes;
    auto payload = std::make_shared<std::vector<std::byte>>(nbytes);
    std::memcpy(payload->data(), bytes, nbytes);
    return pokitlms::model::TensorReader(tensor, payload);
}

}  // namespace

struct pkref_moe35 {
    std::uint32_t hidden{}, experts{}, ffn{}, shared_ffn{}, top_k{};
    bool normalize{};
    float scale{};
    std::unique_ptr<pokitlms::model::TensorReader> router, shared_router, shared_gate, shared_up,
        shared_down;
    std::vector<pokitlms::model::TensorReader> gate, up, down;
};

extern "C" {

int pkref_select_experts(const float* logits, std::uint32_t count, std::uint32_t top_k,
                         int normalize, std::uint32_t* ids, float* weights) {
    try {
        const auto routes = pokitlms::model::select_experts(
            std::span<const float>(logits, count), top_k, normalize != 0);
        for (std::size_t r = 0; r < routes.size(); ++r) {
            ids[r] = static_cast<std::uint32_t>(routes[r].id);
            weights[r] = routes[r].weight;
        }
        return 0;
    } catch (...) {
        return status35_of_current_exception();
    }
}

pkref_moe35* pkref_moe35_create(const float* router, std::uint32_t hidden, std::uint32_t experts,
                                std::uint32_t ffn, std::uint32_t gate_type, const void* gate,
                                std::uint32_t up_type, const void* up, std::uint32_t down_type,
                                const void* down, std::uint32_t top_k, int normalize, float scale,
                                const float* shared_router, std::uint32_t shared_ffn,
                                std::uint32_t sgate_type, const void* sgate,
                                std::uint32_t sup_type, const void* sup,
                                std::uint32_t sdown_type, const void* sdown) {
    try {
        auto m = std::make_unique<pkref_moe35>();
        m->hidden = hidden;
        m->experts = experts;
        m->ffn = ffn;
        m->shared_ffn = shared_ffn;
        m->top_k = top_k;
        m->normalize = normalize != 0;
        m->scale = scale;
        m->router = std::make_unique<pokitlms::model::TensorReader>(reader35(0, hidden, experts, router));
        m->shared_router = std::make_unique<pokitlms::model::TensorReader>(reader35(0, hidden, 1, shared_router));
        m->shared_gate = std::make_unique<pokitlms::model::TensorReader>(reader35(sgate_type, hidden, shared_ffn, sgate));
        m->shared_up = std::make_unique<pokitlms::model::TensorReader>(reader35(sup_type, hidden, shared_ffn, sup));
        m->shared_down = std::make_unique<pokitlms::model::TensorReader>(reader35(sdown_type, shared_ffn, hidden, sdown));
        const auto gs = gguf_bytes(gate_type, hidden, ffn), us = gguf_bytes(up_type, hidden, ffn),
                   ds = gguf_bytes(down_type, ffn, hidden);
        for (std::uint32_t e = 0; e < experts; ++e) {
            m->gate.push_back(reader35(gate_type, hidden, ffn, static_cast<const std::byte*>(gate) + e * gs));
            m->up.push_back(reader35(up_type, hidden, ffn, static_cast<const std::byte*>(up) + e * us));
            m->down.push_back(reader35(down_type, ffn, hidden, static_cast<const std::byte*>(down) + e * ds));
        }
        return m.release();
    } catch (...) {
        return nullptr;
    }
}

void pkref_moe35_destroy(pkref_moe35* m) { delete m; }

// src/qwen35_runner.cpp:690-761 with the reference's tensor_linear,
// select_experts, silu and sigmoid; y receives mixer_output.
int pkref_moe35_forward(pkref_moe35* m, const float* x, float* y, std::uint32_t* ids,
                        float* weights) {
    try {
        using pokitlms::model::tensor_linear;
        const std::span<const float> normalized(x, m->hidden);
        pokitlms::model::TensorLinearScratch scratch;
        std::vector<float> router_logits(m->experts), gate(std::max(m->ffn, m->shared_ffn)),
            up(gate.size()), activated(gate.size()), expert_output(m->hidden),
            moe_result(m->hidden, 0.0F);
        tensor_linear(*m->router, normalized, router_logits, 0, &scratch);
        const auto routes = pokitlms::model::select_experts(router_logits, m->top_k, m->normalize);
        for (std::size_t r = 0; r < routes.size(); ++r) {
            const auto& route = routes[r];
            ids[r] = static_cast<std::uint32_t>(route.id);
            weights[r] = route.weight;
            auto g = std::span<float>(gate).first(m->ffn);
            auto u = std::span<float>(up).first(m->ffn);
            auto a = std::span<float>(activated).first(m->ffn);
            tensor_linear(m->gate[route.id], normalized, g, 0, &scratch);
            tensor_linear(m->up[route.id], normalized, u, 0, &scratch);
            for (std::size_t i = 0; i < a.size(); ++i) a[i] = pokitlms::model::silu(g[i]) * u[i];
            tensor_linear(m->down[route.id], a, expert_output, 0, &scratch);
            const float route_scale = route.weight * m->scale;
            for (std::size_t i = 0; i < m->hidden; ++i) moe_result[i] += route_scale * expert_output[i];
        }
        float shared_gate_value = 0.0F;
        tensor_linear(*m->shared_router, normalized, std::span<float>(&shared_gate_value, 1), 0,
                      &scratch);
        auto g = std::span<float>(gate).first(m->shared_ffn);
        auto u = std::span<float>(up).first(m->shared_ffn);
        auto a = std::span<float>(activated).first(m->shared_ffn);
        tensor_linear(*m->shared_gate, normalized, g, 0, &scratch);
        tensor_linear(*m->shared_up, normalized, u, 0, &scratch);
        for (std::size_t i = 0; i < a.size(); ++i) a[i] = pokitlms::model::silu(g[i]) * u[i];
        tensor_linear(*m->shared_down, a, expert_output, 0, &scratch);
        const float shared_scale = pokitlms::model::sigmoid(shared_gate_value);
        for (std::size_t i = 0; i < m->hidden; ++i)
            y[i] = moe_result[i] + shared_scale * expert_output[i];
        return 0;
    } catch (...) {
        return status35_of_current_exception();
    }
}

}  // extern "C"
