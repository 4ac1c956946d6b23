// ref_shim.cpp -- C entry points into the compiled reference CPU path.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's own sources, read in place from /root/reference/src (nothing
// is copied into this repository), into oracle/_ref/libpkref.so.  The library
// writes the golden vectors under tests/golden/ and serves as the timed CPU
// baseline ("kind": "reference").  route_experts lives in an anonymous
// namespace of src/qwen3_moe_runner.cpp, so that translation unit is included
// here to make it reachable.
#include "qwen3_moe_runner.cpp"  // resolved through -I/root/reference/src

#include "pokitlms/model/tensor_linear.hpp"
#include "pokitlms/model/tensor_reader.hpp"
#include "pokitlms/ops/quantized_linear.hpp"
#include "pokitlms/ops/rms_norm.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <thread>
#include <vector>

namespace {

int status_of_current_exception() {
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

pokitlms::model::TensorReader make_reader(std::uint32_t type, std::uint64_t in,
                                          std::uint64_t rows, const void* bytes,
                                          std::uint64_t nbytes) {
    pokitlms::model::TensorInfo tensor;
    tensor.name = "pkref";
    tensor.dimensions = {in, rows};
    tensor.type = type;
    tensor.payload_size = nbytes;
    auto payload = std::make_shared<std::vector<std::byte>>(nbytes);
    std::memcpy(payload->data(), bytes, nbytes);
    return pokitlms::model::TensorReader(tensor, payload);
}

}  // namespace

extern "C" {

// Worker count of the reference row pool (src/tensor_linear.cpp:56-64).
unsigned pkref_row_workers(void) {
    const auto hardware = std::thread::hardware_concurrency();
    return std::min(6U, std::max(2U, hardware > 1 ? hardware - 1 : 2U));
}

// tensor_linear over an in-memory GGUF matrix [in, rows] (src/tensor_linear.cpp:232-263).
int pkref_tensor_linear(std::uint32_t type, std::uint64_t in, std::uint64_t rows,
                        const void* bytes, std::uint64_t nbytes, const float* x, float* y) {
    try {
        const auto reader = make_reader(type, in, rows, bytes, nbytes);
        pokitlms::model::tensor_linear(reader, std::span<const float>(x, in),
                                       std::span<float>(y, rows));
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

// Same, repeated `calls` times on one prepared reader (CPU baseline timing).
int pkref_tensor_linear_repeat(std::uint32_t type, std::uint64_t in, std::uint64_t rows,
                               const void* bytes, std::uint64_t nbytes, const float* x,
                               float* y, std::uint32_t calls) {
    try {
        const auto reader = make_reader(type, in, rows, bytes, nbytes);
        for (std::uint32_t c = 0; c < calls; ++c) {
            pokitlms::model::tensor_linear(reader, std::span<const float>(x, in),
                                           std::span<float>(y, rows));
        }
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

// The reference rms_norm (src/rms_norm.cpp:9-27) of each row.
int pkref_rms_norm(const float* x, const float* w, std::uint64_t rows, std::uint64_t n, float eps,
                   float* out) {
    try {
        for (std::uint64_t r = 0; r < rows; ++r)
            pokitlms::rms_norm(std::span<const float>(x + r * n, n), std::span<const float>(w, n),
                               std::span<float>(out + r * n, n), eps);
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

int pkref_dequantize_row(std::uint32_t type, const void* encoded, std::uint64_t nbytes,
                         float* out, std::uint64_t count) {
    try {
        pokitlms::dequantize_quantized_row(
            type, std::span<const std::byte>(static_cast<const std::byte*>(encoded), nbytes),
            std::span<float>(out, count));
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

int pkref_route_experts(const float* logits, std::uint32_t count, std::uint32_t top_k,
                        int normalize, std::uint32_t* ids, float* selected_logits,
                        float* probabilities) {
    try {
        const auto routes = pokitlms::model::route_experts(
            std::span<const float>(logits, count), top_k, normalize != 0);
        for (std::size_t i = 0; i < routes.size(); ++i) {
            ids[i] = static_cast<std::uint32_t>(routes[i].id);
            if (selected_logits) selected_logits[i] = routes[i].logit;
            probabilities[i] = routes[i].probability;
        }
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

// A prepared MoE layer: readers over the router and every expert slice.
struct pkref_moe {
    std::uint32_t hidden{}, experts{}, ffn{}, top_k{};
    bool normalize{};
    std::unique_ptr<pokitlms::model::TensorReader> router;
    std::vector<pokitlms::model::TensorReader> gate, up, down;
};

void pkref_moe_destroy(pkref_moe* moe) { delete moe; }

pkref_moe* pkref_moe_create(const float* router, std::uint32_t hidden, std::uint32_t experts,
                            std::uint32_t ffn, std::uint32_t gate_type, const void* gate,
                            std::uint32_t up_type, const void* up, std::uint32_t down_type,
                            const void* down, std::uint32_t top_k, int normalize) {
    try {
        auto moe = std::make_unique<pkref_moe>();
        moe->hidden = hidden;
        moe->experts = experts;
        moe->ffn = ffn;
        moe->top_k = top_k;
        moe->normalize = normalize != 0;
        moe->router = std::make_unique<pokitlms::model::TensorReader>(
            make_reader(0, hidden, experts, router, std::uint64_t{hidden} * experts * 4));
        const auto slice_bytes = [](std::uint32_t type, std::uint64_t in, std::uint64_t out) {
            std::uint64_t block = 32, bytes = 0;
            switch (type) {  // src/gguf_reader.cpp:21-57
                case 2: bytes = 18; break;
                case 3: bytes = 20; break;
                case 8: bytes = 34; break;
                case 12: block = 256; bytes = 144; break;
                case 13: block = 256; bytes = 176; break;
                case 14: block = 256; bytes = 210; break;
                default: throw std::invalid_argument("expert type outside the shim's list");
            }
            return out * (in / block) * bytes;
        };
        const auto gs = slice_bytes(gate_type, hidden, ffn);
        const auto us = slice_bytes(up_type, hidden, ffn);
        const auto ds = slice_bytes(down_type, ffn, hidden);
        for (std::uint32_t e = 0; e < experts; ++e) {
            moe->gate.push_back(make_reader(gate_type, hidden, ffn,
                                            static_cast<const std::byte*>(gate) + e * gs, gs));
            moe->up.push_back(make_reader(up_type, hidden, ffn,
                                          static_cast<const std::byte*>(up) + e * us, us));
            moe->down.push_back(make_reader(down_type, ffn, hidden,
                                            static_cast<const std::byte*>(down) + e * ds, ds));
        }
        return moe.release();
    } catch (...) {
        return nullptr;
    }
}

// The MoE block of src/qwen3_moe_runner.cpp:644-691, statement for statement,
// over the reference's own tensor_linear and route_experts.  y = moe_result.
int pkref_moe_forward(pkref_moe* moe, const float* x, float* y, std::uint32_t* ids,
                      float* probabilities) {
    try {
        using pokitlms::model::tensor_linear;
        const std::span<const float> normalized(x, moe->hidden);
        std::vector<float> router_logits(moe->experts), gate(moe->ffn), up(moe->ffn),
            activated(moe->ffn), expert_output(moe->hidden);
        pokitlms::model::TensorLinearScratch scratch;
        tensor_linear(*moe->router, normalized, router_logits, 0, &scratch);
        const auto routes = pokitlms::model::route_experts(router_logits, moe->top_k,
                                                           moe->normalize);
        std::span<float> moe_result(y, moe->hidden);
        std::fill(moe_result.begin(), moe_result.end(), 0.0F);
        for (std::size_t r = 0; r < routes.size(); ++r) {
            const auto& route = routes[r];
            ids[r] = static_cast<std::uint32_t>(route.id);
            probabilities[r] = route.probability;
            tensor_linear(moe->gate[route.id], normalized, gate, 0, &scratch);
            tensor_linear(moe->up[route.id], normalized, up, 0, &scratch);
            for (std::size_t i = 0; i < activated.size(); ++i) {
                activated[i] = (gate[i] / (1.0F + std::exp(-gate[i]))) * up[i];
            }
            tensor_linear(moe->down[route.id], activated, expert_output, 0, &scratch);
            for (std::size_t i = 0; i < moe_result.size(); ++i) {
                moe_result[i] += route.probability * expert_output[i];
            }
        }
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

// Greedy generation with the reference Qwen3MoeRunner on a GGUF file: every
// prompt token through forward_token (:785-790), then n_new tokens by
// first-max argmax (sample_token at temperature 0, :320-333) without an EOS
// stop.  out_tokens[n_new]; last_logits (optional, vocab floats) receives the
// logits after the final prompt token.  decode_seconds (optional) receives
// the wall time of the n_new - 1 decode forwards.
int pkref_qwen3moe_greedy(const char* path, const std::uint32_t* prompt, std::uint32_t n_prompt,
                          std::uint32_t n_new, std::uint64_t expert_cache_bytes,
                          std::uint32_t* out_tokens, float* last_logits, double* decode_seconds) {
    try {
        if (!path || !prompt || n_prompt == 0 || !out_tokens) {
            throw std::invalid_argument("path, prompt and output are required");
        }
        pokitlms::model::Qwen3MoeRunner runner(path, static_cast<std::size_t>(expert_cache_bytes));
        std::vector<float> logits;
        for (std::uint32_t i = 0; i < n_prompt; ++i) logits = runner.forward_token(prompt[i], i);
        if (last_logits) std::copy(logits.begin(), logits.end(), last_logits);
        const auto argmax = [](const std::vector<float>& l) {
            std::size_t best = 0;
            for (std::size_t i = 0; i < l.size(); ++i) {
                if (!std::isfinite(l[i])) throw std::runtime_error("model produced non-finite logits");
                if (l[i] > l[best]) best = i;
            }
            return static_cast<std::uint32_t>(best);
        };
        const auto start = std::chrono::steady_clock::now();
        for (std::uint32_t j = 0; j < n_new; ++j) {
            out_tokens[j] = argmax(logits);
            if (j + 1 < n_new) logits = runner.forward_token(out_tokens[j], n_prompt + j);
        }
        if (decode_seconds) {
            *decode_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - start)
                                  .count();
        }
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

// Steady-state decode cost of the reference runner: feeds the prompt, then
// n_forwards greedy forwards, writing each forward's wall seconds (argmax
// included, as the runner's generate loop pays it).
int pkref_qwen3moe_forward_times(const char* path, const std::uint32_t* prompt,
                                 std::uint32_t n_prompt, std::uint32_t n_forwards,
                                 std::uint64_t expert_cache_bytes, double* seconds) {
    try {
        if (!path || !prompt || n_prompt == 0 || !seconds) {
            throw std::invalid_argument("path, prompt and output are required");
        }
        pokitlms::model::Qwen3MoeRunner runner(path, static_cast<std::size_t>(expert_cache_bytes));
        std::vector<float> logits;
        for (std::uint32_t i = 0; i < n_prompt; ++i) logits = runner.forward_token(prompt[i], i);
        for (std::uint32_t j = 0; j < n_forwards; ++j) {
            const auto start = std::chrono::steady_clock::now();
            const auto best = static_cast<std::uint32_t>(
                std::max_element(logits.begin(), logits.end()) - logits.begin());
            logits = runner.forward_token(best, n_prompt + j);
            seconds[j] = std::chrono::duration<double>(std::chrono::steady_clock::now() - start)
                             .count();
        }
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}


// One layer's attention for positions 0 .. steps - 1 with the reference's own
// functions, in the order of the runner's token step (:610-628): rms_norm of
// every q and k head, prepare_qwen_rope / apply_qwen_rope, KvCache::append
// and KvCache::attend with an FP16 cache of `capacity` positions.
int pkref_attention_steps(std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t head_dim,
                          std::uint32_t capacity, float eps, float theta, const float* q_norm,
                          const float* k_norm, std::uint32_t steps, const float* q,
                          const float* k, const float* v, float* out) {
    try {
        const std::size_t qd = std::size_t{heads} * head_dim, kd = std::size_t{kv_heads} * head_dim;
        pokitlms::KvCache cache(capacity, kv_heads, head_dim, head_dim,
                                pokitlms::KvCachePrecision::Float16, heads);
        std::vector<float> query(qd), key(kd), cosine(head_dim / 2), sine(head_dim / 2);
        const std::span<const float> qn(q_norm, head_dim), kn(k_norm, head_dim);
        for (std::uint32_t t = 0; t < steps; ++t) {
            std::copy_n(q + t * qd, qd, query.begin());
            std::copy_n(k + t * kd, kd, key.begin());
            for (std::size_t h = 0; h < heads; ++h) {
                auto* b = query.data() + h * head_dim;
                pokitlms::rms_norm(std::span<const float>(b, head_dim), qn,
                                   std::span<float>(b, head_dim), eps);
            }
            for (std::size_t h = 0; h < kv_heads; ++h) {
                auto* b = key.data() + h * head_dim;
                pokitlms::rms_norm(std::span<const float>(b, head_dim), kn,
                                   std::span<float>(b, head_dim), eps);
            }
            pokitlms::model::prepare_qwen_rope(t, head_dim, theta, cosine, sine);
            pokitlms::model::apply_qwen_rope(query, head_dim, head_dim, cosine, sine);
            pokitlms::model::apply_qwen_rope(key, head_dim, head_dim, cosine, sine);
            cache.append(t, key.data(), kd, v + t * kd, kd);
            cache.attend(query.data(), qd, out + t * qd, qd);
        }
        return 0;
    } catch (...) {
        return status_of_current_exception();
    }
}

}  // extern "C"
