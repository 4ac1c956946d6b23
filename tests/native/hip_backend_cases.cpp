// hip_backend_cases.cpp -- parity of HipLinearBackend inside the reference's
// own call sites.
//
// TEST INFRASTRUCTURE.  oracle/Makefile builds this program against the
// reference headers and its compiled CPU library (oracle/_ref/libpkref.so,
// built in place from /root/reference/src) and links the product's C ABI
// library; tests/test_native_backend.py runs it.  It plays the role of the
// reference's Vulkan harness (tests/vulkan_linear_cases.hpp:16-104): the same
// shapes (37 rows; 257 columns for float types, 512 for block types), three
// repeats with a rescaled input so stale buffers cannot pass, and the CPU
// kernels as the comparison, here through tensor_linear's backend hook
// (src/tensor_linear.cpp:213) rather than by calling try_linear directly.
//
//   hip_backend_cases [DENSE.gguf MOE.gguf]
//                                     run every case on HIP device 0; with the
//                                     two Qwen3.5 smoke models, also the runner
//                                     parity of tests/vulkan_linear_test.cpp:9-36
//   hip_backend_cases --expect-no-device
//                                     check that construction fails cleanly
//                                     on a host without a GPU
#include "hip_linear_backend.hpp"

#include "pokitlms/model/qwen35_runner.hpp"
#include "pokitlms/model/tensor_linear.hpp"
#include "pokitlms/model/tensor_reader.hpp"
#include "pokitlms/storage/model_file.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <numbers>
#include <stdexcept>
#include <string>
#include <unistd.h>
#include <vector>

// The reference MoE block, compiled from src/qwen3_moe_runner.cpp by oracle/ref_shim.cpp.
extern "C" {
struct pkref_moe;
pkref_moe* pkref_moe_create(const float* router, std::uint32_t hidden, std::uint32_t experts,
                            std::uint32_t ffn, std::uint32_t gate_type, const void* gate,
                            std::uint32_t up_type, const void* up, std::uint32_t down_type,
                            const void* down, std::uint32_t top_k, int normalize);
int pkref_moe_forward(pkref_moe* moe, const float* x, float* y, std::uint32_t* ids,
                      float* probabilities);
void pkref_moe_destroy(pkref_moe* moe);

// The reference Qwen3.5-MoE block (src/qwen35_runner.cpp:670-764, with its
// select_experts, silu and sigmoid), compiled by oracle/ref_shim35.cpp.
struct pkref_moe35;
pkref_moe35* pkref_moe35_create(const float* router, std::uint32_t hidden, std::uint32_t experts,
                                std::uint32_t ffn, std::uint32_t gate_type, const void* gate,
                                std::uint32_t up_type, const void* up, std::uint32_t down_type,
                                const void* down, std::uint32_t top_k, int normalize, float scale,
                                const float* shared_router, std::uint32_t shared_ffn,
                                std::uint32_t sgate_type, const void* sgate,
                                std::uint32_t sup_type, const void* sup,
                                std::uint32_t sdown_type, const void* sdown);
int pkref_moe35_forward(pkref_moe35* m, const float* x, float* y, std::uint32_t* ids,
                        float* weights);
void pkref_moe35_destroy(pkref_moe35* m);
}

namespace {

using pokitlms::gpu::HipLinearBackend;
using pokitlms::gpu::HipLinearOptions;
using pokitlms::model::TensorInfo;
using pokitlms::model::TensorReader;

int g_failed = 0, g_passed = 0;

void report(bool ok, const std::string& name, const std::string& detail) {
    std::printf("%s %s %s\n", ok ? "PASS" : "FAIL", name.c_str(), detail.c_str());
    std::fflush(stdout);
    (ok ? g_passed : g_failed) += 1;
}

// splitmix64: a small seeded generator for bytes, uniforms and normals.
struct Rng {
    std::uint64_t s;
    explicit Rng(std::uint64_t seed) : s(seed) {}
    std::uint64_t next() {
        std::uint64_t z = (s += 0x9e3779b97f4a7c15ULL);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        return z ^ (z >> 31);
    }
    double uniform() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }
    float normal(float sigma) {
        const double u1 = std::max(uniform(), 1e-300), u2 = uniform();
        return static_cast<float>(sigma * std::sqrt(-2.0 * std::log(u1)) *
                                  std::cos(2.0 * std::numbers::pi * u2));
    }
};

std::size_t block_elements(std::uint32_t type) {
    return type == 0 || type == 1 || type == 30 ? 1 : type >= 10 && type != 30 ? 256 : 32;
}

std::size_t block_bytes(std::uint32_t type) {
    switch (type) {
        case 0: return 4;
        case 1: case 30: return 2;
        case 2: return 18;
        case 3: return 20;
        case 6: return 22;
        case 7: return 24;
        case 8: return 34;
        case 10: return 84;
        case 11: return 110;
        case 12: return 144;
        case 13: return 176;
        case 14: return 210;
        default: throw std::invalid_argument("type not in this harness");
    }
}

void put_half(std::byte* p, std::uint16_t v) {
    p[0] = static_cast<std::byte>(v & 0xff);
    p[1] = static_cast<std::byte>(v >> 8);
}

// A positive binary16 scale in [2^-8, 2^-5): the reference harness's scale
// magnitudes (2^-5 / 2^-6), randomised; finite products for any quants.
std::uint16_t scale_half(Rng& g) { return static_cast<std::uint16_t>(0x1c00 + g.next() % 0x0c00); }

// rows x in GGUF payload: random quant fields, bounded scales; float types hold
// finite values of both signs.
std::vector<std::byte> make_matrix(std::uint32_t type, std::size_t rows, std::size_t in, Rng& g) {
    const std::size_t be = block_elements(type), bb = block_bytes(type);
    const std::size_t blocks = rows * (in / be);
    std::vector<std::byte> out(blocks * bb);
    if (type == 0) {
        for (std::size_t i = 0; i < rows * in; ++i) {
            const float v = static_cast<float>(g.uniform() * 2.0 - 1.0);
            std::memcpy(out.data() + 4 * i, &v, 4);
        }
        return out;
    }
    if (type == 1 || type == 30) {
        for (std::size_t i = 0; i < rows * in; ++i) {
            const std::uint64_t r = g.next();
            const std::uint16_t mag = type == 1 ? 0x3400 + (r & 0x7ff) : 0x3e80 + (r & 0xff);
            put_half(out.data() + 2 * i, static_cast<std::uint16_t>(mag | ((r >> 16) & 0x8000)));
        }
        return out;
    }
    for (auto& b : out) b = static_cast<std::byte>(g.next() & 0xff);
    for (std::size_t k = 0; k < blocks; ++k) {
        std::byte* blk = out.data() + k * bb;
        switch (type) {  // scale fields (src/quantized_linear.cpp:54-55,98-99,140,167-168,334)
            case 14: put_half(blk + 208, scale_half(g)); break;
            case 11: put_half(blk + 108, scale_half(g)); break;
            case 10:
                put_half(blk + 80, scale_half(g));
                put_half(blk + 82, scale_half(g));
                break;
            case 12: case 13: case 3: case 7:
                put_half(blk, scale_half(g));
                put_half(blk + 2, scale_half(g));
                break;
            default: put_half(blk, scale_half(g)); break;  // Q4_0, Q5_0, Q8_0
        }
    }
    return out;
}

TensorReader memory_reader(std::uint32_t type, std::size_t rows, std::size_t in,
                           std::vector<std::byte> bytes) {
    TensorInfo t;
    t.name = "hip_case";
    t.dimensions = {in, rows};
    t.type = type;
    t.payload_size = bytes.size();
    return TensorReader(t, std::make_shared<const std::vector<std::byte>>(std::move(bytes)));
}

struct Errors {
    double normwise = 0.0;  // max|g - c| / max|c|
    bool harness_ok = true; // |g - c| <= 1e-3 + 2e-5 |c| (vulkan_linear_cases.hpp:81)
};

Errors compare(const std::vector<float>& got, const std::vector<float>& want) {
    Errors e;
    double max_diff = 0.0, max_ref = 0.0;
    for (std::size_t i = 0; i < want.size(); ++i) {
        const double d = std::abs(static_cast<double>(got[i]) - want[i]);
        if (!std::isfinite(got[i]) || d > 1e-3 + 2e-5 * std::abs(want[i])) e.harness_ok = false;
        max_diff = std::max(max_diff, d);
        max_ref = std::max(max_ref, std::abs(static_cast<double>(want[i])));
    }
    e.normwise = max_ref > 0 ? max_diff / max_ref : max_diff;
    return e;
}

// ---- try_linear through tensor_linear's hook -------------------------------------

void linear_cases(HipLinearBackend& hip) {
    Rng g(0x5eed0001);
    // every type tensor_linear dispatches (src/tensor_linear.cpp:162-188)
    for (const std::uint32_t type : {0U, 1U, 30U, 2U, 3U, 6U, 7U, 8U, 10U, 11U, 12U, 13U, 14U}) {
        const std::size_t in = block_elements(type) == 1 ? 257 : 512, rows = 37;
        const auto reader = memory_reader(type, rows, in, make_matrix(type, rows, in, g));
        std::vector<float> x(in), cpu(rows), gpu(rows);
        for (auto& v : x) v = static_cast<float>(static_cast<int>(g.next() % 2049) - 1024) / 1024.0F;
        pokitlms::model::TensorLinearScratch scratch;
        scratch.backend = &hip;
        double worst = 0.0;
        bool ok = true;
        for (int repeat = 0; repeat < 3; ++repeat) {
            const auto before = hip.stats().linear_calls;
            pokitlms::model::tensor_linear(reader, x, cpu);
            std::fill(gpu.begin(), gpu.end(), std::nanf(""));
            pokitlms::model::tensor_linear(reader, x, gpu, 0, &scratch);
            const auto e = compare(gpu, cpu);
            worst = std::max(worst, e.normwise);
            ok = ok && e.harness_ok && e.normwise <= 1e-4 && hip.stats().linear_calls == before + 1;
            for (auto& v : x) v *= -0.75F;
        }
        char d[160];
        std::snprintf(d, sizeof d, "type=%u rows=%zu in=%zu max_normwise=%.3g", type, rows, in, worst);
        report(ok, "try_linear_parity", d);
    }
}

void unsupported_cases(HipLinearBackend& hip) {
    // A GGUF type without a kernel here (Q8_K, 15; tensor_linear's own type
    // gate rejects it too, src/tensor_linear.cpp:205-211): try_linear answers
    // false and counts it, as the Vulkan backend does for types outside its
    // list (src/vulkan_linear.cpp:615).
    Rng g(0x5eed0002);
    const std::size_t in = 256, rows = 4;
    std::vector<std::byte> bytes(rows * 292);
    for (auto& b : bytes) b = static_cast<std::byte>(g.next() & 0xff);
    const auto reader = memory_reader(15, rows, in, std::move(bytes));
    std::vector<float> x(in, 1.0F), y(rows, 0.0F);
    const auto before = hip.stats();
    bool direct = true;
    try {
        direct = hip.try_linear(reader, x, y);
    } catch (const std::exception&) {
        direct = true;
    }
    const auto after = hip.stats();
    const bool ok = !direct && after.linear_calls == before.linear_calls &&
                    after.unsupported_calls == before.unsupported_calls + 1;
    report(ok, "try_linear_unsupported", "type=15");
}

template <typename E, typename F>
bool throws(F&& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

void shape_error_cases(HipLinearBackend& hip) {
    Rng g(0x5eed0003);
    const auto reader = memory_reader(12, 8, 512, make_matrix(12, 8, 512, g));
    std::vector<float> x(512, 1.0F), y(8), short_y(7), short_x(256, 1.0F);
    report(throws<std::invalid_argument>([&] { (void)hip.try_linear(reader, x, short_y); }),
           "try_linear_shape_error", "output rows");
    report(throws<std::invalid_argument>([&] { (void)hip.try_linear(reader, short_x, y); }),
           "try_linear_shape_error", "input columns");
    // Still usable after argument errors (they do not fail the backend).
    report(hip.try_linear(reader, x, y), "try_linear_after_shape_error", "");
}

// ---- file-backed tensors stay resident ----------------------------------------------

void file_backed_cases(HipLinearBackend& hip) {
    Rng g(0x5eed0004);
    const std::size_t rows = 96, in = 1024, offset = 4096;
    const auto bytes = make_matrix(14, rows, in, g);
    char path[] = "/tmp/pk_hip_caseXXXXXX";
    const int fd = mkstemp(path);
    if (fd < 0) {
        report(false, "file_backed", "mkstemp failed");
        return;
    }
    close(fd);
    {
        std::ofstream f(path, std::ios::binary);
        const std::vector<char> pad(offset, 0);
        f.write(pad.data(), static_cast<std::streamsize>(pad.size()));
        f.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
    }
    auto file = std::make_shared<pokitlms::storage::ModelFile>(path);
    TensorInfo t;
    t.name = "resident";
    t.dimensions = {in, rows};
    t.type = 14;
    t.file_offset = offset;
    t.payload_size = bytes.size();
    const TensorReader reader(file, t);
    std::vector<float> x(in), cpu(rows), gpu(rows);
    for (auto& v : x) v = g.normal(1.0F);
    const auto before = hip.stats();
    bool ok = true;
    double worst = 0.0;
    for (int call = 0; call < 3; ++call) {
        pokitlms::model::tensor_linear(reader, x, cpu);
        ok = ok && hip.try_linear(reader, x, gpu);
        const auto e = compare(gpu, cpu);
        worst = std::max(worst, e.normwise);
        ok = ok && e.harness_ok && e.normwise <= 1e-4;
        for (auto& v : x) v *= 1.5F;
    }
    const auto after = hip.stats();
    ok = ok && after.resident_tensors == before.resident_tensors + 1 &&
         after.transient_uploads == before.transient_uploads &&
         after.uploaded_bytes == before.uploaded_bytes + bytes.size();
    std::filesystem::remove(path);
    char d[160];
    std::snprintf(d, sizeof d, "Q6_K %zux%zu, 3 calls, 1 upload, max_normwise=%.3g", rows, in, worst);
    report(ok, "file_backed_resident", d);
}

// Two files opened one after the other, with different tensors at the same
// offset: the second must not be served the first one's resident copy, even
// when its ModelFile lands at the address the first one had.
void file_reload_cases(HipLinearBackend& hip) {
    Rng g(0x5eed0014);
    const std::size_t rows = 40, in = 512, offset = 4096;
    char path[] = "/tmp/pk_hip_reloadXXXXXX";
    const int fd = mkstemp(path);
    if (fd < 0) {
        report(false, "file_reload", "mkstemp failed");
        return;
    }
    close(fd);
    const std::uint32_t types[2] = {12, 14};
    bool ok = true;
    double worst = 0.0;
    const auto before = hip.stats();
    for (int round = 0; round < 2; ++round) {
        const auto bytes = make_matrix(types[round], rows, in, g);
        {
            std::ofstream f(path, std::ios::binary | std::ios::trunc);
            const std::vector<char> pad(offset, 0);
            f.write(pad.data(), static_cast<std::streamsize>(pad.size()));
            f.write(reinterpret_cast<const char*>(bytes.data()),
                    static_cast<std::streamsize>(bytes.size()));
        }
        auto file = std::make_shared<pokitlms::storage::ModelFile>(path);
        TensorInfo t;
        t.name = "reloaded";
        t.dimensions = {in, rows};
        t.type = types[round];
        t.file_offset = offset;
        t.payload_size = bytes.size();
        const TensorReader reader(file, t);
        std::vector<float> x(in), cpu(rows), gpu(rows);
        for (auto& v : x) v = g.normal(1.0F);
        pokitlms::model::tensor_linear(reader, x, cpu);
        ok = ok && hip.try_linear(reader, x, gpu);
        const auto e = compare(gpu, cpu);
        worst = std::max(worst, e.normwise);
        ok = ok && e.harness_ok && e.normwise <= 1e-4;
    }  // each file is released before the next one is opened
    const auto after = hip.stats();
    ok = ok && after.resident_tensors == before.resident_tensors + 2;
    std::filesystem::remove(path);
    char d[160];
    std::snprintf(d, sizeof d, "Q4_K then Q6_K at one offset, 2 uploads, max_normwise=%.3g", worst);
    report(ok, "file_reload", d);
}

// In-memory tensors: with the LRU set opted in, a repeat with the same bytes is
// served from it and the same name, offset and shape with different bytes is
// uploaded again; by default (no set, as the Vulkan backend) every call uploads.
void transient_cache_round(HipLinearBackend& hip, bool opted_in) {
    Rng g(0x5eed0015);
    const std::size_t rows = 48, in = 1024;
    std::vector<float> x(in), cpu(rows), gpu(rows);
    for (auto& v : x) v = g.normal(1.0F);
    bool ok = true;
    double worst = 0.0;
    const auto before = hip.stats();
    for (int round = 0; round < 3; ++round) {
        // rounds 0 and 1: one matrix; round 2: new bytes under the same key
        static std::vector<std::byte> bytes;
        if (round != 1) bytes = make_matrix(13, rows, in, g);
        TensorInfo t;
        t.name = "blk.0.ffn_gate_exps.weight";
        t.dimensions = {in, rows};
        t.type = 13;
        t.file_offset = 123456;
        t.payload_size = bytes.size();
        auto payload = std::make_shared<std::vector<std::byte>>(bytes.size());
        std::memcpy(payload->data(), bytes.data(), bytes.size());
        const TensorReader reader(t, payload);
        pokitlms::model::tensor_linear(reader, x, cpu);
        ok = ok && hip.try_linear(reader, x, gpu);
        const auto e = compare(gpu, cpu);
        worst = std::max(worst, e.normwise);
        ok = ok && e.harness_ok && e.normwise <= 1e-4;
    }
    const auto after = hip.stats();
    const std::uint64_t hits = opted_in ? 1 : 0, uploads = opted_in ? 2 : 3;
    ok = ok && after.transient_hits == before.transient_hits + hits &&
         after.transient_uploads == before.transient_uploads + uploads &&
         (opted_in || after.transient_bytes == 0);
    char d[160];
    std::snprintf(d, sizeof d, "Q5_K in-memory, %s: %llu uploads, %llu hits, max_normwise=%.3g",
                  opted_in ? "LRU set of 1 GiB" : "default (no set)",
                  static_cast<unsigned long long>(uploads), static_cast<unsigned long long>(hits),
                  worst);
    report(ok, opted_in ? "transient_cache" : "transient_default", d);
}

void transient_cache_cases(HipLinearBackend& hip) {
    transient_cache_round(hip, false);
    HipLinearOptions options;
    options.transient_cache_bytes = std::size_t{1} << 30;
    HipLinearBackend cached(options);
    transient_cache_round(cached, true);
}

// The reference runner driven through the backend (tests/vulkan_linear_test.cpp:9-36):
// Qwen35Runner::set_linear_backend, then generate_chat must equal the CPU runner's,
// with and without the file-tensor cache, on the dense and MoE smoke models.
void runner_cases(const char* dense, const char* moe) {
    for (const bool cache : {true, false}) {
        HipLinearOptions options;
        options.cache_file_tensors = cache;
        auto backend = std::make_shared<HipLinearBackend>(options);
        bool ok = true;
        std::string detail;
        for (const char* path : {dense, moe}) {
            pokitlms::model::Qwen35Runner cpu(path), gpu(path);
            gpu.set_linear_backend(backend);
            for (const char* prompt : {"hi", "hello", "again"}) {
                const auto expected = cpu.generate_chat(prompt, 5);
                const auto got = gpu.generate_chat(prompt, 5);
                if (got != expected) {
                    ok = false;
                    detail += std::string(" mismatch on '") + prompt + "'";
                }
            }
        }
        const auto s = backend->stats();
        ok = ok && s.linear_calls > 0 && (cache ? s.resident_tensors > 0 : s.resident_tensors == 0);
        char d[200];
        std::snprintf(d, sizeof d, "file cache %s: linear_calls=%llu resident=%llu transient=%llu/%llu%s",
                      cache ? "on" : "off", static_cast<unsigned long long>(s.linear_calls),
                      static_cast<unsigned long long>(s.resident_tensors),
                      static_cast<unsigned long long>(s.transient_hits),
                      static_cast<unsigned long long>(s.transient_uploads), detail.c_str());
        report(ok, "runner_parity", d);
    }
}

// ---- the MoE block hook -----------------------------------------------------------------

struct Layer {
    std::uint32_t hidden, experts, ffn, top_k;
    bool normalize;
    std::vector<float> router;
    std::vector<std::byte> gate, up, down;
};

Layer make_layer(std::uint32_t hidden, std::uint32_t experts, std::uint32_t ffn,
                 std::uint32_t top_k, bool normalize, std::uint64_t seed) {
    Rng g(seed);
    Layer L{hidden, experts, ffn, top_k, normalize, {}, {}, {}, {}};
    L.router.resize(std::size_t{hidden} * experts);
    for (auto& v : L.router) v = g.normal(0.02F);
    L.gate = make_matrix(12, std::size_t{experts} * ffn, hidden, g);
    L.up = make_matrix(12, std::size_t{experts} * ffn, hidden, g);
    L.down = make_matrix(14, std::size_t{experts} * hidden, ffn, g);
    return L;
}

TensorReader tensor3(std::uint32_t type, std::uint64_t in, std::uint64_t out,
                     std::uint64_t experts, const std::vector<std::byte>& bytes) {
    TensorInfo t;
    t.name = "experts";
    t.dimensions = {in, out, experts};
    t.type = type;
    t.payload_size = bytes.size();
    return TensorReader(t, std::make_shared<const std::vector<std::byte>>(bytes));
}

void moe_cases(HipLinearBackend& hip, const Layer& L, const char* label, int tokens) {
    std::vector<std::byte> router_bytes(L.router.size() * 4);
    std::memcpy(router_bytes.data(), L.router.data(), router_bytes.size());
    TensorInfo rt;
    rt.name = "router";
    rt.dimensions = {L.hidden, L.experts};
    rt.type = 0;
    rt.payload_size = router_bytes.size();
    const TensorReader router(rt, std::make_shared<const std::vector<std::byte>>(router_bytes));
    const auto layer = hip.upload_moe_layer(router, tensor3(12, L.hidden, L.ffn, L.experts, L.gate),
                                            tensor3(12, L.hidden, L.ffn, L.experts, L.up),
                                            tensor3(14, L.ffn, L.hidden, L.experts, L.down),
                                            L.top_k, L.normalize);
    pkref_moe* ref = pkref_moe_create(L.router.data(), L.hidden, L.experts, L.ffn, 12,
                                      L.gate.data(), 12, L.up.data(), 14, L.down.data(), L.top_k,
                                      L.normalize ? 1 : 0);
    if (!ref) {
        report(false, "moe_block", std::string(label) + ": reference block not created");
        return;
    }
    Rng g(0x70c0 + L.hidden);
    std::vector<float> x(L.hidden), y(L.hidden), cy(L.hidden), probs(L.top_k), cprobs(L.top_k);
    std::vector<std::uint32_t> ids(L.top_k), cids(L.top_k);
    bool ok = true;
    double worst = 0.0, worst_p = 0.0;
    for (int t = 0; t < tokens; ++t) {
        for (auto& v : x) v = g.normal(1.0F);
        ok = ok && hip.try_moe_block(*layer, x, y, ids, probs);
        ok = ok && pkref_moe_forward(ref, x.data(), cy.data(), cids.data(), cprobs.data()) == 0;
        ok = ok && ids == cids;
        for (std::uint32_t r = 0; r < L.top_k; ++r)
            worst_p = std::max(worst_p, std::abs(static_cast<double>(probs[r]) - cprobs[r]) /
                                            std::max(1e-30, static_cast<double>(cprobs[r])));
        worst = std::max(worst, compare(y, cy).normwise);
    }
    ok = ok && worst <= 1e-4 && worst_p <= 1e-5;
    pkref_moe_destroy(ref);
    char d[200];
    std::snprintf(d, sizeof d, "%s: %d tokens, ids equal, max_normwise=%.3g, max_prob_rel=%.3g",
                  label, tokens, worst, worst_p);
    report(ok, "moe_block_parity", d);
}

TensorReader tensor2(std::uint32_t type, std::uint64_t in, std::uint64_t out,
                     const std::vector<std::byte>& bytes) {
    TensorInfo t;
    t.name = "shared";
    t.dimensions = {in, out};
    t.type = type;
    t.payload_size = bytes.size();
    return TensorReader(t, std::make_shared<const std::vector<std::byte>>(bytes));
}

// The Qwen3.5 block through try_moe_block with the shared expert attached,
// against the reference block: ids equal, weights and mixer outputs within
// 1e-4 normwise.
void moe35_cases(HipLinearBackend& hip, const Layer& L, float scale, const char* label, int tokens) {
    Rng g(0x35 + L.hidden);
    std::vector<float> shared_router(L.hidden);
    for (auto& v : shared_router) v = g.normal(0.2F);
    const auto sgate = make_matrix(12, L.ffn, L.hidden, g), sup = make_matrix(12, L.ffn, L.hidden, g);
    const auto sdown = make_matrix(14, L.hidden, L.ffn, g);
    std::vector<std::byte> router_bytes(L.router.size() * 4), srouter_bytes(L.hidden * 4);
    std::memcpy(router_bytes.data(), L.router.data(), router_bytes.size());
    std::memcpy(srouter_bytes.data(), shared_router.data(), srouter_bytes.size());
    TensorInfo rt;
    rt.name = "router";
    rt.dimensions = {L.hidden, L.experts};
    rt.type = 0;
    rt.payload_size = router_bytes.size();
    const TensorReader router(rt, std::make_shared<const std::vector<std::byte>>(router_bytes));
    TensorInfo st;
    st.name = "ffn_gate_inp_shexp";
    st.dimensions = {L.hidden};
    st.type = 0;
    st.payload_size = srouter_bytes.size();
    const TensorReader srouter(st, std::make_shared<const std::vector<std::byte>>(srouter_bytes));
    const auto layer = hip.upload_moe_layer(router, tensor3(12, L.hidden, L.ffn, L.experts, L.gate),
                                            tensor3(12, L.hidden, L.ffn, L.experts, L.up),
                                            tensor3(14, L.ffn, L.hidden, L.experts, L.down),
                                            L.top_k, L.normalize, scale);
    hip.attach_shared_expert(*layer, srouter, tensor2(12, L.hidden, L.ffn, sgate),
                             tensor2(12, L.hidden, L.ffn, sup), tensor2(14, L.ffn, L.hidden, sdown));
    pkref_moe35* ref = pkref_moe35_create(
        L.router.data(), L.hidden, L.experts, L.ffn, 12, L.gate.data(), 12, L.up.data(), 14,
        L.down.data(), L.top_k, L.normalize ? 1 : 0, scale, shared_router.data(), L.ffn, 12,
        sgate.data(), 12, sup.data(), 14, sdown.data());
    if (!ref) {
        report(false, "moe35_block", std::string(label) + ": reference block not created");
        return;
    }
    std::vector<float> x(L.hidden), y(L.hidden), cy(L.hidden), w(L.top_k), cw(L.top_k);
    std::vector<std::uint32_t> ids(L.top_k), cids(L.top_k);
    bool ok = true;
    double worst = 0.0, worst_w = 0.0;
    for (int t = 0; t < tokens; ++t) {
        for (auto& v : x) v = g.normal(1.0F);
        ok = ok && hip.try_moe_block(*layer, x, y, ids, w);
        ok = ok && pkref_moe35_forward(ref, x.data(), cy.data(), cids.data(), cw.data()) == 0;
        ok = ok && ids == cids;
        for (auto& v : cw) v *= scale;  // the shim returns select_experts' weights before the scale
        worst_w = std::max(worst_w, compare(w, cw).normwise);
        worst = std::max(worst, compare(y, cy).normwise);
    }
    ok = ok && worst <= 1e-4 && worst_w <= 1e-4;
    pkref_moe35_destroy(ref);
    char d[200];
    std::snprintf(d, sizeof d, "%s: %d tokens, ids equal, max_normwise=%.3g, weights %.3g", label,
                  tokens, worst, worst_w);
    report(ok, "moe35_block_parity", d);
}

void moe_error_cases(HipLinearBackend& hip) {
    Layer L = make_layer(512, 16, 256, 4, true, 0xbad);
    L.router[5 * 512 + 17] = INFINITY;  // expert 5's logit is not finite
    std::vector<std::byte> router_bytes(L.router.size() * 4);
    std::memcpy(router_bytes.data(), L.router.data(), router_bytes.size());
    TensorInfo rt;
    rt.name = "router";
    rt.dimensions = {L.hidden, L.experts};
    rt.type = 0;
    rt.payload_size = router_bytes.size();
    const TensorReader router(rt, std::make_shared<const std::vector<std::byte>>(router_bytes));
    const auto layer = hip.upload_moe_layer(router, tensor3(12, 512, 256, 16, L.gate),
                                            tensor3(12, 512, 256, 16, L.up),
                                            tensor3(14, 256, 512, 16, L.down), 4, true);
    std::vector<float> x(512, 1.0F), y(512);
    report(throws<std::runtime_error>([&] { (void)hip.try_moe_block(*layer, x, y); }),
           "moe_non_finite_router", "route_experts throws on non-finite logits");
    // A data error leaves the backend usable.
    Rng g(3);
    const auto reader = memory_reader(12, 8, 512, make_matrix(12, 8, 512, g));
    std::vector<float> y8(8);
    report(hip.try_linear(reader, x, y8), "usable_after_data_error", "");
    std::vector<float> short_x(256);
    report(throws<std::invalid_argument>([&] { (void)hip.try_moe_block(*layer, short_x, y); }),
           "moe_shape_error", "hidden size");
}

}  // namespace

int main(int argc, char** argv) {
    if (argc > 1 && std::string(argv[1]) == "--expect-no-device") {
        try {
            HipLinearBackend hip;
            std::printf("FAIL construction succeeded without a device\n");
            return 1;
        } catch (const std::runtime_error& e) {
            std::printf("PASS no_device %s\n", e.what());
            return 0;
        }
    }
    try {
        HipLinearBackend hip;
        std::printf("device %s\n", hip.device_name().c_str());
        linear_cases(hip);
        unsupported_cases(hip);
        shape_error_cases(hip);
        file_backed_cases(hip);
        file_reload_cases(hip);
        transient_cache_cases(hip);
        moe_cases(hip, make_layer(512, 16, 256, 4, false, 0x5eed0005), "hidden 512, 16 experts, top-4", 16);
        moe35_cases(hip, make_layer(1024, 32, 512, 6, true, 0x5eed0035), 2.5F,
                    "Qwen3.5 hidden 1024, 32 experts, top-6, scale 2.5", 16);
        moe_cases(hip, make_layer(2048, 128, 768, 8, true, 0x5eed0006),
                  "hidden 2048, 128 experts, top-8 (config 3 shape)", 16);
        moe_error_cases(hip);
        const auto ec = hip.expert_cache_stats();
        report(ec.capacity_bytes == 0 && ec.hits > 0 && ec.misses == 0, "expert_cache_stats",
               "layers released: no resident expert bytes, every routed access a hit");
        if (argc > 2) runner_cases(argv[1], argv[2]);
        const auto s = hip.stats();
        std::printf("stats linear_calls=%llu moe_calls=%llu dispatches=%llu resident_tensors=%llu "
                    "transient_uploads=%llu router_fallbacks=%llu\n",
                    static_cast<unsigned long long>(s.linear_calls),
                    static_cast<unsigned long long>(s.moe_calls),
                    static_cast<unsigned long long>(s.dispatches),
                    static_cast<unsigned long long>(s.resident_tensors),
                    static_cast<unsigned long long>(s.transient_uploads),
                    static_cast<unsigned long long>(s.router_fallbacks));
    } catch (const std::exception& e) {
        std::printf("FAIL exception %s\n", e.what());
        ++g_failed;
    }
    std::printf("hip_backend_cases: %d passed, %d failed\n", g_passed, g_failed);
    return g_failed ? 1 : 0;
}
