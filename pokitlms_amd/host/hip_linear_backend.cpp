// hip_linear_backend.cpp -- HipLinearBackend over the libpokit_hip C ABI.
//
// Mirrors the behaviour of VulkanLinearBackend::try_linear
// (src/vulkan_linear.cpp:612-736): the same type gate, the same shape and
// row-size checks with std::invalid_argument, one internal mutex, and a
// permanent failed state after any device error.  Weights differ by design:
// file-backed tensors are uploaded once and stay resident in HBM, keyed by
// model file and offset and held only while that file is alive (the Vulkan
// cache holds the file's shared_ptr, src/vulkan_linear.cpp:519-526); in-memory
// tensors go through a content-checked LRU set.
#include "hip_linear_backend.hpp"

#include "pokit_hip.h"

#include <dlfcn.h>

#include <array>
#include <cstring>
#include <fstream>
#include <iterator>
#include <limits>
#include <list>
#include <map>
#include <tuple>
#include <mutex>
#include <stdexcept>
#include <utility>
#include <vector>

namespace pokitlms::gpu {
namespace {

constexpr std::size_t kErrorCapacity = 512;

struct ErrorBuffer {
    std::array<char, kErrorCapacity> text{};
    char* data() noexcept { return text.data(); }
    [[nodiscard]] std::string str() const { return std::string(text.data()); }
};

// Encoded bytes of one row of `in` elements; 0 for types without a kernel.
std::size_t encoded_row_bytes(std::uint32_t type, std::uint64_t in) {
    switch (type) {
        case 0: return in * 4;
        case 1: case 30: return in * 2;
        case 2: return in % 32 ? 0 : in / 32 * 18;
        case 3: return in % 32 ? 0 : in / 32 * 20;
        case 6: return in % 32 ? 0 : in / 32 * 22;
        case 7: return in % 32 ? 0 : in / 32 * 24;
        case 8: return in % 32 ? 0 : in / 32 * 34;
        case 10: return in % 256 ? 0 : in / 256 * 84;
        case 11: return in % 256 ? 0 : in / 256 * 110;
        case 12: return in % 256 ? 0 : in / 256 * 144;
        case 13: return in % 256 ? 0 : in / 256 * 176;
        case 14: return in % 256 ? 0 : in / 256 * 210;
        default: return 0;
    }
}

bool block_aligned(std::uint32_t type, std::uint64_t in) {
    switch (type) {
        case 2: case 3: case 6: case 7: case 8: return in % 32 == 0;
        case 10: case 11: case 12: case 13: case 14: return in % 256 == 0;
        default: return true;
    }
}

// The (input bits, result bits) pairs of a libm_expf.bin file ("PKEXPF01",
// a uint32 count, then the pairs); an empty path selects the file beside the
// loaded libpokit_hip.so.
std::vector<std::uint32_t> read_libm_expf(std::string path) {
    if (path.empty()) {
        Dl_info info{};
        if (!dladdr(reinterpret_cast<const void*>(&pk_hip_create), &info) || !info.dli_fname)
            throw std::runtime_error("HIP backend: cannot locate libpokit_hip.so");
        path = info.dli_fname;
        path = path.substr(0, path.find_last_of('/') + 1) + "libm_expf.bin";
    }
    std::ifstream in(path, std::ios::binary);
    char magic[8] = {};
    std::uint32_t count = 0;
    if (!in.read(magic, 8) || std::memcmp(magic, "PKEXPF01", 8) != 0 ||
        !in.read(reinterpret_cast<char*>(&count), 4))
        throw std::runtime_error("HIP backend: " + path + " is not an expf exception table");
    std::vector<std::uint32_t> pairs(2ull * count);
    if (!in.read(reinterpret_cast<char*>(pairs.data()),
                 static_cast<std::streamsize>(pairs.size() * 4)))
        throw std::runtime_error("HIP backend: " + path + " is truncated");
    return pairs;
}

struct WeightDeleter {
    void operator()(pk_hip_weight* w) const noexcept { pk_hip_weight_release(w); }
};
using WeightPtr = std::unique_ptr<pk_hip_weight, WeightDeleter>;

}  // namespace

class HipLinearBackend::Impl {
public:
    explicit Impl(const HipLinearOptions& options)
        : cache_file_tensors(options.cache_file_tensors),
          reference_order(options.reference_order),
          transient_budget(options.transient_cache_bytes) {
        pk_hip_options opts{};
        opts.struct_size = sizeof(opts);
        opts.time_kernels = options.time_kernels ? 1U : 0U;
        ErrorBuffer err;
        const auto st = pk_hip_create(options.device_index, &opts, &ctx, err.data(), kErrorCapacity);
        if (st == PK_HIP_STATUS_INVALID_ARGUMENT) throw std::invalid_argument(err.str());
        if (st != PK_HIP_STATUS_OK) throw std::runtime_error("HIP backend: " + err.str());
        if (reference_order) {
            try {
                const auto pairs = read_libm_expf(options.libm_expf_table);
                const auto ts = pk_hip_set_libm_expf(ctx, pairs.data(), pairs.size() / 2, err.data(),
                                                     kErrorCapacity);
                if (ts != PK_HIP_STATUS_OK) throw std::runtime_error("HIP backend: " + err.str());
            } catch (...) {
                pk_hip_destroy(ctx);
                ctx = nullptr;
                throw;
            }
        }
    }
    ~Impl() {
        resident.clear();  // weights before the context that owns them
        transient_index.clear();
        transient_lru.clear();
        if (ctx) pk_hip_destroy(ctx);
    }
    Impl(const Impl&) = delete;
    Impl& operator=(const Impl&) = delete;

    // Throws for a non-OK status: invalid_argument for argument errors,
    // runtime_error for everything else.  A device error leaves the C context
    // failed (every later call on it fails), and then this backend is failed
    // for good too; a data error such as non-finite router logits does not.
    void raise(pk_hip_status st, const ErrorBuffer& err) {
        if (st == PK_HIP_STATUS_INVALID_ARGUMENT) throw std::invalid_argument(err.str());
        ErrorBuffer probe;
        if (pk_hip_sync(ctx, nullptr, probe.data(), kErrorCapacity) != PK_HIP_STATUS_OK)
            failed = true;
        throw std::runtime_error("HIP backend: " + err.str());
    }

    void require_usable() const {
        if (failed) throw std::runtime_error("HIP backend failed during an earlier operation");
    }

    WeightPtr upload(const model::TensorReader& reader, std::uint64_t in, std::uint64_t out,
                     std::uint32_t experts) {
        return upload_bytes(reader.tensor().type, in, out, experts, reader.read_all());
    }

    // The resident copy of a file-backed matrix, uploading it on first use;
    // nullptr for an in-memory reader.  An entry belongs to the file it was
    // read from: it is dropped once that file is gone (another file opened at
    // the same address is a different key) or when the tensor at the offset
    // no longer has the entry's type and shape.
    pk_hip_weight* resident_matrix(const model::TensorReader& reader, std::uint64_t in,
                                   std::uint64_t out) {
        const auto& file = reader.model_file();
        if (!file || !cache_file_tensors) return nullptr;
        const auto type = reader.tensor().type;
        const Key key{file.get(), reader.tensor().file_offset};
        if (const auto it = resident.find(key); it != resident.end()) {
            const auto& e = it->second;
            if (e.file.lock() == file && e.type == type && e.in == in && e.out == out)
                return e.weight.get();
            resident.erase(it);
        }
        for (auto it = resident.begin(); it != resident.end();)  // files closed since
            it = it->second.file.expired() ? resident.erase(it) : std::next(it);
        auto w = upload(reader, in, out, 0);
        auto* raw = w.get();
        resident.emplace(key, ResidentEntry{file, type, in, out, std::move(w)});
        ++counters.resident_tensors;
        return raw;
    }

    // An in-memory matrix from the LRU set, uploading it on a miss; `bytes`
    // is the reader's payload.  Sets `transient` (and returns it) when the
    // set is disabled or the tensor is larger than the whole set.
    pk_hip_weight* cached_transient(const model::TensorReader& reader, std::uint64_t in,
                                    std::uint64_t out, std::vector<std::byte>&& bytes,
                                    WeightPtr& transient) {
        const auto& t = reader.tensor();
        if (transient_budget == 0 || bytes.size() > transient_budget) {
            transient = upload_bytes(t.type, in, out, 0, bytes);
            ++counters.transient_uploads;
            return transient.get();
        }
        TransientKey key{t.name, t.file_offset, t.type, in, out};
        if (const auto it = transient_index.find(key); it != transient_index.end()) {
            auto entry = it->second;
            if (entry->host == bytes) {
                transient_lru.splice(transient_lru.begin(), transient_lru, entry);
                ++counters.transient_hits;
                return entry->weight.get();
            }
            transient_held -= entry->host.size();
            transient_index.erase(it);
            transient_lru.erase(entry);
        }
        while (!transient_lru.empty() && transient_held + bytes.size() > transient_budget) {
            auto& last = transient_lru.back();
            transient_held -= last.host.size();
            transient_index.erase(last.key);
            transient_lru.pop_back();
        }
        auto w = upload_bytes(t.type, in, out, 0, bytes);
        ++counters.transient_uploads;
        transient_held += bytes.size();
        transient_lru.push_front(TransientEntry{key, std::move(bytes), std::move(w)});
        transient_index.emplace(std::move(key), transient_lru.begin());
        return transient_lru.front().weight.get();
    }

    WeightPtr upload_bytes(std::uint32_t type, std::uint64_t in, std::uint64_t out,
                           std::uint32_t experts, const std::vector<std::byte>& bytes) {
        pk_hip_weight* w = nullptr;
        ErrorBuffer err;
        const auto st = pk_hip_upload(ctx, type, in, out, experts, bytes.data(), bytes.size(), &w,
                                      err.data(), kErrorCapacity);
        if (st != PK_HIP_STATUS_OK) raise(st, err);
        return WeightPtr(w);
    }

    using Key = std::pair<const void*, std::uint64_t>;
    struct ResidentEntry {
        std::weak_ptr<storage::ModelFile> file;
        std::uint32_t type;
        std::uint64_t in, out;
        WeightPtr weight;
    };
    struct TransientKey {
        std::string name;
        std::uint64_t offset;
        std::uint32_t type;
        std::uint64_t in, out;
        bool operator<(const TransientKey& o) const {
            return std::tie(name, offset, type, in, out) <
                   std::tie(o.name, o.offset, o.type, o.in, o.out);
        }
    };
    struct TransientEntry {
        TransientKey key;
        std::vector<std::byte> host;
        WeightPtr weight;
    };

    pk_hip_ctx* ctx = nullptr;
    bool cache_file_tensors = true;
    bool reference_order = false;
    std::size_t transient_budget = 0;
    std::size_t transient_held = 0;
    bool failed = false;
    std::mutex mutex;
    std::map<Key, ResidentEntry> resident;
    std::list<TransientEntry> transient_lru;  // most recent first
    std::map<TransientKey, std::list<TransientEntry>::iterator> transient_index;
    std::uint64_t expert_bytes = 0;  // expert tensors of live MoE layers
    HipLinearStats counters{};  // fields the C ABI does not keep
};

class HipMoeLayer {
public:
    std::shared_ptr<HipLinearBackend::Impl> owner;
    WeightPtr router, gate, up, down;
    WeightPtr shared_router, shared_gate, shared_up, shared_down;  // Qwen3.5 only
    std::uint32_t hidden = 0, ffn = 0, experts = 0, top_k = 0;
    bool normalize = false;
    float scale = 1.0F;
    std::uint64_t expert_bytes = 0;  // gate + up + down payload bytes

    ~HipMoeLayer() {
        std::lock_guard lock(owner->mutex);
        owner->expert_bytes -= expert_bytes;
        for (WeightPtr* w : {&router, &gate, &up, &down, &shared_router, &shared_gate, &shared_up,
                             &shared_down})
            w->reset();
    }
};

HipLinearBackend::HipLinearBackend(const HipLinearOptions& options)
    : impl_(std::make_shared<Impl>(options)) {}

HipLinearBackend::~HipLinearBackend() = default;

bool HipLinearBackend::try_linear(const model::TensorReader& weights,
                                  std::span<const float> input, std::span<float> output) {
    const auto& tensor = weights.tensor();
    if (!pk_hip_type_supported(tensor.type)) {
        std::lock_guard lock(impl_->mutex);
        ++impl_->counters.unsupported_calls;
        return false;
    }
    if (input.empty() || output.empty() || tensor.dimensions.empty() ||
        tensor.dimensions.front() != input.size() || weights.row_count() != output.size()) {
        throw std::invalid_argument("HIP matrix dimensions do not match input/output");
    }
    if (!block_aligned(tensor.type, input.size()))
        throw std::invalid_argument("HIP quantized row is not block-aligned");
    if (weights.row_bytes() != encoded_row_bytes(tensor.type, input.size()))
        throw std::invalid_argument("HIP encoded row size mismatch");
    if (input.size() > std::numeric_limits<std::uint32_t>::max() ||
        output.size() > std::numeric_limits<std::uint32_t>::max()) {
        std::lock_guard lock(impl_->mutex);
        ++impl_->counters.unsupported_calls;
        return false;
    }
    std::lock_guard lock(impl_->mutex);
    impl_->require_usable();
    pk_hip_weight* w = impl_->resident_matrix(weights, input.size(), output.size());
    WeightPtr transient;
    if (!w)
        w = impl_->cached_transient(weights, input.size(), output.size(), weights.read_all(),
                                    transient);
    ErrorBuffer err;
    const auto st = impl_->reference_order
                        ? pk_hip_matvec_reference_order(impl_->ctx, w, UINT32_MAX, input.data(),
                                                        output.data(), err.data(), kErrorCapacity)
                        : pk_hip_matvec(impl_->ctx, w, UINT32_MAX, input.data(), 1, output.data(),
                                        err.data(), kErrorCapacity);
    if (st == PK_HIP_STATUS_UNSUPPORTED) {
        ++impl_->counters.unsupported_calls;
        return false;
    }
    if (st != PK_HIP_STATUS_OK) impl_->raise(st, err);
    ++impl_->counters.linear_calls;
    return true;
}

std::shared_ptr<HipMoeLayer> HipLinearBackend::upload_moe_layer(
    const model::TensorReader& router, const model::TensorReader& gate_exps,
    const model::TensorReader& up_exps, const model::TensorReader& down_exps,
    std::size_t experts_per_token, bool expert_weights_norm, float expert_weights_scale) {
    const auto& rd = router.tensor().dimensions;
    const auto& gd = gate_exps.tensor().dimensions;
    const auto& ud = up_exps.tensor().dimensions;
    const auto& dd = down_exps.tensor().dimensions;
    if (rd.size() != 2 || gd.size() != 3 || ud.size() != 3 || dd.size() != 3)
        throw std::invalid_argument("HIP MoE layer: router must be 2-D and experts 3-D");
    const std::uint64_t hidden = rd[0], experts = rd[1], ffn = gd[1];
    if (gd != ud || gd[0] != hidden || gd[2] != experts || dd[0] != ffn || dd[1] != hidden ||
        dd[2] != experts)
        throw std::invalid_argument("HIP MoE layer: expert tensor dimensions disagree");
    if (experts_per_token == 0 || experts_per_token > experts)
        throw std::invalid_argument("HIP MoE layer: experts_per_token out of range");
    if (hidden > UINT32_MAX || ffn > UINT32_MAX || experts > UINT32_MAX)
        throw std::invalid_argument("HIP MoE layer: dimensions exceed 32 bits");
    // The layer exists before the lock is taken, so if an upload throws it is
    // destroyed (and takes the lock itself) only after the lock is released.
    auto layer = std::make_shared<HipMoeLayer>();
    layer->owner = impl_;
    std::lock_guard lock(impl_->mutex);
    impl_->require_usable();
    const auto n = static_cast<std::uint32_t>(experts);
    layer->router = impl_->upload(router, hidden, experts, 0);
    layer->gate = impl_->upload(gate_exps, hidden, ffn, n);
    layer->up = impl_->upload(up_exps, hidden, ffn, n);
    layer->down = impl_->upload(down_exps, ffn, hidden, n);
    layer->expert_bytes = gate_exps.tensor().payload_size.value_or(0) +
                          up_exps.tensor().payload_size.value_or(0) +
                          down_exps.tensor().payload_size.value_or(0);
    impl_->expert_bytes += layer->expert_bytes;
    layer->hidden = static_cast<std::uint32_t>(hidden);
    layer->ffn = static_cast<std::uint32_t>(ffn);
    layer->experts = static_cast<std::uint32_t>(experts);
    layer->top_k = static_cast<std::uint32_t>(experts_per_token);
    layer->normalize = expert_weights_norm;
    layer->scale = expert_weights_scale;
    return layer;
}

void HipLinearBackend::attach_shared_expert(HipMoeLayer& layer,
                                            const model::TensorReader& shared_router,
                                            const model::TensorReader& shared_gate,
                                            const model::TensorReader& shared_up,
                                            const model::TensorReader& shared_down) {
    if (layer.owner != impl_)
        throw std::invalid_argument("HIP MoE layer belongs to another backend");
    const auto& rd = shared_router.tensor().dimensions;
    const auto& gd = shared_gate.tensor().dimensions;
    const auto& ud = shared_up.tensor().dimensions;
    const auto& dd = shared_down.tensor().dimensions;
    const bool router_ok = (rd.size() == 1 && rd[0] == layer.hidden) ||
                           (rd.size() == 2 && rd[0] == layer.hidden && rd[1] == 1);
    if (!router_ok || gd.size() != 2 || ud != gd || dd.size() != 2 || gd[0] != layer.hidden ||
        dd[0] != gd[1] || dd[1] != layer.hidden || gd[1] > UINT32_MAX)
        throw std::invalid_argument("HIP MoE layer: shared expert dimensions disagree");
    const std::uint64_t ffn = gd[1];
    WeightPtr r, g, u, d;
    {
        std::lock_guard lock(impl_->mutex);
        impl_->require_usable();
        r = impl_->upload(shared_router, layer.hidden, 1, 0);
        g = impl_->upload(shared_gate, layer.hidden, ffn, 0);
        u = impl_->upload(shared_up, layer.hidden, ffn, 0);
        d = impl_->upload(shared_down, ffn, layer.hidden, 0);
        layer.shared_router = std::move(r);
        layer.shared_gate = std::move(g);
        layer.shared_up = std::move(u);
        layer.shared_down = std::move(d);
    }
}

bool HipLinearBackend::try_moe_block(const HipMoeLayer& layer, std::span<const float> normalized,
                                     std::span<float> moe_result,
                                     std::span<std::uint32_t> route_ids,
                                     std::span<float> route_probabilities) {
    if (layer.owner != impl_)
        throw std::invalid_argument("HIP MoE layer belongs to another backend");
    if (normalized.size() != layer.hidden || moe_result.size() != layer.hidden)
        throw std::invalid_argument("HIP MoE block: hidden size mismatch");
    if ((!route_ids.empty() && route_ids.size() != layer.top_k) ||
        (!route_probabilities.empty() && route_probabilities.size() != layer.top_k))
        throw std::invalid_argument("HIP MoE block: route outputs must hold experts_per_token");
    std::vector<std::uint32_t> ids(layer.top_k);
    std::vector<float> probs(layer.top_k);
    pk_hip_moe_layer desc{};
    desc.router = layer.router.get();
    desc.gate = layer.gate.get();
    desc.up = layer.up.get();
    desc.down = layer.down.get();
    desc.top_k = layer.top_k;
    desc.normalize = layer.normalize ? 1U : 0U;
    desc.scale = layer.scale;
    std::lock_guard lock(impl_->mutex);
    impl_->require_usable();
    ErrorBuffer err;
    pk_hip_status st;
    if (impl_->reference_order) {
        if (layer.shared_router) return false;  // the CPU block runs
        st = pk_hip_moe_decode_reference_order(impl_->ctx, &desc, normalized.data(),
                                               moe_result.data(), ids.data(), probs.data(),
                                               err.data(), kErrorCapacity);
    } else if (layer.shared_router) {  // Qwen3.5: select_experts weights and the shared expert
        pk_hip_moe35_layer desc35{};
        desc35.routed = desc;
        desc35.shared_router = layer.shared_router.get();
        desc35.shared_gate = layer.shared_gate.get();
        desc35.shared_up = layer.shared_up.get();
        desc35.shared_down = layer.shared_down.get();
        st = pk_hip_moe35_decode(impl_->ctx, &desc35, normalized.data(), moe_result.data(),
                                 ids.data(), probs.data(), err.data(), kErrorCapacity);
    } else {
        st = pk_hip_moe_decode(impl_->ctx, &desc, normalized.data(), moe_result.data(), ids.data(),
                               probs.data(), err.data(), kErrorCapacity);
    }
    if (st == PK_HIP_STATUS_UNSUPPORTED) return false;
    if (st != PK_HIP_STATUS_OK) impl_->raise(st, err);
    if (!route_ids.empty()) std::copy(ids.begin(), ids.end(), route_ids.begin());
    if (!route_probabilities.empty())
        std::copy(probs.begin(), probs.end(), route_probabilities.begin());
    ++impl_->counters.moe_calls;
    return true;
}

HipLinearStats HipLinearBackend::stats() const {
    std::lock_guard lock(impl_->mutex);
    HipLinearStats out = impl_->counters;
    pk_hip_stats s{};
    if (pk_hip_get_stats(impl_->ctx, &s) == PK_HIP_STATUS_OK) {
        out.dispatches = s.dispatches;
        out.q4_0_dispatches = s.q4_0_dispatches;
        out.q8_0_dispatches = s.q8_0_dispatches;
        out.q4_k_dispatches = s.q4_k_dispatches;
        out.q5_k_dispatches = s.q5_k_dispatches;
        out.q6_k_dispatches = s.q6_k_dispatches;
        out.other_dispatches = s.float_dispatches + s.q4_1_dispatches + s.q5_0_dispatches +
                               s.q5_1_dispatches + s.q2_k_dispatches + s.q3_k_dispatches;
        out.weight_bytes = s.weight_bytes;
        out.gpu_time_ns = s.matvec_ns + s.router_ns + s.gate_up_ns + s.down_ns;
        out.resident_bytes = s.resident_bytes;
        out.uploaded_bytes = s.uploaded_bytes;
        out.router_fallbacks = s.router_fallbacks;
        out.expert_hits = s.expert_hits;
        out.expert_misses = s.expert_misses;
    }
    out.transient_bytes = impl_->transient_held;
    out.expert_resident_bytes = impl_->expert_bytes;
    return out;
}

HipExpertCacheStats HipLinearBackend::expert_cache_stats() const {
    std::lock_guard lock(impl_->mutex);
    HipExpertCacheStats out;
    out.capacity_bytes = static_cast<std::size_t>(impl_->expert_bytes);
    out.resident_bytes = static_cast<std::size_t>(impl_->expert_bytes);
    pk_hip_stats s{};
    if (pk_hip_get_stats(impl_->ctx, &s) == PK_HIP_STATUS_OK) {
        out.hits = s.expert_hits;
        out.misses = s.expert_misses;
    }
    return out;
}

std::string HipLinearBackend::device_name() const {
    std::array<char, 256> text{};
    std::lock_guard lock(impl_->mutex);
    (void)pk_hip_device_name(impl_->ctx, text.data(), text.size());
    return std::string(text.data());
}

}  // namespace pokitlms::gpu
