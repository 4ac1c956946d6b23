// api.hip -- the extern "C" boundary of libpokit_hip.so (include/pokit_hip.h).
//
// Error model of the reference backends: invalid shapes -> INVALID_ARGUMENT,
// uncovered types/widths -> UNSUPPORTED (the caller's CPU fallback, like
// try_linear returning false), device failures -> RUNTIME_ERROR and a sticky
// failed state (src/vulkan_linear.cpp:636, 731-735 of the reference).  No C++
// exception crosses the ABI (src/c_api.cpp:87-101).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <chrono>
#include <cmath>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/pokit_hip.h"
#include "launch.hpp"
#include "layout.hpp"

namespace {

struct ArgError : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct Unsupported : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct DeviceError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void set_error(char* dst, size_t cap, const char* msg) noexcept {
    if (!dst || cap == 0) return;
    const size_t n = std::min(cap - 1, std::strlen(msg));
    std::memcpy(dst, msg, n);
    dst[n] = '\0';
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw DeviceError(std::string(what) + ": " + hipGetErrorString(e));
}

uint32_t block_elements(uint32_t t) {
    switch (t) {
        case 0: case 1: case 30: return 1;
        case 2: case 3: case 6: case 7: case 8: return 32;
        case 10: case 11: case 12: case 13: case 14: return 256;
        default: return 0;
    }
}

uint32_t block_bytes(uint32_t t) {
    switch (t) {
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
        default: return 0;
    }
}

// Set while an entry point enqueues onto a stream that is being captured:
// scratch may not grow then (an allocation would not be part of the graph).
thread_local bool t_capturing = false;

// Context scratch.  Growing it retires the old allocation instead of freeing
// it: a graph captured from an earlier call keeps its pointers, and they stay
// valid until the context is destroyed.  Growth is refused during capture.
template <typename T>
struct DeviceBuffer {
    T* ptr = nullptr;
    size_t count = 0;
    std::vector<T*> retired;
    void ensure(size_t n) {
        if (n <= count) return;
        if (t_capturing)
            throw ArgError("scratch for this shape must be sized by a call outside stream "
                           "capture first");
        T* fresh = nullptr;
        check(hipMalloc(&fresh, n * sizeof(T)), "hipMalloc scratch");
        if (ptr) retired.push_back(ptr);
        ptr = fresh;
        count = n;
    }
    void release() noexcept {
        if (ptr) (void)hipFree(ptr);
        for (T* p : retired) (void)hipFree(p);
        retired.clear();
        ptr = nullptr;
        count = 0;
    }
};

// Marks the calling thread as enqueueing onto `s` for the guard's lifetime,
// recording whether `s` is being captured.
struct CaptureScope {
    explicit CaptureScope(hipStream_t s) {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        t_capturing = hipStreamIsCapturing(s, &st) == hipSuccess &&
                      st == hipStreamCaptureStatusActive;
    }
    ~CaptureScope() { t_capturing = false; }
    CaptureScope(const CaptureScope&) = delete;
    CaptureScope& operator=(const CaptureScope&) = delete;
};

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of pk_hip_moe_decode_noalloc: one static device array per GPU (each
// device holds its own copy until the process ends).  Its host-side name is
// only a stand-in for the symbol; the device address comes from
// hipGetSymbolAddress, resolved once per device with that device current.
// Layout: status words | row sums | row bounds | activations.
namespace noalloc {
constexpr uint32_t kMaxExperts = 256;
constexpr uint32_t kMaxTopK = 8;
constexpr uint32_t kMaxFfn = 2048;
constexpr size_t kStatusBytes = 256;
constexpr size_t kSumBytes = kMaxExperts * sizeof(double);
constexpr size_t kActBytes = static_cast<size_t>(kMaxTopK) * kMaxFfn * sizeof(float);
constexpr size_t kBytes = kStatusBytes + 2 * kSumBytes + kActBytes;  // 69,888 bytes
constexpr int kMaxDevices = 64;
}  // namespace noalloc

static __device__ __align__(256) uint8_t scratch[noalloc::kBytes];

namespace {
std::mutex g_scratch_mutex;
uint8_t* g_scratch_ptr[noalloc::kMaxDevices] = {};

// The calling thread's current device must be `device`.
uint8_t* resolve_scratch(int device) {
    if (device < 0 || device >= noalloc::kMaxDevices) return nullptr;
    std::lock_guard lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void* ptr = nullptr;
        check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[device] = static_cast<uint8_t*>(ptr);
    }
    return g_scratch_ptr[device];
}
}  // namespace

struct pk_hip_ctx {
    int device = 0;
    uint8_t* noalloc_scratch = nullptr;  // this device's static scratch array
    hipStream_t stream = nullptr;
    bool failed = false;
    bool time_kernels = false;
    mutable std::mutex mutex;
    pk_hip_stats stats{};
    uint64_t live_weights = 0;
    // scratch
    DeviceBuffer<float> x, y, act, probs;
    DeviceBuffer<uint32_t> ids, words;  // words: [1..4] status
    DeviceBuffer<double> row_sum, row_bound;
    DeviceBuffer<float> mvpart;  // the K-sliced batched matvec's slice sums
    // prefill scratch (grown on demand)
    DeviceBuffer<float> px, py, pprobs, pout, pxsum, pasum;
    DeviceBuffer<uint32_t> pids, poffsets, ptiles, pperm;
    DeviceBuffer<uint16_t> pxparts, paparts;
    DeviceBuffer<double> prow_sum, prow_bound;
    // reference-order MoE block: its scratch and the host libm's expf
    // exceptions (pk_hip_set_libm_expf)
    DeviceBuffer<float> ref_scratch;
    DeviceBuffer<uint32_t> expf_slots;
    pk::LibmExpf expf{nullptr, 0, 0, 0};
    hipEvent_t ev[10] = {};
    int wall_rate_khz = 100000;  // wall_clock64() rate

    void set_device() const { check(hipSetDevice(device), "hipSetDevice"); }
};

struct pk_hip_weight {
    pk_hip_ctx* ctx = nullptr;
    uint32_t type = 0;
    uint64_t in = 0, out = 0;
    uint32_t n_experts = 0;
    uint64_t row_bytes = 0, slice_bytes = 0, nbytes = 0;
    // Device bytes between consecutive expert slices: slice_bytes, rounded up
    // to pk::kSlicePitchAlign for the planar types (see layout.hpp).
    uint64_t slice_pitch = 0;
    uint8_t* dptr = nullptr;
};

namespace {

constexpr uint32_t kStatusError = 1;

uint32_t* status_words(pk_hip_ctx* c) { return c->words.ptr + 1; }

template <typename F>
pk_hip_status guarded(pk_hip_ctx* ctx, char* err, size_t cap, F&& body) {
    try {
        body();
        set_error(err, cap, "");
        return PK_HIP_STATUS_OK;
    } catch (const Unsupported& e) {
        set_error(err, cap, e.what());
        return PK_HIP_STATUS_UNSUPPORTED;
    } catch (const ArgError& e) {
        set_error(err, cap, e.what());
        return PK_HIP_STATUS_INVALID_ARGUMENT;
    } catch (const DeviceError& e) {
        if (ctx) ctx->failed = true;
        set_error(err, cap, e.what());
        return PK_HIP_STATUS_RUNTIME_ERROR;
    } catch (const std::bad_alloc&) {
        set_error(err, cap, "out of host memory");
        return PK_HIP_STATUS_RUNTIME_ERROR;
    } catch (const std::exception& e) {
        set_error(err, cap, e.what());
        return PK_HIP_STATUS_RUNTIME_ERROR;
    } catch (...) {
        set_error(err, cap, "unknown HIP backend failure");
        return PK_HIP_STATUS_INTERNAL_ERROR;
    }
}

void require_usable(const pk_hip_ctx* ctx) {
    if (!ctx) throw ArgError("HIP backend context is required");
    if (ctx->failed) throw DeviceError("HIP backend failed during an earlier operation");
}

void count_dispatch(pk_hip_ctx* c, uint32_t type) {
    ++c->stats.dispatches;
    switch (type) {
        case 2: ++c->stats.q4_0_dispatches; break;
        case 3: ++c->stats.q4_1_dispatches; break;
        case 6: ++c->stats.q5_0_dispatches; break;
        case 7: ++c->stats.q5_1_dispatches; break;
        case 8: ++c->stats.q8_0_dispatches; break;
        case 10: ++c->stats.q2_k_dispatches; break;
        case 11: ++c->stats.q3_k_dispatches; break;
        case 12: ++c->stats.q4_k_dispatches; break;
        case 13: ++c->stats.q5_k_dispatches; break;
        case 14: ++c->stats.q6_k_dispatches; break;
        default: ++c->stats.float_dispatches; break;
    }
}

pk_hip_weight* make_weight(pk_hip_ctx* ctx, uint32_t type, uint64_t in, uint64_t out,
                           uint32_t n_experts, uint64_t nbytes) {
    require_usable(ctx);
    const uint32_t be = block_elements(type), bb = block_bytes(type);
    if (be == 0) throw Unsupported("GGUF type has no HIP kernel");
    if (in == 0 || out == 0) throw ArgError("GGUF matrix dimensions must be non-zero");
    if (in % be) throw ArgError("GGUF row is not a whole number of blocks");
    if (in > 0xffffffffull || out > 0xffffffffull) throw Unsupported("matrix too large");
    const uint64_t row = in / be * bb;
    const uint64_t slice = row * out;
    const uint64_t experts = n_experts ? n_experts : 1;
    if (slice > UINT64_MAX / experts || slice * experts != nbytes)
        throw ArgError("GGUF payload size does not match its dimensions");
    auto w = new pk_hip_weight;
    w->ctx = ctx;
    w->type = type;
    w->in = in;
    w->out = out;
    w->n_experts = n_experts;
    w->row_bytes = row;
    w->slice_bytes = slice;
    w->nbytes = nbytes;
    w->slice_pitch = slice;
    if (pk::planar_type(type) && n_experts > 1)
        w->slice_pitch = (slice + pk::kSlicePitchAlign - 1) / pk::kSlicePitchAlign * pk::kSlicePitchAlign;
    const uint64_t device_bytes = w->slice_pitch * experts;
    ctx->set_device();
    const hipError_t e = hipMalloc(&w->dptr, device_bytes + pk::kWeightTailPad);
    if (e != hipSuccess) {
        delete w;
        throw DeviceError(std::string("hipMalloc weights: ") + hipGetErrorString(e));
    }
    check(hipMemsetAsync(w->dptr + device_bytes, 0, pk::kWeightTailPad, ctx->stream), "pad weights");
    return w;
}

uint32_t slices_of(const pk_hip_weight* w) { return w->n_experts ? w->n_experts : 1u; }
uint64_t slice_blocks(const pk_hip_weight* w) {
    return w->slice_bytes / block_bytes(w->type);
}

// Fills w from GGUF-form bytes at src (device memory, slices slice_bytes
// apart), moving planar types into their planes.  Enqueued on the context
// stream.
void fill_from_device(pk_hip_ctx* c, pk_hip_weight* w, const uint8_t* src) {
    if (!pk::planar_type(w->type)) {
        check(hipMemcpyAsync(w->dptr, src, w->nbytes, hipMemcpyDeviceToDevice, c->stream),
              "weight copy");
        return;
    }
    check(pk::launch_to_planar(w->type, src, w->slice_bytes, w->dptr, w->slice_pitch,
                               slice_blocks(w), slices_of(w), c->stream),
          "planar weight layout");
}

// Staging bound for host uploads of planar types (whole slices per chunk).
constexpr uint64_t kStageBytes = 256ull << 20;

// As fill_from_device from host (or device, `kind`) bytes; synchronises.
void fill_weight(pk_hip_ctx* c, pk_hip_weight* w, const void* src, hipMemcpyKind kind) {
    if (!pk::planar_type(w->type)) {
        check(hipMemcpyAsync(w->dptr, src, w->nbytes, kind, c->stream), "weight upload");
        check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        return;
    }
    if (kind == hipMemcpyDeviceToDevice) {
        fill_from_device(c, w, static_cast<const uint8_t*>(src));
        check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        return;
    }
    const uint32_t n = slices_of(w);
    const uint32_t per = static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>(n, kStageBytes / w->slice_bytes)));
    DeviceBuffer<uint8_t> stage;
    stage.ensure(static_cast<size_t>(per) * w->slice_bytes);
    try {
        for (uint32_t s0 = 0; s0 < n; s0 += per) {
            const uint32_t k = std::min(per, n - s0);
            const uint8_t* hs = static_cast<const uint8_t*>(src) + static_cast<uint64_t>(s0) * w->slice_bytes;
            check(hipMemcpyAsync(stage.ptr, hs, static_cast<uint64_t>(k) * w->slice_bytes, kind, c->stream),
                  "weight upload");
            check(pk::launch_to_planar(w->type, stage.ptr, w->slice_bytes,
                                       w->dptr + static_cast<uint64_t>(s0) * w->slice_pitch,
                                       w->slice_pitch, slice_blocks(w), k, c->stream),
                  "planar weight layout");
            check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        }
    } catch (...) {
        (void)hipStreamSynchronize(c->stream);
        stage.release();
        throw;
    }
    stage.release();
}

// Holds the stream for `ticks` of the constant-rate wall clock so that the
// launches and events of one timed call are all queued before the GPU reaches
// them; event intervals then cover dispatch + execution, not host latency.
// The wait is bounded by the clock alone.
__global__ void k_hold(uint64_t ticks) {
    const uint64_t t0 = wall_clock64();
    while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(16);
}

constexpr uint64_t kHoldMicroseconds = 100;

void hold_stream(pk_hip_ctx* c, hipStream_t s) {
    const uint64_t ticks = kHoldMicroseconds * static_cast<uint64_t>(c->wall_rate_khz) / 1000u;
    hipLaunchKernelGGL(k_hold, dim3(1), dim3(64), 0, s, ticks);
    check(hipGetLastError(), "hold launch");
}

void begin_timing(pk_hip_ctx* c, hipStream_t s, int slot) {
    if (c->time_kernels) check(hipEventRecord(c->ev[slot], s), "hipEventRecord");
}

uint64_t elapsed_ns(pk_hip_ctx* c, int a, int b) {
    float ms = 0.0f;
    check(hipEventElapsedTime(&ms, c->ev[a], c->ev[b]), "hipEventElapsedTime");
    return static_cast<uint64_t>(static_cast<double>(ms) * 1.0e6);
}

void launch_checked(hipError_t e, const char* what) {
    if (e == hipErrorInvalidValue) throw Unsupported(std::string(what) + ": shape not covered");
    check(e, what);
}

void enqueue_matvec(pk_hip_ctx* c, const pk_hip_weight* w, uint32_t expert, const float* dx,
                    uint32_t batch, float* dy, hipStream_t s) {
    if (!w || w->ctx != c) throw ArgError("weight handle does not belong to this context");
    if (batch == 0 || batch > 8) throw ArgError("batch must be between 1 and 8");
    if (!dx || !dy) throw ArgError("input and output buffers are required");
    uint64_t offset = 0;
    if (expert != UINT32_MAX) {
        if (w->n_experts == 0 || expert >= w->n_experts)
            throw ArgError("expert index out of range");
        offset = static_cast<uint64_t>(expert) * w->slice_pitch;
    }
    if (!pk::matvec_supported(w->type, static_cast<uint32_t>(w->in), batch))
        throw Unsupported("matrix width/batch not covered by the HIP matvec kernels");
    const size_t part = pk::matvec_partial_floats(w->type, static_cast<uint32_t>(w->in), batch,
                                                  static_cast<uint32_t>(w->out));
    if (part) c->mvpart.ensure(part);
    if (c->time_kernels) hold_stream(c, s);
    begin_timing(c, s, 0);
    launch_checked(pk::launch_matvec(w->type, w->dptr + offset, w->row_bytes,
                                     static_cast<uint32_t>(w->out), static_cast<uint32_t>(w->in),
                                     dx, dy, batch, s, part ? c->mvpart.ptr : nullptr),
                   "matvec launch");
    begin_timing(c, s, 1);
    ++c->stats.matvec_calls;
    ++c->stats.matvec_launches;
    count_dispatch(c, w->type);
    c->stats.weight_bytes += w->slice_bytes;
}

struct MoeShape {
    uint32_t hidden, ffn, experts;
};

MoeShape check_layer(pk_hip_ctx* c, const pk_hip_moe_layer* L) {
    if (!L || !L->router || !L->gate || !L->up || !L->down)
        throw ArgError("MoE layer needs router, gate, up and down weights");
    for (const pk_hip_weight* w : {L->router, L->gate, L->up, L->down})
        if (w->ctx != c) throw ArgError("weight handle does not belong to this context");
    if (L->router->type != 0 || L->router->n_experts != 0)
        throw Unsupported("router must be a plain F32 matrix");
    MoeShape m{static_cast<uint32_t>(L->router->in), static_cast<uint32_t>(L->gate->out),
               static_cast<uint32_t>(L->router->out)};
    if (L->gate->n_experts != m.experts || L->up->n_experts != m.experts ||
        L->down->n_experts != m.experts)
        throw ArgError("expert tensors must have one slice per router output");
    if (L->gate->in != m.hidden || L->up->in != m.hidden || L->up->out != m.ffn ||
        L->down->in != m.ffn || L->down->out != m.hidden)
        throw ArgError("MoE tensor dimensions do not match");
    if (L->top_k == 0 || L->top_k > m.experts) throw ArgError("invalid expert top-k");
    if (!(L->scale > 0.0f) || !(L->scale < 1.0e30f)) throw ArgError("invalid route scale");
    return m;
}

MoeShape check_decode_layer(pk_hip_ctx* c, const pk_hip_moe_layer* L) {
    const MoeShape m = check_layer(c, L);
    if (!pk::moe_decode_supported(L->gate->type, L->up->type, L->down->type, m.hidden, m.ffn,
                                  m.experts, L->top_k))
        throw Unsupported("MoE shape not covered by the HIP kernels");
    return m;
}

// The Qwen3.5 layer's shared expert, checked against the routed experts.
MoeShape check_decode35(pk_hip_ctx* c, const pk_hip_moe35_layer* L) {
    if (!L) throw ArgError("MoE layer is required");
    const MoeShape m = check_layer(c, &L->routed);
    const pk_hip_weight* sw[4] = {L->shared_router, L->shared_gate, L->shared_up, L->shared_down};
    for (const pk_hip_weight* w : sw) {
        if (!w) throw ArgError("Qwen3.5 layer needs the shared expert's router, gate, up and down");
        if (w->ctx != c) throw ArgError("weight handle does not belong to this context");
        if (w->n_experts != 0) throw ArgError("shared expert tensors are plain matrices");
    }
    const pk_hip_weight *r = L->shared_router, *g = L->shared_gate, *u = L->shared_up,
                        *d = L->shared_down;
    if (r->in != m.hidden || r->out != 1) throw ArgError("shared expert router must be [hidden]");
    if (g->in != m.hidden || u->in != m.hidden || u->out != g->out || d->in != g->out ||
        d->out != m.hidden)
        throw ArgError("shared expert dimensions do not match");
    if (r->type != 0) throw Unsupported("shared expert router must be F32");
    if (g->out != m.ffn || g->type != L->routed.gate->type || u->type != L->routed.up->type ||
        d->type != L->routed.down->type)
        throw Unsupported("shared expert must have the routed experts' types and width");
    if (!pk::moe_decode_supported(L->routed.gate->type, L->routed.up->type,
                                  L->routed.down->type, m.hidden, m.ffn, m.experts,
                                  L->routed.top_k, 1))
        throw Unsupported("MoE shape not covered by the HIP kernels");
    return m;
}

void ensure_moe_scratch(pk_hip_ctx* c, const MoeShape& m, uint32_t top_k) {
    // one more route and router row for a shared expert
    c->act.ensure(static_cast<size_t>(top_k + 1) * m.ffn);
    c->row_sum.ensure(m.experts + 1);
    c->row_bound.ensure(m.experts + 1);
    c->ids.ensure(16);
    c->probs.ensure(16);
}

// Device scratch of one decode call: router sums and bounds, activations and
// status words.
struct MoeScratch {
    double* row_sum;
    double* row_bound;
    float* act;
    uint32_t* status;
};

MoeScratch context_scratch(pk_hip_ctx* c, const MoeShape& m, uint32_t top_k) {
    ensure_moe_scratch(c, m, top_k);
    return MoeScratch{c->row_sum.ptr, c->row_bound.ptr, c->act.ptr, status_words(c)};
}

void enqueue_moe(pk_hip_ctx* c, const pk_hip_moe_layer* L, const MoeShape& m, const float* dx,
                 float* dy, uint32_t* dids, float* dprobs, hipStream_t s,
                 const pk_hip_moe35_layer* shared = nullptr, const MoeScratch* scratch = nullptr,
                 uint64_t* trace = nullptr) {
    const MoeScratch sc = scratch ? *scratch : context_scratch(c, m, L->top_k);
    pk::MoeDecodeArgs a{};
    a.trace = trace;
    if (shared) {
        a.variant = 1;
        a.shared_router = reinterpret_cast<const float*>(shared->shared_router->dptr);
        a.shared_gate = shared->shared_gate->dptr;
        a.shared_up = shared->shared_up->dptr;
        a.shared_down = shared->shared_down->dptr;
        c->stats.weight_bytes += shared->shared_router->nbytes + shared->shared_gate->nbytes +
                                 shared->shared_up->nbytes + shared->shared_down->nbytes;
    }
    a.router = reinterpret_cast<const float*>(L->router->dptr);
    a.gate = L->gate->dptr;
    a.up = L->up->dptr;
    a.down = L->down->dptr;
    a.gate_type = L->gate->type;
    a.up_type = L->up->type;
    a.down_type = L->down->type;
    a.gate_slice = L->gate->slice_pitch;
    a.up_slice = L->up->slice_pitch;
    a.down_slice = L->down->slice_pitch;
    a.gate_row = L->gate->row_bytes;
    a.up_row = L->up->row_bytes;
    a.down_row = L->down->row_bytes;
    a.hidden = m.hidden;
    a.ffn = m.ffn;
    a.n_experts = m.experts;
    a.top_k = L->top_k;
    a.normalize = L->normalize ? 1u : 0u;
    a.scale = L->scale;
    a.x = dx;
    a.y = dy;
    a.ids = dids;
    a.probs = dprobs;
    a.row_sum = sc.row_sum;
    a.row_bound = sc.row_bound;
    a.act = sc.act;
    a.status = sc.status;
    if (c->time_kernels) hold_stream(c, s);
    begin_timing(c, s, 2);
    launch_checked(pk::launch_moe_router(a, s), "router launch");
    begin_timing(c, s, 3);
    launch_checked(pk::launch_moe_gate_up(a, s), "gate/up launch");
    begin_timing(c, s, 4);
    launch_checked(pk::launch_moe_down(a, s), "down launch");
    begin_timing(c, s, 5);
    ++c->stats.router_launches;
    ++c->stats.gate_up_launches;
    ++c->stats.down_launches;
    c->stats.dispatches += 3;
    ++c->stats.moe_decode_calls;
    count_dispatch(c, L->gate->type);
    count_dispatch(c, L->down->type);
    c->stats.dispatches -= 2;  // the two per-format counts above are the same launches
    c->stats.weight_bytes += L->router->nbytes +
                             static_cast<uint64_t>(L->top_k) *
                                 (L->gate->slice_bytes + L->up->slice_bytes + L->down->slice_bytes);
    c->stats.expert_hits += L->top_k;
}

void collect_timing_matvec(pk_hip_ctx* c) {
    if (c->time_kernels) c->stats.matvec_ns += elapsed_ns(c, 0, 1);
}

void collect_timing_moe(pk_hip_ctx* c) {
    if (!c->time_kernels) return;
    c->stats.router_ns += elapsed_ns(c, 2, 3);
    c->stats.gate_up_ns += elapsed_ns(c, 3, 4);
    c->stats.down_ns += elapsed_ns(c, 4, 5);
}

void sync_and_check(pk_hip_ctx* c, hipStream_t s) {
    uint32_t err_word = 0;
    check(hipMemcpyAsync(&err_word, status_words(c) + (kStatusError - 1), sizeof(err_word),
                         hipMemcpyDeviceToHost, s),
          "read router status");
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (err_word) {
        check(hipMemsetAsync(status_words(c) + (kStatusError - 1), 0, sizeof(uint32_t), s),
              "clear router status");
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        throw std::runtime_error("expert router produced non-finite logits");
    }
}

}  // namespace

extern "C" {

const char* pk_hip_version(void) { return "0.1.0"; }

int pk_hip_type_supported(uint32_t t) {
    switch (t) {
        case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 10: case 11: case 12:
        case 13: case 14: case 30: return 1;
        default: return 0;
    }
}

pk_hip_status pk_hip_create(int device, const pk_hip_options* options, pk_hip_ctx** out_ctx,
                            char* err, size_t cap) {
    if (out_ctx) *out_ctx = nullptr;
    pk_hip_ctx* c = nullptr;
    const pk_hip_status st = guarded(nullptr, err, cap, [&] {
        if (!out_ctx) throw ArgError("output handle is required");
        if (options && options->struct_size != sizeof(pk_hip_options))
            throw ArgError("pk_hip_options.struct_size mismatch");
        int count = 0;
        check(hipGetDeviceCount(&count), "hipGetDeviceCount");
        const int dev = device < 0 ? 0 : device;
        if (dev >= count) throw ArgError("HIP device index out of range");
        c = new pk_hip_ctx;
        c->device = dev;
        c->time_kernels = options && options->time_kernels;
        c->set_device();
        int rate = 0;
        if (hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, dev) == hipSuccess &&
            rate > 0)
            c->wall_rate_khz = rate;
        check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
        // timing-only events: no system-scope fence (cache writeback) on record
        for (auto& e : c->ev)
            check(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreate");
        c->noalloc_scratch = resolve_scratch(dev);
        c->words.ensure(8);
        check(hipMemsetAsync(c->words.ptr, 0, 8 * sizeof(uint32_t), c->stream), "init status");
        check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        *out_ctx = c;
    });
    if (st != PK_HIP_STATUS_OK && c) pk_hip_destroy(c);
    return st;
}

void pk_hip_destroy(pk_hip_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    c->x.release();
    c->y.release();
    c->act.release();
    c->probs.release();
    c->ids.release();
    c->words.release();
    c->row_sum.release();
    c->row_bound.release();
    c->mvpart.release();
    for (auto* b : {&c->px, &c->py, &c->pprobs, &c->pout, &c->pxsum, &c->pasum})
        b->release();
    for (auto* b : {&c->pids, &c->poffsets, &c->ptiles, &c->pperm}) b->release();
    c->pxparts.release();
    c->paparts.release();
    c->prow_sum.release();
    c->prow_bound.release();
    c->ref_scratch.release();
    c->expf_slots.release();
    for (auto& e : c->ev)
        if (e) (void)hipEventDestroy(e);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

static pk_hip_status upload_impl(pk_hip_ctx* ctx, uint32_t type, uint64_t in, uint64_t out,
                                 uint32_t n_experts, const void* src, uint64_t nbytes,
                                 hipMemcpyKind kind, pk_hip_weight** out_w, char* err,
                                 size_t cap) {
    if (out_w) *out_w = nullptr;
    return guarded(ctx, err, cap, [&] {
        if (!out_w || !src) throw ArgError("source bytes and output handle are required");
        require_usable(ctx);
        std::lock_guard lock(ctx->mutex);
        pk_hip_weight* w = make_weight(ctx, type, in, out, n_experts, nbytes);
        // Device sources may still be in production on another stream (the
        // caller's generator or loader): uploads are rare, so wait for all
        // earlier work on the device before copying.
        if (kind == hipMemcpyDeviceToDevice) check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        try {
            fill_weight(ctx, w, src, kind);
        } catch (...) {
            (void)hipFree(w->dptr);
            delete w;
            throw;
        }
        // the batched matvec's slice sums for this shape, reserved now (an
        // allocation cannot happen later inside a captured graph)
        if (in <= UINT32_MAX && out <= UINT32_MAX) {
            const size_t part = pk::matvec_partial_floats(type, static_cast<uint32_t>(in), 8u,
                                                          static_cast<uint32_t>(out));
            if (part) ctx->mvpart.ensure(part);
        }
        ctx->stats.resident_bytes += nbytes;
        ctx->stats.uploaded_bytes += nbytes;
        ++ctx->live_weights;
        *out_w = w;
    });
}

pk_hip_status pk_hip_upload(pk_hip_ctx* ctx, uint32_t type, uint64_t in, uint64_t out,
                            uint32_t n_experts, const void* host_bytes, uint64_t nbytes,
                            pk_hip_weight** out_w, char* err, size_t cap) {
    return upload_impl(ctx, type, in, out, n_experts, host_bytes, nbytes, hipMemcpyHostToDevice,
                       out_w, err, cap);
}

pk_hip_status pk_hip_upload_device(pk_hip_ctx* ctx, uint32_t type, uint64_t in, uint64_t out,
                                   uint32_t n_experts, const void* device_bytes, uint64_t nbytes,
                                   pk_hip_weight** out_w, char* err, size_t cap) {
    return upload_impl(ctx, type, in, out, n_experts, device_bytes, nbytes,
                       hipMemcpyDeviceToDevice, out_w, err, cap);
}

void pk_hip_weight_release(pk_hip_weight* w) {
    if (!w) return;
    if (w->ctx) {
        std::lock_guard lock(w->ctx->mutex);
        (void)hipSetDevice(w->ctx->device);
        (void)hipStreamSynchronize(w->ctx->stream);
        (void)hipFree(w->dptr);
        w->ctx->stats.resident_bytes -= w->nbytes;
        --w->ctx->live_weights;
    }
    delete w;
}

uint64_t pk_hip_weight_bytes(const pk_hip_weight* w) { return w ? w->nbytes : 0; }

pk_hip_status pk_hip_weight_download(const pk_hip_weight* w, void* host_bytes, uint64_t nbytes,
                                     char* err, size_t cap) {
    pk_hip_ctx* ctx = w ? w->ctx : nullptr;
    return guarded(ctx, err, cap, [&] {
        if (!w || !host_bytes) throw ArgError("weight and destination are required");
        if (nbytes != w->nbytes) throw ArgError("destination size does not match the weight");
        require_usable(ctx);
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        if (!pk::planar_type(w->type)) {
            check(hipMemcpyAsync(host_bytes, w->dptr, nbytes, hipMemcpyDeviceToHost, ctx->stream),
                  "weight download");
            check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
            return;
        }
        const uint32_t n = slices_of(w);
        const uint32_t per = static_cast<uint32_t>(
            std::max<uint64_t>(1, std::min<uint64_t>(n, kStageBytes / w->slice_bytes)));
        DeviceBuffer<uint8_t> stage;
        stage.ensure(static_cast<size_t>(per) * w->slice_bytes);
        try {
            for (uint32_t s0 = 0; s0 < n; s0 += per) {
                const uint32_t k = std::min(per, n - s0);
                check(pk::launch_from_planar(w->type, w->dptr + static_cast<uint64_t>(s0) * w->slice_pitch,
                                             w->slice_pitch, stage.ptr, w->slice_bytes,
                                             slice_blocks(w), k, ctx->stream),
                      "GGUF weight layout");
                check(hipMemcpyAsync(static_cast<uint8_t*>(host_bytes) + static_cast<uint64_t>(s0) * w->slice_bytes,
                                     stage.ptr, static_cast<uint64_t>(k) * w->slice_bytes,
                                     hipMemcpyDeviceToHost, ctx->stream),
                      "weight download");
                check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
            }
        } catch (...) {
            (void)hipStreamSynchronize(ctx->stream);
            stage.release();
            throw;
        }
        stage.release();
    });
}
const void* pk_hip_weight_device_ptr(const pk_hip_weight* w) { return w ? w->dptr : nullptr; }

pk_hip_status pk_hip_matvec(pk_hip_ctx* ctx, const pk_hip_weight* w, uint32_t expert,
                            const float* x, uint32_t batch, float* y, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!w || !x || !y) throw ArgError("weight, input and output are required");
        if (batch == 0 || batch > 8) throw ArgError("batch must be between 1 and 8");
        std::lock_guard lock(ctx->mutex);
        if (!pk::matvec_supported(w->type, static_cast<uint32_t>(w->in), batch))
            throw Unsupported("matrix width/batch not covered by the HIP matvec kernels");
        ctx->set_device();
        ctx->x.ensure(static_cast<size_t>(batch) * w->in);
        ctx->y.ensure(static_cast<size_t>(batch) * w->out);
        check(hipMemcpyAsync(ctx->x.ptr, x, batch * w->in * sizeof(float), hipMemcpyHostToDevice,
                             ctx->stream),
              "copy input");
        enqueue_matvec(ctx, w, expert, ctx->x.ptr, batch, ctx->y.ptr, ctx->stream);
        check(hipMemcpyAsync(y, ctx->y.ptr, batch * w->out * sizeof(float),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy output");
        check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        collect_timing_matvec(ctx);
    });
}

pk_hip_status pk_hip_matvec_reference_order(pk_hip_ctx* ctx, const pk_hip_weight* w,
                                           uint32_t expert, const float* x, float* y, char* err,
                                           size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!w || !x || !y) throw ArgError("weight, input and output are required");
        std::lock_guard lock(ctx->mutex);
        if (!pk::ref_matvec_supported(w->type, static_cast<uint32_t>(w->in)))
            throw Unsupported("matrix type/width not covered by the reference-order kernels");
        if (w->n_experts && expert >= w->n_experts) throw ArgError("expert index out of range");
        if (!w->n_experts && expert != UINT32_MAX) throw ArgError("not an expert tensor");
        ctx->set_device();
        ctx->x.ensure(w->in);
        ctx->y.ensure(w->out);
        check(hipMemcpyAsync(ctx->x.ptr, x, w->in * sizeof(float), hipMemcpyHostToDevice,
                             ctx->stream),
              "copy input");
        pk::RefMatvecArgs a{};
        a.W = w->dptr + (w->n_experts ? uint64_t(expert) * w->slice_pitch : 0u);
        a.row_bytes = w->row_bytes;
        a.rows = static_cast<uint32_t>(w->out);
        a.in = static_cast<uint32_t>(w->in);
        a.x = ctx->x.ptr;
        a.y = ctx->y.ptr;
        launch_checked(pk::launch_ref_matvec(w->type, a, 1, ctx->stream), "reference matvec");
        check(hipMemcpyAsync(y, ctx->y.ptr, w->out * sizeof(float), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy output");
        check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        ++ctx->stats.matvec_calls;
    });
}

pk_hip_status pk_hip_matvec_async(pk_hip_ctx* ctx, const pk_hip_weight* w, uint32_t expert,
                                  const float* dx, uint32_t batch, float* dy, void* stream,
                                  char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
        const CaptureScope capture(s);
        enqueue_matvec(ctx, w, expert, dx, batch, dy, s);
        if (ctx->time_kernels) {
            check(hipStreamSynchronize(s), "hipStreamSynchronize");
            collect_timing_matvec(ctx);
        }
    });
}

pk_hip_status pk_hip_moe_decode(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer, const float* x,
                                float* y, uint32_t* ids, float* probs, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!x || !y || !ids || !probs) throw ArgError("input and output buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode_layer(ctx, layer);
        ctx->set_device();
        ctx->x.ensure(m.hidden);
        ctx->y.ensure(m.hidden);
        ensure_moe_scratch(ctx, m, layer->top_k);
        check(hipMemcpyAsync(ctx->x.ptr, x, m.hidden * sizeof(float), hipMemcpyHostToDevice,
                             ctx->stream),
              "copy input");
        enqueue_moe(ctx, layer, m, ctx->x.ptr, ctx->y.ptr, ctx->ids.ptr, ctx->probs.ptr,
                    ctx->stream);
        check(hipMemcpyAsync(y, ctx->y.ptr, m.hidden * sizeof(float), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy output");
        check(hipMemcpyAsync(ids, ctx->ids.ptr, layer->top_k * sizeof(uint32_t),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy ids");
        check(hipMemcpyAsync(probs, ctx->probs.ptr, layer->top_k * sizeof(float),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy probabilities");
        sync_and_check(ctx, ctx->stream);
        collect_timing_moe(ctx);
    });
}

pk::LibmExpf build_expf_cuckoo(const uint32_t* pairs, uint64_t n, std::vector<uint32_t>& slots);

pk_hip_status pk_hip_set_libm_expf(pk_hip_ctx* ctx, const uint32_t* pairs, uint64_t count,
                                   char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (count && !pairs) throw ArgError("libm_expf_pairs: missing table");
        if (count > (1ull << 24)) throw ArgError("libm_expf_pairs: oversized table");
        for (uint64_t i = 0; i < count; ++i)
            if (pairs[2 * i] == pk::kExpfEmpty || (i && pairs[2 * i] <= pairs[2 * i - 2]))
                throw ArgError("libm_expf_pairs: inputs not increasing");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        ctx->expf_slots.release();
        ctx->expf = pk::LibmExpf{nullptr, 0, 0, 0};
        if (!count) return;
        std::vector<uint32_t> host;
        const pk::LibmExpf t = build_expf_cuckoo(pairs, count, host);
        ctx->expf_slots.ensure(host.size());
        check(hipMemcpy(ctx->expf_slots.ptr, host.data(), host.size() * 4, hipMemcpyHostToDevice),
              "copy expf table");
        ctx->expf = t;
        ctx->expf.slots = ctx->expf_slots.ptr;
    });
}

pk_hip_status pk_hip_moe_decode_reference_order(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                                const float* x, float* y, uint32_t* ids,
                                                float* probs, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!x || !y || !ids || !probs) throw ArgError("input and output buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_layer(ctx, layer);
        pk::MoeDecodeArgs a{};
        a.router = reinterpret_cast<const float*>(layer->router->dptr);
        a.gate = layer->gate->dptr;
        a.up = layer->up->dptr;
        a.down = layer->down->dptr;
        a.gate_type = layer->gate->type;
        a.up_type = layer->up->type;
        a.down_type = layer->down->type;
        a.gate_slice = layer->gate->slice_pitch;
        a.up_slice = layer->up->slice_pitch;
        a.down_slice = layer->down->slice_pitch;
        a.gate_row = layer->gate->row_bytes;
        a.up_row = layer->up->row_bytes;
        a.down_row = layer->down->row_bytes;
        a.hidden = m.hidden;
        a.ffn = m.ffn;
        a.n_experts = m.experts;
        a.top_k = layer->top_k;
        a.normalize = layer->normalize ? 1u : 0u;
        a.scale = layer->scale;
        if (a.scale != 1.0f || !pk::ref_moe_block_supported(a))
            throw Unsupported("MoE shape not covered by the reference-order kernels");
        ctx->set_device();
        ctx->x.ensure(m.hidden);
        ctx->y.ensure(m.hidden);
        ctx->ids.ensure(16);
        ctx->probs.ensure(16);
        ctx->ref_scratch.ensure(pk::ref_scratch_floats(a.top_k, m.ffn, m.hidden));
        a.x = ctx->x.ptr;
        a.y = ctx->y.ptr;
        a.ids = ctx->ids.ptr;
        a.probs = ctx->probs.ptr;
        a.status = status_words(ctx);
        check(hipMemcpyAsync(ctx->x.ptr, x, m.hidden * sizeof(float), hipMemcpyHostToDevice,
                             ctx->stream),
              "copy input");
        launch_checked(pk::launch_ref_moe_block(a, ctx->ref_scratch.ptr, ctx->expf, ctx->stream),
                       "reference-order MoE launch");
        check(hipMemcpyAsync(y, ctx->y.ptr, m.hidden * sizeof(float), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy output");
        check(hipMemcpyAsync(ids, ctx->ids.ptr, layer->top_k * sizeof(uint32_t),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy ids");
        check(hipMemcpyAsync(probs, ctx->probs.ptr, layer->top_k * sizeof(float),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy probabilities");
        sync_and_check(ctx, ctx->stream);
        ++ctx->stats.moe_decode_calls;
        ctx->stats.expert_hits += layer->top_k;
        ctx->stats.weight_bytes += layer->router->nbytes +
                                   static_cast<uint64_t>(layer->top_k) *
                                       (layer->gate->slice_bytes + layer->up->slice_bytes +
                                        layer->down->slice_bytes);
    });
}

pk_hip_status pk_hip_moe_decode_async(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                      const float* dx, float* dy, uint32_t* dids, float* dprobs,
                                      void* stream, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!dx || !dy || !dids || !dprobs) throw ArgError("device buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode_layer(ctx, layer);
        ctx->set_device();
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
        const CaptureScope capture(s);
        enqueue_moe(ctx, layer, m, dx, dy, dids, dprobs, s);
        if (ctx->time_kernels) {
            check(hipStreamSynchronize(s), "hipStreamSynchronize");
            collect_timing_moe(ctx);
        }
    });
}

pk_hip_status pk_hip_moe_decode_traced_async(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                             const float* dx, float* dy, uint32_t* dids,
                                             float* dprobs, uint64_t* dtrace, void* stream,
                                             char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!dx || !dy || !dids || !dprobs || !dtrace) throw ArgError("device buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode_layer(ctx, layer);
        ctx->set_device();
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
        const CaptureScope capture(s);
        enqueue_moe(ctx, layer, m, dx, dy, dids, dprobs, s, nullptr, nullptr, dtrace);
    });
}

pk_hip_status pk_hip_moe_decode_noalloc(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                        const float* dx, float* dy, uint32_t* dids, float* dprobs,
                                        void* stream, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!dx || !dy || !dids || !dprobs) throw ArgError("device buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode_layer(ctx, layer);
        if (m.experts > noalloc::kMaxExperts || layer->top_k > noalloc::kMaxTopK ||
            m.ffn > noalloc::kMaxFfn)
            throw ArgError("layer exceeds the no-allocation scratch (at most 256 experts, top-k 8, "
                           "ffn 2048)");
        if (!ctx->noalloc_scratch) throw ArgError("no static scratch on this device");
        ctx->set_device();
        uint8_t* base = ctx->noalloc_scratch;
        const MoeScratch sc{reinterpret_cast<double*>(base + noalloc::kStatusBytes),
                            reinterpret_cast<double*>(base + noalloc::kStatusBytes + noalloc::kSumBytes),
                            reinterpret_cast<float*>(base + noalloc::kStatusBytes + 2 * noalloc::kSumBytes),
                            reinterpret_cast<uint32_t*>(base)};
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
        const CaptureScope capture(s);
        enqueue_moe(ctx, layer, m, dx, dy, dids, dprobs, s, nullptr, &sc);
        if (ctx->time_kernels) {
            check(hipStreamSynchronize(s), "hipStreamSynchronize");
            collect_timing_moe(ctx);
        }
    });
}

pk_hip_status pk_hip_moe35_decode(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                  const float* x, float* y, uint32_t* ids, float* weights,
                                  char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!x || !y || !ids || !weights) throw ArgError("input and output buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode35(ctx, layer);
        ctx->set_device();
        ctx->x.ensure(m.hidden);
        ctx->y.ensure(m.hidden);
        ensure_moe_scratch(ctx, m, layer->routed.top_k);
        check(hipMemcpyAsync(ctx->x.ptr, x, m.hidden * sizeof(float), hipMemcpyHostToDevice,
                             ctx->stream),
              "copy input");
        enqueue_moe(ctx, &layer->routed, m, ctx->x.ptr, ctx->y.ptr, ctx->ids.ptr, ctx->probs.ptr,
                    ctx->stream, layer);
        check(hipMemcpyAsync(y, ctx->y.ptr, m.hidden * sizeof(float), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy output");
        check(hipMemcpyAsync(ids, ctx->ids.ptr, layer->routed.top_k * sizeof(uint32_t),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy ids");
        check(hipMemcpyAsync(weights, ctx->probs.ptr, layer->routed.top_k * sizeof(float),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy weights");
        sync_and_check(ctx, ctx->stream);
        collect_timing_moe(ctx);
    });
}

pk_hip_status pk_hip_moe35_decode_async(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                        const float* dx, float* dy, uint32_t* dids,
                                        float* dweights, void* stream, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!dx || !dy || !dids || !dweights) throw ArgError("device buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode35(ctx, layer);
        ctx->set_device();
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
        const CaptureScope capture(s);
        enqueue_moe(ctx, &layer->routed, m, dx, dy, dids, dweights, s, layer);
        if (ctx->time_kernels) {
            check(hipStreamSynchronize(s), "hipStreamSynchronize");
            collect_timing_moe(ctx);
        }
    });
}

namespace {

MoeShape check_prefill(pk_hip_ctx* c, const pk_hip_moe_layer* L, uint32_t tokens,
                       uint32_t variant = 0) {
    const MoeShape m = check_layer(c, L);
    if (tokens == 0 || tokens > pk::kMaxPrefillTokens)
        throw ArgError("prefill token count must be between 1 and " +
                       std::to_string(pk::kMaxPrefillTokens));
    if (!pk::moe_prefill_supported(L->gate->type, L->up->type, L->down->type, m.hidden, m.ffn,
                                   m.experts, L->top_k, tokens, variant))
        throw Unsupported("MoE prefill shape not covered by the HIP kernels");
    return m;
}

// Variant 1 (shared != nullptr): the shared expert is one more route per token
// and one more router row and expert group.
void enqueue_prefill(pk_hip_ctx* c, const pk_hip_moe_layer* L, const MoeShape& m, uint32_t tokens,
                     const float* dx, float* dy, uint32_t* dids, float* dprobs, hipStream_t s,
                     const pk_hip_moe35_layer* shared = nullptr) {
    const uint64_t V = shared ? 1u : 0u;
    const uint64_t T = tokens, K = L->top_k + V, E = m.experts + V;
    const uint32_t max_tiles = pk::moe_prefill_max_tiles(tokens, static_cast<uint32_t>(K),
                                                         static_cast<uint32_t>(E));
    c->prow_sum.ensure(T * E);
    c->prow_bound.ensure(T * E);
    c->poffsets.ensure(E + 1);
    c->ptiles.ensure(static_cast<size_t>(max_tiles) + 1);
    c->pperm.ensure(T * K);
    c->pxparts.ensure(3 * T * m.hidden);
    c->pxsum.ensure(T * m.hidden / 16);
    c->paparts.ensure(3 * T * K * m.ffn);
    c->pasum.ensure(T * K * m.ffn / 16);
    c->pout.ensure(T * K * m.hidden);
    pk::MoePrefillArgs a{};
    pk::MoeDecodeArgs& l = a.layer;
    l.router = reinterpret_cast<const float*>(L->router->dptr);
    l.gate = L->gate->dptr;
    l.up = L->up->dptr;
    l.down = L->down->dptr;
    l.gate_type = L->gate->type;
    l.up_type = L->up->type;
    l.down_type = L->down->type;
    l.gate_slice = L->gate->slice_pitch;
    l.up_slice = L->up->slice_pitch;
    l.down_slice = L->down->slice_pitch;
    l.gate_row = L->gate->row_bytes;
    l.up_row = L->up->row_bytes;
    l.down_row = L->down->row_bytes;
    l.hidden = m.hidden;
    l.ffn = m.ffn;
    l.n_experts = m.experts;
    l.top_k = L->top_k;
    l.normalize = L->normalize ? 1u : 0u;
    l.scale = L->scale;
    l.status = status_words(c);
    if (shared) {
        l.variant = 1;
        l.shared_router = reinterpret_cast<const float*>(shared->shared_router->dptr);
        l.shared_gate = shared->shared_gate->dptr;
        l.shared_up = shared->shared_up->dptr;
        l.shared_down = shared->shared_down->dptr;
    }
    a.tokens = tokens;
    a.max_tiles = max_tiles;
    a.x = dx;
    a.y = dy;
    a.ids = dids;
    a.probs = dprobs;
    a.row_sum = c->prow_sum.ptr;
    a.row_bound = c->prow_bound.ptr;
    a.offsets = c->poffsets.ptr;
    a.tiles = c->ptiles.ptr;
    a.n_tiles = c->ptiles.ptr + max_tiles;
    a.perm = c->pperm.ptr;
    a.x_parts = c->pxparts.ptr;
    a.x_sums = c->pxsum.ptr;
    a.act_parts = c->paparts.ptr;
    a.act_sums = c->pasum.ptr;
    a.out = c->pout.ptr;
    a.status = status_words(c);
    if (c->time_kernels) hold_stream(c, s);
    begin_timing(c, s, 6);
    launch_checked(pk::launch_prefill_routing(a, s), "prefill routing launch");
    begin_timing(c, s, 7);
    launch_checked(pk::launch_prefill_gate_up(a, s), "prefill gate/up launch");
    begin_timing(c, s, 8);
    launch_checked(pk::launch_prefill_down(a, s), "prefill down launch");
    begin_timing(c, s, 9);
    ++c->stats.prefill_calls;
    c->stats.prefill_tokens += tokens;
    c->stats.dispatches += 6;
    count_dispatch(c, L->gate->type);
    count_dispatch(c, L->down->type);
    c->stats.dispatches -= 2;
}

void collect_timing_prefill(pk_hip_ctx* c) {
    if (!c->time_kernels) return;
    c->stats.prefill_ns += elapsed_ns(c, 6, 9);
    c->stats.prefill_route_ns += elapsed_ns(c, 6, 7);
    c->stats.prefill_gate_up_ns += elapsed_ns(c, 7, 8);
    c->stats.prefill_down_ns += elapsed_ns(c, 8, 9);
}

}  // namespace

pk_hip_status pk_hip_moe_prefill(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer, const float* x,
                                 uint32_t tokens, float* y, uint32_t* ids, float* probs,
                                 char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!x || !y || !ids || !probs) throw ArgError("input and output buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_prefill(ctx, layer, tokens);
        ctx->set_device();
        const uint64_t T = tokens, K = layer->top_k;
        ctx->px.ensure(T * m.hidden);
        ctx->py.ensure(T * m.hidden);
        ctx->pids.ensure(T * K);
        ctx->pprobs.ensure(T * K);
        check(hipMemcpyAsync(ctx->px.ptr, x, T * m.hidden * sizeof(float), hipMemcpyHostToDevice,
                             ctx->stream),
              "copy input");
        enqueue_prefill(ctx, layer, m, tokens, ctx->px.ptr, ctx->py.ptr, ctx->pids.ptr,
                        ctx->pprobs.ptr, ctx->stream);
        check(hipMemcpyAsync(y, ctx->py.ptr, T * m.hidden * sizeof(float), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy output");
        check(hipMemcpyAsync(ids, ctx->pids.ptr, T * K * sizeof(uint32_t), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy ids");
        check(hipMemcpyAsync(probs, ctx->pprobs.ptr, T * K * sizeof(float),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy probabilities");
        sync_and_check(ctx, ctx->stream);
        collect_timing_prefill(ctx);
    });
}

pk_hip_status pk_hip_moe_prefill_async(pk_hip_ctx* ctx, const pk_hip_moe_layer* layer,
                                       const float* dx, uint32_t tokens, float* dy,
                                       uint32_t* dids, float* dprobs, void* stream, char* err,
                                       size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!dx || !dy || !dids || !dprobs) throw ArgError("device buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_prefill(ctx, layer, tokens);
        ctx->set_device();
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
        const CaptureScope capture(s);
        enqueue_prefill(ctx, layer, m, tokens, dx, dy, dids, dprobs, s);
        if (ctx->time_kernels) {
            check(hipStreamSynchronize(s), "hipStreamSynchronize");
            collect_timing_prefill(ctx);
        }
    });
}

pk_hip_status pk_hip_moe35_prefill(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                   const float* x, uint32_t tokens, float* y, uint32_t* ids,
                                   float* weights, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!x || !y || !ids || !weights) throw ArgError("input and output buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode35(ctx, layer);
        check_prefill(ctx, &layer->routed, tokens, 1);
        ctx->set_device();
        const uint64_t T = tokens, K = layer->routed.top_k;
        ctx->px.ensure(T * m.hidden);
        ctx->py.ensure(T * m.hidden);
        ctx->pids.ensure(T * K);
        ctx->pprobs.ensure(T * K);
        check(hipMemcpyAsync(ctx->px.ptr, x, T * m.hidden * sizeof(float), hipMemcpyHostToDevice,
                             ctx->stream),
              "copy input");
        enqueue_prefill(ctx, &layer->routed, m, tokens, ctx->px.ptr, ctx->py.ptr, ctx->pids.ptr,
                        ctx->pprobs.ptr, ctx->stream, layer);
        check(hipMemcpyAsync(y, ctx->py.ptr, T * m.hidden * sizeof(float), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy output");
        check(hipMemcpyAsync(ids, ctx->pids.ptr, T * K * sizeof(uint32_t), hipMemcpyDeviceToHost,
                             ctx->stream),
              "copy ids");
        check(hipMemcpyAsync(weights, ctx->pprobs.ptr, T * K * sizeof(float),
                             hipMemcpyDeviceToHost, ctx->stream),
              "copy weights");
        sync_and_check(ctx, ctx->stream);
        collect_timing_prefill(ctx);
    });
}

pk_hip_status pk_hip_moe35_prefill_async(pk_hip_ctx* ctx, const pk_hip_moe35_layer* layer,
                                         const float* dx, uint32_t tokens, float* dy,
                                         uint32_t* dids, float* dweights, void* stream, char* err,
                                         size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!dx || !dy || !dids || !dweights) throw ArgError("device buffers are required");
        std::lock_guard lock(ctx->mutex);
        const MoeShape m = check_decode35(ctx, layer);
        check_prefill(ctx, &layer->routed, tokens, 1);
        ctx->set_device();
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : ctx->stream;
        const CaptureScope capture(s);
        enqueue_prefill(ctx, &layer->routed, m, tokens, dx, dy, dids, dweights, s, layer);
        if (ctx->time_kernels) {
            check(hipStreamSynchronize(s), "hipStreamSynchronize");
            collect_timing_prefill(ctx);
        }
    });
}

pk_hip_status pk_hip_sync(pk_hip_ctx* ctx, void* stream, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        if (stream) check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "sync stream");
        sync_and_check(ctx, ctx->stream);
    });
}

// ---------------------------------------------------------------------------
// Whole-model greedy decode (Qwen3MoeRunner on the device).

// prepare_qwen_rope (src/qwen3_moe_runner.cpp:141-155) with this host's libm
// for positions 0 .. positions - 1: per position cos [head_dim / 2], then sin.
std::vector<float> rope_table_host(uint32_t positions, uint32_t head_dim, float theta) {
    const uint32_t half = head_dim / 2;
    std::vector<float> table(uint64_t(positions) * head_dim);
    for (uint32_t pos = 0; pos < positions; ++pos) {
        float* row = table.data() + uint64_t(pos) * head_dim;
        for (uint32_t p = 0; p < half; ++p) {
            const float angle = static_cast<float>(pos) *
                std::pow(theta, -static_cast<float>(p) / static_cast<float>(half));
            row[p] = std::cos(angle);
            row[half + p] = std::sin(angle);
        }
    }
    return table;
}

// Two-choice cuckoo table of (input bits, libm result bits) for the device's
// expf_libm: each half holds 1 << bits slots, at most a third of all slots
// used; the hash multipliers are the first pair from a fixed list with which
// every insertion settles (deterministic for a given table).
pk::LibmExpf build_expf_cuckoo(const uint32_t* pairs, uint64_t n, std::vector<uint32_t>& slots) {
    static const uint32_t kMul[] = {0x9E3779B1u, 0x85EBCA77u, 0xC2B2AE3Du, 0x27D4EB2Fu,
                                    0x165667B1u, 0xD3A2646Du, 0xFD7046C5u, 0xB55A4F09u};
    uint32_t bits = 4;
    while ((2ull << bits) < 3 * n) ++bits;
    const uint64_t half = 1ull << bits;
    for (uint32_t t0 = 0; t0 < 8; ++t0) {
        for (uint32_t t1 = 0; t1 < 8; ++t1) {
            if (t0 == t1) continue;
            const uint32_t mul[2] = {kMul[t0], kMul[t1]};
            slots.assign(4 * half, pk::kExpfEmpty);
            bool ok = true;
            for (uint64_t i = 0; i < n && ok; ++i) {
                uint32_t key = pairs[2 * i], val = pairs[2 * i + 1];
                uint32_t side = 0;
                ok = false;
                for (int step = 0; step < 512; ++step) {
                    const uint64_t at = 2 * (side * half + ((key * mul[side]) >> (32 - bits)));
                    std::swap(key, slots[at]);
                    std::swap(val, slots[at + 1]);
                    if (key == pk::kExpfEmpty) {
                        ok = true;
                        break;
                    }
                    side ^= 1u;
                }
            }
            if (ok) return pk::LibmExpf{nullptr, bits, mul[0], mul[1]};
        }
    }
    throw Unsupported("libm_expf_pairs: no cuckoo placement found");
}

struct pk_hip_qwen3moe {
    pk_hip_ctx* ctx = nullptr;
    pk_hip_qwen3moe_config cfg{};
    pk::ModelArgs args{};
    std::vector<pk::ModelLayer> layers;
    DeviceBuffer<uint32_t> state, tokens, ids, moe_status;
    DeviceBuffer<float> work, probs, act, moe_out, rope_table, ref_scratch;
    DeviceBuffer<uint32_t> expf_slots;
    DeviceBuffer<double> row_sum, row_bound;
    DeviceBuffer<uint16_t> kv;
    DeviceBuffer<uint8_t> qkv;  // fast mode: each layer's q, k and v rows back to back
    hipGraphExec_t step_logits = nullptr, step_plain = nullptr;
    hipEvent_t ev[2] = {};
};

namespace {

const uint8_t* weight_bytes(const pk_hip_weight* w) { return w->dptr; }

void require_weight(const pk_hip_weight* w, const char* what, uint64_t in, uint64_t out) {
    if (!w) throw ArgError(std::string("missing weight: ") + what);
    if (w->in != in || w->out != out || w->n_experts != 0)
        throw ArgError(std::string("unexpected dimensions for weight: ") + what);
}

void require_vector(const pk_hip_weight* w, const char* what, uint64_t n) {
    require_weight(w, what, n, 1);
    if (w->type != 0) throw ArgError(std::string("norm weight must be F32: ") + what);
}

void require_matvec(const pk_hip_weight* w, const char* what, uint64_t in, uint64_t out,
                    bool exact) {
    require_weight(w, what, in, out);
    const bool ok = exact ? pk::ref_matvec_supported(w->type, static_cast<uint32_t>(in))
                          : pk::matvec_supported(w->type, static_cast<uint32_t>(in), 1);
    if (!ok) throw Unsupported(std::string("no matvec kernel for weight: ") + what);
}

hipGraphExec_t capture_step(pk_hip_qwen3moe* m, bool logits) {
    hipStream_t s = m->ctx->stream;
    check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    const hipError_t launched = pk::launch_model_step(m->args, m->layers.data(), logits, s);
    hipGraph_t graph = nullptr;
    const hipError_t ended = hipStreamEndCapture(s, &graph);
    check(launched, "model step launch");
    check(ended, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    check(inst, "hipGraphInstantiate");
    return exec;
}

void release_model(pk_hip_qwen3moe* m) {
    if (m->step_logits) (void)hipGraphExecDestroy(m->step_logits);
    if (m->step_plain) (void)hipGraphExecDestroy(m->step_plain);
    for (auto& e : m->ev)
        if (e) (void)hipEventDestroy(e);
    m->state.release();
    m->tokens.release();
    m->ids.release();
    m->moe_status.release();
    m->work.release();
    m->probs.release();
    m->act.release();
    m->moe_out.release();
    m->rope_table.release();
    m->ref_scratch.release();
    m->expf_slots.release();
    m->row_sum.release();
    m->row_bound.release();
    m->kv.release();
    m->qkv.release();
}

}  // namespace

pk_hip_status pk_hip_qwen3moe_create(pk_hip_ctx* ctx, const pk_hip_qwen3moe_config* cfg,
                                     const pk_hip_qwen3moe_weights* w, pk_hip_qwen3moe** out,
                                     char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!cfg || !w || !out || !w->layers) throw ArgError("config, weights and output are required");
        const pk_hip_qwen3moe_config& c = *cfg;
        if (c.layers == 0 || c.hidden == 0 || c.heads == 0 || c.kv_heads == 0 || c.head_dim == 0 ||
            c.vocab == 0 || c.kv_capacity == 0 || c.context == 0)
            throw ArgError("model dimensions must be non-zero");
        if (c.kv_capacity > c.context) throw ArgError("KV window exceeds the model context");
        if (c.heads % c.kv_heads) throw ArgError("query heads must be evenly grouped over KV heads");
        if (!(c.rms_eps > 0.0f) || !(c.rope_theta > 0.0f)) throw ArgError("invalid norm epsilon or RoPE base");
        const uint64_t qd = uint64_t(c.heads) * c.head_dim, kd = uint64_t(c.kv_heads) * c.head_dim;
        require_weight(w->token_embd, "token_embd", c.hidden, c.vocab);
        require_vector(w->output_norm, "output_norm", c.hidden);
        const bool exact = c.reference_order != 0;
        require_matvec(w->output, "output", c.hidden, c.vocab, exact);
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        auto m = std::make_unique<pk_hip_qwen3moe>();
        m->ctx = ctx;
        m->cfg = c;
        pk::ModelArgs& a = m->args;
        a.layers = c.layers;
        a.hidden = c.hidden;
        a.heads = c.heads;
        a.kv_heads = c.kv_heads;
        a.head_dim = c.head_dim;
        a.vocab = c.vocab;
        a.capacity = c.kv_capacity;
        a.embd_type = w->token_embd->type;
        a.out_type = w->output->type;
        a.embd_row = w->token_embd->row_bytes;
        a.out_row = w->output->row_bytes;
        a.rms_eps = c.rms_eps;
        a.rope_theta = c.rope_theta;
        a.exact = exact ? 1u : 0u;
        a.attn_scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));  // KvCache::attend default
        a.embd = weight_bytes(w->token_embd);
        a.out_norm = reinterpret_cast<const float*>(weight_bytes(w->output_norm));
        a.out = weight_bytes(w->output);
        if (!pk::model_supported(a)) throw Unsupported("model shape not covered by the HIP kernels");
        // device state and activations
        m->state.ensure(4);
        m->tokens.ensure(1);
        const uint64_t wf = 4ull * c.hidden + 2 * qd + 2 * kd + c.vocab + 2ull * (c.vocab / 2048 + 1);
        m->work.ensure(wf);
        float* p = m->work.ptr;
        a.hidden_state = p; p += c.hidden;
        a.normed = p; p += c.hidden;
        a.attn_out = p; p += c.hidden;
        a.hidden_alt = p; p += c.hidden;
        a.q = p; p += qd;  // q, k, v back to back: one matvec fills all three
        a.k = p; p += kd;
        a.v = p; p += kd;
        a.att = p; p += qd;
        a.logits = p; p += c.vocab;
        a.argmax_part = p;
        a.state = m->state.ptr;
        m->kv.ensure(2ull * c.layers * c.kv_capacity * kd);
        uint32_t max_experts = 1, max_k = 1, max_ffn = 1;
        for (uint32_t l = 0; l < c.layers; ++l) {
            const pk_hip_qwen3moe_layer& L = w->layers[l];
            if (!L.router || !L.gate || !L.up || !L.down) throw ArgError("missing MoE weight");
            max_experts = std::max<uint32_t>(max_experts, static_cast<uint32_t>(L.router->out));
            max_ffn = std::max<uint32_t>(max_ffn, static_cast<uint32_t>(L.gate->out));
        }
        max_k = c.top_k;
        m->ids.ensure(16);
        m->probs.ensure(16);
        m->moe_status.ensure(4);
        m->act.ensure(uint64_t(max_k) * max_ffn);
        m->row_sum.ensure(max_experts);
        m->row_bound.ensure(max_experts);
        m->moe_out.ensure(c.hidden);
        if (!pk::ref_attention_supported(c.head_dim, c.kv_capacity))
            throw Unsupported("attention covers head_dim 64/128/256");
        const std::vector<float> table = rope_table_host(c.context, c.head_dim, c.rope_theta);
        m->rope_table.ensure(table.size());
        check(hipMemcpy(m->rope_table.ptr, table.data(), table.size() * sizeof(float),
                        hipMemcpyHostToDevice),
              "copy RoPE table");
        a.rope_table = m->rope_table.ptr;
        if (exact) {
            if (max_experts > pk::kMaxExperts256 || c.top_k > pk::kMaxRefTopK)
                throw Unsupported("reference-order MoE covers up to 256 experts and top-16");
            if (c.hidden > pk::kMaxRefNormWidth)
                throw Unsupported("reference-order kernels cover hidden <= 4096");
            m->ref_scratch.ensure(pk::ref_scratch_floats(c.top_k, max_ffn, c.hidden));
            a.ref_scratch = m->ref_scratch.ptr;
            if (c.libm_expf_count) {
                if (!c.libm_expf_pairs || c.libm_expf_count > (1ull << 24))
                    throw ArgError("libm_expf_pairs: missing or oversized table");
                const uint32_t* p = c.libm_expf_pairs;
                for (uint64_t i = 0; i < c.libm_expf_count; ++i) {
                    if (p[2 * i] == pk::kExpfEmpty || (i && p[2 * i] <= p[2 * i - 2]))
                        throw ArgError("libm_expf_pairs: inputs not increasing");
                }
                std::vector<uint32_t> slots;
                a.expf = build_expf_cuckoo(p, c.libm_expf_count, slots);
                m->expf_slots.ensure(slots.size());
                check(hipMemcpy(m->expf_slots.ptr, slots.data(), slots.size() * 4,
                                hipMemcpyHostToDevice),
                      "copy expf table");
                a.expf.slots = m->expf_slots.ptr;
            }
        }
        check(hipMemsetAsync(m->moe_status.ptr, 0, 4 * sizeof(uint32_t), ctx->stream), "clear status");
        // fast mode, GGUF-form rows (planar types keep a plane per tensor): each
        // layer's q, k and v rows are copied back to back, so one launch computes
        // all three.  Layers may use different attention formats, so the offsets
        // are a prefix sum of each eligible layer's own 256-byte-rounded size and
        // the buffer is allocated once, before any copy.
        std::vector<uint64_t> qkv_off(c.layers, ~0ull);
        if (!exact) {
            uint64_t total = 0;
            for (uint32_t l = 0; l < c.layers; ++l) {
                const pk_hip_qwen3moe_layer& L = w->layers[l];
                if (!L.q || !L.k || !L.v || pk::planar_type(L.q->type)) continue;
                if (L.k->type != L.q->type || L.v->type != L.q->type) continue;
                if (L.k->row_bytes != L.q->row_bytes || L.v->row_bytes != L.q->row_bytes) continue;
                const uint64_t bytes = uint64_t(qd + 2 * kd) * L.q->row_bytes + pk::kWeightTailPad;
                qkv_off[l] = total;
                total += (bytes + 255) / 256 * 256;
            }
            if (total) m->qkv.ensure(total);
        }
        m->layers.resize(c.layers);
        for (uint32_t l = 0; l < c.layers; ++l) {
            const pk_hip_qwen3moe_layer& L = w->layers[l];
            pk::ModelLayer& D = m->layers[l];
            require_vector(L.attn_norm, "attn_norm", c.hidden);
            require_vector(L.q_norm, "attn_q_norm", c.head_dim);
            require_vector(L.k_norm, "attn_k_norm", c.head_dim);
            require_vector(L.ffn_norm, "ffn_norm", c.hidden);
            require_matvec(L.q, "attn_q", c.hidden, qd, exact);
            require_matvec(L.k, "attn_k", c.hidden, kd, exact);
            require_matvec(L.v, "attn_v", c.hidden, kd, exact);
            require_matvec(L.o, "attn_output", qd, c.hidden, exact);
            if (L.k->type != L.q->type || L.v->type != L.q->type || L.o->type != L.q->type)
                throw Unsupported("attention weights must share one format");
            const pk_hip_moe_layer ml{L.router, L.gate, L.up, L.down, c.top_k, c.normalize, 1.0f};
            const MoeShape ms = check_decode_layer(ctx, &ml);
            if (ms.hidden != c.hidden) throw ArgError("MoE layer width does not match the model");
            D.attn_norm = reinterpret_cast<const float*>(weight_bytes(L.attn_norm));
            D.q_norm = reinterpret_cast<const float*>(weight_bytes(L.q_norm));
            D.k_norm = reinterpret_cast<const float*>(weight_bytes(L.k_norm));
            D.ffn_norm = reinterpret_cast<const float*>(weight_bytes(L.ffn_norm));
            D.q = weight_bytes(L.q);
            D.k = weight_bytes(L.k);
            D.v = weight_bytes(L.v);
            D.o = weight_bytes(L.o);
            D.attn_type = L.q->type;
            D.q_row = L.q->row_bytes;
            D.k_row = L.k->row_bytes;
            D.v_row = L.v->row_bytes;
            D.o_row = L.o->row_bytes;
            D.qkv = nullptr;
            if (qkv_off[l] != ~0ull) {
                const uint64_t qb = qd * D.q_row, kb = kd * D.q_row;
                uint8_t* dst = m->qkv.ptr + qkv_off[l];
                check(hipMemcpyAsync(dst, D.q, qb, hipMemcpyDeviceToDevice, ctx->stream), "copy q rows");
                check(hipMemcpyAsync(dst + qb, D.k, kb, hipMemcpyDeviceToDevice, ctx->stream), "copy k rows");
                check(hipMemcpyAsync(dst + qb + kb, D.v, kb, hipMemcpyDeviceToDevice, ctx->stream),
                      "copy v rows");
                D.qkv = dst;
            }
            D.kcache = m->kv.ptr + 2ull * l * c.kv_capacity * kd;
            D.vcache = D.kcache + uint64_t(c.kv_capacity) * kd;
            pk::MoeDecodeArgs& g = D.moe;
            g = pk::MoeDecodeArgs{};
            g.router = reinterpret_cast<const float*>(L.router->dptr);
            g.gate = L.gate->dptr;
            g.up = L.up->dptr;
            g.down = L.down->dptr;
            g.gate_type = L.gate->type;
            g.up_type = L.up->type;
            g.down_type = L.down->type;
            g.gate_slice = L.gate->slice_pitch;
            g.up_slice = L.up->slice_pitch;
            g.down_slice = L.down->slice_pitch;
            g.gate_row = L.gate->row_bytes;
            g.up_row = L.up->row_bytes;
            g.down_row = L.down->row_bytes;
            g.hidden = ms.hidden;
            g.ffn = ms.ffn;
            g.n_experts = ms.experts;
            g.top_k = c.top_k;
            g.normalize = c.normalize ? 1u : 0u;
            g.scale = 1.0f;
            g.x = a.normed;
            g.y = m->moe_out.ptr;
            g.ids = m->ids.ptr;
            g.probs = m->probs.ptr;
            g.row_sum = m->row_sum.ptr;
            g.row_bound = m->row_bound.ptr;
            g.act = m->act.ptr;
            g.status = m->moe_status.ptr;
        }
        for (auto& e : m->ev) check(hipEventCreate(&e), "hipEventCreate");
        *out = m.release();
    });
}

void pk_hip_qwen3moe_destroy(pk_hip_qwen3moe* m) {
    if (!m) return;
    if (m->ctx) {
        std::lock_guard lock(m->ctx->mutex);
        (void)hipSetDevice(m->ctx->device);
        (void)hipStreamSynchronize(m->ctx->stream);
        release_model(m);
    }
    delete m;
}

pk_hip_status pk_hip_qwen3moe_generate(pk_hip_qwen3moe* m, const uint32_t* prompt,
                                       uint32_t n_prompt, uint32_t n_new, uint32_t* out_tokens,
                                       float* last_logits, pk_hip_generation_stats* stats,
                                       char* err, size_t cap) {
    pk_hip_ctx* ctx = m ? m->ctx : nullptr;
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!prompt || n_prompt == 0 || (n_new && !out_tokens))
            throw ArgError("a prompt and an output buffer are required");
        const pk::ModelArgs& a = m->args;
        for (uint32_t i = 0; i < n_prompt; ++i)
            if (prompt[i] >= a.vocab) throw ArgError("token id exceeds model vocabulary");
        if (uint64_t(n_prompt) + n_new > m->cfg.context)
            throw ArgError("prompt and new tokens exceed the model context");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        hipStream_t s = ctx->stream;
        const uint64_t total = uint64_t(n_prompt) + n_new + 1;
        if (m->tokens.count < total) {
            m->tokens.ensure(total);
            // the graphs hold the old token buffer: capture again
            if (m->step_logits) (void)hipGraphExecDestroy(m->step_logits);
            if (m->step_plain) (void)hipGraphExecDestroy(m->step_plain);
            m->step_logits = m->step_plain = nullptr;
        }
        m->args.tokens = m->tokens.ptr;
        check(hipMemcpyAsync(m->tokens.ptr, prompt, n_prompt * sizeof(uint32_t),
                             hipMemcpyHostToDevice, s),
              "copy prompt");
        const uint32_t init[4] = {0, n_prompt, 0, 0};
        check(hipMemcpyAsync(m->state.ptr, init, sizeof(init), hipMemcpyHostToDevice, s), "reset state");
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        if (!m->step_logits) m->step_logits = capture_step(m, true);
        if (!m->step_plain) m->step_plain = capture_step(m, false);
        const auto t0 = std::chrono::steady_clock::now();
        for (uint32_t i = 0; i + 1 < n_prompt; ++i) check(hipGraphLaunch(m->step_plain, s), "prefill step");
        check(hipGraphLaunch(m->step_logits, s), "prefill logits step");
        if (last_logits)
            check(hipMemcpyAsync(last_logits, a.logits, uint64_t(a.vocab) * sizeof(float),
                                 hipMemcpyDeviceToHost, s),
                  "copy logits");
        check(hipStreamSynchronize(s), "hipStreamSynchronize");
        const auto t1 = std::chrono::steady_clock::now();
        check(hipEventRecord(m->ev[0], s), "hipEventRecord");
        for (uint32_t j = 0; j + 1 < n_new; ++j) check(hipGraphLaunch(m->step_logits, s), "decode step");
        check(hipEventRecord(m->ev[1], s), "hipEventRecord");
        check(hipEventSynchronize(m->ev[1]), "hipEventSynchronize");
        float ms = 0.0f;
        check(hipEventElapsedTime(&ms, m->ev[0], m->ev[1]), "hipEventElapsedTime");
        uint32_t flags[4] = {}, moe_flags[4] = {};
        check(hipMemcpy(flags, m->state.ptr, sizeof(flags), hipMemcpyDeviceToHost), "read state");
        check(hipMemcpy(moe_flags, m->moe_status.ptr, sizeof(moe_flags), hipMemcpyDeviceToHost),
              "read router status");
        if (moe_flags[0] || flags[2]) {
            const uint32_t zero[4] = {};
            (void)hipMemcpy(m->moe_status.ptr, zero, sizeof(zero), hipMemcpyHostToDevice);
            throw std::runtime_error(moe_flags[0] ? "expert router produced non-finite logits"
                                                  : "model produced non-finite logits");
        }
        if (n_new)
            check(hipMemcpy(out_tokens, m->tokens.ptr + n_prompt, n_new * sizeof(uint32_t),
                            hipMemcpyDeviceToHost),
                  "copy tokens");
        if (stats) {
            stats->prefill_ns = static_cast<uint64_t>(
                std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count());
            stats->decode_ns = static_cast<uint64_t>(static_cast<double>(ms) * 1.0e6);
            stats->prompt_tokens = n_prompt;
            stats->decode_forwards = n_new ? n_new - 1 : 0;
        }
    });
}

pk_hip_status pk_hip_synth_weight(pk_hip_ctx* ctx, uint32_t type, uint64_t in, uint64_t out,
                                  uint32_t n_experts, uint64_t key, uint32_t kind,
                                  pk_hip_weight** out_w, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!out_w) throw ArgError("output handle is required");
        const uint32_t be = block_elements(type), bb = block_bytes(type);
        if (be == 0) throw Unsupported("GGUF type has no HIP kernel");
        if (in == 0 || out == 0 || in % be) throw ArgError("invalid GGUF matrix dimensions");
        const bool kq = kind == 1 && (type == 12 || type == 13), q6 = kind == 2 && type == 14;
        const bool f32 = (kind == 3 || kind == 4) && type == 0;
        if (!(kind == 0 || kq || q6 || f32)) throw ArgError("synthetic recipe does not match the type");
        const uint64_t nbytes = in / be * bb * out * (n_experts ? n_experts : 1);
        std::lock_guard lock(ctx->mutex);
        pk_hip_weight* w = make_weight(ctx, type, in, out, n_experts, nbytes);
        // planar types: generated in GGUF form in a staging buffer, then moved
        DeviceBuffer<uint8_t> stage;
        try {
            uint8_t* dst = w->dptr;
            if (pk::planar_type(type)) {
                stage.ensure(nbytes);
                dst = stage.ptr;
            }
            check(pk::launch_synth_fill(dst, nbytes, key, kind, bb, ctx->stream), "synthetic weights");
            if (pk::planar_type(type)) fill_from_device(ctx, w, dst);
            check(hipStreamSynchronize(ctx->stream), "synthetic weights");
        } catch (...) {
            (void)hipStreamSynchronize(ctx->stream);
            stage.release();
            (void)hipFree(w->dptr);
            delete w;
            throw;
        }
        stage.release();
        ctx->stats.resident_bytes += nbytes;
        ++ctx->live_weights;
        *out_w = w;
    });
}

pk_hip_status pk_hip_dequantize_rows(pk_hip_ctx* ctx, const pk_hip_weight* w, uint32_t expert,
                                     uint64_t first_row, uint32_t rows, float* out, char* err,
                                     size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!w || !out) throw ArgError("weight and output are required");
        if (w->ctx != ctx) throw ArgError("weight handle does not belong to this context");
        if (rows == 0) return;
        if (first_row > w->out || rows > w->out - first_row) throw ArgError("rows out of range");
        uint64_t offset = 0;
        if (expert != UINT32_MAX) {
            if (w->n_experts == 0 || expert >= w->n_experts) throw ArgError("expert index out of range");
            offset = static_cast<uint64_t>(expert) * w->slice_pitch;
        } else if (w->n_experts) {
            throw ArgError("an expert tensor needs an expert index");
        }
        if (w->in > 0xffffffffull || !pk::dequant_rows_supported(w->type, static_cast<uint32_t>(w->in)))
            throw Unsupported("row decoding not covered for this type/width");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        const size_t n = static_cast<size_t>(rows) * w->in;
        ctx->y.ensure(n);
        launch_checked(pk::launch_dequant_rows(w->type, w->dptr + offset, w->out,
                                               static_cast<uint32_t>(w->in), first_row, rows,
                                               ctx->y.ptr, ctx->stream),
                       "row decode launch");
        check(hipMemcpyAsync(out, ctx->y.ptr, n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
              "copy rows");
        check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    });
}

pk_hip_status pk_hip_rmsnorm(pk_hip_ctx* ctx, const float* x, const float* w, uint32_t rows,
                             uint32_t n, float eps, float* out, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!x || !w || !out) throw ArgError("input, weight and output are required");
        if (rows == 0) return;
        if (n == 0 || n > pk::kMaxRefWidth) throw ArgError("row width must be between 1 and 8192");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        const size_t total = static_cast<size_t>(rows) * n;
        DeviceBuffer<float> dx, dw;
        try {
            dx.ensure(total);
            dw.ensure(n);
            check(hipMemcpyAsync(dx.ptr, x, total * sizeof(float), hipMemcpyHostToDevice, ctx->stream),
                  "copy rows");
            check(hipMemcpyAsync(dw.ptr, w, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream),
                  "copy weight");
            launch_checked(pk::launch_ref_rmsnorm(dx.ptr, pk::RefResidual{nullptr, nullptr, nullptr, 0},
                                                  dw.ptr, dx.ptr, n, rows, eps, ctx->stream),
                           "rmsnorm launch");
            check(hipMemcpyAsync(out, dx.ptr, total * sizeof(float), hipMemcpyDeviceToHost, ctx->stream),
                  "copy output");
            check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        } catch (...) {
            (void)hipStreamSynchronize(ctx->stream);
            dx.release();
            dw.release();
            throw;
        }
        dx.release();
        dw.release();
    });
}

pk_hip_status pk_hip_expf_block_sums(pk_hip_ctx* ctx, const uint32_t* pairs, uint64_t count,
                                     uint32_t first_bits, uint32_t block_size, uint32_t n_blocks,
                                     uint64_t* sums, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!sums || (count && !pairs)) throw ArgError("output and pairs are required");
        if (block_size == 0 || n_blocks == 0) return;
        if (static_cast<uint64_t>(first_bits) + static_cast<uint64_t>(block_size) * n_blocks > (1ull << 32))
            throw ArgError("input bit patterns past 0xffffffff");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        pk::LibmExpf t{nullptr, 0, 0, 0};
        DeviceBuffer<uint32_t> slots;
        DeviceBuffer<unsigned long long> dsums;
        try {
            if (count) {
                std::vector<uint32_t> host;
                t = build_expf_cuckoo(pairs, count, host);
                slots.ensure(host.size());
                check(hipMemcpy(slots.ptr, host.data(), host.size() * 4, hipMemcpyHostToDevice),
                      "copy expf table");
                t.slots = slots.ptr;
            }
            dsums.ensure(n_blocks);
            check(pk::launch_expf_block_sums(t, first_bits, block_size, n_blocks, dsums.ptr,
                                             ctx->stream),
                  "expf launch");
            check(hipMemcpyAsync(sums, dsums.ptr, n_blocks * sizeof(uint64_t), hipMemcpyDeviceToHost,
                                 ctx->stream),
                  "copy sums");
            check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        } catch (...) {
            (void)hipStreamSynchronize(ctx->stream);
            slots.release();
            dsums.release();
            throw;
        }
        slots.release();
        dsums.release();
    });
}

pk_hip_status pk_hip_add_rmsnorm(pk_hip_ctx* ctx, const float* hidden, const float* delta,
                                 const float* w, uint32_t rows, uint32_t n, float eps,
                                 float* hidden_out, float* out, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!hidden || !w || !hidden_out || !out) throw ArgError("hidden, weight and outputs are required");
        if (rows == 0) return;
        if (n == 0) throw ArgError("row width must be non-zero");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        const size_t total = static_cast<size_t>(rows) * n;
        DeviceBuffer<float> buf;
        try {
            // rows of x | delta | out, then w; 16-byte aligned when n % 4 == 0
            buf.ensure(3 * total + n);
            float* dx = buf.ptr;
            float* dd = dx + total;
            float* dout = dd + total;
            float* dw = dout + total;
            check(hipMemcpyAsync(dx, hidden, total * 4, hipMemcpyHostToDevice, ctx->stream), "copy rows");
            if (delta)
                check(hipMemcpyAsync(dd, delta, total * 4, hipMemcpyHostToDevice, ctx->stream), "copy delta");
            check(hipMemcpyAsync(dw, w, n * 4, hipMemcpyHostToDevice, ctx->stream), "copy weight");
            for (uint32_t r = 0; r < rows; ++r) {
                const uint64_t o = uint64_t(r) * n;
                launch_checked(pk::launch_fast_add_rmsnorm(dx + o, delta ? dd + o : nullptr, dw, dout + o,
                                                           n, eps, ctx->stream),
                               "add_rmsnorm launch");
            }
            check(hipMemcpyAsync(hidden_out, dx, total * 4, hipMemcpyDeviceToHost, ctx->stream), "copy hidden");
            check(hipMemcpyAsync(out, dout, total * 4, hipMemcpyDeviceToHost, ctx->stream), "copy output");
            check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        } catch (...) {
            (void)hipStreamSynchronize(ctx->stream);
            buf.release();
            throw;
        }
        buf.release();
    });
}

pk_hip_status pk_hip_matvec_add_rmsnorm(pk_hip_ctx* ctx, const pk_hip_weight* w, const float* hidden,
                                        const float* delta, const float* norm_w, float eps,
                                        float* hidden_out, float* y, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!w || !hidden || !norm_w || !hidden_out || !y)
            throw ArgError("weight, hidden, norm weight and outputs are required");
        if (w->n_experts) throw ArgError("not a plain matrix");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        const size_t n = w->in;
        DeviceBuffer<float> buf;
        try {
            // hidden | delta | norm weight | hidden_out, 16-byte aligned when n % 4 == 0
            buf.ensure(4 * n);
            float* dh = buf.ptr;
            float* dd = dh + n;
            float* dw = dd + n;
            float* dho = dw + n;
            ctx->y.ensure(w->out);
            check(hipMemcpyAsync(dh, hidden, n * 4, hipMemcpyHostToDevice, ctx->stream), "copy hidden");
            if (delta)
                check(hipMemcpyAsync(dd, delta, n * 4, hipMemcpyHostToDevice, ctx->stream), "copy delta");
            check(hipMemcpyAsync(dw, norm_w, n * 4, hipMemcpyHostToDevice, ctx->stream), "copy weight");
            const pk::MatvecNorm nm{delta ? dd : nullptr, dw, dho, eps};
            const hipError_t e = pk::launch_matvec_norm(w->type, w->dptr, static_cast<uint32_t>(w->out),
                                                        static_cast<uint32_t>(n), dh, nm, ctx->y.ptr,
                                                        ctx->stream);
            if (e == hipErrorNotSupported)
                throw Unsupported("type/width not covered by the one-launch norm + matvec kernel");
            launch_checked(e, "matvec_add_rmsnorm launch");
            check(hipMemcpyAsync(hidden_out, dho, n * 4, hipMemcpyDeviceToHost, ctx->stream), "copy hidden");
            check(hipMemcpyAsync(y, ctx->y.ptr, w->out * 4, hipMemcpyDeviceToHost, ctx->stream), "copy output");
            check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        } catch (...) {
            (void)hipStreamSynchronize(ctx->stream);
            buf.release();
            throw;
        }
        buf.release();
    });
}

pk_hip_status pk_hip_attention_steps(pk_hip_ctx* ctx, const pk_hip_attention_config* cfg,
                                     const float* q_norm, const float* k_norm, uint32_t steps,
                                     const float* q, const float* k, const float* v, float* out,
                                     char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!cfg || !q_norm || !k_norm || !q || !k || !v || !out)
            throw ArgError("config, norms, projections and output are required");
        const pk_hip_attention_config& c = *cfg;
        if (steps == 0) return;
        if (c.heads == 0 || c.kv_heads == 0 || c.heads % c.kv_heads || c.capacity == 0)
            throw ArgError("invalid head counts or KV window");
        if (!(c.rms_eps > 0.0f) || !(c.rope_theta > 0.0f)) throw ArgError("invalid norm epsilon or RoPE base");
        if (!pk::ref_attention_supported(c.head_dim, c.capacity))
            throw Unsupported("attention covers head_dim 64/128/256 and windows whose scores fit LDS");
        if (c.reference_order && c.libm_expf_count && !c.libm_expf_pairs)
            throw ArgError("libm_expf_pairs: missing table");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        const uint64_t qd = uint64_t(c.heads) * c.head_dim, kd = uint64_t(c.kv_heads) * c.head_dim;
        const std::vector<float> table = rope_table_host(steps, c.head_dim, c.rope_theta);
        std::vector<uint32_t> state(4ull * steps, 0u);
        for (uint32_t t = 0; t < steps; ++t) state[4ull * t] = t;
        DeviceBuffer<float> fbuf;
        DeviceBuffer<uint32_t> sbuf, slots;
        DeviceBuffer<uint16_t> kv;
        try {
            const uint64_t nf = 2 * steps * qd + 2 * steps * kd + table.size() + 2ull * c.head_dim;
            fbuf.ensure(nf);
            float* dq = fbuf.ptr;
            float* dk = dq + steps * qd;
            float* dv = dk + steps * kd;
            float* datt = dv + steps * kd;
            float* drope = datt + steps * qd;
            float* dnorm = drope + table.size();
            sbuf.ensure(state.size());
            kv.ensure(2ull * c.capacity * kd);
            check(hipMemcpyAsync(dq, q, steps * qd * 4, hipMemcpyHostToDevice, ctx->stream), "copy q");
            check(hipMemcpyAsync(dk, k, steps * kd * 4, hipMemcpyHostToDevice, ctx->stream), "copy k");
            check(hipMemcpyAsync(dv, v, steps * kd * 4, hipMemcpyHostToDevice, ctx->stream), "copy v");
            check(hipMemcpyAsync(drope, table.data(), table.size() * 4, hipMemcpyHostToDevice, ctx->stream),
                  "copy RoPE table");
            check(hipMemcpyAsync(dnorm, q_norm, c.head_dim * 4, hipMemcpyHostToDevice, ctx->stream), "copy q_norm");
            check(hipMemcpyAsync(dnorm + c.head_dim, k_norm, c.head_dim * 4, hipMemcpyHostToDevice, ctx->stream),
                  "copy k_norm");
            check(hipMemcpyAsync(sbuf.ptr, state.data(), state.size() * 4, hipMemcpyHostToDevice, ctx->stream),
                  "copy positions");
            pk::ModelArgs a{};
            a.heads = c.heads;
            a.kv_heads = c.kv_heads;
            a.head_dim = c.head_dim;
            a.capacity = c.capacity;
            a.rms_eps = c.rms_eps;
            a.rope_theta = c.rope_theta;
            a.attn_scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));  // KvCache::attend default
            a.rope_table = drope;
            a.exact = c.reference_order ? 1u : 0u;
            if (c.reference_order && c.libm_expf_count) {
                std::vector<uint32_t> host;
                a.expf = build_expf_cuckoo(c.libm_expf_pairs, c.libm_expf_count, host);
                slots.ensure(host.size());
                check(hipMemcpyAsync(slots.ptr, host.data(), host.size() * 4, hipMemcpyHostToDevice,
                                     ctx->stream),
                      "copy expf table");
                a.expf.slots = slots.ptr;
            }
            pk::ModelLayer L{};
            L.q_norm = dnorm;
            L.k_norm = dnorm + c.head_dim;
            L.kcache = kv.ptr;
            L.vcache = kv.ptr + uint64_t(c.capacity) * kd;
            for (uint32_t t = 0; t < steps; ++t) {
                a.state = sbuf.ptr + 4ull * t;
                a.q = dq + t * qd;
                a.k = dk + t * kd;
                a.v = dv + t * kd;
                a.att = datt + t * qd;
                launch_checked(c.reference_order ? pk::launch_ref_attention(a, L, ctx->stream)
                                                 : pk::launch_fast_attention(a, L, ctx->stream),
                               "attention launch");
            }
            check(hipMemcpyAsync(out, datt, steps * qd * 4, hipMemcpyDeviceToHost, ctx->stream), "copy output");
            check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        } catch (...) {
            (void)hipStreamSynchronize(ctx->stream);
            fbuf.release();
            sbuf.release();
            slots.release();
            kv.release();
            throw;
        }
        fbuf.release();
        sbuf.release();
        slots.release();
        kv.release();
    });
}

pk_hip_status pk_hip_read_floor_async(pk_hip_ctx* ctx, const void* src, uint64_t bytes,
                                      uint32_t* sink, void* stream, char* err, size_t cap) {
    return guarded(ctx, err, cap, [&] {
        require_usable(ctx);
        if (!src || !sink) throw ArgError("source and sink are required");
        if (bytes == 0 || bytes % 16u || (reinterpret_cast<uintptr_t>(src) & 15u))
            throw ArgError("the read covers whole 16-byte pieces of a 16-byte aligned source");
        std::lock_guard lock(ctx->mutex);
        ctx->set_device();
        launch_checked(pk::launch_read_floor(static_cast<const uint8_t*>(src), bytes, sink,
                                             static_cast<hipStream_t>(stream)),
                       "read floor launch");
    });
}

pk_hip_status pk_hip_get_stats(const pk_hip_ctx* ctx, pk_hip_stats* out) {
    if (!ctx || !out) return PK_HIP_STATUS_INVALID_ARGUMENT;
    std::lock_guard lock(ctx->mutex);
    *out = ctx->stats;
    uint32_t words[4] = {};
    if (hipSetDevice(ctx->device) == hipSuccess &&
        hipStreamSynchronize(ctx->stream) == hipSuccess &&
        hipMemcpy(words, ctx->words.ptr + 1, sizeof(words), hipMemcpyDeviceToHost) == hipSuccess) {
        out->router_fallbacks = words[1];
        out->router_candidates = words[2];
    }
    return PK_HIP_STATUS_OK;
}

pk_hip_status pk_hip_device_name(const pk_hip_ctx* ctx, char* buf, size_t cap) {
    if (!ctx || !buf || cap == 0) return PK_HIP_STATUS_INVALID_ARGUMENT;
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, ctx->device) != hipSuccess) {
        set_error(buf, cap, "hipGetDeviceProperties failed");
        return PK_HIP_STATUS_RUNTIME_ERROR;
    }
    const std::string name = prop.name[0] ? std::string(prop.name)
                                          : "HIP device " + std::to_string(ctx->device);
    const std::string text = name + " (" + prop.gcnArchName + ", " +
                             std::to_string(prop.multiProcessorCount) + " CUs, " +
                             std::to_string(prop.totalGlobalMem >> 30) + " GiB)";
    set_error(buf, cap, text.c_str());
    return text.size() < cap ? PK_HIP_STATUS_OK : PK_HIP_STATUS_BUFFER_TOO_SMALL;
}

pk_hip_status pk_hip_set_kernel_timing(pk_hip_ctx* ctx, int enabled) {
    if (!ctx) return PK_HIP_STATUS_INVALID_ARGUMENT;
    std::lock_guard lock(ctx->mutex);
    ctx->time_kernels = enabled != 0;
    return PK_HIP_STATUS_OK;
}

void pk_hip_reset_stats(pk_hip_ctx* ctx) {
    if (!ctx) return;
    std::lock_guard lock(ctx->mutex);
    const uint64_t resident = ctx->stats.resident_bytes, uploaded = ctx->stats.uploaded_bytes;
    ctx->stats = pk_hip_stats{};
    ctx->stats.resident_bytes = resident;
    ctx->stats.uploaded_bytes = uploaded;
    // device-side router counters (status words 1 and 2); the error word stays
    if (hipSetDevice(ctx->device) == hipSuccess &&
        hipStreamSynchronize(ctx->stream) == hipSuccess) {
        (void)hipMemset(status_words(ctx) + 1, 0, 2 * sizeof(uint32_t));
    }
}

}  // extern "C"
