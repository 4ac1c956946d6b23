// moe.hip -- single-token routed-MoE layer on gfx950.
//
// Three launches replace the MoE block of the reference runner
// (src/qwen3_moe_runner.cpp:643-692) and its route_experts (:267-305):
//
//  1. k_router: one workgroup per expert row computes the router logit's
//     exact value S (FP64 sum of the FP32 products the CPU forms) and a
//     rigorous bound B on how far the CPU's serial, unfused FP32 sum
//     (src/linear.cpp:26-30, src/simd_kernels.hpp:22) can be from S:
//         |serial - S| <= u * sum_i |T_i| / (1 - n u),  T_i = exact prefix sums.
//  2. k_gate_up: wave 0 of every workgroup ranks the experts by S and shares
//     the result through LDS.  When the intervals [S-B, S+B] prove the
//     top-k set and order, that ranking is the CPU's; otherwise the
//     workgroup recomputes every expert that could still enter the top-k
//     with the CPU's exact serial FP32 recurrence and ranks those bit-exact
//     logits.  Workgroup 0 writes ids and route weights (FP64 exp, FP32
//     probabilities, FP32 renormalisation, as route_experts).  Every (route,
//     ffn row) pair then dots the gate and up rows of the selected expert
//     with the register-resident input and stores the SwiGLU activation
//     g / (1 + expf(-g)) * u (:682-684).
//  3. k_down: a workgroup of top_k waves computes one down-row dot per route
//     and combines them in route order, y = ((0 + p0*o0) + p1*o1) + ...
//     (:688-690), deterministically and without atomics.
//
// Ranking lives in every gate/up workgroup because on this GPU any handoff
// between workgroups of one launch costs several dependent memory round
// trips (a release fence writes back the whole L2; coherent stores, counter
// atomics and polls each cost about a microsecond), more than the kernel
// boundary it would save.  Every wave issues all its loads before it consumes
// any: a load inside a branch, or behind a use, waits for every load issued
// before it.
#include <math.h>

#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

constexpr uint32_t kMaxExperts = 256;
constexpr uint32_t kRouterThreads = 256;
constexpr uint32_t kMaxTopK = 8;      // routes per token: waves of the down/combine workgroup
constexpr uint32_t kGateUpPasses = 2;  // row passes whose loads a gate/up wave keeps in flight
constexpr uint32_t kDownPasses = 2;    // row passes per down workgroup

// Status words (MoeDecodeArgs::status).  ST_ERROR: 1 = non-finite router
// logits; it stays set until the host reads and clears it.
enum : uint32_t { ST_ERROR = 0, ST_FALLBACKS = 1, ST_CANDIDATES = 2 };

// route_experts' sorted-insertion order: larger logit first, then smaller id.
__device__ __forceinline__ bool key_before(double av, uint32_t aid, double bv, uint32_t bid) {
    return av > bv || (av == bv && aid < bid);
}

// Block-wide sum/max over the workgroup (DPP inside each wave, LDS across).
template <bool MAX>
__device__ __forceinline__ double block_reduce_d(double v, double* red) {
    v = lane63(MAX ? group_max<64>(v) : group_sum<64>(v));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = red[0];
    for (uint32_t w = 1; w < (blockDim.x >> 6); ++w) r = MAX ? fmax(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
}

// The CPU's router logit, bit for bit: s = fl(s + fl(w_i * x_i)), i ascending,
// then linear()'s bias-free 0.0F + dot (src/linear.cpp:203-204).  Two register
// buffers of 32 weights ping-pong so loads run ahead of the dependent add
// chain (hidden is a multiple of 256).
__device__ __forceinline__ void serial_add32(float& s, const float4 (&w)[8], const float* xv) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        s = __fadd_rn(s, __fmul_rn(w[j].x, xv[4 * j + 0]));
        s = __fadd_rn(s, __fmul_rn(w[j].y, xv[4 * j + 1]));
        s = __fadd_rn(s, __fmul_rn(w[j].z, xv[4 * j + 2]));
        s = __fadd_rn(s, __fmul_rn(w[j].w, xv[4 * j + 3]));
    }
}

__device__ __forceinline__ float serial_logit(const float* __restrict__ w,
                                              const float* __restrict__ xs, uint32_t hidden) {
    float s = 0.0f;
    float4 a[8], b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = *reinterpret_cast<const float4*>(w + 4 * j);
    for (uint32_t i = 0; i < hidden; i += 64) {
#pragma unroll
        for (int j = 0; j < 8; ++j) b[j] = *reinterpret_cast<const float4*>(w + i + 32 + 4 * j);
        serial_add32(s, a, xs + i);
        const uint32_t next = i + 64 < hidden ? i + 64 : i;  // last pair: harmless reload
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = *reinterpret_cast<const float4*>(w + next + 4 * j);
        serial_add32(s, b, xs + i + 32);
    }
    return __fadd_rn(0.0f, s);
}

// Ranks of all experts by key_before over v[0..E), two threads per expert
// (E <= blockDim/2) or one; selected ids in rank order land in sel[0..K).
__device__ __forceinline__ void rank_select(const double* __restrict__ v, uint32_t E, uint32_t K,
                                            uint32_t* __restrict__ rank,
                                            uint32_t* __restrict__ sel) {
    const uint32_t t = threadIdx.x;
    const bool paired = E <= blockDim.x / 2;
    const uint32_t c = paired ? t >> 1 : t;
    uint32_t cnt = 0;
    if (c < E) {
        const double vc = v[c];
        const uint32_t half = (E + 1) / 2;
        const uint32_t j0 = paired ? (t & 1u) * half : 0u;
        const uint32_t j1 = paired ? ((t & 1u) ? E : half) : E;
        for (uint32_t j = j0; j < j1; ++j) cnt += key_before(v[j], j, vc, c) ? 1u : 0u;
    }
    if (paired) cnt += static_cast<uint32_t>(__shfl_xor(static_cast<int>(cnt), 1, 64));
    if (c < E && (!paired || (t & 1u) == 0u)) {
        rank[c] = cnt;
        if (cnt < K) sel[cnt] = c;
    }
    __syncthreads();
}

// Order-preserving 32-bit key of an FP32 value.
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_keep_u(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
        static_cast<int>(v), static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_keep_u<0xb1>(v));
    v = max(v, dpp_keep_u<0x4e>(v));
    v = max(v, dpp_keep_u<0x141>(v));
    v = max(v, dpp_keep_u<0x140>(v));
    v = max(v, dpp_keep_u<0x142, 0xa>(v));
    v = max(v, dpp_keep_u<0x143, 0xc>(v));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

__device__ __forceinline__ double readlane_d(double v, uint32_t lane) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __builtin_amdgcn_readlane(p.x, static_cast<int>(lane));
    r.y = __builtin_amdgcn_readlane(p.y, static_cast<int>(lane));
    return __builtin_bit_cast(double, r);
}

// Experts sit in the lane/slot layout e = lane + 64 * slot: NS slots per lane
// cover up to 64 * NS experts.
constexpr int slots_for(uint32_t experts) { return experts <= 64 ? 1 : experts <= 128 ? 2 : 4; }

// Expert e's entry (e uniform) of a per-lane slot array.
template <int NS>
__device__ __forceinline__ double slot_at(const double (&v)[NS], uint32_t e) {
    double x = v[0];
#pragma unroll
    for (int m = 1; m < NS; ++m) x = (e >> 6) == static_cast<uint32_t>(m) ? v[m] : x;
    return readlane_d(x, e & 63u);
}
template <int NS>
__device__ __forceinline__ float slot_at(const float (&v)[NS], uint32_t e) {
    float x = v[0];
#pragma unroll
    for (int m = 1; m < NS; ++m) x = (e >> 6) == static_cast<uint32_t>(m) ? v[m] : x;
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x),
                                                               static_cast<int>(e & 63u)));
}

// Routes as one wave computes them, without LDS or barriers.
template <int NS>
struct WaveRoutes {
    uint32_t sel[kMaxTopK];
    float logit[NS];  // FP32 of S for experts lane + 64 * m (-inf past n_experts)
    bool certified;
    bool finite;
    double lo_min_sel;
};

// The routing data of the experts lane + 64 * m, loaded before anything
// uses it (absent experts re-read expert 0): a load inside a branch would
// wait for every load issued before it.
template <int NS>
struct RouteData {
    double S[NS], B[NS];
};

template <int NS>
__device__ __forceinline__ RouteData<NS> load_route_data(const MoeDecodeArgs& a) {
    const uint32_t lane = threadIdx.x & 63u, E = a.n_experts;
    RouteData<NS> d;
#pragma unroll
    for (int m = 0; m < NS; ++m) {
        const uint32_t e = lane + 64u * m;
        d.S[m] = a.row_sum[e < E ? e : 0u];
        d.B[m] = a.row_bound[e < E ? e : 0u];
    }
    return d;
}

// Top-k by (S desc, id asc) using 32-bit keys (FP32 value with its low byte
// replaced by 255 - id).  The key only proposes an order: certification
// below checks it against the exact intervals [S - B, S + B], so an ordering
// the truncated key gets wrong is never certified and goes to the exact
// path.  Branch-free: always kMaxTopK selection rounds (ranks past top_k
// only tighten the check), each taking the winner's interval by readlane.
template <int NS>
__device__ __forceinline__ WaveRoutes<NS> wave_route(const MoeDecodeArgs& a, const RouteData<NS>& d) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t E = a.n_experts, K = a.top_k;
    uint32_t key[NS];
    double lo[NS], hi[NS];
    bool fin = true;
    WaveRoutes<NS> w;
#pragma unroll
    for (int m = 0; m < NS; ++m) {
        const uint32_t e = lane + 64u * m;
        const bool present = e < E;
        const float f = static_cast<float>(d.S[m]);
        fin = fin && (!present || isfinite(f));
        key[m] = present ? (order_key(f) & ~0xffu) | (255u - e) : 0u;
        lo[m] = d.S[m] - d.B[m];
        hi[m] = d.S[m] + d.B[m];
        w.logit[m] = present ? f : -INFINITY;
    }
    w.finite = __all(fin);
    double lo_r[kMaxTopK], hi_r[kMaxTopK];
#pragma unroll
    for (uint32_t r = 0; r < kMaxTopK; ++r) {
        uint32_t mk = key[0];
#pragma unroll
        for (int m = 1; m < NS; ++m) mk = max(mk, key[m]);
        const uint32_t best = wave_max_u32(mk);
        const uint32_t e = 255u - (best & 0xffu);
        w.sel[r] = e;
        const bool present = best != 0u;  // fewer than kMaxTopK experts
        lo_r[r] = present ? slot_at<NS>(lo, e) : -INFINITY;
        hi_r[r] = present ? slot_at<NS>(hi, e) : -INFINITY;
#pragma unroll
        for (int m = 0; m < NS; ++m) key[m] = key[m] == best ? 0u : key[m];
    }
    // route r < top_k is certain when its lower bound clears the upper bound
    // of everything ranked after it
    double after = -INFINITY, lmin = INFINITY;
    bool ok = true;
#pragma unroll
    for (int r = kMaxTopK - 1; r >= 0; --r) {
        const bool routed = static_cast<uint32_t>(r) < K;
        ok = ok && (!routed || lo_r[r] > after);
        lmin = routed ? fmin(lmin, lo_r[r]) : lmin;
        after = fmax(after, hi_r[r]);
    }
    // ... including every expert outside the first kMaxTopK ranks
    bool reach = false;
#pragma unroll
    for (int m = 0; m < NS; ++m) reach = reach || (key[m] != 0u && hi[m] >= lmin);
    w.certified = ok && !__any(reach);
    w.lo_min_sel = lmin;
    return w;
}

// Exact routing of an uncertified token, by the whole workgroup (rare).
struct FallbackShared {
    double logit[kMaxExperts];
    uint32_t rank[kMaxExperts];
    uint32_t sel[kMaxTopK];
    uint32_t bad;  // a non-finite exact logit
};

__device__ __forceinline__ void exact_routes(const MoeDecodeArgs& a, double lo_min_sel,
                                             const float* xs, FallbackShared& fb, bool count) {
    const uint32_t t = threadIdx.x, E = a.n_experts;
    if (t < E) {
        const double s = a.row_sum[t], b = a.row_bound[t];
        // An expert with hi < lo_min_sel is below k certain experts; every other
        // expert gets its exact CPU logit.  FP32 rounding of S keeps the rest
        // below lo_min_sel (|fl(S) - S| <= u|S| <= bound).
        if (!(s + b < lo_min_sel)) {
            fb.logit[t] = static_cast<double>(
                serial_logit(a.router + static_cast<uint64_t>(t) * a.hidden, xs, a.hidden));
            if (count) atomicAdd(a.status + ST_CANDIDATES, 1u);
        } else {
            fb.logit[t] = static_cast<double>(static_cast<float>(s));
        }
    }
    if (t == 0 && count) atomicAdd(a.status + ST_FALLBACKS, 1u);
    if (t == 0) fb.bad = 0u;
    __syncthreads();
    // route_experts throws on any non-finite logit (src/qwen3_moe_runner.cpp:270-276)
    if (t < E && !isfinite(fb.logit[t])) fb.bad = 1u;
    __syncthreads();
    rank_select(fb.logit, E, a.top_k, fb.rank, fb.sel);
}

// Wave 0 of gate/up workgroup 0: route weights as route_experts (FP64
// softmax over all experts, FP32 probabilities, FP32 renormalisation,
// optional scale), written with the ids.  l[m] is the FP32 logit the ranking
// used for expert lane + 64 * m (unused slots: -inf).
template <int NS>
__device__ __forceinline__ void write_routes(const MoeDecodeArgs& a, const uint32_t (&sel)[kMaxTopK],
                                             const float (&l)[NS]) {
    const uint32_t lane = threadIdx.x & 63u, K = a.top_k;
    const float mxf = slot_at<NS>(l, sel[0]);
    double ex = 0.0;
#pragma unroll
    for (int m = 0; m < NS; ++m)
        if (lane + 64u * m < a.n_experts) ex += exp(static_cast<double>(l[m] - mxf));
    const double denom = lane63(group_sum<64>(ex));
    float mine = mxf;  // logit of route `lane`
    uint32_t my_id = 0u;
#pragma unroll
    for (uint32_t r = 0; r < kMaxTopK; ++r) {
        if (r < K) {
            const float v = slot_at<NS>(l, sel[r]);
            if (lane == r) {
                mine = v;
                my_id = sel[r];
            }
        }
    }
    float p = 0.0f;
    if (lane < K) p = static_cast<float>(exp(static_cast<double>(mine - mxf)) / denom);
    float selected_sum = 0.0f;
    for (uint32_t r = 0; r < K; ++r)
        selected_sum = __fadd_rn(selected_sum, __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                                        __builtin_bit_cast(int, p),
                                                                        static_cast<int>(r))));
    if (lane < K) {
        float q = a.normalize ? p / selected_sum : p;
        if (a.scale != 1.0f) q = __fmul_rn(q, a.scale);
        a.ids[lane] = my_id;
        a.probs[lane] = q;
    }
}

// ---------------------------------------------------------------------------
// 1. Router: exact sum and serial-error bound of one expert row per workgroup.

template <int C>  // consecutive products per thread: hidden = 256 * C
__global__ __launch_bounds__(kRouterThreads) void k_router(MoeDecodeArgs a) {
    __shared__ double wtot[kRouterThreads / 64];
    __shared__ double red[kRouterThreads / 64];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t e = blockIdx.x;
    const float* w = a.router + static_cast<uint64_t>(e) * a.hidden + t * C;
    const float* xx = a.x + t * C;
    static_assert(C % 2 == 0, "router rows split into pairs of products per thread");
    float p[C];
    if constexpr (C % 4 == 0) {
#pragma unroll
        for (int i = 0; i < C; i += 4) {
            const float4 wv = *reinterpret_cast<const float4*>(w + i);
            const float4 xv = *reinterpret_cast<const float4*>(xx + i);
            p[i + 0] = __fmul_rn(wv.x, xv.x);  // the CPU's rounded products, exactly
            p[i + 1] = __fmul_rn(wv.y, xv.y);
            p[i + 2] = __fmul_rn(wv.z, xv.z);
            p[i + 3] = __fmul_rn(wv.w, xv.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < C; i += 2) {
            const float2 wv = *reinterpret_cast<const float2*>(w + i);
            const float2 xv = *reinterpret_cast<const float2*>(xx + i);
            p[i + 0] = __fmul_rn(wv.x, xv.x);
            p[i + 1] = __fmul_rn(wv.y, xv.y);
        }
    }
    double local = 0.0, abs_p = 0.0;
#pragma unroll
    for (int i = 0; i < C; ++i) {
        local += static_cast<double>(p[i]);
        abs_p += fabs(static_cast<double>(p[i]));
    }
    // exclusive prefix of the thread totals: wave scan + wave offsets
    const double incl = wave_inclusive_scan(local);
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    double off = incl - local;
    for (uint32_t v = 0; v < wave; ++v) off += wtot[v];
    double prefix_abs = 0.0;
#pragma unroll
    for (int i = 0; i < C; ++i) {
        off += static_cast<double>(p[i]);
        prefix_abs += fabs(off);
    }
    double total = 0.0;
    for (uint32_t v = 0; v < (kRouterThreads >> 6); ++v) total += wtot[v];
    prefix_abs = block_reduce_d<false>(prefix_abs, red);
    abs_p = block_reduce_d<false>(abs_p, red);
    if (t == 0) {
        // u = 2^-24.  (1 + 2^-10) >= 1/(1 - n u) for n <= 2^13 and also covers
        // the FP64 rounding of the prefix sums; abs_p * 2^-40 covers S itself.
        double bound = prefix_abs * 0x1p-24 * (1.0 + 0x1p-10) + abs_p * 0x1p-40;
        if (!(abs_p < 1.0e36)) bound = INFINITY;  // near FP32 overflow: always recompute
        a.row_sum[e] = total;
        a.row_bound[e] = bound;
    }
}

// ---------------------------------------------------------------------------
// 2. Routing + gate/up + SwiGLU.  All (route, row) items share the input x,
// so one unit mapping (and one register copy of x per lane) serves them all.

// Marks a router error (wave 0 of gate/up workgroup 0): route_experts throws
// on non-finite logits (src/qwen3_moe_runner.cpp:270-276).
__device__ __forceinline__ void flag_router_error(const MoeDecodeArgs& a) {
    const uint32_t lane = threadIdx.x & 63u;
    if (lane == 0) atomicOr(a.status + ST_ERROR, 1u);
    if (lane < a.top_k) {
        a.ids[lane] = 0xffffffffu;
        a.probs[lane] = 0.0f;
    }
}

// A workgroup's share of a float vector held in registers: float4 pieces
// i * blockDim + threadIdx, i < kXPieces (hidden <= 4 * 256 * kXPieces).  All
// loads are issued before any is used.
constexpr uint32_t kXPieces = 8;  // hidden <= 8192, the widest router (32 * 256)
struct XRegs {
    float4 v[kXPieces];
};

// Pieces past the end load and store the last piece again (the same values
// as its own thread writes), so neither the loads nor the stores sit in a
// branch: a load sunk into a branch next to its use would wait for every
// load issued before it.
__device__ __forceinline__ uint32_t x_piece(uint32_t i, uint32_t n) {
    const uint32_t k = (i * blockDim.x + threadIdx.x) * 4u;
    return k < n ? k : n - 4u;
}

__device__ __forceinline__ XRegs load_x_regs(const float* x, uint32_t n) {
    XRegs r;
#pragma unroll
    for (uint32_t i = 0; i < kXPieces; ++i)
        r.v[i] = *reinterpret_cast<const float4*>(x + x_piece(i, n));
    return r;
}

__device__ __forceinline__ void store_x_regs(float* xs, const XRegs& r, uint32_t n) {
#pragma unroll
    for (uint32_t i = 0; i < kXPieces; ++i) *reinterpret_cast<float4*>(xs + x_piece(i, n)) = r.v[i];
}

// The ranking wave 0 hands to the workgroup.
struct SharedRoutes {
    uint32_t sel[kMaxTopK];
    uint32_t state;  // 0 certified, 1 needs the exact path, 2 a logit is not finite
    double lo_min_sel;
};

template <int T, int UB, int NU, int NP, int NS>
__global__ __launch_bounds__(256) void k_gate_up(MoeDecodeArgs a, uint32_t units, uint32_t glog2) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [hidden]
    __shared__ FallbackShared fb;
    __shared__ SharedRoutes sr;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const bool first_wave = blockIdx.x == 0 && wave == 0;
    // x and (wave 0) the routing data go out together; x is stored first
    const XRegs xr = load_x_regs(a.x, a.hidden);
    RouteData<NS> rd;
    if (wave == 0) rd = load_route_data<NS>(a);
    store_x_regs(xs, xr, a.hidden);
    WaveRoutes<NS> w;
    if (wave == 0) {
        w = wave_route<NS>(a, rd);
        if (lane == 0) {
#pragma unroll
            for (uint32_t r = 0; r < kMaxTopK; ++r) sr.sel[r] = w.sel[r];
            sr.state = !w.finite ? 2u : w.certified ? 0u : 1u;
            sr.lo_min_sel = w.lo_min_sel;
        }
    }
    __syncthreads();
    const uint32_t state = sr.state;  // uniform
    if (state == 2u) {
        if (first_wave) flag_router_error(a);
        return;
    }
    uint32_t sel[kMaxTopK];
    if (state == 1u) {  // rare: exact serial logits of the candidates
        exact_routes(a, sr.lo_min_sel, xs, fb, blockIdx.x == 0);
        if (fb.bad) {  // uniform
            if (first_wave) flag_router_error(a);
            return;
        }
#pragma unroll
        for (uint32_t r = 0; r < kMaxTopK; ++r) sel[r] = r < a.top_k ? fb.sel[r] : 0u;
        if (first_wave) {
#pragma unroll
            for (int m = 0; m < NS; ++m)
                w.logit[m] = lane + 64u * m < a.n_experts ? static_cast<float>(fb.logit[lane + 64u * m])
                                                          : -INFINITY;
        }
    } else {
#pragma unroll
        for (uint32_t r = 0; r < kMaxTopK; ++r) sel[r] = sr.sel[r];
    }
    if (first_wave) write_routes<NS>(a, sel, w.logit);

    const uint32_t G = 1u << glog2, RPP = 64u >> glog2;
    const uint32_t sub = lane >> glog2, ul = lane & (G - 1u);
    UnitPos pos[NU];
    bool valid[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const uint32_t u = ul + G * k;
        valid[k] = u < units;
        pos[k] = unit_pos<T, UB>(valid[k] ? u : 0u);
    }
    const uint32_t items = a.top_k * a.ffn;
    const uint32_t passes = (items + RPP - 1u) / RPP;
    const uint32_t first = (blockIdx.x * (blockDim.x >> 6) + wave) * NP;

    // Loads are unconditional (items past the end re-read the last item,
    // absent units re-read unit 0, results unused), so no branch splits
    // them and none waits on another.
    UnitRaw<T, UB> rg[NP][NU], ru[NP][NU];
    uint32_t item[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        item[q] = (first + q) * RPP + sub;
        const uint32_t it = item[q] < items ? item[q] : items - 1u;
        const uint32_t route_i = it / a.ffn, row = it % a.ffn;
        uint32_t e = 0u;
#pragma unroll
        for (uint32_t r = 0; r < kMaxTopK; ++r)
            if (route_i == r) e = sel[r];
        const uint8_t* gr = a.gate + static_cast<uint64_t>(e) * a.gate_slice + row * a.gate_row;
        const uint8_t* ur = a.up + static_cast<uint64_t>(e) * a.up_slice + row * a.up_row;
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            unit_load<T, UB>(gr, pos[k], rg[q][k]);
            unit_load<T, UB>(ur, pos[k], ru[q][k]);
        }
    }
    UnitX<T, UB, 1> ux[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) load_unit_x<T, UB, 1>(xs, 0, pos[k], valid[k], ux[k]);

#pragma unroll
    for (int q = 0; q < NP; ++q) {
        const bool live = first + q < passes && item[q] < items;
        float g[1] = {0.0f}, u[1] = {0.0f};
        if (live) {
#pragma unroll
            for (int k = 0; k < NU; ++k) {
                if (valid[k]) {
                    unit_compute<T, UB, 1>(rg[q][k], pos[k], ux[k], g);
                    unit_compute<T, UB, 1>(ru[q][k], pos[k], ux[k], u);
                }
            }
        }
        const float gs = group_sum_dyn(g[0], G);
        const float us = group_sum_dyn(u[0], G);
        if (live && ul == G - 1u) a.act[item[q]] = (gs / (1.0f + expf(-gs))) * us;
    }
}


// ---------------------------------------------------------------------------
// 3. down + combine.  blockDim = 64 * top_k: wave k owns route k; the
// workgroup covers kDownPasses * RPP output rows.

template <int T, int UB, int NU, int kDownPasses>
__global__ __launch_bounds__(64 * kMaxTopK) void k_down(MoeDecodeArgs a, uint32_t units,
                                                         uint32_t glog2) {
    extern __shared__ float part[];  // [top_k][kDownPasses * RPP]
    const uint32_t lane = threadIdx.x & 63u, k = threadIdx.x >> 6;
    const uint32_t G = 1u << glog2, RPP = 64u >> glog2;
    const uint32_t sub = lane >> glog2, ul = lane & (G - 1u);
    uint64_t e = a.ids[k];
    const bool ok = e < a.n_experts;  // router error: ids are marked invalid, output unused
    if (!ok) e = 0;
    UnitPos pos[NU];
    bool valid[NU];
#pragma unroll
    for (int q = 0; q < NU; ++q) {
        const uint32_t u = ul + G * q;
        valid[q] = u < units;
        pos[q] = unit_pos<T, UB>(valid[q] ? u : 0u);
    }
    const uint8_t* base = a.down + e * a.down_slice;
    const uint32_t rows = a.hidden;
    const uint32_t row0 = blockIdx.x * kDownPasses * RPP;
    // unconditional loads (rows past the end re-read the last row, unused)
    UnitRaw<T, UB> raw[kDownPasses][NU];
#pragma unroll
    for (int p = 0; p < kDownPasses; ++p) {
        const uint32_t row = row0 + p * RPP + sub;
        const uint8_t* rp = base + static_cast<uint64_t>(row < rows ? row : rows - 1u) * a.down_row;
#pragma unroll
        for (int q = 0; q < NU; ++q) unit_load<T, UB>(rp, pos[q], raw[p][q]);
    }
    UnitX<T, UB, 1> ux[NU];
    const float* act = a.act + k * a.ffn;
#pragma unroll
    for (int q = 0; q < NU; ++q) load_unit_x<T, UB, 1>(act, 0, pos[q], valid[q], ux[q]);
    const uint32_t RB = kDownPasses * RPP;
#pragma unroll
    for (int p = 0; p < kDownPasses; ++p) {
        const uint32_t row = row0 + p * RPP + sub;
        float acc[1] = {0.0f};
        if (ok && row < rows) {
#pragma unroll
            for (int q = 0; q < NU; ++q)
                if (valid[q]) unit_compute<T, UB, 1>(raw[p][q], pos[q], ux[q], acc);
        }
        const float v = group_sum_dyn(acc[0], G);
        if (ul == G - 1u) part[k * RB + p * RPP + sub] = v;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < RB; i += blockDim.x) {
        const uint32_t orow = row0 + i;
        if (orow < rows) {
            float y = 0.0f;
            for (uint32_t r = 0; r < a.top_k; ++r)
                y = __fadd_rn(y, __fmul_rn(a.probs[r], part[r * RB + i]));
            a.y[orow] = y;
        }
    }
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }
uint32_t log2_ceil(uint32_t v) {
    uint32_t l = 0;
    while ((1u << l) < v) ++l;
    return l;
}

template <int T>
constexpr int moe_ub() { return Fmt<T>::MAXUB < 16 ? Fmt<T>::MAXUB : 16; }

// Units per row and the lane grouping for a row of `in` elements.
template <int T>
bool moe_plan(uint32_t in, uint32_t& units, uint32_t& glog2, uint32_t& nu) {
    constexpr int UB = moe_ub<T>();
    if (in == 0 || in % Fmt<T>::BE) return false;
    units = in / Fmt<T>::BE * (Fmt<T>::PRIM / UB);
    if (units >= 64u) {
        glog2 = 6;
        nu = ceil_div(units, 64u);
    } else {
        glog2 = log2_ceil(units);
        nu = 1;
    }
    return nu <= 2u;
}

template <int T>
hipError_t gate_up_t(const MoeDecodeArgs& a, hipStream_t s) {
    constexpr int UB = moe_ub<T>();
    uint32_t units, glog2, nu;
    if (!moe_plan<T>(a.hidden, units, glog2, nu)) return hipErrorInvalidValue;
    const uint32_t RPP = 64u >> glog2;
    const uint32_t passes = ceil_div(a.top_k * a.ffn, RPP);
    const uint32_t blocks = ceil_div(passes, 4u * kGateUpPasses);
    const size_t lds = a.hidden * sizeof(float);
#define PK_GU(N, NS)                                                                            \
    hipLaunchKernelGGL((k_gate_up<T, UB, N, kGateUpPasses, NS>), dim3(blocks), dim3(256), lds, s, a, \
                       units, glog2)
    const int ns = slots_for(a.n_experts);
    if (nu == 1 && ns == 1) PK_GU(1, 1);
    else if (nu == 1 && ns == 2) PK_GU(1, 2);
    else if (nu == 1 && ns == 4) PK_GU(1, 4);
    else if (nu == 2 && ns == 1) PK_GU(2, 1);
    else if (nu == 2 && ns == 2) PK_GU(2, 2);
    else if (nu == 2 && ns == 4) PK_GU(2, 4);
    else return hipErrorInvalidValue;
#undef PK_GU
    return hipGetLastError();
}

template <int T>
hipError_t down_t(const MoeDecodeArgs& a, hipStream_t s) {
    constexpr int UB = moe_ub<T>();
    uint32_t units, glog2, nu;
    if (!moe_plan<T>(a.ffn, units, glog2, nu)) return hipErrorInvalidValue;
    const uint32_t RPP = 64u >> glog2;
    const uint32_t blocks = ceil_div(a.hidden, kDownPasses * RPP);
    const size_t lds = static_cast<size_t>(a.top_k) * kDownPasses * RPP * sizeof(float);
#define PK_DN(N)                                                                              \
    case N:                                                                                   \
        hipLaunchKernelGGL((k_down<T, UB, N, kDownPasses>), dim3(blocks), dim3(64u * a.top_k), lds, s, a,  \
                           units, glog2);                                                     \
        break;
    switch (nu) { PK_DN(1) PK_DN(2) default: return hipErrorInvalidValue; }
#undef PK_DN
    return hipGetLastError();
}

template <int T>
bool plan_ok(uint32_t in) {
    uint32_t units, glog2, nu;
    return moe_plan<T>(in, units, glog2, nu);
}

bool quant_plan_ok(uint32_t type, uint32_t in) {
    switch (type) {
        case T_Q4_0: return plan_ok<T_Q4_0>(in);
        case T_Q8_0: return plan_ok<T_Q8_0>(in);
        case T_Q4_K: return plan_ok<T_Q4_K>(in);
        case T_Q5_K: return plan_ok<T_Q5_K>(in);
        case T_Q6_K: return plan_ok<T_Q6_K>(in);
        default: return false;
    }
}

bool router_width_ok(uint32_t hidden) {
    if (hidden % kRouterThreads) return false;
    switch (hidden / kRouterThreads) {
        case 2: case 4: case 8: case 12: case 16: case 24: case 32: return true;
        default: return false;
    }
}

}  // namespace

bool moe_decode_supported(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                          uint32_t hidden, uint32_t ffn, uint32_t n_experts, uint32_t top_k) {
    return gate_type == up_type && quant_plan_ok(gate_type, hidden) &&
           quant_plan_ok(down_type, ffn) && n_experts >= 1 && n_experts <= kMaxExperts &&
           top_k >= 1 && top_k <= kMaxTopK && top_k <= n_experts && router_width_ok(hidden);
}

hipError_t launch_moe_router(const MoeDecodeArgs& a, hipStream_t s) {
    switch (a.hidden / kRouterThreads) {
#define PK_RT(C)                                                                                \
    case C:                                                                                     \
        hipLaunchKernelGGL(k_router<C>, dim3(a.n_experts), dim3(kRouterThreads), a.hidden * sizeof(float), s, a); \
        break;
        PK_RT(2) PK_RT(4) PK_RT(8) PK_RT(12) PK_RT(16) PK_RT(24) PK_RT(32)
#undef PK_RT
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(const MoeDecodeArgs& a, hipStream_t s) {
    switch (a.gate_type) {
        case T_Q4_0: return gate_up_t<T_Q4_0>(a, s);
        case T_Q8_0: return gate_up_t<T_Q8_0>(a, s);
        case T_Q4_K: return gate_up_t<T_Q4_K>(a, s);
        case T_Q5_K: return gate_up_t<T_Q5_K>(a, s);
        case T_Q6_K: return gate_up_t<T_Q6_K>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_down(const MoeDecodeArgs& a, hipStream_t s) {
    switch (a.down_type) {
        case T_Q4_0: return down_t<T_Q4_0>(a, s);
        case T_Q8_0: return down_t<T_Q8_0>(a, s);
        case T_Q4_K: return down_t<T_Q4_K>(a, s);
        case T_Q5_K: return down_t<T_Q5_K>(a, s);
        case T_Q6_K: return down_t<T_Q6_K>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_moe_decode(const MoeDecodeArgs& a, hipStream_t s) {
    hipError_t err = launch_moe_router(a, s);
    if (err == hipSuccess) err = launch_moe_gate_up(a, s);
    if (err == hipSuccess) err = launch_moe_down(a, s);
    return err;
}

}  // namespace pk
