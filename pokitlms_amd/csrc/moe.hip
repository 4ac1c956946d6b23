// moe.hip -- single-token routed-MoE layer on gfx950.
//
// Three launches replace the MoE block of the reference runner
// (src/qwen3_moe_runner.cpp:643-692) and its route_experts (:267-305):
//
//  1. k_router: one wave per expert row computes the router logit's
//     exact value S (FP64 sum of the FP32 products the CPU forms) and a
//     rigorous bound B on how far the CPU's serial, unfused FP32 sum
//     (src/linear.cpp:26-30, src/simd_kernels.hpp:22) can be from S:
//         |serial - S| <= u * sum_i |T_i| / (1 - n u),  T_i = exact prefix sums.
//  2. k_gate_up: the four waves of every workgroup rank the experts by S
//     (each expert's rank counted as the number of larger keys) and share
//     the routed ones through LDS.  When the intervals [S-B, S+B] prove the
//     top-k set and order, that ranking is the CPU's; otherwise the
//     workgroup recomputes every expert that could still enter the top-k
//     with the CPU's exact serial FP32 recurrence and ranks those bit-exact
//     logits.  Workgroup 0 writes ids and route weights (FP64 exp, FP32
//     probabilities, FP32 renormalisation, as route_experts).  Every (route,
//     ffn row) pair then dots the gate and up rows of the selected expert
//     with the register-resident input and stores the SwiGLU activation
//     g / (1 + expf(-g)) * u (:682-684; here with the hardware exp2 and
//     reciprocal).
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
#include "route.hpp"

namespace pk {
namespace {

constexpr uint32_t kGateUpPasses = 2;  // row passes whose loads a gate/up wave keeps in flight
constexpr uint32_t kDownPasses = 2;    // row passes per down workgroup

// ---------------------------------------------------------------------------
// 1. Router: exact sum and serial-error bound of one expert row per
// single-wave workgroup (router_wave_sum_bound, the batched prefill router's
// arithmetic, so the same bits).

template <int C>  // hidden = 256 * C: 4 * C consecutive products per lane
__global__ __launch_bounds__(64) void k_router(MoeDecodeArgs a) {
    trace_stamp(a.trace, 0, 0);
    const uint32_t e = blockIdx.x;  // row n_experts: the shared expert's gate (variant 1)
    const uint32_t lane = threadIdx.x;
    const float* row = e < a.n_experts ? a.router + static_cast<uint64_t>(e) * a.hidden : a.shared_router;
    rf32x4 w[C], x[C];
    if constexpr (C <= 16) {
        // through LDS: loaded with consecutive lanes on consecutive float4s
        // (whole cache lines per load), read back lane-contiguous, one float4
        // of padding per C so no two lanes of a read meet in one bank
        __shared__ rf32x4 buf[2][64u * (C + 1u)];
        const rf32x4* wg = reinterpret_cast<const rf32x4*>(row);
        const rf32x4* xg = reinterpret_cast<const rf32x4*>(a.x);
#pragma unroll
        for (uint32_t m = 0; m < C; ++m) {
            w[m] = wg[m * 64u + lane];
            x[m] = xg[m * 64u + lane];
        }
#pragma unroll
        for (uint32_t m = 0; m < C; ++m) {
            const uint32_t g = m * 64u + lane, pos = g + g / C;
            buf[0][pos] = w[m];
            buf[1][pos] = x[m];
        }
        __syncthreads();
#pragma unroll
        for (uint32_t j = 0; j < C; ++j) {
            w[j] = buf[0][lane * (C + 1u) + j];
            x[j] = buf[1][lane * (C + 1u) + j];
        }
    } else {
        router_lane_load<C>(row, lane, w);
        router_lane_load<C>(a.x, lane, x);
        __builtin_amdgcn_sched_barrier(0);  // every load out before the first is waited for
    }
    trace_stamp(a.trace, 0, 1);
    RouterLane<C> r;
    double total, bound;
    router_lane_sums<C>(w, x, r);
    router_wave_sum_bound<C>(r, total, bound);
    if (lane == 0) {
        a.row_sum[e] = total;
        a.row_bound[e] = bound;
    }
    trace_stamp(a.trace, 0, 2);
}

// ---------------------------------------------------------------------------
// 2. Routing + gate/up + SwiGLU.  All (route, row) items share the input x,
// so one unit mapping (and one register copy of x per lane) serves them all.

// x pieces per thread (float4s of a 256-thread workgroup) for the widest
// hidden that NU units per lane cover
template <int T, int UB, int NU>
constexpr uint32_t gate_up_x_pieces() {
    constexpr int per_unit = Fmt<T>::BE * UB / Fmt<T>::PRIM;  // elements per unit
    constexpr int xp = NU * 64 * per_unit / 1024;
    return xp < 1 ? 1u : xp > static_cast<int>(kXPieces) ? kXPieces : static_cast<uint32_t>(xp);
}

// G64: every row on the 64 lanes of a wave (glog2 == 6), so the row sums are
// straight-line DPP code the compiler can interleave.
template <int T, int UB, int NU, int NP, int NS, bool G64, uint32_t XP = gate_up_x_pieces<T, UB, NU>()>
__global__ __launch_bounds__(256) void k_gate_up(MoeDecodeArgs a, uint32_t units, uint32_t glog2) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [hidden]
    __shared__ FallbackShared<128> fb;
    __shared__ SharedRank<NS> sr;
    trace_stamp(a.trace, 1, 0);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const bool first_wave = blockIdx.x == 0 && wave == 0;
    // x and the routing data go out together; x is stored first
    const XRegs<XP> xr = load_x_regs<XP>(a.x, a.hidden);
    const RouteData<NS> rd = load_route_data<NS>(a);
    const RankData<NS> rk = load_rank_data<NS>(a);
    // everything about this wave's items but the experts, while the loads fly
    if constexpr (G64) glog2 = 6u;
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
    const uint32_t items = (a.top_k + a.variant) * a.ffn;  // variant 1: the shared expert last
    const uint32_t passes = (items + RPP - 1u) / RPP;
    const uint32_t first = (blockIdx.x * (blockDim.x >> 6) + wave) * NP;
    const uint32_t nb = a.hidden / Fmt<T>::BE;  // blocks per gate/up row
    const uint64_t nblk = static_cast<uint64_t>(a.ffn) * nb;  // blocks per expert slice
    uint32_t item[NP], route_of[NP];
    uint64_t blk0[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        item[q] = (first + q) * RPP + sub;
        const uint32_t it = item[q] < items ? item[q] : items - 1u;
        route_of[q] = it / a.ffn;
        blk0[q] = static_cast<uint64_t>(it % a.ffn) * nb;
    }
    store_x_regs(xs, xr, a.hidden);
    wg_rank<NS>(a, rd, rk, sr);
    trace_stamp(a.trace, 1, 1);
    __syncthreads();
    WaveRoutes<NS> w = wg_certify<NS>(a, rd, sr);
    trace_stamp(a.trace, 1, 2);
    const uint32_t state = !w.finite ? 2u : w.certified ? 0u : 1u;  // the same in every wave
    if (state == 2u) {
        if (first_wave) flag_router_error(a);
        return;
    }
    uint32_t sel[kMaxTopK];
    if (state == 1u) {  // rare: exact serial logits of the candidates
        exact_routes<4, 128>(a, w.lo_min_sel, xs, fb, blockIdx.x == 0);
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
        for (uint32_t r = 0; r < kMaxTopK; ++r) sel[r] = w.sel[r];
    }
    if (first_wave) write_routes<NS>(a, sel, w.logit);

    // Loads are unconditional (items past the end re-read the last item,
    // absent units re-read unit 0, results unused), so no branch splits
    // them and none waits on another.
    UnitRaw<T, UB> rg[NP][NU], ru[NP][NU];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        uint32_t e = 0u;
#pragma unroll
        for (uint32_t r = 0; r < kMaxTopK; ++r)
            if (route_of[q] == r) e = sel[r];
        const bool shared = route_of[q] >= a.top_k;
        const QRow gr{shared ? a.shared_gate : a.gate + static_cast<uint64_t>(e) * a.gate_slice, nblk, blk0[q]};
        const QRow ur{shared ? a.shared_up : a.up + static_cast<uint64_t>(e) * a.up_slice, nblk, blk0[q]};
#pragma unroll
        for (int k = 0; k < NU; ++k) {
            unit_load<T, UB>(gr, pos[k], rg[q][k]);
            unit_load<T, UB>(ur, pos[k], ru[q][k]);
        }
    }
    trace_stamp(a.trace, 1, 3);
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
        const float gs = G64 ? group_sum<64>(g[0]) : group_sum_dyn(g[0], G);
        const float us = G64 ? group_sum<64>(u[0]) : group_sum_dyn(u[0], G);
        // SwiGLU g / (1 + exp(-g)) * u with the hardware exp2 and reciprocal
        // (a few ulps from the libm form, inside the fast path's tolerance; the
        // reference-order kernels keep the CPU's expf and division)
        if (live && ul == G - 1u)
            a.act[item[q]] = a.variant ? silu(gs) * us : (gs * __builtin_amdgcn_rcpf(1.0f + __expf(-gs))) * us;
    }
    trace_stamp(a.trace, 1, 4);
}


// ---------------------------------------------------------------------------
// 3. down + combine.  blockDim = 64 * (top_k + variant): wave k owns route k
// (variant 1: wave top_k the shared expert); the workgroup covers
// kDownPasses * RPP output rows.

template <int T, int UB, int NU, int kDownPasses, bool SHARED, bool HALVES>
__global__ __launch_bounds__(64 * (kMaxTopK + (SHARED ? 1 : 0))) void k_down(
    uint32_t* ids, float* act_in, const uint8_t* down, uint64_t down_slice, uint32_t ffn,
    uint32_t n_experts, uint32_t units, uint32_t glog2, MoeDecodeArgs a) {
    // The fields the first loads need lead the argument list: they arrive in
    // SGPRs with the waves (kernel-argument preloading), not after a load of
    // the argument block.
    a.ids = ids;
    a.act = act_in;
    a.down = down;
    a.down_slice = down_slice;
    a.ffn = ffn;
    a.n_experts = n_experts;
    extern __shared__ float part[];  // [top_k + variant][kDownPasses * RPP]
    trace_stamp(a.trace, 2, 0);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t k = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar bases
    if constexpr (HALVES) glog2 = 5u;
    const uint32_t G = 1u << glog2, RPP = 64u >> glog2;
    const uint32_t sub = lane >> glog2, ul = lane & (G - 1u);
    const bool shared = SHARED && k >= a.top_k;
    // the route's expert id through the scalar cache (constant address space:
    // written by the previous launch, read-only here)
    using cu32 = const __attribute__((address_space(4))) uint32_t;
    uint64_t e = shared ? 0u : ((cu32*)(a.ids))[k];
    UnitPos pos[NU];
    bool valid[NU];
#pragma unroll
    for (int q = 0; q < NU; ++q) {
        const uint32_t u = ul + G * q;
        valid[q] = u < units;
        pos[q] = unit_pos<T, UB>(valid[q] ? u : 0u);
    }
    // the route's activations first: they do not depend on its expert id, so
    // they are in flight while the id arrives, and they come back before the
    // weights (unconditional loads; absent units are zeroed afterwards)
    const float* act = a.act + k * a.ffn;
    constexpr int XP = x_pieces<T, UB>() / (HALVES ? 2 : 1);
    XRaw<XP> xr[NU];
#pragma unroll
    for (int q = 0; q < NU; ++q) {
        if constexpr (HALVES) load_x_half<T, UB>(act, pos[q], sub, xr[q]);
        else load_x_pieces<T, UB>(act, pos[q], xr[q]);
    }
    __builtin_amdgcn_sched_barrier(0);  // the activation loads out before the id is waited for
    const bool ok = shared || e < a.n_experts;  // router error: ids are invalid, output unused
    if (!ok) e = 0;
    const uint8_t* base = shared ? a.shared_down : a.down + e * a.down_slice;
    const uint32_t rows = a.hidden;
    const uint32_t nb = a.ffn / Fmt<T>::BE;  // blocks per down row
    const uint32_t row0 = blockIdx.x * kDownPasses * RPP;
    // unconditional loads (rows past the end re-read the last row, unused)
    UnitRaw<T, UB> raw[kDownPasses][NU];
#pragma unroll
    for (int p = 0; p < kDownPasses; ++p) {
        const uint32_t row = row0 + p * RPP + sub;
        const QRow qr{base, static_cast<uint64_t>(rows) * nb,
                      static_cast<uint64_t>(row < rows ? row : rows - 1u) * nb};
#pragma unroll
        for (int q = 0; q < NU; ++q) unit_load<T, UB>(qr, pos[q], raw[p][q]);
    }
    trace_stamp(a.trace, 2, 1);
    UnitX<T, UB, 1> ux[NU];
#pragma unroll
    for (int q = 0; q < NU; ++q) {
        if constexpr (HALVES) unit_x_from_halves<T, UB>(xr[q], valid[q], ux[q]);
        else unit_x_from_pieces<T, UB>(xr[q], valid[q], ux[q]);
    }
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
        const float v = HALVES ? group_sum<32>(acc[0]) : group_sum_dyn(acc[0], G);
        if (ul == G - 1u) part[k * RB + p * RPP + sub] = v;
    }
    // variant 1: mixer_output = moe_result + sigmoid(shared gate) * shared output
    // (src/qwen35_runner.cpp:752-761)
    const float shared_scale = SHARED ? sigmoid35(static_cast<float>(a.row_sum[a.n_experts])) : 0.0f;
    trace_stamp(a.trace, 2, 2);
    __syncthreads();
    trace_stamp(a.trace, 2, 3);
    for (uint32_t i = threadIdx.x; i < RB; i += blockDim.x) {
        const uint32_t orow = row0 + i;
        if (orow < rows) {
            float y = 0.0f;
            for (uint32_t r = 0; r < a.top_k; ++r)
                y = __fadd_rn(y, __fmul_rn(a.probs[r], part[r * RB + i]));
            if (SHARED) y = __fadd_rn(y, __fmul_rn(shared_scale, part[a.top_k * RB + i]));
            a.y[orow] = y;
        }
    }
    trace_stamp(a.trace, 2, 4);
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
    const uint32_t passes = ceil_div((a.top_k + a.variant) * a.ffn, RPP);
    const uint32_t blocks = ceil_div(passes, 4u * kGateUpPasses);
    const size_t lds = a.hidden * sizeof(float);
#define PK_GU(N, NS, G64)                                                                        \
    hipLaunchKernelGGL((k_gate_up<T, UB, N, kGateUpPasses, NS, G64>), dim3(blocks), dim3(256), lds, s, \
                       a, units, glog2)
    const int ns = slots_for(a.n_experts);
    const bool g64 = glog2 == 6u;  // always when nu == 2
    if (nu == 1 && ns == 1) {
        if (g64) PK_GU(1, 1, true);
        else PK_GU(1, 1, false);
    } else if (nu == 1 && ns == 2) {
        if (g64) PK_GU(1, 2, true);
        else PK_GU(1, 2, false);
    } else if (nu == 1 && ns == 4) {
        if (g64) PK_GU(1, 4, true);
        else PK_GU(1, 4, false);
    } else if (nu == 2 && ns == 1) PK_GU(2, 1, true);
    else if (nu == 2 && ns == 2) PK_GU(2, 2, true);
    else if (nu == 2 && ns == 4) PK_GU(2, 4, true);
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
    const uint32_t waves = a.top_k + a.variant;
    const size_t lds = static_cast<size_t>(waves) * kDownPasses * RPP * sizeof(float);
#define PK_DN(N, SH, HV)                                                                          \
    hipLaunchKernelGGL((k_down<T, UB, N, kDownPasses, SH, HV>), dim3(blocks), dim3(64u * waves), lds, \
                       s, a.ids, a.act, a.down, a.down_slice, a.ffn, a.n_experts, units, glog2, a)
    const bool halves = glog2 == 5u;  // nu == 1: lanes l and l + 32 hold the same unit
    if (nu == 1 && !a.variant) {
        if (halves) PK_DN(1, false, true);
        else PK_DN(1, false, false);
    } else if (nu == 2 && !a.variant) PK_DN(2, false, false);
    else if (nu == 1) {
        if (halves) PK_DN(1, true, true);
        else PK_DN(1, true, false);
    } else if (nu == 2) PK_DN(2, true, false);
    else return hipErrorInvalidValue;
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
        case T_Q4_1: return plan_ok<T_Q4_1>(in);
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
                          uint32_t hidden, uint32_t ffn, uint32_t n_experts, uint32_t top_k,
                          uint32_t variant) {
    return gate_type == up_type && quant_plan_ok(gate_type, hidden) &&
           quant_plan_ok(down_type, ffn) && n_experts >= 1 && n_experts <= kMaxExperts &&
           top_k >= 1 && top_k <= kMaxTopK && top_k <= n_experts &&
           variant <= 1u && router_width_ok(hidden);
}

hipError_t launch_moe_router(const MoeDecodeArgs& a, hipStream_t s) {
    switch (a.hidden / kRouterThreads) {
#define PK_RT(C)                                                                                \
    case C:                                                                                     \
        hipLaunchKernelGGL(k_router<C>, dim3(a.n_experts + a.variant), dim3(64), 0, s, a);     \
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
        case T_Q4_1: return gate_up_t<T_Q4_1>(a, s);
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
        case T_Q4_1: return down_t<T_Q4_1>(a, s);
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
