// moe.hip -- single-token routed-MoE layer on gfx950.
//
// Three launches replace the MoE block of the reference runner
// (src/qwen3_moe_runner.cpp:643-692) and its route_experts (:267-305):
//
//  1. k_router: one wave per expert row computes the router logit's exact
//     value S (FP64 sum of the FP32 products the CPU forms) and a rigorous
//     bound B on how far the CPU's serial, unfused FP32 sum
//     (src/linear.cpp:26-30, src/simd_kernels.hpp:22) can be from S:
//         |serial - S| <= u * sum_i |T_i| / (1 - n u),  T_i = exact prefix sums.
//     The last workgroup to finish ranks the experts by S.  When the
//     intervals [S-B, S+B] prove the top-k set and order, that ranking is the
//     CPU's; otherwise every expert that could still enter the top-k is
//     recomputed with the CPU's exact serial FP32 recurrence (one lane per
//     row) and the ranking is redone on those bit-exact logits.  Softmax
//     (FP64 exp, FP32 probabilities, FP32 renormalisation) follows
//     route_experts.
//  2. k_gate_up: every (route, ffn row) pair dots the gate and up rows of the
//     selected expert with the register-resident input and writes the SwiGLU
//     activation g / (1 + expf(-g)) * u (:682-684).
//  3. k_down: a workgroup of top_k waves computes one down-row dot per route
//     and combines them in route order, y = ((0 + p0*o0) + p1*o1) + ...
//     (:688-690), deterministically and without atomics.
#include <math.h>

#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

constexpr uint32_t kRouterMaxExperts = 256;
constexpr uint32_t kRouterMaxHidden = 8192;  // 128 products per lane
constexpr uint32_t kRouterWaves = 4;
constexpr uint32_t kMaxTopK = 8;  // routes per token: waves of the down/combine workgroup

bool router_width_ok(uint32_t hidden) {
    if (hidden % 64u || hidden > kRouterMaxHidden) return false;
    switch (hidden / 64u) {
        case 8: case 16: case 32: case 48: case 64: case 96: case 128: return true;
        default: return false;
    }
}

// Status words (MoeDecodeArgs::status).
enum : uint32_t { ST_ERROR = 0, ST_FALLBACKS = 1, ST_CANDIDATES = 2 };

// Order of route_experts' sorted insertion: larger logit first, then smaller id.
__device__ __forceinline__ bool key_before(double av, uint32_t aid, double bv, uint32_t bid) {
    return av > bv || (av == bv && aid < bid);
}

__device__ __forceinline__ double shfl_xor_d(double v, int m) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __shfl_xor(p.x, m, 64);
    r.y = __shfl_xor(p.y, m, 64);
    return __builtin_bit_cast(double, r);
}

__device__ __forceinline__ double shfl_up_d(double v, int d) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __shfl_up(p.x, d, 64);
    r.y = __shfl_up(p.y, d, 64);
    return __builtin_bit_cast(double, r);
}

__device__ __forceinline__ double shfl_d(double v, int src) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __shfl(p.x, src, 64);
    r.y = __shfl(p.y, src, 64);
    return __builtin_bit_cast(double, r);
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_d(v, m);
    return v;
}

// The CPU's router logit, bit for bit: s = fl(s + fl(w_i * x_i)), i ascending,
// then linear()'s bias-free 0.0F + dot (src/linear.cpp:203-204).  Loads run one
// 32-element batch ahead of the dependent add chain.
__device__ float serial_logit(const float* __restrict__ w, const float* __restrict__ xs,
                              uint32_t hidden) {
    float s = 0.0f;
    float4 cur[8], nxt[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cur[j] = *reinterpret_cast<const float4*>(w + 4 * j);
    for (uint32_t i = 0; i < hidden; i += 32) {
        const bool more = i + 32 < hidden;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            nxt[j] = more ? *reinterpret_cast<const float4*>(w + i + 32 + 4 * j) : cur[j];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float* xv = xs + i + 4 * j;
            s = __fadd_rn(s, __fmul_rn(cur[j].x, xv[0]));
            s = __fadd_rn(s, __fmul_rn(cur[j].y, xv[1]));
            s = __fadd_rn(s, __fmul_rn(cur[j].z, xv[2]));
            s = __fadd_rn(s, __fmul_rn(cur[j].w, xv[3]));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) cur[j] = nxt[j];
    }
    return __fadd_rn(0.0f, s);
}

__device__ __forceinline__ double block_max_d(double v, double* red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmax(v, shfl_xor_d(v, m));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = red[0];
    for (uint32_t w = 1; w < (blockDim.x >> 6); ++w) r = fmax(r, red[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ double block_sum_d(double v, double* red) {
    v = wave_sum_d(v);
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double r = red[0];
    for (uint32_t w = 1; w < (blockDim.x >> 6); ++w) r += red[w];
    __syncthreads();
    return r;
}

// Block-wide top-k over `count` keys in LDS, ordered by key_before; selected
// ids land in sel[0..k) and are flagged in `taken`.  blockDim.x == 256.
__device__ void block_topk(const double* __restrict__ v, uint32_t count, uint32_t k,
                           uint32_t* __restrict__ sel, uint32_t* __restrict__ taken, double* wv,
                           uint32_t* wid) {
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    if (t < kRouterMaxExperts) taken[t] = 0u;
    __syncthreads();
    for (uint32_t r = 0; r < k; ++r) {
        double bv = -INFINITY;
        uint32_t bid = 0xffffffffu;
        if (t < count && !taken[t]) {
            bv = v[t];
            bid = t;
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const double ov = shfl_xor_d(bv, m);
            const uint32_t oid = static_cast<uint32_t>(__shfl_xor(static_cast<int>(bid), m, 64));
            if (oid != 0xffffffffu && (bid == 0xffffffffu || key_before(ov, oid, bv, bid))) {
                bv = ov;
                bid = oid;
            }
        }
        if (lane == 0) {
            wv[wave] = bv;
            wid[wave] = bid;
        }
        __syncthreads();
        if (t == 0) {
            double best = wv[0];
            uint32_t best_id = wid[0];
            for (uint32_t w = 1; w < (blockDim.x >> 6); ++w) {
                if (wid[w] != 0xffffffffu &&
                    (best_id == 0xffffffffu || key_before(wv[w], wid[w], best, best_id))) {
                    best = wv[w];
                    best_id = wid[w];
                }
            }
            sel[r] = best_id;
            if (best_id < kRouterMaxExperts) taken[best_id] = 1u;
        }
        __syncthreads();
    }
}

template <int C>  // contiguous products per lane: hidden = 64 * C
__global__ __launch_bounds__(256) void k_router(MoeDecodeArgs a) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t e = blockIdx.x * kRouterWaves + wave;
    const uint32_t H = a.hidden;

    // ---- phase 1: exact sum and serial-error bound of this wave's row ----
    if (e < a.n_experts) {
        const float* w = a.router + static_cast<uint64_t>(e) * H + lane * C;
        const float* xx = a.x + lane * C;
        float p[C];
#pragma unroll
        for (int i = 0; i < C; i += 4) {
            const float4 wv = *reinterpret_cast<const float4*>(w + i);
            const float4 xv = *reinterpret_cast<const float4*>(xx + i);
            p[i + 0] = __fmul_rn(wv.x, xv.x);  // the CPU's rounded products, exactly
            p[i + 1] = __fmul_rn(wv.y, xv.y);
            p[i + 2] = __fmul_rn(wv.z, xv.z);
            p[i + 3] = __fmul_rn(wv.w, xv.w);
        }
        double local = 0.0, abs_p = 0.0;
#pragma unroll
        for (int i = 0; i < C; ++i) {
            local += static_cast<double>(p[i]);
            abs_p += fabs(static_cast<double>(p[i]));
        }
        double incl = local;  // inclusive scan of lane totals
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const double o = shfl_up_d(incl, d);
            if (static_cast<int>(lane) >= d) incl += o;
        }
        double t = incl - local;  // prefix before this lane's first product
        double prefix_abs = 0.0;
#pragma unroll
        for (int i = 0; i < C; ++i) {
            t += static_cast<double>(p[i]);
            prefix_abs += fabs(t);
        }
        const double total = shfl_d(incl, 63);
        prefix_abs = wave_sum_d(prefix_abs);
        abs_p = wave_sum_d(abs_p);
        if (lane == 0) {
            // u = 2^-24.  (1 + 2^-10) >= 1/(1 - n u) for n <= 2^13 and also covers
            // the FP64 rounding of the prefix sums; abs_p * 2^-40 covers S itself.
            double bound = prefix_abs * 0x1p-24 * (1.0 + 0x1p-10) + abs_p * 0x1p-40;
            if (!(abs_p < 1.0e36)) bound = INFINITY;  // near FP32 overflow: recompute
            a.row_sum[e] = total;
            a.row_bound[e] = bound;
        }
    }

    // ---- the last block to finish ranks, certifies, falls back, normalises ----
    __shared__ uint32_t is_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(a.counter, 1u) == gridDim.x - 1u;
    __syncthreads();
    if (!is_last) return;
    __threadfence();

    __shared__ double logit[kRouterMaxExperts];
    __shared__ double lo[kRouterMaxExperts];
    __shared__ double hi[kRouterMaxExperts];
    __shared__ double red[4];
    __shared__ uint32_t wid[4];
    __shared__ uint32_t sel[16];
    __shared__ uint32_t taken[kRouterMaxExperts];
    __shared__ float probs[16];
    __shared__ float xs[64 * C];
    const uint32_t t = threadIdx.x;
    const uint32_t E = a.n_experts, K = a.top_k;
    if (t < E) {
        const double s = __builtin_nontemporal_load(a.row_sum + t);
        const double b = __builtin_nontemporal_load(a.row_bound + t);
        logit[t] = s;
        lo[t] = s - b;
        hi[t] = s + b;
    }
    __syncthreads();
    block_topk(logit, E, K, sel, taken, red, wid);

    // Certified when lo(sel[r]) > max hi over everything ranked after r.
    const double mx_rest = block_max_d(t < E && !taken[t] ? hi[t] : -INFINITY, red);
    __shared__ uint32_t need_serial;
    __shared__ double lo_min_sel;
    if (t == 0) {
        double after = mx_rest, lmin = INFINITY;
        uint32_t ok = 1u;
        for (int r = static_cast<int>(K) - 1; r >= 0; --r) {
            const uint32_t id = sel[r];
            if (!(lo[id] > after)) ok = 0u;
            after = fmax(after, hi[id]);
            lmin = fmin(lmin, lo[id]);
        }
        need_serial = ok ? 0u : 1u;
        lo_min_sel = lmin;
    }
    __syncthreads();

    if (need_serial) {
        for (uint32_t i = t; i < H; i += blockDim.x) xs[i] = a.x[i];
        __syncthreads();
        // An expert with hi < lo_min_sel is below k certain experts; every other
        // expert gets its exact CPU logit.  FP32 rounding of S keeps the rest
        // below lo_min_sel (|fl(S) - S| <= u|S| <= bound).
        if (t < E) {
            if (!(hi[t] < lo_min_sel)) {
                logit[t] = static_cast<double>(
                    serial_logit(a.router + static_cast<uint64_t>(t) * H, xs, H));
                atomicAdd(a.status + ST_CANDIDATES, 1u);
            } else {
                logit[t] = static_cast<double>(static_cast<float>(logit[t]));
            }
        }
        if (t == 0) atomicAdd(a.status + ST_FALLBACKS, 1u);
        __syncthreads();
        block_topk(logit, E, K, sel, taken, red, wid);
    } else {
        if (t < E) logit[t] = static_cast<double>(static_cast<float>(logit[t]));
        __syncthreads();
    }

    // Non-finite logits make route_experts throw (src/qwen3_moe_runner.cpp:270-276).
    const double finite_all = block_max_d(t < E && !isfinite(logit[t]) ? 1.0 : 0.0, red);
    if (finite_all != 0.0) {
        if (t == 0) {
            a.status[ST_ERROR] = 1u;
            *a.counter = 0u;
        }
        if (t < K) {
            a.ids[t] = 0xffffffffu;
            a.probs[t] = 0.0f;
        }
        return;
    }

    // Softmax over all experts: FP64 exp of the FP32 difference, FP32 result.
    const double mx = block_max_d(t < E ? logit[t] : -INFINITY, red);
    const float mxf = static_cast<float>(mx);
    const double denom = block_sum_d(
        t < E ? exp(static_cast<double>(static_cast<float>(logit[t]) - mxf)) : 0.0, red);
    if (t < K) {
        const float l = static_cast<float>(logit[sel[t]]);
        probs[t] = static_cast<float>(exp(static_cast<double>(l - mxf)) / denom);
    }
    __syncthreads();
    if (t < K) {
        float selected_sum = 0.0f;
        for (uint32_t r = 0; r < K; ++r) selected_sum = __fadd_rn(selected_sum, probs[r]);
        float q = a.normalize ? probs[t] / selected_sum : probs[t];
        if (a.scale != 1.0f) q = __fmul_rn(q, a.scale);
        a.ids[t] = sel[t];
        a.probs[t] = q;
    }
    if (t == 0) {
        a.status[ST_ERROR] = 0u;
        *a.counter = 0u;  // ready for the next launch on this stream
    }
}

// ---------------------------------------------------------------------------
// gate/up + SwiGLU.  All (route, row) items share the input x, so one unit
// mapping (and one register copy of x per lane) serves every item.

template <int T, int UB, int NU>
__global__ __launch_bounds__(256) void k_gate_up(MoeDecodeArgs a, uint32_t units, uint32_t glog2) {
    extern __shared__ float xsh[];
    for (uint32_t i = threadIdx.x; i < a.hidden; i += blockDim.x) xsh[i] = a.x[i];
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t G = 1u << glog2, RPP = 64u >> glog2;
    const uint32_t sub = lane >> glog2, ul = lane & (G - 1u);
    UnitPos pos[NU];
    bool valid[NU];
    UnitX<T, UB, 1> ux[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const uint32_t u = ul + G * k;
        valid[k] = u < units;
        pos[k] = unit_pos<T, UB>(valid[k] ? u : 0u);
        load_unit_x<T, UB, 1>(xsh, 0, pos[k], valid[k], ux[k]);
    }
    const uint32_t items = a.top_k * a.ffn;
    const uint32_t passes = (items + RPP - 1u) / RPP;
    const uint32_t nw = gridDim.x * (blockDim.x >> 6);
    for (uint32_t p = blockIdx.x * (blockDim.x >> 6) + wave; p < passes; p += nw) {
        const uint32_t item = p * RPP + sub;
        const bool live = item < items;
        float g[1] = {0.0f}, u[1] = {0.0f};
        if (live) {
            const uint32_t route = item / a.ffn, row = item % a.ffn;
            uint64_t e = a.ids[route];
            if (e >= a.n_experts) e = 0;  // router error: ids are marked invalid, output unused
            const uint8_t* gr = a.gate + e * a.gate_slice + row * a.gate_row;
            const uint8_t* ur = a.up + e * a.up_slice + row * a.up_row;
#pragma unroll
            for (int k = 0; k < NU; ++k) {
                if (valid[k]) {
                    unit_fma<T, UB, 1>(gr, pos[k], ux[k], g);
                    unit_fma<T, UB, 1>(ur, pos[k], ux[k], u);
                }
            }
        }
        const float gs = group_sum_dyn(g[0], G);
        const float us = group_sum_dyn(u[0], G);
        if (live && ul == 0) a.act[item] = (gs / (1.0f + expf(-gs))) * us;
    }
}

// ---------------------------------------------------------------------------
// down + combine.  blockDim = 64 * top_k: wave k owns route k.

template <int T, int UB, int NU>
__global__ __launch_bounds__(64 * kMaxTopK) void k_down(MoeDecodeArgs a, uint32_t units, uint32_t glog2) {
    extern __shared__ float part[];  // [top_k][RPP]
    const uint32_t lane = threadIdx.x & 63u, k = threadIdx.x >> 6;
    const uint32_t G = 1u << glog2, RPP = 64u >> glog2;
    const uint32_t sub = lane >> glog2, ul = lane & (G - 1u);
    uint64_t e = a.ids[k];
    if (e >= a.n_experts) e = 0;  // router error: ids are marked invalid, output unused
    const float* act = a.act + k * a.ffn;
    UnitPos pos[NU];
    bool valid[NU];
    UnitX<T, UB, 1> ux[NU];
#pragma unroll
    for (int q = 0; q < NU; ++q) {
        const uint32_t u = ul + G * q;
        valid[q] = u < units;
        pos[q] = unit_pos<T, UB>(valid[q] ? u : 0u);
        load_unit_x<T, UB, 1>(act, 0, pos[q], valid[q], ux[q]);
    }
    const uint8_t* base = a.down + e * a.down_slice;
    const uint32_t rows = a.hidden;
    const uint32_t passes = (rows + RPP - 1u) / RPP;
    float route_p[kMaxTopK];
    for (uint32_t r = 0; r < kMaxTopK; ++r) route_p[r] = r < a.top_k ? a.probs[r] : 0.0f;
    for (uint32_t p = blockIdx.x; p < passes; p += gridDim.x) {
        const uint32_t row = p * RPP + sub;
        float acc[1] = {0.0f};
        if (row < rows) {
            const uint8_t* rp = base + static_cast<uint64_t>(row) * a.down_row;
#pragma unroll
            for (int q = 0; q < NU; ++q)
                if (valid[q]) unit_fma<T, UB, 1>(rp, pos[q], ux[q], acc);
        }
        const float v = group_sum_dyn(acc[0], G);
        if (ul == 0) part[k * RPP + sub] = v;
        __syncthreads();
        if (k == 0 && lane < RPP) {
            const uint32_t orow = p * RPP + lane;
            if (orow < rows) {
                float y = 0.0f;
                for (uint32_t r = 0; r < a.top_k; ++r)
                    y = __fadd_rn(y, __fmul_rn(route_p[r], part[r * RPP + lane]));
                a.y[orow] = y;
            }
        }
        __syncthreads();
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
    return nu <= 4u;
}

template <int T>
hipError_t gate_up_t(const MoeDecodeArgs& a, hipStream_t s) {
    constexpr int UB = moe_ub<T>();
    uint32_t units, glog2, nu;
    if (!moe_plan<T>(a.hidden, units, glog2, nu)) return hipErrorInvalidValue;
    const uint32_t RPP = 64u >> glog2;
    const uint32_t passes = ceil_div(a.top_k * a.ffn, RPP);
    uint32_t blocks = ceil_div(passes, 4u);
    if (blocks > 512u) blocks = 512u;
    const size_t lds = a.hidden * sizeof(float);
#define PK_GU(N)                                                                              \
    case N:                                                                                   \
        hipLaunchKernelGGL((k_gate_up<T, UB, N>), dim3(blocks), dim3(256), lds, s, a, units, \
                           glog2);                                                            \
        break;
    switch (nu) { PK_GU(1) PK_GU(2) PK_GU(3) PK_GU(4) default: return hipErrorInvalidValue; }
#undef PK_GU
    return hipGetLastError();
}

template <int T>
hipError_t down_t(const MoeDecodeArgs& a, hipStream_t s) {
    constexpr int UB = moe_ub<T>();
    uint32_t units, glog2, nu;
    if (!moe_plan<T>(a.ffn, units, glog2, nu)) return hipErrorInvalidValue;
    const uint32_t RPP = 64u >> glog2;
    const uint32_t passes = ceil_div(a.hidden, RPP);
    uint32_t blocks = passes < 256u ? passes : 256u;
    const size_t lds = static_cast<size_t>(a.top_k) * RPP * sizeof(float);
#define PK_DN(N)                                                                              \
    case N:                                                                                   \
        hipLaunchKernelGGL((k_down<T, UB, N>), dim3(blocks), dim3(64u * a.top_k), lds, s, a,  \
                           units, glog2);                                                     \
        break;
    switch (nu) { PK_DN(1) PK_DN(2) PK_DN(3) PK_DN(4) default: return hipErrorInvalidValue; }
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

}  // namespace

bool moe_decode_supported(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                          uint32_t hidden, uint32_t ffn, uint32_t n_experts, uint32_t top_k) {
    return gate_type == up_type && quant_plan_ok(gate_type, hidden) &&
           quant_plan_ok(down_type, ffn) && n_experts >= 1 && n_experts <= kRouterMaxExperts &&
           top_k >= 1 && top_k <= kMaxTopK && top_k <= n_experts && router_width_ok(hidden);
}

hipError_t launch_moe_router(const MoeDecodeArgs& a, hipStream_t s) {
    const uint32_t blocks = ceil_div(a.n_experts, kRouterWaves);
    switch (a.hidden / 64u) {
#define PK_RT(C)                                                                       \
    case C:                                                                            \
        hipLaunchKernelGGL(k_router<C>, dim3(blocks), dim3(64 * kRouterWaves), 0, s, a); \
        break;
        PK_RT(8) PK_RT(16) PK_RT(32) PK_RT(48) PK_RT(64) PK_RT(96) PK_RT(128)
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
