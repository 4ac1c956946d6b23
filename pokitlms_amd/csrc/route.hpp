// route.hpp -- expert routing shared by the decode and prefill kernels.
//
// The reference's route_experts (src/qwen3_moe_runner.cpp:267-305) ranks
// FP32 router logits that the CPU sums serially.  Here the router computes,
// per (token, expert), the exact value S of that logit and a rigorous bound
// B on the CPU's rounding; one wave ranks the experts by S and certifies the
// ranking against the intervals [S - B, S + B], falling back to the CPU's
// exact serial FP32 logits for the experts that could still enter the top-k.
// Route weights follow route_experts: FP64 softmax over all experts, FP32
// probabilities, FP32 renormalisation.
#pragma once

#include <math.h>

#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

constexpr uint32_t kMaxExperts = 256;
constexpr uint32_t kRouterThreads = 256;
constexpr uint32_t kMaxTopK = 8;      // routes per token: waves of the down/combine workgroup

// Status words (MoeDecodeArgs::status).  ST_ERROR: 1 = non-finite router
// logits; it stays set until the host reads and clears it.
enum : uint32_t { ST_ERROR = 0, ST_FALLBACKS = 1, ST_CANDIDATES = 2 };

// Qwen3.5's sigmoid and silu (src/qwen35_runner.cpp:111-123).
__device__ __forceinline__ float sigmoid35(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}
__device__ __forceinline__ float silu(float v) { return v * sigmoid35(v); }

// Phase stamp of a traced step (MoeDecodeArgs::trace; a uniform branch when off).
__device__ __forceinline__ void trace_stamp(uint64_t* trace, uint32_t kernel, uint32_t slot) {
    if (trace) {
        const uint32_t w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
        const uint64_t t = __builtin_amdgcn_s_memrealtime();
        if ((threadIdx.x & 63u) == 0u && w < kTraceWaves)
            trace[(static_cast<uint64_t>(kernel) * kTraceWaves + w) * kTraceSlots + slot] = t;
    }
}

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

// (ext_vector_type arrays stay in registers; arrays of HIP's float4 class
// can be left in scratch.)
typedef float rf32x4 __attribute__((ext_vector_type(4)));

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
        // unrolled so the LDS reads of several experts are in flight together
#pragma unroll 16
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

// Ranking key of expert e (e < 256) with logit f: the top 23 bits of the
// FP32 order key, then 255 - e in the low byte, so keys are distinct and a
// larger key means a larger logit or, between logits equal in those bits, a
// smaller id.  The key only proposes an order: certification checks it
// against the exact intervals [S - B, S + B], so an order the truncated key
// gets wrong is never certified and goes to the exact path.  Keys have 31
// bits, so k > mine is the sign bit of mine - k.
__device__ __forceinline__ uint32_t route_key(float f, uint32_t e) {
    return ((order_key(f) >> 1) & ~0xffu) | (255u - e);
}

// v of the lane CTRL selects, 0 (the identity of an unsigned maximum) in
// lanes outside ROW_MASK: with that identity the compiler folds the move into
// the maximum (one v_max_u32_dpp per step instead of a copy, a DPP move and a
// maximum on the ranking's dependent chain).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u0max(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK,
                                                             0xf, ROW_MASK == 0xf));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u0max<0xb1>(v));
    v = max(v, dpp_u0max<0x4e>(v));
    v = max(v, dpp_u0max<0x141>(v));
    v = max(v, dpp_u0max<0x140>(v));
    v = max(v, dpp_u0max<0x142, 0xa>(v));
    v = max(v, dpp_u0max<0x143, 0xc>(v));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Experts sit in the lane/slot layout e = lane + 64 * slot: NS slots per lane
// cover up to 64 * NS experts.
constexpr int slots_for(uint32_t experts) { return experts <= 64 ? 1 : experts <= 128 ? 2 : 4; }

__device__ __forceinline__ double readlane_d(double v, uint32_t lane) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __builtin_amdgcn_readlane(p.x, static_cast<int>(lane));
    r.y = __builtin_amdgcn_readlane(p.y, static_cast<int>(lane));
    return __builtin_bit_cast(double, r);
}

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

// Top-k by (S desc, id asc) using route_key, by one wave: top_k selection
// rounds (a uniform condition per unrolled round), each taking the winner's
// interval by readlane; then one wave maximum of the unselected experts'
// upper bounds.
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
        key[m] = present ? route_key(f, e) : 0u;
        lo[m] = d.S[m] - d.B[m];
        hi[m] = d.S[m] + d.B[m];
        w.logit[m] = present ? f : -INFINITY;
    }
    w.finite = __all(fin);
    double lo_r[kMaxTopK], hi_r[kMaxTopK];
#pragma unroll
    for (uint32_t r = 0; r < kMaxTopK; ++r) {
        w.sel[r] = 0u;
        lo_r[r] = -INFINITY;
        hi_r[r] = -INFINITY;
        if (r < K) {  // uniform
            uint32_t mk = key[0];
#pragma unroll
            for (int m = 1; m < NS; ++m) mk = max(mk, key[m]);
            const uint32_t best = wave_max_u32(mk);
            const uint32_t e = 255u - (best & 0xffu);
            w.sel[r] = e;
            lo_r[r] = slot_at<NS>(lo, e);
            hi_r[r] = slot_at<NS>(hi, e);
#pragma unroll
            for (int m = 0; m < NS; ++m) key[m] = key[m] == best ? 0u : key[m];
        }
    }
    // the largest upper bound of the experts left out (selected and absent
    // experts have key 0)
    double u = -INFINITY;
#pragma unroll
    for (int m = 0; m < NS; ++m) u = key[m] != 0u ? fmax(u, hi[m]) : u;
    u = readlane_d(group_max<64>(u), 63u);
    // route r < top_k is certain when its lower bound clears the upper bound
    // of every expert ranked after it, routed or not
    double after = u, lmin = INFINITY;
    bool ok = true;
#pragma unroll
    for (int r = kMaxTopK - 1; r >= 0; --r) {
        const bool routed = static_cast<uint32_t>(r) < K;
        ok = ok && (!routed || lo_r[r] > after);
        lmin = routed ? fmin(lmin, lo_r[r]) : lmin;
        after = fmax(after, hi_r[r]);
    }
    w.certified = ok;
    w.lo_min_sel = lmin;
    return w;
}

// The same ranking and certification by a workgroup of four waves, as
// counts instead of top_k dependent wave maxima: the rank of expert e is the
// number of experts whose key exceeds its key.  Wave w ranks experts
// 32 w + (lane & 31) + 128 p; each 32-lane half of the wave compares against
// half of the keys, read back from the wave's own LDS row (written and read
// by one wave, so no workgroup barrier), and v_permlane32_swap adds the two
// halves' counts.  A routed expert's lanes (rank < top_k) store its id, key
// and interval by rank; after the workgroup's barrier every wave certifies
// the same ranking from those and its own copy of the routing data.
template <int NS>
constexpr int rank_passes() { return NS > 2 ? NS / 2 : 1; }

template <int NS>
struct SharedRank {
    alignas(16) uint32_t keys[4][64 * NS];
    uint32_t sel[kMaxTopK];
    uint32_t key[kMaxTopK];
    double lo[kMaxTopK], hi[kMaxTopK];
};

// S and B of the experts this lane ranks (absent experts re-read expert 0).
template <int NS>
struct RankData {
    double S[rank_passes<NS>()], B[rank_passes<NS>()];
};

__device__ __forceinline__ uint32_t rank_expert(uint32_t p) {
    return 128u * p + 32u * (threadIdx.x >> 6) + (threadIdx.x & 31u);
}

template <int NS>
__device__ __forceinline__ RankData<NS> load_rank_data(const MoeDecodeArgs& a) {
    RankData<NS> d;
#pragma unroll
    for (int p = 0; p < rank_passes<NS>(); ++p) {
        const uint32_t e = rank_expert(p);
        d.S[p] = a.row_sum[e < a.n_experts ? e : 0u];
        d.B[p] = a.row_bound[e < a.n_experts ? e : 0u];
    }
    return d;
}

// Before the workgroup barrier: this wave's ranks; routed experts into sr.
template <int NS>
__device__ __forceinline__ void wg_rank(const MoeDecodeArgs& a, const RouteData<NS>& d,
                                        const RankData<NS>& rk, SharedRank<NS>& sr) {
    constexpr uint32_t HK = 32u * NS;  // keys per half
    const uint32_t lane = threadIdx.x & 63u, E = a.n_experts, K = a.top_k;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t* kw = sr.keys[wave];
#pragma unroll
    for (int m = 0; m < NS; ++m) {
        const uint32_t e = lane + 64u * m;
        kw[e] = e < E ? route_key(static_cast<float>(d.S[m]), e) : 0u;
    }
    // the wave reads what its other lanes wrote: LDS keeps one wave's
    // accesses in order, the fences keep the compiler from reordering them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t* kh = kw + HK * (lane >> 5);
#pragma unroll
    for (int p = 0; p < rank_passes<NS>(); ++p) {
        const uint32_t e = rank_expert(p);
        const bool present = e < E;
        const uint32_t mine = present ? route_key(static_cast<float>(rk.S[p]), e) : 0u;
        uint32_t cnt = 0u;
#pragma unroll
        for (uint32_t i = 0; i < HK; i += 4u) {
            const u32x4_t k4 = *reinterpret_cast<const u32x4_t*>(kh + i);  // one address per half
            cnt += ((mine - k4.x) >> 31) + ((mine - k4.y) >> 31);
            cnt += ((mine - k4.z) >> 31) + ((mine - k4.w) >> 31);
        }
        const auto both = __builtin_amdgcn_permlane32_swap(cnt, cnt, false, false);
        const uint32_t rank = both[0] + both[1];
        if (lane < 32u && present && rank < K) {
            sr.sel[rank] = e;
            sr.key[rank] = mine;
            sr.lo[rank] = rk.S[p] - rk.B[p];
            sr.hi[rank] = rk.S[p] + rk.B[p];
        }
    }
}

// After the barrier, in every wave: the routes and their certification, as
// wave_route gives them.  Rank r is certain when its lower bound clears the
// upper bound of every expert ranked after it: of the routed ones after it
// (a chain over the top_k stored intervals), and of every unrouted expert
// (key below the top_k-th key), which must stay below the smallest routed
// lower bound.
template <int NS>
__device__ __forceinline__ WaveRoutes<NS> wg_certify(const MoeDecodeArgs& a, const RouteData<NS>& d,
                                                     const SharedRank<NS>& sr) {
    const uint32_t lane = threadIdx.x & 63u, E = a.n_experts, K = a.top_k;
    WaveRoutes<NS> w;
    double after = -INFINITY, lmin = INFINITY;
    bool ok = true;
#pragma unroll
    for (int r = kMaxTopK - 1; r >= 0; --r) {
        const bool routed = static_cast<uint32_t>(r) < K;
        w.sel[r] = routed ? sr.sel[r] : 0u;
        const double lo = routed ? sr.lo[r] : INFINITY, hi = routed ? sr.hi[r] : -INFINITY;
        ok = ok && (!routed || lo > after);
        lmin = fmin(lmin, lo);
        after = fmax(after, hi);
    }
    const uint32_t kth = sr.key[K - 1u];
    bool fin = true, below = true;
#pragma unroll
    for (int m = 0; m < NS; ++m) {
        const uint32_t e = lane + 64u * m;
        const bool present = e < E;
        const float f = static_cast<float>(d.S[m]);
        fin = fin && (!present || isfinite(f));
        const bool unrouted = present && route_key(f, e) < kth;
        below = below && (!unrouted || d.S[m] + d.B[m] < lmin);
        w.logit[m] = present ? f : -INFINITY;
    }
    w.finite = __all(fin);
    w.certified = ok && __all(below);
    w.lo_min_sel = lmin;
    return w;
}

// Exact routing of an uncertified token, by the whole workgroup of 256
// threads (rare).  The candidate experts' serial logits are chains of
// dependent adds; fed from global memory one chunk ahead, each chunk would
// wait a full memory latency.  Instead the workgroup streams the candidate
// rows through LDS: up to kStageRows rows at a time, CH values per row and
// chunk, D chunks in flight in registers spread over all threads,
// two LDS buffers; one thread per candidate runs the chain over the staged
// chunk.
constexpr uint32_t kStageRows = 16;

template <uint32_t CH>  // hidden is a multiple of CH
struct FallbackShared {
    double logit[kMaxExperts];
    uint32_t rank[kMaxExperts];
    uint32_t sel[kMaxTopK];
    uint32_t cand[kMaxExperts];
    uint32_t ncand;
    uint32_t bad;  // a non-finite exact logit
    alignas(16) float stage[2][kStageRows * (CH + 4u)];  // rows start on different banks
};

// The decode gate/up kernel stages 128-value chunks (its LDS and register
// budget), the prefill ranking kernel 256-value chunks (half the barriers).
template <uint32_t D, uint32_t CH>
__device__ __forceinline__ void exact_routes(const MoeDecodeArgs& a, double lo_min_sel,
                                             const float* xs, FallbackShared<CH>& fb, bool count) {
    constexpr uint32_t PP = kStageRows * CH / 4u / 256u;  // float4 pieces per thread and chunk
    constexpr uint32_t SS = CH + 4u;
    static_assert(PP * 256u * 4u == kStageRows * CH, "whole pieces per thread of 256");
    const uint32_t t = threadIdx.x, E = a.n_experts, H = a.hidden;
    if (t == 0) {
        fb.ncand = 0u;
        fb.bad = 0u;
    }
    __syncthreads();
    if (t < E) {
        const double s = a.row_sum[t], b = a.row_bound[t];
        // An expert with hi < lo_min_sel is below k certain experts; every other
        // expert gets its exact CPU logit.  FP32 rounding of S keeps the rest
        // below lo_min_sel (|fl(S) - S| <= u|S| <= bound).
        if (!(s + b < lo_min_sel)) fb.cand[atomicAdd(&fb.ncand, 1u)] = t;
        else fb.logit[t] = static_cast<double>(static_cast<float>(s));
    }
    __syncthreads();
    const uint32_t nc = fb.ncand, nch = H / CH;
    if (t == 0 && count) {
        atomicAdd(a.status + ST_FALLBACKS, 1u);
        atomicAdd(a.status + ST_CANDIDATES, nc);
    }
    for (uint32_t g0 = 0; g0 < nc; g0 += kStageRows) {
        const uint32_t rows = nc - g0 < kStageRows ? nc - g0 : kStageRows;
        const float* src[PP];
        uint32_t dst[PP], xcol[PP];
#pragma unroll
        for (uint32_t p = 0; p < PP; ++p) {
            const uint32_t q = t + 256u * p, r = q / (CH / 4u), col = 4u * (q % (CH / 4u));
            const uint32_t rr = r < rows ? r : 0u;  // rows past the group repeat row 0's loads
            src[p] = a.router + static_cast<uint64_t>(fb.cand[g0 + rr]) * H + col;
            dst[p] = r * SS + col;
            xcol[p] = col;
        }
        rf32x4 ring[D][PP];
#pragma unroll
        for (uint32_t d = 0; d + 1u < D; ++d)
#pragma unroll
            for (uint32_t p = 0; p < PP; ++p)
                ring[d][p] = *reinterpret_cast<const rf32x4*>(src[p] + (d < nch ? d : nch - 1u) * CH);
        float s = 0.0f;
        for (uint32_t c0 = 0; c0 < nch; c0 += D) {
#pragma unroll
            for (uint32_t k = 0; k < D; ++k) {
                const uint32_t c = c0 + k;
                if (c >= nch) break;  // uniform; only when nch is not a multiple of D
                const uint32_t cn = c + D - 1u < nch ? c + D - 1u : nch - 1u;  // tail: harmless reload
                // stage the CPU's rounded products fl(w_i * x_i); the chain then
                // only adds (dot_f32's order, src/simd_kernels.hpp:12-24)
#pragma unroll
                for (uint32_t p = 0; p < PP; ++p) {
                    const rf32x4 xv = *reinterpret_cast<const rf32x4*>(xs + c * CH + xcol[p]);
                    rf32x4 pr;
                    pr.x = __fmul_rn(ring[k][p].x, xv.x);
                    pr.y = __fmul_rn(ring[k][p].y, xv.y);
                    pr.z = __fmul_rn(ring[k][p].z, xv.z);
                    pr.w = __fmul_rn(ring[k][p].w, xv.w);
                    *reinterpret_cast<rf32x4*>(&fb.stage[c & 1u][dst[p]]) = pr;
                    ring[(k + D - 1u) % D][p] = *reinterpret_cast<const rf32x4*>(src[p] + cn * CH);
                }
                __syncthreads();
                if (t < rows) {
                    // 32 products in registers while the previous 32 are added, so
                    // the dependent adds do not wait on LDS latency
                    const float* pr = &fb.stage[c & 1u][t * SS];
                    rf32x4 A[8], B[8];
#pragma unroll
                    for (uint32_t i = 0; i < 8; ++i) A[i] = *reinterpret_cast<const rf32x4*>(pr + 4u * i);
#pragma unroll
                    for (uint32_t j = 0; j < CH / 32u; ++j) {
                        rf32x4(&cur)[8] = (j & 1u) ? B : A;
                        rf32x4(&nxt)[8] = (j & 1u) ? A : B;
                        if (j + 1u < CH / 32u) {
#pragma unroll
                            for (uint32_t i = 0; i < 8; ++i)
                                nxt[i] = *reinterpret_cast<const rf32x4*>(pr + 32u * (j + 1u) + 4u * i);
                        }
#pragma unroll
                        for (uint32_t i = 0; i < 8; ++i) {
                            s = __fadd_rn(s, cur[i].x);
                            s = __fadd_rn(s, cur[i].y);
                            s = __fadd_rn(s, cur[i].z);
                            s = __fadd_rn(s, cur[i].w);
                        }
                    }
                }
            }
        }
        // linear()'s bias-free 0.0F + dot (src/linear.cpp:203-204)
        if (t < rows) fb.logit[fb.cand[g0 + t]] = static_cast<double>(__fadd_rn(0.0f, s));
        __syncthreads();  // the next group's stores reuse both buffers
    }
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
    float exf = 0.0f;  // variant 1: select_experts' FP32 softmax (src/qwen35_runner.cpp:139-148)
#pragma unroll
    for (int m = 0; m < NS; ++m)
        if (lane + 64u * m < a.n_experts) {
            if (a.variant) exf += expf(l[m] - mxf);
            else ex += exp(static_cast<double>(l[m] - mxf));
        }
    const double denom = a.variant ? 0.0 : lane63(group_sum<64>(ex));
    const float denomf = a.variant ? lane63(group_sum<64>(exf)) : 0.0f;
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
    if (lane < K)
        p = a.variant ? expf(mine - mxf) / denomf
                      : static_cast<float>(exp(static_cast<double>(mine - mxf)) / denom);
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
// Router rows: the exact value S of the CPU's logit (FP64 sum of the FP32
// products it forms) and a rigorous bound B on how far the CPU's serial,
// unfused FP32 sum (src/linear.cpp:26-30, src/simd_kernels.hpp:22) can be
// from S:  |serial - S| <= u * sum_i |T_i| / (1 - n u),  T_i = exact prefix
// sums.  One wave handles a row, lane l holding the N = 4 * N4 consecutive
// products l*N .. l*N + N - 1 (hidden = 64 * N): no barrier and no LDS.

// The row's and x's pieces of one lane (float4 pieces, loads only).
template <int N4>
__device__ __forceinline__ void router_lane_load(const float* v, uint32_t lane, rf32x4 (&r)[N4]) {
    const rf32x4* p = reinterpret_cast<const rf32x4*>(v) + lane * N4;
#pragma unroll
    for (int j = 0; j < N4; ++j) r[j] = p[j];
}

// A lane's products in chunks of 8 consecutive elements (K = N / 8 chunks):
// per chunk the sum L and the sum of |running sums| over its elements.  The
// chunks' chains are independent, so their adds overlap.
template <int N4>
struct RouterLane {
    static constexpr int K = N4 / 2;  // N = 4 * N4 = 8 * K
    double local[K], run_abs[K];
};

// One chunk's running sums over its products fl(w_i * x_i) (the CPU's
// rounded products, exactly), in element order (w, x: the chunk's two float4
// pieces from index j).
__device__ __forceinline__ void router_chunk_sums(const rf32x4* w, const rf32x4* x, double& l,
                                                  double& ra) {
    l = 0.0;
    ra = 0.0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            l += static_cast<double>(__fmul_rn(w[j][c], x[j][c]));
            ra += fabs(l);
        }
    }
}

// Every chunk of the lane.
template <int N4>
__device__ __forceinline__ void router_lane_sums(const rf32x4 (&w)[N4], const rf32x4 (&x)[N4],
                                                 RouterLane<N4>& r) {
    static_assert(N4 % 2 == 0, "whole chunks of 8 products per lane");
#pragma unroll
    for (int k = 0; k < RouterLane<N4>::K; ++k) router_chunk_sums(&w[2 * k], &x[2 * k], r.local[k], r.run_abs[k]);
}

// S and B of the row whose chunk sums the wave holds (uniform results).
//
// S: the FP64 sum of the products (chunk sums in chunk order within a lane,
// then a wave scan; S is the last lane's inclusive value).  B bounds the
// CPU's serial FP32 rounding, u * sum_i |T_i| with T_i the exact prefix sums,
// in one pass through the triangle inequality per chunk of 8: with O the
// chunk's offset (every earlier product) and L_i its own running sum,
// sum_i |O + L_i| <= 8 |O| + sum_i |L_i| (about 8% above the exact prefixes
// on router-like rows of 2,048).  sum_i |p_i| <= 2 sum_i |T_i| covers the FP64
// rounding of S.  The batched prefill router calls the same functions, so
// both paths rank on the same bits.
template <int N4>
__device__ __forceinline__ void router_wave_sum_bound(const RouterLane<N4>& r, double& total,
                                                      double& bound) {
    constexpr int K = RouterLane<N4>::K;
    double lane_sum = r.local[0];
#pragma unroll
    for (int k = 1; k < K; ++k) lane_sum += r.local[k];
    const double incl = wave_inclusive_scan(lane_sum);
    total = lane63(incl);
    double off = incl - lane_sum, qs = 0.0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        qs += __builtin_fma(8.0, fabs(off), r.run_abs[k]);
        off += r.local[k];
    }
    const double q = lane63(group_sum<64>(qs));
    // u = 2^-24; (1 + 2^-10) >= 1/(1 - n u) for n <= 2^13 and covers the FP64
    // rounding of the prefix sums; q * 2^-39 >= sum |p| * 2^-40 covers S
    bound = q * (0x1p-24 * (1.0 + 0x1p-10) + 0x1p-39);
    if (!(q < 5.0e35)) bound = INFINITY;  // near FP32 overflow: always recompute
}

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
template <uint32_t XP = kXPieces>  // pieces per thread: hidden <= 1024 * XP
struct XRegs {
    float4 v[XP];
};

// Pieces past the end load and store the last piece again (the same values
// as its own thread writes), so neither the loads nor the stores sit in a
// branch: a load sunk into a branch next to its use would wait for every
// load issued before it.
__device__ __forceinline__ uint32_t x_piece(uint32_t i, uint32_t n) {
    const uint32_t k = (i * blockDim.x + threadIdx.x) * 4u;
    return k < n ? k : n - 4u;
}

template <uint32_t XP = kXPieces>
__device__ __forceinline__ XRegs<XP> load_x_regs(const float* x, uint32_t n) {
    XRegs<XP> r;
#pragma unroll
    for (uint32_t i = 0; i < XP; ++i)
        r.v[i] = *reinterpret_cast<const float4*>(x + x_piece(i, n));
    return r;
}

template <uint32_t XP>
__device__ __forceinline__ void store_x_regs(float* xs, const XRegs<XP>& r, uint32_t n) {
#pragma unroll
    for (uint32_t i = 0; i < XP; ++i) *reinterpret_cast<float4*>(xs + x_piece(i, n)) = r.v[i];
}

}  // namespace
}  // namespace pk
