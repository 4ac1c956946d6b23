// prefill.hip -- batched routed-MoE prefill on gfx950 (MFMA grouped GEMM).
//
// The reference prefills a prompt one token at a time through the MoE block
// of src/qwen3_moe_runner.cpp:643-692 (the loop at :785-790), so every
// token's routes and output are those of a single-token pass.  Here the
// whole batch goes through six launches:
//
//  1. k_router_batch: the exact logit value S and rounding bound B of every
//     (token, expert) pair (the decode router's arithmetic, one expert row
//     held in registers across a tile of tokens).
//  2. k_route_batch: one workgroup per token ranks the experts exactly as the
//     decode path does (certified wave ranking, exact serial fallback),
//     writes ids and route weights, and counts each expert's tokens.
//  3. k_group: one workgroup turns the counts into per-expert row ranges,
//     a list of 32-row tiles and the assignments (token * top_k + route)
//     grouped by expert; it leaves the counts at zero for the next call.
//  4. k_gate_up_mfma: per tile and 128 ffn rows, gate and up GEMMs on
//     v_mfma_f32_32x32x2f32 with the weights dequantised into LDS exactly as
//     the reference decodes them (FP32 values), and the SwiGLU epilogue.
//  5. k_down_mfma: per tile and 128 hidden rows, the down GEMM; each
//     output row goes to its (token, route) slot.
//  6. k_combine: y = ((0 + p0*o0) + p1*o1) + ... per token in route order
//     (:688-690).
//
// Launch sizes depend only on the token count; tiles past the actual count
// exit at once, so the host never waits for the grouping.
#include <math.h>

#include "kquant.hpp"
#include "launch.hpp"
#include "route.hpp"

namespace pk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kTileM = 32;      // tokens per GEMM tile (MFMA M)
constexpr uint32_t kTileN = 128;     // output rows per workgroup: 4 waves x 32
constexpr uint32_t kChunk = 32;      // K elements staged per step
constexpr uint32_t kRouterTokens = 8;  // tokens per batched-router workgroup

// ---------------------------------------------------------------------------
// Dequantisation of 32 consecutive elements k0 .. k0 + 31 (k0 % 32 == 0) of
// one GGUF row to the reference's FP32 values (src/quantized_linear.cpp:
// 166-205, 286-358, 387-423): loads first (Raw32), values later.

template <int T>
struct Raw32;
template <> struct Raw32<T_Q4_K> { uint32_t h[4]; uint32_t q[8]; };
template <> struct Raw32<T_Q5_K> { uint32_t h[4]; uint32_t q[8]; uint32_t qh[8]; };
template <> struct Raw32<T_Q6_K> { uint32_t ql[8]; uint32_t qh[8]; int32_t s0, s1; uint32_t d; };
template <> struct Raw32<T_Q8_0> { uint32_t q[8]; uint32_t d; };
template <> struct Raw32<T_Q4_0> { uint32_t q[4]; uint32_t d; };

template <int T>
__device__ __forceinline__ void raw32_load(const uint8_t* row, uint32_t k0, Raw32<T>& r) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = row + (k0 / 256u) * Fmt<T>::BB;
        const uint32_t j = (k0 % 256u) / 32u, chunk = j / 2u;
        ld_words<4>(blk, r.h);
        ld_words<8>(blk + (T == T_Q4_K ? 16u : 48u) + 32u * chunk, r.q);
        if constexpr (T == T_Q5_K) ld_words<8>(blk + 16u, r.qh);
    } else if constexpr (T == T_Q6_K) {
        const uint8_t* blk = row + (k0 / 256u) * 210u;
        const uint32_t c = (k0 % 256u) / 32u, half = c / 4u, g = c % 4u;
        ld_words_2a<8>(blk + 64u * half + 32u * (g & 1u), r.ql);
        ld_words_2a<8>(blk + 128u + 32u * half, r.qh);
        r.s0 = static_cast<int8_t>(blk[192u + 8u * half + 2u * g]);
        r.s1 = static_cast<int8_t>(blk[192u + 8u * half + 2u * g + 1u]);
        r.d = ld_u16(blk + 208u);
    } else if constexpr (T == T_Q8_0) {
        const uint8_t* blk = row + (k0 / 32u) * 34u;
        ld_words_2a<8>(blk + 2u, r.q);
        r.d = ld_u16(blk);
    } else {  // Q4_0
        const uint8_t* blk = row + (k0 / 32u) * 18u;
        ld_words_2a<4>(blk + 2u, r.q);
        r.d = ld_u16(blk);
    }
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, uint32_t i) {
    return (w[i >> 2] >> (8u * (i & 3u))) & 0xffu;
}

template <int T>
__device__ __forceinline__ void raw32_decode(const Raw32<T>& r, uint32_t k0, float (&v)[32]) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint32_t j = (k0 % 256u) / 32u, chunk = j / 2u, hi = j & 1u;
        const float d = half_bits_to_float(r.h[0] & 0xffffu);
        const float dmin = half_bits_to_float(r.h[0] >> 16);
        float sc, mn;
        kq_scale_min(r.h, j, sc, mn);
        const float ds = __fmul_rn(d, sc), dm = __fmul_rn(dmin, mn);
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) {
            uint32_t q = byte_of(r.q, i);
            q = hi ? q >> 4 : q & 15u;
            if constexpr (T == T_Q5_K) q += ((byte_of(r.qh, i) >> (2u * chunk + hi)) & 1u) << 4;
            v[i] = __fsub_rn(__fmul_rn(ds, static_cast<float>(q)), dm);  // fl(fl(d*s)*q) - fl(dmin*m)
        }
    } else if constexpr (T == T_Q6_K) {
        const uint32_t c = (k0 % 256u) / 32u, g = c % 4u;
        const float d = half_bits_to_float(r.d);
        const float ds0 = __fmul_rn(d, static_cast<float>(r.s0));
        const float ds1 = __fmul_rn(d, static_cast<float>(r.s1));
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) {
            const uint32_t lb = byte_of(r.ql, i), hb = byte_of(r.qh, i);
            const uint32_t nib = g >= 2u ? lb >> 4 : lb & 15u;
            const int q = static_cast<int>(nib | (((hb >> (2u * g)) & 3u) << 4)) - 32;
            v[i] = __fmul_rn(i < 16u ? ds0 : ds1, static_cast<float>(q));  // fl(fl(d*s)*q)
        }
    } else if constexpr (T == T_Q8_0) {
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i)
            v[i] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(byte_of(r.q, i))));
    } else {  // Q4_0: low nibbles are elements 0..15, high nibbles 16..31
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
            const uint32_t b = byte_of(r.q, i);
            v[i] = __fmul_rn(d, static_cast<float>(static_cast<int>(b & 15u) - 8));
            v[i + 16] = __fmul_rn(d, static_cast<float>(static_cast<int>(b >> 4) - 8));
        }
    }
}

// ---------------------------------------------------------------------------
// 1. Batched router.

template <int C>
__global__ __launch_bounds__(kRouterThreads) void k_router_batch(MoePrefillArgs a) {
    __shared__ double wtot[kRouterThreads / 64];
    __shared__ double red[kRouterThreads / 64];
    const uint32_t e = blockIdx.x, E = a.layer.n_experts, H = a.layer.hidden;
    const uint32_t t0 = blockIdx.y * kRouterTokens;
    const uint32_t t1 = t0 + kRouterTokens < a.tokens ? t0 + kRouterTokens : a.tokens;
    const float* w = a.layer.router + static_cast<uint64_t>(e) * H + threadIdx.x * C;
    float wr[C];
#pragma unroll
    for (int i = 0; i < C; i += 2) {
        const float2 v = *reinterpret_cast<const float2*>(w + i);
        wr[i] = v.x;
        wr[i + 1] = v.y;
    }
    for (uint32_t t = t0; t < t1; ++t) {
        const float* xx = a.x + static_cast<uint64_t>(t) * H + threadIdx.x * C;
        float p[C];
#pragma unroll
        for (int i = 0; i < C; i += 2) {
            const float2 xv = *reinterpret_cast<const float2*>(xx + i);
            p[i] = __fmul_rn(wr[i], xv.x);  // the CPU's rounded products, exactly
            p[i + 1] = __fmul_rn(wr[i + 1], xv.y);
        }
        double total, bound;
        router_sum_bound<C>(p, wtot, red, total, bound);
        if (threadIdx.x == 0) {
            a.row_sum[static_cast<uint64_t>(t) * E + e] = total;
            a.row_bound[static_cast<uint64_t>(t) * E + e] = bound;
        }
    }
}

// ---------------------------------------------------------------------------
// 2. Per-token ranking, route weights and expert counts.

template <int NS>
__global__ __launch_bounds__(256) void k_route_batch(MoePrefillArgs A) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [hidden]
    __shared__ FallbackShared fb;
    __shared__ uint32_t s_sel[kMaxTopK];
    __shared__ uint32_t s_state;
    __shared__ double s_lo;
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t E = A.layer.n_experts, K = A.layer.top_k;
    MoeDecodeArgs a = A.layer;  // this token's view
    a.x = A.x + static_cast<uint64_t>(t) * a.hidden;
    a.row_sum = A.row_sum + static_cast<uint64_t>(t) * E;
    a.row_bound = A.row_bound + static_cast<uint64_t>(t) * E;
    a.ids = A.ids + static_cast<uint64_t>(t) * K;
    a.probs = A.probs + static_cast<uint64_t>(t) * K;
    a.status = A.status;

    const XRegs xr = load_x_regs(a.x, a.hidden);
    RouteData<NS> rd;
    if (wave == 0) rd = load_route_data<NS>(a);
    store_x_regs(xs, xr, a.hidden);
    WaveRoutes<NS> w;
    if (wave == 0) {
        w = wave_route<NS>(a, rd);
        if (lane == 0) {
#pragma unroll
            for (uint32_t r = 0; r < kMaxTopK; ++r) s_sel[r] = w.sel[r];
            s_state = !w.finite ? 2u : w.certified ? 0u : 1u;
            s_lo = w.lo_min_sel;
        }
    }
    __syncthreads();
    const uint32_t state = s_state;  // uniform
    if (state == 2u) {
        if (wave == 0) flag_router_error(a);
        return;
    }
    uint32_t sel[kMaxTopK];
    if (state == 1u) {  // rare: exact serial logits of the candidates
        exact_routes(a, s_lo, xs, fb, true);
        if (fb.bad) {
            if (wave == 0) flag_router_error(a);
            return;
        }
#pragma unroll
        for (uint32_t r = 0; r < kMaxTopK; ++r) sel[r] = r < K ? fb.sel[r] : 0u;
        if (wave == 0) {
#pragma unroll
            for (int m = 0; m < NS; ++m)
                w.logit[m] = lane + 64u * m < E ? static_cast<float>(fb.logit[lane + 64u * m]) : -INFINITY;
        }
    } else {
#pragma unroll
        for (uint32_t r = 0; r < kMaxTopK; ++r) sel[r] = s_sel[r];
    }
    if (wave == 0) {
        write_routes<NS>(a, sel, w.logit);
        uint32_t mine = 0u;
#pragma unroll
        for (uint32_t r = 0; r < kMaxTopK; ++r)
            if (lane == r) mine = sel[r];
        if (lane < K) atomicAdd(A.counts + mine, 1u);
    }
}

// ---------------------------------------------------------------------------
// 3. Grouping (one workgroup of 1024 threads).

constexpr uint32_t kGroupThreads = 1024;

__global__ __launch_bounds__(kGroupThreads) void k_group(MoePrefillArgs a) {
    __shared__ uint32_t cnt[kMaxExperts], off[kMaxExperts + 1], tb[kMaxExperts + 1],
        fill[kMaxExperts];
    const uint32_t E = a.layer.n_experts, K = a.layer.top_k, tid = threadIdx.x;
    if (tid < E) {
        cnt[tid] = a.counts[tid];
        a.counts[tid] = 0u;  // zero for the next call
        fill[tid] = 0u;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t o = 0, b = 0;
        for (uint32_t e = 0; e < E; ++e) {
            off[e] = o;
            tb[e] = b;
            o += cnt[e];
            b += (cnt[e] + kTileM - 1u) / kTileM;
        }
        off[E] = o;
        tb[E] = b;
        a.n_tiles[0] = b;
    }
    __syncthreads();
    if (tid <= E) a.offsets[tid] = off[tid];
    if (tid < E)
        for (uint32_t j = 0; j < (cnt[tid] + kTileM - 1u) / kTileM; ++j)
            a.tiles[tb[tid] + j] = (tid << 16) | j;
    // assignments t * top_k + r grouped by expert (order inside a group is
    // free: every row's result is independent of its neighbours)
    const uint32_t n = a.tokens * K;
    for (uint32_t i = tid; i < n; i += kGroupThreads) {
        const uint32_t e = a.ids[i];
        if (e < E) a.perm[off[e] + atomicAdd(&fill[e], 1u)] = i;
    }
}

// ---------------------------------------------------------------------------
// 4-5. Grouped GEMMs on MFMA.  A workgroup of 4 waves owns one 32-row tile
// of one expert and 128 output rows (32 per wave); K advances kChunk
// elements at a time: activations and dequantised weights are staged in LDS
// (the next chunk's loads are in flight while the MFMAs run on this one).

struct TileRef {
    uint32_t e, base, rows;  // expert, first grouped row, valid rows (<= kTileM)
};

__device__ __forceinline__ bool tile_ref(const MoePrefillArgs& a, TileRef& r) {
    if (blockIdx.x >= a.n_tiles[0]) return false;
    const uint32_t code = a.tiles[blockIdx.x];
    r.e = code >> 16;
    const uint32_t m0 = (code & 0xffffu) * kTileM;
    const uint32_t lo = a.offsets[r.e], hi = a.offsets[r.e + 1];
    r.base = lo + m0;
    r.rows = hi - r.base < kTileM ? hi - r.base : kTileM;
    return true;
}

constexpr uint32_t kLdsA = kChunk + 1;     // padded A row (tokens x K)
constexpr uint32_t kLdsB = kTileN + 4;     // padded B row (K x N)

template <int TG>
__global__ __launch_bounds__(256) void k_gate_up_mfma(MoePrefillArgs a) {
    __shared__ float As[kTileM * kLdsA];
    __shared__ float Bg[kChunk * kLdsB], Bu[kChunk * kLdsB];
    __shared__ const float* s_xrow[kTileM];
    TileRef tr;
    if (!tile_ref(a, tr)) return;  // uniform
    const MoeDecodeArgs& L = a.layer;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t H = L.hidden, K = L.top_k, n0 = blockIdx.y * kTileN;
    if (tid < kTileM) {
        const uint32_t i = tid < tr.rows ? tid : 0u;  // absent rows reuse row 0
        s_xrow[tid] = a.x + static_cast<uint64_t>(a.perm[tr.base + i] / K) * H;
    }
    __syncthreads();
    // this thread's staging jobs: A row tid / 8, 4 columns; B matrix tid / 128, row tid % 128
    const float* xrow = s_xrow[tid / 8u] + (tid % 8u) * 4u;
    const bool up_row = tid >= 128u;
    const uint8_t* wrow = (up_row ? L.up : L.gate) + static_cast<uint64_t>(tr.e) *
                                                       (up_row ? L.up_slice : L.gate_slice) +
                          static_cast<uint64_t>(n0 + (tid % 128u)) * (up_row ? L.up_row : L.gate_row);
    float* bdst = (up_row ? Bu : Bg) + (tid % 128u);

    f32x16 accg = {}, accu = {};
    float4 xa = *reinterpret_cast<const float4*>(xrow);
    Raw32<TG> raw;
    raw32_load<TG>(wrow, 0, raw);
    for (uint32_t k0 = 0; k0 < H; k0 += kChunk) {
        // stage chunk k0
        float* adst = As + (tid / 8u) * kLdsA + (tid % 8u) * 4u;
        adst[0] = xa.x;
        adst[1] = xa.y;
        adst[2] = xa.z;
        adst[3] = xa.w;
        float v[32];
        raw32_decode<TG>(raw, k0, v);
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) bdst[i * kLdsB] = v[i];
        __syncthreads();
        // next chunk's loads in flight during the MFMAs
        if (k0 + kChunk < H) {
            xa = *reinterpret_cast<const float4*>(xrow + k0 + kChunk);
            raw32_load<TG>(wrow, k0 + kChunk, raw);
        }
        const float* ap = As + (lane % 32u) * kLdsA + lane / 32u;
        const float* bgp = Bg + (lane / 32u) * kLdsB + wave * 32u + (lane % 32u);
        const float* bup = Bu + (lane / 32u) * kLdsB + wave * 32u + (lane % 32u);
#pragma unroll
        for (uint32_t kk = 0; kk < kChunk; kk += 2) {
            const float av = ap[kk];
            accg = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bgp[kk * kLdsB], accg, 0, 0, 0);
            accu = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bup[kk * kLdsB], accu, 0, 0, 0);
        }
        __syncthreads();
    }
    // epilogue: SwiGLU g / (1 + expf(-g)) * u (src/qwen3_moe_runner.cpp:682-684)
    const uint32_t col = n0 + wave * 32u + (lane % 32u);
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) {
        const uint32_t row = (r / 4u) * 8u + (lane / 32u) * 4u + (r % 4u);
        if (row < tr.rows) {
            const float g = accg[r], u = accu[r];
            a.act[static_cast<uint64_t>(tr.base + row) * L.ffn + col] = (g / (1.0f + expf(-g))) * u;
        }
    }
}

template <int TD>
__global__ __launch_bounds__(256) void k_down_mfma(MoePrefillArgs a) {
    __shared__ float As[kTileM * (2 * kChunk + 1)];
    __shared__ float Bd[2 * kChunk * kLdsB];
    TileRef tr;
    if (!tile_ref(a, tr)) return;  // uniform
    const MoeDecodeArgs& L = a.layer;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t F = L.ffn, H = L.hidden, n0 = blockIdx.y * kTileN;
    constexpr uint32_t KC = 2 * kChunk, LA = KC + 1;
    // staging jobs: A row tid / 8, 8 columns; B row tid % 128, half tid / 128
    const uint32_t arow = tid / 8u < tr.rows ? tid / 8u : 0u;
    const float* xrow = a.act + static_cast<uint64_t>(tr.base + arow) * F + (tid % 8u) * 8u;
    const uint32_t half = tid / 128u;
    const uint8_t* wrow = L.down + static_cast<uint64_t>(tr.e) * L.down_slice +
                          static_cast<uint64_t>(n0 + (tid % 128u)) * L.down_row;
    float* bdst = Bd + half * kChunk * kLdsB + (tid % 128u);

    f32x16 acc = {};
    float4 xa0 = *reinterpret_cast<const float4*>(xrow);
    float4 xa1 = *reinterpret_cast<const float4*>(xrow + 4);
    Raw32<TD> raw;
    raw32_load<TD>(wrow, half * kChunk, raw);
    for (uint32_t k0 = 0; k0 < F; k0 += KC) {
        float* adst = As + (tid / 8u) * LA + (tid % 8u) * 8u;
        adst[0] = xa0.x;
        adst[1] = xa0.y;
        adst[2] = xa0.z;
        adst[3] = xa0.w;
        adst[4] = xa1.x;
        adst[5] = xa1.y;
        adst[6] = xa1.z;
        adst[7] = xa1.w;
        float v[32];
        raw32_decode<TD>(raw, k0 + half * kChunk, v);
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) bdst[i * kLdsB] = v[i];
        __syncthreads();
        if (k0 + KC < F) {
            xa0 = *reinterpret_cast<const float4*>(xrow + k0 + KC);
            xa1 = *reinterpret_cast<const float4*>(xrow + k0 + KC + 4);
            raw32_load<TD>(wrow, k0 + KC + half * kChunk, raw);
        }
        const float* ap = As + (lane % 32u) * LA + lane / 32u;
        const float* bp = Bd + (lane / 32u) * kLdsB + wave * 32u + (lane % 32u);
#pragma unroll
        for (uint32_t kk = 0; kk < KC; kk += 2)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ap[kk], bp[kk * kLdsB], acc, 0, 0, 0);
        __syncthreads();
    }
    const uint32_t col = n0 + wave * 32u + (lane % 32u);
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) {
        const uint32_t row = (r / 4u) * 8u + (lane / 32u) * 4u + (r % 4u);
        if (row < tr.rows) {
            const uint32_t slot = a.perm[tr.base + row];  // token * top_k + route
            a.out[static_cast<uint64_t>(slot) * H + col] = acc[r];
        }
    }
}

// ---------------------------------------------------------------------------
// 6. Ordered combine.

__global__ __launch_bounds__(256) void k_combine(MoePrefillArgs a) {
    const uint32_t t = blockIdx.x, i = blockIdx.y * 256u + threadIdx.x;
    const uint32_t K = a.layer.top_k, H = a.layer.hidden, E = a.layer.n_experts;
    if (i >= H) return;
    bool ok = true;
    for (uint32_t r = 0; r < K; ++r) ok = ok && a.ids[t * K + r] < E;
    if (!ok) return;  // the router flagged this token
    float y = 0.0f;
    for (uint32_t r = 0; r < K; ++r)
        y = __fadd_rn(y, __fmul_rn(a.probs[t * K + r],
                                   a.out[(static_cast<uint64_t>(t) * K + r) * H + i]));
    a.y[static_cast<uint64_t>(t) * H + i] = y;
}

// ---------------------------------------------------------------------------
// Host side.

template <int T>
constexpr bool prefill_type() {
    return T == T_Q4_K || T == T_Q5_K || T == T_Q6_K || T == T_Q8_0 || T == T_Q4_0;
}

bool prefill_type_ok(uint32_t t) {
    return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_Q8_0 || t == T_Q4_0;
}

uint32_t ceil_div_u(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }

template <int TG>
hipError_t gate_up_mfma_t(const MoePrefillArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((k_gate_up_mfma<TG>), dim3(a.max_tiles, a.layer.ffn / kTileN), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int TD>
hipError_t down_mfma_t(const MoePrefillArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((k_down_mfma<TD>), dim3(a.max_tiles, a.layer.hidden / kTileN), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

uint32_t moe_prefill_max_tiles(uint32_t tokens, uint32_t top_k, uint32_t n_experts) {
    const uint32_t pairs = tokens * top_k;
    return pairs / kTileM + (n_experts < pairs ? n_experts : pairs);
}

bool moe_prefill_supported(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                           uint32_t hidden, uint32_t ffn, uint32_t n_experts, uint32_t top_k,
                           uint32_t tokens) {
    if (gate_type != up_type || !prefill_type_ok(gate_type) || !prefill_type_ok(down_type))
        return false;
    if (tokens == 0 || tokens > kMaxPrefillTokens) return false;
    if (hidden % 256u || ffn % 256u || hidden / 256u > 32u) return false;
    switch (hidden / 256u) {
        case 2: case 4: case 8: case 12: case 16: case 24: case 32: break;
        default: return false;
    }
    if (ffn % kTileN || hidden % kTileN || ffn % (2 * kChunk)) return false;
    return n_experts >= 1 && n_experts <= kMaxExperts && top_k >= 1 && top_k <= kMaxTopK &&
           top_k <= n_experts;
}

hipError_t launch_moe_prefill(const MoePrefillArgs& a, hipStream_t s) {
    const MoeDecodeArgs& L = a.layer;
    // 1. router
    const dim3 rgrid(L.n_experts, ceil_div_u(a.tokens, kRouterTokens));
    switch (L.hidden / kRouterThreads) {
#define PK_RB(C)                                                                              \
    case C:                                                                                   \
        hipLaunchKernelGGL(k_router_batch<C>, rgrid, dim3(kRouterThreads), 0, s, a);           \
        break;
        PK_RB(2) PK_RB(4) PK_RB(8) PK_RB(12) PK_RB(16) PK_RB(24) PK_RB(32)
#undef PK_RB
        default: return hipErrorInvalidValue;
    }
    // 2. ranking
    const size_t xlds = L.hidden * sizeof(float);
    switch (slots_for(L.n_experts)) {
        case 1: hipLaunchKernelGGL(k_route_batch<1>, dim3(a.tokens), dim3(256), xlds, s, a); break;
        case 2: hipLaunchKernelGGL(k_route_batch<2>, dim3(a.tokens), dim3(256), xlds, s, a); break;
        default: hipLaunchKernelGGL(k_route_batch<4>, dim3(a.tokens), dim3(256), xlds, s, a); break;
    }
    // 3. grouping
    hipLaunchKernelGGL(k_group, dim3(1), dim3(kGroupThreads), 0, s, a);
    // 4. gate/up
    hipError_t err = hipSuccess;
    switch (L.gate_type) {
        case T_Q4_K: err = gate_up_mfma_t<T_Q4_K>(a, s); break;
        case T_Q5_K: err = gate_up_mfma_t<T_Q5_K>(a, s); break;
        case T_Q6_K: err = gate_up_mfma_t<T_Q6_K>(a, s); break;
        case T_Q8_0: err = gate_up_mfma_t<T_Q8_0>(a, s); break;
        case T_Q4_0: err = gate_up_mfma_t<T_Q4_0>(a, s); break;
        default: return hipErrorInvalidValue;
    }
    if (err != hipSuccess) return err;
    // 5. down
    switch (L.down_type) {
        case T_Q4_K: err = down_mfma_t<T_Q4_K>(a, s); break;
        case T_Q5_K: err = down_mfma_t<T_Q5_K>(a, s); break;
        case T_Q6_K: err = down_mfma_t<T_Q6_K>(a, s); break;
        case T_Q8_0: err = down_mfma_t<T_Q8_0>(a, s); break;
        case T_Q4_0: err = down_mfma_t<T_Q4_0>(a, s); break;
        default: return hipErrorInvalidValue;
    }
    if (err != hipSuccess) return err;
    // 6. combine
    hipLaunchKernelGGL(k_combine, dim3(a.tokens, ceil_div_u(L.hidden, 256u)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace pk
