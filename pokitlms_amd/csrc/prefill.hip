// prefill.hip -- batched routed-MoE prefill on gfx950 (MFMA grouped GEMM).
//
// The reference prefills a prompt one token at a time through the MoE block
// of src/qwen3_moe_runner.cpp:643-692 (the loop at :785-790), so every
// token's routes and output are those of a single-token pass.  Here the
// whole batch goes through six launches:
//
//  1. k_router_batch: the logit value S and rounding bound B of every
//     (token, expert) pair (the decode router's arithmetic, one expert row
//     per wave held in registers across a tile of tokens).
//  2. k_route_batch: one workgroup per token ranks the experts exactly as the
//     decode path does (certified wave ranking, exact serial fallback) and
//     writes ids and route weights.
//  3. k_group: one workgroup counts each expert's tokens and lays out
//     per-expert row ranges, a list of 32-row tiles and the assignments
//     (token * top_k + route) grouped by expert; its other workgroups split
//     x into the gate/up GEMM's operands meanwhile.
//  4. k_expert_gemm<gate/up>: per tile and 128 ffn rows,
//     gate and up GEMMs on bf16 MFMA with exact products (x split into three
//     bf16 planes, the quantised weights as bf16 integers, the scales applied
//     per group outside the MFMA), and the SwiGLU epilogue, which writes the
//     activations already split for the down GEMM.  Q4_K and Q6_K weights go
//     from memory straight into the registers of the wave that uses them
//     (k_expert_gemm_w); the other formats are staged through LDS.
//  5. k_expert_gemm<down>: per tile and 128 hidden rows; each output row goes
//     to its (token, route) slot.
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
constexpr uint32_t kRouterTokens = 8;  // tokens per batched-router workgroup

// ---------------------------------------------------------------------------
// The quant fields of 32 consecutive elements k0 .. k0 + 31 (k0 % 32 == 0)
// of one GGUF row (block layouts of src/quantized_linear.cpp:166-205,
// 286-358, 387-423): loads first (Raw32), values later.

template <int T>
struct Raw32;
template <> struct Raw32<T_Q4_K> { uint32_t h[4]; uint32_t q[8]; };
template <> struct Raw32<T_Q5_K> { uint32_t h[4]; uint32_t q[8]; uint32_t qh[8]; };
// Q6_K, Q8_0 and Q4_0 are stored planar (layout.hpp): every field is an
// aligned load of its own.
template <> struct Raw32<T_Q6_K> { uint32_t ql[8], qh[8]; uint32_t sc, d; };
template <> struct Raw32<T_Q8_0> { uint32_t q[8]; uint32_t d; };
template <> struct Raw32<T_Q4_0> { uint32_t q[4]; uint32_t d; };
template <> struct Raw32<T_Q4_1> { uint32_t q[4]; uint32_t dm; };  // 20-byte blocks keep 4-byte alignment

__device__ __forceinline__ uint32_t ld_word(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(__builtin_assume_aligned(p, 4));
}

template <int T>
__device__ __forceinline__ void raw32_load(const QRow& row, uint32_t k0, Raw32<T>& r) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = block_ptr<Fmt<T>::BB>(row, k0 / 256u);
        const uint32_t j = (k0 % 256u) / 32u, chunk = j / 2u;
        ld_words<4>(blk, r.h);
        ld_words<8>(blk + (T == T_Q4_K ? 16u : 48u) + 32u * chunk, r.q);
        if constexpr (T == T_Q5_K) ld_words<8>(blk + 16u, r.qh);
    } else if constexpr (T == T_Q6_K) {
        using L = Planar<T_Q6_K>;
        const uint32_t b = k0 / 256u, c = (k0 % 256u) / 32u, half = c / 4u, g = c % 4u;
        ld_words<8>(field_ptr<L::QL, 128>(row, b) + 64u * half + 32u * (g & 1u), r.ql);
        ld_words<8>(field_ptr<L::QH, 64>(row, b) + 32u * half, r.qh);
        r.sc = ld_u16(field_ptr<L::SC, 16>(row, b) + 8u * half + 2u * g);  // int8 scales of both 16-halves
        r.d = ld_u16(field_ptr<L::D, 2>(row, b));
    } else if constexpr (T == T_Q8_0) {
        using L = Planar<T_Q8_0>;
        ld_words<8>(field_ptr<L::QS, 32>(row, k0 / 32u), r.q);
        r.d = ld_u16(field_ptr<L::D, 2>(row, k0 / 32u));
    } else if constexpr (T == T_Q4_1) {
        const uint8_t* blk = block_ptr<20>(row, k0 / 32u);
        r.dm = ld_word(blk);
        ld_words<4>(blk + 4u, r.q);
    } else {  // Q4_0
        using L = Planar<T_Q4_0>;
        ld_words<4>(field_ptr<L::QS, 16>(row, k0 / 32u), r.q);
        r.d = ld_u16(field_ptr<L::D, 2>(row, k0 / 32u));
    }
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, uint32_t i) {
    return (w[i >> 2] >> (8u * (i & 3u))) & 0xffu;
}

// The same 32 elements as bf16 bit patterns of their integer fields, two per
// dword (element 2i in the low half of bw[i]): each field is converted to
// float exactly (v_cvt_f32_ubyteN) and its upper half kept, which is exact
// for integers below 256.  Per scale group of the 32 (one group; two of 16
// for Q6_K) the reference's weight is w = ds * (f - o) - dm with f the
// unsigned field and o its offset, so the group's dot product with x is
// ds * sum(x * f) + cn * sum(x) with cn = -(dm + o * ds): K-quants o = 0
// (cn = -dm), Q6_K o = 32, Q4_0 o = 8, Q8_0 o = 128 (its int8 read as
// q + 128).

template <int T>
__device__ __forceinline__ void raw32_bf16(const Raw32<T>& r, uint32_t k0, uint32_t (&bw)[16],
                                           float (&ds)[2], float (&cn)[2]) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint32_t j = (k0 % 256u) / 32u, hi = j & 1u;
        const float d = half_bits_to_float(r.h[0] & 0xffffu);
        const float dmin = half_bits_to_float(r.h[0] >> 16);
        float sc, mn;
        kq_scale_min(r.h, j, sc, mn);
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            uint32_t q = (hi ? r.q[i] >> 4 : r.q[i]) & 0x0f0f0f0fu;
            if constexpr (T == T_Q5_K) q |= ((r.qh[i] >> j) & 0x01010101u) << 4;
            bf16_bytes(q, bw[2 * i], bw[2 * i + 1]);
        }
        ds[0] = ds[1] = __fmul_rn(d, sc);
        cn[0] = cn[1] = -__fmul_rn(dmin, mn);
    } else if constexpr (T == T_Q6_K) {
        const uint32_t c = (k0 % 256u) / 32u, g = c % 4u;
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const uint32_t ql = r.ql[i], qh = r.qh[i];
            const uint32_t nib = (g >= 2u ? ql >> 4 : ql) & 0x0f0f0f0fu;
            bf16_bytes(nib | (((qh >> (2u * g)) & 0x03030303u) << 4), bw[2 * i], bw[2 * i + 1]);
        }
        ds[0] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(r.sc & 0xffu)));
        ds[1] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(r.sc >> 8)));
        cn[0] = __fmul_rn(-32.0f, ds[0]);
        cn[1] = __fmul_rn(-32.0f, ds[1]);
    } else if constexpr (T == T_Q8_0) {
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i)
            bf16_bytes(r.q[i] ^ 0x80808080u, bw[2 * i], bw[2 * i + 1]);
        ds[0] = ds[1] = d;
        cn[0] = cn[1] = __fmul_rn(-128.0f, d);
    } else if constexpr (T == T_Q4_1) {  // w = d * q + m: ds = d, cn = m (o = 0)
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            bf16_bytes(r.q[i] & 0x0f0f0f0fu, bw[2 * i], bw[2 * i + 1]);
            bf16_bytes((r.q[i] >> 4) & 0x0f0f0f0fu, bw[8 + 2 * i], bw[9 + 2 * i]);
        }
        ds[0] = ds[1] = half_bits_to_float(r.dm & 0xffffu);
        cn[0] = cn[1] = half_bits_to_float(r.dm >> 16);
    } else {  // Q4_0: low nibbles are elements 0..15, high nibbles 16..31
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t q = r.q[i];
            bf16_bytes(q & 0x0f0f0f0fu, bw[2 * i], bw[2 * i + 1]);
            bf16_bytes((q >> 4) & 0x0f0f0f0fu, bw[8 + 2 * i], bw[9 + 2 * i]);
        }
        ds[0] = ds[1] = d;
        cn[0] = cn[1] = __fmul_rn(-8.0f, d);
    }
}

// ---------------------------------------------------------------------------
// 1. Batched router.

// Expert rows per wave: C = hidden / 256, so 4 * C router values per lane
// and row stay in registers.
template <int C>
constexpr uint32_t router_rows_per_wave() { return C <= 8 ? 4u : C <= 16 ? 2u : 1u; }

// Per (token, expert) the S and B of router_wave_sum_bound, from the same
// lane sums (so the decode path's bits).  Each wave holds R expert rows in
// registers and walks kRouterTokens tokens, reading each token's x once for
// its R rows (the next token's x while the current one is summed); the four
// waves of a workgroup take 4 R rows and the same tokens.  No barrier: the
// waves never wait for one another.
template <int C>
__global__ __launch_bounds__(256) void k_router_batch(MoePrefillArgs a) {
    constexpr uint32_t R = router_rows_per_wave<C>();
    const uint32_t E = a.layer.n_experts, ER = E + a.layer.variant, H = a.layer.hidden;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    // rows: the n_experts router rows, then (variant 1) the shared expert's gate
    const uint32_t e0 = (blockIdx.x * 4u + wave) * R;
    const uint32_t t0 = blockIdx.y * kRouterTokens;
    const uint32_t t1 = t0 + kRouterTokens < a.tokens ? t0 + kRouterTokens : a.tokens;
    rf32x4 w[R][C], xc[C];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
        const uint32_t ee = e0 + r < ER ? e0 + r : ER - 1u;  // rows past the end repeat the last, write nothing
        const float* row = ee < E ? a.layer.router + static_cast<uint64_t>(ee) * H : a.layer.shared_router;
        router_lane_load<C>(row, lane, w[r]);
    }
    router_lane_load<C>(a.x + static_cast<uint64_t>(t0) * H, lane, xc);
    for (uint32_t t = t0; t < t1; ++t) {
        // the next token's x (the last token reloads its own: unconditional)
        const uint32_t tn = t + 1u < t1 ? t + 1u : t;
        rf32x4 xn[C];
        router_lane_load<C>(a.x + static_cast<uint64_t>(tn) * H, lane, xn);
        __builtin_amdgcn_sched_barrier(0);  // the loads out before the sums wait
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            RouterLane<C> rl;
            double total, bound;
            router_lane_sums<C>(w[r], xc, rl);
            router_wave_sum_bound<C>(rl, total, bound);
            if (lane == 0 && e0 + r < ER) {
                a.row_sum[static_cast<uint64_t>(t) * ER + e0 + r] = total;
                a.row_bound[static_cast<uint64_t>(t) * ER + e0 + r] = bound;
            }
        }
#pragma unroll
        for (int j = 0; j < C; ++j) xc[j] = xn[j];
    }
}

// ---------------------------------------------------------------------------
// 2. Per-token ranking, route weights and expert counts.

template <int NS>
__global__ __launch_bounds__(256) void k_route_batch(MoePrefillArgs A) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [hidden]
    __shared__ FallbackShared<256> fb;
    __shared__ uint32_t s_sel[kMaxTopK];
    __shared__ uint32_t s_state;
    __shared__ double s_lo;
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t E = A.layer.n_experts, K = A.layer.top_k;
    MoeDecodeArgs a = A.layer;  // this token's view
    a.x = A.x + static_cast<uint64_t>(t) * a.hidden;
    a.row_sum = A.row_sum + static_cast<uint64_t>(t) * (E + a.variant);
    a.row_bound = A.row_bound + static_cast<uint64_t>(t) * (E + a.variant);
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
        exact_routes<4, 256>(a, s_lo, xs, fb, true);
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
    if (wave == 0) write_routes<NS>(a, sel, w.logit);
}

// ---------------------------------------------------------------------------
// 3. Split-bf16 operands.  Every FP32 value x is exactly hi + mid + lo with
// three bf16 values (8 significant bits each and FP32's exponent range:
// hi = RNE(x), mid = RNE(x - hi), lo = x - hi - mid, each difference exact).
// With the weights' integer fields as bf16 (raw32_bf16), every product of the
// expert GEMMs is exact in the FP32 accumulators of the bf16 MFMA; the
// per-group scales are applied outside it.  split_piece writes the three planes
// of `rows` x `cols` FP32 values and, per G consecutive values of a row,
// their sum (accumulated in FP64, rounded once).

template <uint32_t G>
__device__ __forceinline__ void split_piece(const float* __restrict__ src, uint32_t i,
                                            uint32_t pieces, uint16_t* __restrict__ parts,
                                            uint64_t plane, float* __restrict__ sums) {
    // i: this lane's 16-value piece (pairs of pieces in neighbouring lanes)
    const uint32_t ic = i < pieces ? i : pieces - 1u;    // every lane loads (and shuffles)
    const float4* sp = reinterpret_cast<const float4*>(src + static_cast<uint64_t>(ic) * 16u);
    float v[16];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const float4 f = sp[j];
        v[4 * j] = f.x;
        v[4 * j + 1] = f.y;
        v[4 * j + 2] = f.z;
        v[4 * j + 3] = f.w;
    }
    uint32_t ph[8], pm[8], pl[8];
    double sum = 0.0;
#pragma unroll
    for (uint32_t e = 0; e < 16; e += 2) {
        uint32_t h2[2], m2[2], l2[2];
#pragma unroll
        for (uint32_t t = 0; t < 2; ++t) {
            const float x = v[e + t];
            sum += static_cast<double>(x);
            h2[t] = bf16_rne_bits(x);
            const float r1 = x - __uint_as_float(h2[t] << 16);
            m2[t] = bf16_rne_bits(r1);
            const float r2 = r1 - __uint_as_float(m2[t] << 16);
            l2[t] = __float_as_uint(r2) >> 16;  // r2 has at most 8 significant bits
        }
        ph[e / 2] = h2[0] | (h2[1] << 16);
        pm[e / 2] = m2[0] | (m2[1] << 16);
        pl[e / 2] = l2[0] | (l2[1] << 16);
    }
    if constexpr (G == 32) sum += __shfl_xor(sum, 1);
    if (i >= pieces) return;
    uint4* d0 = reinterpret_cast<uint4*>(parts + static_cast<uint64_t>(i) * 16u);
    uint4* d1 = reinterpret_cast<uint4*>(parts + plane + static_cast<uint64_t>(i) * 16u);
    uint4* d2 = reinterpret_cast<uint4*>(parts + 2u * plane + static_cast<uint64_t>(i) * 16u);
    d0[0] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
    d0[1] = make_uint4(ph[4], ph[5], ph[6], ph[7]);
    d1[0] = make_uint4(pm[0], pm[1], pm[2], pm[3]);
    d1[1] = make_uint4(pm[4], pm[5], pm[6], pm[7]);
    d2[0] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
    d2[1] = make_uint4(pl[4], pl[5], pl[6], pl[7]);
    if (G == 16 || (i & 1u) == 0u) sums[i * 16u / G] = static_cast<float>(sum);
}

// ---------------------------------------------------------------------------
// 4. Grouping (workgroup 0, 1024 threads): per-expert counts from the
// ids (LDS atomics), row ranges, the 32-row tile list and the assignments
// (token * top_k + route) grouped by expert.  Tokens the router flagged
// (ids 0xffffffff) take no rows.

constexpr uint32_t kGroupThreads = 1024;

// Workgroup 0 groups; the others split x into the gate/up GEMM's operands
// (G: the gate/up format's scale group) while it does, since the grouping
// alone would leave the rest of the chip idle.
template <uint32_t G>
__global__ __launch_bounds__(kGroupThreads) void k_group(MoePrefillArgs a) {
    if (blockIdx.x > 0u) {
        const uint64_t plane = static_cast<uint64_t>(a.tokens) * a.layer.hidden;
        split_piece<G>(a.x, (blockIdx.x - 1u) * kGroupThreads + threadIdx.x,
                       static_cast<uint32_t>(plane / 16u), a.x_parts, plane, a.x_sums);
        return;
    }
    constexpr uint32_t NE = kMaxExperts + 1;  // + the shared expert (variant 1)
    __shared__ uint32_t cnt[NE], off[NE + 1], tb[NE + 1], fill[NE];
    const uint32_t E = a.layer.n_experts, K = a.layer.top_k, V = a.layer.variant, tid = threadIdx.x;
    const uint32_t EE = E + V, KR = K + V, n = a.tokens * K;
    if (tid < EE) {
        cnt[tid] = 0u;
        fill[tid] = 0u;
    }
    __syncthreads();
    for (uint32_t i = tid; i < n; i += kGroupThreads) {
        const uint32_t e = a.ids[i];
        if (e < E) atomicAdd(&cnt[e], 1u);
    }
    // the shared expert takes every token the router did not flag
    if (V)
        for (uint32_t t = tid; t < a.tokens; t += kGroupThreads)
            if (a.ids[t * K] < E) atomicAdd(&cnt[E], 1u);
    __syncthreads();
    if (tid < 64) {  // exclusive prefix of rows and tiles: PER experts a lane, one wave scan
        constexpr uint32_t PER = (NE + 63u) / 64u;
        uint32_t c[PER], tl[PER];
        double lc = 0.0, lt = 0.0;  // integer sums, exact in FP64
#pragma unroll
        for (uint32_t k = 0; k < PER; ++k) {
            const uint32_t e = tid * PER + k;
            c[k] = e < EE ? cnt[e] : 0u;
            tl[k] = (c[k] + kTileM - 1u) / kTileM;
            lc += static_cast<double>(c[k]);
            lt += static_cast<double>(tl[k]);
        }
        const double ic = wave_inclusive_scan(lc), it = wave_inclusive_scan(lt);
        uint32_t o = static_cast<uint32_t>(ic - lc), b = static_cast<uint32_t>(it - lt);
#pragma unroll
        for (uint32_t k = 0; k < PER; ++k) {
            const uint32_t e = tid * PER + k;
            if (e < EE) {
                off[e] = o;
                tb[e] = b;
            }
            o += c[k];
            b += tl[k];
        }
        if (tid == 63u) {
            off[EE] = static_cast<uint32_t>(ic);
            tb[EE] = static_cast<uint32_t>(it);
            a.n_tiles[0] = static_cast<uint32_t>(it);
        }
    }
    __syncthreads();
    if (tid <= EE) a.offsets[tid] = off[tid];
    if (tid < EE)
        for (uint32_t j = 0; j < (cnt[tid] + kTileM - 1u) / kTileM; ++j)
            a.tiles[tb[tid] + j] = (tid << 16) | j;
    // grouped rows hold slots token * (top_k + variant) + route (the shared
    // expert is route top_k); the order inside a group is free: every row's
    // result is independent
    for (uint32_t i = tid; i < n; i += kGroupThreads) {
        const uint32_t e = a.ids[i];
        if (e < E) a.perm[off[e] + atomicAdd(&fill[e], 1u)] = (i / K) * KR + i % K;
    }
    if (V)
        for (uint32_t t = tid; t < a.tokens; t += kGroupThreads)
            if (a.ids[t * K] < E) a.perm[off[E] + atomicAdd(&fill[E], 1u)] = t * KR + K;
}

// ---------------------------------------------------------------------------
// 5. Grouped GEMMs on bf16 MFMA (v_mfma_f32_32x32x16_bf16).  A workgroup of
// 4 waves owns one 32-row tile of one expert and 256 staged weight rows, two
// 32-row blocks per wave: 128 gate rows and the same 128 up rows, or 256
// down rows.  K advances one
// stage at a time through two LDS buffers: the three activation planes, the
// weights' integer fields as bf16, and per scale group the row scales ds, the bias
// coefficients cn and the activations' group sums.  Per group g and tile,
// P = sum over the three planes of A_part x q on MFMA, then acc += ds_g * P;
// the bias term sum_g xs_g * cn_g (two groups at a time) goes through a
// v_mfma_f32_32x32x2f32 into the same accumulator.

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct TileRef {
    uint32_t e, base, rows;  // expert, first grouped row, valid rows (<= kTileM)
};

__device__ __forceinline__ bool tile_ref(const MoePrefillArgs& a, uint32_t tile, TileRef& r) {
    if (tile >= a.n_tiles[0]) return false;
    const uint32_t code = a.tiles[tile];
    r.e = code >> 16;
    const uint32_t m0 = (code & 0xffffu) * kTileM;
    const uint32_t lo = a.offsets[r.e], hi = a.offsets[r.e + 1];
    r.base = lo + m0;
    r.rows = hi - r.base < kTileM ? hi - r.base : kTileM;
    return true;
}

// Workgroups go to the 8 XCDs round robin by linear id.  Block L runs on XCD
// L % 8; on each XCD, the blocks walk its tiles (tile % 8 == XCD) with all
// `nb` row blocks of one tile next to each other, so a tile's activations
// are fetched into that XCD's L2 once and the tiles that share an expert run
// there side by side.
__device__ __forceinline__ void xcd_tile(uint32_t nb, uint32_t& tile, uint32_t& yb) {
    const uint32_t L = blockIdx.x, xcd = L % 8u, slot = L / 8u;
    tile = 8u * (slot / nb) + xcd;
    yb = slot % nb;
}

template <int TW, bool DUAL>
struct GemmCfg {
    static constexpr uint32_t G = TW == T_Q6_K ? 16u : 32u;  // scale group
    static constexpr uint32_t NRW = 256u;                    // weight rows staged (2 x 128)
    static constexpr uint32_t PARTS = 256u / NRW;            // 32-value parts per row and stage
    static constexpr uint32_t KC = 32u * PARTS;              // K per stage
    static constexpr uint32_t NG = KC / G;                   // scale groups per stage
    static constexpr uint32_t GP = 32u / G;                  // groups per part
    static constexpr uint32_t SR = KC * 2u + 16u;            // LDS row stride (bytes)
    static constexpr uint32_t NQ = 3u * kTileM * KC / 8u;    // 16-byte activation pieces
};

template <int TW, bool DUAL>
struct alignas(16) GemmStage {
    using C = GemmCfg<TW, DUAL>;
    uint8_t a[3 * kTileM * C::SR];  // planes hi, mid, lo: [m][k]
    uint8_t b[C::NRW * C::SR];      // weights: [n][k]
    float xs[C::NG * kTileM];       // [g][m]
    float ds[C::NG * C::NRW];       // [g][n]
    float cn[C::NG * C::NRW];       // [g][n]
};

template <int TW, bool DUAL>
struct GemmPrefetch {
    Raw32<TW> raw;
    u32x4_t ap0, ap1;  // two 16-byte activation pieces (native vectors: they stay in registers)
    float xs;
};

// A thread's global sources (at k = 0) and LDS destinations, fixed for the
// whole K loop: activation pieces tid and tid + 256 of a stage's 384 (three
// planes x 32 rows x 4), and group sum tid.  Pieces and sums past the
// stage's count repeat the last one, so every thread loads and stores
// unconditionally (the duplicate stores write the same values to the same
// places).
template <int TW, bool DUAL>
struct GemmSrc {
    QRow wrow;
    const uint16_t *ap0, *ap1;
    uint32_t adst0, adst1;
    const float* xs;
    uint32_t xdst;
};

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_piece(const uint16_t* parts, uint64_t plane, uint32_t kdim,
                                           const uint32_t* arow, uint32_t q, const uint16_t*& src,
                                           uint32_t& dst) {
    using C = GemmCfg<TW, DUAL>;
    q = q < C::NQ ? q : C::NQ - 1u;
    const uint32_t p = q / (kTileM * C::KC / 8u), rem = q % (kTileM * C::KC / 8u);
    const uint32_t m = rem / (C::KC / 8u), kk = (rem % (C::KC / 8u)) * 8u;
    src = parts + p * plane + static_cast<uint64_t>(arow[m]) * kdim + kk;
    dst = (p * kTileM + m) * C::SR + kk * 2u;
}

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_src(GemmSrc<TW, DUAL>& g, const QRow& wrow,
                                         const uint16_t* parts, uint64_t plane, uint32_t kdim,
                                         const float* sums, const uint32_t* arow) {
    using C = GemmCfg<TW, DUAL>;
    static_assert(C::NQ > 256u && C::NQ <= 512u, "two activation pieces per thread");
    const uint32_t tid = threadIdx.x;
    g.wrow = wrow;
    gemm_piece<TW, DUAL>(parts, plane, kdim, arow, tid, g.ap0, g.adst0);
    gemm_piece<TW, DUAL>(parts, plane, kdim, arow, tid + 256u, g.ap1, g.adst1);
    const uint32_t t = tid < C::NG * kTileM ? tid : C::NG * kTileM - 1u;
    g.xs = sums + static_cast<uint64_t>(arow[t % kTileM]) * (kdim / C::G) + t / kTileM;
    g.xdst = t;
}

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_load_act(GemmPrefetch<TW, DUAL>& f, const GemmSrc<TW, DUAL>& g,
                                              uint32_t k0) {
    using C = GemmCfg<TW, DUAL>;
    f.ap0 = *reinterpret_cast<const u32x4_t*>(g.ap0 + k0);
    f.ap1 = *reinterpret_cast<const u32x4_t*>(g.ap1 + k0);
    f.xs = g.xs[k0 / C::G];
}

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_load(GemmPrefetch<TW, DUAL>& f, const GemmSrc<TW, DUAL>& g,
                                          uint32_t k0) {
    using C = GemmCfg<TW, DUAL>;
    raw32_load<TW>(g.wrow, k0 + 32u * (threadIdx.x / C::NRW), f.raw);
    f.ap0 = *reinterpret_cast<const u32x4_t*>(g.ap0 + k0);
    f.ap1 = *reinterpret_cast<const u32x4_t*>(g.ap1 + k0);
    f.xs = g.xs[k0 / C::G];
}

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_store_raw(GemmStage<TW, DUAL>& st, const Raw32<TW>& raw,
                                               const GemmPrefetch<TW, DUAL>& f,
                                               const GemmSrc<TW, DUAL>& g, uint32_t k0) {
    using C = GemmCfg<TW, DUAL>;
    const uint32_t tid = threadIdx.x, wr = tid % C::NRW, part = tid / C::NRW;
    uint32_t bw[16];
    float ds[2], cn[2];
    raw32_bf16<TW>(raw, k0 + 32u * part, bw, ds, cn);
    uint4* bd = reinterpret_cast<uint4*>(st.b + wr * C::SR + part * 64u);
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
        bd[j] = make_uint4(bw[4 * j], bw[4 * j + 1], bw[4 * j + 2], bw[4 * j + 3]);
#pragma unroll
    for (uint32_t q = 0; q < C::GP; ++q) {
        st.ds[(part * C::GP + q) * C::NRW + wr] = ds[q];
        st.cn[(part * C::GP + q) * C::NRW + wr] = cn[q];
    }
    *reinterpret_cast<u32x4_t*>(st.a + g.adst0) = f.ap0;
    *reinterpret_cast<u32x4_t*>(st.a + g.adst1) = f.ap1;
    st.xs[g.xdst] = f.xs;
}

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_store(GemmStage<TW, DUAL>& st, const GemmPrefetch<TW, DUAL>& f,
                                           const GemmSrc<TW, DUAL>& g, uint32_t k0) {
    gemm_store_raw<TW, DUAL>(st, f.raw, f, g, k0);
}

__device__ __forceinline__ bf16x8 lds_bf16x8(const uint8_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// One stage of one wave: tile rows m, staged weight rows n and n + 128 (gate
// and up rows, or two down row blocks).  Each scale group's MFMA sum is
// scaled into the accumulator as soon as it is complete.
template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_compute(const GemmStage<TW, DUAL>& st, f32x16& acc,
                                             f32x16& acc2) {
    using C = GemmCfg<TW, DUAL>;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t m = lane % 32u, kq = lane / 32u, n = wave * 32u + m;
    // bias term first: its MFMA result is long complete when the scaled
    // group sums are added below
#pragma unroll
    for (uint32_t gp = 0; gp < (C::NG + 1u) / 2u; ++gp) {
        const uint32_t gi = 2u * gp + kq;
        const bool ok = gi < C::NG;  // an odd group count pads with a zero group
        const uint32_t gc = ok ? gi : 0u;
        const float av = ok ? st.xs[gc * kTileM + m] : 0.0f;
        const float bv = st.cn[gc * C::NRW + n], bv2 = st.cn[gc * C::NRW + n + 128u];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv2, acc2, 0, 0, 0);
    }
    f32x16 P, Q;
#pragma unroll
    for (uint32_t h = 0; h < C::KC / 16u; ++h) {
        const uint32_t koff = (16u * h + 8u * kq) * 2u;
        const bf16x8 a0 = lds_bf16x8(st.a + (0u * kTileM + m) * C::SR + koff);
        const bf16x8 a1 = lds_bf16x8(st.a + (1u * kTileM + m) * C::SR + koff);
        const bf16x8 a2 = lds_bf16x8(st.a + (2u * kTileM + m) * C::SR + koff);
        const bf16x8 b = lds_bf16x8(st.b + n * C::SR + koff);
        const bf16x8 bu = lds_bf16x8(st.b + (n + 128u) * C::SR + koff);
        const bool first = (16u * h) % C::G == 0u, closes = (16u * h + 16u) % C::G == 0u;
        P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b, first ? f32x16{} : P, 0, 0, 0);
        Q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, bu, first ? f32x16{} : Q, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b, P, 0, 0, 0);
        Q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bu, Q, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b, P, 0, 0, 0);
        Q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bu, Q, 0, 0, 0);
        if (closes) {
            const uint32_t g = 16u * h / C::G;
            const float d = st.ds[g * C::NRW + n], du = st.ds[g * C::NRW + n + 128u];
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(d, P[r], acc[r]);
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) acc2[r] = __builtin_fmaf(du, Q[r], acc2[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_K / Q6_K weights: each wave streams its own rows into registers.
//
// A wave computes rows n (lane % 32) of its two 32-row matrices (gate and up,
// or the two down row blocks) and gives the MFMA its B operand straight from
// registers: lane (n, kq = lane / 32) holds, of every 32-value stage of its
// row, the elements 8kq .. 8kq + 7 (first MFMA of the stage) and
// 16 + 8kq .. 16 + 8kq + 7 (second), which is the B fragment of
// v_mfma_f32_32x32x16_bf16, and computes the row's scales itself.  Only the
// activation planes, which the four waves share, pass through LDS, so a
// workgroup needs a fraction of the LDS of the staged-weight kernel and more
// waves fit on a SIMD to hide each other's waits.
//
// A lane's unit is half a block (128 values, four stages) of one row:
//  * Q4_K: the 16-byte header and, of the half's two 32-byte nibble chunks,
//    bytes 8kq..8kq+7 and 16+8kq..16+8kq+7 of each (stage 2c of the half:
//    chunk c's low nibbles, stage 2c + 1: its high nibbles);
//  * Q6_K: bytes 8kq.. and 16+8kq.. of each of the half's two 32-byte ql runs
//    (stages g and g + 2 share run g & 1: low and high nibbles), of its 32 qh
//    bytes (all four stages: bits 2g, 2g + 1), its 8 int8 scales and d.
// A 32-byte run is loaded as one 16-byte piece per lane (lane kq: bytes
// 16kq..16kq+15, half the load instructions of two 8-byte pieces) and the two
// lanes of a row exchange the middle 8 bytes with v_permlane32_swap when a
// stage uses the run (run_words), not at the load, which would wait for it.
template <int T> struct WUnit;
template <> struct WUnit<T_Q4_K> { uint32_t h[4]; uint32_t q[8]; };
template <> struct WUnit<T_Q6_K> { uint32_t ql[8], qh[4], sc[2]; uint32_t d; };

// Words (bytes 8kq..8kq+7, then 16+8kq..16+8kq+7) of a 32-byte run loaded as
// lane kq's bytes 16kq..16kq+15 (w[0..3]): lanes 32-63 of the first operand
// of v_permlane32_swap trade with lanes 0-31 of the second.
__device__ __forceinline__ void run_words(const uint32_t* w, uint32_t (&o)[4]) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
    o[0] = s02[0];
    o[1] = s13[0];
    o[2] = s02[1];
    o[3] = s13[1];
}

__device__ __forceinline__ void ld8(const uint8_t* p, uint32_t& lo, uint32_t& hi) {
    const uint2 v = *reinterpret_cast<const uint2*>(__builtin_assume_aligned(p, 8));
    lo = v.x;
    hi = v.y;
}

// Unit u of the row (block u / 2, half u % 2) for lanes kq.  Without HEAD the
// fields the block's two halves share (Q4_K: the header; Q6_K: d) are left to
// the caller, who copies them from the block's other unit.
template <int T, bool HEAD = true>
__device__ __forceinline__ void wunit_load(const QRow& row, uint32_t u, uint32_t kq, WUnit<T>& U) {
    const uint32_t b = u / 2u, hh = u % 2u;
    if constexpr (T == T_Q4_K) {
        const uint8_t* blk = block_ptr<144>(row, b);
        if constexpr (HEAD) ld_words<4>(blk, U.h);
        const uint8_t* qs = blk + 16u + 64u * hh + 16u * kq;
        ld_words<4>(qs, *reinterpret_cast<uint32_t(*)[4]>(&U.q[0]));
        ld_words<4>(qs + 32u, *reinterpret_cast<uint32_t(*)[4]>(&U.q[4]));
    } else {
        using L = Planar<T_Q6_K>;
        const uint8_t* ql = field_ptr<L::QL, 128>(row, b) + 64u * hh + 16u * kq;
        ld_words<4>(ql, *reinterpret_cast<uint32_t(*)[4]>(&U.ql[0]));
        ld_words<4>(ql + 32u, *reinterpret_cast<uint32_t(*)[4]>(&U.ql[4]));
        ld_words<4>(field_ptr<L::QH, 64>(row, b) + 32u * hh + 16u * kq, U.qh);
        ld8(field_ptr<L::SC, 16>(row, b) + 8u * hh, U.sc[0], U.sc[1]);
        if constexpr (HEAD) U.d = ld_u16(field_ptr<L::D, 2>(row, b));
    }
}

// The fields of a block that its two halves share.
template <int T>
__device__ __forceinline__ void wunit_share(const WUnit<T>& from, WUnit<T>& to) {
    if constexpr (T == T_Q4_K) {
#pragma unroll
        for (int i = 0; i < 4; ++i) to.h[i] = from.h[i];
    } else {
        to.d = from.d;
    }
}

// Stage j (0..3) of the unit in half hh of its block: the lane's two bf16x8
// B fragments, the scale of each (Q4_K: one scale group per stage, Q6_K: one
// per fragment) and the bias operand cb of scale group kq of the stage (of
// its single group for Q4_K).  Weights are ds * f + cn per group as in
// raw32_bf16; the fragments hold 128 + f (bf16_bytes_b128), so
// cb = cn - 128 ds.
template <int T>
__device__ __forceinline__ void wunit_stage(const WUnit<T>& U, uint32_t hh, uint32_t j, uint32_t kq,
                                            bf16x8 (&b)[2], float (&ds)[2], float& cb) {
    uint32_t w[8];
    if constexpr (T == T_Q4_K) {
        const uint32_t c = j / 2u, hi = j & 1u;
        uint32_t qc[4];
        run_words(&U.q[4u * c], qc);
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t q = (hi ? qc[i] >> 4 : qc[i]) & 0x0f0f0f0fu;
            bf16_bytes_b128(q, w[2u * i], w[2u * i + 1u]);
        }
        const float d = half_bits_to_float(U.h[0] & 0xffffu);
        const float dmin = half_bits_to_float(U.h[0] >> 16);
        float sc, mn;
        kq_scale_min(U.h, 4u * hh + j, sc, mn);
        ds[0] = ds[1] = __fmul_rn(d, sc);
        cb = -__fmaf_rn(128.0f, ds[0], __fmul_rn(dmin, mn));  // every lane: see gemm_compute_w
    } else {
        const uint32_t r = 4u * (j & 1u), sh = j >= 2u ? 4u : 0u;
        uint32_t ql[4], qh[4];
        run_words(&U.ql[r], ql);
        run_words(U.qh, qh);
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t nib = (ql[i] >> sh) & 0x0f0f0f0fu;
            const uint32_t hb = ((qh[i] >> (2u * j)) & 0x03030303u) << 4;
            bf16_bytes_b128(nib | hb, w[2u * i], w[2u * i + 1u]);
        }
        const float d = half_bits_to_float(U.d);
        const uint32_t s2 = (U.sc[j / 2u] >> (16u * (j & 1u))) & 0xffffu;  // scales of the two halves
        ds[0] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s2 & 0xffu)));
        ds[1] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s2 >> 8)));
        cb = __fmul_rn(-160.0f, kq ? ds[1] : ds[0]);  // (q - 32) * ds as (128 + q) * ds - 160 ds
    }
    b[0] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
    b[1] = __builtin_bit_cast(bf16x8, make_uint4(w[4], w[5], w[6], w[7]));
}

// The register-weight kernel's activation loads per stage, with no duplicate
// loads: the stage's 384 pieces go to pieces tid (every thread) and tid + 256
// (waves 0 and 1), its group sums to wave 2 (lane t: sum t, clamped).  The
// branches are uniform per wave.
template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_src_w(GemmSrc<TW, DUAL>& g, const QRow& wrow,
                                           const uint16_t* parts, uint64_t plane, uint32_t kdim,
                                           const float* sums, const uint32_t* arow) {
    using C = GemmCfg<TW, DUAL>;
    static_assert(C::NQ == 384u, "pieces tid and, in waves 0 and 1, tid + 256");
    static_assert(C::NG * kTileM <= 64u, "one wave of group sums");
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    g.wrow = wrow;
    gemm_piece<TW, DUAL>(parts, plane, kdim, arow, tid, g.ap0, g.adst0);
    gemm_piece<TW, DUAL>(parts, plane, kdim, arow, tid + 256u, g.ap1, g.adst1);
    const uint32_t t = lane < C::NG * kTileM ? lane : C::NG * kTileM - 1u;
    g.xs = sums + static_cast<uint64_t>(arow[t % kTileM]) * (kdim / C::G) + t / kTileM;
    g.xdst = t;
}

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_load_act_w(GemmPrefetch<TW, DUAL>& f, const GemmSrc<TW, DUAL>& g,
                                                uint32_t k0) {
    using C = GemmCfg<TW, DUAL>;
    const uint32_t wave = threadIdx.x >> 6;
    f.ap0 = *reinterpret_cast<const u32x4_t*>(g.ap0 + k0);
    if (wave < 2u) f.ap1 = *reinterpret_cast<const u32x4_t*>(g.ap1 + k0);
    if (wave == 2u) f.xs = g.xs[k0 / C::G];
}

// Activation planes and group sums of one stage, shared by the workgroup.
template <int TW, bool DUAL>
struct alignas(16) GemmStageA {
    using C = GemmCfg<TW, DUAL>;
    uint8_t a[3 * kTileM * C::SR];  // planes hi, mid, lo: [m][k]
    float xs[C::NG * kTileM];       // [g][m]
};

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_store_a(GemmStageA<TW, DUAL>& st, const GemmPrefetch<TW, DUAL>& f,
                                             const GemmSrc<TW, DUAL>& g) {
    const uint32_t wave = threadIdx.x >> 6;
    *reinterpret_cast<u32x4_t*>(st.a + g.adst0) = f.ap0;
    if (wave < 2u) *reinterpret_cast<u32x4_t*>(st.a + g.adst1) = f.ap1;
    if (wave == 2u) st.xs[g.xdst] = f.xs;
}

// One stage of one wave from register weights: the bias MFMA, then per
// fragment h the three plane MFMAs; each scale group's sum is scaled into the
// accumulator when it closes.  The bias MFMA (K = 2: lanes kq hold group kq)
// covers the stage's two groups (Q6_K) or, for one group per stage (Q4_K),
// the groups of stages j - 1 and j at odd j: even stages keep their group
// sum and bias operands in bias_prev.
struct BiasPrev {
    float av, c0, c1;
};

template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_compute_w(const GemmStageA<TW, DUAL>& st, const WUnit<TW>& U0,
                                               const WUnit<TW>& U1, uint32_t hh, uint32_t j,
                                               f32x16& acc, f32x16& acc2, BiasPrev& bp) {
    using C = GemmCfg<TW, DUAL>;
    const uint32_t lane = threadIdx.x & 63u, m = lane % 32u, kq = lane / 32u;
    bf16x8 b0[2], b1[2];
    float d0[2], d1[2], c0, c1;
    wunit_stage<TW>(U0, hh, j, kq, b0, d0, c0);
    wunit_stage<TW>(U1, hh, j, kq, b1, d1, c1);
    if constexpr (C::NG == 1u) {
        const float av = st.xs[m];
        if ((j & 1u) == 0u) {
            bp.av = av;
            bp.c0 = c0;
            bp.c1 = c1;
        } else {
            const float a2 = kq ? av : bp.av;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a2, kq ? c0 : bp.c0, acc, 0, 0, 0);
            acc2 = __builtin_amdgcn_mfma_f32_32x32x2f32(a2, kq ? c1 : bp.c1, acc2, 0, 0, 0);
        }
    } else {
        const float av = st.xs[kq * kTileM + m];
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, c0, acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_32x32x2f32(av, c1, acc2, 0, 0, 0);
    }
    f32x16 P, Q;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t koff = (16u * h + 8u * kq) * 2u;
        const bf16x8 a0 = lds_bf16x8(st.a + (0u * kTileM + m) * C::SR + koff);
        const bf16x8 a1 = lds_bf16x8(st.a + (1u * kTileM + m) * C::SR + koff);
        const bf16x8 a2 = lds_bf16x8(st.a + (2u * kTileM + m) * C::SR + koff);
        const bool first = C::G == 16u || h == 0u;
        P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b0[h], first ? f32x16{} : P, 0, 0, 0);
        Q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2, b1[h], first ? f32x16{} : Q, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0[h], P, 0, 0, 0);
        Q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1[h], Q, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0[h], P, 0, 0, 0);
        Q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1[h], Q, 0, 0, 0);
        if (C::G == 16u || h == 1u) {
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(d0[h], P[r], acc[r]);
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) acc2[r] = __builtin_fmaf(d1[h], Q[r], acc2[r]);
        }
    }
}

// The tile's results: DUAL, the SwiGLU activations split for the down GEMM;
// otherwise each output row to its (token, route) slot.
template <int TW, bool DUAL>
__device__ __forceinline__ void gemm_epilogue(const MoePrefillArgs& a, const TileRef& tr, uint32_t n0,
                                              const uint32_t* oslot, const f32x16& acc,
                                              const f32x16& acc2) {
    const MoeDecodeArgs& L = a.layer;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t ndim = DUAL ? L.ffn : L.hidden;
    const uint32_t col = n0 + wave * 32u + (lane % 32u);
    if constexpr (DUAL) {
        // SwiGLU g / (1 + expf(-g)) * u (src/qwen3_moe_runner.cpp:682-684);
        // variant 1: silu(g) * u (src/qwen35_runner.cpp:111-123).  The value goes
        // straight into the down GEMM's operands, as split_piece writes x:
        // three exact bf16 parts and, per scale group of the down format (16
        // values for Q6_K, else 32: consecutive columns, so consecutive lanes),
        // the FP64 sum of the group rounded once.  Absent rows (they repeat a
        // real row) join the lane sums but are not stored.
        const uint32_t gd = L.down_type == T_Q6_K ? 16u : 32u;
        const uint64_t plane = static_cast<uint64_t>(a.tokens) * (L.top_k + L.variant) * ndim;
#pragma unroll
        for (uint32_t r = 0; r < 16; ++r) {
            const uint32_t row = (r / 4u) * 8u + (lane / 32u) * 4u + (r % 4u);
            const float g = acc[r], u = acc2[r];
            const float v = L.variant ? silu(g) * u : (g / (1.0f + expf(-g))) * u;
            const uint32_t h = bf16_rne_bits(v);
            const float r1 = v - __uint_as_float(h << 16);
            const uint32_t m = bf16_rne_bits(r1);
            const float r2 = r1 - __uint_as_float(m << 16);  // at most 8 significant bits
            const double sv = static_cast<double>(v);
            const double gs = gd == 16u ? group_sum<16>(sv) : group_sum<32>(sv);
            if (row < tr.rows) {
                const uint64_t e = static_cast<uint64_t>(tr.base + row) * ndim + col;
                a.act_parts[e] = static_cast<uint16_t>(h);
                a.act_parts[plane + e] = static_cast<uint16_t>(m);
                a.act_parts[2u * plane + e] = static_cast<uint16_t>(__float_as_uint(r2) >> 16);
                if (col % gd == gd - 1u)
                    a.act_sums[static_cast<uint64_t>(tr.base + row) * (ndim / gd) + col / gd] =
                        static_cast<float>(gs);
            }
        }
    } else {
#pragma unroll
        for (uint32_t r = 0; r < 16; ++r) {
            const uint32_t row = (r / 4u) * 8u + (lane / 32u) * 4u + (r % 4u);
            if (row < tr.rows) {
                float* o = a.out + static_cast<uint64_t>(oslot[row]) * ndim + col;
                o[0] = acc[r];
                o[kTileN] = acc2[r];
            }
        }
    }
}

// DUAL: gate/up over x (token rows), SwiGLU into act (grouped rows).
// Otherwise: down over act, each row to its (token, route) slot of out.
// Global loads run two stages ahead of the MFMAs (two register sets), LDS
// holds two stages.
template <int TW, bool DUAL>
__global__ __launch_bounds__(256, 2) void k_expert_gemm(MoePrefillArgs a) {
    using C = GemmCfg<TW, DUAL>;
    __shared__ GemmStage<TW, DUAL> st[2];
    __shared__ uint32_t arow[kTileM], oslot[kTileM];
    const MoeDecodeArgs& L = a.layer;
    const uint32_t kdim = DUAL ? L.hidden : L.ffn, ndim = DUAL ? L.ffn : L.hidden;
    const uint32_t nblk = DUAL ? kTileN : 2u * kTileN;  // output rows per workgroup
    uint32_t tile, yb;
    xcd_tile(ndim / nblk, tile, yb);
    TileRef tr;
    if (!tile_ref(a, tile, tr)) return;  // uniform
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n0 = yb * nblk;
    if (tid < kTileM) {
        const uint32_t i = tid < tr.rows ? tid : tr.rows - 1u;  // absent rows repeat a real one
        const uint32_t slot = a.perm[tr.base + i];  // token * top_k + route
        arow[tid] = DUAL ? slot / (L.top_k + L.variant) : tr.base + i;
        oslot[tid] = slot;
    }
    const uint32_t wr = tid % C::NRW;
    const bool sh = tr.e >= L.n_experts;  // the shared expert (variant 1): its own tensors
    // the slice, its blocks and the row's first block (gate/up rows have hidden
    // elements, down rows ffn)
    const uint32_t rnb = kdim / Fmt<TW>::BE;
    QRow wrow;
    if constexpr (DUAL) {
        wrow.slice = wr < 128u ? (sh ? L.shared_gate : L.gate + static_cast<uint64_t>(tr.e) * L.gate_slice)
                               : (sh ? L.shared_up : L.up + static_cast<uint64_t>(tr.e) * L.up_slice);
        wrow.nblk = static_cast<uint64_t>(L.ffn) * rnb;
        wrow.blk0 = static_cast<uint64_t>(wr < 128u ? n0 + wr : n0 + wr - 128u) * rnb;
    } else {  // rows n0 .. n0 + 255
        wrow.slice = sh ? L.shared_down : L.down + static_cast<uint64_t>(tr.e) * L.down_slice;
        wrow.nblk = static_cast<uint64_t>(L.hidden) * rnb;
        wrow.blk0 = static_cast<uint64_t>(n0 + wr) * rnb;
    }
    const uint16_t* parts = DUAL ? a.x_parts : a.act_parts;
    const uint64_t plane = DUAL ? static_cast<uint64_t>(a.tokens) * L.hidden
                                : static_cast<uint64_t>(a.tokens) * (L.top_k + L.variant) * L.ffn;
    const float* sums = DUAL ? a.x_sums : a.act_sums;
    __syncthreads();
    GemmSrc<TW, DUAL> src;
    gemm_src<TW, DUAL>(src, wrow, parts, plane, kdim, sums, arow);

    const uint32_t nst = kdim / C::KC, last = nst - 1u;
    auto stage_k = [&](uint32_t s) { return (s < last ? s : last) * C::KC; };  // tail: harmless reloads
    GemmPrefetch<TW, DUAL> f0, f1;
    f32x16 acc = {}, acc2 = {};
    gemm_load<TW, DUAL>(f0, src, 0u);
    gemm_load<TW, DUAL>(f1, src, stage_k(1u));
    gemm_store<TW, DUAL>(st[0], f0, src, 0u);
    gemm_load<TW, DUAL>(f0, src, stage_k(2u));
    __syncthreads();
    // Stage j's loads live in f(j % 2); step s computes stage s, stages s + 1
    // and loads s + 3.  The steps carry no conditions, so the load counters
    // the compiler tracks stay exact across the loop (two sets in flight).
    auto step = [&](uint32_t s, GemmPrefetch<TW, DUAL>& f) {
        gemm_compute<TW, DUAL>(st[s & 1u], acc, acc2);
        gemm_store<TW, DUAL>(st[(s + 1u) & 1u], f, src, (s + 1u) * C::KC);
        gemm_load<TW, DUAL>(f, src, stage_k(s + 3u));
        __syncthreads();
    };
    uint32_t s = 0;
    for (; s + 2u < nst; s += 2u) {
        step(s, f1);
        step(s + 1u, f0);
    }
    if (s + 1u < nst) step(s++, f1);
    gemm_compute<TW, DUAL>(st[s & 1u], acc, acc2);
    gemm_epilogue<TW, DUAL>(a, tr, n0, oslot, acc, acc2);
}

// Activation stages in flight in k_expert_gemm_w: four register sets (246
// VGPRs, still two waves per SIMD) took the Zipf batch's gate/up GEMM from
// 200.6-203.8 to 196.2-197.1 us and down from 140.2-141.5 to 136.6-137.4 us
// against two sets on one box; eight spill.
constexpr uint32_t kActSets = 4;

// Q4_K and Q6_K weights: the same tiles and results as k_expert_gemm, with
// each wave's weight rows in registers (half-block units, one unit ahead) and
// only the activation planes staged through LDS (two stages; their global
// loads run two stages ahead).
template <int TW, bool DUAL>
__global__ __launch_bounds__(256, 2) void k_expert_gemm_w(MoePrefillArgs a) {
    using C = GemmCfg<TW, DUAL>;
    __shared__ GemmStageA<TW, DUAL> st[2];
    __shared__ uint32_t arow[kTileM], oslot[kTileM];
    const MoeDecodeArgs& L = a.layer;
    const uint32_t kdim = DUAL ? L.hidden : L.ffn, ndim = DUAL ? L.ffn : L.hidden;
    const uint32_t nblk = DUAL ? kTileN : 2u * kTileN;  // output rows per workgroup
    uint32_t tile, yb;
    xcd_tile(ndim / nblk, tile, yb);
    TileRef tr;
    if (!tile_ref(a, tile, tr)) return;  // uniform
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n0 = yb * nblk, kq = lane / 32u;
    if (tid < kTileM) {
        const uint32_t i = tid < tr.rows ? tid : tr.rows - 1u;  // absent rows repeat a real one
        const uint32_t slot = a.perm[tr.base + i];  // token * top_k + route
        arow[tid] = DUAL ? slot / (L.top_k + L.variant) : tr.base + i;
        oslot[tid] = slot;
    }
    const bool sh = tr.e >= L.n_experts;  // the shared expert (variant 1): its own tensors
    const uint32_t rnb = kdim / Fmt<TW>::BE;
    const uint32_t r = n0 + wave * 32u + lane % 32u;  // this lane's row of matrix 0
    QRow w0, w1;
    if constexpr (DUAL) {  // gate row r, up row r
        w0 = QRow{sh ? L.shared_gate : L.gate + static_cast<uint64_t>(tr.e) * L.gate_slice,
                  static_cast<uint64_t>(L.ffn) * rnb, static_cast<uint64_t>(r) * rnb};
        w1 = QRow{sh ? L.shared_up : L.up + static_cast<uint64_t>(tr.e) * L.up_slice,
                  static_cast<uint64_t>(L.ffn) * rnb, static_cast<uint64_t>(r) * rnb};
    } else {  // down rows r and r + 128
        const uint8_t* base = sh ? L.shared_down : L.down + static_cast<uint64_t>(tr.e) * L.down_slice;
        w0 = QRow{base, static_cast<uint64_t>(L.hidden) * rnb, static_cast<uint64_t>(r) * rnb};
        w1 = QRow{base, static_cast<uint64_t>(L.hidden) * rnb, static_cast<uint64_t>(r + kTileN) * rnb};
    }
    const uint32_t nu = kdim / 128u, lastu = nu - 1u;  // units per row
    WUnit<TW> ua0, ua1, ub0, ub1;  // matrices 0 and 1: units 2i (a) and 2i + 1 (b)
    // units a and b are the two halves of one block (clamped units stay in
    // the last block): b takes the shared fields from a
    wunit_load<TW>(w0, 0u, kq, ua0);
    wunit_load<TW>(w1, 0u, kq, ua1);
    wunit_load<TW, false>(w0, 1u < lastu ? 1u : lastu, kq, ub0);
    wunit_load<TW, false>(w1, 1u < lastu ? 1u : lastu, kq, ub1);
    wunit_share<TW>(ua0, ub0);
    wunit_share<TW>(ua1, ub1);
    const uint16_t* parts = DUAL ? a.x_parts : a.act_parts;
    const uint64_t plane = DUAL ? static_cast<uint64_t>(a.tokens) * L.hidden
                                : static_cast<uint64_t>(a.tokens) * (L.top_k + L.variant) * L.ffn;
    const float* sums = DUAL ? a.x_sums : a.act_sums;
    __syncthreads();
    GemmSrc<TW, DUAL> src;
    gemm_src_w<TW, DUAL>(src, w0, parts, plane, kdim, sums, arow);
    const uint32_t nst = kdim / C::KC, last = nst - 1u;  // a multiple of 8 (kdim % 256 == 0)
    auto stage_k = [&](uint32_t s) { return (s < last ? s : last) * C::KC; };  // tail: harmless reloads
    // kActSets register sets of activation loads in flight: stage s's live in
    // f[s % kActSets]; step s computes stage s, stores stage s + 1 and loads
    // stage s + 1 + kActSets into the set it freed.
    GemmPrefetch<TW, DUAL> f[kActSets];
#pragma unroll
    for (uint32_t i = 0; i < kActSets; ++i) gemm_load_act_w<TW, DUAL>(f[i], src, stage_k(i));
    gemm_store_a<TW, DUAL>(st[0], f[0], src);
    gemm_load_act_w<TW, DUAL>(f[0], src, stage_k(kActSets));
    __syncthreads();
    f32x16 acc = {}, acc2 = {};
    BiasPrev bp{0.0f, 0.0f, 0.0f};
    // Steps 0-3 of an iteration use units a, steps 4-7 units b; each buffer
    // reloads (two units on) after its last step, four steps before its next
    // use.
    for (uint32_t s0 = 0; s0 < nst; s0 += 8u) {
        const uint32_t u0 = s0 / 4u;
#pragma unroll
        for (uint32_t t = 0; t < 8u; ++t) {
            const uint32_t s = s0 + t;
            GemmPrefetch<TW, DUAL>& fs = f[(t + 1u) % kActSets];
            if (t < 4u) gemm_compute_w<TW, DUAL>(st[s & 1u], ua0, ua1, 0u, t, acc, acc2, bp);
            else gemm_compute_w<TW, DUAL>(st[s & 1u], ub0, ub1, 1u, t - 4u, acc, acc2, bp);
            gemm_store_a<TW, DUAL>(st[(s + 1u) & 1u], fs, src);
            gemm_load_act_w<TW, DUAL>(fs, src, stage_k(s + 1u + kActSets));
            if (t == 3u) {
                const uint32_t un = u0 + 2u < lastu ? u0 + 2u : lastu;
                wunit_load<TW>(w0, un, kq, ua0);
                wunit_load<TW>(w1, un, kq, ua1);
            }
            if (t == 7u) {
                const uint32_t un = u0 + 3u < lastu ? u0 + 3u : lastu;
                wunit_load<TW, false>(w0, un, kq, ub0);
                wunit_load<TW, false>(w1, un, kq, ub1);
                wunit_share<TW>(ua0, ub0);  // ua holds unit u0 + 2, of the same block
                wunit_share<TW>(ua1, ub1);
            }
            __syncthreads();
        }
    }
    gemm_epilogue<TW, DUAL>(a, tr, n0, oslot, acc, acc2);
}

// ---------------------------------------------------------------------------
// 6. Ordered combine.

// Four consecutive outputs per thread (hidden is a multiple of 256), every
// route's loads issued before the ordered sums.
__global__ __launch_bounds__(256) void k_combine(MoePrefillArgs a) {
    const uint32_t t = blockIdx.x, i = (blockIdx.y * 256u + threadIdx.x) * 4u;
    const uint32_t K = a.layer.top_k, H = a.layer.hidden, E = a.layer.n_experts;
    const uint32_t V = a.layer.variant, KR = K + V;
    if (i >= H) return;
    bool ok = true;
    for (uint32_t r = 0; r < K; ++r) ok = ok && a.ids[t * K + r] < E;
    if (!ok) return;  // the router flagged this token
    rf32x4 o[kMaxTopK + 1];
    float p[kMaxTopK + 1];
#pragma unroll
    for (uint32_t r = 0; r < kMaxTopK + 1; ++r) {
        const uint32_t rr = r < KR ? r : 0u;  // routes past the last re-read route 0 (unused)
        o[r] = *reinterpret_cast<const rf32x4*>(a.out + (static_cast<uint64_t>(t) * KR + rr) * H + i);
        p[r] = r < K ? a.probs[t * K + rr] : 0.0f;
    }
    rf32x4 y = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t r = 0; r < kMaxTopK; ++r) {
        if (r < K) {
            y.x = __fadd_rn(y.x, __fmul_rn(p[r], o[r].x));
            y.y = __fadd_rn(y.y, __fmul_rn(p[r], o[r].y));
            y.z = __fadd_rn(y.z, __fmul_rn(p[r], o[r].z));
            y.w = __fadd_rn(y.w, __fmul_rn(p[r], o[r].w));
        }
    }
    if (V) {  // mixer_output = moe_result + sigmoid(shared gate) * shared (src/qwen35_runner.cpp:752-761)
        const float g = sigmoid35(static_cast<float>(a.row_sum[static_cast<uint64_t>(t) * (E + 1u) + E]));
        rf32x4 sh = o[0];
#pragma unroll
        for (uint32_t r = 1; r < kMaxTopK + 1; ++r) sh = r == K ? o[r] : sh;
        y.x = __fadd_rn(y.x, __fmul_rn(g, sh.x));
        y.y = __fadd_rn(y.y, __fmul_rn(g, sh.y));
        y.z = __fadd_rn(y.z, __fmul_rn(g, sh.z));
        y.w = __fadd_rn(y.w, __fmul_rn(g, sh.w));
    }
    *reinterpret_cast<rf32x4*>(a.y + static_cast<uint64_t>(t) * H + i) = y;
}

// ---------------------------------------------------------------------------
// Host side.

bool prefill_type_ok(uint32_t t) {
    return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_Q8_0 || t == T_Q4_0 || t == T_Q4_1;
}

uint32_t ceil_div_u(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }

template <int TW, bool DUAL>
hipError_t expert_gemm_t(const MoePrefillArgs& a, hipStream_t s) {
    const MoeDecodeArgs& L = a.layer;
    // (x is split beside the grouping, the activations by the gate/up epilogue)
    const uint32_t nb = DUAL ? L.ffn / kTileN : L.hidden / (2u * kTileN);
    const uint32_t blocks = 8u * ceil_div_u(a.max_tiles, 8u) * nb;  // xcd_tile's layout
    if constexpr (TW == T_Q4_K || TW == T_Q6_K)
        hipLaunchKernelGGL((k_expert_gemm_w<TW, DUAL>), dim3(blocks), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((k_expert_gemm<TW, DUAL>), dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <bool DUAL>
hipError_t expert_gemm(uint32_t type, const MoePrefillArgs& a, hipStream_t s) {
    switch (type) {
        case T_Q4_K: return expert_gemm_t<T_Q4_K, DUAL>(a, s);
        case T_Q5_K: return expert_gemm_t<T_Q5_K, DUAL>(a, s);
        case T_Q6_K: return expert_gemm_t<T_Q6_K, DUAL>(a, s);
        case T_Q8_0: return expert_gemm_t<T_Q8_0, DUAL>(a, s);
        case T_Q4_0: return expert_gemm_t<T_Q4_0, DUAL>(a, s);
        case T_Q4_1: return expert_gemm_t<T_Q4_1, DUAL>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

uint32_t moe_prefill_max_tiles(uint32_t tokens, uint32_t top_k, uint32_t n_experts) {
    const uint32_t pairs = tokens * top_k;
    return pairs / kTileM + (n_experts < pairs ? n_experts : pairs);
}

bool moe_prefill_supported(uint32_t gate_type, uint32_t up_type, uint32_t down_type,
                           uint32_t hidden, uint32_t ffn, uint32_t n_experts, uint32_t top_k,
                           uint32_t tokens, uint32_t variant) {
    if (variant > 1u) return false;
    if (gate_type != up_type || !prefill_type_ok(gate_type) || !prefill_type_ok(down_type))
        return false;
    if (tokens == 0 || tokens > kMaxPrefillTokens) return false;
    if (hidden % 256u || ffn % 256u || hidden / 256u > 32u) return false;
    switch (hidden / 256u) {
        case 2: case 4: case 8: case 12: case 16: case 24: case 32: break;
        default: return false;
    }
    // hidden and ffn are multiples of 256: whole 128-row blocks, 32- and 64-value stages

    return n_experts >= 1 && n_experts <= kMaxExperts && top_k >= 1 && top_k <= kMaxTopK &&
           top_k <= n_experts;
}

hipError_t launch_prefill_routing(const MoePrefillArgs& a, hipStream_t s) {
    const MoeDecodeArgs& L = a.layer;
    // 1. router
    const uint32_t per = L.hidden / kRouterThreads;
    const uint32_t rw = per <= 8u ? 4u : per <= 16u ? 2u : 1u;  // router_rows_per_wave<per>()
    const dim3 rgrid(ceil_div_u(L.n_experts + L.variant, 4u * rw), ceil_div_u(a.tokens, kRouterTokens));
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
    const uint32_t xpieces = a.tokens * L.hidden / 16u;
    const dim3 ggrid(1u + ceil_div_u(xpieces, kGroupThreads));
    if (L.gate_type == T_Q6_K) hipLaunchKernelGGL(k_group<16>, ggrid, dim3(kGroupThreads), 0, s, a);
    else hipLaunchKernelGGL(k_group<32>, ggrid, dim3(kGroupThreads), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_prefill_gate_up(const MoePrefillArgs& a, hipStream_t s) {
    return expert_gemm<true>(a.layer.gate_type, a, s);
}

hipError_t launch_prefill_down(const MoePrefillArgs& a, hipStream_t s) {
    const MoeDecodeArgs& L = a.layer;
    const hipError_t err = expert_gemm<false>(L.down_type, a, s);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_combine, dim3(a.tokens, ceil_div_u(L.hidden, 1024u)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace pk
