// exact.hip -- reference-order kernels for the whole-model decode.
//
// Greedy decoding over many layers amplifies any difference in the hidden
// state: an FP16 KV element that rounds the other way, or an expert logit
// near-tie, changes later tokens.  These kernels therefore repeat the
// reference's own operation order so that, given equal inputs, they return
// the CPU's bits:
//  * matvecs as linear_k / linear_quantized / linear (src/quantized_linear.cpp:
//    360-423, src/linear.cpp:10-31): per row, sum = ((0 + dot_0) + dot_1) + ...
//    over blocks, each block dot a left-to-right FP32 chain of rounded
//    products (dot_f32 / dot_i8_f32, src/simd_kernels.hpp:12-48, x86 branch);
//    one lane per (row, block), then one lane per row adds the block dots;
//  * RMSNorm with the serial sum of squares (src/rms_norm.cpp:9-27);
//  * attention with the serial softmax denominator (src/kv_cache.cpp:185-293);
//  * route_experts (src/qwen3_moe_runner.cpp:267-305) over the serial logits;
//  * float exponentials as the host libm's expf: exp in double rounded once
//    to float (the correctly rounded value), replaced by libm's result on the
//    inputs of the host's exception table (glibc: 170,648 of the 2.24e9
//    floats in [-104, 89], each one ulp away).
// Everything is unfused (-ffp-contract=off) and round-to-nearest.
#include <hip/hip_fp16.h>
#include <math.h>

#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

// Two independent loads (one slot in each half of the cuckoo table), so the
// exception costs one memory round trip whether or not the input has one.
__device__ float expf_libm(float x, const LibmExpf& t) {
    float r = static_cast<float>(exp(static_cast<double>(x)));
    if (t.slots) {
        const uint32_t b = __float_as_uint(x);
        const uint32_t i0 = (b * t.mul0) >> (32u - t.bits), i1 = (b * t.mul1) >> (32u - t.bits);
        const uint2 e0 = reinterpret_cast<const uint2*>(t.slots)[i0];
        const uint2 e1 = reinterpret_cast<const uint2*>(t.slots)[(1u << t.bits) + i1];
        if (e0.x == b) r = __uint_as_float(e0.y);
        if (e1.x == b) r = __uint_as_float(e1.y);
    }
    return r;
}

// Reference-decoded weight i (0..255) of one K-quant block, or of a 32-block.
template <int T>
struct RefBlock;

template <>
struct RefBlock<T_Q4_K> {
    static constexpr uint32_t BE = 256, BB = 144;
};
template <>
struct RefBlock<T_Q5_K> {
    static constexpr uint32_t BE = 256, BB = 176;
};
template <>
struct RefBlock<T_Q6_K> {
    static constexpr uint32_t BE = 256, BB = 210;
};
template <>
struct RefBlock<T_Q8_0> {
    static constexpr uint32_t BE = 32, BB = 34;
};
template <>
struct RefBlock<T_Q4_0> {
    static constexpr uint32_t BE = 32, BB = 18;
};
template <>
struct RefBlock<T_Q4_1> {
    static constexpr uint32_t BE = 32, BB = 20;
};
template <>
struct RefBlock<T_Q5_0> {
    static constexpr uint32_t BE = 32, BB = 22;
};
template <>
struct RefBlock<T_Q5_1> {
    static constexpr uint32_t BE = 32, BB = 24;
};
template <>
struct RefBlock<T_Q2_K> {
    static constexpr uint32_t BE = 256, BB = 84;
};
template <>
struct RefBlock<T_Q3_K> {
    static constexpr uint32_t BE = 256, BB = 110;
};

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float add16(float s, const f32x16 v) {
    s = __fadd_rn(s, v[0]); s = __fadd_rn(s, v[1]); s = __fadd_rn(s, v[2]); s = __fadd_rn(s, v[3]);
    s = __fadd_rn(s, v[4]); s = __fadd_rn(s, v[5]); s = __fadd_rn(s, v[6]); s = __fadd_rn(s, v[7]);
    s = __fadd_rn(s, v[8]); s = __fadd_rn(s, v[9]); s = __fadd_rn(s, v[10]); s = __fadd_rn(s, v[11]);
    s = __fadd_rn(s, v[12]); s = __fadd_rn(s, v[13]); s = __fadd_rn(s, v[14]);
    return __fadd_rn(s, v[15]);
}

// LDS floats an array summed by serial_sum needs beyond n rounded up to 16.
constexpr uint32_t kChainPad = 32;
__host__ __device__ constexpr uint32_t chain_floats(uint32_t n) { return (n + 15u) / 16u * 16u + kChainPad; }

// x of the reference matvec sits in LDS one block (BE values) per 16-byte
// padded stretch: the lanes of a wave read the same offset of different
// blocks, and without the pad those reads (1 KB apart for 256-value blocks)
// all fall in one LDS bank.
template <uint32_t BE>
__host__ __device__ constexpr uint32_t xpad(uint32_t i) { return i + i / BE * 4u; }
template <uint32_t BE>
__host__ __device__ constexpr uint32_t xpad_floats(uint32_t n) { return n + (n + BE - 1u) / BE * 4u; }

// s = ((s + p[0]) + p[1]) + ... + p[n - 1], by the calling lane.  p is in LDS,
// 64-byte aligned, readable for chain_floats(n) floats: the next 32 values
// are read while the current 32 are added, so the chain of dependent adds
// does not wait on LDS latency.
__device__ float serial_sum(const float* p, uint32_t n, float s) {
    const f32x16* v = reinterpret_cast<const f32x16*>(p);
    const uint32_t nb = n / 16u;
    // two register sets, each refilled right after its 32 values are added,
    // so the reads of one run under the adds of the other and no set is
    // copied (the scheduler would otherwise sink the reads next to their use,
    // or move each loaded set into the one the loop carries)
    f32x16 a0 = v[0], a1 = v[1];
    uint32_t k = 0;
    for (; k + 4u <= nb; k += 4u) {
        const f32x16 b0 = v[k + 2u], b1 = v[k + 3u];
        __builtin_amdgcn_sched_barrier(0);
        s = add16(s, a0);
        s = add16(s, a1);
        a0 = v[k + 4u];
        a1 = v[k + 5u];
        __builtin_amdgcn_sched_barrier(0);
        s = add16(s, b0);
        s = add16(s, b1);
    }
    // a0, a1 hold blocks k, k + 1 (read within the pad); up to three remain
    if (k < nb) s = add16(s, a0);
    if (k + 1u < nb) s = add16(s, a1);
    if (k + 2u < nb) s = add16(s, v[k + 2u]);
    for (uint32_t i = 16u * nb; i < n; ++i) s = __fadd_rn(s, p[i]);
    return s;
}

// v of the lane the DPP control selects, 0 where it selects none.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u0(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
}

// Inclusive prefix sum of uint32 values over the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
    v += dpp_u0<0x111>(v);       // row_shr:1
    v += dpp_u0<0x112>(v);       // row_shr:2
    v += dpp_u0<0x114>(v);       // row_shr:4
    v += dpp_u0<0x118>(v);       // row_shr:8
    v += dpp_u0<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    v += dpp_u0<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

// ((0 + p[0]) + p[1]) + ... + p[n - 1] for values p >= 0 in LDS (the squares
// of an RMSNorm), bit for bit the serial FP32 chain, computed by one whole
// wave (every lane active; the result is uniform).  p is readable for
// chain_floats(n) floats.
//
// While the running sum s stays in one binade [2^e, 2^(e+1)), every step
// rounds to that binade's grid u = 2^(e-23): RN(s + p) = s + u * rn(p / u),
// except when p / u is exactly half an integer (the tie goes to the even
// multiple of u, which depends on s) or when s + p reaches 2^(e+1) (the grid
// changes).  Between such steps the chain is therefore an integer prefix sum
// of rn(p / u), which the wave forms 256 values at a time (four consecutive
// per lane, a wave scan).  The first lane holding a tie, a non-finite value or
// the step that reaches 2^(e+1) starts from the exact sum in front of it and
// adds its four values by plain FP32 adds; the scan restarts after them.  The
// first 64 values (where the binade still changes at almost every step), a
// zero or extreme running sum take the plain serial add.
__device__ float serial_sum_nonneg(const float* p, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63u;
    constexpr uint32_t kTop = 1u << 24;  // a + P reaching this is a binade crossing
    uint32_t t = n < 64u ? n : 64u;
    float s = serial_sum(p, t, 0.0f);
    while (t < n) {  // uniform
        const uint32_t bits = __builtin_bit_cast(uint32_t, s);
        const int e = static_cast<int>((bits >> 23) & 0xffu) - 127;
        if (!(s > 0.0f) || !(s < INFINITY) || e < -100 || e > 100) {  // uniform
            s = __fadd_rn(s, p[t]);
            ++t;
            continue;
        }
        const float inv_u = __builtin_bit_cast(float, static_cast<uint32_t>(150 - e) << 23);  // 2^(23-e)
        const float u = __builtin_bit_cast(float, static_cast<uint32_t>(104 + e) << 23);      // 2^(e-23)
        const uint32_t a = static_cast<uint32_t>(__fmul_rn(s, inv_u));  // in [2^23, 2^24), exact
        const uint32_t i0 = t + 4u * lane;
        float x[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) x[i] = p[min(i0 + i, n - 1u)];
        uint32_t c = 0u;
        bool stop = false;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const float xi = i0 + i < n ? x[i] : 0.0f;
            const float q = __fmul_rn(xi, inv_u);  // exact: a power-of-two scale
            const float r = __builtin_rintf(q);
            // a tie (|q - r| is exact) or a non-finite value
            stop = stop || fabsf(__fsub_rn(q, r)) == 0.5f || !(xi < INFINITY);
            c += static_cast<uint32_t>(fminf(r, 16777216.0f));  // 2^24 forces a stop
        }
        c = min(c, kTop);  // at most 2^24 per lane: the wave's sum fits 32 bits
        const uint32_t incl = wave_scan_u32(c);
        const uint64_t any = __ballot(stop || a + incl >= kTop);
        if (any == 0u) {  // uniform: the whole chunk stays on the grid
            const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63));
            s = __fmul_rn(static_cast<float>(a + total), u);  // a + total < 2^24: exact
            t = n - t > 256u ? t + 256u : n;
        } else {
            const int L = __ffsll(static_cast<unsigned long long>(any)) - 1;
            const uint32_t pb = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl - c), L));
            s = __fmul_rn(static_cast<float>(a + pb), u);  // the sum in front of lane L: exact
            const uint32_t b = t + 4u * static_cast<uint32_t>(L);
            float y[4];
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) y[i] = p[min(b + i, n - 1u)];
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i)
                if (b + i < n) s = __fadd_rn(s, y[i]);
            t = n - b > 4u ? b + 4u : n;
        }
    }
    return s;
}

// s + ((ds * q) - dm) * x: one element of a K-quant block dot (decode_q4_k /
// decode_q5_k weight, then dot_f32's rounded product and add).
__device__ __forceinline__ float kq_step(float s, float ds, float dm, float q, float x) {
    return __fadd_rn(s, __fmul_rn(__fsub_rn(__fmul_rn(ds, q), dm), x));
}

// Four elements whose quants are the bytes of v, x the matching float4.
__device__ __forceinline__ float kq_step4(float s, float ds, float dm, uint32_t v, float4 x) {
    s = kq_step(s, ds, dm, ub<0>(v), x.x);
    s = kq_step(s, ds, dm, ub<1>(v), x.y);
    s = kq_step(s, ds, dm, ub<2>(v), x.z);
    return kq_step(s, ds, dm, ub<3>(v), x.w);
}

// Q6_K: s + (dsc * (q - 32)) * x for the four 6-bit quants in the bytes of v.
__device__ __forceinline__ float q6_step4(float s, float dsc, uint32_t v, float4 x) {
    s = __fadd_rn(s, __fmul_rn(__fmul_rn(dsc, ub<0>(v) - 32.0f), x.x));
    s = __fadd_rn(s, __fmul_rn(__fmul_rn(dsc, ub<1>(v) - 32.0f), x.y));
    s = __fadd_rn(s, __fmul_rn(__fmul_rn(dsc, ub<2>(v) - 32.0f), x.z));
    return __fadd_rn(s, __fmul_rn(__fmul_rn(dsc, ub<3>(v) - 32.0f), x.w));
}

// Block b of row `row`, loaded whole into registers (whole words; the planar
// formats field by field), so a kernel can issue the loads before it stages x.
template <int T> struct RefRaw;
template <> struct RefRaw<T_Q4_K> { uint32_t w[36]; };
template <> struct RefRaw<T_Q5_K> { uint32_t w[44]; };
template <> struct RefRaw<T_Q6_K> { uint32_t ql[32], qh[16], sw[4]; float d; };
template <> struct RefRaw<T_Q8_0> { uint32_t w[8]; float d; };
template <> struct RefRaw<T_Q4_1> { uint32_t w[5]; };
template <> struct RefRaw<T_Q5_0> { uint32_t qs[4], qh[1]; float d; };
template <> struct RefRaw<T_Q5_1> { uint32_t w[6]; };
template <> struct RefRaw<T_Q2_K> { uint32_t sw[4], qw[16], dd[1]; };
template <> struct RefRaw<T_Q3_K> { uint32_t qw[16], hw[8], p3[3]; float d; };
template <> struct RefRaw<T_Q4_0> { uint32_t w[4]; float d; };

template <int T>
__device__ __forceinline__ void ref_load(const QRow& row, uint32_t b, RefRaw<T>& r) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        ld_words<T == T_Q4_K ? 36 : 44>(block_ptr<RefBlock<T>::BB>(row, b), r.w);
    } else if constexpr (T == T_Q6_K) {
        using L = Planar<T_Q6_K>;
        ld_words<32>(field_ptr<L::QL, 128>(row, b), r.ql);
        ld_words<16>(field_ptr<L::QH, 64>(row, b), r.qh);
        ld_words<4>(field_ptr<L::SC, 16>(row, b), r.sw);
        r.d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, b)));
    } else if constexpr (T == T_Q8_0) {
        using L = Planar<T_Q8_0>;
        ld_words<8>(field_ptr<L::QS, 32>(row, b), r.w);
        r.d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, b)));
    } else if constexpr (T == T_Q4_1) {
        ld_words<5>(block_ptr<20>(row, b), r.w);
    } else if constexpr (T == T_Q5_0) {
        using L = Planar<T_Q5_0>;
        ld_words<4>(field_ptr<L::QS, 16>(row, b), r.qs);
        ld_words<1>(field_ptr<L::QH, 4>(row, b), r.qh);
        r.d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, b)));
    } else if constexpr (T == T_Q5_1) {
        ld_words<6>(block_ptr<24>(row, b), r.w);
    } else if constexpr (T == T_Q2_K) {
        const uint8_t* blk = block_ptr<84>(row, b);
        ld_words<4>(blk, r.sw);
        ld_words<16>(blk + 16, r.qw);
        ld_words<1>(blk + 80, r.dd);
    } else if constexpr (T == T_Q3_K) {
        using L = Planar<T_Q3_K>;
        ld_words<16>(field_ptr<L::QS, 64>(row, b), r.qw);
        ld_words<8>(field_ptr<L::HM, 32>(row, b), r.hw);
        ld_words<3>(field_ptr<L::SC, 12>(row, b), r.p3);
        r.d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, b)));
    } else {  // Q4_0
        using L = Planar<T_Q4_0>;
        ld_words<4>(field_ptr<L::QS, 16>(row, b), r.w);
        r.d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, b)));
    }
}

// Eight float4 of x from LDS.  The block dots below read x one 32-value
// chunk ahead of the chain: the reads of chunk c + 1 take their address from
// a zero that depends on the chain's value at the start of chunk c.  Without
// that the scheduler hoists all 256 reads of a block to the top, and the
// registers they need spill into AGPRs, on the chain's critical path.
struct X8 {
    float4 v[8];
};
__device__ __forceinline__ X8 ldx8(const float4* x4, uint32_t i) {
    X8 r;
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) r.v[k] = x4[i + k];
    return r;
}
// 0, computed from v so that nothing using it can move above v's definition.
__device__ __forceinline__ uint32_t zero_after(float v) {
    uint32_t z;
    asm volatile("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(__builtin_bit_cast(uint32_t, v)));
    return z;
}

// dot of a loaded block with x (x in LDS, 16-byte aligned), in element
// order.  K-quants and Q4_1: the decoded FP32 weight times x; Q8_0/Q4_0:
// d * dot_i8_f32 (the int8 value times x, then the scale once).
template <int T>
__device__ float ref_dot(const RefRaw<T>& r, const float* x) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float s = 0.0f;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        constexpr int QS = T == T_Q4_K ? 4 : 12;
        const uint32_t* w = r.w;
        const uint32_t h[4] = {w[0], w[1], w[2], w[3]};
        const float d = half_bits_to_float(w[0] & 0xffffu), dmin = half_bits_to_float(w[0] >> 16);
        X8 xa = ldx8(x4, 0u);
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            X8 xb;
            if (j < 7u) xb = ldx8(x4 + zero_after(s), 8u * (j + 1u));
            float sc, mn;
            kq_scale_min(h, j, sc, mn);
            const float ds = __fmul_rn(d, sc), dm = __fmul_rn(dmin, mn);
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) {
                const uint32_t raw = w[QS + 8u * (j / 2u) + k];
                uint32_t v = (j & 1u) ? (raw >> 4) & 0x0f0f0f0fu : raw & 0x0f0f0f0fu;
                if constexpr (T == T_Q5_K) v |= ((w[4u + k] >> j) & 0x01010101u) << 4;
                s = kq_step4(s, ds, dm, v, xa.v[k]);
            }
            if (j < 7u) xa = xb;
        }
    } else if constexpr (T == T_Q6_K) {
        const float d = r.d;
        X8 xa = ldx8(x4, 0u);
#pragma unroll
        for (uint32_t c = 0; c < 8; ++c) {
            X8 xb;
            if (c < 7u) xb = ldx8(x4 + zero_after(s), 8u * (c + 1u));
            const uint32_t half = c / 4u, g = c % 4u;
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) {
                const uint32_t sb = 8u * half + 2u * g + (k >= 4u ? 1u : 0u);
                const int sc = static_cast<int8_t>(r.sw[sb / 4u] >> (8u * (sb % 4u)));
                const float dsc = __fmul_rn(d, static_cast<float>(sc));
                const uint32_t lw = r.ql[16u * half + 8u * (g & 1u) + k];
                const uint32_t hw = r.qh[8u * half + k];
                const uint32_t v = (g >= 2u ? (lw >> 4) & 0x0f0f0f0fu : lw & 0x0f0f0f0fu) |
                                   (((hw >> (2u * g)) & 0x03030303u) << 4);
                s = q6_step4(s, dsc, v, xa.v[k]);
            }
            if (c < 7u) xa = xb;
        }
    } else if constexpr (T == T_Q8_0) {
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const float4 xv = x4[k];
            const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (uint32_t m = 0; m < 4; ++m) {
                const int q = static_cast<int8_t>(r.w[k] >> (8u * m));
                s = __fadd_rn(s, __fmul_rn(xs[m], static_cast<float>(q)));
            }
        }
        s = __fmul_rn(r.d, s);
    } else if constexpr (T == T_Q4_1) {  // weight fl(fl(q * d) + m), low nibbles first
        const uint32_t* w = r.w;         // d | m << 16, then quants 0..15
        const float d = half_bits_to_float(w[0] & 0xffffu), m = half_bits_to_float(w[0] >> 16);
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const uint32_t raw = w[1u + (k & 3u)];
            const uint32_t v = k < 4u ? raw & 0x0f0f0f0fu : (raw >> 4) & 0x0f0f0f0fu;
            const float4 xv = x4[k];
            s = __fadd_rn(s, __fmul_rn(__fadd_rn(__fmul_rn(ub<0>(v), d), m), xv.x));
            s = __fadd_rn(s, __fmul_rn(__fadd_rn(__fmul_rn(ub<1>(v), d), m), xv.y));
            s = __fadd_rn(s, __fmul_rn(__fadd_rn(__fmul_rn(ub<2>(v), d), m), xv.z));
            s = __fadd_rn(s, __fmul_rn(__fadd_rn(__fmul_rn(ub<3>(v), d), m), xv.w));
        }
    } else if constexpr (T == T_Q5_0 || T == T_Q5_1) {
        // decode_q5_0: fl((q - 16) * d); decode_q5_1: fl(fl(q * d) + m)
        // (src/quantized_linear.cpp:64-93), then dot_f32's order
        uint32_t qs[4], qh;
        float d, m = 0.0f;
        if constexpr (T == T_Q5_0) {
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) qs[i] = r.qs[i];
            qh = r.qh[0];
            d = r.d;
        } else {  // d | m << 16, qh, quants
            d = half_bits_to_float(r.w[0] & 0xffffu);
            m = half_bits_to_float(r.w[0] >> 16);
            qh = r.w[1];
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) qs[i] = r.w[2u + i];
        }
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const float4 xv = x4[k];
            const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const uint32_t i = 4u * k + j, byte = i & 15u;
                const uint32_t v = (qs[byte / 4u] >> (8u * (byte % 4u))) & 0xffu;
                const uint32_t q = (i < 16u ? (v & 15u) : (v >> 4)) | (((qh >> i) & 1u) << 4);
                const float w = T == T_Q5_0 ? __fmul_rn(static_cast<float>(static_cast<int>(q) - 16), d)
                                            : __fadd_rn(__fmul_rn(static_cast<float>(q), d), m);
                s = __fadd_rn(s, __fmul_rn(w, xs[j]));
            }
        }
    } else if constexpr (T == T_Q2_K || T == T_Q3_K) {
        // decode_q2_k: fl(fl(dl * q) - ml); decode_q3_k: fl(ds * (q - 4 + 4 * hbit))
        // (src/quantized_linear.cpp:95-164); element 128h + 32s + 16t + i
        uint32_t sw[4];
        float d, dmin = 0.0f;
        const uint32_t* qw = r.qw;
        if constexpr (T == T_Q2_K) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) sw[j] = r.sw[j];
            d = half_bits_to_float(r.dd[0] & 0xffffu);
            dmin = half_bits_to_float(r.dd[0] >> 16);
        } else {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {  // the 16 unpacked 6-bit scales, 4 per word
                sw[j] = q3k_scale(r.p3, 4u * j) | (q3k_scale(r.p3, 4u * j + 1u) << 8) |
                        (q3k_scale(r.p3, 4u * j + 2u) << 16) | (q3k_scale(r.p3, 4u * j + 3u) << 24);
            }
            d = r.d;
        }
        X8 xa = ldx8(x4, 0u), xb;
#pragma unroll
        for (uint32_t g = 0; g < 16; ++g) {  // 16-element groups in element order
            if ((g & 1u) == 0u && g < 14u)  // the next two groups' x ahead of this pair
                xb = ldx8(x4 + zero_after(s), 4u * (g + 2u));
            const uint32_t h = g / 8u, sh = (g % 8u) / 2u, t = g % 2u;
            const uint32_t scb = (sw[g / 4u] >> (8u * (g % 4u))) & 0xffu;
            float mul, off;
            if constexpr (T == T_Q2_K) {
                mul = __fmul_rn(d, static_cast<float>(scb & 15u));
                off = __fmul_rn(dmin, static_cast<float>(scb >> 4));
            } else {
                mul = __fmul_rn(d, static_cast<float>(static_cast<int>(scb) - 32));
                off = 0.0f;
            }
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) {
                const uint32_t qv = qw[(32u * h + 16u * t) / 4u + k];
                const float4 xv = xa.v[4u * (g & 1u) + k];
                const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) {
                    const uint32_t q = (qv >> (8u * j + 2u * sh)) & 3u;
                    float w;
                    if constexpr (T == T_Q2_K) {
                        w = __fsub_rn(__fmul_rn(mul, static_cast<float>(q)), off);
                    } else {
                        const uint32_t hb = (r.hw[(16u * t) / 4u + k] >> (8u * j + 4u * h + sh)) & 1u;
                        w = __fmul_rn(mul, static_cast<float>(static_cast<int>(q) - (hb ? 0 : 4)));
                    }
                    s = __fadd_rn(s, __fmul_rn(w, xs[j]));
                }
            }
            if ((g & 1u) == 1u && g < 15u) xa = xb;
        }
    } else {  // Q4_0: low nibbles are elements 0..15, high 16..31
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const float4 xv = x4[k];
            const float xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (uint32_t m = 0; m < 4; ++m) {
                const uint32_t i = 4u * k + m, byte = i & 15u;
                const uint32_t v = (r.w[byte / 4u] >> (8u * (byte % 4u))) & 0xffu;
                const int q = static_cast<int>(i < 16u ? (v & 15u) : (v >> 4)) - 8;
                s = __fadd_rn(s, __fmul_rn(xs[m], static_cast<float>(q)));
            }
        }
        s = __fmul_rn(r.d, s);
    }
    return s;
}

// ---------------------------------------------------------------------------
// Prologues shared by the matvec kernels (whole workgroup of NT threads).

// v = x + residual (route-order combine from 0, or delta) for the n values,
// eight per thread per batch with every load of a batch in flight together;
// the serial FP32 sum of the squares; then xs = (v * scale) * w with
// scale = 1 / sqrt(sum / n + eps) (rms_norm, src/rms_norm.cpp:9-27, and the
// residual adds of src/qwen3_moe_runner.cpp:640,692).  The leader writes v
// and xs to x_out / normed_out.  LDS: xs [n], sq [chain_floats(n)], wb [n].
template <uint32_t NT, uint32_t PADB = 0>
__device__ void ref_norm_stage(const RefNormIn& p, uint32_t n, float* xs, float* sq, float* wb,
                               float& s_scale, bool leader) {
    auto xi = [](uint32_t i) { return PADB ? xpad<(PADB ? PADB : 1u)>(i) : i; };
    const uint32_t tid = threadIdx.x;
    for (uint32_t base = 0; base < n; base += 8u * NT) {
        uint32_t ic[8];
        float v[8], wv[8];
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const uint32_t i = base + tid + NT * k;
            ic[k] = i < n ? i : 0u;
            v[k] = p.x[ic[k]];
            wv[k] = p.w[ic[k]];
        }
        if (p.res.parts) {
            float yv[8];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) yv[k] = 0.0f;
            for (uint32_t r0 = 0; r0 < p.res.K; r0 += 8u) {
                float pr[8], pv[8][8];
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) {
                    const uint32_t rc = r0 + j < p.res.K ? r0 + j : 0u;
                    pr[j] = p.res.probs[rc];
#pragma unroll
                    for (uint32_t k = 0; k < 8; ++k)
                        pv[j][k] = p.res.parts[static_cast<uint64_t>(rc) * n + ic[k]];
                }
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j)
                    if (r0 + j < p.res.K) {
#pragma unroll
                        for (uint32_t k = 0; k < 8; ++k) yv[k] = __fadd_rn(yv[k], __fmul_rn(pr[j], pv[j][k]));
                    }
            }
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) v[k] = __fadd_rn(v[k], yv[k]);
        } else if (p.res.delta) {
            float dv[8];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) dv[k] = p.res.delta[ic[k]];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) v[k] = __fadd_rn(v[k], dv[k]);
        }
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const uint32_t i = base + tid + NT * k;
            if (i < n) {
                xs[xi(i)] = v[k];
                sq[i] = __fmul_rn(v[k], v[k]);
                wb[i] = wv[k];
            }
        }
    }
    __syncthreads();
    if (tid < 64u) {  // wave 0
        const float sum = serial_sum_nonneg(sq, n);
        if (tid == 0) s_scale = 1.0f / sqrtf(sum / static_cast<float>(n) + p.eps);
    }
    __syncthreads();
    const float scale = s_scale;
    for (uint32_t i = tid; i < n; i += NT) {
        const float vi = xs[xi(i)], o = __fmul_rn(__fmul_rn(vi, scale), wb[i]);
        if (leader) {
            if (p.x_out) p.x_out[i] = vi;
            if (p.normed_out) p.normed_out[i] = o;
        }
        xs[xi(i)] = o;
    }
    __syncthreads();
}

struct RouteShared {
    float lg[kMaxExperts256];
    double ex[kMaxExperts256];
    float wmax[4];
    uint32_t sel[kMaxRefTopK];
    float pr[kMaxRefTopK];
    double den;
};

// route_experts (src/qwen3_moe_runner.cpp:267-305) over the serial FP32
// logits, one thread per expert (256 threads, E <= 256): the route order is
// each expert's rank under (logit desc, id asc) -- the order the reference's
// stable insertion produces.  Returns the expert of `route`.  The leader also
// forms the FP64 exponentials' sum in expert order, the FP32 probabilities and
// the FP32 renormalisation, and writes ids and probs.  Non-finite logits: the
// leader flags the status word and every workgroup uses expert 0 (its reads
// stay in bounds; the result is reported as an error).
__device__ uint32_t ref_route_block(const RefRouteIn& R, uint32_t route, bool leader,
                                    RouteShared& sh) {
    const uint32_t t = threadIdx.x, E = R.n_experts, K = R.top_k;
    const bool on = t < E;
    const float l = on ? R.logits[t] : -INFINITY;
    sh.lg[t] = l;  // -inf past E: never ranks before a finite logit
    if (__syncthreads_or(on && !isfinite(l))) {
        if (leader) {
            if (t < K) {
                R.ids[t] = 0u;
                R.probs[t] = 0.0f;
            }
            if (t == 0) atomicOr(R.status, 1u);
        }
        return 0u;
    }
    // the maximum (its value does not depend on the order it is found in)
    float m = l;
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((t & 63u) == 0u) sh.wmax[t >> 6] = m;
    uint32_t rank = 0;
    if (on) {
        const uint32_t E4 = (E + 3u) / 4u;
        for (uint32_t j4 = 0; j4 < E4; ++j4) {
            const f32x4 q = reinterpret_cast<const f32x4*>(sh.lg)[j4];
            const uint32_t j = 4u * j4;
            rank += (q.x > l || (q.x == l && j < t)) ? 1u : 0u;
            rank += (q.y > l || (q.y == l && j + 1u < t)) ? 1u : 0u;
            rank += (q.z > l || (q.z == l && j + 2u < t)) ? 1u : 0u;
            rank += (q.w > l || (q.w == l && j + 3u < t)) ? 1u : 0u;
        }
        if (rank < K) sh.sel[rank] = t;
    }
    __syncthreads();
    if (leader) {  // uniform across the workgroup
        const float mx = fmaxf(fmaxf(sh.wmax[0], sh.wmax[1]), fmaxf(sh.wmax[2], sh.wmax[3]));
        const double e = on ? exp(static_cast<double>(__fsub_rn(l, mx))) : 0.0;
        if (on) sh.ex[t] = e;
        __syncthreads();
        if (t == 0) {
            double den = 0.0;
            for (uint32_t i = 0; i < E; ++i) den += sh.ex[i];
            sh.den = den;
        }
        __syncthreads();
        if (on && rank < K) sh.pr[rank] = static_cast<float>(e / sh.den);
        __syncthreads();
        if (t == 0) {
            float sum = 0.0f;
            for (uint32_t r = 0; r < K; ++r) sum = __fadd_rn(sum, sh.pr[r]);
            for (uint32_t r = 0; r < K; ++r) {
                R.ids[r] = sh.sel[r];
                R.probs[r] = R.normalize ? __fdiv_rn(sh.pr[r], sum) : sh.pr[r];
            }
        }
    }
    return sh.sel[route];
}

// ---------------------------------------------------------------------------
// y[route][row] for rows of W (route: the expert slice ids[route], or the one
// routing selects), x[route] staged in LDS -- or, with x_up, the SwiGLU
// activation g / (1 + expf(-g)) * u of x[route] and x_up[route]
// (src/qwen3_moe_runner.cpp:682-684), or, with a norm, RMSNorm of the residual
// stream.  Lanes (row, block); one lane per row then sums the block dots in
// block order starting from 0.  With segments, workgroups along x are split
// between up to three matrices that share the input.  With act (gate and up,
// segments 0 and 1), half of each workgroup's lanes take rows of gate and
// half the same rows of up, and the row sums become the SwiGLU activations
// g / (1 + expf(-g)) * u (src/qwen3_moe_runner.cpp:682-684), bit for bit
// what staging them in the down projection computes.
template <int T>
__global__ __launch_bounds__(256) void k_ref_matvec(RefMatvecArgs a) {
    // xs [in], part [256]; with a norm also sq [chain_floats(in)], wb [in]
    extern __shared__ __attribute__((aligned(64))) float lds[];
    __shared__ RouteShared rsh;
    __shared__ float s_scale;
    constexpr uint32_t BE = RefBlock<T>::BE, BB = RefBlock<T>::BB;
    const uint32_t r = blockIdx.y, tid = threadIdx.x;
    const bool leader = blockIdx.x == 0 && blockIdx.y == 0;
    const bool paired = a.act != nullptr;
    const uint32_t mat = paired ? tid / 128u : 0u, lt = paired ? tid % 128u : tid;
    const uint32_t nb = a.in / BE, rpw = (paired ? 128u : 256u) / nb;
    const uint8_t* W = a.W;
    uint64_t row_bytes = a.row_bytes, slice_bytes = a.slice_bytes;
    uint32_t rows = a.rows, bx = blockIdx.x;
    float* y = a.y;
    if (paired) {
        W = a.seg[mat].W;
        row_bytes = a.seg[mat].row_bytes;
        slice_bytes = a.seg[mat].slice_bytes;
        rows = a.seg[mat].rows;
    } else if (a.nseg) {
#pragma unroll
        for (uint32_t j = 0; j < kMaxRefSegs; ++j) {
            if (j < a.nseg && blockIdx.x >= a.seg[j].block0) {
                W = a.seg[j].W;
                row_bytes = a.seg[j].row_bytes;
                slice_bytes = a.seg[j].slice_bytes;
                rows = a.seg[j].rows;
                y = a.seg[j].y;
                bx = blockIdx.x - a.seg[j].block0;
            }
        }
    }
    float* xs = lds;  // padded: block b at b * (BE + 4)
    float* part = lds + xpad_floats<BE>(a.in);
    const uint32_t row0 = bx * rpw, lr = lt / nb, b = lt % nb, row = row0 + lr;
    const bool active = lr < rpw && row < rows;
    const uint64_t nblk = static_cast<uint64_t>(rows) * nb;
    const QRow qrow{W, nblk, static_cast<uint64_t>(active ? row : 0u) * nb};
    // With the expert known up front (a plain matrix, or ids of an earlier
    // launch) the block is loaded before x is staged, so the weight loads
    // overlap the staging (the norm's serial sum, the SwiGLU exponentials).
    RefRaw<T> raw;
    if (a.route.logits) {
        const uint64_t expert = ref_route_block(a.route, r, leader, rsh);
        ref_load<T>(QRow{W + expert * slice_bytes, nblk, qrow.blk0}, b, raw);
    } else {
        // the id of an earlier launch, read through the scalar cache (constant
        // address space: read-only here)
        using cu32 = const __attribute__((address_space(4))) uint32_t;
        const uint64_t expert = a.ids ? ((cu32*)(a.ids))[r] : 0u;
        ref_load<T>(QRow{W + expert * slice_bytes, nblk, qrow.blk0}, b, raw);
    }
    const float* x = a.x + static_cast<uint64_t>(r) * a.x_stride;
    const uint32_t n4 = a.in / 4u;  // in is a multiple of 32
    if (a.norm.w) {
        ref_norm_stage<256, BE>(a.norm, a.in, xs, part + 256, part + 256 + chain_floats(a.in),
                                s_scale, leader);
    } else if (a.x_up) {
        const f32x4* g4 = reinterpret_cast<const f32x4*>(x);
        const f32x4* u4 = reinterpret_cast<const f32x4*>(a.x_up + static_cast<uint64_t>(r) * a.x_stride);
        for (uint32_t base = 0; base < n4; base += 256u) {
            const uint32_t i = base + tid, ic = i < n4 ? i : 0u;
            const f32x4 gv = g4[ic], uv = u4[ic];
            f32x4 act;
            act.x = __fmul_rn(__fdiv_rn(gv.x, __fadd_rn(1.0f, expf_libm(-gv.x, a.expf))), uv.x);
            act.y = __fmul_rn(__fdiv_rn(gv.y, __fadd_rn(1.0f, expf_libm(-gv.y, a.expf))), uv.y);
            act.z = __fmul_rn(__fdiv_rn(gv.z, __fadd_rn(1.0f, expf_libm(-gv.z, a.expf))), uv.z);
            act.w = __fmul_rn(__fdiv_rn(gv.w, __fadd_rn(1.0f, expf_libm(-gv.w, a.expf))), uv.w);
            if (i < n4) *reinterpret_cast<f32x4*>(xs + xpad<BE>(4u * i)) = act;
        }
    } else {
        const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
        for (uint32_t base = 0; base < n4; base += 512u) {
            const uint32_t i0 = base + tid, i1 = i0 + 256u;
            const f32x4 v0 = x4[i0 < n4 ? i0 : 0u], v1 = x4[i1 < n4 ? i1 : 0u];
            if (i0 < n4) *reinterpret_cast<f32x4*>(xs + xpad<BE>(4u * i0)) = v0;
            if (i1 < n4) *reinterpret_cast<f32x4*>(xs + xpad<BE>(4u * i1)) = v1;
        }
    }
    __syncthreads();
    if (active) part[tid] = ref_dot<T>(raw, xs + b * (BE + 4u));
    __syncthreads();
    if (paired) {
        // the gate and up row sums (xs is free now), then the activations
        float* gu = xs;  // [2][rpw]
        if (tid < 2u * rpw) {
            const uint32_t m = tid / rpw, rr = tid % rpw;
            float acc = 0.0f;
            for (uint32_t k = 0; k < nb; ++k) acc = __fadd_rn(acc, part[128u * m + rr * nb + k]);
            gu[tid] = acc;
        }
        __syncthreads();
        if (tid < rpw && row0 + tid < rows) {
            const float g = gu[tid], u = gu[rpw + tid];
            a.act[static_cast<uint64_t>(r) * a.y_stride + row0 + tid] =
                __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf_libm(-g, a.expf))), u);
        }
        return;
    }
    if (tid < rpw && row0 + tid < rows) {
        float acc = 0.0f;
        for (uint32_t k = 0; k < nb; ++k) acc = __fadd_rn(acc, part[tid * nb + k]);
        y[static_cast<uint64_t>(r) * a.y_stride + row0 + tid] = acc;
    }
}

// F32 linear: 0 + dot_f32(w_row, x), one 256-thread workgroup per row: x (or
// RMSNorm of the residual stream) staged in LDS, the products formed in
// parallel from coalesced loads, then one lane adds them in order.
__global__ __launch_bounds__(256) void k_ref_linear_f32(RefMatvecArgs a) {
    // prod [chain_floats(in)], xs [in]; with a norm also sq [chain_floats(in)], wb [in]
    extern __shared__ __attribute__((aligned(64))) float lds[];
    __shared__ float s_scale;
    const uint32_t row = blockIdx.x, r = blockIdx.y, tid = threadIdx.x;
    const bool leader = blockIdx.x == 0 && blockIdx.y == 0;
    const uint32_t cf = chain_floats(a.in);
    float* prod = lds;
    float* xs = lds + cf;
    const float* w = reinterpret_cast<const float*>(a.W + static_cast<uint64_t>(row) * a.row_bytes);
    // the first 2048 weights of the row go out before x is staged (the norm's
    // serial sum runs while they arrive)
    float w0[8];
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t i = tid + 256u * k;
        w0[k] = w[i < a.in ? i : 0u];
    }
    if (a.norm.w) {
        ref_norm_stage<256>(a.norm, a.in, xs, xs + a.in, xs + a.in + cf, s_scale, leader);
    } else {
        const float* x = a.x + static_cast<uint64_t>(r) * a.x_stride;
        for (uint32_t i = tid; i < a.in; i += 256u) xs[i] = x[i];
        __syncthreads();
    }
    for (uint32_t base = 0; base < a.in; base += 2048u) {
        float wv[8];
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const uint32_t i = base + tid + 256u * k;
            wv[k] = base == 0u ? w0[k] : w[i < a.in ? i : 0u];
        }
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const uint32_t i = base + tid + 256u * k;
            if (i < a.in) prod[i] = __fmul_rn(wv[k], xs[i]);
        }
    }
    __syncthreads();
    if (tid == 0)
        a.y[static_cast<uint64_t>(r) * a.y_stride + row] = __fadd_rn(0.0f, serial_sum(prod, a.in, 0.0f));
}

// Standalone RMSNorm (the output norm): x += the residual; out = (x * scale) * w.
// One 1024-thread workgroup per row of n <= 1024 * PER values; every load is
// issued before any is used, and the values stay in registers across the sum.
template <int PER>
__global__ __launch_bounds__(1024) void k_ref_rmsnorm(float* x, RefResidual res, const float* w,

                                                      float* out, uint32_t n, float eps) {
    extern __shared__ __attribute__((aligned(64))) float sq[];  // [chain_floats(n)]
    __shared__ float s_scale;
    const uint32_t tid = threadIdx.x;
    float* xr = x + static_cast<uint64_t>(blockIdx.x) * n;
    float* orow = out + static_cast<uint64_t>(blockIdx.x) * n;
    uint32_t ic[PER];
    float v[PER], wv[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t i = tid + 1024u * k;
        ic[k] = i < n ? i : 0u;
        v[k] = xr[ic[k]];
        wv[k] = w[ic[k]];
    }
    if (res.parts) {
        // routes in batches of RB whose loads are all in flight together
        constexpr uint32_t RB = PER <= 2 ? kMaxRefTopK : 32u / PER;
        float yv[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) yv[k] = 0.0f;
        for (uint32_t r0 = 0; r0 < res.K; r0 += RB) {
            float pr[RB], pv[RB][PER];
#pragma unroll
            for (uint32_t j = 0; j < RB; ++j) {
                const uint32_t rc = r0 + j < res.K ? r0 + j : 0u;
                pr[j] = res.probs[rc];
#pragma unroll
                for (int k = 0; k < PER; ++k) pv[j][k] = res.parts[static_cast<uint64_t>(rc) * n + ic[k]];
            }
#pragma unroll
            for (uint32_t j = 0; j < RB; ++j)
                if (r0 + j < res.K) {
#pragma unroll
                    for (int k = 0; k < PER; ++k) yv[k] = __fadd_rn(yv[k], __fmul_rn(pr[j], pv[j][k]));
                }
        }
#pragma unroll
        for (int k = 0; k < PER; ++k) v[k] = __fadd_rn(v[k], yv[k]);
    } else if (res.delta) {
        float dv[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) dv[k] = res.delta[ic[k]];
#pragma unroll
        for (int k = 0; k < PER; ++k) v[k] = __fadd_rn(v[k], dv[k]);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (tid + 1024u * k < n) sq[tid + 1024u * k] = __fmul_rn(v[k], v[k]);
    __syncthreads();
    if (tid < 64u) {  // wave 0
        const float sum = serial_sum_nonneg(sq, n);
        if (tid == 0) s_scale = 1.0f / sqrtf(sum / static_cast<float>(n) + eps);
    }
    __syncthreads();
    const float scale = s_scale;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t i = tid + 1024u * k;
        if (i < n) {
            if (res.parts || res.delta) xr[i] = v[k];
            orow[i] = __fmul_rn(__fmul_rn(v[k], scale), wv[k]);
        }
    }
}

// Attention of one q head over its KV window, in position order
// (KvCache::attend, src/kv_cache.cpp:185-293), with the step's own q/k/v
// work in front of it (src/qwen3_moe_runner.cpp:600-640): RMSNorm of the q
// head and of its kv head's k (serial sums, head-norm weights), RoPE from the
// host-computed table (cos, then sin, per position), k and v rounded to FP16
// as the ring stores them (the first q head of each group writes them).  Then
// score_i = (serial dot of q and k_i) * scale; the maximum;
// p_i = expf(score_i - max); the serial denominator;
// out[d] = ((0 + (p_0 / den) v_0[d]) + (p_1 / den) v_1[d]) + ...  The
// current position's k and v come from LDS, older ones from the ring: each
// FP16 K row loaded whole (HD / 8 16-byte loads), V rows staged through LDS a
// tile of positions at a time.
constexpr uint32_t kAttnTileBytes = 64u * 1024u;
template <int HD>
__global__ __launch_bounds__(256) void k_ref_attention(ModelArgs a, ModelLayer L) {
    extern __shared__ __attribute__((aligned(64))) float lds[];  // sc [chain_floats(capacity)], V tile
    __shared__ float qv[HD], kcur[HD], sqq[HD], sqk[HD];
    __shared__ __attribute__((aligned(16))) uint16_t vcur[HD];
    __shared__ float red[4];
    __shared__ float s_den, s_qscale, s_kscale;
    constexpr uint32_t TILE = kAttnTileBytes / (2u * HD), HALF = HD / 2u;
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const uint32_t group = a.heads / a.kv_heads, kvh = h / group;
    const uint32_t pos = a.state[0], slot_now = pos % a.capacity;
    const uint32_t n = pos + 1u < a.capacity ? pos + 1u : a.capacity;
    const uint32_t first = pos + 1u - n;
    const uint64_t row_halves = static_cast<uint64_t>(a.kv_heads) * HD;
    float* sc = lds;
    uint16_t* vt = reinterpret_cast<uint16_t*>(lds + chain_floats(a.capacity));
    // q / k head norms and RoPE, v to FP16
    float qx = 0.0f, kx = 0.0f, vx = 0.0f, qw = 0.0f, kw = 0.0f, c0 = 0.0f, s0 = 0.0f;
    const uint32_t d = tid < HD ? tid : 0u, dp = d % HALF;
    const float* cs = a.rope_table + static_cast<uint64_t>(pos) * HD;  // cos [HALF], sin [HALF]
    qx = a.q[h * HD + d];
    kx = a.k[kvh * HD + d];
    vx = a.v[kvh * HD + d];
    qw = L.q_norm[d];
    kw = L.k_norm[d];
    c0 = cs[dp];
    s0 = cs[HALF + dp];
    if (tid < HD) {
        sqq[tid] = __fmul_rn(qx, qx);
        sqk[tid] = __fmul_rn(kx, kx);
    }
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (uint32_t i = 0; i < HD; ++i) sum = __fadd_rn(sum, sqq[i]);
        s_qscale = 1.0f / sqrtf(sum / static_cast<float>(HD) + a.rms_eps);
    } else if (tid == 64) {
        float sum = 0.0f;
        for (uint32_t i = 0; i < HD; ++i) sum = __fadd_rn(sum, sqk[i]);
        s_kscale = 1.0f / sqrtf(sum / static_cast<float>(HD) + a.rms_eps);
    }
    __syncthreads();
    if (tid < HD) {  // normed values (the squares are no longer needed)
        sqq[tid] = __fmul_rn(__fmul_rn(qx, s_qscale), qw);
        sqk[tid] = __fmul_rn(__fmul_rn(kx, s_kscale), kw);
    }
    __syncthreads();
    if (tid < HD) {
        float rq, rk;
        if (tid < HALF) {
            rq = __fsub_rn(__fmul_rn(sqq[tid], c0), __fmul_rn(sqq[tid + HALF], s0));
            rk = __fsub_rn(__fmul_rn(sqk[tid], c0), __fmul_rn(sqk[tid + HALF], s0));
        } else {
            rq = __fadd_rn(__fmul_rn(sqq[tid], c0), __fmul_rn(sqq[dp], s0));
            rk = __fadd_rn(__fmul_rn(sqk[tid], c0), __fmul_rn(sqk[dp], s0));
        }
        const uint16_t kb = __half_as_ushort(__float2half_rn(rk));
        const uint16_t vb = __half_as_ushort(__float2half_rn(vx));
        qv[tid] = rq;
        kcur[tid] = __half2float(__ushort_as_half(kb));
        vcur[tid] = vb;
        if (h % group == 0u) {
            L.kcache[static_cast<uint64_t>(slot_now) * row_halves + kvh * HD + tid] = kb;
            L.vcache[static_cast<uint64_t>(slot_now) * row_halves + kvh * HD + tid] = vb;
        }
    }
    __syncthreads();
    float m = -INFINITY;
    for (uint32_t i = tid; i < n; i += 256u) {
        float s = 0.0f;
        if (i + 1u == n) {  // the current position
            for (uint32_t e = 0; e < HD; ++e) s = __fadd_rn(s, __fmul_rn(qv[e], kcur[e]));
        } else {
            const uint32_t slot = (first + i) % a.capacity;
            const u32x4_t* kr = reinterpret_cast<const u32x4_t*>(L.kcache + slot * row_halves + kvh * HD);
            u32x4_t kwv[HD / 8];
#pragma unroll
            for (int j = 0; j < HD / 8; ++j) kwv[j] = kr[j];
#pragma unroll
            for (int j = 0; j < HD / 8; ++j) {
                const uint32_t w4[4] = {kwv[j].x, kwv[j].y, kwv[j].z, kwv[j].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint16_t bits = static_cast<uint16_t>(w4[e / 2] >> (16 * (e % 2)));
                    s = __fadd_rn(s, __fmul_rn(qv[8 * j + e], __half2float(__ushort_as_half(bits))));
                }
            }
        }
        s = __fmul_rn(s, a.attn_scale);
        sc[i] = s;
        m = fmaxf(m, s);
    }
    // the maximum (its value does not depend on the order it is found in)
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63u) == 0u) red[tid >> 6] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (uint32_t i = tid; i < n; i += 256u) {
        const float e = __fsub_rn(sc[i], mx);
        sc[i] = expf_libm(e, a.expf);
    }
    // stage V rows t0 .. t0 + tn (HD / 8 16-byte pieces per row) with threads
    // t0th .. t0th + nt - 1: 8 pieces per thread, every global load
    // unconditional (the current position reads a ring row and takes the LDS
    // copy instead), so a pass waits for memory once
    constexpr uint32_t PPR = HD / 8;
    auto stage = [&](uint32_t t0, uint32_t tn, uint32_t t, uint32_t nt) {
        constexpr int KL = 8;
        for (uint32_t base = 0; base < tn * PPR; base += nt * KL) {
            u32x4_t pv[KL];
#pragma unroll
            for (int k = 0; k < KL; ++k) {
                const uint32_t q = base + t + nt * k, qc = q < tn * PPR ? q : 0u;
                const uint32_t i = t0 + qc / PPR;
                const uint32_t slot = (first + i) % a.capacity;
                pv[k] = reinterpret_cast<const u32x4_t*>(L.vcache + slot * row_halves + kvh * HD)[qc % PPR];
            }
#pragma unroll
            for (int k = 0; k < KL; ++k) {
                const uint32_t q = base + t + nt * k, qc = q < tn * PPR ? q : 0u;
                if (t0 + qc / PPR + 1u == n) pv[k] = reinterpret_cast<const u32x4_t*>(vcur)[qc % PPR];
                if (q < tn * PPR) reinterpret_cast<u32x4_t*>(vt)[q] = pv[k];
            }
        }
    };
    __syncthreads();
    // the serial denominator by thread 0 while waves 1-3 stage the first V tile
    if (tid == 0) s_den = serial_sum(sc, n, 0.0f);
    else if (tid >= 64u) stage(0u, n < TILE ? n : TILE, tid - 64u, 192u);
    __syncthreads();
    const float den = s_den;
    for (uint32_t i = tid; i < n; i += 256u) sc[i] = __fdiv_rn(sc[i], den);
    float o = 0.0f;
    for (uint32_t t0 = 0; t0 < n; t0 += TILE) {
        const uint32_t tn = n - t0 < TILE ? n - t0 : TILE;
        __syncthreads();  // the weights written (first tile), or the previous tile consumed
        if (t0 > 0u) {    // uniform
            stage(t0, tn, tid, 256u);
            __syncthreads();
        }
        if (tid < HD) {
            for (uint32_t i = 0; i < tn; ++i) {
                const float v = __half2float(__ushort_as_half(vt[i * HD + tid]));
                o = __fadd_rn(o, __fmul_rn(sc[t0 + i], v));
            }
        }
    }
    if (tid < HD) a.att[h * HD + tid] = o;
}

// Fast-mode attention (no parity claim; within 1e-4 of the reference's
// KvCache::attend, src/kv_cache.cpp:185-294): the same q/k head norms, RoPE
// and FP16 KV ring as k_ref_attention, with every sum reassociated into
// parallel partial sums except the norms' sums of squares, kept serial so
// that the FP16 k of the ring rounds as the reference's.  One workgroup of
// four waves per q head:
//  * scores: one position per thread, four interleaved partial dots;
//  * maximum and denominator: workgroup reductions;
//  * output: interleaved position streams with 16-byte V loads, their
//    partial sums added through LDS.
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

template <int HD>
__global__ __launch_bounds__(256) void k_fast_attention(ModelArgs a, ModelLayer L) {
    extern __shared__ __attribute__((aligned(64))) float lds[];  // scores [capacity]
    __shared__ float qv[HD], kcur[HD], sq[2][HD], part[4u * (64u / (HD / 8))][HD], red[2][4];
    __shared__ __attribute__((aligned(16))) uint16_t vcur[HD];
    constexpr uint32_t HALF = HD / 2u;
    const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t group = a.heads / a.kv_heads, kvh = h / group;
    const uint32_t pos = a.state[0], slot_now = pos % a.capacity;
    const uint32_t n = pos + 1u < a.capacity ? pos + 1u : a.capacity;
    const uint32_t first = pos + 1u - n;
    const uint64_t row_halves = static_cast<uint64_t>(a.kv_heads) * HD;
    float* sc = lds;
    const uint32_t d = tid < HD ? tid : 0u, dp = d % HALF;
    const float* cs = a.rope_table + static_cast<uint64_t>(pos) * HD;
    const float qx = a.q[h * HD + d], kx = a.k[kvh * HD + d], vx = a.v[kvh * HD + d];
    const float qw = L.q_norm[d], kw = L.k_norm[d], c0 = cs[dp], s0 = cs[HALF + dp];
    // the sums of squares in the reference's serial order (two threads at
    // once): the FP16 rounding of this position's k then matches the
    // reference's, and the ring holds the same k for later positions
    if (tid < HD) {
        sq[0][tid] = __fmul_rn(qx, qx);
        sq[1][tid] = __fmul_rn(kx, kx);
    }
    __syncthreads();
    if (tid == 0u || tid == 64u) {
        const float* v = sq[tid == 0u ? 0 : 1];
        float sum = 0.0f;
        for (uint32_t i = 0; i < HD; ++i) sum = __fadd_rn(sum, v[i]);
        red[tid == 0u ? 0 : 1][0] = sum;
    }
    __syncthreads();
    const float qs = 1.0f / sqrtf(red[0][0] / static_cast<float>(HD) + a.rms_eps);
    const float ks = 1.0f / sqrtf(red[1][0] / static_cast<float>(HD) + a.rms_eps);
    __syncthreads();  // the squares read before the normed values replace them
    if (tid < HD) {
        sq[0][tid] = qx * qs * qw;
        sq[1][tid] = kx * ks * kw;
    }
    __syncthreads();
    if (tid < HD) {  // RoPE on (d, d + HD / 2) pairs, the current position's FP16 k and v
        float rq, rk;
        if (tid < HALF) {
            rq = sq[0][tid] * c0 - sq[0][tid + HALF] * s0;
            rk = sq[1][tid] * c0 - sq[1][tid + HALF] * s0;
        } else {
            rq = sq[0][tid] * c0 + sq[0][dp] * s0;
            rk = sq[1][tid] * c0 + sq[1][dp] * s0;
        }
        const uint16_t kb = __half_as_ushort(__float2half_rn(rk));
        const uint16_t vb = __half_as_ushort(__float2half_rn(vx));
        qv[tid] = rq;
        kcur[tid] = __half2float(__ushort_as_half(kb));
        vcur[tid] = vb;
        if (h % group == 0u) {
            L.kcache[static_cast<uint64_t>(slot_now) * row_halves + kvh * HD + tid] = kb;
            L.vcache[static_cast<uint64_t>(slot_now) * row_halves + kvh * HD + tid] = vb;
        }
    }
    __syncthreads();
    // scores, one position per thread (four partial dots), and their maximum
    float m = -INFINITY;
    for (uint32_t i = tid; i < n; i += 256u) {
        float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
        if (i + 1u == n) {
#pragma unroll 8
            for (uint32_t e = 0; e < HD; e += 4u) {
                p0 = __builtin_fmaf(qv[e], kcur[e], p0);
                p1 = __builtin_fmaf(qv[e + 1u], kcur[e + 1u], p1);
                p2 = __builtin_fmaf(qv[e + 2u], kcur[e + 2u], p2);
                p3 = __builtin_fmaf(qv[e + 3u], kcur[e + 3u], p3);
            }
        } else {
            const uint32_t slot = (first + i) % a.capacity;
            const u32x4_t* kr = reinterpret_cast<const u32x4_t*>(L.kcache + slot * row_halves + kvh * HD);
            u32x4_t kwv[HD / 8];
#pragma unroll
            for (int j = 0; j < HD / 8; ++j) kwv[j] = kr[j];
#pragma unroll
            for (int j = 0; j < HD / 8; ++j) {
                const uint32_t w4[4] = {kwv[j].x, kwv[j].y, kwv[j].z, kwv[j].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float k0 = __half2float(__ushort_as_half(static_cast<uint16_t>(w4[e] & 0xffffu)));
                    const float k1 = __half2float(__ushort_as_half(static_cast<uint16_t>(w4[e] >> 16)));
                    if (e & 1) {
                        p2 = __builtin_fmaf(qv[8 * j + 2 * e], k0, p2);
                        p3 = __builtin_fmaf(qv[8 * j + 2 * e + 1], k1, p3);
                    } else {
                        p0 = __builtin_fmaf(qv[8 * j + 2 * e], k0, p0);
                        p1 = __builtin_fmaf(qv[8 * j + 2 * e + 1], k1, p1);
                    }
                }
            }
        }
        const float sv = ((p0 + p1) + (p2 + p3)) * a.attn_scale;
        sc[i] = sv;
        m = fmaxf(m, sv);
    }
    m = wave_max_f(m);
    if (lane == 0u) red[0][wave] = m;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    float den = 0.0f;
    for (uint32_t i = tid; i < n; i += 256u) {
        const float e = expf(sc[i] - mx);
        sc[i] = e;
        den += e;
    }
    den = wave_sum_f(den);
    __syncthreads();  // every score exponentiated, and red[0] read
    if (lane == 0u) red[1][wave] = den;
    __syncthreads();
    const float inv = 1.0f / (red[1][0] + red[1][1] + red[1][2] + red[1][3]);
    // output: LP = HD / 8 lanes hold one position's row (8 dimensions, one
    // 16-byte load each), so a wave reads 64 / LP positions per load and the
    // workgroup runs S = 4 * 64 / LP interleaved position streams; batches of
    // U positions per stream have every load issued (unconditional, clamped
    // to a valid row) before any is used; the streams' sums meet in LDS.
    constexpr uint32_t LP = HD / 8, S = 4u * (64u / LP), U = 8;
    const uint32_t stream = tid / LP, d0 = 8u * (tid % LP);
    float acc[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) acc[j] = 0.0f;
    const uint16_t* vbase = L.vcache + kvh * HD + d0;
    for (uint32_t i0 = stream; i0 < n; i0 += S * U) {
        u32x4_t raw[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = i0 + S * u, ic = i < n ? i : i0;
            raw[u] = *reinterpret_cast<const u32x4_t*>(vbase + ((first + ic) % a.capacity) * row_halves);
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = i0 + S * u;
            if (i < n) {
                const float p = sc[i];
                const bool now = i + 1u == n;  // the current position: its LDS copy
                const u32x4_t w = now ? *reinterpret_cast<const u32x4_t*>(vcur + d0) : raw[u];
                const uint32_t w4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j) {
                    const uint16_t b = static_cast<uint16_t>(w4[j / 2] >> (16 * (j % 2)));
                    acc[j] = __builtin_fmaf(p, __half2float(__ushort_as_half(b)), acc[j]);
                }
            }
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) part[stream][d0 + j] = acc[j];
    __syncthreads();
    if (tid < HD) {
        float o = 0.0f;
#pragma unroll
        for (uint32_t t = 0; t < S; ++t) o += part[t][tid];
        a.att[h * HD + tid] = o * inv;
    }
}


uint32_t ref_block_elems(uint32_t type) {
    return type == T_Q8_0 || type == T_Q4_0 || type == T_Q4_1 || type == T_Q5_0 ||
                   type == T_Q5_1
               ? 32u
               : 256u;
}

template <int T>
hipError_t ref_matvec_t(const RefMatvecArgs& a, uint32_t blocks, uint32_t routes, hipStream_t s) {
    size_t lds = (xpad_floats<RefBlock<T>::BE>(a.in) + 256u) * sizeof(float);
    if (a.norm.w) lds += (chain_floats(a.in) + a.in) * sizeof(float);
    hipLaunchKernelGGL(k_ref_matvec<T>, dim3(blocks, routes), dim3(256), lds, s, a);
    return hipGetLastError();
}

hipError_t ref_matvec_launch(uint32_t type, const RefMatvecArgs& a, uint32_t blocks,
                             uint32_t routes, hipStream_t s) {
    switch (type) {
        case T_Q4_K: return ref_matvec_t<T_Q4_K>(a, blocks, routes, s);
        case T_Q5_K: return ref_matvec_t<T_Q5_K>(a, blocks, routes, s);
        case T_Q6_K: return ref_matvec_t<T_Q6_K>(a, blocks, routes, s);
        case T_Q8_0: return ref_matvec_t<T_Q8_0>(a, blocks, routes, s);
        case T_Q4_0: return ref_matvec_t<T_Q4_0>(a, blocks, routes, s);
        case T_Q4_1: return ref_matvec_t<T_Q4_1>(a, blocks, routes, s);
        case T_Q5_0: return ref_matvec_t<T_Q5_0>(a, blocks, routes, s);
        case T_Q5_1: return ref_matvec_t<T_Q5_1>(a, blocks, routes, s);
        case T_Q2_K: return ref_matvec_t<T_Q2_K>(a, blocks, routes, s);
        case T_Q3_K: return ref_matvec_t<T_Q3_K>(a, blocks, routes, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool ref_matvec_supported(uint32_t type, uint32_t in) {
    switch (type) {
        case T_F32: return in >= 1u && in <= kMaxRefWidth;
        case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K:
            return in % 256u == 0u && in <= kMaxRefWidth && in / 256u <= 256u;
        case T_Q8_0: case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1:
            return in % 32u == 0u && in <= kMaxRefWidth && in / 32u <= 256u;
        default: return false;
    }
}

// Prologue limits: a fused norm covers one residual row of up to
// kMaxRefNormWidth values, routing up to 256 experts and top-16.
bool ref_prologue_ok(const RefMatvecArgs& a, uint32_t routes) {
    if (a.norm.w && (a.in > kMaxRefNormWidth || a.norm.res.K > kMaxRefTopK || routes != 1u))
        return false;
    if (a.route.logits &&
        (a.route.n_experts > kMaxExperts256 || a.route.top_k > kMaxRefTopK || routes > a.route.top_k))
        return false;
    return true;
}

hipError_t launch_ref_matvec(uint32_t type, const RefMatvecArgs& a, uint32_t routes, hipStream_t s) {
    if (!ref_prologue_ok(a, routes)) return hipErrorInvalidValue;
    if (type == T_F32) {
        if (a.route.logits || a.x_up || a.nseg) return hipErrorInvalidValue;
        size_t lds = (chain_floats(a.in) + a.in) * sizeof(float);
        if (a.norm.w) lds += (chain_floats(a.in) + a.in) * sizeof(float);
        hipLaunchKernelGGL(k_ref_linear_f32, dim3(a.rows, routes), dim3(256), lds, s, a);
        return hipGetLastError();
    }
    if (a.nseg) return hipErrorInvalidValue;
    const uint32_t rpw = 256u / (a.in / ref_block_elems(type));
    return ref_matvec_launch(type, a, (a.rows + rpw - 1u) / rpw, routes, s);
}

hipError_t launch_ref_matvec_multi(uint32_t type, RefMatvecArgs a, const RefSeg* segs, uint32_t n,
                                   uint32_t routes, hipStream_t s) {
    if (type == T_F32 || n == 0 || n > kMaxRefSegs || !ref_prologue_ok(a, routes))
        return hipErrorInvalidValue;
    const uint32_t rpw = 256u / (a.in / ref_block_elems(type));
    uint32_t blocks = 0;
    a.nseg = n;
    for (uint32_t j = 0; j < n; ++j) {
        a.seg[j] = segs[j];
        a.seg[j].block0 = blocks;
        blocks += (segs[j].rows + rpw - 1u) / rpw;
    }
    return ref_matvec_launch(type, a, blocks, routes, s);
}

bool ref_gate_up_act_supported(uint32_t type, uint32_t in) {
    return type != T_F32 && ref_matvec_supported(type, in) && in / ref_block_elems(type) <= 128u;
}

hipError_t launch_ref_gate_up_act(uint32_t type, RefMatvecArgs a, const RefSeg& gate,
                                  const RefSeg& up, uint32_t routes, hipStream_t s) {
    if (!ref_gate_up_act_supported(type, a.in) || !a.act || gate.rows != up.rows ||
        !ref_prologue_ok(a, routes))
        return hipErrorInvalidValue;
    const uint32_t rpw = 128u / (a.in / ref_block_elems(type));
    a.nseg = 2;
    a.seg[0] = gate;
    a.seg[1] = up;
    return ref_matvec_launch(type, a, (gate.rows + rpw - 1u) / rpw, routes, s);
}

hipError_t launch_ref_rmsnorm(float* x, const RefResidual& res, const float* w, float* out,
                              uint32_t n, uint32_t rows, float eps, hipStream_t s) {
    const size_t lds = chain_floats(n) * sizeof(float);
    if (n == 0 || n > kMaxRefWidth || res.K > kMaxRefTopK) return hipErrorInvalidValue;
    if (n <= 1024u) hipLaunchKernelGGL(k_ref_rmsnorm<1>, dim3(rows), dim3(1024), lds, s, x, res, w, out, n, eps);
    else if (n <= 2048u) hipLaunchKernelGGL(k_ref_rmsnorm<2>, dim3(rows), dim3(1024), lds, s, x, res, w, out, n, eps);
    else if (n <= 4096u) hipLaunchKernelGGL(k_ref_rmsnorm<4>, dim3(rows), dim3(1024), lds, s, x, res, w, out, n, eps);
    else hipLaunchKernelGGL(k_ref_rmsnorm<8>, dim3(rows), dim3(1024), lds, s, x, res, w, out, n, eps);
    return hipGetLastError();
}

bool ref_attention_supported(uint32_t head_dim, uint32_t capacity) {
    return (head_dim == 64u || head_dim == 128u || head_dim == 256u) &&
           (chain_floats(capacity) * 4ull + kAttnTileBytes) <= 160ull * 1024u - 8192u;
}

hipError_t launch_ref_attention(const ModelArgs& a, const ModelLayer& L, hipStream_t s) {
    const size_t lds = chain_floats(a.capacity) * sizeof(float) + kAttnTileBytes;
    switch (a.head_dim) {
        case 64: hipLaunchKernelGGL(k_ref_attention<64>, dim3(a.heads), dim3(256), lds, s, a, L); break;
        case 128: hipLaunchKernelGGL(k_ref_attention<128>, dim3(a.heads), dim3(256), lds, s, a, L); break;
        case 256: hipLaunchKernelGGL(k_ref_attention<256>, dim3(a.heads), dim3(256), lds, s, a, L); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_fast_attention(const ModelArgs& a, const ModelLayer& L, hipStream_t s) {
    const size_t lds = static_cast<size_t>(a.capacity) * sizeof(float);
    switch (a.head_dim) {
        case 64: hipLaunchKernelGGL(k_fast_attention<64>, dim3(a.heads), dim3(256), lds, s, a, L); break;
        case 128: hipLaunchKernelGGL(k_fast_attention<128>, dim3(a.heads), dim3(256), lds, s, a, L); break;
        case 256: hipLaunchKernelGGL(k_fast_attention<256>, dim3(a.heads), dim3(256), lds, s, a, L); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Six launches per layer; the residual stream alternates between
// hidden_state and hidden_alt so no workgroup reads a row another one of the
// same launch overwrites.
hipError_t launch_ref_step(const ModelArgs& a, const ModelLayer* layers, bool logits, hipStream_t s) {
    const uint32_t qd = a.heads * a.head_dim, kd = a.kv_heads * a.head_dim;
    RefResidual res{};  // what the next RMSNorm adds to the residual stream first
    hipError_t err = hipSuccess;
    for (uint32_t l = 0; l < a.layers; ++l) {
        const ModelLayer& L = layers[l];
        const MoeDecodeArgs& m = L.moe;
        // 1. attention RMSNorm (hidden_state + residual -> hidden_alt) and q/k/v
        RefMatvecArgs qkv{};
        qkv.in = a.hidden;
        qkv.norm = RefNormIn{a.hidden_state, res, L.attn_norm, a.hidden_alt, nullptr, a.rms_eps};
        const RefSeg qkv_segs[3] = {{L.q, L.q_row, 0, qd, 0, a.q},
                                    {L.k, L.k_row, 0, kd, 0, a.k},
                                    {L.v, L.v_row, 0, kd, 0, a.v}};
        if ((err = launch_ref_matvec_multi(L.attn_type, qkv, qkv_segs, 3, 1, s))) return err;
        // 2. q/k norms, RoPE, KV ring, attention
        if ((err = launch_ref_attention(a, L, s))) return err;
        // 3. output projection
        RefMatvecArgs o{};
        o.W = L.o;
        o.row_bytes = L.o_row;
        o.rows = a.hidden;
        o.in = qd;
        o.x = a.att;
        o.y = a.attn_out;
        if ((err = launch_ref_matvec(L.attn_type, o, 1, s))) return err;
        // 4. FFN RMSNorm (hidden_alt + attn_out -> hidden_state, normed) and router logits
        float* rl = a.ref_scratch;
        float* g = rl + kMaxExperts256;
        float* u = g + static_cast<uint64_t>(m.top_k) * m.ffn;
        float* out = u + static_cast<uint64_t>(m.top_k) * m.ffn;
        RefMatvecArgs router{};
        router.W = reinterpret_cast<const uint8_t*>(m.router);
        router.row_bytes = static_cast<uint64_t>(m.hidden) * 4u;
        router.rows = m.n_experts;
        router.in = m.hidden;
        router.norm = RefNormIn{a.hidden_alt, RefResidual{a.attn_out, nullptr, nullptr, 0},
                                L.ffn_norm, a.hidden_state, a.normed, a.rms_eps};
        router.y = rl;
        if ((err = launch_ref_matvec(T_F32, router, 1, s))) return err;
        // 5. routing and gate/up of every route
        RefMatvecArgs gu{};
        gu.in = m.hidden;
        gu.x = a.normed;
        gu.y_stride = m.ffn;
        gu.route = RefRouteIn{rl, m.n_experts, m.top_k, m.normalize, m.ids, m.probs, m.status};
        const RefSeg gu_segs[2] = {{m.gate, m.gate_row, m.gate_slice, m.ffn, 0, g},
                                   {m.up, m.up_row, m.up_slice, m.ffn, 0, u}};
        const bool paired = m.gate_type == m.up_type && ref_gate_up_act_supported(m.gate_type, m.hidden);
        if (paired) {  // the SwiGLU activations written by gate/up, into g
            gu.act = g;
            gu.expf = a.expf;
            if ((err = launch_ref_gate_up_act(m.gate_type, gu, gu_segs[0], gu_segs[1], m.top_k, s)))
                return err;
        } else if (m.gate_type == m.up_type) {
            if ((err = launch_ref_matvec_multi(m.gate_type, gu, gu_segs, 2, m.top_k, s))) return err;
        } else {
            if ((err = launch_ref_matvec_multi(m.gate_type, gu, gu_segs, 1, m.top_k, s))) return err;
            gu.route.logits = nullptr;  // the ids are written by now
            gu.ids = m.ids;
            if ((err = launch_ref_matvec_multi(m.up_type, gu, gu_segs + 1, 1, m.top_k, s))) return err;
        }
        // 6. down (the SwiGLU staged in it unless gate/up wrote the activations)
        RefMatvecArgs d{};
        d.ids = m.ids;
        d.W = m.down;
        d.row_bytes = m.down_row;
        d.slice_bytes = m.down_slice;
        d.rows = m.hidden;
        d.in = m.ffn;
        d.x = g;
        d.x_up = paired ? nullptr : u;
        d.x_stride = m.ffn;
        d.expf = a.expf;
        d.y = out;
        d.y_stride = m.hidden;
        if ((err = launch_ref_matvec(m.down_type, d, m.top_k, s))) return err;
        res = RefResidual{nullptr, out, m.probs, m.top_k};
    }
    if (!logits) return hipGetLastError();
    if ((err = launch_ref_rmsnorm(a.hidden_state, res, a.out_norm, a.normed, a.hidden, 1, a.rms_eps,
                                  s)))
        return err;
    RefMatvecArgs h{};
    h.W = a.out;
    h.row_bytes = a.out_row;
    h.rows = a.vocab;
    h.in = a.hidden;
    h.x = a.normed;
    h.y = a.logits;
    return launch_ref_matvec(a.out_type, h, 1, s);
}

namespace {

// moe_result = ((0 + p0 * o0) + p1 * o1) + ... in route order
// (src/qwen3_moe_runner.cpp:652,688-690: the zero-filled result, then
// moe_result[i] += probability * expert_output[i] per route).
__global__ __launch_bounds__(256) void k_ref_combine(const float* __restrict__ parts,
                                                     const float* __restrict__ probs, uint32_t K,
                                                     uint32_t n, float* __restrict__ y) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    float acc = 0.0f;
    for (uint32_t r = 0; r < K; ++r)
        acc = __fadd_rn(acc, __fmul_rn(probs[r], parts[static_cast<uint64_t>(r) * n + i]));
    y[i] = acc;
}

__global__ __launch_bounds__(256) void k_expf_block_sums(LibmExpf t, uint32_t first_bits,
                                                         uint32_t block_size,
                                                         unsigned long long* sums) {
    const uint32_t base = first_bits + blockIdx.x * block_size;
    unsigned long long acc = 0;
    for (uint32_t i = threadIdx.x; i < block_size; i += 256u) {
        const uint32_t b = base + i;
        const uint32_t r = __float_as_uint(expf_libm(__uint_as_float(b), t));
        acc += ((static_cast<unsigned long long>(r) << 32) | b) * 0xD6E8FEB86659FD93ull;
    }
    __shared__ unsigned long long part[4];
    // wave sums with integer shuffles (order-independent: addition mod 2^64)
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63u) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) sums[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

}  // namespace

bool ref_moe_block_supported(const MoeDecodeArgs& m) {
    return m.variant == 0 && m.n_experts >= 1 && m.n_experts <= kMaxExperts256 && m.top_k >= 1 &&
           m.top_k <= kMaxRefTopK && m.top_k <= m.n_experts &&
           ref_matvec_supported(T_F32, m.hidden) && ref_matvec_supported(m.gate_type, m.hidden) &&
           ref_matvec_supported(m.up_type, m.hidden) && ref_matvec_supported(m.down_type, m.ffn) &&
           m.gate_type != T_F32 && m.up_type != T_F32 && m.down_type != T_F32;
}

// The MoE block in the reference's order: the router rows, routing and
// gate/up (with the SwiGLU activations where the pairing covers the width),
// down, then the route-order combine -- stages 4-6 of launch_ref_step without
// the RMSNorm, on a caller's normalised x.
hipError_t launch_ref_moe_block(const MoeDecodeArgs& m, float* scratch, const LibmExpf& expf,
                                hipStream_t s) {
    if (!ref_moe_block_supported(m)) return hipErrorInvalidValue;
    float* rl = scratch;
    float* g = rl + kMaxExperts256;
    float* u = g + static_cast<uint64_t>(m.top_k) * m.ffn;
    float* out = u + static_cast<uint64_t>(m.top_k) * m.ffn;
    hipError_t err;
    RefMatvecArgs router{};
    router.W = reinterpret_cast<const uint8_t*>(m.router);
    router.row_bytes = static_cast<uint64_t>(m.hidden) * 4u;
    router.rows = m.n_experts;
    router.in = m.hidden;
    router.x = m.x;
    router.y = rl;
    if ((err = launch_ref_matvec(T_F32, router, 1, s))) return err;
    RefMatvecArgs gu{};
    gu.in = m.hidden;
    gu.x = m.x;
    gu.y_stride = m.ffn;
    gu.route = RefRouteIn{rl, m.n_experts, m.top_k, m.normalize, m.ids, m.probs, m.status};
    const RefSeg gu_segs[2] = {{m.gate, m.gate_row, m.gate_slice, m.ffn, 0, g},
                               {m.up, m.up_row, m.up_slice, m.ffn, 0, u}};
    const bool paired = m.gate_type == m.up_type && ref_gate_up_act_supported(m.gate_type, m.hidden);
    if (paired) {
        gu.act = g;
        gu.expf = expf;
        if ((err = launch_ref_gate_up_act(m.gate_type, gu, gu_segs[0], gu_segs[1], m.top_k, s)))
            return err;
    } else if (m.gate_type == m.up_type) {
        if ((err = launch_ref_matvec_multi(m.gate_type, gu, gu_segs, 2, m.top_k, s))) return err;
    } else {
        if ((err = launch_ref_matvec_multi(m.gate_type, gu, gu_segs, 1, m.top_k, s))) return err;
        gu.route.logits = nullptr;  // the ids are written by now
        gu.ids = m.ids;
        if ((err = launch_ref_matvec_multi(m.up_type, gu, gu_segs + 1, 1, m.top_k, s))) return err;
    }
    RefMatvecArgs d{};
    d.ids = m.ids;
    d.W = m.down;
    d.row_bytes = m.down_row;
    d.slice_bytes = m.down_slice;
    d.rows = m.hidden;
    d.in = m.ffn;
    d.x = g;
    d.x_up = paired ? nullptr : u;
    d.x_stride = m.ffn;
    d.expf = expf;
    d.y = out;
    d.y_stride = m.hidden;
    if ((err = launch_ref_matvec(m.down_type, d, m.top_k, s))) return err;
    hipLaunchKernelGGL(k_ref_combine, dim3((m.hidden + 255u) / 256u), dim3(256), 0, s, out, m.probs,
                       m.top_k, m.hidden, m.y);
    return hipGetLastError();
}

hipError_t launch_expf_block_sums(const LibmExpf& t, uint32_t first_bits, uint32_t block_size,
                                  uint32_t n_blocks, unsigned long long* sums, hipStream_t s) {
    if (n_blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(k_expf_block_sums, dim3(n_blocks), dim3(256), 0, s, t, first_bits,
                       block_size, sums);
    return hipGetLastError();
}

}  // namespace pk
