// kquant.hpp -- device-side GGUF block decoding for gfx950 matrix-vector work.
//
// A row of a GGUF matrix is a run of encoded blocks.  Each block is split into
// "units": UB consecutive bytes of the block's primary quant stream, the
// natural 4/8/16-byte load of one lane.  Decoding a unit yields RUNS runs of
// UB elements whose activation columns are fixed for a given unit index, so a
// lane keeps the activations of its units in registers and streams rows past
// them.  Per-run sums use the factored form
//     sum_i w_i x_i = (d*sc) * sum_i q_i x_i  -  (dmin*m) * sum_i x_i
// (with a bias folded into sum_i x_i for the signed formats), which is
// algebraically the reference decode-then-dot of src/quantized_linear.cpp
// (:166-205, :286-358, :387-423) with a different FP32 rounding order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "layout.hpp"

namespace pk {

enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q2_K = 10,
    T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30
};

template <int T> struct Fmt;
// BE: elements per block, BB: bytes per block, PRIM: bytes of the primary
// quant stream per block, RUNS: element runs per unit.
template <> struct Fmt<T_Q4_K> { static constexpr int BE = 256, BB = 144, PRIM = 128, RUNS = 2, MAXUB = 32; };
template <> struct Fmt<T_Q5_K> { static constexpr int BE = 256, BB = 176, PRIM = 128, RUNS = 2, MAXUB = 32; };
template <> struct Fmt<T_Q6_K> { static constexpr int BE = 256, BB = 210, PRIM = 128, RUNS = 2, MAXUB = 16; };
template <> struct Fmt<T_Q8_0> { static constexpr int BE = 32, BB = 34, PRIM = 32, RUNS = 1, MAXUB = 16; };
template <> struct Fmt<T_Q4_0> { static constexpr int BE = 32, BB = 18, PRIM = 16, RUNS = 2, MAXUB = 16; };
template <> struct Fmt<T_Q4_1> { static constexpr int BE = 32, BB = 20, PRIM = 16, RUNS = 2, MAXUB = 16; };
template <> struct Fmt<T_Q5_0> { static constexpr int BE = 32, BB = 22, PRIM = 16, RUNS = 2, MAXUB = 16; };
template <> struct Fmt<T_Q5_1> { static constexpr int BE = 32, BB = 24, PRIM = 16, RUNS = 2, MAXUB = 16; };
// Q2_K / Q3_K: a quant byte holds four 2-bit fields, one per shift pair, so
// a unit of UB quant bytes covers four runs of UB elements.
template <> struct Fmt<T_Q2_K> { static constexpr int BE = 256, BB = 84, PRIM = 64, RUNS = 4, MAXUB = 16; };
template <> struct Fmt<T_Q3_K> { static constexpr int BE = 256, BB = 110, PRIM = 64, RUNS = 4, MAXUB = 16; };

// ---------------------------------------------------------------------------
// Loads.  Q4_K/Q5_K blocks (144/176 B) keep 16-byte alignment and Q4_1,
// Q5_1 and Q2_K (20/24/84 B) 4-byte alignment: they are read in GGUF form.
// Q6_K, Q8_0, Q4_0, Q5_0 and Q3_K only keep 2-byte alignment and are held in
// the planar layout of layout.hpp, each field an aligned load.

template <int N>
__device__ __forceinline__ void ld_words(const uint8_t* p, uint32_t (&w)[N]) {
    __builtin_memcpy(w, __builtin_assume_aligned(p, 4), 4 * N);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Streaming variant for weights read once: nontemporal loads (16-byte
// pieces, then single dwords), so they do not displace reused data in L2.
template <int N>
__device__ __forceinline__ void ld_words_nt(const uint8_t* p, uint32_t (&w)[N]) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
        const u32x4_t v = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(__builtin_assume_aligned(p + 16 * i, 4)));
        w[4 * i + 0] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = 4 * (N / 4); i < N; ++i)
        w[i] = __builtin_nontemporal_load(
            reinterpret_cast<const uint32_t*>(__builtin_assume_aligned(p + 4 * i, 4)));
}

#ifndef PK_WEIGHT_NT
#define PK_WEIGHT_NT 1
#endif
template <int N>
__device__ __forceinline__ void ld_weights(const uint8_t* p, uint32_t (&w)[N]) {
    if constexpr (PK_WEIGHT_NT) ld_words_nt<N>(p, w);
    else ld_words<N>(p, w);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(__builtin_assume_aligned(p, 2));
}

// v_cvt_f32_ubyteN: byte N of a word as float in one instruction (the
// compiler otherwise emits bfe + cvt for pre-masked words).
template <int N>
__device__ __forceinline__ float ub(uint32_t v) {
    float r;
    if constexpr (N == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (N == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (N == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// dot += bytes(v) . x[0..3]
__device__ __forceinline__ float dot4(uint32_t v, const float* x, float acc) {
    acc = __builtin_fmaf(ub<0>(v), x[0], acc);
    acc = __builtin_fmaf(ub<1>(v), x[1], acc);
    acc = __builtin_fmaf(ub<2>(v), x[2], acc);
    acc = __builtin_fmaf(ub<3>(v), x[3], acc);
    return acc;
}

// 6-bit (scale, min) pair j of a Q4_K/Q5_K block from header words h[1..3]
// (the 12 packed bytes at block+4; scale_min, src/quantized_linear.cpp:176-188).
__device__ __forceinline__ void kq_scale_min(const uint32_t (&h)[4], uint32_t j, float& s,
                                             float& m) {
    const uint32_t sh = 8u * (j & 3u);
    const uint32_t by = (h[1] >> sh) & 0xffu, bz = (h[2] >> sh) & 0xffu, bw = (h[3] >> sh) & 0xffu;
    const uint32_t s_lo = by & 63u, m_lo = bz & 63u;
    const uint32_t s_hi = (bw & 15u) | ((by >> 6) << 4), m_hi = (bw >> 4) | ((bz >> 6) << 4);
    s = static_cast<float>(j < 4 ? s_lo : s_hi);
    m = static_cast<float>(j < 4 ? m_lo : m_hi);
}

// Pairs 2c and 2c + 1 (c = 0..3) of a Q4_K/Q5_K block at once, without
// branches: both sit in the low-index form (c < 2: six bits of byte j of
// h[1] / h[2]) or both in the high-index form (c >= 2: a nibble of byte j & 3
// of h[3] and two bits of h[1] / h[2]); a zero-width extract drops the top
// bits of the low-index form.
__device__ __forceinline__ void kq_scale_min_pair(const uint32_t (&h)[4], uint32_t c, uint32_t& s0,
                                                  uint32_t& m0, uint32_t& s1, uint32_t& m1) {
    const bool lo = c < 2u;
    const uint32_t o0 = 16u * (c & 1u), o1 = o0 + 8u;
    const uint32_t hs = lo ? h[1] : h[3], hm = lo ? h[2] : h[3];
    const uint32_t w = lo ? 6u : 4u, wt = lo ? 0u : 2u, om = lo ? 0u : 4u;
    s0 = __builtin_amdgcn_ubfe(hs, o0, w) | (__builtin_amdgcn_ubfe(h[1], o0 + 6u, wt) << 4);
    s1 = __builtin_amdgcn_ubfe(hs, o1, w) | (__builtin_amdgcn_ubfe(h[1], o1 + 6u, wt) << 4);
    m0 = __builtin_amdgcn_ubfe(hm, o0 + om, w) | (__builtin_amdgcn_ubfe(h[2], o0 + 6u, wt) << 4);
    m1 = __builtin_amdgcn_ubfe(hm, o1 + om, w) | (__builtin_amdgcn_ubfe(h[2], o1 + 6u, wt) << 4);
}

// The fp16 value of the low / high half of a word, widened to fp32.  Used on
// masked quant words, whose halves are fp16 subnormals (small integers times
// 2^-24): an FMA on the result compiles to one v_fma_mix_f32.
__device__ __forceinline__ float half_lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// Bits 0..3 of b to bit 4 of bytes 0..3 (the Q5_0/Q5_1 fifth bits).
__device__ __forceinline__ uint32_t spread4(uint32_t b) {
    return ((b & 1u) << 4) | ((b & 2u) << 11) | ((b & 4u) << 18) | ((b & 8u) << 25);
}

// 6-bit scale j of a Q3_K block from its 12 packed bytes (words w[0..2]): the
// low nibble in byte j (j < 8) or in the high nibble of byte j - 8, the top two
// bits at bits 2 * (j / 4) of byte 8 + j % 4 (decode_q3_k,
// src/quantized_linear.cpp:127-139).
__device__ __forceinline__ uint32_t q3k_scale(const uint32_t (&w)[3], uint32_t j) {
    const uint32_t jl = j & 7u;
    const uint32_t lob = (w[jl / 4u] >> (8u * (jl % 4u))) & 0xffu;
    const uint32_t lo = j < 8u ? lob & 15u : lob >> 4;
    const uint32_t hib = (w[2] >> (8u * (j % 4u))) & 0xffu;
    return lo | (((hib >> (2u * (j / 4u))) & 3u) << 4);
}

// ---------------------------------------------------------------------------
// Unit geometry.  Unit u of a row: block b = u / UPB, unit j = u % UPB inside
// the block, primary byte offset k0 = j * UB.  col[r] is the activation column
// of the first element of run r.  All of it is row-independent.

struct UnitPos {
    uint32_t b;       // block index inside the row
    uint32_t k0;      // primary-stream byte offset inside the block
    uint32_t col[4];  // activation column of the first element of each run
};

template <int T, int UB>
__device__ __forceinline__ UnitPos unit_pos(uint32_t u) {
    using F = Fmt<T>;
    constexpr uint32_t UPB = F::PRIM / UB;
    const uint32_t b = u / UPB, j = u % UPB, k0 = j * UB;
    UnitPos p;
    p.b = b;
    p.k0 = k0;
    const uint32_t base = b * F::BE;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        p.col[0] = base + 64u * (k0 / 32u) + (k0 % 32u);
        p.col[1] = p.col[0] + 32u;
    } else if constexpr (T == T_Q6_K) {
        const uint32_t kk = k0 % 64u;
        p.col[0] = base + 128u * (k0 / 64u) + (kk >= 32u ? 32u : 0u) + (kk % 32u);
        p.col[1] = p.col[0] + 64u;
    } else if constexpr (T == T_Q8_0) {
        p.col[0] = base + k0;
        p.col[1] = p.col[0];
    } else if constexpr (T == T_Q2_K || T == T_Q3_K) {
        // quant byte 32h + 16t + i holds element 128h + 32s + 16t + i at bits 2s
        const uint32_t h = k0 / 32u, t = (k0 % 32u) / 16u;
#pragma unroll
        for (uint32_t s = 0; s < 4; ++s) p.col[s] = base + 128u * h + 32u * s + 16u * t + (k0 % 16u);
    } else {  // Q4_0, Q4_1, Q5_0, Q5_1: low nibbles are elements 0..15, high nibbles 16..31
        p.col[0] = base + k0;
        p.col[1] = p.col[0] + 16u;
    }
    return p;
}

// Activations of one unit for B vectors: xv[b][r*UB + i] = x[b][col[r] + i],
// xs[b][r] = sum_i xv[b][r*UB + i].
template <int T, int UB, int B>
struct UnitX {
    static constexpr int R = Fmt<T>::RUNS;
    float v[B][R * UB];
    float s[B][R];
};

// The loads are unconditional (an absent unit's position is unit 0's, in
// bounds) and the values are zeroed afterwards: a load inside a branch makes
// the wave wait at the branch's end for every load issued before it, here
// the weight loads the caller has just issued.
template <int T, int UB, int B>
__device__ __forceinline__ void load_unit_x(const float* x, uint32_t x_stride, const UnitPos& p,
                                            bool valid, UnitX<T, UB, B>& ux) {
    constexpr int R = Fmt<T>::RUNS;
#pragma unroll
    for (int b = 0; b < B; ++b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < UB; i += 4) {
                float4 v = *reinterpret_cast<const float4*>(x + b * x_stride + p.col[r] + i);
                if (!valid) v = make_float4(0.f, 0.f, 0.f, 0.f);
                ux.v[b][r * UB + i + 0] = v.x;
                ux.v[b][r * UB + i + 1] = v.y;
                ux.v[b][r * UB + i + 2] = v.z;
                ux.v[b][r * UB + i + 3] = v.w;
                sum += (v.x + v.y) + (v.z + v.w);
            }
            ux.s[b][r] = sum;
        }
    }
}

// One vector's activations staged in LDS lane-major, for waves that share
// them: piece q (float4 q of the unit's runs, run q / (UB / 4)) of unit slot
// k of unit lane ul sits at [(k * Q + q) * G + ul], so every LDS read of a
// wave is G consecutive float4s (lanes that share a unit read the same
// address) and no two lanes of a read meet in one bank, whatever the format's
// column pattern.
template <int T, int UB>
constexpr int x_pieces() { return Fmt<T>::RUNS * UB / 4; }

// (a vector type: an array of HIP's float4 class would live in scratch)
typedef float xf32x4 __attribute__((ext_vector_type(4)));

// Activation column of piece q of the unit at p: selects, not an indexed
// array (which would live in scratch when q is not a constant).
template <int T, int UB>
__device__ __forceinline__ uint32_t piece_col(const UnitPos& p, uint32_t q) {
    const uint32_t r = q / (UB / 4), i = q % (UB / 4);
    uint32_t col = p.col[0];
#pragma unroll
    for (int rr = 1; rr < Fmt<T>::RUNS; ++rr) col = r == static_cast<uint32_t>(rr) ? p.col[rr] : col;
    return col + 4u * i;
}

// load_unit_x from staged pieces (slot = the unit slot's piece 0 for this
// lane, pieces G float4s apart; vector b's pieces follow vector b - 1's).
template <int T, int UB, int B = 1>
__device__ __forceinline__ void load_unit_x_staged(const xf32x4* slot, uint32_t G,
                                                   UnitX<T, UB, B>& ux) {
    constexpr int R = Fmt<T>::RUNS, Q = x_pieces<T, UB>();
#pragma unroll
    for (int b = 0; b < B; ++b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < UB; i += 4) {
                const xf32x4 v = slot[(b * Q + r * (UB / 4) + i / 4) * G];
                ux.v[b][r * UB + i + 0] = v.x;
                ux.v[b][r * UB + i + 1] = v.y;
                ux.v[b][r * UB + i + 2] = v.z;
                ux.v[b][r * UB + i + 3] = v.w;
                sum += (v.x + v.y) + (v.z + v.w);
            }
            ux.s[b][r] = sum;
        }
    }
}

// Activation pieces of one unit as loaded, before they become a UnitX: a
// wave issues them ahead of its weight loads and converts them after, since
// the first use of a load waits for every load issued before it.  NP = Q
// (every piece of the unit) or Q / 2 (one half of a wave whose two 32-lane
// halves hold the same units, lane l and lane l + 32 dotting two rows
// against one vector).
template <int NP>
struct XRaw {
    xf32x4 v[NP];
};

template <int T, int UB>
__device__ __forceinline__ void load_x_pieces(const float* x, const UnitPos& p,
                                              XRaw<x_pieces<T, UB>()>& r) {
#pragma unroll
    for (int q = 0; q < x_pieces<T, UB>(); ++q)
        r.v[q] = *reinterpret_cast<const xf32x4*>(x + piece_col<T, UB>(p, q));
}

// Half h of the wave loads pieces [h Q/2, (h + 1) Q/2) of its lane's unit.
template <int T, int UB>
__device__ __forceinline__ void load_x_half(const float* x, const UnitPos& p, uint32_t h,
                                            XRaw<x_pieces<T, UB>() / 2>& r) {
    constexpr int H = x_pieces<T, UB>() / 2;
    static_assert(x_pieces<T, UB>() % 2 == 0, "pieces split evenly between the halves");
#pragma unroll
    for (int i = 0; i < H; ++i) r.v[i] = *reinterpret_cast<const xf32x4*>(x + piece_col<T, UB>(p, h * H + i));
}

// The UnitX of load_unit_x (same values, same sums) from loaded pieces.
template <int T, int UB>
__device__ __forceinline__ void unit_x_sums(UnitX<T, UB, 1>& ux) {
#pragma unroll
    for (int r = 0; r < Fmt<T>::RUNS; ++r) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < UB; i += 4)
            sum += (ux.v[0][r * UB + i] + ux.v[0][r * UB + i + 1]) +
                   (ux.v[0][r * UB + i + 2] + ux.v[0][r * UB + i + 3]);
        ux.s[0][r] = sum;
    }
}

template <int T, int UB>
__device__ __forceinline__ void unit_x_from_pieces(const XRaw<x_pieces<T, UB>()>& r, bool valid,
                                                   UnitX<T, UB, 1>& ux) {
#pragma unroll
    for (int q = 0; q < x_pieces<T, UB>(); ++q)
#pragma unroll
        for (int c = 0; c < 4; ++c) ux.v[0][4 * q + c] = valid ? r.v[q][c] : 0.0f;
    unit_x_sums<T, UB>(ux);
}

// From the two halves' pieces: v_permlane32_swap exchanges lanes 32..63 of
// its first operand with lanes 0..31 of its second; with both operands the
// same register, the first result is half 0's value and the second half 1's,
// in every lane.  Every activation float so passes the vector load path once
// per wave instead of twice.
template <int T, int UB>
__device__ __forceinline__ void unit_x_from_halves(const XRaw<x_pieces<T, UB>() / 2>& r, bool valid,
                                                   UnitX<T, UB, 1>& ux) {
    constexpr int H = x_pieces<T, UB>() / 2;
#pragma unroll
    for (int i = 0; i < H; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t w = valid ? __float_as_uint(r.v[i][c]) : 0u;
            const auto sw = __builtin_amdgcn_permlane32_swap(w, w, false, false);
            ux.v[0][4 * i + c] = __uint_as_float(sw[0]);
            ux.v[0][4 * H + 4 * i + c] = __uint_as_float(sw[1]);
        }
    unit_x_sums<T, UB>(ux);
}

// As load_unit_x_staged, with the run sums from piece sums staged beside the
// pieces: ps holds this lane's Q piece sums of vector 0 ((v.x + v.y) + (v.z +
// v.w) of each piece), vector b's 64 * Q floats later.  The run sum adds them
// in piece order from zero, the same additions as load_unit_x_staged, so the
// same bits, without every wave repeating them.
template <int T, int UB, int B = 1>
__device__ __forceinline__ void load_unit_x_staged_ps(const xf32x4* slot, uint32_t G, const float* ps,
                                                      UnitX<T, UB, B>& ux) {
    constexpr int R = Fmt<T>::RUNS, Q = x_pieces<T, UB>();
#pragma unroll
    for (int b = 0; b < B; ++b) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < UB; i += 4) {
                const xf32x4 v = slot[(b * Q + r * (UB / 4) + i / 4) * G];
                ux.v[b][r * UB + i + 0] = v.x;
                ux.v[b][r * UB + i + 1] = v.y;
                ux.v[b][r * UB + i + 2] = v.z;
                ux.v[b][r * UB + i + 3] = v.w;
                sum += ps[b * 64 * Q + r * (UB / 4) + i / 4];
            }
            ux.s[b][r] = sum;
        }
    }
}

// ---------------------------------------------------------------------------
// Unit decode in two phases, so a wave can issue the loads of several rows
// before it consumes any of them.

template <int T, int UB>
struct UnitRaw {
    static constexpr int NW = UB / 4;
    // h: Q4_K/Q5_K block header; Q4_1/Q5_1 d | m << 16; Q2_K d | dmin << 16.
    // q: the unit's quant bytes.  qh: Q5_K fifth bits, Q6_K high bits, Q3_K
    // hmask bytes (per unit byte), Q5_0/Q5_1 the block's 32-bit qh.  sc: Q6_K
    // scale dwords of the half block, Q2_K scale/min bytes 8h..8h+7, Q3_K the
    // 12 packed scale bytes.  d: fp16 bits of d (Q6_K, Q8_0, Q4_0, Q5_0, Q3_K).
    static constexpr int NH = (T == T_Q4_K || T == T_Q5_K) ? 4 : 1;
    static constexpr int NQH = (T == T_Q5_K || T == T_Q6_K || T == T_Q3_K) ? NW : 1;
    static constexpr int NSC = T == T_Q3_K ? 3 : (T == T_Q6_K || T == T_Q2_K) ? 2 : 1;
    uint32_t h[NH];
    uint32_t q[NW];
    uint32_t qh[NQH];
    uint32_t sc[NSC];
    uint32_t d;
};

// Loads of one unit of row `r`: quants with one (UB = 16) aligned load per
// field, scales as whole dwords.
template <int T, int UB>
__device__ __forceinline__ void unit_load(const QRow& r, const UnitPos& p, UnitRaw<T, UB>& u) {
    constexpr int NW = UB / 4;
    if constexpr (T == T_Q4_1) {  // 20-byte blocks keep 4-byte alignment: d, m, then quants
        const uint8_t* blk = block_ptr<20>(r, p.b);
        ld_weights<1>(blk, u.h);
        ld_weights<NW>(blk + 4 + p.k0, u.q);
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = block_ptr<Fmt<T>::BB>(r, p.b);
        ld_weights<4>(blk, u.h);
        ld_weights<NW>(blk + (T == T_Q4_K ? 16 : 48) + p.k0, u.q);
        if constexpr (T == T_Q5_K) ld_weights<NW>(blk + 16 + (p.k0 % 32u), u.qh);
    } else if constexpr (T == T_Q6_K) {
        using L = Planar<T_Q6_K>;
        const uint32_t half = p.k0 / 64u, kk = p.k0 % 64u;
        ld_weights<NW>(field_ptr<L::QL, 128>(r, p.b) + p.k0, u.q);
        ld_weights<NW>(field_ptr<L::QH, 64>(r, p.b) + 32u * half + (kk % 32u), u.qh);
        ld_weights<2>(field_ptr<L::SC, 16>(r, p.b) + 8u * half, u.sc);
        u.d = ld_u16(field_ptr<L::D, 2>(r, p.b));
    } else if constexpr (T == T_Q8_0) {
        using L = Planar<T_Q8_0>;
        ld_weights<NW>(field_ptr<L::QS, 32>(r, p.b) + p.k0, u.q);
        u.d = ld_u16(field_ptr<L::D, 2>(r, p.b));
    } else if constexpr (T == T_Q5_0) {
        using L = Planar<T_Q5_0>;
        ld_weights<NW>(field_ptr<L::QS, 16>(r, p.b) + p.k0, u.q);
        ld_weights<1>(field_ptr<L::QH, 4>(r, p.b), u.qh);
        u.d = ld_u16(field_ptr<L::D, 2>(r, p.b));
    } else if constexpr (T == T_Q5_1) {  // 24-byte blocks: d, m, qh, quants
        const uint8_t* blk = block_ptr<24>(r, p.b);
        ld_weights<1>(blk, u.h);
        ld_weights<1>(blk + 4, u.qh);
        ld_weights<NW>(blk + 8 + p.k0, u.q);
    } else if constexpr (T == T_Q2_K) {  // 84-byte blocks: scales[16], qs[64], d, dmin
        const uint8_t* blk = block_ptr<84>(r, p.b);
        ld_weights<NW>(blk + 16 + p.k0, u.q);
        ld_weights<2>(blk + 8u * (p.k0 / 32u), u.sc);
        ld_weights<1>(blk + 80, u.h);
    } else if constexpr (T == T_Q3_K) {
        using L = Planar<T_Q3_K>;
        ld_weights<NW>(field_ptr<L::QS, 64>(r, p.b) + p.k0, u.q);
        ld_weights<NW>(field_ptr<L::HM, 32>(r, p.b) + (p.k0 % 32u), u.qh);
        ld_weights<3>(field_ptr<L::SC, 12>(r, p.b), u.sc);
        u.d = ld_u16(field_ptr<L::D, 2>(r, p.b));
    } else {  // Q4_0
        using L = Planar<T_Q4_0>;
        ld_weights<NW>(field_ptr<L::QS, 16>(r, p.b) + p.k0, u.q);
        u.d = ld_u16(field_ptr<L::D, 2>(r, p.b));
    }
}

// The two nibble runs of a unit's quant words (low nibbles: run 0, high:
// run 1) dotted with the activations in element order.  One vector: element
// pairs (0, 2) and (1, 3) of each word sit in the two halves of a masked word,
// and a nibble q there is the fp16 subnormal q * 2^-24 (16 q * 2^-24 for the
// high nibbles, masked in place), which v_fma_mix_f32 widens exactly inside
// the FMA: the dots are the exact 2^-24 / 2^-20 multiples of the plain q.x
// sums (same order, same roundings), and the caller scales them back.
// Several vectors: bytes converted once (dot4) and shared by the vectors.
template <int UB, int B, int T>
__device__ __forceinline__ void nibble_dots(const uint32_t (&q)[UB / 4], const UnitX<T, UB, B>& ux,
                                            float (&dot0)[B], float (&dot1)[B]) {
#pragma unroll
    for (int t = 0; t < UB / 4; ++t) {
        if constexpr (B == 1) {
            const uint32_t s = q[t] >> 8;
            const uint32_t l02 = q[t] & 0x000f000fu, l13 = s & 0x000f000fu;
            const uint32_t h02 = q[t] & 0x00f000f0u, h13 = s & 0x00f000f0u;
            const float* x0 = &ux.v[0][4 * t];
            const float* x1 = &ux.v[0][UB + 4 * t];
            dot0[0] = __builtin_fmaf(half_lo(l02), x0[0], dot0[0]);
            dot0[0] = __builtin_fmaf(half_lo(l13), x0[1], dot0[0]);
            dot0[0] = __builtin_fmaf(half_hi(l02), x0[2], dot0[0]);
            dot0[0] = __builtin_fmaf(half_hi(l13), x0[3], dot0[0]);
            dot1[0] = __builtin_fmaf(half_lo(h02), x1[0], dot1[0]);
            dot1[0] = __builtin_fmaf(half_lo(h13), x1[1], dot1[0]);
            dot1[0] = __builtin_fmaf(half_hi(h02), x1[2], dot1[0]);
            dot1[0] = __builtin_fmaf(half_hi(h13), x1[3], dot1[0]);
        } else {
            const uint32_t lo = q[t] & 0x0f0f0f0fu, hi = (q[t] >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                dot0[b] = dot4(lo, &ux.v[b][4 * t], dot0[b]);
                dot1[b] = dot4(hi, &ux.v[b][UB + 4 * t], dot1[b]);
            }
        }
    }
}

template <int T, int UB, int B>
__device__ __forceinline__ void unit_compute(const UnitRaw<T, UB>& r, const UnitPos& p,
                                             const UnitX<T, UB, B>& ux, float (&acc)[B]) {
    constexpr int NW = UB / 4;
    float dot0[B], dot1[B];
#pragma unroll
    for (int b = 0; b < B; ++b) dot0[b] = dot1[b] = 0.0f;

    if constexpr (T == T_Q4_K) {
        // the scales carry nibble_dots' 2^24 / 2^20 factors back (one vector)
        const uint32_t c = p.k0 / 32u;
        nibble_dots<UB, B>(r.q, ux, dot0, dot1);
        uint32_t s0, m0, s1, m1;
        kq_scale_min_pair(r.h, c, s0, m0, s1, m1);
        const float d = half_bits_to_float(r.h[0] & 0xffffu);
        const float dmin = half_bits_to_float(r.h[0] >> 16);
        const float ds0 = (B == 1 ? d * 0x1p24f : d) * static_cast<float>(s0);
        const float ds1 = (B == 1 ? d * 0x1p20f : d) * static_cast<float>(s1);
        const float dm0 = dmin * static_cast<float>(m0), dm1 = dmin * static_cast<float>(m1);
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float t0 = __builtin_fmaf(ds0, dot0[b], -dm0 * ux.s[b][0]);
            const float t1 = __builtin_fmaf(ds1, dot1[b], -dm1 * ux.s[b][1]);
            acc[b] += t0 + t1;
        }
    } else if constexpr (T == T_Q5_K) {
        const uint32_t c = p.k0 / 32u;
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            uint32_t lo = r.q[t] & 0x0f0f0f0fu;
            uint32_t hi = (r.q[t] >> 4) & 0x0f0f0f0fu;
            if constexpr (T == T_Q5_K) {
                lo |= ((r.qh[t] >> (2u * c)) & 0x01010101u) << 4;
                hi |= ((r.qh[t] >> (2u * c + 1u)) & 0x01010101u) << 4;
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                dot0[b] = dot4(lo, &ux.v[b][4 * t], dot0[b]);
                dot1[b] = dot4(hi, &ux.v[b][UB + 4 * t], dot1[b]);
            }
        }
        const float d = half_bits_to_float(r.h[0] & 0xffffu);
        const float dmin = half_bits_to_float(r.h[0] >> 16);
        float s0, m0, s1, m1;
        kq_scale_min(r.h, 2u * c, s0, m0);
        kq_scale_min(r.h, 2u * c + 1u, s1, m1);
        const float ds0 = d * s0, dm0 = dmin * m0, ds1 = d * s1, dm1 = dmin * m1;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float t0 = __builtin_fmaf(ds0, dot0[b], -dm0 * ux.s[b][0]);
            const float t1 = __builtin_fmaf(ds1, dot1[b], -dm1 * ux.s[b][1]);
            acc[b] += t0 + t1;
        }
    } else if constexpr (T == T_Q6_K) {
        const uint32_t sl = (p.k0 % 64u) >= 32u ? 2u : 0u;
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            const uint32_t ql = r.q[t], qh = r.qh[t];
            const uint32_t lo = (ql & 0x0f0f0f0fu) | ((qh << (4u - sl)) & 0x30303030u);
            const uint32_t hi = ((ql >> 4) & 0x0f0f0f0fu) | ((qh >> sl) & 0x30303030u);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                dot0[b] = dot4(lo, &ux.v[b][4 * t], dot0[b]);
                dot1[b] = dot4(hi, &ux.v[b][UB + 4 * t], dot1[b]);
            }
        }
        // the unit's scales: sc[s] and sc[s + 4] of the block, s = its 16-group
        // (s % 4 is the same byte of the half's two scale dwords)
        const uint32_t sb = 8u * (((p.k0 % 64u) >= 32u ? 2u : 0u) + ((p.k0 % 32u) / 16u));
        const float d = half_bits_to_float(r.d);
        const float s0 = static_cast<float>(static_cast<int8_t>((r.sc[0] >> sb) & 0xffu));
        const float s1 = static_cast<float>(static_cast<int8_t>((r.sc[1] >> sb) & 0xffu));
        const float ds0 = d * s0, ds1 = d * s1;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float t0 = __builtin_fmaf(-32.0f, ux.s[b][0], dot0[b]);
            const float t1 = __builtin_fmaf(-32.0f, ux.s[b][1], dot1[b]);
            acc[b] += __builtin_fmaf(ds0, t0, ds1 * t1);
        }
    } else if constexpr (T == T_Q8_0) {
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            const uint32_t biased = r.q[t] ^ 0x80808080u;  // int8 q -> q + 128
#pragma unroll
            for (int b = 0; b < B; ++b) dot0[b] = dot4(biased, &ux.v[b][4 * t], dot0[b]);
        }
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (int b = 0; b < B; ++b) acc[b] += d * __builtin_fmaf(-128.0f, ux.s[b][0], dot0[b]);
    } else if constexpr (T == T_Q5_0 || T == T_Q5_1) {
        // 5-bit q = nibble | qh bit << 4 (qh bit j for element j of the block):
        // Q5_0 w = (q - 16) * d (decode_q5_0, src/quantized_linear.cpp:64-77),
        // Q5_1 w = q * d + m (decode_q5_1, :79-93)
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            const uint32_t bl = (r.qh[0] >> (p.k0 + 4u * t)) & 0xfu;
            const uint32_t bh = (r.qh[0] >> (16u + p.k0 + 4u * t)) & 0xfu;
            const uint32_t lo = (r.q[t] & 0x0f0f0f0fu) | spread4(bl);
            const uint32_t hi = ((r.q[t] >> 4) & 0x0f0f0f0fu) | spread4(bh);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                dot0[b] = dot4(lo, &ux.v[b][4 * t], dot0[b]);
                dot1[b] = dot4(hi, &ux.v[b][UB + 4 * t], dot1[b]);
            }
        }
        if constexpr (T == T_Q5_0) {
            const float d = half_bits_to_float(r.d);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float t0 = __builtin_fmaf(-16.0f, ux.s[b][0], dot0[b]);
                const float t1 = __builtin_fmaf(-16.0f, ux.s[b][1], dot1[b]);
                acc[b] += d * (t0 + t1);
            }
        } else {
            const float d = half_bits_to_float(r.h[0] & 0xffffu);
            const float m = half_bits_to_float(r.h[0] >> 16);
#pragma unroll
            for (int b = 0; b < B; ++b)
                acc[b] += __builtin_fmaf(d, dot0[b] + dot1[b], m * (ux.s[b][0] + ux.s[b][1]));
        }
    } else if constexpr (T == T_Q2_K || T == T_Q3_K) {
        // run s: the 2-bit fields at bits 2s of the unit's quant bytes, scale
        // group g = 8h + 2s + t.  Q2_K w = dl * q - ml with dl = d * (sc & 15),
        // ml = dmin * (sc >> 4) (decode_q2_k, src/quantized_linear.cpp:95-121);
        // Q3_K w = d * (scale - 32) * (q + 4 * hbit - 4) with the hmask bit
        // 4h + s (decode_q3_k, :123-164).
        const uint32_t h = p.k0 / 32u, tt = (p.k0 % 32u) / 16u;
        float dots[4][B];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
            for (int b = 0; b < B; ++b) dots[s4][b] = 0.0f;
#pragma unroll
        for (int t = 0; t < NW; ++t) {
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                uint32_t v = (r.q[t] >> (2 * s4)) & 0x03030303u;
                if constexpr (T == T_Q3_K) v |= ((r.qh[t] >> (4u * h + s4)) & 0x01010101u) << 2;
#pragma unroll
                for (int b = 0; b < B; ++b) dots[s4][b] = dot4(v, &ux.v[b][s4 * UB + 4 * t], dots[s4][b]);
            }
        }
        if constexpr (T == T_Q2_K) {
            const float d = half_bits_to_float(r.h[0] & 0xffffu);
            const float dmin = half_bits_to_float(r.h[0] >> 16);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const uint32_t sb = 2u * s4 + tt;  // byte of the 8 loaded (group g = 8h + sb)
                const uint32_t scb = (r.sc[sb / 4u] >> (8u * (sb % 4u))) & 0xffu;
                const float dl = d * static_cast<float>(scb & 15u);
                const float ml = dmin * static_cast<float>(scb >> 4);
#pragma unroll
                for (int b = 0; b < B; ++b) acc[b] += __builtin_fmaf(dl, dots[s4][b], -ml * ux.s[b][s4]);
            }
        } else {
            const float d = half_bits_to_float(r.d);
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const uint32_t g = 8u * h + 2u * s4 + tt;
                const float ds = d * static_cast<float>(static_cast<int>(q3k_scale(r.sc, g)) - 32);
#pragma unroll
                for (int b = 0; b < B; ++b)
                    acc[b] += ds * __builtin_fmaf(-4.0f, ux.s[b][s4], dots[s4][b]);
            }
        }
    } else if constexpr (T == T_Q4_1) {  // w = d * q + m (decode_q4_1, src/quantized_linear.cpp:53-62)
#pragma unroll
        for (int t = 0; t < NW; ++t) {
            const uint32_t lo = r.q[t] & 0x0f0f0f0fu;
            const uint32_t hi = (r.q[t] >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                dot0[b] = dot4(lo, &ux.v[b][4 * t], dot0[b]);
                dot1[b] = dot4(hi, &ux.v[b][UB + 4 * t], dot1[b]);
            }
        }
        const float d = half_bits_to_float(r.h[0] & 0xffffu);
        const float m = half_bits_to_float(r.h[0] >> 16);
#pragma unroll
        for (int b = 0; b < B; ++b)
            acc[b] += __builtin_fmaf(d, dot0[b] + dot1[b], m * (ux.s[b][0] + ux.s[b][1]));
    } else {  // Q4_0
        nibble_dots<UB, B>(r.q, ux, dot0, dot1);
        const float d = half_bits_to_float(r.d);
        constexpr float f0 = B == 1 ? 0x1p24f : 1.0f, f1 = B == 1 ? 0x1p20f : 1.0f;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float t0 = __builtin_fmaf(-8.0f, ux.s[b][0], dot0[b] * f0);
            const float t1 = __builtin_fmaf(-8.0f, ux.s[b][1], dot1[b] * f1);
            acc[b] += d * (t0 + t1);
        }
    }
}

// ---------------------------------------------------------------------------
// Cross-lane sums with DPP (row_shr / quad_perm / mirrors / row_bcast): VALU
// latency instead of the LDS round trip of a bpermute shuffle.

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 CTRL, ROW_MASK, BANK_MASK,
                                                                 false));
}

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ double dpp(double v) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __builtin_amdgcn_update_dpp(0, p.x, CTRL, ROW_MASK, BANK_MASK, false);
    r.y = __builtin_amdgcn_update_dpp(0, p.y, CTRL, ROW_MASK, BANK_MASK, false);
    return __builtin_bit_cast(double, r);
}

// As dpp(), but lanes outside ROW_MASK keep their own value (for max).
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ double dpp_keep(double v) {
    const int2 p = __builtin_bit_cast(int2, v);
    int2 r;
    r.x = __builtin_amdgcn_update_dpp(p.x, p.x, CTRL, ROW_MASK, BANK_MASK, false);
    r.y = __builtin_amdgcn_update_dpp(p.y, p.y, CTRL, ROW_MASK, BANK_MASK, false);
    return __builtin_bit_cast(double, r);
}

// Maximum over aligned groups of G lanes, exact in the group's last lane.
template <int G>
__device__ __forceinline__ double group_max(double v) {
    if constexpr (G >= 2) v = fmax(v, dpp_keep<0xb1>(v));
    if constexpr (G >= 4) v = fmax(v, dpp_keep<0x4e>(v));
    if constexpr (G >= 8) v = fmax(v, dpp_keep<0x141>(v));
    if constexpr (G >= 16) v = fmax(v, dpp_keep<0x140>(v));
    if constexpr (G >= 32) v = fmax(v, dpp_keep<0x142, 0xa>(v));
    if constexpr (G >= 64) v = fmax(v, dpp_keep<0x143, 0xc>(v));
    return v;
}

// Sum over aligned groups of G lanes (G a power of two <= 64).  The group
// total is exact in the group's last lane (all lanes when G <= 16).
template <int G, typename V>
__device__ __forceinline__ V group_sum(V v) {
    if constexpr (G >= 2) v += dpp<0xb1>(v);         // quad_perm [1,0,3,2]
    if constexpr (G >= 4) v += dpp<0x4e>(v);         // quad_perm [2,3,0,1]
    if constexpr (G >= 8) v += dpp<0x141>(v);        // row_half_mirror
    if constexpr (G >= 16) v += dpp<0x140>(v);       // row_mirror
    if constexpr (G >= 32) v += dpp<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    if constexpr (G >= 64) v += dpp<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

template <typename V>
__device__ __forceinline__ V group_sum_dyn(V v, uint32_t g) {
    switch (g) {
        case 1: return v;
        case 2: return group_sum<2>(v);
        case 4: return group_sum<4>(v);
        case 8: return group_sum<8>(v);
        case 16: return group_sum<16>(v);
        case 32: return group_sum<32>(v);
        default: return group_sum<64>(v);
    }
}

// Inclusive prefix sum over the 64 lanes of a wave.
template <typename V>
__device__ __forceinline__ V wave_inclusive_scan(V v) {
    v += dpp<0x111>(v);        // row_shr:1
    v += dpp<0x112>(v);        // row_shr:2
    v += dpp<0x114>(v);        // row_shr:4
    v += dpp<0x118>(v);        // row_shr:8
    v += dpp<0x142, 0xa>(v);   // row_bcast:15
    v += dpp<0x143, 0xc>(v);   // row_bcast:31
    return v;
}

template <typename V>
__device__ __forceinline__ V lane63(V v) {
    if constexpr (sizeof(V) == 4) {
        return __builtin_bit_cast(V, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    } else {
        const int2 p = __builtin_bit_cast(int2, v);
        int2 r;
        r.x = __builtin_amdgcn_readlane(p.x, 63);
        r.y = __builtin_amdgcn_readlane(p.y, 63);
        return __builtin_bit_cast(V, r);
    }
}

// The upper halves of two floats as one dword of bf16 (exact for small
// integers).
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Four unsigned byte fields (each < 256) to two dwords of bf16: one
// v_cvt_f32_ubyteN per field (no separate byte extraction), one v_perm per pair.
__device__ __forceinline__ void bf16_bytes(uint32_t w, uint32_t& lo, uint32_t& hi) {
    lo = bf16_pair(ub<0>(w), ub<1>(w));
    hi = bf16_pair(ub<2>(w), ub<3>(w));
}

// bf16 bits of a finite x, rounded to nearest even.
__device__ __forceinline__ uint32_t bf16_rne_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// The bytes f0..f3 of w as the bf16 pairs of 128 + f (bits 0x4300 | f: the
// exponent of 128 leaves f in the low mantissa bits), one v_perm per pair:
// the weight operand of the MFMA kernels, whose group bias absorbs the
// -128 * ds (a bf16 of 128 + f is exact for f < 128).
__device__ __forceinline__ void bf16_bytes_b128(uint32_t w, uint32_t& lo, uint32_t& hi) {
    lo = __builtin_amdgcn_perm(0x43434343u, w, 0x04010400u);  // bytes f0, 0x43, f1, 0x43
    hi = __builtin_amdgcn_perm(0x43434343u, w, 0x04030402u);  // bytes f2, 0x43, f3, 0x43
}

}  // namespace pk
