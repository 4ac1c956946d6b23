// matvec_mfma.hip -- batched matvecs (5 to 8 vectors, and 4 where the grid
// is small) on bf16 MFMA, for Q4_K, Q5_K, Q6_K, Q8_0 and Q4_0.
//
// The batched case of tensor_linear (src/tensor_linear.cpp:232-263 of the
// reference, per-row linear_k / linear_quantized of
// src/quantized_linear.cpp:360-423): y[b][r] = W[r] . x[b].  The register
// kernels of matvec.hip hold every vector's activations in each lane and
// reduce every (row, vector) dot across the 64 lanes, which costs about 36
// VALU operations per weight at 8 vectors.  Here the vectors are the A
// operand and the decoded weights the B operand of v_mfma_f32_16x16x32_bf16,
// so the dots and their reductions run on the matrix cores:
//
//  * A wave owns 16·NT rows (NT tiles of 16, lane n = lane % 16 of each tile)
//    and KB consecutive 256-value ranges of K; the waves of a workgroup own
//    the same rows and consecutive K ranges, and their partial results are
//    added through LDS in wave order (deterministic).  Where that grid has
//    at most 128 row groups, k_matvec_mfma_ks (below) takes the matrix
//    instead: 64 rows and a K slice per workgroup, partial sums per slice
//    added in slice order by a second launch.
//  * A scale group of 32 values is one MFMA K step, lane kq = lane / 16
//    holding values 8kq .. 8kq+7 of it (Q6_K's two 16-value groups per step:
//    two MFMAs, each with the other group's lanes zeroed).  Per 256 values
//    lane (n, kq) loads (Q4_K, Q5_K) the block header and bytes 8kq .. 8kq+7
//    of each 32-byte nibble chunk (chunk c's low nibbles are group 2c, its
//    high nibbles group 2c+1; Q5_K also bytes 8kq .. 8kq+7 of qh, bit g for
//    group g), or (Q8_0, Q4_0) the 8 bytes of each of 8 blocks that hold its
//    values and the 8 blocks' scales in one 16-byte load.
//  * Weights enter the MFMA as bf16 of an unsigned field f (128 + q for the
//    nibble formats, one v_perm per pair; q + 128 for Q8_0), all exact; per
//    group the CPU's weight is ds·f + cb, so acc += ds · (x . f) + cb · sum(x).
//  * x enters as three bf16 planes (hi, mid, lo: x = hi + mid + lo exactly),
//    split by each lane from FP32 for its (vector m = lane % 16, kq) slot;
//    rows m >= batch repeat vector 0 and their outputs are not stored.  The
//    group sums go in through one v_mfma_f32_16x16x4f32 per group whose K
//    runs over the four kq partial sums of 8 values, against cb.
//
// Results differ from the CPU's serial FP32 sum only in rounding order, like
// the register kernels' (within 1e-4 normwise).
#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

typedef __bf16 mbf16x8 __attribute__((ext_vector_type(8)));
typedef float mf32x4 __attribute__((ext_vector_type(4)));

// One lane's share of 256 values of a row.
template <int T> struct MmPart;
template <> struct MmPart<T_Q4_K> { uint32_t h[4], q[8]; };           // q[2c..2c+1]: chunk c
template <> struct MmPart<T_Q5_K> { uint32_t h[4], q[8], qh[2]; };
template <> struct MmPart<T_Q8_0> { uint32_t q[16], d[4]; };          // q[2i..2i+1]: block i
template <> struct MmPart<T_Q4_0> { uint32_t q[16], d[4]; };
template <> struct MmPart<T_Q6_K> { uint32_t ql[8], qh[4], sc[4], d; };  // ql[2r..2r+1]: run r

__device__ __forceinline__ void ld2(const uint8_t* p, uint32_t* w) {
    const uint2 v = *reinterpret_cast<const uint2*>(__builtin_assume_aligned(p, 8));
    w[0] = v.x;
    w[1] = v.y;
}

__device__ __forceinline__ void ld4_16(const uint8_t* p, uint32_t* w) {
    const uint4 v = *reinterpret_cast<const uint4*>(__builtin_assume_aligned(p, 16));
    w[0] = v.x;
    w[1] = v.y;
    w[2] = v.z;
    w[3] = v.w;
}

// Values 256·sb .. 256·sb + 255 of the row (K-quants: block sb; Q8_0/Q4_0:
// blocks 8sb .. 8sb+7, whose scales are 16 consecutive bytes of the d plane).
template <int T>
__device__ __forceinline__ void mm_load(const QRow& r, uint32_t sb, uint32_t kq, MmPart<T>& p) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = block_ptr<Fmt<T>::BB>(r, sb);
        ld_words<4>(blk, p.h);
        const uint8_t* qs = blk + (T == T_Q4_K ? 16u : 48u) + 8u * kq;
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) ld2(qs + 32u * c, &p.q[2u * c]);
        if constexpr (T == T_Q5_K) ld2(blk + 16u + 8u * kq, p.qh);
    } else if constexpr (T == T_Q6_K) {
        // run r = 2h + (s & 1) of ql (64h + 32(s & 1)) and qh bytes 32h.. for
        // the values 128h + 32s + 8kq .. (decode_q6_k's layout)
        using L = Planar<T_Q6_K>;
        const uint8_t* ql = field_ptr<L::QL, 128>(r, sb) + 8u * kq;
        const uint8_t* qh = field_ptr<L::QH, 64>(r, sb) + 8u * kq;
#pragma unroll
        for (uint32_t run = 0; run < 4; ++run) ld2(ql + 32u * run, &p.ql[2u * run]);
        ld2(qh, &p.qh[0]);
        ld2(qh + 32u, &p.qh[2]);
        ld4_16(field_ptr<L::SC, 16>(r, sb), p.sc);
        p.d = ld_u16(field_ptr<L::D, 2>(r, sb));
    } else if constexpr (T == T_Q8_0) {
        using L = Planar<T_Q8_0>;
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) ld2(field_ptr<L::QS, 32>(r, 8u * sb + i) + 8u * kq, &p.q[2u * i]);
        ld4_16(field_ptr<L::D, 2>(r, 8u * sb), p.d);
    } else {  // Q4_0: values 8kq.. are the low (kq < 2) or high nibbles of bytes 8(kq & 1)..
        using L = Planar<T_Q4_0>;
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i)
            ld2(field_ptr<L::QS, 16>(r, 8u * sb + i) + 8u * (kq & 1u), &p.q[2u * i]);
        ld4_16(field_ptr<L::D, 2>(r, 8u * sb), p.d);
    }
}

// x[m][k0 + 8kq .. k0 + 8kq + 7] as loaded, and as three exact bf16 planes
// (hi = bf16(x), mid = bf16(x - hi), lo = x - hi - mid, which has at most
// 8 significant bits left) with their sum.
struct XRaw {
    float4 a, b;
};

struct XFrag {
    mbf16x8 hi, mid, lo;
    float part;
};

typedef __bf16 mbf16x2 __attribute__((ext_vector_type(2)));
typedef float mf32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void x_load(const float* x, uint32_t in, uint32_t m, uint32_t k0,
                                       uint32_t kq, XRaw& r) {
    const float* p = x + static_cast<uint64_t>(m) * in + k0 + 8u * kq;
    r.a = *reinterpret_cast<const float4*>(p);
    r.b = *reinterpret_cast<const float4*>(p + 4);
}

__device__ __forceinline__ void x_split(const XRaw& r, XFrag& f) {
    const float v[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    uint32_t h[4], md[4], lo[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const mf32x2 x2 = {v[e], v[e + 1]};
        const mbf16x2 h2 = __builtin_convertvector(x2, mbf16x2);  // v_cvt_pk_bf16_f32, RNE
        const mf32x2 r1 = x2 - __builtin_convertvector(h2, mf32x2);
        const mbf16x2 m2 = __builtin_convertvector(r1, mbf16x2);
        const mf32x2 r2 = r1 - __builtin_convertvector(m2, mf32x2);
        const mbf16x2 l2 = __builtin_convertvector(r2, mbf16x2);  // exact
        h[e / 2] = __builtin_bit_cast(uint32_t, h2);
        md[e / 2] = __builtin_bit_cast(uint32_t, m2);
        lo[e / 2] = __builtin_bit_cast(uint32_t, l2);
    }
    f.hi = __builtin_bit_cast(mbf16x8, make_uint4(h[0], h[1], h[2], h[3]));
    f.mid = __builtin_bit_cast(mbf16x8, make_uint4(md[0], md[1], md[2], md[3]));
    f.lo = __builtin_bit_cast(mbf16x8, make_uint4(lo[0], lo[1], lo[2], lo[3]));
    f.part = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

// Group g (0..7) of a part: the lane's B fragment, ds and cb.
template <int T>
__device__ __forceinline__ void mm_group(const MmPart<T>& p, uint32_t g, uint32_t kq, mbf16x8& b,
                                         float& ds, float& cb) {
    uint32_t w[4];
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint32_t c = g / 2u, sh = 4u * (g & 1u);
#pragma unroll
        for (uint32_t i = 0; i < 2; ++i) {
            uint32_t q = (p.q[2u * c + i] >> sh) & 0x0f0f0f0fu;
            if constexpr (T == T_Q5_K) q |= ((p.qh[i] >> g) & 0x01010101u) << 4;
            bf16_bytes_b128(q, w[2u * i], w[2u * i + 1u]);
        }
        const float d = half_bits_to_float(p.h[0] & 0xffffu);
        const float dmin = half_bits_to_float(p.h[0] >> 16);
        float sc, mn;
        kq_scale_min(p.h, g, sc, mn);
        ds = __fmul_rn(d, sc);
        cb = -__fmaf_rn(128.0f, ds, __fmul_rn(dmin, mn));  // ds·q - dmin·m
    } else {
        ds = half_bits_to_float((p.d[g / 2u] >> (16u * (g & 1u))) & 0xffffu);
        if constexpr (T == T_Q8_0) {
#pragma unroll
            for (uint32_t i = 0; i < 2; ++i) bf16_bytes(p.q[2u * g + i] ^ 0x80808080u, w[2u * i], w[2u * i + 1u]);
            cb = __fmul_rn(-128.0f, ds);  // d·q = d·(q + 128) - 128·d
        } else {
            const uint32_t sh = 4u * (kq >> 1);
#pragma unroll
            for (uint32_t i = 0; i < 2; ++i)
                bf16_bytes_b128((p.q[2u * g + i] >> sh) & 0x0f0f0f0fu, w[2u * i], w[2u * i + 1u]);
            cb = __fmul_rn(-136.0f, ds);  // d·(q - 8) = d·(128 + q) - 136·d
        }
    }
    b = __builtin_bit_cast(mbf16x8, make_uint4(w[0], w[1], w[2], w[3]));
}

// Q6_K group g (0..7): 32 values of two 16-value scale groups, lanes kq < 2
// holding the first.  The lane's fragment f (128 + the 6-bit field) goes to
// two MFMAs, each with the other group's lanes zeroed; w = ds·(f - 32) =
// ds·(128 + f) - 160·ds, and cb is that of the lane's own group.
__device__ __forceinline__ void q6k_group(const MmPart<T_Q6_K>& p, uint32_t g, uint32_t kq,
                                          mbf16x8& b0, mbf16x8& b1, float& ds0, float& ds1,
                                          float& cb) {
    const uint32_t h = g >> 2, s = g & 3u, run = 2u * h + (s & 1u);
    uint32_t w[4];
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
        const uint32_t nib = ((s < 2u ? p.ql[2u * run + i] : p.ql[2u * run + i] >> 4)) & 0x0f0f0f0fu;
        const uint32_t hb = ((p.qh[2u * h + i] >> (2u * s)) & 0x03030303u) << 4;
        bf16_bytes_b128(nib | hb, w[2u * i], w[2u * i + 1u]);
    }
    const uint4 z = make_uint4(0u, 0u, 0u, 0u), v = make_uint4(w[0], w[1], w[2], w[3]);
    b0 = __builtin_bit_cast(mbf16x8, kq < 2u ? v : z);
    b1 = __builtin_bit_cast(mbf16x8, kq < 2u ? z : v);
    const float d = half_bits_to_float(p.d);
    const uint32_t i0 = 8u * h + 2u * s;  // scale index of the first group
    const uint32_t s2 = (p.sc[i0 >> 2] >> (8u * (i0 & 3u))) & 0xffffu;
    ds0 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s2 & 0xffu)));
    ds1 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s2 >> 8)));
    cb = __fmul_rn(-160.0f, kq < 2u ? ds0 : ds1);
}

template <int T, int NT, int KB>
__global__ __launch_bounds__(1024) void k_matvec_mfma(const uint8_t* W, uint32_t nb,
                                                     const float* x, float* __restrict__ y,
                                                     uint32_t rows, uint32_t batch) {
    // W and x are not __restrict__: loads the compiler may not take for
    // invariant stay in program order, so every weight load and the first x
    // loads are issued before the first wait (the memory counter is in order)
    // [wave][tile][lane][4]: the waves' partial tiles
    extern __shared__ mf32x4 red[];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t waves = blockDim.x >> 6;
    const uint32_t n = lane & 15u, kq = lane >> 4;
    const uint32_t r0 = blockIdx.x * 16u * NT;
    const uint32_t kbase = wave * KB;
    const uint32_t in = nb * 256u;

    // nb: 256-value ranges per row
    constexpr uint32_t kPer = 256u / Fmt<T>::BE;  // GGUF blocks per 256 values
    const uint64_t nblk = static_cast<uint64_t>(rows) * nb * kPer;
    MmPart<T> part[NT][KB];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t row = r0 + 16u * t + n;
        const QRow qr{W, nblk, static_cast<uint64_t>(row < rows ? row : rows - 1u) * nb * kPer};
#pragma unroll
        for (int j = 0; j < KB; ++j) mm_load<T>(qr, kbase + j, kq, part[t][j]);
    }

    // the x of the wave's first XD groups, then XD groups ahead of their use
    constexpr int NG = KB * 8, XD = NG < 4 ? NG : 4;
    // A operand row m = n of this lane; rows m >= batch repeat vector 0 and
    // only feed output rows that are not stored
    const uint32_t m = n < batch ? n : 0u, kw = kbase * 256u;
    XRaw xr[XD];
#pragma unroll
    for (int i = 0; i < XD; ++i) x_load(x, in, m, kw + 32u * i, kq, xr[i]);
    __builtin_amdgcn_sched_barrier(0);

    mf32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = mf32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        XFrag xf;
        x_split(xr[gi % XD], xf);
        if (gi + XD < NG) x_load(x, in, m, kw + 32u * (gi + XD), kq, xr[gi % XD]);
        const int j = gi / 8, g = gi % 8;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const mf32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
            float cb;
            if constexpr (T == T_Q6_K) {
                mbf16x8 b0, b1;
                float ds0, ds1;
                q6k_group(part[t][j], g, kq, b0, b1, ds0, ds1, cb);
                mf32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.lo, b0, zero, 0, 0, 0);
                mf32x4 Q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.lo, b1, zero, 0, 0, 0);
                P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.mid, b0, P, 0, 0, 0);
                Q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.mid, b1, Q, 0, 0, 0);
                P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.hi, b0, P, 0, 0, 0);
                Q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.hi, b1, Q, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[t][i] = __builtin_fmaf(ds0, P[i], acc[t][i]);
                    acc[t][i] = __builtin_fmaf(ds1, Q[i], acc[t][i]);
                }
            } else {
                mbf16x8 b;
                float ds;
                mm_group<T>(part[t][j], g, kq, b, ds, cb);
                mf32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.lo, b, zero, 0, 0, 0);
                P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.mid, b, P, 0, 0, 0);
                P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.hi, b, P, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_fmaf(ds, P[i], acc[t][i]);
            }
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xf.part, cb, acc[t], 0, 0, 0);
        }
    }

    // lane holds vectors 4kq .. 4kq+3 of row n of each tile
#pragma unroll
    for (int t = 0; t < NT; ++t) red[(wave * NT + t) * 64u + lane] = acc[t];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            mf32x4 s = red[t * 64u + lane];
            for (uint32_t w = 1; w < waves; ++w) s += red[(w * NT + t) * 64u + lane];
            const uint32_t row = r0 + 16u * t + n;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = 4u * kq + i;
                if (m < batch && row < rows) y[static_cast<uint64_t>(m) * rows + row] = s[i];
            }
        }
    }
}

// K-sliced layout for small row counts.  In the kernel above every 16-row
// tile reads and splits all of x (at 2048x6144 and 8 vectors, 25 MB of x
// reads for 7 MB of weights, and the split is about half the VALU work).
// Here a workgroup owns 64 rows (four tiles, one per wave column) and KR
// consecutive 256-value ranges of K (one per wave row): it splits only its
// K slice of x, once, into LDS (the 32 distinct A fragments per 32-value
// group: vectors 0..7 x kq; lanes of rows m >= 8 read vector m - 8's, their
// outputs are never stored), every wave reads its fragments from there, the
// waves of a tile add their K ranges through LDS in range order, and the
// slice's sums go to partial[slice][b][row].  k_mm_reduce adds the slices in
// slice order (deterministic).  One slice (nb <= 4) writes y directly.
constexpr uint32_t kKsTiles = 4;  // 16-row tiles per workgroup

template <int T, int KR>
__global__ __launch_bounds__(1024) void k_matvec_mfma_ks(const uint8_t* W, uint32_t nb,
                                                        const float* x, float* out, uint32_t rows,
                                                        uint32_t batch) {
    constexpr uint32_t G = 8u * KR;  // 32-value groups of the slice
    // [hi | mid | lo][G][32 slots] fragments, then the slots' 8-value sums
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    mbf16x8* ah = reinterpret_cast<mbf16x8*>(smem);
    mbf16x8* am = ah + G * 32u;
    mbf16x8* al = am + G * 32u;
    float* ap = reinterpret_cast<float*>(al + G * 32u);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tile = wave % kKsTiles, kr = wave / kKsTiles;
    const uint32_t n = lane & 15u, kq = lane >> 4;
    const uint32_t row = (blockIdx.x * kKsTiles + tile) * 16u + n;
    constexpr uint32_t kPer = 256u / Fmt<T>::BE;  // GGUF blocks per 256 values
    const uint64_t nblk = static_cast<uint64_t>(rows) * nb * kPer;
    // the weight loads first (HBM), then the slice's x (L2)
    MmPart<T> part;
    const QRow qr{W, nblk, static_cast<uint64_t>(row < rows ? row : rows - 1u) * nb * kPer};
    mm_load<T>(qr, blockIdx.y * KR + kr, kq, part);
    const uint32_t in = nb * 256u, k0 = blockIdx.y * KR * 256u;
    for (uint32_t i = tid; i < G * 32u; i += blockDim.x) {  // G * 32 is a multiple of blockDim
        const uint32_t gi = i / 32u, slot = i % 32u, m = slot & 7u;
        XRaw xr;
        x_load(x, in, m < batch ? m : 0u, k0 + 32u * gi, slot >> 3, xr);
        XFrag f;
        x_split(xr, f);
        ah[i] = f.hi;
        am[i] = f.mid;
        al[i] = f.lo;
        ap[i] = f.part;
    }
    __syncthreads();
    mf32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t slot = (n & 7u) + 8u * kq;
#pragma unroll
    for (uint32_t g = 0; g < 8u; ++g) {
        const uint32_t i = (kr * 8u + g) * 32u + slot;
        const mbf16x8 xh = ah[i], xm = am[i], xl = al[i];
        const float xp = ap[i];
        const mf32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
        float cb;
        if constexpr (T == T_Q6_K) {
            mbf16x8 b0, b1;
            float ds0, ds1;
            q6k_group(part, g, kq, b0, b1, ds0, ds1, cb);
            mf32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, b0, zero, 0, 0, 0);
            mf32x4 Q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, b1, zero, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, b0, P, 0, 0, 0);
            Q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, b1, Q, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, b0, P, 0, 0, 0);
            Q = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, b1, Q, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[j] = __builtin_fmaf(ds0, P[j], acc[j]);
                acc[j] = __builtin_fmaf(ds1, Q[j], acc[j]);
            }
        } else {
            mbf16x8 b;
            float ds;
            mm_group<T>(part, g, kq, b, ds, cb);
            mf32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, b, zero, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, b, P, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, b, P, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __builtin_fmaf(ds, P[j], acc[j]);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xp, cb, acc, 0, 0, 0);
    }
    // the tile's K ranges in range order (the fragments are dead: reuse LDS)
    __syncthreads();
    mf32x4* red = reinterpret_cast<mf32x4*>(smem);  // [kr][tile][lane]
    red[(kr * kKsTiles + tile) * 64u + lane] = acc;
    __syncthreads();
    if (kr == 0u) {
        mf32x4 sum = red[tile * 64u + lane];
        for (uint32_t k = 1; k < KR; ++k) sum += red[(k * kKsTiles + tile) * 64u + lane];
        // lane holds vectors 4kq .. 4kq+3 of its row
        float* o = out + static_cast<uint64_t>(blockIdx.y) * batch * rows;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t m = 4u * kq + j;
            if (m < batch && row < rows) o[static_cast<uint64_t>(m) * rows + row] = sum[j];
        }
    }
}

// y[i] = partial[0][i] + partial[1][i] + ... in slice order.
__global__ __launch_bounds__(256) void k_mm_reduce(const float* __restrict__ partial,
                                                   float* __restrict__ y, uint32_t n,
                                                   uint32_t slices) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    float v = partial[i];
    for (uint32_t s = 1; s < slices; ++s) v += partial[static_cast<uint64_t>(s) * n + i];
    y[i] = v;
}

// K ranges per workgroup (KR) and slices for the K-sliced kernel: the
// largest KR <= 4 dividing nb that still gives at least 256 workgroups, else
// the smallest divisor; 0 where the kernel does not apply.
uint32_t ks_ranges(uint32_t nb, uint32_t rows) {
    const uint32_t groups = (rows + 16u * kKsTiles - 1u) / (16u * kKsTiles);
    uint32_t best = 0;
    for (uint32_t kr = 1; kr <= 4u; ++kr) {
        if (nb % kr) continue;
        if (best == 0 || groups * (nb / kr) >= 256u) best = kr;
    }
    return best;
}

template <int T, int KR>
hipError_t launch_ks(const uint8_t* W, uint32_t nb, uint32_t rows, const float* x, float* y,
                     uint32_t batch, float* partial, hipStream_t s) {
    const uint32_t slices = nb / KR;
    const uint32_t groups = (rows + 16u * kKsTiles - 1u) / (16u * kKsTiles);
    float* out = slices > 1u ? partial : y;
    if (!out) return hipErrorInvalidValue;
    constexpr size_t kFrag = 8u * KR * 32u * (3u * sizeof(mbf16x8) + sizeof(float));
    constexpr size_t kRed = KR * kKsTiles * 64u * sizeof(mf32x4);
    const size_t lds = kFrag > kRed ? kFrag : kRed;
    hipLaunchKernelGGL((k_matvec_mfma_ks<T, KR>), dim3(groups, slices), dim3(64u * kKsTiles * KR),
                       lds, s, W, nb, x, out, rows, batch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || slices == 1u) return e;
    const uint32_t n = batch * rows;
    hipLaunchKernelGGL(k_mm_reduce, dim3((n + 255u) / 256u), dim3(256), 0, s, partial, y, n, slices);
    return hipGetLastError();
}

template <int T>
hipError_t launch_ks_t(const uint8_t* W, uint32_t nb, uint32_t rows, const float* x, float* y,
                       uint32_t batch, float* partial, hipStream_t s) {
    switch (ks_ranges(nb, rows)) {
        case 1: return launch_ks<T, 1>(W, nb, rows, x, y, batch, partial, s);
        case 2: return launch_ks<T, 2>(W, nb, rows, x, y, batch, partial, s);
        case 3: return launch_ks<T, 3>(W, nb, rows, x, y, batch, partial, s);
        case 4: return launch_ks<T, 4>(W, nb, rows, x, y, batch, partial, s);
        default: return hipErrorInvalidValue;
    }
}

template <int T, int NT, int KB>
hipError_t launch_nt_kb(const uint8_t* W, uint32_t nb, uint32_t rows, const float* x, float* y,
                        uint32_t batch, hipStream_t s) {
    const uint32_t waves = nb / KB;
    const uint32_t blocks = (rows + 16u * NT - 1u) / (16u * NT);
    const size_t lds = static_cast<size_t>(waves) * NT * 64u * sizeof(mf32x4);
    hipLaunchKernelGGL((k_matvec_mfma<T, NT, KB>), dim3(blocks), dim3(64u * waves), lds, s, W, nb,
                       x, y, rows, batch);
    return hipGetLastError();
}

template <int T>
hipError_t launch_t(uint32_t kb, const uint8_t* W, uint32_t nb, uint32_t rows, const float* x,
                    float* y, uint32_t batch, hipStream_t s) {
    switch (kb) {
        case 1: return launch_nt_kb<T, 2, 1>(W, nb, rows, x, y, batch, s);
        case 2: return launch_nt_kb<T, 1, 2>(W, nb, rows, x, y, batch, s);
        case 3: return launch_nt_kb<T, 1, 3>(W, nb, rows, x, y, batch, s);
        case 4:  // (mfma_kb gives 4 to Q4_K/Q5_K only)
            if constexpr (T == T_Q4_K || T == T_Q5_K) return launch_nt_kb<T, 1, 4>(W, nb, rows, x, y, batch, s);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// 256-value ranges of K per wave: one (two row tiles per wave) up to 8 per
// row, else the fewest (2..4, Q8_0/Q4_0/Q6_K 2..3) that leave at most 16
// waves (one tile per wave); 0 where the kernel does not apply.
uint32_t mfma_kb(uint32_t type, uint32_t in) {
    if (type != T_Q4_K && type != T_Q5_K && type != T_Q6_K && type != T_Q8_0 && type != T_Q4_0)
        return 0;
    if (in == 0 || in % 256u) return 0;
    const uint32_t nb = in / 256u;
    if (nb <= 8u) return 1;
    // four ranges of Q6_K, or of 8 Q8_0/Q4_0 blocks, would spill
    const uint32_t max_kb = type == T_Q4_K || type == T_Q5_K ? 4u : 3u;
    for (uint32_t kb = 2; kb <= max_kb; ++kb)
        if (nb % kb == 0 && nb / kb <= 16u) return kb;
    return 0;
}

uint32_t matvec_mfma_blocks_per_wave(uint32_t type, uint32_t in, uint32_t batch) {
    return batch >= 5u && batch <= 8u ? mfma_kb(type, in) : 0u;
}

// Grids of at most 128 row groups of the one-pass kernel (half the CUs:
// 2048-row matrices) take the K-sliced kernel instead; 4 vectors go to MFMA
// only there (the staged register kernel leads elsewhere: 6.7 against 11.1 us
// at 6144x2048).
bool ks_takes(uint32_t type, uint32_t in, uint32_t rows) {
    const uint32_t kb = mfma_kb(type, in);
    if (kb == 0) return false;
    const uint32_t nt = kb == 1u ? 2u : 1u;
    return (rows + 16u * nt - 1u) / (16u * nt) <= 128u && ks_ranges(in / 256u, rows) != 0;
}

bool matvec_mfma_takes(uint32_t type, uint32_t in, uint32_t batch, uint32_t rows) {
    if (batch >= 5u) return matvec_mfma_blocks_per_wave(type, in, batch) != 0;
    return batch == 4u && ks_takes(type, in, rows);
}

size_t matvec_mfma_partial_floats(uint32_t type, uint32_t in, uint32_t batch, uint32_t rows) {
    if (!ks_takes(type, in, rows)) return 0;
    const uint32_t nb = in / 256u, slices = nb / ks_ranges(nb, rows);
    return slices > 1u ? static_cast<size_t>(slices) * batch * rows : 0u;
}

hipError_t launch_matvec_mfma(uint32_t type, const uint8_t* W, uint32_t rows, uint32_t in,
                              const float* x, float* y, uint32_t batch, hipStream_t s,
                              float* partial) {
    const uint32_t kb = mfma_kb(type, in);
    const uint32_t nb = in / 256u;
    if (ks_takes(type, in, rows)) {
        switch (type) {
            case T_Q4_K: return launch_ks_t<T_Q4_K>(W, nb, rows, x, y, batch, partial, s);
            case T_Q5_K: return launch_ks_t<T_Q5_K>(W, nb, rows, x, y, batch, partial, s);
            case T_Q6_K: return launch_ks_t<T_Q6_K>(W, nb, rows, x, y, batch, partial, s);
            case T_Q8_0: return launch_ks_t<T_Q8_0>(W, nb, rows, x, y, batch, partial, s);
            case T_Q4_0: return launch_ks_t<T_Q4_0>(W, nb, rows, x, y, batch, partial, s);
            default: return hipErrorInvalidValue;
        }
    }
    switch (type) {
        case T_Q4_K: return launch_t<T_Q4_K>(kb, W, nb, rows, x, y, batch, s);
        case T_Q5_K: return launch_t<T_Q5_K>(kb, W, nb, rows, x, y, batch, s);
        case T_Q6_K: return launch_t<T_Q6_K>(kb, W, nb, rows, x, y, batch, s);
        case T_Q8_0: return launch_t<T_Q8_0>(kb, W, nb, rows, x, y, batch, s);
        case T_Q4_0: return launch_t<T_Q4_0>(kb, W, nb, rows, x, y, batch, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace pk
