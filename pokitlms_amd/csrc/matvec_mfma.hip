// matvec_mfma.hip -- batched Q4_K matvecs (5 to 8 vectors) on bf16 MFMA.
//
// The batched case of tensor_linear (src/tensor_linear.cpp:232-263 of the
// reference, per-row linear_k of src/quantized_linear.cpp:360-423): y[b][r] =
// W[r] . x[b].  The register kernels of matvec.hip hold every vector's
// activations in each lane and reduce every (row, vector) dot across the 64
// lanes, which costs about 36 VALU operations per weight at 8 vectors.  Here
// the vectors are the A operand and the decoded weights the B operand of
// v_mfma_f32_16x16x32_bf16, so the dots and their reductions run on the
// matrix cores:
//
//  * A wave owns 16·NT rows (NT tiles of 16, lane n = lane % 16 of each tile)
//    and KB consecutive 256-value blocks of K; the W waves of a workgroup own
//    the same rows and consecutive K ranges, and their partial results are
//    added through LDS in wave order (deterministic).
//  * Lane (n, kq = lane / 16) loads, per block and tile, the 16-byte header
//    and bytes 8kq .. 8kq+7 of each 32-byte nibble chunk: chunk c's low
//    nibbles are scale group 2c, its high nibbles group 2c+1, each group one
//    MFMA K step of 32 values (lane kq holding values 8kq .. 8kq+7).
//  * Weights enter the MFMA as bf16 of 128 + q (one v_perm per pair, exact);
//    per group, acc += ds · (x . (128 + q)) + cb · sum(x) with ds = d·sc and
//    cb = -(128·ds + dmin·m), the CPU's ds·q - dmin·m per weight.
//  * x enters as three bf16 planes (hi, mid, lo: x = hi + mid + lo exactly),
//    split by each lane from FP32 for its (vector m = lane % 16, kq) slot;
//    vectors m >= batch are zero.  The group sums go in through one
//    v_mfma_f32_16x16x4f32 per group whose K runs over the four kq partial
//    sums of 8 values, against cb.
//
// Results differ from the CPU's serial FP32 sum only in rounding order, like
// the register kernels' (within 1e-4 normwise).
#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

typedef __bf16 mbf16x8 __attribute__((ext_vector_type(8)));
typedef float mf32x4 __attribute__((ext_vector_type(4)));

// One lane's share of one 256-value Q4_K block: the header words and the
// 8 bytes it takes of each of the four nibble chunks.
struct Q4kPart {
    uint32_t h[4];
    uint32_t q[8];  // chunk c: q[2c], q[2c + 1]
};

__device__ __forceinline__ void q4k_part_load(const uint8_t* blk, uint32_t kq, Q4kPart& p) {
    ld_words<4>(blk, p.h);
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
        const uint2 v = *reinterpret_cast<const uint2*>(
            __builtin_assume_aligned(blk + 16u + 32u * c + 8u * kq, 8));
        p.q[2u * c] = v.x;
        p.q[2u * c + 1u] = v.y;
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

__device__ __forceinline__ void x_split(const XRaw& r, bool live, XFrag& f) {
    float v[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = live ? v[e] : 0.0f;
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

// Group g (0..7) of a block part: the lane's B fragment, ds and cb.
__device__ __forceinline__ void q4k_group(const Q4kPart& p, uint32_t g, mbf16x8& b, float& ds,
                                          float& cb) {
    const uint32_t c = g / 2u, sh = 4u * (g & 1u);
    uint32_t w[4];
    bf16_bytes_b128((p.q[2u * c] >> sh) & 0x0f0f0f0fu, w[0], w[1]);
    bf16_bytes_b128((p.q[2u * c + 1u] >> sh) & 0x0f0f0f0fu, w[2], w[3]);
    b = __builtin_bit_cast(mbf16x8, make_uint4(w[0], w[1], w[2], w[3]));
    const float d = half_bits_to_float(p.h[0] & 0xffffu);
    const float dmin = half_bits_to_float(p.h[0] >> 16);
    float sc, mn;
    kq_scale_min(p.h, g, sc, mn);
    ds = __fmul_rn(d, sc);
    cb = -__fmaf_rn(128.0f, ds, __fmul_rn(dmin, mn));
}

template <int NT, int KB>
__global__ __launch_bounds__(1024) void k_matvec_mfma_q4k(const uint8_t* W, uint32_t nb,
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
    const uint32_t in = nb * 256u;
    const bool live = n < batch;  // A operand row m = n of this lane

    Q4kPart part[NT][KB];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint32_t row = r0 + 16u * t + n;
        const uint8_t* rp = W + static_cast<uint64_t>(row < rows ? row : rows - 1u) * nb * 144u;
#pragma unroll
        for (int j = 0; j < KB; ++j) q4k_part_load(rp + (wave * KB + j) * 144u, kq, part[t][j]);
    }

    // the x of the wave's first XD groups, then XD groups ahead of their use
    constexpr int NG = KB * 8, XD = NG < 4 ? NG : 4;
    const uint32_t m = live ? n : 0u, kw = wave * KB * 256u;
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
        x_split(xr[gi % XD], live, xf);
        if (gi + XD < NG) x_load(x, in, m, kw + 32u * (gi + XD), kq, xr[gi % XD]);
        const int j = gi / 8, g = gi % 8;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            mbf16x8 b;
            float ds, cb;
            q4k_group(part[t][j], g, b, ds, cb);
            mf32x4 P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.lo, b, mf32x4{0.0f, 0.0f, 0.0f, 0.0f},
                                                               0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.mid, b, P, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf.hi, b, P, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_fmaf(ds, P[i], acc[t][i]);
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

template <int NT, int KB>
hipError_t launch_nt_kb(const uint8_t* W, uint32_t nb, uint32_t rows, const float* x, float* y,
                        uint32_t batch, hipStream_t s) {
    const uint32_t waves = nb / KB;
    const uint32_t blocks = (rows + 16u * NT - 1u) / (16u * NT);
    const size_t lds = static_cast<size_t>(waves) * NT * 64u * sizeof(mf32x4);
    hipLaunchKernelGGL((k_matvec_mfma_q4k<NT, KB>), dim3(blocks), dim3(64u * waves), lds, s, W, nb,
                       x, y, rows, batch);
    return hipGetLastError();
}

}  // namespace

// K blocks per wave: one (two row tiles per wave) up to 8 blocks per row,
// else the fewest (2..4) that leave at most 16 waves (one tile per wave).
// Batches of 5 to 8: at 4 vectors the register kernels are faster.
uint32_t matvec_mfma_blocks_per_wave(uint32_t type, uint32_t in, uint32_t batch) {
    if (type != T_Q4_K || batch < 5u || batch > 8u || in == 0 || in % 256u) return 0;
    const uint32_t nb = in / 256u;
    if (nb <= 8u) return 1;
    for (uint32_t kb = 2; kb <= 4u; ++kb)
        if (nb % kb == 0 && nb / kb <= 16u) return kb;
    return 0;
}

hipError_t launch_matvec_mfma(uint32_t type, const uint8_t* W, uint32_t rows, uint32_t in,
                              const float* x, float* y, uint32_t batch, hipStream_t s) {
    const uint32_t kb = matvec_mfma_blocks_per_wave(type, in, batch);
    const uint32_t nb = in / 256u;
    switch (kb) {
        case 1: return launch_nt_kb<2, 1>(W, nb, rows, x, y, batch, s);
        case 2: return launch_nt_kb<1, 2>(W, nb, rows, x, y, batch, s);
        case 3: return launch_nt_kb<1, 3>(W, nb, rows, x, y, batch, s);
        case 4: return launch_nt_kb<1, 4>(W, nb, rows, x, y, batch, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace pk
