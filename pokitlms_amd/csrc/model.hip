// model.hip -- whole Qwen3-MoE greedy decode on gfx950: every layer of a
// token step on the device, one step replayed per token from a HIP graph.
//
// The step follows Qwen3MoeRunner::forward_into (src/qwen3_moe_runner.cpp:
// 580-704): embedding row -> per layer [RMSNorm, q/k/v matvecs, per-head
// q/k RMSNorm, NeoX RoPE, FP16 KV ring append, grouped-query attention, o
// matvec, residual, RMSNorm, routed MoE block, residual] -> final RMSNorm,
// output head, first-max argmax (sample_token at temperature 0, :320-333).
// The token and position of a step live in device memory (ModelArgs::state,
// ::tokens), so the same captured graph serves every step: k_argmax writes
// the next token (or keeps the prompt's) and advances the position.
//
// Also here: the device side of the seeded synthetic weight generator
// (the same bytes as pokitlms_amd/synth_model.py).
#include <hip/hip_fp16.h>
#include <math.h>

#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

// ---------------------------------------------------------------------------
// Synthetic weights: word i of a tensor is splitmix64's output for key + i;
// fix-ups rewrite the scale fields from the stream's own bytes.

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_synth_words(uint8_t* dst, uint64_t nbytes, uint64_t key) {
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (i >= (nbytes + 7u) / 8u) return;
    const uint64_t w = mix64(key + i);
    if (i * 8u + 8u <= nbytes) {
        *reinterpret_cast<uint64_t*>(dst + i * 8u) = w;
    } else {
        for (uint64_t b = 0; i * 8u + b < nbytes; ++b) dst[i * 8u + b] = static_cast<uint8_t>(w >> (8u * b));
    }
}

__device__ __forceinline__ uint32_t synth_fp16(uint32_t b0, uint32_t b1, uint32_t exp) {
    return ((exp + (b1 >> 7)) << 10) | ((b1 & 3u) << 8) | b0;
}

// kind 1: K-quant block of `bb` bytes; kind 2: Q6_K block; kind 3/4: F32 words.
__global__ __launch_bounds__(256) void k_synth_fix(uint8_t* dst, uint64_t units, uint32_t kind,
                                                   uint32_t bb) {
    const uint64_t u = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    if (u >= units) return;
    if (kind == 1u) {
        uint8_t* b = dst + u * bb;
        const uint32_t d = synth_fp16(b[0], b[1], 5u);
        b[0] = b[2] = static_cast<uint8_t>(d);
        b[1] = b[3] = static_cast<uint8_t>(d >> 8);
        uint32_t sc[8], m[8];
        for (int j = 0; j < 8; ++j) {
            sc[j] = 1u + (b[4 + j] & 7u);
            m[j] = (15u * sc[j] + 1u) >> 1;
        }
        for (int j = 0; j < 4; ++j) {
            b[4 + j] = static_cast<uint8_t>((sc[j] & 63u) | ((sc[j + 4] >> 4) << 6));
            b[8 + j] = static_cast<uint8_t>((m[j] & 63u) | ((m[j + 4] >> 4) << 6));
            b[12 + j] = static_cast<uint8_t>((sc[j + 4] & 15u) | ((m[j + 4] & 15u) << 4));
        }
    } else if (kind == 2u) {
        uint8_t* b = dst + u * 210u;
        const uint32_t d = synth_fp16(b[208], b[209], 1u);
        b[208] = static_cast<uint8_t>(d);
        b[209] = static_cast<uint8_t>(d >> 8);
    } else {
        uint32_t* w = reinterpret_cast<uint32_t*>(dst) + u;
        *w = kind == 3u ? (0x3F800000u | (*w & 0x000FFFFFu)) : ((*w & 0x807FFFFFu) | (120u << 23));
    }
}

// ---------------------------------------------------------------------------
// Reductions over a workgroup (wave DPP sums, then LDS).

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = lane63(group_sum<64>(v));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = 0.0f;
    for (uint32_t w = 0; w < (blockDim.x >> 6); ++w) r += red[w];
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------------------
// Embedding row: the reference's FP32 values of 32 consecutive elements
// (dequantize_quantized_row, src/quantized_linear.cpp:427-493, with the
// linear decoders' arithmetic: :166-205, 286-358, 387-423).

template <int T>
__device__ void decode32(const QRow& row, uint32_t k0, float* v) {
    if constexpr (T == T_F32) {  // blocks of one element
        const float* f = reinterpret_cast<const float*>(block_ptr<4>(row, k0));
        for (uint32_t i = 0; i < 32; ++i) v[i] = f[i];
    } else if constexpr (T == T_F16 || T == T_BF16) {  // read_float_rows_into (src/tensor_reader.cpp:164-198)
        const uint16_t* h = reinterpret_cast<const uint16_t*>(block_ptr<2>(row, k0));
        for (uint32_t i = 0; i < 32; ++i)
            v[i] = T == T_F16 ? half_bits_to_float(h[i]) : __uint_as_float(static_cast<uint32_t>(h[i]) << 16);
    } else if constexpr (T == T_Q4_1) {  // decode_q4_1: fl(fl(q * d) + m) (src/quantized_linear.cpp:53-62)
        const uint8_t* blk = block_ptr<20>(row, k0 / 32u);
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        const float m = half_bits_to_float(blk[2] | (blk[3] << 8));
        for (uint32_t i = 0; i < 16; ++i) {
            v[i] = __fadd_rn(__fmul_rn(static_cast<float>(blk[4 + i] & 15u), d), m);
            v[i + 16] = __fadd_rn(__fmul_rn(static_cast<float>(blk[4 + i] >> 4), d), m);
        }
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = block_ptr<Fmt<T>::BB>(row, k0 / 256u);
        const uint32_t j = (k0 % 256u) / 32u, chunk = j / 2u, hi = j & 1u;
        uint32_t h[4];
        for (int i = 0; i < 4; ++i)
            h[i] = blk[4 * i] | (blk[4 * i + 1] << 8) | (blk[4 * i + 2] << 16) | (blk[4 * i + 3] << 24);
        const float d = half_bits_to_float(h[0] & 0xffffu), dmin = half_bits_to_float(h[0] >> 16);
        float sc, mn;
        kq_scale_min(h, j, sc, mn);
        const float ds = __fmul_rn(d, sc), dm = __fmul_rn(dmin, mn);
        const uint8_t* qs = blk + (T == T_Q4_K ? 16u : 48u) + 32u * chunk;
        for (uint32_t i = 0; i < 32; ++i) {
            uint32_t q = hi ? qs[i] >> 4 : qs[i] & 15u;
            if constexpr (T == T_Q5_K) q += ((blk[16u + i] >> j) & 1u) << 4;
            v[i] = __fsub_rn(__fmul_rn(ds, static_cast<float>(q)), dm);
        }
    } else if constexpr (T == T_Q6_K) {  // planar fields (layout.hpp)
        using L = Planar<T_Q6_K>;
        const uint32_t b = k0 / 256u, c = (k0 % 256u) / 32u, half = c / 4u, g = c % 4u;
        const float d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, b)));
        const uint8_t* ql = field_ptr<L::QL, 128>(row, b) + 64u * half + 32u * (g & 1u);
        const uint8_t* qh = field_ptr<L::QH, 64>(row, b) + 32u * half;
        const uint8_t* sc = field_ptr<L::SC, 16>(row, b) + 8u * half + 2u * g;
        for (uint32_t i = 0; i < 32; ++i) {
            const int s = static_cast<int8_t>(sc[i >= 16u ? 1u : 0u]);
            const uint32_t nib = g >= 2u ? ql[i] >> 4 : ql[i] & 15u;
            const int q = static_cast<int>(nib | (((qh[i] >> (2u * g)) & 3u) << 4)) - 32;
            v[i] = __fmul_rn(__fmul_rn(d, static_cast<float>(s)), static_cast<float>(q));
        }
    } else if constexpr (T == T_Q5_0 || T == T_Q5_1) {  // decode_q5_0 / q5_1 (:64-93)
        const uint8_t* qs;
        uint32_t qh;
        float d, m = 0.0f;
        if constexpr (T == T_Q5_0) {
            using L = Planar<T_Q5_0>;
            qs = field_ptr<L::QS, 16>(row, k0 / 32u);
            qh = *reinterpret_cast<const uint32_t*>(field_ptr<L::QH, 4>(row, k0 / 32u));
            d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, k0 / 32u)));
        } else {
            const uint8_t* blk = block_ptr<24>(row, k0 / 32u);
            d = half_bits_to_float(blk[0] | (blk[1] << 8));
            m = half_bits_to_float(blk[2] | (blk[3] << 8));
            qh = *reinterpret_cast<const uint32_t*>(blk + 4);
            qs = blk + 8;
        }
        for (uint32_t i = 0; i < 16; ++i) {
            const uint32_t q0 = (qs[i] & 15u) | (((qh >> i) & 1u) << 4);
            const uint32_t q1 = (qs[i] >> 4) | (((qh >> (i + 16u)) & 1u) << 4);
            if constexpr (T == T_Q5_0) {
                v[i] = __fmul_rn(static_cast<float>(static_cast<int>(q0) - 16), d);
                v[i + 16] = __fmul_rn(static_cast<float>(static_cast<int>(q1) - 16), d);
            } else {
                v[i] = __fadd_rn(__fmul_rn(static_cast<float>(q0), d), m);
                v[i + 16] = __fadd_rn(__fmul_rn(static_cast<float>(q1), d), m);
            }
        }
    } else if constexpr (T == T_Q2_K || T == T_Q3_K) {  // decode_q2_k / q3_k (:95-164)
        const uint32_t b = k0 / 256u, c = (k0 % 256u) / 32u;  // elements 32c .. 32c + 31
        const uint32_t h = c / 4u, sh = c % 4u;               // groups 2c, 2c + 1 (t = 0, 1)
        for (uint32_t i = 0; i < 32; ++i) {
            const uint32_t t = i / 16u, l = i % 16u, g = 2u * c + t;
            if constexpr (T == T_Q2_K) {
                const uint8_t* blk = block_ptr<84>(row, b);
                const float d = half_bits_to_float(blk[80] | (blk[81] << 8));
                const float dmin = half_bits_to_float(blk[82] | (blk[83] << 8));
                const uint32_t q = (blk[16u + 32u * h + 16u * t + l] >> (2u * sh)) & 3u;
                const float dl = __fmul_rn(d, static_cast<float>(blk[g] & 15u));
                const float ml = __fmul_rn(dmin, static_cast<float>(blk[g] >> 4));
                v[i] = __fsub_rn(__fmul_rn(dl, static_cast<float>(q)), ml);
            } else {
                using L = Planar<T_Q3_K>;
                const uint8_t* qs = field_ptr<L::QS, 64>(row, b);
                const uint8_t* hm = field_ptr<L::HM, 32>(row, b);
                const uint8_t* ps = field_ptr<L::SC, 12>(row, b);
                const uint32_t pw[3] = {*reinterpret_cast<const uint32_t*>(ps),
                                        *reinterpret_cast<const uint32_t*>(ps + 4),
                                        *reinterpret_cast<const uint32_t*>(ps + 8)};
                const float d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, b)));
                const uint32_t q = (qs[32u * h + 16u * t + l] >> (2u * sh)) & 3u;
                const uint32_t hb = (hm[16u * t + l] >> (4u * h + sh)) & 1u;
                const float ds = __fmul_rn(d, static_cast<float>(static_cast<int>(q3k_scale(pw, g)) - 32));
                v[i] = __fmul_rn(ds, static_cast<float>(static_cast<int>(q) - (hb ? 0 : 4)));
            }
        }
    } else if constexpr (T == T_Q8_0) {
        using L = Planar<T_Q8_0>;
        const uint8_t* qs = field_ptr<L::QS, 32>(row, k0 / 32u);
        const float d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, k0 / 32u)));
        for (uint32_t i = 0; i < 32; ++i)
            v[i] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(qs[i])));
    } else {  // Q4_0
        using L = Planar<T_Q4_0>;
        const uint8_t* qs = field_ptr<L::QS, 16>(row, k0 / 32u);
        const float d = half_bits_to_float(ld_u16(field_ptr<L::D, 2>(row, k0 / 32u)));
        for (uint32_t i = 0; i < 16; ++i) {
            v[i] = __fmul_rn(d, static_cast<float>(static_cast<int>(qs[i] & 15u) - 8));
            v[i + 16] = __fmul_rn(d, static_cast<float>(static_cast<int>(qs[i] >> 4) - 8));
        }
    }
}

// Step start: hidden = embedding row of tokens[pos].
template <int T>
__global__ __launch_bounds__(256) void k_embed(ModelArgs a) {
    const uint32_t pos = a.state[0];
    const uint32_t token = a.tokens[pos];
    const uint32_t tid = threadIdx.x;
    // blocks per row (one element per block for the float types)
    uint32_t nb = a.hidden;
    if constexpr (!(T == T_F32 || T == T_F16 || T == T_BF16)) nb = a.hidden / Fmt<T>::BE;
    const QRow row{a.embd, static_cast<uint64_t>(a.vocab) * nb, static_cast<uint64_t>(token) * nb};
    for (uint32_t c = tid; c < a.hidden / 32u; c += blockDim.x) {
        float v[32];
        decode32<T>(row, 32u * c, v);
        for (uint32_t i = 0; i < 32; ++i) a.hidden_state[32u * c + i] = v[i];
    }
}

// hidden += delta (if any), then out = RMSNorm(hidden) * w (src/rms_norm.cpp:9-27:
// out = x * (1 / sqrt(mean(x^2) + eps)) * w).
__global__ __launch_bounds__(256) void k_add_rmsnorm(float* __restrict__ x, const float* __restrict__ delta,
                                                     const float* __restrict__ w, float* __restrict__ out,
                                                     uint32_t n, float eps) {
    __shared__ float red[4];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        float v = x[i];
        if (delta) {
            v = v + delta[i];
            x[i] = v;
        }
        ss += v * v;
    }
    const float total = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(n) + eps);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * scale * w[i];
}

// The same for n % 4 == 0, n <= 1024·NI, 16-byte-aligned rows: each thread
// loads its float4s of x, delta and w at once and keeps them in registers, so
// the kernel waits for memory once (the loop above reloads x after storing
// it, and loads w only after the sum).
// x + delta goes to xo (x itself, or a buffer of its own).
template <int NI>
__global__ __launch_bounds__(256) void k_add_rmsnorm4(const float* x,
                                                      const float* __restrict__ delta,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ out, uint32_t n,
                                                      float eps, float* xo) {
    __shared__ float red[4];
    const uint32_t n4 = n / 4u;
    float4 v[NI], wv[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const uint32_t c = threadIdx.x + 256u * i, cc = c < n4 ? c : 0u;
        v[i] = reinterpret_cast<const float4*>(x)[cc];
        wv[i] = reinterpret_cast<const float4*>(w)[cc];
        if (delta) {
            const float4 d = reinterpret_cast<const float4*>(delta)[cc];
            v[i].x = v[i].x + d.x;
            v[i].y = v[i].y + d.y;
            v[i].z = v[i].z + d.z;
            v[i].w = v[i].w + d.w;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        if (threadIdx.x + 256u * i < n4) {
            ss += v[i].x * v[i].x;
            ss += v[i].y * v[i].y;
            ss += v[i].z * v[i].z;
            ss += v[i].w * v[i].w;
        }
    }
    const float total = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(n) + eps);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const uint32_t c = threadIdx.x + 256u * i;
        if (c < n4) {
            if (delta || xo != x) reinterpret_cast<float4*>(xo)[c] = v[i];
            reinterpret_cast<float4*>(out)[c] =
                make_float4(v[i].x * scale * wv[i].x, v[i].y * scale * wv[i].y,
                            v[i].z * scale * wv[i].z, v[i].w * scale * wv[i].w);
        }
    }
}

// First-max argmax of the logits in two launches: each workgroup of
// k_argmax_part the maximum of one 2048-logit chunk (larger value, then smaller
// index: the first maximum), non-finite logits flagged; k_argmax the maximum
// of the chunks, then the next step's token: the prompt's while prompt tokens
// remain, else the argmax (sample_token at temperature 0,
// src/qwen3_moe_runner.cpp:320-333).
constexpr uint32_t kArgmaxChunk = 2048;

__device__ __forceinline__ void argmax_merge(float& best, uint32_t& idx, float ov, uint32_t oi) {
    if (ov > best || (ov == best && oi < idx)) {
        best = ov;
        idx = oi;
    }
}

__device__ __forceinline__ void argmax_wave(float& best, uint32_t& idx) {
    for (uint32_t off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_down(best, off);
        const uint32_t oi = __shfl_down(idx, off);
        argmax_merge(best, idx, ov, oi);
    }
}

__global__ __launch_bounds__(256) void k_argmax_part(ModelArgs a) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const uint32_t tid = threadIdx.x, base = blockIdx.x * kArgmaxChunk;
    float v[kArgmaxChunk / 256];
#pragma unroll
    for (uint32_t k = 0; k < kArgmaxChunk / 256; ++k) {
        const uint32_t i = base + tid + 256u * k;
        v[k] = a.logits[i < a.vocab ? i : 0u];
    }
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    bool bad = false;
#pragma unroll
    for (uint32_t k = 0; k < kArgmaxChunk / 256; ++k) {  // ascending: strict > keeps the first
        const uint32_t i = base + tid + 256u * k;
        if (i < a.vocab) {
            bad = bad || !isfinite(v[k]);
            if (v[k] > best || idx == 0xffffffffu) {
                best = v[k];
                idx = i;
            }
        }
    }
    argmax_wave(best, idx);
    const uint32_t any_bad = __any(bad);
    if ((tid & 63u) == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = idx;
        if (any_bad) atomicOr(a.state + 2, 1u);
    }
    __syncthreads();
    if (tid == 0) {
        for (uint32_t w = 1; w < 4; ++w) argmax_merge(bv[0], bi[0], bv[w], bi[w]);
        a.argmax_part[2u * blockIdx.x] = bv[0];
        a.argmax_part[2u * blockIdx.x + 1u] = __uint_as_float(bi[0]);
    }
}

__global__ __launch_bounds__(256) void k_argmax(ModelArgs a, uint32_t parts) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4];
    const uint32_t tid = threadIdx.x;
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    for (uint32_t c = tid; c < parts; c += 256u)
        argmax_merge(best, idx, a.argmax_part[2u * c], __float_as_uint(a.argmax_part[2u * c + 1u]));
    argmax_wave(best, idx);
    if ((tid & 63u) == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (uint32_t w = 1; w < 4; ++w) argmax_merge(bv[0], bi[0], bv[w], bi[w]);
        const uint32_t pos = a.state[0];
        if (pos + 1u >= a.state[1]) a.tokens[pos + 1u] = bi[0];  // past the prompt: generated
        a.state[0] = pos + 1u;
    }
}

__global__ void k_advance(uint32_t* state) {
    if (threadIdx.x == 0) state[0] = state[0] + 1u;
}

hipError_t launch_argmax(const ModelArgs& a, hipStream_t s) {
    const uint32_t parts = (a.vocab + kArgmaxChunk - 1u) / kArgmaxChunk;
    hipLaunchKernelGGL(k_argmax_part, dim3(parts), dim3(256), 0, s, a);
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(256), 0, s, a, parts);
    return hipGetLastError();
}

template <int T>
hipError_t embed_t(const ModelArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_embed<T>, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

namespace {

// One thread per 32 consecutive elements of the requested rows.
template <int T>
__global__ __launch_bounds__(256) void k_dequant_rows(const uint8_t* __restrict__ slice,
                                                      uint64_t rows_in_slice, uint32_t in,
                                                      uint64_t first_row, uint32_t rows,
                                                      float* __restrict__ out) {
    const uint64_t chunks = static_cast<uint64_t>(rows) * (in / 32u);
    uint32_t nb = in;
    if constexpr (!(T == T_F32 || T == T_F16 || T == T_BF16)) nb = in / Fmt<T>::BE;
    for (uint64_t k = blockIdx.x * 256ull + threadIdx.x; k < chunks;
         k += static_cast<uint64_t>(gridDim.x) * 256u) {
        const uint64_t r = k / (in / 32u), c = k % (in / 32u);
        const QRow row{slice, rows_in_slice * nb, (first_row + r) * nb};
        float v[32];
        decode32<T>(row, 32u * static_cast<uint32_t>(c), v);
        float* o = out + r * in + 32u * c;
        for (uint32_t i = 0; i < 32; ++i) o[i] = v[i];
    }
}

template <int T>
hipError_t dequant_t(const uint8_t* slice, uint64_t rows_in_slice, uint32_t in, uint64_t first_row,
                     uint32_t rows, float* out, hipStream_t s) {
    const uint64_t chunks = static_cast<uint64_t>(rows) * (in / 32u);
    const uint32_t blocks = static_cast<uint32_t>(chunks / 256u + 1u < 4096u ? chunks / 256u + 1u : 4096u);
    hipLaunchKernelGGL(k_dequant_rows<T>, dim3(blocks), dim3(256), 0, s, slice, rows_in_slice, in,
                       first_row, rows, out);
    return hipGetLastError();
}

}  // namespace

bool dequant_rows_supported(uint32_t type, uint32_t in) {
    if (in == 0 || in % 32u) return false;
    switch (type) {
        case T_F32: case T_F16: case T_BF16: case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1:
        case T_Q8_0: return true;
        case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: return in % 256u == 0;
        default: return false;
    }
}

hipError_t launch_dequant_rows(uint32_t type, const uint8_t* slice, uint64_t rows_in_slice,
                               uint32_t in, uint64_t first_row, uint32_t rows, float* out,
                               hipStream_t s) {
    if (!dequant_rows_supported(type, in)) return hipErrorInvalidValue;
    switch (type) {
#define PK_DQ(TT) case TT: return dequant_t<TT>(slice, rows_in_slice, in, first_row, rows, out, s);
        PK_DQ(T_F32) PK_DQ(T_F16) PK_DQ(T_BF16) PK_DQ(T_Q4_0) PK_DQ(T_Q4_1) PK_DQ(T_Q5_0)
        PK_DQ(T_Q5_1) PK_DQ(T_Q8_0) PK_DQ(T_Q2_K) PK_DQ(T_Q3_K) PK_DQ(T_Q4_K) PK_DQ(T_Q5_K)
        PK_DQ(T_Q6_K)
#undef PK_DQ
        default: return hipErrorInvalidValue;
    }
}

bool model_supported(const ModelArgs& a) {
    // every type dequantize_quantized_row and read_float_rows_into take
    const bool embd_ok = a.embd_type == T_F32 || a.embd_type == T_F16 || a.embd_type == T_BF16 ||
                         a.embd_type == T_Q2_K || a.embd_type == T_Q3_K || a.embd_type == T_Q4_K ||
                         a.embd_type == T_Q5_K || a.embd_type == T_Q6_K || a.embd_type == T_Q8_0 ||
                         a.embd_type == T_Q4_0 || a.embd_type == T_Q4_1 || a.embd_type == T_Q5_0 ||
                         a.embd_type == T_Q5_1;
    return embd_ok && a.head_dim >= 2u && a.head_dim <= 256u && a.head_dim % 64u == 0u &&
           a.kv_heads >= 1u && a.heads % a.kv_heads == 0u && a.hidden % 256u == 0u &&
           a.capacity >= 1u && a.capacity <= kMaxModelContext;
}

hipError_t launch_synth_fill(uint8_t* dst, uint64_t nbytes, uint64_t key, uint32_t kind,
                             uint32_t block_bytes, hipStream_t s) {
    const uint64_t words = (nbytes + 7u) / 8u;
    hipLaunchKernelGGL(k_synth_words, dim3(static_cast<uint32_t>((words + 255u) / 256u)), dim3(256),
                       0, s, dst, nbytes, key);
    uint64_t units = 0;
    if (kind == 1u || kind == 2u) units = nbytes / block_bytes;
    if (kind == 3u || kind == 4u) units = nbytes / 4u;
    if (units)
        hipLaunchKernelGGL(k_synth_fix, dim3(static_cast<uint32_t>((units + 255u) / 256u)), dim3(256), 0,
                           s, dst, units, kind, block_bytes);
    return hipGetLastError();
}

// x + d into xo (default: x), its RMSNorm into out.
hipError_t launch_fast_add_rmsnorm(float* x, const float* d, const float* w, float* out, uint32_t n,
                                   float eps, hipStream_t s, float* xo) {
    if (n == 0) return hipErrorInvalidValue;
    const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const uint32_t ni = (n + 1023u) / 1024u;
    if (n % 4u == 0 && ni <= 8u && al16(x) && al16(d) && al16(w) && al16(out) && al16(xo)) {
        float* o = xo ? xo : x;
        const dim3 g(1), b(256);
        if (ni == 1u) hipLaunchKernelGGL(k_add_rmsnorm4<1>, g, b, 0, s, x, d, w, out, n, eps, o);
        else if (ni == 2u) hipLaunchKernelGGL(k_add_rmsnorm4<2>, g, b, 0, s, x, d, w, out, n, eps, o);
        else if (ni <= 4u) hipLaunchKernelGGL(k_add_rmsnorm4<4>, g, b, 0, s, x, d, w, out, n, eps, o);
        else hipLaunchKernelGGL(k_add_rmsnorm4<8>, g, b, 0, s, x, d, w, out, n, eps, o);
    } else {
        if (xo && xo != x) {  // the plain kernel adds in place: copy x to xo first
            hipError_t err = hipMemcpyAsync(xo, x, static_cast<size_t>(n) * sizeof(float),
                                            hipMemcpyDeviceToDevice, s);
            if (err != hipSuccess) return err;
            x = xo;
        }
        hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(256), 0, s, x, d, w, out, n, eps);
    }
    return hipGetLastError();
}

hipError_t launch_model_step(const ModelArgs& a, const ModelLayer* layers, bool logits,
                             hipStream_t s) {
    hipError_t err = hipSuccess;
    switch (a.embd_type) {
        case T_F32: err = embed_t<T_F32>(a, s); break;
        case T_F16: err = embed_t<T_F16>(a, s); break;
        case T_BF16: err = embed_t<T_BF16>(a, s); break;
        case T_Q4_1: err = embed_t<T_Q4_1>(a, s); break;
        case T_Q5_0: err = embed_t<T_Q5_0>(a, s); break;
        case T_Q5_1: err = embed_t<T_Q5_1>(a, s); break;
        case T_Q2_K: err = embed_t<T_Q2_K>(a, s); break;
        case T_Q3_K: err = embed_t<T_Q3_K>(a, s); break;
        case T_Q4_K: err = embed_t<T_Q4_K>(a, s); break;
        case T_Q5_K: err = embed_t<T_Q5_K>(a, s); break;
        case T_Q6_K: err = embed_t<T_Q6_K>(a, s); break;
        case T_Q8_0: err = embed_t<T_Q8_0>(a, s); break;
        case T_Q4_0: err = embed_t<T_Q4_0>(a, s); break;
        default: return hipErrorInvalidValue;
    }
    if (err != hipSuccess) return err;
    if (a.exact) {
        if ((err = launch_ref_step(a, layers, logits, s))) return err;
        if (logits) return launch_argmax(a, s);
        hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, a.state);
        return hipGetLastError();
    }
    const uint32_t qd = a.heads * a.head_dim, kd = a.kv_heads * a.head_dim;
    const float* delta = nullptr;  // the residual the next RMSNorm adds first
    auto norm = [&](const float* d, const float* w) -> hipError_t {
        return launch_fast_add_rmsnorm(a.hidden_state, d, w, a.normed, a.hidden, a.rms_eps, s);
    };
    auto matvec = [&](uint32_t type, const uint8_t* W, uint64_t row_bytes, uint32_t rows,
                      uint32_t in, const float* x, float* y) -> hipError_t {
        return launch_matvec(type, W, row_bytes, rows, in, x, y, 1, s, nullptr);
    };
    for (uint32_t l = 0; l < a.layers; ++l) {
        const ModelLayer& L = layers[l];
        const bool qkv = L.qkv && a.k == a.q + qd && a.v == a.k + kd;  // q, k and v in one launch
        // The attention RMSNorm inside the q/k/v matvec's staging: hidden_state
        // + delta goes to hidden_alt, and the FFN norm brings hidden_alt +
        // attn_out back to hidden_state (every workgroup reads hidden_state
        // while one writes the sum, so the sum needs a buffer of its own).
        bool fused = false;
        if (qkv) {
            const MatvecNorm nm{delta, L.attn_norm, a.hidden_alt, a.rms_eps};
            err = launch_matvec_norm(L.attn_type, L.qkv, qd + 2u * kd, a.hidden, a.hidden_state, nm,
                                     a.q, s);
            if (err != hipSuccess && err != hipErrorNotSupported) return err;
            fused = err == hipSuccess;
        }
        if (!fused) {
            if ((err = norm(delta, L.attn_norm))) return err;
            if (qkv) {
                if ((err = matvec(L.attn_type, L.qkv, L.q_row, qd + 2u * kd, a.hidden, a.normed, a.q)))
                    return err;
            } else {
                if ((err = matvec(L.attn_type, L.q, L.q_row, qd, a.hidden, a.normed, a.q))) return err;
                if ((err = matvec(L.attn_type, L.k, L.k_row, kd, a.hidden, a.normed, a.k))) return err;
                if ((err = matvec(L.attn_type, L.v, L.v_row, kd, a.hidden, a.normed, a.v))) return err;
            }
        }
        if ((err = launch_fast_attention(a, L, s))) return err;
        if ((err = matvec(L.attn_type, L.o, L.o_row, a.hidden, qd, a.att, a.attn_out))) return err;
        if (fused) {
            if ((err = launch_fast_add_rmsnorm(a.hidden_alt, a.attn_out, L.ffn_norm, a.normed,
                                               a.hidden, a.rms_eps, s, a.hidden_state)))
                return err;
        } else if ((err = norm(a.attn_out, L.ffn_norm))) {
            return err;
        }
        err = launch_moe_decode(L.moe, s);  // normed -> moe_out
        if (err != hipSuccess) return err;
        delta = L.moe.y;
    }
    if (logits) {
        if ((err = norm(delta, a.out_norm))) return err;
        if ((err = matvec(a.out_type, a.out, a.out_row, a.vocab, a.hidden, a.normed, a.logits)))
            return err;
        return launch_argmax(a, s);
    } else {
        hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, a.state);
    }
    return hipGetLastError();
}

}  // namespace pk
