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

__device__ __forceinline__ float block_max(float v, float* red) {
    v = lane63(group_max<64>(v));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
    for (uint32_t w = 1; w < (blockDim.x >> 6); ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------------------
// Embedding row: the reference's FP32 values of 32 consecutive elements
// (dequantize_quantized_row, src/quantized_linear.cpp:427-493, with the
// linear decoders' arithmetic: :166-205, 286-358, 387-423).

template <int T>
__device__ void decode32(const uint8_t* row, uint32_t k0, float* v) {
    if constexpr (T == T_F32) {
        for (uint32_t i = 0; i < 32; ++i) v[i] = reinterpret_cast<const float*>(row)[k0 + i];
    } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = row + (k0 / 256u) * Fmt<T>::BB;
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
    } else if constexpr (T == T_Q6_K) {
        const uint8_t* blk = row + (k0 / 256u) * 210u;
        const uint32_t c = (k0 % 256u) / 32u, half = c / 4u, g = c % 4u;
        const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
        const uint8_t* ql = blk + 64u * half + 32u * (g & 1u);
        const uint8_t* qh = blk + 128u + 32u * half;
        for (uint32_t i = 0; i < 32; ++i) {
            const int s = static_cast<int8_t>(blk[192u + 8u * half + 2u * g + (i >= 16u ? 1u : 0u)]);
            const uint32_t nib = g >= 2u ? ql[i] >> 4 : ql[i] & 15u;
            const int q = static_cast<int>(nib | (((qh[i] >> (2u * g)) & 3u) << 4)) - 32;
            v[i] = __fmul_rn(__fmul_rn(d, static_cast<float>(s)), static_cast<float>(q));
        }
    } else if constexpr (T == T_Q8_0) {
        const uint8_t* blk = row + (k0 / 32u) * 34u;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        for (uint32_t i = 0; i < 32; ++i)
            v[i] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(blk[2 + i])));
    } else {  // Q4_0
        const uint8_t* blk = row + (k0 / 32u) * 18u;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        for (uint32_t i = 0; i < 16; ++i) {
            v[i] = __fmul_rn(d, static_cast<float>(static_cast<int>(blk[2 + i] & 15u) - 8));
            v[i + 16] = __fmul_rn(d, static_cast<float>(static_cast<int>(blk[2 + i] >> 4) - 8));
        }
    }
}

// Step start: hidden = embedding row of tokens[pos]; the RoPE table of pos
// (prepare_qwen_rope, src/qwen3_moe_runner.cpp:141-155).
template <int T>
__global__ __launch_bounds__(256) void k_embed(ModelArgs a) {
    const uint32_t pos = a.state[0];
    const uint32_t token = a.tokens[pos];
    const uint32_t tid = threadIdx.x, half = a.head_dim / 2u;
    const uint8_t* row = a.embd + static_cast<uint64_t>(token) * a.embd_row;
    for (uint32_t c = tid; c < a.hidden / 32u; c += blockDim.x) {
        float v[32];
        decode32<T>(row, 32u * c, v);
        for (uint32_t i = 0; i < 32; ++i) a.hidden_state[32u * c + i] = v[i];
    }
    for (uint32_t p = tid; p < half; p += blockDim.x) {
        const float angle = static_cast<float>(pos) *
                            powf(a.rope_theta, -static_cast<float>(p) / static_cast<float>(half));
        a.rope[p] = cosf(angle);
        a.rope[half + p] = sinf(angle);
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

// Per-head q/k RMSNorm and NeoX RoPE (apply_qwen_rope: pairs (i, i + half));
// k and v go to the FP16 ring slot pos % capacity (src/kv_cache.cpp:131-183,
// round to nearest even).  One workgroup of head_dim threads per head:
// q heads, then k heads, then v heads.
__global__ __launch_bounds__(128) void k_qk_rope_kv(ModelArgs a, ModelLayer L) {
    __shared__ float vals[256];
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, d = threadIdx.x, hd = a.head_dim, half = hd / 2u;
    const uint32_t slot = a.state[0] % a.capacity;
    if (h >= a.heads + a.kv_heads) {  // v heads: copy to the cache
        const uint32_t j = h - a.heads - a.kv_heads;
        L.vcache[(static_cast<uint64_t>(slot) * a.kv_heads + j) * hd + d] =
            __half_as_ushort(__float2half_rn(a.v[j * hd + d]));
        return;
    }
    const bool is_q = h < a.heads;
    float* src = is_q ? a.q + h * hd : a.k + (h - a.heads) * hd;
    const float* nw = is_q ? L.q_norm : L.k_norm;
    const float x = src[d];
    const float total = block_sum(x * x, red);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(hd) + a.rms_eps);
    vals[d] = x * scale * nw[d];
    __syncthreads();
    float r;
    if (d < half) {
        r = vals[d] * a.rope[d] - vals[d + half] * a.rope[half + d];
    } else {
        const uint32_t i = d - half;
        r = vals[d] * a.rope[i] + vals[i] * a.rope[half + i];
    }
    if (is_q) {
        src[d] = r;
    } else {
        const uint32_t j = h - a.heads;
        L.kcache[(static_cast<uint64_t>(slot) * a.kv_heads + j) * hd + d] =
            __half_as_ushort(__float2half_rn(r));
    }
}

// Grouped-query attention of one q head over the ring's positions
// (KvCache::attend, src/kv_cache.cpp:185-293): scores q.k in key order,
// times 1/sqrt(head_dim); softmax; out[d] += p_i * v_i[d] in position order.
__global__ __launch_bounds__(256) void k_attention(ModelArgs a, ModelLayer L) {
    extern __shared__ float sc[];  // [capacity]
    __shared__ float qv[256];
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, tid = threadIdx.x, hd = a.head_dim;
    const uint32_t kvh = h / (a.heads / a.kv_heads);
    const uint32_t pos = a.state[0];
    const uint32_t n = pos + 1u < a.capacity ? pos + 1u : a.capacity;
    const uint32_t first = pos + 1u - n;
    for (uint32_t d = tid; d < hd; d += blockDim.x) qv[d] = a.q[h * hd + d];
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t i = tid; i < n; i += blockDim.x) {
        const uint32_t slot = (first + i) % a.capacity;
        const uint16_t* kr = L.kcache + (static_cast<uint64_t>(slot) * a.kv_heads + kvh) * hd;
        float s = 0.0f;
        for (uint32_t d = 0; d < hd; ++d) s = s + qv[d] * __half2float(__ushort_as_half(kr[d]));
        s = s * a.attn_scale;
        sc[i] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, red);
    float part = 0.0f;
    for (uint32_t i = tid; i < n; i += blockDim.x) {
        const float e = expf(sc[i] - mx);
        sc[i] = e;
        part += e;
    }
    const float denom = block_sum(part, red);
    for (uint32_t d = tid; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t slot = (first + i) % a.capacity;
            const float v = __half2float(__ushort_as_half(
                L.vcache[(static_cast<uint64_t>(slot) * a.kv_heads + kvh) * hd + d]));
            o = o + (sc[i] / denom) * v;
        }
        a.att[h * hd + d] = o;
    }
}

// First-max argmax of the logits (NaN/inf flagged), then the next step's
// token: the prompt's while prompt tokens remain, else the argmax.
__global__ __launch_bounds__(1024) void k_argmax(ModelArgs a) {
    __shared__ float bv[16];
    __shared__ uint32_t bi[16];
    const uint32_t tid = threadIdx.x;
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    bool bad = false;
    for (uint32_t i = tid; i < a.vocab; i += blockDim.x) {  // ascending: strict > keeps the first
        const float v = a.logits[i];
        bad = bad || !isfinite(v);
        if (v > best || idx == 0xffffffffu) {
            best = v;
            idx = i;
        }
    }
    // wave reduction: larger value, then smaller index
    for (uint32_t off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_down(best, off);
        const uint32_t oi = __shfl_down(idx, off);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    const uint32_t any_bad = __any(bad);
    if ((tid & 63u) == 0) {
        bv[tid >> 6] = best;
        bi[tid >> 6] = idx;
        if (any_bad) atomicOr(a.state + 2, 1u);
    }
    __syncthreads();
    if (tid == 0) {
        float b = bv[0];
        uint32_t id = bi[0];
        for (uint32_t w = 1; w < (blockDim.x >> 6); ++w)
            if (bv[w] > b || (bv[w] == b && bi[w] < id)) {
                b = bv[w];
                id = bi[w];
            }
        const uint32_t pos = a.state[0];
        if (pos + 1u >= a.state[1]) a.tokens[pos + 1u] = id;  // past the prompt: generated
        a.state[0] = pos + 1u;
    }
}

__global__ void k_advance(uint32_t* state) {
    if (threadIdx.x == 0) state[0] = state[0] + 1u;
}

template <int T>
hipError_t embed_t(const ModelArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(k_embed<T>, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

bool model_supported(const ModelArgs& a) {
    const bool embd_ok = a.embd_type == T_F32 || a.embd_type == T_Q4_K || a.embd_type == T_Q5_K ||
                         a.embd_type == T_Q6_K || a.embd_type == T_Q8_0 || a.embd_type == T_Q4_0;
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

hipError_t launch_model_step(const ModelArgs& a, const ModelLayer* layers, bool logits,
                             hipStream_t s) {
    hipError_t err = hipSuccess;
    switch (a.embd_type) {
        case T_F32: err = embed_t<T_F32>(a, s); break;
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
        if (logits) hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, a);
        else hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, a.state);
        return hipGetLastError();
    }
    const uint32_t qd = a.heads * a.head_dim, kd = a.kv_heads * a.head_dim;
    const float* delta = nullptr;  // the residual the next RMSNorm adds first
    auto norm = [&](const float* d, const float* w) -> hipError_t {
        hipLaunchKernelGGL(k_add_rmsnorm, dim3(1), dim3(256), 0, s, a.hidden_state, d, w, a.normed,
                           a.hidden, a.rms_eps);
        return hipGetLastError();
    };
    auto matvec = [&](uint32_t type, const uint8_t* W, uint64_t row_bytes, uint32_t rows,
                      uint32_t in, const float* x, float* y) -> hipError_t {
        return launch_matvec(type, W, row_bytes, rows, in, x, y, 1, s);
    };
    for (uint32_t l = 0; l < a.layers; ++l) {
        const ModelLayer& L = layers[l];
        if ((err = norm(delta, L.attn_norm))) return err;
        if ((err = matvec(L.attn_type, L.q, L.q_row, qd, a.hidden, a.normed, a.q))) return err;
        if ((err = matvec(L.attn_type, L.k, L.k_row, kd, a.hidden, a.normed, a.k))) return err;
        if ((err = matvec(L.attn_type, L.v, L.v_row, kd, a.hidden, a.normed, a.v))) return err;
        hipLaunchKernelGGL(k_qk_rope_kv, dim3(a.heads + 2u * a.kv_heads), dim3(a.head_dim), 0, s,
                           a, L);
        hipLaunchKernelGGL(k_attention, dim3(a.heads), dim3(256), a.capacity * sizeof(float), s, a,
                           L);
        if ((err = matvec(L.attn_type, L.o, L.o_row, a.hidden, qd, a.att, a.attn_out))) return err;
        if ((err = norm(a.attn_out, L.ffn_norm))) return err;
        err = launch_moe_decode(L.moe, s);  // normed -> moe_out
        if (err != hipSuccess) return err;
        delta = L.moe.y;
    }
    if (logits) {
        if ((err = norm(delta, a.out_norm))) return err;
        if ((err = matvec(a.out_type, a.out, a.out_row, a.vocab, a.hidden, a.normed, a.logits)))
            return err;
        hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, a);
    } else {
        hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, a.state);
    }
    return hipGetLastError();
}

}  // namespace pk
