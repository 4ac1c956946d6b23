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

// bucket[t] .. bucket[t + 1]: the pairs whose input's top 16 bits are t
// (at most a few hundred per bucket for glibc), binary-searched.
__device__ float expf_libm(float x, const uint32_t* bucket, const uint32_t* pairs) {
    float r = static_cast<float>(exp(static_cast<double>(x)));
    if (bucket) {
        const uint32_t b = __float_as_uint(x);
        uint32_t lo = bucket[b >> 16], hi = bucket[(b >> 16) + 1u];
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (pairs[2u * mid] < b) lo = mid + 1u;
            else hi = mid;
        }
        if (lo < bucket[(b >> 16) + 1u] && pairs[2u * lo] == b) r = __uint_as_float(pairs[2u * lo + 1u]);
    }
    return r;
}

__device__ __forceinline__ uint32_t u16_at(const uint8_t* p) { return p[0] | (p[1] << 8); }

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

// dot of one block with x (x in LDS), in element order.  K-quants: the
// decoded FP32 weight times x; Q8_0/Q4_0: d * dot_i8_f32 (the int8 value
// times x, then the scale once).
template <int T>
__device__ float block_dot(const uint8_t* blk, const float* x) {
    float s = 0.0f;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        uint32_t h[4];
        for (int i = 0; i < 4; ++i) h[i] = u16_at(blk + 4 * i) | (u16_at(blk + 4 * i + 2) << 16);
        const float d = half_bits_to_float(h[0] & 0xffffu), dmin = half_bits_to_float(h[0] >> 16);
        for (uint32_t j = 0; j < 8; ++j) {
            float sc, mn;
            kq_scale_min(h, j, sc, mn);
            const float ds = __fmul_rn(d, sc), dm = __fmul_rn(dmin, mn);
            const uint8_t* qs = blk + (T == T_Q4_K ? 16u : 48u) + 32u * (j / 2u);
            for (uint32_t i = 0; i < 32; ++i) {
                uint32_t q = (j & 1u) ? qs[i] >> 4 : qs[i] & 15u;
                if constexpr (T == T_Q5_K) q += ((blk[16u + i] >> j) & 1u) << 4;
                const float w = __fsub_rn(__fmul_rn(ds, static_cast<float>(q)), dm);
                s = __fadd_rn(s, __fmul_rn(w, x[32u * j + i]));
            }
        }
    } else if constexpr (T == T_Q6_K) {
        const float d = half_bits_to_float(u16_at(blk + 208));
        for (uint32_t c = 0; c < 8; ++c) {
            const uint32_t half = c / 4u, g = c % 4u;
            const uint8_t* ql = blk + 64u * half + 32u * (g & 1u);
            const uint8_t* qh = blk + 128u + 32u * half;
            for (uint32_t i = 0; i < 32; ++i) {
                const int sc = static_cast<int8_t>(blk[192u + 8u * half + 2u * g + (i >= 16u ? 1u : 0u)]);
                const uint32_t nib = g >= 2u ? ql[i] >> 4 : ql[i] & 15u;
                const int q = static_cast<int>(nib | (((qh[i] >> (2u * g)) & 3u) << 4)) - 32;
                const float w = __fmul_rn(__fmul_rn(d, static_cast<float>(sc)), static_cast<float>(q));
                s = __fadd_rn(s, __fmul_rn(w, x[32u * c + i]));
            }
        }
    } else if constexpr (T == T_Q8_0) {
        for (uint32_t i = 0; i < 32; ++i)
            s = __fadd_rn(s, __fmul_rn(x[i], static_cast<float>(static_cast<int8_t>(blk[2 + i]))));
        s = __fmul_rn(half_bits_to_float(u16_at(blk)), s);
    } else {  // Q4_0: low nibbles are elements 0..15, high 16..31
        for (uint32_t i = 0; i < 32; ++i) {
            const uint32_t b = blk[2 + (i & 15u)];
            const int q = static_cast<int>(i < 16u ? (b & 15u) : (b >> 4)) - 8;
            s = __fadd_rn(s, __fmul_rn(x[i], static_cast<float>(q)));
        }
        s = __fmul_rn(half_bits_to_float(u16_at(blk)), s);
    }
    return s;
}

// y[route][row] for rows of W (route: the expert ids[route] slice when ids
// is set), x[route] staged in LDS.  Lanes (row, block); one lane per row then
// sums the block dots in block order starting from 0.
template <int T>
__global__ __launch_bounds__(256) void k_ref_matvec(RefMatvecArgs a) {
    extern __shared__ float lds[];  // x [in], then partial dots [256]
    constexpr uint32_t BE = RefBlock<T>::BE, BB = RefBlock<T>::BB;
    const uint32_t r = blockIdx.y, tid = threadIdx.x;
    const uint32_t nb = a.in / BE, rpw = 256u / nb;
    const float* x = a.x + static_cast<uint64_t>(r) * a.x_stride;
    float* xs = lds;
    float* part = lds + a.in;
    for (uint32_t i = tid; i < a.in; i += 256u) xs[i] = x[i];
    __syncthreads();
    const uint8_t* W = a.W + (a.ids ? static_cast<uint64_t>(a.ids[r]) * a.slice_bytes : 0u);
    const uint32_t row0 = blockIdx.x * rpw, lr = tid / nb, b = tid % nb, row = row0 + lr;
    if (lr < rpw && row < a.rows)
        part[tid] = block_dot<T>(W + static_cast<uint64_t>(row) * a.row_bytes + b * BB, xs + b * BE);
    __syncthreads();
    if (tid < rpw && row0 + tid < a.rows) {
        float s = 0.0f;
        for (uint32_t k = 0; k < nb; ++k) s = __fadd_rn(s, part[tid * nb + k]);
        a.y[static_cast<uint64_t>(r) * a.y_stride + row0 + tid] = s;
    }
}

// F32 linear: 0 + dot_f32(w_row, x), one lane per row over the whole width.
__global__ __launch_bounds__(256) void k_ref_linear_f32(RefMatvecArgs a) {
    extern __shared__ float xs[];
    const uint32_t r = blockIdx.y, tid = threadIdx.x;
    const float* x = a.x + static_cast<uint64_t>(r) * a.x_stride;
    for (uint32_t i = tid; i < a.in; i += 256u) xs[i] = x[i];
    __syncthreads();
    const uint32_t row = blockIdx.x * 256u + tid;
    if (row >= a.rows) return;
    const float* w = reinterpret_cast<const float*>(a.W + static_cast<uint64_t>(row) * a.row_bytes);
    float s = 0.0f;
    for (uint32_t i = 0; i < a.in; ++i) s = __fadd_rn(s, __fmul_rn(w[i], xs[i]));
    a.y[static_cast<uint64_t>(r) * a.y_stride + row] = __fadd_rn(0.0f, s);
}

// x += delta (if any); out = (x * scale) * w, scale = 1 / sqrt(sum_sq / n + eps)
// with sum_sq the serial FP32 sum of the rounded squares.  One workgroup per
// row of `n` values (rows: the per-head q/k norms).
__global__ __launch_bounds__(256) void k_ref_rmsnorm(float* x, const float* delta, const float* w,
                                                     float* out, uint32_t n, float eps) {
    extern __shared__ float sq[];
    __shared__ float s_scale;
    float* xr = x + static_cast<uint64_t>(blockIdx.x) * n;
    float* orow = out + static_cast<uint64_t>(blockIdx.x) * n;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        float v = xr[i];
        if (delta) {
            v = __fadd_rn(v, delta[i]);
            xr[i] = v;
        }
        sq[i] = __fmul_rn(v, v);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (uint32_t i = 0; i < n; ++i) s = __fadd_rn(s, sq[i]);
        s_scale = 1.0f / sqrtf(s / static_cast<float>(n) + eps);
    }
    __syncthreads();
    const float scale = s_scale;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x)
        orow[i] = __fmul_rn(__fmul_rn(xr[i], scale), w[i]);
}

// Per-head q/k RMSNorm (serial) and RoPE from the host-computed table, k and
// v to the FP16 ring: q heads, then k heads, then v heads.
__global__ __launch_bounds__(128) void k_ref_qk_rope_kv(ModelArgs a, ModelLayer L) {
    __shared__ float vals[256];
    __shared__ float s_scale;
    const uint32_t h = blockIdx.x, d = threadIdx.x, hd = a.head_dim, half = hd / 2u;
    const uint32_t pos = a.state[0], slot = pos % a.capacity;
    if (h >= a.heads + a.kv_heads) {
        const uint32_t j = h - a.heads - a.kv_heads;
        L.vcache[(static_cast<uint64_t>(slot) * a.kv_heads + j) * hd + d] =
            __half_as_ushort(__float2half_rn(a.v[j * hd + d]));
        return;
    }
    const bool is_q = h < a.heads;
    float* src = is_q ? a.q + h * hd : a.k + (h - a.heads) * hd;
    const float* nw = is_q ? L.q_norm : L.k_norm;
    const float x = src[d];
    vals[d] = __fmul_rn(x, x);
    __syncthreads();
    if (d == 0) {
        float s = 0.0f;
        for (uint32_t i = 0; i < hd; ++i) s = __fadd_rn(s, vals[i]);
        s_scale = 1.0f / sqrtf(s / static_cast<float>(hd) + a.rms_eps);
    }
    __syncthreads();
    const float nv = __fmul_rn(__fmul_rn(x, s_scale), nw[d]);
    __syncthreads();
    vals[d] = nv;
    __syncthreads();
    const float* cs = a.rope_table + static_cast<uint64_t>(pos) * hd;  // cos [half], sin [half]
    float r;
    if (d < half) {
        r = __fsub_rn(__fmul_rn(vals[d], cs[d]), __fmul_rn(vals[d + half], cs[half + d]));
    } else {
        const uint32_t i = d - half;
        r = __fadd_rn(__fmul_rn(vals[d], cs[i]), __fmul_rn(vals[i], cs[half + i]));
    }
    if (is_q) {
        src[d] = r;
    } else {
        L.kcache[(static_cast<uint64_t>(slot) * a.kv_heads + (h - a.heads)) * hd + d] =
            __half_as_ushort(__float2half_rn(r));
    }
}

// Attention of one q head: serial scores, max, exp, serial denominator,
// out[d] = ((0 + p0 v0[d]) + p1 v1[d]) + ... in position order.
__global__ __launch_bounds__(256) void k_ref_attention(ModelArgs a, ModelLayer L) {
    extern __shared__ float sc[];  // [capacity]
    __shared__ float qv[256];
    __shared__ float s_max, s_den;
    const uint32_t h = blockIdx.x, tid = threadIdx.x, hd = a.head_dim;
    const uint32_t kvh = h / (a.heads / a.kv_heads);
    const uint32_t pos = a.state[0];
    const uint32_t n = pos + 1u < a.capacity ? pos + 1u : a.capacity;
    const uint32_t first = pos + 1u - n;
    for (uint32_t d = tid; d < hd; d += blockDim.x) qv[d] = a.q[h * hd + d];
    __syncthreads();
    for (uint32_t i = tid; i < n; i += blockDim.x) {
        const uint32_t slot = (first + i) % a.capacity;
        const uint16_t* kr = L.kcache + (static_cast<uint64_t>(slot) * a.kv_heads + kvh) * hd;
        float s = 0.0f;
        for (uint32_t d = 0; d < hd; ++d)
            s = __fadd_rn(s, __fmul_rn(qv[d], __half2float(__ushort_as_half(kr[d]))));
        sc[i] = __fmul_rn(s, a.attn_scale);
    }
    __syncthreads();
    if (tid == 0) {
        float m = -INFINITY;
        for (uint32_t i = 0; i < n; ++i) m = fmaxf(m, sc[i]);
        s_max = m;
    }
    __syncthreads();
    for (uint32_t i = tid; i < n; i += blockDim.x) sc[i] = expf_libm(__fsub_rn(sc[i], s_max), a.expf_bucket, a.expf_pairs);
    __syncthreads();
    if (tid == 0) {
        float den = 0.0f;
        for (uint32_t i = 0; i < n; ++i) den = __fadd_rn(den, sc[i]);
        s_den = den;
    }
    __syncthreads();
    const float den = s_den;
    for (uint32_t d = tid; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t slot = (first + i) % a.capacity;
            const float v = __half2float(__ushort_as_half(
                L.vcache[(static_cast<uint64_t>(slot) * a.kv_heads + kvh) * hd + d]));
            o = __fadd_rn(o, __fmul_rn(__fdiv_rn(sc[i], den), v));
        }
        a.att[h * hd + d] = o;
    }
}

// route_experts over the serial FP32 logits: FP64 denominator in expert
// order, stable top-k by (logit desc, id asc), FP32 probabilities, FP32
// renormalisation.  One thread.  Non-finite logits flag the status word.
__global__ void k_ref_routes(const float* logits, uint32_t E, uint32_t K, uint32_t normalize,
                             uint32_t* ids, float* probs, uint32_t* status) {
    if (threadIdx.x != 0) return;
    float mx = logits[0];
    bool bad = false;
    for (uint32_t e = 0; e < E; ++e) {
        bad = bad || !isfinite(logits[e]);
        if (logits[e] > mx) mx = logits[e];
    }
    if (bad || !isfinite(mx)) {
        atomicOr(status, 1u);
        for (uint32_t r = 0; r < K; ++r) {
            ids[r] = 0u;  // keep the expert reads in bounds; the error is reported
            probs[r] = 0.0f;
        }
        return;
    }
    double den = 0.0;
    for (uint32_t e = 0; e < E; ++e) den += exp(static_cast<double>(__fsub_rn(logits[e], mx)));
    uint32_t sel[kMaxRefTopK];
    uint32_t n = 0;
    for (uint32_t e = 0; e < E; ++e) {
        const float l = logits[e];
        uint32_t at = n;  // lower_bound: first place whose entry is not before e
        for (uint32_t j = 0; j < n; ++j) {
            const float lj = logits[sel[j]];
            if (!(lj > l || (lj == l && sel[j] < e))) {
                at = j;
                break;
            }
        }
        if (n < K) {
            for (uint32_t j = n; j > at; --j) sel[j] = sel[j - 1];
            sel[at] = e;
            ++n;
        } else if (at < n) {
            for (uint32_t j = n - 1; j > at; --j) sel[j] = sel[j - 1];
            sel[at] = e;
        }
    }
    float p[kMaxRefTopK];
    float sum = 0.0f;
    for (uint32_t r = 0; r < K; ++r) {
        p[r] = static_cast<float>(exp(static_cast<double>(__fsub_rn(logits[sel[r]], mx))) / den);
        sum = __fadd_rn(sum, p[r]);
    }
    for (uint32_t r = 0; r < K; ++r) {
        ids[r] = sel[r];
        probs[r] = normalize ? __fdiv_rn(p[r], sum) : p[r];
    }
}

// act = (g / (1 + expf(-g))) * u for every route (src/qwen3_moe_runner.cpp:682-684).
__global__ __launch_bounds__(256) void k_ref_swiglu(const float* g, const float* u, float* act,
                                                    uint32_t n, const uint32_t* expf_bucket,
                                                    const uint32_t* expf_pairs) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float e = expf_libm(-g[i], expf_bucket, expf_pairs);
    act[i] = __fmul_rn(__fdiv_rn(g[i], __fadd_rn(1.0f, e)), u[i]);
}

// moe[i] = ((0 + p0 o0[i]) + p1 o1[i]) + ... in route order.
__global__ __launch_bounds__(256) void k_ref_combine(const float* out, const float* probs,
                                                     uint32_t K, uint32_t H, float* moe) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= H) return;
    float y = 0.0f;
    for (uint32_t r = 0; r < K; ++r)
        y = __fadd_rn(y, __fmul_rn(probs[r], out[static_cast<uint64_t>(r) * H + i]));
    moe[i] = y;
}

template <int T>
hipError_t ref_matvec_t(const RefMatvecArgs& a, uint32_t routes, hipStream_t s) {
    constexpr uint32_t BE = RefBlock<T>::BE;
    const uint32_t nb = a.in / BE, rpw = 256u / nb;
    const size_t lds = (a.in + 256u) * sizeof(float);
    hipLaunchKernelGGL(k_ref_matvec<T>, dim3((a.rows + rpw - 1u) / rpw, routes), dim3(256), lds, s, a);
    return hipGetLastError();
}

}  // namespace

bool ref_matvec_supported(uint32_t type, uint32_t in) {
    switch (type) {
        case T_F32: return in >= 1u && in <= kMaxRefWidth;
        case T_Q4_K: case T_Q5_K: case T_Q6_K:
            return in % 256u == 0u && in <= kMaxRefWidth && in / 256u <= 256u;
        case T_Q8_0: case T_Q4_0: return in % 32u == 0u && in <= kMaxRefWidth && in / 32u <= 256u;
        default: return false;
    }
}

hipError_t launch_ref_matvec(uint32_t type, const RefMatvecArgs& a, uint32_t routes, hipStream_t s) {
    switch (type) {
        case T_F32: {
            hipLaunchKernelGGL(k_ref_linear_f32, dim3((a.rows + 255u) / 256u, routes), dim3(256),
                               a.in * sizeof(float), s, a);
            return hipGetLastError();
        }
        case T_Q4_K: return ref_matvec_t<T_Q4_K>(a, routes, s);
        case T_Q5_K: return ref_matvec_t<T_Q5_K>(a, routes, s);
        case T_Q6_K: return ref_matvec_t<T_Q6_K>(a, routes, s);
        case T_Q8_0: return ref_matvec_t<T_Q8_0>(a, routes, s);
        case T_Q4_0: return ref_matvec_t<T_Q4_0>(a, routes, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_ref_rmsnorm(float* x, const float* delta, const float* w, float* out, uint32_t n,
                              uint32_t rows, float eps, hipStream_t s) {
    hipLaunchKernelGGL(k_ref_rmsnorm, dim3(rows), dim3(256), n * sizeof(float), s, x, delta, w, out,
                       n, eps);
    return hipGetLastError();
}

hipError_t launch_ref_layer_attention(const ModelArgs& a, const ModelLayer& L, hipStream_t s) {
    hipLaunchKernelGGL(k_ref_qk_rope_kv, dim3(a.heads + 2u * a.kv_heads), dim3(a.head_dim), 0, s, a,
                       L);
    hipLaunchKernelGGL(k_ref_attention, dim3(a.heads), dim3(256), a.capacity * sizeof(float), s, a, L);
    return hipGetLastError();
}

hipError_t launch_ref_moe(const ModelArgs& a, const ModelLayer& L, hipStream_t s) {
    const MoeDecodeArgs& m = L.moe;
    RefMatvecArgs r{};
    // router logits into the act buffer's tail (free until the gate/up rows)
    float* logits = a.ref_scratch;
    float* g = logits + kMaxExperts256;
    float* u = g + static_cast<uint64_t>(m.top_k) * m.ffn;
    float* act = u + static_cast<uint64_t>(m.top_k) * m.ffn;
    float* out = act + static_cast<uint64_t>(m.top_k) * m.ffn;
    r.W = reinterpret_cast<const uint8_t*>(m.router);
    r.row_bytes = static_cast<uint64_t>(m.hidden) * 4u;
    r.rows = m.n_experts;
    r.in = m.hidden;
    r.x = m.x;
    r.y = logits;
    hipError_t err = launch_ref_matvec(T_F32, r, 1, s);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_ref_routes, dim3(1), dim3(64), 0, s, logits, m.n_experts, m.top_k,
                       m.normalize, m.ids, m.probs, m.status);
    // gate / up of every selected expert
    RefMatvecArgs e{};
    e.ids = m.ids;
    e.rows = m.ffn;
    e.in = m.hidden;
    e.x = m.x;
    e.x_stride = 0;
    e.y_stride = m.ffn;
    e.W = m.gate;
    e.row_bytes = m.gate_row;
    e.slice_bytes = m.gate_slice;
    e.y = g;
    if ((err = launch_ref_matvec(m.gate_type, e, m.top_k, s))) return err;
    e.W = m.up;
    e.row_bytes = m.up_row;
    e.slice_bytes = m.up_slice;
    e.y = u;
    if ((err = launch_ref_matvec(m.up_type, e, m.top_k, s))) return err;
    const uint32_t n = m.top_k * m.ffn;
    hipLaunchKernelGGL(k_ref_swiglu, dim3((n + 255u) / 256u), dim3(256), 0, s, g, u, act, n,
                       a.expf_bucket, a.expf_pairs);
    RefMatvecArgs d{};
    d.ids = m.ids;
    d.W = m.down;
    d.row_bytes = m.down_row;
    d.slice_bytes = m.down_slice;
    d.rows = m.hidden;
    d.in = m.ffn;
    d.x = act;
    d.x_stride = m.ffn;
    d.y = out;
    d.y_stride = m.hidden;
    if ((err = launch_ref_matvec(m.down_type, d, m.top_k, s))) return err;
    hipLaunchKernelGGL(k_ref_combine, dim3((m.hidden + 255u) / 256u), dim3(256), 0, s, out, m.probs,
                       m.top_k, m.hidden, m.y);
    return hipGetLastError();
}

}  // namespace pk
