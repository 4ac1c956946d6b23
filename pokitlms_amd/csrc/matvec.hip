// matvec.hip -- decode-time GGUF matrix-vector products on gfx950.
//
// Replaces the CPU row loop of tensor_linear (src/tensor_linear.cpp:232-263 of
// the reference) and its per-format kernels linear_k / linear_quantized /
// linear (src/quantized_linear.cpp:360-423, src/linear.cpp:10-31).
//
// Work layout: a lane owns a fixed set of units (see kquant.hpp) of every
// row and keeps their activations in registers; a wave streams whole rows
// (or 64/G rows at once when a row has G < 64 units) with coalesced 4..16-byte
// loads, reduces with cross-lane shuffles, and lane 0 of the row writes y.
// When one wave cannot hold a row's activations (large batch or wide rows),
// S waves of the workgroup split the row's units (K-split) and combine their
// partial sums through LDS in a fixed order.
#include "kquant.hpp"
#include "launch.hpp"

namespace pk {
namespace {

constexpr int kMaxS = 12;  // waves per K-split group

// Row passes whose loads a wave keeps in flight, and the workgroup bound: a
// batch above 4 holds 64 activation floats per lane, so it keeps one pass in
// flight and may split a row over up to 12 waves.
template <int B> constexpr int passes_for() { return B > 4 ? 1 : 2; }
template <int B> constexpr int max_threads_for() { return B > 4 ? 768 : 512; }

template <int T, int B, int UB, int NU, bool PIPE, int P = passes_for<B>()>
struct MvState {
    static constexpr int kPasses = P;
    static constexpr int kBufs = PIPE ? 2 : 1;
    UnitPos pos[NU];
    bool valid[NU];
    UnitX<T, UB, B> ux[NU];
    UnitRaw<T, UB> raw[kBufs][kPasses][NU];
    uint32_t row[kBufs][kPasses];
    bool live[kBufs][kPasses];
};

template <int I>
struct Buf {
    static constexpr int value = I;
};

// Each wave issues its first passes' weight loads, then reads its units'
// activations (kept in registers for every later row), then dots.  x is read
// from global memory (L2) by every wave (k_matvec_q_staged shares one vector
// through LDS instead).  PIPE (waves that walk many rows, such as an output
// head): two register sets, the next passes' loads issued before the current
// ones are consumed; past the last pass the extra issue re-reads the current
// rows (cache hits), so every issue is unconditional and the load counts stay
// static.  G64: every row on the 64 lanes of a wave (glog2 == 6), so the row
// sums are straight-line DPP code.
template <int T, int B, int UB, int NU, bool PIPE, bool G64 = false>
__global__ __launch_bounds__(max_threads_for<B>()) void k_matvec_q(
    const uint8_t* __restrict__ W, uint32_t nb, const float* __restrict__ x,
    uint32_t x_stride, float* __restrict__ y, uint32_t y_stride, uint32_t rows, uint32_t units,
    uint32_t slice_units, uint32_t S, uint32_t glog2) {
    extern __shared__ float partial[];  // [waves][kPasses][RPP][B] when S > 1
    constexpr int kPasses = passes_for<B>();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t waves = blockDim.x >> 6;
    const uint32_t groups = waves / S;               // independent row streams per block
    const uint32_t group = wave / S, slice = wave % S;
    if constexpr (G64) glog2 = 6u;
    const uint32_t G = 1u << glog2, RPP = 64u >> glog2;
    const uint32_t sub = lane >> glog2, ul = lane & (G - 1u);
    const uint64_t nblk = static_cast<uint64_t>(rows) * nb;
    const uint32_t passes = (rows + RPP - 1u) / RPP;
    const uint32_t stride = gridDim.x * groups * kPasses;
    uint32_t p0 = blockIdx.x * groups * kPasses;
    if (p0 >= passes) return;  // uniform per workgroup

    MvState<T, B, UB, NU, PIPE> st;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const uint32_t local = ul + G * k;
        const uint32_t u = slice * slice_units + local;
        st.valid[k] = local < slice_units && u < units;
        st.pos[k] = unit_pos<T, UB>(st.valid[k] ? u : 0u);
    }
    auto issue = [&](uint32_t pp, auto buf) {  // weight loads of passes pp + group*kPasses + q
        constexpr int bi = decltype(buf)::value;
#pragma unroll
        for (int q = 0; q < kPasses; ++q) {
            const uint32_t p = pp + group * kPasses + q;
            st.row[bi][q] = p * RPP + sub;
            st.live[bi][q] = p < passes && st.row[bi][q] < rows;
            const QRow qr{W, nblk, static_cast<uint64_t>(st.live[bi][q] ? st.row[bi][q] : 0u) * nb};
#pragma unroll
            for (int k = 0; k < NU; ++k) unit_load<T, UB>(qr, st.pos[k], st.raw[bi][q][k]);
        }
    };
    auto finish = [&](uint32_t pp, auto buf) {  // dots, reductions and stores of the issued passes
        constexpr int bi = decltype(buf)::value;
#pragma unroll
        for (int q = 0; q < kPasses; ++q) {
            float acc[B];
#pragma unroll
            for (int b = 0; b < B; ++b) acc[b] = 0.0f;
#pragma unroll
            for (int k = 0; k < NU; ++k)
                if (st.valid[k]) unit_compute<T, UB, B>(st.raw[bi][q][k], st.pos[k], st.ux[k], acc);
#pragma unroll
            for (int b = 0; b < B; ++b) acc[b] = G64 ? group_sum<64>(acc[b]) : group_sum_dyn(acc[b], G);
            if (ul == G - 1u) {
                if (S == 1) {
                    if (st.live[bi][q]) {
#pragma unroll
                        for (int b = 0; b < B; ++b) y[b * y_stride + st.row[bi][q]] = acc[b];
                    }
                } else {
#pragma unroll
                    for (int b = 0; b < B; ++b)
                        partial[((wave * kPasses + q) * RPP + sub) * B + b] = acc[b];
                }
            }
        }
        if (S > 1) {
            __syncthreads();
            // the group's first wave finalises (pass q, row sub, batch b)
            if (slice == 0) {
                for (uint32_t t = lane; t < kPasses * RPP * B; t += 64u) {
                    const uint32_t q = t / (RPP * B), rs = (t / B) % RPP, b = t % B;
                    const uint32_t p = pp + group * kPasses + q;
                    const uint32_t s_row = p * RPP + rs;
                    if (p < passes && s_row < rows) {
                        float v = 0.0f;
                        for (uint32_t s = 0; s < S; ++s)
                            v += partial[(((group * S + s) * kPasses + q) * RPP + rs) * B + b];
                        y[b * y_stride + s_row] = v;
                    }
                }
            }
            __syncthreads();
        }
    };

    issue(p0, Buf<0>{});  // the first passes' weight loads, then the activations
#pragma unroll
    for (int k = 0; k < NU; ++k) load_unit_x<T, UB, B>(x, x_stride, st.pos[k], st.valid[k], st.ux[k]);
    if constexpr (!PIPE) {
        finish(p0, Buf<0>{});
        for (p0 += stride; p0 < passes; p0 += stride) {
            issue(p0, Buf<0>{});
            finish(p0, Buf<0>{});
        }
    } else {
        for (;;) {  // uniform per workgroup; p0 < passes here
            const uint32_t pn = p0 + stride;
            issue(pn < passes ? pn : p0, Buf<1>{});
            finish(p0, Buf<0>{});
            if (pn >= passes) break;
            const uint32_t pm = pn + stride;
            issue(pm < passes ? pm : pn, Buf<0>{});
            finish(pn, Buf<1>{});
            if (pm >= passes) break;
            p0 = pm;
        }
    }
}

// ---------------------------------------------------------------------------
// Up to four vectors, every row on the 64 lanes of a wave (G = 64), and XG
// waves per K-slice in a workgroup: the workgroup stages x once in LDS instead
// of every wave reading all of it from L2 (for a 4096-wide Q4_K row and one
// vector that is 16 KB per wave against 4.6 KB of weights, and the loads'
// issue, not HBM, set the pace).  Piece q of vector b of unit slot k of lane
// l (a float4 of run q / (UB / 4)) sits at [((slice * NU + k) * B + b) * Q +
// q][l], so each LDS read of a wave is 64 consecutive float4s.  Each wave
// stages NU * B * Q / XG pieces per lane, its share of its slice's slots.
//
// The staging loads go out first, then the weight loads, then the stores to
// LDS, which wait for the staging loads alone (the memory counter is in
// order).  W and x are not __restrict__ here: loads the compiler may not take
// for invariant keep that program order around the barrier.

//
// With NORM (one vector, one slice) x is the RMSNorm of h + d instead: every
// workgroup loads h, d and the norm weights w coalesced, one float4 of each
// per thread and pass, issues its first weight loads, then sums the squares
// over the workgroup, writes (v * scale) * w into an LDS row from which the
// waves take their pieces, and workgroup 0 writes v = h + d to h_out (d null:
// v = h).  n = nb * BE elements, at most 4096, a multiple of four.

template <int T, int B, int UB, int NU, int XG, int P, bool NORM = false>
__global__ __launch_bounds__(512) void k_matvec_q_staged(
    const uint8_t* W, uint32_t nb, const float* x, float* y, uint32_t rows, uint32_t units,
    uint32_t slice_units, uint32_t S, const float* nd, const float* nw, float* h_out,
    float eps) {
    // vector b of x starts at b * nb * BE, of y at b * rows
    // staged x [S][NU][B][Q][64], with one vector its piece sums [S][NU][64][Q]
    // (batches: the LDS they would take costs occupancy), then partial
    // [waves][kPasses][B] when S > 1
    extern __shared__ xf32x4 smem[];
    constexpr bool PS = B == 1;
    constexpr int kPasses = P, Q = x_pieces<T, UB>(), QB = Q * B, XP = NU * QB / XG;
    static_assert(XP * XG == NU * QB, "pieces split evenly over the waves of a slice");
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t group = wave / S, slice = wave % S;
    const uint64_t nblk = static_cast<uint64_t>(rows) * nb;
    const uint32_t stride = gridDim.x * XG * kPasses;
    float* psum = reinterpret_cast<float*>(smem + S * NU * QB * 64u);
    float* partial = psum + (PS ? S * NU * QB * 64u : 0u);
    static_assert(!NORM || (B == 1 && XG * 64 == 512), "the norm: one vector, 512 threads");
    constexpr int kNormPasses = NORM ? 2 : 0;  // float4s of h per thread (n <= 4096)
    float* xs = partial;                       // NORM: the normed row [n] (S == 1: no partials)
    uint32_t p0 = blockIdx.x * XG * kPasses;
    if (p0 >= rows) return;  // uniform per workgroup

    MvState<T, B, UB, NU, false, P> st;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const uint32_t local = lane + 64u * k;
        const uint32_t u = slice * slice_units + local;
        st.valid[k] = local < slice_units && u < units;
        st.pos[k] = unit_pos<T, UB>(st.valid[k] ? u : 0u);
    }
    auto issue = [&](uint32_t pp) {
#pragma unroll
        for (int q = 0; q < kPasses; ++q) {
            const uint32_t row = pp + group * kPasses + q;
            st.row[0][q] = row;
            st.live[0][q] = row < rows;
            const QRow qr{W, nblk, static_cast<uint64_t>(row < rows ? row : 0u) * nb};
#pragma unroll
            for (int k = 0; k < NU; ++k) unit_load<T, UB>(qr, st.pos[k], st.raw[0][q][k]);
        }
    };
    auto finish = [&](uint32_t pp) {
#pragma unroll
        for (int q = 0; q < kPasses; ++q) {
            float acc[B];
#pragma unroll
            for (int b = 0; b < B; ++b) acc[b] = 0.0f;
#pragma unroll
            for (int k = 0; k < NU; ++k) {
                // unconditional, the absent unit's share dropped by a select:
                // a branch around the dots would let the compiler sink their
                // weight loads past the staging barrier
                float t[B];
#pragma unroll
                for (int b = 0; b < B; ++b) t[b] = 0.0f;
                unit_compute<T, UB, B>(st.raw[0][q][k], st.pos[k], st.ux[k], t);
#pragma unroll
                for (int b = 0; b < B; ++b) acc[b] += st.valid[k] ? t[b] : 0.0f;
            }
#pragma unroll
            for (int b = 0; b < B; ++b) acc[b] = group_sum<64>(acc[b]);
            if (lane == 63u) {
                if (S == 1) {
                    if (st.live[0][q]) {
#pragma unroll
                        for (int b = 0; b < B; ++b) y[b * rows + st.row[0][q]] = acc[b];
                    }
                } else {
#pragma unroll
                    for (int b = 0; b < B; ++b) partial[(wave * kPasses + q) * B + b] = acc[b];
                }
            }
        }
        if (S > 1) {
            __syncthreads();
            // the group's first wave adds the slices in order: lane (pass, vector)
            if (slice == 0 && lane < kPasses * B) {
                const uint32_t q = lane / B, b = lane % B, row = pp + group * kPasses + q;
                if (row < rows) {
                    float v = 0.0f;
                    for (uint32_t sl = 0; sl < S; ++sl) v += partial[((group * S + sl) * kPasses + q) * B + b];
                    y[b * rows + row] = v;
                }
            }
            __syncthreads();
        }
    };

    xf32x4 xv[XP];
    if constexpr (NORM) {
        const uint32_t n4 = nb * (Fmt<T>::BE / 4u);
        xf32x4 hv[kNormPasses], wv[kNormPasses];
#pragma unroll
        for (int i = 0; i < kNormPasses; ++i) {
            const uint32_t c = threadIdx.x + 512u * i, cc = c < n4 ? c : 0u;
            hv[i] = reinterpret_cast<const xf32x4*>(x)[cc];
            wv[i] = reinterpret_cast<const xf32x4*>(nw)[cc];
            if (nd) hv[i] = hv[i] + reinterpret_cast<const xf32x4*>(nd)[cc];
        }
        issue(p0);
        __builtin_amdgcn_sched_barrier(0);
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < kNormPasses; ++i) {
            if (threadIdx.x + 512u * i < n4) {
                ss += hv[i].x * hv[i].x;
                ss += hv[i].y * hv[i].y;
                ss += hv[i].z * hv[i].z;
                ss += hv[i].w * hv[i].w;
            }
        }
        ss = group_sum<64>(ss);  // the wave's sum in lane 63
        __shared__ float red[8];
        if (lane == 63u) red[wave] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) total += red[i];
        const float scale = 1.0f / sqrtf(total / static_cast<float>(4u * n4) + eps);
#pragma unroll
        for (int i = 0; i < kNormPasses; ++i) {
            const uint32_t c = threadIdx.x + 512u * i;
            if (c < n4) {
                if (blockIdx.x == 0 && h_out) reinterpret_cast<xf32x4*>(h_out)[c] = hv[i];
                reinterpret_cast<xf32x4*>(xs)[c] = (hv[i] * scale) * wv[i];
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < XP; ++j) {
            const uint32_t piece = group * XP + j, k = piece / Q, q = piece % Q;
            const uint32_t local = lane + 64u * k;
            const bool valid = local < slice_units && local < units;
            xv[j] = *reinterpret_cast<const xf32x4*>(
                xs + piece_col<T, UB>(unit_pos<T, UB>(valid ? local : 0u), q));
        }
    } else {
    // staging loads: unconditional (an absent unit reads unit 0's
    // activations, which no lane uses)
#pragma unroll
    for (int j = 0; j < XP; ++j) {
        const uint32_t piece = group * XP + j;  // (k, vector, q) of this lane's units
        const uint32_t k = piece / QB, bq = piece % QB;
        const uint32_t b = B == 1 ? 0u : bq / Q, q = B == 1 ? bq : bq % Q;
        const uint32_t local = lane + 64u * k, u = slice * slice_units + local;
        const bool valid = local < slice_units && u < units;
        const UnitPos pos = unit_pos<T, UB>(valid ? u : 0u);
        xv[j] = *reinterpret_cast<const xf32x4*>(x + b * (nb * Fmt<T>::BE) + piece_col<T, UB>(pos, q));
    }
    issue(p0);
    __builtin_amdgcn_sched_barrier(0);
    }
    // (always true: a block of its own ends at the barrier, so no
    // dequantisation of the weights is scheduled, and waited for, above it)
    if (wave < (blockDim.x >> 6)) {
#pragma unroll
        for (int j = 0; j < XP; ++j) {
            const uint32_t piece = group * XP + j;  // (k * B + b) * Q + q
            smem[(slice * (NU * QB) + piece) * 64u + lane] = xv[j];
            if constexpr (PS)
                psum[((slice * NU * B + piece / Q) * 64u + lane) * Q + piece % Q] =
                    (xv[j].x + xv[j].y) + (xv[j].z + xv[j].w);
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const xf32x4* slot = smem + (slice * NU + k) * QB * 64u + lane;
        if constexpr (PS)
            load_unit_x_staged_ps<T, UB, B>(slot, 64u, psum + ((slice * NU + k) * B * 64u + lane) * Q,
                                            st.ux[k]);
        else
            load_unit_x_staged<T, UB, B>(slot, 64u, st.ux[k]);
    }
    finish(p0);
    for (p0 += stride; p0 < rows; p0 += stride) {
        issue(p0);
        finish(p0);
    }
}

// F32 / F16 / BF16 rows (router-style matrices): one wave per row, lanes
// stride the row; activations are read from memory each row.
template <int T, int B>
__global__ __launch_bounds__(256) void k_matvec_float(
    const uint8_t* __restrict__ W, uint64_t row_bytes, const float* __restrict__ x,
    uint32_t x_stride, float* __restrict__ y, uint32_t y_stride, uint32_t rows, uint32_t in) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * (blockDim.x >> 6);
    for (uint32_t row = wave; row < rows; row += nwaves) {
        const uint8_t* rp = W + static_cast<uint64_t>(row) * row_bytes;
        float acc[B];
#pragma unroll
        for (int b = 0; b < B; ++b) acc[b] = 0.0f;
        for (uint32_t i = lane; i < in; i += 64u) {
            float w;
            if constexpr (T == T_F32) {
                w = reinterpret_cast<const float*>(rp)[i];
            } else if constexpr (T == T_F16) {
                w = half_bits_to_float(reinterpret_cast<const uint16_t*>(rp)[i]);
            } else {
                w = __builtin_bit_cast(float,
                                       static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(rp)[i]) << 16);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) acc[b] = __builtin_fmaf(w, x[b * x_stride + i], acc[b]);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float v = group_sum<64>(acc[b]);
            if (lane == 63) y[b * y_stride + row] = v;
        }
    }
}

template <int T>
constexpr int block_elems() { return Fmt<T>::BE; }

// Unit bytes per lane by batch: activations held per unit are RUNS*UB*B
// floats, kept at <= 64 by narrowing the unit as the batch grows (four-run
// formats at the 4-byte minimum hold up to 128 for batches above 4).
constexpr int unit_bytes_for(uint32_t batch, int maxub, int runs) {
    const int cap = maxub < 16 ? maxub : 16;
    if (runs <= 2) return batch <= 2 ? cap : (batch <= 4 ? 8 : 4);
    return batch <= 1 ? cap : (batch <= 2 ? 8 : 4);
}

constexpr uint32_t kMaxUnitsPerLane = 2;

struct Plan {
    uint32_t units, S, slice_units, glog2, nu, waves_per_block;
};

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }
uint32_t log2_ceil(uint32_t v) {
    uint32_t l = 0;
    while ((1u << l) < v) ++l;
    return l;
}

template <int T>
bool plan_for(uint32_t in, uint32_t batch, int ub, Plan& p) {
    const uint32_t max_s = batch > 4 ? 12u : 8u;
    using F = Fmt<T>;
    if (in == 0 || in % F::BE) return false;
    p.units = in / F::BE * (F::PRIM / ub);
    // units one lane may hold: activation floats per unit = RUNS*ub*batch
    const uint32_t per_unit = F::RUNS * ub * batch;
    uint32_t nu_cap = 64u / per_unit;
    if (nu_cap == 0) nu_cap = 1;
    if (nu_cap > kMaxUnitsPerLane) nu_cap = kMaxUnitsPerLane;
    p.S = ceil_div(p.units, 64u * nu_cap);
    if (p.S > max_s) return false;
    p.slice_units = ceil_div(p.units, p.S);
    if (p.slice_units >= 64u) {
        p.glog2 = 6;
        p.nu = ceil_div(p.slice_units, 64u);
    } else {
        p.glog2 = log2_ceil(p.slice_units);
        p.nu = 1;
    }
    p.waves_per_block = p.S >= 4 ? p.S : (4u / p.S) * p.S;
    return p.nu <= kMaxUnitsPerLane;
}

// XG row streams of P rows each per workgroup, every stream split over the
// plan's S waves; the activations (xl bytes) staged once per workgroup.
template <int T, int B, int UB, int NU, int XG, int P, bool NORM = false>
hipError_t run_staged(const Plan& pl, const uint8_t* W, uint32_t nb, uint32_t rows,
                      const float* x, float* y, uint32_t xl, hipStream_t stream,
                      const MatvecNorm* nm = nullptr) {
    const uint32_t waves = XG * pl.S;
    uint32_t blocks = ceil_div(rows, XG * P);
    const uint32_t max_blocks = 256u * 16u / waves;
    if (blocks > max_blocks) blocks = max_blocks;
    // x pieces, with one vector their sums (a float per 16-byte piece), the
    // slices' partials (with the norm: the normed row)
    const size_t lds = xl + (B == 1 ? xl / 4u : 0u) +
                       (pl.S > 1 ? static_cast<size_t>(waves) * P * B * sizeof(float) : 0) +
                       (NORM ? static_cast<size_t>(nb) * Fmt<T>::BE * sizeof(float) : 0);
    hipLaunchKernelGGL((k_matvec_q_staged<T, B, UB, NU, XG, P, NORM>), dim3(blocks),
                       dim3(64u * waves), lds, stream, W, nb, x, y, rows, pl.units, pl.slice_units,
                       pl.S, NORM ? nm->delta : nullptr, NORM ? nm->w : nullptr,
                       NORM ? nm->h_out : nullptr, NORM ? nm->eps : 0.0f);
    return hipGetLastError();
}

template <int T, int B, int UB, int NU>
hipError_t run_q(const Plan& pl, const uint8_t* W, uint32_t nb, uint32_t rows,
                 const float* x, uint32_t in, float* y, hipStream_t stream) {
    const uint32_t RPP = 64u >> pl.glog2;
    constexpr int kPasses = passes_for<B>();
    const uint32_t groups = pl.waves_per_block / pl.S;
    const uint32_t passes = ceil_div(rows, RPP);
    uint32_t blocks = ceil_div(passes, groups * kPasses);
    // up to 16 waves per CU: loads of four waves per SIMD in flight
    const uint32_t max_blocks = 256u * 16u / pl.waves_per_block;
    if (blocks > max_blocks) blocks = max_blocks;
    const size_t lds =
        pl.S > 1 ? static_cast<size_t>(pl.waves_per_block) * kPasses * RPP * B * sizeof(float) : 0;
    // the pipelined loop: one vector whose waves walk three or more passes
    // (the output head), or batches whose rows are split over eight or more
    // waves (their extra registers cost narrower splits more occupancy than
    // the overlap gains; Q2_K/Q3_K batches would spill)
    if constexpr (T != T_Q2_K && T != T_Q3_K) {
        if (passes >= 3u * blocks * groups * kPasses && (B == 1 || pl.S >= 8u)) {
            if (pl.glog2 == 6u)
                hipLaunchKernelGGL((k_matvec_q<T, B, UB, NU, true, true>), dim3(blocks),
                                   dim3(64u * pl.waves_per_block), lds, stream, W, nb, x, in, y, rows,
                                   rows, pl.units, pl.slice_units, pl.S, pl.glog2);
            else
                hipLaunchKernelGGL((k_matvec_q<T, B, UB, NU, true>), dim3(blocks),
                                   dim3(64u * pl.waves_per_block), lds, stream, W, nb, x, in, y, rows,
                                   rows, pl.units, pl.slice_units, pl.S, pl.glog2);
            return hipGetLastError();
        }
    }
    // up to four vectors (one for Q2_K/Q3_K, whose batches would spill), rows
    // on 64 lanes, two, four or eight row streams per workgroup sharing a
    // slice: the activations staged once in LDS (at most 32 KB)
    if constexpr (B == 1 || (B <= 4 && T != T_Q2_K && T != T_Q3_K)) {
        // (each wave of a slice stages the same number of pieces)
        constexpr int kPieces = NU * x_pieces<T, UB>() * B;
        const uint32_t xl = pl.S * kPieces * 64u * 16u;
        if (pl.glog2 == 6u && xl <= 32768u) {
            // one vector over one K-slice: eight one-row streams (a wave's dots
            // follow its single row's loads sooner); otherwise the plan's
            // streams, two rows each
            const bool one = B == 1 && pl.S == 1u;
            if constexpr (B == 1 && kPieces % 8 == 0) {
                if (one && groups == 4u)
                    return run_staged<T, B, UB, NU, 8, 1>(pl, W, nb, rows, x, y, xl, stream);
            }
            if constexpr (kPieces % 4 == 0) {
                if (groups == 4u)
                    return run_staged<T, B, UB, NU, 4, 2>(pl, W, nb, rows, x, y, xl, stream);
            }
            if constexpr (kPieces % 2 == 0) {
                if (groups == 2u)
                    return run_staged<T, B, UB, NU, 2, 2>(pl, W, nb, rows, x, y, xl, stream);
            }
        }
    }
    if (pl.glog2 == 6u)
        hipLaunchKernelGGL((k_matvec_q<T, B, UB, NU, false, true>), dim3(blocks),
                           dim3(64u * pl.waves_per_block), lds, stream, W, nb, x, in, y, rows, rows,
                           pl.units, pl.slice_units, pl.S, pl.glog2);
    else
        hipLaunchKernelGGL((k_matvec_q<T, B, UB, NU, false>), dim3(blocks), dim3(64u * pl.waves_per_block),
                           lds, stream, W, nb, x, in, y, rows, rows, pl.units, pl.slice_units, pl.S,
                           pl.glog2);
    return hipGetLastError();
}

template <int T, int B, int UB>
hipError_t dispatch_nu(const Plan& pl, const uint8_t* W, uint32_t nb, uint32_t rows,
                       const float* x, uint32_t in, float* y, hipStream_t s) {
    if constexpr (Fmt<T>::RUNS * UB * B > 32) {
        return run_q<T, B, UB, 1>(pl, W, nb, rows, x, in, y, s);  // plan_for caps nu at 1
    } else {
        if (pl.nu == 1) return run_q<T, B, UB, 1>(pl, W, nb, rows, x, in, y, s);
        return run_q<T, B, UB, 2>(pl, W, nb, rows, x, in, y, s);
    }
}

template <int T, int B>
hipError_t dispatch_q(const uint8_t* W, uint64_t rb, uint32_t rows, const float* x,
                      uint32_t in, float* y, hipStream_t s) {
    constexpr int UB = unit_bytes_for(B, Fmt<T>::MAXUB, Fmt<T>::RUNS);
    Plan pl;
    if (!plan_for<T>(in, B, UB, pl)) return hipErrorInvalidValue;
    (void)rb;
    return dispatch_nu<T, B, UB>(pl, W, in / Fmt<T>::BE, rows, x, in, y, s);
}

template <int T>
hipError_t dispatch_batch_q(uint32_t batch, const uint8_t* W, uint64_t rb, uint32_t rows,
                            const float* x, uint32_t in, float* y, hipStream_t s) {
    switch (batch) {
        case 1: return dispatch_q<T, 1>(W, rb, rows, x, in, y, s);
        case 2: return dispatch_q<T, 2>(W, rb, rows, x, in, y, s);
        case 3: return dispatch_q<T, 3>(W, rb, rows, x, in, y, s);
        case 4: return dispatch_q<T, 4>(W, rb, rows, x, in, y, s);
        case 5: return dispatch_q<T, 5>(W, rb, rows, x, in, y, s);
        case 6: return dispatch_q<T, 6>(W, rb, rows, x, in, y, s);
        case 7: return dispatch_q<T, 7>(W, rb, rows, x, in, y, s);
        case 8: return dispatch_q<T, 8>(W, rb, rows, x, in, y, s);
        default: return hipErrorInvalidValue;
    }
}

template <int T>
hipError_t dispatch_batch_f(uint32_t batch, const uint8_t* W, uint64_t rb, uint32_t rows,
                            const float* x, uint32_t in, float* y, hipStream_t s) {
    uint32_t blocks = ceil_div(rows, 4u);
    if (blocks > 2048u) blocks = 2048u;
#define PK_F(BB)                                                                              \
    case BB:                                                                                  \
        hipLaunchKernelGGL((k_matvec_float<T, BB>), dim3(blocks), dim3(256), 0, s, W, rb, x, \
                           in, y, rows, rows, in);                                            \
        return hipGetLastError();
    switch (batch) {
        PK_F(1) PK_F(2) PK_F(3) PK_F(4) PK_F(5) PK_F(6) PK_F(7) PK_F(8)
        default: return hipErrorInvalidValue;
    }
#undef PK_F
}

template <int T, int UB, int NU>
hipError_t run_norm(const Plan& pl, const uint8_t* W, uint32_t nb, uint32_t rows, const float* h,
                    const MatvecNorm& nm, float* y, hipStream_t s) {
    constexpr int kPieces = NU * x_pieces<T, UB>();
    if constexpr (kPieces % 8 == 0) {
        const uint32_t xl = kPieces * 64u * 16u;
        if (xl <= 32768u) return run_staged<T, 1, UB, NU, 8, 1, true>(pl, W, nb, rows, h, y, xl, s, &nm);
    }
    return hipErrorNotSupported;
}

template <int T>
hipError_t dispatch_norm(const uint8_t* W, uint32_t rows, const float* h, uint32_t in,
                         const MatvecNorm& nm, float* y, hipStream_t s) {
    constexpr int UB = unit_bytes_for(1, Fmt<T>::MAXUB, Fmt<T>::RUNS);
    Plan pl;
    if (!plan_for<T>(in, 1, UB, pl)) return hipErrorNotSupported;
    // the staged kernel's one-vector case: one K-slice, eight one-row streams
    if (pl.glog2 != 6u || pl.S != 1u || pl.waves_per_block != 4u) return hipErrorNotSupported;
    const uint32_t nb = in / Fmt<T>::BE;
    if constexpr (Fmt<T>::RUNS * UB > 32) {
        return run_norm<T, UB, 1>(pl, W, nb, rows, h, nm, y, s);
    } else {
        if (pl.nu == 1) return run_norm<T, UB, 1>(pl, W, nb, rows, h, nm, y, s);
        return run_norm<T, UB, 2>(pl, W, nb, rows, h, nm, y, s);
    }
}

template <int T>
bool supported_q(uint32_t in, uint32_t batch) {
    Plan pl;
    return plan_for<T>(in, batch, unit_bytes_for(batch, Fmt<T>::MAXUB, Fmt<T>::RUNS), pl);
}

}  // namespace

bool matvec_supported(uint32_t type, uint32_t in, uint32_t batch) {
    if (batch == 0 || batch > 8 || in == 0) return false;
    if (matvec_mfma_blocks_per_wave(type, in, batch)) return true;
    switch (type) {
        case T_F32: case T_F16: case T_BF16: return true;
        case T_Q4_0: return supported_q<T_Q4_0>(in, batch);
        case T_Q4_1: return supported_q<T_Q4_1>(in, batch);
        case T_Q5_0: return supported_q<T_Q5_0>(in, batch);
        case T_Q5_1: return supported_q<T_Q5_1>(in, batch);
        case T_Q2_K: return supported_q<T_Q2_K>(in, batch);
        case T_Q3_K: return supported_q<T_Q3_K>(in, batch);
        case T_Q8_0: return supported_q<T_Q8_0>(in, batch);
        case T_Q4_K: return supported_q<T_Q4_K>(in, batch);
        case T_Q5_K: return supported_q<T_Q5_K>(in, batch);
        case T_Q6_K: return supported_q<T_Q6_K>(in, batch);
        default: return false;
    }
}

size_t matvec_partial_floats(uint32_t type, uint32_t in, uint32_t batch, uint32_t rows) {
    if (rows == 0 || !matvec_mfma_takes(type, in, batch, rows)) return 0;
    return matvec_mfma_partial_floats(type, in, batch, rows);
}

hipError_t launch_matvec(uint32_t type, const uint8_t* W, uint64_t row_bytes, uint32_t rows,
                         uint32_t in, const float* x, float* y, uint32_t batch,
                         hipStream_t stream, float* partial) {
    if (rows == 0) return hipSuccess;
    if (matvec_mfma_takes(type, in, batch, rows))
        return launch_matvec_mfma(type, W, rows, in, x, y, batch, stream, partial);
    switch (type) {
        case T_F32: return dispatch_batch_f<T_F32>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_F16: return dispatch_batch_f<T_F16>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_BF16: return dispatch_batch_f<T_BF16>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q4_0: return dispatch_batch_q<T_Q4_0>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q4_1: return dispatch_batch_q<T_Q4_1>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q5_0: return dispatch_batch_q<T_Q5_0>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q5_1: return dispatch_batch_q<T_Q5_1>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q2_K: return dispatch_batch_q<T_Q2_K>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q3_K: return dispatch_batch_q<T_Q3_K>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q8_0: return dispatch_batch_q<T_Q8_0>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q4_K: return dispatch_batch_q<T_Q4_K>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q5_K: return dispatch_batch_q<T_Q5_K>(batch, W, row_bytes, rows, x, in, y, stream);
        case T_Q6_K: return dispatch_batch_q<T_Q6_K>(batch, W, row_bytes, rows, x, in, y, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec_norm(uint32_t type, const uint8_t* W, uint32_t rows, uint32_t in,
                              const float* h, const MatvecNorm& nm, float* y,
                              hipStream_t stream) {
    if (rows == 0 || in == 0 || in % 4u || in > 4096u) return hipErrorNotSupported;
    if (nm.h_out && (nm.h_out == h || nm.h_out == nm.delta)) return hipErrorInvalidValue;
    switch (type) {
        case T_Q4_0: return dispatch_norm<T_Q4_0>(W, rows, h, in, nm, y, stream);
        case T_Q4_1: return dispatch_norm<T_Q4_1>(W, rows, h, in, nm, y, stream);
        case T_Q5_0: return dispatch_norm<T_Q5_0>(W, rows, h, in, nm, y, stream);
        case T_Q5_1: return dispatch_norm<T_Q5_1>(W, rows, h, in, nm, y, stream);
        case T_Q8_0: return dispatch_norm<T_Q8_0>(W, rows, h, in, nm, y, stream);
        case T_Q4_K: return dispatch_norm<T_Q4_K>(W, rows, h, in, nm, y, stream);
        case T_Q5_K: return dispatch_norm<T_Q5_K>(W, rows, h, in, nm, y, stream);
        case T_Q6_K: return dispatch_norm<T_Q6_K>(W, rows, h, in, nm, y, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace pk
