// layout.hip -- moving quantized GGUF slices between their GGUF form and the
// planar form the kernels read (see layout.hpp).
#include "layout.hpp"

namespace pk {
namespace {

constexpr int kMaxFields = 4;

struct FieldTable {
    uint32_t nf, block_bytes;
    uint32_t src[kMaxFields], size[kMaxFields], cum[kMaxFields];
};

template <int T>
FieldTable table_of() {
    FieldTable t{};
    t.nf = Planar<T>::NF;
    uint32_t cum = 0;
    for (int f = 0; f < Planar<T>::NF; ++f) {
        t.src[f] = Planar<T>::F[f].src;
        t.size[f] = Planar<T>::F[f].size;
        t.cum[f] = cum;
        cum += Planar<T>::F[f].size;
    }
    t.block_bytes = cum;
    return t;
}

bool table_for(uint32_t type, FieldTable& t) {
    switch (type) {
        case 2: t = table_of<2>(); return true;
        case 6: t = table_of<6>(); return true;
        case 8: t = table_of<8>(); return true;
        case 11: t = table_of<11>(); return true;
        case 14: t = table_of<14>(); return true;
        default: return false;
    }
}

// One thread per (slice, block, field, half-word): every field size and
// offset is even, so each thread moves one 16-bit word.
template <bool TO_PLANAR>
__global__ __launch_bounds__(256) void k_relayout(FieldTable t, const uint8_t* __restrict__ src,
                                                  uint64_t src_pitch, uint8_t* __restrict__ dst,
                                                  uint64_t dst_pitch, uint64_t nblk,
                                                  uint32_t slices) {
    const uint32_t hw = t.block_bytes / 2u;  // half-words per block
    const uint64_t total = static_cast<uint64_t>(slices) * nblk * hw;
    for (uint64_t k = blockIdx.x * 256ull + threadIdx.x; k < total;
         k += static_cast<uint64_t>(gridDim.x) * 256u) {
        const uint64_t s = k / (nblk * hw);
        const uint64_t rem = k % (nblk * hw);
        // half-word w of the planar block order: field f, byte 2 * (w - cum_f / 2)
        const uint64_t i = rem % nblk;  // consecutive threads: consecutive blocks of one field word
        const uint32_t w = static_cast<uint32_t>(rem / nblk);
        uint32_t f = 0;
        while (f + 1u < t.nf && 2u * w >= t.cum[f + 1u]) ++f;
        const uint32_t byte = 2u * w - t.cum[f];
        const uint64_t gguf = i * t.block_bytes + t.src[f] + byte;
        const uint64_t planar = nblk * t.cum[f] + i * t.size[f] + byte;
        if constexpr (TO_PLANAR) {
            const uint16_t v = *reinterpret_cast<const uint16_t*>(src + s * src_pitch + gguf);
            *reinterpret_cast<uint16_t*>(dst + s * dst_pitch + planar) = v;
        } else {
            const uint16_t v = *reinterpret_cast<const uint16_t*>(src + s * src_pitch + planar);
            *reinterpret_cast<uint16_t*>(dst + s * dst_pitch + gguf) = v;
        }
    }
}

template <bool TO_PLANAR>
hipError_t relayout(uint32_t type, const uint8_t* src, uint64_t src_pitch, uint8_t* dst,
                    uint64_t dst_pitch, uint64_t nblk, uint32_t slices, hipStream_t stream) {
    FieldTable t;
    if (!table_for(type, t)) return hipErrorInvalidValue;
    if (nblk == 0 || slices == 0) return hipSuccess;
    const uint64_t total = static_cast<uint64_t>(slices) * nblk * (t.block_bytes / 2u);
    uint64_t blocks = (total + 255u) / 256u;
    if (blocks > 65536u) blocks = 65536u;
    hipLaunchKernelGGL(k_relayout<TO_PLANAR>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       stream, t, src, src_pitch, dst, dst_pitch, nblk, slices);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_to_planar(uint32_t type, const uint8_t* src, uint64_t src_pitch, uint8_t* dst,
                            uint64_t dst_pitch, uint64_t nblk, uint32_t slices,
                            hipStream_t stream) {
    return relayout<true>(type, src, src_pitch, dst, dst_pitch, nblk, slices, stream);
}

hipError_t launch_from_planar(uint32_t type, const uint8_t* src, uint64_t src_pitch, uint8_t* dst,
                              uint64_t dst_pitch, uint64_t nblk, uint32_t slices,
                              hipStream_t stream) {
    return relayout<false>(type, src, src_pitch, dst, dst_pitch, nblk, slices, stream);
}

}  // namespace pk
