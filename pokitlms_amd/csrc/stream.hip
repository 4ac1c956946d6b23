// stream.hip -- a plain streaming read: the measured floor of an HBM-bound
// kernel that reads a given number of bytes (no counterpart in the reference;
// the benchmark compares the MoE step against it).
#include "launch.hpp"

namespace pk {
namespace {

typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));

// Each thread keeps kLoads 16-byte loads in flight per pass; consecutive
// lanes read consecutive 16-byte pieces, so every wave load covers whole
// cache lines.
constexpr uint32_t kLoads = 4;

__global__ __launch_bounds__(256) void k_read_floor(const u32x4_v* __restrict__ src, uint64_t n16,
                                                    uint32_t* __restrict__ sink) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    uint32_t acc = 0;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * 256u * kLoads + threadIdx.x; base < n16;
         base += stride * kLoads) {
        u32x4_v v[kLoads];
#pragma unroll
        for (uint32_t k = 0; k < kLoads; ++k) {
            const uint64_t i = base + static_cast<uint64_t>(k) * 256u;
            v[k] = __builtin_nontemporal_load(src + (i < n16 ? i : n16 - 1u));
        }
#pragma unroll
        for (uint32_t k = 0; k < kLoads; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace

hipError_t launch_read_floor(const uint8_t* src, uint64_t bytes, uint32_t* sink, hipStream_t s) {
    if (!src || !sink || bytes == 0 || bytes % 16u || (reinterpret_cast<uintptr_t>(src) & 15u))
        return hipErrorInvalidValue;
    const uint64_t n16 = bytes / 16u;
    // one pass of kLoads pieces per thread covers 16 KB per workgroup; at most
    // 8 workgroups per CU of the 256
    const uint64_t want = (n16 + 256u * kLoads - 1u) / (256u * kLoads);
    const uint32_t grid = static_cast<uint32_t>(want < 2048u ? want : 2048u);
    hipLaunchKernelGGL(k_read_floor, dim3(grid), dim3(256), 0, s,
                       reinterpret_cast<const u32x4_v*>(src), n16, sink);
    return hipGetLastError();
}

}  // namespace pk
