// layout.hpp -- how quantized GGUF tensors sit in HBM.
//
// GGUF stores a row as a run of encoded blocks (src/gguf_reader.cpp:21-57 of
// the reference).  Blocks of 144 (Q4_K), 176 (Q5_K), 20 (Q4_1), 24 (Q5_1) and
// 84 (Q2_K) bytes keep 4- or 16-byte alignment and stay in that form.  Blocks
// of 18 (Q4_0), 34 (Q8_0), 210 (Q6_K), 22 (Q5_0) and 110 (Q3_K) bytes only
// keep 2-byte alignment: fetching their fields takes one extra dword per
// field, a byte realignment, and byte or half-word loads for the scales.
// Those types are stored "planar" instead: within each slice (a plain matrix,
// or one expert of an expert tensor) every field of every block is moved to
// its own plane,
//
//     plane f = [slice blocks][size_f],  at  slice + nblk * cum_f,
//
// in the order of the table below (largest field first), so every quant field
// starts on a 16-byte boundary and every scale field on a 2- or 4-byte one.
// The byte count is unchanged, and so is each field's content; only the
// position of the fields moves.  Expert slices of planar types start on
// kSlicePitchAlign boundaries (the padding sits between slices).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pk {

constexpr uint64_t kSlicePitchAlign = 256;

// Field f of a planar type: its offset in the GGUF block and its size.
struct FieldSpec {
    uint16_t src, size;
};

template <int T>
struct Planar {
    static constexpr bool kPlanar = false;
};
// Q4_0 (linear_quantized, src/quantized_linear.cpp:387-423): d, qs[16]
template <>
struct Planar<2> {
    static constexpr bool kPlanar = true;
    static constexpr int NF = 2;
    static constexpr FieldSpec F[NF] = {{2, 16}, {0, 2}};
    enum { QS = 0, D = 16 };  // cumulative offsets
};
// Q8_0 (same): d, qs[32]
template <>
struct Planar<8> {
    static constexpr bool kPlanar = true;
    static constexpr int NF = 2;
    static constexpr FieldSpec F[NF] = {{2, 32}, {0, 2}};
    enum { QS = 0, D = 32 };
};
// Q6_K (decode_q6_k, :330-358): ql[128], qh[64], scales[16], d
template <>
struct Planar<14> {
    static constexpr bool kPlanar = true;
    static constexpr int NF = 4;
    static constexpr FieldSpec F[NF] = {{0, 128}, {128, 64}, {192, 16}, {208, 2}};
    enum { QL = 0, QH = 128, SC = 192, D = 208 };
};
// Q5_0 (decode_q5_0, :64-77): d, qh[4], qs[16]
template <>
struct Planar<6> {
    static constexpr bool kPlanar = true;
    static constexpr int NF = 3;
    static constexpr FieldSpec F[NF] = {{6, 16}, {2, 4}, {0, 2}};
    enum { QS = 0, QH = 16, D = 20 };
};
// Q3_K (decode_q3_k, :123-164): hmask[32], qs[64], scales[12], d
template <>
struct Planar<11> {
    static constexpr bool kPlanar = true;
    static constexpr int NF = 4;
    static constexpr FieldSpec F[NF] = {{32, 64}, {0, 32}, {96, 12}, {108, 2}};
    enum { QS = 0, HM = 64, SC = 96, D = 108 };
};

// Host-side: whether `type` is stored planar, and its field table.
inline bool planar_type(uint32_t type) {
    return type == 2 || type == 8 || type == 14 || type == 6 || type == 11;
}

// A row of a resident weight as the kernels address it: the slice it lives
// in, the slice's block count (planar types locate their planes with it) and
// the row's first block.  Block i of the slice is GGUF block i, whichever
// form it is stored in.
struct QRow {
    const uint8_t* slice;
    uint64_t nblk;
    uint64_t blk0;
};

// Start of block i (GGUF-form types).
template <int BB>
__device__ __forceinline__ const uint8_t* block_ptr(const QRow& r, uint64_t b) {
    return r.slice + (r.blk0 + b) * BB;
}

// Field of block b of the row (planar types): CUM is the field's cumulative
// offset (Planar<T>::QS ...), SIZE its size.
template <uint32_t CUM, uint32_t SIZE>
__device__ __forceinline__ const uint8_t* field_ptr(const QRow& r, uint64_t b) {
    return r.slice + r.nblk * CUM + (r.blk0 + b) * SIZE;
}

// Moves `slices` slices of GGUF-form blocks (src, src_pitch bytes apart) into
// planar form (dst, dst_pitch bytes apart), nblk blocks per slice.
hipError_t launch_to_planar(uint32_t type, const uint8_t* src, uint64_t src_pitch, uint8_t* dst,
                            uint64_t dst_pitch, uint64_t nblk, uint32_t slices,
                            hipStream_t stream);
// The reverse (reading a weight back in its GGUF encoding).
hipError_t launch_from_planar(uint32_t type, const uint8_t* src, uint64_t src_pitch, uint8_t* dst,
                              uint64_t dst_pitch, uint64_t nblk, uint32_t slices,
                              hipStream_t stream);

}  // namespace pk
