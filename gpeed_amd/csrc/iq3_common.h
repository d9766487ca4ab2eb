// Shared definitions for the gfx950 IQ3_XXS kernels.
//
// Source block format (GGUF, quant.cpp:186-210): 98 bytes per 256 weights,
//   [0,2)   fp16 d
//   [2,66)  qs[64]: 8-bit grid indices, two per 8-weight group
//   [66,98) 8 little-endian u32 words aux[ib], one per 32-weight sub-block:
//           bits 28..31 scale s, bits 7l..7l+6 the sign index of group l
//   w[32ib + 8l + j] = d*(0.5+s)*0.5 * grid(qs[8ib+2l+j/4])[j%4] * sign_j
//   with signs = sign index | parity << 7 (8 signs of even parity).
//
// Tiled layout "T16" (what the matvec / matmul kernels stream). It is a
// byte-for-byte bijection of the GGUF payload and the same size (98 bytes per
// 256 weights; a trailing partial tile of rows is padded to 16 rows):
//   rows are grouped in tiles of 16; the record of (tile t, block b) is 1568 B
//   at byte offset (t*nb + b)*1568, nb = in_dim/256;
//   record = [unit j=0: 64 x 12 B][unit j=1: 64 x 12 B][d: 16 x fp16]
//   12-byte unit at index L = n + 16g (row n of the tile, g = 0..3) of half j
//   belongs to sub-block ib = 4j+g of row n:
//     word0 = qs[8ib..8ib+3], word1 = qs[8ib+4..8ib+7] (bytes unchanged)
//     word2 = W, the sign/scale word, bit-sliced for the decode:
//        the signs of elements (2d, 2d+1) of group l sit at bits
//        15-k and 31-k with k = 4d + l, so (W << k) puts them on the fp16
//        sign bits of one packed pair; the position of element 7 (implied:
//        parity of the other seven) holds the scale instead, i.e. bits
//        16..19 = s.
// Lane L = n + 16g of a wavefront loads unit L of each half, which is exactly
// the B operand it feeds to v_mfma_f32_16x16x32_f16 (column n, k-slots of
// lane group g), so a record is consumed with fully coalesced 12-byte loads
// and no cross-lane traffic.
//
// Grid table (64 KiB, built by build_grid_table, kept in LDS): the 256
// codebook entries as 4 unsigned fp16 each, replicated 32 times so that lane
// L reads its own copy at byte (idx << 8) | ((L & 31) << 3): within every
// 16-lane LDS pass the lanes hit 16 distinct bank pairs whatever the indices.
#pragma once

#include <cstddef>
#include <cstdint>

#include "iq3_tables.h"

namespace gpeed {

constexpr int kQK = 256;
constexpr int kBlockBytes = 98;
constexpr int kTileRows = 16;
constexpr int kRecordBytes = kTileRows * kBlockBytes;  // 1568
constexpr int kUnitHalfBytes = 64 * 12;                // 768
constexpr int kGridTableBytes = 65536;
constexpr int kGridReplicas = 32;

inline size_t iq3_row_bytes(long long in_dim) { return (size_t)(in_dim / kQK) * kBlockBytes; }
inline size_t t16_bytes(unsigned long long n_rows, long long in_dim) {
    const unsigned long long tiles = (n_rows + kTileRows - 1) / kTileRows;
    return (size_t)tiles * (size_t)(in_dim / kQK) * kRecordBytes;
}

// Exact fp16 encoding of a small non-negative integer (< 2048).
inline uint16_t host_f16_of_small_uint(unsigned a) {
    if (a == 0) return 0;
    int e = 31 - __builtin_clz(a);  // a in [2^e, 2^(e+1))
    const unsigned man = (a << (10 - e)) & 0x3FFu;
    return (uint16_t)(((unsigned)(e + 15) << 10) | man);
}

// Host-side construction of the replicated grid table (32768 fp16 patterns).
inline void build_grid_table(uint16_t* out) {
    for (int idx = 0; idx < 256; ++idx)
        for (int r = 0; r < kGridReplicas; ++r)
            for (int j = 0; j < 4; ++j)
                out[((idx << 8) | (r << 3)) / 2 + j] =
                    host_f16_of_small_uint((kIq3xxsGrid[idx] >> (8 * j)) & 255u);
}

// T16 sign/scale word from a GGUF aux word (see the layout above).
inline uint32_t aux_to_t16(uint32_t aux) {
    uint32_t w = ((aux >> 28) & 15u) << 16;
    for (int l = 0; l < 4; ++l) {
        const uint32_t s7 = (aux >> (7 * l)) & 127u;
        for (int j = 0; j < 7; ++j) {
            const int d = j >> 1, k = 4 * d + l;
            w |= ((s7 >> j) & 1u) << ((j & 1) ? 31 - k : 15 - k);
        }
    }
    return w;
}

}  // namespace gpeed

#ifdef __HIPCC__
#include <hip/hip_runtime.h>

namespace gpeed {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t aux_to_t16_dev(uint32_t aux) {
    uint32_t w = ((aux >> 28) & 15u) << 16;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t s7 = (aux >> (7 * l)) & 127u;
#pragma unroll
        for (int j = 0; j < 7; ++j) {
            const int d = j >> 1, k = 4 * d + l;
            w |= ((s7 >> j) & 1u) << ((j & 1) ? 31 - k : 15 - k);
        }
    }
    return w;
}

__device__ __forceinline__ uint32_t t16_to_aux_dev(uint32_t w) {
    uint32_t aux = ((w >> 16) & 15u) << 28;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
#pragma unroll
        for (int j = 0; j < 7; ++j) {
            const int d = j >> 1, k = 4 * d + l;
            aux |= ((w >> ((j & 1) ? 31 - k : 15 - k)) & 1u) << (7 * l + j);
        }
    }
    return aux;
}

// The T16 sign word with the four implied signs (element 7 of each group,
// the parity of the other seven) written over the scale nibble. Group l's
// bits are exactly the positions = 3-l (mod 4), so three xor-folds give all
// four parities at once, in bits 3-l.
__device__ __forceinline__ uint32_t t16_full_signs(uint32_t w) {
    const uint32_t m = w & 0xFFF0FFFFu;
    uint32_t t = m ^ (m >> 16);
    t ^= t >> 8;
    t ^= t >> 4;
    return m | ((t & 15u) << 16);
}

// fp16 bit pattern -> fp32, integer-only (exact for every pattern, NaN
// payload kept as man << 13), following quant.cpp:130-154.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            const int lz = __builtin_clz(man) - 21;  // shifts to bring bit 10 up
            bits = sign | ((uint32_t)(113 - lz) << 23) | (((man << lz) & 0x3FFu) << 13);
        }
    } else if (ex == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    return __uint_as_float(bits);
}

}  // namespace gpeed
#endif
