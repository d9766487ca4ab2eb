// Shared definitions for the gfx950 IQ3_XXS kernels.
//
// Source block format (GGUF, quant.cpp:186-210): 98 bytes per 256 weights,
//   [0,2)   fp16 d
//   [2,66)  qs[64]: 8-bit grid indices, two per 8-weight group
//   [66,98) 8 little-endian u32 words aux[ib], one per 32-weight sub-block:
//           bits 28..31 scale s, bits 7l..7l+6 the sign index of group l
//   w[32ib + 8l + j] = d*(0.5+s)*0.5 * grid(qs[8ib+2l+j/4])[j%4] * sign
//   with sign byte = sign index | parity << 7 (8 signs of even parity).
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
//     word2 = aux' : byte l describes group l of the sub-block
//        bits 0-2 = s0,s1,s2   bit 3 = t3 = s0^s1^s2^s3
//        bits 4-6 = s4,s5,s6   bit 7 = bit l of the 4-bit scale
//     (s_i = sign bit i of the group; s7 = parity of s0..s6 is implied.)
// Lane L = n + 16g of a wavefront loads unit L of each half, which is exactly
// the B operand it feeds to v_mfma_f32_16x16x32_f16 (column n, k-slots of
// lane group g), so a record is consumed with fully coalesced 12-byte loads
// and no cross-lane traffic.
//
// Signed lookup table (64 KiB, built by build_sign_table, kept in LDS):
//   entry at byte (idx << 8) | (half << 7) | (c << 3): 4 fp16 = +/-grid bytes
//   half 0 (elements 0-3 of a group): c = aux' byte bits 0-3 = (s0,s1,s2,t3),
//          signs (c0, c1, c2, c0^c1^c2^c3)
//   half 1 (elements 4-7):            c = aux' byte bits 3-6 = (t3,s4,s5,s6),
//          signs (c1, c2, c3, c0^c1^c2^c3)
// so both addresses come from one v_perm_b32 each (grid index byte -> bits
// 8-15, code byte -> bits 0-7), with the code bytes of all four groups made
// by two and one VALU ops respectively.
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
constexpr int kSignTableBytes = 65536;

inline size_t iq3_row_bytes(long long in_dim) { return (size_t)(in_dim / kQK) * kBlockBytes; }
inline size_t t16_bytes(unsigned long long n_rows, long long in_dim) {
    const unsigned long long tiles = (n_rows + kTileRows - 1) / kTileRows;
    return (size_t)tiles * (size_t)(in_dim / kQK) * kRecordBytes;
}

// Host-side construction of the 64 KiB signed table (uint16 fp16 bit patterns).
inline uint16_t host_f16_of_small_int(int v) {
    // exact fp16 encoding of an integer |v| < 2048
    if (v == 0) return 0;
    const uint16_t sgn = v < 0 ? 0x8000 : 0;
    unsigned a = (unsigned)(v < 0 ? -v : v);
    int e = 31 - __builtin_clz(a);  // a in [2^e, 2^(e+1))
    const unsigned man = (a << (10 - e)) & 0x3FFu;
    return (uint16_t)(sgn | ((unsigned)(e + 15) << 10) | man);
}

inline void build_sign_table(uint16_t* out /* 32768 entries */) {
    for (int idx = 0; idx < 256; ++idx) {
        const uint32_t g = kIq3xxsGrid[idx];
        for (int half = 0; half < 2; ++half) {
            for (int c = 0; c < 16; ++c) {
                const int c0 = c & 1, c1 = (c >> 1) & 1, c2 = (c >> 2) & 1, c3 = (c >> 3) & 1;
                const int par = c0 ^ c1 ^ c2 ^ c3;
                int sg[4];
                if (half == 0) {
                    sg[0] = c0; sg[1] = c1; sg[2] = c2; sg[3] = par;
                } else {
                    sg[0] = c1; sg[1] = c2; sg[2] = c3; sg[3] = par;
                }
                const int base = ((idx << 8) | (half << 7) | (c << 3)) / 2;
                for (int j = 0; j < 4; ++j) {
                    const int v = (int)((g >> (8 * j)) & 255u);
                    out[base + j] = host_f16_of_small_int(sg[j] ? -v : v);
                }
            }
        }
    }
}

// Sign/scale word of the tiled layout from a GGUF aux word, and back.
inline uint32_t aux_to_t16(uint32_t aux) {
    uint32_t out = 0;
    for (int l = 0; l < 4; ++l) {
        const uint32_t s7 = (aux >> (7 * l)) & 127u;
        const uint32_t t3 = (s7 ^ (s7 >> 1) ^ (s7 >> 2) ^ (s7 >> 3)) & 1u;
        const uint32_t b = (s7 & 7u) | (t3 << 3) | (((s7 >> 4) & 7u) << 4) | (((aux >> (28 + l)) & 1u) << 7);
        out |= b << (8 * l);
    }
    return out;
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
    uint32_t out = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t s7 = (aux >> (7 * l)) & 127u;
        const uint32_t t3 = (s7 ^ (s7 >> 1) ^ (s7 >> 2) ^ (s7 >> 3)) & 1u;
        const uint32_t b =
            (s7 & 7u) | (t3 << 3) | (((s7 >> 4) & 7u) << 4) | (((aux >> (28 + l)) & 1u) << 7);
        out |= b << (8 * l);
    }
    return out;
}

__device__ __forceinline__ uint32_t t16_to_aux_dev(uint32_t a) {
    uint32_t out = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t b = (a >> (8 * l)) & 255u;
        const uint32_t lo3 = b & 7u;
        const uint32_t s3 = ((b >> 3) ^ lo3 ^ (lo3 >> 1) ^ (lo3 >> 2)) & 1u;
        const uint32_t s7 = lo3 | (s3 << 3) | (((b >> 4) & 7u) << 4);
        out |= s7 << (7 * l);
        out |= ((b >> 7) & 1u) << (28 + l);
    }
    return out;
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

// 4-bit scale of a T16 sign/scale word (bit 7 of each byte).
__device__ __forceinline__ uint32_t t16_scale(uint32_t a) {
    return __builtin_amdgcn_udot4((a >> 7) & 0x01010101u, 0x08040201u, 0u, false);
}

}  // namespace gpeed
#endif
