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
// Tiled layout "T64" (what the GEMV kernels stream). It is a byte-for-byte
// bijection of the GGUF payload and the same size (98 bytes per 256 weights;
// a trailing partial tile of rows is padded to 64 rows with zero bytes):
//   rows are grouped in tiles of 64; the record of (tile t, block b) is
//   6272 B at byte offset (t*nb + b)*6272, nb = in_dim/256;
//   record = [unit u=0..5: 64 lanes x 16 B][d: 64 x fp16]
//   lane n (row n of the tile) owns a 24-dword sequence spread over the six
//   units (dwords 4u..4u+3 in unit u, at byte u*1024 + 16n). Sub-block ib
//   of the row sits at dwords 3ib..3ib+2:
//     q0 = qs[8ib..8ib+3], q1 = qs[8ib+4..8ib+7] (bytes unchanged)
//     W  = the sign/scale word. Decoded (t64_signs), it holds the 32
//          element signs: the 8 elements 8l..8l+7 of group l form four
//          pairs (elements 2c, 2c+1 for c = 0..3), and pair c of group l owns
//          bits a and a+16 with a = 4c + l (lower element at bit a), so
//          rotr(S, a + 17) puts a pair's two signs on the fp16 sign bits of
//          a packed pair. Group l's bits are 4k + l for k = 0..7, a chain
//          visiting elements 0, 2, 4, 6, 1, 3, 5, 7. W stores, at chain
//          position k < 7, the parity of the group's signs at positions
//          0..k (a prefix parity); the signs are then S = W ^ (W << 4) over
//          the 28 chain bits, and position 7 (the implied eighth sign, the
//          parity of all seven stored ones) comes out of the shift as the
//          stored parity at position 6. Bits 28..31 of W hold the scale s,
//          bit 28+l = bit l of s.
// A wavefront loads one record with six fully coalesced 16-byte loads and a
// 2-byte load; lane n then holds all 256 weights of row n for block b.
//
// Grid table (64 KiB, built in LDS by every GEMV workgroup): the 256 codebook
// entries as 4 unsigned fp16 each, replicated 32 times so that lane L reads
// its own copy at byte (idx << 8) | ((L & 31) << 3): within every 32-lane
// LDS pass the lanes hit 32 distinct bank pairs whatever the indices.
#pragma once

#include <cstddef>
#include <cstdint>

#include "iq3_tables.h"

namespace gpeed {

constexpr int kQK = 256;
constexpr int kBlockBytes = 98;
constexpr int kTileRows = 64;
constexpr int kRecordBytes = kTileRows * kBlockBytes;  // 6272
constexpr int kUnitBytes = 64 * 16;                    // 1024
constexpr int kRecordDOffset = 6 * kUnitBytes;         // 6144
constexpr int kGridTableBytes = 65536;
constexpr int kGridReplicas = 32;

inline size_t iq3_row_bytes(long long in_dim) { return (size_t)(in_dim / kQK) * kBlockBytes; }
inline size_t t64_bytes(unsigned long long n_rows, long long in_dim) {
    const unsigned long long tiles = (n_rows + kTileRows - 1) / kTileRows;
    return (size_t)tiles * (size_t)(in_dim / kQK) * kRecordBytes;
}

// Exact fp16 encoding of a small non-negative integer (< 2048).
constexpr uint16_t host_f16_of_small_uint(unsigned a) {
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

// Bit of the T64 sign word that holds the sign of element e (0..31) of a
// sub-block (e = 8l + j).
constexpr int t64_sign_bit(int e) {
    return 4 * ((e & 7) >> 1) + (e >> 3) + 16 * (e & 1);
}

// Element (within its group of 8) at chain position k of the T64 sign word.
constexpr int t64_chain_elem(int k) { return k < 4 ? 2 * k : 2 * (k - 4) + 1; }

// T64 sign/scale word from a GGUF aux word (see the layout above): prefix
// parities of each group's seven stored signs along the chain, and the scale.
__host__ __device__ inline uint32_t aux_to_t64(uint32_t aux) {
    uint32_t w = (aux >> 28) << 28;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        uint32_t p = 0;
#pragma unroll
        for (int k = 0; k < 7; ++k) {
            p ^= (aux >> (7 * l + t64_chain_elem(k))) & 1u;
            w |= p << (4 * k + l);
        }
    }
    return w;
}

// The 32 element signs of a T64 sign word at their t64_sign_bit positions,
// the implied eighth sign of each group included.
__host__ __device__ inline uint32_t t64_signs(uint32_t w) { return (w & 0x0FFFFFFFu) ^ (w << 4); }

__host__ __device__ inline uint32_t t64_to_aux(uint32_t w) {
    const uint32_t sgn = t64_signs(w);
    uint32_t aux = (w >> 28) << 28;
#pragma unroll
    for (int l = 0; l < 4; ++l)
#pragma unroll
        for (int j = 0; j < 7; ++j) aux |= ((sgn >> t64_sign_bit(8 * l + j)) & 1u) << (7 * l + j);
    return aux;
}

}  // namespace gpeed

#ifdef __HIPCC__
#include <hip/hip_runtime.h>

namespace gpeed {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// SwiGLU with the reference's clamp (model_batch.cpp:245-253):
// silu(min(g, lim)) * clamp(u, -lim, lim) as std::min and std::clamp
// compute them: min(g, lim) = lim < g ? lim : g and clamp(u, lo, hi) =
// u < lo ? lo : (hi < u ? hi : u), so a NaN g or u stays NaN (fminf and
// fmaxf would turn it into a bound).
__device__ __forceinline__ float swiglu1(float gv, float uv, float lim) {
    const float gi = lim < gv ? lim : gv;
    const float ui = uv < -lim ? -lim : (lim < uv ? lim : uv);
    return (gi / (1.0f + expf(-gi))) * ui;
}

// Maximum of m over the wavefront's 64 lanes, returned in every lane: DPP
// exchanges inside each row of 16 lanes (pairs, quads, half-row and row
// mirrors), then the four row maxima read back with v_readlane — no LDS
// round trip.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_max(float m) {
    m = fmaxf(m, dpp_f32<0xB1>(m));   // quad_perm [1, 0, 3, 2]
    m = fmaxf(m, dpp_f32<0x4E>(m));   // quad_perm [2, 3, 0, 1]
    m = fmaxf(m, dpp_f32<0x141>(m));  // row_half_mirror
    m = fmaxf(m, dpp_f32<0x140>(m));  // row_mirror
    const int b = __builtin_bit_cast(int, m);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// v << N as one v_lshlrev_b64 (the compiler splits a constant 64-bit shift
// into two 32-bit ones). The amount reaches it through an SGPR, so the shift
// stays an ordinary instruction that the compiler schedules and checks for
// hazards (a shift written as inline assembly is invisible to its MFMA
// read-after-write and write-after-read checks).
template <int N>
__device__ __forceinline__ uint64_t shl64(uint64_t v) {
    int sh;
    asm("s_mov_b32 %0, %1" : "=s"(sh) : "n"(N));
    return v << sh;
}

// Power of two that brings a maximum magnitude m into [2^13, 2^14) (0 when
// m is 0, infinite or NaN), clamped to +-120.
__device__ __forceinline__ int pow2_scale_of_max(float m) {
    int sc = 0;
    if (m > 0.0f && m < __builtin_inff()) {
        int ex;
        (void)frexpf(m, &ex);  // m in [2^(ex-1), 2^ex)
        sc = 14 - ex;
        sc = sc > 120 ? 120 : (sc < -120 ? -120 : sc);
    }
    return sc;
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
