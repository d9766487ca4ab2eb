// Device building blocks shared by the GEMV kernels over the T64 layout:
// the LDS grid table, one record's loads (weights + activation images) and
// its decode-and-multiply with v_mfma_f32_4x4x4_16b_f16.
#pragma once

#include <type_traits>

#include "iq3_common.h"

namespace gpeed {

// Compile-time loop (the MFMA broadcast block ABID is an instruction field).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Workgroup barrier that orders LDS only: outstanding global loads (the
// record ring) stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The replicated grid table, built by a workgroup of kThreads threads: the
// codebook words are fetched first (grid_words), the LDS writes done later
// (grid_table_store) so that loads issued in between stay in flight.
template <int kThreads>
struct GridWords {
    static constexpr int kPer = (1024 + kThreads - 1) / kThreads;
    uint32_t v[kPer];
};

template <int kThreads>
__device__ __forceinline__ void grid_words(GridWords<kThreads>& gw, int tid) {
#pragma unroll
    for (int i = 0; i < GridWords<kThreads>::kPer; ++i)
        gw.v[i] = kIq3xxsGrid[((tid + i * kThreads) >> 2) & 255];
}

__device__ __forceinline__ uint32_t f16_pair_of_bytes(uint32_t lo, uint32_t hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)hi) << 16);
}

// Exact fp16 bit pattern of a small non-negative integer (< 2048).
constexpr uint32_t f16_bits_of_uint(uint32_t a) {
    if (a == 0) return 0;
    int e = 0;
    while ((a >> (e + 1)) != 0) ++e;  // a in [2^e, 2^(e+1))
    return ((uint32_t)(e + 15) << 10) | ((a << (10 - e)) & 0x3FFu);
}

// Grid entry idx as two packed fp16 pairs: half 0 = values 0, 1; half 1 =
// values 2, 3.
constexpr uint32_t grid_f16_pair(int idx, int half) {
    return f16_bits_of_uint((kIq3xxsGrid[idx] >> (16 * half)) & 255u) |
           (f16_bits_of_uint((kIq3xxsGrid[idx] >> (16 * half + 8)) & 255u) << 16);
}

// The replicated grid table written from immediate operands (no memory
// loads, so no wait behind other loads): wavefront w of W writes entries
// [w*256/W, (w+1)*256/W), two per store (lanes 0-31 the even entry's 32
// replicas, lanes 32-63 the odd one's).
template <int W>
__device__ __forceinline__ void grid_table_literal(uint8_t* tbl, int wave, uint32_t lane) {
    static_assert(256 % (2 * W) == 0, "wavefront share");
    constexpr int kPer = 256 / W;
    const bool odd = lane >= 32;
    uint8_t* base = tbl + ((lane >> 5) << 8) + ((lane & 31u) << 3);
    static_for<0, W>([&](auto wc) {
        constexpr int w = decltype(wc)::value;
        if (wave == w) {
            static_for<0, kPer / 2>([&](auto ic) {
                constexpr int e0 = w * kPer + 2 * decltype(ic)::value;
                const uint32_t lo = odd ? grid_f16_pair(e0 + 1, 0) : grid_f16_pair(e0, 0);
                const uint32_t hi = odd ? grid_f16_pair(e0 + 1, 1) : grid_f16_pair(e0, 1);
                *reinterpret_cast<u32x2_t*>(base + (e0 << 8)) = u32x2_t{lo, hi};
            });
        }
    });
}

// Entry idx, replica r at byte (idx << 8) | (r << 3): 4 unsigned fp16.
template <int kThreads>
__device__ __forceinline__ void grid_table_store(uint8_t* tbl, const GridWords<kThreads>& gw, int tid) {
#pragma unroll
    for (int i = 0; i < GridWords<kThreads>::kPer; ++i) {
        const int it = tid + i * kThreads;
        if (it < 1024) {
            const int idx = it >> 2, q4 = it & 3;
            const uint32_t v = gw.v[i];
            const uint32_t h01 = f16_pair_of_bytes(v & 255u, (v >> 8) & 255u);
            const uint32_t h23 = f16_pair_of_bytes((v >> 16) & 255u, v >> 24);
            u32x4_t* dst = reinterpret_cast<u32x4_t*>(tbl + (idx << 8) + q4 * 64);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j] = u32x4_t{h01, h23, h01, h23};
        }
    }
}

// One record as a lane holds it: its row's 24 dwords and d, the NP
// activation register images (token pairs) of the record's block and, where
// the unscales come from global memory, token (lane & 7)'s unscale of the
// block (read back with v_readlane: loaded with the record, it is covered by
// the record's wait).
template <int NP>
struct Rec {
    u32x4_t u[6];
    uint32_t d;
    u32x2_t a[NP][4];
    uint32_t xs;
};

// Token t's block unscale from a record's lane-distributed copy.
template <int NP>
__device__ __forceinline__ float rec_unscale(const Rec<NP>& r, int t) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(r.xs, t));
}

// rec: the record; ab: its block's prepared activation (n_tok vectors,
// 2*NP - 1 <= n_tok <= 2*NP) in the lane-major layout of the grouped
// products: pair p at p * 2048, lane slot L (32 bytes: its 4 register
// images) at L * 32, two 16-byte loads per pair. A last pair holding one
// token stores the 32 slots of rows 0, 1 only (1 KiB); rows 2, 3 then read
// a duplicate and are never used. The loads do not depend on a branch, so
// the compiler can wait for one ring slot at a time.
template <int NP>
__device__ __forceinline__ void load_record(Rec<NP>& r, const uint8_t* rec, const uint8_t* ab,
                                            uint32_t lane, int n_tok) {
    // the record non-temporal (read once per item), so the weight stream
    // leaves the activation images in L2
#pragma unroll
    for (int i = 0; i < 6; ++i)
        r.u[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(rec + i * kUnitBytes + lane * 16u));
    r.d = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(rec + kRecordDOffset + lane * 2u));
    const uint32_t slot_half = (lane >> 2) * 2 + (lane & 1);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const bool half = (p == NP - 1) && (n_tok & 1);
        const uint8_t* src = ab + p * 2048 + (half ? slot_half : lane) * 32u;
        const u32x4_t v0 = *reinterpret_cast<const u32x4_t*>(src);
        const u32x4_t v1 = *reinterpret_cast<const u32x4_t*>(src + 16);
        r.a[p][0] = u32x2_t{v0.x, v0.y};
        r.a[p][1] = u32x2_t{v0.z, v0.w};
        r.a[p][2] = u32x2_t{v1.x, v1.y};
        r.a[p][3] = u32x2_t{v1.z, v1.w};
    }
}

// The 8 grid lookups of one sub-block (two index words, 4 bytes each).
__device__ __forceinline__ void grid_lookups(const uint8_t* tbl, uint32_t lb, uint32_t q0, uint32_t q1,
                                             u32x2_t (&g)[8]) {
    static_for<0, 8>([&](auto mc) {
        constexpr int m = decltype(mc)::value;
        const uint32_t q = m < 4 ? q0 : q1;
        constexpr uint32_t sel = 0x0C0C0000u | ((4u + (m & 3)) << 8);
        g[m] = *reinterpret_cast<const u32x2_t*>(tbl + __builtin_amdgcn_perm(q, lb, sel));  // (idx << 8) | lb
    });
}

// Sub-block ib of a record: sign word w, the 8 lookups g, products with the
// NP token-pair images a; D[p] += A_p . B over the sub-block's 32 weights.
template <int NP, int ib>
__device__ __forceinline__ void subblock_dot(uint32_t w, const u32x2_t (&g)[8], const u32x2_t (&a)[NP][4],
                                             float4_t (&D)[NP]) {
    const uint32_t sw = t64_signs(w);
    // The signs of a group's second pair sit 4 bits above those of its first
    // pair, so {sw >> 4, sw} shifted left by one 64-bit shift puts both
    // pairs' signs on bits 15 and 31 of the two halves.
    const uint64_t sw2 = ((uint64_t)(sw >> 4) << 32) | sw;
    static_for<0, 8>([&](auto mc) {
        constexpr int m = decltype(mc)::value;
        constexpr int a0 = 8 * (m & 1) + (m >> 1);  // first pair's sign bits: a0, a0 + 16
        const uint64_t rs = shl64<15 - a0>(sw2);
        const uint32_t bx = ((uint32_t)rs & 0x80008000u) | g[m].x;
        const uint32_t by = ((uint32_t)(rs >> 32) & 0x80008000u) | g[m].y;
        const half4_t B = __builtin_bit_cast(half4_t, u32x2_t{bx, by});
#pragma unroll
        for (int p = 0; p < NP; ++p)
            D[p] = __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4_t, a[p][ib >> 1]), B, D[p], 4,
                                                      8 * (ib & 1) + m, 0);
    });
}

// One record: lane n's 256 weights of row n against the NP token pairs.
// Per group of 4 weights one LDS lookup in the lane's own replica of the
// grid table (4 unsigned fp16), the signs set with a shift and a masked or,
// and one v_mfma_f32_4x4x4_16b_f16 whose A operand is broadcast (CBSZ=4)
// from block ABID of a register pair holding 16 activation slices.
// kPerImage (one vector): blk[a] += (2s+1) * partial of register image a
// (sub-blocks 2a, 2a+1); else blk[t] += (2s+1) * partial of token t
// (blk[2p+1] of a single-token last pair is meaningless). With kPipe the
// lookups of sub-block ib+1 are issued before the products of sub-block ib
// (16 more VGPRs; off for 3-4 token pairs, whose rings fill the register
// file).
template <int NP, bool kPerImage = false, bool kPipe = (NP <= 2)>
__device__ __forceinline__ void record_dot(const uint8_t* tbl, const Rec<NP>& r, uint32_t lb,
                                           float (&blk)[kPerImage ? 4 : 2 * NP]) {
    static_assert(!kPerImage || NP == 1, "per-image partials take one vector");
    const uint32_t* dw = reinterpret_cast<const uint32_t*>(&r.u[0]);
    u32x2_t g[2][8];
    if constexpr (kPipe) grid_lookups(tbl, lb, dw[0], dw[1], g[0]);
    static_for<0, 8>([&](auto ibc) {
        constexpr int ib = decltype(ibc)::value;
        if constexpr (!kPipe) grid_lookups(tbl, lb, dw[3 * ib], dw[3 * ib + 1], g[ib & 1]);
        else if constexpr (ib < 7) grid_lookups(tbl, lb, dw[3 * (ib + 1)], dw[3 * (ib + 1) + 1], g[(ib + 1) & 1]);
        const uint32_t w = dw[3 * ib + 2];
        const float sc = (float)((w >> 27) | 1u);  // 2s+1
        float4_t D[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) D[p] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
        subblock_dot<NP, ib>(w, g[ib & 1], r.a, D);
        if constexpr (kPerImage) {
            blk[ib >> 1] = fmaf(sc, D[0][0] + D[0][1], blk[ib >> 1]);
        } else {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                blk[2 * p] = fmaf(sc, D[p][0] + D[p][1], blk[2 * p]);
                blk[2 * p + 1] = fmaf(sc, D[p][2] + D[p][3], blk[2 * p + 1]);
            }
        }
    });
}

}  // namespace gpeed
