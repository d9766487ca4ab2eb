// The other GGUF formats of a UD-IQ3_XXS file on the GPU (gfx950): F32, F16,
// BF16, Q8_0, Q2_K, Q3_K, Q6_K, IQ2_S, IQ3_S, IQ4_XS (and IQ3_XXS through the
// same code): dequantization and products over raw GGUF rows.
//
// The unit of work is a 32-weight sub-block: every format's scales are
// constant over 16 or 32 weights, so one lane decodes 32 weights with two
// scales at most. Each decoder mirrors the reference's block function
// (quant.cpp:165-502) operation for operation with FP contraction off, so
// every dequantized value is bit-identical to the CPU decode; the products
// then accumulate y * x in fp32 with fused multiply-adds.
//
// The codebooks (IQ2_S 1024 x 8 bytes, IQ3_S 512 x 4, IQ3_XXS 256 x 4, the
// 16 IQ4 levels) are expanded at compile time and copied into LDS by each
// workgroup.
#include "iq3_common.h"
#include "iq3_kernels.h"
#include "quant_grids.h"

#include <type_traits>

namespace gpeed {

namespace {

constexpr int kDtF32 = 0, kDtF16 = 1, kDtQ8_0 = 8, kDtQ2_K = 10, kDtQ3_K = 11, kDtQ6_K = 14, kDtIQ3_XXS = 18,
              kDtIQ3_S = 21, kDtIQ2_S = 22, kDtIQ4_XS = 23, kDtBF16 = 30;

struct Iq2sGrid { uint64_t v[1024]; };
struct Iq3sGrid { uint32_t v[512]; };
constexpr uint16_t kIq2sPacked[1024] = {GPEED_IQ2S_PACKED};
constexpr uint16_t kIq3sPacked[512] = {GPEED_IQ3S_PACKED};
constexpr uint8_t kIq2sLevel[3] = {GPEED_IQ2S_LEVELS};
constexpr int8_t kIq4nl[16] = {GPEED_IQ4NL_VALUES};

constexpr Iq2sGrid expand_iq2s() {
    Iq2sGrid g{};
    for (int i = 0; i < 1024; ++i) {
        uint64_t e = 0;
        for (int j = 0; j < 8; ++j) e |= (uint64_t)kIq2sLevel[(kIq2sPacked[i] >> (2 * j)) & 3] << (8 * j);
        g.v[i] = e;
    }
    return g;
}
constexpr Iq3sGrid expand_iq3s() {
    Iq3sGrid g{};
    for (int i = 0; i < 512; ++i) {
        uint32_t e = 0;
        for (int j = 0; j < 4; ++j) e |= (2u * ((kIq3sPacked[i] >> (3 * j)) & 7u) + 1u) << (8 * j);
        g.v[i] = e;
    }
    return g;
}
constexpr Iq2sGrid kIq2sGrid = expand_iq2s();
constexpr Iq3sGrid kIq3sGrid = expand_iq3s();

// Geometry (quant.cpp:52-114): weights per block, bytes per block. Scalar
// types are handled in 32-weight runs.
template <int DT> struct Fmt;
template <> struct Fmt<kDtF32> { static constexpr int kElems = 32, kBytes = 128; };
template <> struct Fmt<kDtF16> { static constexpr int kElems = 32, kBytes = 64; };
template <> struct Fmt<kDtBF16> { static constexpr int kElems = 32, kBytes = 64; };
template <> struct Fmt<kDtQ8_0> { static constexpr int kElems = 32, kBytes = 34; };
template <> struct Fmt<kDtQ2_K> { static constexpr int kElems = 256, kBytes = 84; };
template <> struct Fmt<kDtQ3_K> { static constexpr int kElems = 256, kBytes = 110; };
template <> struct Fmt<kDtQ6_K> { static constexpr int kElems = 256, kBytes = 210; };
template <> struct Fmt<kDtIQ3_XXS> { static constexpr int kElems = 256, kBytes = 98; };
template <> struct Fmt<kDtIQ3_S> { static constexpr int kElems = 256, kBytes = 110; };
template <> struct Fmt<kDtIQ2_S> { static constexpr int kElems = 256, kBytes = 82; };
template <> struct Fmt<kDtIQ4_XS> { static constexpr int kElems = 256, kBytes = 136; };

// Codebook copies in LDS (only the one the format uses is sized).
template <int DT>
struct Tables {
    static constexpr int kN = DT == kDtIQ2_S ? 1024 : DT == kDtIQ3_S ? 512 : DT == kDtIQ3_XXS ? 256 : 16;
    using T = typename std::conditional<DT == kDtIQ2_S, uint64_t, uint32_t>::type;
    T v[kN];
    __device__ void load(int tid, int nthreads) {
        for (int i = tid; i < kN; i += nthreads) {
            if constexpr (DT == kDtIQ2_S) v[i] = kIq2sGrid.v[i];
            else if constexpr (DT == kDtIQ3_S) v[i] = kIq3sGrid.v[i];
            else if constexpr (DT == kDtIQ3_XXS) v[i] = kIq3xxsGrid[i];
            else v[i] = (uint32_t)(int32_t)kIq4nl[i];
        }
    }
};

// Loads of block fields: blocks sit at 2-byte-aligned addresses (every
// block size is even), so wider fields are assembled from 16-bit loads.
__device__ __forceinline__ uint32_t u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ uint32_t u32a2(const uint8_t* p) { return u16(p) | (u16(p + 2) << 16); }
// 32 bytes from a 2-byte-aligned address as 8 little-endian words
__device__ __forceinline__ void bytes32(const uint8_t* p, uint32_t (&w)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = u32a2(p + 4 * i);
}
__device__ __forceinline__ uint32_t byte_of(const uint32_t (&w)[8], int i) { return (w[i >> 2] >> (8 * (i & 3))) & 255u; }

// decode32: weights 32*sb .. 32*sb+31 of the block at blk into y. Each
// formula restates the reference's block function for those weights; the
// comment gives its lines and the byte layout.
template <int DT>
__device__ __forceinline__ void decode32(const uint8_t* __restrict__ blk, int sb, const Tables<DT>& tb, float (&y)[32]) {
#pragma clang fp contract(off)
    if constexpr (DT == kDtF32) {
        // quant.cpp:528-531: a copy
        const float* f = reinterpret_cast<const float*>(blk);
#pragma unroll
        for (int i = 0; i < 32; ++i) y[i] = f[i];
    } else if constexpr (DT == kDtF16 || DT == kDtBF16) {
        // quant.cpp:532-545 (f16_to_f32 :130-154, bf16_to_f32 :156-161); the
        // hardware fp16 conversion is exact (subnormals included)
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const uint32_t h = u16(blk + 2 * i);
            y[i] = DT == kDtF16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h) : __uint_as_float(h << 16);
        }
    } else if constexpr (DT == kDtQ8_0) {
        // quant.cpp:165-184: d (fp16), 32 int8 codes; y = d * q
        const float d = f16_bits_to_f32(u16(blk));
        uint32_t w[8];
        bytes32(blk + 2, w);
#pragma unroll
        for (int i = 0; i < 32; ++i) y[i] = d * (float)(int8_t)byte_of(w, i);
    } else if constexpr (DT == kDtQ6_K) {
        // quant.cpp:212-306: ql[128] qh[64] sc[16] d. Sub-block sb: half
        // h = sb/4, quarter q = sb%4; weight l < 32 takes the low (q < 2)
        // or high nibble of ql[64h + 32(q&1) + l], bits 2q of qh[32h + l],
        // scale sc[8h + 2q + l/16]; y = (d * sc) * (v - 32).
        const int h = sb >> 2, q = sb & 3;
        const float d = f16_bits_to_f32(u16(blk + 208));
        const float ds0 = d * (float)(int8_t)u8(blk + 192 + 8 * h + 2 * q);
        const float ds1 = d * (float)(int8_t)u8(blk + 192 + 8 * h + 2 * q + 1);
        uint32_t lo[8], hi[8];
        bytes32(blk + 64 * h + 32 * (q & 1), lo);
        bytes32(blk + 128 + 32 * h, hi);
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint32_t b = byte_of(lo, l);
            const uint32_t nib = q >= 2 ? b >> 4 : b & 15u;
            const int v = (int)(nib | (((byte_of(hi, l) >> (2 * q)) & 3u) << 4)) - 32;
            y[l] = (l < 16 ? ds0 : ds1) * (float)v;
        }
    } else if constexpr (DT == kDtQ2_K) {
        // quant.cpp:309-335: scales[16] qs[64] d dmin. Sub-block sb: half
        // h = sb/4, plane j = sb%4; weight l < 32: code (qs[32h + l] >> 2j)
        // & 3, scale byte scales[8h + 2j + l/16];
        // y = (d * (sc & 15)) * code - dmin * (sc >> 4).
        const int h = sb >> 2, j = sb & 3;
        const float d = f16_bits_to_f32(u16(blk + 80));
        const float mn = f16_bits_to_f32(u16(blk + 82));
        const uint32_t s0 = u8(blk + 8 * h + 2 * j), s1 = u8(blk + 8 * h + 2 * j + 1);
        const float dl0 = d * (float)(s0 & 15u), ml0 = mn * (float)(s0 >> 4);
        const float dl1 = d * (float)(s1 & 15u), ml1 = mn * (float)(s1 >> 4);
        uint32_t w[8];
        bytes32(blk + 16 + 32 * h, w);
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const float c = (float)((byte_of(w, l) >> (2 * j)) & 3u);
            y[l] = l < 16 ? dl0 * c - ml0 : dl1 * c - ml1;
        }
    } else if constexpr (DT == kDtQ3_K) {
        // quant.cpp:337-370: hmask[32] qs[64] scales[12] d. Sub-block sb:
        // h = sb/4, j = sb%4; weight l < 32: code (qs[32h + l] >> 2j) & 3,
        // minus 4 where bit 4h + j of hmask[l] is clear; 6-bit scale k =
        // 8h + 2j + l/16 unpacked from the 12 bytes (low nibble of byte k,
        // or high nibble of byte k-8 for k >= 8; top bits from byte 8 + k%4
        // at 2*(k/4)); y = (d * (scale - 32)) * value.
        const int h = sb >> 2, j = sb & 3;
        const float d = f16_bits_to_f32(u16(blk + 108));
        float dl[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int k = 8 * h + 2 * j + s;
            const uint32_t low = k < 8 ? u8(blk + 96 + k) & 15u : u8(blk + 96 + k - 8) >> 4;
            const uint32_t top = (u8(blk + 104 + (k & 3)) >> (2 * (k >> 2))) & 3u;
            dl[s] = d * (float)((int)(int8_t)(uint8_t)(low | (top << 4)) - 32);
        }
        uint32_t w[8], m[8];
        bytes32(blk + 32 + 32 * h, w);
        bytes32(blk, m);
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const int code = (int)((byte_of(w, l) >> (2 * j)) & 3u);
            const int v = code - (((byte_of(m, l) >> (4 * h + j)) & 1u) ? 0 : 4);
            y[l] = dl[l >> 4] * (float)v;
        }
    } else if constexpr (DT == kDtIQ3_XXS) {
        // quant.cpp:186-210: d, qs[64] grid indices, 8 words of 4 x 7 sign
        // bits + 4-bit scale; the eighth sign of a group makes the parity
        // even. y = ((d * (0.5 + s)) * 0.5) * grid * sign.
        const float d = f16_bits_to_f32(u16(blk));
        const uint32_t aux = u32a2(blk + 66 + 4 * sb);
        const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t qq = u16(blk + 2 + 8 * sb + 2 * l);
            const uint32_t s7 = (aux >> (7 * l)) & 127u;
            const uint32_t sg = s7 | ((__builtin_popcount(s7) & 1u) << 7);
            const uint32_t g1 = tb.v[qq & 255u], g2 = tb.v[qq >> 8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t gv = ((e < 4 ? g1 : g2) >> (8 * (e & 3))) & 255u;
                y[8 * l + e] = db * (float)gv * (((sg >> e) & 1u) ? -1.0f : 1.0f);
            }
        }
    } else if constexpr (DT == kDtIQ2_S) {
        // quant.cpp:373-418: d, qs[32] grid low bytes, signs[32], qh[8],
        // scales[8]. Group l < 4 of sub-block sb: index qs[4sb + l] | bits
        // 2l, 2l+1 of qh[sb] as bits 8-9; scale nibble (low for l < 2) of
        // scales[sb]; y = ((d * (0.5 + s)) * 0.25) * grid * sign, sign bit e
        // of signs[4sb + l].
        const float d = f16_bits_to_f32(u16(blk));
        const uint32_t qh = u8(blk + 66 + sb), sc = u8(blk + 74 + sb);
        const float db0 = d * (0.5f + (float)(sc & 15u)) * 0.25f;
        const float db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
        const uint32_t qs = u32a2(blk + 2 + 4 * sb), sg = u32a2(blk + 34 + 4 * sb);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t idx = ((qs >> (8 * l)) & 255u) | ((qh << (8 - 2 * l)) & 0x300u);
            const uint64_t g = tb.v[idx];
            const uint32_t s = sg >> (8 * l);
            const float dl = l < 2 ? db0 : db1;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                y[8 * l + e] = dl * (float)(uint32_t)((g >> (8 * e)) & 255u) * (((s >> e) & 1u) ? -1.0f : 1.0f);
        }
    } else if constexpr (DT == kDtIQ3_S) {
        // quant.cpp:421-482: d, qs[64], qh[8], signs[32], scales[4]. Group
        // l < 4 of sub-block sb: indices qs[8sb + 2l], qs[8sb + 2l + 1] with
        // bit 8 from bits 2l and 2l+1 of qh[sb]; scale nibble of
        // scales[sb/2] (low for even sb); y = (d * (1 + 2s)) * grid * sign,
        // sign bit e of signs[4sb + l].
        const float d = f16_bits_to_f32(u16(blk));
        const uint32_t qh = u8(blk + 66 + sb);
        const uint32_t scb = u8(blk + 106 + (sb >> 1));
        const float db = d * (1.0f + 2.0f * (float)((sb & 1) ? scb >> 4 : scb & 15u));
        const uint32_t sg = u32a2(blk + 74 + 4 * sb);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t qq = u16(blk + 2 + 8 * sb + 2 * l);
            const uint32_t i1 = (qq & 255u) | ((qh << (8 - 2 * l)) & 256u);
            const uint32_t i2 = (qq >> 8) | ((qh << (7 - 2 * l)) & 256u);
            const uint32_t g1 = tb.v[i1], g2 = tb.v[i2];
            const uint32_t s = sg >> (8 * l);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t gv = ((e < 4 ? g1 : g2) >> (8 * (e & 3))) & 255u;
                y[8 * l + e] = db * (float)gv * (((s >> e) & 1u) ? -1.0f : 1.0f);
            }
        }
    } else if constexpr (DT == kDtIQ4_XS) {
        // quant.cpp:485-502: d, scales_h (u16), scales_l[4], qs[128].
        // Sub-block sb: 6-bit scale = nibble sb%2 of scales_l[sb/2] | bits
        // 2sb, 2sb+1 of scales_h << 4; weight i < 16 is the low nibble of
        // qs[16sb + i], weight 16 + i its high nibble;
        // y = (d * (ls - 32)) * level[code].
        const float d = f16_bits_to_f32(u16(blk));
        const uint32_t sh = u16(blk + 2);
        const int ls = (int)(((u8(blk + 4 + (sb >> 1)) >> (4 * (sb & 1))) & 15u) | (((sh >> (2 * sb)) & 3u) << 4));
        const float dl = d * (float)(ls - 32);
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = u32a2(blk + 8 + 16 * sb + 4 * i);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t b = (w[i >> 2] >> (8 * (i & 3))) & 255u;
            y[i] = dl * (float)(int32_t)tb.v[b & 15u];
            y[16 + i] = dl * (float)(int32_t)tb.v[b >> 4];
        }
    }
}

// Sub-blocks per block and the sub-block's block address.
template <int DT>
__device__ __forceinline__ const uint8_t* sub_block(const uint8_t* row, long long sbi, int& sb) {
    constexpr int kSub = Fmt<DT>::kElems / 32;
    sb = (int)(sbi % kSub);
    return row + (size_t)(sbi / kSub) * Fmt<DT>::kBytes;
}

// One thread per 32-weight sub-block, grid-stride; y written as 8 float4.
template <int DT>
__global__ __launch_bounds__(256) void k_dequant_rows(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                      long long n_sub) {
    __shared__ Tables<DT> tb;
    tb.load(threadIdx.x, 256);
    __syncthreads();
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n_sub; i += (long long)gridDim.x * 256) {
        int sb;
        const uint8_t* blk = sub_block<DT>(src, i, sb);
        float y[32];
        decode32<DT>(blk, sb, tb, y);
        float4* out = reinterpret_cast<float4*>(dst + i * 32);
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = make_float4(y[4 * k], y[4 * k + 1], y[4 * k + 2], y[4 * k + 3]);
    }
}

// Scalar types with any element count: one thread per element.
template <int DT>
__global__ __launch_bounds__(256) void k_dequant_scalar(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                        long long n) {
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
        if constexpr (DT == kDtF32) dst[i] = reinterpret_cast<const float*>(src)[i];
        else if constexpr (DT == kDtF16) dst[i] = (float)__builtin_bit_cast(_Float16, (uint16_t)u16(src + 2 * i));
        else dst[i] = __uint_as_float(u16(src + 2 * i) << 16);
    }
}

// Rows per wavefront and the bytes of one 64-sub-block chunk of a row.
template <int DT, int NT = 1> struct RowsCfg {
    // rows per wavefront: two for one token (more wavefronts in flight; on
    // 6144 x 6144, 12.3-16.3 us against 14.9-23.1 us with four and 21.7-24.9
    // with one), four for 2-8 tokens (each token's activations loaded once
    // serve four rows), two for F16/BF16
    static constexpr int kRW = DT == kDtF32 ? 1 : (NT == 1 || DT == kDtF16 || DT == kDtBF16) ? 2 : 4;
    static constexpr int kChunkBytes = 64 * 32 / Fmt<DT>::kElems * Fmt<DT>::kBytes;  // 64 sub-blocks
    static constexpr int kSegs = (kChunkBytes + 15) / 16 + 1;  // 16-byte segments covering it, any alignment
    static constexpr int kLoads = (kSegs + 63) / 64;           // per lane
    static constexpr int kStride = kLoads * 64 * 16;           // LDS bytes per staged row chunk
};

constexpr int kBufferDword3 = 0x00020000;

// Y[t][j] = sum_i W[j][i] * X[t][i] over raw GGUF rows (w = the first row of
// this launch's slice at byte `lead` of base[0, base_bytes), base 16-byte
// aligned; Y rows ldy apart). Each wavefront takes kRW consecutive rows
// (grid-stride) and walks them in chunks of 64 sub-blocks: a chunk of each
// row is fetched with coalesced 16-byte buffer loads (the next chunk's loads
// are in flight while this one is decoded), staged in the wavefront's LDS
// region, and lane l decodes sub-block l of it for every row, against the
// same 32 activations per token. fp32 FMA accumulation and a butterfly
// reduction per row and token. (Splitting a row group's K range over the
// workgroup's wavefronts measured no faster.)
template <int DT, int NT>
__global__ __launch_bounds__(256) void k_matmul_rows(const uint8_t* base, int base_bytes, uint32_t lead,
                                                     uint32_t row_bytes, int in_dim, int out_dim,
                                                     const float* __restrict__ X, int n_tok, float* __restrict__ Y,
                                                     int ldy) {
    using C = RowsCfg<DT, NT>;
    constexpr int RW = C::kRW, kSub = Fmt<DT>::kElems / 32, kBB = Fmt<DT>::kBytes;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), 0, base_bytes, kBufferDword3);
    __shared__ Tables<DT> tb;
    __shared__ __attribute__((aligned(16))) uint8_t stage[4][RW][C::kStride];
    tb.load(threadIdx.x, 256);
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = blockIdx.y * NT;
    const int nt = n_tok - t0 < NT ? n_tok - t0 : NT;
    const int n_sub = in_dim / 32;
    // segment loads of the chunk at sub-block sb of the rows into registers
    auto fetch = [&](int j0, int sb, u32x4_t (&seg)[RW][C::kLoads]) {
        const int cnt = n_sub - sb < 64 ? n_sub - sb : 64;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int j = j0 + r;
            const uint32_t a0 = lead + (uint32_t)j * row_bytes + (uint32_t)(sb / kSub) * kBB;
            const uint32_t a1 = a0 + (uint32_t)(cnt / kSub) * kBB;
            const uint32_t b0 = a0 & ~15u;
            const uint32_t nseg = j < out_dim ? (a1 - b0 + 15) >> 4 : 0;
#pragma unroll
            for (int k = 0; k < C::kLoads; ++k) {
                const uint32_t i = (uint32_t)(lane + 64 * k);
                const uint32_t off = i < nseg ? b0 + 16 * i : 0x80000000u;  // past the range: zeros, no access
                // non-temporal: the rows are read once
                seg[r][k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 2));
            }
        }
    };
    for (int j0 = (blockIdx.x * 4 + wave) * RW; j0 < out_dim; j0 += gridDim.x * 4 * RW) {
        float acc[RW][NT];
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[r][t] = 0.0f;
        u32x4_t seg[RW][C::kLoads];
        fetch(j0, 0, seg);
        for (int sb = 0; sb < n_sub; sb += 64) {
            // stage this chunk (the reads of the previous one came first: one
            // wavefront's LDS operations complete in order)
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int k = 0; k < C::kLoads; ++k)
                    *reinterpret_cast<u32x4_t*>(&stage[wave][r][(lane + 64 * k) * 16]) = seg[r][k];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (sb + 64 < n_sub) fetch(j0, sb + 64, seg);
            const int s = sb + lane;
            if (s < n_sub) {
                const uint32_t lead_c = (lead + (uint32_t)(sb / kSub) * kBB) & 15u;
                float xs[NT == 1 ? 32 : 1];
                if constexpr (NT == 1) {
                    const float4* xv = reinterpret_cast<const float4*>(X + (size_t)t0 * in_dim + 32 * s);
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        const float4 v = xv[k];
                        xs[4 * k] = v.x; xs[4 * k + 1] = v.y; xs[4 * k + 2] = v.z; xs[4 * k + 3] = v.w;
                    }
                }
                // the rows' chunks start (their byte addresses) mod 16 bytes into
                // their staged copies; row_bytes is even, so blocks stay 2-byte
                // aligned
                auto decode_row = [&](int r, float (&y)[32]) {
                    const uint32_t o = (lead_c + (uint32_t)(j0 + r) * row_bytes) & 15u;
                    decode32<DT>(&stage[wave][r][o + (uint32_t)((s - sb) / kSub) * kBB], s % kSub, tb, y);
                };
                if constexpr (NT == 1) {
#pragma unroll
                    for (int r = 0; r < RW; ++r) {
                        float y[32];
                        decode_row(r, y);
#pragma unroll
                        for (int e = 0; e < 32; ++e) acc[r][0] = fmaf(y[e], xs[e], acc[r][0]);
                    }
                } else {
                    // every row decoded first, then each token's 32 activations
                    // loaded once for all of them
                    float y[RW][32];
#pragma unroll
                    for (int r = 0; r < RW; ++r) decode_row(r, y[r]);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        if (t < nt) {
                            const float4* xv = reinterpret_cast<const float4*>(X + (size_t)(t0 + t) * in_dim + 32 * s);
#pragma unroll
                            for (int k = 0; k < 8; ++k) {
                                const float4 v = xv[k];
#pragma unroll
                                for (int r = 0; r < RW; ++r) {
                                    acc[r][t] = fmaf(y[r][4 * k], v.x, acc[r][t]);
                                    acc[r][t] = fmaf(y[r][4 * k + 1], v.y, acc[r][t]);
                                    acc[r][t] = fmaf(y[r][4 * k + 2], v.z, acc[r][t]);
                                    acc[r][t] = fmaf(y[r][4 * k + 3], v.w, acc[r][t]);
                                }
                            }
                        }
                    }
                }
            }
            // every lane's reads of this chunk before the next chunk's writes
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float v = acc[r][t];
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
                if (lane == 0 && t < nt && j0 + r < out_dim) Y[(size_t)(t0 + t) * ldy + j0 + r] = v;
            }
        }
    }
}

// Prefill-sized products over raw GGUF rows (every format but F32, whose
// products keep dot_f32's order): Y[t][j] = sum_i W[j][i] X[t][i]. A
// workgroup takes an RT-row x 64-token tile and walks K in chunks of 128
// columns: lane l < 4 RT decodes sub-block l % 4 of the chunk of row l / 4
// (decode32: the exact dequantization) into an fp32 LDS tile, X's chunk is
// copied beside it, and the four wavefronts multiply their share of the tile
// with fp32 MFMAs (v_mfma_f32_16x16x4f32: operands exact, fp32 accumulation
// in another order than the reference's, as in every product here). W is
// decoded once per 64 tokens instead of once per 8. Every output's sum runs
// over the same chunks and 4-column steps whatever RT is, so the tile shape
// does not change a bit.
constexpr int kRgTok = 64, kRgK = 128, kRgStride = kRgK + 4;  // (+4: conflict-free reads)

template <int DT, int RT>
__global__ __launch_bounds__(256, 2) void k_gemm_rows(const uint8_t* __restrict__ w, size_t rb, int in_dim,
                                                      int out_dim, const float* __restrict__ X, int n_tok,
                                                      float* __restrict__ Y, int ldy) {
    constexpr int kE = Fmt<DT>::kElems, kB = Fmt<DT>::kBytes;
    // wavefront grid over the tile's 16 x 16 MFMA tiles: WR x WT wavefronts,
    // each R2 row tiles x U2 token tiles
    constexpr int RM = RT / 16, WR = RM < 2 ? RM : 2, WT = 4 / WR, R2 = RM / WR, U2 = (kRgTok / 16) / WT;
    static_assert(RT == 16 || RT == 32 || RT == 64, "row tile");
    __shared__ Tables<DT> tb;
    __shared__ __attribute__((aligned(16))) float wt[RT][kRgStride];
    __shared__ __attribute__((aligned(16))) float xt[kRgTok][kRgStride];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    tb.load(tid, 256);
    const int j0 = blockIdx.x * RT, t0 = blockIdx.y * kRgTok;
    const int drow = tid >> 2, dsb = tid & 3;  // this lane's decode: row, sub-block of the chunk
    // (rows past out_dim decode the last row; tokens past n_tok copy the
    // last token: their outputs are not stored)
    const uint8_t* wrow = w + (size_t)min(j0 + min(drow, RT - 1), out_dim - 1) * rb;
    // this wavefront's share: rows qr .. qr + 16 R2 - 1, tokens qt .. qt + 16 U2 - 1
    const int qr = (wave % WR) * 16 * R2, qt = (wave / WR) * 16 * U2;
    const int li = lane & 15, lk = lane >> 4;
    float4_t acc[R2][U2];
#pragma unroll
    for (int r = 0; r < R2; ++r)
#pragma unroll
        for (int u = 0; u < U2; ++u) acc[r][u] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < in_dim; k0 += kRgK) {
        __syncthreads();  // the MFMAs of the previous chunk have read their operands
        if (drow < RT) {
            const int col = k0 + 32 * dsb;
            float y[32];
            if (col < in_dim) {
                decode32<DT>(wrow + (size_t)(col / kE) * kB, (col % kE) / 32, tb, y);
            } else {
#pragma unroll
                for (int e = 0; e < 32; ++e) y[e] = 0.0f;  // past K: zero operands
            }
            float4* dst = reinterpret_cast<float4*>(&wt[drow][32 * dsb]);
#pragma unroll
            for (int q = 0; q < 8; ++q) dst[q] = make_float4(y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = tid + 256 * i, t = idx >> 5, c4 = idx & 31;
            const int col = k0 + 4 * c4;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (col < in_dim)
                v = *reinterpret_cast<const float4*>(X + (size_t)min(t0 + t, n_tok - 1) * in_dim + col);
            *reinterpret_cast<float4*>(&xt[t][4 * c4]) = v;
        }
        __syncthreads();
        // A: W rows (lane: row li, column lk of the 4-column step); B: X
        // tokens (token li, column lk); D[row 4 lk + i][token li]
#pragma unroll 4
        for (int k = 0; k < kRgK; k += 4) {
            float a[R2], b[U2];
#pragma unroll
            for (int r = 0; r < R2; ++r) a[r] = wt[qr + 16 * r + li][k + lk];
#pragma unroll
            for (int u = 0; u < U2; ++u) b[u] = xt[qt + 16 * u + li][k + lk];
#pragma unroll
            for (int r = 0; r < R2; ++r)
#pragma unroll
                for (int u = 0; u < U2; ++u) acc[r][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], b[u], acc[r][u], 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < R2; ++r)
#pragma unroll
        for (int u = 0; u < U2; ++u) {
            const int t = t0 + qt + 16 * u + li;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = j0 + qr + 16 * r + 4 * lk + i;
                if (j < out_dim && t < n_tok) Y[(size_t)t * ldy + j] = acc[r][u][i];
            }
        }
}

template <int DT, int RT>
hipError_t gemm_rows_rt(const uint8_t* w, size_t rb, int in_dim, int out_dim, const float* X, int n_tok, float* Y,
                        hipStream_t s) {
    constexpr int kMaxTok = 65535 * kRgTok;  // token tiles per launch (grid y)
    const unsigned gx = (unsigned)((out_dim + RT - 1) / RT);
    for (int t = 0; t < n_tok; t += kMaxTok) {
        const int nt = n_tok - t < kMaxTok ? n_tok - t : kMaxTok;
        hipLaunchKernelGGL((k_gemm_rows<DT, RT>), dim3(gx, (unsigned)((nt + kRgTok - 1) / kRgTok)), dim3(256), 0, s,
                           w, rb, in_dim, out_dim, X + (size_t)t * in_dim, nt, Y + (size_t)t * out_dim, out_dim);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// The row tile: 64 rows where the tiles make 256 workgroups (one per CU of a
// 256-CU device), else 32 or 16 (more workgroups, each with fewer MFMAs:
// 6144 rows at up to 64 tokens are 96 tiles of 64 rows, 384 of 16)
template <int DT>
hipError_t gemm_rows_dt(const uint8_t* w, size_t rb, int in_dim, int out_dim, const float* X, int n_tok, float* Y,
                        hipStream_t s) {
    const long long tt = (n_tok + kRgTok - 1) / kRgTok;
    if ((long long)((out_dim + 63) / 64) * tt >= 256) return gemm_rows_rt<DT, 64>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
    if ((long long)((out_dim + 31) / 32) * tt >= 256) return gemm_rows_rt<DT, 32>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
    return gemm_rows_rt<DT, 16>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
}

template <int DT>
hipError_t dequant_dt(const uint8_t* src, float* dst, unsigned long long n, hipStream_t s) {
    if constexpr (DT == kDtF32 || DT == kDtF16 || DT == kDtBF16) {
        unsigned long long grid = (n + 255) / 256;
        if (grid > 8192) grid = 8192;
        hipLaunchKernelGGL(k_dequant_scalar<DT>, dim3((unsigned)grid), dim3(256), 0, s, src, dst, (long long)n);
    } else {
        const unsigned long long n_sub = n / 32;
        unsigned long long grid = (n_sub + 255) / 256;
        if (grid > 8192) grid = 8192;
        hipLaunchKernelGGL(k_dequant_rows<DT>, dim3((unsigned)grid), dim3(256), 0, s, src, dst, (long long)n_sub);
    }
    return hipGetLastError();
}

template <int DT, int NT>
hipError_t matmul_dt_nt(const uint8_t* w, size_t rb, int in_dim, int out_dim, const float* X, int n_tok, float* Y,
                        hipStream_t s) {
    // row slices whose bytes stay below 2 GiB (32-bit buffer offsets); at
    // most 32768 token columns per launch
    constexpr int RW = RowsCfg<DT, NT>::kRW;
    const long long max_rows = ((1ll << 31) - 64) / (long long)rb / (4 * RW) * (4 * RW);
    // rows so long that one wavefront's rows pass 2 GiB cannot be sliced
    if (max_rows < 1) return hipErrorInvalidValue;
    constexpr int kMaxTok = 32768 * NT;
    for (int j = 0; j < out_dim; j += (int)max_rows) {
        const int rows = out_dim - j < max_rows ? out_dim - j : (int)max_rows;
        const uint8_t* wj = w + (size_t)j * rb;
        const uint8_t* base = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(wj) & ~(uintptr_t)15);
        const uint32_t lead = (uint32_t)(wj - base);
        const int base_bytes = (int)(lead + (size_t)rows * rb);
        int grid = (rows + 4 * RW - 1) / (4 * RW);
        if (grid > 2048) grid = 2048;
        for (int t = 0; t < n_tok; t += kMaxTok) {
            const int nt = n_tok - t < kMaxTok ? n_tok - t : kMaxTok;
            hipLaunchKernelGGL((k_matmul_rows<DT, NT>), dim3(grid, (nt + NT - 1) / NT), dim3(256), 0, s, base, base_bytes, lead,
                               (uint32_t)rb, in_dim, rows, X + (size_t)t * in_dim, nt,
                               Y + (size_t)t * out_dim + j, out_dim);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// F32 rows (matmul_quant of an F32 tensor: the rows are copied, then
// dot_f32, weights.cpp:86-203, simd.h:12-37) in dot_f32's own order, so the
// products are bitwise the reference's: its two 8-lane AVX accumulators are
// 16 independent fma chains (chain c takes the elements i = 16k + c of the
// 16-wide steps, and chains 0..7 the one 8-wide step after them), then
// s[l] = a0[l] + a1[l], lo[l] = s[l] + s[l + 4], (lo0 + lo1) + (lo2 + lo3),
// and an fma per element of the tail. Here chain c is lane c of a 16-lane
// group and the adds are lane exchanges in the same order. This is the
// router product of moe_batch (ffn_gate_inp, model_batch.cpp:172): with its
// logits bitwise the reference's, so are the routing integers.
// Tiling: a workgroup takes RW = R NR rows x TW = TT NT tokens; lane c of
// group (rs, ts) (tid >> 4 = rs + NR ts) runs chain c of the R x TT products
// of rows rs R .. +R-1 and tokens ts TT .. +TT-1, its operands read from LDS
// (R + TT floats per column, R TT fmas). Column chunks of CH go straight from
// global memory into a ring of NB LDS buffers, NB - 1 chunks ahead of the
// sums: each row's CH columns are CH / (64 V) wavefront copies
// (global_load_lds of V dwords per lane). A buffer holds the RW rows then the
// TW token rows, each padded by 16 / R floats, so the NR row groups of a
// wavefront read four different bank quarters.
template <int R, int TT, int NR, int NT, int CH, int NB, int V>
struct DotTile {
    static constexpr int kThreads = 16 * NR * NT, kWaves = kThreads / 64;
    static constexpr int kRW = R * NR, kTW = TT * NT, kRows = kRW + kTW;
    static constexpr int kStride = CH + 16 / R;
    static constexpr int kPieces = CH / (64 * V);                  // copies per row and chunk
    static constexpr int kPerWave = kRows * kPieces / kWaves;      // copies per wavefront and chunk
    static constexpr size_t kLds = (size_t)NB * kRows * kStride * 4;  // bytes
    static_assert(CH % (64 * V) == 0 && (kRows * kPieces) % kWaves == 0, "whole copies per wavefront");
    static_assert((16 / R) % 4 == 0 || V == 1, "16-byte aligned LDS rows for 16-byte copies");
    static_assert(NB >= 2 && (NB - 2) * kPerWave <= 63, "the copies in flight fit vmcnt");
    static_assert(kLds <= 160 * 1024, "LDS");
};

// s_waitcnt vmcnt(N) (N < 64; expcnt and lgkmcnt not waited for)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int R, int TT, int NR, int NT, int CH, int NB, int V>
__global__ __launch_bounds__(16 * NR * NT) void k_dot_rows_f32(const float* __restrict__ w, int in_dim, int out_dim,
                                                               const float* __restrict__ X, int n_tok,
                                                               float* __restrict__ Y, int ldy) {
    using D = DotTile<R, TT, NR, NT, CH, NB, V>;
    constexpr int RW = D::kRW, S = D::kStride;
    __shared__ float dot_lds[NB * D::kRows * S];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = tid & 15, rs = (tid >> 4) % NR, ts = (tid >> 4) / NR;
    const int j0 = blockIdx.x * RW, t0 = blockIdx.y * D::kTW;
    const int cols = in_dim & ~15;  // the columns of the 16-wide steps
    const int nchunk = (cols + CH - 1) / CH;

    // copy q of a chunk: row q / kPieces of the buffer (rows past the matrix
    // and tokens past the batch repeat the last one), columns (q % kPieces)
    // 64 V + V lane .. + V - 1 (past the 16-wide steps: clamped; those words
    // go unused)
    auto copy = [&](int n) {
        float* buf = dot_lds + (size_t)(n % NB) * D::kRows * S;
        const int col0 = n * CH;
#pragma unroll 8
        for (int p = 0; p < D::kPerWave; ++p) {
            const int q = wave + D::kWaves * p;
            const int row = q / D::kPieces, piece = q % D::kPieces;
            const float* base = row < RW ? w + (size_t)min(j0 + row, out_dim - 1) * in_dim
                                         : X + (size_t)min(t0 + row - RW, n_tok - 1) * in_dim;
            const int col = min(col0 + piece * 64 * V + V * lane, cols - V);
            float* dst = buf + row * S + piece * 64 * V;
            if constexpr (V == 4) __builtin_amdgcn_global_load_lds(base + col, dst, 16, 0, 0);
            else __builtin_amdgcn_global_load_lds(base + col, dst, 4, 0, 0);
        }
    };

    float acc[R][TT];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int u = 0; u < TT; ++u) acc[i][u] = 0.0f;
    for (int n = 0; n < NB - 1 && n < nchunk; ++n) copy(n);
    for (int n = 0; n < nchunk; ++n) {
        // chunk n's copies are done when at most the later chunks' are in
        // flight; the barrier then also says every wavefront is done with
        // chunk n - 1, whose buffer the next copy takes
        asm volatile("" ::: "memory");
        if (n + NB - 2 < nchunk) wait_vmcnt<(NB - 2) * D::kPerWave>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (n + NB - 1 < nchunk) copy(n + NB - 1);
        const float* buf = dot_lds + (size_t)(n % NB) * D::kRows * S;
        const float* wl = buf + (rs * R) * S;
        const float* xl = buf + (RW + ts * TT) * S;
        const int len = min(CH, cols - n * CH);
#pragma unroll 4
        for (int k0 = 0; k0 < len; k0 += 16) {  // (len is a multiple of 16)
            const int k = k0 + c;
            float a[R], b[TT];
#pragma unroll
            for (int i = 0; i < R; ++i) a[i] = wl[i * S + k];
#pragma unroll
            for (int u = 0; u < TT; ++u) b[u] = xl[u * S + k];
#pragma unroll
            for (int i = 0; i < R; ++i)
#pragma unroll
                for (int u = 0; u < TT; ++u) acc[i][u] = fmaf(a[i], b[u], acc[i][u]);
        }
    }

#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int j = j0 + rs * R + i;
        const float* a = w + (size_t)min(j, out_dim - 1) * in_dim;
#pragma unroll
        for (int u = 0; u < TT; ++u) {
            const int t = t0 + ts * TT + u;
            const float* b = X + (size_t)min(t, n_tok - 1) * in_dim;
            float v = acc[i][u];
            int e = cols;
            if (e + 8 <= in_dim) {  // the 8-wide step: accumulator a0 (chains 0..7)
                if (c < 8) v = fmaf(a[e + c], b[e + c], v);
                e += 8;
            }
            // s[l] = a0[l] + a1[l]; lo[l] = s[l] + s[l + 4]; h = lo[2m] + lo[2m + 1];
            // sum = h0 + h1 (lane exchanges within the 16-lane group)
            v = v + __shfl_xor(v, 8, 16);
            v = v + __shfl_xor(v, 4, 16);
            v = v + __shfl_xor(v, 1, 16);
            v = v + __shfl_xor(v, 2, 16);
            if (c == 0 && j < out_dim && t < n_tok) {
                for (; e < in_dim; ++e) v = fmaf(a[e], b[e], v);
                Y[(size_t)t * ldy + j] = v;
            }
        }
    }
}

template <int R, int TT, int NR, int NT, int CH, int NB, int V>
hipError_t launch_dot_rows_f32(const float* w, int in_dim, int out_dim, const float* X, int n_tok, float* Y,
                               hipStream_t s) {
    using D = DotTile<R, TT, NR, NT, CH, NB, V>;
    const long long gy = (n_tok + D::kTW - 1) / D::kTW;
    if (gy > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_dot_rows_f32<R, TT, NR, NT, CH, NB, V>),
                       dim3((unsigned)((out_dim + D::kRW - 1) / D::kRW), (unsigned)gy), dim3(D::kThreads), 0, s, w,
                       in_dim, out_dim, X, n_tok, Y, out_dim);
    return hipGetLastError();
}

// 16-byte copies need 16-byte aligned rows (in_dim % 4 == 0) and bases; the
// dword copies (four times as many) prefetch one chunk ahead
template <int R, int TT, int NR, int NT, int CH, int NB>
hipError_t launch_dot_rows_f32_any(const float* w, int in_dim, int out_dim, const float* X, int n_tok, float* Y,
                                   hipStream_t s) {
    if (in_dim % 4 == 0 && ((uintptr_t)w | (uintptr_t)X) % 16 == 0)
        return launch_dot_rows_f32<R, TT, NR, NT, CH, NB, 4>(w, in_dim, out_dim, X, n_tok, Y, s);
    return launch_dot_rows_f32<R, TT, NR, NT, CH, 2, 1>(w, in_dim, out_dim, X, n_tok, Y, s);
}

template <int DT>
hipError_t matmul_dt(const uint8_t* w, size_t rb, unsigned long long row0, int in_dim, int out_dim, const float* X,
                     int n_tok, float* Y, hipStream_t s) {
    w += (size_t)row0 * rb;
    if constexpr (DT == kDtF32) {
        // 8 x 8 tiles where they make a workgroup per CU (256 CUs), else 4 x 4:
        // each workgroup streams its rows and tokens through one CU's copies
        // (about 25 GB/s each, measured), so the tile is as large as keeps
        // every CU busy
        const float* wf = reinterpret_cast<const float*>(w);
        const long long tiles8 = (long long)((out_dim + 7) / 8) * ((n_tok + 7) / 8);
        if (tiles8 >= 256) return launch_dot_rows_f32_any<2, 2, 4, 4, 256, 4>(wf, in_dim, out_dim, X, n_tok, Y, s);
        return launch_dot_rows_f32_any<1, 1, 4, 4, 1024, 3>(wf, in_dim, out_dim, X, n_tok, Y, s);
    }
    // The MFMA GEMM (W decoded once per 64 tokens) from 32 tokens for the
    // block formats and from 16 for F16/BF16; below, the 8-token slices
    // (measured on 6144 x 6144, every format: 24 tokens 129-173 us against
    // 130-149 us, 32 tokens 151-209 against 133-152; F16/BF16 8 tokens 76
    // against 122, 16 tokens 140 against 121; 512 tokens 0.5-0.6 ms against
    // 8 ms)
    if constexpr (DT != kDtF32)
        if (n_tok >= (DT == kDtF16 || DT == kDtBF16 ? 16 : 32))
            return gemm_rows_dt<DT>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
    if (n_tok == 1) return matmul_dt_nt<DT, 1>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
    if (n_tok == 2) return matmul_dt_nt<DT, 2>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
    if (n_tok <= 4) return matmul_dt_nt<DT, 4>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
    return matmul_dt_nt<DT, 8>(w, rb, in_dim, out_dim, X, n_tok, Y, s);
}

}  // namespace

int rows_block_elems(int dtype) {
    switch (dtype) {
        case kDtF32: case kDtF16: case kDtBF16: return 1;
        case kDtQ8_0: return 32;
        case kDtQ2_K: case kDtQ3_K: case kDtQ6_K: case kDtIQ3_XXS: case kDtIQ3_S: case kDtIQ2_S: case kDtIQ4_XS:
            return 256;
        default: return 0;
    }
}

size_t rows_block_bytes(int dtype) {
    switch (dtype) {
        case kDtF32: return 4;
        case kDtF16: case kDtBF16: return 2;
        case kDtQ8_0: return Fmt<kDtQ8_0>::kBytes;
        case kDtQ2_K: return Fmt<kDtQ2_K>::kBytes;
        case kDtQ3_K: return Fmt<kDtQ3_K>::kBytes;
        case kDtQ6_K: return Fmt<kDtQ6_K>::kBytes;
        case kDtIQ3_XXS: return Fmt<kDtIQ3_XXS>::kBytes;
        case kDtIQ3_S: return Fmt<kDtIQ3_S>::kBytes;
        case kDtIQ2_S: return Fmt<kDtIQ2_S>::kBytes;
        case kDtIQ4_XS: return Fmt<kDtIQ4_XS>::kBytes;
        default: return 0;
    }
}

hipError_t launch_dequant_rows(int dtype, const uint8_t* src, float* dst, unsigned long long n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    switch (dtype) {
        case kDtF32: return dequant_dt<kDtF32>(src, dst, n, s);
        case kDtF16: return dequant_dt<kDtF16>(src, dst, n, s);
        case kDtBF16: return dequant_dt<kDtBF16>(src, dst, n, s);
        case kDtQ8_0: return dequant_dt<kDtQ8_0>(src, dst, n, s);
        case kDtQ2_K: return dequant_dt<kDtQ2_K>(src, dst, n, s);
        case kDtQ3_K: return dequant_dt<kDtQ3_K>(src, dst, n, s);
        case kDtQ6_K: return dequant_dt<kDtQ6_K>(src, dst, n, s);
        case kDtIQ3_XXS: return dequant_dt<kDtIQ3_XXS>(src, dst, n, s);
        case kDtIQ3_S: return dequant_dt<kDtIQ3_S>(src, dst, n, s);
        case kDtIQ2_S: return dequant_dt<kDtIQ2_S>(src, dst, n, s);
        case kDtIQ4_XS: return dequant_dt<kDtIQ4_XS>(src, dst, n, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matmul_rows(int dtype, const uint8_t* w, size_t row_bytes, unsigned long long row0, int in_dim,
                              int out_dim, const float* X, int n_tok, float* Y, hipStream_t s) {
    if (n_tok <= 0 || out_dim <= 0) return hipSuccess;
    switch (dtype) {
        case kDtF32: return matmul_dt<kDtF32>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtF16: return matmul_dt<kDtF16>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtBF16: return matmul_dt<kDtBF16>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtQ8_0: return matmul_dt<kDtQ8_0>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtQ2_K: return matmul_dt<kDtQ2_K>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtQ3_K: return matmul_dt<kDtQ3_K>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtQ6_K: return matmul_dt<kDtQ6_K>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtIQ3_XXS: return matmul_dt<kDtIQ3_XXS>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtIQ3_S: return matmul_dt<kDtIQ3_S>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtIQ2_S: return matmul_dt<kDtIQ2_S>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        case kDtIQ4_XS: return matmul_dt<kDtIQ4_XS>(w, row_bytes, row0, in_dim, out_dim, X, n_tok, Y, s);
        default: return hipErrorInvalidValue;
    }
}

// Expanded codebook entries (host copies of the tables the kernels use).
uint64_t rows_iq2s_grid(int i) { return kIq2sGrid.v[i & 1023]; }
uint32_t rows_iq3s_grid(int i) { return kIq3sGrid.v[i & 511]; }

}  // namespace gpeed
