// IQ3_XXS dequantization and layout conversion kernels (gfx950).
#include "iq3_common.h"
#include "iq3_kernels.h"

namespace gpeed {

namespace {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}
// 2-byte aligned little-endian u32 (GGUF blocks are 98 bytes, so the words
// inside them are only 2-byte aligned).
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
    return ld_u16(p) | (ld_u16(p + 2) << 16);
}

// One thread per 8-weight group (2 grid indices, one sign index). Mirrors
// blk_iq3_xxs (quant.cpp:186-210) operation for operation; every product is
// exact in fp32, so the result is bit-identical to the CPU decode.
__global__ __launch_bounds__(256) void k_dequant_raw(const uint8_t* __restrict__ src,
                                                     float* __restrict__ dst,
                                                     unsigned long long n_groups) {
    __shared__ uint32_t grid[256];
    grid[threadIdx.x] = kIq3xxsGrid[threadIdx.x];
    __syncthreads();
    const unsigned long long gi = (unsigned long long)blockIdx.x * 256 + threadIdx.x;
    if (gi >= n_groups) return;
    const unsigned long long b = gi >> 5;
    const int ib = (int)(gi >> 2) & 7;
    const int l = (int)gi & 3;
    const uint8_t* blk = src + b * kBlockBytes;
    const float d = f16_bits_to_f32(ld_u16(blk));
    const uint32_t aux = ld_u32_a2(blk + 66 + 4 * ib);
    const uint32_t qq = ld_u16(blk + 2 + 8 * ib + 2 * l);
    const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    const uint32_t s7 = (aux >> (7 * l)) & 127u;
    const uint32_t sg = s7 | ((__builtin_popcount(s7) & 1u) << 7);
    const uint32_t g1 = grid[qq & 255u];
    const uint32_t g2 = grid[qq >> 8];
    float y[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        y[j] = db * (float)((g1 >> (8 * j)) & 255u) * (((sg >> j) & 1u) ? -1.0f : 1.0f);
        y[j + 4] = db * (float)((g2 >> (8 * j)) & 255u) * (((sg >> (j + 4)) & 1u) ? -1.0f : 1.0f);
    }
    float4* out = reinterpret_cast<float4*>(dst + gi * 8);
    out[0] = make_float4(y[0], y[1], y[2], y[3]);
    out[1] = make_float4(y[4], y[5], y[6], y[7]);
}

// One thread per (record, lane): lane n of record (tile t, block b) takes
// row 64t+n's block b (24 dwords + d, T64 order). Rows past n_rows (padding
// of the last tile) are written as zeros.
__global__ __launch_bounds__(256) void k_tile(const uint8_t* __restrict__ raw,
                                              unsigned long long n_rows, int nb,
                                              uint8_t* __restrict__ t64,
                                              unsigned long long n_items) {
    const unsigned long long u = (unsigned long long)blockIdx.x * 256 + threadIdx.x;
    if (u >= n_items) return;
    const int n = (int)(u & 63);
    const unsigned long long rec = u >> 6;
    const int b = (int)(rec % (unsigned long long)nb);
    const unsigned long long t = rec / (unsigned long long)nb;
    const unsigned long long row = t * kTileRows + n;
    uint8_t* dst = t64 + rec * kRecordBytes;
    uint32_t seq[24];
    uint32_t d = 0;
    if (row < n_rows) {
        const uint8_t* blk = raw + row * ((size_t)nb * kBlockBytes) + (size_t)b * kBlockBytes;
#pragma unroll
        for (int ib = 0; ib < 8; ++ib) {
            seq[3 * ib] = ld_u32_a2(blk + 2 + 8 * ib);
            seq[3 * ib + 1] = ld_u32_a2(blk + 2 + 8 * ib + 4);
            seq[3 * ib + 2] = aux_to_t64(ld_u32_a2(blk + 66 + 4 * ib));
        }
        d = ld_u16(blk);
    } else {
#pragma unroll
        for (int i = 0; i < 24; ++i) seq[i] = 0;
    }
#pragma unroll
    for (int i = 0; i < 6; ++i)
        *reinterpret_cast<uint4*>(dst + i * kUnitBytes + n * 16) =
            make_uint4(seq[4 * i], seq[4 * i + 1], seq[4 * i + 2], seq[4 * i + 3]);
    *reinterpret_cast<uint16_t*>(dst + kRecordDOffset + n * 2) = (uint16_t)d;
}

__global__ __launch_bounds__(256) void k_untile(const uint8_t* __restrict__ t64,
                                                unsigned long long n_rows, int nb,
                                                uint8_t* __restrict__ raw,
                                                unsigned long long n_items) {
    const unsigned long long u = (unsigned long long)blockIdx.x * 256 + threadIdx.x;
    if (u >= n_items) return;
    const int n = (int)(u & 63);
    const unsigned long long rec = u >> 6;
    const int b = (int)(rec % (unsigned long long)nb);
    const unsigned long long t = rec / (unsigned long long)nb;
    const unsigned long long row = t * kTileRows + n;
    if (row >= n_rows) return;
    const uint8_t* src = t64 + rec * kRecordBytes;
    uint32_t seq[24];
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const uint4 v = *reinterpret_cast<const uint4*>(src + i * kUnitBytes + n * 16);
        seq[4 * i] = v.x; seq[4 * i + 1] = v.y; seq[4 * i + 2] = v.z; seq[4 * i + 3] = v.w;
    }
    // 16-bit stores: the fields are 2-byte aligned inside the 98-byte block
    uint16_t* blk = reinterpret_cast<uint16_t*>(raw + row * ((size_t)nb * kBlockBytes) + (size_t)b * kBlockBytes);
    blk[0] = *reinterpret_cast<const uint16_t*>(src + kRecordDOffset + n * 2);
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
        const uint32_t q0 = seq[3 * ib], q1 = seq[3 * ib + 1], a = t64_to_aux(seq[3 * ib + 2]);
        blk[1 + 4 * ib] = (uint16_t)q0; blk[2 + 4 * ib] = (uint16_t)(q0 >> 16);
        blk[3 + 4 * ib] = (uint16_t)q1; blk[4 + 4 * ib] = (uint16_t)(q1 >> 16);
        blk[33 + 2 * ib] = (uint16_t)a; blk[34 + 2 * ib] = (uint16_t)(a >> 16);
    }
}

// Streaming read (measurement aid): workgroup i reads the i-th contiguous
// share of `bytes` once, 16 bytes per lane per load, eight loads in flight
// per lane, and folds what it read into one word (so no load is dead).
__global__ __launch_bounds__(512) void k_stream_read(const uint8_t* __restrict__ p, unsigned long long bytes,
                                                     uint32_t* __restrict__ out) {
    const unsigned long long share = (bytes / gridDim.x + 4095) & ~4095ull;
    const unsigned long long beg = share * blockIdx.x;
    const unsigned long long end = beg + share < bytes ? beg + share : bytes;
    uint32_t acc = 0;
    constexpr unsigned long long kStep = 512 * 16;  // bytes one load of the workgroup covers
    unsigned long long o = beg + threadIdx.x * 16ull;
    for (; o + 7 * kStep + 16 <= end; o += 8 * kStep) {  // eight unguarded loads
        uint4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const uint4*>(p + o + i * kStep);
        __builtin_amdgcn_sched_barrier(0);  // all eight loads issue before the first use
#pragma unroll
        for (int i = 0; i < 8; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    for (; o + 16 <= end; o += kStep) {  // the share's tail
        const uint4 v = *reinterpret_cast<const uint4*>(p + o);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    __shared__ uint32_t red[8];
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t a = 0;
        for (int w = 0; w < 8; ++w) a ^= red[w];
        out[blockIdx.x] = a;
    }
}

__global__ __launch_bounds__(256) void k_add(const float* __restrict__ a, const float* __restrict__ b,
                                             float* __restrict__ d, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) d[i] = a[i] + b[i];
}

// n16 16-byte words set to zero, grid-stride.
__global__ __launch_bounds__(256) void k_fill_zero(u32x4_t* __restrict__ p, unsigned long long n16) {
    const unsigned long long stride = (unsigned long long)gridDim.x * 256;
    for (unsigned long long i = (unsigned long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
        p[i] = u32x4_t{0u, 0u, 0u, 0u};
}

}  // namespace

hipError_t launch_fill_zero(void* p, size_t n, hipStream_t s) {
    const unsigned long long n16 = n / 16;
    if (n16 == 0) return hipSuccess;
    unsigned long long grid = (n16 + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)grid), dim3(256), 0, s, static_cast<u32x4_t*>(p), n16);
    return hipGetLastError();
}

hipError_t launch_stream_read(const uint8_t* p, unsigned long long bytes, uint32_t* out, int n_groups,
                              hipStream_t s) {
    if (bytes == 0 || n_groups <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_stream_read, dim3(n_groups), dim3(512), 0, s, p, bytes, out);
    return hipGetLastError();
}

hipError_t launch_dequant_raw(const uint8_t* src, float* dst, unsigned long long n, hipStream_t s) {
    const unsigned long long groups = n / 8;
    if (groups == 0) return hipSuccess;
    const unsigned long long grid = (groups + 255) / 256;
    hipLaunchKernelGGL(k_dequant_raw, dim3((unsigned)grid), dim3(256), 0, s, src, dst, groups);
    return hipGetLastError();
}

hipError_t launch_tile(const uint8_t* raw, unsigned long long n_rows, int in_dim, uint8_t* t64,
                       hipStream_t s) {
    const int nb = in_dim / kQK;
    const unsigned long long tiles = (n_rows + kTileRows - 1) / kTileRows;
    const unsigned long long items = tiles * (unsigned long long)nb * 64ull;
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(k_tile, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, raw, n_rows, nb,
                       t64, items);
    return hipGetLastError();
}

hipError_t launch_untile(const uint8_t* t64, unsigned long long n_rows, int in_dim, uint8_t* raw,
                         hipStream_t s) {
    const int nb = in_dim / kQK;
    const unsigned long long tiles = (n_rows + kTileRows - 1) / kTileRows;
    const unsigned long long items = tiles * (unsigned long long)nb * 64ull;
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(k_untile, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, t64, n_rows,
                       nb, raw, items);
    return hipGetLastError();
}

hipError_t launch_add(const float* a, const float* b, float* dst, int n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_add, dim3((n + 255) / 256), dim3(256), 0, s, a, b, dst, n);
    return hipGetLastError();
}

}  // namespace gpeed
