// IQ3_XXS decode matvec kernels (gfx950).
//
// k_matvec_t16: batch-1 y = W x over the T16 layout. Each wavefront streams
// records of one 16-row tile with 12-byte coalesced loads, turns every
// 8-weight group into an fp16 B operand with two LDS lookups (signed grid
// values) scaled by the exact small integer (2s+1), and feeds
// v_mfma_f32_16x16x32_f16. The activation is carried as two fp16 rows
// (x = hi + lo after a power-of-two scaling), so products are exact and the
// only rounding is fp32 accumulation. The block scale d/4 is applied once per
// 256-weight block to the MFMA accumulator.
#include "iq3_common.h"
#include "iq3_kernels.h"

namespace gpeed {

namespace {

constexpr int kMatvecWaves = 4;

// Half index of activation element k in the M=1 A-operand layout
// [block][j][l][g][hl][8]: the 16 bytes lane (16g + hl) loads for MFMA (j, l).
__device__ __forceinline__ size_t x16_index_m1(int k, int hl) {
    const int blk = k >> 8, ib = (k >> 5) & 7, j = ib >> 2, g = ib & 3, l = (k >> 3) & 3, r = k & 7;
    return ((((size_t)(blk * 2 + j) * 4 + l) * 4 + g) * 2 + hl) * 8 + r;
}

// One workgroup per token: max|v| -> power-of-two scale -> fp16 hi/lo split
// into the A-operand layout. MODE 0: v = x. MODE 1: v = SwiGLU with clamp,
// silu(min(g,lim)) * clamp(u,-lim,lim) (model.cpp:683-688,
// model_batch.cpp:245-253), with g = x and u = x2.
template <int MODE>
__global__ __launch_bounds__(256) void k_prep_x(const float* __restrict__ x,
                                                const float* __restrict__ x2, float lim,
                                                int in_dim, _Float16* __restrict__ x16,
                                                float* __restrict__ xscale) {
    __shared__ float red[256];
    const int t = blockIdx.x;
    const float* xt = x + (size_t)t * in_dim;
    const float* ut = MODE == 1 ? x2 + (size_t)t * in_dim : nullptr;
    auto value = [&](int k) -> float {
        if (MODE == 0) return xt[k];
        const float gi = fminf(xt[k], lim);
        const float ui = fminf(fmaxf(ut[k], -lim), lim);
        return (gi / (1.0f + expf(-gi))) * ui;
    };
    float m = 0.0f;
    for (int k = threadIdx.x; k < in_dim; k += 256) m = fmaxf(m, fabsf(value(k)));
    red[threadIdx.x] = m;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (threadIdx.x < w) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + w]);
        __syncthreads();
    }
    m = red[0];
    int e = 0;
    if (m > 0.0f && m < __builtin_inff()) {
        int ex;
        (void)frexpf(m, &ex);  // m in [2^(ex-1), 2^ex)
        e = 14 - ex;           // scaled max in [2^13, 2^14)
        e = e > 120 ? 120 : (e < -120 ? -120 : e);
    }
    _Float16* out = x16 + (size_t)t * ((size_t)in_dim * 2);
    for (int k = threadIdx.x; k < in_dim; k += 256) {
        const float xs = ldexpf(value(k), e);
        const _Float16 hi = (_Float16)xs;
        const _Float16 lo = (_Float16)(xs - (float)hi);
        out[x16_index_m1(k, 0)] = hi;
        out[x16_index_m1(k, 1)] = lo;
    }
    if (threadIdx.x == 0) xscale[t] = ldexpf(1.0f, -e);
}

__device__ __forceinline__ u32x2_t lds_lookup(const uint8_t* tbl, uint32_t addr) {
    return *reinterpret_cast<const u32x2_t*>(tbl + addr);
}

__device__ __forceinline__ uint32_t pk_mul_f16(uint32_t v, half2_t f) {
    half2_t h = __builtin_bit_cast(half2_t, v);
    return __builtin_bit_cast(uint32_t, h * f);
}

// B operand of group l of a unit (q0, q1 = grid index words, cb1/cb2 = code
// bytes of the four groups), scaled by f = (2s+1).
template <int L>
__device__ __forceinline__ half8_t decode_group(const uint8_t* tbl, uint32_t q0, uint32_t q1,
                                                uint32_t cb1, uint32_t cb2, half2_t f) {
    const uint32_t q = (L < 2) ? q0 : q1;
    constexpr uint32_t p1 = (2 * L) & 3, p2 = p1 + 1;
    constexpr uint32_t sel1 = 0x0C0C0000u | ((4u + p1) << 8) | (uint32_t)L;
    constexpr uint32_t sel2 = 0x0C0C0000u | ((4u + p2) << 8) | (uint32_t)L;
    const uint32_t a1 = __builtin_amdgcn_perm(q, cb1, sel1);
    const uint32_t a2 = __builtin_amdgcn_perm(q, cb2, sel2);
    const u32x2_t v1 = lds_lookup(tbl, a1);
    const u32x2_t v2 = lds_lookup(tbl, a2);
    u32x4_t r;
    r.x = pk_mul_f16(v1.x, f);
    r.y = pk_mul_f16(v1.y, f);
    r.z = pk_mul_f16(v2.x, f);
    r.w = pk_mul_f16(v2.y, f);
    return __builtin_bit_cast(half8_t, r);
}

struct Unit {
    uint32_t q0, q1, a;
};

__device__ __forceinline__ Unit load_unit(const uint8_t* p) {
    const uint32_t* u = reinterpret_cast<const uint32_t*>(p);
    return Unit{u[0], u[1], u[2]};
}

// Accumulates the 4 MFMAs of one unit into acc.
__device__ __forceinline__ float4_t unit_mfma(const uint8_t* tbl, const Unit& u, const half8_t* A,
                                              float4_t acc) {
    const uint32_t cb1 = (u.a << 3) & 0x78787878u;
    const uint32_t cb2 = (u.a & 0x78787878u) | 0x80808080u;
    const uint32_t s = t16_scale(u.a);
    const _Float16 fs = (_Float16)(float)(2u * s + 1u);
    const half2_t f = {fs, fs};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], decode_group<0>(tbl, u.q0, u.q1, cb1, cb2, f), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1], decode_group<1>(tbl, u.q0, u.q1, cb1, cb2, f), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[2], decode_group<2>(tbl, u.q0, u.q1, cb1, cb2, f), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[3], decode_group<3>(tbl, u.q0, u.q1, cb1, cb2, f), acc, 0, 0, 0);
    return acc;
}

// Workgroup = kMatvecWaves wavefronts sharing one 16-row tile; wave w takes
// a contiguous range of blocks along K; partial row sums meet in LDS.
__global__ __launch_bounds__(kMatvecWaves * 64) void k_matvec_t16(
    const uint8_t* __restrict__ w, int nb, long long tile0, int out_dim,
    const half8_t* __restrict__ x16, const float* __restrict__ xscale, float* __restrict__ y,
    const u32x4_t* __restrict__ sign_table) {
    __shared__ __attribute__((aligned(16))) uint8_t tbl[kSignTableBytes];
    __shared__ float red[kMatvecWaves][16];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int n = lane & 15, g = lane >> 4;
    const long long t = tile0 + blockIdx.x;
    const int b0 = (nb * wave) / kMatvecWaves, b1 = (nb * (wave + 1)) / kMatvecWaves;

    for (int i = tid; i < kSignTableBytes / 16; i += kMatvecWaves * 64)
        reinterpret_cast<u32x4_t*>(tbl)[i] = sign_table[i];
    __syncthreads();

    const bool a_lane = n < 2;  // rows 0 (hi) and 1 (lo) of the A operand
    const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
    float acc = 0.0f;
    const uint8_t* rec = w + ((size_t)t * nb + b0) * kRecordBytes;
    for (int b = b0; b < b1; ++b, rec += kRecordBytes) {
        const Unit u0 = load_unit(rec + lane * 12);
        const Unit u1 = load_unit(rec + kUnitHalfBytes + lane * 12);
        const uint32_t dh = *reinterpret_cast<const uint16_t*>(rec + 2 * kUnitHalfBytes + 2 * n);
        half8_t A0[4], A1[4];
        const half8_t* xb = x16 + (size_t)b * 64 + g * 2 + n;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            A0[l] = a_lane ? xb[(0 * 4 + l) * 8] : zero8;
            A1[l] = a_lane ? xb[(1 * 4 + l) * 8] : zero8;
        }
        float4_t D = {0.0f, 0.0f, 0.0f, 0.0f};
        D = unit_mfma(tbl, u0, A0, D);
        D = unit_mfma(tbl, u1, A1, D);
        const float d4 = f16_bits_to_f32(dh) * 0.25f;
        acc += d4 * (D[0] + D[1]);
    }
    if (g == 0) red[wave][n] = acc;
    __syncthreads();
    if (wave == 0 && g == 0) {
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < kMatvecWaves; ++v) s += red[v][n];
        const int row = (int)blockIdx.x * 16 + n;
        if (row < out_dim) y[row] = s * xscale[0];
    }
}

// Raw GGUF rows, one wavefront per output row, VALU decode of 32-weight
// sub-blocks (lane = sub-block), butterfly reduction.
__global__ __launch_bounds__(256) void k_matvec_raw(const uint8_t* __restrict__ w, int nb,
                                                    unsigned long long row0, int out_dim,
                                                    const float* __restrict__ x,
                                                    float* __restrict__ y) {
    __shared__ uint32_t grid[256];
    grid[threadIdx.x] = kIq3xxsGrid[threadIdx.x];
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j = blockIdx.x * 4 + wave;
    if (j >= out_dim) return;
    const size_t rb = (size_t)nb * kBlockBytes;
    const uint8_t* row = w + (row0 + (unsigned long long)j) * rb;
    float acc = 0.0f;
    for (int sb = lane; sb < nb * 8; sb += 64) {
        const int b = sb >> 3, ib = sb & 7;
        const uint8_t* blk = row + (size_t)b * kBlockBytes;
        const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
        const float d = f16_bits_to_f32(h[0]);
        const uint32_t aux = (uint32_t)h[33 + 2 * ib] | ((uint32_t)h[34 + 2 * ib] << 16);
        const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        const float4* xv = reinterpret_cast<const float4*>(x + (size_t)b * 256 + ib * 32);
        float part = 0.0f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t qq = h[1 + 4 * ib + l];
            const uint32_t s7 = (aux >> (7 * l)) & 127u;
            const uint32_t sg = s7 | ((__builtin_popcount(s7) & 1u) << 7);
            const uint32_t g1 = grid[qq & 255u], g2 = grid[qq >> 8];
            const float4 xa = xv[2 * l], xb = xv[2 * l + 1];
            const float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t gv = ((e < 4 ? g1 : g2) >> (8 * (e & 3))) & 255u;
                const float v = ((sg >> e) & 1u) ? -(float)gv : (float)gv;
                part = fmaf(v, xs[e], part);
            }
        }
        acc = fmaf(db, part, acc);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) y[j] = acc;
}

}  // namespace

size_t prep_x_bytes(int n_tok, int in_dim) {
    return (size_t)n_tok * (size_t)in_dim * 4 + 256;
}

hipError_t launch_prep_x(const float* x, int n_tok, int in_dim, uint32_t* x16, float* xscale,
                         hipStream_t s) {
    hipLaunchKernelGGL(k_prep_x<0>, dim3(n_tok), dim3(256), 0, s, x, nullptr, 0.0f, in_dim,
                       reinterpret_cast<_Float16*>(x16), xscale);
    return hipGetLastError();
}

hipError_t launch_prep_swiglu(const float* g, const float* u, float lim, int n_tok, int in_dim,
                              uint32_t* x16, float* xscale, hipStream_t s) {
    hipLaunchKernelGGL(k_prep_x<1>, dim3(n_tok), dim3(256), 0, s, g, u, lim, in_dim,
                       reinterpret_cast<_Float16*>(x16), xscale);
    return hipGetLastError();
}

hipError_t launch_matvec_t16(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const uint32_t* x16, const float* xscale, float* y,
                             const void* sign_table, hipStream_t s) {
    const int nb = in_dim / kQK;
    const int tiles = (out_dim + kTileRows - 1) / kTileRows;
    hipLaunchKernelGGL(k_matvec_t16, dim3(tiles), dim3(kMatvecWaves * 64), 0, s, w, nb,
                       (long long)(row0 / kTileRows), out_dim,
                       reinterpret_cast<const half8_t*>(x16), xscale, y,
                       reinterpret_cast<const u32x4_t*>(sign_table));
    return hipGetLastError();
}

hipError_t launch_matvec_raw(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const float* x, float* y, hipStream_t s) {
    const int nb = in_dim / kQK;
    hipLaunchKernelGGL(k_matvec_raw, dim3((out_dim + 3) / 4), dim3(256), 0, s, w, nb, row0, out_dim, x,
                       y);
    return hipGetLastError();
}

}  // namespace gpeed
