// IQ3_XXS decode matvec kernels (gfx950).
//
// k_matvec_t16: batch-1 y = W x over the T16 layout, persistent: one
// 1024-thread workgroup per CU keeps the 64 KiB signed grid table and the
// prepared activation in LDS and walks groups of up to kMvMaxR 16-row tiles.
// The (tile, block) records of a group are split evenly over its 16
// wavefronts; each streams its records with 12-byte coalesced loads through
// a kMvPF-deep register ring and meets the others in LDS per tile.
//
// Per record (16 rows x 256 weights) a wavefront issues 8
// v_mfma_f32_16x16x32_f16. Lane n+16g owns sub-block 4j+g of row n: its two
// LDS lookups per 8-weight group give the signed grid values as fp16, the
// A operand carries the activation as two fp16 rows (hi, lo) placed in rows
// 4g and 4g+1, so accumulator rows 4g/4g+1 of lane n+16g hold exactly that
// sub-block's partial sum and the lane applies its own scale
// d*(0.5+s)*0.5 (times the activation block's power-of-two unscale) to it.
// All products are exact; only fp32 accumulation order differs from the CPU.
#include "iq3_common.h"
#include "iq3_kernels.h"

namespace gpeed {

namespace {

constexpr int kMvMaxR = 8;         // tiles per group
constexpr int kMvMaxStageNb = 64;  // activations up to 16384 elements live in LDS
constexpr int kZeroBytes = 1024;

// Half index of element kk (0..255) of a block in the activation layout
// [j][l][g][hl][8]: the 16 bytes lane (m = 4g + hl, group g) feeds MFMA (j, l).
__device__ __forceinline__ int act_half_index(int kk, int hl) {
    const int ib = kk >> 5, j = ib >> 2, g = ib & 3, l = (kk >> 3) & 3, r = kk & 7;
    return (((j * 4 + l) * 4 + g) * 2 + hl) * 8 + r;
}

// One wavefront per 256-element block: max|v| -> power-of-two scale ->
// fp16 hi/lo split. MODE 0: v = x. MODE 1: v = silu(min(g,lim)) *
// clamp(u,-lim,lim) (model.cpp:683-688, model_batch.cpp:245-253), g = x, u = x2.
template <int MODE>
__global__ __launch_bounds__(256) void k_prep_act(const float* __restrict__ x,
                                                  const float* __restrict__ x2, float lim, int nb,
                                                  _Float16* __restrict__ x16,
                                                  float* __restrict__ xsc) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + wave;
    if (b >= nb) return;
    const float4 v = *reinterpret_cast<const float4*>(x + (size_t)b * 256 + 4 * lane);
    float e[4] = {v.x, v.y, v.z, v.w};
    if (MODE == 1) {
        const float4 u = *reinterpret_cast<const float4*>(x2 + (size_t)b * 256 + 4 * lane);
        const float us[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float gi = fminf(e[c], lim);
            const float ui = fminf(fmaxf(us[c], -lim), lim);
            e[c] = (gi / (1.0f + expf(-gi))) * ui;
        }
    }
    float m = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    int sc = 0;
    if (m > 0.0f && m < __builtin_inff()) {
        int ex;
        (void)frexpf(m, &ex);  // m in [2^(ex-1), 2^ex)
        sc = 14 - ex;          // scaled max in [2^13, 2^14)
        sc = sc > 120 ? 120 : (sc < -120 ? -120 : sc);
    }
    _Float16 hi[4], lo[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float xs = ldexpf(e[c], sc);
        hi[c] = (_Float16)xs;
        lo[c] = (_Float16)(xs - (float)hi[c]);
    }
    _Float16* out = x16 + (size_t)b * 512 + act_half_index(4 * lane, 0);
    *reinterpret_cast<u32x2_t*>(out) = __builtin_bit_cast(u32x2_t, hi);
    *reinterpret_cast<u32x2_t*>(out + 8) = __builtin_bit_cast(u32x2_t, lo);
    if (lane == 0) xsc[b] = ldexpf(1.0f, -sc);
}

__device__ __forceinline__ u32x2_t lds_lookup(const uint8_t* tbl, uint32_t addr) {
    return *reinterpret_cast<const u32x2_t*>(tbl + addr);
}

// B operand of group L of a unit: two lookups of 4 unsigned fp16 grid values
// (the lane's own replica of the table, so no bank conflicts) and the eight
// signs inserted on the fp16 sign bits with v_bfi_b32. lb = (lane & 31) << 3.
template <int L>
__device__ __forceinline__ half8_t decode_group(const uint8_t* tbl, uint32_t q0, uint32_t q1,
                                                uint32_t lb, uint32_t sw) {
    const uint32_t q = (L < 2) ? q0 : q1;
    constexpr uint32_t p1 = (2 * L) & 3, p2 = p1 + 1;
    constexpr uint32_t sel1 = 0x0C0C0000u | ((4u + p1) << 8);
    constexpr uint32_t sel2 = 0x0C0C0000u | ((4u + p2) << 8);
    const u32x2_t g1 = lds_lookup(tbl, __builtin_amdgcn_perm(q, lb, sel1));
    const u32x2_t g2 = lds_lookup(tbl, __builtin_amdgcn_perm(q, lb, sel2));
    const u32x4_t r = {((sw << (0 + L)) & 0x80008000u) | g1.x,
                       ((sw << (4 + L)) & 0x80008000u) | g1.y,
                       ((sw << (8 + L)) & 0x80008000u) | g2.x,
                       ((sw << (12 + L)) & 0x80008000u) | g2.y};
    return __builtin_bit_cast(half8_t, r);
}

// 7 dwords per lane per record: two 12-byte units and the row's fp16 d.
struct Rec {
    uint32_t u[7];
};

__device__ __forceinline__ void load_rec(Rec& r, const uint8_t* rec, uint32_t lane, uint32_t n) {
    // uniform record base + 32-bit unsigned lane offset: SGPR-based addressing
    const uint32_t* p0 = reinterpret_cast<const uint32_t*>(rec + lane * 12u);
    const uint32_t* p1 = reinterpret_cast<const uint32_t*>(rec + kUnitHalfBytes + lane * 12u);
    r.u[0] = p0[0];
    r.u[1] = p0[1];
    r.u[2] = p0[2];
    r.u[3] = p1[0];
    r.u[4] = p1[1];
    r.u[5] = p1[2];
    r.u[6] = *reinterpret_cast<const uint16_t*>(rec + 2 * kUnitHalfBytes + 2u * n);
}

// A operands of one unit (4 MFMAs). Only lanes 4g and 4g+1 of lane group g
// carry data. From LDS every lane reads (idle lanes from a 1 KiB zero region,
// a same-address broadcast), so no branch and no register zeroing; from
// global memory the idle lanes skip the load.
template <bool STAGE>
__device__ __forceinline__ void load_a4(half8_t (&A)[4], const uint8_t* a_lds, const half8_t* a_g,
                                        bool a_lane) {
    if (STAGE) {
#pragma unroll
        for (int i = 0; i < 4; ++i) A[i] = *reinterpret_cast<const half8_t*>(a_lds + i * 128);
    } else if (a_lane) {
#pragma unroll
        for (int i = 0; i < 4; ++i) A[i] = a_g[i * 8];
    } else {
        const half8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) A[i] = z;
    }
}

// One record: 2 units x 4 chained MFMAs; acc += db * (hi + lo partial).
// a_lds / a_g point at this lane's A bytes of the record's block.
template <bool STAGE>
__device__ __forceinline__ float record_dot(const uint8_t* tbl, const Rec& r, uint32_t lb,
                                            const uint8_t* a_lds, const half8_t* a_g, bool a_lane,
                                            float d4, float acc) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t q0 = r.u[3 * j], q1 = r.u[3 * j + 1], w = r.u[3 * j + 2];
        const uint32_t sw = t16_full_signs(w);
        const float db = (float)(2u * ((w >> 16) & 15u) + 1u) * d4;
        half8_t A[4];
        load_a4<STAGE>(A, a_lds + j * 512, a_g + j * 32, a_lane);
        float4_t D = {0.0f, 0.0f, 0.0f, 0.0f};
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], decode_group<0>(tbl, q0, q1, lb, sw), D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1], decode_group<1>(tbl, q0, q1, lb, sw), D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[2], decode_group<2>(tbl, q0, q1, lb, sw), D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[3], decode_group<3>(tbl, q0, q1, lb, sw), D, 0, 0, 0);
        acc = fmaf(db, D[0] + D[1], acc);
    }
    return acc;
}

struct MvArgs {
    const uint8_t* w[2];  // T16 records of the first requested tile, per tensor
    float* y[2];
    int n_tensors;
    int nb;
    int n_tiles;  // tiles per tensor
    int out_dim;
    const uint8_t* act;  // x16 [nb][1024 B] then xscale [nb]
    const u32x4_t* table;
};

// Workgroup barrier that orders LDS only: outstanding global loads (the
// record ring) stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <bool STAGE, int WAVES, int PF>
__global__ __launch_bounds__(WAVES * 64) void k_matvec_t16(MvArgs args) {
    constexpr int kThreads = WAVES * 64;
    // One LDS arena so the table sits at address 0 and lookup addresses need
    // no base: [grid table 64 KiB][activation nb KiB][zeros 1 KiB][unscales][partials]
    constexpr int kXsBytes = STAGE ? kMvMaxStageNb * 1024 : 0;
    constexpr int kZeroOff = kGridTableBytes + kXsBytes;
    constexpr int kXscOff = kZeroOff + (STAGE ? kZeroBytes : 0);
    constexpr int kRedOff = kXscOff + kMvMaxStageNb * 4;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kRedOff + kMvMaxR * WAVES * 16 * 4];
    uint8_t* const tbl = lds;
    uint8_t* const xs = lds + kGridTableBytes;
    float* const xsc = reinterpret_cast<float*>(lds + kXscOff);
    float(*const red)[WAVES][16] = reinterpret_cast<float(*)[WAVES][16]>(lds + kRedOff);
    const int tid = threadIdx.x;
    // wave-uniform: keeps the record ranges and loop control in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lane = tid & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const int nb = args.nb;
    const bool a_lane = (n >> 1) == 2 * g;  // rows 4g (hi) and 4g+1 (lo) of the A operand
    const int a_lane_off = g * 32 + (n & 1) * 16;
    const uint32_t lb = (lane & 31u) << 3;  // this lane's replica of the grid table
    const uint8_t* act = args.act;
    const float* xsc_g = reinterpret_cast<const float*>(act + (size_t)nb * 1024);

    // Table (and staged activation) loads go out first so the LDS writes
    // that need them do not also wait for the record ring issued after them.
    constexpr int kTblPerThread = kGridTableBytes / 16 / kThreads;
    u32x4_t tv[kTblPerThread];
#pragma unroll
    for (int i = 0; i < kTblPerThread; ++i) tv[i] = args.table[tid + i * kThreads];
    constexpr int kXPerThread = STAGE ? (kMvMaxStageNb * 64 + kThreads - 1) / kThreads : 1;
    u32x4_t xv[kXPerThread];
    const int nchunk = nb * 64;
    if (STAGE) {
        const u32x4_t* src = reinterpret_cast<const u32x4_t*>(act);
#pragma unroll
        for (int i = 0; i < kXPerThread; ++i) xv[i] = src[min(tid + i * kThreads, nchunk - 1)];
    }
    float xsc_v = 0.0f;
    if (STAGE && tid < nb) xsc_v = xsc_g[tid];

    // Tiles are dealt round-robin over the grid (tile' = blockIdx + k*G, tile'
    // counting the tensors' tiles in order) and, inside a workgroup, records
    // round-robin over its wavefronts, so at any moment the whole GPU reads
    // one contiguous window of the weights rather than one chunk per CU.
    const int T_all = args.n_tiles * args.n_tensors;
    const int G = gridDim.x;
    const int my_tiles = (T_all - (int)blockIdx.x + G - 1) / G;
    bool first = true;
    for (int k0 = 0; k0 < my_tiles; k0 += kMvMaxR) {
        const int nt = min(kMvMaxR, my_tiles - k0);
        const int P = nt * nb;
        auto rec_ptr = [&](int p) -> const uint8_t* {
            const int kt = p / nb;
            const int tp = (int)blockIdx.x + (k0 + kt) * G;
            const int ten = tp >= args.n_tiles ? 1 : 0;
            const int t = tp - ten * args.n_tiles;
            return args.w[ten] + ((size_t)t * nb + (p - kt * nb)) * kRecordBytes;
        };

        // Ring loads are unconditional: past the wave's records they re-read
        // the round's last record (valid, cache-resident), so no load waits
        // on a branch.
        Rec buf[PF];
#pragma unroll
        for (int s = 0; s < PF; ++s) load_rec(buf[s], rec_ptr(min(wave + s * WAVES, P - 1)), lane, n);

        if (first) {
#pragma unroll
            for (int i = 0; i < kTblPerThread; ++i) reinterpret_cast<u32x4_t*>(tbl)[tid + i * kThreads] = tv[i];
            if (STAGE) {
#pragma unroll
                for (int i = 0; i < kXPerThread; ++i)
                    if (tid + i * kThreads < nchunk) reinterpret_cast<u32x4_t*>(xs)[tid + i * kThreads] = xv[i];
                if (tid < nb) xsc[tid] = xsc_v;
                if (tid < kZeroBytes / 16) {
                    const u32x4_t z = {0u, 0u, 0u, 0u};
                    reinterpret_cast<u32x4_t*>(lds + kZeroOff)[tid] = z;
                }
            }
            for (int i = tid; i < kMvMaxR * WAVES * 16; i += kThreads) (&red[0][0][0])[i] = 0.0f;
            first = false;
            lds_barrier();
        }

        int tl = wave / nb, b = wave - (wave / nb) * nb;  // (tile, block) of record p
        float acc = 0.0f;
        for (int i = 0; wave + i * WAVES < P; i += PF) {
#pragma unroll
            for (int s = 0; s < PF; ++s) {
                const int p = wave + (i + s) * WAVES;
                if (p < P) {
                    const float xsb = STAGE ? xsc[b] : xsc_g[b];
                    const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)buf[s].u[6]);
                    const float d4 = d * 0.25f * xsb;
                    acc = record_dot<STAGE>(tbl, buf[s], lb, a_lane ? xs + b * 1024 + a_lane_off : lds + kZeroOff,
                                            reinterpret_cast<const half8_t*>(act + (size_t)b * 1024 + a_lane_off),
                                            a_lane, d4, acc);
                    // refill unconditionally (clamped like the prologue) so the
                    // slot has one live copy
                    load_rec(buf[s], rec_ptr(min(p + PF * WAVES, P - 1)), lane, n);
                    // keep records from interleaving: the ring, not the
                    // scheduler, provides the overlap, and registers stay at
                    // ring + one record's temporaries
                    __builtin_amdgcn_sched_barrier(0);
                    // next record of this wave: flush the partial on a tile change
                    int nb_ = b + WAVES, ntl = tl;
                    while (nb_ >= nb) {
                        nb_ -= nb;
                        ++ntl;
                    }
                    if (ntl != tl || p + WAVES >= P) {
                        float v = acc + __shfl_xor(acc, 16);
                        v += __shfl_xor(v, 32);
                        if (g == 0) red[tl][wave][n] = v;
                        acc = 0.0f;
                    }
                    tl = ntl;
                    b = nb_;
                }
            }
        }
        lds_barrier();
        // sum the wavefront partials in a fixed order; the reader re-zeroes
        // its slots for the next round
        if (tid < nt * 16) {
            const int tt = tid >> 4, nn = tid & 15;
            float sum = 0.0f;
#pragma unroll
            for (int v = 0; v < WAVES; ++v) {
                sum += red[tt][v][nn];
                red[tt][v][nn] = 0.0f;
            }
            const int tp = (int)blockIdx.x + (k0 + tt) * G;
            const int ten = tp >= args.n_tiles ? 1 : 0;
            const int row = (tp - ten * args.n_tiles) * 16 + nn;
            if (row < args.out_dim) args.y[ten][row] = sum;
        }
        lds_barrier();
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

size_t act_bytes(int in_dim) {
    // fp16 hi/lo operand (4 bytes per element) + one fp32 unscale per block,
    // rounded up to 256 bytes
    const size_t b = (size_t)in_dim * 4 + (size_t)(in_dim / kQK) * 4;
    return (b + 255) / 256 * 256;
}

hipError_t launch_prep_act(const float* x, int in_dim, uint8_t* act, hipStream_t s) {
    const int nb = in_dim / kQK;
    hipLaunchKernelGGL(k_prep_act<0>, dim3((nb + 3) / 4), dim3(256), 0, s, x, nullptr, 0.0f, nb,
                       reinterpret_cast<_Float16*>(act), reinterpret_cast<float*>(act + (size_t)in_dim * 4));
    return hipGetLastError();
}

hipError_t launch_prep_swiglu(const float* g, const float* u, float lim, int in_dim, uint8_t* act,
                              hipStream_t s) {
    const int nb = in_dim / kQK;
    hipLaunchKernelGGL(k_prep_act<1>, dim3((nb + 3) / 4), dim3(256), 0, s, g, u, lim, nb,
                       reinterpret_cast<_Float16*>(act), reinterpret_cast<float*>(act + (size_t)in_dim * 4));
    return hipGetLastError();
}

// Launch configuration: activation staged in LDS (K <= 16384), 16 wavefronts
// per workgroup, 8-record ring, one workgroup per CU.
#ifndef MV_STAGE
#define MV_STAGE 1
#endif
#ifndef MV_WAVES
#define MV_WAVES 16
#endif
#ifndef MV_PF
#define MV_PF 8
#endif
#ifndef MV_WG_PER_CU
#define MV_WG_PER_CU 1
#endif

template <bool STAGE, int WAVES, int PF>
static hipError_t launch_cfg(const MvArgs& a, int slots, hipStream_t s) {
    const int total = a.n_tiles * a.n_tensors;
    const int grid = total < slots ? total : slots;
    hipLaunchKernelGGL((k_matvec_t16<STAGE, WAVES, PF>), dim3(grid), dim3(WAVES * 64), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_matvec_t16(const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                             unsigned long long row0, int out_dim, const uint8_t* act,
                             const void* grid_table, int num_cus, hipStream_t s) {
    MvArgs a;
    a.nb = in_dim / kQK;
    const size_t skip = (size_t)(row0 / kTileRows) * a.nb * kRecordBytes;
    for (int i = 0; i < 2; ++i) {
        const int k = i < n_tensors ? i : 0;
        a.w[i] = w[k] + skip;
        a.y[i] = y[k];
    }
    a.n_tensors = n_tensors;
    a.n_tiles = (out_dim + kTileRows - 1) / kTileRows;
    a.out_dim = out_dim;
    a.act = act;
    a.table = reinterpret_cast<const u32x4_t*>(grid_table);
    const int cus = num_cus > 0 ? num_cus : 256;
    if (MV_STAGE && a.nb <= kMvMaxStageNb)
        return launch_cfg<(MV_STAGE != 0), MV_WAVES, MV_PF>(a, cus * MV_WG_PER_CU, s);
    return launch_cfg<false, MV_WAVES, MV_PF>(a, cus * MV_WG_PER_CU, s);
}

hipError_t launch_matvec_raw(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const float* x, float* y, hipStream_t s) {
    const int nb = in_dim / kQK;
    hipLaunchKernelGGL(k_matvec_raw, dim3((out_dim + 3) / 4), dim3(256), 0, s, w, nb, row0, out_dim, x,
                       y);
    return hipGetLastError();
}

}  // namespace gpeed
