// IQ3_XXS prefill GEMM (gfx950): Y[m][n] = sum_k X[m][k] * W[row0+n][k]
// for many tokens (matmul_quant, weights.cpp:86-165, at prefill sizes).
//
// Operands. W is decoded to fp16 holding +-grid * (2s+1): an integer of at
// most 62 * 31 = 1922, exact in fp16 (bf16 would round it), so the only
// per-weight scale left is the block's d/4, applied once per 256-wide block
// to the fp32 partial of that block. X is converted once (k_gemm_prep_x) to
// fp16 with a power-of-two scale per token row (bf16 input: one image, exact
// for every value within 2^24 of the row maximum; fp32 input: an fp16 hi
// image and an fp16 lo image, two MFMAs per step). Products are exact; sums
// are fp32 in v_mfma_f32_16x16x32_f16.
//
// Tiling. A workgroup computes 128 (or 64) tokens x 192 W rows and decodes
// every W value of its rows exactly once, straight into MFMA B operand
// registers. Workgroups are ordered so that the eight XCDs each work on
// their own band of W rows (the band stays in that XCD's L2 while all token
// tiles use it). k_gemm5 (bf16 X of more than 64 tokens, and fp32 X) and
// k_gemm3 (bf16 X of at most 64 tokens) differ in how the wavefronts split
// the tile and how W and X reach them; see each kernel.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "iq3_common.h"
#include "iq3_gemv_core.h"
#include "iq3_kernels.h"
#include "iq3_prof.h"

namespace gpeed {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2v_t __attribute__((ext_vector_type(2)));

constexpr int kGemmThreads = 256;
// cache policy of k_gemm5's W loads: non-temporal (each W tile is read by
// at most a few token tiles; k_gemm6's many token tiles re-read W from L2
// and keep the default: 324.5 -> 328.4 us at M = 2048 with it)
constexpr int kWNt = 2;

__device__ __forceinline__ uint32_t f16_pair_of_floats(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

// ---------------------------------------------------------------------------
// X -> fp16 images with a power-of-two scale per token row. One workgroup per
// row. IN = 0: fp32 input (hi and lo images); IN = 1: bf16 input (one image);
// IN = 2: X = SwiGLU(X, U) of fp32 gate and up rows (hi and lo images).
// CPT > 0: the row is at most 256 * CPT chunks of 8 values, each thread holds
// its CPT chunks in registers, so the row is read once and every load is in
// flight before the first wait (a row of 12288 SwiGLU values: one memory
// round trip instead of twelve); CPT = 0: any length, two passes.
// The workgroups also clear the n_cnt split-K tickets of the GEMM launch
// that follows on the same stream, so a workspace needs no initialisation.
// gather (may be null): image row m is X row gather[m] (bucket slots of
// routed experts: the slot's token).
template <int IN, int CPT, int NTHR = 256>
__global__ __launch_bounds__(NTHR) void k_gemm_prep_x(const void* __restrict__ X, const float* __restrict__ U,
                                                     float lim, int M, int K, _Float16* __restrict__ xh,
                                                     float* __restrict__ unscale, uint32_t* __restrict__ cnt,
                                                     int n_cnt, const int* __restrict__ gather) {
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    const int src = gather ? gather[m] : m;  // the X (and U) row of image row m
    for (int i = m * NTHR + tid; i < n_cnt; i += M * NTHR) cnt[i] = 0u;
    constexpr int kW = NTHR / 64;
    __shared__ float red[kW];
    // the 8 raw values of chunk c (16-byte loads; K is a multiple of 256)
    struct Raw {
        u32x4_t a, b, ua, ub;
    };
    auto load8 = [&](int c, Raw& r) {
        if constexpr (IN == 1) {
            r.a = reinterpret_cast<const u32x4_t*>(X)[((size_t)src * K >> 3) + c];
        } else {
            const u32x4_t* p = reinterpret_cast<const u32x4_t*>(X) + ((size_t)src * K >> 2) + 2 * c;
            r.a = p[0];
            r.b = p[1];
            if constexpr (IN == 2) {
                const u32x4_t* q = reinterpret_cast<const u32x4_t*>(U) + ((size_t)src * K >> 2) + 2 * c;
                r.ua = q[0];
                r.ub = q[1];
            }
        }
    };
    auto values8 = [&](const Raw& r, float (&v)[8]) {
        if constexpr (IN == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[2 * i] = __uint_as_float(r.a[i] << 16);
                v[2 * i + 1] = __uint_as_float(r.a[i] & 0xFFFF0000u);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = __uint_as_float(r.a[i]);
                v[4 + i] = __uint_as_float(r.b[i]);
            }
            if constexpr (IN == 2) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = swiglu1(v[i], __uint_as_float(r.ua[i]), lim);
                    v[4 + i] = swiglu1(v[4 + i], __uint_as_float(r.ub[i]), lim);
                }
            }
        }
    };
    const size_t plane = (size_t)M * K;
    auto store8 = [&](int c, const float (&v)[8], int sc) {
        u32x4_t hi, lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = ldexpf(v[2 * i], sc), b = ldexpf(v[2 * i + 1], sc);
            const _Float16 ha = (_Float16)a, hb = (_Float16)b;
            hi[i] = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
            lo[i] = f16_pair_of_floats(a - (float)ha, b - (float)hb);
        }
        reinterpret_cast<u32x4_t*>(xh + (size_t)m * K)[c] = hi;
        if constexpr (IN != 1) reinterpret_cast<u32x4_t*>(xh + plane + (size_t)m * K)[c] = lo;
    };
    auto row_scale = [&](float mx) {
        mx = wave_max(mx);
        if ((tid & 63) == 0) red[tid >> 6] = mx;
        __syncthreads();
        float r = red[0];
#pragma unroll
        for (int w = 1; w < kW; ++w) r = fmaxf(r, red[w]);
        return pow2_scale_of_max(r);
    };
    const int n8 = K >> 3;
    float mx = 0.0f;
    if constexpr (CPT > 0) {
        // loads of chunks past the row are clamped to its last chunk (they
        // leave the maximum unchanged) and their results are not stored
        Raw r[CPT];
#pragma unroll
        for (int j = 0; j < CPT; ++j) load8(min(tid + NTHR * j, n8 - 1), r[j]);
        float v[CPT][8];
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            values8(r[j], v[j]);
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[j][i]));
        }
        const int sc = row_scale(mx);
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (tid + NTHR * j < n8) store8(tid + NTHR * j, v[j], sc);
        if (tid == 0) unscale[m] = ldexpf(1.0f, -sc);
    } else {
        for (int c = tid; c < n8; c += NTHR) {
            Raw r;
            float v[8];
            load8(c, r);
            values8(r, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
        }
        const int sc = row_scale(mx);
        for (int c = tid; c < n8; c += NTHR) {
            Raw r;
            float v[8];
            load8(c, r);
            values8(r, v);
            store8(c, v, sc);
        }
        if (tid == 0) unscale[m] = ldexpf(1.0f, -sc);
    }
}

// The preparation launch for rows of K values: chunks per thread in
// registers where the row has at most 2048 chunks. Fewer rows than CUs
// take 1024 threads a row: four wavefronts per SIMD hide more of the
// latency of each one's loads and SwiGLU chain (the decode mix's step,
// whose two preparations have 64 rows, 93.4 -> 92.9 us, bitwise equal).
template <int IN>
hipError_t launch_prep_x(int M, int K, hipStream_t s, const void* X, const float* U, float lim, _Float16* xh,
                         float* uns, uint32_t* cnt, int n_cnt, const int* gather = nullptr) {
    if (M < 256 && K >= 8 * 1024) {
        const int per4 = (K / 8 + 1023) / 1024;
        const dim3 grid(M), block(1024);
        if (per4 <= 1)
            hipLaunchKernelGGL((k_gemm_prep_x<IN, 1, 1024>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt,
                               gather);
        else if (per4 <= 2)
            hipLaunchKernelGGL((k_gemm_prep_x<IN, 2, 1024>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt,
                               gather);
        else
            hipLaunchKernelGGL((k_gemm_prep_x<IN, 0, 1024>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt,
                               gather);
        return hipGetLastError();
    }
    const int per = (K / 8 + 255) / 256;
    const dim3 grid(M), block(256);
    if (per <= 1)
        hipLaunchKernelGGL((k_gemm_prep_x<IN, 1>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt, gather);
    else if (per <= 2)
        hipLaunchKernelGGL((k_gemm_prep_x<IN, 2>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt, gather);
    else if (per <= 3)
        hipLaunchKernelGGL((k_gemm_prep_x<IN, 3>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt, gather);
    else if (per <= 4)
        hipLaunchKernelGGL((k_gemm_prep_x<IN, 4>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt, gather);
    else if (per <= 6)
        hipLaunchKernelGGL((k_gemm_prep_x<IN, 6>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt, gather);
    else if (per <= 8)
        hipLaunchKernelGGL((k_gemm_prep_x<IN, 8>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt, gather);
    else
        hipLaunchKernelGGL((k_gemm_prep_x<IN, 0>), grid, block, 0, s, X, U, lim, M, K, xh, uns, cnt, n_cnt, gather);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GEMM

// A launch's second problem (k_gemm5, non-grouped; the same M): workgroups
// wg0 .. grid - 1 compute it, from its own images (xh, unscale, K, nb), split
// count, tickets and partials, one or two tensors like the first. wg0 0:
// no second problem.
struct GemmProb {
    const uint8_t* w;
    const _Float16* xh;
    const float* unscale;
    float* y;
    int N, K, nb, tiles_n, ks;
    uint32_t* cnt;
    float* part;
    const uint8_t* w2;
    float* y2;
    int N2, tiles_n1;
    int wg0;
};

struct GemmArgs {
    const uint8_t* w;       // T64 records of the first requested tile
    const _Float16* xh;     // [V][M][K] fp16 images
    const float* unscale;   // [M]
    float* y;               // [M][N]
    int M, N, K, nb;
    int tiles_m, tiles_n;   // tiles_n: result tiles of both tensors
    int ks;                 // K splits per result tile (1: no partials)
    uint32_t* cnt;          // ks > 1: tickets per tile (cleared by k_gemm_prep_x)
    float* part;            // ks > 1: [tile][split][128][192] fp32 partials
    uint32_t* err;          // the workspace's error word (kWs* flags)
    // a second tensor on the same X: result tiles tn >= tiles_n1 are its
    // tiles tn - tiles_n1 (w2, y2 [M][N2]); tiles_n1 = tiles_n for one tensor
    const uint8_t* w2;
    float* y2;
    int N2, tiles_n1;
    // grouped (routed experts; k_gemm5 only): X rows are bucket slots,
    // expert e's at grp_eptr[e] .. grp_eptr[e + 1] of [V][grp_rows][K]
    // images; workgroup id / tiles_n picks entry grp_tile[.] = e << 16 | its
    // token tile (grp_count[0] entries); the tensors' rows of expert e start
    // grp_w_stride bytes of records after those of expert e - 1; Y rows are
    // slots too. grp_eptr null: one GEMM over rows 0 .. M - 1.
    // grp_tok (may be null): slot p's image row (and unscale) is
    // grp_tok[p] of images of grp_img_rows rows (per-token images of the
    // batch, shared by every slot of a token) instead of row p.
    const int* grp_eptr;
    const int* grp_tile;
    const int* grp_count;
    int grp_rows;
    unsigned long long grp_w_stride;
    const int* grp_tok;
    int grp_img_rows;
    // grp_sh_e >= 0: table entries of that expert id are the shared expert
    // (grp_sh_rows slots from grp_eptr[grp_sh_e], its tensors grp_w_sh /
    // grp_w2_sh); with grp_tok its slot m reads image row m (token m)
    int grp_sh_e, grp_sh_rows;
    const uint8_t* grp_w_sh;
    const uint8_t* grp_w2_sh;
    GemmProb p2;
};

constexpr int kTileN = 192;  // result tile: 128 (or 64) tokens x 192 W rows

// Workgroup -> result tile (tm, tn) and K split kz (blocks [b0, b1)); the
// splits of a tile have consecutive workgroup ids. Tiles are ordered so
// that the eight XCDs (workgroup id % 8) each work on their own band of W
// row tiles when the row tiles split evenly into 8 bands.
struct GemmTile {
    int tm, tn, kz, b0, b1;
};
__device__ __forceinline__ GemmTile gemm_tile(const GemmArgs& g, int bid) {
    GemmTile t;
    t.kz = bid % g.ks;
    const int id = bid / g.ks;
    if (g.ks == 1 && g.tiles_n % 8 == 0) {
        const int per_band = g.tiles_n / 8;
        const int xcd = id & 7, local = id >> 3;
        t.tn = xcd * per_band + local % per_band;
        t.tm = local / per_band;
    } else {
        t.tn = id % g.tiles_n;
        t.tm = id / g.tiles_n;
    }
    t.b0 = t.kz * g.nb / g.ks;
    t.b1 = (t.kz + 1) * g.nb / g.ks;
    return t;
}

// The arguments of the tensor that result tile t belongs to (w, y, N its
// own) and the tile's index inside that tensor.
__device__ __forceinline__ GemmArgs gemm_tensor(const GemmArgs& g, const GemmTile& t, int& tn_local) {
    GemmArgs a = g;
    tn_local = t.tn;
    if (t.tn >= g.tiles_n1) {
        a.w = g.w2;
        a.y = g.y2;
        a.N = g.N2;
        tn_local = t.tn - g.tiles_n1;
    }
    return a;
}

// The result tile (16 MT tokens x 192 rows) from this workgroup's fp32 sums acc[mt][j][i] (token
// m0 + 16 mt + 4 lg + i, W row n0 + 48 wave + 16 j + lr). One K split:
// Y = acc * unscale[m]. Several: each split stores its partial with
// device-coherent stores; after vmcnt(0) it takes the tile's ticket, and
// the last one adds the partials in split order (bitwise repeatable) and
// writes Y, then clears the ticket.
//
// Why this hand-off is ordered without release/acquire fences (gfx950
// memory model): the partials are agent-scope atomic stores, which the
// compiler emits as stores that write through this XCD's L2 (sc1) instead
// of leaving dirty lines there; s_waitcnt vmcnt(0) returns only once every
// one of them is acknowledged by memory; the ticket is an agent-scope
// atomic performed at memory after that, so a split that sees the last
// ticket value sees every earlier split's completed stores; and the reader
// loads with sc1, missing in its own L2, which can hold stale lines of the
// workspace from an earlier call. A release fence would add a write-back of
// all of this XCD's dirty L2 lines (other tiles' Y) that no reader needs. A
// ticket past the split count (two launches sharing the workspace) sets
// kWsTicket.
// BN: the tile's W rows, NTHR: the workgroup's threads. The wavefront's
// rows are n0 + rbase + 16 j + lr (j < JT); a wavefront with active false
// holds no rows of its own (its sums went to another wavefront) and only
// joins the barriers and the last split's sum.
template <int BM, int kTileN, int NTHR>
__device__ __forceinline__ void gemm_split_finish(const GemmArgs& g, const GemmTile& t, int m0, int n0, int tid,
                                                  int* flag);

template <int MT, int JT = 3, int BN = kTileN, int NTHR = kGemmThreads>
__device__ __forceinline__ void gemm_store(const GemmArgs& g, const GemmTile& t, const float4_t (&acc)[MT][JT],
                                           int m0, int n0, int rbase, int lr, int lg, int tid, int* flag,
                                           bool active = true) {
    constexpr int BM = 16 * MT;
    constexpr int kTileN = BN;  // (shadows the 192-row default)
    if (g.ks == 1) {
        if (!active) return;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + mt * 16 + lg * 4 + i;
                if (m >= g.M) continue;
                const float us = g.unscale[m];
#pragma unroll
                for (int j = 0; j < JT; ++j) {
                    const int n = n0 + rbase + j * 16 + lr;
                    if (n < g.N) g.y[(size_t)m * g.N + n] = acc[mt][j][i] * us;
                }
            }
        return;
    }
    const int tile = t.tm * g.tiles_n + t.tn;
    float* base = g.part + (size_t)tile * g.ks * (BM * kTileN);
    float* mine = base + (size_t)t.kz * (BM * kTileN);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ml = mt * 16 + lg * 4 + i;
            if (!active || m0 + ml >= g.M) continue;
#pragma unroll
            for (int j = 0; j < JT; ++j) {
                const int nl = rbase + j * 16 + lr;
                if (n0 + nl < g.N)
                    __hip_atomic_store(mine + ml * kTileN + nl, acc[mt][j][i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    gemm_split_finish<BM, kTileN, NTHR>(g, t, m0, n0, tid, flag);
}

// After this split's partial went out (agent-scope write-through stores):
// wait for their acknowledgement, take the tile's ticket; the last split adds
// the partials in split order and writes Y, then clears the ticket.
template <int BM, int kTileN, int NTHR>
__device__ __forceinline__ void gemm_split_finish(const GemmArgs& g, const GemmTile& t, int m0, int n0, int tid,
                                                  int* flag) {
    const int tile = t.tm * g.tiles_n + t.tn;
    float* base = g.part + (size_t)tile * g.ks * (BM * kTileN);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this split's partial is acknowledged
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(g.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == (uint32_t)(g.ks - 1);
        if (old >= (uint32_t)g.ks) __hip_atomic_fetch_or(g.err, kWsTicket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*flag) return;  // uniform
    // four columns per item; a thread takes kR items per step and issues
    // every split's loads of all of them before the first add, so a 64-token
    // tile is one memory round trip (the loads miss in L2 by design: buffer
    // loads with sc1, past this XCD's L2, which may hold the workspace from
    // an earlier call)
    constexpr int kR = 6;
    const int rows = min(BM, g.M - m0), cols = min(kTileN, g.N - n0);
    const int n_items = rows * (kTileN / 4);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(base, 0, (int)(g.ks * BM * kTileN * 4), 0x00020000);
    for (int q0 = tid; q0 < n_items; q0 += kR * NTHR) {
        float4 v[kR][8];
#pragma unroll
        for (int u = 0; u < kR; ++u) {
            const int q = q0 + u * NTHR;
            const int ml = q / (kTileN / 4), nl = (q - ml * (kTileN / 4)) * 4;
            const bool ok = q < n_items && nl < cols;
#pragma unroll
            for (int z = 0; z < 8; ++z) {
                if (z >= g.ks) break;  // uniform: no load for splits that do not exist
                const uint32_t off = ok ? (uint32_t)(((z * BM + ml) * kTileN + nl) * 4) : 0x80000000u;
                v[u][z] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 16));
            }
        }
#pragma unroll
        for (int u = 0; u < kR; ++u) {
            const int q = q0 + u * NTHR;
            const int ml = q / (kTileN / 4), nl = (q - ml * (kTileN / 4)) * 4;
            if (q >= n_items || nl >= cols) continue;
            float4 sum = v[u][0];
#pragma unroll
            for (int z = 1; z < 8; ++z)
                if (z < g.ks) {
                    sum.x += v[u][z].x;
                    sum.y += v[u][z].y;
                    sum.z += v[u][z].z;
                    sum.w += v[u][z].w;
                }
            const float us = g.unscale[m0 + ml];
            float* yrow = g.y + (size_t)(m0 + ml) * g.N + n0 + nl;
            const float o[4] = {sum.x * us, sum.y * us, sum.z * us, sum.w * us};
            if (nl + 4 <= cols && (reinterpret_cast<uintptr_t>(yrow) & 15u) == 0) {
                *reinterpret_cast<float4*>(yrow) = float4{o[0], o[1], o[2], o[3]};
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (nl + c < cols) yrow[c] = o[c];
            }
        }
    }
    if (tid == 0) __hip_atomic_store(g.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// GEMM, one wavefront per SIMD (bf16 X of at most 64 tokens, as 64-token
// tiles; the fallback for X images of 4 GiB or more). A 256-thread
// workgroup computes BM tokens x 192 rows; wavefront w owns rows
// 48w..48w+47 and all BM tokens, arranged so that the matrix cores are fed
// every cycle the wavefront can give them:
//   * W arrives as whole record units: per 256-wide block the workgroup
//     copies the three row tiles' six 1 KiB units and their d values into
//     LDS (coalesced 16-byte loads, one block ahead), and the decode reads
//     its two words per (row, sub-block) from there;
//   * the B operands of stage s+1 (64 columns) are decoded while the MFMAs
//     of stage s run, from a grid table that already holds grid * (2s+1)
//     (entry (idx, s) at (idx << 8) | (s << 4), two replicas), so a group of
//     8 weights costs two lookups, the sign word's decode and two
//     64-bit shifts that put four pairs of signs on the fp16 sign bits;
//   * A operands are read one half-stage ahead from a ring of three X
//     stages, loaded two stages ahead into registers;
//   * one workgroup barrier per stage.
// Products stay exact (|q (2s+1)| <= 1922 in fp16, X an exact fp16 image);
// the block's d/4 scales its fp32 partial once per 256 columns. (Folding d
// into B would round every weight to fp16: about 3e-4 rms relative error
// per product, which exceeds 1e-3 of max(|y_i|, rms(y)) on outputs near
// the rms.)

constexpr int BN3 = 192, BK3 = 64;
constexpr int kRow3 = BK3 + 8;                       // X LDS row stride (halves)
constexpr int kWBlk3 = 3 * 6 * kUnitBytes;           // one block: 3 row tiles x 6 units
constexpr int kWItems3 = 5;                          // W copy items per lane-slot per block

template <int BM, int V>
struct GemmSmem3 {
    uint8_t tbl[kGridTableBytes];                    // grid * (2s+1), see above
    _Float16 xs[3][V][BM * kRow3];                   // X stages (ring of 3), V images each
    uint8_t wb[2][kWBlk3];                           // W blocks: [tile][unit][64 lanes x 16 B]
    uint8_t wd[2][512];                              // their d: [tile][64 fp16] (+ padding)
    int last_flag;                                   // this workgroup completes its tile
};

// Entry (idx, s) of the scaled grid, both replicas: thread (s = tid & 15)
// fills 16 entries idx = (tid >> 4) + 16 i; 16 lanes write 256 contiguous
// bytes per store.
__device__ __forceinline__ void scaled_grid_table(uint8_t* tbl, int tid) {
    const uint32_t s = tid & 15;
    const float m = (float)(2 * s + 1);
#pragma unroll 4
    for (int i = 0; i < 16; ++i) {
        const uint32_t idx = (tid >> 4) + 16 * i;
        const uint32_t v = kIq3xxsGrid[idx];
        const uint32_t lo = f16_pair_of_floats((float)(v & 255u) * m, (float)((v >> 8) & 255u) * m);
        const uint32_t hi = f16_pair_of_floats((float)((v >> 16) & 255u) * m, (float)(v >> 24) * m);
        *reinterpret_cast<u32x4_t*>(tbl + (idx << 8) + (s << 4)) = u32x4_t{lo, hi, lo, hi};
    }
}

// B operand of v_mfma_f32_16x16x32_f16 for one lane: the 8 weights of group
// lg (columns 8lg..8lg+7 of a sub-block) of one W row, as fp16
// +-grid*(2s+1), from the sub-block's grid-index word q (bytes p0, p0+1
// hold the group's two indices) and sign/scale word w. sel0/sel1 pick those
// bytes; rs = replica offset (0 or 8).
__device__ __forceinline__ half8_t decode_group(const uint8_t* tbl, uint32_t q, uint32_t w, uint32_t lg,
                                                uint32_t sel0, uint32_t sel1, uint32_t rs) {
    // group lg's signs, the eighth included: pair c at bits 4c and 4c+16
    const uint32_t sw = t64_signs(w);
    const uint32_t wg = __builtin_amdgcn_alignbit(sw, sw, lg);
    // pairs 0/1 and 2/3: one 64-bit shift of {wg >> 4, wg} each puts a
    // pair's two signs on bits 15 and 31 of both halves
    const uint64_t sw2 = ((uint64_t)(wg >> 4) << 32) | wg;
    const uint64_t r01 = shl64<15>(sw2), r23 = shl64<7>(sw2);
    const uint32_t sr = ((w >> 24) & 0xF0u) | rs;  // (s << 4) | replica
    const u32x2_t g0 = *reinterpret_cast<const u32x2_t*>(tbl + __builtin_amdgcn_perm(q, sr, sel0));
    const u32x2_t g1 = *reinterpret_cast<const u32x2_t*>(tbl + __builtin_amdgcn_perm(q, sr, sel1));
    const u32x4_t r = {((uint32_t)r01 & 0x80008000u) | g0.x, ((uint32_t)(r01 >> 32) & 0x80008000u) | g0.y,
                       ((uint32_t)r23 & 0x80008000u) | g1.x, ((uint32_t)(r23 >> 32) & 0x80008000u) | g1.y};
    return __builtin_bit_cast(half8_t, r);
}

template <int BM, int V>
__global__ __launch_bounds__(kGemmThreads) void k_gemm3(GemmArgs g_all) {
    constexpr int MT = BM / 16;  // token tiles per wavefront
    constexpr int XP = BM / 32;  // X pieces per thread per image and stage
    __shared__ __attribute__((aligned(16))) GemmSmem3<BM, V> sm;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lane = tid & 63;
    const int lr = lane & 15;
    const uint32_t lg = lane >> 4;

    const GemmTile tl = gemm_tile(g_all, blockIdx.x);
    if (tl.tm >= g_all.tiles_m || tl.tn >= g_all.tiles_n) return;  // uniform
    int tn;
    const GemmArgs g = gemm_tensor(g_all, tl, tn);
    const int tm = tl.tm;
    const int m0 = tm * BM, n0 = tn * BN3;
    const uint32_t kboff = (uint32_t)tl.b0 * kRecordBytes;  // this split's first block

    const int last_tile = (g.N + kTileRows - 1) / kTileRows - 1;
    scaled_grid_table(sm.tbl, tid);

    // W copy items of this lane-slot (wave * 5 + i): 0..17 = (row tile
    // item / 6, unit item % 6), 18 and 19 = the three tiles' d (lanes
    // 0..23, 16 bytes each; 19 repeats 18). Row tiles past the tensor are
    // clamped to its last tile (their rows are computed, never stored).
    uint32_t w_goff[kWItems3], w_loff[kWItems3];
#pragma unroll
    for (int i = 0; i < kWItems3; ++i) {
        const int item = wave * kWItems3 + i;
        if (item < 18) {
            const int jt = item / 6, u = item % 6;
            const int tile = min(n0 / kTileRows + jt, last_tile);
            w_goff[i] = (uint32_t)tile * (uint32_t)g.nb * kRecordBytes + kboff + u * kUnitBytes + lane * 16u;
            w_loff[i] = (uint32_t)(jt * 6 + u) * kUnitBytes + lane * 16u;
        } else {
            const uint32_t l = min(lane, 23u);
            const int jt = l >> 3;
            const int tile = min(n0 / kTileRows + jt, last_tile);
            w_goff[i] = (uint32_t)tile * (uint32_t)g.nb * kRecordBytes + kboff + kRecordDOffset + (l & 7) * 16u;
            w_loff[i] = kWBlk3 + (uint32_t)jt * 128u + (l & 7) * 16u;  // past wb: into wd
        }
    }
    u32x4_t wreg[kWItems3];
    auto load_w = [&](int b) {
        const uint32_t boff = (uint32_t)b * kRecordBytes;
#pragma unroll
        for (int i = 0; i < kWItems3; ++i) wreg[i] = *reinterpret_cast<const u32x4_t*>(g.w + (w_goff[i] + boff));
    };
    auto store_w = [&](int slot) {
#pragma unroll
        for (int i = 0; i < kWItems3; ++i) {
            const uint32_t lo = w_loff[i];
            uint8_t* dst = lo < (uint32_t)kWBlk3 ? &sm.wb[slot][lo] : &sm.wd[slot][lo - kWBlk3];
            *reinterpret_cast<u32x4_t*>(dst) = wreg[i];
        }
    };

    // This lane's rows (j = 0..2): row tile and lane slot inside the block copy.
    uint32_t w_rowoff[3], d_off[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int r = wave * 48 + j * 16 + lr;  // 0..191
        w_rowoff[j] = (uint32_t)(r >> 6) * 6 * kUnitBytes + (uint32_t)(r & 63) * 16u;
        d_off[j] = (uint32_t)(r >> 6) * 128u + (uint32_t)(r & 63) * 2u;
    }
    const uint32_t p0 = 2 * (lg & 1);
    const uint32_t sel0 = 0x0C0C0000u | ((4u + p0) << 8);
    const uint32_t sel1 = 0x0C0C0000u | ((5u + p0) << 8);
    // lanes of one row that share an index word read different replicas
    const uint32_t rs = (lg & 1u) << 3;
    const bool hiq = lg >= 2;  // the group's indices sit in the sub-block's second index word

    // B operands of sub-block t of stage s: [j]
    auto decode_half = [&](half8_t (&bop)[3], int s, int t) {
        const uint8_t* wb = sm.wb[(s >> 2) & 1];
        const int ib = 2 * (s & 3) + t;
        const int dq = 3 * ib + (hiq ? 1 : 0), dw = 3 * ib + 2;
        const uint32_t oq = (uint32_t)(dq >> 2) * kUnitBytes + (dq & 3) * 4;
        const uint32_t ow = (uint32_t)(dw >> 2) * kUnitBytes + (dw & 3) * 4;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const uint32_t q = *reinterpret_cast<const uint32_t*>(wb + w_rowoff[j] + oq);
            const uint32_t w = *reinterpret_cast<const uint32_t*>(wb + w_rowoff[j] + ow);
            bop[j] = decode_group(sm.tbl, q, w, lg, sel0, sel1, rs);
        }
    };

    // X staging: piece tid + 256 i = row (tid >> 3) + 32 i, columns (tid & 7) * 8 .. +7
    const int xr = tid >> 3, xc = (tid & 7) * 8;
    const _Float16* xsrc[V][XP];
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
        for (int i = 0; i < XP; ++i)
            xsrc[v][i] = g.xh + (size_t)v * g.M * g.K + (size_t)min(m0 + xr + 32 * i, g.M - 1) * g.K + tl.b0 * kQK + xc;
    u32x4_t xreg[2][V][XP];
    auto load_x = [&](u32x4_t (&r)[V][XP], int s) {
#pragma unroll
        for (int v = 0; v < V; ++v)
#pragma unroll
            for (int i = 0; i < XP; ++i) r[v][i] = *reinterpret_cast<const u32x4_t*>(xsrc[v][i] + s * BK3);
    };
    auto store_x = [&](const u32x4_t (&r)[V][XP], int xb) {
#pragma unroll
        for (int v = 0; v < V; ++v)
#pragma unroll
            for (int i = 0; i < XP; ++i)
                *reinterpret_cast<u32x4_t*>(&sm.xs[xb][v][(xr + 32 * i) * kRow3 + xc]) = r[v][i];
    };
    // A operands of sub-block t of the stage in X buffer xb: [image][mt]
    auto read_a = [&](half8_t (&a)[V][MT], int xb, int t) {
#pragma unroll
        for (int v = 0; v < V; ++v)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                a[v][mt] = *reinterpret_cast<const half8_t*>(&sm.xs[xb][v][(mt * 16 + lr) * kRow3 + t * 32 + lg * 8]);
    };

    float4_t acc[MT][3], blk[MT][3];
    // per row: the sum of d - d over its blocks, 0 while every d is finite
    // and NaN after an infinite or NaN one; added at the end, it makes such
    // a row NaN, as the reference's sum of the block's +-inf products of
    // both signs does (d/4 times the finite partial would give +-inf)
    float pz[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const float4_t zero4 = {0.0f, 0.0f, 0.0f, 0.0f};

    const int nblk = tl.b1 - tl.b0;  // this split's blocks
    const int steps = nblk * (kQK / BK3);
    // Prologue: X stages 0, 1 in LDS (buffers 0, 1), stage 2 in registers,
    // W block 0 in LDS; then the A operands of stage 0's first sub-block and
    // the B operands of stage 0.
    load_w(0);
    load_x(xreg[0], 0);
    load_x(xreg[1], min(1, steps - 1));
    store_w(0);
    store_x(xreg[0], 0);
    store_x(xreg[1], 1);
    load_x(xreg[0], min(2, steps - 1));
    __syncthreads();  // table, W block 0, X stages 0 and 1
    half8_t a[2][V][MT];
    half8_t bop[2][2][3];  // [stage parity][t][j]
    read_a(a[0], 0, 0);
    decode_half(bop[0][0], 0, 0);
    decode_half(bop[0][1], 0, 1);

    // X buffer of stage s: s % 3. Stage s stores X(s + 2) into (s + 2) % 3,
    // the buffer of stage s - 1, whose last reads (its second sub-block)
    // happened before the previous stage's barrier.
    int xb0 = 0;
    for (int s0 = 0; s0 < steps; s0 += 4) {
        static_for<0, 4>([&](auto Uc) {
            constexpr int U = decltype(Uc)::value;
            const int s = s0 + U;
            const int c = s >> 2;  // block
            const int xb1 = xb0 == 2 ? 0 : xb0 + 1, xb2 = xb1 == 2 ? 0 : xb1 + 1;
            load_x(xreg[(U + 1) & 1], min(s + 3, steps - 1));
            if constexpr (U == 0) load_w(min(c + 1, nblk - 1));
            // sub-block 0: MFMAs on a[0]; meanwhile A of sub-block 1 and the
            // next stage's B operands of its sub-block 0
            read_a(a[1], xb0, 1);
            decode_half(bop[(U + 1) & 1][0], s + 1, 0);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int j = 0; j < 3; ++j)
#pragma unroll
                    for (int v = 0; v < V; ++v)
                        blk[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            a[0][v][mt], bop[U & 1][0][j], U == 0 && v == 0 ? zero4 : blk[mt][j], 0, 0, 0);
            // sub-block 1: MFMAs on a[1]; meanwhile A of the next stage's
            // sub-block 0 and its B operands of sub-block 1
            read_a(a[0], xb1, 0);
            decode_half(bop[(U + 1) & 1][1], s + 1, 1);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int j = 0; j < 3; ++j)
#pragma unroll
                    for (int v = 0; v < V; ++v)
                        blk[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1][v][mt], bop[U & 1][1][j],
                                                                             blk[mt][j], 0, 0, 0);
            if constexpr (U == 3) {
                // block complete: acc += d/4 * partial (column = this lane's row)
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const uint16_t dh = *reinterpret_cast<const uint16_t*>(&sm.wd[c & 1][d_off[j]]);
                    const float d4 = (float)__builtin_bit_cast(_Float16, dh) * 0.25f;
                    pz[j] += d4 - d4;
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[mt][j][i] = fmaf(d4, blk[mt][j][i], acc[mt][j][i]);
                }
            }
            store_x(xreg[U & 1], xb2);  // X(s + 2), loaded a stage ago
            if constexpr (U == 2) store_w((c + 1) & 1);
            __syncthreads();
            xb0 = xb1;
        });
    }
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][j] += pz[j];

    gemm_store<MT>(g, tl, acc, m0, n0, wave * 48, lr, (int)lg, tid, &sm.last_flag);
}


// ---------------------------------------------------------------------------
// GEMM, K-halves form (one X image: bf16 input; every bf16 X of more than
// 64 tokens). k_gemm3's workgroup tile (128 tokens x 192 W rows) on 512
// threads: wavefront w owns rows 48 (w & 3) .. +47 (3 column tiles of
// v_mfma_f32_16x16x32_f16, all 8 token tiles) over the blocks of K half
// kh = w >> 2, so every SIMD runs two wavefronts and every W value is still
// decoded once per workgroup.
//   * One accumulator per output: the partial of a 256-wide block is not
//     kept apart to be scaled by its d; the accumulator holds the sum in
//     units of a running d (the row's last nonzero one). When a block's d
//     differs, the accumulator is rescaled by d_old / d_new before the
//     block's MFMAs; the end multiplies by d/4. Products stay exact (B is
//     +-grid*(2s+1) in fp16); each change of d adds one rounding.
//   * Each K half has its own double-buffered rings in LDS, filled by its
//     own four wavefronts with copies straight from global memory
//     (global_load_lds_dwordx4): 64-column X stages (rows swizzled by
//     16-byte chunk) and W half blocks (units 0-2 or 3-5 of the three row
//     tiles, i.e. 4 sub-blocks) with the blocks' d. One workgroup barrier
//     per stage, which also waits for the copies.
//   * The B operands of a sub-block are decoded while the MFMAs of the
//     previous one run (W is in LDS a stage ahead, so the next stage's
//     operands are decoded before the barrier that ends this one), from a
//     grid table with 2s+1 folded in; rows whose block has d = 0 read a zero
//     row of the table.
//   * At the end the K half 1 wavefronts leave their sums in LDS, the K half
//     0 wavefronts add them (half 0 + half 1, fixed order) and lay the tile
//     out in LDS by rows, and all threads store it with 16-byte stores.

constexpr int BN5 = 192, BK5 = 64;
constexpr int kThreads5 = 512;
constexpr int kWHalf5 = 3 * 3 * kUnitBytes;      // 9 KiB: 3 row tiles x 3 units
constexpr int kTbl5 = 16 * 256 * 8;              // 32 KiB: the grid times every 2s+1
constexpr uint32_t kZeroEntry5 = kTbl5;          // 2 KiB of zeros after the scaled grid

// XS: bytes of one X stage (16 KiB: 128 image rows; 20 KiB: 160, the
// 80-token tiles of fp32 X)
constexpr int kXStageMax5 = 160 * BK5 * 2;
template <int XS>
struct GemmSmem5 {
    uint8_t tbl[kTbl5 + 2048];   // grid * (2s+1) as [s][idx], then a zero "scale"
    uint8_t xs[2][2][XS];        // [K half][buffer]
    uint8_t wb[2][2][kWHalf5];   // [K half][buffer]: [tile][unit][64 lanes x 16 B]
    uint8_t wd[2][2][1024];      // [K half][block parity]: [tile][64 fp16] (a whole wavefront's copy)
    int last_flag;
};

// Entry (idx, s) = 4 fp16 values grid(idx)[0..3] * (2s+1), at (s << 11) |
// (idx << 3): the bank of a lookup follows the index's low five bits, so
// the four lanes that decode one row (same s) spread like any others. Then
// 2 KiB of zeros (the row that zero-d blocks read). The table is device data
// built at compile time (every value is an integer below 2048, exact in
// fp16) and copied into LDS at a launch's start.
struct ScaledGrid5 {
    uint32_t w[(kTbl5 + 2048) / 4];
};
constexpr ScaledGrid5 make_scaled_grid5() {
    ScaledGrid5 t{};
    for (uint32_t s = 0; s < 16; ++s)
        for (uint32_t idx = 0; idx < 256; ++idx) {
            const uint32_t v = kIq3xxsGrid[idx], m = 2 * s + 1;
            const uint32_t o = ((s << 11) | (idx << 3)) / 4;
            t.w[o] = host_f16_of_small_uint((v & 255u) * m) |
                     ((uint32_t)host_f16_of_small_uint(((v >> 8) & 255u) * m) << 16);
            t.w[o + 1] = host_f16_of_small_uint(((v >> 16) & 255u) * m) |
                         ((uint32_t)host_f16_of_small_uint((v >> 24) * m) << 16);
        }
    return t;
}
__device__ __attribute__((aligned(16))) const ScaledGrid5 kScaledGrid5 = make_scaled_grid5();
static_assert((kTbl5 + 2048) % 1024 == 0, "whole 1 KiB pieces");

// A workgroup of NTHR threads copies the table into tbl with
// global_load_lds_dwordx4 (1 KiB per wavefront instruction); the copies
// complete at the caller's next barrier, like its other copies.
template <int NTHR>
__device__ __forceinline__ void scaled_grid_table5(uint8_t* tbl, int tid) {
    constexpr int kPieces = (kTbl5 + 2048) / 1024, kWaves = NTHR / 64;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t* src = reinterpret_cast<const uint8_t*>(&kScaledGrid5) + (tid & 63) * 16;
#pragma unroll
    for (int i = 0; i < (kPieces + kWaves - 1) / kWaves; ++i) {
        const int piece = wave + kWaves * i;
        if (piece < kPieces) __builtin_amdgcn_global_load_lds(src + piece * 1024, tbl + piece * 1024, 16, 0, 0);
    }
}

// B operand of v_mfma_f32_16x16x32_f16 for one lane: the 8 weights of group
// lg (columns 8lg..8lg+7 of a sub-block) of one W row, as fp16
// +-grid*(2s+1), from its grid-index word q (bytes p0, p0+1) and sign/scale
// word w, looked up in the [s][idx] table: the scale's 2 KiB row at (s << 11) comes from rotating w
// (whose top four bits are s) right by 17; a row with smask = 0, szero =
// kZeroEntry5 reads the zero row instead.
__device__ __forceinline__ half8_t decode_group5(const uint8_t* tbl, uint32_t q, uint32_t w, uint32_t lg,
                                                 uint32_t p0, uint32_t smask, uint32_t szero) {
    const uint32_t sw = t64_signs(w);
    const uint32_t wg = __builtin_amdgcn_alignbit(sw, sw, lg);
    const uint64_t sw2 = ((uint64_t)(wg >> 4) << 32) | wg;
    const uint64_t r01 = shl64<15>(sw2), r23 = shl64<7>(sw2);
    const uint32_t srow = (__builtin_amdgcn_alignbit(w, w, 17) & smask) | szero;
    const uint32_t i0 = __builtin_amdgcn_ubfe(q, 8 * p0, 8), i1 = __builtin_amdgcn_ubfe(q, 8 * p0 + 8, 8);
    const uint32_t a0 = (i0 << 3) | srow;
    const uint32_t a1 = (i1 << 3) | srow;
    const u32x2_t g0 = *reinterpret_cast<const u32x2_t*>(tbl + a0);
    const u32x2_t g1 = *reinterpret_cast<const u32x2_t*>(tbl + a1);
    const u32x4_t r = {((uint32_t)r01 & 0x80008000u) | g0.x, ((uint32_t)(r01 >> 32) & 0x80008000u) | g0.y,
                       ((uint32_t)r23 & 0x80008000u) | g1.x, ((uint32_t)(r23 >> 32) & 0x80008000u) | g1.y};
    return __builtin_bit_cast(half8_t, r);
}

// decode_group5 in two halves, so that a software pipeline can put an LDS
// round trip between them: the table addresses of the group's two entries
// (from the index word q and the sign/scale word w), then the B operand from
// the two entries read there and w's signs.
__device__ __forceinline__ void group5_addr(uint32_t q, uint32_t w, uint32_t p0, uint32_t smask, uint32_t szero,
                                            uint32_t& a0, uint32_t& a1) {
    const uint32_t srow = (__builtin_amdgcn_alignbit(w, w, 17) & smask) | szero;
    a0 = (__builtin_amdgcn_ubfe(q, 8 * p0, 8) << 3) | srow;
    a1 = (__builtin_amdgcn_ubfe(q, 8 * p0 + 8, 8) << 3) | srow;
}
__device__ __forceinline__ half8_t group5_signed(u32x2_t g0, u32x2_t g1, uint32_t w, uint32_t lg) {
    const uint32_t sw = t64_signs(w);
    const uint32_t wg = __builtin_amdgcn_alignbit(sw, sw, lg);
    const uint64_t sw2 = ((uint64_t)(wg >> 4) << 32) | wg;
    const uint64_t r01 = shl64<15>(sw2), r23 = shl64<7>(sw2);
    const u32x4_t r = {((uint32_t)r01 & 0x80008000u) | g0.x, ((uint32_t)(r01 >> 32) & 0x80008000u) | g0.y,
                       ((uint32_t)r23 & 0x80008000u) | g1.x, ((uint32_t)(r23 >> 32) & 0x80008000u) | g1.y};
    return __builtin_bit_cast(half8_t, r);
}

// MT token tiles of V images each (MT * V = 8: bf16 X, 128 tokens, one
// image; fp32 X, 64 tokens, hi and lo images): the X stage, the A reads per
// sub-block and the MFMAs per decoded B operand are the same for both.
template <int MT, int V>
__global__ __launch_bounds__(kThreads5) void k_gemm5(GemmArgs g_all) {
    static_assert(MT * V >= 4 && MT * V <= 10 && MT * V % 2 == 0, "an 8 to 20 KiB X stage");
    constexpr int BM = 16 * MT;   // tokens per tile
    constexpr int JT = 3;         // column tiles per wavefront
    constexpr int XS = MT * V * 16 * BK5 * 2;  // one X stage: V images of BM rows x 64 columns
    constexpr int XP = MT * V / 2;              // its 1 KiB pieces per wavefront of a K half
    // (one layout, sized for the larger stage, for every instantiation: an
    // array bound or a __shared__ variable's type that depends on MT and V
    // here drops the kernel's host-side stub)
    __shared__ __attribute__((aligned(16))) GemmSmem5<kXStageMax5> sm;
    static_assert(XS <= kXStageMax5 && XP <= 5, "X stage");
    // the K half 1 sums overlay xs and wb
    static_assert(4 * MT * JT * 64 * 16 <= 2 * 2 * kXStageMax5 + 2 * 2 * kWHalf5, "reduction area");

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rq = wave & 3, kh = wave >> 2;
    const uint32_t lane = tid & 63;
    const int lr = lane & 15;
    const uint32_t lg = lane >> 4;

    GemmTile tl;
    int tn;
    GemmArgs g;
    // X rows [xrow0, xrow0 + g.M) of images of xplane rows each (tokmap:
    // row tokmap[m] for the tile's row m instead)
    int xrow0 = 0, xplane = g_all.M;
    const int* tokmap = nullptr;
    if (!g_all.grp_eptr) {
        GemmArgs ga = g_all;
        int bid = blockIdx.x;
        if (g_all.p2.wg0 > 0 && bid >= g_all.p2.wg0) {  // uniform: the second problem
            const GemmProb& q = g_all.p2;
            ga.w = q.w;
            ga.xh = q.xh;
            ga.unscale = q.unscale;
            ga.y = q.y;
            ga.N = q.N;
            ga.K = q.K;
            ga.nb = q.nb;
            ga.tiles_n = q.tiles_n;
            ga.ks = q.ks;
            ga.cnt = q.cnt;
            ga.part = q.part;
            ga.w2 = q.w2;
            ga.y2 = q.y2;
            ga.N2 = q.N2;
            ga.tiles_n1 = q.tiles_n1;
            bid -= q.wg0;
        }
        tl = gemm_tile(ga, bid);
        if (tl.tm >= ga.tiles_m || tl.tn >= ga.tiles_n) return;  // uniform
        g = gemm_tensor(ga, tl, tn);
    } else {
        // grouped: entry id / tiles_n of the expert tile table, result tile
        // id % tiles_n of that expert's rows (one K split)
        const int id = blockIdx.x / g_all.tiles_n;
        tl.tn = blockIdx.x - id * g_all.tiles_n;
        if (id >= *g_all.grp_count) return;  // uniform
        const int ent = g_all.grp_tile[id];
        const int e = ent >> 16;
        tl.tm = ent & 0xFFFF;
        tl.kz = 0;
        tl.b0 = 0;
        tl.b1 = g_all.nb;
        g = gemm_tensor(g_all, tl, tn);
        const bool sh = e == g_all.grp_sh_e;
        xrow0 = min(max(g_all.grp_eptr[e], 0), g_all.grp_rows);
        xplane = g_all.grp_rows;
        g.M = (sh ? min(xrow0 + g_all.grp_sh_rows, g_all.grp_rows) : min(g_all.grp_eptr[e + 1], g_all.grp_rows)) -
              xrow0;
        if (g.M <= tl.tm * BM) return;  // uniform: no rows of this tile
        if (sh)
            g.w = tl.tn >= g_all.tiles_n1 ? g_all.grp_w2_sh : g_all.grp_w_sh;
        else
            g.w += (size_t)e * g_all.grp_w_stride;
        g.y += (size_t)xrow0 * g.N;
        if (g_all.grp_tok) {
            xplane = g_all.grp_img_rows;
            if (sh) {
                g.M = min(g.M, xplane);
                xrow0 = 0;  // the shared expert's slot m is token m
            } else {
                tokmap = g_all.grp_tok + xrow0;
            }
        } else {
            g.unscale += xrow0;
        }
    }
    const int m0 = tl.tm * BM, n0 = tn * BN5;
    const int last_tile = (g.N + kTileRows - 1) / kTileRows - 1;

    // K halves: blocks [b0 + kh * nh, ...) of this split, nh per half (the
    // second half of an odd count has one block fewer: its last block is
    // loaded clamped and contributes zeros)
    const int nblk = tl.b1 - tl.b0;
    const int nh = (nblk + 1) >> 1;
    const int kb0 = tl.b0 + kh * nh;
    const int steps = nh * (kQK / BK5);
    auto blk_of = [&](int c) { return min(kb0 + c, tl.b1 - 1); };

    // Loads go straight from global memory into LDS (global_load_lds_dwordx4:
    // lane i of a wavefront writes the 16 bytes at the destination + 16 i),
    // issued at a stage's start and complete at its closing barrier.
    // X: the stage's V images of BM rows x 64 columns are 4 XP pieces of 8
    // rows (piece p: image p / (2 MT), rows 8 (p % (2 MT)) ..); wavefront rq
    // of the K half copies pieces rq + 4 i. Lane l of a piece fills LDS
    // chunk l & 7 of row l >> 3 with global chunk (l & 7) ^ (row & 7), the
    // swizzle the A reads undo. (Byte offsets from xh: the images are under
    // 4 GiB, as the launch checks.)
    uint32_t xsrc[5];  // XP of them
#pragma unroll
    for (int i = 0; i < XP; ++i) {
        const int p = rq + 4 * i, v = p / (2 * MT);
        const int r = 8 * (p % (2 * MT)) + (int)(lane >> 3);
        const int mr = min(m0 + r, g.M - 1);
        const int xr = tokmap ? min(max(tokmap[mr], 0), xplane - 1) : xrow0 + mr;
        xsrc[i] = ((uint32_t)v * (uint32_t)xplane * (uint32_t)g.K + (uint32_t)xr * (uint32_t)g.K) * 2u +
                  (((lane & 7u) ^ (lane >> 3)) << 4);
    }
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(g.xh);
    // X stage s (past the last: the last one's columns again) into buffer s & 1
    auto load_x = [&](int s) {
        const int sc = min(s, steps - 1);
        const uint32_t kc = (uint32_t)(blk_of(sc >> 2) * kQK + (sc & 3) * BK5) * 2u;
        uint8_t* dst = sm.xs[kh][s & 1];
#pragma unroll
        for (int i = 0; i < XP; ++i)
            __builtin_amdgcn_global_load_lds(xbase + (xsrc[i] + kc), dst + (rq + 4 * i) * 1024, 16, 0, 0);
    };
    // W half block hb (block hb >> 1, units 3 (hb & 1) .. +2 of the three row
    // tiles: 9 units of 1 KiB): wavefront rq copies units rq + 4 k; at a
    // block's first half, wavefront 3 also copies the tiles' d (lanes 0..23;
    // the other lanes repeat lane 23's piece).
    uint32_t wsrc[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int ui = min(rq + 4 * k, 8);
        const int tile = min(n0 / kTileRows + ui / 3, last_tile);
        wsrc[k] = (uint32_t)tile * (uint32_t)g.nb * kRecordBytes + (ui % 3) * kUnitBytes + lane * 16u;
    }
    const uint32_t dl = min(lane, 23u);
    const uint32_t dsrc = (uint32_t)min(n0 / kTileRows + (int)(dl >> 3), last_tile) * (uint32_t)g.nb * kRecordBytes +
                          kRecordDOffset + (dl & 7u) * 16u;
    // (past the last half block: the last block's units again)
    auto load_w = [&](int hb) {
        const uint32_t boff = (uint32_t)blk_of(min(hb, 2 * nh - 1) >> 1) * kRecordBytes;
        const uint32_t hoff = (uint32_t)(hb & 1) * 3 * kUnitBytes;
        uint8_t* dst = sm.wb[kh][hb & 1];
#pragma unroll
        for (int k = 0; k < 3; ++k)
            if (rq + 4 * k < 9)
                __builtin_amdgcn_global_load_lds(g.w + (wsrc[k] + boff + hoff), dst + (rq + 4 * k) * 1024, 16, 0, kWNt);
        if ((hb & 1) == 0 && rq == 3)
            __builtin_amdgcn_global_load_lds(g.w + (dsrc + boff), &sm.wd[0][0][0] + (kh * 2 + ((hb >> 1) & 1)) * 1024,
                                             16, 0, kWNt);
    };

    // this lane's rows j < JT: lane slot in the staged half block, and d
    const uint8_t* wrow[JT];
    uint32_t d_off[JT];
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const int r = rq * 48 + j * 16 + lr;
        wrow[j] = &sm.wb[kh][0][0] + (r >> 6) * 3 * kUnitBytes + (r & 63) * 16;
        d_off[j] = (uint32_t)(r >> 6) * 128u + (uint32_t)(r & 63) * 2u;
    }
    const uint32_t p0 = 2 * (lg & 1);
    const bool hiq = lg >= 2;
    const uint8_t* arow = &sm.xs[kh][0][0] + lr * 128;
    // A operand chunk of sub-block t (of 2 per stage), swizzled
    uint32_t a_off[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) a_off[t] = (uint32_t)((t * 4 + (int)lg) ^ (lr & 7)) << 4;

    float4_t acc[MT][JT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float dcur[JT], dnext[JT];
    // per row: the sum of d - d over its blocks (0 while every d is finite,
    // NaN after an infinite or NaN one), added at the end: such a row is
    // NaN, as the reference's sum of the block's +-inf products of both
    // signs is (the running-d rescale alone would give +-inf or 0)
    float pz[JT];
#pragma unroll
    for (int j = 0; j < JT; ++j) pz[j] = 0.0f;
    uint32_t amask[JT], azero[JT];

    // block c's d per row (0 past this half's blocks): the table masks for
    // its decode, and dnext
    auto block_d = [&](int c) {
        const bool live = kb0 + c < tl.b1;
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const float dn =
                live ? (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(&sm.wd[kh][c & 1][d_off[j]]))
                     : 0.0f;
            const bool z = dn == 0.0f;
            amask[j] = z ? 0u : 0x7800u;
            azero[j] = z ? kZeroEntry5 : 0u;
            dnext[j] = dn;
            pz[j] += dn - dn;
        }
    };
    // the accumulators move to the units of dnext where it is nonzero and differs
    auto rescale = [&]() {
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const bool change = dnext[j] != 0.0f && dnext[j] != dcur[j];
            const float r = change ? dcur[j] * __builtin_amdgcn_rcpf(dnext[j]) : 1.0f;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][j] *= r;
            dcur[j] = change ? dnext[j] : dcur[j];
        }
    };
    // The B operands go through a three-step software pipeline, one step per
    // sub-block, so that neither of a decode's two LDS round trips stalls the
    // MFMAs: while sub-block i's MFMAs run, the grid entries of sub-block
    // i + 1 arrive (their addresses were made under sub-block i - 1) and
    // become its B operands, and the index and sign/scale words of sub-block
    // i + 2 arrive and become its table addresses. Each sub-block first
    // issues all of its LDS reads (A operands, entries, words), then the
    // MFMAs and the VALU work that consumes the reads.
    uint32_t pq[JT], pw[JT];            // words of sub-block i + 2
    uint32_t ad0[JT], ad1[JT], aw[JT];  // entry addresses and sign/scale words of sub-block i + 1
    // the index and sign/scale words of sub-block ib (0..7) of a block from W buffer `buf`
    auto read_words = [&](int buf, int ib) {
        const int lib = ib & 3;  // inside the half block
        const int dq = 3 * lib + (hiq ? 1 : 0), dw = 3 * lib + 2;
        const int oq = buf * kWHalf5 + (dq >> 2) * kUnitBytes + (dq & 3) * 4;
        const int ow = buf * kWHalf5 + (dw >> 2) * kUnitBytes + (dw & 3) * 4;
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            pq[j] = *reinterpret_cast<const uint32_t*>(wrow[j] + oq);
            pw[j] = *reinterpret_cast<const uint32_t*>(wrow[j] + ow);
        }
    };
    // the words just read -> table addresses (with the masks of their block)
    auto addresses = [&]() {
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            group5_addr(pq[j], pw[j], p0, amask[j], azero[j], ad0[j], ad1[j]);
            aw[j] = pw[j];
        }
    };

    // prologue: X stage 0 and W half block 0 (with block 0's d) in LDS;
    // block 0's d, the B operands of its first sub-block and the table
    // addresses of its second
    load_x(0);
    load_w(0);
    // the table is copied with the first stages
    scaled_grid_table5<kThreads5>(sm.tbl, tid);
    __syncthreads();  // table, X stage 0, W half block 0 with block 0's d
    block_d(0);
#pragma unroll
    for (int j = 0; j < JT; ++j) dcur[j] = dnext[j];  // the accumulators are zero
    half8_t bop[2][JT];
    read_words(0, 0);
    addresses();
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const u32x2_t g0 = *reinterpret_cast<const u32x2_t*>(sm.tbl + ad0[j]);
        const u32x2_t g1 = *reinterpret_cast<const u32x2_t*>(sm.tbl + ad1[j]);
        bop[0][j] = group5_signed(g0, g1, aw[j], lg);
    }
    read_words(0, 1);
    addresses();

    // Stage s: the loads of X(s + 1) (and at a half block's first stage of
    // W(hb + 1)) into the buffers last read in stage s - 1, before its
    // barrier; then its two sub-blocks, each as above. Sub-block i + 2 lies
    // in stage s + 1, whose W half block is in LDS already; the words of a
    // block's first two sub-blocks take the masks of that block's d (read
    // under the previous block's seventh sub-block). Past the last stage the
    // same steps run on clamped blocks (zero-d masks) and their results go
    // unused, so a stage has no branch.
    for (int c = 0; c < nh; ++c) {
        static_for<0, 4>([&](auto Uc) {
            constexpr int U = decltype(Uc)::value;
            const int s = 4 * c + U;
            load_x(s + 1);
            if constexpr ((U & 1) == 0) load_w((s >> 1) + 1);
            const uint8_t* xa = arow + (s & 1) * kXStageMax5;  // the buffers' stride
            static_for<0, 2>([&](auto tc) {
                constexpr int t = decltype(tc)::value;
                half8_t a[MT][V];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int v = 0; v < V; ++v)
                        a[mt][v] = *reinterpret_cast<const half8_t*>(xa + v * BM * 128 + mt * 16 * 128 + a_off[t]);
                u32x2_t g0[JT], g1[JT];
#pragma unroll
                for (int j = 0; j < JT; ++j) {
                    g0[j] = *reinterpret_cast<const u32x2_t*>(sm.tbl + ad0[j]);
                    g1[j] = *reinterpret_cast<const u32x2_t*>(sm.tbl + ad1[j]);
                }
                read_words(((s + 1) >> 1) & 1, (2 * U + 2 + t) & 7);
                __builtin_amdgcn_sched_barrier(0);  // every LDS read above issues before the MFMAs
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int j = 0; j < JT; ++j)
#pragma unroll
                        for (int v = 0; v < V; ++v)
                            acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][v], bop[t][j], acc[mt][j], 0, 0, 0);
#pragma unroll
                for (int j = 0; j < JT; ++j) bop[t ^ 1][j] = group5_signed(g0[j], g1[j], aw[j], lg);
                if constexpr (U == 3 && t == 0) block_d(c + 1);
                addresses();
            });
            if constexpr (U == 3) {
                if (c + 1 < nh) rescale();
            }
            __syncthreads();
        });
    }
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const float f = dcur[j] * 0.25f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][j] = acc[mt][j] * f + pz[j];
    }
    // K half 1 -> LDS (over xs and wb, free after the last barrier); K half 0 adds
    float4_t* red = reinterpret_cast<float4_t*>(&sm.xs[0][0][0]) + (size_t)rq * (MT * JT * 64) + lane;
    if (kh == 1) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < JT; ++j) red[(mt * JT + j) * 64] = acc[mt][j];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < JT; ++j) acc[mt][j] += red[(mt * JT + j) * 64];
    }
    // The K half 0 wavefronts leave the tile in LDS as rows of 192 floats
    // (stride 196: the four token rows a store instruction touches fall on
    // different banks), then every thread copies whole rows out 16 bytes at
    // a time: one K split, Y times the token's unscale; several, this
    // split's partial as write-through stores (cache policy sc1, agent
    // scope) for the split-K sum.
    constexpr int kTStride = BN5 + 4;
    static_assert(BM * kTStride * 4 <= 2 * 2 * kXStageMax5 + 2 * 2 * kWHalf5, "output tile area");
    float* tile = reinterpret_cast<float*>(&sm.xs[0][0][0]);
    __syncthreads();  // the K half 1 sums are read
    if (kh == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < JT; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    tile[(mt * 16 + (int)lg * 4 + i) * kTStride + rq * 48 + j * 16 + lr] = acc[mt][j][i];
    }
    __syncthreads();
    const int rows = min(BM, g.M - m0), cols = min(BN5, g.N - n0);
    if (g.ks > 1) {
        const int tile_id = tl.tm * g.tiles_n + tl.tn;
        float* mine = g.part + ((size_t)tile_id * g.ks + tl.kz) * (BM * kTileN);
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(mine, 0, BM * kTileN * 4, 0x00020000);
        for (int f = tid; f < rows * (BN5 / 4); f += kThreads5) {
            const int m = f / (BN5 / 4), c4 = (f - m * (BN5 / 4)) * 4;
            if (c4 >= cols) continue;
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&tile[m * kTStride + c4]);
            __builtin_amdgcn_raw_buffer_store_b128(v, rs, (uint32_t)((m * kTileN + c4) * 4), 0, 16);
        }
        gemm_split_finish<BM, kTileN, kThreads5>(g, tl, m0, n0, tid, &sm.last_flag);
        return;
    }
    const bool vec = (g.N & 3) == 0 && (reinterpret_cast<uintptr_t>(g.y) & 15u) == 0;
    for (int f = tid; f < rows * (BN5 / 4); f += kThreads5) {
        const int m = f / (BN5 / 4), c4 = (f - m * (BN5 / 4)) * 4;
        if (c4 >= cols) continue;
        const float us = tokmap ? g.unscale[min(max(tokmap[m0 + m], 0), xplane - 1)] : g.unscale[m0 + m];
        const float4 v = *reinterpret_cast<const float4*>(&tile[m * kTStride + c4]);
        float* yrow = g.y + (size_t)(m0 + m) * g.N + n0 + c4;
        if (vec && c4 + 4 <= cols) {
            *reinterpret_cast<float4*>(yrow) = float4{v.x * us, v.y * us, v.z * us, v.w * us};
        } else {
            const float o[4] = {v.x * us, v.y * us, v.z * us, v.w * us};
            for (int e = 0; e < 4 && c4 + e < cols; ++e) yrow[e] = o[e];
        }
    }
}

// ---------------------------------------------------------------------------
// GEMM, 32x32 form (one K split; bf16 X, or fp32 X as two images). A
// 512-thread workgroup computes 128 / V tokens x 256 W rows (four T64 row
// tiles) with v_mfma_f32_32x32x16_f16: a single wavefront keeps that
// instruction's pipe nearly full and leaves room for four VALU instructions
// per MFMA, where v_mfma_f32_16x16x32_f16 needs two wavefronts and no VALU
// to come close. Wavefront w owns row tile rg = w & 3 (two 32-row B tiles)
// for all tokens over the blocks of K half kh = w >> 2; each decoded group of
// 8 weights (one per lane and B tile) feeds 4 MFMAs of 32 x 32 x 16. The
// rest follows k_gemm5: accumulators in units of the row's running d,
// per-K-half LDS rings filled by global_load_lds_dwordx4 (X stages swizzled
// by 16-byte chunk, W half blocks with the blocks' d), the next K step's B
// operands decoded under the current MFMAs, one barrier per 64-column
// stage, and at the end the K halves added in LDS and the tile stored as
// whole rows.
//
// Operand layouts of v_mfma_f32_32x32x16_f16 (lane l): A holds token l & 31
// of a 32-token tile at K elements 8 (l >> 5) .. +7; B holds W row l & 31 of
// a 32-row tile at the same K elements; the 16 results of lane l are W row
// l & 31, tokens 8 (i >> 2) + 4 (l >> 5) + (i & 3) for i < 16.

constexpr int BN6 = 256, BK6 = 64;
constexpr int kThreads6 = 512;
constexpr int kXStage6 = 128 * BK6 * 2;          // 16 KiB: 128 rows (all images) x 128 bytes
constexpr int kWHalf6 = 4 * 3 * kUnitBytes;      // 12 KiB: 4 row tiles x 3 units
constexpr int kTStride6 = BN6 + 4;               // output tile row stride (floats)

typedef float float16_t __attribute__((ext_vector_type(16)));

struct GemmSmem6 {
    // tbl, xs and wb are contiguous: after the main loop they hold the K
    // half 1 sums, then the output tile
    uint8_t tbl[kTbl5 + 2048];   // grid * (2s+1) as [s][idx], then a zero "scale"
    uint8_t xs[2][2][kXStage6];  // [K half][buffer]
    uint8_t wb[2][2][kWHalf6];   // [K half][buffer]: [tile][unit][64 lanes x 16 B]
    uint8_t wd[2][2][1024];      // [K half][block parity]: [tile][64 fp16] (a whole wavefront's copy)
};
static_assert(kTbl5 + 2048 + 2 * 2 * kXStage6 + 2 * 2 * kWHalf6 >= 128 * kTStride6 * 4, "output tile area");
static_assert(kTbl5 + 2048 + 2 * 2 * kXStage6 + 2 * 2 * kWHalf6 >= 4 * 128 * 64 * 4, "K half 1 sums");

template <int V>
__global__ __launch_bounds__(kThreads6) void k_gemm6(GemmArgs g_all) {
    constexpr int BM = 128 / V;   // tokens per tile
    constexpr int MT = BM / 32;   // 32-token A tiles per image
    constexpr int JT = 2;         // 32-row B tiles per wavefront
    __shared__ __attribute__((aligned(16))) GemmSmem6 sm;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wave & 3, kh = wave >> 2;
    const uint32_t lane = tid & 63;
    const int l32 = lane & 31;
    const uint32_t hk = lane >> 5;  // which 8 of a K step's 16 elements

    const GemmTile tl = gemm_tile(g_all, blockIdx.x);
    if (tl.tm >= g_all.tiles_m || tl.tn >= g_all.tiles_n) return;  // uniform
    int tn;
    const GemmArgs g = gemm_tensor(g_all, tl, tn);
    const int m0 = tl.tm * BM, n0 = tn * BN6;
    const int last_tile = (g.N + kTileRows - 1) / kTileRows - 1;

    const int nblk = tl.b1 - tl.b0;
    const int nh = (nblk + 1) >> 1;
    const int kb0 = tl.b0 + kh * nh;
    const int steps = nh * (kQK / BK6);
    auto blk_of = [&](int c) { return min(kb0 + c, tl.b1 - 1); };

    // X: the stage's V images of BM rows x 64 columns are 16 pieces of 8 rows
    // (piece p: image p / (BM / 8), rows 8 (p % (BM / 8)) ..); wavefront rg of
    // the K half copies pieces rg + 4 i, lane l into LDS chunk l & 7 of row
    // l >> 3 from global chunk (l & 7) ^ (row & 7).
    uint32_t xsrc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = rg + 4 * i, v = p / (BM / 8);
        const int r = 8 * (p % (BM / 8)) + (int)(lane >> 3);
        xsrc[i] = ((uint32_t)v * (uint32_t)g.M * (uint32_t)g.K + (uint32_t)min(m0 + r, g.M - 1) * (uint32_t)g.K) * 2u +
                  (((lane & 7u) ^ (lane >> 3)) << 4);
    }
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(g.xh);
    auto load_x = [&](int s) {
        const int sc = min(s, steps - 1);
        const uint32_t kc = (uint32_t)(blk_of(sc >> 2) * kQK + (sc & 3) * BK6) * 2u;
        uint8_t* dst = sm.xs[kh][s & 1];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(xbase + (xsrc[i] + kc), dst + (rg + 4 * i) * 1024, 16, 0, 0);
    };
    // W half block hb: wavefront rg copies the three units of row tile rg; at
    // a block's first half, wavefront 3 also copies the four tiles' d (lanes
    // 0..31; the others repeat lane 31's piece).
    const int wtile = min(n0 / kTileRows + rg, last_tile);
    const uint32_t wsrc = (uint32_t)wtile * (uint32_t)g.nb * kRecordBytes + lane * 16u;
    const uint32_t dl = min(lane, 31u);
    const uint32_t dsrc = (uint32_t)min(n0 / kTileRows + (int)(dl >> 3), last_tile) * (uint32_t)g.nb * kRecordBytes +
                          kRecordDOffset + (dl & 7u) * 16u;
    auto load_w = [&](int hb) {
        const uint32_t boff = (uint32_t)blk_of(min(hb, 2 * nh - 1) >> 1) * kRecordBytes;
        const uint32_t hoff = (uint32_t)(hb & 1) * 3 * kUnitBytes;
        uint8_t* dst = &sm.wb[0][0][0] + (kh * 2 + (hb & 1)) * kWHalf6 + rg * 3 * kUnitBytes;
#pragma unroll
        for (int k = 0; k < 3; ++k)
            __builtin_amdgcn_global_load_lds(g.w + (wsrc + boff + hoff + k * kUnitBytes), dst + k * kUnitBytes, 16, 0, 0);
        if ((hb & 1) == 0 && rg == 3)
            __builtin_amdgcn_global_load_lds(g.w + (dsrc + boff), &sm.wd[0][0][0] + (kh * 2 + ((hb >> 1) & 1)) * 1024,
                                             16, 0, 0);
    };

    // this lane's rows j < JT (row l32 of B tile j of row tile rg): lane slot
    // in the staged half block, and d
    const uint8_t* wrow[JT];
    uint32_t d_off[JT];
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const int r = j * 32 + l32;  // inside row tile rg
        wrow[j] = &sm.wb[kh][0][0] + rg * 3 * kUnitBytes + r * 16;
        d_off[j] = (uint32_t)rg * 128u + (uint32_t)r * 2u;
    }
    const uint32_t p0 = 2 * hk;  // the group's grid indices: bytes p0, p0 + 1 of its index word
    const uint8_t* arow = &sm.xs[kh][0][0] + l32 * 128;

    float16_t acc[MT][JT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j) acc[i][j] = float16_t{};
    float dcur[JT], dnext[JT];
    // per row: the sum of d - d over its blocks (0 while every d is finite,
    // NaN after an infinite or NaN one), added at the end: such a row is
    // NaN, as the reference's sum of the block's +-inf products of both
    // signs is (the running-d rescale alone would give +-inf or 0)
    float pz[JT];
#pragma unroll
    for (int j = 0; j < JT; ++j) pz[j] = 0.0f;
    uint32_t smask[JT], szero[JT];

    auto block_d = [&](int c) {
        const bool live = kb0 + c < tl.b1;
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const float dn =
                live ? (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(&sm.wd[kh][c & 1][d_off[j]]))
                     : 0.0f;
            const bool z = dn == 0.0f;
            smask[j] = z ? 0u : 0x7800u;
            szero[j] = z ? kZeroEntry5 : 0u;
            dnext[j] = dn;
            pz[j] += dn - dn;
        }
    };
    auto rescale = [&]() {
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const bool change = dnext[j] != 0.0f && dnext[j] != dcur[j];
            const float r = change ? dcur[j] * __builtin_amdgcn_rcpf(dnext[j]) : 1.0f;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][j] *= r;
            dcur[j] = change ? dnext[j] : dcur[j];
        }
    };
    // B operands of K step ks (0..15) of a block (sub-block ks >> 1, group
    // 2 (ks & 1) + hk) from W buffer `buf`
    auto decode = [&](half8_t (&bop)[JT], int buf, int ks) {
        const int lib = (ks >> 1) & 3;  // sub-block inside the half block
        const int dq = 3 * lib + (ks & 1), dw = 3 * lib + 2;
        const int oq = buf * kWHalf6 + (dq >> 2) * kUnitBytes + (dq & 3) * 4;
        const int ow = buf * kWHalf6 + (dw >> 2) * kUnitBytes + (dw & 3) * 4;
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const uint32_t q = *reinterpret_cast<const uint32_t*>(wrow[j] + oq);
            const uint32_t w = *reinterpret_cast<const uint32_t*>(wrow[j] + ow);
            bop[j] = decode_group5(sm.tbl, q, w, 2 * (ks & 1) + hk, p0, smask[j], szero[j]);
        }
    };

    load_x(0);
    load_w(0);
    scaled_grid_table5<kThreads6>(sm.tbl, tid);
    __syncthreads();  // table, X stage 0, W half block 0 with block 0's d
    block_d(0);
#pragma unroll
    for (int j = 0; j < JT; ++j) dcur[j] = dnext[j];
    half8_t bop[2][JT];
    decode(bop[0], 0, 0);

    // Stage s (64 columns, K steps 4 (s & 3) .. +3 of its block): the copies
    // of X(s + 1) and, at a half block's first stage, W(hb + 1); four K
    // steps of MFMAs, each with the next K step's B operands decoded under it
    // (after a block's last step, with the next block's d). Past the last
    // stage the same steps run on clamped blocks and their results go unused.
    for (int c = 0; c < nh; ++c) {
        static_for<0, 4>([&](auto Uc) {
            constexpr int U = decltype(Uc)::value;
            const int s = 4 * c + U;
            load_x(s + 1);
            if constexpr ((U & 1) == 0) load_w((s >> 1) + 1);
            const uint8_t* xa = arow + (s & 1) * kXStage6;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int ks = 4 * U + k;  // K step inside the block
                const int cur = k & 1;
                if (ks < 15) {
                    decode(bop[cur ^ 1], ((ks + 1) >> 3) & 1, ks + 1);
                } else {
                    block_d(c + 1);
                    decode(bop[cur ^ 1], 0, 0);  // next block, first half (buffer 0)
                }
                const uint32_t ac = (uint32_t)(((2 * k + (int)hk) ^ (l32 & 7)) << 4);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    half8_t a[V];
#pragma unroll
                    for (int v = 0; v < V; ++v)
                        a[v] = *reinterpret_cast<const half8_t*>(xa + v * BM * 128 + mt * 32 * 128 + ac);
#pragma unroll
                    for (int j = 0; j < JT; ++j)
#pragma unroll
                        for (int v = 0; v < V; ++v)
                            acc[mt][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[v], bop[cur][j], acc[mt][j], 0, 0, 0);
                }
            }
            if constexpr (U == 3) {
                if (c + 1 < nh) rescale();
            }
            __syncthreads();
        });
    }
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const float f = dcur[j] * 0.25f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][j] = acc[mt][j] * f + pz[j];
    }
    // K half 1 -> LDS (over tbl, xs and wb, free after the last barrier); K half 0 adds
    float4* red = reinterpret_cast<float4*>(&sm.tbl[0]) + (size_t)rg * (MT * JT * 4 * 64) + lane;
    if (kh == 1) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < JT; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    red[((mt * JT + j) * 4 + q) * 64] =
                        float4{acc[mt][j][4 * q], acc[mt][j][4 * q + 1], acc[mt][j][4 * q + 2], acc[mt][j][4 * q + 3]};
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < JT; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 o = red[((mt * JT + j) * 4 + q) * 64];
                    acc[mt][j][4 * q] += o.x;
                    acc[mt][j][4 * q + 1] += o.y;
                    acc[mt][j][4 * q + 2] += o.z;
                    acc[mt][j][4 * q + 3] += o.w;
                }
    }
    __syncthreads();  // the K half 1 sums are read
    // the tile as rows of 256 floats (stride 260), then whole rows out
    float* tile = reinterpret_cast<float*>(&sm.tbl[0]);
    if (kh == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < JT; ++j)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    tile[(mt * 32 + 8 * (i >> 2) + 4 * (int)hk + (i & 3)) * kTStride6 + rg * 64 + j * 32 + l32] =
                        acc[mt][j][i];
    }
    __syncthreads();
    const int rows = min(BM, g.M - m0), cols = min(BN6, g.N - n0);
    const bool vec = (g.N & 3) == 0 && (reinterpret_cast<uintptr_t>(g.y) & 15u) == 0;
    for (int f = tid; f < rows * (BN6 / 4); f += kThreads6) {
        const int m = f / (BN6 / 4), c4 = (f - m * (BN6 / 4)) * 4;
        if (c4 >= cols) continue;
        const float us = g.unscale[m0 + m];
        const float4 v = *reinterpret_cast<const float4*>(&tile[m * kTStride6 + c4]);
        float* yrow = g.y + (size_t)(m0 + m) * g.N + n0 + c4;
        if (vec && c4 + 4 <= cols) {
            *reinterpret_cast<float4*>(yrow) = float4{v.x * us, v.y * us, v.z * us, v.w * us};
        } else {
            const float o[4] = {v.x * us, v.y * us, v.z * us, v.w * us};
            for (int e = 0; e < 4 && c4 + e < cols; ++e) yrow[e] = o[e];
        }
    }
}

}  // namespace

// K splits per result tile: one when the tiles fill half the CUs, else
// enough to fill them (at most 8, at least one block per split).
// Token rows per result tile: 128 for bf16 X of more than 64 tokens, else 64
// (fp32 X: two images per token; at most 64 tokens: no padding).
int gemm_tile_m(int M, int x_bf16) { return x_bf16 && M > 64 ? 128 : 64; }

// k_gemm5 / k_gemm6 (K halves inside the workgroup, two wavefronts per
// SIMD) take bf16 X of more than 64 tokens and fp32 X; their X offsets are
// 32-bit. k_gemm6 (v_mfma_f32_32x32x16_f16, 256-row tiles) runs where its
// tiles cover every CU, k_gemm5 (16x16x32, 192-row tiles) elsewhere.
// Measured at 12288 x 6144: 512 tokens, k_gemm5 97.6-103 us (k_gemm6, on
// 192 of 256 CUs, 110 us; k_gemm3 126-130 us); 2048 tokens, k_gemm6 333 us,
// k_gemm5 344 us, a 384-row 8-wavefront form with the full K per wavefront
// (removed) 356 us.
static bool gemm_halves(int M, int x_bf16, int K) {
    return (x_bf16 ? M > 64 : true) && (size_t)(x_bf16 ? 1 : 2) * M * (size_t)K * 2 < (1ull << 32);
}

int gemm_splits(int M, int N, int K, int num_cus, int x_bf16, int tile_n) {
    const int bm = gemm_tile_m(M, x_bf16);
    const long long tiles = (long long)((M + bm - 1) / bm) * ((N + tile_n - 1) / tile_n);
    const int cus = num_cus > 0 ? num_cus : 256;
    const int nb = K / kQK;
    // The split count with the least modelled time: rounds of workgroups
    // over the CUs (ceil(tiles * ks / CUs)) times the blocks one split
    // streams (with K halves inside the workgroup an odd count runs as long
    // as the next even one) at ~3.4 us per block, plus, split, ~2 us and the
    // partials written and read back at ~1.8 TB/s. Fitted to 12288 x 6144 and
    // 2048 / 4096 x 6144 at 64-512 fp32 tokens; rounds matter: 88 tiles in 3
    // splits make 264 workgroups, a second round for 8 of them (71 us), in 2
    // one round of 176 (52 us), while 176 tiles stay unsplit (81 us; 4
    // splits, 99 us, most of it the partials).
    const bool halves = gemm_halves(M, x_bf16, K);
    int best = 1;
    double best_t = 0.0;
    for (int ks = 1; ks <= 8 && ks <= nb; ++ks) {
        int per = (nb + ks - 1) / ks;
        if (halves) per += per & 1;
        double t = (double)((tiles * ks + cus - 1) / cus) * per * 3.4;
        if (ks > 1) t += 2.0 + (double)tiles * ks * bm * tile_n * 4 * 2 / 1.8e6;
        if (ks == 1 || t < best_t) {
            best = ks;
            best_t = t;
        }
    }
    return best;
}

namespace {
struct GemmWs {
    size_t img, uns, cnt, part, total;
};
GemmWs gemm_ws(int M, int N, int K, int x_bf16, int ks, int tile_n = kTileN) {
    const auto a256 = [](size_t b) { return (b + 255) / 256 * 256; };
    GemmWs w{};
    const size_t v = x_bf16 ? 1 : 2;
    w.img = 0;
    w.uns = a256(v * (size_t)M * K * 2);
    w.cnt = w.uns + a256((size_t)M * 4);
    const int bm = gemm_tile_m(M, x_bf16);
    const size_t tiles = (size_t)((M + bm - 1) / bm) * ((N + tile_n - 1) / tile_n);
    w.part = w.cnt + (ks > 1 ? a256(tiles * 4) : 0);
    w.total = w.part + (ks > 1 ? tiles * ks * bm * tile_n * 4 : 0);
    return w;
}
}  // namespace

size_t gemm_ws_bytes(int M, int N, int K, int x_bf16, int num_cus) {
    return gemm_ws(M, N, K, x_bf16, gemm_splits(M, N, K, num_cus, x_bf16)).total;
}

hipError_t launch_gemm2(const uint8_t* wa, unsigned long long row0a, int out_a, const uint8_t* wb,
                        unsigned long long row0b, int out_b, int in_dim, const void* X, int x_bf16, int M, float* Ya,
                        float* Yb, uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s, const float* U,
                        float lim) {
    if (M <= 0 || out_a <= 0) return hipSuccess;
    if (!wb) out_b = 0;
    const int tiles_a = (out_a + kTileN - 1) / kTileN, tiles_b = (out_b + kTileN - 1) / kTileN;
    // record offsets inside a tensor's requested rows are 32-bit
    const size_t nb_sz = (size_t)(in_dim / kQK);
    if ((size_t)tiles_a * 3 * nb_sz * kRecordBytes >= (1ull << 32) ||
        (size_t)tiles_b * 3 * nb_sz * kRecordBytes >= (1ull << 32))
        return hipErrorInvalidValue;
    const bool halves = gemm_halves(M, x_bf16, in_dim);
    // k_gemm6 (256-row tiles) where its tiles give every CU at least one
    // and its rounds of workgroups over the CUs take less time than
    // k_gemm5's: a 256-row tile of the 32x32 form takes ~1.2x a 192-row one
    // (M = 2048 bf16: 768 tiles in 3 rounds of ~110 us, against 90 us for
    // k_gemm5's round at M = 512), so 512 fp32 tokens (384 tiles: two
    // rounds, the second half empty) stay on k_gemm5 (512 tiles, two full
    // rounds)
    const int tiles6_a = (out_a + BN6 - 1) / BN6, tiles6_b = (out_b + BN6 - 1) / BN6;
    const int cus = num_cus > 0 ? num_cus : 256;
    const long long tm = (M + gemm_tile_m(M, x_bf16) - 1) / gemm_tile_m(M, x_bf16);
    const long long t6 = tm * (tiles6_a + tiles6_b), t5 = tm * (tiles_a + tiles_b);
    const bool wide6 = halves && t6 >= cus && 6 * ((t6 + cus - 1) / cus) < 5 * ((t5 + cus - 1) / cus);
    const int n_eq = (tiles_a + tiles_b) * kTileN;  // both tensors' result tiles, as one width
    const int ks = wide6 ? 1 : gemm_splits(M, n_eq, in_dim, num_cus, x_bf16, kTileN);
    const GemmWs L = gemm_ws(M, n_eq, in_dim, x_bf16, ks);
    _Float16* xh = reinterpret_cast<_Float16*>(ws + L.img);
    float* uns = reinterpret_cast<float*>(ws + L.uns);
    const int bm = gemm_tile_m(M, x_bf16);
    const int tiles_m = (M + bm - 1) / bm;
    uint32_t* cnt = reinterpret_cast<uint32_t*>(ws + L.cnt);
    const int n_cnt = ks > 1 ? tiles_m * (tiles_a + tiles_b) : 0;
    hipError_t e = x_bf16 ? launch_prep_x<1>(M, in_dim, s, X, nullptr, 0.0f, xh, uns, cnt, n_cnt)
                          : (U ? launch_prep_x<2>(M, in_dim, s, X, U, lim, xh, uns, cnt, n_cnt)
                               : launch_prep_x<0>(M, in_dim, s, X, nullptr, 0.0f, xh, uns, cnt, n_cnt));
    if (e != hipSuccess) return e;
    GemmArgs a{};
    a.nb = in_dim / kQK;
    a.w = wa + (size_t)(row0a / kTileRows) * a.nb * kRecordBytes;
    a.xh = xh;
    a.unscale = uns;
    a.y = Ya;
    a.M = M;
    a.N = out_a;
    a.K = in_dim;
    a.tiles_m = tiles_m;
    a.tiles_n1 = wide6 ? tiles6_a : tiles_a;
    a.tiles_n = wide6 ? tiles6_a + tiles6_b : tiles_a + tiles_b;
    a.w2 = out_b > 0 ? wb + (size_t)(row0b / kTileRows) * a.nb * kRecordBytes : a.w;
    a.y2 = out_b > 0 ? Yb : Ya;
    a.N2 = out_b > 0 ? out_b : out_a;
    a.ks = ks;
    a.cnt = cnt;
    a.part = reinterpret_cast<float*>(ws + L.part);
    a.err = err;
    const int grid = a.tiles_n * a.tiles_m * ks;
    if (wide6)
        return x_bf16 ? launch_timed(kProfGemm, k_gemm6<1>, dim3(grid), dim3(kThreads6), 0, s, a)
                      : launch_timed(kProfGemm, k_gemm6<2>, dim3(grid), dim3(kThreads6), 0, s, a);
    if (halves)
        return x_bf16 ? launch_timed(kProfGemm, k_gemm5<8, 1>, dim3(grid), dim3(kThreads5), 0, s, a)
                      : launch_timed(kProfGemm, k_gemm5<4, 2>, dim3(grid), dim3(kThreads5), 0, s, a);
    const dim3 gd(grid), bd(kGemmThreads);
    if (bm == 64)
        return x_bf16 ? launch_timed(kProfGemm, k_gemm3<64, 1>, gd, bd, 0, s, a)
                      : launch_timed(kProfGemm, k_gemm3<64, 2>, gd, bd, 0, s, a);
    return launch_timed(kProfGemm, k_gemm3<128, 1>, gd, bd, 0, s, a);
}

hipError_t launch_gemm(const uint8_t* w, unsigned long long row0, int in_dim, int out_dim, const void* X, int x_bf16,
                       int M, float* Y, uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s, const float* U,
                       float lim) {
    return launch_gemm2(w, row0, out_dim, nullptr, 0, 0, in_dim, X, x_bf16, M, Y, nullptr, ws, err, num_cus, s, U,
                        lim);
}

// ---------------------------------------------------------------------------
// Batched dense MLP as GEMMs (model_batch.cpp:62-72: matmul_quant of gate and
// up over the same X, SwiGLU, matmul_quant of down): the gate+up two-tensor
// GEMM, the SwiGLU images of its rows, and the down GEMM, with up to two
// more tensors of the same X (extra) computed in the down launch. At up to
// 64 tokens of fp32 X that launch holds two problems, down on the SwiGLU
// images and the extra tensors on the X images the gate+up GEMM made, with
// K splits chosen so that every workgroup streams the same number of blocks
// and the grid fits the CUs (64 tokens, 6144 x 12288 down with kv_a 576 and
// q_a 1536 over 6144: down in 6 splits of 8 blocks, the extra tensors in 3
// of 8, 225 workgroups). Elsewhere the extra tensors are a two-tensor GEMM
// launch of their own.

namespace {
struct MlpGemmPlan {
    bool merged;
    int ks_gu, ks_d, ks_e, tiles_m, tiles_d, tiles_e1, tiles_e2;
    size_t yg, yu, a, b_img, b_uns, b_cnt, b_part, total;  // region offsets after the header
};

MlpGemmPlan mlp_gemm_plan(int H, int I, int M, int x_bf16, int out_e1, int out_e2, int num_cus) {
    const auto a256 = [](size_t b) { return (b + 255) / 256 * 256; };
    const auto tiles = [](int n) { return n > 0 ? (n + kTileN - 1) / kTileN : 0; };
    const int cus = num_cus > 0 ? num_cus : 256;
    MlpGemmPlan p{};
    p.tiles_m = (M + gemm_tile_m(M, x_bf16) - 1) / gemm_tile_m(M, x_bf16);
    p.tiles_d = tiles(H);
    p.tiles_e1 = tiles(out_e1);
    p.tiles_e2 = tiles(out_e2);
    const int tiles_e = p.tiles_e1 + p.tiles_e2;
    const int nb_h = H / kQK, nb_i = I / kQK;
    p.ks_gu = gemm_splits(M, 2 * tiles(I) * kTileN, H, num_cus, x_bf16);
    p.yg = 0;
    p.yu = a256((size_t)M * I * 4);
    p.a = p.yu + a256((size_t)M * I * 4);
    // the smallest even number of blocks per split (at most 8 splits per
    // tile) whose workgroups fit the CUs
    if (tiles_e > 0 && !x_bf16 && M <= 64 && gemm_halves(M, 0, I) && gemm_halves(M, 0, H)) {
        for (int blk = 2; blk <= nb_i || blk <= nb_h; blk += 2) {
            const int kd = (nb_i + blk - 1) / blk, ke = (nb_h + blk - 1) / blk;
            if (kd > 8 || ke > 8) continue;
            if ((long long)p.tiles_m * (p.tiles_d * kd + tiles_e * ke) <= cus) {
                p.merged = true;
                p.ks_d = kd;
                p.ks_e = ke;
                break;
            }
        }
    }
    if (p.merged) {
        const GemmWs la = gemm_ws(M, 2 * tiles(I) * kTileN, H, 0, p.ks_gu);
        p.b_img = p.a + a256(la.total);
        p.b_uns = p.b_img + a256((size_t)2 * M * I * 2);
        p.b_cnt = p.b_uns + a256((size_t)M * 4);
        p.b_part = p.b_cnt + a256((size_t)p.tiles_m * (p.tiles_d + tiles_e) * 4);
        p.total = p.b_part + (size_t)p.tiles_m * (p.tiles_d * p.ks_d + tiles_e * p.ks_e) * 64 * kTileN * 4;
    } else {
        // gate+up, down and the extra tensors one after another through
        // one scratch region
        size_t sc = gemm2_ws_bytes(M, I, I, H, x_bf16, num_cus);
        sc = std::max(sc, gemm_ws_bytes(M, H, I, 0, num_cus));
        if (tiles_e > 0) sc = std::max(sc, gemm2_ws_bytes(M, std::max(out_e1, 1), out_e2, H, x_bf16, num_cus));
        p.total = p.a + sc;
    }
    return p;
}
}  // namespace

size_t mlp_gemm_ws_bytes(int H, int I, int M, int x_bf16, int out_e1, int out_e2, int num_cus) {
    return mlp_gemm_plan(H, I, M, x_bf16, out_e1, out_e2, num_cus).total;
}

hipError_t launch_mlp_gemm(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int H, int I,
                           const void* X, int x_bf16, int M, float lim, float* Y, const uint8_t* w_e1, int out_e1,
                           float* y_e1, const uint8_t* w_e2, int out_e2, float* y_e2, uint8_t* ws, uint32_t* err,
                           int num_cus, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    if (!w_e1) out_e1 = 0;
    if (!w_e2) out_e2 = 0;
    if (out_e1 <= 0 && out_e2 > 0) {  // the extra tensor in the first place
        w_e1 = w_e2, out_e1 = out_e2, y_e1 = y_e2;
        w_e2 = nullptr, out_e2 = 0;
    }
    const MlpGemmPlan p = mlp_gemm_plan(H, I, M, x_bf16, out_e1, out_e2, num_cus);
    float* yg = reinterpret_cast<float*>(ws + p.yg);
    float* yu = reinterpret_cast<float*>(ws + p.yu);
    uint8_t* wa = ws + p.a;
    hipError_t e = launch_gemm2(w_gate, 0, I, w_up, 0, I, H, X, x_bf16, M, yg, yu, wa, err, num_cus, s);
    if (e != hipSuccess) return e;
    if (!p.merged) {
        e = launch_gemm(w_down, 0, I, H, yg, 0, M, Y, wa, err, num_cus, s, yu, lim);
        if (e != hipSuccess || out_e1 <= 0) return e;
        return launch_gemm2(w_e1, 0, out_e1, w_e2, 0, out_e2, H, X, x_bf16, M, y_e1, y_e2, wa, err, num_cus, s);
    }
    // the gate+up GEMM's X images (its workspace layout), and the SwiGLU
    // images of its rows (tickets of both problems cleared on the way)
    const GemmWs la = gemm_ws(M, 2 * ((I + kTileN - 1) / kTileN) * kTileN, H, 0, p.ks_gu);
    _Float16* xa = reinterpret_cast<_Float16*>(wa + la.img);
    float* ua = reinterpret_cast<float*>(wa + la.uns);
    _Float16* xb = reinterpret_cast<_Float16*>(ws + p.b_img);
    float* ub = reinterpret_cast<float*>(ws + p.b_uns);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(ws + p.b_cnt);
    float* part = reinterpret_cast<float*>(ws + p.b_part);
    const int tiles_e = p.tiles_e1 + p.tiles_e2;
    e = launch_prep_x<2>(M, I, s, yg, yu, lim, xb, ub, cnt, p.tiles_m * (p.tiles_d + tiles_e));
    if (e != hipSuccess) return e;
    GemmArgs a{};
    a.w = w_down;
    a.xh = xb;
    a.unscale = ub;
    a.y = Y;
    a.M = M;
    a.N = H;
    a.K = I;
    a.nb = I / kQK;
    a.tiles_m = p.tiles_m;
    a.tiles_n = a.tiles_n1 = p.tiles_d;
    a.w2 = w_down;
    a.y2 = Y;
    a.N2 = H;
    a.ks = p.ks_d;
    a.cnt = cnt;
    a.part = part;
    a.err = err;
    GemmProb& q = a.p2;
    q.w = w_e1;
    q.xh = xa;
    q.unscale = ua;
    q.y = y_e1;
    q.N = out_e1;
    q.K = H;
    q.nb = H / kQK;
    q.tiles_n = tiles_e;
    q.tiles_n1 = p.tiles_e1;
    q.w2 = out_e2 > 0 ? w_e2 : w_e1;
    q.y2 = out_e2 > 0 ? y_e2 : y_e1;
    q.N2 = out_e2 > 0 ? out_e2 : out_e1;
    q.ks = p.ks_e;
    q.cnt = cnt + p.tiles_m * p.tiles_d;
    q.part = part + (size_t)p.tiles_m * p.tiles_d * p.ks_d * 64 * kTileN;
    q.wg0 = p.tiles_m * p.tiles_d * p.ks_d;
    const int grid = q.wg0 + p.tiles_m * tiles_e * p.ks_e;
    return launch_timed(kProfGemm, k_gemm5<4, 2>, dim3(grid), dim3(kThreads5), 0, s, a);
}

// ---------------------------------------------------------------------------
// Grouped GEMM over routed-expert buckets (the prefill-sized moe_batch,
// model_batch.cpp:224-262: one matmul_quant per expert over its g tokens).

// Tokens per tile of the grouped GEMMs (fp32 X, two images): 16 * mt for
// mt = 2..5, chosen from the mean bucket (grp_tile_mt). Every tile decodes
// its W rows once, so the count of tiles sets the decode work and their
// padding the MFMA work: a 512-token chunk at top-8 of 64 experts (buckets
// of 48-82 slots) makes 95 tiles of 64 for 4096 slots, 65 of 80.
constexpr int kGrpMinTile = 32;

namespace {
// The expert tile table: for every expert e with tokens, one entry
// e << 16 | mt per bm-token tile mt of its bucket eptr[e] .. eptr[e + 1],
// then (sh_rows > 0) E << 16 | mt per tile of the shared expert's sh_rows
// slots; count[0] = the number of entries (at most cap). One workgroup, one
// thread per expert; bucket sizes are clamped to [0, S], so the table stays
// in bounds whatever eptr holds.
__global__ __launch_bounds__(1024) void k_grp_tiles(const int* __restrict__ eptr, int E, int S, int bm, int sh_rows,
                                                    int* __restrict__ tiles, int* __restrict__ count, int cap) {
    __shared__ int sc[1024];
    const int e = threadIdx.x;
    int n = 0;
    if (e < E) {
        const int g = min(max(eptr[e + 1] - eptr[e], 0), S);
        n = (g + bm - 1) / bm;
    }
    sc[e] = n;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int v = e >= off ? sc[e - off] : 0;
        __syncthreads();
        sc[e] += v;
        __syncthreads();
    }
    const int start = sc[e] - n;
    for (int i = 0; i < n && start + i < cap; ++i) tiles[start + i] = (e << 16) | i;
    // then the shared expert's tiles (id E) after the routed ones
    const int total = sc[1023];
    const int n_sh = sh_rows > 0 ? (min(sh_rows, S) + bm - 1) / bm : 0;
    for (int i = e; i < n_sh && total + i < cap; i += 1024) tiles[total + i] = (E << 16) | i;
    if (e == 1023) count[0] = min(total + n_sh, cap);
}
}  // namespace

int grp_tiles_cap(int S, int E, int mt) { return S / (16 * (mt > 0 ? mt : kGrpMinTile / 16)) + E; }

int grp_tile_mt(int S, int E) {
    // the mean bucket plus two of its Poisson deviations, in 16-token tiles
    const double avg = (double)S / (E > 0 ? E : 1);
    const int mt = (int)std::ceil((avg + 2.0 * std::sqrt(avg)) / 16.0);
    return std::min(std::max(mt, kGrpMinTile / 16), 5);
}

hipError_t launch_grp_tiles(const int* eptr, int E, int S, int mt, int* tiles, int* count, hipStream_t s,
                            int sh_rows) {
    if (E < 1 || E > 1024 || mt < kGrpMinTile / 16 || mt > 5) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_grp_tiles, dim3(1), dim3(1024), 0, s, eptr, E, S + sh_rows, 16 * mt, sh_rows, tiles, count,
                       grp_tiles_cap(S + sh_rows, E + (sh_rows > 0 ? 1 : 0), mt));
    return hipGetLastError();
}

hipError_t launch_gemm_grouped(const uint8_t* wa, const uint8_t* wb, int rows, int in_dim, int E, const int* eptr,
                               int S, const _Float16* xh, const float* uns, float* ya, float* yb, const int* tiles,
                               const int* count, uint32_t* err, hipStream_t s, int mt, const int* tok,
                               int img_rows, const uint8_t* wa_sh, const uint8_t* wb_sh, int sh_rows) {
    if (rows <= 0 || rows % kTileRows || S <= 0 || (tok && img_rows <= 0)) return hipErrorInvalidValue;
    // image offsets are 32-bit (two fp16 images of S, or img_rows, rows)
    if ((size_t)2 * (tok ? img_rows : S) * in_dim * 2 >= (1ull << 32)) return hipErrorInvalidValue;
    const size_t nb = (size_t)(in_dim / kQK);
    const size_t stride = (size_t)(rows / kTileRows) * nb * kRecordBytes;
    if (stride >= (1ull << 32)) return hipErrorInvalidValue;
    GemmArgs a{};
    a.nb = (int)nb;
    a.w = wa;
    a.xh = xh;
    a.unscale = uns;
    a.y = ya;
    a.M = S;
    a.N = rows;
    a.K = in_dim;
    const int tn1 = (rows + kTileN - 1) / kTileN;
    a.tiles_n1 = tn1;
    a.tiles_n = wb ? 2 * tn1 : tn1;
    a.w2 = wb ? wb : wa;
    a.y2 = wb ? yb : ya;
    a.N2 = rows;
    a.ks = 1;
    a.err = err;
    a.grp_eptr = eptr;
    a.grp_tile = tiles;
    a.grp_count = count;
    a.grp_rows = S;
    a.grp_w_stride = stride;
    a.grp_tok = tok;
    a.grp_img_rows = tok ? img_rows : S;
    // the shared expert's slots are the last sh_rows of the S
    a.grp_sh_e = sh_rows > 0 ? E : -1;
    a.grp_sh_rows = sh_rows;
    a.grp_w_sh = wa_sh;
    a.grp_w2_sh = wb_sh ? wb_sh : wa_sh;
    if (mt < kGrpMinTile / 16 || mt > 5 || (sh_rows > 0 && (!wa_sh || (wb && !wb_sh) || sh_rows > S)))
        return hipErrorInvalidValue;
    const int cap = grp_tiles_cap(S, E + (sh_rows > 0 ? 1 : 0), mt);
    a.tiles_m = cap;
    const dim3 grid(cap * a.tiles_n), block(kThreads5);
    switch (mt) {
        case 2: return launch_timed(kProfGemm, k_gemm5<2, 2>, grid, block, 0, s, a);
        case 3: return launch_timed(kProfGemm, k_gemm5<3, 2>, grid, block, 0, s, a);
        case 4: return launch_timed(kProfGemm, k_gemm5<4, 2>, grid, block, 0, s, a);
        default: return launch_timed(kProfGemm, k_gemm5<5, 2>, grid, block, 0, s, a);
    }
}

hipError_t launch_prep_x_rows(int M, int K, hipStream_t s, const float* X, const float* U, float lim, _Float16* xh,
                              float* uns, const int* gather) {
    return U ? launch_prep_x<2>(M, K, s, X, U, lim, xh, uns, nullptr, 0, gather)
             : launch_prep_x<0>(M, K, s, X, nullptr, 0.0f, xh, uns, nullptr, 0, gather);
}

size_t gemm2_ws_bytes(int M, int out_a, int out_b, int K, int x_bf16, int num_cus) {
    const int n_eq = ((out_a + kTileN - 1) / kTileN + (out_b + kTileN - 1) / kTileN) * kTileN;
    return gemm_ws_bytes(M, n_eq, K, x_bf16, num_cus);
}

}  // namespace gpeed
