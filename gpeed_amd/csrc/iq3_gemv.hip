// IQ3_XXS GEMV kernels (gfx950): y[t] = W x[t] for 1..8 activation vectors
// ("tokens") over the T64 layout.
//
// Work split. The (tile, block) records of the requested rows (of one or two
// same-shape tensors) are numbered tile-major and cut into equal contiguous
// chunks, one per workgroup, so every CU streams the same number of bytes
// whatever the tile count. Inside a workgroup the chunk's records are dealt
// round-robin to the wavefronts; a wavefront streams its records through a
// register ring (six coalesced 16-byte loads and one 2-byte load per lane)
// and keeps a per-row partial sum per tile, which meets the other
// wavefronts' partials in LDS. A tile cut by a chunk boundary is finished by
// whichever of its workgroups arrives last (atomic ticket in a caller-owned
// workspace); it adds the workgroups' partials in chunk order, so results do
// not depend on timing.
//
// Decode and product. Lane n of a wavefront holds row n of the tile. Per
// group of 4 weights it makes one LDS lookup in its own replica of the grid
// table (4 unsigned fp16, no bank conflicts), sets the fp16 sign bits with a
// rotate and a masked or, and issues one v_mfma_f32_4x4x4_16b_f16 whose A
// operand is broadcast (CBSZ=4) from the lanes of block ABID of a register
// pair that holds 16 such 4-element activation slices: row 2p / 2p+1 carry
// token 2p as fp16 hi / lo parts, rows 2 / 3 token 2p+1. Accumulator row
// rho of lane n is then exactly (activation variant rho) . (the lane's 4
// weights), summed over a 32-weight sub-block; the lane scales it by its own
// (2s+1), and by d/4 times the activation block's power-of-two unscale once
// per block. Products are exact in fp32; only the accumulation order differs
// from the CPU path.
#include "iq3_common.h"
#include "iq3_gemv_core.h"
#include "iq3_kernels.h"
#include "iq3_prof.h"

namespace gpeed {

namespace {

// ---------------------------------------------------------------------------
// Prepared activation: per 256-element block and token pair p, four 512-byte
// register images (a = 0..3, one per pair of sub-blocks), lane l = 4*beta+rho
// holding 4 fp16 of variant rho (0: token 2p hi, 1: 2p lo, 2: 2p+1 hi,
// 3: 2p+1 lo) of slice beta (sub-block 2a + beta/8, elements 4*(beta%8)..+3).
// A last pair with a single token stores only rho = 0, 1 (256-byte images).
// Block stride n_tok * 1 KiB; then one fp32 unscale per (block, token).

__device__ __forceinline__ size_t act_offset(int n_tok, int b, int t, int a, int beta, int hl) {
    const int p = t >> 1;
    const bool half_pair = (n_tok & 1) && (p == (n_tok >> 1));
    const size_t base = (size_t)b * n_tok * 1024 + (size_t)p * 2048;
    if (half_pair) return base + a * 256 + (2 * beta + hl) * 8;
    return base + a * 512 + (4 * beta + 2 * (t & 1) + hl) * 8;
}

// One wavefront per (block, token): max|v| -> power-of-two scale -> fp16
// hi/lo split. Lane l owns elements 4l..4l+3, i.e. slice beta = l & 15 of
// register image a = l >> 4. MODE 0: v = x. MODE 1: v = silu(min(g,lim)) *
// clamp(u,-lim,lim) (model.cpp:683-688, model_batch.cpp:245-253).
template <int MODE>
__global__ __launch_bounds__(256) void k_prep_act(const float* __restrict__ x,
                                                  const float* __restrict__ x2, float lim, int nb,
                                                  int n_tok, uint8_t* __restrict__ act) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + wave;
    if (item >= nb * n_tok) return;
    const int t = item / nb, b = item - t * nb;
    const size_t src = (size_t)t * nb * 256 + (size_t)b * 256 + 4 * lane;
    const float4 v = *reinterpret_cast<const float4*>(x + src);
    float e[4] = {v.x, v.y, v.z, v.w};
    if (MODE == 1) {
        const float4 u = *reinterpret_cast<const float4*>(x2 + src);
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
    const int a = lane >> 4, beta = lane & 15;
    *reinterpret_cast<u32x2_t*>(act + act_offset(n_tok, b, t, a, beta, 0)) = __builtin_bit_cast(u32x2_t, hi);
    *reinterpret_cast<u32x2_t*>(act + act_offset(n_tok, b, t, a, beta, 1)) = __builtin_bit_cast(u32x2_t, lo);
    if (lane == 0) {
        float* xsc = reinterpret_cast<float*>(act + (size_t)nb * n_tok * 1024);
        xsc[(size_t)b * n_tok + t] = ldexpf(1.0f, -sc);
    }
}

// ---------------------------------------------------------------------------
// GEMV

#ifndef GEMV_WAVES
#define GEMV_WAVES 8
#endif
#ifndef GEMV_PF
#define GEMV_PF 2
#endif
#ifndef GEMV_PRE
#define GEMV_PRE 1
#endif

template <int NT>
struct GemvCfg {
    static constexpr int kPairs = (NT + 1) / 2;
    static constexpr int kWaves = GEMV_WAVES;
    static constexpr int kPF = GEMV_PF;
    // ring slots filled before the prologue barrier: a wavefront stuck
    // issuing record loads (the CU's queue full) must not hold the barrier
    static constexpr int kPre = GEMV_PRE;
    // tiles one chunk may touch (LDS partial slots)
    static constexpr int kSlots = NT == 1 ? 8 : (NT == 2 ? 4 : 2);
};

// Largest chunk (records per workgroup) that touches at most kSlots tiles.
template <int NT>
constexpr int max_chunk(int nb) {
    return (GemvCfg<NT>::kSlots - 1) * nb + 1;
}

struct GemvArgs {
    const uint8_t* w[2];   // T64 records of the first requested tile, per tensor
    float* y[2];           // [n_tok][out_dim] per tensor
    const uint8_t* act;    // prepared activation
    const float* xsc;      // [nb][n_tok] activation unscales
    uint32_t* cnt;         // [n_tiles_all] tickets (zero between launches)
    float* part;           // [n_tiles_all][max_parts][NT][64] chunk partials
    int nb;
    int n_tiles;           // tiles per tensor
    int n_records;         // n_tensors * n_tiles * nb
    int out_dim;
    int chunk;             // records per workgroup
    int max_parts;
    const float* x;        // fused preparation: fp32 x (or g) ...
    const float* x2;       // ... and u for the SwiGLU input
    float lim;
};

// Fused activation preparation (one vector, K <= 16384): the workgroup
// prepares the blocks its chunk touches straight into LDS.
constexpr int kPrepMaxNb = 64;
// buffer resource word 3 for raw (untyped) buffer loads on gfx9
constexpr int kBufferDword3 = 0x00020000;
template <int NT, int MODE>
struct Slots {
    static constexpr int value = MODE == 0 ? GemvCfg<NT>::kSlots : 4;
};

template <int NT, int MODE>
__device__ __forceinline__ void load_rec(Rec<(NT + 1) / 2>& r, const GemvArgs& g, int rec, uint32_t lane) {
    const int per_tensor = g.n_tiles * g.nb;
    const int ten = rec >= per_tensor ? 1 : 0;
    const int rl = rec - ten * per_tensor;
    if constexpr (MODE != 0) {
        load_record_w(r, g.w[ten] + (size_t)rl * kRecordBytes, lane);  // images come from LDS
    } else {
        const int b = rl - (rl / g.nb) * g.nb;
        load_record<(NT + 1) / 2>(r, g.w[ten] + (size_t)rl * kRecordBytes, g.act + (size_t)b * NT * 1024, lane, NT);
    }
}

__device__ __forceinline__ float swiglu1(float gv, float uv, float lim) {
    const float gi = fminf(gv, lim);
    const float ui = fminf(fmaxf(uv, -lim), lim);
    return (gi / (1.0f + expf(-gi))) * ui;
}

// Power-of-two block scale (max |v| of the wavefront's 256 values into
// [2^13, 2^14)) and the fp16 hi/lo split of this lane's 4 values; returns
// the unscale.
__device__ __forceinline__ float split_hi_lo(const float (&e)[4], u32x2_t& hi2, u32x2_t& lo2) {
    float m = fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    int sc = 0;
    if (m > 0.0f && m < __builtin_inff()) {
        int ex;
        (void)frexpf(m, &ex);
        sc = 14 - ex;
        sc = sc > 120 ? 120 : (sc < -120 ? -120 : sc);
    }
    _Float16 hi[4], lo[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float xs = ldexpf(e[c], sc);
        hi[c] = (_Float16)xs;
        lo[c] = (_Float16)(xs - (float)hi[c]);
    }
    hi2 = __builtin_bit_cast(u32x2_t, hi);
    lo2 = __builtin_bit_cast(u32x2_t, lo);
    return ldexpf(1.0f, -sc);
}

// MODE 0: prepared activation from global memory (act / xsc); MODE 1: fp32
// x prepared in the kernel; MODE 2: SwiGLU(g = x, u = x2) prepared in the
// kernel (MODE 1 and 2 take one vector).
template <int NT, int MODE>
__global__ __launch_bounds__(GemvCfg<NT>::kWaves * 64) void k_gemv_t64(GemvArgs g) {
    static_assert(MODE == 0 || NT == 1, "fused preparation takes one vector");
    constexpr int W = GemvCfg<NT>::kWaves;
    constexpr int PF = GemvCfg<NT>::kPF;
    constexpr int S = Slots<NT, MODE>::value;
    constexpr int NP = GemvCfg<NT>::kPairs;
    constexpr int kThreads = W * 64;
    __shared__ __attribute__((aligned(16))) uint8_t tbl[kGridTableBytes];
    __shared__ float red[S][W][NT][64];
    __shared__ int last_flag[S];
    __shared__ __attribute__((aligned(16))) uint8_t xsl[MODE ? kPrepMaxNb * 1024 : 16];
    __shared__ float xscl[MODE ? kPrepMaxNb : 1];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lane = tid & 63;
    const uint32_t lb = (lane & 31u) << 3;  // this lane's replica of the grid table

    const int c0 = blockIdx.x * g.chunk;
    const int c1 = min(c0 + g.chunk, g.n_records);
    const int n_mine = c1 - c0 > wave ? (c1 - c0 - wave + W - 1) / W : 0;
    const int tile0 = c0 / g.nb;

    // The activation blocks (fused preparation) go out first, then the
    // first record of every wavefront; the grid table (immediate data) and
    // the activation images are built while those are in flight.
    constexpr int PRE = GemvCfg<NT>::kPre;
    constexpr int kPrepPer = (kPrepMaxNb + W - 1) / W;  // blocks per wave
    const int n_pblk = MODE ? min(c1 - c0, g.nb) : 0;   // the chunk's blocks: b = (c0 + i) % nb
    float4 xv[MODE ? kPrepPer : 1], uv[MODE == 2 ? kPrepPer : 1];
    if constexpr (MODE != 0) {
        // buffer loads: an offset past the end returns zeros without a
        // memory access, so every wave issues the same loads, unbranched
        const auto xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.x), 0, g.nb * 1024, kBufferDword3);
        const auto ur = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.x2), 0, g.nb * 1024, kBufferDword3);
#pragma unroll
        for (int j = 0; j < kPrepPer; ++j) {
            const int i = wave + j * W;
            const uint32_t off = i < n_pblk ? (uint32_t)((c0 + i) % g.nb) * 1024u + lane * 16u : 0x80000000u;
            xv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            if constexpr (MODE == 2)
                uv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, 0));
        }
    }
    // A CU serves its vector memory queue in order: the small loads above
    // must all be queued before any wave's records, or a late wave's
    // activation (and with it the barrier below) waits for HBM. s_barrier
    // waits for issue only, not for data.
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    Rec<NP> ring[PF];
#pragma unroll
    for (int s = 0; s < PRE; ++s) load_rec<NT, MODE>(ring[s], g, min(c0 + wave + s * W, c1 - 1), lane);
    grid_table_literal<W>(tbl, wave, lane);
    for (int i = tid; i < S * W * NT * 64; i += kThreads) (&red[0][0][0][0])[i] = 0.0f;
    if constexpr (MODE != 0) {
#pragma unroll
        for (int j = 0; j < kPrepPer; ++j) {
            const int i = wave + j * W;
            if (i < n_pblk) {
                const int b = (c0 + i) % g.nb;
                float e[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
                if constexpr (MODE == 2) {
                    const float us[4] = {uv[j].x, uv[j].y, uv[j].z, uv[j].w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) e[c] = swiglu1(e[c], us[c], g.lim);
                }
                u32x2_t hi, lo;
                const float unscale = split_hi_lo(e, hi, lo);
                // single-vector images: lane 4*beta+rho of register a holds
                // variant rho (0 hi, 1 lo) of slice beta at a*256 + (2*beta+rho)*8
                const int a = lane >> 4, beta = lane & 15;
                *reinterpret_cast<u32x2_t*>(xsl + b * 1024 + a * 256 + (2 * beta) * 8) = hi;
                *reinterpret_cast<u32x2_t*>(xsl + b * 1024 + a * 256 + (2 * beta + 1) * 8) = lo;
                if (lane == 0) xscl[b] = unscale;
            }
        }
    }
    lds_barrier();
#pragma unroll
    for (int s = PRE; s < PF; ++s) load_rec<NT, MODE>(ring[s], g, min(c0 + wave + s * W, c1 - 1), lane);

    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    int cur_slot = -1;
    // Every iteration issues the same loads whatever the branch (a refill
    // past the wave's last record re-reads the chunk's last one), so the
    // compiler waits for exactly the ring slot it needs, not for every load.
    for (int k0 = 0; k0 < n_mine; k0 += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            const int k = k0 + s;
            const bool valid = k < n_mine;
            const int rec = min(c0 + wave + k * W, c1 - 1);
            const int tile = rec / g.nb;
            const int b = rec - tile * g.nb;
            const int slot = tile - tile0;
            if (valid && slot != cur_slot) {
                if (cur_slot >= 0) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) red[cur_slot][wave][t][lane] = acc[t];
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
                cur_slot = slot;
            }
            if (valid) {
                if constexpr (MODE != 0) {
                    const uint32_t off_half = ((lane >> 2) * 2 + (lane & 1)) * 8u;
#pragma unroll
                    for (int a = 0; a < 4; ++a)
                        ring[s].a[0][a] = *reinterpret_cast<const u32x2_t*>(xsl + b * 1024 + a * 256 + off_half);
                }
                float blk[2 * NP];
#pragma unroll
                for (int t = 0; t < 2 * NP; ++t) blk[t] = 0.0f;
                record_dot<NP>(tbl, ring[s], lb, blk);
                const float d4 = (float)__builtin_bit_cast(_Float16, (uint16_t)ring[s].d) * 0.25f;
                if constexpr (MODE != 0) {
                    acc[0] = fmaf(d4 * xscl[b], blk[0], acc[0]);
                } else {
                    const float* xs = g.xsc + (size_t)b * NT;
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[t] = fmaf(d4 * xs[t], blk[t], acc[t]);
                }
            }
            // refill, clamped to the chunk's last record (a valid address)
            load_rec<NT, MODE>(ring[s], g, min(c0 + wave + (k + PF) * W, c1 - 1), lane);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (cur_slot >= 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) red[cur_slot][wave][t][lane] = acc[t];
    }
    lds_barrier();

    // Sum the wavefront partials per (tile, token, row) in wave order; whole
    // tiles go straight to y, tiles shared with a neighbouring chunk (only
    // the chunk's first and last can be) to the workspace.
    const int n_slots = (c1 - 1) / g.nb - tile0 + 1;
    auto first_chunk = [&](int tile) { return tile * g.nb / g.chunk; };
    auto last_chunk = [&](int tile) { return ((tile + 1) * g.nb - 1) / g.chunk; };
    for (int o = tid; o < n_slots * NT * 64; o += kThreads) {
        const int slot = o / (NT * 64), t = (o / 64) % NT, n = o & 63;
        float sum = 0.0f;
#pragma unroll
        for (int v = 0; v < W; ++v) sum += red[slot][v][t][n];
        const int tile = tile0 + slot;
        const int first = first_chunk(tile);
        if (first == last_chunk(tile)) {
            const int ten = tile >= g.n_tiles ? 1 : 0;
            const int row = (tile - ten * g.n_tiles) * kTileRows + n;
            if (row < g.out_dim) g.y[ten][(size_t)t * g.out_dim + row] = sum;
        } else {
            // coherent across the XCDs' L2s without a full-cache writeback
            __hip_atomic_store(g.part + (((size_t)tile * g.max_parts + (blockIdx.x - first)) * NT + t) * 64 + n,
                               sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const int tile_end = tile0 + n_slots - 1;
    const bool any_shared = first_chunk(tile0) != last_chunk(tile0) ||
                            first_chunk(tile_end) != last_chunk(tile_end);
    if (!any_shared) return;  // uniform
    // Partials complete (vmcnt(0)) before any thread of the workgroup takes
    // a ticket; the ticket holder that completes a tile then reads the other
    // chunks' partials with coherent loads.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (tid < n_slots) {
        const int tile = tile0 + tid;
        const int first = first_chunk(tile), last = last_chunk(tile);
        int is_last = 0;
        if (first != last) {
            const uint32_t old = __hip_atomic_fetch_add(g.cnt + tile, 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            is_last = old == (uint32_t)(last - first);
        }
        last_flag[tid] = is_last;
    }
    __syncthreads();
    for (int o = tid; o < n_slots * NT * 64; o += kThreads) {
        const int slot = o / (NT * 64), t = (o / 64) % NT, n = o & 63;
        if (!last_flag[slot]) continue;
        const int tile = tile0 + slot;
        const int parts = last_chunk(tile) - first_chunk(tile) + 1;
        float sum = 0.0f;
        for (int j = 0; j < parts; ++j)
            sum += __hip_atomic_load(g.part + (((size_t)tile * g.max_parts + j) * NT + t) * 64 + n,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int ten = tile >= g.n_tiles ? 1 : 0;
        const int row = (tile - ten * g.n_tiles) * kTileRows + n;
        if (row < g.out_dim) g.y[ten][(size_t)t * g.out_dim + row] = sum;
    }
    if (tid < n_slots && last_flag[tid])
        __hip_atomic_store(g.cnt + tile0 + tid, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

template <int NT, int MODE = 0>
hipError_t launch_gemv_nt(const GemvPlan& plan, GemvArgs a, hipStream_t s) {
    a.chunk = plan.chunk;
    a.max_parts = plan.max_parts;
    return launch_timed(kProfGemv, k_gemv_t64<NT, MODE>, dim3(plan.grid), dim3(GemvCfg<NT>::kWaves * 64), 0, s, a);
}

}  // namespace

size_t act_bytes(int in_dim, int n_tok) {
    const size_t nb = (size_t)(in_dim / kQK);
    const size_t b = nb * n_tok * 1024 + nb * n_tok * 4;
    return (b + 255) / 256 * 256;
}

hipError_t launch_prep_act(const float* x, int in_dim, int n_tok, uint8_t* act, hipStream_t s) {
    const int nb = in_dim / kQK;
    const int items = nb * n_tok;
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(k_prep_act<0>, dim3((items + 3) / 4), dim3(256), 0, s, x, nullptr, 0.0f, nb, n_tok,
                       act);
    return hipGetLastError();
}

hipError_t launch_prep_swiglu(const float* g, const float* u, float lim, int in_dim, int n_tok,
                              uint8_t* act, hipStream_t s) {
    const int nb = in_dim / kQK;
    const int items = nb * n_tok;
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(k_prep_act<1>, dim3((items + 3) / 4), dim3(256), 0, s, g, u, lim, nb, n_tok, act);
    return hipGetLastError();
}

GemvPlan plan_gemv(int n_tensors, int in_dim, int out_dim, int n_tok, int num_cus, bool fused) {
    GemvPlan p{};
    const int nb = in_dim / kQK;
    const int n_tiles = (out_dim + kTileRows - 1) / kTileRows;
    p.n_tiles_all = (long long)n_tiles * n_tensors;
    const long long recs = p.n_tiles_all * nb;
    p.n_records = recs;
    const int cus = num_cus > 0 ? num_cus : 256;
    long long chunk = (recs + cus - 1) / cus;
    int cap = 0;
    switch (n_tok) {
        case 1: cap = fused ? (Slots<1, 1>::value - 1) * nb + 1 : max_chunk<1>(nb); break;
        case 2: cap = max_chunk<2>(nb); break;
        case 3: case 4: cap = max_chunk<4>(nb); break;
        default: cap = max_chunk<8>(nb); break;
    }
    if (chunk > cap) chunk = cap;
    if (chunk < 1) chunk = 1;
    p.chunk = (int)chunk;
    p.grid = recs > 0 ? (int)((recs + chunk - 1) / chunk) : 0;
    p.max_parts = (int)((nb - 1) / chunk + 2);
    if (p.max_parts > nb) p.max_parts = nb;
    return p;
}

size_t gemv_ws_bytes(int n_tensors, int in_dim, int out_dim, int n_tok) {
    const long long nb = in_dim / kQK;
    const long long tiles = (long long)((out_dim + kTileRows - 1) / kTileRows) * n_tensors;
    const size_t cnt = ((size_t)tiles * 4 + 255) / 256 * 256;
    return cnt + (size_t)tiles * (size_t)nb * (size_t)n_tok * 64 * 4;
}

hipError_t launch_gemv_t64(const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                           unsigned long long row0, int out_dim, int n_tok, const uint8_t* act,
                           uint8_t* ws, int num_cus, hipStream_t s) {
    const GemvPlan plan = plan_gemv(n_tensors, in_dim, out_dim, n_tok, num_cus, false);
    if (plan.grid == 0) return hipSuccess;
    GemvArgs a{};
    a.nb = in_dim / kQK;
    const size_t skip = (size_t)(row0 / kTileRows) * a.nb * kRecordBytes;
    for (int i = 0; i < 2; ++i) {
        const int k = i < n_tensors ? i : 0;
        a.w[i] = w[k] + skip;
        a.y[i] = y[k];
    }
    a.act = act;
    a.xsc = reinterpret_cast<const float*>(act + (size_t)a.nb * n_tok * 1024);
    a.n_tiles = (out_dim + kTileRows - 1) / kTileRows;
    a.n_records = (int)plan.n_records;
    a.out_dim = out_dim;
    a.cnt = reinterpret_cast<uint32_t*>(ws);
    a.part = reinterpret_cast<float*>(ws + ((size_t)plan.n_tiles_all * 4 + 255) / 256 * 256);
    switch (n_tok) {
        case 1: return launch_gemv_nt<1>(plan, a, s);
        case 2: return launch_gemv_nt<2>(plan, a, s);
        case 3: return launch_gemv_nt<3>(plan, a, s);
        case 4: return launch_gemv_nt<4>(plan, a, s);
        case 5: return launch_gemv_nt<5>(plan, a, s);
        case 6: return launch_gemv_nt<6>(plan, a, s);
        case 7: return launch_gemv_nt<7>(plan, a, s);
        case 8: return launch_gemv_nt<8>(plan, a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_x(const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                         unsigned long long row0, int out_dim, const float* x, const float* x2, float lim,
                         uint8_t* ws, int num_cus, hipStream_t s) {
    const GemvPlan plan = plan_gemv(n_tensors, in_dim, out_dim, 1, num_cus, true);
    if (plan.grid == 0) return hipSuccess;
    GemvArgs a{};
    a.nb = in_dim / kQK;
    const size_t skip = (size_t)(row0 / kTileRows) * a.nb * kRecordBytes;
    for (int i = 0; i < 2; ++i) {
        const int k = i < n_tensors ? i : 0;
        a.w[i] = w[k] + skip;
        a.y[i] = y[k];
    }
    a.n_tiles = (out_dim + kTileRows - 1) / kTileRows;
    a.n_records = (int)plan.n_records;
    a.out_dim = out_dim;
    a.cnt = reinterpret_cast<uint32_t*>(ws);
    a.part = reinterpret_cast<float*>(ws + ((size_t)plan.n_tiles_all * 4 + 255) / 256 * 256);
    a.x = x;
    a.x2 = x2;
    a.lim = lim;
    if (x2) return launch_gemv_nt<1, 2>(plan, a, s);
    return launch_gemv_nt<1, 1>(plan, a, s);
}

hipError_t launch_matvec_raw(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const float* x, float* y, hipStream_t s) {
    const int nb = in_dim / kQK;
    hipLaunchKernelGGL(k_matvec_raw, dim3((out_dim + 3) / 4), dim3(256), 0, s, w, nb, row0, out_dim, x,
                       y);
    return hipGetLastError();
}

}  // namespace gpeed
