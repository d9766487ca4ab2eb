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

template <int NT>
struct GemvCfg {
    static constexpr int kPairs = (NT + 1) / 2;
    static constexpr int kWaves = GEMV_WAVES;
    // records in flight per wavefront (register ring)
    static constexpr int kPF = NT <= 2 ? GEMV_PF : 2;
    // tiles one chunk may touch (LDS partial slots)
    static constexpr int kSlots = NT == 1 ? 8 : (NT == 2 ? 4 : 2);
};

// Activation sources (MODE):
//   0  prepared images in global memory, one unscale per (block, token)
//      (act_bytes layout), loaded with every record;
//   1  one fp32 vector x, prepared inside the kernel;
//   2  SwiGLU(g = x, u = x2) of one vector, prepared inside the kernel;
//   3  prepared images of one vector with one unscale per 64 elements
//      (act64 layout: the output of EPI 1), loaded with every record.
// Epilogues (EPI):
//   0  y = W x (per tensor);
//   1  two tensors (gate, up) with records interleaved per row tile; the
//      workgroup that completes a row tile writes h = SwiGLU(gate, up) of
//      its 64 rows as act64 images (the down projection's activation).
template <int MODE>
struct ModeCfg {
    // the activation of each record sits in the wavefront's own LDS region
    // (prepared from x, g/u, or copied from act64 images)
    static constexpr bool kPrep = MODE == 1 || MODE == 2 || MODE == 3;
    // MODE 1/2: records per wavefront (chunk <= kWaves * kMaxPer); each
    // wavefront prepares the activation blocks of its own records
    static constexpr int kMaxPer = 6;
};

// act64 layout (one vector, n = K/256 blocks): block b at b*1024, its
// image a (elements 64a..64a+63) at +a*256, slice beta (elements
// 64a+4beta..+3) at +beta*16: 4 fp16 hi then 4 fp16 lo (x ~ (hi+lo) * unscale);
// then unscales [n][4] (fp32) at n*1024.
size_t act64_bytes_n(int nb) { return ((size_t)nb * 1024 + (size_t)nb * 16 + 255) / 256 * 256; }

struct GemvArgs {
    const uint8_t* w[2];   // T64 records of the first requested tile, per tensor
    float* y[2];           // [n_tok][out_dim] per tensor
    const uint8_t* act;    // MODE 0/3: prepared activation
    const float* xsc;      // MODE 0: [nb][n_tok]; MODE 3: [nb][4] unscales
    uint32_t* cnt;         // tickets (zero between launches)
    float* part;           // chunk partials of shared tiles
    int nb;
    int n_tiles;           // row tiles per tensor
    int n_records;         // n_tensors * n_tiles * nb
    int out_dim;
    int chunk;             // records per workgroup
    int max_parts;
    const float* x;        // MODE 1/2: fp32 x (or g) ...
    const float* x2;       // ... and u for the SwiGLU input
    float lim;
    uint8_t* act_out;      // EPI 1: act64 images of SwiGLU(gate, up)
};

// buffer resource word 3 for raw (untyped) buffer loads on gfx9
constexpr int kBufferDword3 = 0x00020000;

template <int NT, int MODE>
struct Slots {
    static constexpr int value = ModeCfg<MODE>::kPrep ? 4 : GemvCfg<NT>::kSlots;
};

// Record rec of the launch (in chunk order): virtual tile vt = rec / nb;
// EPI 0 keeps the tensors one after the other (vt = tensor * n_tiles +
// row tile), EPI 1 interleaves them (vt = 2 * row tile + tensor).
template <int EPI>
__device__ __forceinline__ const uint8_t* record_ptr(const GemvArgs& g, int rec) {
    const int vt = rec / g.nb;
    const int b = rec - vt * g.nb;
    int ten, rt;
    if constexpr (EPI == 1) {
        ten = vt & 1;
        rt = vt >> 1;
    } else {
        ten = vt >= g.n_tiles ? 1 : 0;
        rt = vt - ten * g.n_tiles;
    }
    return g.w[ten] + ((size_t)rt * g.nb + b) * kRecordBytes;
}

template <int NT, int MODE, int EPI>
__device__ __forceinline__ void load_rec(Rec<(NT + 1) / 2>& r, const GemvArgs& g, int rec, uint32_t lane) {
    const uint8_t* p = record_ptr<EPI>(g, rec);
    if constexpr (ModeCfg<MODE>::kPrep) {
        load_record_w(r, p, lane);  // images come from LDS
    } else {
        const int b = rec % g.nb;
        load_record<(NT + 1) / 2>(r, p, g.act + (size_t)b * NT * 1024, lane, NT);
    }
}

__device__ __forceinline__ float swiglu1(float gv, float uv, float lim) {
    const float gi = fminf(gv, lim);
    const float ui = fminf(fmaxf(uv, -lim), lim);
    return (gi / (1.0f + expf(-gi))) * ui;
}

// Power of two that brings max|v| over the wavefront (m: this lane's max)
// into [2^13, 2^14).
__device__ __forceinline__ int pow2_scale(float m) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    int sc = 0;
    if (m > 0.0f && m < __builtin_inff()) {
        int ex;
        (void)frexpf(m, &ex);  // m in [2^(ex-1), 2^ex)
        sc = 14 - ex;
        sc = sc > 120 ? 120 : (sc < -120 ? -120 : sc);
    }
    return sc;
}

// Block scale of the wavefront's 256 values and the fp16 hi/lo split of
// this lane's 4 values; returns the unscale.
__device__ __forceinline__ float split_hi_lo(const float (&e)[4], u32x2_t& hi2, u32x2_t& lo2) {
    const int sc =
        pow2_scale(fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3]))));
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

// y (per tensor) or, EPI 1, act64 images from the per-workgroup row sums.
// Structure:
//   prologue  grid table from immediates, the wavefronts' activation loads
//             (MODE 1/2), one workgroup barrier (no memory wait before it),
//             then the record ring and each wavefront's own preparation;
//   loop      wavefront w streams records c0+w, c0+w+W, ... of its chunk;
//   epilogue  per-tile sums over the wavefronts, shared tiles completed by
//             the last workgroup to arrive (ticket), partials added in chunk
//             order (results do not depend on timing).
template <int NT, int MODE, int EPI>
__global__ __launch_bounds__(GemvCfg<NT>::kWaves * 64) void k_gemv_t64(GemvArgs g) {
    static_assert(MODE == 0 || NT == 1, "prepared-in-kernel and act64 activations take one vector");
    static_assert(EPI == 0 || (NT == 1 && MODE == 1), "the SwiGLU epilogue takes gate/up of one vector");
    constexpr int W = GemvCfg<NT>::kWaves;
    constexpr int PF = GemvCfg<NT>::kPF;
    constexpr int S = Slots<NT, MODE>::value;
    constexpr int NP = GemvCfg<NT>::kPairs;
    constexpr int kThreads = W * 64;
    constexpr bool kPrep = ModeCfg<MODE>::kPrep;
    constexpr int KP = kPrep ? ModeCfg<MODE>::kMaxPer : 1;
    __shared__ __attribute__((aligned(16))) uint8_t tbl[kGridTableBytes];
    __shared__ float red[S][W][NT][64];
    __shared__ int last_flag[S];
    __shared__ __attribute__((aligned(16))) uint8_t xsl[kPrep ? W * KP * 1024 : 16];
    __shared__ __attribute__((aligned(16))) float xscl[kPrep ? W * KP * (MODE == 3 ? 4 : 1) : 1];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lane = tid & 63;
    const uint32_t lb = (lane & 31u) << 3;  // this lane's replica of the grid table

    // grid table and zeroed partials: LDS writes only, no memory dependence
    grid_table_literal<W>(tbl, wave, lane);
    for (int i = tid; i < S * W * NT * 64; i += kThreads) (&red[0][0][0][0])[i] = 0.0f;

    const int c0 = blockIdx.x * g.chunk;
    const int c1 = min(c0 + g.chunk, g.n_records);
    const int n_mine = c1 - c0 > wave ? (c1 - c0 - wave + W - 1) / W : 0;
    const int tile0 = c0 / g.nb;

    // The activation of each of this wavefront's records: its fp32 block
    // (MODE 1), g and u blocks (MODE 2) or its act64 images and unscales
    // (MODE 3), 16 bytes per lane. Buffer loads: an offset past the end
    // returns zeros without a memory access, so every wavefront issues the
    // same loads, unbranched.
    float4 xv[KP], uv[MODE == 2 ? KP : 1], sv[MODE == 3 ? KP : 1];
    if constexpr (kPrep) {
        const void* src = MODE == 3 ? static_cast<const void*>(g.act) : static_cast<const void*>(g.x);
        const auto xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(src), 0, g.nb * 1024, kBufferDword3);
        const auto ur = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(MODE == 3 ? g.xsc : g.x2), 0,
                                                          MODE == 3 ? g.nb * 16 : g.nb * 1024, kBufferDword3);
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            const int b = (c0 + wave + k * W) % g.nb;
            const bool ok = k < n_mine;
            const uint32_t off = ok ? (uint32_t)b * 1024u + lane * 16u : 0x80000000u;
            xv[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
            if constexpr (MODE == 2)
                uv[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, 0));
            if constexpr (MODE == 3)
                sv[k] = __builtin_bit_cast(
                    float4, __builtin_amdgcn_raw_buffer_load_b128(ur, ok ? (uint32_t)b * 16u : 0x80000000u, 0, 0));
        }
    }
    // One barrier: the table is complete, and (a CU serves its vector memory
    // queue in order) every wavefront's activation loads are queued ahead of
    // all record loads. Nothing before it waits for memory.
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // First ring slot, then this wavefront's activation (its loads were
    // queued first, so waiting for them does not wait for the records),
    // then the remaining slots: a CU takes only so many outstanding loads,
    // and a wavefront stalled issuing records cannot prepare.
    Rec<NP> ring[PF];
    load_rec<NT, MODE, EPI>(ring[0], g, min(c0 + wave, c1 - 1), lane);

    if constexpr (MODE == 3) {
        // copy: the act64 block keeps its layout in the private region
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            if (k < n_mine) {
                *reinterpret_cast<float4*>(xsl + (wave * KP + k) * 1024 + lane * 16) = xv[k];
                if (lane == 0) *reinterpret_cast<float4*>(&xscl[(wave * KP + k) * 4]) = sv[k];
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else if constexpr (kPrep) {
        // this wavefront's images (private LDS region: no workgroup barrier)
        const int a = lane >> 4, beta = lane & 15;
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            if (k < n_mine) {
                float e[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
                if constexpr (MODE == 2) {
                    const float us[4] = {uv[k].x, uv[k].y, uv[k].z, uv[k].w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) e[c] = swiglu1(e[c], us[c], g.lim);
                }
                u32x2_t hi, lo;
                const float unscale = split_hi_lo(e, hi, lo);
                // lane 4*beta+rho of register a holds variant rho (0 hi, 1 lo)
                // of slice beta at a*256 + (2*beta+rho)*8
                uint8_t* dst = xsl + (wave * KP + k) * 1024 + a * 256 + beta * 16;
                *reinterpret_cast<u32x2_t*>(dst) = hi;
                *reinterpret_cast<u32x2_t*>(dst + 8) = lo;
                if (lane == 0) xscl[wave * KP + k] = unscale;
            }
        }
        // lanes read other lanes' writes of the same wavefront: LDS
        // operations of one wavefront complete in order
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
#pragma unroll
    for (int s = 1; s < PF; ++s) load_rec<NT, MODE, EPI>(ring[s], g, min(c0 + wave + s * W, c1 - 1), lane);

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
                const float d4 = (float)__builtin_bit_cast(_Float16, (uint16_t)ring[s].d) * 0.25f;
                if constexpr (kPrep) {
                    const uint8_t* src = xsl + (wave * KP + k) * 1024 + ((lane >> 2) * 2 + (lane & 1)) * 8;
#pragma unroll
                    for (int a = 0; a < 4; ++a) ring[s].a[0][a] = *reinterpret_cast<const u32x2_t*>(src + a * 256);
                }
                if constexpr (MODE == 3) {
                    float blk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    record_dot_img(tbl, ring[s], lb, blk);
                    const float4 xs = *reinterpret_cast<const float4*>(&xscl[(wave * KP + k) * 4]);
                    acc[0] = fmaf(d4, fmaf(xs.x, blk[0], fmaf(xs.y, blk[1], fmaf(xs.z, blk[2], xs.w * blk[3]))),
                                  acc[0]);
                } else {
                    float us = 0.0f;
                    if constexpr (kPrep) us = xscl[wave * KP + k];
                    float blk[2 * NP];
#pragma unroll
                    for (int t = 0; t < 2 * NP; ++t) blk[t] = 0.0f;
                    record_dot<NP>(tbl, ring[s], lb, blk);
                    if constexpr (kPrep) {
                        acc[0] = fmaf(d4 * us, blk[0], acc[0]);
                    } else {
                        const float* xs = g.xsc + (size_t)b * NT;
#pragma unroll
                        for (int t = 0; t < NT; ++t) acc[t] = fmaf(d4 * xs[t], blk[t], acc[t]);
                    }
                }
            }
            // refill, clamped to the chunk's last record (a valid address)
            load_rec<NT, MODE, EPI>(ring[s], g, min(c0 + wave + (k + PF) * W, c1 - 1), lane);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (cur_slot >= 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) red[cur_slot][wave][t][lane] = acc[t];
    }
    lds_barrier();

    const int n_slots = (c1 - 1) / g.nb - tile0 + 1;
    auto first_chunk = [&](int vt) { return vt * g.nb / g.chunk; };
    auto last_chunk = [&](int vt) { return ((vt + 1) * g.nb - 1) / g.chunk; };
    if constexpr (EPI == 0) {
        // Sum the wavefront partials per (tile, token, row) in wave order;
        // whole tiles go straight to y, tiles shared with a neighbouring
        // chunk (only the chunk's first and last can be) to the workspace.
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
        // Partials complete (vmcnt(0)) before any thread of the workgroup
        // takes a ticket; the ticket holder that completes a tile then reads
        // the other chunks' partials with coherent loads.
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
    } else {
        // EPI 1: virtual tiles 2r (gate) and 2r+1 (up) of row tile r; the
        // pair is shared by the chunks first_chunk(2r) .. last_chunk(2r+1).
        __shared__ int pair_state[S];  // 1: this workgroup completes the pair
        const int p0 = tile0 >> 1;
        const int n_pairs = (tile0 + n_slots - 1) / 2 - p0 + 1;
        // (a) wave sums of every touched virtual tile
        __shared__ float vsum[S][64];
        for (int o = tid; o < n_slots * 64; o += kThreads) {
            const int slot = o / 64, n = o & 63;
            float sum = 0.0f;
#pragma unroll
            for (int v = 0; v < W; ++v) sum += red[slot][v][0][n];
            vsum[slot][n] = sum;
        }
        __syncthreads();
        // (b) pairs wholly inside this chunk are final; the others publish
        // their partials and take a ticket
        for (int o = tid; o < n_slots * 64; o += kThreads) {
            const int slot = o / 64, n = o & 63;
            const int vt = tile0 + slot, pr = vt >> 1;
            const int first = first_chunk(2 * pr), last = last_chunk(2 * pr + 1);
            if (first != last)
                __hip_atomic_store(g.part + (((size_t)pr * g.max_parts + (blockIdx.x - first)) * 2 + (vt & 1)) * 64 + n,
                                   vsum[slot][n], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if (tid < n_pairs) {
            const int pr = p0 + tid;
            const int first = first_chunk(2 * pr), last = last_chunk(2 * pr + 1);
            int st = 1;
            if (first != last) {
                const uint32_t old = __hip_atomic_fetch_add(g.cnt + pr, 1u, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                st = old == (uint32_t)(last - first) ? 1 : 0;
            }
            pair_state[tid] = st;
        }
        __syncthreads();
        // (c) wavefront q completes pair p0+q: gate and up rows, SwiGLU,
        // power-of-two scale over the 64 values, fp16 hi/lo act64 images
        for (int q = wave; q < n_pairs; q += W) {
            if (!pair_state[q]) continue;  // uniform per wavefront
            const int pr = p0 + q;
            const int first = first_chunk(2 * pr), last = last_chunk(2 * pr + 1);
            float v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int vt = 2 * pr + h;
                if (first == last) {
                    v[h] = vsum[vt - tile0][lane];
                } else {
                    v[h] = 0.0f;
                    const int j0 = first_chunk(vt) - first, j1 = last_chunk(vt) - first;
                    for (int j = j0; j <= j1; ++j)
                        v[h] += __hip_atomic_load(g.part + (((size_t)pr * g.max_parts + j) * 2 + h) * 64 + lane,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            const float hv = swiglu1(v[0], v[1], g.lim);
            const int sc = pow2_scale(fabsf(hv));
            const float xs = ldexpf(hv, sc);
            const _Float16 hi = (_Float16)xs;
            const _Float16 lo = (_Float16)(xs - (float)hi);
            const int blk = pr >> 2, a = pr & 3, beta = lane >> 2, c = lane & 3;
            uint8_t* dst = g.act_out + (size_t)blk * 1024 + a * 256 + beta * 16 + c * 2;
            *reinterpret_cast<_Float16*>(dst) = hi;
            *reinterpret_cast<_Float16*>(dst + 8) = lo;
            if (lane == 0) {
                float* usc = reinterpret_cast<float*>(g.act_out + (size_t)(g.n_tiles / 4) * 1024);
                usc[blk * 4 + a] = ldexpf(1.0f, -sc);
            }
            if (lane == 0 && first != last)
                __hip_atomic_store(g.cnt + pr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
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

template <int NT, int MODE = 0, int EPI = 0>
hipError_t launch_gemv_nt(const GemvPlan& plan, GemvArgs a, hipStream_t s) {
    a.chunk = plan.chunk;
    a.max_parts = plan.max_parts;
    return launch_timed(kProfGemv, k_gemv_t64<NT, MODE, EPI>, dim3(plan.grid), dim3(GemvCfg<NT>::kWaves * 64), 0, s,
                        a);
}

// Largest chunk (records per workgroup) that touches at most S tiles.
constexpr int max_chunk_slots(int slots, int nb) { return (slots - 1) * nb + 1; }

GemvArgs base_args(const GemvPlan& plan, const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                   unsigned long long row0, int out_dim, uint8_t* ws) {
    GemvArgs a{};
    a.nb = in_dim / kQK;
    const size_t skip = (size_t)(row0 / kTileRows) * a.nb * kRecordBytes;
    for (int i = 0; i < 2; ++i) {
        const int k = i < n_tensors ? i : 0;
        a.w[i] = w[k] + skip;
        a.y[i] = y ? y[k] : nullptr;
    }
    a.n_tiles = (out_dim + kTileRows - 1) / kTileRows;
    a.n_records = (int)plan.n_records;
    a.out_dim = out_dim;
    a.cnt = reinterpret_cast<uint32_t*>(ws);
    a.part = reinterpret_cast<float*>(ws + ((size_t)plan.n_tiles_all * 4 + 255) / 256 * 256);
    return a;
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

GemvPlan plan_gemv(int n_tensors, int in_dim, int out_dim, int n_tok, int num_cus, int kind) {
    GemvPlan p{};
    const int nb = in_dim / kQK;
    const int n_tiles = (out_dim + kTileRows - 1) / kTileRows;
    p.n_tiles_all = (long long)n_tiles * n_tensors;
    const long long recs = p.n_tiles_all * nb;
    p.n_records = recs;
    const int cus = num_cus > 0 ? num_cus : 256;
    long long chunk = (recs + cus - 1) / cus;
    long long cap = 0;
    if (kind == kPlanPrep || kind == kPlanSwigluPairs) {
        cap = max_chunk_slots(Slots<1, 1>::value, nb);
        const long long per_wave = (long long)GemvCfg<1>::kWaves * ModeCfg<1>::kMaxPer;
        if (cap > per_wave) cap = per_wave;
    } else {
        switch (n_tok) {
            case 1: cap = max_chunk_slots(Slots<1, 0>::value, nb); break;
            case 2: cap = max_chunk_slots(Slots<2, 0>::value, nb); break;
            case 3: case 4: cap = max_chunk_slots(Slots<4, 0>::value, nb); break;
            default: cap = max_chunk_slots(Slots<8, 0>::value, nb); break;
        }
    }
    if (chunk > cap) chunk = cap;
    if (chunk < 1) chunk = 1;
    p.chunk = (int)chunk;
    p.grid = recs > 0 ? (int)((recs + chunk - 1) / chunk) : 0;
    // chunks one shared unit (a tile, or a gate/up pair of tiles) can span
    const long long unit = kind == kPlanSwigluPairs ? 2LL * nb : nb;
    p.max_parts = (int)((unit - 1) / chunk + 2);
    if (p.max_parts > unit) p.max_parts = (int)unit;
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
    const GemvPlan plan = plan_gemv(n_tensors, in_dim, out_dim, n_tok, num_cus, kPlanAct);
    if (plan.grid == 0) return hipSuccess;
    GemvArgs a = base_args(plan, w, y, n_tensors, in_dim, row0, out_dim, ws);
    a.act = act;
    a.xsc = reinterpret_cast<const float*>(act + (size_t)a.nb * n_tok * 1024);
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
    const GemvPlan plan = plan_gemv(n_tensors, in_dim, out_dim, 1, num_cus, kPlanPrep);
    if (plan.grid == 0) return hipSuccess;
    GemvArgs a = base_args(plan, w, y, n_tensors, in_dim, row0, out_dim, ws);
    a.x = x;
    a.x2 = x2;
    a.lim = lim;
    if (x2) return launch_gemv_nt<1, 2>(plan, a, s);
    return launch_gemv_nt<1, 1>(plan, a, s);
}

size_t act64_bytes(int in_dim) { return act64_bytes_n(in_dim / kQK); }

size_t gate_up_ws_bytes(int in_dim, int out_dim) {
    const long long nb = in_dim / kQK;
    const long long tiles = (out_dim + kTileRows - 1) / kTileRows;
    const size_t cnt = ((size_t)(2 * tiles) * 4 + 255) / 256 * 256;
    return cnt + (size_t)tiles * (size_t)(2 * nb) * 2 * 64 * 4;
}

hipError_t launch_gate_up_swiglu(const uint8_t* w_gate, const uint8_t* w_up, int in_dim, int out_dim,
                                 const float* x, float lim, uint8_t* act_out, uint8_t* ws, int num_cus,
                                 hipStream_t s) {
    if (out_dim % kQK) return hipErrorInvalidValue;  // act64 blocks of the output
    const GemvPlan plan = plan_gemv(2, in_dim, out_dim, 1, num_cus, kPlanSwigluPairs);
    if (plan.grid == 0) return hipSuccess;
    const uint8_t* w[2] = {w_gate, w_up};
    GemvArgs a = base_args(plan, w, nullptr, 2, in_dim, 0, out_dim, ws);
    a.x = x;
    a.x2 = x;
    a.lim = lim;
    a.act_out = act_out;
    return launch_gemv_nt<1, 1, 1>(plan, a, s);
}

hipError_t launch_gemv_act64(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const uint8_t* act64, float* y, uint8_t* ws, int num_cus, hipStream_t s) {
    const GemvPlan plan = plan_gemv(1, in_dim, out_dim, 1, num_cus, kPlanPrep);
    if (plan.grid == 0) return hipSuccess;
    float* yy[1] = {y};
    const uint8_t* ww[1] = {w};
    GemvArgs a = base_args(plan, ww, yy, 1, in_dim, row0, out_dim, ws);
    a.act = act64;
    a.xsc = reinterpret_cast<const float*>(act64 + (size_t)a.nb * 1024);
    return launch_gemv_nt<1, 3>(plan, a, s);
}

hipError_t launch_matvec_raw(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const float* x, float* y, hipStream_t s) {
    const int nb = in_dim / kQK;
    hipLaunchKernelGGL(k_matvec_raw, dim3((out_dim + 3) / 4), dim3(256), 0, s, w, nb, row0, out_dim, x,
                       y);
    return hipGetLastError();
}

}  // namespace gpeed
