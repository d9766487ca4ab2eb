// IQ3_XXS GEMV kernels (gfx950): y[t] = W x[t] for 1..8 activation vectors
// ("tokens") over the T64 layout.
//
// Work split. The (tile, block) records of the requested rows (of one or two
// same-shape tensors) are numbered tile-major and cut into equal contiguous
// chunks, one per workgroup, so every CU streams the same number of bytes
// whatever the tile count. Inside a workgroup the chunk's records are dealt
// round-robin to the wavefronts; a wavefront streams its records through a
// register ring (six coalesced 16-byte buffer loads and one 2-byte load per
// lane)
// and keeps a per-row partial sum per tile, which meets the other
// wavefronts' partials in LDS. A tile cut by a chunk boundary is finished by
// whichever of its workgroups arrives last (atomic ticket in a caller-owned
// workspace); it adds the workgroups' partials in chunk order, so results do
// not depend on timing. (The dense step's down launch instead adds such
// parts into an output the gate/up launch zero-filled, with atomic adds.)
//
// Decode and product. Lane n of a wavefront holds row n of the tile. Per
// group of 4 weights it makes one LDS lookup in its own replica of the grid
// table (4 unsigned fp16, no bank conflicts), sets the fp16 sign bits (one
// 64-bit shift places both pairs' signs, then two masked ors), and issues
// one v_mfma_f32_4x4x4_16b_f16 whose A
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
            e[c] = swiglu1(e[c], us[c], lim);
        }
    }
    const int sc =
        pow2_scale_of_max(wave_max(fmaxf(fmaxf(fabsf(e[0]), fabsf(e[1])), fmaxf(fabsf(e[2]), fabsf(e[3])))));
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

// Wavefronts per workgroup. (16 decode a record 13% faster in isolation,
// but the dense step measured 32.3 us with 16 for single-token records
// against 30.1 us with 8: fewer records per wavefront, more partial sums.)
constexpr int kGemvWaves = 8;

template <int NT>
struct GemvCfg {
    static constexpr int kPairs = (NT + 1) / 2;
    static constexpr int kWaves = kGemvWaves;
    // records in flight per wavefront (register ring; 3 measured slower)
    static constexpr int kPF = 2;
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
    // wavefront prepares the activation blocks of its own records (48
    // records, 48 KB of images, per workgroup)
    static constexpr int kMaxPer = 48 / kGemvWaves;
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
    uint64_t* part;        // chunk partials of shared tiles (tagged words)
    uint32_t* err;         // the workspace's error word (kWs* flags)
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
    uint32_t w_bytes;      // bytes of each tensor's records from w[i] (< 2^31)
    // MODE 1: row tiles [h*tiles_per_head, (h+1)*tiles_per_head) take their
    // activation from x + h*head_stride bytes (one input vector per head of
    // a per-head projection); one vector for all rows: tiles_per_head huge,
    // head_stride 0. x_bytes: bytes readable from x.
    int tiles_per_head;
    uint32_t head_stride;
    uint32_t x_bytes;
    // EPI 1: n_zero floats at y_zero set to zero (the next launch's output)
    float* y_zero;
    int n_zero;
    // EPI 0: y is zero at the launch's start; shared row tiles are added into
    // it with atomic adds
    int y_atomic;
};

// buffer resource word 3 for raw (untyped) buffer loads on gfx9
constexpr int kBufferDword3 = 0x00020000;
// a buffer offset no resource here reaches: the load returns zeros and
// touches no memory
constexpr uint32_t kOutOfRange = 0x80000000u;

template <int NT, int MODE>
struct Slots {
    static constexpr int value = ModeCfg<MODE>::kPrep ? 4 : GemvCfg<NT>::kSlots;
};

// Record rec of the launch (in chunk order): virtual tile vt = rec / nb;
// EPI 0 keeps the tensors one after the other (vt = tensor * n_tiles +
// row tile), EPI 1 interleaves them (vt = 2 * row tile + tensor).
template <int NT, int MODE, int EPI>
__device__ __forceinline__ void load_rec(Rec<(NT + 1) / 2>& r, const GemvArgs& g, int rec, bool live,
                                         uint32_t lane) {
    constexpr int NP = (NT + 1) / 2;
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
    // buffer loads: a slot refilled past the wavefront's records gets an
    // out-of-range offset, so it costs no memory traffic (and no place in
    // the queue ahead of the epilogue's loads and stores)
    // (the tensor's base by arithmetic on both fields, not an index into
    // w: the kernel's copy of the arguments then stays in registers)
    const uintptr_t w0 = reinterpret_cast<uintptr_t>(g.w[0]), w1 = reinterpret_cast<uintptr_t>(g.w[1]);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<uint8_t*>(w0 + (ten ? w1 - w0 : 0)), 0,
                                                      g.w_bytes, kBufferDword3);
    const uint32_t off = live ? (uint32_t)(rt * g.nb + b) * (uint32_t)kRecordBytes : kOutOfRange;
#pragma unroll
    for (int i = 0; i < 6; ++i)
        r.u[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, off + i * kUnitBytes + lane * 16u, 0, 0));
    r.d = __builtin_amdgcn_raw_buffer_load_b16(rs, off + kRecordDOffset + lane * 2u, 0, 0);
    if constexpr (!ModeCfg<MODE>::kPrep) {
        // the record's prepared activation (n_tok vectors; a last pair with
        // one token stores rows 0, 1 only, 256-byte images)
        const auto ra =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(g.act), 0, g.nb * NT * 1024, kBufferDword3);
        const uint32_t aoff = live ? (uint32_t)b * NT * 1024u : kOutOfRange;
        const uint32_t off_half = ((lane >> 2) * 2 + (lane & 1)) * 8u;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const bool half = (p == NP - 1) && (NT & 1);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const uint32_t o = aoff + p * 2048 + (half ? a * 256u + off_half : a * 512u + lane * 8u);
                r.a[p][a] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(ra, o, 0, 0));
            }
        }
        if constexpr (MODE == 0) {
            const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.xsc), 0, g.nb * NT * 4, kBufferDword3);
            const uint32_t t = min(lane & 7u, (uint32_t)NT - 1u);
            r.xs = __builtin_amdgcn_raw_buffer_load_b32(rx, live ? ((uint32_t)b * NT + t) * 4u : kOutOfRange, 0, 0);
        }
    }
}

// Power of two that brings max|v| over the wavefront (m: this lane's max)
// into [2^13, 2^14).
__device__ __forceinline__ int pow2_scale(float m) { return pow2_scale_of_max(wave_max(m)); }

// ---------------------------------------------------------------------------
// GEMV workgroup building blocks. A workgroup owns records [c0, c1) of a
// launch (chunk order); wavefront w streams records c0+w, c0+w+W, ... (its
// k-th record is c0 + w + k*W) through a register ring of PF slots.

// LDS of one workgroup; layout L = 1 when the activation images sit in
// per-wavefront regions (MODE 1, 2, 3), 0 when they come with the records.
template <int MODE>
constexpr int shared_layout() { return ModeCfg<MODE>::kPrep ? 1 : 0; }

template <int NT, int L>
struct GemvShared {
    static constexpr int W = GemvCfg<NT>::kWaves;
    static constexpr int S = L ? 4 : GemvCfg<NT>::kSlots;
    static constexpr bool kPrep = L != 0;
    static constexpr int KP = kPrep ? ModeCfg<1>::kMaxPer : 1;
    __attribute__((aligned(16))) uint8_t tbl[kGridTableBytes];  // replicated grid table
    float red[S][W][NT][64];                                     // wavefront row sums per tile slot
    __attribute__((aligned(16))) uint8_t xsl[kPrep ? W * KP * 1024 : 16];  // per-wavefront activation images
    __attribute__((aligned(16))) float xscl[kPrep ? W * KP * 4 : 4];      // and their unscales
    float vsum[S][64];                                           // workgroup row sums (SwiGLU epilogue)
};

// The chunk of workgroup `blk` and this wavefront's share of it.
struct Chunk {
    int c0, c1, n_mine, tile0;
    __device__ Chunk(const GemvArgs& g, int blk, int wave, int W) {
        c0 = blk * g.chunk;
        c1 = min(c0 + g.chunk, g.n_records);
        n_mine = c1 - c0 > wave ? (c1 - c0 - wave + W - 1) / W : 0;
        tile0 = c0 / g.nb;
    }
    __device__ int rec(int k, int wave, int W) const { return min(c0 + wave + k * W, c1 - 1); }
};

// Records of one launch for the ring: k-th record of this wavefront.
template <int NT, int MODE, int EPI>
struct OnePhase {
    const GemvArgs& g;
    Chunk ch;
    int wave;
    static constexpr int W = GemvCfg<NT>::kWaves;
    __device__ void load(Rec<(NT + 1) / 2>& r, int k, uint32_t lane) const {
        load_rec<NT, MODE, EPI>(r, g, ch.rec(k, wave, W), k < ch.n_mine, lane);
    }
};

// Grid table (immediate data) and zeroed row sums: LDS writes only.
template <int NT, int MODE>
__device__ __forceinline__ void gemv_lds_init(GemvShared<NT, shared_layout<MODE>()>& sh, int wave, uint32_t lane,
                                              int tid) {
    constexpr int W = GemvCfg<NT>::kWaves, S = GemvShared<NT, shared_layout<MODE>()>::S;
    grid_table_literal<W>(sh.tbl, wave, lane);
    for (int i = tid; i < S * W * NT * 64; i += W * 64) (&sh.red[0][0][0][0])[i] = 0.0f;
}

// The activation of each of this wavefront's records: its fp32 block
// (MODE 1), g and u blocks (MODE 2) or its act64 images and unscales
// (MODE 3), 16 bytes per lane. Buffer loads: an offset past the end returns
// zeros without a memory access, so every wavefront issues the same loads,
// unbranched. kCoherent: read past other XCDs' caches (data written by
// other workgroups of the same launch).
template <int MODE, int KP, int W, bool kCoherent = false>
struct ActLoads {
    float4 xv[KP], uv[MODE == 2 ? KP : 1], sv[MODE == 3 ? KP : 1];
    __device__ void issue(const GemvArgs& g, const Chunk& ch, int wave, uint32_t lane) {
        constexpr int kAux = kCoherent ? 16 : 0;  // sc1
        const void* src = MODE == 3 ? static_cast<const void*>(g.act) : static_cast<const void*>(g.x);
        const auto xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(src), 0,
                                                          MODE == 3 ? g.nb * 1024 : (int)g.x_bytes, kBufferDword3);
        const auto ur = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(MODE == 3 ? g.xsc : g.x2), 0,
                                                          MODE == 3 ? g.nb * 16 : g.nb * 1024, kBufferDword3);
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            const int rec = ch.c0 + wave + k * W;
            const int b = rec % g.nb;
            const bool ok = k < ch.n_mine;
            // the head of the record's row tile (MODE 1 per-head inputs)
            const uint32_t hoff = MODE == 1 ? (uint32_t)(rec / g.nb / g.tiles_per_head) * g.head_stride : 0u;
            const uint32_t off = ok ? hoff + (uint32_t)b * 1024u + lane * 16u : 0x80000000u;
            xv[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, kAux));
            if constexpr (MODE == 2)
                uv[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, kAux));
            if constexpr (MODE == 3)
                sv[k] = __builtin_bit_cast(
                    float4, __builtin_amdgcn_raw_buffer_load_b128(ur, ok ? (uint32_t)b * 16u : 0x80000000u, 0, kAux));
        }
    }
    // images (prepared, or copied for MODE 3) into the wavefront's region
    template <int NT>
    __device__ void commit(GemvShared<NT, 1>& sh, const GemvArgs& g, const Chunk& ch, int wave, uint32_t lane) {
        if constexpr (MODE == 3) {
#pragma unroll
            for (int k = 0; k < KP; ++k) {
                if (k < ch.n_mine) {
                    uint8_t* region = sh.xsl + (wave * KP + k) * 1024;
                    *reinterpret_cast<float4*>(region + lane * 16) = xv[k];  // act64 keeps its layout
                    if (lane == 0) *reinterpret_cast<float4*>(&sh.xscl[(wave * KP + k) * 4]) = sv[k];
                }
            }
        } else {
            // the block scales of all records first, unbranched (a record
            // past the wavefront's share holds zeros), so their wavefront
            // reductions overlap
            float e[KP][4];
            int sc[KP];
#pragma unroll
            for (int k = 0; k < KP; ++k) {
                e[k][0] = xv[k].x;
                e[k][1] = xv[k].y;
                e[k][2] = xv[k].z;
                e[k][3] = xv[k].w;
                if constexpr (MODE == 2) {
                    const float us[4] = {uv[k].x, uv[k].y, uv[k].z, uv[k].w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) e[k][c] = swiglu1(e[k][c], us[c], g.lim);
                }
                sc[k] = pow2_scale(fmaxf(fmaxf(fabsf(e[k][0]), fabsf(e[k][1])), fmaxf(fabsf(e[k][2]), fabsf(e[k][3]))));
            }
#pragma unroll
            for (int k = 0; k < KP; ++k) {
                if (k < ch.n_mine) {
                    _Float16 hi[4], lo[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const float xs = ldexpf(e[k][c], sc[k]);
                        hi[c] = (_Float16)xs;
                        lo[c] = (_Float16)(xs - (float)hi[c]);
                    }
                    // lane 4*beta+rho of register a holds variant rho (0 hi,
                    // 1 lo) of slice beta at a*256 + (2*beta+rho)*8
                    uint8_t* dst = sh.xsl + (wave * KP + k) * 1024 + (lane >> 4) * 256 + (lane & 15) * 16;
                    *reinterpret_cast<u32x2_t*>(dst) = __builtin_bit_cast(u32x2_t, hi);
                    *reinterpret_cast<u32x2_t*>(dst + 8) = __builtin_bit_cast(u32x2_t, lo);
                    if (lane == 0) sh.xscl[(wave * KP + k) * 4] = ldexpf(1.0f, -sc[k]);
                }
            }
        }
        // lanes read other lanes' writes of the same wavefront: LDS
        // operations of one wavefront complete in order
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
};

// Records k in [kbeg, kend) of this wavefront's sequence `src`, whose ring
// slot k % PF already holds record k; the row sums go to sh.red by tile
// slot. A slot is refilled with record k + PF after its use, and only
// then: past kend it keeps its record (the next phase's), so the loads stay
// the same whatever the branch and the compiler waits for exactly the slot
// it needs.
template <int NT, int MODE, int EPI, typename Src>
__device__ __forceinline__ void gemv_stream(GemvShared<NT, shared_layout<MODE>()>& sh, const GemvArgs& g,
                                            Rec<(NT + 1) / 2> (&ring)[GemvCfg<NT>::kPF],
                                            const Src& src, const Chunk& ch, int kbeg, int kend, int wave,
                                            uint32_t lane) {
    constexpr int W = GemvCfg<NT>::kWaves, PF = GemvCfg<NT>::kPF, NP = GemvCfg<NT>::kPairs;
    constexpr bool kPrep = ModeCfg<MODE>::kPrep;
    constexpr int KP = GemvShared<NT, shared_layout<MODE>()>::KP;
    const uint32_t lb = (lane & 31u) << 3;  // this lane's replica of the grid table
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    int cur_slot = -1;
    for (int k0 = kbeg - kbeg % PF; k0 < kend; k0 += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            const int k = k0 + s;
            const int kk = k - kbeg;  // index within this phase
            const bool valid = k >= kbeg && k < kend;
            const int rec = ch.rec(kk, wave, W);
            const int slot = rec / g.nb - ch.tile0;
            if (valid && slot != cur_slot) {
                if (cur_slot >= 0) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) sh.red[cur_slot][wave][t][lane] = acc[t];
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
                cur_slot = slot;
            }
            if (valid) {
                const float d4 = (float)__builtin_bit_cast(_Float16, (uint16_t)ring[s].d) * 0.25f;
                // 0 for a finite d, NaN for an infinite or NaN one: the
                // reference sums a block of d = +-inf as +-inf products of
                // both signs (NaN), where d * (finite partial) would give
                // +-inf, so such a block makes the row NaN
                const float dz = d4 - d4;
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[t] += dz;
                if constexpr (kPrep) {
                    const uint8_t* a_src = sh.xsl + (wave * KP + kk) * 1024 + ((lane >> 2) * 2 + (lane & 1)) * 8;
#pragma unroll
                    for (int a = 0; a < 4; ++a) ring[s].a[0][a] = *reinterpret_cast<const u32x2_t*>(a_src + a * 256);
                }
                if constexpr (MODE == 3) {
                    float blk[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    record_dot<1, true>(sh.tbl, ring[s], lb, blk);
                    const float4 xs = *reinterpret_cast<const float4*>(&sh.xscl[(wave * KP + kk) * 4]);
                    acc[0] = fmaf(d4, fmaf(xs.x, blk[0], fmaf(xs.y, blk[1], fmaf(xs.z, blk[2], xs.w * blk[3]))),
                                  acc[0]);
                } else {
                    float blk[2 * NP];
#pragma unroll
                    for (int t = 0; t < 2 * NP; ++t) blk[t] = 0.0f;
                    record_dot<NP>(sh.tbl, ring[s], lb, blk);
                    if constexpr (kPrep) {
                        acc[0] = fmaf(d4 * sh.xscl[(wave * KP + kk) * 4], blk[0], acc[0]);
                    } else {
#pragma unroll
                        for (int t = 0; t < NT; ++t) acc[t] = fmaf(d4 * rec_unscale(ring[s], t), blk[t], acc[t]);
                    }
                }
            }
            // refill with record k + PF once used; otherwise reload what the
            // slot holds (k + PF before kbeg, k itself from kend on)
            src.load(ring[s], k < kend ? k + PF : k, lane);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (cur_slot >= 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) sh.red[cur_slot][wave][t][lane] = acc[t];
    }
}

// Shared-tile partials. A tile (or gate/up pair) cut by chunk boundaries
// has one part per chunk; each part's values are published as tagged 64-bit
// words (value bits | 1 << 32, single-copy atomic), so a reader knows a
// value has landed without waiting for the writer's stores to complete
// (the tag is the only ordering the hand-off needs: no fence is required).
// The workgroup that takes the unit's last ticket (one relaxed atomic per
// unit, issued right after its own words) sums the parts in part order;
// another part's word not yet landed is read again (its writer issued it
// before taking its ticket, so it lands: the bound only guards against a
// corrupted or shared workspace, and giving up sets kWsTimeout). A ticket
// beyond the unit's part count (a workspace not zero-filled, or shared by
// overlapping launches) sets kWsTicket. The summing workgroup clears the
// words and the ticket, leaving the workspace zero for the next launch.
constexpr int kTagSpin = 1 << 20;

__device__ __forceinline__ void flag_ws(uint32_t* err, uint32_t bits) {
    __hip_atomic_fetch_or(err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void put_tagged(uint64_t* p, float v) {
    __hip_atomic_store(p, (1ull << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_tagged(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// acc[t] = sum over parts j0[t]..j1[t] (in order) of word p[j * part_stride
// + t * 64]; part `me` contributes mine[t] instead. The loads of up to four
// parts are in flight at once. The words read are cleared.
template <int NT>
__device__ __forceinline__ void sum_tagged_parts(uint64_t* p, size_t part_stride, const int (&j0)[NT],
                                                 const int (&j1)[NT], int me, const float (&mine)[NT],
                                                 float (&acc)[NT], uint32_t* err) {
    int lo = j0[0], hi = j1[0];
#pragma unroll
    for (int t = 1; t < NT; ++t) {
        lo = min(lo, j0[t]);
        hi = max(hi, j1[t]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    for (int jb = lo; jb <= hi; jb += 4) {
        uint64_t v[4][NT];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = jb + i;
#pragma unroll
            for (int t = 0; t < NT; ++t)
                v[i][t] = (j >= j0[t] && j <= j1[t] && j != me) ? get_tagged(p + j * part_stride + t * 64) : 0;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = jb + i;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (j < j0[t] || j > j1[t]) continue;
                float x = mine[t];
                if (j != me) {
                    uint64_t w = v[i][t];
                    for (int spin = 0; (w >> 32) == 0 && spin < kTagSpin; ++spin)
                        w = get_tagged(p + j * part_stride + t * 64);
                    if ((w >> 32) == 0) flag_ws(err, kWsTimeout);
                    x = __builtin_bit_cast(float, (uint32_t)w);
                }
                acc[t] += x;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
        for (int j = j0[t]; j <= j1[t]; ++j)
            __hip_atomic_store(p + j * part_stride + t * 64, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Ticket of a shared unit with n_parts parts, taken by lane 0 and returned
// to the wavefront; a ticket past the last sets kWsTicket.
__device__ __forceinline__ uint32_t take_ticket(uint32_t* cnt, uint32_t lane, int n_parts, uint32_t* err) {
    uint32_t old = 0;
    if (lane == 0) {
        old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old >= (uint32_t)n_parts) flag_ws(err, kWsTicket);
    }
    return __builtin_amdgcn_readfirstlane(old);
}

// EPI 0 epilogue: wavefront w finishes the chunk's tile slots w, w + W, ...:
// the wavefront partials summed in wave order; a whole tile goes straight
// to y, a shared tile's part is published, and the last ticket holder adds
// the parts in chunk order — bitwise repeatable; or, with g.y_atomic, the
// part is added into the zero-filled y. Call after a barrier that completes
// sh.red.
template <int NT, int MODE>
__device__ __forceinline__ void gemv_epilogue_y(GemvShared<NT, shared_layout<MODE>()>& sh, const GemvArgs& g,
                                                const Chunk& ch, int blk, int wave, uint32_t lane) {
    constexpr int W = GemvCfg<NT>::kWaves;
    const int n_slots = (ch.c1 - 1) / g.nb - ch.tile0 + 1;
    for (int slot = wave; slot < n_slots; slot += W) {
        const int tile = ch.tile0 + slot;
        const int first = tile * g.nb / g.chunk, last = ((tile + 1) * g.nb - 1) / g.chunk;
        float sum[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            sum[t] = 0.0f;
#pragma unroll
            for (int v = 0; v < W; ++v) sum[t] += sh.red[slot][v][t][lane];
        }
        if (first != last && g.y_atomic) {
            // y started at zero: each part adds its sums and leaves (the
            // order of the two to four adds varies from run to run, so the
            // result is repeatable to within their fp32 rounding)
            const int ten = tile >= g.n_tiles ? 1 : 0;
            const int row = (tile - ten * g.n_tiles) * kTileRows + lane;
            if (row < g.out_dim) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    __hip_atomic_fetch_add((ten ? g.y[1] : g.y[0]) + (size_t)t * g.out_dim + row, sum[t],
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            continue;
        }
        if (first != last) {
            uint64_t* p = g.part + ((size_t)tile * g.max_parts * NT) * 64 + lane;
#pragma unroll
            for (int t = 0; t < NT; ++t) put_tagged(p + ((size_t)(blk - first) * NT + t) * 64, sum[t]);
            if (take_ticket(g.cnt + tile, lane, last - first + 1, g.err) != (uint32_t)(last - first)) continue;
            float tot[NT];
            int j0[NT], j1[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                j0[t] = 0;
                j1[t] = last - first;
            }
            sum_tagged_parts<NT>(p, (size_t)NT * 64, j0, j1, blk - first, sum, tot, g.err);
#pragma unroll
            for (int t = 0; t < NT; ++t) sum[t] = tot[t];
            if (lane == 0) __hip_atomic_store(g.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const int ten = tile >= g.n_tiles ? 1 : 0;
        const int row = (tile - ten * g.n_tiles) * kTileRows + lane;
        if (row < g.out_dim) {
#pragma unroll
            for (int t = 0; t < NT; ++t) (ten ? g.y[1] : g.y[0])[(size_t)t * g.out_dim + row] = sum[t];
        }
    }
}

// EPI 1 epilogue: virtual tiles 2r (gate) and 2r+1 (up) of row tile r form
// a pair shared by chunks first_chunk(2r) .. last_chunk(2r+1); wavefront q
// finishes the chunk's pair p0 + q (publishes its parts; if it completes
// the pair, writes SwiGLU of the 64 rows as act64 images).
__device__ __forceinline__ void gemv_epilogue_swiglu(GemvShared<1, 1>& sh, const GemvArgs& g, const Chunk& ch,
                                                     int blk, int tid, int wave, uint32_t lane) {
    constexpr int W = GemvCfg<1>::kWaves, kThreads = W * 64;
    const int n_slots = (ch.c1 - 1) / g.nb - ch.tile0 + 1;
    auto first_chunk = [&](int vt) { return vt * g.nb / g.chunk; };
    auto last_chunk = [&](int vt) { return ((vt + 1) * g.nb - 1) / g.chunk; };
    const int p0 = ch.tile0 >> 1;
    const int n_pairs = (ch.tile0 + n_slots - 1) / 2 - p0 + 1;
    // wavefront sums of every touched virtual tile
    for (int o = tid; o < n_slots * 64; o += kThreads) {
        const int slot = o / 64, n = o & 63;
        float sum = 0.0f;
#pragma unroll
        for (int v = 0; v < W; ++v) sum += sh.red[slot][v][0][n];
        sh.vsum[slot][n] = sum;
    }
    lds_barrier();
    for (int q = wave; q < n_pairs; q += W) {
        const int pr = p0 + q;
        const int first = first_chunk(2 * pr), last = last_chunk(2 * pr + 1);
        float v[2];
        if (first == last) {
            v[0] = sh.vsum[2 * pr - ch.tile0][lane];
            v[1] = sh.vsum[2 * pr + 1 - ch.tile0][lane];
        } else {
            uint64_t* p = g.part + ((size_t)pr * g.max_parts * 2) * 64 + lane;
            const int me = blk - first;
            float mine[2] = {0.0f, 0.0f};
            int j0[2], j1[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int vt = 2 * pr + h, slot = vt - ch.tile0;
                j0[h] = first_chunk(vt) - first;
                j1[h] = last_chunk(vt) - first;
                if (slot >= 0 && slot < n_slots) {
                    mine[h] = sh.vsum[slot][lane];
                    put_tagged(p + ((size_t)me * 2 + h) * 64, mine[h]);
                }
            }
            if (take_ticket(g.cnt + pr, lane, last - first + 1, g.err) != (uint32_t)(last - first)) continue;
            sum_tagged_parts<2>(p, 2 * 64, j0, j1, me, mine, v, g.err);
            if (lane == 0) __hip_atomic_store(g.cnt + pr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const float hv = swiglu1(v[0], v[1], g.lim);
        const int sc = pow2_scale(fabsf(hv));
        const float xs = ldexpf(hv, sc);
        const _Float16 hi = (_Float16)xs;
        const _Float16 lo = (_Float16)(xs - (float)hi);
        // element `lane` of image a = pr & 3 of block pr >> 2: slice beta =
        // lane >> 2 at +beta*16, hi at +2c, lo at +8+2c (c = lane & 3)
        const int blk_o = pr >> 2, a = pr & 3, beta = lane >> 2, c = lane & 3;
        uint8_t* dst = g.act_out + (size_t)blk_o * 1024 + a * 256 + beta * 16;
        float* usc = reinterpret_cast<float*>(g.act_out + (size_t)(g.n_tiles / 4) * 1024);
        *reinterpret_cast<_Float16*>(dst + 2 * c) = hi;
        *reinterpret_cast<_Float16*>(dst + 8 + 2 * c) = lo;
        if (lane == 0) usc[blk_o * 4 + a] = ldexpf(1.0f, -sc);
    }
}

// y (per tensor) or, EPI 1, act64 images: prologue (the wavefronts'
// activation loads, a workgroup barrier with no memory wait, the first ring
// slot, the grid table, the wavefront's own activation images, the other
// slots), the record stream, the epilogue.
// The fields the prologue needs first come as leading scalar arguments,
// which the launch preloads into SGPRs (-amdgpu-kernarg-preload-count): the
// first record loads then wait for no kernel-argument read (0.4 us earlier
// on the 6144x12288 launch). The copy g takes them and reads the rest from
// the kernel arguments; no field of it is indexed at run time, so it stays
// in registers.
template <int NT, int MODE, int EPI>
__global__ __launch_bounds__(GemvCfg<NT>::kWaves * 64) void k_gemv_t64(const uint8_t* w0, const uint8_t* w1,
                                                                        const void* asrc, int chunk, int n_records,
                                                                        int nb, GemvArgs g_in) {
    GemvArgs g = g_in;
    g.w[0] = w0;
    g.w[1] = w1;
    g.chunk = chunk;
    g.n_records = n_records;
    g.nb = nb;
    if constexpr (MODE == 1 || MODE == 2)
        g.x = static_cast<const float*>(asrc);
    else
        g.act = static_cast<const uint8_t*>(asrc);
    static_assert(MODE == 0 || NT == 1, "prepared-in-kernel and act64 activations take one vector");
    static_assert(EPI == 0 || (NT == 1 && MODE == 1), "the SwiGLU epilogue takes gate/up of one vector");
    constexpr int W = GemvCfg<NT>::kWaves;
    constexpr int PF = GemvCfg<NT>::kPF;
    constexpr bool kPrep = ModeCfg<MODE>::kPrep;
    constexpr int KP = GemvShared<NT, shared_layout<MODE>()>::KP;
    __shared__ GemvShared<NT, shared_layout<MODE>()> sh;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t lane = tid & 63;
    const Chunk ch(g, blockIdx.x, wave, W);
    ActLoads<MODE, KP, W> act;
    if constexpr (kPrep) act.issue(g, ch, wave, lane);
    // (a CU serves its vector memory queue in order) every wavefront's
    // activation loads are queued ahead of all record loads
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const OnePhase<NT, MODE, EPI> src{g, ch, wave};
    Rec<(NT + 1) / 2> ring[PF];
    src.load(ring[0], 0, lane);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EPI == 1) {
        // this workgroup's slice of the next launch's output, behind the
        // first record loads
        const int per = (g_in.n_zero + (int)gridDim.x - 1) / (int)gridDim.x;
        const int z0 = (int)blockIdx.x * per;
        for (int i = z0 + tid; i < min(z0 + per, g_in.n_zero); i += W * 64) g_in.y_zero[i] = 0.0f;
    }
    // the LDS set-up runs while the first loads are in flight
    gemv_lds_init<NT, MODE>(sh, wave, lane, tid);
    lds_barrier();
    if constexpr (kPrep) act.commit(sh, g, ch, wave, lane);
#pragma unroll
    for (int s = 1; s < PF; ++s) src.load(ring[s], s, lane);
    gemv_stream<NT, MODE, EPI>(sh, g, ring, src, ch, 0, ch.n_mine, wave, lane);
    lds_barrier();
    // the epilogues read the kernel arguments themselves (g_in holds the
    // same values as g)
    if constexpr (EPI == 0) {
        gemv_epilogue_y<NT, MODE>(sh, g_in, ch, blockIdx.x, wave, lane);
    } else {
        gemv_epilogue_swiglu(sh, g_in, ch, blockIdx.x, tid, wave, lane);
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
        // an infinite or NaN d makes the row NaN (the reference's +-inf
        // products of both signs)
        acc += d - d;
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
    // records are addressed by 32-bit buffer offsets below kOutOfRange
    if ((size_t)a.n_tiles * a.nb * kRecordBytes >= kOutOfRange) return hipErrorInvalidValue;
    a.chunk = plan.chunk;
    a.max_parts = plan.max_parts;
    const void* asrc = (MODE == 1 || MODE == 2) ? static_cast<const void*>(a.x) : static_cast<const void*>(a.act);
    return launch_timed(kProfGemv, k_gemv_t64<NT, MODE, EPI>, dim3(plan.grid), dim3(GemvCfg<NT>::kWaves * 64), 0, s,
                        a.w[0], a.w[1], asrc, a.chunk, a.n_records, a.nb, a);
}

// Largest chunk (records per workgroup) that touches at most S tiles.
constexpr int max_chunk_slots(int slots, int nb) { return (slots - 1) * nb + 1; }

GemvArgs base_args(const GemvPlan& plan, const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                   unsigned long long row0, int out_dim, uint8_t* ws, uint32_t* err) {
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
    a.part = reinterpret_cast<uint64_t*>(ws + ((size_t)plan.n_tiles_all * 4 + 255) / 256 * 256);
    a.err = err;
    a.tiles_per_head = 1 << 30;
    a.head_stride = 0;
    a.x_bytes = (uint32_t)a.nb * 1024u;
    a.w_bytes = (uint32_t)((size_t)a.n_tiles * a.nb * kRecordBytes);
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
    return cnt + (size_t)tiles * (size_t)nb * (size_t)n_tok * 64 * 8;
}

size_t gemv_ws_bytes_planned(int n_tensors, int in_dim, int out_dim, int n_tok, int num_cus, int kind) {
    const GemvPlan p = plan_gemv(n_tensors, in_dim, out_dim, n_tok, num_cus, kind);
    const size_t cnt = ((size_t)p.n_tiles_all * 4 + 255) / 256 * 256;
    return cnt + (size_t)p.n_tiles_all * (size_t)p.max_parts * (size_t)n_tok * 64 * 8;
}

hipError_t launch_gemv_t64(const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                           unsigned long long row0, int out_dim, int n_tok, const uint8_t* act,
                           uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s) {
    const GemvPlan plan = plan_gemv(n_tensors, in_dim, out_dim, n_tok, num_cus, kPlanAct);
    if (plan.grid == 0) return hipSuccess;
    GemvArgs a = base_args(plan, w, y, n_tensors, in_dim, row0, out_dim, ws, err);
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
                         uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s) {
    const GemvPlan plan = plan_gemv(n_tensors, in_dim, out_dim, 1, num_cus, kPlanPrep);
    if (plan.grid == 0) return hipSuccess;
    GemvArgs a = base_args(plan, w, y, n_tensors, in_dim, row0, out_dim, ws, err);
    a.x = x;
    a.x2 = x2;
    a.lim = lim;
    if (x2) return launch_gemv_nt<1, 2>(plan, a, s);
    return launch_gemv_nt<1, 1>(plan, a, s);
}

hipError_t launch_gemv_heads(const uint8_t* w, int in_dim, unsigned long long row0, int rows_per_head, int n_heads,
                             const float* x, float* y, uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s) {
    const int out_dim = rows_per_head * n_heads;
    const GemvPlan plan = plan_gemv(1, in_dim, out_dim, 1, num_cus, kPlanPrep);
    if (plan.grid == 0) return hipSuccess;
    if ((size_t)n_heads * in_dim * 4 >= kOutOfRange) return hipErrorInvalidValue;
    const uint8_t* ww[1] = {w};
    float* yy[1] = {y};
    GemvArgs a = base_args(plan, ww, yy, 1, in_dim, row0, out_dim, ws, err);
    a.x = x;
    a.tiles_per_head = rows_per_head / kTileRows;
    a.head_stride = (uint32_t)in_dim * 4u;
    a.x_bytes = (uint32_t)((size_t)n_heads * in_dim * 4);
    return launch_gemv_nt<1, 1>(plan, a, s);
}

size_t act64_bytes(int in_dim) { return act64_bytes_n(in_dim / kQK); }

size_t gate_up_ws_bytes(int in_dim, int out_dim) {
    const long long nb = in_dim / kQK;
    const long long tiles = (out_dim + kTileRows - 1) / kTileRows;
    const size_t cnt = ((size_t)(2 * tiles) * 4 + 255) / 256 * 256;
    return cnt + (size_t)tiles * (size_t)(2 * nb) * 2 * 64 * 8;
}

hipError_t launch_gate_up_swiglu(const uint8_t* w_gate, const uint8_t* w_up, int in_dim, int out_dim,
                                 const float* x, float lim, uint8_t* act_out, uint8_t* ws, uint32_t* err,
                                 int num_cus, hipStream_t s, float* y_zero, int n_zero) {
    if (out_dim % kQK) return hipErrorInvalidValue;  // act64 blocks of the output
    const GemvPlan plan = plan_gemv(2, in_dim, out_dim, 1, num_cus, kPlanSwigluPairs);
    if (plan.grid == 0) return hipSuccess;
    const uint8_t* w[2] = {w_gate, w_up};
    GemvArgs a = base_args(plan, w, nullptr, 2, in_dim, 0, out_dim, ws, err);
    a.x = x;
    a.x2 = x;
    a.lim = lim;
    a.act_out = act_out;
    a.y_zero = y_zero;
    a.n_zero = y_zero ? n_zero : 0;
    return launch_gemv_nt<1, 1, 1>(plan, a, s);
}

// [header][gate/up region][down region][act64]: the regions that must stay
// zero between launches come first, the scratch last.
size_t dense_mlp_ws_bytes(int hidden, int inter) {
    const auto a256 = [](size_t b) { return (b + 255) / 256 * 256; };
    return kWsHeader + a256(gate_up_ws_bytes(hidden, inter)) + a256(gemv_ws_bytes(1, inter, hidden, 1)) +
           a256(act64_bytes(inter));
}

hipError_t launch_dense_mlp(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int hidden, int inter,
                            const float* x, float lim, float* y, uint8_t* ws, int num_cus, hipStream_t s) {
    const auto a256 = [](size_t b) { return (b + 255) / 256 * 256; };
    uint32_t* err = reinterpret_cast<uint32_t*>(ws);
    uint8_t* ws_a = ws + kWsHeader;
    uint8_t* ws_b = ws_a + a256(gate_up_ws_bytes(hidden, inter));
    uint8_t* act = ws_b + a256(gemv_ws_bytes(1, inter, hidden, 1));
    // The gate/up launch zero-fills y and the down launch adds the parts of
    // its shared row tiles into it, unless y overlaps x (which the gate/up
    // launch reads): then the down launch sums them in chunk order.
    const uintptr_t xb = reinterpret_cast<uintptr_t>(x), yb = reinterpret_cast<uintptr_t>(y);
    const bool apart = yb + (size_t)hidden * 4 <= xb || xb + (size_t)hidden * 4 <= yb;
    hipError_t e = launch_gate_up_swiglu(w_gate, w_up, hidden, inter, x, lim, act, ws_a, err, num_cus, s,
                                         apart ? y : nullptr, hidden);
    if (e != hipSuccess) return e;
    return launch_gemv_act64(w_down, inter, 0, hidden, act, y, ws_b, err, num_cus, s, apart);
}

hipError_t launch_gemv_act64(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const uint8_t* act64, float* y, uint8_t* ws, uint32_t* err, int num_cus,
                             hipStream_t s, bool y_zeroed) {
    const GemvPlan plan = plan_gemv(1, in_dim, out_dim, 1, num_cus, kPlanPrep);
    if (plan.grid == 0) return hipSuccess;
    float* yy[1] = {y};
    const uint8_t* ww[1] = {w};
    GemvArgs a = base_args(plan, ww, yy, 1, in_dim, row0, out_dim, ws, err);
    a.act = act64;
    a.xsc = reinterpret_cast<const float*>(act64 + (size_t)a.nb * 1024);
    a.y_atomic = y_zeroed ? 1 : 0;
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
