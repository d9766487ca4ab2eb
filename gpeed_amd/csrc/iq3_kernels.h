// Kernel launchers shared between the .hip translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gpeed {

// Every product workspace starts with this many bytes of header; word 0
// collects the error flags below (read by gpeed_ws_status). The launchers
// take the header's error word and the region after the header.
constexpr size_t kWsHeader = 256;
constexpr uint32_t kWsTicket = 1u;   // a ticket counted more arrivals than the unit has parts
constexpr uint32_t kWsTimeout = 2u;  // a bounded wait for another workgroup's partial gave up
constexpr uint32_t kWsBuckets = 4u;  // expert buckets break the router's invariants

// Zero-fill of n bytes (16-byte aligned, n a multiple of 16) with a kernel.
hipError_t launch_fill_zero(void* p, size_t n, hipStream_t s);

// quant.cpp:186-210 over n/256 raw GGUF blocks -> fp32 (bit-exact).
hipError_t launch_dequant_raw(const uint8_t* src, float* dst, unsigned long long n, hipStream_t s);

// Raw GGUF rows of any format the reference decodes (quant_rows.hip):
// geometry (0 for other types), dequantization of n weights, and
// Y[t][j] = sum_i W[row0 + j][i] * X[t][i].
int rows_block_elems(int dtype);
size_t rows_block_bytes(int dtype);
hipError_t launch_dequant_rows(int dtype, const uint8_t* src, float* dst, unsigned long long n, hipStream_t s);
hipError_t launch_matmul_rows(int dtype, const uint8_t* w, size_t row_bytes, unsigned long long row0, int in_dim,
                              int out_dim, const float* X, int n_tok, float* Y, hipStream_t s);
uint64_t rows_iq2s_grid(int i);
uint32_t rows_iq3s_grid(int i);
// Streaming read of `bytes` from p (16-byte aligned) by n_groups workgroups;
// out[i] = a fold of what workgroup i read.
hipError_t launch_stream_read(const uint8_t* p, unsigned long long bytes, uint32_t* out, int n_groups,
                              hipStream_t s);
// GGUF rows -> T64 (tiled) and back. n_rows rows of in_dim weights.
hipError_t launch_tile(const uint8_t* raw, unsigned long long n_rows, int in_dim, uint8_t* t64,
                       hipStream_t s);
hipError_t launch_untile(const uint8_t* t64, unsigned long long n_rows, int in_dim, uint8_t* raw,
                         hipStream_t s);

// Prepared activation ("act") of n_tok fp32 vectors [n_tok][in_dim]: per
// 256-element block the fp16 hi/lo MFMA A-operand images scaled by a power
// of two (n_tok KiB), then one fp32 unscale per (block, token). act_bytes()
// is its size, rounded to 256 bytes.
size_t act_bytes(int in_dim, int n_tok);
hipError_t launch_prep_act(const float* x, int in_dim, int n_tok, uint8_t* act, hipStream_t s);
// Same for h = silu(min(g,lim)) * clamp(u,-lim,lim) (SwiGLU epilogue).
hipError_t launch_prep_swiglu(const float* g, const float* u, float lim, int in_dim, int n_tok,
                              uint8_t* act, hipStream_t s);

// Work split of one GEMV launch (records per workgroup, grid, parts bound).
struct GemvPlan {
    long long n_tiles_all;
    long long n_records;
    int chunk;
    int grid;
    int max_parts;
};
// kind: how the launch gets its activation (prepared images, prepared in
// the kernel, or prepared in the kernel with the gate/up SwiGLU epilogue).
enum { kPlanAct = 0, kPlanPrep = 1, kPlanSwigluPairs = 2 };
GemvPlan plan_gemv(int n_tensors, int in_dim, int out_dim, int n_tok, int num_cus, int kind);
// Workspace region of a GEMV launch (after the header): tickets for the
// tiles shared between workgroups, then their tagged partial sums, indexed
// so that a region sized for n_tok covers every launch with fewer tokens.
// Zero-filled once before first use; every launch leaves the words it used
// at zero again.
size_t gemv_ws_bytes(int n_tensors, int in_dim, int out_dim, int n_tok);
// The region one launch of this plan kind actually touches on a device with
// num_cus CUs (part words for max_parts parts per tile rather than one per
// block): what a fixed-size scratch must hold.
size_t gemv_ws_bytes_planned(int n_tensors, int in_dim, int out_dim, int n_tok, int num_cus, int kind);
// y_i[t][j] = sum_k W_i[row0+j][k] x_t[k] over the T64 payloads of n_tensors
// (1 or 2) same-shape tensors sharing one prepared activation of n_tok
// (1..8) vectors.
hipError_t launch_gemv_t64(const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                           unsigned long long row0, int out_dim, int n_tok, const uint8_t* act,
                           uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s);
// One fp32 vector x, prepared inside the GEMV workgroups
// (no separate preparation launch); with x2 != null the input is
// silu(min(x,lim)) * clamp(x2,-lim,lim) (SwiGLU of gate x and up x2).
hipError_t launch_gemv_x(const uint8_t* const* w, float* const* y, int n_tensors, int in_dim,
                         unsigned long long row0, int out_dim, const float* x, const float* x2, float lim,
                         uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s);
// Per-head products in one launch: head h < n_heads multiplies its own
// vector x[h*in_dim ..] by rows row0 + h*rows_per_head .. (rows_per_head a
// multiple of 64), y[h*rows_per_head + j]. ws/err as launch_gemv_x with
// out_dim = n_heads * rows_per_head.
hipError_t launch_gemv_heads(const uint8_t* w, int in_dim, unsigned long long row0, int rows_per_head, int n_heads,
                             const float* x, float* y, uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s);
// Dense-MLP pair of launches (model.cpp:677-690) without a host round trip:
// launch_gate_up_swiglu runs gate and up (same shape, out_dim rows of
// in_dim) against one fp32 x, and the workgroup that completes a row tile
// writes h = silu(min(g,lim)) * clamp(u,-lim,lim) of its 64 rows as
// "act64": per 256-element block four fp16 hi/lo images of 64 elements,
// each with its own power-of-two unscale (act64_bytes(out_dim) bytes).
// launch_gemv_act64 then multiplies an act64 activation (the down
// projection). gate_up_ws_bytes: the first launch's workspace region
// (zero-filled once, left at zero by every launch).
size_t act64_bytes(int in_dim);
size_t gate_up_ws_bytes(int in_dim, int out_dim);
// y_zero (n_zero floats, may be null): zero-filled by the gate/up launch
// for a down launch that adds into it (launch_gemv_act64 with y_zeroed).
hipError_t launch_gate_up_swiglu(const uint8_t* w_gate, const uint8_t* w_up, int in_dim, int out_dim,
                                 const float* x, float lim, uint8_t* act_out, uint8_t* ws, uint32_t* err,
                                 int num_cus, hipStream_t s, float* y_zero = nullptr, int n_zero = 0);
// y_zeroed: y holds zeros when the launch starts; the parts of a row tile
// shared by several workgroups are then added into y with atomic adds (no
// ticket, no wait) instead of being summed in chunk order by the last part.
hipError_t launch_gemv_act64(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const uint8_t* act64, float* y, uint8_t* ws, uint32_t* err, int num_cus,
                             hipStream_t s, bool y_zeroed = false);
// Both (the header, the act64 buffer, then each launch's tickets and
// partials in one workspace of dense_mlp_ws_bytes, zero-filled once).
size_t dense_mlp_ws_bytes(int hidden, int inter);
hipError_t launch_dense_mlp(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int hidden, int inter,
                            const float* x, float lim, float* y, uint8_t* ws, int num_cus, hipStream_t s);
// Same product (one vector) straight from GGUF rows (VALU decode, no repacking).
hipError_t launch_matvec_raw(const uint8_t* w, int in_dim, unsigned long long row0, int out_dim,
                             const float* x, float* y, hipStream_t s);
hipError_t launch_add(const float* a, const float* b, float* dst, int n, hipStream_t s);

// Router (model_batch.cpp:178-219) on the device: top-k per token of
// logits [T][E], then the stable expert buckets eptr[E+1], tok[T*K],
// wt[T*K] (and the per-token ranked choices sel[T*K] if sel != null).
// ws: moe_route_ws_bytes(T, K) bytes of scratch.
size_t moe_route_ws_bytes(int T, int K);
hipError_t launch_moe_route(const float* logits, int T, int E, int K, int mode, const float* bias,
                            float routed_scale, int norm_topk, int* eptr, int* tok, float* wt, int* sel,
                            uint8_t* ws, hipStream_t s);
// Routed experts (model_batch.cpp:221-262): gate/up/down of every touched
// expert over its bucket of tokens, SwiGLU between, weighted combine into
// Y [T][H] (overwritten). ws: moe_ws_bytes(...) bytes (header included);
// buckets that break the router's invariants set kWsBuckets and give Y = 0.
size_t moe_ws_bytes(int T, int E, int K, int H, int I);
hipError_t launch_moe_experts(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int E, int H,
                              int I, const float* X, int T, int K, const int* eptr, const int* tok,
                              const float* wt, float lim, float* Y, uint8_t* ws, int num_cus, hipStream_t s);
// A whole routed step from the router logits (model_batch.cpp:174-280) in
// five launches: router + bucket sort + work plan with the per-token X
// images, grouped gate/up (the shared expert's segments included, w_gate_sh
// non-null), SwiGLU images, grouped down, combine (+ shared expert).
// eptr/tok/wt_out: optional device outputs of the routing.
size_t moe_batch_ws_bytes(int T, int E, int K, int H, int I, int shared, int num_cus);
hipError_t launch_moe_batch(const float* logits, int T, int E, int K, int mode, const float* bias,
                            float routed_scale, int norm_topk, const uint8_t* w_gate, const uint8_t* w_up,
                            const uint8_t* w_down, const uint8_t* w_gate_sh, const uint8_t* w_up_sh,
                            const uint8_t* w_down_sh, int H, int I, const float* X, float lim, float* Y,
                            int* eptr_out, int* tok_out, float* wt_out, uint8_t* ws, int num_cus, hipStream_t s);

// Prefill GEMM: Y[m][j] = sum_k X[m][k] W[row0+j][k] for M tokens from the
// T64 copy. X is fp32 (x_bf16 = 0) or bf16 (x_bf16 = 1), row-major [M][in_dim];
// ws: a region of gemm_ws_bytes(M, out_dim, in_dim, x_bf16, num_cus) bytes
// (fp16 images; when the result tiles fill fewer than half the CUs, K is
// split and the region also holds tickets, cleared by the X preparation of
// every launch, and fp32 partials). Returns hipErrorInvalidValue when a
// tensor's requested rows hold 4 GiB of records or more (32-bit offsets).
int gemm_splits(int M, int N, int K, int num_cus, int x_bf16, int tile_n = 192);
// Token rows of one result tile (64, or 128 for bf16 X of more than 64 tokens).
int gemm_tile_m(int M, int x_bf16);
size_t gemm_ws_bytes(int M, int N, int K, int x_bf16, int num_cus);
// U (fp32, with x_bf16 = 0): X is SwiGLU(X, U) with clamp lim, formed while
// the images are prepared.
hipError_t launch_gemm(const uint8_t* w, unsigned long long row0, int in_dim, int out_dim, const void* X, int x_bf16,
                       int M, float* Y, uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s,
                       const float* U = nullptr, float lim = 0.0f);
// Two tensors on the same X in one launch (X prepared once): Ya [M][out_a]
// from wa, Yb [M][out_b] from wb; ws: gemm2_ws_bytes bytes.
size_t gemm2_ws_bytes(int M, int out_a, int out_b, int K, int x_bf16, int num_cus);
hipError_t launch_gemm2(const uint8_t* wa, unsigned long long row0a, int out_a, const uint8_t* wb,
                        unsigned long long row0b, int out_b, int in_dim, const void* X, int x_bf16, int M, float* Ya,
                        float* Yb, uint8_t* ws, uint32_t* err, int num_cus, hipStream_t s, const float* U = nullptr,
                        float lim = 0.0f);

// Batched dense MLP as GEMMs over M tokens: Y [M][H] = down(SwiGLU(gate X,
// up X)) for whole T64 tensors gate/up [I][H] and down [H][I], plus up to two
// more whole T64 tensors of the same X (w_e1 [out_e1][H] -> y_e1, w_e2 ->
// y_e2; null for none) computed in the down launch where that balances;
// ws: mlp_gemm_ws_bytes bytes.
size_t mlp_gemm_ws_bytes(int H, int I, int M, int x_bf16, int out_e1, int out_e2, int num_cus);
hipError_t launch_mlp_gemm(const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down, int H, int I,
                           const void* X, int x_bf16, int M, float lim, float* Y, const uint8_t* w_e1, int out_e1,
                           float* y_e1, const uint8_t* w_e2, int out_e2, float* y_e2, uint8_t* ws, uint32_t* err,
                           int num_cus, hipStream_t s);

// Grouped GEMM over routed-expert buckets: for every expert e, rows
// eptr[e] .. eptr[e + 1] of the [2][S][in_dim] fp16 images xh (fp32 X as hi
// and lo, unscales uns[S]) times rows e * rows .. of wa (and wb, the second
// tensor on the same X; null for one), into rows eptr[e] .. of ya / yb
// ([S][rows]). tiles / count: the expert tile table launch_grp_tiles makes
// from eptr (grp_tiles_cap(S, E, mt) entries) for tiles of 16 mt tokens
// (mt = 2..5; grp_tile_mt picks it from the mean bucket; a cap for mt 0
// holds any). rows a multiple of 64. tok (may be null): the images hold
// img_rows rows (one per token) and slot p reads row tok[p]. sh_rows > 0:
// the last sh_rows of the S slots are the shared expert's (tensors wa_sh,
// wb_sh; one table entry id E per tile of them, from launch_grp_tiles with
// the same sh_rows and S less them); with tok its slot m reads row m.
int grp_tiles_cap(int S, int E, int mt);
int grp_tile_mt(int S, int E);
hipError_t launch_grp_tiles(const int* eptr, int E, int S, int mt, int* tiles, int* count, hipStream_t s,
                            int sh_rows = 0);
hipError_t launch_gemm_grouped(const uint8_t* wa, const uint8_t* wb, int rows, int in_dim, int E, const int* eptr,
                               int S, const _Float16* xh, const float* uns, float* ya, float* yb, const int* tiles,
                               const int* count, uint32_t* err, hipStream_t s, int mt, const int* tok = nullptr,
                               int img_rows = 0, const uint8_t* wa_sh = nullptr, const uint8_t* wb_sh = nullptr,
                               int sh_rows = 0);
// fp32 rows -> the GEMM's hi and lo images (unscale per row): X rows
// gather[m] (gather null: row m), or SwiGLU(X, U) with clamp lim when U is
// given.
hipError_t launch_prep_x_rows(int M, int K, hipStream_t s, const float* X, const float* U, float lim, _Float16* xh,
                              float* uns, const int* gather);

}  // namespace gpeed
